// Synthetic checkpoint generator: a model.safetensors with the reference's tensor names
// (runtime/crates/laya-mlx/src/lib.rs:990-1131, runtime/crates/laya-core/src/decode.rs:130-136)
// and seeded random-init bf16 values, so that a real checkpoint drops into the same loader.
//
// Values: every Linear weight and embedding ~ N(0, 0.02). LayerNorm weights are 1 and biases 0,
// or, with `jitter`, 1 + N(0, 0.02) and N(0, 0.02), which lets parity tests see a dropped or
// misplaced bias. Each value is drawn in double by Box-Muller from two splitmix64 outputs keyed
// by (seed, tensor name, element index), rounded to f32 and then to bf16 (nearest even), so the
// bytes do not depend on thread count or generation order.
#include <thread>

#include "synth.hpp"

namespace s1 {

static inline uint64_t splitmix64(uint64_t x) {
  x += 0x9E3779B97F4A7C15ull;
  x = (x ^ (x >> 30)) * 0xBF58476D1CE4E5B9ull;
  x = (x ^ (x >> 27)) * 0x94D049BB133111EBull;
  return x ^ (x >> 31);
}

static inline uint64_t fnv1a64(const std::string& s) {
  uint64_t h = 0xcbf29ce484222325ull;
  for (unsigned char c : s) {
    h ^= c;
    h *= 0x100000001b3ull;
  }
  return h;
}

double synth_normal(uint64_t key, uint64_t e) {
  uint64_t a = splitmix64(key + 2 * e);
  uint64_t b = splitmix64(key + 2 * e + 1);
  double u1 = double((a >> 11) + 1) * 0x1.0p-53;  // (0, 1]
  double u2 = double(b >> 11) * 0x1.0p-53;        // [0, 1)
  return std::sqrt(-2.0 * std::log(u1)) * std::cos(6.283185307179586476925286766559 * u2);
}

uint64_t synth_key(uint64_t seed, const std::string& name) { return splitmix64(seed ^ fnv1a64(name)); }

std::vector<TensorSpec> checkpoint_layout(const ModelConfig& c, int scorer_width, int n_act) {
  using V = std::vector<int64_t>;
  std::vector<TensorSpec> t;
  const int64_t d = c.d, I = c.inter, V_ = c.vocab;
  t.push_back({"encoder.embeddings.tok_embeddings.weight", V{V_, d}, TensorKind::Weight});
  t.push_back({"encoder.embeddings.norm.weight", V{d}, TensorKind::NormWeight});
  for (int i = 0; i < c.layers; ++i) {
    std::string p = "encoder.layers." + std::to_string(i);
    if (i != 0) t.push_back({p + ".attn_norm.weight", V{d}, TensorKind::NormWeight});
    t.push_back({p + ".attn.Wqkv.weight", V{3 * d, d}, TensorKind::Weight});
    t.push_back({p + ".attn.Wo.weight", V{d, d}, TensorKind::Weight});
    t.push_back({p + ".mlp_norm.weight", V{d}, TensorKind::NormWeight});
    t.push_back({p + ".mlp.Wi.weight", V{2 * I, d}, TensorKind::Weight});
    t.push_back({p + ".mlp.Wo.weight", V{d, I}, TensorKind::Weight});
  }
  t.push_back({"encoder.final_norm.weight", V{d}, TensorKind::NormWeight});
  t.push_back({"type_emb.weight", V{3, d}, TensorKind::Weight});
  for (int j = 0; j < c.head_layers; ++j) {
    std::string p = "head.layers." + std::to_string(j);
    t.push_back({p + ".norm1.weight", V{d}, TensorKind::NormWeight});
    t.push_back({p + ".norm1.bias", V{d}, TensorKind::Bias});
    t.push_back({p + ".self_attn.in_proj_weight", V{3 * d, d}, TensorKind::Weight});
    t.push_back({p + ".self_attn.in_proj_bias", V{3 * d}, TensorKind::Bias});
    t.push_back({p + ".self_attn.out_proj.weight", V{d, d}, TensorKind::Weight});
    t.push_back({p + ".self_attn.out_proj.bias", V{d}, TensorKind::Bias});
    t.push_back({p + ".norm2.weight", V{d}, TensorKind::NormWeight});
    t.push_back({p + ".norm2.bias", V{d}, TensorKind::Bias});
    t.push_back({p + ".linear1.weight", V{4 * d, d}, TensorKind::Weight});
    t.push_back({p + ".linear1.bias", V{4 * d}, TensorKind::Bias});
    t.push_back({p + ".linear2.weight", V{d, 4 * d}, TensorKind::Weight});
    t.push_back({p + ".linear2.bias", V{d}, TensorKind::Bias});
  }
  const int64_t S = scorer_width;
  t.push_back({"scorer.0.weight", V{d}, TensorKind::NormWeight});
  t.push_back({"scorer.0.bias", V{d}, TensorKind::Bias});
  t.push_back({"scorer.1.weight", V{S, d}, TensorKind::Weight});
  t.push_back({"scorer.1.bias", V{S}, TensorKind::Bias});
  t.push_back({"scorer.3.weight", V{1, S}, TensorKind::Weight});
  t.push_back({"scorer.3.bias", V{1}, TensorKind::Bias});
  t.push_back({"act_head.0.weight", V{256, d + 4}, TensorKind::Weight});
  t.push_back({"act_head.0.bias", V{256}, TensorKind::Bias});
  t.push_back({"act_head.2.weight", V{n_act, 256}, TensorKind::Weight});
  t.push_back({"act_head.2.bias", V{n_act}, TensorKind::Bias});
  return t;
}

std::vector<uint8_t> synth_checkpoint(const ModelConfig& c, uint64_t seed, int scorer_width, int n_act, bool jitter) {
  std::vector<TensorSpec> layout = checkpoint_layout(c, scorer_width, n_act);
  std::vector<OutTensor> out;
  out.reserve(layout.size());
  unsigned nthreads = std::max(1u, std::min(16u, std::thread::hardware_concurrency()));
  for (const auto& spec : layout) {
    OutTensor t;
    t.name = spec.name;
    t.shape = spec.shape;
    int64_t n = 1;
    for (auto s : spec.shape) n *= s;
    t.bf16.resize(size_t(n));
    double mean = 0.0, std_ = 0.02;
    if (spec.kind == TensorKind::NormWeight) {
      mean = 1.0;
      std_ = jitter ? 0.02 : 0.0;
    } else if (spec.kind == TensorKind::Bias) {
      std_ = jitter ? 0.02 : 0.0;
    }
    const uint64_t key = synth_key(seed, spec.name);
    auto work = [&](int64_t b, int64_t e) {
      for (int64_t i = b; i < e; ++i) {
        double v = mean + (std_ != 0.0 ? std_ * synth_normal(key, uint64_t(i)) : 0.0);
        t.bf16[size_t(i)] = f32_to_bf16(float(v));
      }
    };
    if (n < (1 << 16) || nthreads == 1) {
      work(0, n);
    } else {
      std::vector<std::thread> th;
      int64_t chunk = (n + nthreads - 1) / nthreads;
      for (unsigned k = 0; k < nthreads; ++k) {
        int64_t b = int64_t(k) * chunk, e = std::min(n, b + chunk);
        if (b < e) th.emplace_back(work, b, e);
      }
      for (auto& x : th) x.join();
    }
    out.push_back(std::move(t));
  }
  return write_safetensors_bf16(out);
}

}  // namespace s1
