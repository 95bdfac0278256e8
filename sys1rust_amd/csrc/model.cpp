// Host runtime of libsys1hip: checkpoint load, request planning and the kernel sequence of one
// forward. The sequence follows MlxBackend::encode / head_forward / score / forward
// (runtime/crates/laya-mlx/src/lib.rs:1525-1863) op for op, in the packed token layout that the
// reference's `unpad` setting uses (Packing, lib.rs:894-943): activations are [T, ·] over the real
// tokens only, and attention reads each row's token range directly instead of expanding to
// [n, len].
#include "model.hpp"
#include "selfcheck.hpp"

#include <chrono>
#include <cstdio>

namespace s1 {

namespace {

void hip_check(hipError_t e, const char* what) {
  if (e != hipSuccess) fail(kBackend, std::string(what) + ": " + hipGetErrorString(e));
}

size_t align256(size_t x) { return (x + 255) & ~size_t(255); }

}  // namespace

Settings Settings::parse(const std::string& spec) {
  Settings s;
  size_t i = 0;
  while (i <= spec.size()) {
    size_t j = spec.find(',', i);
    if (j == std::string::npos) j = spec.size();
    std::string kv = spec.substr(i, j - i);
    i = j + 1;
    if (kv.empty()) {
      if (j == spec.size()) break;
      continue;
    }
    std::string key = kv, val;
    bool has_val = false;
    size_t eq = kv.find('=');
    if (eq != std::string::npos) {
      key = kv.substr(0, eq);
      val = kv.substr(eq + 1);
      has_val = true;
    }
    auto bad = [&](const std::string& what) { fail(kConfig, "hip settings: `" + kv + "`: " + what); };
    // A flag is on when bare or `=1`, off when `=0`; nothing else.
    auto flag = [&]() -> bool {
      if (!has_val || val == "1") return true;
      if (val == "0") return false;
      bad("`" + val + "` is not 0 or 1");
      return false;
    };
    auto value = [&]() -> const std::string& {
      if (!has_val) bad("needs a value (`key=value`)");
      return val;
    };
    auto number = [&](const std::string& v) -> size_t {
      if (v.empty() || v.size() > 19 || v.find_first_not_of("0123456789") != std::string::npos)
        bad("`" + v + "` is not a whole number");
      return size_t(std::stoull(v));
    };
    auto list = [&]() {
      const std::string& v = value();
      std::vector<size_t> out;
      size_t a = 0;
      while (a <= v.size()) {
        size_t b = v.find(':', a);
        if (b == std::string::npos) b = v.size();
        out.push_back(number(v.substr(a, b - a)));
        a = b + 1;
      }
      return out;
    };
    auto one_of = [&](std::initializer_list<const char*> allowed) -> std::string {
      const std::string& v = value();
      std::string names;
      for (const char* a : allowed) {
        if (v == a) return v;
        names += std::string(names.empty() ? "" : ", ") + a;
      }
      bad("`" + v + "` is not one of " + names);
      return v;
    };
    // Knobs' keys (lib.rs:196-256), with its value checks.
    if (key == "geglu") one_of({"shapeless", "compiled", "plain"});
    else if (key == "addmm") flag();
    else if (key == "mask") s.bool_mask = one_of({"bool", "additive"}) == "bool";
    else if (key == "windowed") s.windowed = flag();
    else if (key == "clear") s.clear = flag();
    else if (key == "trace") s.trace = flag();
    else if (key == "layers") s.layers = flag();
    else if (key == "ops") s.ops = flag();
    else if (key == "wcopy") one_of({"view", "gpu", "t"});
    else if (key == "f16gelu") flag();
    else if (key == "buckets") {
      s.buckets = list();
      std::sort(s.buckets.begin(), s.buckets.end());
    } else if (key == "pad") {
      s.pad = number(value());
      if (s.pad == 0) bad("pad must be at least 1");
    } else if (key == "warm") s.warm = list();
    else if (key == "cache") number(value());
    else if (key == "wired") number(value());
    else if (key == "dense_upto") s.dense_upto = long(number(value()));
    else if (key == "headprune") s.headprune = flag();
    else if (key == "unpad") s.unpad = flag();
    else if (key == "fuserope") s.fuserope = flag();
    else if (key == "band") s.band = number(value());
    else if (key == "nax") one_of({"0", "all"});
    else if (key == "directload") flag();
    else if (key == "sharehead") flag();
    else if (key == "parallel_load") flag();  // read by the runtime (backend.rs:44-69); checked here too
    // This backend's own.
    else if (key == "fusegeglu") s.fusegeglu = flag();
    else if (key == "fuseln") s.fuseln = flag();
    else if (key == "graphs") s.graphs = flag();
    else if (key == "dtype") {
      const std::string t = one_of({"bf16", "f16", "f32"});
      s.f16 = t == "f16";
      s.f32 = t == "f32";
    }
    else fail(kConfig, "hip settings: unknown setting `" + key + "` in `" + spec + "`");
    if (j == spec.size()) break;
  }
  return s;
}

struct Model::Acts {
  float* h;           // [T, d] residual stream (f32)
  uint16_t* x;        // [T, d] normalised GEMM input
  uint16_t *q, *k, *v;  // [H, T, 64]
  uint16_t* qkv;      // [T, 3d]
  uint16_t* att;      // [T, d]
  uint16_t* mid;      // [T, max(2I, 4d)]
  uint16_t* act;      // [T, I]
  float* enc;         // [T, d] encoder output (encoder_hidden)
  float* hh;          // [T, d] head stream
  float* hp;          // [P, d] picked rows
  uint16_t* xp;       // [P, d]
  uint16_t* attp;     // [P, d]
  uint16_t* midp;     // [P, 4d]
  uint16_t* sx;       // [R, d]
  uint16_t* s1;       // [R, S]
  float* logits;      // [R]
  float* pooled;      // [n, d]
  float* ws;          // split-K partials of the largest GEMM that splits
};

Model::Model(const SafeTensors& st, const std::string& enc_json, const std::string& agent_json,
             const std::string& settings, int dev)
    : device(dev) {
  // A load that fails part way gives back what it had already allocated (the destructor does not
  // run for a constructor that throws).
  try {
    init(st, enc_json, agent_json, settings);
  } catch (...) {
    teardown();
    throw;
  }
}

void Model::init(const SafeTensors& st, const std::string& enc_json, const std::string& agent_json,
                 const std::string& settings) {
  const int dev = device;
  cfg = parse_model_config(enc_json, agent_json);
  set = Settings::parse(settings);
  // headprune prunes the last head layer; with no head layers the scorer reads the encoder's
  // stream whole, as head_forward's loop then leaves it (lib.rs:1726-1765).
  if (cfg.head_layers == 0) set.headprune = false;
  // dtype=f32 runs the plain f32 kernels: no fused kernels, and the head's last layer over every
  // row (headprune skips only rows nobody reads, so the outputs are the same). fuserope keeps its
  // other meaning there: with `band` it chooses the banded local attention (lib.rs:330-361).
  if (set.f32) set.fusegeglu = set.fuseln = set.headprune = false;
  elem = set.f16 ? ELEM_F16 : ELEM_BF16;
  // The forwards `warm` runs at load (warm_buckets) are checked before any device work.
  if (std::any_of(set.warm.begin(), set.warm.end(), [](size_t n) { return n > 0; }))
    for (size_t len : set.buckets) {
      if (len < 3) fail(kConfig, "hip settings: warm needs buckets of at least 3 tokens");
      if (len > size_t(cfg.max_pos))
        fail(kConfig, "hip settings: warm bucket " + std::to_string(len) + " is longer than max_position_embeddings (" +
                          std::to_string(cfg.max_pos) + ")");
    }
  if (cfg.head_dim() != 64)
    fail(kConfig, "the HIP kernels need a head dim of 64; this encoder has " + std::to_string(cfg.head_dim()));
  if (cfg.d % 128 != 0 || cfg.d > kMaxHidden)
    fail(kConfig, "the HIP kernels need hidden_size to be a multiple of 128 up to " + std::to_string(kMaxHidden) +
                      "; got " + std::to_string(cfg.d));
  if (cfg.inter % 64 != 0)
    fail(kConfig, "the HIP kernels need intermediate_size to be a multiple of 64; got " + std::to_string(cfg.inter));
  const std::string& what = st.what();

  // Weights::verify (weights.rs:68-78)
  {
    auto names = st.names();
    for (const char* prefix : {"encoder.", "type_emb.", "scorer.", "act_head."}) {
      bool any = false;
      for (const auto& n : names) any = any || n.rfind(prefix, 0) == 0;
      if (!any)
        fail(kWeights, std::string("checkpoint is missing '") + prefix +
                           "' parameters; expected an RL Agent decision model");
    }
  }
  const int64_t d = cfg.d, I = cfg.inter;
  const auto& sc1 = st.get("scorer.1.weight");
  if (sc1.shape.size() != 2 || sc1.shape[1] != d) fail(kWeights, what + ": scorer.1.weight must be [S, " + std::to_string(d) + "]");
  scorer_width = int(sc1.shape[0]);
  if (scorer_width % 128 != 0) fail(kConfig, "the HIP kernels need the scorer width to be a multiple of 128");

  // Every tensor present with its expected shape before any device work (errors name the tensor).
  struct Item {
    std::string name;
    std::vector<int64_t> shape;
    bool bf16;
    int perm;  // 0 none, 1 Wi interleave
    void** dst;
  };
  std::vector<Item> items;
  auto addw = [&](const std::string& n, std::vector<int64_t> s, uint16_t** dst, int perm = 0) {
    items.push_back({n, s, true, perm, reinterpret_cast<void**>(dst)});
  };
  auto addf = [&](const std::string& n, std::vector<int64_t> s, float** dst) {
    items.push_back({n, s, false, 0, reinterpret_cast<void**>(dst)});
  };
  layers.resize(cfg.layers);
  head.resize(cfg.head_layers);
  addw("encoder.embeddings.tok_embeddings.weight", {cfg.vocab, d}, &tok_emb);
  addf("encoder.embeddings.norm.weight", {d}, &emb_norm);
  for (int i = 0; i < cfg.layers; ++i) {
    std::string p = "encoder.layers." + std::to_string(i);
    LayerWeights& L = layers[i];
    L.local = cfg.layer_local[i];
    if (i != 0) addf(p + ".attn_norm.weight", {d}, &L.attn_norm);
    addw(p + ".attn.Wqkv.weight", {3 * d, d}, &L.wqkv);
    addw(p + ".attn.Wo.weight", {d, d}, &L.wo);
    addf(p + ".mlp_norm.weight", {d}, &L.mlp_norm);
    addw(p + ".mlp.Wi.weight", {2 * I, d}, &L.wi, 1);
    addw(p + ".mlp.Wo.weight", {d, I}, &L.wo2);
  }
  addf("encoder.final_norm.weight", {d}, &final_norm);
  addf("type_emb.weight", {3, d}, &type_emb);
  for (int j = 0; j < cfg.head_layers; ++j) {
    std::string p = "head.layers." + std::to_string(j);
    HeadWeights& H = head[j];
    addf(p + ".norm1.weight", {d}, &H.n1w);
    addf(p + ".norm1.bias", {d}, &H.n1b);
    addw(p + ".self_attn.in_proj_weight", {3 * d, d}, &H.in_w);
    addf(p + ".self_attn.in_proj_bias", {3 * d}, &H.in_b);
    addw(p + ".self_attn.out_proj.weight", {d, d}, &H.out_w);
    addf(p + ".self_attn.out_proj.bias", {d}, &H.out_b);
    addf(p + ".norm2.weight", {d}, &H.n2w);
    addf(p + ".norm2.bias", {d}, &H.n2b);
    addw(p + ".linear1.weight", {4 * d, d}, &H.l1_w);
    addf(p + ".linear1.bias", {4 * d}, &H.l1_b);
    addw(p + ".linear2.weight", {d, 4 * d}, &H.l2_w);
    addf(p + ".linear2.bias", {d}, &H.l2_b);
  }
  const int64_t S = scorer_width;
  addf("scorer.0.weight", {d}, &sc0_w);
  addf("scorer.0.bias", {d}, &sc0_b);
  addw("scorer.1.weight", {S, d}, &sc1_w);
  addf("scorer.1.bias", {S}, &sc1_b);
  addf("scorer.3.weight", {1, S}, &sc3_w);
  addf("scorer.3.bias", {1}, &sc3_b);
  for (const auto& it : items) {
    const TensorView& tv = st.get(it.name);
    if (tv.shape != it.shape) (void)st.to_f32(it.name, it.shape);  // throws the shape message
  }

  int ndev = 0;
  hip_check(hipGetDeviceCount(&ndev), "hipGetDeviceCount");
  if (dev < 0 || dev >= ndev) fail(kBackend, "no GPU with ordinal " + std::to_string(dev) + " (" + std::to_string(ndev) + " visible)");
  hip_check(hipSetDevice(dev), "hipSetDevice");
  hipDeviceProp_t prop;
  hip_check(hipGetDeviceProperties(&prop, dev), "hipGetDeviceProperties");
  if (std::string(prop.gcnArchName).rfind("gfx950", 0) != 0)
    fail(kBackend, std::string("libsys1hip is built for gfx950 (MI355X); device ") + std::to_string(dev) + " is " + prop.gcnArchName);
  hip_check(hipStreamCreateWithFlags(&stream, hipStreamNonBlocking), "hipStreamCreate");

  // ---- RoPE tables, with the reference kernel's angle arithmetic (split_rope.metal:46-49):
  // inv_freq_i = exp2(-(i / half) * log2(theta)) and angle = p * inv_freq_i, both in f32; the
  // cosine and sine of that f32 angle are taken in double and rounded once.
  const int half = cfg.head_dim() / 2;
  const size_t rope_bytes = align256(size_t(cfg.max_pos) * half * 4);
  hip_check(hipMalloc(&rmem, 4 * rope_bytes), "hipMalloc(rope tables)");
  for (int which = 0; which < 2; ++which) {
    const float theta = float(which == 0 ? cfg.global_theta : cfg.local_theta);
    const float lbase = float(std::log2(double(theta)));
    std::vector<float> inv(half), c(size_t(cfg.max_pos) * half), s(size_t(cfg.max_pos) * half);
    for (int i = 0; i < half; ++i) {
      const float ex = -(float(i) / float(half)) * lbase;
      inv[i] = float(std::exp2(double(ex)));
    }
    for (int p = 0; p < cfg.max_pos; ++p)
      for (int i = 0; i < half; ++i) {
        const float ang = float(p) * inv[i];
        c[size_t(p) * half + i] = float(std::cos(double(ang)));
        s[size_t(p) * half + i] = float(std::sin(double(ang)));
      }
    char* base = static_cast<char*>(rmem);
    rope_cos[which] = reinterpret_cast<float*>(base + (2 * which) * rope_bytes);
    rope_sin[which] = reinterpret_cast<float*>(base + (2 * which + 1) * rope_bytes);
    hip_check(hipMemcpy(rope_cos[which], c.data(), c.size() * 4, hipMemcpyHostToDevice), "upload rope");
    hip_check(hipMemcpy(rope_sin[which], s.data(), s.size() * 4, hipMemcpyHostToDevice), "upload rope");
  }

  // ---- load-time checks of the fused kernels (lib.rs:319-362): decided here, never in a request.
  // A kernel that does not match its unfused twin is turned off for this load, with one line on
  // stderr, and the forward runs the unfused kernels instead.
  // Tests plant a wrong value in one check through the environment (SYS1HIP_CHECK_FAULT=fuserope,
  // fusegeglu or fuseln), never through the settings string that production passes.
  const char* fault_env = std::getenv("SYS1HIP_CHECK_FAULT");
  const std::string check_fault = fault_env ? fault_env : "";
  if (!check_fault.empty() && check_fault != "fuserope" && check_fault != "fusegeglu" && check_fault != "fuseln")
    fail(kConfig, "SYS1HIP_CHECK_FAULT=" + check_fault + " is not one of fuserope, fusegeglu, fuseln");
  auto decide = [&](bool& on, const char* nm, const char* instead, auto&& check) {
    if (!on || set.f32) return;  // the f32 path runs none of the fused kernels
    const std::string why = check(check_fault == nm);
    if (why.empty()) return;
    on = false;
    std::fprintf(stderr, "libsys1hip: %s is off for this load, %s run instead: %s\n", nm, instead, why.c_str());
  };
  decide(set.fuserope, "fuserope", "the Wqkv GEMM and split_rope_kernel", [&](bool fault) {
    return check_fuserope(elem, cfg.d, cfg.max_pos, rope_cos[0], rope_sin[0], stream, fault);
  });
  decide(set.fusegeglu, "fusegeglu", "the Wi GEMM and geglu_kernel", [&](bool fault) {
    return check_fusegeglu(elem, cfg.d, cfg.inter, stream, fault);
  });
  decide(set.fuseln, "fuseln", "the split-K reduce kernel and layernorm_kernel", [&](bool fault) {
    return check_fuseln(elem, cfg.d, float(cfg.eps), stream, fault);
  });

  // ---- weights, one allocation
  size_t total = 0;
  std::vector<size_t> offs;
  for (const auto& it : items) {
    int64_t n = 1;
    for (auto s : it.shape) n *= s;
    offs.push_back(total);
    total += align256(size_t(n) * (it.bf16 && !set.f32 ? 2 : 4));
  }
  hip_check(hipMalloc(&wmem, total), "hipMalloc(weights)");
  char* base = static_cast<char*>(wmem);
  std::vector<uint16_t> hb;
  for (size_t k = 0; k < items.size(); ++k) {
    const Item& it = items[k];
    void* dptr = base + offs[k];
    *it.dst = dptr;
    if (!it.bf16 || set.f32) {
      std::vector<float> f = st.to_f32(it.name, it.shape);
      hip_check(hipMemcpy(dptr, f.data(), f.size() * 4, hipMemcpyHostToDevice), "upload weight");
      continue;
    }
    const TensorView& tv = st.get(it.name);
    const size_t n = size_t(tv.numel());
    hb.resize(n);
    // The tensor's bits when it is stored in the model's 16-bit type, else rounded from f32 (every
    // bf16 and f16 value is exact in f32, so a tensor is rounded once).
    const DType want = set.f16 ? DType::F16 : DType::BF16;
    if (tv.dtype == want) {
      std::memcpy(hb.data(), tv.data, n * 2);
    } else {
      std::vector<float> f = st.to_f32(it.name, it.shape);
      for (size_t e = 0; e < n; ++e) hb[e] = set.f16 ? f32_to_f16(f[e]) : f32_to_bf16(f[e]);
    }
    if (it.perm == 1 && set.fusegeglu) {
      // Wi [2I, d] -> rows interleaved in blocks of 32: (x rows 32j.., gate rows I + 32j..).
      std::vector<uint16_t> o(n);
      const size_t rowb = size_t(d);
      for (int64_t j = 0; j < I / 32; ++j) {
        std::memcpy(&o[size_t(64 * j) * rowb], &hb[size_t(32 * j) * rowb], 32 * rowb * 2);
        std::memcpy(&o[size_t(64 * j + 32) * rowb], &hb[size_t(I + 32 * j) * rowb], 32 * rowb * 2);
      }
      hb.swap(o);
    }
    hip_check(hipMemcpy(dptr, hb.data(), n * 2, hipMemcpyHostToDevice), "upload weight");
  }

  char nb[64];
  std::snprintf(nb, sizeof nb, "hip(gfx950,%s)", set.f32 ? "f32" : set.f16 ? "f16" : "bf16");
  name = nb;
  // Backend::active_kernels (backend.rs:111-116): the custom kernels requested, built and checked
  // at this load.
  auto listed = [&](bool on, const char* k) {
    if (on && !set.f32) kernels += std::string(kernels.empty() ? "" : ",") + k;
  };
  listed(set.fuserope, "fuserope");
  listed(set.fusegeglu, "fusegeglu");
  listed(set.fuseln, "fuseln");
  warm_buckets();
}

Model::~Model() { teardown(); }

void Model::teardown() {
  // Errors here have nowhere to go, the process keeps running.
  if (stream) (void)hipStreamSynchronize(stream);
  drop_graphs();
  for (auto& r : pending) {
    (void)hipEventDestroy(r.a);
    (void)hipEventDestroy(r.b);
  }
  for (auto e : event_pool) (void)hipEventDestroy(e);
  if (wmem) (void)hipFree(wmem);
  if (rmem) (void)hipFree(rmem);
  if (amem) (void)hipFree(amem);
  if (fmem) (void)hipFree(fmem);
  if (dmeta) (void)hipFree(dmeta);
  if (hmeta) (void)hipHostFree(hmeta);
  if (hout) (void)hipHostFree(hout);
  if (stream) (void)hipStreamDestroy(stream);
  pending.clear();
  event_pool.clear();
  wmem = rmem = amem = fmem = nullptr;
  dmeta = nullptr;
  hmeta = hout = nullptr;
  stream = nullptr;
}

// One forward per (bucket length, warm row count) at load (MlxBackend::warm_buckets,
// lib.rs:1152-1173), so the first request of each shape finds its buffers and graph ready.
void Model::warm_buckets() {
  for (size_t len : set.buckets)
    for (size_t n : set.warm) {
      if (n == 0) continue;
      const uint32_t kmax = 2;
      if (len < 3) fail(kConfig, "hip settings: warm needs buckets of at least 3 tokens");
      std::vector<uint32_t> ids(n * len, 0u), mask(n * len, 1u), mpos, qt(n, 0u);
      for (size_t r = 0; r < n; ++r) mpos.insert(mpos.end(), {1u, 2u});
      std::vector<uint64_t> sl(n, len), mc(n, kmax);
      std::vector<float> lg(n * kmax), pl(n * size_t(cfg.d));
      Plan p = plan(uint32_t(n), uint32_t(len), kmax, ids.data(), mask.data(), sl.data(), mpos.data(), mc.data(),
                    qt.data());
      forward(p, lg.data(), pl.data());
    }
}

// The `clear` setting (MLX's clear_cache after every forward, lib.rs:1858-1860): give the
// activation arena, the batch staging and the captured graphs back after each call.
void Model::release() {
  hip_check(hipStreamSynchronize(stream), "sync");
  drop_graphs();
  if (amem) hip_check(hipFree(amem), "hipFree(arena)");
  if (fmem) hip_check(hipFree(fmem), "hipFree(arena)");
  if (dmeta) hip_check(hipFree(dmeta), "hipFree(meta)");
  amem = fmem = nullptr;
  dmeta = nullptr;
  acap = fcap = dmeta_cap = 0;
}

size_t Model::padded_len(size_t len) const {
  for (size_t b : set.buckets)
    if (b >= len) return b;
  return (len + set.pad - 1) / set.pad * set.pad;
}

Packed pack_batch(uint32_t n, uint32_t len, uint32_t kmax, const uint32_t* mask, const uint64_t* seq_lens,
                  const uint32_t* marker_pos, const uint64_t* marker_count, int max_pos) {
  Packed k;
  k.row_start.resize(n + 1);
  if (n == 0) return k;
  if (len == 0) fail(kBatch, "batch: len is 0 with n > 0");
  if (!mask || !seq_lens || !marker_count || (kmax && !marker_pos)) fail(kBatch, "batch: a required array is NULL");
  int64_t T = 0;
  for (uint32_t r = 0; r < n; ++r) {
    const uint64_t sl = seq_lens[r];
    if (sl == 0 || sl > len)
      fail(kBatch, "batch: seq_lens[" + std::to_string(r) + "] = " + std::to_string(sl) + " is not in 1..len");
    if (sl > uint64_t(max_pos))
      fail(kBatch, "batch: row " + std::to_string(r) + " has " + std::to_string(sl) +
                       " tokens, past max_position_embeddings " + std::to_string(max_pos));
    for (uint32_t q = 0; q < len; ++q) {
      const uint32_t want = q < sl ? 1u : 0u;
      if (mask[size_t(r) * len + q] != want)
        fail(kBatch, "batch: attention_mask of row " + std::to_string(r) +
                         " is not seq_lens ones followed by zeros (right-padded rows only)");
    }
    if (marker_count[r] > kmax) fail(kBatch, "batch: marker_count[" + std::to_string(r) + "] exceeds kmax");
    for (uint64_t j = 0; j < marker_count[r]; ++j)
      if (marker_pos[size_t(r) * kmax + j] >= sl)
        fail(kBatch, "batch: marker_pos of row " + std::to_string(r) + " points past the row");
    k.row_start[r] = int(T);
    T += int64_t(sl);
    if (T > (int64_t(1) << 30)) fail(kBatch, "batch: too many tokens");
  }
  k.row_start[n] = int(T);
  k.T = int(T);
  k.pack.reserve(size_t(T));
  k.row.reserve(size_t(T));
  for (uint32_t r = 0; r < n; ++r)
    for (uint64_t q = 0; q < seq_lens[r]; ++q) {
      k.pack.push_back(int(size_t(r) * len + q));
      k.row.push_back(int(r));
    }
  k.scorer_rows.reserve(size_t(n) * (1 + kmax));
  for (uint32_t r = 0; r < n; ++r) {
    k.scorer_rows.push_back(k.row_start[r]);
    for (uint32_t j = 0; j < kmax; ++j)
      k.scorer_rows.push_back(k.row_start[r] + (j < marker_count[r] ? int(marker_pos[size_t(r) * kmax + j]) : 0));
  }
  return k;
}

Plan Model::plan(uint32_t n, uint32_t len, uint32_t kmax, const uint32_t* ids, const uint32_t* mask,
                 const uint64_t* seq_lens, const uint32_t* marker_pos, const uint64_t* marker_count,
                 const uint32_t* qtype) const {
  Plan p;
  p.n = int(n);
  p.len = int(len);
  p.kmax = int(kmax);
  if (n == 0) return p;
  if (!ids || !qtype) fail(kBatch, "batch: a required array is NULL");
  Packed pk = pack_batch(n, len, kmax, mask, seq_lens, marker_pos, marker_count, cfg.max_pos);
  for (uint32_t r = 0; r < n; ++r)
    if (qtype[r] > 2) fail(kBatch, "batch: qtype[" + std::to_string(r) + "] is not 0, 1 or 2");
  p.row_start = pk.row_start;
  const int64_t T = pk.T;
  p.T = int(T);
  p.P = set.headprune ? int(n * (1 + kmax)) : 0;
  p.R = int(n * kmax);

  std::vector<int>& m = p.meta;
  m.reserve(size_t(3 * T) + 64);
  p.off_ids = m.size();
  for (uint32_t r = 0; r < n; ++r)
    for (uint64_t q = 0; q < seq_lens[r]; ++q) {
      const uint32_t id = ids[size_t(r) * len + q];
      if (id >= uint32_t(cfg.vocab))
        fail(kBatch, "batch: token id " + std::to_string(id) + " in row " + std::to_string(r) + " is past the vocabulary");
      m.push_back(int(id));
    }
  p.off_pos = m.size();
  for (uint32_t r = 0; r < n; ++r)
    for (uint64_t q = 0; q < seq_lens[r]; ++q) m.push_back(int(q));
  p.off_seg = m.size();
  for (uint32_t r = 0; r < n; ++r)
    for (uint64_t q = 0; q < seq_lens[r]; ++q) m.push_back(int(qtype[r]));
  auto pad4 = [&]() {
    while (m.size() % 4) m.push_back(0);
  };
  pad4();
  // Attention work tiles: query blocks of one row; for global layers 256 queries (one workgroup
  // of 8 waves), or 128 or 32 for a short batch; for local ones 128 (4 waves; their keys are only
  // the window), or 32 for a short batch.
  p.off_tiles = m.size();
  p.gq = attn_plan_tiles(p.row_start.data(), int(n), cfg.heads, -1, m);
  p.ntiles = int(m.size() - p.off_tiles) / 4;
  p.off_ltiles = m.size();
  p.lq = attn_plan_tiles(p.row_start.data(), int(n), cfg.heads, cfg.window(), m);
  p.nltiles = int(m.size() - p.off_ltiles) / 4;
  const int per = 1 + int(kmax);
  if (set.headprune) {
    p.off_ptiles = m.size();
    for (uint32_t r = 0; r < n; ++r) {
      const int s0 = int(r) * per, s1 = s0 + per;
      for (int q0 = s0; q0 < s1; q0 += 128) {
        m.push_back(q0);
        m.push_back(std::min(q0 + 128, s1));
        m.push_back(p.row_start[r]);
        m.push_back(p.row_start[r + 1]);
        ++p.nptiles;
      }
    }
    p.off_picked = m.size();
    m.insert(m.end(), pk.scorer_rows.begin(), pk.scorer_rows.end());
  }
  p.off_scorer = m.size();
  for (uint32_t r = 0; r < n; ++r)
    for (uint32_t k = 0; k < kmax; ++k) {
      if (set.headprune)
        m.push_back(int(r) * per + 1 + int(k));
      else
        m.push_back(pk.scorer_rows[size_t(r) * per + 1 + k]);
    }
  p.off_pooled = m.size();
  for (uint32_t r = 0; r < n; ++r) m.push_back(set.headprune ? int(r) * per : p.row_start[r]);
  pad4();
  if (set.f32) {
    // Every token's keys: its row (global layers), the row within the window (local layers).
    const int W = cfg.window();
    auto entries = [&](bool local) {
      for (uint32_t r = 0; r < n; ++r) {
        const int rs = p.row_start[r], re = p.row_start[r + 1];
        for (int t = rs; t < re; ++t) {
          const int e[8] = {t, local ? std::max(rs, t - W) : rs, local ? std::min(re, t + W + 1) : re, rs, rs, 0, 0, 0};
          m.insert(m.end(), e, e + 8);
        }
      }
    };
    p.off_eg = m.size();
    entries(false);
    p.off_el = m.size();
    entries(true);
  }
  return p;
}

Plan Model::plan_padded(uint32_t n, uint32_t len, const uint32_t* ids, const uint32_t* mask,
                        const uint64_t* seq_lens) const {
  Plan p;
  p.n = int(n);
  p.len = int(len);
  p.padded = true;
  if (n == 0) return p;
  if (!ids) fail(kBatch, "batch: a required array is NULL");
  const std::vector<uint64_t> no_markers(n, 0);
  (void)pack_batch(n, len, 0, mask, seq_lens, nullptr, no_markers.data(), cfg.max_pos);  // the batch checks
  if (len > uint32_t(cfg.max_pos))
    fail(kBatch, "batch: len " + std::to_string(len) + " is past max_position_embeddings " +
                     std::to_string(cfg.max_pos) + " (the padded layout gives every position a RoPE angle)");
  const int64_t T = int64_t(n) * len;
  if (T > (int64_t(1) << 30)) fail(kBatch, "batch: too many positions");
  p.T = int(T);
  p.row_start.resize(n + 1);
  for (uint32_t r = 0; r <= n; ++r) p.row_start[r] = int(r * len);
  std::vector<int>& m = p.meta;
  m.reserve(size_t(3 * T) + 64);
  p.off_ids = m.size();
  for (int64_t t = 0; t < T; ++t) {
    if (ids[t] >= uint32_t(cfg.vocab))
      fail(kBatch, "batch: token id " + std::to_string(ids[t]) + " in row " + std::to_string(t / len) +
                       " is past the vocabulary");
    m.push_back(int(ids[t]));
  }
  p.off_pos = m.size();
  for (uint32_t r = 0; r < n; ++r)
    for (uint32_t q = 0; q < len; ++q) m.push_back(int(q));
  p.off_seg = m.size();
  m.insert(m.end(), size_t(T), 0);
  auto pad4 = [&]() {
    while (m.size() % 4) m.push_back(0);
  };
  pad4();
  // Keys of a padding query at position q of a row with L real tokens (positions relative to the
  // row). Global layers: the real keys [0, L) under either mask form (lib.rs:1227-1235). Local
  // layers, by the path the reference takes for the batch's len (lib.rs:1241-1270):
  //  additive masks (the key-padding mask plus the window mask, -1e4 each): a query with a real
  //   key within the window (q < L + window) sees those keys alone, as a real token does (the
  //   local tiles take it). A farther one gets -1e4 on every key it can reach and sees them all:
  //   dense: the real keys [0, L) and the window [q - W, q + W] within the row;
  //   chunked (S = W; chunk c = q / S gathers positions (c - 1) S .. (c + 2) S - 1, clamped to
  //   the row, lib.rs:804-814): the real keys among them and the window, the window's positions
  //   past the row each one more copy of key len - 1;
  //   banded: as chunked, with zero key and value at the positions past the row (the banded
  //   layout is zero outside the sequence, split_rope.rs:18-21);
  //  boolean masks: every padding query sees every real key (dense, lib.rs:1259-1264) or every
  //   gathered slot, clamped positions included (chunked, lib.rs:1279-1291).
  const int W = cfg.window(), S = W;
  const long dense_upto = set.dense_upto >= 0 ? set.dense_upto : 4L * W;
  const bool banded = set.band > 0 && set.fuserope && !set.bool_mask && len >= set.band;
  const bool chunked = banded || (set.windowed && long(len) > dense_upto);
  std::vector<int> kend(n), lqend(n), far;
  for (uint32_t r = 0; r < n; ++r) {
    const int rs = p.row_start[r], L = int(seq_lens[r]), ln = int(len);
    kend[r] = rs + L;
    lqend[r] = rs + (set.bool_mask ? L : std::min(ln, L + W));
    for (int q = lqend[r] - rs; q < ln; ++q) {
      const int c = q / S, g0 = (c - 1) * S, g1 = (c + 2) * S;  // the chunk's gathered positions
      int e[8] = {rs + q, rs, rs, rs, rs, 0, 0, 0};
      if (set.bool_mask && !chunked) {
        e[2] = rs + L;
      } else if (set.bool_mask) {
        e[1] = rs + std::max(0, g0);
        e[2] = rs + std::min(ln, g1);
        e[5] = std::max(0, -g0);
        e[6] = std::max(0, g1 - ln);
      } else {
        const int a0 = chunked ? std::max(0, g0) : 0;
        e[1] = rs + std::min(a0, L);
        e[2] = rs + L;
        e[3] = rs + q - W;
        e[4] = rs + std::min(ln, q + W + 1);
        const int past = std::max(0, q + W + 1 - ln);  // window positions past the row
        if (banded) e[7] = past;
        else if (chunked) e[6] = past;
      }
      far.insert(far.end(), e, e + 8);
    }
  }
  p.off_tiles = m.size();
  p.gq = attn_plan_tiles(p.row_start.data(), int(n), cfg.heads, -1, m, nullptr, kend.data());
  p.ntiles = int(m.size() - p.off_tiles) / 4;
  p.off_ltiles = m.size();
  p.lq = attn_plan_tiles(p.row_start.data(), int(n), cfg.heads, W, m, lqend.data(), kend.data());
  p.nltiles = int(m.size() - p.off_ltiles) / 4;
  p.off_far = m.size();
  m.insert(m.end(), far.begin(), far.end());
  p.nfar = int(far.size() / 8);
  if (set.f32) {
    // Every position's keys in one table per layer kind: the real keys (global), the real keys
    // of the window or, past lqend, the far entry above (local).
    p.off_eg = m.size();
    for (uint32_t r = 0; r < n; ++r)
      for (int t = p.row_start[r]; t < p.row_start[r + 1]; ++t) {
        const int e[8] = {t, p.row_start[r], kend[r], p.row_start[r], p.row_start[r], 0, 0, 0};
        m.insert(m.end(), e, e + 8);
      }
    p.off_el = m.size();
    size_t fi = 0;
    for (uint32_t r = 0; r < n; ++r)
      for (int t = p.row_start[r]; t < p.row_start[r + 1]; ++t) {
        if (t < lqend[r]) {
          const int e[8] = {t, std::max(p.row_start[r], t - W), std::min(kend[r], t + W + 1), p.row_start[r],
                            p.row_start[r], 0, 0, 0};
          m.insert(m.end(), e, e + 8);
        } else {
          m.insert(m.end(), far.begin() + fi, far.begin() + fi + 8);
          fi += 8;
        }
      }
  }
  p.off_scorer = p.off_pooled = m.size();
  return p;
}

void Model::upload(const Plan& p) {
  const size_t bytes = p.meta.size() * 4;
  if (bytes > hmeta_cap) {
    if (hmeta) hip_check(hipHostFree(hmeta), "hipHostFree");
    hmeta_cap = std::max(bytes, hmeta_cap * 3 / 2);
    hip_check(hipHostMalloc(&hmeta, hmeta_cap, hipHostMallocDefault), "hipHostMalloc(meta)");
  }
  if (bytes > dmeta_cap) {
    drop_graphs();
    if (dmeta) {
      hip_check(hipStreamSynchronize(stream), "sync");
      hip_check(hipFree(dmeta), "hipFree");
    }
    dmeta_cap = std::max(bytes, dmeta_cap * 3 / 2);
    hip_check(hipMalloc(&dmeta, dmeta_cap), "hipMalloc(meta)");
  }
  // The previous request's copy out of the staging buffer has finished: every call ends with a
  // stream synchronisation.
  std::memcpy(hmeta, p.meta.data(), bytes);
  hip_check(hipMemcpyAsync(dmeta, hmeta, bytes, hipMemcpyHostToDevice, stream), "upload batch");
}

Model::Acts Model::arena(const Plan& p) {
  const size_t T = size_t(p.T), P = size_t(p.P), R = size_t(p.R), n = size_t(p.n);
  const size_t d = size_t(cfg.d), I = size_t(cfg.inter), S = size_t(scorer_width);
  const size_t midw = std::max(2 * I, 4 * d);
  // Split-K workspace: the largest of the forward's GEMMs that split (small M only).
  size_t wsf = 0;
  const int Ti = p.T, Pi = p.P, Ri = p.R, di = cfg.d, Ii = cfg.inter, Si = scorer_width;
  const int shapes[][3] = {{Ti, 3 * di, di}, {Ti, di, di}, {Ti, 2 * Ii, di}, {Ti, di, Ii}, {Ti, 4 * di, di},
                           {Ti, di, 4 * di}, {Pi, di, di}, {Pi, 4 * di, di}, {Pi, di, 4 * di}, {Ri, Si, di}};
  for (const auto& sh : shapes)
    if (sh[0] > 0) wsf = std::max(wsf, gemm_plan(sh[0], sh[1], sh[2], true).ws_floats);  // >= the unfolded plan's
  const size_t vbytes = d * size_t(vt_ld(int(T))) * 2;  // v transposed, [H, 64, ldv]
  size_t sizes[] = {T * d * 4, T * d * 2, T * d * 2, T * d * 2, vbytes, T * 3 * d * 2, T * d * 2,
                    T * midw * 2, T * I * 2, T * d * 4, T * d * 4, P * d * 4, P * d * 2, P * d * 2,
                    P * 4 * d * 2, R * d * 2, R * S * 2, R * 4, n * d * 4, wsf * 4};
  constexpr int NS = sizeof(sizes) / sizeof(sizes[0]);
  size_t off[NS], total = 0;
  for (int i = 0; i < NS; ++i) {
    off[i] = total;
    total += align256(std::max<size_t>(sizes[i], 16));
  }
  if (total > acap) {
    drop_graphs();
    if (amem) {
      hip_check(hipStreamSynchronize(stream), "sync");
      hip_check(hipFree(amem), "hipFree(arena)");
      amem = nullptr;
    }
    const size_t cap = std::max(total, acap * 3 / 2);
    hip_check(hipMalloc(&amem, cap), "hipMalloc(activations)");
    acap = cap;
  }
  char* b = static_cast<char*>(amem);
  Acts a;
  a.h = reinterpret_cast<float*>(b + off[0]);
  a.x = reinterpret_cast<uint16_t*>(b + off[1]);
  a.q = reinterpret_cast<uint16_t*>(b + off[2]);
  a.k = reinterpret_cast<uint16_t*>(b + off[3]);
  a.v = reinterpret_cast<uint16_t*>(b + off[4]);
  a.qkv = reinterpret_cast<uint16_t*>(b + off[5]);
  a.att = reinterpret_cast<uint16_t*>(b + off[6]);
  a.mid = reinterpret_cast<uint16_t*>(b + off[7]);
  a.act = reinterpret_cast<uint16_t*>(b + off[8]);
  a.enc = reinterpret_cast<float*>(b + off[9]);
  a.hh = reinterpret_cast<float*>(b + off[10]);
  a.hp = reinterpret_cast<float*>(b + off[11]);
  a.xp = reinterpret_cast<uint16_t*>(b + off[12]);
  a.attp = reinterpret_cast<uint16_t*>(b + off[13]);
  a.midp = reinterpret_cast<uint16_t*>(b + off[14]);
  a.sx = reinterpret_cast<uint16_t*>(b + off[15]);
  a.s1 = reinterpret_cast<uint16_t*>(b + off[16]);
  a.logits = reinterpret_cast<float*>(b + off[17]);
  a.pooled = reinterpret_cast<float*>(b + off[18]);
  a.ws = reinterpret_cast<float*>(b + off[19]);
  return a;
}

template <class F>
void Model::op(const char* nm, F&& f) {
  if (!set.ops) {
    f();
    return;
  }
  auto ev = [&]() {
    hipEvent_t e;
    if (!event_pool.empty()) {
      e = event_pool.back();
      event_pool.pop_back();
    } else {
      hip_check(hipEventCreate(&e), "hipEventCreate");
    }
    return e;
  };
  OpRec r{nm, ev(), ev()};
  hip_check(hipEventRecord(r.a, stream), "hipEventRecord");
  f();
  hip_check(hipEventRecord(r.b, stream), "hipEventRecord");
  pending.push_back(r);
}

// The `layers` setting (lib.rs:1555-1563, 1677-1687): an event between encoder layers, and after
// the forward one stderr line of each layer's time.
void Model::layer_mark() {
  if (!set.layers) return;
  hipEvent_t e;
  if (!event_pool.empty()) {
    e = event_pool.back();
    event_pool.pop_back();
  } else {
    hip_check(hipEventCreate(&e), "hipEventCreate");
  }
  hip_check(hipEventRecord(e, stream), "hipEventRecord");
  layer_ev.push_back(e);
}

void Model::layer_report() {
  if (layer_ev.size() >= 2) {
    std::string line = "layers us:";
    for (size_t i = 1; i < layer_ev.size(); ++i) {
      float ms = 0.0f;
      hip_check(hipEventElapsedTime(&ms, layer_ev[i - 1], layer_ev[i]), "hipEventElapsedTime");
      char b[32];
      std::snprintf(b, sizeof b, " %.1f", ms * 1e3);
      line += b;
    }
    std::fprintf(stderr, "%s\n", line.c_str());
  }
  event_pool.insert(event_pool.end(), layer_ev.begin(), layer_ev.end());
  layer_ev.clear();
}

void Model::collect_stats() {
  for (auto& r : pending) {
    float ms = 0.0f;
    hip_check(hipEventElapsedTime(&ms, r.a, r.b), "hipEventElapsedTime");
    bool found = false;
    for (auto& s : stats)
      if (s.first == r.name) {
        s.second.first += 1;
        s.second.second += ms;
        found = true;
        break;
      }
    if (!found) stats.push_back({r.name, {1, double(ms)}});
    event_pool.push_back(r.a);
    event_pool.push_back(r.b);
  }
  pending.clear();
}

namespace {

GemmArgs gemm_args(int elem, float* ws, const uint16_t* A, int lda, const uint16_t* W, int K, void* C, int ldc,
                   const float* bias, int M, int N, int epi, int act = ACT_NONE, bool reduce_folded = false) {
  GemmArgs g;
  g.elem = elem;
  g.splits = gemm_plan(M, N, K, reduce_folded).splits;
  g.ws = ws;
  g.A = A;
  g.W = W;
  g.C = C;
  g.bias = bias;
  g.M = M;
  g.N = N;
  g.K = K;
  g.lda = lda;
  g.ldw = K;
  g.ldc = ldc;
  g.epi = epi;
  g.act = act;
  if (const char* e = gemm_check(g)) fail(kBackend, e);
  return g;
}

void gemm(int elem, hipStream_t st, float* ws, const uint16_t* A, int lda, const uint16_t* W, int K, void* C, int ldc,
          const float* bias, int M, int N, int epi, int act = ACT_NONE) {
  gemm_launch(gemm_args(elem, ws, A, lda, W, K, C, ldc, bias, M, N, epi, act), st);
}

}  // namespace

int Model::run_encoder(const Plan& p, const Acts& a, bool fold_last) {
  const int T = p.T, d = cfg.d, I = cfg.inter, H = cfg.heads;
  const float eps = float(cfg.eps);
  const int* ids = dmeta + p.off_ids;
  const int* pos = dmeta + p.off_pos;
  const AttnTile* tiles = reinterpret_cast<const AttnTile*>(dmeta + p.off_tiles);
  const AttnTile* ltiles = reinterpret_cast<const AttnTile*>(dmeta + p.off_ltiles);

  // h = LN(tok_emb[ids]) (lib.rs:1534-1551); x = h for layer 0, which has no attn_norm.
  op("embed_ln", [&] { embed_ln_launch(tok_emb, ids, emb_norm, eps, T, d, a.h, a.x, stream, elem); });
  // A residual GEMM that splits K hands its partials to the kernel of the LayerNorm after it,
  // which adds them into h and writes x = LN(h); x_ready marks an attn_norm done that way.
  bool x_ready = false;
  layer_mark();
  for (int l = 0; l < cfg.layers; ++l) {
    if (l) layer_mark();
    const LayerWeights& L = layers[l];
    const int tw = L.local ? 1 : 0;
    if (L.attn_norm && !x_ready)
      op("attn_norm", [&] {
        layernorm_launch(a.h, nullptr, L.attn_norm, nullptr, eps, T, d, a.x, nullptr, nullptr, nullptr, nullptr, stream, elem);
      });
    if (set.fuserope) {
      op("wqkv_rope", [&] {
        GemmArgs g;
        g.elem = elem;
        g.A = a.x;
        g.W = L.wqkv;
        g.M = T;
        g.N = 3 * d;
        g.K = d;
        g.lda = d;
        g.ldw = d;
        g.epi = EPI_ROPE;
        g.rope_q = a.q;
        g.rope_k = a.k;
        g.rope_v = a.v;
        g.rope_pos = pos;
        g.rope_cos = rope_cos[tw];
        g.rope_sin = rope_sin[tw];
        g.rope_T = T;
        g.rope_d = d;
        g.rope_ldv = vt_ld(T);
        g.splits = gemm_plan(T, 3 * d, d).splits;
        g.ws = a.ws;
        if (const char* e = gemm_check(g)) fail(kBackend, e);
        gemm_launch(g, stream);
      });
    } else {
      op("wqkv", [&] { gemm(elem, stream, a.ws, a.x, d, L.wqkv, d, a.qkv, 3 * d, nullptr, T, 3 * d, EPI_BF16); });
      op("split_rope", [&] { split_rope_launch(a.qkv, T, d, pos, rope_cos[tw], rope_sin[tw], a.q, a.k, a.v, vt_ld(T), stream, elem); });
    }
    op(L.local ? "attn_local" : "attn_global", [&] {
      AttnArgs at;
      at.elem = elem;
      at.q = a.q;
      at.k = a.k;
      at.v = a.v;
      at.out = a.att;
      at.tiles = L.local ? ltiles : tiles;
      at.ntiles = L.local ? p.nltiles : p.ntiles;
      at.heads = H;
      at.Tq = T;
      at.Tk = T;
      at.ldv = vt_ld(T);
      at.ldo = d;
      at.scale = 1.0f / std::sqrt(float(cfg.head_dim()));
      at.window = L.local ? cfg.window() : -1;
      at.tile_q = L.local ? p.lq : p.gq;
      attn_launch(at, stream);
    });
    if (L.local && p.nfar > 0)
      op("attn_far_pad", [&] {
        FallbackArgs fa;
        fa.elem = elem;
        fa.q = a.q;
        fa.k = a.k;
        fa.v = a.v;
        fa.out = a.att;
        fa.far = dmeta + p.off_far;
        fa.nfar = p.nfar;
        fa.heads = H;
        fa.T = T;
        fa.ldv = vt_ld(T);
        fa.ldo = d;
        fa.scale = 1.0f / std::sqrt(float(cfg.head_dim()));
        attn_fallback_launch(fa, stream);
      });
    x_ready = false;
    // h = h + att . Wo^T (lib.rs:1666), x = mlp_norm(h) (lib.rs:1669)
    // Wo and Wo2 plan their split as finished by the LayerNorm after them (structurally, so the
    // fuseln=0 path splits the same way and stays bit-identical).
    const GemmArgs gwo = gemm_args(elem, a.ws, a.att, d, L.wo, d, a.h, d, nullptr, T, d, EPI_RESID, ACT_NONE, true);
    if (set.fuseln && gwo.splits > 1) {
      op("wo", [&] { gemm_launch_partials(gwo, stream); });
      op("mlp_norm", [&] { splitk_resid_ln_launch(a.ws, gwo.splits, nullptr, a.h, L.mlp_norm, eps, T, d, a.x, stream, elem); });
    } else {
      op("wo", [&] { gemm_launch(gwo, stream); });
      op("mlp_norm", [&] {
        layernorm_launch(a.h, nullptr, L.mlp_norm, nullptr, eps, T, d, a.x, nullptr, nullptr, nullptr, nullptr, stream, elem);
      });
    }
    if (set.fusegeglu) {
      op("wi_geglu", [&] { gemm(elem, stream, a.ws, a.x, d, L.wi, d, a.act, I, nullptr, T, 2 * I, EPI_GEGLU); });
    } else {
      op("wi", [&] { gemm(elem, stream, a.ws, a.x, d, L.wi, d, a.mid, 2 * I, nullptr, T, 2 * I, EPI_BF16); });
      op("geglu", [&] { geglu_launch(a.mid, T, I, a.act, stream, elem); });
    }
    // h = h + act . Wo2^T (lib.rs:1675), and the next layer's x = attn_norm(h) (lib.rs:1592-1595)
    // or, after the last layer, final_norm in the caller's kernel. Every Wo2 is planned as
    // folded, so the unfused paths split it the same way and stay bit-identical.
    const bool last = l + 1 == cfg.layers;
    const float* next_norm = last ? nullptr : layers[l + 1].attn_norm;
    const GemmArgs gwo2 = gemm_args(elem, a.ws, a.act, I, L.wo2, I, a.h, d, nullptr, T, d, EPI_RESID, ACT_NONE,
                                    next_norm != nullptr || last);
    if (set.fuseln && gwo2.splits > 1 && next_norm) {
      op("wo2", [&] { gemm_launch_partials(gwo2, stream); });
      op("attn_norm", [&] { splitk_resid_ln_launch(a.ws, gwo2.splits, nullptr, a.h, next_norm, eps, T, d, a.x, stream, elem); });
      x_ready = true;
    } else if (last && fold_last && gwo2.splits > 1) {
      op("wo2", [&] { gemm_launch_partials(gwo2, stream); });
      layer_mark();
      return gwo2.splits;
    } else {
      op("wo2", [&] { gemm_launch(gwo2, stream); });
    }
  }
  layer_mark();
  return 0;
}

// Enqueue one forward's kernels: eagerly the first time a shape is seen, then from a captured
// HIP graph (one per shape, kept until the buffers it points into move). The graph holds
// kernel nodes only; the batch tables are uploaded into the same device buffer before each
// replay, and outputs are copied after it, on the same stream.
template <class F>
void Model::run(const Plan& p, int kind, F&& enqueue) {
  if (!set.graphs || set.ops || set.layers) {
    enqueue();
    hip_check(hipGetLastError(), "kernel launch");
    return;
  }
  std::vector<int64_t> key = {kind, p.T, p.n, p.kmax, p.gq, p.lq, p.ntiles, p.nltiles, p.nptiles, p.P, p.R, int64_t(p.off_ltiles),
                              int64_t(p.off_ids), int64_t(p.off_pos), int64_t(p.off_seg), int64_t(p.off_tiles),
                              int64_t(p.off_ptiles), int64_t(p.off_picked), int64_t(p.off_scorer),
                              int64_t(p.off_pooled), int64_t(p.off_far), p.nfar, int64_t(p.padded),
                              int64_t(reinterpret_cast<intptr_t>(amem)),
                              int64_t(reinterpret_cast<intptr_t>(dmeta))};
  ++graph_clock;
  for (auto& g : graphs)
    if (g.key == key) {
      g.last_use = graph_clock;
      hip_check(hipGraphLaunch(g.exec, stream), "hipGraphLaunch");
      return;
    }
  bool seen_before = false;
  for (const auto& k : graph_seen) seen_before = seen_before || k == key;
  if (!seen_before) {
    if (graph_seen.size() >= 64) graph_seen.erase(graph_seen.begin());
    graph_seen.push_back(key);
    enqueue();
    hip_check(hipGetLastError(), "kernel launch");
    return;
  }
  hip_check(hipStreamBeginCapture(stream, hipStreamCaptureModeThreadLocal), "hipStreamBeginCapture");
  hipGraph_t graph = nullptr;
  try {
    enqueue();
  } catch (...) {
    (void)hipStreamEndCapture(stream, &graph);
    if (graph) (void)hipGraphDestroy(graph);
    throw;
  }
  hip_check(hipStreamEndCapture(stream, &graph), "hipStreamEndCapture");
  hipGraphExec_t exec = nullptr;
  const hipError_t ie = hipGraphInstantiate(&exec, graph, nullptr, nullptr, 0);
  (void)hipGraphDestroy(graph);
  hip_check(ie, "hipGraphInstantiate");
  if (graphs.size() >= kMaxGraphs) {
    size_t lru = 0;
    for (size_t i = 1; i < graphs.size(); ++i)
      if (graphs[i].last_use < graphs[lru].last_use) lru = i;
    (void)hipGraphExecDestroy(graphs[lru].exec);
    graphs.erase(graphs.begin() + lru);
  }
  graphs.push_back({key, exec, graph_clock});
  hip_check(hipGraphLaunch(exec, stream), "hipGraphLaunch");
}

void Model::drop_graphs() {
  for (auto& g : graphs) (void)hipGraphExecDestroy(g.exec);
  graphs.clear();
  graph_seen.clear();
}

void Model::enqueue_forward(const Plan& p, const Acts& a) {
  const int T = p.T, d = cfg.d, P = p.P, R = p.R, n = p.n, S = scorer_width;
  const float eps = float(cfg.eps);
  const int* seg = dmeta + p.off_seg;
  const int nh = cfg.head_layers;
  // final_norm (lib.rs:1689), then h + type_emb[qtype] per row (lib.rs:1702-1709) in one pass.
  // With fuseln the same kernel first adds the last Wo2's split-K partials into h and then writes
  // the first head layer's x = norm1(h) (lib.rs:1726): three kernels in one.
  bool hx_ready = false;   // x = norm1(h) of this head layer already written
  bool head_done = false;  // the scorer's LayerNorm and the pooled rows already written
  if (set.fuseln) {
    const int pending = run_encoder(p, a, true);
    op("final_norm", [&] {
      encoder_end_launch(a.ws, pending, a.h, final_norm, eps, type_emb, seg, a.hh, nh ? head[0].n1w : nullptr,
                         nh ? head[0].n1b : nullptr, 1e-5f, nh ? a.x : nullptr, T, d, stream, elem);
    });
    hx_ready = nh > 0;
  } else {
    run_encoder(p, a);
    op("final_norm", [&] {
      layernorm_launch(a.h, nullptr, final_norm, nullptr, eps, T, d, nullptr, nullptr, type_emb, seg, a.hh, stream, elem);
    });
  }
  const AttnTile* tiles = reinterpret_cast<const AttnTile*>(dmeta + p.off_tiles);
  const float hscale = 1.0f / std::sqrt(float(d / cfg.head_nheads()));  // head_scale (lib.rs:576-578)
  // A residual GEMM g into hbuf, then y = LN(hbuf) (weight w, bias b) over M rows: when g splits
  // K and fuseln is on, the LayerNorm's kernel sums the partials (and g's bias) into hbuf first.
  auto resid_then_ln = [&](const char* gname, const char* lname, const GemmArgs& g, float* hbuf, const float* w,
                           const float* b, int M, uint16_t* y) {
    if (set.fuseln && g.splits > 1) {
      op(gname, [&] { gemm_launch_partials(g, stream); });
      op(lname, [&] { splitk_resid_ln_launch(a.ws, g.splits, g.bias, hbuf, w, 1e-5f, M, d, y, stream, elem, b); });
    } else {
      op(gname, [&] { gemm_launch(g, stream); });
      op(lname, [&] {
        layernorm_launch(hbuf, nullptr, w, b, 1e-5f, M, d, y, nullptr, nullptr, nullptr, nullptr, stream, elem);
      });
    }
  };
  // As in the encoder, a residual GEMM that splits K hands its partials to the kernel of the
  // LayerNorm after it (out_proj -> norm2, linear2 -> the next layer's norm1); the split is
  // planned as folded on both paths, so fuseln=0 splits the same way and stays bit-identical.
  for (int j = 0; j < nh; ++j) {
    const HeadWeights& Hw = head[j];
    const bool pruned = set.headprune && j + 1 == nh;
    // x = norm1(h); qkv = x . in_proj^T + b; split heads (lib.rs:1726-1741)
    if (!hx_ready)
      op("head_norm1", [&] {
        layernorm_launch(a.hh, nullptr, Hw.n1w, Hw.n1b, 1e-5f, T, d, a.x, nullptr, nullptr, nullptr, nullptr, stream, elem);
      });
    hx_ready = false;
    // in_proj + bias with the head split fused in its epilogue (no rotation in the head)
    op("head_in_proj", [&] {
      GemmArgs g;
      g.elem = elem;
      g.A = a.x;
      g.W = Hw.in_w;
      g.bias = Hw.in_b;
      g.M = T;
      g.N = 3 * d;
      g.K = d;
      g.lda = d;
      g.ldw = d;
      g.epi = EPI_ROPE;
      g.rope_q = a.q;
      g.rope_k = a.k;
      g.rope_v = a.v;
      g.rope_T = T;
      g.rope_d = d;
      g.rope_ldv = vt_ld(T);
      g.splits = gemm_plan(T, 3 * d, d).splits;
      g.ws = a.ws;
      if (const char* e = gemm_check(g)) fail(kBackend, e);
      gemm_launch(g, stream);
    });
    if (!pruned) {
      op("head_attn", [&] {
        AttnArgs at;
        at.elem = elem;
        at.q = a.q;
        at.k = a.k;
        at.v = a.v;
        at.out = a.att;
        at.tiles = tiles;
        at.ntiles = p.ntiles;
        at.tile_q = p.gq;
        at.heads = cfg.head_nheads();
        at.Tq = T;
        at.Tk = T;
        at.ldv = vt_ld(T);
        at.ldo = d;
        at.scale = hscale;
        attn_launch(at, stream);
      });
      resid_then_ln("head_out_proj", "head_norm2", gemm_args(elem, a.ws, a.att, d, Hw.out_w, d, a.hh, d, Hw.out_b, T, d,
                                                             EPI_RESID, ACT_NONE, true),
                    a.hh, Hw.n2w, Hw.n2b, T, a.x);
      op("head_linear1", [&] { gemm(elem, stream, a.ws, a.x, d, Hw.l1_w, d, a.mid, 4 * d, Hw.l1_b, T, 4 * d, EPI_BF16, ACT_RELU); });
      // linear2, and the next head layer's norm1 (lib.rs:1726) when the split folds into it
      const GemmArgs gl2 = gemm_args(elem, a.ws, a.mid, 4 * d, Hw.l2_w, 4 * d, a.hh, d, Hw.l2_b, T, d, EPI_RESID, ACT_NONE,
                                     j + 1 < nh);
      if (set.fuseln && gl2.splits > 1 && j + 1 < nh) {
        op("head_linear2", [&] { gemm_launch_partials(gl2, stream); });
        op("head_norm1", [&] {
          splitk_resid_ln_launch(a.ws, gl2.splits, Hw.l2_b, a.hh, head[j + 1].n1w, 1e-5f, T, d, a.x, stream, elem,
                                 head[j + 1].n1b);
        });
        hx_ready = true;
      } else {
        op("head_linear2", [&] { gemm_launch(gl2, stream); });
      }
    } else {
      // headprune (lib.rs:1728-1748): every token supplies k and v; queries, out_proj, norm2 and
      // the FFN run at rows {0, markers} only.
      const int* picked = dmeta + p.off_picked;
      op("head_attn", [&] {
        AttnArgs at;
        at.elem = elem;
        at.q = a.q;
        at.k = a.k;
        at.v = a.v;
        at.out = a.attp;
        at.tiles = reinterpret_cast<const AttnTile*>(dmeta + p.off_ptiles);
        at.ntiles = p.nptiles;
        // A row's picked slots are one tile (up to 128); up to 32 of them take 8 waves that
        // split the keys, since these tiles are few.
        at.tile_q = 1 + p.kmax <= 32 ? 32 : 128;
        at.key_waves = 8;
        at.qkey = picked;
        at.heads = cfg.head_nheads();
        at.Tq = T;
        at.Tk = T;
        at.ldv = vt_ld(T);
        at.ldo = d;
        at.scale = hscale;
        attn_launch(at, stream);
      });
      // The residual of the picked rows: gathered from h, or, when out_proj's split folds into
      // norm2's kernel, read by that kernel from h through the picked-row index.
      const GemmArgs gop = gemm_args(elem, a.ws, a.attp, d, Hw.out_w, d, a.hp, d, Hw.out_b, P, d, EPI_RESID, ACT_NONE, true);
      if (set.fuseln && gop.splits > 1) {
        op("head_out_proj", [&] { gemm_launch_partials(gop, stream); });
        op("head_norm2", [&] {
          splitk_resid_ln_launch(a.ws, gop.splits, gop.bias, a.hp, Hw.n2w, 1e-5f, P, d, a.xp, stream, elem, Hw.n2b, a.hh,
                                 picked);
        });
      } else {
        op("head_pick", [&] { gather_f32_launch(a.hh, picked, P, d, a.hp, stream); });
        resid_then_ln("head_out_proj", "head_norm2", gop, a.hp, Hw.n2w, Hw.n2b, P, a.xp);
      }
      op("head_linear1", [&] { gemm(elem, stream, a.ws, a.xp, d, Hw.l1_w, d, a.midp, 4 * d, Hw.l1_b, P, 4 * d, EPI_BF16, ACT_RELU); });
      // linear2, planned as folded on both paths: with fuseln its split-K partials, the scorer's
      // LayerNorm and the pooled rows finish in one kernel after it (head_end_launch).
      const GemmArgs gl2 = gemm_args(elem, a.ws, a.midp, 4 * d, Hw.l2_w, 4 * d, a.hp, d, Hw.l2_b, P, d, EPI_RESID, ACT_NONE,
                                     true);
      if (set.fuseln) {
        if (gl2.splits > 1) op("head_linear2", [&] { gemm_launch_partials(gl2, stream); });
        else op("head_linear2", [&] { gemm_launch(gl2, stream); });
        op("scorer_norm", [&] {
          head_end_launch(a.ws, gl2.splits > 1 ? gl2.splits : 0, gl2.bias, a.hp, 1 + p.kmax, sc0_w, sc0_b, 1e-5f, a.pooled,
                          a.sx, P, d, stream, elem);
        });
        head_done = true;
      } else {
        op("head_linear2", [&] { gemm_launch(gl2, stream); });
      }
    }
  }
  // score (lib.rs:1768-1800): LN_b at the marker rows, scorer1 + GELU, scorer3; pooled row 0.
  // head_done: the LayerNorm and the pooled rows are already written.
  const float* src = set.headprune ? a.hp : a.hh;
  const int* srows = dmeta + p.off_scorer;
  const int* prows = dmeta + p.off_pooled;
  if (R > 0) {
    if (!head_done)
      op("scorer_norm", [&] {
        layernorm_launch(src, srows, sc0_w, sc0_b, 1e-5f, R, d, a.sx, nullptr, nullptr, nullptr, nullptr, stream, elem);
      });
    op("scorer1", [&] { gemm(elem, stream, a.ws, a.sx, d, sc1_w, d, a.s1, S, sc1_b, R, S, EPI_BF16, ACT_GELU); });
    op("scorer3", [&] { rowdot_launch(a.s1, sc3_w, sc3_b, R, S, a.logits, stream, elem); });
  }
  if (!head_done) op("pooled", [&] { gather_f32_launch(src, prows, n, d, a.pooled, stream); });
}

void Model::forward(const Plan& p, float* logits_out, float* pooled_out) {
  if (p.n == 0) return;
  if (set.f32) {
    forward32(p, logits_out, pooled_out);
    return;
  }
  const auto t0 = std::chrono::steady_clock::now();
  hip_check(hipSetDevice(device), "hipSetDevice");
  upload(p);
  Acts a = arena(p);
  const int d = cfg.d, R = p.R, n = p.n;
  run(p, 0, [&] { enqueue_forward(p, a); });
  hip_check(hipGetLastError(), "kernel launch");

  const size_t out_bytes = size_t(R) * 4 + size_t(n) * d * 4;
  if (out_bytes > hout_cap) {
    if (hout) hip_check(hipHostFree(hout), "hipHostFree");
    hout_cap = std::max(out_bytes, hout_cap * 3 / 2);
    hip_check(hipHostMalloc(&hout, hout_cap, hipHostMallocDefault), "hipHostMalloc(out)");
  }
  float* hl = static_cast<float*>(hout);
  float* hpool = hl + R;
  if (R > 0) hip_check(hipMemcpyAsync(hl, a.logits, size_t(R) * 4, hipMemcpyDeviceToHost, stream), "download logits");
  hip_check(hipMemcpyAsync(hpool, a.pooled, size_t(n) * d * 4, hipMemcpyDeviceToHost, stream), "download pooled");
  hip_check(hipStreamSynchronize(stream), "forward");
  if (set.ops) collect_stats();
  if (set.layers) layer_report();
  std::memcpy(logits_out, hl, size_t(R) * 4);
  std::memcpy(pooled_out, hpool, size_t(n) * d * 4);
  if (set.trace) {
    const double us = std::chrono::duration<double, std::micro>(std::chrono::steady_clock::now() - t0).count();
    std::fprintf(stderr, "forward n=%d len=%d T=%d us=%.1f\n", p.n, p.len, p.T, us);
  }
  if (set.clear) release();
}

void Model::encoder_hidden(const Plan& p, float* hidden) {
  if (p.n == 0) return;
  if (!p.padded) fail(kBackend, "encoder_hidden: the plan is not the padded layout");
  if (set.f32) {
    encoder_hidden32(p, hidden);
    return;
  }
  hip_check(hipSetDevice(device), "hipSetDevice");
  upload(p);
  Acts a = arena(p);
  const int T = p.T, d = cfg.d;
  run(p, 1, [&] {
    run_encoder(p, a);
    op("final_norm", [&] {
      layernorm_launch(a.h, nullptr, final_norm, nullptr, float(cfg.eps), T, d, nullptr, a.enc, nullptr, nullptr,
                       nullptr, stream, elem);
    });
  });
  // The padded layout's rows are the [n, len] positions in order: [T, d] is [n, len, d].
  hip_check(hipMemcpyAsync(hidden, a.enc, size_t(T) * d * 4, hipMemcpyDeviceToHost, stream), "download hidden");
  hip_check(hipStreamSynchronize(stream), "encoder_hidden");
  if (set.ops) collect_stats();
  if (set.layers) layer_report();
  if (set.clear) release();
}

// ---- dtype=f32 (BackendOptions::f32, backend.rs:25-27): the same graph with f32 weights and
// activations on the plain f32 kernels, eagerly enqueued (no graphs, no fused kernels, the
// head's last layer over every row). Every attention query reads its key set from the plan's
// entry tables.

struct Model::Acts32 {
  float *h, *x, *qkv, *q, *k, *v, *att, *mid, *act, *enc, *hh, *sx, *s1, *logits, *pooled;
};

Model::Acts32 Model::arena32(const Plan& p) {
  const size_t T = size_t(p.T), R = size_t(p.R), n = size_t(p.n);
  const size_t d = size_t(cfg.d), I = size_t(cfg.inter), S = size_t(scorer_width);
  const size_t sizes[] = {T * d, T * d, T * 3 * d, T * d, T * d, T * d, T * d, T * std::max(2 * I, 4 * d), T * I,
                          T * d, T * d, R * d, R * S, R, n * d};
  constexpr int NS = sizeof(sizes) / sizeof(sizes[0]);
  size_t off[NS], total = 0;
  for (int i = 0; i < NS; ++i) {
    off[i] = total;
    total += align256(std::max<size_t>(sizes[i] * 4, 16));
  }
  if (total > fcap) {
    if (fmem) {
      hip_check(hipStreamSynchronize(stream), "sync");
      hip_check(hipFree(fmem), "hipFree(arena)");
      fmem = nullptr;
    }
    const size_t cap = std::max(total, fcap * 3 / 2);
    hip_check(hipMalloc(&fmem, cap), "hipMalloc(activations)");
    fcap = cap;
  }
  float* b[NS];
  for (int i = 0; i < NS; ++i) b[i] = reinterpret_cast<float*>(static_cast<char*>(fmem) + off[i]);
  return Acts32{b[0], b[1], b[2], b[3], b[4], b[5], b[6], b[7], b[8], b[9], b[10], b[11], b[12], b[13], b[14]};
}

namespace {

// C (+)= act(A . W^T + bias) on the f32 GEMM, shapes checked first.
void gemm32(const float* A, int lda, const float* W, int ldw, float* C, int ldc, const float* bias, int M, int N, int K,
            int act, bool accumulate, hipStream_t st) {
  Gemm32Args g;
  g.A = A;
  g.W = W;
  g.C = C;
  g.bias = bias;
  g.M = M;
  g.N = N;
  g.K = K;
  g.lda = lda;
  g.ldw = ldw;
  g.ldc = ldc;
  g.act = act;
  g.accumulate = accumulate;
  if (const char* e = gemm32_check(g)) fail(kBackend, e);
  gemm32_launch(g, st);
}

}  // namespace

// encode (lib.rs:1525-1693) in f32 over the plan's rows; a.h holds the residual stream after it.
void Model::run_encoder32(const Plan& p, const Acts32& a) {
  const int T = p.T, d = cfg.d, I = cfg.inter, H = cfg.heads;
  const float eps = float(cfg.eps);
  const int* ids = dmeta + p.off_ids;
  const int* pos = dmeta + p.off_pos;
  // h = LN(tok_emb[ids]) (lib.rs:1534-1551)
  op("embed", [&] {
    gather_f32_launch(w32(tok_emb), ids, T, d, a.x, stream);
    layernorm_launch(a.x, nullptr, emb_norm, nullptr, eps, T, d, nullptr, a.h, nullptr, nullptr, nullptr, stream, elem);
  });
  for (int l = 0; l < cfg.layers; ++l) {
    const LayerWeights& L = layers[l];
    const int tw = L.local ? 1 : 0;
    const float* xin = a.h;  // layer 0 attends from the embedding itself
    if (l > 0) {
      op("attn_norm", [&] {
        layernorm_launch(a.h, nullptr, L.attn_norm, nullptr, eps, T, d, nullptr, a.x, nullptr, nullptr, nullptr, stream,
                         elem);
      });
      xin = a.x;
    }
    op("wqkv", [&] { gemm32(xin, d, w32(L.wqkv), d, a.qkv, 3 * d, nullptr, T, 3 * d, d, ACT_NONE, false, stream); });
    op("split_rope", [&] { split32_launch(a.qkv, T, d, pos, rope_cos[tw], rope_sin[tw], a.q, a.k, a.v, stream); });
    op(L.local ? "attn_local" : "attn_global", [&] {
      Attn32Args at;
      at.q = a.q;
      at.k = a.k;
      at.v = a.v;
      at.out = a.att;
      at.entries = dmeta + (L.local ? p.off_el : p.off_eg);
      at.n = T;
      at.heads = H;
      at.T = T;
      at.ldo = d;
      at.scale = 1.0f / std::sqrt(float(cfg.head_dim()));
      attn32_launch(at, stream);
    });
    op("wo", [&] { gemm32(a.att, d, w32(L.wo), d, a.h, d, nullptr, T, d, d, ACT_NONE, true, stream); });
    op("mlp_norm", [&] {
      layernorm_launch(a.h, nullptr, L.mlp_norm, nullptr, eps, T, d, nullptr, a.x, nullptr, nullptr, nullptr, stream, elem);
    });
    op("wi", [&] { gemm32(a.x, d, w32(L.wi), d, a.mid, 2 * I, nullptr, T, 2 * I, d, ACT_NONE, false, stream); });
    op("geglu", [&] { geglu32_launch(a.mid, T, I, a.act, stream); });
    op("wo2", [&] { gemm32(a.act, I, w32(L.wo2), I, a.h, d, nullptr, T, d, I, ACT_NONE, true, stream); });
    layer_mark();
  }
}

void Model::forward32(const Plan& p, float* logits_out, float* pooled_out) {
  const auto t0 = std::chrono::steady_clock::now();
  hip_check(hipSetDevice(device), "hipSetDevice");
  upload(p);
  Acts32 a = arena32(p);
  const int T = p.T, d = cfg.d, R = p.R, n = p.n, S = scorer_width;
  const int Hh = cfg.head_nheads();
  const float hscale = 1.0f / std::sqrt(float(d / Hh));  // head_scale (lib.rs:576-578)
  layer_mark();
  run_encoder32(p, a);
  // final_norm, then the head stream hh = enc + type_emb[qtype] (lib.rs:1689, 1700-1703)
  op("final_norm", [&] {
    layernorm_launch(a.h, nullptr, final_norm, nullptr, float(cfg.eps), T, d, nullptr, a.enc, type_emb, dmeta + p.off_seg,
                     a.hh, stream, elem);
  });
  // head_forward (lib.rs:1698-1765): pre-norm layers with biases, ReLU FFN, every row
  for (int j = 0; j < cfg.head_layers; ++j) {
    const HeadWeights& Hw = head[j];
    op("head_norm1", [&] {
      layernorm_launch(a.hh, nullptr, Hw.n1w, Hw.n1b, 1e-5f, T, d, nullptr, a.x, nullptr, nullptr, nullptr, stream, elem);
    });
    op("head_in_proj", [&] { gemm32(a.x, d, w32(Hw.in_w), d, a.qkv, 3 * d, Hw.in_b, T, 3 * d, d, ACT_NONE, false, stream); });
    op("head_split", [&] { split32_launch(a.qkv, T, d, nullptr, nullptr, nullptr, a.q, a.k, a.v, stream); });
    op("head_attn", [&] {
      Attn32Args at;
      at.q = a.q;
      at.k = a.k;
      at.v = a.v;
      at.out = a.att;
      at.entries = dmeta + p.off_eg;
      at.n = T;
      at.heads = Hh;
      at.T = T;
      at.ldo = d;
      at.scale = hscale;
      attn32_launch(at, stream);
    });
    op("head_out_proj", [&] { gemm32(a.att, d, w32(Hw.out_w), d, a.hh, d, Hw.out_b, T, d, d, ACT_NONE, true, stream); });
    op("head_norm2", [&] {
      layernorm_launch(a.hh, nullptr, Hw.n2w, Hw.n2b, 1e-5f, T, d, nullptr, a.x, nullptr, nullptr, nullptr, stream, elem);
    });
    op("head_linear1",
       [&] { gemm32(a.x, d, w32(Hw.l1_w), d, a.mid, 4 * d, Hw.l1_b, T, 4 * d, d, ACT_RELU, false, stream); });
    op("head_linear2",
       [&] { gemm32(a.mid, 4 * d, w32(Hw.l2_w), 4 * d, a.hh, d, Hw.l2_b, T, d, 4 * d, ACT_NONE, true, stream); });
  }
  // score (lib.rs:1768-1800): LayerNorm with bias at the marker rows, scorer1 + exact GELU,
  // scorer3; pooled = position 0 of each row
  if (R > 0) {
    op("scorer_norm", [&] {
      layernorm_launch(a.hh, dmeta + p.off_scorer, sc0_w, sc0_b, 1e-5f, R, d, nullptr, a.sx, nullptr, nullptr, nullptr,
                       stream, elem);
    });
    op("scorer1", [&] { gemm32(a.sx, d, w32(sc1_w), d, a.s1, S, sc1_b, R, S, d, ACT_GELU, false, stream); });
    op("scorer3", [&] { gemm32(a.s1, S, sc3_w, S, a.logits, 1, sc3_b, R, 1, S, ACT_NONE, false, stream); });
  }
  op("pooled", [&] { gather_f32_launch(a.hh, dmeta + p.off_pooled, n, d, a.pooled, stream); });
  hip_check(hipGetLastError(), "kernel launch");
  if (R > 0) hip_check(hipMemcpyAsync(logits_out, a.logits, size_t(R) * 4, hipMemcpyDeviceToHost, stream), "download logits");
  hip_check(hipMemcpyAsync(pooled_out, a.pooled, size_t(n) * d * 4, hipMemcpyDeviceToHost, stream), "download pooled");
  hip_check(hipStreamSynchronize(stream), "forward");
  if (set.ops) collect_stats();
  if (set.layers) layer_report();
  if (set.trace) {
    const double us = std::chrono::duration<double, std::micro>(std::chrono::steady_clock::now() - t0).count();
    std::fprintf(stderr, "forward n=%d len=%d T=%d us=%.1f\n", p.n, p.len, p.T, us);
  }
  if (set.clear) release();
}

void Model::encoder_hidden32(const Plan& p, float* hidden) {
  hip_check(hipSetDevice(device), "hipSetDevice");
  upload(p);
  Acts32 a = arena32(p);
  const int T = p.T, d = cfg.d;
  layer_mark();
  run_encoder32(p, a);
  op("final_norm", [&] {
    layernorm_launch(a.h, nullptr, final_norm, nullptr, float(cfg.eps), T, d, nullptr, a.enc, nullptr, nullptr, nullptr,
                     stream, elem);
  });
  hip_check(hipGetLastError(), "kernel launch");
  hip_check(hipMemcpyAsync(hidden, a.enc, size_t(T) * d * 4, hipMemcpyDeviceToHost, stream), "download hidden");
  hip_check(hipStreamSynchronize(stream), "encoder_hidden");
  if (set.ops) collect_stats();
  if (set.layers) layer_report();
  if (set.clear) release();
}

}  // namespace s1
