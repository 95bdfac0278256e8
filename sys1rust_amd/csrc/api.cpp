// The C ABI of libsys1hip (include/sys1hip.h). Every entry point catches all exceptions and
// turns them into an error kind plus a thread-local message; nothing aborts.
#include "sys1hip.h"

#include <fstream>
#include <memory>
#include <mutex>
#include <new>

#include "kernels.hpp"
#include "model.hpp"
#include "synth.hpp"

struct s1_model {
  std::unique_ptr<s1::Model> m;
};

namespace {

thread_local std::string g_err;

int set_err(int kind, const std::string& msg) {
  g_err = msg;
  return kind;
}

template <class F>
int guard(F&& f) {
  try {
    f();
    return S1_OK;
  } catch (const s1::Error& e) {
    return set_err(e.kind, e.what());
  } catch (const std::bad_alloc&) {
    return set_err(S1_ERR_BACKEND, "out of host memory");
  } catch (const std::exception& e) {
    return set_err(S1_ERR_BACKEND, e.what());
  } catch (...) {
    return set_err(S1_ERR_BACKEND, "unknown error");
  }
}

std::string str_or_empty(const char* s) { return s ? std::string(s) : std::string(); }

// `tensors` parses (or checks) the caller's weights; it runs inside the guard so that its errors
// come back as error kinds too.
template <class MakeTensors>
int create(MakeTensors&& tensors, const char* enc, const char* agent, const char* settings, int dev, s1_model** out) {
  if (out) *out = nullptr;
  return guard([&] {
    if (!out) s1::fail(s1::kConfig, "s1_model_create: out is NULL");
    if (!enc) s1::fail(s1::kConfig, "s1_model_create: encoder_config_json is NULL");
    // Settings first: a bad settings string is reported as such whatever the weights hold.
    (void)s1::Settings::parse(str_or_empty(settings));
    const s1::SafeTensors st = tensors();
    auto h = std::make_unique<s1_model>();
    h->m = std::make_unique<s1::Model>(st, enc, str_or_empty(agent), str_or_empty(settings), dev);
    *out = h.release();
  });
}

void hip_ok(hipError_t e, const char* what) {
  if (e != hipSuccess) s1::fail(s1::kBackend, std::string(what) + ": " + hipGetErrorString(e));
}

}  // namespace

extern "C" {

int s1_model_create(const char* path, const char* enc, const char* agent, const char* settings, int dev,
                    s1_model** out) {
  std::vector<uint8_t> bytes;
  int rc = guard([&] {
    if (!path) s1::fail(s1::kWeights, "s1_model_create: safetensors_path is NULL");
    std::ifstream f(path, std::ios::binary | std::ios::ate);
    if (!f) s1::fail(s1::kWeights, std::string(path) + ": cannot open");
    std::streamsize sz = f.tellg();
    f.seekg(0);
    bytes.resize(size_t(sz));
    if (sz && !f.read(reinterpret_cast<char*>(bytes.data()), sz)) s1::fail(s1::kWeights, std::string(path) + ": read failed");
  });
  if (rc) {
    if (out) *out = nullptr;
    return rc;
  }
  return create([&] { return s1::SafeTensors(bytes.data(), bytes.size(), path); }, enc, agent, settings, dev, out);
}

int s1_model_create_from_bytes(const void* b, size_t n, const char* enc, const char* agent, const char* settings,
                               int dev, s1_model** out) {
  if (!b) {
    if (out) *out = nullptr;
    return set_err(S1_ERR_WEIGHTS, "s1_model_create_from_bytes: bytes is NULL");
  }
  return create([&] { return s1::SafeTensors(static_cast<const uint8_t*>(b), n, "model.safetensors"); }, enc, agent,
                settings, dev, out);
}

int s1_model_create_from_tensors(const s1_tensor* tensors, size_t count, const char* enc, const char* agent,
                                 const char* settings, int dev, s1_model** out) {
  return create(
      [&] {
        if (!tensors && count) s1::fail(s1::kWeights, "s1_model_create_from_tensors: tensors is NULL");
        std::vector<std::pair<std::string, s1::TensorView>> v;
        v.reserve(count);
        for (size_t i = 0; i < count; ++i) {
          const s1_tensor& t = tensors[i];
          if (!t.name) s1::fail(s1::kWeights, "s1_model_create_from_tensors: tensor " + std::to_string(i) + " has no name");
          s1::TensorView tv;
          switch (t.dtype) {
            case S1_DTYPE_F32: tv.dtype = s1::DType::F32; break;
            case S1_DTYPE_F16: tv.dtype = s1::DType::F16; break;
            case S1_DTYPE_BF16: tv.dtype = s1::DType::BF16; break;
            case S1_DTYPE_F64: tv.dtype = s1::DType::F64; break;
            default:
              s1::fail(s1::kWeights, std::string("tensor '") + t.name + "': unsupported dtype " + std::to_string(t.dtype));
          }
          if (t.ndim && !t.shape) s1::fail(s1::kWeights, std::string("tensor '") + t.name + "': shape is NULL");
          for (uint32_t k = 0; k < t.ndim; ++k) {
            if (t.shape[k] > uint64_t(INT64_MAX)) s1::fail(s1::kWeights, std::string("tensor '") + t.name + "' has a bad shape");
            tv.shape.push_back(int64_t(t.shape[k]));
          }
          tv.data = static_cast<const uint8_t*>(t.data);
          tv.nbytes = t.nbytes;
          v.emplace_back(t.name, tv);
        }
        return s1::SafeTensors(v, "model.safetensors");
      },
      enc, agent, settings, dev, out);
}

int s1_check_settings(const char* settings) {
  return guard([&] { (void)s1::Settings::parse(str_or_empty(settings)); });
}

int s1_forward(s1_model* h, uint32_t n, uint32_t len, uint32_t kmax, const uint32_t* ids, const uint32_t* mask,
               const uint64_t* seq_lens, const uint32_t* marker_pos, const uint64_t* marker_count,
               const uint32_t* qtype, float* logits, float* pooled) {
  return guard([&] {
    if (!h || !h->m) s1::fail(s1::kBackend, "s1_forward: model is NULL");
    if (n && ((kmax && !logits) || !pooled)) s1::fail(s1::kBatch, "s1_forward: an output buffer is NULL");
    s1::Plan p = h->m->plan(n, len, kmax, ids, mask, seq_lens, marker_pos, marker_count, qtype);
    h->m->forward(p, logits, pooled);
    // forward (lib.rs:1852-1856): logits past a row's marker count are LOGIT_MASKED.
    for (uint32_t r = 0; r < n; ++r)
      for (uint64_t k = marker_count[r]; k < kmax; ++k) logits[size_t(r) * kmax + k] = -1e4f;
  });
}

int s1_encoder_hidden(s1_model* h, uint32_t n, uint32_t len, uint32_t kmax, const uint32_t* ids, const uint32_t* mask,
                      const uint64_t* seq_lens, const uint32_t* marker_pos, const uint64_t* marker_count,
                      const uint32_t* qtype, float* hidden) {
  return guard([&] {
    if (!h || !h->m) s1::fail(s1::kBackend, "s1_encoder_hidden: model is NULL");
    if (n && !hidden) s1::fail(s1::kBatch, "s1_encoder_hidden: hidden_out is NULL");
    (void)kmax;
    (void)marker_pos;
    (void)marker_count;
    (void)qtype;
    s1::Plan p = h->m->plan_padded(n, len, ids, mask, seq_lens);
    h->m->encoder_hidden(p, hidden);
  });
}

size_t s1_padded_len(const s1_model* h, size_t len, size_t rows) {
  (void)rows;
  if (!h || !h->m) return len;
  return h->m->padded_len(len);
}

const char* s1_name(const s1_model* h) { return (h && h->m) ? h->m->name.c_str() : ""; }

const char* s1_active_kernels(const s1_model* h) { return (h && h->m) ? h->m->kernels.c_str() : ""; }

int s1_warmup(s1_model* h) {
  return guard([&] {
    if (!h || !h->m) s1::fail(s1::kBackend, "s1_warmup: model is NULL");
    s1::Model& m = *h->m;
    // One 64-token row with two markers: touches every kernel of the forward once.
    const uint32_t len = 64, kmax = 2;
    std::vector<uint32_t> ids(len), mask(len, 1u), mpos = {1, 2}, qt = {0};
    for (uint32_t i = 0; i < len; ++i) ids[i] = i % uint32_t(m.cfg.vocab);
    std::vector<uint64_t> sl = {len}, mc = {kmax};
    std::vector<float> lg(kmax), pl(size_t(m.cfg.d));
    s1::Plan p = m.plan(1, len, kmax, ids.data(), mask.data(), sl.data(), mpos.data(), mc.data(), qt.data());
    m.forward(p, lg.data(), pl.data());
  });
}

const char* s1_last_error(void) { return g_err.c_str(); }

void s1_model_destroy(s1_model* h) { delete h; }

int s1_synth_checkpoint(const char* enc, const char* agent, uint64_t seed, int scorer_width, int n_act, int jitter,
                        void* out, size_t cap, size_t* len) {
  return guard([&] {
    if (!enc) s1::fail(s1::kConfig, "s1_synth_checkpoint: encoder_config_json is NULL");
    if (!len) s1::fail(s1::kConfig, "s1_synth_checkpoint: len is NULL");
    if (scorer_width <= 0 || n_act <= 0) s1::fail(s1::kConfig, "s1_synth_checkpoint: scorer_width and n_act must be positive");
    s1::ModelConfig c = s1::parse_model_config(enc, str_or_empty(agent));
    if (!out) {
      // Size only: header + payload, computed without generating values.
      std::vector<s1::TensorSpec> lay = s1::checkpoint_layout(c, scorer_width, n_act);
      std::vector<s1::OutTensor> shell;
      for (auto& t : lay) shell.push_back({t.name, t.shape, {}});
      *len = s1::write_safetensors_bf16(shell).size();
      return;
    }
    std::vector<uint8_t> b = s1::synth_checkpoint(c, seed, scorer_width, n_act, jitter != 0);
    *len = b.size();
    if (cap < b.size()) s1::fail(s1::kConfig, "s1_synth_checkpoint: buffer too small");
    std::memcpy(out, b.data(), b.size());
  });
}

int s1_pack_tables(uint32_t n, uint32_t len, uint32_t kmax, const uint32_t* mask, const uint64_t* seq_lens,
                   const uint32_t* marker_pos, const uint64_t* marker_count, int32_t* row_start, int32_t* pack,
                   int32_t* row, int32_t* scorer_rows, uint32_t* t_out) {
  return guard([&] {
    s1::Packed k = s1::pack_batch(n, len, kmax, mask, seq_lens, marker_pos, marker_count, 1 << 30);
    if (row_start) std::copy(k.row_start.begin(), k.row_start.end(), row_start);
    if (pack) std::copy(k.pack.begin(), k.pack.end(), pack);
    if (row) std::copy(k.row.begin(), k.row.end(), row);
    if (scorer_rows) std::copy(k.scorer_rows.begin(), k.scorer_rows.end(), scorer_rows);
    if (t_out) *t_out = uint32_t(k.T);
  });
}

int s1_op_stats(const s1_model* h, char* names_out, size_t names_cap, uint64_t* counts, double* total_ms, int cap) {
  if (!h || !h->m) return 0;
  const auto& st = h->m->stats;
  int k = 0;
  std::string names;
  for (const auto& s : st) {
    if (k >= cap) break;
    if (counts) counts[k] = s.second.first;
    if (total_ms) total_ms[k] = s.second.second;
    names += s.first;
    names += '\n';
    ++k;
  }
  if (names_out && names_cap) {
    size_t c = std::min(names_cap - 1, names.size());
    std::memcpy(names_out, names.data(), c);
    names_out[c] = 0;
  }
  return k;
}

void s1_op_stats_reset(s1_model* h) {
  if (h && h->m) h->m->stats.clear();
}

}  // extern "C"

namespace {

// Split-K workspace of the kernel-level entry points: grown on demand, kept for the thread.
struct Workspace {
  float* p = nullptr;
  size_t floats = 0;
};
thread_local Workspace g_ws;

float* workspace(size_t floats, hipStream_t st) {
  if (floats == 0) return nullptr;
  if (floats > g_ws.floats) {
    if (g_ws.p) {
      hip_ok(hipStreamSynchronize(st), "sync");
      hip_ok(hipFree(g_ws.p), "hipFree");
      g_ws.p = nullptr;
    }
    hip_ok(hipMalloc(&g_ws.p, floats * 4), "hipMalloc(workspace)");
    g_ws.floats = floats;
  }
  return g_ws.p;
}

// The arguments of s1k_gemm / s1k_gemm_noalloc, checked; g.ws is left to the caller.
s1::GemmArgs gemm_entry_args(const char* fn, const void* A, int lda, const void* W, int ldw, void* C, int ldc,
                             const float* bias, int M, int N, int K, int epi, int act) {
  if (epi < 0 || epi > 3) s1::fail(s1::kConfig, std::string(fn) + ": epi must be 0..3");
  if (act < 0 || act > 2) s1::fail(s1::kConfig, std::string(fn) + ": act must be 0..2");
  if (!A || !W || !C) s1::fail(s1::kConfig, std::string(fn) + ": NULL buffer");
  s1::GemmArgs g;
  g.A = static_cast<const uint16_t*>(A);
  g.W = static_cast<const uint16_t*>(W);
  g.C = C;
  g.bias = bias;
  g.M = M;
  g.N = N;
  g.K = K;
  g.lda = lda;
  g.ldw = ldw;
  g.ldc = ldc;
  g.epi = epi;
  g.act = act;
  g.splits = s1::gemm_plan(M, N, K).splits;
  return g;
}

// Split-K scratch of s1k_gemm_noalloc: one array per GPU, in the library's code object, so the
// entry point never allocates. No split plan needs more: a split GEMM runs at most 256 tiles'
// worth of workgroups (splits x tiles <= 256), each with one 64 x 128 f32 partial tile, and
// every partial is written in full before the reduce reads it, so nothing needs clearing.
constexpr size_t kScratchFloats = size_t(256) * 64 * 128;  // 8 MiB
static __device__ __align__(256) float scratch[kScratchFloats];

// The device address of `scratch` on each GPU, looked up once per device with it current.
std::mutex g_scratch_mu;
std::vector<float*> g_scratch_ptr;

float* scratch_on_current_device(hipStream_t st) {
  int dev = 0;
  hip_ok(hipGetDevice(&dev), "hipGetDevice");
  std::lock_guard<std::mutex> lk(g_scratch_mu);
  if (size_t(dev) >= g_scratch_ptr.size()) g_scratch_ptr.resize(size_t(dev) + 1, nullptr);
  if (!g_scratch_ptr[dev]) {
    // The lookup is a runtime call of its own; it is not made while the caller captures a graph.
    hipStreamCaptureStatus cs = hipStreamCaptureStatusNone;
    if (hipStreamIsCapturing(st, &cs) == hipSuccess && cs != hipStreamCaptureStatusNone)
      s1::fail(s1::kConfig, "s1k_gemm_noalloc: the first call on a GPU must come before any graph capture on it "
                            "(that call looks up the scratch array's address)");
    float* p = nullptr;
    hip_ok(hipGetSymbolAddress(reinterpret_cast<void**>(&p), HIP_SYMBOL(scratch)), "hipGetSymbolAddress(scratch)");
    g_scratch_ptr[dev] = p;
  }
  return g_scratch_ptr[dev];
}

}  // namespace

extern "C" {

int s1k_gemm(const void* A, int lda, const void* W, int ldw, void* C, int ldc, const float* bias, int M, int N, int K,
             int epi, int act, void* stream) {
  return guard([&] {
    s1::GemmArgs g = gemm_entry_args("s1k_gemm", A, lda, W, ldw, C, ldc, bias, M, N, K, epi, act);
    hipStream_t st = static_cast<hipStream_t>(stream);
    g.ws = workspace(s1::gemm_plan(M, N, K).ws_floats, st);
    if (const char* e = s1::gemm_check(g)) s1::fail(s1::kConfig, e);
    s1::gemm_launch(g, st);
    hip_ok(hipGetLastError(), "s1k_gemm launch");
  });
}

int s1k_gemm_noalloc(const void* A, int lda, const void* W, int ldw, void* C, int ldc, const float* bias, int M, int N,
                     int K, int epi, int act, void* stream) {
  return guard([&] {
    s1::GemmArgs g = gemm_entry_args("s1k_gemm_noalloc", A, lda, W, ldw, C, ldc, bias, M, N, K, epi, act);
    const size_t need = s1::gemm_plan(M, N, K).ws_floats;
    if (need > kScratchFloats)
      s1::fail(s1::kConfig, "s1k_gemm_noalloc: this shape's split-K partials need " + std::to_string(need * 4) +
                                " bytes, more than the " + std::to_string(kScratchFloats * 4) + "-byte scratch");
    g.ws = need ? scratch_on_current_device(static_cast<hipStream_t>(stream)) : nullptr;
    if (const char* e = s1::gemm_check(g)) s1::fail(s1::kConfig, e);
    s1::gemm_launch(g, static_cast<hipStream_t>(stream));
    hip_ok(hipGetLastError(), "s1k_gemm_noalloc launch");
  });
}

namespace {

struct RopeTable {
  float* c = nullptr;
  float* s = nullptr;
  int maxpos = 0;
  double theta = 0;
};

// Device cos/sin table for the kernel-level entry points, rebuilt when theta or the position
// range changes (same arithmetic as the model's tables).
void rope_table(RopeTable& t, double theta, int maxpos, hipStream_t st) {
  if (t.c && t.theta == theta && t.maxpos >= maxpos) return;
  if (t.c) {
    hip_ok(hipStreamSynchronize(st), "sync");
    hip_ok(hipFree(t.c), "hipFree");
    hip_ok(hipFree(t.s), "hipFree");
    t.c = t.s = nullptr;
  }
  const int half = 32;
  const float lbase = float(std::log2(double(float(theta))));
  std::vector<float> inv(half), c(size_t(maxpos) * half), s(size_t(maxpos) * half);
  for (int i = 0; i < half; ++i) inv[i] = float(std::exp2(double(-(float(i) / float(half)) * lbase)));
  for (int p = 0; p < maxpos; ++p)
    for (int i = 0; i < half; ++i) {
      const float ang = float(p) * inv[i];
      c[size_t(p) * half + i] = float(std::cos(double(ang)));
      s[size_t(p) * half + i] = float(std::sin(double(ang)));
    }
  hip_ok(hipMalloc(&t.c, c.size() * 4), "hipMalloc");
  hip_ok(hipMalloc(&t.s, s.size() * 4), "hipMalloc");
  hip_ok(hipMemcpy(t.c, c.data(), c.size() * 4, hipMemcpyHostToDevice), "upload");
  hip_ok(hipMemcpy(t.s, s.data(), s.size() * 4, hipMemcpyHostToDevice), "upload");
  t.theta = theta;
  t.maxpos = maxpos;
}

thread_local RopeTable g_rope;

int max_pos_of(const int32_t* pos, int M, hipStream_t st) {
  std::vector<int32_t> h(static_cast<size_t>(M));
  hip_ok(hipMemcpyAsync(h.data(), pos, size_t(M) * 4, hipMemcpyDeviceToHost, st), "read pos");
  hip_ok(hipStreamSynchronize(st), "sync");
  int mx = 0;
  for (int v : h) {
    if (v < 0) s1::fail(s1::kConfig, "negative position");
    mx = std::max(mx, v);
  }
  return mx + 1;
}

}  // namespace

int s1k_qkv_rope(const void* A, const void* W, int M, int d, const int32_t* pos, double theta, void* q, void* k, void* v,
                 int v_ld, void* stream) {
  return guard([&] {
    hipStream_t st = static_cast<hipStream_t>(stream);
    if (theta <= 0) s1::fail(s1::kConfig, "s1k_qkv_rope: theta must be positive");
    if (v_ld % 8 || v_ld < M + 64) s1::fail(s1::kConfig, "s1k_qkv_rope: v_ld must be a multiple of 8 and >= M + 64");
    rope_table(g_rope, theta, max_pos_of(pos, M, st), st);
    s1::GemmArgs g;
    g.A = static_cast<const uint16_t*>(A);
    g.W = static_cast<const uint16_t*>(W);
    g.M = M;
    g.N = 3 * d;
    g.K = d;
    g.lda = d;
    g.ldw = d;
    g.epi = s1::EPI_ROPE;
    g.rope_q = static_cast<uint16_t*>(q);
    g.rope_k = static_cast<uint16_t*>(k);
    g.rope_v = static_cast<uint16_t*>(v);
    g.rope_pos = pos;
    g.rope_cos = g_rope.c;
    g.rope_sin = g_rope.s;
    g.rope_T = M;
    g.rope_d = d;
    g.rope_ldv = v_ld;
    const s1::GemmPlan gp = s1::gemm_plan(M, 3 * d, d);
    g.splits = gp.splits;
    g.ws = workspace(gp.ws_floats, st);
    if (const char* e = s1::gemm_check(g)) s1::fail(s1::kConfig, e);
    s1::gemm_launch(g, st);
    hip_ok(hipGetLastError(), "s1k_qkv_rope launch");
  });
}

int s1k_split_rope(const void* qkv, int M, int d, const int32_t* pos, double theta, void* q, void* k, void* v,
                   int v_ld, void* stream) {
  return guard([&] {
    hipStream_t st = static_cast<hipStream_t>(stream);
    if (d % 64) s1::fail(s1::kConfig, "s1k_split_rope: d must be a multiple of 64");
    if (v_ld < (M + 7) / 8 * 8 || v_ld % 8)
      s1::fail(s1::kConfig, "s1k_split_rope: v_ld must be a multiple of 8 and at least M rounded up to 8");
    const float* c = nullptr;
    const float* s = nullptr;
    if (theta > 0) {
      rope_table(g_rope, theta, max_pos_of(pos, M, st), st);
      c = g_rope.c;
      s = g_rope.s;
    }
    s1::split_rope_launch(static_cast<const uint16_t*>(qkv), M, d, pos, c, s, static_cast<uint16_t*>(q),
                          static_cast<uint16_t*>(k), static_cast<uint16_t*>(v), v_ld, st);
    hip_ok(hipGetLastError(), "s1k_split_rope launch");
  });
}

int s1k_attention(const void* q, const void* k, const void* v, int v_ld, int T, int H, const int32_t* seq_starts,
                  int nseq, int window, float scale, void* out, void* stream) {
  return guard([&] {
    hipStream_t st = static_cast<hipStream_t>(stream);
    if (!seq_starts || nseq < 1) s1::fail(s1::kConfig, "s1k_attention: need seq_starts");
    if (seq_starts[0] != 0 || seq_starts[nseq] != T) s1::fail(s1::kConfig, "s1k_attention: seq_starts must run 0..T");
    if (v_ld < s1::vt_ld(T)) s1::fail(s1::kConfig, "s1k_attention: v_ld must be at least T rounded up to 8, plus 64");
    for (int r = 0; r < nseq; ++r)
      if (seq_starts[r + 1] <= seq_starts[r]) s1::fail(s1::kConfig, "s1k_attention: empty or decreasing sequence");
    std::vector<int> tiles;
    const int qb = s1::attn_plan_tiles(seq_starts, nseq, H, window, tiles);
    int* dt = nullptr;
    hip_ok(hipMalloc(&dt, tiles.size() * 4), "hipMalloc");
    hip_ok(hipMemcpyAsync(dt, tiles.data(), tiles.size() * 4, hipMemcpyHostToDevice, st), "upload tiles");
    s1::AttnArgs a;
    a.q = static_cast<const uint16_t*>(q);
    a.k = static_cast<const uint16_t*>(k);
    a.v = static_cast<const uint16_t*>(v);
    a.out = static_cast<uint16_t*>(out);
    a.tiles = reinterpret_cast<const s1::AttnTile*>(dt);
    a.ntiles = int(tiles.size() / 4);
    a.heads = H;
    a.Tq = T;
    a.Tk = T;
    a.ldv = v_ld;
    a.ldo = H * 64;
    a.scale = scale;
    a.window = window;
    a.tile_q = qb;
    s1::attn_launch(a, st);
    hipError_t e = hipGetLastError();
    hip_ok(hipStreamSynchronize(st), "s1k_attention");
    hip_ok(hipFree(dt), "hipFree");
    hip_ok(e, "s1k_attention launch");
  });
}

int s1k_layernorm(const float* x, const float* w, const float* b, float eps, int M, int d, void* y, void* stream) {
  return guard([&] {
    if (d <= 0 || d % 128 || d > s1::Model::kMaxHidden)
      s1::fail(s1::kConfig, "s1k_layernorm: d must be a multiple of 128 up to 2048");
    s1::layernorm_launch(x, nullptr, w, b, eps, M, d, static_cast<uint16_t*>(y), nullptr, nullptr, nullptr, nullptr,
                         static_cast<hipStream_t>(stream));
    hip_ok(hipGetLastError(), "s1k_layernorm launch");
  });
}

}  // extern "C"
