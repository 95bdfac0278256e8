// Load-time checks of the fused kernels (selfcheck.hpp). Inputs are seeded and synthetic: A
// uniform in [-1.7, 1.7) (unit variance), weights uniform in [-0.035, 0.035) (the 0.02 standard
// deviation of the checkpoints), stored in the model's 16-bit type. The GEMMs run at three row
// counts: 40 (the reduce kernel of a split-K GEMM finishes the epilogue), 200 (one request's
// 64 x 128 tiles) and 4437 (the wide tiles of a batch of requests, with a ragged last row tile).
#include "selfcheck.hpp"

#include <algorithm>
#include <cmath>
#include <cstdio>
#include <vector>

#include "common.hpp"
#include "kernels.hpp"

namespace s1 {

namespace {

void hc(hipError_t e, const char* what) {
  if (e != hipSuccess) fail(kBackend, std::string("load check: ") + what + ": " + hipGetErrorString(e));
}

// A device buffer freed when it leaves scope (the checks allocate only at load).
struct Dev {
  void* p = nullptr;
  explicit Dev(size_t bytes) { hc(hipMalloc(&p, bytes < 16 ? 16 : bytes), "hipMalloc"); }
  ~Dev() {
    if (p) (void)hipFree(p);
  }
  Dev(const Dev&) = delete;
  Dev& operator=(const Dev&) = delete;
  template <class T>
  T* as() const {
    return static_cast<T*>(p);
  }
};

uint64_t mix(uint64_t x) {
  x += 0x9E3779B97F4A7C15ull;
  x = (x ^ (x >> 30)) * 0xBF58476D1CE4E5B9ull;
  x = (x ^ (x >> 27)) * 0x94D049BB133111EBull;
  return x ^ (x >> 31);
}

float uniform(uint64_t seed, size_t i, float half_width) {
  const float u = float(mix(seed * 0x100000001B3ull + i) >> 40) * 0x1.0p-24f;  // [0, 1)
  return (2.0f * u - 1.0f) * half_width;
}

std::vector<uint16_t> rand16(size_t n, uint64_t seed, float half_width, bool f16) {
  std::vector<uint16_t> v(n);
  for (size_t i = 0; i < n; ++i) {
    const float x = uniform(seed, i, half_width);
    v[i] = f16 ? f32_to_f16(x) : f32_to_bf16(x);
  }
  return v;
}

float val(uint16_t h, bool f16) { return f16 ? f16_to_f32(h) : bf16_to_f32(h); }

template <class T>
void up(void* dst, const std::vector<T>& v, hipStream_t st) {
  hc(hipMemcpyAsync(dst, v.data(), v.size() * sizeof(T), hipMemcpyHostToDevice, st), "upload");
}
template <class T>
std::vector<T> down(const void* src, size_t n, hipStream_t st) {
  std::vector<T> v(n);
  hc(hipMemcpyAsync(v.data(), src, n * sizeof(T), hipMemcpyDeviceToHost, st), "download");
  hc(hipStreamSynchronize(st), "sync");
  return v;
}

// Replace element 0 of a 16-bit device buffer by a value far from it (the check's fault
// injection): a wrong result that the comparison must catch.
void perturb16(void* buf, bool f16, hipStream_t st) {
  const std::vector<uint16_t> h = down<uint16_t>(buf, 1, st);
  const float x = val(h[0], f16);
  const std::vector<uint16_t> w = {f16 ? f32_to_f16(4.0f * std::fabs(x) + 1.0f) : f32_to_bf16(4.0f * std::fabs(x) + 1.0f)};
  up(buf, w, st);
}

GemmArgs plain_gemm(int elem, const void* A, const void* W, void* C, int M, int N, int K, int epi, float* ws) {
  GemmArgs g;
  g.elem = elem;
  g.A = static_cast<const uint16_t*>(A);
  g.W = static_cast<const uint16_t*>(W);
  g.C = C;
  g.M = M;
  g.N = N;
  g.K = K;
  g.lda = K;
  g.ldw = K;
  g.ldc = epi == EPI_GEGLU ? N / 2 : N;
  g.epi = epi;
  g.splits = gemm_plan(M, N, K).splits;
  g.ws = ws;
  // The q|k|v epilogue's own fields are set by the caller, which checks the arguments then.
  if (epi != EPI_ROPE)
    if (const char* e = gemm_check(g)) fail(kBackend, std::string("load check: ") + e);
  return g;
}

constexpr int kRows[] = {40, 200, 4437};

}  // namespace

// Split + RoPE. Unfused, x1 and x2 (a rotation pair) are rounded to 16 bits by the GEMM, rotated
// in f32 and rounded again; fused, the f32 products are rotated and rounded once. With u the unit
// roundoff (2^-8 for bf16, 2^-11 for f16), |fused - unfused| <= u (|x1| + |x2|) + 2u |y| + O(u^2),
// and |x1| + |x2| <= sqrt(2) |(y1, y2)| since the rotation keeps the pair's norm. The check allows
// 8u |(y1, y2)|, about twice that bound. v is a plain copy either way and must match exactly.
std::string check_fuserope(int elem, int d, int max_pos, const float* rope_cos, const float* rope_sin, hipStream_t st,
                           bool fault) {
  char buf_msg[256];
  const bool f16 = elem == ELEM_F16;
  const float u = f16 ? 0x1.0p-11f : 0x1.0p-8f;
  const int H = d / 64, N = 3 * d, K = d;
  const std::vector<uint16_t> w = rand16(size_t(N) * K, 11, 0.035f, f16);
  Dev dw(w.size() * 2);
  up(dw.p, w, st);
  for (int M : kRows) {
    const std::vector<uint16_t> a = rand16(size_t(M) * K, 12 + M, 1.7f, f16);
    std::vector<int> pos(M);
    for (int i = 0; i < M; ++i) pos[i] = int((int64_t(i) * 131 + 7) % max_pos);
    const int ldv = vt_ld(M), m8 = (M + 7) / 8 * 8;
    const size_t qn = size_t(H) * M * 64, vn = size_t(d) * ldv;
    Dev da(a.size() * 2), dpos(size_t(M) * 4), dqkv(size_t(M) * N * 2);
    Dev q1(qn * 2), k1(qn * 2), v1(vn * 2), q2(qn * 2), k2(qn * 2), v2(vn * 2);
    const GemmPlan gp = gemm_plan(M, N, K);
    Dev ws(gp.ws_floats * 4);
    up(da.p, a, st);
    up(dpos.p, pos, st);
    GemmArgs g = plain_gemm(elem, da.p, dw.p, nullptr, M, N, K, EPI_ROPE, ws.as<float>());
    g.rope_q = q1.as<uint16_t>();
    g.rope_k = k1.as<uint16_t>();
    g.rope_v = v1.as<uint16_t>();
    g.rope_pos = dpos.as<int>();
    g.rope_cos = rope_cos;
    g.rope_sin = rope_sin;
    g.rope_T = M;
    g.rope_d = d;
    g.rope_ldv = ldv;
    if (const char* e = gemm_check(g)) fail(kBackend, std::string("load check: ") + e);
    gemm_launch(g, st);
    gemm_launch(plain_gemm(elem, da.p, dw.p, dqkv.p, M, N, K, EPI_BF16, ws.as<float>()), st);
    split_rope_launch(dqkv.as<uint16_t>(), M, d, dpos.as<int>(), rope_cos, rope_sin, q2.as<uint16_t>(),
                      k2.as<uint16_t>(), v2.as<uint16_t>(), ldv, st, elem);
    hc(hipGetLastError(), "launch");
    if (fault) perturb16(q1.p, f16, st);
    for (int part = 0; part < 2; ++part) {
      const auto x = down<uint16_t>(part ? k1.p : q1.p, qn, st);
      const auto y = down<uint16_t>(part ? k2.p : q2.p, qn, st);
      for (size_t r = 0; r < size_t(H) * M; ++r)
        for (int i = 0; i < 32; ++i) {
          const size_t e1 = r * 64 + i, e2 = e1 + 32;
          const float y1 = val(y[e1], f16), y2 = val(y[e2], f16);
          const float tol = 8.0f * u * std::sqrt(y1 * y1 + y2 * y2) + 1e-6f;
          const float d1 = std::fabs(val(x[e1], f16) - y1), d2 = std::fabs(val(x[e2], f16) - y2);
          if (!(d1 <= tol && d2 <= tol)) {
            std::snprintf(buf_msg, sizeof buf_msg, "%s of head %d, row %d, dims %d/%d: fused %g %g, unfused %g %g (M=%d)",
                          part ? "k" : "q", int(r / M), int(r % M), i, i + 32, val(x[e1], f16), val(x[e2], f16), y1, y2,
                          M);
            return buf_msg;
          }
        }
    }
    const auto x = down<uint16_t>(v1.p, vn, st);
    const auto y = down<uint16_t>(v2.p, vn, st);
    for (size_t r = 0; r < size_t(d); ++r)
      for (int t = 0; t < m8; ++t)
        if (x[r * ldv + t] != y[r * ldv + t]) {
          std::snprintf(buf_msg, sizeof buf_msg, "v of dim %d, token %d differs (M=%d)", int(r), t, M);
          return buf_msg;
        }
  }
  return "";
}

// GeGLU. Unfused, x and the gate g are rounded to 16 bits, then gelu(x) g is computed in f32 and
// rounded; fused, the f32 products go straight into gelu(x) g. With |gelu'| <= 1.13 and
// |gelu(x)| <= |x|: |fused - unfused| <= u (1 + 1.13) |x| |g| + u (|a| + |a'|) + O(u^2)
// <= 4.2 u |x| |g|. The check allows 8 u |x| |g| (x, g the unfused GEMM's output).
std::string check_fusegeglu(int elem, int d, int inter, hipStream_t st, bool fault) {
  char buf_msg[256];
  const bool f16 = elem == ELEM_F16;
  const float u = f16 ? 0x1.0p-11f : 0x1.0p-8f;
  const int I = inter, N = 2 * I, K = d;
  const std::vector<uint16_t> w = rand16(size_t(N) * K, 21, 0.035f, f16);
  // The fused epilogue reads Wi with rows interleaved by 32: (x rows 32j.., gate rows I + 32j..).
  std::vector<uint16_t> wi(w.size());
  for (int j = 0; j < I / 32; ++j)
    for (int r = 0; r < 32; ++r) {
      std::copy_n(&w[size_t(32 * j + r) * K], K, &wi[size_t(64 * j + r) * K]);
      std::copy_n(&w[size_t(I + 32 * j + r) * K], K, &wi[size_t(64 * j + 32 + r) * K]);
    }
  Dev dw(w.size() * 2), dwi(wi.size() * 2);
  up(dw.p, w, st);
  up(dwi.p, wi, st);
  for (int M : kRows) {
    const std::vector<uint16_t> a = rand16(size_t(M) * K, 22 + M, 1.7f, f16);
    Dev da(a.size() * 2), act1(size_t(M) * I * 2), mid(size_t(M) * N * 2), act2(size_t(M) * I * 2);
    Dev ws(gemm_plan(M, N, K).ws_floats * 4);
    up(da.p, a, st);
    gemm_launch(plain_gemm(elem, da.p, dwi.p, act1.p, M, N, K, EPI_GEGLU, ws.as<float>()), st);
    gemm_launch(plain_gemm(elem, da.p, dw.p, mid.p, M, N, K, EPI_BF16, ws.as<float>()), st);
    geglu_launch(mid.as<uint16_t>(), M, I, act2.as<uint16_t>(), st, elem);
    hc(hipGetLastError(), "launch");
    if (fault) perturb16(act1.p, f16, st);
    const auto x = down<uint16_t>(act1.p, size_t(M) * I, st);
    const auto y = down<uint16_t>(act2.p, size_t(M) * I, st);
    const auto m = down<uint16_t>(mid.p, size_t(M) * N, st);
    for (int r = 0; r < M; ++r)
      for (int i = 0; i < I; ++i) {
        const float xv = val(m[size_t(r) * N + i], f16), gv = val(m[size_t(r) * N + I + i], f16);
        const float tol = 8.0f * u * std::fabs(xv * gv) + 1e-6f;
        const float a1 = val(x[size_t(r) * I + i], f16), a2 = val(y[size_t(r) * I + i], f16);
        if (!(std::fabs(a1 - a2) <= tol)) {
          std::snprintf(buf_msg, sizeof buf_msg, "row %d, column %d: fused %g, unfused %g (M=%d)", r, i, a1, a2, M);
          return buf_msg;
        }
      }
  }
  return "";
}

// Split-K residual GEMM + LayerNorm: the same partial sums in the same order, so h and the
// LayerNorm output must match bit for bit.
std::string check_fuseln(int elem, int d, float eps, hipStream_t st, bool fault) {
  char buf_msg[256];
  const bool f16 = elem == ELEM_F16;
  const int M = 96, N = d, K = d;
  const std::vector<uint16_t> a = rand16(size_t(M) * K, 31, 1.7f, f16);
  const std::vector<uint16_t> w = rand16(size_t(N) * K, 32, 0.035f, f16);
  std::vector<float> h0(size_t(M) * N), lw(N);
  for (size_t i = 0; i < h0.size(); ++i) h0[i] = uniform(33, i, 1.7f);
  for (int i = 0; i < N; ++i) lw[i] = 1.0f + uniform(34, size_t(i), 0.035f);
  Dev da(a.size() * 2), dw(w.size() * 2), h1(h0.size() * 4), h2(h0.size() * 4), dlw(size_t(N) * 4);
  Dev x1(size_t(M) * N * 2), x2(size_t(M) * N * 2);
  const GemmPlan gp = gemm_plan(M, N, K, true);
  // A width too narrow to split at one request's size has nothing to fold: only the encoder's
  // end is checked then, without partials.
  const bool split = gp.splits > 1;
  Dev ws(std::max<size_t>(gp.ws_floats, 1) * 4);
  up(da.p, a, st);
  up(dw.p, w, st);
  up(h1.p, h0, st);
  up(h2.p, h0, st);
  up(dlw.p, lw, st);
  GemmArgs g = plain_gemm(elem, da.p, dw.p, h1.p, M, N, K, EPI_RESID, ws.as<float>());
  g.splits = gp.splits;
  if (const char* e = gemm_check(g)) fail(kBackend, std::string("load check: ") + e);
  if (split) {
    gemm_launch_partials(g, st);
    splitk_resid_ln_launch(ws.as<float>(), g.splits, nullptr, h1.as<float>(), dlw.as<float>(), eps, M, N,
                           x1.as<uint16_t>(), st, elem);
    g.C = h2.p;
    gemm_launch(g, st);
    layernorm_launch(h2.as<float>(), nullptr, dlw.as<float>(), nullptr, eps, M, N, x2.as<uint16_t>(), nullptr, nullptr,
                     nullptr, nullptr, st, elem);
    hc(hipGetLastError(), "launch");
    if (fault) perturb16(x1.p, f16, st);
    const auto ha = down<uint32_t>(h1.p, h0.size(), st), hb = down<uint32_t>(h2.p, h0.size(), st);
    for (size_t i = 0; i < ha.size(); ++i)
      if (ha[i] != hb[i]) {
        std::snprintf(buf_msg, sizeof buf_msg, "h row %d, column %d differs", int(i / N), int(i % N));
        return buf_msg;
      }
    const auto xa = down<uint16_t>(x1.p, size_t(M) * N, st), xb = down<uint16_t>(x2.p, size_t(M) * N, st);
    for (size_t i = 0; i < xa.size(); ++i)
      if (xa[i] != xb[i]) {
        std::snprintf(buf_msg, sizeof buf_msg, "LayerNorm output row %d, column %d differs", int(i / N), int(i % N));
        return buf_msg;
      }
  }
  // The encoder's end: the same partials (still in ws) into the original h, final_norm with the
  // add of a per-row vector, and the head's norm1 with a bias, in one kernel, against h2 (the
  // reduce's sum), layernorm_launch with add_rowvec, and layernorm_launch with the bias.
  std::vector<float> addv(size_t(2) * N), lb(N), lw1(N);
  std::vector<int> seg(M);
  for (size_t i = 0; i < addv.size(); ++i) addv[i] = uniform(35, i, 0.5f);
  for (int i = 0; i < N; ++i) {
    lb[i] = uniform(36, size_t(i), 0.035f);
    lw1[i] = 1.0f + uniform(37, size_t(i), 0.035f);
  }
  for (int r = 0; r < M; ++r) seg[r] = (r / 3) % 2;
  Dev h3(h0.size() * 4), dadd(addv.size() * 4), dseg(size_t(M) * 4), dlb(size_t(N) * 4), dlw1(size_t(N) * 4);
  Dev hh1(h0.size() * 4), hh2(h0.size() * 4), x3(size_t(M) * N * 2), x4(size_t(M) * N * 2);
  up(h3.p, h0, st);
  up(dadd.p, addv, st);
  up(dseg.p, seg, st);
  up(dlb.p, lb, st);
  up(dlw1.p, lw1, st);
  encoder_end_launch(ws.as<float>(), split ? g.splits : 0, h3.as<float>(), dlw.as<float>(), eps, dadd.as<float>(), dseg.as<int>(),
                     hh1.as<float>(), dlw1.as<float>(), dlb.as<float>(), 1e-5f, x3.as<uint16_t>(), M, N, st, elem);
  layernorm_launch(h2.as<float>(), nullptr, dlw.as<float>(), nullptr, eps, M, N, nullptr, nullptr, dadd.as<float>(),
                   dseg.as<int>(), hh2.as<float>(), st, elem);
  layernorm_launch(hh2.as<float>(), nullptr, dlw1.as<float>(), dlb.as<float>(), 1e-5f, M, N, x4.as<uint16_t>(), nullptr,
                   nullptr, nullptr, nullptr, st, elem);
  hc(hipGetLastError(), "launch");
  if (fault && !split) perturb16(x3.p, f16, st);
  const auto ga = down<uint32_t>(hh1.p, h0.size(), st), gb = down<uint32_t>(hh2.p, h0.size(), st);
  for (size_t i = 0; i < ga.size(); ++i)
    if (ga[i] != gb[i]) {
      std::snprintf(buf_msg, sizeof buf_msg, "encoder end: head stream row %d, column %d differs", int(i / N), int(i % N));
      return buf_msg;
    }
  const auto ya = down<uint16_t>(x3.p, size_t(M) * N, st), yb = down<uint16_t>(x4.p, size_t(M) * N, st);
  for (size_t i = 0; i < ya.size(); ++i)
    if (ya[i] != yb[i]) {
      std::snprintf(buf_msg, sizeof buf_msg, "encoder end: norm1 output row %d, column %d differs", int(i / N), int(i % N));
      return buf_msg;
    }
  // The pruned head's end: the M rows as 24 requests of [row 0, 3 scorer rows]; the same partials
  // plus a bias, the pooled rows and the scorer's LayerNorm in one kernel, against the GEMM's
  // reduce with the bias, layernorm_launch over the scorer rows and the gather of the pooled rows.
  const int per = 4, nreq = M / per, R = nreq * (per - 1);
  std::vector<int> srows(R), prows(nreq);
  for (int r = 0; r < nreq; ++r) {
    prows[r] = r * per;
    for (int k = 0; k + 1 < per; ++k) srows[r * (per - 1) + k] = r * per + 1 + k;
  }
  Dev h4(h0.size() * 4), h5(h0.size() * 4), dsr(size_t(R) * 4), dpr(size_t(nreq) * 4);
  Dev pa(size_t(nreq) * N * 4), pb(size_t(nreq) * N * 4), ya2(size_t(R) * N * 2), yb2(size_t(R) * N * 2);
  up(h4.p, h0, st);
  up(h5.p, h0, st);
  up(dsr.p, srows, st);
  up(dpr.p, prows, st);
  if (split) {
    g.C = h5.p;
    g.bias = dlb.as<float>();
    gemm_launch(g, st);  // the partials again (no bias in them), then their sum and the bias into h5
  }
  head_end_launch(ws.as<float>(), split ? g.splits : 0, dlb.as<float>(), h4.as<float>(), per, dlw1.as<float>(),
                  dlb.as<float>(), 1e-5f, pa.as<float>(), ya2.as<uint16_t>(), M, N, st, elem);
  layernorm_launch(h5.as<float>(), dsr.as<int>(), dlw1.as<float>(), dlb.as<float>(), 1e-5f, R, N, yb2.as<uint16_t>(),
                   nullptr, nullptr, nullptr, nullptr, st, elem);
  gather_f32_launch(h5.as<float>(), dpr.as<int>(), nreq, N, pb.as<float>(), st);
  hc(hipGetLastError(), "launch");
  const auto qa = down<uint32_t>(pa.p, size_t(nreq) * N, st), qb = down<uint32_t>(pb.p, size_t(nreq) * N, st);
  for (size_t i = 0; i < qa.size(); ++i)
    if (qa[i] != qb[i]) {
      std::snprintf(buf_msg, sizeof buf_msg, "head end: pooled row %d, column %d differs", int(i / N), int(i % N));
      return buf_msg;
    }
  const auto za = down<uint16_t>(ya2.p, size_t(R) * N, st), zb = down<uint16_t>(yb2.p, size_t(R) * N, st);
  for (size_t i = 0; i < za.size(); ++i)
    if (za[i] != zb[i]) {
      std::snprintf(buf_msg, sizeof buf_msg, "head end: scorer row %d, column %d differs", int(i / N), int(i % N));
      return buf_msg;
    }
  if (!split) return "";
  // The pruned head's norm2: each output row's residual is a row of a longer stream, picked through
  // a row index (hsrc / hrows), with the out_proj bias and the LayerNorm's bias. Against the gather
  // of those rows, the GEMM's own split-K reduce with the bias and layernorm_launch with the bias.
  const int Hrows = 2 * M;
  std::vector<float> hs(size_t(Hrows) * N);
  std::vector<int> hr(M);
  for (size_t i = 0; i < hs.size(); ++i) hs[i] = uniform(38, i, 1.7f);
  for (int r = 0; r < M; ++r) hr[r] = (r * 37 + 11) % Hrows;  // distinct rows, out of order
  Dev dhs(hs.size() * 4), dhr(size_t(M) * 4), hA(size_t(M) * N * 4), hB(size_t(M) * N * 4);
  Dev yA(size_t(M) * N * 2), yB(size_t(M) * N * 2);
  up(dhs.p, hs, st);
  up(dhr.p, hr, st);
  GemmArgs gp2 = g;
  gp2.C = hB.p;
  gp2.bias = dlb.as<float>();
  gemm_launch_partials(gp2, st);
  splitk_resid_ln_launch(ws.as<float>(), gp2.splits, dlb.as<float>(), hA.as<float>(), dlw1.as<float>(), 1e-5f, M, N,
                         yA.as<uint16_t>(), st, elem, dlb.as<float>(), dhs.as<float>(), dhr.as<int>());
  gather_f32_launch(dhs.as<float>(), dhr.as<int>(), M, N, hB.as<float>(), st);
  gemm_launch(gp2, st);
  layernorm_launch(hB.as<float>(), nullptr, dlw1.as<float>(), dlb.as<float>(), 1e-5f, M, N, yB.as<uint16_t>(), nullptr,
                   nullptr, nullptr, nullptr, st, elem);
  hc(hipGetLastError(), "launch");
  const auto pa2 = down<uint32_t>(hA.p, size_t(M) * N, st), pb2 = down<uint32_t>(hB.p, size_t(M) * N, st);
  for (size_t i = 0; i < pa2.size(); ++i)
    if (pa2[i] != pb2[i]) {
      std::snprintf(buf_msg, sizeof buf_msg, "picked rows: h row %d, column %d differs", int(i / N), int(i % N));
      return buf_msg;
    }
  const auto ua = down<uint16_t>(yA.p, size_t(M) * N, st), ub = down<uint16_t>(yB.p, size_t(M) * N, st);
  for (size_t i = 0; i < ua.size(); ++i)
    if (ua[i] != ub[i]) {
      std::snprintf(buf_msg, sizeof buf_msg, "picked rows: norm2 output row %d, column %d differs", int(i / N),
                    int(i % N));
      return buf_msg;
    }
  return "";
}

}  // namespace s1
