// Kernels of the dtype=f32 path: the reference's BackendOptions::f32 (f32 weights and compute,
// runtime/crates/laya-core/src/backend.rs:25-27; laya-mlx/tests/parity.rs:54-65 checks it). It
// is a numerics mode, not the serving path: plain f32 arithmetic throughout (FMA GEMMs, an exact
// erf GELU, softmax with expf), written for clarity rather than speed.
#include <hip/hip_runtime.h>

#include "device.hpp"
#include "kernels.hpp"

namespace s1 {
namespace {

// C[M, N] (+)= act(A[M, K] . W[N, K]^T + bias): 64 x 64 tiles, 16-deep slabs of A and W staged
// transposed in LDS, each of the 256 threads 4 x 4 outputs (rows 4 ty .., columns 4 tx ..).
constexpr int GT = 64, GK = 16, GP = GT + 4;

__device__ __forceinline__ float gelu_exact(float x) { return 0.5f * x * (1.0f + erff(x * 0.70710678118654752f)); }

__global__ __launch_bounds__(256) void gemm32_kernel(Gemm32Args g) {
  __shared__ __attribute__((aligned(16))) float sA[GK][GP];
  __shared__ __attribute__((aligned(16))) float sW[GK][GP];
  const int tx = threadIdx.x & 15, ty = threadIdx.x >> 4;
  const int m0 = blockIdx.y * GT, n0 = blockIdx.x * GT;
  const int lr = threadIdx.x >> 2, lk = (threadIdx.x & 3) * 4;  // this thread's float4 of each slab
  float acc[4][4];
#pragma unroll
  for (int i = 0; i < 4; ++i)
#pragma unroll
    for (int j = 0; j < 4; ++j) acc[i][j] = 0.0f;
  for (int k0 = 0; k0 < g.K; k0 += GK) {
    float4 av = make_float4(0.0f, 0.0f, 0.0f, 0.0f), wv = av;
    if (m0 + lr < g.M) av = *reinterpret_cast<const float4*>(g.A + size_t(m0 + lr) * g.lda + k0 + lk);
    if (n0 + lr < g.N) wv = *reinterpret_cast<const float4*>(g.W + size_t(n0 + lr) * g.ldw + k0 + lk);
    __syncthreads();  // the previous slab has been read
    sA[lk][lr] = av.x;
    sA[lk + 1][lr] = av.y;
    sA[lk + 2][lr] = av.z;
    sA[lk + 3][lr] = av.w;
    sW[lk][lr] = wv.x;
    sW[lk + 1][lr] = wv.y;
    sW[lk + 2][lr] = wv.z;
    sW[lk + 3][lr] = wv.w;
    __syncthreads();
#pragma unroll
    for (int kk = 0; kk < GK; ++kk) {
      const float4 a = *reinterpret_cast<const float4*>(&sA[kk][ty * 4]);
      const float4 w = *reinterpret_cast<const float4*>(&sW[kk][tx * 4]);
      const float ar[4] = {a.x, a.y, a.z, a.w}, wr[4] = {w.x, w.y, w.z, w.w};
#pragma unroll
      for (int i = 0; i < 4; ++i)
#pragma unroll
        for (int j = 0; j < 4; ++j) acc[i][j] = fmaf(ar[i], wr[j], acc[i][j]);
    }
  }
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const int row = m0 + ty * 4 + i;
    if (row >= g.M) continue;
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const int col = n0 + tx * 4 + j;
      if (col >= g.N) continue;
      float v = acc[i][j] + (g.bias ? g.bias[col] : 0.0f);
      if (g.act == ACT_RELU) v = fmaxf(v, 0.0f);
      else if (g.act == ACT_GELU) v = gelu_exact(v);
      float* c = g.C + size_t(row) * g.ldc + col;
      *c = g.accumulate ? *c + v : v;
    }
  }
}

// qkv [T, 3d] -> q, k, v [H, T, 64], with the half-split RoPE rotation of q and k at pos[t] when
// the tables are given (split_rope.rs:44-54). One thread per (token, head, pair i < 32).
__global__ __launch_bounds__(256) void split32_kernel(const float* __restrict__ qkv, int T, int d, const int* __restrict__ pos,
                                                      const float* __restrict__ cs, const float* __restrict__ sn,
                                                      float* __restrict__ q, float* __restrict__ k, float* __restrict__ v) {
  const long long gid = (long long)blockIdx.x * 256 + threadIdx.x;
  const int H = d / 64;
  if (gid >= (long long)T * H * 32) return;
  const int i = int(gid % 32), h = int((gid / 32) % H), t = int(gid / (32LL * H));
  const float* row = qkv + size_t(t) * 3 * d + h * 64;
  const size_t o = (size_t(h) * T + t) * 64;
  float c = 1.0f, s = 0.0f;
  const bool rot = cs != nullptr;
  if (rot) {
    c = cs[size_t(pos[t]) * 32 + i];
    s = sn[size_t(pos[t]) * 32 + i];
  }
  for (int part = 0; part < 2; ++part) {
    const float x1 = row[part * d + i], x2 = row[part * d + i + 32];
    float* dst = (part == 0 ? q : k) + o;
    if (rot) {
      dst[i] = x1 * c - x2 * s;
      dst[i + 32] = x1 * s + x2 * c;
    } else {
      dst[i] = x1;
      dst[i + 32] = x2;
    }
  }
  v[o + i] = row[2 * d + i];
  v[o + i + 32] = row[2 * d + i + 32];
}

// Attention of single queries over a key set each (the entry format of attn_fallback_launch):
// one wave per (entry, head), 64 keys a step, lane j scoring key j of the step against the query
// held in LDS, lane c accumulating output dim c; softmax with expf.
__global__ __launch_bounds__(64) void attn32_kernel(Attn32Args a) {
  __shared__ float sq[64];
  __shared__ float sp[64];
  const int fi = blockIdx.x / a.heads, head = blockIdx.x % a.heads;
  const int* e = a.entries + size_t(fi) * 8;  // query, a0, a1, b0, b1, lo, hi, zeros
  const int qrow = e[0], a0 = e[1], a1 = e[2], b0 = e[3], b1 = e[4], lo = e[5], hi = e[6], zeros = e[7];
  const int lane = threadIdx.x;
  const float* Qh = a.q + size_t(head) * a.T * 64;
  const float* Kh = a.k + size_t(head) * a.T * 64;
  const float* Vh = a.v + size_t(head) * a.T * 64;
  sq[lane] = Qh[size_t(qrow) * 64 + lane];
  __syncthreads();
  const int khi = (b1 > b0 ? b1 : a1) - 1;
  const float llo = logf(float(1 + lo)), lhi = logf(float(1 + hi));
  float m = -INFINITY, l = 0.0f, o = 0.0f;
  auto keys = [&](int j0, int j1) {
    for (int b = j0; b < j1; b += 64) {
      const int j = b + lane;
      float s = -INFINITY;
      if (j < j1) {
        const float4* kr = reinterpret_cast<const float4*>(Kh + size_t(j) * 64);
        float dot = 0.0f;
#pragma unroll
        for (int c = 0; c < 16; ++c) {
          const float4 kv = kr[c];
          dot = fmaf(sq[4 * c], kv.x, dot);
          dot = fmaf(sq[4 * c + 1], kv.y, dot);
          dot = fmaf(sq[4 * c + 2], kv.z, dot);
          dot = fmaf(sq[4 * c + 3], kv.w, dot);
        }
        s = dot * a.scale + (j == a0 ? llo : 0.0f) + (j == khi ? lhi : 0.0f);
      }
      const float mn = fmaxf(m, wave_max(s));
      const float p = j < j1 ? expf(s - mn) : 0.0f;
      const float alpha = m == -INFINITY ? 0.0f : expf(m - mn);
      l = l * alpha + wave_sum(p);
      o *= alpha;
      m = mn;
      sp[lane] = p;
      __syncthreads();
      const int cnt = min(64, j1 - b);
      for (int t = 0; t < cnt; ++t) o = fmaf(sp[t], Vh[size_t(b + t) * 64 + lane], o);
      __syncthreads();
    }
  };
  keys(a0, a1);
  keys(b0, b1);
  if (zeros > 0) {  // zero slots: score 0, value 0
    const float sz = logf(float(zeros));
    const float mn = fmaxf(m, sz);
    const float alpha = m == -INFINITY ? 0.0f : expf(m - mn);
    l = l * alpha + expf(sz - mn);
    o *= alpha;
  }
  a.out[size_t(qrow) * a.ldo + head * 64 + lane] = o / l;
}

// act[t, i] = gelu(x[t, i]) * x[t, I + i] over x [T, 2I].
__global__ __launch_bounds__(256) void geglu32_kernel(const float* __restrict__ x, int T, int I, float* __restrict__ act) {
  const long long gid = (long long)blockIdx.x * 256 + threadIdx.x;
  if (gid >= (long long)T * I) return;
  const int t = int(gid / I), i = int(gid % I);
  const float* row = x + size_t(t) * 2 * I;
  act[gid] = gelu_exact(row[i]) * row[I + i];
}

}  // namespace

const char* gemm32_check(const Gemm32Args& g) {
  if (g.M < 0 || g.N <= 0 || g.K <= 0) return "f32 GEMM: empty shape";
  if (g.K % GK || g.lda % 4 || g.ldw % 4) return "f32 GEMM: K must be a multiple of 16, lda and ldw of 4";
  if ((reinterpret_cast<uintptr_t>(g.A) | reinterpret_cast<uintptr_t>(g.W)) % 16) return "f32 GEMM: A and W must be 16-byte aligned";
  if ((g.M + GT - 1) / GT > 65535) return "f32 GEMM: more than 65535 row tiles (4,194,240 rows)";
  return nullptr;
}

void gemm32_launch(const Gemm32Args& g, hipStream_t st) {
  if (g.M <= 0) return;
  const dim3 grid((g.N + GT - 1) / GT, (g.M + GT - 1) / GT);
  hipLaunchKernelGGL(gemm32_kernel, grid, dim3(256), 0, st, g);
}

void split32_launch(const float* qkv, int T, int d, const int* pos, const float* cos_t, const float* sin_t, float* q,
                    float* k, float* v, hipStream_t st) {
  const long long n = (long long)T * (d / 64) * 32;
  if (n <= 0) return;
  hipLaunchKernelGGL(split32_kernel, dim3(unsigned((n + 255) / 256)), dim3(256), 0, st, qkv, T, d, pos, cos_t, sin_t,
                     q, k, v);
}

void attn32_launch(const Attn32Args& a, hipStream_t st) {
  if (a.n <= 0) return;
  hipLaunchKernelGGL(attn32_kernel, dim3(unsigned(a.n) * unsigned(a.heads)), dim3(64), 0, st, a);
}

void geglu32_launch(const float* x, int T, int I, float* act, hipStream_t st) {
  const long long n = (long long)T * I;
  if (n <= 0) return;
  hipLaunchKernelGGL(geglu32_kernel, dim3(unsigned((n + 255) / 256)), dim3(256), 0, st, x, T, I, act);
}

}  // namespace s1
