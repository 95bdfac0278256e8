// LDS-tiled bf16 MFMA GEMM for gfx950: C[M, N] = A[M, K] . W[N, K]^T, f32 accumulation.
//
// Replaces the encoder's and the head's linears (runtime/crates/laya-mlx/src/lib.rs:612-628,
// 1363-1390; the NAX kernels of runtime/crates/laya-mlx/src/nax_gemm.rs:371-430). Both operands
// are K-contiguous ("NT"), the layout the MFMA operands want: every lane reads 8 consecutive k
// of one row with a single 16-byte LDS read.
//
// Tiling: a BM x BN x 64 block tile in 4 or 8 wavefronts; each wave owns a (BM/WM) x (BN/WN)
// sub-tile computed with v_mfma_f32_32x32x16_bf16. Global -> register -> LDS staging is double
// buffered so the next k-tile's loads are in flight while the current one feeds the MFMAs, with
// one barrier per k-tile. LDS rows are padded by 16 bytes so the 16-byte operand reads of 8
// consecutive lanes hit distinct banks.
//
// MFMA 32x32x16 lane layout (per operand, lane l, h = l / 32): A supplies row l % 32, k = 8h..8h+7;
// B supplies column l % 32, k = 8h..8h+7; the 16 accumulators of lane l hold column l % 32 and
// rows 8g + 4h + r for g, r in 0..3 (acc[4g + r]).
//
// Epilogues (fused, no extra pass over C):
//   EPI_BF16   C bf16 = acc (+ bias) (then relu or gelu)
//   EPI_RESID  C f32 += acc (+ bias)            residual add of Wo / Wo2 / out_proj / linear2
//   EPI_GEGLU  W rows interleaved by 32 (x block, gate block): C bf16 [M, N/2] = gelu(x) * gate
//   EPI_F32    C f32 = acc (+ bias)
//   EPI_ROPE   the encoder's Wqkv: split into q|k|v, RoPE on q and k (cos/sin table by token
//              position), written head-major as [H, T, 64] bf16 each
#include "device.hpp"
#include "kernels.hpp"

namespace s1 {

namespace {

constexpr int BK = 64;
constexpr int LDK = BK + 8;  // padded LDS row, in bf16 elements (144 bytes)

template <int BM, int BN, int WM, int WN, int EPI>
__global__ __launch_bounds__(WM* WN * 64) void gemm_kernel(GemmArgs g) {
  constexpr int NT = WM * WN * 64;
  constexpr int TM = BM / WM, TN = BN / WN;
  constexpr int FM = TM / 32, FN = TN / 32;
  constexpr int A_CH = BM * BK / 8 / NT;
  constexpr int W_CH = BN * BK / 8 / NT;
  static_assert(A_CH * NT * 8 == BM * BK && W_CH * NT * 8 == BN * BK, "tile not divisible");
  static_assert(EPI != EPI_GEGLU || (FN % 2) == 0, "geglu needs fragment pairs");

  __shared__ __attribute__((aligned(16))) uint16_t sA[2][BM * LDK];
  __shared__ __attribute__((aligned(16))) uint16_t sW[2][BN * LDK];

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = tid >> 6;
  const int wm = wave / WN, wn = wave % WN;

  const int mt = (g.M + BM - 1) / BM;
  const int bid = xcd_remap(blockIdx.x, gridDim.x);
  const int tile_m = bid % mt, tile_n = bid / mt;
  const int m0 = tile_m * BM, n0 = tile_n * BN;
  const int KT = g.K / BK;

  const uint16_t* __restrict__ A = g.A;
  const uint16_t* __restrict__ W = g.W;

  uint4 ra[A_CH], rw[W_CH];
#define S1_GLOAD(kt)                                                                         \
  do {                                                                                       \
    _Pragma("unroll") for (int i = 0; i < A_CH; ++i) {                                       \
      const int c = tid + i * NT;                                                            \
      const int gr = min(m0 + (c >> 3), g.M - 1);                                            \
      ra[i] = *reinterpret_cast<const uint4*>(A + size_t(gr) * g.lda + (kt) * BK + (c & 7) * 8); \
    }                                                                                        \
    _Pragma("unroll") for (int i = 0; i < W_CH; ++i) {                                       \
      const int c = tid + i * NT;                                                            \
      rw[i] = *reinterpret_cast<const uint4*>(W + size_t(n0 + (c >> 3)) * g.ldw + (kt) * BK + (c & 7) * 8); \
    }                                                                                        \
  } while (0)
#define S1_SSTORE(buf)                                                                       \
  do {                                                                                       \
    _Pragma("unroll") for (int i = 0; i < A_CH; ++i) {                                       \
      const int c = tid + i * NT;                                                            \
      *reinterpret_cast<uint4*>(&sA[buf][(c >> 3) * LDK + (c & 7) * 8]) = ra[i];             \
    }                                                                                        \
    _Pragma("unroll") for (int i = 0; i < W_CH; ++i) {                                       \
      const int c = tid + i * NT;                                                            \
      *reinterpret_cast<uint4*>(&sW[buf][(c >> 3) * LDK + (c & 7) * 8]) = rw[i];             \
    }                                                                                        \
  } while (0)

  f32x16 acc[FM][FN];
#pragma unroll
  for (int i = 0; i < FM; ++i)
#pragma unroll
    for (int j = 0; j < FN; ++j)
#pragma unroll
      for (int e = 0; e < 16; ++e) acc[i][j][e] = 0.0f;

  S1_GLOAD(0);
  S1_SSTORE(0);
  __syncthreads();

  const int lrow = lane & 31;
  const int lk = (lane >> 5) * 8;
  for (int kt = 0; kt < KT; ++kt) {
    const int buf = kt & 1;
    // The last iteration reloads its own tile into the idle buffer: harmless, and it keeps the
    // staging registers free of control flow.
    S1_GLOAD(min(kt + 1, KT - 1));
#pragma unroll
    for (int ks = 0; ks < BK / 16; ++ks) {
      bf16x8 af[FM], bw[FN];
#pragma unroll
      for (int i = 0; i < FM; ++i)
        af[i] = *reinterpret_cast<const bf16x8*>(&sA[buf][(wm * TM + i * 32 + lrow) * LDK + ks * 16 + lk]);
#pragma unroll
      for (int j = 0; j < FN; ++j)
        bw[j] = *reinterpret_cast<const bf16x8*>(&sW[buf][(wn * TN + j * 32 + lrow) * LDK + ks * 16 + lk]);
#pragma unroll
      for (int i = 0; i < FM; ++i)
#pragma unroll
        for (int j = 0; j < FN; ++j)
          acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(af[i], bw[j], acc[i][j], 0, 0, 0);
    }
    S1_SSTORE(buf ^ 1);
    __syncthreads();
  }

#undef S1_GLOAD
#undef S1_SSTORE

  // Epilogue. Lane holds column (lane & 31) and rows 8q + 4h + r of each 32x32 fragment.
  const int h = lane >> 5;
  const int colbase = n0 + wn * TN + (lane & 31);
  const int rowbase = m0 + wm * TM + 4 * h;
  if constexpr (EPI == EPI_GEGLU) {
    uint16_t* C = reinterpret_cast<uint16_t*>(g.C);
#pragma unroll
    for (int i = 0; i < FM; ++i)
#pragma unroll
      for (int p = 0; p < FN / 2; ++p) {
        const int oc = (n0 + wn * TN) / 2 + p * 32 + (lane & 31);
#pragma unroll
        for (int e = 0; e < 16; ++e) {
          const int row = rowbase + i * 32 + (e >> 2) * 8 + (e & 3);
          if (row < g.M) {
            const float x = acc[i][2 * p][e], gate = acc[i][2 * p + 1][e];
            C[size_t(row) * g.ldc + oc] = f2bf(gelu_erf(x) * gate);
          }
        }
      }
  } else if constexpr (EPI == EPI_ROPE) {
    // Columns [0, d) are q, [d, 2d) k, [2d, 3d) v; within a head of 64, dims i and i + 32 form a
    // rotation pair. With TN a multiple of 64 and fragments of 32 columns, fragment 2p holds dim
    // i = lane & 31 of a head and fragment 2p + 1 holds dim i + 32 of the same head, same rows.
    const int d = g.rope_d;
#pragma unroll
    for (int p = 0; p < FN / 2; ++p) {
      const int c0 = n0 + wn * TN + p * 64;  // first column of this head
      const int part = c0 / d;                 // 0 q, 1 k, 2 v
      const int head = (c0 - part * d) >> 6;
      const int i = lane & 31;
      uint16_t* dst = part == 0 ? g.rope_q : (part == 1 ? g.rope_k : g.rope_v);
#pragma unroll
      for (int mi = 0; mi < FM; ++mi)
#pragma unroll
        for (int e = 0; e < 16; ++e) {
          const int row = rowbase + mi * 32 + (e >> 2) * 8 + (e & 3);
          if (row < g.M) {
            float x1 = acc[mi][2 * p][e], x2 = acc[mi][2 * p + 1][e];
            if (part < 2) {
              const int pos = g.rope_pos[row];
              const float c = g.rope_cos[pos * 32 + i], s = g.rope_sin[pos * 32 + i];
              const float y1 = x1 * c - x2 * s;
              const float y2 = x1 * s + x2 * c;
              x1 = y1;
              x2 = y2;
            }
            uint16_t* o = dst + (size_t(head) * g.rope_T + row) * 64;
            o[i] = f2bf(x1);
            o[i + 32] = f2bf(x2);
          }
        }
    }
  } else {
#pragma unroll
    for (int j = 0; j < FN; ++j) {
      const int col = colbase + j * 32;
      const float bias = g.bias ? g.bias[col] : 0.0f;
#pragma unroll
      for (int i = 0; i < FM; ++i)
#pragma unroll
        for (int e = 0; e < 16; ++e) {
          const int row = rowbase + i * 32 + (e >> 2) * 8 + (e & 3);
          if (row < g.M) {
            float v = acc[i][j][e] + bias;
            if constexpr (EPI == EPI_RESID) {
              float* C = reinterpret_cast<float*>(g.C);
              C[size_t(row) * g.ldc + col] += v;
            } else if constexpr (EPI == EPI_F32) {
              float* C = reinterpret_cast<float*>(g.C);
              C[size_t(row) * g.ldc + col] = v;
            } else {
              if (g.act == ACT_RELU) v = fmaxf(v, 0.0f);
              else if (g.act == ACT_GELU) v = gelu_erf(v);
              uint16_t* C = reinterpret_cast<uint16_t*>(g.C);
              C[size_t(row) * g.ldc + col] = f2bf(v);
            }
          }
        }
    }
  }
}

template <int BM, int BN, int WM, int WN, int EPI>
void launch_t(const GemmArgs& g, hipStream_t st) {
  const int mt = (g.M + BM - 1) / BM, nt = g.N / BN;
  hipLaunchKernelGGL((gemm_kernel<BM, BN, WM, WN, EPI>), dim3(mt * nt), dim3(WM * WN * 64), 0, st, g);
}

template <int EPI>
void launch_e(const GemmArgs& g, hipStream_t st) {
  // Small M: 64-row tiles so more workgroups stream the weight; otherwise 128 x 128.
  if (g.M <= 256)
    launch_t<64, 128, 2, 2, EPI>(g, st);
  else
    launch_t<128, 128, 2, 2, EPI>(g, st);
}

}  // namespace

const char* gemm_check(const GemmArgs& g) {
  if (g.M <= 0) return "gemm: M must be positive";
  if (g.K <= 0 || g.K % BK) return "gemm: K must be a positive multiple of 64";
  if (g.N <= 0 || g.N % 128) return "gemm: N must be a positive multiple of 128";
  if (g.lda < g.K || g.ldw < g.K || (g.lda % 8) || (g.ldw % 8)) return "gemm: bad leading dimension";
  if (g.epi == EPI_ROPE && (g.rope_d % 64 || g.N != 3 * g.rope_d)) return "gemm: rope epilogue needs N = 3d, d % 64 == 0";
  return nullptr;
}

void gemm_launch(const GemmArgs& g, hipStream_t st) {
  switch (g.epi) {
    case EPI_BF16: launch_e<EPI_BF16>(g, st); break;
    case EPI_RESID: launch_e<EPI_RESID>(g, st); break;
    case EPI_GEGLU: launch_e<EPI_GEGLU>(g, st); break;
    case EPI_F32: launch_e<EPI_F32>(g, st); break;
    case EPI_ROPE: launch_e<EPI_ROPE>(g, st); break;
  }
}

}  // namespace s1
