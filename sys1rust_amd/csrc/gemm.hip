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
//   EPI_ROPE   a q|k|v product (+ bias): split, RoPE on q and k when a cos/sin table is given
//              (by token position), q and k written head-major [H, T, 64], v transposed
//              [H, 64, ldv], bf16; the encoder's Wqkv and the decision head's in_proj
#include <algorithm>

#include "device.hpp"
#include "kernels.hpp"

namespace s1 {

namespace {

constexpr int BK = 64;

template <int N>
__device__ __forceinline__ void wait_vmcnt() {
  asm volatile("s_waitcnt vmcnt(%0)" ::"n"(N) : "memory");
}

// Workgroup barrier without the memory fence of __syncthreads: the fence would make the compiler
// drain every outstanding global->LDS load (vmcnt(0)) at each k-tile and serialise the pipeline.
// The "memory" clobber keeps LDS accesses on their side of it; completion of the async loads is
// awaited explicitly with wait_vmcnt before it.
__device__ __forceinline__ void barrier_lds() { asm volatile("s_barrier" ::: "memory"); }

// Wait until at most `ahead` k-tiles of this wave's loads (LPW loads each) are in flight.
template <int LPW, int MAXA>
__device__ __forceinline__ void wait_ahead(int ahead) {
  if constexpr (MAXA > 0) {
    if (ahead >= MAXA) {
      wait_vmcnt<MAXA * LPW>();
      return;
    }
    wait_ahead<LPW, MAXA - 1>(ahead);
  } else {
    wait_vmcnt<0>();
  }
}

template <int BM, int BN, int BK, int STAGES, int WM, int WN, int EPI>
__global__ __launch_bounds__(WM * WN * 64) void gemm_kernel(GemmArgs g) {
  constexpr int NW = WM * WN;                // waves; each owns a TM x TN sub-tile
  constexpr int TM = BM / WM, TN = BN / WN;
  constexpr int FM = TM / 32, FN = TN / 32;  // 32 x 32 MFMA fragments per wave
  constexpr int CH = BK / 8;                 // 16-byte chunks per LDS row
  constexpr int ROWB = BK * 2;               // bytes per LDS row
  constexpr int RG = 1024 / ROWB;            // rows per 1 KiB direct load
  constexpr int AG = BM / RG, WG = BN / RG;  // direct loads per k-tile
  constexpr int LPW = (AG + WG) / NW;        // loads per wave per k-tile
  constexpr int A_BYTES = BM * ROWB, STAGE_BYTES = (BM + BN) * ROWB;
  static_assert(FN % 2 == 0 && TN % 64 == 0, "epilogues pair the fragments of 64-column groups");
  constexpr int SW = 16 / CH;                // rows sharing one 256-byte bank line
  static_assert(BK == 32 || BK == 64, "BK");
  static_assert(LPW * NW == AG + WG, "load groups must split evenly over the waves");
  static_assert((STAGES - 2) * LPW < 64, "vmcnt range");

  // STAGES k-tiles of A [BM][BK] and W [BN][BK], bf16, rows of ROWB bytes. The 16-byte chunk c
  // of row r sits at slot c ^ ((r / SW) % CH): the 16 lanes of one LDS access phase (16
  // consecutive rows, the same k; 64 banks of 4 bytes) then hit 16 distinct 16-byte bank groups
  // without padding, which the direct loads (whole 1 KiB runs) could not write.
  __shared__ __attribute__((aligned(1024))) char smem[STAGES * STAGE_BYTES];

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = tid >> 6;
  const int wm = wave / WN, wn = wave % WN;

  // Tile order: each XCD takes a contiguous run of logical tiles (xcd_remap), and the run walks
  // groups of GM row tiles across all column tiles, GM fastest. The ~32 workgroups an XCD holds
  // at once then cover a GM x (32 / GM) patch, so its L2 serves every A row panel to many
  // column tiles instead of re-reading the activations from HBM once per column tile.
  constexpr int GM = BM >= 256 ? 4 : 8;
  const int mt = (g.M + BM - 1) / BM;
  const int nt = g.N / BN;
  const int bid = xcd_remap(blockIdx.x, gridDim.x);
  const int grp = bid / (GM * nt);
  const int gm = min(GM, mt - grp * GM);
  const int loc = bid - grp * GM * nt;
  const int tile_m = grp * GM + loc % gm, tile_n = loc / gm;
  const int m0 = tile_m * BM, n0 = tile_n * BN;
  // This workgroup's k-tiles: [kt0, kt0 + NK) of the K / BK (split-K divides them evenly).
  const int KT_ALL = g.K / BK;
  const int split = blockIdx.y, S = gridDim.y;
  const int kt0 = (split * KT_ALL) / S;
  const int NK = ((split + 1) * KT_ALL) / S - kt0;

  // Global -> LDS without registers (global_load_lds_dwordx4): lane l of a load moves 16 bytes
  // of row l / CH of its RG-row group, chunk (l % CH) ^ swizzle, into slot l % CH.
  const int lrow = lane / CH, lslot = lane % CH;
  auto issue = [&](int stage, int kt) {
    char* sb = smem + stage * STAGE_BYTES;
#pragma unroll
    for (int j = 0; j < LPW; ++j) {
      const int gi = wave + j * NW;
      if (gi < AG) {
        const int r = gi * RG + lrow;
        const int c = lslot ^ ((r / SW) % CH);
        const uint16_t* src = g.A + size_t(min(m0 + r, g.M - 1)) * g.lda + kt * BK + c * 8;
        __builtin_amdgcn_global_load_lds(src, sb + gi * 1024, 16, 0, 0);
      } else {
        const int r = (gi - AG) * RG + lrow;
        const int c = lslot ^ ((r / SW) % CH);
        const uint16_t* src = g.W + size_t(n0 + r) * g.ldw + kt * BK + c * 8;
        __builtin_amdgcn_global_load_lds(src, sb + A_BYTES + (gi - AG) * 1024, 16, 0, 0);
      }
    }
  };

  f32x16 acc[FM][FN];
#pragma unroll
  for (int i = 0; i < FM; ++i)
#pragma unroll
    for (int j = 0; j < FN; ++j)
#pragma unroll
      for (int e = 0; e < 16; ++e) acc[i][j][e] = 0.0f;

#pragma unroll
  for (int s = 0; s < STAGES - 1; ++s)
    if (s < NK) issue(s, kt0 + s);

  const int lr = lane & 31, lh = lane >> 5;
  for (int it = 0; it < NK; ++it) {
    // This wave's loads of k-tile `it` are done once at most `ahead` later k-tiles are in flight.
    wait_ahead<LPW, STAGES - 2>(min(STAGES - 2, NK - 1 - it));
    // Every wave's loads of `it` have landed, and every wave is done with k-tile it - 1, whose
    // buffer the next issue overwrites.
    barrier_lds();
    if (it + STAGES - 1 < NK) issue((it + STAGES - 1) % STAGES, kt0 + it + STAGES - 1);
    const char* sa = smem + (it % STAGES) * STAGE_BYTES;
    const char* sw = sa + A_BYTES;
    bf16x8 af[2][FM], bw[2][FN];
    auto frag = [&](int ks, int buf) {
#pragma unroll
      for (int i = 0; i < FM; ++i) {
        const int row = wm * TM + i * 32 + lr;
        af[buf][i] = *reinterpret_cast<const bf16x8*>(sa + row * ROWB + (((ks * 2 + lh) ^ ((row / SW) % CH)) << 4));
      }
#pragma unroll
      for (int j = 0; j < FN; ++j) {
        const int row = wn * TN + j * 32 + lr;
        bw[buf][j] = *reinterpret_cast<const bf16x8*>(sw + row * ROWB + (((ks * 2 + lh) ^ ((row / SW) % CH)) << 4));
      }
    };
    frag(0, 0);
#pragma unroll
    for (int ks = 0; ks < BK / 16; ++ks) {
      if (ks + 1 < BK / 16) frag(ks + 1, (ks + 1) & 1);
#pragma unroll
      for (int i = 0; i < FM; ++i)
#pragma unroll
        for (int j = 0; j < FN; ++j)
          acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(af[ks & 1][i], bw[ks & 1][j], acc[i][j], 0, 0, 0);
    }
  }

  if (S > 1) {
    // Split-K: this k-range's partial tile goes to ws[split] as f32; splitk_epilogue_kernel
    // sums the splits and applies the epilogue.
    float* part = g.ws + size_t(split) * g.M * g.N;
    const int lh2 = lane >> 5;
#pragma unroll
    for (int j = 0; j < FN; ++j)
#pragma unroll
      for (int i = 0; i < FM; ++i)
#pragma unroll
        for (int e = 0; e < 16; ++e) {
          const int row = m0 + wm * TM + i * 32 + (e >> 2) * 8 + 4 * lh2 + (e & 3);
          if (row < g.M) part[size_t(row) * g.N + n0 + wn * TN + j * 32 + (lane & 31)] = acc[i][j][e];
        }
    return;
  }

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
    // q and k go out as [H, T, 64]; v goes out transposed, [H, 64, ldv], which is the layout the
    // attention kernel stages: a lane's 4 consecutive rows of one dim are one 8-byte store.
    const int d = g.rope_d;
    const int i = lane & 31;
#pragma unroll
    for (int p = 0; p < FN / 2; ++p) {
      const int c0 = n0 + wn * TN + p * 64;  // first column of this head
      const int part = c0 / d;                 // 0 q, 1 k, 2 v
      const int head = (c0 - part * d) >> 6;
      if (part == 2) {
        uint16_t* v1 = g.rope_v + (size_t(head) * 64 + i) * g.rope_ldv;
        uint16_t* v2 = v1 + size_t(32) * g.rope_ldv;
        const float b1 = g.bias ? g.bias[c0 + i] : 0.0f, b2 = g.bias ? g.bias[c0 + 32 + i] : 0.0f;
#pragma unroll
        for (int mi = 0; mi < FM; ++mi)
#pragma unroll
          for (int q4 = 0; q4 < 4; ++q4) {
            const int row = rowbase + mi * 32 + q4 * 8;  // 4 rows row .. row + 3
            const f32x16& a1 = acc[mi][2 * p];
            const f32x16& a2 = acc[mi][2 * p + 1];
            if (row + 3 < g.M) {
              *reinterpret_cast<uint2*>(v1 + row) = make_uint2(pack2(a1[q4 * 4 + 0] + b1, a1[q4 * 4 + 1] + b1),
                                                               pack2(a1[q4 * 4 + 2] + b1, a1[q4 * 4 + 3] + b1));
              *reinterpret_cast<uint2*>(v2 + row) = make_uint2(pack2(a2[q4 * 4 + 0] + b2, a2[q4 * 4 + 1] + b2),
                                                               pack2(a2[q4 * 4 + 2] + b2, a2[q4 * 4 + 3] + b2));
            } else {
#pragma unroll
              for (int r = 0; r < 4; ++r)
                if (row + r < g.M) {
                  v1[row + r] = f2bf(a1[q4 * 4 + r] + b1);
                  v2[row + r] = f2bf(a2[q4 * 4 + r] + b2);
                }
            }
          }
        continue;
      }
      uint16_t* dst = part == 0 ? g.rope_q : g.rope_k;
      const float b1 = g.bias ? g.bias[c0 + i] : 0.0f, b2 = g.bias ? g.bias[c0 + 32 + i] : 0.0f;
#pragma unroll
      for (int mi = 0; mi < FM; ++mi)
#pragma unroll
        for (int e = 0; e < 16; ++e) {
          const int row = rowbase + mi * 32 + (e >> 2) * 8 + (e & 3);
          if (row < g.M) {
            float x1 = acc[mi][2 * p][e] + b1, x2 = acc[mi][2 * p + 1][e] + b2;
            if (g.rope_cos) {
              const int pos = g.rope_pos[row];
              const float c = g.rope_cos[pos * 32 + i], s = g.rope_sin[pos * 32 + i];
              const float y1 = x1 * c - x2 * s;
              x2 = x1 * s + x2 * c;
              x1 = y1;
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

template <int BM, int BN, int BK, int STAGES, int WM, int WN, int EPI>
void launch_t(const GemmArgs& g, hipStream_t st) {
  const int mt = (g.M + BM - 1) / BM, nt = g.N / BN;
  hipLaunchKernelGGL((gemm_kernel<BM, BN, BK, STAGES, WM, WN, EPI>), dim3(mt * nt, g.splits), dim3(WM * WN * 64), 0,
                     st, g);
}

template <int EPI>
void launch_e(const GemmArgs& g, hipStream_t st) {
  // 64-row tiles for tiny M; otherwise 128 x 128 with two k-tiles in LDS (64 KiB), which lets
  // two workgroups share a CU (two waves per SIMD).
  if (g.M <= 64)
    launch_t<64, 128, 64, 2, 1, 2, EPI>(g, st);
  else
    launch_t<128, 128, 64, 2, 2, 2, EPI>(g, st);
}

// Sum of the split-K partials in split order, then the GEMM's epilogue. One thread per row and
// column pair (c, c + 32) of a 64-column group, the pair the GeGLU and RoPE epilogues combine.
__global__ __launch_bounds__(256) void splitk_epilogue_kernel(GemmArgs g) {
  const long long gid = (long long)blockIdx.x * 256 + threadIdx.x;
  const int half = g.N / 2;
  if (gid >= (long long)g.M * half) return;
  const int row = int(gid / half);
  const int p = int(gid % half);
  const int c1 = (p / 32) * 64 + (p % 32), c2 = c1 + 32;
  float x1 = 0.0f, x2 = 0.0f;
  for (int s = 0; s < g.splits; ++s) {
    const float* part = g.ws + (size_t(s) * g.M + row) * g.N;
    x1 += part[c1];
    x2 += part[c2];
  }
  if (g.epi == EPI_GEGLU) {
    uint16_t* C = reinterpret_cast<uint16_t*>(g.C);
    C[size_t(row) * g.ldc + p] = f2bf(gelu_erf(x1) * x2);
    return;
  }
  if (g.epi == EPI_ROPE) {
    const int part = c1 / g.rope_d;
    const int head = (c1 - part * g.rope_d) >> 6;
    const int i = c1 & 63;
    if (g.bias) {
      x1 += g.bias[c1];
      x2 += g.bias[c2];
    }
    if (part < 2 && g.rope_cos) {
      const int pos = g.rope_pos[row];
      const float c = g.rope_cos[pos * 32 + i], sn = g.rope_sin[pos * 32 + i];
      const float y1 = x1 * c - x2 * sn, y2 = x1 * sn + x2 * c;
      x1 = y1;
      x2 = y2;
    }
    if (part == 2) {  // v transposed, [H, 64, ldv]
      uint16_t* o = g.rope_v + (size_t(head) * 64 + i) * g.rope_ldv + row;
      o[0] = f2bf(x1);
      o[size_t(32) * g.rope_ldv] = f2bf(x2);
      return;
    }
    uint16_t* o = (part == 0 ? g.rope_q : g.rope_k) + (size_t(head) * g.rope_T + row) * 64;
    o[i] = f2bf(x1);
    o[i + 32] = f2bf(x2);
    return;
  }
  const float b1 = g.bias ? g.bias[c1] : 0.0f, b2 = g.bias ? g.bias[c2] : 0.0f;
  x1 += b1;
  x2 += b2;
  if (g.epi == EPI_RESID || g.epi == EPI_F32) {
    float* C = reinterpret_cast<float*>(g.C) + size_t(row) * g.ldc;
    if (g.epi == EPI_RESID) {
      C[c1] += x1;
      C[c2] += x2;
    } else {
      C[c1] = x1;
      C[c2] = x2;
    }
    return;
  }
  if (g.act == ACT_RELU) {
    x1 = fmaxf(x1, 0.0f);
    x2 = fmaxf(x2, 0.0f);
  } else if (g.act == ACT_GELU) {
    x1 = gelu_erf(x1);
    x2 = gelu_erf(x2);
  }
  uint16_t* C = reinterpret_cast<uint16_t*>(g.C) + size_t(row) * g.ldc;
  C[c1] = f2bf(x1);
  C[c2] = f2bf(x2);
}

}  // namespace

GemmPlan gemm_plan(int M, int N, int K) {
  GemmPlan p;
  const int bm = M <= 64 ? 64 : 128;
  const int tiles = ((M + bm - 1) / bm) * (N / 128);
  const int KT = K / BK;
  // Few tiles (small M): split K so the workgroups cover the 256 CUs about twice, each keeping
  // at least 2 k-tiles.
  int s = 1;
  if (tiles < 192) s = std::max(1, std::min(KT / 2, (512 + tiles - 1) / tiles));
  p.splits = s;
  p.ws_floats = s > 1 ? size_t(s) * M * N : 0;
  return p;
}

const char* gemm_check(const GemmArgs& g) {
  if (g.M <= 0) return "gemm: M must be positive";
  if (g.K <= 0 || g.K % BK) return "gemm: K must be a positive multiple of 64";
  if (g.N <= 0 || g.N % 128) return "gemm: N must be a positive multiple of 128";
  if (g.lda < g.K || g.ldw < g.K || (g.lda % 8) || (g.ldw % 8)) return "gemm: bad leading dimension";
  if (g.epi == EPI_ROPE && (g.rope_d % 64 || g.N != 3 * g.rope_d)) return "gemm: rope epilogue needs N = 3d, d % 64 == 0";
  if (g.epi == EPI_ROPE && (g.rope_ldv % 8 || g.rope_ldv < g.M + 64)) return "gemm: v row stride must be a multiple of 8 and >= M + 64";
  if (g.splits < 1 || g.splits > g.K / BK) return "gemm: splits must be in 1..K/64";
  if (g.splits > 1 && !g.ws) return "gemm: split-K needs a workspace";
  return nullptr;
}

void gemm_launch(const GemmArgs& g, hipStream_t st) {
  if (g.splits > 1) {
    launch_e<EPI_F32>(g, st);  // partials only: the kernel returns before its epilogue
    const long long n = (long long)g.M * (g.N / 2);
    hipLaunchKernelGGL(splitk_epilogue_kernel, dim3(unsigned((n + 255) / 256)), dim3(256), 0, st, g);
    return;
  }
  switch (g.epi) {
    case EPI_BF16: launch_e<EPI_BF16>(g, st); break;
    case EPI_RESID: launch_e<EPI_RESID>(g, st); break;
    case EPI_GEGLU: launch_e<EPI_GEGLU>(g, st); break;
    case EPI_F32: launch_e<EPI_F32>(g, st); break;
    case EPI_ROPE: launch_e<EPI_ROPE>(g, st); break;
  }
}

}  // namespace s1
