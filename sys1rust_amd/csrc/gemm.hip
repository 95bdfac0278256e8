// LDS-tiled bf16 MFMA GEMM for gfx950: C[M, N] = A[M, K] . W[N, K]^T, f32 accumulation.
//
// Replaces the encoder's and the head's linears (runtime/crates/laya-mlx/src/lib.rs:612-628,
// 1363-1390; the NAX kernels of runtime/crates/laya-mlx/src/nax_gemm.rs:371-430). Both operands
// are K-contiguous ("NT"), the layout the MFMA operands want: every lane reads 8 consecutive k
// of one row with a single 16-byte LDS read.
//
// Tiling: a BM x BN x 64 block tile in 4 wavefronts; each wave owns a (BM/WM) x (BN/WN) sub-tile
// computed with v_mfma_f32_32x32x16_bf16 (v_mfma_f32_32x32x16_f16 for f16 operands: the element
// type E is a template parameter). Operands move global -> LDS directly (buffer_load_dwordx4 with
// lds, no registers), STAGES k-tiles deep, one barrier per k-tile; a 16-byte-chunk XOR swizzle
// keeps the fragment reads free of bank conflicts. The addresses the k-loop needs are computed
// before it: per lane, a 32-bit offset per direct load (a k-tile adds one scalar offset) and a
// base per k-step and operand (a fragment adds an immediate), so the loop issues almost nothing
// but its loads, LDS reads and MFMAs.
//
// MFMA 32x32x16 lane layout (per operand, lane l, h = l / 32): the first operand supplies row
// l % 32, k = 8h..8h+7; the second supplies column l % 32, k = 8h..8h+7; the 16 accumulators of
// lane l hold column l % 32 and rows 8g + 4h + r for g, r in 0..3 (acc[4g + r]). The k-loop
// computes C^T = W . A^T (W first), so a lane ends up with 4 consecutive output columns of one
// row per g: the epilogues convert them with packed instructions and store 8 or 16 bytes at once.
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

// buffer_load_dwordx4 ... lds: a direct global -> LDS load (LDS address from M0, lane l at + 16 l)
// whose global address is a buffer resource (scalar) plus a per-lane 32-bit offset and a scalar
// offset; offsets past the resource's size read 0. The LLVM intrinsic behind it is bound by name,
// outside any namespace so that the declaration keeps external linkage.
typedef int i32x4 __attribute__((ext_vector_type(4)));
__device__ void raw_buffer_load_lds(i32x4 rsrc, __attribute__((address_space(3))) void* lds, int size, int voffset,
                                    int soffset, int offset, int aux) __asm("llvm.amdgcn.raw.buffer.load.lds");

namespace s1 {

namespace {

constexpr int BK = 64;

template <int N>
__device__ __forceinline__ void wait_vmcnt() {
  asm volatile("s_waitcnt vmcnt(%0)" ::"n"(N) : "memory");
}

// 16 bytes from LDS at an address that is only 8-byte aligned (the staged output tiles pad their
// rows by 8 bytes, which keeps the fragment writes free of bank conflicts but leaves every other
// row's 16-byte pieces 8 bytes off): two 8-byte reads, where one misaligned 16-byte read would
// stall the LDS.
__device__ __forceinline__ uint4 lds_load16_a8(const char* p) {
  const uint2 lo = *reinterpret_cast<const uint2*>(p), hi = *reinterpret_cast<const uint2*>(p + 8);
  return make_uint4(lo.x, lo.y, hi.x, hi.y);
}

// Workgroup barrier without the memory fence of __syncthreads: the fence would make the compiler
// drain every outstanding global->LDS load (vmcnt(0)) at each k-tile and serialise the pipeline.
// The "memory" clobber keeps LDS accesses on their side of it; completion of the async loads is
// awaited explicitly with wait_vmcnt before it.
__device__ __forceinline__ void barrier_lds() { asm volatile("s_barrier" ::: "memory"); }

// Raw buffer resource over [p, p + bytes): base address, no stride, the byte count, and the third
// dword of every gfx9 buffer resource (32-bit data format, no swizzle).
__device__ __forceinline__ i32x4 buffer_rsrc(const void* p, uint32_t bytes) {
  const uint64_t a = reinterpret_cast<uint64_t>(p);
  i32x4 r;
  r.x = __builtin_amdgcn_readfirstlane(int(uint32_t(a)));
  r.y = __builtin_amdgcn_readfirstlane(int(uint32_t(a >> 32) & 0xffff));
  r.z = __builtin_amdgcn_readfirstlane(int(bytes));
  r.w = 0x00020000;
  return r;
}

// Bytes from the start of a [rows, ld] 16-bit matrix to the end of its k columns. Every launch
// keeps both operands' spans below 4 GiB (W by gemm_check; A by gemm_launch, which runs a longer
// A as row pieces), so a 32-bit offset reaches every element.
__host__ __device__ inline size_t span_bytes(int rows, int ld, int k) { return (size_t(rows - 1) * ld + k) * 2; }
constexpr size_t kMaxSpan = (size_t(1) << 32) - 1;

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

// One BM x BN output tile: the k-loop over [kt0, kt0 + NK) and the epilogue.
//
// TR selects the MFMA operand order. TR: D = W . A^T, so a lane's 16 accumulators of a fragment
// hold one output row (lane & 31) and columns 8g + 4h + r: four consecutive columns per g, stored
// as one 8-byte (bf16) or 16-byte (f32) access after a packed conversion. !TR: D = A . W^T, a
// lane holds one column and four consecutive rows per g; only the transposed v output of the
// q|k|v epilogue ([H, 64, ldv], rows = tokens contiguous) wants that.
template <class E, int BM, int BN, int BK, int STAGES, int WM, int WN, int EPI, bool TR, int KG, bool PIPE = false>
__device__ __forceinline__ void gemm_tile(const GemmArgs& g, char* smem0, int m0, int n0, int kt0, int NK, int split) {
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

  // KG > 1 (k-groups): the workgroup holds KG groups of NW waves; group k runs k-tiles
  // [kt0 + k NK / KG, kt0 + (k + 1) NK / KG) on stage buffers of its own (NK divides by KG, so
  // every group passes the same barriers), and group 0 adds the other groups' accumulators, in
  // group order, from LDS and runs the epilogue alone. A short GEMM's chain of dependent k-tiles
  // is then KG times shorter on the same tiles.
  const int grp = KG > 1 ? __builtin_amdgcn_readfirstlane(int(threadIdx.x) >> 6) / NW : 0;
  const int tid = threadIdx.x - grp * NW * 64;
  char* const smem = smem0 + grp * STAGES * STAGE_BYTES;
  if constexpr (KG > 1) {
    kt0 += grp * (NK / KG);
    NK /= KG;
  }
  const int lane = tid & 63;
  // Wave-uniform, so everything derived from it (load row groups, LDS destinations) is scalar.
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int wm = wave / WN, wn = wave % WN;

  // Global -> LDS without registers: lane l of a load moves 16 bytes of row l / CH of its RG-row
  // group, chunk (l % CH) ^ swizzle, into slot l % CH. Load group gi (A groups first) fills KiB gi
  // of its stage; the wave's load j is group wave + j NW, which reads A exactly when j < AG / NW.
  static_assert(AG % NW == 0 && A_BYTES == AG * 1024, "a wave's j-th load reads one operand, into KiB gi");
  const int lrow = lane / CH, lslot = lane % CH;
  // Per-lane byte offset of each of this wave's loads from the start of its operand at k = 0.
  uint32_t voff[LPW];
#pragma unroll
  for (int j = 0; j < LPW; ++j) {
    const int gi = wave + j * NW;
    const bool isA = j < AG / NW;
    const int r = (isA ? gi : gi - AG) * RG + lrow;
    const int c = lslot ^ ((r / SW) % CH);
    voff[j] = isA ? uint32_t((size_t(min(m0 + r, g.M - 1)) * g.lda + c * 8) * 2)
                  : uint32_t((size_t(n0 + r) * g.ldw + c * 8) * 2);
  }
  const i32x4 rsrcA = buffer_rsrc(g.A, uint32_t(span_bytes(g.M, g.lda, g.K)));
  const i32x4 rsrcW = buffer_rsrc(g.W, uint32_t(span_bytes(g.N, g.ldw, g.K)));
  // Loads j in [jlo, jhi) of this wave's LPW for k-tile kt into stage `stage`.
  auto issue = [&](int stage, int kt, int jlo, int jhi) __attribute__((always_inline)) {
    const int koff = __builtin_amdgcn_readfirstlane(kt * BK * 2);
    char* sb = smem + stage * STAGE_BYTES + wave * 1024;
#pragma unroll
    for (int j = 0; j < LPW; ++j) {
      if (j < jlo || j >= jhi) continue;
      const bool isA = j < AG / NW;
      raw_buffer_load_lds(isA ? rsrcA : rsrcW,
                          reinterpret_cast<__attribute__((address_space(3))) void*>(
                              uint32_t(reinterpret_cast<uintptr_t>(sb + j * NW * 1024))),
                          16, int(voff[j]), koff, 0, 0);
    }
  };

  f32x16 acc[FM][FN];
#pragma unroll
  for (int i = 0; i < FM; ++i)
#pragma unroll
    for (int j = 0; j < FN; ++j)
#pragma unroll
      for (int e = 0; e < 16; ++e) acc[i][j][e] = 0.0f;

  if constexpr (PIPE) {
    // One workgroup per CU (one wave per SIMD), so no other wave hides this one's waits: four
    // stages (three k-tiles in flight), fragments read one k-step ahead of their MFMAs into four
    // register sets, and the barrier that publishes k-tile it + 1 placed after k-step 1 of k-tile
    // it, so that it + 1's first two k-steps are read during it's last two. The loads of k-tile
    // it + 3 go out in two halves, after that barrier and after k-step 2 (in one burst they fill
    // the address queue and hold the wave before its MFMAs: Wo2 at a 10-question request 44.9
    // against 40.9 µs). Past the last k-tile the loads repeat it, so every k-tile waits on the
    // same vmcnt. The sched_barriers keep each k-step's MFMAs, reads and loads in this order.
    static_assert(STAGES == 4 && BK == 64 && TR && KG == 1, "pipelined k-loop shape");
    typedef typename E::v8 v8;
    const int lr = lane & 31, lh = lane >> 5;
    constexpr int KS = BK / 16;
    int kA[KS], kW[KS];
    {
      const int lsw = lh ^ ((lr / SW) % CH);
#pragma unroll
      for (int ks = 0; ks < KS; ++ks) {
        const int part = lr * ROWB + (((ks * 2) ^ lsw) << 4);
        kA[ks] = wm * TM * ROWB + part;
        kW[ks] = A_BYTES + wn * TN * ROWB + part;
      }
    }
    v8 fa[4][FM], fb[4][FN];
    auto rd = [&](int buf, int tile, int ks) __attribute__((always_inline)) {
      const char* st = smem + (tile & 3) * STAGE_BYTES;
      const char* pa = st + kA[ks];
      const char* pw = st + kW[ks];
#pragma unroll
      for (int i = 0; i < FM; ++i) fa[buf][i] = *reinterpret_cast<const v8*>(pa + i * 32 * ROWB);
#pragma unroll
      for (int j = 0; j < FN; ++j) fb[buf][j] = *reinterpret_cast<const v8*>(pw + j * 32 * ROWB);
    };
    auto mm = [&](int buf) __attribute__((always_inline)) {
#pragma unroll
      for (int i = 0; i < FM; ++i)
#pragma unroll
        for (int j = 0; j < FN; ++j) acc[i][j] = E::mfma(fb[buf][j], fa[buf][i], acc[i][j]);
    };
#pragma unroll
    for (int s = 0; s < STAGES - 1; ++s) issue(s, kt0 + min(s, NK - 1), 0, LPW);
    wait_vmcnt<2 * LPW>();
    barrier_lds();
    rd(0, 0, 0);
    rd(1, 0, 1);
    for (int it = 0; it < NK; ++it) {
      mm(0);
      rd(2, it, 2);
      __builtin_amdgcn_sched_barrier(0);
      mm(1);
      rd(3, it, 3);
      __builtin_amdgcn_sched_barrier(0);
      wait_vmcnt<LPW>();
      barrier_lds();
      issue((it + 3) & 3, kt0 + min(it + 3, NK - 1), 0, LPW / 2);
      __builtin_amdgcn_sched_barrier(0);
      mm(2);
      rd(0, min(it + 1, NK - 1), 0);
      __builtin_amdgcn_sched_barrier(0);
      issue((it + 3) & 3, kt0 + min(it + 3, NK - 1), LPW / 2, LPW);
      __builtin_amdgcn_sched_barrier(0);
      mm(3);
      rd(1, min(it + 1, NK - 1), 1);
      __builtin_amdgcn_sched_barrier(0);
    }
    wait_vmcnt<0>();
  } else {
#pragma unroll
    for (int s = 0; s < STAGES - 1; ++s)
      if (s < NK) issue(s, kt0 + s, 0, LPW);
  
    const int lr = lane & 31, lh = lane >> 5;
    // Fragment reads: lane (lr, lh) of k-step ks reads A row wm TM + 32 i + lr and W row
    // wn TN + 32 j + lr, chunk (2 ks + lh) ^ ((row / SW) % CH). A row base 32 i + (multiple of 16)
    // leaves the swizzle to the lane alone (SW CH = 16), so each k-step has one LDS base per operand
    // and a fragment adds 32 i ROWB (an immediate) to it.
    static_assert(SW * CH == 16 && TM % 16 == 0 && TN % 16 == 0, "lane-only fragment swizzle");
    constexpr int KS = BK / 16;
    int kA[KS], kW[KS];
    {
      const int lsw = lh ^ ((lr / SW) % CH);
  #pragma unroll
      for (int ks = 0; ks < KS; ++ks) {
        const int part = lr * ROWB + (((ks * 2) ^ lsw) << 4);
        kA[ks] = wm * TM * ROWB + part;
        kW[ks] = A_BYTES + wn * TN * ROWB + part;
      }
    }
    for (int it = 0; it < NK; ++it) {
      // This wave's loads of k-tile `it` are done once at most `ahead` later k-tiles are in flight.
      wait_ahead<LPW, STAGES - 2>(min(STAGES - 2, NK - 1 - it));
      // Every wave's loads of `it` have landed, and every wave is done with k-tile it - 1, whose
      // buffer the next issue overwrites.
      barrier_lds();
      // The next k-tile's loads go out over the first two k-steps of this one: issued as one burst
      // they fill the address queue and stall the wave before its MFMAs (the two then do not
      // overlap); issued later they have too little of the k-tile left to land in.
      const bool pre = it + STAGES - 1 < NK;
      const int pstage = (it + STAGES - 1) % STAGES, pkt = kt0 + it + STAGES - 1;
      const char* sa = smem + (it % STAGES) * STAGE_BYTES;
      typedef typename E::v8 v8;
      v8 af[2][FM], bw[2][FN];
      auto frag = [&](int ks, int buf) __attribute__((always_inline)) {
        const char* pa = sa + kA[ks];
        const char* pw = sa + kW[ks];
  #pragma unroll
        for (int i = 0; i < FM; ++i) af[buf][i] = *reinterpret_cast<const v8*>(pa + i * 32 * ROWB);
  #pragma unroll
        for (int j = 0; j < FN; ++j) bw[buf][j] = *reinterpret_cast<const v8*>(pw + j * 32 * ROWB);
      };
      frag(0, 0);
      constexpr int LPK = (LPW + 1) / 2;
  #pragma unroll
      for (int ks = 0; ks < KS; ++ks) {
        if (pre && ks < 2) issue(pstage, pkt, ks * LPK, min(LPW, (ks + 1) * LPK));
        if (ks + 1 < KS) frag(ks + 1, (ks + 1) & 1);
  #pragma unroll
        for (int i = 0; i < FM; ++i)
  #pragma unroll
          for (int j = 0; j < FN; ++j) {
            if constexpr (TR)
              acc[i][j] = E::mfma(bw[ks & 1][j], af[ks & 1][i], acc[i][j]);
            else
              acc[i][j] = E::mfma(af[ks & 1][i], bw[ks & 1][j], acc[i][j]);
          }
      }
    }
  }

  if constexpr (KG > 1) {
    // Groups 1.. leave their accumulators in their own stage buffers, in register order (float4
    // e4 of fragment (i, j) of wave w at ((w FM + i) FN + j) 4 + e4, 64 lanes apart), and end;
    // waves that have ended take no part in the barriers that follow.
    static_assert(BM * BN * 4 <= STAGES * STAGE_BYTES, "a group's partial tile must fit its stage buffers");
    __syncthreads();  // every group is done reading its stage buffers
    if (grp > 0) {
      float4* dst = reinterpret_cast<float4*>(smem);
#pragma unroll
      for (int i = 0; i < FM; ++i)
#pragma unroll
        for (int j = 0; j < FN; ++j)
#pragma unroll
          for (int e4 = 0; e4 < 4; ++e4)
            dst[(((wave * FM + i) * FN + j) * 4 + e4) * 64 + lane] =
                make_float4(acc[i][j][4 * e4], acc[i][j][4 * e4 + 1], acc[i][j][4 * e4 + 2], acc[i][j][4 * e4 + 3]);
    }
    __syncthreads();
    if (grp > 0) return;
#pragma unroll
    for (int gg = 1; gg < KG; ++gg) {
      const float4* src = reinterpret_cast<const float4*>(smem0 + gg * STAGES * STAGE_BYTES);
#pragma unroll
      for (int i = 0; i < FM; ++i)
#pragma unroll
        for (int j = 0; j < FN; ++j)
#pragma unroll
          for (int e4 = 0; e4 < 4; ++e4) {
            const float4 v = src[(((wave * FM + i) * FN + j) * 4 + e4) * 64 + lane];
            acc[i][j][4 * e4] += v.x;
            acc[i][j][4 * e4 + 1] += v.y;
            acc[i][j][4 * e4 + 2] += v.z;
            acc[i][j][4 * e4 + 3] += v.w;
          }
    }
  }
  const int l32 = lane & 31, h = lane >> 5;
  constexpr int NT = NW * 64;
  // bf16 results leave through LDS: after the k-loop the stage buffers are free, each wave
  // writes its fragments there (8 bytes per lane, padded rows keep the 32 rows of one access on
  // distinct banks), and the block then stores whole rows with 16-byte lane accesses, so every
  // store instruction writes full cache lines instead of 16-byte pieces of 32 rows.
  char* stg = smem;
  if constexpr (!TR) {
    // q|k|v epilogue, v blocks: columns [2d, 3d) go out transposed, [H, 64, ldv]. Lane holds
    // column (lane & 31) of fragment 2p (dim i of a head; 2p + 1 has dim i + 32) and rows
    // 8q + 4h .. + 3: 4 consecutive tokens of one dim, staged as [column][token].
    static_assert(EPI == EPI_ROPE, "column-per-lane order is only used for the transposed v output");
    constexpr int PV = BM * 2 + 8;
    constexpr int NH = BN * PV <= STAGES * STAGE_BYTES ? 1 : 2;  // column halves staged one after the other
    constexpr int HC = BN / NH;
    static_assert(HC * PV <= STAGES * STAGE_BYTES && HC % 64 == 0, "v staging must fit the stage buffers");
    const int head0 = (n0 - 2 * g.rope_d) >> 6;
#pragma unroll
    for (int half = 0; half < NH; ++half) {
      __syncthreads();
#pragma unroll
      for (int p = 0; p < FN / 2; ++p) {
        const int cl = wn * TN + p * 64 + l32;
        if ((wn * TN + p * 64) / HC != half) continue;
        const float b1 = g.bias ? g.bias[n0 + cl] : 0.0f, b2 = g.bias ? g.bias[n0 + cl + 32] : 0.0f;
        char* col1 = stg + (cl - half * HC) * PV;
        char* col2 = col1 + 32 * PV;
#pragma unroll
        for (int mi = 0; mi < FM; ++mi)
#pragma unroll
          for (int q4 = 0; q4 < 4; ++q4) {
            const int rl = wm * TM + mi * 32 + q4 * 8 + 4 * h;
            const f32x16& a1 = acc[mi][2 * p];
            const f32x16& a2 = acc[mi][2 * p + 1];
            *reinterpret_cast<uint2*>(col1 + rl * 2) =
                make_uint2(E::pack2(a1[q4 * 4] + b1, a1[q4 * 4 + 1] + b1), E::pack2(a1[q4 * 4 + 2] + b1, a1[q4 * 4 + 3] + b1));
            *reinterpret_cast<uint2*>(col2 + rl * 2) =
                make_uint2(E::pack2(a2[q4 * 4] + b2, a2[q4 * 4 + 1] + b2), E::pack2(a2[q4 * 4 + 2] + b2, a2[q4 * 4 + 3] + b2));
          }
      }
      __syncthreads();
      for (int idx = tid; idx < HC * (BM / 8); idx += NT) {
        const int c = idx / (BM / 8), k8 = idx % (BM / 8);
        const int tok = m0 + k8 * 8;
        if (tok >= g.M) continue;
        const int cg = half * HC + c;  // column within the tile
        const uint4 v = lds_load16_a8(stg + c * PV + k8 * 16);
        uint16_t* dst = g.rope_v + (size_t(head0 + cg / 64) * 64 + cg % 64) * g.rope_ldv + tok;
        // The row's last, partial 8-token group is written whole, zeros past M (ldv >= M
        // rounded up to 8): readers may then load V^T in 8-byte pieces without masking them.
        *reinterpret_cast<uint4*>(dst) = tok + 8 <= g.M ? v : keep_first(v, g.M - tok);
      }
    }
    return;
  } else {
    // Lane holds row rbase + 32 i and columns cbase + 32 j + 8 q .. + 3 (acc[i][j][4 q + r]).
    const int rbase = m0 + wm * TM + l32;
    const int cbase = n0 + wn * TN + 4 * h;
    const int rl0 = wm * TM + l32;        // the same row and column, local to the tile
    const int cl0 = wn * TN + 4 * h;
    const float4 zero4 = make_float4(0.0f, 0.0f, 0.0f, 0.0f);
    if constexpr (EPI == EPI_RESID || EPI == EPI_F32) {
      // f32 out: with split-K (which gemm_launch always runs with this epilogue) this k-range's
      // partial tile into ws[split], summed in split order by splitk_epilogue_kernel or
      // splitk_resid_ln_kernel; else C (+)= acc + bias. The tile leaves through LDS like the bf16
      // results: staged [rows][BN] (rows padded by 16 bytes), then written as whole rows, 16 bytes
      // per lane and BN / 4 lanes per row, so every access covers whole cache lines (straight
      // from the fragments an access is a 32-byte piece of each of 32 rows).
      const bool part = g.splits > 1;
      float* out = part ? g.ws + size_t(split) * g.M * g.N : reinterpret_cast<float*>(g.C);
      const int ld = part ? g.N : g.ldc;
      constexpr int PF = BN * 4 + 16;
      constexpr int NHF = BM * PF <= STAGES * STAGE_BYTES ? 1 : BM / 2 * PF <= STAGES * STAGE_BYTES ? 2 : 4;
      constexpr int HRF = BM / NHF;
      static_assert(HRF * PF <= STAGES * STAGE_BYTES && HRF % 32 == 0, "f32 staging must fit the stage buffers");
      const bool addb = !part && g.bias != nullptr;  // uniform branch, 16-byte bias loads
      const bool rmw = EPI == EPI_RESID && !part;
#pragma unroll
      for (int half = 0; half < NHF; ++half) {
        __syncthreads();
#pragma unroll
        for (int j = 0; j < FN; ++j)
#pragma unroll
          for (int q = 0; q < 4; ++q) {
            float4 b = zero4;
            if (addb) b = *reinterpret_cast<const float4*>(g.bias + cbase + j * 32 + q * 8);
#pragma unroll
            for (int i = 0; i < FM; ++i) {
              if ((wm * TM + i * 32) / HRF != half) continue;
              *reinterpret_cast<float4*>(stg + (rl0 + i * 32 - half * HRF) * PF + (cl0 + j * 32 + q * 8) * 4) =
                  make_float4(acc[i][j][4 * q] + b.x, acc[i][j][4 * q + 1] + b.y, acc[i][j][4 * q + 2] + b.z,
                              acc[i][j][4 * q + 3] + b.w);
            }
          }
        __syncthreads();
        // A thread's pieces of the half: one column group c4, rows r0, r0 + RS, ... In groups of
        // at most 8, every old residual value of a group is loaded before any is waited on, so a
        // group costs one memory round trip, not one per piece (groups of 8 keep the 192-row
        // tile within two workgroups per CU).
        static_assert(NT % (BN / 4) == 0, "whole rows per thread pass");
        constexpr int RS = NT / (BN / 4);
        constexpr int PT = HRF / RS;
        static_assert(PT * RS == HRF, "the staged rows split evenly over the threads");
        constexpr int PG = PT <= 8 ? PT : PT % 8 == 0 ? 8 : PT % 6 == 0 ? 6 : PT % 4 == 0 ? 4 : PT % 2 == 0 ? 2 : 1;
        static_assert(PT % PG == 0 && PG <= 8, "piece groups");
        const int r0 = tid / (BN / 4), c4 = tid % (BN / 4);
        const int row0 = m0 + half * HRF + r0;
        const char* sp = stg + r0 * PF + c4 * 16;
        float* op = out + size_t(row0) * ld + n0 + c4 * 4;
#pragma unroll
        for (int u0 = 0; u0 < PT; u0 += PG) {
          float4 v[PG], old[PG];
#pragma unroll
          for (int u = 0; u < PG; ++u) {
            v[u] = *reinterpret_cast<const float4*>(sp + (u0 + u) * RS * PF);
            old[u] = zero4;
            if (rmw && row0 + (u0 + u) * RS < g.M)
              old[u] = *reinterpret_cast<const float4*>(op + size_t((u0 + u) * RS) * ld);
          }
#pragma unroll
          for (int u = 0; u < PG; ++u) {
            if (row0 + (u0 + u) * RS >= g.M) continue;
            float4* c = reinterpret_cast<float4*>(op + size_t((u0 + u) * RS) * ld);
            *c = rmw ? make_float4(old[u].x + v[u].x, old[u].y + v[u].y, old[u].z + v[u].z, old[u].w + v[u].w) : v[u];
          }
          __builtin_amdgcn_sched_barrier(0);  // keep the next group's loads after these stores
        }
      }
      return;
    } else if constexpr (EPI == EPI_GEGLU) {
      // W rows interleaved by 32: fragment 2p is x, 2p + 1 its gate; output columns
      // (n0 + wn TN) / 2 + 32 p + 8 q + 4 h .. + 3. Stored directly (8 bytes per lane): the
      // half-width rows gain less from LDS staging than its two barriers cost.
      uint16_t* C = reinterpret_cast<uint16_t*>(g.C);
#pragma unroll
      for (int i = 0; i < FM; ++i) {
        const int row = rbase + i * 32;
        if (row >= g.M) continue;
        uint16_t* crow = C + size_t(row) * g.ldc + (n0 + wn * TN) / 2 + 4 * h;
#pragma unroll
        for (int p = 0; p < FN / 2; ++p)
#pragma unroll
          for (int q = 0; q < 4; ++q) {
            const f32x16& x = acc[i][2 * p];
            const f32x16& gt = acc[i][2 * p + 1];
            *reinterpret_cast<uint2*>(crow + p * 32 + q * 8) =
                make_uint2(E::pack2(gelu_erf(x[4 * q]) * gt[4 * q], gelu_erf(x[4 * q + 1]) * gt[4 * q + 1]),
                           E::pack2(gelu_erf(x[4 * q + 2]) * gt[4 * q + 2], gelu_erf(x[4 * q + 3]) * gt[4 * q + 3]));
          }
      }
    } else {
      // Staged bf16 tile [BM][BN], in row halves when the whole tile does not fit. The q|k
      // rotation's cos / sin rows (TP bytes each) are staged behind it where they fit beside the
      // whole tile (not for the 192-row tile: there, staging in two halves cost more than the
      // tables' loads saved); else each lane loads its own pieces.
      constexpr int P = BN * 2 + 8;
      constexpr int TOFF = (BM * P + 1023) / 1024 * 1024;
      constexpr bool TLDS = EPI == EPI_ROPE && TOFF + BM * 256 <= STAGES * STAGE_BYTES;
      constexpr int TP = TLDS ? 256 : 0;
      constexpr int NH = BM * P <= STAGES * STAGE_BYTES ? 1 : 2;
      constexpr int HR = BM / NH;
      static_assert(HR * P <= STAGES * STAGE_BYTES && HR % 32 == 0, "output staging must fit the stage buffers");
      const bool rot = EPI == EPI_ROPE && g.rope_cos != nullptr;
      int pos[FM];
      if constexpr (EPI == EPI_ROPE && !TLDS) {
#pragma unroll
        for (int i = 0; i < FM; ++i) pos[i] = rot ? g.rope_pos[min(rbase + i * 32, g.M - 1)] : 0;
      }
      if constexpr (TLDS) {
        if (rot) {
          // The tile's rows of the cos / sin tables (f32, 32 each per position) into LDS by
          // direct loads, each row read once for the block and in whole cache lines: straight
          // from the fragments every 16-byte piece was a load of its own, 32 rows apart, and
          // both column waves of a row fetched it. Load j moves rows 4 j .. 4 j + 3; lane l
          // fetches piece (l % 16) ^ (row % 16) of its row (pieces 0-7 cos, 8-15 sin) into slot
          // l % 16, so the 32 rows of one fragment read land on distinct bank groups.
          static_assert((BM / 4) % NW == 0, "table loads split evenly over the waves");
          __syncthreads();  // every wave is past its last k-tile's reads of the stage buffers
          int tpos[BM / 4 / NW];
#pragma unroll
          for (int u = 0; u < BM / 4 / NW; ++u)
            tpos[u] = g.rope_pos[min(m0 + (wave + u * NW) * 4 + (lane >> 4), g.M - 1)];
#pragma unroll
          for (int u = 0; u < BM / 4 / NW; ++u) {
            const int j = wave + u * NW, c = (lane & 15) ^ ((j * 4 + (lane >> 4)) & 15);
            const float* src = (c < 8 ? g.rope_cos : g.rope_sin) + tpos[u] * 32 + (c & 7) * 4;
            __builtin_amdgcn_global_load_lds(src, smem + TOFF + j * 1024, 16, 0, 0);
          }
          wait_vmcnt<0>();  // then the barrier that opens the staging makes them visible
        }
      }
#pragma unroll
      for (int half = 0; half < NH; ++half) {
        __syncthreads();
        if constexpr (EPI == EPI_ROPE) {
          // q and k blocks: columns [0, d) q, [d, 2d) k; within a head of 64, dims i and i + 32
          // form a rotation pair. Fragment 2p holds dims 0..31 of a head and 2p + 1 dims 32..63,
          // so a lane has dims i0 .. i0 + 3 (i0 = 8 q + 4 h) and their partners, same row.
          // (Biases, which only the head's in_proj has, and it has no rotation, load per column
          // group: holding them all would cost the registers of a second workgroup per CU.)
#pragma unroll
          for (int p = 0; p < FN / 2; ++p) {
            const int c0 = n0 + wn * TN + p * 64;  // first column of this head
#pragma unroll
            for (int i = 0; i < FM; ++i) {
              if ((wm * TM + i * 32) / HR != half) continue;
              float4 c4[4], s4[4];
              if (rot) {
                if constexpr (TLDS) {
                  // This lane's dims 8 q + 4 h .. + 3: cos piece 2 q + h, sin piece 8 + 2 q + h.
                  const char* tr = smem + TOFF + (rl0 + i * 32) * TP;
                  const int sw = (rl0 + i * 32) & 15;
#pragma unroll
                  for (int q = 0; q < 4; ++q) {
                    c4[q] = *reinterpret_cast<const float4*>(tr + ((2 * q + h) ^ sw) * 16);
                    s4[q] = *reinterpret_cast<const float4*>(tr + ((8 + 2 * q + h) ^ sw) * 16);
                  }
                } else {
                  // All 8 pieces of the fragment row are loaded before any is used.
#pragma unroll
                  for (int q = 0; q < 4; ++q) {
                    c4[q] = *reinterpret_cast<const float4*>(g.rope_cos + pos[i] * 32 + q * 8 + 4 * h);
                    s4[q] = *reinterpret_cast<const float4*>(g.rope_sin + pos[i] * 32 + q * 8 + 4 * h);
                  }
                }
              }
              const f32x16& a1 = acc[i][2 * p];
              const f32x16& a2 = acc[i][2 * p + 1];
#pragma unroll
              for (int q = 0; q < 4; ++q) {
                const int i0 = q * 8 + 4 * h;
                float4 b1 = zero4, b2 = zero4;
                if (g.bias) {
                  b1 = *reinterpret_cast<const float4*>(g.bias + c0 + i0);
                  b2 = *reinterpret_cast<const float4*>(g.bias + c0 + 32 + i0);
                }
                float x1[4] = {a1[4 * q] + b1.x, a1[4 * q + 1] + b1.y, a1[4 * q + 2] + b1.z, a1[4 * q + 3] + b1.w};
                float x2[4] = {a2[4 * q] + b2.x, a2[4 * q + 1] + b2.y, a2[4 * q + 2] + b2.z, a2[4 * q + 3] + b2.w};
                if (rot) {
                  const float cs[4] = {c4[q].x, c4[q].y, c4[q].z, c4[q].w}, sn[4] = {s4[q].x, s4[q].y, s4[q].z, s4[q].w};
#pragma unroll
                  for (int r = 0; r < 4; ++r) {
                    // Explicit fused forms, so the rounding does not depend on which product the
                    // compiler chooses to contract.
                    const float y1 = fmaf(x1[r], cs[r], -(x2[r] * sn[r]));
                    x2[r] = fmaf(x2[r], cs[r], x1[r] * sn[r]);
                    x1[r] = y1;
                  }
                }
                char* o = stg + (rl0 + i * 32 - half * HR) * P + (c0 - n0 + i0) * 2;
                *reinterpret_cast<uint2*>(o) = make_uint2(E::pack2(x1[0], x1[1]), E::pack2(x1[2], x1[3]));
                *reinterpret_cast<uint2*>(o + 64) = make_uint2(E::pack2(x2[0], x2[1]), E::pack2(x2[2], x2[3]));
              }
            }
          }
        } else {
#pragma unroll
          for (int j = 0; j < FN; ++j)
#pragma unroll
            for (int q = 0; q < 4; ++q) {
              const float4 b = g.bias ? *reinterpret_cast<const float4*>(g.bias + cbase + j * 32 + q * 8) : zero4;
#pragma unroll
              for (int i = 0; i < FM; ++i) {
                if ((wm * TM + i * 32) / HR != half) continue;
                float v[4] = {acc[i][j][4 * q] + b.x, acc[i][j][4 * q + 1] + b.y, acc[i][j][4 * q + 2] + b.z,
                              acc[i][j][4 * q + 3] + b.w};
#pragma unroll
                for (int r = 0; r < 4; ++r) {
                  if (g.act == ACT_RELU) v[r] = fmaxf(v[r], 0.0f);
                  else if (g.act == ACT_GELU) v[r] = gelu_erf(v[r]);
                }
                *reinterpret_cast<uint2*>(stg + (rl0 + i * 32 - half * HR) * P + (cl0 + j * 32 + q * 8) * 2) =
                    make_uint2(E::pack2(v[0], v[1]), E::pack2(v[2], v[3]));
              }
            }
        }
        __syncthreads();
        // Whole rows out: 16 bytes per lane, BN / 8 lanes per row.
        for (int idx = tid; idx < HR * (BN / 8); idx += NT) {
          const int r = idx / (BN / 8), c8 = idx % (BN / 8);
          const int row = m0 + half * HR + r;
          if (row >= g.M) continue;
          const uint4 v = lds_load16_a8(stg + r * P + c8 * 16);
          uint16_t* dst;
          if constexpr (EPI == EPI_ROPE) {
            const int c0 = n0 + (c8 / 8) * 64;
            const int part = c0 / g.rope_d;  // 0 q, 1 k
            const int head = (c0 - part * g.rope_d) >> 6;
            dst = (part == 0 ? g.rope_q : g.rope_k) + (size_t(head) * g.rope_T + row) * 64 + (c8 % 8) * 8;
          } else {
            dst = reinterpret_cast<uint16_t*>(g.C) + size_t(row) * g.ldc + n0 + c8 * 8;
          }
          *reinterpret_cast<uint4*>(dst) = v;
        }
      }
    }
  }
}

template <class E, int BM, int BN, int BK, int STAGES, int WM, int WN, int EPI, int KG, bool PIPE = false>
__global__ __launch_bounds__(WM * WN * 64 * KG) void gemm_kernel(GemmArgs g) {
  // STAGES k-tiles of A [BM][BK] and W [BN][BK], bf16, rows of BK * 2 bytes. The 16-byte chunk c
  // of row r sits at slot c ^ ((r / SW) % CH): the 16 lanes of one LDS access phase (16
  // consecutive rows, the same k; 64 banks of 4 bytes) then hit 16 distinct 16-byte bank groups
  // without padding, which the direct loads (whole 1 KiB runs) could not write.
  __shared__ __attribute__((aligned(1024))) char smem[KG * STAGES * (BM + BN) * BK * 2];

  // Tile order: each XCD takes a contiguous run of logical tiles (xcd_remap), and the run walks
  // groups of GM row tiles across all column tiles, GM fastest. The workgroups an XCD holds at
  // once then cover a GM-row patch, so its L2 serves every A row panel to many column tiles
  // instead of re-reading the activations from HBM once per column tile. GM = 4 measured best
  // at the 10-question request against 1, 2, 3, 5, 6, 8 and 16 (Wqkv 53.6 -> 49.8 µs from 8;
  // 59.5 at 2, 58-61 at 3, 5 and 6).
  constexpr int GM = 4;
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

  if constexpr (EPI == EPI_ROPE) {
    if (n0 >= 2 * g.rope_d) {
      gemm_tile<E, BM, BN, BK, STAGES, WM, WN, EPI, false, KG>(g, smem, m0, n0, kt0, NK, split);
      return;
    }
  }
  gemm_tile<E, BM, BN, BK, STAGES, WM, WN, EPI, true, KG, PIPE>(g, smem, m0, n0, kt0, NK, split);
}

template <class E, int BM, int BN, int BK, int STAGES, int WM, int WN, int EPI, int KG = 1, bool PIPE = false>
void launch_t(const GemmArgs& g, hipStream_t st) {
  const int mt = (g.M + BM - 1) / BM, nt = g.N / BN;
  hipLaunchKernelGGL((gemm_kernel<E, BM, BN, BK, STAGES, WM, WN, EPI, KG, PIPE>), dim3(mt * nt, g.splits),
                     dim3(WM * WN * 64 * KG), 0, st, g);
}

// Tile configurations, chosen from the number of tiles the GEMM has (the GPU holds two
// workgroups on each of its 256 CUs):
//   small  (one request of up to ~1000 tokens, or fewer than 200 128 x 128 tiles): 64 x 128
//          tiles in 4 waves of 32 x 64 with three k-tiles in flight (72 KiB of LDS, two
//          workgroups per CU), or four (96 KiB, one per CU) when the launch has at most 256
//          workgroups; these GEMMs stream their weights, so load depth matters more than
//          operand reuse;
//   wide   (at least 400 192 x 128 tiles, e.g. Wqkv and Wi at a 10-question request): 192 x 128
//          tiles in 4 waves of 96 x 64, two stages (80 KiB, two per CU, the whole LDS). Per
//          k-tile a CU moves 40 KiB for 3.1 MFLOP (128 x 128: 32 KiB for 2.1 MFLOP), and each
//          wave's 6 MFMAs per fragment pair cover the LDS reads of the next k-step;
//   long   (200 to 256 192 x 128 tiles and K >= 2048, e.g. Wo2 at a 10-question request): one
//          round of 192 x 128 tiles, one workgroup per CU with the pipelined k-loop (four stages,
//          160 KiB); Wo2 there 43.5 -> 40.9 µs against the mid tiles (bit-identical), where the
//          1024-deep Wo runs 23.3 -> 25.0 and stays mid. Not for the q|k|v epilogue (mid);
//   mid    (the rest, e.g. the 1024-wide Wo at a 10-question request): the same 64 x 128
//          tiles as small, two stages (48 KiB, three per CU); three times the tiles of 192-row
//          tiles, spread evenly over the CUs where 192-row tiles would leave some CUs idle.
// (A tile count that reaches 700 128 x 128 tiles always reaches 400 192 x 128 tiles, so 128-row
// tiles are not used.)
constexpr int SMALL_M = 1024;
enum TileCfg { TC_SMALL, TC_WIDE, TC_MID, TC_LONG };
inline TileCfg tile_cfg(int M, int N, int K) {
  if (M <= SMALL_M) return TC_SMALL;
  const long long t128 = (long long)((M + 127) / 128) * (N / 128);
  if (t128 < 200) return TC_SMALL;
  const long long t192 = (long long)((M + 191) / 192) * (N / 128);
  if (t192 >= 200 && t192 <= 256 && K >= 2048) return TC_LONG;
  return t192 >= 400 ? TC_WIDE : TC_MID;
}
inline int tile_m_of(int M, int N, int K) {
  switch (tile_cfg(M, N, K)) {
    case TC_WIDE: return 192;
    case TC_LONG: return 192;
    default: return 64;
  }
}

template <class E, int EPI>
void launch_te(const GemmArgs& g, hipStream_t st) {
  switch (tile_cfg(g.M, g.N, g.K)) {
    case TC_SMALL: {
      // Four k-tiles in flight when the launch fits one workgroup per CU (96 KiB of LDS each):
      // deeper prefetch for the weight stream. Past one workgroup per CU, 128 x 128 tiles with
      // three stages while they still fit about one per CU (up to 320 of them), else 64-row
      // tiles with three stages, two workgroups per CU. In a one-request forward at 565 tokens
      // (weights cold in HBM) the wide GeGLU product (N = 2I, 369 64-row tiles) drops from 17.6
      // to 14.9 µs per launch with the 128 x 128 tiles; two stages there lose to 64-row tiles.
      // Except for the k-groups below, the k-loop order is the same for every tile, so the results
      // are the same bits. The q|k|v product takes 64 x 64 tiles while they fit one workgroup per
      // CU (a third fewer bytes per k-tile, twice the workgroups): at 174 tokens 13.0 -> 12.2 µs
      // per launch (the GeGLU product lost 2% that way). A GEMM with a 16-bit epilogue whose
      // 64 x 64 tiles fit one workgroup per CU runs them in two k-groups of 4 waves (8 k-tiles
      // each where there were 16): at 174 tokens q|k|v 9.9 -> 8.9 µs and GeGLU 9.8 -> 8.2 µs
      // (GeGLU on twice the workgroups of its 64 x 128 tiles), weights cold in HBM.
      constexpr bool KGOK = EPI != EPI_RESID && EPI != EPI_F32;
      if (KGOK && g.splits == 1 && (g.K / BK) % 2 == 0 && (long long)((g.M + 63) / 64) * (g.N / 64) <= 256)
        launch_t<E, 64, 64, 64, 4, 2, 1, EPI, KGOK ? 2 : 1>(g, st);
      else if (EPI == EPI_ROPE && (long long)((g.M + 63) / 64) * (g.N / 64) * g.splits <= 256)
        launch_t<E, 64, 64, 64, 4, 2, 1, EPI>(g, st);
      else if ((long long)((g.M + 63) / 64) * (g.N / 128) * g.splits <= 256)
        launch_t<E, 64, 128, 64, 4, 2, 2, EPI>(g, st);
      else if ((long long)((g.M + 127) / 128) * (g.N / 128) * g.splits <= 320)
        launch_t<E, 128, 128, 64, 3, 2, 2, EPI>(g, st);
      else
        launch_t<E, 64, 128, 64, 3, 2, 2, EPI>(g, st);
      break;
    }
    case TC_WIDE: launch_t<E, 192, 128, 64, 2, 2, 2, EPI>(g, st); break;
    case TC_MID: launch_t<E, 64, 128, 64, 2, 2, 2, EPI>(g, st); break;
    case TC_LONG:
      if constexpr (EPI == EPI_ROPE) launch_t<E, 64, 128, 64, 2, 2, 2, EPI>(g, st);
      else launch_t<E, 192, 128, 64, 4, 2, 2, EPI, 1, true>(g, st);
      break;
  }
}

template <int EPI>
void launch_e(const GemmArgs& g, hipStream_t st) {
  if (g.elem == ELEM_F16) launch_te<F16, EPI>(g, st);
  else launch_te<Bf16, EPI>(g, st);
}

// Sum of the split-K partials in split order, then the GEMM's epilogue. One thread per row and
// column pair (c, c + 32) of a 64-column group, the pair the GeGLU and RoPE epilogues combine.
template <class E>
__global__ __launch_bounds__(256) void splitk_epilogue_kernel(GemmArgs g) {
  const long long gid = (long long)blockIdx.x * 256 + threadIdx.x;
  const int half = g.N / 2;
  if (gid >= (long long)g.M * half) return;
  const int row = int(gid / half);
  const int p = int(gid % half);
  const int c1 = (p / 32) * 64 + (p % 32), c2 = c1 + 32;
  float x1 = 0.0f, x2 = 0.0f;
  // Eight splits' loads go out before any is added (in split order), not one round trip each.
  for (int s0 = 0; s0 < g.splits; s0 += 8) {
    float a1[8], a2[8];
#pragma unroll
    for (int u = 0; u < 8; ++u) {
      const float* part = g.ws + (size_t(min(s0 + u, g.splits - 1)) * g.M + row) * g.N;
      a1[u] = part[c1];
      a2[u] = part[c2];
    }
#pragma unroll
    for (int u = 0; u < 8; ++u)
      if (s0 + u < g.splits) {
        x1 += a1[u];
        x2 += a2[u];
      }
  }
  if (g.epi == EPI_GEGLU) {
    uint16_t* C = reinterpret_cast<uint16_t*>(g.C);
    C[size_t(row) * g.ldc + p] = E::bits(gelu_erf(x1) * x2);
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
      o[0] = E::bits(x1);
      o[size_t(32) * g.rope_ldv] = E::bits(x2);
      if (row == g.M - 1)  // zeros up to the next multiple of 8 tokens, as the GEMM's own epilogue
        for (int t = 1; row + t < (g.M + 7) / 8 * 8; ++t) {
          o[t] = 0;
          o[size_t(32) * g.rope_ldv + t] = 0;
        }
      return;
    }
    uint16_t* o = (part == 0 ? g.rope_q : g.rope_k) + (size_t(head) * g.rope_T + row) * 64;
    o[i] = E::bits(x1);
    o[i + 32] = E::bits(x2);
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
  C[c1] = E::bits(x1);
  C[c2] = E::bits(x2);
}

}  // namespace

GemmPlan gemm_plan(int M, int N, int K, bool reduce_folded) {
  GemmPlan p;
  const int bm = tile_m_of(M, N, K);
  const int tiles = ((M + bm - 1) / bm) * (N / 128);
  const int KT = K / BK;
  // Few tiles (a short request on a narrow output): split K so that up to 256 workgroups run
  // (one per CU, which takes the four-deep pipeline), each keeping at least 4 k-tiles, and the f32 partials (s M N 4 bytes, written and read
  // back) stay within twice the weight bytes (N K 2) the GEMM streams anyway, or eight times
  // them when the reduce is folded. The partials need a second pass: a reduce kernel of its own
  // (about as long as a whole-K pass over 32-95 tiles saves, launch included), unless the
  // caller folds it into the kernel that follows (the LayerNorm after Wo / Wo2), where it costs
  // little. So split below 96 tiles when folded, below 32 otherwise.
  int s = 1;
  if (tiles < (reduce_folded ? 96 : 32))
    s = std::max(1, std::min({KT / 4, std::max(1, 256 / tiles), (reduce_folded ? 4 : 1) * K / std::max(M, 1)}));
  p.splits = s;
  p.ws_floats = s > 1 ? size_t(s) * M * N : 0;
  return p;
}

const char* gemm_check(const GemmArgs& g) {
  if (g.M <= 0) return "gemm: M must be positive";
  if (g.K <= 0 || g.K % BK) return "gemm: K must be a positive multiple of 64";
  if (g.N <= 0 || g.N % 128) return "gemm: N must be a positive multiple of 128";
  if (g.lda < g.K || g.ldw < g.K || (g.lda % 8) || (g.ldw % 8)) return "gemm: bad leading dimension";
  // The direct loads address each operand by a 32-bit byte offset from its start: W must span
  // less than 4 GiB; a longer A runs as row pieces (unsplit only, and at least 8 rows a piece).
  if (span_bytes(g.N, g.ldw, g.K) > kMaxSpan) return "gemm: W must span less than 4 GiB";
  if (span_bytes(g.M, g.lda, g.K) > kMaxSpan && (g.splits > 1 || span_bytes(8, g.lda, g.K) > kMaxSpan))
    return "gemm: an A spanning 4 GiB or more needs an unsplit product and rows under 512 MiB";
  if (g.epi == EPI_ROPE && (g.rope_d % 64 || g.N != 3 * g.rope_d)) return "gemm: rope epilogue needs N = 3d, d % 64 == 0";
  if (g.epi == EPI_ROPE && (g.rope_ldv % 8 || g.rope_ldv < g.M + 64)) return "gemm: v row stride must be a multiple of 8 and >= M + 64";
  if (g.splits < 1 || g.splits > g.K / BK) return "gemm: splits must be in 1..K/64";
  if (g.splits > 1 && !g.ws) return "gemm: split-K needs a workspace";
  if (g.epi == EPI_GEGLU && g.bias) return "gemm: the GeGLU epilogue takes no bias";
  // The epilogues store 4 consecutive columns per access (8 bytes bf16, 16 bytes f32) and read
  // bias and RoPE tables 4 floats at a time.
  auto mis = [](const void* p, uintptr_t a) { return (reinterpret_cast<uintptr_t>(p) & (a - 1)) != 0; };
  const bool f32out = g.epi == EPI_RESID || g.epi == EPI_F32;
  if (g.epi != EPI_ROPE && ((g.ldc % (f32out ? 4 : 8)) || mis(g.C, 16)))
    return "gemm: C must be 16-byte aligned with 16-byte row strides";
  if (mis(g.bias, 16) || mis(g.ws, 16)) return "gemm: bias and workspace must be 16-byte aligned";
  if (g.epi == EPI_ROPE && (mis(g.rope_q, 16) || mis(g.rope_k, 16) || mis(g.rope_v, 16) || mis(g.rope_cos, 16) ||
                            mis(g.rope_sin, 16)))
    return "gemm: q, k, v and the RoPE tables must be 16-byte aligned";
  return nullptr;
}

void gemm_launch_partials(const GemmArgs& g, hipStream_t st) { launch_e<EPI_F32>(g, st); }

namespace {

// Rows per launch for an A spanning 4 GiB or more: the fewest equal pieces, each a whole number of
// 384 rows (a multiple of every tile height, so only the last piece has a partial tile) or of 8
// (the q|k|v epilogue's token groups) when 384 rows already pass the limit.
int rows_per_piece(const GemmArgs& g) {
  const long long rmax = (long long)((kMaxSpan - size_t(g.K) * 2) / (size_t(g.lda) * 2)) + 1;
  const long long unit = rmax >= 384 ? 384 : 8;
  for (long long np = (g.M + rmax - 1) / rmax;; ++np) {
    const long long r = ((g.M + np - 1) / np + unit - 1) / unit * unit;
    if (r <= rmax) return int(r);
  }
}

void gemm_launch_one(const GemmArgs& g, hipStream_t st) {
  if (g.splits > 1) {
    gemm_launch_partials(g, st);  // partials only: the kernel returns before its epilogue
    const long long n = (long long)g.M * (g.N / 2);
    const dim3 grid(unsigned((n + 255) / 256)), block(256);
    if (g.elem == ELEM_F16) hipLaunchKernelGGL(splitk_epilogue_kernel<F16>, grid, block, 0, st, g);
    else hipLaunchKernelGGL(splitk_epilogue_kernel<Bf16>, grid, block, 0, st, g);
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

}  // namespace

void gemm_launch(const GemmArgs& g, hipStream_t st) {
  if (span_bytes(g.M, g.lda, g.K) <= kMaxSpan) {
    gemm_launch_one(g, st);
    return;
  }
  // Row pieces (gemm_check allows this only unsplit): each piece is the product over its rows,
  // launched with A, the output rows and the row positions offset to its first row.
  const int step = rows_per_piece(g);
  const bool f32out = g.epi == EPI_RESID || g.epi == EPI_F32;
  for (int m0 = 0; m0 < g.M; m0 += step) {
    GemmArgs p = g;
    p.M = std::min(step, g.M - m0);
    p.A = g.A + size_t(m0) * g.lda;
    if (g.epi == EPI_ROPE) {
      // q and k are [H, rope_T, 64] (rope_T, the head stride, stays), v is [H, 64, rope_ldv].
      p.rope_q = g.rope_q + size_t(m0) * 64;
      p.rope_k = g.rope_k + size_t(m0) * 64;
      p.rope_v = g.rope_v + m0;
      if (g.rope_pos) p.rope_pos = g.rope_pos + m0;
    } else {
      p.C = static_cast<char*>(g.C) + size_t(m0) * g.ldc * (f32out ? 4 : 2);
    }
    gemm_launch_one(p, st);
  }
}

}  // namespace s1
