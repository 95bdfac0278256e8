// Fused attention for gfx950: softmax(q k^T * scale + mask) v over packed variable-length rows,
// one pass over the keys with an online softmax (f32 statistics), both products on MFMA.
//
// Replaces MLX's scaled_dot_product_attention on the encoder's global layers (pad mask only,
// runtime/crates/laya-mlx/src/lib.rs:1653-1656), its local layers (pad + |i - j| <= 64 window,
// lib.rs:1399-1417, 1644-1649; the banded form 1600-1622) and the decision head's attention
// (lib.rs:1710-1712). The reference's additive -1e4 masks give every masked key an exp() of
// exactly 0 in f32 for any query that has one visible key, which every real token has (itself),
// so a hard mask over the row's own keys computes the same values; padding never enters the
// packed layout at all.
//
// Work split: a workgroup of NW wavefronts takes up to 32 NW queries of one sequence and one
// head; each wave owns 32 queries. Keys stream through LDS in chunks of 64 (double-buffered on
// global layers): K as [key][dim] and V as [dim][key], copied with 16-byte accesses from the
// transposed v buffer. On local layers waves skip chunks, and 32-key halves, outside their
// window, and only chunks that cross a window or row edge pay for masking. Short batches (fewer
// tiles than CUs) take 32-query tiles whose keys several waves split and merge at the end
// (attn_ksplit_kernel): all of the row's keys on global layers, the tile's window range on local
// ones.
//
// The products are computed transposed so that every softmax statistic lives in one lane:
//   S^T[key, q] = K . Q^T   (A = K rows from LDS, B = the wave's Q held in registers)
// lane l then holds query l % 32 and keys 8g + 4h + r (h = l / 32), so the row max and sum are a
// lane-local reduction plus one exchange with lane l ^ 32.
//   O^T[dim, q] += V^T . P^T
// reuses P^T straight from the S^T accumulators: within a 16-key MFMA step, operand slot
// 8h + j stands for key 16s + 8(j / 4) + 4h + (j % 4), and the V^T operand is read from LDS with
// the same key order, so no shuffle of P is needed.
//
// Softmax weights are 2^x by the bare v_exp_f32 (__builtin_amdgcn_exp2f): it flushes results
// below 2^-126 to 0, weights far below anything the f32 sums or the bf16 P can hold next to the
// row maximum's 1. exp2f wraps the instruction in a denormal-range fixup of five more VALU
// instructions per weight, and these kernels are VALU-bound.
#include <algorithm>
#include <vector>

#include "device.hpp"
#include "kernels.hpp"

namespace s1 {

namespace {

constexpr int KC = 64;  // keys per chunk
constexpr float NEG_INF = -__builtin_huge_valf();

// LDS rows of 128 bytes (64 bf16: a K row, or 64 keys of a V^T row) hold 16-byte chunk c of row
// r at slot c ^ ((r / 2) % 8): the 16 rows of one 16-lane read phase then start in 16 distinct
// bank groups, and each 8-row group is one contiguous KiB that a single direct global -> LDS
// load (global_load_lds_dwordx4) fills.
__device__ __forceinline__ int kslot(int r, int c) { return c ^ ((r >> 1) & 7); }

// The launch is one-dimensional, ntiles x heads workgroups; workgroup -> (tile, head) with the
// tile fastest, through xcd_remap, so that consecutive tiles of one head (the query blocks of one
// row, which read the same keys and values, or overlapping windows of them) run on one XCD and
// share its L2.
__device__ __forceinline__ int2 tile_head(int ntiles) {
  const int lid = xcd_remap(blockIdx.x, gridDim.x);
  const int head = lid / ntiles;
  return make_int2(lid - head * ntiles, head);
}

// Three waves per SIMD for the local kernel (register budget 168), four for the global one.
template <class E, bool LOCAL, int NW>
__global__ __launch_bounds__(NW * 64) __attribute__((amdgpu_waves_per_eu(LOCAL ? 3 : 4)))
void attn_kernel(AttnArgs a) {
  typedef typename E::v8 v8;
  // K and V^T double buffers, [K0 | K1 | V0 | V1], 8 KiB each.
  __shared__ __attribute__((aligned(1024))) uint16_t smem[4 * KC * 64];
  auto sK = [&](int buf) { return smem + buf * KC * 64; };
  auto sVt = [&](int buf) { return smem + (2 + buf) * KC * 64; };

  const int2 th = tile_head(a.ntiles);
  const AttnTile tl = a.tiles[th.x];
  const int head = th.y;
  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);  // wave-uniform: scalar branches
  const int hl = lane >> 5;   // lane half
  const int col = lane & 31;  // query column within the wave

  const uint16_t* __restrict__ Qh = a.q + size_t(head) * a.Tq * 64;
  const uint16_t* __restrict__ Kh = a.k + size_t(head) * a.Tk * 64;
  const uint16_t* __restrict__ Vt = a.v + size_t(head) * 64 * a.ldv;

  const int wq0 = tl.q0 + wave * 32;
  const bool wave_active = wq0 < tl.q1;
  const int qi = wq0 + col;
  const bool qvalid = qi < tl.q1;
  const int qld = min(qi, tl.q1 - 1);
  const int qk = a.qkey ? a.qkey[qld] : qld;  // q row and key index of this query

  // Key range of the workgroup and of this wave.
  int kb0 = tl.k0, kb1 = tl.k1;
  int wk0 = tl.k0, wk1 = tl.k1;
  int wf_key = 0, wl_key = 0;  // key index of the wave's first and last query (local layers)
  if constexpr (LOCAL) {
    const int first = a.qkey ? a.qkey[tl.q0] : tl.q0;
    const int last = a.qkey ? a.qkey[tl.q1 - 1] : tl.q1 - 1;
    kb0 = max(tl.k0, first - a.window);
    kb1 = min(tl.k1, last + a.window + 1);
    if (wave_active) {
      const int wf = a.qkey ? a.qkey[wq0] : wq0;
      const int wlq = min(wq0 + 31, tl.q1 - 1);
      const int wl = a.qkey ? a.qkey[wlq] : wlq;
      wk0 = max(tl.k0, wf - a.window);
      wk1 = min(tl.k1, wl + a.window + 1);
      wf_key = wf;
      wl_key = wl;
    }
  }
  // Chunks start 8-aligned so the V^T rows are read with aligned 16-byte loads; keys before kb0
  // and from kb1 on are masked (and their V entries zeroed in LDS).
  const int cstart = kb0 & ~7;

  // This lane's slice of its query: dims 16kb + 8h .. +7 for kb = 0..3 (MFMA B operand).
  v8 qf[4];
#pragma unroll
  for (int kb = 0; kb < 4; ++kb)
    qf[kb] = *reinterpret_cast<const v8*>(Qh + size_t(qk) * 64 + kb * 16 + hl * 8);

  // A chunk's K goes global -> LDS by direct loads: 8 groups of 8 rows, one KiB each, spread
  // over the waves; rows past kb1 repeat the last key. V^T goes through registers (one 16-byte
  // piece of 8 keys per thread and wave of 64 threads per KiB): loaded with the K loads, stored
  // after the chunk's math. (Direct loads for V^T too make the compiler wait for all of them
  // before the chunk's first V^T read.) V^T pieces from kb1 on load the piece holding key
  // kb1 - 1 (finite values that meet weights of 0); that piece may read up to 7 keys past kb1:
  // the next sequence's, or the zeros every v writer leaves up to the next multiple of 8 tokens.
  const int vlast = cstart + (((kb1 - 1) - cstart) & ~7);
  constexpr int VPT = 64 * 8 / (NW * 64);  // V^T pieces per thread
  static_assert(VPT * NW * 64 == 64 * 8, "V^T pieces split evenly over the threads");
  uint4 vreg[VPT];
  auto stage = [&](int c0, int buf) {
    const int r8 = lane >> 3, slot = lane & 7;
    for (int gi = wave; gi < 8; gi += NW) {
      const int row = gi * 8 + r8;
      const uint16_t* src = Kh + size_t(min(c0 + row, kb1 - 1)) * 64 + kslot(row, slot) * 8;
      __builtin_amdgcn_global_load_lds(src, reinterpret_cast<char*>(sK(buf)) + gi * 1024, 16, 0, 0);
    }
#pragma unroll
    for (int it = 0; it < VPT; ++it) {
      const int p = tid + it * NW * 64;
      const int dim = p >> 3, c = p & 7;
      vreg[it] = *reinterpret_cast<const uint4*>(Vt + size_t(dim) * a.ldv + min(c0 + c * 8, vlast));
    }
  };
  // V^T rows hold each 16-key block's keys in the PV operand order: key 16s + 8a + 4h + r at
  // position 16s + 8h + 4a + r, so a lane's 8 operand keys (4h .. 4h + 3 and 8 + 4h .. 8 + 4h + 3
  // of the block) are one 16-byte chunk (2s + h), read with one access. The 16-byte chunks are
  // then placed by kslot like K's.
  auto vstore = [&](int buf) {
#pragma unroll
    for (int it = 0; it < VPT; ++it) {
      const int p = tid + it * NW * 64;
      const int dim = p >> 3, c = p & 7;  // keys 8c .. 8c + 7 = 16 (c / 2) + 8 (c % 2) + 0 .. 7
      uint16_t* row = sVt(buf) + dim * 64 + (c & 1) * 4;
      *reinterpret_cast<uint2*>(row + kslot(dim, c & ~1) * 8) = make_uint2(vreg[it].x, vreg[it].y);
      *reinterpret_cast<uint2*>(row + kslot(dim, c | 1) * 8) = make_uint2(vreg[it].z, vreg[it].w);
    }
  };
  auto landed = [] { asm volatile("s_waitcnt vmcnt(0)" ::: "memory"); };  // this wave's direct loads

  const float sl2 = a.scale * 1.4426950408889634f;  // fold log2(e): exp(x) = exp2(x log2 e)
  float m = NEG_INF, l = 0.0f;
  f32x16 o[2];
#pragma unroll
  for (int e = 0; e < 16; ++e) { o[0][e] = 0.0f; o[1][e] = 0.0f; }

  // Global layers double-buffer the chunks (the next chunk's loads overlap this one's math);
  // local layers visit few chunks per wave and keep the lighter single buffer, which leaves
  // registers for three waves per SIMD.
  constexpr bool DB = !LOCAL;
  if constexpr (DB) {
    stage(cstart, 0);
    vstore(0);
    landed();
    __syncthreads();
  }
  int buf = 0;
  for (int c0 = cstart; c0 < kb1; c0 += KC, buf ^= (DB ? 1 : 0)) {
    const bool more = DB && c0 + KC < kb1;
    if constexpr (DB) {
      if (more) stage(c0 + KC, buf ^ 1);  // the other buffer was last read before the previous barrier
    } else {
      if (c0 != cstart) __syncthreads();  // every wave is done with the previous chunk
      stage(c0, 0);
      vstore(0);
      landed();
      __syncthreads();
    }
    bool work = wave_active;
    if constexpr (LOCAL) work = work && !(c0 + KC <= wk0 || c0 >= wk1);
    if (work) {
      // 32-key tiles of this chunk that hold keys this wave may see (local layers skip the rest).
      bool need[2] = {true, true};
      if constexpr (LOCAL) {
#pragma unroll
        for (int t = 0; t < 2; ++t) need[t] = c0 + 32 * t < wk1 && c0 + 32 * t + 32 > wk0;
      }
      // Masks are needed only where the chunk crosses the key range or some query's window.
      bool edge = c0 < kb0 || c0 + KC > kb1;
      if constexpr (LOCAL) edge = edge || c0 < wl_key - a.window || c0 + KC > wf_key + a.window + 1;
      // S^T for the needed 32-key tiles (raw logits; masked entries -inf): the K fragments of the
      // chunk read first, then the two tiles' k-steps interleaved (two independent MFMA chains).
      f32x16 s[2];
      float mx = NEG_INF;
      v8 kf[2][4];
#pragma unroll
      for (int kb = 0; kb < 4; ++kb)
#pragma unroll
        for (int t = 0; t < 2; ++t) {
          const int kr = t * 32 + col;
          if (need[t]) kf[t][kb] = *reinterpret_cast<const v8*>(sK(buf) + kr * 64 + kslot(kr, kb * 2 + hl) * 8);
        }
#pragma unroll
      for (int t = 0; t < 2; ++t)
#pragma unroll
        for (int e = 0; e < 16; ++e) s[t][e] = need[t] ? 0.0f : NEG_INF;
#pragma unroll
      for (int kb = 0; kb < 4; ++kb)
#pragma unroll
        for (int t = 0; t < 2; ++t)
          if (need[t]) s[t] = E::mfma(kf[t][kb], qf[kb], s[t]);
#pragma unroll
      for (int t = 0; t < 2; ++t) {
        if (!need[t]) continue;
        if (edge) {
          // Element e of the tile is key kbase + (e / 4) * 8 + e % 4: bounds on that constant
          // offset, one compare per element for each side the chunk crosses.
          const int kbase = c0 + t * 32 + hl * 4;
          if constexpr (LOCAL) {
            const int lo = max(kb0, qk - a.window) - kbase, hi = min(kb1, qk + a.window + 1) - kbase;
#pragma unroll
            for (int e = 0; e < 16; ++e) {
              const int off = (e >> 2) * 8 + (e & 3);
              s[t][e] = off >= lo && off < hi ? s[t][e] : NEG_INF;
            }
          } else {
            if (c0 < kb0) {
              const int lo = kb0 - kbase;
#pragma unroll
              for (int e = 0; e < 16; ++e) s[t][e] = (e >> 2) * 8 + (e & 3) >= lo ? s[t][e] : NEG_INF;
            }
            if (c0 + KC > kb1) {
              const int hi = kb1 - kbase;
#pragma unroll
              for (int e = 0; e < 16; ++e) s[t][e] = (e >> 2) * 8 + (e & 3) < hi ? s[t][e] : NEG_INF;
            }
          }
        }
#pragma unroll
        for (int e = 0; e < 16; ++e) mx = fmaxf(mx, s[t][e]);
      }
      // Online softmax in base 2: p = 2^(s * sl2 - m). sl2 > 0, so the raw max scales.
      mx = half_max(mx);
      const float mn = fmaxf(m, mx * sl2);
      const float ms = mn == NEG_INF ? 0.0f : mn;  // nothing visible yet: every p is exp2(-inf) = 0
      const float alpha = __builtin_amdgcn_exp2f(m - ms);
      float psum = 0.0f;
      v8 pf[2][2];
#pragma unroll
      for (int t = 0; t < 2; ++t)
#pragma unroll
        for (int sb = 0; sb < 2; ++sb)
#pragma unroll
          for (int j = 0; j < 8; ++j) {
            const float p = __builtin_amdgcn_exp2f(fmaf(s[t][sb * 8 + j], sl2, -ms));
            psum += p;
            pf[t][sb][j] = typename E::scalar(p);
          }
      l = l * alpha + psum;
      m = mn;
      // Once the running maximum settles, alpha is exactly 1 on every lane and the branch (taken
      // by lanes, skipped by the wave when none needs it) saves the 32 multiplies.
      if (alpha != 1.0f) {
#pragma unroll
        for (int e = 0; e < 16; ++e) { o[0][e] *= alpha; o[1][e] *= alpha; }
      }

      // O^T += V^T . P^T over the needed tiles (MFMA k-steps of 16 keys), both 32-dim halves.
#pragma unroll
      for (int t = 0; t < 2; ++t) {
        if (!need[t]) continue;
#pragma unroll
        for (int sb = 0; sb < 2; ++sb) {
#pragma unroll
          for (int dt = 0; dt < 2; ++dt) {
            const int dr = dt * 32 + col;
            const v8 vf = *reinterpret_cast<const v8*>(sVt(buf) + dr * 64 + kslot(dr, (t * 2 + sb) * 2 + hl) * 8);
            o[dt] = E::mfma(vf, pf[t][sb], o[dt]);
          }
        }
      }
    }
    if constexpr (DB) {
      if (more) {
        vstore(buf ^ 1);  // the other buffer was last read before the previous barrier
        landed();
      }
      __syncthreads();
    }
  }

  if (!wave_active) return;
  const float lt = half_sum(l);
  if (!qvalid) return;
  const float inv = 1.0f / lt;
  uint16_t* orow = a.out + size_t(qi) * a.ldo + head * 64;
#pragma unroll
  for (int dt = 0; dt < 2; ++dt)
#pragma unroll
    for (int g = 0; g < 4; ++g) {
      const int dim = dt * 32 + g * 8 + hl * 4;
      uint2 w;
      w.x = E::pack2(o[dt][g * 4 + 0] * inv, o[dt][g * 4 + 1] * inv);
      w.y = E::pack2(o[dt][g * 4 + 2] * inv, o[dt][g * 4 + 3] * inv);
      *reinterpret_cast<uint2*>(orow + dim) = w;
    }
}

// Local layers with a window of at most 64 keys: a workgroup's 128 queries see at most
// 128 + 2 * 64 keys, so the whole key range is staged in LDS at once (every load of the
// workgroup in flight together, one barrier) and each wave then runs its queries' softmax over
// its own window in a single pass (at most 6 tiles of 32 keys, raw logits kept in registers).
// K and V^T take turns in one LDS buffer (38 KiB): K for the logits, then V^T, loaded while the
// softmax weights are computed. At the 10-request headline that fits four workgroups per CU,
// all 800 tiles in one round, where K and V^T side by side (71 KiB) fit two and took 1.56
// rounds (16.4 -> 15.0 µs per launch, the same bits).
constexpr int LQ = 128;                 // queries per workgroup: 4 waves x 32
constexpr int LMAXW = 64;               // largest window this kernel stages
constexpr int LMAXK = LQ + 2 * LMAXW + 8;  // staged keys: the range plus 8-alignment slack
// V^T rows in LDS: LVC 16-byte chunks of 8 keys (LVC odd, so the 16 rows of one 16-lane read
// phase start in 16 distinct bank groups); LVC x 8 >= LMAXK rounded up to 32 keys, the furthest
// column a tile reads. Each KiB of the 64 rows is filled by one direct global -> LDS load.
constexpr int LVC = 37;
constexpr int LVW = LVC * 8;
constexpr int LTILES = (32 + 2 * LMAXW + 7 + 31) / 32;  // 32-key tiles a wave's window spans
constexpr int LBUF = LMAXK * 64 > 64 * LVW ? LMAXK * 64 : 64 * LVW;  // 16-bit elements of the buffer
static_assert(LVC % 2 == 1 && LVC * 8 >= (LMAXK + 31) / 32 * 32 && 64 * LVC % 64 == 0, "V^T layout");

template <class E>
__global__ __launch_bounds__(256) __attribute__((amdgpu_waves_per_eu(2))) void attn_local_kernel(AttnArgs a) {
  typedef typename E::v8 v8;
  __shared__ __attribute__((aligned(1024))) uint16_t sbuf[LBUF];
  uint16_t* const sK = sbuf;   // [LMAXK][64] until every wave has its logits
  uint16_t* const sVt = sbuf;  // then [64][LVW]

  const int2 th = tile_head(a.ntiles);
  const AttnTile tl = a.tiles[th.x];
  const int head = th.y;
  const int tid = threadIdx.x, lane = tid & 63;
  // Wave-uniform values go through readfirstlane so the branches on them are scalar branches,
  // not exec-mask regions around every tile.
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int hl = lane >> 5, col = lane & 31;
  const int W = a.window;

  const uint16_t* __restrict__ Qh = a.q + size_t(head) * a.Tq * 64;
  const uint16_t* __restrict__ Kh = a.k + size_t(head) * a.Tk * 64;
  const uint16_t* __restrict__ Vt = a.v + size_t(head) * 64 * a.ldv;

  // The workgroup's keys [kb0, kb1), staged from the 8-aligned cstart (keys outside them are
  // masked out of S, so their weights are exactly 0 and their V entries only need be finite).
  const int kb0 = max(tl.k0, tl.q0 - W), kb1 = min(tl.k1, tl.q1 + W);
  const int cstart = kb0 & ~7;
  const int nk8 = (kb1 - cstart + 7) >> 3;  // 8-key groups staged (<= LMAXK / 8)
  const int lim = nk8 * 8;                  // staged keys
  // A wave past the tile's queries computes nothing but takes part in both barriers.
  const int wq0 = tl.q0 + wave * 32;
  const bool wact = wq0 < tl.q1;
  const int qi = wq0 + col;
  const bool qvalid = qi < tl.q1;
  const int qk = min(qi, tl.q1 - 1);
  v8 qf[4];
#pragma unroll
  for (int kb = 0; kb < 4; ++kb)
    qf[kb] = *reinterpret_cast<const v8*>(Qh + size_t(qk) * 64 + kb * 16 + hl * 8);
  // K by direct global -> LDS loads: 8-row groups, groups w, w + 4, ... from wave w; rows past
  // kb1 repeat the last key (masked out of S).
  {
    const int r = lane >> 3, slot = lane & 7;
    for (int gi = wave; gi < nk8; gi += 4) {
      const int row = gi * 8 + r;
      const uint16_t* src = Kh + size_t(min(cstart + row, kb1 - 1)) * 64 + kslot(row, slot) * 8;
      __builtin_amdgcn_global_load_lds(src, reinterpret_cast<char*>(sK) + gi * 1024, 16, 0, 0);
    }
    asm volatile("s_waitcnt vmcnt(0)" ::: "memory");  // this wave's direct loads have landed
  }
  __syncthreads();

  // This wave's window: keys [ws, we) cover every query's |key - q| <= W within the row.
  const int ws = max(kb0, wq0 - W), we = min(kb1, min(wq0 + 31, tl.q1 - 1) + W + 1);
  int t0 = (ws - cstart) & ~7;                 // LDS key offset of the first tile
  const int nt = wact ? __builtin_amdgcn_readfirstlane((we - cstart - t0 + 31) >> 5) : 0;  // tiles (<= LTILES)
  // Shift the tiles left so they end within the staged keys (keys before ws are masked); a range
  // shorter than the tiles starts at 0 and reads up to the zeroed V^T columns.
  if (t0 + 32 * nt > lim) t0 = max(0, lim - 32 * nt);
  t0 = __builtin_amdgcn_readfirstlane(t0);

  // Keys this lane's query sees, as LDS key offsets: [vlo, vhi). Tiles inside the band that every
  // query of the wave sees, [blo, bhi), need no mask.
  const int vlo = max(kb0, qk - W) - cstart, vhi = min(kb1, qk + W + 1) - cstart;
  const int blo = __builtin_amdgcn_readfirstlane(max(kb0, min(wq0 + 31, tl.q1 - 1) - W) - cstart);
  const int bhi = __builtin_amdgcn_readfirstlane(min(kb1, wq0 + W + 1) - cstart);
  f32x16 s[LTILES];
  float mx = NEG_INF;
#pragma unroll
  for (int t = 0; t < LTILES; ++t) {
#pragma unroll
    for (int e = 0; e < 16; ++e) s[t][e] = NEG_INF;
    if (t >= nt) continue;
    f32x16 acc;
#pragma unroll
    for (int e = 0; e < 16; ++e) acc[e] = 0.0f;
#pragma unroll
    for (int kb = 0; kb < 4; ++kb) {
      const int kr = t0 + t * 32 + col;
      const v8 kf = *reinterpret_cast<const v8*>(&sK[kr * 64 + kslot(kr, kb * 2 + hl) * 8]);
      acc = E::mfma(kf, qf[kb], acc);
    }
    const int tb = t0 + t * 32;  // LDS key offset of the tile
    if (tb >= blo && tb + 32 <= bhi) {
#pragma unroll
      for (int e = 0; e < 16; ++e) {
        s[t][e] = acc[e];
        mx = fmaxf(mx, acc[e]);
      }
    } else {
      const int lo = vlo - tb - hl * 4, hi = vhi - tb - hl * 4;  // bounds on (e >> 2) * 8 + (e & 3)
#pragma unroll
      for (int e = 0; e < 16; ++e) {
        const int off = (e >> 2) * 8 + (e & 3);
        s[t][e] = off >= lo && off < hi ? acc[e] : NEG_INF;
        mx = fmaxf(mx, s[t][e]);
      }
    }
  }
  __syncthreads();  // every wave has read K
  // V^T into the same buffer: chunk S of the 64 x LVC chunks is row S / LVC, keys
  // cstart + 8 (S % LVC) .. + 7. Chunks from kb1 on load the chunk holding key kb1 - 1 instead:
  // finite values that meet weights of 0. The chunk holding kb1 - 1 may read up to 7 keys past
  // kb1, which are the next sequence's or the zeros every v writer leaves up to the next
  // multiple of 8 tokens.
  {
    const int last = cstart + (((kb1 - 1) - cstart) & ~7);
    for (int i = wave; i < LVC; i += 4) {
      const int S = i * 64 + lane;
      const int dim = S / LVC, c = S - dim * LVC;
      const int key = min(cstart + 8 * c, last);
      __builtin_amdgcn_global_load_lds(Vt + size_t(dim) * a.ldv + key, reinterpret_cast<char*>(sVt) + i * 1024, 16, 0,
                                       0);
    }
  }
  // The softmax weights while V^T lands. Every real query sees itself, so the row maximum is
  // finite.
  const float sl2 = a.scale * 1.4426950408889634f;
  const float ms = wact ? half_max(mx) * sl2 : 0.0f;
  float psum = 0.0f;
  v8 pf[LTILES][2];
#pragma unroll
  for (int t = 0; t < LTILES; ++t) {
    if (t >= nt) continue;
#pragma unroll
    for (int sb = 0; sb < 2; ++sb)
#pragma unroll
      for (int j = 0; j < 8; ++j) {
        const float p = __builtin_amdgcn_exp2f(fmaf(s[t][sb * 8 + j], sl2, -ms));
        psum += p;
        pf[t][sb][j] = typename E::scalar(p);
      }
  }
  asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
  __syncthreads();
  if (!wact) return;  // no barrier follows
  f32x16 o[2];
#pragma unroll
  for (int e = 0; e < 16; ++e) { o[0][e] = 0.0f; o[1][e] = 0.0f; }
#pragma unroll
  for (int t = 0; t < LTILES; ++t) {
    if (t >= nt) continue;
#pragma unroll
    for (int sb = 0; sb < 2; ++sb) {
      const int kbase = t0 + t * 32 + sb * 16 + hl * 4;
#pragma unroll
      for (int dt = 0; dt < 2; ++dt) {
        const uint16_t* vr = &sVt[(dt * 32 + col) * LVW];
        const uint2 lo = *reinterpret_cast<const uint2*>(vr + kbase);
        const uint2 hi = *reinterpret_cast<const uint2*>(vr + kbase + 8);
        const uint4 pk = make_uint4(lo.x, lo.y, hi.x, hi.y);
        const v8 vf = *reinterpret_cast<const v8*>(&pk);
        o[dt] = E::mfma(vf, pf[t][sb], o[dt]);
      }
    }
  }
  const float lt = half_sum(psum);
  if (!qvalid) return;
  const float inv = 1.0f / lt;
  uint16_t* orow = a.out + size_t(qi) * a.ldo + head * 64;
#pragma unroll
  for (int dt = 0; dt < 2; ++dt)
#pragma unroll
    for (int g = 0; g < 4; ++g) {
      const int dim = dt * 32 + g * 8 + hl * 4;
      uint2 w;
      w.x = E::pack2(o[dt][g * 4 + 0] * inv, o[dt][g * 4 + 1] * inv);
      w.y = E::pack2(o[dt][g * 4 + 2] * inv, o[dt][g * 4 + 3] * inv);
      *reinterpret_cast<uint2*>(orow + dim) = w;
    }
}


// Global attention for a short batch (one request): a workgroup of KW waves takes 32 queries of
// one row and head, and wave w visits the row's key chunks w, w + KW, ... with softmax statistics
// of its own; the KW partial results merge through LDS at the end (the online-softmax
// combination). A short row then runs KW times as many waves, each with 1/KW of the chain of
// dependent chunks. Each wave stages its own chunks in a private 16 KiB of LDS (K rows and V^T
// in the layouts attn_kernel uses), so the chunk loop has no barriers; the next chunk is loaded
// into registers during this one's math and stored after it (a wave's LDS accesses run in
// order), which keeps 4 waves at 64 KiB (two workgroups per CU) and 8 at 128 KiB.
// LOCAL: a local layer's short batch; the tile's keys are its window range, and every key
// outside a query's own window (|key - query| > a.window) is masked.
template <class E, int KW, bool LOCAL>
__global__ __launch_bounds__(KW * 64) __attribute__((amdgpu_waves_per_eu(2))) void attn_ksplit_kernel(AttnArgs a) {
  typedef typename E::v8 v8;
  constexpr int REG = KC * 64;  // 16-bit elements of one 8 KiB K or V^T chunk
  // [wave] x (K | V^T); after the chunk loop the same memory holds the merge tables.
  __shared__ __attribute__((aligned(1024))) uint16_t smem[KW * 2 * REG];

  const int2 th = tile_head(a.ntiles);
  const AttnTile tl = a.tiles[th.x];
  const int head = th.y;
  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int hl = lane >> 5, col = lane & 31;
  const uint16_t* __restrict__ Qh = a.q + size_t(head) * a.Tq * 64;
  const uint16_t* __restrict__ Kh = a.k + size_t(head) * a.Tk * 64;
  const uint16_t* __restrict__ Vt = a.v + size_t(head) * 64 * a.ldv;
  uint16_t* const sK = smem + wave * 2 * REG;
  uint16_t* const sVt = sK + REG;

  const int qi = tl.q0 + col;
  const bool qvalid = qi < tl.q1;
  const int qld = min(qi, tl.q1 - 1);
  const int qk = a.qkey ? a.qkey[qld] : qld;  // q row of this slot
  const int kb0 = tl.k0, kb1 = tl.k1;
  const int cstart = kb0 & ~7;
  const int vlast = cstart + (((kb1 - 1) - cstart) & ~7);
  v8 qf[4];
#pragma unroll
  for (int kb = 0; kb < 4; ++kb)
    qf[kb] = *reinterpret_cast<const v8*>(Qh + size_t(qk) * 64 + kb * 16 + hl * 8);

  // A chunk in registers: 16-byte piece p = lane + 64 it is K row p / 8, slot p % 8 (rows past
  // kb1 repeat the last key), and V^T dim p / 8, keys 8 (p % 8) .. + 7 (from kb1 on, the piece
  // holding key kb1 - 1; it may read up to 7 keys past kb1, the next sequence's or the zeros
  // every v writer leaves up to the next multiple of 8 tokens).
  uint4 kreg[8], vreg[8];
  auto load = [&](int c0) {
#pragma unroll
    for (int it = 0; it < 8; ++it) {
      const int p = lane + it * 64;
      const int r = p >> 3, c = p & 7;
      kreg[it] = *reinterpret_cast<const uint4*>(Kh + size_t(min(c0 + r, kb1 - 1)) * 64 + c * 8);
      vreg[it] = *reinterpret_cast<const uint4*>(Vt + size_t(r) * a.ldv + min(c0 + c * 8, vlast));
    }
  };
  auto store = [&] {  // K rows by kslot; V^T in the PV operand order of attn_kernel
#pragma unroll
    for (int it = 0; it < 8; ++it) {
      const int p = lane + it * 64;
      const int r = p >> 3, c = p & 7;
      const uint4 kv = kreg[it];
      *reinterpret_cast<uint4*>(sK + r * 64 + kslot(r, c) * 8) = make_uint4(kv.x, kv.y, kv.z, kv.w);
      uint16_t* row = sVt + r * 64 + (c & 1) * 4;
      *reinterpret_cast<uint2*>(row + kslot(r, c & ~1) * 8) = make_uint2(vreg[it].x, vreg[it].y);
      *reinterpret_cast<uint2*>(row + kslot(r, c | 1) * 8) = make_uint2(vreg[it].z, vreg[it].w);
    }
  };

  const float sl2 = a.scale * 1.4426950408889634f;
  float m = NEG_INF, l = 0.0f;
  f32x16 o[2];
#pragma unroll
  for (int e = 0; e < 16; ++e) { o[0][e] = 0.0f; o[1][e] = 0.0f; }

  int c0 = cstart + wave * KC;
  if (c0 < kb1) {
    load(c0);
    store();
  }
  for (; c0 < kb1; c0 += KW * KC) {
    const bool more = c0 + KW * KC < kb1;
    if (more) load(c0 + KW * KC);
    f32x16 s[2];
    float mx = NEG_INF;
    // As in attn_kernel: the chunk's K fragments first, the two tiles' k-steps interleaved, and
    // one-sided masks on chunks that cross the key range.
    v8 kf[2][4];
#pragma unroll
    for (int kb = 0; kb < 4; ++kb)
#pragma unroll
      for (int t = 0; t < 2; ++t) {
        const int kr = t * 32 + col;
        kf[t][kb] = *reinterpret_cast<const v8*>(sK + kr * 64 + kslot(kr, kb * 2 + hl) * 8);
      }
#pragma unroll
    for (int t = 0; t < 2; ++t)
#pragma unroll
      for (int e = 0; e < 16; ++e) s[t][e] = 0.0f;
#pragma unroll
    for (int kb = 0; kb < 4; ++kb)
#pragma unroll
      for (int t = 0; t < 2; ++t) s[t] = E::mfma(kf[t][kb], qf[kb], s[t]);
#pragma unroll
    for (int t = 0; t < 2; ++t) {
      const int kbase = c0 + t * 32 + hl * 4;
      if constexpr (LOCAL) {
        // A 32-query tile's window range is at most 160 keys: every chunk crosses some edge.
        const int lo = max(kb0, qk - a.window) - kbase, hi = min(kb1, qk + a.window + 1) - kbase;
#pragma unroll
        for (int e = 0; e < 16; ++e) {
          const int kk = (e >> 2) * 8 + (e & 3);
          s[t][e] = kk >= lo && kk < hi ? s[t][e] : NEG_INF;
        }
      } else {
      if (c0 < kb0) {
        const int lo = kb0 - kbase;
#pragma unroll
        for (int e = 0; e < 16; ++e) s[t][e] = (e >> 2) * 8 + (e & 3) >= lo ? s[t][e] : NEG_INF;
      }
      if (c0 + KC > kb1) {
        const int hi = kb1 - kbase;
#pragma unroll
        for (int e = 0; e < 16; ++e) s[t][e] = (e >> 2) * 8 + (e & 3) < hi ? s[t][e] : NEG_INF;
      }
      }
#pragma unroll
      for (int e = 0; e < 16; ++e) mx = fmaxf(mx, s[t][e]);
    }
    mx = half_max(mx);
    const float mn = fmaxf(m, mx * sl2);
    const float ms = mn == NEG_INF ? 0.0f : mn;
    const float alpha = __builtin_amdgcn_exp2f(m - ms);
    float psum = 0.0f;
    v8 pf[2][2];
#pragma unroll
    for (int t = 0; t < 2; ++t)
#pragma unroll
      for (int sb = 0; sb < 2; ++sb)
#pragma unroll
        for (int j = 0; j < 8; ++j) {
          const float p = __builtin_amdgcn_exp2f(fmaf(s[t][sb * 8 + j], sl2, -ms));
          psum += p;
          pf[t][sb][j] = typename E::scalar(p);
        }
    l = l * alpha + psum;
    m = mn;
    if (alpha != 1.0f) {
#pragma unroll
      for (int e = 0; e < 16; ++e) { o[0][e] *= alpha; o[1][e] *= alpha; }
    }
#pragma unroll
    for (int t = 0; t < 2; ++t)
#pragma unroll
      for (int sb = 0; sb < 2; ++sb)
#pragma unroll
        for (int dt = 0; dt < 2; ++dt) {
          const int dr = dt * 32 + col;
          const v8 vf = *reinterpret_cast<const v8*>(sVt + dr * 64 + kslot(dr, (t * 2 + sb) * 2 + hl) * 8);
          o[dt] = E::mfma(vf, pf[t][sb], o[dt]);
        }
    if (more) store();  // after this chunk's reads
  }

  // Merge: wave w leaves (m, l, o) per lane in LDS; wave 0 combines them. A wave that visited no
  // chunk has m = -inf and contributes 0.
  const float lw = half_sum(l);
  __syncthreads();  // every wave is done with its chunk buffers
  float* mt = reinterpret_cast<float*>(smem);  // [KW][64] m, [KW][64] l, [KW][32][64] o
  float* lt = mt + KW * 64;
  float* ot = lt + KW * 64;
  mt[wave * 64 + lane] = m;
  lt[wave * 64 + lane] = lw;
#pragma unroll
  for (int e = 0; e < 32; ++e) ot[(wave * 32 + e) * 64 + lane] = o[e >> 4][e & 15];
  __syncthreads();
  if (wave != 0 || !qvalid) return;
  float M = NEG_INF;
#pragma unroll
  for (int w = 0; w < KW; ++w) M = fmaxf(M, mt[w * 64 + lane]);
  float f[KW], L = 0.0f;
#pragma unroll
  for (int w = 0; w < KW; ++w) {
    const float mw = mt[w * 64 + lane];
    f[w] = mw == NEG_INF ? 0.0f : __builtin_amdgcn_exp2f(mw - M);
    L += lt[w * 64 + lane] * f[w];
  }
  const float inv = 1.0f / L;
  uint16_t* orow = a.out + size_t(qi) * a.ldo + head * 64;
#pragma unroll
  for (int dt = 0; dt < 2; ++dt)
#pragma unroll
    for (int g = 0; g < 4; ++g) {
      float v[4];
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        const int e = dt * 16 + g * 4 + r;
        float acc = 0.0f;
#pragma unroll
        for (int w = 0; w < KW; ++w) acc += ot[(w * 32 + e) * 64 + lane] * f[w];
        v[r] = acc * inv;
      }
      const int dim = dt * 32 + g * 8 + hl * 4;
      *reinterpret_cast<uint2*>(orow + dim) = make_uint2(E::pack2(v[0], v[1]), E::pack2(v[2], v[3]));
    }
}

// Attention of the padded layout's padding queries that the local-attention tiles do not take:
// those whose softmax the reference's masks leave over a key set other than the real keys of
// the window. Each entry names the set, as the host works it out from the masks
// (lib.rs:1241-1310): {query, a0, a1, b0, b1, lo, hi, zeros} = keys [a0, a1) and [b0, b1) (packed
// indices), key a0 counted 1 + lo times, the last key of the last non-empty range 1 + hi times
// (gathered slots clamped to one key), and `zeros` slots of zero key and value (score 0, value
// 0). One wave per (entry, head), 64 keys a step: lane j scores key j of the step in f32, lane d
// accumulates output dim d.
template <class E>
__global__ __launch_bounds__(64) void attn_fallback_kernel(FallbackArgs a) {
  __shared__ float sp[64];
  const int fi = blockIdx.x / a.heads, head = blockIdx.x % a.heads;
  const int4 f0 = reinterpret_cast<const int4*>(a.far)[2 * fi];      // query, a0, a1, b0
  const int4 f1 = reinterpret_cast<const int4*>(a.far)[2 * fi + 1];  // b1, lo, hi, zeros
  const int lane = threadIdx.x;
  const uint16_t* __restrict__ Qh = a.q + size_t(head) * a.T * 64;
  const uint16_t* __restrict__ Kh = a.k + size_t(head) * a.T * 64;
  const uint16_t* __restrict__ Vt = a.v + size_t(head) * 64 * a.ldv;
  float qv[64];
#pragma unroll
  for (int c = 0; c < 8; ++c) unpack8<E>(*reinterpret_cast<const uint4*>(Qh + size_t(f0.x) * 64 + c * 8), qv + c * 8);
  const float sl2 = a.scale * 1.4426950408889634f;
  // Repeated keys: the weight of n copies is exp2(s + log2 n).
  const int klo = f0.y, khi = (f1.x > f0.w ? f1.x : f0.z) - 1;
  const float llo = log2f(float(1 + f1.y)), lhi = log2f(float(1 + f1.z));
  float m = NEG_INF, l = 0.0f, o = 0.0f;
  auto keys = [&](int j0, int j1) {
    for (int b = j0; b < j1; b += 64) {
      const int j = b + lane;
      float s = NEG_INF;
      if (j < j1) {
        float kv[8], dot = 0.0f;
#pragma unroll
        for (int c = 0; c < 8; ++c) {
          unpack8<E>(*reinterpret_cast<const uint4*>(Kh + size_t(j) * 64 + c * 8), kv);
#pragma unroll
          for (int e = 0; e < 8; ++e) dot = fmaf(qv[c * 8 + e], kv[e], dot);
        }
        s = dot * sl2 + (j == klo ? llo : 0.0f) + (j == khi ? lhi : 0.0f);
      }
      const float mn = fmaxf(m, wave_max(s));
      const float p = j < j1 ? __builtin_amdgcn_exp2f(s - mn) : 0.0f;
      const float alpha = m == NEG_INF ? 0.0f : __builtin_amdgcn_exp2f(m - mn);
      l = l * alpha + wave_sum(p);
      o *= alpha;
      m = mn;
      sp[lane] = p;
      __syncthreads();
      const uint16_t* vr = Vt + size_t(lane) * a.ldv + b;  // dim `lane`, keys b ..
      const int cnt = min(64, j1 - b);
      for (int t = 0; t < cnt; ++t) o = fmaf(sp[t], E::f32(vr[t]), o);
      __syncthreads();
    }
  };
  keys(f0.y, f0.z);
  keys(f0.w, f1.x);
  if (f1.w > 0) {  // zero slots: score 0, value 0, weight `zeros`
    const float sz = log2f(float(f1.w));
    const float mn = fmaxf(m, sz);
    const float alpha = m == NEG_INF ? 0.0f : __builtin_amdgcn_exp2f(m - mn);
    l = l * alpha + __builtin_amdgcn_exp2f(sz - mn);
    o *= alpha;
  }
  a.out[size_t(f0.x) * a.ldo + head * 64 + lane] = E::bits(o / l);
}

}  // namespace

// Query count of row r: up to q_end[r] when given, else the whole row.
static int row_queries(const int* row_start, const int* q_end, int r) {
  return (q_end ? q_end[r] : row_start[r + 1]) - row_start[r];
}

// Local layers: 128-query tiles (attn_local_kernel) while they give at least one workgroup per
// CU; a shorter batch takes 32-query tiles whose keys are the tile's window range, split over 4
// waves (attn_ksplit_kernel<LOCAL>). Windows wider than attn_local_kernel stages keep 128.
static int local_tile(const int* row_start, const int* q_end, int n, int heads, int window) {
  if (window > LMAXW) return LQ;
  long long c = 0;
  for (int r = 0; r < n; ++r) c += (row_queries(row_start, q_end, r) + LQ - 1) / LQ;
  return c * heads >= 256 ? LQ : 32;
}
int attn_local_tile(const int* row_start, int n, int heads, int window) {
  return local_tile(row_start, nullptr, n, heads, window);
}

int attn_row_step(int len, int qb) {
  if (qb <= 32) return qb;
  const int nt = (len + qb - 1) / qb;
  return std::min(qb, ((len + nt - 1) / nt + 31) / 32 * 32);
}

// 256-query tiles (8 waves, every K/V chunk shared by 256 queries) while they give at least one
// workgroup per CU; then 128 (4 waves) while they give 128 workgroups; a shorter batch takes
// 32-query tiles whose keys are split over 4 waves (attn_ksplit_kernel).
static int global_tile(const int* row_start, const int* q_end, int n, int heads) {
  auto count = [&](int qb) {
    long long c = 0;
    for (int r = 0; r < n; ++r) c += (row_queries(row_start, q_end, r) + qb - 1) / qb;
    return c * heads;
  };
  if (count(256) >= 256) return 256;
  if (count(128) >= 128) return 128;
  return 32;  // attn_ksplit_kernel
}
int attn_global_tile(const int* row_start, int n, int heads) { return global_tile(row_start, nullptr, n, heads); }

int attn_plan_tiles(const int* row_start, int n, int heads, int window, std::vector<int>& out, const int* q_end,
                    const int* k_end) {
  const int qb = window >= 0 ? local_tile(row_start, q_end, n, heads, window) : global_tile(row_start, q_end, n, heads);
  for (int r = 0; r < n; ++r) {
    const int rs = row_start[r], qe = q_end ? q_end[r] : row_start[r + 1], ke = k_end ? k_end[r] : row_start[r + 1];
    const int step = attn_row_step(qe - rs, qb);
    for (int q0 = rs; q0 < qe; q0 += step) {
      const int q1 = std::min(q0 + step, qe);
      const bool win = window >= 0 && qb == 32;
      out.push_back(q0);
      out.push_back(q1);
      out.push_back(win ? std::max(rs, q0 - window) : rs);
      out.push_back(win ? std::min(ke, q1 + window) : ke);
    }
  }
  return qb;
}

template <class E>
void attn_launch_t(const AttnArgs& a, hipStream_t st) {
  const dim3 grid(a.ntiles * a.heads);
  if (a.window >= 0 && a.window <= LMAXW && !a.qkey && a.tile_q == 32)
    hipLaunchKernelGGL((attn_ksplit_kernel<E, 4, true>), grid, dim3(256), 0, st, a);
  else if (a.window >= 0 && a.window <= LMAXW && !a.qkey)
    hipLaunchKernelGGL(attn_local_kernel<E>, grid, dim3(256), 0, st, a);  // tiles of <= LQ queries
  else if (a.window >= 0)
    hipLaunchKernelGGL((attn_kernel<E, true, 4>), grid, dim3(256), 0, st, a);
  else if (a.tile_q == 256)
    hipLaunchKernelGGL((attn_kernel<E, false, 8>), grid, dim3(512), 0, st, a);
  else if (a.tile_q == 128)
    hipLaunchKernelGGL((attn_kernel<E, false, 4>), grid, dim3(256), 0, st, a);
  else if (a.key_waves == 8)  // tile_q 32
    hipLaunchKernelGGL((attn_ksplit_kernel<E, 8, false>), grid, dim3(512), 0, st, a);
  else
    hipLaunchKernelGGL((attn_ksplit_kernel<E, 4, false>), grid, dim3(256), 0, st, a);
}

void attn_launch(const AttnArgs& a, hipStream_t st) {
  if (a.ntiles <= 0) return;
  if (a.elem == ELEM_F16) attn_launch_t<F16>(a, st);
  else attn_launch_t<Bf16>(a, st);
}

void attn_fallback_launch(const FallbackArgs& a, hipStream_t st) {
  if (a.nfar <= 0) return;
  const dim3 grid(unsigned(a.nfar) * unsigned(a.heads));
  if (a.elem == ELEM_F16) hipLaunchKernelGGL(attn_fallback_kernel<F16>, grid, dim3(64), 0, st, a);
  else hipLaunchKernelGGL(attn_fallback_kernel<Bf16>, grid, dim3(64), 0, st, a);
}

}  // namespace s1
