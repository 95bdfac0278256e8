// Host-side launch interface of the HIP kernels. Every pointer is a device pointer; bf16 data is
// passed as uint16_t. Launchers enqueue on the given stream and never synchronise.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include <vector>

namespace s1 {

// The 16-bit type of weights and activations (every "bf16" buffer below holds this type): bf16
// by default, f16 with the model setting dtype=f16.
enum Elem { ELEM_BF16 = 0, ELEM_F16 = 1 };

enum GemmEpi { EPI_BF16 = 0, EPI_RESID = 1, EPI_GEGLU = 2, EPI_F32 = 3, EPI_ROPE = 4 };
enum Act { ACT_NONE = 0, ACT_RELU = 1, ACT_GELU = 2 };

struct GemmArgs {
  const uint16_t* A = nullptr;  // [M, lda] bf16
  const uint16_t* W = nullptr;  // [N, ldw] bf16 (row n = output column n)
  void* C = nullptr;            // bf16 or f32 by epilogue
  const float* bias = nullptr;  // [N] or null
  int M = 0, N = 0, K = 0;
  int lda = 0, ldw = 0, ldc = 0;
  int epi = EPI_BF16;
  int act = ACT_NONE;
  int elem = ELEM_BF16;
  // Split-K: `splits` workgroups share each output tile, each over a contiguous k-range, and
  // write f32 partials [splits, M, N] to `ws`; a second kernel sums them in split order and runs
  // the epilogue. splits = 1 runs the epilogue in the GEMM and needs no workspace.
  int splits = 1;
  float* ws = nullptr;
  // EPI_ROPE only
  uint16_t* rope_q = nullptr;  // [H, rope_T, 64]
  uint16_t* rope_k = nullptr;
  uint16_t* rope_v = nullptr;  // transposed: [H, 64, rope_ldv]
  int rope_ldv = 0;
  const int* rope_pos = nullptr;   // [M] position of each row in its sequence
  const float* rope_cos = nullptr;  // [max_pos, 32]
  const float* rope_sin = nullptr;
  int rope_T = 0;
  int rope_d = 0;
};

// Null when the shape is supported, else a message.
const char* gemm_check(const GemmArgs& g);
void gemm_launch(const GemmArgs& g, hipStream_t st);
// The first half of a split-K gemm_launch (g.splits > 1): the f32 partials into g.ws, no
// epilogue. splitk_resid_ln_launch finishes a residual GEMM launched this way.
void gemm_launch_partials(const GemmArgs& g, hipStream_t st);

// The split-K factor gemm_launch should use for M x N x K (1: none), and the workspace it needs
// in f32 elements. reduce_folded: the caller finishes a split in a kernel it runs anyway
// (splitk_resid_ln_launch), so splitting pays at more tile counts. A folded plan splits wherever
// an unfolded one does, with the same factor.
struct GemmPlan {
  int splits;
  size_t ws_floats;
};
GemmPlan gemm_plan(int M, int N, int K, bool reduce_folded = false);

// The row stride of a transposed v buffer for T tokens: T rounded up to 8 (16-byte rows) plus
// 64 columns of slack, so a 64-key chunk read never leaves the row. Every writer of v stores
// zeros in columns [T, T rounded up to 8); the rest of the slack is never written.
inline int vt_ld(int T) { return (T + 7) / 8 * 8 + 64; }

// Attention over packed variable-length rows. q, k are [H, Tq or Tk, 64] bf16 (head-major) and v
// is transposed, [H, 64, ldv] (vt_ld(Tk)).
// Queries are numbered by output slot; each work tile is up to tile_q consecutive slots of one
// sequence: {q0, q1, k0, k1} = slots [q0, q1) and the sequence's key range [k0, k1). Slot s reads
// q row qkey[s] (or s when qkey is null), writes out row s, and sits at key index qkey[s] for
// the window test. The decision head's pruned last layer uses qkey to attend from a few picked
// tokens only; the encoder passes null.
struct AttnTile {
  int q0, q1, k0, k1;
};
struct AttnArgs {
  const uint16_t* q = nullptr;
  const uint16_t* k = nullptr;
  const uint16_t* v = nullptr;
  uint16_t* out = nullptr;  // [slots, ldo] bf16, head h at columns h*64 .. h*64+63
  const AttnTile* tiles = nullptr;
  const int* qkey = nullptr;  // [slots] q row / key index of each slot, or null for identity
  int ntiles = 0;
  int heads = 0;
  int Tq = 0, Tk = 0;  // rows of the q buffer and of the k buffer (head strides)
  int ldv = 0;         // row stride of the transposed v
  int ldo = 0;
  float scale = 0.125f;
  int window = -1;  // < 0: global attention; else keys with |i - j| <= window
  // Queries per tile. Global attention: 256 or 128 (8 or 4 waves, each with 32 queries and every
  // key), or 32: then key_waves (4 or 8) waves split each tile's keys. Local (window <= 64): 128,
  // or 32, whose keys (the tile's window range) 4 waves split.
  int tile_q = 256;
  int key_waves = 4;
  int elem = ELEM_BF16;
};
void attn_launch(const AttnArgs& a, hipStream_t st);
// Queries per work tile the attention kernel takes, given the rows' lengths: on global layers 256
// or 128 when that still gives the GPU enough workgroups, else 32; on local layers 128, or 32 for
// a short batch.
int attn_global_tile(const int* row_start, int n, int heads);
int attn_local_tile(const int* row_start, int n, int heads, int window);
// Appends the work tiles {q0, q1, k0, k1} of the rows (window < 0: a global layer) to out and
// returns the queries per tile, the AttnArgs::tile_q to launch them with. Keys [k0, k1) are the
// row's, or for 32-query local tiles the tile's window range within the row. With q_end / k_end
// (per row), row r's queries stop at q_end[r] and its keys at k_end[r] instead of at the row's
// end (the padded layout: every position a query, only the real tokens keys).
int attn_plan_tiles(const int* row_start, int n, int heads, int window, std::vector<int>& out,
                    const int* q_end = nullptr, const int* k_end = nullptr);

// Attention of single queries over a key set given per query: the padded layout's padding
// queries on local layers whose keys under the reference's masks are not the real keys of their
// window. far: nfar entries of 8 int32 (device, 16-byte aligned) {query, a0, a1, b0, b1, lo, hi,
// zeros}: keys [a0, a1) and [b0, b1), key a0 counted 1 + lo times, the last key of the last
// non-empty range 1 + hi times, plus `zeros` slots of zero key and value. Every entry has a key.
struct FallbackArgs {
  const uint16_t* q = nullptr;
  const uint16_t* k = nullptr;
  const uint16_t* v = nullptr;  // transposed, [H, 64, ldv]
  uint16_t* out = nullptr;      // [T, ldo]
  const int* far = nullptr;
  int nfar = 0, heads = 0, T = 0, ldv = 0, ldo = 0;
  float scale = 0.125f;
  int elem = ELEM_BF16;
};
void attn_fallback_launch(const FallbackArgs& a, hipStream_t st);
// The query step that cuts a row of len tokens into tiles of at most qb queries: as many tiles
// as qb needs, of even sizes rounded up to whole waves (570 tokens at 256: 192, 192, 186), so a
// row's last tile is not a nearly idle workgroup beside full ones.
int attn_row_step(int len, int qb);

// h[t] = LN(tok_emb[ids[t]]) (no bias), written as f32 and as bf16.
void embed_ln_launch(const uint16_t* tok_emb, const int* ids, const float* w, float eps, int T, int d, float* h_out,
                     uint16_t* x_out, hipStream_t st, int elem = ELEM_BF16);

// y = LN(x) (optional bias) over rows of d, x f32; y bf16 and/or f32 (null to skip). With
// `rows` the input row of output row t is rows[t]. With `add_rowvec`, the f32 output also gets
// add_rowvec[seg[t]] (the type embedding of the row's question), used to start the head stream.
void layernorm_launch(const float* x, const int* rows, const float* w, const float* b, float eps, int T, int d,
                      uint16_t* y_bf16, float* y_f32, const float* add_rowvec, const int* seg, float* y_plus,
                      hipStream_t st, int elem = ELEM_BF16);

// The end of a split-K residual GEMM and the LayerNorm after it, one wave per row:
// h[t] += (sum over s of ws[s, t] in split order) + bias, then y[t] = LN(h[t]) (weight w, bias
// lnb or none) in bf16. Bit for bit the GEMM's own split-K epilogue followed by layernorm_launch.
// ws is [splits, T, d] f32, h is [T, d] f32.
// With hsrc, the residual of row r is row hrows[r] of hsrc (a row gather folded in); the sum
// still goes to row r of h.
void splitk_resid_ln_launch(const float* ws, int splits, const float* bias, float* h, const float* w, float eps, int T,
                            int d, uint16_t* y, hipStream_t st, int elem = ELEM_BF16, const float* lnb = nullptr,
                            const float* hsrc = nullptr, const int* hrows = nullptr);

// End of the pruned decision head over its P = n per picked rows ([row 0, kmax scorer rows] per
// request, per = 1 + kmax): h (+ the sum of `splits` f32 partials in ws [splits, P, d] and then
// bias, when splits > 1) -> row 0 of request i to pooled[i] (f32), scorer row k of request i to
// y[i kmax + k] = LayerNorm(weight w, bias b, eps) in 16 bits. Bit for bit the split-K epilogue,
// layernorm_launch over the scorer rows and gather_f32_launch of the pooled rows. h is only read.
void head_end_launch(const float* ws, int splits, const float* bias, const float* h, int per, const float* w,
                     const float* b, float eps, float* pooled, uint16_t* y, int P, int d, hipStream_t st,
                     int elem = ELEM_BF16);

// End of the encoder and start of the decision head in one pass over the T rows: h (+ the sum of
// `splits` f32 partials in ws [splits, T, d] when splits > 1, as splitk_resid_ln_launch adds
// them, with no bias) -> LayerNorm (weight wf, no bias) + addv[seg[row]] -> hh (f32), then, when
// x is given, LayerNorm(hh) (weight w1, bias b1, eps1) -> x (16-bit). Bit for bit the split-K
// epilogue, layernorm_launch with add_rowvec, and layernorm_launch again. h is only read.
void encoder_end_launch(const float* ws, int splits, const float* h, const float* wf, float eps, const float* addv,
                        const int* seg, float* hh, const float* w1, const float* b1, float eps1, uint16_t* x, int T,
                        int d, hipStream_t st, int elem = ELEM_BF16);

// Plain split (+ RoPE when cos/sin are given): qkv [T, 3d] bf16 -> q, k [H, T, 64] and v
// transposed [H, 64, ldv] (ldv >= T), bf16.
void split_rope_launch(const uint16_t* qkv, int T, int d, const int* pos, const float* cos_t, const float* sin_t,
                       uint16_t* q, uint16_t* k, uint16_t* v, int ldv, hipStream_t st, int elem = ELEM_BF16);

// act[t, i] = gelu(wi[t, i]) * wi[t, I + i] for the un-interleaved Wi product.
void geglu_launch(const uint16_t* wi, int T, int I, uint16_t* act, hipStream_t st, int elem = ELEM_BF16);

// Gather rows: out[r] = x[rows[r]] for f32 rows of d.
void gather_f32_launch(const float* x, const int* rows, int R, int d, float* out, hipStream_t st);

// logits[r] = dot(x[r], w) + b, x bf16 [R, d], w f32 [d].
void rowdot_launch(const uint16_t* x, const float* w, const float* b, int R, int d, float* out, hipStream_t st,
                   int elem = ELEM_BF16);

// ---- The dtype=f32 path (BackendOptions::f32): f32 weights and activations, plain kernels.

// C[M, N] (+)= act(A[M, K] . W[N, K]^T + bias), all f32; accumulate adds to C (the residual).
struct Gemm32Args {
  const float* A = nullptr;  // [M, lda]
  const float* W = nullptr;  // [N, ldw]
  float* C = nullptr;        // [M, ldc]
  const float* bias = nullptr;
  int M = 0, N = 0, K = 0, lda = 0, ldw = 0, ldc = 0;
  int act = ACT_NONE;
  bool accumulate = false;
};
// Null when the shape is supported (K a multiple of 16, 16-byte aligned rows), else a message.
const char* gemm32_check(const Gemm32Args& g);
void gemm32_launch(const Gemm32Args& g, hipStream_t st);
// qkv [T, 3d] -> q, k, v [d / 64, T, 64] f32, q and k rotated at pos[t] when cos_t is given.
void split32_launch(const float* qkv, int T, int d, const int* pos, const float* cos_t, const float* sin_t, float* q,
                    float* k, float* v, hipStream_t st);
// Attention of n single queries, each over its key set: entries of 8 int32 as attn_fallback_launch
// takes them ({query, a0, a1, b0, b1, lo, hi, zeros}); q, k, v [heads, T, 64] f32, out [T, ldo].
struct Attn32Args {
  const float* q = nullptr;
  const float* k = nullptr;
  const float* v = nullptr;
  float* out = nullptr;
  const int* entries = nullptr;
  int n = 0, heads = 0, T = 0, ldo = 0;
  float scale = 0.125f;
};
void attn32_launch(const Attn32Args& a, hipStream_t st);
// act[t, i] = gelu(x[t, i]) * x[t, I + i] (exact erf) over x [T, 2I] f32.
void geglu32_launch(const float* x, int T, int I, float* act, hipStream_t st);

}  // namespace s1
