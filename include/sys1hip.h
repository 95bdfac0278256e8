/*
 * libsys1hip: the MI355X (gfx950) backend of sys1rust's decision model, as a plain C ABI.
 *
 * The entry points replace laya_mlx's MlxBackend behind laya_core's `Backend` trait
 * (runtime/crates/laya-core/src/backend.rs:109-133) and its factory `make_backend`
 * (runtime/crates/laya-mlx/src/lib.rs:593-599, BackendFactory in
 * runtime/crates/laya-core/src/agent.rs:28-30). A Rust crate binds them one to one.
 *
 * Conventions:
 *  - Return value 0 is success; otherwise an S1_ERR_* kind, with the message in s1_last_error()
 *    (thread-local, valid until the next failing call on that thread).
 *  - No call aborts the process. A model whose weights or config do not fit is refused at create.
 *  - Calls on one model must be serialised by the caller (the Rust side calls from one inference
 *    thread); different models may be used from different threads.
 *  - Input and output buffers are caller-owned host memory. Batch arrays are row-major, exactly
 *    laya_core::Batch (backend.rs:72-98): `input_ids`, `attention_mask` [n*len];
 *    `seq_lens`, `marker_count`, `qtype` [n]; `marker_pos` [n*kmax].
 */
#ifndef SYS1HIP_H
#define SYS1HIP_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define S1_OK 0
#define S1_ERR_CONFIG 1  /* laya_core::Error::Config  */
#define S1_ERR_WEIGHTS 2 /* laya_core::Error::Weights */
#define S1_ERR_BACKEND 3 /* laya_core::Error::Backend */
#define S1_ERR_BATCH 4   /* malformed batch (a Backend error on the Rust side) */

typedef struct s1_model s1_model;

/* Load a checkpoint onto GPU `device_ordinal` (MlxBackend::new, lib.rs:960-1150).
 * `encoder_config_json`: encoder/config.json text (EncoderConfig::from_value, config.rs:96-159).
 * `agent_config_json`: rl_agent_config.json text or NULL (AgentConfig, config.rs:9-40).
 * `settings`: strict comma list like BackendOptions::tuning (backend.rs:22-32); an unknown key is
 * S1_ERR_CONFIG (Knobs::parse, lib.rs:155-259). NULL or "" selects the defaults. `dtype=f16`
 * keeps weights and activations in f16, the checkpoints' own type (BackendOptions::f32 = false,
 * backend.rs:25-27, keeps the checkpoint's f16 weights); the default `dtype=bf16` rounds them to
 * bf16. Accumulation, LayerNorm, softmax and the residual stream are f32 either way. `dtype=f32`
 * is BackendOptions::f32 = true: f32 weights and compute on plain f32 kernels (no fused kernels,
 * a numerics mode, not the serving path). */
int s1_model_create(const char* safetensors_path, const char* encoder_config_json,
                    const char* agent_config_json, const char* settings, int device_ordinal,
                    s1_model** out);

/* Same, from a safetensors image in memory that the caller owns (an mmap, say); the bytes are
 * only read during the call (Weights::open, runtime/crates/laya-core/src/weights.rs:22-43). */
int s1_model_create_from_bytes(const void* safetensors_bytes, size_t nbytes,
                               const char* encoder_config_json, const char* agent_config_json,
                               const char* settings, int device_ordinal, s1_model** out);

/* Element types of s1_tensor (the safetensors dtypes the loader converts, weights.rs:82-115). */
#define S1_DTYPE_F32 0
#define S1_DTYPE_F16 1
#define S1_DTYPE_BF16 2
#define S1_DTYPE_F64 3

/* One checkpoint tensor as the caller's safetensors view yields it (safetensors::TensorView:
 * name, dtype, shape, data): row-major little-endian elements, nbytes = product(shape) * size. */
typedef struct s1_tensor {
  const char* name;
  int32_t dtype; /* S1_DTYPE_* */
  uint32_t ndim;
  const uint64_t* shape; /* [ndim] */
  const void* data;
  size_t nbytes;
} s1_tensor;

/* Same, from the tensors of a checkpoint the caller has already opened and located:
 * laya_core::Weights::view() (runtime/crates/laya-core/src/weights.rs:46-48) parses the mmapped
 * file into exactly these (name, dtype, shape, bytes) views, so the binding needs no access to
 * the mapping itself. The data is only read during the call; names must be unique. */
int s1_model_create_from_tensors(const s1_tensor* tensors, size_t count, const char* encoder_config_json,
                                 const char* agent_config_json, const char* settings, int device_ordinal,
                                 s1_model** out);

/* check_settings (runtime/crates/laya-mlx/src/lib.rs:264-266): check a settings string without
 * loading a model. S1_ERR_CONFIG names the first unknown setting or bad value, exactly as
 * s1_model_create would with it; 0 otherwise. Every key of laya-mlx's Knobs (lib.rs:196-256) is
 * accepted with its value checks, so sys1rust's DEFAULT_TUNING (sys1rust/src/config.rs:29) passes. */
int s1_check_settings(const char* settings);

/* Backend::forward (lib.rs:1833-1863): logits_out [n*kmax] (-1e4 where k >= marker_count[r]),
 * pooled_out [n*d] (head output at position 0 of each row), both f32. */
int s1_forward(s1_model* m, uint32_t n, uint32_t len, uint32_t kmax, const uint32_t* input_ids,
               const uint32_t* attention_mask, const uint64_t* seq_lens, const uint32_t* marker_pos,
               const uint64_t* marker_count, const uint32_t* qtype, float* logits_out,
               float* pooled_out);

/* Backend::encoder_hidden (lib.rs:1864-1878): the encoder's last_hidden_state as f32
 * [n*len*d], computed at every position including padding: the encoder runs the padded layout
 * (every position a row, RoPE position = index in the row), and a padding position attends as
 * the reference's masks let it, which the settings mask / windowed / dense_upto / band / fuserope
 * decide as they decide MlxBackend's path for this len (lib.rs:1241-1310). The batch checks are
 * s1_forward's; kmax, marker_pos, marker_count and qtype are not read; len must be at most
 * max_position_embeddings. */
int s1_encoder_hidden(s1_model* m, uint32_t n, uint32_t len, uint32_t kmax,
                      const uint32_t* input_ids, const uint32_t* attention_mask,
                      const uint64_t* seq_lens, const uint32_t* marker_pos,
                      const uint64_t* marker_count, const uint32_t* qtype, float* hidden_out);

/* Backend::padded_len (lib.rs:1826-1831): `len` rounded up to the first `buckets=` entry that
 * holds it, else to a multiple of `pad=`. */
size_t s1_padded_len(const s1_model* m, size_t len, size_t rows);

/* Backend::name (lib.rs:1804-1812), e.g. "hip(gfx950,bf16)" ("f16", "f32" by dtype). Owned by
 * the model. */
const char* s1_name(const s1_model* m);

/* Backend::active_kernels (lib.rs:1814-1824, contract backend.rs:111-116): comma list of the
 * custom kernels requested, built and checked at load (fuserope, fusegeglu, fuseln). A kernel
 * that failed its load check is not listed, and its unfused twin runs instead. */
const char* s1_active_kernels(const s1_model* m);

/* Backend::warmup (backend.rs:122-124): run one small forward so first-request costs are paid. */
int s1_warmup(s1_model* m);

/* Message of the last failing call on this thread ("" if none). */
const char* s1_last_error(void);

void s1_model_destroy(s1_model* m);

/* ---- Harness entry points (no counterpart in the reference) --------------------------------
 * A synthetic decision-model checkpoint with the reference's tensor names
 * (lib.rs:990-1131, decode.rs:130-136) and seeded N(0, 0.02) bf16 weights. Call with out=NULL
 * to get the size in *len, then with a buffer of that size. scorer_width is the width of
 * scorer.1, n_act the action count of act_head.2; jitter != 0 draws LayerNorm weights
 * 1 + N(0, 0.02) and biases N(0, 0.02) instead of 1 and 0. */
int s1_synth_checkpoint(const char* encoder_config_json, const char* agent_config_json,
                        uint64_t seed, int scorer_width, int n_act, int jitter, void* out,
                        size_t cap, size_t* len);

/* The packed token layout the forward runs in (Packing::new and MlxBackend::scorer_rows,
 * runtime/crates/laya-mlx/src/lib.rs:894-943, 1502-1521), with the batch checks of s1_forward.
 * Buffers: row_start [n+1], pack [n*len] (padded flat index of each packed token), row [n*len]
 * (row of each packed token), scorer_rows [n*(1+kmax)] (position 0, then the marker slots).
 * *t_out receives the packed token count T; pack and row are filled up to T. */
int s1_pack_tables(uint32_t n, uint32_t len, uint32_t kmax, const uint32_t* attention_mask,
                   const uint64_t* seq_lens, const uint32_t* marker_pos,
                   const uint64_t* marker_count, int32_t* row_start, int32_t* pack, int32_t* row,
                   int32_t* scorer_rows, uint32_t* t_out);

/* Per-kernel timing of the forwards run since the last reset, collected with HIP events on the
 * model's stream when the `ops` setting is on. Writes up to `cap` entries; returns the count.
 * names: "\n"-separated kernel names into names_out (names_cap bytes). */
int s1_op_stats(const s1_model* m, char* names_out, size_t names_cap, uint64_t* counts,
                double* total_ms, int cap);
void s1_op_stats_reset(s1_model* m);

/* ---- Kernel-level entry points on device pointers (tests and microbenchmarks) --------------
 * They mirror the reference's kernel wrappers that its load-time checks call: NaxGemm::matmul /
 * addmm (runtime/crates/laya-mlx/src/nax_gemm.rs:371-430) and SplitRope::apply
 * (runtime/crates/laya-mlx/src/split_rope.rs:360-364). `stream` is a hipStream_t (NULL = the
 * null stream). bf16 buffers are uint16 bit patterns. */

/* C = A[M,K] . W[N,K]^T. epi 0: C bf16 (+bias, act 0 none / 1 relu / 2 gelu); 1: C f32 += acc
 * (+bias); 2: GeGLU on W with rows interleaved by 32 (x, gate), C bf16 [M, N/2];
 * 3: C f32 = acc (+bias). K a multiple of 64, N of 128; W spans less than 4 GiB ((N - 1) ldw
 * + K elements), and an A that spans more runs as row pieces (8 rows of it must span less),
 * else S1_ERR_CONFIG before anything reaches the GPU. */
int s1k_gemm(const void* A, int lda, const void* W, int ldw, void* C, int ldc, const float* bias,
             int M, int N, int K, int epi, int act, void* stream);

/* s1k_gemm without any allocation: no counterpart in the reference; it is for callers that cannot
 * allocate device memory (code under HIP graph capture, tight serving loops, harnesses that
 * forbid hipMalloc). Same arguments and results as s1k_gemm (bit for bit: the same kernels and
 * split-K plan), but a shape that splits K keeps its f32 partials in a static array of the
 * library (8 MiB per GPU, held until the process ends) instead of a workspace the library
 * allocates; every split plan fits it, and a shape that would not is refused with S1_ERR_CONFIG.
 * All calls on one GPU share that array: calls that overlap on one GPU (other streams, other
 * threads) race and must be serialised by the caller. The first call on each GPU looks up the
 * array's device address and must not be made under graph capture (it is then refused with
 * S1_ERR_CONFIG); later calls may be captured and replayed. */
int s1k_gemm_noalloc(const void* A, int lda, const void* W, int ldw, void* C, int ldc, const float* bias,
                     int M, int N, int K, int epi, int act, void* stream);

/* Wqkv product with the q|k|v split and RoPE fused in its epilogue (the fuserope path):
 * A [M, d] bf16, W [3d, d] bf16, pos [M] int32 positions, theta the RoPE base; writes q and k
 * as [d/64, M, 64] bf16 and v transposed as [d/64, 64, v_ld] bf16 (v_ld a multiple of 8,
 * at least M + 64: the layout the attention kernel reads); v columns from M up to the next
 * multiple of 8 are written as zeros. */
int s1k_qkv_rope(const void* A, const void* W, int M, int d, const int32_t* pos, double theta,
                 void* q, void* k, void* v, int v_ld, void* stream);

/* Standalone split + RoPE pass: qkv [M, 3d] bf16 -> q, k [d/64, M, 64] bf16 and v transposed
 * [d/64, 64, v_ld] bf16 (v_ld a multiple of 8, at least M rounded up to 8; v columns from M
 * up to that are written as zeros). theta <= 0 means no rotation (the decision head's split). */
int s1k_split_rope(const void* qkv, int M, int d, const int32_t* pos, double theta, void* q,
                   void* k, void* v, int v_ld, void* stream);

/* Attention over packed rows: q, k [H, T, 64] bf16, v transposed [H, 64, v_ld] bf16 (v_ld >=
 * T rounded up to 8, plus 64), seq_starts [nseq + 1] int32 (host memory), window < 0 for
 * global, else |i - j| <= window; out [T, H*64] bf16. */
int s1k_attention(const void* q, const void* k, const void* v, int v_ld, int T, int H,
                  const int32_t* seq_starts, int nseq, int window, float scale, void* out,
                  void* stream);

/* LayerNorm over rows of d: x f32 [M, d] -> y bf16 [M, d]; b may be NULL. */
int s1k_layernorm(const float* x, const float* w, const float* b, float eps, int M, int d,
                  void* y, void* stream);

#ifdef __cplusplus
}
#endif

#endif /* SYS1HIP_H */
