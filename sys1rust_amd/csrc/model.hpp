// The loaded decision model on one GPU: device weights, activation arena, stream and the
// per-request plan. Mirrors MlxBackend (runtime/crates/laya-mlx/src/lib.rs:960-1879).
#pragma once

#include <hip/hip_runtime.h>

#include <string>
#include <vector>

#include "common.hpp"
#include "kernels.hpp"
#include "safetensors.hpp"

namespace s1 {

// Strict settings, parsed like the reference's Knobs (lib.rs:155-259): a comma list of `key` or
// `key=value`, the last mention wins, an unknown key or a bad value is a config error. Every key
// Knobs accepts is accepted with Knobs' value checks, so the runtime's production string
// (sys1rust/src/config.rs:29) loads unchanged. Keys shared with Knobs default as Knobs does (off);
// this backend's own fusions default on.
struct Settings {
  // Keys with the same meaning as in Knobs.
  bool trace = false;      // print per-forward timings to stderr
  bool layers = false;     // per-layer timing to stderr (runs without graphs)
  bool ops = false;        // per-kernel HIP-event timing (s1_op_stats)
  bool clear = false;      // release the activation arena and graphs after every forward
  bool headprune = false;  // last head layer only at the scorer's rows (lib.rs:1728-1748)
  bool fuserope = false;   // RoPE + split fused into the Wqkv GEMM epilogue
  size_t pad = 1;          // padded_len multiple
  std::vector<size_t> buckets;
  std::vector<size_t> warm;  // row counts to run one forward for at every bucket length at load
  // The reference's local-attention mask choices (lib.rs:1241-1270). At real tokens every choice
  // gives the same attention (masks are exact exclusion here, the same values as either MLX
  // form), so the forward ignores them; the padded layout of encoder_hidden follows them at the
  // padding positions, whose key sets they decide.
  bool bool_mask = false;  // mask=bool
  bool windowed = true;    // chunked local attention above dense_upto
  long dense_upto = -1;    // -1: 4 * window
  size_t band = 0;         // banded (zero-filled) chunks from this padded length up; needs fuserope
  // Keys of Knobs whose MLX mechanism has no counterpart here; parsed and checked, no effect:
  // unpad (this path always runs the packed token layout), geglu / f16gelu (GeGLU always in
  // f32), addmm (the residual add is always in the GEMM epilogue), nax / wcopy / directload /
  // sharehead (weight layout and MLX gemm choice), cache / wired (MLX memory limits),
  // parallel_load (the runtime's).
  bool unpad = false;
  // This backend's own.
  bool fusegeglu = true;   // GeGLU fused into the Wi GEMM epilogue (Wi rows interleaved at load)
  bool fuseln = true;      // a split-K Wo / Wo2 finishes in the kernel of the LayerNorm after it
  bool graphs = true;      // replay each repeated batch shape from a captured HIP graph
  bool f16 = false;        // dtype=f16: weights and activations in f16 (the checkpoint's type), not bf16
  bool f32 = false;        // dtype=f32: f32 weights and compute (BackendOptions::f32), the plain f32 kernels
  static Settings parse(const std::string& spec);
};

struct LayerWeights {
  uint16_t* wqkv = nullptr;  // [3d, d]
  uint16_t* wo = nullptr;    // [d, d]
  uint16_t* wi = nullptr;    // [2I, d], rows interleaved by 32 when fusegeglu
  uint16_t* wo2 = nullptr;   // [d, I]
  float* attn_norm = nullptr;  // null for layer 0
  float* mlp_norm = nullptr;
  bool local = false;
};

struct HeadWeights {
  float *n1w, *n1b, *n2w, *n2b;
  uint16_t* in_w;
  float* in_b;
  uint16_t* out_w;
  float* out_b;
  uint16_t* l1_w;
  float* l1_b;
  uint16_t* l2_w;
  float* l2_b;
};

// The packed token layout of a right-padded batch (Packing::new and MlxBackend::scorer_rows,
// runtime/crates/laya-mlx/src/lib.rs:894-943, 1502-1521). Validates the batch on the way.
struct Packed {
  int T = 0;
  std::vector<int> row_start;    // [n + 1] packed index of position 0 of each row, then T
  std::vector<int> pack;         // [T] padded flat index r * len + pos of each packed token
  std::vector<int> row;          // [T] row of each packed token
  std::vector<int> scorer_rows;  // [n * (1 + kmax)] packed index of position 0, then the kmax
                                 // marker slots (slots past marker_count point at position 0)
};
Packed pack_batch(uint32_t n, uint32_t len, uint32_t kmax, const uint32_t* mask, const uint64_t* seq_lens,
                  const uint32_t* marker_pos, const uint64_t* marker_count, int max_pos);

// A validated batch in packed form, plus every index table the kernels read.
struct Plan {
  int n = 0, len = 0, kmax = 0;
  int T = 0;  // rows of the forward: the real tokens (packed layout) or n * len (padded)
  int P = 0;  // picked rows of the pruned head layer (n * (1 + kmax))
  int R = 0;  // scorer rows (n * kmax)
  std::vector<int> row_start;  // [n + 1]
  // device-bound tables (int32), concatenated in `meta`
  std::vector<int> meta;
  size_t off_ids = 0, off_pos = 0, off_seg = 0, off_tiles = 0, off_ltiles = 0, off_ptiles = 0, off_picked = 0,
         off_scorer = 0, off_pooled = 0;
  int ntiles = 0, nltiles = 0, nptiles = 0;
  int gq = 256;  // queries per global-attention tile
  int lq = 128;  // queries per local-attention tile
  // The padded layout (encoder_hidden): every one of the n * len positions is a row of the
  // forward (T = n * len). The local-attention tiles take the real tokens and the padding
  // queries whose keys are the real keys of their window; the other padding queries of local
  // layers are listed at off_far with their key sets (attn_fallback_launch's entries).
  bool padded = false;
  size_t off_far = 0;
  int nfar = 0;
  // dtype=f32: every query's key set in attn32_launch's entry format, for global (off_eg) and
  // local (off_el) layers, T entries each.
  size_t off_eg = 0, off_el = 0;
};

struct Model {
  ModelConfig cfg;
  Settings set;
  int elem = ELEM_BF16;  // 16-bit type of weights and activations (set.f16)
  int device = 0;
  int scorer_width = 0;
  hipStream_t stream = nullptr;
  std::string name, kernels;

  // weights (one device allocation) and the RoPE tables (another)
  void* wmem = nullptr;
  void* rmem = nullptr;
  uint16_t* tok_emb = nullptr;
  float* emb_norm = nullptr;
  std::vector<LayerWeights> layers;
  float* final_norm = nullptr;
  float* type_emb = nullptr;  // [3, d] f32
  std::vector<HeadWeights> head;
  float *sc0_w = nullptr, *sc0_b = nullptr;
  uint16_t* sc1_w = nullptr;
  float* sc1_b = nullptr;
  float* sc3_w = nullptr;
  float* sc3_b = nullptr;
  float* rope_cos[2] = {nullptr, nullptr};  // [max_pos, hd/2] for global (0) and local (1)
  float* rope_sin[2] = {nullptr, nullptr};

  // activation arena, grown on demand
  void* amem = nullptr;
  size_t acap = 0;
  // the dtype=f32 path's activation arena
  void* fmem = nullptr;
  size_t fcap = 0;
  // pinned host staging
  void* hmeta = nullptr;
  size_t hmeta_cap = 0;
  void* hout = nullptr;
  size_t hout_cap = 0;
  int* dmeta = nullptr;
  size_t dmeta_cap = 0;

  // per-kernel timing (Settings::ops)
  struct OpRec {
    const char* name;
    hipEvent_t a, b;
  };
  std::vector<OpRec> pending;
  std::vector<hipEvent_t> event_pool;
  std::vector<std::pair<std::string, std::pair<uint64_t, double>>> stats;
  std::vector<hipEvent_t> layer_ev;  // Settings::layers

  // HIP graphs of repeated batch shapes (Settings::graphs)
  struct GraphEntry {
    std::vector<int64_t> key;
    hipGraphExec_t exec;
    uint64_t last_use;
  };
  static constexpr size_t kMaxGraphs = 32;
  std::vector<GraphEntry> graphs;
  std::vector<std::vector<int64_t>> graph_seen;
  uint64_t graph_clock = 0;

  // The row kernels keep a hidden-state row in registers: up to this width.
  static constexpr int kMaxHidden = 2048;

  Model(const SafeTensors& st, const std::string& enc_json, const std::string& agent_json,
        const std::string& settings, int device);
  ~Model();

  Plan plan(uint32_t n, uint32_t len, uint32_t kmax, const uint32_t* ids, const uint32_t* mask,
            const uint64_t* seq_lens, const uint32_t* marker_pos, const uint64_t* marker_count,
            const uint32_t* qtype) const;
  // The encoder over the padded layout (plan_padded), as MlxBackend::encoder_hidden runs it.
  Plan plan_padded(uint32_t n, uint32_t len, const uint32_t* ids, const uint32_t* mask, const uint64_t* seq_lens) const;
  void forward(const Plan& p, float* logits, float* pooled);
  void encoder_hidden(const Plan& p, float* hidden);
  size_t padded_len(size_t len) const;

 private:
  struct Acts;
  struct Acts32;
  Acts32 arena32(const Plan& p);
  void run_encoder32(const Plan& p, const Acts32& a);
  void forward32(const Plan& p, float* logits, float* pooled);
  void encoder_hidden32(const Plan& p, float* hidden);
  // The f32 GEMM weights: with dtype=f32 the 16-bit weight pointers hold f32 tensors.
  static const float* w32(const uint16_t* w) { return reinterpret_cast<const float*>(w); }
  void init(const SafeTensors& st, const std::string& enc_json, const std::string& agent_json,
            const std::string& settings);
  void teardown();
  Acts arena(const Plan& p);
  void upload(const Plan& p);
  // Enqueues the encoder; with fold_last, the last layer's Wo2 may leave its split-K partials in
  // the workspace for the caller's next kernel: returns their count then (else 0).
  int run_encoder(const Plan& p, const Acts& a, bool fold_last = false);
  void enqueue_forward(const Plan& p, const Acts& a);
  template <class F>
  void run(const Plan& p, int kind, F&& enqueue);
  void drop_graphs();
  void warm_buckets();
  void release();
  template <class F>
  void op(const char* name, F&& f);
  void collect_stats();
  void layer_mark();
  void layer_report();
};

}  // namespace s1
