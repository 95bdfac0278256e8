// Shared host-side types of libsys1hip: error kinds, the model configuration and bf16 helpers.
#pragma once

#include <algorithm>
#include <cmath>
#include <cstdint>
#include <cstring>
#include <stdexcept>
#include <string>
#include <vector>

#include "json_mini.hpp"

namespace s1 {

// Error kinds of the C ABI (0 is success). They mirror laya_core::Error's variants
// (runtime/crates/laya-core/src/error.rs:1-17): Config, Weights, Backend, plus Batch for a
// malformed batch that the Rust side would have rejected before calling the backend.
enum ErrKind : int { kOk = 0, kConfig = 1, kWeights = 2, kBackend = 3, kBatch = 4 };

struct Error : std::runtime_error {
  ErrKind kind;
  Error(ErrKind k, const std::string& m) : std::runtime_error(m), kind(k) {}
};

[[noreturn]] inline void fail(ErrKind k, const std::string& m) { throw Error(k, m); }

// The ModernBERT encoder shape, normalised across the transformers 4.x and 5.x config layouts
// (runtime/crates/laya-core/src/config.rs:96-159), plus the agent-level fields the backend reads
// (config.rs:9-40): head layers, max lengths.
struct ModelConfig {
  int vocab = 0;
  int d = 0;
  int layers = 0;
  int heads = 0;
  int inter = 0;
  double eps = 1e-5;
  int global_every = 3;
  int local_attention = 128;
  double global_theta = 160000.0;
  double local_theta = 10000.0;
  int pad_token_id = 0;
  int max_pos = 8192;
  std::vector<uint8_t> layer_local;
  int head_layers = 2;
  int max_len = 512;
  int head_max_len = 192;

  int head_dim() const { return d / heads; }
  int window() const { return local_attention / 2; }
  int head_nheads() const { return std::max(1, d / 64); }
};

// encoder/config.json -> ModelConfig, with the same defaults and checks as
// EncoderConfig::from_value (config.rs:96-201).
inline ModelConfig parse_model_config(const std::string& enc_json, const std::string& agent_json) {
  ModelConfig c;
  JsonValue v, a;
  try {
    v = parse_json(enc_json);
  } catch (const std::exception& e) {
    fail(kConfig, std::string("encoder config: ") + e.what());
  }
  if (!agent_json.empty()) {
    try {
      a = parse_json(agent_json);
    } catch (const std::exception& e) {
      fail(kConfig, std::string("agent config: ") + e.what());
    }
  }
  auto get_u = [&](const char* k) -> int64_t {
    const JsonValue* x = v.get(k);
    if (!x || x->kind != JsonValue::Number || !x->is_int || x->i < 0)
      fail(kConfig, std::string("encoder config: missing integer '") + k + "'");
    return x->i;
  };
  auto get_u_or = [&](const char* k, int64_t d) -> int64_t {
    const JsonValue* x = v.get(k);
    if (!x || x->kind != JsonValue::Number || !x->is_int || x->i < 0) return d;
    return x->i;
  };
  auto get_f_or = [&](const JsonValue& src, const char* k, double d) -> double {
    const JsonValue* x = src.get(k);
    if (!x || x->kind != JsonValue::Number) return d;
    return x->num;
  };
  const JsonValue* mt = v.get("model_type");
  if (!mt || mt->kind != JsonValue::String || mt->str != "modernbert")
    fail(kConfig, "unsupported encoder model_type; only 'modernbert' is implemented");
  c.layers = int(get_u("num_hidden_layers"));
  c.global_every = int(get_u_or("global_attn_every_n_layers", 3));
  if (c.global_every == 0) fail(kConfig, "encoder config: global_attn_every_n_layers must be at least 1");
  c.global_theta = get_f_or(v, "global_rope_theta", 160000.0);
  c.local_theta = get_f_or(v, "local_rope_theta", 10000.0);
  if (const JsonValue* t = v.path({"rope_parameters", "full_attention", "rope_theta"}))
    if (t->kind == JsonValue::Number) c.global_theta = t->num;
  if (const JsonValue* t = v.path({"rope_parameters", "sliding_attention", "rope_theta"}))
    if (t->kind == JsonValue::Number) c.local_theta = t->num;
  const JsonValue* lt = v.get("layer_types");
  c.layer_local.resize(c.layers);
  if (lt && lt->kind == JsonValue::Array && int(lt->arr.size()) == c.layers) {
    for (int i = 0; i < c.layers; ++i)
      c.layer_local[i] = lt->arr[i].kind == JsonValue::String && lt->arr[i].str == "sliding_attention";
  } else {
    for (int i = 0; i < c.layers; ++i) c.layer_local[i] = (i % c.global_every) != 0;
  }
  c.vocab = int(get_u("vocab_size"));
  c.d = int(get_u("hidden_size"));
  c.heads = int(get_u("num_attention_heads"));
  c.inter = int(get_u("intermediate_size"));
  c.eps = get_f_or(v, "norm_eps", get_f_or(v, "layer_norm_eps", 1e-5));
  c.local_attention = int(get_u_or("local_attention", 128));
  const JsonValue* pt = v.get("pad_token_id");
  c.pad_token_id = (pt && pt->kind == JsonValue::Number && pt->is_int) ? int(pt->i) : 0;
  c.max_pos = int(get_u_or("max_position_embeddings", 8192));
  // check_shapes (config.rs:166-190)
  if (c.heads == 0) fail(kConfig, "encoder config: num_attention_heads must be at least 1");
  if (c.d == 0) fail(kConfig, "encoder config: hidden_size must be at least 1");
  if (c.d % c.heads != 0)
    fail(kConfig, "encoder config: hidden_size " + std::to_string(c.d) +
                      " is not a multiple of num_attention_heads " + std::to_string(c.heads));
  if (c.d % c.head_nheads() != 0)
    fail(kConfig, "encoder config: hidden_size is not a multiple of the decision-head attention heads");
  if (c.local_attention < 2) fail(kConfig, "encoder config: local_attention must be at least 2");
  if (a.kind == JsonValue::Object) {
    auto au = [&](const char* k, int dflt) {
      const JsonValue* x = a.get(k);
      return (x && x->kind == JsonValue::Number && x->is_int && x->i >= 0) ? int(x->i) : dflt;
    };
    c.head_layers = au("head_layers", 2);
    c.max_len = au("max_len", 512);
    c.head_max_len = au("head_max_len", 192);
  }
  return c;
}

// Round-to-nearest-even f32 -> bf16 (NaN kept quiet).
inline uint16_t f32_to_bf16(float f) {
  uint32_t u;
  std::memcpy(&u, &f, 4);
  if ((u & 0x7fffffffu) > 0x7f800000u) return uint16_t((u >> 16) | 0x40);
  u += 0x7fffu + ((u >> 16) & 1u);
  return uint16_t(u >> 16);
}
inline float bf16_to_f32(uint16_t h) {
  uint32_t u = uint32_t(h) << 16;
  float f;
  std::memcpy(&f, &u, 4);
  return f;
}
inline float f16_to_f32(uint16_t h) {
  uint32_t sign = uint32_t(h & 0x8000u) << 16;
  uint32_t exp = (h >> 10) & 0x1fu;
  uint32_t man = h & 0x3ffu;
  uint32_t u;
  if (exp == 0) {
    if (man == 0) {
      u = sign;
    } else {  // subnormal: renormalise
      int e = -1;
      do {
        man <<= 1;
        ++e;
      } while (!(man & 0x400u));
      man &= 0x3ffu;
      u = sign | (uint32_t(127 - 15 - e) << 23) | (man << 13);
    }
  } else if (exp == 31) {
    u = sign | 0x7f800000u | (man << 13);
  } else {
    u = sign | ((exp + 127 - 15) << 23) | (man << 13);
  }
  float f;
  std::memcpy(&f, &u, 4);
  return f;
}
// f32 -> f16, round to nearest even; overflow goes to infinity, NaN stays a (quiet) NaN.
inline uint16_t f32_to_f16(float f) {
  uint32_t x;
  std::memcpy(&x, &f, 4);
  const uint16_t sign = uint16_t((x >> 16) & 0x8000u);
  const uint32_t ax = x & 0x7fffffffu;
  if (ax > 0x7f800000u) return uint16_t(sign | 0x7e00u);
  if (ax >= 0x477ff000u) return uint16_t(sign | 0x7c00u);  // >= 65520 rounds past 65504
  if (ax < 0x38800000u) {                                  // below 2^-14: a subnormal f16, units of 2^-24
    const int e = int(ax >> 23);
    const int shift = 126 - e;
    if (e == 0 || shift > 24) return sign;
    const uint32_t m = (ax & 0x7fffffu) | 0x800000u;
    uint32_t q = m >> shift;
    const uint32_t rem = m & ((1u << shift) - 1u), half = 1u << (shift - 1);
    if (rem > half || (rem == half && (q & 1u))) ++q;
    return uint16_t(sign | q);
  }
  const uint32_t r = ax + 0xfffu + ((ax >> 13) & 1u) - ((127u - 15u) << 23);
  return uint16_t(sign | (r >> 13));
}

}  // namespace s1
