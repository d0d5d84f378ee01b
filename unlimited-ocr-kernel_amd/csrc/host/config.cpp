// ModelConfig (src/model/config.rs:30-115): required fields, defaults, and
// the validation rules (unsupported attention/routing -> Unsupported,
// inconsistent sizes -> Shape). Malformed or mistyped JSON -> Json.
#include <cmath>
#include <fstream>
#include <sstream>

#include "../../../include/uocr.hpp"
#include "json.hpp"

namespace uocr {

ModelConfig ModelConfig::load(const std::string& path) {
  std::ifstream in(path, std::ios::binary);
  if (!in) throw OcrError(ErrorKind::Io, "cannot read " + path);
  std::ostringstream ss;
  ss << in.rdbuf();
  return from_json(ss.str());
}

ModelConfig ModelConfig::from_json(const std::string& text) {
  host::Json j;
  std::string err;
  if (!host::parse_json(text.data(), text.size(), j, err))
    throw OcrError(ErrorKind::Json, "config: " + err);
  if (j.kind != host::Json::Object) throw OcrError(ErrorKind::Json, "config is not an object");
  auto bad = [](const char* key) {
    return OcrError(ErrorKind::Json, std::string("config: missing or invalid ") + key);
  };
  auto get_size = [&](const char* key, size_t& out, bool required) {
    const host::Json* v = j.find(key);
    if (!v) {
      if (required) throw bad(key);
      return;
    }
    if (!v->is_uint()) throw bad(key);
    out = (size_t)v->as_uint();
  };
  auto get_bool = [&](const char* key, bool& out, bool required) {
    const host::Json* v = j.find(key);
    if (!v) {
      if (required) throw bad(key);
      return;
    }
    if (v->kind != host::Json::Bool) throw bad(key);
    out = v->b;
  };
  auto get_f32 = [&](const char* key, float& out) {
    const host::Json* v = j.find(key);
    if (!v) return;
    if (v->kind != host::Json::Number) throw bad(key);
    out = (float)v->as_double();
  };
  auto get_string = [&](const char* key, std::string& out, bool required) {
    const host::Json* v = j.find(key);
    if (!v) {
      if (required) throw bad(key);
      return;
    }
    if (v->kind != host::Json::String) throw bad(key);
    out = v->text;
  };
  ModelConfig c;
  get_string("model_type", c.model_type, true);
  get_size("hidden_size", c.hidden_size, true);
  get_size("intermediate_size", c.intermediate_size, true);
  get_size("moe_intermediate_size", c.moe_intermediate_size, true);
  get_size("num_hidden_layers", c.num_hidden_layers, true);
  get_size("num_attention_heads", c.num_attention_heads, true);
  get_size("num_key_value_heads", c.num_key_value_heads, true);
  get_size("n_routed_experts", c.n_routed_experts, true);
  get_size("n_shared_experts", c.n_shared_experts, true);
  get_size("num_experts_per_tok", c.num_experts_per_tok, true);
  get_size("first_k_dense_replace", c.first_k_dense_replace, true);
  get_bool("use_mla", c.use_mla, true);
  get_size("vocab_size", c.vocab_size, true);
  get_size("sliding_window", c.sliding_window, false);
  get_f32("rms_norm_eps", c.rms_norm_eps);
  get_f32("rope_theta", c.rope_theta);
  get_bool("norm_topk_prob", c.norm_topk_prob, false);
  get_f32("routed_scaling_factor", c.routed_scaling_factor);
  get_size("max_position_embeddings", c.max_position_embeddings, false);
  get_string("topk_method", c.topk_method, false);
  get_string("scoring_func", c.scoring_func, false);
  get_size("moe_layer_freq", c.moe_layer_freq, false);
  if (const host::Json* v = j.find("rope_scaling")) c.has_rope_scaling = v->kind != host::Json::Null;
  get_bool("attention_bias", c.attention_bias, false);

  if (c.model_type != "unlimited-ocr" || c.use_mla || c.attention_bias || c.has_rope_scaling ||
      c.topk_method != "greedy" || c.scoring_func != "softmax" || c.moe_layer_freq != 1)
    throw OcrError(ErrorKind::Unsupported, "model attention or routing configuration");
  if (c.hidden_size == 0 || c.num_attention_heads == 0 ||
      c.hidden_size % c.num_attention_heads != 0 ||
      (c.hidden_size / c.num_attention_heads) % 2 != 0 ||
      c.num_attention_heads != c.num_key_value_heads || c.num_hidden_layers == 0 ||
      c.vocab_size == 0 || c.intermediate_size == 0 || c.moe_intermediate_size == 0 ||
      c.n_shared_experts == 0 || c.num_experts_per_tok == 0 ||
      c.num_experts_per_tok > c.n_routed_experts ||
      c.first_k_dense_replace > c.num_hidden_layers || c.sliding_window == 0 ||
      c.max_position_embeddings == 0 || !std::isfinite(c.rms_norm_eps) || c.rms_norm_eps <= 0 ||
      !std::isfinite(c.rope_theta) || c.rope_theta <= 0 ||
      !std::isfinite(c.routed_scaling_factor) || c.routed_scaling_factor <= 0)
    throw OcrError(ErrorKind::Shape, "invalid decoder configuration");
  return c;
}

uocr_moe_config ModelConfig::moe() const {
  uocr_moe_config m;
  m.hidden_size = (uint32_t)hidden_size;
  m.moe_intermediate_size = (uint32_t)moe_intermediate_size;
  m.n_routed_experts = (uint32_t)n_routed_experts;
  m.n_shared_experts = (uint32_t)n_shared_experts;
  m.num_experts_per_tok = (uint32_t)num_experts_per_tok;
  m.norm_topk_prob = norm_topk_prob ? 1u : 0u;
  m.routed_scaling_factor = routed_scaling_factor;
  m.rms_norm_eps = rms_norm_eps;
  return m;
}

}  // namespace uocr
