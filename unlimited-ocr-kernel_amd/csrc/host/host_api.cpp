// C entry points over the C++ host surface (include/uocr.hpp): safetensors
// checkpoints, INT8 overlays, model configs and whole-model loading. Every
// OcrError becomes its status code with the message in uocr_last_error.
#include <cstring>
#include <new>

#include "../../../include/uocr.hpp"

namespace uocr::host {
int set_last_error(int status, const char* message);
}

struct uocr_checkpoint {
  std::unique_ptr<uocr::Checkpoint> ck;
  std::vector<std::string> names;
};

struct uocr_model {
  std::unique_ptr<uocr::Model> model;
};

namespace {

template <typename F>
int guarded(F f) {
  try {
    f();
    return UOCR_OK;
  } catch (const uocr::OcrError& e) {
    return uocr::host::set_last_error(e.status(), e.what());
  } catch (const std::bad_alloc&) {
    return uocr::host::set_last_error(UOCR_ERR_RESOURCE, "host allocation failed");
  } catch (const std::exception& e) {
    return uocr::host::set_last_error(UOCR_ERR_IO, e.what());
  }
}

int dtype_code(uocr::DType d) {
  switch (d) {
    case uocr::DType::BF16: return UOCR_DTYPE_BF16;
    case uocr::DType::F16: return UOCR_DTYPE_F16;
    case uocr::DType::F32: return UOCR_DTYPE_F32;
    case uocr::DType::I64: return UOCR_DTYPE_I64;
    case uocr::DType::I8: return UOCR_DTYPE_I8;
  }
  return -1;
}

}  // namespace

extern "C" {

int uocr_checkpoint_open(const char* path, uocr_checkpoint** out) {
  if (!path || !out) return uocr::host::set_last_error(UOCR_ERR_SHAPE, "null argument");
  *out = nullptr;
  return guarded([&] {
    std::unique_ptr<uocr_checkpoint> c(new uocr_checkpoint());
    c->ck = uocr::Checkpoint::open(path);
    c->names = c->ck->names();
    *out = c.release();
  });
}

void uocr_checkpoint_close(uocr_checkpoint* c) { delete c; }

int uocr_checkpoint_sha256(const uocr_checkpoint* c, char out[65]) {
  if (!c || !out) return uocr::host::set_last_error(UOCR_ERR_SHAPE, "null argument");
  return guarded([&] {
    const std::string h = c->ck->sha256();
    std::memcpy(out, h.c_str(), 65);
  });
}

size_t uocr_checkpoint_count(const uocr_checkpoint* c) { return c ? c->names.size() : 0; }

const char* uocr_checkpoint_name(const uocr_checkpoint* c, size_t i) {
  return c && i < c->names.size() ? c->names[i].c_str() : nullptr;
}

const char* uocr_checkpoint_metadata(const uocr_checkpoint* c, const char* key) {
  if (!c || !key) return nullptr;
  const auto& md = c->ck->metadata();
  const auto it = md.find(key);
  return it == md.end() ? nullptr : it->second.c_str();
}

int uocr_checkpoint_tensor(const uocr_checkpoint* c, const char* name, int* dtype, size_t* shape,
                           size_t max_dims, size_t* ndim, const void** data, size_t* bytes) {
  if (!c || !name) return uocr::host::set_last_error(UOCR_ERR_SHAPE, "null argument");
  return guarded([&] {
    const uocr::WeightView w = c->ck->tensor(name);
    if (dtype) *dtype = dtype_code(w.dtype);
    if (ndim) *ndim = w.shape->size();
    if (shape)
      for (size_t i = 0; i < w.shape->size() && i < max_dims; i++) shape[i] = (*w.shape)[i];
    if (data) *data = w.bytes;
    if (bytes) *bytes = w.size;
  });
}

int uocr_overlay_validate(const char* overlay_path, const uocr_checkpoint* source,
                          size_t* matrices) {
  if (!overlay_path || !source) return uocr::host::set_last_error(UOCR_ERR_SHAPE, "null argument");
  return guarded([&] {
    const auto q = uocr::QuantizedWeights::load(overlay_path, *source->ck);
    if (matrices) *matrices = q->size();
  });
}

int uocr_config_load(const char* path, uocr_model_config* out) {
  if (!path || !out) return uocr::host::set_last_error(UOCR_ERR_SHAPE, "null argument");
  return guarded([&] {
    const uocr::ModelConfig c = uocr::ModelConfig::load(path);
    out->hidden_size = (uint32_t)c.hidden_size;
    out->intermediate_size = (uint32_t)c.intermediate_size;
    out->moe_intermediate_size = (uint32_t)c.moe_intermediate_size;
    out->num_hidden_layers = (uint32_t)c.num_hidden_layers;
    out->num_attention_heads = (uint32_t)c.num_attention_heads;
    out->num_key_value_heads = (uint32_t)c.num_key_value_heads;
    out->n_routed_experts = (uint32_t)c.n_routed_experts;
    out->n_shared_experts = (uint32_t)c.n_shared_experts;
    out->num_experts_per_tok = (uint32_t)c.num_experts_per_tok;
    out->first_k_dense_replace = (uint32_t)c.first_k_dense_replace;
    out->vocab_size = (uint32_t)c.vocab_size;
    out->norm_topk_prob = c.norm_topk_prob ? 1u : 0u;
    out->routed_scaling_factor = c.routed_scaling_factor;
    out->rms_norm_eps = c.rms_norm_eps;
  });
}

int uocr_model_load(uocr_gpu_ctx* ctx, const char* directory, const char* overlay,
                    uocr_quant_mode mode, uocr_model** out) {
  if (!directory || !out) return uocr::host::set_last_error(UOCR_ERR_SHAPE, "null argument");
  *out = nullptr;
  if (mode != UOCR_QUANT_WEIGHTS_ONLY && mode != UOCR_QUANT_DYNAMIC_ACTIVATIONS)
    return uocr::host::set_last_error(UOCR_ERR_SHAPE, "mode must be a QuantizationMode");
  return guarded([&] {
    const std::string ov = overlay ? overlay : "";
    std::unique_ptr<uocr_model> m(new uocr_model());
    m->model = uocr::Model::load_with_quantization(
        directory, overlay ? &ov : nullptr,
        mode == UOCR_QUANT_WEIGHTS_ONLY ? uocr::QuantizationMode::WeightsOnly
                                        : uocr::QuantizationMode::DynamicActivations,
        ctx);
    *out = m.release();
  });
}

const char* uocr_model_precision(const uocr_model* m) {
  return m ? m->model->precision() : nullptr;
}

const uocr_moe_layer* uocr_model_layer(const uocr_model* m, size_t layer) {
  return m ? m->model->moe_layer(layer) : nullptr;
}

int uocr_model_experts(uocr_gpu_ctx* ctx, const uocr_model* m, size_t layer, const float* x,
                       size_t T, float* y, uint32_t flags) {
  if (!ctx || !m) return uocr::host::set_last_error(UOCR_ERR_SHAPE, "null argument");
  return guarded([&] { m->model->experts(ctx, layer, x, T, y, flags); });
}

int uocr_model_logits(uocr_gpu_ctx* ctx, const uocr_model* m, const float* hidden, size_t T,
                      float* logits) {
  if (!ctx || !m) return uocr::host::set_last_error(UOCR_ERR_SHAPE, "null argument");
  return guarded([&] { m->model->logits(ctx, hidden, T, logits); });
}

void uocr_model_destroy(uocr_model* m) { delete m; }

}  // extern "C"
