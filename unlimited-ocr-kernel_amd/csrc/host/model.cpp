// OcrError, CpuContext (src/cpu/mod.rs:18-79) and the MoE part of Model
// (src/model/mod.rs:60-109): the decoder shape rules of Decoder::new
// (src/decoder/mod.rs:32-88) and one uploaded GPU layer per MoE decoder
// layer, with the overlay attached when given.
#include <cstring>

#include "../../../include/uocr.hpp"

namespace uocr {

OcrError::OcrError(ErrorKind kind, const std::string& message)
    : std::runtime_error(message), kind_(kind) {}

const char* to_string(QuantizationMode mode) {
  return mode == QuantizationMode::WeightsOnly ? "weights_only" : "dynamic_activations";
}

namespace {

[[noreturn]] void throw_status(int status) {
  throw OcrError(static_cast<ErrorKind>(status), uocr_last_error(nullptr));
}

void check(int status) {
  if (status != UOCR_OK) throw_status(status);
}

}  // namespace

CpuContext::CpuContext(Backend backend, size_t threads, size_t scratch_limit)
    : backend_(backend), threads_(threads), scratch_limit_(scratch_limit) {
  if (threads == 0 || scratch_limit == 0)
    throw OcrError(ErrorKind::Resource, "threads and scratch limit must be nonzero");
#if !defined(__aarch64__)
  if (backend == Backend::Neon) throw OcrError(ErrorKind::Unsupported, "NEON requires AArch64");
#endif
#if !defined(__APPLE__)
  if (backend == Backend::Accelerate)
    throw OcrError(ErrorKind::Unsupported, "Accelerate requires macOS");
#endif
  if (backend == Backend::Gpu) check(uocr_gpu_ctx_create(0, scratch_limit, &gpu_));
}

CpuContext::~CpuContext() {
  if (gpu_) uocr_gpu_ctx_destroy(gpu_);
}

namespace {

void expect(const Checkpoint& ck, const std::string& name, std::initializer_list<size_t> shape) {
  const WeightView w = ck.tensor(name);
  if (*w.shape != std::vector<size_t>(shape)) {
    std::string got;
    for (size_t d : *w.shape) got += (got.empty() ? "" : ", ") + std::to_string(d);
    throw OcrError(ErrorKind::Shape, name + ": unexpected shape [" + got + "]");
  }
}

void validate_decoder(const Checkpoint& ck, const ModelConfig& c) {
  const size_t h = c.hidden_size;
  expect(ck, "model.embed_tokens.weight", {c.vocab_size, h});
  expect(ck, "lm_head.weight", {c.vocab_size, h});
  expect(ck, "model.norm.weight", {h});
  for (size_t layer = 0; layer < c.num_hidden_layers; layer++) {
    const std::string prefix = "model.layers." + std::to_string(layer);
    for (const char* part : {"input_layernorm", "post_attention_layernorm"})
      expect(ck, prefix + "." + part + ".weight", {h});
    for (const char* part : {"q_proj", "k_proj", "v_proj", "o_proj"})
      expect(ck, prefix + ".self_attn." + part + ".weight", {h, h});
    auto ffn = [&](const std::string& name, size_t width) {
      expect(ck, name + ".gate_proj.weight", {width, h});
      expect(ck, name + ".up_proj.weight", {width, h});
      expect(ck, name + ".down_proj.weight", {h, width});
    };
    if (layer < c.first_k_dense_replace) {
      ffn(prefix + ".mlp", c.intermediate_size);
    } else {
      expect(ck, prefix + ".mlp.gate.weight", {c.n_routed_experts, h});
      ffn(prefix + ".mlp.shared_experts", c.moe_intermediate_size * c.n_shared_experts);
      for (size_t e = 0; e < c.n_routed_experts; e++)
        ffn(prefix + ".mlp.experts." + std::to_string(e), c.moe_intermediate_size);
    }
  }
}

// Raw bf16 bits of a BF16 checkpoint tensor (the GPU layers store BF16).
const uint16_t* bf16_of(const Checkpoint& ck, const std::string& name) {
  const WeightView w = ck.tensor(name);
  if (w.dtype != DType::BF16)
    throw OcrError(ErrorKind::Unsupported, name + ": the GPU layers take BF16 tensors");
  return reinterpret_cast<const uint16_t*>(w.bytes);
}

// A vector tensor widened to f32 (Tensor::to_f32, src/checkpoint.rs:79-101):
// BF16 and F16 widen exactly, F32 is copied.
std::vector<float> f32_of(const Checkpoint& ck, const std::string& name) {
  const WeightView w = ck.tensor(name);
  size_t n = 1;
  for (size_t d : *w.shape) n *= d;
  std::vector<float> out(n);
  for (size_t i = 0; i < n; i++) {
    uint32_t bits;
    if (w.dtype == DType::F32) {
      std::memcpy(&bits, w.bytes + 4 * i, 4);
    } else if (w.dtype == DType::BF16) {
      uint16_t h;
      std::memcpy(&h, w.bytes + 2 * i, 2);
      bits = (uint32_t)h << 16;
    } else if (w.dtype == DType::F16) {
      uint16_t h;
      std::memcpy(&h, w.bytes + 2 * i, 2);
      const uint32_t sign = (uint32_t)(h >> 15) << 31, ex = (h >> 10) & 0x1f, man = h & 0x3ff;
      if (ex == 0x1f) {
        bits = sign | 0x7f800000u | (man << 13);  // inf / nan
      } else if (ex != 0) {
        bits = sign | ((ex + 112) << 23) | (man << 13);
      } else if (man == 0) {
        bits = sign;  // signed zero
      } else {
        // Subnormal half: man * 2^-24, exact in f32.
        float f = (float)man * 5.9604644775390625e-8f;
        std::memcpy(&bits, &f, 4);
        bits |= sign;
      }
    } else {
      throw OcrError(ErrorKind::Unsupported, name + ": expected a floating-point tensor");
    }
    std::memcpy(&out[i], &bits, 4);
  }
  return out;
}

// Copies the per-expert tensors of one kind into one [E, rows, cols] buffer.
template <typename T, typename Get>
std::vector<T> gather(size_t experts, size_t elems, Get get) {
  std::vector<T> out(experts * elems);
  for (size_t e = 0; e < experts; e++) std::memcpy(out.data() + e * elems, get(e), elems * sizeof(T));
  return out;
}

}  // namespace

std::unique_ptr<Model> Model::load(const std::string& directory, CpuContext& cpu) {
  return load_with_quantization(directory, nullptr, QuantizationMode::WeightsOnly, cpu);
}

std::unique_ptr<Model> Model::load_with_quantization(const std::string& directory,
                                                     const std::string* overlay,
                                                     QuantizationMode mode, CpuContext& cpu) {
  // Every backend runs the reference's validation (same errors); only the
  // upload needs Backend::Gpu.
  return load_with_quantization(directory, overlay, mode, cpu.gpu());
}

std::unique_ptr<Model> Model::load_with_quantization(const std::string& directory,
                                                     const std::string* overlay,
                                                     QuantizationMode mode, uocr_gpu_ctx* gpu) {
  if (!overlay && mode == QuantizationMode::DynamicActivations)
    throw OcrError(ErrorKind::Format, "dynamic INT8 requires a quantized weight overlay");
  std::unique_ptr<Model> m(new Model());
  m->config_ = ModelConfig::load(directory + "/config.json");
  const std::unique_ptr<Checkpoint> ck =
      Checkpoint::open(directory + "/model-00001-of-000001.safetensors");
  validate_decoder(*ck, m->config_);
  std::unique_ptr<QuantizedWeights> q;
  if (overlay) q = QuantizedWeights::load(*overlay, *ck);
  if (!gpu)
    throw OcrError(ErrorKind::Unsupported, "the MoE layers of this library run on Backend::Gpu");
  m->quantized_ = q != nullptr;
  m->mode_ = mode;

  const ModelConfig& c = m->config_;
  const uocr_moe_config cfg = c.moe();
  const size_t H = c.hidden_size, I = c.moe_intermediate_size, E = c.n_routed_experts;
  m->layers_.assign(c.num_hidden_layers, nullptr);
  for (size_t layer = c.first_k_dense_replace; layer < c.num_hidden_layers; layer++) {
    const std::string p = "model.layers." + std::to_string(layer) + ".mlp.";
    auto expert = [&](size_t e, const char* part) {
      return p + "experts." + std::to_string(e) + "." + part + ".weight";
    };
    const std::vector<uint16_t> gate = gather<uint16_t>(
        E, I * H, [&](size_t e) { return bf16_of(*ck, expert(e, "gate_proj")); });
    const std::vector<uint16_t> up = gather<uint16_t>(
        E, I * H, [&](size_t e) { return bf16_of(*ck, expert(e, "up_proj")); });
    const std::vector<uint16_t> down = gather<uint16_t>(
        E, H * I, [&](size_t e) { return bf16_of(*ck, expert(e, "down_proj")); });
    uocr_moe_bf16_weights w;
    w.router = bf16_of(*ck, p + "gate.weight");
    w.expert_gate = gate.data();
    w.expert_up = up.data();
    w.expert_down = down.data();
    w.shared_gate = bf16_of(*ck, p + "shared_experts.gate_proj.weight");
    w.shared_up = bf16_of(*ck, p + "shared_experts.up_proj.weight");
    w.shared_down = bf16_of(*ck, p + "shared_experts.down_proj.weight");
    w.norm_weight = bf16_of(*ck, "model.layers." + std::to_string(layer) +
                                     ".post_attention_layernorm.weight");
    uocr_moe_layer* handle = nullptr;
    check(uocr_moe_layer_create(gpu, &cfg, &w, UOCR_MEMORY_HOST, &handle));
    m->layers_[layer] = handle;
    if (!q) continue;
    auto mat = [&](const std::string& name) {
      const Int8Matrix* x = q->get(name);
      if (!x) throw OcrError(ErrorKind::Format, "overlay lacks " + name);
      return x;
    };
    auto qs = [&](const char* part, size_t elems) {
      return gather<int8_t>(E, elems, [&](size_t e) { return mat(expert(e, part))->weights().data(); });
    };
    auto ss = [&](const char* part, size_t elems) {
      return gather<float>(E, elems, [&](size_t e) { return mat(expert(e, part))->scales().data(); });
    };
    const std::vector<int8_t> qg = qs("gate_proj", I * H), qu = qs("up_proj", I * H),
                              qd = qs("down_proj", H * I);
    const std::vector<float> sg = ss("gate_proj", I * (H / 32)), su = ss("up_proj", I * (H / 32)),
                             sd = ss("down_proj", H * (I / 32));
    const Int8Matrix* shg = mat(p + "shared_experts.gate_proj.weight");
    const Int8Matrix* shu = mat(p + "shared_experts.up_proj.weight");
    const Int8Matrix* shd = mat(p + "shared_experts.down_proj.weight");
    uocr_moe_int8_weights iw;
    iw.expert_gate = qg.data();
    iw.expert_gate_scales = sg.data();
    iw.expert_up = qu.data();
    iw.expert_up_scales = su.data();
    iw.expert_down = qd.data();
    iw.expert_down_scales = sd.data();
    iw.shared_gate = shg->weights().data();
    iw.shared_gate_scales = shg->scales().data();
    iw.shared_up = shu->weights().data();
    iw.shared_up_scales = shu->scales().data();
    iw.shared_down = shd->weights().data();
    iw.shared_down_scales = shd->scales().data();
    check(uocr_moe_layer_attach_int8(
        gpu, handle, &iw, UOCR_MEMORY_HOST,
        mode == QuantizationMode::WeightsOnly ? UOCR_QUANT_WEIGHTS_ONLY : UOCR_QUANT_DYNAMIC_ACTIVATIONS));
  }
  // Decoder::logits: model.norm.weight, and lm_head.weight in BF16 or, when
  // the overlay holds it, INT8 (src/decoder/mod.rs:99-112, 367-379).
  const std::vector<float> final_norm = f32_of(*ck, "model.norm.weight");
  uocr_lm_head_weights lw{};
  lw.vocab_size = (uint32_t)c.vocab_size;
  lw.hidden_size = (uint32_t)H;
  lw.rms_norm_eps = c.rms_norm_eps;
  lw.norm_weight = final_norm.data();
  const Int8Matrix* head_q = q ? q->get("lm_head.weight") : nullptr;
  if (head_q) {
    lw.q = head_q->weights().data();
    lw.scales = head_q->scales().data();
    lw.quant_mode = mode == QuantizationMode::WeightsOnly ? UOCR_QUANT_WEIGHTS_ONLY
                                                          : UOCR_QUANT_DYNAMIC_ACTIVATIONS;
  } else {
    lw.weight = bf16_of(*ck, "lm_head.weight");
    lw.quant_mode = UOCR_QUANT_NONE;
  }
  check(uocr_lm_head_create(gpu, &lw, UOCR_MEMORY_HOST, &m->lm_head_));
  return m;
}

Model::~Model() {
  for (uocr_moe_layer* l : layers_)
    if (l) uocr_moe_layer_destroy(l);
  if (lm_head_) uocr_lm_head_destroy(lm_head_);
}

void Model::logits(CpuContext& cpu, const float* hidden, size_t T, float* logits) const {
  if (cpu.backend() != Backend::Gpu || !cpu.gpu())
    throw OcrError(ErrorKind::Unsupported, "the vocabulary projection runs on Backend::Gpu");
  this->logits(cpu.gpu(), hidden, T, logits);
}

void Model::logits(uocr_gpu_ctx* gpu, const float* hidden, size_t T, float* logits) const {
  check(uocr_lm_head_logits(gpu, lm_head_, hidden, T, logits));
}

const char* Model::precision() const {
  if (!quantized_) return "bf16_weights_fp32";
  return mode_ == QuantizationMode::WeightsOnly ? "int8_weights_fp32"
                                                : "int8_weights_dynamic_activations";
}

bool Model::is_moe_layer(size_t layer) const {
  return layer < layers_.size() && layers_[layer] != nullptr;
}

const uocr_moe_layer* Model::moe_layer(size_t layer) const {
  return is_moe_layer(layer) ? layers_[layer] : nullptr;
}

void Model::experts(CpuContext& cpu, size_t layer, const float* x, size_t T, float* y,
                    uint32_t flags) const {
  if (cpu.backend() != Backend::Gpu || !cpu.gpu())
    throw OcrError(ErrorKind::Unsupported, "the MoE layers of this library run on Backend::Gpu");
  experts(cpu.gpu(), layer, x, T, y, flags);
}

void Model::experts(uocr_gpu_ctx* gpu, size_t layer, const float* x, size_t T, float* y,
                    uint32_t flags) const {
  if (!is_moe_layer(layer)) throw OcrError(ErrorKind::Shape, "not a MoE decoder layer");
  check(uocr_moe_forward(gpu, layers_[layer], x, T, y, flags, nullptr));
}

}  // namespace uocr
