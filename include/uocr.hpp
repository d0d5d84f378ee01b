// C++ host surface of the MI355X MoE path, mirroring the reference crate's
// public types for this path (same names, argument meaning and error
// behaviour) over the C ABI in uocr_moe.h:
//   OcrError                    src/error.rs:1-19
//   Backend / CpuContext        src/cpu/mod.rs:10-79 (plus Backend::Gpu)
//   QuantizationMode            src/cpu/quantized.rs:242-247
//   DType / WeightView /
//   Checkpoint                  src/checkpoint.rs:14-223 (safetensors)
//   Int8Matrix /
//   QuantizedWeights            src/cpu/quantized.rs:9-42, 239-369 (overlay)
//   ModelConfig                 src/model/config.rs:30-115
//   Model                       src/model/mod.rs:60-109, the MoE seam of
//                               Decoder (src/decoder/mod.rs:32-88, 124-220)
//                               and Decoder::logits (:367-379)
// Errors are thrown as OcrError; the C entry points return the same kinds as
// status codes. Vision, tokenizer, attention and generation are not part of
// this library: Model holds the MoE layers of the decoder and its
// vocabulary projection.
#pragma once

#include <cstddef>
#include <cstdint>
#include <map>
#include <memory>
#include <optional>
#include <stdexcept>
#include <string>
#include <vector>

#include "uocr_moe.h"

namespace uocr {

enum class ErrorKind { Io = 1, Json, Format, Shape, Unsupported, Resource, Numerical };

class OcrError : public std::runtime_error {
 public:
  OcrError(ErrorKind kind, const std::string& message);
  ErrorKind kind() const { return kind_; }
  int status() const { return static_cast<int>(kind_); }

 private:
  ErrorKind kind_;
};

enum class Backend { Scalar, Neon, Accelerate, Auto, Gpu };

enum class QuantizationMode { WeightsOnly, DynamicActivations };
// serde snake_case names: "weights_only", "dynamic_activations".
const char* to_string(QuantizationMode mode);

// CpuContext::new(backend, threads, scratch_limit): threads == 0 or
// scratch_limit == 0 -> Resource; Neon off AArch64 and Accelerate off macOS
// -> Unsupported. Backend::Gpu binds device 0 and reserves scratch_limit
// bytes of device scratch.
class CpuContext {
 public:
  CpuContext(Backend backend, size_t threads, size_t scratch_limit);
  ~CpuContext();
  CpuContext(const CpuContext&) = delete;
  CpuContext& operator=(const CpuContext&) = delete;

  Backend backend() const { return backend_; }
  size_t threads() const { return threads_; }
  size_t scratch_limit() const { return scratch_limit_; }
  uocr_gpu_ctx* gpu() const { return gpu_; }  // null unless Backend::Gpu

 private:
  Backend backend_;
  size_t threads_, scratch_limit_;
  uocr_gpu_ctx* gpu_ = nullptr;
};

enum class DType { BF16, F16, F32, I64, I8 };
size_t dtype_bytes(DType d);

struct WeightView {
  DType dtype;
  const std::vector<size_t>* shape;
  const uint8_t* bytes;
  size_t size;  // bytes
};

// Read-only, memory-mapped safetensors file.
class Checkpoint {
 public:
  static std::unique_ptr<Checkpoint> open(const std::string& path);
  ~Checkpoint();
  Checkpoint(const Checkpoint&) = delete;
  Checkpoint& operator=(const Checkpoint&) = delete;

  const std::map<std::string, std::string>& metadata() const { return metadata_; }
  // SHA-256 of the whole file, read through the file descriptor.
  std::string sha256() const;
  size_t file_bytes() const { return size_; }
  WeightView tensor(const std::string& name) const;  // missing -> Format
  bool contains(const std::string& name) const;
  std::vector<std::string> names() const;             // sorted

 private:
  Checkpoint() = default;
  struct Descriptor {
    DType dtype;
    std::vector<size_t> shape;
    size_t begin, end;
  };
  int fd_ = -1;
  const uint8_t* map_ = nullptr;
  size_t size_ = 0, data_start_ = 0;
  std::map<std::string, Descriptor> tensors_;
  std::map<std::string, std::string> metadata_;
};

class Int8Matrix {
 public:
  // Int8Matrix::from_parts: storage sizes -> Shape; non-finite or negative
  // scales -> Numerical.
  static Int8Matrix from_parts(size_t rows, size_t cols, std::vector<int8_t> weights,
                               std::vector<float> scales);
  size_t rows() const { return rows_; }
  size_t cols() const { return cols_; }
  const std::vector<int8_t>& weights() const { return weights_; }
  const std::vector<float>& scales() const { return scales_; }

 private:
  size_t rows_ = 0, cols_ = 0;
  std::vector<int8_t> weights_;
  std::vector<float> scales_;
};

// The "uocr-q8-block32-v1" overlay: a safetensors file of int8 matrices and
// their ".q8_scales", plus a JSON manifest beside it (same stem, ".json"),
// bound to the source checkpoint by SHA-256.
class QuantizedWeights {
 public:
  static std::unique_ptr<QuantizedWeights> load(const std::string& path, const Checkpoint& source);
  const Int8Matrix* get(const std::string& name) const;
  size_t size() const { return matrices_.size(); }

 private:
  std::map<std::string, Int8Matrix> matrices_;
};

// Matrices an overlay must hold (the router is never among them).
bool overlay_eligible(const std::string& name);

struct ModelConfig {
  std::string model_type;
  size_t hidden_size = 0, intermediate_size = 0, moe_intermediate_size = 0,
         num_hidden_layers = 0, num_attention_heads = 0, num_key_value_heads = 0,
         n_routed_experts = 0, n_shared_experts = 0, num_experts_per_tok = 0,
         first_k_dense_replace = 0, vocab_size = 0;
  bool use_mla = false;
  size_t sliding_window = 128;
  float rms_norm_eps = 1e-6f;
  float rope_theta = 10000.0f;
  bool norm_topk_prob = false;
  float routed_scaling_factor = 1.0f;
  size_t max_position_embeddings = 32768;
  std::string topk_method = "greedy", scoring_func = "softmax";
  size_t moe_layer_freq = 1;
  bool has_rope_scaling = false;
  bool attention_bias = false;

  static ModelConfig load(const std::string& path);
  static ModelConfig from_json(const std::string& json);
  uocr_moe_config moe() const;  // the MoE fields in the C ABI's form
};

// The MoE decoder layers of a model directory (config.json +
// model-00001-of-000001.safetensors), uploaded to the GPU once.
class Model {
 public:
  // Model::load_with_quantization: DynamicActivations without an overlay ->
  // Format; then config, checkpoint, the decoder shape rules, the overlay.
  // The context must use Backend::Gpu (else Unsupported).
  static std::unique_ptr<Model> load_with_quantization(const std::string& directory,
                                                       const std::string* overlay,
                                                       QuantizationMode mode, CpuContext& cpu);
  static std::unique_ptr<Model> load(const std::string& directory, CpuContext& cpu);
  // The same on an existing GPU context (the C entry point's form).
  static std::unique_ptr<Model> load_with_quantization(const std::string& directory,
                                                       const std::string* overlay,
                                                       QuantizationMode mode, uocr_gpu_ctx* gpu);
  ~Model();
  Model(const Model&) = delete;
  Model& operator=(const Model&) = delete;

  // "bf16_weights_fp32", "int8_weights_fp32" or
  // "int8_weights_dynamic_activations".
  const char* precision() const;
  const ModelConfig& config() const { return config_; }
  // Decoder layers with a MoE feed-forward (index >= first_k_dense_replace).
  bool is_moe_layer(size_t layer) const;
  const uocr_moe_layer* moe_layer(size_t layer) const;  // null for dense layers
  // Decoder::experts of decoder layer `layer`: y[T, H] from x[T, H], device
  // pointers, on the context's stream; synchronous.
  void experts(CpuContext& cpu, size_t layer, const float* x, size_t T, float* y,
               uint32_t flags = UOCR_FLAG_FP32_CLASS) const;
  void experts(uocr_gpu_ctx* gpu, size_t layer, const float* x, size_t T, float* y,
               uint32_t flags = UOCR_FLAG_FP32_CLASS) const;
  // Decoder::logits (src/decoder/mod.rs:367-379): logits[vocab_size] of the
  // last row of hidden[T, H] (device pointers); synchronous. T == 0 ->
  // Shape.
  void logits(CpuContext& cpu, const float* hidden, size_t T, float* logits) const;
  void logits(uocr_gpu_ctx* gpu, const float* hidden, size_t T, float* logits) const;
  const uocr_lm_head* lm_head() const { return lm_head_; }

 private:
  Model() = default;
  ModelConfig config_;
  bool quantized_ = false;
  QuantizationMode mode_ = QuantizationMode::WeightsOnly;
  std::vector<uocr_moe_layer*> layers_;  // per decoder layer, null if dense
  uocr_lm_head* lm_head_ = nullptr;       // final norm + lm_head.weight
};

}  // namespace uocr
