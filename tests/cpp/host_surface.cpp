// Exercises the C++ host surface (include/uocr.hpp) the way a C++ caller of
// the reference's types would, on the CPU: error kinds of CpuContext,
// Int8Matrix, ModelConfig, Checkpoint, QuantizedWeights and
// Model::load_with_quantization (which validates everything before it needs
// a GPU). Arguments: <overlay fixture dir> <model dir> <source sha256>.
#include <cmath>
#include <cstdio>
#include <cstdlib>
#include <functional>
#include <string>

#include "uocr.hpp"

using uocr::ErrorKind;

static int failures = 0;

static void expect_error(const char* what, ErrorKind kind, const std::function<void()>& f) {
  try {
    f();
    std::printf("FAIL %s: no error\n", what);
    failures++;
  } catch (const uocr::OcrError& e) {
    if (e.kind() != kind) {
      std::printf("FAIL %s: kind %d (%s)\n", what, e.status(), e.what());
      failures++;
    } else {
      std::printf("ok   %s: %s\n", what, e.what());
    }
  }
}

static void expect(const char* what, bool ok) {
  std::printf("%s %s\n", ok ? "ok  " : "FAIL", what);
  failures += ok ? 0 : 1;
}

int main(int argc, char** argv) {
  if (argc != 4) return 2;
  const std::string fixture = argv[1], model = argv[2], source_sha = argv[3];

  expect_error("CpuContext threads 0", ErrorKind::Resource,
               [] { uocr::CpuContext c(uocr::Backend::Auto, 0, 1024); });
  expect_error("CpuContext scratch 0", ErrorKind::Resource,
               [] { uocr::CpuContext c(uocr::Backend::Auto, 1, 0); });
  expect_error("CpuContext NEON on x86-64", ErrorKind::Unsupported,
               [] { uocr::CpuContext c(uocr::Backend::Neon, 1, 1024); });
  expect_error("CpuContext Accelerate off macOS", ErrorKind::Unsupported,
               [] { uocr::CpuContext c(uocr::Backend::Accelerate, 1, 1024); });
  uocr::CpuContext cpu(uocr::Backend::Auto, 8, 1 << 20);
  expect("CpuContext Auto", cpu.backend() == uocr::Backend::Auto && cpu.threads() == 8);

  expect("QuantizationMode names",
         std::string(uocr::to_string(uocr::QuantizationMode::WeightsOnly)) == "weights_only" &&
             std::string(uocr::to_string(uocr::QuantizationMode::DynamicActivations)) ==
                 "dynamic_activations");

  expect_error("Int8Matrix storage", ErrorKind::Shape,
               [] { uocr::Int8Matrix::from_parts(1, 2, {1}, {1.0f}); });
  expect_error("Int8Matrix NaN scale", ErrorKind::Numerical,
               [] { uocr::Int8Matrix::from_parts(1, 2, {1, -2}, {NAN}); });
  expect_error("Int8Matrix negative scale", ErrorKind::Numerical,
               [] { uocr::Int8Matrix::from_parts(1, 2, {1, -2}, {-1.0f}); });

  expect_error("ModelConfig model_type", ErrorKind::Unsupported, [] {
    uocr::ModelConfig::from_json(
        R"({"model_type":"x","hidden_size":64,"intermediate_size":1,"moe_intermediate_size":1,)"
        R"("num_hidden_layers":1,"num_attention_heads":4,"num_key_value_heads":4,)"
        R"("n_routed_experts":2,"n_shared_experts":1,"num_experts_per_tok":1,)"
        R"("first_k_dense_replace":0,"use_mla":false,"vocab_size":8})");
  });
  expect_error("ModelConfig missing field", ErrorKind::Json,
               [] { uocr::ModelConfig::from_json(R"({"model_type":"unlimited-ocr"})"); });
  expect_error("ModelConfig malformed", ErrorKind::Json,
               [] { uocr::ModelConfig::from_json("{"); });

  const auto source = uocr::Checkpoint::open(fixture + "/source.safetensors");
  expect("Checkpoint sha256", source->sha256() == source_sha);
  expect("Checkpoint names", source->names() == std::vector<std::string>{"lm_head.weight"});
  const uocr::WeightView w = source->tensor("lm_head.weight");
  expect("Checkpoint tensor", w.dtype == uocr::DType::F32 && w.size == 8 &&
                                  *w.shape == std::vector<size_t>{1, 2});
  expect_error("Checkpoint missing tensor", ErrorKind::Format,
               [&] { source->tensor("model.norm.weight"); });
  expect_error("Checkpoint missing file", ErrorKind::Io,
               [&] { uocr::Checkpoint::open(fixture + "/absent.safetensors"); });

  const auto q = uocr::QuantizedWeights::load(fixture + "/q.safetensors", *source);
  const uocr::Int8Matrix* m = q->get("lm_head.weight");
  expect("QuantizedWeights matrix", m && m->rows() == 1 && m->cols() == 2 &&
                                        m->weights()[0] == 1 && m->weights()[1] == -2 &&
                                        m->scales()[0] == 1.0f);
  expect("QuantizedWeights absent name", q->get("model.norm.weight") == nullptr);
  expect("overlay_eligible", uocr::overlay_eligible("model.layers.3.mlp.experts.7.up_proj.weight") &&
                                 !uocr::overlay_eligible("model.layers.3.mlp.gate.weight"));

  const std::string overlay = model + "/overlay.safetensors";
  expect_error("Model dynamic without overlay", ErrorKind::Format, [&] {
    uocr::Model::load_with_quantization(model, nullptr, uocr::QuantizationMode::DynamicActivations,
                                        cpu);
  });
  expect_error("Model on a CPU backend", ErrorKind::Unsupported, [&] {
    uocr::Model::load_with_quantization(model, &overlay, uocr::QuantizationMode::WeightsOnly, cpu);
  });
  const uocr::ModelConfig cfg = uocr::ModelConfig::load(model + "/config.json");
  expect("ModelConfig load", cfg.hidden_size == 64 && cfg.n_routed_experts == 8 &&
                                 cfg.num_experts_per_tok == 2 && cfg.norm_topk_prob);
  std::printf("%d failures\n", failures);
  return failures == 0 ? 0 : 1;
}
