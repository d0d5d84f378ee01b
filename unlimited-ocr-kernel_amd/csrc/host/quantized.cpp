// The INT8 block-32 overlay (src/cpu/quantized.rs:9-42, 239-369): manifest,
// metadata and SHA-256 binding to the source checkpoint, the eligible matrix
// set, and per-matrix storage rules.
#include <cmath>
#include <cstring>
#include <fstream>
#include <sstream>

#include "../../../include/uocr.hpp"
#include "json.hpp"

namespace uocr {

namespace {

constexpr const char* kFormat = "uocr-q8-block32-v1";
constexpr const char* kScaleSuffix = ".q8_scales";
constexpr size_t kBlock = 32;

bool all_digits(const std::string& s) {
  if (s.empty()) return false;
  for (char c : s)
    if (c < '0' || c > '9') return false;
  return true;
}

bool strip_prefix(std::string& s, const std::string& prefix) {
  if (s.compare(0, prefix.size(), prefix) != 0) return false;
  s.erase(0, prefix.size());
  return true;
}

// Path::with_extension("json"): replace the file name's last extension.
std::string with_json_extension(const std::string& path) {
  const size_t slash = path.find_last_of('/');
  const size_t name = slash == std::string::npos ? 0 : slash + 1;
  const size_t dot = path.find_last_of('.');
  if (dot == std::string::npos || dot <= name) return path + ".json";
  return path.substr(0, dot) + ".json";
}

std::string read_file(const std::string& path) {
  std::ifstream in(path, std::ios::binary);
  if (!in) throw OcrError(ErrorKind::Io, "cannot read " + path);
  std::ostringstream ss;
  ss << in.rdbuf();
  return ss.str();
}

}  // namespace

bool overlay_eligible(const std::string& name) {
  if (name == "lm_head.weight") return true;
  std::string rest = name;
  if (!strip_prefix(rest, "model.layers.")) return false;
  const size_t dot = rest.find('.');
  if (dot == std::string::npos || !all_digits(rest.substr(0, dot))) return false;
  rest.erase(0, dot + 1);
  if (strip_prefix(rest, "self_attn."))
    return rest == "q_proj.weight" || rest == "k_proj.weight" || rest == "v_proj.weight" ||
           rest == "o_proj.weight";
  if (!strip_prefix(rest, "mlp.")) return false;
  if (!strip_prefix(rest, "shared_experts.") && strip_prefix(rest, "experts.")) {
    const size_t d = rest.find('.');
    if (d == std::string::npos || !all_digits(rest.substr(0, d))) return false;
    rest.erase(0, d + 1);
  }
  return rest == "gate_proj.weight" || rest == "up_proj.weight" || rest == "down_proj.weight";
}

Int8Matrix Int8Matrix::from_parts(size_t rows, size_t cols, std::vector<int8_t> weights,
                                  std::vector<float> scales) {
  const size_t blocks = (cols + kBlock - 1) / kBlock;
  if (rows == 0 || cols == 0 || weights.size() / cols != rows || weights.size() % cols != 0 ||
      scales.size() != rows * blocks)
    throw OcrError(ErrorKind::Shape, "INT8 matrix storage");
  for (float s : scales)
    if (!std::isfinite(s) || s < 0.0f)
      throw OcrError(ErrorKind::Numerical, "INT8 scales must be finite and nonnegative");
  Int8Matrix m;
  m.rows_ = rows;
  m.cols_ = cols;
  m.weights_ = std::move(weights);
  m.scales_ = std::move(scales);
  return m;
}

std::unique_ptr<QuantizedWeights> QuantizedWeights::load(const std::string& path,
                                                         const Checkpoint& source) {
  const std::string manifest_text = read_file(with_json_extension(path));
  host::Json manifest;
  std::string err;
  if (!host::parse_json(manifest_text.data(), manifest_text.size(), manifest, err))
    throw OcrError(ErrorKind::Json, "overlay manifest: " + err);
  auto field = [&](const char* key) -> const host::Json& {
    const host::Json* v = manifest.kind == host::Json::Object ? manifest.find(key) : nullptr;
    if (!v) throw OcrError(ErrorKind::Json, std::string("overlay manifest: missing ") + key);
    return *v;
  };
  auto uint_field = [&](const char* key, uint64_t max) {
    const host::Json& v = field(key);
    if (!v.is_uint() || v.as_uint() > max)
      throw OcrError(ErrorKind::Json, std::string("overlay manifest: invalid ") + key);
    return v.as_uint();
  };
  auto string_field = [&](const char* key) {
    const host::Json& v = field(key);
    if (v.kind != host::Json::String)
      throw OcrError(ErrorKind::Json, std::string("overlay manifest: invalid ") + key);
    return v.text;
  };
  const uint64_t schema_version = uint_field("schema_version", 0xffffffffull);
  const std::string format = string_field("format");
  const uint64_t block_size = uint_field("block_size", ~0ull);
  const std::string source_sha256 = string_field("source_sha256");
  const std::string output_sha256 = string_field("output_sha256");
  const uint64_t matrix_count = uint_field("matrix_count", ~0ull);
  const uint64_t bytes = uint_field("bytes", ~0ull);

  const std::unique_ptr<Checkpoint> overlay = Checkpoint::open(path);
  const auto& md = overlay->metadata();
  auto meta_is = [&](const char* key, const std::string& want) {
    const auto it = md.find(key);
    return it != md.end() && it->second == want;
  };
  if (schema_version != 1 || format != kFormat || block_size != kBlock ||
      !meta_is("format", kFormat) || !meta_is("block_size", "32") ||
      !meta_is("source_sha256", source_sha256) || overlay->file_bytes() != bytes)
    throw OcrError(ErrorKind::Format, "INT8 overlay version or metadata mismatch");
  // The large source first, so the overlay is the most recently read file.
  if (source.sha256() != source_sha256 || overlay->sha256() != output_sha256)
    throw OcrError(ErrorKind::Format, "INT8 checksum or source model mismatch");

  std::vector<std::string> expected;
  for (const std::string& n : source.names())
    if (overlay_eligible(n)) expected.push_back(n);
  if (expected.empty() || expected.size() != matrix_count ||
      overlay->names().size() != expected.size() * 2)
    throw OcrError(ErrorKind::Format, "INT8 matrix set mismatch");

  std::unique_ptr<QuantizedWeights> q(new QuantizedWeights());
  for (const std::string& name : expected) {
    const WeightView original = source.tensor(name);
    const WeightView weight = overlay->tensor(name);
    const WeightView scales = overlay->tensor(name + kScaleSuffix);
    bool ok = weight.dtype == DType::I8 && weight.shape->size() == 2 &&
              *weight.shape == *original.shape &&
              (original.dtype == DType::BF16 || original.dtype == DType::F16 ||
               original.dtype == DType::F32) &&
              scales.dtype == DType::F32;
    if (ok) {
      const size_t rows = (*weight.shape)[0], cols = (*weight.shape)[1];
      ok = scales.shape->size() == 2 && (*scales.shape)[0] == rows &&
           (*scales.shape)[1] == (cols + kBlock - 1) / kBlock &&
           std::memchr(weight.bytes, 128, weight.size) == nullptr;
    }
    if (!ok) throw OcrError(ErrorKind::Format, "invalid INT8 matrix " + name);
    std::vector<int8_t> w(weight.size);
    std::memcpy(w.data(), weight.bytes, weight.size);
    std::vector<float> s(scales.size / 4);
    std::memcpy(s.data(), scales.bytes, scales.size);  // little-endian f32
    q->matrices_.emplace(name, Int8Matrix::from_parts((*weight.shape)[0], (*weight.shape)[1],
                                                      std::move(w), std::move(s)));
  }
  return q;
}

const Int8Matrix* QuantizedWeights::get(const std::string& name) const {
  const auto it = matrices_.find(name);
  return it == matrices_.end() ? nullptr : &it->second;
}

}  // namespace uocr
