// Safetensors checkpoint (src/checkpoint.rs:114-223): header length, JSON
// header of tensor descriptors, and a payload that the tensors must cover
// exactly, without gaps or overlaps.
#include <fcntl.h>
#include <sys/mman.h>
#include <sys/stat.h>
#include <unistd.h>

#include <algorithm>
#include <cerrno>
#include <cstring>

#include "../../../include/uocr.hpp"
#include "json.hpp"
#include "sha256.hpp"

namespace uocr {

size_t dtype_bytes(DType d) {
  switch (d) {
    case DType::BF16:
    case DType::F16: return 2;
    case DType::F32: return 4;
    case DType::I64: return 8;
    case DType::I8: return 1;
  }
  return 0;
}

namespace {

[[noreturn]] void io_error(const std::string& what) {
  throw OcrError(ErrorKind::Io, what + ": " + std::strerror(errno));
}

bool parse_dtype(const std::string& s, DType& d) {
  if (s == "BF16") d = DType::BF16;
  else if (s == "F16") d = DType::F16;
  else if (s == "F32") d = DType::F32;
  else if (s == "I64") d = DType::I64;
  else if (s == "I8") d = DType::I8;
  else return false;
  return true;
}

bool checked_mul(size_t a, size_t b, size_t& out) { return !__builtin_mul_overflow(a, b, &out); }

}  // namespace

std::unique_ptr<Checkpoint> Checkpoint::open(const std::string& path) {
  std::unique_ptr<Checkpoint> ck(new Checkpoint());
  ck->fd_ = ::open(path.c_str(), O_RDONLY | O_CLOEXEC);
  if (ck->fd_ < 0) io_error(path);
  struct stat st;
  if (fstat(ck->fd_, &st) != 0) io_error(path);
  if (st.st_size < 8) throw OcrError(ErrorKind::Format, "missing header length");
  ck->size_ = (size_t)st.st_size;
  void* m = mmap(nullptr, ck->size_, PROT_READ, MAP_PRIVATE, ck->fd_, 0);
  if (m == MAP_FAILED) io_error(path);
  ck->map_ = static_cast<const uint8_t*>(m);

  uint64_t header_len = 0;
  for (int i = 7; i >= 0; i--) header_len = (header_len << 8) | ck->map_[i];
  if (header_len > 100000000ull) throw OcrError(ErrorKind::Format, "header exceeds 100 MB");
  const size_t data_start = 8 + (size_t)header_len;
  if (data_start > ck->size_) throw OcrError(ErrorKind::Format, "truncated header");
  ck->data_start_ = data_start;

  host::Json header;
  std::string err;
  if (!host::parse_json(reinterpret_cast<const char*>(ck->map_ + 8), (size_t)header_len, header,
                        err))
    throw OcrError(ErrorKind::Json, "safetensors header: " + err);
  if (header.kind != host::Json::Object)
    throw OcrError(ErrorKind::Json, "safetensors header is not an object");
  const size_t payload = ck->size_ - data_start;
  for (const auto& [name, value] : header.members) {
    if (name == "__metadata__") {
      if (value.kind != host::Json::Object)
        throw OcrError(ErrorKind::Json, "__metadata__ is not a string map");
      std::map<std::string, std::string> md;
      for (const auto& [k, v] : value.members) {
        if (v.kind != host::Json::String)
          throw OcrError(ErrorKind::Json, "__metadata__ value is not a string");
        md[k] = v.text;
      }
      ck->metadata_ = std::move(md);
      continue;
    }
    const host::Json* dt = value.find("dtype");
    const host::Json* sh = value.find("shape");
    const host::Json* off = value.find("data_offsets");
    Descriptor d;
    if (value.kind != host::Json::Object || !dt || dt->kind != host::Json::String ||
        !parse_dtype(dt->text, d.dtype) || !sh || sh->kind != host::Json::Array || !off ||
        off->kind != host::Json::Array || off->items.size() != 2)
      throw OcrError(ErrorKind::Json, "invalid tensor descriptor: " + name);
    for (const auto& dim : sh->items) {
      if (!dim.is_uint()) throw OcrError(ErrorKind::Json, "invalid tensor shape: " + name);
      d.shape.push_back((size_t)dim.as_uint());
    }
    if (!off->items[0].is_uint() || !off->items[1].is_uint())
      throw OcrError(ErrorKind::Json, "invalid tensor offsets: " + name);
    d.begin = (size_t)off->items[0].as_uint();
    d.end = (size_t)off->items[1].as_uint();
    size_t count = 1;
    for (size_t dim : d.shape)
      if (!checked_mul(count, dim, count))
        throw OcrError(ErrorKind::Format, "tensor size overflow: " + name);
    if (!checked_mul(count, dtype_bytes(d.dtype), count))
      throw OcrError(ErrorKind::Format, "tensor size overflow: " + name);
    if (d.end < d.begin || d.end - d.begin != count || d.end > payload)
      throw OcrError(ErrorKind::Format, "invalid tensor offsets: " + name);
    ck->tensors_[name] = std::move(d);
  }
  std::vector<std::pair<size_t, size_t>> spans;
  for (const auto& kv : ck->tensors_) spans.emplace_back(kv.second.begin, kv.second.end);
  std::sort(spans.begin(), spans.end());
  size_t cursor = 0;
  for (const auto& [b, e] : spans) {
    if (b != cursor) throw OcrError(ErrorKind::Format, "payload gaps or overlapping tensors");
    cursor = e;
  }
  if (cursor != payload) throw OcrError(ErrorKind::Format, "unclaimed trailing payload");
  return ck;
}

Checkpoint::~Checkpoint() {
  if (map_) munmap(const_cast<uint8_t*>(map_), size_);
  if (fd_ >= 0) ::close(fd_);
}

std::string Checkpoint::sha256() const {
  // Hash through the descriptor (the same file as the mapping) without
  // faulting the mapping in; the size must not have changed.
  host::Sha256 h;
  std::vector<uint8_t> buf(1 << 20);
  size_t at = 0;
  while (at < size_) {
    const size_t want = std::min(buf.size(), size_ - at);
    const ssize_t got = pread(fd_, buf.data(), want, (off_t)at);
    if (got < 0) io_error("checkpoint read");
    if (got == 0) throw OcrError(ErrorKind::Format, "checkpoint file size changed");
    h.update(buf.data(), (size_t)got);
    at += (size_t)got;
  }
  uint8_t extra;
  const ssize_t more = pread(fd_, &extra, 1, (off_t)size_);
  if (more < 0) io_error("checkpoint read");
  if (more != 0) throw OcrError(ErrorKind::Format, "checkpoint file size changed");
  return h.hex();
}

WeightView Checkpoint::tensor(const std::string& name) const {
  const auto it = tensors_.find(name);
  if (it == tensors_.end()) throw OcrError(ErrorKind::Format, "missing tensor: " + name);
  const Descriptor& d = it->second;
  return WeightView{d.dtype, &d.shape, map_ + data_start_ + d.begin, d.end - d.begin};
}

bool Checkpoint::contains(const std::string& name) const { return tensors_.count(name) != 0; }

std::vector<std::string> Checkpoint::names() const {
  std::vector<std::string> out;
  for (const auto& kv : tensors_) out.push_back(kv.first);
  return out;
}

}  // namespace uocr
