// SHA-256 (FIPS 180-4) for the overlay's source/output checksums.
#pragma once

#include <cstddef>
#include <cstdint>
#include <string>

namespace uocr::host {

class Sha256 {
 public:
  Sha256();
  void update(const void* data, size_t size);
  // Lowercase hexadecimal digest; the object is spent afterwards.
  std::string hex();

 private:
  void block(const uint8_t* p);
  uint32_t h_[8];
  uint8_t buf_[64];
  size_t fill_ = 0;
  uint64_t total_ = 0;
};

}  // namespace uocr::host
