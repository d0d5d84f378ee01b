// Minimal JSON reader for the host side: safetensors headers, overlay
// manifests and config.json. Objects keep their key order; numbers keep
// their source text so integers up to 2^64 - 1 convert exactly.
#pragma once

#include <cstdint>
#include <string>
#include <utility>
#include <vector>

namespace uocr::host {

struct Json {
  enum Kind { Null, Bool, Number, String, Array, Object } kind = Null;
  bool b = false;
  std::string text;  // String: the decoded value; Number: the literal
  std::vector<Json> items;
  std::vector<std::pair<std::string, Json>> members;

  const Json* find(const std::string& key) const;
  bool is_uint() const;       // a non-negative integer literal
  uint64_t as_uint() const;   // exact; valid when is_uint()
  double as_double() const;   // valid for numbers
};

// Parses one JSON document (surrounding whitespace allowed). Returns false
// and sets `error` on malformed input.
bool parse_json(const char* data, size_t size, Json& out, std::string& error);

}  // namespace uocr::host
