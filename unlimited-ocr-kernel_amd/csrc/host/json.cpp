#include "json.hpp"

#include <cerrno>
#include <cstdlib>

namespace uocr::host {

namespace {

struct Parser {
  const char* p;
  const char* end;
  std::string error;
  int depth = 0;

  void ws() {
    while (p < end && (*p == ' ' || *p == '\t' || *p == '\n' || *p == '\r')) p++;
  }
  bool fail(const char* msg) {
    if (error.empty()) error = msg;
    return false;
  }
  bool literal(const char* word) {
    for (const char* w = word; *w; w++, p++)
      if (p >= end || *p != *w) return fail("invalid literal");
    return true;
  }
  static void put_utf8(std::string& s, uint32_t c) {
    if (c < 0x80) {
      s += (char)c;
    } else if (c < 0x800) {
      s += (char)(0xC0 | (c >> 6));
      s += (char)(0x80 | (c & 0x3F));
    } else if (c < 0x10000) {
      s += (char)(0xE0 | (c >> 12));
      s += (char)(0x80 | ((c >> 6) & 0x3F));
      s += (char)(0x80 | (c & 0x3F));
    } else {
      s += (char)(0xF0 | (c >> 18));
      s += (char)(0x80 | ((c >> 12) & 0x3F));
      s += (char)(0x80 | ((c >> 6) & 0x3F));
      s += (char)(0x80 | (c & 0x3F));
    }
  }
  bool hex4(uint32_t& v) {
    v = 0;
    for (int i = 0; i < 4; i++, p++) {
      if (p >= end) return fail("truncated escape");
      const char c = *p;
      v <<= 4;
      if (c >= '0' && c <= '9') v |= (uint32_t)(c - '0');
      else if (c >= 'a' && c <= 'f') v |= (uint32_t)(c - 'a' + 10);
      else if (c >= 'A' && c <= 'F') v |= (uint32_t)(c - 'A' + 10);
      else return fail("invalid escape");
    }
    return true;
  }
  bool string(std::string& s) {
    if (p >= end || *p != '"') return fail("expected string");
    p++;
    while (true) {
      if (p >= end) return fail("unterminated string");
      const char c = *p++;
      if (c == '"') return true;
      if ((unsigned char)c < 0x20) return fail("control character in string");
      if (c != '\\') {
        s += c;
        continue;
      }
      if (p >= end) return fail("truncated escape");
      const char e = *p++;
      switch (e) {
        case '"': s += '"'; break;
        case '\\': s += '\\'; break;
        case '/': s += '/'; break;
        case 'b': s += '\b'; break;
        case 'f': s += '\f'; break;
        case 'n': s += '\n'; break;
        case 'r': s += '\r'; break;
        case 't': s += '\t'; break;
        case 'u': {
          uint32_t c1;
          if (!hex4(c1)) return false;
          if (c1 >= 0xD800 && c1 < 0xDC00) {
            uint32_t c2;
            if (p + 1 >= end || p[0] != '\\' || p[1] != 'u') return fail("lone surrogate");
            p += 2;
            if (!hex4(c2) || c2 < 0xDC00 || c2 >= 0xE000) return fail("invalid surrogate pair");
            c1 = 0x10000 + ((c1 - 0xD800) << 10) + (c2 - 0xDC00);
          } else if (c1 >= 0xDC00 && c1 < 0xE000) {
            return fail("lone surrogate");
          }
          put_utf8(s, c1);
          break;
        }
        default: return fail("invalid escape");
      }
    }
  }
  bool number(Json& v) {
    const char* start = p;
    if (p < end && *p == '-') p++;
    if (p >= end) return fail("invalid number");
    if (*p == '0') {
      p++;
    } else if (*p >= '1' && *p <= '9') {
      while (p < end && *p >= '0' && *p <= '9') p++;
    } else {
      return fail("invalid number");
    }
    if (p < end && *p == '.') {
      p++;
      if (p >= end || *p < '0' || *p > '9') return fail("invalid number");
      while (p < end && *p >= '0' && *p <= '9') p++;
    }
    if (p < end && (*p == 'e' || *p == 'E')) {
      p++;
      if (p < end && (*p == '+' || *p == '-')) p++;
      if (p >= end || *p < '0' || *p > '9') return fail("invalid number");
      while (p < end && *p >= '0' && *p <= '9') p++;
    }
    v.kind = Json::Number;
    v.text.assign(start, p);
    return true;
  }
  bool value(Json& v) {
    if (++depth > 256) return fail("nesting too deep");
    ws();
    if (p >= end) return fail("unexpected end");
    bool ok;
    switch (*p) {
      case '{': ok = object(v); break;
      case '[': ok = array(v); break;
      case '"': v.kind = Json::String; ok = string(v.text); break;
      case 't': v.kind = Json::Bool; v.b = true; ok = literal("true"); break;
      case 'f': v.kind = Json::Bool; v.b = false; ok = literal("false"); break;
      case 'n': v.kind = Json::Null; ok = literal("null"); break;
      default: ok = number(v); break;
    }
    depth--;
    return ok;
  }
  bool array(Json& v) {
    v.kind = Json::Array;
    p++;
    ws();
    if (p < end && *p == ']') {
      p++;
      return true;
    }
    while (true) {
      v.items.emplace_back();
      if (!value(v.items.back())) return false;
      ws();
      if (p >= end) return fail("unterminated array");
      if (*p == ',') {
        p++;
        continue;
      }
      if (*p == ']') {
        p++;
        return true;
      }
      return fail("expected , or ]");
    }
  }
  bool object(Json& v) {
    v.kind = Json::Object;
    p++;
    ws();
    if (p < end && *p == '}') {
      p++;
      return true;
    }
    while (true) {
      ws();
      std::string key;
      if (!string(key)) return false;
      ws();
      if (p >= end || *p != ':') return fail("expected :");
      p++;
      v.members.emplace_back(std::move(key), Json());
      if (!value(v.members.back().second)) return false;
      ws();
      if (p >= end) return fail("unterminated object");
      if (*p == ',') {
        p++;
        continue;
      }
      if (*p == '}') {
        p++;
        return true;
      }
      return fail("expected , or }");
    }
  }
};

}  // namespace

const Json* Json::find(const std::string& key) const {
  // Duplicate keys: the last one wins, as in a map built by insertion.
  const Json* hit = nullptr;
  for (const auto& m : members)
    if (m.first == key) hit = &m.second;
  return hit;
}

bool Json::is_uint() const {
  if (kind != Number || text.empty()) return false;
  for (char c : text)
    if (c < '0' || c > '9') return false;
  if (text.size() > 1 && text[0] == '0') return false;
  errno = 0;
  (void)std::strtoull(text.c_str(), nullptr, 10);
  return errno == 0;
}

uint64_t Json::as_uint() const { return std::strtoull(text.c_str(), nullptr, 10); }

double Json::as_double() const { return std::strtod(text.c_str(), nullptr); }

bool parse_json(const char* data, size_t size, Json& out, std::string& error) {
  Parser ps{data, data + size, {}};
  out = Json();
  if (!ps.value(out)) {
    error = ps.error;
    return false;
  }
  ps.ws();
  if (ps.p != ps.end) {
    error = "trailing characters";
    return false;
  }
  return true;
}

}  // namespace uocr::host
