// JSON for the host code (internal header): a value tree with a complete
// recursive-descent reader (every string escape, numbers kept as their
// literal, nesting bounded) and a writer that emits the layout Python's
// json.dumps(indent=2) gives (two-space indent, ", " free separators, ASCII
// output with \uXXXX escapes).
#pragma once

#include <cstdint>
#include <cstdio>
#include <cstdlib>
#include <filesystem>
#include <fstream>
#include <iterator>
#include <stdexcept>
#include <string>
#include <string_view>
#include <utility>
#include <vector>

namespace rtxllm {
namespace json {

// ---- JSON value tree --------------------------------------------------------------

struct Json {
  enum Kind { Null, Bool, Number, String, Array, Object } kind = Null;
  bool b = false;
  std::string text;  // String: the value; Number: its literal
  std::vector<Json> items;
  std::vector<std::pair<std::string, Json>> members;

  const Json* find(std::string_view key) const {
    if (kind != Object) return nullptr;
    for (const auto& m : members)
      if (m.first == key) return &m.second;
    return nullptr;
  }
};

class Reader {
 public:
  explicit Reader(std::string_view s) : s_(s) {}
  Json document() {
    Json v = value(0);
    ws();
    if (i_ != s_.size()) error("trailing characters");
    return v;
  }

 private:
  std::string_view s_;
  std::size_t i_ = 0;
  static constexpr int kMaxDepth = 256;

  [[noreturn]] void error(const char* what) const {
    throw std::runtime_error(std::string("manifest JSON: ") + what + " at byte " + std::to_string(i_));
  }
  void ws() {
    while (i_ < s_.size() && (s_[i_] == ' ' || s_[i_] == '\t' || s_[i_] == '\n' || s_[i_] == '\r')) ++i_;
  }
  bool take(char c) {
    ws();
    if (i_ < s_.size() && s_[i_] == c) {
      ++i_;
      return true;
    }
    return false;
  }
  void expect(char c) {
    if (!take(c)) error("unexpected character");
  }
  bool literal(std::string_view word) {
    if (s_.compare(i_, word.size(), word) != 0) return false;
    i_ += word.size();
    return true;
  }
  static void utf8(std::string& out, std::uint32_t cp) {
    if (cp < 0x80) {
      out += static_cast<char>(cp);
    } else if (cp < 0x800) {
      out += static_cast<char>(0xC0 | (cp >> 6));
      out += static_cast<char>(0x80 | (cp & 0x3F));
    } else if (cp < 0x10000) {
      out += static_cast<char>(0xE0 | (cp >> 12));
      out += static_cast<char>(0x80 | ((cp >> 6) & 0x3F));
      out += static_cast<char>(0x80 | (cp & 0x3F));
    } else {
      out += static_cast<char>(0xF0 | (cp >> 18));
      out += static_cast<char>(0x80 | ((cp >> 12) & 0x3F));
      out += static_cast<char>(0x80 | ((cp >> 6) & 0x3F));
      out += static_cast<char>(0x80 | (cp & 0x3F));
    }
  }
  std::uint32_t hex4() {
    if (i_ + 4 > s_.size()) error("short \\u escape");
    std::uint32_t v = 0;
    for (int k = 0; k < 4; ++k) {
      const char c = s_[i_++];
      v <<= 4;
      if (c >= '0' && c <= '9') v |= static_cast<std::uint32_t>(c - '0');
      else if (c >= 'a' && c <= 'f') v |= static_cast<std::uint32_t>(c - 'a' + 10);
      else if (c >= 'A' && c <= 'F') v |= static_cast<std::uint32_t>(c - 'A' + 10);
      else error("bad \\u escape");
    }
    return v;
  }
  std::string string() {
    expect('"');
    std::string out;
    while (true) {
      if (i_ >= s_.size()) error("unterminated string");
      const char c = s_[i_++];
      if (c == '"') return out;
      if (static_cast<unsigned char>(c) < 0x20) error("control character in string");
      if (c != '\\') {
        out += c;
        continue;
      }
      if (i_ >= s_.size()) error("unterminated escape");
      const char e = s_[i_++];
      switch (e) {
        case '"': case '\\': case '/': out += e; break;
        case 'b': out += '\b'; break;
        case 'f': out += '\f'; break;
        case 'n': out += '\n'; break;
        case 'r': out += '\r'; break;
        case 't': out += '\t'; break;
        case 'u': {
          std::uint32_t cp = hex4();
          if (cp >= 0xD800 && cp < 0xDC00) {  // surrogate pair
            if (!literal("\\u")) error("lone surrogate");
            const std::uint32_t lo = hex4();
            if (lo < 0xDC00 || lo >= 0xE000) error("bad surrogate pair");
            cp = 0x10000 + ((cp - 0xD800) << 10) + (lo - 0xDC00);
          }
          utf8(out, cp);
          break;
        }
        default: error("unsupported escape");
      }
    }
  }
  std::string number() {
    const std::size_t b = i_;
    if (i_ < s_.size() && s_[i_] == '-') ++i_;
    auto digits = [&] {
      const std::size_t d = i_;
      while (i_ < s_.size() && s_[i_] >= '0' && s_[i_] <= '9') ++i_;
      return i_ > d;
    };
    if (!digits()) error("bad number");
    if (i_ < s_.size() && s_[i_] == '.') {
      ++i_;
      if (!digits()) error("bad number");
    }
    if (i_ < s_.size() && (s_[i_] == 'e' || s_[i_] == 'E')) {
      ++i_;
      if (i_ < s_.size() && (s_[i_] == '+' || s_[i_] == '-')) ++i_;
      if (!digits()) error("bad number");
    }
    return std::string(s_.substr(b, i_ - b));
  }
  Json value(int depth) {
    if (depth > kMaxDepth) error("nesting too deep");
    ws();
    if (i_ >= s_.size()) error("unexpected end");
    Json v;
    const char c = s_[i_];
    if (c == '{') {
      ++i_;
      v.kind = Json::Object;
      if (take('}')) return v;
      do {
        ws();
        std::string key = string();
        expect(':');
        v.members.emplace_back(std::move(key), value(depth + 1));
      } while (take(','));
      expect('}');
    } else if (c == '[') {
      ++i_;
      v.kind = Json::Array;
      if (take(']')) return v;
      do v.items.push_back(value(depth + 1));
      while (take(','));
      expect(']');
    } else if (c == '"') {
      v.kind = Json::String;
      v.text = string();
    } else if (literal("true")) {
      v.kind = Json::Bool, v.b = true;
    } else if (literal("false")) {
      v.kind = Json::Bool;
    } else if (literal("null")) {
      v.kind = Json::Null;
    } else {
      v.kind = Json::Number;
      v.text = number();
    }
    return v;
  }
};

inline std::string read_text(const std::filesystem::path& path, const char* what) {
  std::ifstream in(path, std::ios::binary);
  if (!in) throw std::runtime_error(std::string("failed to open ") + what + ": " + path.string());
  std::string text((std::istreambuf_iterator<char>(in)), std::istreambuf_iterator<char>());
  if (in.bad()) throw std::runtime_error(std::string("failed to read ") + what + ": " + path.string());
  return text;
}

// A non-negative integer literal (no sign, fraction or exponent).
inline bool as_u64(const Json& v, std::uint64_t& out) {
  if (v.kind != Json::Number || v.text.empty()) return false;
  std::uint64_t x = 0;
  for (const char c : v.text) {
    if (c < '0' || c > '9') return false;
    const std::uint64_t d = static_cast<std::uint64_t>(c - '0');
    if (x > (UINT64_MAX - d) / 10u) return false;
    x = x * 10u + d;
  }
  out = x;
  return true;
}

// ---- building and writing ------------------------------------------------------------

inline Json null_value() { return Json{}; }
inline Json boolean(bool b) {
  Json v;
  v.kind = Json::Bool, v.b = b;
  return v;
}
inline Json string(std::string s) {
  Json v;
  v.kind = Json::String, v.text = std::move(s);
  return v;
}
inline Json integer(std::uint64_t x) {
  Json v;
  v.kind = Json::Number, v.text = std::to_string(x);
  return v;
}
inline Json integer_signed(std::int64_t x) {
  Json v;
  v.kind = Json::Number, v.text = std::to_string(x);
  return v;
}
// A finite double as Python's repr writes it: the shortest digits that read
// back to the same value, positional for decimal exponents -4..15 (with ".0"
// when integral), else d.ddde+XX.
inline Json real(double x) {
  if (!(x == x) || x - x != 0.0) throw std::runtime_error("JSON number is not finite");
  char sci[40];
  int prec = 0;
  for (prec = 1; prec <= 17; ++prec) {  // shortest %.{prec-1}e that round-trips
    std::snprintf(sci, sizeof sci, "%.*e", prec - 1, x);
    if (std::strtod(sci, nullptr) == x) break;
  }
  // split "[-]d.ddde[+-]XX" into sign, digits and exponent
  std::string t(sci);
  const bool neg = t[0] == '-';
  if (neg) t.erase(0, 1);
  const std::size_t e = t.find('e');
  const int exp10 = std::atoi(t.c_str() + e + 1);
  std::string digits = t.substr(0, e);
  if (digits.size() > 1) digits.erase(1, 1);  // drop the point
  while (digits.size() > 1 && digits.back() == '0') digits.pop_back();
  std::string out = neg ? "-" : "";
  if (exp10 >= -4 && exp10 < 16) {
    if (exp10 < 0) {
      out += "0." + std::string(static_cast<std::size_t>(-exp10 - 1), '0') + digits;
    } else if (static_cast<int>(digits.size()) <= exp10 + 1) {
      out += digits + std::string(static_cast<std::size_t>(exp10 + 1) - digits.size(), '0') + ".0";
    } else {
      out += digits.substr(0, static_cast<std::size_t>(exp10 + 1)) + "." +
             digits.substr(static_cast<std::size_t>(exp10 + 1));
    }
  } else {
    out += digits.substr(0, 1);
    if (digits.size() > 1) out += "." + digits.substr(1);
    char ex[16];
    std::snprintf(ex, sizeof ex, "e%c%02d", exp10 < 0 ? '-' : '+', exp10 < 0 ? -exp10 : exp10);
    out += ex;
  }
  Json v;
  v.kind = Json::Number, v.text = out;
  return v;
}
inline Json array() {
  Json v;
  v.kind = Json::Array;
  return v;
}
inline Json object() {
  Json v;
  v.kind = Json::Object;
  return v;
}
// Appends a member (keys keep their insertion order).
inline Json& set(Json& obj, std::string key, Json value) {
  obj.members.emplace_back(std::move(key), std::move(value));
  return obj;
}

inline void write_string(std::string& out, const std::string& s) {
  out += '"';
  auto u = [&](std::uint32_t cp) {
    char b[16];
    std::snprintf(b, sizeof b, "\\u%04x", cp);
    out += b;
  };
  for (std::size_t i = 0; i < s.size();) {
    const unsigned char c = static_cast<unsigned char>(s[i]);
    if (c < 0x80) {
      ++i;
      switch (c) {
        case '"': out += "\\\""; break;
        case '\\': out += "\\\\"; break;
        case '\n': out += "\\n"; break;
        case '\r': out += "\\r"; break;
        case '\t': out += "\\t"; break;
        case '\b': out += "\\b"; break;
        case '\f': out += "\\f"; break;
        default:
          if (c < 0x20) u(c);
          else out += static_cast<char>(c);
      }
      continue;
    }
    // UTF-8 sequence -> code point -> \uXXXX (a surrogate pair above U+FFFF);
    // a malformed byte is written as U+FFFD
    int n = c >= 0xF0 ? 3 : c >= 0xE0 ? 2 : c >= 0xC0 ? 1 : -1;
    std::uint32_t cp = n == 3 ? (c & 0x07u) : n == 2 ? (c & 0x0Fu) : (c & 0x1Fu);
    bool ok = n > 0;
    for (int k = 1; ok && k <= n; ++k) {
      if (i + static_cast<std::size_t>(k) >= s.size()) {
        ok = false;
        break;
      }
      const unsigned char d = static_cast<unsigned char>(s[i + static_cast<std::size_t>(k)]);
      if ((d & 0xC0u) != 0x80u) ok = false;
      cp = (cp << 6) | (d & 0x3Fu);
    }
    if (!ok) {
      u(0xFFFD);
      ++i;
      continue;
    }
    i += static_cast<std::size_t>(n) + 1;
    if (cp >= 0x10000u) {
      cp -= 0x10000u;
      u(0xD800u + (cp >> 10));
      u(0xDC00u + (cp & 0x3FFu));
    } else {
      u(cp);
    }
  }
  out += '"';
}

// json.dumps(value, indent=indent) layout.
inline void write(std::string& out, const Json& v, int indent = 2, int depth = 0) {
  const auto newline = [&](int d) {
    out += '\n';
    out.append(static_cast<std::size_t>(indent * d), ' ');
  };
  switch (v.kind) {
    case Json::Null: out += "null"; return;
    case Json::Bool: out += v.b ? "true" : "false"; return;
    case Json::Number: out += v.text; return;
    case Json::String: write_string(out, v.text); return;
    case Json::Array:
      if (v.items.empty()) {
        out += "[]";
        return;
      }
      out += '[';
      for (std::size_t i = 0; i < v.items.size(); ++i) {
        if (i) out += ',';
        newline(depth + 1);
        write(out, v.items[i], indent, depth + 1);
      }
      newline(depth);
      out += ']';
      return;
    case Json::Object:
      if (v.members.empty()) {
        out += "{}";
        return;
      }
      out += '{';
      for (std::size_t i = 0; i < v.members.size(); ++i) {
        if (i) out += ',';
        newline(depth + 1);
        write_string(out, v.members[i].first);
        out += ": ";
        write(out, v.members[i].second, indent, depth + 1);
      }
      newline(depth);
      out += '}';
      return;
  }
}

inline std::string dump(const Json& v, int indent = 2) {
  std::string out;
  write(out, v, indent);
  return out;
}

}  // namespace json
}  // namespace rtxllm
