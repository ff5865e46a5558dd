// A small JSON reader for manifests (objects keep their key order; every value records the span of its
// text, so a caller can hand a sub-document on unchanged). Shared by the manifest-op runner and the
// program runtime.
#pragma once
#include <cctype>
#include <cerrno>
#include <cstdint>
#include <cstdlib>
#include <cstring>
#include <string>
#include <utility>
#include <vector>

namespace kern_json {

struct JVal {
  enum Kind { Null, Bool, Int, Float, Str, Arr, Obj } kind = Null;
  size_t off = 0, len = 0;  // the value's text: bytes [off, off + len) of the parsed document
  bool b = false;
  int64_t i = 0;
  uint64_t u = 0;      // the integer as unsigned (for values above INT64_MAX)
  bool is_u64 = false;  // integer text that only fits unsigned
  double f = 0;
  std::string s;
  std::vector<JVal> a;
  std::vector<std::pair<std::string, JVal>> o;
  const JVal* get(const char* key) const {
    for (auto& kv : o)
      if (kv.first == key) return &kv.second;
    return nullptr;
  }
  bool is_num() const { return kind == Int || kind == Float; }
};

struct JParser {
  const char* p;
  const char* end;
  std::string err;
  void ws() {
    while (p < end && (*p == ' ' || *p == '\n' || *p == '\t' || *p == '\r')) ++p;
  }
  bool fail(const char* what) {
    if (err.empty()) err = what;
    return false;
  }
  bool str(std::string& out) {
    if (p >= end || *p != '"') return fail("expected a string");
    ++p;
    while (p < end && *p != '"') {
      char c = *p++;
      if (c != '\\') {
        out += c;
        continue;
      }
      if (p >= end) return fail("unterminated escape");
      char e = *p++;
      switch (e) {
        case '"': out += '"'; break;
        case '\\': out += '\\'; break;
        case '/': out += '/'; break;
        case 'b': out += '\b'; break;
        case 'f': out += '\f'; break;
        case 'n': out += '\n'; break;
        case 'r': out += '\r'; break;
        case 't': out += '\t'; break;
        case 'u': {
          if (end - p < 4) return fail("short \\u escape");
          unsigned cp = (unsigned)strtoul(std::string(p, 4).c_str(), nullptr, 16);
          p += 4;
          if (cp < 0x80) {
            out += (char)cp;
          } else if (cp < 0x800) {
            out += (char)(0xC0 | (cp >> 6));
            out += (char)(0x80 | (cp & 0x3F));
          } else {
            out += (char)(0xE0 | (cp >> 12));
            out += (char)(0x80 | ((cp >> 6) & 0x3F));
            out += (char)(0x80 | (cp & 0x3F));
          }
          break;
        }
        default: return fail("bad escape");
      }
    }
    if (p >= end) return fail("unterminated string");
    ++p;
    return true;
  }
  const char* begin = nullptr;
  bool val(JVal& v, int depth) {
    if (depth > 64) return fail("nesting too deep");
    ws();
    if (p >= end) return fail("unexpected end");
    const char* start = p;
    const bool ok = val_at(v, depth);
    v.off = (size_t)(start - begin), v.len = (size_t)(p - start);
    return ok;
  }
  bool val_at(JVal& v, int depth) {
    char c = *p;
    if (c == '{') {
      v.kind = JVal::Obj;
      ++p;
      ws();
      if (p < end && *p == '}') {
        ++p;
        return true;
      }
      for (;;) {
        ws();
        std::string k;
        if (!str(k)) return false;
        ws();
        if (p >= end || *p != ':') return fail("expected ':'");
        ++p;
        v.o.emplace_back(k, JVal());
        if (!val(v.o.back().second, depth + 1)) return false;
        ws();
        if (p < end && *p == ',') {
          ++p;
          continue;
        }
        if (p < end && *p == '}') {
          ++p;
          return true;
        }
        return fail("expected ',' or '}'");
      }
    }
    if (c == '[') {
      v.kind = JVal::Arr;
      ++p;
      ws();
      if (p < end && *p == ']') {
        ++p;
        return true;
      }
      for (;;) {
        v.a.emplace_back();
        if (!val(v.a.back(), depth + 1)) return false;
        ws();
        if (p < end && *p == ',') {
          ++p;
          continue;
        }
        if (p < end && *p == ']') {
          ++p;
          return true;
        }
        return fail("expected ',' or ']'");
      }
    }
    if (c == '"') {
      v.kind = JVal::Str;
      return str(v.s);
    }
    if (!strncmp(p, "true", 4)) {
      v.kind = JVal::Bool, v.b = true, p += 4;
      return true;
    }
    if (!strncmp(p, "false", 5)) {
      v.kind = JVal::Bool, v.b = false, p += 5;
      return true;
    }
    if (!strncmp(p, "null", 4)) {
      v.kind = JVal::Null, p += 4;
      return true;
    }
    const char* s = p;
    if (p < end && (*p == '-' || *p == '+')) ++p;
    bool flt = false;
    while (p < end && (isdigit((unsigned char)*p) || *p == '.' || *p == 'e' || *p == 'E' || *p == '-' || *p == '+')) {
      if (*p == '.' || *p == 'e' || *p == 'E') flt = true;
      ++p;
    }
    if (p == s) return fail("unexpected character");
    std::string t(s, p);
    errno = 0;
    if (!flt) {
      v.kind = JVal::Int;
      if (t[0] != '-') {
        v.u = strtoull(t.c_str(), nullptr, 10);
        if (errno) return fail("integer out of range");
        v.is_u64 = v.u > (uint64_t)INT64_MAX;
        v.i = (int64_t)v.u;
      } else {
        v.i = strtoll(t.c_str(), nullptr, 10);
        if (errno) return fail("integer out of range");
        v.u = (uint64_t)v.i;
      }
      v.f = v.is_u64 ? (double)v.u : (double)v.i;
    } else {
      v.kind = JVal::Float;
      v.f = strtod(t.c_str(), nullptr);
    }
    return true;
  }
};

inline bool parse_json(const char* text, JVal& out, std::string& err) {
  JParser ps{text, text + strlen(text), {}};
  ps.begin = text;
  if (!ps.val(out, 0)) {
    err = ps.err + " at byte " + std::to_string(ps.p - text);
    return false;
  }
  ps.ws();
  if (ps.p != ps.end) {
    err = "trailing characters at byte " + std::to_string(ps.p - text);
    return false;
  }
  return true;
}

}  // namespace kern_json
