// A small JSON reader and writer for the host side: transformer/config.json,
// safetensors headers and adapter metadata. Objects keep their key order, so
// a config rewritten by the pack writer keeps every key where it was.
#pragma once

#include <cstdint>
#include <cstdio>
#include <cstdlib>
#include <string>
#include <utility>
#include <vector>

namespace ming::json {

struct Value {
  enum Kind { Null, Bool, Num, Str, Arr, Obj };
  Kind kind = Null;
  bool b = false;
  double num = 0.0;
  std::string str;
  std::vector<Value> arr;
  std::vector<std::pair<std::string, Value>> obj;

  bool is_obj() const { return kind == Obj; }
  bool is_arr() const { return kind == Arr; }
  bool is_num() const { return kind == Num; }
  bool is_str() const { return kind == Str; }
  bool is_bool() const { return kind == Bool; }
  const Value* get(const std::string& k) const {
    if (kind != Obj) return nullptr;
    for (const auto& kv : obj)
      if (kv.first == k) return &kv.second;
    return nullptr;
  }
  void set(const std::string& k, Value v) {
    kind = Obj;
    for (auto& kv : obj)
      if (kv.first == k) {
        kv.second = std::move(v);
        return;
      }
    obj.emplace_back(k, std::move(v));
  }
  static Value number(double d) {
    Value v;
    v.kind = Num;
    v.num = d;
    return v;
  }
  static Value string(std::string s) {
    Value v;
    v.kind = Str;
    v.str = std::move(s);
    return v;
  }
  static Value object() {
    Value v;
    v.kind = Obj;
    return v;
  }
  static Value array() {
    Value v;
    v.kind = Arr;
    return v;
  }
};

namespace detail {

struct Parser {
  const char* p;
  const char* end;
  std::string err;
  int depth = 0;

  bool fail(const char* what) {
    if (err.empty()) err = what;
    return false;
  }
  void ws() {
    while (p < end && (*p == ' ' || *p == '\t' || *p == '\n' || *p == '\r')) ++p;
  }
  bool lit(const char* s) {
    const char* q = p;
    for (; *s; ++s, ++q)
      if (q >= end || *q != *s) return false;
    p = q;
    return true;
  }
  static void utf8(uint32_t c, std::string* o) {
    if (c < 0x80) {
      o->push_back((char)c);
    } else if (c < 0x800) {
      o->push_back((char)(0xC0 | (c >> 6)));
      o->push_back((char)(0x80 | (c & 0x3F)));
    } else if (c < 0x10000) {
      o->push_back((char)(0xE0 | (c >> 12)));
      o->push_back((char)(0x80 | ((c >> 6) & 0x3F)));
      o->push_back((char)(0x80 | (c & 0x3F)));
    } else {
      o->push_back((char)(0xF0 | (c >> 18)));
      o->push_back((char)(0x80 | ((c >> 12) & 0x3F)));
      o->push_back((char)(0x80 | ((c >> 6) & 0x3F)));
      o->push_back((char)(0x80 | (c & 0x3F)));
    }
  }
  bool hex4(uint32_t* c) {
    if (end - p < 4) return fail("truncated \\u escape");
    uint32_t v = 0;
    for (int i = 0; i < 4; ++i) {
      const char h = *p++;
      v <<= 4;
      if (h >= '0' && h <= '9') v |= (uint32_t)(h - '0');
      else if (h >= 'a' && h <= 'f') v |= (uint32_t)(h - 'a' + 10);
      else if (h >= 'A' && h <= 'F') v |= (uint32_t)(h - 'A' + 10);
      else return fail("bad \\u escape");
    }
    *c = v;
    return true;
  }
  bool str(std::string* o) {
    if (p >= end || *p != '"') return fail("expected a string");
    ++p;
    while (true) {
      if (p >= end) return fail("unterminated string");
      const char ch = *p++;
      if (ch == '"') return true;
      if ((unsigned char)ch < 0x20) return fail("control character in a string");
      if (ch != '\\') {
        o->push_back(ch);
        continue;
      }
      if (p >= end) return fail("unterminated escape");
      const char e = *p++;
      switch (e) {
        case '"': o->push_back('"'); break;
        case '\\': o->push_back('\\'); break;
        case '/': o->push_back('/'); break;
        case 'b': o->push_back('\b'); break;
        case 'f': o->push_back('\f'); break;
        case 'n': o->push_back('\n'); break;
        case 'r': o->push_back('\r'); break;
        case 't': o->push_back('\t'); break;
        case 'u': {
          uint32_t c;
          if (!hex4(&c)) return false;
          if (c >= 0xD800 && c < 0xDC00) {  // a surrogate pair
            uint32_t lo;
            if (end - p < 6 || p[0] != '\\' || p[1] != 'u') return fail("lone surrogate");
            p += 2;
            if (!hex4(&lo) || lo < 0xDC00 || lo >= 0xE000) return fail("bad surrogate pair");
            c = 0x10000 + ((c - 0xD800) << 10) + (lo - 0xDC00);
          }
          utf8(c, o);
          break;
        }
        default: return fail("unknown escape");
      }
    }
  }
  bool num(double* o) {
    const char* s = p;
    if (p < end && *p == '-') ++p;
    if (p >= end || !((*p >= '0' && *p <= '9'))) return fail("bad number");
    while (p < end && ((*p >= '0' && *p <= '9') || *p == '.' || *p == 'e' || *p == 'E' ||
                       *p == '+' || *p == '-'))
      ++p;
    std::string t(s, p);
    char* q = nullptr;
    *o = std::strtod(t.c_str(), &q);
    if (q != t.c_str() + t.size()) return fail("bad number");
    return true;
  }
  bool value(Value* v) {
    if (++depth > 64) return fail("nesting too deep");
    ws();
    if (p >= end) return fail("unexpected end");
    bool ok = true;
    const char c = *p;
    if (c == '{') {
      ++p;
      v->kind = Value::Obj;
      ws();
      if (p < end && *p == '}') {
        ++p;
      } else {
        while (true) {
          ws();
          std::string k;
          if (!str(&k)) return false;
          ws();
          if (p >= end || *p != ':') return fail("expected ':'");
          ++p;
          Value child;
          if (!value(&child)) return false;
          v->obj.emplace_back(std::move(k), std::move(child));
          ws();
          if (p < end && *p == ',') {
            ++p;
            continue;
          }
          if (p < end && *p == '}') {
            ++p;
            break;
          }
          return fail("expected ',' or '}'");
        }
      }
    } else if (c == '[') {
      ++p;
      v->kind = Value::Arr;
      ws();
      if (p < end && *p == ']') {
        ++p;
      } else {
        while (true) {
          Value child;
          if (!value(&child)) return false;
          v->arr.push_back(std::move(child));
          ws();
          if (p < end && *p == ',') {
            ++p;
            continue;
          }
          if (p < end && *p == ']') {
            ++p;
            break;
          }
          return fail("expected ',' or ']'");
        }
      }
    } else if (c == '"') {
      v->kind = Value::Str;
      ok = str(&v->str);
    } else if (lit("true")) {
      v->kind = Value::Bool;
      v->b = true;
    } else if (lit("false")) {
      v->kind = Value::Bool;
      v->b = false;
    } else if (lit("null")) {
      v->kind = Value::Null;
    } else if (lit("NaN")) {  // Python's json writes these for non-finite floats
      v->kind = Value::Num;
      v->num = std::strtod("nan", nullptr);
    } else if (lit("Infinity")) {
      v->kind = Value::Num;
      v->num = 1.0 / 0.0;
    } else if (lit("-Infinity")) {
      v->kind = Value::Num;
      v->num = -1.0 / 0.0;
    } else {
      v->kind = Value::Num;
      ok = num(&v->num);
    }
    --depth;
    return ok;
  }
};

inline void dump_str(const std::string& s, std::string* o) {
  o->push_back('"');
  for (unsigned char c : s) {
    switch (c) {
      case '"': *o += "\\\""; break;
      case '\\': *o += "\\\\"; break;
      case '\n': *o += "\\n"; break;
      case '\r': *o += "\\r"; break;
      case '\t': *o += "\\t"; break;
      default:
        if (c < 0x20) {
          char b[8];
          std::snprintf(b, sizeof b, "\\u%04x", c);
          *o += b;
        } else {
          o->push_back((char)c);
        }
    }
  }
  o->push_back('"');
}

inline void dump(const Value& v, std::string* o, int indent, int level) {
  auto nl = [&](int l) {
    if (indent <= 0) return;
    o->push_back('\n');
    o->append((size_t)(indent * l), ' ');
  };
  switch (v.kind) {
    case Value::Null: *o += "null"; break;
    case Value::Bool: *o += v.b ? "true" : "false"; break;
    case Value::Num: {
      char b[40];
      const double d = v.num;
      if (d == (double)(int64_t)d && d > -9.0e15 && d < 9.0e15)
        std::snprintf(b, sizeof b, "%lld", (long long)d);
      else
        std::snprintf(b, sizeof b, "%.17g", d);
      *o += b;
      break;
    }
    case Value::Str: dump_str(v.str, o); break;
    case Value::Arr: {
      o->push_back('[');
      for (size_t i = 0; i < v.arr.size(); ++i) {
        if (i) *o += indent > 0 ? ", " : ",";
        dump(v.arr[i], o, 0, 0);  // arrays on one line
      }
      o->push_back(']');
      break;
    }
    case Value::Obj: {
      o->push_back('{');
      for (size_t i = 0; i < v.obj.size(); ++i) {
        if (i) o->push_back(',');
        nl(level + 1);
        dump_str(v.obj[i].first, o);
        *o += indent > 0 ? ": " : ":";
        dump(v.obj[i].second, o, indent, level + 1);
      }
      if (!v.obj.empty()) nl(level);
      o->push_back('}');
      break;
    }
  }
}

}  // namespace detail

// Parses one JSON document (trailing whitespace allowed, nothing else).
inline bool parse(const char* text, size_t n, Value* out, std::string* err) {
  detail::Parser ps{text, text + n, {}};
  Value v;
  bool ok = ps.value(&v);
  if (ok) {
    ps.ws();
    if (ps.p != ps.end) ok = ps.fail("trailing characters");
  }
  if (!ok) {
    if (err) *err = ps.err + " at byte " + std::to_string(ps.p - text);
    return false;
  }
  *out = std::move(v);
  return true;
}

inline std::string dump(const Value& v, int indent = 0) {
  std::string o;
  detail::dump(v, &o, indent, 0);
  return o;
}

}  // namespace ming::json
