// The LKV2 snapshot format (kv_disk.rs): CRC-32, the manifest's JSON, and
// the file reader and writer primitives. Host code; no device calls here
// (the cache's export and import, which move rows to and from the device,
// are in cache.hip).
#include "lkv.hpp"

#include <cstdio>
#include <cstring>
#include <limits>

#include "common.hpp"

namespace tqkv {
namespace lkv {

size_t elem_size(uint8_t tag) {
  switch (tag) {
    case kBool: case kU8: case kI8: return 1;
    case kU16: case kI16: case kF16: case kBF16: return 2;
    case kU32: case kI32: case kF32: return 4;
    case kU64: case kI64: case kF64: return 8;
  }
  return 0;
}

namespace {

struct CrcTable {
  uint32_t t[256];
  CrcTable() {
    for (uint32_t i = 0; i < 256; ++i) {
      uint32_t c = i;
      for (int k = 0; k < 8; ++k) c = (c & 1) ? 0xEDB88320u ^ (c >> 1) : c >> 1;
      t[i] = c;
    }
  }
};
const CrcTable kCrc;

void put_u32(uint8_t* p, uint32_t v) {
  for (int i = 0; i < 4; ++i) p[i] = uint8_t(v >> (8 * i));
}
void put_u64(uint8_t* p, uint64_t v) {
  for (int i = 0; i < 8; ++i) p[i] = uint8_t(v >> (8 * i));
}
uint32_t get_u32(const uint8_t* p) {
  return uint32_t(p[0]) | uint32_t(p[1]) << 8 | uint32_t(p[2]) << 16 | uint32_t(p[3]) << 24;
}
uint64_t get_u64(const uint8_t* p) {
  return uint64_t(get_u32(p)) | uint64_t(get_u32(p + 4)) << 32;
}

// ---------------------------------------------------------------- writing JSON
void json_string(std::string& o, const std::string& s) {
  static const char* hex = "0123456789abcdef";
  o += '"';
  for (unsigned char c : s) {
    switch (c) {
      case '"': o += "\\\""; break;
      case '\\': o += "\\\\"; break;
      case '\b': o += "\\b"; break;
      case '\f': o += "\\f"; break;
      case '\n': o += "\\n"; break;
      case '\r': o += "\\r"; break;
      case '\t': o += "\\t"; break;
      default:
        if (c < 0x20) {
          o += "\\u00";
          o += hex[c >> 4];
          o += hex[c & 15];
        } else {
          o += char(c);
        }
    }
  }
  o += '"';
}

void json_uint(std::string& o, uint64_t v) { o += std::to_string(v); }

void json_opt(std::string& o, const char* name, const Opt& v) {
  if (!v.has) return;
  o += ",\"";
  o += name;
  o += "\":";
  json_uint(o, v.v);
}

// ---------------------------------------------------------------- parsing JSON
struct Value {
  enum Kind { Null, Bool, Num, Str, Arr, Obj } kind = Null;
  bool b = false;
  bool num_int = false, num_neg = false;
  uint64_t num_mag = 0;  // integer magnitude when num_int
  std::string s;
  std::vector<Value> a;
  std::vector<std::pair<std::string, Value>> o;
};

struct Parser {
  const char* begin;
  const char* p;
  const char* end;
  std::string err;
  int depth = 0;

  bool fail_at(const char* what) {
    if (err.empty()) err = std::string(what) + " at byte " + std::to_string(p - begin);
    return false;
  }
  void ws() {
    while (p < end && (*p == ' ' || *p == '\t' || *p == '\n' || *p == '\r')) ++p;
  }
  bool lit(const char* w) {
    const size_t n = strlen(w);
    if (size_t(end - p) < n || memcmp(p, w, n) != 0) return fail_at("invalid literal");
    p += n;
    return true;
  }
  static void utf8(std::string& s, uint32_t cp) {
    if (cp < 0x80) {
      s += char(cp);
    } else if (cp < 0x800) {
      s += char(0xC0 | (cp >> 6));
      s += char(0x80 | (cp & 0x3F));
    } else if (cp < 0x10000) {
      s += char(0xE0 | (cp >> 12));
      s += char(0x80 | ((cp >> 6) & 0x3F));
      s += char(0x80 | (cp & 0x3F));
    } else {
      s += char(0xF0 | (cp >> 18));
      s += char(0x80 | ((cp >> 12) & 0x3F));
      s += char(0x80 | ((cp >> 6) & 0x3F));
      s += char(0x80 | (cp & 0x3F));
    }
  }
  bool hex4(uint32_t* v) {
    if (end - p < 4) return fail_at("truncated \\u escape");
    uint32_t x = 0;
    for (int i = 0; i < 4; ++i) {
      const char c = p[i];
      x <<= 4;
      if (c >= '0' && c <= '9') x |= uint32_t(c - '0');
      else if (c >= 'a' && c <= 'f') x |= uint32_t(c - 'a' + 10);
      else if (c >= 'A' && c <= 'F') x |= uint32_t(c - 'A' + 10);
      else return fail_at("invalid \\u escape");
    }
    p += 4;
    *v = x;
    return true;
  }
  // Raw UTF-8 must be well formed (serde_json::from_slice checks it).
  bool utf8_raw(std::string& s) {
    const unsigned char c = static_cast<unsigned char>(*p);
    int n = c >= 0xF0 ? 3 : c >= 0xE0 ? 2 : c >= 0xC0 ? 1 : -1;
    if (n < 0 || c >= 0xF8) return fail_at("invalid UTF-8");
    if (end - p < n + 1) return fail_at("truncated UTF-8");
    uint32_t cp = c & (n == 1 ? 0x1F : n == 2 ? 0x0F : 0x07);
    for (int i = 1; i <= n; ++i) {
      const unsigned char d = static_cast<unsigned char>(p[i]);
      if ((d & 0xC0) != 0x80) return fail_at("invalid UTF-8");
      cp = (cp << 6) | (d & 0x3F);
    }
    const uint32_t lo = n == 1 ? 0x80 : n == 2 ? 0x800 : 0x10000;
    if (cp < lo || cp > 0x10FFFF || (cp >= 0xD800 && cp <= 0xDFFF)) return fail_at("invalid UTF-8");
    s.append(p, size_t(n) + 1);
    p += n + 1;
    return true;
  }
  bool string(std::string& s) {
    ++p;  // opening quote
    while (true) {
      if (p >= end) return fail_at("unterminated string");
      const unsigned char c = static_cast<unsigned char>(*p);
      if (c == '"') {
        ++p;
        return true;
      }
      if (c < 0x20) return fail_at("control character in string");
      if (c == '\\') {
        if (++p >= end) return fail_at("unterminated escape");
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
            uint32_t cp;
            if (!hex4(&cp)) return false;
            if (cp >= 0xD800 && cp <= 0xDBFF) {
              if (end - p < 2 || p[0] != '\\' || p[1] != 'u') return fail_at("lone surrogate");
              p += 2;
              uint32_t lo;
              if (!hex4(&lo)) return false;
              if (lo < 0xDC00 || lo > 0xDFFF) return fail_at("lone surrogate");
              cp = 0x10000 + ((cp - 0xD800) << 10) + (lo - 0xDC00);
            } else if (cp >= 0xDC00 && cp <= 0xDFFF) {
              return fail_at("lone surrogate");
            }
            utf8(s, cp);
            break;
          }
          default: return fail_at("invalid escape");
        }
      } else if (c < 0x80) {
        s += char(c);
        ++p;
      } else if (!utf8_raw(s)) {
        return false;
      }
    }
  }
  bool number(Value& v) {
    v.kind = Value::Num;
    if (*p == '-') {
      v.num_neg = true;
      ++p;
    }
    if (p >= end || *p < '0' || *p > '9') return fail_at("invalid number");
    if (*p == '0' && p + 1 < end && p[1] >= '0' && p[1] <= '9') return fail_at("leading zero");
    bool overflow = false;
    uint64_t mag = 0;
    while (p < end && *p >= '0' && *p <= '9') {
      const uint64_t d = uint64_t(*p - '0');
      if (mag > (std::numeric_limits<uint64_t>::max() - d) / 10) overflow = true;
      mag = mag * 10 + d;
      ++p;
    }
    bool frac = false;
    if (p < end && *p == '.') {
      frac = true;
      ++p;
      if (p >= end || *p < '0' || *p > '9') return fail_at("invalid number");
      while (p < end && *p >= '0' && *p <= '9') ++p;
    }
    if (p < end && (*p == 'e' || *p == 'E')) {
      frac = true;
      ++p;
      if (p < end && (*p == '+' || *p == '-')) ++p;
      if (p >= end || *p < '0' || *p > '9') return fail_at("invalid number");
      while (p < end && *p >= '0' && *p <= '9') ++p;
    }
    v.num_int = !frac && !overflow;
    v.num_mag = mag;
    return true;
  }
  bool value(Value& v) {
    if (++depth > 64) return fail_at("nesting too deep");
    ws();
    if (p >= end) return fail_at("unexpected end of JSON");
    bool okv = true;
    switch (*p) {
      case 'n': okv = lit("null"); v.kind = Value::Null; break;
      case 't': okv = lit("true"); v.kind = Value::Bool; v.b = true; break;
      case 'f': okv = lit("false"); v.kind = Value::Bool; v.b = false; break;
      case '"': v.kind = Value::Str; okv = string(v.s); break;
      case '[': {
        v.kind = Value::Arr;
        ++p;
        ws();
        if (p < end && *p == ']') {
          ++p;
          break;
        }
        while (okv) {
          v.a.emplace_back();
          if (!value(v.a.back())) return false;
          ws();
          if (p < end && *p == ',') {
            ++p;
            continue;
          }
          if (p < end && *p == ']') {
            ++p;
            break;
          }
          return fail_at("expected , or ] in array");
        }
        break;
      }
      case '{': {
        v.kind = Value::Obj;
        ++p;
        ws();
        if (p < end && *p == '}') {
          ++p;
          break;
        }
        while (okv) {
          ws();
          if (p >= end || *p != '"') return fail_at("expected a key");
          std::string k;
          if (!string(k)) return false;
          ws();
          if (p >= end || *p != ':') return fail_at("expected :");
          ++p;
          v.o.emplace_back(std::move(k), Value());
          if (!value(v.o.back().second)) return false;
          ws();
          if (p < end && *p == ',') {
            ++p;
            continue;
          }
          if (p < end && *p == '}') {
            ++p;
            break;
          }
          return fail_at("expected , or } in object");
        }
        break;
      }
      default:
        if (*p == '-' || (*p >= '0' && *p <= '9')) okv = number(v);
        else okv = fail_at("unexpected character");
    }
    --depth;
    return okv;
  }
};

// Field readers with serde's type rules for the manifest's fields.
struct Fields {
  std::string* err;
  bool bad(const std::string& msg) {
    if (err->empty()) *err = msg;
    return false;
  }
  bool u64(const Value& v, const char* name, uint64_t max, uint64_t* out) {
    if (v.kind != Value::Num || !v.num_int || (v.num_neg && v.num_mag != 0) || v.num_mag > max)
      return bad(std::string("invalid value for field `") + name + "`");
    *out = v.num_mag;
    return true;
  }
  bool i32(const Value& v, const char* name, int64_t* out) {
    if (v.kind != Value::Num || !v.num_int) return bad(std::string("invalid value for `") + name + "`");
    if (v.num_neg ? v.num_mag > 2147483648ull : v.num_mag > 2147483647ull)
      return bad(std::string("out of range value for `") + name + "`");
    *out = v.num_neg ? -int64_t(v.num_mag) : int64_t(v.num_mag);
    return true;
  }
  bool opt(const Value& v, const char* name, uint64_t max, Opt* out) {
    if (v.kind == Value::Null) {
      out->has = false;
      return true;
    }
    out->has = true;
    return u64(v, name, max, &out->v);
  }
};

constexpr uint64_t kUsize = std::numeric_limits<uint64_t>::max();
constexpr uint64_t kU32Max = 0xFFFFFFFFull;

bool is_kind(const std::string& k) {
  static const char* const kinds[] = {"Full", "Linear", "FullTurboquant", "Sliding",
                                      "FullQuantized", "SlidingQuantized", "SlidingTurboquant"};
  for (const char* x : kinds)
    if (k == x) return true;
  return false;
}

bool layer_from(const Value& v, Layer* L, Fields& f) {
  if (v.kind != Value::Obj) return f.bad("invalid type for a layer: expected struct LayerMeta");
  bool have_kind = false, have_offset = false;
  std::vector<std::string> seen;
  for (const auto& kv : v.o) {
    const std::string& k = kv.first;
    const Value& x = kv.second;
    for (const std::string& s : seen)
      if (s == k) return f.bad("duplicate field `" + k + "`");
    seen.push_back(k);
    if (k == "kind") {
      if (x.kind != Value::Str || !is_kind(x.s)) return f.bad("unknown variant for `kind`");
      L->kind = x.s;
      have_kind = true;
    } else if (k == "offset") {
      if (!f.u64(x, "offset", kUsize, &L->offset)) return false;
      have_offset = true;
    } else if (k == "base_offset") {
      if (!f.u64(x, "base_offset", kUsize, &L->base_offset)) return false;
    } else if (k == "arrays") {
      if (x.kind != Value::Arr) return f.bad("invalid type for `arrays`");
      L->arrays.clear();
      for (const Value& e : x.a) {
        if (e.kind == Value::Null) {
          L->arrays.push_back(-1);
        } else {
          uint64_t id;
          if (!f.u64(e, "arrays", uint64_t(std::numeric_limits<int64_t>::max()), &id)) return false;
          L->arrays.push_back(int64_t(id));
        }
      }
    } else if (k == "lengths_id") {
      if (!f.opt(x, "lengths_id", kUsize, &L->lengths_id)) return false;
    } else if (k == "left_padding_id") {
      if (!f.opt(x, "left_padding_id", kUsize, &L->left_padding_id)) return false;
    } else if (k == "max_size") {
      if (!f.opt(x, "max_size", kUsize, &L->max_size)) return false;
    } else if (k == "keep") {
      if (!f.opt(x, "keep", kUsize, &L->keep)) return false;
    } else if (k == "idx") {
      if (!f.opt(x, "idx", kUsize, &L->idx)) return false;
    } else if (k == "bits") {
      if (!f.opt(x, "bits", kU32Max, &L->bits)) return false;
    } else if (k == "qjl_m") {
      if (!f.opt(x, "qjl_m", kUsize, &L->qjl_m)) return false;
    } else if (k == "group_size") {
      if (x.kind == Value::Null) {
        L->has_group_size = false;
      } else {
        if (!f.i32(x, "group_size", &L->group_size)) return false;
        L->has_group_size = true;
      }
    }
  }
  if (!have_kind) return f.bad("missing field `kind`");
  if (!have_offset) return f.bad("missing field `offset`");
  return true;
}

}  // namespace

uint32_t crc32(const void* data, size_t n, uint32_t crc) {
  const uint8_t* p = static_cast<const uint8_t*>(data);
  uint32_t c = ~crc;
  for (size_t i = 0; i < n; ++i) c = kCrc.t[(c ^ p[i]) & 0xFF] ^ (c >> 8);
  return ~c;
}

std::string manifest_json(const Manifest& m) {
  std::string o = "{\"model_fingerprint\":";
  json_string(o, m.model_fingerprint);
  o += ",\"created_at_unix\":";
  json_uint(o, m.created_at_unix);
  o += ",\"position\":";
  json_uint(o, m.position);
  o += ",\"prefix_tokens\":[";
  for (size_t i = 0; i < m.prefix_tokens.size(); ++i) {
    if (i) o += ',';
    json_uint(o, m.prefix_tokens[i]);
  }
  o += ']';
  json_opt(o, "last_token", m.last_token);
  o += ",\"is_deep\":";
  o += m.is_deep ? "true" : "false";
  o += ",\"layers\":[";
  for (size_t li = 0; li < m.layers.size(); ++li) {
    const Layer& L = m.layers[li];
    if (li) o += ',';
    o += "{\"kind\":";
    json_string(o, L.kind);
    o += ",\"offset\":";
    json_uint(o, L.offset);
    o += ",\"base_offset\":";
    json_uint(o, L.base_offset);
    o += ",\"arrays\":[";
    for (size_t i = 0; i < L.arrays.size(); ++i) {
      if (i) o += ',';
      if (L.arrays[i] < 0) o += "null";
      else json_uint(o, uint64_t(L.arrays[i]));
    }
    o += ']';
    json_opt(o, "lengths_id", L.lengths_id);
    json_opt(o, "left_padding_id", L.left_padding_id);
    json_opt(o, "max_size", L.max_size);
    json_opt(o, "keep", L.keep);
    json_opt(o, "idx", L.idx);
    json_opt(o, "bits", L.bits);
    json_opt(o, "qjl_m", L.qjl_m);
    if (L.has_group_size) {
      o += ",\"group_size\":";
      o += std::to_string(L.group_size);
    }
    o += '}';
  }
  o += "]}";
  return o;
}

bool parse_manifest(const char* s, size_t n, Manifest* m, std::string* err) {
  Parser ps{s, s, s + n, {}};
  Value root;
  if (!ps.value(root)) {
    *err = "deserialize manifest: " + ps.err;
    return false;
  }
  ps.ws();
  if (ps.p != ps.end) {
    *err = "deserialize manifest: trailing characters";
    return false;
  }
  std::string ferr;
  Fields f{&ferr};
  auto failed = [&]() {
    *err = "deserialize manifest: " + ferr;
    return false;
  };
  if (root.kind != Value::Obj) {
    f.bad("invalid type: expected struct KvManifest");
    return failed();
  }
  bool have_fp = false, have_created = false, have_pos = false, have_prefix = false,
       have_layers = false;
  std::vector<std::string> seen;
  *m = Manifest{};
  for (const auto& kv : root.o) {
    const std::string& k = kv.first;
    const Value& x = kv.second;
    for (const std::string& q : seen)
      if (q == k) {
        f.bad("duplicate field `" + k + "`");
        return failed();
      }
    seen.push_back(k);
    if (k == "model_fingerprint") {
      if (x.kind != Value::Str) {
        f.bad("invalid type for `model_fingerprint`");
        return failed();
      }
      m->model_fingerprint = x.s;
      have_fp = true;
    } else if (k == "created_at_unix") {
      if (!f.u64(x, "created_at_unix", kUsize, &m->created_at_unix)) return failed();
      have_created = true;
    } else if (k == "position") {
      if (!f.u64(x, "position", kUsize, &m->position)) return failed();
      have_pos = true;
    } else if (k == "prefix_tokens") {
      if (x.kind != Value::Arr) {
        f.bad("invalid type for `prefix_tokens`");
        return failed();
      }
      for (const Value& e : x.a) {
        uint64_t t;
        if (!f.u64(e, "prefix_tokens", kU32Max, &t)) return failed();
        m->prefix_tokens.push_back(uint32_t(t));
      }
      have_prefix = true;
    } else if (k == "last_token") {
      if (!f.opt(x, "last_token", kU32Max, &m->last_token)) return failed();
    } else if (k == "is_deep") {
      if (x.kind != Value::Bool) {
        f.bad("invalid type for `is_deep`");
        return failed();
      }
      m->is_deep = x.b;
    } else if (k == "layers") {
      if (x.kind != Value::Arr) {
        f.bad("invalid type for `layers`");
        return failed();
      }
      for (const Value& e : x.a) {
        m->layers.emplace_back();
        if (!layer_from(e, &m->layers.back(), f)) return failed();
      }
      have_layers = true;
    }
  }
  if (!have_fp) f.bad("missing field `model_fingerprint`");
  else if (!have_created) f.bad("missing field `created_at_unix`");
  else if (!have_pos) f.bad("missing field `position`");
  else if (!have_prefix) f.bad("missing field `prefix_tokens`");
  else if (!have_layers) f.bad("missing field `layers`");
  if (!ferr.empty()) return failed();
  return true;
}

bool parse(const uint8_t* p, size_t n, Manifest* m, std::vector<RecordView>* recs,
           std::string* err) {
  size_t at = 0;
  auto need = [&](size_t k, const char* what) {
    if (n - at < k) {
      *err = std::string("truncated file: ") + what;
      return false;
    }
    return true;
  };
  if (!need(4, "read magic")) return false;
  if (memcmp(p, "LKV2", 4) != 0) {
    char b[96];
    snprintf(b, sizeof(b), "bad magic [%u, %u, %u, %u] (expected \"LKV2\")", p[0], p[1], p[2], p[3]);
    *err = b;
    return false;
  }
  at = 4;
  if (!need(4, "read version")) return false;
  const uint32_t version = get_u32(p + at);
  at += 4;
  if (version != kVersion) {
    *err = "unsupported version " + std::to_string(version) + " (expected 2)";
    return false;
  }
  if (!need(4, "read manifest length")) return false;
  const uint32_t json_len = get_u32(p + at);
  at += 4;
  if (!need(json_len, "read manifest")) return false;
  const char* json = reinterpret_cast<const char*>(p + at);
  at += json_len;
  if (!need(4, "read manifest CRC")) return false;
  if (get_u32(p + at) != crc32(json, json_len)) {
    *err = "manifest CRC mismatch (corrupt file)";
    return false;
  }
  at += 4;
  if (!parse_manifest(json, json_len, m, err)) return false;
  if (!need(4, "read record count")) return false;
  const uint32_t count = get_u32(p + at);
  at += 4;
  recs->clear();
  for (uint32_t r = 0; r < count; ++r) {
    const size_t rec0 = at;
    RecordView v;
    if (!need(1, "read record dtype")) return false;
    v.dtype = p[at++];
    const size_t es = elem_size(v.dtype);
    if (es == 0) {
      *err = "unknown dtype tag byte " + std::to_string(unsigned(v.dtype));
      return false;
    }
    if (!need(4, "read record ndim")) return false;
    const uint32_t ndim = get_u32(p + at);
    at += 4;
    if (ndim > 8) {
      *err = "implausible ndim " + std::to_string(ndim) + " (corrupt record)";
      return false;
    }
    uint64_t expected = ndim ? 1 : 0;
    bool overflow = false;
    for (uint32_t d = 0; d < ndim; ++d) {
      if (!need(4, "read record shape")) return false;
      const int32_t dim = int32_t(get_u32(p + at));
      at += 4;
      if (dim < 0) {
        *err = "negative dimension " + std::to_string(dim) + " (corrupt record)";
        return false;
      }
      v.shape.push_back(dim);
      if (dim != 0 && expected > std::numeric_limits<uint64_t>::max() / uint64_t(dim)) overflow = true;
      expected *= uint64_t(dim);
    }
    if (expected > std::numeric_limits<uint64_t>::max() / es) overflow = true;
    expected *= es;
    if (!need(8, "read record length")) return false;
    const uint64_t data_len = get_u64(p + at);
    at += 8;
    if (overflow || data_len != expected) {
      *err = "record declares " + std::to_string(data_len) +
             " payload bytes but its shape and dtype imply " +
             (overflow ? std::string("more than 2^64") : std::to_string(expected)) +
             " (corrupt record)";
      return false;
    }
    if (uint64_t(n - at) < data_len) {
      *err = "truncated file: record payload of " + std::to_string(data_len) + " bytes";
      return false;
    }
    v.data = p + at;
    v.bytes = data_len;
    at += size_t(data_len);
    if (!need(4, "read record CRC")) return false;
    if (get_u32(p + at) != crc32(p + rec0, at - rec0)) {
      *err = "record CRC mismatch (corrupt file)";
      return false;
    }
    at += 4;
    recs->push_back(std::move(v));
  }
  if (at != n) {
    *err = "trailing bytes after " + std::to_string(count) + " records (corrupt record count)";
    return false;
  }
  return true;
}

uint64_t write_header(uint8_t* out, const std::string& json, uint32_t n_records) {
  memcpy(out, "LKV2", 4);
  put_u32(out + 4, kVersion);
  put_u32(out + 8, uint32_t(json.size()));
  memcpy(out + 12, json.data(), json.size());
  put_u32(out + 12 + json.size(), crc32(json.data(), json.size()));
  put_u32(out + 16 + json.size(), n_records);
  return header_size(json.size());
}

uint64_t write_record_header(uint8_t* out, uint8_t dtype, const std::vector<int64_t>& shape,
                             uint64_t data_bytes) {
  out[0] = dtype;
  put_u32(out + 1, uint32_t(shape.size()));
  for (size_t i = 0; i < shape.size(); ++i) put_u32(out + 5 + 4 * i, uint32_t(int32_t(shape[i])));
  put_u64(out + 5 + 4 * shape.size(), data_bytes);
  return 1 + 4 + 4 * uint64_t(shape.size()) + 8;
}

void finish_record(uint8_t* rec, uint64_t len) { put_u32(rec + len, crc32(rec, size_t(len))); }

}  // namespace lkv
}  // namespace tqkv

using namespace tqkv;

extern "C" {

int32_t tqkv_crc32(const void* data, size_t bytes, uint32_t* out) {
  if ((!data && bytes) || !out) return fail(TQKV_EINVAL_ARG, "null pointer");
  *out = lkv::crc32(data, bytes);
  return ok();
}

int32_t tqkv_lkv_check(const uint8_t* data, size_t bytes) {
  if (!data && bytes) return fail(TQKV_EINVAL_ARG, "null pointer");
  lkv::Manifest m;
  std::vector<lkv::RecordView> recs;
  std::string err;
  if (!lkv::parse(data ? data : reinterpret_cast<const uint8_t*>(""), bytes, &m, &recs, &err))
    return fail(TQKV_ECORRUPT, "kv_disk: %s", err.c_str());
  return ok();
}

int32_t tqkv_lkv_manifest(const uint8_t* data, size_t bytes, char* json, size_t capacity,
                          size_t* json_bytes, int32_t* n_layers, int32_t* n_records) {
  if (!data && bytes) return fail(TQKV_EINVAL_ARG, "null pointer");
  lkv::Manifest m;
  std::vector<lkv::RecordView> recs;
  std::string err;
  if (!lkv::parse(data ? data : reinterpret_cast<const uint8_t*>(""), bytes, &m, &recs, &err))
    return fail(TQKV_ECORRUPT, "kv_disk: %s", err.c_str());
  const uint32_t len = uint32_t(data[8]) | uint32_t(data[9]) << 8 | uint32_t(data[10]) << 16 |
                       uint32_t(data[11]) << 24;
  if (json_bytes) *json_bytes = len;
  if (n_layers) *n_layers = int32_t(m.layers.size());
  if (n_records) *n_records = int32_t(recs.size());
  if (json) {
    if (capacity < size_t(len) + 1) return fail(TQKV_EINVAL_ARG, "manifest needs %u + 1 bytes", len);
    memcpy(json, data + 12, len);
    json[len] = '\0';
  }
  return ok();
}

int32_t tqkv_lkv_rewrite(const uint8_t* data, size_t bytes, uint8_t* out, size_t capacity,
                         size_t* out_bytes) {
  if ((!data && bytes) || !out_bytes) return fail(TQKV_EINVAL_ARG, "null pointer");
  lkv::Manifest m;
  std::vector<lkv::RecordView> recs;
  std::string err;
  if (!lkv::parse(data ? data : reinterpret_cast<const uint8_t*>(""), bytes, &m, &recs, &err))
    return fail(TQKV_ECORRUPT, "kv_disk: %s", err.c_str());
  const std::string json = lkv::manifest_json(m);
  uint64_t total = lkv::header_size(json.size());
  for (const lkv::RecordView& r : recs) total += lkv::record_size(r.shape.size(), r.bytes);
  *out_bytes = size_t(total);
  if (!out) return ok();
  if (capacity < total) return fail(TQKV_EINVAL_ARG, "needs %llu bytes", (unsigned long long)total);
  uint64_t at = lkv::write_header(out, json, uint32_t(recs.size()));
  for (const lkv::RecordView& r : recs) {
    uint8_t* rec = out + at;
    const uint64_t h = lkv::write_record_header(rec, r.dtype, r.shape, r.bytes);
    if (r.bytes) memcpy(rec + h, r.data, size_t(r.bytes));
    lkv::finish_record(rec, h + r.bytes);
    at += lkv::record_size(r.shape.size(), r.bytes);
  }
  return ok();
}

}  // extern "C"
