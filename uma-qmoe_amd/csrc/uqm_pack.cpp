// ExpertPack / TargetPack reader and device staging (host code).
//
// One read-only mapping per pack. uqm_pack_open validates the whole file in
// the order the reference's readers do (src/uma_qmoe/expert_pack.py:317-556,
// src/uma_qmoe/target_pack.py:493-812) and reports the first violation in
// that order with the same message: prefix, header hash, header padding,
// payload hash, canonical JSON, schema, identities, then tensor by tensor
// (layout, bits per weight, zero padding, SHA-256, payload semantics), then
// unclaimed payload bytes and the TargetPack encoding counts. The byte-heavy
// work (the payload SHA-256 and every tensor's hash, padding and payload
// scans) runs on worker threads; the ordering of the reported error does not
// depend on which thread finishes first.
//
// The header must be the canonical JSON of its own value: keys sorted, no
// whitespace, "," and ":" separators, non-ASCII escaped as \uXXXX, numbers
// as Python's json module writes them (integers in decimal, floats in their
// shortest round-trip form). It is parsed into a small value tree and written
// back in that form; the pack is refused unless the bytes agree.
//
// Staging copies a projection of all experts of a layer from the mapping into
// two pinned host buffers in turn (threads gather, one DMA per buffer fill)
// and from there to expert-major device memory: no Python objects, no clone.
#include <hip/hip_runtime_api.h>
#include <openssl/evp.h>
#include <fcntl.h>
#include <sys/mman.h>
#include <sys/stat.h>
#include <unistd.h>

#include <algorithm>
#include <atomic>
#include <cerrno>
#include <charconv>
#include <cmath>
#include <cstdarg>
#include <cstdio>
#include <cstring>
#include <map>
#include <memory>
#include <string>
#include <thread>
#include <unordered_map>
#include <utility>
#include <vector>

#include "../../include/uma_qmoe_pack.h"

namespace uqm {
int api_fail(int code, const char* fmt, ...);
}

namespace {

// ------------------------------------------------------------------ JSON --
struct Json {
  enum Kind : uint8_t { kNull, kBool, kInt, kFloat, kString, kArray, kObject };
  Kind kind = kNull;
  bool b = false;
  int64_t i = 0;
  double f = 0.0;
  std::string s;                                        // UTF-8 (lone surrogates kept as 3-byte sequences)
  std::vector<Json> a;
  std::vector<std::pair<std::string, Json>> o;          // in input order

  const Json* get(const char* key) const {
    if (kind != kObject) return nullptr;
    const Json* found = nullptr;
    for (const auto& kv : o)
      if (kv.first == key) found = &kv.second;  // the last duplicate wins, as in Python's json
    return found;
  }
  bool is_int() const { return kind == kInt; }
  bool is_str(const char* v) const { return kind == kString && s == v; }
};

class Parser {
 public:
  Parser(const char* p, size_t n) : p_(p), end_(p + n) {}
  bool parse(Json& out) {
    ws();
    if (!value(out, 0)) return false;
    ws();
    return p_ == end_;
  }

 private:
  const char* p_;
  const char* end_;

  void ws() {
    while (p_ < end_ && (*p_ == ' ' || *p_ == '\t' || *p_ == '\n' || *p_ == '\r')) ++p_;
  }
  bool lit(const char* word) {
    size_t n = std::strlen(word);
    if (static_cast<size_t>(end_ - p_) < n || std::memcmp(p_, word, n) != 0) return false;
    p_ += n;
    return true;
  }
  bool value(Json& v, int depth) {
    if (depth > 64 || p_ >= end_) return false;
    switch (*p_) {
      case '{': return object(v, depth);
      case '[': return array(v, depth);
      case '"': v.kind = Json::kString; return string(v.s);
      case 't': v.kind = Json::kBool; v.b = true; return lit("true");
      case 'f': v.kind = Json::kBool; v.b = false; return lit("false");
      case 'n': v.kind = Json::kNull; return lit("null");
      default: return number(v);
    }
  }
  bool object(Json& v, int depth) {
    v.kind = Json::kObject;
    ++p_;
    ws();
    if (p_ < end_ && *p_ == '}') { ++p_; return true; }
    for (;;) {
      ws();
      std::string key;
      if (p_ >= end_ || *p_ != '"' || !string(key)) return false;
      ws();
      if (p_ >= end_ || *p_ != ':') return false;
      ++p_;
      ws();
      v.o.emplace_back(std::move(key), Json{});
      if (!value(v.o.back().second, depth + 1)) return false;
      ws();
      if (p_ >= end_) return false;
      if (*p_ == ',') { ++p_; continue; }
      if (*p_ == '}') { ++p_; return true; }
      return false;
    }
  }
  bool array(Json& v, int depth) {
    v.kind = Json::kArray;
    ++p_;
    ws();
    if (p_ < end_ && *p_ == ']') { ++p_; return true; }
    for (;;) {
      ws();
      v.a.emplace_back();
      if (!value(v.a.back(), depth + 1)) return false;
      ws();
      if (p_ >= end_) return false;
      if (*p_ == ',') { ++p_; continue; }
      if (*p_ == ']') { ++p_; return true; }
      return false;
    }
  }
  static void put_utf8(std::string& s, uint32_t cp) {
    if (cp < 0x80) {
      s += static_cast<char>(cp);
    } else if (cp < 0x800) {
      s += static_cast<char>(0xC0 | (cp >> 6));
      s += static_cast<char>(0x80 | (cp & 0x3F));
    } else if (cp < 0x10000) {
      s += static_cast<char>(0xE0 | (cp >> 12));
      s += static_cast<char>(0x80 | ((cp >> 6) & 0x3F));
      s += static_cast<char>(0x80 | (cp & 0x3F));
    } else {
      s += static_cast<char>(0xF0 | (cp >> 18));
      s += static_cast<char>(0x80 | ((cp >> 12) & 0x3F));
      s += static_cast<char>(0x80 | ((cp >> 6) & 0x3F));
      s += static_cast<char>(0x80 | (cp & 0x3F));
    }
  }
  bool hex4(uint32_t& v) {
    if (end_ - p_ < 4) return false;
    v = 0;
    for (int k = 0; k < 4; ++k) {
      char c = *p_++;
      v <<= 4;
      if (c >= '0' && c <= '9') v |= static_cast<uint32_t>(c - '0');
      else if (c >= 'a' && c <= 'f') v |= static_cast<uint32_t>(c - 'a' + 10);
      else if (c >= 'A' && c <= 'F') v |= static_cast<uint32_t>(c - 'A' + 10);
      else return false;
    }
    return true;
  }
  bool string(std::string& s) {
    ++p_;  // opening quote
    while (p_ < end_) {
      unsigned char c = static_cast<unsigned char>(*p_);
      if (c == '"') { ++p_; return true; }
      if (c < 0x20) return false;  // control characters must be escaped
      if (c != '\\') { s += static_cast<char>(c); ++p_; continue; }
      if (++p_ >= end_) return false;
      char e = *p_++;
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
          if (!hex4(cp)) return false;
          if (cp >= 0xD800 && cp < 0xDC00 && end_ - p_ >= 6 && p_[0] == '\\' && p_[1] == 'u') {
            const char* save = p_;
            p_ += 2;
            uint32_t lo;
            if (hex4(lo) && lo >= 0xDC00 && lo < 0xE000) {
              cp = 0x10000 + ((cp - 0xD800) << 10) + (lo - 0xDC00);
            } else {
              p_ = save;
            }
          }
          put_utf8(s, cp);
          break;
        }
        default: return false;
      }
    }
    return false;
  }
  bool number(Json& v) {
    const char* start = p_;
    if (p_ < end_ && *p_ == '-') ++p_;
    if (p_ >= end_) return false;
    if (*p_ == '0') {
      ++p_;
    } else if (*p_ >= '1' && *p_ <= '9') {
      while (p_ < end_ && *p_ >= '0' && *p_ <= '9') ++p_;
    } else {
      return false;
    }
    bool is_float = false;
    if (p_ < end_ && *p_ == '.') {
      is_float = true;
      ++p_;
      if (p_ >= end_ || *p_ < '0' || *p_ > '9') return false;
      while (p_ < end_ && *p_ >= '0' && *p_ <= '9') ++p_;
    }
    if (p_ < end_ && (*p_ == 'e' || *p_ == 'E')) {
      is_float = true;
      ++p_;
      if (p_ < end_ && (*p_ == '+' || *p_ == '-')) ++p_;
      if (p_ >= end_ || *p_ < '0' || *p_ > '9') return false;
      while (p_ < end_ && *p_ >= '0' && *p_ <= '9') ++p_;
    }
    if (is_float) {
      v.kind = Json::kFloat;
      auto r = std::from_chars(start, p_, v.f);
      return r.ec == std::errc() && r.ptr == p_ && std::isfinite(v.f);
    }
    v.kind = Json::kInt;
    auto r = std::from_chars(start, p_, v.i);
    return r.ec == std::errc() && r.ptr == p_;  // beyond int64: refused
  }
};

// Python's repr(float), which json.dumps writes: the shortest round-trip
// digits, positional for decimal exponents in (-4, 16], scientific outside.
void dump_float(double x, std::string& out) {
  if (std::signbit(x)) {
    out += '-';
    x = -x;
  }
  char buf[64];
  auto r = std::to_chars(buf, buf + sizeof(buf), x, std::chars_format::scientific);
  std::string sci(buf, r.ptr);
  size_t epos = sci.find('e');
  std::string digits;
  for (size_t k = 0; k < epos; ++k)
    if (sci[k] != '.') digits += sci[k];
  int exp10 = std::atoi(sci.c_str() + epos + 1);
  int decpt = exp10 + 1;
  const int nd = static_cast<int>(digits.size());
  if (decpt <= -4 || decpt > 16) {
    out += digits[0];
    if (nd > 1) {
      out += '.';
      out.append(digits, 1, std::string::npos);
    }
    int e = decpt - 1;
    out += 'e';
    out += e < 0 ? '-' : '+';
    int ae = e < 0 ? -e : e;
    if (ae < 10) out += '0';
    out += std::to_string(ae);
  } else if (decpt <= 0) {
    out += "0.";
    out.append(static_cast<size_t>(-decpt), '0');
    out += digits;
  } else if (decpt >= nd) {
    out += digits;
    out.append(static_cast<size_t>(decpt - nd), '0');
    out += ".0";
  } else {
    out.append(digits, 0, static_cast<size_t>(decpt));
    out += '.';
    out.append(digits, static_cast<size_t>(decpt), std::string::npos);
  }
}

// Decodes one UTF-8 sequence (also the 3-byte form of a lone surrogate).
uint32_t next_cp(const std::string& s, size_t& k) {
  unsigned char c = static_cast<unsigned char>(s[k]);
  if (c < 0x80) { ++k; return c; }
  int n = c >= 0xF0 ? 3 : c >= 0xE0 ? 2 : 1;
  uint32_t cp = c & (0x3F >> n);
  for (int j = 0; j < n && k + 1 < s.size(); ++j) cp = (cp << 6) | (static_cast<unsigned char>(s[++k]) & 0x3F);
  ++k;
  return cp;
}

void dump_string(const std::string& s, std::string& out) {
  static const char* hexd = "0123456789abcdef";
  auto u = [&](uint32_t v) {
    out += "\\u";
    for (int sh = 12; sh >= 0; sh -= 4) out += hexd[(v >> sh) & 0xF];
  };
  out += '"';
  for (size_t k = 0; k < s.size();) {
    uint32_t cp = next_cp(s, k);
    switch (cp) {
      case '"': out += "\\\""; break;
      case '\\': out += "\\\\"; break;
      case '\n': out += "\\n"; break;
      case '\r': out += "\\r"; break;
      case '\t': out += "\\t"; break;
      case '\b': out += "\\b"; break;
      case '\f': out += "\\f"; break;
      default:
        if (cp < 0x20 || cp > 0x7E) {  // json escapes everything outside ' '..'~'
          if (cp >= 0x10000) {
            uint32_t v = cp - 0x10000;
            u(0xD800 | (v >> 10));
            u(0xDC00 | (v & 0x3FF));
          } else {
            u(cp);
          }
        } else {
          out += static_cast<char>(cp);
        }
    }
  }
  out += '"';
}

// json.dumps(value, sort_keys=True, separators=(",", ":"), ensure_ascii=True).
void dump(const Json& v, std::string& out) {
  switch (v.kind) {
    case Json::kNull: out += "null"; break;
    case Json::kBool: out += v.b ? "true" : "false"; break;
    case Json::kInt: out += std::to_string(v.i); break;
    case Json::kFloat: dump_float(v.f, out); break;
    case Json::kString: dump_string(v.s, out); break;
    case Json::kArray:
      out += '[';
      for (size_t k = 0; k < v.a.size(); ++k) {
        if (k) out += ',';
        dump(v.a[k], out);
      }
      out += ']';
      break;
    case Json::kObject: {
      std::vector<const std::pair<std::string, Json>*> items;
      for (const auto& kv : v.o) items.push_back(&kv);
      // UTF-8 byte order is code point order, which is how Python sorts str keys
      std::stable_sort(items.begin(), items.end(), [](auto* x, auto* y) { return x->first < y->first; });
      out += '{';
      for (size_t k = 0; k < items.size(); ++k) {
        if (k) out += ',';
        dump_string(items[k]->first, out);
        out += ':';
        dump(items[k]->second, out);
      }
      out += '}';
      break;
    }
  }
}

bool has_duplicate_keys(const Json& v) {
  if (v.kind == Json::kArray) {
    for (const auto& x : v.a)
      if (has_duplicate_keys(x)) return true;
  } else if (v.kind == Json::kObject) {
    std::vector<std::string> keys;
    for (const auto& kv : v.o) {
      keys.push_back(kv.first);
      if (has_duplicate_keys(kv.second)) return true;
    }
    std::sort(keys.begin(), keys.end());
    if (std::adjacent_find(keys.begin(), keys.end()) != keys.end()) return true;
  }
  return false;
}

// Python's == between two decoded JSON values: numbers compare by value
// across bool / int / float, containers element by element, objects by key set.
bool numeric(const Json& v, double& out) {
  if (v.kind == Json::kBool) { out = v.b ? 1.0 : 0.0; return true; }
  if (v.kind == Json::kInt) { out = static_cast<double>(v.i); return true; }
  if (v.kind == Json::kFloat) { out = v.f; return true; }
  return false;
}

bool py_equal(const Json& x, const Json& y) {
  double dx, dy;
  if (numeric(x, dx) && numeric(y, dy)) {
    if (x.kind != Json::kFloat && y.kind != Json::kFloat) {
      int64_t ix = x.kind == Json::kBool ? x.b : x.i;
      int64_t iy = y.kind == Json::kBool ? y.b : y.i;
      return ix == iy;
    }
    return dx == dy;
  }
  if (x.kind != y.kind) return false;
  switch (x.kind) {
    case Json::kNull: return true;
    case Json::kString: return x.s == y.s;
    case Json::kArray:
      if (x.a.size() != y.a.size()) return false;
      for (size_t k = 0; k < x.a.size(); ++k)
        if (!py_equal(x.a[k], y.a[k])) return false;
      return true;
    case Json::kObject: {
      std::map<std::string, const Json*> mx, my;
      for (const auto& kv : x.o) mx[kv.first] = &kv.second;
      for (const auto& kv : y.o) my[kv.first] = &kv.second;
      if (mx.size() != my.size()) return false;
      for (const auto& kv : mx) {
        auto it = my.find(kv.first);
        if (it == my.end() || !py_equal(*kv.second, *it->second)) return false;
      }
      return true;
    }
    default: return false;
  }
}

// `value == integer` with Python semantics (None or a string never equal).
bool eq_int(const Json* v, int64_t want) {
  if (v == nullptr) return false;
  if (v->kind == Json::kInt) return v->i == want;
  if (v->kind == Json::kBool) return static_cast<int64_t>(v->b) == want;
  if (v->kind == Json::kFloat) return v->f == static_cast<double>(want);
  return false;
}

Json parse_literal(const char* text) {
  Json v;
  Parser p(text, std::strlen(text));
  p.parse(v);
  return v;
}

Json str_json(const std::string& s) {
  Json v;
  v.kind = Json::kString;
  v.s = s;
  return v;
}

// -------------------------------------------------------------- SHA-256 --
class Sha256 {
 public:
  Sha256() : ctx_(EVP_MD_CTX_new()) { EVP_DigestInit_ex(ctx_, EVP_sha256(), nullptr); }
  ~Sha256() { EVP_MD_CTX_free(ctx_); }
  Sha256(const Sha256&) = delete;
  Sha256& operator=(const Sha256&) = delete;
  void update(const void* p, size_t n) {
    const uint8_t* b = static_cast<const uint8_t*>(p);
    while (n > 0) {  // bounded chunks
      size_t step = std::min<size_t>(n, size_t{1} << 30);
      EVP_DigestUpdate(ctx_, b, step);
      b += step;
      n -= step;
    }
  }
  void final(uint8_t out[32]) {
    unsigned int len = 32;
    EVP_DigestFinal_ex(ctx_, out, &len);
  }

 private:
  EVP_MD_CTX* ctx_;
};

std::string hex(const uint8_t* d, size_t n) {
  static const char* hexd = "0123456789abcdef";
  std::string s(2 * n, '0');
  for (size_t k = 0; k < n; ++k) {
    s[2 * k] = hexd[d[k] >> 4];
    s[2 * k + 1] = hexd[d[k] & 0xF];
  }
  return s;
}

std::string sha256_hex(const std::string& s) {
  Sha256 h;
  h.update(s.data(), s.size());
  uint8_t d[32];
  h.final(d);
  return hex(d, 32);
}

// sha256 of json.dumps(value, sort_keys=True, separators=(",", ":")).
std::string sha256_json(const Json& v) {
  std::string out;
  dump(v, out);
  return sha256_hex(out);
}

bool hex64(const Json* v) {
  if (v == nullptr || v->kind != Json::kString || v->s.size() != 64) return false;
  for (char c : v->s)
    if (!((c >= '0' && c <= '9') || (c >= 'a' && c <= 'f'))) return false;
  return true;
}

// ------------------------------------------------------------ the format --
constexpr uint32_t kVersion = 1;
constexpr uint64_t kHeaderAlignment = 4096;
constexpr size_t kPrefixBytes = 96;
constexpr int kGroup = 128;
const char* const kQwenModelId = "Qwen/Qwen1.5-MoE-A2.7B";

const char* const kQ4Contract =
    R"({"bits":4,"nibble_order":"low_first_twos_complement","rounding":"nearest_even",)"
    R"("scale_dtype":"float32_le","signed_range":[-7,7],"zero_point":null})";
const char* const kTargetEncodings =
    R"({"bf16_le":{"bits":16,"byte_order":"little"},)"
    R"("q4_group128":{"bits":4,"group_size":128,"nibble_order":"low_first_twos_complement",)"
    R"("rounding":"nearest_even","scale_dtype":"float32_le","signed_range":[-7,7],"zero_point":null},)"
    R"("q8_group128":{"bits":8,"group_size":128,"rounding":"nearest_even","scale_dtype":"float32_le",)"
    R"("signed_range":[-127,127],"zero_point":null}})";

struct EncodingInfo {
  const char* name;
  int code;
  int bits;
  bool grouped;
};
const EncodingInfo kEncodings[3] = {{"bf16_le", UQM_BF16, 16, false},
                                    {"q4_group128", UQM_Q4, 4, true},
                                    {"q8_group128", UQM_Q8, 8, true}};  // sorted by name

const EncodingInfo* encoding_by_name(const Json* v) {
  if (v == nullptr || v->kind != Json::kString) return nullptr;
  for (const auto& e : kEncodings)
    if (v->s == e.name) return &e;
  return nullptr;
}

const EncodingInfo* encoding_by_code(int code) {
  for (const auto& e : kEncodings)
    if (e.code == code) return &e;
  return nullptr;
}

// a * b and a + b with overflow detection (Python integers do not overflow;
// a value this large cannot describe a valid pack)
bool mul_ok(int64_t a, int64_t b, int64_t& out) { return !__builtin_mul_overflow(a, b, &out); }
bool add_ok(int64_t a, int64_t b, int64_t& out) { return !__builtin_add_overflow(a, b, &out); }
int64_t ceil_div(int64_t a, int64_t b) { return a / b + (a % b != 0 ? 1 : 0); }
int64_t align_up(int64_t v, int64_t a) { return ceil_div(v, a) * a; }

bool safe_name(const std::string& s) {
  if (s.empty()) return false;
  for (char c : s)
    if (!((c >= 'A' && c <= 'Z') || (c >= 'a' && c <= 'z') || (c >= '0' && c <= '9') || c == '_' || c == '.' ||
          c == '-'))
      return false;
  return true;
}

bool parse_digits(const std::string& s, size_t& k, int64_t& v) {
  size_t start = k;
  v = 0;
  while (k < s.size() && s[k] >= '0' && s[k] <= '9') {
    if (v > (INT64_MAX - 9) / 10) return false;
    v = v * 10 + (s[k] - '0');
    ++k;
  }
  return k > start;
}

// model.layers.<L>.mlp.experts.<E>.<gate_proj|up_proj|down_proj>.weight
bool expert_name(const std::string& s, int64_t& layer, int64_t& expert, std::string& proj) {
  static const std::string a = "model.layers.", b = ".mlp.experts.", c = ".weight";
  if (s.compare(0, a.size(), a) != 0) return false;
  size_t k = a.size();
  if (!parse_digits(s, k, layer)) return false;
  if (s.compare(k, b.size(), b) != 0) return false;
  k += b.size();
  if (!parse_digits(s, k, expert)) return false;
  if (k >= s.size() || s[k] != '.') return false;
  ++k;
  for (const char* p : {"gate_proj", "up_proj", "down_proj"}) {
    size_t n = std::strlen(p);
    if (s.compare(k, n, p) == 0 && s.size() == k + n + c.size() && s.compare(k + n, c.size(), c) == 0) {
      proj = p;
      return true;
    }
  }
  return false;
}

// Python int(str) in base 10: optional surrounding whitespace and sign,
// digits with single underscores between them.
bool py_int(const std::string& s, int64_t& v) {
  size_t k = 0, n = s.size();
  auto space = [](char c) { return c == ' ' || c == '\t' || c == '\n' || c == '\r' || c == '\f' || c == '\v'; };
  while (k < n && space(s[k])) ++k;
  while (n > k && space(s[n - 1])) --n;
  bool neg = false;
  if (k < n && (s[k] == '+' || s[k] == '-')) neg = s[k++] == '-';
  if (k >= n) return false;
  int64_t acc = 0;
  bool prev_digit = false;
  for (; k < n; ++k) {
    char c = s[k];
    if (c == '_') {
      if (!prev_digit || k + 1 >= n || s[k + 1] < '0' || s[k + 1] > '9') return false;
      prev_digit = false;
      continue;
    }
    if (c < '0' || c > '9') return false;
    if (acc > (INT64_MAX - 9) / 10) return false;
    acc = acc * 10 + (c - '0');
    prev_digit = true;
  }
  v = neg ? -acc : acc;
  return true;
}

std::string repr(const std::string& s) { return "'" + s + "'"; }

struct TensorEntry {
  std::string name;
  const Json* meta = nullptr;
  const EncodingInfo* enc = nullptr;
  int64_t shape[4] = {0, 0, 0, 0};
  int ndim = 0;
  int64_t n = 0;
  int64_t start = 0, nbytes = 0, scale_at = 0, sbytes = 0, end = 0, lead_from = 0;
  int group = 0;
};

struct PinnedBuffer {
  void* p = nullptr;
  size_t bytes = 0;
  hipEvent_t done = nullptr;
  bool pending = false;
};

}  // namespace

struct uqm_pack {
  int fd = -1;
  const uint8_t* map = nullptr;
  size_t size = 0;
  int kind = UQM_PACK_EXPERT;
  std::string label;
  uint32_t hlen = 0;
  uint64_t poff = 0, plen = 0;
  Json header;
  int group = kGroup;
  int layers = 0, experts = 0;
  std::vector<int> layer_enc;  // TargetPack: encoding code per layer
  std::vector<TensorEntry> tensors;
  std::unordered_map<std::string, size_t> index;
  PinnedBuffer staging[2];

  ~uqm_pack() {
    for (auto& b : staging) {
      if (b.done != nullptr) {
        if (b.pending) (void)hipEventSynchronize(b.done);
        (void)hipEventDestroy(b.done);
      }
      if (b.p != nullptr) (void)hipHostFree(b.p);
    }
    if (map != nullptr) munmap(const_cast<uint8_t*>(map), size);
    if (fd >= 0) close(fd);
  }
};

namespace {

unsigned worker_count() {
  unsigned n = std::thread::hardware_concurrency();
  return std::max(1u, std::min(n == 0 ? 4u : n, 16u));
}

// Runs fn(k) for k in [0, n) on up to `threads` threads.
template <class F>
void parallel_for(size_t n, unsigned threads, F fn) {
  threads = static_cast<unsigned>(std::min<size_t>(threads, n));
  if (threads <= 1) {
    for (size_t k = 0; k < n; ++k) fn(k);
    return;
  }
  std::atomic<size_t> next{0};
  std::vector<std::thread> pool;
  for (unsigned t = 0; t < threads; ++t)
    pool.emplace_back([&] {
      for (size_t k; (k = next.fetch_add(1)) < n;) fn(k);
    });
  for (auto& th : pool) th.join();
}

bool all_zero(const uint8_t* p, size_t n) {
  for (size_t k = 0; k < n; ++k)
    if (p[k] != 0) return false;
  return true;
}

// The byte checks of one tensor in the reference's order: zero padding
// before, between and after, the SHA-256 of data + scales, then the payload
// semantics (formats.check_payload). Returns "" when clean.
std::string heavy_checks(const uqm_pack& pk, const TensorEntry& t) {
  const uint8_t* base = pk.map + pk.poff;
  const std::string what = pk.label + " tensor " + repr(t.name);
  if (!all_zero(base + t.lead_from, static_cast<size_t>(t.start - t.lead_from)))
    return pk.label + " tensor " + repr(t.name) + " leading padding must be zero";
  if (!all_zero(base + t.start + t.nbytes, static_cast<size_t>(t.scale_at - t.start - t.nbytes)))
    return pk.label + " tensor " + repr(t.name) + " data-to-scale padding must be zero";
  if (!all_zero(base + t.scale_at + t.sbytes, static_cast<size_t>(t.end - t.scale_at - t.sbytes)))
    return pk.label + " tensor " + repr(t.name) + " trailing padding must be zero";
  const uint8_t* data = base + t.start;
  const uint8_t* scales = base + t.scale_at;
  Sha256 h;
  h.update(data, static_cast<size_t>(t.nbytes));
  h.update(scales, static_cast<size_t>(t.sbytes));
  uint8_t d[32];
  h.final(d);
  const Json* want = t.meta->get("tensor_payload_sha256");
  if (want == nullptr || want->kind != Json::kString || want->s != hex(d, 32)) return what + " hash mismatch";
  if (t.enc->code == UQM_Q4) {
    bool reserved = false;
    for (int64_t k = 0; k < t.nbytes; ++k) {
      uint8_t b = data[k];
      reserved |= ((b & 0x0F) == 8) | ((b >> 4) == 8);
    }
    if (reserved) return what + " contains the reserved Q4 -8 code";
    if ((t.n & 1) && t.nbytes > 0 && (data[t.nbytes - 1] >> 4) != 0) return what + " has non-zero Q4 odd tail padding";
  }
  if (t.enc->grouped) {
    for (int64_t k = 0; k < t.sbytes / 4; ++k) {
      float s;
      std::memcpy(&s, scales + 4 * k, 4);
      if (!(std::isfinite(s) && s > 0.0f)) return what + " scales must be finite and positive";
    }
  }
  return "";
}

struct Expected {
  int kind;
  const char* model_id;
  const char* revision;
  const char* manifest;
  const char* policy;
};

// Metadata checks of tensor `t` (validate_tensor before the byte checks).
std::string tensor_layout(uqm_pack& pk, const Json& t, int64_t alignment, int64_t end_prev,
                          std::unordered_map<std::string, int>& seen, TensorEntry& e) {
  const std::string& L = pk.label;
  if (t.kind != Json::kObject) return L + " tensor header must be an object";
  const Json* name = t.get("name");
  if (pk.kind == UQM_PACK_EXPERT) {
    if (name == nullptr || name->kind != Json::kString || !safe_name(name->s) || seen.count(name->s))
      return "ExpertPack tensor names must be unique and safe";
    e.enc = encoding_by_code(UQM_Q4);
  } else {
    int64_t layer, expert;
    std::string proj;
    if (name == nullptr || name->kind != Json::kString || !expert_name(name->s, layer, expert, proj) ||
        seen.count(name->s))
      return "TargetPack tensor names must be unique fixed expert tensors";
    const Json* enc = t.get("encoding");
    const Json* lp = t.get("projection");
    bool layer_ok = layer < pk.layers && expert < pk.experts && eq_int(t.get("layer_index"), layer) &&
                    eq_int(t.get("expert_index"), expert) && lp != nullptr && lp->kind == Json::kString &&
                    lp->s == proj;
    const EncodingInfo* ei = encoding_by_name(enc);
    if (!layer_ok || ei == nullptr || ei->code != pk.layer_enc[static_cast<size_t>(layer)])
      return "TargetPack tensor " + repr(name->s) + " policy identity is invalid";
    e.enc = ei;
  }
  e.name = name->s;
  e.meta = &t;
  seen[e.name] = 1;
  const Json* shape = t.get("shape");
  bool shape_ok = shape != nullptr && shape->kind == Json::kArray && !shape->a.empty();
  int64_t n = 1;
  bool overflow = false;
  if (shape_ok) {
    for (const auto& d : shape->a) {
      if (d.kind != Json::kInt || d.i <= 0) {
        shape_ok = false;
        break;
      }
      if (!mul_ok(n, d.i, n)) overflow = true;
    }
  }
  if (!shape_ok) return L + " tensor " + repr(e.name) + " has invalid shape";
  const std::string layout_err = L + " tensor " + repr(e.name) + " layout is invalid";
  if (overflow) return layout_err;
  e.ndim = static_cast<int>(shape->a.size());
  for (int k = 0; k < std::min(e.ndim, 4); ++k) e.shape[k] = shape->a[static_cast<size_t>(k)].i;
  e.n = n;
  e.group = e.enc->grouped ? pk.group : 0;
  const char* data_field = pk.kind == UQM_PACK_EXPERT ? "packed" : "data";
  const Json* start = t.get((std::string(data_field) + "_offset").c_str());
  const Json* nbytes = t.get((std::string(data_field) + "_bytes").c_str());
  const Json* scale_at = t.get("scale_offset");
  const Json* sbytes = t.get("scale_bytes");
  const Json* end = t.get("storage_end_offset");
  for (const Json* v : {start, nbytes, scale_at, sbytes, end})
    if (v == nullptr || v->kind != Json::kInt) return layout_err;
  int64_t want_data = n;  // Q8: one byte per element
  if (e.enc->bits == 4) want_data = n / 2 + (n & 1);
  if (e.enc->bits == 16 && !mul_ok(n, 2, want_data)) return layout_err;
  int64_t want_scales = e.enc->grouped ? 4 * ceil_div(n, pk.group) : 0;
  int64_t want_groups = e.enc->grouped ? ceil_div(n, pk.group) : 0;
  e.start = start->i;
  e.nbytes = nbytes->i;
  e.scale_at = scale_at->i;
  e.sbytes = sbytes->i;
  e.end = end->i;
  bool group_ok = true;
  if (pk.kind == UQM_PACK_TARGET) {
    const Json* g = t.get("group_size");
    group_ok = e.enc->grouped ? eq_int(g, pk.group) : (g == nullptr || g->kind == Json::kNull);
  }
  int64_t s1, s2;
  if (!eq_int(t.get("element_count"), n) || e.nbytes != want_data || e.sbytes != want_scales ||
      !eq_int(t.get("group_count"), want_groups) || !group_ok || ((e.start % alignment) + alignment) % alignment ||
      e.start < end_prev || !add_ok(e.start, e.nbytes, s1) || e.scale_at != align_up(s1, 4) ||
      !add_ok(e.scale_at, e.sbytes, s2) || e.end != align_up(s2, alignment) ||
      e.end > static_cast<int64_t>(pk.plen))
    return layout_err;
  const Json* bpw = t.get("effective_bits_per_weight");
  double want_bpw = static_cast<double>((e.end - e.start) * 8) / static_cast<double>(n);
  double got;
  if (bpw == nullptr || !numeric(*bpw, got) || got != want_bpw)
    return L + " tensor " + repr(e.name) + " effective bpw is invalid";
  e.lead_from = end_prev;
  return "";
}

std::string validate(uqm_pack& pk, const Expected& want) {
  if (pk.size < kPrefixBytes) return "pack is shorter than its fixed prefix";
  const uint8_t* m = pk.map;
  uint32_t version, hlen;
  uint64_t poff, plen;
  std::memcpy(&version, m + 8, 4);
  std::memcpy(&hlen, m + 12, 4);
  std::memcpy(&poff, m + 16, 8);
  std::memcpy(&plen, m + 24, 8);
  int kind = std::memcmp(m, "UQMOEPK1", 8) == 0 ? UQM_PACK_EXPERT
             : std::memcmp(m, "UQMOTPK1", 8) == 0 ? UQM_PACK_TARGET
                                                  : -1;
  if (kind < 0 || version != kVersion || (want.kind != UQM_PACK_ANY && kind != want.kind)) {
    int k = want.kind != UQM_PACK_ANY ? want.kind : kind >= 0 ? kind : UQM_PACK_EXPERT;
    return std::string(k == UQM_PACK_TARGET ? "TargetPack" : "ExpertPack") + " magic/version mismatch";
  }
  pk.kind = kind;
  pk.label = kind == UQM_PACK_TARGET ? "TargetPack" : "ExpertPack";
  const std::string& L = pk.label;
  if (poff % kHeaderAlignment || poff < kPrefixBytes + hlen) return L + " payload offset/alignment is invalid";
  if (poff + plen != pk.size || poff + plen < poff) return L + " payload length does not match file size";
  const uint8_t* hb = m + kPrefixBytes;
  {
    Sha256 h;
    h.update(hb, hlen);
    uint8_t d[32];
    h.final(d);
    if (std::memcmp(d, m + 32, 32) != 0) return L + " header hash mismatch";
  }
  if (!all_zero(hb + hlen, poff - kPrefixBytes - hlen)) return L + " header padding must be zero";
  pk.hlen = hlen;
  pk.poff = poff;
  pk.plen = plen;

  // the payload hash on its own thread; its error outranks every later one
  bool payload_ok = false;
  std::thread payload_thread([&] {
    Sha256 h;
    h.update(m + poff, plen);
    uint8_t d[32];
    h.final(d);
    payload_ok = std::memcmp(d, m + 64, 32) == 0;
  });
  std::string err;
  auto finish = [&](std::string e) {
    if (payload_thread.joinable()) payload_thread.join();
    return payload_ok ? e : L + " payload hash mismatch";
  };

  // UTF-8 check of the raw header (Python decodes it before parsing)
  for (size_t k = 0; k < hlen;) {
    uint8_t c = hb[k];
    int n = c < 0x80 ? 0 : (c >> 5) == 6 ? 1 : (c >> 4) == 14 ? 2 : (c >> 3) == 30 ? 3 : -1;
    if (n < 0 || k + static_cast<size_t>(n) >= hlen) return finish(L + " header is not canonical JSON");
    for (int j = 1; j <= n; ++j)
      if ((hb[k + j] & 0xC0) != 0x80) return finish(L + " header is not canonical JSON");
    k += n + 1;
  }
  Parser parser(reinterpret_cast<const char*>(hb), hlen);
  if (!parser.parse(pk.header)) return finish(L + " header is not canonical JSON");
  {
    std::string canon;
    dump(pk.header, canon);
    if (pk.header.kind != Json::kObject || has_duplicate_keys(pk.header) || canon.size() != hlen ||
        std::memcmp(canon.data(), hb, hlen) != 0)
      return finish(L + " header JSON is not canonical");
  }
  const Json& H = pk.header;
  const char* fmt = kind == UQM_PACK_EXPERT ? "canonical_q4_symmetric_grouped" : "mixed_precision_target_pack";
  const Json* fmtv = H.get("format");
  if (!eq_int(H.get("schema_version"), kVersion) || fmtv == nullptr || !fmtv->is_str(fmt))
    return finish(L + " header schema is unsupported");
  const Json* model = H.get("model");
  const Json* tensors = H.get("tensors");
  if (model == nullptr || model->kind != Json::kObject || tensors == nullptr || tensors->kind != Json::kArray)
    return finish(L + " header is incomplete");
  {
    Json ident;
    ident.kind = Json::kObject;
    for (const char* k : {"model_id", "model_revision", "model_manifest_sha256"}) {
      const Json* v = model->get(k);
      ident.o.emplace_back(k, v != nullptr ? *v : str_json(""));
    }
    const Json* have = model->get("model_identity_sha256");
    if (have == nullptr || have->kind != Json::kString || have->s != sha256_json(ident))
      return finish(L + " model identity hash mismatch");
  }
  const Json* policy = kind == UQM_PACK_TARGET ? H.get("policy") : nullptr;
  {
    struct Check {
      const char* want;
      const Json* seen;
      const char* what;
    };
    const Json* policy_id = policy != nullptr && policy->kind == Json::kObject ? policy->get("policy_id") : nullptr;
    Check checks[4] = {{want.model_id, model->get("model_id"), "model id"},
                       {want.revision, model->get("model_revision"), "model revision"},
                       {want.manifest, model->get("model_manifest_sha256"), "model manifest"},
                       {kind == UQM_PACK_TARGET ? want.policy : nullptr, policy_id, "policy id"}};
    for (const auto& c : checks)
      if (c.want != nullptr && (c.seen == nullptr || c.seen->kind != Json::kString || c.seen->s != c.want))
        return finish(L + " " + c.what + " mismatch");
  }
  const Json* mid = model->get("model_id");
  const bool qwen = mid != nullptr && mid->is_str(kQwenModelId);
  pk.layers = qwen ? 24 : 16;
  pk.experts = qwen ? 60 : 64;
  if (kind == UQM_PACK_EXPERT) {
    const Json* q = H.get("quantization");
    const Json* g = q != nullptr && q->kind == Json::kObject ? q->get("group_size") : nullptr;
    Json expect = parse_literal(kQ4Contract);
    expect.o.emplace_back("group_size", g != nullptr ? *g : Json{});
    if (q == nullptr || !py_equal(*q, expect) || g == nullptr || g->kind != Json::kInt || g->i <= 0 ||
        g->i > INT32_MAX)
      return finish("ExpertPack quantization contract mismatch");
    pk.group = static_cast<int>(g->i);
  } else {
    const char* model_name = qwen ? "Qwen" : "OLMoE";
    const Json* le = policy != nullptr && policy->kind == Json::kObject ? policy->get("layer_encodings") : nullptr;
    if (le == nullptr || le->kind != Json::kObject) return finish("TargetPack layer policy is invalid");
    std::map<int64_t, const Json*> by_layer;  // dict comprehension: later keys replace earlier ones
    for (const auto& kv : le->o) {
      int64_t idx;
      if (!py_int(kv.first, idx)) return finish("TargetPack layer policy is invalid");
      by_layer[idx] = &kv.second;
    }
    const Json* pid = policy->get("policy_id");
    if (pid == nullptr || pid->kind != Json::kString || pid->s.empty())
      return finish("TargetPack policy id must be non-empty");
    bool complete = static_cast<int>(by_layer.size()) == pk.layers;
    for (const auto& kv : by_layer) complete = complete && kv.first >= 0 && kv.first < pk.layers;
    if (!complete)
      return finish(std::string("TargetPack policy must assign every ") + model_name + " layer exactly once");
    for (const auto& kv : by_layer)
      if (encoding_by_name(kv.second) == nullptr) return finish("TargetPack policy contains an unsupported encoding");
    const Json* ev = policy->get("policy_evidence_sha256");
    if (!hex64(ev)) return finish("TargetPack policy evidence identity must be SHA-256");
    Json layers_obj;
    layers_obj.kind = Json::kObject;
    pk.layer_enc.assign(static_cast<size_t>(pk.layers), UQM_Q4);
    for (int l = 0; l < pk.layers; ++l) {
      const Json* v = by_layer[l];
      layers_obj.o.emplace_back(std::to_string(l), *v);
      pk.layer_enc[static_cast<size_t>(l)] = encoding_by_name(v)->code;
    }
    Json ident;
    ident.kind = Json::kObject;
    ident.o.emplace_back("policy_id", *pid);
    ident.o.emplace_back("layer_encodings", layers_obj);
    ident.o.emplace_back("policy_evidence_sha256", *ev);
    Json expect = ident;
    expect.o.emplace_back("policy_identity_sha256", str_json(sha256_json(ident)));
    if (!py_equal(*policy, expect)) return finish("TargetPack policy identity hash mismatch");
    const Json* encs = H.get("encodings");
    if (encs == nullptr || !py_equal(*encs, parse_literal(kTargetEncodings)))
      return finish("TargetPack encoding contract mismatch");
    pk.group = kGroup;
  }
  const Json* align = H.get("tensor_alignment_bytes");
  if (align == nullptr || align->kind != Json::kInt || align->i <= 0 || (align->i & (align->i - 1)))
    return finish("alignment must be a positive power of two");
  const int64_t alignment = align->i;
  if (tensors->a.empty() || !eq_int(H.get("tensor_count"), static_cast<int64_t>(tensors->a.size())))
    return finish(L + " tensor count is inconsistent");

  // metadata of every tensor in order, up to the first violation
  std::unordered_map<std::string, int> seen;
  std::string meta_err;
  int64_t end_prev = 0;
  int counts[3] = {0, 0, 0};  // bf16, q4, q8
  pk.tensors.clear();
  for (const auto& t : tensors->a) {
    TensorEntry e;
    meta_err = tensor_layout(pk, t, alignment, end_prev, seen, e);
    if (!meta_err.empty()) break;
    end_prev = e.end;
    counts[e.enc - kEncodings]++;
    pk.tensors.push_back(std::move(e));
  }
  // byte checks of the tensors before it, in parallel; the first in order wins
  std::vector<std::string> heavy(pk.tensors.size());
  parallel_for(pk.tensors.size(), worker_count(), [&](size_t k) { heavy[k] = heavy_checks(pk, pk.tensors[k]); });
  for (const auto& h : heavy)
    if (!h.empty()) return finish(h);
  if (!meta_err.empty()) return finish(meta_err);
  if (end_prev != static_cast<int64_t>(plen)) return finish(L + " payload has unclaimed trailing bytes");
  if (kind == UQM_PACK_TARGET) {
    Json expect;
    expect.kind = Json::kObject;
    for (int k = 0; k < 3; ++k) {
      Json c;
      c.kind = Json::kInt;
      c.i = counts[k];
      expect.o.emplace_back(kEncodings[k].name, c);
    }
    const Json* have = H.get("encoding_tensor_counts");
    if (have == nullptr || !py_equal(*have, expect)) return finish("TargetPack encoding tensor counts are inconsistent");
  }
  std::string done = finish("");
  if (!done.empty()) return done;
  for (size_t k = 0; k < pk.tensors.size(); ++k) pk.index.emplace(pk.tensors[k].name, k);
  return "";
}

int pack_fail(const std::string& msg) { return uqm::api_fail(UQM_ERR_PACK, "%s", msg.c_str()); }

int hip_fail(hipError_t e, const char* what) {
  return uqm::api_fail(UQM_ERR_HIP, "%s: %s", what, hipGetErrorString(e));
}

const TensorEntry* find(const uqm_pack* pk, const std::string& name) {
  auto it = pk->index.find(name);
  return it == pk->index.end() ? nullptr : &pk->tensors[it->second];
}

constexpr size_t kStagingBytes = size_t{32} << 20;

}  // namespace

extern "C" {

int uqm_pack_open(const char* path, int32_t expected_kind, const char* expected_model_id,
                  const char* expected_model_revision, const char* expected_model_manifest_sha256,
                  const char* expected_policy_id, uqm_pack** pack) {
  if (path == nullptr || pack == nullptr) return uqm::api_fail(UQM_ERR_ARGUMENT, "path and pack must not be NULL");
  if (expected_kind < UQM_PACK_ANY || expected_kind > UQM_PACK_TARGET)
    return uqm::api_fail(UQM_ERR_ARGUMENT, "unknown pack kind %d", expected_kind);
  *pack = nullptr;
  std::unique_ptr<uqm_pack> pk(new uqm_pack());
  const char* label = expected_kind == UQM_PACK_TARGET ? "TargetPack" : expected_kind == UQM_PACK_EXPERT ? "ExpertPack" : "pack";
  pk->fd = open(path, O_RDONLY | O_CLOEXEC);
  struct stat st;
  if (pk->fd < 0 || fstat(pk->fd, &st) != 0)
    return pack_fail(std::string("cannot map ") + label + " " + path + ": " + std::strerror(errno));
  pk->size = static_cast<size_t>(st.st_size);
  if (pk->size == 0) return pack_fail(std::string("cannot map ") + label + " " + path + ": cannot mmap an empty file");
  void* m = mmap(nullptr, pk->size, PROT_READ, MAP_PRIVATE, pk->fd, 0);
  if (m == MAP_FAILED) return pack_fail(std::string("cannot map ") + label + " " + path + ": " + std::strerror(errno));
  pk->map = static_cast<const uint8_t*>(m);
  madvise(m, pk->size, MADV_WILLNEED);
  Expected want{expected_kind, expected_model_id, expected_model_revision, expected_model_manifest_sha256,
                expected_policy_id};
  std::string err = validate(*pk, want);
  if (!err.empty()) return pack_fail(err);
  *pack = pk.release();
  return UQM_OK;
}

int uqm_pack_close(uqm_pack* pack) {
  delete pack;
  return UQM_OK;
}

int uqm_pack_info(const uqm_pack* pack, int32_t* kind, uint64_t* payload_offset, uint64_t* payload_length,
                  int32_t* group_size) {
  if (pack == nullptr) return uqm::api_fail(UQM_ERR_ARGUMENT, "pack is NULL");
  if (kind) *kind = pack->kind;
  if (payload_offset) *payload_offset = pack->poff;
  if (payload_length) *payload_length = pack->plen;
  if (group_size) *group_size = pack->group;
  return UQM_OK;
}

int uqm_pack_header(const uqm_pack* pack, const char** json, size_t* length) {
  if (pack == nullptr || json == nullptr || length == nullptr)
    return uqm::api_fail(UQM_ERR_ARGUMENT, "pack, json and length must not be NULL");
  *json = reinterpret_cast<const char*>(pack->map + kPrefixBytes);
  *length = pack->hlen;
  return UQM_OK;
}

int uqm_pack_lookup(const uqm_pack* pack, const char* name, uqm_pack_tensor* tensor) {
  if (pack == nullptr || name == nullptr || tensor == nullptr)
    return uqm::api_fail(UQM_ERR_ARGUMENT, "pack, name and tensor must not be NULL");
  const TensorEntry* t = find(pack, name);
  if (t == nullptr) return pack_fail(pack->label + " has no tensor " + repr(name));
  if (t->ndim > 4) return pack_fail("tensor " + repr(name) + " has more than four dimensions");
  std::memset(tensor, 0, sizeof(*tensor));
  const uint8_t* base = pack->map + pack->poff;
  tensor->data = base + t->start;
  tensor->data_bytes = static_cast<uint64_t>(t->nbytes);
  tensor->scales = t->sbytes > 0 ? base + t->scale_at : nullptr;
  tensor->scale_bytes = static_cast<uint64_t>(t->sbytes);
  tensor->element_count = t->n;
  tensor->ndim = t->ndim;
  for (int k = 0; k < t->ndim; ++k) tensor->shape[k] = t->shape[k];
  tensor->encoding = t->enc->code;
  tensor->group_size = t->group;
  return UQM_OK;
}

int uqm_pack_layer_encoding(const uqm_pack* pack, int64_t layer, int32_t* encoding) {
  if (pack == nullptr || encoding == nullptr) return uqm::api_fail(UQM_ERR_ARGUMENT, "pack and encoding must not be NULL");
  if (pack->kind == UQM_PACK_EXPERT) {
    *encoding = UQM_Q4;
    return UQM_OK;
  }
  if (layer < 0 || layer >= pack->layers)
    return pack_fail("TargetPack layer index must be in [0, " + std::to_string(pack->layers - 1) + "]");
  *encoding = pack->layer_enc[static_cast<size_t>(layer)];
  return UQM_OK;
}

int uqm_pack_stage_projection(uqm_pack* pack, int64_t layer, int32_t projection, int64_t num_experts,
                              void* data_dst, void* scales_dst, void* stream) {
  if (pack == nullptr || data_dst == nullptr) return uqm::api_fail(UQM_ERR_ARGUMENT, "pack and data_dst must not be NULL");
  if (projection < UQM_PROJ_GATE || projection > UQM_PROJ_DOWN)
    return uqm::api_fail(UQM_ERR_ARGUMENT, "unknown projection %d", projection);
  if (num_experts <= 0 || num_experts > 4096) return uqm::api_fail(UQM_ERR_ARGUMENT, "num_experts must be in [1, 4096]");
  int32_t enc;
  if (int rc = uqm_pack_layer_encoding(pack, layer, &enc)) return rc;
  static const char* const names[3] = {"gate_proj", "up_proj", "down_proj"};
  std::vector<const TensorEntry*> ts(static_cast<size_t>(num_experts));
  for (int64_t e = 0; e < num_experts; ++e) {
    std::string name = "model.layers." + std::to_string(layer) + ".mlp.experts." + std::to_string(e) + "." +
                       names[projection] + ".weight";
    const TensorEntry* t = find(pack, name);
    if (t == nullptr) return pack_fail(pack->label + " has no tensor " + repr(name));
    if (t->enc->code != enc)
      return pack_fail("tensor " + repr(name) + " is " + t->enc->name + ", layer " + std::to_string(layer) + " is " +
                       encoding_by_code(enc)->name);
    if (t->ndim != 2) return pack_fail("expert tensor " + repr(name) + " is not a matrix");
    const TensorEntry* t0 = e == 0 ? t : ts[0];
    if (t->shape[0] != t0->shape[0] || t->shape[1] != t0->shape[1])
      return pack_fail("expert tensor " + repr(name) + " has unexpected shape");
    if (t->nbytes != t0->nbytes || t->sbytes != t0->sbytes)
      return pack_fail("layer " + std::to_string(layer) + " " + names[projection] + " tensors differ in size");
    ts[static_cast<size_t>(e)] = t;
  }
  const size_t db = static_cast<size_t>(ts[0]->nbytes), sb = static_cast<size_t>(ts[0]->sbytes);
  if (sb > 0 && scales_dst == nullptr) return uqm::api_fail(UQM_ERR_ARGUMENT, "scales_dst is NULL for a grouped encoding");
  hipStream_t s = static_cast<hipStream_t>(stream);
  hipError_t he;
  for (auto& b : pack->staging) {
    if (b.p == nullptr) {
      if ((he = hipHostMalloc(&b.p, kStagingBytes, hipHostMallocDefault)) != hipSuccess) {
        b.p = nullptr;
        return hip_fail(he, "pinned staging buffer");
      }
      b.bytes = kStagingBytes;
    }
    if (b.done == nullptr && (he = hipEventCreateWithFlags(&b.done, hipEventDisableTiming)) != hipSuccess) {
      b.done = nullptr;
      return hip_fail(he, "staging event");
    }
  }
  // Two streams of (source, destination offset, bytes) pieces: the experts'
  // data into data_dst, then their scales into scales_dst. Each pinned
  // buffer fill gathers whole pieces (split when one piece exceeds a buffer).
  struct Piece {
    const uint8_t* src;
    uint8_t* dst;
    size_t bytes;
  };
  std::vector<Piece> pieces;
  const uint8_t* base = pack->map + pack->poff;
  for (int64_t e = 0; e < num_experts; ++e)
    pieces.push_back({base + ts[e]->start, static_cast<uint8_t*>(data_dst) + e * db, db});
  for (int64_t e = 0; sb > 0 && e < num_experts; ++e)
    pieces.push_back({base + ts[e]->scale_at, static_cast<uint8_t*>(scales_dst) + e * sb, sb});
  int which = 0;
  size_t k = 0, off = 0;  // next piece, bytes of it already staged
  const unsigned threads = worker_count();
  while (k < pieces.size()) {
    PinnedBuffer& b = pack->staging[which];
    if (b.pending) {
      if ((he = hipEventSynchronize(b.done)) != hipSuccess) return hip_fail(he, "staging wait");
      b.pending = false;
    }
    // fill: a run of pieces that are contiguous on the device goes in one copy
    struct Job {
      const uint8_t* src;
      size_t at, bytes;
    };
    std::vector<Job> jobs;
    uint8_t* dst0 = pieces[k].dst + off;
    size_t used = 0;
    while (k < pieces.size() && used < b.bytes && pieces[k].dst + off == dst0 + used) {
      size_t take = std::min(pieces[k].bytes - off, b.bytes - used);
      jobs.push_back({pieces[k].src + off, used, take});
      used += take;
      off += take;
      if (off == pieces[k].bytes) {
        ++k;
        off = 0;
      }
    }
    uint8_t* host = static_cast<uint8_t*>(b.p);
    parallel_for(jobs.size(), threads, [&](size_t j) { std::memcpy(host + jobs[j].at, jobs[j].src, jobs[j].bytes); });
    if ((he = hipMemcpyAsync(dst0, host, used, hipMemcpyHostToDevice, s)) != hipSuccess) return hip_fail(he, "staging copy");
    if ((he = hipEventRecord(b.done, s)) != hipSuccess) return hip_fail(he, "staging record");
    b.pending = true;
    which ^= 1;
  }
  for (auto& b : pack->staging) {
    if (b.pending) {
      if ((he = hipEventSynchronize(b.done)) != hipSuccess) return hip_fail(he, "staging wait");
      b.pending = false;
    }
  }
  return UQM_OK;
}

}  // extern "C"
