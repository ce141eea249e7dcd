// Model-level driver on the GPU engine: pipeline::quantize_model (src/pipeline.rs:79-227) and
// pipeline::dequantize_packed (src/pipeline.rs:239-275), with the safetensors side of src/io.rs
// (memory-mapped shards, the Hessian store with aliases, the packed container's six tensors).
//
// Every per-weight operation runs on the device: the F16 / BF16 / F32 decode of weights and
// Hessians, the non-finite scan, quantize_layer, the dequantized output in the checkpoint dtype and
// the bit-packing. The host parses headers, orders the jobs, and writes the files.
//
// safetensors layout written here: 8-byte little-endian header length, a JSON header
// {"__metadata__": {...}, "<name>": {"dtype", "shape", "data_offsets"}, ...} padded with spaces to a
// multiple of 8, then the tensor bytes, ordered by dtype (widest first) and name as the safetensors
// crate does. Metadata keys are written sorted (the reference's writer takes a HashMap's order).
#include <fcntl.h>
#include <hip/hip_runtime.h>
#include <sys/mman.h>
#include <sys/stat.h>
#include <unistd.h>

#include <algorithm>
#include <cerrno>
#include <chrono>
#include <cmath>
#include <cstdio>
#include <cstdlib>
#include <cstring>
#include <map>
#include <memory>
#include <string>
#include <vector>

#include "cdclq.h"
#include "ctx.h"
#include "kernels.h"

namespace {

using namespace cdclq;

double now_secs() {
  using namespace std::chrono;
  return duration<double>(steady_clock::now().time_since_epoch()).count();
}

// ------------------------------------------------------------------ minimal JSON
struct JVal {
  enum Kind { NUL, BOOL, NUM, STR, ARR, OBJ } kind = NUL;
  bool b = false;
  std::string text;  // number text or string value
  std::vector<JVal> arr;
  std::vector<std::pair<std::string, JVal>> obj;
  const JVal* get(const std::string& k) const {
    for (const auto& kv : obj)
      if (kv.first == k) return &kv.second;
    return nullptr;
  }
};

struct JParser {
  const char* p;
  const char* e;
  std::string err;
  void ws() {
    while (p < e && (*p == ' ' || *p == '\t' || *p == '\n' || *p == '\r')) ++p;
  }
  bool fail(const char* m) {
    if (err.empty()) err = m;
    return false;
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
  bool hex4(uint32_t* v) {
    if (e - p < 4) return fail("bad \\u escape");
    *v = 0;
    for (int i = 0; i < 4; ++i) {
      const char c = *p++;
      *v <<= 4;
      if (c >= '0' && c <= '9') *v |= (uint32_t)(c - '0');
      else if (c >= 'a' && c <= 'f') *v |= (uint32_t)(c - 'a' + 10);
      else if (c >= 'A' && c <= 'F') *v |= (uint32_t)(c - 'A' + 10);
      else return fail("bad \\u escape");
    }
    return true;
  }
  bool str(std::string& out) {
    if (p >= e || *p != '"') return fail("expected string");
    ++p;
    while (p < e && *p != '"') {
      if ((unsigned char)*p < 0x20) return fail("control character in string");
      if (*p != '\\') {
        out += *p++;
        continue;
      }
      if (++p >= e) return fail("bad escape");
      const char c = *p++;
      switch (c) {
        case '"': out += '"'; break;
        case '\\': out += '\\'; break;
        case '/': out += '/'; break;
        case 'b': out += '\b'; break;
        case 'f': out += '\f'; break;
        case 'n': out += '\n'; break;
        case 'r': out += '\r'; break;
        case 't': out += '\t'; break;
        case 'u': {
          uint32_t v;
          if (!hex4(&v)) return false;
          if (v >= 0xD800 && v < 0xDC00) {
            uint32_t lo;
            if (e - p < 6 || p[0] != '\\' || p[1] != 'u') return fail("lone surrogate");
            p += 2;
            if (!hex4(&lo) || lo < 0xDC00 || lo >= 0xE000) return fail("bad surrogate pair");
            v = 0x10000 + ((v - 0xD800) << 10) + (lo - 0xDC00);
          } else if (v >= 0xDC00 && v < 0xE000) {
            return fail("lone surrogate");
          }
          put_utf8(out, v);
          break;
        }
        default:
          return fail("bad escape");
      }
    }
    if (p >= e) return fail("unterminated string");
    ++p;
    return true;
  }
  bool value(JVal& v, int depth) {
    if (depth > 64) return fail("nesting too deep");
    ws();
    if (p >= e) return fail("unexpected end");
    if (*p == '{') {
      v.kind = JVal::OBJ;
      ++p;
      ws();
      if (p < e && *p == '}') {
        ++p;
        return true;
      }
      for (;;) {
        ws();
        std::string k;
        if (!str(k)) return false;
        ws();
        if (p >= e || *p != ':') return fail("expected ':'");
        ++p;
        JVal c;
        if (!value(c, depth + 1)) return false;
        v.obj.emplace_back(std::move(k), std::move(c));
        ws();
        if (p < e && *p == ',') {
          ++p;
          continue;
        }
        if (p < e && *p == '}') {
          ++p;
          return true;
        }
        return fail("expected ',' or '}'");
      }
    }
    if (*p == '[') {
      v.kind = JVal::ARR;
      ++p;
      ws();
      if (p < e && *p == ']') {
        ++p;
        return true;
      }
      for (;;) {
        JVal c;
        if (!value(c, depth + 1)) return false;
        v.arr.push_back(std::move(c));
        ws();
        if (p < e && *p == ',') {
          ++p;
          continue;
        }
        if (p < e && *p == ']') {
          ++p;
          return true;
        }
        return fail("expected ',' or ']'");
      }
    }
    if (*p == '"') {
      v.kind = JVal::STR;
      return str(v.text);
    }
    if (e - p >= 4 && !std::strncmp(p, "true", 4)) {
      v.kind = JVal::BOOL;
      v.b = true;
      p += 4;
      return true;
    }
    if (e - p >= 5 && !std::strncmp(p, "false", 5)) {
      v.kind = JVal::BOOL;
      p += 5;
      return true;
    }
    if (e - p >= 4 && !std::strncmp(p, "null", 4)) {
      p += 4;
      return true;
    }
    const char* s = p;
    if (p < e && *p == '-') ++p;
    while (p < e && ((*p >= '0' && *p <= '9') || *p == '.' || *p == 'e' || *p == 'E' || *p == '+' || *p == '-')) ++p;
    if (p == s) return fail("unexpected character");
    v.kind = JVal::NUM;
    v.text.assign(s, p);
    return true;
  }
};

bool parse_json(const char* s, size_t len, JVal& out, std::string& err) {
  JParser jp{s, s + len, {}};
  if (!jp.value(out, 0)) {
    err = jp.err;
    return false;
  }
  jp.ws();
  if (jp.p != jp.e) {
    err = "trailing characters";
    return false;
  }
  return true;
}

bool json_uint(const JVal& v, uint64_t* out) {
  if (v.kind != JVal::NUM || v.text.empty()) return false;
  uint64_t x = 0;
  for (char c : v.text) {
    if (c < '0' || c > '9') return false;
    if (x > (UINT64_MAX - (uint64_t)(c - '0')) / 10) return false;
    x = x * 10 + (uint64_t)(c - '0');
  }
  *out = x;
  return true;
}

void json_escape(std::string& o, const std::string& s) {
  o += '"';
  for (unsigned char c : s) {
    switch (c) {
      case '"': o += "\\\""; break;
      case '\\': o += "\\\\"; break;
      case '\n': o += "\\n"; break;
      case '\r': o += "\\r"; break;
      case '\t': o += "\\t"; break;
      case '\b': o += "\\b"; break;
      case '\f': o += "\\f"; break;
      default:
        if (c < 0x20) {
          char b[8];
          std::snprintf(b, sizeof b, "\\u%04x", c);
          o += b;
        } else {
          o += (char)c;
        }
    }
  }
  o += '"';
}

// shortest round-trip digits of v (> 0, finite) and the decimal exponent of the first digit
void shortest_digits(double v, std::string& digits, int& exp10) {
  char buf[64];
  for (int p = 0; p < 17; ++p) {
    std::snprintf(buf, sizeof buf, "%.*e", p, v);
    if (std::strtod(buf, nullptr) == v) break;
  }
  std::string s(buf);
  const size_t epos = s.find('e');
  exp10 = std::atoi(s.c_str() + epos + 1);
  digits.clear();
  for (size_t i = 0; i < epos; ++i)
    if (s[i] != '.') digits += s[i];
  while (digits.size() > 1 && digits.back() == '0') digits.pop_back();
}

// serde_json's f64 text (ryu): shortest digits; fixed notation while the decimal point stays within
// 16 digits of the first one and the value is >= 1e-5, else d.ddde<exp>; integral values end ".0".
std::string json_f64(double v) {
  if (!std::isfinite(v)) return "null";
  if (v == 0.0) return std::signbit(v) ? "-0.0" : "0.0";
  std::string sign = v < 0 ? "-" : "";
  std::string d;
  int e10;
  shortest_digits(std::fabs(v), d, e10);
  const int n = (int)d.size();
  const int kk = e10 + 1;  // digits before the decimal point
  std::string out;
  if (kk >= n && kk <= 16) {
    out = d + std::string(kk - n, '0') + ".0";
  } else if (kk > 0 && kk <= 16) {
    out = d.substr(0, kk) + "." + d.substr(kk);
  } else if (kk > -5 && kk <= 0) {
    out = "0." + std::string(-kk, '0') + d;
  } else if (n == 1) {
    out = d + "e" + std::to_string(kk - 1);
  } else {
    out = d.substr(0, 1) + "." + d.substr(1) + "e" + std::to_string(kk - 1);
  }
  return sign + out;
}

// Rust `{:?}` of an f64: decimal with at least one fractional digit for 1e-4 <= |v| < 1e16, else
// the shortest exponential form ("1e-5", "1.5e20").
std::string rust_debug_f64(double v) {
  if (std::isnan(v)) return "NaN";
  if (std::isinf(v)) return v < 0 ? "-inf" : "inf";
  if (v == 0.0) return std::signbit(v) ? "-0.0" : "0.0";
  const std::string sign = v < 0 ? "-" : "";
  const double a = std::fabs(v);
  std::string d;
  int e10;
  shortest_digits(a, d, e10);
  const int n = (int)d.size();
  if (a >= 1e-4 && a < 1e16) {
    const int kk = e10 + 1;
    std::string out;
    if (kk >= n) out = d + std::string(kk - n, '0') + ".0";
    else if (kk > 0) out = d.substr(0, kk) + "." + d.substr(kk);
    else out = "0." + std::string(-kk, '0') + d;
    return sign + out;
  }
  return sign + d.substr(0, 1) + (n > 1 ? "." + d.substr(1) : std::string()) + "e" + std::to_string(e10);
}

// Rust `{}` of an f32 (shortest digits, no exponent)
std::string rust_display_f32(float v) {
  if (std::isnan(v)) return "NaN";
  if (std::isinf(v)) return v < 0 ? "-inf" : "inf";
  if (v == 0.0f) return std::signbit(v) ? "-0" : "0";
  char buf[64];
  for (int p = 0; p < 10; ++p) {
    std::snprintf(buf, sizeof buf, "%.*e", p, (double)v);
    if (std::strtof(buf, nullptr) == v) break;
  }
  std::string s(buf);
  const bool neg = s[0] == '-';
  if (neg) s = s.substr(1);
  const size_t epos = s.find('e');
  const int ex = std::atoi(s.c_str() + epos + 1);
  std::string d;
  for (size_t i = 0; i < epos; ++i)
    if (s[i] != '.') d += s[i];
  while (d.size() > 1 && d.back() == '0') d.pop_back();
  const int point = ex + 1;
  std::string out;
  if (point <= 0) out = "0." + std::string(-point, '0') + d;
  else if ((size_t)point >= d.size()) out = d + std::string(point - d.size(), '0');
  else out = d.substr(0, point) + "." + d.substr(point);
  return (neg ? "-" : "") + out;
}

std::string rust_lower_exp4(double v) {  // {:.4e}
  char buf[64];
  std::snprintf(buf, sizeof buf, "%.4e", v);
  char* e = std::strchr(buf, 'e');
  const int ex = std::atoi(e + 1);
  *e = 0;
  return std::string(buf) + "e" + std::to_string(ex);
}

// ------------------------------------------------------------------ safetensors
struct DtypeInfo {
  const char* name;
  size_t size;
  int order;  // the crate's Dtype enum order
};
const DtypeInfo kDtypes[] = {{"BOOL", 1, 0}, {"U8", 1, 1},   {"I8", 1, 2},   {"F8_E5M2", 1, 3}, {"F8_E4M3", 1, 4},
                             {"I16", 2, 5},  {"U16", 2, 6},  {"F16", 2, 7},  {"BF16", 2, 8},    {"I32", 4, 9},
                             {"U32", 4, 10}, {"F32", 4, 11}, {"F64", 8, 12}, {"I64", 8, 13},    {"U64", 8, 14}};

const DtypeInfo* dtype_info(const std::string& n) {
  for (const auto& d : kDtypes)
    if (n == d.name) return &d;
  return nullptr;
}

int code_of_dtype(const std::string& n) {
  if (n == "F32") return CDCLQ_DTYPE_F32;
  if (n == "F16") return CDCLQ_DTYPE_F16;
  if (n == "BF16") return CDCLQ_DTYPE_BF16;
  return -1;
}
const char* dtype_of_code(int c) { return c == CDCLQ_DTYPE_F32 ? "F32" : c == CDCLQ_DTYPE_F16 ? "F16" : "BF16"; }

std::string shape_debug(const std::vector<size_t>& sh) {  // Rust {:?} of a Vec<usize>
  std::string s = "[";
  for (size_t i = 0; i < sh.size(); ++i) s += (i ? ", " : "") + std::to_string(sh[i]);
  return s + "]";
}

struct StTensor {
  std::string dtype;
  std::vector<size_t> shape;
  size_t begin = 0, end = 0;
};

struct StFile {
  std::string path;
  int fd = -1;
  void* map = nullptr;
  size_t size = 0;
  size_t data_start = 0;
  std::map<std::string, StTensor> tensors;  // by name
  std::map<std::string, std::string> metadata;
  StFile() = default;
  StFile(const StFile&) = delete;
  StFile& operator=(const StFile&) = delete;
  ~StFile() {
    if (map && map != MAP_FAILED) munmap(map, size);
    if (fd >= 0) close(fd);
  }
  const uint8_t* data(const StTensor& t) const { return static_cast<const uint8_t*>(map) + data_start + t.begin; }
  const StTensor* get(const std::string& name) const {
    auto it = tensors.find(name);
    return it == tensors.end() ? nullptr : &it->second;
  }
};

bool st_open(const std::string& path, StFile& f, std::string& err) {
  f.path = path;
  f.fd = open(path.c_str(), O_RDONLY);
  if (f.fd < 0) {
    err = "cannot open " + path + ": " + std::strerror(errno);
    return false;
  }
  struct stat sb;
  if (fstat(f.fd, &sb) != 0) {
    err = "cannot mmap " + path;
    return false;
  }
  f.size = (size_t)sb.st_size;
  if (f.size > 0) {
    f.map = mmap(nullptr, f.size, PROT_READ, MAP_PRIVATE, f.fd, 0);
    if (f.map == MAP_FAILED) {
      f.map = nullptr;
      err = "cannot mmap " + path;
      return false;
    }
  }
  const uint8_t* b = static_cast<const uint8_t*>(f.map);
  if (f.size < 8) {
    err = path + ": HeaderTooSmall";
    return false;
  }
  uint64_t n = 0;
  for (int i = 7; i >= 0; --i) n = (n << 8) | b[i];
  if (n > f.size - 8 || n > ((uint64_t)100 << 20)) {
    err = path + ": InvalidHeaderLength";
    return false;
  }
  f.data_start = 8 + (size_t)n;
  JVal h;
  std::string jerr;
  if (!parse_json(reinterpret_cast<const char*>(b + 8), (size_t)n, h, jerr) || h.kind != JVal::OBJ) {
    err = path + ": InvalidHeaderDeserialization (" + (jerr.empty() ? "not an object" : jerr) + ")";
    return false;
  }
  const size_t dlen = f.size - f.data_start;
  std::vector<std::pair<size_t, size_t>> spans;
  for (const auto& kv : h.obj) {
    if (kv.first == "__metadata__") {
      if (kv.second.kind != JVal::OBJ) {
        err = path + ": InvalidHeaderDeserialization (__metadata__)";
        return false;
      }
      for (const auto& m : kv.second.obj) {
        if (m.second.kind != JVal::STR) {
          err = path + ": InvalidHeaderDeserialization (metadata values must be strings)";
          return false;
        }
        f.metadata[m.first] = m.second.text;
      }
      continue;
    }
    const JVal& t = kv.second;
    const JVal* dt = t.get("dtype");
    const JVal* sh = t.get("shape");
    const JVal* off = t.get("data_offsets");
    if (t.kind != JVal::OBJ || !dt || dt->kind != JVal::STR || !sh || sh->kind != JVal::ARR || !off ||
        off->kind != JVal::ARR || off->arr.size() != 2) {
      err = path + ": InvalidHeaderDeserialization (tensor " + kv.first + ")";
      return false;
    }
    StTensor st;
    st.dtype = dt->text;
    const DtypeInfo* di = dtype_info(st.dtype);
    if (!di) {
      err = path + ": InvalidHeaderDeserialization (dtype " + st.dtype + ")";
      return false;
    }
    size_t numel = 1;
    for (const auto& d : sh->arr) {
      uint64_t x;
      if (!json_uint(d, &x)) {
        err = path + ": InvalidHeaderDeserialization (shape of " + kv.first + ")";
        return false;
      }
      st.shape.push_back((size_t)x);
      if (__builtin_mul_overflow(numel, (size_t)x, &numel)) {  // the crate's checked_mul fold
        err = path + ": ValidationOverflow";
        return false;
      }
    }
    size_t nbytes;
    if (__builtin_mul_overflow(numel, (size_t)di->size, &nbytes)) {
      err = path + ": ValidationOverflow";
      return false;
    }
    uint64_t a, bb;
    if (!json_uint(off->arr[0], &a) || !json_uint(off->arr[1], &bb) || a > bb || bb > dlen) {
      err = path + ": InvalidOffset(\"" + kv.first + "\")";
      return false;
    }
    st.begin = (size_t)a;
    st.end = (size_t)bb;
    if (st.end - st.begin != nbytes) {
      err = path + ": TensorInvalidInfo";
      return false;
    }
    spans.emplace_back(st.begin, st.end);
    f.tensors[kv.first] = std::move(st);
  }
  std::sort(spans.begin(), spans.end());
  size_t at = 0;
  for (const auto& s : spans) {
    if (s.first != at) {
      err = path + ": InvalidOffset";
      return false;
    }
    at = s.second;
  }
  if (at != dlen) {
    err = path + ": MetadataIncompleteBuffer";
    return false;
  }
  return true;
}

struct OutTensor {
  std::string name, dtype;
  std::vector<size_t> shape;
  std::vector<uint8_t> owned;
  const uint8_t* ptr = nullptr;  // borrowed bytes (pass-through from a mapped input)
  size_t len = 0;
  const uint8_t* bytes() const { return ptr ? ptr : owned.data(); }
  size_t size() const { return ptr ? len : owned.size(); }
};

bool mkdirs(const std::string& dir) {
  if (dir.empty()) return true;
  std::string cur;
  for (size_t i = 0; i <= dir.size(); ++i) {
    if (i == dir.size() || dir[i] == '/') {
      if (!cur.empty()) {
        struct stat sb;
        if (stat(cur.c_str(), &sb) != 0 && mkdir(cur.c_str(), 0777) != 0 && errno != EEXIST) return false;
      }
    }
    if (i < dir.size()) cur += dir[i];
  }
  return true;
}

std::string parent_of(const std::string& p) {
  const size_t k = p.rfind('/');
  return k == std::string::npos ? std::string() : p.substr(0, k);
}
std::string file_name(const std::string& p) {
  const size_t k = p.rfind('/');
  return k == std::string::npos ? p : p.substr(k + 1);
}
std::string join(const std::string& a, const std::string& b) {
  if (a.empty()) return b;
  return a.back() == '/' ? a + b : a + "/" + b;
}

// io::write_tensors (src/io.rs:107-124)
bool st_write(const std::string& path, std::vector<OutTensor>& ts, const std::map<std::string, std::string>& meta,
              std::string& err) {
  for (const auto& t : ts) {
    const DtypeInfo* di = dtype_info(t.dtype);
    size_t numel = 1;
    for (size_t d : t.shape) numel *= d;
    if (!di || numel * di->size != t.size()) {
      err = "tensor " + t.name + ": InvalidTensorView";
      return false;
    }
  }
  std::vector<size_t> ord(ts.size());
  for (size_t i = 0; i < ord.size(); ++i) ord[i] = i;
  std::sort(ord.begin(), ord.end(), [&](size_t x, size_t y) {
    const int ox = dtype_info(ts[x].dtype)->order, oy = dtype_info(ts[y].dtype)->order;
    if (ox != oy) return ox > oy;
    return ts[x].name < ts[y].name;
  });
  std::string h = "{";
  bool first = true;
  if (!meta.empty()) {
    h += "\"__metadata__\":{";
    bool f2 = true;
    for (const auto& kv : meta) {
      if (!f2) h += ",";
      f2 = false;
      json_escape(h, kv.first);
      h += ":";
      json_escape(h, kv.second);
    }
    h += "}";
    first = false;
  }
  size_t off = 0;
  for (size_t i : ord) {
    const OutTensor& t = ts[i];
    if (!first) h += ",";
    first = false;
    json_escape(h, t.name);
    h += ":{\"dtype\":\"" + t.dtype + "\",\"shape\":[";
    for (size_t k = 0; k < t.shape.size(); ++k) h += (k ? "," : "") + std::to_string(t.shape[k]);
    h += "],\"data_offsets\":[" + std::to_string(off) + "," + std::to_string(off + t.size()) + "]}";
    off += t.size();
  }
  h += "}";
  while (h.size() % 8) h += ' ';
  if (!mkdirs(parent_of(path))) {
    err = "cannot create the directory of " + path;
    return false;
  }
  FILE* fp = std::fopen(path.c_str(), "wb");
  if (!fp) {
    err = "writing " + path + ": " + std::strerror(errno);
    return false;
  }
  uint8_t lenb[8];
  const uint64_t hn = h.size();
  for (int i = 0; i < 8; ++i) lenb[i] = (uint8_t)(hn >> (8 * i));
  bool ok = std::fwrite(lenb, 1, 8, fp) == 8 && std::fwrite(h.data(), 1, h.size(), fp) == h.size();
  for (size_t i : ord)
    if (ok && ts[i].size()) ok = std::fwrite(ts[i].bytes(), 1, ts[i].size(), fp) == ts[i].size();
  ok = (std::fclose(fp) == 0) && ok;
  if (!ok) err = "writing " + path + ": " + std::strerror(errno);
  return ok;
}

// ------------------------------------------------------------------ device buffers
struct Dev {
  void* p = nullptr;
  size_t cap = 0;
  Dev() = default;
  Dev(const Dev&) = delete;
  Dev& operator=(const Dev&) = delete;
  ~Dev() {
    if (p) (void)hipFree(p);
  }
  hipError_t ensure(size_t bytes) {
    if (bytes == 0) bytes = 256;
    if (cap >= bytes) return hipSuccess;
    if (p) (void)hipFree(p);
    p = nullptr;
    cap = 0;
    hipError_t e = hipMalloc(&p, bytes);
    if (e == hipSuccess) cap = bytes;
    return e;
  }
  template <class T>
  T* as() const {
    return static_cast<T*>(p);
  }
};

// io::tensor_to_f32 on the device: raw little-endian bytes -> f32 in `out`.
int decode_tensor(cdclq_ctx* ctx, const StFile& f, const StTensor& t, Dev& stage, Dev& out, const std::string& name) {
  const int code = code_of_dtype(t.dtype);
  if (code < 0)
    return fail(ctx, CDCLQ_INVALID_ARG, "unsupported weight dtype " + t.dtype + " (need F32/F16/BF16)");
  const size_t bytes = t.end - t.begin;
  const size_t count = bytes / (code == CDCLQ_DTYPE_F32 ? 4 : 2);
  HIPCK(stage.ensure(bytes));
  HIPCK(out.ensure(count * 4));
  // stream-ordered: an earlier decode on the stream may still read `stage`
  if (bytes) HIPCK(hipMemcpyAsync(stage.p, f.data(t), bytes, hipMemcpyHostToDevice, ctx->st));
  HIPCK(decode_to_f32(ctx->st, (long)count, code, stage.p, out.as<float>()));
  (void)name;
  return CDCLQ_OK;
}

// io::HessianStore (src/io.rs:150-226)
struct HessianStore {
  std::vector<std::unique_ptr<StFile>> files;
  std::map<std::string, size_t> index;  // layer -> file (layers that own an .H)
  std::map<std::string, std::string> aliases;

  int open_all(cdclq_ctx* ctx, const std::vector<std::string>& paths) {
    for (size_t fi = 0; fi < paths.size(); ++fi) {
      files.emplace_back(new StFile());
      std::string err;
      if (!st_open(paths[fi], *files.back(), err)) return fail(ctx, CDCLQ_INVALID_ARG, err);
      for (const auto& kv : files.back()->tensors) {
        const std::string& nm = kv.first;
        if (nm.size() > 2 && nm.compare(nm.size() - 2, 2, ".H") == 0) index[nm.substr(0, nm.size() - 2)] = fi;
      }
      auto it = files.back()->metadata.find("aliases");
      if (it != files.back()->metadata.end()) {
        JVal a;
        std::string jerr;
        if (!parse_json(it->second.data(), it->second.size(), a, jerr) || a.kind != JVal::OBJ)
          return fail(ctx, CDCLQ_INVALID_ARG, "invalid 'aliases' metadata");
        for (const auto& kv : a.obj) {
          if (kv.second.kind != JVal::STR) return fail(ctx, CDCLQ_INVALID_ARG, "invalid 'aliases' metadata");
          aliases[kv.first] = kv.second.text;
        }
      }
    }
    return CDCLQ_OK;
  }
  bool resolve(const std::string& layer, std::string* owner) const {
    if (index.count(layer)) {
      *owner = layer;
      return true;
    }
    auto it = aliases.find(layer);
    if (it == aliases.end() || !index.count(it->second)) return false;
    *owner = it->second;
    return true;
  }
  // HessianStore::tensor (src/io.rs:190-213): *found = false when the optional tensor is absent.
  int tensor(cdclq_ctx* ctx, const std::string& owner, const char* suffix, Dev& stage, Dev& out, Dev& scan,
             size_t* dim, bool* found) {
    auto it = index.find(owner);
    if (it == index.end()) return fail(ctx, CDCLQ_INVALID_ARG, "no Hessian for " + owner);
    const StFile& f = *files[it->second];
    const std::string key = owner + "." + suffix;
    const StTensor* t = f.get(key);
    *found = t != nullptr;
    if (!t) return CDCLQ_OK;
    if (t->shape.size() != 2 || t->shape[0] != t->shape[1])
      return fail(ctx, CDCLQ_INVALID_ARG, key + ": expected a square matrix, got " + shape_debug(t->shape));
    CK(decode_tensor(ctx, f, *t, stage, out, key));
    const size_t d = t->shape[0], count = d * d;
    HIPCK(scan.ensure(8));
    const unsigned long long init = ~0ull;
    HIPCK(hipMemcpyAsync(scan.p, &init, 8, hipMemcpyHostToDevice, ctx->st));
    HIPCK(first_non_finite(ctx->st, (long)count, out.as<float>(), scan.as<unsigned long long>()));
    unsigned long long first = 0;
    HIPCK(hipMemcpyAsync(&first, scan.p, 8, hipMemcpyDeviceToHost, ctx->st));
    HIPCK(hipStreamSynchronize(ctx->st));
    if (first != ~0ull) {
      float v = 0.0f;
      HIPCK(hipMemcpy(&v, out.as<float>() + first, 4, hipMemcpyDeviceToHost));
      const size_t r = first / d, c = first % d;
      return fail(ctx, CDCLQ_NON_FINITE,
                  key + ": " + std::to_string(d) + " x " + std::to_string(d) + " matrix has a non-finite entry (" +
                      rust_display_f32(v) + ") at [ " + std::to_string(r) + ", " + std::to_string(c) +
                      " ]; the calibration data or the captured forward is corrupt, refusing to quantize");
    }
    *dim = d;
    return CDCLQ_OK;
  }
};

// pipeline::LayerReport (src/pipeline.rs:44-60)
struct LayerReport {
  std::string name;
  size_t d_out, d_in;
  double loss_gptq, loss_final, gain_pct;
  uint64_t subblocks_refined, subblocks_total, code_updates, skeleton_groups;
  double bits_codes, bits_total, secs_prepare, secs_quant;
};

std::string config_debug(const cdclq_config& c) {  // `format!("{:?}", cfg)` of engine::Config
  return "Config { bits: " + std::to_string(c.bits) + ", group: " + std::to_string(c.group) +
         ", block: " + std::to_string(c.block) + ", damp: " + rust_debug_f64(c.damp) +
         ", act_order: " + (c.act_order ? "true" : "false") + ", skeleton_pct: " + rust_debug_f64(c.skeleton_pct) +
         ", skeleton_bits: " + std::to_string(c.skeleton_bits) + ", mse_grid: " + (c.mse_grid ? "true" : "false") +
         ", method: " + (c.method == CDCLQ_METHOD_CDCL ? "Cdcl" : "Gptq") +
         ", refine_frac: " + rust_debug_f64(c.refine_frac) + ", sub_block: " + std::to_string(c.sub_block) +
         ", cd_sweeps: " + std::to_string(c.cd_sweeps) + ", passes: " + std::to_string(c.passes) +
         ", tol: " + rust_debug_f64(c.tol) + ", refit_scales: " + (c.refit_scales ? "true" : "false") +
         ", row_chunk: " + std::to_string(c.row_chunk) + " }";
}

// serde_json::to_string_pretty of pipeline::Report (src/pipeline.rs:62-71)
std::string report_json(const std::string& cfg, const std::vector<LayerReport>& layers, double tg, double tf,
                        double gain, double secs) {
  std::string o = "{\n  \"config\": ";
  json_escape(o, cfg);
  o += ",\n  \"layers\": ";
  if (layers.empty()) {
    o += "[]";
  } else {
    o += "[\n";
    for (size_t i = 0; i < layers.size(); ++i) {
      const LayerReport& l = layers[i];
      o += "    {\n      \"name\": ";
      json_escape(o, l.name);
      o += ",\n      \"d_out\": " + std::to_string(l.d_out) + ",\n      \"d_in\": " + std::to_string(l.d_in) +
           ",\n      \"loss_gptq\": " + json_f64(l.loss_gptq) + ",\n      \"loss_final\": " + json_f64(l.loss_final) +
           ",\n      \"gain_pct\": " + json_f64(l.gain_pct) +
           ",\n      \"subblocks_refined\": " + std::to_string(l.subblocks_refined) +
           ",\n      \"subblocks_total\": " + std::to_string(l.subblocks_total) +
           ",\n      \"code_updates\": " + std::to_string(l.code_updates) +
           ",\n      \"skeleton_groups\": " + std::to_string(l.skeleton_groups) +
           ",\n      \"bits_codes\": " + json_f64(l.bits_codes) + ",\n      \"bits_total\": " + json_f64(l.bits_total) +
           ",\n      \"secs_prepare\": " + json_f64(l.secs_prepare) +
           ",\n      \"secs_quant\": " + json_f64(l.secs_quant) + "\n    }";
      o += (i + 1 < layers.size()) ? ",\n" : "\n";
    }
    o += "  ]";
  }
  o += ",\n  \"total_loss_gptq\": " + json_f64(tg) + ",\n  \"total_loss_final\": " + json_f64(tf) +
       ",\n  \"total_gain_pct\": " + json_f64(gain) + ",\n  \"total_secs\": " + json_f64(secs) + "\n}";
  return o;
}

bool contains_any(const std::string& s, const std::vector<std::string>& pats) {
  for (const auto& p : pats)
    if (s.find(p) != std::string::npos) return true;
  return false;
}

std::vector<std::string> strings_of(const char* const* v, size_t n) {
  std::vector<std::string> out;
  for (size_t i = 0; i < n; ++i) out.emplace_back(v[i] ? v[i] : "");
  return out;
}

template <class T>
void append_le(std::vector<uint8_t>& dst, const T* src, size_t count) {  // little-endian host
  const size_t k = dst.size();
  dst.resize(k + count * sizeof(T));
  if (count) std::memcpy(dst.data() + k, src, count * sizeof(T));
}

int quantize_model(cdclq_ctx* ctx, const cdclq_quant_opts* o, std::string* report_out) {
  const double t_all = now_secs();
  HIPCK(hipSetDevice(ctx->device));
  HessianStore store;
  CK(store.open_all(ctx, strings_of(o->hessians, o->n_hessians)));
  const std::vector<std::string> only = strings_of(o->only, o->n_only), skip = strings_of(o->skip, o->n_skip);
  const std::string out_dir = o->out_dir ? o->out_dir : "";
  const size_t nthreads = o->nthreads ? o->nthreads : 1;
  std::vector<LayerReport> layers;
  Dev stage, wd, hd, md, scan, codes, scales, zeros, permd, outd, qw, s16, qz, p32;

  for (size_t si = 0; si < o->n_weights; ++si) {
    StFile shard;
    std::string err;
    if (!st_open(o->weights[si] ? o->weights[si] : "", shard, err)) return fail(ctx, CDCLQ_INVALID_ARG, err);
    // jobs: 2-D `.weight` tensors with a Hessian, ordered by (owner, layer) (src/pipeline.rs:92-113)
    struct Job {
      std::string name, layer, owner;
    };
    std::vector<Job> jobs;
    for (const auto& kv : shard.tensors) {  // names sorted
      const std::string& name = kv.first;
      if (name.size() < 7 || name.compare(name.size() - 7, 7, ".weight") != 0) continue;
      const std::string layer = name.substr(0, name.size() - 7);
      if (kv.second.shape.size() != 2) continue;
      if (!only.empty() && !contains_any(layer, only)) continue;
      if (contains_any(layer, skip)) continue;
      std::string owner;
      if (store.resolve(layer, &owner)) jobs.push_back({name, layer, owner});
    }
    std::stable_sort(jobs.begin(), jobs.end(), [](const Job& a, const Job& b) {
      if (a.owner != b.owner) return a.owner < b.owner;
      return a.layer < b.layer;
    });
    std::vector<OutTensor> deq_out, pk_out;
    std::map<std::string, bool> done;
    CK(cdclq_ctx_clear_cache(ctx));  // a fresh PrepCache per shard (src/pipeline.rs:117)
    std::string orig_dtype;
    std::string h_owner;  // the device H / M hold this owner's matrices
    bool has_m = false;
    size_t hn = 0;
    for (size_t ji = 0; ji < jobs.size(); ++ji) {
      const Job& jb = jobs[ji];
      const StTensor& t = *shard.get(jb.name);
      const size_t d_out = t.shape[0], d_in = t.shape[1];
      CK(decode_tensor(ctx, shard, t, stage, wd, jb.name));
      if (jb.owner != h_owner) {
        bool found = false;
        h_owner.clear();
        CK(store.tensor(ctx, jb.owner, "H", stage, hd, scan, &hn, &found));
        if (!found) return fail(ctx, CDCLQ_INVALID_ARG, "missing " + jb.owner + ".H");
        size_t mn = 0;
        CK(store.tensor(ctx, jb.owner, "M", stage, md, scan, &mn, &has_m));
        h_owner = jb.owner;
      }
      if (hn != d_in)
        return fail(ctx, CDCLQ_INVALID_ARG,
                    jb.layer + ": Hessian is " + std::to_string(hn) + "x" + std::to_string(hn) +
                        " but the weight has " + std::to_string(d_in) + " input columns");
      const size_t ng = cdclq_num_groups(&o->cfg, d_in);
      const size_t g = (o->cfg.group == 0 || o->cfg.group >= d_in) ? d_in : (size_t)o->cfg.group;
      HIPCK(codes.ensure(d_out * d_in));
      HIPCK(scales.ensure(d_out * ng * 4));
      HIPCK(zeros.ensure(d_out * ng * 4));
      std::vector<uint32_t> perm(d_in);
      std::vector<uint8_t> gbits(ng);
      cdclq_layer_stats s;
      CK(cdclq_quantize_layer_device(ctx, wd.as<float>(), d_out, d_in, hd.as<float>(), has_m ? md.as<float>() : nullptr,
                                     jb.owner.c_str(), &o->cfg, nthreads, codes.as<uint8_t>(), scales.as<float>(),
                                     zeros.as<float>(), perm.data(), gbits.data(), &s));
      const double gain = s.loss_gptq > 0.0 ? 100.0 * (s.loss_gptq - s.loss_final) / s.loss_gptq : 0.0;
      if (o->verbose) {
        std::fprintf(stderr, "[%3zu/%-3zu] %s [%zux%zu] loss %s -> %s (%+.1f%%) | %.2f bpw | prep %.1fs quant %.1fs\n",
                     ji + 1, jobs.size(), jb.layer.c_str(), d_out, d_in, rust_lower_exp4(s.loss_gptq).c_str(),
                     rust_lower_exp4(s.loss_final).c_str(), -gain, s.bits_total, s.secs_prepare, s.secs_quant);
      }
      layers.push_back(LayerReport{jb.layer, d_out, d_in, s.loss_gptq, s.loss_final, gain, s.subblocks_refined,
                                   s.subblocks_total, s.code_updates, s.skeleton_groups, s.bits_codes, s.bits_total,
                                   s.secs_prepare, s.secs_quant});
      if (orig_dtype.empty()) orig_dtype = t.dtype;
      HIPCK(permd.ensure(d_in * 4));
      HIPCK(hipMemcpyAsync(permd.p, perm.data(), d_in * 4, hipMemcpyHostToDevice, ctx->st));
      HIPCK(hipStreamSynchronize(ctx->st));
      if (o->emit_dequant) {
        // the checkpoint's own dtype, rounded once from the exact dequantized f32 (src/pipeline.rs:153-162)
        const int code = code_of_dtype(t.dtype);
        const size_t ob = d_out * d_in * (code == CDCLQ_DTYPE_F32 ? 4 : 2);
        HIPCK(outd.ensure(ob));
        CK(cdclq_dequantize_layer_device(ctx, d_out, d_in, g, ng, codes.as<uint8_t>(), scales.as<float>(),
                                         zeros.as<float>(), permd.as<uint32_t>(), code, outd.p));
        OutTensor ot;
        ot.name = jb.name;
        ot.dtype = t.dtype;
        ot.shape = {d_out, d_in};
        ot.owned.resize(ob);
        HIPCK(hipMemcpy(ot.owned.data(), outd.p, ob, hipMemcpyDeviceToHost));
        deq_out.push_back(std::move(ot));
      }
      if (o->emit_packed) {  // io::packed_tensors (src/io.rs:244-264)
        size_t rb = 0;
        if (cdclq_row_bytes(d_in, g, gbits.data(), ng, &rb) != CDCLQ_OK)
          return fail(ctx, CDCLQ_INVALID_ARG, jb.layer + ": invalid group widths");
        HIPCK(qw.ensure(d_out * rb));
        HIPCK(s16.ensure(d_out * ng * 2));
        HIPCK(qz.ensure(d_out * ng));
        HIPCK(p32.ensure(d_in * 4));
        CK(cdclq_pack_layer_device(ctx, d_out, d_in, g, gbits.data(), ng, codes.as<uint8_t>(), scales.as<float>(),
                                   zeros.as<float>(), permd.as<uint32_t>(), qw.as<uint8_t>(), d_out * rb,
                                   s16.as<uint16_t>(), qz.as<uint8_t>(), p32.as<int32_t>()));
        OutTensor a, b, c, d, e, f;
        a.name = jb.layer + ".qweight", a.dtype = "U8", a.shape = {d_out, rb}, a.owned.resize(d_out * rb);
        b.name = jb.layer + ".scales", b.dtype = "F16", b.shape = {d_out, ng}, b.owned.resize(d_out * ng * 2);
        c.name = jb.layer + ".qzeros", c.dtype = "U8", c.shape = {d_out, ng}, c.owned.resize(d_out * ng);
        d.name = jb.layer + ".perm", d.dtype = "I32", d.shape = {d_in}, d.owned.resize(d_in * 4);
        HIPCK(hipMemcpy(a.owned.data(), qw.p, a.owned.size(), hipMemcpyDeviceToHost));
        HIPCK(hipMemcpy(b.owned.data(), s16.p, b.owned.size(), hipMemcpyDeviceToHost));
        HIPCK(hipMemcpy(c.owned.data(), qz.p, c.owned.size(), hipMemcpyDeviceToHost));
        HIPCK(hipMemcpy(d.owned.data(), p32.p, d.owned.size(), hipMemcpyDeviceToHost));
        e.name = jb.layer + ".gbits", e.dtype = "U8", e.shape = {ng}, e.owned = gbits;
        const int32_t gs = (int32_t)g;
        f.name = jb.layer + ".gsize", f.dtype = "I32", f.shape = {1};
        append_le(f.owned, &gs, 1);
        for (OutTensor* x : {&a, &b, &c, &d, &e, &f}) pk_out.push_back(std::move(*x));
      }
      done[jb.name] = true;
    }
    // pass-through of every tensor not quantized (src/pipeline.rs:176-191)
    for (const auto& kv : shard.tensors) {
      if (done.count(kv.first)) continue;
      OutTensor ot;
      ot.name = kv.first;
      ot.dtype = kv.second.dtype;
      ot.shape = kv.second.shape;
      ot.ptr = shard.data(kv.second);
      ot.len = kv.second.end - kv.second.begin;
      if (o->emit_dequant) deq_out.push_back(ot);
      if (o->emit_packed) pk_out.push_back(ot);
    }
    const std::string fname = file_name(shard.path);
    std::map<std::string, std::string> meta{{"format", "pt"}};
    if (o->emit_dequant && !deq_out.empty())
      if (!st_write(join(join(out_dir, "dequant"), fname), deq_out, meta, err))
        return fail(ctx, CDCLQ_INVALID_ARG, err);
    if (o->emit_packed && !pk_out.empty()) {
      meta["quantization"] = "cdclq-v1";
      const std::string od = orig_dtype.empty() ? std::string("F16") : orig_dtype;
      meta["orig_dtype"] = (od == "F32" || od == "F16" || od == "BF16") ? od : std::string("OTHER");
      meta["bits"] = std::to_string(o->cfg.bits);
      if (!st_write(join(join(out_dir, "packed"), fname), pk_out, meta, err))
        return fail(ctx, CDCLQ_INVALID_ARG, err);
    }
  }
  double tg = 0.0, tf = 0.0;
  for (const auto& l : layers) {
    tg += l.loss_gptq;
    tf += l.loss_final;
  }
  const double gain = tg > 0.0 ? 100.0 * (tg - tf) / tg : 0.0;
  *report_out = report_json(config_debug(o->cfg), layers, tg, tf, gain, now_secs() - t_all);
  if (!mkdirs(out_dir)) return fail(ctx, CDCLQ_INVALID_ARG, "cannot create " + out_dir);
  const std::string rp = join(out_dir, "report.json");
  FILE* fp = std::fopen(rp.c_str(), "wb");
  if (!fp) return fail(ctx, CDCLQ_INVALID_ARG, "writing " + rp + ": " + std::strerror(errno));
  const bool ok = std::fwrite(report_out->data(), 1, report_out->size(), fp) == report_out->size();
  if ((std::fclose(fp) != 0) || !ok) return fail(ctx, CDCLQ_INVALID_ARG, "writing " + rp);
  return CDCLQ_OK;
}

// pipeline::dequantize_packed (src/pipeline.rs:239-275)
int dequantize_model(cdclq_ctx* ctx, const char* input, const char* output, int dtype, size_t* nlayers) {
  HIPCK(hipSetDevice(ctx->device));
  StFile st;
  std::string err;
  if (!st_open(input ? input : "", st, err)) return fail(ctx, CDCLQ_INVALID_ARG, err);
  int dt = dtype;
  if (dt < 0) {  // --dtype, else the header's orig_dtype (src/io.rs:72-80 spellings), else F16
    dt = CDCLQ_DTYPE_F16;
    auto it = st.metadata.find("orig_dtype");
    if (it != st.metadata.end()) {
      std::string u = it->second;
      for (auto& c : u) c = (char)std::toupper((unsigned char)c);
      if (u == "F32" || u == "FLOAT32") dt = CDCLQ_DTYPE_F32;
      else if (u == "F16" || u == "FLOAT16" || u == "HALF") dt = CDCLQ_DTYPE_F16;
      else if (u == "BF16" || u == "BFLOAT16") dt = CDCLQ_DTYPE_BF16;
    }
  }
  if (dt != CDCLQ_DTYPE_F32 && dt != CDCLQ_DTYPE_F16 && dt != CDCLQ_DTYPE_BF16)
    return fail(ctx, CDCLQ_INVALID_ARG, "unsupported output dtype " + std::to_string(dtype));
  std::vector<std::string> layers;
  for (const auto& kv : st.tensors)
    if (kv.first.size() > 8 && kv.first.compare(kv.first.size() - 8, 8, ".qweight") == 0)
      layers.push_back(kv.first.substr(0, kv.first.size() - 8));
  static const char* kSuffixes[6] = {"qweight", "scales", "qzeros", "perm", "gbits", "gsize"};
  std::vector<OutTensor> out;
  Dev qw, s16, qz, p32, od;
  for (const auto& l : layers) {  // io::read_packed_layer (src/io.rs:270-293) + dequantize
    const StTensor* t[6];
    for (int k = 0; k < 6; ++k) {
      const std::string key = l + "." + kSuffixes[k];
      t[k] = st.get(key);
      if (!t[k]) return fail(ctx, CDCLQ_INVALID_ARG, key + ": TensorNotFound(\"" + key + "\")");
    }
    if (t[0]->shape.empty() || t[3]->shape.empty() || t[5]->end - t[5]->begin < 4 || t[0]->dtype != "U8" ||
        t[1]->dtype != "F16" || t[2]->dtype != "U8" || t[3]->dtype != "I32" || t[4]->dtype != "U8" ||
        t[5]->dtype != "I32")
      return fail(ctx, CDCLQ_INVALID_ARG, l + ": malformed packed layer");
    const size_t d_out = t[0]->shape[0], d_in = t[3]->shape[0];
    int32_t gs;
    std::memcpy(&gs, st.data(*t[5]), 4);
    const size_t group = (size_t)(int64_t)gs;
    const size_t ng = t[4]->end - t[4]->begin;
    const uint8_t* gbits = st.data(*t[4]);
    const size_t nm = d_out * ng;
    if ((t[1]->end - t[1]->begin) < nm * 2 || (t[2]->end - t[2]->begin) < nm)
      return fail(ctx, CDCLQ_INVALID_ARG, l + ": scales / qzeros smaller than d_out x ngroups");
    const size_t qb = t[0]->end - t[0]->begin;
    HIPCK(qw.ensure(qb));
    HIPCK(s16.ensure(nm * 2));
    HIPCK(qz.ensure(nm));
    HIPCK(p32.ensure(d_in * 4));
    HIPCK(hipMemcpy(qw.p, st.data(*t[0]), qb, hipMemcpyHostToDevice));
    HIPCK(hipMemcpy(s16.p, st.data(*t[1]), nm * 2, hipMemcpyHostToDevice));
    HIPCK(hipMemcpy(qz.p, st.data(*t[2]), nm, hipMemcpyHostToDevice));
    HIPCK(hipMemcpy(p32.p, st.data(*t[3]), d_in * 4, hipMemcpyHostToDevice));
    const size_t ob = d_out * d_in * (dt == CDCLQ_DTYPE_F32 ? 4 : 2);
    HIPCK(od.ensure(ob));
    CK(cdclq_dequantize_packed_device(ctx, d_out, d_in, group, gbits, ng, qw.as<uint8_t>(), qb, s16.as<uint16_t>(),
                                      qz.as<uint8_t>(), p32.as<int32_t>(), dt, od.p));
    OutTensor ot;
    ot.name = l + ".weight";
    ot.dtype = dtype_of_code(dt);
    ot.shape = {d_out, d_in};
    ot.owned.resize(ob);
    HIPCK(hipMemcpy(ot.owned.data(), od.p, ob, hipMemcpyDeviceToHost));
    out.push_back(std::move(ot));
  }
  std::map<std::string, bool> lset;
  for (const auto& l : layers) lset[l] = true;
  for (const auto& kv : st.tensors) {
    bool packed = false;
    for (const char* s : kSuffixes) {
      const std::string suf = std::string(".") + s;
      if (kv.first.size() > suf.size() && kv.first.compare(kv.first.size() - suf.size(), suf.size(), suf) == 0 &&
          lset.count(kv.first.substr(0, kv.first.size() - suf.size())))
        packed = true;
    }
    if (packed) continue;
    OutTensor ot;
    ot.name = kv.first;
    ot.dtype = kv.second.dtype;
    ot.shape = kv.second.shape;
    ot.ptr = st.data(kv.second);
    ot.len = kv.second.end - kv.second.begin;
    out.push_back(ot);
  }
  if (!st_write(output ? output : "", out, {{"format", "pt"}}, err)) return fail(ctx, CDCLQ_INVALID_ARG, err);
  if (nlayers) *nlayers = layers.size();
  return CDCLQ_OK;
}

}  // namespace

extern "C" {

int cdclq_quantize_model(cdclq_ctx* ctx, const cdclq_quant_opts* opts, char* report_json, size_t report_cap,
                         size_t* report_len) {
  if (!ctx) return CDCLQ_INVALID_ARG;
  ctx->err.clear();
  if (!opts) return fail(ctx, CDCLQ_INVALID_ARG, "opts is null");
  if ((opts->n_weights && !opts->weights) || (opts->n_hessians && !opts->hessians) || (opts->n_only && !opts->only) ||
      (opts->n_skip && !opts->skip))
    return fail(ctx, CDCLQ_INVALID_ARG, "null list argument");
  std::string rep;
  CK(quantize_model(ctx, opts, &rep));
  if (report_len) *report_len = rep.size();
  if (report_json && report_cap) {
    const size_t k = std::min(report_cap - 1, rep.size());
    std::memcpy(report_json, rep.data(), k);
    report_json[k] = 0;
  }
  return CDCLQ_OK;
}

int cdclq_dequantize_model(cdclq_ctx* ctx, const char* input, const char* output, int dtype, size_t* nlayers) {
  if (!ctx) return CDCLQ_INVALID_ARG;
  ctx->err.clear();
  if (!input || !output) return fail(ctx, CDCLQ_INVALID_ARG, "null path");
  return dequantize_model(ctx, input, output, dtype, nlayers);
}

}  // extern "C"
