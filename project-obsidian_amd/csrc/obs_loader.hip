// obs_loader.hip — checkpoint → HBM expert table.
//
// Replaces the reference's load path for the MoE tensors:
//   Qwen3MoeConfig::from_file            src/model.rs:7-35
//   Weights::load_non_expert             src/weight_loader.rs:19-71 (router gate, norm)
//   ExpertIndex::open                    src/disk_io.rs:36-63
//   read_experts_parallel                src/disk_io.rs:79-102
//   the split files' format              tools/split_experts.py:9-19, :30, :68-75
//
// The reference pages eight experts per token from SSD into small Metal
// buffers; here the whole stacked expert table of a layer (128 experts,
// 340 MB at the 30B-A3B shape) is made resident in HBM once, in the layout the
// kernels read, so the per-token path never touches the host.
//
// Two on-disk layouts are accepted and presented as one "stacked" view:
//   * the MLX checkpoint itself: model.layers.{l}.mlp.switch_mlp.{proj}.{kind}
//     stacked [E, ...] (bf16 scales), found through model.safetensors.index.json
//     or a single model.safetensors;
//   * the split files <expert_dir>/layer_{l}_experts.safetensors holding
//     e{N}.{proj}.{kind} per expert (tools/split_experts.py; f16 scales).
// The stacked tensor wins when both exist (it keeps the bf16 scales exactly).
// f16 scales and biases of split files are converted to bf16 on the device.
//
// The safetensors parsing restates the rules of the `safetensors` crate 0.4.5
// (Cargo.lock:1313-1314; SafeTensors::deserialize, used at disk_io.rs:43 and
// weight_loader.rs:38): 8-byte little-endian header length n <= 100,000,000;
// 8 + n <= file length; the header is UTF-8 JSON starting with '{'; entries
// {dtype, shape, data_offsets} sorted by offsets must tile the data area from
// 0 without holes or overlaps, each spanning prod(shape) * dtype size bytes;
// the last end + 8 + n must equal the file length; "__metadata__" is a
// string-to-string map and is skipped.
#include <fcntl.h>
#include <sys/stat.h>
#include <unistd.h>

#include <algorithm>
#include <atomic>
#include <cerrno>
#include <cmath>
#include <cstdlib>
#include <cstring>
#include <map>
#include <memory>
#include <mutex>
#include <thread>
#include <unordered_map>

#include "obs_internal.hpp"

// ---------------------------------------------------------------------------
// JSON (RFC 8259), enough for safetensors headers, index files and config.json
// ---------------------------------------------------------------------------
namespace obsj {

struct Value {
  enum Kind { Null, Bool, Num, Str, Arr, Obj } kind = Null;
  bool b = false;
  double num = 0.0;
  std::string text;  // the number's token, or the string's decoded UTF-8
  std::vector<Value> arr;
  std::vector<std::pair<std::string, Value>> obj;

  const Value* get(const char* key) const {
    if (kind != Obj) return nullptr;
    for (const auto& kv : obj)
      if (kv.first == key) return &kv.second;
    return nullptr;
  }
};

// Exact unsigned integer from a number token (digits only, fits in 64 bits) —
// the values serde accepts for a usize field.
inline bool as_u64(const Value& v, uint64_t& out) {
  if (v.kind != Value::Num || v.text.empty()) return false;
  uint64_t r = 0;
  for (char c : v.text) {
    if (c < '0' || c > '9') return false;
    const uint64_t d = static_cast<uint64_t>(c - '0');
    if (r > (UINT64_MAX - d) / 10u) return false;
    r = r * 10u + d;
  }
  out = r;
  return true;
}

class Parser {
 public:
  Parser(const char* s, size_t n) : p_(s), end_(s + n) {}

  bool parse(Value& out, std::string& err) {
    ws();
    if (!value(out, 0)) { err = err_.empty() ? "malformed JSON" : err_; return false; }
    ws();
    if (p_ != end_) { err = "trailing characters after JSON value"; return false; }
    return true;
  }

 private:
  const char* p_;
  const char* end_;
  std::string err_;
  static constexpr int kMaxDepth = 64;

  bool fail(const char* m) { if (err_.empty()) err_ = m; return false; }
  void ws() {
    while (p_ < end_ && (*p_ == ' ' || *p_ == '\t' || *p_ == '\n' || *p_ == '\r')) ++p_;
  }
  bool lit(const char* s) {
    const size_t n = std::strlen(s);
    if (static_cast<size_t>(end_ - p_) < n || std::memcmp(p_, s, n) != 0) return fail("invalid literal");
    p_ += n;
    return true;
  }
  bool value(Value& v, int depth) {
    if (depth > kMaxDepth) return fail("JSON nested too deeply");
    if (p_ >= end_) return fail("unexpected end of JSON");
    switch (*p_) {
      case '{': return object(v, depth);
      case '[': return array(v, depth);
      case '"': v.kind = Value::Str; return string(v.text);
      case 't': v.kind = Value::Bool; v.b = true; return lit("true");
      case 'f': v.kind = Value::Bool; v.b = false; return lit("false");
      case 'n': v.kind = Value::Null; return lit("null");
      default: return number(v);
    }
  }
  bool object(Value& v, int depth) {
    v.kind = Value::Obj;
    ++p_;
    ws();
    if (p_ < end_ && *p_ == '}') { ++p_; return true; }
    for (;;) {
      ws();
      if (p_ >= end_ || *p_ != '"') return fail("expected object key");
      std::string key;
      if (!string(key)) return false;
      ws();
      if (p_ >= end_ || *p_ != ':') return fail("expected ':'");
      ++p_;
      ws();
      v.obj.emplace_back(std::move(key), Value());
      if (!value(v.obj.back().second, depth + 1)) return false;
      ws();
      if (p_ < end_ && *p_ == ',') { ++p_; continue; }
      if (p_ < end_ && *p_ == '}') { ++p_; return true; }
      return fail("expected ',' or '}'");
    }
  }
  bool array(Value& v, int depth) {
    v.kind = Value::Arr;
    ++p_;
    ws();
    if (p_ < end_ && *p_ == ']') { ++p_; return true; }
    for (;;) {
      ws();
      v.arr.emplace_back();
      if (!value(v.arr.back(), depth + 1)) return false;
      ws();
      if (p_ < end_ && *p_ == ',') { ++p_; continue; }
      if (p_ < end_ && *p_ == ']') { ++p_; return true; }
      return fail("expected ',' or ']'");
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
  bool hex4(uint32_t& cp) {
    if (end_ - p_ < 4) return fail("short \\u escape");
    cp = 0;
    for (int i = 0; i < 4; ++i) {
      const char c = *p_++;
      cp <<= 4;
      if (c >= '0' && c <= '9') cp |= static_cast<uint32_t>(c - '0');
      else if (c >= 'a' && c <= 'f') cp |= static_cast<uint32_t>(c - 'a' + 10);
      else if (c >= 'A' && c <= 'F') cp |= static_cast<uint32_t>(c - 'A' + 10);
      else return fail("bad \\u escape");
    }
    return true;
  }
  bool string(std::string& s) {
    ++p_;  // opening quote
    s.clear();
    while (p_ < end_) {
      const unsigned char c = static_cast<unsigned char>(*p_++);
      if (c == '"') return true;
      if (c < 0x20) return fail("control character in string");
      if (c != '\\') { s += static_cast<char>(c); continue; }
      if (p_ >= end_) break;
      const char e = *p_++;
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
          if (cp >= 0xD800 && cp <= 0xDBFF) {  // high surrogate: a low one must follow
            uint32_t lo;
            if (end_ - p_ < 2 || p_[0] != '\\' || p_[1] != 'u') return fail("lone surrogate");
            p_ += 2;
            if (!hex4(lo)) return false;
            if (lo < 0xDC00 || lo > 0xDFFF) return fail("lone surrogate");
            cp = 0x10000 + ((cp - 0xD800) << 10) + (lo - 0xDC00);
          } else if (cp >= 0xDC00 && cp <= 0xDFFF) {
            return fail("lone surrogate");
          }
          put_utf8(s, cp);
          break;
        }
        default: return fail("bad escape");
      }
    }
    return fail("unterminated string");
  }
  bool number(Value& v) {
    const char* b = p_;
    if (p_ < end_ && *p_ == '-') ++p_;
    if (p_ >= end_ || *p_ < '0' || *p_ > '9') return fail("invalid value");
    if (*p_ == '0') ++p_;
    else while (p_ < end_ && *p_ >= '0' && *p_ <= '9') ++p_;
    if (p_ < end_ && *p_ == '.') {
      ++p_;
      if (p_ >= end_ || *p_ < '0' || *p_ > '9') return fail("invalid number");
      while (p_ < end_ && *p_ >= '0' && *p_ <= '9') ++p_;
    }
    if (p_ < end_ && (*p_ == 'e' || *p_ == 'E')) {
      ++p_;
      if (p_ < end_ && (*p_ == '+' || *p_ == '-')) ++p_;
      if (p_ >= end_ || *p_ < '0' || *p_ > '9') return fail("invalid number");
      while (p_ < end_ && *p_ >= '0' && *p_ <= '9') ++p_;
    }
    v.kind = Value::Num;
    v.text.assign(b, p_);
    v.num = std::strtod(v.text.c_str(), nullptr);
    return true;
  }
};

inline bool parse(const char* s, size_t n, Value& out, std::string& err) { return Parser(s, n).parse(out, err); }

inline bool valid_utf8(const unsigned char* s, size_t n) {
  size_t i = 0;
  while (i < n) {
    const unsigned char c = s[i];
    if (c < 0x80) { ++i; continue; }
    size_t len;
    uint32_t cp;
    if ((c & 0xE0) == 0xC0) { len = 2; cp = c & 0x1F; }
    else if ((c & 0xF0) == 0xE0) { len = 3; cp = c & 0x0F; }
    else if ((c & 0xF8) == 0xF0) { len = 4; cp = c & 0x07; }
    else return false;
    if (i + len > n) return false;
    for (size_t k = 1; k < len; ++k) {
      if ((s[i + k] & 0xC0) != 0x80) return false;
      cp = (cp << 6) | (s[i + k] & 0x3F);
    }
    if ((len == 2 && cp < 0x80) || (len == 3 && cp < 0x800) || (len == 4 && (cp < 0x10000 || cp > 0x10FFFF)) ||
        (cp >= 0xD800 && cp <= 0xDFFF))
      return false;  // overlong, out of range or a surrogate
    i += len;
  }
  return true;
}

}  // namespace obsj

// ---------------------------------------------------------------------------
// safetensors files
// ---------------------------------------------------------------------------
namespace {

struct DtypeName {
  const char* name;
  int code;
  uint32_t size;
};
const DtypeName kDtypes[] = {
    {"BOOL", OBS_DT_BOOL, 1}, {"U8", OBS_DT_U8, 1},   {"I8", OBS_DT_I8, 1},     {"F8_E5M2", OBS_DT_F8_E5M2, 1},
    {"F8_E4M3", OBS_DT_F8_E4M3, 1}, {"I16", OBS_DT_I16, 2}, {"U16", OBS_DT_U16, 2}, {"F16", OBS_DT_F16, 2},
    {"BF16", OBS_DT_BF16, 2}, {"I32", OBS_DT_I32, 4}, {"U32", OBS_DT_U32, 4}, {"F32", OBS_DT_F32, 4},
    {"F64", OBS_DT_F64, 8},   {"I64", OBS_DT_I64, 8}, {"U64", OBS_DT_U64, 8},
};
uint32_t dtype_size(int code) {
  for (const auto& d : kDtypes)
    if (d.code == code) return d.size;
  return 0;
}
const char* dtype_name(int code) {
  for (const auto& d : kDtypes)
    if (d.code == code) return d.name;
  return "?";
}

constexpr uint64_t kMaxHeader = 100000000ull;  // the crate's MAX_HEADER_SIZE

struct StTensor {
  int dtype = 0;
  std::vector<uint64_t> shape;
  uint64_t begin = 0, end = 0;  // relative to the data area
};

struct StFile {
  std::string path;
  int fd = -1;
  uint64_t file_size = 0, data_start = 0;
  std::unordered_map<std::string, StTensor> tensors;
  ~StFile() {
    if (fd >= 0) ::close(fd);
  }
};

std::string fmt(const char* f, ...) {
  char buf[1024];
  va_list ap;
  va_start(ap, f);
  vsnprintf(buf, sizeof buf, f, ap);
  va_end(ap);
  return buf;
}

// Reads exactly n bytes at off (pread may return short counts).
bool pread_full(int fd, void* dst, size_t n, uint64_t off) {
  char* p = static_cast<char*>(dst);
  while (n) {
    const ssize_t r = ::pread(fd, p, n, static_cast<off_t>(off));
    if (r < 0) {
      if (errno == EINTR) continue;
      return false;
    }
    if (r == 0) return false;  // the file shrank under us
    p += r;
    n -= static_cast<size_t>(r);
    off += static_cast<uint64_t>(r);
  }
  return true;
}

// Opens and validates one safetensors file.
int st_open(const std::string& path, std::unique_ptr<StFile>& out, std::string& err) {
  auto f = std::make_unique<StFile>();
  f->path = path;
  f->fd = ::open(path.c_str(), O_RDONLY | O_CLOEXEC);
  if (f->fd < 0) { err = fmt("open %s: %s", path.c_str(), std::strerror(errno)); return OBS_E_INVALID; }
  struct stat sb;
  if (::fstat(f->fd, &sb) != 0) { err = fmt("stat %s: %s", path.c_str(), std::strerror(errno)); return OBS_E_INVALID; }
  f->file_size = static_cast<uint64_t>(sb.st_size);
  if (f->file_size < 8) { err = fmt("%s: header too small (%llu bytes)", path.c_str(), (unsigned long long)f->file_size); return OBS_E_SHAPE; }
  unsigned char len8[8];
  if (!pread_full(f->fd, len8, 8, 0)) { err = fmt("%s: read failed", path.c_str()); return OBS_E_INVALID; }
  uint64_t n = 0;
  for (int i = 7; i >= 0; --i) n = (n << 8) | len8[i];
  if (n > kMaxHeader) { err = fmt("%s: header too large (%llu bytes)", path.c_str(), (unsigned long long)n); return OBS_E_SHAPE; }
  if (8 + n > f->file_size) { err = fmt("%s: header length %llu exceeds the file", path.c_str(), (unsigned long long)n); return OBS_E_SHAPE; }
  std::string hdr(static_cast<size_t>(n), '\0');
  if (n && !pread_full(f->fd, &hdr[0], static_cast<size_t>(n), 8)) { err = fmt("%s: read failed", path.c_str()); return OBS_E_INVALID; }
  if (!obsj::valid_utf8(reinterpret_cast<const unsigned char*>(hdr.data()), hdr.size())) {
    err = fmt("%s: header is not UTF-8", path.c_str());
    return OBS_E_SHAPE;
  }
  if (hdr.empty() || hdr[0] != '{') { err = fmt("%s: header does not start with '{'", path.c_str()); return OBS_E_SHAPE; }
  obsj::Value root;
  std::string jerr;
  if (!obsj::parse(hdr.data(), hdr.size(), root, jerr) || root.kind != obsj::Value::Obj) {
    err = fmt("%s: header JSON: %s", path.c_str(), jerr.c_str());
    return OBS_E_SHAPE;
  }
  struct Span { uint64_t b, e; const std::string* name; };
  std::vector<Span> spans;
  for (const auto& kv : root.obj) {
    const std::string& name = kv.first;
    const obsj::Value& v = kv.second;
    if (name == "__metadata__") {
      if (v.kind == obsj::Value::Null) continue;
      if (v.kind != obsj::Value::Obj) { err = fmt("%s: __metadata__ is not an object", path.c_str()); return OBS_E_SHAPE; }
      for (const auto& m : v.obj)
        if (m.second.kind != obsj::Value::Str) { err = fmt("%s: __metadata__ value of '%s' is not a string", path.c_str(), m.first.c_str()); return OBS_E_SHAPE; }
      continue;
    }
    if (f->tensors.count(name)) { err = fmt("%s: tensor '%s' listed twice", path.c_str(), name.c_str()); return OBS_E_SHAPE; }
    const obsj::Value* dt = v.get("dtype");
    const obsj::Value* sh = v.get("shape");
    const obsj::Value* of = v.get("data_offsets");
    if (!dt || !sh || !of || dt->kind != obsj::Value::Str || sh->kind != obsj::Value::Arr ||
        of->kind != obsj::Value::Arr || of->arr.size() != 2) {
      err = fmt("%s: tensor '%s' needs dtype, shape and two data_offsets", path.c_str(), name.c_str());
      return OBS_E_SHAPE;
    }
    StTensor t;
    t.dtype = -1;
    for (const auto& d : kDtypes)
      if (dt->text == d.name) t.dtype = d.code;
    if (t.dtype < 0) { err = fmt("%s: tensor '%s' has unknown dtype '%s'", path.c_str(), name.c_str(), dt->text.c_str()); return OBS_E_SHAPE; }
    uint64_t nel = 1;
    for (const auto& d : sh->arr) {
      uint64_t x;
      if (!obsj::as_u64(d, x)) { err = fmt("%s: tensor '%s' has a bad shape entry", path.c_str(), name.c_str()); return OBS_E_SHAPE; }
      if (x && nel > UINT64_MAX / x) { err = fmt("%s: tensor '%s' size overflows", path.c_str(), name.c_str()); return OBS_E_SHAPE; }
      nel *= x;
      t.shape.push_back(x);
    }
    if (!obsj::as_u64(of->arr[0], t.begin) || !obsj::as_u64(of->arr[1], t.end)) {
      err = fmt("%s: tensor '%s' has bad data_offsets", path.c_str(), name.c_str());
      return OBS_E_SHAPE;
    }
    const uint64_t sz = dtype_size(t.dtype);
    if (nel > UINT64_MAX / sz) { err = fmt("%s: tensor '%s' size overflows", path.c_str(), name.c_str()); return OBS_E_SHAPE; }
    if (t.end < t.begin) {
      err = fmt("%s: tensor '%s' data_offsets end before they begin", path.c_str(), name.c_str());
      return OBS_E_SHAPE;
    }
    if (t.end - t.begin != nel * sz) {
      err = fmt("%s: tensor '%s' spans %llu bytes, its dtype and shape need %llu", path.c_str(), name.c_str(),
                (unsigned long long)(t.end - t.begin), (unsigned long long)(nel * sz));
      return OBS_E_SHAPE;
    }
    f->tensors.emplace(name, std::move(t));
  }
  for (const auto& kv : f->tensors) spans.push_back({kv.second.begin, kv.second.end, &kv.first});
  std::sort(spans.begin(), spans.end(), [](const Span& a, const Span& b) { return a.b != b.b ? a.b < b.b : a.e < b.e; });
  uint64_t at = 0;
  for (const auto& s : spans) {
    if (s.b != at) { err = fmt("%s: tensor '%s' data does not start where the previous one ends", path.c_str(), s.name->c_str()); return OBS_E_SHAPE; }
    at = s.e;
  }
  f->data_start = 8 + n;
  if (f->data_start + at != f->file_size) {
    err = fmt("%s: data area is %llu bytes, the tensors cover %llu", path.c_str(),
              (unsigned long long)(f->file_size - f->data_start), (unsigned long long)at);
    return OBS_E_SHAPE;
  }
  out = std::move(f);
  return OBS_OK;
}

bool read_text(const std::string& path, std::string& out) {
  const int fd = ::open(path.c_str(), O_RDONLY | O_CLOEXEC);
  if (fd < 0) return false;
  out.clear();
  char buf[65536];
  for (;;) {
    const ssize_t r = ::read(fd, buf, sizeof buf);
    if (r < 0 && errno == EINTR) continue;
    if (r <= 0) break;
    out.append(buf, static_cast<size_t>(r));
  }
  ::close(fd);
  return true;
}
bool exists(const std::string& path) {
  struct stat sb;
  return ::stat(path.c_str(), &sb) == 0;
}
bool is_dir(const std::string& path) {
  struct stat sb;
  return ::stat(path.c_str(), &sb) == 0 && S_ISDIR(sb.st_mode);
}

// One byte range of a file that lands at a byte offset of a (virtual) tensor.
struct Piece {
  const StFile* file;
  uint64_t off;  // absolute file offset
  uint64_t n;
};

// A resolved tensor: dtype, shape and the ordered pieces that hold its bytes.
struct Resolved {
  bool found = false;  // false: no file holds the name (not an error by itself)
  int dtype = 0;
  std::vector<uint64_t> shape;
  uint64_t nbytes = 0;
  std::vector<Piece> pieces;
};

thread_local std::string g_ckpt_open_error;

}  // namespace

struct obs_ckpt {
  std::string model_dir, expert_dir;
  std::string err;
  std::mutex mu;
  obsj::Value config;
  bool have_config = false;
  std::map<std::string, std::string> weight_map;  // tensor name -> shard file name
  std::map<std::string, std::unique_ptr<StFile>> files;  // by path, opened on first use
  void* staging = nullptr;  // pinned host ring of the device loader
  int staging_dev = -1;
  ~obs_ckpt() {
    if (staging) (void)hipHostFree(staging);
  }
};

namespace {

int ck_fail(obs_ckpt* ck, int code, const std::string& m) {
  ck->err = m;
  return code;
}

int file_for(obs_ckpt* ck, const std::string& path, const StFile** out) {
  auto it = ck->files.find(path);
  if (it == ck->files.end()) {
    std::unique_ptr<StFile> f;
    std::string err;
    const int rc = st_open(path, f, err);
    if (rc != OBS_OK) return ck_fail(ck, rc, err);
    it = ck->files.emplace(path, std::move(f)).first;
  }
  *out = it->second.get();
  return OBS_OK;
}

// Parses "model.layers.{l}.mlp.switch_mlp.{proj}.{kind}".
bool parse_stacked_name(const std::string& name, uint32_t& layer, std::string& proj, std::string& kind) {
  static const char pre[] = "model.layers.";
  if (name.compare(0, sizeof(pre) - 1, pre) != 0) return false;
  size_t i = sizeof(pre) - 1, j = i;
  uint64_t l = 0;
  while (j < name.size() && name[j] >= '0' && name[j] <= '9' && j - i < 9) l = l * 10 + static_cast<uint64_t>(name[j++] - '0');
  if (j == i) return false;
  static const char mid[] = ".mlp.switch_mlp.";
  if (name.compare(j, sizeof(mid) - 1, mid) != 0) return false;
  const std::string rest = name.substr(j + sizeof(mid) - 1);
  const size_t dot = rest.find('.');
  if (dot == std::string::npos || rest.find('.', dot + 1) != std::string::npos) return false;
  proj = rest.substr(0, dot);
  kind = rest.substr(dot + 1);
  layer = static_cast<uint32_t>(l);
  return !proj.empty() && !kind.empty();
}

uint32_t config_experts(const obs_ckpt* ck) {
  uint64_t e = 0;
  const obsj::Value* v = ck->have_config ? ck->config.get("num_experts") : nullptr;
  return (v && obsj::as_u64(*v, e) && e > 0 && e <= 65536) ? static_cast<uint32_t>(e) : 0;
}

// Resolves a tensor name to its pieces: weight_map / model.safetensors first,
// then, for stacked switch_mlp names, the split per-expert files. A name that
// no file holds returns OBS_OK with r.found false; malformed files are errors.
int resolve_any(obs_ckpt* ck, const std::string& name, Resolved& r) {
  r = Resolved();
  std::string shard;
  auto wm = ck->weight_map.find(name);
  if (wm != ck->weight_map.end()) shard = wm->second;
  else if (ck->weight_map.empty() && exists(ck->model_dir + "/model.safetensors")) shard = "model.safetensors";
  if (!shard.empty()) {
    const StFile* f;
    const int rc = file_for(ck, ck->model_dir + "/" + shard, &f);
    if (rc != OBS_OK) return rc;
    auto t = f->tensors.find(name);
    if (t != f->tensors.end()) {
      r.dtype = t->second.dtype;
      r.shape = t->second.shape;
      r.nbytes = t->second.end - t->second.begin;
      r.pieces = {{f, f->data_start + t->second.begin, r.nbytes}};
      r.found = true;
      return OBS_OK;
    }
    if (wm != ck->weight_map.end())
      return ck_fail(ck, OBS_E_INVALID, fmt("tensor '%s' is mapped to %s but that file does not hold it", name.c_str(), shard.c_str()));
  }
  uint32_t layer;
  std::string proj, kind;
  if (!ck->expert_dir.empty() && parse_stacked_name(name, layer, proj, kind)) {
    const std::string path = ck->expert_dir + "/layer_" + std::to_string(layer) + "_experts.safetensors";
    if (exists(path)) {
      const uint32_t E = config_experts(ck);
      if (!E) return ck_fail(ck, OBS_E_INVALID, "split expert files need num_experts from config.json");
      const StFile* f;
      const int rc = file_for(ck, path, &f);
      if (rc != OBS_OK) return rc;
      for (uint32_t e = 0; e < E; ++e) {
        const std::string key = "e" + std::to_string(e) + "." + proj + "." + kind;
        auto t = f->tensors.find(key);
        if (t == f->tensors.end())
          return ck_fail(ck, OBS_E_INVALID, fmt("%s: tensor '%s' missing (num_experts = %u)", path.c_str(), key.c_str(), E));
        if (e == 0) {
          r.dtype = t->second.dtype;
          r.shape = t->second.shape;
        } else if (t->second.dtype != r.dtype || t->second.shape != r.shape) {
          return ck_fail(ck, OBS_E_SHAPE, fmt("%s: '%s' differs in dtype or shape from expert 0", path.c_str(), key.c_str()));
        }
        const uint64_t n = t->second.end - t->second.begin;
        r.pieces.push_back({f, f->data_start + t->second.begin, n});
        r.nbytes += n;
      }
      r.shape.insert(r.shape.begin(), E);
      r.found = true;
      return OBS_OK;
    }
  }
  return OBS_OK;
}

int resolve(obs_ckpt* ck, const std::string& name, Resolved& r) {
  const int rc = resolve_any(ck, name, r);
  if (rc != OBS_OK || r.found) return rc;
  return ck_fail(ck, OBS_E_INVALID, fmt("tensor '%s' not found in %s", name.c_str(), ck->model_dir.c_str()));
}

// f16 -> bf16 in place: exact widening to fp32, then round to nearest even.
__global__ void __launch_bounds__(256) f16_to_bf16_kernel(uint16_t* p, size_t n) {
  for (size_t i = blockIdx.x * 256ull + threadIdx.x; i < n; i += static_cast<size_t>(gridDim.x) * 256ull) {
    const _Float16 h = __builtin_bit_cast(_Float16, p[i]);
    p[i] = obsd::f32_to_bf16(static_cast<float>(h));
  }
}

// ---- pipelined file -> pinned host -> HBM copies ----------------------------
constexpr size_t kChunk = 4u << 20;  // bytes per staging slot
constexpr int kWorkers = 8;          // reader threads, each with 2 slots and a stream

struct CopyJob {
  int fd;
  uint64_t off;
  uint64_t n;
  char* dst;
};

int copy_to_device(obs_ckpt* ck, obs_ctx* ctx, const std::vector<CopyJob>& jobs) {
  if (!ck->staging || ck->staging_dev != ctx->device) {
    if (ck->staging) (void)hipHostFree(ck->staging);
    ck->staging = nullptr;
    void* p = nullptr;
    const hipError_t e = hipHostMalloc(&p, static_cast<size_t>(kWorkers) * 2 * kChunk, hipHostMallocDefault);
    if (e != hipSuccess) return obs::set_error(ctx, OBS_E_NOMEM, "hipHostMalloc(staging) failed: %s", hipGetErrorString(e));
    ck->staging = p;
    ck->staging_dev = ctx->device;
  }
  std::vector<CopyJob> chunks;
  for (const auto& j : jobs)
    for (uint64_t o = 0; o < j.n; o += kChunk)
      chunks.push_back({j.fd, j.off + o, std::min<uint64_t>(kChunk, j.n - o), j.dst + o});
  if (chunks.empty()) return OBS_OK;
  // Work already queued on the context's stream may still read the destination.
  OBS_HIP_TRY(ctx, hipStreamSynchronize(ctx->stream));

  std::atomic<size_t> next{0};
  std::atomic<bool> failed{false};
  std::mutex emu;
  std::string first_err;
  const int nw = static_cast<int>(std::min<size_t>(kWorkers, chunks.size()));
  auto worker = [&](int w) {
    auto fail = [&](const std::string& m) {
      std::lock_guard<std::mutex> g(emu);
      if (first_err.empty()) first_err = m;
      failed = true;
    };
    if (hipSetDevice(ctx->device) != hipSuccess) { fail("hipSetDevice failed in a loader thread"); return; }
    hipStream_t s = nullptr;
    hipEvent_t ev[2] = {nullptr, nullptr};
    if (hipStreamCreateWithFlags(&s, hipStreamNonBlocking) != hipSuccess ||
        hipEventCreateWithFlags(&ev[0], hipEventDisableTiming) != hipSuccess ||
        hipEventCreateWithFlags(&ev[1], hipEventDisableTiming) != hipSuccess) {
      fail("loader stream/event creation failed");
    } else {
      char* slots = static_cast<char*>(ck->staging) + static_cast<size_t>(w) * 2 * kChunk;
      for (uint64_t it = 0; !failed; ++it) {
        const size_t c = next.fetch_add(1);
        if (c >= chunks.size()) break;
        const int slot = static_cast<int>(it & 1u);
        char* buf = slots + slot * kChunk;
        hipError_t e = hipSuccess;
        if (it >= 2) e = hipEventSynchronize(ev[slot]);  // the slot's previous copy has left it
        if (e != hipSuccess) { fail(fmt("hipEventSynchronize: %s", hipGetErrorString(e))); break; }
        const CopyJob& j = chunks[c];
        if (!pread_full(j.fd, buf, static_cast<size_t>(j.n), j.off)) {
          fail(fmt("read of %llu bytes at offset %llu failed: %s", (unsigned long long)j.n, (unsigned long long)j.off,
                   std::strerror(errno)));
          break;
        }
        e = hipMemcpyAsync(j.dst, buf, static_cast<size_t>(j.n), hipMemcpyHostToDevice, s);
        if (e == hipSuccess) e = hipEventRecord(ev[slot], s);
        if (e != hipSuccess) { fail(fmt("hipMemcpyAsync: %s", hipGetErrorString(e))); break; }
      }
    }
    if (s) {
      const hipError_t e = hipStreamSynchronize(s);
      if (e != hipSuccess) fail(fmt("loader stream: %s", hipGetErrorString(e)));
    }
    for (hipEvent_t x : ev)
      if (x) (void)hipEventDestroy(x);
    if (s) (void)hipStreamDestroy(s);
  };
  std::vector<std::thread> th;
  for (int w = 1; w < nw; ++w) th.emplace_back(worker, w);
  worker(0);
  for (auto& t : th) t.join();
  (void)hipSetDevice(ctx->device);
  if (failed) return obs::set_error(ctx, OBS_E_HIP, "checkpoint load: %s", first_err.c_str());
  return OBS_OK;
}

int launch_f16_to_bf16(obs_ctx* ctx, uint16_t* p, size_t n) {
  if (!n) return OBS_OK;
  const size_t blocks = std::min<size_t>((n + 255) / 256, 8192);
  OBS_LAUNCH(ctx, "f16_to_bf16", f16_to_bf16_kernel<<<static_cast<uint32_t>(blocks), 256, 0, ctx->stream>>>(p, n));
  return OBS_OK;
}

size_t align256(size_t x) { return (x + 255u) & ~static_cast<size_t>(255u); }

// The 13 tensors of one layer's table, in device-block order.
struct LayerSlot {
  const char* what;     // name suffix after "model.layers.{l}."
  bool scale;           // bf16 destination (f16 sources converted)
  uint64_t dim[3];      // expected shape, trailing zeros unused
  uint32_t ndim;
};

std::vector<LayerSlot> layer_slots(const obs_moe_config* c) {
  const uint64_t E = c->n_exp, H = c->hidden, I = c->inter, G = c->group;
  return {
      {"mlp.switch_mlp.gate_proj.weight", false, {E, I, H / 8}, 3},
      {"mlp.switch_mlp.gate_proj.scales", true, {E, I, H / G}, 3},
      {"mlp.switch_mlp.gate_proj.biases", true, {E, I, H / G}, 3},
      {"mlp.switch_mlp.up_proj.weight", false, {E, I, H / 8}, 3},
      {"mlp.switch_mlp.up_proj.scales", true, {E, I, H / G}, 3},
      {"mlp.switch_mlp.up_proj.biases", true, {E, I, H / G}, 3},
      {"mlp.switch_mlp.down_proj.weight", false, {E, H, I / 8}, 3},
      {"mlp.switch_mlp.down_proj.scales", true, {E, H, I / G}, 3},
      {"mlp.switch_mlp.down_proj.biases", true, {E, H, I / G}, 3},
      {"mlp.gate.weight", false, {E, H / 4, 0}, 2},
      {"mlp.gate.scales", true, {E, H / G, 0}, 2},
      {"mlp.gate.biases", true, {E, H / G, 0}, 2},
      {"post_attention_layernorm.weight", true, {H, 0, 0}, 1},
  };
}

uint64_t slot_bytes(const LayerSlot& s) {
  uint64_t n = s.scale ? 2 : 4;
  for (uint32_t i = 0; i < s.ndim; ++i) n *= s.dim[i];
  return n;
}

bool layer_config_ok(const obs_moe_config* c) {
  return c && c->n_exp > 0 && c->hidden > 0 && c->inter > 0 && c->group > 0 && c->hidden % 8 == 0 &&
         c->inter % 8 == 0 && c->hidden % c->group == 0 && c->inter % c->group == 0;
}

std::string shape_str(const std::vector<uint64_t>& s) {
  std::string r = "[";
  for (size_t i = 0; i < s.size(); ++i) r += (i ? ", " : "") + std::to_string(s[i]);
  return r + "]";
}

}  // namespace

extern "C" {

int obs_ckpt_open(const char* model_dir, const char* expert_dir, obs_ckpt** out) {
  g_ckpt_open_error.clear();
  if (!model_dir || !out) { g_ckpt_open_error = "obs_ckpt_open: null argument"; return OBS_E_INVALID; }
  *out = nullptr;
  auto ck = std::make_unique<obs_ckpt>();
  ck->model_dir = model_dir;
  while (ck->model_dir.size() > 1 && ck->model_dir.back() == '/') ck->model_dir.pop_back();
  if (!is_dir(ck->model_dir)) { g_ckpt_open_error = fmt("%s is not a directory", model_dir); return OBS_E_INVALID; }
  // config.json (Qwen3MoeConfig::from_file, model.rs:26-30): optional here, required by obs_ckpt_config.
  std::string text;
  if (read_text(ck->model_dir + "/config.json", text)) {
    std::string err;
    if (!obsj::parse(text.data(), text.size(), ck->config, err) || ck->config.kind != obsj::Value::Obj) {
      g_ckpt_open_error = fmt("%s/config.json: %s", ck->model_dir.c_str(), err.empty() ? "not an object" : err.c_str());
      return OBS_E_SHAPE;
    }
    ck->have_config = true;
  }
  // model.safetensors.index.json's weight_map (weight_loader.rs:20-30).
  if (read_text(ck->model_dir + "/model.safetensors.index.json", text)) {
    obsj::Value idx;
    std::string err;
    if (!obsj::parse(text.data(), text.size(), idx, err)) {
      g_ckpt_open_error = fmt("model.safetensors.index.json: %s", err.c_str());
      return OBS_E_SHAPE;
    }
    const obsj::Value* wm = idx.get("weight_map");
    if (!wm || wm->kind != obsj::Value::Obj) { g_ckpt_open_error = "model.safetensors.index.json: no weight_map"; return OBS_E_SHAPE; }
    for (const auto& kv : wm->obj) {
      if (kv.second.kind != obsj::Value::Str || kv.second.text.empty() || kv.second.text.find('/') != std::string::npos) {
        g_ckpt_open_error = fmt("weight_map entry '%s' is not a file name in the model directory", kv.first.c_str());
        return OBS_E_SHAPE;
      }
      ck->weight_map[kv.first] = kv.second.text;
    }
  }
  // Split expert files: expert_dir, or <model_dir>/splitted_moe (main.rs:70-73).
  if (expert_dir && *expert_dir) {
    if (!is_dir(expert_dir)) { g_ckpt_open_error = fmt("%s is not a directory", expert_dir); return OBS_E_INVALID; }
    ck->expert_dir = expert_dir;
  } else if (is_dir(ck->model_dir + "/splitted_moe")) {
    ck->expert_dir = ck->model_dir + "/splitted_moe";
  }
  *out = ck.release();
  return OBS_OK;
}

void obs_ckpt_close(obs_ckpt* ck) { delete ck; }

const char* obs_ckpt_error(const obs_ckpt* ck) { return ck ? ck->err.c_str() : g_ckpt_open_error.c_str(); }

int obs_ckpt_config(obs_ckpt* ck, obs_moe_config* cfg, uint32_t* n_layers) {
  if (!ck) return OBS_E_INVALID;
  if (!cfg) return ck_fail(ck, OBS_E_INVALID, "obs_ckpt_config: null cfg");
  if (!ck->have_config) return ck_fail(ck, OBS_E_INVALID, fmt("%s/config.json not found", ck->model_dir.c_str()));
  const obsj::Value& c = ck->config;
  // The fields Qwen3MoeConfig requires (model.rs:9-22), as non-negative integers.
  static const char* kUsize[] = {"num_hidden_layers", "hidden_size", "num_attention_heads", "num_key_value_heads",
                                 "num_experts", "num_experts_per_tok", "moe_intermediate_size", "vocab_size"};
  uint64_t u[8];
  for (int i = 0; i < 8; ++i) {
    const obsj::Value* v = c.get(kUsize[i]);
    if (!v) return ck_fail(ck, OBS_E_SHAPE, fmt("config.json: missing field `%s`", kUsize[i]));
    if (!obsj::as_u64(*v, u[i]) || u[i] > UINT32_MAX)
      return ck_fail(ck, OBS_E_SHAPE, fmt("config.json: `%s` is not a non-negative 32-bit integer", kUsize[i]));
  }
  static const char* kF32[] = {"rms_norm_eps", "rope_theta"};
  float fv[2];
  for (int i = 0; i < 2; ++i) {
    const obsj::Value* v = c.get(kF32[i]);
    if (!v) return ck_fail(ck, OBS_E_SHAPE, fmt("config.json: missing field `%s`", kF32[i]));
    if (v->kind != obsj::Value::Num) return ck_fail(ck, OBS_E_SHAPE, fmt("config.json: `%s` is not a number", kF32[i]));
    fv[i] = static_cast<float>(v->num);
  }
  bool norm_topk = false;  // #[serde(default)] (model.rs:21-22)
  if (const obsj::Value* v = c.get("norm_topk_prob"); v && v->kind != obsj::Value::Null) {
    if (v->kind != obsj::Value::Bool) return ck_fail(ck, OBS_E_SHAPE, "config.json: `norm_topk_prob` is not a boolean");
    norm_topk = v->b;
  }
  // MLX quantization block; the reference fixes group_size 64 (forward.rs:306, :316, :393).
  uint64_t group = 64;
  if (const obsj::Value* q = c.get("quantization"); q && q->kind == obsj::Value::Obj) {
    if (const obsj::Value* g = q->get("group_size"); g && (!obsj::as_u64(*g, group) || group == 0 || group > 4096))
      return ck_fail(ck, OBS_E_SHAPE, "config.json: quantization.group_size is not a positive integer");
  }
  cfg->n_exp = static_cast<uint32_t>(u[4]);
  cfg->top_k = static_cast<uint32_t>(u[5]);
  cfg->hidden = static_cast<uint32_t>(u[1]);
  cfg->inter = static_cast<uint32_t>(u[6]);
  cfg->group = static_cast<uint32_t>(group);
  cfg->norm_topk = norm_topk ? 1 : 0;
  cfg->rms_eps = fv[0];
  cfg->route_rule = OBS_ROUTE_REF;  // the reference engine routes on f16 logits
  if (n_layers) *n_layers = static_cast<uint32_t>(u[0]);
  return OBS_OK;
}

int obs_ckpt_tensor_info(obs_ckpt* ck, const char* name, obs_tensor_info* info) {
  if (!ck) return OBS_E_INVALID;
  if (!name || !info) return ck_fail(ck, OBS_E_INVALID, "obs_ckpt_tensor_info: null argument");
  std::lock_guard<std::mutex> g(ck->mu);
  Resolved r;
  const int rc = resolve(ck, name, r);
  if (rc != OBS_OK) return rc;
  if (r.shape.size() > 8) return ck_fail(ck, OBS_E_SHAPE, fmt("tensor '%s' has %zu dimensions (at most 8)", name, r.shape.size()));
  std::memset(info, 0, sizeof *info);
  info->dtype = r.dtype;
  info->ndim = static_cast<uint32_t>(r.shape.size());
  for (size_t i = 0; i < r.shape.size(); ++i) info->shape[i] = r.shape[i];
  info->nbytes = r.nbytes;
  info->n_pieces = static_cast<uint32_t>(r.pieces.size());
  return OBS_OK;
}

int obs_ckpt_read(obs_ckpt* ck, const char* name, void* dst_host, size_t bytes) {
  if (!ck) return OBS_E_INVALID;
  if (!name || (!dst_host && bytes)) return ck_fail(ck, OBS_E_INVALID, "obs_ckpt_read: null argument");
  std::lock_guard<std::mutex> g(ck->mu);
  Resolved r;
  const int rc = resolve(ck, name, r);
  if (rc != OBS_OK) return rc;
  if (bytes < r.nbytes)
    return ck_fail(ck, OBS_E_NOMEM, fmt("obs_ckpt_read: '%s' needs %llu bytes, buffer has %zu", name, (unsigned long long)r.nbytes, bytes));
  char* d = static_cast<char*>(dst_host);
  for (const auto& p : r.pieces) {
    if (!pread_full(p.file->fd, d, static_cast<size_t>(p.n), p.off))
      return ck_fail(ck, OBS_E_INVALID, fmt("%s: read failed: %s", p.file->path.c_str(), std::strerror(errno)));
    d += p.n;
  }
  return OBS_OK;
}

size_t obs_moe_layer_bytes(const obs_moe_config* cfg) {
  if (!layer_config_ok(cfg)) return 0;
  size_t total = 0;
  for (const auto& s : layer_slots(cfg)) total += align256(static_cast<size_t>(slot_bytes(s)));
  return total;
}

int obs_ckpt_load_tensor(obs_ctx* ctx, obs_ckpt* ck, const char* name, void* dst_dev, size_t bytes) {
  if (!ctx) return OBS_E_INVALID;
  if (!ck || !name || !dst_dev) return obs::set_error(ctx, OBS_E_INVALID, "obs_ckpt_load_tensor: null argument");
  std::lock_guard<std::mutex> g(ck->mu);
  Resolved r;
  if (resolve(ck, name, r) != OBS_OK) return obs::set_error(ctx, OBS_E_INVALID, "%s", ck->err.c_str());
  if (bytes < r.nbytes)
    return obs::set_error(ctx, OBS_E_NOMEM, "obs_ckpt_load_tensor: '%s' needs %llu bytes, buffer has %zu", name,
                          (unsigned long long)r.nbytes, bytes);
  std::vector<CopyJob> jobs;
  char* d = static_cast<char*>(dst_dev);
  for (const auto& p : r.pieces) {
    jobs.push_back({p.file->fd, p.off, p.n, d});
    d += p.n;
  }
  return copy_to_device(ck, ctx, jobs);
}

int obs_ckpt_load_moe_layer(obs_ctx* ctx, obs_ckpt* ck, uint32_t layer, const obs_moe_config* cfg, void* dst_dev,
                            size_t bytes, obs_moe_layer* out) {
  if (!ctx) return OBS_E_INVALID;
  if (!ck || !cfg || !dst_dev || !out) return obs::set_error(ctx, OBS_E_INVALID, "obs_ckpt_load_moe_layer: null argument");
  if (!layer_config_ok(cfg))
    return obs::set_error(ctx, OBS_E_SHAPE, "obs_ckpt_load_moe_layer: config needs hidden, inter multiples of 8 and of group");
  if (!obs::aligned(dst_dev, 256)) return obs::set_error(ctx, OBS_E_ALIGN, "obs_ckpt_load_moe_layer: dst must be 256-byte aligned");
  const size_t need = obs_moe_layer_bytes(cfg);
  if (bytes < need)
    return obs::set_error(ctx, OBS_E_NOMEM, "obs_ckpt_load_moe_layer: table needs %zu bytes, buffer has %zu", need, bytes);
  std::lock_guard<std::mutex> g(ck->mu);
  const auto slots = layer_slots(cfg);
  const std::string pre = "model.layers." + std::to_string(layer) + ".";
  std::vector<CopyJob> jobs;
  std::vector<std::pair<uint16_t*, size_t>> convert;  // f16 sources, converted after the copies
  std::vector<char*> where(slots.size(), nullptr);
  char* d = static_cast<char*>(dst_dev);
  for (size_t i = 0; i < slots.size(); ++i) {
    const LayerSlot& s = slots[i];
    const std::string name = pre + s.what;
    Resolved r;
    const bool optional = (i == slots.size() - 1);  // post_attention_layernorm.weight
    const int rc = optional ? resolve_any(ck, name, r) : resolve(ck, name, r);
    if (rc != OBS_OK) return obs::set_error(ctx, rc, "%s", ck->err.c_str());
    if (!r.found) continue;  // no norm weight: norm_w stays NULL
    std::vector<uint64_t> want(s.dim, s.dim + s.ndim);
    if (r.shape != want)
      return obs::set_error(ctx, OBS_E_SHAPE, "%s: shape %s, the config needs %s%s", name.c_str(), shape_str(r.shape).c_str(),
                            shape_str(want).c_str(),
                            i == 9 ? " (an 8-bit router gate)" : (!s.scale ? " (4-bit packed experts)" : ""));
    const bool ok = s.scale ? (r.dtype == OBS_DT_BF16 || r.dtype == OBS_DT_F16) : (r.dtype == OBS_DT_U32);
    if (!ok)
      return obs::set_error(ctx, OBS_E_SHAPE, "%s: dtype %s, expected %s", name.c_str(), dtype_name(r.dtype),
                            s.scale ? "BF16 or F16" : "U32");
    where[i] = d;
    char* p = d;
    for (const auto& pc : r.pieces) {
      jobs.push_back({pc.file->fd, pc.off, pc.n, p});
      p += pc.n;
    }
    if (r.dtype == OBS_DT_F16) convert.emplace_back(reinterpret_cast<uint16_t*>(d), static_cast<size_t>(r.nbytes / 2));
    d += align256(static_cast<size_t>(slot_bytes(s)));
  }
  int rc = copy_to_device(ck, ctx, jobs);
  if (rc != OBS_OK) return rc;
  for (const auto& c : convert)
    if ((rc = launch_f16_to_bf16(ctx, c.first, c.second)) != OBS_OK) return rc;
  OBS_HIP_TRY(ctx, hipStreamSynchronize(ctx->stream));
  out->gate_w = reinterpret_cast<const uint32_t*>(where[0]);
  out->gate_s = reinterpret_cast<const uint16_t*>(where[1]);
  out->gate_b = reinterpret_cast<const uint16_t*>(where[2]);
  out->up_w = reinterpret_cast<const uint32_t*>(where[3]);
  out->up_s = reinterpret_cast<const uint16_t*>(where[4]);
  out->up_b = reinterpret_cast<const uint16_t*>(where[5]);
  out->down_w = reinterpret_cast<const uint32_t*>(where[6]);
  out->down_s = reinterpret_cast<const uint16_t*>(where[7]);
  out->down_b = reinterpret_cast<const uint16_t*>(where[8]);
  out->router_w = reinterpret_cast<const uint32_t*>(where[9]);
  out->router_s = reinterpret_cast<const uint16_t*>(where[10]);
  out->router_b = reinterpret_cast<const uint16_t*>(where[11]);
  out->norm_w = reinterpret_cast<const uint16_t*>(where[12]);
  return OBS_OK;
}

}  // extern "C"
