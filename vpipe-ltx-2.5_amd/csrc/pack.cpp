// The on-disk pack reader: a .safetensors file mapped read-only, its header
// parsed on the host, and the tensors of one linear bound as an
// ltx25_qweight in device memory the pack owns.
//
// Replaces the reference's weight-set reads for this path
// (src/ltx25-dit-weights.cc):
//   need_q_       :352-403  quantized iff NAME.scales and NAME.weight are
//                           both 2-D; bits and group from the shapes alone
//                           (group = K / scales cols, bits = codes cols *
//                           32 / K), one group per checkpoint; codes u32
//                           uploaded untouched, scales and biases read as
//                           bf16; otherwise NAME.weight is the dense weight
//   get_as_bf16_  :230-278  F16 (what the quantizer writes for scales and
//                           biases) and F32 converted to bf16 with round to
//                           nearest even; BF16 taken as stored
// and the quantizer's selection rule for the DiT component
// (src/ltx25-quant-family.cc:44-71), which says which tensors a pack holds
// quantized.
//
// safetensors layout: an 8-byte little-endian header length H, H bytes of
// JSON (`{"__metadata__": {str: str}, NAME: {"dtype": .., "shape": [..],
// "data_offsets": [begin, end]}, ...}`, offsets relative to the end of the
// header), then the data. The JSON reader below accepts exactly JSON.
#include "ltx25_qlinear.h"

#include "common.h"

#include <hip/hip_runtime.h>

#include <fcntl.h>
#include <sys/mman.h>
#include <sys/stat.h>
#include <unistd.h>

#include <cerrno>
#include <cstdio>
#include <cstring>
#include <map>
#include <memory>
#include <string>
#include <vector>

struct ltx25_pack {
  struct Tensor {
    std::string dtype;
    std::vector<long> shape;
    size_t begin = 0, end = 0;   // absolute file offsets
  };
  std::string path;
  int fd = -1;
  const unsigned char* map = nullptr;
  size_t size = 0;
  std::map<std::string, Tensor> tensors;
  std::map<std::string, std::string> meta;
  std::vector<void*> device;   // buffers this pack allocated
  std::map<std::string, const void*> bf16_cache;  // name -> device bf16 copy
};

namespace {

using ltx25::set_error;

// ---- a strict JSON reader, enough for a safetensors header -------------------------

struct JsonValue {
  enum Kind { kNull, kBool, kNumber, kString, kArray, kObject } kind = kNull;
  bool b = false;
  double num = 0.0;
  std::string str;
  std::vector<JsonValue> arr;
  std::vector<std::pair<std::string, JsonValue>> obj;
};

class JsonReader {
public:
  JsonReader(const char* p, size_t n) : p_(p), end_(p + n) {}

  bool parse(JsonValue* out)
  {
    if (!value(out, 0)) { return false; }
    ws();
    return p_ == end_ || error("trailing characters after the header object");
  }
  const std::string& err() const { return err_; }

private:
  bool error(const char* what)
  {
    if (err_.empty()) { err_ = what; }
    return false;
  }
  void ws()
  {
    while (p_ < end_ && (*p_ == ' ' || *p_ == '\t' || *p_ == '\n' || *p_ == '\r')) { ++p_; }
  }
  bool lit(const char* s)
  {
    const size_t n = std::strlen(s);
    if ((size_t)(end_ - p_) < n || std::memcmp(p_, s, n) != 0) { return false; }
    p_ += n;
    return true;
  }
  static void utf8(std::string* s, unsigned cp)
  {
    if (cp < 0x80) {
      s->push_back((char)cp);
    } else if (cp < 0x800) {
      s->push_back((char)(0xc0 | (cp >> 6)));
      s->push_back((char)(0x80 | (cp & 0x3f)));
    } else if (cp < 0x10000) {
      s->push_back((char)(0xe0 | (cp >> 12)));
      s->push_back((char)(0x80 | ((cp >> 6) & 0x3f)));
      s->push_back((char)(0x80 | (cp & 0x3f)));
    } else {
      s->push_back((char)(0xf0 | (cp >> 18)));
      s->push_back((char)(0x80 | ((cp >> 12) & 0x3f)));
      s->push_back((char)(0x80 | ((cp >> 6) & 0x3f)));
      s->push_back((char)(0x80 | (cp & 0x3f)));
    }
  }
  bool hex4(unsigned* v)
  {
    if (end_ - p_ < 4) { return error("truncated \\u escape"); }
    *v = 0;
    for (int i = 0; i < 4; ++i) {
      const char c = *p_++;
      *v <<= 4;
      if (c >= '0' && c <= '9') { *v |= (unsigned)(c - '0'); }
      else if (c >= 'a' && c <= 'f') { *v |= (unsigned)(c - 'a' + 10); }
      else if (c >= 'A' && c <= 'F') { *v |= (unsigned)(c - 'A' + 10); }
      else { return error("bad hex digit in \\u escape"); }
    }
    return true;
  }
  bool string(std::string* s)
  {
    if (p_ >= end_ || *p_ != '"') { return error("expected a string"); }
    ++p_;
    while (p_ < end_ && *p_ != '"') {
      const unsigned char c = (unsigned char)*p_++;
      if (c < 0x20) { return error("control character in a string"); }
      if (c != '\\') {
        s->push_back((char)c);
        continue;
      }
      if (p_ >= end_) { return error("truncated escape"); }
      const char e = *p_++;
      switch (e) {
        case '"': s->push_back('"'); break;
        case '\\': s->push_back('\\'); break;
        case '/': s->push_back('/'); break;
        case 'b': s->push_back('\b'); break;
        case 'f': s->push_back('\f'); break;
        case 'n': s->push_back('\n'); break;
        case 'r': s->push_back('\r'); break;
        case 't': s->push_back('\t'); break;
        case 'u': {
          unsigned cp = 0;
          if (!hex4(&cp)) { return false; }
          if (cp >= 0xd800 && cp < 0xdc00) {   // surrogate pair
            unsigned lo = 0;
            if (!lit("\\u") || !hex4(&lo) || lo < 0xdc00 || lo >= 0xe000) {
              return error("unpaired surrogate");
            }
            cp = 0x10000 + ((cp - 0xd800) << 10) + (lo - 0xdc00);
          }
          utf8(s, cp);
          break;
        }
        default: return error("unknown escape");
      }
    }
    if (p_ >= end_) { return error("unterminated string"); }
    ++p_;
    return true;
  }
  bool number(double* v)
  {
    const char* s = p_;
    if (p_ < end_ && *p_ == '-') { ++p_; }
    if (p_ >= end_ || *p_ < '0' || *p_ > '9') { return error("expected a number"); }
    while (p_ < end_ && ((*p_ >= '0' && *p_ <= '9') || *p_ == '.' || *p_ == 'e' ||
                         *p_ == 'E' || *p_ == '+' || *p_ == '-')) {
      ++p_;
    }
    const std::string t(s, p_);
    char* stop = nullptr;
    *v = std::strtod(t.c_str(), &stop);
    return (stop != nullptr && *stop == '\0') || error("malformed number");
  }
  bool value(JsonValue* v, int depth)
  {
    if (depth > 64) { return error("nesting too deep"); }
    ws();
    if (p_ >= end_) { return error("unexpected end of header"); }
    const char c = *p_;
    if (c == '{') {
      ++p_;
      v->kind = JsonValue::kObject;
      ws();
      if (p_ < end_ && *p_ == '}') { ++p_; return true; }
      for (;;) {
        ws();
        std::string key;
        if (!string(&key)) { return false; }
        ws();
        if (p_ >= end_ || *p_ != ':') { return error("expected ':'"); }
        ++p_;
        JsonValue item;
        if (!value(&item, depth + 1)) { return false; }
        v->obj.emplace_back(std::move(key), std::move(item));
        ws();
        if (p_ < end_ && *p_ == ',') { ++p_; continue; }
        if (p_ < end_ && *p_ == '}') { ++p_; return true; }
        return error("expected ',' or '}'");
      }
    }
    if (c == '[') {
      ++p_;
      v->kind = JsonValue::kArray;
      ws();
      if (p_ < end_ && *p_ == ']') { ++p_; return true; }
      for (;;) {
        JsonValue item;
        if (!value(&item, depth + 1)) { return false; }
        v->arr.push_back(std::move(item));
        ws();
        if (p_ < end_ && *p_ == ',') { ++p_; continue; }
        if (p_ < end_ && *p_ == ']') { ++p_; return true; }
        return error("expected ',' or ']'");
      }
    }
    if (c == '"') {
      v->kind = JsonValue::kString;
      return string(&v->str);
    }
    if (lit("true")) { v->kind = JsonValue::kBool; v->b = true; return true; }
    if (lit("false")) { v->kind = JsonValue::kBool; v->b = false; return true; }
    if (lit("null")) { v->kind = JsonValue::kNull; return true; }
    v->kind = JsonValue::kNumber;
    return number(&v->num);
  }

  const char* p_;
  const char* end_;
  std::string err_;
};

size_t dtype_bytes(const std::string& dt)
{
  if (dt == "F64" || dt == "I64" || dt == "U64") { return 8; }
  if (dt == "F32" || dt == "I32" || dt == "U32") { return 4; }
  if (dt == "F16" || dt == "BF16" || dt == "I16" || dt == "U16") { return 2; }
  if (dt == "I8" || dt == "U8" || dt == "BOOL" || dt == "F8_E4M3" || dt == "F8_E5M2") { return 1; }
  return 0;
}

// A non-negative integer that a double holds exactly.
bool as_index(const JsonValue& v, long* out)
{
  if (v.kind != JsonValue::kNumber || v.num < 0 || v.num > 9.007199254740992e15 ||
      v.num != (double)(long)v.num) {
    return false;
  }
  *out = (long)v.num;
  return true;
}

int parse_header(ltx25_pack* p)
{
  if (p->size < 8) { return set_error(LTX25_E_INVAL, "%s: shorter than a header", p->path.c_str()); }
  uint64_t hlen = 0;
  for (int i = 7; i >= 0; --i) { hlen = (hlen << 8) | p->map[i]; }
  if (hlen == 0 || hlen > p->size - 8 || hlen > (uint64_t)100 << 20) {
    return set_error(LTX25_E_INVAL, "%s: header length %llu does not fit the file",
                     p->path.c_str(), (unsigned long long)hlen);
  }
  JsonValue root;
  JsonReader rd((const char*)p->map + 8, (size_t)hlen);
  if (!rd.parse(&root)) {
    return set_error(LTX25_E_INVAL, "%s: header is not JSON: %s", p->path.c_str(),
                     rd.err().c_str());
  }
  if (root.kind != JsonValue::kObject) {
    return set_error(LTX25_E_INVAL, "%s: header is not a JSON object", p->path.c_str());
  }
  const size_t base = 8 + (size_t)hlen;
  for (const auto& kv : root.obj) {
    const JsonValue& t = kv.second;
    if (kv.first == "__metadata__") {
      if (t.kind != JsonValue::kObject) {
        return set_error(LTX25_E_INVAL, "%s: __metadata__ is not an object", p->path.c_str());
      }
      for (const auto& m : t.obj) {
        if (m.second.kind != JsonValue::kString) {
          return set_error(LTX25_E_INVAL, "%s: metadata '%s' is not a string", p->path.c_str(),
                           m.first.c_str());
        }
        p->meta[m.first] = m.second.str;
      }
      continue;
    }
    if (t.kind != JsonValue::kObject) {
      return set_error(LTX25_E_INVAL, "%s: entry '%s' is not an object", p->path.c_str(),
                       kv.first.c_str());
    }
    const JsonValue* dt = nullptr;
    const JsonValue* shape = nullptr;
    const JsonValue* offs = nullptr;
    for (const auto& f : t.obj) {
      if (f.first == "dtype") { dt = &f.second; }
      else if (f.first == "shape") { shape = &f.second; }
      else if (f.first == "data_offsets") { offs = &f.second; }
    }
    if (dt == nullptr || dt->kind != JsonValue::kString || shape == nullptr ||
        shape->kind != JsonValue::kArray || offs == nullptr || offs->kind != JsonValue::kArray ||
        offs->arr.size() != 2) {
      return set_error(LTX25_E_INVAL, "%s: tensor '%s' lacks dtype, shape or data_offsets",
                       p->path.c_str(), kv.first.c_str());
    }
    ltx25_pack::Tensor ten;
    ten.dtype = dt->str;
    size_t count = 1;
    for (const JsonValue& d : shape->arr) {
      long n = 0;
      if (!as_index(d, &n)) {
        return set_error(LTX25_E_INVAL, "%s: tensor '%s' has a bad dimension", p->path.c_str(),
                         kv.first.c_str());
      }
      ten.shape.push_back(n);
      count *= (size_t)n;
    }
    long b = 0, e = 0;
    if (!as_index(offs->arr[0], &b) || !as_index(offs->arr[1], &e) || e < b ||
        (size_t)e > p->size - base) {
      return set_error(LTX25_E_INVAL, "%s: tensor '%s' has data_offsets outside the file",
                       p->path.c_str(), kv.first.c_str());
    }
    const size_t eb = dtype_bytes(ten.dtype);
    if (eb != 0 && (size_t)(e - b) != count * eb) {
      return set_error(LTX25_E_INVAL, "%s: tensor '%s' holds %ld bytes, its %s shape needs %zu",
                       p->path.c_str(), kv.first.c_str(), e - b, ten.dtype.c_str(), count * eb);
    }
    ten.begin = base + (size_t)b;
    ten.end = base + (size_t)e;
    p->tensors[kv.first] = std::move(ten);
  }
  return LTX25_OK;
}

const ltx25_pack::Tensor* find(const ltx25_pack* p, const std::string& name)
{
  const auto it = p->tensors.find(name);
  return it == p->tensors.end() ? nullptr : &it->second;
}

int hip_err(hipError_t e, const char* what)
{
  return set_error(LTX25_E_HIP, "%s: %s", what, hipGetErrorString(e));
}

int device_alloc(ltx25_pack* p, size_t bytes, void** out)
{
  void* d = nullptr;
  const hipError_t e = hipMalloc(&d, bytes < 16 ? 16 : bytes);
  if (e != hipSuccess) { return hip_err(e, "hipMalloc (pack tensor)"); }
  p->device.push_back(d);
  *out = d;
  return LTX25_OK;
}

// Raw bytes to the device, untouched (the codes).
int upload_raw(ltx25_pack* p, hipStream_t st, const ltx25_pack::Tensor& t, const void** out)
{
  void* d = nullptr;
  int rc = device_alloc(p, t.end - t.begin, &d);
  if (rc != LTX25_OK) { return rc; }
  const hipError_t e = hipMemcpyAsync(d, p->map + t.begin, t.end - t.begin,
                                      hipMemcpyHostToDevice, st);
  if (e != hipSuccess) { return hip_err(e, "hipMemcpyAsync (pack tensor)"); }
  *out = d;
  return LTX25_OK;
}

// Round-to-nearest-even of an f32 bit pattern to bf16, the loader's rule
// (src/ltx25-dit-weights.cc:257-259,266-268).
uint16_t f32_bits_to_bf16(uint32_t u)
{
  const uint32_t r = ((u >> 16) & 1u) + 0x7fffu;
  return (uint16_t)((u + r) >> 16);
}

// get_as_bf16_: BF16 as stored, F16 converted on the device after upload
// (both two bytes wide, so in place), F32 converted on the host. Cached per
// name, as the reference's `derived` entries are.
int read_bf16(ltx25_pack* p, hipStream_t st, const std::string& name, const void** out,
              size_t* count)
{
  const ltx25_pack::Tensor* t = find(p, name);
  if (t == nullptr || t->shape.empty()) {
    return set_error(LTX25_E_INVAL, "%s: no tensor '%s'", p->path.c_str(), name.c_str());
  }
  size_t n = 1;
  for (long d : t->shape) { n *= (size_t)d; }
  if (count != nullptr) { *count = n; }
  const auto hit = p->bf16_cache.find(name);
  if (hit != p->bf16_cache.end()) {
    *out = hit->second;
    return LTX25_OK;
  }
  const void* d = nullptr;
  int rc = LTX25_OK;
  if (t->dtype == "BF16") {
    rc = upload_raw(p, st, *t, &d);
  } else if (t->dtype == "F16") {
    rc = upload_raw(p, st, *t, &d);
    if (rc == LTX25_OK && n > 0) {
      const hipError_t e = ltx25::launch_f16_to_bf16((const uint16_t*)d, (uint16_t*)d, n, st);
      if (e != hipSuccess) { return hip_err(e, "F16 -> bf16 launch"); }
    }
  } else if (t->dtype == "F32") {
    std::vector<uint16_t> host(n);
    for (size_t i = 0; i < n; ++i) {
      uint32_t u;
      std::memcpy(&u, p->map + t->begin + 4 * i, 4);
      host[i] = f32_bits_to_bf16(u);
    }
    void* dd = nullptr;
    rc = device_alloc(p, n * 2, &dd);
    if (rc != LTX25_OK) { return rc; }
    // synchronous: `host` is released on return
    const hipError_t e = hipMemcpy(dd, host.data(), n * 2, hipMemcpyHostToDevice);
    if (e != hipSuccess) { return hip_err(e, "hipMemcpy (F32 -> bf16 tensor)"); }
    d = dd;
  } else {
    return set_error(LTX25_E_UNSUPPORTED, "%s: tensor '%s' is %s; only BF16, F16 and F32 "
                     "are read as bf16", p->path.c_str(), name.c_str(), t->dtype.c_str());
  }
  if (rc != LTX25_OK) { return rc; }
  p->bf16_cache[name] = d;
  *out = d;
  return LTX25_OK;
}

void set_miss(char* miss, size_t len, const std::string& name)
{
  if (miss != nullptr && len > 0 && miss[0] == '\0') {
    std::snprintf(miss, len, "%s", name.c_str());
  }
}

bool contains(const std::string& s, const char* part) { return s.find(part) != std::string::npos; }

}  // namespace

extern "C" {

int ltx25_pack_open(const char* path, ltx25_pack** out)
{
  if (path == nullptr || out == nullptr) { return set_error(LTX25_E_INVAL, "null argument"); }
  *out = nullptr;
  std::unique_ptr<ltx25_pack> p(new ltx25_pack);
  p->path = path;
  p->fd = ::open(path, O_RDONLY | O_CLOEXEC);
  if (p->fd < 0) { return set_error(LTX25_E_INVAL, "%s: cannot open: %s", path, std::strerror(errno)); }
  struct stat st;
  if (::fstat(p->fd, &st) != 0 || st.st_size <= 0) {
    ::close(p->fd);
    return set_error(LTX25_E_INVAL, "%s: empty or unreadable", path);
  }
  p->size = (size_t)st.st_size;
  void* m = ::mmap(nullptr, p->size, PROT_READ, MAP_PRIVATE, p->fd, 0);
  if (m == MAP_FAILED) {
    ::close(p->fd);
    return set_error(LTX25_E_INVAL, "%s: mmap failed: %s", path, std::strerror(errno));
  }
  p->map = (const unsigned char*)m;
  const int rc = parse_header(p.get());
  if (rc != LTX25_OK) {
    ::munmap((void*)p->map, p->size);
    ::close(p->fd);
    return rc;
  }
  *out = p.release();
  return LTX25_OK;
}

void ltx25_pack_close(ltx25_pack* p)
{
  if (p == nullptr) { return; }
  if (!p->device.empty()) {
    (void)hipDeviceSynchronize();   // uploads may still be in flight
    for (void* d : p->device) { (void)hipFree(d); }
  }
  if (p->map != nullptr) { ::munmap((void*)p->map, p->size); }
  if (p->fd >= 0) { ::close(p->fd); }
  delete p;
}

int ltx25_pack_tensor(const ltx25_pack* p, const char* name, char dtype[16], int* ndim,
                      long dims[8])
{
  if (p == nullptr || name == nullptr) { return set_error(LTX25_E_INVAL, "null argument"); }
  const ltx25_pack::Tensor* t = find(p, name);
  if (t == nullptr) { return set_error(LTX25_E_INVAL, "%s: no tensor '%s'", p->path.c_str(), name); }
  if (t->shape.size() > 8) {
    return set_error(LTX25_E_UNSUPPORTED, "tensor '%s' has %zu dimensions", name, t->shape.size());
  }
  if (dtype != nullptr) { std::snprintf(dtype, 16, "%s", t->dtype.c_str()); }
  if (ndim != nullptr) { *ndim = (int)t->shape.size(); }
  if (dims != nullptr) {
    for (size_t i = 0; i < t->shape.size(); ++i) { dims[i] = t->shape[i]; }
  }
  return LTX25_OK;
}

const char* ltx25_pack_metadata(const ltx25_pack* p, const char* key)
{
  if (p == nullptr || key == nullptr) { return nullptr; }
  const auto it = p->meta.find(key);
  return it == p->meta.end() ? nullptr : it->second.c_str();
}

int ltx25_pack_read_bf16(ltx25_pack* p, void* stream, const char* name, const void** dev,
                         size_t* n)
{
  if (p == nullptr || name == nullptr || dev == nullptr) {
    return set_error(LTX25_E_INVAL, "null argument");
  }
  const int rc = ltx25_init();
  if (rc != LTX25_OK) { return rc; }
  return read_bf16(p, (hipStream_t)stream, name, dev, n);
}

int ltx25_pack_bind_qlinear(ltx25_pack* p, void* stream, const char* name, int K, int* group,
                            ltx25_qweight* out, char* miss, size_t miss_len)
{
  if (p == nullptr || name == nullptr || group == nullptr || out == nullptr) {
    return set_error(LTX25_E_INVAL, "null argument");
  }
  std::memset(out, 0, sizeof *out);
  const std::string base = name;
  const hipStream_t st = (hipStream_t)stream;
  const ltx25_pack::Tensor* si = find(p, base + ".scales");
  const ltx25_pack::Tensor* ci = find(p, base + ".weight");
  if (si != nullptr && ci != nullptr && si->shape.size() == 2 && ci->shape.size() == 2 && K > 0) {
    int bits = 0;
    int g = *group;
    int rc = ltx25_qweight_infer(K, si->shape[1], ci->shape[1], &bits, &g);
    if (rc != LTX25_OK) {
      return set_error(rc, "'%s' %s", name, ltx25_last_error());
    }
    if (dtype_bytes(ci->dtype) != 4) {
      return set_error(LTX25_E_INVAL, "'%s.weight' looks quantized but is %s, not u32 words",
                       name, ci->dtype.c_str());
    }
    const ltx25_pack::Tensor* bi = find(p, base + ".biases");
    if (bi == nullptr) {
      set_miss(miss, miss_len, base + ".biases");
      return set_error(LTX25_E_INVAL, "%s: no tensor '%s.biases'", p->path.c_str(), name);
    }
    if (si->shape[0] != ci->shape[0] || bi->shape != si->shape) {
      return set_error(LTX25_E_INVAL, "'%s': codes, scales and biases disagree on their rows",
                       name);
    }
    rc = ltx25_init();
    if (rc != LTX25_OK) { return rc; }
    const void* codes = nullptr;
    const void* scales = nullptr;
    const void* biases = nullptr;
    if ((rc = upload_raw(p, st, *ci, &codes)) != LTX25_OK ||
        (rc = read_bf16(p, st, base + ".scales", &scales, nullptr)) != LTX25_OK ||
        (rc = read_bf16(p, st, base + ".biases", &biases, nullptr)) != LTX25_OK) {
      return rc;
    }
    *group = g;
    out->codes = codes;
    out->scales = scales;
    out->qbias = biases;
    out->bits = bits;
    out->group = g;
    out->quantized = 1;
    return LTX25_OK;
  }
  if (ci == nullptr) {
    set_miss(miss, miss_len, base + ".weight");
    return set_error(LTX25_E_INVAL, "%s: no tensor '%s.weight'", p->path.c_str(), name);
  }
  const int rc = ltx25_init();
  if (rc != LTX25_OK) { return rc; }
  const void* w = nullptr;
  const int r2 = read_bf16(p, st, base + ".weight", &w, nullptr);
  if (r2 != LTX25_OK) { return r2; }
  out->w = w;
  out->quantized = 0;
  return LTX25_OK;
}

int ltx25_pack_quantizable(const char* name, const char* dtype, int ndim)
{
  if (name == nullptr || dtype == nullptr) { return 0; }
  const std::string n = name;
  const std::string dt = dtype;
  const bool is_float = dt == "BF16" || dt == "F16" || dt == "F32";
  const size_t w = n.size() >= 7 ? n.size() - 7 : std::string::npos;
  const bool weight = w != std::string::npos && n.compare(w, 7, ".weight") == 0;
  return contains(n, "_blocks.") && weight && ndim == 2 && is_float && !contains(n, "norm") &&
                 !contains(n, "embed") && !contains(n, "scale_shift") &&
                 !contains(n, "to_gate_logits")
             ? 1
             : 0;
}

}  // extern "C"
