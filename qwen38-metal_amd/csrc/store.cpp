// MLX safetensors weight store: the on-disk format of the reference's Q4
// checkpoints, read on the host and copied into HBM.
//
//   * open_mlx_safetensors_dir (/root/reference/src/model.rs:136-197): the
//     directory's model.safetensors.index.json maps tensor -> shard file; every
//     indexed tensor must appear in its shard's header with a data range inside
//     the shard (validate_tensor_range, model.rs:418-431); shard names must be
//     plain relative paths (resolve_shard, model.rs:312-323).
//   * read_safetensors_header (model.rs:336-416): 8-byte little-endian header
//     length (at most 128 MiB and inside the file), a JSON object of
//     {name: {dtype, shape, data_offsets}} plus an ignored __metadata__; data
//     begins after the header; empty dtype or shape is rejected.
//   * Q4AffineMatrix::from_store / from_tensors / validate_affine_tensor
//     (native.rs:5384-5516): `<base>.weight` is U32 [rows][K/8], and
//     `<base>.scales` / `<base>.biases` are BF16 [rows][K/64], with K a
//     non-zero multiple of 64 and exact byte lengths.
//
// Shards are memory-mapped read-only; uploads copy a tensor's bytes from the
// mapping into a fresh 256-byte-aligned device allocation.
#include <errno.h>
#include <fcntl.h>
#include <stdint.h>
#include <string.h>
#include <sys/mman.h>
#include <sys/stat.h>
#include <unistd.h>

#include <algorithm>
#include <map>
#include <memory>
#include <string>
#include <vector>

#include "runtime_internal.h"

using namespace qm;

namespace {

// ---- a small JSON reader (objects, arrays, strings, numbers, literals) ----
struct JValue {
  enum Kind { Null, Bool, Number, String, Array, Object } kind = Null;
  bool b = false;
  double num = 0.0;
  uint64_t u64 = 0;       // exact value of a non-negative integer literal
  bool is_uint = false;
  std::string str;
  std::vector<JValue> arr;
  std::vector<std::pair<std::string, JValue>> obj;

  const JValue* get(const char* key) const {
    for (const auto& kv : obj)
      if (kv.first == key) return &kv.second;
    return nullptr;
  }
};

class JParser {
 public:
  JParser(const char* p, size_t n) : p_(p), end_(p + n) {}
  bool parse(JValue& out) {
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
  bool lit(const char* s) {
    const size_t n = strlen(s);
    if ((size_t)(end_ - p_) < n || memcmp(p_, s, n) != 0) return false;
    p_ += n;
    return true;
  }
  static void put_utf8(std::string& s, uint32_t cp) {
    if (cp < 0x80) {
      s += (char)cp;
    } else if (cp < 0x800) {
      s += (char)(0xC0 | (cp >> 6));
      s += (char)(0x80 | (cp & 0x3F));
    } else if (cp < 0x10000) {
      s += (char)(0xE0 | (cp >> 12));
      s += (char)(0x80 | ((cp >> 6) & 0x3F));
      s += (char)(0x80 | (cp & 0x3F));
    } else {
      s += (char)(0xF0 | (cp >> 18));
      s += (char)(0x80 | ((cp >> 12) & 0x3F));
      s += (char)(0x80 | ((cp >> 6) & 0x3F));
      s += (char)(0x80 | (cp & 0x3F));
    }
  }
  bool hex4(uint32_t& v) {
    if (end_ - p_ < 4) return false;
    v = 0;
    for (int i = 0; i < 4; ++i) {
      const char c = *p_++;
      v <<= 4;
      if (c >= '0' && c <= '9') v |= (uint32_t)(c - '0');
      else if (c >= 'a' && c <= 'f') v |= (uint32_t)(c - 'a' + 10);
      else if (c >= 'A' && c <= 'F') v |= (uint32_t)(c - 'A' + 10);
      else return false;
    }
    return true;
  }
  bool string(std::string& s) {
    if (p_ >= end_ || *p_ != '"') return false;
    ++p_;
    while (p_ < end_ && *p_ != '"') {
      const char c = *p_++;
      if ((unsigned char)c < 0x20) return false;
      if (c != '\\') {
        s += c;
        continue;
      }
      if (p_ >= end_) return false;
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
          if (cp >= 0xD800 && cp < 0xDC00) {  // surrogate pair
            uint32_t lo;
            if (!lit("\\u") || !hex4(lo) || lo < 0xDC00 || lo >= 0xE000) return false;
            cp = 0x10000 + ((cp - 0xD800) << 10) + (lo - 0xDC00);
          }
          put_utf8(s, cp);
          break;
        }
        default: return false;
      }
    }
    if (p_ >= end_) return false;
    ++p_;
    return true;
  }
  bool number(JValue& v) {
    const char* s = p_;
    if (p_ < end_ && *p_ == '-') ++p_;
    const char* digits = p_;
    while (p_ < end_ && *p_ >= '0' && *p_ <= '9') ++p_;
    if (p_ == digits) return false;
    bool integer = true;
    if (p_ < end_ && *p_ == '.') {
      integer = false;
      ++p_;
      while (p_ < end_ && *p_ >= '0' && *p_ <= '9') ++p_;
    }
    if (p_ < end_ && (*p_ == 'e' || *p_ == 'E')) {
      integer = false;
      ++p_;
      if (p_ < end_ && (*p_ == '+' || *p_ == '-')) ++p_;
      while (p_ < end_ && *p_ >= '0' && *p_ <= '9') ++p_;
    }
    const std::string text(s, p_);
    v.kind = JValue::Number;
    v.num = strtod(text.c_str(), nullptr);
    if (integer && text[0] != '-' && text.size() <= 20) {
      errno = 0;
      char* e = nullptr;
      const unsigned long long u = strtoull(text.c_str(), &e, 10);
      if (errno == 0 && e && *e == '\0') {
        v.u64 = u;
        v.is_uint = true;
      }
    }
    return true;
  }
  bool value(JValue& v, int depth) {
    if (depth > 64) return false;
    ws();
    if (p_ >= end_) return false;
    const char c = *p_;
    if (c == '{') {
      ++p_;
      v.kind = JValue::Object;
      ws();
      if (p_ < end_ && *p_ == '}') {
        ++p_;
        return true;
      }
      for (;;) {
        ws();
        std::string key;
        if (!string(key)) return false;
        ws();
        if (p_ >= end_ || *p_ != ':') return false;
        ++p_;
        JValue child;
        if (!value(child, depth + 1)) return false;
        v.obj.emplace_back(std::move(key), std::move(child));
        ws();
        if (p_ < end_ && *p_ == ',') {
          ++p_;
          continue;
        }
        if (p_ < end_ && *p_ == '}') {
          ++p_;
          return true;
        }
        return false;
      }
    }
    if (c == '[') {
      ++p_;
      v.kind = JValue::Array;
      ws();
      if (p_ < end_ && *p_ == ']') {
        ++p_;
        return true;
      }
      for (;;) {
        JValue child;
        if (!value(child, depth + 1)) return false;
        v.arr.push_back(std::move(child));
        ws();
        if (p_ < end_ && *p_ == ',') {
          ++p_;
          continue;
        }
        if (p_ < end_ && *p_ == ']') {
          ++p_;
          return true;
        }
        return false;
      }
    }
    if (c == '"') {
      v.kind = JValue::String;
      return string(v.str);
    }
    if (lit("true")) {
      v.kind = JValue::Bool;
      v.b = true;
      return true;
    }
    if (lit("false")) {
      v.kind = JValue::Bool;
      return true;
    }
    if (lit("null")) return true;
    return number(v);
  }
};

constexpr uint64_t kMaxHeaderBytes = 128ull * 1024 * 1024;  // MAX_SAFETENSORS_HEADER_BYTES, model.rs:13

struct Tensor {
  std::string dtype;
  std::vector<uint64_t> shape;
  size_t shard = 0;
  uint64_t offset = 0;  // from the start of the shard file
  uint64_t bytes = 0;
};

struct Shard {
  std::string path;
  const uint8_t* map = nullptr;
  size_t size = 0;
};

bool read_file(const std::string& path, std::string& out) {
  const int fd = open(path.c_str(), O_RDONLY | O_CLOEXEC);
  if (fd < 0) return false;
  struct stat st;
  if (fstat(fd, &st) != 0) {
    close(fd);
    return false;
  }
  out.resize((size_t)st.st_size);
  size_t got = 0;
  while (got < out.size()) {
    const ssize_t n = read(fd, &out[got], out.size() - got);
    if (n <= 0) {
      close(fd);
      return false;
    }
    got += (size_t)n;
  }
  close(fd);
  return true;
}

// resolve_shard (model.rs:312-323): a relative path of plain components.
bool safe_relative(const std::string& name) {
  if (name.empty() || name[0] == '/') return false;
  size_t start = 0;
  while (start <= name.size()) {
    const size_t slash = name.find('/', start);
    const std::string part = name.substr(start, slash == std::string::npos ? std::string::npos : slash - start);
    if (part.empty() || part == "." || part == "..") return false;
    if (slash == std::string::npos) break;
    start = slash + 1;
  }
  return true;
}

}  // namespace

struct qm_weight_store {
  std::vector<Shard> shards;
  std::map<std::string, Tensor> tensors;
  ~qm_weight_store() {
    for (auto& s : shards)
      if (s.map) munmap((void*)s.map, s.size);
  }
};

namespace {

// read_safetensors_header (model.rs:336-416), on the mapped file.
qm_status parse_shard_header(const Shard& sh, size_t shard_index, std::map<std::string, Tensor>& out) {
  if (sh.size < 8)
    return fail(QM_ERR_MODEL_FORMAT, "%s: header length 0 does not fit a %zu-byte file", sh.path.c_str(), sh.size);
  uint64_t header_bytes = 0;
  for (int i = 7; i >= 0; --i) header_bytes = (header_bytes << 8) | sh.map[i];
  if (header_bytes > kMaxHeaderBytes || header_bytes > sh.size - 8)
    return fail(QM_ERR_MODEL_FORMAT, "%s: header length %llu does not fit a %zu-byte file", sh.path.c_str(),
                (unsigned long long)header_bytes, sh.size);
  JValue root;
  if (!JParser((const char*)sh.map + 8, (size_t)header_bytes).parse(root) || root.kind != JValue::Object)
    return fail(QM_ERR_MODEL_FORMAT, "%s: safetensors header is not a JSON object", sh.path.c_str());
  const uint64_t data_offset = 8 + header_bytes, data_bytes = sh.size - data_offset;
  for (const auto& kv : root.obj) {
    if (kv.first == "__metadata__") continue;
    const JValue& t = kv.second;
    const JValue* dtype = t.get("dtype");
    const JValue* shape = t.get("shape");
    const JValue* offs = t.get("data_offsets");
    if (t.kind != JValue::Object || !dtype || dtype->kind != JValue::String || !shape ||
        shape->kind != JValue::Array || !offs || offs->kind != JValue::Array || offs->arr.size() != 2 ||
        !offs->arr[0].is_uint || !offs->arr[1].is_uint)
      return fail(QM_ERR_MODEL_FORMAT, "%s: malformed header entry for %s", sh.path.c_str(), kv.first.c_str());
    Tensor ten;
    ten.dtype = dtype->str;
    for (const JValue& d : shape->arr) {
      if (!d.is_uint)
        return fail(QM_ERR_MODEL_FORMAT, "%s: malformed shape for %s", sh.path.c_str(), kv.first.c_str());
      ten.shape.push_back(d.u64);
    }
    if (ten.dtype.empty() || ten.shape.empty())
      return fail(QM_ERR_MODEL_FORMAT, "%s: tensor %s has empty dtype or shape", sh.path.c_str(), kv.first.c_str());
    const uint64_t b0 = offs->arr[0].u64, b1 = offs->arr[1].u64;
    // validate_tensor_range (model.rs:418-431)
    if (b0 > b1 || b1 > data_bytes)
      return fail(QM_ERR_MODEL_FORMAT, "%s: tensor %s has data offsets outside the shard", sh.path.c_str(),
                  kv.first.c_str());
    ten.shard = shard_index;
    ten.offset = data_offset + b0;
    ten.bytes = b1 - b0;
    out[kv.first] = std::move(ten);
  }
  return QM_OK;
}

qm_status upload_bytes(qm_runtime* rt, const uint8_t* src, uint64_t bytes, void** out) {
  *out = nullptr;
  DeviceGuard g(rt->device);
  if (!g.ok()) return no_device();
  void* dev = nullptr;
  hipError_t e = hipMalloc(&dev, bytes ? bytes : 1);
  if (e != hipSuccess) return hip_check(e, "weight upload allocation");
  // Straight from the mapped file pages (pageable; the HIP runtime stages
  // them), ordered on the runtime's stream.
  if (bytes) e = hipMemcpyAsync(dev, src, bytes, hipMemcpyHostToDevice, rt->stream);
  if (e == hipSuccess) e = hipStreamSynchronize(rt->stream);
  if (e != hipSuccess) {
    (void)hipFree(dev);
    return hip_check(e, "weight upload");
  }
  *out = dev;
  return QM_OK;
}

const Tensor* find(const qm_weight_store* s, const std::string& name) {
  const auto it = s->tensors.find(name);
  return it == s->tensors.end() ? nullptr : &it->second;
}

// validate_affine_tensor (native.rs:5492-5516)
qm_status check_affine(const std::string& weight, const char* label, const Tensor* t, uint64_t rows, uint64_t groups) {
  if (t->dtype != "BF16" || t->shape.size() != 2 || t->shape[0] != rows || t->shape[1] != groups)
    return fail(QM_ERR_INVALID_TENSOR, "%s: %s must be BF16 [%llu, %llu]", weight.c_str(), label,
                (unsigned long long)rows, (unsigned long long)groups);
  if (t->bytes != rows * groups * 2)
    return fail(QM_ERR_INVALID_TENSOR, "%s.%s holds %llu bytes, expected %llu", weight.c_str(), label,
                (unsigned long long)t->bytes, (unsigned long long)(rows * groups * 2));
  return QM_OK;
}

}  // namespace

extern "C" {

qm_status qm_store_open(const char* dir, qm_weight_store** out) {
  if (!dir || !out) return fail(QM_ERR_NULL_POINTER, "NULL argument");
  *out = nullptr;
  const std::string root(dir);
  std::string text;
  const std::string index_path = root + "/model.safetensors.index.json";
  if (!read_file(index_path, text)) return fail(QM_ERR_MODEL_FORMAT, "cannot read %s", index_path.c_str());
  JValue index;
  if (!JParser(text.data(), text.size()).parse(index) || index.kind != JValue::Object)
    return fail(QM_ERR_MODEL_FORMAT, "%s is not a JSON object", index_path.c_str());
  // tensor -> shard, grouped by shard (WeightIndex.weight_map; an absent map is empty)
  std::map<std::string, std::vector<std::string>> by_shard;
  if (const JValue* wm = index.get("weight_map")) {
    if (wm->kind != JValue::Object) return fail(QM_ERR_MODEL_FORMAT, "%s: weight_map is not an object", index_path.c_str());
    for (const auto& kv : wm->obj) {
      if (kv.second.kind != JValue::String)
        return fail(QM_ERR_MODEL_FORMAT, "%s: shard of %s is not a string", index_path.c_str(), kv.first.c_str());
      by_shard[kv.second.str].push_back(kv.first);
    }
  }
  std::unique_ptr<qm_weight_store> store(new qm_weight_store());
  for (const auto& entry : by_shard) {
    if (!safe_relative(entry.first)) return fail(QM_ERR_MODEL_FORMAT, "unsafe shard path %s", entry.first.c_str());
    Shard sh;
    sh.path = root + "/" + entry.first;
    const int fd = open(sh.path.c_str(), O_RDONLY | O_CLOEXEC);
    if (fd < 0) return fail(QM_ERR_MODEL_FORMAT, "cannot open shard %s", sh.path.c_str());
    struct stat st;
    if (fstat(fd, &st) != 0) {
      close(fd);
      return fail(QM_ERR_MODEL_FORMAT, "cannot stat shard %s", sh.path.c_str());
    }
    sh.size = (size_t)st.st_size;
    if (sh.size) {
      void* m = mmap(nullptr, sh.size, PROT_READ, MAP_PRIVATE, fd, 0);
      if (m == MAP_FAILED) {
        close(fd);
        return fail(QM_ERR_MODEL_FORMAT, "cannot map shard %s", sh.path.c_str());
      }
      sh.map = (const uint8_t*)m;
    }
    close(fd);
    const size_t shard_index = store->shards.size();
    store->shards.push_back(sh);
    std::map<std::string, Tensor> header;
    qm_status st_ = parse_shard_header(store->shards.back(), shard_index, header);
    if (st_ != QM_OK) return st_;
    for (const std::string& name : entry.second) {
      const auto it = header.find(name);
      if (it == header.end())
        return fail(QM_ERR_MODEL_FORMAT, "shard %s does not hold indexed tensor %s", sh.path.c_str(), name.c_str());
      store->tensors[name] = it->second;
    }
  }
  *out = store.release();
  return QM_OK;
}

void qm_store_close(qm_weight_store* s) { delete s; }

uint32_t qm_store_tensor_count(const qm_weight_store* s) { return s ? (uint32_t)s->tensors.size() : 0; }

qm_status qm_store_tensor_info(const qm_weight_store* s, const char* name, char* dtype, size_t dtype_cap,
                               uint32_t* ndim, uint64_t* shape, uint32_t shape_cap, uint64_t* bytes) {
  if (!s || !name) return fail(QM_ERR_NULL_POINTER, "NULL argument");
  const Tensor* t = find(s, name);
  if (!t) return fail(QM_ERR_INVALID_TENSOR, "missing tensor %s", name);
  if (dtype && dtype_cap) {
    const size_t n = std::min(dtype_cap - 1, t->dtype.size());
    memcpy(dtype, t->dtype.data(), n);
    dtype[n] = '\0';
  }
  if (ndim) *ndim = (uint32_t)t->shape.size();
  if (shape)
    for (uint32_t i = 0; i < shape_cap && i < t->shape.size(); ++i) shape[i] = t->shape[i];
  if (bytes) *bytes = t->bytes;
  return QM_OK;
}

qm_status qm_store_upload(qm_runtime* rt, const qm_weight_store* s, const char* name, void** out, uint64_t* bytes) {
  if (!rt || !s || !name || !out) return fail(QM_ERR_NULL_POINTER, "NULL argument");
  *out = nullptr;
  const Tensor* t = find(s, name);
  if (!t) return fail(QM_ERR_INVALID_TENSOR, "missing tensor %s", name);
  if (bytes) *bytes = t->bytes;
  return upload_bytes(rt, s->shards[t->shard].map + t->offset, t->bytes, out);
}

qm_status qm_store_upload_q4(qm_runtime* rt, const qm_weight_store* s, const char* weight_name, qm_q4_matrix* out) {
  if (!rt || !s || !weight_name || !out) return fail(QM_ERR_NULL_POINTER, "NULL argument");
  memset(out, 0, sizeof(*out));
  const std::string name(weight_name);
  // Q4AffineMatrix::from_store / from_tensors (native.rs:5398-5490)
  const Tensor* w = find(s, name);
  if (!w) return fail(QM_ERR_INVALID_TENSOR, "missing tensor %s", name.c_str());
  const std::string suffix = ".weight";
  if (name.size() <= suffix.size() || name.compare(name.size() - suffix.size(), suffix.size(), suffix) != 0)
    return fail(QM_ERR_INVALID_TENSOR, "%s is not a quantized weight (no .weight suffix)", name.c_str());
  const std::string base = name.substr(0, name.size() - suffix.size());
  const Tensor* sc = find(s, base + ".scales");
  const Tensor* bi = find(s, base + ".biases");
  if (!sc) return fail(QM_ERR_INVALID_TENSOR, "missing tensor %s.scales", base.c_str());
  if (!bi) return fail(QM_ERR_INVALID_TENSOR, "missing tensor %s.biases", base.c_str());
  if (w->dtype != "U32" || w->shape.size() != 2)
    return fail(QM_ERR_INVALID_TENSOR, "%s must be a U32 matrix", name.c_str());
  const uint64_t rows = w->shape[0], words = w->shape[1];
  if (words > UINT64_MAX / 8) return fail(QM_ERR_DIMENSION_OVERFLOW, "%s", name.c_str());
  const uint64_t K = words * 8;
  if (rows == 0 || K == 0 || K % 64 != 0)
    return fail(QM_ERR_INVALID_TENSOR, "%s: shape [%llu, %llu] is not a grouped Q4 matrix", name.c_str(),
                (unsigned long long)rows, (unsigned long long)words);
  if (rows > 0xFFFFFFFFull || K > 0xFFFFFFFFull || rows > UINT64_MAX / (words * 4))
    return fail(QM_ERR_DIMENSION_OVERFLOW, "%s", name.c_str());
  if (w->bytes != rows * words * 4)
    return fail(QM_ERR_INVALID_TENSOR, "%s holds %llu bytes, expected %llu", name.c_str(),
                (unsigned long long)w->bytes, (unsigned long long)(rows * words * 4));
  qm_status st = check_affine(name, "scales", sc, rows, K / 64);
  if (st == QM_OK) st = check_affine(name, "biases", bi, rows, K / 64);
  if (st != QM_OK) return st;
  void *dw = nullptr, *ds = nullptr, *db = nullptr;
  st = upload_bytes(rt, s->shards[w->shard].map + w->offset, w->bytes, &dw);
  if (st == QM_OK) st = upload_bytes(rt, s->shards[sc->shard].map + sc->offset, sc->bytes, &ds);
  if (st == QM_OK) st = upload_bytes(rt, s->shards[bi->shard].map + bi->offset, bi->bytes, &db);
  if (st != QM_OK) {
    DeviceGuard g(rt->device);
    (void)hipFree(dw);
    (void)hipFree(ds);
    (void)hipFree(db);
    return st;
  }
  out->weights = (uint32_t*)dw;
  out->scales = (uint16_t*)ds;
  out->biases = (uint16_t*)db;
  out->out_rows = (uint32_t)rows;
  out->in_elems = (uint32_t)K;
  return QM_OK;
}

}  // extern "C"
