// moe_checkpoint.hip -- safetensors checkpoints for the MoE layer
// (gptoss_checkpoint_* and the upload behind
// gptoss_moe_layer_init_from_checkpoint).
//
// Covers the MoE part of gptoss::WeightLoader (src/memory/weight_loader.cu):
// shard discovery, mmap and header parsing (:297-345, 456-575), the packed
// and per-expert MXFP4 expert formats (:782-895) and the router, norm and
// bias tensors (:1083-1165).  Differences by design:
//  - one device allocation per layer instead of one hipMalloc per tensor and
//    per expert;
//  - the MXFP4 experts go straight into the tiled expert-major layout the
//    kernels read: expert matrices stream through two pinned host slots and
//    two device slots, so copying out of the mapping (several threads) for
//    one chunk of experts overlaps the host-to-device copy and the on-device
//    repack of the previous chunk;
//  - malformed files, missing tensors and shape mismatches return an error
//    code instead of aborting.
#include <hip/hip_runtime.h>

#include <dirent.h>
#include <fcntl.h>
#include <sys/mman.h>
#include <sys/stat.h>
#include <unistd.h>

#include <algorithm>
#include <memory>
#include <mutex>
#include <cerrno>
#include <cstdint>
#include <cstring>
#include <string>
#include <thread>
#include <unordered_map>
#include <vector>

#include "../../include/gptoss_moe.h"
#include "moe_checkpoint.h"
#include "moe_kernels.h"
#include "moe_stages.h"
#include "moe_status.h"

using namespace gxmoe;

namespace {

constexpr size_t kMaxHeaderBytes = size_t(100) << 20;  // safetensors' own header limit
constexpr size_t kDefaultStaging = size_t(32) << 20;
constexpr int kMaxDims = 8;

struct Shard {
  std::string path;
  int fd = -1;
  uint8_t* base = nullptr;  // whole-file mapping
  size_t size = 0;
  const uint8_t* data = nullptr;  // first byte after the header
  size_t data_len = 0;
};

struct Tensor {
  std::string name;
  std::string dtype;
  int ndim = 0;
  int64_t shape[kMaxDims] = {0};
  uint64_t begin = 0, end = 0;
  int shard = 0;
};

// Bytes per element of the safetensors dtypes; 0 for names outside the
// format's list (their sizes are then not checked).
size_t dtype_bytes(const std::string& d) {
  if (d == "BOOL" || d == "U8" || d == "I8" || d == "F8_E4M3" || d == "F8_E5M2") return 1;
  if (d == "BF16" || d == "F16" || d == "I16" || d == "U16") return 2;
  if (d == "F32" || d == "I32" || d == "U32") return 4;
  if (d == "F64" || d == "I64" || d == "U64") return 8;
  return 0;
}

// ---- header JSON ----------------------------------------------------------
// The header is one JSON object: tensor name -> {"dtype", "shape",
// "data_offsets"}, plus an optional "__metadata__" object (skipped).
struct Json {
  const char* p;
  const char* end;
  std::string err;

  void ws() {
    while (p < end && (*p == ' ' || *p == '\t' || *p == '\n' || *p == '\r')) ++p;
  }
  bool peek(char c) {
    ws();
    return p < end && *p == c;
  }
  bool eat(char c) {
    if (!peek(c)) return false;
    ++p;
    return true;
  }
  bool expect(char c) {
    if (eat(c)) return true;
    err = std::string("expected '") + c + "'";
    return false;
  }
  static int hex(char c) {
    if (c >= '0' && c <= '9') return c - '0';
    if (c >= 'a' && c <= 'f') return c - 'a' + 10;
    if (c >= 'A' && c <= 'F') return c - 'A' + 10;
    return -1;
  }
  bool u4(uint32_t& v) {
    if (end - p < 4) return false;
    v = 0;
    for (int i = 0; i < 4; ++i) {
      const int h = hex(p[i]);
      if (h < 0) return false;
      v = v * 16 + static_cast<uint32_t>(h);
    }
    p += 4;
    return true;
  }
  static void utf8(std::string& out, uint32_t cp) {
    if (cp < 0x80) {
      out += static_cast<char>(cp);
    } else if (cp < 0x800) {
      out += static_cast<char>(0xc0 | (cp >> 6));
      out += static_cast<char>(0x80 | (cp & 0x3f));
    } else if (cp < 0x10000) {
      out += static_cast<char>(0xe0 | (cp >> 12));
      out += static_cast<char>(0x80 | ((cp >> 6) & 0x3f));
      out += static_cast<char>(0x80 | (cp & 0x3f));
    } else {
      out += static_cast<char>(0xf0 | (cp >> 18));
      out += static_cast<char>(0x80 | ((cp >> 12) & 0x3f));
      out += static_cast<char>(0x80 | ((cp >> 6) & 0x3f));
      out += static_cast<char>(0x80 | (cp & 0x3f));
    }
  }
  bool string(std::string& out) {
    out.clear();
    if (!expect('"')) return false;
    while (p < end) {
      const char c = *p++;
      if (c == '"') return true;
      if (static_cast<unsigned char>(c) < 0x20) {
        err = "control character in string";
        return false;
      }
      if (c != '\\') {
        // JSON text is UTF-8 (and safetensors requires it): take whole,
        // well-formed sequences only
        const int n = utf8_seq_len(reinterpret_cast<const unsigned char*>(p - 1), static_cast<size_t>(end - p + 1));
        if (n == 0) {
          err = "string is not UTF-8";
          return false;
        }
        out.append(p - 1, static_cast<size_t>(n));
        p += n - 1;
        continue;
      }
      if (p >= end) break;
      const char e = *p++;
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
          uint32_t cp;
          if (!u4(cp)) {
            err = "bad \\u escape";
            return false;
          }
          if (cp >= 0xd800 && cp < 0xdc00 && end - p >= 6 && p[0] == '\\' && p[1] == 'u') {
            const char* save = p;
            p += 2;
            uint32_t lo;
            if (u4(lo) && lo >= 0xdc00 && lo < 0xe000) {
              cp = 0x10000 + ((cp - 0xd800) << 10) + (lo - 0xdc00);
            } else {
              p = save;
            }
          }
          // a surrogate left unpaired has no UTF-8 form; NUL cannot pass
          // the C ABI's name strings
          if ((cp >= 0xd800 && cp < 0xe000) || cp == 0) {
            err = cp == 0 ? "NUL in string" : "unpaired surrogate in \\u escape";
            return false;
          }
          utf8(out, cp);
          break;
        }
        default:
          err = "bad escape in string";
          return false;
      }
    }
    err = "unterminated string";
    return false;
  }
  // A JSON integer (no fraction or exponent), as the offsets and dims are.
  bool integer(int64_t& v) {
    ws();
    bool neg = false;
    if (p < end && *p == '-') {
      neg = true;
      ++p;
    }
    if (p >= end || *p < '0' || *p > '9') {
      err = "expected an integer";
      return false;
    }
    uint64_t u = 0;
    while (p < end && *p >= '0' && *p <= '9') {
      const uint64_t d = static_cast<uint64_t>(*p - '0');
      if (u > (UINT64_C(0x7fffffffffffffff) - d) / 10) {
        err = "integer out of range";
        return false;
      }
      u = u * 10 + d;
      ++p;
    }
    if (p < end && (*p == '.' || *p == 'e' || *p == 'E')) {
      err = "expected an integer";
      return false;
    }
    v = neg ? -static_cast<int64_t>(u) : static_cast<int64_t>(u);
    return true;
  }
  bool literal(const char* word) {
    const size_t n = strlen(word);
    if (static_cast<size_t>(end - p) < n || memcmp(p, word, n) != 0) {
      err = "bad literal";
      return false;
    }
    p += n;
    return true;
  }
  bool skip(int depth) {
    if (depth > 64) {
      err = "nesting too deep";
      return false;
    }
    ws();
    if (p >= end) {
      err = "unexpected end of header";
      return false;
    }
    std::string tmp;
    switch (*p) {
      case '"': return string(tmp);
      case '{':
        ++p;
        if (eat('}')) return true;
        do {
          if (!string(tmp) || !expect(':') || !skip(depth + 1)) return false;
        } while (eat(','));
        return expect('}');
      case '[':
        ++p;
        if (eat(']')) return true;
        do {
          if (!skip(depth + 1)) return false;
        } while (eat(','));
        return expect(']');
      case 't': return literal("true");
      case 'f': return literal("false");
      case 'n': return literal("null");
      default: {
        // number: sign, digits, fraction, exponent
        const char* s = p;
        if (*p == '-') ++p;
        while (p < end && ((*p >= '0' && *p <= '9') || *p == '.' || *p == 'e' || *p == 'E' || *p == '+' ||
                           *p == '-'))
          ++p;
        if (p == s) {
          err = "unexpected character";
          return false;
        }
        return true;
      }
    }
  }
  bool int_array(std::vector<int64_t>& out) {
    out.clear();
    if (!expect('[')) return false;
    if (eat(']')) return true;
    do {
      int64_t v;
      if (!integer(v)) return false;
      out.push_back(v);
    } while (eat(','));
    return expect(']');
  }
};

// One tensor's entry: {"dtype": "...", "shape": [...], "data_offsets": [b, e]}.
bool parse_entry(Json& j, Tensor& t) {
  bool has_dtype = false, has_shape = false, has_off = false;
  if (!j.expect('{')) return false;
  if (!j.eat('}')) {
    do {
      std::string key;
      if (!j.string(key) || !j.expect(':')) return false;
      if (key == "dtype") {
        if (!j.string(t.dtype)) return false;
        has_dtype = true;
      } else if (key == "shape") {
        std::vector<int64_t> v;
        if (!j.int_array(v)) return false;
        if (v.size() > static_cast<size_t>(kMaxDims)) {
          j.err = "more than 8 dimensions";
          return false;
        }
        t.ndim = static_cast<int>(v.size());
        for (int i = 0; i < t.ndim; ++i) t.shape[i] = v[i];
        has_shape = true;
      } else if (key == "data_offsets") {
        std::vector<int64_t> v;
        if (!j.int_array(v)) return false;
        if (v.size() != 2 || v[0] < 0 || v[1] < v[0]) {
          j.err = "data_offsets must be [begin, end] with 0 <= begin <= end";
          return false;
        }
        t.begin = static_cast<uint64_t>(v[0]);
        t.end = static_cast<uint64_t>(v[1]);
        has_off = true;
      } else if (!j.skip(1)) {
        return false;
      }
    } while (j.eat(','));
    if (!j.expect('}')) return false;
  }
  if (!has_dtype || !has_shape || !has_off) {
    j.err = "entry lacks dtype, shape or data_offsets";
    return false;
  }
  return true;
}

// Element count of a shape, or -1 for a negative or overflowing shape.
int64_t numel_of(const int64_t* shape, int ndim) {
  int64_t n = 1;
  for (int i = 0; i < ndim; ++i) {
    if (shape[i] < 0) return -1;
    if (shape[i] != 0 && n > (INT64_C(1) << 62) / shape[i]) return -1;
    n *= shape[i];
  }
  return n;
}

std::string shape_str(const Tensor& t) {
  std::string s = "[";
  for (int i = 0; i < t.ndim; ++i) s += (i ? "," : "") + std::to_string(t.shape[i]);
  return s + "]";
}

// ---- host conversions to bf16 ---------------------------------------------
uint16_t bf16_from_f32(uint32_t u) {
  if ((u & 0x7fffffffu) > 0x7f800000u) return static_cast<uint16_t>((u >> 16) | 0x40u);  // quiet NaN
  u += 0x7fffu + ((u >> 16) & 1u);  // round to nearest even
  return static_cast<uint16_t>(u >> 16);
}

uint32_t f32_from_f16(uint16_t h) {
  const uint32_t sign = static_cast<uint32_t>(h & 0x8000u) << 16;
  uint32_t ex = (h >> 10) & 0x1fu, man = h & 0x3ffu;
  if (ex == 0x1f) return sign | 0x7f800000u | (man << 13);
  if (ex != 0) return sign | ((ex + 112u) << 23) | (man << 13);
  if (man == 0) return sign;
  // subnormal: man * 2^-24, normalised
  uint32_t e = 113;
  while ((man & 0x400u) == 0) {
    man <<= 1;
    --e;
  }
  return sign | (e << 23) | ((man & 0x3ffu) << 13);
}

// Parallel copy of a list of (dst, src, bytes) pieces out of the mapping.
struct Piece {
  uint8_t* dst;
  const uint8_t* src;
  size_t n;
};

void copy_pieces(const std::vector<Piece>& pieces) {
  size_t total = 0;
  for (const Piece& q : pieces) total += q.n;
  const unsigned hw = std::max(1u, std::thread::hardware_concurrency());
  const size_t nt = std::min<size_t>({size_t(8), hw, std::max<size_t>(1, total >> 22)});
  auto run = [&](size_t lo, size_t hi) {
    size_t at = 0;
    for (const Piece& q : pieces) {
      const size_t a = std::max(lo, at), b = std::min(hi, at + q.n);
      if (a < b) memcpy(q.dst + (a - at), q.src + (a - at), b - a);
      at += q.n;
      if (at >= hi) break;
    }
  };
  if (nt <= 1) {
    run(0, total);
    return;
  }
  std::vector<std::thread> th;
  size_t started = 0;
  try {
    th.reserve(nt);
    for (; started < nt; ++started) th.emplace_back(run, total * started / nt, total * (started + 1) / nt);
  } catch (...) {
    // fewer threads than asked for: this thread copies the ranges not handed out
  }
  for (size_t t = started; t < nt; ++t) run(total * t / nt, total * (t + 1) / nt);
  for (std::thread& t : th) t.join();
}

// Ask the kernel to start reading a source range ahead of its copy.
void prefetch(const uint8_t* p, size_t n) {
  const uintptr_t pg = static_cast<uintptr_t>(sysconf(_SC_PAGESIZE));
  const uintptr_t a = reinterpret_cast<uintptr_t>(p) & ~(pg - 1);
  (void)madvise(reinterpret_cast<void*>(a), reinterpret_cast<uintptr_t>(p) + n - a, MADV_WILLNEED);
}

size_t align_up(size_t x, size_t a) { return (x + a - 1) / a * a; }

// Two pinned host slots and two device slots on one device; slot i is free
// again once its event has completed.  A checkpoint keeps its staging per
// device between layer loads, so a model load pins host memory once.
struct Staging {
  int device = 0;
  uint8_t* host = nullptr;
  uint8_t* dev = nullptr;
  size_t slot = 0;
  hipStream_t stream = nullptr;
  hipEvent_t ev[2] = {nullptr, nullptr};
  bool pending[2] = {false, false};
  int next = 0;

  hipError_t init(int device_id, size_t bytes) {
    device = device_id;
    slot = bytes;
    hipError_t e = hipHostMalloc(reinterpret_cast<void**>(&host), 2 * slot, hipHostMallocDefault);
    if (e == hipSuccess) e = hipMalloc(reinterpret_cast<void**>(&dev), 2 * slot);
    if (e == hipSuccess) e = hipStreamCreateWithFlags(&stream, hipStreamNonBlocking);
    for (int i = 0; i < 2 && e == hipSuccess; ++i) e = hipEventCreateWithFlags(&ev[i], hipEventDisableTiming);
    return e;
  }
  ~Staging() {
    int prev = -1;
    const bool swap = hipGetDevice(&prev) == hipSuccess && prev != device && hipSetDevice(device) == hipSuccess;
    if (stream) (void)hipStreamSynchronize(stream);
    for (hipEvent_t x : ev)
      if (x) (void)hipEventDestroy(x);
    if (stream) (void)hipStreamDestroy(stream);
    if (dev) (void)hipFree(dev);
    if (host) (void)hipHostFree(host);
    if (swap) (void)hipSetDevice(prev);
  }
};


}  // namespace

struct gptoss_checkpoint {
  std::vector<Shard> shards;
  std::vector<Tensor> tensors;
  std::unordered_map<std::string, int> index;
  size_t staging = kDefaultStaging;
  // staging per device, kept between layer loads; loads from one checkpoint
  // take the lock, so they run one at a time
  mutable std::mutex mu;
  mutable std::vector<std::unique_ptr<Staging>> stagings;

  // The staging of `device` with slots of `slot` bytes, made or remade on
  // demand.  Caller holds mu; `device` is current.
  Staging* staging_for(int device, size_t slot, hipError_t* err) const {
    *err = hipSuccess;
    for (auto& st : stagings) {
      if (st->device != device) continue;
      if (st->slot == slot) return st.get();
      st.reset();
      st = std::unique_ptr<Staging>(new Staging());
      *err = st->init(device, slot);
      return *err == hipSuccess ? st.get() : nullptr;
    }
    stagings.emplace_back(new Staging());
    *err = stagings.back()->init(device, slot);
    return *err == hipSuccess ? stagings.back().get() : nullptr;
  }

  ~gptoss_checkpoint() {
    stagings.clear();
    for (Shard& s : shards) {
      if (s.base) munmap(s.base, s.size);
      if (s.fd >= 0) close(s.fd);
    }
  }
  const Tensor* find(const std::string& name) const {
    auto it = index.find(name);
    return it == index.end() ? nullptr : &tensors[it->second];
  }
  const uint8_t* data(const Tensor& t) const { return shards[t.shard].data + t.begin; }
};

namespace {

int open_shard(gptoss_checkpoint* ck, const std::string& path) {
  Shard sh;
  sh.path = path;
  sh.fd = open(path.c_str(), O_RDONLY | O_CLOEXEC);
  if (sh.fd < 0) return set_error(GPTOSS_ERR_IO, "cannot open %s: %s", path.c_str(), strerror(errno));
  struct stat st;
  if (fstat(sh.fd, &st) != 0) {
    const int e = errno;
    close(sh.fd);
    return set_error(GPTOSS_ERR_IO, "cannot stat %s: %s", path.c_str(), strerror(e));
  }
  sh.size = static_cast<size_t>(st.st_size);
  if (sh.size < 8) {
    close(sh.fd);
    return set_error(GPTOSS_ERR_IO, "%s: %zu bytes is too short for a safetensors file", path.c_str(), sh.size);
  }
  void* m = mmap(nullptr, sh.size, PROT_READ, MAP_PRIVATE, sh.fd, 0);
  if (m == MAP_FAILED) {
    const int e = errno;
    close(sh.fd);
    return set_error(GPTOSS_ERR_IO, "cannot map %s: %s", path.c_str(), strerror(e));
  }
  sh.base = static_cast<uint8_t*>(m);
  (void)madvise(sh.base, sh.size, MADV_SEQUENTIAL);
  const int idx = static_cast<int>(ck->shards.size());
  ck->shards.push_back(sh);  // owned from here on: closed by the destructor
  Shard& s = ck->shards.back();

  uint64_t hlen = 0;
  memcpy(&hlen, s.base, 8);  // little-endian u64
  if (hlen > s.size - 8 || hlen > kMaxHeaderBytes)
    return set_error(GPTOSS_ERR_IO, "%s: header length %llu exceeds the file (%zu bytes)", path.c_str(),
                     static_cast<unsigned long long>(hlen), s.size);
  s.data = s.base + 8 + hlen;
  s.data_len = s.size - 8 - hlen;

  Json j{reinterpret_cast<const char*>(s.base + 8), reinterpret_cast<const char*>(s.base + 8 + hlen), {}};
  bool good = j.expect('{');
  if (good && !j.eat('}')) {
    do {
      std::string key;
      if (!(good = j.string(key) && j.expect(':'))) break;
      if (key == "__metadata__") {
        if (!(good = j.skip(1))) break;
        continue;
      }
      Tensor t;
      t.name = key;
      t.shard = idx;
      if (!(good = parse_entry(j, t))) {
        j.err = "tensor '" + key + "': " + j.err;
        break;
      }
      if (t.end > s.data_len) {
        return set_error(GPTOSS_ERR_IO, "%s: tensor '%s' ends at byte %llu past the data (%zu bytes)",
                         path.c_str(), key.c_str(), static_cast<unsigned long long>(t.end), s.data_len);
      }
      const int64_t n = numel_of(t.shape, t.ndim);
      const size_t eb = dtype_bytes(t.dtype);
      if (n < 0) return set_error(GPTOSS_ERR_IO, "%s: tensor '%s' has a bad shape", path.c_str(), key.c_str());
      if (eb != 0 && static_cast<uint64_t>(n) * eb != t.end - t.begin)
        return set_error(GPTOSS_ERR_IO, "%s: tensor '%s' %s %s holds %llu bytes, expected %llu", path.c_str(),
                         key.c_str(), t.dtype.c_str(), shape_str(t).c_str(),
                         static_cast<unsigned long long>(t.end - t.begin),
                         static_cast<unsigned long long>(static_cast<uint64_t>(n) * eb));
      ck->tensors.push_back(std::move(t));
    } while (j.eat(','));
    if (good) good = j.expect('}');
  }
  if (good) {
    j.ws();
    if (j.p != j.end) {
      good = false;
      j.err = "trailing bytes after the header object";
    }
  }
  if (!good) return set_error(GPTOSS_ERR_IO, "%s: bad safetensors header: %s", path.c_str(), j.err.c_str());
  return GPTOSS_OK;
}

bool ends_with(const std::string& s, const char* suf) {
  const size_t n = strlen(suf);
  return s.size() > n && s.compare(s.size() - n, n, suf) == 0;
}

// ---- layer upload ------------------------------------------------------------

// A bf16 tensor of the given shape, converted on the host if stored as F32
// or F16.  Empty `out` with GPTOSS_OK when the tensor is absent and optional.
int read_bf16(const gptoss_checkpoint* ck, const Tensor* t, std::initializer_list<int64_t> shape,
              std::vector<uint16_t>& out) {
  const std::vector<int64_t> want(shape);
  bool same = t->ndim == static_cast<int>(want.size());
  for (int i = 0; same && i < t->ndim; ++i) same = t->shape[i] == want[i];
  if (!same) {
    std::string w = "[";
    for (size_t i = 0; i < want.size(); ++i) w += (i ? "," : "") + std::to_string(want[i]);
    return set_error(GPTOSS_ERR_INVALID, "tensor '%s' has shape %s, expected %s]", t->name.c_str(),
                     shape_str(*t).c_str(), w.c_str());
  }
  const size_t n = static_cast<size_t>(numel_of(t->shape, t->ndim));
  const uint8_t* src = ck->data(*t);
  out.resize(n);
  if (t->dtype == "BF16") {
    memcpy(out.data(), src, n * 2);
  } else if (t->dtype == "F32") {
    for (size_t i = 0; i < n; ++i) {
      uint32_t u;
      memcpy(&u, src + 4 * i, 4);
      out[i] = bf16_from_f32(u);
    }
  } else if (t->dtype == "F16") {
    for (size_t i = 0; i < n; ++i) {
      uint16_t h;
      memcpy(&h, src + 2 * i, 2);
      out[i] = bf16_from_f32(f32_from_f16(h));
    }
  } else {
    return set_error(GPTOSS_ERR_INVALID, "tensor '%s' has dtype %s (expected BF16, F32 or F16)", t->name.c_str(),
                     t->dtype.c_str());
  }
  return GPTOSS_OK;
}

// Where expert e's packed [N][K/2] nibbles and [N][K/32] scales lie in the
// mapping.
struct ExpertSource {
  std::vector<const uint8_t*> blocks, scales;
};

bool is_byte_dtype(const std::string& d) { return d == "U8" || d == "I8"; }

// Packed format: one [E][N][K/32][16] (or [E][N][K/2]) blocks tensor and one
// [E][N][K/32] scales tensor for all experts (weight_loader.cu:782-842).
int packed_source(const gptoss_checkpoint* ck, const Tensor* b, const Tensor* s, int E, int N, int K,
                  ExpertSource& src) {
  if (!s) return set_error(GPTOSS_ERR_NOT_FOUND, "tensor '%s' has no scales tensor beside it", b->name.c_str());
  const bool b_ok = is_byte_dtype(b->dtype) &&
                    ((b->ndim == 4 && b->shape[0] == E && b->shape[1] == N && b->shape[2] == K / 32 &&
                      b->shape[3] == 16) ||
                     (b->ndim == 3 && b->shape[0] == E && b->shape[1] == N && b->shape[2] == K / 2));
  if (!b_ok)
    return set_error(GPTOSS_ERR_INVALID, "tensor '%s' is %s %s, expected U8 [%d,%d,%d,16]", b->name.c_str(),
                     b->dtype.c_str(), shape_str(*b).c_str(), E, N, K / 32);
  const bool s_ok = is_byte_dtype(s->dtype) && s->ndim == 3 && s->shape[0] == E && s->shape[1] == N &&
                    s->shape[2] == K / 32;
  if (!s_ok)
    return set_error(GPTOSS_ERR_INVALID, "tensor '%s' is %s %s, expected U8 [%d,%d,%d]", s->name.c_str(),
                     s->dtype.c_str(), shape_str(*s).c_str(), E, N, K / 32);
  const size_t nb = static_cast<size_t>(N) * K / 2, sb = static_cast<size_t>(N) * K / 32;
  for (int e = 0; e < E; ++e) {
    src.blocks.push_back(ck->data(*b) + nb * e);
    src.scales.push_back(ck->data(*s) + sb * e);
  }
  return GPTOSS_OK;
}

// Per-expert format: mlp.experts.<e>.<name>.weight and .weight_scale
// (weight_loader.cu:847-895; the first name present wins).
int per_expert_source(const gptoss_checkpoint* ck, const std::string& prefix, int E, int N, int K,
                      const char* const* names, int n_names, const char* const* scale_names, int n_scale_names,
                      ExpertSource& src) {
  const size_t nb = static_cast<size_t>(N) * K / 2, sb = static_cast<size_t>(N) * K / 32;
  for (int e = 0; e < E; ++e) {
    const std::string base = prefix + "mlp.experts." + std::to_string(e) + ".";
    const Tensor *b = nullptr, *s = nullptr;
    for (int i = 0; i < n_names && !b; ++i) b = ck->find(base + names[i] + ".weight");
    for (int i = 0; i < n_scale_names && !s; ++i) s = ck->find(base + scale_names[i] + ".weight_scale");
    if (!b)
      return set_error(GPTOSS_ERR_NOT_FOUND, "expert %d: no %s%s.weight (nor the other names) in the checkpoint", e,
                       base.c_str(), names[0]);
    if (!s)
      return set_error(GPTOSS_ERR_NOT_FOUND, "expert %d: no %s%s.weight_scale in the checkpoint", e, base.c_str(),
                       scale_names[0]);
    if (!is_byte_dtype(b->dtype) || b->end - b->begin != nb || b->ndim < 1 || b->shape[0] != N)
      return set_error(GPTOSS_ERR_INVALID, "tensor '%s' is %s %s, expected %zu bytes of U8 with %d rows",
                       b->name.c_str(), b->dtype.c_str(), shape_str(*b).c_str(), nb, N);
    if (!is_byte_dtype(s->dtype) || s->end - s->begin != sb || s->ndim < 1 || s->shape[0] != N)
      return set_error(GPTOSS_ERR_INVALID, "tensor '%s' is %s %s, expected %zu bytes of U8 with %d rows",
                       s->name.c_str(), s->dtype.c_str(), shape_str(*s).c_str(), sb, N);
    src.blocks.push_back(ck->data(*b));
    src.scales.push_back(ck->data(*s));
  }
  return GPTOSS_OK;
}

// Stream E expert matrices [N][K] from the mapping into the tiled buffers:
// chunks of experts fill a pinned slot (threads copying out of the mapping),
// one host-to-device copy moves the slot, and one repack launch per expert
// writes its tiled nibbles and scales.
int upload_experts(Staging& st, const ExpertSource& src, int E, int N, int K, uint8_t* nib, uint8_t* sc) {
  const TiledGeom g = tiled_geom(N, K);
  const size_t nb = static_cast<size_t>(N) * K / 2, sb = static_cast<size_t>(N) * K / 32;
  const size_t per = align_up(nb, 256) + align_up(sb, 256);
  const int cpe = static_cast<int>(std::max<size_t>(1, st.slot / per));
  for (int e0 = 0; e0 < E; e0 += cpe) {
    const int ne = std::min(cpe, E - e0);
    const int s = st.next;
    st.next ^= 1;
    if (st.pending[s]) {
      hipError_t e = hipEventSynchronize(st.ev[s]);
      if (e != hipSuccess) return set_error(GPTOSS_ERR_HIP, "staging event: %s", hipGetErrorString(e));
    }
    uint8_t* h = st.host + st.slot * s;
    uint8_t* d = st.dev + st.slot * s;
    std::vector<Piece> pieces;
    for (int i = 0; i < ne; ++i) {
      pieces.push_back({h + per * i, src.blocks[e0 + i], nb});
      pieces.push_back({h + per * i + align_up(nb, 256), src.scales[e0 + i], sb});
    }
    copy_pieces(pieces);
    // the next chunk's source pages, read ahead while this one moves
    for (int i = ne; i < 2 * ne && e0 + i < E; ++i) {
      prefetch(src.blocks[e0 + i], nb);
      prefetch(src.scales[e0 + i], sb);
    }
    hipError_t e = hipMemcpyAsync(d, h, per * ne, hipMemcpyHostToDevice, st.stream);
    for (int i = 0; i < ne && e == hipSuccess; ++i)
      e = launch_pack_tiled(d + per * i, d + per * i + align_up(nb, 256), N, K, nib + g.nib_bytes * (e0 + i),
                            sc + g.scale_bytes * (e0 + i), st.stream);
    if (e == hipSuccess) e = hipEventRecord(st.ev[s], st.stream);
    if (e != hipSuccess) return set_error(GPTOSS_ERR_HIP, "expert upload: %s", hipGetErrorString(e));
    st.pending[s] = true;
  }
  return GPTOSS_OK;
}

}  // namespace

extern "C" {

static int gptoss_checkpoint_open_impl(const char* path, gptoss_checkpoint** out) {
  if (path == nullptr || out == nullptr) return set_error(GPTOSS_ERR_INVALID, "null argument");
  *out = nullptr;
  struct stat st;
  if (stat(path, &st) != 0) return set_error(GPTOSS_ERR_NOT_FOUND, "%s: %s", path, strerror(errno));
  std::vector<std::string> files;
  if (S_ISDIR(st.st_mode)) {
    DIR* dir = opendir(path);
    if (!dir) return set_error(GPTOSS_ERR_IO, "cannot open directory %s: %s", path, strerror(errno));
    while (struct dirent* de = readdir(dir)) {
      const std::string name = de->d_name;
      if (ends_with(name, ".safetensors")) files.push_back(std::string(path) + "/" + name);
    }
    closedir(dir);
    std::sort(files.begin(), files.end());
    if (files.empty()) return set_error(GPTOSS_ERR_NOT_FOUND, "no .safetensors files in %s", path);
  } else {
    files.push_back(path);
  }
  std::unique_ptr<gptoss_checkpoint> ck(new gptoss_checkpoint());
  for (const std::string& f : files) {
    const int rc = open_shard(ck.get(), f);
    if (rc != GPTOSS_OK) return rc;
  }
  // name -> tensor; a later shard's entry replaces an earlier one
  for (size_t i = 0; i < ck->tensors.size(); ++i) ck->index[ck->tensors[i].name] = static_cast<int>(i);
  *out = ck.release();
  clear_error();
  return GPTOSS_OK;
}

int gptoss_checkpoint_open(const char* path, gptoss_checkpoint** out) {
  return guarded([&] { return gptoss_checkpoint_open_impl(path, out); });
}

void gptoss_checkpoint_close(gptoss_checkpoint* ckpt) { delete ckpt; }

int gptoss_checkpoint_num_tensors(const gptoss_checkpoint* ckpt) {
  return ckpt ? static_cast<int>(ckpt->tensors.size()) : 0;
}

static void fill_info(const gptoss_checkpoint* ck, const Tensor& t, gptoss_tensor_info* info) {
  info->name = t.name.c_str();
  info->dtype = t.dtype.c_str();
  info->ndim = t.ndim;
  for (int i = 0; i < kMaxDims; ++i) info->shape[i] = i < t.ndim ? t.shape[i] : 0;
  info->nbytes = t.end - t.begin;
  info->data = ck->data(t);
  info->shard = t.shard;
}

int gptoss_checkpoint_tensor_at(const gptoss_checkpoint* ckpt, int i, gptoss_tensor_info* info) {
  if (!ckpt || !info) return set_error(GPTOSS_ERR_INVALID, "null argument");
  if (i < 0 || i >= static_cast<int>(ckpt->tensors.size()))
    return set_error(GPTOSS_ERR_INVALID, "tensor index %d outside [0, %zu)", i, ckpt->tensors.size());
  fill_info(ckpt, ckpt->tensors[i], info);
  clear_error();
  return GPTOSS_OK;
}

static int gptoss_checkpoint_find_impl(const gptoss_checkpoint* ckpt, const char* name,
                                       gptoss_tensor_info* info) {
  if (!ckpt || !name) return set_error(GPTOSS_ERR_INVALID, "null argument");
  const Tensor* t = ckpt->find(name);
  if (!t) return set_error(GPTOSS_ERR_NOT_FOUND, "tensor '%s' not found", name);
  if (info) fill_info(ckpt, *t, info);
  clear_error();
  return GPTOSS_OK;
}

int gptoss_checkpoint_find(const gptoss_checkpoint* ckpt, const char* name, gptoss_tensor_info* info) {
  return guarded([&] { return gptoss_checkpoint_find_impl(ckpt, name, info); });
}

int gptoss_checkpoint_set_staging_bytes(gptoss_checkpoint* ckpt, size_t bytes) {
  if (!ckpt) return set_error(GPTOSS_ERR_INVALID, "null argument");
  if (bytes == 0) return set_error(GPTOSS_ERR_INVALID, "staging bytes must be positive");
  ckpt->staging = bytes;
  clear_error();
  return GPTOSS_OK;
}

}  // extern "C"

namespace gxmoe {

struct LayerSource {
  const gptoss_checkpoint* ck = nullptr;
  int E = 0, H = 0, I = 0;
  std::vector<uint16_t> v_rw, v_rb, v_nw, v_b1, v_b2;  // bf16, converted on the host
  ExpertSource s1, s2;                                // gate_up [2I][H], down [H][I]
};

}  // namespace gxmoe

namespace {

int resolve(const gptoss_checkpoint* ck, const gptoss_moe_config& cfg, int layer, LayerSource& L) {
  const int H = cfg.hidden_size, E = cfg.num_experts, I = cfg.intermediate_size;
  L.E = E;
  L.H = H;
  L.I = I;
  L.ck = ck;
  if (layer < 0) return set_error(GPTOSS_ERR_INVALID, "layer_index=%d must be >= 0", layer);
  const std::string P = "model.layers." + std::to_string(layer) + ".";
  auto first = [&](std::initializer_list<const char*> names) -> const Tensor* {
    for (const char* n : names)
      if (const Tensor* t = ck->find(P + n)) return t;
    return nullptr;
  };

  // router, norm and biases (weight_loader.cu:1083-1117, 1146-1165)
  const Tensor* rw = first({"mlp.gate.weight", "mlp.router.weight"});
  if (!rw) return set_error(GPTOSS_ERR_NOT_FOUND, "no %smlp.gate.weight or %smlp.router.weight", P.c_str(), P.c_str());
  const Tensor* rb = first({"mlp.gate.bias", "mlp.router.bias"});
  const Tensor* nw = first({"post_attention_layernorm.weight"});
  const Tensor* b1 = first({"mlp.experts.gate_up_proj_bias"});
  const Tensor* b2 = first({"mlp.experts.down_proj_bias"});
  int rc;
  if ((rc = read_bf16(ck, rw, {E, H}, L.v_rw)) || (rb && (rc = read_bf16(ck, rb, {E}, L.v_rb))) ||
      (nw && (rc = read_bf16(ck, nw, {H}, L.v_nw))) || (b1 && (rc = read_bf16(ck, b1, {E, 2 * I}, L.v_b1))) ||
      (b2 && (rc = read_bf16(ck, b2, {E, H}, L.v_b2))))
    return rc;

  // experts: packed if the layer has gate_up_proj_blocks (weight_loader.cu:1119-1144)
  ExpertSource &s1 = L.s1, &s2 = L.s2;
  if (const Tensor* g = first({"mlp.experts.gate_up_proj_blocks"})) {
    const Tensor* d = first({"mlp.experts.down_proj_blocks"});
    if (!d) return set_error(GPTOSS_ERR_NOT_FOUND, "no %smlp.experts.down_proj_blocks", P.c_str());
    if ((rc = packed_source(ck, g, first({"mlp.experts.gate_up_proj_scales"}), E, 2 * I, H, s1)) ||
        (rc = packed_source(ck, d, first({"mlp.experts.down_proj_scales"}), E, H, I, s2)))
      return rc;
  } else {
    static const char* const n1[] = {"mlp1", "gate_up_proj", "w1"};
    static const char* const c1[] = {"mlp1", "gate_up_proj"};
    static const char* const n2[] = {"mlp2", "down_proj", "w2"};
    static const char* const c2[] = {"mlp2", "down_proj"};
    if ((rc = per_expert_source(ck, P, E, 2 * I, H, n1, 3, c1, 2, s1)) ||
        (rc = per_expert_source(ck, P, E, H, I, n2, 3, c2, 2, s2)))
      return rc;
  }
  return GPTOSS_OK;
}

}  // namespace

namespace gxmoe {

void ckpt_free_source(LayerSource* src) { delete src; }

int ckpt_resolve_layer(const gptoss_checkpoint* ck, const gptoss_moe_config& cfg, int layer, LayerSource** out) {
  *out = nullptr;
  LayerSource* L = new (std::nothrow) LayerSource();
  if (!L) return set_error(GPTOSS_ERR_OOM, "out of host memory");
  const int rc = resolve(ck, cfg, layer, *L);
  if (rc != GPTOSS_OK) {
    delete L;
    return rc;
  }
  *out = L;
  return GPTOSS_OK;
}

int ckpt_upload_layer(const LayerSource* src, void** blob, gptoss_moe_weights* wt) {
  *blob = nullptr;
  const int H = src->H, E = src->E, I = src->I;
  const std::vector<uint16_t>&v_rw = src->v_rw, &v_rb = src->v_rb, &v_nw = src->v_nw, &v_b1 = src->v_b1,
                 &v_b2 = src->v_b2;
  int rc = GPTOSS_OK;

  // one allocation: tiled experts, then the bf16 tensors
  const TiledGeom g1 = tiled_geom(2 * I, H), g2 = tiled_geom(H, I);
  size_t off = 0;
  auto take = [&](size_t bytes) {
    const size_t at = off;
    off = align_up(off + bytes, 256);
    return at;
  };
  const size_t o_w1n = take(g1.nib_bytes * E), o_w1s = take(g1.scale_bytes * E);
  const size_t o_w2n = take(g2.nib_bytes * E), o_w2s = take(g2.scale_bytes * E);
  const size_t o_rw = take(v_rw.size() * 2), o_rb = take(v_rb.size() * 2), o_nw = take(v_nw.size() * 2);
  const size_t o_b1 = take(v_b1.size() * 2), o_b2 = take(v_b2.size() * 2);
  struct DeviceBlob {  // freed unless handed to the caller (error returns, exceptions)
    uint8_t* p = nullptr;
    ~DeviceBlob() {
      if (p) (void)hipFree(p);
    }
  } blob_guard;
  hipError_t e = hipMalloc(reinterpret_cast<void**>(&blob_guard.p), off);
  if (e != hipSuccess)
    return set_error(GPTOSS_ERR_OOM, "hipMalloc(%zu) for the layer weights: %s", off, hipGetErrorString(e));
  uint8_t* const base = blob_guard.p;

  struct Small {
    size_t off;
    const std::vector<uint16_t>* v;
  } smalls[] = {{o_rw, &v_rw}, {o_rb, &v_rb}, {o_nw, &v_nw}, {o_b1, &v_b1}, {o_b2, &v_b2}};
  for (const Small& s : smalls)
    if (e == hipSuccess && !s.v->empty())
      e = hipMemcpy(base + s.off, s.v->data(), s.v->size() * 2, hipMemcpyHostToDevice);
  if (e != hipSuccess) return set_error(GPTOSS_ERR_HIP, "weight upload: %s", hipGetErrorString(e));

  {
    const size_t n1 = static_cast<size_t>(2 * I) * H, n2 = static_cast<size_t>(H) * I;
    const size_t per1 = align_up(n1 / 2, 256) + align_up(n1 / 32, 256);
    const size_t per2 = align_up(n2 / 2, 256) + align_up(n2 / 32, 256);
    const gptoss_checkpoint* ck = src->ck;
    const size_t want = std::max({ck->staging, per1, per2});
    // slots hold whole experts: no more than the larger matrix's experts need
    const size_t slot = align_up(std::min(want, std::max(per1, per2) * static_cast<size_t>(E)), 256);
    std::lock_guard<std::mutex> lock(ck->mu);
    int device = 0;
    e = hipGetDevice(&device);
    Staging* st = e == hipSuccess ? ck->staging_for(device, slot, &e) : nullptr;
    if (st == nullptr)
      return set_error(GPTOSS_ERR_OOM, "staging buffers (2 x %zu bytes): %s", slot, hipGetErrorString(e));
    st->pending[0] = st->pending[1] = false;  // the previous load ended with a stream sync
    struct StreamSync {  // the repack launches end before the blob can be freed on any way out
      hipStream_t s;
      ~StreamSync() { (void)hipStreamSynchronize(s); }
    } drain{st->stream};
    rc = upload_experts(*st, src->s1, E, 2 * I, H, base + o_w1n, base + o_w1s);
    if (rc == GPTOSS_OK) rc = upload_experts(*st, src->s2, E, H, I, base + o_w2n, base + o_w2s);
    e = hipStreamSynchronize(st->stream);
    if (rc == GPTOSS_OK && e != hipSuccess) rc = set_error(GPTOSS_ERR_HIP, "expert upload: %s", hipGetErrorString(e));
    if (rc != GPTOSS_OK) return rc;
  }

  *wt = gptoss_moe_weights{};
  wt->router_weight = reinterpret_cast<const uint16_t*>(base + o_rw);
  wt->router_bias = v_rb.empty() ? nullptr : reinterpret_cast<const uint16_t*>(base + o_rb);
  wt->moe_norm_weight = v_nw.empty() ? nullptr : reinterpret_cast<const uint16_t*>(base + o_nw);
  wt->gate_up_bias = v_b1.empty() ? nullptr : reinterpret_cast<const uint16_t*>(base + o_b1);
  wt->down_bias = v_b2.empty() ? nullptr : reinterpret_cast<const uint16_t*>(base + o_b2);
  wt->mlp1_tiled_nibbles = base + o_w1n;
  wt->mlp1_tiled_scales = base + o_w1s;
  wt->mlp2_tiled_nibbles = base + o_w2n;
  wt->mlp2_tiled_scales = base + o_w2s;
  *blob = blob_guard.p;
  blob_guard.p = nullptr;
  return GPTOSS_OK;
}

}  // namespace gxmoe
