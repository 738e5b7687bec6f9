// gguf.cpp -- GGUF parsing and the tensor byte path (see gguf.hpp).
#include "gguf.hpp"

#include <fcntl.h>
#include <stdarg.h>
#include <string.h>
#include <sys/mman.h>
#include <sys/stat.h>
#include <unistd.h>

#include <limits>

#include "../../include/hipq.h"

namespace light {
namespace gguf {

namespace {

constexpr int64_t kMaxInt = std::numeric_limits<int64_t>::max();
// Structural limits (gguf/reader.go:190-200).
constexpr uint32_t kMaxRank = 16;
constexpr int kMaxArrayDepth = 8;
constexpr int64_t kMaxAlign = int64_t(1) << 30;

std::string vfmt(const char *fmt, va_list ap) {
  char buf[512];
  vsnprintf(buf, sizeof buf, fmt, ap);
  return buf;
}
std::string fmt(const char *f, ...) __attribute__((format(printf, 1, 2)));
std::string fmt(const char *f, ...) {
  va_list ap;
  va_start(ap, f);
  std::string s = vfmt(f, ap);
  va_end(ap);
  return s;
}
// Go's %q for the names in messages.
std::string q(const std::string &s) { return "\"" + s + "\""; }

// Error wrapping as fmt.Errorf("...: %w", err).
[[noreturn]] void wrap(const std::string &prefix, const Error &e) { throw Error(prefix + ": " + e.what()); }

class Memory final : public Source {
 public:
  Memory(std::vector<uint8_t> b, bool sized) : b_(std::move(b)), sized_(sized) {}
  int64_t Size() const override { return sized_ ? (int64_t)b_.size() : -1; }
  void ReadAt(void *dst, size_t n, int64_t off) const override {
    if (off < 0 || (uint64_t)off > b_.size() || n > b_.size() - (size_t)off) {
      // io.ReaderAt: a short read reports io.EOF.
      const size_t avail = off >= 0 && (uint64_t)off < b_.size() ? b_.size() - (size_t)off : 0;
      if (avail) memcpy(dst, b_.data() + off, avail);
      throw Error("EOF");
    }
    if (n) memcpy(dst, b_.data() + off, n);
  }
  const uint8_t *Direct(int64_t off, size_t n) const override {
    if (off < 0 || (uint64_t)off > b_.size() || n > b_.size() - (size_t)off) return nullptr;
    return b_.data() + off;
  }

 private:
  std::vector<uint8_t> b_;
  bool sized_;
};

class Mapped final : public Source {
 public:
  explicit Mapped(const std::string &path) {
    fd_ = open(path.c_str(), O_RDONLY | O_CLOEXEC);
    if (fd_ < 0) throw Error(fmt("open %s: %s", path.c_str(), strerror(errno)));
    struct stat st;
    if (fstat(fd_, &st) != 0) {
      close(fd_);
      throw Error(fmt("stat %s: %s", path.c_str(), strerror(errno)));
    }
    size_ = st.st_size;
    if (size_ > 0) {
      map_ = mmap(nullptr, (size_t)size_, PROT_READ, MAP_PRIVATE, fd_, 0);
      if (map_ == MAP_FAILED) {
        close(fd_);
        throw Error(fmt("mmap %s: %s", path.c_str(), strerror(errno)));
      }
    }
  }
  ~Mapped() override {
    if (map_ && map_ != MAP_FAILED) munmap(map_, (size_t)size_);
    if (fd_ >= 0) close(fd_);
  }
  int64_t Size() const override { return size_; }
  void ReadAt(void *dst, size_t n, int64_t off) const override {
    const uint8_t *p = Direct(off, n);
    if (!p) throw Error("EOF");
    if (n) memcpy(dst, p, n);
  }
  const uint8_t *Direct(int64_t off, size_t n) const override {
    if (off < 0 || off > size_ || (int64_t)n > size_ - off) return nullptr;
    return static_cast<const uint8_t *>(map_) + off;
  }

 private:
  int fd_ = -1;
  void *map_ = nullptr;
  int64_t size_ = 0;
};

// Sequential little-endian reader over a Source (the cursor of gguf/reader.go:320-417).
struct Cursor {
  const Source &src;
  int64_t pos = 0;
  int64_t size;

  explicit Cursor(const Source &s) : src(s), size(s.Size()) {}

  // Rejects a count of items, each at least min_bytes long, that cannot fit in the rest of
  // a sized input.
  void fits(uint64_t n, uint64_t min_bytes, const char *what) const {
    if (size < 0) return;
    const uint64_t rest = (uint64_t)std::max<int64_t>(size - pos, 0);
    if (n > rest / min_bytes)
      throw Error(fmt("gguf: %s %llu cannot fit in the %llu remaining bytes", what, (unsigned long long)n,
                      (unsigned long long)rest));
  }
  // A long read from an unsized input goes in chunks, so a lying length fails on the short
  // read rather than on one huge allocation.
  std::string read(uint64_t n) {
    constexpr uint64_t chunk = 1 << 20;
    std::string buf;
    while (buf.size() < n) {
      const uint64_t k = std::min<uint64_t>(chunk, n - buf.size());
      const size_t at = buf.size();
      buf.resize(at + k);
      src.ReadAt(&buf[at], k, pos + (int64_t)at);
    }
    pos += (int64_t)n;
    return buf;
  }
  template <class T>
  T le() {
    T v;
    src.ReadAt(&v, sizeof v, pos);
    pos += sizeof v;
    return v;
  }
  uint8_t u8() { return le<uint8_t>(); }
  uint16_t u16() { return le<uint16_t>(); }
  uint32_t u32() { return le<uint32_t>(); }
  uint64_t u64() { return le<uint64_t>(); }

  std::string str() {
    const uint64_t n = u64();
    if (n > (uint64_t(1) << 30)) throw Error(fmt("gguf: string length %llu too large", (unsigned long long)n));
    fits(n, 1, "string length");
    return read(n);
  }

  // The smallest encoding of a value of type t (gguf/reader.go:419-433).
  static uint64_t min_value_bytes(uint32_t t) {
    switch (t) {
      case TypeUInt16: case TypeInt16: return 2;
      case TypeUInt32: case TypeInt32: case TypeFloat32: return 4;
      case TypeUInt64: case TypeInt64: case TypeFloat64: case TypeString: return 8;
      case TypeArray: return 4 + 8;
    }
    return 1;
  }

  Value value(uint32_t t, int depth) {
    Value v;
    v.type = t;
    switch (t) {
      case TypeUInt8: v.u = u8(); return v;
      case TypeInt8: v.i = (int8_t)u8(); return v;
      case TypeUInt16: v.u = u16(); return v;
      case TypeInt16: v.i = (int16_t)u16(); return v;
      case TypeUInt32: v.u = u32(); return v;
      case TypeInt32: v.i = (int32_t)u32(); return v;
      case TypeUInt64: v.u = u64(); return v;
      case TypeInt64: v.i = (int64_t)u64(); return v;
      case TypeFloat32: {
        const uint32_t b = u32();
        float f;
        memcpy(&f, &b, 4);
        v.f = f;
        return v;
      }
      case TypeFloat64: {
        const uint64_t b = u64();
        memcpy(&v.f, &b, 8);
        return v;
      }
      case TypeBool: v.b = u8() != 0; return v;
      case TypeString: v.s = str(); return v;
      case TypeArray: {
        if (depth >= kMaxArrayDepth) throw Error(fmt("gguf: arrays nested deeper than %d", kMaxArrayDepth));
        const uint32_t et = u32();
        const uint64_t n = u64();
        fits(n, min_value_bytes(et), "array length");
        // Every element consumes input, so a lying count on an unsized input still ends at
        // EOF; the vector is not pre-sized by it.
        for (uint64_t k = 0; k < n; k++) v.arr.push_back(value(et, depth + 1));
        return v;
      }
    }
    throw Error(fmt("gguf: unknown value type %u", t));
  }
};

// toInt64 (gguf/reader.go:290-318): any integer type, unsigned values that fit.
bool to_int64(const Value &v, int64_t *out) {
  switch (v.type) {
    case TypeUInt8: case TypeUInt16: case TypeUInt32: *out = (int64_t)v.u; return true;
    case TypeInt8: case TypeInt16: case TypeInt32: case TypeInt64: *out = v.i; return true;
    case TypeUInt64:
      if (v.u > (uint64_t)kMaxInt) return false;
      *out = (int64_t)v.u;
      return true;
  }
  return false;
}

std::string dims_str(const std::vector<int64_t> &d, size_t n) {
  std::string s = "[";
  for (size_t i = 0; i < n && i < d.size(); i++) s += (i ? " " : "") + std::to_string(d[i]);
  return s + "]";
}

}  // namespace

std::shared_ptr<Source> MemorySource(std::vector<uint8_t> bytes, bool sized) {
  return std::make_shared<Memory>(std::move(bytes), sized);
}
std::shared_ptr<Source> FileSource(const std::string &path) { return std::make_shared<Mapped>(path); }

DType DTypeFromGGML(uint32_t t) {
  switch (t) {
    case 0: return DType::F32;
    case 1: return DType::F16;
    case 30: return DType::BF16;
    case 28: return DType::F64;
    case 24: return DType::I8;
    case 25: return DType::I16;
    case 26: return DType::I32;
    case 27: return DType::I64;
    case 2: return DType::Q4_0;
    case 3: return DType::Q4_1;
    case 6: return DType::Q5_0;
    case 7: return DType::Q5_1;
    case 8: return DType::Q8_0;
    case 9: return DType::Q8_1;
    case 10: return DType::Q2_K;
    case 11: return DType::Q3_K;
    case 12: return DType::Q4_K;
    case 13: return DType::Q5_K;
    case 14: return DType::Q6_K;
    case 15: return DType::Q8_K;
  }
  throw Error(fmt("gguf: unsupported ggml type %u", t));
}

std::shared_ptr<File> File::Open(std::shared_ptr<Source> src) {
  Cursor r(*src);
  uint32_t m;
  try {
    m = r.u32();
  } catch (const Error &e) {
    wrap("gguf: read magic", e);
  }
  if (m != kMagic) throw Error(fmt("gguf: bad magic %#x (want %#x)", m, kMagic));
  uint32_t ver;
  try {
    ver = r.u32();
  } catch (const Error &e) {
    wrap("gguf: read version", e);
  }
  if (ver < kMinVersion || ver > kMaxVersion)
    throw Error(fmt("gguf: version %u not in [%u, %u]", ver, kMinVersion, kMaxVersion));
  const uint64_t n_tensors = r.u64();
  const uint64_t n_kv = r.u64();
  // Each KV needs at least a key length, a type tag and one value byte; each tensor-info
  // entry a name length, rank, type and offset.
  r.fits(n_kv, 8 + 4 + 1, "metadata count");
  r.fits(n_tensors, 8 + 4 + 4 + 8, "tensor count");

  auto f = std::make_shared<File>();
  f->version = ver;
  f->src_ = src;
  for (uint64_t i = 0; i < n_kv; i++) {
    std::string key;
    try {
      key = r.str();
    } catch (const Error &e) {
      wrap(fmt("gguf: kv[%llu] key", (unsigned long long)i), e);
    }
    uint32_t vt;
    try {
      vt = r.u32();
    } catch (const Error &e) {
      wrap("gguf: kv[" + q(key) + "] type", e);
    }
    Value v;
    try {
      v = r.value(vt, 0);
    } catch (const Error &e) {
      wrap("gguf: kv[" + q(key) + "] value", e);
    }
    f->meta[key] = std::move(v);
    f->key_order.push_back(key);
  }

  for (uint64_t i = 0; i < n_tensors; i++) {
    TensorInfo ti;
    try {
      ti.name = r.str();
    } catch (const Error &e) {
      wrap(fmt("gguf: tensor[%llu] name", (unsigned long long)i), e);
    }
    const std::string nq = q(ti.name);
    const uint32_t nd = r.u32();
    if (nd > kMaxRank) throw Error(fmt("gguf: tensor[%s] rank %u exceeds %u", nq.c_str(), nd, kMaxRank));
    int64_t n_elems = 1;
    for (uint32_t j = 0; j < nd; j++) {
      const uint64_t d = r.u64();
      if (d > (uint64_t)kMaxInt)
        throw Error(fmt("gguf: tensor[%s] dim %llu too large", nq.c_str(), (unsigned long long)d));
      ti.dims.push_back((int64_t)d);
      if (d != 0 && n_elems > kMaxInt / (int64_t)d)
        throw Error(fmt("gguf: tensor[%s] dims %s element count overflows", nq.c_str(), dims_str(ti.dims, j + 1).c_str()));
      n_elems *= (int64_t)d;
    }
    const uint32_t ggml = r.u32();
    try {
      ti.dtype = DTypeFromGGML(ggml);
    } catch (const Error &e) {
      wrap("gguf: tensor[" + nq + "]", e);
    }
    const uint64_t off = r.u64();
    const int64_t be = BlockElems(ti.dtype), bb = BlockBytes(ti.dtype);
    const int64_t blocks = n_elems == 0 ? 0 : (n_elems - 1) / be + 1;
    if (blocks > kMaxInt / bb)
      throw Error(fmt("gguf: tensor[%s] %s %s byte size overflows", nq.c_str(), DTypeName(ti.dtype),
                      dims_str(ti.dims, ti.dims.size()).c_str()));
    if (off > (uint64_t)kMaxInt)
      throw Error(fmt("gguf: tensor[%s] offset %llu too large", nq.c_str(), (unsigned long long)off));
    ti.offset = off;
    ti.bytes = blocks * bb;
    f->order.push_back(ti.name);
    f->tensors[ti.name] = std::move(ti);
  }

  // Tensor data begins after the info table, padded up to general.alignment.
  int64_t align = 32;
  auto it = f->meta.find("general.alignment");
  if (it != f->meta.end()) {
    int64_t n;
    if (to_int64(it->second, &n) && n > 0) align = n;
  }
  if (align > kMaxAlign)
    throw Error(fmt("gguf: general.alignment %lld exceeds %lld", (long long)align, (long long)kMaxAlign));
  f->data_base = (r.pos + align - 1) / align * align;
  // Every tensor's [offset, offset + bytes) must fit after the data base without wrapping,
  // and inside the input when its size is known.
  for (const auto &name : f->order) {
    const TensorInfo &ti = f->tensors[name];
    const int64_t off = (int64_t)ti.offset;
    if (off > kMaxInt - f->data_base || ti.bytes > kMaxInt - f->data_base - off)
      throw Error(fmt("gguf: tensor[%s] offset %llu + %lld bytes overflows", q(name).c_str(),
                      (unsigned long long)ti.offset, (long long)ti.bytes));
    const int64_t end = f->data_base + off + ti.bytes;
    if (r.size >= 0 && end > r.size)
      throw Error(fmt("gguf: tensor[%s] data [%lld, %lld) past end of %lld-byte input", q(name).c_str(),
                      (long long)(f->data_base + off), (long long)end, (long long)r.size));
  }
  return f;
}

const TensorInfo &File::Info(const std::string &name) const {
  auto it = tensors.find(name);
  if (it == tensors.end()) throw Error("gguf: tensor " + q(name) + " not found");
  return it->second;
}

// Before anything is allocated for a tensor's data: its byte range must be addressable and
// its last byte readable.  A sized input was checked at Open; on an unsized one (a stream)
// a header that lies about the size then fails as the short read Light's TensorBytes would
// meet (gguf/reader.go:254-264), not as an allocation of the claimed size first.
void File::ProbeData(const TensorInfo &ti, const std::string &name) const {
  if (ti.bytes <= 0) return;
  const uint64_t room = (uint64_t)INT64_MAX - (uint64_t)data_base;
  if (ti.offset > room || (uint64_t)ti.bytes > room - ti.offset)
    throw Error("gguf: read tensor " + q(name) + ": offset out of range");
  uint8_t last;
  try {
    src_->ReadAt(&last, 1, data_base + (int64_t)(ti.offset + (uint64_t)ti.bytes - 1));
  } catch (const Error &e) {
    wrap("gguf: read tensor " + q(name), e);
  }
}

std::vector<uint8_t> File::TensorBytes(const std::string &name) const {
  const TensorInfo &ti = Info(name);
  ProbeData(ti, name);
  std::vector<uint8_t> buf((size_t)ti.bytes);
  try {
    src_->ReadAt(buf.data(), buf.size(), data_base + (int64_t)ti.offset);
  } catch (const Error &e) {
    wrap("gguf: read tensor " + q(name), e);
  }
  return buf;
}

const uint8_t *File::Payload(const std::string &name, std::vector<uint8_t> *tmp) const {
  const TensorInfo &ti = Info(name);
  const uint8_t *p = src_->Direct(data_base + (int64_t)ti.offset, (size_t)ti.bytes);
  if (p) return p;
  *tmp = TensorBytes(name);
  return tmp->data();
}

void File::CopyTensorTo(const std::string &name, void *dst, Device dev) const {
  const TensorInfo &ti = Info(name);
  if (!ti.bytes) return;
  std::vector<uint8_t> tmp;
  const uint8_t *p = Payload(name, &tmp);
  if (dev.kind == DeviceKind::CPU)
    memcpy(dst, p, (size_t)ti.bytes);
  else
    Check(hq_memcpy_h2d(dst, p, (size_t)ti.bytes, nullptr));
}

Tensor File::LoadTensor(const std::string &name, Device dev) const {
  const TensorInfo &ti = Info(name);
  ProbeData(ti, name);
  Tensor t = Tensor::Empty(ti.dtype, ti.dims, dev);
  CopyTensorTo(name, t.data(), dev);
  return t;
}

Tensor File::TensorRowMajor(const std::string &name, Device dev) const {
  const TensorInfo &ti = Info(name);
  ProbeData(ti, name);
  std::vector<int64_t> dims(ti.dims.rbegin(), ti.dims.rend());
  Tensor t = Tensor::Empty(ti.dtype, dims, dev);
  CopyTensorTo(name, t.data(), dev);
  return t;
}

bool File::String(const std::string &key, std::string *out) const {
  auto it = meta.find(key);
  if (it == meta.end() || it->second.type != TypeString) return false;
  *out = it->second.s;
  return true;
}

bool File::Int64(const std::string &key, int64_t *out) const {
  auto it = meta.find(key);
  return it != meta.end() && to_int64(it->second, out);
}

bool File::Float64(const std::string &key, double *out) const {
  auto it = meta.find(key);
  if (it == meta.end() || (it->second.type != TypeFloat32 && it->second.type != TypeFloat64)) return false;
  *out = it->second.f;
  return true;
}

namespace {
// Light's Half.ToF32 / BF16 widening (dtype/half.go:84-113): exact.
float half_to_f32(uint16_t h) {
  const uint32_t sign = (uint32_t)(h >> 15) << 31, exp = (h >> 10) & 31, man = h & 0x3ff;
  uint32_t bits;
  if (exp == 0) {
    if (!man) {
      bits = sign;
    } else {  // subnormal: normalise
      int e = -1;
      uint32_t m = man;
      do {
        e++;
        m <<= 1;
      } while (!(m & 0x400));
      bits = sign | (uint32_t)(127 - 15 - e) << 23 | (m & 0x3ff) << 13;
    }
  } else if (exp == 31) {
    bits = sign | 0x7f800000u | man << 13;
  } else {
    bits = sign | (exp + 127 - 15) << 23 | man << 13;
  }
  float f;
  memcpy(&f, &bits, 4);
  return f;
}

// The stack bytes of one expert as the target dtype: quantized and F32 stacks as stored,
// F16 / BF16 widened to F32 (ops.Cast in models/llama_gguf.go:202-206).
void put_slab(const uint8_t *src, DType dt, int64_t elems, uint8_t *dst, Device dev) {
  std::vector<float> wide;
  const void *p = src;
  size_t n = (size_t)ByteSize(dt, elems);
  if (dt == DType::F16 || dt == DType::BF16) {
    wide.resize((size_t)elems);
    for (int64_t i = 0; i < elems; i++) {
      uint16_t h;
      memcpy(&h, src + 2 * i, 2);
      if (dt == DType::F16) {
        wide[i] = half_to_f32(h);
      } else {
        const uint32_t bits = (uint32_t)h << 16;
        memcpy(&wide[i], &bits, 4);
      }
    }
    p = wide.data();
    n = wide.size() * 4;
  }
  if (dev.kind == DeviceKind::CPU)
    memcpy(dst, p, n);
  else
    Check(hq_memcpy_h2d(dst, p, n, nullptr));
}
}  // namespace

ExpertStacks LoadExperts(const File &f, const std::string &p, Device dev) {
  auto gi = f.tensors.find(p + "ffn_gate_exps.weight");
  if (gi == f.tensors.end()) throw Error(p + "ffn_gate_exps.weight missing");
  auto ui = f.tensors.find(p + "ffn_up_exps.weight");
  if (ui == f.tensors.end() || ui->second.dtype != gi->second.dtype || gi->second.dims.size() != 3)
    throw Error(p + "ffn_up_exps.weight missing or mismatched");
  const DType dt = gi->second.dtype;
  const int64_t H = gi->second.dims[0], I = gi->second.dims[1], E = gi->second.dims[2];
  if (ui->second.dims != gi->second.dims) throw Error(p + "ffn_up_exps.weight missing or mismatched");
  const bool widen = dt == DType::F16 || dt == DType::BF16;
  const DType odt = widen ? DType::F32 : dt;
  const int64_t slab = ByteSize(dt, I * H), oslab = ByteSize(odt, I * H);  // one expert's (I, H) block
  ExpertStacks out;
  // Expert e: its I gate rows, then its I up rows (models/llama_gguf.go:186-191), copied
  // from the file's payloads straight into place (payloads read, or probed, before the
  // stacks are allocated).
  std::vector<uint8_t> gt, ut;
  const uint8_t *gb = f.Payload(gi->first, &gt), *ub = f.Payload(ui->first, &ut);
  out.gate_up = Tensor::Empty(odt, {E, 2 * I, H}, dev);
  for (int64_t e = 0; e < E; e++) {
    uint8_t *dst = static_cast<uint8_t *>(out.gate_up.data()) + 2 * e * oslab;
    put_slab(gb + e * slab, dt, I * H, dst, dev);
    put_slab(ub + e * slab, dt, I * H, dst + oslab, dev);
  }
  const TensorInfo &di = f.Info(p + "ffn_down_exps.weight");
  if (di.dtype == DType::F16 || di.dtype == DType::BF16) {
    std::vector<int64_t> dims(di.dims.rbegin(), di.dims.rend());
    std::vector<uint8_t> dt_;
    const uint8_t *db = f.Payload(di.name, &dt_);
    out.down = Tensor::Empty(DType::F32, dims, dev);
    int64_t n = 1;
    for (int64_t d : dims) n *= d;
    put_slab(db, di.dtype, n, static_cast<uint8_t *>(out.down.data()), dev);
  } else {
    out.down = f.TensorRowMajor(p + "ffn_down_exps.weight", dev);
  }
  return out;
}

}  // namespace gguf
}  // namespace light
