// kiln_host.cpp — implementation of the C++ host layer (kiln_host.hpp).
#include "kiln_host.hpp"

#include <algorithm>
#include <cmath>
#include <cstdio>
#include <cstring>
#include <fstream>
#include <mutex>
#include <set>
#include <sstream>

#include <fcntl.h>
#include <sys/mman.h>
#include <sys/stat.h>
#include <unistd.h>

namespace kiln {

size_t dtype_size(Dtype d) {
  switch (d) {
    case Dtype::Bool:
    case Dtype::Uint8: return 1;
    case Dtype::Uint16:
    case Dtype::Float16:
    case Dtype::Bfloat16: return 2;
    default: return 4;
  }
}

const char* dtype_name(Dtype d) {
  switch (d) {
    case Dtype::Bool: return "bool";
    case Dtype::Uint8: return "uint8";
    case Dtype::Uint16: return "uint16";
    case Dtype::Uint32: return "uint32";
    case Dtype::Int32: return "int32";
    case Dtype::Float16: return "float16";
    case Dtype::Float32: return "float32";
    case Dtype::Bfloat16: return "bfloat16";
  }
  return "?";
}

namespace {

Error hip_error(const char* what, hipError_t e) {
  return Error{std::string(what) + ": " + hipGetErrorString(e)};
}

Error kh_error(int status) {
  const char* m = kh_last_error();
  return Error{m && *m ? std::string(m) : "kiln_hip call failed with status " + std::to_string(status)};
}

// ---------------------------------------------------------------------------
// Caching allocator: size classes of powers of two (>= 256 B), free blocks
// kept per (device, stream). A block freed on stream S is only handed out
// again on S, where stream order makes the reuse safe without a sync.
class Allocator {
 public:
  static Allocator& get() {
    static Allocator a;
    return a;
  }

  Result<void*> alloc(size_t bytes, hipStream_t s, size_t* cap) {
    const size_t c = round_up(bytes);
    int dev = 0;
    (void)hipGetDevice(&dev);
    {
      std::lock_guard<std::mutex> lock(mu_);
      auto& fl = free_[Key{dev, s, c}];
      if (!fl.empty()) {
        void* p = fl.back();
        fl.pop_back();
        stats_.cached -= c;
        stats_.in_use += c;
        *cap = c;
        return p;
      }
    }
    void* p = nullptr;
    hipError_t e = hipMalloc(&p, c);
    if (e != hipSuccess) {
      allocator_trim();  // give cached blocks back and retry once
      e = hipMalloc(&p, c);
      if (e != hipSuccess) return hip_error("hipMalloc", e);
    }
    std::lock_guard<std::mutex> lock(mu_);
    stats_.in_use += c;
    stats_.device_allocs += 1;
    *cap = c;
    return p;
  }

  void release(void* p, size_t cap, hipStream_t s) {
    int dev = 0;
    (void)hipGetDevice(&dev);
    std::lock_guard<std::mutex> lock(mu_);
    free_[Key{dev, s, cap}].push_back(p);
    stats_.in_use -= cap;
    stats_.cached += cap;
  }

  void trim() {
    std::lock_guard<std::mutex> lock(mu_);
    (void)hipDeviceSynchronize();
    for (auto& kv : free_) {
      for (void* p : kv.second) (void)hipFree(p);
      stats_.cached -= kv.first.cap * kv.second.size();
      kv.second.clear();
    }
  }

  AllocatorStats stats() {
    std::lock_guard<std::mutex> lock(mu_);
    return stats_;
  }

 private:
  struct Key {
    int dev;
    hipStream_t s;
    size_t cap;
    bool operator<(const Key& o) const {
      if (dev != o.dev) return dev < o.dev;
      if (s != o.s) return s < o.s;
      return cap < o.cap;
    }
  };
  static size_t round_up(size_t b) {
    size_t c = 256;
    while (c < b) c <<= 1;
    return c;
  }
  std::mutex mu_;
  std::map<Key, std::vector<void*>> free_;
  AllocatorStats stats_;
};

}  // namespace

AllocatorStats allocator_stats() { return Allocator::get().stats(); }
void allocator_trim() { Allocator::get().trim(); }

// ---------------------------------------------------------------------------
// Stream

Stream Stream::gpu() { return Stream(nullptr, false); }

Result<Stream> Stream::create() {
  hipStream_t s = nullptr;
  hipError_t e = hipStreamCreateWithFlags(&s, hipStreamNonBlocking);
  if (e != hipSuccess) return hip_error("hipStreamCreate", e);
  return Stream(s, true);
}

Stream::~Stream() {
  if (owned_ && s_) (void)hipStreamDestroy(s_);
}

Result<void> Stream::synchronize() const {
  hipError_t e = hipStreamSynchronize(s_);
  if (e != hipSuccess) return hip_error("hipStreamSynchronize", e);
  return {};
}

// ---------------------------------------------------------------------------
// Array

Array& Array::operator=(Array&& o) noexcept {
  if (this != &o) {
    if (owner_ && data_) Allocator::get().release(data_, cap_, stream_);
    data_ = o.data_;
    cap_ = o.cap_;
    shape_ = std::move(o.shape_);
    dtype_ = o.dtype_;
    stream_ = o.stream_;
    owner_ = o.owner_;
    o.data_ = nullptr;
    o.owner_ = false;
    o.cap_ = 0;
  }
  return *this;
}

Array::~Array() {
  if (owner_ && data_) Allocator::get().release(data_, cap_, stream_);
}

int64_t Array::size() const {
  int64_t n = 1;
  for (int64_t d : shape_) n *= d;
  return n;
}

Result<Array> Array::empty(const std::vector<int64_t>& shape, Dtype dtype, const Stream& s) {
  if ((int)shape.size() > KH_MAX_NDIM) return Error{"array rank exceeds " + std::to_string(KH_MAX_NDIM)};
  Array a;
  a.shape_ = shape;
  a.dtype_ = dtype;
  a.stream_ = s.raw();
  // element count with overflow checks: no shape may ask for more than 2^48 bytes
  uint64_t n = 1;
  for (int64_t d : shape) {
    if (d < 0) return Error{"array shape has a negative dimension"};
    if (d != 0 && n > (uint64_t(1) << 48) / (uint64_t)d) return Error{"array shape is too large"};
    n *= (uint64_t)d;
  }
  if (n > (uint64_t(1) << 48) / (uint64_t)std::max<size_t>(dtype_size(dtype), 1))
    return Error{"array shape is too large"};
  const size_t bytes = a.nbytes();
  if (bytes > 0) {
    auto p = Allocator::get().alloc(bytes, s.raw(), &a.cap_);
    if (!p) return p.error();
    a.data_ = p.value();
    a.owner_ = true;
  }
  return a;
}

Result<Array> Array::from_bytes(const void* bytes, size_t nbytes, const std::vector<int64_t>& shape,
                                Dtype dtype, const Stream& s) {
  auto r = Array::empty(shape, dtype, s);
  if (!r) return r;
  Array a = r.take();
  if (a.nbytes() != nbytes)
    return Error{"byte buffer of " + std::to_string(nbytes) + " does not hold " + std::to_string(a.size()) +
                 " " + dtype_name(dtype) + " elements"};
  if (nbytes) {
    hipError_t e = hipMemcpyAsync(a.data_, bytes, nbytes, hipMemcpyHostToDevice, s.raw());
    if (e == hipSuccess) e = hipStreamSynchronize(s.raw());  // `bytes` may not outlive the call
    if (e != hipSuccess) return hip_error("hipMemcpy", e);
  }
  return a;
}

Array Array::share() const {
  Array a;
  a.data_ = data_;
  a.cap_ = cap_;
  a.shape_ = shape_;
  a.dtype_ = dtype_;
  a.stream_ = stream_;
  a.owner_ = false;
  return a;
}

Result<Array> Array::view(const std::vector<int64_t>& shape) const {
  int64_t n = 1;
  for (int64_t d : shape) n *= d;
  if (n != size()) return Error{"[view] shape does not hold the same number of elements"};
  Array a = share();
  a.shape_ = shape;
  return a;
}

Result<std::vector<uint8_t>> Array::to_bytes(const Stream& s) const {
  std::vector<uint8_t> out(nbytes());
  if (!out.empty()) {
    hipError_t e = hipMemcpyAsync(out.data(), data_, out.size(), hipMemcpyDeviceToHost, s.raw());
    if (e == hipSuccess) e = hipStreamSynchronize(s.raw());
    if (e != hipSuccess) return hip_error("hipMemcpy", e);
  }
  return out;
}

kh_array Array::desc() const {
  kh_array d{};
  d.data = data_;
  d.dtype = (int32_t)dtype_;
  d.ndim = ndim();
  for (int i = 0; i < ndim(); ++i) d.shape[i] = shape_[i];
  return d;
}

// ---------------------------------------------------------------------------
// ops

namespace ops {

namespace {
kh_optional_int opt(int v) { return kh_optional_int{v, true}; }

// MLX promotion over (x, scales, biases) for the float types used here.
Dtype promote(Dtype a, Dtype b) { return a == b ? a : Dtype::Float32; }
}  // namespace

Result<Array> quantized_matmul(const Array& x, const Array& w, const Array& scales,
                               const Array& biases, bool transpose, int group_size, int bits,
                               const Stream& s) {
  if (x.ndim() < 1 || w.ndim() != 2) return Error{"[quantized_matmul] x must be [..., K] and w 2-D"};
  const int64_t per = (bits == 4 || bits == 8) ? 32 / bits : 1;
  const int64_t N = transpose ? w.dim(0) : w.dim(1) * per;
  std::vector<int64_t> shape = x.shape();
  shape.back() = N;
  auto r = Array::empty(shape, promote(x.dtype(), scales.dtype()), s);
  if (!r) return r;
  Array out = r.take();
  kh_array res = out.desc(), xd = x.desc(), wd = w.desc(), sd = scales.desc(), bd = biases.desc();
  const int st = kh_quantized_matmul(&res, &xd, &wd, &sd, &bd, transpose, opt(group_size), opt(bits),
                                     "affine", s.raw());
  if (st) return kh_error(st);
  return out;
}

Result<Array> gather_qmm(const Array& x, const Array& w, const Array& scales, const Array& biases,
                         const Array& indices, bool transpose, int group_size, int bits,
                         bool sorted_indices, const Stream& s) {
  if (x.ndim() < 2 || w.ndim() != 3)
    return Error{"[gather_qmm] x must be [..., M, K] and w an expert stack [E, N, K*bits/32]"};
  if (!transpose) return Error{"[gather_qmm] transpose=false is not supported (Kiln passes true)"};
  // batch = broadcast(x.shape[:-2], indices.shape), numpy rules
  const int xb = x.ndim() - 2, ib = indices.ndim(), nd = std::max(xb, ib);
  std::vector<int64_t> shape(nd);
  for (int d = 0; d < nd; ++d) {
    const int dx = d - (nd - xb), di = d - (nd - ib);
    const int64_t sx = dx >= 0 ? x.dim(dx) : 1, si = di >= 0 ? indices.dim(di) : 1;
    if (sx != si && sx != 1 && si != 1) return Error{"[gather_qmm] x and indices do not broadcast"};
    shape[d] = sx == 1 ? si : sx;
  }
  shape.push_back(x.dim(-2));
  shape.push_back(w.dim(1));
  auto r = Array::empty(shape, promote(x.dtype(), scales.dtype()), s);
  if (!r) return r;
  Array out = r.take();
  kh_array res = out.desc(), xd = x.desc(), wd = w.desc(), sd = scales.desc(), bd = biases.desc(),
           id = indices.desc();
  const int st = kh_gather_qmm(&res, &xd, &wd, &sd, &bd, &id, transpose, opt(group_size), opt(bits), "affine",
                               sorted_indices, s.raw());
  if (st) return kh_error(st);
  return out;
}

Result<Array> stack(const std::vector<Array>& parts, const Stream& s) {
  if (parts.empty()) return Error{"[stack] no arrays to stack"};
  for (const Array& p : parts)
    if (p.shape() != parts[0].shape() || p.dtype() != parts[0].dtype())
      return Error{"[stack] arrays differ in shape or dtype"};
  std::vector<int64_t> shape = parts[0].shape();
  shape.insert(shape.begin(), (int64_t)parts.size());
  auto r = Array::empty(shape, parts[0].dtype(), s);
  if (!r) return r;
  Array out = r.take();
  const size_t each = parts[0].nbytes();
  for (size_t i = 0; i < parts.size(); ++i) {
    if (each == 0) break;
    const hipError_t e = hipMemcpyAsync(static_cast<char*>(out.data()) + i * each, parts[i].data(), each,
                                        hipMemcpyDeviceToDevice, s.raw());
    if (e != hipSuccess) return Error{std::string("[stack] ") + hipGetErrorString(e)};
  }
  return out;
}

Result<Array> dequantize(const Array& w, const Array& scales, const Array& biases, int group_size,
                         int bits, const Stream& s) {
  if (w.ndim() < 1) return Error{"[dequantize] w must have ndim >= 1"};
  const int64_t per = (bits == 4 || bits == 8) ? 32 / bits : 1;
  std::vector<int64_t> shape = w.shape();
  shape.back() *= per;
  auto r = Array::empty(shape, scales.dtype(), s);
  if (!r) return r;
  Array out = r.take();
  kh_array res = out.desc(), wd = w.desc(), sd = scales.desc(), bd = biases.desc();
  const int st = kh_dequantize(&res, &wd, &sd, &bd, opt(group_size), opt(bits), "affine", s.raw());
  if (st) return kh_error(st);
  return out;
}

Result<Array> take(const Array& a, const Array& indices, int axis, const Stream& s) {
  if (axis != 0) return Error{"[take] only axis 0 is supported"};
  if (a.ndim() < 1) return Error{"[take] cannot take along axis 0 of a scalar"};
  std::vector<int64_t> shape = indices.shape();
  for (int i = 1; i < a.ndim(); ++i) shape.push_back(a.dim(i));
  auto r = Array::empty(shape, a.dtype(), s);
  if (!r) return r;
  Array out = r.take();
  kh_array res = out.desc(), ad = a.desc(), id = indices.desc();
  const int st = kh_take(&res, &ad, &id, s.raw());
  if (st) return kh_error(st);
  return out;
}

Result<Array> quantized_embedding(const Array& ids, const Array& w, const Array& scales,
                                  const Array& biases, int group_size, int bits, const Stream& s) {
  if (w.ndim() != 2) return Error{"[quantized_embedding] table must be 2-D"};
  const int64_t per = (bits == 4 || bits == 8) ? 32 / bits : 1;
  std::vector<int64_t> shape = ids.shape();
  shape.push_back(w.dim(1) * per);
  auto r = Array::empty(shape, scales.dtype(), s);
  if (!r) return r;
  Array out = r.take();
  kh_array res = out.desc(), idd = ids.desc(), wd = w.desc(), sd = scales.desc(), bd = biases.desc();
  const int st = kh_quantized_embedding(&res, &idd, &wd, &sd, &bd, opt(group_size), opt(bits), "affine",
                                        s.raw());
  if (st) return kh_error(st);
  return out;
}

Result<Array> add(const Array& a, const Array& b, const Stream& s) {
  const int nd = std::max(a.ndim(), b.ndim());
  std::vector<int64_t> shape(nd);
  for (int d = 0; d < nd; ++d) {  // numpy broadcasting; the library checks compatibility
    const int da = d - (nd - a.ndim()), db = d - (nd - b.ndim());
    const int64_t ea = da >= 0 ? a.dim(da) : 1, eb = db >= 0 ? b.dim(db) : 1;
    shape[d] = ea == 1 ? eb : ea;
  }
  auto r = Array::empty(shape, promote(a.dtype(), b.dtype()), s);
  if (!r) return r;
  Array out = r.take();
  kh_array res = out.desc(), ad = a.desc(), bd = b.desc();
  const int st = kh_add(&res, &ad, &bd, s.raw());
  if (st) return kh_error(st);
  return out;
}

Result<Array> linear(const Array& x, const Array& w, const Array& scales, const Array& biases,
                     const std::optional<Array>& bias, int group_size, int bits, const Stream& s) {
  if (x.ndim() < 1 || w.ndim() != 2) return Error{"[linear] x must be [..., K] and w 2-D"};
  std::vector<int64_t> shape = x.shape();
  shape.back() = w.dim(0);
  Dtype dt = promote(x.dtype(), scales.dtype());
  if (bias) dt = promote(dt, bias->dtype());
  auto r = Array::empty(shape, dt, s);
  if (!r) return r;
  Array out = r.take();
  kh_array res = out.desc(), xd = x.desc(), wd = w.desc(), sd = scales.desc(), bd = biases.desc();
  kh_array bsd{};
  if (bias) bsd = bias->desc();
  const int st = kh_linear(&res, &xd, &wd, &sd, &bd, bias ? &bsd : nullptr, opt(group_size), opt(bits),
                           "affine", s.raw());
  if (st) return kh_error(st);
  return out;
}

}  // namespace ops

// ---------------------------------------------------------------------------
// WeightStore

namespace {

Result<std::string> read_file(const std::string& path) {
  std::ifstream f(path, std::ios::binary);
  if (!f) return Error{"failed to read " + path + ": cannot open"};
  std::ostringstream ss;
  ss << f.rdbuf();
  return ss.str();
}

Result<Dtype> safetensors_dtype(const std::string& name, const std::string& t) {
  if (t == "F16") return Dtype::Float16;
  if (t == "BF16") return Dtype::Bfloat16;
  if (t == "F32") return Dtype::Float32;
  if (t == "U32") return Dtype::Uint32;
  if (t == "I32") return Dtype::Int32;
  return Error{"tensor " + name + " has unsupported dtype " + t};
}

// A JSON number that is an integer in [0, 2^53].
bool as_count(const json::Value& v, uint64_t* out) {
  if (v.kind != json::Value::Number || !(v.num >= 0) || v.num > 9007199254740992.0 || std::floor(v.num) != v.num)
    return false;
  *out = (uint64_t)v.num;
  return true;
}

// A read-only private mapping of a whole file, unmapped on destruction.
class MappedFile {
 public:
  static Result<MappedFile> open(const std::string& path) {
    const int fd = ::open(path.c_str(), O_RDONLY | O_CLOEXEC);
    if (fd < 0) return Error{"failed to read " + path + ": cannot open"};
    struct stat st;
    if (fstat(fd, &st) != 0) {
      ::close(fd);
      return Error{"failed to read " + path + ": cannot stat"};
    }
    MappedFile m;
    m.size_ = (size_t)st.st_size;
    if (m.size_ > 0) {
      void* p = mmap(nullptr, m.size_, PROT_READ, MAP_PRIVATE, fd, 0);
      if (p == MAP_FAILED) {
        ::close(fd);
        return Error{"failed to map " + path};
      }
      m.data_ = static_cast<const unsigned char*>(p);
      (void)madvise(p, m.size_, MADV_SEQUENTIAL);
    }
    ::close(fd);
    return m;
  }
  MappedFile() = default;
  MappedFile(MappedFile&& o) noexcept : data_(o.data_), size_(o.size_) { o.data_ = nullptr, o.size_ = 0; }
  MappedFile& operator=(MappedFile&& o) noexcept {
    std::swap(data_, o.data_);
    std::swap(size_, o.size_);
    return *this;
  }
  MappedFile(const MappedFile&) = delete;
  ~MappedFile() {
    if (data_) munmap(const_cast<unsigned char*>(data_), size_);
  }
  const unsigned char* data() const { return data_; }
  size_t size() const { return size_; }
  // Give back the pages wholly inside [from, to) (they are re-read from the
  // file if touched again).
  void release(size_t from, size_t to) const {
    const size_t pg = (size_t)sysconf(_SC_PAGESIZE);
    const size_t a = (from + pg - 1) / pg * pg, b = to / pg * pg;
    if (data_ && b > a) (void)madvise(const_cast<unsigned char*>(data_) + a, b - a, MADV_DONTNEED);
  }

 private:
  const unsigned char* data_ = nullptr;
  size_t size_ = 0;
};

// Host -> device copies through two pinned buffers of kStageBytes each: a
// chunk is copied from the mapping into a free buffer, sent asynchronously,
// and the buffer is reused once its event has completed.
class StagedUpload {
 public:
  static constexpr size_t kStageBytes = size_t(32) << 20;
  ~StagedUpload() {
    for (int i = 0; i < 2; ++i) {
      if (ev_[i]) (void)hipEventSynchronize(ev_[i]), (void)hipEventDestroy(ev_[i]);
      if (buf_[i]) (void)hipHostFree(buf_[i]);
    }
  }
  Result<void> init() {
    for (int i = 0; i < 2; ++i) {
      hipError_t e = hipHostMalloc(&buf_[i], kStageBytes, hipHostMallocDefault);
      if (e == hipSuccess) e = hipEventCreateWithFlags(&ev_[i], hipEventDisableTiming);
      if (e != hipSuccess) return hip_error("pinned staging buffer", e);
    }
    return {};
  }
  // Copies file bytes [off, off + n) to dst on stream s, releasing the pages.
  Result<void> copy(const MappedFile& f, size_t off, size_t n, void* dst, hipStream_t s) {
    size_t done = 0;
    while (done < n) {
      const size_t c = std::min(kStageBytes, n - done);
      hipError_t e = hipEventSynchronize(ev_[cur_]);  // this buffer's previous copy has finished
      if (e != hipSuccess) return hip_error("staging copy", e);
      std::memcpy(buf_[cur_], f.data() + off + done, c);
      f.release(off + done, off + done + c);
      e = hipMemcpyAsync(static_cast<char*>(dst) + done, buf_[cur_], c, hipMemcpyHostToDevice, s);
      if (e == hipSuccess) e = hipEventRecord(ev_[cur_], s);
      if (e != hipSuccess) return hip_error("staging copy", e);
      cur_ ^= 1;
      done += c;
    }
    return {};
  }

 private:
  void* buf_[2] = {nullptr, nullptr};
  hipEvent_t ev_[2] = {nullptr, nullptr};
  int cur_ = 0;
};

}  // namespace

Result<std::vector<SafetensorsEntry>> read_safetensors_header(const void* data, size_t size,
                                                              const std::string& path) {
  const auto bad = [&](const std::string& what) { return Error{"invalid safetensors file " + path + ": " + what}; };
  if (size < 8) return bad("too short");
  uint64_t hlen = 0;
  std::memcpy(&hlen, data, 8);  // little-endian u64 header length
  if (hlen > size - 8 || hlen > (uint64_t(100) << 20)) return bad("header length");
  json::Value header;
  try {
    header = json::parse(std::string(static_cast<const char*>(data) + 8, (size_t)hlen));
  } catch (const std::exception& e) {
    return bad(e.what());
  }
  if (!header.is_object()) return bad("header is not an object");
  const uint64_t avail = size - 8 - hlen;
  std::vector<SafetensorsEntry> out;
  for (const auto& kv : header.obj) {
    if (kv.first == "__metadata__") continue;
    const json::Value& t = kv.second;
    const json::Value* dt = t.get("dtype");
    const json::Value* sh = t.get("shape");
    const json::Value* off = t.get("data_offsets");
    if (!dt || !dt->is_string() || !sh || !sh->is_array() || !off || !off->is_array() || off->arr.size() != 2)
      return bad("bad entry " + kv.first);
    auto dtype = safetensors_dtype(kv.first, dt->str);
    if (!dtype) return dtype.error();
    if (sh->arr.size() > KH_MAX_NDIM) return bad("rank of " + kv.first);
    SafetensorsEntry e;
    e.name = kv.first;
    e.dtype = dtype.value();
    uint64_t count = 1;
    for (const auto& d : sh->arr) {
      uint64_t v;
      if (!as_count(d, &v)) return bad("shape of " + kv.first);
      if (v != 0 && count > (uint64_t(1) << 48) / v) return bad("shape of " + kv.first);
      count *= v;
      e.shape.push_back((int64_t)v);
    }
    uint64_t o0, o1;
    if (!as_count(off->arr[0], &o0) || !as_count(off->arr[1], &o1) || o1 < o0 || o1 > avail)
      return bad("data offsets of " + kv.first);
    if (count * (uint64_t)dtype_size(e.dtype) != o1 - o0)
      return bad("data offsets of " + kv.first + " do not match its shape");
    e.offset = o0;
    e.nbytes = o1 - o0;
    out.push_back(std::move(e));
  }
  return out;
}

Result<WeightStore> WeightStore::from_model_dir(const std::string& dir, const Stream& s) {
  std::set<std::string> files;
  const std::string index_path = dir + "/model.safetensors.index.json";
  {
    std::ifstream probe(index_path);
    if (probe) {
      auto text = read_file(index_path);
      if (!text) return text.error();
      json::Value idx;
      try {
        idx = json::parse(text.value());
      } catch (const std::exception& e) {
        return Error{"invalid weight index " + index_path + ": " + e.what()};
      }
      const json::Value* wm = idx.get("weight_map");
      if (!wm || !wm->is_object()) return Error{"invalid weight index " + index_path + ": no weight_map object"};
      for (const auto& kv : wm->obj)
        if (kv.second.is_string()) files.insert(kv.second.str);
    } else {
      files.insert("model.safetensors");
    }
  }
  WeightStore store;
  StagedUpload up;
  bool staged = false;
  for (const std::string& file : files) {
    const std::string path = dir + "/" + file;
    auto mf = MappedFile::open(path);
    if (!mf) return mf.error();
    const MappedFile& m = mf.value();
    auto entries = read_safetensors_header(m.data(), m.size(), path);
    if (!entries) return entries.error();
    uint64_t hlen = 0;
    std::memcpy(&hlen, m.data(), 8);
    const size_t base = 8 + (size_t)hlen;
    for (const SafetensorsEntry& e : entries.value()) {
      auto r = Array::empty(e.shape, e.dtype, s);
      if (!r) return Error{"tensor " + e.name + ": " + r.error().message};
      Array arr = r.take();
      if (e.nbytes) {
        if (!staged) {
          auto ok = up.init();
          if (!ok) return ok.error();
          staged = true;
        }
        auto ok = up.copy(m, base + e.offset, e.nbytes, arr.data(), s.raw());
        if (!ok) return Error{"tensor " + e.name + ": " + ok.error().message};
      }
      store.tensors_[e.name] = std::move(arr);
    }
    // the mapping is dropped at the end of this iteration: finish its copies
    const hipError_t err = hipStreamSynchronize(s.raw());
    if (err != hipSuccess) return hip_error("checkpoint upload", err);
  }
  return store;
}

Result<Array> WeightStore::take(const std::string& name) {
  auto it = tensors_.find(name);
  if (it == tensors_.end()) return Error{"missing tensor " + name};
  Array a = std::move(it->second);
  tensors_.erase(it);
  return a;
}

std::optional<Array> WeightStore::take_optional(const std::string& name) {
  auto it = tensors_.find(name);
  if (it == tensors_.end()) return std::nullopt;
  Array a = std::move(it->second);
  tensors_.erase(it);
  return std::optional<Array>(std::move(a));
}

std::vector<std::string> WeightStore::remaining() const {
  std::vector<std::string> names;
  for (const auto& kv : tensors_) names.push_back(kv.first);
  std::sort(names.begin(), names.end());
  return names;
}

// ---------------------------------------------------------------------------
// Quantization config

Result<void> validate_quant_params(const std::optional<Quantization>& q) {
  if (q && ((q->bits != 4 && q->bits != 8) ||
            (q->group_size != 32 && q->group_size != 64 && q->group_size != 128)))
    return Error{"unsupported quantization: bits=" + std::to_string(q->bits) + " group_size=" +
                 std::to_string(q->group_size) + " (supported: 4/8 bits, 32/64/128 groups)"};
  return {};
}

Result<void> validate_quantization(const json::Value& config) {
  const json::Value* quant = config.get("quantization");
  if (!quant || !quant->is_object()) return {};
  const json::Value* mode = quant->get("mode");
  if (mode && !(mode->is_string() && mode->str == "affine")) {
    const std::string shown = mode->is_string() ? "\"" + mode->str + "\"" : "(non-string)";
    return Error{"unsupported quantization: quantization mode " + shown + " (supported: \"affine\")"};
  }
  std::vector<std::string> offending;
  for (const auto& kv : quant->obj)
    if (kv.first != "group_size" && kv.first != "bits" && kv.first != "mode") offending.push_back(kv.first);
  if (offending.empty()) return {};
  std::sort(offending.begin(), offending.end());
  std::string list = "[";
  for (size_t i = 0; i < offending.size(); ++i) list += (i ? ", \"" : "\"") + offending[i] + "\"";
  list += "]";
  return Error{"unsupported quantization: per-module quantization overrides " + list +
               " — only uniform affine group_size/bits are supported"};
}

Result<std::optional<Quantization>> quantization_from_config(const json::Value& config) {
  auto v = validate_quantization(config);
  if (!v) return v.error();
  const json::Value* quant = config.get("quantization");
  if (!quant || !quant->is_object()) return std::optional<Quantization>();
  const json::Value* gs = quant->get("group_size");
  const json::Value* bits = quant->get("bits");
  if (!gs || !gs->is_number() || !bits || !bits->is_number())
    return Error{"unsupported quantization: quantization block needs numeric group_size and bits"};
  std::optional<Quantization> q = Quantization{(int)gs->num, (int)bits->num};
  auto p = validate_quant_params(q);
  if (!p) return p.error();
  return q;
}

// ---------------------------------------------------------------------------
// nn

namespace nn {

Result<Linear> Linear::load(WeightStore& store, const std::string& prefix,
                            const std::optional<Quantization>& q) {
  Linear l;
  l.bias_ = store.take_optional(prefix + ".bias");
  if (store.contains(prefix + ".scales")) {
    if (!q)
      return Error{"weights/config mismatch: " + prefix +
                   " has quantized tensors but config.json has no quantization block"};
    auto w = store.take(prefix + ".weight");
    if (!w) return w.error();
    auto s = store.take(prefix + ".scales");
    if (!s) return s.error();
    auto b = store.take(prefix + ".biases");
    if (!b) return b.error();
    l.quantized_ = true;
    l.weight_ = w.take();
    l.scales_ = s.take();
    l.biases_ = b.take();
    l.group_size_ = q->group_size;
    l.bits_ = q->bits;
  } else {
    auto w = store.take(prefix + ".weight");
    if (!w) return w.error();
    l.weight_ = w.take();
  }
  return l;
}

Result<Array> Linear::forward(const Array& x, const Stream& s) const {
  if (!quantized_) return Error{"dense Linear is outside the quantized path this library implements"};
  return ops::linear(x, weight_, scales_, biases_, bias_, group_size_, bits_, s);
}

Result<Mlp> Mlp::load(WeightStore& store, const std::string& prefix, const std::optional<Quantization>& q,
                      Activation activation) {
  Mlp m;
  auto g = Linear::load(store, prefix + ".gate_proj", q);
  if (!g) return g.error();
  auto u = Linear::load(store, prefix + ".up_proj", q);
  if (!u) return u.error();
  auto d = Linear::load(store, prefix + ".down_proj", q);
  if (!d) return d.error();
  m.gate_proj_ = g.take();
  m.up_proj_ = u.take();
  m.down_proj_ = d.take();
  m.activation_ = activation;
  return m;
}

Result<Array> Mlp::forward(const Array& x, const Stream& s) const {
  const Linear& g = gate_proj_;
  const Linear& u = up_proj_;
  if (!g.quantized_ || !u.quantized_)
    return Error{"dense Linear is outside the quantized path this library implements"};
  std::vector<int64_t> shape = x.shape();
  shape.back() = g.weight_.dim(0);
  Dtype dt = ops::promote(x.dtype(), g.scales_.dtype());
  if (g.bias_) dt = ops::promote(dt, g.bias_->dtype());
  auto r = Array::empty(shape, dt, s);
  if (!r) return r.error();
  Array act = r.take();
  kh_array res = act.desc(), xd = x.desc();
  kh_array gw = g.weight_.desc(), gs = g.scales_.desc(), gb = g.biases_.desc();
  kh_array uw = u.weight_.desc(), us = u.scales_.desc(), ub = u.biases_.desc();
  kh_array gbias{}, ubias{};
  if (g.bias_) gbias = g.bias_->desc();
  if (u.bias_) ubias = u.bias_->desc();
  const int st = kh_mlp_gate_up(&res, &xd, &gw, &gs, &gb, g.bias_ ? &gbias : nullptr, &uw, &us, &ub,
                                u.bias_ ? &ubias : nullptr, static_cast<int>(activation_),
                                ops::opt(g.group_size_), ops::opt(g.bits_), "affine", s.raw());
  if (st) return kh_error(st);
  return down_proj_.forward(act, s);
}

std::pair<int64_t, int64_t> Linear::io_features() const {
  if (quantized_) return {scales_.dim(1) * group_size_, scales_.dim(0)};
  return {weight_.dim(1), weight_.dim(0)};
}

Result<SwitchLinear> SwitchLinear::load(WeightStore& store, const std::string& mlp_prefix,
                                        const std::string& proj, int num_experts,
                                        const std::optional<Quantization>& q, const Stream& s) {
  const std::string stacked = mlp_prefix + ".switch_mlp." + proj;
  auto per = [&](int e, const char* name) {
    return mlp_prefix + ".experts." + std::to_string(e) + "." + proj + "." + name;
  };
  const bool is_stacked = store.contains(stacked + ".scales");
  if (!is_stacked && !store.contains(per(0, "scales")))
    return Error{"dense " + stacked + " is outside the quantized path this library implements"};
  if (!q)
    return Error{"weights/config mismatch: " + stacked +
                 " has quantized tensors but config.json has no quantization block"};
  if (num_experts < 1) return Error{"[SwitchLinear] num_experts must be >= 1"};
  // one tensor of every expert, stacked along axis 0
  auto gather = [&](const char* name) -> Result<Array> {
    std::vector<Array> parts;
    for (int e = 0; e < num_experts; ++e) {
      auto t = store.take(per(e, name));
      if (!t) return t.error();
      parts.push_back(t.take());
    }
    return ops::stack(parts, s);
  };
  auto one = [&](const char* name) -> Result<Array> {
    return is_stacked ? store.take(stacked + "." + name) : gather(name);
  };
  SwitchLinear l;
  auto w = one("weight");
  if (!w) return w.error();
  auto sc = one("scales");
  if (!sc) return sc.error();
  auto bi = one("biases");
  if (!bi) return bi.error();
  l.weight_ = w.take();
  l.scales_ = sc.take();
  l.biases_ = bi.take();
  if (l.weight_.ndim() != 3 || l.weight_.dim(0) != num_experts)
    return Error{"[SwitchLinear] " + stacked + ".weight is not a stack of " + std::to_string(num_experts) +
                 " experts"};
  if (is_stacked ? store.contains(stacked + ".bias") : store.contains(per(0, "bias"))) {
    auto b = one("bias");
    if (!b) return b.error();
    l.bias_ = b.take();
  }
  l.group_size_ = q->group_size;
  l.bits_ = q->bits;
  return l;
}

Result<Array> SwitchLinear::forward(const Array& x, const Array& indices, bool sorted_indices,
                                    const Stream& s) const {
  auto y = ops::gather_qmm(x, weight_, scales_, biases_, indices, true, group_size_, bits_, sorted_indices, s);
  if (!y || !bias_) return y;
  // y + expand_dims(bias[indices], -2): bias rows gathered to indices.shape +
  // [1, N], broadcast against y [batch..., M, N]
  auto g = ops::take(*bias_, indices, 0, s);
  if (!g) return g;
  std::vector<int64_t> shape = g.value().shape();
  shape.insert(shape.end() - 1, 1);
  auto gv = g.value().view(shape);
  if (!gv) return gv.error();
  return ops::add(y.value(), gv.value(), s);
}

Result<Embedding> Embedding::load(WeightStore& store, const std::string& prefix,
                                  const std::optional<Quantization>& q) {
  Embedding e;
  if (store.contains(prefix + ".scales")) {
    if (!q)
      return Error{"weights/config mismatch: " + prefix +
                   " has quantized tensors but config.json has no quantization block"};
    auto w = store.take(prefix + ".weight");
    if (!w) return w.error();
    auto s = store.take(prefix + ".scales");
    if (!s) return s.error();
    auto b = store.take(prefix + ".biases");
    if (!b) return b.error();
    e.quantized_ = true;
    e.weight_ = w.take();
    e.scales_ = s.take();
    e.biases_ = b.take();
    e.group_size_ = q->group_size;
    e.bits_ = q->bits;
  } else {
    auto w = store.take(prefix + ".weight");
    if (!w) return w.error();
    e.weight_ = w.take();
  }
  return e;
}

Result<Array> Embedding::lookup(const Array& ids, const Stream& s) const {
  if (!quantized_) return ops::take(weight_, ids, 0, s);
  return ops::quantized_embedding(ids, weight_, scales_, biases_, group_size_, bits_, s);
}

Result<Array> Embedding::as_linear(const Array& h, const Stream& s) const {
  if (!quantized_) return Error{"dense tied head is outside the quantized path this library implements"};
  return ops::quantized_matmul(h, weight_, scales_, biases_, true, group_size_, bits_, s);
}

Result<int> probe_row_stability(int64_t k, const Array& base, const Stream& s,
                                const std::function<Result<Array>(const Array&)>& f) {
  if (base.ndim() != 3 || base.dim(0) != 1 || base.dim(1) != 1) return Error{"base must be [1, 1, hidden]"};
  auto hb = base.to_bytes(s);
  if (!hb) return hb.error();
  const size_t esz = dtype_size(base.dtype());
  const int64_t hidden = base.dim(2);
  std::vector<uint8_t> row((size_t)k * esz);
  for (int64_t i = 0; i < k; ++i)
    std::memcpy(row.data() + i * esz, hb.value().data() + (i % hidden) * esz, esz);
  auto row0 = [&](int m) -> Result<std::vector<uint8_t>> {
    std::vector<uint8_t> rows;
    rows.reserve(row.size() * m);
    for (int j = 0; j < m; ++j) rows.insert(rows.end(), row.begin(), row.end());
    auto x = Array::from_bytes(rows.data(), rows.size(), {1, m, k}, base.dtype(), s);
    if (!x) return x.error();
    auto y = f(x.value());
    if (!y) return y.error();
    auto bytes = y.value().to_bytes(s);
    if (!bytes) return bytes.error();
    const size_t rb = bytes.value().size() / (size_t)m;
    return std::vector<uint8_t>(bytes.value().begin(), bytes.value().begin() + rb);
  };
  auto ref = row0(1);
  if (!ref) return ref.error();
  for (int m = 2; m <= 32; ++m) {
    auto r = row0(m);
    if (!r) return r.error();
    if (r.value() != ref.value()) return m;
  }
  return 33;
}

}  // namespace nn
}  // namespace kiln
