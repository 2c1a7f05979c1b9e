// kiln_host.hpp — C++ host layer over the kiln_hip C ABI.
//
// Mirrors, for the quantized-linear path, the Rust surface Kiln's models are
// written against, so that layer code ports one-to-one:
//   kiln::Array / Stream / Error / Result   crates/kiln-mlx/src/{array,stream,error}.rs
//   kiln::ops::{quantized_matmul, gather_qmm, dequantize, take, add}   crates/kiln-mlx/src/ops.rs
//   kiln::WeightStore                      crates/kiln-models/src/weights.rs:37-130
//   kiln::Quantization, validate_*         crates/kiln-models/src/config.rs:28-33, 137-148, 735-760
//   kiln::nn::Linear / Embedding           crates/kiln-models/src/nn.rs:30-194
//   kiln::nn::SwitchLinear                 crates/kiln-models/src/moe.rs:47-176
//   kiln::nn::probe_row_stability          crates/kiln-models/src/nn.rs:301-327
//
// Conventions carried over: fallible calls return Result (never abort); an
// Array owns one device buffer, moves are cheap, copies are explicit
// (clone aliases in MLX; here `share()` returns a non-owning alias); all work
// is enqueued on a Stream and is complete after Stream::synchronize().
// Device buffers come from a stream-aware caching allocator, so the steady
// state of a decode loop performs no hipMalloc/hipFree.
#pragma once

#include <hip/hip_runtime.h>

#include <cstdint>
#include <functional>
#include <map>
#include <memory>
#include <optional>
#include <string>
#include <utility>
#include <vector>

#include "../../include/kiln_hip.h"
#include "json_min.hpp"

namespace kiln {

// Element types used on this path (subset of mlx_dtype, array.rs:22-69).
enum class Dtype : int32_t {
  Bool = KH_BOOL,
  Uint8 = KH_UINT8,
  Uint16 = KH_UINT16,
  Uint32 = KH_UINT32,
  Int32 = KH_INT32,
  Float16 = KH_FLOAT16,
  Float32 = KH_FLOAT32,
  Bfloat16 = KH_BFLOAT16,
};

size_t dtype_size(Dtype d);
const char* dtype_name(Dtype d);

struct Error {
  std::string message;
};

// Result<T>: a value or an Error (the Rust `Result<T, MlxError>`).
template <class T>
class Result {
 public:
  Result(T v) : val_(std::move(v)) {}  // NOLINT(google-explicit-constructor)
  Result(Error e) : err_(std::move(e)) {}  // NOLINT(google-explicit-constructor)
  bool ok() const { return val_.has_value(); }
  explicit operator bool() const { return ok(); }
  T& value() { return *val_; }
  const T& value() const { return *val_; }
  T take() { return std::move(*val_); }
  const Error& error() const { return err_; }

 private:
  std::optional<T> val_;
  Error err_;
};

template <>
class Result<void> {
 public:
  Result() = default;
  Result(Error e) : ok_(false), err_(std::move(e)) {}  // NOLINT(google-explicit-constructor)
  bool ok() const { return ok_; }
  explicit operator bool() const { return ok_; }
  const Error& error() const { return err_; }

 private:
  bool ok_ = true;
  Error err_;
};

// An execution stream (hipStream_t). `Stream::gpu()` is the device's null
// stream; `Stream::create()` makes a new one (default priority), owned.
class Stream {
 public:
  static Stream gpu();
  static Result<Stream> create();
  Stream(Stream&& o) noexcept : s_(o.s_), owned_(o.owned_) { o.owned_ = false; }
  Stream& operator=(Stream&&) = delete;
  Stream(const Stream&) = delete;
  ~Stream();
  Result<void> synchronize() const;
  hipStream_t raw() const { return s_; }

 private:
  Stream(hipStream_t s, bool owned) : s_(s), owned_(owned) {}
  hipStream_t s_;
  bool owned_;
};

// An owning N-d array in device memory (row-contiguous).
class Array {
 public:
  Array() = default;
  Array(Array&& o) noexcept { *this = std::move(o); }
  Array& operator=(Array&& o) noexcept;
  Array(const Array&) = delete;
  Array& operator=(const Array&) = delete;
  ~Array();

  // New uninitialised array, memory from the caching allocator, usable on `s`.
  static Result<Array> empty(const std::vector<int64_t>& shape, Dtype dtype, const Stream& s);
  // Copy `bytes` (row-major, element type `dtype`) into a new device array.
  static Result<Array> from_bytes(const void* bytes, size_t nbytes, const std::vector<int64_t>& shape,
                                  Dtype dtype, const Stream& s);
  // A non-owning alias of the same buffer (MLX Clone aliases too).
  Array share() const;
  // A non-owning alias with another shape of the same element count (a
  // reshape of a row-contiguous array).
  Result<Array> view(const std::vector<int64_t>& shape) const;

  Result<std::vector<uint8_t>> to_bytes(const Stream& s) const;  // synchronises `s`
  int ndim() const { return (int)shape_.size(); }
  int64_t dim(int i) const { return shape_[i < 0 ? i + ndim() : i]; }
  const std::vector<int64_t>& shape() const { return shape_; }
  Dtype dtype() const { return dtype_; }
  int64_t size() const;
  size_t nbytes() const { return (size_t)size() * dtype_size(dtype_); }
  void* data() const { return data_; }
  kh_array desc() const;

 private:
  void* data_ = nullptr;
  size_t cap_ = 0;
  std::vector<int64_t> shape_;
  Dtype dtype_ = Dtype::Float32;
  hipStream_t stream_ = nullptr;  // allocation stream (reuse is stream-ordered)
  bool owner_ = false;
};

// Bytes held by the caching allocator (in use, cached) and a trim that
// returns cached blocks to the device.
struct AllocatorStats {
  size_t in_use = 0, cached = 0, device_allocs = 0;
};
AllocatorStats allocator_stats();
void allocator_trim();

namespace ops {
// crates/kiln-mlx/src/ops.rs:359-388 (mode "affine"; output dtype follows
// MLX promotion of x, scales, biases).
Result<Array> quantized_matmul(const Array& x, const Array& w, const Array& scales,
                               const Array& biases, bool transpose, int group_size, int bits,
                               const Stream& s);
// ops.rs:390-429 with null lhs_indices: per batch pair, x[b] @ w[e_b]^T over
// expert stacks w/scales/biases [E, N, ..]; batch = broadcast(x.shape[:-2],
// indices.shape); result [batch..., M, N].
Result<Array> gather_qmm(const Array& x, const Array& w, const Array& scales, const Array& biases,
                         const Array& indices, bool transpose, int group_size, int bits,
                         bool sorted_indices, const Stream& s);
// Arrays of one shape and dtype stacked along a new axis 0 (mx.stack).
Result<Array> stack(const std::vector<Array>& parts, const Stream& s);
// ops.rs:456-484 (output dtype = scales dtype).
Result<Array> dequantize(const Array& w, const Array& scales, const Array& biases, int group_size,
                         int bits, const Stream& s);
// ops.rs:249-254, axis 0 only.
Result<Array> take(const Array& a, const Array& indices, int axis, const Stream& s);
// Embedding::lookup's take x3 + dequantize in one pass (nn.rs:159-176).
Result<Array> quantized_embedding(const Array& ids, const Array& w, const Array& scales,
                                  const Array& biases, int group_size, int bits, const Stream& s);
// a + b with numpy broadcasting (mlx_add); the Linear bias add of
// nn.rs:98-100 and SwitchLinear's expert bias (moe.rs:166-172).
Result<Array> add(const Array& a, const Array& b, const Stream& s);
// Linear::forward's quantized matmul (transpose=true) and optional bias in
// one launch (kh_linear): the product in its own dtype, then + bias.
Result<Array> linear(const Array& x, const Array& w, const Array& scales, const Array& biases,
                     const std::optional<Array>& bias, int group_size, int bits, const Stream& s);
}  // namespace ops

// One tensor of a safetensors file: dtype, shape and its byte range within
// the data section (after the 8-byte length and the JSON header).
struct SafetensorsEntry {
  std::string name;
  Dtype dtype;
  std::vector<int64_t> shape;
  uint64_t offset = 0, nbytes = 0;
};
// Parses and validates the header of a safetensors file held in `data`
// (`size` bytes): dtypes, non-negative integral dims whose element count
// times the element size equals the entry's byte range, and byte ranges
// inside the file. Malformed input is an error, never a huge allocation.
Result<std::vector<SafetensorsEntry>> read_safetensors_header(const void* data, size_t size,
                                                              const std::string& path);

// safetensors checkpoint store: weights.rs:37-130 (single file or sharded
// through model.safetensors.index.json; F16/BF16/F32/U32/I32 tensors). Each
// file is memory-mapped read-only (as weights.rs:76 maps it through
// MappedFile, io.rs:22-30) and copied to the device through a bounded pinned
// staging buffer; pages already copied are released, so the host memory a
// load holds stays near the staging buffer's size.
class WeightStore {
 public:
  static Result<WeightStore> from_model_dir(const std::string& dir, const Stream& s);
  Result<Array> take(const std::string& name);
  std::optional<Array> take_optional(const std::string& name);
  bool contains(const std::string& name) const { return tensors_.count(name) != 0; }
  std::vector<std::string> remaining() const;

 private:
  std::map<std::string, Array> tensors_;
};

// mlx-lm affine quantization parameters (config.rs:28-33).
struct Quantization {
  int group_size = 64;
  int bits = 4;
};
// config.rs:137-148: bits 4|8, group_size 32|64|128.
Result<void> validate_quant_params(const std::optional<Quantization>& q);
// config.rs:735-760: mode must be "affine"; no per-module overrides.
Result<void> validate_quantization(const json::Value& config);
// The `quantization` block of a config.json, validated.
Result<std::optional<Quantization>> quantization_from_config(const json::Value& config);

namespace nn {

// Linear (nn.rs:30-114): quantized iff `{prefix}.scales` exists.
class Linear {
 public:
  static Result<Linear> load(WeightStore& store, const std::string& prefix,
                             const std::optional<Quantization>& q);
  Result<Array> forward(const Array& x, const Stream& s) const;
  std::pair<int64_t, int64_t> io_features() const;  // (in, out)
  bool quantized() const { return quantized_; }

 private:
  friend class Mlp;
  bool quantized_ = false;
  Array weight_, scales_, biases_;
  std::optional<Array> bias_;
  int group_size_ = 64, bits_ = 4;
};

// The gated MLP's activation (nn.rs:259-294).
enum class Activation { Silu = KH_ACT_SILU, GeluApprox = KH_ACT_GELU_APPROX };

// Mlp (nn.rs:259-294): down(act(gate(x)) * up(x)), the gate/up half in one
// kh_mlp_gate_up call (one launch at decode sizes).
class Mlp {
 public:
  static Result<Mlp> load(WeightStore& store, const std::string& prefix,
                          const std::optional<Quantization>& q, Activation activation);
  Result<Array> forward(const Array& x, const Stream& s) const;

 private:
  Linear gate_proj_, up_proj_, down_proj_;
  Activation activation_ = Activation::Silu;
};

// Embedding (nn.rs:116-194): quantized or dense, also the tied LM head.
class Embedding {
 public:
  static Result<Embedding> load(WeightStore& store, const std::string& prefix,
                                const std::optional<Quantization>& q);
  Result<Array> lookup(const Array& ids, const Stream& s) const;   // [..] -> [.., hidden]
  Result<Array> as_linear(const Array& h, const Stream& s) const;  // [.., hidden] -> [.., vocab]
  bool quantized() const { return quantized_; }

 private:
  bool quantized_ = false;
  Array weight_, scales_, biases_;
  int group_size_ = 64, bits_ = 4;
};

// SwitchLinear (moe.rs:47-176), quantized form: one projection per expert,
// stacked [E, out, in], applied with gather_qmm on per-token expert ids.
// Loads `{mlp_prefix}.switch_mlp.{proj}` (already stacked, as mlx-lm saves
// after conversion) or `{mlp_prefix}.experts.{e}.{proj}` (stacked here along
// axis 0, as the reference's load does).
class SwitchLinear {
 public:
  static Result<SwitchLinear> load(WeightStore& store, const std::string& mlp_prefix, const std::string& proj,
                                   int num_experts, const std::optional<Quantization>& q, const Stream& s);
  // x @ W[indices]^T (+ bias[indices]); sorted_indices is the caller's
  // do_sort (a scheduling hint, moe.rs:124-176). With an expert bias, each
  // batch pair must hold one row (SwitchGlu's use).
  Result<Array> forward(const Array& x, const Array& indices, bool sorted_indices, const Stream& s) const;
  int num_experts() const { return (int)weight_.dim(0); }

 private:
  Array weight_, scales_, biases_;
  std::optional<Array> bias_;
  int group_size_ = 64, bits_ = 4;
};

// nn.rs:301-327: smallest M in 2..=32 at which row 0 of f([x1; ...; x1])
// stops being bit-identical to f(x1) (33 when it never diverges). `base` is a
// [1, 1, hidden] row tiled to k features.
Result<int> probe_row_stability(int64_t k, const Array& base, const Stream& s,
                                const std::function<Result<Array>(const Array&)>& f);

}  // namespace nn
}  // namespace kiln
