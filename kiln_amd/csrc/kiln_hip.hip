// kiln_hip.hip — the extern "C" boundary (include/kiln_hip.h): argument
// validation, MLX-compatible shape rules, thread-local error reporting, and
// dispatch to the gfx950 kernels.
//
// Error behaviour mirrors the Kiln/mlx-c contract (crates/kiln-mlx/src/error.rs:24-72):
// a failing call returns non-zero and leaves a message retrievable on the
// calling thread; nothing aborts. Every argument check runs before any HIP
// call, so validation behaves identically on a machine without a GPU.
#include <hip/hip_runtime.h>

#include <algorithm>
#include <cstdarg>
#include <cstdio>
#include <cstring>
#include <map>
#include <tuple>
#include <mutex>
#include <string>
#include <utility>
#include <vector>

#include "../../include/kiln_hip.h"
#include "kh_kernels.h"

namespace {

thread_local std::string g_last_error;

int fail(int code, const char* fmt, ...) {
  char buf[512];
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(buf, sizeof buf, fmt, ap);
  va_end(ap);
  g_last_error = buf;
  return code;
}

const char* dtype_name(int dt) {
  switch (dt) {
    case KH_BOOL: return "bool";
    case KH_UINT8: return "uint8";
    case KH_UINT16: return "uint16";
    case KH_UINT32: return "uint32";
    case KH_UINT64: return "uint64";
    case KH_INT8: return "int8";
    case KH_INT16: return "int16";
    case KH_INT32: return "int32";
    case KH_INT64: return "int64";
    case KH_FLOAT16: return "float16";
    case KH_FLOAT32: return "float32";
    case KH_FLOAT64: return "float64";
    case KH_BFLOAT16: return "bfloat16";
    case KH_COMPLEX64: return "complex64";
    default: return "unknown";
  }
}

int64_t dtype_size(int dt) {
  switch (dt) {
    case KH_BOOL: case KH_UINT8: case KH_INT8: return 1;
    case KH_UINT16: case KH_INT16: case KH_FLOAT16: case KH_BFLOAT16: return 2;
    case KH_UINT32: case KH_INT32: case KH_FLOAT32: return 4;
    case KH_UINT64: case KH_INT64: case KH_FLOAT64: case KH_COMPLEX64: return 8;
    default: return 0;
  }
}

bool is_float(int dt) { return dt == KH_FLOAT16 || dt == KH_BFLOAT16 || dt == KH_FLOAT32; }

std::string shape_str(const kh_array* a) {
  std::string s = "(";
  for (int i = 0; i < a->ndim; ++i) {
    if (i) s += ",";
    s += std::to_string(a->shape[i]);
  }
  return s + ")";
}

int64_t numel(const kh_array* a) {
  int64_t n = 1;
  for (int i = 0; i < a->ndim; ++i) n *= a->shape[i];
  return n;
}

// Structural checks shared by every entry point.
int check_array(const kh_array* a, const char* op, const char* name) {
  if (!a) return fail(KH_ERR_INVALID_ARGUMENT, "[%s] %s is NULL", op, name);
  if (a->ndim < 0 || a->ndim > KH_MAX_NDIM)
    return fail(KH_ERR_INVALID_ARGUMENT, "[%s] %s has ndim %d (0..%d)", op, name, a->ndim, KH_MAX_NDIM);
  if (dtype_size(a->dtype) == 0)
    return fail(KH_ERR_INVALID_ARGUMENT, "[%s] %s has invalid dtype %d", op, name, a->dtype);
  for (int i = 0; i < a->ndim; ++i)
    if (a->shape[i] < 0)
      return fail(KH_ERR_INVALID_ARGUMENT, "[%s] %s has negative dimension %lld", op, name,
                  (long long)a->shape[i]);
  if (!a->data && numel(a) > 0) return fail(KH_ERR_INVALID_ARGUMENT, "[%s] %s data is NULL", op, name);
  return KH_OK;
}

// Quantization parameters: the domain Kiln accepts
// (crates/kiln-models/src/config.rs:137-148, 735-760) with MLX's defaults.
int check_quant(const char* op, kh_optional_int gs_opt, kh_optional_int bits_opt, const char* mode,
                int* gs, int* bits) {
  if (mode && std::strcmp(mode, "affine") != 0)
    return fail(KH_ERR_INVALID_ARGUMENT, "[%s] quantization mode \"%s\" (supported: \"affine\")", op, mode);
  *gs = gs_opt.has_value ? gs_opt.value : 64;
  *bits = bits_opt.has_value ? bits_opt.value : 4;
  if ((*bits != 4 && *bits != 8) || (*gs != 32 && *gs != 64 && *gs != 128))
    return fail(KH_ERR_INVALID_ARGUMENT,
                "[%s] bits=%d group_size=%d (supported: 4/8 bits, 32/64/128 groups)", op, *bits, *gs);
  return KH_OK;
}

// Packed weights plus scales/biases of matching shape: w [..., R, C*bits/32]
// with scales/biases [..., R, C/gs].
int check_packed(const char* op, const kh_array* w, const kh_array* s, const kh_array* b, int gs,
                 int bits, int64_t* rows, int64_t* cols) {
  int rc;
  if ((rc = check_array(w, op, "w")) || (rc = check_array(s, op, "scales")) ||
      (rc = check_array(b, op, "biases")))
    return rc;
  if (w->dtype != KH_UINT32)
    return fail(KH_ERR_INVALID_ARGUMENT, "[%s] packed weights must be uint32, got %s", op, dtype_name(w->dtype));
  if (w->ndim < 2) return fail(KH_ERR_INVALID_ARGUMENT, "[%s] w must have ndim >= 2, got %d", op, w->ndim);
  if (!is_float(s->dtype))
    return fail(KH_ERR_INVALID_ARGUMENT, "[%s] scales must be float16/bfloat16/float32, got %s", op, dtype_name(s->dtype));
  if (s->dtype != b->dtype)
    return fail(KH_ERR_INVALID_ARGUMENT, "[%s] scales (%s) and biases (%s) must share a dtype", op,
                dtype_name(s->dtype), dtype_name(b->dtype));
  if (s->ndim != w->ndim || b->ndim != w->ndim)
    return fail(KH_ERR_INVALID_ARGUMENT, "[%s] w %s, scales %s, biases %s: ranks differ", op,
                shape_str(w).c_str(), shape_str(s).c_str(), shape_str(b).c_str());
  for (int i = 0; i < w->ndim; ++i)
    if (s->shape[i] != b->shape[i])
      return fail(KH_ERR_INVALID_ARGUMENT, "[%s] scales %s and biases %s differ in shape", op,
                  shape_str(s).c_str(), shape_str(b).c_str());
  for (int i = 0; i < w->ndim - 1; ++i)
    if (s->shape[i] != w->shape[i])
      return fail(KH_ERR_INVALID_ARGUMENT, "[%s] w %s and scales %s disagree", op,
                  shape_str(w).c_str(), shape_str(s).c_str());
  const int64_t c = w->shape[w->ndim - 1] * (32 / bits);
  if (s->shape[s->ndim - 1] * gs != c)
    return fail(KH_ERR_INVALID_ARGUMENT,
                "[%s] w %s holds %lld columns at %d bits but scales %s cover %lld at group_size %d",
                op, shape_str(w).c_str(), (long long)c, bits, shape_str(s).c_str(),
                (long long)(s->shape[s->ndim - 1] * gs), gs);
  *cols = c;
  int64_t r = 1;
  for (int i = 0; i < w->ndim - 1; ++i) r *= w->shape[i];
  *rows = r;
  return KH_OK;
}

int check_result(const char* op, const kh_array* res, const kh_array& want) {
  int rc = check_array(res, op, "res");
  if (rc) return rc;
  if (!is_float(res->dtype))
    return fail(KH_ERR_INVALID_ARGUMENT, "[%s] res dtype must be float16/bfloat16/float32, got %s", op,
                dtype_name(res->dtype));
  bool same = res->ndim == want.ndim;
  for (int i = 0; same && i < want.ndim; ++i) same = res->shape[i] == want.shape[i];
  if (!same)
    return fail(KH_ERR_INVALID_ARGUMENT, "[%s] res has shape %s, expected %s", op,
                shape_str(res).c_str(), shape_str(&want).c_str());
  return KH_OK;
}

int hip_fail(const char* op, hipError_t e) {
  return fail(KH_ERR_DEVICE, "[%s] HIP error %d: %s", op, (int)e, hipGetErrorString(e));
}

// One-time per device: the code objects are built for gfx950 only.
int check_device(const char* op) {
  static std::mutex mu;
  static std::map<int, bool> ok;
  int dev = 0;
  hipError_t e = hipGetDevice(&dev);
  if (e != hipSuccess) return fail(KH_ERR_NO_DEVICE, "[%s] no HIP device: %s", op, hipGetErrorString(e));
  std::lock_guard<std::mutex> lock(mu);
  auto it = ok.find(dev);
  if (it == ok.end()) {
    hipDeviceProp_t p;
    e = hipGetDeviceProperties(&p, dev);
    if (e != hipSuccess) return hip_fail(op, e);
    it = ok.emplace(dev, std::strncmp(p.gcnArchName, "gfx950", 6) == 0).first;
    if (!it->second)
      return fail(KH_ERR_NO_DEVICE, "[%s] device %d is %s; this library is built for gfx950 only",
                  op, dev, p.gcnArchName);
  }
  return it->second ? KH_OK : fail(KH_ERR_NO_DEVICE, "[%s] device %d is not gfx950", op, dev);
}

// Per (device, stream) workspace of float scratch (split-K partials, the
// prefill GEMM's float16 activations and row scales, grouped-gather plans).
// Grown on demand and never shrunk, so the steady state performs no
// allocation; the first call that needs more than the stream's buffer holds
// allocates (hipMalloc). Calls on one stream are ordered, so they can share it.
//
// A buffer that a HIP graph captured may be used by every later replay of
// that graph, so once a slot has been handed out while its stream was
// capturing, the buffer is never freed: when it has to grow it is retired
// (kept until the process ends) and a new one is allocated. Buffers never
// seen by a capture are freed after synchronising their stream.
std::vector<void*>& retired() {
  static std::vector<void*> v;
  return v;
}

struct Workspace {
  float* data;
};

struct WsSlot {
  void* p = nullptr;
  size_t bytes = 0;
  bool captured = false;  // handed out to a capturing stream at least once
};

// `which` selects one of several independent buffers of the stream (0: the
// kernels' own scratch; 1: intermediates of a composite call whose steps use
// buffer 0).
// A caller-fixed scratch buffer that replaces the stream workspace for the
// duration of one call on this thread (kh_quantized_matmul_noalloc).
struct FixedScratch {
  void* p;
  size_t bytes;
};
thread_local const FixedScratch* g_fixed_scratch = nullptr;

bool workspace(hipStream_t stream, size_t floats, Workspace* ws, int* rc, const char* op,
               int which = 0) {
  if (g_fixed_scratch) {
    const size_t need = floats * sizeof(float);
    if (need > g_fixed_scratch->bytes) {
      *rc = fail(KH_ERR_UNSUPPORTED,
                 "[%s] this call needs %zu bytes of scratch; the fixed scratch holds %zu "
                 "(use kh_quantized_matmul, which allocates a workspace)",
                 op, need, g_fixed_scratch->bytes);
      return false;
    }
    *rc = KH_OK;
    ws->data = static_cast<float*>(g_fixed_scratch->p);
    return true;
  }
  static std::mutex mu;
  static std::map<std::tuple<int, hipStream_t, int>, WsSlot> pool;
  int dev = 0;
  (void)hipGetDevice(&dev);
  hipStreamCaptureStatus cs = hipStreamCaptureStatusNone;
  hipError_t e = hipStreamIsCapturing(stream, &cs);
  if (e != hipSuccess) {
    *rc = hip_fail(op, e);
    return false;
  }
  const bool capturing = cs != hipStreamCaptureStatusNone;
  std::lock_guard<std::mutex> lock(mu);
  WsSlot& slot = pool[{dev, stream, which}];
  const size_t bytes = floats * sizeof(float);
  if (slot.bytes < bytes) {
    if (slot.p) {
      if (capturing || slot.captured) {
        retired().push_back(slot.p);
      } else {
        e = hipStreamSynchronize(stream);
        if (e == hipSuccess) e = hipFree(slot.p);
      }
    }
    slot = WsSlot{};
    void* p = nullptr;
    const size_t want = bytes < (size_t(4) << 20) ? (size_t(4) << 20) : bytes;
    if (e == hipSuccess) {
      // under capture the allocation runs in relaxed capture mode
      hipStreamCaptureMode mode = hipStreamCaptureModeRelaxed;
      if (capturing) (void)hipThreadExchangeStreamCaptureMode(&mode);
      e = hipMalloc(&p, want);
      if (capturing) (void)hipThreadExchangeStreamCaptureMode(&mode);
    }
    if (e != hipSuccess) {
      *rc = hip_fail(op, e);
      return false;
    }
    slot.p = p;
    slot.bytes = want;
  }
  slot.captured |= capturing;
  *rc = KH_OK;
  ws->data = static_cast<float*>(slot.p);
  return true;
}

bool aligned16(const void* p) { return (reinterpret_cast<uintptr_t>(p) & 15u) == 0; }

}  // namespace

extern "C" {

const char* kh_last_error(void) { return g_last_error.c_str(); }

const char* kh_version(void) { return "kiln-hip 0.1.0 (gfx950)"; }

namespace {

// Validation of one quantized_matmul call (ops.rs:359-388 argument rules);
// on success *a describes the call, *empty says there is nothing to compute.
// The device check is the caller's, after every part has been validated.
int prepare_qmm(const char* op, kh_array* res, const kh_array* x, const kh_array* w,
                const kh_array* scales, const kh_array* biases, bool transpose,
                kh_optional_int group_size, kh_optional_int bits_opt, const char* mode,
                kh_stream stream, kh::QmvArgs* a, bool* empty) {
  int gs, bits, rc;
  if ((rc = check_quant(op, group_size, bits_opt, mode, &gs, &bits))) return rc;
  if ((rc = check_array(x, op, "x"))) return rc;
  if (!is_float(x->dtype))
    return fail(KH_ERR_INVALID_ARGUMENT, "[%s] x must be float16/bfloat16/float32, got %s", op, dtype_name(x->dtype));
  if (x->ndim < 1) return fail(KH_ERR_INVALID_ARGUMENT, "[%s] x must have ndim >= 1", op);
  int64_t rows, cols;
  if ((rc = check_packed(op, w, scales, biases, gs, bits, &rows, &cols))) return rc;
  if (w->ndim != 2)
    return fail(KH_ERR_UNSUPPORTED, "[%s] batched w %s is not supported (2-D weights only)", op,
                shape_str(w).c_str());
  const int64_t K = x->shape[x->ndim - 1];
  const int64_t wK = transpose ? cols : w->shape[0];
  const int64_t N = transpose ? w->shape[0] : cols;
  if (wK != K)
    return fail(KH_ERR_INVALID_ARGUMENT,
                "[%s] x %s has %lld input features but w %s (transpose=%s) expects %lld", op,
                shape_str(x).c_str(), (long long)K, shape_str(w).c_str(), transpose ? "true" : "false",
                (long long)wK);
  kh_array want = *x;
  want.shape[want.ndim - 1] = N;
  if ((rc = check_result(op, res, want))) return rc;
  const int64_t M = K ? numel(x) / K : numel(res) / (N ? N : 1);
  if (M > INT32_MAX || N > INT32_MAX || K > INT32_MAX)
    return fail(KH_ERR_UNSUPPORTED, "[%s] dimensions beyond 2^31 are not supported", op);
  *empty = M == 0 || N == 0;
  if (*empty) return KH_OK;
  *a = kh::QmvArgs{x->data, x->dtype, w->data, scales->data, biases->data, scales->dtype, res->data,
                   res->dtype, (int)M, (int)N, (int)K, gs, bits, static_cast<hipStream_t>(stream)};
  return KH_OK;
}

// The fast kernels take transpose=true, 16-bit x and scales, 16-byte aligned x and w.
bool fast_path(const kh::QmvArgs& a, bool transpose) {
  return a.K > 0 && transpose && a.xdt != KH_FLOAT32 && a.sdt != KH_FLOAT32 && aligned16(a.x) &&
         aligned16(a.w);
}

constexpr int kSkinnyMinM = 5;         // smallest M the skinny MFMA kernel takes over from the GEMV (measured)
constexpr int kSkinnyMinWaves = 1024;  // narrower skinny launches leave the GEMV the M it serves (measured)
bool skinny_path(const kh::QmvArgs& a) {
  if (a.M < kSkinnyMinM || !kh::skinny_supported(a.M, a.N, a.K, a.bits, a.gs)) return false;
  // Narrow shapes (k/v 1024x4096: 64 workgroups, 512 waves) fill the chip
  // better through the decode GEMV up to its M limit (7.4 -> 6.3 us at
  // M = 8); a rule on N and K, so rows stay M-invariant within each kernel.
  return !(a.M <= kh::gemv_max_m(a.K, a.bits) && kh::gemv_fits(a.M, a.N, a.K, a.bits, a.gs) &&
           kh::skinny_waves(a.N, a.K) < kSkinnyMinWaves);
}
constexpr int kGroupMinRows = 64;  // gather_qmm: fewest rows (pairs * M) for the grouped GEMM
constexpr int kGroupMinAvg = 2;    // ... and fewest rows per possible expert group
bool gemv_path(const kh::QmvArgs& a) {
  return a.M <= kh::gemv_max_m(a.K, a.bits) && kh::gemv_fits(a.M, a.N, a.K, a.bits, a.gs);
}

// True when run_qmm takes the prefill GEMM for this call.
bool gemm_path(const kh::QmvArgs& a, bool transpose) {
  return fast_path(a, transpose) && !skinny_path(a) && !gemv_path(a) && kh::gemm_supported(a.K);
}

// The prefill GEMM for n parts that share x (M, K, bits, x dtype): the
// activations are converted once, then each part's GEMM runs on them.
// Results are those of n separate calls.
int run_gemm_parts(const char* op, const kh::QmvArgs* a, int n) {
  int rc;
  const int64_t M = a[0].M, K = a[0].K;
  std::vector<kh::GemmPlan> plan(n);
  int nsplit_parts = 0;
  size_t part = 0, part_sum = 0;
  for (int i = 0; i < n; ++i) {
    plan[i] = kh::plan_gemm((int)M, a[i].N, (int)K, a[i].bits);
    const size_t b = kh::gemm_partial_bytes(plan[i], (int)M, a[i].N);
    part = std::max(part, b);
    part_sum += (b + 255) / 256 * 256;
    nsplit_parts += plan[i].nsplit > 1;
  }
  // Compatible parts run as one GEMM launch; split-K parts then keep their
  // partial sums side by side and one launch reduces them all (also for two
  // or more split-K parts launched one by one).
  const bool one_launch = n > 1 && kh::gemm_multi_compatible(a, plan.data(), n);
  const bool joint = (one_launch && nsplit_parts >= 1) || (nsplit_parts >= 2 && n <= 4);
  // workspace: float16 activations | per-row scales | split-K partials
  const size_t xb = (size_t)M * K * 2, rb = ((size_t)M * 4 + 255) / 256 * 256;
  Workspace ws;
  if (!workspace(a[0].stream, (xb + rb + (joint ? part_sum : part) + 3) / 4, &ws, &rc, op)) return rc;
  char* base = reinterpret_cast<char*>(ws.data);
  float* rsc = reinterpret_cast<float*>(base + xb);
  hipError_t e = kh::launch_prep_x(a[0], base, rsc);
  std::vector<float*> pbuf(n);
  kh::QmvArgs ra[4];
  kh::GemmPlan rp[4];
  float* rpart[4];
  int nr = 0;
  size_t off = xb + rb;
  for (int i = 0; i < n; ++i) {
    pbuf[i] = reinterpret_cast<float*>(base + (joint ? off : xb + rb));
    if (joint && plan[i].nsplit > 1) {
      ra[nr] = a[i];
      rp[nr] = plan[i];
      rpart[nr++] = pbuf[i];
      off += (kh::gemm_partial_bytes(plan[i], (int)M, a[i].N) + 255) / 256 * 256;
    }
  }
  if (one_launch) {
    if (e == hipSuccess) e = kh::launch_gemm_multi(a, plan.data(), base, rsc, pbuf.data(), n);
  } else {
    for (int i = 0; i < n && e == hipSuccess; ++i)
      e = kh::launch_gemm(a[i], plan[i], base, rsc, pbuf[i], !(joint && plan[i].nsplit > 1));
  }
  if (e == hipSuccess && nr > 0) e = kh::launch_gemm_reduce_multi(ra, rp, rpart, nr);
  return e == hipSuccess ? KH_OK : hip_fail(op, e);
}

// Kernel dispatch of one validated call.
int run_qmm(const char* op, const kh::QmvArgs& a, bool transpose) {
  int rc;
  hipError_t e;
  const hipStream_t st = a.stream;
  const int64_t M = a.M, N = a.N, K = a.K;
  // K == 0 takes the general kernel too: its empty sums write zeros (a
  // kernel, not a memset, so the call stays safe under graph capture).
  if (!fast_path(a, transpose)) {
    e = kh::launch_qmm_generic(a, transpose);
  } else if (skinny_path(a)) {
    e = kh::launch_skinny(a);
  } else if (gemv_path(a)) {
    e = kh::launch_gemv(a);
  } else if (kh::gemm_supported((int)K)) {
    return run_gemm_parts(op, &a, 1);
  } else if (M <= kh::kDecodeMaxM) {
    e = kh::launch_qmv(a);
  } else {
    Workspace ws;
    const size_t bytes = kh::qmm_workspace_bytes((int)M, (int)K);
    if (!workspace(st, (bytes + 3) / 4, &ws, &rc, op)) return rc;
    e = kh::launch_qmm(a, ws.data);
  }
  return e == hipSuccess ? KH_OK : hip_fail(op, e);
}

}  // namespace

int kh_quantized_matmul_plan(int64_t M, int64_t N, int64_t K, int group_size, int bits, int x_dtype,
                             int scales_dtype, char* buf, size_t len) {
  if (!buf || len == 0) return fail(KH_ERR_INVALID_ARGUMENT, "[quantized_matmul_plan] buf is NULL");
  if (M < 0 || N < 0 || K < 0 || M > INT32_MAX || N > INT32_MAX || K > INT32_MAX)
    return fail(KH_ERR_INVALID_ARGUMENT, "[quantized_matmul_plan] M/N/K out of range");
  alignas(16) static const char dummy[16] = {};
  const kh::QmvArgs a{dummy, x_dtype, dummy, dummy, dummy, scales_dtype, nullptr, KH_FLOAT32,
                      (int)M, (int)N, (int)K, group_size, bits, nullptr};
  if (!fast_path(a, true)) {
    snprintf(buf, len, "generic");
  } else if (skinny_path(a)) {
    snprintf(buf, len, "skinny");
  } else if (gemv_path(a)) {
    snprintf(buf, len, "gemv");
  } else if (kh::gemm_supported((int)K)) {
    const kh::GemmPlan p = kh::plan_gemm((int)M, (int)N, (int)K, bits);
    snprintf(buf, len, "gemm mt=%d nsplit=%d tail=%d", p.mt, p.nsplit, p.tail);
  } else {
    snprintf(buf, len, M <= kh::kDecodeMaxM ? "qmv" : "qmm");
  }
  return KH_OK;
}

int kh_quantized_matmul(kh_array* res, const kh_array* x, const kh_array* w,
                        const kh_array* scales, const kh_array* biases, bool transpose,
                        kh_optional_int group_size, kh_optional_int bits_opt, const char* mode,
                        kh_stream stream) {
  const char* op = "quantized_matmul";
  kh::QmvArgs a;
  bool empty = false;
  int rc = prepare_qmm(op, res, x, w, scales, biases, transpose, group_size, bits_opt, mode, stream, &a,
                       &empty);
  if (rc || empty) return rc;
  if ((rc = check_device(op))) return rc;
  return run_qmm(op, a, transpose);
}

static __device__ __align__(256) unsigned char scratch[size_t(64) << 20];

namespace {

// Scratch of kh_quantized_matmul_noalloc (`scratch` above): one array per device, allocated by
// the runtime when the code object is loaded and held until the process
// ends. Host code never uses the name `scratch` as an address: it is a
// host-side stand-in. The device address comes from hipGetSymbolAddress, once
// per device (with that device current), and is kept in g_scratch_ptr.
constexpr size_t kNoAllocScratchBytes = size_t(64) << 20;

constexpr int kMaxDevices = 64;
void* g_scratch_ptr[kMaxDevices] = {};

int scratch_for_device(const char* op, void** out) {
  static std::mutex mu;
  int dev = 0;
  hipError_t e = hipGetDevice(&dev);
  if (e != hipSuccess) return hip_fail(op, e);
  if (dev < 0 || dev >= kMaxDevices) return fail(KH_ERR_UNSUPPORTED, "[%s] device %d beyond %d", op, dev, kMaxDevices);
  std::lock_guard<std::mutex> lock(mu);
  if (!g_scratch_ptr[dev]) {
    void* p = nullptr;
    e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
    if (e != hipSuccess) return hip_fail(op, e);
    if (!p) return fail(KH_ERR_DEVICE, "[%s] no device address for the scratch array", op);
    g_scratch_ptr[dev] = p;
  }
  *out = g_scratch_ptr[dev];
  return KH_OK;
}
static_assert(sizeof(scratch) == kNoAllocScratchBytes, "scratch size");

}  // namespace

int kh_quantized_matmul_noalloc(kh_array* res, const kh_array* x, const kh_array* w,
                                const kh_array* scales, const kh_array* biases, bool transpose,
                                kh_optional_int group_size, kh_optional_int bits_opt, const char* mode,
                                kh_stream stream) {
  const char* op = "quantized_matmul_noalloc";
  kh::QmvArgs a;
  bool empty = false;
  int rc = prepare_qmm(op, res, x, w, scales, biases, transpose, group_size, bits_opt, mode, stream, &a,
                       &empty);
  if (rc || empty) return rc;
  if ((rc = check_device(op))) return rc;
  void* p = nullptr;
  if ((rc = scratch_for_device(op, &p))) return rc;
  const FixedScratch fixed{p, kNoAllocScratchBytes};
  g_fixed_scratch = &fixed;
  rc = run_qmm(op, a, transpose);
  g_fixed_scratch = nullptr;
  return rc;
}

size_t kh_noalloc_scratch_bytes(void) { return kNoAllocScratchBytes; }

namespace {

int prepare_bias(const char* op, const char* name, const kh_array* bias, const kh_array* res,
                 kh::QmvArgs* a);

// n linears on one x (parts with optional biases): one GEMV launch, one
// activation conversion for the prefill GEMMs, or the parts one by one.
int multi(const char* op, int n, kh_array* const* res, const kh_array* x, const kh_array* const* w,
          const kh_array* const* scales, const kh_array* const* biases, const kh_array* const* bias,
          bool transpose, kh_optional_int group_size, kh_optional_int bits, const char* mode,
          kh_stream stream);

}  // namespace

int kh_quantized_matmul_multi(int n, kh_array* const* res, const kh_array* x,
                              const kh_array* const* w, const kh_array* const* scales,
                              const kh_array* const* biases, bool transpose,
                              kh_optional_int group_size, kh_optional_int bits, const char* mode,
                              kh_stream stream) {
  return multi("quantized_matmul_multi", n, res, x, w, scales, biases, nullptr, transpose, group_size, bits,
               mode, stream);
}

namespace {

int multi(const char* op, int n, kh_array* const* res, const kh_array* x, const kh_array* const* w,
          const kh_array* const* scales, const kh_array* const* biases, const kh_array* const* bias,
          bool transpose, kh_optional_int group_size, kh_optional_int bits, const char* mode,
          kh_stream stream) {
  if (n < 1 || !res || !w || !scales || !biases)
    return fail(KH_ERR_INVALID_ARGUMENT, "[%s] n must be >= 1 with non-null part arrays (n=%d)", op, n);
  std::vector<kh::QmvArgs> a(n);
  bool any_empty = false;
  for (int i = 0; i < n; ++i) {
    bool empty = false;
    int rc = prepare_qmm(op, res[i], x, w[i], scales[i], biases[i], transpose, group_size, bits, mode,
                         stream, &a[i], &empty);
    if (rc) return rc;
    if (!empty && bias && (rc = prepare_bias(op, "bias", bias[i], res[i], &a[i]))) return rc;
    any_empty |= empty;
  }
  if (int rc = check_device(op)) return rc;
  if (any_empty) {  // some part has N == 0 (or M == 0): run the others one by one
    for (int i = 0; i < n; ++i) {
      int rc = bias ? kh_linear(res[i], x, w[i], scales[i], biases[i], bias[i], group_size, bits, mode, stream)
                    : kh_quantized_matmul(res[i], x, w[i], scales[i], biases[i], transpose, group_size, bits,
                                          mode, stream);
      if (rc) return rc;
    }
    return KH_OK;
  }
  // Parts taking the same kernel class share launches: the decode GEMV's
  // parts one multi-part launch, the small-batch MFMA kernel's parts one
  // launch, the prefill GEMM's parts one activation conversion. Every part's
  // result is what its own call gives.
  std::vector<kh::QmvArgs> gv, sk, gm, rest;
  for (int i = 0; i < n; ++i) {
    const kh::QmvArgs& p = a[i];
    if (!fast_path(p, transpose) || n > 4)
      rest.push_back(p);
    else if (skinny_path(p) && p.sdt == a[0].sdt)
      sk.push_back(p);
    else if (gemv_path(p) && p.sdt == a[0].sdt && p.odt == a[0].odt)
      gv.push_back(p);
    else if (gemm_path(p, transpose))
      gm.push_back(p);
    else
      rest.push_back(p);
  }
  hipError_t e = hipSuccess;
  if (!gv.empty()) e = gv.size() == 1 ? kh::launch_gemv(gv[0]) : kh::launch_gemv_multi(gv.data(), (int)gv.size());
  if (e == hipSuccess && !sk.empty())
    e = sk.size() == 1 ? kh::launch_skinny(sk[0]) : kh::launch_skinny_multi(sk.data(), (int)sk.size());
  if (e != hipSuccess) return hip_fail(op, e);
  if (!gm.empty())
    if (int rc = run_gemm_parts(op, gm.data(), (int)gm.size())) return rc;
  for (const kh::QmvArgs& p : rest)
    if (int rc = run_qmm(op, p, transpose)) return rc;
  return KH_OK;
}

}  // namespace

namespace {

// MLX's result dtype of an op on two float arrays: equal dtypes keep theirs,
// any other pair (float16 with bfloat16, or with float32) gives float32.
int promote(int a, int b) { return a == b ? a : KH_FLOAT32; }

// Linear::forward's optional bias (crates/kiln-models/src/nn.rs:98-100) for
// a validated call *a: a float [N] vector; the product is an array of MLX's
// result dtype for (x, scales) and res has the dtype of product + bias.
int prepare_bias(const char* op, const char* name, const kh_array* bias, const kh_array* res,
                 kh::QmvArgs* a) {
  if (!bias) return KH_OK;
  int rc;
  if ((rc = check_array(bias, op, name))) return rc;
  if (!is_float(bias->dtype))
    return fail(KH_ERR_INVALID_ARGUMENT, "[%s] %s must be float16/bfloat16/float32, got %s", op, name,
                dtype_name(bias->dtype));
  if (bias->ndim != 1 || bias->shape[0] != a->N)
    return fail(KH_ERR_INVALID_ARGUMENT, "[%s] %s has shape %s, expected (%d)", op, name,
                shape_str(bias).c_str(), a->N);
  const int ydt = promote(a->xdt, a->sdt);
  const int want = promote(ydt, bias->dtype);
  if (res->dtype != want)
    return fail(KH_ERR_INVALID_ARGUMENT,
                "[%s] res is %s but the product (%s) plus %s (%s) is %s", op, dtype_name(res->dtype),
                dtype_name(ydt), name, dtype_name(bias->dtype), dtype_name(want));
  a->bias = bias->data;
  a->bdt = bias->dtype;
  a->ydt = ydt;
  return KH_OK;
}

// The gated MLP's input to its down projection: act(gate(x)) * up(x), the
// linears with optional biases.
int gate_up(const char* op, kh_array* res, const kh_array* x, const kh_array* w_gate,
            const kh_array* scales_gate, const kh_array* biases_gate, const kh_array* bias_gate,
            const kh_array* w_up, const kh_array* scales_up, const kh_array* biases_up,
            const kh_array* bias_up, int activation, kh_optional_int group_size, kh_optional_int bits,
            const char* mode, kh_stream stream) {
  if (activation != KH_ACT_SILU && activation != KH_ACT_GELU_APPROX)
    return fail(KH_ERR_INVALID_ARGUMENT, "[%s] activation %d (supported: silu 0, gelu_approx 1)", op,
                activation);
  kh::QmvArgs g, u;
  bool eg = false, eu = false;
  int rc = prepare_qmm(op, res, x, w_gate, scales_gate, biases_gate, true, group_size, bits, mode, stream,
                       &g, &eg);
  if (rc) return rc;
  if ((rc = prepare_qmm(op, res, x, w_up, scales_up, biases_up, true, group_size, bits, mode, stream, &u,
                        &eu)))
    return rc;
  if (eg || eu) return KH_OK;
  if ((rc = prepare_bias(op, "bias_gate", bias_gate, res, &g)) ||
      (rc = prepare_bias(op, "bias_up", bias_up, res, &u)))
    return rc;
  if ((rc = check_device(op))) return rc;
  if (fast_path(g, true) && fast_path(u, true) && gemv_path(g) && !skinny_path(g) && g.sdt == u.sdt) {
    const hipError_t e = kh::launch_gemv_gate_up(g, u, activation);
    return e == hipSuccess ? KH_OK : hip_fail(op, e);
  }
  if (fast_path(g, true) && fast_path(u, true) && skinny_path(g) && g.sdt == u.sdt && kh::skinny_pairable(g)) {
    const hipError_t e = kh::launch_skinny_gate_up(g, u, activation);
    return e == hipSuccess ? KH_OK : hip_fail(op, e);
  }
  // Two split-K GEMMs on one activation conversion, reduced together with
  // the activation (the partials of both stay in the workspace).
  if (gemm_path(g, true) && gemm_path(u, true) && g.sdt == u.sdt) {
    const kh::GemmPlan pg = kh::plan_gemm((int)g.M, g.N, (int)g.K, g.bits);
    const kh::GemmPlan pu = kh::plan_gemm((int)u.M, u.N, (int)u.K, u.bits);
    if (pg.nsplit > 1 && pu.nsplit > 1) {
      const int64_t M = g.M, K = g.K;
      const size_t xb = (size_t)M * K * 2, rb = ((size_t)M * 4 + 255) / 256 * 256;
      const size_t bg = (kh::gemm_partial_bytes(pg, (int)M, g.N) + 255) / 256 * 256;
      const size_t bu = kh::gemm_partial_bytes(pu, (int)M, u.N);
      Workspace ws;
      if (!workspace(g.stream, (xb + rb + bg + bu + 3) / 4, &ws, &rc, op)) return rc;
      char* base = reinterpret_cast<char*>(ws.data);
      float* rsc = reinterpret_cast<float*>(base + xb);
      float* part_g = reinterpret_cast<float*>(base + xb + rb);
      float* part_u = reinterpret_cast<float*>(base + xb + rb + bg);
      g.out = res->data;
      hipError_t e = kh::launch_prep_x(g, base, rsc);
      const kh::QmvArgs gu[2] = {g, u};
      const kh::GemmPlan pgu[2] = {pg, pu};
      float* const parts[2] = {part_g, part_u};
      if (e == hipSuccess) {
        if (kh::gemm_multi_compatible(gu, pgu, 2)) {
          e = kh::launch_gemm_multi(gu, pgu, base, rsc, parts, 2);
        } else {
          e = kh::launch_gemm(g, pg, base, rsc, part_g, false);
          if (e == hipSuccess) e = kh::launch_gemm(u, pu, base, rsc, part_u, false);
        }
      }
      if (e == hipSuccess) e = kh::launch_gemm_reduce_gate_up(g, pg, part_g, u, pu, part_u, activation);
      return e == hipSuccess ? KH_OK : hip_fail(op, e);
    }
  }
  // Composite: gate and up into intermediates of the result dtype (workspace
  // buffer 1; the matmuls use buffer 0), then the activation.
  const size_t esz = dtype_size(res->dtype), count = (size_t)g.M * g.N;
  Workspace ws;
  if (!workspace(g.stream, (2 * count * esz + 255) / 4 + 64, &ws, &rc, op, 1)) return rc;
  char* gbuf = reinterpret_cast<char*>(ws.data);
  char* ubuf = gbuf + (count * esz + 255) / 256 * 256;
  g.out = gbuf;
  u.out = ubuf;
  if (gemm_path(g, true) && gemm_path(u, true)) {
    const kh::QmvArgs gu[2] = {g, u};
    if ((rc = run_gemm_parts(op, gu, 2))) return rc;
  } else {
    if ((rc = run_qmm(op, g, true))) return rc;
    if ((rc = run_qmm(op, u, true))) return rc;
  }
  const hipError_t e =
      kh::launch_act_mul(gbuf, ubuf, res->data, res->dtype, (int64_t)count, activation, g.stream);
  return e == hipSuccess ? KH_OK : hip_fail(op, e);
}

}  // namespace

int kh_quantized_gate_up(kh_array* res, const kh_array* x, const kh_array* w_gate,
                         const kh_array* scales_gate, const kh_array* biases_gate,
                         const kh_array* w_up, const kh_array* scales_up, const kh_array* biases_up,
                         kh_optional_int group_size, kh_optional_int bits, const char* mode,
                         kh_stream stream) {
  return gate_up("quantized_gate_up", res, x, w_gate, scales_gate, biases_gate, nullptr, w_up, scales_up,
                 biases_up, nullptr, KH_ACT_SILU, group_size, bits, mode, stream);
}

int kh_mlp_gate_up(kh_array* res, const kh_array* x, const kh_array* w_gate, const kh_array* scales_gate,
                   const kh_array* biases_gate, const kh_array* bias_gate, const kh_array* w_up,
                   const kh_array* scales_up, const kh_array* biases_up, const kh_array* bias_up,
                   int activation, kh_optional_int group_size, kh_optional_int bits, const char* mode,
                   kh_stream stream) {
  return gate_up("mlp_gate_up", res, x, w_gate, scales_gate, biases_gate, bias_gate, w_up, scales_up,
                 biases_up, bias_up, activation, group_size, bits, mode, stream);
}

int kh_linear(kh_array* res, const kh_array* x, const kh_array* w, const kh_array* scales,
              const kh_array* biases, const kh_array* bias, kh_optional_int group_size,
              kh_optional_int bits, const char* mode, kh_stream stream) {
  const char* op = "linear";
  kh::QmvArgs a;
  bool empty = false;
  int rc = prepare_qmm(op, res, x, w, scales, biases, true, group_size, bits, mode, stream, &a, &empty);
  if (rc || empty) return rc;
  if ((rc = prepare_bias(op, "bias", bias, res, &a))) return rc;
  if ((rc = check_device(op))) return rc;
  return run_qmm(op, a, true);
}

int kh_linear_multi(int n, kh_array* const* res, const kh_array* x, const kh_array* const* w,
                    const kh_array* const* scales, const kh_array* const* biases,
                    const kh_array* const* bias, kh_optional_int group_size, kh_optional_int bits,
                    const char* mode, kh_stream stream) {
  return multi("linear_multi", n, res, x, w, scales, biases, bias, true, group_size, bits, mode, stream);
}

int kh_gather_qmm(kh_array* res, const kh_array* x, const kh_array* w, const kh_array* scales,
                  const kh_array* biases, const kh_array* rhs_indices, bool transpose,
                  kh_optional_int group_size, kh_optional_int bits_opt, const char* mode,
                  bool sorted_indices, kh_stream stream) {
  (void)sorted_indices;  // a scheduling hint; results do not depend on it
  const char* op = "gather_qmm";
  int gs, bits, rc;
  if ((rc = check_quant(op, group_size, bits_opt, mode, &gs, &bits))) return rc;
  if ((rc = check_array(x, op, "x")) || (rc = check_array(rhs_indices, op, "rhs_indices"))) return rc;
  if (!is_float(x->dtype))
    return fail(KH_ERR_INVALID_ARGUMENT, "[%s] x must be float16/bfloat16/float32, got %s", op, dtype_name(x->dtype));
  if (x->ndim < 2) return fail(KH_ERR_INVALID_ARGUMENT, "[%s] x must have ndim >= 2, got %d", op, x->ndim);
  if (rhs_indices->dtype != KH_UINT32 && rhs_indices->dtype != KH_INT32)
    return fail(KH_ERR_INVALID_ARGUMENT, "[%s] rhs_indices must be uint32 or int32, got %s", op,
                dtype_name(rhs_indices->dtype));
  if (!transpose)
    return fail(KH_ERR_UNSUPPORTED, "[%s] transpose=false is not supported (Kiln passes true)", op);
  int64_t rows, cols;
  if ((rc = check_packed(op, w, scales, biases, gs, bits, &rows, &cols))) return rc;
  if (w->ndim != 3)
    return fail(KH_ERR_INVALID_ARGUMENT, "[%s] w must be an expert stack [E, N, K*bits/32], got %s", op,
                shape_str(w).c_str());
  const int64_t E = w->shape[0], N = w->shape[1], K = cols;
  const int64_t M = x->shape[x->ndim - 2];
  if (x->shape[x->ndim - 1] != K)
    return fail(KH_ERR_INVALID_ARGUMENT, "[%s] x %s has %lld input features but w %s expects %lld", op,
                shape_str(x).c_str(), (long long)x->shape[x->ndim - 1], shape_str(w).c_str(), (long long)K);
  // batch = broadcast(x.shape[:-2], rhs_indices.shape), numpy rules
  const int xb = x->ndim - 2, ib = rhs_indices->ndim;
  const int nd = xb > ib ? xb : ib;
  if (nd > 8) return fail(KH_ERR_UNSUPPORTED, "[%s] more than 8 batch dimensions", op);
  kh::GatherArgs g{};
  g.idx = rhs_indices->data;
  g.idx_signed = rhs_indices->dtype == KH_INT32;
  g.E = (int)E;
  g.nd = nd;
  int64_t xstride = M * K, istride = 1, pairs = 1;
  for (int d = nd - 1; d >= 0; --d) {
    const int dx = d - (nd - xb), di = d - (nd - ib);
    const int64_t sx = dx >= 0 ? x->shape[dx] : 1, si = di >= 0 ? rhs_indices->shape[di] : 1;
    if (sx != si && sx != 1 && si != 1)
      return fail(KH_ERR_INVALID_ARGUMENT, "[%s] x %s and rhs_indices %s do not broadcast", op,
                  shape_str(x).c_str(), shape_str(rhs_indices).c_str());
    const int64_t sd = sx == 1 ? si : sx;  // numpy: a size-1 dim takes the other (also 0)
    if (sd > INT32_MAX) return fail(KH_ERR_UNSUPPORTED, "[%s] batch dimension beyond 2^31", op);
    g.shape[d] = (int)sd;
    g.xs[d] = sx == 1 ? 0 : xstride;
    g.is[d] = si == 1 ? 0 : istride;
    if (dx >= 0) xstride *= sx;
    if (di >= 0) istride *= si;
    pairs *= sd;
  }
  g.pairs = pairs;
  kh_array want{};
  want.dtype = res ? res->dtype : 0;
  want.ndim = nd + 2;
  for (int d = 0; d < nd; ++d) want.shape[d] = g.shape[d];
  want.shape[nd] = M;
  want.shape[nd + 1] = N;
  if ((rc = check_result(op, res, want))) return rc;
  if (M > INT32_MAX || N > INT32_MAX || K > INT32_MAX || E > INT32_MAX)
    return fail(KH_ERR_UNSUPPORTED, "[%s] dimensions beyond 2^31 are not supported", op);
  if (pairs == 0 || M == 0 || N == 0) return KH_OK;
  if ((rc = check_device(op))) return rc;
  kh::QmvArgs a{x->data, x->dtype, w->data, scales->data, biases->data, scales->dtype, res->data,
                res->dtype, (int)M, (int)N, (int)K, gs, bits, static_cast<hipStream_t>(stream)};
  hipError_t e;
  const bool fast = fast_path(a, true);
  const bool gemv = fast && gemv_path(a);
  // Grouped GEMM once the expert groups hold a few rows each (a pair-by-pair
  // GEMV streams the expert's weights once per pair), and for every M the
  // GEMV does not take.
  const int64_t groups = std::min<int64_t>(E + 1, pairs), nrows = pairs * M;
  const bool grouped = fast && kh::gemm_supported((int)K) && E <= kh::kGroupMaxE &&
                       (!gemv || (nrows >= kGroupMinRows && nrows >= kGroupMinAvg * groups));
  if (grouped) {
    const kh::GroupPlan gp = kh::plan_group(a, g);
    if (gp.padded > INT32_MAX)
      return fail(KH_ERR_UNSUPPORTED, "[%s] %lld rows after grouping exceed 2^31", op, (long long)gp.padded);
    Workspace ws;
    const size_t bytes = kh::group_workspace_bytes(gp, a, g);
    if (!workspace(a.stream, (bytes + 3) / 4, &ws, &rc, op)) return rc;
    e = kh::launch_gather_grouped(a, g, gp, ws.data);
  } else if (gemv) {
    e = kh::launch_gemv_gather(a, g);
  } else {
    e = kh::launch_gather_generic(a, g);
  }
  return e == hipSuccess ? KH_OK : hip_fail(op, e);
}

// mlx_quantize (mode "affine"): w [..., K] -> codes, scales, biases.
int kh_quantize(kh_array* w_q, kh_array* scales, kh_array* biases, const kh_array* w,
                kh_optional_int group_size, kh_optional_int bits_opt, const char* mode,
                kh_stream stream) {
  const char* op = "quantize";
  int gs, bits, rc;
  if ((rc = check_quant(op, group_size, bits_opt, mode, &gs, &bits))) return rc;
  if ((rc = check_array(w, op, "w")) || (rc = check_array(w_q, op, "w_q")) ||
      (rc = check_array(scales, op, "scales")) || (rc = check_array(biases, op, "biases")))
    return rc;
  if (!is_float(w->dtype))
    return fail(KH_ERR_INVALID_ARGUMENT, "[%s] w must be float16/bfloat16/float32, got %s", op,
                dtype_name(w->dtype));
  if (w->ndim < 2)
    return fail(KH_ERR_INVALID_ARGUMENT, "[%s] w must have ndim >= 2, got %d", op, w->ndim);
  const int64_t K = w->shape[w->ndim - 1];
  if (K % gs != 0)
    return fail(KH_ERR_INVALID_ARGUMENT,
                "[%s] the last dimension of w (%lld) must be divisible by group_size %d", op,
                (long long)K, gs);
  kh_array want_q = *w, want_s = *w;
  want_q.dtype = KH_UINT32;
  want_q.shape[w->ndim - 1] = K * bits / 32;
  want_s.shape[w->ndim - 1] = K / gs;
  const kh_array* outs[3] = {w_q, scales, biases};
  const kh_array* wants[3] = {&want_q, &want_s, &want_s};
  const char* names[3] = {"w_q", "scales", "biases"};
  for (int o = 0; o < 3; ++o) {
    bool same = outs[o]->dtype == wants[o]->dtype && outs[o]->ndim == wants[o]->ndim;
    for (int i = 0; same && i < wants[o]->ndim; ++i) same = outs[o]->shape[i] == wants[o]->shape[i];
    if (!same)
      return fail(KH_ERR_INVALID_ARGUMENT, "[%s] %s is %s %s, expected %s %s", op, names[o],
                  dtype_name(outs[o]->dtype), shape_str(outs[o]).c_str(),
                  dtype_name(wants[o]->dtype), shape_str(wants[o]).c_str());
  }
  int64_t rows = 1;
  for (int i = 0; i < w->ndim - 1; ++i) rows *= w->shape[i];
  if (rows == 0 || K == 0) return KH_OK;
  if ((rc = check_device(op))) return rc;
  hipError_t e = kh::launch_quantize(w->data, w->dtype, w_q->data, scales->data, biases->data, rows,
                                     K, gs, bits, static_cast<hipStream_t>(stream));
  return e == hipSuccess ? KH_OK : hip_fail(op, e);
}

int kh_dequantize(kh_array* res, const kh_array* w, const kh_array* scales, const kh_array* biases,
                  kh_optional_int group_size, kh_optional_int bits_opt, const char* mode,
                  kh_stream stream) {
  const char* op = "dequantize";
  int gs, bits, rc;
  if ((rc = check_quant(op, group_size, bits_opt, mode, &gs, &bits))) return rc;
  int64_t rows, cols;
  if ((rc = check_packed(op, w, scales, biases, gs, bits, &rows, &cols))) return rc;
  kh_array want = *w;
  want.shape[want.ndim - 1] = cols;
  if ((rc = check_result(op, res, want))) return rc;
  if (rows == 0 || cols == 0) return KH_OK;
  if ((rc = check_device(op))) return rc;
  hipError_t e = kh::launch_dequantize(w->data, scales->data, biases->data, scales->dtype, res->data,
                                       res->dtype, rows, cols, gs, bits, static_cast<hipStream_t>(stream));
  return e == hipSuccess ? KH_OK : hip_fail(op, e);
}

int kh_take(kh_array* res, const kh_array* a, const kh_array* indices, kh_stream stream) {
  const char* op = "take";
  int rc;
  if ((rc = check_array(a, op, "a")) || (rc = check_array(indices, op, "indices")) ||
      (rc = check_array(res, op, "res")))
    return rc;
  if (a->ndim < 1) return fail(KH_ERR_INVALID_ARGUMENT, "[%s] cannot take along axis 0 of a scalar", op);
  if (indices->dtype != KH_UINT32 && indices->dtype != KH_INT32)
    return fail(KH_ERR_INVALID_ARGUMENT, "[%s] indices must be uint32 or int32, got %s", op, dtype_name(indices->dtype));
  if (indices->ndim + a->ndim - 1 > KH_MAX_NDIM)
    return fail(KH_ERR_INVALID_ARGUMENT, "[%s] result rank exceeds %d", op, KH_MAX_NDIM);
  kh_array want{};
  want.dtype = a->dtype;
  want.ndim = indices->ndim + a->ndim - 1;
  for (int i = 0; i < indices->ndim; ++i) want.shape[i] = indices->shape[i];
  for (int i = 1; i < a->ndim; ++i) want.shape[indices->ndim + i - 1] = a->shape[i];
  if (res->dtype != a->dtype)
    return fail(KH_ERR_INVALID_ARGUMENT, "[%s] res dtype %s differs from a dtype %s", op,
                dtype_name(res->dtype), dtype_name(a->dtype));
  bool same = res->ndim == want.ndim;
  for (int i = 0; same && i < want.ndim; ++i) same = res->shape[i] == want.shape[i];
  if (!same)
    return fail(KH_ERR_INVALID_ARGUMENT, "[%s] res has shape %s, expected %s", op,
                shape_str(res).c_str(), shape_str(&want).c_str());
  const int64_t T = numel(indices);
  const int64_t V = a->shape[0];
  int64_t row = dtype_size(a->dtype);
  for (int i = 1; i < a->ndim; ++i) row *= a->shape[i];
  if (T == 0 || row == 0) return KH_OK;
  if (V == 0) return fail(KH_ERR_INVALID_ARGUMENT, "[%s] cannot take from an empty axis", op);
  if ((rc = check_device(op))) return rc;
  hipError_t e = kh::launch_take(a->data, V, row, indices->data, indices->dtype == KH_INT32, T,
                                 res->data, static_cast<hipStream_t>(stream));
  return e == hipSuccess ? KH_OK : hip_fail(op, e);
}

int kh_add(kh_array* res, const kh_array* a, const kh_array* b, kh_stream stream) {
  const char* op = "add";
  int rc;
  if ((rc = check_array(a, op, "a")) || (rc = check_array(b, op, "b"))) return rc;
  if (!is_float(a->dtype) || !is_float(b->dtype))
    return fail(KH_ERR_INVALID_ARGUMENT, "[%s] operands must be float16/bfloat16/float32, got %s and %s",
                op, dtype_name(a->dtype), dtype_name(b->dtype));
  // numpy broadcasting, dimensions aligned from the right
  const int nd = a->ndim > b->ndim ? a->ndim : b->ndim;
  kh_array want{};
  want.dtype = res ? res->dtype : 0;
  want.ndim = nd;
  kh::AddShape sh{};
  sh.nd = nd;
  int64_t sa = 1, sb = 1;
  bool suffix = b->ndim <= a->ndim;  // b.shape == a.shape[-b.ndim:]: the plain kernel
  for (int d = nd - 1; d >= 0; --d) {
    const int da = d - (nd - a->ndim), db = d - (nd - b->ndim);
    const int64_t ea = da >= 0 ? a->shape[da] : 1, eb = db >= 0 ? b->shape[db] : 1;
    if (ea != eb && ea != 1 && eb != 1)
      return fail(KH_ERR_INVALID_ARGUMENT, "[%s] cannot broadcast %s with %s", op, shape_str(a).c_str(),
                  shape_str(b).c_str());
    const int64_t e = ea == 1 ? eb : ea;
    want.shape[d] = e;
    sh.shape[d] = e;
    sh.as[d] = ea == 1 ? 0 : sa;
    sh.bs[d] = eb == 1 ? 0 : sb;
    if (db >= 0 && eb != ea) suffix = false;
    if (da >= 0) sa *= ea;
    if (db >= 0) sb *= eb;
  }
  if ((rc = check_result(op, res, want))) return rc;
  const int64_t n = numel(&want), nb = numel(b);
  if (n == 0) return KH_OK;
  if ((rc = check_device(op))) return rc;
  const hipStream_t st = static_cast<hipStream_t>(stream);
  const hipError_t e = suffix ? kh::launch_add(a->data, a->dtype, b->data, b->dtype, res->data, res->dtype, n,
                                               nb, st)
                              : kh::launch_add_bcast(a->data, a->dtype, b->data, b->dtype, res->data,
                                                     res->dtype, n, sh, st);
  return e == hipSuccess ? KH_OK : hip_fail(op, e);
}

int kh_quantized_embedding(kh_array* res, const kh_array* ids, const kh_array* w,
                           const kh_array* scales, const kh_array* biases,
                           kh_optional_int group_size, kh_optional_int bits_opt, const char* mode,
                           kh_stream stream) {
  const char* op = "quantized_embedding";
  int gs, bits, rc;
  if ((rc = check_quant(op, group_size, bits_opt, mode, &gs, &bits))) return rc;
  if ((rc = check_array(ids, op, "ids"))) return rc;
  if (ids->dtype != KH_UINT32 && ids->dtype != KH_INT32)
    return fail(KH_ERR_INVALID_ARGUMENT, "[%s] ids must be uint32 or int32, got %s", op, dtype_name(ids->dtype));
  int64_t rows, cols;
  if ((rc = check_packed(op, w, scales, biases, gs, bits, &rows, &cols))) return rc;
  if (w->ndim != 2)
    return fail(KH_ERR_INVALID_ARGUMENT, "[%s] embedding table must be 2-D, got %s", op, shape_str(w).c_str());
  if (ids->ndim + 1 > KH_MAX_NDIM)
    return fail(KH_ERR_INVALID_ARGUMENT, "[%s] result rank exceeds %d", op, KH_MAX_NDIM);
  kh_array want{};
  want.ndim = ids->ndim + 1;
  for (int i = 0; i < ids->ndim; ++i) want.shape[i] = ids->shape[i];
  want.shape[ids->ndim] = cols;
  if ((rc = check_result(op, res, want))) return rc;
  const int64_t T = numel(ids);
  if (T == 0 || cols == 0) return KH_OK;
  if (w->shape[0] == 0) return fail(KH_ERR_INVALID_ARGUMENT, "[%s] empty embedding table", op);
  if ((rc = check_device(op))) return rc;
  hipError_t e = kh::launch_embedding(ids->data, ids->dtype == KH_INT32, T, w->data, scales->data,
                                      biases->data, scales->dtype, res->data, res->dtype,
                                      w->shape[0], cols, gs, bits, static_cast<hipStream_t>(stream));
  return e == hipSuccess ? KH_OK : hip_fail(op, e);
}

}  // extern "C"
