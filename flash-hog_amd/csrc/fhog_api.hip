// C-ABI entry points: argument validation and dispatch to the templated
// launchers. Error reporting follows the reference's FFI handler
// (flash_hog/csrc/tk_bwdbwd/ffi.cu:35-39, 74-76): invalid shapes are rejected
// before anything is enqueued, launch failures are reported with the runtime's
// message. Messages are kept per thread; there is no other global state.
#include <stdint.h>
#include <stdio.h>
#include <stdarg.h>
#include <string.h>

#include <atomic>
#include <mutex>

#include "flash_hog.h"
#include "fhog_params.h"

namespace {

thread_local char g_last_error[512] = "";

int fail(int status, const char* fmt, ...) {
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(g_last_error, sizeof(g_last_error), fmt, ap);
  va_end(ap);
  return status;
}

int ok() {
  g_last_error[0] = '\0';
  return FHOG_OK;
}

// Tensors are read with 16-byte vector loads; fp32 row statistics with scalar loads.
bool aligned(const void* p, uintptr_t bytes) {
  return p != nullptr && (reinterpret_cast<uintptr_t>(p) & (bytes - 1)) == 0;
}

struct Shape {
  int batch, n_q, n_k, heads, kv_heads, head_dim, dtype, causal;
  float scale;
  // Key j is visible to query i iff j <= i + coff (causal kernels only).
  int coff() const { return causal == FHOG_CAUSAL_BOTTOM_RIGHT ? n_k - n_q : 0; }
};

int check_shape(const Shape& s, const char* who) {
  if (!(s.scale == s.scale) || s.scale - s.scale != 0.0f)
    return fail(FHOG_ERR_INVALID_ARGUMENT, "%s: scale must be finite", who);
  // With scale 0 every logit is 0 and masked ones are -inf * 0; the kernels
  // also divide by the scale. Any other finite scale, negative included, works.
  if (s.scale == 0.0f) return fail(FHOG_ERR_UNSUPPORTED, "%s: scale must be nonzero", who);
  if (s.causal != FHOG_CAUSAL_NONE && s.causal != FHOG_CAUSAL_TOP_LEFT && s.causal != FHOG_CAUSAL_BOTTOM_RIGHT)
    return fail(FHOG_ERR_INVALID_ARGUMENT, "%s: causal must be 0 (none), 1 (top-left) or 2 (bottom-right), got %d",
                who, s.causal);
  if (s.batch < 1 || s.n_q < 1 || s.n_k < 1 || s.heads < 1 || s.kv_heads < 1)
    return fail(FHOG_ERR_INVALID_ARGUMENT, "%s: sizes must be >= 1 (batch=%d n_q=%d n_k=%d heads=%d kv_heads=%d)",
                who, s.batch, s.n_q, s.n_k, s.heads, s.kv_heads);
  if (s.dtype != FHOG_DTYPE_F32 && s.dtype != FHOG_DTYPE_F16 && s.dtype != FHOG_DTYPE_BF16)
    return fail(FHOG_ERR_INVALID_ARGUMENT, "%s: unknown dtype %d", who, s.dtype);
  if (s.head_dim < 1)
    return fail(FHOG_ERR_INVALID_ARGUMENT, "%s: head_dim must be >= 1, got %d", who, s.head_dim);
  if (s.heads % s.kv_heads != 0)
    return fail(FHOG_ERR_INVALID_ARGUMENT, "%s: heads (%d) must be a multiple of kv_heads (%d)", who, s.heads,
                s.kv_heads);
  if (s.dtype == FHOG_DTYPE_F32 && s.head_dim != 64 && s.head_dim != 128)
    return fail(FHOG_ERR_UNSUPPORTED, "%s: fp32 head_dim must be 64 or 128, got %d", who, s.head_dim);
  if (s.head_dim != 64 && s.head_dim != 128 && s.head_dim != 256)
    return fail(FHOG_ERR_UNSUPPORTED, "%s: head_dim must be 64, 128 or 256, got %d", who, s.head_dim);
  const long long rows = (long long)s.batch * s.heads * (s.n_q > s.n_k ? s.n_q : s.n_k);
  if (rows * s.head_dim >= (1ll << 40) || (long long)s.batch * s.heads * ((s.n_q > s.n_k ? s.n_q : s.n_k) + 31) / 32 >= (1ll << 31))
    return fail(FHOG_ERR_INVALID_ARGUMENT, "%s: problem too large", who);
  return FHOG_OK;
}

int check_ptrs(const char* who, std::initializer_list<std::pair<const char*, const void*>> tensors,
               std::initializer_list<std::pair<const char*, const void*>> row_stats) {
  for (const auto& p : tensors)
    if (!aligned(p.second, 16))
      return fail(FHOG_ERR_INVALID_ARGUMENT, "%s: %s is null or not 16-byte aligned", who, p.first);
  for (const auto& p : row_stats)
    if (!aligned(p.second, 4))
      return fail(FHOG_ERR_INVALID_ARGUMENT, "%s: %s is null or not 4-byte aligned", who, p.first);
  return FHOG_OK;
}

int launch_status(hipError_t e, const char* who) {
  if (e != hipSuccess) return fail(FHOG_ERR_LAUNCH, "%s: %s", who, hipGetErrorString(e));
  return ok();
}

// Calls f.template operator()<T, D, CAUSAL>() for the runtime (dtype, head_dim, causal).
template <typename F>
hipError_t dispatch(int dtype, int head_dim, bool causal, F&& f) {
#define FHOG_CASE(T, D)                                          \
  return causal ? f.template operator()<T, D, true>() : f.template operator()<T, D, false>();
  if (dtype == FHOG_DTYPE_BF16) {
    if (head_dim == 64) { FHOG_CASE(__bf16, 64) }
    if (head_dim == 128) { FHOG_CASE(__bf16, 128) }
    FHOG_CASE(__bf16, 256)
  }
  if (dtype == FHOG_DTYPE_F16) {
    if (head_dim == 64) { FHOG_CASE(_Float16, 64) }
    if (head_dim == 128) { FHOG_CASE(_Float16, 128) }
    FHOG_CASE(_Float16, 256)
  }
  if (head_dim == 64) { FHOG_CASE(float, 64) }
  FHOG_CASE(float, 128)
#undef FHOG_CASE
}

}  // namespace

extern "C" {

int fhog_abi_version(void) { return 103; }

const char* fhog_status_string(int status) {
  switch (status) {
    case FHOG_OK: return "ok";
    case FHOG_ERR_INVALID_ARGUMENT: return "invalid argument";
    case FHOG_ERR_UNSUPPORTED: return "unsupported";
    case FHOG_ERR_LAUNCH: return "kernel launch failed";
    default: return "unknown status";
  }
}

const char* fhog_last_error(void) { return g_last_error; }

int fhog_attention_supported(int device, int batch, int n_q, int n_k, int heads, int kv_heads, int head_dim,
                             int dtype, int causal, float scale) {
  static const char* who = "fhog_attention_supported";
  const Shape s{batch, n_q, n_k, heads, kv_heads, head_dim, dtype, causal, scale};
  if (int st = check_shape(s, who)) return st;
  if (device >= 0) {
    hipDeviceProp_t prop;
    const hipError_t e = hipGetDeviceProperties(&prop, device);
    if (e != hipSuccess)
      return fail(FHOG_ERR_UNSUPPORTED, "%s: no HIP device %d (%s)", who, device, hipGetErrorString(e));
    if (strncmp(prop.gcnArchName, "gfx950", 6) != 0)
      return fail(FHOG_ERR_UNSUPPORTED, "%s: device %d is %s; the kernels are built for gfx950", who, device,
                  prop.gcnArchName);
  }
  return ok();
}

size_t fhog_row_stat_bytes(int batch, int heads, int n_q) {
  if (batch < 1 || heads < 1 || n_q < 1) return 0;
  return (size_t)batch * heads * n_q * sizeof(float);
}

int fhog_attention_fwd(fhog_stream_t stream, const void* q, const void* k, const void* v, void* o, float* lse,
                       int batch, int n_q, int n_k, int heads, int kv_heads, int head_dim, int dtype, int causal,
                       float scale) {
  static const char* who = "fhog_attention_fwd";
  const Shape s{batch, n_q, n_k, heads, kv_heads, head_dim, dtype, causal, scale};
  if (int st = check_shape(s, who)) return st;
  if (int st = check_ptrs(who, {{"q", q}, {"k", k}, {"v", v}, {"o", o}}, {{"lse", lse}})) return st;
  auto run = [&]<typename T, int D, bool C>() {
    fhog::FwdParams<T> p{(const T*)q, (const T*)k, (const T*)v, (T*)o, lse, batch, n_q, n_k, heads, kv_heads,
                         s.coff(), scale};
    return fhog::launch_fwd<T, D, C>(p, (hipStream_t)stream);
  };
  return launch_status(dispatch(dtype, head_dim, causal != 0, run), who);
}

int fhog_attention_bwd(fhog_stream_t stream, const void* q, const void* k, const void* v, const void* o,
                       const void* dout, const float* lse, void* dq, void* dk, void* dv, float* delta, int batch,
                       int n_q, int n_k, int heads, int kv_heads, int head_dim, int dtype, int causal, float scale) {
  static const char* who = "fhog_attention_bwd";
  const Shape s{batch, n_q, n_k, heads, kv_heads, head_dim, dtype, causal, scale};
  if (int st = check_shape(s, who)) return st;
  if (int st = check_ptrs(who, {{"q", q}, {"k", k}, {"v", v}, {"o", o}, {"dout", dout}, {"dq", dq}, {"dk", dk},
                                {"dv", dv}},
                           {{"lse", lse}, {"delta", delta}}))
    return st;
  auto run = [&]<typename T, int D, bool C>() {
    fhog::BwdParams<T> p{(const T*)q, (const T*)k, (const T*)v, (const T*)o, (const T*)dout, lse,
                         (T*)dq, (T*)dk, (T*)dv, delta, batch, n_q, n_k, heads, kv_heads, s.coff(), scale};
    return fhog::launch_bwd<T, D, C>(p, (hipStream_t)stream);
  };
  return launch_status(dispatch(dtype, head_dim, causal != 0, run), who);
}

namespace {

int bwdbwd_impl(const char* who, int stages, fhog_stream_t stream, const void* q, const void* k, const void* v,
                const void* o, const void* dout, const void* ddq, const void* ddk, const void* ddv,
                const float* lse, void* dq2, void* dk2, void* dv2, void* ddo, float* delta, float* ddelta,
                float* bstat, int batch, int n_q, int n_k, int heads, int kv_heads, int head_dim, int dtype,
                int causal, float scale) {
  const Shape s{batch, n_q, n_k, heads, kv_heads, head_dim, dtype, causal, scale};
  if (int st = check_shape(s, who)) return st;
  if (int st = check_ptrs(who, {{"q", q}, {"k", k}, {"v", v}, {"dout", dout}, {"ddq", ddq}, {"ddk", ddk},
                                {"ddv", ddv}},
                           {{"lse", lse}, {"delta", delta}, {"ddelta", ddelta}, {"bstat", bstat}}))
    return st;
  if (stages & 1)
    if (int st = check_ptrs(who, {{"o", o}, {"dq2", dq2}, {"ddo", ddo}}, {})) return st;
  if (stages & 2)
    if (int st = check_ptrs(who, {{"dk2", dk2}, {"dv2", dv2}}, {})) return st;
  auto run = [&]<typename T, int D, bool C>() {
    fhog::BwdBwdParams<T> p{(const T*)q,   (const T*)k,   (const T*)v,   (const T*)o, (const T*)dout,
                            (const T*)ddq, (const T*)ddk, (const T*)ddv, lse,         (T*)dq2,
                            (T*)dk2,       (T*)dv2,       (T*)ddo,       delta,       ddelta,
                            bstat,         batch,         n_q,           n_k,         heads,
                            kv_heads,      s.coff(),      scale};
    return fhog::launch_bwdbwd<T, D, C>(p, (hipStream_t)stream, stages);
  };
  return launch_status(dispatch(dtype, head_dim, causal != 0, run), who);
}

// ---------------------------------------------------------------------------
// Row statistics of fhog_attention_bwdbwd_noalloc: D, dD and B of up to
// kScratchRows (batch, head, query) rows each, in one file-scope device array
// (12 MiB per device, held until the process ends). Every call on a device
// uses that device's copy; the kernels write every row they later read, so
// nothing needs clearing between calls, but two calls that overlap on one
// device race on it.
// ---------------------------------------------------------------------------
constexpr long long kScratchRows = 1ll << 20;
static __device__ __align__(256) float scratch[3 * kScratchRows];

// Device address of `scratch` per device, looked up once per device (with
// that device current) and kept: in host code the array's name is not a
// device address.
constexpr int kMaxDevices = 64;
std::atomic<float*> g_scratch[kMaxDevices];
std::mutex g_scratch_mu;

int scratch_address(const char* who, hipStream_t stream, float** out) {
  int dev = -1;
  hipError_t e = stream ? hipStreamGetDevice(stream, &dev) : hipGetDevice(&dev);
  if (e != hipSuccess) return fail(FHOG_ERR_LAUNCH, "%s: cannot find the stream's device: %s", who, hipGetErrorString(e));
  if (dev < 0 || dev >= kMaxDevices) return fail(FHOG_ERR_UNSUPPORTED, "%s: device %d out of range", who, dev);
  float* ptr = g_scratch[dev].load(std::memory_order_acquire);
  if (ptr == nullptr) {
    std::lock_guard<std::mutex> lock(g_scratch_mu);
    ptr = g_scratch[dev].load(std::memory_order_relaxed);
    if (ptr == nullptr) {
      int cur = -1;
      if ((e = hipGetDevice(&cur)) == hipSuccess && cur != dev) e = hipSetDevice(dev);
      void* addr = nullptr;
      if (e == hipSuccess) e = hipGetSymbolAddress(&addr, HIP_SYMBOL(scratch));
      if (cur >= 0 && cur != dev) {
        const hipError_t back = hipSetDevice(cur);
        if (e == hipSuccess) e = back;
      }
      if (e != hipSuccess || addr == nullptr)
        return fail(FHOG_ERR_LAUNCH, "%s: no address for the static scratch on device %d: %s", who, dev,
                    hipGetErrorString(e));
      ptr = static_cast<float*>(addr);
      g_scratch[dev].store(ptr, std::memory_order_release);
    }
  }
  *out = ptr;
  return FHOG_OK;
}

}  // namespace

int fhog_attention_bwdbwd(fhog_stream_t stream, const void* q, const void* k, const void* v, const void* o,
                          const void* dout, const void* ddq, const void* ddk, const void* ddv, const float* lse,
                          void* dq2, void* dk2, void* dv2, void* ddo, float* delta, float* ddelta, float* bstat,
                          int batch, int n_q, int n_k, int heads, int kv_heads, int head_dim, int dtype, int causal,
                          float scale) {
  return bwdbwd_impl("fhog_attention_bwdbwd", 3, stream, q, k, v, o, dout, ddq, ddk, ddv, lse, dq2, dk2, dv2,
                     ddo, delta, ddelta, bstat, batch, n_q, n_k, heads, kv_heads, head_dim, dtype, causal, scale);
}

int fhog_attention_bwdbwd_stage(fhog_stream_t stream, int stage, const void* q, const void* k, const void* v,
                                const void* o, const void* dout, const void* ddq, const void* ddk,
                                const void* ddv, const float* lse, void* dq2, void* dk2, void* dv2, void* ddo,
                                float* delta, float* ddelta, float* bstat, int batch, int n_q, int n_k,
                                int heads, int kv_heads, int head_dim, int dtype, int causal, float scale) {
  static const char* who = "fhog_attention_bwdbwd_stage";
  if (stage != 1 && stage != 2) return fail(FHOG_ERR_INVALID_ARGUMENT, "%s: stage must be 1 or 2, got %d", who, stage);
  return bwdbwd_impl(who, stage, stream, q, k, v, o, dout, ddq, ddk, ddv, lse, dq2, dk2, dv2, ddo, delta,
                     ddelta, bstat, batch, n_q, n_k, heads, kv_heads, head_dim, dtype, causal, scale);
}

int fhog_attention_bwdbwd_noalloc(fhog_stream_t stream, const void* q, const void* k, const void* v,
                                  const void* o, const void* dout, const void* ddq, const void* ddk,
                                  const void* ddv, const float* lse, void* dq2, void* dk2, void* dv2, void* ddo,
                                  int batch, int n_q, int n_k, int heads, int kv_heads, int head_dim, int dtype,
                                  int causal, float scale) {
  static const char* who = "fhog_attention_bwdbwd_noalloc";
  const Shape s{batch, n_q, n_k, heads, kv_heads, head_dim, dtype, causal, scale};
  if (int st = check_shape(s, who)) return st;
  if (int st = check_ptrs(who, {{"q", q}, {"k", k}, {"v", v}, {"o", o}, {"dout", dout}, {"ddq", ddq},
                                {"ddk", ddk}, {"ddv", ddv}, {"dq2", dq2}, {"dk2", dk2}, {"dv2", dv2},
                                {"ddo", ddo}},
                           {{"lse", lse}}))
    return st;
  const long long rows = (long long)batch * heads * n_q;
  if (rows > kScratchRows)
    return fail(FHOG_ERR_UNSUPPORTED,
                "%s: batch * heads * n_q = %lld exceeds the static scratch's %lld rows; use fhog_attention_bwdbwd "
                "with caller-owned row statistics",
                who, rows, kScratchRows);
  float* ws = nullptr;
  if (int st = scratch_address(who, (hipStream_t)stream, &ws)) return st;
  return bwdbwd_impl(who, 3, stream, q, k, v, o, dout, ddq, ddk, ddv, lse, dq2, dk2, dv2, ddo, ws,
                     ws + kScratchRows, ws + 2 * kScratchRows, batch, n_q, n_k, heads, kv_heads, head_dim, dtype,
                     causal, scale);
}

}  // extern "C"
