// api.cpp -- libhipq's C ABI: errors, runtime wrappers, trace spans and the
// validated op entry points.  Kernels live in the .hip translation units.
#include <stdarg.h>
#include <stdio.h>
#include <string.h>

#include <algorithm>
#include <map>
#include <atomic>
#include <mutex>
#include <string>
#include <vector>

#include "internal.hpp"

namespace hq {

static thread_local char g_err[512] = "";
static std::atomic<hipStream_t> g_current{nullptr};  // hq_stream_set_current, from any thread

int fail(int code, const char *call, const char *fmt, ...) {
  char msg[400];
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(msg, sizeof msg, fmt, ap);
  va_end(ap);
  snprintf(g_err, sizeof g_err, "hipq: %s: %s (code %d)", call, msg, code);
  return code;
}

int check(hipError_t e, const char *call) {
  if (e == hipSuccess) return HQ_OK;
  return fail((int)e, call, "%s", hipGetErrorString(e));
}

hipStream_t resolve(hq_stream_t s) { return s ? (hipStream_t)s : g_current.load(); }

// Library-owned workspace for calls made with ws == NULL, one buffer per (device, stream):
// work on one stream runs in order, so a stream's buffer is never used by two kernels at
// once, while calls on different streams get different buffers.  A buffer that has to grow
// is replaced, and the old one is retired, not freed: a kernel enqueued from another thread,
// or a graph captured earlier, may still hold its address.  Retired buffers are freed by
// hq_workspace_release() (after a device synchronisation) or at process exit.
static std::mutex g_ws_mu;
static std::map<std::pair<int, hipStream_t>, std::pair<void *, size_t>> g_ws;
struct Retired {
  int dev;
  hipStream_t stream;
  void *p;
};
static std::vector<Retired> g_ws_retired;

int workspace(size_t bytes, hipStream_t stream, void **out, const char *call) {
  int dev = 0;
  if (int rc = check(hipGetDevice(&dev), call)) return rc;
  std::lock_guard<std::mutex> lk(g_ws_mu);
  auto &slot = g_ws[{dev, stream}];
  if (slot.second < bytes) {
    hipStreamCaptureStatus cs = hipStreamCaptureStatusNone;
    if (stream && hipStreamIsCapturing(stream, &cs) == hipSuccess && cs != hipStreamCaptureStatusNone)
      return fail(HQ_EUNSUPPORTED, call,
                  "stream is capturing and the library workspace must grow to %zu bytes: pass a workspace", bytes);
    size_t cap = bytes < (1u << 20) ? (1u << 20) : bytes + bytes / 4;
    void *p = nullptr;
    if (hipMalloc(&p, cap) != hipSuccess) return fail(HQ_ENOMEM, call, "workspace of %zu bytes", cap);
    if (slot.first) g_ws_retired.push_back({dev, stream, slot.first});
    slot = {p, cap};
  }
  *out = slot.first;
  return HQ_OK;
}

int workspace_release() {
  std::lock_guard<std::mutex> lk(g_ws_mu);
  int rc = HQ_OK, cur = 0;
  if (int e = check(hipGetDevice(&cur), "hq_workspace_release")) return e;
  auto drop = [&](int dev, void *p) {
    if (rc) return;
    rc = check(hipSetDevice(dev), "hipSetDevice");
    if (!rc) rc = check(hipDeviceSynchronize(), "hipDeviceSynchronize");
    if (!rc) rc = check(hipFree(p), "hipFree");
  };
  for (auto &r : g_ws_retired) drop(r.dev, r.p);
  for (auto &kv : g_ws)
    if (kv.second.first) drop(kv.first.first, kv.second.first);
  if (!rc) {
    g_ws_retired.clear();
    g_ws.clear();
  }
  (void)hipSetDevice(cur);
  return rc;
}

// Frees the workspace buffers (current and retired, on every device) of a stream that is
// being destroyed, after the stream has drained.
static int workspace_forget_stream(hipStream_t stream) {
  std::lock_guard<std::mutex> lk(g_ws_mu);
  int rc = HQ_OK;
  for (auto it = g_ws.begin(); it != g_ws.end();) {
    if (it->first.second == stream) {
      if (it->second.first && !rc) rc = check(hipFree(it->second.first), "hipFree");
      it = g_ws.erase(it);
    } else {
      ++it;
    }
  }
  for (auto it = g_ws_retired.begin(); it != g_ws_retired.end();) {
    if (it->stream == stream) {
      if (!rc) rc = check(hipFree(it->p), "hipFree");
      it = g_ws_retired.erase(it);
    } else {
      ++it;
    }
  }
  return rc;
}

// ---- allocation-free scratch ----
// hq_matmul_q_noalloc's scratch: a file-scope device array that every GPU the library runs
// on holds until the process ends.  Host code never passes `scratch` itself to a kernel (on
// the host the name is only a stand-in); it uses the device address that
// hipGetSymbolAddress returns, looked up once per device.
static __device__ __align__(256) unsigned char scratch[HQ_NOALLOC_SCRATCH_BYTES];
static std::mutex g_scr_mu;
static std::map<int, void *> g_scr;

static int scratch_ptr(void **out, const char *call) {
  int dev = 0;
  if (int rc = check(hipGetDevice(&dev), call)) return rc;
  std::lock_guard<std::mutex> lk(g_scr_mu);
  auto it = g_scr.find(dev);
  if (it == g_scr.end()) {
    void *p = nullptr;
    if (int rc = check(hipGetSymbolAddress(&p, HIP_SYMBOL(scratch)), "hipGetSymbolAddress")) return rc;
    it = g_scr.emplace(dev, p).first;
  }
  *out = it->second;
  return HQ_OK;
}

// ---- trace spans ----
struct TraceRec {
  int calls = 0;
  double us = 0;
};
static std::mutex g_tr_mu;
static bool g_tracing = false;
static std::vector<std::pair<std::string, std::pair<hipEvent_t, hipEvent_t>>> g_spans;

TraceSpan::TraceSpan(const char *n, hipStream_t s) : name(n), stream(s) {
  if (!g_tracing) return;
  if (hipEventCreate(&ev0) != hipSuccess || hipEventCreate(&ev1) != hipSuccess) {
    ev0 = ev1 = nullptr;
    return;
  }
  (void)hipEventRecord(ev0, stream);
}

TraceSpan::~TraceSpan() {
  if (!ev0) return;
  (void)hipEventRecord(ev1, stream);
  std::lock_guard<std::mutex> lk(g_tr_mu);
  g_spans.push_back({name, {ev0, ev1}});
}

}  // namespace hq

using namespace hq;

// Byte fill: `head` bytes up to 16-byte alignment, n16 16-byte stores, then `tail` bytes.
__global__ void fill_bytes_kernel(unsigned char *dst, size_t head, size_t n16, size_t tail, uint32_t b) {
  const size_t stride = (size_t)gridDim.x * blockDim.x;
  const size_t t0 = (size_t)blockIdx.x * blockDim.x + threadIdx.x;
  uint4 *v = reinterpret_cast<uint4 *>(dst + head);
  for (size_t i = t0; i < n16; i += stride) v[i] = make_uint4(b, b, b, b);
  for (size_t i = t0; i < head; i += stride) dst[i] = (unsigned char)b;
  for (size_t i = t0; i < tail; i += stride) dst[head + n16 * 16 + i] = (unsigned char)b;
}

extern "C" {

const char *hq_last_error(void) { return g_err; }
int hq_version(void) { return 100; }

int hq_ceiling_read(const void *buf, int64_t bytes, int order, int depth, uint32_t *sink, hq_stream_t stream) {
  return launch_ceiling_read(buf, bytes, order, depth, sink, resolve(stream));
}

int hq_ceiling_mix(int mode, int64_t iters, float *sink, hq_stream_t stream) {
  return launch_ceiling_mix(mode, iters, sink, resolve(stream));
}

int hq_ceiling_mfma(int64_t iters, float *sink, int64_t *flops, hq_stream_t stream) {
  if (flops) *flops = ceiling_mfma_flops(iters);
  return launch_ceiling_mfma(iters, sink, resolve(stream));
}

int hq_device_count(int *count) {
  if (!count) return fail(HQ_EINVAL, "hq_device_count", "count is NULL");
  return check(hipGetDeviceCount(count), "hipGetDeviceCount");
}

int hq_set_device(int device) { return check(hipSetDevice(device), "hipSetDevice"); }

int hq_malloc(void **ptr, size_t bytes) {
  if (!ptr) return fail(HQ_EINVAL, "hq_malloc", "ptr is NULL");
  *ptr = nullptr;
  if (bytes == 0) return HQ_OK;
  return check(hipMalloc(ptr, bytes), "hipMalloc");
}

int hq_free(void *ptr) { return ptr ? check(hipFree(ptr), "hipFree") : HQ_OK; }

int hq_memcpy_h2d(void *dst, const void *src, size_t bytes, hq_stream_t s) {
  hipStream_t st = resolve(s);
  if (int rc = check(hipMemcpyAsync(dst, src, bytes, hipMemcpyHostToDevice, st), "hipMemcpyHtoD")) return rc;
  return check(hipStreamSynchronize(st), "hipStreamSynchronize");
}

int hq_memcpy_d2h(void *dst, const void *src, size_t bytes, hq_stream_t s) {
  hipStream_t st = resolve(s);
  if (int rc = check(hipMemcpyAsync(dst, src, bytes, hipMemcpyDeviceToHost, st), "hipMemcpyDtoH")) return rc;
  return check(hipStreamSynchronize(st), "hipStreamSynchronize");
}

int hq_memcpy_d2d(void *dst, const void *src, size_t bytes, hq_stream_t s) {
  return check(hipMemcpyAsync(dst, src, bytes, hipMemcpyDeviceToDevice, resolve(s)), "hipMemcpyDtoD");
}

int hq_memset(void *dst, int value, size_t bytes, hq_stream_t s) {
  if (bytes == 0) return HQ_OK;
  if (!dst) return fail(HQ_EINVAL, "hq_memset", "dst is NULL");
  // A fill kernel rather than hipMemsetAsync: memset nodes recorded into captured graphs
  // are not reliable on replay, and callers may capture this.
  const unsigned char *p = static_cast<const unsigned char *>(dst);
  const size_t head = std::min(bytes, (size_t)((16 - ((uintptr_t)p & 15)) & 15));
  const size_t n16 = (bytes - head) / 16, tail = bytes - head - n16 * 16;
  const uint32_t b = (uint32_t)(value & 0xff) * 0x01010101u;
  const size_t work = n16 + head + tail;
  const unsigned blocks = (unsigned)std::min<size_t>((work + 255) / 256, 65536);
  fill_bytes_kernel<<<blocks, 256, 0, resolve(s)>>>(static_cast<unsigned char *>(dst), head, n16, tail, b);
  return check_launch("hq_memset");
}

int hq_stream_create(hq_stream_t *stream) {
  if (!stream) return fail(HQ_EINVAL, "hq_stream_create", "stream is NULL");
  hipStream_t s = nullptr;
  int rc = check(hipStreamCreateWithFlags(&s, hipStreamNonBlocking), "hipStreamCreate");
  *stream = (hq_stream_t)s;
  return rc;
}

int hq_stream_destroy(hq_stream_t stream) {
  if (!stream) return HQ_OK;
  hipStream_t s = (hipStream_t)stream;
  hipStream_t cur = s;
  g_current.compare_exchange_strong(cur, nullptr);
  // The stream's library workspace goes with it (its last kernels have finished first).
  if (int rc = check(hipStreamSynchronize(s), "hipStreamSynchronize")) return rc;
  if (int rc = workspace_forget_stream(s)) return rc;
  moe_block_forget_stream(s);
  return check(hipStreamDestroy(s), "hipStreamDestroy");
}

int hq_stream_synchronize(hq_stream_t stream) {
  return check(hipStreamSynchronize(resolve(stream)), "hipStreamSynchronize");
}

int hq_stream_set_current(hq_stream_t stream) {
  g_current = (hipStream_t)stream;
  return HQ_OK;
}

hq_stream_t hq_stream_get_current(void) { return (hq_stream_t)g_current.load(); }

int hq_trace_start(void) {
  std::lock_guard<std::mutex> lk(g_tr_mu);
  g_spans.clear();
  g_tracing = true;
  return HQ_OK;
}

int hq_trace_stop(char *names, int *calls, double *total_us, int n_max) {
  std::vector<std::pair<std::string, std::pair<hipEvent_t, hipEvent_t>>> spans;
  {
    std::lock_guard<std::mutex> lk(g_tr_mu);
    g_tracing = false;
    spans.swap(g_spans);
  }
  std::map<std::string, TraceRec> agg;
  int rc = HQ_OK;
  for (auto &sp : spans) {
    float ms = 0;
    if (!rc) rc = check(hipEventSynchronize(sp.second.second), "hipEventSynchronize");
    if (!rc) rc = check(hipEventElapsedTime(&ms, sp.second.first, sp.second.second), "hipEventElapsedTime");
    auto &r = agg[sp.first];
    r.calls++;
    r.us += ms * 1000.0;
    (void)hipEventDestroy(sp.second.first);
    (void)hipEventDestroy(sp.second.second);
  }
  if (rc) return rc;
  int i = 0;
  for (auto &kv : agg) {
    if (i >= n_max) break;
    if (names) snprintf(names + 32 * i, 32, "%s", kv.first.c_str());
    if (calls) calls[i] = kv.second.calls;
    if (total_us) total_us[i] = kv.second.us;
    i++;
  }
  return i;
}

// ---------------------------------------------------------------------------
// ops
// ---------------------------------------------------------------------------

static bool is_gguf(int dt) {
  return dt == HQ_Q4_0 || dt == HQ_Q5_0 || dt == HQ_Q8_0 || dt == HQ_Q4_K || dt == HQ_Q5_K || dt == HQ_Q6_K;
}

// hq_matmul_q's weight formats: the GGUF six and the repacked Q6_K.
static bool is_matmul_w(int dt) { return is_gguf(dt) || dt == HQ_Q6_K_R; }

size_t hq_matmul_q_ws_bytes(int64_t M, int64_t N, int64_t K, int w_dtype) { return matmul_q_ws_bytes(M, N, K, w_dtype); }

int hq_matmul_q(const float *x, const void *w, float *out, int64_t M, int64_t N, int64_t K, int w_dtype,
                void *ws, size_t ws_bytes, hq_stream_t stream) {
  const char *call = "hq_matmul_q";
  if (!is_matmul_w(w_dtype)) return fail(HQ_EUNSUPPORTED, call, "weight dtype %d has no fused kernel", w_dtype);
  if (M < 0 || N < 0 || K <= 0) return fail(HQ_EINVAL, call, "bad shape M=%lld N=%lld K=%lld", (long long)M,
                                            (long long)N, (long long)K);
  BlockInfo bi = block_info(w_dtype);
  if (K % bi.elems)
    return fail(HQ_EINVAL, call, "K=%lld not a multiple of block size %d", (long long)K, bi.elems);
  if (M == 0 || N == 0) return HQ_OK;
  if (!x || !w || !out) return fail(HQ_EINVAL, call, "NULL pointer");
  if (((uintptr_t)x & 15) || ((uintptr_t)w & 15) || ((uintptr_t)out & 3))
    return fail(HQ_EINVAL, call, "x and w must be 16-byte aligned, out 4-byte aligned");
  hipStream_t s = resolve(stream);
  size_t need = matmul_q_ws_bytes(M, N, K, w_dtype);
  if (!ws) {
    if (int rc = workspace(need, s, &ws, call)) return rc;
  } else if (ws_bytes < need) {
    return fail(HQ_ENOMEM, call, "workspace %zu bytes < %zu needed", ws_bytes, need);
  }
  TraceSpan span(matmul_q_kernel_name(M, w_dtype), s);
  return launch_matmul_q(x, w, out, M, N, K, w_dtype, ws, s);
}

int hq_matmul_q_noalloc(const float *x, const void *w, float *out, int64_t M, int64_t N, int64_t K, int w_dtype,
                        hq_stream_t stream) {
  const char *call = "hq_matmul_q_noalloc";
  if (!is_matmul_w(w_dtype)) return fail(HQ_EUNSUPPORTED, call, "weight dtype %d has no fused kernel", w_dtype);
  if (M < 0 || N < 0 || K <= 0) return fail(HQ_EINVAL, call, "bad shape M=%lld N=%lld K=%lld", (long long)M,
                                            (long long)N, (long long)K);
  BlockInfo bi = block_info(w_dtype);
  if (K % bi.elems)
    return fail(HQ_EINVAL, call, "K=%lld not a multiple of block size %d", (long long)K, bi.elems);
  if (M == 0 || N == 0) return HQ_OK;
  if (!x || !w || !out) return fail(HQ_EINVAL, call, "NULL pointer");
  if (((uintptr_t)x & 15) || ((uintptr_t)w & 15) || ((uintptr_t)out & 3))
    return fail(HQ_EINVAL, call, "x and w must be 16-byte aligned, out 4-byte aligned");
  size_t need = matmul_q_ws_bytes(M, N, K, w_dtype);
  if (need > HQ_NOALLOC_SCRATCH_BYTES)
    return fail(HQ_ENOMEM, call, "needs %zu bytes of scratch, more than the %zu-byte static scratch", need,
                (size_t)HQ_NOALLOC_SCRATCH_BYTES);
  void *ws = nullptr;
  if (int rc = scratch_ptr(&ws, call)) return rc;
  hipStream_t s = resolve(stream);
  TraceSpan span(matmul_q_kernel_name(M, w_dtype), s);
  return launch_matmul_q(x, w, out, M, N, K, w_dtype, ws, s);
}

int hq_workspace_release(void) { return workspace_release(); }

size_t hq_matmul_q_gated_ws_bytes(int64_t M, int64_t N, int64_t K, int w_dtype) {
  return matmul_q_gated_ws_bytes(M, N, K, w_dtype);
}

int hq_matmul_q_gated(const float *x, const void *wg, const void *wu, float *out, int64_t M, int64_t N, int64_t K,
                      int w_dtype, int act, void *ws, size_t ws_bytes, hq_stream_t stream) {
  const char *call = "hq_matmul_q_gated";
  if (!is_gguf(w_dtype)) return fail(HQ_EUNSUPPORTED, call, "weight dtype %d has no fused kernel", w_dtype);
  if (act != HQ_ACT_SILU && act != HQ_ACT_GELU_ERF) return fail(HQ_EINVAL, call, "activation %d", act);
  if (M < 0 || N < 0 || K <= 0) return fail(HQ_EINVAL, call, "bad shape M=%lld N=%lld K=%lld", (long long)M,
                                            (long long)N, (long long)K);
  BlockInfo bi = block_info(w_dtype);
  if (K % bi.elems)
    return fail(HQ_EINVAL, call, "K=%lld not a multiple of block size %d", (long long)K, bi.elems);
  if (M == 0 || N == 0) return HQ_OK;
  if (!x || !wg || !wu || !out) return fail(HQ_EINVAL, call, "NULL pointer");
  if (((uintptr_t)x & 15) || ((uintptr_t)wg & 15) || ((uintptr_t)wu & 15) || ((uintptr_t)out & 3))
    return fail(HQ_EINVAL, call, "x, wg and wu must be 16-byte aligned, out 4-byte aligned");
  hipStream_t s = resolve(stream);
  size_t need = matmul_q_gated_ws_bytes(M, N, K, w_dtype);
  if (!ws) {
    if (int rc = workspace(need, s, &ws, call)) return rc;
  } else if (ws_bytes < need) {
    return fail(HQ_ENOMEM, call, "workspace %zu bytes < %zu needed", ws_bytes, need);
  }
  TraceSpan span("matmul_q_gated", s);
  return launch_matmul_q_gated(x, wg, wu, out, M, N, K, w_dtype, act, ws, s);
}

size_t hq_matmul_q_gated_act_ws_bytes(int64_t M, int64_t N, int64_t K, int w_dtype) {
  return matmul_q_gated_act_ws_bytes(M, N, K, w_dtype);
}

int hq_matmul_q_gated_act(const float *x, const void *wg, const void *wu, void *act_out, int64_t M, int64_t N,
                          int64_t K, int w_dtype, int act, void *ws, size_t ws_bytes, hq_stream_t stream) {
  const char *call = "hq_matmul_q_gated_act";
  if (!is_gguf(w_dtype)) return fail(HQ_EUNSUPPORTED, call, "weight dtype %d has no fused kernel", w_dtype);
  if (act != HQ_ACT_SILU && act != HQ_ACT_GELU_ERF) return fail(HQ_EINVAL, call, "activation %d", act);
  if (M < 0 || N < 0 || K <= 0 || N % 32)
    return fail(HQ_EINVAL, call, "bad shape M=%lld N=%lld K=%lld (N must be a multiple of 32)", (long long)M,
                (long long)N, (long long)K);
  BlockInfo bi = block_info(w_dtype);
  if (K % bi.elems)
    return fail(HQ_EINVAL, call, "K=%lld not a multiple of block size %d", (long long)K, bi.elems);
  if (M == 0 || N == 0) return HQ_OK;
  if (!x || !wg || !wu || !act_out) return fail(HQ_EINVAL, call, "NULL pointer");
  if (((uintptr_t)x & 15) || ((uintptr_t)wg & 15) || ((uintptr_t)wu & 15) || ((uintptr_t)act_out & 15))
    return fail(HQ_EINVAL, call, "x, wg, wu and act_out must be 16-byte aligned");
  hipStream_t s = resolve(stream);
  size_t need = matmul_q_gated_act_ws_bytes(M, N, K, w_dtype);
  if (!ws) {
    if (int rc = workspace(need, s, &ws, call)) return rc;
  } else if (ws_bytes < need) {
    return fail(HQ_ENOMEM, call, "workspace %zu bytes < %zu needed", ws_bytes, need);
  }
  TraceSpan span("matmul_q_gated_act", s);
  return launch_matmul_q_gated_act(x, wg, wu, static_cast<uint8_t *>(act_out), M, N, K, w_dtype, act, ws, s);
}

size_t hq_mlp_q_ws_bytes(int64_t M, int64_t H, int64_t I, int w_dtype) { return mlp_q_ws_bytes(M, H, I, w_dtype); }

int hq_mlp_q(const float *x, const void *wg, const void *wu, const void *wd, float *out, int64_t M, int64_t H,
             int64_t I, int w_dtype, int act, void *ws, size_t ws_bytes, hq_stream_t stream) {
  const char *call = "hq_mlp_q";
  if (!is_gguf(w_dtype)) return fail(HQ_EUNSUPPORTED, call, "weight dtype %d has no fused kernel", w_dtype);
  if (act != HQ_ACT_SILU && act != HQ_ACT_GELU_ERF) return fail(HQ_EINVAL, call, "activation %d", act);
  if (M < 0 || H <= 0 || I <= 0)
    return fail(HQ_EINVAL, call, "bad shape M=%lld H=%lld I=%lld", (long long)M, (long long)H, (long long)I);
  BlockInfo bi = block_info(w_dtype);
  if (H % bi.elems || I % bi.elems)
    return fail(HQ_EINVAL, call, "H=%lld, I=%lld not multiples of block size %d", (long long)H, (long long)I,
                bi.elems);
  if (M == 0) return HQ_OK;
  if (!x || !wg || !wu || !wd || !out) return fail(HQ_EINVAL, call, "NULL pointer");
  if (((uintptr_t)x & 15) || ((uintptr_t)wg & 15) || ((uintptr_t)wu & 15) || ((uintptr_t)wd & 15) ||
      ((uintptr_t)out & 3))
    return fail(HQ_EINVAL, call, "x and the weights must be 16-byte aligned, out 4-byte aligned");
  hipStream_t s = resolve(stream);
  size_t need = mlp_q_ws_bytes(M, H, I, w_dtype);
  if (!ws) {
    if (int rc = workspace(need, s, &ws, call)) return rc;
  } else if (ws_bytes < need) {
    return fail(HQ_ENOMEM, call, "workspace %zu bytes < %zu needed", ws_bytes, need);
  }
  TraceSpan span("mlp_q", s);
  return launch_mlp_q(x, wg, wu, wd, out, M, H, I, w_dtype, act, ws, s);
}

size_t hq_act_bytes(int64_t M, int64_t K) {
  if (M <= 0 || K <= 0 || K % 32) return 0;
  return (size_t)act_bytes(M, K);
}

int hq_quantize_act(const void *x, int x_dtype, void *act, int64_t M, int64_t K, hq_stream_t stream) {
  const char *call = "hq_quantize_act";
  if (x_dtype != HQ_F32 && x_dtype != HQ_BF16 && x_dtype != HQ_F16)
    return fail(HQ_EUNSUPPORTED, call, "x dtype %d", x_dtype);
  if (M < 0 || K < 0 || K % 32) return fail(HQ_EINVAL, call, "K=%lld not a multiple of 32", (long long)K);
  if (M == 0 || K == 0) return HQ_OK;
  if (!x || !act) return fail(HQ_EINVAL, call, "NULL pointer");
  if (((uintptr_t)x & 15) || ((uintptr_t)act & 15)) return fail(HQ_EINVAL, call, "x and act must be 16-byte aligned");
  hipStream_t s = resolve(stream);
  TraceSpan span("quantize_act", s);
  return launch_quantize_act(x, x_dtype, act, M, K, s);
}

size_t hq_matmul_q_act_ws_bytes(int64_t M, int64_t N, int64_t K, int w_dtype) {
  return matmul_act_ws_bytes(M, N, K, w_dtype);
}

int hq_matmul_q_act(const void *act, const void *w, float *out, int64_t M, int64_t N, int64_t K, int w_dtype,
                    void *ws, size_t ws_bytes, hq_stream_t stream) {
  const char *call = "hq_matmul_q_act";
  if (!is_gguf(w_dtype)) return fail(HQ_EUNSUPPORTED, call, "weight dtype %d has no fused kernel", w_dtype);
  if (M < 0 || N < 0 || K <= 0) return fail(HQ_EINVAL, call, "bad shape");
  BlockInfo bi = block_info(w_dtype);
  if (K % bi.elems)
    return fail(HQ_EINVAL, call, "K=%lld not a multiple of block size %d", (long long)K, bi.elems);
  if (M == 0 || N == 0) return HQ_OK;
  if (!act || !w || !out) return fail(HQ_EINVAL, call, "NULL pointer");
  if (((uintptr_t)act & 15) || ((uintptr_t)out & 3)) return fail(HQ_EINVAL, call, "act must be 16-byte aligned");
  // Calls that take the GEMV (M <= 8, or K not a multiple of the GEMM's 64-k step) read the
  // weight through the int8 GEMV, whose rows must be whole 16-byte pieces (rows longer than
  // one team or slice run as K parts).
  if (!matmul_act_takes_gemm(M, K, w_dtype) && !gemv_fast_ok(w_dtype, K, w) &&
      !act_long_rows_ok(M, N, K, w_dtype, w, act))
    return fail(HQ_EUNSUPPORTED, call, "weight layout needs the F32 path (hq_matmul_q)");
  hipStream_t s = resolve(stream);
  size_t need = hq_matmul_q_act_ws_bytes(M, N, K, w_dtype);
  if (need && !ws) {
    if (int rc = workspace(need, s, &ws, call)) return rc;
  } else if (need && ws_bytes < need) {
    return fail(HQ_ENOMEM, call, "workspace %zu bytes < %zu needed", ws_bytes, need);
  }
  TraceSpan span(matmul_q_kernel_name(M, w_dtype), s);
  return launch_matmul_act(act, w, out, M, N, K, w_dtype, ws, s);
}

int hq_dequant(const void *src, void *dst, int64_t n, int src_dtype, int out_dtype, hq_stream_t stream) {
  const char *call = "hq_dequant";
  if (!is_gguf(src_dtype) && src_dtype != HQ_Q8_1)
    return fail(HQ_EUNSUPPORTED, call, "source dtype %d", src_dtype);
  if (out_dtype != HQ_F32 && out_dtype != HQ_BF16) return fail(HQ_EUNSUPPORTED, call, "out dtype %d", out_dtype);
  BlockInfo bi = block_info(src_dtype);
  if (n < 0 || n % bi.elems) return fail(HQ_EINVAL, call, "n=%lld not a multiple of %d", (long long)n, bi.elems);
  if (n == 0) return HQ_OK;
  if (!src || !dst) return fail(HQ_EINVAL, call, "NULL pointer");
  hipStream_t s = resolve(stream);
  TraceSpan span("dequant", s);
  return launch_dequant(src, dst, n, src_dtype, out_dtype, s);
}

size_t hq_repack_q6k_bytes(int64_t N, int64_t K) {
  if (N < 0 || K <= 0 || K % 256) return 0;
  return (size_t)(N * q6kr_row_bytes(K));
}

int hq_repack_q6k(const void *src, void *dst, int64_t N, int64_t K, hq_stream_t stream) {
  const char *call = "hq_repack_q6k";
  if (N < 0 || K <= 0 || K % 256) return fail(HQ_EINVAL, call, "K=%lld not a positive multiple of 256", (long long)K);
  if (N > INT32_MAX || K > INT32_MAX) return fail(HQ_EINVAL, call, "shape too large");
  if (N == 0) return HQ_OK;
  if (!src || !dst) return fail(HQ_EINVAL, call, "NULL pointer");
  if (((uintptr_t)src & 1) || ((uintptr_t)dst & 15))
    return fail(HQ_EINVAL, call, "src must be 2-byte aligned, dst 16-byte aligned");
  hipStream_t s = resolve(stream);
  TraceSpan span("repack_q6k", s);
  return launch_repack_q6k(src, dst, N, K, s);
}

int hq_dequant_rows(const void *src, void *dst, int64_t N, int64_t K, int src_dtype, int out_dtype,
                    hq_stream_t stream) {
  const char *call = "hq_dequant_rows";
  if (src_dtype != HQ_Q6_K_R) {
    if (N < 0 || K < 0) return fail(HQ_EINVAL, call, "bad shape N=%lld K=%lld", (long long)N, (long long)K);
    if (src_dtype != HQ_Q8_1 && !is_gguf(src_dtype)) return fail(HQ_EUNSUPPORTED, call, "source dtype %d", src_dtype);
    if (K % block_info(src_dtype).elems) return fail(HQ_EINVAL, call, "K=%lld not a multiple of the block", (long long)K);
    return hq_dequant(src, dst, N * K, src_dtype, out_dtype, stream);
  }
  if (out_dtype != HQ_F32 && out_dtype != HQ_BF16) return fail(HQ_EUNSUPPORTED, call, "out dtype %d", out_dtype);
  if (N < 0 || K <= 0 || K % 256) return fail(HQ_EINVAL, call, "K=%lld not a positive multiple of 256", (long long)K);
  if (N == 0) return HQ_OK;
  if (!src || !dst) return fail(HQ_EINVAL, call, "NULL pointer");
  if (((uintptr_t)src & 15) || ((uintptr_t)dst & 15)) return fail(HQ_EINVAL, call, "src and dst must be 16-byte aligned");
  hipStream_t s = resolve(stream);
  TraceSpan span("dequant", s);
  return launch_dequant_q6kr(src, dst, N, K, out_dtype, s);
}

int hq_quantize_q8_1(const void *x, int x_dtype, void *dst, int64_t M, int64_t K, hq_stream_t stream) {
  const char *call = "hq_quantize_q8_1";
  if (x_dtype != HQ_F32 && x_dtype != HQ_BF16 && x_dtype != HQ_F16)
    return fail(HQ_EUNSUPPORTED, call, "x dtype %d", x_dtype);
  if (M < 0 || K < 0 || K % 32) return fail(HQ_EINVAL, call, "K=%lld not a multiple of 32", (long long)K);
  if (M == 0 || K == 0) return HQ_OK;
  if (!x || !dst) return fail(HQ_EINVAL, call, "NULL pointer");
  hipStream_t s = resolve(stream);
  TraceSpan span("quantize_q8_1", s);
  return launch_quantize_q8_1(x, x_dtype, dst, M, K, s);
}

size_t hq_int4_matmul_ws_bytes(int64_t M, int64_t N, int64_t K, int G, int x_dtype) {
  return int4_ws_bytes(M, N, K, G, x_dtype);
}

int hq_int4_matmul(const void *x, int x_dtype, const uint32_t *codes, const float *scales, const float *zeros,
                   void *y, int64_t M, int64_t N, int64_t K, int G, void *ws, size_t ws_bytes,
                   hq_stream_t stream) {
  const char *call = "hq_int4_matmul";
  if (x_dtype != HQ_F32 && x_dtype != HQ_BF16 && x_dtype != HQ_F16)
    return fail(HQ_EUNSUPPORTED, call, "activations dtype %d, want F32, BF16 or F16", x_dtype);
  if (M < 0 || N < 0 || K <= 0 || G <= 0 || K % G)
    return fail(HQ_EINVAL, call, "group %d does not divide K %lld", G, (long long)K);
  if (K % 32 || G % 32) return fail(HQ_EUNSUPPORTED, call, "K=%lld and G=%d must be multiples of 32", (long long)K, G);
  if (M == 0 || N == 0) return HQ_OK;
  if (!x || !codes || !scales || !zeros || !y) return fail(HQ_EINVAL, call, "NULL pointer");
  hipStream_t s = resolve(stream);
  if (((uintptr_t)x & 15)) return fail(HQ_EINVAL, call, "x must be 16-byte aligned");
  size_t need = int4_ws_bytes(M, N, K, G, x_dtype);
  if (!ws) {
    if (int rc = workspace(need, s, &ws, call)) return rc;
  } else if (ws_bytes < need) {
    return fail(HQ_ENOMEM, call, "workspace %zu bytes < %zu needed", ws_bytes, need);
  }
  TraceSpan span("int4_matmul", s);
  return launch_int4_matmul(x, x_dtype, codes, scales, zeros, y, M, N, K, G, ws, s);
}

int hq_int4_from_gptq(const void *qweight, const void *qzeros, const float *scales, const int64_t *perm, int64_t K,
                      int64_t N, int group, int v2, uint32_t *codes, float *scales_out, float *zeros_out,
                      hq_stream_t stream) {
  const char *call = "hq_int4_from_gptq";
  if (K <= 0 || N <= 0 || K % 8 || N % 8) return fail(HQ_EINVAL, call, "K=%lld N=%lld (multiples of 8)", (long long)K, (long long)N);
  if (group <= 0 || K % group) return fail(HQ_EINVAL, call, "group %d does not divide K %lld", group, (long long)K);
  if (!qweight || !qzeros || !scales || !codes || !scales_out || !zeros_out) return fail(HQ_EINVAL, call, "NULL pointer");
  hipStream_t s = resolve(stream);
  TraceSpan span("int4_from_gptq", s);
  return launch_int4_from_gptq(static_cast<const uint32_t *>(qweight), static_cast<const uint32_t *>(qzeros), scales,
                               perm, K, N, group, v2 != 0, codes, scales_out, zeros_out, s);
}

int hq_int4_from_awq(const void *qweight, const void *qzeros, const float *scales, int64_t K, int64_t N, int group,
                     uint32_t *codes, float *scales_out, float *zeros_out, hq_stream_t stream) {
  const char *call = "hq_int4_from_awq";
  if (K <= 0 || N <= 0 || K % 8 || N % 8) return fail(HQ_EINVAL, call, "K=%lld N=%lld (multiples of 8)", (long long)K, (long long)N);
  if (group <= 0 || K % group) return fail(HQ_EINVAL, call, "group %d does not divide K %lld", group, (long long)K);
  if (!qweight || !qzeros || !scales || !codes || !scales_out || !zeros_out) return fail(HQ_EINVAL, call, "NULL pointer");
  hipStream_t s = resolve(stream);
  TraceSpan span("int4_from_awq", s);
  return launch_int4_from_awq(static_cast<const uint32_t *>(qweight), static_cast<const uint32_t *>(qzeros), scales,
                              K, N, group, codes, scales_out, zeros_out, s);
}

int hq_int4_dequant(const uint32_t *codes, const float *scales, const float *zeros, void *out, int out_dtype,
                    int64_t N, int64_t K, int G, int64_t out_offset, hq_stream_t stream) {
  const char *call = "hq_int4_dequant";
  if (G <= 0 || K <= 0 || K % G) return fail(HQ_EINVAL, call, "group %d does not divide K %lld", G, (long long)K);
  if (K % 8) return fail(HQ_EINVAL, call, "K=%lld not a multiple of 8", (long long)K);
  if (out_dtype != HQ_F32 && out_dtype != HQ_BF16) return fail(HQ_EUNSUPPORTED, call, "out dtype %d", out_dtype);
  if (N < 0 || out_offset < 0) return fail(HQ_EINVAL, call, "bad N or offset");
  if (N == 0) return HQ_OK;
  if (!codes || !scales || !zeros || !out) return fail(HQ_EINVAL, call, "NULL pointer");
  hipStream_t s = resolve(stream);
  TraceSpan span("int4_dequant", s);
  return launch_int4_dequant(codes, scales, zeros, out, out_dtype, N, K, G, out_offset, s);
}

size_t hq_moe_gemm_q_ws_bytes(int64_t rows, int64_t K, int w_dtype) { return moe_ws_bytes(rows, K, w_dtype); }

int hq_moe_gemm_q(const float *x, const void *w, const int64_t *sorted_pairs, const int64_t *sorted_expts,
                  int32_t *counts, int32_t *offsets, const float *topk_w, float *out, int topk, int64_t size_m,
                  int64_t M, int64_t rows, int64_t E, int64_t N, int64_t K, int row_per_pair, int w_dtype,
                  void *ws, size_t ws_bytes, hq_stream_t stream) {
  const char *call = "hq_moe_gemm_q";
  if (!is_gguf(w_dtype)) return fail(HQ_EUNSUPPORTED, call, "weight dtype %d has no fused kernel", w_dtype);
  if (E <= 0 || N < 0 || K <= 0 || M < 0 || size_m < 0 || rows < 0 || topk < 1)
    return fail(HQ_EINVAL, call, "bad shape");
  BlockInfo bi = block_info(w_dtype);
  if (K % bi.elems) return fail(HQ_EINVAL, call, "K=%lld not a multiple of block size %d", (long long)K, bi.elems);
  if (row_per_pair ? rows != M : rows != M / topk)
    return fail(HQ_EINVAL, call, "input rows %lld must be M=%lld (per pair) or M/topk=%lld (per token)",
                (long long)rows, (long long)M, (long long)(M / topk));
  if (M == 0 || N == 0) return HQ_OK;
  if (!x || !w || !sorted_pairs || !sorted_expts || !counts || !offsets || !out)
    return fail(HQ_EINVAL, call, "NULL pointer");
  hipStream_t s = resolve(stream);
  if (((uintptr_t)x & 15)) return fail(HQ_EINVAL, call, "x must be 16-byte aligned");
  size_t need = moe_ws_bytes(rows, K, w_dtype);
  if (need && !ws) {
    if (int rc = workspace(need, s, &ws, call)) return rc;
  } else if (need && ws_bytes < need) {
    return fail(HQ_ENOMEM, call, "workspace %zu bytes < %zu needed", ws_bytes, need);
  }
  TraceSpan span("moe_gemm_q", s);
  return launch_moe_q(x, w, sorted_pairs, sorted_expts, counts, offsets, topk_w, out, topk, size_m, M, rows, E, N, K,
                      row_per_pair, w_dtype, ws, s);
}

int hq_moe_combine(const float *pair_out, float *out, int64_t M, int64_t N, int topk, hq_stream_t stream) {
  const char *call = "hq_moe_combine";
  if (topk < 1 || M < 0 || N < 0 || M % topk)
    return fail(HQ_EINVAL, call, "%lld rows not divisible by topk %d", (long long)M, topk);
  if (M == 0 || N == 0) return HQ_OK;
  if (!pair_out || !out) return fail(HQ_EINVAL, call, "NULL pointer");
  hipStream_t s = resolve(stream);
  TraceSpan span("moe_combine", s);
  return launch_moe_combine(pair_out, out, M / topk, N, topk, s);
}

size_t hq_moe_gemm_q_combine_ws_bytes(int64_t T, int topk, int64_t E, int64_t N, int64_t K, int w_dtype) {
  if (T <= 0 || topk < 1 || E <= 0 || N <= 0 || K <= 0) return 0;
  return moe_combine_ws_bytes(T * topk, E, N, K, w_dtype);
}

int hq_moe_gemm_q_combine(const float *h, const void *w, const int64_t *sorted_pairs, const int64_t *sorted_expts,
                          int32_t *counts, int32_t *offsets, const float *topk_w, float *y, int topk, int64_t T,
                          int64_t E, int64_t N, int64_t K, int w_dtype, void *ws, size_t ws_bytes,
                          hq_stream_t stream) {
  const char *call = "hq_moe_gemm_q_combine";
  if (!is_gguf(w_dtype)) return fail(HQ_EUNSUPPORTED, call, "weight dtype %d has no fused kernel", w_dtype);
  if (E <= 0 || N < 0 || K <= 0 || T < 0 || topk < 1) return fail(HQ_EINVAL, call, "bad shape");
  BlockInfo bi = block_info(w_dtype);
  if (K % bi.elems) return fail(HQ_EINVAL, call, "K=%lld not a multiple of block size %d", (long long)K, bi.elems);
  if (T == 0 || N == 0) return HQ_OK;
  if (!h || !w || !sorted_pairs || !sorted_expts || !y) return fail(HQ_EINVAL, call, "NULL pointer");
  if (((uintptr_t)h & 15)) return fail(HQ_EINVAL, call, "h must be 16-byte aligned");
  hipStream_t s = resolve(stream);
  const size_t need = moe_combine_ws_bytes(T * topk, E, N, K, w_dtype);
  if (!ws) {
    if (int rc = workspace(need, s, &ws, call)) return rc;
  } else if (ws_bytes < need) {
    return fail(HQ_ENOMEM, call, "workspace %zu bytes < %zu needed", ws_bytes, need);
  }
  TraceSpan span("moe_gemm_q_combine", s);
  return launch_moe_q_combine(h, w, sorted_pairs, sorted_expts, counts, offsets, topk_w, y, topk, T, E, N, K,
                              w_dtype, ws, s);
}

int hq_moe_route(const float *probs, int64_t T, int64_t E, int topk, int normalize, int64_t *topk_ids,
                 float *weights, int64_t *sorted_pairs, int64_t *sorted_expts, int32_t *counts, int32_t *offsets,
                 hq_stream_t stream) {
  const char *call = "hq_moe_route";
  if (T < 0 || E < 1) return fail(HQ_EINVAL, call, "probs must be (T, E), got (%lld, %lld)", (long long)T, (long long)E);
  if (topk < 1 || topk > E) return fail(HQ_EINVAL, call, "topk %d out of range [1, %lld]", topk, (long long)E);
  if (T == 0) return HQ_OK;
  if (topk > 64 || !moe_route_fits(T * topk, E))
    return fail(HQ_EUNSUPPORTED, call, "T=%lld E=%lld topk=%d beyond the one-workgroup sort", (long long)T,
                (long long)E, topk);
  if (!probs || !topk_ids || !weights || !sorted_pairs || !sorted_expts) return fail(HQ_EINVAL, call, "NULL pointer");
  hipStream_t s = resolve(stream);
  TraceSpan span("moe_route", s);
  return launch_moe_route(probs, T, E, topk, normalize, topk_ids, weights, sorted_pairs, sorted_expts, counts,
                          offsets, s);
}

int hq_moe_sort_ids(const int64_t *ids, int64_t M, int64_t E, int64_t *sorted_pairs, int64_t *sorted_expts,
                    int32_t *counts, int32_t *offsets, hq_stream_t stream) {
  const char *call = "hq_moe_sort_ids";
  if (M < 0 || E < 1) return fail(HQ_EINVAL, call, "bad shape");
  if (M == 0) return HQ_OK;
  if (!moe_route_fits(M, E))
    return fail(HQ_EUNSUPPORTED, call, "M=%lld E=%lld beyond the one-workgroup sort", (long long)M, (long long)E);
  if (!ids || !sorted_pairs || !sorted_expts) return fail(HQ_EINVAL, call, "NULL pointer");
  hipStream_t s = resolve(stream);
  TraceSpan span("moe_sort", s);
  return launch_moe_sort_ids(ids, M, E, sorted_pairs, sorted_expts, counts, offsets, s);
}

size_t hq_moe_gemm_q_gated_ws_bytes(int64_t size_m, int64_t rows, int64_t I, int64_t K, int w_dtype) {
  if (size_m < 0 || rows < 0 || I < 0 || K <= 0) return 0;
  return moe_gated_ws_bytes(size_m, rows, I, K, w_dtype);
}

int hq_moe_gemm_q_gated(const float *x, const void *w, const int64_t *sorted_pairs, const int64_t *sorted_expts,
                        int32_t *counts, int32_t *offsets, float *out, int topk, int64_t size_m, int64_t M,
                        int64_t rows, int64_t E, int64_t I, int64_t K, int row_per_pair, int w_dtype, int act,
                        void *ws, size_t ws_bytes, hq_stream_t stream) {
  const char *call = "hq_moe_gemm_q_gated";
  if (!is_gguf(w_dtype)) return fail(HQ_EUNSUPPORTED, call, "weight dtype %d has no fused kernel", w_dtype);
  if (act != HQ_ACT_SILU && act != HQ_ACT_GELU_ERF) return fail(HQ_EINVAL, call, "activation %d", act);
  if (E <= 0 || I < 0 || K <= 0 || M < 0 || size_m < 0 || rows < 0 || topk < 1)
    return fail(HQ_EINVAL, call, "bad shape");
  BlockInfo bi = block_info(w_dtype);
  if (K % bi.elems) return fail(HQ_EINVAL, call, "K=%lld not a multiple of block size %d", (long long)K, bi.elems);
  if (row_per_pair ? rows != M : rows != M / topk)
    return fail(HQ_EINVAL, call, "input rows %lld must be M=%lld (per pair) or M/topk=%lld (per token)",
                (long long)rows, (long long)M, (long long)(M / topk));
  if (M == 0 || I == 0) return HQ_OK;
  if (!x || !w || !sorted_pairs || !sorted_expts || !counts || !offsets || !out)
    return fail(HQ_EINVAL, call, "NULL pointer");
  if (((uintptr_t)x & 15)) return fail(HQ_EINVAL, call, "x must be 16-byte aligned");
  hipStream_t s = resolve(stream);
  const size_t need = moe_gated_ws_bytes(size_m, rows, I, K, w_dtype);
  if (!ws) {
    if (int rc = workspace(need, s, &ws, call)) return rc;
  } else if (ws_bytes < need) {
    return fail(HQ_ENOMEM, call, "workspace %zu bytes < %zu needed", ws_bytes, need);
  }
  TraceSpan span("moe_gemm_q_gated", s);
  return launch_moe_q_gated(x, w, sorted_pairs, sorted_expts, counts, offsets, out, topk, size_m, M, rows, E, I, K,
                            row_per_pair, w_dtype, act, ws, s);
}

size_t hq_moe_route_gated_ws_bytes(int64_t T, int topk, int64_t E, int64_t I, int64_t K, int w_dtype) {
  if (T <= 0 || topk < 1 || E <= 0 || I <= 0 || K <= 0) return 0;
  return moe_route_gated_ws_bytes(T, topk, E, I, K, w_dtype);
}

int hq_moe_route_gated(const float *probs, const float *x, const void *w, float *h, int64_t T, int64_t E, int topk,
                       int normalize, int64_t I, int64_t K, int w_dtype, int act, int64_t *topk_ids, float *weights,
                       int64_t *sorted_pairs, int64_t *sorted_expts, int32_t *counts, int32_t *offsets, void *ws,
                       size_t ws_bytes, hq_stream_t stream) {
  const char *call = "hq_moe_route_gated";
  if (!is_gguf(w_dtype)) return fail(HQ_EUNSUPPORTED, call, "weight dtype %d has no fused kernel", w_dtype);
  if (act != HQ_ACT_SILU && act != HQ_ACT_GELU_ERF) return fail(HQ_EINVAL, call, "activation %d", act);
  if (T < 0 || E < 1) return fail(HQ_EINVAL, call, "probs must be (T, E), got (%lld, %lld)", (long long)T, (long long)E);
  if (topk < 1 || topk > E) return fail(HQ_EINVAL, call, "topk %d out of range [1, %lld]", topk, (long long)E);
  if (I < 0 || K <= 0) return fail(HQ_EINVAL, call, "bad shape");
  BlockInfo bi = block_info(w_dtype);
  if (K % bi.elems) return fail(HQ_EINVAL, call, "K=%lld not a multiple of block size %d", (long long)K, bi.elems);
  if (T == 0) return HQ_OK;
  if (topk > 64 || !moe_route_fits(T * topk, E))
    return fail(HQ_EUNSUPPORTED, call, "T=%lld E=%lld topk=%d beyond the one-workgroup sort", (long long)T,
                (long long)E, topk);
  if (!probs || !x || !w || !h || !topk_ids || !weights || !sorted_pairs || !sorted_expts)
    return fail(HQ_EINVAL, call, "NULL pointer");
  if (((uintptr_t)x & 15)) return fail(HQ_EINVAL, call, "x must be 16-byte aligned");
  hipStream_t s = resolve(stream);
  const size_t need = moe_route_gated_ws_bytes(T, topk, E, I, K, w_dtype);
  if (!ws) {
    if (int rc = workspace(need, s, &ws, call)) return rc;
  } else if (ws_bytes < need) {
    return fail(HQ_ENOMEM, call, "workspace %zu bytes < %zu needed", ws_bytes, need);
  }
  TraceSpan span("moe_route_gated", s);
  return launch_moe_route_gated_any(probs, x, w, h, T, E, topk, normalize, I, K, w_dtype, act, topk_ids, weights,
                                    sorted_pairs, sorted_expts, counts, offsets, ws, s);
}

int hq_moe_block_q_check(hq_stream_t stream) { return moe_block_check(resolve(stream), "hq_moe_block_q_check"); }

void hq_debug_moe_block_spin_limit(uint32_t limit) { moe_block_set_spin_limit(limit); }

size_t hq_moe_block_q_ws_bytes(int64_t T, int topk, int64_t E, int64_t H, int64_t I, int w_dtype) {
  if (T <= 0 || topk < 1 || E <= 0 || H <= 0 || I <= 0) return 0;
  return moe_block_ws_bytes(T, topk, E, H, I, w_dtype);
}

int hq_moe_block_q(const float *probs, const float *x, const void *w_gate_up, const void *w_down, float *h, float *y,
                   int64_t T, int64_t E, int topk, int normalize, int64_t H, int64_t I, int w_dtype, int act,
                   int64_t *topk_ids, float *weights, int64_t *sorted_pairs, int64_t *sorted_expts, int32_t *counts,
                   int32_t *offsets, void *ws, size_t ws_bytes, hq_stream_t stream) {
  const char *call = "hq_moe_block_q";
  if (!is_gguf(w_dtype)) return fail(HQ_EUNSUPPORTED, call, "weight dtype %d has no fused kernel", w_dtype);
  if (act != HQ_ACT_SILU && act != HQ_ACT_GELU_ERF) return fail(HQ_EINVAL, call, "activation %d", act);
  if (T < 0 || E < 1) return fail(HQ_EINVAL, call, "probs must be (T, E), got (%lld, %lld)", (long long)T, (long long)E);
  if (topk < 1 || topk > E) return fail(HQ_EINVAL, call, "topk %d out of range [1, %lld]", topk, (long long)E);
  if (H <= 0 || I <= 0) return fail(HQ_EINVAL, call, "bad shape H=%lld I=%lld", (long long)H, (long long)I);
  BlockInfo bi = block_info(w_dtype);
  if (H % bi.elems || I % bi.elems)
    return fail(HQ_EINVAL, call, "H=%lld, I=%lld not multiples of block size %d", (long long)H, (long long)I,
                bi.elems);
  if (T == 0) return HQ_OK;
  if (topk > 64 || !moe_route_fits(T * topk, E))
    return fail(HQ_EUNSUPPORTED, call, "T=%lld E=%lld topk=%d beyond the one-workgroup sort", (long long)T,
                (long long)E, topk);
  if (!probs || !x || !w_gate_up || !w_down || !h || !y || !topk_ids || !weights || !sorted_pairs || !sorted_expts)
    return fail(HQ_EINVAL, call, "NULL pointer");
  if (((uintptr_t)x & 15) || ((uintptr_t)h & 15)) return fail(HQ_EINVAL, call, "x and h must be 16-byte aligned");
  hipStream_t s = resolve(stream);
  const size_t need = moe_block_ws_bytes(T, topk, E, H, I, w_dtype);
  if (!ws) {
    if (int rc = workspace(need, s, &ws, call)) return rc;
  } else if (ws_bytes < need) {
    return fail(HQ_ENOMEM, call, "workspace %zu bytes < %zu needed", ws_bytes, need);
  }
  TraceSpan span("moe_block_q", s);
  return launch_moe_block_any(probs, x, w_gate_up, w_down, h, y, T, E, topk, normalize, H, I, w_dtype, act, topk_ids,
                              weights, sorted_pairs, sorted_expts, counts, offsets, ws, s);
}

size_t hq_moe_int4_ws_bytes(int64_t T, int topk, int64_t I) {
  if (T <= 0 || topk < 1 || I <= 0) return 0;
  return moe_int4_ws_bytes(T, topk, I);
}

int hq_moe_int4(const void *x, int x_dtype, const void *const *expert_tab, int64_t E, const int64_t *topk_ids,
                const float *weights, void *y, int64_t T, int topk, int64_t H, int64_t I, int G, int act, void *ws,
                size_t ws_bytes, hq_stream_t stream) {
  const char *call = "hq_moe_int4";
  if (x_dtype != HQ_F32 && x_dtype != HQ_BF16 && x_dtype != HQ_F16)
    return fail(HQ_EUNSUPPORTED, call, "activations dtype %d, want F32, BF16 or F16", x_dtype);
  if (act != HQ_ACT_SILU && act != HQ_ACT_GELU_ERF) return fail(HQ_EINVAL, call, "activation %d", act);
  if (E < 1 || T < 0 || topk < 1 || H <= 0 || I <= 0 || G <= 0)
    return fail(HQ_EINVAL, call, "x (%lld, %lld), %lld experts, topk %d, I %lld, group %d", (long long)T,
                (long long)H, (long long)E, topk, (long long)I, G);
  if (H % G || I % G || H % 8 || I % 8)
    return fail(HQ_EINVAL, call, "group %d must divide hidden %lld and intermediate %lld (multiples of 8)", G,
                (long long)H, (long long)I);
  if (T == 0) return HQ_OK;
  if (!x || !expert_tab || !topk_ids || !weights || !y) return fail(HQ_EINVAL, call, "NULL pointer");
  if (((uintptr_t)x & 15) || ((uintptr_t)y & 3)) return fail(HQ_EINVAL, call, "x must be 16-byte aligned");
  hipStream_t s = resolve(stream);
  const size_t need = moe_int4_ws_bytes(T, topk, I);
  if (!ws) {
    if (int rc = workspace(need, s, &ws, call)) return rc;
  } else if (ws_bytes < need) {
    return fail(HQ_ENOMEM, call, "workspace %zu bytes < %zu needed", ws_bytes, need);
  }
  TraceSpan span("moe_int4", s);
  return launch_moe_int4(x, x_dtype, expert_tab, E, topk_ids, weights, y, T, topk, H, I, G, act, ws, s);
}

int hq_gather_cols(const void *x, const int64_t *idx, void *y, int64_t M, int64_t K, int elem_bytes,
                   hq_stream_t stream) {
  const char *call = "hq_gather_cols";
  if (elem_bytes != 2 && elem_bytes != 4) return fail(HQ_EINVAL, call, "element size %d", elem_bytes);
  if (M < 0 || K < 0) return fail(HQ_EINVAL, call, "bad shape");
  if (M == 0 || K == 0) return HQ_OK;
  if (!x || !idx || !y) return fail(HQ_EINVAL, call, "NULL pointer");
  hipStream_t s = resolve(stream);
  return launch_gather_cols(x, idx, y, M, K, elem_bytes, s);
}

}  // extern "C"
