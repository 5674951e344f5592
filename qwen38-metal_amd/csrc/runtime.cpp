// qm38 C-ABI runtime: object lifetimes, argument validation and kernel
// dispatch.  Mirrors the entry points of MetalRuntime
// (/root/reference/src/metal_runtime.rs); each function below cites the one it
// replaces in include/qm38.h.
#include "runtime_internal.h"

#include <stdarg.h>
#include <stdio.h>
#include <stdlib.h>
#include <string.h>

#include <string>

using namespace qm;

namespace {
thread_local std::string g_last_error;
}

qm_status qm::fail(qm_status status, const char* fmt, ...) {
  char buf[512];
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(buf, sizeof(buf), fmt, ap);
  va_end(ap);
  g_last_error = std::string(qm_status_string(status)) + ": " + buf;
  return status;
}

qm_status qm::hip_check(hipError_t err, const char* what) {
  if (err == hipSuccess) return QM_OK;
  // Reported here; cleared so that a later launch's hipGetLastError() does
  // not see it again.
  (void)hipGetLastError();
  if (err == hipErrorOutOfMemory) return fail(QM_ERR_OUT_OF_MEMORY, "%s: %s", what, hipGetErrorString(err));
  return fail(QM_ERR_COMMAND_FAILED, "%s: %s", what, hipGetErrorString(err));
}

qm::DeviceGuard::DeviceGuard(int device) {
  dev_ = device;
  if (device < 0) {  // a runtime without a device (argument checks only)
    prev_ = device;
    return;
  }
  if (hipGetDevice(&prev_) != hipSuccess) prev_ = -1;
  ok_ = prev_ == device || hipSetDevice(device) == hipSuccess;
  if (!ok_) (void)hipGetLastError();  // the caller reports QM_ERR_NO_DEVICE
}
qm::DeviceGuard::~DeviceGuard() {
  if (ok_ && prev_ >= 0 && prev_ != dev_) (void)hipSetDevice(prev_);
}

qm_status qm::no_device() {
  return fail(QM_ERR_NO_DEVICE, "this runtime has no usable device (created with QM_DEVICE_NONE = %d, or its "
                                "device could not be made current)", QM_DEVICE_NONE);
}

// Growing a buffer allocates and synchronises, which a stream under graph
// capture cannot do: such a call fails instead of corrupting the capture.
static qm_status capture_guard(qm_runtime* rt, const char* what) {
  if (qm::stream_capturing(rt->stream))
    return qm::fail(QM_ERR_INVALID_ARGUMENT, "%s: workspace must grow while the stream is being captured", what);
  return QM_OK;
}

qm_status qm::ensure_scratch(qm_runtime* rt, size_t bytes) {
  if (rt->scratch_bytes >= bytes) return QM_OK;
  if (rt->device < 0) return no_device();
  if (qm_status st_cap = capture_guard(rt, "ensure_scratch"); st_cap != QM_OK) return st_cap;
  if (rt->scratch) {
    // Work already enqueued may still use the old buffer.
    hipError_t e = hipStreamSynchronize(rt->stream);
    if (e != hipSuccess) return hip_check(e, "scratch resize sync");
    (void)hipFree(rt->scratch);
    rt->scratch = nullptr;
    rt->scratch_bytes = 0;
  }
  size_t want = bytes < (1u << 20) ? (1u << 20) : bytes;
  want = (want + 255) & ~size_t(255);
  hipError_t e = hipMalloc(&rt->scratch, want);
  if (e != hipSuccess) return hip_check(e, "scratch hipMalloc");
  rt->scratch_bytes = want;
  return QM_OK;
}

qm_status qm::ensure_partials(qm_runtime* rt, size_t bytes) {
  if (rt->partial_bytes >= bytes) return QM_OK;
  if (rt->device < 0) return no_device();
  if (qm_status st_cap = capture_guard(rt, "ensure_partials"); st_cap != QM_OK) return st_cap;
  if (rt->partials) {
    hipError_t e = hipStreamSynchronize(rt->stream);
    if (e != hipSuccess) return hip_check(e, "partials resize sync");
    (void)hipFree(rt->partials);
    rt->partials = nullptr;
    rt->partial_bytes = 0;
  }
  size_t want = bytes < (1u << 20) ? (1u << 20) : bytes;
  want = (want + 255) & ~size_t(255);
  hipError_t e = hipMalloc(&rt->partials, want);
  if (e != hipSuccess) return hip_check(e, "partials hipMalloc");
  rt->partial_bytes = want;
  return QM_OK;
}

qm_status qm::ensure_xh(qm_runtime* rt, size_t bytes) {
  if (rt->xh_bytes >= bytes) return QM_OK;
  if (rt->device < 0) return no_device();
  if (qm_status st_cap = capture_guard(rt, "ensure_xh"); st_cap != QM_OK) return st_cap;
  if (rt->xh) {
    hipError_t e = hipStreamSynchronize(rt->stream);
    if (e != hipSuccess) return hip_check(e, "xh resize sync");
    (void)hipFree(rt->xh);
    rt->xh = nullptr;
    rt->xh_bytes = 0;
  }
  const size_t want = (bytes + 255) & ~size_t(255);
  hipError_t e = hipMalloc(&rt->xh, want);
  if (e != hipSuccess) return hip_check(e, "xh hipMalloc");
  rt->xh_bytes = want;
  return QM_OK;
}

qm_status qm::ensure_counters(qm_runtime* rt, size_t count) {
  if (rt->counter_count >= count) return QM_OK;
  if (rt->device < 0) return no_device();
  if (qm_status st_cap = capture_guard(rt, "ensure_counters"); st_cap != QM_OK) return st_cap;
  if (rt->counters) {
    hipError_t e = hipStreamSynchronize(rt->stream);
    if (e != hipSuccess) return hip_check(e, "counters resize sync");
    (void)hipFree(rt->counters);
    rt->counters = nullptr;
    rt->counter_count = 0;
  }
  size_t want = count < 4096 ? 4096 : count;
  hipError_t e = hipMalloc(&rt->counters, want * sizeof(unsigned int));
  if (e != hipSuccess) return hip_check(e, "counters hipMalloc");
  // Counters start at zero once; every kernel that uses them resets them.
  e = hipMemsetAsync(rt->counters, 0, want * sizeof(unsigned int), rt->stream);
  if (e == hipSuccess) e = hipStreamSynchronize(rt->stream);
  if (e != hipSuccess) return hip_check(e, "counters clear");
  rt->counter_count = want;
  return QM_OK;
}

bool qm::stream_capturing(hipStream_t s) {
  hipStreamCaptureStatus cs = hipStreamCaptureStatusNone;
  if (hipStreamIsCapturing(s, &cs) != hipSuccess) {
    // The legacy stream cannot be queried while another blocking stream is
    // capturing; the query's error must not reach a later launch's check.
    (void)hipGetLastError();
    return true;
  }
  return cs != hipStreamCaptureStatusNone;
}

qm_status qm::stream_after(qm_runtime* waiter, qm_runtime* signaler) {
  if (!waiter || !signaler || waiter == signaler || waiter->stream == signaler->stream) return QM_OK;
  if (waiter->device < 0 || signaler->device < 0) return QM_OK;
  if (stream_capturing(waiter->stream) || stream_capturing(signaler->stream)) return QM_OK;
  if (!signaler->order_event) {
    hipError_t e = hipEventCreateWithFlags(&signaler->order_event, hipEventDisableTiming);
    if (e != hipSuccess) return hip_check(e, "stream order event");
  }
  hipError_t e = hipEventRecord(signaler->order_event, signaler->stream);
  if (e == hipSuccess) e = hipStreamWaitEvent(waiter->stream, signaler->order_event, 0);
  return hip_check(e, "stream order");
}

qm_status qm::ensure_keys(qm_runtime* rt) {
  if (rt->keys) return QM_OK;
  if (rt->device < 0) return no_device();
  if (qm_status st_cap = capture_guard(rt, "ensure_keys"); st_cap != QM_OK) return st_cap;
  const size_t bytes = 16 * sizeof(unsigned long long);
  hipError_t e = hipMalloc(&rt->keys, bytes);
  if (e == hipSuccess) e = hipMemsetAsync(rt->keys, 0, bytes, rt->stream);
  if (e == hipSuccess) e = hipStreamSynchronize(rt->stream);
  if (e != hipSuccess) {
    if (rt->keys) (void)hipFree(rt->keys);
    rt->keys = nullptr;
    return hip_check(e, "argmax keys");
  }
  return QM_OK;
}

void qm::release_buffers(qm_runtime* rt) {
  if (rt->scratch) (void)hipFree(rt->scratch);
  if (rt->counters) (void)hipFree(rt->counters);
  if (rt->partials) (void)hipFree(rt->partials);
  if (rt->xh) (void)hipFree(rt->xh);
  if (rt->keys) (void)hipFree(rt->keys);
  rt->keys = nullptr;
  rt->scratch = rt->counters = nullptr;
  rt->partials = rt->xh = nullptr;
  rt->scratch_bytes = rt->counter_count = rt->partial_bytes = rt->xh_bytes = 0;
}

qm::Workspace qm::workspace(qm_runtime* rt) {
  return Workspace{(float*)rt->partials, rt->partial_bytes, rt->counters, rt->counter_count, (uint16_t*)rt->xh,
                   rt->xh_bytes, &rt->tune};
}

qm::Tuning qm::read_tuning(int cu_count) {
  auto get = [](const char* name, int fallback) {
    const char* v = getenv(name);
    return v ? atoi(v) : fallback;
  };
  Tuning t{};
  t.cus = cu_count;
  t.q4_nt = get("QM38_Q4_NT", 0);
  t.q4_xstage = get("QM38_Q4_XSTAGE", 1);
  t.q4_xstage_max = get("QM38_Q4_XSTAGE_MAX", 0);
  t.q4_target_waves = get("QM38_Q4_TARGET_WAVES", 0);
  t.q4_rpw = get("QM38_Q4_RPW", 0);
  t.q4_split = get("QM38_Q4_SPLIT", 0);
  t.q4_plan_log = get("QM38_Q4_PLAN_LOG", 0);
  t.q4_fuse = get("QM38_Q4_FUSE", 1);
  t.q4_stream = get("QM38_Q4_STREAM", 1);
  t.q4_stream_wgs = get("QM38_Q4_STREAM_WGS", 0);
  t.q4_stream_rows = get("QM38_Q4_STREAM_ROWS", 2);
  t.q4_stream_mw = get("QM38_Q4_STREAM_MW", 0);
  t.q4_stream_c = get("QM38_Q4_STREAM_C", 0);
  t.q4_stream_w = get("QM38_Q4_STREAM_W", 0);
  t.q4_mma_lo = get("QM38_Q4_MMA_LO", 3);
  t.q4_mma_hi = get("QM38_Q4_MMA_HI", 4);
  t.q4_mma_k = get("QM38_Q4_MMA_K", 8192);
  t.q4_mma_w = get("QM38_Q4_MMA_W", 0);
  t.q4_mma_c = get("QM38_Q4_MMA_C", 0);
  t.q4_mma_sb = get("QM38_Q4_MMA_SB", 0);
  t.q4_mma_wgs = get("QM38_Q4_MMA_WGS", 0);
  t.gemm_splits = get("QM38_GEMM_SPLITS", 0);
  t.gemm_q = get("QM38_GEMM_Q", 0);
  t.gemm_plan_log = get("QM38_GEMM_PLAN_LOG", 0);
  t.attn_pps = get("QM38_ATTN_PPS", 0);
  t.attn_waves = get("QM38_ATTN_WAVES", 0);
  t.attn_target_wgs = get("QM38_ATTN_TARGET_WGS", 0);
  t.prefill_cb = get("QM38_PREFILL_CB", 0);
  t.dn_step_head = get("QM38_DN_STEP_HEAD", -1);
  t.dn_chunked = get("QM38_DN_CHUNKED", -1);
  t.dn_pair = get("QM38_DN_PAIR", -1);
  return t;
}

extern "C" {

const char* qm_status_string(qm_status status) {
  switch (status) {
    case QM_OK: return "QM_OK";
    case QM_ERR_NO_DEVICE: return "QM_ERR_NO_DEVICE";
    case QM_ERR_EMPTY_DIMENSION: return "QM_ERR_EMPTY_DIMENSION";
    case QM_ERR_INPUT_NOT_GROUPED: return "QM_ERR_INPUT_NOT_GROUPED";
    case QM_ERR_WRONG_LENGTH: return "QM_ERR_WRONG_LENGTH";
    case QM_ERR_INVALID_DELTANET_CONFIG: return "QM_ERR_INVALID_DELTANET_CONFIG";
    case QM_ERR_INVALID_ATTENTION_SHAPE: return "QM_ERR_INVALID_ATTENTION_SHAPE";
    case QM_ERR_INVALID_SEQUENCE_LENGTH: return "QM_ERR_INVALID_SEQUENCE_LENGTH";
    case QM_ERR_INVALID_BUFFER_OFFSET: return "QM_ERR_INVALID_BUFFER_OFFSET";
    case QM_ERR_MAPPED_TENSOR_OUT_OF_RANGE: return "QM_ERR_MAPPED_TENSOR_OUT_OF_RANGE";
    case QM_ERR_DIMENSION_OVERFLOW: return "QM_ERR_DIMENSION_OVERFLOW";
    case QM_ERR_COMMAND_FAILED: return "QM_ERR_COMMAND_FAILED";
    case QM_ERR_ZERO_CAPACITY: return "QM_ERR_ZERO_CAPACITY";
    case QM_ERR_EMPTY_APPEND: return "QM_ERR_EMPTY_APPEND";
    case QM_ERR_CAPACITY_EXCEEDED: return "QM_ERR_CAPACITY_EXCEEDED";
    case QM_ERR_NULL_POINTER: return "QM_ERR_NULL_POINTER";
    case QM_ERR_OUT_OF_MEMORY: return "QM_ERR_OUT_OF_MEMORY";
    case QM_ERR_MISALIGNED: return "QM_ERR_MISALIGNED";
    case QM_ERR_INVALID_ARGUMENT: return "QM_ERR_INVALID_ARGUMENT";
    case QM_ERR_INVALID_SNAPSHOT: return "QM_ERR_INVALID_SNAPSHOT";
    case QM_ERR_INVALID_SNAPSHOT_ROW: return "QM_ERR_INVALID_SNAPSHOT_ROW";
    case QM_ERR_MODEL_FORMAT: return "QM_ERR_MODEL_FORMAT";
    case QM_ERR_INVALID_TENSOR: return "QM_ERR_INVALID_TENSOR";
    case QM_ERR_GRAPH_STALE: return "QM_ERR_GRAPH_STALE";
  }
  return "QM_ERR_UNKNOWN";
}

const char* qm_last_error_message(void) { return g_last_error.c_str(); }

qm_status qm_runtime_create(int device, qm_runtime** out) {
  if (!out) return fail(QM_ERR_NULL_POINTER, "out is NULL");
  *out = nullptr;
  if (device == QM_DEVICE_NONE) {
    qm_runtime* rt = new qm_runtime();
    rt->device = QM_DEVICE_NONE;
    rt->tune = read_tuning(rt->cu_count);
    *out = rt;
    return QM_OK;
  }
  int count = 0;
  if (hipGetDeviceCount(&count) != hipSuccess || count <= 0)
    return fail(QM_ERR_NO_DEVICE, "no HIP device is available");
  if (device < 0 || device >= count)
    return fail(QM_ERR_NO_DEVICE, "device %d out of range (%d devices)", device, count);
  qm_runtime* rt = new qm_runtime();
  rt->device = device;
  DeviceGuard g(device);
  if (!g.ok()) return no_device();
  hipDeviceProp_t prop;
  if (hipGetDeviceProperties(&prop, device) == hipSuccess) rt->cu_count = prop.multiProcessorCount;
  rt->tune = read_tuning(rt->cu_count);
  *out = rt;
  return QM_OK;
}

void qm_runtime_destroy(qm_runtime* rt) {
  if (!rt) return;
  if (rt->device < 0) {
    delete rt;
    return;
  }
  DeviceGuard g(rt->device);
  (void)hipStreamSynchronize(rt->stream);
  qm::release_buffers(rt);
  if (rt->order_event) (void)hipEventDestroy(rt->order_event);
  delete rt;
}

qm_status qm_runtime_set_stream(qm_runtime* rt, void* hip_stream) {
  if (!rt) return fail(QM_ERR_NULL_POINTER, "runtime is NULL");
  rt->stream = (hipStream_t)hip_stream;
  return QM_OK;
}

qm_status qm_runtime_synchronize(qm_runtime* rt) {
  if (!rt) return fail(QM_ERR_NULL_POINTER, "runtime is NULL");
  DeviceGuard g(rt->device);
  if (!g.ok()) return no_device();
  return hip_check(hipStreamSynchronize(rt->stream), "stream synchronize");
}

qm_status qm_device_alloc(qm_runtime* rt, size_t bytes, void** out) {
  if (!rt || !out) return fail(QM_ERR_NULL_POINTER, "runtime/out is NULL");
  if (bytes == 0) return fail(QM_ERR_EMPTY_DIMENSION, "zero-byte allocation");
  DeviceGuard g(rt->device);
  if (!g.ok()) return no_device();
  return hip_check(hipMalloc(out, bytes), "hipMalloc");
}

qm_status qm_device_free(qm_runtime* rt, void* ptr) {
  if (!rt) return fail(QM_ERR_NULL_POINTER, "runtime is NULL");
  if (!ptr) return QM_OK;
  DeviceGuard g(rt->device);
  if (!g.ok()) return no_device();
  return hip_check(hipFree(ptr), "hipFree");
}

qm_status qm_upload(qm_runtime* rt, const void* host, size_t bytes, void** out) {
  if (!host) return fail(QM_ERR_NULL_POINTER, "host pointer is NULL");
  qm_status st = qm_device_alloc(rt, bytes, out);
  if (st != QM_OK) return st;
  return qm_copy_to_device(rt, *out, host, bytes);
}

qm_status qm_copy_to_device(qm_runtime* rt, void* dst, const void* host, size_t bytes) {
  if (!rt || !dst || !host) return fail(QM_ERR_NULL_POINTER, "NULL argument");
  DeviceGuard g(rt->device);
  if (!g.ok()) return no_device();
  qm_status st = hip_check(hipMemcpyAsync(dst, host, bytes, hipMemcpyHostToDevice, rt->stream), "H2D copy");
  if (st != QM_OK) return st;
  return hip_check(hipStreamSynchronize(rt->stream), "H2D sync");
}

qm_status qm_copy_to_host(qm_runtime* rt, void* host, const void* src, size_t bytes) {
  if (!rt || !src || !host) return fail(QM_ERR_NULL_POINTER, "NULL argument");
  DeviceGuard g(rt->device);
  if (!g.ok()) return no_device();
  qm_status st = hip_check(hipMemcpyAsync(host, src, bytes, hipMemcpyDeviceToHost, rt->stream), "D2H copy");
  if (st != QM_OK) return st;
  return hip_check(hipStreamSynchronize(rt->stream), "D2H sync");
}

}  // extern "C"
