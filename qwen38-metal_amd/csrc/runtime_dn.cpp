// C-ABI entry points of the Gated DeltaNet layer (see include/qm38.h).
#include <stdint.h>
#include <string.h>

#include "deltanet.h"
#include "runtime_internal.h"

using namespace qm;

struct qm_dn_weights {
  qm_runtime* rt = nullptr;
  qm_dn_config cfg{};
  uint32_t channels = 0;
  float* conv_w = nullptr;
  float* a_log = nullptr;
  float* dt_bias = nullptr;
  float* norm = nullptr;
};

// The conv history is double-buffered (hist[cur] is current); see deltanet.hip.
struct qm_dn_state {
  qm_runtime* rt = nullptr;
  qm_dn_config cfg{};
  uint32_t channels = 0;
  size_t hist_elems = 0;  // channels * (kernel - 1)
  size_t rec_elems = 0;   // VH * dv * dk
  float* hist[2] = {nullptr, nullptr};
  int cur = 0;
  float* rec = nullptr;
};

// Verification images: hist [rows][max(hist_elems, 1)], rec [rows][rec_elems].
struct qm_dn_snapshots {
  qm_runtime* rt = nullptr;
  qm_dn_config cfg{};
  uint32_t rows = 0;
  size_t hist_elems = 0, hist_stride = 0, rec_elems = 0;
  float* hist = nullptr;
  float* rec = nullptr;
};

namespace {

// validate_deltanet_config (metal_runtime.rs:9151-9168).
qm_status validate_config(const qm_dn_config* c) {
  if (c->key_heads == 0 || c->value_heads == 0 || c->key_head_dim == 0 || c->value_head_dim == 0 ||
      c->conv_kernel_size == 0 || c->value_heads % c->key_heads != 0 || c->key_head_dim > 256 ||
      c->value_head_dim > 256)
    return fail(QM_ERR_INVALID_DELTANET_CONFIG,
                "heads and dimensions must be non-zero, value heads must divide by key heads, and head dimensions "
                "must fit one GPU threadgroup");
  const uint64_t channels =
      2ull * c->key_heads * c->key_head_dim + (uint64_t)c->value_heads * c->value_head_dim;
  if (channels > 0xFFFFFFFFull || channels * c->conv_kernel_size > 0xFFFFFFFFull)
    return fail(QM_ERR_DIMENSION_OVERFLOW, "DeltaNet channel count");
  return QM_OK;
}

uint32_t channels_of(const qm_dn_config& c) {
  return 2 * c.key_heads * c.key_head_dim + c.value_heads * c.value_head_dim;
}

void free_weights(qm_dn_weights* w) {
  DeviceGuard g(w->rt->device);
  (void)hipFree(w->conv_w);
  (void)hipFree(w->a_log);
  (void)hipFree(w->dt_bias);
  (void)hipFree(w->norm);
  delete w;
}

void free_state(qm_dn_state* s) {
  DeviceGuard g(s->rt->device);
  (void)hipFree(s->hist[0]);
  (void)hipFree(s->hist[1]);
  (void)hipFree(s->rec);
  delete s;
}

qm_status alloc_state(qm_runtime* rt, const qm_dn_config& cfg, qm_dn_state** out) {
  qm_dn_state* s = new qm_dn_state();
  s->rt = rt;
  s->cfg = cfg;
  s->channels = channels_of(cfg);
  s->hist_elems = (size_t)s->channels * (cfg.conv_kernel_size - 1);
  s->rec_elems = (size_t)cfg.value_heads * cfg.value_head_dim * cfg.key_head_dim;
  // A one-element history keeps the pointers valid for a kernel-size-one model.
  const size_t hb = (s->hist_elems ? s->hist_elems : 1) * sizeof(float);
  DeviceGuard g(rt->device);
  if (!g.ok()) {
    delete s;
    return no_device();
  }
  hipError_t e = hipMalloc(&s->hist[0], hb);
  if (e == hipSuccess) e = hipMalloc(&s->hist[1], hb);
  if (e == hipSuccess) e = hipMalloc(&s->rec, s->rec_elems * sizeof(float));
  if (e == hipSuccess) e = hipMemsetAsync(s->hist[0], 0, hb, rt->stream);
  if (e == hipSuccess) e = hipMemsetAsync(s->hist[1], 0, hb, rt->stream);
  if (e == hipSuccess) e = hipMemsetAsync(s->rec, 0, s->rec_elems * sizeof(float), rt->stream);
  if (e == hipSuccess) e = hipStreamSynchronize(rt->stream);
  if (e != hipSuccess) {
    free_state(s);
    return hip_check(e, "DeltaNet state allocation");
  }
  *out = s;
  return QM_OK;
}

qm_status run(qm_runtime* rt, const qm_dn_weights* w, const qm_dn_state* from, qm_dn_state* to, const float* qkv,
              const float* z, const float* b, const float* a, uint32_t M, float eps, float* out,
              qm_dn_snapshots* snaps = nullptr, uint16_t* out_bf16 = nullptr) {
  if (!rt || !w || !to || !qkv || !z || !b || !a || !out) return fail(QM_ERR_NULL_POINTER, "NULL argument");
  if (!from) from = to;
  if (M == 0) return fail(QM_ERR_EMPTY_DIMENSION, "DeltaNet prefill needs at least one token");
  // Token-major rows are indexed with 32-bit element counts in places (the
  // gate norm's rows, the bf16 copy): keep M x channels within int32.
  if ((uint64_t)M * w->channels > 0x7FFFFFFFull)
    return fail(QM_ERR_DIMENSION_OVERFLOW, "DeltaNet prefill of %u tokens x %u channels exceeds the runtime limit", M,
                w->channels);
  // Weights and states are device memory: any runtime on their device may use them.
  if (w->rt->device != rt->device || from->rt->device != rt->device || to->rt->device != rt->device)
    return fail(QM_ERR_INVALID_ARGUMENT, "weights and states must live on this runtime's device");
  if (memcmp(&from->cfg, &w->cfg, sizeof(qm_dn_config)) != 0 || memcmp(&to->cfg, &w->cfg, sizeof(qm_dn_config)) != 0)
    return fail(QM_ERR_WRONG_LENGTH, "DeltaNet state was created for another configuration");
  if (snaps) {
    if (snaps->rt != rt || memcmp(&snaps->cfg, &w->cfg, sizeof(qm_dn_config)) != 0 || M - 1 > snaps->rows)
      return fail(QM_ERR_INVALID_SNAPSHOT, "snapshot set has %u rows for a %u-row verification (or another model)",
                  snaps->rows, M);
  }
  const qm_dn_config& c = w->cfg;
  const size_t conv_bytes = ((size_t)M * w->channels * sizeof(float) + 255) & ~size_t(255);
  DnArgs d{};
  d.key_heads = c.key_heads;
  d.value_heads = c.value_heads;
  d.dk = c.key_head_dim;
  d.dv = c.value_head_dim;
  d.kernel = c.conv_kernel_size;
  d.channels = w->channels;
  d.M = M;
  d.eps = eps;
  d.tune_step_head = rt->tune.dn_step_head;
  d.tune_chunked = rt->tune.dn_chunked;
  d.tune_dn_pair = rt->tune.dn_pair;
  d.conv_w = w->conv_w;
  d.a_log = w->a_log;
  d.dt_bias = w->dt_bias;
  d.norm = w->norm;
  d.qkv = qkv;
  d.z = z;
  d.b = b;
  d.a = a;
  // New history goes to the buffer that is not being read.
  const int next = from == to ? 1 - from->cur : to->cur;
  d.hist_in = from->hist[from->cur];
  d.hist_out = to->hist[next];
  d.s_in = from->rec;
  d.s_out = to->rec;
  if (snaps && M > 1) d.snap_rows = M - 1;  // decides the path below
  const size_t chunk_bytes = dn_use_chunked(d) ? dn_chunk_ws_bytes(M, c.value_heads) : 0;
  const size_t step_bytes = dn_step_split(d) ? ((size_t)c.value_heads * c.value_head_dim * 4 + 255) & ~size_t(255) : 0;
  qm_status st = ensure_scratch(rt, conv_bytes + chunk_bytes + step_bytes);
  if (st == QM_OK && step_bytes) st = ensure_counters(rt, c.value_heads);
  if (st != QM_OK) return st;
  d.conv_out = (float*)rt->scratch;
  d.chunk_ws = chunk_bytes ? (float*)((char*)rt->scratch + conv_bytes) : nullptr;
  d.step_o = step_bytes ? (float*)((char*)rt->scratch + conv_bytes + chunk_bytes) : nullptr;
  d.step_ctr = step_bytes ? rt->counters : nullptr;
  d.out = out;
  // The single-token kernels also write the bf16 copy; other paths
  // convert afterwards.
  const bool fused_bf16 = out_bf16 && M == 1 && c.key_head_dim <= 128 && c.value_head_dim <= 128;
  if (fused_bf16) d.out_bf16 = out_bf16;
  if (snaps && M > 1) {
    d.snap_hist = snaps->hist;
    d.snap_s = snaps->rec;
    d.snap_rows = M - 1;
    d.snap_hist_stride = snaps->hist_stride;
    d.snap_s_stride = snaps->rec_elems;
  }
  DeviceGuard g(rt->device);
  if (!g.ok()) return no_device();
  // States owned by another runtime: their pending work on that runtime's
  // stream comes first, and later work there sees this call's result.
  if ((st = stream_after(rt, from->rt)) != QM_OK || (st = stream_after(rt, to->rt)) != QM_OK) return st;
  hipError_t e = launch_deltanet(d, rt->stream);
  if (e != hipSuccess) return hip_check(e, "DeltaNet launch");
  if (out_bf16 && !fused_bf16) {
    const ConvSeg seg{out, out_bf16, M * c.value_heads * c.value_head_dim, 0};
    if ((e = launch_convert(&seg, 1, rt->stream)) != hipSuccess) return hip_check(e, "DeltaNet bf16 output");
  }
  if (c.conv_kernel_size > 1) to->cur = next;
  return stream_after(to->rt, rt);
}

}  // namespace

size_t qm::dn_step_scratch_bytes(const qm_dn_config& c) {
  const size_t channels = 2ull * c.key_heads * c.key_head_dim + (size_t)c.value_heads * c.value_head_dim;
  return ((channels * 4 + 255) & ~size_t(255)) + (((size_t)c.value_heads * c.value_head_dim * 4 + 255) & ~size_t(255));
}

qm_status qm::dn_step_bf16(qm_runtime* rt, const qm_dn_weights* w, qm_dn_state* st, const float* qkv, const float* z,
                           const float* b, const float* a, float eps, float* out, uint16_t* out_bf16) {
  if (!out_bf16) return fail(QM_ERR_NULL_POINTER, "bf16 output is NULL");
  return run(rt, w, st, st, qkv, z, b, a, 1, eps, out, nullptr, out_bf16);
}

const qm_dn_config& qm::dn_weights_config(const qm_dn_weights* w) { return w->cfg; }
const qm_runtime* qm::dn_weights_runtime(const qm_dn_weights* w) { return w->rt; }
qm::DnStateView qm::dn_state_view(const qm_dn_state* s) {
  return DnStateView{s->hist[0], s->hist[1], s->rec, s->cur, s->rt, s->cfg};
}
void qm::dn_state_set_cur(qm_dn_state* s, int cur) { s->cur = cur; }

extern "C" {

qm_status qm_dn_weights_create(qm_runtime* rt, const qm_dn_config* cfg, const float* conv_weight,
                               const float* a_log, const float* dt_bias, const float* norm, qm_dn_weights** out) {
  if (!rt || !cfg || !conv_weight || !a_log || !dt_bias || !norm || !out)
    return fail(QM_ERR_NULL_POINTER, "NULL argument");
  *out = nullptr;
  qm_status st = validate_config(cfg);
  if (st != QM_OK) return st;
  qm_dn_weights* w = new qm_dn_weights();
  w->rt = rt;
  w->cfg = *cfg;
  w->channels = channels_of(*cfg);
  const size_t nconv = (size_t)w->channels * cfg->conv_kernel_size;
  DeviceGuard g(rt->device);
  if (!g.ok()) {
    delete w;
    return no_device();
  }
  hipError_t e = hipMalloc(&w->conv_w, nconv * 4);
  if (e == hipSuccess) e = hipMalloc(&w->a_log, cfg->value_heads * 4);
  if (e == hipSuccess) e = hipMalloc(&w->dt_bias, cfg->value_heads * 4);
  if (e == hipSuccess) e = hipMalloc(&w->norm, cfg->value_head_dim * 4);
  if (e == hipSuccess) e = hipMemcpyAsync(w->conv_w, conv_weight, nconv * 4, hipMemcpyHostToDevice, rt->stream);
  if (e == hipSuccess)
    e = hipMemcpyAsync(w->a_log, a_log, cfg->value_heads * 4, hipMemcpyHostToDevice, rt->stream);
  if (e == hipSuccess)
    e = hipMemcpyAsync(w->dt_bias, dt_bias, cfg->value_heads * 4, hipMemcpyHostToDevice, rt->stream);
  if (e == hipSuccess)
    e = hipMemcpyAsync(w->norm, norm, cfg->value_head_dim * 4, hipMemcpyHostToDevice, rt->stream);
  if (e == hipSuccess) e = hipStreamSynchronize(rt->stream);
  if (e != hipSuccess) {
    free_weights(w);
    return hip_check(e, "DeltaNet weight upload");
  }
  *out = w;
  return QM_OK;
}

void qm_dn_weights_destroy(qm_dn_weights* w) {
  if (!w) return;
  (void)hipStreamSynchronize(w->rt->stream);
  free_weights(w);
}

qm_status qm_dn_state_create(qm_runtime* rt, const qm_dn_weights* w, qm_dn_state** out) {
  if (!rt || !w || !out) return fail(QM_ERR_NULL_POINTER, "NULL argument");
  *out = nullptr;
  return alloc_state(rt, w->cfg, out);
}

void qm_dn_state_destroy(qm_dn_state* s) {
  if (!s) return;
  (void)hipStreamSynchronize(s->rt->stream);
  free_state(s);
}

qm_status qm_dn_state_clone(const qm_dn_state* src, qm_dn_state** out) {
  if (!src || !out) return fail(QM_ERR_NULL_POINTER, "NULL argument");
  *out = nullptr;
  qm_dn_state* s = nullptr;
  qm_status st = alloc_state(src->rt, src->cfg, &s);
  if (st != QM_OK) return st;
  DeviceGuard g(src->rt->device);
  if (!g.ok()) return no_device();
  hipStream_t stream = src->rt->stream;
  hipError_t e = hipSuccess;
  if (src->hist_elems)
    e = hipMemcpyAsync(s->hist[0], src->hist[src->cur], src->hist_elems * 4, hipMemcpyDeviceToDevice, stream);
  if (e == hipSuccess) e = hipMemcpyAsync(s->rec, src->rec, src->rec_elems * 4, hipMemcpyDeviceToDevice, stream);
  if (e == hipSuccess) e = hipStreamSynchronize(stream);
  if (e != hipSuccess) {
    free_state(s);
    return hip_check(e, "DeltaNet state clone");
  }
  *out = s;
  return QM_OK;
}

qm_status qm_dn_state_read(const qm_dn_state* s, float* conv_history, float* recurrent) {
  if (!s) return fail(QM_ERR_NULL_POINTER, "state is NULL");
  DeviceGuard g(s->rt->device);
  if (!g.ok()) return no_device();
  hipStream_t stream = s->rt->stream;
  hipError_t e = hipSuccess;
  if (conv_history && s->hist_elems)
    e = hipMemcpyAsync(conv_history, s->hist[s->cur], s->hist_elems * 4, hipMemcpyDeviceToHost, stream);
  if (e == hipSuccess && recurrent)
    e = hipMemcpyAsync(recurrent, s->rec, s->rec_elems * 4, hipMemcpyDeviceToHost, stream);
  if (e == hipSuccess) e = hipStreamSynchronize(stream);
  return hip_check(e, "DeltaNet state read");
}

qm_status qm_dn_state_write(qm_dn_state* s, const float* conv_history, const float* recurrent) {
  if (!s) return fail(QM_ERR_NULL_POINTER, "state is NULL");
  DeviceGuard g(s->rt->device);
  if (!g.ok()) return no_device();
  hipStream_t stream = s->rt->stream;
  hipError_t e = hipSuccess;
  if (conv_history && s->hist_elems)
    e = hipMemcpyAsync(s->hist[s->cur], conv_history, s->hist_elems * 4, hipMemcpyHostToDevice, stream);
  if (e == hipSuccess && recurrent)
    e = hipMemcpyAsync(s->rec, recurrent, s->rec_elems * 4, hipMemcpyHostToDevice, stream);
  if (e == hipSuccess) e = hipStreamSynchronize(stream);
  return hip_check(e, "DeltaNet state write");
}

qm_status qm_dn_step(qm_runtime* rt, const qm_dn_weights* w, qm_dn_state* st, const float* qkv, const float* z,
                     const float* b, const float* a, float epsilon, float* out) {
  return run(rt, w, st, st, qkv, z, b, a, 1, epsilon, out);
}

qm_status qm_dn_prefill(qm_runtime* rt, const qm_dn_weights* w, const qm_dn_state* from, qm_dn_state* to,
                        const float* qkv, const float* z, const float* b, const float* a, uint32_t M, float epsilon,
                        float* out) {
  return run(rt, w, from, to, qkv, z, b, a, M, epsilon, out);
}

qm_status qm_dn_snapshots_create(qm_runtime* rt, const qm_dn_weights* w, uint32_t rows, qm_dn_snapshots** out) {
  if (!rt || !w || !out) return fail(QM_ERR_NULL_POINTER, "NULL argument");
  *out = nullptr;
  if (rows == 0) return fail(QM_ERR_EMPTY_DIMENSION, "a snapshot set needs at least one row");
  if (w->rt != rt) return fail(QM_ERR_INVALID_ARGUMENT, "weights belong to another runtime");
  qm_dn_snapshots* s = new qm_dn_snapshots();
  s->rt = rt;
  s->cfg = w->cfg;
  s->rows = rows;
  s->hist_elems = (size_t)w->channels * (w->cfg.conv_kernel_size - 1);
  s->hist_stride = s->hist_elems ? s->hist_elems : 1;  // the state's buffer size, so one-row sets can swap
  s->rec_elems = (size_t)w->cfg.value_heads * w->cfg.value_head_dim * w->cfg.key_head_dim;
  DeviceGuard g(rt->device);
  if (!g.ok()) {
    delete s;
    return no_device();
  }
  hipError_t e = hipMalloc(&s->hist, (size_t)rows * s->hist_stride * sizeof(float));
  if (e == hipSuccess) e = hipMalloc(&s->rec, (size_t)rows * s->rec_elems * sizeof(float));
  if (e == hipSuccess) e = hipMemsetAsync(s->hist, 0, (size_t)rows * s->hist_stride * sizeof(float), rt->stream);
  if (e == hipSuccess) e = hipMemsetAsync(s->rec, 0, (size_t)rows * s->rec_elems * sizeof(float), rt->stream);
  if (e == hipSuccess) e = hipStreamSynchronize(rt->stream);
  if (e != hipSuccess) {
    (void)hipFree(s->hist);
    (void)hipFree(s->rec);
    delete s;
    return hip_check(e, "DeltaNet snapshot allocation");
  }
  *out = s;
  return QM_OK;
}

void qm_dn_snapshots_destroy(qm_dn_snapshots* s) {
  if (!s) return;
  DeviceGuard g(s->rt->device);
  (void)hipStreamSynchronize(s->rt->stream);
  (void)hipFree(s->hist);
  (void)hipFree(s->rec);
  delete s;
}

qm_status qm_dn_prefill_snapshots(qm_runtime* rt, const qm_dn_weights* w, const qm_dn_state* from, qm_dn_state* to,
                                  qm_dn_snapshots* snaps, const float* qkv, const float* z, const float* b,
                                  const float* a, uint32_t M, float epsilon, float* out) {
  if (!snaps) return fail(QM_ERR_NULL_POINTER, "snapshot set is NULL");
  return run(rt, w, from, to, qkv, z, b, a, M, epsilon, out, snaps);
}

qm_status qm_dn_snapshot_restore(qm_dn_snapshots* s, uint32_t row, qm_dn_state* dst) {
  if (!s || !dst) return fail(QM_ERR_NULL_POINTER, "NULL argument");
  if (row >= s->rows) return fail(QM_ERR_INVALID_SNAPSHOT_ROW, "row %u of a %u-row snapshot set", row, s->rows);
  if (dst->rt != s->rt || memcmp(&dst->cfg, &s->cfg, sizeof(qm_dn_config)) != 0)
    return fail(QM_ERR_INVALID_SNAPSHOT, "state and snapshot set belong to different models or runtimes");
  if (s->rows == 1) {
    // Same buffer sizes as the state's: later work on the stream uses the
    // exchanged pointers, earlier work already holds its own.
    float* h = dst->hist[dst->cur];
    dst->hist[dst->cur] = s->hist;
    s->hist = h;
    float* r = dst->rec;
    dst->rec = s->rec;
    s->rec = r;
    return QM_OK;
  }
  DeviceGuard g(s->rt->device);
  if (!g.ok()) return no_device();
  hipStream_t stream = s->rt->stream;
  hipError_t e = hipSuccess;
  if (s->hist_elems)
    e = hipMemcpyAsync(dst->hist[dst->cur], s->hist + (size_t)row * s->hist_stride, s->hist_elems * sizeof(float),
                       hipMemcpyDeviceToDevice, stream);
  if (e == hipSuccess)
    e = hipMemcpyAsync(dst->rec, s->rec + (size_t)row * s->rec_elems, s->rec_elems * sizeof(float),
                       hipMemcpyDeviceToDevice, stream);
  return hip_check(e, "DeltaNet snapshot restore");
}

}  // extern "C"
