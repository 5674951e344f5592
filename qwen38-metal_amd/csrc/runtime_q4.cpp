// C-ABI entry points of the MLX affine-Q4 projections (see include/qm38.h).
#include <stdint.h>
#include <stdio.h>

#include "runtime_internal.h"

using namespace qm;

namespace {

constexpr uint32_t kGroup = 64;       // AFFINE_GROUP_SIZE (metal_runtime.rs)
constexpr uint32_t kDecodeMaxRows = 16;
// Widest input: the kernels address a tile's rows (up to 256 rows of in/2
// bytes) with 32-bit offsets.
constexpr uint32_t kMaxInElems = 1u << 24;

bool aligned(const void* p, uintptr_t a) { return ((uintptr_t)p & (a - 1)) == 0; }

// validate_mapped_q4_affine_shape / MatvecShape::validate
// (metal_runtime.rs:8854-8898, 8932-8984) for device-resident jobs.
qm_status validate_job(const qm_q4_job* job, uint32_t in_elems, const char* name) {
  if (!job) return fail(QM_ERR_NULL_POINTER, "%s job is NULL", name);
  if (in_elems == 0 || job->out_rows == 0)
    return fail(QM_ERR_EMPTY_DIMENSION, "%s: matrix dimensions must be greater than zero", name);
  if (in_elems % kGroup != 0)
    return fail(QM_ERR_INPUT_NOT_GROUPED,
                "%s: input dimension %u is not divisible by affine group size %u", name, in_elems, kGroup);
  if (in_elems > kMaxInElems)
    return fail(QM_ERR_DIMENSION_OVERFLOW, "%s: input dimension %u exceeds the runtime limit %u", name, in_elems,
                kMaxInElems);
  if (!job->weights || !job->scales || !job->biases)
    return fail(QM_ERR_NULL_POINTER, "%s: weights/scales/biases pointer is NULL", name);
  if (!aligned(job->weights, 8) || !aligned(job->scales, 8) || !aligned(job->biases, 8))
    return fail(QM_ERR_MISALIGNED, "%s: weights/scales/biases must be 8-byte aligned", name);
  const uint64_t words = (uint64_t)job->out_rows * (in_elems / 8);
  if (words > (1ull << 40)) return fail(QM_ERR_DIMENSION_OVERFLOW, "%s: packed weight count exceeds runtime limits", name);
  return QM_OK;
}

// The allocation holding [p, p + bytes) must exist and be long enough: the
// device-pointer form of validate_mapped_q4_affine_shape's buffer checks
// (metal_runtime.rs:8868-8895).  A runtime without a device has no
// allocations to resolve and skips it.
qm_status check_range(const qm_runtime* rt, const void* p, uint64_t bytes, const char* what) {
  if (rt->device < 0) return QM_OK;
  // The lookup is not allowed while the stream is being captured (HIP treats
  // it as touching the legacy stream); captured calls were checked when the
  // capture's caller validated its jobs (qm_decode_graph_create does).
  if (stream_capturing(rt->stream)) return QM_OK;
  hipDeviceptr_t base = nullptr;
  size_t size = 0;
  if (hipMemGetAddressRange(&base, &size, (hipDeviceptr_t)p) != hipSuccess || !base) {
    (void)hipGetLastError();
    return fail(QM_ERR_INVALID_BUFFER_OFFSET, "%s (%p) lies inside no device allocation", what, p);
  }
  const uint64_t off = (uint64_t)((uintptr_t)p - (uintptr_t)base);
  if ((uintptr_t)p < (uintptr_t)base || off > size)
    return fail(QM_ERR_INVALID_BUFFER_OFFSET, "%s (%p) lies outside its allocation", what, p);
  if (bytes > size - off)
    return fail(QM_ERR_MAPPED_TENSOR_OUT_OF_RANGE,
                "%s needs %llu bytes but its allocation holds %llu past offset %llu", what,
                (unsigned long long)bytes, (unsigned long long)(size - off), (unsigned long long)off);
  return QM_OK;
}

}  // namespace

qm_status qm::q4_job_ranges(const qm_runtime* rt, const qm_q4_job& j, uint32_t in_elems, const char* name) {
  char what[96];
  const uint64_t wbytes = (uint64_t)j.out_rows * (in_elems / 8) * 4;
  const uint64_t abytes = (uint64_t)j.out_rows * (in_elems / kGroup) * 2;
  qm_status st;
  snprintf(what, sizeof(what), "%s weights", name);
  if ((st = check_range(rt, j.weights, wbytes, what)) != QM_OK) return st;
  snprintf(what, sizeof(what), "%s scales", name);
  if ((st = check_range(rt, j.scales, abytes, what)) != QM_OK) return st;
  snprintf(what, sizeof(what), "%s biases", name);
  return check_range(rt, j.biases, abytes, what);
}

namespace {

qm_status check_job_ranges(const qm_runtime* rt, const qm_q4_job& j, uint32_t in_elems, const char* name) {
  return q4_job_ranges(rt, j, in_elems, name);
}

qm_status validate_x(const void* x, uint32_t M) {
  if (!x) return fail(QM_ERR_NULL_POINTER, "activation pointer is NULL");
  if (M == 0) return fail(QM_ERR_EMPTY_DIMENSION, "batch size must be greater than zero");
  if (!aligned(x, 16)) return fail(QM_ERR_MISALIGNED, "activation must be 16-byte aligned");
  return QM_OK;
}

Q4Job to_job(const qm_q4_job& j, uint16_t* out) {
  Q4Job q{};
  q.w = j.weights;
  q.s = j.scales;
  q.b = j.biases;
  q.rows = j.out_rows;
  q.out = out;
  return q;
}

// One or two activation rows on the streaming kernel (its K-split workspace first).
qm_status stream_launch(qm_runtime* rt, const Q4Job* jobs, int n, const uint16_t* x, uint32_t K, uint32_t M,
                        const char* what) {
  size_t pbytes = 0, counters = 0;
  q4_stream_workspace(jobs, n, K, M, rt->tune, &pbytes, &counters);
  qm_status st = ensure_partials(rt, pbytes);
  if (st == QM_OK) st = ensure_counters(rt, counters);
  if (st != QM_OK) return st;
  return hip_check(launch_q4_stream(jobs, n, x, K, M, workspace(rt), rt->stream), what);
}

// Prefill rows on the GEMM (its split-K workspace and fp16 activation copy
// first).  swiglu: jobs = {gate, up}; otherwise plain jobs and folded pairs
// may mix.
qm_status gemm_launch(qm_runtime* rt, const Q4Job* jobs, int n, bool swiglu, const uint16_t* x, uint32_t K,
                      uint32_t M, const char* what) {
  size_t pbytes = 0, counters = 0;
  q4_gemm_workspace(jobs, n, swiglu, K, M, rt->tune, &pbytes, &counters);
  qm_status st = ensure_partials(rt, pbytes);
  if (st == QM_OK) st = ensure_counters(rt, counters);
  if (st == QM_OK) st = ensure_xh(rt, q4_gemm_xh_bytes(K, M));
  if (st != QM_OK) return st;
  return hip_check(launch_q4_gemm(jobs, n, swiglu, x, K, M, workspace(rt), rt->stream), what);
}

// 1..8 activation rows on the MFMA streaming kernel (its K-part workspace first).
qm_status mma_launch(qm_runtime* rt, const Q4Job* jobs, int n, const uint16_t* x, uint32_t K, uint32_t M,
                     const char* what) {
  size_t pbytes = 0, counters = 0;
  q4_mma_workspace(jobs, n, K, M, rt->tune, &pbytes, &counters);
  qm_status st = ensure_partials(rt, pbytes);
  if (st == QM_OK) st = ensure_counters(rt, counters);
  if (st != QM_OK) return st;
  return hip_check(launch_q4_mma(jobs, n, x, K, M, workspace(rt), rt->stream), what);
}

qm_status launch(qm_runtime* rt, const Q4Job* jobs, int n, bool swiglu, const uint16_t* x, uint32_t K,
                 uint32_t M, const char* what) {
  if (M <= 8) {
    // One or two activation rows: the streaming kernel; up to 8: the MFMA
    // streaming kernel; both take a gate/up pair as one job.
    Q4Job sj[kMaxQ4Jobs];
    int ns = 0;
    if (swiglu) {
      sj[0] = jobs[0];
      sj[0].uw = jobs[1].w;
      sj[0].us = jobs[1].s;
      sj[0].ub = jobs[1].b;
      sj[0].mode = kQ4OutSwiglu;
      ns = 1;
    } else {
      for (int i = 0; i < n; ++i) sj[ns++] = jobs[i];
    }
    if (M >= 2 && q4_mma_supported(sj, ns, K, M, rt->tune)) return mma_launch(rt, sj, ns, x, K, M, what);
    if (q4_stream_supported(sj, ns, K, M, rt->tune)) return stream_launch(rt, sj, ns, x, K, M, what);
    if (q4_mma_supported(sj, ns, K, M, rt->tune)) return mma_launch(rt, sj, ns, x, K, M, what);
  }
  if (M > kDecodeMaxRows) return gemm_launch(rt, jobs, n, swiglu, x, K, M, what);
  return hip_check(launch_q4_decode(jobs, n, swiglu, x, K, M, workspace(rt), rt->stream), what);
}

}  // namespace

qm_status qm::q4_reserve_workspace(qm_runtime* rt, const qm_q4_job* jobs, int n_jobs, uint32_t in_elems) {
  if (n_jobs <= 0 || n_jobs > kMaxQ4Jobs) return QM_OK;
  Q4Job q[kMaxQ4Jobs];
  for (int i = 0; i < n_jobs; ++i) q[i] = to_job(jobs[i], nullptr);
  if (!q4_stream_supported(q, n_jobs, in_elems, 1, rt->tune)) return QM_OK;
  size_t pbytes = 0, counters = 0;
  q4_stream_workspace(q, n_jobs, in_elems, 1, rt->tune, &pbytes, &counters);
  qm_status st = ensure_partials(rt, pbytes);
  return st == QM_OK ? ensure_counters(rt, counters) : st;
}

qm_status qm::q4_project_modes(qm_runtime* rt, const qm_q4_job* jobs, void* const* outs, const uint32_t* modes,
                               int n_jobs, const uint16_t* x, uint32_t in_elems, uint32_t M) {
  if (!rt || !jobs || !outs || !modes) return fail(QM_ERR_NULL_POINTER, "NULL argument");
  if (n_jobs <= 0 || n_jobs > kMaxQ4Jobs) return fail(QM_ERR_INVALID_ARGUMENT, "1..%d jobs per call", kMaxQ4Jobs);
  qm_status st = validate_x(x, M);
  if (st != QM_OK) return st;
  Q4Job q[kMaxQ4Jobs];
  for (int i = 0; i < n_jobs; ++i) {
    if ((st = validate_job(&jobs[i], in_elems, "Q4 projection")) != QM_OK) return st;
    if (!outs[i]) return fail(QM_ERR_NULL_POINTER, "output %d is NULL", i);
    if (modes[i] > kQ4OutAddF32 || (modes[i] != kQ4OutBf16 && M > kDecodeMaxRows))
      return fail(QM_ERR_INVALID_ARGUMENT, "output mode %u needs the decode path (M <= %u)", modes[i],
                  kDecodeMaxRows);
    q[i] = to_job(jobs[i], (uint16_t*)outs[i]);
    q[i].mode = modes[i];
  }
  DeviceGuard g(rt->device);
  if (!g.ok()) return no_device();
  if ((st = check_range(rt, x, (uint64_t)M * in_elems * 2, "activation")) != QM_OK) return st;
  for (int i = 0; i < n_jobs; ++i) {
    if ((st = check_job_ranges(rt, jobs[i], in_elems, "Q4 projection")) != QM_OK) return st;
    const uint64_t ob = (uint64_t)M * jobs[i].out_rows * (modes[i] == kQ4OutBf16 ? 2 : 4);
    if ((st = check_range(rt, outs[i], ob, "output")) != QM_OK) return st;
  }
  return launch(rt, q, n_jobs, false, x, in_elems, M, "Q4 projection launch");
}

extern "C" {

qm_status qm_q4_project(qm_runtime* rt, const qm_q4_job* jobs, int n_jobs, const uint16_t* x,
                        uint32_t in_elems, uint32_t M, uint16_t* const* outputs) {
  if (!rt) return fail(QM_ERR_NULL_POINTER, "runtime is NULL");
  if (!jobs || n_jobs <= 0) return fail(QM_ERR_EMPTY_DIMENSION, "at least one Q4 job is required");
  if (n_jobs > kMaxQ4Jobs) return fail(QM_ERR_INVALID_ARGUMENT, "at most %d jobs per call", kMaxQ4Jobs);
  if (!outputs) return fail(QM_ERR_NULL_POINTER, "outputs is NULL");
  qm_status st = validate_x(x, M);
  if (st != QM_OK) return st;
  Q4Job q[kMaxQ4Jobs];
  for (int i = 0; i < n_jobs; ++i) {
    st = validate_job(&jobs[i], in_elems, "Q4 projection");
    if (st != QM_OK) return st;
    if (!outputs[i]) return fail(QM_ERR_NULL_POINTER, "output %d is NULL", i);
    q[i] = to_job(jobs[i], outputs[i]);
  }
  DeviceGuard g(rt->device);
  if (!g.ok()) return no_device();
  if ((st = check_range(rt, x, (uint64_t)M * in_elems * 2, "activation")) != QM_OK) return st;
  for (int i = 0; i < n_jobs; ++i) {
    if ((st = check_job_ranges(rt, jobs[i], in_elems, "Q4 projection")) != QM_OK) return st;
    if ((st = check_range(rt, outputs[i], (uint64_t)M * jobs[i].out_rows * 2, "output")) != QM_OK) return st;
  }
  return launch(rt, q, n_jobs, false, x, in_elems, M, "Q4 projection launch");
}

qm_status qm_q4_project_set(qm_runtime* rt, const qm_q4_job* jobs, const qm_q4_job* const* ups, int n_jobs,
                            const uint16_t* x, uint32_t in_elems, uint32_t M, uint16_t* const* outputs) {
  if (!rt) return fail(QM_ERR_NULL_POINTER, "runtime is NULL");
  if (!jobs || n_jobs <= 0) return fail(QM_ERR_EMPTY_DIMENSION, "at least one Q4 job is required");
  if (n_jobs > kMaxQ4Jobs) return fail(QM_ERR_INVALID_ARGUMENT, "at most %d jobs per call", kMaxQ4Jobs);
  if (!outputs) return fail(QM_ERR_NULL_POINTER, "outputs is NULL");
  qm_status st = validate_x(x, M);
  if (st != QM_OK) return st;
  Q4Job q[kMaxQ4Jobs];
  for (int i = 0; i < n_jobs; ++i) {
    if ((st = validate_job(&jobs[i], in_elems, "Q4 projection")) != QM_OK) return st;
    const qm_q4_job* up = ups ? ups[i] : nullptr;
    if (up) {
      if ((st = validate_job(up, in_elems, "up")) != QM_OK) return st;
      if (up->out_rows != jobs[i].out_rows)
        return fail(QM_ERR_WRONG_LENGTH, "up %d has %u rows, expected %u", i, up->out_rows, jobs[i].out_rows);
    }
    if (!outputs[i]) return fail(QM_ERR_NULL_POINTER, "output %d is NULL", i);
    q[i] = to_job(jobs[i], outputs[i]);
    if (up) {
      q[i].uw = up->weights;
      q[i].us = up->scales;
      q[i].ub = up->biases;
      q[i].mode = kQ4OutSwiglu;
    }
  }
  DeviceGuard g(rt->device);
  if (!g.ok()) return no_device();
  if ((st = check_range(rt, x, (uint64_t)M * in_elems * 2, "activation")) != QM_OK) return st;
  for (int i = 0; i < n_jobs; ++i) {
    if ((st = check_job_ranges(rt, jobs[i], in_elems, "Q4 projection")) != QM_OK) return st;
    if (ups && ups[i] && (st = check_job_ranges(rt, *ups[i], in_elems, "up")) != QM_OK) return st;
    if ((st = check_range(rt, outputs[i], (uint64_t)M * jobs[i].out_rows * 2, "output")) != QM_OK) return st;
  }
  if (M >= 2 && q4_mma_supported(q, n_jobs, in_elems, M, rt->tune))
    return mma_launch(rt, q, n_jobs, x, in_elems, M, "Q4 set launch");
  if (q4_stream_supported(q, n_jobs, in_elems, M, rt->tune))
    return stream_launch(rt, q, n_jobs, x, in_elems, M, "Q4 set launch");
  if (q4_mma_supported(q, n_jobs, in_elems, M, rt->tune)) return mma_launch(rt, q, n_jobs, x, in_elems, M, "Q4 set launch");
  // Prefill rows: one GEMM launch over the whole set (plain and pair tiles).
  if (M > kDecodeMaxRows) return gemm_launch(rt, q, n_jobs, false, x, in_elems, M, "Q4 set GEMM launch");
  // Otherwise: the plain jobs in one launch, each pair in its own.
  Q4Job plain[kMaxQ4Jobs];
  int np = 0;
  for (int i = 0; i < n_jobs; ++i)
    if (q[i].mode != kQ4OutSwiglu) plain[np++] = q[i];
  if (np && (st = launch(rt, plain, np, false, x, in_elems, M, "Q4 set launch")) != QM_OK) return st;
  for (int i = 0; i < n_jobs; ++i) {
    if (q[i].mode != kQ4OutSwiglu) continue;
    Q4Job pair[2] = {to_job(jobs[i], outputs[i]), to_job(*ups[i], nullptr)};
    if ((st = launch(rt, pair, 2, true, x, in_elems, M, "Q4 set pair launch")) != QM_OK) return st;
  }
  return QM_OK;
}

qm_status qm_q4_swiglu(qm_runtime* rt, const qm_q4_job* gate, const qm_q4_job* up, const uint16_t* x,
                       uint32_t in_elems, uint32_t M, uint16_t* h) {
  if (!rt) return fail(QM_ERR_NULL_POINTER, "runtime is NULL");
  qm_status st = validate_x(x, M);
  if (st != QM_OK) return st;
  if ((st = validate_job(gate, in_elems, "gate")) != QM_OK) return st;
  if ((st = validate_job(up, in_elems, "up")) != QM_OK) return st;
  if (gate->out_rows != up->out_rows)
    return fail(QM_ERR_WRONG_LENGTH, "up has %u rows, expected %u", up->out_rows, gate->out_rows);
  if (!h) return fail(QM_ERR_NULL_POINTER, "h is NULL");
  Q4Job q[2] = {to_job(*gate, h), to_job(*up, nullptr)};
  DeviceGuard g(rt->device);
  if (!g.ok()) return no_device();
  if ((st = check_range(rt, x, (uint64_t)M * in_elems * 2, "activation")) != QM_OK) return st;
  if ((st = check_job_ranges(rt, *gate, in_elems, "gate")) != QM_OK) return st;
  if ((st = check_job_ranges(rt, *up, in_elems, "up")) != QM_OK) return st;
  if ((st = check_range(rt, h, (uint64_t)M * gate->out_rows * 2, "h")) != QM_OK) return st;
  return launch(rt, q, 2, true, x, in_elems, M, "Q4 SwiGLU launch");
}

qm_status qm_q4_mlp(qm_runtime* rt, const qm_q4_job* gate, const qm_q4_job* up, const qm_q4_job* down,
                    const uint16_t* x, uint32_t in_elems, uint32_t M, uint16_t* y) {
  if (!rt) return fail(QM_ERR_NULL_POINTER, "runtime is NULL");
  qm_status st = validate_x(x, M);
  if (st != QM_OK) return st;
  if ((st = validate_job(gate, in_elems, "gate")) != QM_OK) return st;
  if ((st = validate_job(up, in_elems, "up")) != QM_OK) return st;
  if (gate->out_rows != up->out_rows)
    return fail(QM_ERR_WRONG_LENGTH, "up has %u rows, expected %u", up->out_rows, gate->out_rows);
  if ((st = validate_job(down, gate->out_rows, "down")) != QM_OK) return st;
  if (!y) return fail(QM_ERR_NULL_POINTER, "y is NULL");
  DeviceGuard g(rt->device);
  if (!g.ok()) return no_device();
  if ((st = check_range(rt, x, (uint64_t)M * in_elems * 2, "activation")) != QM_OK) return st;
  if ((st = check_job_ranges(rt, *gate, in_elems, "gate")) != QM_OK) return st;
  if ((st = check_job_ranges(rt, *up, in_elems, "up")) != QM_OK) return st;
  if ((st = check_job_ranges(rt, *down, gate->out_rows, "down")) != QM_OK) return st;
  if ((st = check_range(rt, y, (uint64_t)M * down->out_rows * 2, "y")) != QM_OK) return st;
  const size_t h_bytes = (size_t)M * gate->out_rows * 2;
  if ((st = ensure_scratch(rt, h_bytes)) != QM_OK) return st;
  uint16_t* h = (uint16_t*)rt->scratch;
  Q4Job q[2] = {to_job(*gate, h), to_job(*up, nullptr)};
  if ((st = launch(rt, q, 2, true, x, in_elems, M, "MLP gate/up launch")) != QM_OK) return st;
  Q4Job d = to_job(*down, y);
  return launch(rt, &d, 1, false, h, gate->out_rows, M, "MLP down launch");
}

qm_status qm_q4_argmax(qm_runtime* rt, const qm_q4_job* job, const uint16_t* x, uint32_t in_elems, uint32_t M,
                       uint32_t* ids) {
  if (!rt) return fail(QM_ERR_NULL_POINTER, "runtime is NULL");
  qm_status st = validate_x(x, M);
  if (st != QM_OK) return st;
  if ((st = validate_job(job, in_elems, "argmax")) != QM_OK) return st;
  if (!ids) return fail(QM_ERR_NULL_POINTER, "ids is NULL");
  DeviceGuard g(rt->device);
  if (!g.ok()) return no_device();
  if ((st = check_range(rt, x, (uint64_t)M * in_elems * 2, "activation")) != QM_OK) return st;
  if ((st = check_job_ranges(rt, *job, in_elems, "argmax")) != QM_OK) return st;
  if ((st = check_range(rt, ids, (uint64_t)M * 4, "ids")) != QM_OK) return st;
  // One 64-bit key per row of a chunk of at most 16 rows (zero between
  // calls; the finishing kernel clears them).  Larger M runs the decode
  // kernel chunk by chunk: each row's argmax is independent of the others.
  if ((st = ensure_keys(rt)) != QM_OK) return st;
  Q4Job q = to_job(*job, (uint16_t*)rt->keys);
  q.mode = kQ4OutArgmax;
  const bool stream = q4_stream_supported(&q, 1, in_elems, 1, rt->tune);
  if (stream) {
    size_t pbytes = 0, counters = 0;
    q4_stream_workspace(&q, 1, in_elems, 1, rt->tune, &pbytes, &counters);
    if ((st = ensure_partials(rt, pbytes)) != QM_OK || (st = ensure_counters(rt, counters)) != QM_OK) return st;
  }
  const Workspace ws = workspace(rt);
  for (uint32_t m0 = 0; m0 < M; m0 += kDecodeMaxRows) {
    const uint32_t mc = M - m0 < kDecodeMaxRows ? M - m0 : kDecodeMaxRows;
    hipError_t e = mc == 1 && stream
                       ? launch_q4_stream(&q, 1, x + (size_t)m0 * in_elems, in_elems, 1, ws, rt->stream)
                       : launch_q4_decode(&q, 1, false, x + (size_t)m0 * in_elems, in_elems, mc, ws, rt->stream);
    if (e == hipSuccess) e = launch_q4_argmax_finish(rt->keys, ids + m0, mc, rt->stream);
    if ((st = hip_check(e, "Q4 argmax launch")) != QM_OK) return st;
  }
  return QM_OK;
}

qm_status qm_q4_job_from_mapped(const qm_q4_mapped_job* m, uint32_t in_elems, qm_q4_job* out) {
  if (!m || !out) return fail(QM_ERR_NULL_POINTER, "NULL argument");
  if (in_elems == 0 || m->out_rows == 0)
    return fail(QM_ERR_EMPTY_DIMENSION, "matrix dimensions must be greater than zero");
  if (in_elems % kGroup != 0)
    return fail(QM_ERR_INPUT_NOT_GROUPED, "input dimension %u is not divisible by affine group size %u", in_elems,
                kGroup);
  if (m->weight_offset > m->weights.length || m->scale_offset > m->scales.length ||
      m->bias_offset > m->biases.length)
    return fail(QM_ERR_INVALID_BUFFER_OFFSET, "a tensor offset lies beyond its buffer");
  // Both products fit in 64 bits (u32 x u32); the byte lengths are checked
  // against the buffers' remaining lengths below.
  const uint64_t wbytes = (uint64_t)m->out_rows * (in_elems / 8) * 4;
  const uint64_t abytes = (uint64_t)m->out_rows * (in_elems / kGroup) * 2;
  if (wbytes > m->weights.length - m->weight_offset || abytes > m->scales.length - m->scale_offset ||
      abytes > m->biases.length - m->bias_offset)
    return fail(QM_ERR_MAPPED_TENSOR_OUT_OF_RANGE, "a tensor of %u x %u runs past the end of its buffer",
                m->out_rows, in_elems);
  if (!m->weights.base || !m->scales.base || !m->biases.base)
    return fail(QM_ERR_NULL_POINTER, "a buffer base is NULL");
  qm_q4_job j{};
  j.weights = (const uint32_t*)((const uint8_t*)m->weights.base + m->weight_offset);
  j.scales = (const uint16_t*)((const uint8_t*)m->scales.base + m->scale_offset);
  j.biases = (const uint16_t*)((const uint8_t*)m->biases.base + m->bias_offset);
  j.out_rows = m->out_rows;
  if (!aligned(j.weights, 8) || !aligned(j.scales, 8) || !aligned(j.biases, 8))
    return fail(QM_ERR_MISALIGNED, "weights/scales/biases must resolve to 8-byte aligned addresses");
  *out = j;
  return QM_OK;
}

}  // extern "C"
