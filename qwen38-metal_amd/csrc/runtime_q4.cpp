// C-ABI entry points of the MLX affine-Q4 projections (see include/qm38.h).
#include <stdint.h>

#include "runtime_internal.h"

using namespace qm;

namespace {

constexpr uint32_t kGroup = 64;       // AFFINE_GROUP_SIZE (metal_runtime.rs)
constexpr uint32_t kDecodeMaxRows = 16;

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
  if (!job->weights || !job->scales || !job->biases)
    return fail(QM_ERR_NULL_POINTER, "%s: weights/scales/biases pointer is NULL", name);
  if (!aligned(job->weights, 8) || !aligned(job->scales, 8) || !aligned(job->biases, 8))
    return fail(QM_ERR_MISALIGNED, "%s: weights/scales/biases must be 8-byte aligned", name);
  const uint64_t words = (uint64_t)job->out_rows * (in_elems / 8);
  if (words > (1ull << 40)) return fail(QM_ERR_DIMENSION_OVERFLOW, "%s: packed weight count exceeds runtime limits", name);
  return QM_OK;
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

qm_status launch(qm_runtime* rt, const Q4Job* jobs, int n, bool swiglu, const uint16_t* x, uint32_t K,
                 uint32_t M, const char* what) {
  // The decode kernel needs no workspace; the GEMM's split-K plans do.
  size_t pbytes = 0, counters = 0;
  if (M > kDecodeMaxRows) q4_gemm_workspace(jobs, n, swiglu, K, M, &pbytes, &counters);
  qm_status st = ensure_partials(rt, pbytes);
  if (st == QM_OK) st = ensure_counters(rt, counters);
  if (st == QM_OK && M > kDecodeMaxRows) st = ensure_xh(rt, q4_gemm_xh_bytes(K, M));
  if (st != QM_OK) return st;
  const Workspace ws = workspace(rt);
  hipError_t e = M <= kDecodeMaxRows ? launch_q4_decode(jobs, n, swiglu, x, K, M, ws, rt->stream)
                                     : launch_q4_gemm(jobs, n, swiglu, x, K, M, ws, rt->stream);
  return hip_check(e, what);
}

}  // namespace

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
  return launch(rt, q, n_jobs, false, x, in_elems, M, "Q4 projection launch");
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
  const size_t h_bytes = (size_t)M * gate->out_rows * 2;
  if ((st = ensure_scratch(rt, h_bytes)) != QM_OK) return st;
  uint16_t* h = (uint16_t*)rt->scratch;
  Q4Job q[2] = {to_job(*gate, h), to_job(*up, nullptr)};
  if ((st = launch(rt, q, 2, true, x, in_elems, M, "MLP gate/up launch")) != QM_OK) return st;
  Q4Job d = to_job(*down, y);
  return launch(rt, &d, 1, false, h, gate->out_rows, M, "MLP down launch");
}

}  // extern "C"
