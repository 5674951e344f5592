// Host-side launch interface between the C-ABI runtime (runtime.cpp) and the
// HIP kernels.  Nothing here is exported from the shared library.
#pragma once
#include <hip/hip_runtime.h>
#include <stdint.h>

namespace qm {

constexpr int kMaxQ4Jobs = 8;

struct Q4Job {
  const uint32_t* w;
  const uint16_t* s;
  const uint16_t* b;
  uint16_t* out;
  // The up half of a gate/up pair (mode kQ4OutSwiglu): out = bf16 silu(w x) * (uw x).
  const uint32_t* uw;
  const uint16_t* us;
  const uint16_t* ub;
  uint32_t rows;
  uint32_t tile_begin;  // filled by the launcher
  // Output of a decode (M <= 16) projection: 0 bf16; 1 fp32 holding the bf16-
  // rounded value (as if converted afterwards); 2 fp32 += the bf16-rounded
  // value (a residual add).  `out` then points at fp32.  3: argmax keys, one
  // uint64 per activation row (`out` points at them; they must be zero and are
  // maxed with atomics; launch_q4_argmax_finish turns them into row ids and
  // clears them).  4: a gate/up pair with SwiGLU (the streaming kernel and the
  // GEMM).  The GEMM takes 0 and 4 only.
  uint32_t mode;
};
constexpr uint32_t kQ4OutBf16 = 0, kQ4OutF32 = 1, kQ4OutAddF32 = 2, kQ4OutArgmax = 3, kQ4OutSwiglu = 4;

// Planner inputs: the device's compute units and the QM38_* tuning overrides
// (forced plans for measurements), read from the environment once, when a
// runtime is created.  A value <= 0 (or -1 for the switches) keeps the
// planner's own choice.
struct Tuning {
  int cus = 256;            // compute units (hipDeviceProp_t::multiProcessorCount)
  int q4_nt = 0;            // QM38_Q4_NT: 16-row tiles per decode workgroup (1, 2)
  int q4_xstage = 1;        // QM38_Q4_XSTAGE: 0 disables staged activations
  int q4_xstage_max = 0;    // QM38_Q4_XSTAGE_MAX: LDS bytes of staged activations
  int q4_target_waves = 0;  // QM38_Q4_TARGET_WAVES: resident waves the K split aims at
  int q4_rpw = 0;           // QM38_Q4_RPW: rows per decode workgroup
  int q4_split = 0;         // QM38_Q4_SPLIT: waves per decode workgroup
  int q4_plan_log = 0;      // QM38_Q4_PLAN_LOG: print each new decode plan
  int q4_fuse = 1;          // QM38_Q4_FUSE: 0 runs the MLP's down projection as its own launch
  int q4_stream = 1;        // QM38_Q4_STREAM: 0 keeps single-row projections on the MFMA decode kernel
  int q4_stream_mw = 0;     // QM38_Q4_STREAM_MW: waves per K part with several activation rows
  int q4_stream_rows = 2;   // QM38_Q4_STREAM_ROWS: most activation rows on the streaming kernel (1, 2)
  int q4_stream_wgs = 0;    // QM38_Q4_STREAM_WGS: workgroups per K part of the single-row kernel
  int q4_stream_c = 0;      // QM38_Q4_STREAM_C: chunks per wave of the single-row kernel (1..4)
  int q4_stream_w = 0;      // QM38_Q4_STREAM_W: waves per workgroup with QM38_Q4_STREAM_C
  int q4_mma_lo = 3;        // QM38_Q4_MMA_LO: fewest activation rows on the MFMA streaming kernel (0: off)
  int q4_mma_hi = 4;        // QM38_Q4_MMA_HI: most activation rows on it (at most 8)
  int q4_mma_k = 8192;      // QM38_Q4_MMA_K: 2..8 rows with K above this also take it (0: never)
  int q4_mma_w = 0;         // QM38_Q4_MMA_W: most waves per K part of the MFMA streaming kernel
  int q4_mma_c = 0;         // QM38_Q4_MMA_C: 4 or 8 spans per wave with up to four activation rows
  int q4_mma_sb = 0;        // QM38_Q4_MMA_SB: 2 forces 32-row blocks for plain projections
  int q4_mma_wgs = 0;       // QM38_Q4_MMA_WGS: workgroups per K part of the MFMA streaming kernel
  int gemm_splits = 0;      // QM38_GEMM_SPLITS: K splits of the prefill GEMM
  int gemm_q = 0;           // QM38_GEMM_Q: stream-K steps per worker
  int gemm_plan_log = 0;    // QM38_GEMM_PLAN_LOG
  int attn_pps = 0;         // QM38_ATTN_PPS: pages per decode split
  int attn_waves = 0;       // QM38_ATTN_WAVES: 4 or 8 waves per decode workgroup
  int attn_target_wgs = 0;  // QM38_ATTN_TARGET_WGS
  int prefill_cb = 0;       // QM38_PREFILL_CB: column blocks per prefill wave (1, 2, 4)
  int dn_step_head = -1;    // QM38_DN_STEP_HEAD: 0 forces the split step kernel (-1: default)
  int dn_chunked = -1;      // QM38_DN_CHUNKED: 1 / 0 forces the chunked / token-serial prefill (-1: default)
  int dn_pair = -1;         // QM38_DN_PAIR: 0 forces the one-value-head chunk preparation (-1: default)
};
Tuning read_tuning(int cu_count);

// Device workspace for kernels whose workgroups combine partial results:
// `counters` are zero between launches (each kernel leaves them at zero).
struct Workspace {
  float* partials;
  size_t partial_bytes;
  unsigned int* counters;
  size_t counter_count;
  uint16_t* xh;  // prefill GEMM: fp16 copy of the activations
  size_t xh_bytes;
  const Tuning* tune;
};

// Decode (weight-streaming) Q4 projection: M <= 16 activation rows.
// swiglu: jobs[0] = gate, jobs[1] = up, result written to jobs[0].out.
hipError_t launch_q4_decode(const Q4Job* jobs, int n_jobs, bool swiglu, const uint16_t* x,
                            uint32_t K, uint32_t M, const Workspace& ws, hipStream_t stream);

// One or two activation rows (QM38_Q4_STREAM_ROWS=1 keeps two rows on the
// MFMA decode kernel): the K-resident streaming kernel (q4_stream.hip).  Jobs may mix
// plain projections and gate/up pairs (kQ4OutSwiglu); an argmax launch has
// one job and one row.
bool q4_stream_supported(const Q4Job* jobs, int n_jobs, uint32_t K, uint32_t M, const Tuning& tn);
hipError_t launch_q4_stream(const Q4Job* jobs, int n_jobs, const uint16_t* x, uint32_t K, uint32_t M,
                            const Workspace& ws, hipStream_t stream);
// 1..8 activation rows on the matrix cores with the weights streamed once
// (q4_mma.hip): QM38_Q4_MMA_LO <= M <= QM38_Q4_MMA_HI (3..4 by default), and
// 2..8 rows when K > QM38_Q4_MMA_K.  Jobs may mix plain projections and
// gate/up pairs; no argmax.
bool q4_mma_supported(const Q4Job* jobs, int n_jobs, uint32_t K, uint32_t M, const Tuning& tn);
hipError_t launch_q4_mma(const Q4Job* jobs, int n_jobs, const uint16_t* x, uint32_t K, uint32_t M,
                         const Workspace& ws, hipStream_t stream);
void q4_mma_workspace(const Q4Job* jobs, int n_jobs, uint32_t K, uint32_t M, const Tuning& tn,
                      size_t* partial_bytes, size_t* counters);
// Workspace of a streaming launch: fp32 partial rows and counters when K is
// split over several workgroups (zero otherwise).
void q4_stream_workspace(const Q4Job* jobs, int n_jobs, uint32_t K, uint32_t M, const Tuning& tn,
                         size_t* partial_bytes, size_t* counters);

// ids[m] from the argmax keys of a kQ4OutArgmax decode launch; zeroes the keys.
hipError_t launch_q4_argmax_finish(unsigned long long* keys, uint32_t* ids, uint32_t M, hipStream_t stream);

// Prefill Q4 GEMM (M > 16): Y[M][N] = X[M][K] * dequant(W)^T, bf16 out.
// swiglu as above.
size_t q4_gemm_xh_bytes(uint32_t K, uint32_t M);
// Split-K partial bytes / counters a GEMM launch needs (0 when it does not split).
void q4_gemm_workspace(const Q4Job* jobs, int n_jobs, bool swiglu, uint32_t K, uint32_t M, const Tuning& tune,
                       size_t* partial_bytes, size_t* counters);
hipError_t launch_q4_gemm(const Q4Job* jobs, int n_jobs, bool swiglu, const uint16_t* x,
                          uint32_t K, uint32_t M, const Workspace& ws, hipStream_t stream);

// Residual stream helpers of the decode graph (residual.hip).
// hidden fp32 [M][n] (+= delta bf16 when delta != NULL), out = bf16 RMSNorm(hidden) * w.
hipError_t launch_residual_rmsnorm(float* hidden, const uint16_t* delta, const float* w, uint16_t* out, uint32_t M,
                                   uint32_t n, float eps, hipStream_t stream);
hipError_t launch_residual_add(float* hidden, const uint16_t* delta, size_t count, hipStream_t stream);
constexpr int kMaxConvSegs = 6;
struct ConvSeg {
  const void* src;
  void* dst;
  uint32_t n;       // elements
  uint32_t to_f32;  // 1: bf16 -> fp32, 0: fp32 -> bf16
};
hipError_t launch_convert(const ConvSeg* segs, int nseg, hipStream_t stream);
hipError_t launch_set_u32x3(uint32_t* dst, uint32_t a, uint32_t b, uint32_t c, hipStream_t stream);

}  // namespace qm
