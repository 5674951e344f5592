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
  uint32_t rows;
  uint32_t tile_begin;  // filled by the launcher
};

// Decode (weight-streaming) Q4 projection: M <= 16 activation rows.
// swiglu: jobs[0] = gate, jobs[1] = up, result written to jobs[0].out.
hipError_t launch_q4_decode(const Q4Job* jobs, int n_jobs, bool swiglu, const uint16_t* x,
                            uint32_t K, uint32_t M, hipStream_t stream);

// Prefill Q4 GEMM (M > 16): Y[M][N] = X[M][K] * dequant(W)^T, bf16 out.
// swiglu as above.
hipError_t launch_q4_gemm(const Q4Job* jobs, int n_jobs, bool swiglu, const uint16_t* x,
                          uint32_t K, uint32_t M, hipStream_t stream);

}  // namespace qm
