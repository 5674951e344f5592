// Q4 prefill projection (M > 16 rows).
#include "common.h"
#include "internal.h"

namespace qm {

hipError_t launch_q4_gemm(const Q4Job* jobs, int n_jobs, bool swiglu, const uint16_t* x, uint32_t K,
                          uint32_t M, const Workspace& ws, hipStream_t stream) {
  // Row blocks of 16 through the decode kernel.
  for (uint32_t m0 = 0; m0 < M; m0 += 16) {
    Q4Job js[kMaxQ4Jobs];
    for (int i = 0; i < n_jobs; ++i) {
      js[i] = jobs[i];
      if (js[i].out) js[i].out += (size_t)m0 * jobs[i].rows;
    }
    const uint32_t mm = M - m0 < 16 ? M - m0 : 16;
    hipError_t e = launch_q4_decode(js, n_jobs, swiglu, x + (size_t)m0 * K, K, mm, ws, stream);
    if (e != hipSuccess) return e;
  }
  return hipSuccess;
}

}  // namespace qm
