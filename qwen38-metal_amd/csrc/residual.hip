// Residual stream of the per-token decode graph: RMSNorm rows with an
// optional fused residual add (qwen38_rms_norm / _rms_norm_rows followed by
// qwen38_add_in_place / _add_rows, /root/reference/shaders/qwen38.metal:
// 4250-4333), the residual add alone, and the bf16 <-> fp32 conversions that
// join the bf16 Q4 projections to the fp32 DeltaNet and attention inputs.
//
// RMSNorm follows the reference's formula: out = (x * rsqrt(mean(x^2) + eps))
// * w, in fp32, with the weights used as given (not 1 + w).  The residual
// stream `hidden` stays fp32 (the reference's activations are fp32); the
// normalised rows are rounded to bf16, the Q4 projections' input type.
// One 1024-thread workgroup per row: the row is read with 16-byte loads
// (kept in registers up to 8192 elements), the sum of squares is reduced
// across lanes by DPP and across the 16 waves in LDS, and the output is
// written from the registers.
#include "common.h"
#include "internal.h"

#include <algorithm>

namespace qm {
namespace {

constexpr int kNormThreads = 1024;
constexpr int kNormCache = 2;  // float4s per thread kept in registers between the two passes

struct NormArgs {
  float* hidden;          // [M][n] fp32, updated in place when delta != NULL
  const uint16_t* delta;  // [M][n] bf16 or NULL
  const float* w;         // [n]
  uint16_t* out;          // [M][n] bf16
  uint32_t n;
  uint32_t vec;  // 16-byte path: n % 4 == 0 and aligned rows
  float eps;
};

__device__ __forceinline__ u32x2 norm4(const floatx4& v, const floatx4& w, float scale) {
  u32x2 r;
  r.x = f32_to_bf16(v[0] * scale * w[0]) | ((uint32_t)f32_to_bf16(v[1] * scale * w[1]) << 16);
  r.y = f32_to_bf16(v[2] * scale * w[2]) | ((uint32_t)f32_to_bf16(v[3] * scale * w[3]) << 16);
  return r;
}

// One 1024-thread workgroup per row.  A thread's first kNormCache float4s
// (all of a 8192-wide row) stay in registers from the first pass to the
// second, with their weights loaded up front; wider rows re-read the rest.
__global__ __launch_bounds__(kNormThreads) void residual_rmsnorm_kernel(NormArgs a) {
  __shared__ float part[kNormThreads / 64];
  const uint32_t row = blockIdx.x, tid = threadIdx.x, n = a.n;
  float* h = a.hidden + (size_t)row * n;
  const uint16_t* d = a.delta ? a.delta + (size_t)row * n : nullptr;
  uint16_t* o = a.out + (size_t)row * n;
  const uint32_t n4 = a.vec ? n / 4 : 0;  // else element by element
  floatx4 v[kNormCache], wv[kNormCache];
#pragma unroll
  for (int k = 0; k < kNormCache; ++k) {
    const uint32_t i = min(tid + k * kNormThreads, n4 > 0 ? n4 - 1 : 0);
    if (n4 > 0) {
      v[k] = *(const floatx4*)(h + 4 * i);
      wv[k] = *(const floatx4*)(a.w + 4 * i);
    }
  }
  float ss = 0.0f;
#pragma unroll
  for (int k = 0; k < kNormCache; ++k) {
    const uint32_t i = tid + k * kNormThreads;
    if (i < n4) {
      if (d) {
        const u32x2 dv = *(const u32x2*)(d + 4 * i);
        v[k][0] += bf16_to_f32(dv.x & 0xFFFFu);
        v[k][1] += bf16_to_f32(dv.x >> 16);
        v[k][2] += bf16_to_f32(dv.y & 0xFFFFu);
        v[k][3] += bf16_to_f32(dv.y >> 16);
        *(floatx4*)(h + 4 * i) = v[k];
      }
      ss += v[k][0] * v[k][0] + v[k][1] * v[k][1] + v[k][2] * v[k][2] + v[k][3] * v[k][3];
    }
  }
  for (uint32_t i = tid + kNormCache * kNormThreads; i < n4; i += kNormThreads) {
    floatx4 x = *(const floatx4*)(h + 4 * i);
    if (d) {
      const u32x2 dv = *(const u32x2*)(d + 4 * i);
      x[0] += bf16_to_f32(dv.x & 0xFFFFu);
      x[1] += bf16_to_f32(dv.x >> 16);
      x[2] += bf16_to_f32(dv.y & 0xFFFFu);
      x[3] += bf16_to_f32(dv.y >> 16);
      *(floatx4*)(h + 4 * i) = x;
    }
    ss += x[0] * x[0] + x[1] * x[1] + x[2] * x[2] + x[3] * x[3];
  }
  for (uint32_t i = 4 * n4 + tid; i < n; i += kNormThreads) {
    float x = h[i];
    if (d) {
      x += bf16_to_f32(d[i]);
      h[i] = x;
    }
    ss += x * x;
  }
  ss = wave_allsum(ss);
  if ((tid & 63) == 0) part[tid >> 6] = ss;
  __syncthreads();
  float total = 0.0f;
#pragma unroll
  for (int w = 0; w < kNormThreads / 64; ++w) total += part[w];
  const float scale = 1.0f / sqrtf(total / (float)n + a.eps);
#pragma unroll
  for (int k = 0; k < kNormCache; ++k) {
    const uint32_t i = tid + k * kNormThreads;
    if (i < n4) *(u32x2*)(o + 4 * i) = norm4(v[k], wv[k], scale);
  }
  for (uint32_t i = tid + kNormCache * kNormThreads; i < n4; i += kNormThreads)
    *(u32x2*)(o + 4 * i) = norm4(*(const floatx4*)(h + 4 * i), *(const floatx4*)(a.w + 4 * i), scale);
  for (uint32_t i = 4 * n4 + tid; i < n; i += kNormThreads) o[i] = f32_to_bf16(h[i] * scale * a.w[i]);
}

__global__ __launch_bounds__(256) void residual_add_kernel(float* __restrict__ hidden,
                                                           const uint16_t* __restrict__ delta, size_t count) {
  const size_t stride = (size_t)gridDim.x * 256;
  for (size_t i = (size_t)blockIdx.x * 256 + threadIdx.x; i < count; i += stride) hidden[i] += bf16_to_f32(delta[i]);
}

struct ConvArgs {
  ConvSeg seg[kMaxConvSegs];
  int nseg;
};

// blockIdx.y selects the segment; bf16 -> fp32 is exact, fp32 -> bf16 rounds
// to nearest even (the reference's rule).
__global__ __launch_bounds__(256) void convert_kernel(ConvArgs a) {
  const ConvSeg s = a.seg[blockIdx.y];
  const uint32_t stride = gridDim.x * 256;
  for (uint32_t i = blockIdx.x * 256 + threadIdx.x; i < s.n; i += stride) {
    if (s.to_f32)
      ((float*)s.dst)[i] = bf16_to_f32(((const uint16_t*)s.src)[i]);
    else
      ((uint16_t*)s.dst)[i] = f32_to_bf16(((const float*)s.src)[i]);
  }
}

__global__ void set_u32x3_kernel(uint32_t* dst, uint32_t a, uint32_t b, uint32_t c) {
  if (threadIdx.x == 0) {
    dst[0] = a;
    dst[1] = b;
    dst[2] = c;
  }
}

}  // namespace

hipError_t launch_residual_rmsnorm(float* hidden, const uint16_t* delta, const float* w, uint16_t* out, uint32_t M,
                                   uint32_t n, float eps, hipStream_t stream) {
  if (M == 0 || n == 0 || M > 0x7FFFFFFFu) return hipErrorInvalidValue;
  const uint32_t vec = n % 4 == 0 && ((uintptr_t)hidden % 16 == 0) && ((uintptr_t)w % 16 == 0) &&
                       ((uintptr_t)out % 8 == 0) && (!delta || (uintptr_t)delta % 8 == 0);
  NormArgs a{hidden, delta, w, out, n, vec, eps};
  hipLaunchKernelGGL(residual_rmsnorm_kernel, dim3(M), dim3(kNormThreads), 0, stream, a);
  return hipGetLastError();
}

hipError_t launch_residual_add(float* hidden, const uint16_t* delta, size_t count, hipStream_t stream) {
  if (count == 0) return hipSuccess;
  const size_t blocks = std::min<size_t>((count + 255) / 256, 4096);
  hipLaunchKernelGGL(residual_add_kernel, dim3((unsigned)blocks), dim3(256), 0, stream, hidden, delta, count);
  return hipGetLastError();
}

hipError_t launch_convert(const ConvSeg* segs, int nseg, hipStream_t stream) {
  if (nseg < 1 || nseg > kMaxConvSegs) return hipErrorInvalidValue;
  ConvArgs a{};
  uint32_t longest = 0;
  for (int i = 0; i < nseg; ++i) {
    a.seg[i] = segs[i];
    longest = std::max(longest, segs[i].n);
  }
  a.nseg = nseg;
  if (longest == 0) return hipSuccess;
  const uint32_t blocks = std::min<uint32_t>((longest + 255) / 256, 1024);
  hipLaunchKernelGGL(convert_kernel, dim3(blocks, nseg), dim3(256), 0, stream, a);
  return hipGetLastError();
}

hipError_t launch_set_u32x3(uint32_t* dst, uint32_t a, uint32_t b, uint32_t c, hipStream_t stream) {
  hipLaunchKernelGGL(set_u32x3_kernel, dim3(1), dim3(64), 0, stream, dst, a, b, c);
  return hipGetLastError();
}

}  // namespace qm
