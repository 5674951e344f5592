// Gated DeltaNet (linear-attention) layer for MI355X (gfx950).
//
// One token, or a causal run of M tokens, goes through three kernels:
//  1. dn_conv_prepare_kernel  (qwen38_deltanet_conv + _prepare,
//     /root/reference/shaders/qwen38.metal:4376-4446): depthwise causal
//     conv over the channel history, SiLU, then per key head
//     q^ = q * rsqrt(mean q^2 + eps) / dk and k^ = k * rsqrt(mean k^2 + eps)
//     / sqrt(dk).  Parallel over (token, head).  The conv history is
//     double-buffered: tokens read the old window from one buffer and the last
//     token writes the new window into the other, so no block overwrites
//     history another block still reads.
//  2. dn_scan_kernel  (qwen38_deltanet_recurrence, qwen38.metal:4449-4495):
//     per value head h, g = exp(-e^{A_log} softplus(a + dt_bias)),
//     beta = sigmoid(b), S <- g S, delta = beta (v - S k^), S <- S + delta k^T,
//     o = S q^.  Row i of S (one value channel) only ever meets v_i and the
//     shared k^, q^, g, beta, so rows are independent: each workgroup owns
//     16 rows of one head, keeps them in registers for all M tokens and
//     reads / writes S from HBM exactly once per call.  This is the step
//     recurrence itself, applied token by token, so prefill equals M steps.
//  3. dn_gate_norm_kernel  (qwen38_deltanet_gate_norm, :4497-4527):
//     o <- o * rsqrt(mean o^2 + eps) * norm * silu(z).
#include "common.h"
#include "deltanet.h"

namespace qm {
namespace {

constexpr int kThreads = 256;
constexpr int kRowsPerWg = 16;   // S rows per scan workgroup (16 lanes per row)
constexpr int kTokChunk = 32;    // tokens staged in LDS per scan iteration

__device__ __forceinline__ float block_sum(float v, float* red) {
#pragma unroll
  for (int off = 32; off >= 1; off >>= 1) v += __shfl_xor(v, off);
  const int wave = threadIdx.x >> 6;
  __syncthreads();  // `red` may still be read from a previous call
  if ((threadIdx.x & 63) == 0) red[wave] = v;
  __syncthreads();
  float s = 0.0f;
  for (int w = 0; w < (int)(blockDim.x >> 6); ++w) s += red[w];
  return s;
}

// x(t) of channel ch: t >= 0 from this call's input, t < 0 from the history window.
__device__ __forceinline__ float conv_input(const DnArgs& a, uint32_t ch, int t) {
  const int hw = (int)a.kernel - 1;
  return t >= 0 ? a.qkv[(size_t)t * a.channels + ch] : a.hist_in[(size_t)ch * hw + hw + t];
}

__device__ __forceinline__ float conv_silu(const DnArgs& a, uint32_t ch, int t) {
  const int hw = (int)a.kernel - 1;
  const float* w = a.conv_w + (size_t)ch * a.kernel;
  float sum = w[hw] * conv_input(a, ch, t);
  for (int tap = 0; tap < hw; ++tap) sum += w[tap] * conv_input(a, ch, t - hw + tap);
  return silu_f(sum);
}

__device__ __forceinline__ void shift_history(const DnArgs& a, uint32_t ch) {
  const int hw = (int)a.kernel - 1;
  for (int tap = 0; tap < hw; ++tap)
    a.hist_out[(size_t)ch * hw + tap] = conv_input(a, ch, (int)a.M - hw + tap);
}

// grid: M * (KH + VH) blocks of 256 threads.
__global__ __launch_bounds__(kThreads) void dn_conv_prepare_kernel(DnArgs a) {
  __shared__ float red[kThreads / 64];
  const uint32_t units = a.key_heads + a.value_heads;
  const uint32_t t = blockIdx.x / units, u = blockIdx.x % units;
  const uint32_t i = threadIdx.x;
  const uint32_t key_el = a.key_heads * a.dk;
  float* row = a.conv_out + (size_t)t * a.channels;
  const bool last = t + 1 == a.M && a.kernel > 1;
  if (u < a.key_heads) {
    const uint32_t qc = u * a.dk + i, kc = key_el + u * a.dk + i;
    const bool ok = i < a.dk;
    const float cq = ok ? conv_silu(a, qc, (int)t) : 0.0f;
    const float ck = ok ? conv_silu(a, kc, (int)t) : 0.0f;
    const float qs = block_sum(cq * cq, red);
    const float ks = block_sum(ck * ck, red);
    const float inv = 1.0f / sqrtf((float)a.dk);
    const float qscale = 1.0f / sqrtf(qs / (float)a.dk + a.eps);
    const float kscale = 1.0f / sqrtf(ks / (float)a.dk + a.eps);
    if (ok) {
      row[qc] = cq * qscale * inv * inv;
      row[kc] = ck * kscale * inv;
      if (last) {
        shift_history(a, qc);
        shift_history(a, kc);
      }
    }
  } else {
    const uint32_t vh = u - a.key_heads;
    if (i < a.dv) {
      const uint32_t ch = 2 * key_el + vh * a.dv + i;
      row[ch] = conv_silu(a, ch, (int)t);
      if (last) shift_history(a, ch);
    }
  }
}

// grid: VH * ceil(dv / 16) blocks; thread (r = tid / 16, l = tid % 16) holds
// S[row0 + r][l + 16 e] for e < EPT (EPT * 16 >= dk).
template <int EPT>
__global__ __launch_bounds__(kThreads) void dn_scan_kernel(DnArgs a) {
  constexpr int kCols = 16 * EPT;
  __shared__ float qk_s[kTokChunk][2][kCols];
  __shared__ float v_s[kTokChunk][kRowsPerWg];
  __shared__ float o_s[kTokChunk][kRowsPerWg];
  __shared__ float g_s[kTokChunk], beta_s[kTokChunk];

  const uint32_t groups = (a.dv + kRowsPerWg - 1) / kRowsPerWg;
  const uint32_t vh = blockIdx.x / groups;
  const uint32_t row0 = (blockIdx.x % groups) * kRowsPerWg;
  const uint32_t kh = vh / (a.value_heads / a.key_heads);
  const uint32_t key_el = a.key_heads * a.dk;
  const int r = threadIdx.x / 16, l = threadIdx.x % 16;
  const uint32_t row = row0 + r;
  const bool row_ok = row < a.dv;

  float s[EPT];
  const size_t srow = ((size_t)vh * a.dv + row) * a.dk;
#pragma unroll
  for (int e = 0; e < EPT; ++e) {
    const uint32_t j = l + 16 * e;
    s[e] = row_ok && j < a.dk ? a.s_in[srow + j] : 0.0f;
  }
  const float neg_a = -expf(a.a_log[vh]);
  const float dt_bias = a.dt_bias[vh];

  for (uint32_t t0 = 0; t0 < a.M; t0 += kTokChunk) {
    const uint32_t nt = min((uint32_t)kTokChunk, a.M - t0);
    for (uint32_t idx = threadIdx.x; idx < kTokChunk * kCols; idx += kThreads) {
      const uint32_t tt = idx / kCols, j = idx % kCols;
      const bool ok = tt < nt && j < a.dk;
      const float* crow = a.conv_out + (size_t)(t0 + tt) * a.channels;
      qk_s[tt][0][j] = ok ? crow[kh * a.dk + j] : 0.0f;
      qk_s[tt][1][j] = ok ? crow[key_el + kh * a.dk + j] : 0.0f;
    }
    for (uint32_t idx = threadIdx.x; idx < kTokChunk * kRowsPerWg; idx += kThreads) {
      const uint32_t tt = idx / kRowsPerWg, rr = idx % kRowsPerWg;
      const bool ok = tt < nt && row0 + rr < a.dv;
      v_s[tt][rr] = ok ? a.conv_out[(size_t)(t0 + tt) * a.channels + 2 * key_el + vh * a.dv + row0 + rr] : 0.0f;
    }
    if (threadIdx.x < nt) {
      const size_t ti = (size_t)(t0 + threadIdx.x) * a.value_heads + vh;
      g_s[threadIdx.x] = expf(neg_a * softplus_f(a.a[ti] + dt_bias));
      beta_s[threadIdx.x] = sigmoid_f(a.b[ti]);
    }
    __syncthreads();

    for (uint32_t tt = 0; tt < nt; ++tt) {
      const float g = g_s[tt], beta = beta_s[tt];
      float kv_mem = 0.0f;
#pragma unroll
      for (int e = 0; e < EPT; ++e) {
        s[e] *= g;
        kv_mem += s[e] * qk_s[tt][1][l + 16 * e];
      }
#pragma unroll
      for (int off = 8; off >= 1; off >>= 1) kv_mem += __shfl_xor(kv_mem, off);
      const float delta = (v_s[tt][r] - kv_mem) * beta;
      float acc = 0.0f;
#pragma unroll
      for (int e = 0; e < EPT; ++e) {
        s[e] += qk_s[tt][1][l + 16 * e] * delta;
        acc += s[e] * qk_s[tt][0][l + 16 * e];
      }
#pragma unroll
      for (int off = 8; off >= 1; off >>= 1) acc += __shfl_xor(acc, off);
      if (l == 0) o_s[tt][r] = acc;
    }
    __syncthreads();
    for (uint32_t idx = threadIdx.x; idx < nt * kRowsPerWg; idx += kThreads) {
      const uint32_t tt = idx / kRowsPerWg, rr = idx % kRowsPerWg;
      if (row0 + rr < a.dv)
        a.out[(size_t)(t0 + tt) * a.value_heads * a.dv + vh * a.dv + row0 + rr] = o_s[tt][rr];
    }
    // The next chunk's staging overwrites qk_s / v_s only after every wave
    // passed the barrier above; o_s is rewritten after the next barrier.
  }

  if (row_ok) {
#pragma unroll
    for (int e = 0; e < EPT; ++e) {
      const uint32_t j = l + 16 * e;
      if (j < a.dk) a.s_out[srow + j] = s[e];
    }
  }
}

// grid: M * VH blocks of 256 threads; in place on `out`.
__global__ __launch_bounds__(kThreads) void dn_gate_norm_kernel(DnArgs a) {
  __shared__ float red[kThreads / 64];
  const uint32_t i = threadIdx.x;
  float* o = a.out + (size_t)blockIdx.x * a.dv;
  const float* z = a.z + (size_t)blockIdx.x * a.dv;
  const float v = i < a.dv ? o[i] : 0.0f;
  const float ss = block_sum(v * v, red);
  const float scale = 1.0f / sqrtf(ss / (float)a.dv + a.eps);
  if (i < a.dv) o[i] = v * scale * a.norm[i] * silu_f(z[i]);
}

template <int EPT>
void launch_scan(const DnArgs& a, hipStream_t st) {
  const uint32_t groups = (a.dv + kRowsPerWg - 1) / kRowsPerWg;
  hipLaunchKernelGGL(dn_scan_kernel<EPT>, dim3(a.value_heads * groups), dim3(kThreads), 0, st, a);
}

}  // namespace

hipError_t launch_deltanet(const DnArgs& a, hipStream_t st) {
  if (a.dk == 0 || a.dk > 256 || a.dv == 0 || a.dv > 256 || a.M == 0) return hipErrorInvalidValue;
  hipLaunchKernelGGL(dn_conv_prepare_kernel, dim3(a.M * (a.key_heads + a.value_heads)), dim3(kThreads), 0, st,
                     a);
  const uint32_t ept = (a.dk + 15) / 16;
  if (ept <= 1)
    launch_scan<1>(a, st);
  else if (ept <= 2)
    launch_scan<2>(a, st);
  else if (ept <= 4)
    launch_scan<4>(a, st);
  else if (ept <= 8)
    launch_scan<8>(a, st);
  else
    launch_scan<16>(a, st);
  hipLaunchKernelGGL(dn_gate_norm_kernel, dim3(a.M * a.value_heads), dim3(kThreads), 0, st, a);
  return hipGetLastError();
}

}  // namespace qm
