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
#include <stdlib.h>

#include <algorithm>

#include "common.h"
#include "deltanet.h"

namespace qm {
namespace {

constexpr int kThreads = 256;
typedef float f32x4 __attribute__((ext_vector_type(4)));
constexpr int kLanesPerRow = 16;                   // lanes sharing one S row in the scan
constexpr int kRowsPerWg = kThreads / kLanesPerRow;  // S rows per scan workgroup
constexpr int kTokChunk = 32;                      // tokens staged in LDS per scan iteration

// x(t) of channel ch: t >= 0 from this call's input, t < 0 from the history window.
__device__ __forceinline__ float conv_input(const DnArgs& a, uint32_t ch, int t) {
  const int hw = (int)a.kernel - 1;
  return t >= 0 ? a.qkv[(size_t)t * a.channels + ch] : a.hist_in[(size_t)ch * hw + hw + t];
}

// History window after token t (inputs t - hw + 1 .. t) into dst.
__device__ __forceinline__ void shift_history(const DnArgs& a, uint32_t ch, int t, float* dst) {
  const int hw = (int)a.kernel - 1;
  for (int tap = 0; tap < hw; ++tap) dst[(size_t)ch * hw + tap] = conv_input(a, ch, t - hw + 1 + tap);
}
// Where token t's history window goes: the state's new buffer after the last
// token, a snapshot image after an earlier one, else nowhere.
__device__ __forceinline__ float* history_target(const DnArgs& a, uint32_t t) {
  if (a.kernel <= 1) return nullptr;
  if (t + 1 == a.M) return a.hist_out;
  return t < a.snap_rows ? a.snap_hist + (size_t)t * a.snap_hist_stride : nullptr;
}

// Operands of one conv output for kernels of up to kTaps taps: tap j holds
// weight w[j] and input x(t - hw + j).  Loaded in one batch (addresses picked
// by select, no branches) so that several outputs' loads are in flight
// together; conv_finish then forms the sum in the order of the loop below.
constexpr int kTaps = 4;
struct ConvIn {
  float w[kTaps], x[kTaps];
};
__device__ __forceinline__ void conv_load(const DnArgs& a, uint32_t ch, int t, ConvIn& c) {
  const int hw = (int)a.kernel - 1;
#pragma unroll
  for (int j = 0; j < kTaps; ++j) {
    // Taps past the kernel read a valid address and are zeroed, so every
    // load is unconditional.
    const int jj = j <= hw ? j : hw;
    const int tj = t - hw + jj;
    const float* src = tj >= 0 ? a.qkv + (size_t)tj * a.channels + ch : a.hist_in + (size_t)ch * hw + hw + tj;
    const float wv = a.conv_w[(size_t)ch * a.kernel + jj];
    const float xv = *src;
    c.w[j] = j <= hw ? wv : 0.0f;
    c.x[j] = j <= hw ? xv : 0.0f;
  }
}
// History window after the token of c: inputs x(t - hw + 1 .. t), taps 1..hw.
__device__ __forceinline__ void conv_store_history(const DnArgs& a, uint32_t ch, const ConvIn& c, float* dst) {
  const int hw = (int)a.kernel - 1;
#pragma unroll
  for (int j = 0; j < kTaps - 1; ++j)
    if (j < hw) dst[(size_t)ch * hw + j] = c.x[j + 1];
}
__device__ __forceinline__ float conv_finish(const DnArgs& a, const ConvIn& c) {
  const int hw = (int)a.kernel - 1;
  float wl = c.w[0], xl = c.x[0];
#pragma unroll
  for (int j = 1; j < kTaps; ++j) {
    wl = hw == j ? c.w[j] : wl;
    xl = hw == j ? c.x[j] : xl;
  }
  // Roundings spelled out (one product, then fused multiply-adds) so that
  // every kernel computing a conv output rounds it identically.
  float sum = __fmul_rn(wl, xl);
#pragma unroll
  for (int j = 0; j < kTaps - 1; ++j)
    if (j < hw) sum = fmaf(c.w[j], c.x[j], sum);
  return silu_f(sum);
}
// Longer kernels: the same sum, one tap at a time.
__device__ __forceinline__ float conv_silu_loop(const DnArgs& a, uint32_t ch, int t) {
  const int hw = (int)a.kernel - 1;
  const float* w = a.conv_w + (size_t)ch * a.kernel;
  float sum = __fmul_rn(w[hw], conv_input(a, ch, t));
  for (int tap = 0; tap < hw; ++tap) sum = fmaf(w[tap], conv_input(a, ch, t - hw + tap), sum);
  return silu_f(sum);
}
// One conv output; with a history target it also writes the channel's window
// after token t there.
__device__ __forceinline__ float conv_silu(const DnArgs& a, uint32_t ch, int t, float* hist_dst) {
  if (a.kernel > kTaps) {
    const float y = conv_silu_loop(a, ch, t);
    if (hist_dst) shift_history(a, ch, t, hist_dst);
    return y;
  }
  ConvIn c;
  conv_load(a, ch, t, c);
  if (hist_dst) conv_store_history(a, ch, c, hist_dst);
  return conv_finish(a, c);
}


// Sum over the 16 lanes of a DPP row: quad swaps, then rotations by 4 and 8
// within the row; every lane ends with the total.
__device__ __forceinline__ float row16_sum(float v) {
  v += __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), 0xB1, 0xF, 0xF, false));  // quad [1,0,3,2]
  v += __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), 0x4E, 0xF, 0xF, false));  // quad [2,3,0,1]
  v += __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), 0x124, 0xF, 0xF, false));  // row_ror:4
  v += __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), 0x128, 0xF, 0xF, false));  // row_ror:8
  return v;
}
// Sum over the 64 lanes of a wave: the 16-lane rows, then the row pairs and
// halves meet through v_permlane16_swap / v_permlane32_swap.
__device__ __forceinline__ float wave_sum(float v) {
  v = row16_sum(v);
  const auto p = __builtin_amdgcn_permlane16_swap(__float_as_uint(v), __float_as_uint(v), false, false);
  v = __uint_as_float(p[0]) + __uint_as_float(p[1]);
  const auto q = __builtin_amdgcn_permlane32_swap(__float_as_uint(v), __float_as_uint(v), false, false);
  return __uint_as_float(q[0]) + __uint_as_float(q[1]);
}
// Sum over the lanes sharing one S row in the scan.
__device__ __forceinline__ float row_sum(float v) {
  static_assert(kLanesPerRow == 16, "one DPP row per S row");
  return row16_sum(v);
}

// q^ and k^ of key head kh at token t, computed by one wave: lane holds
// channels c = lane + 64 i (i < 4; dk <= 256).  Shared by the prefill path
// and the step kernels so both round identically.
// NQ: channel slots per lane that can be live (ceil(dk / 64)); the others
// stay zero, as they would with all four slots (their squares add nothing).
// PART: 1 = q only, 2 = k only, 3 = both (each with the same operations).
template <int NQ = 4, int PART = 3>
__device__ __forceinline__ void prep_key_head(const DnArgs& a, uint32_t t, uint32_t kh, uint32_t lane, float (&qo)[4],
                                              float (&ko)[4], float* hist_dst) {
  static_assert(NQ >= 1 && NQ <= 4, "slots");
  const uint32_t key_el = a.key_heads * a.dk;
  float qs = 0.0f, ks = 0.0f;
#pragma unroll
  for (int i = NQ; i < 4; ++i) qo[i] = ko[i] = 0.0f;
  if (a.kernel <= kTaps) {
    // All operands of the lane's (up to 8) outputs in flight at once.
    ConvIn cq[4], ck[4];
#pragma unroll
    for (int i = 0; i < NQ; ++i) {
      const uint32_t c = min(lane + 64 * i, a.dk - 1);
      if (PART & 1) conv_load(a, kh * a.dk + c, (int)t, cq[i]);
      if (PART & 2) conv_load(a, key_el + kh * a.dk + c, (int)t, ck[i]);
    }
#pragma unroll
    for (int i = 0; i < NQ; ++i) {
      const uint32_t c = lane + 64 * i;
      const bool ok = c < a.dk;
      qo[i] = ok && (PART & 1) ? conv_finish(a, cq[i]) : 0.0f;
      ko[i] = ok && (PART & 2) ? conv_finish(a, ck[i]) : 0.0f;
      if (ok && hist_dst) {
        if (PART & 1) conv_store_history(a, kh * a.dk + c, cq[i], hist_dst);
        if (PART & 2) conv_store_history(a, key_el + kh * a.dk + c, ck[i], hist_dst);
      }
    }
  } else {
#pragma unroll
    for (int i = 0; i < NQ; ++i) {
      const uint32_t c = lane + 64 * i;
      const bool ok = c < a.dk;
      qo[i] = ok && (PART & 1) ? conv_silu_loop(a, kh * a.dk + c, (int)t) : 0.0f;
      ko[i] = ok && (PART & 2) ? conv_silu_loop(a, key_el + kh * a.dk + c, (int)t) : 0.0f;
      if (ok && hist_dst) {
        if (PART & 1) shift_history(a, kh * a.dk + c, (int)t, hist_dst);
        if (PART & 2) shift_history(a, key_el + kh * a.dk + c, (int)t, hist_dst);
      }
    }
  }
#pragma unroll
  for (int i = 0; i < NQ; ++i) {
    qs = fmaf(qo[i], qo[i], qs);
    ks = fmaf(ko[i], ko[i], ks);
  }
  if (PART & 1) qs = wave_sum(qs);
  if (PART & 2) ks = wave_sum(ks);
  const float inv = 1.0f / sqrtf((float)a.dk);
  const float qscale = 1.0f / sqrtf(qs / (float)a.dk + a.eps);
  const float kscale = 1.0f / sqrtf(ks / (float)a.dk + a.eps);
#pragma unroll
  for (int i = 0; i < NQ; ++i) {
    qo[i] = qo[i] * qscale * inv * inv;
    ko[i] = ko[i] * kscale * inv;
  }
}

// One wave per (token, unit); blocks of 1 or 4 waves (grid covers every item).
// A key unit convolves its head's q and k channels and rms-normalises both
// (wave reductions, no barriers); a value unit convolves its v channels.
__global__ __launch_bounds__(kThreads) void dn_conv_prepare_kernel(DnArgs a) {
  const uint32_t units = a.key_heads + a.value_heads;
  const uint32_t item = blockIdx.x * (blockDim.x >> 6) + (threadIdx.x >> 6);
  if (item >= a.M * units) return;
  const uint32_t t = item / units, u = item % units;
  const uint32_t lane = threadIdx.x & 63;
  const uint32_t key_el = a.key_heads * a.dk;
  float* row = a.conv_out + (size_t)t * a.channels;
  float* hist_dst = history_target(a, t);
  if (u < a.key_heads) {
    float cq[4], ck[4];
    prep_key_head(a, t, u, lane, cq, ck, hist_dst);
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const uint32_t c = lane + 64 * i;
      if (c < a.dk) {
        row[u * a.dk + c] = cq[i];
        row[key_el + u * a.dk + c] = ck[i];
      }
    }
  } else {
    const uint32_t vh = u - a.key_heads;
    for (uint32_t c = lane; c < a.dv; c += 64) {
      const uint32_t ch = 2 * key_el + vh * a.dv + c;
      row[ch] = conv_silu(a, ch, (int)t, hist_dst);
    }
  }
}

// One token of the delta rule on the EPT-element segment of one S row that a
// lane holds (lane l: columns l + 16 e): returns o = S q^ for the row (all
// 16 lanes of the row get it).  Shared by the scan and the step kernels.
template <int EPT>
__device__ __forceinline__ float delta_row_token(float (&s)[EPT], const float (&kk)[EPT], const float (&qq)[EPT],
                                                 float g, float beta, float v) {
  float m0 = 0.0f, m1 = 0.0f;
#pragma unroll
  for (int e = 0; e < EPT; ++e) {
    s[e] *= g;
    if (e & 1)
      m1 = fmaf(s[e], kk[e], m1);
    else
      m0 = fmaf(s[e], kk[e], m0);
  }
  const float kv_mem = row_sum(m0 + m1);
  const float delta = (v - kv_mem) * beta;
  float a0 = 0.0f, a1 = 0.0f;
#pragma unroll
  for (int e = 0; e < EPT; ++e) {
    s[e] = fmaf(kk[e], delta, s[e]);
    if (e & 1)
      a1 = fmaf(s[e], qq[e], a1);
    else
      a0 = fmaf(s[e], qq[e], a0);
  }
  return row_sum(a0 + a1);
}

// grid: VH * ceil(dv / 16) blocks; thread (r = tid / 16, l = tid % 16) holds
// S[row0 + r][l + 16 e] for e < EPT (EPT * 16 >= dk).  Per token: two
// 16-lane DPP reductions, k^ and q^ read as EPT contiguous floats per lane.
// The next chunk of 32 tokens is fetched into registers while the current
// one is scanned.
template <int EPT>
__global__ __launch_bounds__(kThreads) void dn_scan_kernel(DnArgs a) {
  constexpr int kCols = kLanesPerRow * EPT;
  constexpr int kStage = kTokChunk * 2 * kCols / kThreads;  // k^/q^ floats per thread per chunk
  constexpr int kVStage = kTokChunk * kRowsPerWg / kThreads;  // v floats per thread per chunk
  static_assert(kStage * kThreads == kTokChunk * 2 * kCols && kVStage * kThreads == kTokChunk * kRowsPerWg,
                "staging split");
  // [token][q | k][lane][e]: lane l's EPT values are contiguous.
  __shared__ __attribute__((aligned(16))) float qk_s[kTokChunk][2][kLanesPerRow][EPT];
  __shared__ float v_s[kTokChunk][kRowsPerWg];
  __shared__ float o_s[kTokChunk][kRowsPerWg];
  __shared__ float g_s[kTokChunk], beta_s[kTokChunk];

  const uint32_t groups = (a.dv + kRowsPerWg - 1) / kRowsPerWg;
  const uint32_t vh = blockIdx.x / groups;
  const uint32_t row0 = (blockIdx.x % groups) * kRowsPerWg;
  const uint32_t kh = vh / (a.value_heads / a.key_heads);
  const uint32_t key_el = a.key_heads * a.dk;
  const int r = threadIdx.x / kLanesPerRow, l = threadIdx.x % kLanesPerRow;
  const uint32_t row = row0 + r;
  const bool row_ok = row < a.dv;

  float s[EPT];
  const size_t srow = ((size_t)vh * a.dv + row) * a.dk;
#pragma unroll
  for (int e = 0; e < EPT; ++e) {
    const uint32_t j = l + kLanesPerRow * e;
    s[e] = row_ok && j < a.dk ? a.s_in[srow + j] : 0.0f;
  }
  const float neg_a = -expf(a.a_log[vh]);
  const float dt_bias = a.dt_bias[vh];

  // Chunk staging registers: element p of thread t is flat index t + 256 p of
  // [token][q | k][column] (coalesced global reads), v likewise over [token][row].
  float qk_r[kStage], v_r[kVStage], a_r = 0.0f, b_r = 0.0f;
  auto fetch = [&](uint32_t t0) __attribute__((always_inline)) {
    const uint32_t nt = min((uint32_t)kTokChunk, a.M - t0);
#pragma unroll
    for (int p = 0; p < kStage; ++p) {
      const uint32_t idx = threadIdx.x + kThreads * p;
      const uint32_t tt = idx / (2 * kCols), kind = (idx / kCols) & 1, j = idx % kCols;
      const bool ok = tt < nt && j < a.dk;
      const float* crow = a.conv_out + (size_t)(t0 + tt) * a.channels;
      qk_r[p] = ok ? crow[(kind ? key_el : 0) + kh * a.dk + j] : 0.0f;
    }
#pragma unroll
    for (int p = 0; p < kVStage; ++p) {
      const uint32_t idx = threadIdx.x + kThreads * p;
      const uint32_t tt = idx / kRowsPerWg, rr = idx % kRowsPerWg;
      const bool ok = tt < nt && row0 + rr < a.dv;
      v_r[p] = ok ? a.conv_out[(size_t)(t0 + tt) * a.channels + 2 * key_el + vh * a.dv + row0 + rr] : 0.0f;
    }
    if (threadIdx.x < nt) {
      const size_t ti = (size_t)(t0 + threadIdx.x) * a.value_heads + vh;
      a_r = a.a[ti];
      b_r = a.b[ti];
    }
  };
  auto stage = [&](uint32_t t0) __attribute__((always_inline)) {
    const uint32_t nt = min((uint32_t)kTokChunk, a.M - t0);
#pragma unroll
    for (int p = 0; p < kStage; ++p) {
      const uint32_t idx = threadIdx.x + kThreads * p;
      const uint32_t tt = idx / (2 * kCols), kind = (idx / kCols) & 1, j = idx % kCols;
      qk_s[tt][kind][j % kLanesPerRow][j / kLanesPerRow] = qk_r[p];
    }
#pragma unroll
    for (int p = 0; p < kVStage; ++p) {
      const uint32_t idx = threadIdx.x + kThreads * p;
      v_s[idx / kRowsPerWg][idx % kRowsPerWg] = v_r[p];
    }
    if (threadIdx.x < nt) {
      g_s[threadIdx.x] = expf(neg_a * softplus_f(a_r + dt_bias));
      beta_s[threadIdx.x] = sigmoid_f(b_r);
    }
  };

  fetch(0);
  stage(0);
  __syncthreads();
  for (uint32_t t0 = 0; t0 < a.M; t0 += kTokChunk) {
    const uint32_t nt = min((uint32_t)kTokChunk, a.M - t0);
    const bool more = t0 + kTokChunk < a.M;
    if (more) fetch(t0 + kTokChunk);

#pragma unroll 2
    for (uint32_t tt = 0; tt < nt; ++tt) {
      const float g = g_s[tt], beta = beta_s[tt];
      float kk[EPT], qq[EPT];
      if constexpr (EPT % 4 == 0) {
#pragma unroll
        for (int e4 = 0; e4 < EPT; e4 += 4) {
          const floatx4 k4 = *(const floatx4*)&qk_s[tt][1][l][e4];
          const floatx4 q4 = *(const floatx4*)&qk_s[tt][0][l][e4];
#pragma unroll
          for (int i = 0; i < 4; ++i) {
            kk[e4 + i] = k4[i];
            qq[e4 + i] = q4[i];
          }
        }
      } else {
#pragma unroll
        for (int e = 0; e < EPT; ++e) {
          kk[e] = qk_s[tt][1][l][e];
          qq[e] = qk_s[tt][0][l][e];
        }
      }
      const float acc = delta_row_token<EPT>(s, kk, qq, g, beta, v_s[tt][r]);
      if (l == 0) o_s[tt][r] = acc;
      if (t0 + tt < a.snap_rows && row_ok) {  // state image after this token
        float* img = a.snap_s + (size_t)(t0 + tt) * a.snap_s_stride + srow;
#pragma unroll
        for (int e = 0; e < EPT; ++e) {
          const uint32_t j = l + kLanesPerRow * e;
          if (j < a.dk) img[j] = s[e];
        }
      }
    }
    __syncthreads();  // every wave is done with this chunk's LDS
    for (uint32_t idx = threadIdx.x; idx < nt * kRowsPerWg; idx += kThreads) {
      const uint32_t tt = idx / kRowsPerWg, rr = idx % kRowsPerWg;
      if (row0 + rr < a.dv)
        a.out[(size_t)(t0 + tt) * a.value_heads * a.dv + vh * a.dv + row0 + rr] = o_s[tt][rr];
    }
    if (more) {
      stage(t0 + kTokChunk);
      __syncthreads();
    }
  }

  if (row_ok) {
#pragma unroll
    for (int e = 0; e < EPT; ++e) {
      const uint32_t j = l + kLanesPerRow * e;
      if (j < a.dk) a.s_out[srow + j] = s[e];
    }
  }
}

// Gated RMS norm of (token, value head) output rows: out[c] = o *
// rsqrt(mean o^2 + eps) * norm * silu(z).  A row is held by LPR lanes (64, or
// 32 when dv <= 128 so two rows share a wave); lane rl of the row holds
// elements 4 rl .. 4 rl + 3 (dv <= 256).  The sum of squares is reduced over
// the row's lanes; with dv <= 128 a 64-lane row's upper lanes add only zeros,
// so both widths give the same bits.
__device__ __forceinline__ float half_sum(float v) {  // wave_sum within each 32-lane half
  v = row16_sum(v);
  const auto p = __builtin_amdgcn_permlane16_swap(__float_as_uint(v), __float_as_uint(v), false, false);
  return __uint_as_float(p[0]) + __uint_as_float(p[1]);
}
template <int LPR = 64, bool VEC = false>
__device__ __forceinline__ void gate_norm_core(const DnArgs& a, const float (&v)[4], const float (&nrm)[4],
                                               const float (&sz)[4], float* out, uint32_t rl, uint16_t* out_bf16,
                                               bool live = true) {
  float ss = 0.0f;
#pragma unroll
  for (int i = 0; i < 4; ++i) ss += v[i] * v[i];
  ss = LPR == 64 ? wave_sum(ss) : half_sum(ss);
  const float scale = 1.0f / sqrtf(ss / (float)a.dv + a.eps);
  if (!live) return;
  if (VEC) {  // dv % 4 == 0: the lane's four elements are all in the row or all past it
    if (4 * rl < a.dv) {
      f32x4 r;
#pragma unroll
      for (int i = 0; i < 4; ++i) r[i] = v[i] * scale * nrm[i] * sz[i];
      *(f32x4*)(out + 4 * rl) = r;
    }
    return;
  }
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const uint32_t c = 4 * rl + i;
    if (c < a.dv) {
      const float r = v[i] * scale * nrm[i] * sz[i];
      out[c] = r;
      if (out_bf16) out_bf16[c] = f32_to_bf16(r);
    }
  }
}
// Norm weights and silu(z) of one row (zero past dv).
__device__ __forceinline__ void gate_norm_operands(const DnArgs& a, const float* z, uint32_t rl, float (&nrm)[4],
                                                   float (&sz)[4]) {
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const uint32_t c = 4 * rl + i;
    nrm[i] = c < a.dv ? a.norm[c] : 0.0f;
    sz[i] = c < a.dv ? silu_f(z[c]) : 0.0f;
  }
}
// The same operands in two halves, so the loads can go out early and the
// SiLU wait for them only where it is needed: raw loads (clamped
// addresses), then the zeroing past dv and silu(z).
__device__ __forceinline__ void gate_norm_load(const DnArgs& a, const float* z, uint32_t rl, float (&nrm)[4],
                                               float (&zr)[4]) {
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const uint32_t c = min(4 * rl + i, a.dv - 1);
    nrm[i] = a.norm[c];
    zr[i] = z[c];
  }
}
__device__ __forceinline__ void gate_norm_finish(const DnArgs& a, uint32_t rl, float (&nrm)[4], const float (&zr)[4],
                                                 float (&sz)[4]) {
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const bool ok = 4 * rl + i < a.dv;
    nrm[i] = ok ? nrm[i] : 0.0f;
    sz[i] = ok ? silu_f(zr[i]) : 0.0f;
  }
}
// In place on `out`, kNormSlots x (64 / LPR) rows per wave, all of their
// loads (16 bytes a lane when VEC, dv % 4 == 0) issued before the first row
// is normalised; the per-row arithmetic is gate_norm_core's.
constexpr int kNormSlots = 4;
template <int LPR, bool VEC>
__global__ __launch_bounds__(kThreads) void dn_gate_norm_kernel(DnArgs a) {
  constexpr int kRows = 64 / LPR;  // rows per slot
  const uint32_t items = a.M * a.value_heads;
  const uint32_t first = (blockIdx.x * (blockDim.x >> 6) + (threadIdx.x >> 6)) * kNormSlots * kRows;
  if (first >= items) return;
  const uint32_t lane = threadIdx.x & 63, rl = lane % LPR, hs = lane / LPR;
  const bool lane_live = 4 * rl < a.dv;
  float v[kNormSlots][4], sz[kNormSlots][4], nrm[4];
#pragma unroll
  for (int q = 0; q < kNormSlots; ++q) {
    const size_t base = (size_t)min(first + q * kRows + hs, items - 1) * a.dv + 4 * min(rl, (a.dv - 1) / 4);
    if (VEC) {
      const f32x4 ov = *(const f32x4*)(a.out + base), zv = *(const f32x4*)(a.z + base);
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        v[q][i] = lane_live ? ov[i] : 0.0f;
        sz[q][i] = lane_live ? zv[i] : 0.0f;
      }
    } else {
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const bool ok = 4 * rl + i < a.dv;
        v[q][i] = ok ? a.out[base + i] : 0.0f;
        sz[q][i] = ok ? a.z[base + i] : 0.0f;
      }
    }
  }
#pragma unroll
  for (int i = 0; i < 4; ++i) nrm[i] = 4 * rl + i < a.dv ? a.norm[4 * rl + i] : 0.0f;
#pragma unroll
  for (int q = 0; q < kNormSlots; ++q) {
    if (first + q * kRows >= items) break;  // wave-uniform
    const uint32_t row = first + q * kRows + hs;
#pragma unroll
    for (int i = 0; i < 4; ++i) sz[q][i] = silu_f(sz[q][i]);  // gate_norm_operands
    gate_norm_core<LPR, VEC>(a, v[q], nrm, sz[q], a.out + (size_t)row * a.dv, rl, nullptr, row < items);
  }
}

// Rows of S per pass of the split step kernel's 256 threads (16 lanes a row).
constexpr int kStepThreads = 256;
constexpr int kStepRows = kStepThreads / 16;

// The decode step with one 1024-thread workgroup per value head (dv <= 128):
// 64 rows of S per pass, so a head takes at most two passes, and the gated
// norm has all dv outputs in its own LDS: no exchange between workgroups.
// Waves 0 and 2 prepare q^ and k^ (one half each), wave 1 convolves the
// head's v channels, thread 192 forms g and beta.  Every output is formed by
// the device functions of the other step kernels and the prefill path, so
// a step still equals a one-token prefill bit for bit.
constexpr int kHeadThreads = 1024;
constexpr int kHeadRows = kHeadThreads / 16;  // S rows per pass
template <int EPT>
__global__ __launch_bounds__(kHeadThreads) void dn_step_head_kernel(DnArgs a) {
  constexpr int PASSES = 2;
  __shared__ __attribute__((aligned(16))) float qk_s[2][16][EPT];  // [q | k][lane][e]
  __shared__ float v_s[kHeadRows * PASSES], o_s[kHeadRows * PASSES];
  __shared__ float gb_s[2];
  const uint32_t vh = blockIdx.x;
  const uint32_t group = a.value_heads / a.key_heads;
  const uint32_t kh = vh / group;
  const uint32_t key_el = a.key_heads * a.dk;
  const uint32_t wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6), lane = threadIdx.x & 63;
  const bool key_hist = vh % group == 0 && a.kernel > 1;

  const int r = threadIdx.x / 16, l = threadIdx.x % 16;
  float s[PASSES][EPT];
#pragma unroll
  for (int p = 0; p < PASSES; ++p) {
    const uint32_t row = kHeadRows * p + r;
    const size_t srow = ((size_t)vh * a.dv + row) * a.dk;
#pragma unroll
    for (int e = 0; e < EPT; ++e) {
      const uint32_t j = l + 16 * e;
      s[p][e] = row < a.dv && j < a.dk ? a.s_in[srow + j] : 0.0f;
    }
  }

  // Wave 0 loads the gated norm's operands first (it applies the norm at the
  // end, and forms silu(z) only then), then prepares q^; wave 2 prepares k^
  // meanwhile.
  float nrm[4], zr[4], sz[4];
  if (wave == 0 || wave == 2) {
    if (wave == 0) gate_norm_load(a, a.z + (size_t)vh * a.dv, lane, nrm, zr);
    float cq[4], ck[4];
    if (wave == 0)
      prep_key_head<EPT / 4, 1>(a, 0, kh, lane, cq, ck, key_hist ? a.hist_out : nullptr);
    else
      prep_key_head<EPT / 4, 2>(a, 0, kh, lane, cq, ck, key_hist ? a.hist_out : nullptr);
    const int qk = wave == 0 ? 0 : 1;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const uint32_t c = lane + 64 * i;
      if (c < 16 * EPT) qk_s[qk][c % 16][c / 16] = c < a.dk ? (qk == 0 ? cq[i] : ck[i]) : 0.0f;
    }
  } else if (wave == 1) {
    constexpr int kV = (kHeadRows * PASSES + 63) / 64;
    if (a.kernel <= kTaps) {
      ConvIn cv[kV];
#pragma unroll
      for (int i = 0; i < kV; ++i) conv_load(a, 2 * key_el + vh * a.dv + min(lane + 64 * i, a.dv - 1), 0, cv[i]);
#pragma unroll
      for (int i = 0; i < kV; ++i) {
        const uint32_t c = lane + 64 * i;
        if (c < kHeadRows * PASSES) v_s[c] = c < a.dv ? conv_finish(a, cv[i]) : 0.0f;
        if (c < a.dv && a.kernel > 1) conv_store_history(a, 2 * key_el + vh * a.dv + c, cv[i], a.hist_out);
      }
    } else {
      for (uint32_t c = lane; c < kHeadRows * PASSES; c += 64) {
        const uint32_t ch = 2 * key_el + vh * a.dv + c;
        v_s[c] = c < a.dv ? conv_silu(a, ch, 0, a.kernel > 1 && c < a.dv ? a.hist_out : nullptr) : 0.0f;
      }
    }
  } else if (threadIdx.x == 192) {
    const float neg_a = -expf(a.a_log[vh]);
    gb_s[0] = expf(neg_a * softplus_f(a.a[vh] + a.dt_bias[vh]));
    gb_s[1] = sigmoid_f(a.b[vh]);
  }
  __syncthreads();

  float kk[EPT], qq[EPT];
#pragma unroll
  for (int e = 0; e < EPT; ++e) {
    kk[e] = qk_s[1][l][e];
    qq[e] = qk_s[0][l][e];
  }
  const float g = gb_s[0], beta = gb_s[1];
#pragma unroll
  for (int p = 0; p < PASSES; ++p) {
    const uint32_t row = kHeadRows * p + r;
    const float o = delta_row_token<EPT>(s[p], kk, qq, g, beta, v_s[row]);
    if (l == 0) o_s[row] = o;
    if (row < a.dv) {
      const size_t srow = ((size_t)vh * a.dv + row) * a.dk;
#pragma unroll
      for (int e = 0; e < EPT; ++e) {
        const uint32_t j = l + 16 * e;
        if (j < a.dk) a.s_out[srow + j] = s[p][e];
      }
    }
  }
  __syncthreads();
  if (wave == 0) {
    gate_norm_finish(a, lane, nrm, zr, sz);
    float ov[4];
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const uint32_t c = 4 * lane + i;
      ov[i] = c < a.dv ? o_s[c] : 0.0f;
    }
    gate_norm_core(a, ov, nrm, sz, a.out + (size_t)vh * a.dv, lane,
                   a.out_bf16 ? a.out_bf16 + (size_t)vh * a.dv : nullptr);
  }
}

// The decode step split over 16-row groups of S: grid VH * ceil(dv / 16),
// one workgroup per (value head, row group), so the 4 MiB of S stream from
// every CU instead of one per head.  Per workgroup:
//  waves 0 and 2: q^ and k^ of key head kh (prep_key_head, one half each;
//          only group 0 of the first value head of the key group writes that
//          key head's history);
//  wave 1: conv of the group's 16 v channels;
//  thread 192: g and beta;
// then the 16-lane row groups update the 16 rows (delta_row_token).  The
// gated norm needs all dv outputs of the head: every group stores its o
// values (written through to memory) and counts itself in; the last of the
// head's groups to arrive reads the dv values back and applies
// gate_norm_core.  Every output is formed by the same device functions as in
// the per-head step and the prefill path, so a step still equals a one-token
// prefill bit for bit.
template <int EPT>
__global__ __launch_bounds__(kStepThreads) void dn_step_split_kernel(DnArgs a) {
  __shared__ __attribute__((aligned(16))) float qk_s[2][16][EPT];  // [q | k][lane][e]
  __shared__ float v_s[kStepRows];
  __shared__ float gb_s[2];
  __shared__ unsigned last_s;
  const uint32_t groups = (a.dv + kStepRows - 1) / kStepRows;
  const uint32_t vh = blockIdx.x / groups, rg = blockIdx.x % groups;
  const uint32_t row0 = rg * kStepRows;
  const uint32_t group = a.value_heads / a.key_heads;
  const uint32_t kh = vh / group;
  const uint32_t key_el = a.key_heads * a.dk;
  const uint32_t wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6), lane = threadIdx.x & 63;
  const bool key_hist = rg == 0 && vh % group == 0 && a.kernel > 1;

  const int r = threadIdx.x / 16, l = threadIdx.x % 16;
  const uint32_t row = row0 + r;
  const size_t srow = ((size_t)vh * a.dv + row) * a.dk;
  float s[EPT];
#pragma unroll
  for (int e = 0; e < EPT; ++e) {
    const uint32_t j = l + 16 * e;
    s[e] = row < a.dv && j < a.dk ? a.s_in[srow + j] : 0.0f;
  }

  // Wave 0 of every group loads the gated norm's operands early: the group
  // that arrives last needs them right away.
  float nrm[4], sz[4];
  if (wave == 0) {
    gate_norm_operands(a, a.z + (size_t)vh * a.dv, lane, nrm, sz);
    float cq[4], ck[4];
    prep_key_head<EPT / 4, 1>(a, 0, kh, lane, cq, ck, key_hist ? a.hist_out : nullptr);
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const uint32_t c = lane + 64 * i;
      if (c < 16 * EPT) qk_s[0][c % 16][c / 16] = c < a.dk ? cq[i] : 0.0f;
    }
  } else if (wave == 2) {
    float cq[4], ck[4];
    prep_key_head<EPT / 4, 2>(a, 0, kh, lane, cq, ck, key_hist ? a.hist_out : nullptr);
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const uint32_t c = lane + 64 * i;
      if (c < 16 * EPT) qk_s[1][c % 16][c / 16] = c < a.dk ? ck[i] : 0.0f;
    }
  } else if (wave == 1) {
    if (lane < kStepRows) {
      const uint32_t c = row0 + lane;
      const uint32_t ch = 2 * key_el + vh * a.dv + min(c, a.dv - 1);
      float vv = 0.0f;
      if (a.kernel <= kTaps) {
        ConvIn cv;
        conv_load(a, ch, 0, cv);
        vv = conv_finish(a, cv);
        if (c < a.dv && a.kernel > 1) conv_store_history(a, ch, cv, a.hist_out);
      } else {
        vv = conv_silu(a, ch, 0, c < a.dv && a.kernel > 1 ? a.hist_out : nullptr);
      }
      v_s[lane] = c < a.dv ? vv : 0.0f;
    }
  } else if (threadIdx.x == 192) {
    const float neg_a = -expf(a.a_log[vh]);
    gb_s[0] = expf(neg_a * softplus_f(a.a[vh] + a.dt_bias[vh]));
    gb_s[1] = sigmoid_f(a.b[vh]);
  }
  __syncthreads();

  float kk[EPT], qq[EPT];
#pragma unroll
  for (int e = 0; e < EPT; ++e) {
    kk[e] = qk_s[1][l][e];
    qq[e] = qk_s[0][l][e];
  }
  const float o = delta_row_token<EPT>(s, kk, qq, gb_s[0], gb_s[1], v_s[r]);
  if (row < a.dv) {
#pragma unroll
    for (int e = 0; e < EPT; ++e) {
      const uint32_t j = l + 16 * e;
      if (j < a.dk) a.s_out[srow + j] = s[e];
    }
  }
  // Publish this group's outputs, written through to memory (the head's
  // groups run on different XCDs, whose L2s are not coherent), and count in.
  constexpr int kSys = 0x11;  // sc0 sc1
  const __amdgpu_buffer_rsrc_t ro = __builtin_amdgcn_make_buffer_rsrc(
      a.step_o + (size_t)vh * a.dv, (short)0, (int)(a.dv * 4), 0x00020000);
  if (l == 0 && row < a.dv) __builtin_amdgcn_raw_buffer_store_b32(__float_as_uint(o), ro, row * 4, 0, kSys);
  __builtin_amdgcn_s_waitcnt(0x0F70);  // vmcnt(0): the stores are complete
  __syncthreads();
  if (threadIdx.x == 0) {
    const unsigned prev = __hip_atomic_fetch_add(a.step_ctr + vh, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    const bool last = prev == groups - 1;
    if (last) __hip_atomic_store(a.step_ctr + vh, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    last_s = last ? 1u : 0u;
  }
  __syncthreads();
  if (last_s == 0u || wave != 0) return;
  // The head's dv outputs (lane l: 4 l .. 4 l + 3), then the shared gated norm.
  float ov[4];
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const uint32_t c = 4 * lane + i;
    const float v = __uint_as_float(__builtin_amdgcn_raw_buffer_load_b32(ro, min(c, a.dv - 1) * 4, 0, kSys));
    ov[i] = c < a.dv ? v : 0.0f;
  }
  gate_norm_core(a, ov, nrm, sz, a.out + (size_t)vh * a.dv, lane,
                 a.out_bf16 ? a.out_bf16 + (size_t)vh * a.dv : nullptr);
}

// ---------------------------------------------------------------------------
// Prefill conv + prepare over token tiles
// ---------------------------------------------------------------------------
// One wave per (tile of kConvTile tokens, unit); 4 waves per block.  A lane
// keeps its channels' last kernel-1 inputs in registers and walks the tile,
// so every input is loaded once (the per-token kernel loads each kernel
// times), four tokens' inputs at a time.  The arithmetic is conv_finish /
// prep_key_head's, operation for operation, so the outputs equal the
// per-token kernel's bit for bit.  NS = channel slots per lane and class
// (ceil(head dim / 64)); kernels of up to kTaps taps.
constexpr int kConvTile = 32;
constexpr int kConvBatch = 4;  // tokens whose inputs are loaded together
// One wave's tile: KEY units carry q and k (2 NS slots), value units v (NS);
// HW = kernel - 1 history taps.
template <int NS, int HW, bool KEY>
__device__ __forceinline__ void conv_tile(const DnArgs& a, uint32_t tile, uint32_t u, uint32_t lane) {
  constexpr int S = KEY ? 2 * NS : NS;  // q slots 0..NS-1, k slots NS..2NS-1
  const uint32_t key_el = a.key_heads * a.dk;
  const uint32_t width = KEY ? a.dk : a.dv;
  uint32_t ch[S];
  bool ok[S];
#pragma unroll
  for (int i = 0; i < NS; ++i) {
    const uint32_t c = lane + 64 * i;
    const uint32_t cc = c < width ? c : 0;
    ok[i] = c < width;
    ch[i] = KEY ? u * a.dk + cc : 2 * key_el + (u - a.key_heads) * a.dv + cc;
    if (KEY) {
      ok[NS + i] = ok[i];
      ch[NS + i] = key_el + u * a.dk + cc;
    }
  }
  float w[S][HW + 1], win[S][HW + 1];  // win[s][j] = x(t - HW + j) for j < HW
  const int t0 = (int)(tile * kConvTile);
  const int t1 = min((int)a.M, t0 + kConvTile);
#pragma unroll
  for (int s = 0; s < S; ++s)
#pragma unroll
    for (int j = 0; j <= HW; ++j) {
      w[s][j] = a.conv_w[(size_t)ch[s] * a.kernel + j];
      win[s][j] = j < HW ? conv_input(a, ch[s], t0 - HW + j) : 0.0f;
    }
  const float inv = 1.0f / sqrtf((float)a.dk);
  // Inputs of kConvBatch tokens per batch; the next batch's loads are issued
  // before the current batch is computed.
  auto load_batch = [&](int tb, float (&xs)[kConvBatch][S]) __attribute__((always_inline)) {
#pragma unroll
    for (int k = 0; k < kConvBatch; ++k)
#pragma unroll
      for (int s = 0; s < S; ++s) xs[k][s] = a.qkv[(size_t)min(tb + k, t1 - 1) * a.channels + ch[s]];
  };
  float xn[kConvBatch][S];
  load_batch(t0, xn);
  for (int tb = t0; tb < t1; tb += kConvBatch) {
    float xs[kConvBatch][S];
#pragma unroll
    for (int k = 0; k < kConvBatch; ++k)
#pragma unroll
      for (int s = 0; s < S; ++s) xs[k][s] = xn[k][s];
    load_batch(tb + kConvBatch, xn);  // clamped to the tile: past its end a harmless reload
#pragma unroll
    for (int k = 0; k < kConvBatch; ++k) {
      const int t = tb + k;
      if (t >= t1) break;
      float* row = a.conv_out + (size_t)t * a.channels;
      float* hist_dst = history_target(a, (uint32_t)t);
      float y[S];
#pragma unroll
      for (int s = 0; s < S; ++s) {
        const float x = xs[k][s];
        // conv_finish's roundings: w[HW] * x(t), then taps 0 .. HW - 1 in order.
        float sum = __fmul_rn(w[s][HW], x);
#pragma unroll
        for (int jx = 0; jx < HW; ++jx) sum = fmaf(w[s][jx], win[s][jx], sum);
        y[s] = silu_f(sum);
        // Slide the window: x(t - HW + 1 .. t).
#pragma unroll
        for (int jx = 0; jx + 1 < HW; ++jx) win[s][jx] = win[s][jx + 1];
        if (HW > 0) win[s][HW - 1] = x;
        if (HW > 0 && hist_dst && ok[s]) {
#pragma unroll
          for (int jx = 0; jx < HW; ++jx) hist_dst[(size_t)ch[s] * HW + jx] = win[s][jx];
        }
      }
      if (KEY) {
        float qs = 0.0f, ks = 0.0f;
#pragma unroll
        for (int i = 0; i < NS; ++i) {
          const float yq = ok[i] ? y[i] : 0.0f, yk = ok[i] ? y[NS + i] : 0.0f;
          qs = fmaf(yq, yq, qs);
          ks = fmaf(yk, yk, ks);
        }
        qs = wave_sum(qs);
        ks = wave_sum(ks);
        const float qscale = 1.0f / sqrtf(qs / (float)a.dk + a.eps);
        const float kscale = 1.0f / sqrtf(ks / (float)a.dk + a.eps);
#pragma unroll
        for (int i = 0; i < NS; ++i)
          if (ok[i]) {
            row[ch[i]] = y[i] * qscale * inv * inv;
            row[ch[NS + i]] = y[NS + i] * kscale * inv;
          }
      } else {
#pragma unroll
        for (int i = 0; i < NS; ++i)
          if (ok[i]) row[ch[i]] = y[i];
      }
    }
  }
}
template <int NS, int HW>
__global__ __launch_bounds__(kThreads) void dn_conv_tiled_kernel(DnArgs a) {
  const uint32_t units = a.key_heads + a.value_heads;
  const uint32_t tiles = (a.M + kConvTile - 1) / kConvTile;
  const uint32_t item = blockIdx.x * (kThreads / 64) + (threadIdx.x >> 6);
  if (item >= tiles * units) return;
  // Units of one tile are consecutive: a block's waves share token rows.
  const uint32_t tile = item / units, u = item % units;
  const uint32_t lane = threadIdx.x & 63;
  if (u < a.key_heads)
    conv_tile<NS, HW, true>(a, tile, u, lane);
  else
    conv_tile<NS, HW, false>(a, tile, u, lane);
}

// ---------------------------------------------------------------------------
// Chunked scan (WY / UT form), head dims 128 / 128
// ---------------------------------------------------------------------------
// Within a chunk of C = 64 tokens (t = 0..63 from the chunk start), with
// per-token log decay lg_t = -e^{A_log} softplus(a_t + dt_bias), cumulative
// G_t = sum_{i<=t} lg_i, Gamma_t = e^{G_t}, the step recurrence
//   S_t = g_t S_{t-1} + u_t k_t^T,  u_t = beta_t (v_t - g_t S_{t-1} k_t)
// unrolls to S_t = Gamma_t S_0 + sum_{i<=t} e^{G_t - G_i} u_i k_i^T.  The
// pseudo-values u solve the unit lower-triangular system
//   (I + A) U = diag(beta) V - diag(beta Gamma) K S_0^T,
//   A_ti = beta_t e^{G_t - G_i} k_t.k_i  (i < t),
// so U = U~ - W S_0^T with W = (I+A)^{-1} diag(beta Gamma) K and
// U~ = (I+A)^{-1} diag(beta) V, which do not depend on S.  Per chunk then
//   O   = diag(Gamma) Q S_0^T + P U,   P_ti = e^{G_t - G_i} q_t.k_i (i <= t)
//   S_C = Gamma_C S_0 + U^T diag(e^{G_C - G_i}) K.
// dn_chunk_prep_kernel forms W, U~, P and G for every (chunk, value head) in
// parallel (fp32 MFMA for K K^T and Q K^T, a blocked MFMA solve), and q^, k^
// once per key head; dn_chunk_scan_kernel then walks the chunks in order.  Rows of S
// stay independent (row j of S only meets column j of U), so each workgroup
// owns 16 rows of one head in the same way as the token scan.
__device__ __forceinline__ floatx4 mfma_f32_4(float a, float b, floatx4 c) {
  return __builtin_amdgcn_mfma_f32_16x16x4f32(a, b, c, 0, 0, 0);
}

constexpr int kCD = 128;        // head dims of the chunked path
constexpr int kCStride = 132;   // LDS row stride (floats) of [64][128] tiles: conflict-free 16-byte reads
constexpr int kAStride = 68;    // LDS row stride of the 64 x 64 triangular matrix

// SiLU from the hardware exp2 and reciprocal (about 2 ulp; the chunked path
// is held to the fp64 oracle, not to the token-serial path's bits).
__device__ __forceinline__ float silu_fast(float v) {
  return v * __builtin_amdgcn_rcpf(1.0f + __builtin_amdgcn_exp2f(-v * 1.4426950408889634f));
}

// fp32 x = hi + lo + O(2^-18 |x|) in bf16 (both rounded to nearest even):
// products of split operands as hi*hi + hi*lo + lo*hi on the bf16 MFMA keep
// about 2^-17 relative error per product, against 2^-9 for plain bf16.
// Eight floats become the bf16x8 operands hi and lo (element e = float e).
__device__ __forceinline__ void split_bf16x8(const f32x4& a, const f32x4& b, u32x4& hi, u32x4& lo) {
  typedef __bf16 bf2 __attribute__((ext_vector_type(2)));
  const float v[8] = {a[0], a[1], a[2], a[3], b[0], b[1], b[2], b[3]};
#pragma unroll
  for (int p = 0; p < 4; ++p) {
    const bf2 h = {(__bf16)v[2 * p], (__bf16)v[2 * p + 1]};
    const uint32_t hb = __builtin_bit_cast(uint32_t, h);
    const bf2 l = {(__bf16)(v[2 * p] - __uint_as_float(hb << 16)),
                   (__bf16)(v[2 * p + 1] - __uint_as_float(hb & 0xFFFF0000u))};
    hi[p] = hb;
    lo[p] = __builtin_bit_cast(uint32_t, l);
  }
}
// Split-bf16 operand blocks in the workspace: block (nb, s) of an operand
// with S steps of 32 along its reduction dimension holds, for lane
// (j, g) = (lane % 16, lane / 16), the 8 elements [16 nb + j][32 s + 8 g + e]:
// hi at 8 lane + e, lo 512 further (in bf16 units; 2 KB per block).
__device__ __forceinline__ uint32_t dn_b3_block(uint32_t nb, uint32_t s, uint32_t S) { return (nb * S + s) * 1024; }

// The scan's B operands of one key head as split bf16 blocks (dn_b3_block),
// 2 x 16 bytes per item (1024 items each): k^^T[c][i] = k^[i][c] (8 column
// blocks, 2 steps over i) for the state update and q^[t][k] (4 token blocks,
// 4 steps over k) for the output.  The decays enter in the scan.
__device__ __forceinline__ void dn_chunk_store_k(const float* ks_s, uint16_t* kt3, uint32_t item) {
  const uint32_t ln = item % 64, blk = item / 64;  // blk = nb * 2 + s
  const uint32_t col = 16 * (blk / 2) + ln % 16, i0 = 32 * (blk % 2) + 8 * (ln / 16);
  f32x4 v0, v1;
#pragma unroll
  for (int e = 0; e < 4; ++e) {
    v0[e] = ks_s[(i0 + e) * kCStride + col];
    v1[e] = ks_s[(i0 + 4 + e) * kCStride + col];
  }
  u32x4 hi, lo;
  split_bf16x8(v0, v1, hi, lo);
  *(u32x4*)(kt3 + blk * 1024 + 8 * ln) = hi;
  *(u32x4*)(kt3 + blk * 1024 + 512 + 8 * ln) = lo;
}
__device__ __forceinline__ void dn_chunk_store_q(const float* qs_s, uint16_t* q3, uint32_t item) {
  const uint32_t ln = item % 64, blk = item / 64;  // blk = nb * 4 + s
  const uint32_t t = 16 * (blk / 4) + ln % 16, k0 = 32 * (blk % 4) + 8 * (ln / 16);
  const float* src = qs_s + t * kCStride + k0;
  u32x4 hi, lo;
  split_bf16x8(*(const f32x4*)src, *(const f32x4*)(src + 4), hi, lo);
  *(u32x4*)(q3 + blk * 1024 + 8 * ln) = hi;
  *(u32x4*)(q3 + blk * 1024 + 512 + 8 * ln) = lo;
}

// One 16 x 16 tile of X Y^T over the 128 columns of rows 16 tm .. of xs and
// 16 tn .. of ys ([64][kCStride] fp32 in LDS), on split-bf16 16x16x32 MFMAs:
// each operand is hi + lo in bf16, the product hi.hi + hi.lo + lo.hi with
// fp32 accumulation (about 2^-17 relative error per product, five times
// fewer MFMA cycles than 16x16x4 fp32).  Lane (j, grp) of the result holds
// rows 4 grp .. 4 grp + 3 of column j.
__device__ __forceinline__ floatx4 dn_gram_tile(const float* xs, const float* ys, int tm, int tn, uint32_t j,
                                                uint32_t grp) {
  const float* xa = xs + (16 * tm + j) * kCStride + 8 * grp;
  const float* yb = ys + (16 * tn + j) * kCStride + 8 * grp;
  floatx4 ac[3] = {{0.f, 0.f, 0.f, 0.f}, {0.f, 0.f, 0.f, 0.f}, {0.f, 0.f, 0.f, 0.f}};
#pragma unroll
  for (int m = 0; m < 4; ++m) {
    u32x4 ah, al, bh, bl;
    split_bf16x8(*(const f32x4*)(xa + 32 * m), *(const f32x4*)(xa + 32 * m + 4), ah, al);
    split_bf16x8(*(const f32x4*)(yb + 32 * m), *(const f32x4*)(yb + 32 * m + 4), bh, bl);
    ac[0] = mfma16x16x32(ah, bh, ac[0]);
    ac[1] = mfma16x16x32(ah, bl, ac[1]);
    ac[2] = mfma16x16x32(al, bh, ac[2]);
  }
  return ac[0] + (ac[1] + ac[2]);
}

// LDS of dn_chunk_prep_kernel (dynamic, so the compiler's register budget
// follows the VGPR occupancy target rather than the LDS-bound one): k^ and
// q^ rows of the chunk, then G and beta.  Once the products are formed the
// q^ rows' space holds the 64 x 64 triangular matrix A.
constexpr uint32_t kPrepLds = (2 * 64 * kCStride + 9 * 64) * 4;
constexpr int kPrepThreads = 512;  // 8 waves
__global__ __launch_bounds__(kPrepThreads, 2) void dn_chunk_prep_kernel(DnArgs a) {
  extern __shared__ __attribute__((aligned(16))) float prep_lds[];
  float* ks_s = prep_lds;
  float* qs_s = prep_lds + 64 * kCStride;
  float* g_s = prep_lds + 2 * 64 * kCStride;
  float* beta_s = g_s + 64;
  float* dk_s = g_s + 128;  // e^{G_63 - G_i}
  float* bg_s = g_s + 192;  // beta_i e^{G_i}
  float* gm_s = g_s + 256;  // e^{G_i}
  float* sc_s = g_s + 320;  // RMS scales of the chunk's q rows (0..63) and k rows (64..127)
  double* gd_s = (double*)(g_s + 448);  // G in fp64: pairwise differences without cancellation
  float* a_s = qs_s;  // [64][kAStride], once the q^ rows are consumed
  const uint32_t VH = a.value_heads;
  const uint32_t h = blockIdx.x % VH, c = blockIdx.x / VH;
  const uint32_t kh = h / (VH / a.key_heads);
  const uint32_t key_el = a.key_heads * kCD;
  const uint32_t t0 = c * kDnChunk;
  const uint32_t nt = min(kDnChunk, a.M - t0);
  const uint32_t tid = threadIdx.x, lane = tid & 63;
  const uint32_t wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const uint32_t j = lane & 15, grp = lane >> 4;
  float* ws = a.chunk_ws + ((size_t)c * VH + h) * kDnChunkFloats;
  float* Wg = ws + kDnWsW;
  float* Ug = ws + kDnWsU;
  float* Pg = ws + kDnWsP;
  float* Gg = ws + kDnWsG;
  float* KTg = ws + kDnWsKT;
  float* Qg = ws + kDnWsQ;

  // The chunk's conv (kernel 4): threads tid and tid + 256 own key channel
  // tid % 256 of key head kh (q 0..127, k 128..255), the first half of the
  // 64 tokens and the second, and write silu(conv) into the q / k rows in LDS
  // (zero past the last token).  The sums are conv_finish's, operation for
  // operation; the SiLU is silu_fast.
  const uint32_t kc = tid % 256, th0 = 32 * (tid / 256);
  const uint32_t kch = kc < kCD ? kh * kCD + kc : key_el + kh * kCD + (kc - kCD);
  // Every conv input of the thread is loaded before any is used, so the
  // workgroup pays one memory round trip for its inputs: the v values of the
  // wave's U~ columns (16 w + j) for the solve at the end (tokens
  // 16 b + 4 grp + r need the inputs from three tokens earlier on; rows past
  // the last token are masked at use), then the key channel's 32 tokens.
  float vw[4], vx[4][7];
  {
    const uint32_t vch = 2 * key_el + h * kCD + 16 * wave + j;
#pragma unroll
    for (int q = 0; q < 4; ++q) vw[q] = a.conv_w[(size_t)vch * 4 + q];
#pragma unroll
    for (int b = 0; b < 4; ++b)
#pragma unroll
      for (int q = 0; q < 7; ++q)
        vx[b][q] = conv_input(a, vch, min((int)(t0 + 16 * b + 4 * grp) - 3 + q, (int)a.M - 1));
  }
  {
    float w[4], win[3], xk[32];
#pragma unroll
    for (int q = 0; q < 4; ++q) w[q] = a.conv_w[(size_t)kch * 4 + q];
#pragma unroll
    for (int q = 0; q < 3; ++q) win[q] = conv_input(a, kch, min((int)(t0 + th0) - 3 + q, (int)a.M - 1));
#pragma unroll
    for (int k = 0; k < 32; ++k) xk[k] = a.qkv[(size_t)min(t0 + th0 + k, a.M - 1) * a.channels + kch];
    float* dst = kc < kCD ? qs_s + kc : ks_s + (kc - kCD);
#pragma unroll
    for (int k = 0; k < 32; ++k) {
      const float x = xk[k];
      float sum = __fmul_rn(w[3], x);
      sum = fmaf(w[0], win[0], sum);
      sum = fmaf(w[1], win[1], sum);
      sum = fmaf(w[2], win[2], sum);
      win[0] = win[1];
      win[1] = win[2];
      win[2] = x;
      const uint32_t t = th0 + k;
      dst[t * kCStride] = t < nt ? silu_fast(sum) : 0.0f;
    }
  }
  float vpre[4][4];
#pragma unroll
  for (int b = 0; b < 4; ++b)
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      float sum = __fmul_rn(vw[3], vx[b][r + 3]);
      sum = fmaf(vw[0], vx[b][r], sum);
      sum = fmaf(vw[1], vx[b][r + 1], sum);
      sum = fmaf(vw[2], vx[b][r + 2], sum);
      vpre[b][r] = silu_fast(sum);
    }
  // The state's conv history after the last token: raw inputs of the final
  // three tokens (from the old history when M < 3), written by the last
  // chunk's workgroups (key channels by the first value head of each key head).
  if (c + 1 == (a.M + kDnChunk - 1) / kDnChunk) {
    if (tid < 256 && h % (VH / a.key_heads) == 0)
#pragma unroll
      for (int q = 0; q < 3; ++q) a.hist_out[(size_t)kch * 3 + q] = conv_input(a, kch, (int)a.M - 3 + q);
    if (tid >= 256 && tid < 256 + kCD) {
      const uint32_t vch = 2 * key_el + h * kCD + (tid - 256);
#pragma unroll
      for (int q = 0; q < 3; ++q) a.hist_out[(size_t)vch * 3 + q] = conv_input(a, vch, (int)a.M - 3 + q);
    }
  }
  // Log decays, their running sum and beta (wave 0; padding tokens: lg = 0,
  // beta = 0, so they change nothing).
  if (wave == 0) {
    float lg = 0.0f, beta = 0.0f;
    if (lane < nt) {
      const size_t ti = (size_t)(t0 + lane) * VH + h;
      lg = -expf(a.a_log[h]) * softplus_f(a.a[ti] + a.dt_bias[h]);
      beta = sigmoid_f(a.b[ti]);
    }
    // The running sum in fp64: a decay e^{G_t - G_i} taken from two long fp32
    // sums would lose the low bits of G_t - G_i to cancellation.
    double Gd = lg;
#pragma unroll
    for (int off = 1; off < 64; off <<= 1) {
      const double o = __shfl_up(Gd, off);
      if (lane >= (uint32_t)off) Gd += o;
    }
    const float G = (float)Gd;
    gd_s[lane] = Gd;
    g_s[lane] = G;
    beta_s[lane] = beta;
    dk_s[lane] = expf((float)(__shfl(Gd, 63) - Gd));
    bg_s[lane] = beta * expf(G);
    gm_s[lane] = expf(G);
    Gg[lane] = G;
    Gg[kDnWsGM - kDnWsG + lane] = gm_s[lane];
    Gg[kDnWsDK - kDnWsG + lane] = dk_s[lane];
  }
  __syncthreads();
  // prep_key_head's RMS scales: row ri (q rows 0..63, k rows 64..127), lane l
  // sums the squares of columns l and l + 64, then a wave sum.  The wave's 16
  // rows are reduced side by side, and lane q forms row q's scale.
  {
    float ss[16];
#pragma unroll
    for (int q = 0; q < 16; ++q) {
      const uint32_t ri = 16 * wave + q;
      const float* row = (ri < 64 ? qs_s + ri * kCStride : ks_s + (ri - 64) * kCStride) + lane;
      ss[q] = fmaf(row[64], row[64], fmaf(row[0], row[0], 0.0f));
    }
#pragma unroll
    for (int q = 0; q < 16; ++q) ss[q] = wave_sum(ss[q]);
    float mine = ss[0];
#pragma unroll
    for (int q = 1; q < 16; ++q) mine = lane == (uint32_t)q ? ss[q] : mine;
    if (lane < 16) sc_s[16 * wave + lane] = 1.0f / sqrtf(mine / (float)kCD + a.eps);
  }
  __syncthreads();
  {
    const float inv = 1.0f / sqrtf((float)kCD);
#pragma unroll
    for (int p = 0; p < 8; ++p) {
      const uint32_t idx = tid + kPrepThreads * p;  // float4 index over [128 rows][32]
      const uint32_t ri = idx / 32, c4 = idx % 32;
      float* px = (ri < 64 ? qs_s + ri * kCStride : ks_s + (ri - 64) * kCStride) + 4 * c4;
      const float sc = sc_s[ri];
      f32x4 v = *(const f32x4*)px;
#pragma unroll
      for (int e = 0; e < 4; ++e) v[e] = ri < 64 ? v[e] * sc * inv * inv : v[e] * sc * inv;
      *(f32x4*)px = v;
    }
  }
  __syncthreads();

  // The scan's B operands of the key head (first value head of each key
  // head only): dn_chunk_store_qk.
  if (h % (VH / a.key_heads) == 0) {
#pragma unroll
    for (int p = 0; p < 2; ++p) dn_chunk_store_k(ks_s, (uint16_t*)KTg, tid + kPrepThreads * p);
#pragma unroll
    for (int p = 0; p < 2; ++p) dn_chunk_store_q(qs_s, (uint16_t*)Qg, tid + kPrepThreads * p);
  }

  // Q K^T, then K K^T, on the lower-triangular 16 x 16 tiles (tn <= tm):
  // 10 tiles each over the 8 waves.  Q K^T goes straight to P; once every
  // wave is past it the q^ rows' space takes A from K K^T (dn_gram_tile).
  auto tile = [&](const float* xs, int tix, floatx4& acc, int& tm, int& tn) __attribute__((always_inline)) {
    int rem = tix;
    tm = 0;
    while (rem > tm) rem -= ++tm;
    tn = rem;
    acc = dn_gram_tile(xs, ks_s, tm, tn, j, grp);
  };
  for (int tix = (int)wave; tix < 10; tix += 8) {
    floatx4 acc;
    int tm, tn;
    tile(qs_s, tix, acc, tm, tn);
    // acc[r]: row t = 16 tm + 4 grp + r, column i = 16 tn + j.
    const uint32_t i = 16 * tn + j;
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      const uint32_t t = 16 * tm + 4 * grp + r;
      Pg[dn_ws_index(tm, tn, 4 * grp + r, j, 4)] = i <= t ? expf((float)(gd_s[t] - gd_s[i])) * acc[r] : 0.0f;
    }
  }
  __syncthreads();  // the q^ rows are consumed; their space becomes A
  for (int tix = 9 - (int)wave; tix >= 0; tix -= 8) {
    floatx4 acc;
    int tm, tn;
    tile(ks_s, tix, acc, tm, tn);
    const uint32_t i = 16 * tn + j;
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      const uint32_t t = 16 * tm + 4 * grp + r;
      a_s[t * kAStride + i] = i < t ? -(beta_s[t] * expf((float)(gd_s[t] - gd_s[i])) * acc[r]) : 0.0f;  // -A
    }
  }
  // P is zero above the diagonal blocks too, so its readers need no bounds.
  for (uint32_t idx = tid; idx < 6 * 256; idx += kPrepThreads) {
    const uint32_t tile = idx / 256, e = idx % 256;
    const uint32_t tm = tile < 3 ? 0 : tile < 5 ? 1 : 2;  // (0,1) (0,2) (0,3) (1,2) (1,3) (2,3)
    const uint32_t tn = tile < 3 ? tile + 1 : tile < 5 ? tile - 1 : 3;
    Pg[256 * (4 * tm + tn) + e] = 0.0f;
  }
  __syncthreads();

  // Solve (I + A) X = R in 16-row blocks b (A unit lower triangular):
  //   X_b = T_b (R_b - sum_{c<b} A_bc X_c),  T_b = (I + A_bb)^{-1},
  // on fp32 MFMA.  R's columns are beta Gamma k (giving W) and beta v (giving
  // U~); wave w owns W columns 16 w .. 16 w + 15 (tile n = 0) and the same
  // U~ columns (tile n = 1).
  // With the reduction index of MFMA step r permuted to k = 4 grp + r, an
  // output tile (rows 4 grp + r, column j in lane (j, grp)) is directly the
  // B operand of the next product, so X stays in registers.
  // T_b first: wave b < 4, lane jj < 16 owns column jj (T_b[t][jj] =
  // delta_t,jj + sum_{i<t} (-A)[t][i] T_b[i][jj]).
  float* t_s = a_s + 64 * kAStride;  // T_b [4][16][17]
  if (wave < 4 && lane < 16) {
    const uint32_t b = wave, jj = lane;
    const float* ab = a_s + 16 * b * kAStride + 16 * b;
    float tc[16];
#pragma unroll
    for (int t = 0; t < 16; ++t) {
      float v = (uint32_t)t == jj ? 1.0f : 0.0f;
#pragma unroll
      for (int i = 0; i < t; ++i) v = fmaf(ab[t * kAStride + i], tc[i], v);
      tc[t] = v;
      t_s[(16 * b + t) * 17 + jj] = v;
    }
  }
  __syncthreads();
  const uint32_t cw = 16 * wave + j;  // the lane's column within W and within U~
  floatx4 X[4][2];  // [block b][tile n]: X[16 b + 4 grp + r][tile column]
#pragma unroll
  for (int b = 0; b < 4; ++b) {
    floatx4 acc[2];
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      const uint32_t t = 16 * b + 4 * grp + r;
      acc[0][r] = bg_s[t] * ks_s[t * kCStride + cw];
      acc[1][r] = t < nt ? beta_s[t] * vpre[b][r] : 0.0f;
    }
#pragma unroll
    for (int cb = 0; cb < b; ++cb) {
      const f32x4 av = *(const f32x4*)(a_s + (16 * b + j) * kAStride + 16 * cb + 4 * grp);  // (-A)_bc
#pragma unroll
      for (int r = 0; r < 4; ++r)
#pragma unroll
        for (int n = 0; n < 2; ++n) acc[n] = mfma_f32_4(av[r], X[cb][n][r], acc[n]);
    }
    const f32x4 tv = *(const f32x4*)(t_s + (16 * b + j) * 17 + 4 * grp);
#pragma unroll
    for (int n = 0; n < 2; ++n) {
      X[b][n] = floatx4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
      for (int r = 0; r < 4; ++r) X[b][n] = mfma_f32_4(tv[r], acc[n][r], X[b][n]);
    }
  }
  // X[b][n][r] is token 16 b + 4 grp + r, column 16 wave + j: four tokens of
  // one column per lane, while the workspace order wants consecutive columns
  // of one token.  Each wave transposes its tiles through its own LDS rows
  // (W tiles, then U~ tiles).
  __syncthreads();  // every wave is past k^, A and T: their LDS is free
  float* xt = prep_lds + wave * (4 * 16 * 20);  // 4 tiles of 16 x 16, row stride 20
#pragma unroll
  for (int n = 0; n < 2; ++n) {
#pragma unroll
    for (int b = 0; b < 4; ++b)
#pragma unroll
      for (int r = 0; r < 4; ++r) xt[b * 320 + (4 * grp + r) * 20 + j] = X[b][n][r];
    __builtin_amdgcn_wave_barrier();
    if (n == 0) {
      // W[token][k] as split bf16, block (token block b, step s = wave / 2):
      // the step's lanes with grp in {2 (wave % 2), 2 (wave % 2) + 1} hold
      // columns 16 (wave % 2) + 8 (grp % 2) + e, i.e. this wave's tile.
      uint16_t* w3 = (uint16_t*)Wg;
      if (grp / 2 == wave % 2) {
#pragma unroll
        for (int b = 0; b < 4; ++b) {
          const float* src = xt + b * 320 + j * 20 + 8 * (grp % 2);
          u32x4 hi, lo;
          split_bf16x8(*(const f32x4*)src, *(const f32x4*)(src + 4), hi, lo);
          *(u32x4*)(w3 + dn_b3_block(b, wave / 2, 4) + 8 * lane) = hi;
          *(u32x4*)(w3 + dn_b3_block(b, wave / 2, 4) + 512 + 8 * lane) = lo;
        }
      }
    } else {
      // U~: row group wave, token block b (fp32, dn_ws_index order).
#pragma unroll
      for (int b = 0; b < 4; ++b) {
        const f32x4 v = *(const f32x4*)(xt + b * 320 + (lane % 16) * 20 + 4 * (lane / 16));
        *(f32x4*)(Ug + 256 * (4 * wave + b) + 4 * lane) = v;
      }
    }
    __builtin_amdgcn_wave_barrier();
  }
}

// Per-head LDS pieces of the two-head preparation: one head's decays (G,
// beta, e^{G_63 - G}, beta e^G, e^G, then G in fp64) and its T blocks.
constexpr uint32_t kPairG = 448;
constexpr uint32_t kPairT = 4 * 16 * 17;

// dn_chunk_prep_kernel's work for the two value heads of one key head
// (value_heads == 2 key_heads) in one 8-wave workgroup, two per CU.  The q^ /
// k^ conv, their RMS scales and the raw products Q K^T and K K^T depend only
// on the key head, so they are formed once and written out for both heads
// with each head's decays; waves 4 r .. 4 r + 3 then take value head
// 2 kh + r through its decays, v conv, solve and stores with the one-head
// kernel's arithmetic (same bits), each owning two of that kernel's
// 16-column slices (16 v and 16 (v + 4) for its v = wave % 4).  Both heads'
// -A overlay the q^ rows once Q K^T is formed (row stride 66 instead of 68 so
// that the two fit), which keeps the LDS at 80 KB.
constexpr uint32_t kP8AStride = 66;
constexpr uint32_t kP8A = 64 * kP8AStride;
constexpr uint32_t kP8Lds = (2 * 64 * kCStride + 2 * kPairT + 2 * kPairG + 128) * 4;
constexpr int kP8Threads = 512;
static_assert(2 * kP8A <= 64 * kCStride, "both heads' -A fit the q^ rows");
static_assert(2 * kP8Lds <= 160 * 1024, "two workgroups per CU");
static_assert(8 * 4 * 16 * 20 <= 2 * 64 * kCStride, "transpose rows fit the k^ and q^ rows");
__global__ __launch_bounds__(kP8Threads, 4) void dn_chunk_prep_pair_kernel(DnArgs a) {
  extern __shared__ __attribute__((aligned(16))) float prep_lds[];
  float* ks_s = prep_lds;
  float* qs_s = prep_lds + 64 * kCStride;
  float* t_base = prep_lds + 2 * 64 * kCStride;  // [2][4][16][17]
  float* g_base = t_base + 2 * kPairT;           // [2][kPairG]
  float* sc_s = g_base + 2 * kPairG;             // RMS scales: q rows 0..63, k rows 64..127
  const uint32_t VH = a.value_heads;
  const uint32_t KH = a.key_heads;
  const uint32_t kh = blockIdx.x % KH, c = blockIdx.x / KH;
  const uint32_t key_el = KH * kCD;
  const uint32_t t0 = c * kDnChunk;
  const uint32_t nt = min(kDnChunk, a.M - t0);
  const uint32_t tid = threadIdx.x, lane = tid & 63;
  const uint32_t wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const uint32_t r = wave / 4, hw = wave % 4, htid = tid % 256;
  const uint32_t h = 2 * kh + r;
  const uint32_t j = lane & 15, grp = lane >> 4;
  float* a_s = qs_s + r * kP8A;  // once Q K^T is formed
  float* t_s = t_base + r * kPairT;
  auto gsets = [&](uint32_t rr) { return g_base + rr * kPairG; };
  float* g_s = gsets(r);
  float* beta_s = g_s + 64;
  float* dk_s = g_s + 128;  // e^{G_63 - G_i}
  float* bg_s = g_s + 192;  // beta_i e^{G_i}
  float* gm_s = g_s + 256;  // e^{G_i}
  double* gd_s = (double*)(g_s + 320);  // G in fp64
  float* ws = a.chunk_ws + ((size_t)c * VH + h) * kDnChunkFloats;
  float* Wg = ws + kDnWsW;
  float* Ug = ws + kDnWsU;
  float* Pg = ws + kDnWsP;
  float* Gg = ws + kDnWsG;

  // Conv: thread t owns key channel t % 256 and tokens 32 (t / 256) .. + 31,
  // and the v columns of its two slices; every input is loaded first.
  const uint32_t kc = tid % 256, th0 = 32 * (tid / 256);
  const uint32_t kch = kc < kCD ? kh * kCD + kc : key_el + kh * kCD + (kc - kCD);
  float vw[2][4], vx[2][4][7];
#pragma unroll
  for (int sl = 0; sl < 2; ++sl) {
    const uint32_t vch = 2 * key_el + h * kCD + 16 * (hw + 4 * sl) + j;
#pragma unroll
    for (int q = 0; q < 4; ++q) vw[sl][q] = a.conv_w[(size_t)vch * 4 + q];
#pragma unroll
    for (int b = 0; b < 4; ++b)
#pragma unroll
      for (int q = 0; q < 7; ++q)
        vx[sl][b][q] = conv_input(a, vch, min((int)(t0 + 16 * b + 4 * grp) - 3 + q, (int)a.M - 1));
  }
  {
    float w[4], win[3], xk[32];
#pragma unroll
    for (int q = 0; q < 4; ++q) w[q] = a.conv_w[(size_t)kch * 4 + q];
#pragma unroll
    for (int q = 0; q < 3; ++q) win[q] = conv_input(a, kch, min((int)(t0 + th0) - 3 + q, (int)a.M - 1));
#pragma unroll
    for (int k = 0; k < 32; ++k) xk[k] = a.qkv[(size_t)min(t0 + th0 + k, a.M - 1) * a.channels + kch];
    float* dst = kc < kCD ? qs_s + kc : ks_s + (kc - kCD);
#pragma unroll
    for (int k = 0; k < 32; ++k) {
      const float x = xk[k];
      float sum = __fmul_rn(w[3], x);
      sum = fmaf(w[0], win[0], sum);
      sum = fmaf(w[1], win[1], sum);
      sum = fmaf(w[2], win[2], sum);
      win[0] = win[1];
      win[1] = win[2];
      win[2] = x;
      const uint32_t t = th0 + k;
      dst[t * kCStride] = t < nt ? silu_fast(sum) : 0.0f;
    }
  }
  float vpre[2][4][4];
#pragma unroll
  for (int sl = 0; sl < 2; ++sl)
#pragma unroll
    for (int b = 0; b < 4; ++b)
#pragma unroll
      for (int rr = 0; rr < 4; ++rr) {
        float sum = __fmul_rn(vw[sl][3], vx[sl][b][rr + 3]);
        sum = fmaf(vw[sl][0], vx[sl][b][rr], sum);
        sum = fmaf(vw[sl][1], vx[sl][b][rr + 1], sum);
        sum = fmaf(vw[sl][2], vx[sl][b][rr + 2], sum);
        vpre[sl][b][rr] = silu_fast(sum);
      }
  if (c + 1 == (a.M + kDnChunk - 1) / kDnChunk) {
    if (tid < 256)
#pragma unroll
      for (int q = 0; q < 3; ++q) a.hist_out[(size_t)kch * 3 + q] = conv_input(a, kch, (int)a.M - 3 + q);
    if (htid < kCD) {
      const uint32_t vch = 2 * key_el + h * kCD + htid;
#pragma unroll
      for (int q = 0; q < 3; ++q) a.hist_out[(size_t)vch * 3 + q] = conv_input(a, vch, (int)a.M - 3 + q);
    }
  }
  if (hw == 0) {
    float lg = 0.0f, beta = 0.0f;
    if (lane < nt) {
      const size_t ti = (size_t)(t0 + lane) * VH + h;
      lg = -expf(a.a_log[h]) * softplus_f(a.a[ti] + a.dt_bias[h]);
      beta = sigmoid_f(a.b[ti]);
    }
    double Gd = lg;
#pragma unroll
    for (int off = 1; off < 64; off <<= 1) {
      const double o = __shfl_up(Gd, off);
      if (lane >= (uint32_t)off) Gd += o;
    }
    const float G = (float)Gd;
    gd_s[lane] = Gd;
    g_s[lane] = G;
    beta_s[lane] = beta;
    dk_s[lane] = expf((float)(__shfl(Gd, 63) - Gd));
    bg_s[lane] = beta * expf(G);
    gm_s[lane] = expf(G);
    Gg[lane] = G;
    Gg[kDnWsGM - kDnWsG + lane] = gm_s[lane];
    Gg[kDnWsDK - kDnWsG + lane] = dk_s[lane];
  }
  __syncthreads();
  {
    float ss[16];
#pragma unroll
    for (int q = 0; q < 16; ++q) {
      const uint32_t ri = 16 * wave + q;
      const float* row = (ri < 64 ? qs_s + ri * kCStride : ks_s + (ri - 64) * kCStride) + lane;
      ss[q] = fmaf(row[64], row[64], fmaf(row[0], row[0], 0.0f));
    }
#pragma unroll
    for (int q = 0; q < 16; ++q) ss[q] = wave_sum(ss[q]);
    float mine = ss[0];
#pragma unroll
    for (int q = 1; q < 16; ++q) mine = lane == (uint32_t)q ? ss[q] : mine;
    if (lane < 16) sc_s[16 * wave + lane] = 1.0f / sqrtf(mine / (float)kCD + a.eps);
  }
  __syncthreads();
  {
    const float inv = 1.0f / sqrtf((float)kCD);
#pragma unroll
    for (int p = 0; p < 8; ++p) {
      const uint32_t idx = tid + kP8Threads * p;
      const uint32_t ri = idx / 32, c4 = idx % 32;
      float* px = (ri < 64 ? qs_s + ri * kCStride : ks_s + (ri - 64) * kCStride) + 4 * c4;
      const float sc = sc_s[ri];
      f32x4 v = *(const f32x4*)px;
#pragma unroll
      for (int e = 0; e < 4; ++e) v[e] = ri < 64 ? v[e] * sc * inv * inv : v[e] * sc * inv;
      *(f32x4*)px = v;
    }
  }
  __syncthreads();
  {
    float* ws0 = a.chunk_ws + ((size_t)c * VH + 2 * kh) * kDnChunkFloats;
#pragma unroll
    for (int p = 0; p < 4; ++p) {
      if (r == 0)
        dn_chunk_store_k(ks_s, (uint16_t*)(ws0 + kDnWsKT), htid + 256 * p);
      else
        dn_chunk_store_q(qs_s, (uint16_t*)(ws0 + kDnWsQ), htid + 256 * p);
    }
  }
  auto tile = [&](const float* xs, int tix, floatx4& acc, int& tm, int& tn) __attribute__((always_inline)) {
    int rem = tix;
    tm = 0;
    while (rem > tm) rem -= ++tm;
    tn = rem;
    acc = dn_gram_tile(xs, ks_s, tm, tn, j, grp);
  };
  // Q K^T (P for both heads), then, once every wave is past the q^ rows,
  // K K^T (-A for both heads in their space).
  for (int tix = (int)wave; tix < 10; tix += 8) {
    floatx4 acc;
    int tm, tn;
    tile(qs_s, tix, acc, tm, tn);
    const uint32_t i = 16 * tn + j;
#pragma unroll
    for (int hr = 0; hr < 2; ++hr) {
      const double* gdh = (const double*)(gsets(hr) + 320);
      float* P = a.chunk_ws + ((size_t)c * VH + 2 * kh + hr) * kDnChunkFloats + kDnWsP;
#pragma unroll
      for (int rr = 0; rr < 4; ++rr) {
        const uint32_t t = 16 * tm + 4 * grp + rr;
        P[dn_ws_index(tm, tn, 4 * grp + rr, j, 4)] = i <= t ? expf((float)(gdh[t] - gdh[i])) * acc[rr] : 0.0f;
      }
    }
  }
  __syncthreads();
  for (int tix = 9 - (int)wave; tix >= 0; tix -= 8) {
    floatx4 acc;
    int tm, tn;
    tile(ks_s, tix, acc, tm, tn);
    const uint32_t i = 16 * tn + j;
#pragma unroll
    for (int hr = 0; hr < 2; ++hr) {
      const float* gh = gsets(hr);
      const double* gdh = (const double*)(gh + 320);
      float* A = qs_s + hr * kP8A;
#pragma unroll
      for (int rr = 0; rr < 4; ++rr) {
        const uint32_t t = 16 * tm + 4 * grp + rr;
        A[t * kP8AStride + i] = i < t ? -(gh[64 + t] * expf((float)(gdh[t] - gdh[i])) * acc[rr]) : 0.0f;  // -A
      }
    }
  }
  for (uint32_t idx = htid; idx < 6 * 256; idx += 256) {
    const uint32_t tl = idx / 256, e = idx % 256;
    const uint32_t tm = tl < 3 ? 0 : tl < 5 ? 1 : 2;  // (0,1) (0,2) (0,3) (1,2) (1,3) (2,3)
    const uint32_t tn = tl < 3 ? tl + 1 : tl < 5 ? tl - 1 : 3;
    Pg[256 * (4 * tm + tn) + e] = 0.0f;
  }
  __syncthreads();
  if (lane < 16) {
    const uint32_t b = hw, jj = lane;
    const float* ab = a_s + 16 * b * kP8AStride + 16 * b;
    float tc[16];
#pragma unroll
    for (int t = 0; t < 16; ++t) {
      float v = (uint32_t)t == jj ? 1.0f : 0.0f;
#pragma unroll
      for (int i = 0; i < t; ++i) v = fmaf(ab[t * kP8AStride + i], tc[i], v);
      tc[t] = v;
      t_s[(16 * b + t) * 17 + jj] = v;
    }
  }
  __syncthreads();
  floatx4 X[2][4][2];  // [slice][block b][tile n]
#pragma unroll
  for (int sl = 0; sl < 2; ++sl) {
    const uint32_t cw = 16 * (hw + 4 * sl) + j;
#pragma unroll
    for (int b = 0; b < 4; ++b) {
      floatx4 acc[2];
#pragma unroll
      for (int rr = 0; rr < 4; ++rr) {
        const uint32_t t = 16 * b + 4 * grp + rr;
        acc[0][rr] = bg_s[t] * ks_s[t * kCStride + cw];
        acc[1][rr] = t < nt ? beta_s[t] * vpre[sl][b][rr] : 0.0f;
      }
#pragma unroll
      for (int cb = 0; cb < b; ++cb) {
        const f32x4 av = *(const f32x4*)(a_s + (16 * b + j) * kP8AStride + 16 * cb + 4 * grp);  // (-A)_bc
#pragma unroll
        for (int rr = 0; rr < 4; ++rr)
#pragma unroll
          for (int n = 0; n < 2; ++n) acc[n] = mfma_f32_4(av[rr], X[sl][cb][n][rr], acc[n]);
      }
      const f32x4 tv = *(const f32x4*)(t_s + (16 * b + j) * 17 + 4 * grp);
#pragma unroll
      for (int n = 0; n < 2; ++n) {
        X[sl][b][n] = floatx4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
        for (int rr = 0; rr < 4; ++rr) X[sl][b][n] = mfma_f32_4(tv[rr], acc[n][rr], X[sl][b][n]);
      }
    }
  }
  __syncthreads();  // every wave is past k^, A and T: their LDS is free
  float* xt = prep_lds + wave * (4 * 16 * 20);
#pragma unroll
  for (int sl = 0; sl < 2; ++sl) {
    const uint32_t vwv = hw + 4 * sl;  // the one-head kernel's wave index of this slice
#pragma unroll
    for (int n = 0; n < 2; ++n) {
#pragma unroll
      for (int b = 0; b < 4; ++b)
#pragma unroll
        for (int rr = 0; rr < 4; ++rr) xt[b * 320 + (4 * grp + rr) * 20 + j] = X[sl][b][n][rr];
      __builtin_amdgcn_wave_barrier();
      if (n == 0) {
        uint16_t* w3 = (uint16_t*)Wg;
        if (grp / 2 == vwv % 2) {
#pragma unroll
          for (int b = 0; b < 4; ++b) {
            const float* src = xt + b * 320 + j * 20 + 8 * (grp % 2);
            u32x4 hi, lo;
            split_bf16x8(*(const f32x4*)src, *(const f32x4*)(src + 4), hi, lo);
            *(u32x4*)(w3 + dn_b3_block(b, vwv / 2, 4) + 8 * lane) = hi;
            *(u32x4*)(w3 + dn_b3_block(b, vwv / 2, 4) + 512 + 8 * lane) = lo;
          }
        }
      } else {
#pragma unroll
        for (int b = 0; b < 4; ++b) {
          const f32x4 v = *(const f32x4*)(xt + b * 320 + (lane % 16) * 20 + 4 * (lane / 16));
          *(f32x4*)(Ug + 256 * (4 * vwv + b) + 4 * lane) = v;
        }
      }
      __builtin_amdgcn_wave_barrier();
    }
  }
}

// grid: VH * 8 blocks (block = rg * VH + h: the 8 row groups of a head share
// blockIdx mod 8, i.e. one XCD and its L2, where they read the same chunk
// operands), 512 threads.  The group's 16 rows of S live in LDS.  Waves w and
// w + 4 share tokens 16 w .. 16 w + 15 and split the reduction over k of
//   U_w^T = U~_w^T - S W_w^T,   O_w^T = (S Q_w^T) diag(Gamma_w)   (k halves)
// (partials meet in LDS; q^ and k^ are the key head's, the decays this
// head's); then, after U^T and U^T diag(e^{G_C - G_i}) are exchanged, wave v
// of 8 updates columns 16 v .. 16 v + 15 of S as
// Gamma_C S + U^T diag(e^{G_C - G_i}) K over the chunk's 64 tokens, and
// waves 0..3 add the intra-chunk term sum_{i <= t} U^T P and store O.  Waves w and w + 4 run on one SIMD, so one's memory and LDS waits
// overlap the other's MFMAs.  The products with S and with U^T are split-bf16
// triples on the bf16 MFMA; P U^T is fp32.  The next chunk's operands are
// loaded while the current chunk is computed.
constexpr int kScanThreads = 512;
__global__ __launch_bounds__(kScanThreads) void dn_chunk_scan_kernel(DnArgs a) {
  __shared__ __attribute__((aligned(16))) float u_s[16 * kAStride];   // U^T [row][token]
  __shared__ __attribute__((aligned(16))) float ud_s[16 * kAStride];  // U^T [row][i] e^{G_63 - G_i}
  __shared__ __attribute__((aligned(16))) float s_s[16 * kCStride];   // S [row][col]
  __shared__ __attribute__((aligned(16))) float xp_s[4][64][8];      // the upper k half's partials
  const uint32_t VH = a.value_heads;
  const uint32_t h = blockIdx.x % VH, rg = blockIdx.x / VH;
  const uint32_t row0 = rg * 16;
  const uint32_t tid = threadIdx.x, lane = tid & 63;
  const uint32_t wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const uint32_t tw = wave % 4, khalf = wave / 4;  // token block, k half
  const uint32_t j = lane & 15, grp = lane >> 4;
  const uint32_t nchunks = (a.M + kDnChunk - 1) / kDnChunk;
  const uint32_t tok = 16 * tw + j;   // this lane's token column in U and O
  const uint32_t col_w = 16 * wave;   // first of the wave's S columns

  u32x4 Wh[2], Wl[2], Qh[2], Ql[2], Kh[2], Kl[2];  // split bf16 B operands (the wave's k half / columns)
  f32x4 Uv, Pv[4];
  float G_last, gm_tok, dk_tok;
  auto ws_of = [&](uint32_t c) { return a.chunk_ws + ((size_t)c * VH + h) * kDnChunkFloats; };
  // k^ and q^ of the key head live with its first value head.
  const uint32_t h_key = h - h % (VH / a.key_heads);
  auto qk_of = [&](uint32_t c) { return a.chunk_ws + ((size_t)c * VH + h_key) * kDnChunkFloats; };
  const uint32_t lofs = 4 * (16 * grp + j);  // the lane's float4 within a 64-float4 block
  // Rows past the last token read valid data and are weighted by zero.
  auto load_wqu = [&](uint32_t c) __attribute__((always_inline)) {
    const float* ws = ws_of(c);
    G_last = ws[kDnWsG + 63];
    gm_tok = ws[kDnWsGM + tok];
    dk_tok = ws[kDnWsDK + tok];
    const uint16_t* w3 = (const uint16_t*)(ws + kDnWsW);
    const uint16_t* q3 = (const uint16_t*)(qk_of(c) + kDnWsQ);
#pragma unroll
    for (int s = 0; s < 2; ++s) {
      const uint32_t o = dn_b3_block(tw, 2 * khalf + s, 4) + 8 * lane;
      Wh[s] = *(const u32x4*)(w3 + o);
      Wl[s] = *(const u32x4*)(w3 + o + 512);
      Qh[s] = *(const u32x4*)(q3 + o);
      Ql[s] = *(const u32x4*)(q3 + o + 512);
    }
    if (khalf == 0) Uv = *(const f32x4*)(ws + kDnWsU + 1024 * rg + 256 * tw + lofs);
  };
  // P[tok][i] (fp32, i = 16 m + 4 grp + e; waves 0..3) and K~^T[col][i]
  // (split bf16, the wave's 16 columns).
  auto load_pk = [&](uint32_t c) __attribute__((always_inline)) {
    const float* ws = ws_of(c);
    const uint16_t* kt3 = (const uint16_t*)(qk_of(c) + kDnWsKT);
    if (khalf == 0) {
#pragma unroll
      for (int m = 0; m < 4; ++m) Pv[m] = *(const f32x4*)(ws + kDnWsP + 256 * (4 * tw + m) + lofs);
    }
#pragma unroll
    for (int s = 0; s < 2; ++s) {
      const uint32_t o = dn_b3_block(wave, s, 2) + 8 * lane;
      Kh[s] = *(const u32x4*)(kt3 + o);
      Kl[s] = *(const u32x4*)(kt3 + o + 512);
    }
  };

  // Initial rows of S into LDS.
  {
    const float* sin = a.s_in + ((size_t)h * kCD + row0) * kCD;
    const uint32_t r = tid / 32, c4 = tid % 32;  // float4 index over [16][32]
    *(f32x4*)(s_s + r * kCStride + 4 * c4) = *(const f32x4*)(sin + r * kCD + 4 * c4);
  }
  load_wqu(0);
  load_pk(0);
  __syncthreads();

  floatx4 d;  // the wave's 16 columns of S in the MFMA output layout (rows 4 grp + r, column col_w + j)
  for (uint32_t c = 0; c < nchunks; ++c) {
    const uint32_t t0 = c * kDnChunk, nt = min(kDnChunk, a.M - t0);
    const uint32_t cn = min(c + 1, nchunks - 1);  // the last chunk reloads itself (unused)
    // (a) U^T[row][tok] = U~[tok][row] - sum_k S[row][k] W[tok][k]
    // (b1) O^T[row][tok] = Gamma_tok sum_k S[row][k] q[tok][k]
    // over this wave's k half: S (A operand, row j, k = 32 s + 8 grp + e) is
    // split here, W and q come split.
    floatx4 au[3] = {{0.f, 0.f, 0.f, 0.f}, {0.f, 0.f, 0.f, 0.f}, {0.f, 0.f, 0.f, 0.f}};
    floatx4 ao[3] = {{0.f, 0.f, 0.f, 0.f}, {0.f, 0.f, 0.f, 0.f}, {0.f, 0.f, 0.f, 0.f}};
#pragma unroll
    for (int s = 0; s < 2; ++s) {
      const float* sp = s_s + j * kCStride + 32 * (2 * khalf + s) + 8 * grp;
      u32x4 sh, sl;
      split_bf16x8(*(const f32x4*)sp, *(const f32x4*)(sp + 4), sh, sl);
      au[0] = mfma16x16x32(sh, Wh[s], au[0]);
      ao[0] = mfma16x16x32(sh, Qh[s], ao[0]);
      au[1] = mfma16x16x32(sh, Wl[s], au[1]);
      ao[1] = mfma16x16x32(sh, Ql[s], ao[1]);
      au[2] = mfma16x16x32(sl, Wh[s], au[2]);
      ao[2] = mfma16x16x32(sl, Qh[s], ao[2]);
    }
    const float gam_c = expf(G_last);
    floatx4 acc_u = au[0] + (au[1] + au[2]);
    floatx4 acc_o = ao[0] + (ao[1] + ao[2]);
    // The S columns this wave updates, in the output layout, before any
    // wave writes the new values (after the second barrier below).
#pragma unroll
    for (int r = 0; r < 4; ++r) d[r] = gam_c * s_s[(4 * grp + r) * kCStride + col_w + j];
    if (khalf == 1) {
      *(f32x4*)&xp_s[tw][lane][0] = acc_u;
      *(f32x4*)&xp_s[tw][lane][4] = acc_o;
    }
    lds_barrier();  // the upper halves' partials are in LDS
    if (khalf == 0) {
      acc_u += *(const f32x4*)&xp_s[tw][lane][0];
      acc_o += *(const f32x4*)&xp_s[tw][lane][4];
      acc_o *= gm_tok;
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        const float u = Uv[r] - acc_u[r];
        u_s[(4 * grp + r) * kAStride + tok] = u;
        ud_s[(4 * grp + r) * kAStride + tok] = dk_tok * u;
      }
    }
    load_wqu(cn);  // W, q and U~ of this chunk are consumed
    lds_barrier();  // U^T complete; every wave is done reading S and the partials
    // S[:, cols_w] += U^T diag(e^{G_63 - G_i}) K[:, cols_w] over the chunk's 64 tokens.
    floatx4 dx[2] = {{0.f, 0.f, 0.f, 0.f}, {0.f, 0.f, 0.f, 0.f}};
#pragma unroll
    for (int s = 0; s < 2; ++s) {
      const float* up = ud_s + j * kAStride + 32 * s + 8 * grp;
      u32x4 uh, ul;
      split_bf16x8(*(const f32x4*)up, *(const f32x4*)(up + 4), uh, ul);
      d = mfma16x16x32(uh, Kh[s], d);
      dx[0] = mfma16x16x32(uh, Kl[s], dx[0]);
      dx[1] = mfma16x16x32(ul, Kh[s], dx[1]);
    }
    d += dx[0] + dx[1];
    if (khalf == 0) {
      // (b2) O^T[row][tok] += sum_{i <= tok} U^T[row][i] P[tok][i] (all four
      // token blocks: P is zero past the diagonal block, so no branch).
      floatx4 ap[2] = {acc_o, {0.f, 0.f, 0.f, 0.f}};
#pragma unroll
      for (int m = 0; m < 4; ++m) {
        const f32x4 ua = *(const f32x4*)(u_s + j * kAStride + 16 * m + 4 * grp);
#pragma unroll
        for (int e = 0; e < 4; ++e) ap[e & 1] = mfma_f32_4(ua[e], Pv[m][e], ap[e & 1]);
      }
      acc_o = ap[0] + ap[1];
      // A buffer store bounded to the chunk's nt rows: tokens past the end
      // are dropped by the hardware, so the store needs no branch.
      const uint32_t row_bytes = VH * kCD * 4;
      const __amdgpu_buffer_rsrc_t ro = __builtin_amdgcn_make_buffer_rsrc(
          a.out + (size_t)t0 * VH * kCD, (short)0, (int)(nt * row_bytes), 0x00020000);
      __builtin_amdgcn_raw_buffer_store_b128(
          u32x4{__float_as_uint(acc_o[0]), __float_as_uint(acc_o[1]), __float_as_uint(acc_o[2]),
                __float_as_uint(acc_o[3])},
          ro, tok * row_bytes + (h * kCD + row0 + 4 * grp) * 4, 0, 0);
    }
    load_pk(cn);
#pragma unroll
    for (int r = 0; r < 4; ++r) s_s[(4 * grp + r) * kCStride + col_w + j] = d[r];
    lds_barrier();  // the new S is complete; U^T is consumed
  }
  float* sout = a.s_out + ((size_t)h * kCD + row0) * kCD;
#pragma unroll
  for (int r = 0; r < 4; ++r) sout[(4 * grp + r) * kCD + col_w + j] = d[r];
}

template <int EPT>
void launch_scan(const DnArgs& a, hipStream_t st) {
  const uint32_t groups = (a.dv + kRowsPerWg - 1) / kRowsPerWg;
  hipLaunchKernelGGL(dn_scan_kernel<EPT>, dim3(a.value_heads * groups), dim3(kThreads), 0, st, a);
}

}  // namespace

// One token with head dims <= 128: one 1024-thread workgroup per value head
// (QM38_DN_STEP_HEAD=0 forces the split kernel instead).
bool dn_step_head(const DnArgs& a) {
  if (a.M != 1 || a.dk > 128 || a.dv > 128) return false;
  return a.tune_step_head != 0;
}

bool dn_step_split(const DnArgs& a) { return a.M == 1 && a.dk <= 128 && a.dv <= 256 && !dn_step_head(a); }

bool dn_use_chunked(const DnArgs& a) {
  if (a.dk != kCD || a.dv != kCD || a.kernel != 4 || a.snap_rows > 0 || a.M <= 1 ||
      a.value_heads % a.key_heads != 0)
    return false;
  if (a.tune_chunked >= 0) return a.tune_chunked != 0;
  return a.M >= 2 * kDnChunk;
}

template <int NS>
void launch_conv_tiled_ns(const DnArgs& a, dim3 grid, dim3 block, hipStream_t st) {
  switch (a.kernel) {
    case 1: hipLaunchKernelGGL((dn_conv_tiled_kernel<NS, 0>), grid, block, 0, st, a); break;
    case 2: hipLaunchKernelGGL((dn_conv_tiled_kernel<NS, 1>), grid, block, 0, st, a); break;
    case 3: hipLaunchKernelGGL((dn_conv_tiled_kernel<NS, 2>), grid, block, 0, st, a); break;
    default: hipLaunchKernelGGL((dn_conv_tiled_kernel<NS, 3>), grid, block, 0, st, a); break;
  }
}
void launch_conv_tiled(const DnArgs& a, uint32_t ns, dim3 grid, dim3 block, hipStream_t st) {
  if (ns <= 1)
    launch_conv_tiled_ns<1>(a, grid, block, st);
  else if (ns <= 2)
    launch_conv_tiled_ns<2>(a, grid, block, st);
  else
    launch_conv_tiled_ns<4>(a, grid, block, st);
}

hipError_t launch_deltanet(const DnArgs& a, hipStream_t st) {
  if (a.dk == 0 || a.dk > 256 || a.dv == 0 || a.dv > 256 || a.M == 0) return hipErrorInvalidValue;
  // One token with S rows that fit the fused kernel's registers: one launch.
  if (dn_step_head(a)) {
    if (a.dk <= 64)
      hipLaunchKernelGGL(dn_step_head_kernel<4>, dim3(a.value_heads), dim3(kHeadThreads), 0, st, a);
    else
      hipLaunchKernelGGL(dn_step_head_kernel<8>, dim3(a.value_heads), dim3(kHeadThreads), 0, st, a);
    return hipGetLastError();
  }
  if (dn_step_split(a)) {
    if (!a.step_o || !a.step_ctr) return hipErrorInvalidValue;
    const dim3 grid(a.value_heads * ((a.dv + kStepRows - 1) / kStepRows)), block(kStepThreads);
    if (a.dk <= 64)
      hipLaunchKernelGGL(dn_step_split_kernel<4>, grid, block, 0, st, a);
    else
      hipLaunchKernelGGL(dn_step_split_kernel<8>, grid, block, 0, st, a);
    return hipGetLastError();
  }
  const uint32_t units = a.key_heads + a.value_heads;
  const bool chunked = dn_use_chunked(a);
  if (chunked) {
    // The chunk prep kernel convolves its own inputs.
  } else if (a.kernel <= kTaps) {
    const uint32_t items = ((a.M + kConvTile - 1) / kConvTile) * units;
    const dim3 grid((items + 3) / 4), block(kThreads);
    const uint32_t ns = (std::max(a.dk, a.dv) + 63) / 64;
    launch_conv_tiled(a, ns, grid, block, st);
  } else {
    const uint32_t prep_items = a.M * units;
    hipLaunchKernelGGL(dn_conv_prepare_kernel, dim3((prep_items + 3) / 4), dim3(kThreads), 0, st, a);
  }
  if (chunked) {
    if (!a.chunk_ws) return hipErrorInvalidValue;
    const uint32_t nchunks = (a.M + kDnChunk - 1) / kDnChunk;
    if (a.value_heads == 2 * a.key_heads && a.tune_dn_pair != 0)
      hipLaunchKernelGGL(dn_chunk_prep_pair_kernel, dim3(nchunks * a.key_heads), dim3(kP8Threads), kP8Lds, st, a);
    else
      hipLaunchKernelGGL(dn_chunk_prep_kernel, dim3(nchunks * a.value_heads), dim3(kPrepThreads), kPrepLds, st, a);
    hipLaunchKernelGGL(dn_chunk_scan_kernel, dim3(a.value_heads * (kCD / 16)), dim3(kScanThreads), 0, st, a);
  } else {
    const uint32_t ept = (a.dk + kLanesPerRow - 1) / kLanesPerRow;
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
  }
  const uint32_t lpr = a.dv <= 128 ? 32 : 64, per_wave = kNormSlots * (64 / lpr);
  const uint32_t norm_waves = (a.M * a.value_heads + per_wave - 1) / per_wave;
  const uint32_t wpb = norm_waves >= 1024 ? kThreads / 64 : 1;
  const dim3 ngrid((norm_waves + wpb - 1) / wpb), nblock(64 * wpb);
  const bool vec = a.dv % 4 == 0;
  if (lpr == 32 && vec)
    hipLaunchKernelGGL((dn_gate_norm_kernel<32, true>), ngrid, nblock, 0, st, a);
  else if (lpr == 32)
    hipLaunchKernelGGL((dn_gate_norm_kernel<32, false>), ngrid, nblock, 0, st, a);
  else if (vec)
    hipLaunchKernelGGL((dn_gate_norm_kernel<64, true>), ngrid, nblock, 0, st, a);
  else
    hipLaunchKernelGGL((dn_gate_norm_kernel<64, false>), ngrid, nblock, 0, st, a);
  return hipGetLastError();
}

}  // namespace qm
