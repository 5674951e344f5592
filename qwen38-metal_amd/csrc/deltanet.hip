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
  float sum = wl * xl;
#pragma unroll
  for (int j = 0; j < kTaps - 1; ++j)
    if (j < hw) sum += c.w[j] * c.x[j];
  return silu_f(sum);
}
// Longer kernels: the same sum, one tap at a time.
__device__ __forceinline__ float conv_silu_loop(const DnArgs& a, uint32_t ch, int t) {
  const int hw = (int)a.kernel - 1;
  const float* w = a.conv_w + (size_t)ch * a.kernel;
  float sum = w[hw] * conv_input(a, ch, t);
  for (int tap = 0; tap < hw; ++tap) sum += w[tap] * conv_input(a, ch, t - hw + tap);
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
// and the fused step so both round identically.
__device__ __forceinline__ void prep_key_head(const DnArgs& a, uint32_t t, uint32_t kh, uint32_t lane, float (&qo)[4],
                                              float (&ko)[4], float* hist_dst) {
  const uint32_t key_el = a.key_heads * a.dk;
  float qs = 0.0f, ks = 0.0f;
  if (a.kernel <= kTaps) {
    // All operands of the lane's (up to 8) outputs in flight at once.
    ConvIn cq[4], ck[4];
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const uint32_t c = min(lane + 64 * i, a.dk - 1);
      conv_load(a, kh * a.dk + c, (int)t, cq[i]);
      conv_load(a, key_el + kh * a.dk + c, (int)t, ck[i]);
    }
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const uint32_t c = lane + 64 * i;
      const bool ok = c < a.dk;
      qo[i] = ok ? conv_finish(a, cq[i]) : 0.0f;
      ko[i] = ok ? conv_finish(a, ck[i]) : 0.0f;
      if (ok && hist_dst) {
        conv_store_history(a, kh * a.dk + c, cq[i], hist_dst);
        conv_store_history(a, key_el + kh * a.dk + c, ck[i], hist_dst);
      }
    }
  } else {
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const uint32_t c = lane + 64 * i;
      const bool ok = c < a.dk;
      qo[i] = ok ? conv_silu_loop(a, kh * a.dk + c, (int)t) : 0.0f;
      ko[i] = ok ? conv_silu_loop(a, key_el + kh * a.dk + c, (int)t) : 0.0f;
      if (ok && hist_dst) {
        shift_history(a, kh * a.dk + c, (int)t, hist_dst);
        shift_history(a, key_el + kh * a.dk + c, (int)t, hist_dst);
      }
    }
  }
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    qs += qo[i] * qo[i];
    ks += ko[i] * ko[i];
  }
  qs = wave_sum(qs);
  ks = wave_sum(ks);
  const float inv = 1.0f / sqrtf((float)a.dk);
  const float qscale = 1.0f / sqrtf(qs / (float)a.dk + a.eps);
  const float kscale = 1.0f / sqrtf(ks / (float)a.dk + a.eps);
#pragma unroll
  for (int i = 0; i < 4; ++i) {
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
// 16 lanes of the row get it).  Shared by the scan and the fused step.
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

// Gated RMS norm of one (token, value head) output row by one wave: reads
// o_in[c], writes out[c] = o * rsqrt(mean o^2 + eps) * norm * silu(z).
// Shared by the prefill path and the fused step.
__device__ __forceinline__ void gate_norm_row(const DnArgs& a, const float* o_in, const float* z, float* out,
                                              uint32_t lane, uint16_t* out_bf16 = nullptr) {
  float v[4];  // dv <= 256
  float ss = 0.0f;
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const uint32_t c = lane + 64 * i;
    v[i] = c < a.dv ? o_in[c] : 0.0f;
    ss += v[i] * v[i];
  }
  ss = wave_sum(ss);
  const float scale = 1.0f / sqrtf(ss / (float)a.dv + a.eps);
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const uint32_t c = lane + 64 * i;
    if (c < a.dv) {
      const float r = v[i] * scale * a.norm[c] * silu_f(z[c]);
      out[c] = r;
      if (out_bf16) out_bf16[c] = f32_to_bf16(r);
    }
  }
}

// One wave per (token, value head), blocks of 1 or 4 waves; in place on `out`.
__global__ __launch_bounds__(kThreads) void dn_gate_norm_kernel(DnArgs a) {
  const uint32_t item = blockIdx.x * (blockDim.x >> 6) + (threadIdx.x >> 6);
  if (item >= a.M * a.value_heads) return;
  float* o = a.out + (size_t)item * a.dv;
  gate_norm_row(a, o, a.z + (size_t)item * a.dv, o, threadIdx.x & 63);
}

// The whole decode step (M = 1) in one launch: block = value head vh.
//  wave 0: q^, k^ of key head kh (prep_key_head); wave 1: conv of vh's v
//  channels; thread 128: g and beta.  Then the 16-lane row groups update the
//  dv rows of S in dv / 16 passes (delta_row_token), and wave 0 applies the
//  gated norm (gate_norm_row).  The arithmetic is the three-launch path's,
//  call for call, so a step equals a one-token prefill bit for bit.  (A
//  1024-thread block with 64 rows per pass compiled to code whose results
//  differ from the prefill path's in the last bit for some heads, so the
//  block stays at 256 threads.)
constexpr int kStepThreads = 256;
constexpr int kStepRows = kStepThreads / 16;  // S rows per pass
template <int EPT, int PASSES>
__global__ __launch_bounds__(kStepThreads) void dn_step_kernel(DnArgs a) {
  __shared__ __attribute__((aligned(16))) float qk_s[2][16][EPT];  // [q | k][lane][e]
  __shared__ float v_s[kStepRows * PASSES], o_s[kStepRows * PASSES];
  __shared__ float gb_s[2];
  const uint32_t vh = blockIdx.x;
  const uint32_t group = a.value_heads / a.key_heads;
  const uint32_t kh = vh / group;
  const uint32_t key_el = a.key_heads * a.dk;
  const uint32_t wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
  // The first value head of a key group also writes that key head's history.
  const bool key_hist = vh % group == 0 && a.kernel > 1;

  // S rows of this block: pass p, row kStepRows p + r, columns l + 16 e.
  const int r = threadIdx.x / 16, l = threadIdx.x % 16;
  float s[PASSES][EPT];
#pragma unroll
  for (int p = 0; p < PASSES; ++p) {
    const uint32_t row = kStepRows * p + r;
    const size_t srow = ((size_t)vh * a.dv + row) * a.dk;
#pragma unroll
    for (int e = 0; e < EPT; ++e) {
      const uint32_t j = l + 16 * e;
      s[p][e] = row < a.dv && j < a.dk ? a.s_in[srow + j] : 0.0f;
    }
  }

  if (wave == 0) {
    float cq[4], ck[4];
    prep_key_head(a, 0, kh, lane, cq, ck, key_hist ? a.hist_out : nullptr);
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const uint32_t c = lane + 64 * i;
      if (c < 16 * EPT) {
        qk_s[0][c % 16][c / 16] = c < a.dk ? cq[i] : 0.0f;
        qk_s[1][c % 16][c / 16] = c < a.dk ? ck[i] : 0.0f;
      }
    }
  } else if (wave == 1) {
    // Both of the lane's value channels loaded before either is finished.
    constexpr int kV = (kStepRows * PASSES + 63) / 64;
    if (a.kernel <= kTaps) {
      ConvIn cv[kV];
#pragma unroll
      for (int i = 0; i < kV; ++i) conv_load(a, 2 * key_el + vh * a.dv + min(lane + 64 * i, a.dv - 1), 0, cv[i]);
#pragma unroll
      for (int i = 0; i < kV; ++i) {
        const uint32_t c = lane + 64 * i;
        if (c < kStepRows * PASSES) v_s[c] = c < a.dv ? conv_finish(a, cv[i]) : 0.0f;
        if (c < a.dv && a.kernel > 1) conv_store_history(a, 2 * key_el + vh * a.dv + c, cv[i], a.hist_out);
      }
    } else {
      for (uint32_t c = lane; c < kStepRows * PASSES; c += 64) {
        const uint32_t ch = 2 * key_el + vh * a.dv + c;
        v_s[c] = c < a.dv ? conv_silu(a, ch, 0, a.kernel > 1 && c < a.dv ? a.hist_out : nullptr) : 0.0f;
      }
    }
  } else if (threadIdx.x == 128) {
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
    const uint32_t row = kStepRows * p + r;
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
    float* out = a.out + (size_t)vh * a.dv;
    gate_norm_row(a, o_s, a.z + (size_t)vh * a.dv, out, lane, a.out_bf16 ? a.out_bf16 + (size_t)vh * a.dv : nullptr);
  }
}

template <int EPT>
void launch_scan(const DnArgs& a, hipStream_t st) {
  const uint32_t groups = (a.dv + kRowsPerWg - 1) / kRowsPerWg;
  hipLaunchKernelGGL(dn_scan_kernel<EPT>, dim3(a.value_heads * groups), dim3(kThreads), 0, st, a);
}

}  // namespace

hipError_t launch_deltanet(const DnArgs& a, hipStream_t st) {
  if (a.dk == 0 || a.dk > 256 || a.dv == 0 || a.dv > 256 || a.M == 0) return hipErrorInvalidValue;
  // One token with S rows that fit the fused kernel's registers: one launch.
  if (a.M == 1 && a.dk <= 128 && a.dv <= 128) {
    const dim3 grid(a.value_heads), block(kStepThreads);
    const uint32_t ept = (a.dk + 15) / 16, passes = (a.dv + kStepRows - 1) / kStepRows;
    if (ept <= 4 && passes <= 4)
      hipLaunchKernelGGL((dn_step_kernel<4, 4>), grid, block, 0, st, a);
    else if (ept <= 4)
      hipLaunchKernelGGL((dn_step_kernel<4, 8>), grid, block, 0, st, a);
    else if (passes <= 4)
      hipLaunchKernelGGL((dn_step_kernel<8, 4>), grid, block, 0, st, a);
    else
      hipLaunchKernelGGL((dn_step_kernel<8, 8>), grid, block, 0, st, a);
    return hipGetLastError();
  }
  // Few items (decode): one wave per block so they spread over more CUs.
  const uint32_t prep_items = a.M * (a.key_heads + a.value_heads);
  const uint32_t wpb = prep_items >= 1024 ? kThreads / 64 : 1;
  hipLaunchKernelGGL(dn_conv_prepare_kernel, dim3((prep_items + wpb - 1) / wpb), dim3(64 * wpb), 0, st, a);
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
  const uint32_t norm_items = a.M * a.value_heads;
  hipLaunchKernelGGL(dn_gate_norm_kernel, dim3((norm_items + wpb - 1) / wpb), dim3(64 * wpb), 0, st, a);
  return hipGetLastError();
}

}  // namespace qm
