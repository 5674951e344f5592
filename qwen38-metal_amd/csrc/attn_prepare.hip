// Full-attention q/k preparation, the step between the Q4 projections and the
// Q8 KV append / attention:
//   * query heads: the packed projection holds [query | gate] per head
//     (split_query_and_gate, native.rs:4917-4942); the query half is
//     RMS-normalised with q_norm, rotated, and written as bf16, the gate half
//     copied through;
//   * key heads: RMS-normalised with k_norm and rotated, written as fp32 (the
//     input of the Q8 append).
// RMSNorm: x * rsqrt(mean x^2 + eps) * w (rms_norm_slice, native.rs:5153-5161).
// RoPE on the first rotary_dim elements in half-split pairs (i, i + rd/2) with
// angle pos(axis) / theta^(2i/rd), the axis chosen per frequency by the
// interleaved M-RoPE rule (MropePosition::axis_for_frequency, native.rs:
// 136-148; apply_mrope, native.rs:5163-5180; GPU twins
// qwen38_gqa_prepare_query(_rows) / _key(_rows), qwen38.metal:4761-5029).
// The angle is formed in fp64 and reduced modulo 2 pi in fp64 before an fp32
// sine and cosine: the reference's fp32 angle moves by ~1e-2 rad per ulp of
// powf at positions near 128K.
//
// Block = (row, head group).  Its threads first build the row's rotation
// table (one angle, sine and cosine per frequency, shared by all heads) in
// LDS; then each of the 8 waves prepares every (8 * groups)-th head of the
// row, issuing the loads of up to 8 heads at once.  Short calls (decode) use
// many head groups, long prompts one per row.  A wave holds two heads when
// head_dim <= 128 (32 lanes each), else one; lane l of a head holds elements
// 4 l .. 4 l + 3: the sum of squares is a reduction over the head's lanes and
// each rotation partner (element c +- rd/2) is fetched from its lane by a
// cross-lane shuffle.
#include "common.h"
#include "prepare.h"

#include <algorithm>
#include <cmath>

namespace qm {
namespace {

constexpr int kPrepWaves = 8;  // waves per block (one block per row)
constexpr int kPrepBatch = 8;  // heads whose loads a wave issues together

__device__ __forceinline__ float pick4(const float (&x)[4], uint32_t k) {
  return k == 0 ? x[0] : k == 1 ? x[1] : k == 2 ? x[2] : x[3];
}

// Rotation partner of this lane's element j (c = 4 lane + j): element c + half
// for c < half, c - half above.  For a given j every lower receiver wants
// element (j + half) % 4 of its source lane and every upper receiver element
// (j - half) % 4, so each lane sends those two and each receiver keeps one.
// hl: the lane's index within its head's lanes, which start at lane `base`.
__device__ __forceinline__ float partner(const float (&x)[4], uint32_t hl, uint32_t base, uint32_t j,
                                         uint32_t half) {
  const uint32_t c = 4 * hl + j;
  const bool lower = c < half;
  const float up_val = __shfl(pick4(x, (j + half) & 3u), (int)(base + (((c + half) >> 2) & 63)) & 63);
  const float dn_val = __shfl(pick4(x, (j - half) & 3u), (int)(base + (((c - half) >> 2) & 63)) & 63);
  return lower ? up_val : dn_val;
}

// Sum over each 32-lane half of the wave (wave_allsum without its last step).
__device__ __forceinline__ float half_allsum(float v) {
  v += __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), 0xB1, 0xF, 0xF, false));   // quad [1,0,3,2]
  v += __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), 0x4E, 0xF, 0xF, false));   // quad [2,3,0,1]
  v += __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), 0x124, 0xF, 0xF, false));  // row_ror:4
  v += __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), 0x128, 0xF, 0xF, false));  // row_ror:8
  const auto p = __builtin_amdgcn_permlane16_swap(__float_as_uint(v), __float_as_uint(v), false, false);
  return __uint_as_float(p[0]) + __uint_as_float(p[1]);
}

// HPW heads per wave: 2 when head_dim <= 128 (32 lanes per head), else 1.
// For head_dim <= 128 the one-head form's upper 32 lanes add only zeros, so
// both forms give the same sums bit for bit.
template <int HPW>
__global__ __launch_bounds__(64 * kPrepWaves) void attn_prepare_kernel(PrepArgs a) {
  constexpr uint32_t kLanesPerHead = 64 / HPW;
  __shared__ float cos_s[kPrepMaxHeadDim / 2], sin_s[kPrepMaxHeadDim / 2];
  const uint32_t wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
  const uint32_t row = a.row0 + blockIdx.x;
  // Heads of this block: blockIdx.y * waves + wave + k * waves * gridDim.y.
  const uint32_t hstride = kPrepWaves * gridDim.y;
  const uint32_t hd = a.head_dim, rd = a.rotary_dim, half = rd / 2;

  // Rotation table of this row: frequency i turns by pos(axis(i)) / theta^(2i/rd).
  for (uint32_t i = threadIdx.x; i < half; i += blockDim.x) {
    uint32_t axis = 0;
    if (a.has_sections) {
      if (i % 3 == 1 && i / 3 < a.section1) axis = 1;
      if (i % 3 == 2 && i / 3 < a.section2) axis = 2;
    }
    const uint32_t p = a.positions ? a.positions[(size_t)axis * a.M + row] : a.base + row;
    // fp64 angle, reduced to [-pi, pi] with a two-part 2 pi (error ~1e-11 rad
    // at 1e5 rad), then single-precision sine and cosine of the small argument.
    const double angle = (double)p * a.inv_freq[i];
    const double turns = rint(angle * 0.15915494309189535);
    double r = fma(-turns, 6.283185307179586, angle);
    r = fma(-turns, 2.4492935982947064e-16, r);
    float sn, cs;
    sincosf((float)r, &sn, &cs);
    cos_s[i] = cs;
    sin_s[i] = sn;
  }
  __syncthreads();

  const uint32_t units = a.H + a.KVH;  // query heads, then key heads
  const uint32_t slots = (units + HPW - 1) / HPW;  // wave work items of HPW heads
  const bool vec = hd % 4 == 0;
  const uint32_t hl = lane % kLanesPerHead, hsel = lane / kLanesPerHead, base = hsel * kLanesPerHead;
  const uint32_t c0 = 4 * hl;
  const bool mine = c0 < hd;
  // This lane's norm weights, read once (not inside each head's chain).
  float wq[4], wk[4];
#pragma unroll
  for (int j = 0; j < 4; ++j) {
    wq[j] = c0 + j < hd ? a.q_norm[c0 + j] : 0.0f;
    wk[j] = c0 + j < hd ? a.k_norm[c0 + j] : 0.0f;
  }
  for (uint32_t first = blockIdx.y * kPrepWaves + wave; first < slots; first += hstride * kPrepBatch) {
    // Issue the loads of up to kPrepBatch slots (and the query heads' gates).
    uint2 in[kPrepBatch], gt[kPrepBatch];
#pragma unroll
    for (int b = 0; b < kPrepBatch; ++b) {
      const uint32_t u = (first + hstride * b) * HPW + hsel;
      in[b] = uint2{0u, 0u};
      gt[b] = uint2{0u, 0u};
      if (u < units && mine) {
        const bool is_q = u < a.H;
        const uint16_t* src = is_q ? a.q_with_gate + ((size_t)row * a.H + u) * 2 * hd
                                   : a.k_in + ((size_t)row * a.KVH + (u - a.H)) * hd;
        if (vec) {
          in[b] = *(const uint2*)(src + c0);
          if (is_q) gt[b] = *(const uint2*)(src + hd + c0);
        } else {
#pragma unroll
          for (int j = 0; j < 4; ++j)
            if (c0 + j < hd) {
              const uint32_t sh = 16 * (j % 2);
              if (j < 2) {
                in[b].x |= (uint32_t)src[c0 + j] << sh;
                if (is_q) gt[b].x |= (uint32_t)src[hd + c0 + j] << sh;
              } else {
                in[b].y |= (uint32_t)src[c0 + j] << sh;
                if (is_q) gt[b].y |= (uint32_t)src[hd + c0 + j] << sh;
              }
            }
        }
      }
    }
#pragma unroll
    for (int b = 0; b < kPrepBatch; ++b) {
      const uint32_t slot = first + hstride * b;
      if (slot >= slots) break;  // wave-uniform
      const uint32_t u = slot * HPW + hsel;
      const bool live = u < units;  // the second head of the last slot may not exist
      const bool is_q = u < a.H;
      const uint32_t bits[2] = {in[b].x, in[b].y};
      float x[4];
      float ss = 0.0f;
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        x[j] = bf16_to_f32((bits[j / 2] >> (16 * (j % 2))) & 0xFFFFu);
        ss += x[j] * x[j];
      }
      ss = HPW == 2 ? half_allsum(ss) : wave_allsum(ss);
      const float scale = 1.0f / sqrtf(ss / (float)hd + a.eps);
#pragma unroll
      for (int j = 0; j < 4; ++j) x[j] = mine && c0 + j < hd ? x[j] * scale * (is_q ? wq[j] : wk[j]) : 0.0f;
      float y[4];
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        const uint32_t c = c0 + j;
        const float other = partner(x, hl, base, (uint32_t)j, half);  // every lane joins the shuffles
        y[j] = x[j];
        if (c < rd) {
          const uint32_t f = c < half ? c : c - half;
          y[j] = c < half ? x[j] * cos_s[f] - other * sin_s[f] : x[j] * cos_s[f] + other * sin_s[f];
        }
      }
      if (!mine || !live) continue;
      if (is_q) {
        const size_t o = ((size_t)row * a.H + u) * hd + c0;
        if (vec) {
          *(uint2*)(a.q_out + o) = uint2{f32_to_bf16(y[0]) | ((uint32_t)f32_to_bf16(y[1]) << 16),
                                         f32_to_bf16(y[2]) | ((uint32_t)f32_to_bf16(y[3]) << 16)};
          *(uint2*)(a.gate_out + o) = gt[b];
        } else {
          const uint32_t gb[2] = {gt[b].x, gt[b].y};
#pragma unroll
          for (int j = 0; j < 4; ++j)
            if (c0 + j < hd) {
              a.q_out[o + j] = f32_to_bf16(y[j]);
              a.gate_out[o + j] = (uint16_t)(gb[j / 2] >> (16 * (j % 2)));
            }
        }
      } else {
        float* ko = a.k_out + ((size_t)row * a.KVH + (u - a.H)) * hd + c0;
        if (vec) {
          *(float4*)ko = float4{y[0], y[1], y[2], y[3]};
        } else {
#pragma unroll
          for (int j = 0; j < 4; ++j)
            if (c0 + j < hd) ko[j] = y[j];
        }
      }
    }
  }
}

}  // namespace

hipError_t launch_attn_prepare(const PrepArgs& a, hipStream_t st) {
  constexpr uint32_t kMaxGridY = 65535;  // rows per launch (kept below the y limit for symmetry)
  PrepArgs f = a;
  for (uint32_t i = 0; i < a.rotary_dim / 2 && i < kPrepMaxHeadDim / 2; ++i)
    f.inv_freq[i] = pow((double)a.theta, -(double)(2 * i) / (double)a.rotary_dim);
  for (uint32_t r0 = 0; r0 < a.M; r0 += kMaxGridY) {
    PrepArgs c = f;
    c.row0 = r0;
    // Head groups per row: enough blocks to cover the CUs a few times over
    // (one head per wave at M = 1; one block per row for long prompts).
    const uint32_t rows = std::min(kMaxGridY, a.M - r0);
    const uint32_t hpw = a.head_dim <= 64 * 4 / 2 ? 2 : 1;
    const uint32_t slots = (a.H + a.KVH + hpw - 1) / hpw;
    const uint32_t max_groups = (slots + kPrepWaves - 1) / kPrepWaves;
    const uint32_t groups = std::max(1u, std::min(max_groups, (1024u + rows - 1) / rows));
    const dim3 grid(rows, groups);
    if (hpw == 2)
      hipLaunchKernelGGL(attn_prepare_kernel<2>, grid, dim3(64 * kPrepWaves), 0, st, c);
    else
      hipLaunchKernelGGL(attn_prepare_kernel<1>, grid, dim3(64 * kPrepWaves), 0, st, c);
    const hipError_t e = hipGetLastError();
    if (e != hipSuccess) return e;
  }
  return hipSuccess;
}

}  // namespace qm
