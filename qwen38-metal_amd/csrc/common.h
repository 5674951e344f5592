// Device-side helpers shared by every qm38 kernel (gfx950 / CDNA4 only).
#pragma once
#include <hip/hip_runtime.h>
#include <stdint.h>

namespace qm {

typedef __attribute__((__vector_size__(8 * sizeof(__bf16)))) __bf16 bf16x8;
typedef short short4_t __attribute__((ext_vector_type(4)));
typedef float floatx4 __attribute__((ext_vector_type(4)));
typedef float floatx16 __attribute__((ext_vector_type(16)));
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
typedef uint32_t u32x2 __attribute__((ext_vector_type(2)));

// bf16 <-> f32 exactly as the reference (qwen38.metal:18-26): widening is a
// shift, narrowing is round-to-nearest-even via +0x7fff+lsb (NaN is not
// special-cased).
__device__ __forceinline__ float bf16_to_f32(uint32_t bits16) {
  return __uint_as_float(bits16 << 16);
}
__device__ __forceinline__ uint16_t f32_to_bf16(float v) {
  const uint32_t bits = __float_as_uint(v);
  return (uint16_t)((bits + 0x7fffu + ((bits >> 16) & 1u)) >> 16);
}

// sigmoid / silu / softplus with the reference's formulas
// (qwen38.metal:4090-4096, 4364-4372).
__device__ __forceinline__ float sigmoid_f(float v) { return 1.0f / (1.0f + expf(-v)); }
__device__ __forceinline__ float silu_f(float v) { return v * sigmoid_f(v); }
__device__ __forceinline__ float softplus_f(float v) {
  if (v > 20.0f) return v;
  if (v < -20.0f) return expf(v);
  return logf(1.0f + expf(v));
}

// v_perm_b32: result byte i = byte sel_i of the 8-byte value {hi:lo}.
__device__ __forceinline__ uint32_t perm_b32(uint32_t hi, uint32_t lo, uint32_t sel) {
  return __builtin_amdgcn_perm(hi, lo, sel);
}

// Eight consecutive bf16 values x0..x7 held as four u32 pairs (x0,x1)(x2,x3)
// (x4,x5)(x6,x7) are reordered into (x0,x4)(x1,x5)(x2,x6)(x3,x7): the element
// order produced by q4_word_to_bf16x8 below.
__device__ __forceinline__ u32x4 interleave_bf16x8(u32x4 a) {
  u32x4 r;
  r.x = perm_b32(a.z, a.x, 0x05040100u);
  r.y = perm_b32(a.z, a.x, 0x07060302u);
  r.z = perm_b32(a.w, a.y, 0x05040100u);
  r.w = perm_b32(a.w, a.y, 0x07060302u);
  return r;
}

// One packed MLX Q4 word -> eight bf16 values (128 + q) in the order
// (q0,q4)(q1,q5)(q2,q6)(q3,q7).  0x4300|q is the bf16 encoding of 128+q for
// q in 0..15, so the conversion is exact and costs one AND-OR per pair.
__device__ __forceinline__ u32x4 q4_word_to_bf16x8(uint32_t w) {
  u32x4 r;
  r.x = (w & 0x000F000Fu) | 0x43004300u;
  r.y = ((w >> 4) & 0x000F000Fu) | 0x43004300u;
  r.z = ((w >> 8) & 0x000F000Fu) | 0x43004300u;
  r.w = ((w >> 12) & 0x000F000Fu) | 0x43004300u;
  return r;
}

__device__ __forceinline__ bf16x8 as_bf16x8(u32x4 v) { return __builtin_bit_cast(bf16x8, v); }

// D(16x16) += A(16x32) * B(32x16), bf16 in, fp32 accumulate.  Lane l holds
// A row (l & 15) / B column (l & 15) and the 8 K-elements 8*(l>>4)..+7; the
// result holds column (l & 15), rows 4*(l>>4)+0..3.
__device__ __forceinline__ floatx4 mfma16x16x32(u32x4 a, u32x4 b, floatx4 c) {
  return __builtin_amdgcn_mfma_f32_16x16x32_bf16(as_bf16x8(a), as_bf16x8(b), c, 0, 0, 0);
}
// D(16x16) += A(16x16) * B(16x16): lane holds 4 K-elements 4*(l>>4)..+3.
__device__ __forceinline__ floatx4 mfma16x16x16(u32x2 a, u32x2 b, floatx4 c) {
  return __builtin_amdgcn_mfma_f32_16x16x16bf16_1k(__builtin_bit_cast(short4_t, a),
                                                    __builtin_bit_cast(short4_t, b), c, 0, 0, 0);
}
// D(32x32) += A(32x16) * B(16x32): lane holds A row / B column (l & 31) and
// K-elements 8*(l>>5)..+7; result: column (l & 31), rows
// 8*(i>>2) + 4*(l>>5) + (i&3) for i = 0..15.
__device__ __forceinline__ floatx16 mfma32x32x16(u32x4 a, u32x4 b, floatx16 c) {
  return __builtin_amdgcn_mfma_f32_32x32x16_bf16(as_bf16x8(a), as_bf16x8(b), c, 0, 0, 0);
}

// Sum over the 64 lanes: DPP within 16-lane rows (quad swaps, row rotations
// by 4 and 8), then v_permlane16_swap / v_permlane32_swap across rows.
__device__ __forceinline__ float wave_allsum(float v) {
  v += __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), 0xB1, 0xF, 0xF, false));   // quad [1,0,3,2]
  v += __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), 0x4E, 0xF, 0xF, false));   // quad [2,3,0,1]
  v += __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), 0x124, 0xF, 0xF, false));  // row_ror:4
  v += __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), 0x128, 0xF, 0xF, false));  // row_ror:8
  const auto p = __builtin_amdgcn_permlane16_swap(__float_as_uint(v), __float_as_uint(v), false, false);
  v = __uint_as_float(p[0]) + __uint_as_float(p[1]);
  const auto q = __builtin_amdgcn_permlane32_swap(__float_as_uint(v), __float_as_uint(v), false, false);
  return __uint_as_float(q[0]) + __uint_as_float(q[1]);
}

// Maximum over the 64 lanes with the same DPP / permlane steps (exact in any
// order, so it equals a shuffle tree's result).
__device__ __forceinline__ float wave_allmax(float v) {
  v = fmaxf(v, __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), 0xB1, 0xF, 0xF, false)));
  v = fmaxf(v, __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), 0x4E, 0xF, 0xF, false)));
  v = fmaxf(v, __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), 0x124, 0xF, 0xF, false)));
  v = fmaxf(v, __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), 0x128, 0xF, 0xF, false)));
  const auto p = __builtin_amdgcn_permlane16_swap(__float_as_uint(v), __float_as_uint(v), false, false);
  v = fmaxf(__uint_as_float(p[0]), __uint_as_float(p[1]));
  const auto q = __builtin_amdgcn_permlane32_swap(__float_as_uint(v), __float_as_uint(v), false, false);
  return fmaxf(__uint_as_float(q[0]), __uint_as_float(q[1]));
}

// Workgroup barrier that orders LDS only: waits for the wave's own LDS
// operations (lgkmcnt) but leaves its global loads and stores in flight,
// unlike __syncthreads(), whose workgroup fence also drains vmcnt.  Use it
// where only LDS data passes between the waves.
__device__ __forceinline__ void lds_barrier() {
  __builtin_amdgcn_fence(__ATOMIC_RELEASE, "workgroup", "local");
  __builtin_amdgcn_s_barrier();
  __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "workgroup", "local");
}

}  // namespace qm
