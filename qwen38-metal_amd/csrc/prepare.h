// Launch interface of the full-attention q/k preparation kernel
// (attn_prepare.hip).
#pragma once
#include <hip/hip_runtime.h>
#include <stdint.h>

namespace qm {

constexpr uint32_t kPrepMaxHeadDim = 256;

struct PrepArgs {
  const uint16_t* q_with_gate;  // bf16 [M][H][2 hd]: query | gate per head
  const uint16_t* k_in;         // bf16 [M][KVH][hd]
  const float* q_norm;          // [hd]
  const float* k_norm;          // [hd]
  const uint32_t* positions;    // [3][M] axis-major, or null: every axis = base + row
  uint16_t* q_out;              // bf16 [M][H][hd]
  uint16_t* gate_out;           // bf16 [M][H][hd]
  float* k_out;                 // fp32 [M][KVH][hd]
  uint32_t M, H, KVH, head_dim, rotary_dim;
  uint32_t row0;  // first row of this launch (the launcher splits M into grid-sized chunks)
  uint32_t base, section1, section2, has_sections;
  float theta, eps;
  // theta^(-2 i / rotary_dim) in fp64 for i < rotary_dim / 2, filled by
  // launch_attn_prepare (the launch arguments carry them to every block).
  double inv_freq[kPrepMaxHeadDim / 2];
};

hipError_t launch_attn_prepare(const PrepArgs& a, hipStream_t st);

}  // namespace qm
