// Launch interface of the Gated DeltaNet kernels (deltanet.hip).
#pragma once
#include <hip/hip_runtime.h>
#include <stdint.h>

namespace qm {

struct DnArgs {
  // config
  uint32_t key_heads, value_heads, dk, dv, kernel, channels;
  uint32_t M;  // tokens in this call
  float eps;
  // weights
  const float* conv_w;   // [channels][kernel]
  const float* a_log;    // [VH]
  const float* dt_bias;  // [VH]
  const float* norm;     // [dv]
  // activations
  const float* qkv;  // [M][channels]
  const float* z;    // [M][VH][dv]
  const float* b;    // [M][VH]
  const float* a;    // [M][VH]
  // state
  const float* hist_in;  // [channels][kernel-1]
  float* hist_out;       // distinct from hist_in
  const float* s_in;     // [VH][dv][dk]
  float* s_out;          // may equal s_in
  // workspace / output
  float* conv_out;  // [M][channels]: q^, k^, v after conv + prepare
  float* chunk_ws;  // chunked prefill: per (chunk, value head) dn_chunk_floats() floats
  // Single-token step over 16-row groups of S: the rows' outputs o [VH][dv]
  // before the gated norm, and per-head arrival counters [VH] (zero between
  // launches; the last group of a head to arrive resets its counter).
  float* step_o;
  unsigned* step_ctr;
  float* out;       // [M][VH][dv]
  uint16_t* out_bf16;  // single-token step only: the output rounded to bf16 as well (or NULL)
  // optional state images after tokens 0 .. snap_rows - 1 (speculative
  // verification; snap_rows <= M - 1): history [row][channels][kernel-1] and
  // S [row][VH][dv][dk], strides in floats
  float* snap_hist;
  float* snap_s;
  uint32_t snap_rows;
  uint64_t snap_hist_stride, snap_s_stride;
  // kernel choice overrides (-1: default): the per-head step kernel, the
  // chunked prefill, the two-value-head chunk preparation
  int32_t tune_step_head, tune_chunked, tune_dn_pair;
};

// Chunked prefill (WY / UT form over chunks of kDnChunk tokens): used for
// long prefills without state images at head dims 128 / 128 (or when
// QM38_DN_CHUNKED forces it on or off).  Its workspace per (chunk, value
// head): W [64][128], U~ [64][128], P [64][64], G [64], Gamma = e^G [64],
// e^{G_63 - G} [64], the keys transposed, k^^T [128][64], and q^ [64][128].
// The keys and queries depend only on the key head: they are stored with the
// first value head of each key head only (the scan applies the decays).  The
// matrices are stored in the scan's MFMA operand
// order: element (r, c) of a matrix with row blocks R = r / 16 and column
// blocks C = c / 16 sits at dn_ws_index(R, C, r % 16, c % 16) of its 16 x 16
// block sequence, i.e. lane (j = r % 16, g = (c % 16) / 4) holds the float4
// of c % 4 = 0..3, and 64 lanes read one contiguous 1 KB block.  U~ is
// stored per row group of S ([rg][token block] blocks, rows of U~ = tokens).
constexpr uint32_t kDnChunk = 64;
constexpr size_t kDnWsW = 0, kDnWsU = 8192, kDnWsP = 16384, kDnWsG = 20480, kDnWsGM = 20544, kDnWsDK = 20608,
                 kDnWsKT = 20672, kDnWsQ = 28864;
constexpr size_t kDnChunkFloats = kDnWsQ + 8192;
// Element (row r, column c) of block (R, C) of a matrix with `cb` column
// blocks: block base 256 (R cb + C), float4 16 (c / 4) + r, element c % 4.
__host__ __device__ constexpr uint32_t dn_ws_index(uint32_t R, uint32_t C, uint32_t r, uint32_t c, uint32_t cb) {
  return 256 * (R * cb + C) + 4 * (16 * (c / 4) + r) + c % 4;
}
bool dn_use_chunked(const DnArgs& a);
inline size_t dn_chunk_ws_bytes(uint32_t M, uint32_t value_heads) {
  return (size_t)((M + kDnChunk - 1) / kDnChunk) * value_heads * kDnChunkFloats * sizeof(float);
}

// Whether a single-token step runs split over 16-row groups of S (then
// step_o and step_ctr must be set).
bool dn_step_split(const DnArgs& a);

hipError_t launch_deltanet(const DnArgs& a, hipStream_t st);

}  // namespace qm
