// Paged Q8-KV GQA attention for MI355X (gfx950).
//
// Cache layout (per sequence; physical page ids come from its page table):
//   K pages  int8 [page][kv_head][16 tokens][D]
//   V pages  int8 [page][kv_head][D][16 tokens]   (d-major: the PV operand)
//   scales   fp32 [page][kv_head][16]             (one array for K, one for V)
//
// Kernels
//  * q8_append_kernel: quantises new K/V rows exactly as qwen38_q8_kv_append
//    (/root/reference/shaders/qwen38.metal:5031-5140): s = max(absmax/127,
//    FLT_MIN), q = (int8) round(clamp(x / s, -127, 127)) with IEEE division
//    and round-half-away-from-zero, and writes page-table entries of pages
//    materialised by this append.
//  * q8_prefill_kernel (causal prefill) and q8_decode_kernel (decode):
//    flash attention over Q8 pages.  A wave owns one KV head and the GQA group
//    of <= 16 query heads sharing it (decode), or CB blocks of 16 (row, head)
//    columns (prefill).  Per 16-token page:
//      S^T = K Q^T on fp16 MFMA 16x16x32 (K bytes -> fp16 of 1024 + (k + 128)
//      exactly, one AND-OR per pair; 1152 * sum(q) is removed per column),
//      online softmax in fp32 (exp2 domain, lazy rescaling),
//      O^T += V^T P^T on bf16 MFMA 16x16x32 with V as exact signed bf16 and
//      P' = p * v_scale split into bf16 hi + lo (error ~2^-16), both halves
//      in the MFMA's K dimension.
//    The S^T/O^T orientation keeps every head in one lane column, so the
//    softmax statistics never move between lanes except for the 4-way max.
//    Decode splits the pages of a sequence over workgroups (combined in
//    LDS): one 8-wave workgroup per CU when all splits fit one such round,
//    else two 4-wave ones per CU.  With one workgroup the CU's waves share
//    one split, and the waves whose first loads queued behind the others'
//    no longer hold up a second workgroup's.  Split partials are merged by
//    q8_combine_kernel.
//  Head dimensions 1..256 run on pages of the next storage width Dp (64,
//  128 or 256) whose extra dimensions hold zero; queries, gates, outputs and
//  the appended K/V rows keep the caller's real head dimension.
#include <float.h>
#include <stdlib.h>

#include <mutex>

#include "attention.h"
#include "common.h"

namespace qm {
namespace {

constexpr float kLog2e = 1.4426950408889634f;

// A row's values 4 lane .. 4 lane + 3 (zero past dr): one 16-byte load when
// dr is a multiple of 4.
__device__ __forceinline__ void q8_load_row(const float* src, uint32_t dr, int lane, float (&vals)[4]) {
  if (dr % 4 == 0) {
    const floatx4 v = (uint32_t)lane * 4 < dr ? *(const floatx4*)(src + lane * 4) : floatx4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int i = 0; i < 4; ++i) vals[i] = v[i];
  } else {
#pragma unroll
    for (int i = 0; i < 4; ++i) vals[i] = (uint32_t)lane * 4 + i < dr ? src[lane * 4 + i] : 0.0f;
  }
}

// Quantises one row held 4 values per lane as qwen38_q8_kv_append does:
// s = max(absmax / 127, FLT_MIN), q = round-half-away(clamp(x / s, -127,
// 127)), IEEE division.  Returns s.
__device__ __forceinline__ float q8_quant_vals(const float (&vals)[4], int8_t (&qv)[4]) {
  float amax = 0.0f;
#pragma unroll
  for (int i = 0; i < 4; ++i) amax = fmaxf(amax, fabsf(vals[i]));
  amax = wave_allmax(amax);
  const float s = fmaxf(amax / 127.0f, FLT_MIN);
#pragma unroll
  for (int i = 0; i < 4; ++i) qv[i] = (int8_t)roundf(fminf(fmaxf(vals[i] / s, -127.0f), 127.0f));
  return s;
}

__device__ __forceinline__ float q8_quant_row(const float* src, uint32_t dr, int lane, int8_t (&qv)[4]) {
  float vals[4];
  q8_load_row(src, dr, lane, vals);
  return q8_quant_vals(vals, qv);
}

__device__ __forceinline__ uint32_t pack_q8x4(const int8_t (&qv)[4]) {
  return (uint32_t)(uint8_t)qv[0] | ((uint32_t)(uint8_t)qv[1] << 8) | ((uint32_t)(uint8_t)qv[2] << 16) |
         ((uint32_t)(uint8_t)qv[3] << 24);
}

// Quantises one (token, kv_head) row of K (kind 0) or V (kind 1) with one
// 64-lane wave and stores it into page `page` slot `slot`.  `src` holds the
// dr real dimensions; the page row has Dp, and dimensions dr..Dp-1 store
// zero.
__device__ __forceinline__ void q8_store_row(const AttnSeq& sq, const float* src, uint32_t kind, int32_t page,
                                             uint32_t slot, uint32_t kvh, uint32_t kvh_count, uint32_t dr,
                                             uint32_t Dp, int lane) {
  int8_t qv[4];
  const float s = q8_quant_row(src, dr, lane, qv);
  const size_t pkv = (size_t)page * kvh_count + kvh;
  if ((uint32_t)lane * 4 < Dp) {
    if (kind == 0) {
      *(uint32_t*)(sq.k + (pkv * 16 + slot) * Dp + lane * 4) = pack_q8x4(qv);
    } else {
#pragma unroll
      for (int i = 0; i < 4; ++i) sq.v[(pkv * Dp + lane * 4 + i) * 16 + slot] = qv[i];
    }
  }
  if (lane == 0) (kind == 0 ? sq.ks : sq.vs)[pkv * 16 + slot] = s;
}

// Eight bf16 of a query/gate row starting at element d0, zero past the real
// dimension dr; `full` (dr == Dp) takes one 16-byte load.
__device__ __forceinline__ u32x4 load_bf16x8(const uint16_t* row, uint32_t d0, uint32_t dr, bool full) {
  if (full) return *(const u32x4*)(row + d0);
  uint32_t h[8];
#pragma unroll
  for (int e = 0; e < 8; ++e) h[e] = d0 + e < dr ? (uint32_t)row[d0 + e] : 0u;
  return u32x4{h[0] | (h[1] << 16), h[2] | (h[3] << 16), h[4] | (h[5] << 16), h[6] | (h[7] << 16)};
}

// Physical page of logical page p: pages materialised by this call are not
// in the device table until this call writes them.
__device__ __forceinline__ int32_t page_id(const AttnSeq& sq, uint32_t p) {
  return sq.new_page_count > 0 && (int32_t)p >= sq.new_page_first ? sq.new_page_id + ((int32_t)p - sq.new_page_first)
                                                                 : sq.pt[p];
}

// ---------------------------------------------------------------------------
// Append
// ---------------------------------------------------------------------------
__global__ __launch_bounds__(64) void q8_append_kernel(AppendArgs args) {
  // blockIdx.x -> (item, kv_head, kind); item = sequence (decode) or row (prefill).
  const uint32_t kvh_count = args.kv_heads;
  const uint32_t kind = blockIdx.x % 2;
  const uint32_t kvh = (blockIdx.x / 2) % kvh_count;
  const uint32_t item = blockIdx.x / (2 * kvh_count);
  const int lane = threadIdx.x;
  const uint32_t D = args.head_dim, Dp = args.head_dim_pad;
  const AttnSeq& sq = args.seqs[args.decode ? item : 0];
  const uint32_t token = args.decode ? sq.len - 1 : args.start + item;
  // Page-table entries of newly materialised pages (written once per call).
  if (kind == 0 && kvh == 0 && (args.decode || item == 0) && lane == 0) {
    for (int32_t i = 0; i < sq.new_page_count; ++i) sq.pt[sq.new_page_first + i] = sq.new_page_id + i;
  }
  const float* src = (kind == 0 ? args.k : args.v) + ((size_t)item * kvh_count + kvh) * D;
  q8_store_row(sq, src, kind, page_id(sq, token / 16), token % 16, kvh, kvh_count, D, Dp, lane);
}

// Prefill append, one workgroup per (page, kv_head) of the rows' pages: each
// wave quantises tokens of the page (K rows go straight to the page, V values
// into an LDS copy of the page's d-major V block), then each thread stores one
// 16-token V row of the block with one 16-byte write.  A page the call only
// partly fills first takes its existing V rows into LDS, so the slots of
// earlier tokens keep their bytes.  The same quantiser as q8_store_row: the
// bytes and scales do not depend on the kernel that wrote them.
constexpr int kAppendWaves = 4;
__global__ __launch_bounds__(64 * kAppendWaves) void q8_append_pages_kernel(AppendArgs args) {
  __shared__ __attribute__((aligned(16))) uint8_t vb[256 * 16];  // [d][slot], Dp <= 256
  const uint32_t KVH = args.kv_heads, D = args.head_dim, Dp = args.head_dim_pad;
  const AttnSeq& sq = args.seqs[0];
  const uint32_t p = args.start / 16 + blockIdx.x / KVH, kvh = blockIdx.x % KVH;
  const uint32_t tid = threadIdx.x, wave = tid >> 6;
  const int lane = tid & 63;
  const uint32_t lo = max(args.start, 16 * p) - 16 * p, hi = min(sq.len, 16 * p + 16) - 16 * p;
  // Page-table entry of a page this call materialises (one writer per page).
  if (kvh == 0 && tid == 0 && sq.new_page_count > 0 && (int32_t)p >= sq.new_page_first &&
      (int32_t)p < sq.new_page_first + sq.new_page_count)
    sq.pt[p] = sq.new_page_id + ((int32_t)p - sq.new_page_first);
  const size_t pkv = (size_t)page_id(sq, p) * KVH + kvh;
  int8_t* vpage = sq.v + pkv * Dp * 16;
  if ((lo > 0 || hi < 16) && tid < Dp) *(u32x4*)(vb + 16 * tid) = *(const u32x4*)(vpage + 16 * tid);
  __syncthreads();
  // A wave's (up to) four tokens: every K and V load in flight first.
  constexpr int kPer = 16 / kAppendWaves;
  float kx[kPer][4], vx[kPer][4];
#pragma unroll
  for (int t = 0; t < kPer; ++t) {
    const uint32_t slot = lo + wave + kAppendWaves * t;
    const size_t row = ((size_t)(16 * p + min(slot, hi - 1) - args.start) * KVH + kvh) * D;
    q8_load_row(args.k + row, D, lane, kx[t]);
    q8_load_row(args.v + row, D, lane, vx[t]);
  }
#pragma unroll
  for (int t = 0; t < kPer; ++t) {
    const uint32_t slot = lo + wave + kAppendWaves * t;
    if (slot >= hi) break;  // wave-uniform
    int8_t qk[4], qv[4];
    const float sk = q8_quant_vals(kx[t], qk);
    const float sv = q8_quant_vals(vx[t], qv);
    if ((uint32_t)lane * 4 < Dp) {
      *(uint32_t*)(sq.k + (pkv * 16 + slot) * Dp + lane * 4) = pack_q8x4(qk);
#pragma unroll
      for (int i = 0; i < 4; ++i) vb[(lane * 4 + i) * 16 + slot] = (uint8_t)qv[i];
    }
    if (lane == 0) {
      sq.ks[pkv * 16 + slot] = sk;
      sq.vs[pkv * 16 + slot] = sv;
    }
  }
  __syncthreads();
  if (tid < Dp) *(u32x4*)(vpage + 16 * tid) = *(const u32x4*)(vb + 16 * tid);
}

// ---------------------------------------------------------------------------
// Decode: pages stream through a per-wave LDS ring by buffer->LDS DMA
// ---------------------------------------------------------------------------
__device__ __forceinline__ __amdgpu_buffer_rsrc_t make_rsrc(const void* base, uint32_t bytes) {
  return __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(base), (short)0, (int)bytes, 0x00020000);
}

// Lane i's `size` bytes land at lds + i*size.  The builtin exists only in the
// device pass; the host pass of single-source HIP must not see it.
#if defined(__HIP_DEVICE_COMPILE__)
#define QM_LDS_PTR(p) ((__attribute__((address_space(3))) void*)(p))
__device__ __forceinline__ void dma16(__amdgpu_buffer_rsrc_t r, void* lds, uint32_t voff) {
  __builtin_amdgcn_raw_ptr_buffer_load_lds(r, QM_LDS_PTR(lds), 16, voff, 0, 0, 0);
}
__device__ __forceinline__ void dma4(__amdgpu_buffer_rsrc_t r, void* lds, uint32_t voff) {
  __builtin_amdgcn_raw_ptr_buffer_load_lds(r, QM_LDS_PTR(lds), 4, voff, 0, 0, 0);
}
#undef QM_LDS_PTR
#else
__device__ void dma16(__amdgpu_buffer_rsrc_t, void*, uint32_t);
__device__ void dma4(__amdgpu_buffer_rsrc_t, void*, uint32_t);
#endif

// s_waitcnt vmcnt(n) (gfx9 encoding; expcnt and lgkmcnt left at their maxima).
template <int N>
__device__ __forceinline__ void wait_vmcnt() {
  static_assert(N >= 0 && N < 64, "vmcnt range");
  __builtin_amdgcn_s_waitcnt(0x0F70 | (N & 0xF) | ((N >> 4) << 14));
  __asm__ volatile("" ::: "memory");
}

// XOR swizzle of the 16-byte chunks of one token row of a K page in LDS, so
// the 16 lanes of one ds_read_b128 phase (16 tokens, same chunk) hit
// distinct banks.
template <int D>
__device__ __forceinline__ uint32_t k_chunk_slot(uint32_t tok, uint32_t j) {
  constexpr uint32_t kChunks = D / 16;
  const uint32_t sw = kChunks == 16 ? tok : kChunks == 8 ? ((tok & 7) ^ (tok >> 3)) : (tok & 3);
  return tok * kChunks + (j ^ sw);
}

// Two fp32 values -> packed bf16 (round to nearest even, v_cvt_pk_bf16_f32).
typedef __bf16 bf16x2_t __attribute__((ext_vector_type(2)));
__device__ __forceinline__ uint32_t pack_bf16x2(float lo, float hi) {
  const bf16x2_t v = {(__bf16)lo, (__bf16)hi};
  return __builtin_bit_cast(uint32_t, v);
}
__device__ __forceinline__ float bf16_lo_f32(uint32_t w) { return __uint_as_float(w << 16); }
__device__ __forceinline__ float bf16_hi_f32(uint32_t w) { return __uint_as_float(w & 0xFFFF0000u); }

// 4 int8 -> fp16 of 1024 + (int8 + 128), exact: (0x64 << 8 | u) is the fp16
// 1024 + u.  Element order (b0, b2), (b1, b3): one AND-OR per pair.
__device__ __forceinline__ u32x2 q8x4_to_f16_biased(uint32_t w) {
  const uint32_t u = w ^ 0x80808080u;
  return u32x2{(u & 0x00FF00FFu) | 0x64006400u, ((u >> 8) & 0x00FF00FFu) | 0x64006400u};
}
typedef _Float16 half8_t __attribute__((ext_vector_type(8)));
// 4 signed int8 -> bf16 pairs (b0, b1), (b2, b3), exact (v_cvt_f32_i32 with a
// sign-extended byte select, then v_cvt_pk_bf16_f32).
__device__ __forceinline__ u32x2 q8x4_to_bf16_signed(uint32_t w) {
  return u32x2{pack_bf16x2((float)(int8_t)w, (float)(int8_t)(w >> 8)),
               pack_bf16x2((float)(int8_t)(w >> 16), (float)(int8_t)(w >> 24))};
}

__device__ __forceinline__ floatx4 mfma16x16x32_f16(u32x4 a, u32x4 b, floatx4 c) {
  return __builtin_amdgcn_mfma_f32_16x16x32_f16(__builtin_bit_cast(half8_t, a), __builtin_bit_cast(half8_t, b), c,
                                                0, 0, 0);
}
// Maximum over the four lanes l, l^16, l^32, l^48 (the kq lanes of one MFMA
// column) with the gfx950 row-swap permutes instead of LDS shuffles.
__device__ __forceinline__ float max4_across_kq(float v) {
  const auto a = __builtin_amdgcn_permlane16_swap(__float_as_uint(v), __float_as_uint(v), false, false);
  // fmaxf is v_max_f32 (one operation; the operands are never NaN), where a
  // compare and select would be two plus a VCC hazard wait.
  const float m = fmaxf(__uint_as_float(a[0]), __uint_as_float(a[1]));
  const auto b = __builtin_amdgcn_permlane32_swap(__float_as_uint(m), __float_as_uint(m), false, false);
  return fmaxf(__uint_as_float(b[0]), __uint_as_float(b[1]));
}

template <bool B>
struct BoolTag {
  static constexpr bool value = B;
};

template <int D, int W>
struct DecodeLds {
  static constexpr int kWaves = W;
  static constexpr int kRing = D == 256 ? 2 : 4;  // pages in flight per wave
  static constexpr int kK = 16 * D, kV = 16 * D, kS = 512;  // K, V, scales (K 256 B + V 256 B)
  static constexpr int kPage = kK + kV + kS;
  static constexpr int kWaveRing = kRing * kPage;
  static constexpr int kPad = 17;  // floats per (wave, d) row of the O reduction (16 columns + 1)
  static constexpr int kRed = W * D * kPad * 4 + (3 * W + 2) * 16 * 4;  // O, m, l, weights, max, sums
  static constexpr int kBytes = W * kWaveRing > kRed ? W * kWaveRing : kRed;
};

template <int D, int W>
__global__ __launch_bounds__(64 * W) void q8_decode_kernel(AttnArgs args) {
  using L = DecodeLds<D, W>;
  constexpr int kWaves = W, kDB = D / 16, kKS = D / 32, kRing = L::kRing;
  constexpr int kKChunks = D / 16;          // 16-byte chunks per K token row
  constexpr int kKDma = D / 64;             // DMA instructions per K (and V) page
  constexpr int kDmaPerPage = 2 * kKDma + 2;
  __shared__ __attribute__((aligned(16))) uint8_t lds[L::kBytes];

  const int lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int col = lane & 15, kq = lane >> 4, tok = lane & 15;
  const uint32_t H = args.heads, KVH = args.kv_heads, gh = H / KVH;

  uint32_t b = 0;
  const uint32_t unit = blockIdx.x;
  while (b + 1 < args.n_seqs && unit >= args.seqs[b + 1].unit_begin) ++b;
  const AttnSeq& sq = args.seqs[b];
  const uint32_t u = unit - sq.unit_begin;
  const uint32_t kvh = u % KVH, split = u / KVH;
  const uint32_t pages = (sq.len + 15) / 16;
  const uint32_t p_begin = split * args.pages_per_split;
  const uint32_t p_end = min(pages, p_begin + args.pages_per_split);

  const bool col_ok = (uint32_t)col < gh;
  const uint32_t head = kvh * gh + col;
  const uint32_t visible = sq.len;

  // Q operand (B of QK^T), filled after the first page DMAs are in flight.
  u32x4 qb[kKS];
  float qcorr = 0.0f;
  const uint32_t dr = args.head_dim;  // real head dimension; D is the page storage width
  const bool full_d = dr == (uint32_t)D;
  const float sm_scale = kLog2e / sqrtf((float)dr);

  floatx4 o[kDB];
#pragma unroll
  for (int i = 0; i < kDB; ++i) o[i] = floatx4{0.f, 0.f, 0.f, 0.f};
  float m_run = -INFINITY, l_lane = 0.0f;

  // ---- this wave's pages: p_begin + wave + 4 i ------------------------------
  uint8_t* ring = lds + wave * L::kWaveRing;
  const size_t kv_page_stride = (size_t)KVH * 16 * D;
  // Per-lane source offsets of the K DMA (chunk slot -> (token, chunk)).
  uint32_t k_src[kKDma];
#pragma unroll
  for (int h = 0; h < kKDma; ++h) {
    const uint32_t slot = h * 64 + lane;
    const uint32_t t = slot / kKChunks, jj = slot % kKChunks;
    const uint32_t sw = kKChunks == 16 ? t : kKChunks == 8 ? ((t & 7) ^ (t >> 3)) : (t & 3);
    k_src[h] = t * D + (jj ^ sw) * 16;
  }
  const uint32_t first = p_begin + wave;
  const uint32_t n_mine = first < p_end ? (p_end - first + kWaves - 1) / kWaves : 0;
  // The last split of each (sequence, KV head) appends the new token first
  // (waves 0 and 1 quantise K and V); the barrier below orders those stores
  // before any wave's DMA of the last page.  KV head 0 also records pages
  // materialised by this call in the page table.
  if (split + 1 == sq.nsplit) {
    const uint32_t token = sq.len - 1;
    if (wave < 2) {
      const float* src = (wave == 0 ? args.k_new : args.v_new) + ((size_t)b * KVH + kvh) * dr;
      q8_store_row(sq, src, wave, page_id(sq, token / 16), token % 16, kvh, KVH, dr, D, lane);
    } else if (wave == 2 && kvh == 0 && lane == 0) {
      for (int32_t i = 0; i < sq.new_page_count; ++i) sq.pt[sq.new_page_first + i] = sq.new_page_id + i;
    }
    wait_vmcnt<0>();
    __syncthreads();
  }
  // Physical ids of this wave's first 64 pages, lane j holding page j, read
  // once before any DMA and taken with v_readlane at issue time.  A scalar
  // load per refill would leave an SMEM access outstanding, and since SMEM
  // returns out of order every later LDS read would wait for it (lgkmcnt(0)):
  // one memory round trip per ring step.  Pages beyond the 64th (splits over
  // 256 pages) fall back to scalar loads through the constant address space.
  // The only table entries this kernel writes are pages materialised by this
  // call, whose ids are computed without a read.
  const __attribute__((address_space(4))) int32_t* pt_s =
      (const __attribute__((address_space(4))) int32_t*)sq.pt;
  auto phys_of = [&](uint32_t p) __attribute__((always_inline)) {
    return sq.new_page_count > 0 && (int32_t)p >= sq.new_page_first ? sq.new_page_id + ((int32_t)p - sq.new_page_first)
                                                                     : -1;
  };
  int32_t ids_v;
  {
    const uint32_t p = first + kWaves * (uint32_t)lane;
    const int32_t fresh = phys_of(p);
    ids_v = (uint32_t)lane < n_mine && fresh < 0 ? sq.pt[p] : fresh;
  }
  auto issue = [&](uint32_t j, int slot_idx) __attribute__((always_inline)) {
    const uint32_t p = first + kWaves * j;
    int32_t phys;
    if (j < 64) {
      phys = __builtin_amdgcn_readlane(ids_v, (int)j);
    } else {
      const int32_t fresh = phys_of(p);
      phys = fresh >= 0 ? fresh : pt_s[p];
    }
    uint8_t* dst = ring + slot_idx * L::kPage;
    const size_t pbase = (size_t)phys * kv_page_stride;
    const __amdgpu_buffer_rsrc_t rk = make_rsrc(sq.k + pbase + (size_t)kvh * 16 * D, 16 * D);
    const __amdgpu_buffer_rsrc_t rv = make_rsrc(sq.v + pbase + (size_t)kvh * 16 * D, 16 * D);
    const size_t sbase = ((size_t)phys * KVH + kvh) * 16;
    const __amdgpu_buffer_rsrc_t rks = make_rsrc(sq.ks + sbase, 64);
    const __amdgpu_buffer_rsrc_t rvs = make_rsrc(sq.vs + sbase, 64);
#pragma unroll
    for (int h = 0; h < kKDma; ++h) dma16(rk, dst + h * 1024, k_src[h]);
#pragma unroll
    for (int h = 0; h < kKDma; ++h) dma16(rv, dst + L::kK + h * 1024, (h * 64 + lane) * 16);
    dma4(rks, dst + L::kK + L::kV, (lane & 15) * 4);
    dma4(rvs, dst + L::kK + L::kV + 256, (lane & 15) * 4);
  };
  // Scores of one page: S^T[token][col] over D in kKS steps of 32.
  auto qk = [&](const uint8_t* src) {
    floatx4 s4 = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int j = 0; j < kKS / 2; ++j) {
      const uint32_t chunk = (D / 64) * kq + j;
      const u32x4 kb = *(const u32x4*)(src + 16 * k_chunk_slot<D>(tok, chunk));
      const u32x2 l0 = q8x4_to_f16_biased(kb.x), h0 = q8x4_to_f16_biased(kb.y);
      const u32x2 l1 = q8x4_to_f16_biased(kb.z), h1 = q8x4_to_f16_biased(kb.w);
      s4 = mfma16x16x32_f16(u32x4{l0.x, l0.y, h0.x, h0.y}, qb[2 * j], s4);
      s4 = mfma16x16x32_f16(u32x4{l1.x, l1.y, h1.x, h1.y}, qb[2 * j + 1], s4);
    }
    return s4;
  };
  // Two pages per step (the second may be absent): two independent QK
  // chains, one running-max update per 32 tokens, then P'V for both.
  auto process2 = [&](uint32_t pA, int sA, uint32_t pB, int sB, bool hasB) {
    const uint8_t* srcA = ring + sA * L::kPage;
    const uint8_t* srcB = ring + sB * L::kPage;
    const floatx4 s4A = qk(srcA);
    const floatx4 s4B = qk(srcB);
    const floatx4 ksA = *(const floatx4*)(srcA + L::kK + L::kV + 16 * kq);
    const floatx4 vsA = *(const floatx4*)(srcA + L::kK + L::kV + 256 + 16 * kq);
    const floatx4 ksB = *(const floatx4*)(srcB + L::kK + L::kV + 16 * kq);
    const floatx4 vsB = *(const floatx4*)(srcB + L::kK + L::kV + 256 + 16 * kq);
    float sc[8];
    float bmax = -INFINITY;
#pragma unroll
    for (int rr = 0; rr < 4; ++rr) {
      const uint32_t tA = pA * 16 + 4 * kq + rr, tB = pB * 16 + 4 * kq + rr;
      sc[rr] = col_ok && tA < visible ? (s4A[rr] - qcorr) * ksA[rr] * sm_scale : -INFINITY;
      sc[4 + rr] = col_ok && hasB && tB < visible ? (s4B[rr] - qcorr) * ksB[rr] * sm_scale : -INFINITY;
      bmax = fmaxf(bmax, fmaxf(sc[rr], sc[4 + rr]));
    }
    bmax = max4_across_kq(bmax);
    // Lazy rescaling: the reference maximum only moves when a score exceeds it
    // by more than 2^8, so exp2(s - m_run) <= 256 stays exact in fp32 and the
    // O / l rescale (a pass over every accumulator) is rare.  The final
    // division by l makes the result independent of the reference chosen.
    const float m_new = bmax > m_run + 8.0f ? bmax : m_run;
    const bool moved = m_new != m_run;
    const float corr = moved ? exp2f(m_run - m_new) : 1.0f;
    m_run = m_new;
    float pw[8];
    float psum = 0.0f;
#pragma unroll
    for (int rr = 0; rr < 8; ++rr) {
      // v_exp_f32 directly: arguments are <= 8 here, and a flushed tiny
      // probability is below fp32 resolution of the running sum anyway.
      const float e = sc[rr] == -INFINITY ? 0.0f : __builtin_amdgcn_exp2f(sc[rr] - m_new);
      psum += e;
      pw[rr] = e * (rr < 4 ? vsA[rr] : vsB[rr - 4]);
    }
    l_lane = l_lane * corr + psum;
    if (__builtin_amdgcn_ballot_w64(moved)) {
#pragma unroll
      for (int db = 0; db < kDB; ++db) o[db] *= corr;
    }
    // P' = p * v_scale as bf16 hi + lo (error ~2^-16).  Both halves ride in
    // the K dimension of one 16x16x32 MFMA: lane (d, kq) supplies
    // A = V^T[d][4kq..4kq+3] twice and B = (hi, lo) of the same four tokens.
    u32x4 pb[2];
#pragma unroll
    for (int h = 0; h < 2; ++h) {
      const float* w = pw + 4 * h;
      const uint32_t h01 = pack_bf16x2(w[0], w[1]), h23 = pack_bf16x2(w[2], w[3]);
      pb[h] = u32x4{h01, h23, pack_bf16x2(w[0] - bf16_lo_f32(h01), w[1] - bf16_hi_f32(h01)),
                    pack_bf16x2(w[2] - bf16_lo_f32(h23), w[3] - bf16_hi_f32(h23))};
    }
    // V enters unbiased (signed bytes -> bf16): nothing accumulates into O but
    // sum_t v_t p'_t, however long the sequence.
#pragma unroll
    for (int db = 0; db < kDB; ++db) {
      const uint32_t off = L::kK + (16 * db + tok) * 16 + 4 * kq;
      const u32x2 va = q8x4_to_bf16_signed(*(const uint32_t*)(srcA + off));
      const u32x2 vb = q8x4_to_bf16_signed(*(const uint32_t*)(srcB + off));
      o[db] = mfma16x16x32(u32x4{va.x, va.y, va.x, va.y}, pb[0], o[db]);
      o[db] = mfma16x16x32(u32x4{vb.x, vb.y, vb.x, vb.y}, pb[1], o[db]);
    }
  };

  // Pages issued so far land in ring slots in order; a pair (i, i+1) needs
  // every DMA up to page i+1 complete: vmcnt <= (pages issued after it) *
  // kDmaPerPage.
  // Q rows are loaded before the first page DMAs so that waiting for them
  // does not wait for the pages (vmcnt retires in order).
  u32x4 qraw[kKS];
  {
    const uint16_t* qp = args.q + ((size_t)b * H + head) * dr;
#pragma unroll
    for (int jj = 0; jj < kKS; ++jj)
      qraw[jj] = col_ok ? load_bf16x8(qp, D / 4 * kq + 8 * jj, dr, full_d) : u32x4{0u, 0u, 0u, 0u};
  }
  __builtin_amdgcn_sched_barrier(0);
  const uint32_t pre = min(n_mine, (uint32_t)kRing);
  for (uint32_t i = 0; i < pre; ++i) issue(i, i);
  uint32_t issued = pre;
  // Q operand (B of QK^T) in fp16: lane (col, kq) holds q[head][D/4 kq + 8 j
  // .. + 7] in the element order d0,d2,d1,d3,d4,d6,d5,d7 that the int8 -> fp16
  // unpack of K produces.  bf16 -> fp16 is exact within fp16's range.
  {
    float qsum = 0.0f;
#pragma unroll
    for (int jj = 0; jj < kKS; ++jj) {
      const u32x4 v = qraw[jj];
      float f[8];
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        f[2 * e] = bf16_to_f32(v[e] & 0xFFFFu);
        f[2 * e + 1] = bf16_to_f32(v[e] >> 16);
      }
      const int order[8] = {0, 2, 1, 3, 4, 6, 5, 7};
      uint32_t h[8];
#pragma unroll
      for (int e = 0; e < 8; ++e) {
        const _Float16 x = (_Float16)f[order[e]];
        qsum += (float)x;
        h[e] = __builtin_bit_cast(uint16_t, x);
      }
      qb[jj] = u32x4{h[0] | (h[1] << 16), h[2] | (h[3] << 16), h[4] | (h[5] << 16), h[6] | (h[7] << 16)};
    }
    qsum += __shfl_xor(qsum, 16);
    qsum += __shfl_xor(qsum, 32);
    qcorr = 1152.0f * qsum;  // K enters as 1024 + (k + 128)
  }

  for (uint32_t i = 0; i < n_mine; i += 2) {
    const bool hasB = i + 1 < n_mine;
    const uint32_t last = hasB ? i + 1 : i;
    const uint32_t later = issued - 1 - last;
    if (later >= 2) wait_vmcnt<2 * kDmaPerPage>();
    else if (later == 1) wait_vmcnt<kDmaPerPage>();
    else wait_vmcnt<0>();
    process2(first + kWaves * i, i % kRing, first + kWaves * last, last % kRing, hasB);
    for (uint32_t j = i; j <= last; ++j)
      if (j + kRing < n_mine) {
        issue(j + kRing, j % kRing);
        ++issued;
      }
  }

  // ---- combine the waves of the workgroup ------------------------------------
  float l_tot = l_lane + __shfl_xor(l_lane, 16);
  l_tot += __shfl_xor(l_tot, 32);
  __syncthreads();  // the rings are reused for the reduction
  constexpr int kPad = L::kPad;
  float* red_o = reinterpret_cast<float*>(lds);  // [wave][d][kPad]
  float(*red_m)[16] = reinterpret_cast<float(*)[16]>(lds + kWaves * D * kPad * 4);
  float(*red_l)[16] = red_m + kWaves;
#pragma unroll
  for (int db = 0; db < kDB; ++db)
#pragma unroll
    for (int r = 0; r < 4; ++r) red_o[(wave * D + 16 * db + 4 * kq + r) * kPad + col] = o[db][r];
  if (kq == 0) {
    red_m[wave][col] = m_run;
    red_l[wave][col] = l_tot;
  }
  __syncthreads();
  // Per (wave, column) weights exp2(m_w - max) and the column sums, once;
  // the element loop below is then multiply-adds only.
  float(*red_f)[16] = red_l + kWaves;  // [wave][col]
  float* red_mx = red_l[2 * kWaves];
  float* red_L = red_mx + 16;
  if (threadIdx.x < 16) {
    const uint32_t c = threadIdx.x;
    float mx = -INFINITY;
#pragma unroll
    for (int w = 0; w < kWaves; ++w) mx = fmaxf(mx, red_m[w][c]);
    float Ls = 0.0f;
#pragma unroll
    for (int w = 0; w < kWaves; ++w) {
      const float f = red_m[w][c] == -INFINITY ? 0.0f : exp2f(red_m[w][c] - mx);
      red_f[w][c] = f;
      Ls += f * red_l[w][c];
    }
    red_mx[c] = mx;
    red_L[c] = Ls;
  }
  __syncthreads();
  const uint32_t nsplit = sq.nsplit;
  // Split partials: O [split row][H][D], then (m, l) [split row][H][2];
  // q8_combine_kernel merges them after this launch.
  const size_t o_rows = (size_t)args.part_rows * H;
  float* po = args.partials;
  float* pm = args.partials + o_rows * D;
  constexpr uint32_t kD4 = D / 4;
  for (uint32_t e = threadIdx.x; e < gh * kD4; e += 64 * kWaves) {
    const uint32_t c = e / kD4, d0 = 4 * (e % kD4);
    floatx4 O = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int w = 0; w < kWaves; ++w)
#pragma unroll
      for (int i = 0; i < 4; ++i) O[i] += red_f[w][c] * red_o[(w * D + d0 + i) * kPad + c];
    const uint32_t hh = kvh * gh + c;
    if (nsplit == 1) {
      const float inv = 1.0f / fmaxf(red_L[c], FLT_MIN);
      const size_t oi = ((size_t)b * H + hh) * dr + d0;
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        if (d0 + i >= dr) break;
        float v = O[i] * inv;
        if (args.gate) v *= sigmoid_f(bf16_to_f32(args.gate[oi + i]));
        args.o[oi + i] = f32_to_bf16(v);
      }
    } else {
      const size_t row = (size_t)(sq.part_begin + split) * H + hh;
      *(floatx4*)(po + row * D + d0) = O;
      if (d0 == 0) *(float2*)(pm + row * 2) = float2{red_mx[c], red_L[c]};
    }
  }
}

// Merge the split partials of one (sequence, head, 32-wide d slice): grid
// (n_seqs * H * D/32), 256 threads.  Thread t owns float4 slice c = t % 8 of
// the workgroup's 32 d and the splits s = t / 8 + 32 k, and loads every
// (O slice, m, l) it needs in one go, so the merge costs one memory round
// trip spread over many workgroups; the per-head maximum and the sums over
// splits then meet in LDS.
template <int D>
__global__ __launch_bounds__(256) void q8_combine_kernel(AttnArgs args) {
  constexpr int kWgPerHead = D / 32;  // workgroups per (sequence, head)
  constexpr int kGroups = 32;         // split groups (threads per slice)
  constexpr int kMaxPer = 4;          // splits a thread holds in registers per pass
  __shared__ float red_m[256];
  __shared__ floatx4 red_o[256];
  __shared__ float red_l[256];
  const uint32_t H = args.heads, dr = args.head_dim;
  const uint32_t wq = blockIdx.x % kWgPerHead;
  const uint32_t bh = blockIdx.x / kWgPerHead;
  const uint32_t b = bh / H, hh = bh % H;
  const AttnSeq& sq = args.seqs[b];
  const uint32_t ns = sq.nsplit;
  if (ns <= 1 || 32 * wq >= dr) return;
  const size_t o_rows = (size_t)args.part_rows * H;
  const float* obase = args.partials + ((size_t)sq.part_begin * H + hh) * D;
  const float* mbase = args.partials + o_rows * D + ((size_t)sq.part_begin * H + hh) * 2;
  const uint32_t t = threadIdx.x, c = t % 8, g = t / 8;
  const uint32_t d0 = 32 * wq + 4 * c;

  float mloc = -INFINITY;
  floatx4 acc = {0.f, 0.f, 0.f, 0.f};
  float lacc = 0.0f;
  for (uint32_t s0 = 0; s0 < ns; s0 += kGroups * kMaxPer) {
    floatx4 ov[kMaxPer];
    float2 ml[kMaxPer];
    // Unconditional loads (index clamped, weight masked) so all of them are
    // in flight together.
#pragma unroll
    for (int k = 0; k < kMaxPer; ++k) {
      const uint32_t s = s0 + g + k * kGroups;
      const size_t row = s < ns ? s : ns - 1;
      ov[k] = *(const floatx4*)(obase + row * H * D + d0);
      ml[k] = *(const float2*)(mbase + row * H * 2);
    }
    float mv[kMaxPer];
#pragma unroll
    for (int k = 0; k < kMaxPer; ++k) mv[k] = s0 + g + k * kGroups < ns ? ml[k].x : -INFINITY;
    float mnew = mloc;
#pragma unroll
    for (int k = 0; k < kMaxPer; ++k) mnew = fmaxf(mnew, mv[k]);
    if (mnew != -INFINITY) {
      const float r = mloc == -INFINITY ? 0.0f : exp2f(mloc - mnew);
      acc *= r;
      lacc *= r;
#pragma unroll
      for (int k = 0; k < kMaxPer; ++k) {
        const float f = mv[k] == -INFINITY ? 0.0f : exp2f(mv[k] - mnew);
        acc += ov[k] * f;
        lacc += ml[k].y * f;
      }
      mloc = mnew;
    }
  }
  red_m[t] = mloc;
  __syncthreads();
  float mx = -INFINITY;
  for (int k = 0; k < kGroups; ++k) mx = fmaxf(mx, red_m[c + 8 * k]);
  const float f = mloc == -INFINITY ? 0.0f : exp2f(mloc - mx);
  red_o[t] = acc * f;
  red_l[t] = lacc * f;
  __syncthreads();
  if (g == 0) {
    floatx4 o = red_o[c];
    float L = red_l[c];
    for (int k = 1; k < kGroups; ++k) {
      o += red_o[c + 8 * k];
      L += red_l[c + 8 * k];
    }
    const float inv = 1.0f / fmaxf(L, FLT_MIN);
    const size_t oi = ((size_t)b * H + hh) * dr + d0;
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      if (d0 + e >= dr) break;
      float v = o[e] * inv;
      if (args.gate) v *= sigmoid_f(bf16_to_f32(args.gate[oi + e]));
      args.o[oi + e] = f32_to_bf16(v);
    }
  }
}

// The same merge when every sequence has at most 32 splits: one wave per
// (sequence, head, 32-wide d slice).  Lane (c, g) = (t % 8, t / 8) holds
// float4 slice c and splits g, g + 8, g + 16, g + 24, all loaded at once;
// the maximum and the sums over g meet through lane swaps (xor 8, 16, 32),
// so the merge needs no LDS and no barrier.
template <int D>
__global__ __launch_bounds__(64) void q8_combine_small_kernel(AttnArgs args) {
  constexpr int kWgPerHead = D / 32;
  constexpr int kPer = 4;  // splits per lane
  const uint32_t H = args.heads, dr = args.head_dim;
  const uint32_t wq = blockIdx.x % kWgPerHead;
  const uint32_t bh = blockIdx.x / kWgPerHead;
  const uint32_t b = bh / H, hh = bh % H;
  const AttnSeq& sq = args.seqs[b];
  const uint32_t ns = sq.nsplit;
  if (ns <= 1 || 32 * wq >= dr) return;
  const size_t o_rows = (size_t)args.part_rows * H;
  const float* obase = args.partials + ((size_t)sq.part_begin * H + hh) * D;
  const float* mbase = args.partials + o_rows * D + ((size_t)sq.part_begin * H + hh) * 2;
  const uint32_t t = threadIdx.x, c = t % 8, g = t / 8;
  const uint32_t d0 = 32 * wq + 4 * c;
  floatx4 ov[kPer];
  float2 ml[kPer];
#pragma unroll
  for (int k = 0; k < kPer; ++k) {
    const uint32_t s = g + 8 * k;
    const size_t row = s < ns ? s : ns - 1;
    ov[k] = *(const floatx4*)(obase + row * H * D + d0);
    ml[k] = *(const float2*)(mbase + row * H * 2);
  }
  float mv[kPer];
  float mx = -INFINITY;
#pragma unroll
  for (int k = 0; k < kPer; ++k) {
    mv[k] = g + 8 * k < ns ? ml[k].x : -INFINITY;
    mx = fmaxf(mx, mv[k]);
  }
  mx = fmaxf(mx, __shfl_xor(mx, 8));
  mx = fmaxf(mx, __shfl_xor(mx, 16));
  mx = fmaxf(mx, __shfl_xor(mx, 32));
  floatx4 acc = {0.f, 0.f, 0.f, 0.f};
  float L = 0.0f;
#pragma unroll
  for (int k = 0; k < kPer; ++k) {
    const float f = mv[k] == -INFINITY ? 0.0f : exp2f(mv[k] - mx);
    acc += ov[k] * f;
    L += ml[k].y * f;
  }
#pragma unroll
  for (int m = 8; m < 64; m <<= 1) {
#pragma unroll
    for (int e = 0; e < 4; ++e) acc[e] += __shfl_xor(acc[e], m);
    L += __shfl_xor(L, m);
  }
  if (g == 0) {
    const float inv = 1.0f / fmaxf(L, FLT_MIN);
    const size_t oi = ((size_t)b * H + hh) * dr + d0;
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      if (d0 + e >= dr) break;
      float v = acc[e] * inv;
      if (args.gate) v *= sigmoid_f(bf16_to_f32(args.gate[oi + e]));
      args.o[oi + e] = f32_to_bf16(v);
    }
  }
}

// Causal prefill: blockIdx.x = rb * KVH + kvh.  A wave owns CB column
// blocks of 16 (row, head) columns, i.e. CB * 16 / gh query rows of one KV
// head; the workgroup's four waves own consecutive rows and walk the same
// pages, which are unpacked once per workgroup into LDS (each wave a
// quarter) and serve every wave's CB blocks.
template <int D, int CB>
__global__ __launch_bounds__(256) void q8_prefill_kernel(AttnArgs args) {
  constexpr int kWaves = 4;
  constexpr int kDB = D / 16;  // 16-wide d blocks of O^T
  constexpr int kKS = D / 32;  // QK k-steps

  const int lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int col = lane & 15;  // (row, head) column within a block
  const int kq = lane >> 4;
  const uint32_t H = args.heads, KVH = args.kv_heads, gh = H / KVH;  // gh <= 16

  const uint32_t rows_per_block = 16 / gh, rows_per_wave = CB * rows_per_block;
  const uint32_t row_blocks = (args.rows + rows_per_wave * kWaves - 1) / (rows_per_wave * kWaves);
  // KV head = blockIdx % KVH: workgroups are dealt round-robin to the 8 XCDs,
  // so every row block of one KV head runs on the same XCD(s) and its pages
  // (1.5 MiB per head at 6K tokens, d = 128) stay in that XCD's L2.
  const uint32_t kvh = blockIdx.x % KVH;
  // Row blocks are dealt last first: the later rows see the most pages, and
  // starting the longest workgroups first lets the short ones fill the
  // slots they free (the grid runs in about two residency rounds).
  const uint32_t rb = row_blocks - 1 - blockIdx.x / KVH;
  const uint32_t row_base = (rb * kWaves + wave) * rows_per_wave;
  const AttnSeq& sq = args.seqs[0];

  const uint32_t ch = col % gh, cr = col / gh;
  const uint32_t head = kvh * gh + ch;
  bool col_ok[CB];
  uint32_t qrow[CB], visible[CB];
#pragma unroll
  for (int cb = 0; cb < CB; ++cb) {
    qrow[cb] = row_base + cb * rows_per_block + cr;
    col_ok[cb] = (uint32_t)col < rows_per_block * gh && qrow[cb] < args.rows;
    visible[cb] = min(args.start + qrow[cb] + 1, sq.len);
  }

  // Q operands (B of QK^T) in fp16: lane (col, kq) of block cb holds
  // q[qrow][head][D/4 kq + 8 j .. + 7] in the element order d0,d2,d1,d3,
  // d4,d6,d5,d7 that the int8 -> fp16 unpack of K produces.  bf16 -> fp16 is
  // exact within fp16's range.  K enters as 1024 + (k + 128): 1152 * sum(q)
  // is subtracted from every score.
  const uint32_t dr = args.head_dim;  // real head dimension; D is the page storage width
  const bool full_d = dr == (uint32_t)D;
  u32x4 qb[CB][kKS];
  float qcorr[CB];
#pragma unroll
  for (int cb = 0; cb < CB; ++cb) {
    const uint16_t* qp = args.q + ((size_t)qrow[cb] * H + head) * dr;
    float qsum = 0.0f;
#pragma unroll
    for (int jj = 0; jj < kKS; ++jj) {
      const u32x4 v = col_ok[cb] ? load_bf16x8(qp, D / 4 * kq + 8 * jj, dr, full_d) : u32x4{0u, 0u, 0u, 0u};
      float f[8];
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        f[2 * e] = bf16_to_f32(v[e] & 0xFFFFu);
        f[2 * e + 1] = bf16_to_f32(v[e] >> 16);
      }
      const int order[8] = {0, 2, 1, 3, 4, 6, 5, 7};
      uint32_t h[8];
#pragma unroll
      for (int e = 0; e < 8; ++e) {
        const _Float16 x = (_Float16)f[order[e]];
        qsum += (float)x;
        h[e] = __builtin_bit_cast(uint16_t, x);
      }
      qb[cb][jj] = u32x4{h[0] | (h[1] << 16), h[2] | (h[3] << 16), h[4] | (h[5] << 16), h[6] | (h[7] << 16)};
    }
    qsum += __shfl_xor(qsum, 16);
    qsum += __shfl_xor(qsum, 32);
    qcorr[cb] = 1152.0f * qsum;
  }
  const float sm_scale = kLog2e / sqrtf((float)dr);

  floatx4 o[CB][kDB];
  float m_run[CB], l_lane[CB];
#pragma unroll
  for (int cb = 0; cb < CB; ++cb) {
#pragma unroll
    for (int i = 0; i < kDB; ++i) o[cb][i] = floatx4{0.f, 0.f, 0.f, 0.f};
    m_run[cb] = -INFINITY;
    l_lane[cb] = 0.0f;
  }

  const size_t kv_page_stride = (size_t)KVH * 16 * D;
  const int tok = lane & 15;  // A-operand row: token of QK^T, d row of PV^T

  // The four waves walk the same pages.  Each page is unpacked once per
  // workgroup into an LDS stage (each wave a quarter of it) and every wave
  // reads its MFMA operands from there:
  //   K: u32x4 unit (j, kq, tok) = fp16 of 1024 + (k + 128) for
  //      K[tok][D/4 kq + 8 j .. + 7] in the order d0,d2,d1,d3,d4,d6,d5,d7,
  //      at row j * 4 + kq, slot tok ^ (row & 15);
  //   V: u32x2 unit (db, kq, d) = bf16 of V^T[16 db + d][4 kq .. 4 kq + 3]
  //      at row db * 4 + kq, slot d ^ 4 kq;
  //   scales: K scale * softmax scale, then V scale, per token.
  // The slot swizzles keep both the unpacking writes and the operand reads
  // (16 lanes, one row, all slots) free of bank conflicts.
  constexpr int kKUnits = 16 * D / 8;  // 8-byte units of one page's K (or V)
  constexpr int kPerLane = (kKUnits / kWaves + 63) / 64;
  constexpr int kStage = 16 * D * 2 + 16 * D * 2 + 128;
  __shared__ __attribute__((aligned(16))) uint8_t lds[2 * kStage];
  const int wave_unit0 = wave * (kKUnits / kWaves);

  // Last row of the workgroup bounds every wave's page walk, so all waves
  // pass the same barriers; pages past a wave's own rows are fully masked.
  const uint32_t wg_row0 = rb * kWaves * rows_per_wave;
  const uint32_t wg_last = min(args.rows, wg_row0 + kWaves * rows_per_wave) - 1;
  const uint32_t n_pages = (min(args.start + wg_last + 1, sq.len) + 15) / 16;

  struct Raw {
    u32x2 k[kPerLane], v[kPerLane];
    float sc;
  };
  auto fetch = [&](int32_t phys, Raw& r) __attribute__((always_inline)) {
    const size_t base = (size_t)phys * kv_page_stride + (size_t)kvh * 16 * D;
#pragma unroll
    for (int i = 0; i < kPerLane; ++i) {
      const int u = lane + 64 * i;
      if (u < kKUnits / kWaves) {
        const size_t off = base + 8 * (size_t)(wave_unit0 + u);
        r.k[i] = *(const u32x2*)(sq.k + off);
        r.v[i] = *(const u32x2*)(sq.v + off);
      }
    }
    if (wave == 0 && lane < 32) {
      const size_t si = ((size_t)phys * KVH + kvh) * 16 + (lane & 15);
      r.sc = lane < 16 ? sq.ks[si] * sm_scale : sq.vs[si];
    }
  };
  auto stage_in = [&](const Raw& r, int st) __attribute__((always_inline)) {
    uint8_t* base = lds + st * kStage;
#pragma unroll
    for (int i = 0; i < kPerLane; ++i) {
      const int u = lane + 64 * i;
      if (u < kKUnits / kWaves) {
        const int g = wave_unit0 + u;
        // K unit: token g / (D / 8), 8-byte chunk c = kq * kKS + j.
        const int kt = g / (D / 8), c = g % (D / 8);
        const u32x2 l = q8x4_to_f16_biased(r.k[i].x), h = q8x4_to_f16_biased(r.k[i].y);
        const int krow = (c % kKS) * 4 + c / kKS;
        *(u32x4*)(base + 16 * (krow * 16 + (kt ^ (krow & 15)))) = u32x4{l.x, l.y, h.x, h.y};
        // V unit: d row g / 2, tokens 8 (g & 1) .. + 7 = kq 2 (g & 1), + 1.
        const int d = g >> 1, kq0 = 2 * (g & 1);
        const u32x2 v0 = q8x4_to_bf16_signed(r.v[i].x), v1 = q8x4_to_bf16_signed(r.v[i].y);
        uint8_t* vb = base + 16 * D * 2;
        *(u32x2*)(vb + 8 * (((d >> 4) * 4 + kq0) * 16 + ((d & 15) ^ (4 * kq0)))) = v0;
        *(u32x2*)(vb + 8 * (((d >> 4) * 4 + kq0 + 1) * 16 + ((d & 15) ^ (4 * kq0 + 4)))) = v1;
      }
    }
    if (wave == 0 && lane < 32) *(float*)(base + 16 * D * 4 + 4 * lane) = r.sc;
  };

  // Softmax and P'V of page p from LDS stage st.  MASKED is false for pages
  // every column of the wave sees whole (all but the last few): those skip
  // the causal compare and select per score.
  auto compute = [&](uint32_t p, int st, auto masked) __attribute__((always_inline)) {
    constexpr bool MASKED = decltype(masked)::value;
    const uint8_t* base = lds + st * kStage;
    const u32x4* kl = (const u32x4*)base;
    const u32x2* vl = (const u32x2*)(base + 16 * D * 2);
    const floatx4 kss = *(const floatx4*)(base + 16 * D * 4 + 16 * kq);
    const floatx4 vs = *(const floatx4*)(base + 16 * D * 4 + 64 + 16 * kq);
    // S^T[token][col] over D in kKS steps of 32; the blocks' chains are
    // independent and interleave.
    floatx4 s4[CB];
#pragma unroll
    for (int cb = 0; cb < CB; ++cb) s4[cb] = floatx4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int j = 0; j < kKS; ++j) {
      const u32x4 ka = kl[(j * 4 + kq) * 16 + (tok ^ ((j * 4 + kq) & 15))];
#pragma unroll
      for (int cb = 0; cb < CB; ++cb) s4[cb] = mfma16x16x32_f16(ka, qb[cb][j], s4[cb]);
    }
    u32x4 pb[CB];
#pragma unroll
    for (int cb = 0; cb < CB; ++cb) {
      // Columns without a query row hold q = 0: their scores are finite and
      // their results are never stored.
      float sc[4];
#pragma unroll
      for (int rr = 0; rr < 4; ++rr) {
        sc[rr] = (s4[cb][rr] - qcorr[cb]) * kss[rr];
        if constexpr (MASKED) {
          if (p * 16 + 4 * kq + rr >= visible[cb]) sc[rr] = -INFINITY;
        }
      }
      const float bmax = max4_across_kq(fmaxf(fmaxf(sc[0], sc[1]), fmaxf(sc[2], sc[3])));
      // Lazy rescaling: the reference maximum moves only when a score exceeds
      // it by more than 2^8, so exp2(s - m) <= 256 stays exact in fp32 and the
      // pass over every accumulator is rare; the final division by l removes
      // the choice of reference.  Page 0 holds a visible token for every
      // column, so m_run is finite from the first page on.
      const float m_new = bmax > m_run[cb] + 8.0f ? bmax : m_run[cb];
      const bool moved = m_new != m_run[cb];
      const float corr = moved ? __builtin_amdgcn_exp2f(m_run[cb] - m_new) : 1.0f;
      m_run[cb] = m_new;
      float pw[4];
      float psum = 0.0f;
#pragma unroll
      for (int rr = 0; rr < 4; ++rr) {
        // v_exp_f32 directly: arguments are <= 8, exp2(-inf) = 0 for masked
        // tokens, and a flushed tiny probability is below the fp32
        // resolution of the running sum.
        const float e = __builtin_amdgcn_exp2f(sc[rr] - m_new);
        psum += e;
        pw[rr] = e * vs[rr];  // fold the V scale
        if constexpr (MASKED) {
          if (sc[rr] == -INFINITY) pw[rr] = 0.0f;  // whatever an unwritten slot's scale holds
        }
      }
      l_lane[cb] = l_lane[cb] * corr + psum;
      if (__builtin_amdgcn_ballot_w64(moved)) {
#pragma unroll
        for (int db = 0; db < kDB; ++db) o[cb][db] *= corr;
      }
      // P'^T as bf16 hi + lo (error ~2^-16), both in the K dimension of one
      // 16x16x32 MFMA: lane (d, kq) supplies A = V^T[d][4 kq .. 4 kq + 3]
      // twice and B = (hi, lo) of the same four tokens (the legacy 16x16x16
      // form costs as many cycles as the 16x16x32 one).
      const uint32_t h01 = pack_bf16x2(pw[0], pw[1]), h23 = pack_bf16x2(pw[2], pw[3]);
      pb[cb] = u32x4{h01, h23, pack_bf16x2(pw[0] - bf16_lo_f32(h01), pw[1] - bf16_hi_f32(h01)),
                     pack_bf16x2(pw[2] - bf16_lo_f32(h23), pw[3] - bf16_hi_f32(h23))};
    }
    // V unbiased (signed bytes -> bf16, exact): O accumulates only
    // sum_t v_t p'_t.
#pragma unroll
    for (int db = 0; db < kDB; ++db) {
      const u32x2 va = vl[(db * 4 + kq) * 16 + (tok ^ (4 * kq))];
      const u32x4 vv = {va.x, va.y, va.x, va.y};
#pragma unroll
      for (int cb = 0; cb < CB; ++cb) o[cb][db] = mfma16x16x32(vv, pb[cb], o[cb][db]);
    }
  };

  // Pipeline, one barrier per page: page p + 1's quarter (fetched a page
  // earlier) is unpacked into the other stage, page p + 2's quarter is
  // fetched, then page p is reduced from its stage.  The barrier waits on LDS
  // only, so the fetch stays in flight across it.
  Raw raw;
  if (n_pages > 0) {
    fetch(sq.pt[0], raw);
    stage_in(raw, 0);
    if (n_pages > 1) fetch(sq.pt[1], raw);
  }
  lds_barrier();
  int32_t ph_next = n_pages > 2 ? sq.pt[2] : 0;
  auto step = [&](uint32_t p, auto masked) __attribute__((always_inline)) {
    const int st = p & 1;
    if (p + 1 < n_pages) stage_in(raw, st ^ 1);
    if (p + 2 < n_pages) {
      fetch(ph_next, raw);
      if (p + 3 < n_pages) ph_next = sq.pt[p + 3];
    }
    compute(p, st, masked);
    lds_barrier();
  };
  // Pages below full_end are visible to every row of the wave.
  const uint32_t full_end = min(min(args.start + row_base + 1, sq.len) / 16, n_pages);
  for (uint32_t p = 0; p < full_end; ++p) step(p, BoolTag<false>{});
  for (uint32_t p = full_end; p < n_pages; ++p) step(p, BoolTag<true>{});

  // O^T lane layout: column col, rows d = 16 db + 4 kq + r.
#pragma unroll
  for (int cb = 0; cb < CB; ++cb) {
    float l_tot = l_lane[cb] + __shfl_xor(l_lane[cb], 16);
    l_tot += __shfl_xor(l_tot, 32);
    if (!col_ok[cb]) continue;
    const float inv = 1.0f / fmaxf(l_tot, FLT_MIN);
    const size_t obase = ((size_t)qrow[cb] * H + head) * dr;
#pragma unroll
    for (int db = 0; db < kDB; ++db)
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        const uint32_t d = 16 * db + 4 * kq + r;
        if (d >= dr) continue;
        float v = o[cb][db][r] * inv;
        if (args.gate) v *= sigmoid_f(bf16_to_f32(args.gate[obase + d]));
        args.o[obase + d] = f32_to_bf16(v);
      }
  }
}

template <int D, int CB>
hipError_t launch_prefill(const AttnArgs& a, hipStream_t st) {
  const uint32_t gh = a.heads / a.kv_heads;
  const uint32_t rows_per_wg = CB * (16 / gh) * 4;
  const uint32_t units = a.kv_heads * ((a.rows + rows_per_wg - 1) / rows_per_wg);
  hipLaunchKernelGGL((q8_prefill_kernel<D, CB>), dim3(units), dim3(256), 0, st, a);
  return hipGetLastError();
}

template <int D>
hipError_t launch_attn_d(const AttnArgs& a, uint32_t units, bool need_combine, hipStream_t st) {
  if (a.prefill) {
    // Column blocks per wave: two up to D = 128 (registers for both blocks'
    // accumulators), one above; QM38_PREFILL_CB overrides (1, 2, 4).
    int cb = a.prefill_cb > 0 ? a.prefill_cb : (D <= 128 ? 2 : 1);
    if (D > 128 && cb > 2) cb = 2;
    if (cb >= 4 && D <= 128) return launch_prefill<D, (D <= 128 ? 4 : 2)>(a, st);
    if (cb >= 2) return launch_prefill<D, 2>(a, st);
    return launch_prefill<D, 1>(a, st);
  }
  if (need_combine && !a.partials) return hipErrorInvalidValue;
  if (a.wg_waves == 8)
    hipLaunchKernelGGL((q8_decode_kernel<D, 8>), dim3(units), dim3(512), 0, st, a);
  else
    hipLaunchKernelGGL((q8_decode_kernel<D, 4>), dim3(units), dim3(256), 0, st, a);
  if (need_combine) {
    uint32_t max_split = 0;
    for (uint32_t i = 0; i < a.n_seqs; ++i) max_split = max_split > a.seqs[i].nsplit ? max_split : a.seqs[i].nsplit;
    if (max_split <= 32)
      hipLaunchKernelGGL(q8_combine_small_kernel<D>, dim3(a.n_seqs * a.heads * (D / 32)), dim3(64), 0, st, a);
    else
      hipLaunchKernelGGL(q8_combine_kernel<D>, dim3(a.n_seqs * a.heads * (D / 32)), dim3(256), 0, st, a);
  }
  return hipGetLastError();
}

}  // namespace

hipError_t launch_q8_append(const AppendArgs& a, uint32_t items, hipStream_t st) {
  if (items == 0) return hipSuccess;
  if (a.decode) {
    hipLaunchKernelGGL(q8_append_kernel, dim3(items * a.kv_heads * 2), dim3(64), 0, st, a);
  } else {
    // Rows start .. start + items - 1 of seqs[0] (whose len is start + items).
    const uint32_t pages = (a.start + items - 1) / 16 - a.start / 16 + 1;
    hipLaunchKernelGGL(q8_append_pages_kernel, dim3(pages * a.kv_heads), dim3(64 * kAppendWaves), 0, st, a);
  }
  return hipGetLastError();
}

hipError_t launch_q8_attention(const AttnArgs& a, uint32_t units, bool need_combine, hipStream_t st) {
  switch (a.head_dim_pad) {
    case 64: return launch_attn_d<64>(a, units, need_combine, st);
    case 128: return launch_attn_d<128>(a, units, need_combine, st);
    case 256: return launch_attn_d<256>(a, units, need_combine, st);
    default: return hipErrorInvalidValue;
  }
}

}  // namespace qm

// ---------------------------------------------------------------------------
// No-allocation workspace (qm_attn_decode_noalloc)
// ---------------------------------------------------------------------------
namespace qm {
namespace {

// Split partials (O, then (m, l)) of one decode call.  Every slot is written
// before it is read, so nothing needs clearing.
constexpr size_t kScratchPartialBytes = 16u << 20;
// One copy per GPU, held until the process ends.  In host code this name is
// not a device address: kernels get the address hipGetSymbolAddress returns.
static __device__ __align__(256) uint8_t scratch[kScratchPartialBytes];

constexpr int kMaxDevices = 64;
void* g_scratch_ptr[kMaxDevices];
hipError_t g_scratch_err[kMaxDevices];
std::once_flag g_scratch_once[kMaxDevices];

// Calls sharing one GPU's array are ordered: a call on another stream than
// the previous one waits for that call's completion event first.
struct ScratchOrder {
  std::mutex mu;
  hipEvent_t done = nullptr;
  hipStream_t last = nullptr;
  bool used = false;
};
ScratchOrder g_order[kMaxDevices];

}  // namespace

hipError_t attn_noalloc_scratch(int device, AttnScratch* out) {
  if (device < 0 || device >= kMaxDevices) return hipErrorInvalidDevice;
  // Once per device, with that device current (the caller holds a DeviceGuard).
  std::call_once(g_scratch_once[device], [device] {
    void* ptr = nullptr;
    g_scratch_err[device] = hipGetSymbolAddress(&ptr, HIP_SYMBOL(scratch));
    g_scratch_ptr[device] = ptr;
    if (g_scratch_err[device] == hipSuccess)
      g_scratch_err[device] = hipEventCreateWithFlags(&g_order[device].done, hipEventDisableTiming);
  });
  if (g_scratch_err[device] != hipSuccess) return g_scratch_err[device];
  out->partials = (float*)g_scratch_ptr[device];
  out->partial_bytes = kScratchPartialBytes;
  return hipSuccess;
}

hipError_t attn_noalloc_begin(int device, hipStream_t stream) {
  if (device < 0 || device >= kMaxDevices || !g_order[device].done) return hipErrorInvalidDevice;
  ScratchOrder& o = g_order[device];
  o.mu.lock();
  if (o.used && o.last != stream) {
    const hipError_t e = hipStreamWaitEvent(stream, o.done, 0);
    if (e != hipSuccess) {
      o.mu.unlock();
      return e;
    }
  }
  return hipSuccess;
}

hipError_t attn_noalloc_end(int device, hipStream_t stream) {
  ScratchOrder& o = g_order[device];
  hipError_t e = hipEventRecord(o.done, stream);
  if (e == hipSuccess) {
    o.used = true;
    o.last = stream;
  } else {
    // Without the event a later call on another stream could not wait for
    // this one: finish this call's work before releasing the array.
    (void)hipGetLastError();
    const hipError_t s = hipStreamSynchronize(stream);
    o.used = false;
    if (s != hipSuccess) e = s;
  }
  o.mu.unlock();
  return e;
}

}  // namespace qm
