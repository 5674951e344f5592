// MLX affine-Q4 decode projection for MI355X (gfx950).
//
// Computes y[m][n] = sum_g ( s[n][g] * sum_{i in g} q[n][i] x[m][i]
//                          + b[n][g] * sum_{i in g} x[m][i] )
// for M <= 16 activation rows (decode lanes), the math of
// qwen38_q4_affine_matvec_simd / qwen38_q4_affine_matmul_batch_simd
// (/root/reference/shaders/qwen38.metal:213-246, 1140).
//
// Design (HBM-bound weight stream):
//  * A workgroup owns NT tiles of 16 output rows (SwiGLU: 16 gate rows and
//    the same 16 up rows); its waves split the K groups and meet in LDS at
//    the end, so even the 5120-row down projection streams from thousands of
//    waves.
//  * Weights: each iteration covers 4 groups (128 bytes of every row).  A
//    wave's loads are coalesced 16-byte buffer loads (eight lanes read one
//    row's 128-byte line) into a ring of register sets (three with staged
//    activations, else two), so iterations stay in flight while one is
//    transposed through a per-wave XOR-swizzled LDS buffer and consumed.
//  * Activations: when all M rows fit (<= 36 KiB), each wave DMAs its K slice
//    of them into LDS, reorders it in place to the element order of the weight
//    unpack below, and every lane reads its MFMA operand from there.  The
//    start-up waits only for these DMAs and the scale/bias tables; the first
//    weight loads stay in flight.  Larger M * K keep a register path that
//    fetches each iteration's activations as it starts.
//  * Scales and biases of a wave's K slice are staged once by buffer->LDS DMA.
//  * Nibbles become bf16 (128+q) with one AND-OR per pair (exact); the dot
//    products run on MFMA 16x16x32 with the activation rows as the A operand
//    (rows >= M carry don't-care data and are never stored).  A second MFMA
//    against an all-ones B gives sum_{i in g} x[m][i].  Per group
//        acc += s * D(128+q) + (b - 128 s) * D(1)
//    which equals s*sum(q x) + b*sum(x) in real arithmetic.  Only the R =
//    min(M, 4) accumulator rows a lane can own are updated.
//  * SwiGLU mode writes bf16(silu(gate) * up) (qwen38.metal:4090-4096,
//    4188-4199).
#include "common.h"
#include "internal.h"

#include <stdio.h>
#include <stdlib.h>

#include <algorithm>
#include <cstring>
#include <mutex>

namespace qm {
namespace {

constexpr int kMaxWaves = 8;
constexpr int kGroupsPerIter = 4;  // 4 groups = 32 words = 128 bytes per row
constexpr int kTileBytes = 16 * 128;
constexpr int kNonTemporal = 2;    // buffer cache policy: nt (weights are streamed once)
constexpr uint32_t kXStageMax = 36 * 1024;  // LDS bytes of workgroup-staged activations

// Weight ring depth (iterations of register sets in flight): single-tile
// waves with staged activations have registers for four, the others two.
// Slices are planned in multiples of 4 * depth groups.
__host__ __device__ constexpr int ring_depth(int nt, bool xw) { return (xw && nt == 1) ? 4 : 2; }

struct DecodeArgs {
  const uint16_t* x;
  uint32_t K;
  uint32_t M;
  uint32_t G;        // groups per row = K / 64
  uint32_t gps;      // groups per wave slice (multiple of 4)
  uint32_t x_bytes;  // LDS bytes of one wave's staged activations (0: register path)
  uint32_t rpw;      // rows per workgroup and projection (<= 16 * tiles per projection)
  uint32_t n_jobs;
  Q4Job jobs[kMaxQ4Jobs];  // tile_begin: first tile set (workgroup) of the job
};

// DMA entries per tile of the scale/bias table (16 bytes = 8 groups, or one
// group per 4-byte LDS word).  Exact: the last DMA instruction of a table runs
// with the lanes past its end masked off, so they write no LDS.
__host__ __device__ constexpr uint32_t sb_tile_entries(bool sb16, uint32_t gps) {
  return 16 * (sb16 ? gps / 8 : gps);
}
// LDS bytes per staged activation row of one wave's K slice: the slice's
// groups (rounded up to whole iterations) plus 16 bytes, so the rows read by
// one ds_read_b128 fall on different banks.
__host__ __device__ constexpr uint32_t x_slice_pitch(uint32_t gps) { return gps * 128 + 16; }
// Per-wave LDS layout (bytes):
//   transpose buffer   NT x 2 KB: one iteration of weights in row-major form
//   scales, biases     raw bf16 per [tile][row][group] (DMA target)
//   activations        (staged mode) M rows of the wave's K slice
struct WaveLayout {
  uint32_t s_off, b_off, sb_bytes, x_off, total;
};
__host__ __device__ inline WaveLayout wave_layout(int nt, bool sb16, uint32_t gps, uint32_t x_bytes) {
  WaveLayout l{};
  l.s_off = nt * kTileBytes;
  l.sb_bytes = nt * sb_tile_entries(sb16, gps) * (sb16 ? 16 : 4);
  l.b_off = l.s_off + l.sb_bytes;
  l.x_off = l.b_off + l.sb_bytes;
  l.total = l.x_off + x_bytes;
  return l;
}

__device__ __forceinline__ __amdgpu_buffer_rsrc_t make_rsrc(const void* base, uint64_t bytes) {
  const uint32_t n = bytes > 0xFFFFFFF0ull ? 0xFFFFFFF0u : (uint32_t)bytes;
  return __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(base), (short)0, (int)n, 0x00020000);
}

// Buffer -> LDS DMA: lane i's `size` bytes land at lds + i*size (4-byte LDS
// words for sizes < 4).  The builtin exists only in the device pass; the host
// pass of single-source HIP must not see it or it drops the kernel's stub.
#if defined(__HIP_DEVICE_COMPILE__)
#define QM_LDS_PTR(p) ((__attribute__((address_space(3))) void*)(p))
__device__ __forceinline__ void dma16(__amdgpu_buffer_rsrc_t r, void* lds, uint32_t voff, uint32_t soff) {
  __builtin_amdgcn_raw_ptr_buffer_load_lds(r, QM_LDS_PTR(lds), 16, voff, soff, 0, 0);
}
__device__ __forceinline__ void dma2(__amdgpu_buffer_rsrc_t r, void* lds, uint32_t voff, uint32_t soff) {
  __builtin_amdgcn_raw_ptr_buffer_load_lds(r, QM_LDS_PTR(lds), 2, voff, soff, 0, 0);
}
#undef QM_LDS_PTR
#else
__device__ void dma16(__amdgpu_buffer_rsrc_t, void*, uint32_t, uint32_t);
__device__ void dma2(__amdgpu_buffer_rsrc_t, void*, uint32_t, uint32_t);
#endif

// s_waitcnt vmcnt(N) (gfx9 encoding; expcnt and lgkmcnt left at their maxima).
template <int N>
__device__ __forceinline__ void wait_vmcnt() {
  static_assert(N >= 0 && N < 64, "vmcnt range");
  __builtin_amdgcn_s_waitcnt(0x0F70 | (N & 0xF) | ((N >> 4) << 14));
}
__device__ __forceinline__ void wait_lgkmcnt0() { __builtin_amdgcn_s_waitcnt(0xC07F); }

__device__ __forceinline__ u32x4 unpack_word(uint32_t w, uint32_t mask_s, uint32_t or_v) {
  u32x4 r;
  r.x = (w & mask_s) | or_v;
  r.y = ((w >> 4) & mask_s) | or_v;
  r.z = ((w >> 8) & mask_s) | or_v;
  r.w = ((w >> 12) & mask_s) | or_v;
  return r;
}

template <int NT>
struct WRegs {
  u32x4 v[NT][2];
};
struct XRegs {
  u32x4 x[4][2];  // activations of one iteration (register path)
};

// NT: 16-row tiles per wave.  R: accumulator rows per lane that can be valid
// (min(M, 4)).  SB16: G % 8 == 0 and gps % 8 == 0 (scales/biases fetched 16
// bytes a lane).  XW: activations staged per workgroup in LDS.
template <int NT, int R, bool SWIGLU, bool SB16, bool XW>
__global__ __launch_bounds__(512) void q4_decode_kernel(DecodeArgs args) {
  extern __shared__ __attribute__((aligned(16))) uint8_t smem[];
  constexpr int kHalf = SWIGLU ? NT / 2 : NT;  // tiles per projection
  constexpr int kJobs = SWIGLU ? 2 : 1;

  const int lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int nwaves = blockDim.x >> 6;
  const int nl = lane & 15;
  const int kq = lane >> 4;
  const uint32_t tile = blockIdx.x;
  const uint32_t gps = args.gps;
  const WaveLayout L = wave_layout(NT, SB16, gps, XW ? args.x_bytes : 0);
  uint8_t* wl = smem + wave * L.total;
  uint8_t* tbuf = wl;
  uint8_t* s_tab = wl + L.s_off;
  uint8_t* b_tab = wl + L.b_off;
  uint8_t* xl = wl + L.x_off;  // staged activations of this wave's K slice (XW)
  const uint32_t x_pitch = x_slice_pitch(gps);

  int j = 0;
  if (!SWIGLU) {
    while (j + 1 < (int)args.n_jobs && tile >= args.jobs[j + 1].tile_begin) ++j;
  }
  const uint32_t row_base = (tile - args.jobs[j].tile_begin) * args.rpw;
  const uint32_t K = args.K;
  const uint32_t G = args.G;
  const uint32_t row_bytes = K >> 1;

  // The workgroup owns rows [row_base, row_base + n_valid) of each projection
  // (the gate and up pair share them).  Its buffer resources start at
  // row_base and end after n_valid rows, so the lanes of the remaining rows of
  // its 16-row tiles load zeros without touching memory.
  __amdgpu_buffer_rsrc_t rw[kJobs], rs[kJobs], rb[kJobs];
  uint32_t rows_j[kJobs];
  const uint32_t n_valid = min(args.rpw, args.jobs[SWIGLU ? 0 : j].rows - row_base);
#pragma unroll
  for (int q = 0; q < kJobs; ++q) {
    const Q4Job& jb = args.jobs[SWIGLU ? q : j];
    rows_j[q] = jb.rows;
    rw[q] = make_rsrc(jb.w + (size_t)row_base * (row_bytes / 4), (uint64_t)n_valid * row_bytes);
    rs[q] = make_rsrc(jb.s + (size_t)row_base * G, (uint64_t)n_valid * G * 2);
    rb[q] = make_rsrc(jb.b + (size_t)row_base * G, (uint64_t)n_valid * G * 2);
  }

  const uint32_t g_begin = wave * gps;
  const uint32_t g_end = min(G, g_begin + gps);
  const uint32_t span = g_end > g_begin ? g_end - g_begin : 0;
  const uint32_t n_iter = (span + kGroupsPerIter - 1) / kGroupsPerIter;
  constexpr int kDepth = ring_depth(NT, XW);
  // Iterations rounded up to whole ring rounds; the extra ones (only in a
  // workgroup's last, shorter slice) see zero scales and biases.
  const uint32_t n_pad = (n_iter + kDepth - 1) / kDepth * kDepth;

  floatx4 acc[NT];
#pragma unroll
  for (int t = 0; t < NT; ++t) acc[t] = floatx4{0.f, 0.f, 0.f, 0.f};

  // Weights: lane -> row 8h + lane/8, 16-byte chunk lane%8 of the row's
  // 128-byte line (coalesced); written to the transpose buffer at slot
  // chunk ^ row%8 (XOR swizzle against LDS bank conflicts on the reads).
  const int lrow = lane >> 3;
  const int lchunk = lane & 7;
  uint32_t vw[NT][2];
  uint32_t row_of[NT];
#pragma unroll
  for (int t = 0; t < NT; ++t) {
    const uint32_t base = 16u * (t % kHalf);  // local to the workgroup's rows
    row_of[t] = base + nl;
#pragma unroll
    for (int h = 0; h < 2; ++h) vw[t][h] = (base + 8 * h + lrow) * row_bytes + 16 * lchunk;
  }
  const uint32_t wst = lrow * 128 + 16 * (lchunk ^ (lrow & 7));  // transpose-buffer store offset

  // Activation row this lane reads as MFMA A operand (rows >= M reuse row 0).
  const uint32_t am = (uint32_t)nl < args.M ? nl : 0;
  const uint16_t* xrow_g = args.x + (size_t)am * K + 16 * kq;

  auto load_w = [&](uint32_t it, WRegs<NT>& r) __attribute__((always_inline)) {
    const uint32_t g = g_begin + it * kGroupsPerIter;
#pragma unroll
    for (int t = 0; t < NT; ++t)
#pragma unroll
      for (int h = 0; h < 2; ++h)
        r.v[t][h] = __builtin_amdgcn_raw_buffer_load_b128(rw[SWIGLU ? t / kHalf : 0], vw[t][h], g * 32,
                                                          kNonTemporal);
  };
  // Register path: an iteration's activations, fetched one iteration ahead.
  auto load_x = [&](uint32_t it, XRegs& r) __attribute__((always_inline)) {
    if (XW) return;
    const uint32_t g = g_begin + it * kGroupsPerIter;
#pragma unroll
    for (int u = 0; u < 4; ++u) {
      const uint32_t gx = min(g + u, G - 1);
      r.x[u][0] = *(const u32x4*)(xrow_g + (size_t)gx * 64);
      r.x[u][1] = *(const u32x4*)(xrow_g + (size_t)gx * 64 + 8);
    }
  };

  WRegs<NT> wr[kDepth];
  XRegs xp;
  const uint32_t pad = sb_tile_entries(SB16, gps);
  // --- one-time staging: scales and biases, first weights, activations --------
  const uint32_t x_chunks = span * 8;  // 16-byte activation chunks per row of the slice
  {
    const uint32_t cols = SB16 ? gps / 8 : gps;  // DMA entries per row
    const uint32_t per_tile = 16 * cols;
    if (n_iter > 0) {
      if (XW) {
        // The wave's K slice of all M activation rows, by buffer->LDS DMA in
        // natural order (reordered in place once it has landed).
        const __amdgpu_buffer_rsrc_t rx = make_rsrc(args.x, (uint64_t)args.M * K * 2);
        for (uint32_t m = 0; m < args.M; ++m)
          for (uint32_t c0 = 0; c0 < x_chunks; c0 += 64)
            if (c0 + lane < x_chunks)
              dma16(rx, xl + m * x_pitch + c0 * 16, (m * K + g_begin * 64) * 2 + (c0 + lane) * 16, 0);
      }
#pragma unroll
      for (int t = 0; t < NT; ++t) {
        const int q = SWIGLU ? t / kHalf : 0;
        for (uint32_t i = 0; i < (per_tile + 63) / 64; ++i) {
          const uint32_t e = i * 64 + lane;
          if (e >= per_tile) continue;
          const uint32_t row = e / cols;
          const uint32_t col = e - row * cols;
          const uint32_t rc = 16u * (t % kHalf) + row;  // local row; past n_valid loads zeros
          if (SB16) {
            const uint32_t off = (rc * G + g_begin + col * 8) * 2;
            dma16(rs[q], s_tab + (t * pad + i * 64) * 16, off, 0);
            dma16(rb[q], b_tab + (t * pad + i * 64) * 16, off, 0);
          } else {
            const uint32_t off = (rc * G + g_begin + col) * 2;
            dma2(rs[q], s_tab + (t * pad + i * 64) * 4, off, 0);
            dma2(rb[q], b_tab + (t * pad + i * 64) * 4, off, 0);
          }
        }
      }
      // The first iterations' weights stream while everything else lands
      // (three with staged activations, two on the register path).
      // Every ring slot is filled (short slices repeat their last iteration)
      // so all paths below see the same outstanding loads and the compiler's
      // waits stay exact.
#pragma unroll
      for (int d = 0; d < kDepth; ++d) {
        load_w(min((uint32_t)d, n_iter - 1), wr[d]);
        __builtin_amdgcn_sched_barrier(0);  // keep the slots in issue order
      }
      load_x(0, xp);
      // Wait for the DMAs (activations, tables) only: the weight loads issued
      // after them stay in flight.
      if constexpr (!XW) {
        static_assert(kDepth == 2, "register path waits for two weight sets");
        wait_vmcnt<2 * (2 * NT) + 8>();
      } else {
        wait_vmcnt<kDepth * (2 * NT)>();
      }
      // Groups past the slice end get scale = bias = 0 (they contribute 0).
      if (span < n_pad * kGroupsPerIter) {
        const uint32_t dead = n_pad * kGroupsPerIter - span;
        for (uint32_t e = lane; e < NT * 16 * dead; e += 64) {
          const uint32_t t = e / (16 * dead), row = (e / dead) % 16, gl = span + e % dead;
          if (SB16) {
            ((uint16_t*)s_tab)[t * pad * 8 + row * gps + gl] = 0;
            ((uint16_t*)b_tab)[t * pad * 8 + row * gps + gl] = 0;
          } else {
            ((uint32_t*)s_tab)[t * pad + row * gps + gl] = 0;
            ((uint32_t*)b_tab)[t * pad + row * gps + gl] = 0;
          }
        }
      }
      if (XW) {
        // Each 8-element chunk reordered (x0,x4)(x1,x5)(x2,x6)(x3,x7) to match
        // unpack_word.
        for (uint32_t e = lane; e < args.M * x_chunks; e += 64) {
          const uint32_t m = e / x_chunks, c = e - m * x_chunks;
          u32x4* px = (u32x4*)(xl + m * x_pitch + c * 16);
          *px = interleave_bf16x8(*px);
        }
      }
    }
    wait_lgkmcnt0();
    __builtin_amdgcn_sched_barrier(0);
  }

  const u32x4 ones = {0x3F803F80u, 0x3F803F80u, 0x3F803F80u, 0x3F803F80u};
  const uint32_t mask_s = __builtin_amdgcn_readfirstlane(0x000F000Fu);
  uint32_t or_v = 0x43004300u;
  asm volatile("" : "+v"(or_v));
  const uint8_t* xlr = xl + am * x_pitch + 32 * kq;  // this lane's staged row, chunk pair 2kq

  auto consume = [&](uint32_t it, const WRegs<NT>& r, const XRegs& xr) __attribute__((always_inline)) {
    const uint32_t gl = it * kGroupsPerIter;  // group offset inside the slice
    // Scales / biases of the 4 groups (bf16 -> fp32 by shifting).
    uint32_t sv[NT][4], bv[NT][4];
#pragma unroll
    for (int t = 0; t < NT; ++t) {
      if (SB16) {
        const uint32_t e = t * pad * 8 + nl * gps + gl;
        const u32x2 s2 = *(const u32x2*)(s_tab + e * 2);
        const u32x2 b2 = *(const u32x2*)(b_tab + e * 2);
        sv[t][0] = s2.x << 16; sv[t][1] = s2.x & 0xFFFF0000u; sv[t][2] = s2.y << 16; sv[t][3] = s2.y & 0xFFFF0000u;
        bv[t][0] = b2.x << 16; bv[t][1] = b2.x & 0xFFFF0000u; bv[t][2] = b2.y << 16; bv[t][3] = b2.y & 0xFFFF0000u;
      } else {
        const uint32_t e = t * pad + nl * gps + gl;
        const u32x4 s4 = *(const u32x4*)(s_tab + e * 4);
        const u32x4 b4 = *(const u32x4*)(b_tab + e * 4);
        sv[t][0] = s4.x << 16; sv[t][1] = s4.y << 16; sv[t][2] = s4.z << 16; sv[t][3] = s4.w << 16;
        bv[t][0] = b4.x << 16; bv[t][1] = b4.y << 16; bv[t][2] = b4.z << 16; bv[t][3] = b4.w << 16;
      }
    }
    // Row-major weights -> transpose buffer.
#pragma unroll
    for (int t = 0; t < NT; ++t)
#pragma unroll
      for (int h = 0; h < 2; ++h) *(u32x4*)(tbuf + t * kTileBytes + h * 1024 + wst) = r.v[t][h];
    __builtin_amdgcn_wave_barrier();
#pragma unroll
    for (int u = 0; u < 4; ++u) {
      u32x4 xa0, xa1;
      if (XW) {
        // Groups past the slice (dead iterations) read its last group: finite
        // data, zero scale and bias.
        const uint8_t* p = xlr + min(gl + u, span - 1) * 128;
        xa0 = *(const u32x4*)p;
        xa1 = *(const u32x4*)(p + 16);
      } else {
        xa0 = interleave_bf16x8(xr.x[u][0]);
        xa1 = interleave_bf16x8(xr.x[u][1]);
      }
      floatx4 dsum = mfma16x16x32(xa0, ones, floatx4{0.f, 0.f, 0.f, 0.f});
      dsum = mfma16x16x32(xa1, ones, dsum);
#pragma unroll
      for (int t = 0; t < NT; ++t) {
        const uint32_t chunk = 2 * u + (kq >> 1);
        const u32x2 wv =
            *(const u32x2*)(tbuf + t * kTileBytes + nl * 128 + 16 * (chunk ^ (nl & 7)) + 8 * (kq & 1));
        floatx4 dq = mfma16x16x32(xa0, unpack_word(wv.x, mask_s, or_v), floatx4{0.f, 0.f, 0.f, 0.f});
        dq = mfma16x16x32(xa1, unpack_word(wv.y, mask_s, or_v), dq);
        const float s = __uint_as_float(sv[t][u]);
        const float c = fmaf(-128.0f, s, __uint_as_float(bv[t][u]));
#pragma unroll
        for (int rr = 0; rr < R; ++rr) acc[t][rr] = fmaf(c, dsum[rr], fmaf(s, dq[rr], acc[t][rr]));
      }
    }
    __builtin_amdgcn_wave_barrier();
  };

  // Whole ring rounds: each iteration consumes its slot and refills it
  // kDepth iterations ahead, unconditionally (dead iterations reload the
  // last real one), so every path carries the same outstanding loads and the
  // compiler's waits stay exact; the final round drains the ring.  The
  // register path (larger M * K) fetches an iteration's activations as it
  // starts.
  auto step = [&](uint32_t i, WRegs<NT>& w, bool refill) __attribute__((always_inline)) {
    if (!XW && i > 0) load_x(min(i, n_iter - 1), xp);
    consume(i, w, xp);
    if (refill) {
      __builtin_amdgcn_sched_barrier(0);
      load_w(min(i + kDepth, n_iter - 1), w);
      __builtin_amdgcn_sched_barrier(0);  // refills stay in slot order
    }
  };
  if (n_iter > 0) {
    uint32_t it = 0;
    for (; it + kDepth < n_pad; it += kDepth) {
#pragma unroll
      for (int d = 0; d < kDepth; ++d) step(it + d, wr[d], true);
    }
#pragma unroll
    for (int d = 0; d < kDepth; ++d) step(it + d, wr[d], false);
  }

  if (nwaves > 1) {
    __syncthreads();  // all waves are done with their LDS
    float* red = (float*)smem;
#pragma unroll
    for (int t = 0; t < NT; ++t)
#pragma unroll
      for (int rr = 0; rr < R; ++rr) red[((wave * NT + t) * 4 + rr) * 64 + lane] = acc[t][rr];
    __syncthreads();
    if (wave != 0) return;
#pragma unroll
    for (int t = 0; t < NT; ++t)
#pragma unroll
      for (int rr = 0; rr < R; ++rr) {
        float v = red[(t * 4 + rr) * 64 + lane];
        for (int w = 1; w < nwaves; ++w) v += red[((w * NT + t) * 4 + rr) * 64 + lane];
        acc[t][rr] = v;
      }
  }

  if (!SWIGLU && args.jobs[j].mode == kQ4OutArgmax) {
    // Greedy token per activation row (qwen38_argmax_rows, qwen38.metal:
    // 4202-4244): the largest fp32 value, the lowest row index on ties, NaN
    // never winning.  Key = (order-preserving bits of the value) << 32 |
    // ~row, so one unsigned 64-bit maximum picks both; -0 counts as +0 (the
    // reference compares values, and -0 == +0).  The tile's 16 lanes of a row
    // group reduce, then one atomic per row and workgroup.
    unsigned long long* keys = (unsigned long long*)args.jobs[j].out;
#pragma unroll
    for (int rr = 0; rr < R; ++rr) {
      unsigned long long best = 0;
#pragma unroll
      for (int t = 0; t < NT; ++t) {
        const float v = acc[t][rr];
        if (row_of[t] < n_valid && !__builtin_isnan(v)) {
          const uint32_t b = v == 0.0f ? 0u : __float_as_uint(v);
          const uint32_t ord = (b & 0x80000000u) ? ~b : (b | 0x80000000u);
          const unsigned long long key =
              ((unsigned long long)ord << 32) | (0xFFFFFFFFu - (row_base + row_of[t]));
          best = key > best ? key : best;
        }
      }
#pragma unroll
      for (int off = 8; off >= 1; off >>= 1) {
        const unsigned long long o = __shfl_xor(best, off);
        best = o > best ? o : best;
      }
      const uint32_t m = 4 * kq + rr;
      if (nl == 0 && m < args.M && best != 0) atomicMax(keys + m, best);
    }
    return;
  }

#pragma unroll
  for (int rr = 0; rr < R; ++rr) {
    const uint32_t m = 4 * kq + rr;
    if (m >= args.M) continue;
    if (SWIGLU) {
#pragma unroll
      for (int t = 0; t < kHalf; ++t)
        if (row_of[t] < n_valid) {
          const float h = silu_f(acc[t][rr]) * acc[t + kHalf][rr];
          args.jobs[0].out[(size_t)m * rows_j[0] + row_base + row_of[t]] = f32_to_bf16(h);
        }
    } else {
      const uint32_t mode = args.jobs[j].mode;
#pragma unroll
      for (int t = 0; t < NT; ++t)
        if (row_of[t] < n_valid) {
          const size_t idx = (size_t)m * rows_j[0] + row_base + row_of[t];
          const uint16_t v = f32_to_bf16(acc[t][rr]);
          if (mode == kQ4OutBf16)
            args.jobs[j].out[idx] = v;
          else if (mode == kQ4OutF32)
            ((float*)args.jobs[j].out)[idx] = bf16_to_f32(v);
          else
            ((float*)args.jobs[j].out)[idx] += bf16_to_f32(v);
        }
    }
  }
}


// Kernel instance for the template parameters a plan selects.
template <int NT, int R, bool SW>
const void* instance_of(bool sb16, bool xw) {
  if (xw) return sb16 ? (const void*)q4_decode_kernel<NT, R, SW, true, true>
                      : (const void*)q4_decode_kernel<NT, R, SW, false, true>;
  return sb16 ? (const void*)q4_decode_kernel<NT, R, SW, true, false>
              : (const void*)q4_decode_kernel<NT, R, SW, false, false>;
}
template <int NT, bool SW>
const void* instance_m(uint32_t M, bool sb16, bool xw) {
  if (M == 1) return instance_of<NT, 1, SW>(sb16, xw);
  if (M == 2) return instance_of<NT, 2, SW>(sb16, xw);
  return instance_of<NT, 4, SW>(sb16, xw);
}

struct Plan {
  const void* fn;
  int nt;
  uint32_t tiles, waves, gps, lds, x_bytes, rpw;
};

// Work decomposition.  A workgroup owns `rpw` rows of each projection (at most
// its 16-row tiles: 16 * NT, or a gate/up pair of 16 in SwiGLU mode); its
// waves split K.
//  * HBM throughput is set by the bytes in flight, so the K split aims at
//    about `target` resident waves.
//  * All workgroups should be resident at once: a second dispatch round
//    starts only when the first drains.  The wave count is lowered until the
//    occupancy query says they fit.
//  * The busiest CU sets the time.  With whole 16-row tiles, tile counts just
//    above a multiple of the CU count leave some CUs one workgroup more than
//    others (320 tiles on 256 CUs: a quarter of the CUs carry twice the rows).
//    Fewer rows per workgroup can spread the rows more evenly; the masked rows
//    of a tile cost arithmetic on zeros but no memory traffic.  Each candidate
//    is scored by the rows on the busiest CU, with rounds past the first
//    weighted by a quarter.
Plan make_plan(const Q4Job* jobs, int n_jobs, bool swiglu, uint32_t K, uint32_t M, const Tuning& tn) {
  Plan best{};
  const uint32_t G = K / 64;
  uint64_t rows = 0;
  for (int i = 0; i < n_jobs; ++i) rows += jobs[i].rows;
  const uint32_t cus = tn.cus > 0 ? (uint32_t)tn.cus : 256;
  int nt = swiglu ? 2 : ((rows / 32 >= (uint64_t)cus * 2) ? 2 : 1);
  if (!swiglu && tn.q4_nt > 0) nt = tn.q4_nt >= 2 ? 2 : 1;
  // Staged activations for one row when it fits (each wave holds its K
  // slice); several rows take the register path, whatever their size (two
  // or three 5120-wide rows fit the staging buffer but ran the QKV + gate/up
  // set in 61-64 us staged against 40 us for four rows on registers).
  const uint32_t x_max = tn.q4_xstage_max > 0 ? (uint32_t)tn.q4_xstage_max : kXStageMax;
  const bool xw = (M == 1 || tn.q4_xstage_max > 0) && M * (K * 2 + 16) <= x_max && tn.q4_xstage != 0;
  const bool g8 = (G % 8) == 0;
  const void* fn = swiglu ? instance_m<2, true>(M, g8, xw)
                          : (nt == 2 ? instance_m<2, false>(M, g8, xw) : instance_m<1, false>(M, g8, xw));
  const uint32_t step = 4 * ring_depth(nt, xw);  // whole ring rounds per slice (also a multiple of 8)
  const uint32_t lds_cu = 160 * 1024;
  const uint32_t target = tn.q4_target_waves > 0 ? (uint32_t)tn.q4_target_waves : cus * 16;
  const uint32_t r_max = 16u * (swiglu ? 1u : (uint32_t)nt);
  // Masked rows still cost arithmetic and activation staging: measured on the
  // BASELINE shapes, workgroups below 13/16 of their tiles lose more than the
  // balance gains.
  uint32_t r_hi = r_max, r_lo = (13 * r_max + 15) / 16;
  if (tn.q4_rpw > 0) r_hi = r_lo = std::min<uint32_t>(r_max, (uint32_t)tn.q4_rpw);
  double best_cost = 0.0;
  for (uint32_t r = r_hi; r >= r_lo && r > 0; --r) {
    Plan p{};
    p.fn = fn;
    p.nt = nt;
    p.rpw = r;
    for (int i = 0; i < (swiglu ? 1 : n_jobs); ++i) p.tiles += (jobs[i].rows + r - 1) / r;
    uint32_t waves = (target + p.tiles - 1) / p.tiles;
    // With several activation rows a ring slot costs several times the
    // arithmetic (per-row FMAs, more registers): at most 4 waves per tile, so
    // each wave's longer slice overlaps its own loads with that work over
    // several ring rounds (measured: M = 4 / 8 sets +7 % / +9 %; slower at M = 1).
    if (M > 1) waves = std::min<uint32_t>(waves, 4);
    if (tn.q4_split > 0) waves = (uint32_t)tn.q4_split;
    waves = std::max<uint32_t>(1, std::min<uint32_t>(waves, kMaxWaves));
    int occ = 0;
    for (;;) {
      uint32_t gps = (G + waves - 1) / waves;
      gps = (gps + step - 1) / step * step;
      const uint32_t w = (G + gps - 1) / gps;
      p.gps = gps;
      p.waves = w;
      p.x_bytes = xw ? M * x_slice_pitch(gps) : 0;
      p.lds = w * wave_layout(nt, g8, gps, p.x_bytes).total;
      // The final cross-wave reduction reuses the LDS from offset 0.
      p.lds = std::max<uint32_t>(p.lds, w * nt * 4 * 64 * 4);
      occ = 0;
      if (p.lds <= lds_cu &&
          hipOccupancyMaxActiveBlocksPerMultiprocessor(&occ, fn, (int)(64 * w), p.lds) != hipSuccess)
        occ = 0;
      if (w == 1 || (occ > 0 && p.tiles <= (uint32_t)occ * cus)) break;
      waves = w - 1;  // fewer, longer slices: less LDS per workgroup, fewer waves
    }
    if (occ <= 0) continue;
    const uint32_t rounds = (p.tiles + (uint32_t)occ * cus - 1) / ((uint32_t)occ * cus);
    const double cost = (double)((p.tiles + cus - 1) / cus) * r * (1.0 + 0.25 * (rounds - 1));
    if (!best.fn || cost < best_cost) {
      best = p;
      best_cost = cost;
    }
  }
  return best;
}

// Plans depend only on the shapes (and the tuning environment), so the last
// few are kept: a decode loop calls with the same shapes every token.
struct PlanKey {
  uint32_t rows[kMaxQ4Jobs];
  int n_jobs;
  bool swiglu;
  uint32_t K, M;
  Tuning tune;
  bool operator==(const PlanKey& o) const {
    return n_jobs == o.n_jobs && swiglu == o.swiglu && K == o.K && M == o.M &&
           std::memcmp(rows, o.rows, sizeof(rows)) == 0 && std::memcmp(&tune, &o.tune, sizeof(tune)) == 0;
  }
};
Plan cached_plan(const Q4Job* jobs, int n_jobs, bool swiglu, uint32_t K, uint32_t M, const Tuning& tn) {
  static std::mutex mu;
  static PlanKey keys[8];
  static Plan plans[8];
  static int used = 0, next = 0;
  PlanKey k{};
  for (int i = 0; i < n_jobs; ++i) k.rows[i] = jobs[i].rows;
  k.n_jobs = n_jobs;
  k.swiglu = swiglu;
  k.K = K;
  k.M = M;
  k.tune = tn;
  std::lock_guard<std::mutex> lock(mu);
  for (int i = 0; i < used; ++i)
    if (keys[i] == k) return plans[i];
  const Plan p = make_plan(jobs, n_jobs, swiglu, K, M, tn);
  if (tn.q4_plan_log > 0)
    fprintf(stderr, "q4 decode plan: K=%u M=%u swiglu=%d rows0=%u -> nt=%d rpw=%u tiles=%u waves=%u gps=%u lds=%u\n", K,
            M, (int)swiglu, jobs[0].rows, p.nt, p.rpw, p.tiles, p.waves, p.gps, p.lds);
  if (p.fn) {
    keys[next] = k;
    plans[next] = p;
    next = (next + 1) % 8;
    used = std::min(used + 1, 8);
  }
  return p;
}

// ids[m] = the row index an argmax key holds (0 for a row whose logits were
// all NaN: no key was stored); the keys return to zero for the next call.
__global__ void q4_argmax_finish_kernel(unsigned long long* keys, uint32_t* ids, uint32_t M) {
  const uint32_t m = blockIdx.x * blockDim.x + threadIdx.x;
  if (m >= M) return;
  const unsigned long long k = keys[m];
  ids[m] = k ? 0xFFFFFFFFu - (uint32_t)(k & 0xFFFFFFFFull) : 0u;
  keys[m] = 0;
}

}  // namespace

hipError_t launch_q4_argmax_finish(unsigned long long* keys, uint32_t* ids, uint32_t M, hipStream_t stream) {
  hipLaunchKernelGGL(q4_argmax_finish_kernel, dim3((M + 63) / 64), dim3(64), 0, stream, keys, ids, M);
  return hipGetLastError();
}

hipError_t launch_q4_decode(const Q4Job* jobs, int n_jobs, bool swiglu, const uint16_t* x,
                            uint32_t K, uint32_t M, const Workspace& ws, hipStream_t stream) {
  if (!ws.tune) return hipErrorInvalidValue;
  const Plan p = cached_plan(jobs, n_jobs, swiglu, K, M, *ws.tune);
  if (!p.fn || p.lds > 160 * 1024) return hipErrorInvalidValue;
  DecodeArgs a{};
  a.x = x;
  a.K = K;
  a.M = M;
  a.G = K / 64;
  a.gps = p.gps;
  a.x_bytes = p.x_bytes;
  a.rpw = p.rpw;
  a.n_jobs = (uint32_t)n_jobs;
  uint32_t ts = 0;
  for (int i = 0; i < n_jobs; ++i) {
    a.jobs[i] = jobs[i];
    a.jobs[i].tile_begin = ts;
    if (!swiglu) ts += (jobs[i].rows + p.rpw - 1) / p.rpw;
  }
  void* args[] = {&a};
  const hipError_t e = hipLaunchKernel(p.fn, dim3(p.tiles), dim3(64 * p.waves), args, p.lds, stream);
  return e != hipSuccess ? e : hipGetLastError();
}

}  // namespace qm
