// MLX affine-Q4 decode projection for MI355X (gfx950).
//
// Computes y[m][n] = sum_g ( s[n][g] * sum_{i in g} q[n][i] x[m][i]
//                          + b[n][g] * sum_{i in g} x[m][i] )
// for M <= 16 activation rows (decode lanes), the math of
// qwen38_q4_affine_matvec_simd / qwen38_q4_affine_matmul_batch_simd
// (/root/reference/shaders/qwen38.metal:213-246, 1140).
//
// Design (HBM-bound weight stream):
//  * A wave owns NT tiles of 16 output rows and a slice of the K groups; the
//    waves of one workgroup split K and are reduced through LDS, so every
//    launch has thousands of waves streaming weights even for the 5120-row
//    down projection.
//  * Everything an iteration (4 groups = 128 bytes of every row) needs is
//    copied straight from HBM into a per-wave LDS slot with buffer->LDS DMA
//    loads: weights (eight consecutive lanes read one row's 128-byte line),
//    activations and scales/biases.  Three slots rotate, so two iterations
//    are always in flight while the third is consumed, without holding the
//    prefetched data in VGPRs.  Buffer range checks turn any read past a
//    tensor into zeros.
//  * Nibbles become bf16 (128+q) with one AND-OR per pair (exact); the dot
//    products run on MFMA 16x16x32 with the activation rows as the A operand
//    (rows >= M carry don't-care data and are never stored).  A second MFMA
//    against an all-ones B gives sum_{i in g} x[m][i].  Per group
//        acc += s * D(128+q) + (b - 128 s) * D(1)
//    which equals s*sum(q x) + b*sum(x) in real arithmetic.  Only the R =
//    min(M, 4) accumulator rows a lane can own are updated.
//  * SwiGLU mode pairs gate tiles with the same rows of the up projection in
//    one wave and writes bf16(silu(gate) * up) (qwen38.metal:4090-4096,
//    4188-4199).
#include "common.h"
#include "internal.h"

#include <stdlib.h>

namespace qm {
namespace {

constexpr int kMaxWaves = 8;
constexpr int kGroupsPerIter = 4;  // 4 groups = 32 words = 128 bytes per row
constexpr int kTileBytes = 16 * 128;
constexpr int kNonTemporal = 2;    // buffer cache policy: nt (weights are streamed once)

struct DecodeArgs {
  const uint16_t* x;
  uint32_t K;
  uint32_t M;
  uint32_t G;    // groups per row = K / 64
  uint32_t gps;  // groups per wave slice (multiple of 4)
  uint32_t n_jobs;
  Q4Job jobs[kMaxQ4Jobs];  // tile_begin: first tile set (workgroup) of the job
};

// DMA entries per tile of the scale/bias table (16 bytes = 8 groups, or one
// group per 4-byte LDS word), padded to whole 64-lane instructions.
__host__ __device__ constexpr uint32_t sb_tile_entries(bool sb16, uint32_t gps) {
  return ((16 * (sb16 ? gps / 8 : gps) + 63) / 64) * 64;
}
// Per-wave LDS layout (bytes):
//   transpose buffer   NT x 2 KB: one iteration of weights in row-major form
//   x slice (XS only)  [gps/4 blocks][XR rows][512 B], interleaved in place
//   scales, biases     raw bf16 per [tile][row][group] (DMA target)
struct WaveLayout {
  uint32_t x_off, s_off, b_off, sb_bytes, total;
};
__host__ __device__ inline WaveLayout wave_layout(int nt, int xr, bool sb16, uint32_t gps, bool xs) {
  WaveLayout l{};
  l.x_off = nt * kTileBytes;
  l.s_off = l.x_off + (xs ? (gps / 4) * xr * 512 : 0);
  l.sb_bytes = nt * sb_tile_entries(sb16, gps) * (sb16 ? 16 : 4);
  l.b_off = l.s_off + l.sb_bytes;
  l.total = l.b_off + l.sb_bytes;
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

__device__ __forceinline__ void wait_vmcnt0() { __builtin_amdgcn_s_waitcnt(0x0F70); }
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

// NT: 16-row tiles per wave.  XR: activation rows staged (>= M, even).
// R: accumulator rows per lane that can be valid (min(M, 4)).
// SB16: G % 8 == 0 and gps % 8 == 0 (scales/biases fetched 16 bytes a lane).
// XS: the wave's whole activation slice is staged (and interleaved) once in
// LDS; otherwise each iteration loads its activations into registers.
template <int NT, int XR, int R, bool SWIGLU, bool SB16, bool XS>
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
  const WaveLayout L = wave_layout(NT, XR, SB16, gps, XS);
  uint8_t* wl = smem + wave * L.total;
  uint8_t* tbuf = wl;
  uint8_t* xl = wl + L.x_off;
  uint8_t* s_tab = wl + L.s_off;
  uint8_t* b_tab = wl + L.b_off;

  int j = 0;
  if (!SWIGLU) {
    while (j + 1 < (int)args.n_jobs && tile >= args.jobs[j + 1].tile_begin) ++j;
  }
  const uint32_t row_base = (tile - args.jobs[j].tile_begin) * 16u * kHalf;
  const uint32_t K = args.K;
  const uint32_t G = args.G;
  const uint32_t row_bytes = K >> 1;

  __amdgpu_buffer_rsrc_t rw[kJobs], rs[kJobs], rb[kJobs];
  uint32_t rows_j[kJobs];
#pragma unroll
  for (int q = 0; q < kJobs; ++q) {
    const Q4Job& jb = args.jobs[SWIGLU ? q : j];
    rows_j[q] = jb.rows;
    rw[q] = make_rsrc(jb.w, (uint64_t)jb.rows * row_bytes);
    rs[q] = make_rsrc(jb.s, (uint64_t)jb.rows * G * 2);
    rb[q] = make_rsrc(jb.b, (uint64_t)jb.rows * G * 2);
  }
  const __amdgpu_buffer_rsrc_t rx = make_rsrc(args.x, (uint64_t)args.M * K * 2);

  const uint32_t g_begin = wave * gps;
  const uint32_t g_end = min(G, g_begin + gps);
  const uint32_t span = g_end > g_begin ? g_end - g_begin : 0;
  const uint32_t n_iter = (span + kGroupsPerIter - 1) / kGroupsPerIter;

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
    const int q = SWIGLU ? t / kHalf : 0;
    const uint32_t base = row_base + 16u * (t % kHalf);
    row_of[t] = base + nl;
#pragma unroll
    for (int h = 0; h < 2; ++h) {
      const uint32_t r = base + 8 * h + lrow;
      const uint32_t rc = r < rows_j[q] ? r : rows_j[q] - 1;
      vw[t][h] = rc * row_bytes + 16 * lchunk;
    }
  }
  const uint32_t wst = lrow * 128 + 16 * (lchunk ^ (lrow & 7));  // transpose-buffer store offset

  auto load_w = [&](uint32_t it, WRegs<NT>& r) {
    const uint32_t g = g_begin + it * kGroupsPerIter;
#pragma unroll
    for (int t = 0; t < NT; ++t)
#pragma unroll
      for (int h = 0; h < 2; ++h)
        r.v[t][h] = __builtin_amdgcn_raw_buffer_load_b128(rw[SWIGLU ? t / kHalf : 0], vw[t][h], g * 32,
                                                          kNonTemporal);
  };

  // Activation DMA into the staged slice: instruction covers rows 2i, 2i+1 of
  // 4 groups; lane -> row 2i + lane/32, LDS slot lane%32 holding chunk slot ^
  // (row%8).  Rows >= M read past the buffer and land as zeros.
  auto stage_x = [&](uint8_t* dst, uint32_t g) {
#pragma unroll
    for (int i = 0; i < XR / 2; ++i) {
      const uint32_t m = 2 * i + (lane >> 5);
      const uint32_t off = m * K * 2 + ((lane & 31) ^ (m & 7)) * 16;
      dma16(rx, dst + 2 * i * 512, off, g * 128);
    }
  };

  WRegs<NT> wa, wb;
  if (n_iter > 0) {
    // --- one-time staging: activation slice, scales and biases -------------
    if (XS)
      for (uint32_t b = 0; b < n_iter; ++b) stage_x(xl + b * XR * 512, g_begin + b * kGroupsPerIter);
    {
      const uint32_t cols = SB16 ? gps / 8 : gps;  // DMA entries per row
      const uint32_t per_tile = 16 * cols;
      const uint32_t pad = sb_tile_entries(SB16, gps);
#pragma unroll
      for (int t = 0; t < NT; ++t) {
        const int q = SWIGLU ? t / kHalf : 0;
        for (uint32_t i = 0; i < pad / 64; ++i) {
          uint32_t e = i * 64 + lane;
          e = e < per_tile ? e : per_tile - 1;
          const uint32_t row = e / cols;
          const uint32_t col = e - row * cols;
          const uint32_t r = row_base + 16u * (t % kHalf) + row;
          const uint32_t rc = r < rows_j[q] ? r : rows_j[q] - 1;
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
    }
    wait_vmcnt0();
    load_w(0, wa);  // first weights stream while the tables are fixed up
    // Interleave the x slice in place: (x0..x7) -> (x0,x4)(x1,x5)(x2,x6)(x3,x7).
    if (XS)
      for (uint32_t c = lane; c < n_iter * XR * 32; c += 64) {
        u32x4* p = (u32x4*)(xl + c * 16);
        *p = interleave_bf16x8(*p);
      }
    // Groups past the slice end get scale = bias = 0 (they contribute 0).
    if (span % kGroupsPerIter) {
      const uint32_t dead = kGroupsPerIter - span % kGroupsPerIter;
      const uint32_t pad = sb_tile_entries(SB16, gps);
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
    wait_lgkmcnt0();
    __builtin_amdgcn_sched_barrier(0);
  }

  const u32x4 ones = {0x3F803F80u, 0x3F803F80u, 0x3F803F80u, 0x3F803F80u};
  const uint32_t mask_s = __builtin_amdgcn_readfirstlane(0x000F000Fu);
  uint32_t or_v = 0x43004300u;
  asm volatile("" : "+v"(or_v));
  // Activation row this lane reads as MFMA A operand (rows >= M reuse row 0).
  const uint32_t am = (uint32_t)nl < args.M ? nl : 0;
  const uint32_t pad = sb_tile_entries(SB16, gps);
  const uint16_t* xrow_g = args.x + (size_t)am * K + 16 * kq;

  auto consume = [&](uint32_t it, const WRegs<NT>& r) {
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
    u32x4 xg[4][2];
    if (!XS) {
      const uint32_t g = g_begin + gl;
#pragma unroll
      for (int u = 0; u < 4; ++u) {
        const uint32_t gx = min(g + u, G - 1);
        xg[u][0] = *(const u32x4*)(xrow_g + (size_t)gx * 64);
        xg[u][1] = *(const u32x4*)(xrow_g + (size_t)gx * 64 + 8);
      }
    }
    // Row-major weights -> transpose buffer.
#pragma unroll
    for (int t = 0; t < NT; ++t)
#pragma unroll
      for (int h = 0; h < 2; ++h) *(u32x4*)(tbuf + t * kTileBytes + h * 1024 + wst) = r.v[t][h];
    __builtin_amdgcn_wave_barrier();
    const uint8_t* xs = xl + (it * XR + am) * 512;
#pragma unroll
    for (int u = 0; u < 4; ++u) {
      u32x4 xa0, xa1;
      if (XS) {
        xa0 = *(const u32x4*)(xs + 16 * (((4 * u + kq) * 2) ^ (am & 7)));
        xa1 = *(const u32x4*)(xs + 16 * (((4 * u + kq) * 2 + 1) ^ (am & 7)));
      } else {
        xa0 = interleave_bf16x8(xg[u][0]);
        xa1 = interleave_bf16x8(xg[u][1]);
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

  // Register double buffer: iteration it+1 is in flight while `it` is
  // transposed and consumed.
  uint32_t it = 0;
  for (; it + 2 <= n_iter; it += 2) {
    load_w(it + 1, wb);
    consume(it, wa);
    if (it + 2 < n_iter) load_w(it + 2, wa);
    consume(it + 1, wb);
  }
  if (it < n_iter) consume(it, wa);

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

#pragma unroll
  for (int rr = 0; rr < R; ++rr) {
    const uint32_t m = 4 * kq + rr;
    if (m >= args.M) continue;
    if (SWIGLU) {
#pragma unroll
      for (int t = 0; t < kHalf; ++t)
        if (row_of[t] < rows_j[0]) {
          const float h = silu_f(acc[t][rr]) * acc[t + kHalf][rr];
          args.jobs[0].out[(size_t)m * rows_j[0] + row_of[t]] = f32_to_bf16(h);
        }
    } else {
#pragma unroll
      for (int t = 0; t < NT; ++t)
        if (row_of[t] < rows_j[0])
          args.jobs[j].out[(size_t)m * rows_j[0] + row_of[t]] = f32_to_bf16(acc[t][rr]);
    }
  }
}

int env_int(const char* name, int fallback) {
  const char* v = getenv(name);
  return v ? atoi(v) : fallback;
}

struct Plan {
  int nt;
  uint32_t tiles, waves, gps, lds;
  bool sb16, xs;
};

int xrows_for(uint32_t M) { return M <= 2 ? 2 : (M <= 4 ? 4 : (M <= 8 ? 8 : 16)); }

// Work decomposition: workgroups own 16*NT rows (a gate/up pair of 16 rows in
// SwiGLU mode); their waves split K.  HBM throughput here is set by the bytes
// in flight, so the split aims at about `target` resident waves.
Plan make_plan(const Q4Job* jobs, int n_jobs, bool swiglu, uint32_t K, uint32_t M) {
  Plan p{};
  const uint32_t G = K / 64;
  uint64_t rows = 0;
  for (int i = 0; i < n_jobs; ++i) rows += jobs[i].rows;
  const uint32_t cus = (uint32_t)env_int("QM38_CUS", 256);
  p.nt = swiglu ? 2 : ((rows / 32 >= (uint64_t)cus * 2) ? 2 : 1);
  if (!swiglu && env_int("QM38_Q4_NT", 0) > 0) p.nt = env_int("QM38_Q4_NT", 1) >= 2 ? 2 : 1;
  const uint32_t rows_per_set = swiglu ? 16u : 16u * p.nt;
  p.tiles = 0;
  if (swiglu) {
    p.tiles = (jobs[0].rows + rows_per_set - 1) / rows_per_set;
  } else {
    for (int i = 0; i < n_jobs; ++i) p.tiles += (jobs[i].rows + rows_per_set - 1) / rows_per_set;
  }
  const int xr = xrows_for(M);
  const bool g8 = (G % 8) == 0;
  const uint32_t step = g8 ? 8 : 4;
  const uint32_t lds_cu = 160 * 1024;
  // Stage the activation slices whole when all of them fit comfortably.
  p.xs = env_int("QM38_Q4_XSTAGE", 0) != 0 && (uint64_t)xr * K * 2 <= 80 * 1024;
  const uint32_t target = (uint32_t)env_int("QM38_Q4_TARGET_WAVES", (int)(cus * 16));
  uint32_t waves = (target + p.tiles - 1) / p.tiles;
  if (env_int("QM38_Q4_SPLIT", 0) > 0) waves = (uint32_t)env_int("QM38_Q4_SPLIT", 1);
  waves = waves < 1 ? 1 : (waves > (uint32_t)kMaxWaves ? (uint32_t)kMaxWaves : waves);
  // Fewer, longer slices lower the total LDS (fixed per-wave buffers); the
  // wave count only decreases, so the search ends.
  for (int guard = 0; guard < 64; ++guard) {
    uint32_t gps = (G + waves - 1) / waves;
    gps = (gps + step - 1) / step * step;
    const uint32_t w = (G + gps - 1) / gps;
    p.gps = gps;
    p.waves = w;
    p.lds = w * wave_layout(p.nt, xr, g8, gps, p.xs).total;
    if (p.lds <= lds_cu / 2 || w == 1) break;
    waves = w - 1;
  }
  p.sb16 = g8;
  return p;
}

template <int NT, int XR, int R, bool SW>
hipError_t launch_one(const DecodeArgs& a, const Plan& p, hipStream_t st) {
  const dim3 grid(p.tiles), block(64 * p.waves);
  if (p.xs) {
    if (p.sb16)
      hipLaunchKernelGGL((q4_decode_kernel<NT, XR, R, SW, true, true>), grid, block, p.lds, st, a);
    else
      hipLaunchKernelGGL((q4_decode_kernel<NT, XR, R, SW, false, true>), grid, block, p.lds, st, a);
  } else {
    if (p.sb16)
      hipLaunchKernelGGL((q4_decode_kernel<NT, XR, R, SW, true, false>), grid, block, p.lds, st, a);
    else
      hipLaunchKernelGGL((q4_decode_kernel<NT, XR, R, SW, false, false>), grid, block, p.lds, st, a);
  }
  return hipGetLastError();
}

template <int NT, bool SW>
hipError_t dispatch_m(const DecodeArgs& a, const Plan& p, hipStream_t st) {
  switch (a.M) {
    case 1: return launch_one<NT, 2, 1, SW>(a, p, st);
    case 2: return launch_one<NT, 2, 2, SW>(a, p, st);
    case 3:
    case 4: return launch_one<NT, 4, 4, SW>(a, p, st);
    case 5:
    case 6:
    case 7:
    case 8: return launch_one<NT, 8, 4, SW>(a, p, st);
    default: return launch_one<NT, 16, 4, SW>(a, p, st);
  }
}

}  // namespace

void q4_decode_workspace(const Q4Job*, int, bool, uint32_t, uint32_t, size_t* partial_bytes, size_t* counters) {
  *partial_bytes = 0;
  *counters = 0;
}

hipError_t launch_q4_decode(const Q4Job* jobs, int n_jobs, bool swiglu, const uint16_t* x,
                            uint32_t K, uint32_t M, const Workspace&, hipStream_t stream) {
  const Plan p = make_plan(jobs, n_jobs, swiglu, K, M);
  if (p.lds > 160 * 1024) return hipErrorInvalidValue;
  DecodeArgs a{};
  a.x = x;
  a.K = K;
  a.M = M;
  a.G = K / 64;
  a.gps = p.gps;
  a.n_jobs = (uint32_t)n_jobs;
  uint32_t ts = 0;
  const uint32_t rows_per_set = swiglu ? 16u : 16u * p.nt;
  for (int i = 0; i < n_jobs; ++i) {
    a.jobs[i] = jobs[i];
    a.jobs[i].tile_begin = ts;
    if (!swiglu) ts += (jobs[i].rows + rows_per_set - 1) / rows_per_set;
  }
  if (swiglu) return dispatch_m<2, true>(a, p, stream);
  return p.nt == 2 ? dispatch_m<2, false>(a, p, stream) : dispatch_m<1, false>(a, p, stream);
}

}  // namespace qm
