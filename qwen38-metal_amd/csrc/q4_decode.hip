// MLX affine-Q4 decode projection for MI355X (gfx950).
//
// Computes y[m][n] = sum_g ( s[n][g] * sum_{i in g} q[n][i] x[m][i]
//                          + b[n][g] * sum_{i in g} x[m][i] )
// for M <= 16 activation rows (decode lanes), the math of
// qwen38_q4_affine_matvec_simd / qwen38_q4_affine_matmul_batch_simd
// (/root/reference/shaders/qwen38.metal:213-246, 1140).
//
// Design (HBM-bound weight stream):
//  * A wave owns a tile of 16 output rows (x NT tiles) and a slice of the K
//    groups; the waves of one workgroup split K and are reduced through LDS,
//    so every launch has thousands of waves streaming weights even for the
//    5120-row down projection.
//  * Per 64-element group a lane loads 8 bytes of packed nibbles (words 2kq,
//    2kq+1 of its row), the four lanes of a row cover the group's 32 bytes.
//  * Nibbles become bf16 (128+q) with one AND-OR per pair (exact), and the
//    dot products run on MFMA 16x16x32 with the activation rows as the A
//    operand (rows >= M are zero).  A second MFMA against an all-ones B gives
//    sum_{i in g} x[m][i].  Then, per group,
//        acc += s * D(128+q) + (b - 128 s) * D(1)
//    which equals s*sum(q x) + b*sum(x) exactly in real arithmetic.
//  * SwiGLU mode pairs a gate tile with the same rows of the up projection in
//    one wave and writes bf16(silu(gate) * up).
#include "common.h"
#include "internal.h"

#include <stdlib.h>

namespace qm {
namespace {

constexpr int kMaxWaves = 16;
constexpr int kUnroll = 4;

struct DecodeArgs {
  const uint16_t* x;
  uint32_t K;
  uint32_t M;
  uint32_t G;    // groups per row = K / 64
  uint32_t gps;  // groups per wave slice
  uint32_t n_jobs;
  Q4Job jobs[kMaxQ4Jobs];
};

template <int NT, bool SWIGLU, bool VEC>
__global__ __launch_bounds__(1024) void q4_decode_kernel(DecodeArgs args) {
  __shared__ float red[kMaxWaves][NT][4][64];

  const int lane = threadIdx.x & 63;
  const int wave = threadIdx.x >> 6;
  const int nwaves = blockDim.x >> 6;
  const int nl = lane & 15;
  const int kq = lane >> 4;
  const uint32_t tile = blockIdx.x;

  int j = 0;
  if (!SWIGLU) {
    while (j + 1 < (int)args.n_jobs && tile >= args.jobs[j + 1].tile_begin) ++j;
  }
  const uint32_t rows_per_tile = SWIGLU ? 16u : 16u * NT;
  const uint32_t row_base = (tile - args.jobs[j].tile_begin) * rows_per_tile;
  const uint32_t K = args.K;
  const uint32_t G = args.G;
  const uint32_t words_per_row = K >> 3;

  const uint32_t* wrow[NT];
  const uint16_t* srow[NT];
  const uint16_t* brow[NT];
  uint32_t row_of[NT];
  uint32_t rows_of[NT];
#pragma unroll
  for (int t = 0; t < NT; ++t) {
    const Q4Job& jb = args.jobs[SWIGLU ? t : j];
    const uint32_t row = row_base + (SWIGLU ? 0u : 16u * t) + nl;
    const uint32_t rc = row < jb.rows ? row : jb.rows - 1;
    row_of[t] = row;
    rows_of[t] = jb.rows;
    wrow[t] = jb.w + (size_t)rc * words_per_row + 2 * kq;
    srow[t] = jb.s + (size_t)rc * G;
    brow[t] = jb.b + (size_t)rc * G;
  }

  const bool mvalid = (uint32_t)nl < args.M;
  const uint16_t* xrow = args.x + (size_t)(mvalid ? nl : 0) * K + 16 * kq;

  floatx4 acc[NT];
#pragma unroll
  for (int t = 0; t < NT; ++t) acc[t] = floatx4{0.f, 0.f, 0.f, 0.f};

  const u32x4 ones = {0x3F803F80u, 0x3F803F80u, 0x3F803F80u, 0x3F803F80u};
  const u32x4 zero4 = {0u, 0u, 0u, 0u};
  const uint32_t g_begin = wave * args.gps;
  const uint32_t g_end = min(G, g_begin + args.gps);

  for (uint32_t g = g_begin; g < g_end; g += kUnroll) {
    u32x2 wv[kUnroll][NT];
    u32x4 xv[kUnroll][2];
    uint32_t sv[kUnroll][NT], bv[kUnroll][NT];
#pragma unroll
    for (int u = 0; u < kUnroll; ++u) {
      const bool ok = VEC || (g + u < g_end);
      const uint32_t gg = ok ? g + u : g;
#pragma unroll
      for (int t = 0; t < NT; ++t)
        wv[u][t] = __builtin_nontemporal_load((const u32x2*)(wrow[t] + (size_t)gg * 8));
      if (mvalid) {
        xv[u][0] = *(const u32x4*)(xrow + (size_t)gg * 64);
        xv[u][1] = *(const u32x4*)(xrow + (size_t)gg * 64 + 8);
      } else {
        xv[u][0] = zero4;
        xv[u][1] = zero4;
      }
      if (!ok) {
        xv[u][0] = zero4;
        xv[u][1] = zero4;
      }
    }
    if (VEC) {
#pragma unroll
      for (int t = 0; t < NT; ++t) {
        const u32x2 s4 = *(const u32x2*)(srow[t] + g);
        const u32x2 b4 = *(const u32x2*)(brow[t] + g);
        sv[0][t] = s4.x & 0xFFFFu; sv[1][t] = s4.x >> 16; sv[2][t] = s4.y & 0xFFFFu; sv[3][t] = s4.y >> 16;
        bv[0][t] = b4.x & 0xFFFFu; bv[1][t] = b4.x >> 16; bv[2][t] = b4.y & 0xFFFFu; bv[3][t] = b4.y >> 16;
      }
    } else {
#pragma unroll
      for (int u = 0; u < kUnroll; ++u) {
        const bool ok = g + u < g_end;
#pragma unroll
        for (int t = 0; t < NT; ++t) {
          sv[u][t] = ok ? srow[t][g + u] : 0u;
          bv[u][t] = ok ? brow[t][g + u] : 0u;
        }
      }
    }
#pragma unroll
    for (int u = 0; u < kUnroll; ++u) {
      const u32x4 xa0 = interleave_bf16x8(xv[u][0]);
      const u32x4 xa1 = interleave_bf16x8(xv[u][1]);
      floatx4 dsum = mfma16x16x32(xa0, ones, floatx4{0.f, 0.f, 0.f, 0.f});
      dsum = mfma16x16x32(xa1, ones, dsum);
#pragma unroll
      for (int t = 0; t < NT; ++t) {
        floatx4 dq = mfma16x16x32(xa0, q4_word_to_bf16x8(wv[u][t].x), floatx4{0.f, 0.f, 0.f, 0.f});
        dq = mfma16x16x32(xa1, q4_word_to_bf16x8(wv[u][t].y), dq);
        const float s = bf16_to_f32(sv[u][t]);
        const float c = fmaf(-128.0f, s, bf16_to_f32(bv[u][t]));
#pragma unroll
        for (int r = 0; r < 4; ++r) acc[t][r] = fmaf(c, dsum[r], fmaf(s, dq[r], acc[t][r]));
      }
    }
  }

  if (nwaves > 1) {
#pragma unroll
    for (int t = 0; t < NT; ++t)
#pragma unroll
      for (int r = 0; r < 4; ++r) red[wave][t][r][lane] = acc[t][r];
    __syncthreads();
    if (wave != 0) return;
#pragma unroll
    for (int t = 0; t < NT; ++t)
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        float v = red[0][t][r][lane];
        for (int w = 1; w < nwaves; ++w) v += red[w][t][r][lane];
        acc[t][r] = v;
      }
  }

#pragma unroll
  for (int r = 0; r < 4; ++r) {
    const uint32_t m = 4 * kq + r;
    if (m >= args.M) continue;
    if (SWIGLU) {
      if (row_of[0] < rows_of[0]) {
        const float h = silu_f(acc[0][r]) * acc[1][r];
        args.jobs[0].out[(size_t)m * rows_of[0] + row_of[0]] = f32_to_bf16(h);
      }
    } else {
#pragma unroll
      for (int t = 0; t < NT; ++t)
        if (row_of[t] < rows_of[t])
          args.jobs[j].out[(size_t)m * rows_of[t] + row_of[t]] = f32_to_bf16(acc[t][r]);
    }
  }
}

int env_int(const char* name, int fallback) {
  const char* v = getenv(name);
  return v ? atoi(v) : fallback;
}

template <int NT, bool SW>
hipError_t dispatch_vec(bool vec, const DecodeArgs& a, uint32_t tiles, int waves, hipStream_t st) {
  if (vec)
    hipLaunchKernelGGL((q4_decode_kernel<NT, SW, true>), dim3(tiles), dim3(64 * waves), 0, st, a);
  else
    hipLaunchKernelGGL((q4_decode_kernel<NT, SW, false>), dim3(tiles), dim3(64 * waves), 0, st, a);
  return hipGetLastError();
}

}  // namespace

hipError_t launch_q4_decode(const Q4Job* jobs, int n_jobs, bool swiglu, const uint16_t* x,
                            uint32_t K, uint32_t M, hipStream_t stream) {
  DecodeArgs a{};
  a.x = x;
  a.K = K;
  a.M = M;
  a.G = K / 64;
  a.n_jobs = (uint32_t)n_jobs;
  uint64_t total_rows = 0;
  for (int i = 0; i < n_jobs; ++i) {
    a.jobs[i] = jobs[i];
    total_rows += jobs[i].rows;
  }
  // Two 16-row tiles per wave when there are enough rows to keep every CU
  // busy; otherwise one, which doubles the number of K-split waves.
  int nt = swiglu ? 2 : (total_rows / 32 >= (uint64_t)env_int("QM38_Q4_NT2_MIN_TILES", 768) ? 2 : 1);
  if (!swiglu && env_int("QM38_Q4_NT", 0) > 0) nt = env_int("QM38_Q4_NT", 1) >= 2 ? 2 : 1;
  const uint32_t rows_per_tile = swiglu ? 16u : 16u * nt;
  uint32_t tiles = 0;
  for (int i = 0; i < n_jobs; ++i) {
    a.jobs[i].tile_begin = tiles;
    if (!swiglu) tiles += (jobs[i].rows + rows_per_tile - 1) / rows_per_tile;
  }
  if (swiglu) tiles = (jobs[0].rows + 15) / 16;

  const bool vec = (a.G % kUnroll) == 0;
  const uint32_t target = (uint32_t)env_int("QM38_Q4_TARGET_WAVES", 4096);
  uint32_t waves = (target + tiles - 1) / tiles;
  if (env_int("QM38_Q4_SPLIT", 0) > 0) waves = (uint32_t)env_int("QM38_Q4_SPLIT", 1);
  waves = waves < 1 ? 1 : (waves > (uint32_t)kMaxWaves ? (uint32_t)kMaxWaves : waves);
  uint32_t gps = (a.G + waves - 1) / waves;
  if (vec) gps = (gps + kUnroll - 1) / kUnroll * kUnroll;
  waves = (a.G + gps - 1) / gps;
  a.gps = gps;

  if (swiglu) return dispatch_vec<2, true>(vec, a, tiles, (int)waves, stream);
  if (nt == 2) return dispatch_vec<2, false>(vec, a, tiles, (int)waves, stream);
  return dispatch_vec<1, false>(vec, a, tiles, (int)waves, stream);
}

}  // namespace qm
