// MLX affine-Q4 projection of 1..8 activation rows on the matrix cores, with
// the weights streamed once and the activations resident in registers, for
// MI355X (gfx950).  The math is qwen38_q4_affine_matvec_simd and its batched
// twins (/root/reference/shaders/qwen38.metal:213-246, 1140, 3451):
//     y[m][n] = sum_g ( s[n][g] * sum_{i in g} q[n][i] x[m][i] + b[n][g] * sum_{i in g} x[m][i] ).
//
// Design:
//  * K is cut into 128-element spans (64 bytes of every weight row).  A load
//    (one 128-bit load per lane) covers 8 weight rows x a pair of spans:
//    lane l reads row l % 8, 16-byte piece g = l / 16 of span (l / 8) % 2 of
//    the pair, so 8 lanes read one contiguous 128-byte run of a row (16 rows
//    x 64 bytes per load measured a third slower).  Two loads (rows 0..7 and
//    8..15) cover a 16-row block.
//  * Each of a lane's 4 words is, as it stands, the B operand of one
//    v_mfma_f32_16x16x32_bf16: AND-OR turns it into 8 bf16 values 128 + q
//    (exact) in the order (q0,q4)(q1,q5)(q2,q6)(q3,q7).  Column n = l % 16 of
//    the MFMA is (weight row l % 8, span n / 8 of the pair) and its k-slots
//    8 g .. 8 g + 7 are piece g of that span (pieces 0, 1: the span's first
//    64-group, 2, 3: its second).
//  * The A operand's 16 rows are (span of the pair, group of the span,
//    activation row 0..3): A row 8 sp + 4 gr + a holds activation row a at
//    span sp in the lanes of group gr's pieces and zeros in the others.  The
//    16x16 result's entry (A row, column) is a group sum when the A row's span
//    is the column's, which is where each lane's 4 outputs sit for half of
//    the lanes (the other half is never read).  Eight activation rows take
//    two MFMAs per word (rows 0..3 and 4..7).  No transpose, no cross-lane
//    move: every weight word is used where it was loaded.
//  * Per lane and slot: D = sum over the 4 words of MFMA(A, B) is
//    sum (128 + q) x over one group; the lane adds s * D + (s - b/128) * Xn
//    with Xn = -128 * sum x over the group (an MFMA of A against a constant
//    -128 operand, once per span pair).  In real arithmetic that is
//    s * sum q x + b * sum x.  The order of the fp32 sums is this kernel's.
//  * A wave owns C spans and keeps their A operands in VGPRs for the whole
//    launch (8 VGPRs per span per 4 activation rows).  Scales and biases of
//    the workgroup's rows and the wave's groups are fetched once, ahead of
//    the weights, and kept in LDS as raw bf16 (s, b) words.
//  * Blocks: SB load pairs per span pair.  SB = 1: 16 rows of a plain
//    projection; SB = 2: 32 rows, or 16 gate rows and the same 16 up rows of
//    a SwiGLU pair.  A workgroup owns a contiguous run of blocks; each
//    finished (block, load, half) adds its two group sums per span across
//    lanes and writes them to the wave's LDS partials; after the stream the
//    workgroup adds each value's partials in a fixed order (deterministic)
//    and stores.
//  * K beyond 12 waves x C spans runs in K parts on separate workgroups whose
//    fp32 sums go to a workspace (device-scope relaxed atomics); the last part
//    to finish adds the parts in part order.
#include "common.h"
#include "internal.h"

#include <stdio.h>

#include <algorithm>
#include <cstring>
#include <mutex>

namespace qm {
namespace {

constexpr int kSpanElems = 128;
constexpr int kMaxWaves = 12;  // 768 threads: 168 VGPRs per lane (3 waves per SIMD)
constexpr int kMaxRows = 8;
constexpr int kNonTemporal = 2;
constexpr uint32_t kOOB = 0xFFFFFFF0u;
constexpr uint32_t kMaxLds = 160 * 1024;  // LDS of one workgroup on gfx950
// Table entries per wave: 64 per load a lane issues (3 with 4 spans per wave,
// 2 with 8, whose entries take two 16-byte loads each).
__host__ __device__ constexpr int tab_loads(int c) { return c == 4 ? 3 : 2; }
__host__ __device__ constexpr uint32_t tab_entries(int c) { return 64u * tab_loads(c); }

struct MmaArgs {
  const uint16_t* x;
  uint32_t K, G, spans;
  uint32_t waves;
  uint32_t n_jobs;
  uint32_t total_blocks;
  uint32_t wgs;         // workgroups per K part; workgroup g owns blocks [g*B/wgs, (g+1)*B/wgs)
  uint32_t max_blocks;  // largest block count of one workgroup (LDS sizing)
  uint32_t parts, part_spans;
  float* partials;
  unsigned* counters;
  uint32_t M;
  Q4Job jobs[kMaxQ4Jobs];
};

__device__ __forceinline__ __amdgpu_buffer_rsrc_t make_rsrc(const void* base, uint64_t bytes) {
  const uint32_t n = bytes > 0xFFFFFFF0ull ? 0xFFFFFFF0u : (uint32_t)bytes;
  return __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(base), (short)0, (int)n, 0x00020000);
}

__host__ __device__ constexpr uint32_t job_blocks(uint32_t rows, uint32_t mode, int sb) {
  return mode == kQ4OutSwiglu ? (rows + 15) / 16 : (rows + 16 * sb - 1) / (16 * sb);
}
__device__ __forceinline__ uint32_t block_row(uint32_t mode, int sb, uint32_t jb, int s) {
  return mode == kQ4OutSwiglu ? 16 * jb : 16 * sb * jb + 16 * s;
}
// LDS: per-wave partials [wave][local row][span of a pair][4 AH activation
// rows], then each wave's tables: per (block, SB, row) entry 2C + 1 words
// (the odd stride spreads a read's 8 rows over distinct banks).
__host__ __device__ constexpr uint32_t head_bytes(uint32_t waves, int sb, uint32_t blocks, int ah) {
  return waves * blocks * sb * 16 * 2 * (4 * ah) * 4;
}
__host__ __device__ constexpr uint32_t entry_words(int c) { return 2 * c + 1; }
__host__ __device__ constexpr uint32_t table_bytes(uint32_t blocks, int sb, int c) {
  return blocks * sb * 16 * entry_words(c) * 4;
}

// One packed word -> 8 bf16 values 128 + q in the order (q0,q4)(q1,q5)(q2,q6)(q3,q7).
__device__ __forceinline__ u32x4 q4_unpack(uint32_t w, uint32_t mask_s, uint32_t or_v) {
  u32x4 r;
  r.x = (w & mask_s) | or_v;
  r.y = ((w >> 4) & mask_s) | or_v;
  r.z = ((w >> 8) & mask_s) | or_v;
  r.w = ((w >> 12) & mask_s) | or_v;
  return r;
}

template <int C, int SB, int RB, int AH>
__global__ __launch_bounds__(64 * kMaxWaves) void q4_mma_kernel(MmaArgs args) {
  extern __shared__ __attribute__((aligned(16))) uint8_t smem[];
  static_assert(C % 4 == 0 && C <= 8, "spans per wave: 4 or 8 (table entries of 8 or 16 groups)");
  static_assert(AH == 1 || AH == 2, "activation row halves");
  constexpr int kP = C / 2;         // span pairs per wave
  constexpr int kPer = SB * C;      // loads per block per wave (SB x 2 halves x kP pairs)
  constexpr int kU = kPer * RB;     // loads per round
  constexpr int kD = kU < 8 ? kU : 8;  // ring slots (8 loads in flight)
  static_assert(kU % kD == 0, "ring");
  constexpr int kRW = 4 * AH;       // activation rows kept per partial
  const int lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const uint32_t W = args.waves;
  const uint32_t K = args.K, G = args.G;
  const uint32_t row_bytes = K >> 1;
  const int n = lane & 15;          // MFMA column: weight row n % 8, span n / 8 of the pair
  const int q = lane >> 4;          // k piece of a span / output row quarter
  const int r8 = lane & 7;
  const int hi = (lane >> 3) & 1;   // span of the pair this lane's weights hold
  const bool valid_out = (q >> 1) == hi;  // this lane's outputs are group sums

  const uint32_t part = blockIdx.x / args.wgs;
  const uint32_t gi = blockIdx.x - part * args.wgs;
  const uint32_t b_begin = (uint32_t)(((uint64_t)gi * args.total_blocks) / args.wgs);
  const uint32_t b_end = (uint32_t)(((uint64_t)(gi + 1) * args.total_blocks) / args.wgs);
  const uint32_t nblk = b_end - b_begin;

  const uint32_t rows_wg = args.max_blocks * SB * 16;  // weight rows of the workgroup
  float* parts = (float*)smem;                         // [W][rows_wg][4][kRW]
  uint32_t* tab =
      (uint32_t*)(smem + head_bytes(W, SB, args.max_blocks, AH) + wave * table_bytes(args.max_blocks, SB, C));

  auto job_of = [&](uint32_t blk) __attribute__((always_inline)) {
    int j = 0;
    while (j + 1 < (int)args.n_jobs && blk >= args.jobs[j + 1].tile_begin) ++j;
    return j;
  };

  // --- scale / bias tables: entry e = (s * nblk + jl) * 16 + r holds the 2C
  // groups [2 c0, 2 c0 + 2C) of row r of load s of local block jl.
  const uint32_t c0 = part * args.part_spans + (uint32_t)wave * C;  // first span of this wave
  const uint32_t n_e = SB * nblk * 16;
  constexpr int kTW = C / 4;  // 16-byte table loads per entry (8 groups each)
  constexpr int kTabLoads = tab_loads(C);
  u32x4 tsv[kTabLoads][kTW], tbv[kTabLoads][kTW];
#pragma unroll
  for (int i = 0; i < kTabLoads; ++i) {
    const uint32_t e = i * 64 + lane;
#pragma unroll
    for (int u = 0; u < kTW; ++u) {
      tsv[i][u] = u32x4{0u, 0u, 0u, 0u};
      tbv[i][u] = u32x4{0u, 0u, 0u, 0u};
    }
    if (e < n_e) {
      const uint32_t r = e % 16, t = e / 16;
      const uint32_t sub = t / nblk, jl = t % nblk;
      const uint32_t blk = b_begin + jl;
      const Q4Job& jb = args.jobs[job_of(blk)];
      const bool up = jb.mode == kQ4OutSwiglu && sub == 1;
      const uint16_t* ts = up ? jb.us : jb.s;
      const uint16_t* tb = up ? jb.ub : jb.b;
      const uint32_t row = block_row(jb.mode, SB, blk - jb.tile_begin, (int)sub) + r;
#pragma unroll
      for (int u = 0; u < kTW; ++u) {
        const uint32_t gcol = 2 * c0 + 8 * u;
        if (row < jb.rows && gcol < G) {
          const size_t idx = (size_t)row * G + gcol;
          if (G % 8 == 0) {
            tsv[i][u] = *(const u32x4*)(ts + idx);
            tbv[i][u] = *(const u32x4*)(tb + idx);
          } else {
            uint16_t sv[8], bv[8];
#pragma unroll
            for (int k = 0; k < 8; ++k) {
              const bool in = gcol + k < G;
              sv[k] = in ? ts[idx + k] : (uint16_t)0;
              bv[k] = in ? tb[idx + k] : (uint16_t)0;
            }
            tsv[i][u] = u32x4{sv[0] | (uint32_t)sv[1] << 16, sv[2] | (uint32_t)sv[3] << 16,
                              sv[4] | (uint32_t)sv[5] << 16, sv[6] | (uint32_t)sv[7] << 16};
            tbv[i][u] = u32x4{bv[0] | (uint32_t)bv[1] << 16, bv[2] | (uint32_t)bv[3] << 16,
                              bv[4] | (uint32_t)bv[5] << 16, bv[6] | (uint32_t)bv[7] << 16};
          }
        }
      }
    }
  }
  __builtin_amdgcn_sched_barrier(0);

  // --- A operands: lane (m' = n, piece q) of pair p, word j, half ah holds
  // activation row 4 ah + m' % 4 at span c0 + 2p + m' / 8, elements
  // [32 q + 8 j, +8) of the span, when piece q is in the A row's group
  // ((m' / 4) % 2 == q / 2) and the activation row exists; zeros otherwise.
  u32x4 xa[kP][AH][4];
  {
    const uint32_t sp = (uint32_t)(n >> 3);
    const bool in_group = ((n >> 2) & 1) == (q >> 1);
    // One resource over all M rows (uniform); lanes that hold zeros load from
    // past its end.
    const __amdgpu_buffer_rsrc_t rx = make_rsrc(args.x, (uint64_t)args.M * K * 2);
#pragma unroll
    for (int ah = 0; ah < AH; ++ah) {
      const uint32_t mi = 4 * ah + (n & 3);
      const bool live = in_group && mi < args.M;
#pragma unroll
      for (int p = 0; p < kP; ++p) {
        const uint32_t span = c0 + 2 * p + sp;
        const uint32_t e0 = span * kSpanElems + 32 * q;
        const bool ok = live && span < args.spans && e0 < K;
        const uint32_t off = (mi * K + e0) * 2;
#pragma unroll
        for (int j = 0; j < 4; ++j)
          xa[p][ah][j] = __builtin_amdgcn_raw_buffer_load_b128(rx, ok ? off + 16 * j : kOOB, 0, 0);
      }
    }
  }
  __builtin_amdgcn_sched_barrier(0);

  // --- weight ring ---------------------------------------------------------
  // Load v of a block: (load s, half i, pair p) with p fastest.  voff[i][p]:
  // this lane's byte offset inside a load.
  uint32_t voff[2][kP];
#pragma unroll
  for (int i = 0; i < 2; ++i)
#pragma unroll
    for (int p = 0; p < kP; ++p) {
      const uint32_t span = c0 + 2 * p + hi;
      voff[i][p] = span < args.spans ? (8 * i + r8) * row_bytes + span * 64 + 16 * q : kOOB;
    }

  int cj = __builtin_amdgcn_readfirstlane(job_of(b_begin));
  uint32_t cj_begin = 0, cj_end = 0, c_rows = 0, c_mode = 0;
  const uint32_t* c_w = nullptr;
  const uint32_t* c_uw = nullptr;
  auto set_job = [&]() __attribute__((always_inline)) {
    const Q4Job& jb = args.jobs[cj];
    cj_begin = jb.tile_begin;
    cj_end = cj + 1 < (int)args.n_jobs ? args.jobs[cj + 1].tile_begin : args.total_blocks;
    c_rows = jb.rows;
    c_mode = jb.mode;
    c_w = jb.w;
    c_uw = jb.uw;
  };
  set_job();
  auto load_w = [&](uint32_t jl, int s, int i, int p) __attribute__((always_inline)) {
    const uint32_t blk = b_begin + jl;
    if (jl < nblk && blk >= cj_end) {
      ++cj;
      set_job();
    }
    const bool live = (jl < nblk) & (b_begin + jl - cj_begin < (1u << 30));
    const bool up = (c_mode == kQ4OutSwiglu) & (s == 1);
    const uint32_t* w = up ? c_uw : c_w;
    const uint32_t base_row = live ? block_row(c_mode, SB, blk - cj_begin, s) : 0;
    const uint32_t left = (live & (base_row < c_rows)) ? c_rows - base_row : 0;
    const uint32_t avail = left >= 0xFFFFFFF0u / row_bytes ? 0xFFFFFFF0u : left * row_bytes;
    const __amdgpu_buffer_rsrc_t r = __builtin_amdgcn_make_buffer_rsrc(
        const_cast<uint32_t*>(w + (size_t)base_row * (row_bytes / 4)), (short)0, (int)avail, 0x00020000);
    return __builtin_amdgcn_raw_buffer_load_b128(r, voff[i][p], 0, kNonTemporal);
  };

  u32x4 ring[kD];
  const uint32_t nrounds = (nblk + RB - 1) / RB;
#pragma unroll
  for (int t = 0; t < kD; ++t) {
    ring[t] = load_w(t / kPer, (t % kPer) / C, ((t % kPer) / kP) % 2, t % kP);
    __builtin_amdgcn_sched_barrier(0);
  }
  // Tables into LDS as (s | b << 16) words, one per (row, group).
#pragma unroll
  for (int i = 0; i < kTabLoads; ++i) {
    const uint32_t e = i * 64 + lane;
    if (e < n_e) {
      uint32_t* te = tab + e * entry_words(C);
#pragma unroll
      for (int u = 0; u < kTW; ++u) {
        const uint32_t sw[4] = {tsv[i][u].x, tsv[i][u].y, tsv[i][u].z, tsv[i][u].w};
        const uint32_t bw[4] = {tbv[i][u].x, tbv[i][u].y, tbv[i][u].z, tbv[i][u].w};
#pragma unroll
        for (int k = 0; k < 4; ++k) {
          te[8 * u + 2 * k] = perm_b32(bw[k], sw[k], 0x05040100u);
          te[8 * u + 2 * k + 1] = perm_b32(bw[k], sw[k], 0x07060302u);
        }
      }
    }
  }
  // Activations into the unpack order, and -128 * (group sums) per pair in
  // the output layout: lane (n, q) output r is A row 4 q + r.
  floatx4 xn[kP][AH];
  {
    const u32x4 m128 = u32x4{0xC300C300u, 0xC300C300u, 0xC300C300u, 0xC300C300u};  // bf16 -128
#pragma unroll
    for (int p = 0; p < kP; ++p)
#pragma unroll
      for (int ah = 0; ah < AH; ++ah) {
#pragma unroll
        for (int j = 0; j < 4; ++j) xa[p][ah][j] = interleave_bf16x8(xa[p][ah][j]);
        floatx4 d = floatx4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
        for (int j = 0; j < 4; ++j) d = mfma16x16x32(xa[p][ah][j], m128, d);
        xn[p][ah] = d;
      }
  }
  // Each wave reads only its own tables (a wave's LDS operations complete in
  // order): no barrier needed.

  const uint32_t mask_s = __builtin_amdgcn_readfirstlane(0x000F000Fu);
  uint32_t or_v = 0x43004300u;
  asm volatile("" : "+v"(or_v));

  // Table word of this lane's outputs: row 8 i + lane % 8 of load s of block
  // jl, group 2 (2p + q / 2) + q % 2 of the wave's groups (= 4p + q).
  auto consume = [&](const u32x4& wv, uint32_t jl, int s, int i, int p, floatx4(&acc)[AH])
                     __attribute__((always_inline)) {
    const uint32_t e = (s * nblk + jl) * 16 + 8 * i + r8;
    const uint32_t tv = tab[e * entry_words(C) + 4 * p + q];
    const float sc = __uint_as_float(tv << 16);
    const float cb = fmaf(__uint_as_float(tv & 0xFFFF0000u), -0.0078125f, sc);  // s - b/128
    const u32x4 b0 = q4_unpack(wv.x, mask_s, or_v), b1 = q4_unpack(wv.y, mask_s, or_v);
    const u32x4 b2 = q4_unpack(wv.z, mask_s, or_v), b3 = q4_unpack(wv.w, mask_s, or_v);
#pragma unroll
    for (int ah = 0; ah < AH; ++ah) {
      floatx4 d = floatx4{0.f, 0.f, 0.f, 0.f};
      d = mfma16x16x32(xa[p][ah][0], b0, d);
      d = mfma16x16x32(xa[p][ah][1], b1, d);
      d = mfma16x16x32(xa[p][ah][2], b2, d);
      d = mfma16x16x32(xa[p][ah][3], b3, d);
#pragma unroll
      for (int r = 0; r < 4; ++r) acc[ah][r] = fmaf(sc, d[r], fmaf(cb, xn[p][ah][r], acc[ah][r]));
    }
  };

  // A finished (block, load s, half i): the two groups of each span are
  // added across the lane pairs (q, q ^ 1) (permlane16 swap); lanes
  // (row, span 0, q = 0) and (row, span 1, q = 2) store the span's sums to
  // the wave's partial row 8 i + lane % 8, slot = span.
  auto finish = [&](uint32_t jl, int s, int i, const floatx4(&acc)[AH]) __attribute__((always_inline)) {
    floatx4 v[AH];
#pragma unroll
    for (int ah = 0; ah < AH; ++ah)
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        const auto sw = __builtin_amdgcn_permlane16_swap(__float_as_uint(acc[ah][r]), __float_as_uint(acc[ah][r]),
                                                         false, false);
        v[ah][r] = __uint_as_float(sw[0]) + __uint_as_float(sw[1]);
      }
    if (valid_out && (q & 1) == 0) {
      float* pr = parts + ((wave * rows_wg + (jl * SB + s) * 16 + 8 * i + r8) * 2 + hi) * kRW;
#pragma unroll
      for (int ah = 0; ah < AH; ++ah) *(floatx4*)(pr + 4 * ah) = v[ah];
    }
  };

  // A round is RB blocks (kU loads); load u sits in ring slot u % kD and is
  // refilled with load u + kD of the stream (the next round's when that is
  // past this round).  The last round issues no loads past its own.
  auto round = [&](uint32_t r, bool refill) __attribute__((always_inline)) {
    floatx4 acc[AH];
#pragma unroll
    for (int u = 0; u < kU; ++u) {
      const int v = u % kPer;
      const uint32_t jl = r * RB + u / kPer;
      const int s = v / C, i = (v / kP) % 2, p = v % kP;
      if (p == 0) {
#pragma unroll
        for (int ah = 0; ah < AH; ++ah) acc[ah] = floatx4{0.f, 0.f, 0.f, 0.f};
      }
      consume(ring[u % kD], jl, s, i, p, acc);
      if (refill || u + kD < kU) {
        const int nu = u + kD, nv = nu % kPer;
#pragma unroll
        for (int ah = 0; ah < AH; ++ah) asm volatile("" : "+v"(acc[ah]) : : "memory");
        __builtin_amdgcn_sched_barrier(0);
        ring[u % kD] = load_w(r * RB + nu / kPer, nv / C, (nv / kP) % 2, nv % kP);
        __builtin_amdgcn_sched_barrier(0);
      }
      if (p == kP - 1 && jl < nblk) finish(jl, s, i, acc);
    }
  };
  if (nrounds > 0) {
    uint32_t r = 0;
    for (; r + 1 < nrounds; ++r) round(r, true);
    round(r, false);
  }

  // --- outputs ---------------------------------------------------------------
  lds_barrier();
  const uint32_t rows_per_block = 16 * SB;
  const uint32_t nvals = nblk * rows_per_block * kMaxRows;  // value f = local row * 8 + activation row
  // Value (local row i, activation row m) over this workgroup's spans: the
  // partials of every wave (in wave order), each the sum of its two spans.
  auto row_sum = [&](uint32_t f) __attribute__((always_inline)) {
    const uint32_t i = f / kMaxRows, m = f % kMaxRows;
    float v = 0.f;
    for (uint32_t w2 = 0; w2 < W; ++w2) {
      const float* pr = parts + ((w2 * rows_wg + i) * 2) * kRW + m;
      v += pr[0] + pr[kRW];
    }
    return v;
  };
  const uint32_t TB = args.total_blocks * rows_per_block * kMaxRows;  // values per K part
  float* pp = args.partials + (size_t)b_begin * rows_per_block * kMaxRows;
  auto part_sum = [&](uint32_t i) __attribute__((always_inline)) {
    float v = 0.f;
    for (uint32_t k = 0; k < args.parts; ++k)
      v += __hip_atomic_load(&pp[(size_t)k * TB + i], __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    return v;
  };
  if (args.parts > 1) {
    for (uint32_t f = threadIdx.x; f < nvals; f += blockDim.x)
      if (f % kMaxRows < args.M)
        __hip_atomic_store(&pp[(size_t)part * TB + f], row_sum(f), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    __builtin_amdgcn_s_waitcnt(0);
    __syncthreads();
    __shared__ uint32_t last;
    if (threadIdx.x == 0) {
      const uint32_t old = __hip_atomic_fetch_add(&args.counters[gi], 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
      last = old == args.parts - 1;
      if (last) __hip_atomic_store(&args.counters[gi], 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    }
    __syncthreads();
    if (!last) return;
  }
  auto value = [&](uint32_t i) __attribute__((always_inline)) {
    return args.parts > 1 ? part_sum(i) : row_sum(i);
  };
  for (uint32_t f = threadIdx.x; f < nvals; f += blockDim.x) {
    const uint32_t i = f / kMaxRows, m = f % kMaxRows;
    if (m >= args.M) continue;
    const uint32_t jl = i / rows_per_block, k = i % rows_per_block;
    const uint32_t blk = b_begin + jl;
    const Q4Job& jb = args.jobs[job_of(blk)];
    const uint32_t lb = blk - jb.tile_begin;
    if (jb.mode == kQ4OutSwiglu) {
      // k < 16: gate sums; k >= 16: the up sums of the same rows.
      const uint32_t row = 16 * lb + k;
      if (k < 16 && row < jb.rows) {
        const float gsum = value((jl * rows_per_block + k) * kMaxRows + m);
        const float usum = value((jl * rows_per_block + 16 + k) * kMaxRows + m);
        jb.out[(size_t)m * jb.rows + row] = f32_to_bf16(silu_f(gsum) * usum);
      }
      continue;
    }
    const uint32_t row = rows_per_block * lb + k;
    if (row >= jb.rows) continue;
    const uint16_t hv = f32_to_bf16(value(f));
    const size_t o = (size_t)m * jb.rows + row;
    if (jb.mode == kQ4OutBf16)
      jb.out[o] = hv;
    else if (jb.mode == kQ4OutF32)
      ((float*)jb.out)[o] = bf16_to_f32(hv);
    else
      ((float*)jb.out)[o] += bf16_to_f32(hv);
  }
}

// Rounds of at least 8 loads (the ring).
template <int C, int SB, int AH>
const void* kernel_for() {
  constexpr int kRB = (8 / (SB * C)) > 1 ? 8 / (SB * C) : 1;
  return (const void*)q4_mma_kernel<C, SB, kRB, AH>;
}
const void* pick_kernel(int c, int sb, int ah) {
  if (ah == 1) {
    if (c == 8) return sb == 2 ? kernel_for<8, 2, 1>() : kernel_for<8, 1, 1>();
    if (c == 4) return sb == 2 ? kernel_for<4, 2, 1>() : kernel_for<4, 1, 1>();
  } else if (c == 4) {
    return sb == 2 ? kernel_for<4, 2, 2>() : kernel_for<4, 1, 2>();
  }
  return nullptr;
}

struct MmaPlan {
  const void* fn = nullptr;
  uint32_t waves = 0, C = 0, SB = 0, AH = 1, wgs = 0, max_blocks = 0, lds = 0, total_blocks = 0;
  uint32_t parts = 1, part_spans = 0;
  size_t partial_bytes = 0, counters = 0;
};

MmaPlan make_mma_plan(const Q4Job* jobs, int n_jobs, uint32_t K, uint32_t M, const Tuning& tn) {
  MmaPlan p{};
  const uint32_t spans = (K + kSpanElems - 1) / kSpanElems;
  bool pair = false;
  for (int i = 0; i < n_jobs; ++i) pair |= jobs[i].mode == kQ4OutSwiglu;
  // Up to four activation rows: 8 spans per wave (64 VGPRs of A operands);
  // up to eight: two A halves of 4 spans.
  // 8 spans per wave when K fits one part of 12 waves, otherwise 4 (more
  // waves per part: measured on the 17408-wide down projection, 16.0 against
  // 17.8 us at M = 4 with 8 spans in two parts).
  p.AH = M <= 4 ? 1 : 2;
  p.C = p.AH == 2 || tn.q4_mma_c == 4 || (tn.q4_mma_c != 8 && spans > (uint32_t)kMaxWaves * 8) ? 4 : 8;
  const uint32_t wmax = tn.q4_mma_w > 0 ? std::min<uint32_t>(tn.q4_mma_w, kMaxWaves) : kMaxWaves;
  p.parts = (spans + wmax * p.C - 1) / (wmax * p.C);
  p.waves = ((spans + p.parts - 1) / p.parts + p.C - 1) / p.C;
  p.part_spans = p.waves * p.C;
  p.SB = (pair || tn.q4_mma_sb == 2) ? 2 : 1;
  for (int i = 0; i < n_jobs; ++i) p.total_blocks += job_blocks(jobs[i].rows, jobs[i].mode, (int)p.SB);
  p.fn = pick_kernel((int)p.C, (int)p.SB, (int)p.AH);
  if (!p.fn) return p;
  const uint32_t cus = tn.cus > 0 ? (uint32_t)tn.cus : 256;
  auto lds_of = [&](uint32_t mb) { return head_bytes(p.waves, p.SB, mb, p.AH) + p.waves * table_bytes(mb, p.SB, p.C); };
  // Blocks per workgroup: at most the wave's table entries, and within the
  // 160 KiB of LDS a workgroup may have (the occupancy query does not check
  // that limit).
  uint32_t cap = tab_entries((int)p.C) / (p.SB * 16);
  while (cap > 0 && lds_of(cap) > kMaxLds) --cap;
  if (cap == 0) {
    p.fn = nullptr;
    return p;
  }
  // Workgroups: the most that stay resident in one dispatch round, with the
  // blocks per workgroup (and so the LDS) that this count implies.
  int occ_regs = 0;
  if (hipOccupancyMaxActiveBlocksPerMultiprocessor(&occ_regs, p.fn, (int)(64 * p.waves), lds_of(1)) != hipSuccess ||
      occ_regs <= 0) {
    p.fn = nullptr;
    return p;
  }
  uint32_t mb = cap;
  for (int occ = occ_regs; occ >= 1; --occ) {
    const uint32_t resident = std::max<uint32_t>(1, (uint32_t)occ * cus / p.parts);
    const uint32_t need = std::max<uint32_t>(1, (p.total_blocks + resident - 1) / resident);
    int fit = 0;
    if (need <= cap &&
        hipOccupancyMaxActiveBlocksPerMultiprocessor(&fit, p.fn, (int)(64 * p.waves), lds_of(need)) == hipSuccess &&
        fit >= occ) {
      mb = need;
      break;
    }
  }
  p.wgs = (p.total_blocks + mb - 1) / mb;
  if (tn.q4_mma_wgs > 0) p.wgs = std::max((p.total_blocks + cap - 1) / cap, std::min(p.total_blocks, (uint32_t)tn.q4_mma_wgs));
  p.max_blocks = (p.total_blocks + p.wgs - 1) / p.wgs;
  p.lds = lds_of(p.max_blocks);
  const int occ = occ_regs;
  if (p.parts > 1) {
    p.partial_bytes = (size_t)p.parts * p.total_blocks * 16 * p.SB * kMaxRows * sizeof(float);
    p.counters = p.wgs;
  }
  if (tn.q4_plan_log > 0)
    fprintf(stderr,
            "q4 mma plan: K=%u M=%u jobs=%d blocks=%u C=%u SB=%u AH=%u waves=%u parts=%u wgs/part=%u "
            "max_blocks=%u lds=%u occ=%d\n",
            K, M, n_jobs, p.total_blocks, p.C, p.SB, p.AH, p.waves, p.parts, p.wgs, p.max_blocks, p.lds, occ);
  return p;
}

struct MmaKey {
  uint32_t rows[kMaxQ4Jobs], modes[kMaxQ4Jobs];
  int n_jobs;
  uint32_t K, AH;
  Tuning tune;
  bool operator==(const MmaKey& o) const { return std::memcmp(this, &o, sizeof(*this)) == 0; }
};

MmaPlan cached_mma_plan(const Q4Job* jobs, int n_jobs, uint32_t K, uint32_t M, const Tuning& tn) {
  static std::mutex mu;
  static MmaKey keys[16];
  static MmaPlan plans[16];
  static int used = 0, next = 0;
  MmaKey k;
  std::memset(&k, 0, sizeof(k));
  for (int i = 0; i < n_jobs; ++i) {
    k.rows[i] = jobs[i].rows;
    k.modes[i] = jobs[i].mode == kQ4OutSwiglu ? 1 : 0;
  }
  k.n_jobs = n_jobs;
  k.K = K;
  k.AH = M <= 4 ? 1 : 2;
  k.tune = tn;
  std::lock_guard<std::mutex> lock(mu);
  for (int i = 0; i < used; ++i)
    if (keys[i] == k) return plans[i];
  const MmaPlan p = make_mma_plan(jobs, n_jobs, K, M, tn);
  keys[next] = k;
  plans[next] = p;
  next = (next + 1) % 16;
  used = std::min(used + 1, 16);
  return p;
}

}  // namespace

bool q4_mma_supported(const Q4Job* jobs, int n_jobs, uint32_t K, uint32_t M, const Tuning& tn) {
  // 3..4 rows (QM38_Q4_MMA_LO / _HI); 2..8 rows when K is long (above
  // QM38_Q4_MMA_K): there the other kernels split K over workgroups (two
  // rows) or cap the waves per tile (five and more), and this one measured
  // faster on the 17408-wide down projection (M = 2: 15.3 against 19.6 us,
  // M = 8: 18.9 against 25.3 us).
  const uint32_t hi = tn.q4_mma_hi > 0 ? std::min<uint32_t>(tn.q4_mma_hi, kMaxRows) : kMaxRows;
  const bool in_range = tn.q4_mma_lo > 0 && M >= (uint32_t)tn.q4_mma_lo && M <= hi;
  const bool long_k = tn.q4_mma_k > 0 && K > (uint32_t)tn.q4_mma_k && M >= 2 && M <= (uint32_t)kMaxRows;
  if (!(in_range || long_k) || n_jobs < 1 || n_jobs > kMaxQ4Jobs || K % 64 != 0) return false;
  for (int i = 0; i < n_jobs; ++i)
    if (jobs[i].mode > kQ4OutAddF32 && jobs[i].mode != kQ4OutSwiglu) return false;
  return cached_mma_plan(jobs, n_jobs, K, M, tn).fn != nullptr;
}

void q4_mma_workspace(const Q4Job* jobs, int n_jobs, uint32_t K, uint32_t M, const Tuning& tn,
                      size_t* partial_bytes, size_t* counters) {
  const MmaPlan p = cached_mma_plan(jobs, n_jobs, K, M, tn);
  *partial_bytes = p.partial_bytes;
  *counters = p.counters;
}

hipError_t launch_q4_mma(const Q4Job* jobs, int n_jobs, const uint16_t* x, uint32_t K, uint32_t M,
                         const Workspace& ws, hipStream_t stream) {
  if (!ws.tune || n_jobs < 1 || n_jobs > kMaxQ4Jobs || M < 1 || M > (uint32_t)kMaxRows) return hipErrorInvalidValue;
  const MmaPlan p = cached_mma_plan(jobs, n_jobs, K, M, *ws.tune);
  if (!p.fn) return hipErrorInvalidValue;
  if (p.parts > 1 &&
      (!ws.partials || ws.partial_bytes < p.partial_bytes || !ws.counters || ws.counter_count < p.counters))
    return hipErrorInvalidValue;
  MmaArgs a{};
  a.x = x;
  a.K = K;
  a.G = K / 64;
  a.spans = (K + kSpanElems - 1) / kSpanElems;
  a.waves = p.waves;
  a.n_jobs = (uint32_t)n_jobs;
  a.total_blocks = p.total_blocks;
  a.wgs = p.wgs;
  a.max_blocks = p.max_blocks;
  a.parts = p.parts;
  a.part_spans = p.part_spans;
  a.partials = ws.partials;
  a.counters = ws.counters;
  a.M = M;
  uint32_t b = 0;
  for (int i = 0; i < n_jobs; ++i) {
    a.jobs[i] = jobs[i];
    a.jobs[i].tile_begin = b;
    b += job_blocks(jobs[i].rows, jobs[i].mode, (int)p.SB);
  }
  void* args[] = {&a};
  const hipError_t e = hipLaunchKernel(p.fn, dim3(p.wgs * p.parts), dim3(64 * p.waves), args, p.lds, stream);
  return e != hipSuccess ? e : hipGetLastError();
}

}  // namespace qm
