// MLX affine-Q4 projection of one or two activation rows (decode) for MI355X
// (gfx950): the math of qwen38_q4_affine_matvec_simd
// (/root/reference/shaders/qwen38.metal:213-246),
//     y[n] = sum_g ( s[n][g] * sum_{i in g} q[n][i] x[i] + b[n][g] * sum_{i in g} x[i] ).
//
// Design (HBM-bound weight stream, activation resident in registers):
//  * K is cut into 512-element chunks (256 bytes of every weight row).  A
//    workgroup has W waves; wave w owns chunks [w*C, w*C + C) and keeps the
//    activation of those chunks in VGPRs for the whole launch, so neither the
//    weights nor the activation pass through LDS.  With two activation rows
//    (MR = 2, one chunk per wave) every unpacked weight word meets both rows'
//    activations.
//  * One 128-bit load per lane covers 4 rows x 256 bytes: lane l reads 16
//    bytes (32 nibbles, half of a 64-group) of row l/16 at column 16*(l%16).
//    Loads are coalesced (16 lanes read one contiguous 256-byte run) and
//    stream into a register ring of D slots issued ahead of consumption.
//  * Each word becomes four bf16 pairs (128+q_j, 128+q_{j+4}) with one
//    AND-OR each (0x4300|q is the bf16 of 128+q, exact), and
//    v_dot2_f32_bf16 multiplies them by the matching activation pairs.  Per
//    lane:  p = sum (128+q) x  over its 32 elements, and the lane adds
//        s * p + (b - 128 s) * X      (X = sum of those 32 activations),
//    which equals s*sum(q x) + b*sum(x) over the half-group in real arithmetic.
//  * Blocks: a workgroup owns a contiguous run of blocks.  A block is SB loads
//    per chunk: SB = 2 gives 8 rows of a plain projection, or 4 rows of a
//    gate/up pair (gate rows, then the same up rows: SwiGLU).  Each wave
//    reduces its 16 lanes per row (DPP) and writes the row's partial over its
//    chunks to LDS.  After the stream the workgroup adds the W partials of
//    each row in wave order (deterministic) and stores the outputs; no global
//    store is issued while weights are in flight.
//  * Scales and biases of the workgroup's rows and the wave's chunks are
//    fetched once (ordinary loads issued before the weight stream) and kept
//    in LDS.
//  * Rows past a projection's end load zeros (buffer bounds) and are never
//    stored; activation elements past K load zeros, and their lanes add 0.
#include "common.h"
#include "internal.h"

#include <stdio.h>

#include <algorithm>
#include <cstring>
#include <mutex>

namespace qm {
namespace {

constexpr int kChunkElems = 512;  // 16 lanes x 32 elements
constexpr int kMaxWaves = 16;
constexpr int kNonTemporal = 2;   // buffer cache policy: weights are streamed once
constexpr uint32_t kOOB = 0xFFFFFFF0u;

struct StreamArgs {
  const uint16_t* x;
  uint32_t K, G, chunks;
  uint32_t waves;         // W: waves per workgroup
  uint32_t n_jobs;
  uint32_t total_blocks;  // blocks of all jobs
  uint32_t wgs;           // workgroups per K part; workgroup g owns blocks [g*B/wgs, (g+1)*B/wgs)
  uint32_t max_blocks;    // largest block count of one workgroup (LDS sizing)
  // K parts: workgroup p * wgs + g covers chunks [p * part_chunks, +part_chunks)
  // of the same blocks as workgroup g.  With parts > 1 each writes its fp32
  // row sums to partials[p][block row], and the last of the parts of a block
  // range to finish (counters[g], zero between launches) adds them in part
  // order and stores the outputs.
  uint32_t parts, part_chunks;
  float* partials;
  unsigned* counters;
  uint32_t M;  // activation rows (x is [M][K]; outputs [M][rows]), at most the kernel's MR
  Q4Job jobs[kMaxQ4Jobs];  // tile_begin = first block of the job
};

__device__ __forceinline__ __amdgpu_buffer_rsrc_t make_rsrc(const void* base, uint64_t bytes) {
  const uint32_t n = bytes > 0xFFFFFFF0ull ? 0xFFFFFFF0u : (uint32_t)bytes;
  return __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(base), (short)0, (int)n, 0x00020000);
}

template <int N>
__device__ __forceinline__ void wait_vmcnt() {
  static_assert(N >= 0 && N < 64, "vmcnt range");
  __builtin_amdgcn_s_waitcnt(0x0F70 | (N & 0xF) | ((N >> 4) << 14));
}

typedef __attribute__((__vector_size__(2 * sizeof(__bf16)))) __bf16 bf16x2;
__device__ __forceinline__ float dot2(uint32_t a, uint32_t b, float c) {
  return __builtin_amdgcn_fdot2_f32_bf16(__builtin_bit_cast(bf16x2, a), __builtin_bit_cast(bf16x2, b), c, false);
}

// Sum over the 16 lanes of a DPP row (every lane of the row gets the sum).
__device__ __forceinline__ float row16_sum(float v) {
  v += __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), 0xB1, 0xF, 0xF, false));   // quad [1,0,3,2]
  v += __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), 0x4E, 0xF, 0xF, false));   // quad [2,3,0,1]
  v += __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), 0x124, 0xF, 0xF, false));  // row_ror:4
  v += __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), 0x128, 0xF, 0xF, false));  // row_ror:8
  return v;
}

__host__ __device__ constexpr uint32_t job_blocks(uint32_t rows, uint32_t mode, int sb) {
  return mode == kQ4OutSwiglu ? (rows + 3) / 4 : (rows + 4 * sb - 1) / (4 * sb);
}
// Scale/bias table entries of one wave (16 bytes each: the 8 groups of one
// chunk of one row): per block SB loads of 4 rows and C chunks.  A wave
// fetches at most kTabEntries of them (kTabLoads loads per lane).
constexpr int kTabLoads = 2;
constexpr uint32_t kTabEntries = 64 * kTabLoads;
__host__ __device__ constexpr uint32_t table_entries(uint32_t blocks, int sb, int c) { return blocks * sb * 4 * c; }
// LDS bytes of one wave's tables: per entry 8 groups of (s, b - 128 s) as fp32.
__host__ __device__ constexpr uint32_t table_bytes(uint32_t blocks, int sb, int c) {
  return table_entries(blocks, sb, c) * 64;
}
// LDS ahead of the tables: every wave's row partials [wave][block][4 SB][MR].
__host__ __device__ constexpr uint32_t head_bytes(uint32_t waves, int sb, uint32_t blocks, uint32_t mr = 1) {
  return waves * blocks * 4 * sb * 4 * mr;
}

// Byte offset, inside a job's tensor, of row `r` of load `s` of block `jb`
// (block index local to the job).
__device__ __forceinline__ uint32_t block_row(uint32_t mode, int sb, uint32_t jb, int s) {
  return mode == kQ4OutSwiglu ? 4 * jb : (4 * sb) * jb + 4 * s;
}

template <int C, int SB, int RB, int MR>
__global__ __launch_bounds__(1024) void q4_stream_kernel(StreamArgs args) {
  extern __shared__ __attribute__((aligned(16))) uint8_t smem[];
  static_assert(MR == 1 || MR == 2, "activation rows");
  constexpr int kPer = SB * C;     // loads per block per wave
  constexpr int kD = kPer * RB;    // ring slots
  const int lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const uint32_t W = args.waves;
  const uint32_t K = args.K, G = args.G;
  const uint32_t row_bytes = K >> 1;
  const int col = lane & 15;
  const int rr = lane >> 4;

  // This workgroup's K part and blocks.
  const uint32_t part = blockIdx.x / args.wgs;
  const uint32_t g = blockIdx.x - part * args.wgs;
  const uint32_t b_begin = (uint32_t)(((uint64_t)g * args.total_blocks) / args.wgs);
  const uint32_t b_end = (uint32_t)(((uint64_t)(g + 1) * args.total_blocks) / args.wgs);
  const uint32_t nblk = b_end - b_begin;

  // LDS: partial slots, then each wave's tables.
  const uint32_t rows_wg = args.max_blocks * 4 * SB;  // partial rows per wave
  float* parts = (float*)smem;                        // [W][max_blocks * 4 SB][MR]
  const uint32_t tab_wave = table_bytes(args.max_blocks, SB, C);
  uint8_t* tab = smem + head_bytes(W, SB, args.max_blocks, MR) + wave * tab_wave;

  // Block -> job (blocks of a job are contiguous).
  auto job_of = [&](uint32_t blk) __attribute__((always_inline)) {
    int j = 0;
    while (j + 1 < (int)args.n_jobs && blk >= args.jobs[j + 1].tile_begin) ++j;
    return j;
  };

  // --- scale / bias tables of the workgroup's rows and this wave's chunks ----
  // Entry e = ((s * nblk + jl) * 4 + r) * C + c holds 16 bytes: 8 groups of
  // chunk c of row r of load s of local block jl (n_e <= kTabEntries entries,
  // the planner's limit).  They are fetched into VGPRs here, ahead of
  // everything else, and written to the wave's LDS tables once the weight
  // ring is in flight (buffer->LDS DMA of the same bytes measured ~4 us
  // slower per launch).
  const uint32_t c0 = part * args.part_chunks + (uint32_t)wave * C;  // first chunk of this wave
  const uint32_t n_e = SB * nblk * 4 * C;
  u32x4 tsv[kTabLoads], tbv[kTabLoads];
#pragma unroll
  for (int i = 0; i < kTabLoads; ++i) {
    const uint32_t e = i * 64 + lane;
    tsv[i] = u32x4{0u, 0u, 0u, 0u};
    tbv[i] = u32x4{0u, 0u, 0u, 0u};
    if (e < n_e) {
      const uint32_t c = e % C, r = (e / C) % 4, t = e / (4 * C);
      const uint32_t sub = t / nblk, jl = t % nblk;
      const uint32_t blk = b_begin + jl;
      const Q4Job& jb = args.jobs[job_of(blk)];
      const bool up = jb.mode == kQ4OutSwiglu && sub == 1;
      const uint16_t* ts = up ? jb.us : jb.s;
      const uint16_t* tb = up ? jb.ub : jb.b;
      const uint32_t row = block_row(jb.mode, SB, blk - jb.tile_begin, (int)sub) + r;
      const uint32_t gcol = (c0 + c) * 8;
      if (row < jb.rows && gcol < G) {
        const size_t idx = (size_t)row * G + gcol;
        if (G % 8 == 0) {  // 16-byte aligned: the entry is 8 whole groups of one row
          tsv[i] = *(const u32x4*)(ts + idx);
          tbv[i] = *(const u32x4*)(tb + idx);
        } else {  // a row's last chunk is partial: element by element, within the row
          uint16_t sv[8], bv[8];
#pragma unroll
          for (int q = 0; q < 8; ++q) {
            const bool in = gcol + q < G;
            sv[q] = in ? ts[idx + q] : (uint16_t)0;
            bv[q] = in ? tb[idx + q] : (uint16_t)0;
          }
          tsv[i] = u32x4{sv[0] | (uint32_t)sv[1] << 16, sv[2] | (uint32_t)sv[3] << 16, sv[4] | (uint32_t)sv[5] << 16,
                         sv[6] | (uint32_t)sv[7] << 16};
          tbv[i] = u32x4{bv[0] | (uint32_t)bv[1] << 16, bv[2] | (uint32_t)bv[3] << 16, bv[4] | (uint32_t)bv[5] << 16,
                         bv[6] | (uint32_t)bv[7] << 16};
        }
      }
    }
  }
  __builtin_amdgcn_sched_barrier(0);  // the tables are issued before everything else

  // --- activation chunks in registers ----------------------------------------
  // Lane (col) holds elements [chunk*512 + 32 col, +32), each 8-element run in
  // the unpack order (x0,x4)(x1,x5)(x2,x6)(x3,x7).
  u32x4 xr[MR][C][4];
  float xsum[MR][C];
  bool valid[C];
  {
#pragma unroll
    for (int c = 0; c < C; ++c) {
      const uint32_t e0 = (c0 + c) * kChunkElems + 32 * col;
      valid[c] = c0 + c < args.chunks && e0 < K;
    }
#pragma unroll
    for (int m = 0; m < MR; ++m) {
      // Rows past M read nothing (a zero-length resource) and stay zero.
      const __amdgpu_buffer_rsrc_t rx =
          make_rsrc(args.x + (size_t)min((uint32_t)m, args.M - 1) * K, (uint32_t)m < args.M ? (uint64_t)K * 2 : 0);
#pragma unroll
      for (int c = 0; c < C; ++c) {
        const uint32_t e0 = (c0 + c) * kChunkElems + 32 * col;
#pragma unroll
        for (int q = 0; q < 4; ++q)
          xr[m][c][q] = __builtin_amdgcn_raw_buffer_load_b128(rx, valid[c] ? e0 * 2 + 16 * q : kOOB, 0, 0);
      }
    }
  }
  __builtin_amdgcn_sched_barrier(0);

  // --- weight ring -------------------------------------------------------------
  // Slot t of a round: local block jl = t / kPer, load s = (t / C) % SB, chunk
  // c = t % C.  voff[c]: this lane's byte offset inside a 4-row load.
  uint32_t voff[C];
#pragma unroll
  for (int c = 0; c < C; ++c) voff[c] = (c0 + c < args.chunks) ? rr * row_bytes + (c0 + c) * 256 + 16 * col : kOOB;

  // The job of the next block to load (blocks are loaded in increasing
  // order): its fields stay in scalar registers until the cursor passes the
  // job's last block, so a load needs no kernel-argument reads.
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
  auto load_w = [&](uint32_t jl, int s, int c) __attribute__((always_inline)) {
    // jl: local block (dead past nblk: no bytes)
    const uint32_t blk = b_begin + jl;
    // Every job has at least one block, so one step moves at most one job on.
    if (jl < nblk && blk >= cj_end) {
      ++cj;
      set_job();
    }
    // Branch-free (selects only), so the load stays in one basic block.
    const bool live = (jl < nblk) & (b_begin + jl - cj_begin < (1u << 30));
    const bool up = (c_mode == kQ4OutSwiglu) & (s == 1);
    const uint32_t* w = up ? c_uw : c_w;
    const uint32_t base_row = live ? block_row(c_mode, SB, blk - cj_begin, s) : 0;
    const uint32_t left = (live & (base_row < c_rows)) ? c_rows - base_row : 0;
    const uint32_t avail = left >= 0xFFFFFFF0u / row_bytes ? 0xFFFFFFF0u : left * row_bytes;
    const __amdgpu_buffer_rsrc_t r = __builtin_amdgcn_make_buffer_rsrc(
        const_cast<uint32_t*>(w + (size_t)base_row * (row_bytes / 4)), (short)0, (int)avail, 0x00020000);
    return __builtin_amdgcn_raw_buffer_load_b128(r, voff[c], 0, kNonTemporal);
  };

  u32x4 ring[kD];
  const uint32_t nrounds = (nblk + RB - 1) / RB;
#pragma unroll
  for (int t = 0; t < kD; ++t) {
    ring[t] = load_w(t / kPer, (t / C) % SB, t % C);
    __builtin_amdgcn_sched_barrier(0);
  }
  // Tables into LDS (their loads were issued first): per group the fp32
  // pair (s, b - 128 s) that a lane's contribution needs.
#pragma unroll
  for (int i = 0; i < kTabLoads; ++i) {
    const uint32_t e = i * 64 + lane;
    if (e < n_e) {
      float* te = (float*)(tab + e * 64);
      const uint32_t sw[4] = {tsv[i].x, tsv[i].y, tsv[i].z, tsv[i].w};
      const uint32_t bw[4] = {tbv[i].x, tbv[i].y, tbv[i].z, tbv[i].w};
#pragma unroll
      for (int q = 0; q < 4; ++q) {
        const float s0 = bf16_to_f32(sw[q] & 0xFFFF), s1 = bf16_to_f32(sw[q] >> 16);
        const float b0 = bf16_to_f32(bw[q] & 0xFFFF), b1 = bf16_to_f32(bw[q] >> 16);
        *(floatx4*)(te + 4 * q) = floatx4{s0, fmaf(-128.0f, s0, b0), s1, fmaf(-128.0f, s1, b1)};
      }
    }
  }
#pragma unroll
  for (int m = 0; m < MR; ++m)
#pragma unroll
    for (int c = 0; c < C; ++c) {
#pragma unroll
      for (int q = 0; q < 4; ++q) xr[m][c][q] = interleave_bf16x8(xr[m][c][q]);
      float sum = 0.f;
#pragma unroll
      for (int q = 0; q < 4; ++q) {
        sum += bf16_to_f32(xr[m][c][q].x & 0xFFFF) + bf16_to_f32(xr[m][c][q].x >> 16);
        sum += bf16_to_f32(xr[m][c][q].y & 0xFFFF) + bf16_to_f32(xr[m][c][q].y >> 16);
        sum += bf16_to_f32(xr[m][c][q].z & 0xFFFF) + bf16_to_f32(xr[m][c][q].z >> 16);
        sum += bf16_to_f32(xr[m][c][q].w & 0xFFFF) + bf16_to_f32(xr[m][c][q].w >> 16);
      }
      xsum[m][c] = sum;
    }

  const uint32_t mask_s = __builtin_amdgcn_readfirstlane(0x000F000Fu);
  uint32_t or_v = 0x43004300u;
  asm volatile("" : "+v"(or_v));

  // One slot: the lane's contribution s*p + (b - 128 s)*X for its row/chunk.
  // Lanes past K see x = 0, X = 0 and a zero table entry: they add 0.
  const uint32_t tlane = rr * C * 64 + (col >> 1) * 8;
  auto consume = [&](const u32x4& wv, uint32_t jl, int s, int c, float (&acc)[MR]) __attribute__((always_inline)) {
    const uint32_t e0 = ((s * nblk + jl) * 4) * C + c;  // entry of row 0 of the load
    const u32x2 tv = *(const u32x2*)(tab + e0 * 64 + tlane);
    const float sc = __uint_as_float(tv.x), cb = __uint_as_float(tv.y);
    float p0[MR], p1[MR];
#pragma unroll
    for (int m = 0; m < MR; ++m) p0[m] = p1[m] = 0.f;
#pragma unroll
    for (int q = 0; q < 4; ++q) {
      const uint32_t wq = q == 0 ? wv.x : q == 1 ? wv.y : q == 2 ? wv.z : wv.w;
      const uint32_t u0 = (wq & mask_s) | or_v, u1 = ((wq >> 4) & mask_s) | or_v;
      const uint32_t u2 = ((wq >> 8) & mask_s) | or_v, u3 = ((wq >> 12) & mask_s) | or_v;
#pragma unroll
      for (int m = 0; m < MR; ++m) {
        const u32x4 xq = xr[m][c][q];
        p0[m] = dot2(u0, xq.x, p0[m]);
        p1[m] = dot2(u1, xq.y, p1[m]);
        p0[m] = dot2(u2, xq.z, p0[m]);
        p1[m] = dot2(u3, xq.w, p1[m]);
      }
    }
#pragma unroll
    for (int m = 0; m < MR; ++m) acc[m] += fmaf(sc, p0[m] + p1[m], cb * xsum[m][c]);
  };

  // A finished block: each row's sum over this wave's chunks (the 16 lanes of
  // the row) goes to the wave's partial row; the waves' partials are added
  // in wave order after the stream (deterministic, no synchronisation here).
  auto finish_block = [&](uint32_t jl, const float (&acc)[SB][MR]) __attribute__((always_inline)) {
#pragma unroll
    for (int s = 0; s < SB; ++s)
#pragma unroll
      for (int m = 0; m < MR; ++m) {
        const float v = row16_sum(acc[s][m]);
        if (col == 0) parts[(wave * rows_wg + jl * 4 * SB + s * 4 + rr) * MR + m] = v;
      }
  };

  auto round = [&](uint32_t r, bool refill) __attribute__((always_inline)) {
#pragma unroll
    for (int bi = 0; bi < RB; ++bi) {
      const uint32_t jl = r * RB + bi;
      float acc[SB][MR];
#pragma unroll
      for (int s = 0; s < SB; ++s)
#pragma unroll
        for (int m = 0; m < MR; ++m) acc[s][m] = 0.f;
#pragma unroll
      for (int s = 0; s < SB; ++s)
#pragma unroll
        for (int c = 0; c < C; ++c) {
          const int t = bi * kPer + s * C + c;
          consume(ring[t], jl, s, c, acc[s]);
          if (refill) {
            // The slot's math is done before its refill is issued (an IR-level
            // barrier too, so the math is not sunk below the load, which would
            // keep both register sets alive and copy the ring every round).
#pragma unroll
            for (int m = 0; m < MR; ++m) asm volatile("" : "+v"(acc[s][m]) : : "memory");
            __builtin_amdgcn_sched_barrier(0);
            ring[t] = load_w(jl + RB, s, c);
            __builtin_amdgcn_sched_barrier(0);
          }
        }
      if (jl < nblk) finish_block(jl, acc);
    }
  };
  if (nrounds > 0) {
    uint32_t r = 0;
    for (; r + 1 < nrounds; ++r) round(r, true);
    round(r, false);
  }

  // --- outputs -----------------------------------------------------------------
  lds_barrier();
  const uint32_t rows_per_block = 4 * SB;
  const uint32_t nrows = nblk * rows_per_block;
  const uint32_t nvals = nrows * MR;  // value f = (local row) * MR + activation row
  // Value f of the workgroup (local block f / (4SB MR), weight row
  // (f / MR) % 4SB, activation row f % MR) over this workgroup's chunks: its
  // waves' partials in wave order.
  auto row_sum = [&](uint32_t f) __attribute__((always_inline)) {
    float v = 0.f;
    for (uint32_t w2 = 0; w2 < W; ++w2) v += parts[w2 * rows_wg * MR + f];
    return v;
  };
  const uint32_t TB = args.total_blocks * rows_per_block * MR;  // partial values per K part
  float* pp = args.partials + (size_t)b_begin * rows_per_block * MR;
  // Row i over all K parts, in part order (the same sum whichever part
  // finishes last).
  // The partial rows and the counter are accessed as device-scope relaxed
  // atomics: each access is coherent across the XCDs' L2 caches by itself,
  // with no whole-cache write-back or invalidate (acquire/release fences at
  // device scope cost ~30 us over a launch of 768 workgroups).  The counter
  // is bumped only after the barrier, by which point every wave's partial
  // stores have completed.
  auto part_sum = [&](uint32_t i) __attribute__((always_inline)) {
    float v = 0.f;
    for (uint32_t q = 0; q < args.parts; ++q)
      v += __hip_atomic_load(&pp[(size_t)q * TB + i], __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    return v;
  };
  if (args.parts > 1) {
    for (uint32_t f = threadIdx.x; f < nvals; f += blockDim.x)
      __hip_atomic_store(&pp[(size_t)part * TB + f], row_sum(f), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    __builtin_amdgcn_s_waitcnt(0);  // this wave's stores have completed
    __syncthreads();
    __shared__ uint32_t last;
    if (threadIdx.x == 0) {
      const uint32_t old = __hip_atomic_fetch_add(&args.counters[g], 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
      last = old == args.parts - 1;
      if (last) __hip_atomic_store(&args.counters[g], 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    }
    __syncthreads();
    if (!last) return;
  }
  auto value = [&](uint32_t i) __attribute__((always_inline)) {
    return args.parts > 1 ? part_sum(i) : row_sum(i);
  };
  unsigned long long best = 0;  // argmax key of this thread's rows (MR = 1)
  for (uint32_t f = threadIdx.x; f < nvals; f += blockDim.x) {
    const uint32_t i = f / MR, m = f % MR;
    if (m >= args.M) continue;
    const uint32_t jl = i / rows_per_block, k = i % rows_per_block;
    const uint32_t blk = b_begin + jl;
    const int j = job_of(blk);
    const Q4Job& jb = args.jobs[j];
    const uint32_t lb = blk - jb.tile_begin;
    if (jb.mode == kQ4OutSwiglu) {
      // k < 4: gate sums; k >= 4: the up sums of the same rows.
      const uint32_t row = 4 * lb + k;
      if (k < 4 && row < jb.rows) {
        const float gsum = value((jl * rows_per_block + k) * MR + m);
        const float usum = value((jl * rows_per_block + 4 + k) * MR + m);
        jb.out[(size_t)m * jb.rows + row] = f32_to_bf16(silu_f(gsum) * usum);
      }
      continue;
    }
    const uint32_t row = rows_per_block * lb + k;
    if (row >= jb.rows) continue;
    const float v = value(f);
    if (jb.mode == kQ4OutArgmax) {
      if (!__builtin_isnan(v)) {
        const uint32_t bits = v == 0.0f ? 0u : __float_as_uint(v);
        const uint32_t ord = (bits & 0x80000000u) ? ~bits : (bits | 0x80000000u);
        const unsigned long long key = ((unsigned long long)ord << 32) | (0xFFFFFFFFu - row);
        best = key > best ? key : best;
      }
      continue;
    }
    const uint16_t h = f32_to_bf16(v);
    const size_t o = (size_t)m * jb.rows + row;
    if (jb.mode == kQ4OutBf16)
      jb.out[o] = h;
    else if (jb.mode == kQ4OutF32)
      ((float*)jb.out)[o] = bf16_to_f32(h);
    else
      ((float*)jb.out)[o] += bf16_to_f32(h);
  }
  if (MR == 1 && args.jobs[0].mode == kQ4OutArgmax) {
    // One atomic per wave: the best key of its threads' rows.
#pragma unroll
    for (int off = 32; off >= 1; off >>= 1) {
      const unsigned long long o = __shfl_xor(best, off);
      best = o > best ? o : best;
    }
    if (lane == 0 && best) atomicMax((unsigned long long*)args.jobs[0].out, best);
  }
}

// Ring: 8 loads in flight per wave.
template <int C, int SB, int MR = 1>
const void* kernel_for() {
  constexpr int kRB = (8 / (SB * C)) > 1 ? 8 / (SB * C) : 1;
  return (const void*)q4_stream_kernel<C, SB, kRB, MR>;
}
const void* pick_kernel(int c, int sb, int mr = 1) {
  if (mr == 2) return c == 1 ? (sb == 2 ? kernel_for<1, 2, 2>() : kernel_for<1, 1, 2>()) : nullptr;
  if (c == 1) return sb == 2 ? kernel_for<1, 2>() : kernel_for<1, 1>();
  if (c == 2) return sb == 2 ? kernel_for<2, 2>() : kernel_for<2, 1>();
  if (c == 3) return sb == 1 ? kernel_for<3, 1>() : kernel_for<3, 2>();
  if (c == 4) return sb == 1 ? kernel_for<4, 1>() : nullptr;
  return nullptr;
}

// One K part: up to 16 waves of 2 chunks (K <= 16384), or for plain jobs of
// 3 chunks (K <= 24576; measured on the 17408-wide down projection: 13 us
// against 17 us split in parts).  Longer K runs in parts of 5 waves of 2
// chunks whose fp32 row sums the last part adds.
constexpr uint32_t kPartWaves = 5, kPartC = 2, kOnePartMax = 32, kOnePartMax3 = 48, kRowsWaves = 8;

struct StreamPlan {
  const void* fn = nullptr;
  uint32_t waves = 0, C = 0, SB = 0, MR = 1, wgs = 0, max_blocks = 0, lds = 0, total_blocks = 0;
  uint32_t parts = 1, part_chunks = 0;
  size_t partial_bytes = 0, counters = 0;
};

StreamPlan make_stream_plan(const Q4Job* jobs, int n_jobs, uint32_t K, uint32_t M, const Tuning& tn) {
  StreamPlan p{};
  const uint32_t chunks = (K + kChunkElems - 1) / kChunkElems;
  bool pair = false;
  for (int i = 0; i < n_jobs; ++i) pair |= jobs[i].mode == kQ4OutSwiglu;
  p.MR = M <= 1 ? 1 : 2;
  if (p.MR > 1) {
    // Two activation rows: one chunk per wave (each row's chunk takes 16
    // VGPRs), K in balanced parts of at most kRowsWaves waves, so that
    // several workgroups share a CU (measured at M = 2, 17408 wide: 19.4 us
    // with 7-wave parts against 20.0 with 5-wave and 19.7 with 9-wave parts).
    const uint32_t wmax = tn.q4_stream_mw > 0 ? std::min<uint32_t>(tn.q4_stream_mw, kMaxWaves) : kRowsWaves;
    p.C = 1;
    p.parts = (chunks + wmax - 1) / wmax;
    p.waves = (chunks + p.parts - 1) / p.parts;
  } else if (chunks <= kOnePartMax) {
    // Two chunks per wave even when one would do: fewer waves per workgroup,
    // more workgroups per CU and each block's per-row work over twice the
    // bytes (measured: QKV + gate/up set 32 -> 28 us).
    p.C = chunks > 1 ? 2 : 1;
    p.waves = (chunks + p.C - 1) / p.C;
    p.parts = 1;
  } else if (chunks <= kOnePartMax3 && !pair) {
    p.C = 3;
    p.waves = (chunks + 2) / 3;
    p.parts = 1;
  } else {
    p.C = kPartC;
    p.waves = kPartWaves;
    p.parts = (chunks + kPartWaves * kPartC - 1) / (kPartWaves * kPartC);
  }
  if (tn.q4_stream_c > 0 && p.MR == 1) {  // forced chunks per wave (and waves per part)
    p.C = (uint32_t)tn.q4_stream_c;
    p.waves = tn.q4_stream_w > 0 ? (uint32_t)tn.q4_stream_w : std::min<uint32_t>(kMaxWaves, (chunks + p.C - 1) / p.C);
    p.parts = (chunks + p.waves * p.C - 1) / (p.waves * p.C);
  }
  p.part_chunks = p.waves * p.C;
  p.SB = pair ? 2 : 1;
  for (int i = 0; i < n_jobs; ++i) p.total_blocks += job_blocks(jobs[i].rows, jobs[i].mode, p.SB);
  p.fn = p.waves >= 1 && p.waves <= (uint32_t)kMaxWaves ? pick_kernel((int)p.C, (int)p.SB, (int)p.MR) : nullptr;
  if (!p.fn) return p;
  const uint32_t cus = tn.cus > 0 ? (uint32_t)tn.cus : 256;
  // Workgroups: as many as stay resident (one dispatch round), with at most
  // `cap` blocks each (the table entries a wave fetches); more workgroups,
  // in several rounds, only when the blocks exceed resident * cap.
  const uint32_t cap = kTabEntries / table_entries(1, (int)p.SB, (int)p.C);
  const uint32_t lds_cap = head_bytes(p.waves, p.SB, cap, p.MR) + p.waves * table_bytes(cap, p.SB, p.C);
  int occ = 0;
  if (hipOccupancyMaxActiveBlocksPerMultiprocessor(&occ, p.fn, (int)(64 * p.waves), lds_cap) != hipSuccess || occ <= 0) {
    p.fn = nullptr;
    return p;
  }
  const uint32_t resident = std::max<uint32_t>(1, (uint32_t)occ * cus / p.parts);
  const uint32_t wgs_min = (p.total_blocks + cap - 1) / cap;
  // At least two blocks per workgroup: a workgroup's fixed part (table and
  // activation loads, the partial-sum exchange) over one block of a small
  // projection costs more than the fuller dispatch gains (4096 x 4096: 7.2 us
  // with 1024 one-block workgroups, 5.8 us with 512; 4096 -> 5120: 7.9 / 5.9).
  p.wgs = std::max(wgs_min, std::min((p.total_blocks + 1) / 2, resident));
  if (tn.q4_stream_wgs > 0) p.wgs = std::max(wgs_min, std::min(p.total_blocks, (uint32_t)tn.q4_stream_wgs));
  p.max_blocks = (p.total_blocks + p.wgs - 1) / p.wgs;
  p.lds = head_bytes(p.waves, p.SB, p.max_blocks, p.MR) + p.waves * table_bytes(p.max_blocks, p.SB, p.C);
  if (p.parts > 1) {
    p.partial_bytes = (size_t)p.parts * p.total_blocks * 4 * p.SB * p.MR * sizeof(float);
    p.counters = p.wgs;
  }
  if (tn.q4_plan_log > 0)
    fprintf(stderr,
            "q4 stream plan: K=%u M=%u jobs=%d blocks=%u C=%u SB=%u waves=%u parts=%u wgs/part=%u max_blocks=%u lds=%u\n",
            K, M, n_jobs, p.total_blocks, p.C, p.SB, p.waves, p.parts, p.wgs, p.max_blocks, p.lds);
  return p;
}

struct StreamKey {
  uint32_t rows[kMaxQ4Jobs], modes[kMaxQ4Jobs];
  int n_jobs;
  uint32_t K, M;
  Tuning tune;
  bool operator==(const StreamKey& o) const { return std::memcmp(this, &o, sizeof(*this)) == 0; }
};

StreamPlan cached_stream_plan(const Q4Job* jobs, int n_jobs, uint32_t K, uint32_t M, const Tuning& tn) {
  static std::mutex mu;
  static StreamKey keys[16];
  static StreamPlan plans[16];
  static int used = 0, next = 0;
  StreamKey k;
  std::memset(&k, 0, sizeof(k));
  for (int i = 0; i < n_jobs; ++i) {
    k.rows[i] = jobs[i].rows;
    k.modes[i] = jobs[i].mode == kQ4OutSwiglu ? 1 : 0;
  }
  k.n_jobs = n_jobs;
  k.K = K;
  k.M = M;
  k.tune = tn;
  std::lock_guard<std::mutex> lock(mu);
  for (int i = 0; i < used; ++i)
    if (keys[i] == k) return plans[i];
  const StreamPlan p = make_stream_plan(jobs, n_jobs, K, M, tn);
  keys[next] = k;
  plans[next] = p;
  next = (next + 1) % 16;
  used = std::min(used + 1, 16);
  return p;
}

}  // namespace

bool q4_stream_supported(const Q4Job* jobs, int n_jobs, uint32_t K, uint32_t M, const Tuning& tn) {
  if (M < 1 || M > (uint32_t)std::min(tn.q4_stream_rows, 2) || tn.q4_stream == 0 || n_jobs < 1 ||
      n_jobs > kMaxQ4Jobs)
    return false;
  for (int i = 0; i < n_jobs; ++i)
    if (jobs[i].mode > kQ4OutSwiglu || (jobs[i].mode == kQ4OutArgmax && (n_jobs > 1 || M > 1))) return false;
  return cached_stream_plan(jobs, n_jobs, K, M, tn).fn != nullptr;
}

void q4_stream_workspace(const Q4Job* jobs, int n_jobs, uint32_t K, uint32_t M, const Tuning& tn,
                         size_t* partial_bytes, size_t* counters) {
  const StreamPlan p = cached_stream_plan(jobs, n_jobs, K, M, tn);
  *partial_bytes = p.partial_bytes;
  *counters = p.counters;
}

hipError_t launch_q4_stream(const Q4Job* jobs, int n_jobs, const uint16_t* x, uint32_t K, uint32_t M,
                            const Workspace& ws, hipStream_t stream) {
  if (!ws.tune || n_jobs < 1 || n_jobs > kMaxQ4Jobs || M < 1 || M > 2) return hipErrorInvalidValue;
  const StreamPlan p = cached_stream_plan(jobs, n_jobs, K, M, *ws.tune);
  if (!p.fn) return hipErrorInvalidValue;
  if (p.parts > 1 && (!ws.partials || ws.partial_bytes < p.partial_bytes || !ws.counters ||
                      ws.counter_count < p.counters))
    return hipErrorInvalidValue;
  StreamArgs a{};
  a.x = x;
  a.K = K;
  a.G = K / 64;
  a.chunks = (K + kChunkElems - 1) / kChunkElems;
  a.waves = p.waves;
  a.n_jobs = (uint32_t)n_jobs;
  a.total_blocks = p.total_blocks;
  a.wgs = p.wgs;
  a.max_blocks = p.max_blocks;
  a.parts = p.parts;
  a.part_chunks = p.part_chunks;
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
