// Q4 prefill projection (M > 16 rows): Y[M][N] = X[M][K] * dequant(W)^T.
//
// Numerics follow the reference's prefill path (qwen38_q4_affine_dequantize_f16
// + fp16 MPS GEMM, /root/reference/shaders/qwen38.metal:4102-4125,
// src/metal_runtime.rs:3897-4048): weights become fp16(q*s + b), activations
// fp16, products accumulate in fp32; the result is stored as bf16.
//
// Two kernels:
//  * x_to_f16_kernel: X (bf16) -> Xh (fp16), once per call.  Within every
//    8-element chunk the elements are stored in the order 0,4,1,5,2,6,3,7,
//    the order in which one packed Q4 word unpacks into fp16 pairs, so the
//    GEMM's dequantised B tile and the A tile agree element by element.
//  * q4_gemm_kernel: 256 x 256 output tile per workgroup (512 threads,
//    8 waves as 4 (M) x 2 (N), 64 x 128 per wave on v_mfma_f32_32x32x16_f16),
//    K in steps of one quantisation group (64).  Per step each thread loads
//    16 B of X and 16 B of packed W, dequantises its four words with
//    (w >> 4j & 0x000F000F) | 0x64006400 (fp16 1024 + q), one packed subtract
//    and one packed FMA per pair, and writes both tiles into the other half
//    of a double-buffered LDS (2 x 64 KiB) while the waves multiply the
//    current half: one barrier per K step.
//    SwiGLU: the 256 W rows of a tile are 128 gate rows and the same 128 up
//    rows, each wave holding gate and up accumulators of the same outputs, so
//    h = silu(gate) * up is formed in registers.
//    Tile order is XCD-aware: workgroups are dealt round-robin to the 8 XCDs,
//    so the tile index is remapped to give each XCD a contiguous run of N
//    tiles with all of their M tiles (W is read from HBM once per XCD and
//    stays in that XCD's L2 while its M tiles pass).
//    Split-K when the tiles alone would leave CUs idle (small M, or few N
//    tiles): each workgroup takes one K slice of a tile and writes its fp32
//    accumulators through to memory; the last slice of the tile to finish (a
//    per-tile counter it resets) adds the slices in slice order, so the sum
//    does not depend on timing, and runs the epilogue.
#include "common.h"
#include "internal.h"

namespace qm {
namespace {

typedef _Float16 half8 __attribute__((ext_vector_type(8)));
typedef _Float16 half2v __attribute__((ext_vector_type(2)));

constexpr int kBM = 256, kBN = 256, kThreads = 512;
constexpr int kTileBytes = 256 * 128;  // 256 rows x 64 fp16
constexpr int kXcds = 8;

struct GemmArgs {
  Q4Job jobs[kMaxQ4Jobs];
  int n_jobs;
  const uint16_t* xh;  // fp16 bits [M][K], chunk-permuted
  uint32_t K, M;
  uint32_t m_tiles, total_tiles;
  // Work assignment over the flattened K steps (step L G + g is group g of
  // tile L).  splits == 1: worker w runs steps [w Q, (w + 1) Q) (Q = G: one
  // tile each; Q > G: stream-K, ranges crossing tile boundaries).  splits > 1:
  // worker w runs slice w % splits (Q steps) of tile w / splits.
  uint32_t q_steps, splits;
  uint32_t workers;
  float* partials;       // fp32 pieces, kThreads * 128 floats per slot

  unsigned* counters;    // [tile], zero between launches
};

constexpr uint32_t kPieceFloats = kThreads * 128;  // one 256 x 256 fp32 tile

// Piece slot of worker w in tile L (splits == 1): 2w for the first tile of
// w's range, 2w + 1 for the last one (a range cuts at most two tiles).
__device__ __forceinline__ uint32_t piece_slot(uint32_t w, uint32_t L, uint32_t Q, uint32_t G) {
  return 2 * w + (L != (w * Q) / G ? 1u : 0u);
}

// s_waitcnt vmcnt(0) (gfx9 encoding; expcnt and lgkmcnt left at their maxima).
__device__ __forceinline__ void wait_vmcnt0() { __builtin_amdgcn_s_waitcnt(0x0F70); }

// Byte offset of 16-byte chunk c (0..7) of row r in a 256 x 128 B tile.  The
// XOR spreads the 16 rows one ds_read_b128 phase touches over distinct banks.
__device__ __forceinline__ uint32_t swz(uint32_t r, uint32_t c) {
  return r * 128u + 16u * (c ^ (r & 7u) ^ ((r >> 3) & 1u));
}

__device__ __forceinline__ __amdgpu_buffer_rsrc_t make_rsrc(const void* base, uint64_t bytes) {
  const uint32_t n = bytes > 0xFFFFFFF0ull ? 0xFFFFFFF0u : (uint32_t)bytes;
  return __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(base), (short)0, (int)n, 0x00020000);
}

__device__ __forceinline__ floatx16 mfma_f16(u32x4 a, u32x4 b, floatx16 c) {
  return __builtin_amdgcn_mfma_f32_32x32x16_f16(__builtin_bit_cast(half8, a), __builtin_bit_cast(half8, b), c, 0,
                                                0, 0);
}

__device__ __forceinline__ uint32_t dq_pair(uint32_t w, int j, half2v s2, half2v b2) {
  const uint32_t t = ((w >> (4 * j)) & 0x000F000Fu) | 0x64006400u;
  half2v q = __builtin_bit_cast(half2v, t) - (half2v){(_Float16)1024.0f, (_Float16)1024.0f};
  return __builtin_bit_cast(uint32_t, q * s2 + b2);
}

__global__ __launch_bounds__(256) void x_to_f16_kernel(const uint16_t* __restrict__ x, uint16_t* __restrict__ xh,
                                                       size_t chunks) {
  const size_t i = (size_t)blockIdx.x * 256 + threadIdx.x;
  if (i >= chunks) return;
  const u32x4 v = *(const u32x4*)(x + 8 * i);
  // v holds bf16 pairs (x0,x1)(x2,x3)(x4,x5)(x6,x7); emit 0,4,1,5,2,6,3,7.
  const uint32_t e[8] = {v.x & 0xFFFFu, v.x >> 16, v.y & 0xFFFFu, v.y >> 16,
                         v.z & 0xFFFFu, v.z >> 16, v.w & 0xFFFFu, v.w >> 16};
  uint32_t h[8];
#pragma unroll
  for (int k = 0; k < 8; ++k) {
    // Saturate to the fp16 range: a bf16 activation beyond +-65504 becomes
    // +-65504 rather than an infinity that would poison the whole output row
    // (NaN compares false both ways and passes through as NaN).
    float v = bf16_to_f32(e[k]);
    v = v > 65504.0f ? 65504.0f : (v < -65504.0f ? -65504.0f : v);
    const _Float16 f = (_Float16)v;
    h[k] = __builtin_bit_cast(uint16_t, f);
  }
  u32x4 o;
  o.x = h[0] | (h[4] << 16);
  o.y = h[1] | (h[5] << 16);
  o.z = h[2] | (h[6] << 16);
  o.w = h[3] | (h[7] << 16);
  *(u32x4*)(xh + 8 * i) = o;
}

// Jobs are plain projections (256 W rows per tile) or SwiGLU pairs (mode
// kQ4OutSwiglu: 128 gate rows from w/s/b and the same 128 up rows from
// uw/us/ub per tile, h = silu(gate) * up in the epilogue); one launch may mix
// them (a same-input set).  Whether a tile is a pair is uniform over a piece,
// so it only changes the piece's row mapping and epilogue.
__global__ __launch_bounds__(kThreads) void q4_gemm_kernel(GemmArgs args) {
  __shared__ __attribute__((aligned(16))) uint8_t lds[2][2][kTileBytes];  // [stage][X | W]
  __shared__ unsigned last;

  const uint32_t tid = threadIdx.x;
  const uint32_t lane = tid & 63;
  const uint32_t wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const uint32_t wm = wave & 3, wn = wave >> 2;
  const uint32_t K = args.K, M = args.M, G = K / 64, Q = args.q_steps, S = args.splits;
  const uint32_t total = args.total_tiles * G;

  // ---- XCD-aware worker remap ---------------------------------------------
  // Workgroups are dealt round-robin to the XCDs; each XCD gets a contiguous
  // run of workers, so the tiles it covers are contiguous (n-major, m inner)
  // and every W tile is read from HBM once per XCD, then from its L2.
  const uint32_t W = args.workers;
  const uint32_t xcd = blockIdx.x % kXcds, local = blockIdx.x / kXcds;
  const uint32_t wq = W / kXcds, wrem = W % kXcds;
  const uint32_t lw = xcd * wq + min(xcd, wrem) + local;
  uint32_t step0, s_end;
  if (S > 1) {
    const uint32_t L = lw / S;
    step0 = L * G + (lw - L * S) * Q;
    s_end = min(step0 + Q, (L + 1) * G);
  } else {
    step0 = lw * Q;
    s_end = min(total, step0 + Q);
  }

  const uint32_t arow0 = 64 * wm + (lane & 31);
  const uint32_t kh = lane >> 5;
  const uint32_t srow = tid >> 1, shalf = tid & 1;  // staging: row of the tiles, chunk half

  for (uint32_t step = step0; step < s_end;) {
    // Uniform values: readfirstlane keeps them (and the buffer offsets built
    // from them) in SGPRs; a VGPR offset would turn every partial-piece store
    // and load into a waterfall loop.
    const uint32_t L = __builtin_amdgcn_readfirstlane(step / G), g0 = step - L * G;
    const uint32_t NG = min(G - g0, s_end - step);  // K steps of this piece (>= 1)
    step += NG;
    const uint32_t n_tile = L / args.m_tiles, m_tile = L % args.m_tiles;
    const uint32_t m0 = m_tile * kBM;

    // ---- this thread's W row and the tile's job ----------------------------
    int jt = 0;
    while (jt + 1 < args.n_jobs && n_tile >= args.jobs[jt + 1].tile_begin) ++jt;
    const Q4Job& jb = args.jobs[jt];
    const bool pair = jb.mode == kQ4OutSwiglu;
    // A pair tile's W rows 128..255 (srow >= 128 <=> wave >= 4) are the up rows.
    const bool upper = pair && wave >= 4;
    const uint32_t n_first = (n_tile - jb.tile_begin) * (pair ? 128u : kBN);
    const uint32_t wrow = min(n_first + (pair ? (srow & 127) : srow), jb.rows - 1);
    // The weight resource starts at the tile's first row, so the 32-bit
    // offsets stay in range whatever the matrix size.
    const uint32_t* w_tile = (upper ? jb.uw : jb.w) + (size_t)n_first * (K / 8);
    const __amdgpu_buffer_rsrc_t rw = make_rsrc(w_tile, (uint64_t)(jb.rows - n_first) * (K / 2));
    const uint16_t* s_row = (upper ? jb.us : jb.s) + (size_t)wrow * G;
    const uint16_t* b_row = (upper ? jb.ub : jb.b) + (size_t)wrow * G;
    // B-tile row bases of this wave's four 32-column blocks (a pair: gate
    // columns in blocks 0, 1 and the matching up columns in blocks 2, 3).
    uint32_t brow[4];
#pragma unroll
    for (int j = 0; j < 4; ++j)
      brow[j] = pair ? (j < 2 ? 64 * wn + 32 * j : 128 + 64 * wn + 32 * (j - 2)) : 128 * wn + 32 * j;
    const uint32_t w_voff = (wrow - n_first) * (K / 2) + shalf * 16;
    const uint32_t xrow = min(m0 + srow, M - 1);
    const uint16_t* x_src = args.xh + (size_t)xrow * K + shalf * 32;

    // ---- staging registers -------------------------------------------------
    u32x4 xr[4];
    u32x4 wr;
    uint16_t sr, br;
    auto load = [&](uint32_t g) {
#pragma unroll
      for (int i = 0; i < 4; ++i) xr[i] = *(const u32x4*)(x_src + g * 64 + 8 * i);
      wr = __builtin_amdgcn_raw_buffer_load_b128(rw, w_voff, g * 32, 0);
      sr = s_row[g];
      br = b_row[g];
    };
    auto store = [&](int stage) {
      uint8_t* xt = lds[stage][0];
      uint8_t* wt = lds[stage][1];
#pragma unroll
      for (int i = 0; i < 4; ++i) *(u32x4*)(xt + swz(srow, shalf * 4 + i)) = xr[i];
      const _Float16 s = (_Float16)bf16_to_f32(sr), b = (_Float16)bf16_to_f32(br);
      const half2v s2 = {s, s}, b2 = {b, b};
      const uint32_t wv[4] = {wr.x, wr.y, wr.z, wr.w};
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        u32x4 d;
        d.x = dq_pair(wv[i], 0, s2, b2);
        d.y = dq_pair(wv[i], 1, s2, b2);
        d.z = dq_pair(wv[i], 2, s2, b2);
        d.w = dq_pair(wv[i], 3, s2, b2);
        *(u32x4*)(wt + swz(srow, shalf * 4 + i)) = d;
      }
    };

    floatx16 acc[2][4];
#pragma unroll
    for (int i = 0; i < 2; ++i)
#pragma unroll
      for (int j = 0; j < 4; ++j) acc[i][j] = floatx16{};

    // The previous piece's last step ended on a barrier: both stages are free.
    load(g0);
    store(0);
    load(g0 + min(1u, NG - 1));
    __syncthreads();

    for (uint32_t i = 0; i < NG; ++i) {
      const int st = i & 1;
      const uint8_t* xt = lds[st][0];
      const uint8_t* wt = lds[st][1];
#pragma unroll
      for (int s = 0; s < 4; ++s) {
        const uint32_t c = 2 * s + kh;
        u32x4 a[2], b[4];
#pragma unroll
        for (int i = 0; i < 2; ++i) a[i] = *(const u32x4*)(xt + swz(arow0 + 32 * i, c));
#pragma unroll
        for (int j = 0; j < 4; ++j) b[j] = *(const u32x4*)(wt + swz(brow[j] + (lane & 31), c));
#pragma unroll
        for (int i = 0; i < 2; ++i)
#pragma unroll
          for (int j = 0; j < 4; ++j) acc[i][j] = mfma_f16(a[i], b[j], acc[i][j]);
      }
      // Branch-free body: the last step stages an unused tile and the last
      // two reload group g0 + NG - 1.
      store(st ^ 1);
      load(g0 + min(i + 2, NG - 1));
      __syncthreads();
    }

    // ---- a partial piece: publish it; the tile's last piece adds them ------
    if (NG < G) {
      // Thread-major float4 layout: element (k4, tid) at (k4 * kThreads + tid) * 4.
      // Stores and loads carry sc0 sc1 (system coherence: written through to
      // memory, read past the caches), so publishing them needs only their
      // completion before the count, not a cache write-back.
      constexpr int kSys = 0x11;  // buffer cache policy: sc0 | sc1
      constexpr uint32_t kPieceBytes = kPieceFloats * 4;
      const uint64_t pbase = (uint64_t)args.partials;
      // readfirstlane returns int: convert through uint32_t (no sign extension).
      const uint32_t p_hi = (uint32_t)__builtin_amdgcn_readfirstlane((uint32_t)(pbase >> 32));
      const uint32_t p_lo = (uint32_t)__builtin_amdgcn_readfirstlane((uint32_t)pbase);
      const uint64_t pb = ((uint64_t)p_hi << 32) | p_lo;
      const __amdgpu_buffer_rsrc_t rp = make_rsrc((const void*)pb, (uint64_t)(S > 1 ? 1 : 2) * W * kPieceBytes);
      const uint32_t own = __builtin_amdgcn_readfirstlane((S > 1 ? lw : piece_slot(lw, L, Q, G)) * kPieceBytes);
#pragma unroll
      for (int i = 0; i < 2; ++i)
#pragma unroll
        for (int j = 0; j < 4; ++j)
#pragma unroll
          for (int e4 = 0; e4 < 4; ++e4) {
            const int k4 = (i * 4 + j) * 4 + e4;
            const u32x4 v = {__float_as_uint(acc[i][j][4 * e4]), __float_as_uint(acc[i][j][4 * e4 + 1]),
                             __float_as_uint(acc[i][j][4 * e4 + 2]), __float_as_uint(acc[i][j][4 * e4 + 3])};
            __builtin_amdgcn_raw_buffer_store_b128(v, rp, (k4 * kThreads + tid) * 16, own, kSys);
          }
      wait_vmcnt0();
      // Workers covering tile L: fw .. lwl, one piece each.
      const uint32_t fw = S > 1 ? L * S : (L * G) / Q;
      const uint32_t lwl = S > 1 ? fw + S - 1 : ((L + 1) * G - 1) / Q;
      __syncthreads();
      if (tid == 0) {
        const unsigned prev =
            __hip_atomic_fetch_add(&args.counters[L], 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        last = prev == lwl - fw;
        if (last) __hip_atomic_store(&args.counters[L], 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
      }
      __syncthreads();
      if (!__builtin_amdgcn_readfirstlane(last)) continue;  // uniform branch
      // The sum does not depend on which piece arrives last: two pieces are
      // added as own + other (fp32 addition commutes); more are re-read and
      // added in worker order.
      const bool two = lwl == fw + 1;
      if (!two) {
#pragma unroll
        for (int i = 0; i < 2; ++i)
#pragma unroll
          for (int j = 0; j < 4; ++j) acc[i][j] = floatx16{};
      }
      for (uint32_t w = two ? (lw == fw ? lwl : fw) : fw; w <= lwl; ++w) {
        const uint32_t off = __builtin_amdgcn_readfirstlane((S > 1 ? w : piece_slot(w, L, Q, G)) * kPieceBytes);
        // Eight loads in flight per batch (issued before any is used).
#pragma unroll
        for (int i = 0; i < 2; ++i)
#pragma unroll
          for (int jp = 0; jp < 4; jp += 2) {
            u32x4 v[8];
#pragma unroll
            for (int t = 0; t < 8; ++t) {
              const int k4 = (i * 4 + jp + (t >> 2)) * 4 + (t & 3);
              v[t] = __builtin_amdgcn_raw_buffer_load_b128(rp, (k4 * kThreads + tid) * 16, off, kSys);
            }
#pragma unroll
            for (int t = 0; t < 8; ++t)
#pragma unroll
              for (int e = 0; e < 4; ++e) acc[i][jp + (t >> 2)][4 * (t & 3) + e] += __uint_as_float(v[t][e]);
          }
        if (two) break;
      }
    }

    // ---- epilogue ----------------------------------------------------------
    // acc[i][j] element e: row 32 i + 8 (e >> 2) + 4 kh + (e & 3) of the wave's
    // 64 rows, column (lane & 31) of block j.
#pragma unroll
    for (int i = 0; i < 2; ++i) {
#pragma unroll
      for (int e = 0; e < 16; ++e) {
        const uint32_t m = m0 + 64 * wm + 32 * i + 8 * (e >> 2) + 4 * kh + (e & 3);
        if (m >= M) continue;
        if (pair) {
#pragma unroll
          for (int j = 0; j < 2; ++j) {
            const uint32_t n = n_first + 64 * wn + 32 * j + (lane & 31);
            if (n < jb.rows) {
              const float gv = acc[i][j][e], uv = acc[i][j + 2][e];
              jb.out[(size_t)m * jb.rows + n] = f32_to_bf16(silu_f(gv) * uv);
            }
          }
        } else {
#pragma unroll
          for (int j = 0; j < 4; ++j) {
            const uint32_t n = n_first + brow[j] + (lane & 31);
            if (n < jb.rows) jb.out[(size_t)m * jb.rows + n] = f32_to_bf16(acc[i][j][e]);
          }
        }
      }
    }
  }
}

}  // namespace

size_t q4_gemm_xh_bytes(uint32_t K, uint32_t M) { return (size_t)M * K * 2; }

namespace {
struct GemmPlan {
  uint32_t m_tiles, tiles, q, splits, workers;
  size_t partial_bytes;  // 0 when every worker's range is whole tiles
};


// Plan cost in units of one K step of one 256 x 256 tile (about 1.9 us on
// MI355X), fitted to the measured BASELINE prefill shapes (M = 512, 2048).
// Workers run in rounds of `cus` (one workgroup per CU).  A K slice costs its
// steps plus about 10 (pipeline fill, epilogue) and 12 for writing its fp32
// piece, and the tile's last slice reads the others back at about 5 per
// piece (one read for two pieces).  A stream-K worker pays about 20 per tile
// it touches, 12 for writing a piece and 5 per piece of the tiles it sums.
double split_cost(uint32_t tiles, uint32_t G, uint32_t S, uint32_t cus) {
  const uint32_t gs = (G + S - 1) / S;
  const uint64_t rounds = ((uint64_t)tiles * S + cus - 1) / cus;
  return rounds * (gs + 10.0 + (S > 1 ? 12.0 : 0.0)) + (S > 1 ? 5.0 * (S == 2 ? 1 : S) : 0.0);
}
double stream_cost(uint32_t tiles, uint32_t G, uint32_t Q, uint32_t cus) {
  const uint64_t workers = ((uint64_t)tiles * G + Q - 1) / Q;
  const uint64_t rounds = (workers + cus - 1) / cus;
  const double pieces = Q >= G ? 1.0 : (double)G / Q + 1.0;
  return rounds * (Q + 20.0 * ((double)Q / G + 1.0) + 12.0 + 5.0 * pieces);
}

// N tiles of a job: 256 rows of a plain projection, 128 of a SwiGLU pair.
uint32_t job_tiles(const Q4Job& j) { return j.mode == kQ4OutSwiglu ? (j.rows + 127) / 128 : (j.rows + kBN - 1) / kBN; }

// The launch's jobs with a gate/up pair given as two jobs (swiglu) folded
// into one pair job; returns the job count.
int fold_jobs(const Q4Job* jobs, int n_jobs, bool swiglu, Q4Job* out) {
  if (!swiglu) {
    for (int i = 0; i < n_jobs; ++i) out[i] = jobs[i];
    return n_jobs;
  }
  out[0] = jobs[0];
  out[0].uw = jobs[1].w;
  out[0].us = jobs[1].s;
  out[0].ub = jobs[1].b;
  out[0].mode = kQ4OutSwiglu;
  return 1;
}

GemmPlan gemm_plan(const Q4Job* jobs, int n_jobs, uint32_t K, uint32_t M, const Tuning& tune) {
  GemmPlan p{};
  p.m_tiles = (M + kBM - 1) / kBM;
  uint32_t n_tiles = 0;
  for (int i = 0; i < n_jobs; ++i) n_tiles += job_tiles(jobs[i]);
  p.tiles = n_tiles * p.m_tiles;
  const uint32_t G = K / 64, cus = tune.cus > 0 ? (uint32_t)tune.cus : 256;
  const uint64_t total = (uint64_t)p.tiles * G;
  // Candidates: K split into S equal slices per tile (S = 1: whole tiles;
  // S <= 8, slices of at least 8 steps), and stream-K with the steps dealt
  // evenly over one or two rounds of workers.
  p.splits = 1;
  p.q = G;
  double best = split_cost(p.tiles, G, 1, cus);
  for (uint32_t s = 2; s <= 8 && G / s >= 8; ++s) {
    const double c = split_cost(p.tiles, G, s, cus);
    if (c < best) {
      best = c;
      p.splits = s;
      p.q = (G + s - 1) / s;
    }
  }
  for (uint32_t r = 1; r <= 2; ++r) {
    const uint64_t q = (total + r * cus - 1) / (r * cus);
    if (q < 8 || q % G == 0 || q >= (1ull << 31)) continue;
    const double c = stream_cost(p.tiles, G, (uint32_t)q, cus);
    if (c < best) {
      best = c;
      p.splits = 1;
      p.q = (uint32_t)q;
    }
  }
  const int fs = tune.gemm_splits, fq = tune.gemm_q;
  if (fs > 0) {
    p.splits = std::min<uint32_t>((uint32_t)fs, G);
    p.q = (G + p.splits - 1) / p.splits;
  } else if (fq > 0) {
    p.splits = 1;
    p.q = (uint32_t)fq;
  }
  p.splits = p.splits > 1 ? (G + p.q - 1) / p.q : 1;  // slices actually used
  p.workers = p.splits > 1 ? p.tiles * p.splits : (uint32_t)((total + p.q - 1) / p.q);
  const bool pieces = p.splits > 1 || p.q % G != 0;
  p.partial_bytes = pieces ? (size_t)(p.splits > 1 ? 1 : 2) * p.workers * kPieceFloats * sizeof(float) : 0;
  return p;
}
}  // namespace

void q4_gemm_workspace(const Q4Job* jobs, int n_jobs, bool swiglu, uint32_t K, uint32_t M, const Tuning& tune,
                       size_t* partial_bytes, size_t* counters) {
  Q4Job f[kMaxQ4Jobs];
  const int nf = fold_jobs(jobs, n_jobs, swiglu, f);
  const GemmPlan p = gemm_plan(f, nf, K, M, tune);
  *partial_bytes = p.partial_bytes;
  *counters = p.partial_bytes ? p.tiles : 0;
}

hipError_t launch_q4_gemm(const Q4Job* jobs, int n_jobs, bool swiglu, const uint16_t* x, uint32_t K, uint32_t M,
                          const Workspace& ws, hipStream_t stream) {
  if (n_jobs < 1 || n_jobs > kMaxQ4Jobs || K % 64 != 0 || M == 0 || (swiglu && n_jobs != 2))
    return hipErrorInvalidValue;
  Q4Job f[kMaxQ4Jobs];
  const int nf = fold_jobs(jobs, n_jobs, swiglu, f);
  for (int i = 0; i < nf; ++i)
    if (f[i].mode != kQ4OutBf16 && f[i].mode != kQ4OutSwiglu) return hipErrorInvalidValue;
  if (!ws.xh || ws.xh_bytes < q4_gemm_xh_bytes(K, M)) return hipErrorInvalidValue;
  if (!ws.tune) return hipErrorInvalidValue;
  const GemmPlan plan = gemm_plan(f, nf, K, M, *ws.tune);
  const bool log_plan = ws.tune->gemm_plan_log != 0;
  static uint64_t logged = 0;  // debug aid: print each new shape's plan once
  const uint64_t key = ((uint64_t)M << 40) ^ ((uint64_t)K << 16) ^ plan.tiles ^ ((uint64_t)plan.q << 56);
  if (log_plan && key != logged && (logged = key))
    fprintf(stderr, "q4_gemm plan: M=%u K=%u tiles=%u splits=%u Q=%u workers=%u\n", M, K, plan.tiles, plan.splits,
            plan.q, plan.workers);
  if (plan.partial_bytes && (ws.partial_bytes < plan.partial_bytes || ws.counter_count < plan.tiles))
    return hipErrorInvalidValue;
  GemmArgs a{};
  a.q_steps = plan.q;
  a.splits = plan.splits;
  a.workers = plan.workers;
  a.partials = ws.partials;
  a.counters = ws.counters;
  a.n_jobs = nf;
  a.xh = ws.xh;
  a.K = K;
  a.M = M;
  a.m_tiles = (M + kBM - 1) / kBM;
  uint32_t n_tiles = 0;
  for (int i = 0; i < nf; ++i) {
    a.jobs[i] = f[i];
    a.jobs[i].tile_begin = n_tiles;
    n_tiles += job_tiles(f[i]);
  }
  a.total_tiles = n_tiles * a.m_tiles;

  const size_t chunks = (size_t)M * K / 8;
  hipLaunchKernelGGL(x_to_f16_kernel, dim3((unsigned)((chunks + 255) / 256)), dim3(256), 0, stream, x, ws.xh, chunks);
  const dim3 grid(plan.workers);
  hipLaunchKernelGGL(q4_gemm_kernel, grid, dim3(kThreads), 0, stream, a);
  return hipGetLastError();
}

}  // namespace qm
