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
  uint32_t splits, gks;  // K slices per tile, groups per slice
  float* partials;       // [tile][slice][kThreads * 128] fp32 (splits > 1)
  unsigned* counters;    // [tile], zero between launches
};

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
    const _Float16 f = (_Float16)bf16_to_f32(e[k]);
    h[k] = __builtin_bit_cast(uint16_t, f);
  }
  u32x4 o;
  o.x = h[0] | (h[4] << 16);
  o.y = h[1] | (h[5] << 16);
  o.z = h[2] | (h[6] << 16);
  o.w = h[3] | (h[7] << 16);
  *(u32x4*)(xh + 8 * i) = o;
}

template <bool SWIGLU>
__global__ __launch_bounds__(kThreads) void q4_gemm_kernel(GemmArgs args) {
  __shared__ __attribute__((aligned(16))) uint8_t lds[2][2][kTileBytes];  // [stage][X | W]

  const uint32_t tid = threadIdx.x;
  const uint32_t lane = tid & 63;
  const uint32_t wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const uint32_t wm = wave & 3, wn = wave >> 2;
  const uint32_t K = args.K, M = args.M, G = K / 64;

  // ---- XCD-aware tile remap (over tile x K-slice units) -------------------
  const uint32_t S = args.splits;
  const uint32_t T = args.total_tiles * S;
  const uint32_t xcd = blockIdx.x % kXcds, local = blockIdx.x / kXcds;
  const uint32_t q = T / kXcds, rem = T % kXcds;
  const uint32_t LS = xcd * q + min(xcd, rem) + local;
  const uint32_t L = LS / S, split = LS - L * S;
  const uint32_t n_tile = L / args.m_tiles, m_tile = L % args.m_tiles;
  const uint32_t g0 = split * args.gks;
  const uint32_t NG = min(G, g0 + args.gks) - g0;  // K steps of this slice (>= 1)
  const uint32_t m0 = m_tile * kBM;

  // ---- this thread's W row and the tile's job ------------------------------
  int jt = 0;
  if (!SWIGLU) {
    while (jt + 1 < args.n_jobs && n_tile >= args.jobs[jt + 1].tile_begin) ++jt;
  }
  const uint32_t srow = tid >> 1, shalf = tid & 1;  // staging: row of the tiles, chunk half
  const Q4Job& wj = args.jobs[SWIGLU ? (srow >= 128 ? 1 : 0) : jt];
  uint32_t n_first, wrow;
  if (SWIGLU) {
    n_first = n_tile * 128;
    wrow = n_first + (srow & 127);
  } else {
    n_first = (n_tile - wj.tile_begin) * kBN;
    wrow = n_first + srow;
  }
  wrow = min(wrow, wj.rows - 1);
  const __amdgpu_buffer_rsrc_t rw = make_rsrc(wj.w, (uint64_t)wj.rows * (K / 2));
  const uint16_t* s_row = wj.s + (size_t)wrow * G;
  const uint16_t* b_row = wj.b + (size_t)wrow * G;
  const uint32_t w_voff = wrow * (K / 2) + shalf * 16;
  const uint32_t xrow = min(m0 + srow, M - 1);
  const uint16_t* x_src = args.xh + (size_t)xrow * K + shalf * 32;

  // ---- staging registers ---------------------------------------------------
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

  // B-tile row bases of this wave's four 32-column blocks.
  uint32_t brow[4];
#pragma unroll
  for (int j = 0; j < 4; ++j)
    brow[j] = SWIGLU ? (j < 2 ? 64 * wn + 32 * j : 128 + 64 * wn + 32 * (j - 2)) : 128 * wn + 32 * j;
  const uint32_t arow0 = 64 * wm + (lane & 31);
  const uint32_t kh = lane >> 5;

  load(g0);
  store(0);
  if (NG > 1) load(g0 + 1);
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
    if (i + 1 < NG) {
      store(st ^ 1);
      if (i + 2 < NG) load(g0 + i + 2);
    }
    __syncthreads();
  }

  // ---- split-K: publish this slice, the last one of the tile adds them -----
  if (S > 1) {
    // Thread-major float4 layout: element (k4, tid) at (k4 * kThreads + tid) * 4.
    // Stores and loads carry sc0 sc1 (system coherence: written through to
    // memory, read past the caches), so publishing them needs only their
    // completion before the count, not a cache write-back.
    constexpr int kSys = 0x11;  // buffer cache policy: sc0 | sc1
    const __amdgpu_buffer_rsrc_t rp =
        make_rsrc(args.partials + (size_t)L * S * (kThreads * 128), (uint64_t)S * kThreads * 128 * 4);
#pragma unroll
    for (int i = 0; i < 2; ++i)
#pragma unroll
      for (int j = 0; j < 4; ++j)
#pragma unroll
        for (int e4 = 0; e4 < 4; ++e4) {
          const int k4 = (i * 4 + j) * 4 + e4;
          const u32x4 v = {__float_as_uint(acc[i][j][4 * e4]), __float_as_uint(acc[i][j][4 * e4 + 1]),
                           __float_as_uint(acc[i][j][4 * e4 + 2]), __float_as_uint(acc[i][j][4 * e4 + 3])};
          __builtin_amdgcn_raw_buffer_store_b128(v, rp, (k4 * kThreads + tid) * 16, split * (kThreads * 128 * 4),
                                                 kSys);
        }
    wait_vmcnt0();
    __shared__ unsigned last;
    __syncthreads();
    if (tid == 0) {
      const unsigned prev = __hip_atomic_fetch_add(&args.counters[L], 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
      last = prev == S - 1;
      if (last) __hip_atomic_store(&args.counters[L], 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    }
    __syncthreads();
    if (!last) return;
#pragma unroll
    for (int i = 0; i < 2; ++i)
#pragma unroll
      for (int j = 0; j < 4; ++j) acc[i][j] = floatx16{};
    for (uint32_t sl = 0; sl < S; ++sl) {
#pragma unroll
      for (int i = 0; i < 2; ++i)
#pragma unroll
        for (int j = 0; j < 4; ++j)
#pragma unroll
          for (int e4 = 0; e4 < 4; ++e4) {
            const int k4 = (i * 4 + j) * 4 + e4;
            const u32x4 v = __builtin_amdgcn_raw_buffer_load_b128(rp, (k4 * kThreads + tid) * 16,
                                                                  sl * (kThreads * 128 * 4), kSys);
#pragma unroll
            for (int e = 0; e < 4; ++e) acc[i][j][4 * e4 + e] += __uint_as_float(v[e]);
          }
    }
  }

  // ---- epilogue ------------------------------------------------------------
  // acc[i][j] element e: row 32 i + 8 (e >> 2) + 4 kh + (e & 3) of the wave's
  // 64 rows, column (lane & 31) of block j.
#pragma unroll
  for (int i = 0; i < 2; ++i) {
#pragma unroll
    for (int e = 0; e < 16; ++e) {
      const uint32_t m = m0 + 64 * wm + 32 * i + 8 * (e >> 2) + 4 * kh + (e & 3);
      if (m >= M) continue;
      if (SWIGLU) {
        const Q4Job& gj = args.jobs[0];
#pragma unroll
        for (int j = 0; j < 2; ++j) {
          const uint32_t n = n_tile * 128 + 64 * wn + 32 * j + (lane & 31);
          if (n < gj.rows) {
            const float gv = acc[i][j][e], uv = acc[i][j + 2][e];
            gj.out[(size_t)m * gj.rows + n] = f32_to_bf16(silu_f(gv) * uv);
          }
        }
      } else {
        const Q4Job& oj = args.jobs[jt];
#pragma unroll
        for (int j = 0; j < 4; ++j) {
          const uint32_t n = n_first + brow[j] + (lane & 31);
          if (n < oj.rows) oj.out[(size_t)m * oj.rows + n] = f32_to_bf16(acc[i][j][e]);
        }
      }
    }
  }
}

}  // namespace

size_t q4_gemm_xh_bytes(uint32_t K, uint32_t M) { return (size_t)M * K * 2; }

namespace {
struct GemmPlan {
  uint32_t m_tiles, tiles, splits, gks;
};
// K slices per tile: when the tiles fill less than one dispatch round of
// `cus` workgroups, split K so the units fill whole rounds as evenly as
// possible (at least 8 K steps per slice, at most 8 slices).
int env_int_gemm(const char* name, int fallback) {
  const char* v = getenv(name);
  return v ? atoi(v) : fallback;
}

GemmPlan gemm_plan(const Q4Job* jobs, int n_jobs, bool swiglu, uint32_t K, uint32_t M) {
  GemmPlan p{};
  p.m_tiles = (M + kBM - 1) / kBM;
  uint32_t n_tiles = 0;
  if (swiglu) {
    n_tiles = (jobs[0].rows + 127) / 128;
  } else {
    for (int i = 0; i < n_jobs; ++i) n_tiles += (jobs[i].rows + kBN - 1) / kBN;
  }
  p.tiles = n_tiles * p.m_tiles;
  const uint32_t G = K / 64, cus = 256;
  // Split-K fills partial dispatch rounds (one workgroup per CU).  Cost in
  // units of one K group of one tile, fitted to measured BASELINE shapes:
  // per round the slice's groups plus about 10 for the pipeline fill and the
  // epilogue, 4 more for writing the fp32 partials when split, and about 10
  // per slice for the last slice's read-back.  (Down at M = 2048, 160 tiles:
  // three slices in two rounds beat one long round by 15 %; QKV's 320 tiles
  // stay unsplit: five rounds of short slices lose to two full rounds.)
  p.splits = 1;
  double best = 0.0;
  for (uint32_t s = 1; s <= 8 && (s == 1 || G / s >= 8); ++s) {
    const uint32_t gks = (G + s - 1) / s;
    const uint32_t units = p.tiles * s, rounds = (units + cus - 1) / cus;
    const double cost = rounds * (gks + 10.0 + (s > 1 ? 4.0 : 0.0)) + (s > 1 ? 10.0 * s : 0.0);
    if (s == 1 || cost < best) {
      best = cost;
      p.splits = s;
    }
  }
  if (env_int_gemm("QM38_GEMM_SPLITS", 0) > 0) p.splits = std::min<uint32_t>(8, (uint32_t)env_int_gemm("QM38_GEMM_SPLITS", 1));
  p.gks = (G + p.splits - 1) / p.splits;
  p.splits = (G + p.gks - 1) / p.gks;
  return p;
}
}  // namespace

void q4_gemm_workspace(const Q4Job* jobs, int n_jobs, bool swiglu, uint32_t K, uint32_t M, size_t* partial_bytes,
                       size_t* counters) {
  const GemmPlan p = gemm_plan(jobs, n_jobs, swiglu, K, M);
  *partial_bytes = p.splits > 1 ? (size_t)p.tiles * p.splits * kThreads * 128 * sizeof(float) : 0;
  *counters = p.splits > 1 ? p.tiles : 0;
}

hipError_t launch_q4_gemm(const Q4Job* jobs, int n_jobs, bool swiglu, const uint16_t* x, uint32_t K, uint32_t M,
                          const Workspace& ws, hipStream_t stream) {
  if (n_jobs < 1 || n_jobs > kMaxQ4Jobs || K % 64 != 0 || M == 0) return hipErrorInvalidValue;
  if (!ws.xh || ws.xh_bytes < q4_gemm_xh_bytes(K, M)) return hipErrorInvalidValue;
  const GemmPlan plan = gemm_plan(jobs, n_jobs, swiglu, K, M);
  if (plan.splits > 1 && (ws.partial_bytes < (size_t)plan.tiles * plan.splits * kThreads * 128 * sizeof(float) ||
                          ws.counter_count < plan.tiles))
    return hipErrorInvalidValue;
  GemmArgs a{};
  a.splits = plan.splits;
  a.gks = plan.gks;
  a.partials = ws.partials;
  a.counters = ws.counters;
  a.n_jobs = n_jobs;
  a.xh = ws.xh;
  a.K = K;
  a.M = M;
  a.m_tiles = (M + kBM - 1) / kBM;
  uint32_t n_tiles = 0;
  for (int i = 0; i < n_jobs; ++i) {
    a.jobs[i] = jobs[i];
    a.jobs[i].tile_begin = n_tiles;
    if (!swiglu) n_tiles += (jobs[i].rows + kBN - 1) / kBN;
  }
  if (swiglu) n_tiles = (jobs[0].rows + 127) / 128;
  a.total_tiles = n_tiles * a.m_tiles;

  const size_t chunks = (size_t)M * K / 8;
  hipLaunchKernelGGL(x_to_f16_kernel, dim3((unsigned)((chunks + 255) / 256)), dim3(256), 0, stream, x, ws.xh, chunks);
  const dim3 grid(a.total_tiles * a.splits);
  if (swiglu)
    hipLaunchKernelGGL(q4_gemm_kernel<true>, grid, dim3(kThreads), 0, stream, a);
  else
    hipLaunchKernelGGL(q4_gemm_kernel<false>, grid, dim3(kThreads), 0, stream, a);
  return hipGetLastError();
}

}  // namespace qm
