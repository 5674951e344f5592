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
//  * q8_attn_kernel: flash-decode over Q8 pages.  A wave owns one KV head and
//    the GQA group of <= 16 query heads sharing it (decode), or 16 (row, head)
//    columns (causal prefill).  Per 16-token page:
//      S^T = K Q^T on MFMA 16x16x32 (K bytes -> bf16 of k+128 exactly, the
//      +128 is removed with a per-head correction),
//      online softmax in fp32 (exp2 domain),
//      O^T += V^T P^T on MFMA 16x16x16 with P' = p * v_scale split into
//      bf16 hi + lo (error ~2^-16), again with a +128 correction.
//    The S^T/O^T orientation keeps every head in one lane column, so the
//    softmax statistics never move between lanes except for the 4-way max.
//    Decode splits the pages of a sequence over workgroups (4 waves each,
//    combined in LDS); split partials are merged by q8_combine_kernel.
#include <float.h>

#include "attention.h"
#include "common.h"

namespace qm {
namespace {

constexpr float kLog2e = 1.4426950408889634f;

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
  const uint32_t D = args.head_dim;

  const AttnSeq& sq = args.seqs[args.decode ? item : 0];
  const uint32_t token = args.decode ? sq.len - 1 : args.start + item;

  // Page-table entries of newly materialised pages (written once per call).
  if (kind == 0 && kvh == 0 && (args.decode || item == 0) && lane == 0) {
    for (int32_t i = 0; i < sq.new_page_count; ++i) sq.pt[sq.new_page_first + i] = sq.new_page_id + i;
  }
  const int32_t page = sq.new_page_count > 0 && (int32_t)(token / 16) >= sq.new_page_first
                           ? sq.new_page_id + ((int32_t)(token / 16) - sq.new_page_first)
                           : sq.pt[token / 16];
  const uint32_t slot = token % 16;

  const float* src = (kind == 0 ? args.k : args.v) + ((size_t)item * kvh_count + kvh) * D;
  float vals[4];
  float amax = 0.0f;
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const uint32_t d = lane * 4 + i;
    vals[i] = d < D ? src[d] : 0.0f;
    amax = fmaxf(amax, fabsf(vals[i]));
  }
#pragma unroll
  for (int off = 32; off >= 1; off >>= 1) amax = fmaxf(amax, __shfl_xor(amax, off));
  const float s = fmaxf(amax / 127.0f, FLT_MIN);
  int8_t qv[4];
#pragma unroll
  for (int i = 0; i < 4; ++i) qv[i] = (int8_t)roundf(fminf(fmaxf(vals[i] / s, -127.0f), 127.0f));

  const size_t pkv = (size_t)page * kvh_count + kvh;
  if (lane * 4 < D) {
    if (kind == 0) {
      const uint32_t packed = (uint32_t)(uint8_t)qv[0] | ((uint32_t)(uint8_t)qv[1] << 8) |
                              ((uint32_t)(uint8_t)qv[2] << 16) | ((uint32_t)(uint8_t)qv[3] << 24);
      *(uint32_t*)(sq.k + (pkv * 16 + slot) * D + lane * 4) = packed;
    } else {
#pragma unroll
      for (int i = 0; i < 4; ++i) sq.v[(pkv * D + lane * 4 + i) * 16 + slot] = qv[i];
    }
  }
  if (lane == 0) (kind == 0 ? sq.ks : sq.vs)[pkv * 16 + slot] = s;
}

// ---------------------------------------------------------------------------
// Attention
// ---------------------------------------------------------------------------
// 4 int8 -> 4 bf16 of (int8 + 128), exact (values 1..255 fit bf16).
__device__ __forceinline__ u32x2 q8x4_to_bf16_biased(uint32_t w) {
  const uint32_t u = w ^ 0x80808080u;
  const float f0 = (float)((u >> 0) & 0xFFu);
  const float f1 = (float)((u >> 8) & 0xFFu);
  const float f2 = (float)((u >> 16) & 0xFFu);
  const float f3 = (float)((u >> 24) & 0xFFu);
  u32x2 r;
  r.x = perm_b32(__float_as_uint(f1), __float_as_uint(f0), 0x07060302u);
  r.y = perm_b32(__float_as_uint(f3), __float_as_uint(f2), 0x07060302u);
  return r;
}

template <int D, bool PREFILL>
__global__ __launch_bounds__(256) void q8_attn_kernel(AttnArgs args) {
  constexpr int kWaves = 4;
  constexpr int kDB = D / 16;   // 16-wide d blocks of O^T
  constexpr int kKS = D / 32;   // QK k-steps
  __shared__ float red_o[kWaves][D][16];
  __shared__ float red_m[kWaves][16], red_l[kWaves][16], red_p[kWaves][16];

  const int lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int col = lane & 15;   // head column (decode) / (row, head) column (prefill)
  const int kq = lane >> 4;
  const uint32_t H = args.heads;
  const uint32_t KVH = args.kv_heads;
  const uint32_t gh = H / KVH;  // heads per KV head (<= 16)

  // ---- work unit -------------------------------------------------------------
  uint32_t b = 0, kvh, p_begin, p_end, row_base = 0;
  const uint32_t unit = blockIdx.x;
  if (!PREFILL) {
    while (b + 1 < args.n_seqs && unit >= args.seqs[b + 1].unit_begin) ++b;
    const uint32_t u = unit - args.seqs[b].unit_begin;
    kvh = u % KVH;
    const uint32_t split = u / KVH;
    const uint32_t pages = (args.seqs[b].len + 15) / 16;
    p_begin = split * args.pages_per_split;
    p_end = min(pages, p_begin + args.pages_per_split);
  } else {
    // blockIdx.x = kvh * row_blocks + rb; each wave owns 16/gh rows.
    const uint32_t rows_per_wave = 16 / gh;
    const uint32_t row_blocks = (args.rows + rows_per_wave * kWaves - 1) / (rows_per_wave * kWaves);
    kvh = unit / row_blocks;
    row_base = ((unit % row_blocks) * kWaves + wave) * rows_per_wave;
    p_begin = 0;
    const uint32_t last_row = min(args.rows, row_base + rows_per_wave) - 1;
    const uint32_t vis_max = min(args.start + last_row + 1, args.seqs[0].len);
    p_end = row_base < args.rows ? (vis_max + 15) / 16 : 0;
  }
  const AttnSeq& sq = args.seqs[b];

  // Column -> (query row, head).
  const uint32_t cr = PREFILL ? col / gh : 0;        // row within the wave's rows
  const uint32_t ch = PREFILL ? col % gh : col;      // head within the group
  const bool col_ok = PREFILL ? (ch < gh && row_base + cr < args.rows && col < (int)((16 / gh) * gh))
                              : ((uint32_t)col < gh);
  const uint32_t qrow = PREFILL ? row_base + cr : b;
  const uint32_t head = kvh * gh + ch;
  const uint32_t visible = PREFILL ? min(args.start + qrow + 1, sq.len) : sq.len;

  // ---- Q operand (B of QK^T): lane (col, kq) holds q[head][32kq + 8j .. +7]
  u32x4 qb[kKS];
  float qsum = 0.0f;
  {
    const uint16_t* qp = args.q + ((size_t)qrow * H + head) * D;
#pragma unroll
    for (int jj = 0; jj < kKS; ++jj) {
      u32x4 v = col_ok ? *(const u32x4*)(qp + D / 4 * kq + 8 * jj) : u32x4{0u, 0u, 0u, 0u};
      qb[jj] = v;
#pragma unroll
      for (int e = 0; e < 4; ++e) qsum += bf16_to_f32(v[e] & 0xFFFFu) + bf16_to_f32(v[e] >> 16);
    }
    qsum += __shfl_xor(qsum, 16);
    qsum += __shfl_xor(qsum, 32);
  }
  const float qcorr = 128.0f * qsum;
  const float sm_scale = kLog2e / sqrtf((float)D);

  floatx4 o[kDB];
#pragma unroll
  for (int i = 0; i < kDB; ++i) o[i] = floatx4{0.f, 0.f, 0.f, 0.f};
  float m_run = -INFINITY, l_lane = 0.0f, ps_lane = 0.0f;

  const size_t kv_page_stride = (size_t)KVH * 16 * D;
  const int tok = lane & 15;  // A-operand row of QK (token)
  for (uint32_t p = p_begin + (PREFILL ? 0 : wave); p < p_end; p += PREFILL ? 1 : kWaves) {
    const int32_t phys = sq.pt[p];
    const int8_t* kpage = sq.k + (size_t)phys * kv_page_stride + (size_t)kvh * 16 * D;
    const int8_t* vpage = sq.v + (size_t)phys * kv_page_stride + (size_t)kvh * D * 16;
    const float* kscale = sq.ks + ((size_t)phys * KVH + kvh) * 16;
    const float* vscale = sq.vs + ((size_t)phys * KVH + kvh) * 16;

    // S^T[token][col] over D in kKS steps of 32: lane (tok, kq) holds K[tok][D/4*kq + 8j ..].
    floatx4 s4 = {0.f, 0.f, 0.f, 0.f};
    {
      const int8_t* kr = kpage + tok * D + D / 4 * kq;
#pragma unroll
      for (int jj = 0; jj < kKS; jj += 2) {
        const u32x4 kb = *(const u32x4*)(kr + 8 * jj);  // 16 bytes = steps jj, jj+1
        u32x4 a0, a1;
        const u32x2 l0 = q8x4_to_bf16_biased(kb.x), h0 = q8x4_to_bf16_biased(kb.y);
        const u32x2 l1 = q8x4_to_bf16_biased(kb.z), h1 = q8x4_to_bf16_biased(kb.w);
        a0 = u32x4{l0.x, l0.y, h0.x, h0.y};
        a1 = u32x4{l1.x, l1.y, h1.x, h1.y};
        s4 = mfma16x16x32(a0, qb[jj], s4);
        s4 = mfma16x16x32(a1, qb[jj + 1], s4);
      }
    }
    const floatx4 ks4 = *(const floatx4*)(kscale + 4 * kq);
    const floatx4 vs4 = *(const floatx4*)(vscale + 4 * kq);
    float sc[4];
    float bmax = -INFINITY;
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      const uint32_t t = p * 16 + 4 * kq + r;
      const bool ok = col_ok && t < visible;
      sc[r] = ok ? (s4[r] - qcorr) * ks4[r] * sm_scale : -INFINITY;
      bmax = fmaxf(bmax, sc[r]);
    }
    bmax = fmaxf(bmax, __shfl_xor(bmax, 16));
    bmax = fmaxf(bmax, __shfl_xor(bmax, 32));
    const float m_new = fmaxf(m_run, bmax);
    const float corr = m_new == -INFINITY ? 1.0f : exp2f(m_run - m_new);
    m_run = m_new;
    float pw[4];
    float psum = 0.0f, pvsum = 0.0f;
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      const float e = sc[r] == -INFINITY ? 0.0f : exp2f(sc[r] - m_new);
      psum += e;
      pw[r] = sc[r] == -INFINITY ? 0.0f : e * vs4[r];  // fold the V scale (never NaN for masked rows)
      pvsum += pw[r];
    }
    l_lane = l_lane * corr + psum;
    ps_lane = ps_lane * corr + pvsum;
    // P'^T as bf16 hi + lo (B operand: k = tokens 4kq..4kq+3, column col).
    uint32_t hi[4], lo[4];
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      hi[r] = __float_as_uint(pw[r]) & 0xFFFF0000u;
      lo[r] = f32_to_bf16(pw[r] - __uint_as_float(hi[r]));
    }
    const u32x2 phi = {(hi[0] >> 16) | hi[1], (hi[2] >> 16) | hi[3]};
    const u32x2 plo = {lo[0] | (lo[1] << 16), lo[2] | (lo[3] << 16)};
#pragma unroll
    for (int db = 0; db < kDB; ++db) {
      const uint32_t vw = *(const uint32_t*)(vpage + (16 * db + tok) * 16 + 4 * kq);
      const u32x2 va = q8x4_to_bf16_biased(vw);
      floatx4 od = o[db] * corr;
      od = mfma16x16x16(va, phi, od);
      o[db] = mfma16x16x16(va, plo, od);
    }
  }

  // ---- combine the waves of the workgroup (decode) / finish (prefill) ------
  float l_tot = l_lane + __shfl_xor(l_lane, 16);
  l_tot += __shfl_xor(l_tot, 32);
  float ps_tot = ps_lane + __shfl_xor(ps_lane, 16);
  ps_tot += __shfl_xor(ps_tot, 32);

  if (PREFILL) {
    // O^T lane layout: column col, rows d = 16 db + 4 kq + r.
    if (col_ok) {
      const float inv = 1.0f / fmaxf(l_tot, FLT_MIN);
      const size_t obase = ((size_t)qrow * H + head) * D;
#pragma unroll
      for (int db = 0; db < kDB; ++db)
#pragma unroll
        for (int r = 0; r < 4; ++r) {
          const uint32_t d = 16 * db + 4 * kq + r;
          float v = (o[db][r] - 128.0f * ps_tot) * inv;
          if (args.gate) v *= sigmoid_f(bf16_to_f32(args.gate[obase + d]));
          args.o[obase + d] = f32_to_bf16(v);
        }
    }
    return;
  }

#pragma unroll
  for (int db = 0; db < kDB; ++db)
#pragma unroll
    for (int r = 0; r < 4; ++r) red_o[wave][16 * db + 4 * kq + r][col] = o[db][r];
  if (kq == 0) {
    red_m[wave][col] = m_run;
    red_l[wave][col] = l_tot;
    red_p[wave][col] = ps_tot;
  }
  __syncthreads();

  const uint32_t nsplit = sq.nsplit;
  const uint32_t split = (unit - sq.unit_begin) / KVH;
  for (uint32_t e = threadIdx.x; e < (uint32_t)D * 16; e += 256) {
    const uint32_t c = e % 16, d = e / 16;
    float mx = -INFINITY;
#pragma unroll
    for (int w = 0; w < kWaves; ++w) mx = fmaxf(mx, red_m[w][c]);
    float L = 0.0f, P = 0.0f, O = 0.0f;
#pragma unroll
    for (int w = 0; w < kWaves; ++w) {
      const float f = red_m[w][c] == -INFINITY ? 0.0f : exp2f(red_m[w][c] - mx);
      L += f * red_l[w][c];
      P += f * red_p[w][c];
      O += f * red_o[w][d][c];
    }
    O -= 128.0f * P;  // V was accumulated as v + 128
    if (c >= gh) continue;
    const uint32_t hh = kvh * gh + c;
    if (nsplit == 1) {
      float v = O / fmaxf(L, FLT_MIN);
      const size_t oi = ((size_t)b * H + hh) * D + d;
      if (args.gate) v *= sigmoid_f(bf16_to_f32(args.gate[oi]));
      args.o[oi] = f32_to_bf16(v);
    } else {
      // partial[(seq split row)][head][D + 2]: O (unnormalised), then m, l.
      float* part = args.partials + ((size_t)(sq.part_begin + split) * H + hh) * (D + 2);
      part[d] = O;
      if (d == 0) {
        part[D] = mx;
        part[D + 1] = L;
      }
    }
  }
}

// Merge the split partials of one (sequence, head): grid (n_seqs * H), D threads.
__global__ __launch_bounds__(256) void q8_combine_kernel(AttnArgs args) {
  const uint32_t H = args.heads;
  const uint32_t b = blockIdx.x / H, hh = blockIdx.x % H;
  const AttnSeq& sq = args.seqs[b];
  if (sq.nsplit <= 1) return;
  const uint32_t D = args.head_dim;
  const uint32_t d = threadIdx.x;
  if (d >= D) return;
  float mx = -INFINITY;
  for (uint32_t s = 0; s < sq.nsplit; ++s)
    mx = fmaxf(mx, args.partials[((size_t)(sq.part_begin + s) * H + hh) * (D + 2) + D]);
  float L = 0.0f, O = 0.0f;
  for (uint32_t s = 0; s < sq.nsplit; ++s) {
    const float* part = args.partials + ((size_t)(sq.part_begin + s) * H + hh) * (D + 2);
    const float f = part[D] == -INFINITY ? 0.0f : exp2f(part[D] - mx);
    L += f * part[D + 1];
    O += f * part[d];
  }
  float v = O / fmaxf(L, FLT_MIN);
  const size_t oi = ((size_t)b * H + hh) * D + d;
  if (args.gate) v *= sigmoid_f(bf16_to_f32(args.gate[oi]));
  args.o[oi] = f32_to_bf16(v);
}

template <int D>
hipError_t launch_attn_d(const AttnArgs& a, uint32_t units, hipStream_t st) {
  if (a.prefill)
    hipLaunchKernelGGL((q8_attn_kernel<D, true>), dim3(units), dim3(256), 0, st, a);
  else
    hipLaunchKernelGGL((q8_attn_kernel<D, false>), dim3(units), dim3(256), 0, st, a);
  return hipGetLastError();
}

}  // namespace

hipError_t launch_q8_append(const AppendArgs& a, uint32_t items, hipStream_t st) {
  hipLaunchKernelGGL(q8_append_kernel, dim3(items * a.kv_heads * 2), dim3(64), 0, st, a);
  return hipGetLastError();
}

hipError_t launch_q8_attention(const AttnArgs& a, uint32_t units, bool need_combine, hipStream_t st) {
  hipError_t e;
  switch (a.head_dim) {
    case 64: e = launch_attn_d<64>(a, units, st); break;
    case 128: e = launch_attn_d<128>(a, units, st); break;
    case 256: e = launch_attn_d<256>(a, units, st); break;
    default: return hipErrorInvalidValue;
  }
  if (e != hipSuccess || !need_combine) return e;
  hipLaunchKernelGGL(q8_combine_kernel, dim3(a.n_seqs * a.heads), dim3(a.head_dim), 0, st, a);
  return hipGetLastError();
}

}  // namespace qm
