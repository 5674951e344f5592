// C-ABI entry points of the paged Q8 KV cache and GQA attention
// (see include/qm38.h).  Host-side page bookkeeping follows
// LogicalPageTable (/root/reference/src/paged_kv.rs:12-98): pages
// materialise lazily, in order, with sequential ids.
#include <float.h>
#include <stdint.h>
#include <stdlib.h>
#include <string.h>

#include <algorithm>
#include <vector>

#include "attention.h"
#include "prepare.h"
#include "runtime_internal.h"

using namespace qm;

struct qm_kv {
  qm_runtime* rt = nullptr;
  uint32_t kv_heads = 0, head_dim = 0, page_tokens = 16, max_tokens = 0, max_pages = 0;
  uint32_t length = 0;
  std::vector<int32_t> pages;  // logical page -> physical id, -1 if not materialised
  int32_t next_page_id = 0;
  int32_t* d_pt = nullptr;     // device page table [max_pages]
  int8_t* k = nullptr;         // [max_pages][kv_heads][16][D]
  int8_t* v = nullptr;         // [max_pages][kv_heads][D][16]
  float* ks = nullptr;         // [max_pages][kv_heads][16]
  float* vs = nullptr;
};

namespace {

int env_int(const char* name, int fallback) {
  const char* v = getenv(name);
  return v ? atoi(v) : fallback;
}

size_t kv_page_bytes(const qm_kv* kv) { return (size_t)kv->kv_heads * kv->page_tokens * kv->head_dim; }
size_t scale_page_count(const qm_kv* kv) { return (size_t)kv->kv_heads * kv->page_tokens; }

void free_kv(qm_kv* kv) {
  if (!kv) return;
  DeviceGuard g(kv->rt->device);
  hipFree(kv->d_pt);
  hipFree(kv->k);
  hipFree(kv->v);
  hipFree(kv->ks);
  hipFree(kv->vs);
  delete kv;
}

// validate_attention_shape (metal_runtime.rs:9186-9193) + this build's kernel limits.
qm_status validate_kv_shape(uint32_t kv_heads, uint32_t head_dim, uint32_t page_tokens) {
  if (kv_heads == 0 || head_dim == 0 || head_dim > 256)
    return fail(QM_ERR_INVALID_ATTENTION_SHAPE, "attention dimensions must be non-zero and fit one GPU threadgroup");
  if (head_dim != 64 && head_dim != 128 && head_dim != 256)
    return fail(QM_ERR_INVALID_ATTENTION_SHAPE, "head_dim %u unsupported (64, 128 or 256)", head_dim);
  if (page_tokens != 16) return fail(QM_ERR_INVALID_ATTENTION_SHAPE, "page_tokens must be 16");
  return QM_OK;
}

// LogicalPageTable::append / allocate: materialise pages covering [start, end).
// Returns the first newly materialised logical page and how many there are.
void materialise(qm_kv* kv, uint32_t start, uint32_t end, int32_t* first_new, int32_t* count, int32_t* first_id) {
  *first_new = -1;
  *count = 0;
  *first_id = -1;
  if (end <= start) return;
  const uint32_t first = start / kv->page_tokens, last = (end - 1) / kv->page_tokens;
  for (uint32_t p = first; p <= last; ++p) {
    if (kv->pages[p] < 0) {
      kv->pages[p] = kv->next_page_id++;
      if (*count == 0) {
        *first_new = (int32_t)p;
        *first_id = kv->pages[p];
      }
      ++*count;
    }
  }
}

AttnSeq seq_desc(const qm_kv* kv) {
  AttnSeq s{};
  s.k = kv->k;
  s.v = kv->v;
  s.ks = kv->ks;
  s.vs = kv->vs;
  s.pt = kv->d_pt;
  s.len = kv->length;
  s.new_page_first = -1;
  s.new_page_count = 0;
  s.new_page_id = -1;
  return s;
}

bool aligned(const void* p, uintptr_t a) { return ((uintptr_t)p & (a - 1)) == 0; }

}  // namespace

uint32_t qm::kv_heads_of(const qm_kv* kv) { return kv->kv_heads; }
uint32_t qm::kv_head_dim_of(const qm_kv* kv) { return kv->head_dim; }
const qm_runtime* qm::kv_runtime_of(const qm_kv* kv) { return kv->rt; }

extern "C" {

qm_status qm_kv_create(qm_runtime* rt, uint32_t kv_heads, uint32_t head_dim, uint32_t page_tokens,
                       uint32_t max_tokens, qm_kv** out) {
  if (!rt || !out) return fail(QM_ERR_NULL_POINTER, "runtime/out is NULL");
  *out = nullptr;
  qm_status st = validate_kv_shape(kv_heads, head_dim, page_tokens);
  if (st != QM_OK) return st;
  if (max_tokens == 0) return fail(QM_ERR_ZERO_CAPACITY, "page table capacity and page size must be non-zero");
  qm_kv* kv = new qm_kv();
  kv->rt = rt;
  kv->kv_heads = kv_heads;
  kv->head_dim = head_dim;
  kv->page_tokens = page_tokens;
  kv->max_tokens = max_tokens;
  kv->max_pages = (max_tokens + page_tokens - 1) / page_tokens;
  kv->pages.assign(kv->max_pages, -1);
  DeviceGuard g(rt->device);
  const size_t pb = kv_page_bytes(kv) * kv->max_pages;
  const size_t sb = scale_page_count(kv) * kv->max_pages * sizeof(float);
  hipError_t e = hipMalloc(&kv->d_pt, kv->max_pages * sizeof(int32_t));
  if (e == hipSuccess) e = hipMalloc(&kv->k, pb);
  if (e == hipSuccess) e = hipMalloc(&kv->v, pb);
  if (e == hipSuccess) e = hipMalloc(&kv->ks, sb);
  if (e == hipSuccess) e = hipMalloc(&kv->vs, sb);
  // Zeroed like the reference's zeroed_shared_buffer; unmaterialised page
  // table entries point at page 0 (never read: only pages below the length are).
  if (e == hipSuccess) e = hipMemsetAsync(kv->d_pt, 0, kv->max_pages * sizeof(int32_t), rt->stream);
  if (e == hipSuccess) e = hipMemsetAsync(kv->k, 0, pb, rt->stream);
  if (e == hipSuccess) e = hipMemsetAsync(kv->v, 0, pb, rt->stream);
  if (e == hipSuccess) e = hipMemsetAsync(kv->ks, 0, sb, rt->stream);
  if (e == hipSuccess) e = hipMemsetAsync(kv->vs, 0, sb, rt->stream);
  if (e == hipSuccess) e = hipStreamSynchronize(rt->stream);
  if (e != hipSuccess) {
    free_kv(kv);
    return hip_check(e, "KV cache allocation");
  }
  *out = kv;
  return QM_OK;
}

void qm_kv_destroy(qm_kv* kv) {
  if (!kv) return;
  hipStreamSynchronize(kv->rt->stream);
  free_kv(kv);
}

uint32_t qm_kv_length(const qm_kv* kv) { return kv ? kv->length : 0; }

uint32_t qm_kv_allocated_pages(const qm_kv* kv) {
  if (!kv) return 0;
  return (uint32_t)std::count_if(kv->pages.begin(), kv->pages.end(), [](int32_t p) { return p >= 0; });
}

int64_t qm_kv_page_for_token(const qm_kv* kv, uint32_t token) {
  if (!kv || token >= kv->length) return -1;
  return kv->pages[token / kv->page_tokens];
}

qm_status qm_kv_reserve(qm_kv* kv, uint32_t additional) {
  if (!kv) return fail(QM_ERR_NULL_POINTER, "kv is NULL");
  const uint64_t end = (uint64_t)kv->length + additional;
  if (end > kv->max_tokens)
    return fail(QM_ERR_CAPACITY_EXCEEDED, "token range ending at %llu exceeds page table capacity %u",
                (unsigned long long)end, kv->max_tokens);
  int32_t first, count, id;
  materialise(kv, kv->length, (uint32_t)end, &first, &count, &id);
  if (count == 0) return QM_OK;
  DeviceGuard g(kv->rt->device);
  hipError_t e = hipMemcpyAsync(kv->d_pt + first, kv->pages.data() + first, count * sizeof(int32_t),
                                hipMemcpyHostToDevice, kv->rt->stream);
  if (e == hipSuccess) e = hipStreamSynchronize(kv->rt->stream);
  return hip_check(e, "page table update");
}

qm_status qm_kv_truncate(qm_kv* kv, uint32_t length) {
  if (!kv) return fail(QM_ERR_NULL_POINTER, "kv is NULL");
  if (length > kv->length)
    return fail(QM_ERR_INVALID_SEQUENCE_LENGTH, "the requested KV sequence length exceeds the active cache");
  kv->length = length;
  return QM_OK;
}

qm_status qm_kv_clone(const qm_kv* src, qm_kv** out) {
  if (!src || !out) return fail(QM_ERR_NULL_POINTER, "src/out is NULL");
  qm_kv* kv = nullptr;
  qm_status st = qm_kv_create(src->rt, src->kv_heads, src->head_dim, src->page_tokens, src->max_tokens, &kv);
  if (st != QM_OK) return st;
  kv->length = src->length;
  kv->pages = src->pages;
  kv->next_page_id = src->next_page_id;
  DeviceGuard g(src->rt->device);
  const size_t n = (size_t)src->next_page_id;
  hipStream_t s = src->rt->stream;
  hipError_t e = hipMemcpyAsync(kv->d_pt, src->d_pt, src->max_pages * sizeof(int32_t), hipMemcpyDeviceToDevice, s);
  if (e == hipSuccess && n) e = hipMemcpyAsync(kv->k, src->k, n * kv_page_bytes(src), hipMemcpyDeviceToDevice, s);
  if (e == hipSuccess && n) e = hipMemcpyAsync(kv->v, src->v, n * kv_page_bytes(src), hipMemcpyDeviceToDevice, s);
  if (e == hipSuccess && n)
    e = hipMemcpyAsync(kv->ks, src->ks, n * scale_page_count(src) * 4, hipMemcpyDeviceToDevice, s);
  if (e == hipSuccess && n)
    e = hipMemcpyAsync(kv->vs, src->vs, n * scale_page_count(src) * 4, hipMemcpyDeviceToDevice, s);
  if (e == hipSuccess) e = hipStreamSynchronize(s);
  if (e != hipSuccess) {
    qm_kv_destroy(kv);
    return hip_check(e, "KV clone");
  }
  *out = kv;
  return QM_OK;
}

qm_status qm_kv_read(const qm_kv* kv, int8_t* keys, int8_t* values, float* key_scales, float* value_scales) {
  if (!kv) return fail(QM_ERR_NULL_POINTER, "kv is NULL");
  DeviceGuard g(kv->rt->device);
  const size_t n = (size_t)kv->next_page_id;
  const uint32_t KVH = kv->kv_heads, D = kv->head_dim, T = kv->length;
  std::vector<int8_t> hk(n * kv_page_bytes(kv)), hv(n * kv_page_bytes(kv));
  std::vector<float> hks(n * scale_page_count(kv)), hvs(n * scale_page_count(kv));
  hipStream_t s = kv->rt->stream;
  hipError_t e = hipSuccess;
  if (n) {
    e = hipMemcpyAsync(hk.data(), kv->k, hk.size(), hipMemcpyDeviceToHost, s);
    if (e == hipSuccess) e = hipMemcpyAsync(hv.data(), kv->v, hv.size(), hipMemcpyDeviceToHost, s);
    if (e == hipSuccess) e = hipMemcpyAsync(hks.data(), kv->ks, hks.size() * 4, hipMemcpyDeviceToHost, s);
    if (e == hipSuccess) e = hipMemcpyAsync(hvs.data(), kv->vs, hvs.size() * 4, hipMemcpyDeviceToHost, s);
    if (e == hipSuccess) e = hipStreamSynchronize(s);
  }
  if (e != hipSuccess) return hip_check(e, "KV read");
  for (uint32_t t = 0; t < T; ++t) {
    const size_t page = (size_t)kv->pages[t / 16];
    const uint32_t slot = t % 16;
    for (uint32_t h = 0; h < KVH; ++h) {
      const size_t pkv = page * KVH + h;
      for (uint32_t d = 0; d < D; ++d) {
        if (keys) keys[((size_t)t * KVH + h) * D + d] = hk[(pkv * 16 + slot) * D + d];
        if (values) values[((size_t)t * KVH + h) * D + d] = hv[(pkv * D + d) * 16 + slot];
      }
      if (key_scales) key_scales[(size_t)t * KVH + h] = hks[pkv * 16 + slot];
      if (value_scales) value_scales[(size_t)t * KVH + h] = hvs[pkv * 16 + slot];
    }
  }
  return QM_OK;
}

qm_status qm_attn_decode(qm_runtime* rt, qm_kv* const* seqs, uint32_t B, const uint16_t* q, const uint16_t* gate,
                         const float* k, const float* v, uint32_t H, uint16_t* o) {
  if (!rt || !seqs || !q || !k || !v || !o) return fail(QM_ERR_NULL_POINTER, "NULL argument");
  if (B == 0 || B > 64) return fail(QM_ERR_INVALID_ARGUMENT, "batch must be 1..64 sequences");
  const qm_kv* s0 = seqs[0];
  if (!s0) return fail(QM_ERR_NULL_POINTER, "sequence 0 is NULL");
  const uint32_t KVH = s0->kv_heads, D = s0->head_dim;
  if (H == 0 || H % KVH != 0 || H / KVH > 16)
    return fail(QM_ERR_INVALID_ATTENTION_SHAPE, "num_heads %u must be a multiple of kv_heads %u with at most 16 per KV head",
                H, KVH);
  if (!aligned(q, 16) || (gate && !aligned(gate, 16)) || !aligned(k, 4) || !aligned(v, 4))
    return fail(QM_ERR_MISALIGNED, "q/gate must be 16-byte aligned");
  for (uint32_t b = 0; b < B; ++b) {
    if (!seqs[b]) return fail(QM_ERR_NULL_POINTER, "sequence %u is NULL", b);
    if (seqs[b]->kv_heads != KVH || seqs[b]->head_dim != D)
      return fail(QM_ERR_INVALID_ATTENTION_SHAPE, "all sequences must share kv_heads and head_dim");
    if (seqs[b]->rt != rt) return fail(QM_ERR_INVALID_ARGUMENT, "sequence %u belongs to another runtime", b);
    if (seqs[b]->length + 1 > seqs[b]->max_tokens)
      return fail(QM_ERR_CAPACITY_EXCEEDED, "token range ending at %u exceeds page table capacity %u",
                  seqs[b]->length + 1, seqs[b]->max_tokens);
    for (uint32_t c = 0; c < b; ++c)
      if (seqs[c] == seqs[b]) return fail(QM_ERR_INVALID_ARGUMENT, "sequence %u appears twice", b);
  }
  DeviceGuard g(rt->device);
  // One residency round of the decode kernel: two 256-thread workgroups per CU (LDS-bound).
  const uint32_t target = (uint32_t)env_int("QM38_ATTN_TARGET_WGS", 2 * rt->cu_count);
  for (uint32_t b0 = 0; b0 < B; b0 += kMaxAttnSeqs) {
    const uint32_t nb = std::min<uint32_t>(kMaxAttnSeqs, B - b0);
    AppendArgs ap{};
    AttnArgs at{};
    uint64_t total_pages = 0;
    for (uint32_t i = 0; i < nb; ++i) {
      qm_kv* kv = seqs[b0 + i];
      AttnSeq sd = seq_desc(kv);
      materialise(kv, kv->length, kv->length + 1, &sd.new_page_first, &sd.new_page_count, &sd.new_page_id);
      kv->length += 1;
      sd.len = kv->length;
      ap.seqs[i] = sd;
      at.seqs[i] = sd;
      total_pages += (sd.len + 15) / 16;
    }
    // Pages per split: about `target` workgroups in the launch, 4 waves each.
    uint64_t pps = (total_pages * KVH + target - 1) / target;
    pps = std::max<uint64_t>(4, (pps + 3) / 4 * 4);
    if (env_int("QM38_ATTN_PPS", 0) > 0) pps = (uint64_t)env_int("QM38_ATTN_PPS", 4);
    // The combine kernel holds at most kMaxSplits split weights per sequence.
    uint32_t max_pages = 0;
    for (uint32_t i = 0; i < nb; ++i) max_pages = std::max(max_pages, (at.seqs[i].len + 15) / 16);
    pps = std::max<uint64_t>(pps, (max_pages + kMaxSplits - 1) / kMaxSplits);
    // Ceil-division per sequence can push the unit count past one residency
    // round, which would leave a nearly empty second round as long as the
    // first: grow the split until every unit fits.
    auto units_for = [&](uint64_t q) {
      uint64_t u = 0;
      for (uint32_t i = 0; i < nb; ++i) u += ((at.seqs[i].len + 15) / 16 + q - 1) / q * KVH;
      return u;
    };
    if (env_int("QM38_ATTN_PPS", 0) <= 0)
      while (pps < kMaxPagesPerSplit && units_for(pps) > target) pps += 4;
    pps = std::min<uint64_t>(pps, kMaxPagesPerSplit);
    if ((uint64_t)max_pages > (uint64_t)kMaxSplits * kMaxPagesPerSplit)
      return fail(QM_ERR_CAPACITY_EXCEEDED, "sequence of %u pages exceeds the decode kernel's limit", max_pages);
    uint32_t units = 0, parts = 0;
    bool combine = false;
    for (uint32_t i = 0; i < nb; ++i) {
      const uint32_t pages = (at.seqs[i].len + 15) / 16;
      const uint32_t ns = (uint32_t)((pages + pps - 1) / pps);
      at.seqs[i].unit_begin = units;
      at.seqs[i].nsplit = ns;
      at.seqs[i].part_begin = parts;
      units += ns * KVH;
      if (ns > 1) {
        parts += ns;
        combine = true;
      }
    }
    qm_status st = QM_OK;
    if (combine) st = ensure_partials(rt, (size_t)parts * H * (D + 2) * sizeof(float));
    if (st != QM_OK) return st;
    ap.k = k + (size_t)b0 * KVH * D;
    ap.v = v + (size_t)b0 * KVH * D;
    ap.kv_heads = KVH;
    ap.head_dim = D;
    ap.decode = 1;
    at.q = q + (size_t)b0 * H * D;
    at.gate = gate ? gate + (size_t)b0 * H * D : nullptr;
    at.o = o + (size_t)b0 * H * D;
    at.partials = (float*)rt->partials;
    at.heads = H;
    at.kv_heads = KVH;
    at.head_dim = D;
    at.n_seqs = nb;
    at.pages_per_split = (uint32_t)pps;
    at.prefill = 0;
    at.k_new = ap.k;  // the decode kernel appends the new rows itself
    at.v_new = ap.v;
    hipError_t e = launch_q8_attention(at, units, combine, rt->stream);
    if (e != hipSuccess) return hip_check(e, "attention decode launch");
  }
  return QM_OK;
}

qm_status qm_attn_prefill(qm_runtime* rt, qm_kv* seq, const uint16_t* q, const uint16_t* gate, const float* k,
                          const float* v, uint32_t H, uint32_t M, uint16_t* o) {
  if (!rt || !seq || !q || !k || !v || !o) return fail(QM_ERR_NULL_POINTER, "NULL argument");
  if (M == 0) return fail(QM_ERR_INVALID_ATTENTION_SHAPE, "prefill needs at least one row");
  const uint32_t KVH = seq->kv_heads, D = seq->head_dim;
  if (H == 0 || H % KVH != 0 || H / KVH > 16)
    return fail(QM_ERR_INVALID_ATTENTION_SHAPE, "num_heads %u must be a multiple of kv_heads %u with at most 16 per KV head",
                H, KVH);
  if (!aligned(q, 16) || (gate && !aligned(gate, 16)) || !aligned(k, 4) || !aligned(v, 4))
    return fail(QM_ERR_MISALIGNED, "q/gate must be 16-byte aligned");
  if ((uint64_t)seq->length + M > seq->max_tokens)
    return fail(QM_ERR_CAPACITY_EXCEEDED, "token range ending at %llu exceeds page table capacity %u",
                (unsigned long long)seq->length + M, seq->max_tokens);
  DeviceGuard g(rt->device);
  const uint32_t start = seq->length;
  AttnSeq sd = seq_desc(seq);
  materialise(seq, start, start + M, &sd.new_page_first, &sd.new_page_count, &sd.new_page_id);
  seq->length = start + M;
  sd.len = seq->length;
  AppendArgs ap{};
  ap.k = k;
  ap.v = v;
  ap.kv_heads = KVH;
  ap.head_dim = D;
  ap.decode = 0;
  ap.start = start;
  ap.seqs[0] = sd;
  AttnArgs at{};
  at.q = q;
  at.gate = gate;
  at.o = o;
  at.heads = H;
  at.kv_heads = KVH;
  at.head_dim = D;
  at.n_seqs = 1;
  at.prefill = 1;
  at.rows = M;
  at.start = start;
  at.seqs[0] = sd;
  hipError_t e = launch_q8_append(ap, M, rt->stream);
  // The prefill launcher sizes its own grid (rows per workgroup depend on the
  // kernel's column blocks).
  if (e == hipSuccess) e = launch_q8_attention(at, 0, false, rt->stream);
  return hip_check(e, "attention prefill launch");
}

}  // extern "C"

qm_status qm_attn_prepare(qm_runtime* rt, const qm_rope_config* rope, uint32_t M, uint32_t H, uint32_t kv_heads,
                          const uint16_t* q_with_gate, const uint16_t* k_in, const float* q_norm, const float* k_norm,
                          float epsilon, const uint32_t* positions, uint32_t position_base, uint16_t* q_out,
                          uint16_t* gate_out, float* k_out) {
  if (!rt || !rope || !q_with_gate || !k_in || !q_norm || !k_norm || !q_out || !gate_out || !k_out)
    return fail(QM_ERR_NULL_POINTER, "NULL argument");
  if (M == 0 || H == 0 || kv_heads == 0) return fail(QM_ERR_EMPTY_DIMENSION, "rows, heads and kv_heads must be > 0");
  const uint32_t hd = rope->head_dim;
  if (hd == 0 || hd > kPrepMaxHeadDim)
    return fail(QM_ERR_INVALID_ATTENTION_SHAPE, "head_dim %u must be 1..%u", hd, kPrepMaxHeadDim);
  if (rope->rotary_dim > hd || rope->rotary_dim % 2 != 0)
    return fail(QM_ERR_INVALID_ATTENTION_SHAPE, "rotary_dim %u must be even and <= head_dim %u", rope->rotary_dim, hd);
  if (!(rope->rope_theta > 0.0f)) return fail(QM_ERR_INVALID_ARGUMENT, "rope_theta must be > 0");
  if (hd % 4 == 0 && (!aligned(q_with_gate, 8) || !aligned(k_in, 8) || !aligned(q_out, 8) || !aligned(gate_out, 8) ||
                      !aligned(k_out, 16)))
    return fail(QM_ERR_MISALIGNED, "attention prepare: bf16 buffers must be 8-byte and k_out 16-byte aligned");
  if ((uint64_t)H + kv_heads > 0x7FFFFFFFull)
    return fail(QM_ERR_DIMENSION_OVERFLOW, "attention prepare: %u + %u heads overflow", H, kv_heads);
  PrepArgs a{};
  a.q_with_gate = q_with_gate;
  a.k_in = k_in;
  a.q_norm = q_norm;
  a.k_norm = k_norm;
  a.positions = positions;
  a.base = position_base;
  a.q_out = q_out;
  a.gate_out = gate_out;
  a.k_out = k_out;
  a.M = M;
  a.H = H;
  a.KVH = kv_heads;
  a.head_dim = hd;
  a.rotary_dim = rope->rotary_dim;
  a.section1 = rope->mrope_section1;
  a.section2 = rope->mrope_section2;
  a.has_sections = rope->has_mrope_sections ? 1u : 0u;
  a.theta = rope->rope_theta;
  a.eps = epsilon;
  return hip_check(launch_attn_prepare(a, rt->stream), "attention prepare launch");
}
