// C-ABI entry points of the paged Q8 KV cache and GQA attention
// (see include/qm38.h).  Host-side page bookkeeping follows
// LogicalPageTable (/root/reference/src/paged_kv.rs:12-98): pages
// materialise lazily, in order, with sequential ids.  Physical capacity
// grows like ensure_q8_kv_capacity (metal_runtime.rs:7406-7421): to the next
// power of two of the required tokens (at least 16), copying the pages held.
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
  uint32_t kv_heads = 0;
  uint32_t head_dim = 0;  // the caller's head dimension
  uint32_t dp = 0;        // storage width of a page row (attn_padded_dim)
  uint32_t page_tokens = 16;
  uint32_t max_tokens = 0;  // hard limit (LogicalPageTable capacity); 0 = grow without limit
  uint32_t cap_pages = 0;   // physical pages allocated
  uint32_t length = 0;
  std::vector<int32_t> pages;  // logical page -> physical id, -1 if not materialised [cap_pages]
  int32_t next_page_id = 0;
  int32_t* d_pt = nullptr;  // device page table [cap_pages]
  int8_t* k = nullptr;      // [cap_pages][kv_heads][16][dp]
  int8_t* v = nullptr;      // [cap_pages][kv_heads][dp][16]
  float* ks = nullptr;      // [cap_pages][kv_heads][16]
  float* vs = nullptr;
};

namespace {


size_t kv_page_bytes(const qm_kv* kv) { return (size_t)kv->kv_heads * kv->page_tokens * kv->dp; }
size_t scale_page_count(const qm_kv* kv) { return (size_t)kv->kv_heads * kv->page_tokens; }

struct KvBuffers {
  int32_t* pt = nullptr;
  int8_t *k = nullptr, *v = nullptr;
  float *ks = nullptr, *vs = nullptr;
};

void free_buffers(const KvBuffers& b) {
  (void)hipFree(b.pt);
  (void)hipFree(b.k);
  (void)hipFree(b.v);
  (void)hipFree(b.ks);
  (void)hipFree(b.vs);
}

// Zeroed device buffers for `pages` physical pages (the reference's
// zeroed_shared_buffer); unmaterialised page-table entries point at page 0
// and are never read (only pages below the length are).
qm_status alloc_buffers(const qm_kv* kv, uint32_t pages, KvBuffers* out) {
  KvBuffers b;
  const size_t pb = kv_page_bytes(kv) * pages;
  const size_t sb = scale_page_count(kv) * pages * sizeof(float);
  hipStream_t s = kv->rt->stream;
  hipError_t e = hipMalloc(&b.pt, (size_t)pages * sizeof(int32_t));
  if (e == hipSuccess) e = hipMalloc(&b.k, pb);
  if (e == hipSuccess) e = hipMalloc(&b.v, pb);
  if (e == hipSuccess) e = hipMalloc(&b.ks, sb);
  if (e == hipSuccess) e = hipMalloc(&b.vs, sb);
  if (e == hipSuccess) e = hipMemsetAsync(b.pt, 0, (size_t)pages * sizeof(int32_t), s);
  if (e == hipSuccess) e = hipMemsetAsync(b.k, 0, pb, s);
  if (e == hipSuccess) e = hipMemsetAsync(b.v, 0, pb, s);
  if (e == hipSuccess) e = hipMemsetAsync(b.ks, 0, sb, s);
  if (e == hipSuccess) e = hipMemsetAsync(b.vs, 0, sb, s);
  if (e != hipSuccess) {
    (void)hipGetLastError();
    free_buffers(b);
    return e == hipErrorOutOfMemory ? fail(QM_ERR_OUT_OF_MEMORY, "KV cache: %u pages do not fit in device memory", pages)
                                    : hip_check(e, "KV cache allocation");
  }
  *out = b;
  return QM_OK;
}

void free_kv(qm_kv* kv) {
  if (!kv) return;
  DeviceGuard g(kv->rt->device);
  free_buffers(KvBuffers{kv->d_pt, kv->k, kv->v, kv->ks, kv->vs});
  delete kv;
}

// validate_attention_shape (metal_runtime.rs:9186-9193): head_dim 1..256.
qm_status validate_kv_shape(uint32_t kv_heads, uint32_t head_dim, uint32_t page_tokens) {
  if (kv_heads == 0 || head_dim == 0 || head_dim > 256)
    return fail(QM_ERR_INVALID_ATTENTION_SHAPE, "kv_heads %u / head_dim %u: both must be non-zero, head_dim <= 256",
                kv_heads, head_dim);
  if (page_tokens != 16) return fail(QM_ERR_INVALID_ATTENTION_SHAPE, "page_tokens must be 16");
  return QM_OK;
}

// Physical capacity for `tokens` tokens: the next power of two (at least 16
// tokens), clamped to the hard limit, copying the materialised pages.
// Synchronous when it grows; a no-op otherwise.
qm_status kv_grow(qm_kv* kv, uint64_t tokens) {
  if (kv->max_tokens && tokens > kv->max_tokens)
    return fail(QM_ERR_CAPACITY_EXCEEDED, "token range ending at %llu exceeds page table capacity %u",
                (unsigned long long)tokens, kv->max_tokens);
  const uint64_t need_pages = (tokens + kv->page_tokens - 1) / kv->page_tokens;
  if (need_pages <= kv->cap_pages) return QM_OK;
  uint64_t cap_tokens = 16;
  while (cap_tokens < tokens) cap_tokens <<= 1;
  if (kv->max_tokens) cap_tokens = std::min<uint64_t>(cap_tokens, kv->max_tokens);
  const uint64_t new_pages = (cap_tokens + kv->page_tokens - 1) / kv->page_tokens;
  if (new_pages > (uint64_t)kMaxSplits * kMaxPagesPerSplit || new_pages * kv_page_bytes(kv) > (1ull << 40))
    return fail(QM_ERR_DIMENSION_OVERFLOW, "Q8 KV token capacity %llu", (unsigned long long)cap_tokens);
  DeviceGuard g(kv->rt->device);
  if (!g.ok()) return no_device();
  KvBuffers nb;
  qm_status st = alloc_buffers(kv, (uint32_t)new_pages, &nb);
  if (st != QM_OK) return st;
  hipStream_t s = kv->rt->stream;
  const size_t n = (size_t)kv->next_page_id;
  hipError_t e = hipSuccess;
  if (kv->cap_pages)
    e = hipMemcpyAsync(nb.pt, kv->d_pt, (size_t)kv->cap_pages * sizeof(int32_t), hipMemcpyDeviceToDevice, s);
  if (e == hipSuccess && n) e = hipMemcpyAsync(nb.k, kv->k, n * kv_page_bytes(kv), hipMemcpyDeviceToDevice, s);
  if (e == hipSuccess && n) e = hipMemcpyAsync(nb.v, kv->v, n * kv_page_bytes(kv), hipMemcpyDeviceToDevice, s);
  if (e == hipSuccess && n)
    e = hipMemcpyAsync(nb.ks, kv->ks, n * scale_page_count(kv) * 4, hipMemcpyDeviceToDevice, s);
  if (e == hipSuccess && n)
    e = hipMemcpyAsync(nb.vs, kv->vs, n * scale_page_count(kv) * 4, hipMemcpyDeviceToDevice, s);
  if (e == hipSuccess) e = hipStreamSynchronize(s);
  if (e != hipSuccess) {
    free_buffers(nb);
    return hip_check(e, "KV cache growth");
  }
  // Work queued by other runtimes' streams may still read the old pages.
  if ((e = hipDeviceSynchronize()) != hipSuccess) {
    free_buffers(nb);
    return hip_check(e, "KV cache growth");
  }
  free_buffers(KvBuffers{kv->d_pt, kv->k, kv->v, kv->ks, kv->vs});
  kv->d_pt = nb.pt;
  kv->k = nb.k;
  kv->v = nb.v;
  kv->ks = nb.ks;
  kv->vs = nb.vs;
  kv->cap_pages = (uint32_t)new_pages;
  kv->pages.resize(new_pages, -1);
  return QM_OK;
}

// The pages an append of [start, end) would materialise, without changing
// the table: the first new logical page, how many, and the first new id
// (ids are sequential, LogicalPageTable::append).
void plan_pages(const qm_kv* kv, uint32_t start, uint32_t end, int32_t* first_new, int32_t* count,
                int32_t* first_id) {
  *first_new = -1;
  *count = 0;
  *first_id = -1;
  if (end <= start) return;
  const uint32_t first = start / kv->page_tokens, last = (end - 1) / kv->page_tokens;
  for (uint32_t p = first; p <= last; ++p)
    if (kv->pages[p] < 0) {
      if (*count == 0) {
        *first_new = (int32_t)p;
        *first_id = kv->next_page_id;
      }
      ++*count;
    }
}

// Records a planned append in the host table.  Materialised pages form a
// prefix of the logical pages (appends are sequential and truncation keeps
// pages), so the new ones are consecutive.
void commit_pages(qm_kv* kv, int32_t first_new, int32_t count) {
  for (int32_t i = 0; i < count; ++i) kv->pages[first_new + i] = kv->next_page_id++;
}

void rollback_pages(qm_kv* kv, int32_t first_new, int32_t count) {
  for (int32_t i = count - 1; i >= 0; --i) {
    kv->pages[first_new + i] = -1;
    --kv->next_page_id;
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

qm_status check_heads(uint32_t H, uint32_t KVH) {
  if (H == 0 || H % KVH != 0 || H / KVH > 16)
    return fail(QM_ERR_INVALID_ATTENTION_SHAPE,
                "num_heads %u must be a multiple of kv_heads %u with at most 16 per KV head", H, KVH);
  return QM_OK;
}

// Query/gate rows are read 16 bytes at a time when their rows are.
qm_status check_q_alignment(const uint16_t* q, const uint16_t* gate, uint32_t D) {
  const uintptr_t qa = D % 8 == 0 ? 16 : 2;
  if (!aligned(q, qa) || (gate && !aligned(gate, qa)))
    return fail(QM_ERR_MISALIGNED, "q/gate must be %u-byte aligned", (unsigned)qa);
  return QM_OK;
}

// One launch's worth of decode work (at most kMaxAttnSeqs sequences).
struct DecodeChunk {
  AttnArgs at{};
  uint32_t units = 0;
  uint32_t parts = 0;
  bool combine = false;
};

// Split plan of one chunk.  Each split is a multiple of 4 pages within the
// kernel's page limits, and all splits should run in one residency round:
// one 8-wave workgroup per CU if the splits fit that (measured faster at 32K:
// the CU's waves share one split), else two 4-wave workgroups per CU.
qm_status plan_decode_chunk(qm_runtime* rt, qm_kv* const* seqs, uint32_t nb, DecodeChunk* c) {
  const uint32_t KVH = seqs[0]->kv_heads;
  AttnArgs& at = c->at;
  uint64_t total_pages = 0;
  uint32_t max_pages = 0;
  for (uint32_t i = 0; i < nb; ++i) {
    const qm_kv* kv = seqs[i];
    AttnSeq sd = seq_desc(kv);
    plan_pages(kv, kv->length, kv->length + 1, &sd.new_page_first, &sd.new_page_count, &sd.new_page_id);
    sd.len = kv->length + 1;
    at.seqs[i] = sd;
    const uint32_t pages = (sd.len + 15) / 16;
    total_pages += pages;
    max_pages = std::max(max_pages, pages);
  }
  if ((uint64_t)max_pages > (uint64_t)kMaxSplits * kMaxPagesPerSplit)
    return fail(QM_ERR_CAPACITY_EXCEEDED, "sequence of %u pages exceeds the decode kernel's limit", max_pages);
  auto units_for = [&](uint64_t q) {
    uint64_t u = 0;
    for (uint32_t i = 0; i < nb; ++i) u += ((at.seqs[i].len + 15) / 16 + q - 1) / q * KVH;
    return u;
  };
  const int forced = rt->tune.attn_pps;
  // Pages per split for about `target` workgroups.  Ceil-division per
  // sequence can push the unit count past one residency round, which would
  // leave a nearly empty second round as long as the first: grow the split
  // until every unit fits.
  auto pps_for = [&](uint32_t target) {
    uint64_t pps = (total_pages * KVH + target - 1) / target;
    pps = std::max<uint64_t>(4, (pps + 3) / 4 * 4);
    if (forced > 0) pps = (uint64_t)forced;
    pps = std::max<uint64_t>(pps, (max_pages + kMaxSplits - 1) / kMaxSplits);
    if (forced <= 0)
      while (pps < kMaxPagesPerSplit && units_for(pps) > target) pps += 4;
    return std::min<uint64_t>(pps, kMaxPagesPerSplit);
  };
  const int waves_env = rt->tune.attn_waves;
  const int target_env = rt->tune.attn_target_wgs;
  uint32_t waves = 8;
  uint64_t pps = pps_for(target_env > 0 ? (uint32_t)target_env : rt->cu_count);
  if (waves_env == 4 || (waves_env != 8 && units_for(pps) > (uint64_t)rt->cu_count)) {
    waves = 4;
    pps = pps_for(target_env > 0 ? (uint32_t)target_env : 2 * rt->cu_count);
  }
  uint32_t units = 0, parts = 0;
  for (uint32_t i = 0; i < nb; ++i) {
    const uint32_t pages = (at.seqs[i].len + 15) / 16;
    const uint32_t ns = (uint32_t)((pages + pps - 1) / pps);
    at.seqs[i].unit_begin = units;
    at.seqs[i].nsplit = ns;
    at.seqs[i].part_begin = parts;
    units += ns * KVH;
    if (ns > 1) {
      parts += ns;
      c->combine = true;
    }
  }
  at.pages_per_split = (uint32_t)pps;
  at.wg_waves = waves;
  c->units = units;
  c->parts = parts;
  return QM_OK;
}

// Shared validation of qm_attn_decode and its no-allocation twin.
qm_status check_decode_args(qm_runtime* rt, qm_kv* const* seqs, uint32_t B, const uint16_t* q, const uint16_t* gate,
                            const float* k, const float* v, uint32_t H, const uint16_t* o) {
  if (!rt || !seqs || !q || !k || !v || !o) return fail(QM_ERR_NULL_POINTER, "NULL argument");
  if (B == 0 || B > 64) return fail(QM_ERR_INVALID_ARGUMENT, "batch must be 1..64 sequences");
  const qm_kv* s0 = seqs[0];
  if (!s0) return fail(QM_ERR_NULL_POINTER, "sequence 0 is NULL");
  const uint32_t KVH = s0->kv_heads, D = s0->head_dim;
  qm_status st = check_heads(H, KVH);
  if (st != QM_OK) return st;
  if ((st = check_q_alignment(q, gate, D)) != QM_OK) return st;
  if (!aligned(k, 4) || !aligned(v, 4)) return fail(QM_ERR_MISALIGNED, "k/v must be 4-byte aligned");
  for (uint32_t b = 0; b < B; ++b) {
    if (!seqs[b]) return fail(QM_ERR_NULL_POINTER, "sequence %u is NULL", b);
    if (seqs[b]->kv_heads != KVH || seqs[b]->head_dim != D)
      return fail(QM_ERR_INVALID_ATTENTION_SHAPE, "all sequences must share kv_heads and head_dim");
    if (seqs[b]->rt->device != rt->device) return fail(QM_ERR_INVALID_ARGUMENT, "sequence %u is on another device", b);
    for (uint32_t c = 0; c < b; ++c)
      if (seqs[c] == seqs[b]) return fail(QM_ERR_INVALID_ARGUMENT, "sequence %u appears twice", b);
  }
  return QM_OK;
}

// Plans every chunk; the caller then commits and launches them.  Nothing is
// modified here.
qm_status plan_decode(qm_runtime* rt, qm_kv* const* seqs, uint32_t B, uint32_t H,
                      std::vector<DecodeChunk>* chunks, size_t* partial_bytes) {
  *partial_bytes = 0;
  chunks->clear();
  for (uint32_t b0 = 0; b0 < B; b0 += kMaxAttnSeqs) {
    DecodeChunk c;
    const uint32_t nb = std::min<uint32_t>(kMaxAttnSeqs, B - b0);
    qm_status st = plan_decode_chunk(rt, seqs + b0, nb, &c);
    if (st != QM_OK) return st;
    c.at.n_seqs = nb;
    chunks->push_back(c);
    *partial_bytes = std::max(*partial_bytes, (size_t)c.parts * H * (seqs[0]->dp + 2) * sizeof(float));
  }
  return QM_OK;
}

qm_status launch_decode(qm_runtime* rt, qm_kv* const* seqs, uint32_t B, const uint16_t* q, const uint16_t* gate,
                        const float* k, const float* v, uint32_t H, uint16_t* o, std::vector<DecodeChunk>& chunks,
                        float* partials, size_t partial_bytes) {
  const uint32_t KVH = seqs[0]->kv_heads, D = seqs[0]->head_dim, Dp = seqs[0]->dp;
  // Caches owned by another runtime: their pending growth copies, reserves or
  // prefills on that runtime's stream come first.
  for (uint32_t b = 0; b < B; ++b) {
    qm_status st = stream_after(rt, seqs[b]->rt);
    if (st != QM_OK) return st;
  }
  for (size_t ci = 0; ci < chunks.size(); ++ci) {
    DecodeChunk& c = chunks[ci];
    const uint32_t b0 = (uint32_t)ci * kMaxAttnSeqs, nb = c.at.n_seqs;
    AttnArgs& at = c.at;
    if (c.combine && (size_t)c.parts * H * (Dp + 2) * sizeof(float) > partial_bytes)
      return fail(QM_ERR_INVALID_ARGUMENT, "attention decode: split partials exceed the workspace");
    for (uint32_t i = 0; i < nb; ++i) {
      qm_kv* kv = seqs[b0 + i];
      commit_pages(kv, at.seqs[i].new_page_first, at.seqs[i].new_page_count);
      kv->length += 1;
    }
    at.q = q + (size_t)b0 * H * D;
    at.gate = gate ? gate + (size_t)b0 * H * D : nullptr;
    at.o = o + (size_t)b0 * H * D;
    at.partials = partials;
    at.part_rows = c.parts;
    at.heads = H;
    at.kv_heads = KVH;
    at.head_dim = D;
    at.head_dim_pad = Dp;
    at.prefill = 0;
    at.k_new = k + (size_t)b0 * KVH * D;  // the decode kernel appends the new rows itself
    at.v_new = v + (size_t)b0 * KVH * D;
    hipError_t e = launch_q8_attention(at, c.units, c.combine, rt->stream);
    if (e != hipSuccess) {
      // Nothing of this chunk ran: put its sequences back.
      for (uint32_t i = 0; i < nb; ++i) {
        qm_kv* kv = seqs[b0 + i];
        kv->length -= 1;
        rollback_pages(kv, at.seqs[i].new_page_first, at.seqs[i].new_page_count);
      }
      return hip_check(e, "attention decode launch");
    }
  }
  // ... and later work on their own runtime's stream sees this token.
  for (uint32_t b = 0; b < B; ++b) {
    qm_status st = stream_after(seqs[b]->rt, rt);
    if (st != QM_OK) return st;
  }
  return QM_OK;
}

}  // namespace

uint32_t qm::kv_heads_of(const qm_kv* kv) { return kv->kv_heads; }
uint32_t qm::kv_head_dim_of(const qm_kv* kv) { return kv->head_dim; }
const qm_runtime* qm::kv_runtime_of(const qm_kv* kv) { return kv->rt; }

// Everything qm_attn_decode of one more token could fail on, checked (and
// capacity grown, workspace sized) before a decode step launches anything.
qm_status qm::attn_decode_prepare(qm_runtime* rt, qm_kv* const* seqs, uint32_t B, uint32_t H) {
  if (!rt || !seqs || B == 0) return fail(QM_ERR_NULL_POINTER, "NULL argument");
  for (uint32_t b = 0; b < B; ++b) {
    if (!seqs[b]) return fail(QM_ERR_NULL_POINTER, "sequence %u is NULL", b);
    qm_status st = check_heads(H, seqs[b]->kv_heads);
    if (st != QM_OK) return st;
    if ((st = kv_grow(seqs[b], (uint64_t)seqs[b]->length + 1)) != QM_OK) return st;
  }
  std::vector<DecodeChunk> chunks;
  size_t pb = 0;
  qm_status st = plan_decode(rt, seqs, B, H, &chunks, &pb);
  if (st != QM_OK) return st;
  if (pb && (st = ensure_partials(rt, pb)) != QM_OK) return st;
  return QM_OK;
}

extern "C" {

qm_status qm_kv_create(qm_runtime* rt, uint32_t kv_heads, uint32_t head_dim, uint32_t page_tokens,
                       uint32_t max_tokens, qm_kv** out) {
  if (!rt || !out) return fail(QM_ERR_NULL_POINTER, "runtime/out is NULL");
  *out = nullptr;
  qm_status st = validate_kv_shape(kv_heads, head_dim, page_tokens);
  if (st != QM_OK) return st;
  qm_kv* kv = new qm_kv();
  kv->rt = rt;
  kv->kv_heads = kv_heads;
  kv->head_dim = head_dim;
  kv->dp = attn_padded_dim(head_dim);
  kv->page_tokens = page_tokens;
  kv->max_tokens = max_tokens;
  // allocate_q8_kv_state(kv_heads, head_dim, 16): one page to start with.
  DeviceGuard g(rt->device);
  if (!g.ok()) {
    delete kv;
    return no_device();
  }
  if ((st = kv_grow(kv, max_tokens ? std::min<uint32_t>(16, max_tokens) : 16)) == QM_OK) st = hip_check(hipStreamSynchronize(rt->stream), "KV cache allocation");
  if (st != QM_OK) {
    free_kv(kv);
    return st;
  }
  *out = kv;
  return QM_OK;
}

void qm_kv_destroy(qm_kv* kv) {
  if (!kv) return;
  (void)hipStreamSynchronize(kv->rt->stream);
  free_kv(kv);
}

uint32_t qm_kv_length(const qm_kv* kv) { return kv ? kv->length : 0; }

uint32_t qm_kv_capacity(const qm_kv* kv) {
  if (!kv) return 0;
  const uint32_t held = kv->cap_pages * kv->page_tokens;
  return kv->max_tokens ? std::min(held, kv->max_tokens) : held;
}

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
  if (end > 0xFFFFFFFFull) return fail(QM_ERR_DIMENSION_OVERFLOW, "Q8 KV token capacity");
  qm_status st = kv_grow(kv, end);
  if (st != QM_OK) return st;
  int32_t first, count, id;
  plan_pages(kv, kv->length, (uint32_t)end, &first, &count, &id);
  if (count == 0) return QM_OK;
  commit_pages(kv, first, count);
  DeviceGuard g(kv->rt->device);
  if (!g.ok()) return no_device();
  hipError_t e = hipMemcpyAsync(kv->d_pt + first, kv->pages.data() + first, count * sizeof(int32_t),
                                hipMemcpyHostToDevice, kv->rt->stream);
  if (e == hipSuccess) e = hipStreamSynchronize(kv->rt->stream);
  if (e != hipSuccess) rollback_pages(kv, first, count);
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
  *out = nullptr;
  qm_kv* kv = nullptr;
  qm_status st = qm_kv_create(src->rt, src->kv_heads, src->head_dim, src->page_tokens, src->max_tokens, &kv);
  if (st != QM_OK) return st;
  // Same capacity as the source (clone_q8_kv_state, :7338-7379): its pages
  // may hold more tokens than max_tokens allows, so grow to what it may hold.
  if ((st = kv_grow(kv, qm_kv_capacity(src))) != QM_OK) {
    qm_kv_destroy(kv);
    return st;
  }
  kv->length = src->length;
  std::copy(src->pages.begin(), src->pages.end(), kv->pages.begin());
  kv->next_page_id = src->next_page_id;
  DeviceGuard g(src->rt->device);
  if (!g.ok()) return no_device();
  const size_t n = (size_t)src->next_page_id;
  hipStream_t s = src->rt->stream;
  hipError_t e = hipMemcpyAsync(kv->d_pt, src->d_pt, src->cap_pages * sizeof(int32_t), hipMemcpyDeviceToDevice, s);
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
  if (!g.ok()) return no_device();
  const size_t n = (size_t)kv->next_page_id;
  const uint32_t KVH = kv->kv_heads, D = kv->head_dim, Dp = kv->dp, T = kv->length;
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
        if (keys) keys[((size_t)t * KVH + h) * D + d] = hk[(pkv * 16 + slot) * Dp + d];
        if (values) values[((size_t)t * KVH + h) * D + d] = hv[(pkv * Dp + d) * 16 + slot];
      }
      if (key_scales) key_scales[(size_t)t * KVH + h] = hks[pkv * 16 + slot];
      if (value_scales) value_scales[(size_t)t * KVH + h] = hvs[pkv * 16 + slot];
    }
  }
  return QM_OK;
}

qm_status qm_attn_decode(qm_runtime* rt, qm_kv* const* seqs, uint32_t B, const uint16_t* q, const uint16_t* gate,
                         const float* k, const float* v, uint32_t H, uint16_t* o) {
  qm_status st = check_decode_args(rt, seqs, B, q, gate, k, v, H, o);
  if (st != QM_OK) return st;
  DeviceGuard g(rt->device);
  if (!g.ok()) return no_device();
  // Growth and workspace first: once a chunk is committed nothing but the
  // launch itself can fail.
  if ((st = attn_decode_prepare(rt, seqs, B, H)) != QM_OK) return st;
  std::vector<DecodeChunk> chunks;
  size_t pb = 0;
  if ((st = plan_decode(rt, seqs, B, H, &chunks, &pb)) != QM_OK) return st;
  return launch_decode(rt, seqs, B, q, gate, k, v, H, o, chunks, (float*)rt->partials, rt->partial_bytes);
}

qm_status qm_attn_decode_noalloc(qm_runtime* rt, qm_kv* const* seqs, uint32_t B, const uint16_t* q,
                                 const uint16_t* gate, const float* k, const float* v, uint32_t H, uint16_t* o) {
  qm_status st = check_decode_args(rt, seqs, B, q, gate, k, v, H, o);
  if (st != QM_OK) return st;
  for (uint32_t b = 0; b < B; ++b) {
    const qm_kv* kv = seqs[b];
    if ((uint64_t)kv->length + 1 > qm_kv_capacity(kv))
      return fail(QM_ERR_CAPACITY_EXCEEDED,
                  "sequence %u: no room for another token without allocating (reserve capacity first)", b);
  }
  DeviceGuard g(rt->device);
  if (!g.ok()) return no_device();
  AttnScratch ws{};
  if ((st = hip_check(attn_noalloc_scratch(rt->device, &ws), "attention scratch")) != QM_OK) return st;
  std::vector<DecodeChunk> chunks;
  size_t pb = 0;
  if ((st = plan_decode(rt, seqs, B, H, &chunks, &pb)) != QM_OK) return st;
  if (pb > ws.partial_bytes)
    return fail(QM_ERR_CAPACITY_EXCEEDED, "split partials of %zu bytes exceed the %zu-byte no-allocation scratch", pb,
                ws.partial_bytes);
  if ((st = hip_check(attn_noalloc_begin(rt->device, rt->stream), "no-allocation ordering")) != QM_OK) return st;
  st = launch_decode(rt, seqs, B, q, gate, k, v, H, o, chunks, ws.partials, ws.partial_bytes);
  const qm_status end = hip_check(attn_noalloc_end(rt->device, rt->stream), "no-allocation ordering");
  return st != QM_OK ? st : end;
}

qm_status qm_attn_prefill(qm_runtime* rt, qm_kv* seq, const uint16_t* q, const uint16_t* gate, const float* k,
                          const float* v, uint32_t H, uint32_t M, uint16_t* o) {
  if (!rt || !seq || !q || !k || !v || !o) return fail(QM_ERR_NULL_POINTER, "NULL argument");
  if (M == 0) return fail(QM_ERR_INVALID_ATTENTION_SHAPE, "prefill needs at least one row");
  const uint32_t KVH = seq->kv_heads, D = seq->head_dim;
  qm_status st = check_heads(H, KVH);
  if (st != QM_OK) return st;
  if ((st = check_q_alignment(q, gate, D)) != QM_OK) return st;
  if (!aligned(k, 4) || !aligned(v, 4)) return fail(QM_ERR_MISALIGNED, "k/v must be 4-byte aligned");
  if (seq->rt->device != rt->device) return fail(QM_ERR_INVALID_ARGUMENT, "the cache is on another device");
  const uint64_t end = (uint64_t)seq->length + M;
  if (end > 0xFFFFFFFFull) return fail(QM_ERR_DIMENSION_OVERFLOW, "Q8 KV token capacity");
  DeviceGuard g(rt->device);
  if (!g.ok()) return no_device();
  if ((st = kv_grow(seq, end)) != QM_OK) return st;
  const uint32_t start = seq->length;
  AttnSeq sd = seq_desc(seq);
  plan_pages(seq, start, start + M, &sd.new_page_first, &sd.new_page_count, &sd.new_page_id);
  sd.len = start + M;
  AppendArgs ap{};
  ap.k = k;
  ap.v = v;
  ap.kv_heads = KVH;
  ap.head_dim = D;
  ap.head_dim_pad = seq->dp;
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
  at.head_dim_pad = seq->dp;
  at.n_seqs = 1;
  at.prefill = 1;
  at.rows = M;
  at.start = start;
  at.seqs[0] = sd;
  at.prefill_cb = rt->tune.prefill_cb;
  // A cache owned by another runtime: its pending work comes first.
  if ((st = stream_after(rt, seq->rt)) != QM_OK) return st;
  commit_pages(seq, sd.new_page_first, sd.new_page_count);
  seq->length = start + M;
  hipError_t e = launch_q8_append(ap, M, rt->stream);
  // The prefill launcher sizes its own grid (rows per workgroup depend on the
  // kernel's column blocks).
  if (e == hipSuccess) e = launch_q8_attention(at, 0, false, rt->stream);
  if (e != hipSuccess) {
    seq->length = start;
    rollback_pages(seq, sd.new_page_first, sd.new_page_count);
    return hip_check(e, "attention prefill launch");
  }
  return stream_after(seq->rt, rt);
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
  DeviceGuard g(rt->device);
  if (!g.ok()) return no_device();
  return hip_check(launch_attn_prepare(a, rt->stream), "attention prepare launch");
}
