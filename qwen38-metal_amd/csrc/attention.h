// Launch interface of the paged Q8-KV attention kernels (q8_attention.hip).
#pragma once
#include <hip/hip_runtime.h>
#include <stdint.h>

namespace qm {

constexpr int kMaxAttnSeqs = 16;  // sequences per launch (kernel-argument table)
constexpr int kMaxSplits = 2048;         // page splits per sequence
constexpr int kMaxPagesPerSplit = 1024;  // pages per decode workgroup

// Storage dimension of a cache with head dimension d (1..256): pages hold
// the next kernel width, the extra dimensions are zero.
inline uint32_t attn_padded_dim(uint32_t d) { return d <= 64 ? 64 : d <= 128 ? 128 : 256; }

struct AttnSeq {
  int8_t* k;          // K pages   [page][kv_head][16][D]
  int8_t* v;          // V pages   [page][kv_head][D][16]
  float* ks;          // K scales  [page][kv_head][16]
  float* vs;          // V scales  [page][kv_head][16]
  int32_t* pt;        // page table: logical page -> physical page
  uint32_t len;       // tokens in the cache after this call's append
  uint32_t unit_begin;  // first workgroup of this sequence (decode)
  uint32_t nsplit;      // page splits (decode)
  uint32_t part_begin;  // first partial row of this sequence (decode)
  int32_t new_page_first;  // logical index of the first page materialised by this call
  int32_t new_page_count;
  int32_t new_page_id;     // physical id of that page (ids are consecutive)
};

struct AppendArgs {
  const float* k;  // [items][kv_heads][D]
  const float* v;
  uint32_t kv_heads;
  uint32_t head_dim;      // real head dimension (strides of k and v)
  uint32_t head_dim_pad;  // storage dimension of the cache pages (64, 128 or 256)
  uint32_t decode;  // 1: item = sequence (one token each); 0: item = row of seqs[0]
  uint32_t start;   // prefill: cache position of row 0
  AttnSeq seqs[kMaxAttnSeqs];
};

struct AttnArgs {
  const uint16_t* q;     // bf16 [rows][H][D]
  const uint16_t* gate;  // bf16 [rows][H][D] or null
  uint16_t* o;           // bf16 [rows][H][D]
  float* partials;       // decode split partials: O [split rows][H][Dp], then (m, l) [split rows][H][2]
  const float* k_new;    // decode: fp32 [n_seqs][kv_heads][D] rows appended by the kernel
  const float* v_new;
  uint32_t heads;
  uint32_t kv_heads;
  uint32_t head_dim;      // real head dimension (strides of q, gate, o, k_new, v_new)
  uint32_t head_dim_pad;  // storage dimension Dp of the cache pages (64, 128 or 256)
  uint32_t part_rows;     // decode: split rows in `partials` (offset of the (m, l) table)
  uint32_t n_seqs;
  uint32_t pages_per_split;  // decode
  uint32_t wg_waves;         // decode: waves per workgroup (4: two workgroups per CU; 8: one)
  int32_t prefill_cb;        // prefill: column blocks per wave (0: the default for D)
  uint32_t prefill;
  uint32_t rows;   // prefill: query rows
  uint32_t start;  // prefill: cache position of row 0
  AttnSeq seqs[kMaxAttnSeqs];
};

// Split partials of qm_attn_decode_noalloc: a file-scope device array of the
// attention source (one copy per GPU, held until the process ends) whose
// address is looked up once per device with that device current.
struct AttnScratch {
  float* partials;
  size_t partial_bytes;
};
hipError_t attn_noalloc_scratch(int device, AttnScratch* out);
// Brackets the launches of one call that uses the array (after
// attn_noalloc_scratch succeeded on the device): begin takes the device's
// lock and, when the previous call ran on another stream, makes `stream`
// wait for that call's completion event; end records this call's event on
// `stream` and releases the lock.  So calls from several streams or threads
// on one GPU run one after another on the device instead of racing on the
// shared partials.
hipError_t attn_noalloc_begin(int device, hipStream_t stream);
hipError_t attn_noalloc_end(int device, hipStream_t stream);

hipError_t launch_q8_append(const AppendArgs& a, uint32_t items, hipStream_t st);
// Decode: `units` workgroups; when need_combine, q8_combine_kernel merges the
// split partials (which must be set) in a second launch.
hipError_t launch_q8_attention(const AttnArgs& a, uint32_t units, bool need_combine, hipStream_t st);

}  // namespace qm
