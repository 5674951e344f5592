/*
 * qm38 — MI355X (gfx950) per-token compute path of a Qwen3.8-style hybrid
 * model: MLX affine-Q4 projections, paged Q8-KV GQA attention and the Gated
 * DeltaNet conv/recurrent update.
 *
 * This is the drop-in C ABI.  Every entry point mirrors one method of the
 * reference runtime (`MetalRuntime` in /root/reference/src/metal_runtime.rs)
 * and cites the function it replaces.  The ABI is plain C: device pointers,
 * sizes and opaque handles, no C++ or torch types.
 *
 * Conventions
 *   - Activation/output pointers are DEVICE pointers (hipMalloc'd or any
 *     allocator's HBM).  Weight creation helpers take HOST pointers, like the
 *     reference's `create_*` constructors, and upload them.
 *   - bf16 values travel as uint16_t bit patterns (bf16 -> f32 is `bits<<16`,
 *     f32 -> bf16 is round-to-nearest-even, reference qwen38.metal:18-26).
 *   - Every call is enqueued on the runtime's stream (qm_runtime_set_stream)
 *     and is asynchronous unless stated otherwise; qm_runtime_synchronize
 *     waits for completion (the reference's commit()+wait_until_completed()).
 *   - Calls that share one runtime must not overlap from several threads on
 *     the same stream unless the caller serialises them; distinct runtimes are
 *     independent.  Errors are returned as qm_status and the message of the
 *     last error on the calling thread is available from
 *     qm_last_error_message().
 */
#ifndef QM38_H
#define QM38_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* Status codes.  One code per variant of MetalRuntimeError
 * (metal_runtime.rs:9219-9247) that can occur on this path, plus the
 * LogicalPageTable errors (paged_kv.rs:100-105). */
typedef enum qm_status {
  QM_OK = 0,
  QM_ERR_NO_DEVICE = 1,             /* MetalRuntimeError::NoDevice */
  QM_ERR_EMPTY_DIMENSION = 2,       /* ::EmptyDimension */
  QM_ERR_INPUT_NOT_GROUPED = 3,     /* ::InputNotGrouped */
  QM_ERR_WRONG_LENGTH = 4,          /* ::WrongLength */
  QM_ERR_INVALID_DELTANET_CONFIG = 5, /* ::InvalidDeltaNetConfig */
  QM_ERR_INVALID_ATTENTION_SHAPE = 6, /* ::InvalidAttentionShape */
  QM_ERR_INVALID_SEQUENCE_LENGTH = 7, /* ::InvalidSequenceLength */
  QM_ERR_INVALID_BUFFER_OFFSET = 8,   /* ::InvalidBufferOffset */
  QM_ERR_MAPPED_TENSOR_OUT_OF_RANGE = 9, /* ::MappedTensorOutOfRange */
  QM_ERR_DIMENSION_OVERFLOW = 10,   /* ::DimensionOverflow */
  QM_ERR_COMMAND_FAILED = 11,       /* ::CommandFailed (HIP launch/runtime error) */
  QM_ERR_ZERO_CAPACITY = 12,        /* PageTableError::ZeroCapacity */
  QM_ERR_EMPTY_APPEND = 13,         /* PageTableError::EmptyAppend */
  QM_ERR_CAPACITY_EXCEEDED = 14,    /* PageTableError::CapacityExceeded */
  QM_ERR_NULL_POINTER = 15,         /* a required pointer argument is NULL */
  QM_ERR_OUT_OF_MEMORY = 16,        /* device allocation failed */
  QM_ERR_MISALIGNED = 17,           /* a device pointer violates the documented alignment */
  QM_ERR_INVALID_ARGUMENT = 18,     /* any other precondition */
  QM_ERR_INVALID_SNAPSHOT = 19,     /* MetalRuntimeError::InvalidDeltaNetSnapshot */
  QM_ERR_INVALID_SNAPSHOT_ROW = 20, /* ::InvalidSnapshotRow */
  QM_ERR_MODEL_FORMAT = 21,         /* model::ModelFormatError (index, shard or header) */
  QM_ERR_INVALID_TENSOR = 22,       /* native::NativeError tensor variants (MissingTensor,
                                       NotQuantizedWeight, InvalidQuantizedWeight,
                                       InvalidAffineTensor, TensorByteLength) */
  QM_ERR_GRAPH_STALE = 23           /* a decode graph's captured buffers or state parity changed */
} qm_status;

/* Human-readable name of a status code (static storage). */
const char* qm_status_string(qm_status status);
/* Message describing the last error raised on the calling thread. */
const char* qm_last_error_message(void);

/* ------------------------------------------------------------------ */
/* Runtime                                                             */
/* ------------------------------------------------------------------ */
typedef struct qm_runtime qm_runtime;

/* Replaces MetalRuntime::new (metal_runtime.rs:641-927): binds HIP device
 * `device`, creates the runtime's scratch pools.  The default stream is the
 * device's null stream.  device = QM_DEVICE_NONE makes a runtime without a
 * device (no counterpart in the reference): every entry point still checks
 * its arguments and returns their error, and returns QM_ERR_NO_DEVICE where
 * it would touch a device.  It lets argument validation run on a host with
 * no GPU (tests, dry runs). */
#define QM_DEVICE_NONE (-1)
qm_status qm_runtime_create(int device, qm_runtime** out);
void qm_runtime_destroy(qm_runtime* rt);
/* Enqueue all later work of `rt` on `hip_stream` (a hipStream_t; NULL selects
 * the null stream).  The stream must belong to the runtime's device. */
qm_status qm_runtime_set_stream(qm_runtime* rt, void* hip_stream);
/* Blocks until all work enqueued by `rt` has finished; surfaces asynchronous
 * kernel failures as QM_ERR_COMMAND_FAILED (the reference checks
 * MTLCommandBufferStatus::Error after wait_until_completed, e.g.
 * metal_runtime.rs:3660-3665). */
qm_status qm_runtime_synchronize(qm_runtime* rt);

/* Device buffers owned by the runtime's allocator (256-byte aligned).
 * Replaces the reference's buffer_from_slice / map_weight_store
 * (metal_runtime.rs:955-984): on MI355X weights must be resident in HBM, so
 * the upload realigns them and the reference's byte-addressed `_unaligned`
 * kernel twins are unnecessary. */
qm_status qm_device_alloc(qm_runtime* rt, size_t bytes, void** out);
qm_status qm_device_free(qm_runtime* rt, void* ptr);
qm_status qm_upload(qm_runtime* rt, const void* host, size_t bytes, void** out);
/* Synchronous copies between host and device memory on the runtime stream. */
qm_status qm_copy_to_device(qm_runtime* rt, void* dst, const void* host, size_t bytes);
qm_status qm_copy_to_host(qm_runtime* rt, void* host, const void* src, size_t bytes);

/* ------------------------------------------------------------------ */
/* MLX affine-Q4 projections                                           */
/* ------------------------------------------------------------------ */
/* One Q4 projection (replaces MappedQ4AffineJob, metal_runtime.rs:155-192).
 * Layout (native.rs:5384-5516): `weights` u32 [out_rows][in/8], eight 4-bit
 * values per word, low nibble first; `scales`/`biases` bf16
 * [out_rows][in/64].  Device pointers; weights and scales/biases must be
 * 8-byte aligned. */
typedef struct qm_q4_job {
  const uint32_t* weights;
  const uint16_t* scales;
  const uint16_t* biases;
  uint32_t out_rows;
} qm_q4_job;

/* Every Q4 entry point below checks, on a device runtime and before anything
 * is launched, that each tensor a job names lies inside one device
 * allocation (hipMemGetAddressRange): weights out_rows*in/8 u32, scales and
 * biases out_rows*in/64 bf16, and likewise the activation and output
 * buffers.  A pointer inside no allocation fails with
 * QM_ERR_INVALID_BUFFER_OFFSET, a tensor running past the end of its
 * allocation with QM_ERR_MAPPED_TENSOR_OUT_OF_RANGE, as
 * validate_mapped_q4_affine_shape does for Metal buffers
 * (metal_runtime.rs:8854-8898). */

/* A device allocation and its length: the C counterpart of the
 * `&metal::Buffer` a MappedQ4AffineJob borrows. */
typedef struct qm_buffer {
  const void* base;
  uint64_t length; /* bytes */
} qm_buffer;

/* MappedQ4AffineJob (metal_runtime.rs:155-192): three tensors given as
 * (buffer, byte offset), for weights mapped from one large checkpoint
 * allocation.  The reference's `aligned` flag selects its unaligned kernel
 * twins; here the resolved pointers must be 8-byte aligned instead. */
typedef struct qm_q4_mapped_job {
  qm_buffer weights;
  uint64_t weight_offset;
  qm_buffer scales;
  uint64_t scale_offset;
  qm_buffer biases;
  uint64_t bias_offset;
  uint32_t out_rows;
} qm_q4_mapped_job;

/* Resolves a mapped job for input width in_elems into a qm_q4_job, with the
 * checks of validate_mapped_q4_affine_shape (metal_runtime.rs:8854-8898), in
 * its order: EMPTY_DIMENSION (in_elems or out_rows zero), INPUT_NOT_GROUPED
 * (in_elems % 64), INVALID_BUFFER_OFFSET (an offset beyond its buffer's
 * length), DIMENSION_OVERFLOW, MAPPED_TENSOR_OUT_OF_RANGE (a tensor longer
 * than what its buffer holds past the offset); then NULL_POINTER and
 * MISALIGNED.  Host only: reads no device memory. */
qm_status qm_q4_job_from_mapped(const qm_q4_mapped_job* mapped, uint32_t in_elems, qm_q4_job* out);

/* y_j[m][n] = sum_g ( s_j[n][g] * sum_{i in g} q_j[n][i] x[m][i]
 *                    + b_j[n][g] * sum_{i in g} x[m][i] )
 * for every job j, all jobs reading the same activation x (bf16 [M][in]).
 * outputs[j] is bf16 [M][out_rows_j].  fp32 accumulation.
 * Replaces q4_affine_matvec_mapped_batch (metal_runtime.rs:3599) for M == 1
 * and q4_affine_matmul_mapped_batch (metal_runtime.rs:3683) for M > 1; rows
 * M <= 16 take the decode (weight-streaming) kernel, larger M the tiled MFMA
 * GEMM.  n_jobs <= 8.  in_elems is at most 2^24 (DIMENSION_OVERFLOW beyond:
 * the kernels address one row's bytes and a tile of rows with 32-bit
 * offsets). */
qm_status qm_q4_project(qm_runtime* rt, const qm_q4_job* jobs, int n_jobs,
                        const uint16_t* x, uint32_t in_elems, uint32_t M,
                        uint16_t* const* outputs);

/* Same-input projections, plain ones and gate/up pairs together: for
 * ups == NULL or ups[j] == NULL, outputs[j] = jobs[j](x) (bf16 [M][rows]);
 * otherwise outputs[j] = bf16( silu(jobs[j](x)) * ups[j](x) ), with
 * ups[j]->out_rows == jobs[j].out_rows.  For one activation row the whole set
 * is one launch that reads x once (the reference's mapped batch, whose jobs
 * would be a QKV projection and the pair kernels' gate/up, metal_runtime.rs:
 * 3599 with qwen38.metal:1404..3643); so are two rows, and M > 16 (one GEMM
 * launch over plain and pair tiles).  M = 3..16 runs the plain jobs together
 * and each pair as qm_q4_swiglu does.  n_jobs <= 8. */
qm_status qm_q4_project_set(qm_runtime* rt, const qm_q4_job* jobs, const qm_q4_job* const* ups, int n_jobs,
                            const uint16_t* x, uint32_t in_elems, uint32_t M, uint16_t* const* outputs);

/* h[m][n] = bf16( silu(gate(x)[m][n]) * up(x)[m][n] ): the gate and up
 * projections of one MLP share the activation read and SwiGLU
 * (qwen38.metal:4188-4199, silu at 4090-4096) runs in the epilogue.
 * gate.out_rows must equal up.out_rows.  Replaces the pair kernels
 * (qwen38.metal:1404..3643, encode_q4_affine_matmul_pair
 * metal_runtime.rs:6372). */
qm_status qm_q4_swiglu(qm_runtime* rt, const qm_q4_job* gate, const qm_q4_job* up,
                       const uint16_t* x, uint32_t in_elems, uint32_t M,
                       uint16_t* h);

/* y = down( silu(gate(x)) * up(x) ): replaces q4_affine_mlp_mapped_batch
 * (metal_runtime.rs:4479-4689).  The bf16 intermediate h [M][gate.out_rows]
 * lives in runtime scratch.  down's input width must equal gate.out_rows. */
qm_status qm_q4_mlp(qm_runtime* rt, const qm_q4_job* gate, const qm_q4_job* up,
                    const qm_q4_job* down, const uint16_t* x, uint32_t in_elems,
                    uint32_t M, uint16_t* y);

/* Greedy token of every row: ids[m] = argmax_n y[m][n] over the fp32 (not
 * bf16-rounded) projection y = job(x), the lowest index winning ties and NaN
 * logits never winning (an all-NaN row gives 0).  Only the M ids reach
 * memory; the logits never do.  ids is a device pointer, uint32 [M].
 * Replaces q4_affine_argmax_mapped_batch (metal_runtime.rs:3797-3890) with
 * qwen38_argmax_rows (qwen38.metal:4202-4244). */
qm_status qm_q4_argmax(qm_runtime* rt, const qm_q4_job* job, const uint16_t* x,
                       uint32_t in_elems, uint32_t M, uint32_t* ids);

/* ------------------------------------------------------------------ */
/* Paged Q8 KV cache                                                   */
/* ------------------------------------------------------------------ */
typedef struct qm_kv qm_kv;

/* Replaces create_q8_kv_state (metal_runtime.rs:7298) and
 * LogicalPageTable::new (paged_kv.rs:22-35).  K/V are int8 with one fp32
 * scale per token and KV head.  Physical layout (HBM), per page of
 * `page_tokens` tokens, with Dp = 64, 128 or 256 the smallest of these
 * >= head_dim (dimensions past head_dim hold zero):
 *   K pages  int8 [page][kv_head][page_tokens][Dp]
 *   V pages  int8 [page][kv_head][Dp][page_tokens]   (d-major)
 *   scales   fp32 [page][kv_head][page_tokens]  (one array for K, one for V)
 * Pages materialise lazily as tokens arrive and receive sequential page ids
 * (paged_kv.rs:89-97).  head_dim 1..256 and kv_heads > 0
 * (validate_attention_shape, metal_runtime.rs:9186-9193); page_tokens must
 * be 16.  Capacity starts at 16 tokens and grows on demand to the next power
 * of two of the required length, copying the cache (ensure_q8_kv_capacity,
 * metal_runtime.rs:7406-7421).  max_tokens = 0 grows without limit, as the
 * reference does; otherwise appends past max_tokens fail with
 * QM_ERR_CAPACITY_EXCEEDED (LogicalPageTable's capacity, paged_kv.rs:54-62). */
qm_status qm_kv_create(qm_runtime* rt, uint32_t kv_heads, uint32_t head_dim,
                       uint32_t page_tokens, uint32_t max_tokens, qm_kv** out);
void qm_kv_destroy(qm_kv* kv);
/* Active sequence length (Q8KvState::sequence_length, metal_runtime.rs:595). */
uint32_t qm_kv_length(const qm_kv* kv);
/* Tokens the cache holds without growing (Q8KvState::capacity_tokens,
 * metal_runtime.rs:578-593). */
uint32_t qm_kv_capacity(const qm_kv* kv);
/* Number of materialised pages (LogicalPageTable::allocated_pages). */
uint32_t qm_kv_allocated_pages(const qm_kv* kv);
/* Physical page id backing `token`, or -1 if token >= length
 * (LogicalPageTable::page_for_token, paged_kv.rs:77-85). */
int64_t qm_kv_page_for_token(const qm_kv* kv, uint32_t token);
/* Ensures capacity for `additional` more tokens (reserve_q8_kv_tokens,
 * metal_runtime.rs:7307-7317): grows the cache if needed and materialises
 * the pages they will need. */
qm_status qm_kv_reserve(qm_kv* kv, uint32_t additional);
/* Moves the logical end backwards (truncate_q8_kv_tokens, :7323-7333). */
qm_status qm_kv_truncate(qm_kv* kv, uint32_t length);
/* Copies the active prefix into a new cache (clone_q8_kv_state, :7338-7379). */
qm_status qm_kv_clone(const qm_kv* src, qm_kv** out);
/* Copies the active tokens' K/V bytes and scales out in the reference's
 * contiguous token-major layout (Q8KvState, metal_runtime.rs:578-593):
 * keys/values int8 [len][kv_heads][head_dim], scales fp32 [len][kv_heads].
 * Host pointers; synchronous.  Any pointer may be NULL to skip it. */
qm_status qm_kv_read(const qm_kv* kv, int8_t* keys, int8_t* values,
                     float* key_scales, float* value_scales);

/* Decode attention for a ragged batch of B sequences (B <= 64): appends one
 * token per sequence (quantised K/V, qwen38_q8_kv_append, qwen38.metal:
 * 5031-5080) and attends over the whole cache including it.
 *   q    bf16 [B][H][head_dim]      gate bf16 [B][H][head_dim] or NULL
 *   k, v fp32 [B][kv_heads][head_dim]
 *   o    bf16 [B][H][head_dim] = softmax(q K^T / sqrt(d)) V * sigmoid(gate)
 * Replaces gqa_attention_q8 (metal_runtime.rs:8230-8425; kernels
 * qwen38_gqa_q8_scores/values, qwen38.metal:5240-5323).  All sequences must
 * share kv_heads/head_dim; H % kv_heads == 0 with at most 16 query heads per
 * KV head.  q/gate must be 16-byte aligned when head_dim % 8 == 0.  Caches
 * grow as needed before anything is launched. */
qm_status qm_attn_decode(qm_runtime* rt, qm_kv* const* seqs, uint32_t B,
                         const uint16_t* q, const uint16_t* gate,
                         const float* k, const float* v, uint32_t H,
                         uint16_t* o);

/* qm_attn_decode that allocates nothing: no counterpart in the reference.
 * For callers that cannot allocate device memory (tight serving loops,
 * harnesses that forbid hipMalloc).  It is not meant for HIP graph capture:
 * each call advances the caches' host-side length and page table when it is
 * made, so a captured call would describe exactly one position (valid for one
 * replay, and only while no later call grows the caches).  The split
 * partials live in a fixed 16 MiB device array of the library, one per GPU,
 * held until the process ends.  The caches are not grown: every sequence
 * must have room for its token (qm_kv_reserve beforehand), else
 * QM_ERR_CAPACITY_EXCEEDED; a split plan needing more than 16 MiB of
 * partials (H * (head_dim_pad + 2) * 4 bytes per split) fails with
 * QM_ERR_CAPACITY_EXCEEDED as well.  All calls on one GPU share the array,
 * so the library orders them: a call made on another stream than the
 * previous call on that GPU first makes its stream wait for the previous
 * call's completion (an event the library records after every call), and
 * calls from several threads take a per-GPU lock while they enqueue.  Calls
 * therefore run one after another on the GPU; they never overlap. */
qm_status qm_attn_decode_noalloc(qm_runtime* rt, qm_kv* const* seqs, uint32_t B,
                                 const uint16_t* q, const uint16_t* gate,
                                 const float* k, const float* v, uint32_t H,
                                 uint16_t* o);

/* Rotary configuration of the full-attention layers (RopeParameters,
 * native.rs:119-197; MetalGqaDecodeConfig, metal_runtime.rs).
 * rotary_dim = round(head_dim * partial_rotary_factor), even, <= head_dim.
 * With has_mrope_sections, RoPE frequency i of the rotary half uses position
 * axis 1 when i % 3 == 1 and i / 3 < mrope_section1, axis 2 when i % 3 == 2
 * and i / 3 < mrope_section2, else axis 0 (native.rs:136-148). */
typedef struct qm_rope_config {
  uint32_t head_dim;   /* 1..256 */
  uint32_t rotary_dim;
  float rope_theta;    /* > 0 */
  uint32_t mrope_section1, mrope_section2;
  uint32_t has_mrope_sections;
} qm_rope_config;

/* Full-attention q/k preparation for M rows, the step between the q/k
 * projections and qm_attn_decode / qm_attn_prefill:
 *   q_with_gate bf16 [M][H][2 head_dim]  query | gate per head (the packed
 *                                        q_proj output)
 *   k_in        bf16 [M][kv_heads][head_dim]
 *   q_norm, k_norm fp32 [head_dim]       per-head RMSNorm weights
 *   positions   uint32 [3][M] (axis-major) or NULL: all axes = position_base + row
 *   q_out, gate_out bf16 [M][H][head_dim];  k_out fp32 [M][kv_heads][head_dim]
 * q = rope(rmsnorm(query) * q_norm), gate copied, k = rope(rmsnorm(k) * k_norm).
 * Replaces qwen38_gqa_prepare_query(_rows) / qwen38_gqa_prepare_key(_rows)
 * (qwen38.metal:4761-5029; encoders metal_runtime.rs:5171-5420) and the CPU
 * split_query_and_gate / rms_norm_slice / apply_mrope (native.rs:4917-4942,
 * 5153-5180).  The rotation angle is evaluated in fp64 (the reference: fp32).
 * Device pointers, asynchronous on the runtime's stream; when head_dim % 4 == 0
 * the bf16 buffers must be 8-byte and k_out 16-byte aligned. */
qm_status qm_attn_prepare(qm_runtime* rt, const qm_rope_config* rope, uint32_t M,
                          uint32_t H, uint32_t kv_heads, const uint16_t* q_with_gate,
                          const uint16_t* k_in, const float* q_norm, const float* k_norm,
                          float epsilon, const uint32_t* positions, uint32_t position_base,
                          uint16_t* q_out, uint16_t* gate_out, float* k_out);

/* Causal prefill of M new rows: appends them (qwen38_q8_kv_append_prefill,
 * qwen38.metal:5085-5140) and computes, for row i, attention over the first
 * min(start+i+1, total) tokens (qwen38_gqa_q8_prefill_attention,
 * qwen38.metal:5146-5238).  Layouts as qm_attn_decode with B replaced by M.
 * Replaces gqa_attention_q8_prefill (metal_runtime.rs:8598). */
qm_status qm_attn_prefill(qm_runtime* rt, qm_kv* seq, const uint16_t* q,
                          const uint16_t* gate, const float* k, const float* v,
                          uint32_t H, uint32_t M, uint16_t* o);

/* ------------------------------------------------------------------ */
/* Gated DeltaNet                                                      */
/* ------------------------------------------------------------------ */
/* DeltaNetConfig (metal_runtime.rs:487-494). */
typedef struct qm_dn_config {
  uint32_t key_heads;
  uint32_t value_heads;
  uint32_t key_head_dim;
  uint32_t value_head_dim;
  uint32_t conv_kernel_size;
} qm_dn_config;

typedef struct qm_dn_weights qm_dn_weights;
typedef struct qm_dn_state qm_dn_state;

/* Replaces create_deltanet_weights (metal_runtime.rs:7143-7183).  HOST
 * pointers: conv_weight fp32 [channels][kernel], a_log/dt_bias fp32
 * [value_heads], norm fp32 [value_head_dim]; channels =
 * 2*key_heads*key_head_dim + value_heads*value_head_dim.  Head dimensions
 * up to 256 and value_heads % key_heads == 0 (validate_deltanet_config,
 * metal_runtime.rs:9151-9168), else QM_ERR_INVALID_DELTANET_CONFIG. */
qm_status qm_dn_weights_create(qm_runtime* rt, const qm_dn_config* cfg,
                               const float* conv_weight, const float* a_log,
                               const float* dt_bias, const float* norm,
                               qm_dn_weights** out);
void qm_dn_weights_destroy(qm_dn_weights* w);
/* Replaces create_deltanet_state (:7185-7199): zeroed conv history fp32
 * [channels][kernel-1] and recurrent state fp32
 * [value_heads][value_head_dim][key_head_dim]. */
qm_status qm_dn_state_create(qm_runtime* rt, const qm_dn_weights* w, qm_dn_state** out);
void qm_dn_state_destroy(qm_dn_state* st);
/* Replaces clone_deltanet_state (:7287-7296). */
qm_status qm_dn_state_clone(const qm_dn_state* src, qm_dn_state** out);
/* Synchronous host copies of the current state (either pointer may be NULL). */
qm_status qm_dn_state_read(const qm_dn_state* st, float* conv_history, float* recurrent);
qm_status qm_dn_state_write(qm_dn_state* st, const float* conv_history, const float* recurrent);

/* One decode token (replaces deltanet_step, metal_runtime.rs:7459-7636;
 * kernels qwen38_deltanet_conv/prepare/recurrence/gate_norm,
 * qwen38.metal:4376-4527).  Device pointers: qkv fp32 [channels], z fp32
 * [value_heads*value_head_dim], b and a fp32 [value_heads]; out fp32
 * [value_heads*value_head_dim]. */
qm_status qm_dn_step(qm_runtime* rt, const qm_dn_weights* w, qm_dn_state* st,
                     const float* qkv, const float* z, const float* b,
                     const float* a, float epsilon, float* out);

/* Causal prefill of M tokens with a chunked scan that equals M applications
 * of qm_dn_step (replaces deltanet_prefill / deltanet_prefill_from,
 * metal_runtime.rs:7933-7990, kernel qwen38_deltanet_prefill
 * qwen38.metal:4530-4758).  `from` (may be NULL, meaning `to`) supplies the
 * initial state and is not modified unless it is `to`.  Layouts as
 * qm_dn_step with a leading [M] dimension.  M x channels (2 key_heads
 * key_head_dim + value_heads value_head_dim) is at most 2^31 - 1
 * (DIMENSION_OVERFLOW beyond). */
qm_status qm_dn_prefill(qm_runtime* rt, const qm_dn_weights* w,
                        const qm_dn_state* from, qm_dn_state* to,
                        const float* qkv, const float* z, const float* b,
                        const float* a, uint32_t M, float epsilon, float* out);

/* State images for speculative verification (MTP).  A verification prefill
 * of M rows can record the state after each of its first M - 1 rows; the
 * final row's state is the destination state as usual.  Replaces
 * MetalDeltaNetSnapshots: create_deltanet_snapshots (metal_runtime.rs:
 * 7201-7232), deltanet_prefill_from_with_snapshots (7998-8024) and
 * restore_deltanet_snapshot (7239-7281). */
typedef struct qm_dn_snapshots qm_dn_snapshots;

/* Room for `rows` images (rows > 0) of states of these weights. */
qm_status qm_dn_snapshots_create(qm_runtime* rt, const qm_dn_weights* w, uint32_t rows,
                                 qm_dn_snapshots** out);
void qm_dn_snapshots_destroy(qm_dn_snapshots* snaps);

/* qm_dn_prefill that also writes the state after row r into image r for
 * r < M - 1 (requires M - 1 <= rows, else QM_ERR_INVALID_SNAPSHOT). */
qm_status qm_dn_prefill_snapshots(qm_runtime* rt, const qm_dn_weights* w,
                                  const qm_dn_state* from, qm_dn_state* to,
                                  qm_dn_snapshots* snaps, const float* qkv,
                                  const float* z, const float* b, const float* a,
                                  uint32_t M, float epsilon, float* out);

/* Makes `dst` the state after verification row `row` (row < rows, else
 * QM_ERR_INVALID_SNAPSHOT_ROW).  A one-row set exchanges its buffers with
 * dst's instead of copying (the image then holds dst's former state), as the
 * reference does; otherwise an asynchronous device copy on the runtime's
 * stream. */
qm_status qm_dn_snapshot_restore(qm_dn_snapshots* snaps, uint32_t row, qm_dn_state* dst);

/* ------------------------------------------------------------------ */
/* MLX safetensors weight store (on-disk format of the Q4 checkpoints)  */
/* ------------------------------------------------------------------ */

/* Opens a model directory: model.safetensors.index.json (tensor -> shard) and
 * the shards it names, memory-mapped read-only.  Every indexed tensor must be
 * present in its shard with a data range inside the file; shard names must be
 * plain relative paths; headers are at most 128 MiB.  Replaces
 * open_mlx_safetensors_dir / read_safetensors_header / validate_tensor_range /
 * resolve_shard (model.rs:136-197, 312-431).  Host only. */
typedef struct qm_weight_store qm_weight_store;
qm_status qm_store_open(const char* dir, qm_weight_store** out);
void qm_store_close(qm_weight_store* store);
uint32_t qm_store_tensor_count(const qm_weight_store* store);

/* dtype as in the header ("U32", "BF16", ...), up to shape_cap dims. */
qm_status qm_store_tensor_info(const qm_weight_store* store, const char* name, char* dtype,
                               size_t dtype_cap, uint32_t* ndim, uint64_t* shape,
                               uint32_t shape_cap, uint64_t* bytes);

/* Copies one tensor's bytes into a new device allocation (free with
 * qm_device_free); synchronous. */
qm_status qm_store_upload(qm_runtime* rt, const qm_weight_store* store, const char* name,
                          void** device_out, uint64_t* bytes);

/* A Q4 matrix in HBM: weights u32 [out_rows][in_elems/8], scales and biases
 * bf16 [out_rows][in_elems/64]; each pointer is a separate allocation (free
 * with qm_device_free).  Use as a qm_q4_job's weights/scales/biases. */
typedef struct qm_q4_matrix {
  uint32_t* weights;
  uint16_t* scales;
  uint16_t* biases;
  uint32_t out_rows;
  uint32_t in_elems;
} qm_q4_matrix;

/* Validates `<base>.weight` (U32 [rows][K/8], K a non-zero multiple of 64)
 * with `<base>.scales` / `<base>.biases` (BF16 [rows][K/64], exact byte
 * lengths) and uploads the three tensors.  Replaces Q4AffineMatrix::
 * from_store / from_tensors / validate_affine_tensor (native.rs:5384-5516)
 * and the weight mapping of map_weight_store (metal_runtime.rs:955-984). */
qm_status qm_store_upload_q4(qm_runtime* rt, const qm_weight_store* store,
                             const char* weight_name, qm_q4_matrix* out);

/* ------------------------------------------------------------------ */
/* Residual stream and per-token decode graph                          */
/* ------------------------------------------------------------------ */

/* hidden fp32 [M][n] += delta (bf16 [M][n], skipped when NULL), then
 * out = bf16((hidden * rsqrt(mean(hidden^2) + epsilon)) * weights) per row
 * (weights fp32 [n], used as given).  Replaces qwen38_add_in_place /
 * _add_rows followed by qwen38_rms_norm / _rms_norm_rows (qwen38.metal:
 * 4250-4333; encoders metal_runtime.rs encode_add_in_place / encode_rms_norm).
 * Device pointers; asynchronous. */
qm_status qm_residual_rmsnorm(qm_runtime* rt, float* hidden, const uint16_t* delta,
                              const float* weights, uint32_t M, uint32_t n, float epsilon,
                              uint16_t* out);
/* hidden fp32 [count] += delta bf16 [count] (qwen38_add_in_place). */
qm_status qm_residual_add(qm_runtime* rt, float* hidden, const uint16_t* delta, size_t count);

/* A Gated DeltaNet decoder layer (MetalDecodeLinearLayer,
 * metal_runtime.rs:304-318; encoder encode_decode_linear_layer, :3301-3521):
 *   x = rmsnorm(hidden) * input_norm;  qkv, z, b, a = Q4(x)
 *   d = deltanet_step(qkv, z, b, a);   hidden += Q4_out(d)
 *   x = rmsnorm(hidden) * post_attention_norm
 *   hidden += down(silu(gate(x)) * up(x))
 * Jobs take K = hidden for qkv/z/b/a/gate/up, value_heads*value_head_dim for
 * out_proj and gate.out_rows for down. */
typedef struct qm_decode_linear_layer {
  const float* input_norm;           /* fp32 [hidden] */
  const float* post_attention_norm;  /* fp32 [hidden] */
  qm_q4_job qkv, z, b, a, out_proj;
  const qm_dn_weights* dn_weights;
  qm_dn_state* dn_state;
  qm_q4_job gate, up, down;
} qm_decode_linear_layer;

/* A full-attention decoder layer (MetalDecodeFullLayer, :385-399; encoder
 * encode_decode_full_layer, :1567-2020): q_proj gives [H][2 head_dim]
 * (query | gate per head), then qm_attn_prepare, qm_attn_decode on `kv`
 * (appends this token), o_proj, and the MLP as above. */
typedef struct qm_decode_full_layer {
  const float* input_norm;
  const float* post_attention_norm;
  qm_q4_job q_proj, k_proj, v_proj, o_proj;
  const float* q_norm;  /* fp32 [head_dim] */
  const float* k_norm;  /* fp32 [head_dim] */
  uint32_t num_heads;
  qm_rope_config rope;  /* rope.head_dim must equal kv's head_dim */
  qm_kv* kv;
  qm_q4_job gate, up, down;
} qm_decode_full_layer;

/* One layer: exactly one of linear / full is non-NULL (MetalDecodeLayer). */
typedef struct qm_decode_layer {
  const qm_decode_linear_layer* linear;
  const qm_decode_full_layer* full;
} qm_decode_layer;

/* Activation state of single-token decode (MetalDecodeState,
 * metal_runtime.rs:246-268): the fp32 residual row `hidden` [hidden_elems]
 * (device memory owned by the state) and grow-only intermediate buffers. */
typedef struct qm_decode_state qm_decode_state;
qm_status qm_decode_state_create(qm_runtime* rt, uint32_t hidden_elems, qm_decode_state** out);
void qm_decode_state_destroy(qm_decode_state* st);
float* qm_decode_state_hidden(qm_decode_state* st);

/* Runs one token through `layers` in order, updating hidden in place
 * (decode_layers, metal_runtime.rs:2022-2084).  position: the three M-RoPE
 * axes of this token (all equal for text).  Asynchronous. */
qm_status qm_decode_layers(qm_runtime* rt, qm_decode_state* st, const qm_decode_layer* layers,
                           uint32_t n_layers, const uint32_t position[3], float epsilon);

/* The same token as HIP graphs: every launch between two attention calls is
 * captured once (two variants, for the parity of the DeltaNet history
 * buffers); a run sets the position, then replays the segments with each
 * layer's qm_attn_decode launched between them (its grid depends on the cache
 * length).  Results equal qm_decode_layers bit for bit.  The graph holds the
 * layer descriptors' pointers: a run fails with QM_ERR_GRAPH_STALE when a
 * DeltaNet state's buffers or history parity, or the decode state's buffers,
 * changed since capture (qm_dn_snapshot_restore of a one-row set exchanges
 * buffers; an eager qm_dn_step in between flips the parity only, which the
 * second variant covers).  Creation captures only; it runs nothing. */
typedef struct qm_decode_graph qm_decode_graph;
qm_status qm_decode_graph_create(qm_runtime* rt, qm_decode_state* st, const qm_decode_layer* layers,
                                 uint32_t n_layers, float epsilon, qm_decode_graph** out);
qm_status qm_decode_graph_run(qm_decode_graph* g, const uint32_t position[3]);
void qm_decode_graph_destroy(qm_decode_graph* g);

#ifdef __cplusplus
}
#endif
#endif /* QM38_H */
