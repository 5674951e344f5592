// Private definitions of the C-ABI objects shared by the runtime sources.
#pragma once
#include <hip/hip_runtime.h>

#include <vector>

#include "../../include/qm38.h"
#include "internal.h"

struct qm_runtime {
  int device = 0;
  int cu_count = 256;
  qm::Tuning tune{};  // planner overrides, read once at creation
  hipStream_t stream = nullptr;
  // Grow-only scratch used by calls that need an intermediate buffer (the
  // MLP's h, attention split partials).  Calls on one runtime are serialised
  // on its stream, so one buffer suffices.
  void* scratch = nullptr;
  size_t scratch_bytes = 0;
  // Zero-initialised completion counters for kernels whose last workgroup
  // combines partial results; every such kernel leaves them at zero again.
  unsigned int* counters = nullptr;
  size_t counter_count = 0;
  // Split-K partial results of the kernels that combine them in their last
  // workgroup (no zeroing needed: every slot is written before it is read).
  void* partials = nullptr;
  size_t partial_bytes = 0;
  // fp16 activations of the prefill GEMM (separate from `scratch`, which may
  // hold the MLP's h while h itself is converted).
  void* xh = nullptr;
  size_t xh_bytes = 0;
  // Argmax keys of qm_q4_argmax (one uint64 per row of a 16-row chunk); zero
  // between calls, like the counters.
  unsigned long long* keys = nullptr;
  // Orders this runtime's stream before another runtime's (stream_after).
  hipEvent_t order_event = nullptr;
};

namespace qm {

qm_status fail(qm_status status, const char* fmt, ...);
qm_status hip_check(hipError_t err, const char* what);
// QM_ERR_NO_DEVICE for a call on a runtime created without a device.
qm_status no_device();
qm_status ensure_scratch(qm_runtime* rt, size_t bytes);
qm_status ensure_partials(qm_runtime* rt, size_t bytes);
qm_status ensure_counters(qm_runtime* rt, size_t count);
qm_status ensure_xh(qm_runtime* rt, size_t bytes);
qm_status ensure_keys(qm_runtime* rt);
// Workspace handed to kernels that split work across workgroups.
Workspace workspace(qm_runtime* rt);
// The device-allocation range checks of every Q4 entry point for one job of
// input width in_elems (INVALID_BUFFER_OFFSET / MAPPED_TENSOR_OUT_OF_RANGE);
// nothing is checked on a runtime without a device or a capturing stream.
qm_status q4_job_ranges(const qm_runtime* rt, const qm_q4_job& j, uint32_t in_elems, const char* name);
// Sizes rt's workspace for single-row projections of these jobs (the K-split
// partials of the streaming kernel), so a later call allocates nothing (graph
// capture).
qm_status q4_reserve_workspace(qm_runtime* rt, const qm_q4_job* jobs, int n_jobs, uint32_t in_elems);
// qm_q4_project with a per-job output mode (kQ4Out*; fp32 modes need M <= 16).
qm_status q4_project_modes(qm_runtime* rt, const qm_q4_job* jobs, void* const* outs, const uint32_t* modes,
                           int n_jobs, const uint16_t* x, uint32_t in_elems, uint32_t M);
// qm_dn_step that also writes the output rounded to bf16 into out_bf16.
qm_status dn_step_bf16(qm_runtime* rt, const qm_dn_weights* w, qm_dn_state* st, const float* qkv, const float* z,
                       const float* b, const float* a, float eps, float* out, uint16_t* out_bf16);
// Scratch bytes a single-token qm_dn_step needs (its counters: value_heads).
size_t dn_step_scratch_bytes(const qm_dn_config& c);
// Makes work enqueued from now on `waiter`'s stream wait for the work enqueued
// so far on `signaler`'s stream (an event record + stream wait), so a cache or
// state owned by one runtime can be used from another without racing its
// pending work.  Nothing to do when both use one stream, or while either
// stream is being captured (a capture cannot wait on an outside event).
qm_status stream_after(qm_runtime* waiter, qm_runtime* signaler);
// True while `s` is being captured, and also when the query itself fails (the
// legacy stream while another stream captures); clears that query's error.
bool stream_capturing(hipStream_t s);
// Frees a runtime's grow-only buffers (not the runtime itself).
void release_buffers(qm_runtime* rt);

// Views of the opaque state objects for the decode graph (runtime_decode.cpp).
const qm_dn_config& dn_weights_config(const qm_dn_weights* w);
const qm_runtime* dn_weights_runtime(const qm_dn_weights* w);
struct DnStateView {
  const void* hist0;
  const void* hist1;
  const void* rec;
  int cur;
  const qm_runtime* rt;
  qm_dn_config cfg;
};
DnStateView dn_state_view(const qm_dn_state* s);
void dn_state_set_cur(qm_dn_state* s, int cur);
// Validates a decode step of one more token for these caches, grows their
// capacity and sizes the runtime's attention workspace (may allocate).
qm_status attn_decode_prepare(qm_runtime* rt, qm_kv* const* seqs, uint32_t B, uint32_t H);
uint32_t kv_heads_of(const qm_kv* kv);
uint32_t kv_head_dim_of(const qm_kv* kv);
const qm_runtime* kv_runtime_of(const qm_kv* kv);

// Makes `device` current for its scope.  ok() is false for a runtime
// without a device (QM_DEVICE_NONE), whose calls stop at no_device().
class DeviceGuard {
 public:
  explicit DeviceGuard(int device);
  ~DeviceGuard();
  // The device exists and is current (false for QM_DEVICE_NONE).
  bool ok() const { return ok_; }

 private:
  int prev_ = 0;
  int dev_ = 0;
  bool ok_ = false;
};

}  // namespace qm
