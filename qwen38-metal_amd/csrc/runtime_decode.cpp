// C-ABI of the residual stream and the per-token decode graph (see
// include/qm38.h): decode_layers / encode_decode_linear_layer /
// encode_decode_full_layer (/root/reference/src/metal_runtime.rs:2022-2084,
// 3301-3521, 1567-2020) composed from this library's entry points.
//
// Activations between the kernels are bf16 where a Q4 projection reads them
// and fp32 where the DeltaNet step or attention does; the residual row stays
// fp32.  Conversions and residual adds are folded into the producing
// kernels' epilogues (see encode_pre), so a DeltaNet layer is seven launches
// and a full-attention layer seven plus its attention.
//
// Graph mode captures every launch between two attention calls into one HIP
// graph segment.  The attention decode is launched eagerly between segments:
// its grid and split plan follow the cache length, which changes every token.
// The token's M-RoPE position is written by a one-thread kernel into a device
// word that the captured q/k preparation reads.  The DeltaNet conv history is
// double-buffered (the step reads one buffer and writes the other), so the
// token is captured twice, once per parity.
#include <stdint.h>
#include <string.h>

#include <algorithm>
#include <vector>

#include "runtime_internal.h"

using namespace qm;

struct qm_decode_state {
  qm_runtime* rt = nullptr;
  uint32_t hidden = 0;
  float* hid = nullptr;      // fp32 [hidden]
  uint32_t* pos = nullptr;   // uint32 [3] (axis-major, one row)
  // Grow-only arena of the intermediates; `generation` changes whenever it is
  // reallocated (a captured graph holds its addresses).
  void* arena = nullptr;
  size_t arena_bytes = 0;
  uint64_t generation = 0;
  struct Sizes {
    uint32_t p[4] = {0, 0, 0, 0};  // projection outputs (elements)
    uint32_t value = 0;            // DeltaNet value elements
    uint32_t qh = 0;               // num_heads * head_dim
    uint32_t kh = 0;               // kv_heads * head_dim
    uint32_t inter = 0;            // MLP intermediate rows
  } cap;
  // Views into the arena.
  uint16_t* x = nullptr;       // bf16 [hidden] normalised row
  uint16_t* p[2] = {};         // bf16 projection outputs (query | gate, key)
  float* f[4] = {};            // fp32 projection outputs (DeltaNet qkv, z, b, a; value)
  float* dn_out = nullptr;     // fp32 [value]
  uint16_t* dn_out_bf = nullptr;
  uint16_t* q = nullptr;       // bf16 [qh]
  uint16_t* gate = nullptr;    // bf16 [qh]
  float* k = nullptr;          // fp32 [kh]
  uint16_t* attn = nullptr;    // bf16 [qh]
  uint16_t* h = nullptr;       // bf16 [inter]
};

namespace {

bool job_ok(const qm_q4_job& j) { return j.weights && j.scales && j.biases && j.out_rows > 0; }

// A layer's job: pointers set, the expected height (rows = 0: any), and its
// tensors inside their allocations for input width in_elems.
qm_status check_job(const qm_runtime* rt, const qm_q4_job& j, uint32_t rows, uint32_t in_elems, const char* what) {
  if (!job_ok(j)) return fail(QM_ERR_NULL_POINTER, "%s: job pointers must be set and out_rows > 0", what);
  if (rows && j.out_rows != rows)
    return fail(QM_ERR_WRONG_LENGTH, "%s has %u output rows, expected %u", what, j.out_rows, rows);
  return q4_job_ranges(rt, j, in_elems, what);
}

// Validates the layers (validate_decode_q4_job and the shape checks of the
// reference's encoders) and accumulates the intermediate sizes they need.
qm_status check_layers(const qm_runtime* rt, uint32_t hidden, const qm_decode_layer* layers, uint32_t n,
                       qm_decode_state::Sizes* need) {
  if (!layers) return fail(QM_ERR_NULL_POINTER, "layers is NULL");
  if (n == 0) return fail(QM_ERR_EMPTY_DIMENSION, "no layers");
  qm_decode_state::Sizes s;
  for (uint32_t i = 0; i < n; ++i) {
    const qm_decode_layer& L = layers[i];
    if (!!L.linear == !!L.full) return fail(QM_ERR_INVALID_ARGUMENT, "layer %u: set exactly one of linear/full", i);
    qm_status st = QM_OK;
    const qm_q4_job *gate, *up, *down;
    const float *in_norm, *post_norm;
    if (L.linear) {
      const qm_decode_linear_layer& l = *L.linear;
      if (!l.dn_weights || !l.dn_state) return fail(QM_ERR_NULL_POINTER, "layer %u: DeltaNet weights/state", i);
      if (dn_weights_runtime(l.dn_weights) != rt || dn_state_view(l.dn_state).rt != rt)
        return fail(QM_ERR_INVALID_ARGUMENT, "layer %u: DeltaNet objects belong to another runtime", i);
      const qm_dn_config& c = dn_weights_config(l.dn_weights);
      const DnStateView sv = dn_state_view(l.dn_state);
      if (memcmp(&c, &sv.cfg, sizeof(c)) != 0)
        return fail(QM_ERR_WRONG_LENGTH, "layer %u: DeltaNet state was created for another configuration", i);
      const uint32_t channels = 2 * c.key_heads * c.key_head_dim + c.value_heads * c.value_head_dim;
      const uint32_t value = c.value_heads * c.value_head_dim;
      if ((st = check_job(rt, l.qkv, channels, hidden, "DeltaNet qkv")) != QM_OK) return st;
      if ((st = check_job(rt, l.z, value, hidden, "DeltaNet z")) != QM_OK) return st;
      if ((st = check_job(rt, l.b, c.value_heads, hidden, "DeltaNet b")) != QM_OK) return st;
      if ((st = check_job(rt, l.a, c.value_heads, hidden, "DeltaNet a")) != QM_OK) return st;
      if ((st = check_job(rt, l.out_proj, hidden, value, "DeltaNet out projection")) != QM_OK) return st;
      if (value % 64 != 0) return fail(QM_ERR_INPUT_NOT_GROUPED, "layer %u: DeltaNet value elements %u", i, value);
      s.p[0] = std::max(s.p[0], channels);
      s.p[1] = std::max(s.p[1], value);
      s.p[2] = std::max(s.p[2], c.value_heads);
      s.p[3] = std::max(s.p[3], c.value_heads);
      s.value = std::max(s.value, value);
      gate = &l.gate, up = &l.up, down = &l.down;
      in_norm = l.input_norm, post_norm = l.post_attention_norm;
    } else {
      const qm_decode_full_layer& l = *L.full;
      if (!l.kv || !l.q_norm || !l.k_norm) return fail(QM_ERR_NULL_POINTER, "layer %u: kv / q_norm / k_norm", i);
      if (kv_runtime_of(l.kv) != rt) return fail(QM_ERR_INVALID_ARGUMENT, "layer %u: KV cache of another runtime", i);
      const uint32_t KVH = kv_heads_of(l.kv), D = kv_head_dim_of(l.kv), H = l.num_heads;
      if (l.rope.head_dim != D || H == 0 || H % KVH != 0)
        return fail(QM_ERR_INVALID_ATTENTION_SHAPE, "layer %u: heads %u / kv heads %u / head_dim %u vs cache %u", i,
                    H, KVH, l.rope.head_dim, D);
      if ((st = check_job(rt, l.q_proj, 2 * H * D, hidden, "query projection")) != QM_OK) return st;
      if ((st = check_job(rt, l.k_proj, KVH * D, hidden, "key projection")) != QM_OK) return st;
      if ((st = check_job(rt, l.v_proj, KVH * D, hidden, "value projection")) != QM_OK) return st;
      if ((st = check_job(rt, l.o_proj, hidden, H * D, "output projection")) != QM_OK) return st;
      if ((H * D) % 64 != 0) return fail(QM_ERR_INPUT_NOT_GROUPED, "layer %u: query elements %u", i, H * D);
      s.p[0] = std::max(s.p[0], 2 * H * D);
      s.p[1] = std::max(s.p[1], KVH * D);
      s.p[2] = std::max(s.p[2], KVH * D);
      s.qh = std::max(s.qh, H * D);
      s.kh = std::max(s.kh, KVH * D);
      gate = &l.gate, up = &l.up, down = &l.down;
      in_norm = l.input_norm, post_norm = l.post_attention_norm;
    }
    if (!in_norm || !post_norm) return fail(QM_ERR_NULL_POINTER, "layer %u: norm weights", i);
    if ((st = check_job(rt, *gate, 0, hidden, "MLP gate")) != QM_OK) return st;
    if ((st = check_job(rt, *up, gate->out_rows, hidden, "MLP up")) != QM_OK) return st;
    if ((st = check_job(rt, *down, hidden, gate->out_rows, "MLP down")) != QM_OK) return st;
    if (gate->out_rows % 64 != 0)
      return fail(QM_ERR_INPUT_NOT_GROUPED, "layer %u: MLP intermediate %u", i, gate->out_rows);
    s.inter = std::max(s.inter, gate->out_rows);
  }
  *need = s;
  return QM_OK;
}

size_t align256(size_t b) { return (b + 255) & ~size_t(255); }

// Lays the intermediates out in the arena (or only measures when base is NULL).
size_t layout(qm_decode_state* st, const qm_decode_state::Sizes& s, uint8_t* base) {
  size_t off = 0;
  auto take = [&](size_t bytes) {
    void* p = base ? base + off : nullptr;
    off += align256(std::max<size_t>(bytes, 4));
    return p;
  };
  const size_t H = st->hidden;
  void* x = take(H * 2);
  void* p[2];
  void* f[4];
  for (int i = 0; i < 2; ++i) p[i] = take((size_t)s.p[i] * 2);
  for (int i = 0; i < 4; ++i) f[i] = take((size_t)s.p[i] * 4);
  void* dn = take((size_t)s.value * 4);
  void* dnb = take((size_t)s.value * 2);
  void* q = take((size_t)s.qh * 2);
  void* g = take((size_t)s.qh * 2);
  void* k = take((size_t)s.kh * 4);
  void* at = take((size_t)s.qh * 2);
  void* h = take((size_t)s.inter * 2);
  if (base) {
    st->x = (uint16_t*)x;
    for (int i = 0; i < 2; ++i) st->p[i] = (uint16_t*)p[i];
    for (int i = 0; i < 4; ++i) st->f[i] = (float*)f[i];
    st->dn_out = (float*)dn;
    st->dn_out_bf = (uint16_t*)dnb;
    st->q = (uint16_t*)q;
    st->gate = (uint16_t*)g;
    st->k = (float*)k;
    st->attn = (uint16_t*)at;
    st->h = (uint16_t*)h;
  }
  return off;
}

qm_status ensure_arena(qm_decode_state* st, const qm_decode_state::Sizes& need) {
  qm_decode_state::Sizes s = st->cap;
  bool grow = false;
  for (int i = 0; i < 4; ++i)
    if (need.p[i] > s.p[i]) s.p[i] = need.p[i], grow = true;
  if (need.value > s.value) s.value = need.value, grow = true;
  if (need.qh > s.qh) s.qh = need.qh, grow = true;
  if (need.kh > s.kh) s.kh = need.kh, grow = true;
  if (need.inter > s.inter) s.inter = need.inter, grow = true;
  if (!grow && st->arena) return QM_OK;
  const size_t bytes = layout(st, s, nullptr);
  DeviceGuard g(st->rt->device);
  if (!g.ok()) return no_device();
  if (st->arena) {
    hipError_t e = hipStreamSynchronize(st->rt->stream);
    if (e != hipSuccess) return hip_check(e, "decode state resize sync");
    (void)hipFree(st->arena);
    st->arena = nullptr;
  }
  hipError_t e = hipMalloc(&st->arena, bytes);
  if (e != hipSuccess) return hip_check(e, "decode state hipMalloc");
  st->arena_bytes = bytes;
  st->cap = s;
  layout(st, s, (uint8_t*)st->arena);
  st->generation += 1;
  return QM_OK;
}

// The launches of one layer before its attention call (all of a DeltaNet
// layer's mixer) and after it.  `rt` carries the stream and the workspace of
// the captured or eager launches.  Projections that feed fp32 consumers
// write fp32 copies of their bf16-rounded outputs, and the mixer and MLP
// outputs are added into the fp32 residual row by the projections' own
// epilogues (hidden += bf16(y), the reference's add_in_place after a bf16
// projection), so no conversion or add launches remain.
qm_status encode_pre(qm_runtime* rt, qm_decode_state* st, const qm_decode_layer& L, float eps) {
  const uint32_t H = st->hidden;
  const float* in_norm = L.linear ? L.linear->input_norm : L.full->input_norm;
  qm_status s = qm_residual_rmsnorm(rt, st->hid, nullptr, in_norm, 1, H, eps, st->x);
  if (s != QM_OK) return s;
  if (L.linear) {
    const qm_decode_linear_layer& l = *L.linear;
    const qm_dn_config& c = dn_weights_config(l.dn_weights);
    const uint32_t value = c.value_heads * c.value_head_dim;
    const qm_q4_job jobs[4] = {l.qkv, l.z, l.b, l.a};
    void* const outs[4] = {st->f[0], st->f[1], st->f[2], st->f[3]};
    const uint32_t modes[4] = {kQ4OutF32, kQ4OutF32, kQ4OutF32, kQ4OutF32};
    if ((s = q4_project_modes(rt, jobs, outs, modes, 4, st->x, H, 1)) != QM_OK) return s;
    if ((s = dn_step_bf16(rt, l.dn_weights, l.dn_state, st->f[0], st->f[1], st->f[2], st->f[3], eps, st->dn_out,
                          st->dn_out_bf)) != QM_OK)
      return s;
    void* const o[1] = {st->hid};
    const uint32_t add[1] = {kQ4OutAddF32};
    return q4_project_modes(rt, &l.out_proj, o, add, 1, st->dn_out_bf, value, 1);
  }
  const qm_decode_full_layer& l = *L.full;
  const uint32_t KVH = kv_heads_of(l.kv);
  const qm_q4_job jobs[3] = {l.q_proj, l.k_proj, l.v_proj};
  void* const outs[3] = {st->p[0], st->p[1], st->f[2]};
  const uint32_t modes[3] = {kQ4OutBf16, kQ4OutBf16, kQ4OutF32};
  if ((s = q4_project_modes(rt, jobs, outs, modes, 3, st->x, H, 1)) != QM_OK) return s;
  return qm_attn_prepare(rt, &l.rope, 1, l.num_heads, KVH, st->p[0], st->p[1], l.q_norm, l.k_norm, eps, st->pos, 0,
                         st->q, st->gate, st->k);
}

// Grows every full-attention layer's cache for this token and sizes the
// attention workspace; fails before anything is launched.
qm_status prepare_attention(qm_runtime* rt, const qm_decode_layer* layers, uint32_t n_layers) {
  for (uint32_t i = 0; i < n_layers; ++i)
    if (layers[i].full) {
      qm_kv* kv = layers[i].full->kv;
      qm_status s = attn_decode_prepare(rt, &kv, 1, layers[i].full->num_heads);
      if (s != QM_OK) return s;
    }
  return QM_OK;
}

qm_status encode_attention(qm_runtime* rt, qm_decode_state* st, const qm_decode_full_layer& l) {
  qm_kv* kv = l.kv;
  return qm_attn_decode(rt, &kv, 1, st->q, st->gate, st->k, st->f[2], l.num_heads, st->attn);
}

qm_status encode_post(qm_runtime* rt, qm_decode_state* st, const qm_decode_layer& L, float eps) {
  const uint32_t H = st->hidden;
  qm_status s;
  void* const o[1] = {st->hid};
  const uint32_t add[1] = {kQ4OutAddF32};
  if (L.full) {
    const uint32_t qh = L.full->num_heads * L.full->rope.head_dim;
    if ((s = q4_project_modes(rt, &L.full->o_proj, o, add, 1, st->attn, qh, 1)) != QM_OK) return s;
  }
  const float* post_norm = L.linear ? L.linear->post_attention_norm : L.full->post_attention_norm;
  const qm_q4_job& gate = L.linear ? L.linear->gate : L.full->gate;
  const qm_q4_job& up = L.linear ? L.linear->up : L.full->up;
  const qm_q4_job& down = L.linear ? L.linear->down : L.full->down;
  if ((s = qm_residual_rmsnorm(rt, st->hid, nullptr, post_norm, 1, H, eps, st->x)) != QM_OK) return s;
  if ((s = qm_q4_swiglu(rt, &gate, &up, st->x, H, 1, st->h)) != QM_OK) return s;
  return q4_project_modes(rt, &down, o, add, 1, st->h, gate.out_rows, 1);
}

}  // namespace

struct qm_decode_graph {
  qm_runtime* rt = nullptr;     // the caller's runtime (stream, eager attention)
  qm_runtime cap{};             // captured launches: private workspace
  hipStream_t cap_stream = nullptr;
  qm_decode_state* st = nullptr;
  uint64_t st_generation = 0;
  std::vector<qm_decode_layer> layers;
  std::vector<qm_decode_linear_layer> lin;
  std::vector<qm_decode_full_layer> full;
  struct DnRecord {
    qm_dn_state* s;
    DnStateView before;
    int cur_after;
  };
  struct Variant {
    std::vector<hipGraphExec_t> segs;  // segs.size() == attention calls + 1
    std::vector<DnRecord> dn;
  };
  Variant var[2];
  int n_var = 0;
  std::vector<uint32_t> attn_layers;  // layer index of each attention call
};

namespace {

void destroy_variant(qm_decode_graph::Variant& v) {
  for (hipGraphExec_t e : v.segs)
    if (e) (void)hipGraphExecDestroy(e);
  v.segs.clear();
}

qm_status end_segment(qm_decode_graph* g, qm_decode_graph::Variant& v) {
  hipGraph_t graph = nullptr;
  hipError_t e = hipStreamEndCapture(g->cap_stream, &graph);
  if (e != hipSuccess) return hip_check(e, "decode graph end capture");
  hipGraphExec_t exec = nullptr;
  e = hipGraphInstantiate(&exec, graph, nullptr, nullptr, 0);
  (void)hipGraphDestroy(graph);
  if (e != hipSuccess) return hip_check(e, "decode graph instantiate");
  v.segs.push_back(exec);
  return QM_OK;
}

// Captures one token (the DeltaNet states' parity at entry selects which
// history buffers the captured steps read and write).
qm_status capture_variant(qm_decode_graph* g, float eps, qm_decode_graph::Variant& v) {
  for (const qm_decode_layer& L : g->layers)
    if (L.linear) v.dn.push_back({L.linear->dn_state, dn_state_view(L.linear->dn_state), 0});
  hipError_t e = hipStreamBeginCapture(g->cap_stream, hipStreamCaptureModeThreadLocal);
  if (e != hipSuccess) return hip_check(e, "decode graph begin capture");
  qm_status s = QM_OK;
  for (size_t i = 0; i < g->layers.size() && s == QM_OK; ++i) {
    const qm_decode_layer& L = g->layers[i];
    s = encode_pre(&g->cap, g->st, L, eps);
    if (s != QM_OK) break;
    if (L.full) {
      if ((s = end_segment(g, v)) != QM_OK) return s;
      e = hipStreamBeginCapture(g->cap_stream, hipStreamCaptureModeThreadLocal);
      if (e != hipSuccess) return hip_check(e, "decode graph begin capture");
    }
    s = encode_post(&g->cap, g->st, L, eps);
  }
  if (s != QM_OK) {
    hipGraph_t graph = nullptr;
    (void)hipStreamEndCapture(g->cap_stream, &graph);
    if (graph) (void)hipGraphDestroy(graph);
    return s;
  }
  if ((s = end_segment(g, v)) != QM_OK) return s;
  for (auto& r : v.dn) r.cur_after = dn_state_view(r.s).cur;
  return QM_OK;
}

}  // namespace

extern "C" {

qm_status qm_residual_rmsnorm(qm_runtime* rt, float* hidden, const uint16_t* delta, const float* weights,
                              uint32_t M, uint32_t n, float epsilon, uint16_t* out) {
  if (!rt || !hidden || !weights || !out) return fail(QM_ERR_NULL_POINTER, "NULL argument");
  if (M == 0 || n == 0) return fail(QM_ERR_EMPTY_DIMENSION, "RMSNorm of an empty row");
  if (!(epsilon >= 0.0f)) return fail(QM_ERR_INVALID_ARGUMENT, "epsilon must be >= 0");
  DeviceGuard g(rt->device);
  if (!g.ok()) return no_device();
  return hip_check(launch_residual_rmsnorm(hidden, delta, weights, out, M, n, epsilon, rt->stream),
                   "RMSNorm launch");
}

qm_status qm_residual_add(qm_runtime* rt, float* hidden, const uint16_t* delta, size_t count) {
  if (!rt || !hidden || !delta) return fail(QM_ERR_NULL_POINTER, "NULL argument");
  DeviceGuard g(rt->device);
  if (!g.ok()) return no_device();
  return hip_check(launch_residual_add(hidden, delta, count, rt->stream), "residual add launch");
}

qm_status qm_decode_state_create(qm_runtime* rt, uint32_t hidden_elems, qm_decode_state** out) {
  if (!rt || !out) return fail(QM_ERR_NULL_POINTER, "NULL argument");
  *out = nullptr;
  if (hidden_elems == 0) return fail(QM_ERR_EMPTY_DIMENSION, "hidden size 0");
  if (hidden_elems % 64 != 0) return fail(QM_ERR_INPUT_NOT_GROUPED, "hidden size %u is not a multiple of 64", hidden_elems);
  qm_decode_state* st = new qm_decode_state();
  st->rt = rt;
  st->hidden = hidden_elems;
  DeviceGuard g(rt->device);
  if (!g.ok()) {
    delete st;
    return no_device();
  }
  hipError_t e = hipMalloc(&st->hid, (size_t)hidden_elems * 4);
  if (e == hipSuccess) e = hipMalloc(&st->pos, 256);
  if (e == hipSuccess) e = hipMemsetAsync(st->hid, 0, (size_t)hidden_elems * 4, rt->stream);
  if (e == hipSuccess) e = hipStreamSynchronize(rt->stream);
  if (e != hipSuccess) {
    (void)hipFree(st->hid);
    (void)hipFree(st->pos);
    delete st;
    return hip_check(e, "decode state allocation");
  }
  *out = st;
  return QM_OK;
}

void qm_decode_state_destroy(qm_decode_state* st) {
  if (!st) return;
  DeviceGuard g(st->rt->device);
  (void)hipStreamSynchronize(st->rt->stream);
  (void)hipFree(st->hid);
  (void)hipFree(st->pos);
  if (st->arena) (void)hipFree(st->arena);
  delete st;
}

float* qm_decode_state_hidden(qm_decode_state* st) { return st ? st->hid : nullptr; }

qm_status qm_decode_layers(qm_runtime* rt, qm_decode_state* st, const qm_decode_layer* layers, uint32_t n_layers,
                           const uint32_t position[3], float epsilon) {
  if (!rt || !st || !position) return fail(QM_ERR_NULL_POINTER, "NULL argument");
  if (st->rt != rt) return fail(QM_ERR_INVALID_ARGUMENT, "decode state belongs to another runtime");
  qm_decode_state::Sizes need;
  qm_status s = check_layers(rt, st->hidden, layers, n_layers, &need);
  if (s != QM_OK) return s;
  if ((s = ensure_arena(st, need)) != QM_OK) return s;
  DeviceGuard g(rt->device);
  if (!g.ok()) return no_device();
  // Everything the attention calls could fail on is settled before the first
  // launch, so a failed token leaves hidden, the DeltaNet states and the
  // caches as they were (decode_layers encodes the whole token before it
  // commits, metal_runtime.rs:2022-2084).
  if ((s = prepare_attention(rt, layers, n_layers)) != QM_OK) return s;
  if ((s = hip_check(launch_set_u32x3(st->pos, position[0], position[1], position[2], rt->stream),
                     "position launch")) != QM_OK)
    return s;
  for (uint32_t i = 0; i < n_layers; ++i) {
    const qm_decode_layer& L = layers[i];
    if ((s = encode_pre(rt, st, L, epsilon)) != QM_OK) return s;
    if (L.full && (s = encode_attention(rt, st, *L.full)) != QM_OK) return s;
    if ((s = encode_post(rt, st, L, epsilon)) != QM_OK) return s;
  }
  return QM_OK;
}

qm_status qm_decode_graph_create(qm_runtime* rt, qm_decode_state* st, const qm_decode_layer* layers,
                                 uint32_t n_layers, float epsilon, qm_decode_graph** out) {
  if (!rt || !st || !out) return fail(QM_ERR_NULL_POINTER, "NULL argument");
  *out = nullptr;
  if (st->rt != rt) return fail(QM_ERR_INVALID_ARGUMENT, "decode state belongs to another runtime");
  qm_decode_state::Sizes need;
  qm_status s = check_layers(rt, st->hidden, layers, n_layers, &need);
  if (s != QM_OK) return s;
  if ((s = ensure_arena(st, need)) != QM_OK) return s;
  qm_decode_graph* g = new qm_decode_graph();
  g->rt = rt;
  g->st = st;
  g->st_generation = st->generation;
  g->cap.device = rt->device;
  g->cap.cu_count = rt->cu_count;
  g->cap.tune = rt->tune;
  // Copy the descriptors (the graph keeps using them for the eager calls).
  g->lin.reserve(n_layers);
  g->full.reserve(n_layers);
  for (uint32_t i = 0; i < n_layers; ++i) {
    qm_decode_layer L{};
    if (layers[i].linear) {
      g->lin.push_back(*layers[i].linear);
      L.linear = &g->lin.back();
    } else {
      g->full.push_back(*layers[i].full);
      L.full = &g->full.back();
      g->attn_layers.push_back(i);
    }
    g->layers.push_back(L);
  }
  DeviceGuard dg(rt->device);
  if (!dg.ok()) {
    delete g;
    return no_device();
  }
  hipError_t e = hipStreamCreate(&g->cap_stream);
  if (e != hipSuccess) {
    delete g;
    return hip_check(e, "decode graph stream");
  }
  g->cap.stream = g->cap_stream;
  // Size the captured calls' workspace beforehand (no allocation may happen
  // while capturing): the DeltaNet step's conv buffer, output exchange and
  // arrival counters are its only ones.
  size_t step_bytes = 4;
  uint32_t step_ctrs = 1;
  for (const qm_decode_layer& L : g->layers)
    if (L.linear) {
      const qm_dn_config& c = dn_weights_config(L.linear->dn_weights);
      step_bytes = std::max(step_bytes, dn_step_scratch_bytes(c));
      step_ctrs = std::max(step_ctrs, c.value_heads);
    }
  s = ensure_scratch(&g->cap, step_bytes);
  if (s == QM_OK) s = ensure_counters(&g->cap, step_ctrs);
  // ... and the single-row projections' split-K partials.
  for (const qm_decode_layer& L : g->layers) {
    if (s != QM_OK) break;
    const uint32_t H = st->hidden;
    const qm_q4_job& gate = L.linear ? L.linear->gate : L.full->gate;
    const qm_q4_job& down = L.linear ? L.linear->down : L.full->down;
    s = q4_reserve_workspace(&g->cap, &down, 1, gate.out_rows);
    if (s == QM_OK && L.linear) {
      const qm_dn_config& c = dn_weights_config(L.linear->dn_weights);
      const qm_q4_job set[4] = {L.linear->qkv, L.linear->z, L.linear->b, L.linear->a};
      s = q4_reserve_workspace(&g->cap, set, 4, H);
      if (s == QM_OK) s = q4_reserve_workspace(&g->cap, &L.linear->out_proj, 1, c.value_heads * c.value_head_dim);
    } else if (s == QM_OK) {
      const qm_q4_job set[3] = {L.full->q_proj, L.full->k_proj, L.full->v_proj};
      s = q4_reserve_workspace(&g->cap, set, 3, H);
      if (s == QM_OK)
        s = q4_reserve_workspace(&g->cap, &L.full->o_proj, 1, L.full->num_heads * L.full->rope.head_dim);
    }
  }
  // Two variants, one per history parity; capturing flips the states'
  // parity exactly as running would, so the second capture starts from the
  // first one's end and ends where the first began.
  bool has_dn = false;
  for (const qm_decode_layer& L : g->layers) has_dn |= L.linear != nullptr;
  g->n_var = has_dn ? 2 : 1;
  for (int v = 0; v < g->n_var && s == QM_OK; ++v) s = capture_variant(g, epsilon, g->var[v]);
  if (s != QM_OK) {
    // Put the parity back to where it was before the failed capture.
    if (!g->var[0].dn.empty())
      for (auto& r : g->var[0].dn) dn_state_set_cur(r.s, r.before.cur);
    qm_decode_graph_destroy(g);
    return s;
  }
  *out = g;
  return QM_OK;
}

qm_status qm_decode_graph_run(qm_decode_graph* g, const uint32_t position[3]) {
  if (!g || !position) return fail(QM_ERR_NULL_POINTER, "NULL argument");
  if (g->st->generation != g->st_generation)
    return fail(QM_ERR_GRAPH_STALE, "the decode state's buffers were reallocated after capture");
  // Pick the variant whose captured parity matches every DeltaNet state now.
  int pick = -1;
  for (int v = 0; v < g->n_var && pick < 0; ++v) {
    bool ok = true;
    for (const auto& r : g->var[v].dn) {
      const DnStateView now = dn_state_view(r.s);
      ok &= now.cur == r.before.cur && now.hist0 == r.before.hist0 && now.hist1 == r.before.hist1 &&
            now.rec == r.before.rec;
    }
    if (ok) pick = v;
  }
  if (pick < 0)
    return fail(QM_ERR_GRAPH_STALE, "a DeltaNet state's buffers or history parity changed after capture");
  qm_decode_graph::Variant& v = g->var[pick];
  qm_runtime* rt = g->rt;
  DeviceGuard dg(rt->device);
  if (!dg.ok()) return no_device();
  qm_status s = prepare_attention(rt, g->layers.data(), (uint32_t)g->layers.size());
  if (s != QM_OK) return s;
  s = hip_check(launch_set_u32x3(g->st->pos, position[0], position[1], position[2], rt->stream),
                          "position launch");
  for (size_t i = 0; i < v.segs.size() && s == QM_OK; ++i) {
    s = hip_check(hipGraphLaunch(v.segs[i], rt->stream), "decode graph launch");
    if (s == QM_OK && i < g->attn_layers.size())
      s = encode_attention(rt, g->st, *g->layers[g->attn_layers[i]].full);
  }
  if (s != QM_OK) return s;
  for (const auto& r : v.dn) dn_state_set_cur(r.s, r.cur_after);
  return QM_OK;
}

void qm_decode_graph_destroy(qm_decode_graph* g) {
  if (!g) return;
  DeviceGuard dg(g->rt->device);
  (void)hipStreamSynchronize(g->rt->stream);
  for (int v = 0; v < 2; ++v) destroy_variant(g->var[v]);
  if (g->cap_stream) {
    (void)hipStreamSynchronize(g->cap_stream);
    release_buffers(&g->cap);
    (void)hipStreamDestroy(g->cap_stream);
  }
  delete g;
}

}  // extern "C"
