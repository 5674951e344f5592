// Host-side error paths of the qm38 C ABI, run on the CPU under
// AddressSanitizer and UndefinedBehaviorSanitizer (built and run by
// tests/test_host_sanitized.py).
//
// A runtime made with QM_DEVICE_NONE checks every argument exactly as a
// device runtime does and stops with QM_ERR_NO_DEVICE where it would touch
// a device, so each argument error below is the one a GPU caller gets.
// Every qm_status the host can produce without a device is forced once and
// printed as "forced <name>"; the CPU oracle's known answers are checked
// under the same sanitizers.
//
// Codes that need device objects (a cache, a state, a graph, a HIP failure)
// are forced by the GPU tests: INVALID_SEQUENCE_LENGTH and CAPACITY_EXCEEDED
// (test_gpu_attention.py), INVALID_SNAPSHOT / INVALID_SNAPSHOT_ROW
// (test_gpu_deltanet.py), GRAPH_STALE (test_gpu_decode.py), OUT_OF_MEMORY
// and COMMAND_FAILED (test_gpu_errors.py).
#include <math.h>
#include <stdint.h>
#include <stdio.h>
#include <stdlib.h>
#include <string.h>
#include <unistd.h>

#include <set>
#include <string>

#include "qm38.h"

extern "C" {
// CPU oracle (oracle/qm_oracle.cpp)
float qo_bf16_to_f32(uint16_t b);
uint16_t qo_f32_to_bf16(float f);
void qo_q8_quantize(const float* x, uint32_t d, int8_t* q, float* scale);
void qo_attention(const float* q, const float* gate, const int8_t* keys, const float* kscale, const int8_t* values,
                  const float* vscale, uint32_t rows, uint32_t H, uint32_t KVH, uint32_t d, uint32_t start,
                  uint32_t total, float* o, int threads);
}

static std::set<std::string> g_forced;
static int g_failures = 0;

static void expect(qm_status got, qm_status want, const char* what) {
  if (got != want) {
    fprintf(stderr, "FAIL %s: got %s, want %s (%s)\n", what, qm_status_string(got), qm_status_string(want),
            qm_last_error_message());
    ++g_failures;
    return;
  }
  if (g_forced.insert(qm_status_string(want)).second) printf("forced %s\n", qm_status_string(want));
}

// A device-pointer stand-in: never dereferenced by argument checks.
template <typename T>
static T* fake(uintptr_t addr) {
  return reinterpret_cast<T*>(addr);
}

static void runtime_cases(qm_runtime* rt) {
  // Q4 projections.
  qm_q4_job job{fake<const uint32_t>(0x10000), fake<const uint16_t>(0x20000), fake<const uint16_t>(0x30000), 64};
  uint16_t* outs[9] = {};
  for (auto& o : outs) o = fake<uint16_t>(0x40000);
  const uint16_t* x = fake<const uint16_t>(0x50000);
  expect(qm_q4_project(rt, &job, 1, x, 128, 1, outs), QM_ERR_NO_DEVICE, "valid projection, no device");
  expect(qm_q4_project(rt, &job, 1, nullptr, 128, 1, outs), QM_ERR_NULL_POINTER, "NULL activation");
  expect(qm_q4_project(rt, &job, 1, x, 128, 0, outs), QM_ERR_EMPTY_DIMENSION, "zero rows");
  expect(qm_q4_project(rt, &job, 1, x, 100, 1, outs), QM_ERR_INPUT_NOT_GROUPED, "K not a multiple of 64");
  expect(qm_q4_project(rt, &job, 1, fake<const uint16_t>(0x50002), 128, 1, outs), QM_ERR_MISALIGNED,
         "misaligned activation");
  qm_q4_job jobs[9];
  for (auto& j : jobs) j = job;
  expect(qm_q4_project(rt, jobs, 9, x, 128, 1, outs), QM_ERR_INVALID_ARGUMENT, "nine jobs");
  qm_q4_job up = job;
  up.out_rows = 128;
  expect(qm_q4_swiglu(rt, &job, &up, x, 128, 1, outs[0]), QM_ERR_WRONG_LENGTH, "gate/up rows differ");
  qm_q4_job huge = job;
  huge.out_rows = 0xFFFFFFFFu;
  expect(qm_q4_project(rt, &huge, 1, x, 0xFFFFFFC0u, 1, outs), QM_ERR_DIMENSION_OVERFLOW, "weight count overflow");
  expect(qm_q4_project(rt, &job, 1, x, (1u << 24) + 64, 1, outs), QM_ERR_DIMENSION_OVERFLOW, "input too wide");
  expect(qm_q4_project(rt, &job, 1, x, 1u << 24, 1, outs), QM_ERR_NO_DEVICE, "widest input, no device");

  // Mapped jobs (validate_mapped_q4_affine_shape, metal_runtime.rs:8854-8898):
  // K = 128, 64 rows -> 4096 B of weights, 256 B of scales and of biases.
  {
    const qm_buffer wb{fake<const void>(0x100000), 8192}, sb{fake<const void>(0x200000), 512};
    const qm_q4_mapped_job ok{wb, 4096, sb, 256, sb, 0, 64};
    qm_q4_job out{};
    expect(qm_q4_job_from_mapped(&ok, 128, &out), QM_OK, "mapped job in range");
    if (out.weights != fake<const uint32_t>(0x101000) || out.scales != fake<const uint16_t>(0x200100) ||
        out.biases != fake<const uint16_t>(0x200000) || out.out_rows != 64) {
      fprintf(stderr, "FAIL mapped job resolves to the wrong pointers\n");
      ++g_failures;
    }
    qm_q4_mapped_job m = ok;
    m.weight_offset = 8193;
    expect(qm_q4_job_from_mapped(&m, 128, &out), QM_ERR_INVALID_BUFFER_OFFSET, "weight offset past the buffer");
    m = ok;
    m.bias_offset = 513;
    expect(qm_q4_job_from_mapped(&m, 128, &out), QM_ERR_INVALID_BUFFER_OFFSET, "bias offset past the buffer");
    m = ok;
    m.weight_offset = 4104;  // 4088 B left for 4096
    expect(qm_q4_job_from_mapped(&m, 128, &out), QM_ERR_MAPPED_TENSOR_OUT_OF_RANGE, "weights run past the buffer");
    m = ok;
    m.scale_offset = 264;  // 248 B left for 256
    expect(qm_q4_job_from_mapped(&m, 128, &out), QM_ERR_MAPPED_TENSOR_OUT_OF_RANGE, "scales run past the buffer");
    m = ok;
    m.out_rows = 65;
    expect(qm_q4_job_from_mapped(&m, 128, &out), QM_ERR_MAPPED_TENSOR_OUT_OF_RANGE, "one row too many");
    m = ok;
    m.weight_offset = 8192;  // offset == length is allowed, the tensor then does not fit
    expect(qm_q4_job_from_mapped(&m, 128, &out), QM_ERR_MAPPED_TENSOR_OUT_OF_RANGE, "offset at the buffer end");
    expect(qm_q4_job_from_mapped(&ok, 100, &out), QM_ERR_INPUT_NOT_GROUPED, "mapped K not grouped");
    m = ok;
    m.out_rows = 0;
    expect(qm_q4_job_from_mapped(&m, 128, &out), QM_ERR_EMPTY_DIMENSION, "mapped zero rows");
    m = ok;
    m.weight_offset = 4;
    m.weights.length = 8200;
    expect(qm_q4_job_from_mapped(&m, 128, &out), QM_ERR_MISALIGNED, "mapped weights misaligned");
    expect(qm_q4_job_from_mapped(nullptr, 128, &out), QM_ERR_NULL_POINTER, "mapped job NULL");
    uint32_t* ids = fake<uint32_t>(0x60000);
    expect(qm_q4_argmax(rt, &job, x, 128, 3, ids), QM_ERR_NO_DEVICE, "valid argmax, no device");
    expect(qm_q4_argmax(rt, &job, x, 128, 3, nullptr), QM_ERR_NULL_POINTER, "argmax ids NULL");
    expect(qm_q4_argmax(rt, &job, x, 96, 3, ids), QM_ERR_INPUT_NOT_GROUPED, "argmax K not grouped");
  }

  // KV cache and attention.
  qm_kv* kv = nullptr;
  expect(qm_kv_create(rt, 8, 300, 16, 0, &kv), QM_ERR_INVALID_ATTENTION_SHAPE, "head_dim 300");
  expect(qm_kv_create(rt, 0, 128, 16, 0, &kv), QM_ERR_INVALID_ATTENTION_SHAPE, "no KV heads");
  expect(qm_kv_create(rt, 8, 128, 16, 0, &kv), QM_ERR_NO_DEVICE, "KV cache, no device");
  if (kv) ++g_failures;
  qm_rope_config rope{128, 32, 1e7f, 0, 0, 0};
  expect(qm_attn_prepare(rt, &rope, 1, 0x7FFFFFFFu, 8, x, x, fake<const float>(0x60000), fake<const float>(0x60000),
                         1e-6f, nullptr, 0, outs[0], outs[1], fake<float>(0x70000)),
         QM_ERR_DIMENSION_OVERFLOW, "head count overflow");
  rope.rotary_dim = 3;
  expect(qm_attn_prepare(rt, &rope, 1, 64, 8, x, x, fake<const float>(0x60000), fake<const float>(0x60000), 1e-6f,
                         nullptr, 0, outs[0], outs[1], fake<float>(0x70000)),
         QM_ERR_INVALID_ATTENTION_SHAPE, "odd rotary_dim");
  rope.rotary_dim = 32;
  expect(qm_attn_prepare(rt, &rope, 0, 64, 8, x, x, fake<const float>(0x60000), fake<const float>(0x60000), 1e-6f,
                         nullptr, 0, outs[0], outs[1], fake<float>(0x70000)),
         QM_ERR_EMPTY_DIMENSION, "zero rows");

  // Gated DeltaNet.
  qm_dn_config cfg{3, 4, 128, 128, 4};  // 4 value heads over 3 key heads
  float host[64] = {};
  qm_dn_weights* w = nullptr;
  expect(qm_dn_weights_create(rt, &cfg, host, host, host, host, &w), QM_ERR_INVALID_DELTANET_CONFIG,
         "value heads not a multiple of key heads");
  cfg = qm_dn_config{1, 1, 2, 2, 4};
  expect(qm_dn_weights_create(rt, &cfg, host, host, host, host, &w), QM_ERR_NO_DEVICE, "DeltaNet weights, no device");
  if (w) ++g_failures;

  // Residual stream and decode state.
  expect(qm_residual_rmsnorm(rt, fake<float>(0x80000), nullptr, fake<const float>(0x60000), 1, 0, 1e-6f, outs[0]),
         QM_ERR_EMPTY_DIMENSION, "empty row");
  qm_decode_state* ds = nullptr;
  expect(qm_decode_state_create(rt, 100, &ds), QM_ERR_INPUT_NOT_GROUPED, "hidden size 100");
  expect(qm_decode_state_create(rt, 128, &ds), QM_ERR_NO_DEVICE, "decode state, no device");
  if (ds) ++g_failures;
  void* dev = nullptr;
  expect(qm_device_alloc(rt, 0, &dev), QM_ERR_EMPTY_DIMENSION, "zero-byte allocation");
  expect(qm_device_alloc(rt, 256, &dev), QM_ERR_NO_DEVICE, "allocation, no device");
  expect(qm_runtime_set_stream(nullptr, nullptr), QM_ERR_NULL_POINTER, "NULL runtime");
}

static void store_cases() {
  qm_weight_store* store = nullptr;
  expect(qm_store_open("/nonexistent/qm38-model", &store), QM_ERR_MODEL_FORMAT, "missing model directory");
  char dir[] = "/tmp/qm38_store_XXXXXX";
  if (!mkdtemp(dir)) {
    ++g_failures;
    return;
  }
  // One shard holding a U32 weight whose shape is not [rows][K/8] with
  // companions: the index and shard parse, the Q4 view is refused.
  const std::string shard = std::string(dir) + "/model.safetensors";
  const std::string header =
      "{\"w.weight\":{\"dtype\":\"U32\",\"shape\":[2,3],\"data_offsets\":[0,24]}}";
  FILE* f = fopen(shard.c_str(), "wb");
  const uint64_t n = header.size();
  fwrite(&n, 8, 1, f);
  fwrite(header.data(), 1, n, f);
  const uint8_t zeros[24] = {};
  fwrite(zeros, 1, sizeof(zeros), f);
  fclose(f);
  f = fopen((std::string(dir) + "/model.safetensors.index.json").c_str(), "wb");
  fputs("{\"weight_map\":{\"w.weight\":\"model.safetensors\"}}", f);
  fclose(f);
  expect(qm_store_open(dir, &store), QM_OK, "small valid store");
  qm_runtime* rt = nullptr;
  qm_runtime_create(QM_DEVICE_NONE, &rt);
  qm_q4_matrix m{};
  expect(qm_store_upload_q4(rt, store, "w.weight", &m), QM_ERR_INVALID_TENSOR, "Q4 view without companions");
  qm_runtime_destroy(rt);
  qm_store_close(store);
  remove(shard.c_str());
  remove((std::string(dir) + "/model.safetensors.index.json").c_str());
  rmdir(dir);
}

static void oracle_cases() {
  // bf16 round to nearest even (qwen38.metal:18-26), Q8 known answer
  // (metal_runtime.rs:11598-11604), one-token attention = the value row.
  if (qo_f32_to_bf16(1.0f) != 0x3F80 || qo_bf16_to_f32(0x3F80) != 1.0f) ++g_failures;
  const float v[2] = {2.0f, -1.0f};
  int8_t q[2];
  float s = 0.0f;
  qo_q8_quantize(v, 2, q, &s);
  if (q[0] != 127 || q[1] != -64 || s != 2.0f / 127.0f) {
    fprintf(stderr, "FAIL q8 known answer\n");
    ++g_failures;
  }
  const float qv[2] = {1.0f, 0.0f};
  const int8_t keys[2] = {127, 0}, vals[2] = {127, -64};
  const float ks = 1.0f / 127.0f, vs = 2.0f / 127.0f;
  float o[2];
  qo_attention(qv, nullptr, keys, &ks, vals, &vs, 1, 1, 1, 2, 0, 1, o, 1);
  if (fabsf(o[0] - 2.0f) > 1e-6f || fabsf(o[1] + 128.0f / 127.0f) > 1e-6f) {
    fprintf(stderr, "FAIL one-token attention\n");
    ++g_failures;
  }
}

int main() {
  qm_runtime* rt = nullptr;
  expect(qm_runtime_create(0, &rt), QM_ERR_NO_DEVICE, "device 0 on a host without a GPU");
  expect(qm_runtime_create(0, nullptr), QM_ERR_NULL_POINTER, "NULL out");
  expect(qm_runtime_create(QM_DEVICE_NONE, &rt), QM_OK, "runtime without a device");
  runtime_cases(rt);
  qm_runtime_destroy(rt);
  store_cases();
  oracle_cases();
  printf("failures %d\n", g_failures);
  return g_failures ? 1 : 0;
}
