// Temporary: entry points whose kernels are not built yet.
#include "runtime_internal.h"
using namespace qm;
extern "C" {
qm_status qm_kv_create(qm_runtime*, uint32_t, uint32_t, uint32_t, uint32_t, qm_kv**) { return fail(QM_ERR_INVALID_ARGUMENT, "not built"); }
void qm_kv_destroy(qm_kv*) {}
uint32_t qm_kv_length(const qm_kv*) { return 0; }
uint32_t qm_kv_allocated_pages(const qm_kv*) { return 0; }
int64_t qm_kv_page_for_token(const qm_kv*, uint32_t) { return -1; }
qm_status qm_kv_reserve(qm_kv*, uint32_t) { return fail(QM_ERR_INVALID_ARGUMENT, "not built"); }
qm_status qm_kv_truncate(qm_kv*, uint32_t) { return fail(QM_ERR_INVALID_ARGUMENT, "not built"); }
qm_status qm_kv_clone(const qm_kv*, qm_kv**) { return fail(QM_ERR_INVALID_ARGUMENT, "not built"); }
qm_status qm_kv_read(const qm_kv*, int8_t*, int8_t*, float*, float*) { return fail(QM_ERR_INVALID_ARGUMENT, "not built"); }
qm_status qm_attn_decode(qm_runtime*, qm_kv* const*, uint32_t, const uint16_t*, const uint16_t*, const float*, const float*, uint32_t, uint16_t*) { return fail(QM_ERR_INVALID_ARGUMENT, "not built"); }
qm_status qm_attn_prefill(qm_runtime*, qm_kv*, const uint16_t*, const uint16_t*, const float*, const float*, uint32_t, uint32_t, uint16_t*) { return fail(QM_ERR_INVALID_ARGUMENT, "not built"); }
qm_status qm_dn_weights_create(qm_runtime*, const qm_dn_config*, const float*, const float*, const float*, const float*, qm_dn_weights**) { return fail(QM_ERR_INVALID_ARGUMENT, "not built"); }
void qm_dn_weights_destroy(qm_dn_weights*) {}
qm_status qm_dn_state_create(qm_runtime*, const qm_dn_weights*, qm_dn_state**) { return fail(QM_ERR_INVALID_ARGUMENT, "not built"); }
void qm_dn_state_destroy(qm_dn_state*) {}
qm_status qm_dn_state_clone(const qm_dn_state*, qm_dn_state**) { return fail(QM_ERR_INVALID_ARGUMENT, "not built"); }
qm_status qm_dn_state_read(const qm_dn_state*, float*, float*) { return fail(QM_ERR_INVALID_ARGUMENT, "not built"); }
qm_status qm_dn_state_write(qm_dn_state*, const float*, const float*) { return fail(QM_ERR_INVALID_ARGUMENT, "not built"); }
qm_status qm_dn_step(qm_runtime*, const qm_dn_weights*, qm_dn_state*, const float*, const float*, const float*, const float*, float, float*) { return fail(QM_ERR_INVALID_ARGUMENT, "not built"); }
qm_status qm_dn_prefill(qm_runtime*, const qm_dn_weights*, const qm_dn_state*, qm_dn_state*, const float*, const float*, const float*, const float*, uint32_t, float, float*) { return fail(QM_ERR_INVALID_ARGUMENT, "not built"); }
}
