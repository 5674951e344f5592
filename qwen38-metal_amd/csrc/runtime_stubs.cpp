// Temporary: entry points whose kernels are not built yet.
#include "runtime_internal.h"
using namespace qm;
extern "C" {
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
