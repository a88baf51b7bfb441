// Routed-expert block entry points (reference include/strix_trellis.h:458-523).
#include "api_internal.hpp"

extern "C" {

void strix_tp_moe_desc_init(strix_tp_moe_desc* d) {
    if (!d) return;
    *d = strix_tp_moe_desc{};
    d->struct_size = sizeof(*d);
    d->abi_version = STRIX_TRELLIS_ABI_VERSION;
    d->input.struct_size = d->output.struct_size = sizeof(strix_tensor_desc);
    d->input.abi_version = d->output.abi_version = STRIX_TRELLIS_ABI_VERSION;
    d->input.dtype = d->output.dtype = STRIX_DTYPE_F32;
    d->alpha = 1.0f;
}

void strix_tp_moe_device_desc_init(strix_tp_moe_device_desc* d) {
    if (!d) return;
    *d = strix_tp_moe_device_desc{};
    d->struct_size = sizeof(*d);
    d->abi_version = STRIX_TRELLIS_ABI_VERSION;
    d->input.struct_size = d->output.struct_size = sizeof(strix_tensor_desc);
    d->input.abi_version = d->output.abi_version = STRIX_TRELLIS_ABI_VERSION;
    d->input.dtype = d->output.dtype = STRIX_DTYPE_F32;
    d->alpha = 1.0f;
}

#define STX_NI_CREATE(out)    \
    if (out) *out = nullptr;   \
    return STRIX_ERROR_NOT_IMPLEMENTED;
#define STX_NI_QUERY(out) \
    if (out) *out = 0;    \
    return STRIX_ERROR_NOT_IMPLEMENTED;

strix_status strix_tp_moe_workspace_bytes(strix_context, const strix_tp_moe_desc*, uint64_t* out) { STX_NI_QUERY(out) }
strix_status strix_tp_moe_plan_create(strix_context, const strix_tp_moe_desc*, const strix_stream*,
                                      strix_tp_moe_plan* out) { STX_NI_CREATE(out) }
strix_status strix_tp_moe_plan_create_device(strix_context, const strix_tp_moe_device_desc*, const strix_stream*,
                                             strix_tp_moe_plan* out) { STX_NI_CREATE(out) }
strix_status strix_tp_moe_split_workspace_bytes(strix_context, const strix_tp_moe_desc*, uint64_t* out) {
    STX_NI_QUERY(out)
}
strix_status strix_tp_moe_plan_create_split(strix_context, const strix_tp_moe_desc*, const strix_stream*,
                                            strix_tp_moe_plan* out) { STX_NI_CREATE(out) }
strix_status strix_tp_moe_plan_create_device_split(strix_context, const strix_tp_moe_device_desc*, const strix_stream*,
                                                   strix_tp_moe_plan* out) { STX_NI_CREATE(out) }
strix_status strix_tp_moe_plan_create_a8r(strix_context, const strix_tp_moe_desc*, const strix_stream*,
                                          strix_tp_moe_plan* out) { STX_NI_CREATE(out) }
strix_status strix_tp_moe_plan_create_device_a8r(strix_context, const strix_tp_moe_device_desc*, const strix_stream*,
                                                 strix_tp_moe_plan* out) { STX_NI_CREATE(out) }
strix_status strix_tp_moe_plan_down_core(strix_tp_moe_plan) { return STRIX_ERROR_NOT_IMPLEMENTED; }
strix_status strix_tp_moe_plan_down_finish(strix_tp_moe_plan) { return STRIX_ERROR_NOT_IMPLEMENTED; }
strix_status strix_tp_moe_plan_down_reference_core(strix_tp_moe_plan) { return STRIX_ERROR_NOT_IMPLEMENTED; }
strix_status strix_tp_moe_plan_submit(strix_tp_moe_plan) { return STRIX_ERROR_NOT_IMPLEMENTED; }
strix_status strix_tp_moe_plan_gate_up(strix_tp_moe_plan) { return STRIX_ERROR_NOT_IMPLEMENTED; }
strix_status strix_tp_moe_plan_down(strix_tp_moe_plan) { return STRIX_ERROR_NOT_IMPLEMENTED; }
strix_status strix_tp_moe_plan_destroy(strix_tp_moe_plan) { return STRIX_ERROR_NOT_IMPLEMENTED; }

}  // extern "C"
