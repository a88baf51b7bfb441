// Tensor-parallel dense plan entry points (reference include/strix_trellis.h:314-414).
//
// These rank-specific plan variants (S4 / LEGACY identities, q_a||kv pair,
// SwiGLU pair) are outside this library's scope: they return
// STRIX_ERROR_NOT_IMPLEMENTED exactly as a reference build without
// STRIX_TRELLIS_ENABLE_EXPERIMENTAL_TP does (reference src/tp_api.inc:663-719),
// with the same output-handle and query-clearing behaviour.  The descriptor
// initialisers stay usable.  A rank's dense projection is served by the
// generic strix_gemv / strix_linear_plan path on the rank's weight slice.
#include "api_internal.hpp"

extern "C" {

void strix_tp_dense_pair_desc_init(strix_tp_dense_pair_desc* d) {
    if (!d) return;
    *d = strix_tp_dense_pair_desc{};
    d->struct_size = sizeof(*d);
    d->abi_version = STRIX_TRELLIS_ABI_VERSION;
    d->input.struct_size = sizeof(strix_tensor_desc);
    d->input.abi_version = STRIX_TRELLIS_ABI_VERSION;
    d->input.dtype = STRIX_DTYPE_F32;
    for (auto& m : d->member) {
        m.output.struct_size = sizeof(strix_tensor_desc);
        m.output.abi_version = STRIX_TRELLIS_ABI_VERSION;
        m.output.dtype = STRIX_DTYPE_F32;
        m.alpha = 1.0f;
    }
}

void strix_tp_swiglu_desc_init(strix_tp_swiglu_desc* d) {
    if (!d) return;
    *d = strix_tp_swiglu_desc{};
    d->struct_size = sizeof(*d);
    d->abi_version = STRIX_TRELLIS_ABI_VERSION;
    d->input.struct_size = d->hidden_output.struct_size = sizeof(strix_tensor_desc);
    d->input.abi_version = d->hidden_output.abi_version = STRIX_TRELLIS_ABI_VERSION;
    d->input.dtype = d->hidden_output.dtype = STRIX_DTYPE_F32;
}

#define STX_NOT_IMPLEMENTED_CREATE(out)           \
    if (out) *out = nullptr;                       \
    return STRIX_ERROR_NOT_IMPLEMENTED;
#define STX_NOT_IMPLEMENTED_QUERY(out) \
    if (out) *out = 0;                 \
    return STRIX_ERROR_NOT_IMPLEMENTED;

strix_status strix_tp_dense_plan_create(strix_context, const strix_matmul_desc*, const strix_stream*,
                                        strix_tp_dense_plan* out) {
    STX_NOT_IMPLEMENTED_CREATE(out)
}
strix_status strix_tp_dense_plan_create_tiled(strix_context, const strix_matmul_desc*, const strix_stream*, uint32_t,
                                              strix_tp_dense_plan* out) {
    STX_NOT_IMPLEMENTED_CREATE(out)
}
strix_status strix_tp_dense_workspace_bytes(strix_context, const strix_matmul_desc*, uint32_t, uint64_t* out) {
    STX_NOT_IMPLEMENTED_QUERY(out)
}
strix_status strix_tp_dense_plan_create_splitk(strix_context, const strix_matmul_desc*, const strix_stream*, uint32_t,
                                               uint32_t, strix_tp_dense_plan* out) {
    STX_NOT_IMPLEMENTED_CREATE(out)
}
strix_status strix_tp_dense_pair_workspace_bytes(strix_context, const strix_tp_dense_pair_desc*, uint64_t* out) {
    STX_NOT_IMPLEMENTED_QUERY(out)
}
strix_status strix_tp_dense_pair_plan_create(strix_context, const strix_tp_dense_pair_desc*, const strix_stream*,
                                             strix_tp_dense_pair_plan* out) {
    STX_NOT_IMPLEMENTED_CREATE(out)
}
strix_status strix_tp_dense_pair_plan_submit(strix_tp_dense_pair_plan) { return STRIX_ERROR_NOT_IMPLEMENTED; }
strix_status strix_tp_dense_pair_plan_destroy(strix_tp_dense_pair_plan) { return STRIX_ERROR_NOT_IMPLEMENTED; }
strix_status strix_tp_swiglu_workspace_bytes(strix_context, const strix_tp_swiglu_desc*, uint64_t* out) {
    STX_NOT_IMPLEMENTED_QUERY(out)
}
strix_status strix_tp_swiglu_plan_create(strix_context, const strix_tp_swiglu_desc*, const strix_stream*,
                                         strix_tp_swiglu_plan* out) {
    STX_NOT_IMPLEMENTED_CREATE(out)
}
strix_status strix_tp_swiglu_plan_submit(strix_tp_swiglu_plan) { return STRIX_ERROR_NOT_IMPLEMENTED; }
strix_status strix_tp_swiglu_plan_destroy(strix_tp_swiglu_plan) { return STRIX_ERROR_NOT_IMPLEMENTED; }
strix_status strix_tp_dense_r1_workspace_bytes(strix_context, const strix_matmul_desc*, uint32_t, uint32_t,
                                               uint64_t* out) {
    STX_NOT_IMPLEMENTED_QUERY(out)
}
strix_status strix_tp_dense_plan_create_r1(strix_context, const strix_matmul_desc*, const strix_stream*, uint32_t,
                                           uint32_t, strix_tp_dense_plan* out) {
    STX_NOT_IMPLEMENTED_CREATE(out)
}
strix_status strix_tp_dense_plan_submit(strix_tp_dense_plan) { return STRIX_ERROR_NOT_IMPLEMENTED; }
strix_status strix_tp_dense_plan_destroy(strix_tp_dense_plan) { return STRIX_ERROR_NOT_IMPLEMENTED; }
strix_status strix_tp_dense_pair_r1_workspace_bytes(strix_context, const strix_tp_dense_pair_desc*, uint32_t,
                                                    uint64_t* out) {
    STX_NOT_IMPLEMENTED_QUERY(out)
}
strix_status strix_tp_dense_pair_plan_create_r1(strix_context, const strix_tp_dense_pair_desc*, const strix_stream*,
                                                uint32_t, strix_tp_dense_plan* out) {
    STX_NOT_IMPLEMENTED_CREATE(out)
}

}  // extern "C"
