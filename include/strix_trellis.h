/*
 * strix_trellis C ABI v1 -- MI355X (gfx950, CDNA4, wave64) implementation.
 *
 * Drop-in boundary.  Every type, enum value, macro and function below has the
 * layout, value and signature of the reference header
 * (reference include/strix_trellis.h:1-531) so that an engine compiled against
 * that header links against libstrix_trellis.so unchanged.  The comments here
 * describe this implementation; the cited reference lines name the interface
 * each declaration replaces.
 *
 * Conventions (reference include/strix_trellis.h:11-14):
 *   - descriptors are zero-initialised, then struct_size / abi_version set;
 *   - reserved fields must be zero;
 *   - dimensions and strides count elements, sizes and offsets count bytes;
 *   - no ownership passes through any call.
 */
#ifndef STRIX_TRELLIS_H
#define STRIX_TRELLIS_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* reference include/strix_trellis.h:15-23 */
#define STRIX_TRELLIS_ABI_VERSION UINT32_C(1)
#define STRIX_TRELLIS_VERSION_MAJOR 0
#define STRIX_TRELLIS_VERSION_MINOR 3
#define STRIX_TRELLIS_VERSION_PATCH 0
#define STRIX_TRELLIS_TRANSPORT_VERSION UINT32_C(1)
#define STRIX_TRELLIS_WORKSPACE_ALIGNMENT UINT32_C(256)
#define STRIX_EXL3_MARKER_3INST UINT32_C(0)
#define STRIX_EXL3_MARKER_MCG UINT32_C(0xCBAC1FED)
#define STRIX_EXL3_MARKER_MUL1 UINT32_C(0x83DCD12D)

/* reference include/strix_trellis.h:25-35 */
typedef enum strix_status {
    STRIX_SUCCESS = 0,
    STRIX_ERROR_INVALID_ARGUMENT = 1,
    STRIX_ERROR_ABI_MISMATCH = 2,
    STRIX_ERROR_UNSUPPORTED_FORMAT = 3,
    STRIX_ERROR_UNSUPPORTED_DEVICE = 4,
    STRIX_ERROR_INSUFFICIENT_BUFFER = 5,
    STRIX_ERROR_OUT_OF_MEMORY = 6,
    STRIX_ERROR_BACKEND = 7,
    STRIX_ERROR_NOT_IMPLEMENTED = 8
} strix_status;

/* reference include/strix_trellis.h:37-42.  F16 and BF16 are reserved values;
 * tensors must be F32. */
typedef enum strix_dtype {
    STRIX_DTYPE_INVALID = 0,
    STRIX_DTYPE_F16 = 1,
    STRIX_DTYPE_BF16 = 2,
    STRIX_DTYPE_F32 = 3
} strix_dtype;

/* reference include/strix_trellis.h:46-49 */
typedef enum strix_transport_format {
    STRIX_TRANSPORT_INVALID = 0,
    STRIX_TRANSPORT_EXL3_CANONICAL = 1
} strix_transport_format;

/* reference include/strix_trellis.h:51-55 */
typedef enum strix_codebook {
    STRIX_CODEBOOK_3INST = 0,
    STRIX_CODEBOOK_MCG = 1,
    STRIX_CODEBOOK_MUL1 = 2
} strix_codebook;

/* Host-native metadata of one EXL3 linear (reference include/strix_trellis.h:57-70).
 * rows = N (outputs), columns = I (inputs); both positive multiples of 128.
 * bits_x2 is an even value 2..16 (integer rates 1..8 bits per weight). */
typedef struct strix_exl3_metadata_v1 {
    uint32_t struct_size;
    uint32_t transport_version;
    uint64_t rows;
    uint64_t columns;
    uint32_t bits_x2;
    strix_codebook codebook;
    uint32_t marker;
    uint32_t flags;
    uint64_t trellis_offset, trellis_bytes;
    uint64_t suh_offset, suh_bytes;
    uint64_t svh_offset, svh_bytes;
    uint64_t bias_offset, bias_bytes;
    uint64_t reserved[4];
} strix_exl3_metadata_v1;

/* One contiguous host blob plus metadata (reference include/strix_trellis.h:72-84). */
typedef struct strix_exl3_transport_desc {
    uint32_t struct_size;
    uint32_t abi_version;
    strix_transport_format format;
    uint32_t transport_version;
    const void *data;
    uint64_t data_bytes;
    const void *metadata;
    uint64_t metadata_bytes;
    uint64_t rows;
    uint64_t columns;
    uint64_t reserved[4];
} strix_exl3_transport_desc;

/* Borrowed host byte range (reference include/strix_trellis.h:89-92). */
typedef struct strix_host_region {
    const void *data;
    uint64_t bytes;
} strix_host_region;

/* Independent host regions instead of one blob (reference include/strix_trellis.h:95-109). */
typedef struct strix_exl3_parts_desc {
    uint32_t struct_size;
    uint32_t abi_version;
    uint32_t transport_version;
    uint32_t bits_x2;
    uint64_t rows;
    uint64_t columns;
    strix_codebook codebook;
    uint32_t marker;
    strix_host_region trellis;
    strix_host_region suh;
    strix_host_region svh;
    strix_host_region bias;
    uint64_t reserved[4];
} strix_exl3_parts_desc;

/* Opaque handles (reference include/strix_trellis.h:113-117). */
typedef struct strix_context_impl *strix_context;
typedef struct strix_weights_impl *strix_weights;
typedef struct strix_linear_plan_impl *strix_linear_plan;
typedef struct strix_tp_dense_plan_impl *strix_tp_dense_plan;
typedef struct strix_tp_moe_plan_impl *strix_tp_moe_plan;
#define STRIX_OPERATION_GEMV UINT32_C(0)
#define STRIX_OPERATION_GEMM UINT32_C(1)

/* Borrowed hipStream_t; NULL selects the context device's default stream
 * (reference include/strix_trellis.h:120-125). */
typedef struct strix_stream {
    uint32_t struct_size;
    uint32_t abi_version;
    void *hip_stream;
    uint64_t reserved[2];
} strix_stream;

/* reference include/strix_trellis.h:127-133 */
typedef struct strix_context_desc {
    uint32_t struct_size;
    uint32_t abi_version;
    int32_t device_ordinal;
    uint32_t flags;
    uint64_t reserved[4];
} strix_context_desc;

/* Contiguous row-major F32 device tensor of rank 1 or 2
 * (reference include/strix_trellis.h:137-147). */
typedef struct strix_tensor_desc {
    uint32_t struct_size;
    uint32_t abi_version;
    void *data;
    uint64_t buffer_bytes;
    strix_dtype dtype;
    uint32_t rank;
    uint64_t shape[2];
    uint64_t strides[2];
    uint64_t reserved[4];
} strix_tensor_desc;

/* output = alpha * Linear(input) + beta * output (reference include/strix_trellis.h:149-166).
 * GEMV: rank 1 [I] -> [N] or rank 2 [B,I] -> [B,N] with B = 0..8.
 * GEMM: rank 2, B = 0..INT_MAX.  beta == 0 never reads the old output. */
typedef struct strix_matmul_desc {
    uint32_t struct_size;
    uint32_t abi_version;
    strix_weights weights;
    strix_tensor_desc input;
    strix_tensor_desc output;
    float alpha;
    float beta;
    void *workspace;
    uint64_t workspace_bytes;
    uint64_t reserved[4];
} strix_matmul_desc;

/* Pre-routed grouped linears sharing one workspace (reference include/strix_trellis.h:168-180). */
typedef struct strix_grouped_moe_desc {
    uint32_t struct_size;
    uint32_t abi_version;
    const strix_matmul_desc *groups;
    uint64_t group_count;
    void *workspace;
    uint64_t workspace_bytes;
    uint64_t reserved[4];
} strix_grouped_moe_desc;

/* Expert-block constants of the reference (reference include/strix_trellis.h:187-190).
 * This implementation accepts these values and, through the same descriptors,
 * larger banks (see strix_tp_moe_plan_create). */
#define STRIX_TP_TOP_K UINT32_C(6)
#define STRIX_TP_MAX_ROWS UINT32_C(8)
#define STRIX_TP_MAX_EXPERTS UINT32_C(48)
#define STRIX_TP_MAX_BANK_EXPERTS UINT32_C(256)

/* reference include/strix_trellis.h:195-205 */
typedef struct strix_tp_expert_desc {
    uint32_t struct_size;
    uint32_t abi_version;
    uint32_t expert_id;
    uint32_t flags;
    strix_weights gate;
    strix_weights up;
    strix_weights down;
    uint64_t reserved[2];
} strix_tp_expert_desc;

/* Host-routed expert window (reference include/strix_trellis.h:207-233). */
typedef struct strix_tp_moe_desc {
    uint32_t struct_size;
    uint32_t abi_version;
    strix_tensor_desc input;
    strix_tensor_desc output;
    const strix_tp_expert_desc *experts;
    uint64_t expert_count;
    const uint32_t *route_ids;
    uint64_t route_ids_count;
    const float *route_scores;
    uint64_t route_scores_count;
    void *workspace;
    uint64_t workspace_bytes;
    float alpha;
    float beta;
    uint64_t reserved[4];
} strix_tp_moe_desc;

/* Persistent bank with device routing (reference include/strix_trellis.h:235-262). */
typedef struct strix_tp_moe_device_desc {
    uint32_t struct_size;
    uint32_t abi_version;
    strix_tensor_desc input;
    strix_tensor_desc output;
    const strix_tp_expert_desc *experts;
    uint64_t expert_count;
    const uint32_t *route_ids;
    uint64_t route_ids_bytes;
    const float *route_scores;
    uint64_t route_scores_bytes;
    void *workspace;
    uint64_t workspace_bytes;
    float alpha;
    float beta;
    uint64_t reserved[4];
} strix_tp_moe_device_desc;

/* ---- core entry points (reference include/strix_trellis.h:264-312) ---- */
uint32_t strix_get_abi_version(void);
const char *strix_status_string(strix_status status);
void strix_matmul_desc_init(strix_matmul_desc *desc);
/* Accepts a gfx950 device (feature suffixes allowed) reporting wave size 64;
 * any other device returns STRIX_ERROR_UNSUPPORTED_DEVICE. */
strix_status strix_context_create(const strix_context_desc *desc, strix_context *out);
strix_status strix_context_destroy(strix_context context);
strix_status strix_weights_prepare(strix_context context,
    const strix_exl3_transport_desc *transport, const strix_stream *stream,
    strix_weights *out);
strix_status strix_weights_prepare_parts(strix_context context,
    const strix_exl3_parts_desc *parts, const strix_stream *stream,
    strix_weights *out);
strix_status strix_weights_destroy(strix_weights weights);
#define STRIX_TRELLIS_HAS_WEIGHTS_SPAN 1
strix_status strix_weights_device_span(strix_weights weights,
    const void **data, uint64_t *bytes);
strix_status strix_matmul_workspace_bytes(strix_context context,
    const strix_matmul_desc *desc, uint64_t *out_bytes);
strix_status strix_gemv(strix_context context, const strix_matmul_desc *desc,
    const strix_stream *stream);
strix_status strix_gemm(strix_context context, const strix_matmul_desc *desc,
    const strix_stream *stream);
/* Prepared plan: validated once, submitted with no allocation, copy,
 * synchronisation or pointer query (reference include/strix_trellis.h:291-305).
 * A GEMV plan with 1..8 rows runs as ONE kernel launch in which the workgroup
 * of the last split of each 128-output group folds the other splits' partial
 * planes; the planes are allocated per plan at creation, owned by the weights
 * handle, and hold an empty marker between submissions. */
strix_status strix_linear_plan_create(strix_context context,
    const strix_matmul_desc *desc, const strix_stream *stream,
    uint32_t operation, strix_linear_plan *out);
strix_status strix_linear_plan_submit(strix_linear_plan plan);
strix_status strix_linear_plan_destroy(strix_linear_plan plan);
strix_status strix_grouped_moe_workspace_bytes(strix_context context,
    const strix_grouped_moe_desc *desc, uint64_t *out_bytes);
strix_status strix_grouped_moe(strix_context context,
    const strix_grouped_moe_desc *desc, const strix_stream *stream);

/* ---- TP dense plans (reference include/strix_trellis.h:314-414) ----
 * One TP rank's dense projections on row views (reference src/tp_api.inc:663-719).
 * Every creator runs the library's decode GEMV, so each output row is
 * bit-identical to strix_gemv on the same row; the workspace queries return 0. */
strix_status strix_tp_dense_plan_create(strix_context context,
    const strix_matmul_desc *desc, const strix_stream *stream,
    strix_tp_dense_plan *out);
strix_status strix_tp_dense_plan_create_tiled(strix_context context,
    const strix_matmul_desc *desc, const strix_stream *stream,
    uint32_t rows_per_block, strix_tp_dense_plan *out);
#define STRIX_TP_SPLITK_SINGLE UINT32_C(0)
#define STRIX_TP_SPLITK_TWO UINT32_C(1)
strix_status strix_tp_dense_workspace_bytes(strix_context context,
    const strix_matmul_desc *desc, uint32_t rows_per_block, uint64_t *out_bytes);
strix_status strix_tp_dense_plan_create_splitk(strix_context context,
    const strix_matmul_desc *desc, const strix_stream *stream,
    uint32_t rows_per_block, uint32_t strategy, strix_tp_dense_plan *out);
typedef struct strix_tp_dense_pair_member {
    strix_weights weights;
    strix_tensor_desc output;
    float alpha;
    float beta;
} strix_tp_dense_pair_member;
typedef struct strix_tp_dense_pair_desc {
    uint32_t struct_size;
    uint32_t abi_version;
    strix_tensor_desc input;
    strix_tp_dense_pair_member member[2];
    void *workspace;
    uint64_t workspace_bytes;
    uint32_t rows_per_block;
    uint32_t strategy;
    uint64_t reserved[4];
} strix_tp_dense_pair_desc;
typedef struct strix_tp_swiglu_desc {
    uint32_t struct_size;
    uint32_t abi_version;
    strix_tensor_desc input;
    strix_weights gate;
    strix_weights up;
    strix_tensor_desc hidden_output;
    void *workspace;
    uint64_t workspace_bytes;
    uint32_t rows_per_block;
    uint32_t strategy;
    float *diagnostic_gate;
    float *diagnostic_up;
    uint64_t diagnostic_bytes;
    uint64_t reserved[4];
} strix_tp_swiglu_desc;
typedef struct strix_tp_dense_pair_plan_impl *strix_tp_dense_pair_plan;
typedef struct strix_tp_dense_pair_plan_impl *strix_tp_swiglu_plan;
void strix_tp_dense_pair_desc_init(strix_tp_dense_pair_desc *desc);
void strix_tp_swiglu_desc_init(strix_tp_swiglu_desc *desc);
strix_status strix_tp_dense_pair_workspace_bytes(strix_context context,
    const strix_tp_dense_pair_desc *desc, uint64_t *out_bytes);
strix_status strix_tp_dense_pair_plan_create(strix_context context,
    const strix_tp_dense_pair_desc *desc, const strix_stream *stream, strix_tp_dense_pair_plan *out);
strix_status strix_tp_dense_pair_plan_submit(strix_tp_dense_pair_plan plan);
strix_status strix_tp_dense_pair_plan_destroy(strix_tp_dense_pair_plan plan);
strix_status strix_tp_swiglu_workspace_bytes(strix_context context,
    const strix_tp_swiglu_desc *desc, uint64_t *out_bytes);
strix_status strix_tp_swiglu_plan_create(strix_context context,
    const strix_tp_swiglu_desc *desc, const strix_stream *stream, strix_tp_swiglu_plan *out);
strix_status strix_tp_swiglu_plan_submit(strix_tp_swiglu_plan plan);
strix_status strix_tp_swiglu_plan_destroy(strix_tp_swiglu_plan plan);
#define STRIX_DENSE_R1_S4 UINT32_C(0)
#define STRIX_DENSE_R1_LEGACY UINT32_C(1)
strix_status strix_tp_dense_r1_workspace_bytes(strix_context context,
    const strix_matmul_desc *desc, uint32_t rows_per_block, uint32_t identity,
    uint64_t *out_bytes);
strix_status strix_tp_dense_plan_create_r1(strix_context context,
    const strix_matmul_desc *desc, const strix_stream *stream,
    uint32_t rows_per_block, uint32_t identity, strix_tp_dense_plan *out);
strix_status strix_tp_dense_plan_submit(strix_tp_dense_plan plan);
strix_status strix_tp_dense_plan_destroy(strix_tp_dense_plan plan);
strix_status strix_tp_dense_pair_r1_workspace_bytes(strix_context context,
    const strix_tp_dense_pair_desc *desc, uint32_t identity, uint64_t *out_bytes);
strix_status strix_tp_dense_pair_plan_create_r1(strix_context context,
    const strix_tp_dense_pair_desc *desc, const strix_stream *stream,
    uint32_t identity, strix_tp_dense_plan *out);

/* ---- grouped strided GEMV (reference include/strix_trellis.h:415-457) ----
 *   output[r][g*output_group_stride + n] = Linear_g(input[r][g*input_group_stride + i])
 * alpha 1, beta 0, rows 1..8.  Every row has the bits of that row submitted
 * alone through strix_gemv (STRIX_GEMV_ROW_INVARIANT_R1, required).
 * This implementation admits any group count 1..STRIX_TP_MAX_BANK_EXPERTS,
 * any common geometry and bit width of the generic GEMV, and bias. */
#define STRIX_TRELLIS_HAS_GROUPED_GEMV 1
#define STRIX_GEMV_ROW_INVARIANT_R1 UINT32_C(1)
typedef struct strix_grouped_gemv_desc {
    uint32_t struct_size;
    uint32_t abi_version;
    const strix_weights *weights;
    uint64_t group_count;
    uint32_t rows;
    uint32_t flags;
    const float *input;
    uint64_t input_row_stride;
    uint64_t input_group_stride;
    uint64_t input_buffer_bytes;
    float *output;
    uint64_t output_row_stride;
    uint64_t output_group_stride;
    uint64_t output_buffer_bytes;
    void *workspace;
    uint64_t workspace_bytes;
    uint64_t reserved[4];
} strix_grouped_gemv_desc;
typedef struct strix_grouped_gemv_plan_impl *strix_grouped_gemv_plan;
strix_status strix_grouped_gemv_workspace_bytes(strix_context context,
    const strix_grouped_gemv_desc *desc, uint64_t *out_bytes);
strix_status strix_grouped_gemv_plan_create(strix_context context,
    const strix_grouped_gemv_desc *desc, const strix_stream *stream, strix_grouped_gemv_plan *out);
strix_status strix_grouped_gemv_plan_submit(strix_grouped_gemv_plan plan);
strix_status strix_grouped_gemv_plan_destroy(strix_grouped_gemv_plan plan);

/* ---- routed-expert block (reference include/strix_trellis.h:458-523) ---- */
void strix_tp_moe_desc_init(strix_tp_moe_desc *desc);
void strix_tp_moe_device_desc_init(strix_tp_moe_device_desc *desc);
strix_status strix_tp_moe_workspace_bytes(strix_context context,
    const strix_tp_moe_desc *desc, uint64_t *out_bytes);
strix_status strix_tp_moe_plan_create(strix_context context,
    const strix_tp_moe_desc *desc, const strix_stream *stream,
    strix_tp_moe_plan *out);
strix_status strix_tp_moe_plan_create_device(strix_context context,
    const strix_tp_moe_device_desc *desc, const strix_stream *stream,
    strix_tp_moe_plan *out);
/* Split plans: the workspace holds hidden F32 [rows][k][H] and, from the next
 * 256-byte boundary, P F32 [rows][k][S][I], the down core's per-split partial
 * sums.  S = 4 with split s over input blocks [s T / 4, (s + 1) T / 4) of the
 * T = H / 16 blocks, as in the reference, for every H up to 5120 (and larger H
 * whose parts fit the kernel; else the down core's own split count).  Every down of a split plan
 * writes P for each computed route (valid token, non-zero score).  The staged
 * calls (split plans only): down_core writes P alone, down_finish folds P as
 * the caller leaves it into the output, down_reference_core recomputes P one
 * route per workgroup with the same bits. */
strix_status strix_tp_moe_split_workspace_bytes(strix_context context,
    const strix_tp_moe_desc *desc, uint64_t *out_bytes);
strix_status strix_tp_moe_plan_create_split(strix_context context,
    const strix_tp_moe_desc *desc, const strix_stream *stream,
    strix_tp_moe_plan *out);
strix_status strix_tp_moe_plan_create_device_split(strix_context context,
    const strix_tp_moe_device_desc *desc, const strix_stream *stream,
    strix_tp_moe_plan *out);
strix_status strix_tp_moe_plan_create_a8r(strix_context context,
    const strix_tp_moe_desc *desc, const strix_stream *stream,
    strix_tp_moe_plan *out);
strix_status strix_tp_moe_plan_create_device_a8r(strix_context context,
    const strix_tp_moe_device_desc *desc, const strix_stream *stream,
    strix_tp_moe_plan *out);
strix_status strix_tp_moe_plan_down_core(strix_tp_moe_plan plan);
strix_status strix_tp_moe_plan_down_finish(strix_tp_moe_plan plan);
strix_status strix_tp_moe_plan_down_reference_core(strix_tp_moe_plan plan);
strix_status strix_tp_moe_plan_submit(strix_tp_moe_plan plan);
strix_status strix_tp_moe_plan_gate_up(strix_tp_moe_plan plan);
strix_status strix_tp_moe_plan_down(strix_tp_moe_plan plan);
strix_status strix_tp_moe_plan_destroy(strix_tp_moe_plan plan);

#ifdef __cplusplus
}
#endif
#endif /* STRIX_TRELLIS_H */
