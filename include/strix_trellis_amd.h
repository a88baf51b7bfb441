/*
 * MI355X extensions of the strix_trellis C ABI: stage checkpoints used by the
 * parity tests.  None of these has a counterpart symbol in the reference
 * header; they expose, through the same validation as the ABI calls, the
 * intermediate results the reference's GPU tests compare byte for byte
 * (decoded Q, core input, output stage from a known core:
 * reference tests/gpu_runtime.hip:252-339, docs/GPU_TESTS.md:44-143).
 * All buffers are device memory on the context device; every call enqueues on
 * the given stream and returns without synchronising.
 */
#ifndef STRIX_TRELLIS_AMD_H
#define STRIX_TRELLIS_AMD_H

#include "strix_trellis.h"

#ifdef __cplusplus
extern "C" {
#endif

/* Decoded FP16 Q[I][N] (row-major, input-major) of prepared weights.
 * q_bytes >= 2*I*N.  Bit-exact with the transport's EXL3 decode. */
strix_status strix_amd_decode(strix_weights weights, void *q_fp16, uint64_t q_bytes,
    const strix_stream *stream);

/* FP16 core input A[rows][I] = RN16(H32(RN16(RN32(x * suh)))) of F32 x[rows][I]. */
strix_status strix_amd_input_stage(strix_weights weights, const float *x, uint64_t rows,
    void *a_fp16, uint64_t a_bytes, const strix_stream *stream);

/* Output stage from a known F32 core[rows][N]:
 * y = alpha * (RN32(H32(core) * svh) [+ bias]) (+ beta * y_old iff beta != 0). */
strix_status strix_amd_output_stage(strix_weights weights, const float *core, uint64_t rows,
    float *y, uint64_t y_bytes, float alpha, float beta, const strix_stream *stream);

/* Split decomposition of the GEMV core for these weights: input blocks of 16
 * channels per split and the split count.  It fixes the core's accumulation
 * order and depends only on the weight geometry. */
strix_status strix_amd_gemv_shape(strix_weights weights, uint32_t *blocks_per_split,
    uint32_t *splits);

/* K split of the prefill GEMM core for a call of `rows` rows (its first pass
 * when the rows run in several): 1 = one K pass per output tile, S > 1 = S
 * partial planes folded in ascending order.  Like the GEMV shape it fixes the
 * accumulation order: S depends on the weight geometry and, from 256 rows, on
 * the number of 256-row blocks.  rows = 0 reports the split of one row. */
strix_status strix_amd_gemm_splits(strix_weights weights, uint64_t rows, uint32_t *splits);

/* Kernel launches one submission of a prepared plan enqueues (1 for a
 * single-launch GEMV plan). */
strix_status strix_amd_plan_launches(strix_linear_plan plan, uint32_t *launches);

/* Routed-expert activation on device F32 buffers: hidden[i] = SwiGLU(gate[i], up[i])
 * with the arithmetic the MoE gate/up finish applies (stable sigmoid over the
 * library's own exp; reference src/tp_moe_activation.hpp:46-60 for the form).
 * Exposes that activation for bit-level checks; count 0 launches nothing. */
strix_status strix_amd_swiglu(strix_context context, const float *gate, const float *up, float *hidden,
    uint64_t count, const strix_stream *stream);

/* Workspace bytes of a device-route routed-expert plan, the counterpart of
 * strix_tp_moe_workspace_bytes (split = 0) and strix_tp_moe_split_workspace_bytes
 * (split != 0) for strix_tp_moe_device_desc, with the same validation as
 * strix_tp_moe_plan_create_device.  Plain plans need hidden F32 [rows][k][H];
 * split plans add P F32 [rows][k][S][I] from the next 256-byte boundary, with
 * the split count of strix_tp_moe_split_workspace_bytes (S = 4 up to H = 5120). */
strix_status strix_amd_tp_moe_device_workspace_bytes(strix_context context,
    const strix_tp_moe_device_desc *desc, uint32_t split, uint64_t *out_bytes);

/* Test hook for the prefill GEMM's split-tile handoff (M = 2048-class passes
 * whose 256 x 256 tile count exceeds a multiple of 256 by at most 128).  The
 * second workgroup of a split tile normally continues from the first one's
 * published FP32 accumulators and only recomputes the first half of K itself
 * when that publication is late (bounded wait).  always_take_over != 0 makes
 * every later call and plan created on this context take that recompute path;
 * 0 restores the default.  Outputs are bit-identical either way. */
strix_status strix_amd_set_gemm_handoff(strix_context context, uint32_t always_take_over);

/* Single-launch GEMV plans (linear plans with rows 1-8, grouped plans, TP
 * dense plans): the workgroup of each output group's last input split waits,
 * with a bounded poll, for the other splits' published partial sums.  A wait
 * that runs out writes NaN outputs, sets STRIX_AMD_GEMV_GAVE_UP in the plan's
 * sticky status word and poisons that output group: workgroups are dispatched
 * in order only within one XCD, so a split of the given-up launch may start
 * after the give-up and publish into the planes the next launch reads.  So
 * every later submission writes NaN to the poisoned output groups until
 * strix_amd_plan_status / strix_amd_grouped_plan_status with clear != 0
 * re-initialises the plan's state (in stream order, after every earlier
 * launch has ended).  TP dense plans have no status call: a give-up there
 * shows as NaN outputs, and the plan is recreated.
 * poll_limit = rounds of that wait for every later submission on the context
 * (a round is a few hundred ns); 0 makes every finisher give up at once (test
 * hook).  strix_amd_set_gemv_poll_limit(context, STRIX_AMD_GEMV_POLL_DEFAULT)
 * restores the default. */
#define STRIX_AMD_GEMV_POLL_DEFAULT 4194304u
#define STRIX_AMD_GEMV_GAVE_UP 1u
strix_status strix_amd_set_gemv_poll_limit(strix_context context, uint32_t poll_limit);

/* Sticky status flags of a single-launch plan (0 for plans that need no
 * wait), read after synchronising the plan's stream; clear != 0 also
 * re-initialises the plan's whole single-launch state (status, launch epochs
 * and partial planes; enqueued before the synchronisation), which lifts a
 * give-up's poison.  The caller orders it after every submission and graph
 * replay of the plan it must follow. */
strix_status strix_amd_plan_status(strix_linear_plan plan, uint32_t clear, uint32_t *flags);
strix_status strix_amd_grouped_plan_status(strix_grouped_gemv_plan plan, uint32_t clear, uint32_t *flags);

/* Single-launch state of destroyed linear and TP dense plans.  By default,
 * as the reference keeps its plans' completion counters, the state of every
 * plan lives until its weights are destroyed and distinct plans never share
 * state, so graphs captured from a destroyed plan may still replay at any
 * time.  enable != 0 lets plans created later on the context take an idle
 * state block of a destroyed plan on the same weights (re-initialised on the
 * new plan's stream), which bounds the state held by the plans alive at one
 * time; the caller then must not replay a destroyed plan's graphs after
 * creating a new plan on those weights. */
strix_status strix_amd_set_plan_state_reuse(strix_context context, uint32_t enable);

/* Streaming read, the measurement kernel of the read ceiling and the call
 * floors: one kernel of `workgroups` x `threads` threads reads `bytes` device
 * bytes from src once, each workgroup a contiguous slice, each lane keeping
 * `depth` 16-byte loads in flight, and stores the XOR of each workgroup's
 * slice (one word per workgroup) into sink.  threads is 64, 128, 256, 512 or
 * 1024; depth is 1, 2, 4, 8 or 16; bytes must be a multiple of
 * 16 * workgroups; nothing else is read or written.  strix_amd_stream_read is
 * the 256-thread, depth-4 shape (the decode GEMV's load depth). */
strix_status strix_amd_stream_read_shaped(strix_context context, const void *src, uint64_t bytes,
    uint32_t workgroups, uint32_t threads, uint32_t depth, uint32_t *sink, const strix_stream *stream);
strix_status strix_amd_stream_read(strix_context context, const void *src, uint64_t bytes, uint32_t workgroups,
    uint32_t *sink, const strix_stream *stream);

/* Grouped GEMV plans come in two folds with the same output bits: the split
 * plan (each output group's input splits run in separate workgroups and the
 * last one folds the others' published partials) and the owner-fold plan (one
 * workgroup per 128-column output group runs every split and folds them
 * itself; reference src/dense_r1_group_owner.hip).  fold: 0 = the library's
 * choice, 1 = split, 2 = owner, for grouped plans created later on the
 * context; strix_amd_grouped_plan_fold reports a plan's fold (1 or 2). */
strix_status strix_amd_set_grouped_fold(strix_context context, uint32_t fold);
strix_status strix_amd_grouped_plan_fold(strix_grouped_gemv_plan plan, uint32_t *fold);

/* strix_gemv for 1-8 rows that allocates nothing.  No counterpart in the
 * reference: it is for callers that cannot allocate (code under HIP graph
 * capture, tight serving loops, harnesses that forbid allocation).  The
 * descriptor is validated as for strix_gemv, but must carry no workspace
 * (workspace NULL, workspace_bytes 0): the GEMV's split partial planes go to a
 * static device array of STRIX_AMD_GEMV_NOALLOC_SCRATCH_BYTES that the library
 * holds on every device it runs on until the process ends.  A layer whose
 * planes (splits x rows x N floats) exceed it is rejected with
 * STRIX_ERROR_INSUFFICIENT_BUFFER; more than 8 rows with
 * STRIX_ERROR_UNSUPPORTED_FORMAT.  The output has strix_gemv's exact bits.
 * Every call on a device shares that device's array: calls that overlap in
 * time on one device (different streams, or graphs replayed concurrently)
 * race and must be ordered by the caller. */
#define STRIX_AMD_GEMV_NOALLOC_SCRATCH_BYTES 4194304u
strix_status strix_amd_gemv_noalloc(strix_context context, const strix_matmul_desc *desc,
    const strix_stream *stream);

#ifdef __cplusplus
}
#endif
#endif /* STRIX_TRELLIS_AMD_H */
