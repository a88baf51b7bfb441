// Internal interface between the C ABI layer (api.cpp) and the HIP kernels.
// Plain structs and host launch functions; nothing here is part of the ABI.
#pragma once
#include <hip/hip_runtime.h>
#include <stddef.h>
#include <stdint.h>

namespace stx {

// Prepared weights as the kernels see them (one private device allocation).
struct DeviceWeights {
    const uint32_t* trellis = nullptr;   // [I/16][N/16][8K] u32, transport order
    const uint16_t* suh = nullptr;       // FP16 [I]
    const uint16_t* svh = nullptr;       // FP16 [N]
    const float* bias = nullptr;         // F32 [N] or null
    uint32_t input = 0;                  // I
    uint32_t output = 0;                 // N
    uint32_t bits = 0;                   // K, 1..8
    uint32_t codebook = 0;               // 0 3inst, 1 mcg, 2 mul1
    uint64_t trellis_bytes = 0;
};

// Per-group weight pointers of a grouped launch (device-resident table).
struct GroupWeights {
    const uint32_t* trellis;
    const uint16_t* suh;
    const uint16_t* svh;
    const float* bias;
};

// GEMV decomposition (a function of I, N and K only, never of the row count,
// so every row has the same bits whatever rows are submitted with it).
struct GemvShape {
    uint32_t bps = 0;      // 16-row input blocks per split, multiple of 8
    uint32_t splits = 0;   // S = (I/16) / bps
};
GemvShape gemv_shape(uint32_t input, uint32_t output, uint32_t bits);
// Splits whose S - 1 other planes one finisher poll round covers at eight rows
// (two rows per wave, 32 loads per round), and the fewest workgroups a shape
// limited to them may have.
constexpr uint32_t kOneRoundSplits = 17;
constexpr uint64_t kOneRoundMinWorkgroups = 384;

// Bytes of the caller workspace one call needs (GEMV partial planes and the
// FP16 core-input matrix of the GEMM path); 256-byte aligned pieces.
uint64_t gemv_workspace_bytes(const DeviceWeights& w, uint32_t rows);
uint64_t gemm_workspace_bytes(const DeviceWeights& w, uint64_t rows);
uint64_t linear_workspace_bytes(const DeviceWeights& w, uint64_t rows);
// Single-launch GEMV state, dedicated to one plan (one allocation, 256-byte
// aligned pieces):
//   status  sticky flags (GEMV_STATUS_*), set by a finisher that gave up;
//   epochs  one launch counter per 128-column group ([groups][N/128] u32);
//   planes  two sets of partial sums of splits 0..S-2, per column group
//           ([2][groups * N/128][S-1][rows][128] F32).
// Created with status and epochs 0 and every plane word GEMV_PLANE_EMPTY.  A
// launch of column group g with epoch e uses set e & 1: each split publishes
// its plane there and re-arms (EMPTY-fills) its plane of the other set, which
// the previous launch used and which nothing of this launch reads; the
// finisher polls set e & 1 until no word is EMPTY, then advances epochs[g].
// A finisher that gives up sets GEMV_EPOCH_POISON in epochs[g] instead: a
// split of that launch that starts only after the give-up cannot be told
// apart from the next launch's splits, so no later finisher of g trusts a
// plane (each writes NaN) until the host re-initialises the whole state
// (init_fused_state) in stream order.
struct FusedState {
    uint32_t* status = nullptr;
    uint32_t* epochs = nullptr;
    float* planes = nullptr;
};
constexpr uint32_t GEMV_PLANE_EMPTY = 0xFFFFFFFFu;
constexpr uint32_t GEMV_STATUS_GAVE_UP = 1u;
constexpr uint32_t GEMV_EPOCH_POISON = 0x80000000u;
// Poll rounds before a finisher gives up (a few hundred ms); 0 gives up at
// once without polling (test hook).
constexpr uint32_t GEMV_DEFAULT_POLL_LIMIT = 1u << 22;
// Bytes of the state (0 when one split suffices: the launch needs none), and
// where its pieces start; the planes run from planes_offset to the end.
uint64_t fused_state_bytes(const DeviceWeights& w, uint64_t rows, uint32_t groups);
uint64_t fused_planes_offset(const DeviceWeights& w, uint32_t groups);
FusedState fused_state_at(void* base, const DeviceWeights& w, uint64_t rows, uint32_t groups);

struct LinearCall {
    const float* x = nullptr;
    float* y = nullptr;
    uint64_t rows = 0;
    uint64_t x_row_stride = 0;   // elements
    uint64_t y_row_stride = 0;
    float alpha = 1.0f;
    float beta = 0.0f;
    void* workspace = nullptr;
    // Prefill GEMM split-tile handoff: polls before the second workgroup of a
    // split tile takes it over from K = 0 (UINT32_MAX: always, a test hook).
    uint32_t handoff_poll_limit = 4096;
    // Single-launch GEMV: poll rounds of a finisher before it gives up.
    uint32_t gemv_poll_limit = GEMV_DEFAULT_POLL_LIMIT;
};

// Generic GEMV (rows 1..8): core kernel + finishing kernel, no counters.
hipError_t launch_gemv(const DeviceWeights& w, const LinearCall& call, hipStream_t stream);
// Single-launch GEMV: the workgroup of the last split of each 128-output group
// waits for the other splits' published planes and finishes (state as above).
hipError_t launch_gemv_fused(const DeviceWeights& w, const LinearCall& call, const FusedState& state,
                             hipStream_t stream);
// Second launch of a split-K core: folds planes[S][rows][N] (row stride N) in
// ascending split order from +0, then H32 and the output stage into call.y.
hipError_t launch_plane_finish(const DeviceWeights& w, const LinearCall& call, const float* planes, uint32_t splits,
                               hipStream_t stream);

// Grouped GEMV over `groups` weights of one geometry (table in device memory).
// With `state` (dedicated to the plan, as for launch_gemv_fused) one launch;
// without, the F32 planes are call.workspace and a finishing kernel folds them.
hipError_t launch_gemv_grouped(const DeviceWeights& geometry, const GroupWeights* table, uint32_t groups,
                               const LinearCall& call, uint64_t x_group_stride, uint64_t y_group_stride,
                               const FusedState* state, hipStream_t stream);
// Owner-fold grouped GEMV: one 16-wave workgroup per 128-column group folds
// all of its splits itself (no partial planes, no waiting); every output has
// the bits of launch_gemv_grouped.  gemv_owner_fits: rows 1..8, a split layer,
// LDS within 64 KiB.
bool gemv_owner_fits(const DeviceWeights& geometry, uint64_t rows);
hipError_t launch_gemv_owner(const DeviceWeights& geometry, const GroupWeights* table, uint32_t groups,
                             const LinearCall& call, uint64_t x_group_stride, uint64_t y_group_stride,
                             hipStream_t stream);
// The library's choice between the owner-fold and the split grouped plan.
bool grouped_owner_preferred(const DeviceWeights& geometry, uint32_t groups, uint64_t rows);
// Prefill path (any row count): input stage to FP16 in the workspace, then the
// MFMA core with the fused output stage.
hipError_t launch_gemm(const DeviceWeights& w, const LinearCall& call, hipStream_t stream);
uint32_t gemm_launch_count(const DeviceWeights& w, uint64_t rows);
// K split of the GEMM core for the first pass of a `rows`-row call (1: none).
uint32_t gemm_split_count(const DeviceWeights& w, uint64_t rows);
uint32_t linear_launch_count(const DeviceWeights& w, uint64_t rows, bool gemm, bool single_launch);
// Dispatch used by strix_gemv / strix_gemm / grouped MoE.
hipError_t launch_linear(const DeviceWeights& w, const LinearCall& call, bool prefer_gemm, hipStream_t stream);

// Diagnostics for parity tests (exported through strix_trellis_amd.h).
hipError_t launch_decode(const DeviceWeights& w, _Float16* q, hipStream_t stream);
hipError_t launch_input_stage(const DeviceWeights& w, const float* x, uint64_t rows, _Float16* a,
                              hipStream_t stream);
hipError_t launch_output_stage(const DeviceWeights& w, const float* core, uint64_t rows, float* y,
                               float alpha, float beta, hipStream_t stream);
hipError_t launch_fill_u32(uint32_t* p, uint32_t value, uint64_t count, hipStream_t stream);
// Allocation-free GEMV (strix_amd_gemv_noalloc): the split partial planes of
// the two-launch GEMV in a static device array of kGemvScratchBytes per
// device (noalloc.hip).  gemv_scratch_address returns that array's address on
// `device`, looked up once per device with the device current.
constexpr uint64_t kGemvScratchBytes = uint64_t(4) << 20;
hipError_t gemv_scratch_address(int device, void** out);

// Streaming read of `bytes` (a multiple of 16 * workgroups) by `workgroups` x
// `threads` threads (64..1024, a power of two), `depth` (1..16, a power of
// two) 16-byte loads in flight per lane, nothing stored but one word per
// workgroup into sink: the read ceiling and the call floor of a kernel that
// reads that many bytes once are the fastest such shapes.
bool stream_read_shape_ok(uint32_t threads, uint32_t depth);
hipError_t launch_stream_read(const void* src, uint64_t bytes, uint32_t workgroups, uint32_t threads, uint32_t depth,
                              uint32_t* sink, hipStream_t stream);

}  // namespace stx
