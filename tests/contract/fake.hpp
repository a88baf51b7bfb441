// Knobs and counters of the fake HIP runtime (fake_hip.cpp) and the fake
// kernel launchers (fake_launch.cpp) that the contract driver links against
// the real C ABI layer.
#pragma once
#include <hip/hip_runtime.h>

#include <cstdint>
#include <map>
#include <string>
#include <vector>

namespace fake {

struct Counters {
    int mallocs = 0, frees = 0, copies = 0, syncs = 0, launches = 0;
    int pointer_queries = 0, range_queries = 0, stream_queries = 0, device_queries = 0;
};
extern Counters n;

// Device model.
extern int current_device;          // hipGetDevice
extern std::string arch;            // gcnArchName
extern int wave;                    // warpSize
extern hipError_t props_error;      // hipGetDeviceProperties result
extern hipError_t get_device_error; // hipGetDevice result

// Failure injection: the k-th call from now fails (-1: never); *_error is
// the error returned.
extern int malloc_fail_at, copy_fail_at, sync_fail_at, launch_fail_at, free_fail_at;
extern hipError_t malloc_error, copy_error, sync_error, launch_error;
void reset_failures();

// Live fake device allocations: base -> (bytes, device).
struct Block {
    size_t bytes;
    int device;
};
extern std::map<uintptr_t, Block> live;
bool in_live_block(const void* p, uint64_t bytes);

// Fake streams carry their device.
hipStream_t make_stream(int device);
void destroy_streams();

// Record of the launchers called, in order.
struct Launch {
    std::string name;
    uint64_t rows = 0;
    const void* workspace = nullptr;
    const void* planes = nullptr;
    hipStream_t stream = nullptr;
    float alpha = 0, beta = 0;
};
extern std::vector<Launch> launches;

// The fake launchers consume one launch_fail_at count per call.
hipError_t launch_result();

}  // namespace fake
