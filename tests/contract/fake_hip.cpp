// Fake HIP runtime over host memory.  "Device" allocations are host blocks
// tracked in fake::live, so pointer and range queries answer as the real
// runtime does for device memory, copies really copy (ASan sees overruns),
// and a leak shows as a block still live after the API call returned.
#include "fake.hpp"

#include <cstdlib>
#include <cstring>
#include <memory>

namespace fake {

Counters n;
int current_device = 0;
std::string arch = "gfx950:sramecc+:xnack-";
int wave = 64;
hipError_t props_error = hipSuccess;
hipError_t get_device_error = hipSuccess;
int malloc_fail_at = -1, copy_fail_at = -1, sync_fail_at = -1, launch_fail_at = -1, free_fail_at = -1;
hipError_t malloc_error = hipErrorOutOfMemory, copy_error = hipErrorUnknown, sync_error = hipErrorUnknown,
           launch_error = hipErrorLaunchFailure;
std::map<uintptr_t, Block> live;
std::vector<Launch> launches;

void reset_failures() {
    malloc_fail_at = copy_fail_at = sync_fail_at = launch_fail_at = free_fail_at = -1;
    malloc_error = hipErrorOutOfMemory;
    copy_error = sync_error = hipErrorUnknown;
    launch_error = hipErrorLaunchFailure;
}

// Counts down a failure knob: true when this call is the one that fails.
static bool trips(int& at) {
    if (at < 0) return false;
    if (at == 0) {
        at = -1;
        return true;
    }
    --at;
    return false;
}

hipError_t launch_result() {
    ++n.launches;
    return trips(launch_fail_at) ? launch_error : hipSuccess;
}

static const Block* find_block(const void* p, uintptr_t* base) {
    const uintptr_t a = reinterpret_cast<uintptr_t>(p);
    auto it = live.upper_bound(a);
    if (it == live.begin()) return nullptr;
    --it;
    if (a >= it->first + it->second.bytes) return nullptr;
    if (base) *base = it->first;
    return &it->second;
}

bool in_live_block(const void* p, uint64_t bytes) {
    uintptr_t base = 0;
    const Block* b = find_block(p, &base);
    return b && reinterpret_cast<uintptr_t>(p) - base + bytes <= b->bytes;
}

struct Stream {
    int device;
};
static std::vector<std::unique_ptr<Stream>> streams;

hipStream_t make_stream(int device) {
    streams.push_back(std::make_unique<Stream>(Stream{device}));
    return reinterpret_cast<hipStream_t>(streams.back().get());
}

void destroy_streams() { streams.clear(); }

static const Stream* find_stream(hipStream_t s) {
    for (const auto& p : streams)
        if (reinterpret_cast<hipStream_t>(p.get()) == s) return p.get();
    return nullptr;
}

}  // namespace fake

using namespace fake;

hipError_t hipGetDevice(int* device) {
    ++n.device_queries;
    *device = current_device;
    return get_device_error;
}

hipError_t hipGetDeviceProperties(hipDeviceProp_t* props, int device) {
    if (props_error != hipSuccess) return props_error;
    if (device < 0 || device > 7) return hipErrorInvalidDevice;
    std::memset(props, 0, sizeof(*props));
    std::strncpy(props->gcnArchName, arch.c_str(), sizeof(props->gcnArchName) - 1);
    props->warpSize = wave;
    props->multiProcessorCount = 256;
    return hipSuccess;
}

hipError_t hipStreamGetDevice(hipStream_t stream, hipDevice_t* device) {
    ++n.stream_queries;
    const Stream* s = find_stream(stream);
    if (!s) return hipErrorInvalidValue;
    *device = s->device;
    return hipSuccess;
}

hipError_t hipStreamGetFlags(hipStream_t stream, unsigned int* flags) {
    ++n.stream_queries;
    if (!find_stream(stream)) return hipErrorInvalidValue;
    *flags = 0;
    return hipSuccess;
}

hipError_t hipPointerGetAttributes(hipPointerAttribute_t* attr, const void* p) {
    ++n.pointer_queries;
    const Block* b = find_block(p, nullptr);
    attr->type = b ? hipMemoryTypeDevice : hipMemoryTypeHost;
    attr->device = b ? b->device : -1;
    attr->isManaged = 0;
    return b ? hipSuccess : hipErrorInvalidValue;
}

hipError_t hipMemGetAddressRange(hipDeviceptr_t* base, size_t* size, hipDeviceptr_t p) {
    ++n.range_queries;
    uintptr_t b = 0;
    const Block* blk = find_block(p, &b);
    if (!blk) return hipErrorInvalidValue;
    *base = reinterpret_cast<hipDeviceptr_t>(b);
    *size = blk->bytes;
    return hipSuccess;
}

hipError_t hipMalloc(void** p, size_t bytes) {
    ++n.mallocs;
    *p = nullptr;
    if (trips(malloc_fail_at)) return malloc_error;
    void* q = std::aligned_alloc(256, (bytes + 255) / 256 * 256 + 256);
    if (!q) return hipErrorOutOfMemory;
    live[reinterpret_cast<uintptr_t>(q)] = Block{bytes, current_device};
    *p = q;
    return hipSuccess;
}

hipError_t hipFree(void* p) {
    ++n.frees;
    if (!p) return hipSuccess;
    if (trips(free_fail_at)) return hipErrorUnknown;
    auto it = live.find(reinterpret_cast<uintptr_t>(p));
    if (it == live.end()) std::abort();   // freeing something not allocated: an API bug
    live.erase(it);
    std::free(p);
    return hipSuccess;
}

hipError_t hipMemcpyAsync(void* dst, const void* src, size_t bytes, hipMemcpyKind kind, hipStream_t) {
    ++n.copies;
    if (trips(copy_fail_at)) return copy_error;
    // the device side of the copy lies in a device allocation
    if (!in_live_block(kind == hipMemcpyDeviceToHost ? src : dst, bytes)) std::abort();
    std::memcpy(dst, src, bytes);
    return hipSuccess;
}

hipError_t hipStreamSynchronize(hipStream_t) {
    ++n.syncs;
    return trips(sync_fail_at) ? sync_error : hipSuccess;
}
