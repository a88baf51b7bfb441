// Host-only stand-in for <hip/hip_runtime.h>, used to compile the C ABI layer
// (api*.cpp, dispatch.cpp, policy.cpp) on the CPU under ASan/UBSan.  It
// declares only the runtime pieces that layer uses; fake_hip.cpp implements
// them over host memory with failure knobs and call counters.  The kernel
// launchers the layer calls are replaced by fake_launch.cpp.
#pragma once
#include <stddef.h>
#include <stdint.h>

enum hipError_t {
    hipSuccess = 0,
    hipErrorInvalidValue = 1,
    hipErrorOutOfMemory = 2,
    hipErrorNoDevice = 100,
    hipErrorInvalidDevice = 101,
    hipErrorLaunchFailure = 719,
    hipErrorUnknown = 999,
};

struct ihipStream_t;
typedef ihipStream_t* hipStream_t;
typedef int hipDevice_t;
typedef void* hipDeviceptr_t;

enum hipMemcpyKind { hipMemcpyHostToDevice = 1, hipMemcpyDeviceToHost = 2 };
enum hipMemoryType { hipMemoryTypeHost = 0, hipMemoryTypeDevice = 1 };

struct hipDeviceProp_t {
    char gcnArchName[256];
    int warpSize;
    int multiProcessorCount;
};

struct hipPointerAttribute_t {
    hipMemoryType type;
    int device;
    int isManaged;
};

hipError_t hipGetDevice(int* device);
hipError_t hipGetDeviceProperties(hipDeviceProp_t* props, int device);
hipError_t hipStreamGetDevice(hipStream_t stream, hipDevice_t* device);
hipError_t hipStreamGetFlags(hipStream_t stream, unsigned int* flags);
hipError_t hipPointerGetAttributes(hipPointerAttribute_t* attr, const void* p);
hipError_t hipMemGetAddressRange(hipDeviceptr_t* base, size_t* size, hipDeviceptr_t p);
hipError_t hipMalloc(void** p, size_t bytes);
hipError_t hipFree(void* p);
hipError_t hipMemcpyAsync(void* dst, const void* src, size_t bytes, hipMemcpyKind kind, hipStream_t stream);
hipError_t hipStreamSynchronize(hipStream_t stream);

template <class T>
inline hipError_t hipMalloc(T** p, size_t bytes) {
    return hipMalloc(reinterpret_cast<void**>(p), bytes);
}
