// Device scratch of the allocation-free GEMV entry point
// (strix_amd_gemv_noalloc): the split partial planes of the two-launch GEMV
// live in this file-scope array instead of a caller workspace.  The runtime
// places one copy of it on every device the library runs on, for the life of
// the process.  Its address on a device is looked up once, with that device
// current, and kept per device; host code passes that address to kernels,
// never the array's own name (on the host the name is only a stand-in).
#include <mutex>

#include "backend.hpp"

namespace stx {

static __device__ __align__(256) unsigned char scratch[kGemvScratchBytes];

namespace {
constexpr int kMaxDevices = 64;
std::mutex g_lock;
void* g_address[kMaxDevices] = {};
}  // namespace

hipError_t gemv_scratch_address(int device, void** out) {
    *out = nullptr;
    if (device < 0 || device >= kMaxDevices) return hipErrorInvalidDevice;
    std::lock_guard<std::mutex> lock(g_lock);
    if (!g_address[device]) {
        int current = 0;
        hipError_t e = hipGetDevice(&current);
        if (e != hipSuccess) return e;
        if (current != device && (e = hipSetDevice(device)) != hipSuccess) return e;
        void* p = nullptr;
        e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
        if (current != device) {
            const hipError_t back = hipSetDevice(current);
            if (e == hipSuccess) e = back;
        }
        if (e != hipSuccess) return e;
        if (!p) return hipErrorInvalidSymbol;
        g_address[device] = p;
    }
    *out = g_address[device];
    return hipSuccess;
}

}  // namespace stx
