// Scratch memory of the allocation-free entry point
// (atn_attention_fwd_noalloc_ex): a file-scope device array, one copy per
// GPU the library runs on, held until the process ends.
//
// In host code `scratch` names a host-side stand-in, not a device address:
// every host use goes through the address hipGetSymbolAddress returns for
// the current device, taken once per device in noalloc_scratch() and kept.
// The array's first bytes are the workspace's sync region (status word,
// epochs, done words, XCD-local counters), which must start zero-filled:
// the set-up clears them with a small fill kernel (no hipMemsetAsync, so
// the clear is safe to capture), once per device.
#include <mutex>

#include "launch.hpp"

namespace atn {

namespace {

static __device__ __align__(256) unsigned char scratch[kNoAllocScratchBytes];

struct Slot {
    void* ptr = nullptr;
    bool cleared = false;
};
constexpr int kMaxDevices = 64;
Slot g_slots[kMaxDevices];
std::mutex g_mu;

__global__ __launch_bounds__(256) void k_zero_words(unsigned* p, int n) {
    for (int i = blockIdx.x * 256 + threadIdx.x; i < n; i += gridDim.x * 256) p[i] = 0u;
}

}  // namespace

bool noalloc_ready(int dev) {
    if (dev < 0 || dev >= kMaxDevices) return false;
    std::lock_guard<std::mutex> lk(g_mu);
    return g_slots[dev].ptr != nullptr && g_slots[dev].cleared;
}

hipError_t noalloc_scratch(int dev, size_t sync_bytes, hipStream_t st, void** ptr) {
    if (dev < 0 || dev >= kMaxDevices) return hipErrorInvalidDevice;
    std::lock_guard<std::mutex> lk(g_mu);
    Slot& s = g_slots[dev];
    if (s.ptr == nullptr) {
        void* p = nullptr;
        const hipError_t e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
        if (e != hipSuccess) return e;
        s.ptr = p;
    }
    if (!s.cleared) {
        const int words = (int)(sync_bytes / 4);
        hipLaunchKernelGGL(k_zero_words, dim3((unsigned)((words + 255) / 256)), dim3(256), 0, st,
                           static_cast<unsigned*>(s.ptr), words);
        const hipError_t e = hipGetLastError();
        if (e != hipSuccess) return e;
        s.cleared = true;
    }
    *ptr = s.ptr;
    return hipSuccess;
}

}  // namespace atn
