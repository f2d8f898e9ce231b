// tmac_scratch.hip -- the fixed device scratch buffer behind the entry points
// that allocate nothing (tmac_attention_decode_ragged_noalloc).
//
// `scratch` is a file-scope device array: every GPU the library runs on holds
// its own copy, at its own address, from the first use on that device until
// the process ends.  In host code the array's name is only a stand-in for the
// device symbol; its device address is obtained once per device with
// hipGetSymbolAddress (tmac_scratch_setup, called by tmac_init with that device
// current) and only that address is handed to kernels.
//
// Every call on a device shares the one array, which keeps the last call's
// contents: calls that overlap on one GPU (several streams, several host
// threads, several contexts) race on it.  No kernel that uses it expects any
// part of it to start at zero.
#include <hip/hip_runtime.h>

#include <mutex>

#include "tmac_attn.h"

namespace {

constexpr int kMaxDevices = 64;

static __device__ __align__(256) unsigned char scratch[TMAC_SCRATCH_BYTES];

std::mutex g_lock;
void* g_ptr[kMaxDevices] = {};  // device address of `scratch` on each device, once resolved

}  // namespace

// Resolves the address of `scratch` on `device`, which must be the current
// device.  Returns a hipError_t value (0 = hipSuccess).
extern "C" __attribute__((visibility("hidden"))) int tmac_scratch_setup(int device, void** ptr) {
    if (device < 0 || device >= kMaxDevices || !ptr) return (int)hipErrorInvalidValue;
    std::lock_guard<std::mutex> guard(g_lock);
    if (!g_ptr[device]) {
        void* p = nullptr;
        const hipError_t e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
        if (e != hipSuccess) return (int)e;
        if (!p) return (int)hipErrorInvalidSymbol;
        g_ptr[device] = p;
    }
    *ptr = g_ptr[device];
    return (int)hipSuccess;
}
