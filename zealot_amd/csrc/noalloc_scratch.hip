// noalloc_scratch.hip -- the device scratch of zk_paged_decode_noalloc.
//
// A file-scope device array, one copy per GPU, held until the process ends.
// It lives in a translation unit of its own, which holds no kernel: the HIP
// runtime loads a code object onto a device on first use, so the array is
// reserved on a GPU only when noalloc_scratch() first looks it up there, not
// when any other kernel of the library first runs.  Host code never uses the
// array's name as a device address (on the host it names a stand-in): the
// device address comes from hipGetSymbolAddress, once per device, with that
// device current, and is kept per device.
#include <hip/hip_runtime.h>

#include <atomic>
#include <mutex>
#include <string>

#include "zk_common.h"

static __device__ __align__(256) unsigned char scratch[ZK_DECODE_SCRATCH_BYTES];

namespace {

constexpr int kMaxDevices = 64;
std::atomic<void *> g_scratch_ptr[kMaxDevices];
std::mutex g_scratch_mu;

}  // namespace

int zk::noalloc_scratch(void **out) {
    int dev = -1;
    ZK_HIP_CHECK(hipGetDevice(&dev), "zk_paged_decode_noalloc: hipGetDevice");
    if (dev < 0 || dev >= kMaxDevices)
        return set_error(ZK_ERR_INVALID_ARGUMENT, "Internal error: zk_paged_decode_noalloc: device ordinal " +
                                                      std::to_string(dev) + " out of range");
    void *p = g_scratch_ptr[dev].load(std::memory_order_acquire);
    if (!p) {
        std::lock_guard<std::mutex> g(g_scratch_mu);
        p = g_scratch_ptr[dev].load(std::memory_order_relaxed);
        if (!p) {
            ZK_HIP_CHECK(hipGetSymbolAddress(&p, HIP_SYMBOL(scratch)), "zk_paged_decode_noalloc: scratch address");
            if (!p) return set_error(ZK_ERR_HIP, "Internal error: zk_paged_decode_noalloc: NULL scratch address");
            g_scratch_ptr[dev].store(p, std::memory_order_release);
        }
    }
    *out = p;
    return ZK_OK;
}
