// q8_noalloc.hip -- the device scratch of q8_matmul_noalloc (include/q8mi.h).
//
// A file-scope device array, Q8_NOALLOC_SCRATCH_BYTES (8 MiB) on every GPU the
// library runs on, held until the process ends.  It is compiled into
// libq8mi.so's own fat binary (this file is built by hipcc with host and
// device code; the hot-path kernels are a separate code object loaded with
// hipModuleLoadData).  In host code `scratch` names a host-side stand-in, not
// the device array: its device address comes from hipGetSymbolAddress, once
// per device with that device current, and only that address is ever handed
// to a kernel.
#include <hip/hip_runtime.h>

#include <mutex>

#include "../../include/q8mi.h"
#include "q8_internal.h"
#include "q8_noalloc_owner.h"

static __device__ __align__(256) unsigned char scratch[Q8_NOALLOC_SCRATCH_BYTES];

namespace {
constexpr int kMaxDevices = q8i::NoallocOwners::kMaxDevices;
std::mutex g_mu;
void *g_ptr[kMaxDevices] = {};
q8i::NoallocOwners g_owners;
}  // namespace

namespace q8i {

// The device address of `scratch` on `device` (which must be current),
// looked up on the first call for that device and kept.
int noalloc_scratch(int device, void **out) {
    if (device < 0 || device >= kMaxDevices)
        return set_error(Q8_ERR_NO_DEVICE, "noalloc scratch: device %d outside 0..%d", device, kMaxDevices - 1);
    std::lock_guard<std::mutex> lock(g_mu);
    if (!g_ptr[device]) {
        void *p = nullptr;
        const hipError_t e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
        if (e != hipSuccess || !p)
            return set_error(Q8_ERR_HIP, "hip: hipGetSymbolAddress(noalloc scratch) failed: %s",
                             hipGetErrorString(e));
        g_ptr[device] = p;
    }
    *out = g_ptr[device];
    return Q8_OK;
}

bool noalloc_claim(int device, const q8_ctx *ctx) { return g_owners.claim(device, ctx); }

void noalloc_release(const q8_ctx *ctx) { g_owners.release(ctx); }

}  // namespace q8i
