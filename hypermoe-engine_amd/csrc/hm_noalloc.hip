// hm_noalloc.hip -- hm_moe_block_forward without allocation (no reference
// counterpart): the block's workspace in a library-owned device array.
//
// The array is the only device symbol of this file, which has no kernels, so
// it is a code object of its own: a device holds the array from the time the
// HIP runtime loads this code object there (the address lookup of the first
// no-alloc call on that device: block calls before it leave the device's
// free memory unchanged, that call takes the 64 MiB) until the process
// ends.
#include "hm_device.h"

#include <mutex>

// ---- The block without allocation (no reference counterpart) ----------
// hm_moe_block_forward_noalloc runs hm_moe_block_forward with its workspace
// in `scratch`, a file-scope device array of HM_NOALLOC_WORKSPACE_BYTES that
// every GPU the library runs on holds until the process ends.  In host code
// `scratch` names a host-side stand-in, not the device array: its device
// address comes from hipGetSymbolAddress, once per device, with that device
// current, and only that address is ever passed on.  Calls that overlap on
// one device share the array and race; a call leaves its contents behind
// (every region the block needs cleared is cleared by its own kernels).
static __device__ __align__(256) unsigned char scratch[HM_NOALLOC_WORKSPACE_BYTES];

namespace {

constexpr int kMaxNoallocDevices = 64;

struct NoallocScratch {
    std::once_flag once;
    void* ptr = nullptr;
    hipError_t err = hipSuccess;
};
NoallocScratch g_noalloc[kMaxNoallocDevices];

// The current device's address of `scratch` (resolved on the first call on
// that device); nullptr and the HIP error when it cannot be resolved.
void* noalloc_scratch(hipError_t* err) {
    int dev = -1;
    hipError_t e = hipGetDevice(&dev);
    if (e != hipSuccess || dev < 0 || dev >= kMaxNoallocDevices) {
        *err = e != hipSuccess ? e : hipErrorInvalidDevice;
        return nullptr;
    }
    NoallocScratch& d = g_noalloc[dev];
    std::call_once(d.once, [&d] {
        void* p = nullptr;
        d.err = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
        if (d.err == hipSuccess) d.ptr = p;
    });
    *err = d.err;
    return d.ptr;
}

}  // namespace

extern "C" {

int hm_moe_block_forward_noalloc(const hm_layer* layer, const float* hidden,
                                 const float* router_w, int64_t tokens, int32_t top_k,
                                 uint32_t route_flags, int32_t limbs_x, int32_t limbs_z,
                                 const hm_block_io* io, void* stream) {
    const size_t need =
        hm_moe_block_workspace_bytes(layer, tokens, top_k, limbs_x, limbs_z, route_flags);
    if (need == 0) return HM_ERR_INVALID;
    if (need > HM_NOALLOC_WORKSPACE_BYTES) return HM_ERR_UNSUPPORTED;
    hipError_t err = hipSuccess;
    void* ws = noalloc_scratch(&err);
    if (!ws) {
        hm_record_hip_error(err);
        return HM_ERR_RUNTIME;
    }
    return hm_moe_block_forward(layer, hidden, router_w, tokens, top_k, route_flags, limbs_x,
                                limbs_z, io, ws, HM_NOALLOC_WORKSPACE_BYTES, stream);
}

}  // extern "C"

