/*
 * qmm_scratch.hip -- the fixed device scratch behind dfq_qmm_noalloc.
 *
 * dfq_qmm takes its workspace from the caller.  Callers that cannot allocate device memory at
 * all (code under HIP graph capture, tight serving loops, harnesses that forbid hipMalloc)
 * call dfq_qmm_noalloc instead, whose workspace is this file-scope array: one per GPU the
 * library runs on, DFQ_SCRATCH_MAX_BYTES long, alive until the process ends.
 *
 * In host code the name `scratch` is a host-side stand-in, not a device address: it is never
 * passed to a kernel or a copy.  scratch_setup (called by dfq_init with the device current)
 * takes the device address once per device with hipGetSymbolAddress, clears the array the
 * first time, and every later use goes through that address.  The fast kernel leaves its
 * workspace zero after every call, so the array stays zero at rest between calls.
 */
#include <hip/hip_runtime.h>

#include <mutex>

#include "qmm_internal.h"

static __device__ __align__(256) unsigned char scratch[DFQ_SCRATCH_MAX_BYTES];

namespace {

constexpr int kMaxDevices = 64;

std::mutex g_mu;
void* g_ptr[kMaxDevices] = {};  // device address of `scratch` on each device, once taken

}  // namespace

namespace dfq {

dfq_status scratch_setup(int device, void** out) {
    *out = nullptr;
    if (device < 0 || device >= kMaxDevices)
        return fail(DFQ_ERR_UNSUPPORTED, "device %d: scratch is kept for devices 0..%d", device,
                    kMaxDevices - 1);
    std::lock_guard<std::mutex> lk(g_mu);
    if (!g_ptr[device]) {
        int cur = -1;
        hipError_t e = hipGetDevice(&cur);
        if (e != hipSuccess || cur != device)
            return fail(DFQ_ERR_STATE, "scratch set-up needs device %d current", device);
        void* p = nullptr;
        if ((e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch))) != hipSuccess || !p)
            return fail(DFQ_ERR_HIP, "hipGetSymbolAddress(scratch): %s", hipGetErrorString(e));
        /* zero once: every call leaves the workspace zero again */
        if ((e = hipMemset(p, 0, DFQ_SCRATCH_MAX_BYTES)) != hipSuccess ||
            (e = hipDeviceSynchronize()) != hipSuccess)
            return fail(DFQ_ERR_HIP, "clearing the scratch: %s", hipGetErrorString(e));
        g_ptr[device] = p;
    }
    *out = g_ptr[device];
    return DFQ_OK;
}

}  // namespace dfq
