// ltx_attn_fwd_static: ltx_attn_fwd for callers that cannot allocate device memory (code
// under HIP graph capture, tight serving loops, harnesses that forbid hipMalloc). The call's
// scratch -- the Q/K statistics, the prepared K' of the K prologue and the split-KV partials,
// which ltx_attn_fwd takes from the caller's workspace -- lives in one file-scope device
// array of kScratchBytes instead. Same plan, same kernels, same results as ltx_attn_fwd with
// a workspace of ltx_attn_workspace_bytes; calls that need more scratch than the array holds
// are refused.
//
// The array's name is only a host-side stand-in: its device address is looked up once per
// device (hipGetSymbolAddress, with that device current) on the first call there, and that
// address is what reaches the kernels. Each device holds its own copy until the process
// ends. Every call on one device shares that device's copy: calls that overlap on one
// device (two streams, two threads) race and must be serialised by the caller. Nothing in
// it has to start at zero: every byte a call reads was written earlier in the same call.
#include <hip/hip_runtime.h>

#include <stdarg.h>

#include <mutex>

#include "../../include/ltx_attn.h"
#include "fmha_params.hpp"

namespace {

__attribute__((format(printf, 2, 3))) ltx_attn_status fail(ltx_attn_status s, const char *fmt,
                                                          ...) {
    va_list ap;
    va_start(ap, fmt);
    ltx::set_error_detail((int)s, fmt, ap);
    va_end(ap);
    return s;
}

constexpr size_t kScratchBytes = LTX_ATTN_STATIC_SCRATCH_BYTES;
constexpr int kMaxDevices = 64;

static __device__ __align__(256) unsigned char scratch[kScratchBytes];

void *g_scratch[kMaxDevices];          // device address of `scratch` per device
hipError_t g_lookup[kMaxDevices];      // result of the one lookup per device
std::once_flag g_once[kMaxDevices];

}  // namespace

extern "C" ltx_attn_status ltx_attn_fwd_static(const ltx_attn_args *a, void *stream) {
    if (!a) return fail(LTX_ATTN_EINVAL, "args is NULL");
    ltx_attn_args b = *a;
    b.workspace = nullptr;
    b.workspace_bytes = 0;
    const size_t need = ltx_attn_workspace_bytes(&b);
    if (need == 0) {
        // invalid arguments (the detail is set), or a call that needs no scratch at all
        if (ltx_attn_status s = ltx_attn_validate(&b)) return s;
        return ltx_attn_fwd(&b, stream);
    }
    if (need > kScratchBytes)
        return fail(LTX_ATTN_EUNSUPPORTED,
                    "this call needs %zu bytes of scratch; ltx_attn_fwd_static holds %zu (use "
                    "ltx_attn_fwd with a workspace, or kprep FUSED / num_splits 1 for a "
                    "smaller plan)",
                    need, kScratchBytes);
    int dev = -1;
    if (hipError_t e = hipGetDevice(&dev))
        return fail(LTX_ATTN_EHIP, "hipGetDevice: %s", hipGetErrorString(e));
    if (dev < 0 || dev >= kMaxDevices)
        return fail(LTX_ATTN_EUNSUPPORTED, "device %d beyond the %d the static scratch serves",
                    dev, kMaxDevices);
    std::call_once(g_once[dev], [dev] {
        g_lookup[dev] = hipGetSymbolAddress(&g_scratch[dev], HIP_SYMBOL(scratch));
    });
    if (g_lookup[dev] != hipSuccess || !g_scratch[dev])
        return fail(LTX_ATTN_EHIP, "hipGetSymbolAddress(scratch) on device %d: %s", dev,
                    hipGetErrorString(g_lookup[dev]));
    // exactly the sized workspace: ltx_attn_fwd then picks the plan it would pick for a
    // caller's workspace of ltx_attn_workspace_bytes (the device's own plan only where that
    // fits in it), so both entry points run the same plan on any part
    b.workspace = g_scratch[dev];
    b.workspace_bytes = need;
    return ltx_attn_fwd(&b, stream);
}
