// The allocation-free MoE layer entry point (lp_moe_forward_noalloc): the
// fused layer with its workspace in a file-scope device array instead of a
// caller-provided buffer, for callers that cannot allocate device memory
// (code under HIP graph capture, tight serving loops, harnesses that forbid
// hipMalloc).
//
// The array below is one per device the library runs on; the runtime gives
// it its own copy on each device, at its own address, held until the process
// ends.  Host code never passes the array's name to the device: its host-side
// name is only a handle for hipGetSymbolAddress, which the context's set-up
// calls once per device with that device current; the address it returns is
// what the kernels get as their workspace.
//
// Every call on a device shares that device's array and leaves its contents
// behind.  Nothing in the workspace needs to start at zero: the dispatch
// kernels write every table the later kernels read (including the status and
// error words) before they are read.  Calls that overlap on one device (on
// different streams, or from different threads without ordering) race on the
// array; callers serialise them.
#include <hip/hip_runtime.h>

#include <mutex>
#include <string>

#include "../../include/llmpager_hip.h"
#include "lp_internal.h"

namespace {

constexpr uint64_t kScratchBytes = LP_NOALLOC_SCRATCH_BYTES;
constexpr int kMaxDevices = 64;

static __device__ __align__(256) uint8_t scratch[kScratchBytes];

std::mutex g_mu;
uint64_t g_ptr[kMaxDevices] = {};  // the array's device address on each device, 0 = not set up

}  // namespace

// Called by lp_init with `device` current: look the array up on this device
// once and keep its address.
int lpi::noalloc_setup(int device) {
    if (device < 0 || device >= kMaxDevices)
        return lpi::set_error(LP_E_UNSUPPORTED, "noalloc scratch: device index out of range");
    std::lock_guard<std::mutex> g(g_mu);
    if (g_ptr[device]) return LP_OK;
    void* p = nullptr;
    const hipError_t e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
    if (e != hipSuccess || !p)
        return lpi::set_error(e != hipSuccess ? (int)e : LP_E_LOAD,
                              std::string("noalloc scratch: hipGetSymbolAddress failed: ") + hipGetErrorString(e));
    g_ptr[device] = reinterpret_cast<uint64_t>(p);
    return LP_OK;
}

extern "C" int lp_moe_forward_noalloc(lp_ctx* ctx, const lp_moe_layer_desc* d, uint64_t x, uint64_t h, int T,
                                      lp_stream s) {
    if (!ctx) return lpi::set_error(LP_E_INVALID, "null context");
    if (!d) return lpi::set_error(LP_E_INVALID, "null layer descriptor");
    lp_moe_ws_layout lay;
    if (int r = lp_moe_ws_layout_get(d, T, &lay)) return r;
    if (lay.total > kScratchBytes)
        return lpi::set_error(LP_E_UNSUPPORTED,
                              "lp_moe_forward_noalloc: this layer needs a " + std::to_string(lay.total) +
                                  "-byte workspace for T = " + std::to_string(T) + ", more than the " +
                                  std::to_string(kScratchBytes) + " bytes of the built-in scratch");
    const int dev = lpi::ctx_device(ctx);
    uint64_t ws = 0;
    {
        std::lock_guard<std::mutex> g(g_mu);
        ws = dev >= 0 && dev < kMaxDevices ? g_ptr[dev] : 0;
    }
    if (!ws) return lpi::set_error(LP_E_LOAD, "lp_moe_forward_noalloc: scratch not set up on this device");
    return lp_moe_forward(ctx, d, x, h, T, ws, kScratchBytes, s);
}

extern "C" uint64_t lp_noalloc_scratch_bytes(void) { return kScratchBytes; }
