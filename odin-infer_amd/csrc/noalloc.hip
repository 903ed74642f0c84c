// noalloc.hip -- the routed-expert FFN for callers that cannot allocate
// device memory (code under HIP graph capture, tight serving loops, harnesses
// that forbid hipMalloc): oi_moe_ffn_launch with its workspace taken from a
// file-scope device array instead of a caller buffer.
//
// The array is one per GPU (each device that runs this library holds its own
// copy until the process ends).  Its device address is looked up once per
// device with hipGetSymbolAddress, on the first call on that device with the
// device current, and kept per device: in host code the array's name is only a
// host-side stand-in and must never be passed to a kernel.
//
// What the workspace holds (router logits, chosen ids and weights, the chosen
// experts' SwiGLU outputs) is written completely by each call before it is
// read, so nothing needs clearing between calls.  Every call on one GPU shares
// that GPU's array: calls that overlap on one GPU (two streams, or two host
// threads) race.

#include <mutex>
#include <string>

#include "oi.h"
#include "oi_kernels.h"

namespace {

// 512 KiB: router logits (<= 1024 experts) + ids and weights (<= 32 each) +
// top_k x inter SwiGLU outputs; enough for every configuration this build
// measures (128 experts top 8 inter 768: 6,288 floats; 512 experts top 10
// inter 512: 5,652 floats) with room for top_k x inter up to ~130k.
constexpr size_t kScratchFloats = 131072;
__device__ __align__(256) float scratch[kScratchFloats];

constexpr int kMaxDevices = 64;
std::mutex g_mu;
void *g_scratch_dev[kMaxDevices];  // device address of `scratch` on each device, once looked up

int scratch_ptr(void **out) {
    int dev = -1;
    if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= kMaxDevices)
        return oi::set_error(OI_E_DEVICE, "moe (no-alloc): no current HIP device");
    std::lock_guard<std::mutex> lk(g_mu);
    if (!g_scratch_dev[dev]) {
        void *p = nullptr;
        const hipError_t r = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
        if (r != hipSuccess || !p)
            return oi::set_error(OI_E_DEVICE, (std::string("moe (no-alloc): hipGetSymbolAddress: ") +
                                               hipGetErrorString(r)).c_str());
        g_scratch_dev[dev] = p;
    }
    *out = g_scratch_dev[dev];
    return OI_OK;
}

}  // namespace

extern "C" int oi_moe_ffn_launch_noalloc(const oi_moe_dims *d, const oi_weights *router, const oi_weights *gate,
                                         const oi_weights *up, const oi_weights *down, const float *x_dev,
                                         float *y_dev, void *stream) {
    const int64_t need = oi_moe_workspace_bytes(d);
    if (need <= 0) return oi::set_error(OI_E_ARG, "moe (no-alloc): bad dims (dim and inter multiples of 64, "
                                                  "top_k <= 32)");
    if ((size_t)need > sizeof(scratch))
        return oi::set_error(OI_E_ARG, ("moe (no-alloc): workspace of " + std::to_string(need) +
                                        " bytes exceeds the library's fixed " + std::to_string(sizeof(scratch)) +
                                        " bytes (n_experts + 2 top_k + top_k * inter floats)").c_str());
    void *ws = nullptr;
    const int rc = scratch_ptr(&ws);
    if (rc) return rc;
    return oi_moe_ffn_launch(d, router, gate, up, down, x_dev, ws, y_dev, stream);
}
