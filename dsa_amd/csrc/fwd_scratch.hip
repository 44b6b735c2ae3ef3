// dsa_fwd_noalloc: the forward call for callers that cannot allocate (code
// under HIP graph capture, serving loops, harnesses that forbid hipMalloc).
// It is dsa_fwd_opts with the split partials -- and, for a plan that merges
// inside the main kernel, the arrival counters -- taken from `scratch`, a
// file-scope device array of fixed size, instead of caller buffers.  It calls
// no hipMalloc / hipFree and no allocating library routine.
//
// Each GPU holds its own copy of `scratch` until the process ends.  In host
// code the name `scratch` is a host-side stand-in, not a device address: the
// device address is fetched once per device with hipGetSymbolAddress (with
// that device current) and only that pointer is ever passed to kernels.
//
// Every call on one GPU shares that GPU's scratch and leaves the last call's
// partials in it; calls that can overlap on one GPU (other streams, or graphs
// replayed concurrently) race on it.  The arrival counters must be zero on
// entry: they are cleared by a fill kernel at the first call on each device
// (no hipMemsetAsync, so a first call under graph capture records a kernel),
// and every call leaves them zero again once its kernel completes.
#include <hip/hip_runtime.h>

#include <mutex>

#include "../../include/dsa_mi355x.h"
#include "kernels.h"

namespace {

constexpr int64_t kPartialBytes = DSA_NOALLOC_PARTIAL_BYTES;  // split partials: part_o, part_m, part_l
constexpr int64_t kCounterWords = 1024;                       // arrival counters of the in-kernel merge
// A fused plan has split >= 2 and >= 16 heads per group, so each (token, head
// group) counter comes with >= 2 * 16 * 2056 bytes of partials: the partial
// region bounds the counters needed below 1024.
static_assert(kPartialBytes / (2 * 16 * 2056) < kCounterWords, "counter region covers every fused plan");

static __device__ __align__(256) uint32_t scratch[kPartialBytes / 4 + kCounterWords];

constexpr int kMaxDevices = 64;
std::mutex g_mu;
char* g_scratch[kMaxDevices] = {};  // device address of `scratch` per device, set once

__global__ void zero_words(uint32_t* p, int n) {
    const int i = blockIdx.x * blockDim.x + threadIdx.x;
    if (i < n) p[i] = 0u;
}

// Device address of this device's scratch; at the first call on a device,
// fetch it (with that device current) and enqueue the counters' zero fill on
// `stream`, ahead of the call's own kernels.
int device_scratch(hipStream_t stream, char** out) {
    int dev = 0;
    hipError_t e = stream ? hipStreamGetDevice(stream, &dev) : hipGetDevice(&dev);
    if (e != hipSuccess) return (int)e;
    if (dev < 0 || dev >= kMaxDevices) return (int)hipErrorInvalidDevice;
    std::lock_guard<std::mutex> lock(g_mu);
    if (!g_scratch[dev]) {
        int cur = 0;
        e = hipGetDevice(&cur);
        if (e == hipSuccess && cur != dev) e = hipSetDevice(dev);
        void* ptr = nullptr;
        if (e == hipSuccess) e = hipGetSymbolAddress(&ptr, HIP_SYMBOL(scratch));
        if (e == hipSuccess && ptr == nullptr) e = hipErrorInvalidSymbol;
        if (e == hipSuccess) {
            uint32_t* counters = reinterpret_cast<uint32_t*>(static_cast<char*>(ptr) + kPartialBytes);
            hipLaunchKernelGGL(zero_words, dim3((unsigned)((kCounterWords + 255) / 256)), dim3(256), 0, stream,
                               counters, (int)kCounterWords);
            e = hipGetLastError();
        }
        if (cur != dev) {
            const hipError_t r = hipSetDevice(cur);
            if (e == hipSuccess) e = r;
        }
        if (e != hipSuccess) return (int)e;
        g_scratch[dev] = static_cast<char*>(ptr);
    }
    *out = g_scratch[dev];
    return 0;
}

}  // namespace

extern "C" int dsa_fwd_noalloc(const uint16_t* q, const uint16_t* kv, const uint16_t* q_rope, const uint16_t* k_rope,
                               const int32_t* idx, uint16_t* out, float* out_max, float* out_sum, int B, int SQ,
                               int H, int L, int TOPK, const dsa_fwd_options* opts, const dsa_plan* plan,
                               void* stream_) {
    const hipStream_t stream = static_cast<hipStream_t>(stream_);
    dsa::FwdCall call;
    // Every check (the partials' size against the scratch included) before
    // anything touches the device.
    if (int rc = dsa::fwd_prepare(q, kv, q_rope, k_rope, idx, out, out_max, out_sum, nullptr, nullptr, nullptr, B,
                                  SQ, H, L, TOPK, opts, plan, true, kPartialBytes, &call))
        return rc;
    char* base = nullptr;
    if (call.split) {
        if (int rc = device_scratch(stream, &base))
            return dsa::set_error(rc, "dsa_fwd_noalloc: scratch set-up failed (%s)",
                                  hipGetErrorString((hipError_t)rc));
        const auto up = [](int64_t b) { return (b + 255) / 256 * 256; };
        const int64_t rows = call.part_rows;
        call.p.part_o = reinterpret_cast<float*>(base);
        call.p.part_m = reinterpret_cast<float*>(base + up(rows * 512 * 4));
        call.p.part_l = reinterpret_cast<float*>(base + up(rows * 512 * 4) + up(rows * 4));
        if (call.fused) call.p.arrivals = reinterpret_cast<uint32_t*>(base + kPartialBytes);
    }
    return dsa::fwd_enqueue(call, stream);
}
