// decode_static.hip -- smoe_hip_moe_decode_static: one token through one MoE
// layer (the single-token form of smoe_hip_moe_decode) with no allocation at
// all, for callers that cannot allocate device memory (code under HIP graph
// capture, tight serving loops, harnesses that forbid hipMalloc).
//
// The kernels are smoe_hip_moe_decode's own: the one-launch layer kernel
// (k_moe_layer) where the shape allows it, else the two launches.  What they
// use beyond the caller's inputs and outputs -- the exchange words of both
// forms, h, the ids / weights / expert table when the caller passes none, an
// error word -- lives in `scratch`, a file-scope device array of fixed size
// (NA_BYTES, about 0.6 MB) that each GPU holds until the process ends.
//
// Host code never passes `scratch` itself to a kernel: its name on the host
// is a stand-in, not a device address.  Each device's address comes from
// hipGetSymbolAddress, taken once per device with that device current (at
// smoe_metal_init, or at the first uncaptured call on the device), and the
// array is cleared there once.  Calls on one GPU share that GPU's array and
// must not overlap (same stream, or ordered); later calls keep its contents:
// the one-launch exchange words carry per-launch tags and are never re-armed,
// the two-launch routing words are re-armed by the down launch.
#include <hip/hip_runtime.h>

#include <cstdio>
#include <mutex>

#include "kernels.hpp"
#include "shape.hpp"
#include "smoe_hip.h"

namespace {

// largest shape of the static scratch
constexpr uint32_t NA_MAX_D = 4096, NA_MAX_I = 2048, NA_MAX_E = 512, NA_MAX_K = 16;

constexpr size_t round32(size_t n) { return (n + 31) & ~size_t(31); }

// layout in 64-bit words
constexpr size_t NA_LX = 0;                                                   // one-launch exchange words
constexpr size_t NA_LL = NA_LX + round32(smoe::lx_words(NA_MAX_D, NA_MAX_E, NA_MAX_I));   // two-launch routing
constexpr size_t NA_H = NA_LL + round32(smoe::ll_token_words(NA_MAX_E));      // h [K x I] fp32
constexpr size_t NA_IDS = NA_H + round32(size_t(NA_MAX_K) * NA_MAX_I / 2);   // ids [K] u32
constexpr size_t NA_W = NA_IDS + 32;                                          // weights [K] fp32
constexpr size_t NA_TBL = NA_W + 32;                                          // expert table [K]
constexpr size_t NA_ERR = NA_TBL + round32(NA_MAX_K * sizeof(smoe::ExpertPtrs) / 8);   // error flags
constexpr size_t NA_WORDS = NA_ERR + 32;
constexpr size_t NA_BYTES = NA_WORDS * sizeof(uint64_t);
static_assert(sizeof(smoe::ExpertPtrs) % 8 == 0, "expert table entries are whole words");

constexpr int NA_MAX_DEVICES = 64;
std::mutex g_mu;
uint64_t* g_ptr[NA_MAX_DEVICES] = {};   // device address of `scratch` per device, once set up

}  // namespace

static __device__ __align__(256) uint64_t scratch[NA_WORDS];

namespace smoe {

// Takes the current device's address of `scratch` and clears the array, once
// per device.  Synchronous (a plain hipMemset): call it outside stream
// capture.  Returns that address, or nullptr on failure.
uint64_t* static_scratch_setup()
{
    int dev = 0;
    if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= NA_MAX_DEVICES) return nullptr;
    std::lock_guard<std::mutex> lock(g_mu);
    if (g_ptr[dev]) return g_ptr[dev];
    void* p = nullptr;
    hipError_t e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
    if (e != hipSuccess || !p) {
        std::fprintf(stderr, "[smoe_hip] hipGetSymbolAddress(scratch) failed on device %d: %s\n", dev,
                     hipGetErrorString(e));
        return nullptr;
    }
    e = hipMemset(p, 0, NA_BYTES);
    if (e == hipSuccess) e = hipDeviceSynchronize();
    if (e != hipSuccess) {
        std::fprintf(stderr, "[smoe_hip] clearing the static scratch failed on device %d: %s\n", dev,
                     hipGetErrorString(e));
        return nullptr;
    }
    g_ptr[dev] = static_cast<uint64_t*>(p);
    (void)deal_probe();   // the one-launch kernel's placement (also synchronous set-up)
    return g_ptr[dev];
}

}  // namespace smoe

namespace {

uint64_t* scratch_of_current_device(hipStream_t s)
{
    int dev = 0;
    if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= NA_MAX_DEVICES) return nullptr;
    {
        std::lock_guard<std::mutex> lock(g_mu);
        if (g_ptr[dev]) return g_ptr[dev];
    }
    // first call on this device: set up now, unless the stream is being
    // captured (the clearing is a synchronous memset)
    hipStreamCaptureStatus st = hipStreamCaptureStatusNone;
    if (hipStreamIsCapturing(s, &st) != hipSuccess || st != hipStreamCaptureStatusNone) return nullptr;
    return smoe::static_scratch_setup();
}

}  // namespace

extern "C" int smoe_hip_moe_decode_static(const SmoeMoeShape* shape, const SmoeMoeLayer* layer, float* hidden,
                                          uint32_t* ids_out, float* weights_out, uint32_t* err_out,
                                          void* hip_stream)
{
    if (!shape || !layer || !hidden || !layer->norm_w || !layer->router_w || !layer->experts) return SMOE_ERR_ARG;
    const int rc = smoe::shape_check(shape);
    if (rc != SMOE_OK) return rc;
    if (shape->d_model > NA_MAX_D || shape->d_ff > NA_MAX_I || shape->n_experts > NA_MAX_E ||
        shape->top_k > NA_MAX_K) {
        std::fprintf(stderr,
                     "[smoe_hip] smoe_hip_moe_decode_static: shape d_model %u, d_ff %u, %u experts, top_k %u "
                     "exceeds its static scratch (d_model <= %u, d_ff <= %u, experts <= %u, top_k <= %u)\n",
                     shape->d_model, shape->d_ff, shape->n_experts, shape->top_k, NA_MAX_D, NA_MAX_I, NA_MAX_E,
                     NA_MAX_K);
        return SMOE_ERR_CAPACITY;
    }
    const hipStream_t s = static_cast<hipStream_t>(hip_stream);
    uint64_t* base = scratch_of_current_device(s);
    if (!base) {
        std::fprintf(stderr, "[smoe_hip] smoe_hip_moe_decode_static: static scratch not set up on this device "
                             "(call smoe_metal_init, or make one call outside stream capture, first)\n");
        return SMOE_ERR_CAPTURE;
    }
    const smoe::MoeDims d = smoe::dims_of(shape);
    const smoe::LayerDesc L = smoe::layer_of(layer);
    uint32_t* ids = ids_out ? ids_out : reinterpret_cast<uint32_t*>(base + NA_IDS);
    float* w = weights_out ? weights_out : reinterpret_cast<float*>(base + NA_W);
    uint32_t* err = err_out ? err_out : reinterpret_cast<uint32_t*>(base + NA_ERR);
    hipError_t e;
    const bool one_launch = smoe::layer_supported(d, L);
    if (d.quant != SMOE_QUANT_SMOEQ4 && !one_launch) return SMOE_ERR_BITS;   // scale+min: one-launch kernel only
    if (one_launch) {
        e = smoe::launch_moe_layer(d, L, hidden, base + NA_LX, ids, w, err, s);
    } else {
        float* h = reinterpret_cast<float*>(base + NA_H);
        auto* tbl = reinterpret_cast<smoe::ExpertPtrs*>(base + NA_TBL);
        e = smoe::launch_moe_up(d, L, hidden, 1, base + NA_LL, h, ids, w, tbl, err, s);
        if (e == hipSuccess) e = smoe::launch_down_combine(d, tbl, h, w, hidden, base + NA_LL, 1, s);
    }
    if (e != hipSuccess) {
        std::fprintf(stderr, "[smoe_hip] smoe_hip_moe_decode_static: launch failed: %s\n", hipGetErrorString(e));
        return SMOE_ERR_HIP;
    }
    return SMOE_OK;
}
