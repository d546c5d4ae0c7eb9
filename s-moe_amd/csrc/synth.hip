// synth.hip -- synthetic inputs and the SMOE-Q4 quantizer on gfx950.
//
// Counter-based generator: one 64-bit SplitMix64-style draw per element,
// two 24-bit uniforms, Box-Muller cosine branch with a log and a cosine built
// only from correctly rounded IEEE operations (fmaf, +, *, /, sqrt) in a fixed
// order, so the host and the device produce the same bits for the same
// (seed, stream, index).  Floating-point contraction is off in this file.
//
// k_quantize_q4 restates quantize_smoeq4 (scripts/shatter_moe.py:331-368):
// absmax per group of 64 (0 -> 1.0), code = clip(rint(w/absmax*7.5 + 7.5),
// 0, 15) with round-half-even, fp16(absmax) scale, low nibble = even index.
// k_quantize_q4_min is this build's scale+min format (no counterpart in the
// reference): m = bf16(min), s = bf16((max - min) / 15) (bf16 1.0 if that is
// 0), code = clip(rint((w - m) / s), 0, 15) from the rounded s and m.
#include "device_common.hpp"
#include "kernels.hpp"

#pragma clang fp contract(off)

namespace smoe {

constexpr uint64_t GAMMA = 0x9E3779B97F4A7C15ull;

__device__ __forceinline__ uint64_t fmix64(uint64_t z)
{
    z = (z ^ (z >> 30)) * 0xBF58476D1CE4E5B9ull;
    z = (z ^ (z >> 27)) * 0x94D049BB133111EBull;
    return z ^ (z >> 31);
}

__host__ __device__ inline uint64_t fmix64_h(uint64_t z)
{
    z = (z ^ (z >> 30)) * 0xBF58476D1CE4E5B9ull;
    z = (z ^ (z >> 27)) * 0x94D049BB133111EBull;
    return z ^ (z >> 31);
}

static uint64_t stream_key(uint64_t seed, uint64_t stream)
{
    return fmix64_h(seed * GAMMA + fmix64_h(stream + GAMMA));
}

__device__ __forceinline__ float det_log(float u)
{
    const uint32_t b = __float_as_uint(u);
    int e = static_cast<int>(b >> 23) - 127;
    float m = __uint_as_float((b & 0x7FFFFFu) | 0x3F800000u);
    if (m > 1.41421356f) { m = m * 0.5f; e += 1; }
    const float f = m - 1.0f;
    const float s = f / (2.0f + f);
    const float z = s * s;
    float p = 0.13333333f;
    p = __builtin_fmaf(p, z, 0.15384615f);
    p = __builtin_fmaf(p, z, 0.18181818f);
    p = __builtin_fmaf(p, z, 0.22222222f);
    p = __builtin_fmaf(p, z, 0.28571429f);
    p = __builtin_fmaf(p, z, 0.4f);
    p = __builtin_fmaf(p, z, 0.66666667f);
    const float lnm = __builtin_fmaf(s * z, p, 2.0f * s);
    const float fe = static_cast<float>(e);
    return __builtin_fmaf(fe, 0.693145751953125f, __builtin_fmaf(fe, 1.42860677e-06f, lnm));
}

__device__ __forceinline__ float det_cos2pi(float t)
{
    float y = t - 0.5f;
    float sign = -1.0f;
    y = fabsf(y);
    if (y > 0.25f) { y = 0.5f - y; sign = -sign; }
    const float a = y * 6.28318531f;
    const float a2 = a * a;
    float c = -1.1470746e-11f;
    c = __builtin_fmaf(c, a2, 2.0876757e-09f);
    c = __builtin_fmaf(c, a2, -2.7557319e-07f);
    c = __builtin_fmaf(c, a2, 2.4801587e-05f);
    c = __builtin_fmaf(c, a2, -1.3888889e-03f);
    c = __builtin_fmaf(c, a2, 4.1666668e-02f);
    c = __builtin_fmaf(c, a2, -0.5f);
    c = __builtin_fmaf(c, a2, 1.0f);
    return sign * c;
}

// Correctly rounded square root for x > 0: v_sqrt_f32 is within 1 ulp; the
// fma residuals x - s_dn*s and x - s_up*s tell on which side of the midpoints
// to the neighbouring floats the exact root lies.
__device__ __forceinline__ float sqrt_rn(float x)
{
    if (!(x > 0.0f)) return __builtin_sqrtf(x);
    float s = __builtin_amdgcn_sqrtf(x);
    const float s_dn = __uint_as_float(__float_as_uint(s) - 1u);
    const float s_up = __uint_as_float(__float_as_uint(s) + 1u);
    const float r_dn = __builtin_fmaf(-s_dn, s, x);
    const float r_up = __builtin_fmaf(-s_up, s, x);
    if (r_dn <= 0.0f) s = s_dn;
    if (r_up > 0.0f) s = s_up;
    return s;
}

__device__ __forceinline__ float det_normal(uint64_t key, uint64_t i)
{
    const uint64_t h = fmix64(key + (i + 1) * GAMMA);
    const float u1 = static_cast<float>(static_cast<uint32_t>((h >> 40) + 1u)) * 5.9604644775390625e-8f;
    const float u2 = static_cast<float>(static_cast<uint32_t>((h >> 16) & 0xFFFFFFu)) * 5.9604644775390625e-8f;
    const float r = sqrt_rn(-2.0f * det_log(u1));
    return r * det_cos2pi(u2);
}

__device__ __forceinline__ uint16_t f32_to_bf16_rne(float f)
{
    uint32_t x = __float_as_uint(f);
    if ((x & 0x7FFFFFFFu) > 0x7F800000u) return static_cast<uint16_t>((x >> 16) | 0x40u);
    x += 0x7FFFu + ((x >> 16) & 1u);
    return static_cast<uint16_t>(x >> 16);
}

__device__ __forceinline__ uint16_t f32_to_f16_rne(float f)
{
    return __builtin_bit_cast(uint16_t, static_cast<_Float16>(f));
}

// quantize one group of G weights held in w[] (G <= 128)
template <int G>
__device__ __forceinline__ void quantize_group(const float (&w)[G], uint8_t* packed, uint16_t* scale)
{
    float absmax = 0.f;
#pragma unroll
    for (int j = 0; j < G; ++j) {
        const float a = fabsf(w[j]);
        absmax = a > absmax ? a : absmax;
    }
    const float best = (absmax == 0.0f) ? 1.0f : absmax;
    *scale = f32_to_f16_rne(best);
    uint32_t words[G / 8];
#pragma unroll
    for (int q = 0; q < G / 8; ++q) words[q] = 0;
#pragma unroll
    for (int j = 0; j < G; ++j) {
        // three separately rounded operations, as numpy's w / absmax * 7.5 + 7.5
        // (written as operators under this file's contract(off): the header
        // helpers __fmul_rn / __fadd_rn would still be fused into one fma)
        float q = w[j] / best;
        q = q * 7.5f;
        q = q + 7.5f;
        int c = static_cast<int>(rintf(q));
        c = c < 0 ? 0 : (c > 15 ? 15 : c);
        words[j / 8] |= static_cast<uint32_t>(c) << (4 * (j % 8));
    }
    uint4* dst = reinterpret_cast<uint4*>(packed);
#pragma unroll
    for (int q = 0; q < G / 32; ++q) dst[q] = make_uint4(words[4 * q], words[4 * q + 1], words[4 * q + 2], words[4 * q + 3]);
}

// quantize one group of G weights to the scale+min format
template <int G>
__device__ __forceinline__ void quantize_group_min(const float (&w)[G], uint8_t* packed, uint16_t* scale,
                                                   uint16_t* minv)
{
    float lo = w[0], hi = w[0];
#pragma unroll
    for (int j = 1; j < G; ++j) {
        lo = w[j] < lo ? w[j] : lo;
        hi = w[j] > hi ? w[j] : hi;
    }
    const float span = (hi - lo) / 15.0f;
    uint16_t sb = f32_to_bf16_rne(span);
    if ((sb & 0x7FFFu) == 0) sb = 0x3F80u;                 // a constant group: s = 1
    const uint16_t mb = f32_to_bf16_rne(lo);
    *scale = sb;
    *minv = mb;
    const float s = __uint_as_float(static_cast<uint32_t>(sb) << 16);
    const float m = __uint_as_float(static_cast<uint32_t>(mb) << 16);
    uint32_t words[G / 8];
#pragma unroll
    for (int q = 0; q < G / 8; ++q) words[q] = 0;
#pragma unroll
    for (int j = 0; j < G; ++j) {
        // two separately rounded operations: (w - m), then / s
        float q = w[j] - m;
        q = q / s;
        int c = static_cast<int>(rintf(q));
        c = c < 0 ? 0 : (c > 15 ? 15 : c);
        words[j / 8] |= static_cast<uint32_t>(c) << (4 * (j % 8));
    }
    uint4* dst = reinterpret_cast<uint4*>(packed);
#pragma unroll
    for (int q = 0; q < G / 32; ++q) dst[q] = make_uint4(words[4 * q], words[4 * q + 1], words[4 * q + 2], words[4 * q + 3]);
}

__global__ void k_synth_normal(float* out, uint64_t n, uint64_t key, float stddev)
{
    for (uint64_t i = blockIdx.x * (uint64_t)blockDim.x + threadIdx.x; i < n; i += (uint64_t)gridDim.x * blockDim.x)
        out[i] = det_normal(key, i) * stddev;
}

__global__ void k_synth_bf16(uint16_t* out, uint64_t n, uint64_t key, float stddev)
{
    for (uint64_t i = blockIdx.x * (uint64_t)blockDim.x + threadIdx.x; i < n; i += (uint64_t)gridDim.x * blockDim.x)
        out[i] = f32_to_bf16_rne(det_normal(key, i) * stddev);
}

template <int G>
__global__ void k_quantize_q4(const float* __restrict__ w, uint64_t n_groups, uint8_t* __restrict__ packed,
                              uint16_t* __restrict__ scales)
{
    for (uint64_t g = blockIdx.x * (uint64_t)blockDim.x + threadIdx.x; g < n_groups; g += (uint64_t)gridDim.x * blockDim.x) {
        float v[G];
#pragma unroll
        for (int j = 0; j < G; ++j) v[j] = w[g * G + j];
        quantize_group<G>(v, packed + g * (G / 2), scales + g);
    }
}

template <int G>
__global__ void k_quantize_q4_min(const float* __restrict__ w, uint64_t n_groups, uint8_t* __restrict__ packed,
                                  uint16_t* __restrict__ scales, uint16_t* __restrict__ mins)
{
    for (uint64_t g = blockIdx.x * (uint64_t)blockDim.x + threadIdx.x; g < n_groups; g += (uint64_t)gridDim.x * blockDim.x) {
        float v[G];
#pragma unroll
        for (int j = 0; j < G; ++j) v[j] = w[g * G + j];
        quantize_group_min<G>(v, packed + g * (G / 2), scales + g, mins + g);
    }
}

// Expert pool: groups are enumerated as (layer, expert, matrix, group); the
// three matrices of a blob hold the same number of groups (D*I/G).  QM: the
// scale+min format, each matrix's mins right after its scales.
template <int G, bool QM>
__global__ void k_synth_pool(uint8_t* base, uint32_t first_layer, uint32_t n_layers, uint32_t n_experts,
                             uint64_t stride, uint64_t groups_per_matrix, uint64_t off0, uint64_t off1,
                             uint64_t off2, uint64_t off3, uint64_t off4, uint64_t off5, uint64_t seed,
                             float stddev)
{
    const uint64_t total = static_cast<uint64_t>(n_layers) * n_experts * 3 * groups_per_matrix;
    for (uint64_t t = blockIdx.x * (uint64_t)blockDim.x + threadIdx.x; t < total; t += (uint64_t)gridDim.x * blockDim.x) {
        const uint64_t g = t % groups_per_matrix;
        const uint64_t rest = t / groups_per_matrix;
        const uint32_t m = static_cast<uint32_t>(rest % 3);
        const uint64_t le = rest / 3;
        const uint32_t e = static_cast<uint32_t>(le % n_experts);
        const uint32_t l = static_cast<uint32_t>(le / n_experts);
        const uint64_t stream = (static_cast<uint64_t>(first_layer + l) << 32) | (static_cast<uint64_t>(e) << 4) | m;
        const uint64_t key = fmix64(seed * GAMMA + fmix64(stream + GAMMA));
        float v[G];
#pragma unroll
        for (int j = 0; j < G; ++j) v[j] = det_normal(key, g * G + j) * stddev;
        uint8_t* blob = base + le * stride;
        const uint64_t po = m == 0 ? off0 : (m == 1 ? off2 : off4);
        const uint64_t so = m == 0 ? off1 : (m == 1 ? off3 : off5);
        uint16_t* sc = reinterpret_cast<uint16_t*>(blob + so) + g;
        if constexpr (QM)
            quantize_group_min<G>(v, blob + po + g * (G / 2), sc, sc + groups_per_matrix);
        else
            quantize_group<G>(v, blob + po + g * (G / 2), sc);
    }
}

static dim3 grid_for(uint64_t n, uint32_t block)
{
    uint64_t b = (n + block - 1) / block;
    if (b > 65536u * 16u) b = 65536u * 16u;
    if (b == 0) b = 1;
    return dim3(static_cast<uint32_t>(b));
}

hipError_t launch_synth_normal(float* out, uint64_t n, uint64_t seed, uint64_t stream, float stddev, hipStream_t s)
{
    hipLaunchKernelGGL(k_synth_normal, grid_for(n, 256), dim3(256), 0, s, out, n, stream_key(seed, stream), stddev);
    return hipGetLastError();
}

hipError_t launch_synth_bf16(uint16_t* out, uint64_t n, uint64_t seed, uint64_t stream, float stddev, hipStream_t s)
{
    hipLaunchKernelGGL(k_synth_bf16, grid_for(n, 256), dim3(256), 0, s, out, n, stream_key(seed, stream), stddev);
    return hipGetLastError();
}

hipError_t launch_quantize_q4(const float* w, uint64_t n, uint32_t group, uint8_t* packed, uint16_t* scales,
                              hipStream_t s)
{
    const uint64_t ng = n / group;
    switch (group) {
        case 32: hipLaunchKernelGGL(k_quantize_q4<32>, grid_for(ng, 128), dim3(128), 0, s, w, ng, packed, scales); break;
        case 64: hipLaunchKernelGGL(k_quantize_q4<64>, grid_for(ng, 128), dim3(128), 0, s, w, ng, packed, scales); break;
        case 128: hipLaunchKernelGGL(k_quantize_q4<128>, grid_for(ng, 128), dim3(128), 0, s, w, ng, packed, scales); break;
        default: return hipErrorInvalidValue;
    }
    return hipGetLastError();
}

hipError_t launch_quantize_q4_min(const float* w, uint64_t n, uint32_t group, uint8_t* packed, uint16_t* scales,
                                  uint16_t* mins, hipStream_t s)
{
    const uint64_t ng = n / group;
    if (group != 64) return hipErrorInvalidValue;
    hipLaunchKernelGGL(k_quantize_q4_min<64>, grid_for(ng, 128), dim3(128), 0, s, w, ng, packed, scales, mins);
    return hipGetLastError();
}

template <int G>
static void synth_pool_g(uint8_t* base, uint32_t first_layer, uint32_t n_layers, uint32_t n_experts, uint64_t stride,
                         uint64_t gpm, const uint64_t* off, uint64_t seed, float stddev, bool qm, hipStream_t s)
{
    const uint64_t total = static_cast<uint64_t>(n_layers) * n_experts * 3 * gpm;
    auto k = qm ? k_synth_pool<G, true> : k_synth_pool<G, false>;
    hipLaunchKernelGGL(k, grid_for(total, 128), dim3(128), 0, s, base, first_layer, n_layers, n_experts, stride, gpm,
                       off[0], off[1], off[2], off[3], off[4], off[5], seed, stddev);
}

hipError_t launch_synth_pool(uint8_t* base, uint32_t first_layer, uint32_t n_layers, uint32_t n_experts,
                             uint64_t stride, uint32_t D, uint32_t I, uint32_t group, const uint64_t* off,
                             uint64_t seed, float stddev, uint32_t quant, hipStream_t s)
{
    const uint64_t gpm = static_cast<uint64_t>(D) * I / group;
    const bool qm = quant == 1;
    switch (group) {
        case 32: synth_pool_g<32>(base, first_layer, n_layers, n_experts, stride, gpm, off, seed, stddev, qm, s); break;
        case 64: synth_pool_g<64>(base, first_layer, n_layers, n_experts, stride, gpm, off, seed, stddev, qm, s); break;
        case 128: synth_pool_g<128>(base, first_layer, n_layers, n_experts, stride, gpm, off, seed, stddev, qm, s); break;
        default: return hipErrorInvalidValue;
    }
    return hipGetLastError();
}

}  // namespace smoe
