// device_common.hpp -- gfx950 device helpers shared by the MoE kernels.
//
// Wave64 reductions on DPP (row-local quad_perm / row_ror steps, then the
// gfx9 row_bcast:15 / row_bcast:31 steps into lane 63), SMOE-Q4 nibble decode,
// number-format conversions and global-address-space streaming loads.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace smoe {

constexpr int WAVE = 64;

// ---- number formats ------------------------------------------------------
__device__ __forceinline__ float bf16_to_f32(uint32_t b16) { return __uint_as_float(b16 << 16); }

__device__ __forceinline__ float f16_bits_to_f32(uint16_t h)
{
    return static_cast<float>(__builtin_bit_cast(_Float16, h));
}

// ---- loads ---------------------------------------------------------------
// Pointers taken from tables in memory are generic; casting them to the global
// address space makes the compiler emit global_load (not flat_load).
template <typename T>
__device__ __forceinline__ const __attribute__((address_space(1))) T* gptr(const T* p)
{
    return (const __attribute__((address_space(1))) T*)(p);
}

// Expert weights are read once per token-layer: non-temporal 128-bit loads so
// they do not evict the activations and h planes held in L2.
__device__ __forceinline__ uint4 load_stream_u4(const void* p)
{
    const __attribute__((address_space(1))) uint32_t* q = gptr(reinterpret_cast<const uint32_t*>(p));
    uint4 r;
    r.x = __builtin_nontemporal_load(q + 0);
    r.y = __builtin_nontemporal_load(q + 1);
    r.z = __builtin_nontemporal_load(q + 2);
    r.w = __builtin_nontemporal_load(q + 3);
    return r;
}

__device__ __forceinline__ uint16_t load_stream_u16(const uint16_t* p)
{
    return __builtin_nontemporal_load(gptr(p));
}

// 16-byte aligned activation / weight loads from the global address space
__device__ __forceinline__ float4 load_f4(const float* p)
{
    const __attribute__((address_space(1))) float* q =
        gptr(static_cast<const float*>(__builtin_assume_aligned(p, 16)));
    return make_float4(q[0], q[1], q[2], q[3]);
}

__device__ __forceinline__ uint4 load_u4(const void* p)
{
    const __attribute__((address_space(1))) uint32_t* q =
        gptr(static_cast<const uint32_t*>(__builtin_assume_aligned(p, 16)));
    return make_uint4(q[0], q[1], q[2], q[3]);
}

// ---- wave64 reductions (DPP) -------------------------------------------------
template <int CTRL, int ROW_MASK = 0xF>
__device__ __forceinline__ uint32_t dpp_u32(uint32_t old, uint32_t v)
{
    return static_cast<uint32_t>(__builtin_amdgcn_update_dpp(static_cast<int>(old), static_cast<int>(v), CTRL,
                                                             ROW_MASK, 0xF, false));
}
template <int CTRL, int ROW_MASK = 0xF>
__device__ __forceinline__ float dpp_f32(float old, float v)
{
    return __uint_as_float(dpp_u32<CTRL, ROW_MASK>(__float_as_uint(old), __float_as_uint(v)));
}

constexpr int DPP_QUAD_XOR1 = 0xB1;   // quad_perm [1,0,3,2]
constexpr int DPP_QUAD_XOR2 = 0x4E;   // quad_perm [2,3,0,1]
constexpr int DPP_ROW_ROR4 = 0x124;
constexpr int DPP_ROW_ROR8 = 0x128;
constexpr int DPP_ROW_BCAST15 = 0x142;
constexpr int DPP_ROW_BCAST31 = 0x143;

__device__ __forceinline__ float readlane_f32(float v, int lane)
{
    return __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), lane));
}
__device__ __forceinline__ uint32_t readlane_u32(uint32_t v, int lane)
{
    return static_cast<uint32_t>(__builtin_amdgcn_readlane(static_cast<int>(v), lane));
}

// Sum over the 64 lanes; the result is wave-uniform.
__device__ __forceinline__ float wave_sum(float v)
{
    v += dpp_f32<DPP_QUAD_XOR1>(0.f, v);
    v += dpp_f32<DPP_QUAD_XOR2>(0.f, v);
    v += dpp_f32<DPP_ROW_ROR4>(0.f, v);
    v += dpp_f32<DPP_ROW_ROR8>(0.f, v);
    v += dpp_f32<DPP_ROW_BCAST15, 0xA>(0.f, v);
    v += dpp_f32<DPP_ROW_BCAST31, 0xC>(0.f, v);
    return readlane_f32(v, 63);
}

__device__ __forceinline__ float wave_max(float v)
{
    v = fmaxf(v, dpp_f32<DPP_QUAD_XOR1>(-INFINITY, v));
    v = fmaxf(v, dpp_f32<DPP_QUAD_XOR2>(-INFINITY, v));
    v = fmaxf(v, dpp_f32<DPP_ROW_ROR4>(-INFINITY, v));
    v = fmaxf(v, dpp_f32<DPP_ROW_ROR8>(-INFINITY, v));
    v = fmaxf(v, dpp_f32<DPP_ROW_BCAST15, 0xA>(-INFINITY, v));
    v = fmaxf(v, dpp_f32<DPP_ROW_BCAST31, 0xC>(-INFINITY, v));
    return readlane_f32(v, 63);
}

__device__ __forceinline__ uint32_t wave_max_u32(uint32_t v)
{
    v = max(v, dpp_u32<DPP_QUAD_XOR1>(0u, v));
    v = max(v, dpp_u32<DPP_QUAD_XOR2>(0u, v));
    v = max(v, dpp_u32<DPP_ROW_ROR4>(0u, v));
    v = max(v, dpp_u32<DPP_ROW_ROR8>(0u, v));
    v = max(v, dpp_u32<DPP_ROW_BCAST15, 0xA>(0u, v));
    v = max(v, dpp_u32<DPP_ROW_BCAST31, 0xC>(0u, v));
    return readlane_u32(v, 63);
}

// ---- SMOE-Q4 16-byte chunk (32 codes, low nibble = even column) -----------
// Returns sum_j code_j * x_j over the 32 columns of the chunk; x holds the
// chunk's 32 activations.  Codes become floats exactly (0..15).
__device__ __forceinline__ float q4_chunk_dot(uint4 v, const float* __restrict__ x)
{
    const uint32_t w[4] = {v.x, v.y, v.z, v.w};
    float a0 = 0.f, a1 = 0.f, a2 = 0.f, a3 = 0.f;
#pragma unroll
    for (int k = 0; k < 4; ++k) {
        const uint32_t lo = w[k] & 0x0F0F0F0Fu;          // codes 0,2,4,6 of this dword
        const uint32_t hi = (w[k] >> 4) & 0x0F0F0F0Fu;   // codes 1,3,5,7
        const float* xk = x + 8 * k;
        a0 = fmaf(static_cast<float>(lo & 0xFFu), xk[0], a0);
        a1 = fmaf(static_cast<float>(hi & 0xFFu), xk[1], a1);
        a2 = fmaf(static_cast<float>((lo >> 8) & 0xFFu), xk[2], a2);
        a3 = fmaf(static_cast<float>((hi >> 8) & 0xFFu), xk[3], a3);
        a0 = fmaf(static_cast<float>((lo >> 16) & 0xFFu), xk[4], a0);
        a1 = fmaf(static_cast<float>((hi >> 16) & 0xFFu), xk[5], a1);
        a2 = fmaf(static_cast<float>(lo >> 24), xk[6], a2);
        a3 = fmaf(static_cast<float>(hi >> 24), xk[7], a3);
    }
    return (a0 + a1) + (a2 + a3);
}

// Per-chunk affine epilogue of the dequant w = (c - 7.5) * (1/7.5) * s:
//   sum_j w_j x_j = s * (sum_j c_j x_j / 7.5 - sum_j x_j)   (kernels.metal:140-145)
__device__ __forceinline__ float q4_chunk_epilogue(float s, float cx, float xsum)
{
    return s * fmaf(cx, 1.0f / 7.5f, -xsum);
}

}  // namespace smoe
