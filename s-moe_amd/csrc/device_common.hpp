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

constexpr int ilog2(int n) { return n <= 1 ? 0 : 1 + ilog2(n / 2); }

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

// ---- transposed reduction of N per-lane values ---------------------------
// Sums value i (i < N, N a power of two <= 16) over the 64 lanes for all i at
// once: each butterfly step over a lane bit halves the values a lane holds
// (lanes with the bit clear keep the lower half of the indices, the others the
// upper half), so N sums cost about N + 6 cross-lane ops instead of 7 N.
// Lane l returns the total of value l >> (6 - log2 N).
//   bit 5: v_permlane32_swap (lanes 32-63 of the first operand <-> lanes 0-31
//          of the second), bit 4: v_permlane16_swap (odd rows of the first
//          operand <-> even rows of the second), bit 3: row_ror:8 (lane ^ 8),
//   bit 2: row_half_mirror (lane -> 7 - lane within 8: flips bit 2; the lower
//          bits are summed over afterwards), bits 1, 0: quad_perm.
constexpr int DPP_ROW_HALF_MIRROR = 0x141;

__device__ __forceinline__ void swap32_sum(float& lo, float hi)
{
    const auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(lo), __float_as_uint(hi), false, false);
    lo = __uint_as_float(r[0]) + __uint_as_float(r[1]);
}
__device__ __forceinline__ void swap16_sum(float& lo, float hi)
{
    const auto r = __builtin_amdgcn_permlane16_swap(__float_as_uint(lo), __float_as_uint(hi), false, false);
    lo = __uint_as_float(r[0]) + __uint_as_float(r[1]);
}
template <int CTRL>
__device__ __forceinline__ void dpp_split_sum(float& lo, float hi, bool upper)
{
    const float keep = upper ? hi : lo;
    const float send = upper ? lo : hi;
    lo = keep + dpp_f32<CTRL>(0.f, send);
}

template <int N>
__device__ __forceinline__ float wave_sum_rows(const float (&v)[N])
{
    static_assert(N == 1 || N == 2 || N == 4 || N == 8 || N == 16, "N must be a power of two <= 16");
    const int lane = threadIdx.x & 63;
    float a[N];
#pragma unroll
    for (int i = 0; i < N; ++i) a[i] = v[i];
    // bit 5
    if constexpr (N >= 2) {
#pragma unroll
        for (int i = 0; i < N / 2; ++i) swap32_sum(a[i], a[i + N / 2]);
    } else {
        swap32_sum(a[0], a[0]);
    }
    // bit 4
    if constexpr (N >= 4) {
#pragma unroll
        for (int i = 0; i < N / 4; ++i) swap16_sum(a[i], a[i + N / 4]);
    } else {
        swap16_sum(a[0], a[0]);
    }
    // bit 3
    if constexpr (N >= 8) {
#pragma unroll
        for (int i = 0; i < N / 8; ++i) dpp_split_sum<DPP_ROW_ROR8>(a[i], a[i + N / 8], lane & 8);
    } else {
        a[0] += dpp_f32<DPP_ROW_ROR8>(0.f, a[0]);
    }
    // bit 2
    if constexpr (N >= 16) {
        dpp_split_sum<DPP_ROW_HALF_MIRROR>(a[0], a[1], lane & 4);
    } else {
        a[0] += dpp_f32<DPP_ROW_HALF_MIRROR>(0.f, a[0]);
    }
    // bits 1, 0
    a[0] += dpp_f32<DPP_QUAD_XOR2>(0.f, a[0]);
    a[0] += dpp_f32<DPP_QUAD_XOR1>(0.f, a[0]);
    return a[0];
}

// ---- segmented transposed reduction ---------------------------------------
// Sums N per-lane values over segments of 2^SEG lanes (the lanes sharing
// l >> SEG), N a power of two with log2 N <= SEG <= 6.  The butterfly runs
// over lane bits SEG-1 .. 0 with the cross-lane steps of wave_sum_rows; the
// first log2 N steps split the values (lanes with the bit clear keep the
// lower half of the indices), the rest are plain sums.  Lane l returns the
// segment total of value (l >> (SEG - log2 N)) & (N - 1).
template <int BIT, bool SPLIT>
__device__ __forceinline__ void red_bit(float& lo, float hi, int lane)
{
    if constexpr (BIT == 5) {
        swap32_sum(lo, SPLIT ? hi : lo);
    } else if constexpr (BIT == 4) {
        swap16_sum(lo, SPLIT ? hi : lo);
    } else {
        constexpr int CTRL = BIT == 3 ? DPP_ROW_ROR8
                           : BIT == 2 ? DPP_ROW_HALF_MIRROR
                           : BIT == 1 ? DPP_QUAD_XOR2
                                      : DPP_QUAD_XOR1;
        if constexpr (SPLIT)
            dpp_split_sum<CTRL>(lo, hi, lane & (1 << BIT));
        else
            lo += dpp_f32<CTRL>(0.f, lo);
    }
}

template <int SEG, int M, int N>
__device__ __forceinline__ void seg_steps(float (&a)[N], int lane)
{
    if constexpr (SEG > 0) {
        if constexpr (M > 1) {
#pragma unroll
            for (int i = 0; i < M / 2; ++i) red_bit<SEG - 1, true>(a[i], a[i + M / 2], lane);
            seg_steps<SEG - 1, M / 2>(a, lane);
        } else {
            red_bit<SEG - 1, false>(a[0], a[0], lane);
            seg_steps<SEG - 1, 1>(a, lane);
        }
    }
}

template <int N, int SEG>
__device__ __forceinline__ float seg_sum_rows(const float (&v)[N])
{
    static_assert((N & (N - 1)) == 0 && ilog2(N) <= SEG && SEG <= 6, "N must be a power of two <= 2^SEG");
    float a[N];
#pragma unroll
    for (int i = 0; i < N; ++i) a[i] = v[i];
    seg_steps<SEG, N>(a, threadIdx.x & 63);
    return a[0];
}

// seg_sum_rows followed by the reverse butterfly: every lane returns all N
// segment totals (out[i] = total of value i over the lane's segment).  The
// gather runs over the split bits from the lowest up; at each bit a lane
// doubles the values it holds with its partner's (the partner differs in that
// bit and, for row_half_mirror, in lower bits whose values agree already).
template <int BIT>
__device__ __forceinline__ void gather_bit(float mine, float& lo, float& hi, int lane)
{
    if constexpr (BIT == 5 || BIT == 4) {
        const auto r = BIT == 5 ? __builtin_amdgcn_permlane32_swap(__float_as_uint(mine), __float_as_uint(mine),
                                                                    false, false)
                                : __builtin_amdgcn_permlane16_swap(__float_as_uint(mine), __float_as_uint(mine),
                                                                    false, false);
        lo = __uint_as_float(r[0]);     // the value of the half with the bit clear
        hi = __uint_as_float(r[1]);
    } else {
        constexpr int CTRL = BIT == 3 ? DPP_ROW_ROR8
                           : BIT == 2 ? DPP_ROW_HALF_MIRROR
                           : BIT == 1 ? DPP_QUAD_XOR2
                                      : DPP_QUAD_XOR1;
        const float other = dpp_f32<CTRL>(0.f, mine);
        const bool upper = lane & (1 << BIT);
        lo = upper ? other : mine;
        hi = upper ? mine : other;
    }
}

template <int SEG, int N, int S = 0>
__device__ __forceinline__ void gather_steps(float (&a)[N], int lane)
{
    constexpr int LOG_N = ilog2(N);
    if constexpr (S < LOG_N) {
        constexpr int C = 1 << S;       // values held before this step
        float t[2 * C];
#pragma unroll
        for (int k = 0; k < C; ++k) gather_bit<SEG - LOG_N + S>(a[k], t[k], t[C + k], lane);
#pragma unroll
        for (int k = 0; k < 2 * C; ++k) a[k] = t[k];
        gather_steps<SEG, N, S + 1>(a, lane);
    }
}

template <int N, int SEG>
__device__ __forceinline__ void seg_allsum(float (&v)[N])
{
    const int lane = threadIdx.x & 63;
    seg_steps<SEG, N>(v, lane);
    gather_steps<SEG, N>(v, lane);
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

// Maximum over the 64 lanes, left in every lane (no readlane): rows by DPP,
// then rows and halves by v_permlane16_swap / v_permlane32_swap, each of
// which hands both sides of the exchange to every lane.
__device__ __forceinline__ uint32_t wave_max_u32_all(uint32_t v)
{
    v = max(v, dpp_u32<DPP_QUAD_XOR1>(0u, v));
    v = max(v, dpp_u32<DPP_QUAD_XOR2>(0u, v));
    v = max(v, dpp_u32<DPP_ROW_ROR4>(0u, v));
    v = max(v, dpp_u32<DPP_ROW_ROR8>(0u, v));
    const auto a = __builtin_amdgcn_permlane16_swap(v, v, false, false);
    v = max(a[0], a[1]);
    const auto b = __builtin_amdgcn_permlane32_swap(v, v, false, false);
    return max(b[0], b[1]);
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

// ---------------------------------------------------------------------------
// Integer form of a 32-value activation chunk for 4-bit dot products.
// The chunk is scaled by 2^sh (sh = 22 - exponent of its absmax) and rounded
// to integers t_k, |t_k| <= 2^22; each t_k is written in six balanced hex
// digits d_l in [-8, 7] (t = sum_l 16^l d_l), stored as two's-complement
// nibbles in the weights' nibble order (nibble k of dword w = element 8w+k).
// Then sum_k (c_k - 8) t_k = sum_l 16^l sum_k (c_k - 8) d_lk is 6 v_dot8 per
// dword of codes, exact in int32 (|sum| <= 32 * 8 * 2^22 = 2^30), and
//   sum_k (c_k - 7.5) a_k / 7.5 = (sum_k (c_k - 8) t_k + X / 2) * 2^-sh / 7.5
// with X = sum_k t_k.  The rounding of a_k to t_k is at most 2^-22 of the
// chunk's absmax, the level of fp32 accumulation error.
// ---------------------------------------------------------------------------
constexpr int Q4_DIGITS = 6;

struct Q4Act {
    uint32_t dig[Q4_DIGITS][4];   // [digit l][dword w]
    float xsum_half;              // X / 2
    float kscale;                 // 2^-sh / 7.5
    float pscale;                 // 2^-sh
};

__device__ __forceinline__ void q4_act_from_floats(const float (&a)[32], Q4Act& q)
{
    float amax = 0.f;
#pragma unroll
    for (int k = 0; k < 32; ++k) amax = fmaxf(amax, fabsf(a[k]));
    // amax < 2^e  ->  |a * 2^(22-e)| < 2^22
    const int e = amax > 0.f ? __builtin_amdgcn_frexp_expf(amax) : 0;
    const int sh = 22 - e;
    // v = a * 2^sh + 1.5 * 2^23 lies in [2^23, 2^24] with spacing 1, so the
    // add rounds to nearest-even integer and bits(v) - bits(1.5 * 2^23) = t;
    // u = t + B with B = 0x888888 has the unsigned digits d_l + 8 and
    // u ^ B their two's-complement nibbles
    constexpr float kMagic = 12582912.0f;               // 1.5 * 2^23, bits 0x4B400000
    constexpr uint32_t kB = 0x888888u;
    uint32_t y[32];
    uint32_t usum = 0;
#pragma unroll
    for (int k = 0; k < 32; ++k) {
        const float v = __builtin_ldexpf(a[k], sh) + kMagic;
        const uint32_t u = __float_as_uint(v) + (kB - 0x4B400000u);
        usum += u;
        y[k] = u ^ kB;
    }
    q.xsum_half = 0.5f * static_cast<float>(static_cast<int>(usum - 32u * kB));
    q.kscale = __builtin_ldexpf(1.0f / 7.5f, -sh);
    q.pscale = __builtin_ldexpf(1.0f, -sh);
#pragma unroll
    for (int w = 0; w < 4; ++w) {
        const uint32_t* t = y + 8 * w;
        // byte b of the even (odd) elements of this dword, in element order
        const uint32_t ea = __builtin_amdgcn_perm(t[2], t[0], 0x05010400u);   // t0.0 t2.0 t0.1 t2.1
        const uint32_t eb = __builtin_amdgcn_perm(t[6], t[4], 0x05010400u);   // t4.0 t6.0 t4.1 t6.1
        const uint32_t ec = __builtin_amdgcn_perm(t[2], t[0], 0x0C0C0602u);   // t0.2 t2.2
        const uint32_t ed = __builtin_amdgcn_perm(t[6], t[4], 0x0C0C0602u);   // t4.2 t6.2
        const uint32_t oa = __builtin_amdgcn_perm(t[3], t[1], 0x05010400u);
        const uint32_t ob = __builtin_amdgcn_perm(t[7], t[5], 0x05010400u);
        const uint32_t oc = __builtin_amdgcn_perm(t[3], t[1], 0x0C0C0602u);
        const uint32_t od = __builtin_amdgcn_perm(t[7], t[5], 0x0C0C0602u);
        const uint32_t E[3] = {__builtin_amdgcn_perm(eb, ea, 0x05040100u), __builtin_amdgcn_perm(eb, ea, 0x07060302u),
                               __builtin_amdgcn_perm(ed, ec, 0x05040100u)};
        const uint32_t O[3] = {__builtin_amdgcn_perm(ob, oa, 0x05040100u), __builtin_amdgcn_perm(ob, oa, 0x07060302u),
                               __builtin_amdgcn_perm(od, oc, 0x05040100u)};
#pragma unroll
        for (int b = 0; b < 3; ++b) {
            q.dig[2 * b][w] = (E[b] & 0x0F0F0F0Fu) | ((O[b] << 4) & 0xF0F0F0F0u);
            q.dig[2 * b + 1][w] = ((E[b] >> 4) & 0x0F0F0F0Fu) | (O[b] & 0xF0F0F0F0u);
        }
    }
}

// sum_k (c_k - 8) t_k over one 16-byte chunk of codes, exact
__device__ __forceinline__ int q4_chunk_int(uint4 v, const Q4Act& q)
{
    // c ^ 8 per nibble is c - 8 as a two's-complement nibble
    const uint32_t c[4] = {v.x ^ 0x88888888u, v.y ^ 0x88888888u, v.z ^ 0x88888888u, v.w ^ 0x88888888u};
    int s[Q4_DIGITS];
#pragma unroll
    for (int l = 0; l < Q4_DIGITS; ++l) {
        s[l] = 0;
#pragma unroll
        for (int w = 0; w < 4; ++w)
            s[l] = __builtin_amdgcn_sdot8(static_cast<int>(c[w]), static_cast<int>(q.dig[l][w]), s[l], false);
    }
    uint32_t acc = static_cast<uint32_t>(s[Q4_DIGITS - 1]);
#pragma unroll
    for (int l = Q4_DIGITS - 2; l >= 0; --l) acc = acc * 16u + static_cast<uint32_t>(s[l]);
    return static_cast<int>(acc);
}

// sum_k (c_k - 7.5) a_k / 7.5 over one 16-byte chunk of codes (before the
// group scale)
__device__ __forceinline__ float q4_chunk_dot8(uint4 v, const Q4Act& q)
{
    return (static_cast<float>(q4_chunk_int(v, q)) + q.xsum_half) * q.kscale;
}

// sum_k (c_k s + m) a_k over one chunk of the scale+min format (scale s and
// min m of the chunk's group): c s + m = (c - 8) s + (m + 8 s), so the
// exact integer sum_k (c_k - 8) t_k and X = sum_k t_k carry it without
// cancelling the min against the codes
__device__ __forceinline__ float q4_chunk_affine(uint4 v, const Q4Act& q, float s, float m)
{
    const float b = fmaf(8.0f, s, m);
    return fmaf(s, static_cast<float>(q4_chunk_int(v, q)), b * (2.0f * q.xsum_half)) * q.pscale;
}

// Per-chunk affine epilogue of the dequant w = (c - 7.5) * (1/7.5) * s:
//   sum_j w_j x_j = s * (sum_j c_j x_j / 7.5 - sum_j x_j)   (kernels.metal:140-145)
__device__ __forceinline__ float q4_chunk_epilogue(float s, float cx, float xsum)
{
    return s * fmaf(cx, 1.0f / 7.5f, -xsum);
}

}  // namespace smoe
