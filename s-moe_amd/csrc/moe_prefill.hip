// moe_prefill.hip -- prefill MoE block over T token rows on gfx950.
//
// The reference runs prefill layer-major in chunks of 64 tokens
// (prefill.cpp:308-453): per token RMSNorm + router + top-k (:319-332), the
// per-expert token lists built by union_add (:38-68), one batched FFN per
// touched expert (metal_bridge.mm:544-645) and a weighted scatter into
// routed_out (:380-385) that is added to hidden (:446-451).  Here the whole
// batch of tokens is one pass (tokens are independent, so the grouping only
// changes fp32 summation order):
//
//   k_route        RMSNorm + fp32 router + exact top-k for TB tokens per
//                  block; writes the normed rows as the GEMM's f16 planes
//                  (the split below) and ids/weights.
//   k_split_rows   per row: power-of-two scale 2^e with |x| < 2^e and the
//                  f16 hi/lo planes of x * 2^-e (hi + lo carries 22 bits),
//                  columns of every 8 in the order 0 2 4 6 1 3 5 7.
//   k_permute      stable counting sort of the T*k (token, rank) pairs by
//                  expert (one workgroup), union order by first appearance.
//   k_grouped_mm   per expert: [pairs x K] x [K x rows] tiles (128 gate +
//                  128 up rows, or 256 down rows, per block) on MFMA
//                  v_mfma_f32_16x16x32_f16, weights and activation rows
//                  streamed through LDS rings.  Weights enter exactly as
//                  (2c - 15)/8 (f16), activations as hi and lo planes (two
//                  MFMAs into one fp32 accumulator); each 64-column group adds
//                  s_g * sum, the row scale 8 * 2^e / 15 closes the dot
//                  (kernels.metal:90-105, 140-145).  Gate+up runs with SiLU
//                  and writes h per (token, rank) pair; down writes y per pair.
//   k_combine_pairs hidden[t] += sum_r w[t][r] * y[t*k + r] in rank order.
//
// Blocks of one expert are mapped to one XCD (block id mod 8), so its token
// rows stay in that XCD's L2 while the expert's weights stream once.
#include <algorithm>
#include <type_traits>

#include "device_common.hpp"
#include "kernels.hpp"
#include "topk.hpp"

namespace smoe {

typedef _Float16 half8_t __attribute__((ext_vector_type(8)));
typedef float f32x4_t __attribute__((ext_vector_type(4)));
typedef uint32_t u32x4_t __attribute__((ext_vector_type(4)));
typedef uint32_t u32x2_t __attribute__((ext_vector_type(2)));

// ---------------------------------------------------------------------------
// 8 consecutive columns x[0..7] of a row with |x| < 2^e -> f16 planes hi, lo of
// x * 2^-e (hi + lo carries 22 bits), in the column order 0 2 4 6 1 3 5 7 in
// which q4_codes_to_f16 unpacks a word of codes.
// ---------------------------------------------------------------------------
__device__ __forceinline__ void split8_f16(const float* x, int e, uint4& hi, uint4& lo)
{
    const float xs[8] = {x[0], x[2], x[4], x[6], x[1], x[3], x[5], x[7]};
    uint32_t h2[4], l2[4];
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        uint32_t hb[2], lb[2];
#pragma unroll
        for (int u = 0; u < 2; ++u) {
            const float xv = __builtin_ldexpf(xs[2 * i + u], -e);
            const _Float16 h = static_cast<_Float16>(xv);
            hb[u] = __builtin_bit_cast(uint16_t, h);
            lb[u] = __builtin_bit_cast(uint16_t, static_cast<_Float16>(xv - static_cast<float>(h)));
        }
        h2[i] = hb[0] | (hb[1] << 16);
        l2[i] = lb[0] | (lb[1] << 16);
    }
    hi = make_uint4(h2[0], h2[1], h2[2], h2[3]);
    lo = make_uint4(l2[0], l2[1], l2[2], l2[3]);
}

// ---------------------------------------------------------------------------
// k_route: RMSNorm (common.hpp:245-256) + router (common.hpp:293-306) +
// softmax/top-k (scout.cpp:77-123) for TB tokens per block of ROUTE_WAVES
// waves.  Every wave normalises all TB tokens (lane l owns the 32-column
// chunks l + 64 j) and computes router rows w, w + ROUTE_WAVES, ... for all of
// them; wave t then selects the experts of token t, and (in the group's
// first block) writes token t's normed row as the GEMM's f16 planes.  With
// ES > 1 (short batches) the E router rows of a token group are split over
// ES blocks, so each wave has few rows and all their loads in flight at once:
// the blocks write their logits with agent-scope stores, wait for them, and
// add themselves to a device-scope counter per token group; the block that
// finds the count at ES - 1 modulo ES runs the group's top-k on agent-scope
// loads of the logits (no device-wide fence anywhere).  Where the registers
// allow (HAND below), wave t alone reads and normalises token t and hands it
// to the other waves through LDS, and every wave requests its first router
// rows before that, so the hidden rows' and the router rows' round trips
// overlap (same bits; 64 tokens of the 235B shape 16.1 -> 13.3 us, 512 of the
// 30B shape 20.3 -> 18.1 us).
// ---------------------------------------------------------------------------
constexpr int ROUTE_WAVES = 8;

template <int CPL, int TB, int VPL, int ES>
__global__ __launch_bounds__(ROUTE_WAVES * WAVE)
void k_route(MoeDims d, LayerDesc L, const float* __restrict__ hidden, uint32_t T, uint16_t* __restrict__ x_hi,
             uint16_t* __restrict__ x_lo, float* __restrict__ x_sc, uint32_t* __restrict__ ids,
             float* __restrict__ w, float* __restrict__ logits, uint32_t* __restrict__ counters)
{
    // router rows per reduction batch (RPB * TB values); with ES > 1 a wave
    // has at most 4 rows (E <= 128 at ES = 4)
    constexpr int RPB = ES > 1 ? 4 : 16 / TB;
    // the counters advance by ES per launch and token group, and one array
    // serves every launch: a single split factor keeps their residues aligned
    static_assert(ES == 1 || ES == 4, "one split factor for the route counters");
    __shared__ float s_logit[TB][SMOE_TOPK_MAX_N];
    __shared__ uint2 s_slots[TB][TOPK_SLOTS];
    __shared__ uint32_t s_last;
    const int lane = threadIdx.x & 63, wv = threadIdx.x >> 6;
    const uint32_t g = blockIdx.x / ES, eg = blockIdx.x % ES;
    const uint32_t t0 = g * TB;
    const uint32_t rows_per = (d.E + ES - 1) / ES, rbeg = eg * rows_per, rend = min(d.E, rbeg + rows_per);
    const uint32_t D = d.D, nch = D >> 5;

    // router rows per load group (see below)
    constexpr int RG_FIT = (208 - 32 * TB * CPL) / (16 * CPL);
    constexpr int RG_ALL = RG_FIT >= RPB ? RPB : RG_FIT >= 8 ? 8 : RG_FIT >= 4 ? 4 : RG_FIT >= 2 ? 2 : 1;
    // HAND: waves 0 .. TB - 1 normalise the tokens and hand them over through
    // LDS while every wave requests its first group of router rows (where that
    // fits the registers without spills: one chunk a lane, or one token at two;
    // E <= 128)
    constexpr bool HAND = ES > 1 || (VPL == 2 && (CPL == 1 || (CPL == 2 && TB == 1)));
    // (two rows a group where a wave's hidden chunks are live beside them)
    constexpr int RG = HAND && CPL > 1 && RG_ALL > 2 ? 2 : RG_ALL;
    static_assert(RPB % RG == 0, "row groups of a batch");
    const uint32_t rfirst = rbeg + wv * RPB;
    uint4 rws[RG][CPL][4];
    float a[TB][CPL][32];
    if constexpr (HAND) {
        // wave t < TB normalises token t (and, in the token group's first
        // block, writes its f16 planes) and hands it to the other waves
        // through LDS; every wave requests its router rows before that, so the
        // round trips overlap and each token is normalised once, not by every wave
        __shared__ __align__(16) float4 s_a[TB][CPL][8][WAVE];
        float4 x[CPL][8];
        uint4 gw[CPL][4];
        if (wv < TB) {
            const float* hv = hidden + static_cast<size_t>(min(t0 + wv, T - 1)) * D;
#pragma unroll
            for (int j = 0; j < CPL; ++j) {
                const uint32_t c = min(lane + WAVE * j, nch - 1);
#pragma unroll
                for (int q = 0; q < 8; ++q) x[j][q] = load_f4(hv + c * 32 + q * 4);
#pragma unroll
                for (int q = 0; q < 4; ++q) gw[j][q] = load_u4(L.norm_w + c * 32 + q * 8);
            }
        }
        if (rfirst < rend) {
#pragma unroll
            for (int ii = 0; ii < RG; ++ii) {
                const uint16_t* wr = L.router_w + static_cast<size_t>(min(rfirst + ii, rend - 1)) * D;
#pragma unroll
                for (int j = 0; j < CPL; ++j) {
                    const uint32_t c = min(lane + WAVE * j, nch - 1);
#pragma unroll
                    for (int q = 0; q < 4; ++q) rws[ii][j][q] = load_u4(wr + c * 32 + q * 8);
                }
            }
        }
        if (wv < TB) {
            float ss = 0.f;
#pragma unroll
            for (int j = 0; j < CPL; ++j) {
                const bool ok = lane + WAVE * j < nch;
#pragma unroll
                for (int q = 0; q < 8; ++q) {
                    if (!ok) x[j][q] = make_float4(0.f, 0.f, 0.f, 0.f);
                    ss = fmaf(x[j][q].x, x[j][q].x, ss);
                    ss = fmaf(x[j][q].y, x[j][q].y, ss);
                    ss = fmaf(x[j][q].z, x[j][q].z, ss);
                    ss = fmaf(x[j][q].w, x[j][q].w, ss);
                }
            }
            ss = wave_sum(ss);
            const float inv = 1.0f / sqrtf(ss / static_cast<float>(D) + 1e-6f);
#pragma unroll
            for (int j = 0; j < CPL; ++j) {
#pragma unroll
                for (int q = 0; q < 8; ++q) {
                    const uint32_t g0 = (q & 1) ? gw[j][q >> 1].z : gw[j][q >> 1].x;
                    const uint32_t g1 = (q & 1) ? gw[j][q >> 1].w : gw[j][q >> 1].y;
                    a[0][j][4 * q + 0] = (x[j][q].x * inv) * bf16_to_f32(g0 & 0xFFFFu);
                    a[0][j][4 * q + 1] = (x[j][q].y * inv) * bf16_to_f32(g0 >> 16);
                    a[0][j][4 * q + 2] = (x[j][q].z * inv) * bf16_to_f32(g1 & 0xFFFFu);
                    a[0][j][4 * q + 3] = (x[j][q].w * inv) * bf16_to_f32(g1 >> 16);
                }
#pragma unroll
                for (int q = 0; q < 8; ++q)
                    s_a[wv][j][q][lane] = make_float4(a[0][j][4 * q], a[0][j][4 * q + 1], a[0][j][4 * q + 2],
                                                      a[0][j][4 * q + 3]);
            }
            if (eg == 0 && t0 + wv < T) {
                float amax = 0.f;
#pragma unroll
                for (int j = 0; j < CPL; ++j)
                    if (lane + WAVE * j < nch) {
#pragma unroll
                        for (int k = 0; k < 32; ++k) amax = fmaxf(amax, fabsf(a[0][j][k]));
                    }
                amax = wave_max(amax);
                const int e = amax > 0.f ? __builtin_amdgcn_frexp_expf(amax) : 0;
                const size_t row = static_cast<size_t>(t0 + wv) * D;
#pragma unroll
                for (int j = 0; j < CPL; ++j) {
                    if (lane + WAVE * j >= nch) continue;
#pragma unroll
                    for (int b = 0; b < 4; ++b) {
                        const size_t o = row + (lane + WAVE * j) * 32 + 8 * b;
                        uint4 hv4, lv4;
                        split8_f16(&a[0][j][8 * b], e, hv4, lv4);
                        *reinterpret_cast<uint4*>(x_hi + o) = hv4;
                        *reinterpret_cast<uint4*>(x_lo + o) = lv4;
                    }
                }
                if (lane == 0) x_sc[t0 + wv] = __builtin_ldexpf(1.0f, e);
            }
        }
        __syncthreads();
#pragma unroll
        for (int t = 0; t < TB; ++t)
#pragma unroll
            for (int j = 0; j < CPL; ++j)
#pragma unroll
                for (int q = 0; q < 8; ++q) {
                    const float4 v = s_a[t][j][q][lane];
                    a[t][j][4 * q] = v.x;
                    a[t][j][4 * q + 1] = v.y;
                    a[t][j][4 * q + 2] = v.z;
                    a[t][j][4 * q + 3] = v.w;
                }
    } else
#pragma unroll
    for (int t = 0; t < TB; ++t) {
        const float* hv = hidden + static_cast<size_t>(min(t0 + t, T - 1)) * D;

        float4 x[CPL][8];
        uint4 g[CPL][4];
#pragma unroll
        for (int j = 0; j < CPL; ++j) {
            const uint32_t c = min(lane + WAVE * j, nch - 1);
#pragma unroll
            for (int q = 0; q < 8; ++q) x[j][q] = load_f4(hv + c * 32 + q * 4);
#pragma unroll
            for (int q = 0; q < 4; ++q) g[j][q] = load_u4(L.norm_w + c * 32 + q * 8);
        }
        float ss = 0.f;
#pragma unroll
        for (int j = 0; j < CPL; ++j) {
            const bool ok = lane + WAVE * j < nch;
#pragma unroll
            for (int q = 0; q < 8; ++q) {
                if (!ok) x[j][q] = make_float4(0.f, 0.f, 0.f, 0.f);
                ss = fmaf(x[j][q].x, x[j][q].x, ss);
                ss = fmaf(x[j][q].y, x[j][q].y, ss);
                ss = fmaf(x[j][q].z, x[j][q].z, ss);
                ss = fmaf(x[j][q].w, x[j][q].w, ss);
            }
        }
        ss = wave_sum(ss);
        const float inv = 1.0f / sqrtf(ss / static_cast<float>(D) + 1e-6f);
#pragma unroll
        for (int j = 0; j < CPL; ++j) {
#pragma unroll
            for (int q = 0; q < 8; ++q) {
                const uint32_t g0 = (q & 1) ? g[j][q >> 1].z : g[j][q >> 1].x;
                const uint32_t g1 = (q & 1) ? g[j][q >> 1].w : g[j][q >> 1].y;
                a[t][j][4 * q + 0] = (x[j][q].x * inv) * bf16_to_f32(g0 & 0xFFFFu);
                a[t][j][4 * q + 1] = (x[j][q].y * inv) * bf16_to_f32(g0 >> 16);
                a[t][j][4 * q + 2] = (x[j][q].z * inv) * bf16_to_f32(g1 & 0xFFFFu);
                a[t][j][4 * q + 3] = (x[j][q].w * inv) * bf16_to_f32(g1 >> 16);
            }
        }
        // wave t of the group's first block writes token t's normed row as the
        // grouped GEMM's f16 planes (the split of k_split_rows, same values)
        if (wv == t && eg == 0 && t0 + t < T) {
            float amax = 0.f;
#pragma unroll
            for (int j = 0; j < CPL; ++j)
                if (lane + WAVE * j < nch) {
#pragma unroll
                    for (int k = 0; k < 32; ++k) amax = fmaxf(amax, fabsf(a[t][j][k]));
                }
            amax = wave_max(amax);
            const int e = amax > 0.f ? __builtin_amdgcn_frexp_expf(amax) : 0;
            const size_t row = static_cast<size_t>(t0 + t) * D;
#pragma unroll
            for (int j = 0; j < CPL; ++j) {
                if (lane + WAVE * j >= nch) continue;
#pragma unroll
                for (int b = 0; b < 4; ++b) {
                    const size_t o = row + (lane + WAVE * j) * 32 + 8 * b;
                    uint4 hv, lv;
                    split8_f16(&a[t][j][8 * b], e, hv, lv);
                    *reinterpret_cast<uint4*>(x_hi + o) = hv;
                    *reinterpret_cast<uint4*>(x_lo + o) = lv;
                }
            }
            if (lane == 0) x_sc[t0 + t] = __builtin_ldexpf(1.0f, e);
        }
    }
    // router rows of this wave, RPB at a time; lane l ends up with value
    // l >> VSH of the batch (value v = row_i * TB + t)
    // The rows are requested RG at a time before any of them is used, so their
    // loads are in flight together (row by row, the compiler waited out one L2
    // round trip per row: 21.4 us for the route at 512 tokens of the 30B
    // shape).  RG: as many rows as fit beside the normed activations
    // (TB * CPL * 32 values) in about 208 VGPRs, 16 CPL registers a row.
    // With ES > 1 the first group was requested before the norm (above).
    for (uint32_t r0 = rfirst; r0 < rend; r0 += ROUTE_WAVES * RPB) {
        float part[RPB * TB];
#pragma unroll
        for (int i = 0; i < RPB; ++i) {
            if (i % RG == 0 && (!HAND || i > 0 || r0 != rfirst)) {
#pragma unroll
                for (int ii = 0; ii < RG; ++ii) {
                    const uint16_t* wr = L.router_w + static_cast<size_t>(min(r0 + i + ii, rend - 1)) * D;
#pragma unroll
                    for (int j = 0; j < CPL; ++j) {
                        const uint32_t c = min(lane + WAVE * j, nch - 1);
#pragma unroll
                        for (int q = 0; q < 4; ++q) rws[ii][j][q] = load_u4(wr + c * 32 + q * 8);
                    }
                }
            }
            const uint4 (&rw)[CPL][4] = rws[i % RG];
#pragma unroll
            for (int t = 0; t < TB; ++t) {
                float acc = 0.f;
#pragma unroll
                for (int j = 0; j < CPL; ++j) {
#pragma unroll
                    for (int q = 0; q < 4; ++q) {
                        const uint32_t w4[4] = {rw[j][q].x, rw[j][q].y, rw[j][q].z, rw[j][q].w};
#pragma unroll
                        for (int u = 0; u < 4; ++u) {
                            acc = fmaf(bf16_to_f32(w4[u] & 0xFFFFu), a[t][j][8 * q + 2 * u], acc);
                            acc = fmaf(bf16_to_f32(w4[u] >> 16), a[t][j][8 * q + 2 * u + 1], acc);
                        }
                    }
                }
                part[i * TB + t] = acc;
            }
        }
        const float tot = wave_sum_rows<RPB * TB>(part);
        constexpr int VSH = 6 - ilog2(RPB * TB);   // lane l holds the total of value l >> VSH
        const uint32_t v = lane >> VSH;
        const uint32_t row = r0 + v / TB;
        if ((lane & ((1 << VSH) - 1)) == 0 && row < rend && row < r0 + RPB) {
            if (ES == 1) s_logit[v % TB][row] = tot;
            else if (t0 + v % TB < T)   // written through to the agent's coherence point
                __hip_atomic_store(&logits[static_cast<size_t>(t0 + v % TB) * d.E + row], tot, __ATOMIC_RELAXED,
                                   __HIP_MEMORY_SCOPE_AGENT);
        }
    }
    if (ES > 1) {
        // every wave's agent-scope stores complete before the block counts
        // itself (no device-wide fence: that writes back and invalidates the
        // whole L2 of the XCD)
        asm volatile("" ::: "memory");
        __builtin_amdgcn_s_waitcnt(0x0F70);   // vmcnt(0)
        asm volatile("" ::: "memory");
        __syncthreads();
        // the count is kept modulo ES (ES divides 2^32): no reset between launches
        if (threadIdx.x == 0) s_last = atomicAdd(&counters[g], 1u) % ES == ES - 1;
        __syncthreads();
        if (!s_last) return;
    } else {
        __syncthreads();
    }
    if (wv < TB && t0 + wv < T) {
        float p[VPL];
#pragma unroll
        for (int j = 0; j < VPL; ++j) {
            const uint32_t pos = lane + WAVE * j;
            p[j] = pos >= d.E ? -INFINITY
                   : ES == 1  ? s_logit[wv][pos]
                              : __hip_atomic_load(&logits[static_cast<size_t>(t0 + wv) * d.E + pos],
                                                  __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        }
        uint32_t my_id;
        float my_w;
        const uint32_t count = topk_latency<VPL>(p, d.E, d.K, d.norm_topk, my_id, my_w, s_slots[wv]);
        if (static_cast<uint32_t>(lane) < count) {
            ids[static_cast<size_t>(t0 + wv) * d.K + lane] = my_id;
            w[static_cast<size_t>(t0 + wv) * d.K + lane] = my_w;
        }
    }
}

// ---------------------------------------------------------------------------
// k_split_rows: src [rows x cols] fp32 -> f16 planes hi/lo of x * 2^-e with
// |x| < 2^e over the row, and scale[row] = 2^e.  hi + lo carries 22 bits of
// x * 2^-e (f16 subnormals below 2^-14 still hold x to 2^-25 of the row max).
// Within every 8 columns the planes hold the columns in the order
// 0 2 4 6 1 3 5 7, the order in which q4_codes_to_f16 unpacks a word of
// codes (the even codes, then the odd ones).  One wave per row, 8 columns
// per lane; rows of 1025 to 2048 columns are read once (kept in registers
// between the maximum and the split).
// ---------------------------------------------------------------------------
__global__ __launch_bounds__(256)
void k_split_rows(const float* __restrict__ src, uint32_t rows, uint32_t cols, uint16_t* __restrict__ hi,
                  uint16_t* __restrict__ lo, float* __restrict__ scale)
{
    const int lane = threadIdx.x & 63;
    for (uint32_t r = blockIdx.x * 4 + (threadIdx.x >> 6); r < rows; r += gridDim.x * 4) {
        const float* x = src + static_cast<size_t>(r) * cols;
        float amax = 0.f;
        if (cols > 2 * WAVE * 8 && cols <= 4 * WAVE * 8) {
            // the row's 8-column pieces of this lane stay in registers: one read of the row
            // (at 1536 columns 4.5 against 5.9 us for 512 rows; at 768 the second read is
            // cheaper than the half-line loads of this mapping, 5.8 against 6.1 us)
            float4 v[4][2];
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                const uint32_t c = lane * 8 + WAVE * 8 * i;
                if (c < cols) {
                    v[i][0] = load_f4(x + c);
                    v[i][1] = load_f4(x + c + 4);
                    const float4 a = v[i][0], b = v[i][1];
                    amax = fmaxf(amax, fmaxf(fmaxf(fmaxf(fabsf(a.x), fabsf(a.y)), fmaxf(fabsf(a.z), fabsf(a.w))),
                                             fmaxf(fmaxf(fabsf(b.x), fabsf(b.y)), fmaxf(fabsf(b.z), fabsf(b.w)))));
                }
            }
            amax = wave_max(amax);
            const int e = amax > 0.f ? __builtin_amdgcn_frexp_expf(amax) : 0;
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                const uint32_t c = lane * 8 + WAVE * 8 * i;
                if (c < cols) {
                    const float xv[8] = {v[i][0].x, v[i][0].y, v[i][0].z, v[i][0].w,
                                         v[i][1].x, v[i][1].y, v[i][1].z, v[i][1].w};
                    uint4 hv, lv;
                    split8_f16(xv, e, hv, lv);
                    const size_t o = static_cast<size_t>(r) * cols + c;
                    *reinterpret_cast<uint4*>(hi + o) = hv;
                    *reinterpret_cast<uint4*>(lo + o) = lv;
                }
            }
            if (lane == 0) scale[r] = __builtin_ldexpf(1.0f, e);
            continue;
        }
        for (uint32_t c = lane * 4; c < cols; c += WAVE * 4) {
            const float4 v = load_f4(x + c);
            amax = fmaxf(amax, fmaxf(fmaxf(fabsf(v.x), fabsf(v.y)), fmaxf(fabsf(v.z), fabsf(v.w))));
        }
        amax = wave_max(amax);
        const int e = amax > 0.f ? __builtin_amdgcn_frexp_expf(amax) : 0;
        for (uint32_t c = lane * 8; c < cols; c += WAVE * 8) {
            const float4 v0 = load_f4(x + c), v1 = load_f4(x + c + 4);
            const float xv[8] = {v0.x, v0.y, v0.z, v0.w, v1.x, v1.y, v1.z, v1.w};
            uint4 hv, lv;
            split8_f16(xv, e, hv, lv);
            const size_t o = static_cast<size_t>(r) * cols + c;
            *reinterpret_cast<uint4*>(hi + o) = hv;
            *reinterpret_cast<uint4*>(lo + o) = lv;
        }
        if (lane == 0) scale[r] = __builtin_ldexpf(1.0f, e);
    }
}

// ---------------------------------------------------------------------------
// k_permute: stable counting sort of the P = T*k pairs p = t*k + r by expert
// ids[p] (prefill.cpp:38-68 builds the same per-expert lists, ascending token
// order), in one workgroup.  Chunk c = pairs [64c, 64c + 64) is one wave's
// step: per-(expert, chunk) counts in LDS, prefix over (expert, chunk), then
// each pair's slot = prefix + its rank among equal ids earlier in the chunk.
// The count table is [expert][chunk] with an odd row stride, so the threads
// that scan one expert's chunks read different banks (the [chunk][expert]
// table put them all in one: 14.2 -> 11.6 us at 512 tokens of the 30B shape).
// Union order (first appearance, token-major, prefill.cpp:55-68) ranks the
// touched experts by their first pair.  ids >= E are skipped and flagged in
// err (bit 1).  sched (optional, [E + 1]) receives the grouped GEMMs' work
// order: sched[0] = number of touched experts, then the touched experts by
// decreasing cost (gm_cost of their pair count), ties by expert id, ranked by
// one key per expert computed with its total.
// ---------------------------------------------------------------------------
constexpr int PERM_THREADS = 1024;

// relative cost of one (expert, row tile) block of the grouped GEMMs with M
// pairs: a fixed share per pass of up to 64 pairs plus one per 16-pair m-tile
__device__ __forceinline__ uint32_t gm_cost(uint32_t M) { return 2u * ((M + 63u) >> 6) + ((M + 15u) >> 4); }

__global__ __launch_bounds__(PERM_THREADS)
void k_permute(const uint32_t* __restrict__ ids, const float* __restrict__ w, uint32_t P, uint32_t K, uint32_t E,
               uint32_t* __restrict__ offsets, uint32_t* __restrict__ sorted_pairs,
               uint32_t* __restrict__ sorted_tokens, float* __restrict__ sorted_w, uint32_t* __restrict__ union_ids,
               uint32_t* __restrict__ union_size, uint32_t* __restrict__ sched, uint32_t* __restrict__ err)
{
    extern __shared__ uint32_t s_mem[];
    // the count table is [E][C | 1]: the odd row stride puts a chunk's experts,
    // and the chunks one expert's threads read, in different banks
    const uint32_t C = (P + 63) / 64, CS = C | 1u;
    uint32_t* s_cnt = s_mem;               // [E x CS]
    uint32_t* s_first = s_cnt + CS * E;    // [E]
    uint32_t* s_tot = s_first + E;         // [E]
    uint32_t* s_off = s_tot + E;           // [E + 1]
    uint32_t* s_key = s_off + E + 1;       // [E] work-order keys
    const int lane = threadIdx.x & 63, wv = threadIdx.x >> 6;
    constexpr int NW = PERM_THREADS / WAVE;

    for (uint32_t i = threadIdx.x; i < CS * E; i += PERM_THREADS) s_cnt[i] = 0;
    for (uint32_t i = threadIdx.x; i < E; i += PERM_THREADS) s_first[i] = 0xFFFFFFFFu;
    // each wave takes chunks wv, wv + NW, ...; the ids of up to PERM_BATCH of
    // them are loaded together (one memory round trip), and kept for the
    // scatter when one batch covers all of the wave's chunks
    constexpr int PERM_BATCH = 8;
    const bool one_batch = C <= NW * PERM_BATCH;
    uint32_t eid[PERM_BATCH];
    auto load_ids = [&](uint32_t c_first) {
#pragma unroll
        for (int k = 0; k < PERM_BATCH; ++k) {
            const uint32_t p = (c_first + k * NW) * 64 + lane;
            eid[k] = p < P ? ids[p] : 0xFFFFFFFFu;
        }
    };
    __syncthreads();
    for (uint32_t cb = wv; cb < C; cb += NW * PERM_BATCH) {
        load_ids(cb);
#pragma unroll
        for (int k = 0; k < PERM_BATCH; ++k) {
            const uint32_t c = cb + k * NW, p = c * 64 + lane;
            if (c >= C || p >= P) continue;
            const uint32_t e = eid[k];
            if (e < E) {
                atomicAdd(&s_cnt[e * CS + c], 1u);
                if (union_ids) atomicMin(&s_first[e], p);
            } else {
                atomicOr(err, 2u);
            }
        }
    }
    __syncthreads();
    // per expert: counts -> exclusive prefix over chunks.  S threads (a power
    // of two, in one wave) share an expert's C chunks in segments: segment sums,
    // an exclusive scan over the segments, then each chunk's prefix.
    {
        uint32_t S = 64;
        while (S > 1 && E * S > PERM_THREADS) S >>= 1;
        const uint32_t e = threadIdx.x / S, sg = threadIdx.x % S;
        const uint32_t Lc = (C + S - 1) / S;
        const uint32_t c0 = min(sg * Lc, C), c1 = min(c0 + Lc, C);
        uint32_t seg = 0;
        if (e < E)
            for (uint32_t c = c0; c < c1; ++c) seg += s_cnt[e * CS + c];
        // inclusive scan over the S segments of this expert (lanes e*S .. e*S + S - 1)
        uint32_t inc = seg;
        for (uint32_t dlt = 1; dlt < S; dlt <<= 1) {
            const uint32_t o = __shfl_up(inc, dlt, S);
            if (sg >= dlt) inc += o;
        }
        if (e < E) {
            uint32_t run = inc - seg;
            for (uint32_t c = c0; c < c1; ++c) {
                const uint32_t t = s_cnt[e * CS + c];
                s_cnt[e * CS + c] = run;
                run += t;
            }
            if (sg == S - 1) {
                s_tot[e] = inc;
                // work-order key: cost, then the lower id first (0: untouched);
                // the cost of P pairs is at most 6 C, so it fits while C * E
                // fits the LDS
                s_key[e] = inc ? gm_cost(inc) * E + (E - 1 - e) : 0u;
            }
        }
    }
    __syncthreads();
    // expert offsets: exclusive scan of the totals by wave 0, eight experts a lane
    if (wv == 0) {
        uint32_t loc[8], sum = 0;
#pragma unroll
        for (int i = 0; i < 8; ++i) {
            const uint32_t e = 8 * lane + i;
            loc[i] = e < E ? s_tot[e] : 0u;
            sum += loc[i];
        }
        uint32_t inc = sum;
        for (int dlt = 1; dlt < WAVE; dlt <<= 1) {
            const uint32_t o = __shfl_up(inc, dlt);
            if (lane >= dlt) inc += o;
        }
        uint32_t run = inc - sum;
#pragma unroll
        for (int i = 0; i < 8; ++i) {
            const uint32_t e = 8 * lane + i;
            if (e <= E) s_off[e] = run;
            run += loc[i];
        }
        if (lane == WAVE - 1) s_off[E] = inc;   // (E = 512 is past the last lane's eight)
    }
    __syncthreads();
    for (uint32_t e = threadIdx.x; e <= E; e += PERM_THREADS) offsets[e] = s_off[e];
    // scatter: rank among equal ids of lower lanes of the same chunk; the
    // lanes holding this lane's id are found bit by bit (one ballot per bit
    // of an id below E)
    uint32_t nbits = 1;
    while ((1u << nbits) < E) ++nbits;
    for (uint32_t cb = wv; cb < C; cb += NW * PERM_BATCH) {
      if (!one_batch) load_ids(cb);
#pragma unroll
      for (int k = 0; k < PERM_BATCH; ++k) {
        const uint32_t c = cb + k * NW;
        if (c >= C) break;
        const uint32_t p = c * 64 + lane;
        const uint32_t e = eid[k];
        const bool ok = e < E;
        uint64_t same = __ballot(ok);
        for (uint32_t b = 0; b < nbits; ++b) {
            const bool bit = (e >> b) & 1u;
            const uint64_t set = __ballot(ok && bit);
            same &= bit ? set : ~set;
        }
        const uint32_t rank = __popcll(same & ((1ull << lane) - 1ull));
        if (ok) {
            const uint32_t dst = s_off[e] + s_cnt[e * CS + c] + rank;
            sorted_pairs[dst] = p;
            if (sorted_tokens) sorted_tokens[dst] = p / K;
            if (sorted_w) sorted_w[dst] = w[p];
        }
      }
    }
    // union order: touched experts ranked by first appearance
    if (union_ids) {
        for (uint32_t e = threadIdx.x; e < E; e += PERM_THREADS) {
            if (s_tot[e] == 0) continue;
            uint32_t r = 0;
            for (uint32_t e2 = 0; e2 < E; ++e2) r += (s_tot[e2] != 0 && s_first[e2] < s_first[e]);
            union_ids[r] = e;
        }
    }
    if (union_size && threadIdx.x == 0) {
        uint32_t n = 0;
        for (uint32_t e = 0; e < E; ++e) n += s_tot[e] != 0;
        *union_size = n;
    }
    // GEMM work order: rank of each touched expert by (cost descending, id).  S
    // threads (a power of two, in one wave) share an expert's comparisons, as in
    // the prefix above, and sum their counts with shuffles.
    if (sched) {
        uint32_t S = 64;
        while (S > 1 && E * S > PERM_THREADS) S >>= 1;
        const uint32_t e = threadIdx.x / S, sg = threadIdx.x % S;
        uint32_t r = 0, n = 0, ke = 0;
        if (e < E) {
            ke = s_key[e];
            for (uint32_t e2 = sg; e2 < E; e2 += S) {
                const uint32_t k2 = s_key[e2];
                n += k2 != 0;
                r += k2 > ke;
            }
        }
        for (uint32_t dlt = 1; dlt < S; dlt <<= 1) {
            r += __shfl_xor(r, dlt, S);
            n += __shfl_xor(n, dlt, S);
        }
        if (e < E && sg == 0) {
            if (ke != 0) sched[1 + r] = e;
            if (e == 0) sched[0] = n;
        }
    }
}

// ---------------------------------------------------------------------------
// k_grouped_mm: for each expert e with M = offsets[e+1] - offsets[e] pairs,
// out[pair][n] for one tile of its weight matrix: 128 rows of gate and of up
// (gate+up, SiLU fused) or 256 rows of down.  Block = 8 waves; wave w owns two
// 16-row MFMA subtiles (gate and up rows 16w.., or down rows 32w.. and
// 32w + 16..) and all m-tiles of the pass (up to 64 pairs, so each weight is
// read once per expert for M <= 64).  Block b works on the schedule's rank
// r = 8 s + x (s even) or 8 s + 7 - x (s odd) for x = b mod 8 (its XCD under
// the round-robin deal) and slot s = (b / 8) / n_tiles, tile (b / 8) mod
// n_tiles: every tile of an expert runs on one XCD (the activation rows stay
// in its L2), and the experts, dealt in decreasing cost down and up the XCDs,
// leave every XCD about the same work whatever the routing.
//
// The k dimension streams through two rings in LDS, filled by direct
// global->LDS loads (global_load_lds_dwordx4) so that nothing in flight holds
// registers:
//   weights      GM_SW stages of two 64-column groups: every wave brings its
//                32 rows x 64 bytes of codes (each row's 64 bytes in one
//                instruction: 32-byte pieces per row halve the stream rate)
//                and the rows' two fp16 scales;
//   activations  GM_SA stages of one group: the pass's rows (f16 hi and lo
//                planes), a share per wave.
// Body c (one group) waits for its stages, passes one barrier, requests
// activation stage c + 3 and then (even c) weight stage c/2 + 3, and computes:
// the weights, from HBM, then have five bodies before a wait covers them.  Each stage
// lives in its own __shared__ object, so the compiler can tell the in-flight
// fills from the stage being read; completion is awaited with an explicit
// vmcnt: every wave issues the same loads in the same order.
//
// v_mfma_f32_16x16x32_f16 operand layout: lane l holds A[l % 16][8 (l/16) + j]
// and B[8 (l/16) + j][l % 16] (j < 8) and receives D[4 (l/16) + i][l % 16].
// Inside a 64-column group, lane quarter q = l/16 of MFMA step s uses the
// physical columns 16 q + 8 s + j (both operands hold a lane's 8 columns in
// the order 0 2 4 6 1 3 5 7).  Weights enter as f16 (2c - 15)/8 (exact), so
// a group's MFMA sum times s_g is 15/60 of its dequantised dot product
// (kernels.metal:90-105, 140-145) and the epilogue is one FMA per output.
// LDS layouts (16-byte slots; XOR swizzles keep the fragment reads free of
// bank conflicts):
//   weights  subtile j of wave w: row n, slot (2 g + h) ^ (n >> 2 & 3) holds
//            bytes 16 h .. 16 h + 15 of group g of the stage;
//   acts     row r, slot x ^ (r & 15) = logical slot x = 8 plane + c8, i.e.
//            columns 8 c8 .. 8 c8 + 7 of the group in plane hi (0) or lo (1).
// ---------------------------------------------------------------------------
constexpr int GM_WAVES = 8;
constexpr int GM_SW = 4;                     // weight ring stages (two 64-column groups each)
constexpr int GM_SA = 4;                     // activation ring stages (one group each)
constexpr int GM_PASS = 64;                  // pair rows per pass (4 m-tiles)
constexpr uint32_t GM_ROWS_GU = 16 * GM_WAVES;   // gate (and up) rows per block
constexpr uint32_t GM_ROWS_DN = 32 * GM_WAVES;   // down rows per block

struct GmW {                                 // one weight stage: 2 groups of the block's rows
    uint8_t w[GM_WAVES * 2048];              // per wave: subtile j (1 KB) = 16 rows x 4 slots of 16 B
    uint32_t sc[GM_WAVES * 64];              // per wave: slot 32 g + 16 j + n holds the fp16 scale
};
struct GmA { uint8_t a[GM_PASS * 256]; };    // one activation stage: row = 16 slots (hi, lo) x 64 columns

#define SMOE_LDS_AS(p) ((__attribute__((address_space(3))) void*)(p))

// 8 codes (a word: byte b holds codes 2b (low nibble) and 2b + 1) -> 8 f16
// (c - 7.5) / 4 in the order 0 2 4 6 1 3 5 7.  A code shifted to bits 4..7 of
// a byte under the byte 0x4C is the f16 16 + c/4 (exponent 4, mantissa
// c << 4), one v_perm per two codes; 16 + c/4 - 17.875 = (c - 7.5)/4 is exact.
__device__ __forceinline__ half8_t q4_codes_to_f16(uint32_t v)
{
    const uint32_t E = (v << 4) & 0xF0F0F0F0u;    // even codes << 4
    const uint32_t O = v & 0xF0F0F0F0u;           // odd codes << 4
    const uint32_t K = 0x4C4C4C4Cu;
    u32x4_t r;
    r.x = __builtin_amdgcn_perm(K, E, 0x04010400u);   // codes 0, 2
    r.y = __builtin_amdgcn_perm(K, E, 0x04030402u);   // codes 4, 6
    r.z = __builtin_amdgcn_perm(K, O, 0x04010400u);   // codes 1, 3
    r.w = __builtin_amdgcn_perm(K, O, 0x04030402u);   // codes 5, 7
    const _Float16 b = static_cast<_Float16>(-17.875f);
    const half8_t bias = {b, b, b, b, b, b, b, b};
    return __builtin_bit_cast(half8_t, r) + bias;
}

__device__ __forceinline__ half8_t lds_half8(const uint8_t* p)
{
    const uint4 v = *reinterpret_cast<const uint4*>(__builtin_assume_aligned(p, 16));
    u32x4_t u;
    u.x = v.x; u.y = v.y; u.z = v.z; u.w = v.w;
    return __builtin_bit_cast(half8_t, u);
}

template <int N>
__device__ __forceinline__ void vm_wait()
{
    static_assert(N >= 0 && N < 64, "vmcnt range");
    __builtin_amdgcn_s_waitcnt((N & 0xF) | ((N >> 4) << 14) | (0x7 << 4) | (0xF << 8));
}
__device__ __forceinline__ void mem_fence_compiler() { asm volatile("" ::: "memory"); }
__device__ __forceinline__ void gm_barrier()
{
    asm volatile("" ::: "memory");
    __builtin_amdgcn_s_barrier();
    asm volatile("" ::: "memory");
}

template <bool GATE_UP, int MS>
__device__ __forceinline__ void grouped_mm_expert(
    const MoeDims& d, const LayerDesc& L, uint32_t e, uint32_t tile, uint32_t base, uint32_t M,
    const uint32_t* __restrict__ sorted_pairs, const uint16_t* __restrict__ a_hi, const uint16_t* __restrict__ a_lo,
    const float* __restrict__ a_scale, uint32_t a_row_div, float* __restrict__ out, uint32_t n_dim, uint32_t k_dim,
    GmW& w0, GmW& w1, GmW& w2, GmW& w3, GmA& a0, GmA& a1, GmA& a2, GmA& a3, uint32_t (&s_row)[GM_PASS],
    uint32_t (&s_pair)[GM_PASS])
{
    constexpr int AN = MS >= 3 ? 2 : 1;          // activation loads per wave and stage (4 rows each;
                                                 // at MS = 3 rows past the pass repeat its last row)
    constexpr int PASS = 16 * MS;
    const int lane = threadIdx.x & 63;
    const uint32_t wv = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const uint32_t G = k_dim >> 6;
    const uint32_t m16 = lane & 15, q = lane >> 4;

    const uint8_t* blob = L.experts + static_cast<size_t>(e) * L.stride;
    const size_t row_bytes = k_dim >> 1;
    auto w_row = [&](uint32_t j, uint32_t n) -> uint32_t {
        const uint32_t r = GATE_UP ? tile * GM_ROWS_GU + 16 * wv + n : tile * GM_ROWS_DN + 32 * wv + 16 * j + n;
        return min(r, n_dim - 1);
    };
    auto w_mat = [&](uint32_t j) -> const uint8_t* { return blob + (GATE_UP ? (j ? L.off[2] : L.off[0]) : L.off[4]); };
    auto s_mat = [&](uint32_t j) -> const uint16_t* {
        return reinterpret_cast<const uint16_t*>(blob + (GATE_UP ? (j ? L.off[3] : L.off[1]) : L.off[5]));
    };
    // weight fill, instruction j: lane -> row n = lane / 4, physical slot p = lane & 3,
    // logical slot s = p ^ (n / 4 & 3) = 2 g + h: bytes 32 g + 16 h of the stage's 64
    const uint32_t fn = lane >> 2, fs = (lane & 3) ^ ((fn >> 2) & 3);
    const uint32_t fg = fs >> 1, fh = fs & 1;
    const uint8_t* w_src[2];
#pragma unroll
    for (int j = 0; j < 2; ++j) w_src[j] = w_mat(j) + static_cast<size_t>(w_row(j, fn)) * row_bytes + 16 * fh;
    // scale fill: lane -> group g = lane / 32 of the stage, subtile (lane / 16) & 1, row lane & 15
    const uint32_t sg = lane >> 5, sj = (lane >> 4) & 1, sn = lane & 15;
    const uint16_t* s_src = s_mat(sj) + static_cast<size_t>(w_row(sj, sn)) * G;
    // (an odd G's last stage has one group: its second group re-reads group G - 1)
    auto issue_w = [&](GmW& S, uint32_t st) {
        const uint32_t g0 = 2 * st + fg, gs = 2 * st + sg;
#pragma unroll
        for (int j = 0; j < 2; ++j)
            __builtin_amdgcn_global_load_lds(w_src[j] + min(g0, G - 1) * 32, SMOE_LDS_AS(&S.w[wv * 2048 + j * 1024]),
                                             16, 0, 0);
        __builtin_amdgcn_global_load_lds(s_src + min(gs, G - 1), SMOE_LDS_AS(&S.sc[wv * 64]), 2, 0, 0);
    };
    // B fragment of this lane for group g of a stage: row m16, bytes 8 q .. 8 q + 7 of the group
    uint32_t boff[2];
#pragma unroll
    for (int g = 0; g < 2; ++g) boff[g] = wv * 2048 + m16 * 64 + 16 * ((2 * g + (q >> 1)) ^ ((m16 >> 2) & 3)) + 8 * (q & 1);
    // A fragment offsets of this lane inside an activation stage (m-tile ms adds 4096 bytes)
    uint32_t aoff[2][2];
#pragma unroll
    for (int stp = 0; stp < 2; ++stp)
#pragma unroll
        for (int pl = 0; pl < 2; ++pl) aoff[stp][pl] = m16 * 256 + 16 * ((8 * pl + 2 * q + stp) ^ m16);

    for (uint32_t m0 = 0; m0 < M; m0 += PASS) {
        __syncthreads();
        if (threadIdx.x < PASS) {
            const uint32_t p = sorted_pairs[base + min(m0 + threadIdx.x, M - 1)];
            s_pair[threadIdx.x] = p;
            s_row[threadIdx.x] = p / a_row_div;
        }
        __syncthreads();
        const uint16_t* a_src[AN];
#pragma unroll
        for (int u = 0; u < AN; ++u) {
            const uint32_t r = wv * 4 * AN + 4 * u + (lane >> 4);
            const uint32_t x = (lane & 15) ^ (r & 15);
            const uint32_t srow = s_row[min(r, static_cast<uint32_t>(PASS - 1))];
            a_src[u] = ((x >> 3) ? a_lo : a_hi) + static_cast<size_t>(srow) * k_dim + 8 * (x & 7);
        }
        auto issue_a = [&](GmA& S, uint32_t c) {
#pragma unroll
            for (int u = 0; u < AN; ++u)
                __builtin_amdgcn_global_load_lds(a_src[u] + c * 64, SMOE_LDS_AS(&S.a[(wv * 4 * AN + 4 * u) * 256]), 16,
                                                 0, 0);
        };

        f32x4_t acc[MS][2];
#pragma unroll
        for (int ms = 0; ms < MS; ++ms)
#pragma unroll
            for (int j = 0; j < 2; ++j) acc[ms][j] = f32x4_t{0.f, 0.f, 0.f, 0.f};

        // Issue order of the loop: body c issues the activation stage c + 3 and then the
        // weight stage c / 2 + 3 (if c is even).  The prologue replays bodies -6 .. -1.
        const uint32_t NWS = (G + 1) / 2;        // weight stages
        if (0 < NWS) issue_w(w0, 0);
        if (1 < NWS) issue_w(w1, 1);
        if (0 < G) issue_a(a0, 0);
        if (1 < G) issue_a(a1, 1);
        if (2 < NWS) issue_w(w2, 2);
        if (2 < G) issue_a(a2, 2);
        mem_fence_compiler();

        auto body = [&](uint32_t c, GmW& W, uint32_t g, GmW& WN, GmA& A, GmA& AN_) {
            // A(c) was the first load of body c - 3; after it came the weight stage of body
            // c - 3 when c - 3 is even, A(c + 1), A(c + 2) and the weight stage of the even
            // one of bodies c - 2, c - 1 ((c + 4 + (c & 1)) / 2, the later of the two).  When
            // all of those were issued, 2 AN + 3 (even c) or 2 AN + 6 (odd c) loads may still
            // be pending; near the end fewer were, and the wait covers everything.
            if (c + 2 < G && (c + 4 + (c & 1)) / 2 < NWS) {
                if (g) vm_wait<2 * AN + 6>();
                else vm_wait<2 * AN + 3>();
            } else {
                vm_wait<0>();
            }
            gm_barrier();
            if (c + 3 < G) issue_a(AN_, c + 3);
            if (g == 0 && c / 2 + 3 < NWS) issue_w(WN, c / 2 + 3);
            mem_fence_compiler();
            half8_t b[2][2];
            float sc[2];
#pragma unroll
            for (int j = 0; j < 2; ++j) {
                const uint2 v = *reinterpret_cast<const uint2*>(&W.w[boff[g] + 1024 * j]);
                b[j][0] = q4_codes_to_f16(v.x);
                b[j][1] = q4_codes_to_f16(v.y);
                sc[j] = f16_bits_to_f32(static_cast<uint16_t>(W.sc[wv * 64 + 32 * g + 16 * j + m16]));
            }
#pragma unroll
            for (int ms = 0; ms < MS; ++ms) {
                half8_t xa[2][2];
#pragma unroll
                for (int stp = 0; stp < 2; ++stp)
#pragma unroll
                    for (int pl = 0; pl < 2; ++pl) xa[stp][pl] = lds_half8(A.a + ms * 4096 + aoff[stp][pl]);
#pragma unroll
                for (int j = 0; j < 2; ++j) {
                    f32x4_t t = {0.f, 0.f, 0.f, 0.f};
                    t = __builtin_amdgcn_mfma_f32_16x16x32_f16(xa[0][0], b[j][0], t, 0, 0, 0);
                    t = __builtin_amdgcn_mfma_f32_16x16x32_f16(xa[0][1], b[j][0], t, 0, 0, 0);
                    t = __builtin_amdgcn_mfma_f32_16x16x32_f16(xa[1][0], b[j][1], t, 0, 0, 0);
                    t = __builtin_amdgcn_mfma_f32_16x16x32_f16(xa[1][1], b[j][1], t, 0, 0, 0);
#pragma unroll
                    for (int i = 0; i < 4; ++i) acc[ms][j][i] = fmaf(sc[j], t[i], acc[ms][j][i]);
                }
            }
            mem_fence_compiler();
        };
        for (uint32_t c = 0; c < G; c += 8) {
            body(c, w0, 0, w3, a0, a3);
            if (c + 1 < G) body(c + 1, w0, 1, w3, a1, a0);
            if (c + 2 < G) body(c + 2, w1, 0, w0, a2, a1);
            if (c + 3 < G) body(c + 3, w1, 1, w0, a3, a2);
            if (c + 4 < G) body(c + 4, w2, 0, w1, a0, a3);
            if (c + 5 < G) body(c + 5, w2, 1, w1, a1, a0);
            if (c + 6 < G) body(c + 6, w3, 0, w2, a2, a1);
            if (c + 7 < G) body(c + 7, w3, 1, w2, a3, a2);
        }
#pragma unroll
        for (int ms = 0; ms < MS; ++ms) {
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                const uint32_t m = 16 * ms + 4 * q + i;
                if (m0 + m >= M) continue;
                const float rs = a_scale[s_row[m]] * (8.0f / 15.0f);   // weights are (2c - 15) / 8
                float* o = out + static_cast<size_t>(s_pair[m]) * n_dim;
                if (GATE_UP) {
                    const uint32_t n = tile * GM_ROWS_GU + 16 * wv + m16;
                    if (n < n_dim) {
                        const float v0 = acc[ms][0][i] * rs, v1 = acc[ms][1][i] * rs;
                        o[n] = (v0 * (1.0f / (1.0f + expf(-v0)))) * v1;
                    }
                } else {
#pragma unroll
                    for (int j = 0; j < 2; ++j) {
                        const uint32_t n = tile * GM_ROWS_DN + 32 * wv + 16 * j + m16;
                        if (n < n_dim) o[n] = acc[ms][j][i] * rs;
                    }
                }
            }
        }
    }
}

template <bool GATE_UP>
__global__ __launch_bounds__(GM_WAVES * WAVE, 1)
void k_grouped_mm(MoeDims d, LayerDesc L, const uint32_t* __restrict__ offsets,
                  const uint32_t* __restrict__ sched, const uint32_t* __restrict__ sorted_pairs, const uint16_t* __restrict__ a_hi,
                  const uint16_t* __restrict__ a_lo, const float* __restrict__ a_scale, uint32_t a_row_div,
                  float* __restrict__ out, uint32_t n_dim, uint32_t k_dim, uint32_t n_tiles)
{
    __shared__ __align__(16) GmW w0, w1, w2, w3;
    __shared__ __align__(16) GmA a0, a1, a2, a3;
    __shared__ uint32_t s_row[GM_PASS];
    __shared__ uint32_t s_pair[GM_PASS];
    const uint32_t b = blockIdx.x, xcd = b & 7u, jb = b >> 3;
    const uint32_t slot = jb / n_tiles, tile = jb % n_tiles;
    const uint32_t r = 8u * slot + ((slot & 1u) ? 7u - xcd : xcd);
    if (r >= sched[0]) return;
    const uint32_t e = sched[1 + r];
    if (e >= d.E) return;
    const uint32_t base = offsets[e], M = offsets[e + 1] - base;
    if (M == 0) return;
    if (M <= 16)
        grouped_mm_expert<GATE_UP, 1>(d, L, e, tile, base, M, sorted_pairs, a_hi, a_lo, a_scale, a_row_div, out,
                                      n_dim, k_dim, w0, w1, w2, w3, a0, a1, a2, a3, s_row, s_pair);
    else if (M <= 32)
        grouped_mm_expert<GATE_UP, 2>(d, L, e, tile, base, M, sorted_pairs, a_hi, a_lo, a_scale, a_row_div, out,
                                      n_dim, k_dim, w0, w1, w2, w3, a0, a1, a2, a3, s_row, s_pair);
    else if (M <= 48)
        grouped_mm_expert<GATE_UP, 3>(d, L, e, tile, base, M, sorted_pairs, a_hi, a_lo, a_scale, a_row_div, out,
                                      n_dim, k_dim, w0, w1, w2, w3, a0, a1, a2, a3, s_row, s_pair);
    else
        grouped_mm_expert<GATE_UP, 4>(d, L, e, tile, base, M, sorted_pairs, a_hi, a_lo, a_scale, a_row_div, out,
                                      n_dim, k_dim, w0, w1, w2, w3, a0, a1, a2, a3, s_row, s_pair);
}

// ---------------------------------------------------------------------------
// k_grouped_down: the down products of k_grouped_mm<false> (same pairs, same
// sums per 64-column group, same epilogue) with the weights streamed into
// registers: each weight row belongs to one wave, so plain loads need neither
// LDS nor a barrier for them.  Blocks of 4 waves x 64 rows (four 16-row
// subtiles a wave), two blocks per CU: every activation fragment read from LDS
// feeds four subtiles (half the LDS reads per weight of the 8 x 32-row block),
// and the two blocks of a CU pass their barriers independently, so one block's
// MFMAs overlap the other's conversion.  Needs an even number of groups (a
// stage's two scales are one dword).  30B layer, 512 tokens: 58.9 us against
// 72 for k_grouped_mm<false> (bench.py --workload prefill).
//   weights  per wave and stage (two groups: 64 bytes of every row), subtile
//            j: lane l loads row l & 15, bytes 16 (l >> 4) .. + 15; one
//            v_permlane32_swap per two dwords then leaves every lane one dword
//            of each (group, MFMA step): quad q, step s of either group holds
//            its 8-column unit 4 (q & 1) + 2 (q >> 1) + s, and the activation
//            fragments are read from those units;
//   acts     the ring of k_grouped_mm (f16 hi/lo planes, XOR-swizzled 16-byte
//            slots), filled by direct loads issued from inline asm: the
//            compiler does not track them, so it adds no waits of its own for
//            the ring (it would drain every load in flight once per unrolled
//            iteration); the explicit vmcnt waits cover them.
// ---------------------------------------------------------------------------
constexpr int GD_WAVES = 4;
constexpr int GD_SUB = 4;                                  // 16-row subtiles a wave
constexpr uint32_t GD_ROWS = 16 * GD_SUB * GD_WAVES;       // down rows per block

__device__ __forceinline__ uint32_t lds_addr(const void* p)
{
    return static_cast<uint32_t>(reinterpret_cast<uintptr_t>((const __attribute__((address_space(3))) void*)p));
}
// lane l's 16 bytes land at LDS byte address lds + 16 l
__device__ __forceinline__ void dma16(const void* g, uint32_t lds)
{
    asm volatile("s_mov_b32 m0, %1\n\ts_nop 0\n\tglobal_load_lds_dwordx4 %0, off" ::"v"(g), "s"(lds) : "memory", "m0");
}

template <int MS>
__device__ __forceinline__ void grouped_down_expert(
    const LayerDesc& L, uint32_t e, uint32_t tile, uint32_t base, uint32_t M, const uint32_t* __restrict__ sorted_pairs,
    const uint16_t* __restrict__ a_hi, const uint16_t* __restrict__ a_lo, const float* __restrict__ a_scale,
    float* __restrict__ out, uint32_t n_dim, uint32_t k_dim, GmA& a0, GmA& a1, GmA& a2, GmA& a3,
    uint32_t (&s_row)[GM_PASS], uint32_t (&s_pair)[GM_PASS])
{
    constexpr int AN = MS;                       // activation loads per wave and stage (4 rows each)
    constexpr int PASS = 16 * MS;
    constexpr int WS = 2 * GD_SUB;               // loads per weight stage (codes, scales)
    const int lane = threadIdx.x & 63;
    const uint32_t wv = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const uint32_t G = k_dim >> 6, NWS = G / 2;
    const uint32_t m16 = lane & 15, q = lane >> 4;

    const uint8_t* blob = L.experts + static_cast<size_t>(e) * L.stride;
    const size_t row_bytes = k_dim >> 1;
    const uint8_t* w_src[GD_SUB];
    const uint32_t* s_src[GD_SUB];
#pragma unroll
    for (int j = 0; j < GD_SUB; ++j) {
        const uint32_t r = min(tile * GD_ROWS + 16 * GD_SUB * wv + 16 * j + m16, n_dim - 1);
        w_src[j] = blob + L.off[4] + static_cast<size_t>(r) * row_bytes + 16 * q;
        s_src[j] = reinterpret_cast<const uint32_t*>(blob + L.off[5] + static_cast<size_t>(r) * G * 2);
    }
    uint4 wr[4][GD_SUB];                         // weight ring: [stage slot][subtile]
    uint32_t sr[4][GD_SUB];                      // the stage's two fp16 scales per subtile
    auto issue_w = [&](int slot, uint32_t st) {
#pragma unroll
        for (int j = 0; j < GD_SUB; ++j) wr[slot][j] = *reinterpret_cast<const uint4*>(w_src[j] + 64 * st);
#pragma unroll
        for (int j = 0; j < GD_SUB; ++j) sr[slot][j] = s_src[j][st];
    };
    uint32_t aoff[2][2];
    const uint32_t u8 = 4 * (q & 1) + 2 * (q >> 1);
#pragma unroll
    for (int stp = 0; stp < 2; ++stp)
#pragma unroll
        for (int pl = 0; pl < 2; ++pl) aoff[stp][pl] = m16 * 256 + 16 * ((8 * pl + u8 + stp) ^ m16);

    for (uint32_t m0 = 0; m0 < M; m0 += PASS) {
        __syncthreads();
        if (threadIdx.x < PASS) {
            const uint32_t p = sorted_pairs[base + min(m0 + threadIdx.x, M - 1)];
            s_pair[threadIdx.x] = p;
            s_row[threadIdx.x] = p;
        }
        __syncthreads();
        const uint16_t* a_src[AN];
#pragma unroll
        for (int u = 0; u < AN; ++u) {
            const uint32_t r = wv * 4 * AN + 4 * u + (lane >> 4);
            const uint32_t x = (lane & 15) ^ (r & 15);
            const uint32_t srow = s_row[min(r, static_cast<uint32_t>(PASS - 1))];
            a_src[u] = ((x >> 3) ? a_lo : a_hi) + static_cast<size_t>(srow) * k_dim + 8 * (x & 7);
        }
        auto issue_a = [&](GmA& S, uint32_t c) {
#pragma unroll
            for (int u = 0; u < AN; ++u) dma16(a_src[u] + c * 64, lds_addr(&S.a[(wv * 4 * AN + 4 * u) * 256]));
        };

        f32x4_t acc[MS][GD_SUB];
#pragma unroll
        for (int ms = 0; ms < MS; ++ms)
#pragma unroll
            for (int j = 0; j < GD_SUB; ++j) acc[ms][j] = f32x4_t{0.f, 0.f, 0.f, 0.f};

        // body c issues the activation stage c + 3 and then (even c) the weight
        // stage c / 2 + 3; the prologue replays bodies -6 .. -1
        if (0 < NWS) issue_w(0, 0);
        if (1 < NWS) issue_w(1, 1);
        issue_a(a0, 0);
        if (1 < G) issue_a(a1, 1);
        if (2 < NWS) issue_w(2, 2);
        if (2 < G) issue_a(a2, 2);
        mem_fence_compiler();

        uint32_t gw[GD_SUB][2][2];               // [subtile][group of the stage][MFMA step]
        auto body = [&](uint32_t c, int slot, int g, int nslot, GmA& A, GmA& AN_) {
            // After A(c) (first load of body c - 3) came: the weight stage of body c - 3
            // when c - 3 is even, A(c + 1), A(c + 2) and the weight stage of the even one
            // of bodies c - 2, c - 1.  When all of those were issued, 2 AN + WS (even c)
            // or 2 AN + 2 WS (odd c) loads may still be pending; near the end fewer
            // were, and the wait covers everything.  A(c) done also means the weight
            // stage c / 2 is: it was issued in body c - 6, before A(c).
            if (c + 2 < G && (c + 4 + (c & 1)) / 2 < NWS) {
                if (g) vm_wait<2 * AN + 2 * WS>();
                else vm_wait<2 * AN + WS>();
            } else {
                vm_wait<0>();
            }
            gm_barrier();
            if (c + 3 < G) issue_a(AN_, c + 3);
            if (g == 0 && c / 2 + 3 < NWS) issue_w(nslot, c / 2 + 3);
            mem_fence_compiler();
            if (g == 0) {
#pragma unroll
                for (int j = 0; j < GD_SUB; ++j)
#pragma unroll
                    for (int s = 0; s < 2; ++s) {
                        // lanes 0-31 hold the stage's group 0 (bytes 0-31 of the 64), lanes
                        // 32-63 group 1: swap dwords 2 + s of the lower half with dwords s
                        // of the upper half
                        const uint32_t lo = s ? wr[slot][j].y : wr[slot][j].x;
                        const uint32_t hi = s ? wr[slot][j].w : wr[slot][j].z;
                        const auto r = __builtin_amdgcn_permlane32_swap(lo, hi, false, false);
                        gw[j][0][s] = r[0];
                        gw[j][1][s] = r[1];
                    }
            }
            half8_t b[GD_SUB][2];
            float sc[GD_SUB];
#pragma unroll
            for (int j = 0; j < GD_SUB; ++j) {
                b[j][0] = q4_codes_to_f16(gw[j][g][0]);
                b[j][1] = q4_codes_to_f16(gw[j][g][1]);
                sc[j] = f16_bits_to_f32(static_cast<uint16_t>(g ? sr[slot][j] >> 16 : sr[slot][j]));
            }
#pragma unroll
            for (int ms = 0; ms < MS; ++ms) {
                half8_t xa[2][2];
#pragma unroll
                for (int stp = 0; stp < 2; ++stp)
#pragma unroll
                    for (int pl = 0; pl < 2; ++pl) xa[stp][pl] = lds_half8(A.a + ms * 4096 + aoff[stp][pl]);
#pragma unroll
                for (int j = 0; j < GD_SUB; ++j) {
                    f32x4_t t = {0.f, 0.f, 0.f, 0.f};
                    t = __builtin_amdgcn_mfma_f32_16x16x32_f16(xa[0][0], b[j][0], t, 0, 0, 0);
                    t = __builtin_amdgcn_mfma_f32_16x16x32_f16(xa[0][1], b[j][0], t, 0, 0, 0);
                    t = __builtin_amdgcn_mfma_f32_16x16x32_f16(xa[1][0], b[j][1], t, 0, 0, 0);
                    t = __builtin_amdgcn_mfma_f32_16x16x32_f16(xa[1][1], b[j][1], t, 0, 0, 0);
#pragma unroll
                    for (int i = 0; i < 4; ++i) acc[ms][j][i] = fmaf(sc[j], t[i], acc[ms][j][i]);
                }
            }
            mem_fence_compiler();
        };
        for (uint32_t c = 0; c < G; c += 8) {
            body(c, 0, 0, 3, a0, a3);
            if (c + 1 < G) body(c + 1, 0, 1, 3, a1, a0);
            if (c + 2 < G) body(c + 2, 1, 0, 0, a2, a1);
            if (c + 3 < G) body(c + 3, 1, 1, 0, a3, a2);
            if (c + 4 < G) body(c + 4, 2, 0, 1, a0, a3);
            if (c + 5 < G) body(c + 5, 2, 1, 1, a1, a0);
            if (c + 6 < G) body(c + 6, 3, 0, 2, a2, a1);
            if (c + 7 < G) body(c + 7, 3, 1, 2, a3, a2);
        }
#pragma unroll
        for (int ms = 0; ms < MS; ++ms) {
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                const uint32_t m = 16 * ms + 4 * q + i;
                if (m0 + m >= M) continue;
                const float rs = a_scale[s_row[m]] * (8.0f / 15.0f);   // weights are (2c - 15) / 8
                float* o = out + static_cast<size_t>(s_pair[m]) * n_dim;
#pragma unroll
                for (int j = 0; j < GD_SUB; ++j) {
                    const uint32_t n = tile * GD_ROWS + 16 * GD_SUB * wv + 16 * j + m16;
                    if (n < n_dim) o[n] = acc[ms][j][i] * rs;
                }
            }
        }
    }
}

__global__ __launch_bounds__(GD_WAVES * WAVE, 2)
void k_grouped_down(MoeDims d, LayerDesc L, const uint32_t* __restrict__ offsets, const uint32_t* __restrict__ sched,
                    const uint32_t* __restrict__ sorted_pairs, const uint16_t* __restrict__ a_hi,
                    const uint16_t* __restrict__ a_lo, const float* __restrict__ a_scale, float* __restrict__ out,
                    uint32_t n_dim, uint32_t k_dim, uint32_t n_tiles)
{
    __shared__ __align__(16) GmA a0, a1, a2, a3;
    __shared__ uint32_t s_row[GM_PASS];
    __shared__ uint32_t s_pair[GM_PASS];
    // the schedule order of k_grouped_mm
    const uint32_t b = blockIdx.x, xcd = b & 7u, jb = b >> 3;
    const uint32_t slot = jb / n_tiles, tile = jb % n_tiles;
    const uint32_t r = 8u * slot + ((slot & 1u) ? 7u - xcd : xcd);
    if (r >= sched[0]) return;
    const uint32_t e = sched[1 + r];
    if (e >= d.E) return;
    const uint32_t base = offsets[e], M = offsets[e + 1] - base;
    if (M == 0) return;
    if (M <= 16)
        grouped_down_expert<1>(L, e, tile, base, M, sorted_pairs, a_hi, a_lo, a_scale, out, n_dim, k_dim, a0, a1, a2,
                               a3, s_row, s_pair);
    else if (M <= 32)
        grouped_down_expert<2>(L, e, tile, base, M, sorted_pairs, a_hi, a_lo, a_scale, out, n_dim, k_dim, a0, a1, a2,
                               a3, s_row, s_pair);
    else if (M <= 48)
        grouped_down_expert<3>(L, e, tile, base, M, sorted_pairs, a_hi, a_lo, a_scale, out, n_dim, k_dim, a0, a1, a2,
                               a3, s_row, s_pair);
    else
        grouped_down_expert<4>(L, e, tile, base, M, sorted_pairs, a_hi, a_lo, a_scale, out, n_dim, k_dim, a0, a1, a2,
                               a3, s_row, s_pair);
}

// ---------------------------------------------------------------------------
// k_combine_pairs: hidden[t][col] += sum_r w[t k + r] * y[(t k + r)][col], in
// rank order (the scatter-add of prefill.cpp:380-385 then :446-451).
// ---------------------------------------------------------------------------
__global__ __launch_bounds__(256)
void k_combine_pairs(const float* __restrict__ y, const float* __restrict__ w, uint32_t K, uint32_t D,
                     float* __restrict__ hidden)
{
    // 4 columns per thread, the K rank rows of token t summed in rank order (one
    // load at a time per thread: the many resident waves hide the latency; loading
    // all K first measured no faster)
    const uint32_t t = blockIdx.y, col = (blockIdx.x * 256 + threadIdx.x) * 4;
    if (col >= D) return;
    float4 acc = make_float4(0.f, 0.f, 0.f, 0.f);
    for (uint32_t r = 0; r < K; ++r) {
        const size_t p = static_cast<size_t>(t) * K + r;
        const float wr = w[p];
        const float4 v = load_f4(y + p * D + col);
        acc.x = fmaf(wr, v.x, acc.x);
        acc.y = fmaf(wr, v.y, acc.y);
        acc.z = fmaf(wr, v.z, acc.z);
        acc.w = fmaf(wr, v.w, acc.w);
    }
    float4* h = reinterpret_cast<float4*>(hidden + static_cast<size_t>(t) * D + col);
    const float4 o = *h;
    *h = make_float4(o.x + acc.x, o.y + acc.y, o.z + acc.z, o.w + acc.w);
}

// ---------------------------------------------------------------------------
// launchers
// ---------------------------------------------------------------------------
template <int CPL, int TB, int ES = 1>
static hipError_t route_c(const MoeDims& d, const LayerDesc& L, const float* hidden, uint32_t T, uint16_t* x_hi,
                          uint16_t* x_lo, float* x_sc, uint32_t* ids, float* w, float* logits, uint32_t* counters,
                          hipStream_t s)
{
    const dim3 grid(((T + TB - 1) / TB) * ES), block(ROUTE_WAVES * WAVE);
    if (d.E <= 128)
        launch_kernel(k_route<CPL, TB, 2, ES>, grid, block, s, d, L, hidden, T, x_hi, x_lo, x_sc, ids, w,
                      logits, counters);
    else
        launch_kernel(k_route<CPL, TB, 8, ES>, grid, block, s, d, L, hidden, T, x_hi, x_lo, x_sc, ids, w,
                      logits, counters);
    return hipGetLastError();
}

hipError_t launch_route(const MoeDims& d, const LayerDesc& L, const float* hidden, uint32_t T, uint16_t* x_hi,
                        uint16_t* x_lo, float* x_sc, uint32_t* ids, float* w, float* logits, uint32_t* counters,
                        hipStream_t s)
{
    if (d.E > SMOE_TOPK_MAX_N || d.K > SMOE_TOPK_MAX_K || d.D % 64 || T == 0) return hipErrorInvalidValue;
    const uint32_t cpl = (d.D / 32 + WAVE - 1) / WAVE;
    // tokens per block: as many as keep one block per CU busy (each block
    // reads the whole router matrix from L2 once), at most what the registers
    // of a chunk per lane allow.  Under 128 tokens (one per block) the router
    // rows of a token are split over 4 blocks (needs E <= 128: 4 rows a wave).
    const uint32_t cus = 256;
    const uint32_t tb = T >= 4 * cus ? 4 : T >= 2 * cus ? 2 : 1;
    const bool split = T < 128 && d.E <= 128 && logits && counters;
    if (cpl == 1) {
        if (tb == 4) return route_c<1, 4>(d, L, hidden, T, x_hi, x_lo, x_sc, ids, w, logits, counters, s);
        if (tb == 2) return route_c<1, 2>(d, L, hidden, T, x_hi, x_lo, x_sc, ids, w, logits, counters, s);
        if (split) return route_c<1, 1, 4>(d, L, hidden, T, x_hi, x_lo, x_sc, ids, w, logits, counters, s);
        return route_c<1, 1>(d, L, hidden, T, x_hi, x_lo, x_sc, ids, w, logits, counters, s);
    }
    if (cpl == 2) {
        if (tb >= 2) return route_c<2, 2>(d, L, hidden, T, x_hi, x_lo, x_sc, ids, w, logits, counters, s);
        if (split) return route_c<2, 1, 4>(d, L, hidden, T, x_hi, x_lo, x_sc, ids, w, logits, counters, s);
        return route_c<2, 1>(d, L, hidden, T, x_hi, x_lo, x_sc, ids, w, logits, counters, s);
    }
    if (cpl <= 4) return route_c<4, 1>(d, L, hidden, T, x_hi, x_lo, x_sc, ids, w, logits, counters, s);
    return hipErrorInvalidValue;
}

hipError_t launch_split_rows(const float* src, uint32_t rows, uint32_t cols, uint16_t* hi, uint16_t* lo,
                             float* scale, hipStream_t s)
{
    if (cols % 64 || rows == 0) return hipErrorInvalidValue;
    const uint32_t blocks = std::min<uint32_t>((rows + 3) / 4, 8192u);
    launch_kernel(k_split_rows, dim3(blocks), dim3(256), s, src, rows, cols, hi, lo, scale);
    return hipGetLastError();
}

size_t permute_lds_bytes(uint32_t P, uint32_t E)
{
    const size_t C = (P + 63) / 64;
    return (C * E + 3 * size_t(E) + 1) * sizeof(uint32_t);
}

// what k_permute allocates: the count table's odd row stride and the keys add
// at most 2 E words to permute_lds_bytes (which bounds the pass sizes)
static size_t permute_lds_alloc(uint32_t P, uint32_t E)
{
    const size_t CS = ((P + 63) / 64) | 1u;
    return (CS * E + 4 * size_t(E) + 1) * sizeof(uint32_t);
}

hipError_t launch_permute(const uint32_t* ids, const float* w, uint32_t P, uint32_t K, uint32_t E, uint32_t* offsets,
                          uint32_t* sorted_pairs, uint32_t* sorted_tokens, float* sorted_w, uint32_t* union_ids,
                          uint32_t* union_size, uint32_t* sched, uint32_t* err, hipStream_t s)
{
    if (P == 0 || E == 0 || permute_lds_bytes(P, E) > PERMUTE_MAX_LDS) return hipErrorInvalidValue;
    const size_t lds = permute_lds_alloc(P, E);
    launch_kernel_lds(k_permute, dim3(1), dim3(PERM_THREADS), static_cast<uint32_t>(lds), s, ids, w, P, K, E,
                      offsets, sorted_pairs, sorted_tokens, sorted_w, union_ids, union_size, sched, err);
    return hipGetLastError();
}

hipError_t launch_grouped_gate_up(const MoeDims& d, const LayerDesc& L, const uint32_t* offsets,
                                  const uint32_t* sched, const uint32_t* sorted_pairs, const uint16_t* x_hi,
                                  const uint16_t* x_lo, const float* x_scale, float* h, hipStream_t s)
{
    if (d.group != 64 || d.I % 64 || d.D % 64 || !offsets || !sched) return hipErrorInvalidValue;
    const uint32_t n_tiles = (d.I + GM_ROWS_GU - 1) / GM_ROWS_GU, eg = (d.E + 7) / 8;
    launch_kernel(k_grouped_mm<true>, dim3(8 * eg * n_tiles), dim3(GM_WAVES * WAVE), s, d, L, offsets, sched,
                  sorted_pairs, x_hi, x_lo, x_scale, d.K, h, d.I, d.D, n_tiles);
    return hipGetLastError();
}

hipError_t launch_grouped_down(const MoeDims& d, const LayerDesc& L, const uint32_t* offsets,
                               const uint32_t* sched, const uint32_t* sorted_pairs, const uint16_t* h_hi,
                               const uint16_t* h_lo, const float* h_scale, float* y, hipStream_t s)
{
    if (d.group != 64 || d.D % 64 || d.I % 64 || !offsets || !sched) return hipErrorInvalidValue;
    const uint32_t eg = (d.E + 7) / 8;
    if (d.I % 128 == 0) {                        // an even number of groups: the register-weight kernel
        const uint32_t nt = (d.D + GD_ROWS - 1) / GD_ROWS;
        launch_kernel(k_grouped_down, dim3(8 * eg * nt), dim3(GD_WAVES * WAVE), s, d, L, offsets, sched, sorted_pairs,
                      h_hi, h_lo, h_scale, y, d.D, d.I, nt);
        return hipGetLastError();
    }
    const uint32_t n_tiles = (d.D + GM_ROWS_DN - 1) / GM_ROWS_DN;
    launch_kernel(k_grouped_mm<false>, dim3(8 * eg * n_tiles), dim3(GM_WAVES * WAVE), s, d, L, offsets, sched,
                  sorted_pairs, h_hi, h_lo, h_scale, 1u, y, d.D, d.I, n_tiles);
    return hipGetLastError();
}

hipError_t launch_combine_pairs(const float* y, const float* w, uint32_t T, uint32_t K, uint32_t D, float* hidden,
                                hipStream_t s)
{
    if (D % 4) return hipErrorInvalidValue;
    launch_kernel(k_combine_pairs, dim3((D / 4 + 255) / 256, T), dim3(256), s, y, w, K, D, hidden);
    return hipGetLastError();
}

}  // namespace smoe
