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
//                  block; writes the normed rows (fp32) and ids/weights.
//   k_split_rows   per (row, 64-column group): power-of-two scale 2^e with
//                  |x| < 2^e, f16 hi/lo planes of x * 2^-e (hi + lo carries
//                  22 bits), and the group sum of hi + lo.
//   k_permute      stable counting sort of the T*k (token, rank) pairs by
//                  expert (one workgroup), union order by first appearance.
//   k_grouped_mm   per expert: [tokens x K] x [K x 64 rows] tiles on MFMA
//                  v_mfma_f32_16x16x32_f16.  Weights enter exactly as c - 8
//                  (f16), activations as hi and lo planes (two MFMAs into one
//                  fp32 accumulator), each 64-column group closes with the
//                  dequant epilogue s_g * 2^e * (acc + 0.5 * sum) / 7.5
//                  (kernels.metal:140-145).  Gate+up runs with SiLU and writes
//                  h per (token, rank) pair; down writes y per pair.
//   k_combine_pairs hidden[t] += sum_r w[t][r] * y[t*k + r] in rank order.
//
// Blocks of one expert are mapped to one XCD (block id mod 8), so its token
// rows stay in that XCD's L2 while the expert's weights stream once.
#include <algorithm>

#include "device_common.hpp"
#include "kernels.hpp"
#include "topk.hpp"

namespace smoe {

typedef _Float16 half8_t __attribute__((ext_vector_type(8)));
typedef float f32x4_t __attribute__((ext_vector_type(4)));
typedef uint32_t u32x4_t __attribute__((ext_vector_type(4)));

// ---------------------------------------------------------------------------
// k_route: RMSNorm (common.hpp:245-256) + router (common.hpp:293-306) +
// softmax/top-k (scout.cpp:77-123) for TB tokens per block of ROUTE_WAVES
// waves.  Every wave normalises all TB tokens (lane l owns the 32-column
// chunks l + 64 j) and computes router rows w, w + ROUTE_WAVES, ... for all of
// them; wave t then selects the experts of token t.
// ---------------------------------------------------------------------------
constexpr int ROUTE_WAVES = 8;

template <int CPL, int TB, int VPL>
__global__ __launch_bounds__(ROUTE_WAVES * WAVE)
void k_route(MoeDims d, LayerDesc L, const float* __restrict__ hidden, uint32_t T, float* __restrict__ normed,
             uint32_t* __restrict__ ids, float* __restrict__ w)
{
    constexpr int RPB = 16 / TB;   // router rows per reduction batch (RPB * TB values)
    __shared__ float s_logit[TB][SMOE_TOPK_MAX_N];
    const int lane = threadIdx.x & 63, wv = threadIdx.x >> 6;
    const uint32_t t0 = blockIdx.x * TB;
    const uint32_t D = d.D, nch = D >> 5;

    float a[TB][CPL][32];
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
        // wave t stores token t's normed row
        if (wv == t && t0 + t < T) {
#pragma unroll
            for (int j = 0; j < CPL; ++j) {
                if (lane + WAVE * j < nch) {
                    float* o = normed + static_cast<size_t>(t0 + t) * D + (lane + WAVE * j) * 32;
#pragma unroll
                    for (int q = 0; q < 8; ++q)
                        *reinterpret_cast<float4*>(o + 4 * q) =
                            make_float4(a[t][j][4 * q], a[t][j][4 * q + 1], a[t][j][4 * q + 2], a[t][j][4 * q + 3]);
                }
            }
        }
    }
    // router rows of this wave, RPB at a time; lane l ends up with value l >> 2
    // of the batch (value v = row_i * TB + t)
    for (uint32_t r0 = wv * RPB; r0 < d.E; r0 += ROUTE_WAVES * RPB) {
        float part[RPB * TB];
#pragma unroll
        for (int i = 0; i < RPB; ++i) {
            const uint16_t* wr = L.router_w + static_cast<size_t>(min(r0 + i, d.E - 1)) * D;
            uint4 rw[CPL][4];
#pragma unroll
            for (int j = 0; j < CPL; ++j) {
                const uint32_t c = min(lane + WAVE * j, nch - 1);
#pragma unroll
                for (int q = 0; q < 4; ++q) rw[j][q] = load_u4(wr + c * 32 + q * 8);
            }
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
        const uint32_t v = lane >> 2;
        const uint32_t row = r0 + v / TB;
        if ((lane & 3) == 0 && row < d.E && row < r0 + RPB) s_logit[v % TB][row] = tot;
    }
    __syncthreads();
    if (wv < TB && t0 + wv < T) {
        float p[VPL];
#pragma unroll
        for (int j = 0; j < VPL; ++j) {
            const uint32_t pos = lane + WAVE * j;
            p[j] = pos < d.E ? s_logit[wv][pos] : -INFINITY;
        }
        uint32_t my_id;
        float my_w;
        const uint32_t count = topk_fast<VPL>(p, d.E, d.K, d.norm_topk, my_id, my_w);
        if (static_cast<uint32_t>(lane) < count) {
            ids[static_cast<size_t>(t0 + wv) * d.K + lane] = my_id;
            w[static_cast<size_t>(t0 + wv) * d.K + lane] = my_w;
        }
    }
}

// ---------------------------------------------------------------------------
// k_split_rows: src [rows x cols] fp32 -> f16 planes hi/lo of x * 2^-e per
// (row, 64-column group) with |x| < 2^e, and st[row][group] = (sum of
// hi + lo over the group, 2^e).  One wave per (row, group).
// ---------------------------------------------------------------------------
__global__ __launch_bounds__(256)
void k_split_rows(const float* __restrict__ src, uint32_t rows, uint32_t cols, uint16_t* __restrict__ hi,
                  uint16_t* __restrict__ lo, float2* __restrict__ st)
{
    const int lane = threadIdx.x & 63;
    const uint32_t G = cols >> 6, total = rows * G;
    for (uint32_t it = blockIdx.x * 4 + (threadIdx.x >> 6); it < total; it += gridDim.x * 4) {
        const uint32_t r = it / G, g = it - r * G;
        const size_t o = static_cast<size_t>(r) * cols + g * 64 + lane;
        const float x = src[o];
        const float amax = wave_max(fabsf(x));
        const int e = amax > 0.f ? __builtin_amdgcn_frexp_expf(amax) : 0;
        const float xs = __builtin_ldexpf(x, -e);
        const _Float16 h = static_cast<_Float16>(xs);
        const _Float16 l = static_cast<_Float16>(xs - static_cast<float>(h));
        hi[o] = __builtin_bit_cast(uint16_t, h);
        lo[o] = __builtin_bit_cast(uint16_t, l);
        const float sum = wave_sum(static_cast<float>(h) + static_cast<float>(l));
        if (lane == 0) st[it] = make_float2(sum, __builtin_ldexpf(1.0f, e));
    }
}

// ---------------------------------------------------------------------------
// k_permute: stable counting sort of the P = T*k pairs p = t*k + r by expert
// ids[p] (prefill.cpp:38-68 builds the same per-expert lists, ascending token
// order), in one workgroup.  Chunk c = pairs [64c, 64c + 64) is one wave's
// step: per-(chunk, expert) counts in LDS, prefix over (expert, chunk), then
// each pair's slot = prefix + its rank among equal ids earlier in the chunk.
// Union order (first appearance, token-major, prefill.cpp:55-68) ranks the
// touched experts by their first pair.  ids >= E are skipped and flagged in
// err (bit 1).
// ---------------------------------------------------------------------------
constexpr int PERM_THREADS = 1024;

__global__ __launch_bounds__(PERM_THREADS)
void k_permute(const uint32_t* __restrict__ ids, const float* __restrict__ w, uint32_t P, uint32_t K, uint32_t E,
               uint32_t* __restrict__ offsets, uint32_t* __restrict__ sorted_pairs,
               uint32_t* __restrict__ sorted_tokens, float* __restrict__ sorted_w, uint32_t* __restrict__ union_ids,
               uint32_t* __restrict__ union_size, uint32_t* __restrict__ err)
{
    extern __shared__ uint32_t s_mem[];
    const uint32_t C = (P + 63) / 64;
    uint32_t* s_cnt = s_mem;               // [C x E]
    uint32_t* s_first = s_cnt + C * E;     // [E]
    uint32_t* s_tot = s_first + E;         // [E]
    uint32_t* s_off = s_tot + E;           // [E + 1]
    const int lane = threadIdx.x & 63, wv = threadIdx.x >> 6;
    constexpr int NW = PERM_THREADS / WAVE;

    for (uint32_t i = threadIdx.x; i < C * E; i += PERM_THREADS) s_cnt[i] = 0;
    for (uint32_t i = threadIdx.x; i < E; i += PERM_THREADS) s_first[i] = 0xFFFFFFFFu;
    __syncthreads();
    for (uint32_t c = wv; c < C; c += NW) {
        const uint32_t p = c * 64 + lane;
        if (p < P) {
            const uint32_t e = ids[p];
            if (e < E) {
                atomicAdd(&s_cnt[c * E + e], 1u);
                atomicMin(&s_first[e], p);
            } else {
                atomicOr(err, 2u);
            }
        }
    }
    __syncthreads();
    // per expert: counts -> exclusive prefix over chunks
    for (uint32_t e = threadIdx.x; e < E; e += PERM_THREADS) {
        uint32_t run = 0;
        for (uint32_t c = 0; c < C; ++c) {
            const uint32_t t = s_cnt[c * E + e];
            s_cnt[c * E + e] = run;
            run += t;
        }
        s_tot[e] = run;
    }
    __syncthreads();
    if (threadIdx.x == 0) {
        uint32_t run = 0;
        for (uint32_t e = 0; e < E; ++e) {
            s_off[e] = run;
            run += s_tot[e];
        }
        s_off[E] = run;
    }
    __syncthreads();
    for (uint32_t e = threadIdx.x; e <= E; e += PERM_THREADS) offsets[e] = s_off[e];
    // scatter: rank among equal ids of lower lanes of the same chunk
    for (uint32_t c = wv; c < C; c += NW) {
        const uint32_t p = c * 64 + lane;
        const uint32_t e = p < P ? ids[p] : 0xFFFFFFFFu;
        const bool ok = e < E;
        uint32_t rank = 0;
        for (uint64_t todo = __ballot(ok); todo != 0;) {
            const uint32_t ev = readlane_u32(e, __builtin_ctzll(todo));
            const uint64_t m = __ballot(ok && e == ev);
            if (ok && e == ev) rank = __popcll(m & ((1ull << lane) - 1ull));
            todo &= ~m;
        }
        if (ok) {
            const uint32_t dst = s_off[e] + s_cnt[c * E + e] + rank;
            sorted_pairs[dst] = p;
            if (sorted_tokens) sorted_tokens[dst] = p / K;
            if (sorted_w) sorted_w[dst] = w[p];
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
}

// ---------------------------------------------------------------------------
// k_grouped_mm: for each expert e with M = offsets[e+1] - offsets[e] pairs,
// out[pair][n] over a 64-row tile of its weight matrix (gate+up or down).
// Block = 4 waves, wave w owns rows n0 + 16 w .. + 16; a pass covers 32
// pairs as two 16-row MFMA tiles.  v_mfma_f32_16x16x32_f16 operand layout:
// lane l holds A[l % 16][8 (l / 16) + j] and B[8 (l / 16) + j][l % 16]
// (j < 8) and receives D[4 (l / 16) + i][l % 16] (i < 4).  Inside a 64-column
// group, lane quarter q = l / 16 of MFMA step s uses physical columns
// 16 q + 8 s + j, so each lane reads 8 contiguous bytes of packed weights and
// 32 contiguous bytes of each activation plane per group.
// ---------------------------------------------------------------------------
constexpr int MM_WAVES = 4;
constexpr int MM_ROWS = 16 * MM_WAVES;   // weight rows per block
constexpr int MM_PASS = 32;              // pairs per pass

// eight codes (one dword, low nibble first) -> f16 (c - 8), exact.
// The bias is added to the whole half8 at once: assembling the half8 element
// by element from four half2 sums was miscompiled by this toolchain (hipcc
// 7.2, gfx950: the four pairs collapsed into copies of the first).
__device__ __forceinline__ half8_t q4_codes_to_f16(uint32_t v)
{
    const uint32_t E = v & 0x0F0F0F0Fu;          // codes 0, 2, 4, 6
    const uint32_t O = (v >> 4) & 0x0F0F0F0Fu;   // codes 1, 3, 5, 7
    // f16 bits 0x6400 | c = 1024 + c exactly; minus 1032 -> c - 8 exactly
    u32x4_t r;
    r.x = __builtin_amdgcn_perm(O, E, 0x0C040C00u) | 0x64006400u;
    r.y = __builtin_amdgcn_perm(O, E, 0x0C050C01u) | 0x64006400u;
    r.z = __builtin_amdgcn_perm(O, E, 0x0C060C02u) | 0x64006400u;
    r.w = __builtin_amdgcn_perm(O, E, 0x0C070C03u) | 0x64006400u;
    const _Float16 b = static_cast<_Float16>(-1032.0f);
    const half8_t bias = {b, b, b, b, b, b, b, b};
    return __builtin_bit_cast(half8_t, r) + bias;
}

__device__ __forceinline__ half8_t load_half8(const uint16_t* p)
{
    const uint4 v = load_u4(p);
    u32x4_t u;
    u.x = v.x; u.y = v.y; u.z = v.z; u.w = v.w;
    return __builtin_bit_cast(half8_t, u);
}

template <bool GATE_UP>
__global__ __launch_bounds__(MM_WAVES * WAVE)
void k_grouped_mm(MoeDims d, LayerDesc L, const uint32_t* __restrict__ offsets,
                  const uint32_t* __restrict__ sorted_pairs, const uint16_t* __restrict__ a_hi,
                  const uint16_t* __restrict__ a_lo, const float2* __restrict__ a_st, uint32_t a_row_div,
                  float* __restrict__ out, uint32_t n_dim, uint32_t k_dim, uint32_t n_tiles)
{
    constexpr int NM = GATE_UP ? 2 : 1;
    __shared__ uint32_t s_row[MM_PASS];    // activation row of pass pair m
    __shared__ uint32_t s_pair[MM_PASS];
    const int lane = threadIdx.x & 63, wv = threadIdx.x >> 6;
    const uint32_t b = blockIdx.x, xcd = b & 7u, j = b >> 3;
    const uint32_t e = xcd + 8u * (j / n_tiles), tile = j % n_tiles;
    if (e >= d.E) return;
    const uint32_t base = offsets[e], M = offsets[e + 1] - base;
    if (M == 0) return;

    const uint32_t G = k_dim >> 6;
    const uint32_t n = tile * MM_ROWS + wv * 16 + (lane & 15);
    const uint32_t q = lane >> 4;
    const uint8_t* blob = L.experts + static_cast<size_t>(e) * L.stride;
    const uint8_t* wp[NM];
    const uint16_t* sp[NM];
    if (GATE_UP) {
        wp[0] = blob + L.off[0];
        sp[0] = reinterpret_cast<const uint16_t*>(blob + L.off[1]);
        wp[NM - 1] = blob + L.off[2];
        sp[NM - 1] = reinterpret_cast<const uint16_t*>(blob + L.off[3]);
    } else {
        wp[0] = blob + L.off[4];
        sp[0] = reinterpret_cast<const uint16_t*>(blob + L.off[5]);
    }
    const size_t row_bytes = k_dim >> 1;

    for (uint32_t m0 = 0; m0 < M; m0 += MM_PASS) {
        __syncthreads();
        if (threadIdx.x < MM_PASS) {
            const uint32_t p = sorted_pairs[base + min(m0 + threadIdx.x, M - 1)];
            s_pair[threadIdx.x] = p;
            s_row[threadIdx.x] = p / a_row_div;
        }
        __syncthreads();
        // A-operand rows of this lane (row l % 16 of each 16-pair tile)
        const uint16_t* ah[2];
        const uint16_t* al[2];
#pragma unroll
        for (int ms = 0; ms < 2; ++ms) {
            const size_t r = s_row[16 * ms + (lane & 15)];
            ah[ms] = a_hi + r * k_dim + 16 * q;
            al[ms] = a_lo + r * k_dim + 16 * q;
        }
        // epilogue rows of this lane: D rows 4 q + i of each tile
        uint32_t er[2][4];
#pragma unroll
        for (int ms = 0; ms < 2; ++ms)
#pragma unroll
            for (int i = 0; i < 4; ++i) er[ms][i] = s_row[16 * ms + 4 * q + i];

        f32x4_t acc[2][NM];
#pragma unroll
        for (int ms = 0; ms < 2; ++ms)
#pragma unroll
            for (int mt = 0; mt < NM; ++mt) acc[ms][mt] = f32x4_t{0.f, 0.f, 0.f, 0.f};

        for (uint32_t g = 0; g < G; ++g) {
            uint2 wq[NM];
            float sc[NM];
#pragma unroll
            for (int mt = 0; mt < NM; ++mt) {
                const uint8_t* wr = wp[mt] + n * row_bytes + g * 32 + 8 * q;
                wq[mt].x = __builtin_nontemporal_load(gptr(reinterpret_cast<const uint32_t*>(wr)));
                wq[mt].y = __builtin_nontemporal_load(gptr(reinterpret_cast<const uint32_t*>(wr) + 1));
                sc[mt] = f16_bits_to_f32(load_stream_u16(sp[mt] + static_cast<size_t>(n) * G + g));
            }
            half8_t xa[2][2][2];   // [ms][step][hi/lo]
#pragma unroll
            for (int ms = 0; ms < 2; ++ms) {
#pragma unroll
                for (int s = 0; s < 2; ++s) {
                    xa[ms][s][0] = load_half8(ah[ms] + g * 64 + 8 * s);
                    xa[ms][s][1] = load_half8(al[ms] + g * 64 + 8 * s);
                }
            }
            float2 st[2][4];
#pragma unroll
            for (int ms = 0; ms < 2; ++ms)
#pragma unroll
                for (int i = 0; i < 4; ++i) st[ms][i] = a_st[static_cast<size_t>(er[ms][i]) * G + g];
#pragma unroll
            for (int mt = 0; mt < NM; ++mt) {
                const half8_t b0 = q4_codes_to_f16(wq[mt].x);
                const half8_t b1 = q4_codes_to_f16(wq[mt].y);
#pragma unroll
                for (int ms = 0; ms < 2; ++ms) {
                    f32x4_t t = {0.f, 0.f, 0.f, 0.f};
                    t = __builtin_amdgcn_mfma_f32_16x16x32_f16(xa[ms][0][0], b0, t, 0, 0, 0);
                    t = __builtin_amdgcn_mfma_f32_16x16x32_f16(xa[ms][0][1], b0, t, 0, 0, 0);
                    t = __builtin_amdgcn_mfma_f32_16x16x32_f16(xa[ms][1][0], b1, t, 0, 0, 0);
                    t = __builtin_amdgcn_mfma_f32_16x16x32_f16(xa[ms][1][1], b1, t, 0, 0, 0);
#pragma unroll
                    for (int i = 0; i < 4; ++i)
                        acc[ms][mt][i] = fmaf(sc[mt] * st[ms][i].y, fmaf(0.5f, st[ms][i].x, t[i]), acc[ms][mt][i]);
                }
            }
        }
        // outputs: pair rows 4 q + i of each tile, column n
#pragma unroll
        for (int ms = 0; ms < 2; ++ms) {
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                const uint32_t m = 16 * ms + 4 * q + i;
                if (m0 + m >= M) continue;
                float* o = out + static_cast<size_t>(s_pair[m]) * n_dim + n;
                const float v0 = acc[ms][0][i] * (1.0f / 7.5f);
                if (GATE_UP) {
                    const float v1 = acc[ms][NM - 1][i] * (1.0f / 7.5f);
                    // h = silu(g) * u, silu(z) = z * (1 / (1 + exp(-z)))  (kernels.metal:61-63)
                    *o = (v0 * (1.0f / (1.0f + expf(-v0)))) * v1;
                } else {
                    *o = v0;
                }
            }
        }
    }
}

// ---------------------------------------------------------------------------
// k_combine_pairs: hidden[t][col] += sum_r w[t k + r] * y[(t k + r)][col], in
// rank order (the scatter-add of prefill.cpp:380-385 then :446-451).
// ---------------------------------------------------------------------------
__global__ __launch_bounds__(256)
void k_combine_pairs(const float* __restrict__ y, const float* __restrict__ w, uint32_t K, uint32_t D,
                     float* __restrict__ hidden)
{
    const uint32_t t = blockIdx.y, col = blockIdx.x * 256 + threadIdx.x;
    if (col >= D) return;
    float acc = 0.f;
    for (uint32_t r = 0; r < K; ++r) {
        const size_t p = static_cast<size_t>(t) * K + r;
        acc = fmaf(w[p], y[p * D + col], acc);
    }
    float* h = hidden + static_cast<size_t>(t) * D + col;
    *h = *h + acc;
}

// ---------------------------------------------------------------------------
// launchers
// ---------------------------------------------------------------------------
template <int CPL, int TB>
static hipError_t route_c(const MoeDims& d, const LayerDesc& L, const float* hidden, uint32_t T, float* normed,
                          uint32_t* ids, float* w, hipStream_t s)
{
    const dim3 grid((T + TB - 1) / TB), block(ROUTE_WAVES * WAVE);
    if (d.E <= 128)
        launch_kernel(k_route<CPL, TB, 2>, grid, block, s, d, L, hidden, T, normed, ids, w);
    else
        launch_kernel(k_route<CPL, TB, 8>, grid, block, s, d, L, hidden, T, normed, ids, w);
    return hipGetLastError();
}

hipError_t launch_route(const MoeDims& d, const LayerDesc& L, const float* hidden, uint32_t T, float* normed,
                        uint32_t* ids, float* w, hipStream_t s)
{
    if (d.E > SMOE_TOPK_MAX_N || d.K > SMOE_TOPK_MAX_K || d.D % 64 || T == 0) return hipErrorInvalidValue;
    const uint32_t cpl = (d.D / 32 + WAVE - 1) / WAVE;
    if (cpl == 1) return route_c<1, 4>(d, L, hidden, T, normed, ids, w, s);
    if (cpl == 2) return route_c<2, 2>(d, L, hidden, T, normed, ids, w, s);
    if (cpl <= 4) return route_c<4, 1>(d, L, hidden, T, normed, ids, w, s);
    return hipErrorInvalidValue;
}

hipError_t launch_split_rows(const float* src, uint32_t rows, uint32_t cols, uint16_t* hi, uint16_t* lo,
                             float2* st, hipStream_t s)
{
    if (cols % 64 || rows == 0) return hipErrorInvalidValue;
    const uint32_t items = rows * (cols / 64);
    const uint32_t blocks = std::min<uint32_t>((items + 3) / 4, 8192u);
    launch_kernel(k_split_rows, dim3(blocks), dim3(256), s, src, rows, cols, hi, lo, st);
    return hipGetLastError();
}

size_t permute_lds_bytes(uint32_t P, uint32_t E)
{
    const size_t C = (P + 63) / 64;
    return (C * E + 3 * size_t(E) + 1) * sizeof(uint32_t);
}

hipError_t launch_permute(const uint32_t* ids, const float* w, uint32_t P, uint32_t K, uint32_t E, uint32_t* offsets,
                          uint32_t* sorted_pairs, uint32_t* sorted_tokens, float* sorted_w, uint32_t* union_ids,
                          uint32_t* union_size, uint32_t* err, hipStream_t s)
{
    const size_t lds = permute_lds_bytes(P, E);
    if (P == 0 || E == 0 || lds > PERMUTE_MAX_LDS) return hipErrorInvalidValue;
    launch_kernel_lds(k_permute, dim3(1), dim3(PERM_THREADS), static_cast<uint32_t>(lds), s, ids, w, P, K, E,
                      offsets, sorted_pairs, sorted_tokens, sorted_w, union_ids, union_size, err);
    return hipGetLastError();
}

hipError_t launch_grouped_gate_up(const MoeDims& d, const LayerDesc& L, const uint32_t* offsets,
                                  const uint32_t* sorted_pairs, const uint16_t* x_hi, const uint16_t* x_lo,
                                  const float2* x_st, float* h, hipStream_t s)
{
    if (d.group != 64 || d.I % MM_ROWS || d.D % 64) return hipErrorInvalidValue;
    const uint32_t n_tiles = d.I / MM_ROWS, eg = (d.E + 7) / 8;
    launch_kernel(k_grouped_mm<true>, dim3(8 * eg * n_tiles), dim3(MM_WAVES * WAVE), s, d, L, offsets, sorted_pairs,
                  x_hi, x_lo, x_st, d.K, h, d.I, d.D, n_tiles);
    return hipGetLastError();
}

hipError_t launch_grouped_down(const MoeDims& d, const LayerDesc& L, const uint32_t* offsets,
                               const uint32_t* sorted_pairs, const uint16_t* h_hi, const uint16_t* h_lo,
                               const float2* h_st, float* y, hipStream_t s)
{
    if (d.group != 64 || d.D % MM_ROWS || d.I % 64) return hipErrorInvalidValue;
    const uint32_t n_tiles = d.D / MM_ROWS, eg = (d.E + 7) / 8;
    launch_kernel(k_grouped_mm<false>, dim3(8 * eg * n_tiles), dim3(MM_WAVES * WAVE), s, d, L, offsets,
                  sorted_pairs, h_hi, h_lo, h_st, 1u, y, d.D, d.I, n_tiles);
    return hipGetLastError();
}

hipError_t launch_combine_pairs(const float* y, const float* w, uint32_t T, uint32_t K, uint32_t D, float* hidden,
                                hipStream_t s)
{
    launch_kernel(k_combine_pairs, dim3((D + 255) / 256, T), dim3(256), s, y, w, K, D, hidden);
    return hipGetLastError();
}

}  // namespace smoe
