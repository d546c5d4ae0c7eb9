// trunk.hip -- dense-trunk kernels on either side of the MoE block (gfx950):
// bf16 GEMVs for the attention projections and the single-token decode
// attention of metal_bridge.h:166-196 (kernels.metal:421-652; CPU form
// decode.cpp:150-229).
//
//   k_gemv_bf16     y[r] = sum_c bf16(W[r][c]) * x[c] (common.hpp:293-306) for
//                   up to GEMV_MAX matrices in one launch.  A 4-wave block owns
//                   4 * RPW rows; x goes out to LDS with its loads issued ahead
//                   of the weight stream (vector-memory returns are in order),
//                   every lane streams NB 16-byte chunks (8 weights) of each of
//                   its wave's RPW rows, all in flight before the FMAs.  RPW is
//                   picked so the launch holds thousands of waves.
//   k_attn_decode   one block per (KV head, group of query heads, context
//                   split), eight waves:
//                     1. the group's query heads: RMSNorm (eps 1e-6, skipped
//                        without norm weights), RoPE on the pairs
//                        (d, d + head_dim/2) (decode.cpp:155-186); in split 0
//                        also the new K row, and K and V appended to the ring
//                        at `slot` (decode.cpp:188-189);
//                     2. the split's positions (position i counts back from
//                        slot, decode.cpp:196-205) in tiles: head_dim/8 lanes
//                        hold the 8-float pieces of one K and V row, each K
//                        row is read once for all query heads of the group;
//                        scores by a segmented butterfly, an online softmax
//                        per wave (running maximum, rescaled sums);
//                     3. the waves merged in LDS: with one split the output
//                        normalised (softmax, decode.cpp:207-226), else the
//                        block's partial (maximum, sum, weighted V) stored.
//   k_attn_combine  the splits of each head rescaled to their common maximum
//                   and normalised.  A kernel of its own: the launch boundary
//                   publishes every partial at once, where an in-kernel
//                   last-block combine needs an agent-scope release per wave
//                   (a full L2 write-back each, serialised per XCD).
#include <algorithm>

#include "device_common.hpp"
#include "kernels.hpp"

namespace smoe {

// ---------------------------------------------------------------------------
// grouped bf16 GEMV
// ---------------------------------------------------------------------------
constexpr int GV_WAVES = 4;
constexpr int GV_THREADS = GV_WAVES * WAVE;

template <int RPW, int NB>
__global__ __launch_bounds__(GV_THREADS)
void k_gemv_bf16(GemvGroup g)
{
    extern __shared__ __align__(16) float xs[];
    // the matrix of this block
    uint32_t m = 0;
    while (m + 1 < g.count && blockIdx.x >= g.block0[m + 1]) ++m;
    const uint16_t* __restrict__ W = g.w[m];
    const float* __restrict__ x = g.x[m];
    float* __restrict__ y = g.y[m];
    const uint32_t rows = g.rows[m], cols = g.cols[m];
    const uint32_t r0 = (blockIdx.x - g.block0[m]) * (GV_WAVES * RPW);
    const int lane = threadIdx.x & 63, wv = threadIdx.x >> 6;
    const uint32_t nch = cols >> 3;             // 8-weight chunks per row
    const uint32_t nx4 = cols >> 2;             // float4 of x

    // x of the first NB * 512 columns: loads issued before the weights'
    constexpr int XPT = NB >= 2 ? NB / 2 : 1;
    float4 xr[XPT];
#pragma unroll
    for (int i = 0; i < XPT; ++i) {
        const uint32_t c4 = threadIdx.x + i * GV_THREADS;
        xr[i] = c4 < nx4 ? load_f4(x + 4 * c4) : make_float4(0.f, 0.f, 0.f, 0.f);
    }
    const uint16_t* wr[RPW];
#pragma unroll
    for (int i = 0; i < RPW; ++i)
        wr[i] = W + static_cast<size_t>(min(r0 + wv * RPW + i, rows - 1)) * cols;
    uint4 v[NB][RPW];
    auto load_batch = [&](uint32_t c0) {
#pragma unroll
        for (int b = 0; b < NB; ++b) {
            const uint32_t c = min(c0 + b * WAVE, nch - 1);
#pragma unroll
            for (int i = 0; i < RPW; ++i) v[b][i] = load_stream_u4(wr[i] + c * 8);
        }
    };
    load_batch(lane);
#pragma unroll
    for (int i = 0; i < XPT; ++i) {
        const uint32_t c4 = threadIdx.x + i * GV_THREADS;
        if (c4 < nx4) *reinterpret_cast<float4*>(xs + 4 * c4) = xr[i];
    }
    for (uint32_t c4 = threadIdx.x + XPT * GV_THREADS; c4 < nx4; c4 += GV_THREADS)   // rows beyond NB * 512
        *reinterpret_cast<float4*>(xs + 4 * c4) = load_f4(x + 4 * c4);
    __syncthreads();

    float acc[RPW];
#pragma unroll
    for (int i = 0; i < RPW; ++i) acc[i] = 0.f;
    for (uint32_t c0 = lane;;) {
#pragma unroll
        for (int b = 0; b < NB; ++b) {
            const uint32_t c = c0 + b * WAVE;
            if (c >= nch) break;
            const float4 xa = *reinterpret_cast<const float4*>(xs + c * 8);
            const float4 xb = *reinterpret_cast<const float4*>(xs + c * 8 + 4);
#pragma unroll
            for (int i = 0; i < RPW; ++i) {
                float a = acc[i];
                a = fmaf(__uint_as_float(v[b][i].x << 16), xa.x, a);
                a = fmaf(__uint_as_float(v[b][i].x & 0xFFFF0000u), xa.y, a);
                a = fmaf(__uint_as_float(v[b][i].y << 16), xa.z, a);
                a = fmaf(__uint_as_float(v[b][i].y & 0xFFFF0000u), xa.w, a);
                a = fmaf(__uint_as_float(v[b][i].z << 16), xb.x, a);
                a = fmaf(__uint_as_float(v[b][i].z & 0xFFFF0000u), xb.y, a);
                a = fmaf(__uint_as_float(v[b][i].w << 16), xb.z, a);
                a = fmaf(__uint_as_float(v[b][i].w & 0xFFFF0000u), xb.w, a);
                acc[i] = a;
            }
        }
        c0 += NB * WAVE;
        if (c0 >= nch) break;
        load_batch(c0);
    }
    // lane l holds the total of row l >> (6 - log2 RPW)
    const float tot = wave_sum_rows<RPW>(acc);
    constexpr int LPR = WAVE / RPW;             // lanes per row after the reduction
    const uint32_t r = r0 + wv * RPW + lane / LPR;
    if ((lane & (LPR - 1)) == 0 && r < rows) y[r] = tot;
}

template <int RPW, int NB>
static void gemv_launch(const GemvGroup& g, uint32_t blocks, uint32_t lds, hipStream_t s)
{
    launch_kernel_lds(k_gemv_bf16<RPW, NB>, dim3(blocks), dim3(GV_THREADS), lds, s, g);
}

hipError_t launch_gemv_bf16(const GemvGroup& in, hipStream_t s)
{
    if (in.count == 0 || in.count > GEMV_MAX) return hipErrorInvalidValue;
    uint32_t total_rows = 0, max_cols = 0;
    for (uint32_t m = 0; m < in.count; ++m) {
        if (!in.w[m] || !in.x[m] || !in.y[m] || in.rows[m] == 0 || in.cols[m] == 0 || in.cols[m] % 8 ||
            in.cols[m] > GEMV_MAX_COLS)
            return hipErrorInvalidValue;
        total_rows += in.rows[m];
        max_cols = std::max(max_cols, in.cols[m]);
    }
    // NB: chunks per lane covering the longest row in one pass (at most 8);
    // RPW: rows per wave, 1 until the launch has 8192+ rows
    const uint32_t nch = max_cols / 8;
    const int nb = nch <= 64 ? 1 : nch <= 128 ? 2 : nch <= 256 ? 4 : 8;
    int rpw = total_rows >= 32768 ? 4 : total_rows >= 8192 ? 2 : 1;
    if (nb == 8 && rpw == 4) rpw = 2;
    GemvGroup g = in;
    uint32_t blocks = 0;
    const uint32_t rows_per_block = GV_WAVES * rpw;
    for (uint32_t m = 0; m < g.count; ++m) {
        g.block0[m] = blocks;
        blocks += (g.rows[m] + rows_per_block - 1) / rows_per_block;
    }
    const uint32_t lds = max_cols * 4u;
    switch (rpw * 16 + nb) {
        case 16 + 1: gemv_launch<1, 1>(g, blocks, lds, s); break;
        case 16 + 2: gemv_launch<1, 2>(g, blocks, lds, s); break;
        case 16 + 4: gemv_launch<1, 4>(g, blocks, lds, s); break;
        case 16 + 8: gemv_launch<1, 8>(g, blocks, lds, s); break;
        case 32 + 1: gemv_launch<2, 1>(g, blocks, lds, s); break;
        case 32 + 2: gemv_launch<2, 2>(g, blocks, lds, s); break;
        case 32 + 4: gemv_launch<2, 4>(g, blocks, lds, s); break;
        case 32 + 8: gemv_launch<2, 8>(g, blocks, lds, s); break;
        case 64 + 1: gemv_launch<4, 1>(g, blocks, lds, s); break;
        case 64 + 2: gemv_launch<4, 2>(g, blocks, lds, s); break;
        default:     gemv_launch<4, 4>(g, blocks, lds, s); break;
    }
    return hipGetLastError();
}

// ---------------------------------------------------------------------------
// decode attention
// ---------------------------------------------------------------------------
constexpr int AT_WAVES = 8;
constexpr int AT_THREADS = AT_WAVES * WAVE;
constexpr int AT_U = 2;                 // position steps per tile
constexpr int AT_MAX_GB = 8;            // query heads per block
constexpr int AT_MAX_GHD = 1024;        // query heads per block x head_dim

struct AttnArgs {
    AttnDims a;
    const float* q;
    const float* k;
    const float* v;
    const uint16_t* q_norm_w;
    const uint16_t* k_norm_w;
    const float* rope_cos;
    const float* rope_sin;
    float* k_cache;
    float* v_cache;
    float* part_ml;                     // [num_heads][ATTN_MAX_SPLITS][2]: maximum, sum
    float* part_acc;                    // [num_heads][ATTN_MAX_SPLITS][head_dim]
    float* out;
    uint32_t slot, valid, chunk, splits, n_sub;
};

// maximum / sum over the lane bits SEG .. 5 (the position groups of a wave)
template <int SEG>
__device__ __forceinline__ float high_max(float v)
{
    if constexpr (SEG <= 3) v = fmaxf(v, dpp_f32<DPP_ROW_ROR8>(-INFINITY, v));
    if constexpr (SEG <= 4) {
        const auto r = __builtin_amdgcn_permlane16_swap(__float_as_uint(v), __float_as_uint(v), false, false);
        v = fmaxf(__uint_as_float(r[0]), __uint_as_float(r[1]));
    }
    const auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(v), __float_as_uint(v), false, false);
    return fmaxf(__uint_as_float(r[0]), __uint_as_float(r[1]));
}
template <int SEG>
__device__ __forceinline__ float high_sum(float v)
{
    if constexpr (SEG <= 3) v += dpp_f32<DPP_ROW_ROR8>(0.f, v);
    if constexpr (SEG <= 4) swap16_sum(v, v);
    swap32_sum(v, v);
    return v;
}
// transposed sum over the lane bits B .. LOWEST (B = 5 first): each step
// halves the values a lane holds (bit clear: the lower half of the indices)
template <int B, int LOWEST, int M, int N>
__device__ __forceinline__ void high_split_steps(float (&a)[N], int lane)
{
    if constexpr (B >= LOWEST) {
#pragma unroll
        for (int i = 0; i < M / 2; ++i) red_bit<B, true>(a[i], a[i + M / 2], lane);
        high_split_steps<B - 1, LOWEST, M / 2>(a, lane);
    }
}

__device__ __forceinline__ float dot8(const float (&q)[8], float4 a, float4 b)
{
    float s = q[0] * a.x;
    s = fmaf(q[1], a.y, s);
    s = fmaf(q[2], a.z, s);
    s = fmaf(q[3], a.w, s);
    s = fmaf(q[4], b.x, s);
    s = fmaf(q[5], b.y, s);
    s = fmaf(q[6], b.z, s);
    s = fmaf(q[7], b.w, s);
    return s;
}

template <int HD, int GB>
__global__ __launch_bounds__(AT_THREADS)
void k_attn_decode(AttnArgs p)
{
    constexpr int LPP = HD / 8;                 // lanes per K / V row
    constexpr int SEG = ilog2(LPP);
    constexpr int P = WAVE / LPP;               // rows per wave step
    constexpr int TILE = P * AT_U;              // rows per wave tile
    constexpr int HALF = HD / 2;
    constexpr int DV = HD / WAVE;               // dims per lane in the norm pass
    constexpr int NV = GB * 8;                  // accumulators per lane
    constexpr int HB = 6 - SEG;                 // lane bits over the position groups
    constexpr int NVR = NV >> HB;               // accumulators per lane after the wave merge
    static_assert(GB * HD <= AT_MAX_GHD && NV >= (1 << HB), "block shape");

    __shared__ __align__(16) float qs[GB * HD];
    __shared__ __align__(16) float kn[HD];
    __shared__ __align__(16) float accw[AT_WAVES * GB * HD];
    __shared__ float mw[AT_WAVES * GB], lw[AT_WAVES * GB];

    const int lane = threadIdx.x & 63, wv = threadIdx.x >> 6;
    const uint32_t G = p.a.num_heads / p.a.num_kv_heads;
    const uint32_t kvh = blockIdx.x / p.n_sub, sg = blockIdx.x % p.n_sub, sp = blockIdx.y;
    const uint32_t hbase = kvh * G + sg * GB;   // first query head of the block
    const uint32_t ng = min(static_cast<uint32_t>(GB), G - sg * GB);
    const uint32_t S = p.splits;

    // ---- 1. query heads (and the new K row in split 0): RMSNorm ----------
    // rms_norm_bf16 per head (common.hpp:245-256): (x * inv) * w
    auto norm_head = [&](const float* src, const uint16_t* nw, float* dst, bool live) {
        float xv[DV];
#pragma unroll
        for (int j = 0; j < DV; ++j) xv[j] = live ? src[lane * DV + j] : 0.f;
        if (nw && live) {
            float ss = 0.f;
#pragma unroll
            for (int j = 0; j < DV; ++j) ss = fmaf(xv[j], xv[j], ss);
            ss = wave_sum(ss);
            const float inv = 1.0f / sqrtf(ss / static_cast<float>(HD) + 1e-6f);
#pragma unroll
            for (int j = 0; j < DV; ++j) xv[j] = (xv[j] * inv) * bf16_to_f32(nw[lane * DV + j]);
        }
#pragma unroll
        for (int j = 0; j < DV; ++j) dst[lane * DV + j] = xv[j];
    };
    for (int g = wv; g < GB; g += AT_WAVES)
        norm_head(p.q + static_cast<size_t>(hbase + g) * HD, p.q_norm_w, qs + g * HD, g < static_cast<int>(ng));
    if (sp == 0 && wv == AT_WAVES - 1)
        norm_head(p.k + static_cast<size_t>(kvh) * HD, p.k_norm_w, kn, true);
    __syncthreads();
    // RoPE in place: (x_d, x_{d+half}) rotated by angle d (decode.cpp:168-186)
    const uint32_t npairs = (GB + (sp == 0 ? 1 : 0)) * HALF;
    for (uint32_t t = threadIdx.x; t < npairs; t += AT_THREADS) {
        const uint32_t g = t / HALF, d = t % HALF;
        float* r = g < GB ? qs + g * HD : kn;
        const float c = p.rope_cos[d], sn = p.rope_sin[d];
        const float x0 = r[d], x1 = r[d + HALF];
        r[d] = x0 * c - x1 * sn;
        r[d + HALF] = x0 * sn + x1 * c;
    }
    __syncthreads();
    if (sp == 0) {
        // KV ring append (every split-0 block of this KV head writes the same
        // values); position 0 of the loop below reads them back
        for (uint32_t d = threadIdx.x; d < HD; d += AT_THREADS) {
            const size_t co = static_cast<size_t>(p.slot) * p.a.kv_dim + kvh * HD + d;
            p.k_cache[co] = kn[d];
            p.v_cache[co] = p.v[kvh * HD + d];
        }
        __syncthreads();
    }

    // ---- 2. the split's positions ------------------------------------------
    const int li = lane & (LPP - 1), pg = lane >> SEG;
    float qv[GB][8];
#pragma unroll
    for (int g = 0; g < GB; ++g) {
        const float4 a = *reinterpret_cast<const float4*>(qs + g * HD + li * 8);
        const float4 b = *reinterpret_cast<const float4*>(qs + g * HD + li * 8 + 4);
        qv[g][0] = a.x; qv[g][1] = a.y; qv[g][2] = a.z; qv[g][3] = a.w;
        qv[g][4] = b.x; qv[g][5] = b.y; qv[g][6] = b.z; qv[g][7] = b.w;
    }
    const uint32_t i0 = sp * p.chunk;
    const uint32_t n = min(p.chunk, p.valid - i0);
    const float* kbase = p.k_cache + kvh * HD + li * 8;
    const float* vbase = p.v_cache + kvh * HD + li * 8;
    const float scale = p.a.scale;
    float mx[GB], lsum[GB], acc[GB][8];
#pragma unroll
    for (int g = 0; g < GB; ++g) {
        mx[g] = -INFINITY;
        lsum[g] = 0.f;
#pragma unroll
        for (int e = 0; e < 8; ++e) acc[g][e] = 0.f;
    }
    for (uint32_t t0 = wv * TILE; t0 < n; t0 += AT_WAVES * TILE) {
        float4 kk[AT_U][2], vv[AT_U][2];
        bool ok[AT_U];
#pragma unroll
        for (int u = 0; u < AT_U; ++u) {
            const uint32_t pos = t0 + u * P + pg;
            ok[u] = pos < n;
            const uint32_t ip = i0 + min(pos, n - 1);
            const uint32_t ri = p.slot >= ip ? p.slot - ip : p.slot + p.a.ctx - ip;
            const size_t off = static_cast<size_t>(ri) * p.a.kv_dim;
            kk[u][0] = load_f4(kbase + off);
            kk[u][1] = load_f4(kbase + off + 4);
            vv[u][0] = load_f4(vbase + off);
            vv[u][1] = load_f4(vbase + off + 4);
        }
        float s[AT_U][GB];
#pragma unroll
        for (int u = 0; u < AT_U; ++u) {
            float d[GB];
#pragma unroll
            for (int g = 0; g < GB; ++g) d[g] = dot8(qv[g], kk[u][0], kk[u][1]);
            seg_allsum<GB, SEG>(d);
#pragma unroll
            for (int g = 0; g < GB; ++g) s[u][g] = ok[u] ? d[g] * scale : -INFINITY;
        }
#pragma unroll
        for (int g = 0; g < GB; ++g) {
            float mt = s[0][g];
#pragma unroll
            for (int u = 1; u < AT_U; ++u) mt = fmaxf(mt, s[u][g]);
            mt = high_max<SEG>(mt);             // wave-uniform
            if (mt > mx[g]) {
                const float f = __expf(mx[g] - mt);
                lsum[g] *= f;
#pragma unroll
                for (int e = 0; e < 8; ++e) acc[g][e] *= f;
                mx[g] = mt;
            }
#pragma unroll
            for (int u = 0; u < AT_U; ++u) {
                const float pe = __expf(s[u][g] - mx[g]);
                lsum[g] += pe;
                acc[g][0] = fmaf(pe, vv[u][0].x, acc[g][0]);
                acc[g][1] = fmaf(pe, vv[u][0].y, acc[g][1]);
                acc[g][2] = fmaf(pe, vv[u][0].z, acc[g][2]);
                acc[g][3] = fmaf(pe, vv[u][0].w, acc[g][3]);
                acc[g][4] = fmaf(pe, vv[u][1].x, acc[g][4]);
                acc[g][5] = fmaf(pe, vv[u][1].y, acc[g][5]);
                acc[g][6] = fmaf(pe, vv[u][1].z, acc[g][6]);
                acc[g][7] = fmaf(pe, vv[u][1].w, acc[g][7]);
            }
        }
    }

    // ---- 3. merge: position groups, then waves, then splits ---------------
#pragma unroll
    for (int g = 0; g < GB; ++g) lsum[g] = high_sum<SEG>(lsum[g]);
    float a2[NV];
#pragma unroll
    for (int g = 0; g < GB; ++g)
#pragma unroll
        for (int e = 0; e < 8; ++e) a2[g * 8 + e] = acc[g][e];
    high_split_steps<5, SEG, NV>(a2, lane);
    // lane holds the flat indices pg * NVR + k, k < NVR (flat = head * 8 + dim)
#pragma unroll
    for (int k = 0; k < NVR; ++k) {
        const int idx = pg * NVR + k;
        accw[(wv * GB + idx / 8) * HD + li * 8 + (idx & 7)] = a2[k];
    }
    if (lane < GB) {
        float mv = mx[0], lv = lsum[0];
#pragma unroll
        for (int g = 1; g < GB; ++g)
            if (lane == g) mv = mx[g], lv = lsum[g];
        mw[wv * GB + lane] = mv;
        lw[wv * GB + lane] = lv;
    }
    __syncthreads();
    for (uint32_t o = threadIdx.x; o < static_cast<uint32_t>(GB * HD); o += AT_THREADS) {
        const uint32_t g = o / HD, d = o % HD;
        if (g >= ng) continue;
        float M = -INFINITY;
#pragma unroll
        for (int w = 0; w < AT_WAVES; ++w) M = fmaxf(M, mw[w * GB + g]);
        float L = 0.f, A = 0.f;
#pragma unroll
        for (int w = 0; w < AT_WAVES; ++w) {
            const float f = __expf(mw[w * GB + g] - M);
            L = fmaf(f, lw[w * GB + g], L);
            A = fmaf(f, accw[(w * GB + g) * HD + d], A);
        }
        const uint32_t h = hbase + g;
        if (S == 1) {
            p.out[static_cast<size_t>(h) * HD + d] = A * (1.0f / L);
        } else {
            p.part_acc[(static_cast<size_t>(h) * ATTN_MAX_SPLITS + sp) * HD + d] = A;
            if (d == 0) {
                p.part_ml[(static_cast<size_t>(h) * ATTN_MAX_SPLITS + sp) * 2] = M;
                p.part_ml[(static_cast<size_t>(h) * ATTN_MAX_SPLITS + sp) * 2 + 1] = L;
            }
        }
    }
}

// one wave per (query head, 64 dims): the splits rescaled to their common
// maximum and normalised, out = sum_s f_s acc_s / sum_s f_s l_s with
// f_s = exp(m_s - max_s m_s); every split's load is in flight at once
__global__ __launch_bounds__(WAVE)
void k_attn_combine(const float* __restrict__ part_ml, const float* __restrict__ part_acc, uint32_t head_dim,
                    uint32_t splits, float* __restrict__ out)
{
    const uint32_t h = blockIdx.x, d = blockIdx.y * WAVE + threadIdx.x, lane = threadIdx.x;
    const float* ml = part_ml + static_cast<size_t>(h) * ATTN_MAX_SPLITS * 2;
    const float* acc = part_acc + static_cast<size_t>(h) * ATTN_MAX_SPLITS * head_dim + d;
    float a[ATTN_MAX_SPLITS];
#pragma unroll
    for (uint32_t s = 0; s < ATTN_MAX_SPLITS; ++s) a[s] = s < splits ? acc[static_cast<size_t>(s) * head_dim] : 0.f;
    const bool live = lane < splits;
    const float m_s = live ? ml[lane * 2] : -INFINITY;
    const float l_s = live ? ml[lane * 2 + 1] : 0.f;
    const float M = wave_max(m_s);
    const float f = live ? __expf(m_s - M) : 0.f;
    const float L = wave_sum(f * l_s);
    float o = 0.f;
#pragma unroll
    for (uint32_t s = 0; s < ATTN_MAX_SPLITS; ++s) o = fmaf(readlane_f32(f, s), a[s], o);
    out[static_cast<size_t>(h) * head_dim + d] = o * (1.0f / L);
}

AttnPlan attn_plan(const AttnDims& a, uint32_t valid)
{
    AttnPlan pl{};
    const uint32_t G = a.num_heads / a.num_kv_heads;
    uint32_t gb = 1;
    while (gb < G && gb < static_cast<uint32_t>(AT_MAX_GB) && gb * 2 * a.head_dim <= AT_MAX_GHD) gb *= 2;
    pl.gb = gb;
    pl.n_sub = (G + gb - 1) / gb;
    const uint32_t bx = a.num_kv_heads * pl.n_sub;
    // at least one tile per wave; about one block per CU (256) in all
    const uint32_t tile_all = AT_WAVES * (WAVE / (a.head_dim / 8)) * AT_U;
    const uint32_t cap = std::max<uint32_t>(1, std::min<uint32_t>(ATTN_MAX_SPLITS, (256 + bx - 1) / bx));
    uint32_t S = std::min<uint32_t>((valid + tile_all - 1) / tile_all, cap);
    S = std::max<uint32_t>(S, 1);
    pl.chunk = (valid + S - 1) / S;
    pl.splits = (valid + pl.chunk - 1) / pl.chunk;      // no empty split
    return pl;
}

// scratch: the maxima / sums, then the weighted V partials of every split
size_t attn_scratch_bytes(const AttnDims& a)
{
    return static_cast<size_t>(a.num_heads) * ATTN_MAX_SPLITS * (2 + a.head_dim) * sizeof(float);
}

template <int HD, int GB>
static void attn_launch(const AttnArgs& args, dim3 grid, hipStream_t s)
{
    launch_kernel(k_attn_decode<HD, GB>, grid, dim3(AT_THREADS), s, args);
}

hipError_t launch_attention(const AttnDims& a, const float* q, const float* k, const float* v,
                            const uint16_t* q_norm_w, const uint16_t* k_norm_w, const float* rope_cos,
                            const float* rope_sin, float* k_cache, float* v_cache, uint32_t slot, uint32_t valid,
                            void* scratch, float* attn_out, hipStream_t s)
{
    if ((a.head_dim != 64 && a.head_dim != 128 && a.head_dim != 256) || a.num_kv_heads == 0 ||
        a.num_heads % a.num_kv_heads || a.kv_dim != a.num_kv_heads * a.head_dim || valid == 0 || valid > a.ctx ||
        slot >= a.ctx || (reinterpret_cast<uintptr_t>(k_cache) | reinterpret_cast<uintptr_t>(v_cache)) % 16)
        return hipErrorInvalidValue;
    const AttnPlan pl = attn_plan(a, valid);
    AttnArgs args{};
    args.a = a;
    args.q = q;
    args.k = k;
    args.v = v;
    args.q_norm_w = q_norm_w;
    args.k_norm_w = k_norm_w;
    args.rope_cos = rope_cos;
    args.rope_sin = rope_sin;
    args.k_cache = k_cache;
    args.v_cache = v_cache;
    args.part_ml = static_cast<float*>(scratch);
    args.part_acc = args.part_ml + static_cast<size_t>(a.num_heads) * ATTN_MAX_SPLITS * 2;
    args.out = attn_out;
    args.slot = slot;
    args.valid = valid;
    args.chunk = pl.chunk;
    args.splits = pl.splits;
    args.n_sub = pl.n_sub;
    const dim3 grid(a.num_kv_heads * pl.n_sub, pl.splits);
    switch (a.head_dim * 16 + pl.gb) {
        case 64 * 16 + 1: attn_launch<64, 1>(args, grid, s); break;
        case 64 * 16 + 2: attn_launch<64, 2>(args, grid, s); break;
        case 64 * 16 + 4: attn_launch<64, 4>(args, grid, s); break;
        case 64 * 16 + 8: attn_launch<64, 8>(args, grid, s); break;
        case 128 * 16 + 1: attn_launch<128, 1>(args, grid, s); break;
        case 128 * 16 + 2: attn_launch<128, 2>(args, grid, s); break;
        case 128 * 16 + 4: attn_launch<128, 4>(args, grid, s); break;
        case 128 * 16 + 8: attn_launch<128, 8>(args, grid, s); break;
        case 256 * 16 + 1: attn_launch<256, 1>(args, grid, s); break;
        case 256 * 16 + 2: attn_launch<256, 2>(args, grid, s); break;
        default:           attn_launch<256, 4>(args, grid, s); break;
    }
    if (pl.splits > 1)
        launch_kernel(k_attn_combine, dim3(a.num_heads, a.head_dim / WAVE), dim3(WAVE), s, args.part_ml,
                      args.part_acc, a.head_dim, pl.splits, attn_out);
    return hipGetLastError();
}

}  // namespace smoe
