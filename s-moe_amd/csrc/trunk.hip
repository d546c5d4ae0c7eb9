// trunk.hip -- dense-trunk kernels on either side of the MoE block (gfx950):
// bf16 GEMVs for the attention projections and the single-token decode
// attention of metal_bridge.h:166-196 (kernels.metal:421-652; CPU form
// decode.cpp:150-229).
//
//   k_gemv_bf16     y[r] = sum_c bf16(W[r][c]) * x[c] (common.hpp:293-306) for
//                   up to GEMV_MAX matrices in one launch: a 4-wave block owns
//                   16 rows of one matrix, stages x in LDS, every lane streams
//                   16-byte chunks of 8 weights of 4 rows, all loads of a batch
//                   in flight before the FMAs; one transposed wave reduction
//                   per block row group.
//   k_attn_prep     per-head RMSNorm of Q and K (eps 1e-6, skipped without
//                   norm weights), RoPE on the pairs (d, d + head_dim/2), K and
//                   V appended to the KV ring at `slot` (decode.cpp:155-190).
//   k_attn_split    one block per (query head, context split): scores
//                   q . k * scale of the split's positions (position i counts
//                   back from slot, decode.cpp:196-205), their maximum, the
//                   exponentials and their sum, and sum_i e_i v_i over the
//                   split, as partials.
//   k_attn_combine  per head: the splits' partials rescaled to the global
//                   maximum and normalised (softmax, decode.cpp:207-226).
#include <algorithm>

#include "device_common.hpp"
#include "kernels.hpp"

namespace smoe {

// ---------------------------------------------------------------------------
// grouped bf16 GEMV
// ---------------------------------------------------------------------------
constexpr int GV_WAVES = 4;
constexpr int GV_RPW = 4;                       // rows per wave
constexpr int GV_ROWS = GV_WAVES * GV_RPW;      // rows per block
constexpr int GV_BATCH = 4;                     // 16-byte chunks per row and batch

__global__ __launch_bounds__(GV_WAVES * WAVE)
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
    const uint32_t r0 = (blockIdx.x - g.block0[m]) * GV_ROWS;
    for (uint32_t c = threadIdx.x * 4; c < cols; c += GV_WAVES * WAVE * 4)
        *reinterpret_cast<float4*>(xs + c) = load_f4(x + c);
    __syncthreads();

    const int lane = threadIdx.x & 63, wv = threadIdx.x >> 6;
    const uint32_t nch = cols >> 3;             // 8-weight chunks per row
    const uint16_t* wr[GV_RPW];
#pragma unroll
    for (int i = 0; i < GV_RPW; ++i)
        wr[i] = W + static_cast<size_t>(min(r0 + wv * GV_RPW + i, rows - 1)) * cols;
    float acc[GV_RPW] = {0.f, 0.f, 0.f, 0.f};
    for (uint32_t c0 = lane; c0 < nch; c0 += GV_BATCH * WAVE) {
        uint4 v[GV_BATCH][GV_RPW];
#pragma unroll
        for (int b = 0; b < GV_BATCH; ++b) {
            const uint32_t c = min(c0 + b * WAVE, nch - 1);
#pragma unroll
            for (int i = 0; i < GV_RPW; ++i) v[b][i] = load_stream_u4(wr[i] + c * 8);
        }
#pragma unroll
        for (int b = 0; b < GV_BATCH; ++b) {
            const uint32_t c = c0 + b * WAVE;
            if (c >= nch) break;
            const float4 xa = *reinterpret_cast<const float4*>(xs + c * 8);
            const float4 xb = *reinterpret_cast<const float4*>(xs + c * 8 + 4);
#pragma unroll
            for (int i = 0; i < GV_RPW; ++i) {
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
    }
    // lane l holds the total of row l >> 4
    const float tot = wave_sum_rows<GV_RPW>(acc);
    const uint32_t r = r0 + wv * GV_RPW + (lane >> 4);
    if ((lane & 15) == 0 && r < rows) y[r] = tot;
}

hipError_t launch_gemv_bf16(const GemvGroup& in, hipStream_t s)
{
    if (in.count == 0 || in.count > GEMV_MAX) return hipErrorInvalidValue;
    GemvGroup g = in;
    uint32_t blocks = 0, max_cols = 0;
    for (uint32_t m = 0; m < g.count; ++m) {
        if (!g.w[m] || !g.x[m] || !g.y[m] || g.rows[m] == 0 || g.cols[m] == 0 || g.cols[m] % 8 ||
            g.cols[m] > GEMV_MAX_COLS)
            return hipErrorInvalidValue;
        g.block0[m] = blocks;
        blocks += (g.rows[m] + GV_ROWS - 1) / GV_ROWS;
        max_cols = std::max(max_cols, g.cols[m]);
    }
    launch_kernel_lds(k_gemv_bf16, dim3(blocks), dim3(GV_WAVES * WAVE), max_cols * 4u, s, g);
    return hipGetLastError();
}

// ---------------------------------------------------------------------------
// decode attention
// ---------------------------------------------------------------------------
// one block per Q head (blockIdx.x < num_heads) or K head, head_dim threads
__global__ __launch_bounds__(ATTN_MAX_HEAD_DIM)
void k_attn_prep(AttnDims a, float* __restrict__ q, float* __restrict__ k, const float* __restrict__ v,
                 const uint16_t* __restrict__ q_norm_w, const uint16_t* __restrict__ k_norm_w,
                 const float* __restrict__ rope_cos, const float* __restrict__ rope_sin, float* __restrict__ k_cache,
                 float* __restrict__ v_cache, uint32_t slot)
{
    __shared__ float vec[ATTN_MAX_HEAD_DIM];
    __shared__ float red[ATTN_MAX_HEAD_DIM / WAVE];
    const bool is_q = blockIdx.x < a.num_heads;
    const uint32_t h = is_q ? blockIdx.x : blockIdx.x - a.num_heads;
    float* head = (is_q ? q : k) + static_cast<size_t>(h) * a.head_dim;
    const uint16_t* nw = is_q ? q_norm_w : k_norm_w;
    const uint32_t t = threadIdx.x;
    float x = head[t];
    if (nw) {
        // rms_norm_bf16 on the head (common.hpp:245-256): normed = (x * inv) * w
        const float ss = wave_sum(x * x);
        if ((t & 63) == 0) red[t >> 6] = ss;
        __syncthreads();
        float tot = 0.f;
        for (uint32_t i = 0; i < a.head_dim / WAVE; ++i) tot += red[i];
        const float inv = 1.0f / sqrtf(tot / static_cast<float>(a.head_dim) + 1e-6f);
        x = (x * inv) * bf16_to_f32(nw[t]);
    }
    vec[t] = x;
    __syncthreads();
    // RoPE: (d, d + half) rotate by angle d (decode.cpp:168-186)
    const uint32_t half = a.head_dim >> 1;
    float r;
    if (t < half) {
        r = vec[t] * rope_cos[t] - vec[t + half] * rope_sin[t];
    } else {
        const uint32_t d = t - half;
        r = vec[d] * rope_sin[d] + vec[t] * rope_cos[d];
    }
    if (is_q) {
        head[t] = r;
    } else {
        const size_t co = static_cast<size_t>(slot) * a.kv_dim + static_cast<size_t>(h) * a.head_dim + t;
        k_cache[co] = r;
        v_cache[co] = v[static_cast<size_t>(h) * a.head_dim + t];
    }
}

// one block per (query head, split of the context); DPL = head_dim / 64
// dimensions per lane
template <int DPL>
__global__ __launch_bounds__(ATTN_THREADS)
void k_attn_split(AttnDims a, const float* __restrict__ q, const float* __restrict__ k_cache,
                  const float* __restrict__ v_cache, uint32_t slot, uint32_t valid, uint32_t chunk,
                  float* __restrict__ part)
{
    extern __shared__ __align__(16) float sc[];           // scores of the split, then reduction scratch
    constexpr int NW = ATTN_THREADS / WAVE;
    constexpr int GP = 8;                                 // positions per wave step
    const int lane = threadIdx.x & 63, wv = threadIdx.x >> 6;
    const uint32_t h = blockIdx.x, sp = blockIdx.y;
    const uint32_t i0 = sp * chunk, i1 = min(valid, i0 + chunk);
    const uint32_t n = i1 > i0 ? i1 - i0 : 0;
    const uint32_t kv_off = (h / (a.num_heads / a.num_kv_heads)) * a.head_dim;
    float qv[DPL];
#pragma unroll
    for (int j = 0; j < DPL; ++j) qv[j] = q[static_cast<size_t>(h) * a.head_dim + lane * DPL + j];
    auto row = [&](const float* base, uint32_t i) {
        const uint32_t ri = (slot + a.ctx - i) % a.ctx;   // position i counts back from slot
        return base + static_cast<size_t>(ri) * a.kv_dim + kv_off + lane * DPL;
    };
    // scores, 8 positions per wave step (padding positions re-read the last one)
    for (uint32_t b = wv * GP; b < n; b += NW * GP) {
        float part_dot[GP];
#pragma unroll
        for (int p = 0; p < GP; ++p) {
            const float* kr = row(k_cache, i0 + min(b + p, n - 1));
            float acc = 0.f;
#pragma unroll
            for (int j = 0; j < DPL; ++j) acc = fmaf(qv[j], kr[j], acc);
            part_dot[p] = acc;
        }
        // lane l holds the dot of position b + (l >> 3)
        const float dot = wave_sum_rows<GP>(part_dot);
        const uint32_t p = b + (lane >> 3);
        if ((lane & 7) == 0 && p < n) sc[p] = dot * a.scale;
    }
    __syncthreads();
    float* red = sc + ((chunk + 3) & ~3u);
    // maximum, exponentials and their sum over the split
    float m = -INFINITY;
    for (uint32_t i = threadIdx.x; i < n; i += ATTN_THREADS) m = fmaxf(m, sc[i]);
    m = wave_max(m);
    if (lane == 0) red[wv] = m;
    __syncthreads();
    m = red[0];
    for (int w = 1; w < NW; ++w) m = fmaxf(m, red[w]);
    __syncthreads();
    float l = 0.f;
    for (uint32_t i = threadIdx.x; i < n; i += ATTN_THREADS) {
        const float e = expf(sc[i] - m);
        sc[i] = e;
        l += e;
    }
    l = wave_sum(l);
    if (lane == 0) red[wv] = l;
    __syncthreads();
    l = 0.f;
    for (int w = 0; w < NW; ++w) l += red[w];
    // sum_i e_i v_i: wave w takes positions w, w + NW, ...; lane l its dims
    float acc[DPL];
#pragma unroll
    for (int j = 0; j < DPL; ++j) acc[j] = 0.f;
    for (uint32_t i = wv; i < n; i += NW) {
        const float* vr = row(v_cache, i0 + i);
        const float e = sc[i];
#pragma unroll
        for (int j = 0; j < DPL; ++j) acc[j] = fmaf(e, vr[j], acc[j]);
    }
    __syncthreads();                                      // red is reused below
    float* accs = red + NW;                               // [NW][head_dim]
#pragma unroll
    for (int j = 0; j < DPL; ++j) accs[wv * a.head_dim + lane * DPL + j] = acc[j];
    __syncthreads();
    float* out = part + (static_cast<size_t>(h) * gridDim.y + sp) * (a.head_dim + 2);
    for (uint32_t d = threadIdx.x; d < a.head_dim; d += ATTN_THREADS) {
        float t = 0.f;
        for (int w = 0; w < NW; ++w) t += accs[w * a.head_dim + d];
        out[2 + d] = t;
    }
    if (threadIdx.x == 0) {
        out[0] = n ? m : -INFINITY;
        out[1] = l;
    }
}

// out[h][d] = sum_s exp(m_s - M) acc_s[d] / sum_s exp(m_s - M) l_s
__global__ __launch_bounds__(ATTN_MAX_HEAD_DIM)
void k_attn_combine(AttnDims a, const float* __restrict__ part, uint32_t n_splits, float* __restrict__ out)
{
    const uint32_t h = blockIdx.x, d = threadIdx.x;
    const float* p = part + static_cast<size_t>(h) * n_splits * (a.head_dim + 2);
    float M = -INFINITY;
    for (uint32_t s = 0; s < n_splits; ++s) M = fmaxf(M, p[s * (a.head_dim + 2)]);
    float L = 0.f, o = 0.f;
    for (uint32_t s = 0; s < n_splits; ++s) {
        const float* ps = p + s * (a.head_dim + 2);
        if (ps[0] == -INFINITY) continue;                 // empty split
        const float f = expf(ps[0] - M);
        L = fmaf(f, ps[1], L);
        o = fmaf(f, ps[2 + d], o);
    }
    out[static_cast<size_t>(h) * a.head_dim + d] = L > 0.f ? o * (1.0f / L) : 0.f;
}

uint32_t attn_splits(const AttnDims& a, uint32_t valid)
{
    // >= 64 positions per split, <= ATTN_MAX_CHUNK, about 512 blocks in all
    uint32_t n = std::max<uint32_t>(1, std::min<uint32_t>((valid + 63) / 64, std::max<uint32_t>(1, 512 / a.num_heads)));
    n = std::max<uint32_t>(n, (valid + ATTN_MAX_CHUNK - 1) / ATTN_MAX_CHUNK);
    return n;
}

size_t attn_part_floats(const AttnDims& a, uint32_t valid)
{
    return static_cast<size_t>(a.num_heads) * attn_splits(a, valid) * (a.head_dim + 2);
}

hipError_t launch_attention(const AttnDims& a, float* q, float* k, const float* v, const uint16_t* q_norm_w,
                            const uint16_t* k_norm_w, const float* rope_cos, const float* rope_sin, float* k_cache,
                            float* v_cache, uint32_t slot, uint32_t valid, float* part, float* attn_out,
                            hipStream_t s)
{
    if (a.head_dim == 0 || a.head_dim % WAVE || a.head_dim > ATTN_MAX_HEAD_DIM || a.num_kv_heads == 0 ||
        a.num_heads % a.num_kv_heads || valid == 0 || valid > a.ctx || slot >= a.ctx)
        return hipErrorInvalidValue;
    launch_kernel(k_attn_prep, dim3(a.num_heads + a.num_kv_heads), dim3(a.head_dim), s, a, q, k, v, q_norm_w,
                  k_norm_w, rope_cos, rope_sin, k_cache, v_cache, slot);
    const uint32_t ns = attn_splits(a, valid);
    const uint32_t chunk = (valid + ns - 1) / ns;
    constexpr int NW = ATTN_THREADS / WAVE;
    const uint32_t lds = (((chunk + 3) & ~3u) + NW + NW * a.head_dim) * 4u;
    const dim3 grid(a.num_heads, ns);
    switch (a.head_dim / WAVE) {
        case 1: launch_kernel_lds(k_attn_split<1>, grid, dim3(ATTN_THREADS), lds, s, a, q, k_cache, v_cache, slot,
                                  valid, chunk, part); break;
        case 2: launch_kernel_lds(k_attn_split<2>, grid, dim3(ATTN_THREADS), lds, s, a, q, k_cache, v_cache, slot,
                                  valid, chunk, part); break;
        case 3: launch_kernel_lds(k_attn_split<3>, grid, dim3(ATTN_THREADS), lds, s, a, q, k_cache, v_cache, slot,
                                  valid, chunk, part); break;
        default: launch_kernel_lds(k_attn_split<4>, grid, dim3(ATTN_THREADS), lds, s, a, q, k_cache, v_cache, slot,
                                   valid, chunk, part); break;
    }
    launch_kernel(k_attn_combine, dim3(a.num_heads), dim3(a.head_dim), s, a, part, ns, attn_out);
    return hipGetLastError();
}

}  // namespace smoe
