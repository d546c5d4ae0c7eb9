// moe_decode.hip -- batch-1 decode MoE block on gfx950.
//
// Three launches per layer, each sized to fill 256 CUs:
//   k_route        RMSNorm (common.hpp:245-256) + bf16 router GEMV
//                  (common.hpp:293-306); the last block to finish runs softmax +
//                  top-k (scout.cpp:77-123) and the renormalisation
//                  (decode.cpp:296-302) in one wave and writes the expert table.
//   k_q4_rows      gate+up+SiLU GEMV of every selected expert in one launch
//                  (kernels.metal:240-337): one wave per block of rows, each
//                  lane owning a fixed 16-byte column chunk of every row, so
//                  its 32 activations stay in VGPRs and the dequant folds into
//                  a per-chunk affine epilogue (kernels.metal:140-145).
//   k_down_combine down GEMV of all k experts (kernels.metal:340-365) with the
//                  routing-weighted combine and the residual add fused
//                  (decode.cpp:482-509): lane p owns (expert, column chunk)
//                  pair p, so every down row of all k experts is one 64-lane
//                  reduction and no per-expert output ever reaches HBM.
//
// Loads of packed nibbles are 128-bit and non-temporal; activations and h
// planes are tiny and stay in L2.
#include <type_traits>

#include "device_common.hpp"
#include "kernels.hpp"

namespace smoe {

// ---------------------------------------------------------------------------
// softmax + selection sort with swaps (scout.cpp:77-123) in one wave.
// Round s scans positions s..n-1 with a strict '>' and swaps the winner into
// position s: the winner is the LOWEST position holding the maximum of the
// not-yet-selected positions (a NaN at position s stays put, as '>' against
// NaN is false).  Positions live in lanes: position p = lane + 64*j.
// ---------------------------------------------------------------------------
// Keys: bits(p) + 1 for candidate positions (probabilities are >= +0, so the
// uint order is the float order; a NaN gets key 1 and, like +0, never wins a
// strict '>' against an earlier position), 0 for positions already selected
// and for padding.  Each round: wave max of the keys on DPP, the lowest
// position holding it from ballots, swap by readlane.
template <int VPL>
__device__ __forceinline__ float sel(const float (&a)[VPL], uint32_t j)
{
    float r = a[0];
#pragma unroll
    for (int t = 1; t < VPL; ++t) r = (static_cast<uint32_t>(t) == j) ? a[t] : r;
    return r;
}
template <int VPL>
__device__ __forceinline__ uint32_t sel(const uint32_t (&a)[VPL], uint32_t j)
{
    uint32_t r = a[0];
#pragma unroll
    for (int t = 1; t < VPL; ++t) r = (static_cast<uint32_t>(t) == j) ? a[t] : r;
    return r;
}

// scores: n values (agent-scope loads: written by other blocks of this grid).
// Lane r < count receives (id_r, w_r); returns count.
template <int VPL>
__device__ uint32_t topk_wave(const float* scores, uint32_t n, uint32_t k, uint32_t norm,
                              uint32_t& my_id, float& my_w)
{
    const int lane = threadIdx.x & (WAVE - 1);
    float p[VPL];
    uint32_t id[VPL], key[VPL];
    float m = -INFINITY;
#pragma unroll
    for (int j = 0; j < VPL; ++j) {
        const uint32_t pos = lane + WAVE * j;
        p[j] = pos < n ? __hip_atomic_load(scores + pos, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT)
                       : -INFINITY;
        id[j] = pos;
        m = fmaxf(m, p[j]);
    }
    m = wave_max(m);
    float sum = 0.f;
#pragma unroll
    for (int j = 0; j < VPL; ++j) {
        const uint32_t pos = lane + WAVE * j;
        p[j] = pos < n ? expf(p[j] - m) : 0.f;
        sum += p[j];
    }
    sum = wave_sum(sum);
    const float inv_sum = (sum > 0.f) ? 1.0f / sum : 0.f;
#pragma unroll
    for (int j = 0; j < VPL; ++j) {
        const uint32_t pos = lane + WAVE * j;
        p[j] *= inv_sum;
        key[j] = pos < n ? (isnan(p[j]) ? 1u : __float_as_uint(p[j]) + 1u) : 0u;
    }

    const uint32_t count = k < n ? k : n;
    float ksum = 0.f;
    my_id = 0;
    my_w = 0.f;
    for (uint32_t s = 0; s < count; ++s) {
        const uint32_t sj = s >> 6;
        const int sl = s & 63;
        const float val_s = readlane_f32(sel(p, sj), sl);
        const uint32_t id_s = readlane_u32(sel(id, sj), sl);
        const uint32_t key_s = readlane_u32(sel(key, sj), sl);
        uint32_t lk = key[0];
#pragma unroll
        for (int j = 1; j < VPL; ++j) lk = max(lk, key[j]);
        const uint32_t K = wave_max_u32(lk);
        uint32_t best = 0xFFFFFFFFu;
#pragma unroll
        for (int j = 0; j < VPL; ++j) {
            const uint64_t mk = __ballot(key[j] == K);
            if (best == 0xFFFFFFFFu && mk != 0) best = WAVE * j + __builtin_ctzll(mk);
        }
        if (isnan(val_s)) best = s;
        const uint32_t bj = best >> 6;
        const int bl = best & 63;
        const float val_b = readlane_f32(sel(p, bj), bl);
        const uint32_t id_b = readlane_u32(sel(id, bj), bl);
#pragma unroll
        for (int j = 0; j < VPL; ++j) {
            if (lane == bl && static_cast<uint32_t>(j) == bj) { p[j] = val_s; id[j] = id_s; key[j] = key_s; }
        }
#pragma unroll
        for (int j = 0; j < VPL; ++j) {
            if (lane == sl && static_cast<uint32_t>(j) == sj) { p[j] = val_b; id[j] = id_b; key[j] = 0u; }
        }
        ksum += val_b;                       // sequential over ranks, as the reference
        if (static_cast<uint32_t>(lane) == s) { my_id = id_b; my_w = val_b; }
    }
    if (norm && ksum > 0.f) my_w = my_w * (1.0f / ksum);
    return count;
}

// positions per lane for n experts: 1, 2, 4 or 8 (n <= 512)
static inline int topk_vpl(uint32_t n) { return n <= 64 ? 1 : n <= 128 ? 2 : n <= 256 ? 4 : 8; }

// ---------------------------------------------------------------------------
// k_route
// ---------------------------------------------------------------------------
constexpr int ROUTE_WAVES = 4;

template <int VPL>
__global__ __launch_bounds__(ROUTE_WAVES * WAVE)
void k_route(MoeDims d, LayerDesc L, const float* __restrict__ hidden,
             float* __restrict__ normed_out, float* __restrict__ logits,
             uint32_t* __restrict__ ids_out, float* __restrict__ w_out,
             ExpertPtrs* __restrict__ tbl, uint32_t* __restrict__ counter)
{
    extern __shared__ float xs[];                  // normed activations [D]
    __shared__ float red[ROUTE_WAVES];
    __shared__ int is_last;
    const int tid = threadIdx.x, lane = tid & 63, wv = tid >> 6;
    const uint32_t D = d.D;
    const uint32_t tok = blockIdx.y;
    hidden += static_cast<size_t>(tok) * D;
    normed_out += static_cast<size_t>(tok) * D;
    logits += static_cast<size_t>(tok) * d.E;
    ids_out += static_cast<size_t>(tok) * d.K;
    w_out += static_cast<size_t>(tok) * d.K;
    tbl += static_cast<size_t>(tok) * d.K;
    counter += tok;

    float ss = 0.f;
    for (uint32_t i = tid * 4; i < D; i += blockDim.x * 4) {
        const float4 v = *reinterpret_cast<const float4*>(hidden + i);
        *reinterpret_cast<float4*>(xs + i) = v;
        ss = fmaf(v.x, v.x, ss);
        ss = fmaf(v.y, v.y, ss);
        ss = fmaf(v.z, v.z, ss);
        ss = fmaf(v.w, v.w, ss);
    }
    ss = wave_sum(ss);
    if (lane == 0) red[wv] = ss;
    __syncthreads();
    float tot = 0.f;
#pragma unroll
    for (int w = 0; w < ROUTE_WAVES; ++w) tot += red[w];
    const float inv = 1.0f / sqrtf(tot / static_cast<float>(D) + 1e-6f);
    for (uint32_t i = tid; i < D; i += blockDim.x) {
        const float v = (xs[i] * inv) * bf16_to_f32(*gptr(L.norm_w + i));
        xs[i] = v;
        if (blockIdx.x == 0) normed_out[i] = v;
    }
    __syncthreads();

    const uint32_t row = blockIdx.x * ROUTE_WAVES + wv;
    if (row < d.E) {
        const uint16_t* wr = L.router_w + static_cast<size_t>(row) * D;
        float a0 = 0.f, a1 = 0.f;
#pragma unroll 4
        for (uint32_t c = lane * 8; c < D; c += 8 * WAVE) {
            const uint4 v = load_u4(wr + c);
            const float4 xa = *reinterpret_cast<const float4*>(xs + c);
            const float4 xb = *reinterpret_cast<const float4*>(xs + c + 4);
            a0 = fmaf(bf16_to_f32(v.x & 0xFFFFu), xa.x, a0);
            a1 = fmaf(bf16_to_f32(v.x >> 16), xa.y, a1);
            a0 = fmaf(bf16_to_f32(v.y & 0xFFFFu), xa.z, a0);
            a1 = fmaf(bf16_to_f32(v.y >> 16), xa.w, a1);
            a0 = fmaf(bf16_to_f32(v.z & 0xFFFFu), xb.x, a0);
            a1 = fmaf(bf16_to_f32(v.z >> 16), xb.y, a1);
            a0 = fmaf(bf16_to_f32(v.w & 0xFFFFu), xb.z, a0);
            a1 = fmaf(bf16_to_f32(v.w >> 16), xb.w, a1);
        }
        const float acc = wave_sum(a0 + a1);
        if (lane == 0) logits[row] = acc;
    }

    // last block to finish runs the selection for the whole layer
    __threadfence();
    __syncthreads();
    if (tid == 0) {
        const uint32_t prev = atomicAdd(counter, 1u);
        is_last = (prev == gridDim.x - 1);
    }
    __syncthreads();
    if (!is_last || wv != 0) return;
    __threadfence();
    uint32_t my_id;
    float my_w;
    const uint32_t count = topk_wave<VPL>(logits, d.E, d.K, d.norm_topk, my_id, my_w);
    if (static_cast<uint32_t>(lane) < count) {
        ids_out[lane] = my_id;
        w_out[lane] = my_w;
        const uint8_t* b = L.experts + static_cast<size_t>(my_id) * L.stride;
        ExpertPtrs e;
        e.pg = b + L.off[0];
        e.sg = reinterpret_cast<const uint16_t*>(b + L.off[1]);
        e.pu = b + L.off[2];
        e.su = reinterpret_cast<const uint16_t*>(b + L.off[3]);
        e.pd = b + L.off[4];
        e.sd = reinterpret_cast<const uint16_t*>(b + L.off[5]);
        e.slot = lane;
        e.pad_ = 0;
        tbl[lane] = e;
    }
    if (lane == 0) *counter = 0;                    // ready for the next launch / replay
}

// ---------------------------------------------------------------------------
// k_topk: one wave per row of scores (Scout::compute_top_k)
// ---------------------------------------------------------------------------
template <int VPL>
__global__ __launch_bounds__(WAVE)
void k_topk(const float* __restrict__ scores, uint32_t n, uint32_t k, uint32_t norm,
            uint32_t* __restrict__ ids, float* __restrict__ w)
{
    const uint32_t row = blockIdx.x;
    uint32_t my_id;
    float my_w;
    const float* sr = scores + static_cast<size_t>(row) * n;
    const uint32_t count = topk_wave<VPL>(sr, n, k, norm, my_id, my_w);
    const uint32_t lane = threadIdx.x;
    if (lane < count) {
        ids[static_cast<size_t>(row) * k + lane] = my_id;
        w[static_cast<size_t>(row) * k + lane] = my_w;
    }
}

// ---------------------------------------------------------------------------
// k_q4_rows: rows of SMOE-Q4 matrices dotted with an activation vector.
//   GATE_UP: rows = I of gate and up, cols = D, x = normed token,
//            out = silu(gate.x) * (up.x)
//   DOWN:    rows = D of down, cols = I, x = h of the table entry's slot
// One wave = RB consecutive rows of one table entry; lane owns chunks
// c = lane + 64 j of every row (CPL chunks), 32 activations each in VGPRs.
// ---------------------------------------------------------------------------
template <int CPL, int RB, bool GATE_UP>
__global__ __launch_bounds__(256)
void k_q4_rows(MoeDims d, const ExpertPtrs* __restrict__ tbl, uint32_t n_exp,
               const float* __restrict__ x, uint32_t x_slot_stride, float* __restrict__ out,
               uint32_t out_stride, uint32_t x_tok_stride, uint32_t tbl_tok_stride,
               uint32_t out_tok_stride)
{
    const int lane = threadIdx.x & 63;
    const uint32_t wave_id = blockIdx.x * 4 + (threadIdx.x >> 6);
    const uint32_t tok = blockIdx.y;
    const uint32_t rows = GATE_UP ? d.I : d.D;
    const uint32_t cols = GATE_UP ? d.D : d.I;
    const uint32_t nrb = rows / RB;
    if (wave_id >= n_exp * nrb) return;
    const uint32_t r = wave_id / nrb;
    const uint32_t row0 = (wave_id - r * nrb) * RB;
    const ExpertPtrs e = tbl[static_cast<size_t>(tok) * tbl_tok_stride + r];
    const float* xv = x + static_cast<size_t>(tok) * x_tok_stride +
                      (GATE_UP ? 0 : static_cast<size_t>(e.slot) * x_slot_stride);
    const uint32_t nch = cols >> 5;
    const uint32_t row_bytes = cols >> 1;
    const uint32_t row_scales = cols / d.group;

    const uint8_t* pa = GATE_UP ? e.pg : e.pd;
    const uint16_t* sa = GATE_UP ? e.sg : e.sd;
    const uint8_t* pb = e.pu;
    const uint16_t* sb = e.su;

    float xr[CPL][32];
    float xsum[CPL];
#pragma unroll
    for (int j = 0; j < CPL; ++j) {
        const uint32_t c = lane + WAVE * j;
        xsum[j] = 0.f;
        if (c < nch) {
#pragma unroll
            for (int q = 0; q < 8; ++q) {
                const float4 v = load_f4(xv + c * 32 + q * 4);
                xr[j][q * 4 + 0] = v.x;
                xr[j][q * 4 + 1] = v.y;
                xr[j][q * 4 + 2] = v.z;
                xr[j][q * 4 + 3] = v.w;
            }
#pragma unroll
            for (int q = 0; q < 32; ++q) xsum[j] += xr[j][q];
        } else {
#pragma unroll
            for (int q = 0; q < 32; ++q) xr[j][q] = 0.f;
        }
    }

    uint4 va[RB][CPL], vb[RB][CPL];
    uint16_t sva[RB][CPL], svb[RB][CPL];
#pragma unroll
    for (int i = 0; i < RB; ++i) {
        const size_t row = row0 + i;
#pragma unroll
        for (int j = 0; j < CPL; ++j) {
            const uint32_t c = lane + WAVE * j;
            if (c < nch) {
                va[i][j] = load_stream_u4(pa + row * row_bytes + c * 16);
                sva[i][j] = load_stream_u16(sa + row * row_scales + (c * 32) / d.group);
                if (GATE_UP) {
                    vb[i][j] = load_stream_u4(pb + row * row_bytes + c * 16);
                    svb[i][j] = load_stream_u16(sb + row * row_scales + (c * 32) / d.group);
                }
            }
        }
    }
    float* o = out + static_cast<size_t>(tok) * out_tok_stride + static_cast<size_t>(e.slot) * out_stride;
#pragma unroll
    for (int i = 0; i < RB; ++i) {
        float aa = 0.f, ab = 0.f;
#pragma unroll
        for (int j = 0; j < CPL; ++j) {
            const uint32_t c = lane + WAVE * j;
            if (c < nch) {
                aa += q4_chunk_epilogue(f16_bits_to_f32(sva[i][j]), q4_chunk_dot(va[i][j], xr[j]), xsum[j]);
                if (GATE_UP)
                    ab += q4_chunk_epilogue(f16_bits_to_f32(svb[i][j]), q4_chunk_dot(vb[i][j], xr[j]), xsum[j]);
            }
        }
        aa = wave_sum(aa);
        if (GATE_UP) ab = wave_sum(ab);
        if (lane == 0) {
            // silu(z) = z * (1 / (1 + exp(-z)))  (kernels.metal:61-63, :334-336)
            o[row0 + i] = GATE_UP ? (aa * (1.0f / (1.0f + expf(-aa)))) * ab : aa;
        }
    }
}

// ---------------------------------------------------------------------------
// k_down_combine
// ---------------------------------------------------------------------------
constexpr int DOWN_RB = 4;
constexpr int DOWN_MAX_WAVES = 8;

template <int PPL>
__global__ __launch_bounds__(DOWN_MAX_WAVES * WAVE)
void k_down_combine(MoeDims d, const ExpertPtrs* __restrict__ tbl, const float* __restrict__ h,
                    const float* __restrict__ w, float* __restrict__ hidden)
{
    __shared__ float part[DOWN_MAX_WAVES][DOWN_RB];
    const int lane = threadIdx.x & 63, wv = threadIdx.x >> 6;
    const int nw = blockDim.x >> 6;
    const uint32_t row0 = blockIdx.x * DOWN_RB;
    const uint32_t tok = blockIdx.y;
    tbl += static_cast<size_t>(tok) * d.K;
    h += static_cast<size_t>(tok) * d.K * d.I;
    w += static_cast<size_t>(tok) * d.K;
    hidden += static_cast<size_t>(tok) * d.D;
    const uint32_t cpr = d.I >> 5;
    const uint32_t npairs = d.K * cpr;
    const uint32_t row_bytes = d.I >> 1, row_scales = d.I / d.group;

    float hr[PPL][32];
    float hsum[PPL], wr[PPL];
    const uint8_t* pd[PPL];
    const uint16_t* sd[PPL];
    uint32_t cc[PPL];
    bool ok[PPL];
#pragma unroll
    for (int j = 0; j < PPL; ++j) {
        const uint32_t p = (wv * PPL + j) * WAVE + lane;
        ok[j] = p < npairs;
        const uint32_t rr = ok[j] ? p / cpr : 0;
        cc[j] = ok[j] ? p - rr * cpr : 0;
        pd[j] = tbl[rr].pd;
        sd[j] = tbl[rr].sd;
        wr[j] = w[rr];
        hsum[j] = 0.f;
        const float* hv = h + static_cast<size_t>(rr) * d.I + cc[j] * 32;
#pragma unroll
        for (int q = 0; q < 8; ++q) {
            const float4 v = ok[j] ? load_f4(hv + q * 4) : make_float4(0.f, 0.f, 0.f, 0.f);
            hr[j][q * 4 + 0] = v.x;
            hr[j][q * 4 + 1] = v.y;
            hr[j][q * 4 + 2] = v.z;
            hr[j][q * 4 + 3] = v.w;
        }
#pragma unroll
        for (int q = 0; q < 32; ++q) hsum[j] += hr[j][q];
    }

    uint4 v[DOWN_RB][PPL];
    uint16_t sv[DOWN_RB][PPL];
#pragma unroll
    for (int i = 0; i < DOWN_RB; ++i) {
        const size_t row = row0 + i;
#pragma unroll
        for (int j = 0; j < PPL; ++j) {
            if (ok[j]) {
                v[i][j] = load_stream_u4(pd[j] + row * row_bytes + cc[j] * 16);
                sv[i][j] = load_stream_u16(sd[j] + row * row_scales + (cc[j] * 32) / d.group);
            }
        }
    }
#pragma unroll
    for (int i = 0; i < DOWN_RB; ++i) {
        float acc = 0.f;
#pragma unroll
        for (int j = 0; j < PPL; ++j) {
            if (ok[j]) {
                const float y = q4_chunk_epilogue(f16_bits_to_f32(sv[i][j]), q4_chunk_dot(v[i][j], hr[j]), hsum[j]);
                acc = fmaf(wr[j], y, acc);
            }
        }
        acc = wave_sum(acc);
        if (lane == 0) part[wv][i] = acc;
    }
    __syncthreads();
    if (threadIdx.x < DOWN_RB) {
        float t = 0.f;
        for (int q = 0; q < nw; ++q) t += part[q][threadIdx.x];
        const uint32_t row = row0 + threadIdx.x;
        hidden[row] = hidden[row] + t;
    }
}

// ---------------------------------------------------------------------------
// launchers
// ---------------------------------------------------------------------------
hipError_t launch_route(const MoeDims& d, const LayerDesc& L, const float* hidden,
                        uint32_t n_tok, float* normed, float* logits, uint32_t* ids, float* w,
                        ExpertPtrs* tbl, uint32_t* counter, hipStream_t s)
{
    const uint32_t nblk = (d.E + ROUTE_WAVES - 1) / ROUTE_WAVES;
    const dim3 grid(nblk, n_tok), block(ROUTE_WAVES * WAVE);
    const size_t lds = d.D * sizeof(float);
    switch (topk_vpl(d.E)) {
        case 1: hipLaunchKernelGGL(k_route<1>, grid, block, lds, s, d, L, hidden, normed, logits, ids, w, tbl, counter); break;
        case 2: hipLaunchKernelGGL(k_route<2>, grid, block, lds, s, d, L, hidden, normed, logits, ids, w, tbl, counter); break;
        case 4: hipLaunchKernelGGL(k_route<4>, grid, block, lds, s, d, L, hidden, normed, logits, ids, w, tbl, counter); break;
        default: hipLaunchKernelGGL(k_route<8>, grid, block, lds, s, d, L, hidden, normed, logits, ids, w, tbl, counter); break;
    }
    return hipGetLastError();
}

hipError_t launch_topk(const float* scores, uint32_t rows, uint32_t n, uint32_t k,
                       uint32_t norm, uint32_t* ids, float* w, hipStream_t s)
{
    switch (topk_vpl(n)) {
        case 1: hipLaunchKernelGGL(k_topk<1>, dim3(rows), dim3(WAVE), 0, s, scores, n, k, norm, ids, w); break;
        case 2: hipLaunchKernelGGL(k_topk<2>, dim3(rows), dim3(WAVE), 0, s, scores, n, k, norm, ids, w); break;
        case 4: hipLaunchKernelGGL(k_topk<4>, dim3(rows), dim3(WAVE), 0, s, scores, n, k, norm, ids, w); break;
        default: hipLaunchKernelGGL(k_topk<8>, dim3(rows), dim3(WAVE), 0, s, scores, n, k, norm, ids, w); break;
    }
    return hipGetLastError();
}

template <bool GATE_UP>
static hipError_t launch_rows(const MoeDims& d, const ExpertPtrs* tbl, uint32_t n_exp,
                              const float* x, uint32_t x_slot_stride, float* out,
                              uint32_t out_stride, uint32_t n_tok, uint32_t x_tok_stride,
                              uint32_t tbl_tok_stride, uint32_t out_tok_stride, hipStream_t s)
{
    constexpr int RB = 4;
    const uint32_t rows = GATE_UP ? d.I : d.D;
    const uint32_t cols = GATE_UP ? d.D : d.I;
    const uint32_t nch = cols / 32;
    const uint32_t cpl = (nch + WAVE - 1) / WAVE;
    const uint32_t waves = n_exp * (rows / RB);
    dim3 grid((waves + 3) / 4, n_tok);
#define SMOE_ROWS_CASE(C)                                                                     \
    case C:                                                                                    \
        hipLaunchKernelGGL((k_q4_rows<C, RB, GATE_UP>), grid, dim3(256), 0, s, d, tbl, n_exp,  \
                           x, x_slot_stride, out, out_stride, x_tok_stride, tbl_tok_stride,    \
                           out_tok_stride);                                                    \
        break;
    switch (cpl) {
        SMOE_ROWS_CASE(1)
        SMOE_ROWS_CASE(2)
        SMOE_ROWS_CASE(3)
        SMOE_ROWS_CASE(4)
        default: return hipErrorInvalidValue;
    }
#undef SMOE_ROWS_CASE
    return hipGetLastError();
}

hipError_t launch_gate_up(const MoeDims& d, const ExpertPtrs* tbl, uint32_t n_exp,
                          const float* x, float* h, uint32_t h_stride, uint32_t n_tok,
                          uint32_t x_tok_stride, uint32_t tbl_tok_stride,
                          uint32_t h_tok_stride, hipStream_t s)
{
    return launch_rows<true>(d, tbl, n_exp, x, 0, h, h_stride, n_tok, x_tok_stride,
                             tbl_tok_stride, h_tok_stride, s);
}

hipError_t launch_down_slots(const MoeDims& d, const ExpertPtrs* tbl, uint32_t n_exp,
                             const float* h, uint32_t h_stride, float* out,
                             uint32_t out_stride, uint32_t n_tok, uint32_t tbl_tok_stride,
                             uint32_t h_tok_stride, uint32_t out_tok_stride, hipStream_t s)
{
    return launch_rows<false>(d, tbl, n_exp, h, h_stride, out, out_stride, n_tok, h_tok_stride,
                              tbl_tok_stride, out_tok_stride, s);
}

hipError_t launch_down_combine(const MoeDims& d, const ExpertPtrs* tbl, const float* h,
                               const float* w, float* hidden, uint32_t n_tok, hipStream_t s)
{
    const uint32_t npairs = d.K * (d.I / 32);
    int ppl = npairs <= 64 ? 1 : npairs <= 128 ? 2 : 3;
    uint32_t nw = (npairs + 64u * ppl - 1) / (64u * ppl);
    if (nw > DOWN_MAX_WAVES) {
        ppl = 4;
        nw = (npairs + 255u) / 256u;
        if (nw > DOWN_MAX_WAVES) return hipErrorInvalidValue;
    }
    dim3 grid(d.D / DOWN_RB, n_tok), block(nw * WAVE);
    switch (ppl) {
        case 1: hipLaunchKernelGGL(k_down_combine<1>, grid, block, 0, s, d, tbl, h, w, hidden); break;
        case 2: hipLaunchKernelGGL(k_down_combine<2>, grid, block, 0, s, d, tbl, h, w, hidden); break;
        case 3: hipLaunchKernelGGL(k_down_combine<3>, grid, block, 0, s, d, tbl, h, w, hidden); break;
        default: hipLaunchKernelGGL(k_down_combine<4>, grid, block, 0, s, d, tbl, h, w, hidden); break;
    }
    return hipGetLastError();
}

}  // namespace smoe
