// moe_decode.hip -- batch-1 decode MoE block on gfx950.
//
// Two launches per layer; the kernel boundary between them is the layer's
// second global synchronisation point (a launch is cheaper on MI355X than an
// in-kernel grid barrier):
//   k_moe_up       RMSNorm (common.hpp:245-256) + bf16 router GEMV
//                  (common.hpp:293-306) in the first blocks, published as
//                  flag-carrying 64-bit words that every block polls; softmax +
//                  top-k (scout.cpp:77-123) with the renormalisation
//                  (decode.cpp:296-302) block-wide in every block; then the
//                  gate+up+SiLU GEMV of every selected expert in one launch
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
#include "topk.hpp"

namespace smoe {

DispatchTimer& dispatch_timer()
{
    static thread_local DispatchTimer t;
    return t;
}

// ---------------------------------------------------------------------------
// k_topk: Scout::compute_top_k (scout.cpp:718-720) on rows of scores, one
// wave per row, through the same selection k_moe_up uses.
// ---------------------------------------------------------------------------
template <int VPL>
__global__ __launch_bounds__(WAVE)
void k_topk(const float* __restrict__ scores, uint32_t n, uint32_t k, uint32_t norm, uint32_t* __restrict__ ids,
            float* __restrict__ w)
{
    __shared__ uint2 slots[TOPK_SLOTS];
    const size_t row = blockIdx.x;
    float v[VPL];
    topk_load<VPL>(scores + row * n, n, v);
    uint32_t my_id;
    float my_w;
    const uint32_t count = topk_latency<VPL>(v, n, k, norm, my_id, my_w, slots);
    if (threadIdx.x < count) {
        ids[row * k + threadIdx.x] = my_id;
        w[row * k + threadIdx.x] = my_w;
    }
}

// ---------------------------------------------------------------------------
// k_moe_up: RMSNorm + router + softmax/top-k + gate/up/SiLU for one layer.
// One wave per block; grid (I / 8, K, T).  Lane l owns the 32 columns of
// chunk l (+64 j) of the hidden dimension throughout.  Every wave:
//   1. loads its hidden and norm-weight chunks and its router rows,
//   2. RMS-normalises them, normed = (x * inv) * w (common.hpp:245-256),
//   3. turns the normed chunk into 4-bit digit words (Q4Act),
//   4. computes its router rows' logits, router_w[row] . normed
//      (common.hpp:293-306), published as flag-carrying 64-bit words,
//   5. polls the E logits of its token and selects the experts itself
//      (softmax + top-k, scout.cpp:77-123; renormalised, decode.cpp:296-302),
//   6. streams 8 rows of gate and up of the expert of rank blockIdx.y and
//      writes h = silu(gate) * up (kernels.metal:240-337).
// The logit exchange is XCD-local when the token's block count is a multiple
// of 8: the dispatcher deals consecutive blocks round-robin over the 8 XCDs
// (from some starting XCD), so block b is the (b/8)-th of its XCD, and the
// blocks of every XCD compute all E rows among themselves (rows b/8,
// b/8 + nb/8, ...).  The words then stay in that XCD's L2 (plain stores; the
// pollers' loads are agent-scope) in the copy of its XCC_ID.  Otherwise block
// b < E computes rows b, b + nb, ... and writes every copy through.  A bounded
// spin reports a timeout (err) instead of hanging.  Block 0 of each token
// publishes ids, weights and the expert table.  Steps 1-3 overlap the router
// rows' latency.
// ---------------------------------------------------------------------------
__device__ __forceinline__ uint64_t ll_word(float v) { return (1ull << 32) | __float_as_uint(v); }

constexpr uint32_t SPIN_LIMIT = 1u << 22;
constexpr int UP_RB = 8;   // rows per wave
constexpr int SMOE_G = 64; // SMOE-Q4 group size (shatter_moe.py Q2_GROUP_SIZE)

template <int CPL, int VPL, bool LOCAL>
__device__ __forceinline__ void moe_up_body(const MoeDims& d, const LayerDesc& L, const float* __restrict__ hv,
                                            uint64_t* __restrict__ ll, float* __restrict__ h,
                                            uint32_t* __restrict__ ids_out, float* __restrict__ w_out,
                                            ExpertPtrs* __restrict__ tbl_out, uint32_t* __restrict__ err)
{
    constexpr int RB = UP_RB;
    const int lane = threadIdx.x;
    const uint32_t tok = blockIdx.z, r = blockIdx.y;
    const uint32_t D = d.D, nch = D >> 5;
    const uint32_t nb = gridDim.x * gridDim.y;
    const uint32_t b = blockIdx.y * gridDim.x + blockIdx.x;
    uint32_t row0, rstep, copy;
    if constexpr (LOCAL) {
        uint32_t xcc;
        asm volatile("s_getreg_b32 %0, hwreg(HW_REG_XCC_ID, 0, 4)" : "=s"(xcc));
        row0 = b >> 3;
        rstep = nb >> 3;
        copy = xcc & (LL_COPIES - 1);
    } else {
        row0 = b;
        rstep = nb;
        copy = b % LL_COPIES;
    }
    const bool producer = row0 < d.E;
    const bool second = row0 + rstep < d.E;

    // 1. chunk loads (router last, so the norm can start before it lands)
    float4 x[CPL][8];
    uint4 g[CPL][4], rw[CPL][4], rw2[CPL][4];
#pragma unroll
    for (int j = 0; j < CPL; ++j) {
        const uint32_t c = min(lane + WAVE * j, nch - 1);
#pragma unroll
        for (int q = 0; q < 8; ++q) x[j][q] = load_f4(hv + c * 32 + q * 4);
#pragma unroll
        for (int q = 0; q < 4; ++q) g[j][q] = load_u4(L.norm_w + c * 32 + q * 8);
    }
    // router rows: plain loads (the previous layer's down kernel may have
    // left them in this XCD's L2)
    if (producer) {
        const uint16_t* wr = L.router_w + static_cast<size_t>(row0) * D;
#pragma unroll
        for (int j = 0; j < CPL; ++j) {
            const uint32_t c = min(lane + WAVE * j, nch - 1);
#pragma unroll
            for (int q = 0; q < 4; ++q) rw[j][q] = load_u4(wr + c * 32 + q * 8);
        }
        if (second) {
            const uint16_t* wr2 = L.router_w + static_cast<size_t>(row0 + rstep) * D;
#pragma unroll
            for (int j = 0; j < CPL; ++j) {
                const uint32_t c = min(lane + WAVE * j, nch - 1);
#pragma unroll
                for (int q = 0; q < 4; ++q) rw2[j][q] = load_u4(wr2 + c * 32 + q * 8);
            }
        }
    }
    // 2. RMS norm over the wave's D columns
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
    // rms_norm_bf16 (common.hpp:245-256): inv = 1 / sqrt(ss / n + 1e-6)
    const float inv = 1.0f / sqrtf(ss / static_cast<float>(D) + 1e-6f);
    float a[CPL][32];
#pragma unroll
    for (int j = 0; j < CPL; ++j) {
#pragma unroll
        for (int q = 0; q < 8; ++q) {
            const uint32_t g0 = (q & 1) ? g[j][q >> 1].z : g[j][q >> 1].x;
            const uint32_t g1 = (q & 1) ? g[j][q >> 1].w : g[j][q >> 1].y;
            a[j][4 * q + 0] = (x[j][q].x * inv) * bf16_to_f32(g0 & 0xFFFFu);
            a[j][4 * q + 1] = (x[j][q].y * inv) * bf16_to_f32(g0 >> 16);
            a[j][4 * q + 2] = (x[j][q].z * inv) * bf16_to_f32(g1 & 0xFFFFu);
            a[j][4 * q + 3] = (x[j][q].w * inv) * bf16_to_f32(g1 >> 16);
        }
    }
    // 4. router rows row0, row0 + rstep, ... (padding lanes hold normed 0)
    uint64_t* llc = ll + copy * ll_copy_words(d.E);
    auto publish = [&](uint32_t row, float acc) {
        if constexpr (LOCAL) {
            if (lane == 0)
                __hip_atomic_store(llc + row, ll_word(acc), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WAVEFRONT);
        } else {
            if (lane < static_cast<int>(LL_COPIES))
                __hip_atomic_store(ll + lane * ll_copy_words(d.E) + row, ll_word(acc), __ATOMIC_RELAXED,
                                   __HIP_MEMORY_SCOPE_AGENT);
        }
    };
    auto row_dot = [&](const uint4 (&w)[CPL][4]) {
        float acc = 0.f;
#pragma unroll
        for (int j = 0; j < CPL; ++j) {
#pragma unroll
            for (int q = 0; q < 4; ++q) {
                const uint32_t w4[4] = {w[j][q].x, w[j][q].y, w[j][q].z, w[j][q].w};
#pragma unroll
                for (int t = 0; t < 4; ++t) {
                    acc = fmaf(bf16_to_f32(w4[t] & 0xFFFFu), a[j][8 * q + 2 * t], acc);
                    acc = fmaf(bf16_to_f32(w4[t] >> 16), a[j][8 * q + 2 * t + 1], acc);
                }
            }
        }
        return wave_sum(acc);
    };
    if (producer) {
        publish(row0, row_dot(rw));
        if (second) {
            publish(row0 + rstep, row_dot(rw2));
            for (uint32_t row = row0 + 2 * rstep; row < d.E; row += rstep) {
                const uint16_t* wr = L.router_w + static_cast<size_t>(row) * D;
#pragma unroll
                for (int j = 0; j < CPL; ++j) {
                    const uint32_t c = min(lane + WAVE * j, nch - 1);
#pragma unroll
                    for (int q = 0; q < 4; ++q) rw[j][q] = load_u4(wr + c * 32 + q * 8);
                }
                publish(row, row_dot(rw));
            }
        }
    }
    // 3. digit form of the normed chunk (overlaps the logit exchange)
    Q4Act qa[CPL];
#pragma unroll
    for (int j = 0; j < CPL; ++j) q4_act_from_floats(a[j], qa[j]);
    // 5. wait for the E logits (in this block's copy), then select
    float v[VPL];
    {
        uint32_t spins = 0;
        bool all;
        do {
            all = true;
            // every load issued before any is waited on (padding lanes re-read word E-1)
#pragma unroll
            for (int j = 0; j < VPL; ++j) {
                const uint32_t pos = lane + WAVE * j;
                const uint64_t w64 =
                    __hip_atomic_load(llc + min(pos, d.E - 1), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
                v[j] = __uint_as_float(static_cast<uint32_t>(w64));
                all &= pos >= d.E || (w64 >> 32) != 0;
            }
            all = __ballot(!all) == 0;
            if (!all && ++spins > SPIN_LIMIT) {
                if (lane == 0) atomicOr(err, 1u);
                break;
            }
        } while (!all);
    }
    uint32_t my_id;
    float my_w;
    __shared__ uint2 slots[TOPK_SLOTS];
    topk_latency<VPL>(v, d.E, d.K, d.norm_topk, my_id, my_w, slots);
    const uint32_t expert = readlane_u32(my_id, r);

    if (b == 0 && static_cast<uint32_t>(lane) < d.K) {
        const size_t o = static_cast<size_t>(tok) * d.K + lane;
        ids_out[o] = my_id;
        w_out[o] = my_w;
        const uint8_t* bb = L.experts + static_cast<size_t>(my_id) * L.stride;
        ExpertPtrs e;
        e.pg = bb + L.off[0];
        e.sg = reinterpret_cast<const uint16_t*>(bb + L.off[1]);
        e.pu = bb + L.off[2];
        e.su = reinterpret_cast<const uint16_t*>(bb + L.off[3]);
        e.pd = bb + L.off[4];
        e.sd = reinterpret_cast<const uint16_t*>(bb + L.off[5]);
        e.slot = lane;
        e.pad_ = 0;
        tbl_out[o] = e;
    }

    // 6. 8 rows of gate and up: every weight load in flight before any is used
    const uint32_t rowg = blockIdx.x * RB;
    const uint8_t* blob = L.experts + static_cast<size_t>(expert) * L.stride;
    const uint8_t* pa = blob + L.off[0];
    const uint16_t* sa = reinterpret_cast<const uint16_t*>(blob + L.off[1]);
    const uint8_t* pb = blob + L.off[2];
    const uint16_t* sb = reinterpret_cast<const uint16_t*>(blob + L.off[3]);
    const uint32_t row_bytes = D >> 1, row_scales = D / SMOE_G;
    uint4 va[RB][CPL], vb[RB][CPL];
    uint16_t sva[RB][CPL], svb[RB][CPL];
#pragma unroll
    for (int i = 0; i < RB; ++i) {
        const size_t row = rowg + i;
#pragma unroll
        for (int j = 0; j < CPL; ++j) {
            const uint32_t c = min(lane + WAVE * j, nch - 1);
            va[i][j] = load_stream_u4(pa + row * row_bytes + c * 16);
            vb[i][j] = load_stream_u4(pb + row * row_bytes + c * 16);
            sva[i][j] = load_stream_u16(sa + row * row_scales + (c * 32) / SMOE_G);
            svb[i][j] = load_stream_u16(sb + row * row_scales + (c * 32) / SMOE_G);
        }
    }
    __builtin_amdgcn_sched_barrier(0);
    // per-lane partial dots: value 2i = gate row i, 2i + 1 = up row i
    float part[2 * RB];
#pragma unroll
    for (int i = 0; i < RB; ++i) {
        float ga = 0.f, ua = 0.f;
#pragma unroll
        for (int j = 0; j < CPL; ++j) {
            ga = fmaf(f16_bits_to_f32(sva[i][j]), q4_chunk_dot8(va[i][j], qa[j]), ga);
            ua = fmaf(f16_bits_to_f32(svb[i][j]), q4_chunk_dot8(vb[i][j], qa[j]), ua);
        }
        part[2 * i] = ga;
        part[2 * i + 1] = ua;
    }
    // lane l holds the total of value l >> SH
    constexpr int SH = 6 - ilog2(2 * RB);
    const float tot = wave_sum_rows<2 * RB>(part);
    const float gv = __shfl(tot, (2 * lane) << SH);
    const float uv = __shfl(tot, (2 * lane + 1) << SH);
    // silu(z) = z * (1 / (1 + exp(-z)))  (kernels.metal:61-63, :334-336), all rows at once
    float* o = h + (static_cast<size_t>(tok) * d.K + r) * d.I;
    if (lane < RB) o[rowg + lane] = (gv * (1.0f / (1.0f + expf(-gv)))) * uv;
}

template <int CPL, int VPL, bool LOCAL>
__global__ __launch_bounds__(WAVE)
void k_moe_up(MoeDims d, LayerDesc L, const float* __restrict__ hidden, uint64_t* __restrict__ ll_all,
              float* __restrict__ h, uint32_t* __restrict__ ids_out, float* __restrict__ w_out,
              ExpertPtrs* __restrict__ tbl_out, uint32_t* __restrict__ err)
{
    const uint32_t tok = blockIdx.z;
    const float* hv = hidden + static_cast<size_t>(tok) * d.D;
    uint64_t* ll = ll_all + static_cast<size_t>(tok) * ll_token_words(d.E);
    moe_up_body<CPL, VPL, LOCAL>(d, L, hv, ll, h, ids_out, w_out, tbl_out, err);
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
    uint4 va[RB][CPL], vb[RB][CPL];
    uint16_t sva[RB][CPL], svb[RB][CPL];
#pragma unroll
    for (int i = 0; i < RB; ++i) {
        const size_t row = row0 + i;
#pragma unroll
        for (int j = 0; j < CPL; ++j) {
            const uint32_t c = min(lane + WAVE * j, nch - 1);
            va[i][j] = load_stream_u4(pa + row * row_bytes + c * 16);
            sva[i][j] = load_stream_u16(sa + row * row_scales + (c * 32) / d.group);
            if (GATE_UP) {
                vb[i][j] = load_stream_u4(pb + row * row_bytes + c * 16);
                svb[i][j] = load_stream_u16(sb + row * row_scales + (c * 32) / d.group);
            }
        }
    }
#pragma unroll
    for (int j = 0; j < CPL; ++j) {
        const uint32_t c = min(lane + WAVE * j, nch - 1);
        const bool ok = lane + WAVE * j < nch;
        xsum[j] = 0.f;
#pragma unroll
        for (int q = 0; q < 8; ++q) {
            const float4 v = load_f4(xv + c * 32 + q * 4);
            xr[j][q * 4 + 0] = ok ? v.x : 0.f;
            xr[j][q * 4 + 1] = ok ? v.y : 0.f;
            xr[j][q * 4 + 2] = ok ? v.z : 0.f;
            xr[j][q * 4 + 3] = ok ? v.w : 0.f;
        }
#pragma unroll
        for (int q = 0; q < 32; ++q) xsum[j] += xr[j][q];
    }
    float* o = out + static_cast<size_t>(tok) * out_tok_stride + static_cast<size_t>(e.slot) * out_stride;
#pragma unroll
    for (int i = 0; i < RB; ++i) {
        float aa = 0.f, ab = 0.f;
#pragma unroll
        for (int j = 0; j < CPL; ++j) {
            aa += q4_chunk_epilogue(f16_bits_to_f32(sva[i][j]), q4_chunk_dot(va[i][j], xr[j]), xsum[j]);
            if (GATE_UP)
                ab += q4_chunk_epilogue(f16_bits_to_f32(svb[i][j]), q4_chunk_dot(vb[i][j], xr[j]), xsum[j]);
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
// k_down_combine: hidden[row] += sum_r w_r * (down_r[row] . h_r).
// Lane p of the block owns (expert, 32-column chunk) pair p of the k experts'
// down rows (PPL pairs per lane); its 32 h values are turned into digit words
// once and reused for the block's DOWN_RB rows, so each row of all k experts
// is one block-wide reduction: a transposed wave reduction over the rows,
// then the waves' partials through LDS.  Loads go out in dependency order:
// expert table and h first, the down weights as soon as the table lands; the
// h conversion overlaps the weight fetch.
// ---------------------------------------------------------------------------
constexpr int DOWN_RB = 8;
constexpr int DOWN_MAX_WAVES = 8;

template <int PPL>
__global__ __launch_bounds__(DOWN_MAX_WAVES * WAVE)
void k_down_combine(MoeDims d, const ExpertPtrs* __restrict__ tbl, const float* __restrict__ h,
                    const float* __restrict__ w, float* __restrict__ hidden, uint64_t* __restrict__ ll_all)
{
    constexpr int RB = DOWN_RB;
    // re-arm the routing exchange words of this token for the next k_moe_up
    // (every k_moe_up that read them has finished: this is the next kernel)
    if (blockIdx.x == 0) {
        uint64_t* ll = ll_all + static_cast<size_t>(blockIdx.y) * ll_token_words(d.E);
        for (uint32_t i = threadIdx.x; i < LL_COPIES * d.E; i += blockDim.x)
            ll[(i / d.E) * ll_copy_words(d.E) + i % d.E] = 0;
    }
    __shared__ float part[DOWN_MAX_WAVES][RB];
    const int lane = threadIdx.x & 63, wv = threadIdx.x >> 6;
    const int nw = blockDim.x >> 6;
    const uint32_t row0 = blockIdx.x * RB;
    const uint32_t tok = blockIdx.y;
    tbl += static_cast<size_t>(tok) * d.K;
    h += static_cast<size_t>(tok) * d.K * d.I;
    w += static_cast<size_t>(tok) * d.K;
    hidden += static_cast<size_t>(tok) * d.D;
    const uint32_t cpr = d.I >> 5;
    const uint32_t npairs = d.K * cpr;
    const uint32_t row_bytes = d.I >> 1, row_scales = d.I / SMOE_G;

    const uint8_t* pd[PPL];
    const uint16_t* sd[PPL];
    uint32_t cc[PPL], rr[PPL];
    bool ok[PPL];
    float4 hx[PPL][8];
    float wr[PPL];
#pragma unroll
    for (int j = 0; j < PPL; ++j) {
        const uint32_t p0 = (wv * PPL + j) * WAVE + lane;
        ok[j] = p0 < npairs;
        const uint32_t p = min(p0, npairs - 1);
        rr[j] = p / cpr;
        cc[j] = p - rr[j] * cpr;
        pd[j] = tbl[rr[j]].pd;
        sd[j] = tbl[rr[j]].sd;
    }
#pragma unroll
    for (int j = 0; j < PPL; ++j) {
        const float* hv = h + static_cast<size_t>(rr[j]) * d.I + cc[j] * 32;
#pragma unroll
        for (int q = 0; q < 8; ++q) hx[j][q] = load_f4(hv + q * 4);
        wr[j] = w[rr[j]];
    }
    __builtin_amdgcn_sched_barrier(0);
    uint4 v[RB][PPL];
    uint16_t sv[RB][PPL];
#pragma unroll
    for (int i = 0; i < RB; ++i) {
        const size_t row = row0 + i;
#pragma unroll
        for (int j = 0; j < PPL; ++j) {
            v[i][j] = load_stream_u4(pd[j] + row * row_bytes + cc[j] * 16);
            sv[i][j] = load_stream_u16(sd[j] + row * row_scales + (cc[j] * 32) / SMOE_G);
        }
    }
    __builtin_amdgcn_sched_barrier(0);
    Q4Act qh[PPL];
#pragma unroll
    for (int j = 0; j < PPL; ++j) {
        float a[32];
#pragma unroll
        for (int q = 0; q < 8; ++q) {
            a[q * 4 + 0] = hx[j][q].x;
            a[q * 4 + 1] = hx[j][q].y;
            a[q * 4 + 2] = hx[j][q].z;
            a[q * 4 + 3] = hx[j][q].w;
        }
        q4_act_from_floats(a, qh[j]);
        if (!ok[j]) wr[j] = 0.f;   // pairs past the end contribute nothing
    }
    float acc[RB];
#pragma unroll
    for (int i = 0; i < RB; ++i) {
        acc[i] = 0.f;
#pragma unroll
        for (int j = 0; j < PPL; ++j) {
            const float y = f16_bits_to_f32(sv[i][j]) * q4_chunk_dot8(v[i][j], qh[j]);
            acc[i] = fmaf(wr[j], y, acc[i]);
        }
    }
    // lane l holds the wave's total of row l >> SH
    constexpr int SH = 6 - ilog2(RB);
    const float tot = wave_sum_rows<RB>(acc);
    if ((lane & ((1 << SH) - 1)) == 0) part[wv][lane >> SH] = tot;
    __syncthreads();
    if (threadIdx.x < RB) {
        float t = 0.f;
        for (int q = 0; q < nw; ++q) t += part[q][threadIdx.x];
        const uint32_t row = row0 + threadIdx.x;
        hidden[row] = hidden[row] + t;
    }
}

// ---------------------------------------------------------------------------
// launchers
// ---------------------------------------------------------------------------
template <int CPL, int VPL>
static void moe_up_v(dim3 grid, hipStream_t s, const MoeDims& d, const LayerDesc& L, const float* hidden,
                     uint64_t* ll, float* h, uint32_t* ids, float* w, ExpertPtrs* tbl, uint32_t* err)
{
    // XCD-local logit exchange when every XCD receives the same number of
    // blocks of each token, they cover the router rows in at most two each,
    // and the whole grid is resident at once (the dispatcher's round-robin
    // over the XCDs is then unbroken)
    const uint32_t nb = grid.x * grid.y;
    if (nb % 8 == 0 && nb / 8 * 2 >= d.E && nb * grid.z <= 1024)
        launch_kernel(k_moe_up<CPL, VPL, true>, grid, dim3(WAVE), s, d, L, hidden, ll, h, ids, w, tbl, err);
    else
        launch_kernel(k_moe_up<CPL, VPL, false>, grid, dim3(WAVE), s, d, L, hidden, ll, h, ids, w, tbl, err);
}

template <int CPL>
static void moe_up_c(dim3 grid, hipStream_t s, const MoeDims& d, const LayerDesc& L, const float* hidden,
                     uint64_t* ll, float* h, uint32_t* ids, float* w, ExpertPtrs* tbl, uint32_t* err)
{
    if (d.E <= 128)
        moe_up_v<CPL, 2>(grid, s, d, L, hidden, ll, h, ids, w, tbl, err);
    else
        moe_up_v<CPL, 8>(grid, s, d, L, hidden, ll, h, ids, w, tbl, err);
}

hipError_t launch_moe_up(const MoeDims& d, const LayerDesc& L, const float* hidden, uint32_t n_tok, uint64_t* ll,
                         float* h, uint32_t* ids, float* w, ExpertPtrs* tbl, uint32_t* err, hipStream_t s)
{
    if (d.group != 64 || d.E > SMOE_TOPK_MAX_N || d.I % UP_RB) return hipErrorInvalidValue;
    const uint32_t row_blocks = d.I / UP_RB;                              // one wave per 8 rows
    const dim3 grid(row_blocks, d.K, n_tok);
    const uint32_t cpl = (d.D / 32 + WAVE - 1) / WAVE;   // 32-column chunks per lane
    if (cpl == 1) moe_up_c<1>(grid, s, d, L, hidden, ll, h, ids, w, tbl, err);
    else if (cpl == 2) moe_up_c<2>(grid, s, d, L, hidden, ll, h, ids, w, tbl, err);
    else if (cpl <= 4) moe_up_c<4>(grid, s, d, L, hidden, ll, h, ids, w, tbl, err);
    else return hipErrorInvalidValue;
    return hipGetLastError();
}

hipError_t launch_topk(const float* scores, uint32_t rows, uint32_t n, uint32_t k,
                       uint32_t norm, uint32_t* ids, float* w, hipStream_t s)
{
    if (topk_vpl(n) == 2)
        launch_kernel(k_topk<2>, dim3(rows), dim3(WAVE), s, scores, n, k, norm, ids, w);
    else
        launch_kernel(k_topk<8>, dim3(rows), dim3(WAVE), s, scores, n, k, norm, ids, w);
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
        launch_kernel(k_q4_rows<C, RB, GATE_UP>, grid, dim3(256), s, d, tbl, n_exp,  \
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

hipError_t launch_down_combine(const MoeDims& d, const ExpertPtrs* tbl, const float* h, const float* w,
                               float* hidden, uint64_t* ll, uint32_t n_tok, hipStream_t s)
{
    // one (expert, chunk) pair per lane while the block fits in DOWN_MAX_WAVES waves
    const uint32_t npairs = d.K * (d.I / 32);
    uint32_t ppl = 1;
    while (ppl < 4 && (npairs + 64u * ppl - 1) / (64u * ppl) > DOWN_MAX_WAVES) ppl *= 2;
    const uint32_t nw = (npairs + 64u * ppl - 1) / (64u * ppl);
    if (nw > DOWN_MAX_WAVES || d.D % DOWN_RB) return hipErrorInvalidValue;
    dim3 grid(d.D / DOWN_RB, n_tok), block(nw * WAVE);
    switch (ppl) {
        case 1:
            launch_kernel(k_down_combine<1>, grid, block, s, d, tbl, h, w, hidden, ll);
            break;
        case 2:
            launch_kernel(k_down_combine<2>, grid, block, s, d, tbl, h, w, hidden, ll);
            break;
        default:
            launch_kernel(k_down_combine<4>, grid, block, s, d, tbl, h, w, hidden, ll);
            break;
    }
    return hipGetLastError();
}

// ---------------------------------------------------------------------------
// k_matvec_bf16: out[r] = sum_c bf16(W[r][c]) * x[c] (common.hpp:293-306), one
// wave per row, any cols (the dense-trunk projections of the reference
// surface, metal_bridge.h:157-161; not on the MoE hot path).
// ---------------------------------------------------------------------------
__global__ __launch_bounds__(256)
void k_matvec_bf16(const uint16_t* __restrict__ W, const float* __restrict__ x, float* __restrict__ out,
                   uint32_t rows, uint32_t cols)
{
    const int lane = threadIdx.x & 63;
    const uint32_t r = blockIdx.x * 4 + (threadIdx.x >> 6);
    if (r >= rows) return;
    const uint16_t* wr = W + static_cast<size_t>(r) * cols;
    float acc = 0.f;
    for (uint32_t c = lane; c < cols; c += WAVE) acc = fmaf(bf16_to_f32(wr[c]), x[c], acc);
    acc = wave_sum(acc);
    if (lane == 0) out[r] = acc;
}

hipError_t launch_matvec_bf16(const uint16_t* W, const float* x, float* out, uint32_t rows, uint32_t cols,
                              hipStream_t s)
{
    if (rows == 0 || cols == 0) return hipErrorInvalidValue;
    launch_kernel(k_matvec_bf16, dim3((rows + 3) / 4), dim3(256), s, W, x, out, rows, cols);
    return hipGetLastError();
}

}  // namespace smoe
