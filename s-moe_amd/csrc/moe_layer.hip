// moe_layer.hip -- batch-1 decode MoE block in one launch on gfx950.
//
// One top-k rank per XCD.  With k = 8 selected experts and the 8 XCDs of
// MI355X, XCD x owns rank x: its waves stream expert ids[x]'s gate/up rows
// and then its down rows, so the two exchanges inside the block stay in that
// XCD's L2; only the final routing-weighted combine crosses XCDs.  Per wave
// (block b, t = b / 8, on XCD x = XCC_ID; the dispatcher deals consecutive
// blocks round-robin over the XCDs from some starting XCD, so t is unique
// within an XCD):
//   1. RMSNorm of the hidden state (common.hpp:245-256) and the bf16 router
//      rows t, t + n, ... (common.hpp:293-306), published as flag-carrying
//      words in XCD x's logit copy;
//   2. softmax + top-k (scout.cpp:77-123) + renormalisation
//      (decode.cpp:296-302) from that copy, in every wave; where registers
//      allow, the gate/up rows of the expert the top-k network proposes for
//      rank x are requested before the softmax and the exact check finish
//      (requested again, for the selected expert, should the check overturn
//      the proposal);
//   3. t < n_up: RB rows (8, or 6 where that fills every wave) of gate and
//      up of expert ids[x] and
//      h = silu(gate) * up (kernels.metal:240-337), published in XCD x's
//      h copy;
//   4. t < n_down: RW rows of expert ids[x]'s down matrix (kernels.metal:
//      340-365) against all of h, staged in LDS; lane group g, lane c owns
//      column chunk c of DR rows; the row totals go out as flag-carrying
//      words through memory to the other XCDs;
//   5. the wave of row block t on XCD t % 8 collects the k partial rows and
//      writes hidden[row] += sum_r w_r * y_r[row] in rank order
//      (decode.cpp:482-509).
// The flag of every exchange word is the launch's tag, read from the epoch
// word at the start; the combiner of row block 0 on XCD 0 advances the
// epoch at its end.  Every wave produces a router row or a gate/up row block
// (host-checked), and that combiner depends on all of them, so every wave has
// read the tag before it changes; words never need re-arming, which keeps a
// captured graph replayable.  All polls are bounded and report a timeout in
// err bit 0.  The whole grid must be resident at once: the host checks it
// against the occupancy of the kernel.
#include <algorithm>
#include <cstdio>
#include <mutex>
#include <vector>

#include "device_common.hpp"
#include "kernels.hpp"
#include "topk.hpp"

namespace smoe {

namespace {

constexpr uint32_t LX_SPIN_LIMIT = 1u << 22;
constexpr int LX_UP_RB = 8;     // gate/up rows per wave (6 where that fills every wave)
constexpr int LX_GROUP = 64;    // SMOE-Q4 group size (shatter_moe.py Q2_GROUP_SIZE)

__device__ __forceinline__ uint64_t lx_word(float v, uint32_t tag)
{
    return (static_cast<uint64_t>(tag) << 32) | __float_as_uint(v);
}

__device__ __forceinline__ uint32_t xcc_id()
{
    uint32_t x;
    asm volatile("s_getreg_b32 %0, hwreg(HW_REG_XCC_ID, 0, 4)" : "=s"(x));
    return x & 7u;
}

// a store that only this XCD's waves read: it stays in this XCD's L2
__device__ __forceinline__ void put_local(uint64_t* p, uint64_t v)
{
    __hip_atomic_store(p, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WAVEFRONT);
}
__device__ __forceinline__ void put_agent(uint64_t* p, uint64_t v)
{
    __hip_atomic_store(p, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ uint64_t get_agent(const uint64_t* p)
{
    return __hip_atomic_load(const_cast<uint64_t*>(p), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ uint32_t get_agent32(const uint32_t* p)
{
    return __hip_atomic_load(const_cast<uint32_t*>(p), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
// 16 bytes that other CUs wrote during the launch: two agent-scope loads,
// which read the L2 past this CU's L1 (a plain load can hit a line the L1
// still holds from before the write: a workgroup-scope invalidate does not
// drop it, and the agent-scope one drops the CU's whole L1 at a cost of
// microseconds)
__device__ __forceinline__ float4 load_f4_agent(const float* p)
{
    const uint64_t a = get_agent(reinterpret_cast<const uint64_t*>(p));
    const uint64_t b = get_agent(reinterpret_cast<const uint64_t*>(p) + 1);
    return make_float4(__uint_as_float(static_cast<uint32_t>(a)), __uint_as_float(static_cast<uint32_t>(a >> 32)),
                       __uint_as_float(static_cast<uint32_t>(b)), __uint_as_float(static_cast<uint32_t>(b >> 32)));
}
__device__ __forceinline__ void vm_wait_all()
{
    asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
}

// Where one layer step reads its input and leaves its output.
struct LayerIO {
    const float* hin;        // the layer's input hidden state [D]
    const uint32_t* wait;    // null, or: the input is complete once wait[0 .. n_down - 1]
    uint32_t wait_tag;       // all equal wait_tag; it was written by other CUs of this XCD
                             // during the launch (read from the L2, not from a stale L1)
    float* hout;             // combined rows go here (null: none)
    bool all_rows;           // every wave combines its row block for its own XCD
                             // (else: row block t on XCD t % 8, once)
    uint32_t* flag;          // null, or: flag[t] = tag once the wave's combined rows are stored
    uint64_t* py;            // the rank partials' exchange words
    uint32_t* abort;         // null, or: a wave that times out stores abort_val here, and
    uint32_t abort_val;      // every wait ends once it reads abort_val
    const uint16_t* next_router;   // null, or: the next layer's router rows (touched into the L2)
};

// a bounded wait's spin count: true once the wait is to end unfinished
__device__ __forceinline__ bool give_up(uint32_t spins, const LayerIO& io)
{
    if (spins > LX_SPIN_LIMIT) return true;
    return io.abort && (spins & 255u) == 0 && get_agent32(io.abort) == io.abort_val;
}

}  // namespace

// One layer of one token, by wave t of XCD x (nbx waves per XCD).  Returns
// true when one of its waits timed out.  NW > 1: the block's NW waves share
// one copy of the hidden state and norm weights and one of the XCD's h in
// LDS (the CU then reads them from the L2 once instead of once per wave); the
// whole block calls the step.
// QF: the group format (0 SMOE-Q4: fp16 scale s, w = (c - 7.5) / 7.5 s; 1 the
// scale+min format: bf16 scale s and min m after all scales of the matrix,
// w = c s + m; GATHER configurations only).
template <int CPL, int VPL, int SEG, int DR, int RB, int NW, bool CHAIN, int QF>
__device__ __forceinline__ bool moe_layer_step(const MoeDims& d, const LayerDesc& L, const LayerIO& io,
                                               uint64_t* __restrict__ lx, uint32_t tag, uint32_t* ids_out,
                                               float* w_out, uint32_t n_up, uint32_t n_down, uint32_t t, uint32_t x,
                                               uint32_t nbx)
{
    constexpr int NR = RB == 6 ? 16 : 2 * RB;   // reduced values (gate, up per row), padded to a power of two
    constexpr int GL = 1 << SEG;       // lanes of one down group
    constexpr int NG = WAVE / GL;      // down groups per wave
    constexpr int RW = NG * DR;        // down rows per wave
    constexpr int SH = SEG - ilog2(DR);
    // (in the chain of the wide family, opaque per layer: values derived from
    // the lane are then recomputed per layer instead of hoisted out of the
    // layer loop and held in registers across it, which left too few for the
    // top-k proposal below; the narrow family measured 0.5 % faster with them
    // hoisted)
    int lane_ = threadIdx.x & (WAVE - 1);
    if constexpr (CHAIN && CPL == 2) asm volatile("" : "+v"(lane_));
    const int lane = lane_;
    const uint32_t wv = NW > 1 ? __builtin_amdgcn_readfirstlane(threadIdx.x >> 6) : 0u;
    const uint32_t D = d.D, nch = D >> 5;
    uint64_t* logc = lx + LX_HEAD + x * lx_pad(d.E);
    uint64_t* hxc = lx + LX_HEAD + 8u * lx_pad(d.E) + x * lx_pad(d.I);
    uint64_t* py = io.py;
    const uint32_t py_stride = lx_pad(D);
    bool timed_out = false;

    // 1. the hidden state, norm weights and router rows t, t + nbx.  Loads
    //    return in order, so the hidden state goes first (the norm can then
    //    start while the router rows arrive) -- unless the input is still to
    //    be waited for: then the norm weights and router rows are requested
    //    first, and the hidden state once it is complete.
    const bool producer = t < d.E;
    const bool second = t + nbx < d.E;
    float4 xv[CPL][8];
    uint4 g[CPL][4], rw[CPL][4], rw2[CPL][4];
    // NW > 1: quad q of 32-column chunk c of the hidden state at float4
    // q * (CPL * WAVE + 1) + c (norm weights: 8-value quad q at uint4
    // q * (...) + c), so that the 64 lanes reading quad q of their chunks
    // touch consecutive addresses; the + 1 spreads the fills over the banks
    constexpr uint32_t QS = CPL * WAVE + 1;
    __shared__ float4 hid_s[NW > 1 ? 8 * QS : 1];
    __shared__ uint4 nrm_s[NW > 1 ? 4 * QS : 1];
    // (coherent: the input was written by other CUs during the launch)
    auto load_hidden = [&](bool coherent) {
        auto ld = [&](const float* p) { return coherent ? load_f4_agent(p) : load_f4(p); };
        if constexpr (NW > 1) {
            for (uint32_t f = threadIdx.x; f < D / 4; f += NW * WAVE)
                hid_s[(f & 7u) * QS + (f >> 3)] = ld(io.hin + 4 * f);
        } else {
#pragma unroll
            for (int j = 0; j < CPL; ++j) {
                const uint32_t c = min(lane + WAVE * j, nch - 1);
#pragma unroll
                for (int q = 0; q < 8; ++q) xv[j][q] = ld(io.hin + c * 32 + q * 4);
            }
        }
    };
    if (!io.wait) load_hidden(false);
    if constexpr (NW > 1) {
        for (uint32_t f = threadIdx.x; f < D / 8; f += NW * WAVE)
            nrm_s[(f & 3u) * QS + (f >> 2)] = load_u4(L.norm_w + 8 * f);
    } else {
#pragma unroll
        for (int j = 0; j < CPL; ++j) {
            const uint32_t c = min(lane + WAVE * j, nch - 1);
#pragma unroll
            for (int q = 0; q < 4; ++q) g[j][q] = load_u4(L.norm_w + c * 32 + q * 8);
        }
    }
    if (producer) {
        const uint16_t* wr = L.router_w + static_cast<size_t>(t) * D;
#pragma unroll
        for (int j = 0; j < CPL; ++j) {
            const uint32_t c = min(lane + WAVE * j, nch - 1);
#pragma unroll
            for (int q = 0; q < 4; ++q) rw[j][q] = load_u4(wr + c * 32 + q * 8);
        }
        if (second) {
            const uint16_t* wr2 = L.router_w + static_cast<size_t>(t + nbx) * D;
#pragma unroll
            for (int j = 0; j < CPL; ++j) {
                const uint32_t c = min(lane + WAVE * j, nch - 1);
#pragma unroll
                for (int q = 0; q < 4; ++q) rw2[j][q] = load_u4(wr2 + c * 32 + q * 8);
            }
        }
    }
    if (io.wait) {
        // the row blocks' flags, as the logit exchange polls its words (one
        // wave of the block polls them)
        if (wv == 0) {
            uint32_t spins = 0;
            bool all;
            do {
                all = true;
                for (uint32_t k = lane; k < n_down; k += WAVE) all &= get_agent32(io.wait + k) == io.wait_tag;
                all = __ballot(!all) == 0;
                if (!all) {
                    if (give_up(++spins, io)) {
                        timed_out = true;
                        break;
                    }
                    __builtin_amdgcn_s_sleep(1);
                }
            } while (!all);
        }
        if constexpr (NW > 1) __syncthreads();
        load_hidden(true);
    }
    if constexpr (NW > 1) {
        __syncthreads();
#pragma unroll
        for (int j = 0; j < CPL; ++j) {
            const uint32_t c = min(lane + WAVE * j, nch - 1);
#pragma unroll
            for (int q = 0; q < 8; ++q) xv[j][q] = hid_s[q * QS + c];
#pragma unroll
            for (int q = 0; q < 4; ++q) g[j][q] = nrm_s[q * QS + c];
        }
    }
    // 2. RMS norm: normed = (x * inv) * w, inv = 1 / sqrt(ss / n + 1e-6)
    float ss = 0.f;
#pragma unroll
    for (int j = 0; j < CPL; ++j) {
        const bool ok = lane + WAVE * j < nch;
#pragma unroll
        for (int q = 0; q < 8; ++q) {
            if (!ok) xv[j][q] = make_float4(0.f, 0.f, 0.f, 0.f);
            ss = fmaf(xv[j][q].x, xv[j][q].x, ss);
            ss = fmaf(xv[j][q].y, xv[j][q].y, ss);
            ss = fmaf(xv[j][q].z, xv[j][q].z, ss);
            ss = fmaf(xv[j][q].w, xv[j][q].w, ss);
        }
    }
    ss = wave_sum(ss);
    const float inv = 1.0f / sqrtf(ss / static_cast<float>(D) + 1e-6f);
    float a[CPL][32];
#pragma unroll
    for (int j = 0; j < CPL; ++j) {
#pragma unroll
        for (int q = 0; q < 8; ++q) {
            const uint32_t g0 = (q & 1) ? g[j][q >> 1].z : g[j][q >> 1].x;
            const uint32_t g1 = (q & 1) ? g[j][q >> 1].w : g[j][q >> 1].y;
            a[j][4 * q + 0] = (xv[j][q].x * inv) * bf16_to_f32(g0 & 0xFFFFu);
            a[j][4 * q + 1] = (xv[j][q].y * inv) * bf16_to_f32(g0 >> 16);
            a[j][4 * q + 2] = (xv[j][q].z * inv) * bf16_to_f32(g1 & 0xFFFFu);
            a[j][4 * q + 3] = (xv[j][q].w * inv) * bf16_to_f32(g1 >> 16);
        }
    }
    auto row_dot = [&](const uint4 (&w)[CPL][4]) {
        float acc = 0.f;
#pragma unroll
        for (int j = 0; j < CPL; ++j) {
#pragma unroll
            for (int q = 0; q < 4; ++q) {
                const uint32_t w4[4] = {w[j][q].x, w[j][q].y, w[j][q].z, w[j][q].w};
#pragma unroll
                for (int u = 0; u < 4; ++u) {
                    acc = fmaf(bf16_to_f32(w4[u] & 0xFFFFu), a[j][8 * q + 2 * u], acc);
                    acc = fmaf(bf16_to_f32(w4[u] >> 16), a[j][8 * q + 2 * u + 1], acc);
                }
            }
        }
        return wave_sum(acc);
    };
    if (producer) {
        const float l0 = row_dot(rw);
        if (lane == 0) put_local(logc + t, lx_word(l0, tag));
        if (second) {
            const float l1 = row_dot(rw2);
            if (lane == 0) put_local(logc + t + nbx, lx_word(l1, tag));
            for (uint32_t row = t + 2 * nbx; row < d.E; row += nbx) {
                const uint16_t* wr = L.router_w + static_cast<size_t>(row) * D;
#pragma unroll
                for (int j = 0; j < CPL; ++j) {
                    const uint32_t c = min(lane + WAVE * j, nch - 1);
#pragma unroll
                    for (int q = 0; q < 4; ++q) rw[j][q] = load_u4(wr + c * 32 + q * 8);
                }
                const float lr = row_dot(rw);
                if (lane == 0) put_local(logc + row, lx_word(lr, tag));
            }
        }
    }
    // digit form of the normed chunk (overlaps the logit exchange)
    Q4Act qa[CPL];
#pragma unroll
    for (int j = 0; j < CPL; ++j) q4_act_from_floats(a[j], qa[j]);

    // 2. the E logits of this XCD's copy, then softmax + top-k
    float v[VPL];
    {
        uint32_t spins = 0;
        bool all;
        do {
            all = true;
#pragma unroll
            for (int j = 0; j < VPL; ++j) {
                const uint32_t pos = lane + WAVE * j;
                const uint64_t w64 = get_agent(logc + min(pos, d.E - 1));
                v[j] = __uint_as_float(static_cast<uint32_t>(w64));
                all &= pos >= d.E || static_cast<uint32_t>(w64 >> 32) == tag;
            }
            all = __ballot(!all) == 0;
            if (!all && give_up(++spins, io)) {
                timed_out = true;
                break;
            }
        } while (!all);
    }
    uint32_t my_id;
    float my_w;
    __shared__ uint2 slots_all[NW][TOPK_SLOTS];
    uint2* slots = slots_all[wv];
    // Where the gate/up rows in flight leave registers for the rest of the
    // top-k: the expert of rank x as the top-k network proposes it (E <= 128),
    // so its weights are requested while the softmax and the check run: the
    // narrow configurations, and the wide ones with 6 rows a wave (two waves
    // a SIMD).  Otherwise (more experts, or 8 wide rows) the exact top-k first.
    constexpr bool PROPOSE = VPL == 2 && (RB * CPL * 2 * 4 <= 64 || (CPL == 2 && RB == 6));
    uint32_t prop, expert;
    NetTopk net;
    if constexpr (PROPOSE) {
        topk_net_begin(v, d.E, net);
        prop = __builtin_amdgcn_readfirstlane(topk_net_rank(net, x, d.E));
    } else {
        topk_latency<VPL>(v, d.E, d.K, d.norm_topk, my_id, my_w, slots);
        prop = min(readlane_u32(my_id, static_cast<int>(x)), d.E - 1);
    }

    // gate/up rows RB t .. RB t + RB - 1 and down rows of rank x: lane
    // (group gi, chunk c) owns chunk c of down rows rowb .. rowb + DR - 1
    const uint32_t rowg = t * RB;
    const uint32_t row_bytes = D >> 1, row_scales = D / LX_GROUP;
    const uint32_t CH = d.I >> 5;
    const int gi = lane >> SEG, c0 = lane & (GL - 1);
    const bool act = static_cast<uint32_t>(c0) < CH;
    const uint32_t dc = act ? static_cast<uint32_t>(c0) : CH - 1;
    const uint32_t rowb = t * RW + gi * DR;
    // GATHER (the narrow configurations with PROPOSE): the scales of the wave's rows
    // are contiguous (RB * D / 32 bytes of gate, as many of up, RW * I / 32
    // of down), loaded as one 16-byte piece per lane (a load instruction
    // costs the CU a request slot whatever its width: at 30B this halves the
    // gate/up requests the top-k check waits behind), issued ahead of the rows
    // and passed to the lanes that use them through LDS.  Host-checked: the
    // pieces are 16-byte aligned and the gate/up ones fit one per lane.  The
    // wide configurations load each lane's scale beside its row piece (the
    // LDS hand-over costs the 235B layer 2.8 us).
    constexpr bool GATHER = PROPOSE && CPL == 1;
    static_assert(QF == 0 || GATHER, "the scale+min format runs on the gathered-scale configurations");
    // (scale+min: a matrix's mins start D * I / 64 entries after its scales)
    const size_t min_bytes = QF ? static_cast<size_t>(D) * d.I / 32 : 0;
    // DFIRST (the same, narrow configurations with 16 down rows a wave, in
    // the chain): the down rows are requested first, ahead of the gate/up
    // rows, so that they have landed when h is published and polled (loads
    // complete in order: requested after the h publication, they held back
    // its poll by their latency).  30B chain 1767 -> 1803 tok/s; the
    // one-launch layer kernel measured 5 % slower with it (1666 -> 1589).
    constexpr bool DFIRST = GATHER && SEG == 5 && CHAIN;
    constexpr uint32_t DN_MAX_I = SEG == 5 ? 1024u : 2048u;
    constexpr int NSD = GATHER ? (RW * DN_MAX_I / 512 + WAVE - 1) / WAVE : 1;   // down scale pieces per lane
    const uint32_t nsq_up = RB * D / 512, nsq_dn = RW * d.I / 512;
    uint4 va[RB][CPL], vb[RB][CPL], qa_s, qb_s, qd_s[NSD];
    uint4 qa_m, qb_m, qd_m[QF ? NSD : 1];
    uint16_t sva[GATHER ? 1 : RB][CPL], svb[GATHER ? 1 : RB][CPL], dsv[GATHER ? 1 : DR];
    uint4 dv[DR];
    __shared__ uint4 sc_up_all[NW][GATHER ? (QF ? 4 : 2) : 1][WAVE];
    __shared__ uint4 sc_dn_all[NW][(QF ? 2 : 1) * NSD * WAVE];
    auto& sc_up = sc_up_all[wv];
    auto& sc_dn = sc_dn_all[wv];
    auto issue_up = [&](const uint8_t* blob) {
        const uint8_t* pa = blob + L.off[0];
        const uint8_t* pb = blob + L.off[2];
        const uint16_t* sa = reinterpret_cast<const uint16_t*>(blob + L.off[1]);
        const uint16_t* sb = reinterpret_cast<const uint16_t*>(blob + L.off[3]);
        if constexpr (GATHER) {
            const uint32_t q = min(static_cast<uint32_t>(lane), nsq_up - 1);
            qa_s = load_stream_u4(blob + L.off[1] + static_cast<size_t>(rowg) * row_scales * 2 + q * 16);
            qb_s = load_stream_u4(blob + L.off[3] + static_cast<size_t>(rowg) * row_scales * 2 + q * 16);
            if constexpr (QF) {
                qa_m = load_stream_u4(blob + L.off[1] + min_bytes + static_cast<size_t>(rowg) * row_scales * 2 + q * 16);
                qb_m = load_stream_u4(blob + L.off[3] + min_bytes + static_cast<size_t>(rowg) * row_scales * 2 + q * 16);
            }
        }
#pragma unroll
        for (int i = 0; i < RB; ++i) {
            const size_t row = rowg + i;
#pragma unroll
            for (int j = 0; j < CPL; ++j) {
                const uint32_t c = min(lane + WAVE * j, nch - 1);
                va[i][j] = load_stream_u4(pa + row * row_bytes + c * 16);
                vb[i][j] = load_stream_u4(pb + row * row_bytes + c * 16);
                if constexpr (!GATHER) {
                    sva[i][j] = load_stream_u16(sa + row * row_scales + (c * 32) / LX_GROUP);
                    svb[i][j] = load_stream_u16(sb + row * row_scales + (c * 32) / LX_GROUP);
                }
            }
        }
    };
    auto issue_down = [&](const uint8_t* blob) {
        const uint8_t* pdn = blob + L.off[4];
        const uint16_t* sdn = reinterpret_cast<const uint16_t*>(blob + L.off[5]);
        const uint32_t drow_bytes = d.I >> 1, drow_scales = d.I / LX_GROUP;
        if constexpr (GATHER) {
#pragma unroll
            for (int k = 0; k < NSD; ++k) {
                const uint32_t q = min(static_cast<uint32_t>(k * WAVE + lane), nsq_dn - 1);
                qd_s[k] = load_stream_u4(blob + L.off[5] + static_cast<size_t>(t) * RW * (d.I / 32) + q * 16);
                if constexpr (QF)
                    qd_m[k] = load_stream_u4(blob + L.off[5] + min_bytes + static_cast<size_t>(t) * RW * (d.I / 32) +
                                             q * 16);
            }
        }
#pragma unroll
        for (int i = 0; i < DR; ++i) {
            const size_t row = rowb + i;
            dv[i] = load_stream_u4(pdn + row * drow_bytes + dc * 16);
            if constexpr (!GATHER) dsv[i] = load_stream_u16(sdn + row * drow_scales + (dc * 32) / LX_GROUP);
        }
    };
    const uint8_t* blob;
    uint32_t touch = 0;
    if constexpr (PROPOSE) {
        if constexpr (DFIRST)
            if (t < n_down) issue_down(L.experts + static_cast<size_t>(prop) * L.stride);
        if (t < n_up) issue_up(L.experts + static_cast<size_t>(prop) * L.stride);
        __builtin_amdgcn_sched_barrier(0);
        // the next layer's router row of this wave, one dword of each 128-byte
        // line into the XCD's L2, behind the expert rows (it lands with them,
        // before anything this layer waits for is requested)
        if constexpr (CHAIN && CPL == 1)
            if (io.next_router && producer) {
                const uint32_t r = (lane >> 5) && second ? t + nbx : t;
                // (a global, not a flat, load: a flat load in flight leaves the
                // compiler unable to count the loads before it, and every later
                // wait then drains all of them -- the gate/up dots would wait
                // for the last row instead of starting as the first rows land)
                touch = *gptr(io.next_router + static_cast<size_t>(r) * D +
                              min((static_cast<uint32_t>(lane) & 31u) * 64u, D - 1));
            }
        // the rest of the top-k while the rows land
        topk_net_finish<VPL>(v, d.E, d.K, d.norm_topk, my_id, my_w, slots, net);
        // (clamped: a timed-out exchange must still index inside the pool)
        expert = min(readlane_u32(my_id, static_cast<int>(x)), d.E - 1);
        blob = L.experts + static_cast<size_t>(expert) * L.stride;
        // a proposal the exact selection overturned (ties, values equal
        // after rounding): the rows again, of the selected expert
        if (expert != prop) {
            if constexpr (DFIRST)
                if (t < n_down) issue_down(blob);
            if (t < n_up) issue_up(blob);
            // (rare: the new rows land before the dots start, so the rows of
            // the usual path keep counted waits, row by row as they land)
            vm_wait_all();
        }
    } else {
        expert = prop;
        blob = L.experts + static_cast<size_t>(prop) * L.stride;
    }
    // (the routing outputs are stored at the end of the layer: a store here,
    // in one wave's branch, would leave the loads in flight uncounted, and
    // the compiler drains the wave's memory operations before it anywhere
    // earlier)
    auto store_routing = [&] {
        if (x == 0 && t == 0 && static_cast<uint32_t>(lane) < d.K) {
            ids_out[lane] = my_id;
            w_out[lane] = my_w;
        }
    };

    // 3. gate/up rows of rank x -> h
    if (t < n_up) {
        if constexpr (!PROPOSE) issue_up(blob);
        __builtin_amdgcn_sched_barrier(0);
        if constexpr (GATHER) {
            sc_up[0][lane] = qa_s;
            sc_up[GATHER ? 1 : 0][lane] = qb_s;
            if constexpr (QF) {
                sc_up[QF ? 2 : 0][lane] = qa_m;
                sc_up[QF ? 3 : 0][lane] = qb_m;
            }
            __builtin_amdgcn_wave_barrier();
        }
        const uint16_t* sga = reinterpret_cast<const uint16_t*>(sc_up[0]);
        const uint16_t* sgb = reinterpret_cast<const uint16_t*>(sc_up[GATHER ? 1 : 0]);
        const uint16_t* mga = reinterpret_cast<const uint16_t*>(sc_up[QF ? 2 : 0]);
        const uint16_t* mgb = reinterpret_cast<const uint16_t*>(sc_up[QF ? 3 : 0]);
        float part[NR];
#pragma unroll
        for (int i = 2 * RB; i < NR; ++i) part[i] = 0.f;
#pragma unroll
        for (int i = 0; i < RB; ++i) {
            float ga = 0.f, ua = 0.f;
#pragma unroll
            for (int j = 0; j < CPL; ++j) {
                const uint32_t si = i * row_scales + (min(lane + WAVE * j, nch - 1) * 32) / LX_GROUP;
                const uint16_t s_a = GATHER ? sga[si] : sva[GATHER ? 0 : i][j];
                const uint16_t s_b = GATHER ? sgb[si] : svb[GATHER ? 0 : i][j];
                if constexpr (QF) {
                    ga += q4_chunk_affine(va[i][j], qa[j], bf16_to_f32(s_a), bf16_to_f32(mga[si]));
                    ua += q4_chunk_affine(vb[i][j], qa[j], bf16_to_f32(s_b), bf16_to_f32(mgb[si]));
                } else {
                    ga = fmaf(f16_bits_to_f32(s_a), q4_chunk_dot8(va[i][j], qa[j]), ga);
                    ua = fmaf(f16_bits_to_f32(s_b), q4_chunk_dot8(vb[i][j], qa[j]), ua);
                }
            }
            part[2 * i] = ga;
            part[2 * i + 1] = ua;
        }
        constexpr int USH = 6 - ilog2(NR);
        const float tot = wave_sum_rows<NR>(part);
        const float gv = __shfl(tot, (2 * lane) << USH);
        const float uv = __shfl(tot, (2 * lane + 1) << USH);
        // silu(z) = z * (1 / (1 + exp(-z)))  (kernels.metal:61-63, :334-336)
        if (lane < RB) put_local(hxc + rowg + lane, lx_word((gv * (1.0f / (1.0f + expf(-gv)))) * uv, tag));
        __builtin_amdgcn_sched_barrier(0);
    }

    // 4. down rows of rank x against all of h, staged in LDS (NW > 1: one
    //    copy per block, gathered by all of its waves when any has down rows).
    //    GATHER configurations store it quad-major: quad q (values 4q ..
    //    4q + 3) of 32-value chunk c at float4 q * (CH + 1) + c, so the 64
    //    lanes reading quad q of their chunks touch consecutive addresses (the
    //    + 1 spreads the writes of a pass over the banks); the wide ones (two
    //    passes of writes per round) keep h in order, which measured 1.1 us
    //    faster at 235B.
    __shared__ __align__(16) float h_s[8 * (LX_MAX_I / 32 + 1) * 4];
    const uint32_t chp = CH + 1;
    auto hpos = [&](uint32_t k) {
        return GATHER ? (((k & 31u) >> 2) * chp + (k >> 5)) * 4u + (k & 3u) : k;
    };
    if ((NW > 1 ? t - wv : t) < n_down) {
        // (after h is published: a memory operation waits for the requests
        // the CU has queued ahead of it, so a publication behind these rows
        // would wait for them; issued with the gate/up rows, or once those
        // have landed, they delay h by more than they save)
        if constexpr (!DFIRST)
            if (t < n_down) issue_down(blob);
        // passes of words per lane, every load of a pass in flight before any
        // is checked
        if constexpr (NW > 1) {
            // wave wv polls words wv * 64 + lane + k * NW * 64
            constexpr uint32_t NPW = (LX_MAX_I + NW * WAVE - 1) / (NW * WAVE);
            uint32_t spins = 0;
            bool all;
            do {
                all = true;
                uint64_t w64[NPW];
#pragma unroll
                for (uint32_t m = 0; m < NPW; ++m) {
                    const uint32_t k = (m * NW + wv) * WAVE + lane;
                    if (k < d.I) w64[m] = get_agent(hxc + k);
                }
#pragma unroll
                for (uint32_t m = 0; m < NPW; ++m) {
                    const uint32_t k = (m * NW + wv) * WAVE + lane;
                    if (k < d.I) {
                        h_s[hpos(k)] = __uint_as_float(static_cast<uint32_t>(w64[m]));
                        all &= static_cast<uint32_t>(w64[m] >> 32) == tag;
                    }
                }
                all = __ballot(!all) == 0;
                if (!all) {
                    if (give_up(++spins, io)) {
                        timed_out = true;
                        break;
                    }
                    __builtin_amdgcn_s_sleep(1);
                }
            } while (!all);
            __syncthreads();
        } else {
            // (addresses past the end re-read word I - 1)
            const uint32_t passes = (d.I + 16 * WAVE - 1) / (16 * WAVE);
            uint32_t spins = 0;
            bool all;
            do {
                all = true;
                for (uint32_t p = 0; p < passes; ++p) {
                    uint64_t w64[16];
#pragma unroll
                    for (int m = 0; m < 16; ++m)
                        w64[m] = get_agent(hxc + min(p * 16 * WAVE + lane + WAVE * m, d.I - 1));
#pragma unroll
                    for (int m = 0; m < 16; ++m) {
                        h_s[hpos(min(p * 16 * WAVE + lane + WAVE * m, d.I - 1))] =
                            __uint_as_float(static_cast<uint32_t>(w64[m]));
                        all &= static_cast<uint32_t>(w64[m] >> 32) == tag;
                    }
                }
                all = __ballot(!all) == 0;
                if (!all) {
                    if (give_up(++spins, io)) {
                        timed_out = true;
                        break;
                    }
                    __builtin_amdgcn_s_sleep(1);
                }
            } while (!all);
            __builtin_amdgcn_wave_barrier();
        }
    }
    if (t < n_down) {
        float hx[32];
        {
            const float4* hp = reinterpret_cast<const float4*>(h_s);
#pragma unroll
            for (int q = 0; q < 8; ++q) {
                const float4 f = hp[GATHER ? q * chp + dc : dc * 8 + q];
                hx[4 * q + 0] = f.x;
                hx[4 * q + 1] = f.y;
                hx[4 * q + 2] = f.z;
                hx[4 * q + 3] = f.w;
            }
        }
        Q4Act qh;
        q4_act_from_floats(hx, qh);
        if constexpr (GATHER) {
#pragma unroll
            for (int k = 0; k < NSD; ++k) sc_dn[k * WAVE + lane] = qd_s[k];
            if constexpr (QF) {
#pragma unroll
                for (int k = 0; k < NSD; ++k) sc_dn[(NSD + k) * WAVE + lane] = qd_m[QF ? k : 0];
            }
            __builtin_amdgcn_wave_barrier();
        }
        const uint16_t* sd = reinterpret_cast<const uint16_t*>(sc_dn);
        const uint16_t* sdm = reinterpret_cast<const uint16_t*>(sc_dn + (QF ? NSD * WAVE : 0));
        float acc[DR];
#pragma unroll
        for (int i = 0; i < DR; ++i) {
            const uint32_t si = (static_cast<uint32_t>(gi) * DR + i) * (d.I / LX_GROUP) + (dc * 32) / LX_GROUP;
            float y;
            if constexpr (QF)
                y = q4_chunk_affine(dv[i], qh, bf16_to_f32(sd[si]), bf16_to_f32(sdm[si]));
            else
                y = f16_bits_to_f32(GATHER ? sd[si] : dsv[GATHER ? 0 : i]) * q4_chunk_dot8(dv[i], qh);
            acc[i] = act ? y : 0.f;
        }
        // lane l holds the total of row (l >> SH) & (DR - 1) of group l >> SEG
        const float tot = seg_sum_rows<DR, SEG>(acc);
        const bool holder = (lane & ((1 << SH) - 1)) == 0;
        const uint32_t myrow = t * RW + (lane >> SEG) * DR + ((lane >> SH) & (DR - 1));
        if (holder) put_agent(py + x * py_stride + myrow, lx_word(tot, tag));

        // 5. combine of row block t (on XCD t % 8, or on every XCD for its own
        //    copy), in rank order
        if ((io.all_rows ? true : (t & 7u) == x) && io.hout) {
            const int src = ((lane / DR) << SEG) | ((lane % DR) << SH);   // holder of row t*RW + lane
            const float own = __shfl(tot, src & (WAVE - 1));
            if (lane < RW) {
                const uint32_t row = t * RW + lane;
                float y[8];
                uint32_t spins = 0;
                bool all;
                do {
                    all = true;
#pragma unroll
                    for (int r = 0; r < 8; ++r) {
                        // the own rank's word is read too (branch-free) and ignored
                        const uint64_t w64 = get_agent(py + r * py_stride + row);
                        const bool mine = static_cast<uint32_t>(r) == x;
                        y[r] = mine ? own : __uint_as_float(static_cast<uint32_t>(w64));
                        all &= mine || static_cast<uint32_t>(w64 >> 32) == tag;
                    }
                    if (!all && give_up(++spins, io)) {
                        timed_out = true;
                        break;
                    }
                } while (!all);
                float sum = 0.f;
#pragma unroll
                for (int r = 0; r < 8; ++r) sum = fmaf(readlane_f32(my_w, r), y[r], sum);
                // (the input as this wave read it at the start of the layer: no
                // other wave writes these rows before this one; blocks of
                // shared loads hold it in LDS)
                float hin_row;
                if constexpr (NW > 1) {
                    const uint32_t f = row >> 2;
                    hin_row = reinterpret_cast<const float*>(hid_s)[((f & 7u) * QS + (f >> 3)) * 4u + (row & 3u)];
                } else {
                    hin_row = io.hin[row];
                }
                io.hout[row] = hin_row + sum;
            }
            if (io.flag) {
                // the rows are in the L2 before the flag says so
                vm_wait_all();
                if (lane == 0) __hip_atomic_store(io.flag + t, tag, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WAVEFRONT);
            }
        }
    }
    store_routing();
    if (timed_out && io.abort && lane == 0)
        __hip_atomic_store(io.abort, io.abort_val, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    // (keeps the touch's register until every load of the layer has landed)
    if constexpr (CHAIN && CPL == 1) asm volatile("" ::"v"(touch));
    return timed_out;
}

// Blocks of NW waves; block b is the (b / 8)-th of its XCD, its wave w has
// t = NW (b / 8) + w.
template <int CPL, int VPL, int SEG, int DR, int RB, int NW, int QF>
__global__ __launch_bounds__(NW * WAVE)
void k_moe_layer(MoeDims d, LayerDesc L, float* __restrict__ hidden, uint64_t* __restrict__ lx,
                 uint32_t* __restrict__ ids_out, float* __restrict__ w_out, uint32_t n_up, uint32_t n_down,
                 uint32_t* __restrict__ err)
{
    const uint32_t nbx = (gridDim.x >> 3) * NW;
    const uint32_t t = (blockIdx.x >> 3) * NW + (NW > 1 ? __builtin_amdgcn_readfirstlane(threadIdx.x >> 6) : 0u);
    const uint32_t x = xcc_id();
    const uint32_t ep = __builtin_amdgcn_readfirstlane(static_cast<uint32_t>(get_agent(lx)));
    const uint32_t tag = tag_at(ep, 0);
    LayerIO io{};
    io.hin = hidden;
    io.hout = hidden;
    io.py = lx + LX_HEAD + 8u * lx_pad(d.E) + 8u * lx_pad(d.I);
    const bool to =
        moe_layer_step<CPL, VPL, SEG, DR, RB, NW, false, QF>(d, L, io, lx, tag, ids_out, w_out, n_up, n_down, t, x, nbx);
    // the combiner of row block 0 on XCD 0 advances the epoch
    if (x == 0 && t == 0 && t < n_down) {
        __builtin_amdgcn_wave_barrier();
        if ((threadIdx.x & (WAVE - 1)) == 0) put_agent(lx, static_cast<uint64_t>(epoch_after(ep, 1)));
    }
    if (to) atomicOr(err, 1u);
}

// Every layer of a decode step in one launch: the wave schedule of
// k_moe_layer per layer, with each XCD combining every row into its own copy
// of the next layer's input (in its L2; one flag per row block, carrying the
// layer's tag, says when it is complete) and the last layer combining into
// `hidden` on XCD 0.  The flags and the copy are only ever read by the XCD
// that wrote them, after the flags, past the CU's L1.  Tags: tag_at(epoch, l)
// for layer l (never 0, and never the same for two consecutive layers, in
// one launch or across launches, whatever the epoch); the rank partials
// alternate between two sets of words by layer parity (an XCD can start
// layer l + 1's partials while another XCD still reads layer l's, never layer
// l - 1's: that needs every XCD's layer l partials).  A wave that times out
// stores the abort word, after which every wait of the launch ends.
template <int CPL, int VPL, int SEG, int DR, int RB, int NW, int QF>
__global__ __launch_bounds__(NW * WAVE)
void k_moe_chain(MoeDims d, const LayerDesc* __restrict__ layers, uint32_t n_layers, float* __restrict__ hidden,
                 uint64_t* __restrict__ lx, float* __restrict__ hcopy, uint32_t* __restrict__ cnt,
                 uint32_t* __restrict__ ids_out, float* __restrict__ w_out, uint32_t n_up, uint32_t n_down,
                 uint32_t* __restrict__ err)
{
    const uint32_t nbx = (gridDim.x >> 3) * NW;
    const uint32_t t = (blockIdx.x >> 3) * NW + (NW > 1 ? __builtin_amdgcn_readfirstlane(threadIdx.x >> 6) : 0u);
    const uint32_t x = xcc_id();
    // read by every wave before any of them can change them (a change needs
    // every wave's router rows of layer 0)
    const uint32_t ep0 = __builtin_amdgcn_readfirstlane(static_cast<uint32_t>(get_agent(lx)));
    uint32_t* flags_x = cnt + x * CHAIN_FLAGS;
    float* hx = hcopy + static_cast<size_t>(x) * d.D;
    uint64_t* py0 = lx + LX_HEAD + 8u * lx_pad(d.E) + 8u * lx_pad(d.I);
    bool to = false;
    for (uint32_t l = 0; l < n_layers; ++l) {
        const LayerDesc L = layers[l];
        const bool last = l + 1 == n_layers;
        LayerIO io{};
        const uint32_t tag = tag_at(ep0, l), prev = tag_at(ep0, l - 1u);   // (prev: l > 0 only)
        io.hin = l == 0 ? hidden : hx;
        io.wait = l > 0 ? flags_x : nullptr;
        io.wait_tag = prev;
        io.hout = last ? (x == 0 ? hidden : nullptr) : hx;
        io.all_rows = true;
        io.flag = last ? nullptr : flags_x;
        io.py = py0 + (l & 1u) * 8u * lx_pad(d.D);
        io.abort = cnt + 8 * CHAIN_FLAGS;
        io.abort_val = tag_at(ep0, 0);
        io.next_router = last ? nullptr : layers[l + 1].router_w;
        to |= moe_layer_step<CPL, VPL, SEG, DR, RB, NW, true, QF>(d, L, io, lx, tag, ids_out + l * d.K,
                                                               w_out + l * d.K, n_up, n_down, t, x, nbx);
    }
    // wave 0 of XCD 0 advances the epoch once its last combine is done (that
    // needs every wave's last partials)
    if (x == 0 && t == 0) {
        __builtin_amdgcn_wave_barrier();
        if ((threadIdx.x & (WAVE - 1)) == 0) put_agent(lx, static_cast<uint64_t>(epoch_after(ep0, n_layers)));
    }
    if (to) atomicOr(err, 1u);
}

namespace {

struct LayerCfg {
    int cpl, vpl, seg, dr, rb;
    uint32_t n_up, n_down, nbx;
};

// Waves per block where the block shares its loads, one block per CU of all
// the CU's waves: the wide (235B) family, 8 or 6 (each wave would otherwise
// read 24 KB of hidden state and norm weights: 28.3 against 29.7 us per layer
// with 6), and the narrow (30B) family in the chained kernel, 4 (the block
// reads the XCD's copy of the input once and polls its flags and the h copy
// with one wave's share each: 1772 against 1755 tok/s; the one-launch layer
// kernel keeps one-wave blocks, 1 % faster there).
constexpr bool shares_loads(int cpl, int seg) { return (cpl == 2 && seg == 6) || (cpl == 1 && seg == 5); }

template <int CPL, int VPL, int SEG, int DR, int RB, bool CHAIN, int NW, int QF>
auto kernel_of()
{
    if constexpr (CHAIN) return k_moe_chain<CPL, VPL, SEG, DR, RB, NW, QF>;
    else return k_moe_layer<CPL, VPL, SEG, DR, RB, NW, QF>;
}

// Dynamic LDS added to a block of NW > 1 waves so that only one fits on a CU
// (its waves then have the CU's memory path to themselves, as the one-wave
// blocks of a grid spread four or six to a CU do).
template <int CPL, int VPL, int SEG, int DR, int RB, bool CHAIN, int NW, int QF>
uint32_t lds_pad()
{
    static uint32_t pad = [] {
        if (NW == 1) return 0u;
        hipFuncAttributes attr{};
        if (hipFuncGetAttributes(&attr, reinterpret_cast<const void*>(kernel_of<CPL, VPL, SEG, DR, RB, CHAIN, NW, QF>())) !=
            hipSuccess)
            return 0u;
        const size_t want = 82u * 1024u;
        return attr.sharedSizeBytes < want ? static_cast<uint32_t>(want - attr.sharedSizeBytes) : 0u;
    }();
    return pad;
}

template <int CPL, int VPL, int SEG, int DR, int RB, bool CHAIN, int NW, int QF>
uint32_t resident_blocks()
{
    static uint32_t cap = [] {
        int dev = 0, per_cu = 0, cus = 0;
        if (hipGetDevice(&dev) != hipSuccess) return 0u;
        if (hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess) return 0u;
        if (hipOccupancyMaxActiveBlocksPerMultiprocessor(&per_cu, kernel_of<CPL, VPL, SEG, DR, RB, CHAIN, NW, QF>(),
                                                         NW * WAVE, lds_pad<CPL, VPL, SEG, DR, RB, CHAIN, NW, QF>()) !=
            hipSuccess)
            return 0u;
        return static_cast<uint32_t>(per_cu) * static_cast<uint32_t>(cus);
    }();
    return cap;
}

bool layer_cfg(const MoeDims& d, LayerCfg& c)
{
    if (d.K != 8 || d.group != 64 || d.E == 0 || d.E > SMOE_TOPK_MAX_N) return false;
    if (d.D % 64 || d.I % 64 || d.I > LX_MAX_I) return false;
    const uint32_t nch = d.D / 32;
    c.cpl = nch <= 64 ? 1 : nch <= 128 ? 2 : 0;
    if (!c.cpl) return false;
    c.vpl = d.E <= 128 ? 2 : 8;
    // the scale+min format: the gathered-scale (narrow, proposing) configurations
    if (d.quant != 0 && (c.cpl != 1 || c.vpl != 2)) return false;
    const uint32_t ch = d.I / 32;
    if (ch <= 32) {
        c.seg = 5;
        c.dr = 8;
    } else {
        // 16 down rows per wave where 6 gate/up rows then give every wave a row
        // block of each (two equal waves per SIMD), else 32
        c.seg = 6;
        c.dr = (d.I % 6 == 0 && d.D % 16 == 0 && d.I / 6 == d.D / 16) ? 16 : 32;
    }
    const uint32_t rw = (64u >> c.seg) * c.dr;
    if (d.D % rw) return false;
    // down scales of a wave's rows: 16-byte pieces, at most NSD per lane
    if ((rw * d.I / 32) % 16 || rw * d.I / 512 > 64u * ((rw * (c.seg == 5 ? 1024u : 2048u) / 512 + 63) / 64))
        return false;
    c.n_down = d.D / rw;
    // 6 gate/up rows per wave where that gives every wave a row block: less
    // dot-product work per wave than 8 rows on 3/4 of them
    c.rb = (d.I % 6 == 0 && d.I / 6 == c.n_down && (6 * d.D / 32) % 16 == 0) ? 6 : LX_UP_RB;
    // gate/up scales of a wave's rows: 16-byte pieces, one per lane
    if ((c.rb * d.D / 32) % 16 || c.rb * d.D / 512 > 64) return false;
    c.n_up = d.I / c.rb;
    c.nbx = std::max(c.n_up, c.n_down);
    // every wave produces a router row or a gate/up row block
    if (c.nbx > std::max(d.E, c.n_up)) return false;
    return true;
}

// the arguments of a launch of either kernel (chain: `layers` [n_layers],
// hcopy and cnt set)
struct LaunchArgs {
    const LayerDesc* L = nullptr;       // one layer (host struct)
    const LayerDesc* layers = nullptr;  // the chain's table (device)
    uint32_t n_layers = 0;
    float* hidden = nullptr;
    uint64_t* lx = nullptr;
    float* hcopy = nullptr;
    uint32_t* cnt = nullptr;
    uint32_t* ids = nullptr;
    float* w = nullptr;
    uint32_t* err = nullptr;
};

template <int CPL, int VPL, int SEG, int DR, int RB, bool CHAIN, int NW, int QF>
hipError_t launch_nw(const LayerCfg& c, const MoeDims& d, const LaunchArgs& a, hipStream_t s, bool dry)
{
    const uint32_t blocks = 8u * c.nbx / NW;
    if (blocks > resident_blocks<CPL, VPL, SEG, DR, RB, CHAIN, NW, QF>() || (CHAIN && c.n_down > CHAIN_FLAGS))
        return hipErrorInvalidConfiguration;
    if (dry) return hipSuccess;
    const uint32_t pad = lds_pad<CPL, VPL, SEG, DR, RB, CHAIN, NW, QF>();
    if constexpr (CHAIN)
        launch_kernel_lds(k_moe_chain<CPL, VPL, SEG, DR, RB, NW, QF>, dim3(blocks), dim3(NW * WAVE), pad, s, d,
                          a.layers, a.n_layers, a.hidden, a.lx, a.hcopy, a.cnt, a.ids, a.w, c.n_up, c.n_down, a.err);
    else
        launch_kernel_lds(k_moe_layer<CPL, VPL, SEG, DR, RB, NW, QF>, dim3(blocks), dim3(NW * WAVE), pad, s, d, *a.L,
                          a.hidden, a.lx, a.ids, a.w, c.n_up, c.n_down, a.err);
    return hipGetLastError();
}

template <int CPL, int VPL, int SEG, int DR, int RB, int QF>
hipError_t launch_cfg(const LayerCfg& c, const MoeDims& d, const LaunchArgs& a, bool chain, hipStream_t s, bool dry)
{
    if constexpr (shares_loads(CPL, SEG) && CPL == 1) {
        if (chain && c.nbx % 4 == 0) return launch_nw<CPL, VPL, SEG, DR, RB, true, 4, QF>(c, d, a, s, dry);
    } else if constexpr (shares_loads(CPL, SEG)) {
        // a block of shared loads where the grid divides into them (one per CU:
        // 256 or 192 waves an XCD)
        if (c.nbx % 8 == 0)
            return chain ? launch_nw<CPL, VPL, SEG, DR, RB, true, 8, QF>(c, d, a, s, dry)
                         : launch_nw<CPL, VPL, SEG, DR, RB, false, 8, QF>(c, d, a, s, dry);
        if (c.nbx % 6 == 0)
            return chain ? launch_nw<CPL, VPL, SEG, DR, RB, true, 6, QF>(c, d, a, s, dry)
                         : launch_nw<CPL, VPL, SEG, DR, RB, false, 6, QF>(c, d, a, s, dry);
    }
    return chain ? launch_nw<CPL, VPL, SEG, DR, RB, true, 1, QF>(c, d, a, s, dry)
                 : launch_nw<CPL, VPL, SEG, DR, RB, false, 1, QF>(c, d, a, s, dry);
}

hipError_t dispatch(const MoeDims& d, const LaunchArgs& a, bool chain, hipStream_t s, bool dry)
{
    LayerCfg c;
    if (!layer_cfg(d, c)) return hipErrorInvalidValue;
#define SMOE_LAYER_CASE_Q(C, V, S, R, Q)                                                      \
    if (c.cpl == C && c.vpl == V && c.seg == S && c.dr == R && c.rb == 8)                     \
        return launch_cfg<C, V, S, R, 8, Q>(c, d, a, chain, s, dry);                          \
    if (c.cpl == C && c.vpl == V && c.seg == S && c.dr == R && c.rb == 6)                     \
        return launch_cfg<C, V, S, R, 6, Q>(c, d, a, chain, s, dry);
#define SMOE_LAYER_CASE(C, V, S, R) SMOE_LAYER_CASE_Q(C, V, S, R, 0)
    if (d.quant != 0) {
        // the scale+min format (layer_cfg admits the narrow configurations only)
        SMOE_LAYER_CASE_Q(1, 2, 5, 8, 1)
        SMOE_LAYER_CASE_Q(1, 2, 6, 16, 1)
        SMOE_LAYER_CASE_Q(1, 2, 6, 32, 1)
        return hipErrorInvalidValue;
    }
    SMOE_LAYER_CASE(1, 2, 5, 8)
    SMOE_LAYER_CASE(1, 2, 6, 16)
    SMOE_LAYER_CASE(1, 2, 6, 32)
    SMOE_LAYER_CASE(1, 8, 5, 8)
    SMOE_LAYER_CASE(1, 8, 6, 16)
    SMOE_LAYER_CASE(1, 8, 6, 32)
    SMOE_LAYER_CASE(2, 2, 5, 8)
    SMOE_LAYER_CASE(2, 2, 6, 16)
    SMOE_LAYER_CASE(2, 2, 6, 32)
    SMOE_LAYER_CASE(2, 8, 5, 8)
    SMOE_LAYER_CASE(2, 8, 6, 16)
    SMOE_LAYER_CASE(2, 8, 6, 32)
#undef SMOE_LAYER_CASE
#undef SMOE_LAYER_CASE_Q
    return hipErrorInvalidValue;
}

}  // namespace

// ---------------------------------------------------------------------------
// The layer kernels take a wave's XCD-local index from its block id (t = b / 8
// on XCD XCC_ID), which holds when the dispatcher deals consecutive blocks
// round-robin over the 8 XCDs.  Checked once per device (at context set-up):
// a grid of one-wave blocks records each block's XCC_ID; anything but
// (XCC_ID - b) mod 8 constant over the grid turns both kernels off (their
// shapes then take the two-launch path, which does not depend on it).
// ---------------------------------------------------------------------------
__global__ __launch_bounds__(WAVE) void k_deal_probe(uint32_t* out)
{
    if (threadIdx.x == 0) out[blockIdx.x] = xcc_id();
}

namespace {
constexpr uint32_t DEAL_BLOCKS = 4096;   // >= 8 x the most waves per XCD a layer kernel launches
constexpr int DEAL_MAX_DEVICES = 64;
std::mutex g_deal_mu;
int g_deal[DEAL_MAX_DEVICES] = {};       // 0 unknown, 1 round-robin, 2 not
}  // namespace

bool deal_probe()
{
    int dev = 0;
    if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= DEAL_MAX_DEVICES) return false;
    std::lock_guard<std::mutex> lock(g_deal_mu);
    if (g_deal[dev]) return g_deal[dev] == 1;
    hipStream_t s = nullptr;
    uint32_t* buf = nullptr;
    std::vector<uint32_t> h(DEAL_BLOCKS, 8u);
    bool ran = hipStreamCreateWithFlags(&s, hipStreamNonBlocking) == hipSuccess &&
               hipMalloc(&buf, DEAL_BLOCKS * sizeof(uint32_t)) == hipSuccess;
    if (ran) {
        hipLaunchKernelGGL(k_deal_probe, dim3(DEAL_BLOCKS), dim3(WAVE), 0, s, buf);
        ran = hipGetLastError() == hipSuccess && hipStreamSynchronize(s) == hipSuccess &&
              hipMemcpy(h.data(), buf, DEAL_BLOCKS * sizeof(uint32_t), hipMemcpyDeviceToHost) == hipSuccess;
    }
    if (buf) (void)hipFree(buf);
    if (s) (void)hipStreamDestroy(s);
    if (!ran) return false;   // unknown: tried again at the next set-up
    bool rr = h[0] < 8;
    for (uint32_t b = 1; rr && b < DEAL_BLOCKS; ++b) rr = h[b] == ((h[0] + b) & 7u);
    if (!rr)
        std::fprintf(stderr, "[smoe_hip] blocks are not dealt round-robin over 8 XCDs on device %d: the one-launch "
                             "decode kernels are off, decode takes two launches per layer\n", dev);
    g_deal[dev] = rr ? 1 : 2;
    return rr;
}

static bool deal_known_round_robin()
{
    int dev = 0;
    if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= DEAL_MAX_DEVICES) return false;
    std::lock_guard<std::mutex> lock(g_deal_mu);
    return g_deal[dev] == 1;
}

static bool layer_aligned(const LayerDesc& L)
{
    // 16-byte pieces of every tensor (the reference's blobs place tensors
    // back to back with sizes that are multiples of 16), the norm weights and
    // router rows included (both read with 16-byte loads)
    bool aligned = reinterpret_cast<uintptr_t>(L.experts) % 16 == 0 && L.stride % 16 == 0 &&
                   reinterpret_cast<uintptr_t>(L.norm_w) % 16 == 0 && reinterpret_cast<uintptr_t>(L.router_w) % 16 == 0;
    for (int i = 0; i < 6; ++i) aligned = aligned && L.off[i] % 16 == 0;
    return aligned;
}

bool layer_supported(const MoeDims& d, const LayerDesc& L)
{
    return layer_aligned(L) && deal_known_round_robin() && dispatch(d, LaunchArgs{}, false, nullptr, true) == hipSuccess;
}

hipError_t launch_moe_layer(const MoeDims& d, const LayerDesc& L, float* hidden, uint64_t* lx, uint32_t* ids,
                            float* w, uint32_t* err, hipStream_t s)
{
    if (!layer_supported(d, L)) return hipErrorInvalidValue;
    LaunchArgs a;
    a.L = &L;
    a.hidden = hidden;
    a.lx = lx;
    a.ids = ids;
    a.w = w;
    a.err = err;
    return dispatch(d, a, false, s, false);
}

bool chain_supported(const MoeDims& d, const LayerDesc* layers_host, uint32_t n_layers)
{
    // the narrow configurations (one chunk of 32 columns per lane), and the
    // wide ones with 16 down rows a wave: with 32 the chained kernel spilled
    // registers (32.2 against 28.3 us per 235B layer for the per-layer launches)
    LayerCfg c;
    if (!layer_cfg(d, c) || (c.cpl != 1 && c.dr != 16)) return false;
    for (uint32_t l = 0; l < n_layers; ++l)
        if (!layer_aligned(layers_host[l])) return false;
    return n_layers > 0 && deal_known_round_robin() && dispatch(d, LaunchArgs{}, true, nullptr, true) == hipSuccess;
}

hipError_t launch_moe_chain(const MoeDims& d, const LayerDesc* layers_dev, uint32_t n_layers, float* hidden,
                            uint64_t* xch, float* hcopy, uint32_t* cnt, uint32_t* ids, float* w, uint32_t* err,
                            hipStream_t s)
{
    LaunchArgs a;
    a.layers = layers_dev;
    a.n_layers = n_layers;
    a.hidden = hidden;
    a.lx = xch;
    a.hcopy = hcopy;
    a.cnt = cnt;
    a.ids = ids;
    a.w = w;
    a.err = err;
    return dispatch(d, a, true, s, false);
}

}  // namespace smoe
