// moe_stack.hip -- one batch-1 decode step through every MoE layer of the
// stack (the decode.cpp:121 layer loop over decode.cpp:236-509) in ONE
// persistent launch.
//
// 256 blocks of 4 waves, one block per CU.  Block b runs on XCD b % 8 (the
// dispatcher's round-robin over the 8 XCDs), so every XCD holds 32 blocks =
// 128 waves; wave jw = (b / 8) * 4 + wave-in-block indexes the waves of one
// XCD.  Per layer:
//   H  every block reads the layer's input hidden [D] into LDS (layer 0: the
//      caller's buffer; later layers: the words its own XCD published in C);
//   N  RMSNorm in every wave (common.hpp:245-256);
//   R  each XCD computes all E router logits (common.hpp:293-306), row jw of
//      wave jw, from router rows that were prefetched into registers during
//      the previous layer, and publishes them for its own waves;
//   T  every wave polls its XCD's E logits and runs softmax + top-k
//      (scout.cpp:77-123, renormalised as decode.cpp:296-302) itself;
//   U  XCD x owns the experts of ranks x, x + 8, ...: each of its waves
//      streams I/128 rows of gate and up (kernels.metal:240-337) and
//      publishes h;
//   D  the XCD's blocks read the rank's h [I] and each wave streams D/128
//      down rows (kernels.metal:340-365), publishing y_r [D] to every XCD;
//   C  every XCD combines hidden + sum_r w_r y_r (decode.cpp:482-509, rank
//      order) for all D rows (D/128 rows per wave) and publishes the next
//      layer's hidden to its own blocks.
// No kernel boundary separates the phases or the layers.  Exchanges are
// 64-bit words (flag << 32 | fp32 value) whose flag is the epoch of the layer:
// a consumer polls the words themselves, so one round trip both synchronises
// and delivers.  Epochs grow by n_layers per call (the last block to finish
// advances a control word), so no word is ever re-armed.  Every wait is
// bounded: a time-out flags err bit 0 and every wave then stops waiting, so
// the grid always drains.
#include "device_common.hpp"
#include "kernels.hpp"
#include "topk.hpp"

namespace smoe {

namespace {

constexpr uint32_t ST_SPIN_LIMIT = 1u << 20;

__device__ __forceinline__ uint64_t xword(uint32_t ep, float v)
{
    return (static_cast<uint64_t>(ep) << 32) | __float_as_uint(v);
}
// A word for every XCD: an agent-scope store, written through to memory.
__device__ __forceinline__ void put_word(uint64_t* p, uint32_t ep, float v)
{
    __hip_atomic_store(p, xword(ep, v), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
// A word for the waves of the writer's own XCD: a plain store, which stays in
// that XCD's L2, where their agent-scope (sc1) loads find it; written through
// like put_word when `local` is off.
__device__ __forceinline__ void put_word_xcd(uint64_t* p, uint32_t ep, float v, bool local)
{
    if (local)
        __hip_atomic_store(p, xword(ep, v), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WAVEFRONT);
    else
        __hip_atomic_store(p, xword(ep, v), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ uint64_t get_word(const uint64_t* p)
{
    return __hip_atomic_load(const_cast<uint64_t*>(p), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ uint32_t get_u32(const uint32_t* p)
{
    return __hip_atomic_load(const_cast<uint32_t*>(p), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ bool flag_is(uint64_t w, uint32_t ep) { return static_cast<uint32_t>(w >> 32) == ep; }
__device__ __forceinline__ float word_value(uint64_t w) { return __uint_as_float(static_cast<uint32_t>(w)); }

// Re-runs `round` (which issues its loads and returns whether this lane's
// words are all present) until it holds on every lane of the wave.  Gives up
// after ST_SPIN_LIMIT rounds (flagging err bit 0) or as soon as any wave has
// flagged an error; `dead` then makes every later wait of this wave return at
// once, so the grid drains instead of hanging.
template <typename F>
__device__ __forceinline__ void poll_until(F&& round, uint32_t* err, bool& dead)
{
    uint32_t spins = 0;
    for (;;) {
        const bool ok = round();
        if (__ballot(!ok) == 0 || dead) return;
        if ((++spins & 63u) == 0) {
            if (__builtin_amdgcn_readfirstlane(static_cast<int>(get_u32(err))) != 0) {
                dead = true;
                return;
            }
            if (spins >= ST_SPIN_LIMIT) {
                if ((threadIdx.x & 63) == 0) atomicOr(err, 1u);
                dead = true;
                return;
            }
        }
    }
}

// A wave-uniform copy of a descriptor read from LDS (scalar registers: the
// weight loads then take a scalar base and a 32-bit lane offset).
template <typename T>
__device__ __forceinline__ T* uniform_ptr(T* p)
{
    const uint64_t v = reinterpret_cast<uint64_t>(p);
    const uint32_t lo = __builtin_amdgcn_readfirstlane(static_cast<uint32_t>(v));
    const uint32_t hi = __builtin_amdgcn_readfirstlane(static_cast<uint32_t>(v >> 32));
    return reinterpret_cast<T*>((static_cast<uint64_t>(hi) << 32) | lo);
}
__device__ __forceinline__ uint64_t uniform_u64(uint64_t v)
{
    const uint32_t lo = __builtin_amdgcn_readfirstlane(static_cast<uint32_t>(v));
    const uint32_t hi = __builtin_amdgcn_readfirstlane(static_cast<uint32_t>(v >> 32));
    return (static_cast<uint64_t>(hi) << 32) | lo;
}
__device__ __forceinline__ LayerDesc uniform_desc(const LayerDesc& s)
{
    LayerDesc d;
    d.norm_w = uniform_ptr(s.norm_w);
    d.router_w = uniform_ptr(s.router_w);
    d.experts = uniform_ptr(s.experts);
    d.stride = uniform_u64(s.stride);
#pragma unroll
    for (int i = 0; i < 6; ++i) d.off[i] = uniform_u64(s.off[i]);
    return d;
}

// LDS float4 index of quad q of 32-value chunk c (f = 8 c + q), rotated so
// that 64 lanes reading quad q of chunks lane, lane + 64, ... spread over the
// banks.
__device__ __forceinline__ uint32_t swz4(uint32_t f) { return (f & ~7u) | ((f ^ (f >> 3)) & 7u); }

// v, or +0 where mask is 0 (a bitwise select: no branch around the LDS read
// that produced v)
__device__ __forceinline__ float4 keep4(float4 v, uint32_t mask)
{
    return make_float4(__uint_as_float(__float_as_uint(v.x) & mask), __uint_as_float(__float_as_uint(v.y) & mask),
                       __uint_as_float(__float_as_uint(v.z) & mask), __uint_as_float(__float_as_uint(v.w) & mask));
}

}  // namespace

// control words (ctl[]): epoch and mode share the line every block reads at
// start; the counters have a line each (tickets: one line per XCD).  Mode 1 =
// an XCD once received more than its share of blocks, so placement by XCD is
// off (block b takes role b % 8, b / 8 and every word is written through)
// from then on.
constexpr uint32_t CTL_EPOCH = 0, CTL_MODE = 1, CTL_DONE = 32, CTL_ARRIVED = 64, CTL_TICKET = 96;

// Exchange words of one layer: logits [8 XCDs][E'], h [K][I'], y [K][D],
// next hidden [8 XCDs][D]; E' and I' rounded up to 32 words.
struct StackLayout {
    uint32_t log_x, hrg_r, yr_r, hid_x;
    size_t layer;
    __host__ __device__ StackLayout(const MoeDims& d)
        : log_x((d.E + 31u) & ~31u), hrg_r((d.I + 31u) & ~31u), yr_r(d.D), hid_x(d.D),
          layer(8 * size_t(log_x) + size_t(d.K) * hrg_r + size_t(d.K) * yr_r + 8 * size_t(hid_x))
    {
    }
};

size_t stack_xch_words(const MoeDims& d, uint32_t n_layers) { return StackLayout(d).layer * n_layers; }

// VPL/RRW: logits per lane / router rows per wave (2/1: E <= 128, 8/4: E <= 512);
// CW: lanes per down row, a power of two >= I / 32 (8, 32 or 64).
// d_model <= 2048 only (stack_supported): one 32-column chunk of D per lane,
// and at most 16 combine rows per wave (D / 128), which is what y_s holds.
template <int VPL, int RRW, int CW>
__global__ __launch_bounds__(ST_THREADS, 1)
void k_decode_stack(MoeDims d, const LayerDesc* __restrict__ layers, uint32_t n_layers, float* __restrict__ hidden,
                    uint64_t* __restrict__ xch, uint32_t* __restrict__ ctl, uint32_t* __restrict__ ids_out,
                    float* __restrict__ w_out, uint32_t* __restrict__ err)
{
    constexpr int CPL = 1;                       // 32-column chunks of D per lane
    constexpr int HG = 2 * CPL;                  // float4 groups of hidden per thread
    constexpr int HGI = (CW * 8 + ST_THREADS - 1) / ST_THREADS;   // float4 groups of h per thread
    constexpr int SEG = ilog2(CW);
    constexpr int DG = CW >= 8 ? 8 : CW;         // down batches per group
    constexpr int LDG = ilog2(DG);
    constexpr int RPB = WAVE / CW;               // down rows per batch
    constexpr int UG = 6;                        // gate/up rows per group
    __shared__ float4 hid_s[CPL * 512];
    __shared__ float4 h_s[CW * 8];
    __shared__ LayerDesc tbl_s[ST_MAX_LAYERS];
    __shared__ uint2 topk_s[ST_WPB][TOPK_SLOTS];
    __shared__ float y_s[SMOE_TOPK_MAX_K][ST_WPB * 16];   // the block's combine rows, all ranks

    // wv is wave-uniform: readfirstlane lets row and address arithmetic stay scalar
    const int tid = threadIdx.x, lane = tid & 63, wv = __builtin_amdgcn_readfirstlane(tid >> 6);
    // Role of this block: XCD x and index jb among that XCD's 32 blocks.  The
    // dispatcher deals blocks round-robin over the 8 XCDs, but not always
    // starting at XCD 0, so each block takes the XCD it runs on (XCC_ID) and a
    // ticket among that XCD's blocks.  Words meant for one XCD's waves then
    // stay in its L2 (plain stores).  Should an XCD ever receive more than 32
    // blocks, the call is flagged and later calls place by block id and write
    // every word through.
    __shared__ uint32_t role_s;
    const uint32_t b = blockIdx.x;
    const bool by_xcd = __builtin_amdgcn_readfirstlane(static_cast<int>(get_u32(ctl + CTL_MODE))) == 0;
    if (tid == 0) {
        uint32_t xcc;
        asm volatile("s_getreg_b32 %0, hwreg(HW_REG_XCC_ID, 0, 4)" : "=s"(xcc));
        uint32_t role = ((b >> 3) << 3) | (b & 7u);
        if (by_xcd) {
            const uint32_t t = __hip_atomic_fetch_add(ctl + CTL_TICKET + 32 * xcc, 1u, __ATOMIC_RELAXED,
                                                      __HIP_MEMORY_SCOPE_AGENT);
            if (t < ST_BLOCKS / 8) {
                role = (t << 3) | xcc;
            } else {
                role = 0xFFFFFFFFu;   // surplus block: no role
                atomicOr(err, 4u);
                __hip_atomic_store(ctl + CTL_MODE, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
            }
        }
        role_s = role;
    }
    __syncthreads();
    const uint32_t role = __builtin_amdgcn_readfirstlane(static_cast<int>(role_s));
    const bool has_role = role != 0xFFFFFFFFu;
    const bool local = by_xcd;
    const uint32_t x = role & 7u, jw = (role >> 3) * ST_WPB + wv;
    const uint32_t D = d.D, E = d.E, K = d.K, I = d.I;
    const uint32_t nch = D >> 5, nchI = I >> 5;
    const StackLayout lay(d);
    auto LOG = [&](uint32_t l) { return xch + l * lay.layer + size_t(x) * lay.log_x; };
    auto HRG = [&](uint32_t l, uint32_t r) { return xch + l * lay.layer + 8 * size_t(lay.log_x) + size_t(r) * lay.hrg_r; };
    auto YR = [&](uint32_t l, uint32_t r) {
        return xch + l * lay.layer + 8 * size_t(lay.log_x) + size_t(K) * lay.hrg_r + size_t(r) * lay.yr_r;
    };
    auto HID = [&](uint32_t l) {
        return xch + l * lay.layer + 8 * size_t(lay.log_x) + size_t(K) * (lay.hrg_r + lay.yr_r) +
               size_t(x) * lay.hid_x;
    };

    const uint32_t ep0 = __builtin_amdgcn_readfirstlane(static_cast<int>(get_u32(ctl + CTL_EPOCH)));
    bool dead = false;
    // the layer table, in LDS for the whole call
    for (uint32_t i = tid; i < n_layers * (sizeof(LayerDesc) / 16); i += ST_THREADS)
        reinterpret_cast<uint4*>(tbl_s)[i] = reinterpret_cast<const uint4*>(layers)[i];
    __syncthreads();

    if (has_role && x < K) {
        // router rows and norm weights of the current layer, in registers
        uint4 rw[RRW][CPL][4];
        uint4 gw[CPL][4];
        auto fetch_router = [&](const LayerDesc& Ld) {
#pragma unroll
            for (int i = 0; i < RRW; ++i) {
                const uint32_t row = jw + ST_WX * i;
                if (row < E) {
                    const uint16_t* p = Ld.router_w + size_t(row) * D;
#pragma unroll
                    for (int j = 0; j < CPL; ++j) {
                        const uint32_t c = min(lane + WAVE * j, nch - 1);
#pragma unroll
                        for (int q = 0; q < 4; ++q) rw[i][j][q] = load_u4(p + c * 32 + q * 8);
                    }
                }
            }
#pragma unroll
            for (int j = 0; j < CPL; ++j) {
                const uint32_t c = min(lane + WAVE * j, nch - 1);
#pragma unroll
                for (int q = 0; q < 4; ++q) gw[j][q] = load_u4(Ld.norm_w + c * 32 + q * 8);
            }
        };
        fetch_router(uniform_desc(tbl_s[0]));

        for (uint32_t l = 0; l < n_layers; ++l) {
            const LayerDesc Ld = uniform_desc(tbl_s[l]);
            const uint32_t ep = ep0 + l + 1;

            // ---- H: the layer's input hidden into LDS ------------------------
            if (l > 0) __syncthreads();   // the previous layer's combine has read hid_s
            {
                const uint32_t ng = D >> 2;
                float4 hv[HG];
                if (l == 0) {
#pragma unroll
                    for (int g = 0; g < HG; ++g) {
                        const uint32_t f = tid + ST_THREADS * g;
                        if (f < ng) hv[g] = load_f4(hidden + 4 * f);
                    }
                } else {
                    const uint64_t* src = HID(l);
                    poll_until(
                        [&] {
                            bool ok = true;
#pragma unroll
                            for (int g = 0; g < HG; ++g) {
                                const uint32_t f = tid + ST_THREADS * g;
                                if (f < ng) {
                                    const uint64_t w0 = get_word(src + 4 * f), w1 = get_word(src + 4 * f + 1);
                                    const uint64_t w2 = get_word(src + 4 * f + 2), w3 = get_word(src + 4 * f + 3);
                                    ok &= flag_is(w0, ep) && flag_is(w1, ep) && flag_is(w2, ep) && flag_is(w3, ep);
                                    hv[g] = make_float4(word_value(w0), word_value(w1), word_value(w2), word_value(w3));
                                }
                            }
                            return ok;
                        },
                        err, dead);
                }
#pragma unroll
                for (int g = 0; g < HG; ++g) {
                    const uint32_t f = tid + ST_THREADS * g;
                    if (f < ng) hid_s[swz4(f)] = hv[g];
                }
            }
            __syncthreads();
            if (l == 0 && tid == 0)
                __hip_atomic_fetch_add(ctl + CTL_ARRIVED, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);

            // ---- N: RMSNorm of the lane's chunks (common.hpp:245-256) --------
            float a[CPL][32];
            float ss = 0.f;
#pragma unroll
            for (int j = 0; j < CPL; ++j) {
                const uint32_t c0 = lane + WAVE * j;
                const uint32_t mask = c0 < nch ? ~0u : 0u;
                const uint32_t c = min(c0, nch - 1);
                // all eight LDS reads in flight before any is used
                float4 xq[8];
#pragma unroll
                for (int q = 0; q < 8; ++q) xq[q] = hid_s[swz4(c * 8 + q)];
                __builtin_amdgcn_sched_barrier(0);
#pragma unroll
                for (int q = 0; q < 8; ++q) {
                    const float4 v = keep4(xq[q], mask);
                    a[j][4 * q + 0] = v.x;
                    a[j][4 * q + 1] = v.y;
                    a[j][4 * q + 2] = v.z;
                    a[j][4 * q + 3] = v.w;
                    ss = fmaf(v.x, v.x, ss);
                    ss = fmaf(v.y, v.y, ss);
                    ss = fmaf(v.z, v.z, ss);
                    ss = fmaf(v.w, v.w, ss);
                }
            }
            ss = wave_sum(ss);
            const float inv = 1.0f / sqrtf(ss / static_cast<float>(D) + 1e-6f);
#pragma unroll
            for (int j = 0; j < CPL; ++j) {
#pragma unroll
                for (int q = 0; q < 4; ++q) {
                    const uint32_t gq[4] = {gw[j][q].x, gw[j][q].y, gw[j][q].z, gw[j][q].w};
#pragma unroll
                    for (int t = 0; t < 4; ++t) {
                        a[j][8 * q + 2 * t] = (a[j][8 * q + 2 * t] * inv) * bf16_to_f32(gq[t] & 0xFFFFu);
                        a[j][8 * q + 2 * t + 1] = (a[j][8 * q + 2 * t + 1] * inv) * bf16_to_f32(gq[t] >> 16);
                    }
                }
            }

            // ---- R: router rows jw, jw + 128, ... of this XCD ----------------
#pragma unroll
            for (int i = 0; i < RRW; ++i) {
                const uint32_t row = jw + ST_WX * i;
                if (row < E) {
                    float acc = 0.f;
#pragma unroll
                    for (int j = 0; j < CPL; ++j) {
#pragma unroll
                        for (int q = 0; q < 4; ++q) {
                            const uint32_t w4[4] = {rw[i][j][q].x, rw[i][j][q].y, rw[i][j][q].z, rw[i][j][q].w};
#pragma unroll
                            for (int t = 0; t < 4; ++t) {
                                acc = fmaf(bf16_to_f32(w4[t] & 0xFFFFu), a[j][8 * q + 2 * t], acc);
                                acc = fmaf(bf16_to_f32(w4[t] >> 16), a[j][8 * q + 2 * t + 1], acc);
                            }
                        }
                    }
                    acc = wave_sum(acc);
                    if (lane == 0) put_word_xcd(LOG(l) + row, ep, acc, local);
                }
            }

            // digit form of the normed chunks (overlaps the logit exchange)
            Q4Act qa[CPL];
#pragma unroll
            for (int j = 0; j < CPL; ++j) {
                q4_act_from_floats(a[j], qa[j]);
                // materialise the digits here, before the poll loop below, so
                // the conversion overlaps the wait instead of following it
#pragma unroll
                for (int dd = 0; dd < Q4_DIGITS; ++dd)
                    asm volatile("" ::"v"(qa[j].dig[dd][0]), "v"(qa[j].dig[dd][1]), "v"(qa[j].dig[dd][2]),
                                 "v"(qa[j].dig[dd][3]));
                asm volatile("" ::"v"(qa[j].xsum_half), "v"(qa[j].kscale));
            }

            // ---- T: the XCD's E logits, softmax + top-k ----------------------
            float v[VPL];
            {
                const uint64_t* src = LOG(l);
                poll_until(
                    [&] {
                        bool ok = true;
#pragma unroll
                        for (int j = 0; j < VPL; ++j) {
                            const uint32_t pos = lane + WAVE * j;
                            const uint64_t w = get_word(src + min(pos, E - 1));
                            v[j] = word_value(w);
                            ok &= pos >= E || flag_is(w, ep);
                        }
                        return ok;
                    },
                    err, dead);
            }
            uint32_t my_id;
            float my_w;
            topk_latency<VPL>(v, E, K, d.norm_topk, my_id, my_w, topk_s[wv]);
            if (x == 0 && jw == 0 && static_cast<uint32_t>(lane) < K) {
                if (ids_out) ids_out[size_t(l) * K + lane] = my_id;
                if (w_out) w_out[size_t(l) * K + lane] = my_w;
            }

            // ---- U + D: the experts of this XCD's ranks ----------------------
            bool prefetched = l + 1 >= n_layers;
            const uint32_t rpw = (I + ST_WX - 1) / ST_WX;     // gate/up rows per wave
            const uint32_t u0 = min(I, jw * rpw), u1 = min(I, u0 + rpw);
            const uint32_t rpd = (D + ST_WX - 1) / ST_WX;     // down rows per wave
            const uint32_t d0 = min(D, jw * rpd), d1 = min(D, d0 + rpd);
            const uint32_t nbat = (rpd + RPB - 1) / RPB;
            const uint32_t cI = lane & (CW - 1), seg = lane >> SEG;
            const bool cact = cI < nchI;
            const uint32_t cIc = min(cI, nchI - 1);
            for (uint32_t r = x; r < K; r += 8) {
                // (clamped: ids from a timed-out exchange must still index inside the pool)
                const uint32_t e = min(readlane_u32(my_id, static_cast<int>(r)), E - 1);
                const uint8_t* blob = Ld.experts + size_t(e) * Ld.stride;
                const uint8_t* pg = blob + Ld.off[0];
                const uint16_t* sg = reinterpret_cast<const uint16_t*>(blob + Ld.off[1]);
                const uint8_t* pu = blob + Ld.off[2];
                const uint16_t* su = reinterpret_cast<const uint16_t*>(blob + Ld.off[3]);
                const uint8_t* pd = blob + Ld.off[4];
                const uint16_t* sd = reinterpret_cast<const uint16_t*>(blob + Ld.off[5]);

                uint4 va[UG][CPL], vb[UG][CPL];
                uint16_t sva[UG][CPL], svb[UG][CPL];
                auto load_gu = [&](uint32_t g0) {
#pragma unroll
                    for (int i = 0; i < UG; ++i) {
                        const size_t row = min(g0 + i, u1 - 1);
#pragma unroll
                        for (int j = 0; j < CPL; ++j) {
                            const uint32_t c = min(lane + WAVE * j, nch - 1);
                            va[i][j] = load_stream_u4(pg + row * (D >> 1) + c * 16);
                            vb[i][j] = load_stream_u4(pu + row * (D >> 1) + c * 16);
                            sva[i][j] = load_stream_u16(sg + row * (D / 64) + c / 2);
                            svb[i][j] = load_stream_u16(su + row * (D / 64) + c / 2);
                        }
                    }
                };
                uint4 dw[DG];
                uint16_t dsc[DG];
                auto load_down = [&](uint32_t g0) {
#pragma unroll
                    for (int t = 0; t < DG; ++t) {
                        const size_t row = min(d0 + (g0 + t) * RPB + seg, d1 - 1);
                        dw[t] = load_stream_u4(pd + row * (I >> 1) + cIc * 16);
                        dsc[t] = load_stream_u16(sd + row * (I / 64) + cIc / 2);
                    }
                };
                // every weight load of the first groups in flight, then the
                // next layer's router rows (issued last, so waiting on the
                // weights never waits on them)
                if (u0 < u1) load_gu(u0);
                __builtin_amdgcn_sched_barrier(0);
                if (d0 < d1) load_down(0);
                __builtin_amdgcn_sched_barrier(0);
                if (!prefetched) {
                    fetch_router(uniform_desc(tbl_s[l + 1]));
                    prefetched = true;
                }
                __builtin_amdgcn_sched_barrier(0);

                // U: gate/up rows [u0, u1) in groups of UG
                for (uint32_t g0 = u0; g0 < u1; g0 += UG) {
                    if (g0 != u0) load_gu(g0);
                    float part[16];
#pragma unroll
                    for (int i = 0; i < UG; ++i) {
                        float ga = 0.f, ua = 0.f;
#pragma unroll
                        for (int j = 0; j < CPL; ++j) {
                            ga = fmaf(f16_bits_to_f32(sva[i][j]), q4_chunk_dot8(va[i][j], qa[j]), ga);
                            ua = fmaf(f16_bits_to_f32(svb[i][j]), q4_chunk_dot8(vb[i][j], qa[j]), ua);
                        }
                        part[2 * i] = ga;
                        part[2 * i + 1] = ua;
                    }
#pragma unroll
                    for (int i = 2 * UG; i < 16; ++i) part[i] = 0.f;
                    // lane l holds the total of value l >> 2
                    const float tot = wave_sum_rows<16>(part);
                    const float gv = __shfl(tot, (8 * lane) & 63);
                    const float uv = __shfl(tot, (8 * lane + 4) & 63);
                    // silu(z) = z * (1 / (1 + exp(-z)))  (kernels.metal:61-63, :334-336)
                    if (lane < UG && g0 + lane < u1)
                        put_word_xcd(HRG(l, r) + g0 + lane, ep, (gv * (1.0f / (1.0f + expf(-gv)))) * uv, local);
                }

                // D: the rank's h [I] into LDS (all 4 waves), then down rows [d0, d1)
                {
                    const uint64_t* src = HRG(l, r);
                    const uint32_t ng = I >> 2;
                    float4 hv[HGI];
                    poll_until(
                        [&] {
                            bool ok = true;
#pragma unroll
                            for (int g = 0; g < HGI; ++g) {
                                const uint32_t f = tid + ST_THREADS * g;
                                if (f < ng) {
                                    const uint64_t w0 = get_word(src + 4 * f), w1 = get_word(src + 4 * f + 1);
                                    const uint64_t w2 = get_word(src + 4 * f + 2), w3 = get_word(src + 4 * f + 3);
                                    ok &= flag_is(w0, ep) && flag_is(w1, ep) && flag_is(w2, ep) && flag_is(w3, ep);
                                    hv[g] = make_float4(word_value(w0), word_value(w1), word_value(w2), word_value(w3));
                                }
                            }
                            return ok;
                        },
                        err, dead);
#pragma unroll
                    for (int g = 0; g < HGI; ++g) {
                        const uint32_t f = tid + ST_THREADS * g;
                        if (f < ng) h_s[swz4(f)] = hv[g];
                    }
                }
                __syncthreads();
                Q4Act qh;
                {
                    float hc[32];
                    const uint32_t mask = cact ? ~0u : 0u;
                    float4 hq[8];
#pragma unroll
                    for (int q = 0; q < 8; ++q) hq[q] = h_s[swz4(cIc * 8 + q)];
                    __builtin_amdgcn_sched_barrier(0);
#pragma unroll
                    for (int q = 0; q < 8; ++q) {
                        const float4 t = keep4(hq[q], mask);
                        hc[4 * q + 0] = t.x;
                        hc[4 * q + 1] = t.y;
                        hc[4 * q + 2] = t.z;
                        hc[4 * q + 3] = t.w;
                    }
                    q4_act_from_floats(hc, qh);
                }
                if (d0 < d1) {
                    for (uint32_t g0 = 0; g0 < nbat; g0 += DG) {
                        if (g0 != 0) load_down(g0);
                        float part[DG];
#pragma unroll
                        for (int t = 0; t < DG; ++t)
                            part[t] = cact ? f16_bits_to_f32(dsc[t]) * q4_chunk_dot8(dw[t], qh) : 0.f;
                        // lane l holds the sum of batch (l >> (SEG - LDG)) & (DG - 1) of row slot l >> SEG
                        const float tot = seg_sum_rows<DG, SEG>(part);
                        const uint32_t bi = g0 + ((static_cast<uint32_t>(lane) >> (SEG - LDG)) & (DG - 1));
                        const uint32_t row = d0 + bi * RPB + seg;
                        if ((lane & ((1 << (SEG - LDG)) - 1)) == 0 && bi < nbat && row < d1)
                            put_word(YR(l, r) + row, ep, tot);
                    }
                }
                __syncthreads();   // h_s is refilled by the next rank
            }
            if (!prefetched) fetch_router(uniform_desc(tbl_s[l + 1]));

            // ---- C: hidden + sum_r w_r y_r for rows [jw rpc, ...) -----------
            // The y words come from every XCD: one wave per block polls the
            // block's rows of all ranks (a quarter of the cross-XCD requests
            // of every wave polling its own) and hands them over through LDS.
            {
                const uint32_t rpc = (D + ST_WX - 1) / ST_WX;          // rows per wave (<= 16: D <= 2048)
                const uint32_t brow0 = (jw - wv) * rpc;                 // the block's first row
                if (wv == 0) {
                    const uint32_t br = brow0 + lane;
                    const bool mine = static_cast<uint32_t>(lane) < ST_WPB * rpc && br < D;
                    const uint32_t brc = min(br, D - 1);
                    float y[SMOE_TOPK_MAX_K];
                    poll_until(
                        [&] {
                            bool ok = true;
                            if (mine) {
#pragma unroll
                                for (int r = 0; r < SMOE_TOPK_MAX_K; ++r) {
                                    if (static_cast<uint32_t>(r) < K) {
                                        const uint64_t w = get_word(YR(l, r) + brc);
                                        y[r] = word_value(w);
                                        ok &= flag_is(w, ep);
                                    }
                                }
                            }
                            return ok;
                        },
                        err, dead);
                    if (mine) {
#pragma unroll
                        for (int r = 0; r < SMOE_TOPK_MAX_K; ++r)
                            if (static_cast<uint32_t>(r) < K) y_s[r][lane] = y[r];
                    }
                }
                __syncthreads();
                const uint32_t row = jw * rpc + lane;
                const bool mine = static_cast<uint32_t>(lane) < rpc && row < D;
                const uint32_t rowc = min(row, D - 1);
                const uint32_t yi = min(wv * rpc + lane, ST_WPB * 16u - 1);
                // routed_out += w_r * y_r in rank order (axpy_f32, common.hpp:346-349),
                // then hidden += routed_out (decode.cpp:506-509)
                float routed = 0.f;
#pragma unroll
                for (int r = 0; r < SMOE_TOPK_MAX_K; ++r)
                    if (static_cast<uint32_t>(r) < K) routed = routed + readlane_f32(my_w, r) * y_s[r][yi];
                const float hnew = reinterpret_cast<const float*>(hid_s)[swz4(rowc >> 2) * 4 + (rowc & 3)] + routed;
                if (l + 1 < n_layers) {
                    if (mine) put_word_xcd(HID(l + 1) + row, ep + 1, hnew, local);
                } else if (x == 0) {
                    // the caller's buffer is overwritten only once every block has read it
                    poll_until([&] { return get_u32(ctl + CTL_ARRIVED) >= gridDim.x; }, err, dead);
                    if (mine) hidden[row] = hnew;
                }
            }
        }
    } else if (tid == 0) {
        // XCDs without a rank (K < 8) and surplus blocks take no part; they
        // never read hidden
        __hip_atomic_fetch_add(ctl + CTL_ARRIVED, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    }

    // the last block to finish re-arms the control words for the next call
    __syncthreads();
    if (tid == 0) {
        const uint32_t old = __hip_atomic_fetch_add(ctl + CTL_DONE, 1u, __ATOMIC_ACQ_REL, __HIP_MEMORY_SCOPE_AGENT);
        if (old == gridDim.x - 1) {
            __hip_atomic_store(ctl + CTL_DONE, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
            __hip_atomic_store(ctl + CTL_ARRIVED, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
            for (uint32_t i = 0; i < 8; ++i)
                __hip_atomic_store(ctl + CTL_TICKET + 32 * i, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
            __hip_atomic_store(ctl + CTL_EPOCH, ep0 + n_layers, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        }
    }
}

// ---------------------------------------------------------------------------
// launcher
// ---------------------------------------------------------------------------
// d_model up to 2048 (one 32-column chunk per lane, D / 128 <= 16 combine
// rows per wave); larger shapes run through the per-layer kernels.
bool stack_supported(const MoeDims& d)
{
    return d.group == 64 && d.D % 64 == 0 && d.D <= 2048 && d.I % 64 == 0 && d.I <= 2048 && d.E >= 1 &&
           d.E <= 512 && d.K >= 1 && d.K <= static_cast<uint32_t>(SMOE_TOPK_MAX_K) && d.K <= d.E;
}

template <int VPL, int RRW>
static void stack_cw(const MoeDims& d, const LayerDesc* layers, uint32_t n_layers, float* hidden, uint64_t* xch,
                     uint32_t* ctl, uint32_t* ids, float* w, uint32_t* err, hipStream_t s)
{
    const uint32_t nchI = d.I / 32;
    const dim3 grid(ST_BLOCKS), block(ST_THREADS);
    if (nchI <= 8)
        launch_kernel(k_decode_stack<VPL, RRW, 8>, grid, block, s, d, layers, n_layers, hidden, xch, ctl, ids, w,
                      err);
    else if (nchI <= 32)
        launch_kernel(k_decode_stack<VPL, RRW, 32>, grid, block, s, d, layers, n_layers, hidden, xch, ctl, ids,
                      w, err);
    else
        launch_kernel(k_decode_stack<VPL, RRW, 64>, grid, block, s, d, layers, n_layers, hidden, xch, ctl, ids,
                      w, err);
}

hipError_t launch_decode_stack(const MoeDims& d, const LayerDesc* layers, uint32_t n_layers, float* hidden,
                               uint64_t* xch, uint32_t* ctl, uint32_t* ids, float* w, uint32_t* err, hipStream_t s)
{
    if (!stack_supported(d) || n_layers == 0 || n_layers > ST_MAX_LAYERS) return hipErrorInvalidValue;
    if (d.E <= 128) stack_cw<2, 1>(d, layers, n_layers, hidden, xch, ctl, ids, w, err, s);
    else stack_cw<8, 4>(d, layers, n_layers, hidden, xch, ctl, ids, w, err, s);
    return hipGetLastError();
}

}  // namespace smoe
