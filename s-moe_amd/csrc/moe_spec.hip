// moe_spec.hip -- one batch-1 decode step through every MoE layer of a stack
// (the decode.cpp:121 layer loop over decode.cpp:236-509) in ONE persistent
// launch, with each layer's expert weights fetched into LDS ahead of time.
//
// Shape: d_model 2048, top-k 8, 8..128 experts, d_ff a multiple of 192 up to
// 768 (Qwen3-30B-A3B: 2048 / 128 / 8 / 768).
//
// Placement.  256 blocks of 12 waves, one block per CU.  Each block takes the
// XCD it runs on (XCC_ID) and a ticket among that XCD's blocks: XCD x, CU
// c = 0..31.  XCD x computes the expert of "slot" x of every layer; CU c of
// it owns gate/up rows [c I/32, (c+1) I/32) and down rows [64 c, 64 c + 64)
// of that expert, and combines output rows [64 c, 64 c + 64).
//
// Waves.  Waves 0-7 (compute) run the layer chain; waves 8-11 (prefetch) copy
// what the compute waves will read into LDS with global_load_lds_dwordx4 (no
// registers in flight): the CU's four router rows of the layers ahead, the
// norm weights, and the CU's slice of its slot expert (gate/up rows, down
// rows, their scales: 78 KB at the 30B shape).  The copies are counted on the
// prefetch waves, so no compute wave's exchange poll waits on them.
//
// Prediction.  Layer l + 1's router applied to layer l's input (with its own
// norm weights) ranks the experts about as layer l + 1's own input will: the
// top 8 of those logits, P_{l+1}, tells the prefetch waves which expert to
// fetch for slot x of layer l + 1 (the x-th predicted) once layer l's slice
// has been read.  When layer l + 1's exact top-k S is known, slot x keeps
// P[x] if P[x] is in S (a hit: its slice is already in LDS); the ranks of S
// not in P go, in rank order, to the slots whose P[x] missed, and those CUs
// fetch the actual expert's slice then.  The combine sums the 8 slots'
// outputs in rank order, so results do not depend on the prediction, only the
// time does.  Layer 0 fetches after its top-k.
//
// Per layer, compute waves of CU c on XCD x:
//   H  all: the layer's input hidden [D] into LDS (layer 0: the caller's
//      buffer; later: the XCD's copy published in C), an eighth per wave;
//   N  all: RMSNorm (common.hpp:245-256); waves 0-3 router row 4c + w of
//      layer l, waves 4-7 the same rows of layer l + 1 on the input normed
//      with layer l + 1's weights (common.hpp:293-306), published into XCD
//      x's logit copy;
//   T  wave 0: all real logits, softmax + top-k + renormalisation
//      (scout.cpp:77-123, decode.cpp:296-302), the slot assignment; wave 1:
//      all predicted logits and their top 8;
//   U  waves 2-7, beside T: the CU's gate/up rows (kernels.metal:240-337) of
//      slot x's predicted expert, from LDS; once T confirms it (or after the
//      actual expert's slice arrives, on a miss), h published into XCD x's h
//      copy;
//   D  all: h into LDS; 8 down rows each (kernels.metal:340-365), published
//      to every XCD;
//   C  all: hidden + sum_r w_r y_r in rank order for the wave's 8 rows
//      (decode.cpp:482-509), published into XCD x's copy of the next input.
// Exchange words are 64-bit (flag << 32 | fp32) whose flag is the layer's
// epoch; epochs grow by n_layers per call (the last block to finish advances
// the control word), so no word is ever re-armed.  Every wait is bounded: a
// time-out flags err bit 0 and every wave of the block then stops waiting.
//
// LDS vectors that every lane reads 32 consecutive values of (hidden, norm
// weights, router rows, h) are stored "quad-major": the 16-byte quad q of
// chunk c sits at q * (chunks) + c, so the 64 lanes reading quad q of their
// chunks touch consecutive addresses (a lane-strided layout reads 3-5x
// slower).
#include "device_common.hpp"
#include "kernels.hpp"
#include "topk.hpp"

namespace smoe {

namespace {

constexpr int SP_D = 2048;
constexpr int SP_MAX_I = 768;
constexpr int SP_CW = 8;                       // compute waves per block
constexpr int SP_PW = 4;                       // prefetch waves per block
constexpr int SP_UW = 6;                       // gate/up waves (compute waves 2..7)
constexpr int SP_THREADS = (SP_CW + SP_PW) * WAVE;
constexpr int SP_BLOCKS = 256;
constexpr int SP_CUS = SP_BLOCKS / 8;          // blocks per XCD
constexpr uint32_t SP_GLOBAL_SPIN = 1u << 20;  // exchange polls (each a memory round trip)
constexpr uint32_t SP_LDS_SPIN = 1u << 22;     // LDS waits (each with a short sleep)

constexpr uint32_t NCH = SP_D / 32;                   // 32-column chunks of d_model (one per lane)
constexpr uint32_t GU_ROWS_MAX = SP_MAX_I / SP_CUS;   // gate (and up) rows per CU
constexpr uint32_t GU_ROW = SP_D / 2;                 // packed bytes of a gate/up row
constexpr uint32_t GU_ROW_SC = SP_D / 32;             // scale bytes of a gate/up row
constexpr uint32_t DN_ROWS = SP_D / SP_CUS;           // down rows per CU
constexpr uint32_t DN_ROWS_W = DN_ROWS / SP_CW;       // down rows per compute wave
constexpr uint32_t GU_BYTES = 2 * GU_ROWS_MAX * (GU_ROW + GU_ROW_SC);
constexpr uint32_t DN_BYTES = DN_ROWS * (SP_MAX_I / 2 + SP_MAX_I / 32);
constexpr uint32_t H_CH = 32;                         // chunk stride of the quad-major h

// signal words (LDS)
enum : uint32_t {
    SG_ROUTE = 0,      // [8] compute wave w: layer l's router / norm buffers read (l + 1)
    SG_GUFREE = 8,     // [8] compute wave w: layer l's gate/up slice read (l + 1)
    SG_DNFREE = 16,    // [8] compute wave w: layer l's down slice read (l + 1)
    SG_RTAG = 24,      // [4] prefetch wave: router layers 0 .. RTAG-1 loaded
    SG_GUTAG = 28,     // [4] prefetch wave: gate/up slice held, ((l + 1) << 12) | expert
    SG_DNTAG = 32,     // [2][4] by buffer (layer parity), prefetch wave: down slice held, same form
    SG_TOPK = 40,      // wave 0: layer l's routing and slots published (l + 1)
    SG_PREDOK = 41,    // wave 1: layer l + 1's prediction published (l + 1)
    SG_SLOT = 42,      // [2] by layer parity: slot expert | hit << 31
    SG_CBAR = 44,      // compute-wave barrier counter
    SG_DEAD = 45,      // a wave of the block timed out
    SG_PRED = 48,      // [2][8] by layer parity: predicted experts of the layer
    SG_SOR = 64,       // [2][8] by layer parity: slot that computes rank r
    SG_W = 80,         // [2][8] by layer parity: routing weight of rank r (fp32 bits)
    SG_WORDS = 96,
};

struct SpecLds {
    uint8_t gu[GU_BYTES];                  // gate p | up p | gate s | up s of the CU's rows
    uint8_t dn[2][DN_BYTES];               // down p | down s of the CU's rows, by layer parity
    uint4 rt[2][4][4 * NCH];               // router rows 4 c .. 4 c + 3 (bf16, quad-major), by layer parity
    uint4 nw[2][4 * NCH];                  // norm weights (bf16, quad-major), by layer parity
    float4 hid[8 * NCH];                   // the layer's input hidden (quad-major)
    float4 h[8 * H_CH];                    // h of slot x's expert (quad-major, chunk stride 32)
    uint2 topk[TOPK_SLOTS];                // wave 0's top-k scratch
    uint32_t sig[SG_WORDS];
};
static_assert(sizeof(SpecLds) <= 160 * 1024, "LDS of one CU");

// exchange words of one layer: logits [8 XCDs][256] (real 0..127, predicted
// 128..255), h [8 XCDs][I'], y [8 slots][D], next hidden [8 XCDs][D]
struct SpecLayout {
    uint32_t hx;
    size_t layer;
    __host__ __device__ explicit SpecLayout(const MoeDims& d)
        : hx((d.I + 63u) & ~63u), layer(8 * 256 + 8 * size_t(hx) + 8 * size_t(SP_D) + 8 * size_t(SP_D))
    {
    }
};

__device__ __forceinline__ uint64_t sword(uint32_t ep, float v)
{
    return (static_cast<uint64_t>(ep) << 32) | __float_as_uint(v);
}
__device__ __forceinline__ void put_wave(uint64_t* p, uint64_t v)
{
    __hip_atomic_store(p, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WAVEFRONT);
}
__device__ __forceinline__ void put_agent(uint64_t* p, uint64_t v)
{
    __hip_atomic_store(p, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
// a word for the writer's own XCD (plain store, stays in its L2) or, with
// placement by block id, for everyone
__device__ __forceinline__ void put_xcd(uint64_t* p, uint64_t v, bool local)
{
    if (local) put_wave(p, v);
    else put_agent(p, v);
}
__device__ __forceinline__ uint64_t get_agent(const uint64_t* p)
{
    return __hip_atomic_load(const_cast<uint64_t*>(p), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ uint32_t get_agent32(const uint32_t* p)
{
    return __hip_atomic_load(const_cast<uint32_t*>(p), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ bool has_tag(uint64_t w, uint32_t ep) { return static_cast<uint32_t>(w >> 32) == ep; }
__device__ __forceinline__ float value_of(uint64_t w) { return __uint_as_float(static_cast<uint32_t>(w)); }

// LDS signal words
__device__ __forceinline__ uint32_t sig_get(const uint32_t* p)
{
    return __hip_atomic_load(const_cast<uint32_t*>(p), __ATOMIC_ACQUIRE, __HIP_MEMORY_SCOPE_WORKGROUP);
}
__device__ __forceinline__ void sig_set(uint32_t* p, uint32_t v)
{
    __hip_atomic_store(p, v, __ATOMIC_RELEASE, __HIP_MEMORY_SCOPE_WORKGROUP);
}
// all of sig[base + i], i in [i0, i1), at least v
__device__ __forceinline__ bool sig_all_ge(const uint32_t* sig, uint32_t base, uint32_t i0, uint32_t i1, uint32_t v)
{
    bool ok = true;
    for (uint32_t i = i0; i < i1; ++i) ok &= sig_get(sig + base + i) >= v;
    return ok;
}
__device__ __forceinline__ bool sig_all_eq(const uint32_t* sig, uint32_t base, uint32_t n, uint32_t v)
{
    bool ok = true;
    for (uint32_t i = 0; i < n; ++i) ok &= sig_get(sig + base + i) == v;
    return ok;
}

#define SP_LDS(p) ((__attribute__((address_space(3))) void*)(p))

// wait until pred() holds (wave-uniform), bounded; a time-out or a dead block
// marks the block dead and returns false
template <typename F>
__device__ __forceinline__ bool lds_wait(uint32_t* sig, F&& pred, uint32_t* err)
{
    for (uint32_t spins = 0;; ++spins) {
        if (pred()) return true;
        if (sig_get(sig + SG_DEAD)) return false;
        if (spins >= SP_LDS_SPIN) {
            if ((threadIdx.x & 63) == 0) atomicOr(err, 1u);
            sig_set(sig + SG_DEAD, 1u);
            return false;
        }
        __builtin_amdgcn_s_sleep(1);
    }
}

// re-run `round` (issues its loads, returns whether this lane's words are all
// present) until it holds on every lane; bounded, and gives up as soon as the
// block is dead or any wave anywhere flagged an error
template <typename F>
__device__ __forceinline__ void poll_words(F&& round, uint32_t* sig, uint32_t* err)
{
    for (uint32_t spins = 0;; ++spins) {
        const bool ok = round();
        if (__ballot(!ok) == 0) return;
        if ((spins & 63u) == 63u) {
            if (sig_get(sig + SG_DEAD) ||
                __builtin_amdgcn_readfirstlane(static_cast<int>(get_agent32(err))) != 0) {
                sig_set(sig + SG_DEAD, 1u);
                return;
            }
            if (spins >= SP_GLOBAL_SPIN) {
                if ((threadIdx.x & 63) == 0) atomicOr(err, 1u);
                sig_set(sig + SG_DEAD, 1u);
                return;
            }
        }
    }
}

// barrier of the block's compute waves (LDS counter; the prefetch waves run
// their own schedule)
__device__ __forceinline__ void compute_barrier(uint32_t* sig, uint32_t& n, uint32_t* err)
{
    n += SP_CW;
    if ((threadIdx.x & 63) == 0)
        __hip_atomic_fetch_add(sig + SG_CBAR, 1u, __ATOMIC_RELEASE, __HIP_MEMORY_SCOPE_WORKGROUP);
    const uint32_t target = n;
    lds_wait(sig, [&] { return sig_get(sig + SG_CBAR) >= target; }, err);
}

// copy `bytes` (a multiple of 16; src and dst 16-byte aligned) from global src
// to LDS dst: 1 KiB per instruction (lane i moves bytes 16 i .. 16 i + 15 of
// it; lanes past the end stay idle), instructions dealt round-robin over the
// prefetch waves
__device__ __forceinline__ void lds_copy(uint8_t* dst, const uint8_t* src, uint32_t bytes, uint32_t pw)
{
    const uint32_t lane = threadIdx.x & 63;
    const uint32_t n = (bytes + 1023u) >> 10;
    for (uint32_t k = pw; k < n; k += SP_PW) {
        const uint32_t off = k << 10;
        if (off + lane * 16 < bytes)
            __builtin_amdgcn_global_load_lds(src + off + lane * 16, SP_LDS(dst + off), 16, 0, 0);
    }
}
// copy `rows` bf16 rows of d_model values into the quad-major layout: quad q
// (8 values) of chunk c (32 values) of row i at uint4 index i * 4 NCH +
// q * NCH + c; instruction (i, q) moves quad q of every chunk of row i
__device__ __forceinline__ void lds_copy_rows_qmajor(uint4* dst, const uint16_t* src, uint32_t rows, uint32_t pw)
{
    const uint32_t lane = threadIdx.x & 63;
    for (uint32_t k = pw; k < rows * 4; k += SP_PW) {
        const uint32_t i = k >> 2, q = k & 3;
        __builtin_amdgcn_global_load_lds(src + size_t(i) * SP_D + lane * 32 + q * 8, SP_LDS(dst + i * 4 * NCH + q * NCH),
                                         16, 0, 0);
    }
}

__device__ __forceinline__ void vm_wait_all()
{
    asm volatile("" ::: "memory");
    __builtin_amdgcn_s_waitcnt(0x0F70);   // vmcnt(0)
    asm volatile("" ::: "memory");
}

__device__ __forceinline__ uint32_t slice_tag(uint32_t l, uint32_t e) { return ((l + 1) << 12) | e; }

__host__ __device__ constexpr uint32_t ceil_div(uint32_t a, uint32_t b) { return (a + b - 1) / b; }

// wait until at most n (< 16) vector memory operations of this wave are in flight
__device__ __forceinline__ void vm_wait_n(uint32_t n)
{
    asm volatile("" ::: "memory");
    switch (min(n, 15u)) {
    case 0: __builtin_amdgcn_s_waitcnt(0x0F70); break;
    case 1: __builtin_amdgcn_s_waitcnt(0x0F71); break;
    case 2: __builtin_amdgcn_s_waitcnt(0x0F72); break;
    case 3: __builtin_amdgcn_s_waitcnt(0x0F73); break;
    case 4: __builtin_amdgcn_s_waitcnt(0x0F74); break;
    case 5: __builtin_amdgcn_s_waitcnt(0x0F75); break;
    case 6: __builtin_amdgcn_s_waitcnt(0x0F76); break;
    case 7: __builtin_amdgcn_s_waitcnt(0x0F77); break;
    case 8: __builtin_amdgcn_s_waitcnt(0x0F78); break;
    case 9: __builtin_amdgcn_s_waitcnt(0x0F79); break;
    case 10: __builtin_amdgcn_s_waitcnt(0x0F7A); break;
    case 11: __builtin_amdgcn_s_waitcnt(0x0F7B); break;
    case 12: __builtin_amdgcn_s_waitcnt(0x0F7C); break;
    case 13: __builtin_amdgcn_s_waitcnt(0x0F7D); break;
    case 14: __builtin_amdgcn_s_waitcnt(0x0F7E); break;
    default: __builtin_amdgcn_s_waitcnt(0x0F7F); break;
    }
    asm volatile("" ::: "memory");
}

__device__ __forceinline__ const uint8_t* uniform_bytes(const uint8_t* p)
{
    const uint64_t v = reinterpret_cast<uint64_t>(p);
    const uint32_t lo = __builtin_amdgcn_readfirstlane(static_cast<uint32_t>(v));
    const uint32_t hi = __builtin_amdgcn_readfirstlane(static_cast<uint32_t>(v >> 32));
    return reinterpret_cast<const uint8_t*>((static_cast<uint64_t>(hi) << 32) | lo);
}

__device__ __forceinline__ uint64_t tstamp() { return __builtin_amdgcn_s_memrealtime(); }

}  // namespace

constexpr uint32_t CTL_EPOCH = 0, CTL_MODE = 1, CTL_DONE = 32, CTL_ARRIVED = 64, CTL_TICKET = 96;

size_t spec_xch_words(const MoeDims& d, uint32_t n_layers) { return SpecLayout(d).layer * n_layers; }

// RB: gate/up rows per gate/up wave (I / 192)
template <int RB>
__global__ __launch_bounds__(SP_THREADS, 1)
void k_decode_spec(MoeDims d, const LayerDesc* __restrict__ layers, uint32_t n_layers, float* __restrict__ hidden,
                   uint64_t* __restrict__ xch, uint32_t* __restrict__ ctl, uint32_t* __restrict__ ids_out,
                   float* __restrict__ w_out, uint32_t* __restrict__ err, uint64_t* __restrict__ trace)
{
    constexpr int NR = 2 * RB <= 8 ? 8 : 16;         // reduced values per gate/up pass (gate, up per row; padded)
    constexpr uint32_t RBC = RB * SP_UW;             // gate/up rows per CU
    static_assert(RBC <= GU_ROWS_MAX, "gate/up rows per CU");
    __shared__ SpecLds S;
    __shared__ uint32_t role_s;

    const int tid = threadIdx.x, lane = tid & 63;
    const int wv = __builtin_amdgcn_readfirstlane(tid >> 6);
    const uint32_t b = blockIdx.x;
    const uint32_t D = SP_D, E = d.E, I = d.I;

    // ---- placement ---------------------------------------------------------
    const bool by_xcd = __builtin_amdgcn_readfirstlane(static_cast<int>(get_agent32(ctl + CTL_MODE))) == 0;
    if (tid < SG_WORDS) S.sig[tid] = 0u;
    if (tid == 0) {
        uint32_t xcc;
        asm volatile("s_getreg_b32 %0, hwreg(HW_REG_XCC_ID, 0, 4)" : "=s"(xcc));
        xcc &= 7u;
        uint32_t role = b;   // (b & 7) = XCD, b >> 3 = CU
        if (by_xcd) {
            const uint32_t t = __hip_atomic_fetch_add(ctl + CTL_TICKET + 32 * xcc, 1u, __ATOMIC_RELAXED,
                                                      __HIP_MEMORY_SCOPE_AGENT);
            if (t < SP_CUS) {
                role = (t << 3) | xcc;
            } else {
                role = 0xFFFFFFFFu;
                atomicOr(err, 4u);
                __hip_atomic_store(ctl + CTL_MODE, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
            }
        }
        role_s = role;
    }
    __syncthreads();
    const uint32_t role = __builtin_amdgcn_readfirstlane(static_cast<int>(role_s));
    const uint32_t ep0 = __builtin_amdgcn_readfirstlane(static_cast<int>(get_agent32(ctl + CTL_EPOCH)));
    const bool local = by_xcd;
    const uint32_t x = role & 7u, c = (role >> 3) & (SP_CUS - 1);
    const SpecLayout lay(d);
    auto LG = [&](uint32_t l, uint32_t xx) { return xch + l * lay.layer + size_t(xx) * 256; };
    auto HX = [&](uint32_t l, uint32_t xx) { return xch + l * lay.layer + 8 * 256 + size_t(xx) * lay.hx; };
    auto YS = [&](uint32_t l, uint32_t s) {
        return xch + l * lay.layer + 8 * 256 + 8 * size_t(lay.hx) + size_t(s) * D;
    };
    auto HN = [&](uint32_t l, uint32_t xx) {
        return xch + l * lay.layer + 8 * 256 + 8 * size_t(lay.hx) + 8 * size_t(D) + size_t(xx) * D;
    };
    uint32_t* sig = S.sig;
    // the CU's slice inside an expert blob
    const uint32_t gu_p = RBC * GU_ROW, gu_s = RBC * GU_ROW_SC;
    const uint32_t dn_row = I / 2, dn_row_sc = I / 32;
    const uint32_t dn_p = DN_ROWS * dn_row, dn_s = DN_ROWS * dn_row_sc;

    if (role != 0xFFFFFFFFu) {
        if (wv >= SP_CW) {
            // ================= prefetch waves =================
            const uint32_t pw = static_cast<uint32_t>(wv - SP_CW);
            auto load_router = [&](uint32_t l) {   // router rows 4c..4c+3 and norm weights of layer l
                const LayerDesc& Ld = layers[l];
                const uint32_t rows = min(4u, E > 4 * c ? E - 4 * c : 0u);
                const uint16_t* rsrc = reinterpret_cast<const uint16_t*>(
                    uniform_bytes(reinterpret_cast<const uint8_t*>(Ld.router_w + size_t(4 * c) * D)));
                if (rows) lds_copy_rows_qmajor(&S.rt[l & 1][0][0], rsrc, rows, pw);
                const uint16_t* nsrc =
                    reinterpret_cast<const uint16_t*>(uniform_bytes(reinterpret_cast<const uint8_t*>(Ld.norm_w)));
                lds_copy_rows_qmajor(&S.nw[l & 1][0], nsrc, 1, pw);
            };
            auto load_slice = [&](uint32_t l, uint32_t e, bool gu, bool dn) {
                const LayerDesc& Ld = layers[l];
                const uint8_t* blob = uniform_bytes(Ld.experts + size_t(e) * Ld.stride);
                if (gu) {
                    lds_copy(S.gu, blob + Ld.off[0] + size_t(c) * gu_p, gu_p, pw);
                    lds_copy(S.gu + gu_p, blob + Ld.off[2] + size_t(c) * gu_p, gu_p, pw);
                    lds_copy(S.gu + 2 * gu_p, blob + Ld.off[1] + size_t(c) * gu_s, gu_s, pw);
                    lds_copy(S.gu + 2 * gu_p + gu_s, blob + Ld.off[3] + size_t(c) * gu_s, gu_s, pw);
                }
                if (dn) {
                    lds_copy(S.dn[l & 1], blob + Ld.off[4] + size_t(c) * dn_p, dn_p, pw);
                    lds_copy(S.dn[l & 1] + dn_p, blob + Ld.off[5] + size_t(c) * dn_s, dn_s, pw);
                }
            };
            // down copies issued by this wave for one slice (vm_wait below):
            // instructions pw, pw + 4, ... of the packed part and of the scales
            const uint32_t n_dn = (ceil_div(dn_p, 1024u) + SP_PW - 1 - pw) / SP_PW +
                                  (ceil_div(dn_s, 1024u) + SP_PW - 1 - pw) / SP_PW;
            load_router(0);
            if (n_layers > 1) load_router(1);
            vm_wait_all();
            if (lane == 0) sig_set(sig + SG_RTAG + pw, min(2u, n_layers));
            bool ok = true;
            for (uint32_t l = 0; l < n_layers && ok; ++l) {
                const uint32_t par = l & 1;
                // layer l's slot: fetch the actual expert if the slice held is not it
                ok = lds_wait(sig, [&] { return sig_get(sig + SG_TOPK) >= l + 1; }, err);
                if (!ok) break;
                const uint32_t slot = sig_get(sig + SG_SLOT + par);
                const uint32_t e = min(slot & 0xFFFFu, E - 1);
                if (!(slot >> 31)) {
                    load_slice(l, e, true, true);
                    vm_wait_n(n_dn);   // everything but the down copies just issued
                    if (lane == 0) sig_set(sig + SG_GUTAG + pw, slice_tag(l, e));
                    vm_wait_all();
                    if (lane == 0) sig_set(sig + SG_DNTAG + par * SP_PW + pw, slice_tag(l, e));
                }
                if (l + 1 >= n_layers) break;
                // the next layer's predicted slice: down rows into the other
                // buffer (layer l - 1's, read) and the router rows of layer l + 2
                // (layer l's, read once both of its logit rows are published)
                // right away; gate/up rows once layer l's gate/up rows are read
                // and its h exchange is over (copies in flight on a CU slow its
                // exchange polls)
                ok = lds_wait(sig, [&] {
                    return sig_get(sig + SG_PREDOK) >= l + 1 && sig_all_ge(sig, SG_ROUTE, 0, SP_CW, l + 1);
                }, err);
                if (!ok) break;
                const uint32_t pe = min(sig_get(sig + SG_PRED + (par ^ 1u) * 8 + x), E - 1);
                load_slice(l + 1, pe, false, true);
                if (l + 2 < n_layers) load_router(l + 2);
                ok = lds_wait(sig, [&] {
                    return sig_all_ge(sig, SG_GUFREE, 0, SP_CW, l + 1) && sig_get(sig + SG_CBAR) >= 2 * SP_CW * (l + 1);
                }, err);
                if (!ok) break;
                vm_wait_all();
                if (lane == 0) {
                    sig_set(sig + SG_DNTAG + (par ^ 1u) * SP_PW + pw, slice_tag(l + 1, pe));
                    if (l + 2 < n_layers) sig_set(sig + SG_RTAG + pw, l + 3);
                }
                load_slice(l + 1, pe, true, false);
                vm_wait_all();
                if (lane == 0) sig_set(sig + SG_GUTAG + pw, slice_tag(l + 1, pe));
            }
            vm_wait_all();
        } else {
            // ================= compute waves =================
            const uint32_t w = static_cast<uint32_t>(wv);
            uint32_t cbar = 0;
            // down rows: segment g (32 lanes) owns rows 4 g .. 4 g + 3 of the
            // wave's 8; lane c0 < I/32 owns chunk c0
            const uint32_t CH = I >> 5;
            const uint32_t g = static_cast<uint32_t>(lane) >> 5, c0 = static_cast<uint32_t>(lane) & 31u;
            const bool cact = c0 < CH;
            const uint32_t dc = cact ? c0 : CH - 1;
            for (uint32_t l = 0; l < n_layers; ++l) {
                const uint32_t ep = ep0 + l + 1;
                const bool nxt = l + 1 < n_layers;
                const uint32_t par = l & 1;
                uint64_t* tr = trace ? trace + ((size_t(l) * SP_BLOCKS + b) * 16) : nullptr;
                const bool trw = tr && lane == 0;
                if (trw && w == 2) {
                    tr[0] = tstamp();
                    tr[12] = role;
                }
                // ---- H: the layer's input into LDS (an eighth per wave) ----
                {
                    const uint32_t q4 = w * 64 + lane;      // float4 index of the layer input
                    float4 v;
                    if (l == 0) {
                        v = load_f4(hidden + 4 * q4);
                    } else {
                        const uint64_t* src = HN(l - 1, x) + 4 * q4;
                        poll_words(
                            [&] {
                                const uint64_t a0 = get_agent(src), a1 = get_agent(src + 1);
                                const uint64_t a2 = get_agent(src + 2), a3 = get_agent(src + 3);
                                v = make_float4(value_of(a0), value_of(a1), value_of(a2), value_of(a3));
                                return has_tag(a0, ep - 1) && has_tag(a1, ep - 1) && has_tag(a2, ep - 1) &&
                                       has_tag(a3, ep - 1);
                            },
                            sig, err);
                    }
                    S.hid[(q4 & 7) * NCH + (q4 >> 3)] = v;   // quad q of chunk q4 / 8
                }
                if (trw && w == 2) tr[13] = tstamp();
                compute_barrier(sig, cbar, err);
                if (l == 0 && w == 0 && lane == 0)
                    __hip_atomic_fetch_add(ctl + CTL_ARRIVED, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
                if (trw && w == 2) tr[1] = tstamp();

                // ---- N: norm, router row of layer l (waves 0-3) or l + 1 (waves 4-7) ----
                float hx[32];
#pragma unroll
                for (int q = 0; q < 8; ++q) {
                    const float4 f = S.hid[q * NCH + lane];
                    hx[4 * q] = f.x;
                    hx[4 * q + 1] = f.y;
                    hx[4 * q + 2] = f.z;
                    hx[4 * q + 3] = f.w;
                }
                float ss = 0.f;
#pragma unroll
                for (int k = 0; k < 32; ++k) ss = fmaf(hx[k], hx[k], ss);
                ss = wave_sum(ss);
                const float inv = 1.0f / sqrtf(ss / static_cast<float>(D) + 1e-6f);
                const bool pred_row = w >= 4;
                const uint32_t need = nxt ? l + 2 : l + 1;
                lds_wait(sig, [&] { return sig_all_ge(sig, SG_RTAG, 0, SP_PW, need); }, err);
                if (trw && w == 2) tr[14] = tstamp();
                // normed chunk with layer l's norm weights (for gate/up) and the router dot
                float a[32];
                float lg = 0.f;
                {
                    const uint32_t jr = w & 3u;
                    const uint32_t rb = pred_row ? (par ^ 1u) : par;     // router / norm buffer used for the dot
#pragma unroll
                    for (int q = 0; q < 4; ++q) {
                        const uint4 gv = S.nw[par][q * NCH + lane];
                        const uint32_t g4[4] = {gv.x, gv.y, gv.z, gv.w};
#pragma unroll
                        for (int t = 0; t < 4; ++t) {
                            const int k = 8 * q + 2 * t;
                            a[k] = (hx[k] * inv) * bf16_to_f32(g4[t] & 0xFFFFu);
                            a[k + 1] = (hx[k + 1] * inv) * bf16_to_f32(g4[t] >> 16);
                        }
                    }
                    if (!pred_row || nxt) {
                        float acc4[4] = {0.f, 0.f, 0.f, 0.f};    // one chain per quad (independent FMAs)
#pragma unroll
                        for (int q = 0; q < 4; ++q) {
                            const uint4 gv = S.nw[rb][q * NCH + lane];
                            const uint4 rv = S.rt[rb][jr][q * NCH + lane];
                            const uint32_t g4[4] = {gv.x, gv.y, gv.z, gv.w};
                            const uint32_t r4[4] = {rv.x, rv.y, rv.z, rv.w};
#pragma unroll
                            for (int t = 0; t < 4; ++t) {
                                const int k = 8 * q + 2 * t;
                                const float p0 = pred_row ? (hx[k] * inv) * bf16_to_f32(g4[t] & 0xFFFFu) : a[k];
                                const float p1 = pred_row ? (hx[k + 1] * inv) * bf16_to_f32(g4[t] >> 16) : a[k + 1];
                                acc4[q] = fmaf(bf16_to_f32(r4[t] & 0xFFFFu), p0, acc4[q]);
                                acc4[q] = fmaf(bf16_to_f32(r4[t] >> 16), p1, acc4[q]);
                            }
                        }
                        lg = (acc4[0] + acc4[1]) + (acc4[2] + acc4[3]);
                    }
                    // (this wave has read the layer's router and norm buffers)
                    if (lane == 0) sig_set(sig + SG_ROUTE + w, l + 1);
                    lg = wave_sum(lg);
                    const uint32_t jw = 4 * c + jr;
                    if (jw < E && lane == 0 && (!pred_row || nxt))
                        put_xcd(LG(l, x) + (pred_row ? 128 : 0) + jw, sword(ep, lg), local);
                }
                if (trw && w == 2) tr[2] = tstamp();

                uint32_t slot_info = 0;   // slot expert | hit << 31, as wave 0 published it
                if (w == 0) {
                    // ---- T: exact top-k, slots ----
                    float v[2];
                    {
                        const uint64_t* src = LG(l, x);
                        poll_words(
                            [&] {
                                bool okw = true;
#pragma unroll
                                for (int j = 0; j < 2; ++j) {
                                    const uint32_t pos = lane + WAVE * j;
                                    const uint64_t a0 = get_agent(src + min(pos, E - 1));
                                    v[j] = value_of(a0);
                                    okw &= pos >= E || has_tag(a0, ep);
                                }
                                return okw;
                            },
                            sig, err);
                    }
                    if (trw) tr[9] = tstamp();
                    uint32_t my_id;
                    float my_w;
                    topk_latency<2>(v, E, 8, d.norm_topk, my_id, my_w, S.topk);
                    my_id = min(my_id, E - 1);
                    if (trw) tr[10] = tstamp();
                    // slot s keeps P[s] when it is selected; the unmatched ranks
                    // fill the unmatched slots in slot order
                    const uint32_t s = static_cast<uint32_t>(lane) & 7u;
                    const uint32_t ps = l > 0 ? min(sig_get(sig + SG_PRED + par * 8 + s), E - 1) : 0xFFFFu;
                    uint32_t match = 8;   // lane s: rank r with S_r == P[s]
#pragma unroll
                    for (int r = 7; r >= 0; --r)
                        match = readlane_u32(my_id, r) == ps ? static_cast<uint32_t>(r) : match;
                    const uint32_t hits = static_cast<uint32_t>(__ballot(lane < 8 && match < 8)) & 0xFFu;
                    // ranks taken by a hit
                    uint32_t taken = 0;
#pragma unroll
                    for (int t = 0; t < 8; ++t) {
                        const uint32_t m = readlane_u32(match, t);
                        taken |= m < 8 ? 1u << m : 0u;
                    }
                    const uint32_t free_slots = ~hits & 0xFFu, free_ranks = ~taken & 0xFFu;
                    const uint32_t j = __popc(free_slots & ((1u << s) - 1u));
                    // the j-th set bit of free_ranks
                    uint32_t fr = free_ranks;
                    for (uint32_t t = 0; t < j; ++t) fr &= fr - 1u;
                    const uint32_t pick = fr ? static_cast<uint32_t>(__ffs(fr) - 1) : 0u;
                    const uint32_t rank_of_slot = match < 8 ? match : pick;
                    const uint32_t my_rank = readlane_u32(rank_of_slot, static_cast<int>(x));
                    const uint32_t slot_e = min(readlane_u32(my_id, static_cast<int>(my_rank)), E - 1);
                    const bool hit = (hits >> x) & 1u;
                    if (lane < 8) {
                        S.sig[SG_SOR + par * 8 + rank_of_slot] = lane;   // slot lane computes rank rank_of_slot
                        S.sig[SG_W + par * 8 + lane] = __float_as_uint(my_w);
                    }
                    slot_info = slot_e | (hit ? 0x80000000u : 0u);
                    if (lane == 0) {
                        S.sig[SG_SLOT + par] = slot_info;
                        sig_set(sig + SG_TOPK, l + 1);
                    }
                    if (x == 0 && c == 0 && lane < 8) {
                        if (ids_out) ids_out[size_t(l) * 8 + lane] = my_id;
                        if (w_out) w_out[size_t(l) * 8 + lane] = my_w;
                    }
                    if (trw) {
                        tr[3] = tstamp();
                        tr[15] = (uint64_t(hits) << 32) | (hit ? 0x10000u : 0u) | slot_e;
                    }
                    if (lane == 0) sig_set(sig + SG_GUFREE + w, l + 1);
                } else if (w == 1) {
                    // ---- T: the prediction for layer l + 1 ----
                    if (nxt) {
                        float vp[2];
                        const uint64_t* src = LG(l, x) + 128;
                        poll_words(
                            [&] {
                                bool okw = true;
#pragma unroll
                                for (int j = 0; j < 2; ++j) {
                                    const uint32_t pos = lane + WAVE * j;
                                    const uint64_t a0 = get_agent(src + min(pos, E - 1));
                                    vp[j] = value_of(a0);
                                    okw &= pos >= E || has_tag(a0, ep);
                                }
                                return okw;
                            },
                            sig, err);
                        const uint32_t pn = top8_positions(vp, E);
                        if (lane < 8) S.sig[SG_PRED + (par ^ 1u) * 8 + lane] = pn;
                        if (lane == 0) sig_set(sig + SG_PREDOK, l + 1);
                    }
                    if (lane == 0) sig_set(sig + SG_GUFREE + w, l + 1);
                } else {
                    // ---- U: gate/up rows of the predicted expert, confirmed by T ----
                    Q4Act qa;
                    q4_act_from_floats(a, qa);
                    const uint32_t u = w - 2;                     // gate/up wave index
                    auto gate_up = [&](float (&part)[NR]) {
#pragma unroll
                        for (int i = 2 * RB; i < NR; ++i) part[i] = 0.f;
#pragma unroll
                        for (int i = 0; i < RB; ++i) {
                            const uint32_t row = u * RB + i;      // CU-local gate/up row
                            const uint4 va = *reinterpret_cast<const uint4*>(&S.gu[row * GU_ROW + lane * 16]);
                            const uint4 vb = *reinterpret_cast<const uint4*>(&S.gu[gu_p + row * GU_ROW + lane * 16]);
                            const uint16_t sa = *reinterpret_cast<const uint16_t*>(
                                &S.gu[2 * gu_p + row * GU_ROW_SC + (lane >> 1) * 2]);
                            const uint16_t sb = *reinterpret_cast<const uint16_t*>(
                                &S.gu[2 * gu_p + gu_s + row * GU_ROW_SC + (lane >> 1) * 2]);
                            part[2 * i] = f16_bits_to_f32(sa) * q4_chunk_dot8(va, qa);
                            part[2 * i + 1] = f16_bits_to_f32(sb) * q4_chunk_dot8(vb, qa);
                        }
                    };
                    float part[NR];
                    uint32_t have = 0xFFFFFFFFu;                 // expert whose rows `part` holds
                    if (l > 0) {
                        const uint32_t pe = min(sig_get(sig + SG_PRED + par * 8 + x), E - 1);
                        const uint32_t ptag = slice_tag(l, pe);
                        // the prefetched slice; should the prefetch waves have
                        // replaced it already (a miss seen first), T decides below
                        lds_wait(sig, [&] {
                            return sig_all_eq(sig, SG_GUTAG, SP_PW, ptag) || sig_get(sig + SG_TOPK) >= l + 1;
                        }, err);
                        if (sig_all_eq(sig, SG_GUTAG, SP_PW, ptag)) {
                            gate_up(part);
                            have = pe;
                        }
                    }
                    if (trw && w == 2) tr[4] = tstamp();
                    lds_wait(sig, [&] { return sig_get(sig + SG_TOPK) >= l + 1; }, err);
                    slot_info = sig_get(sig + SG_SLOT + par);
                    const uint32_t slot_e = slot_info & 0xFFFFu;
                    if (have != slot_e) {
                        const uint32_t tag = slice_tag(l, slot_e);
                        lds_wait(sig, [&] { return sig_all_eq(sig, SG_GUTAG, SP_PW, tag); }, err);
                        gate_up(part);
                    }
                    if (lane == 0) sig_set(sig + SG_GUFREE + w, l + 1);
                    if (trw && w == 2) tr[11] = tstamp();
                    constexpr int USH = 6 - ilog2(NR);
                    const float tot = wave_sum_rows<NR>(part);   // lane l: total of value l >> USH
                    const float gv = __shfl(tot, (2 * lane) << USH);
                    const float uv = __shfl(tot, (2 * lane + 1) << USH);
                    // silu(z) = z * (1 / (1 + exp(-z)))  (kernels.metal:61-63, :334-336)
                    if (lane < RB)
                        put_xcd(HX(l, x) + c * RBC + u * RB + lane,
                                sword(ep, (gv * (1.0f / (1.0f + expf(-gv)))) * uv), local);
                    if (trw && w == 2) tr[5] = tstamp();
                }

                // ---- D: all of h into LDS (an eighth per wave), down rows ----
                {
                    const uint32_t per = I / SP_CW;               // words per wave (<= 96)
                    const uint64_t* src = HX(l, x);
                    float hv[2];
                    poll_words(
                        [&] {
                            bool okw = true;
#pragma unroll
                            for (int m = 0; m < 2; ++m) {
                                const uint32_t i = m * WAVE + lane;
                                if (i < per) {
                                    const uint64_t a0 = get_agent(src + w * per + i);
                                    hv[m] = value_of(a0);
                                    okw &= has_tag(a0, ep);
                                }
                            }
                            return okw;
                        },
                        sig, err);
                    float* hq = reinterpret_cast<float*>(S.h);
#pragma unroll
                    for (int m = 0; m < 2; ++m) {
                        const uint32_t i = m * WAVE + lane;
                        if (i < per) {
                            const uint32_t k = w * per + i;        // element of h: chunk k/32, quad (k%32)/4
                            hq[(((k & 31u) >> 2) * H_CH + (k >> 5)) * 4 + (k & 3u)] = hv[m];
                        }
                    }
                }
                compute_barrier(sig, cbar, err);
                if (trw && w == 2) tr[6] = tstamp();
                if (w < 2) slot_info = sig_get(sig + SG_SLOT + par);
                const uint32_t slot_e = slot_info & 0xFFFFu;
                Q4Act qh;
                {
                    float hc[32];
#pragma unroll
                    for (int q = 0; q < 8; ++q) {
                        const float4 f = S.h[q * H_CH + dc];
                        hc[4 * q] = f.x;
                        hc[4 * q + 1] = f.y;
                        hc[4 * q + 2] = f.z;
                        hc[4 * q + 3] = f.w;
                    }
                    q4_act_from_floats(hc, qh);
                }
                const uint32_t tag = slice_tag(l, slot_e);
                lds_wait(sig, [&] { return sig_all_eq(sig, SG_DNTAG + par * SP_PW, SP_PW, tag); }, err);
                float y_row;
                {
                    float acc[4];
#pragma unroll
                    for (int i = 0; i < 4; ++i) {
                        const uint32_t row = w * DN_ROWS_W + g * 4 + i;   // CU-local down row
                        const uint4 dv = *reinterpret_cast<const uint4*>(&S.dn[par][row * dn_row + dc * 16]);
                        const uint16_t sc =
                            *reinterpret_cast<const uint16_t*>(&S.dn[par][dn_p + row * dn_row_sc + (dc >> 1) * 2]);
                        const float yv = f16_bits_to_f32(sc) * q4_chunk_dot8(dv, qh);
                        acc[i] = cact ? yv : 0.f;
                    }
                    if (lane == 0) sig_set(sig + SG_DNFREE + w, l + 1);
                    // lane l holds the total of row (l >> 3) & 3 of segment l >> 5
                    y_row = seg_sum_rows<4, 5>(acc);
                }
                {
                    const bool holder = (lane & 7) == 0;
                    const uint32_t row = 64 * c + w * DN_ROWS_W + (lane >> 5) * 4 + ((lane >> 3) & 3);
                    if (holder) put_agent(YS(l, x) + row, sword(ep, y_row));
                }
                if (trw && w == 2) tr[7] = tstamp();

                // ---- C: hidden + sum_r w_r y_r for the wave's 8 rows, rank order ----
                {
                    // lane (s = lane >> 3, r8 = lane & 7) polls slot s of row r8
                    const uint32_t r8 = static_cast<uint32_t>(lane) & 7u, sl = static_cast<uint32_t>(lane) >> 3;
                    const uint32_t row = 64 * c + w * DN_ROWS_W + r8;
                    float yv = 0.f;
                    poll_words(
                        [&] {
                            const uint64_t a0 = get_agent(YS(l, sl) + row);
                            yv = value_of(a0);
                            return has_tag(a0, ep);
                        },
                        sig, err);
                    // routed_out += w_r * y_r in rank order (axpy_f32, common.hpp:346-349),
                    // then hidden += routed_out (decode.cpp:506-509)
                    const uint32_t so = S.sig[SG_SOR + par * 8 + (lane & 7)];     // lane r: slot of rank r
                    const float wr = __uint_as_float(S.sig[SG_W + par * 8 + (lane & 7)]);   // lane r: w_r
                    float routed = 0.f;
#pragma unroll
                    for (int r = 0; r < 8; ++r) {
                        const uint32_t sr = readlane_u32(so, r);
                        const float y = __shfl(yv, static_cast<int>((sr << 3) | r8));
                        routed = routed + readlane_f32(wr, r) * y;
                    }
                    const float hnew = reinterpret_cast<const float*>(S.hid)[((row & 31u) >> 2) * NCH * 4 +
                                                                              (row >> 5) * 4 + (row & 3u)] +
                                       routed;
                    if (lane < 8) {
                        if (nxt) {
                            put_xcd(HN(l, x) + row, sword(ep, hnew), local);
                        } else if (x == 0) {
                            // the caller's buffer is overwritten only once every block has read it
                            lds_wait(sig, [&] { return get_agent32(ctl + CTL_ARRIVED) >= gridDim.x; }, err);
                            hidden[row] = hnew;
                        }
                    }
                }
                if (trw && w == 2) tr[8] = tstamp();
            }
        }
    } else if (tid == 0) {
        // a block without a role never reads hidden
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
namespace {

template <int RB>
bool spec_resident()
{
    static const bool ok = [] {
        int dev = 0, per_cu = 0, cus = 0;
        if (hipGetDevice(&dev) != hipSuccess) return false;
        if (hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess) return false;
        if (hipOccupancyMaxActiveBlocksPerMultiprocessor(&per_cu, k_decode_spec<RB>, SP_THREADS, 0) != hipSuccess)
            return false;
        return cus == SP_BLOCKS && per_cu >= 1;
    }();
    return ok;
}

template <int RB>
hipError_t spec_launch(const MoeDims& d, const LayerDesc* layers, uint32_t n_layers, float* hidden, uint64_t* xch,
                       uint32_t* ctl, uint32_t* ids, float* w, uint32_t* err, uint64_t* trace, hipStream_t s,
                       bool dry)
{
    if (!spec_resident<RB>()) return hipErrorInvalidConfiguration;
    if (dry) return hipSuccess;
    launch_kernel(k_decode_spec<RB>, dim3(SP_BLOCKS), dim3(SP_THREADS), s, d, layers, n_layers, hidden, xch, ctl, ids,
                  w, err, trace);
    return hipGetLastError();
}

hipError_t spec_dispatch(const MoeDims& d, const LayerDesc* layers, uint32_t n_layers, float* hidden, uint64_t* xch,
                         uint32_t* ctl, uint32_t* ids, float* w, uint32_t* err, uint64_t* trace, hipStream_t s,
                         bool dry)
{
    if (d.D != SP_D || d.K != 8 || d.group != 64 || d.E < 8 || d.E > 128 || d.I % 192 || d.I == 0 ||
        d.I > SP_MAX_I)
        return hipErrorInvalidValue;
    switch (d.I / 192) {
    case 1: return spec_launch<1>(d, layers, n_layers, hidden, xch, ctl, ids, w, err, trace, s, dry);
    case 2: return spec_launch<2>(d, layers, n_layers, hidden, xch, ctl, ids, w, err, trace, s, dry);
    case 3: return spec_launch<3>(d, layers, n_layers, hidden, xch, ctl, ids, w, err, trace, s, dry);
    case 4: return spec_launch<4>(d, layers, n_layers, hidden, xch, ctl, ids, w, err, trace, s, dry);
    default: return hipErrorInvalidValue;
    }
}

}  // namespace

bool spec_supported(const MoeDims& d)
{
    return spec_dispatch(d, nullptr, 0, nullptr, nullptr, nullptr, nullptr, nullptr, nullptr, nullptr, nullptr,
                         true) == hipSuccess;
}

hipError_t launch_decode_spec(const MoeDims& d, const LayerDesc* layers, uint32_t n_layers, float* hidden,
                              uint64_t* xch, uint32_t* ctl, uint32_t* ids, float* w, uint32_t* err, uint64_t* trace,
                              hipStream_t s)
{
    if (n_layers == 0 || !layers || !hidden || !xch || !ctl || !err) return hipErrorInvalidValue;
    return spec_dispatch(d, layers, n_layers, hidden, xch, ctl, ids, w, err, trace, s, false);
}

}  // namespace smoe
