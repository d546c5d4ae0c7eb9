// kernels.hpp -- host-side launchers of the gfx950 MoE kernels (internal to
// libsmoe_hip.so; the public surface is include/smoe_hip.h).
#pragma once

#include <hip/hip_ext.h>
#include <hip/hip_runtime.h>
#include <stdint.h>

namespace smoe {

// largest expert count a top-k wave handles (8 positions per lane)
constexpr int SMOE_TOPK_MAX_N = 512;
constexpr int SMOE_TOPK_MAX_K = 16;

// Events that time the next kernel dispatches of this thread: when set, the
// launchers dispatch through hipExtLaunchKernel, which records `start` when
// the kernel begins executing and `stop` when it completes (the dispatch's
// own timestamps, no marker packets around it).  Set only around eager
// launches by the profiling path of the C ABI.
struct DispatchTimer {
    hipEvent_t start = nullptr;
    hipEvent_t stop = nullptr;
};
DispatchTimer& dispatch_timer();

template <typename... KArgs, typename... Args>
inline void launch_kernel_lds(void (*k)(KArgs...), dim3 grid, dim3 block, uint32_t lds, hipStream_t s, Args... args)
{
    const DispatchTimer& t = dispatch_timer();
    if (t.start)
        hipExtLaunchKernelGGL(k, grid, block, lds, s, t.start, t.stop, 0, static_cast<KArgs>(args)...);
    else
        hipLaunchKernelGGL(k, grid, block, lds, s, static_cast<KArgs>(args)...);
}

template <typename... KArgs, typename... Args>
inline void launch_kernel(void (*k)(KArgs...), dim3 grid, dim3 block, hipStream_t s, Args... args)
{
    launch_kernel_lds(k, grid, block, 0u, s, args...);
}

// Routing exchange of one token: LL_COPIES copies of its E logit words (flag
// in the high half), ll_copy_words(E) words apart (> 4 KB), so the waves that
// poll them spread over several memory channels instead of queueing on one.
constexpr uint32_t LL_COPIES = 8;
__host__ __device__ constexpr uint32_t ll_copy_words(uint32_t E) { return (E > 512u ? E : 512u) + 32u; }
__host__ __device__ constexpr size_t ll_token_words(uint32_t E) { return size_t(LL_COPIES) * ll_copy_words(E); }

// Six tensor pointers of one expert plus the scratch slot its results use.
struct ExpertPtrs {
    const uint8_t*  pg;
    const uint16_t* sg;
    const uint8_t*  pu;
    const uint16_t* su;
    const uint8_t*  pd;
    const uint16_t* sd;
    uint32_t        slot;
    uint32_t        pad_;
};

struct MoeDims {
    uint32_t D, E, K, I, group, norm_topk;
    uint32_t quant = 0;   // SMOE_QUANT_*: 0 fp16 absmax (SMOE-Q4), 1 bf16 scale + bf16 min
};

struct LayerDesc {
    const uint16_t* norm_w;
    const uint16_t* router_w;
    const uint8_t*  experts;
    uint64_t        stride;
    uint64_t        off[6];   // gate p, gate s, up p, up s, down p, down s
};

// ---- decode, one token (moe_decode.hip) ----------------------------------
// Router + softmax/top-k (+renorm) + gate/up/SiLU of the selected experts:
// h [T x K x I]; publishes ids/w [T x K] and the expert table [T x K].
// ll [T x (E+1)] must be zero on entry (launch_down_combine re-arms it);
// err receives 1 if the routing exchange timed out.
hipError_t launch_moe_up(const MoeDims& d, const LayerDesc& L, const float* hidden, uint32_t n_tok, uint64_t* ll,
                         float* h, uint32_t* ids, float* w, ExpertPtrs* tbl, uint32_t* err, hipStream_t s);
// h[slot * h_stride + row] = silu(gate.x) * (up.x) for n_exp table entries;
// x_tok_stride / tbl_tok_stride / h_tok_stride step blockIdx.y over tokens.
hipError_t launch_gate_up(const MoeDims& d, const ExpertPtrs* tbl, uint32_t n_exp,
                          const float* x, float* h, uint32_t h_stride, uint32_t n_tok,
                          uint32_t x_tok_stride, uint32_t tbl_tok_stride,
                          uint32_t h_tok_stride, hipStream_t s);
// hidden[t][row] += sum_r w[t][r] * (down_r . h[t][r])  (weighted combine + residual);
// zeroes ll [T x (E+1)] for the next launch_moe_up
hipError_t launch_down_combine(const MoeDims& d, const ExpertPtrs* tbl, const float* h, const float* w,
                               float* hidden, uint64_t* ll, uint32_t n_tok, hipStream_t s);
// ---- decode, one token, one launch (moe_layer.hip) -----------------------
// Exchange-word tags of the one-launch decode kernels.  The epoch word holds
// a count e in [0, TAG_PERIOD); the words of layer l of a launch that read e
// carry tag_at(e, l) = ((e + l) mod TAG_PERIOD) + 1, and the launch leaves
// epoch_after(e, n_layers) behind.  Tags therefore run through 1 .. 2^32 - 1
// and wrap from 2^32 - 1 to 1: never 0 (every word's value at allocation),
// and two consecutive layers, in one launch or across launches, never share
// one.  Any 32-bit value read from the word is reduced first, so a word
// holding 2^32 - 1 counts as 0.
constexpr uint32_t TAG_PERIOD = 0xFFFFFFFFu;
__host__ __device__ constexpr uint32_t tag_mod(uint64_t s)
{
    // s mod (2^32 - 1): 2^32 is 1 modulo the period, so fold the high word in
    const uint64_t f = (s & 0xFFFFFFFFull) + (s >> 32);   // < 2^33
    const uint64_t g = (f & 0xFFFFFFFFull) + (f >> 32);   // <= 2^32
    return static_cast<uint32_t>(g >= TAG_PERIOD ? g - TAG_PERIOD : g);
}
__host__ __device__ constexpr uint32_t tag_at(uint32_t epoch, uint32_t l)
{
    return tag_mod(static_cast<uint64_t>(epoch) + l) + 1u;
}
__host__ __device__ constexpr uint32_t epoch_after(uint32_t epoch, uint32_t n_layers)
{
    return tag_mod(static_cast<uint64_t>(epoch) + n_layers);
}
// Exchange words of the one-launch layer: word 0 holds the epoch (above),
// then 8 logit copies of lx_pad(E) words, 8 h copies of lx_pad(I) words and
// 8 rank partials of lx_pad(D) words.  Zero once at allocation; never
// re-armed (a launch that times out leaves them to be cleared by the host).
constexpr uint32_t LX_HEAD = 64;
constexpr uint32_t LX_MAX_I = 2048;
__host__ __device__ constexpr uint32_t lx_pad(uint32_t n) { return ((n + 63u) & ~63u) + 64u; }
__host__ __device__ constexpr size_t lx_words(uint32_t D, uint32_t E, uint32_t I)
{
    return LX_HEAD + 8ull * (lx_pad(E) + lx_pad(I) + lx_pad(D));
}
// Checks once per device (synchronously, outside stream capture) that blocks
// are dealt round-robin over the 8 XCDs, which the one-launch layer kernels
// rely on; later calls return the cached answer.
bool deal_probe();
// true when k == 8, the shape's grid fits on the device at once, the layer's
// tensors are 16-byte aligned and the device deals blocks round-robin (as
// deal_probe found; false before it ran)
bool layer_supported(const MoeDims& d, const LayerDesc& L);
// the whole MoE block of one token: hidden [D] += MoE(RMSNorm(hidden));
// ids/w [K] receive the routing; err bit 0 reports an exchange time-out
hipError_t launch_moe_layer(const MoeDims& d, const LayerDesc& L, float* hidden, uint64_t* lx, uint32_t* ids,
                            float* w, uint32_t* err, hipStream_t s);
// Every layer of a decode step in one launch with k_moe_layer's schedule per
// layer.  xch: chain_xch_words(D, E, I) exchange words; hcopy [8 x D] floats;
// cnt chain_cnt_words() words (per-XCD row-block flags, then an abort word);
// all zero at allocation and never re-armed
// (calls on one set must not overlap).  layers_dev: the layer table in device
// memory; ids/w [n_layers x K].
constexpr uint32_t CHAIN_FLAGS = 256;       // row-block flags per XCD (n_down <= 256)
__host__ __device__ constexpr size_t chain_xch_words(uint32_t D, uint32_t E, uint32_t I)
{
    return lx_words(D, E, I) + 8ull * lx_pad(D);
}
constexpr size_t chain_cnt_words() { return 8 * CHAIN_FLAGS + 64; }
bool chain_supported(const MoeDims& d, const LayerDesc* layers_host, uint32_t n_layers);
hipError_t launch_moe_chain(const MoeDims& d, const LayerDesc* layers_dev, uint32_t n_layers, float* hidden,
                            uint64_t* xch, float* hcopy, uint32_t* cnt, uint32_t* ids, float* w, uint32_t* err,
                            hipStream_t s);
// out[slot * out_stride + row] = down_slot . h_slot   (per-expert outputs)
hipError_t launch_down_slots(const MoeDims& d, const ExpertPtrs* tbl, uint32_t n_exp,
                             const float* h, uint32_t h_stride, float* out,
                             uint32_t out_stride, uint32_t n_tok, uint32_t tbl_tok_stride,
                             uint32_t h_tok_stride, uint32_t out_tok_stride, hipStream_t s);
// softmax + top-k over rows of scores (scout.cpp:77-123)
hipError_t launch_topk(const float* scores, uint32_t rows, uint32_t n, uint32_t k,
                       uint32_t norm, uint32_t* ids, float* w, hipStream_t s);


// out [rows] = W [rows x cols] bf16 . x [cols] (reference-surface dense GEMV)
hipError_t launch_matvec_bf16(const uint16_t* W, const float* x, float* out, uint32_t rows, uint32_t cols,
                              hipStream_t s);

// ---- dense trunk (trunk.hip) ---------------------------------------------
// up to GEMV_MAX independent y = W x (bf16 W [rows x cols], fp32 x, y) in one
// launch; cols % 8 == 0, cols <= GEMV_MAX_COLS, W and x 16-byte aligned
constexpr uint32_t GEMV_MAX = 8;
constexpr uint32_t GEMV_MAX_COLS = 16384;
struct GemvGroup {
    const uint16_t* w[GEMV_MAX];
    const float* x[GEMV_MAX];
    float* y[GEMV_MAX];
    uint32_t rows[GEMV_MAX], cols[GEMV_MAX], block0[GEMV_MAX];
    uint32_t count;
};
hipError_t launch_gemv_bf16(const GemvGroup& g, hipStream_t s);

// single-token decode attention over a KV ring of ctx positions: one fused
// launch (QK norm + RoPE + KV append, attention per (KV head, query-head
// group, context split) with an online softmax), and with several splits a
// combine launch, into attn_out [q_dim].  head_dim 64, 128 or 256.
constexpr uint32_t ATTN_MAX_SPLITS = 64;
struct AttnDims {
    uint32_t head_dim, num_heads, num_kv_heads, kv_dim, ctx;
    float scale;
};
struct AttnPlan {
    uint32_t gb;        // query heads per block (power of two <= 8)
    uint32_t n_sub;     // blocks per KV head along the query heads
    uint32_t splits;    // context splits
    uint32_t chunk;     // positions per split
};
AttnPlan attn_plan(const AttnDims& a, uint32_t valid);
// scratch of the launch: per-(head, split) partials
size_t attn_scratch_bytes(const AttnDims& a);
hipError_t launch_attention(const AttnDims& a, const float* q, const float* k, const float* v,
                            const uint16_t* q_norm_w, const uint16_t* k_norm_w, const float* rope_cos,
                            const float* rope_sin, float* k_cache, float* v_cache, uint32_t slot, uint32_t valid,
                            void* scratch, float* attn_out, hipStream_t s);

// ---- prefill, T token rows (moe_prefill.hip) -----------------------------
// RMSNorm + router + top-k for T tokens: the normed rows as f16 planes
// x_hi/x_lo [T x D] with row scales x_sc [T] (as launch_split_rows writes
// them), ids/w [T x K].  logits [T x E] and counters [T] (zero at allocation;
// every launch adds a multiple of 4) serve the short-batch form; with either
// null every token group runs in one block.
hipError_t launch_route(const MoeDims& d, const LayerDesc& L, const float* hidden, uint32_t T, uint16_t* x_hi,
                        uint16_t* x_lo, float* x_sc, uint32_t* ids, float* w, float* logits, uint32_t* counters,
                        hipStream_t s);
// Per row of src [rows x cols]: f16 hi/lo planes of x * 2^-e (|x| < 2^e over
// the row) and scale[row] = 2^e.
hipError_t launch_split_rows(const float* src, uint32_t rows, uint32_t cols, uint16_t* hi, uint16_t* lo,
                             float* scale, hipStream_t s);
// Stable counting sort of the P pairs by expert: offsets [E+1],
// sorted_pairs [P] (pair = token * K + rank); sorted_tokens, sorted_w,
// union_ids [E], union_size [1] optional (nullptr).  sched [E + 1] optional: the
// grouped GEMMs' work order (count of touched experts, then the experts by
// decreasing cost).  Bad ids set err bit 1.
constexpr size_t PERMUTE_MAX_LDS = 48 * 1024;
size_t permute_lds_bytes(uint32_t P, uint32_t E);
hipError_t launch_permute(const uint32_t* ids, const float* w, uint32_t P, uint32_t K, uint32_t E, uint32_t* offsets,
                          uint32_t* sorted_pairs, uint32_t* sorted_tokens, float* sorted_w, uint32_t* union_ids,
                          uint32_t* union_size, uint32_t* sched, uint32_t* err, hipStream_t s);
// Grouped expert GEMMs over the permuted pairs (MFMA f16, hi/lo activations):
// h [P x I] = silu(x G^T) * (x U^T); y [P x D] = h Dn^T.  sched is the
// permute's work order.
hipError_t launch_grouped_gate_up(const MoeDims& d, const LayerDesc& L, const uint32_t* offsets,
                                  const uint32_t* sched, const uint32_t* sorted_pairs, const uint16_t* x_hi,
                                  const uint16_t* x_lo, const float* x_scale, float* h, hipStream_t s);
hipError_t launch_grouped_down(const MoeDims& d, const LayerDesc& L, const uint32_t* offsets,
                               const uint32_t* sched, const uint32_t* sorted_pairs, const uint16_t* h_hi,
                               const uint16_t* h_lo, const float* h_scale, float* y, hipStream_t s);
// hidden[t] += sum_r w[t][r] * y[t*K + r] (rank order).
hipError_t launch_combine_pairs(const float* y, const float* w, uint32_t T, uint32_t K, uint32_t D, float* hidden,
                                hipStream_t s);

// ---- static scratch of smoe_hip_moe_decode_static (decode_static.hip) -----
// Takes the current device's address of the file-scope scratch array and
// clears it, once per device (synchronous; outside stream capture).
uint64_t* static_scratch_setup();

// ---- measurement (probe.hip) ----------------------------------------------
// Streams `bytes` (a multiple of 16) from src with non-temporal 128-bit loads;
// folds what it read into *sink.
hipError_t launch_stream_read(const void* src, uint64_t bytes, uint32_t* sink, hipStream_t s);

// ---- synthetic generator / quantizer (synth.hip) -------------------------
hipError_t launch_synth_normal(float* out, uint64_t n, uint64_t seed, uint64_t stream,
                               float stddev, hipStream_t s);
hipError_t launch_synth_bf16(uint16_t* out, uint64_t n, uint64_t seed, uint64_t stream,
                             float stddev, hipStream_t s);
hipError_t launch_quantize_q4(const float* w, uint64_t n, uint32_t group, uint8_t* packed,
                              uint16_t* scales, hipStream_t s);
// the scale+min format: scales and mins [n / group] bf16 bits
hipError_t launch_quantize_q4_min(const float* w, uint64_t n, uint32_t group, uint8_t* packed,
                                  uint16_t* scales, uint16_t* mins, hipStream_t s);
// quant: SMOE_QUANT_*; with the scale+min format each matrix's mins follow
// its D*I/group scales
hipError_t launch_synth_pool(uint8_t* base, uint32_t first_layer, uint32_t n_layers,
                             uint32_t n_experts, uint64_t stride, uint32_t D, uint32_t I,
                             uint32_t group, const uint64_t* off6, uint64_t seed,
                             float stddev, uint32_t quant, hipStream_t s);

}  // namespace smoe
