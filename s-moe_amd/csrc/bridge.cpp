// bridge.cpp -- C ABI of the MI355X MoE backend (include/smoe_hip.h).
//
// Implements the reference's compute-backend surface (metal_bridge.h, whose
// Metal implementation is src/compute/metal_bridge.mm) on HIP, plus the
// device-resident entry points.  The context owns one HIP stream (or uses the
// caller's), pre-allocated scratch, and a ring of events backing the
// monotonically increasing handles of the reference (metal_bridge.mm:423-429).
#include "smoe_hip.h"

#include <hip/hip_runtime.h>

#include <algorithm>
#include <atomic>
#include <cstdio>
#include <cstring>
#include <vector>

#include "kernels.hpp"
#include "shape.hpp"

using smoe::ExpertPtrs;
using smoe::LayerDesc;
using smoe::MoeDims;
using smoe::dims_of;
using smoe::layer_of;
using smoe::shape_check;

namespace {

constexpr uint32_t kSlots = SMOE_MAX_ACTIVE;   // scratch regions (metal_bridge.mm:205-210)
constexpr uint32_t kEvents = 256;              // handle ring

struct DeviceScratch {
    // capacities
    uint32_t D = 0, E = 0, K = 0, I = 0, T = 0;
    uint64_t* ll = nullptr;      // [T x ll_token_words(E)] routing exchange words
    uint32_t* ids = nullptr;     // [T x K]
    float* w = nullptr;          // [T x K]
    ExpertPtrs* tbl = nullptr;   // [T x K]
    float* h = nullptr;          // [T x K x I]
    uint64_t* lx = nullptr;      // one-launch layer exchange words (lx_words), zero at allocation
};

// prefill / permute scratch for one batch of up to T tokens (P = T * K pairs)
struct PrefillScratch {
    uint32_t D = 0, E = 0, K = 0, I = 0, T = 0;
    uint16_t* x_hi = nullptr;       // [T x D] f16
    uint16_t* x_lo = nullptr;
    float* x_sc = nullptr;          // [T] row scales
    float* logits = nullptr;        // [T x E] router logits (short batches)
    uint32_t* rt_ctr = nullptr;     // [T] route counters (zero between launches)
    uint32_t* ids = nullptr;        // [T x K]
    float* w = nullptr;             // [T x K]
    uint32_t* offsets = nullptr;    // [E + 1]
    uint32_t* sched = nullptr;      // [E + 1] grouped GEMM work order
    uint32_t* pairs = nullptr;      // [P] sorted pair ids
    float* h = nullptr;             // [P x I]
    uint16_t* h_hi = nullptr;       // [P x I] f16
    uint16_t* h_lo = nullptr;
    float* h_sc = nullptr;          // [P] row scales
    float* y = nullptr;             // [P x D]
};

// the chained decode kernel's device copy of the layer table
struct LayerTable {
    LayerDesc* tbl = nullptr;       // [tbl_cap]
    uint32_t tbl_cap = 0;
    std::vector<LayerDesc> host_tbl;   // what tbl holds
};

// the chained decode kernel: exchange words, per-XCD hidden copies and
// counters (zeroed once; the kernel keeps them), routing outputs nobody asked for
struct ChainScratch {
    size_t words = 0;               // capacity of xch
    uint64_t* xch = nullptr;
    size_t hcopy_n = 0;             // capacity of hcopy (floats)
    float* hcopy = nullptr;
    uint32_t* cnt = nullptr;        // [chain_cnt_words()]
    size_t out_n = 0;               // capacity of ids / w
    uint32_t* ids = nullptr;
    float* w = nullptr;
};

}  // namespace

struct SmoeMetalCtx {
    int device = 0;
    hipStream_t own_stream = nullptr;
    hipStream_t stream = nullptr;
    size_t slot_bytes = 0;
    uint32_t max_rows = 0;

    // reference-surface scratch (metal_bridge.mm:205-217, :269-272)
    float* d_input = nullptr;        // [SMOE_MAX_DIM]
    float* d_hidden = nullptr;       // [kSlots x max_rows]
    float* d_output = nullptr;       // [kSlots x max_rows]
    float* d_batch_in = nullptr;     // [64 x 16384]
    float* d_batch_hidden = nullptr;
    float* d_batch_out = nullptr;
    ExpertPtrs* d_tbl_ref = nullptr; // [kSlots]

    hipEvent_t ev[kEvents] = {};
    uint64_t seq = 0;
    std::atomic<uint64_t> dispatches{0};

    DeviceScratch ds;
    PrefillScratch ps;
    LayerTable lt;
    ChainScratch cs;
    int decode_engine = SMOE_DECODE_CHAIN;      // smoe_hip_moe_decode_stack's engine
    uint32_t* d_err = nullptr;       // [1] device-side error flags (bit 0: exchange time-out, bit 1: bad expert id)
    uint32_t* perm_pairs = nullptr;  // smoe_hip_permute's sorted pair ids
    float* mv_in = nullptr;          // reference-surface GEMV staging
    uint8_t* attn_part = nullptr;    // decode attention: per-(head, split) partials + counters
    size_t attn_part_cap = 0;        // bytes
    float* mv_out = nullptr;
    uint32_t mv_cap = 0;
    uint64_t perm_cap = 0;
    std::vector<std::pair<uintptr_t, size_t>> registered;
    char last_err[256] = {0};

    // per-kernel event timing
    struct ProfSlot {
        hipEvent_t a = nullptr, b = nullptr;
        uint32_t kind = 0;
        bool pending = false;
    };
    bool profiling = false;
    std::vector<ProfSlot> prof;
    size_t prof_head = 0;
    uint64_t prof_launches[SMOE_KERNEL_KINDS] = {};
    double prof_ms[SMOE_KERNEL_KINDS] = {};
    int prof_open = -1;   // slot index between prof_begin and prof_end
};

namespace {

bool hip_ok(SmoeMetalCtx* ctx, hipError_t e, const char* what)
{
    if (e == hipSuccess) return true;
    if (ctx) std::snprintf(ctx->last_err, sizeof(ctx->last_err), "%s: %s", what, hipGetErrorString(e));
    std::fprintf(stderr, "[smoe_hip] %s failed: %s\n", what, hipGetErrorString(e));
    return false;
}

template <typename T>
bool dalloc(SmoeMetalCtx* ctx, T** p, size_t count)
{
    *p = nullptr;
    if (count == 0) count = 1;
    return hip_ok(ctx, hipMalloc(reinterpret_cast<void**>(p), count * sizeof(T)), "hipMalloc");
}

template <typename T>
void dfree(T*& p)
{
    if (p) (void)hipFree(p);
    p = nullptr;
}

void free_device_scratch(DeviceScratch& s)
{
    dfree(s.ll);
    dfree(s.ids);
    dfree(s.w);
    dfree(s.tbl);
    dfree(s.h);
    dfree(s.lx);
    s = DeviceScratch{};
}

void free_prefill_scratch(PrefillScratch& s)
{
    dfree(s.x_hi);
    dfree(s.x_lo);
    dfree(s.x_sc);
    dfree(s.logits);
    dfree(s.rt_ctr);
    dfree(s.ids);
    dfree(s.w);
    dfree(s.offsets);
    dfree(s.sched);
    dfree(s.pairs);
    dfree(s.h);
    dfree(s.h_hi);
    dfree(s.h_lo);
    dfree(s.h_sc);
    dfree(s.y);
    s = PrefillScratch{};
}

// reference-surface shape check (kernels.metal:146-152, metal_bridge.mm:460-461)
bool ref_shape_ok(const SmoeMetalCtx* ctx, uint32_t gate_rows, uint32_t gate_cols, uint32_t down_rows,
                  uint32_t down_cols, uint32_t group_size, uint32_t bits)
{
    if (bits != 4) return false;
    if (group_size == 0 || group_size % 32 != 0 || group_size > 128 || (group_size & (group_size - 1))) return false;
    if (gate_rows != down_cols || gate_cols != down_rows) return false;
    if (gate_cols == 0 || gate_rows == 0) return false;
    if (gate_cols % group_size || gate_rows % group_size) return false;
    if (gate_cols > SMOE_MAX_DIM || gate_rows > SMOE_MAX_DIM) return false;
    if (ctx && (gate_rows > ctx->max_rows || down_rows > ctx->max_rows)) return false;
    return true;
}

bool stream_capturing(hipStream_t s)
{
    hipStreamCaptureStatus st = hipStreamCaptureStatusNone;
    if (hipStreamIsCapturing(s, &st) != hipSuccess) return false;
    return st != hipStreamCaptureStatusNone;
}

int ensure_scratch(SmoeMetalCtx* ctx, const SmoeMoeShape* s, uint32_t T)
{
    DeviceScratch& c = ctx->ds;
    if (c.ll && c.D >= s->d_model && c.E >= s->n_experts && c.K >= s->top_k && c.I >= s->d_ff && c.T >= T)
        return SMOE_OK;
    if (stream_capturing(ctx->stream)) return SMOE_ERR_CAPTURE;
    if (!hip_ok(ctx, hipStreamSynchronize(ctx->stream), "hipStreamSynchronize")) return SMOE_ERR_HIP;
    DeviceScratch n;
    n.D = std::max(c.D, s->d_model);
    n.E = std::max(c.E, s->n_experts);
    n.K = std::max(c.K, s->top_k);
    n.I = std::max(c.I, s->d_ff);
    n.T = std::max(c.T, T);
    free_device_scratch(c);
    const size_t T_ = n.T;
    bool ok = dalloc(ctx, &n.ll, T_ * smoe::ll_token_words(n.E)) && dalloc(ctx, &n.ids, T_ * n.K) &&
              dalloc(ctx, &n.w, T_ * n.K) && dalloc(ctx, &n.tbl, T_ * n.K) && dalloc(ctx, &n.h, T_ * n.K * n.I) &&
              dalloc(ctx, &n.lx, smoe::lx_words(n.D, n.E, n.I));
    // the exchange words start disarmed; every launch pair leaves them so.
    // The one-launch words start at epoch 0 and are never re-armed: a fresh
    // zero word can never carry a live tag (tags start at 1)
    ok = ok && hip_ok(ctx, hipMemset(n.ll, 0, T_ * smoe::ll_token_words(n.E) * sizeof(uint64_t)), "hipMemset") &&
         hip_ok(ctx, hipMemset(n.lx, 0, smoe::lx_words(n.D, n.E, n.I) * sizeof(uint64_t)), "hipMemset");
    if (!ok) {
        free_device_scratch(n);
        return SMOE_ERR_HIP;
    }
    c = n;
    return SMOE_OK;
}

// largest token batch of one prefill pass: the permute's per-(chunk, expert)
// counts live in one workgroup's LDS
uint32_t prefill_max_tokens(uint32_t E, uint32_t K)
{
    uint32_t lo = 1, hi = 1u << 16;
    if (smoe::permute_lds_bytes(K, E) > smoe::PERMUTE_MAX_LDS) return 0;
    while (lo < hi) {
        const uint32_t mid = (lo + hi + 1) / 2;
        if (smoe::permute_lds_bytes(mid * K, E) <= smoe::PERMUTE_MAX_LDS) lo = mid; else hi = mid - 1;
    }
    return lo;
}

int ensure_prefill_scratch(SmoeMetalCtx* ctx, const SmoeMoeShape* s, uint32_t T)
{
    PrefillScratch& c = ctx->ps;
    if (c.x_hi && c.D >= s->d_model && c.E >= s->n_experts && c.K >= s->top_k && c.I >= s->d_ff && c.T >= T)
        return SMOE_OK;
    if (stream_capturing(ctx->stream)) return SMOE_ERR_CAPTURE;
    if (!hip_ok(ctx, hipStreamSynchronize(ctx->stream), "hipStreamSynchronize")) return SMOE_ERR_HIP;
    PrefillScratch n;
    n.D = std::max(c.D, s->d_model);
    n.E = std::max(c.E, s->n_experts);
    n.K = std::max(c.K, s->top_k);
    n.I = std::max(c.I, s->d_ff);
    n.T = std::max(c.T, T);
    free_prefill_scratch(c);
    const size_t T_ = n.T, P = T_ * n.K;
    const bool ok = dalloc(ctx, &n.x_hi, T_ * n.D) &&
                    dalloc(ctx, &n.x_lo, T_ * n.D) && dalloc(ctx, &n.x_sc, T_) &&
                    dalloc(ctx, &n.ids, P) && dalloc(ctx, &n.w, P) && dalloc(ctx, &n.offsets, size_t(n.E) + 1) &&
                    dalloc(ctx, &n.sched, size_t(n.E) + 1) &&
                    dalloc(ctx, &n.pairs, P) && dalloc(ctx, &n.h, P * n.I) && dalloc(ctx, &n.h_hi, P * n.I) &&
                    dalloc(ctx, &n.h_lo, P * n.I) && dalloc(ctx, &n.h_sc, P) && dalloc(ctx, &n.y, P * n.D) &&
                    dalloc(ctx, &n.logits, T_ * n.E) && dalloc(ctx, &n.rt_ctr, T_) &&
                    hip_ok(ctx, hipMemset(n.rt_ctr, 0, T_ * sizeof(uint32_t)), "hipMemset");
    if (!ok) {
        free_prefill_scratch(n);
        return SMOE_ERR_HIP;
    }
    c = n;
    return SMOE_OK;
}

constexpr size_t kProfSlots = 4096;

void prof_flush_slot(SmoeMetalCtx* ctx, SmoeMetalCtx::ProfSlot& p)
{
    if (!p.pending) return;
    float ms = 0.f;
    if (hipEventSynchronize(p.b) == hipSuccess && hipEventElapsedTime(&ms, p.a, p.b) == hipSuccess) {
        ctx->prof_launches[p.kind] += 1;
        ctx->prof_ms[p.kind] += ms;
    }
    p.pending = false;
}

// Time one kernel launch (no-op unless profiling; skipped under stream
// capture): the slot's events are handed to the launcher, which records them
// at the dispatch's own start and end.
void prof_begin(SmoeMetalCtx* ctx, uint32_t kind)
{
    ctx->prof_open = -1;
    if (!ctx->profiling || stream_capturing(ctx->stream)) return;
    const size_t i = ctx->prof_head % kProfSlots;
    auto& p = ctx->prof[i];
    prof_flush_slot(ctx, p);
    p.kind = kind;
    smoe::dispatch_timer() = smoe::DispatchTimer{p.a, p.b};
    ctx->prof_open = static_cast<int>(i);
}

void prof_end(SmoeMetalCtx* ctx)
{
    if (ctx->prof_open < 0) return;
    smoe::dispatch_timer() = smoe::DispatchTimer{};
    ctx->prof[ctx->prof_open].pending = true;
    ctx->prof_head++;
    ctx->prof_open = -1;
}

// launch helper: times the launch when profiling
template <typename F>
bool timed(SmoeMetalCtx* ctx, uint32_t kind, const char* what, F&& launch)
{
    prof_begin(ctx, kind);
    const hipError_t e = launch();
    prof_end(ctx);
    return hip_ok(ctx, e, what);
}

void* record_handle(SmoeMetalCtx* ctx)
{
    const uint64_t h = ++ctx->seq;
    if (!hip_ok(ctx, hipEventRecord(ctx->ev[h % kEvents], ctx->stream), "hipEventRecord")) return nullptr;
    return reinterpret_cast<void*>(static_cast<uintptr_t>(h));
}

bool wait_handle(SmoeMetalCtx* ctx, void* handle)
{
    const uint64_t h = static_cast<uint64_t>(reinterpret_cast<uintptr_t>(handle));
    if (h == 0 || h > ctx->seq) return false;
    // An event older than the ring was re-recorded by later work on the same
    // in-order stream; waiting for that later work also covers `h`.
    return hip_ok(ctx, hipEventSynchronize(ctx->ev[h % kEvents]), "hipEventSynchronize");
}

// one group of same-shaped experts on ctx->d_input (reference surface)
void* dispatch_group(SmoeMetalCtx* ctx, const ExpertPtrs* tbl_host, uint32_t n, const float* input_vec,
                     uint32_t gate_rows, uint32_t gate_cols, uint32_t group_size)
{
    const MoeDims d{gate_cols, 0, n, gate_rows, group_size, 0};
    if (!hip_ok(ctx, hipMemcpyAsync(ctx->d_input, input_vec, gate_cols * sizeof(float), hipMemcpyHostToDevice,
                                    ctx->stream), "hipMemcpyAsync(input)"))
        return nullptr;
    if (!hip_ok(ctx, hipMemcpyAsync(ctx->d_tbl_ref, tbl_host, n * sizeof(ExpertPtrs), hipMemcpyHostToDevice,
                                    ctx->stream), "hipMemcpyAsync(table)"))
        return nullptr;
    if (!timed(ctx, SMOE_KERNEL_GATE_UP, "gate_up", [&] {
            return smoe::launch_gate_up(d, ctx->d_tbl_ref, n, ctx->d_input, ctx->d_hidden, ctx->max_rows, 1, 0, 0, 0,
                                        ctx->stream);
        }))
        return nullptr;
    if (!timed(ctx, SMOE_KERNEL_DOWN_SLOTS, "down", [&] {
            return smoe::launch_down_slots(d, ctx->d_tbl_ref, n, ctx->d_hidden, ctx->max_rows, ctx->d_output,
                                           ctx->max_rows, 1, 0, 0, 0, ctx->stream);
        }))
        return nullptr;
    ctx->dispatches.fetch_add(n, std::memory_order_relaxed);
    return record_handle(ctx);
}

}  // namespace

// ============================================================================
// 1. reference surface
// ============================================================================
extern "C" SmoeMetalCtx* smoe_metal_init(size_t slot_bytes)
{
    int ndev = 0;
    if (hipGetDeviceCount(&ndev) != hipSuccess || ndev == 0) {
        std::fprintf(stderr, "[smoe_hip] ERROR: no HIP device.\n");
        return nullptr;
    }
    SmoeMetalCtx* ctx = new SmoeMetalCtx();
    if (hipGetDevice(&ctx->device) != hipSuccess) ctx->device = 0;
    ctx->slot_bytes = slot_bytes;
    ctx->max_rows = static_cast<uint32_t>(std::min(slot_bytes / sizeof(float), size_t(32768)));
    if (ctx->max_rows < SMOE_MAX_DIM) ctx->max_rows = SMOE_MAX_DIM;
    const size_t plane = size_t(SMOE_MAX_FFN_BATCH) * SMOE_MAX_FFN_BATCH_DIM;
    bool ok = hip_ok(ctx, hipStreamCreateWithFlags(&ctx->own_stream, hipStreamNonBlocking), "hipStreamCreate") &&
              dalloc(ctx, &ctx->d_input, SMOE_MAX_DIM) && dalloc(ctx, &ctx->d_hidden, size_t(kSlots) * ctx->max_rows) &&
              dalloc(ctx, &ctx->d_output, size_t(kSlots) * ctx->max_rows) && dalloc(ctx, &ctx->d_batch_in, plane) &&
              dalloc(ctx, &ctx->d_batch_hidden, plane) && dalloc(ctx, &ctx->d_batch_out, plane) &&
              dalloc(ctx, &ctx->d_tbl_ref, kSlots) && dalloc(ctx, &ctx->d_err, 1) &&
              hip_ok(ctx, hipMemset(ctx->d_err, 0, sizeof(uint32_t)), "hipMemset");
    for (uint32_t i = 0; ok && i < kEvents; ++i)
        ok = hip_ok(ctx, hipEventCreateWithFlags(&ctx->ev[i], hipEventDisableTiming), "hipEventCreate");
    if (!ok) {
        smoe_metal_destroy(ctx);
        return nullptr;
    }
    ctx->stream = ctx->own_stream;
    // the allocation-free decode entry point's per-device scratch (its address
    // and first clearing), here so that later calls need no set-up
    (void)smoe::static_scratch_setup();
    // how the device deals blocks over its XCDs (the one-launch decode kernels need round-robin)
    (void)smoe::deal_probe();
    return ctx;
}

extern "C" void smoe_metal_destroy(SmoeMetalCtx* ctx)
{
    if (!ctx) return;
    (void)hipStreamSynchronize(ctx->stream);
    if (ctx->own_stream && ctx->own_stream != ctx->stream) (void)hipStreamSynchronize(ctx->own_stream);
    free_device_scratch(ctx->ds);
    free_prefill_scratch(ctx->ps);
    dfree(ctx->lt.tbl);
    dfree(ctx->cs.xch);
    dfree(ctx->cs.hcopy);
    dfree(ctx->cs.cnt);
    dfree(ctx->cs.ids);
    dfree(ctx->cs.w);
    dfree(ctx->perm_pairs);
    dfree(ctx->mv_in);
    dfree(ctx->mv_out);
    dfree(ctx->attn_part);
    dfree(ctx->d_err);
    dfree(ctx->d_input);
    dfree(ctx->d_hidden);
    dfree(ctx->d_output);
    dfree(ctx->d_batch_in);
    dfree(ctx->d_batch_hidden);
    dfree(ctx->d_batch_out);
    dfree(ctx->d_tbl_ref);
    for (uint32_t i = 0; i < kEvents; ++i)
        if (ctx->ev[i]) (void)hipEventDestroy(ctx->ev[i]);
    for (auto& p : ctx->prof) {
        if (p.a) (void)hipEventDestroy(p.a);
        if (p.b) (void)hipEventDestroy(p.b);
    }
    if (ctx->own_stream) (void)hipStreamDestroy(ctx->own_stream);
    delete ctx;
}

extern "C" void* smoe_metal_fused_ffn(SmoeMetalCtx* ctx, const uint8_t* packed_gate, const uint16_t* scales_gate,
                                      const uint8_t* packed_up, const uint16_t* scales_up,
                                      const uint8_t* packed_down, const uint16_t* scales_down,
                                      const float* input_vec, float* hidden_vec, float* output_vec,
                                      uint32_t gate_rows, uint32_t gate_cols, uint32_t down_rows,
                                      uint32_t down_cols, uint32_t group_size, uint32_t bits,
                                      uint32_t expert_index)
{
    (void)hidden_vec;
    (void)output_vec;
    if (!ctx || !input_vec || !packed_gate || !scales_gate || !packed_up || !scales_up || !packed_down ||
        !scales_down || expert_index >= kSlots)
        return nullptr;
    if (!ref_shape_ok(ctx, gate_rows, gate_cols, down_rows, down_cols, group_size, bits)) return nullptr;
    ExpertPtrs e{packed_gate, scales_gate, packed_up, scales_up, packed_down, scales_down, expert_index, 0};
    return dispatch_group(ctx, &e, 1, input_vec, gate_rows, gate_cols, group_size);
}

extern "C" void smoe_metal_wait(SmoeMetalCtx* ctx, void* handle, float* output_vec, uint32_t expert_index,
                                uint32_t cols)
{
    if (!ctx || !handle || !output_vec || expert_index >= kSlots || cols > ctx->max_rows) return;
    if (!wait_handle(ctx, handle)) return;
    (void)hip_ok(ctx, hipMemcpy(output_vec, ctx->d_output + size_t(expert_index) * ctx->max_rows,
                                cols * sizeof(float), hipMemcpyDeviceToHost), "hipMemcpy(output)");
}

extern "C" void* smoe_metal_fused_ffn_group(SmoeMetalCtx* ctx, const SmoeExpertBlob* experts, uint32_t n_experts,
                                            const float* input_vec, uint32_t gate_rows, uint32_t gate_cols,
                                            uint32_t down_rows, uint32_t down_cols, uint32_t group_size,
                                            uint32_t bits)
{
    if (!ctx || !experts || !input_vec || n_experts == 0 || n_experts > kSlots) return nullptr;
    if (!ref_shape_ok(ctx, gate_rows, gate_cols, down_rows, down_cols, group_size, bits)) return nullptr;
    ExpertPtrs tbl[kSlots];
    for (uint32_t i = 0; i < n_experts; ++i) {
        const SmoeExpertBlob& b = experts[i];
        if (!b.packed_gate || !b.scales_gate || !b.packed_up || !b.scales_up || !b.packed_down || !b.scales_down ||
            b.slot >= kSlots)
            return nullptr;
        tbl[i] = ExpertPtrs{b.packed_gate, b.scales_gate, b.packed_up, b.scales_up, b.packed_down, b.scales_down,
                            b.slot, 0};
    }
    return dispatch_group(ctx, tbl, n_experts, input_vec, gate_rows, gate_cols, group_size);
}

extern "C" void* smoe_metal_fused_ffn_batch(SmoeMetalCtx* ctx, const uint8_t* packed_gate,
                                            const uint16_t* scales_gate, const uint8_t* packed_up,
                                            const uint16_t* scales_up, const uint8_t* packed_down,
                                            const uint16_t* scales_down, const float* input_mat, uint32_t batch,
                                            uint32_t gate_rows, uint32_t gate_cols, uint32_t down_rows,
                                            uint32_t down_cols, uint32_t group_size, uint32_t bits)
{
    if (!ctx || !input_mat || batch == 0 || batch > SMOE_MAX_FFN_BATCH) return nullptr;
    if (gate_rows > SMOE_MAX_FFN_BATCH_DIM || gate_cols > SMOE_MAX_FFN_BATCH_DIM ||
        down_rows > SMOE_MAX_FFN_BATCH_DIM || down_cols > SMOE_MAX_FFN_BATCH_DIM)
        return nullptr;
    if (!packed_gate || !scales_gate || !packed_up || !scales_up || !packed_down || !scales_down) return nullptr;
    if (!ref_shape_ok(nullptr, gate_rows, gate_cols, down_rows, down_cols, group_size, bits)) return nullptr;
    const MoeDims d{gate_cols, 0, 1, gate_rows, group_size, 0};
    ExpertPtrs e{packed_gate, scales_gate, packed_up, scales_up, packed_down, scales_down, 0, 0};
    if (!hip_ok(ctx, hipMemcpyAsync(ctx->d_batch_in, input_mat, size_t(batch) * gate_cols * sizeof(float),
                                    hipMemcpyHostToDevice, ctx->stream), "hipMemcpyAsync(batch)"))
        return nullptr;
    if (!hip_ok(ctx, hipMemcpyAsync(ctx->d_tbl_ref, &e, sizeof(e), hipMemcpyHostToDevice, ctx->stream),
                "hipMemcpyAsync(table)"))
        return nullptr;
    if (!timed(ctx, SMOE_KERNEL_GATE_UP, "gate_up(batch)", [&] {
            return smoe::launch_gate_up(d, ctx->d_tbl_ref, 1, ctx->d_batch_in, ctx->d_batch_hidden, 0, batch,
                                        gate_cols, 0, gate_rows, ctx->stream);
        }))
        return nullptr;
    if (!timed(ctx, SMOE_KERNEL_DOWN_SLOTS, "down(batch)", [&] {
            return smoe::launch_down_slots(d, ctx->d_tbl_ref, 1, ctx->d_batch_hidden, 0, ctx->d_batch_out, 0, batch,
                                           0, gate_rows, down_rows, ctx->stream);
        }))
        return nullptr;
    ctx->dispatches.fetch_add(1, std::memory_order_relaxed);
    return record_handle(ctx);
}

extern "C" void smoe_metal_wait_ffn_batch(SmoeMetalCtx* ctx, void* handle, float* out_mat, uint32_t batch,
                                          uint32_t cols)
{
    if (!ctx || !handle || !out_mat || batch == 0 || batch > SMOE_MAX_FFN_BATCH || cols > SMOE_MAX_FFN_BATCH_DIM)
        return;
    if (!wait_handle(ctx, handle)) return;
    (void)hip_ok(ctx, hipMemcpy(out_mat, ctx->d_batch_out, size_t(batch) * cols * sizeof(float),
                                hipMemcpyDeviceToHost), "hipMemcpy(batch out)");
}

extern "C" void smoe_metal_register_buffer(SmoeMetalCtx* ctx, const void* ptr, size_t size_in_bytes)
{
    if (!ctx || !ptr || size_in_bytes == 0) return;
    const uintptr_t p = reinterpret_cast<uintptr_t>(ptr);
    for (const auto& r : ctx->registered)
        if (p >= r.first && p + size_in_bytes <= r.first + r.second) return;
    hipPointerAttribute_t attr;
    std::memset(&attr, 0, sizeof(attr));
    if (hipPointerGetAttributes(&attr, ptr) != hipSuccess || attr.type == hipMemoryTypeUnregistered) {
        (void)hipGetLastError();
        std::fprintf(stderr,
                     "[smoe_hip] WARN: register_buffer(%p, %zu): not device or pinned memory; the GPU "
                     "cannot read it (allocate experts with hipMalloc / hipHostMalloc).\n",
                     ptr, size_in_bytes);
        return;
    }
    ctx->registered.emplace_back(p, size_in_bytes);
}

// dense bf16 GEMVs of the reference surface: host vectors in and out
// the grouped GEMV where its layout rules hold, else the plain one-wave-per-row kernel
static hipError_t gemv_or_plain(const uint16_t* w, const float* x, float* y, uint32_t rows, uint32_t cols,
                                hipStream_t st)
{
    if (cols % 8 == 0 && cols <= smoe::GEMV_MAX_COLS && (reinterpret_cast<uintptr_t>(w) & 15) == 0 &&
        (reinterpret_cast<uintptr_t>(x) & 15) == 0) {
        smoe::GemvGroup g{};
        g.w[0] = w;
        g.x[0] = x;
        g.y[0] = y;
        g.rows[0] = rows;
        g.cols[0] = cols;
        g.count = 1;
        return smoe::launch_gemv_bf16(g, st);
    }
    return smoe::launch_matvec_bf16(w, x, y, rows, cols, st);
}

static bool matvec_one(SmoeMetalCtx* ctx, const uint16_t* w, const float* in, float* out, uint32_t rows,
                       uint32_t cols)
{
    if (!w || !in || !out || rows == 0 || cols == 0) return false;
    if (cols > ctx->mv_cap || rows > ctx->mv_cap) {
        dfree(ctx->mv_in);
        dfree(ctx->mv_out);
        ctx->mv_cap = 0;
        const uint32_t cap = std::max(rows, cols);
        if (!dalloc(ctx, &ctx->mv_in, cap) || !dalloc(ctx, &ctx->mv_out, cap)) return false;
        ctx->mv_cap = cap;
    }
    return hip_ok(ctx, hipMemcpyAsync(ctx->mv_in, in, size_t(cols) * sizeof(float), hipMemcpyHostToDevice, ctx->stream),
                  "hipMemcpyAsync") &&
           hip_ok(ctx, gemv_or_plain(w, ctx->mv_in, ctx->mv_out, rows, cols, ctx->stream), "matvec_bf16") &&
           hip_ok(ctx, hipMemcpyAsync(out, ctx->mv_out, size_t(rows) * sizeof(float), hipMemcpyDeviceToHost,
                                      ctx->stream),
                  "hipMemcpyAsync") &&
           hip_ok(ctx, hipStreamSynchronize(ctx->stream), "hipStreamSynchronize");
}

extern "C" void smoe_metal_scout_matvec_bf16(SmoeMetalCtx* ctx, const uint16_t* weight, const float* input_vec,
                                             float* output_vec, uint32_t rows, uint32_t cols)
{
    if (ctx && !matvec_one(ctx, weight, input_vec, output_vec, rows, cols))
        std::fprintf(stderr, "[smoe_hip] scout_matvec_bf16 failed: %s\n", ctx->last_err);
}

extern "C" void smoe_metal_scout_matvec_batch_bf16(SmoeMetalCtx* ctx, const uint16_t** weights, const float** inputs,
                                                   float** outputs, const uint32_t* rows, const uint32_t* cols,
                                                   uint32_t count)
{
    if (!ctx || !weights || !inputs || !outputs || !rows || !cols) return;
    for (uint32_t i = 0; i < count; ++i)
        if (!matvec_one(ctx, weights[i], inputs[i], outputs[i], rows[i], cols[i])) {
            std::fprintf(stderr, "[smoe_hip] scout_matvec_batch_bf16 failed at %u: %s\n", i, ctx->last_err);
            return;
        }
}

extern "C" void smoe_metal_scout_matvec_group_bf16(SmoeMetalCtx* ctx, const uint16_t** weights, const float** inputs,
                                                   float** outputs, const uint32_t* rows, const uint32_t* cols,
                                                   uint32_t count)
{
    smoe_metal_scout_matvec_batch_bf16(ctx, weights, inputs, outputs, rows, cols, count);
}

extern "C" int smoe_hip_matvec_group_bf16(SmoeMetalCtx* ctx, const uint16_t* const* w, const float* const* x,
                                          float* const* y, const uint32_t* rows, const uint32_t* cols, uint32_t count)
{
    if (!ctx || !w || !x || !y || !rows || !cols || count == 0) return SMOE_ERR_ARG;
    for (uint32_t i0 = 0; i0 < count; i0 += smoe::GEMV_MAX) {
        smoe::GemvGroup g{};
        g.count = std::min<uint32_t>(smoe::GEMV_MAX, count - i0);
        for (uint32_t j = 0; j < g.count; ++j) {
            const uint32_t i = i0 + j;
            if (!w[i] || !x[i] || !y[i] || rows[i] == 0 || cols[i] == 0) return SMOE_ERR_ARG;
            if (cols[i] % 8 || cols[i] > smoe::GEMV_MAX_COLS || (reinterpret_cast<uintptr_t>(w[i]) & 15) ||
                (reinterpret_cast<uintptr_t>(x[i]) & 15))
                return SMOE_ERR_SHAPE;
            g.w[j] = w[i];
            g.x[j] = x[i];
            g.y[j] = y[i];
            g.rows[j] = rows[i];
            g.cols[j] = cols[i];
        }
        if (!timed(ctx, SMOE_KERNEL_GEMV, "gemv_bf16", [&] { return smoe::launch_gemv_bf16(g, ctx->stream); }))
            return SMOE_ERR_HIP;
    }
    return SMOE_OK;
}

extern "C" int smoe_hip_matvec_bf16(SmoeMetalCtx* ctx, const uint16_t* w, const float* x, float* y, uint32_t rows,
                                    uint32_t cols)
{
    return smoe_hip_matvec_group_bf16(ctx, &w, &x, &y, &rows, &cols, 1);
}

extern "C" int smoe_hip_attention_layer(SmoeMetalCtx* ctx, const SmoeAttnLayerArgs* a)
{
    if (!ctx || !a) return SMOE_ERR_ARG;
    if (!a->w_q || !a->w_k || !a->w_v || !a->w_o || !a->rope_cos || !a->rope_sin || !a->normed_in || !a->qbuf ||
        !a->kbuf || !a->vbuf || !a->k_cache || !a->v_cache || !a->attn_out || !a->o_out)
        return SMOE_ERR_ARG;
    if ((a->head_dim != 64 && a->head_dim != 128 && a->head_dim != 256) || a->num_heads == 0 ||
        a->num_kv_heads == 0 || a->num_heads % a->num_kv_heads || a->q_dim != a->num_heads * a->head_dim ||
        a->kv_dim != a->num_kv_heads * a->head_dim || a->attn_ctx == 0 || a->slot >= a->attn_ctx ||
        a->valid == 0 || a->valid > a->attn_ctx || a->d_model == 0)
        return SMOE_ERR_SHAPE;
    if ((reinterpret_cast<uintptr_t>(a->k_cache) | reinterpret_cast<uintptr_t>(a->v_cache)) % 16) return SMOE_ERR_ARG;
    const smoe::AttnDims dims{a->head_dim, a->num_heads, a->num_kv_heads, a->kv_dim, a->attn_ctx, a->attn_scale};
    const size_t need = smoe::attn_scratch_bytes(dims);
    if (ctx->attn_part_cap < need) {
        if (stream_capturing(ctx->stream)) return SMOE_ERR_CAPTURE;
        if (!hip_ok(ctx, hipStreamSynchronize(ctx->stream), "hipStreamSynchronize")) return SMOE_ERR_HIP;
        dfree(ctx->attn_part);
        ctx->attn_part_cap = 0;
        if (!dalloc(ctx, &ctx->attn_part, need)) return SMOE_ERR_HIP;
        ctx->attn_part_cap = need;
    }
    // QKV projections in one launch (decode.cpp:151-153)
    const uint16_t* w3[3] = {a->w_q, a->w_k, a->w_v};
    const float* x3[3] = {a->normed_in, a->normed_in, a->normed_in};
    float* y3[3] = {a->qbuf, a->kbuf, a->vbuf};
    const uint32_t r3[3] = {a->q_dim, a->kv_dim, a->kv_dim};
    const uint32_t c3[3] = {a->d_model, a->d_model, a->d_model};
    int rc = smoe_hip_matvec_group_bf16(ctx, w3, x3, y3, r3, c3, 3);
    if (rc != SMOE_OK) return rc;
    if (!timed(ctx, SMOE_KERNEL_ATTENTION, "attention", [&] {
            return smoe::launch_attention(dims, a->qbuf, a->kbuf, a->vbuf, a->q_norm_w, a->k_norm_w, a->rope_cos,
                                          a->rope_sin, a->k_cache, a->v_cache, a->slot, a->valid, ctx->attn_part,
                                          a->attn_out, ctx->stream);
        }))
        return SMOE_ERR_HIP;
    // O projection (decode.cpp:229)
    return smoe_hip_matvec_bf16(ctx, a->w_o, a->attn_out, a->o_out, a->d_model, a->q_dim);
}

extern "C" void smoe_metal_attention_layer(SmoeMetalCtx* ctx, const SmoeAttnLayerArgs* args)
{
    if (!ctx) return;
    const int rc = smoe_hip_attention_layer(ctx, args);
    if (rc != SMOE_OK || !hip_ok(ctx, hipStreamSynchronize(ctx->stream), "hipStreamSynchronize"))
        std::fprintf(stderr, "[smoe_hip] attention_layer failed: %s\n", ctx->last_err);
}

extern "C" uint64_t smoe_metal_kernel_dispatches(const SmoeMetalCtx* ctx)
{
    if (!ctx) return 0;
    return ctx->dispatches.load(std::memory_order_relaxed);
}

// ============================================================================
// 2. device-resident entry points
// ============================================================================
extern "C" int smoe_hip_set_stream(SmoeMetalCtx* ctx, void* hip_stream)
{
    if (!ctx) return SMOE_ERR_ARG;
    ctx->stream = static_cast<hipStream_t>(hip_stream);
    return SMOE_OK;
}

// every decode exchange word of the context back to zero (epochs included),
// synchronously; the stream must be idle
static int rearm_exchange(SmoeMetalCtx* ctx)
{
    DeviceScratch& s = ctx->ds;
    ChainScratch& c = ctx->cs;
    if (s.ll && !hip_ok(ctx, hipMemset(s.ll, 0, size_t(s.T) * smoe::ll_token_words(s.E) * sizeof(uint64_t)),
                        "hipMemset(ll)"))
        return SMOE_ERR_HIP;
    if (s.lx && !hip_ok(ctx, hipMemset(s.lx, 0, smoe::lx_words(s.D, s.E, s.I) * sizeof(uint64_t)), "hipMemset(lx)"))
        return SMOE_ERR_HIP;
    if (c.xch && !hip_ok(ctx, hipMemset(c.xch, 0, c.words * sizeof(uint64_t)), "hipMemset(chain xch)")) return SMOE_ERR_HIP;
    if (c.cnt && !hip_ok(ctx, hipMemset(c.cnt, 0, smoe::chain_cnt_words() * sizeof(uint32_t)), "hipMemset(chain cnt)"))
        return SMOE_ERR_HIP;
    return hip_ok(ctx, hipDeviceSynchronize(), "hipDeviceSynchronize") ? SMOE_OK : SMOE_ERR_HIP;
}

extern "C" int smoe_hip_synchronize(SmoeMetalCtx* ctx)
{
    if (!ctx) return SMOE_ERR_ARG;
    if (!hip_ok(ctx, hipStreamSynchronize(ctx->stream), "hipStreamSynchronize")) return SMOE_ERR_HIP;
    if (ctx->d_err) {
        uint32_t e = 0;
        if (!hip_ok(ctx, hipMemcpy(&e, ctx->d_err, sizeof(e), hipMemcpyDeviceToHost), "hipMemcpy(err)"))
            return SMOE_ERR_HIP;
        if (e) {
            // reported once: clear for the next call
            if (!hip_ok(ctx, hipMemset(ctx->d_err, 0, sizeof(uint32_t)), "hipMemset(err)")) return SMOE_ERR_HIP;
            // After a time-out, waves of the failed launch that started late
            // may have left exchange words tagged for the launches after it:
            // every result since the previous synchronize is suspect, and the
            // exchange words start again from zero.
            if ((e & 1u) && rearm_exchange(ctx) != SMOE_OK) return SMOE_ERR_HIP;
            std::snprintf(ctx->last_err, sizeof(ctx->last_err), "device:%s%s%s (flags %u)",
                          (e & 1u) ? " routing exchange timed out" : "", (e & 2u) ? " expert id out of range" : "",
                          (e & 4u) ? " a stack block ran off its XCD (later calls write exchange words through)"
                                   : "",
                          e);
            return (e & 5u) ? SMOE_ERR_HIP : SMOE_ERR_ARG;
        }
    }
    return SMOE_OK;
}

extern "C" void smoe_hip_exchange_tags(uint32_t epoch, uint32_t n_layers, uint32_t* tags, uint32_t* abort_val,
                                       uint32_t* next_epoch)
{
    for (uint32_t l = 0; tags && l < n_layers; ++l) tags[l] = smoe::tag_at(epoch, l);
    if (abort_val) *abort_val = smoe::tag_at(epoch, 0);
    if (next_epoch) *next_epoch = smoe::epoch_after(epoch, n_layers);
}

extern "C" int smoe_hip_exchange_epoch(SmoeMetalCtx* ctx, const uint32_t* set_chain, const uint32_t* set_layer,
                                       uint32_t* chain, uint32_t* layer)
{
    if (!ctx) return SMOE_ERR_ARG;
    if (stream_capturing(ctx->stream)) return SMOE_ERR_CAPTURE;
    uint64_t* words[2] = {ctx->cs.xch, ctx->ds.lx};
    const uint32_t* set[2] = {set_chain, set_layer};
    uint32_t* get[2] = {chain, layer};
    if (!hip_ok(ctx, hipStreamSynchronize(ctx->stream), "hipStreamSynchronize")) return SMOE_ERR_HIP;
    for (int i = 0; i < 2; ++i) {
        if ((set[i] || get[i]) && !words[i]) return SMOE_ERR_ARG;
        if (set[i]) {
            const uint64_t v = *set[i];
            if (!hip_ok(ctx, hipMemcpy(words[i], &v, sizeof(v), hipMemcpyHostToDevice), "hipMemcpy(epoch)"))
                return SMOE_ERR_HIP;
        }
        if (get[i]) {
            uint64_t v = 0;
            if (!hip_ok(ctx, hipMemcpy(&v, words[i], sizeof(v), hipMemcpyDeviceToHost), "hipMemcpy(epoch)"))
                return SMOE_ERR_HIP;
            *get[i] = static_cast<uint32_t>(v);
        }
    }
    return SMOE_OK;
}

extern "C" int smoe_hip_stream_read(SmoeMetalCtx* ctx, const void* src, uint64_t bytes, uint32_t* sink)
{
    if (!ctx || !src || !sink || bytes < 16 || bytes % 16) return SMOE_ERR_ARG;
    if (!timed(ctx, SMOE_KERNEL_STREAM, "stream_read",
               [&] { return smoe::launch_stream_read(src, bytes, sink, ctx->stream); }))
        return SMOE_ERR_HIP;
    return SMOE_OK;
}

extern "C" int smoe_hip_set_decode_engine(SmoeMetalCtx* ctx, int engine)
{
    if (!ctx || (engine != SMOE_DECODE_LAUNCHES && engine != SMOE_DECODE_SPLIT && engine != SMOE_DECODE_CHAIN))
        return SMOE_ERR_ARG;
    ctx->decode_engine = engine;
    return SMOE_OK;
}

extern "C" int smoe_hip_reserve(SmoeMetalCtx* ctx, const SmoeMoeShape* shape, uint32_t max_tokens)
{
    if (!ctx || !shape || max_tokens == 0) return SMOE_ERR_ARG;
    const int rc = shape_check(shape);
    if (rc != SMOE_OK) return rc;
    return ensure_scratch(ctx, shape, max_tokens);
}

static int moe_forward(SmoeMetalCtx* ctx, const SmoeMoeShape* shape, const SmoeMoeLayer* layer, float* hidden,
                       uint32_t n_tokens, uint32_t* ids_out, float* weights_out)
{
    if (!ctx || !shape || !layer || !hidden || n_tokens == 0) return SMOE_ERR_ARG;
    if (!layer->norm_w || !layer->router_w || !layer->experts) return SMOE_ERR_ARG;
    int rc = shape_check(shape);
    if (rc != SMOE_OK) return rc;
    rc = ensure_scratch(ctx, shape, n_tokens);
    if (rc != SMOE_OK) return rc;
    DeviceScratch& s = ctx->ds;
    const MoeDims d = dims_of(shape);
    const LayerDesc L = layer_of(layer);
    uint32_t* ids = ids_out ? ids_out : s.ids;
    float* w = weights_out ? weights_out : s.w;
    const bool one_launch = n_tokens == 1 && ctx->decode_engine != SMOE_DECODE_SPLIT && smoe::layer_supported(d, L);
    if (d.quant != SMOE_QUANT_SMOEQ4 && !one_launch) {
        std::snprintf(ctx->last_err, sizeof(ctx->last_err),
                      "the scale+min format runs on the one-launch decode kernel only (one token, top_k 8, "
                      "<= 128 experts, d_model <= 2048, not under SMOE_DECODE_SPLIT)");
        return SMOE_ERR_BITS;
    }
    if (one_launch) {
        if (!timed(ctx, SMOE_KERNEL_MOE_LAYER, "moe_layer", [&] {
                return smoe::launch_moe_layer(d, L, hidden, s.lx, ids, w, ctx->d_err, ctx->stream);
            }))
            return SMOE_ERR_HIP;
        ctx->dispatches.fetch_add(d.K, std::memory_order_relaxed);
        return SMOE_OK;
    }
    if (!timed(ctx, SMOE_KERNEL_MOE_UP, "moe_up", [&] {
            return smoe::launch_moe_up(d, L, hidden, n_tokens, s.ll, s.h, ids, w, s.tbl, ctx->d_err, ctx->stream);
        }))
        return SMOE_ERR_HIP;
    if (!timed(ctx, SMOE_KERNEL_MOE_DOWN, "moe_down",
               [&] { return smoe::launch_down_combine(d, s.tbl, s.h, w, hidden, s.ll, n_tokens, ctx->stream); }))
        return SMOE_ERR_HIP;
    ctx->dispatches.fetch_add(uint64_t(n_tokens) * d.K, std::memory_order_relaxed);
    return SMOE_OK;
}

extern "C" int smoe_hip_moe_decode(SmoeMetalCtx* ctx, const SmoeMoeShape* shape, const SmoeMoeLayer* layer,
                                   float* hidden, uint32_t n_tokens, uint32_t* ids_out, float* weights_out)
{
    return moe_forward(ctx, shape, layer, hidden, n_tokens, ids_out, weights_out);
}

static bool same_layer(const LayerDesc& a, const LayerDesc& b)
{
    return std::memcmp(&a, &b, sizeof(LayerDesc)) == 0;
}

// the device copy of the layer table, uploaded when it changes (outside
// capture: under capture a new table gives SMOE_ERR_CAPTURE)
static int upload_table(SmoeMetalCtx* ctx, const SmoeMoeLayer* layers, uint32_t n_layers)
{
    LayerTable& s = ctx->lt;
    bool same = s.tbl && s.host_tbl.size() == n_layers;
    for (uint32_t l = 0; same && l < n_layers; ++l) same = same_layer(s.host_tbl[l], layer_of(&layers[l]));
    if (same) return SMOE_OK;
    if (stream_capturing(ctx->stream)) return SMOE_ERR_CAPTURE;
    std::vector<LayerDesc> t(n_layers);
    for (uint32_t l = 0; l < n_layers; ++l) t[l] = layer_of(&layers[l]);
    // the previous table may still be read by queued work
    if (!hip_ok(ctx, hipStreamSynchronize(ctx->stream), "hipStreamSynchronize")) return SMOE_ERR_HIP;
    if (s.tbl_cap < n_layers) {
        dfree(s.tbl);
        s.tbl_cap = 0;
        if (!dalloc(ctx, &s.tbl, n_layers)) return SMOE_ERR_HIP;
        s.tbl_cap = n_layers;
    }
    if (!hip_ok(ctx, hipMemcpy(s.tbl, t.data(), n_layers * sizeof(LayerDesc), hipMemcpyHostToDevice),
                "hipMemcpy(layer table)"))
        return SMOE_ERR_HIP;
    s.host_tbl = std::move(t);
    return SMOE_OK;
}

// SMOE_DECODE_CHAIN: the whole step in one launch of k_moe_chain
static int decode_chain(SmoeMetalCtx* ctx, const MoeDims& d, const SmoeMoeLayer* layers, uint32_t n_layers,
                        float* hidden, uint32_t* ids_out, float* weights_out)
{
    ChainScratch& c = ctx->cs;
    const size_t words = smoe::chain_xch_words(d.D, d.E, d.I);
    const size_t hn = size_t(8) * d.D, outn = size_t(n_layers) * d.K;
    if (c.words < words || c.hcopy_n < hn || !c.cnt || (!ids_out && c.out_n < outn) || (!weights_out && c.out_n < outn)) {
        if (stream_capturing(ctx->stream)) return SMOE_ERR_CAPTURE;
        if (!hip_ok(ctx, hipStreamSynchronize(ctx->stream), "hipStreamSynchronize")) return SMOE_ERR_HIP;
        if (c.words < words) {
            dfree(c.xch);
            c.words = 0;
            if (!dalloc(ctx, &c.xch, words) ||
                !hip_ok(ctx, hipMemset(c.xch, 0, words * sizeof(uint64_t)), "hipMemset(chain xch)"))
                return SMOE_ERR_HIP;
            c.words = words;
        }
        if (c.hcopy_n < hn) {
            dfree(c.hcopy);
            c.hcopy_n = 0;
            if (!dalloc(ctx, &c.hcopy, hn)) return SMOE_ERR_HIP;
            c.hcopy_n = hn;
        }
        if (!c.cnt && (!dalloc(ctx, &c.cnt, smoe::chain_cnt_words()) ||
                       !hip_ok(ctx, hipMemset(c.cnt, 0, smoe::chain_cnt_words() * sizeof(uint32_t)),
                               "hipMemset(chain counters)")))
            return SMOE_ERR_HIP;
        if (c.out_n < outn) {
            dfree(c.ids);
            dfree(c.w);
            c.out_n = 0;
            if (!dalloc(ctx, &c.ids, outn) || !dalloc(ctx, &c.w, outn)) return SMOE_ERR_HIP;
            c.out_n = outn;
        }
    }
    const int rc = upload_table(ctx, layers, n_layers);
    if (rc != SMOE_OK) return rc;
    if (!timed(ctx, SMOE_KERNEL_CHAIN, "moe_chain", [&] {
            return smoe::launch_moe_chain(d, ctx->lt.tbl, n_layers, hidden, c.xch, c.hcopy, c.cnt,
                                          ids_out ? ids_out : c.ids, weights_out ? weights_out : c.w, ctx->d_err,
                                          ctx->stream);
        }))
        return SMOE_ERR_HIP;
    ctx->dispatches.fetch_add(uint64_t(n_layers) * d.K, std::memory_order_relaxed);
    return SMOE_OK;
}

extern "C" int smoe_hip_moe_decode_stack(SmoeMetalCtx* ctx, const SmoeMoeShape* shape, const SmoeMoeLayer* layers,
                                         uint32_t n_layers, float* hidden, uint32_t* ids_out, float* weights_out)
{
    if (!ctx || !shape || !layers || !hidden || n_layers == 0) return SMOE_ERR_ARG;
    for (uint32_t l = 0; l < n_layers; ++l)
        if (!layers[l].norm_w || !layers[l].router_w || !layers[l].experts) return SMOE_ERR_ARG;
    int rc = shape_check(shape);
    if (rc != SMOE_OK) return rc;
    const MoeDims d = dims_of(shape);
    if (ctx->decode_engine == SMOE_DECODE_CHAIN) {
        std::vector<LayerDesc> host(n_layers);
        for (uint32_t l = 0; l < n_layers; ++l) host[l] = layer_of(&layers[l]);
        if (smoe::chain_supported(d, host.data(), n_layers))
            return decode_chain(ctx, d, layers, n_layers, hidden, ids_out, weights_out);
    }
    // one or two launches per layer
    for (uint32_t l = 0; l < n_layers; ++l) {
        rc = moe_forward(ctx, shape, &layers[l], hidden, 1, ids_out ? ids_out + size_t(l) * d.K : nullptr,
                         weights_out ? weights_out + size_t(l) * d.K : nullptr);
        if (rc != SMOE_OK) return rc;
    }
    return SMOE_OK;
}

extern "C" int smoe_hip_moe_prefill(SmoeMetalCtx* ctx, const SmoeMoeShape* shape, const SmoeMoeLayer* layer,
                                    float* hidden, uint32_t n_tokens, uint32_t* ids_out, float* weights_out,
                                    uint32_t* expert_offsets, uint32_t* sorted_tokens, uint32_t* union_ids,
                                    uint32_t* union_size)
{
    if (!ctx || !shape || !layer || !hidden || n_tokens == 0) return SMOE_ERR_ARG;
    if (!layer->norm_w || !layer->router_w || !layer->experts) return SMOE_ERR_ARG;
    int rc = shape_check(shape);
    if (rc != SMOE_OK) return rc;
    if (shape->quant != SMOE_QUANT_SMOEQ4) return SMOE_ERR_BITS;   // the grouped GEMMs decode SMOE-Q4 only
    const MoeDims d = dims_of(shape);
    const LayerDesc L = layer_of(layer);
    const uint32_t tmax = prefill_max_tokens(d.E, d.K);
    if (tmax == 0) return SMOE_ERR_SHAPE;
    // the permute outputs describe one pass: they need all tokens in one batch
    const bool want_perm = expert_offsets || sorted_tokens || union_ids || union_size;
    if (want_perm && n_tokens > tmax) return SMOE_ERR_SHAPE;
    const uint32_t tb = std::min(n_tokens, tmax);
    rc = ensure_prefill_scratch(ctx, shape, tb);
    if (rc != SMOE_OK) return rc;
    PrefillScratch& s = ctx->ps;
    hipStream_t st = ctx->stream;
    for (uint32_t t0 = 0; t0 < n_tokens; t0 += tb) {
        const uint32_t T = std::min(tb, n_tokens - t0), P = T * d.K;
        float* hv = hidden + size_t(t0) * d.D;
        uint32_t* ids = ids_out ? ids_out + size_t(t0) * d.K : s.ids;
        float* w = weights_out ? weights_out + size_t(t0) * d.K : s.w;
        uint32_t* offs = expert_offsets ? expert_offsets : s.offsets;
        if (!timed(ctx, SMOE_KERNEL_ROUTE, "route",
                   [&] {
                       return smoe::launch_route(d, L, hv, T, s.x_hi, s.x_lo, s.x_sc, ids, w, s.logits, s.rt_ctr, st);
                   }) ||
            !timed(ctx, SMOE_KERNEL_PERMUTE, "permute", [&] {
                return smoe::launch_permute(ids, w, P, d.K, d.E, offs, s.pairs, sorted_tokens, nullptr, union_ids,
                                            union_size, s.sched, ctx->d_err, st);
            }) ||
            !timed(ctx, SMOE_KERNEL_GROUPED_GATE_UP, "grouped_gate_up", [&] {
                return smoe::launch_grouped_gate_up(d, L, offs, s.sched, s.pairs, s.x_hi, s.x_lo, s.x_sc, s.h, st);
            }) ||
            !timed(ctx, SMOE_KERNEL_SPLIT, "split(h)",
                   [&] { return smoe::launch_split_rows(s.h, P, d.I, s.h_hi, s.h_lo, s.h_sc, st); }) ||
            !timed(ctx, SMOE_KERNEL_GROUPED_DOWN, "grouped_down", [&] {
                return smoe::launch_grouped_down(d, L, offs, s.sched, s.pairs, s.h_hi, s.h_lo, s.h_sc, s.y, st);
            }) ||
            !timed(ctx, SMOE_KERNEL_SCATTER, "combine",
                   [&] { return smoe::launch_combine_pairs(s.y, w, T, d.K, d.D, hv, st); }))
            return SMOE_ERR_HIP;
        ctx->dispatches.fetch_add(uint64_t(P), std::memory_order_relaxed);
    }
    return SMOE_OK;
}

extern "C" int smoe_hip_moe_prefill_stack(SmoeMetalCtx* ctx, const SmoeMoeShape* shape,
                                          const SmoeMoeLayer* layers, uint32_t n_layers, float* hidden,
                                          uint32_t n_tokens, uint32_t* ids_out, float* weights_out)
{
    if (!ctx || !shape || !layers || !hidden || n_layers == 0 || n_tokens == 0) return SMOE_ERR_ARG;
    const size_t per_layer = size_t(n_tokens) * shape->top_k;
    for (uint32_t l = 0; l < n_layers; ++l) {
        const int rc = smoe_hip_moe_prefill(ctx, shape, &layers[l], hidden, n_tokens,
                                            ids_out ? ids_out + l * per_layer : nullptr,
                                            weights_out ? weights_out + l * per_layer : nullptr, nullptr, nullptr,
                                            nullptr, nullptr);
        if (rc != SMOE_OK) return rc;
    }
    return SMOE_OK;
}

extern "C" int smoe_hip_compute_top_k(SmoeMetalCtx* ctx, const float* scores, uint32_t n_rows, uint32_t n,
                                      uint32_t k, uint32_t* ids, float* weights, int norm_topk)
{
    if (!ctx || !scores || !ids || !weights || n_rows == 0 || n == 0 || k == 0) return SMOE_ERR_ARG;
    if (n > SMOE_MAX_EXPERTS || k > SMOE_MAX_ACTIVE) return SMOE_ERR_SHAPE;
    return timed(ctx, SMOE_KERNEL_TOPK, "topk",
                 [&] { return smoe::launch_topk(scores, n_rows, n, k, norm_topk ? 1u : 0u, ids, weights, ctx->stream); })
               ? SMOE_OK
               : SMOE_ERR_HIP;
}

extern "C" int smoe_hip_permute(SmoeMetalCtx* ctx, const uint32_t* ids, const float* weights, uint32_t n_tokens,
                                uint32_t top_k, uint32_t n_experts, uint32_t* expert_offsets,
                                uint32_t* sorted_tokens, float* sorted_weights, uint32_t* union_ids,
                                uint32_t* union_size)
{
    if (!ctx || !ids || !expert_offsets || n_tokens == 0 || top_k == 0 || n_experts == 0) return SMOE_ERR_ARG;
    if (sorted_weights && !weights) return SMOE_ERR_ARG;
    if (top_k > SMOE_MAX_ACTIVE || n_experts > SMOE_MAX_EXPERTS) return SMOE_ERR_SHAPE;
    const uint64_t P = uint64_t(n_tokens) * top_k;
    if (P > 0xFFFFFFFFull || smoe::permute_lds_bytes(static_cast<uint32_t>(P), n_experts) > smoe::PERMUTE_MAX_LDS)
        return SMOE_ERR_SHAPE;
    // scratch for the sorted pair ids
    if (!ctx->perm_pairs || ctx->perm_cap < P) {
        if (stream_capturing(ctx->stream)) return SMOE_ERR_CAPTURE;
        if (!hip_ok(ctx, hipStreamSynchronize(ctx->stream), "hipStreamSynchronize")) return SMOE_ERR_HIP;
        dfree(ctx->perm_pairs);
        ctx->perm_cap = 0;
        if (!dalloc(ctx, &ctx->perm_pairs, P)) return SMOE_ERR_HIP;
        ctx->perm_cap = P;
    }
    return timed(ctx, SMOE_KERNEL_PERMUTE, "permute",
                 [&] {
                     return smoe::launch_permute(ids, weights, static_cast<uint32_t>(P), top_k, n_experts,
                                                 expert_offsets, ctx->perm_pairs, sorted_tokens, sorted_weights,
                                                 union_ids, union_size, nullptr, ctx->d_err, ctx->stream);
                 })
               ? SMOE_OK
               : SMOE_ERR_HIP;
}

extern "C" int smoe_hip_quantize_q4(SmoeMetalCtx* ctx, const float* w, uint64_t n, uint32_t group_size,
                                    uint8_t* packed, uint16_t* scales)
{
    if (!ctx || !w || !packed || !scales || n == 0) return SMOE_ERR_ARG;
    if ((group_size != 32 && group_size != 64 && group_size != 128) || n % group_size) return SMOE_ERR_SHAPE;
    return hip_ok(ctx, smoe::launch_quantize_q4(w, n, group_size, packed, scales, ctx->stream), "quantize")
               ? SMOE_OK
               : SMOE_ERR_HIP;
}

extern "C" int smoe_hip_quantize_q4_scale_min(SmoeMetalCtx* ctx, const float* w, uint64_t n, uint32_t group_size,
                                              uint8_t* packed, uint16_t* scales, uint16_t* mins)
{
    if (!ctx || !w || !packed || !scales || !mins || n == 0) return SMOE_ERR_ARG;
    if (group_size != 64 || n % group_size) return SMOE_ERR_SHAPE;
    return hip_ok(ctx, smoe::launch_quantize_q4_min(w, n, group_size, packed, scales, mins, ctx->stream),
                  "quantize_q4_scale_min")
               ? SMOE_OK
               : SMOE_ERR_HIP;
}

extern "C" int smoe_hip_synth_normal(SmoeMetalCtx* ctx, float* out, uint64_t n, uint64_t seed, uint64_t stream,
                                     float stddev)
{
    if (!ctx || !out || n == 0) return SMOE_ERR_ARG;
    return hip_ok(ctx, smoe::launch_synth_normal(out, n, seed, stream, stddev, ctx->stream), "synth_normal")
               ? SMOE_OK
               : SMOE_ERR_HIP;
}

extern "C" int smoe_hip_synth_bf16(SmoeMetalCtx* ctx, uint16_t* out, uint64_t n, uint64_t seed, uint64_t stream,
                                   float stddev)
{
    if (!ctx || !out || n == 0) return SMOE_ERR_ARG;
    return hip_ok(ctx, smoe::launch_synth_bf16(out, n, seed, stream, stddev, ctx->stream), "synth_bf16")
               ? SMOE_OK
               : SMOE_ERR_HIP;
}

extern "C" int smoe_hip_synth_expert_pool(SmoeMetalCtx* ctx, uint8_t* base, uint32_t first_layer,
                                          uint32_t n_layers, uint32_t n_experts, uint64_t expert_stride,
                                          const SmoeMoeShape* shape, uint64_t seed, float stddev)
{
    if (!ctx || !base || !shape || n_layers == 0 || n_experts == 0) return SMOE_ERR_ARG;
    const int rc = shape_check(shape);
    if (rc != SMOE_OK) return rc;
    const uint64_t n = uint64_t(shape->d_model) * shape->d_ff;
    // (scale+min: each matrix's mins follow its scales)
    const uint64_t pb = n / 2, sb = n / shape->group_size * 2 * (shape->quant == SMOE_QUANT_Q4_SCALE_MIN ? 2 : 1);
    const uint64_t off[6] = {0, pb, pb + sb, 2 * pb + sb, 2 * (pb + sb), 3 * pb + 2 * sb};
    if (expert_stride < 3 * (pb + sb) || expert_stride % 16) return SMOE_ERR_SHAPE;
    return hip_ok(ctx, smoe::launch_synth_pool(base, first_layer, n_layers, n_experts, expert_stride,
                                               shape->d_model, shape->d_ff, shape->group_size, off, seed, stddev,
                                               shape->quant, ctx->stream),
                  "synth_pool")
               ? SMOE_OK
               : SMOE_ERR_HIP;
}

extern "C" int smoe_hip_profile_enable(SmoeMetalCtx* ctx, int enable)
{
    if (!ctx) return SMOE_ERR_ARG;
    if (enable && ctx->prof.empty()) {
        ctx->prof.resize(kProfSlots);
        for (auto& p : ctx->prof) {
            if (!hip_ok(ctx, hipEventCreate(&p.a), "hipEventCreate") ||
                !hip_ok(ctx, hipEventCreate(&p.b), "hipEventCreate"))
                return SMOE_ERR_HIP;
        }
    }
    for (auto& p : ctx->prof) p.pending = false;
    ctx->prof_head = 0;
    std::memset(ctx->prof_launches, 0, sizeof(ctx->prof_launches));
    std::memset(ctx->prof_ms, 0, sizeof(ctx->prof_ms));
    ctx->profiling = enable != 0;
    return SMOE_OK;
}

extern "C" int smoe_hip_profile_read(SmoeMetalCtx* ctx, uint32_t kernel, uint64_t* launches, double* total_ms)
{
    if (!ctx || kernel >= SMOE_KERNEL_KINDS || !launches || !total_ms) return SMOE_ERR_ARG;
    for (auto& p : ctx->prof) prof_flush_slot(ctx, p);
    *launches = ctx->prof_launches[kernel];
    *total_ms = ctx->prof_ms[kernel];
    return SMOE_OK;
}

extern "C" const char* smoe_hip_last_error(const SmoeMetalCtx* ctx)
{
    return ctx ? ctx->last_err : "no context";
}
