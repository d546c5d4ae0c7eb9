/*
 * smoe_hip.h -- C ABI of the MI355X (gfx950) MoE compute backend.
 *
 * Drop-in for the FFN part of S-MoE's compute-backend boundary
 * (src/compute/metal_bridge.h in the reference).  Two layers of entry points:
 *
 *  1. The reference's own surface, same names, same argument meaning, same
 *     handle/wait contract (smoe_metal_*).  A caller that linked the Metal
 *     bridge links this library instead.  One difference is forced by the
 *     hardware: expert pointers (packed_*, scales_*) must be device addresses
 *     (HBM-resident expert pool, hipMalloc'd) or hipHostMalloc'd pinned
 *     memory -- the reference wraps unified-memory host pages instead.
 *     Activations stay host pointers, copied in and out as the reference
 *     copies them (metal_bridge.mm:466, :440, :643-644).
 *
 *  2. Device-resident entry points (smoe_hip_*): the whole MoE block of one
 *     layer (RMSNorm, router GEMV, softmax + top-k, fused Q4 expert FFN,
 *     rank-weighted combine, residual) on device pointers, asynchronous on
 *     the context's stream, no host round trip, capturable in a HIP graph.
 *     They return an int status (SMOE_OK or a negative SMOE_ERR_*).
 *
 * All pointers are plain C pointers, all sizes plain integers.  One context
 * is driven by one host thread (the reference's threading contract,
 * metal_bridge.mm:97).
 */
#ifndef SMOE_HIP_H
#define SMOE_HIP_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* status codes of the smoe_hip_* entry points */
#define SMOE_OK            0
#define SMOE_ERR_ARG      -1   /* NULL pointer or zero-sized argument */
#define SMOE_ERR_SHAPE    -2   /* dims not multiples of the group size, k too large, ... */
#define SMOE_ERR_BITS     -3   /* bits != 4 (only SMOE-Q4 is implemented) */
#define SMOE_ERR_HIP      -4   /* a HIP runtime call failed (see smoe_hip_last_error) */
#define SMOE_ERR_CAPACITY -5   /* scratch reserved by smoe_hip_reserve is too small */
#define SMOE_ERR_CAPTURE  -6   /* would allocate while the stream is being captured */
#define SMOE_ERR_VAULT    -7   /* a .smoe vault is malformed or unreadable (smoe_hip_vault_error) */

/* limits (reference: scout.hpp:32 MAX_ACTIVE, metal_bridge.h:134-135) */
#define SMOE_MAX_ACTIVE        16
#define SMOE_MAX_EXPERTS      512
#define SMOE_MAX_DIM         8192
#define SMOE_MAX_FFN_BATCH     64
#define SMOE_MAX_FFN_BATCH_DIM 16384

/* Opaque execution context (reference: metal_bridge.h:35). */
typedef struct SmoeMetalCtx SmoeMetalCtx;

/* ======================================================================== */
/* 1. Reference surface (metal_bridge.h)                                     */
/* ======================================================================== */

/* metal_bridge.h:47 -- select device 0 (or the current device), create a
 * stream, allocate the per-slot scratch sized by slot_bytes.  NULL on failure
 * (no GPU, allocation failure). */
SmoeMetalCtx* smoe_metal_init(size_t slot_bytes);

/* metal_bridge.h:50 -- release everything; NULL-safe. */
void smoe_metal_destroy(SmoeMetalCtx* ctx);

/* metal_bridge.h:74-90 -- one expert: gate+up+SiLU, then down, into the
 * context's scratch region `expert_index`.  hidden_vec and output_vec are
 * accepted for signature compatibility and not written (as in the reference,
 * metal_bridge.mm:304-432): fetch the result with smoe_metal_wait.  Returns a
 * handle, or NULL on invalid arguments. */
void* smoe_metal_fused_ffn(SmoeMetalCtx* ctx,
                           const uint8_t* packed_gate, const uint16_t* scales_gate,
                           const uint8_t* packed_up, const uint16_t* scales_up,
                           const uint8_t* packed_down, const uint16_t* scales_down,
                           const float* input_vec, float* hidden_vec, float* output_vec,
                           uint32_t gate_rows, uint32_t gate_cols,
                           uint32_t down_rows, uint32_t down_cols,
                           uint32_t group_size, uint32_t bits, uint32_t expert_index);

/* metal_bridge.h:92 -- wait for `handle`, copy `cols` floats of scratch region
 * `expert_index` into output_vec (host).  NULL ctx or handle: no-op. */
void smoe_metal_wait(SmoeMetalCtx* ctx, void* handle, float* output_vec,
                     uint32_t expert_index, uint32_t cols);

/* metal_bridge.h:106-114 */
typedef struct {
    const uint8_t*  packed_gate;
    const uint16_t* scales_gate;
    const uint8_t*  packed_up;
    const uint16_t* scales_up;
    const uint8_t*  packed_down;
    const uint16_t* scales_down;
    uint32_t        slot;
} SmoeExpertBlob;

/* metal_bridge.h:116-125 -- n same-shaped experts on one input vector, all
 * gate/up work then all down work, one handle for the group; each expert's
 * result lands in scratch region experts[i].slot.  NULL if n_experts is 0 or
 * above SMOE_MAX_ACTIVE, or a slot is out of range. */
void* smoe_metal_fused_ffn_group(SmoeMetalCtx* ctx, const SmoeExpertBlob* experts,
                                 uint32_t n_experts, const float* input_vec,
                                 uint32_t gate_rows, uint32_t gate_cols,
                                 uint32_t down_rows, uint32_t down_cols,
                                 uint32_t group_size, uint32_t bits);

/* metal_bridge.h:137-151 -- one expert applied to `batch` token rows
 * (input_mat row-major [batch x gate_cols]).  NULL when batch is 0 or above
 * SMOE_MAX_FFN_BATCH or a dim exceeds SMOE_MAX_FFN_BATCH_DIM (the caller falls
 * back to the per-token path, prefill.cpp:386-405). */
void* smoe_metal_fused_ffn_batch(SmoeMetalCtx* ctx,
                                 const uint8_t* packed_gate, const uint16_t* scales_gate,
                                 const uint8_t* packed_up, const uint16_t* scales_up,
                                 const uint8_t* packed_down, const uint16_t* scales_down,
                                 const float* input_mat, uint32_t batch,
                                 uint32_t gate_rows, uint32_t gate_cols,
                                 uint32_t down_rows, uint32_t down_cols,
                                 uint32_t group_size, uint32_t bits);

/* metal_bridge.h:153-154 -- wait, copy out_mat [batch x cols] (host). */
void smoe_metal_wait_ffn_batch(SmoeMetalCtx* ctx, void* handle, float* out_mat,
                               uint32_t batch, uint32_t cols);

/* metal_bridge.h:221 -- the reference wraps host pages for the GPU.  Here it
 * records the range when it is device or pinned memory the GPU can read, and
 * warns on stderr otherwise (host pages cannot be mapped after the fact). */
void smoe_metal_register_buffer(SmoeMetalCtx* ctx, const void* ptr, size_t size_in_bytes);

/* metal_bridge.h:224 -- number of expert-FFN kernel dispatches submitted. */
uint64_t smoe_metal_kernel_dispatches(const SmoeMetalCtx* ctx);

/* Dense-trunk symbols that decode.cpp / prefill.cpp also link (outside the MoE
 * hot path).  metal_bridge.h:157-161 -- output_vec[rows] = weight[rows x cols]
 * (bf16) . input_vec[cols]; weight is device memory, input_vec / output_vec
 * are host vectors; synchronous, like the reference. */
void smoe_metal_scout_matvec_bf16(SmoeMetalCtx* ctx, const uint16_t* weight,
                                  const float* input_vec, float* output_vec,
                                  uint32_t rows, uint32_t cols);
/* metal_bridge.h:198-204 / :210-216 -- count such products, one sync. */
void smoe_metal_scout_matvec_batch_bf16(SmoeMetalCtx* ctx, const uint16_t** weights,
                                        const float** inputs, float** outputs,
                                        const uint32_t* rows, const uint32_t* cols,
                                        uint32_t count);
void smoe_metal_scout_matvec_group_bf16(SmoeMetalCtx* ctx, const uint16_t** weights,
                                        const float** inputs, float** outputs,
                                        const uint32_t* rows, const uint32_t* cols,
                                        uint32_t count);

/* metal_bridge.h:166-196 -- fused decode attention of one token: QKV
 * projections, per-head QK RMSNorm + RoPE + KV ring append, GQA attention over
 * `valid` positions counted back from `slot`, O projection
 * (decode.cpp:150-229; kernels.metal:421-652).  As on the reference, the call
 * is synchronous: o_out is valid on return.  Every pointer is a device
 * address (weights and the KV ring resident in HBM, like the experts); see
 * smoe_hip_attention_layer for the asynchronous form. */
typedef struct {
    const uint16_t* w_q;
    const uint16_t* w_k;
    const uint16_t* w_v;
    const uint16_t* w_o;
    const uint16_t* q_norm_w;
    const uint16_t* k_norm_w;
    const float*    rope_cos;
    const float*    rope_sin;
    const float*    normed_in;
    float*          qbuf;
    float*          kbuf;
    float*          vbuf;
    float*          k_cache;
    float*          v_cache;
    float*          attn_out;
    float*          o_out;
    uint32_t d_model, q_dim, kv_dim, head_dim, num_heads, num_kv_heads;
    uint32_t slot;
    uint32_t valid;
    uint32_t attn_ctx;
    float    attn_scale;
} SmoeAttnLayerArgs;
void smoe_metal_attention_layer(SmoeMetalCtx* ctx, const SmoeAttnLayerArgs* args);

/* ======================================================================== */
/* 2. Device-resident MoE block (MI355X path)                                */
/* ======================================================================== */

/* Shape of one MoE layer (reference: SmoeModelConfig, common.hpp:118-142). */
typedef struct {
    uint32_t d_model;     /* hidden size D            (2048 / 4096) */
    uint32_t n_experts;   /* experts per layer E      (128)         */
    uint32_t top_k;       /* routed experts per token (8), <= 16    */
    uint32_t d_ff;        /* expert intermediate I    (768 / 1536)  */
    uint32_t group_size;  /* SMOE quant group: must be 64 (vault format) */
    uint32_t bits;        /* must be 4                              */
    uint32_t norm_topk;   /* renormalise the k weights (Qwen3: 1)   */
    uint32_t quant;       /* SMOE_QUANT_*: the 4-bit group format   */
} SmoeMoeShape;

/* 4-bit group formats of the expert matrices (groups of group_size
 * consecutive weights of a row-major matrix, two codes a byte, low nibble =
 * even index).
 *   SMOE_QUANT_SMOEQ4: the vault's format (quantize_smoeq4, shatter_moe.py:
 *     331-387; kernels.metal:90-105): one fp16 absmax scale s per group,
 *     w = (code - 7.5) / 7.5 * s.  Each matrix is [packed][scales].
 *   SMOE_QUANT_Q4_SCALE_MIN: one bf16 scale s and one bf16 min m per group,
 *     w = code * s + m (no counterpart in the reference: the format the
 *     benchmark configurations name).  Each matrix is [packed][scales][mins]:
 *     the mins follow the scales of the same matrix, so the layer's six
 *     offsets (SmoeMoeLayer) still describe a blob.  Quantizer
 *     (smoe_hip_quantize_q4_scale_min): m = bf16(min w), s = bf16((max w -
 *     min w) / 15) (1 when that is 0), code = clamp(rint((w - m) / s), 0, 15)
 *     with the rounded s and m, ties to even.  Runs on the one-launch decode
 *     kernels (top_k 8, up to 128 experts, d_model <= 2048: Qwen3-30B-A3B);
 *     other decode shapes, SMOE_DECODE_SPLIT and prefill return
 *     SMOE_ERR_BITS for it. */
#define SMOE_QUANT_SMOEQ4        0
#define SMOE_QUANT_Q4_SCALE_MIN  1

/* Weights of one MoE layer, all device pointers.  Expert e's blob starts at
 * experts + e * expert_stride and holds the six tensors at the offsets of the
 * vault's TensorDescriptors (ExpertLayout, prefill.hpp:38-53;
 * build_expert_blob, shatter_moe.py:627-674). */
typedef struct {
    const uint16_t* norm_w;     /* [d_model] bf16 post-attention norm weight */
    const uint16_t* router_w;   /* [n_experts x d_model] bf16 (mlp.gate.weight) */
    const uint8_t*  experts;    /* blob of expert 0 of this layer */
    uint64_t        expert_stride;
    uint64_t gate_packed_offset, gate_scales_offset;
    uint64_t up_packed_offset,   up_scales_offset;
    uint64_t down_packed_offset, down_scales_offset;
} SmoeMoeLayer;

/* Use `hip_stream` (a hipStream_t, NULL = the null stream) for all later work
 * of this context.  Until it is called, the context uses a non-blocking stream
 * of its own.  No synchronisation is implied. */
int smoe_hip_set_stream(SmoeMetalCtx* ctx, void* hip_stream);

/* Synchronise the context's stream and report the device-side error flags
 * raised since the last call, then clear them: a timed-out routing exchange
 * inside smoe_hip_moe_decode / smoe_hip_moe_decode_stack (SMOE_ERR_HIP) or an
 * expert id >= n_experts given to smoe_hip_permute (SMOE_ERR_ARG).  After a
 * time-out every decode result since the previous call is suspect (waves of
 * the failed launch may have published words tagged for later launches), so
 * the call also clears the context's decode exchange words (epochs included)
 * before it returns; the error itself only arises when a grid the host found
 * co-resident is not. */
int smoe_hip_synchronize(SmoeMetalCtx* ctx);

/* Tags of the exchange words of the one-launch decode kernels (no
 * counterpart in the reference; for tests and diagnostics).  For a launch of
 * n_layers layers that reads `epoch` from its epoch word: tags[l] for layer l
 * (tags may be NULL), the abort value of its bounded waits, and the epoch it
 * leaves behind.  Tags lie in 1 .. 2^32 - 1 and wrap from 2^32 - 1 to 1, so
 * no tag is 0 and no two consecutive layers (within a launch or across
 * launches) share one. */
void smoe_hip_exchange_tags(uint32_t epoch, uint32_t n_layers, uint32_t* tags, uint32_t* abort_val,
                            uint32_t* next_epoch);

/* Read (chain / layer non-NULL) or set (set_chain / set_layer non-NULL) the
 * epoch word of the chained decode kernel's exchange words and of the
 * one-launch layer kernel's (no counterpart in the reference; for tests that
 * walk the tags across their wrap).  Synchronous, outside graph capture;
 * SMOE_ERR_ARG if the words asked for are not allocated yet (they are after
 * the first call of that kernel). */
int smoe_hip_exchange_epoch(SmoeMetalCtx* ctx, const uint32_t* set_chain, const uint32_t* set_layer,
                            uint32_t* chain, uint32_t* layer);

/* Reserve device scratch for layers of this shape and up to max_tokens tokens
 * per call.  Entry points reserve on demand when the stream is not being
 * captured; under graph capture they fail with SMOE_ERR_CAPTURE instead. */
int smoe_hip_reserve(SmoeMetalCtx* ctx, const SmoeMoeShape* shape, uint32_t max_tokens);

/* Decode MoE block (decode.cpp:236-509): for each of n_tokens rows of hidden
 * [n_tokens x d_model] (device, updated in place):
 *   normed = rms_norm_bf16(hidden, norm_w)          common.hpp:245-256
 *   logits = router_w . normed                      common.hpp:293-306
 *   ids, w = top_k(softmax(logits)), renormalised   scout.cpp:77-123, decode.cpp:290-302
 *   hidden += sum_r w_r * FFN_{ids_r}(normed)       kernels.metal:308-365, decode.cpp:482-509
 * ids_out [n_tokens x top_k] and weights_out [n_tokens x top_k] are optional
 * device pointers.  Asynchronous on the context stream.  One token with
 * top_k = 8 (one selected expert per XCD of the MI355X) runs as a single
 * kernel launch (SMOE_KERNEL_MOE_LAYER) when the shape's grid fits on the
 * device at once; other calls, and every call under SMOE_DECODE_SPLIT, run
 * two launches (SMOE_KERNEL_MOE_UP, SMOE_KERNEL_MOE_DOWN).  The two forms
 * select the same experts and agree up to fp32 summation order. */
int smoe_hip_moe_decode(SmoeMetalCtx* ctx, const SmoeMoeShape* shape,
                        const SmoeMoeLayer* layer, float* hidden, uint32_t n_tokens,
                        uint32_t* ids_out, float* weights_out);

/* One batch-1 decode step through a stack of MoE layers: the layer loop of
 * decode.cpp:121 over the block above, hidden [d_model] (device, in place)
 *   for l in 0 .. n_layers-1:  hidden += MoE_l(RMSNorm_l(hidden))
 * with layers [n_layers] a host array of layer descriptors (all of one shape).
 * ids_out / weights_out [n_layers x top_k] are optional device outputs (rank
 * order, renormalised, decode.cpp:285-307).  Engines
 * (smoe_hip_set_decode_engine):
 *   SMOE_DECODE_LAUNCHES: exactly n_layers smoe_hip_moe_decode
 *     calls (one or two launches per layer, as that entry point chooses).
 *   SMOE_DECODE_SPLIT: the same calls, always two launches per layer.
 *   SMOE_DECODE_CHAIN (default): the whole step in one launch that runs, layer after
 *     layer, the single-launch layer kernel's schedule (one top-k rank per
 *     XCD); every XCD combines all rows into its own copy of the next
 *     layer's input, so layer l + 1 starts inside the launch as soon as its
 *     XCD's copy is complete, with its router rows already requested.
 *     Results equal the per-layer calls bit for bit.  Shapes: those of the
 *     single-launch layer kernel whose registers allow a whole grid at once
 *     (both Qwen3 shapes); others take the launches.  Its layer table is
 *     copied to the device when it differs from the previous call's (outside
 *     graph capture; under capture a new table gives SMOE_ERR_CAPTURE). */
int smoe_hip_moe_decode_stack(SmoeMetalCtx* ctx, const SmoeMoeShape* shape,
                              const SmoeMoeLayer* layers, uint32_t n_layers, float* hidden,
                              uint32_t* ids_out, float* weights_out);

#define SMOE_DECODE_LAUNCHES   0
#define SMOE_DECODE_SPLIT      2
#define SMOE_DECODE_CHAIN      4
/* Select the engine of smoe_hip_moe_decode_stack (and, for SMOE_DECODE_SPLIT,
 * the form of smoe_hip_moe_decode) for this context. */
int smoe_hip_set_decode_engine(SmoeMetalCtx* ctx, int engine);

/* Prefill MoE block (prefill.cpp:308-453) over n_tokens rows [n_tokens x
 * d_model]: per token RMSNorm + router + top-k, then the layer-major expert
 * grouping (token-by-expert permute, grouped expert GEMMs on MFMA, weighted
 * combine into the residual).  Tokens are processed in passes of as many as
 * one permute workgroup holds (736 at 128 experts x top-8); results do not
 * depend on the pass size.  ids_out / weights_out [n_tokens x top_k] are
 * optional.  Optional device outputs of the permute (these require all tokens
 * in one pass, else SMOE_ERR_SHAPE):
 *   expert_offsets [n_experts+1], sorted_tokens [n_tokens*top_k],
 *   union_ids [n_experts] (first-appearance order, prefill.cpp:55-68),
 *   union_size [1]. */
int smoe_hip_moe_prefill(SmoeMetalCtx* ctx, const SmoeMoeShape* shape,
                         const SmoeMoeLayer* layer, float* hidden, uint32_t n_tokens,
                         uint32_t* ids_out, float* weights_out,
                         uint32_t* expert_offsets, uint32_t* sorted_tokens,
                         uint32_t* union_ids, uint32_t* union_size);


/* The prefill layer loop (prefill.cpp:125-453, attention aside) over a stack
 * of MoE layers, each over the whole prompt:
 *   for l in 0 .. n_layers-1:  hidden [n_tokens x d_model] += MoE_l(RMSNorm_l(hidden))
 * exactly n_layers smoe_hip_moe_prefill calls.  The reference walks the
 * prompt in chunks of 64 tokens inside every layer (prefill.hpp:33); tokens
 * are independent inside the MoE block, so a layer over all tokens gives the
 * same results and streams each touched expert's weights once per pass of up
 * to 736 tokens instead of once per chunk.  ids_out / weights_out
 * [n_layers x n_tokens x top_k] are optional. */
int smoe_hip_moe_prefill_stack(SmoeMetalCtx* ctx, const SmoeMoeShape* shape,
                               const SmoeMoeLayer* layers, uint32_t n_layers, float* hidden,
                               uint32_t n_tokens, uint32_t* ids_out, float* weights_out);

/* Scout::compute_top_k (scout.cpp:718-720 -> top_k :77-123) on device:
 * scores [n_rows x n] -> ids [n_rows x k], weights [n_rows x k]. */
int smoe_hip_compute_top_k(SmoeMetalCtx* ctx, const float* scores, uint32_t n_rows,
                           uint32_t n, uint32_t k, uint32_t* ids, float* weights,
                           int norm_topk);

/* Token-by-expert permute (prefill.cpp:38-68, :315-332) of ids [n_tokens x
 * top_k] on device: stable counting sort of (token, rank) pairs by expert, in
 * one workgroup (n_tokens*top_k up to ~5900 pairs at 128 experts; larger
 * inputs return SMOE_ERR_SHAPE).  expert_offsets [n_experts+1] (required);
 * sorted_tokens / sorted_weights [n_tokens*top_k] (ascending token order
 * inside each expert); union_ids [n_experts] in order of first appearance;
 * union_size [1] -- all optional.  Ids >= n_experts are skipped and reported
 * by the next smoe_hip_synchronize. */
int smoe_hip_permute(SmoeMetalCtx* ctx, const uint32_t* ids, const float* weights,
                     uint32_t n_tokens, uint32_t top_k, uint32_t n_experts,
                     uint32_t* expert_offsets, uint32_t* sorted_tokens,
                     float* sorted_weights, uint32_t* union_ids, uint32_t* union_size);

/* quantize_smoeq4 (shatter_moe.py:331-368) on device: w [n] fp32 ->
 * packed [n/2] (low nibble = even index), scales [n/group_size] fp16 bits.
 * n must be a multiple of group_size. */
int smoe_hip_quantize_q4(SmoeMetalCtx* ctx, const float* w, uint64_t n,
                         uint32_t group_size, uint8_t* packed, uint16_t* scales);

/* The SMOE_QUANT_Q4_SCALE_MIN quantizer (above) on device: w [n] fp32 ->
 * packed [n/2], scales [n/group_size] and mins [n/group_size] bf16 bits.  No
 * counterpart in the reference. */
int smoe_hip_quantize_q4_scale_min(SmoeMetalCtx* ctx, const float* w, uint64_t n, uint32_t group_size,
                                   uint8_t* packed, uint16_t* scales, uint16_t* mins);

/* ---- synthetic inputs (counter-based RNG, reproducible on the host) ----- */
/* out[i] = stddev * N(0,1)(key(seed, stream), i) */
int smoe_hip_synth_normal(SmoeMetalCtx* ctx, float* out, uint64_t n, uint64_t seed,
                          uint64_t stream, float stddev);
/* bf16 round-to-nearest-even of the same draw */
int smoe_hip_synth_bf16(SmoeMetalCtx* ctx, uint16_t* out, uint64_t n, uint64_t seed,
                        uint64_t stream, float stddev);
/* n_layers x n_experts expert blobs at base + (l*n_experts + e)*expert_stride:
 * each of gate [d_ff x d_model], up, down [d_model x d_ff] drawn
 * N(0, stddev) from stream (first_layer+l)<<32 | e<<4 | m (m = 0 gate, 1 up,
 * 2 down) and quantized to the shape's format (SMOE-Q4 in the
 * build_expert_blob layout, or scale+min with each matrix's mins after its
 * scales). */
int smoe_hip_synth_expert_pool(SmoeMetalCtx* ctx, uint8_t* base, uint32_t first_layer,
                               uint32_t n_layers, uint32_t n_experts,
                               uint64_t expert_stride, const SmoeMoeShape* shape,
                               uint64_t seed, float stddev);


/* ---- dense trunk, device-resident (MI355X path) ---------------------------
 * y [rows] = W [rows x cols] bf16 . x [cols] fp32 (common.hpp:293-306), all
 * device pointers, asynchronous on the context stream.  cols % 8 == 0,
 * cols <= 16384, W and x 16-byte aligned.  The group form runs `count`
 * independent products in one launch (host arrays of device pointers;
 * metal_bridge.h:210-216). */
int smoe_hip_matvec_bf16(SmoeMetalCtx* ctx, const uint16_t* w, const float* x, float* y,
                         uint32_t rows, uint32_t cols);
int smoe_hip_matvec_group_bf16(SmoeMetalCtx* ctx, const uint16_t* const* w, const float* const* x,
                               float* const* y, const uint32_t* rows, const uint32_t* cols,
                               uint32_t count);
/* smoe_metal_attention_layer without the final synchronisation: the result
 * lands in args->o_out in stream order.  head_dim a multiple of 64 up to 256,
 * num_heads a multiple of num_kv_heads, q_dim = num_heads * head_dim,
 * kv_dim = num_kv_heads * head_dim, slot < attn_ctx, 1 <= valid <= attn_ctx.
 * q_norm_w / k_norm_w NULL skip the QK norm.  Scratch for the context splits
 * grows outside graph capture (else SMOE_ERR_CAPTURE). */
int smoe_hip_attention_layer(SmoeMetalCtx* ctx, const SmoeAttnLayerArgs* args);

/* ---- .smoe vault -> HBM-resident expert pool ---------------------------
 * Replaces the reference's expert streamer for this path
 * (src/io/streamer.cpp parse_vault:183-212, main.cpp read_vault_header:96-157,
 * read_expert_layout:167-198): the vault is parsed and checked once, every
 * expert's table entry and three tensor descriptors against one common
 * layout (the reference reads expert 0's descriptors only), and all blobs are
 * copied into one device pool at pool + (m * E + e) * stride for the m-th MoE
 * layer (ascending layer id) -- the layout smoe_hip_moe_decode and
 * smoe_hip_moe_prefill take through SmoeMoeLayer.  Format: common.hpp:57-181.
 * Host-side parsing needs no GPU; failures return SMOE_ERR_VAULT (or
 * SMOE_ERR_BITS / SMOE_ERR_SHAPE / SMOE_ERR_ARG) and smoe_hip_vault_error()
 * describes the last one of the calling thread. */
typedef struct SmoeVault SmoeVault;

typedef struct {
    uint32_t version, num_moe_layers, experts_per_layer, total_experts;
    uint32_t group_size, bits, d_model, d_ff, vocab_size, ffn_dim;
    uint64_t blob_bytes;            /* raw bytes of one expert blob */
    uint64_t stride;                /* page-padded blob size = pool stride */
    uint64_t gate_packed_offset, gate_scales_offset;
    uint64_t up_packed_offset,   up_scales_offset;
    uint64_t down_packed_offset, down_scales_offset;
    /* the v2 arch block (SmoeArchBlock, common.hpp:88-106) when arch_valid */
    uint32_t arch_valid, arch_flags, num_heads, num_kv_heads, head_dim;
    uint32_t moe_top_k, moe_ffn_dim, dense_ffn_dim, shared_expert_ffn_dim, num_hidden_layers;
    float    rope_theta, rms_norm_eps;
    char     model_type[24];
} SmoeVaultInfo;

int smoe_hip_vault_open(const char* path, SmoeVault** out);
void smoe_hip_vault_close(SmoeVault* vault);
int smoe_hip_vault_info(const SmoeVault* vault, SmoeVaultInfo* info);
/* transformer layer id of the moe_index-th MoE layer */
int smoe_hip_vault_layer_id(const SmoeVault* vault, uint32_t moe_index, uint32_t* layer_id);
/* expert pointer, stride and blob offsets of MoE layer moe_index inside a pool
 * loaded by smoe_hip_vault_load (norm_w and router_w are left as they are:
 * they live in the Scout file, not in the vault) */
int smoe_hip_vault_layer(const SmoeVault* vault, uint32_t moe_index, const void* dev_pool, SmoeMoeLayer* layer);
/* copy every blob into dev_pool (>= num_moe_layers * experts_per_layer *
 * stride bytes) through pinned staging, on hip_stream (NULL = null stream);
 * returns when the copies are done */
int smoe_hip_vault_load(const SmoeVault* vault, void* dev_pool, uint64_t pool_bytes, void* hip_stream);
const char* smoe_hip_vault_error(void);

/* ---- allocation-free single-token decode ----------------------------------
 * No counterpart in the reference: for callers that cannot allocate device
 * memory (code under HIP graph capture, tight serving loops, harnesses that
 * forbid hipMalloc).  The same computation and kernels as
 * smoe_hip_moe_decode with n_tokens = 1 (bit-identical results), with no
 * context: every buffer the kernels need beyond the caller's is a fixed
 * file-scope device array in the library (about 0.6 MB per GPU, held until
 * the process ends), so the call allocates nothing and can be captured.
 *   - shape limits: d_model <= 4096, d_ff <= 2048, n_experts <= 512,
 *     top_k <= 16; larger shapes return SMOE_ERR_CAPACITY (message on stderr);
 *   - set-up: smoe_metal_init sets the array up on its device; otherwise the
 *     first call on a device must run outside stream capture
 *     (SMOE_ERR_CAPTURE if not);
 *   - hidden [d_model] fp32, device, updated in place; ids_out / weights_out
 *     [top_k] and err_out [1] are optional device pointers (NULL: the
 *     scratch's own); err_out receives the device-side flags OR-ed in
 *     (bit 0: an exchange timed out);
 *   - all calls on one GPU share its array: calls that overlap on one GPU
 *     (e.g. on two streams without ordering) race.  Sequential calls are safe;
 *     the array keeps the last call's contents. */
int smoe_hip_moe_decode_static(const SmoeMoeShape* shape, const SmoeMoeLayer* layer, float* hidden,
                               uint32_t* ids_out, float* weights_out, uint32_t* err_out, void* hip_stream);

/* ---- per-kernel timing (telemetry; cf. the reference's --instrument buckets,
 * decode.hpp:36-74, and smoe_metal_kernel_dispatches) ------------------------
 * When enabled, every kernel the context launches outside graph capture is
 * bracketed by HIP events on the stream it runs on; profile_read returns the
 * launch count and summed event time of one kernel kind. */
#define SMOE_KERNEL_MOE_UP        0   /* RMSNorm + router + top-k + gate/up GEMV + SiLU */
#define SMOE_KERNEL_GATE_UP       1   /* gate/up GEMV + SiLU (reference surface)        */
#define SMOE_KERNEL_MOE_DOWN      2   /* down GEMV + weighted combine + residual        */
#define SMOE_KERNEL_DOWN_SLOTS    3   /* down GEMV, per-slot outputs          */
#define SMOE_KERNEL_TOPK          4
#define SMOE_KERNEL_PERMUTE       5
#define SMOE_KERNEL_GROUPED_GATE_UP 6
#define SMOE_KERNEL_GROUPED_DOWN  7
#define SMOE_KERNEL_SCATTER       8   /* prefill: weighted combine of pair outputs + residual */
#define SMOE_KERNEL_ROUTE         9   /* prefill: RMSNorm + router + top-k per token          */
#define SMOE_KERNEL_SPLIT        10   /* prefill: f16 hi/lo planes of activations             */
#define SMOE_KERNEL_MOE_LAYER    12   /* decode: the whole MoE block of one token in one launch */
#define SMOE_KERNEL_GEMV         13   /* dense trunk: grouped bf16 GEMV                          */
#define SMOE_KERNEL_ATTENTION    14   /* dense trunk: QK norm/RoPE/KV append + decode attention   */
#define SMOE_KERNEL_STREAM       15   /* measurement: streaming-read ceiling (smoe_hip_stream_read) */
#define SMOE_KERNEL_CHAIN        17 /* decode: every layer in one launch, the one-launch layer's schedule per layer */
#define SMOE_KERNEL_KINDS        20
int smoe_hip_profile_enable(SmoeMetalCtx* ctx, int enable);
int smoe_hip_profile_read(SmoeMetalCtx* ctx, uint32_t kernel, uint64_t* launches, double* total_ms);

/* Measurement only (no counterpart in the reference): reads `bytes` (a
 * multiple of 16) of device memory at `src` with non-temporal 128-bit loads
 * in one launch on the context's stream and XORs a fold of them into the
 * device word *sink.  Timed like the other kernels, it gives the streaming
 * ceiling that decode rooflines are quoted against beside the datasheet
 * peak. */
int smoe_hip_stream_read(SmoeMetalCtx* ctx, const void* src, uint64_t bytes, uint32_t* sink);

/* last HIP error string seen by this context ("" if none) */
const char* smoe_hip_last_error(const SmoeMetalCtx* ctx);

#ifdef __cplusplus
}
#endif
#endif /* SMOE_HIP_H */
