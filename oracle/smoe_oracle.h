/*
 * smoe_oracle.h -- CPU restatement of S-MoE's per-layer MoE arithmetic.
 *
 * TEST INFRASTRUCTURE ONLY.  Nothing in the product (the HIP library, the
 * host C++ layer, the Python binding) links, loads or calls this code.  It is
 * used by tests/, by __graft_entry__.smoke() as the checker and by bench.py's
 * cpu_baseline leg (timed, reported beside the GPU number).
 *
 * Every function restates one piece of the reference (paths relative to the
 * reference tree) and is pinned as noted:
 *   orc_bf16_to_f32 / orc_rms_norm_bf16 / orc_matvec_bf16 / orc_axpy_f32
 *       src/common.hpp:238-256, 293-306, 346-349
 *       pinned: golden vectors from the compiled reference (oracle/_ref).
 *   orc_top_k   src/scout/scout.cpp:77-123
 *       pinned: golden vectors from the compiled reference incl. constructed
 *       ties; brute-force swap-sort equivalence.
 *   orc_quantize_q4 / orc_dequant_q4   scripts/shatter_moe.py:331-387,
 *       src/compute/kernels.metal:90-105
 *       pinned: known-answer tests (+-absmax -> 15/0, half-even ties, zero
 *       group, nibble order, reconstruction bound), numpy float16 cast.
 *   orc_expert_ffn   kernels.metal:61-63, 90-105, 672-769 (prefill's
 *       token-batch kernels: per-weight dequant, sequential fp32 sums)
 *   orc_expert_ffn_decode   kernels.metal:61-63, 159-365 (the decode path's
 *       qrow_dot2 / qrow_dot: lane-strided chunks, affine chunk epilogue,
 *       simd_sum)
 *       both pinned: fp64 brute force on tiny and Qwen3-sized shapes (the
 *       decode form within a bound that a dropped chunk, a wrong lane
 *       stride, scale or nibble order exceeds), dequant identity, zero input,
 *       scale linearity.  (The reference's FFN exists only as Metal shaders;
 *       no reference-held vectors exist, and the order inside Metal's
 *       simd_sum and any fast-math contraction are parity unpinned.)
 *   orc_moe_decode_layer   src/decode.cpp:236-238, 280-302, 338-509 (its
 *       expert FFN is orc_expert_ffn_decode)
 *   orc_permute / orc_union_*   src/prefill.cpp:38-68, 315-332
 *       pinned: compiled reference union_add vectors; brute-force stable sort.
 *   orc_moe_prefill_layer  src/prefill.cpp:308-453
 *   orc_rand_* / orc_normal   synthetic-input generator of this build (not in
 *       the reference); the HIP generator must reproduce it bit for bit.
 */
#ifndef SMOE_ORACLE_H
#define SMOE_ORACLE_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* ---- threads ---------------------------------------------------------------
 * Row-parallel loops (OpenMP) in orc_matvec_bf16, orc_expert_ffn and the
 * per-pair FFNs of orc_moe_prefill_layer.  Each output row remains one
 * sequential fp32 sum on one thread, so every result is bit-identical for
 * any thread count (1 = the reference's single-threaded loops). */
void orc_set_threads(int n);
int  orc_get_threads(void);
int  orc_max_threads(void);

/* ---- number formats ------------------------------------------------------ */
float    orc_bf16_to_f32(uint16_t b);
uint16_t orc_f32_to_bf16(float f);          /* round to nearest even */
float    orc_f16_to_f32(uint16_t h);
uint16_t orc_f32_to_f16(float f);           /* round to nearest even */

/* ---- synthetic generator (counter based, bit-reproducible on the GPU) ---- */
uint64_t orc_stream_key(uint64_t seed, uint64_t stream);
uint64_t orc_rand64(uint64_t key, uint64_t i);
float    orc_normal(uint64_t key, uint64_t i);
void     orc_gen_normal(float* out, size_t n, uint64_t seed, uint64_t stream,
                        float stddev);
void     orc_gen_bf16(uint16_t* out, size_t n, uint64_t seed, uint64_t stream,
                      float stddev);

/* ---- A4: SMOE-Q4 ---------------------------------------------------------- */
/* packed: n/2 bytes (low nibble = even index); scales: n/group fp16 bits */
void  orc_quantize_q4(const float* w, size_t n, uint32_t group,
                      uint8_t* packed, uint16_t* scales);
float orc_dequant_q4(const uint8_t* packed, const uint16_t* scales,
                     size_t wi, uint32_t group);
void  orc_dequant_q4_all(const uint8_t* packed, const uint16_t* scales,
                         size_t n, uint32_t group, float* out);
/* synthetic expert matrix: N(0,stddev) from (seed, stream) then quantize */
void  orc_synth_q4(uint8_t* packed, uint16_t* scales, uint32_t rows,
                   uint32_t cols, uint32_t group, uint64_t seed,
                   uint64_t stream, float stddev);

/* ---- A1, A2, A8 ------------------------------------------------------------ */
void orc_rms_norm_bf16(float* x, const uint16_t* w, uint32_t n);
void orc_matvec_bf16(float* out, const uint16_t* weight, const float* in,
                     uint32_t rows, uint32_t cols);
void orc_axpy_f32(float* y, float a, const float* x, uint32_t n);

/* ---- A3 ------------------------------------------------------------------ */
uint32_t orc_top_k(const float* scores, uint32_t n, uint32_t k,
                   uint32_t* out_indices, float* out_weights, int norm_topk);

/* ---- A5/A6: one expert, per-weight dequant, sequential fp32 sums (the
 *      token-batch kernels of prefill, kernels.metal:672-769) ------------- */
float orc_silu(float x);
void orc_expert_ffn(const uint8_t* pg, const uint16_t* sg,
                    const uint8_t* pu, const uint16_t* su,
                    const uint8_t* pd, const uint16_t* sd,
                    const float* x, float* hidden, float* out,
                    uint32_t d_ff, uint32_t d_model, uint32_t group);
/* ---- A5-A7: one expert as the decode path computes it: smoe_gate_up and
 *      smoe_down over qrow_dot2 / qrow_dot (kernels.metal:159-365): lane-
 *      strided 32-code chunks with the affine chunk epilogue, simd_sum per
 *      row.  cols % 32 == 0, group % 32 == 0. -------------------------------- */
void orc_expert_ffn_decode(const uint8_t* pg, const uint16_t* sg,
                           const uint8_t* pu, const uint16_t* su,
                           const uint8_t* pd, const uint16_t* sd,
                           const float* x, float* hidden, float* out,
                           uint32_t d_ff, uint32_t d_model, uint32_t group);
/* the same lanes and chunks for the scale+min format (no counterpart in the
 * reference): chunk value s * A + m * X, with the mins mg/mu/md */
void orc_expert_ffn_decode_min(const uint8_t* pg, const uint16_t* sg, const uint16_t* mg,
                               const uint8_t* pu, const uint16_t* su, const uint16_t* mu,
                               const uint8_t* pd, const uint16_t* sd, const uint16_t* md,
                               const float* x, float* hidden, float* out,
                               uint32_t d_ff, uint32_t d_model, uint32_t group);
/* ---- the scale+min format (no counterpart in the reference): quantizer and
 *      per-weight dequant w = code * s + m, bf16 s and m per group ---------- */
void orc_quantize_q4_min(const float* w, size_t n, uint32_t group, uint8_t* packed,
                         uint16_t* scales, uint16_t* mins);
float orc_dequant_q4_min(const uint8_t* packed, const uint16_t* scales, const uint16_t* mins,
                         size_t wi, uint32_t group);

/* ---- A11: resident expert pool addressing -------------------------------- */
typedef struct {
    uint32_t d_model, n_experts, top_k, d_ff, group_size, norm_topk;
    uint32_t quant;   /* 0 SMOE-Q4; 1 the scale+min format (mins after each matrix's scales) */
} OrcShape;

typedef struct {
    const uint16_t* norm_w;      /* [d_model] bf16 */
    const uint16_t* router_w;    /* [n_experts x d_model] bf16 */
    const uint8_t*  experts;     /* blob of expert 0 */
    uint64_t        stride;      /* bytes between consecutive expert blobs */
    uint64_t gate_packed, gate_scales, up_packed, up_scales,
             down_packed, down_scales;   /* offsets inside a blob */
} OrcLayer;

/* blob layout of shatter_moe.py build_expert_blob (:627-674) for one shape */
void orc_blob_layout(uint32_t d_model, uint32_t d_ff, uint32_t group,
                     uint64_t* offsets6, uint64_t* blob_bytes);

/* ---- A12: one decode MoE block (RMSNorm -> router -> top-k -> FFN ->
 *      rank-ordered combine -> residual).  hidden is updated in place.
 *      ids/weights [top_k]; optional logits [n_experts], normed [d_model],
 *      expert_out [top_k x d_model]; any optional pointer may be NULL. ---- */
void orc_moe_decode_layer(const OrcShape* s, const OrcLayer* L, float* hidden,
                          uint32_t* ids, float* weights, float* logits,
                          float* normed, float* expert_out);

/* ---- A9: token-by-expert permute ----------------------------------------- */
/* Whole-prompt stable counting sort of (token, rank) pairs by expert id:
 *   offsets[n_experts+1], tok[T*k], w[T*k] (ascending token order inside
 *   each expert), union_ids[<=n_experts] in order of first appearance
 *   (token-major, rank-minor); returns the union size.                     */
uint32_t orc_permute(const uint32_t* ids, const float* w, uint32_t T,
                     uint32_t k, uint32_t n_experts, uint32_t* offsets,
                     uint32_t* tok, float* wout, uint32_t* union_ids);
/* prefill.cpp union_add restated: per-chunk state machine */
void     orc_union_reset(void);
int      orc_union_add(uint32_t expert, uint32_t tok_row, float weight);
uint32_t orc_union_size(void);
uint32_t orc_union_id(uint32_t u);
uint32_t orc_union_count(uint32_t expert);
uint32_t orc_union_tok(uint32_t expert, uint32_t t);
float    orc_union_w(uint32_t expert, uint32_t t);

/* ---- A10: prefill MoE block over T tokens, layer-major in chunks of 64 ---
 *      hidden [T x d_model] updated in place; ids/weights [T x top_k]. ---- */
void orc_moe_prefill_layer(const OrcShape* s, const OrcLayer* L, float* hidden,
                           uint32_t T, uint32_t* ids, float* weights);

/* ---- F4: decode attention of one token -----------------------------------
 * decode.cpp:150-229 (CPU branch): QKV GEMVs, per-head QK RMSNorm (NULL norm
 * weights skip it), RoPE on (d, d + head_dim/2), K and V written to the ring
 * at slot, per head softmax over valid positions counted back from slot
 * (sequential sums, expf), axpy of V rows, O GEMV into o_out [d_model].
 * Pinned by its compiled-reference pieces (matvec_bf16, rms_norm_bf16,
 * axpy_f32) and by closed forms in tests/test_oracle_attention.py: one
 * position returns its V row, identical keys average V, RoPE at angle 0 is
 * the identity and at 90 degrees maps (a, b) to (-b, a), a normed head has
 * unit RMS. */
void orc_attention_layer(const uint16_t* w_q, const uint16_t* w_k, const uint16_t* w_v, const uint16_t* w_o,
                         const uint16_t* q_norm_w, const uint16_t* k_norm_w, const float* rope_cos,
                         const float* rope_sin, const float* normed_in, float* k_cache, float* v_cache,
                         float* o_out, uint32_t d_model, uint32_t head_dim, uint32_t num_heads,
                         uint32_t num_kv_heads, uint32_t slot, uint32_t valid, uint32_t attn_ctx, float scale);

#ifdef __cplusplus
}
#endif
#endif
