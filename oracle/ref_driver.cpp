// ref_driver.cpp -- builds the reference's own CPU routines for this path,
// compiled from the reference sources where they lie (-I <reference>/src), into
// oracle/_ref/libsmoe_ref.so.  TEST INFRASTRUCTURE ONLY: used to write and check
// golden vectors for the oracle; never part of the product.
//
// Nothing from the reference is copied here: the two translation units below
// are included by path, and only thin extern "C" wrappers are defined.  The
// link uses --gc-sections with -z defs, so every reference function that is not
// reachable from a wrapper (and with it every Metal / streamer dependency) is
// dropped instead of being stubbed.
//   top_k          src/scout/scout.cpp:77-123
//   rms_norm_bf16  src/common.hpp:245-256
//   matvec_bf16    src/common.hpp:293-306 (the scalar, non-NEON branch)
//   axpy_f32       src/common.hpp:346-349
//   bf16_to_f32    src/common.hpp:238-243
//   union_add      src/prefill.cpp:48-68 (+ its per-chunk state)
#include "scout/scout.cpp"
#include "prefill.cpp"

#define REF_API extern "C" __attribute__((visibility("default")))

REF_API uint32_t ref_top_k(const float* s, uint32_t n, uint32_t k, uint32_t* ids,
                           float* w, int norm_topk)
{
    return smoe::scout::top_k(s, n, k, ids, w, norm_topk != 0);
}
REF_API void ref_rms_norm_bf16(float* x, const uint16_t* w, uint32_t n) { smoe::rms_norm_bf16(x, w, n); }
REF_API void ref_matvec_bf16(float* out, const uint16_t* w, const float* in, uint32_t rows, uint32_t cols)
{
    smoe::matvec_bf16(out, w, in, rows, cols);
}
REF_API void ref_axpy_f32(float* y, float a, const float* x, uint32_t n) { smoe::axpy_f32(y, a, x, n); }
REF_API float ref_bf16_to_f32(uint16_t b) { return smoe::bf16_to_f32(b); }

REF_API void ref_union_reset(void) { smoe::prefill::union_reset(); }
REF_API int ref_union_add(uint32_t e, uint32_t t, float w) { return smoe::prefill::union_add(e, t, w) ? 1 : 0; }
REF_API uint32_t ref_union_size(void) { return smoe::prefill::g_union_size; }
REF_API uint32_t ref_union_id(uint32_t u) { return smoe::prefill::g_union_ids[u]; }
REF_API uint32_t ref_union_count(uint32_t e) { return smoe::prefill::g_elist[e].count; }
REF_API uint32_t ref_union_tok(uint32_t e, uint32_t t) { return smoe::prefill::g_elist[e].tok[t]; }
REF_API float ref_union_w(uint32_t e, uint32_t t) { return smoe::prefill::g_elist[e].w[t]; }
