// shape.hpp -- checks and conversions of the C ABI's shape and layer structs,
// shared by the translation units that implement entry points.
#pragma once

#include "kernels.hpp"
#include "smoe_hip.h"

namespace smoe {

// An SmoeMoeShape the decode and prefill kernels accept: 4 bits (SMOE-Q4, or
// the scale+min format where an entry point takes it), group 64
// (the vault format's group, shatter_moe.py Q2_GROUP_SIZE), d_model and d_ff
// multiples of 64 up to SMOE_MAX_DIM, top_k <= min(SMOE_MAX_ACTIVE, n_experts).
inline int shape_check(const SmoeMoeShape* s)
{
    if (!s) return SMOE_ERR_ARG;
    if (s->bits != 4) return SMOE_ERR_BITS;
    if (s->quant != SMOE_QUANT_SMOEQ4 && s->quant != SMOE_QUANT_Q4_SCALE_MIN) return SMOE_ERR_BITS;
    const uint32_t g = s->group_size;
    if (g == 0 || g % 32 != 0 || g > 128 || (g & (g - 1))) return SMOE_ERR_SHAPE;
    if (s->d_model == 0 || s->d_ff == 0 || s->n_experts == 0 || s->top_k == 0) return SMOE_ERR_SHAPE;
    if (s->d_model % 64 || s->d_ff % 64 || s->d_model % g || s->d_ff % g) return SMOE_ERR_SHAPE;
    if (s->d_model > SMOE_MAX_DIM || s->d_ff > SMOE_MAX_DIM) return SMOE_ERR_SHAPE;
    if (g != 64) return SMOE_ERR_SHAPE;   // the vault format's group (shatter_moe.py Q2_GROUP_SIZE)
    if (s->top_k > SMOE_MAX_ACTIVE || s->top_k > s->n_experts) return SMOE_ERR_SHAPE;
    if (s->n_experts > SMOE_MAX_EXPERTS) return SMOE_ERR_SHAPE;
    if (static_cast<uint64_t>(s->top_k) * (s->d_ff / 32) > 8ull * 64 * 4) return SMOE_ERR_SHAPE;
    return SMOE_OK;
}

inline MoeDims dims_of(const SmoeMoeShape* s)
{
    return MoeDims{s->d_model, s->n_experts, s->top_k, s->d_ff, s->group_size, s->norm_topk ? 1u : 0u, s->quant};
}

inline LayerDesc layer_of(const SmoeMoeLayer* L)
{
    LayerDesc d;
    d.norm_w = L->norm_w;
    d.router_w = L->router_w;
    d.experts = L->experts;
    d.stride = L->expert_stride;
    d.off[0] = L->gate_packed_offset;
    d.off[1] = L->gate_scales_offset;
    d.off[2] = L->up_packed_offset;
    d.off[3] = L->up_scales_offset;
    d.off[4] = L->down_packed_offset;
    d.off[5] = L->down_scales_offset;
    return d;
}

}  // namespace smoe
