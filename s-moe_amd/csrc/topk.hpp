// topk.hpp -- softmax + top-k of one row of scores held in one wave64, exact
// with the reference's selection sort with swaps (scout.cpp:77-123).
// Shared by the decode kernel (k_moe_up), the standalone k_topk and the
// prefill router (k_route).
#pragma once

#include "device_common.hpp"

namespace smoe {

// ---------------------------------------------------------------------------
// softmax + selection sort with swaps (scout.cpp:77-123) in one wave.
// Round s scans positions s..n-1 with a strict '>' and swaps the winner into
// position s: the winner is the LOWEST position holding the maximum of the
// not-yet-selected positions (a NaN at position s stays put, as '>' against
// NaN is false).  Positions live in lanes: position p = lane + 64*j.
// ---------------------------------------------------------------------------
// Keys: bits(p) + 1 for candidate positions (probabilities are >= +0, so the
// uint order is the float order; a NaN gets key 1 and, like +0, never wins a
// strict '>' against an earlier position), 0 for positions already selected
// and for padding.  Each round: wave max of the keys on DPP, the lowest
// position holding it from ballots, swap by readlane.
template <int VPL>
__device__ __forceinline__ float sel(const float (&a)[VPL], uint32_t j)
{
    float r = a[0];
#pragma unroll
    for (int t = 1; t < VPL; ++t) r = (static_cast<uint32_t>(t) == j) ? a[t] : r;
    return r;
}
template <int VPL>
__device__ __forceinline__ uint32_t sel(const uint32_t (&a)[VPL], uint32_t j)
{
    uint32_t r = a[0];
#pragma unroll
    for (int t = 1; t < VPL; ++t) r = (static_cast<uint32_t>(t) == j) ? a[t] : r;
    return r;
}

// Load the n scores of one row into the positions of this lane (position
// p = lane + 64 j); padding positions get -inf.
template <int VPL>
__device__ __forceinline__ void topk_load(const float* scores, uint32_t n, float (&p)[VPL])
{
    const int lane = threadIdx.x & (WAVE - 1);
#pragma unroll
    for (int j = 0; j < VPL; ++j) {
        const uint32_t pos = lane + WAVE * j;
        p[j] = pos < n ? scores[pos] : -INFINITY;
    }
}

// k rounds of the swap-based selection sort over keys held in lanes (see
// above); lane r < count receives (id_r, w_r), renormalised if norm.
template <int VPL>
__device__ void topk_select(float (&p)[VPL], uint32_t (&id)[VPL], uint32_t (&key)[VPL], uint32_t count,
                            uint32_t norm, uint32_t& my_id, float& my_w)
{
    const int lane = threadIdx.x & (WAVE - 1);
    float ksum = 0.f;
    my_id = 0;
    my_w = 0.f;
    for (uint32_t s = 0; s < count; ++s) {
        const uint32_t sj = s >> 6;
        const int sl = s & 63;
        const float val_s = readlane_f32(sel(p, sj), sl);
        const uint32_t id_s = readlane_u32(sel(id, sj), sl);
        const uint32_t key_s = readlane_u32(sel(key, sj), sl);
        uint32_t lk = key[0];
#pragma unroll
        for (int j = 1; j < VPL; ++j) lk = max(lk, key[j]);
        const uint32_t K = wave_max_u32(lk);
        uint32_t best = 0xFFFFFFFFu;
#pragma unroll
        for (int j = 0; j < VPL; ++j) {
            const uint64_t mk = __ballot(key[j] == K);
            if (best == 0xFFFFFFFFu && mk != 0) best = WAVE * j + __builtin_ctzll(mk);
        }
        if (isnan(val_s)) best = s;
        const uint32_t bj = best >> 6;
        const int bl = best & 63;
        const float val_b = readlane_f32(sel(p, bj), bl);
        const uint32_t id_b = readlane_u32(sel(id, bj), bl);
#pragma unroll
        for (int j = 0; j < VPL; ++j) {
            if (lane == bl && static_cast<uint32_t>(j) == bj) { p[j] = val_s; id[j] = id_s; key[j] = key_s; }
        }
#pragma unroll
        for (int j = 0; j < VPL; ++j) {
            if (lane == sl && static_cast<uint32_t>(j) == sj) { p[j] = val_b; id[j] = id_b; key[j] = 0u; }
        }
        ksum += val_b;                       // sequential over ranks, as the reference
        if (static_cast<uint32_t>(lane) == s) { my_id = id_b; my_w = val_b; }
    }
    if (norm && ksum > 0.f) my_w = my_w * (1.0f / ksum);
}

// ---------------------------------------------------------------------------
// Softmax + top-k of n scores held in one wave (position p = lane + 64 j).
// Fast path: count rounds of max extraction, all in the vector unit.  Round
// s takes the wave maximum K of the remaining keys and marks every position
// holding K with rank s (removing it).  When every round removes exactly one
// position, that position is what the reference's round s of selection with
// swaps (scout.cpp:101-110) picks, whatever the earlier swaps moved, since a
// strict maximum wins the strict '>' scan from any arrangement; a unique
// maximum in the last round is also strictly above every unselected key.  So
// the fast result stands when the rounds removed exactly count positions; a
// tie (two positions removed in one round) or any NaN sends the row to the
// exact swap emulation topk_select.  The ranked (position, probability) pairs
// are gathered through `slots` (16 entries of LDS private to this wave) and
// the renormalisation sum runs in rank order, as the reference's.
// Lane r < count receives (id_r, w_r); returns count.
// ---------------------------------------------------------------------------
constexpr uint32_t TOPK_SLOTS = 16;   // LDS uint2 entries per wave (k <= 16)

template <int VPL>
__device__ uint32_t topk_fast(float (&v)[VPL], uint32_t n, uint32_t k, uint32_t norm, uint32_t& my_id,
                              float& my_w, uint2* slots)
{
    const int lane = threadIdx.x & (WAVE - 1);
    // softmax (scout.cpp:85-98)
    float m = -INFINITY;
#pragma unroll
    for (int j = 0; j < VPL; ++j)
        if (lane + WAVE * j < n) m = fmaxf(m, v[j]);
    m = wave_max(m);
    float sum = 0.f;
#pragma unroll
    for (int j = 0; j < VPL; ++j) {
        const uint32_t pos = lane + WAVE * j;
        v[j] = pos < n ? expf(v[j] - m) : 0.f;
        sum += v[j];
    }
    sum = wave_sum(sum);
    const float inv_sum = (sum > 0.f) ? 1.0f / sum : 0.f;
    uint32_t key[VPL], rem[VPL], rank[VPL];
    bool nan = false;
#pragma unroll
    for (int j = 0; j < VPL; ++j) {
        const uint32_t pos = lane + WAVE * j;
        v[j] *= inv_sum;
        nan |= pos < n && isnan(v[j]);
        key[j] = pos < n ? (isnan(v[j]) ? 1u : __float_as_uint(v[j]) + 1u) : 0u;
        rem[j] = key[j];
        rank[j] = TOPK_SLOTS;
    }
    const uint32_t count = k < n ? k : n;
    if (__ballot(nan) == 0) {
        for (uint32_t s = 0; s < count; ++s) {
            uint32_t lk = rem[0];
#pragma unroll
            for (int j = 1; j < VPL; ++j) lk = max(lk, rem[j]);
            const uint32_t K = wave_max_u32_all(lk);
#pragma unroll
            for (int j = 0; j < VPL; ++j) {
                const bool hit = rem[j] == K;
                rank[j] = hit ? s : rank[j];
                rem[j] = hit ? 0u : rem[j];
            }
        }
        uint32_t removed = 0;
#pragma unroll
        for (int j = 0; j < VPL; ++j) removed += __popcll(__ballot(rank[j] < TOPK_SLOTS));
        if (removed == count) {
#pragma unroll
            for (int j = 0; j < VPL; ++j)
                if (rank[j] < TOPK_SLOTS) slots[rank[j]] = make_uint2(lane + WAVE * j, __float_as_uint(v[j]));
            // the wave's LDS writes complete in order before its read
            const uint2 e = slots[min(static_cast<uint32_t>(lane), TOPK_SLOTS - 1)];
            float ksum = 0.f;
            for (uint32_t r = 0; r < count; ++r) ksum += __uint_as_float(readlane_u32(e.y, static_cast<int>(r)));
            my_id = static_cast<uint32_t>(lane) < count ? e.x : 0u;
            my_w = static_cast<uint32_t>(lane) < count ? __uint_as_float(e.y) : 0.f;
            if (norm && ksum > 0.f) my_w = my_w * (1.0f / ksum);   // rank order, as the reference
            return count;
        }
    }
    uint32_t id[VPL];
#pragma unroll
    for (int j = 0; j < VPL; ++j) id[j] = lane + WAVE * j;
    topk_select<VPL>(v, id, key, count, norm, my_id, my_w);
    return count;
}

// positions per lane for n experts: 2 (n <= 128) or 8 (n <= 512)
static inline int topk_vpl(uint32_t n) { return n <= 128 ? 2 : 8; }

}  // namespace smoe
