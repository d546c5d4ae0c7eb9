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

// ---------------------------------------------------------------------------
// Softmax + top-k for n <= 128 scores (two positions per lane) and k <= 8,
// by a sorting network instead of k serial rounds of max extraction.
//
// Selection runs on 32-bit keys that hold the score's order-preserving bits
// with the low 7 replaced by 127 - position, so every key is distinct and
// the network needs no tie-breaking.  Merging the lists of two lanes keeps
// the top 8 of their union; after one merge per lane bit every lane holds
// the top 8 keys in order.  The bit order is 5, 4 (v_permlane32/16_swap,
// while the lists hold 2 and 4 keys and are merged whole by odd-even merges,
// which compare equal indices only, so the swap's lane order does not
// matter), then within rows: row_ror:8 (lane bit 3), row_half_mirror (lane
// i with lane 7 - i of its 8: after bits 5, 4, 3 they hold the keys of lanes
// with low bits i and 7 - i, disjoint sets) and quad_perm xor 2, xor 1, each
// a bitonic top-8 merge.  The softmax (scout.cpp:85-98) runs beside the
// network; it depends on the scores only.
//
// The keys only PROPOSE ranks.  The result stands when the probabilities of
// the proposed ranks fall strictly, p_0 > ... > p_{c-1}, and the last is
// strictly above every unselected probability: then each round of the
// reference's selection with swaps (scout.cpp:101-110) has a strict unique
// maximum and picks exactly rank s.  Otherwise (ties, probabilities equal
// after rounding, scores equal in their top 25 bits and out of order, any
// non-finite score) the row goes to topk_fast, which is exact everywhere.
// Lane r < count receives (id_r, w_r) as from topk_fast; returns count.
// ---------------------------------------------------------------------------
constexpr int DPP_ROW_SHL1 = 0x101;

__device__ __forceinline__ uint32_t order_bits(float f)
{
    const uint32_t b = __float_as_uint(f);
    return (b & 0x80000000u) ? ~b : (b | 0x80000000u);
}
// hi, lo <- max, min
__device__ __forceinline__ void cmp_swap(uint32_t& hi, uint32_t& lo)
{
    const uint32_t a = hi;
    hi = max(a, lo);
    lo = min(a, lo);
}
// the two values of lane l and of lane l ^ 32 (BIT 5) or l ^ 16 (BIT 4), in an
// order that depends on the lane
template <int BIT>
__device__ __forceinline__ void swap_pair(uint32_t v, uint32_t& x, uint32_t& y)
{
    const auto r = BIT == 5 ? __builtin_amdgcn_permlane32_swap(v, v, false, false)
                            : __builtin_amdgcn_permlane16_swap(v, v, false, false);
    x = r[0];
    y = r[1];
}
// a[j] of a list sorted in descending order, as the minimum of a[0..j] (a
// select chain here is folded into an indexed load from scratch)
__device__ __forceinline__ uint32_t sorted_at(const uint32_t (&a)[8], uint32_t j)
{
    uint32_t r = a[0];
#pragma unroll
    for (int i = 1; i < 8; ++i) r = min(r, static_cast<uint32_t>(i) <= j ? a[i] : 0xFFFFFFFFu);
    return r;
}
// top 8 of the union of this lane's sorted list and the partner's (DPP CTRL)
template <int CTRL>
__device__ __forceinline__ void merge8(uint32_t (&a)[8])
{
    uint32_t h[8];
#pragma unroll
    for (int i = 0; i < 8; ++i) h[i] = max(a[i], dpp_u32<CTRL>(0u, a[7 - i]));   // bitonic
#pragma unroll
    for (int d = 4; d >= 1; d >>= 1) {
#pragma unroll
        for (int i = 0; i < 8; ++i)
            if ((i & d) == 0) cmp_swap(h[i], h[i + d]);
    }
#pragma unroll
    for (int i = 0; i < 8; ++i) a[i] = h[i];
}

// The top 8 of the 128 keys held two per lane (k0, k1), sorted in descending
// order, in every lane's c[0..7] (the network described above).
__device__ __forceinline__ void net_top8(uint32_t k0, uint32_t k1, uint32_t (&c)[8])
{
    // lane bit 5: 2 + 2 keys
    uint32_t a0 = max(k0, k1), a1 = min(k0, k1);
    {
        uint32_t x0, y0, x1, y1;
        swap_pair<5>(a0, x0, y0);
        swap_pair<5>(a1, x1, y1);
        c[0] = max(x0, y0);
        uint32_t mid0 = min(x0, y0), mid1 = max(x1, y1);
        c[3] = min(x1, y1);
        cmp_swap(mid1, mid0);
        c[1] = mid1;
        c[2] = mid0;
    }
    // lane bit 4: 4 + 4 keys, odd-even merge (evens, odds, then neighbours)
    {
        uint32_t x[4], y[4];
#pragma unroll
        for (int i = 0; i < 4; ++i) swap_pair<4>(c[i], x[i], y[i]);
#pragma unroll
        for (int i = 0; i < 4; ++i) cmp_swap(x[i], y[i]);   // x = max, y = min of index i
        // evens: {x0, y0} merged with {x2, y2}
        uint32_t e0 = x[0], e1 = y[0], e2 = x[2], e3 = y[2];
        cmp_swap(e1, e2);
        // odds: {x1, y1} merged with {x3, y3}
        uint32_t o0 = x[1], o1 = y[1], o2 = x[3], o3 = y[3];
        cmp_swap(o1, o2);
        c[0] = e0;
        c[7] = o3;
        cmp_swap(o0, e1);
        cmp_swap(o1, e2);
        cmp_swap(o2, e3);
        c[1] = o0; c[2] = e1; c[3] = o1; c[4] = e2; c[5] = o2; c[6] = e3;
    }
    merge8<DPP_ROW_ROR8>(c);
    merge8<DPP_ROW_HALF_MIRROR>(c);
    merge8<DPP_QUAD_XOR2>(c);
    merge8<DPP_QUAD_XOR1>(c);
}

// Positions of the 8 largest of n <= 128 scores (two per lane, position
// lane + 64 j), largest first, ties to the lower position: lane r < 8 returns
// the position of rank r.  Scores are compared by their order-preserving
// bits (the low 7 replaced by the position, as in topk_net), so scores equal
// in their top 25 bits rank by position; a non-finite score still yields a
// position below n.  Used where an exact top-k is not needed.
__device__ __forceinline__ uint32_t top8_positions(const float (&v)[2], uint32_t n)
{
    const int lane = threadIdx.x & (WAVE - 1);
    uint32_t key[2];
#pragma unroll
    for (int j = 0; j < 2; ++j) {
        const uint32_t pos = lane + WAVE * j;
        key[j] = pos < n ? ((order_bits(v[j]) & ~127u) | (127u - pos)) : 0u;
    }
    uint32_t c[8];
    net_top8(key[0], key[1], c);
    const uint32_t pos = 127u - (sorted_at(c, static_cast<uint32_t>(lane) & 7u) & 127u);
    return min(pos, n - 1);
}

// topk_net in two steps, so that a caller can act on the proposed ranks
// while the softmax and the check run: topk_net_begin builds the keys and
// runs the network; topk_net_rank(s, r) is the position the network proposes
// for rank r (uniform r < 8; what topk_net_finish returns for rank r whenever
// the check passes); topk_net_finish completes as topk_net.
struct NetTopk {
    uint32_t key[2];
    uint32_t c[8];
    bool bad;
};

__device__ __forceinline__ void topk_net_begin(const float (&v)[2], uint32_t n, NetTopk& s)
{
    const int lane = threadIdx.x & (WAVE - 1);
    // keys; a non-finite score fails the final check (the network's result is
    // then unused)
    s.bad = false;
#pragma unroll
    for (int j = 0; j < 2; ++j) {
        const uint32_t pos = lane + WAVE * j;
        s.bad |= pos < n && !isfinite(v[j]);
        s.key[j] = pos < n ? ((order_bits(v[j]) & ~127u) | (127u - pos)) : 0u;
    }
    net_top8(s.key[0], s.key[1], s.c);
}

__device__ __forceinline__ uint32_t topk_net_rank(const NetTopk& s, uint32_t r, uint32_t n)
{
    return min(127u - (sorted_at(s.c, r) & 127u), n - 1);
}

template <int VPL>
__device__ uint32_t topk_net_finish(float (&v)[VPL], uint32_t n, uint32_t k, uint32_t norm, uint32_t& my_id,
                                    float& my_w, uint2* slots, const NetTopk& s)
{
    static_assert(VPL == 2, "topk_net holds two positions per lane");
    const int lane = threadIdx.x & (WAVE - 1);
    const uint32_t count = k < n ? k : n;
    if (count != 0 && count <= 8 && n <= 128) {
        // softmax, as topk_fast
        float m = -INFINITY;
#pragma unroll
        for (int j = 0; j < 2; ++j)
            if (lane + WAVE * j < n) m = fmaxf(m, v[j]);
        m = wave_max(m);
        float e[2], sum = 0.f;
#pragma unroll
        for (int j = 0; j < 2; ++j) {
            e[j] = lane + WAVE * j < n ? expf(v[j] - m) : 0.f;
            sum += e[j];
        }
        sum = wave_sum(sum);
        const float inv_sum = (sum > 0.f) ? 1.0f / sum : 0.f;

        // probabilities: of every position, of the proposed ranks (lane r),
        // and the largest over the unselected positions
        const uint32_t last = sorted_at(s.c, count - 1);
        float p[2], rest = -1.f;
#pragma unroll
        for (int j = 0; j < 2; ++j) {
            p[j] = e[j] * inv_sum;
            if (lane + WAVE * j < n && s.key[j] < last) rest = fmaxf(rest, p[j]);
        }
        rest = wave_max(rest);
        const uint32_t pos = 127u - (sorted_at(s.c, static_cast<uint32_t>(lane) & 7u) & 127u);
        const float q0 = __shfl(p[0], static_cast<int>(pos & 63u));
        const float q1 = __shfl(p[1], static_cast<int>(pos & 63u));
        const float pr = static_cast<uint32_t>(lane) < count ? (pos >= 64u ? q1 : q0) : rest;
        const float next = dpp_f32<DPP_ROW_SHL1>(-1.f, pr);   // lane r + 1's
        if (__ballot(s.bad || (static_cast<uint32_t>(lane) < count && !(pr > next))) == 0) {
            float ksum = 0.f;
#pragma unroll
            for (int r = 0; r < 8; ++r)   // rank order, as the reference (x + 0 = x)
                ksum += static_cast<uint32_t>(r) < count ? readlane_f32(pr, r) : 0.f;
            my_id = static_cast<uint32_t>(lane) < count ? pos : 0u;
            my_w = static_cast<uint32_t>(lane) < count ? pr : 0.f;
            if (norm && ksum > 0.f) my_w = my_w * (1.0f / ksum);
            return count;
        }
    }
    return topk_fast<VPL>(v, n, k, norm, my_id, my_w, slots);
}

template <int VPL>
__device__ uint32_t topk_net(float (&v)[VPL], uint32_t n, uint32_t k, uint32_t norm, uint32_t& my_id, float& my_w,
                             uint2* slots)
{
    NetTopk s;
    topk_net_begin(v, n, s);
    return topk_net_finish<VPL>(v, n, k, norm, my_id, my_w, slots, s);
}

// The latency-bound callers (one row per wave on the critical path): the
// network for up to 128 scores, max extraction above.
template <int VPL>
__device__ __forceinline__ uint32_t topk_latency(float (&v)[VPL], uint32_t n, uint32_t k, uint32_t norm,
                                                 uint32_t& my_id, float& my_w, uint2* slots)
{
    if constexpr (VPL == 2) return topk_net<VPL>(v, n, k, norm, my_id, my_w, slots);
    else return topk_fast<VPL>(v, n, k, norm, my_id, my_w, slots);
}

// positions per lane for n experts: 2 (n <= 128) or 8 (n <= 512)
static inline int topk_vpl(uint32_t n) { return n <= 128 ? 2 : 8; }

}  // namespace smoe
