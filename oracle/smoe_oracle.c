/*
 * smoe_oracle.c -- CPU restatement of S-MoE's MoE block (see smoe_oracle.h).
 *
 * TEST INFRASTRUCTURE ONLY: the checker for the HIP path and the timed CPU
 * baseline.  Build with -ffp-contract=off so that every a*b+c below is two
 * roundings, as in the reference's scalar x86 build of src/common.hpp and
 * src/scout/scout.cpp; the generator uses explicit fmaf only.
 */
#include "smoe_oracle.h"

#include <math.h>
#include <stdlib.h>
#include <string.h>

#ifdef _OPENMP
#include <omp.h>
#endif

/* Threads of the row-parallel loops (orc_set_threads).  Every output row is
 * one sequential fp32 sum computed by one thread, so results do not depend on
 * the thread count. */
static int g_threads = 1;

void orc_set_threads(int n) { g_threads = n < 1 ? 1 : n; }
int orc_get_threads(void) { return g_threads; }
int orc_max_threads(void)
{
#ifdef _OPENMP
    return omp_get_max_threads();
#else
    return 1;
#endif
}

static inline uint32_t f2u(float f) { uint32_t u; memcpy(&u, &f, 4); return u; }
static inline float u2f(uint32_t u) { float f; memcpy(&f, &u, 4); return f; }

/* ------------------------------------------------------------------------ */
/* number formats                                                            */
/* ------------------------------------------------------------------------ */

/* src/common.hpp:238-243: bf16 -> f32 is the 16-bit left shift */
float orc_bf16_to_f32(uint16_t b) { return u2f((uint32_t)b << 16); }

uint16_t orc_f32_to_bf16(float f)
{
    uint32_t x = f2u(f);
    if ((x & 0x7FFFFFFFu) > 0x7F800000u) return (uint16_t)((x >> 16) | 0x40u);
    x += 0x7FFFu + ((x >> 16) & 1u);
    return (uint16_t)(x >> 16);
}

float orc_f16_to_f32(uint16_t h)
{
    uint32_t sign = ((uint32_t)h & 0x8000u) << 16;
    uint32_t e = ((uint32_t)h >> 10) & 0x1Fu;
    uint32_t m = (uint32_t)h & 0x3FFu;
    if (e == 0) {
        if (m == 0) return u2f(sign);
        float v = (float)m * 5.9604644775390625e-8f;   /* m * 2^-24, exact */
        return u2f(f2u(v) | sign);
    }
    if (e == 31) return u2f(sign | 0x7F800000u | (m << 13));
    return u2f(sign | ((e + 112u) << 23) | (m << 13));
}

/* IEEE binary16 round-to-nearest-even, the cast numpy's astype(float16)
 * performs in scripts/shatter_moe.py:354 */
uint16_t orc_f32_to_f16(float f)
{
    uint32_t x = f2u(f);
    uint32_t sign = (x >> 16) & 0x8000u;
    uint32_t a = x & 0x7FFFFFFFu;
    if (a >= 0x7F800000u) {                       /* inf / nan */
        if (a == 0x7F800000u) return (uint16_t)(sign | 0x7C00u);
        return (uint16_t)(sign | 0x7E00u | ((a >> 13) & 0x3FFu));
    }
    if (a >= 0x477FF000u) return (uint16_t)(sign | 0x7C00u);   /* >= 65520 */
    if (a < 0x38800000u) {                        /* fp16 subnormal range */
        if (a < 0x33000000u) return (uint16_t)sign;             /* < 2^-25 */
        uint32_t e = a >> 23;
        uint32_t m = (a & 0x7FFFFFu) | 0x800000u;
        uint32_t shift = 126u - e;                /* 14 .. 24 */
        uint32_t q = m >> shift;
        uint32_t rem = m & ((1u << shift) - 1u);
        uint32_t half = 1u << (shift - 1u);
        if (rem > half || (rem == half && (q & 1u))) q++;
        return (uint16_t)(sign | q);
    }
    uint32_t r = a - 0x38000000u;                 /* rebias 127 -> 15 */
    r += 0xFFFu + ((r >> 13) & 1u);
    return (uint16_t)(sign | (r >> 13));
}

/* ------------------------------------------------------------------------ */
/* synthetic generator (this build's; the HIP twin lives in synth.hip)      */
/* ------------------------------------------------------------------------ */
#define ORC_GAMMA 0x9E3779B97F4A7C15ull

static inline uint64_t fmix64(uint64_t z)
{
    z = (z ^ (z >> 30)) * 0xBF58476D1CE4E5B9ull;
    z = (z ^ (z >> 27)) * 0x94D049BB133111EBull;
    return z ^ (z >> 31);
}

uint64_t orc_stream_key(uint64_t seed, uint64_t stream)
{
    return fmix64(seed * ORC_GAMMA + fmix64(stream + ORC_GAMMA));
}

uint64_t orc_rand64(uint64_t key, uint64_t i) { return fmix64(key + (i + 1) * ORC_GAMMA); }

/* natural log on (0,1], argument split m*2^e, atanh series (fmaf chain) */
static float det_log(float u)
{
    uint32_t b = f2u(u);
    int e = (int)(b >> 23) - 127;
    float m = u2f((b & 0x7FFFFFu) | 0x3F800000u);
    if (m > 1.41421356f) { m = m * 0.5f; e += 1; }
    float f = m - 1.0f;
    float s = f / (2.0f + f);
    float z = s * s;
    float p = 0.13333333f;
    p = fmaf(p, z, 0.15384615f);
    p = fmaf(p, z, 0.18181818f);
    p = fmaf(p, z, 0.22222222f);
    p = fmaf(p, z, 0.28571429f);
    p = fmaf(p, z, 0.4f);
    p = fmaf(p, z, 0.66666667f);
    float lnm = fmaf(s * z, p, 2.0f * s);
    float fe = (float)e;
    return fmaf(fe, 0.693145751953125f, fmaf(fe, 1.42860677e-06f, lnm));
}

/* cos(2*pi*t) for t in [0,1): quadrant folding + Taylor series to a^14 */
static float det_cos2pi(float t)
{
    float y = t - 0.5f;
    float sign = -1.0f;
    y = fabsf(y);
    if (y > 0.25f) { y = 0.5f - y; sign = -sign; }
    float a = y * 6.28318531f;
    float a2 = a * a;
    float c = -1.1470746e-11f;
    c = fmaf(c, a2, 2.0876757e-09f);
    c = fmaf(c, a2, -2.7557319e-07f);
    c = fmaf(c, a2, 2.4801587e-05f);
    c = fmaf(c, a2, -1.3888889e-03f);
    c = fmaf(c, a2, 4.1666668e-02f);
    c = fmaf(c, a2, -0.5f);
    c = fmaf(c, a2, 1.0f);
    return sign * c;
}

/* Box-Muller (cosine branch) on two 24-bit uniforms of one 64-bit draw */
float orc_normal(uint64_t key, uint64_t i)
{
    uint64_t h = orc_rand64(key, i);
    float u1 = (float)((h >> 40) + 1u) * 5.9604644775390625e-8f;        /* (0,1] */
    float u2 = (float)((h >> 16) & 0xFFFFFFu) * 5.9604644775390625e-8f; /* [0,1) */
    float r = sqrtf(-2.0f * det_log(u1));
    return r * det_cos2pi(u2);
}

void orc_gen_normal(float* out, size_t n, uint64_t seed, uint64_t stream, float stddev)
{
    uint64_t key = orc_stream_key(seed, stream);
    for (size_t i = 0; i < n; ++i) out[i] = orc_normal(key, i) * stddev;
}

void orc_gen_bf16(uint16_t* out, size_t n, uint64_t seed, uint64_t stream, float stddev)
{
    uint64_t key = orc_stream_key(seed, stream);
    for (size_t i = 0; i < n; ++i) out[i] = orc_f32_to_bf16(orc_normal(key, i) * stddev);
}

/* ------------------------------------------------------------------------ */
/* A4: SMOE-Q4 (scripts/shatter_moe.py:331-368; kernels.metal:90-105)       */
/* ------------------------------------------------------------------------ */
void orc_quantize_q4(const float* w, size_t n, uint32_t group, uint8_t* packed, uint16_t* scales)
{
    size_t n_groups = (n + group - 1) / group;             /* :341-345 zero pad */
    memset(packed, 0, (n + 1) / 2);
    for (size_t g = 0; g < n_groups; ++g) {
        size_t base = g * (size_t)group;
        float absmax = 0.0f;                               /* :350 */
        for (uint32_t j = 0; j < group; ++j) {
            float v = (base + j < n) ? w[base + j] : 0.0f;
            float a = fabsf(v);
            if (a > absmax) absmax = a;
        }
        float best = (absmax == 0.0f) ? 1.0f : absmax;     /* :351 */
        scales[g] = orc_f32_to_f16(best);                  /* :352 */
        for (uint32_t j = 0; j < group && base + j < n; ++j) {
            float q = w[base + j] / best;                  /* :355 */
            q = q * 7.5f;
            q = q + 7.5f;                                  /* :356 */
            float r = rintf(q);                            /* np.round: half-even */
            int c = (int)r;
            if (c < 0) c = 0;
            if (c > 15) c = 15;
            size_t i = base + j;                           /* :361-365 low nibble even */
            packed[i >> 1] |= (uint8_t)((uint32_t)c << ((i & 1u) * 4u));
        }
    }
}

float orc_dequant_q4(const uint8_t* packed, const uint16_t* scales, size_t wi, uint32_t group)
{
    uint32_t code = ((uint32_t)packed[wi >> 1] >> ((wi & 1u) * 4u)) & 0xFu;
    float scale = orc_f16_to_f32(scales[wi / group]);
    return ((float)code - 7.5f) * (1.0f / 7.5f) * scale;  /* kernels.metal:104 */
}

void orc_dequant_q4_all(const uint8_t* packed, const uint16_t* scales, size_t n,
                        uint32_t group, float* out)
{
    for (size_t i = 0; i < n; ++i) out[i] = orc_dequant_q4(packed, scales, i, group);
}

/* The scale+min format of the benchmark configurations (no counterpart in
 * the reference; this build's definition, the one the GPU quantizer uses):
 * per group m = bf16(min w), s = bf16((max w - min w) / 15) (bf16 1.0 when
 * that rounds to 0), code = clamp(rint((w - m) / s), 0, 15) from the rounded
 * s and m (two roundings: the difference, then the quotient), low nibble =
 * even index.  Dequant: w = code * s + m. */
void orc_quantize_q4_min(const float* w, size_t n, uint32_t group, uint8_t* packed, uint16_t* scales,
                         uint16_t* mins)
{
    size_t n_groups = n / group;
    memset(packed, 0, n / 2);
    for (size_t g = 0; g < n_groups; ++g) {
        const float* v = w + g * (size_t)group;
        float lo = v[0], hi = v[0];
        for (uint32_t j = 1; j < group; ++j) {
            if (v[j] < lo) lo = v[j];
            if (v[j] > hi) hi = v[j];
        }
        float span = (hi - lo) / 15.0f;
        uint16_t sb = orc_f32_to_bf16(span);
        if ((sb & 0x7FFFu) == 0) sb = 0x3F80u;
        uint16_t mb = orc_f32_to_bf16(lo);
        scales[g] = sb;
        mins[g] = mb;
        float s = orc_bf16_to_f32(sb), m = orc_bf16_to_f32(mb);
        for (uint32_t j = 0; j < group; ++j) {
            float q = v[j] - m;
            q = q / s;
            int c = (int)rintf(q);
            if (c < 0) c = 0;
            if (c > 15) c = 15;
            size_t i = g * (size_t)group + j;
            packed[i >> 1] |= (uint8_t)((uint32_t)c << ((i & 1u) * 4u));
        }
    }
}

float orc_dequant_q4_min(const uint8_t* packed, const uint16_t* scales, const uint16_t* mins, size_t wi,
                         uint32_t group)
{
    uint32_t code = ((uint32_t)packed[wi >> 1] >> ((wi & 1u) * 4u)) & 0xFu;
    return (float)code * orc_bf16_to_f32(scales[wi / group]) + orc_bf16_to_f32(mins[wi / group]);
}

void orc_synth_q4(uint8_t* packed, uint16_t* scales, uint32_t rows, uint32_t cols,
                  uint32_t group, uint64_t seed, uint64_t stream, float stddev)
{
    size_t n = (size_t)rows * cols;
    float* w = (float*)malloc(n * sizeof(float));
    if (!w) return;
    orc_gen_normal(w, n, seed, stream, stddev);
    orc_quantize_q4(w, n, group, packed, scales);
    free(w);
}

/* ------------------------------------------------------------------------ */
/* A1, A2, A8 (src/common.hpp)                                               */
/* ------------------------------------------------------------------------ */
void orc_rms_norm_bf16(float* x, const uint16_t* w, uint32_t n)   /* :245-256 */
{
    float ss = 0.0f;
    for (uint32_t i = 0; i < n; ++i) ss += x[i] * x[i];
    ss /= (float)n;
    ss += 1e-6f;
    ss = 1.0f / sqrtf(ss);
    for (uint32_t i = 0; i < n; ++i) x[i] = (x[i] * ss) * orc_bf16_to_f32(w[i]);
}

void orc_matvec_bf16(float* out, const uint16_t* weight, const float* in,
                     uint32_t rows, uint32_t cols)                 /* :293-306 */
{
#pragma omp parallel for num_threads(g_threads) schedule(static) if (g_threads > 1)
    for (uint32_t i = 0; i < rows; ++i) {
        float sum = 0.0f;
        const uint16_t* w_row = weight + (size_t)i * cols;
        for (uint32_t j = 0; j < cols; ++j) sum += orc_bf16_to_f32(w_row[j]) * in[j];
        out[i] = sum;
    }
}

void orc_axpy_f32(float* y, float a, const float* x, uint32_t n)   /* :346-349 */
{
    for (uint32_t i = 0; i < n; ++i) y[i] += a * x[i];
}

/* ------------------------------------------------------------------------ */
/* A3: softmax + partial selection sort with swaps (scout.cpp:77-123)       */
/* ------------------------------------------------------------------------ */
uint32_t orc_top_k(const float* scores, uint32_t n, uint32_t k,
                   uint32_t* out_indices, float* out_weights, int norm_topk)
{
    uint32_t count = k < n ? k : n;
    float* tmp = (float*)malloc((n ? n : 1) * sizeof(float));
    uint32_t* idx = (uint32_t*)malloc((n ? n : 1) * sizeof(uint32_t));
    if (!tmp || !idx) { free(tmp); free(idx); return 0; }

    float max_val = scores[0];
    for (uint32_t i = 1; i < n; ++i)
        if (scores[i] > max_val) max_val = scores[i];
    float sum_exp = 0.0f;
    for (uint32_t i = 0; i < n; ++i) {
        tmp[i] = expf(scores[i] - max_val);
        idx[i] = i;
        sum_exp += tmp[i];
    }
    float inv_sum = (sum_exp > 0.0f) ? 1.0f / sum_exp : 0.0f;
    for (uint32_t i = 0; i < n; ++i) tmp[i] *= inv_sum;

    for (uint32_t s = 0; s < count; ++s) {
        uint32_t best = s;
        for (uint32_t i = s + 1; i < n; ++i)
            if (tmp[i] > tmp[best]) best = i;
        float ft = tmp[s]; tmp[s] = tmp[best]; tmp[best] = ft;
        uint32_t it = idx[s]; idx[s] = idx[best]; idx[best] = it;
        out_indices[s] = idx[s];
        if (out_weights) out_weights[s] = tmp[s];
    }

    if (norm_topk && out_weights) {
        float topk_sum = 0.0f;
        for (uint32_t s = 0; s < count; ++s) topk_sum += out_weights[s];
        if (topk_sum > 0.0f) {
            float inv = 1.0f / topk_sum;
            for (uint32_t s = 0; s < count; ++s) out_weights[s] *= inv;
        }
    }
    free(tmp);
    free(idx);
    return count;
}

/* ------------------------------------------------------------------------ */
/* A5/A6: expert FFN with per-weight dequant (kernels.metal:61-63, 672-769) */
/* ------------------------------------------------------------------------ */
float orc_silu(float x) { return x * (1.0f / (1.0f + expf(-x))); }

/* one row of a Q4 matrix dotted with v, sequential fp32 sum over columns;
 * the level table holds exactly ((float)c - 7.5f) * (1.0f/7.5f) per code, so
 * level[c] * scale is the per-weight dequant of kernels.metal:104 */
static float q4_row_dot(const uint8_t* packed, const uint16_t* scales, size_t row,
                        uint32_t cols, uint32_t group, const float* v)
{
    float level[16];
    for (int c = 0; c < 16; ++c) level[c] = ((float)c - 7.5f) * (1.0f / 7.5f);
    float acc = 0.0f;
    size_t base = row * (size_t)cols;
    for (uint32_t j0 = 0; j0 < cols; j0 += group) {
        float s = orc_f16_to_f32(scales[(base + j0) / group]);
        uint32_t jend = j0 + group < cols ? j0 + group : cols;
        for (uint32_t j = j0; j < jend; ++j) {
            size_t wi = base + j;
            uint32_t code = ((uint32_t)packed[wi >> 1] >> ((wi & 1u) * 4u)) & 0xFu;
            float w = level[code] * s;
            acc += w * v[j];
        }
    }
    return acc;
}

void orc_expert_ffn(const uint8_t* pg, const uint16_t* sg,
                    const uint8_t* pu, const uint16_t* su,
                    const uint8_t* pd, const uint16_t* sd,
                    const float* x, float* hidden, float* out,
                    uint32_t d_ff, uint32_t d_model, uint32_t group)
{
#pragma omp parallel num_threads(g_threads) if (g_threads > 1)
    {
#pragma omp for schedule(static)
        for (uint32_t r = 0; r < d_ff; ++r) {
            float g = q4_row_dot(pg, sg, r, d_model, group, x);
            float u = q4_row_dot(pu, su, r, d_model, group, x);
            hidden[r] = orc_silu(g) * u;                   /* kernels.metal:720-722 */
        }
        /* (the implicit barrier of the loop above: down needs all of hidden) */
#pragma omp for schedule(static)
        for (uint32_t d = 0; d < d_model; ++d)
            out[d] = q4_row_dot(pd, sd, d, d_ff, group, hidden);
    }
}

/* ------------------------------------------------------------------------ */
/* A5-A7 on the decode path: smoe_gate_up / smoe_down (kernels.metal:308-365) */
/* over qrow_dot2 / qrow_dot (kernels.metal:159-305), the arithmetic that     */
/* decode.cpp:386-392's smoe_metal_fused_ffn_group dispatches.  One 32-lane    */
/* simdgroup per row: lane L owns the 16-byte chunks c = L, L + 32, ... (32    */
/* codes each, one scale per chunk); per chunk a float4 accumulator takes      */
/* fma(code, x) over the chunk's 4 words (low 4 codes, then high 4, of each),  */
/* xs += xlo + xhi, and the lane accumulator takes                              */
/* fma(s, (a.x + a.y + a.z + a.w) * (1/7.5) - X, acc); simd_sum closes the     */
/* row.  simd_sum's internal order is Apple's: it is restated here as an xor  */
/* butterfly over the 32 lanes (16, 8, 4, 2, 1), and the source's operations  */
/* are kept as written (no contraction beyond the explicit fma calls).         */
/* ------------------------------------------------------------------------ */
static float simd_sum32(float* v)
{
    for (int m = 16; m >= 1; m >>= 1) {
        float t[32];
        for (int l = 0; l < 32; ++l) t[l] = v[l] + v[l ^ m];
        memcpy(v, t, sizeof t);
    }
    return v[0];
}

/* The row dots below come in two clones picked at load time: one for hosts
 * with FMA instructions and a generic one, where fmaf is libm's.  Both round
 * every fmaf once, so they give the same bits; the clone only makes the
 * timed CPU baseline use the host's fused multiply-add. */
#if defined(__x86_64__) && defined(__GNUC__) && !defined(__clang__)
#define ORC_FMA_CLONES __attribute__((target_clones("fma", "default")))
#else
#define ORC_FMA_CLONES
#endif

/* one 32-code chunk: the float4 code.x accumulator a[4] and the x sum xs[4]
 * (kernels.metal:183-197 / 266-287) */
static inline __attribute__((always_inline)) void q4_chunk(const uint8_t* chunk, const float* xv, float a[4], float xs[4])
{
    for (int k = 0; k < 4; ++k) {
        uint32_t u = (uint32_t)chunk[4 * k] | ((uint32_t)chunk[4 * k + 1] << 8) |
                     ((uint32_t)chunk[4 * k + 2] << 16) | ((uint32_t)chunk[4 * k + 3] << 24);
        const float* xlo = xv + 8 * k;
        const float* xhi = xv + 8 * k + 4;
        for (int j = 0; j < 4; ++j) a[j] = fmaf((float)((u >> (4 * j)) & 0xFu), xlo[j], a[j]);
        for (int j = 0; j < 4; ++j) a[j] = fmaf((float)((u >> (16 + 4 * j)) & 0xFu), xhi[j], a[j]);
        for (int j = 0; j < 4; ++j) xs[j] = xs[j] + (xlo[j] + xhi[j]);
    }
}

/* mins: NULL for SMOE-Q4; else the scale+min format, whose chunk value is
 * s * A + m * X (the same lanes, chunks and sums; the epilogue of w = c s + m) */
ORC_FMA_CLONES static float q4_qrow_dot(const uint8_t* packed, const uint16_t* scales, const uint16_t* mins,
                                        size_t row, uint32_t cols, uint32_t group, const float* x)
{
    const uint8_t* rp = packed + row * (size_t)(cols >> 1);
    const uint16_t* srow = scales + row * (size_t)(cols / group);
    const uint16_t* mrow = mins ? mins + row * (size_t)(cols / group) : NULL;
    const uint32_t nchunks = cols >> 5;
    float acc[32] = {0};
    for (uint32_t c = 0; c < nchunks; ++c) {
        float a[4] = {0, 0, 0, 0}, xs[4] = {0, 0, 0, 0};
        q4_chunk(rp + 16 * (size_t)c, x + 32 * (size_t)c, a, xs);
        const float A = ((a[0] + a[1]) + a[2]) + a[3];
        const float X = ((xs[0] + xs[1]) + xs[2]) + xs[3];
        if (mrow) {
            const float s = orc_bf16_to_f32(srow[(c << 5) / group]), m = orc_bf16_to_f32(mrow[(c << 5) / group]);
            acc[c & 31u] = fmaf(s, A, fmaf(m, X, acc[c & 31u]));
        } else {
            const float s = orc_f16_to_f32(srow[(c << 5) / group]);
            acc[c & 31u] = fmaf(s, A * (1.0f / 7.5f) - X, acc[c & 31u]);
        }
    }
    return simd_sum32(acc);
}

ORC_FMA_CLONES static void q4_qrow_dot2(const uint8_t* gp, const uint16_t* gs, const uint16_t* gm, const uint8_t* up,
                                        const uint16_t* us, const uint16_t* um, size_t row, uint32_t cols,
                                        uint32_t group, const float* x, float* g_out, float* u_out)
{
    const size_t rb = row * (size_t)(cols >> 1), sbase = row * (size_t)(cols / group);
    const uint32_t nchunks = cols >> 5;
    float ga[32] = {0}, ua[32] = {0};
    for (uint32_t c = 0; c < nchunks; ++c) {
        float ag[4] = {0, 0, 0, 0}, au[4] = {0, 0, 0, 0}, xs[4] = {0, 0, 0, 0}, xs2[4] = {0, 0, 0, 0};
        q4_chunk(gp + rb + 16 * (size_t)c, x + 32 * (size_t)c, ag, xs);
        q4_chunk(up + rb + 16 * (size_t)c, x + 32 * (size_t)c, au, xs2);   /* (xs2 == xs) */
        const size_t si = sbase + (c << 5) / group;
        const float X = ((xs[0] + xs[1]) + xs[2]) + xs[3];
        const float Ag = ((ag[0] + ag[1]) + ag[2]) + ag[3], Au = ((au[0] + au[1]) + au[2]) + au[3];
        if (gm) {
            ga[c & 31u] = fmaf(orc_bf16_to_f32(gs[si]), Ag, fmaf(orc_bf16_to_f32(gm[si]), X, ga[c & 31u]));
            ua[c & 31u] = fmaf(orc_bf16_to_f32(us[si]), Au, fmaf(orc_bf16_to_f32(um[si]), X, ua[c & 31u]));
        } else {
            ga[c & 31u] = fmaf(orc_f16_to_f32(gs[si]), Ag * (1.0f / 7.5f) - X, ga[c & 31u]);
            ua[c & 31u] = fmaf(orc_f16_to_f32(us[si]), Au * (1.0f / 7.5f) - X, ua[c & 31u]);
        }
    }
    *g_out = simd_sum32(ga);
    *u_out = simd_sum32(ua);
}

/* mg/mu/md: NULL for SMOE-Q4, else the mins of the scale+min format */
static void expert_ffn_decode_rows(const uint8_t* pg, const uint16_t* sg, const uint16_t* mg, const uint8_t* pu,
                                   const uint16_t* su, const uint16_t* mu, const uint8_t* pd, const uint16_t* sd,
                                   const uint16_t* md, const float* x, float* hidden, float* out, uint32_t d_ff,
                                   uint32_t d_model, uint32_t group)
{
#pragma omp parallel num_threads(g_threads) if (g_threads > 1)
    {
#pragma omp for schedule(static)
        for (uint32_t r = 0; r < d_ff; ++r) {
            float g, u;
            q4_qrow_dot2(pg, sg, mg, pu, su, mu, r, d_model, group, x, &g, &u);
            hidden[r] = orc_silu(g) * u;                   /* kernels.metal:333-335 */
        }
#pragma omp for schedule(static)
        for (uint32_t d = 0; d < d_model; ++d)
            out[d] = q4_qrow_dot(pd, sd, md, d, d_ff, group, hidden);   /* kernels.metal:360-364 */
    }
}

void orc_expert_ffn_decode(const uint8_t* pg, const uint16_t* sg, const uint8_t* pu, const uint16_t* su,
                           const uint8_t* pd, const uint16_t* sd, const float* x, float* hidden, float* out,
                           uint32_t d_ff, uint32_t d_model, uint32_t group)
{
    expert_ffn_decode_rows(pg, sg, NULL, pu, su, NULL, pd, sd, NULL, x, hidden, out, d_ff, d_model, group);
}

void orc_expert_ffn_decode_min(const uint8_t* pg, const uint16_t* sg, const uint16_t* mg, const uint8_t* pu,
                               const uint16_t* su, const uint16_t* mu, const uint8_t* pd, const uint16_t* sd,
                               const uint16_t* md, const float* x, float* hidden, float* out, uint32_t d_ff,
                               uint32_t d_model, uint32_t group)
{
    expert_ffn_decode_rows(pg, sg, mg, pu, su, mu, pd, sd, md, x, hidden, out, d_ff, d_model, group);
}

/* The same FFN with one thread, for callers that already run in parallel. */
static void expert_ffn_serial(const uint8_t* pg, const uint16_t* sg, const uint8_t* pu, const uint16_t* su,
                              const uint8_t* pd, const uint16_t* sd, const float* x, float* hidden, float* out,
                              uint32_t d_ff, uint32_t d_model, uint32_t group)
{
    for (uint32_t r = 0; r < d_ff; ++r) {
        float g = q4_row_dot(pg, sg, r, d_model, group, x);
        float u = q4_row_dot(pu, su, r, d_model, group, x);
        hidden[r] = orc_silu(g) * u;
    }
    for (uint32_t d = 0; d < d_model; ++d) out[d] = q4_row_dot(pd, sd, d, d_ff, group, hidden);
}

/* ------------------------------------------------------------------------ */
/* A11: blob layout (shatter_moe.py:627-674): [gate p][gate s][up p][up s]  */
/* [down p][down s], gate/up [d_ff x d_model], down [d_model x d_ff]         */
/* ------------------------------------------------------------------------ */
void orc_blob_layout(uint32_t d_model, uint32_t d_ff, uint32_t group,
                     uint64_t* off, uint64_t* blob_bytes)
{
    uint64_t n = (uint64_t)d_model * d_ff;
    uint64_t pb = (n + 1) / 2, sb = ((n + group - 1) / group) * 2;
    off[0] = 0;               off[1] = pb;
    off[2] = pb + sb;         off[3] = 2 * pb + sb;
    off[4] = 2 * (pb + sb);   off[5] = 3 * pb + 2 * sb;
    *blob_bytes = 3 * (pb + sb);
}

static void expert_ptrs(const OrcLayer* L, uint32_t e, const uint8_t** pg, const uint16_t** sg,
                        const uint8_t** pu, const uint16_t** su,
                        const uint8_t** pd, const uint16_t** sd)
{
    const uint8_t* b = L->experts + (size_t)e * L->stride;
    *pg = b + L->gate_packed;  *sg = (const uint16_t*)(b + L->gate_scales);
    *pu = b + L->up_packed;    *su = (const uint16_t*)(b + L->up_scales);
    *pd = b + L->down_packed;  *sd = (const uint16_t*)(b + L->down_scales);
}

/* ------------------------------------------------------------------------ */
/* A12: decode MoE block (src/decode.cpp:236-238, 280-302, 338-509)         */
/* ------------------------------------------------------------------------ */
void orc_moe_decode_layer(const OrcShape* s, const OrcLayer* L, float* hidden,
                          uint32_t* ids, float* weights, float* logits_out,
                          float* normed_out, float* expert_out)
{
    const uint32_t D = s->d_model, E = s->n_experts, K = s->top_k, I = s->d_ff;
    float* normed = (float*)malloc(D * sizeof(float));
    float* logits = (float*)malloc(E * sizeof(float));
    float* routed = (float*)calloc(D, sizeof(float));
    float* h = (float*)malloc(I * sizeof(float));
    float* y = (float*)malloc(D * sizeof(float));
    float w[32];
    uint32_t rid[32];

    memcpy(normed, hidden, D * sizeof(float));                 /* :237 */
    orc_rms_norm_bf16(normed, L->norm_w, D);                   /* :238 */
    orc_matvec_bf16(logits, L->router_w, normed, E, D);        /* :280-283 */
    uint32_t nsel = orc_top_k(logits, E, K, rid, w, 0);        /* :290-292 */
    uint32_t nk = nsel < K ? nsel : K;
    float w_sum = 0.0f;
    for (uint32_t e = 0; e < nk; ++e) w_sum += w[e];           /* :296-297 */
    float w_inv = (s->norm_topk && w_sum > 0.0f) ? 1.0f / w_sum : 1.0f;
    for (uint32_t e = 0; e < nk; ++e) w[e] = w[e] * w_inv;     /* :301 */

    for (uint32_t e = 0; e < nk; ++e) {                        /* :482-498 */
        const uint8_t *pg, *pu, *pd; const uint16_t *sg, *su, *sd;
        expert_ptrs(L, rid[e], &pg, &sg, &pu, &su, &pd, &sd);
        if (s->quant) {
            /* scale+min: each matrix's mins follow its D*I/group scales */
            const size_t ng = (size_t)D * I / s->group_size;
            orc_expert_ffn_decode_min(pg, sg, sg + ng, pu, su, su + ng, pd, sd, sd + ng, normed, h, y, I, D,
                                      s->group_size);
        } else {
            orc_expert_ffn_decode(pg, sg, pu, su, pd, sd, normed, h, y, I, D, s->group_size);
        }
        if (expert_out) memcpy(expert_out + (size_t)e * D, y, D * sizeof(float));
        orc_axpy_f32(routed, w[e], y, D);
    }
    for (uint32_t d = 0; d < D; ++d)                           /* :506-509 */
        hidden[d] += 0.0f + routed[d];

    for (uint32_t e = 0; e < nk; ++e) { ids[e] = rid[e]; weights[e] = w[e]; }
    if (logits_out) memcpy(logits_out, logits, E * sizeof(float));
    if (normed_out) memcpy(normed_out, normed, D * sizeof(float));
    free(normed); free(logits); free(routed); free(h); free(y);
}

/* ------------------------------------------------------------------------ */
/* A9: permute (src/prefill.cpp:38-68, 315-332)                              */
/* ------------------------------------------------------------------------ */
#define ORC_CHUNK 64u
#define ORC_MAX_EXPERTS 512u
typedef struct { uint8_t tok[ORC_CHUNK]; float w[ORC_CHUNK]; uint32_t count; } OrcExpertTokens;
static OrcExpertTokens g_elist[ORC_MAX_EXPERTS];
static uint32_t g_union_ids[ORC_MAX_EXPERTS];
static uint32_t g_union_size;

void orc_union_reset(void) { g_union_size = 0; }

int orc_union_add(uint32_t expert, uint32_t tok_row, float weight)
{
    OrcExpertTokens* et = &g_elist[expert];
    int fresh = 1;
    for (uint32_t u = 0; u < g_union_size; ++u)
        if (g_union_ids[u] == expert) { fresh = 0; break; }
    if (fresh) {
        et->count = 0;
        if (g_union_size < ORC_MAX_EXPERTS) g_union_ids[g_union_size++] = expert;
    }
    if (et->count < ORC_CHUNK) {
        et->tok[et->count] = (uint8_t)tok_row;
        et->w[et->count] = weight;
        et->count++;
    }
    return fresh;
}

uint32_t orc_union_size(void) { return g_union_size; }
uint32_t orc_union_id(uint32_t u) { return g_union_ids[u]; }
uint32_t orc_union_count(uint32_t e) { return g_elist[e].count; }
uint32_t orc_union_tok(uint32_t e, uint32_t t) { return g_elist[e].tok[t]; }
float    orc_union_w(uint32_t e, uint32_t t) { return g_elist[e].w[t]; }

uint32_t orc_permute(const uint32_t* ids, const float* w, uint32_t T, uint32_t k,
                     uint32_t n_experts, uint32_t* offsets, uint32_t* tok,
                     float* wout, uint32_t* union_ids)
{
    uint32_t* cnt = (uint32_t*)calloc(n_experts + 1, sizeof(uint32_t));
    uint8_t* seen = (uint8_t*)calloc(n_experts, 1);
    uint32_t nu = 0;
    for (uint32_t p = 0; p < T * k; ++p) {
        uint32_t e = ids[p];
        cnt[e + 1]++;
        if (!seen[e]) { seen[e] = 1; union_ids[nu++] = e; }
    }
    for (uint32_t e = 0; e < n_experts; ++e) cnt[e + 1] += cnt[e];
    memcpy(offsets, cnt, (n_experts + 1) * sizeof(uint32_t));
    for (uint32_t p = 0; p < T * k; ++p) {               /* token-major: stable */
        uint32_t e = ids[p];
        uint32_t dst = cnt[e]++;
        tok[dst] = p / k;
        wout[dst] = w[p];
    }
    free(cnt); free(seen);
    return nu;
}

/* ------------------------------------------------------------------------ */
/* A10: prefill MoE block (src/prefill.cpp:269-276, 308-453), chunks of 64  */
/* ------------------------------------------------------------------------ */
void orc_moe_prefill_layer(const OrcShape* s, const OrcLayer* L, float* hidden,
                           uint32_t T, uint32_t* ids_out, float* w_out)
{
    const uint32_t D = s->d_model, E = s->n_experts, K = s->top_k, I = s->d_ff;
    float* normed = (float*)malloc((size_t)ORC_CHUNK * D * sizeof(float));
    float* routed = (float*)malloc((size_t)ORC_CHUNK * D * sizeof(float));
    float* logits = (float*)malloc(E * sizeof(float));
    const size_t max_pairs = (size_t)ORC_CHUNK * K;
    float* py = (float*)malloc(max_pairs * D * sizeof(float));
    uint32_t* pe = (uint32_t*)malloc(max_pairs * sizeof(uint32_t));
    uint32_t* pt = (uint32_t*)malloc(max_pairs * sizeof(uint32_t));
    float* pw = (float*)malloc(max_pairs * sizeof(float));
    uint32_t tid[32];
    float tw[32];

    for (uint32_t c0 = 0; c0 < T; c0 += ORC_CHUNK) {
        uint32_t B = (T - c0 < ORC_CHUNK) ? T - c0 : ORC_CHUNK;
        for (uint32_t i = 0; i < B; ++i) {                       /* :272-275 */
            memcpy(normed + (size_t)i * D, hidden + (size_t)(c0 + i) * D, D * sizeof(float));
            orc_rms_norm_bf16(normed + (size_t)i * D, L->norm_w, D);
        }
        orc_union_reset();                                       /* :314 */
        memset(routed, 0, (size_t)B * D * sizeof(float));        /* :315 */
        for (uint32_t i = 0; i < B; ++i) {                       /* :319-332 */
            orc_matvec_bf16(logits, L->router_w, normed + (size_t)i * D, E, D);
            uint32_t cnt = orc_top_k(logits, E, K, tid, tw, (int)s->norm_topk);
            for (uint32_t e = 0; e < cnt; ++e) {
                ids_out[(size_t)(c0 + i) * K + e] = tid[e];
                w_out[(size_t)(c0 + i) * K + e] = tw[e];
                if (tid[e] < ORC_MAX_EXPERTS) orc_union_add(tid[e], i, tw[e]);
            }
        }
        /* :339-417: every (expert, token) pair of the chunk, listed in union
         * order; the FFNs are independent (computed in parallel when threads
         * are set), the scatter into routed_out keeps the reference's order */
        uint32_t np_ = 0;
        for (uint32_t u = 0; u < g_union_size; ++u) {
            const OrcExpertTokens* et = &g_elist[g_union_ids[u]];
            for (uint32_t t = 0; t < et->count; ++t) {
                pe[np_] = g_union_ids[u];
                pt[np_] = et->tok[t];
                pw[np_] = et->w[t];
                ++np_;
            }
        }
#pragma omp parallel num_threads(g_threads) if (g_threads > 1)
        {
            float* hh = (float*)malloc(I * sizeof(float));
#pragma omp for schedule(dynamic, 1)
            for (uint32_t p = 0; p < np_; ++p) {
                const uint8_t *pg, *pu, *pd; const uint16_t *sg, *su, *sd;
                expert_ptrs(L, pe[p], &pg, &sg, &pu, &su, &pd, &sd);
                expert_ffn_serial(pg, sg, pu, su, pd, sd, normed + (size_t)pt[p] * D, hh,
                                  py + (size_t)p * D, I, D, s->group_size);
            }
            free(hh);
        }
        for (uint32_t p = 0; p < np_; ++p) {                     /* :380-385 */
            float* ro = routed + (size_t)pt[p] * D;
            const float* y = py + (size_t)p * D;
            const float wt = pw[p];
            for (uint32_t d = 0; d < D; ++d) ro[d] += wt * y[d];
        }
        for (uint32_t i = 0; i < B; ++i) {                       /* :446-451 */
            float* hh = hidden + (size_t)(c0 + i) * D;
            const float* ro = routed + (size_t)i * D;
            for (uint32_t d = 0; d < D; ++d) hh[d] += ro[d];
        }
    }
    free(normed); free(routed); free(logits); free(py); free(pe); free(pt); free(pw);
}

/* ------------------------------------------------------------------------ */
/* F4: decode attention of one token (decode.cpp:150-229, the CPU branch)   */
/* ------------------------------------------------------------------------ */
void orc_attention_layer(const uint16_t* w_q, const uint16_t* w_k, const uint16_t* w_v, const uint16_t* w_o,
                         const uint16_t* q_norm_w, const uint16_t* k_norm_w, const float* rope_cos,
                         const float* rope_sin, const float* normed_in, float* k_cache, float* v_cache,
                         float* o_out, uint32_t d_model, uint32_t head_dim, uint32_t num_heads,
                         uint32_t num_kv_heads, uint32_t slot, uint32_t valid, uint32_t attn_ctx, float scale)
{
    const uint32_t q_dim = num_heads * head_dim, kv_dim = num_kv_heads * head_dim, half = head_dim / 2;
    float* q = (float*)malloc(q_dim * sizeof(float));
    float* k = (float*)malloc(kv_dim * sizeof(float));
    float* v = (float*)malloc(kv_dim * sizeof(float));
    float* att = (float*)calloc(q_dim, sizeof(float));
    float* sc = (float*)malloc((size_t)valid * sizeof(float));
    if (!q || !k || !v || !att || !sc) goto done;
    orc_matvec_bf16(q, w_q, normed_in, q_dim, d_model);                 /* :151-153 */
    orc_matvec_bf16(k, w_k, normed_in, kv_dim, d_model);
    orc_matvec_bf16(v, w_v, normed_in, kv_dim, d_model);
    if (q_norm_w)                                                        /* :156-165 */
        for (uint32_t h = 0; h < num_heads; ++h) orc_rms_norm_bf16(q + h * head_dim, q_norm_w, head_dim);
    if (k_norm_w)
        for (uint32_t h = 0; h < num_kv_heads; ++h) orc_rms_norm_bf16(k + h * head_dim, k_norm_w, head_dim);
    for (uint32_t h = 0; h < num_heads; ++h)                             /* :168-176 */
        for (uint32_t d = 0; d < half; ++d) {
            float* x = q + h * head_dim;
            const float x0 = x[d], x1 = x[d + half];
            x[d] = x0 * rope_cos[d] - x1 * rope_sin[d];
            x[d + half] = x0 * rope_sin[d] + x1 * rope_cos[d];
        }
    for (uint32_t h = 0; h < num_kv_heads; ++h)                          /* :178-186 */
        for (uint32_t d = 0; d < half; ++d) {
            float* x = k + h * head_dim;
            const float x0 = x[d], x1 = x[d + half];
            x[d] = x0 * rope_cos[d] - x1 * rope_sin[d];
            x[d + half] = x0 * rope_sin[d] + x1 * rope_cos[d];
        }
    memcpy(k_cache + (size_t)slot * kv_dim, k, kv_dim * sizeof(float)); /* :189-190 */
    memcpy(v_cache + (size_t)slot * kv_dim, v, kv_dim * sizeof(float));
    for (uint32_t h = 0; h < num_heads; ++h) {                           /* :193-226 */
        const uint32_t kv_h = h / (num_heads / num_kv_heads);
        const float* qh = q + h * head_dim;
        for (uint32_t i = 0; i < valid; ++i) {
            const uint32_t ki = (slot - i + attn_ctx) % attn_ctx;
            const float* kr = k_cache + (size_t)ki * kv_dim + kv_h * head_dim;
            float s = 0.0f;                                              /* dot_f32, common.hpp:339-344 */
            for (uint32_t d = 0; d < head_dim; ++d) s += qh[d] * kr[d];
            sc[i] = s * scale;
        }
        float m = sc[0];
        for (uint32_t i = 1; i < valid; ++i)
            if (sc[i] > m) m = sc[i];
        float sum = 0.0f;
        for (uint32_t i = 0; i < valid; ++i) {
            sc[i] = expf(sc[i] - m);
            sum += sc[i];
        }
        const float inv = sum > 0.0f ? 1.0f / sum : 0.0f;
        for (uint32_t i = 0; i < valid; ++i) sc[i] *= inv;
        for (uint32_t i = 0; i < valid; ++i) {
            const uint32_t vi = (slot - i + attn_ctx) % attn_ctx;
            orc_axpy_f32(att + h * head_dim, sc[i], v_cache + (size_t)vi * kv_dim + kv_h * head_dim, head_dim);
        }
    }
    orc_matvec_bf16(o_out, w_o, att, d_model, q_dim);                   /* :229 */
done:
    free(q);
    free(k);
    free(v);
    free(att);
    free(sc);
}

