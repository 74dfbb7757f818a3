/* cpu_ggml.c - the timed CPU baseline: a CPU restatement of ggml semantics for the Qwen3-MoE block.
 *
 * BENCHMARK INFRASTRUCTURE ONLY (bench.py's cpu_baseline leg and the tests that check it): it is not
 * the product and not the oracle. It restates, for this one path, what the reference's vendored ggml CPU
 * backend computes for router() + moe_apply() + the residual (src/qwen3.cpp:175-214, :250) - ggml at
 * llama.cpp 23b0202a, absent from the reference checkout, so written from its published algorithm:
 *   router       F16 mul_mat (activations rounded to fp16, f32 accumulation), softmax (sum in double),
 *                descending top-k, gather, sum, clamp at 2^-14, divide;
 *   mul_mat_id   for each expert in ascending order its (token, slot) pairs in token-major order; the
 *                activations quantized once per row to the weight type's vec_dot_type (Q8_0 for Q8_0,
 *                Q8_K for Q4_K); integer block dots (Q8_0 x Q8_0: d_w d_x sum q_w q_x per 32; Q4_K x
 *                Q8_K: d_x (d_w sum_j sc_j dot_j - dmin sum_j m_j bsum_j) per 256); work split over
 *                threads by (expert, 16-row block) as ggml's CPU scheduler splits mul_mat rows;
 *   SwiGLU       silu(g) u; the result re-quantized for down; weights; k-way sum in slot order; residual.
 * Integer parts are exact; f32 sums follow this file's SIMD width (AVX-512 VNNI with 512-bit vectors where
 * the host has it, else AVX2), so results equal the oracle's to the MoE tolerance, not bit for bit.
 */
#include <immintrin.h>
#include <math.h>
#include <omp.h>
#include <stdint.h>
#include <stdlib.h>
#include <string.h>

#define QK8_0 32
#define QK_K 256
#define RB 16 /* rows per work item */

typedef struct {
    uint16_t d;
    int8_t qs[QK8_0];
} blk_q8_0;
typedef struct {
    uint16_t d, dmin;
    uint8_t scales[12];
    uint8_t qs[QK_K / 2];
} blk_q4_K;
typedef struct {
    float d;
    int8_t qs[QK_K];
    int16_t bsums[QK_K / 16];
} blk_q8_K;

static inline float h2f(uint16_t h) { return _cvtsh_ss(h); }
static inline uint16_t f2h(float f) { return _cvtss_sh(f, _MM_FROUND_TO_NEAREST_INT); }

static int g_vnni = -1;
static int use_vnni(void) {
    if (g_vnni < 0) {
        __builtin_cpu_init();
        const char *force = getenv("LSTK_CPU_ISA"); /* "avx2": the fallback path even on AVX-512 hosts */
        g_vnni = (!force || strcmp(force, "avx2") != 0) && __builtin_cpu_supports("avx512vnni") &&
                         __builtin_cpu_supports("avx512bw")
                     ? 1
                     : 0;
    }
    return g_vnni;
}
const char *cg_isa(void) { return use_vnni() ? "avx512-vnni" : "avx2"; }

/* ---- activation quantizers (quantize_row_q8_0 x86 path, quantize_row_q8_K_ref) --------------- */

static void quant_q8_0(const float *x, int n, blk_q8_0 *y) {
    for (int i = 0; i < n / QK8_0; i++) {
        float amax = 0.0f;
        for (int j = 0; j < QK8_0; j++) amax = fmaxf(amax, fabsf(x[i * QK8_0 + j]));
        const float id = amax != 0.0f ? 127.0f / amax : 0.0f;
        y[i].d = f2h(amax / 127.0f);
        for (int j = 0; j < QK8_0; j++) y[i].qs[j] = (int8_t) rintf(x[i * QK8_0 + j] * id);
    }
}

static inline int nearest_int(float v) {
    float val = v + 12582912.f;
    int i;
    memcpy(&i, &val, sizeof(int));
    return (i & 0x007fffff) - 0x00400000;
}

static void quant_q8_K(const float *x, int n, blk_q8_K *y) {
    for (int i = 0; i < n / QK_K; i++) {
        const float *xb = x + (size_t) i * QK_K;
        float max = 0.0f, amax = 0.0f;
        for (int j = 0; j < QK_K; j++) {
            const float ax = fabsf(xb[j]);
            if (ax > amax) {
                amax = ax;
                max = xb[j];
            }
        }
        if (amax == 0.0f) {
            memset(&y[i], 0, sizeof(blk_q8_K));
            continue;
        }
        const float iscale = -127.0f / max;
        for (int j = 0; j < QK_K; j++) {
            const int v = nearest_int(iscale * xb[j]);
            y[i].qs[j] = (int8_t) (v < 127 ? v : 127);
        }
        for (int g = 0; g < QK_K / 16; g++) {
            int s = 0;
            for (int l = 0; l < 16; l++) s += y[i].qs[g * 16 + l];
            y[i].bsums[g] = (int16_t) s;
        }
        y[i].d = 1.0f / iscale;
    }
}

/* ---- block dot products ------------------------------------------------------------------------ */

__attribute__((target("avx512f,avx512bw,avx512vnni,avx512vl"))) static float dot_q8_0_vnni(const blk_q8_0 *w,
                                                                                         const blk_q8_0 *x, int nb) {
    __m512 acc = _mm512_setzero_ps();
    const __m512i zero = _mm512_setzero_si512();
    int i = 0;
    for (; i + 1 < nb; i += 2) {
        const __m512i wv = _mm512_inserti64x4(_mm512_castsi256_si512(_mm256_loadu_si256((const __m256i *) w[i].qs)),
                                              _mm256_loadu_si256((const __m256i *) w[i + 1].qs), 1);
        const __m512i xv = _mm512_inserti64x4(_mm512_castsi256_si512(_mm256_loadu_si256((const __m256i *) x[i].qs)),
                                              _mm256_loadu_si256((const __m256i *) x[i + 1].qs), 1);
        /* u8 x s8: |w| against x carrying w's sign */
        const __mmask64 neg = _mm512_movepi8_mask(wv);
        const __m512i xs = _mm512_mask_sub_epi8(xv, neg, zero, xv);
        const __m512i s = _mm512_dpbusd_epi32(zero, _mm512_abs_epi8(wv), xs);
        const float d0 = h2f(w[i].d) * h2f(x[i].d), d1 = h2f(w[i + 1].d) * h2f(x[i + 1].d);
        const __m512 dv = _mm512_mask_blend_ps((__mmask16) 0xFF00, _mm512_set1_ps(d0), _mm512_set1_ps(d1));
        acc = _mm512_fmadd_ps(_mm512_cvtepi32_ps(s), dv, acc);
    }
    float r = _mm512_reduce_add_ps(acc);
    for (; i < nb; i++) {
        int s = 0;
        for (int j = 0; j < QK8_0; j++) s += w[i].qs[j] * x[i].qs[j];
        r += (float) s * (h2f(w[i].d) * h2f(x[i].d));
    }
    return r;
}

__attribute__((target("avx2,fma"))) static float dot_q8_0_avx2(const blk_q8_0 *w, const blk_q8_0 *x, int nb) {
    __m256 acc = _mm256_setzero_ps();
    const __m256i ones = _mm256_set1_epi16(1);
    for (int i = 0; i < nb; i++) {
        const __m256i wv = _mm256_loadu_si256((const __m256i *) w[i].qs);
        const __m256i xv = _mm256_loadu_si256((const __m256i *) x[i].qs);
        const __m256i p = _mm256_maddubs_epi16(_mm256_sign_epi8(wv, wv), _mm256_sign_epi8(xv, wv));
        const __m256 s = _mm256_cvtepi32_ps(_mm256_madd_epi16(p, ones));
        acc = _mm256_fmadd_ps(s, _mm256_set1_ps(h2f(w[i].d) * h2f(x[i].d)), acc);
    }
    const __m128 h = _mm_add_ps(_mm256_castps256_ps128(acc), _mm256_extractf128_ps(acc, 1));
    const __m128 h2 = _mm_add_ps(h, _mm_movehl_ps(h, h));
    return _mm_cvtss_f32(_mm_add_ss(h2, _mm_shuffle_ps(h2, h2, 1)));
}

static inline void scale_min_k4(int j, const uint8_t *q, int *sc, int *m) {
    if (j < 4) {
        *sc = q[j] & 63;
        *m = q[j + 4] & 63;
    } else {
        *sc = (q[j + 4] & 0xF) | ((q[j - 4] >> 6) << 4);
        *m = (q[j + 4] >> 4) | ((q[j] >> 6) << 4);
    }
}

__attribute__((target("avx512f,avx512bw,avx512vnni,avx512vl"))) static float dot_q4_K_vnni(const blk_q4_K *w,
                                                                                         const blk_q8_K *x, int nb) {
    float acc = 0.0f;
    const __m512i zero = _mm512_setzero_si512();
    const __m256i m4 = _mm256_set1_epi8(0x0F);
    for (int i = 0; i < nb; i++) {
        int sc[8], mn[8];
        for (int j = 0; j < 8; j++) scale_min_k4(j, w[i].scales, &sc[j], &mn[j]);
        __m512i isum = zero;
        for (int c = 0; c < 4; c++) {
            const __m256i q4 = _mm256_loadu_si256((const __m256i *) (w[i].qs + 32 * c));
            const __m512i q = _mm512_inserti64x4(_mm512_castsi256_si512(_mm256_and_si256(q4, m4)),
                                                 _mm256_and_si256(_mm256_srli_epi16(q4, 4), m4), 1);
            const __m512i s = _mm512_dpbusd_epi32(zero, q, _mm512_loadu_si512((const void *) (x[i].qs + 64 * c)));
            const __m512i scv = _mm512_inserti64x4(_mm512_castsi256_si512(_mm256_set1_epi32(sc[2 * c])),
                                                   _mm256_set1_epi32(sc[2 * c + 1]), 1);
            isum = _mm512_add_epi32(isum, _mm512_mullo_epi32(s, scv));
        }
        int imin = 0;
        for (int j = 0; j < 8; j++) imin += mn[j] * (x[i].bsums[2 * j] + x[i].bsums[2 * j + 1]);
        const float dx = x[i].d;
        acc += (h2f(w[i].d) * dx) * (float) _mm512_reduce_add_epi32(isum);
        acc -= (h2f(w[i].dmin) * dx) * (float) imin;
    }
    return acc;
}

__attribute__((target("avx2,fma"))) static float dot_q4_K_avx2(const blk_q4_K *w, const blk_q8_K *x, int nb) {
    float acc = 0.0f;
    const __m256i m4 = _mm256_set1_epi8(0x0F);
    for (int i = 0; i < nb; i++) {
        int sc[8], mn[8];
        for (int j = 0; j < 8; j++) scale_min_k4(j, w[i].scales, &sc[j], &mn[j]);
        __m256i isum = _mm256_setzero_si256();
        for (int c = 0; c < 4; c++) {
            const __m256i q4 = _mm256_loadu_si256((const __m256i *) (w[i].qs + 32 * c));
            const __m256i lo = _mm256_and_si256(q4, m4), hi = _mm256_and_si256(_mm256_srli_epi16(q4, 4), m4);
            const __m256i pl = _mm256_madd_epi16(_mm256_maddubs_epi16(lo, _mm256_loadu_si256((const __m256i *) (x[i].qs + 64 * c))),
                                                 _mm256_set1_epi16((short) sc[2 * c]));
            const __m256i ph = _mm256_madd_epi16(_mm256_maddubs_epi16(hi, _mm256_loadu_si256((const __m256i *) (x[i].qs + 64 * c + 32))),
                                                 _mm256_set1_epi16((short) sc[2 * c + 1]));
            isum = _mm256_add_epi32(isum, _mm256_add_epi32(pl, ph));
        }
        const __m128i h = _mm_add_epi32(_mm256_castsi256_si128(isum), _mm256_extracti128_si256(isum, 1));
        const __m128i h2 = _mm_add_epi32(h, _mm_shuffle_epi32(h, 0x4E));
        const int is = _mm_cvtsi128_si32(_mm_add_epi32(h2, _mm_shuffle_epi32(h2, 0xB1)));
        int imin = 0;
        for (int j = 0; j < 8; j++) imin += mn[j] * (x[i].bsums[2 * j] + x[i].bsums[2 * j + 1]);
        const float dx = x[i].d;
        acc += (h2f(w[i].d) * dx) * (float) is;
        acc -= (h2f(w[i].dmin) * dx) * (float) imin;
    }
    return acc;
}

/* one weight row (Q8_0: n/32 blocks, Q4_K: n/256) against one quantized activation row */
static inline float dot_row(int wtype, const void *w, const void *x, int n) {
    if (wtype == 8) return use_vnni() ? dot_q8_0_vnni(w, x, n / QK8_0) : dot_q8_0_avx2(w, x, n / QK8_0);
    return use_vnni() ? dot_q4_K_vnni(w, x, n / QK_K) : dot_q4_K_avx2(w, x, n / QK_K);
}

static size_t row_bytes(int type, int n) { return type == 8 ? (size_t) n / QK8_0 * sizeof(blk_q8_0) : (size_t) n / QK_K * sizeof(blk_q4_K); }
static size_t act_row_bytes(int wtype, int n) {
    return wtype == 8 ? (size_t) n / QK8_0 * sizeof(blk_q8_0) : (size_t) n / QK_K * sizeof(blk_q8_K);
}
static void quant_act(int wtype, const float *x, int n, void *out) {
    if (wtype == 8) quant_q8_0(x, n, (blk_q8_0 *) out);
    else quant_q8_K(x, n, (blk_q8_K *) out);
}

/* F16 x fp16(activation) dot in f32 */
__attribute__((target("avx2,fma,f16c"))) static float dot_f16(const uint16_t *w, const uint16_t *x, int n) {
    __m256 a0 = _mm256_setzero_ps(), a1 = _mm256_setzero_ps();
    int i = 0;
    for (; i + 16 <= n; i += 16) {
        a0 = _mm256_fmadd_ps(_mm256_cvtph_ps(_mm_loadu_si128((const __m128i *) (w + i))),
                             _mm256_cvtph_ps(_mm_loadu_si128((const __m128i *) (x + i))), a0);
        a1 = _mm256_fmadd_ps(_mm256_cvtph_ps(_mm_loadu_si128((const __m128i *) (w + i + 8))),
                             _mm256_cvtph_ps(_mm_loadu_si128((const __m128i *) (x + i + 8))), a1);
    }
    const __m256 a = _mm256_add_ps(a0, a1);
    const __m128 h = _mm_add_ps(_mm256_castps256_ps128(a), _mm256_extractf128_ps(a, 1));
    const __m128 h2 = _mm_add_ps(h, _mm_movehl_ps(h, h));
    float r = _mm_cvtss_f32(_mm_add_ss(h2, _mm_shuffle_ps(h2, h2, 1)));
    for (; i < n; i++) r += h2f(w[i]) * h2f(x[i]);
    return r;
}

/* ---- the MoE block ------------------------------------------------------------------------------ */

/* router() + moe_apply() + residual for T tokens: hnorm [T][h] f32, gate_inp F16 [E][h], experts stacked
 * [E][f][h] (up, gate) and [E][h][f] (down) as GGUF blocks of wtype (8 = Q8_0, 12 = Q4_K); out [T][h]
 * (may alias resid); ids / weights [T][k] receive the routing. Returns 0, or -1 on a bad argument. */
int cg_moe_block(const float *hnorm, int T, int h, int f, int E, int k, const uint16_t *gate_inp, const void *up,
                 const void *gate, const void *down, int wtype, const float *resid, float *out, int32_t *ids,
                 float *weights, int n_threads) {
    if (T < 1 || k < 1 || k > E || (wtype != 8 && wtype != 12) || h % QK_K || f % QK_K) return -1;
    if (n_threads < 1) n_threads = omp_get_max_threads();
    /* router */
    uint16_t *xh = malloc(sizeof(uint16_t) * (size_t) T * h);
    float *logits = malloc(sizeof(float) * (size_t) T * E);
    for (size_t i = 0; i < (size_t) T * h; i++) xh[i] = f2h(hnorm[i]);
#pragma omp parallel for collapse(2) schedule(static) num_threads(n_threads)
    for (int t = 0; t < T; t++)
        for (int e = 0; e < E; e++) logits[(size_t) t * E + e] = dot_f16(gate_inp + (size_t) e * h, xh + (size_t) t * h, h);
    for (int t = 0; t < T; t++) {
        const float *l = logits + (size_t) t * E;
        float mx = -INFINITY;
        for (int e = 0; e < E; e++) mx = fmaxf(mx, l[e]);
        double s = 0.0;
        float p[512];
        for (int e = 0; e < E; e++) {
            p[e] = expf(l[e] - mx);
            s += p[e];
        }
        const float inv = (float) (1.0 / s);
        for (int e = 0; e < E; e++) p[e] *= inv;
        unsigned char taken[512] = {0};
        double ssum = 0.0;
        for (int j = 0; j < k; j++) { /* descending, ties to the lower id */
            int best = -1;
            for (int e = 0; e < E; e++)
                if (!taken[e] && (best < 0 || l[e] > l[best])) best = e;
            taken[best] = 1;
            ids[(size_t) t * k + j] = best;
            weights[(size_t) t * k + j] = p[best];
            ssum += p[best];
        }
        const float sf = fmaxf((float) ssum, 6.103515625e-5f);
        for (int j = 0; j < k; j++) weights[(size_t) t * k + j] /= sf;
    }
    free(xh);
    free(logits);
    /* mul_mat_id grouping: each expert's pairs in token-major order */
    const int np = T * k;
    int *cnt = calloc((size_t) E + 1, sizeof(int)), *off = calloc((size_t) E + 1, sizeof(int)), *pairs = malloc(sizeof(int) * np);
    for (int p = 0; p < np; p++) cnt[ids[p]]++;
    for (int e = 0; e < E; e++) off[e + 1] = off[e] + cnt[e];
    memset(cnt, 0, sizeof(int) * (size_t) E);
    for (int p = 0; p < np; p++) pairs[off[ids[p]] + cnt[ids[p]]++] = p;
    /* activations quantized once per token */
    const size_t xrb = act_row_bytes(wtype, h), arb = act_row_bytes(wtype, f);
    uint8_t *xq = malloc(xrb * (size_t) T);
    for (int t = 0; t < T; t++) quant_act(wtype, hnorm + (size_t) t * h, h, xq + xrb * t);
    /* gate / up + SwiGLU over (expert, 16-row block) items */
    const size_t rbu = row_bytes(wtype, h), rbd = row_bytes(wtype, f);
    float *act = malloc(sizeof(float) * (size_t) np * f);
    int *items = malloc(sizeof(int) * 2 * (size_t) E * ((h > f ? h : f) / RB + 1));
    int ni = 0;
    for (int e = 0; e < E; e++)
        if (off[e + 1] > off[e])
            for (int r0 = 0; r0 < f; r0 += RB) {
                items[2 * ni] = e;
                items[2 * ni + 1] = r0;
                ni++;
            }
#pragma omp parallel for schedule(dynamic, 1) num_threads(n_threads)
    for (int it = 0; it < ni; it++) {
        const int e = items[2 * it], r0 = items[2 * it + 1];
        const uint8_t *gb = (const uint8_t *) gate + ((size_t) e * f + r0) * rbu, *ub = (const uint8_t *) up + ((size_t) e * f + r0) * rbu;
        for (int q = off[e]; q < off[e + 1]; q++) {
            const int p = pairs[q];
            const uint8_t *xr = xq + xrb * (size_t) (p / k);
            for (int r = 0; r < RB; r++) {
                const float g = dot_row(wtype, gb + rbu * r, xr, h), u = dot_row(wtype, ub + rbu * r, xr, h);
                act[(size_t) p * f + r0 + r] = (g / (1.0f + expf(-g))) * u;
            }
        }
    }
    uint8_t *aq = malloc(arb * (size_t) np);
#pragma omp parallel for schedule(static) num_threads(n_threads)
    for (int p = 0; p < np; p++) quant_act(wtype, act + (size_t) p * f, f, aq + arb * p);
    /* down + router weight */
    float *y = malloc(sizeof(float) * (size_t) np * h);
    ni = 0;
    for (int e = 0; e < E; e++)
        if (off[e + 1] > off[e])
            for (int r0 = 0; r0 < h; r0 += RB) {
                items[2 * ni] = e;
                items[2 * ni + 1] = r0;
                ni++;
            }
#pragma omp parallel for schedule(dynamic, 1) num_threads(n_threads)
    for (int it = 0; it < ni; it++) {
        const int e = items[2 * it], r0 = items[2 * it + 1];
        const uint8_t *db = (const uint8_t *) down + ((size_t) e * h + r0) * rbd;
        for (int q = off[e]; q < off[e + 1]; q++) {
            const int p = pairs[q];
            for (int r = 0; r < RB; r++) y[(size_t) p * h + r0 + r] = dot_row(wtype, db + rbd * r, aq + arb * p, f) * weights[p];
        }
    }
    /* k-way sum in slot order, then the residual */
    for (int t = 0; t < T; t++)
        for (int i = 0; i < h; i++) {
            float acc = y[(size_t) t * k * h + i];
            for (int j = 1; j < k; j++) acc = acc + y[((size_t) t * k + j) * h + i];
            out[(size_t) t * h + i] = acc + resid[(size_t) t * h + i];
        }
    free(cnt);
    free(off);
    free(pairs);
    free(xq);
    free(act);
    free(items);
    free(aq);
    free(y);
    return 0;
}
