/* oracle.c - CPU oracle for the Qwen3-MoE expert-FFN path (test infrastructure only).
 *
 * See lstk_oracle.h for scope, what is restated from where, and what stays unpinned.
 * ggml functions cited below are from the llama.cpp submodule pinned at 23b0202a (absent from the
 * reference checkout); they are restated from ggml's published source, not copied.
 * Build: oracle/Makefile (gcc -O3 -fopenmp -ffp-contract=off: no fused multiply-adds except the
 * explicit fmaf calls, so the evaluation order written here is the order executed).
 */
#include "lstk_oracle.h"

#include <immintrin.h>
#include <math.h>
#include <stdio.h>
#include <stdlib.h>
#include <string.h>

/* ------------------------------------------------------------------------------------------ */
/* fp16                                                                                        */
/* ------------------------------------------------------------------------------------------ */

uint16_t or_fp32_to_fp16(float f) {
    uint32_t x;
    memcpy(&x, &f, 4);
    const uint32_t sign = (x >> 16) & 0x8000u;
    const uint32_t a = x & 0x7fffffffu;
    if (a >= 0x7f800000u) return (uint16_t) (sign | 0x7c00u | (a > 0x7f800000u ? 0x200u : 0u));
    if (a >= 0x47800000u) return (uint16_t) (sign | 0x7c00u); /* >= 65536: overflow */
    if (a < 0x38800000u) {                                     /* below the smallest normal 2^-14 */
        if (a < 0x33000000u) return (uint16_t) sign;            /* < 2^-25 rounds to zero */
        const uint32_t e = a >> 23;
        const uint32_t m = (a & 0x7fffffu) | 0x800000u;
        const uint32_t shift = 126u - e; /* value / 2^-24 = m >> shift */
        uint32_t q = m >> shift;
        const uint32_t rem = m & ((1u << shift) - 1u);
        const uint32_t half = 1u << (shift - 1u);
        if (rem > half || (rem == half && (q & 1u))) q++;
        return (uint16_t) (sign | q);
    }
    uint32_t q = ((((a >> 23) - 112u)) << 10) | ((a & 0x7fffffu) >> 13);
    const uint32_t rem = a & 0x1fffu;
    if (rem > 0x1000u || (rem == 0x1000u && (q & 1u))) q++; /* a carry into the exponent is correct */
    return (uint16_t) (sign | q);
}

float or_fp16_to_fp32(uint16_t h) {
    const uint32_t sign = ((uint32_t) h & 0x8000u) << 16;
    const uint32_t e = (h >> 10) & 0x1fu;
    const uint32_t m = h & 0x3ffu;
    uint32_t x;
    if (e == 0) {
        if (m == 0) {
            x = sign;
        } else { /* subnormal: m * 2^-24 */
            float v = (float) m * (1.0f / 16777216.0f);
            memcpy(&x, &v, 4);
            x |= sign;
        }
    } else if (e == 31) {
        x = sign | 0x7f800000u | (m << 13);
    } else {
        x = sign | ((e + 112u) << 23) | (m << 13);
    }
    float f;
    memcpy(&f, &x, 4);
    return f;
}

static inline float h2f(uint16_t h) { return or_fp16_to_fp32(h); }

/* ------------------------------------------------------------------------------------------ */
/* block formats                                                                               */
/* ------------------------------------------------------------------------------------------ */

size_t or_row_bytes(int type, int n) {
    switch (type) {
        case 0: return (size_t) n * 4;
        case 1: return (size_t) n * 2;
        case 8: return (size_t) (n / OR_QK8_0) * sizeof(or_block_q8_0);
        case 10: return (size_t) (n / OR_QK_K) * sizeof(or_block_q2_K);
        case 11: return (size_t) (n / OR_QK_K) * sizeof(or_block_q3_K);
        case 12: return (size_t) (n / OR_QK_K) * sizeof(or_block_q4_K);
        case 13: return (size_t) (n / OR_QK_K) * sizeof(or_block_q5_K);
        case 14: return (size_t) (n / OR_QK_K) * sizeof(or_block_q6_K);
        case 15: return (size_t) (n / OR_QK_K) * sizeof(or_block_q8_K);
        default: return 0;
    }
}

/* ggml-quants.c quantize_row_q8_0_ref: d = amax/127 (stored fp16), id = 1/d, q = roundf(x*id). */
void or_quantize_q8_0_ref(const float *x, int n, void *out) {
    or_block_q8_0 *y = (or_block_q8_0 *) out;
    for (int i = 0; i < n / OR_QK8_0; i++) {
        float amax = 0.0f;
        for (int j = 0; j < OR_QK8_0; j++) amax = fmaxf(amax, fabsf(x[i * OR_QK8_0 + j]));
        const float d = amax / 127.0f;
        const float id = d != 0.0f ? 1.0f / d : 0.0f;
        y[i].d = or_fp32_to_fp16(d);
        for (int j = 0; j < OR_QK8_0; j++) y[i].qs[j] = (int8_t) roundf(x[i * OR_QK8_0 + j] * id);
    }
}

/* ggml-cpu/arch/x86/quants.c quantize_row_q8_0 (AVX2/AVX-512 path, what ggml runs on x86 hosts):
 * d = amax/127 (stored fp16), id = 127/amax, q = round-half-even(x*id). The x86 path is chosen
 * because the CPU it is compared on is x86. */
void or_quantize_q8_0_act(const float *x, int n, void *out) {
    or_block_q8_0 *y = (or_block_q8_0 *) out;
    for (int i = 0; i < n / OR_QK8_0; i++) {
        float amax = 0.0f;
        for (int j = 0; j < OR_QK8_0; j++) amax = fmaxf(amax, fabsf(x[i * OR_QK8_0 + j]));
        const float d = amax / 127.0f;
        const float id = amax != 0.0f ? 127.0f / amax : 0.0f;
        y[i].d = or_fp32_to_fp16(d);
        for (int j = 0; j < OR_QK8_0; j++) y[i].qs[j] = (int8_t) rintf(x[i * OR_QK8_0 + j] * id);
    }
}

/* ggml-quants.c nearest_int: round half to even by adding 1.5 * 2^23. */
static inline int nearest_int(float fval) {
    float val = fval + 12582912.0f;
    int i;
    memcpy(&i, &val, 4);
    return (i & 0x007fffff) - 0x00400000;
}

/* ggml-quants.c quantize_row_q8_K_ref: max = the signed value of the first element with the
 * largest magnitude, iscale = -127/max, q = min(127, nearest_int(iscale*x)), d = 1/iscale,
 * bsums = sums of 16-value groups. */
void or_quantize_q8_K(const float *x, int n, void *out) {
    or_block_q8_K *y = (or_block_q8_K *) out;
    for (int i = 0; i < n / OR_QK_K; i++) {
        const float *xb = x + (size_t) i * OR_QK_K;
        float max = 0.0f, amax = 0.0f;
        for (int j = 0; j < OR_QK_K; j++) {
            const float ax = fabsf(xb[j]);
            if (ax > amax) {
                amax = ax;
                max = xb[j];
            }
        }
        if (amax == 0.0f) {
            y[i].d = 0.0f;
            memset(y[i].qs, 0, sizeof(y[i].qs));
            memset(y[i].bsums, 0, sizeof(y[i].bsums));
            continue;
        }
        const float iscale = -127.0f / max;
        for (int j = 0; j < OR_QK_K; j++) {
            const int v = nearest_int(iscale * xb[j]);
            y[i].qs[j] = (int8_t) (v < 127 ? v : 127);
        }
        for (int g = 0; g < OR_QK_K / 16; g++) {
            int s = 0;
            for (int l = 0; l < 16; l++) s += y[i].qs[g * 16 + l];
            y[i].bsums[g] = (int16_t) s;
        }
        y[i].d = 1.0f / iscale;
    }
}

void or_dequant_q8_0(const void *in, int n, float *y) {
    const or_block_q8_0 *b = (const or_block_q8_0 *) in;
    for (int i = 0; i < n / OR_QK8_0; i++) {
        const float d = h2f(b[i].d);
        for (int j = 0; j < OR_QK8_0; j++) y[i * OR_QK8_0 + j] = d * (float) b[i].qs[j];
    }
}

void or_dequant_q8_K(const void *in, int n, float *y) {
    const or_block_q8_K *b = (const or_block_q8_K *) in;
    for (int i = 0; i < n / OR_QK_K; i++)
        for (int j = 0; j < OR_QK_K; j++) y[i * OR_QK_K + j] = b[i].d * (float) b[i].qs[j];
}

/* ggml-quants.c get_scale_min_k4: 6-bit scale and min of sub-block j from the 12 packed bytes. */
void or_q4_K_scale_min(int j, const uint8_t *q, uint8_t *sc, uint8_t *m) {
    if (j < 4) {
        *sc = q[j] & 63;
        *m = q[j + 4] & 63;
    } else {
        *sc = (uint8_t) ((q[j + 4] & 0xF) | ((q[j - 4] >> 6) << 4));
        *m = (uint8_t) ((q[j + 4] >> 4) | ((q[j] >> 6) << 4));
    }
}

/* ggml-quants.c dequantize_row_q4_K: chunk c of 64 values uses qs[32c..32c+32): low nibbles are
 * sub-block 2c, high nibbles sub-block 2c+1; value = d*sc*q - dmin*m. */
void or_dequant_q4_K(const void *in, int n, float *y) {
    const or_block_q4_K *b = (const or_block_q4_K *) in;
    for (int i = 0; i < n / OR_QK_K; i++) {
        const float d = h2f(b[i].d), dmin = h2f(b[i].dmin);
        const uint8_t *q = b[i].qs;
        for (int c = 0; c < 4; c++) {
            uint8_t sc, m;
            or_q4_K_scale_min(2 * c, b[i].scales, &sc, &m);
            const float d1 = d * sc, m1 = dmin * m;
            or_q4_K_scale_min(2 * c + 1, b[i].scales, &sc, &m);
            const float d2 = d * sc, m2 = dmin * m;
            float *yy = y + (size_t) i * OR_QK_K + 64 * c;
            for (int l = 0; l < 32; l++) yy[l] = d1 * (float) (q[32 * c + l] & 0xF) - m1;
            for (int l = 0; l < 32; l++) yy[32 + l] = d2 * (float) (q[32 * c + l] >> 4) - m2;
        }
    }
}

/* ggml_vec_dot_q8_0_q8_0 (generic): per block an exact int32 sum, then
 * sumf += sumi * (d_w * d_x), blocks in ascending order. */
float or_vec_dot_q8_0_q8_0(int n, const void *w, const void *x) {
    const or_block_q8_0 *a = (const or_block_q8_0 *) w;
    const or_block_q8_0 *b = (const or_block_q8_0 *) x;
    float sumf = 0.0f;
    for (int i = 0; i < n / OR_QK8_0; i++) {
        int sumi = 0;
        for (int j = 0; j < OR_QK8_0; j++) sumi += (int) a[i].qs[j] * (int) b[i].qs[j];
        sumf += (float) sumi * (h2f(a[i].d) * h2f(b[i].d));
    }
    return sumf;
}

/* ggml_vec_dot_q4_K_q8_K (generic): per super-block, isum = sum_j sc_j * (int dot of sub-block j),
 * imin = sum_j m_j * (bsums[2j] + bsums[2j+1]);
 * sumf += (d_w*d_x) * isum, then sumf -= (dmin_w*d_x) * imin, super-blocks in ascending order. */
float or_vec_dot_q4_K_q8_K(int n, const void *w, const void *x) {
    const or_block_q4_K *a = (const or_block_q4_K *) w;
    const or_block_q8_K *b = (const or_block_q8_K *) x;
    float sumf = 0.0f;
    for (int i = 0; i < n / OR_QK_K; i++) {
        int isum = 0, imin = 0;
        for (int c = 0; c < 4; c++) {
            int lo = 0, hi = 0;
            for (int l = 0; l < 32; l++) {
                lo += (int) (a[i].qs[32 * c + l] & 0xF) * (int) b[i].qs[64 * c + l];
                hi += (int) (a[i].qs[32 * c + l] >> 4) * (int) b[i].qs[64 * c + 32 + l];
            }
            uint8_t sc, m;
            or_q4_K_scale_min(2 * c, a[i].scales, &sc, &m);
            isum += sc * lo;
            imin += m * (b[i].bsums[4 * c] + b[i].bsums[4 * c + 1]);
            or_q4_K_scale_min(2 * c + 1, a[i].scales, &sc, &m);
            isum += sc * hi;
            imin += m * (b[i].bsums[4 * c + 2] + b[i].bsums[4 * c + 3]);
        }
        sumf += (h2f(a[i].d) * b[i].d) * (float) isum;
        sumf -= (h2f(a[i].dmin) * b[i].d) * (float) imin;
    }
    return sumf;
}

/* ---- Q2_K, Q3_K, Q5_K, Q6_K ---------------------------------------------------------------- */

/* The 16 6-bit scales of a Q3_K block (dequantize_row_q3_K's kmask unpacking): scale i = 4a + b has
 * low 4 bits from byte 4a + b (a < 2) or the high nibble of byte 4(a - 2) + b, and high 2 bits from
 * bits 2a, 2a + 1 of byte 8 + b; the result is that 6-bit value - 32. */
static int q3_K_scale(const uint8_t *s, int i) {
    const int a = i / 4, b = i % 4;
    const int lo = a < 2 ? s[4 * a + b] & 0xF : s[4 * (a - 2) + b] >> 4;
    const int hi = (s[8 + b] >> (2 * a)) & 3;
    return (lo | hi << 4) - 32;
}

/* Each k-quant block as 256 integer quants, 16 integer scales and 16 mins (one per 16 values) and the
 * block's d / dmin, so that value v = (d * sc[v / 16]) * q[v] - dmin * m[v / 16] is ggml's dequantized
 * value, and ggml's dot with a Q8_K block is (d * d_x) * sum_j sc_j * dot_j - (dmin * d_x) * sum_j
 * m_j * bsums_j in integers per super-block. Layouts (ggml-common.h):
 *   Q2_K  value 128 n + 32 j + l (n < 2, j < 4, l < 32): bits 2j of qs[32 n + l]; scales[8 n + 2 j + l / 16]
 *         holds sc (low nibble) and m (high nibble).
 *   Q3_K  same 2-bit layout; the third bit is bit 4 n + j of hmask[l], and a clear bit subtracts 4;
 *         scale q3_K_scale(), no mins.
 *   Q5_K  Q4_K's nibbles and 6-bit scale / min pairs per 32 values; bit 2 c + h of qh[l] (value
 *         64 c + 32 h + l) adds 16.
 *   Q6_K  value 128 n + 32 j + l: the low (j < 2) or high (j >= 2) nibble of ql[64 n + 32 (j % 2) + l]
 *         and bits 2j, 2j + 1 of qh[32 n + l], minus 32; int8 scale per 16 values, no mins. */
typedef struct {
    float d, dmin;
    int sc[16], m[16];
    int q[256];
} or_kblock;

static void k_unpack(int type, const void *blk, or_kblock *o) {
    memset(o, 0, sizeof(*o));
    if (type == 10) {
        const or_block_q2_K *b = (const or_block_q2_K *) blk;
        o->d = h2f(b->d);
        o->dmin = h2f(b->dmin);
        for (int i = 0; i < 16; i++) {
            o->sc[i] = b->scales[i] & 0xF;
            o->m[i] = b->scales[i] >> 4;
        }
        for (int v = 0; v < 256; v++) {
            const int n = v / 128, j = (v % 128) / 32, l = v % 32;
            o->q[v] = (b->qs[32 * n + l] >> (2 * j)) & 3;
        }
    } else if (type == 11) {
        const or_block_q3_K *b = (const or_block_q3_K *) blk;
        o->d = h2f(b->d);
        for (int i = 0; i < 16; i++) o->sc[i] = q3_K_scale(b->scales, i);
        for (int v = 0; v < 256; v++) {
            const int n = v / 128, j = (v % 128) / 32, l = v % 32;
            o->q[v] = ((b->qs[32 * n + l] >> (2 * j)) & 3) - (((b->hmask[l] >> (4 * n + j)) & 1) ? 0 : 4);
        }
    } else if (type == 13) {
        const or_block_q5_K *b = (const or_block_q5_K *) blk;
        o->d = h2f(b->d);
        o->dmin = h2f(b->dmin);
        for (int j = 0; j < 8; j++) {
            uint8_t sc, m;
            or_q4_K_scale_min(j, b->scales, &sc, &m);
            o->sc[2 * j] = o->sc[2 * j + 1] = sc;
            o->m[2 * j] = o->m[2 * j + 1] = m;
        }
        for (int v = 0; v < 256; v++) {
            const int c = v / 64, h = (v % 64) / 32, l = v % 32;
            const int nib = h ? b->qs[32 * c + l] >> 4 : b->qs[32 * c + l] & 0xF;
            o->q[v] = nib + (((b->qh[l] >> (2 * c + h)) & 1) ? 16 : 0);
        }
    } else { /* 14 */
        const or_block_q6_K *b = (const or_block_q6_K *) blk;
        o->d = h2f(b->d);
        for (int i = 0; i < 16; i++) o->sc[i] = b->scales[i];
        for (int v = 0; v < 256; v++) {
            const int n = v / 128, j = (v % 128) / 32, l = v % 32;
            const int lo = (b->ql[64 * n + 32 * (j % 2) + l] >> (4 * (j / 2))) & 0xF;
            const int hi = (b->qh[32 * n + l] >> (2 * j)) & 3;
            o->q[v] = (lo | hi << 4) - 32;
        }
    }
}

static size_t k_block_bytes(int type) { return or_row_bytes(type, OR_QK_K); }

/* dequantize_row_q2_K / q3_K / q5_K / q6_K: (d * sc) * q - dmin * m, each product rounded in f32 as ggml
 * forms it (dl = d * sc, ml = dmin * m, y = dl * q - ml; the types without mins subtract nothing). */
void or_dequant_k(int type, const void *in, int n, float *y) {
    or_kblock k;
    for (int i = 0; i < n / OR_QK_K; i++) {
        k_unpack(type, (const uint8_t *) in + (size_t) i * k_block_bytes(type), &k);
        for (int v = 0; v < 256; v++) {
            const float dl = k.d * (float) k.sc[v / 16];
            const float yv = dl * (float) k.q[v];
            y[(size_t) i * OR_QK_K + v] = (type == 10 || type == 13) ? yv - k.dmin * (float) k.m[v / 16] : yv;
        }
    }
}

/* ggml_vec_dot_q2_K_q8_K / q3_K / q5_K / q6_K (generic): per super-block the integer isum = sum_j sc_j *
 * (sum of q * x over the 16 values of j) and imin = sum_j m_j * bsums_j; sumf += (d * d_x) * isum, then
 * sumf -= (dmin * d_x) * imin; super-blocks in ascending order. ggml's own float order within a block
 * differs by type (per-lane partial sums); the integers are exact either way. */
float or_vec_dot_k_q8_K(int type, int n, const void *w, const void *x) {
    const or_block_q8_K *b = (const or_block_q8_K *) x;
    float sumf = 0.0f;
    or_kblock k;
    for (int i = 0; i < n / OR_QK_K; i++) {
        k_unpack(type, (const uint8_t *) w + (size_t) i * k_block_bytes(type), &k);
        int isum = 0, imin = 0;
        for (int j = 0; j < 16; j++) {
            int s = 0;
            for (int l = 0; l < 16; l++) s += k.q[16 * j + l] * (int) b[i].qs[16 * j + l];
            isum += k.sc[j] * s;
            imin += k.m[j] * (int) b[i].bsums[j];
        }
        sumf += (k.d * b[i].d) * (float) isum;
        sumf -= (k.dmin * b[i].d) * (float) imin;
    }
    return sumf;
}

/* ------------------------------------------------------------------------------------------ */
/* router                                                                                      */
/* ------------------------------------------------------------------------------------------ */

/* ggml_mul_mat(ffn_gate_inp, hnorm) (src/qwen3.cpp:178). For an F16 weight ggml's CPU path rounds
 * the activations to fp16 first (vec_dot_type F16) and accumulates the exact fp16*fp16 products in
 * f32. ggml's SIMD summation order is unpinned; the order used here, shared bit for bit with the
 * device kernel, is: 64 lane partials, lane l owning elements 256c + 4l + q (c ascending, then
 * q = 0..3), each accumulated with fmaf from 0, then a pairwise tree p[l] + p[l ^ s] for
 * s = 1, 2, 4, 8, 16, 32 (neighbouring lanes first). */
static float router_dot(const float *x, const void *w, int type, int h) {
    float p[64], t[64];
    const uint16_t *wh = (const uint16_t *) w;
    const float *wf = (const float *) w;
    for (int l = 0; l < 64; l++) {
        float acc = 0.0f;
        for (int c = 0; c < h / 256; c++) {
            for (int q = 0; q < 4; q++) {
                const int i = 256 * c + 4 * l + q;
                if (type == 1) acc = fmaf(h2f(or_fp32_to_fp16(x[i])), h2f(wh[i]), acc);
                else acc = fmaf(x[i], wf[i], acc);
            }
        }
        p[l] = acc;
    }
    for (int s = 1; s <= 32; s <<= 1) {
        for (int l = 0; l < 64; l++) t[l] = p[l] + p[l ^ s];
        memcpy(p, t, sizeof(p));
    }
    return p[0];
}

void or_router_logits(const float *hnorm, int T, int h, const void *gate_inp, int gate_type, int E, float *logits) {
    const size_t row = gate_type == 1 ? (size_t) h * 2 : (size_t) h * 4;
#pragma omp parallel for collapse(2) schedule(static)
    for (int t = 0; t < T; t++)
        for (int e = 0; e < E; e++)
            logits[(size_t) t * E + e] =
                router_dot(hnorm + (size_t) t * h, (const uint8_t *) gate_inp + (size_t) e * row, gate_type, h);
}

/* router() src/qwen3.cpp:175-192 for each token:
 *   soft_max (ggml ops.cpp): max, e_i = expf(l_i - max), sum in double, p_i = e_i * (float)(1/sum);
 *   argsort_top_k (:180): descending; probabilities are a monotone function of the logits, so the
 *     selection is made on the logits with ties to the lower id (std::sort leaves ties unspecified);
 *   get_rows (:184) gathers p in selected order; sum_rows (:187) sums them in double;
 *   clamp to >= 6.103515625e-5 (:187); div (:188). */
void or_router(const float *hnorm, int T, int h, const void *gate_inp, int gate_type, int E, int k, int32_t *ids,
               float *weights, float *logits_out, float *probs_out) {
    float *logits = (float *) malloc(sizeof(float) * (size_t) T * E);
    float *p = (float *) malloc(sizeof(float) * (size_t) E);
    unsigned char *taken = (unsigned char *) malloc((size_t) E);
    or_router_logits(hnorm, T, h, gate_inp, gate_type, E, logits);
    for (int t = 0; t < T; t++) {
        const float *l = logits + (size_t) t * E;
        float max = -INFINITY;
        for (int e = 0; e < E; e++) max = fmaxf(max, l[e]);
        double sum = 0.0;
        for (int e = 0; e < E; e++) {
            p[e] = expf(l[e] - max);
            sum += (double) p[e];
        }
        const float inv = (float) (1.0 / sum);
        for (int e = 0; e < E; e++) p[e] = p[e] * inv;
        memset(taken, 0, (size_t) E);
        for (int j = 0; j < k; j++) {
            int best = -1;
            for (int e = 0; e < E; e++) {
                if (taken[e]) continue;
                if (best < 0 || l[e] > l[best]) best = e;
            }
            taken[best] = 1;
            ids[(size_t) t * k + j] = best;
        }
        double s = 0.0;
        for (int j = 0; j < k; j++) s += (double) p[ids[(size_t) t * k + j]];
        float sf = (float) s;
        if (sf < 6.103515625e-5f) sf = 6.103515625e-5f;
        for (int j = 0; j < k; j++) weights[(size_t) t * k + j] = p[ids[(size_t) t * k + j]] / sf;
        if (probs_out) memcpy(probs_out + (size_t) t * E, p, sizeof(float) * (size_t) E);
    }
    if (logits_out) memcpy(logits_out, logits, sizeof(float) * (size_t) T * E);
    free(logits);
    free(p);
    free(taken);
}

/* ------------------------------------------------------------------------------------------ */
/* permutation                                                                                 */
/* ------------------------------------------------------------------------------------------ */

/* Stable counting sort of the (t, j) pairs by bin, the grouping ggml's CPU mul_mat_id builds per
 * expert (t outer, j inner). */
int or_permute(const int32_t *bins, int T, int k, int n_bins, int32_t *counts, int32_t *offsets, int32_t *perm,
               int32_t *active) {
    const int n = T * k;
    memset(counts, 0, sizeof(int32_t) * (size_t) n_bins);
    for (int p = 0; p < n; p++) counts[bins[p]]++;
    offsets[0] = 0;
    for (int b = 0; b < n_bins; b++) offsets[b + 1] = offsets[b] + counts[b];
    int32_t *cur = (int32_t *) malloc(sizeof(int32_t) * (size_t) (n_bins > 0 ? n_bins : 1));
    memcpy(cur, offsets, sizeof(int32_t) * (size_t) n_bins);
    for (int p = 0; p < n; p++) perm[cur[bins[p]]++] = p;
    free(cur);
    int na = 0;
    for (int b = 0; b < n_bins; b++)
        if (counts[b] > 0) active[na++] = b;
    return na;
}

/* ------------------------------------------------------------------------------------------ */
/* expert FFN                                                                                  */
/* ------------------------------------------------------------------------------------------ */

/* ggml's vec_dot_type: Q8_0 for Q8_0 weights, Q8_K for every k-quant */
static int act_type_for(int wtype) { return wtype == 8 ? 8 : 15; }

static void quantize_act(int wtype, const float *x, int n, void *out) {
    if (wtype == 8) or_quantize_q8_0_act(x, n, out);
    else or_quantize_q8_K(x, n, out);
}

static float dot_row(int wtype, int n, const void *w, const void *xq) {
    if (wtype == 8) return or_vec_dot_q8_0_q8_0(n, w, xq);
    if (wtype == 12) return or_vec_dot_q4_K_q8_K(n, w, xq);
    return or_vec_dot_k_q8_K(wtype, n, w, xq);
}

/* moe_apply() src/qwen3.cpp:197-214 with ggml CPU mul_mat_id semantics, then the residual add
 * (:250). up/gate: src1 = hnorm broadcast over j (:200), quantized once per token to the weight's
 * vec_dot_type; swiglu_split(g, u) = silu(g) * u (:203); down: each (t, j) row of the SwiGLU output
 * quantized on its own (:204); mul by the router weight (:205); k-way sum left to right (:206-210). */
void or_moe_ffn(const float *hnorm, int T, int h, int f, int k, const int32_t *slots, const float *weights,
                const float *resid, const void *up, const void *gate, const void *down, size_t stride_up,
                size_t stride_gate, size_t stride_down, int type_up, int type_gate, int type_down, float *out,
                float *y_out, int n_threads) {
    const size_t xu_row = or_row_bytes(act_type_for(type_up), h);
    const size_t xg_row = or_row_bytes(act_type_for(type_gate), h);
    const size_t xd_row = or_row_bytes(act_type_for(type_down), f);
    const size_t wu_row = or_row_bytes(type_up, h), wg_row = or_row_bytes(type_gate, h);
    const size_t wd_row = or_row_bytes(type_down, f);
    uint8_t *xu = (uint8_t *) malloc(xu_row * (size_t) T);
    uint8_t *xg = (uint8_t *) malloc(xg_row * (size_t) T);
    float *act = (float *) malloc(sizeof(float) * (size_t) T * k * f);
    uint8_t *actq = (uint8_t *) malloc(xd_row * (size_t) T * k);
    float *y = (float *) malloc(sizeof(float) * (size_t) T * k * h);
    if (n_threads <= 0) n_threads = 1;
    for (int t = 0; t < T; t++) {
        quantize_act(type_up, hnorm + (size_t) t * h, h, xu + (size_t) t * xu_row);
        quantize_act(type_gate, hnorm + (size_t) t * h, h, xg + (size_t) t * xg_row);
    }
    const int np = T * k;
#pragma omp parallel for collapse(2) schedule(static) num_threads(n_threads)
    for (int p = 0; p < np; p++) {
        for (int r = 0; r < f; r++) {
            const int t = p / k;
            const size_t s = (size_t) slots[p];
            const uint8_t *wu = (const uint8_t *) up + s * stride_up + (size_t) r * wu_row;
            const uint8_t *wg = (const uint8_t *) gate + s * stride_gate + (size_t) r * wg_row;
            const float u = dot_row(type_up, h, wu, xu + (size_t) t * xu_row);
            const float g = dot_row(type_gate, h, wg, xg + (size_t) t * xg_row);
            act[(size_t) p * f + r] = (g / (1.0f + expf(-g))) * u;
        }
    }
    for (int p = 0; p < np; p++) quantize_act(type_down, act + (size_t) p * f, f, actq + (size_t) p * xd_row);
#pragma omp parallel for collapse(2) schedule(static) num_threads(n_threads)
    for (int p = 0; p < np; p++) {
        for (int r = 0; r < h; r++) {
            const size_t s = (size_t) slots[p];
            const uint8_t *wd = (const uint8_t *) down + s * stride_down + (size_t) r * wd_row;
            y[(size_t) p * h + r] = dot_row(type_down, f, wd, actq + (size_t) p * xd_row) * weights[p];
        }
    }
    for (int t = 0; t < T; t++) {
        for (int r = 0; r < h; r++) {
            float acc = y[(size_t) t * k * h + r];
            for (int j = 1; j < k; j++) acc = acc + y[((size_t) t * k + j) * h + r];
            out[(size_t) t * h + r] = acc + resid[(size_t) t * h + r];
        }
    }
    if (y_out) memcpy(y_out, y, sizeof(float) * (size_t) T * k * h);
    free(xu);
    free(xg);
    free(act);
    free(actq);
    free(y);
}

/* ------------------------------------------------------------------------------------------ */
/* ExpertStore slot bookkeeping                                                                */
/* ------------------------------------------------------------------------------------------ */

#define OR_MAX_SLOTS_PER_SHARD 1024 /* kMaxSlotsPerPool, src/expert_store.h:80 */

typedef struct {
    int32_t tu, tg, td;
    uint64_t slab;
    uint32_t n_slots;
    int32_t *owner_layer, *owner_expert, *refcount, *prev, *next;
    int32_t lru_head, lru_tail;
    uint32_t n_in_lru;
} or_shard;

struct or_pool {
    int n_layer, n_expert;
    int n_shards;
    or_shard *shards;
    int32_t *layer_shard;
    int32_t *slot_of; /* [n_layer * n_expert] */
    int32_t *pin_shard, *pin_slot;
    size_t n_pinned, cap_pinned;
    uint64_t hits, misses, bytes_read, acquires;
};

static void lru_push_tail(or_shard *p, int32_t s) {
    p->prev[s] = p->lru_tail;
    p->next[s] = -1;
    if (p->lru_tail >= 0) p->next[p->lru_tail] = s;
    p->lru_tail = s;
    if (p->lru_head < 0) p->lru_head = s;
    p->n_in_lru++;
}

static void lru_unlink(or_shard *p, int32_t s) {
    const int32_t a = p->prev[s], b = p->next[s];
    if (a >= 0) p->next[a] = b;
    else p->lru_head = b;
    if (b >= 0) p->prev[b] = a;
    else p->lru_tail = a;
    p->prev[s] = p->next[s] = -1;
    p->n_in_lru--;
}

static int32_t lru_pop_head(or_shard *p) {
    const int32_t s = p->lru_head;
    if (s < 0) return -1;
    lru_unlink(p, s);
    return s;
}

/* ExpertStore::init (src/expert_store.cpp:106-198): layers grouped by their (up, gate, down) type
 * triple in ascending triple order (std::map); each group's share is pool_bytes * n_layers / n_layer;
 * groups needing more than 1024 slots are split into shards of ceil(layers / n_shards) layers;
 * n_slots = clamp(share / slab, min_slots, 1024); all slots start empty in the LRU, slot 0 at the head. */
or_pool *or_pool_create(int n_layer, int n_expert, const int32_t *types, const uint64_t *strides, uint64_t pool_bytes,
                        uint32_t min_slots, char *err, size_t err_len) {
    if (min_slots > OR_MAX_SLOTS_PER_SHARD) {
        snprintf(err, err_len, "expert pool floor of %u slots exceeds the limit of %d experts per tensor", min_slots,
                 OR_MAX_SLOTS_PER_SHARD);
        return NULL;
    }
    or_pool *P = (or_pool *) calloc(1, sizeof(or_pool));
    P->n_layer = n_layer;
    P->n_expert = n_expert;
    P->layer_shard = (int32_t *) malloc(sizeof(int32_t) * (size_t) n_layer);
    P->slot_of = (int32_t *) malloc(sizeof(int32_t) * (size_t) n_layer * n_expert);
    for (size_t i = 0; i < (size_t) n_layer * n_expert; i++) P->slot_of[i] = -1;
    P->shards = (or_shard *) calloc((size_t) n_layer, sizeof(or_shard)); /* at most one shard per layer */
    int *order = (int *) malloc(sizeof(int) * (size_t) n_layer);
    int *done = (int *) calloc((size_t) n_layer, sizeof(int));
    int *ls = (int *) malloc(sizeof(int) * (size_t) n_layer);
    for (;;) {
        /* next class: the smallest (tu, tg, td) triple among layers not yet assigned */
        int best = -1;
        for (int l = 0; l < n_layer; l++) {
            if (done[l]) continue;
            if (best < 0) {
                best = l;
                continue;
            }
            const int32_t *a = types + 3 * l, *b = types + 3 * best;
            if (a[0] < b[0] || (a[0] == b[0] && (a[1] < b[1] || (a[1] == b[1] && a[2] < b[2])))) best = l;
        }
        if (best < 0) break;
        int nls = 0;
        for (int l = 0; l < n_layer; l++) {
            if (!done[l] && types[3 * l] == types[3 * best] && types[3 * l + 1] == types[3 * best + 1] &&
                types[3 * l + 2] == types[3 * best + 2]) {
                ls[nls++] = l;
                done[l] = 1;
            }
        }
        const uint64_t *st = strides + 3 * ls[0];
        const uint64_t slab = st[0] + st[1] + st[2];
        uint64_t want = pool_bytes * (uint64_t) nls / (uint64_t) n_layer / slab;
        if (want < min_slots) want = min_slots;
        const uint64_t n_sh = (want + OR_MAX_SLOTS_PER_SHARD - 1) / OR_MAX_SLOTS_PER_SHARD;
        const uint64_t per = ((uint64_t) nls + n_sh - 1) / n_sh;
        for (uint64_t i = 0; i < (uint64_t) nls; i += per) {
            or_shard *p = &P->shards[P->n_shards];
            const uint64_t end = i + per < (uint64_t) nls ? i + per : (uint64_t) nls;
            p->tu = types[3 * ls[0]];
            p->tg = types[3 * ls[0] + 1];
            p->td = types[3 * ls[0] + 2];
            p->slab = slab;
            const uint64_t share = pool_bytes * (end - i) / (uint64_t) n_layer;
            uint64_t ns = share / slab;
            if (ns < min_slots) ns = min_slots;
            if (ns > OR_MAX_SLOTS_PER_SHARD) ns = OR_MAX_SLOTS_PER_SHARD;
            p->n_slots = (uint32_t) ns;
            for (uint64_t j = i; j < end; j++) P->layer_shard[ls[j]] = P->n_shards;
            p->owner_layer = (int32_t *) malloc(sizeof(int32_t) * ns);
            p->owner_expert = (int32_t *) malloc(sizeof(int32_t) * ns);
            p->refcount = (int32_t *) calloc(ns, sizeof(int32_t));
            p->prev = (int32_t *) malloc(sizeof(int32_t) * ns);
            p->next = (int32_t *) malloc(sizeof(int32_t) * ns);
            p->lru_head = p->lru_tail = -1;
            for (uint32_t s = 0; s < ns; s++) {
                p->owner_layer[s] = p->owner_expert[s] = -1;
                lru_push_tail(p, (int32_t) s);
            }
            P->n_shards++;
        }
    }
    free(order);
    free(done);
    free(ls);
    return P;
}

void or_pool_destroy(or_pool *P) {
    if (!P) return;
    for (int i = 0; i < P->n_shards; i++) {
        free(P->shards[i].owner_layer);
        free(P->shards[i].owner_expert);
        free(P->shards[i].refcount);
        free(P->shards[i].prev);
        free(P->shards[i].next);
    }
    free(P->shards);
    free(P->layer_shard);
    free(P->slot_of);
    free(P->pin_shard);
    free(P->pin_slot);
    free(P);
}

static void pin(or_pool *P, int shard, int32_t s) {
    if (P->n_pinned == P->cap_pinned) {
        P->cap_pinned = P->cap_pinned ? 2 * P->cap_pinned : 256;
        P->pin_shard = (int32_t *) realloc(P->pin_shard, sizeof(int32_t) * P->cap_pinned);
        P->pin_slot = (int32_t *) realloc(P->pin_slot, sizeof(int32_t) * P->cap_pinned);
    }
    P->pin_shard[P->n_pinned] = shard;
    P->pin_slot[P->n_pinned] = s;
    P->n_pinned++;
}

/* ExpertStore::acquire (src/expert_store.cpp:232-286). A resident expert is a hit: it is pinned
 * (and unlinked from the LRU if its refcount was 0). Because a miss records its slot in slot_of
 * immediately, a repeat of that expert later in the same call is also a hit; the in-call duplicate
 * scan of :250-260 can therefore never match, and is not restated. A miss pops the LRU head
 * (failing when every slot is pinned), evicts the slot's previous owner and counts the three
 * matrix reads in bytes_read. */
int or_pool_acquire(or_pool *P, int layer, const int32_t *experts, int n, int32_t *slots, char *err, size_t err_len) {
    const int sh = P->layer_shard[layer];
    or_shard *p = &P->shards[sh];
    P->acquires++;
    for (int i = 0; i < n; i++) {
        const int32_t e = experts[i];
        int32_t *ref = &P->slot_of[(size_t) layer * P->n_expert + e];
        if (*ref >= 0) {
            const int32_t s = *ref;
            if (p->refcount[s] == 0) lru_unlink(p, s);
            p->refcount[s]++;
            pin(P, sh, s);
            slots[i] = s;
            P->hits++;
            continue;
        }
        const int32_t s = lru_pop_head(p);
        if (s < 0) {
            snprintf(err, err_len, "layer %d: every one of the %u slots is pinned (pool exhausted)", layer, p->n_slots);
            return -1;
        }
        if (p->owner_layer[s] >= 0) P->slot_of[(size_t) p->owner_layer[s] * P->n_expert + p->owner_expert[s]] = -1;
        p->owner_layer[s] = layer;
        p->owner_expert[s] = e;
        *ref = s;
        p->refcount[s] = 1;
        pin(P, sh, s);
        slots[i] = s;
        P->misses++;
        P->bytes_read += p->slab;
    }
    return 0;
}

/* ExpertStore::release_all (src/expert_store.cpp:289-295): unpin in acquisition order; a slot whose
 * refcount reaches 0 goes to the LRU tail. */
void or_pool_release_all(or_pool *P) {
    for (size_t i = 0; i < P->n_pinned; i++) {
        or_shard *p = &P->shards[P->pin_shard[i]];
        const int32_t s = P->pin_slot[i];
        if (--p->refcount[s] == 0) lru_push_tail(p, s);
    }
    P->n_pinned = 0;
}

void or_pool_stats(const or_pool *P, uint64_t out[4]) {
    out[0] = P->hits;
    out[1] = P->misses;
    out[2] = P->bytes_read;
    out[3] = P->acquires;
}

int or_pool_n_shards(const or_pool *P) { return P->n_shards; }
int or_pool_shard_of_layer(const or_pool *P, int layer) { return P->layer_shard[layer]; }
int or_pool_shard_slots(const or_pool *P, int shard) { return (int) P->shards[shard].n_slots; }

int or_pool_slot_owner(const or_pool *P, int shard, int slot, int32_t *layer, int32_t *expert) {
    const or_shard *p = &P->shards[shard];
    *layer = p->owner_layer[slot];
    *expert = p->owner_expert[slot];
    return p->refcount[slot];
}

int or_pool_lru(const or_pool *P, int shard, int32_t *out, int cap) {
    const or_shard *p = &P->shards[shard];
    int n = 0;
    for (int32_t s = p->lru_head; s >= 0 && n < cap; s = p->next[s]) out[n++] = s;
    return n;
}

/* ------------------------------------------------------------------------------------------ */
/* Qwen3-MoE forward pass around the MoE block (src/qwen3.cpp:112-171, :223-259)              */
/* ------------------------------------------------------------------------------------------ */

/* ggml_vec_dot_f16, x86 F16C/AVX path: both operands fp16 (the caller rounds the f32 activations to
 * fp16, ggml's vec_dot_type for F16 weights); 4 accumulators of 8 lanes over steps of 32 values,
 * reduced x0+x2, x1+x3, then x0+x1, then the two 128-bit halves, then two horizontal adds; the tail
 * (n % 32 values) is summed in double. The fp16 products are exact in f32. */
/* Sensitivity probe for the tests: with or_set_f16_double(1) every F16 dot is summed in double instead (a
 * legitimate reordering that ggml itself could make), which shows how far the forward pass's logits move
 * under rounding-level changes of its inputs alone. */
static int g_f16_double = 0;
void or_set_f16_double(int on) { g_f16_double = on; }

float or_dot_f16(const uint16_t *w, const uint16_t *x, int n) {
    if (g_f16_double) {
        double s = 0.0;
        for (int i = 0; i < n; i++) s += (double) h2f(w[i]) * (double) h2f(x[i]);
        return (float) s;
    }
    /* acc[a][l] = acc[a][l] + w * x per lane, each multiply and add rounded on its own (8-lane AVX
     * vectors of the same expression; F16C converts fp16 exactly) */
    float acc[4][8];
    __m256 va[4] = {_mm256_setzero_ps(), _mm256_setzero_ps(), _mm256_setzero_ps(), _mm256_setzero_ps()};
    const int np = n & ~31;
    for (int i = 0; i < np; i += 32)
        for (int a = 0; a < 4; a++) {
            const __m256 wv = _mm256_cvtph_ps(_mm_loadu_si128((const __m128i *) (w + i + 8 * a)));
            const __m256 xv = _mm256_cvtph_ps(_mm_loadu_si128((const __m128i *) (x + i + 8 * a)));
            va[a] = _mm256_add_ps(va[a], _mm256_mul_ps(wv, xv));
        }
    for (int a = 0; a < 4; a++) _mm256_storeu_ps(acc[a], va[a]);
    for (int l = 0; l < 8; l++) {
        acc[0][l] = acc[0][l] + acc[2][l];
        acc[1][l] = acc[1][l] + acc[3][l];
    }
    for (int l = 0; l < 8; l++) acc[0][l] = acc[0][l] + acc[1][l];
    float t[4];
    for (int l = 0; l < 4; l++) t[l] = acc[0][l] + acc[0][l + 4];
    const float h0 = t[0] + t[1], h1 = t[2] + t[3];
    double sum = (double) (h0 + h1);
    for (int i = np; i < n; i++) sum += (double) (h2f(w[i]) * h2f(x[i]));
    return (float) sum;
}

/* ggml_mul_mat(W, x) for an F16 W of `rows` rows x `cols` and f32 x [T][cols]: y [T][rows]. */
void or_matmul_f16(const uint16_t *W, int rows, int cols, const float *x, int T, float *y) {
    uint16_t *xh = (uint16_t *) malloc(sizeof(uint16_t) * (size_t) T * cols);
    for (size_t i = 0; i < (size_t) T * cols; i++) xh[i] = or_fp32_to_fp16(x[i]);
#pragma omp parallel for collapse(2) schedule(static)
    for (int t = 0; t < T; t++)
        for (int r = 0; r < rows; r++)
            y[(size_t) t * rows + r] = or_dot_f16(W + (size_t) r * cols, xh + (size_t) t * cols, cols);
    free(xh);
}

/* ggml_rms_norm (sum of x*x in double, mean rounded to float, scale = 1/sqrtf(mean + eps), y = x * scale)
 * followed by ggml_mul with the weight (src/qwen3.cpp:112-114). w may be NULL (no weight). */
void or_rms_norm(const float *x, int n, const float *w, float eps, float *y) {
    double sum = 0.0;
    for (int i = 0; i < n; i++) sum += (double) (x[i] * x[i]);
    const float mean = (float) (sum / n);
    const float scale = 1.0f / sqrtf(mean + eps);
    for (int i = 0; i < n; i++) y[i] = w ? (x[i] * scale) * w[i] : x[i] * scale;
}

/* ggml_rope_ext, NEOX mode, freq_scale 1, ext_factor 0, attn_factor 1 (src/qwen3.cpp:143-146): pair i
 * = (x[i], x[i + hd/2]) is rotated by theta_i, theta_0 = pos and theta_{i+1} = theta_i * theta_scale
 * (theta_scale = freq_base^(-2/hd), computed by the caller with powf). */
void or_rope_neox(const float *x, int hd, int pos, float theta_scale, float *y) {
    float theta = (float) pos;
    const int half = hd / 2;
    for (int i = 0; i < half; i++) {
        const float c = cosf(theta), s = sinf(theta);
        const float x0 = x[i], x1 = x[i + half];
        y[i] = x0 * c - x1 * s;
        y[i + half] = x0 * s + x1 * c;
        theta *= theta_scale;
    }
}

/* ggml_flash_attn_ext for one query row (src/qwen3.cpp:165-167): q rounded to fp16, s_j = dot_f16(K_j, q) *
 * scale over the n visible cells in cell order, online softmax (running max M, sum S, rescale by
 * expf(M_old - M)), V accumulated in f32 (GGML_PREC_F32), out = acc / S. K, V: n rows of hd fp16 at
 * row stride `ld` values. */
void or_attn_row(const float *q, const uint16_t *K, const uint16_t *V, int n, int hd, int ld, float scale, float *out) {
    uint16_t qh[512];
    float *acc = (float *) calloc((size_t) hd, sizeof(float));
    for (int d = 0; d < hd; d++) qh[d] = or_fp32_to_fp16(q[d]);
    float M = -INFINITY, S = 0.0f;
    for (int j = 0; j < n; j++) {
        const float s = or_dot_f16(K + (size_t) j * ld, qh, hd) * scale;
        float ms = 1.0f, vs = 1.0f;
        const float Mold = M;
        if (s > M) {
            M = s;
            ms = expf(Mold - M);
            for (int d = 0; d < hd; d++) acc[d] *= ms;
        } else {
            vs = expf(s - M);
        }
        const uint16_t *v = V + (size_t) j * ld;
        for (int d = 0; d < hd; d++) acc[d] = acc[d] + h2f(v[d]) * vs;
        S = S * ms + vs;
    }
    for (int d = 0; d < hd; d++) out[d] = acc[d] / S;
    free(acc);
}

struct or_qwen3 {
    or_qwen3_hparams hp;
    or_qwen3_layer *layers;
    const uint16_t *tok_embd, *output;
    const float *output_norm;
    int max_ctx, len;
    float theta_scale;
    uint16_t *K, *V; /* [n_layer][max_ctx][n_head_kv * head_dim] */
};

or_qwen3 *or_qwen3_create(const or_qwen3_hparams *hp, const or_qwen3_layer *layers, const uint16_t *tok_embd,
                          const float *output_norm, const uint16_t *output, int max_ctx) {
    if (hp->head_dim > 512 || hp->n_head % hp->n_head_kv) return NULL;
    or_qwen3 *m = (or_qwen3 *) calloc(1, sizeof(or_qwen3));
    m->hp = *hp;
    m->layers = (or_qwen3_layer *) malloc(sizeof(or_qwen3_layer) * (size_t) hp->n_layer);
    memcpy(m->layers, layers, sizeof(or_qwen3_layer) * (size_t) hp->n_layer);
    m->tok_embd = tok_embd;
    m->output = output ? output : tok_embd;
    m->output_norm = output_norm;
    m->max_ctx = max_ctx;
    m->theta_scale = powf(hp->rope_freq_base, -2.0f / (float) hp->head_dim);
    const size_t kv = (size_t) hp->n_layer * max_ctx * hp->n_head_kv * hp->head_dim;
    m->K = (uint16_t *) calloc(kv, sizeof(uint16_t));
    m->V = (uint16_t *) calloc(kv, sizeof(uint16_t));
    return m;
}

void or_qwen3_destroy(or_qwen3 *m) {
    if (!m) return;
    free(m->layers);
    free(m->K);
    free(m->V);
    free(m);
}

int or_qwen3_len(const or_qwen3 *m) { return m->len; }

void or_qwen3_truncate(or_qwen3 *m, int keep) {
    if (keep < m->len) m->len = keep < 0 ? 0 : keep;
}

/* Layer l of the forward pass (src/qwen3.cpp:128-171 attention + residual, then the MoE block,
 * :239-250) for T tokens at positions len .. len + T - 1: x [T][n_embd] is updated in place and the
 * layer's K / V rows are written at those positions. The last layer runs its MoE block on the last row
 * only (src/qwen3.cpp:233-238); ids [T][k] (optional) receive the router ids, -1 for rows it skips.
 * Does not advance len (or_qwen3_advance does). Returns 0, or -1 when the context is full. */
int or_qwen3_run_layer(or_qwen3 *m, int l, float *x, int T, int32_t *ids_out) {
    const or_qwen3_hparams *hp = &m->hp;
    if (T < 1 || l < 0 || l >= hp->n_layer || m->len + T > m->max_ctx) return -1;
    const int h = hp->n_embd, hd = hp->head_dim, nh = hp->n_head, nkv = hp->n_head_kv, k = hp->n_expert_used;
    const int hq = nh * hd, hk = nkv * hd, E = hp->n_expert, f = hp->n_ff_exp;
    const float kq_scale = 1.0f / sqrtf((float) hd);
    float *hn = (float *) malloc(sizeof(float) * (size_t) T * h);
    float *q = (float *) malloc(sizeof(float) * (size_t) T * hq);
    float *kk = (float *) malloc(sizeof(float) * (size_t) T * hk);
    float *vv = (float *) malloc(sizeof(float) * (size_t) T * hk);
    float *att = (float *) malloc(sizeof(float) * (size_t) T * hq);
    float *o = (float *) malloc(sizeof(float) * (size_t) T * h);
    float *tmp = (float *) malloc(sizeof(float) * (size_t) (hd > h ? hd : h));
    float *wts = (float *) malloc(sizeof(float) * (size_t) T * k);
    int32_t *ids = (int32_t *) malloc(sizeof(int32_t) * (size_t) T * k);
    const or_qwen3_layer *L = &m->layers[l];
    for (int t = 0; t < T; t++) or_rms_norm(x + (size_t) t * h, h, L->attn_norm, hp->rms_eps, hn + (size_t) t * h);
    or_matmul_f16(L->wq, hq, h, hn, T, q);
    or_matmul_f16(L->wk, hk, h, hn, T, kk);
    or_matmul_f16(L->wv, hk, h, hn, T, vv);
    uint16_t *Kl = m->K + (size_t) l * m->max_ctx * hk, *Vl = m->V + (size_t) l * m->max_ctx * hk;
    for (int t = 0; t < T; t++) {
        const int pos = m->len + t;
        for (int j = 0; j < nh; j++) {
            float *qh = q + (size_t) t * hq + (size_t) j * hd;
            if (L->q_norm) or_rms_norm(qh, hd, L->q_norm, hp->rms_eps, qh);
            or_rope_neox(qh, hd, pos, m->theta_scale, tmp);
            memcpy(qh, tmp, sizeof(float) * (size_t) hd);
        }
        for (int j = 0; j < nkv; j++) {
            float *kh = kk + (size_t) t * hk + (size_t) j * hd;
            if (L->k_norm) or_rms_norm(kh, hd, L->k_norm, hp->rms_eps, kh);
            or_rope_neox(kh, hd, pos, m->theta_scale, tmp);
            for (int d = 0; d < hd; d++) {
                Kl[(size_t) pos * hk + (size_t) j * hd + d] = or_fp32_to_fp16(tmp[d]);
                Vl[(size_t) pos * hk + (size_t) j * hd + d] = or_fp32_to_fp16(vv[(size_t) t * hk + (size_t) j * hd + d]);
            }
        }
    }
#pragma omp parallel for collapse(2) schedule(static)
    for (int t = 0; t < T; t++)
        for (int j = 0; j < nh; j++) {
            const int g = j / (nh / nkv);
            or_attn_row(q + (size_t) t * hq + (size_t) j * hd, Kl + (size_t) g * hd, Vl + (size_t) g * hd, m->len + t + 1, hd,
                        hk, kq_scale, att + (size_t) t * hq + (size_t) j * hd);
        }
    or_matmul_f16(L->wo, h, hq, att, T, o);
    for (size_t i = 0; i < (size_t) T * h; i++) x[i] = o[i] + x[i];
    const int last = l == hp->n_layer - 1;
    const int rows = last ? 1 : T;
    float *xr = x + (size_t) (T - rows) * h;
    for (int t = 0; t < rows; t++) or_rms_norm(xr + (size_t) t * h, h, L->ffn_norm, hp->rms_eps, hn + (size_t) t * h);
    or_router(hn, rows, h, L->gate_inp, 1, E, k, ids, wts, NULL, NULL);
    const size_t su = or_row_bytes(L->type_up, h) * f, sg = or_row_bytes(L->type_gate, h) * f,
                 sd = or_row_bytes(L->type_down, f) * h;
    or_moe_ffn(hn, rows, h, f, k, ids, wts, xr, L->up, L->gate, L->down, su, sg, sd, L->type_up, L->type_gate,
               L->type_down, xr, NULL, 8);
    if (ids_out) {
        for (int i = 0; i < (T - rows) * k; i++) ids_out[i] = -1;
        memcpy(ids_out + (size_t) (T - rows) * k, ids, sizeof(int32_t) * (size_t) rows * k);
    }
    free(hn);
    free(q);
    free(kk);
    free(vv);
    free(att);
    free(o);
    free(tmp);
    free(wts);
    free(ids);
    return 0;
}

/* The final RMSNorm and the output head of one row x [n_embd] (src/qwen3.cpp:252-258). */
void or_qwen3_head(const or_qwen3 *m, const float *x, float *logits) {
    const or_qwen3_hparams *hp = &m->hp;
    float *tmp = (float *) malloc(sizeof(float) * (size_t) hp->n_embd);
    or_rms_norm(x, hp->n_embd, m->output_norm, hp->rms_eps, tmp);
    or_matmul_f16(m->output, hp->n_vocab, hp->n_embd, tmp, 1, logits);
    free(tmp);
}

void or_qwen3_advance(or_qwen3 *m, int T) { m->len += T; }

/* Writes the fp16 K and V rows [n][n_head_kv * head_dim] of positions pos .. pos + n - 1 of layer l (a
 * cache given by the test instead of computed from tokens, e.g. a synthetic context). Returns 0, or -1
 * when the positions fall outside the context. */
int or_qwen3_set_kv(or_qwen3 *m, int l, int pos, int n, const uint16_t *k, const uint16_t *v) {
    const or_qwen3_hparams *hp = &m->hp;
    if (l < 0 || l >= hp->n_layer || pos < 0 || n < 0 || pos + n > m->max_ctx) return -1;
    const size_t hk = (size_t) hp->n_head_kv * hp->head_dim, base = ((size_t) l * m->max_ctx + (size_t) pos) * hk;
    memcpy(m->K + base, k, sizeof(uint16_t) * hk * (size_t) n);
    memcpy(m->V + base, v, sizeof(uint16_t) * hk * (size_t) n);
    return 0;
}

/* One step of the forward pass (src/qwen3.cpp:223-259) over T tokens: embedding, every layer (the last on
 * the last row only), logits [n_vocab] of the last token. trace (optional) [n_layer][T][k] receives the
 * router ids, -1 for the rows the last layer skips. Returns 0, or -1 when the context is full. */
int or_qwen3_decode(or_qwen3 *m, const int32_t *tokens, int T, float *logits, int32_t *trace) {
    const or_qwen3_hparams *hp = &m->hp;
    if (T < 1 || m->len + T > m->max_ctx) return -1;
    const int h = hp->n_embd, k = hp->n_expert_used;
    float *x = (float *) malloc(sizeof(float) * (size_t) T * h);
    for (int t = 0; t < T; t++)
        for (int i = 0; i < h; i++) x[(size_t) t * h + i] = h2f(m->tok_embd[(size_t) tokens[t] * h + i]);
    for (int l = 0; l < hp->n_layer; l++) or_qwen3_run_layer(m, l, x, T, trace ? trace + (size_t) l * T * k : NULL);
    or_qwen3_head(m, x + (size_t) (T - 1) * h, logits);
    m->len += T;
    free(x);
    return 0;
}
