/*
 * le_oracle.c -- CPU oracle for the GGUF quantized-matmul hot path.
 *
 * TEST INFRASTRUCTURE ONLY. This file is the parity checker: only tests/, the smoke() entry and
 * bench.py's cpu_baseline leg load it. The product (lastengine_amd/) never links or calls it.
 *
 * It restates, in plain C with the same floating-point operation order, the reference's CPU path:
 *   - f16_to_f32            src/quant.rs:37-49
 *   - block_info/row_bytes  src/quant.rs:24-35
 *   - scale_min_k4          src/quant.rs:52-55
 *   - ksign                 src/quant.rs:57
 *   - dequant_row           src/quant.rs:59-170 (Q4_0 :64-67, Q8_0 :68-71, Q4_K :72-82,
 *                           Q5_K :83-95, Q6_K :96-112, Q3_K :113-126, IQ3_XXS :127-141,
 *                           IQ2_XXS :142-154, IQ2_S :155-167)
 *   - quant_x               src/cuda/kernels.cu:15-25 (int8 activations per 32 values)
 *   - rms                   src/cpu_ref.rs:32-36 (RMSNorm)
 *   - swiglu                src/cpu_ref.rs:37 silu, applied as silu(g) * u (:255)
 *   - matvec_<ty> on int8 activations: udot<ty> per 32-value unit, src/cuda/kernels.cu:36-110,
 *                           summed per row in mv_impl's lane order, :371-392
 *   - Model::matvec         src/cpu_ref.rs:109-118 (per-row dequant, sequential f32 sum)
 *   - Model::matmat         src/cpu_ref.rs:266-276
 *   - Model::moe routed part src/cpu_ref.rs:242-259 (softmax, stable sort, top-k, renormalise,
 *                           out += w * down(silu(gate) * up) in selection order)
 *
 * Build with -ffp-contract=off and without fast-math: Rust does not contract a*b+c into an FMA,
 * and the sums must be evaluated strictly left to right.
 *
 * Parity pins (tests/test_oracle.py): f16 conversion against numpy over all 65536 codes; closed
 * forms per format (Q8_0 = d*q, Q4_K with sc=1/m=0 = d*q, Q6_K with sc=1 = d*(q-32), IQ index 0 =
 * grid[0]); grid invariants; even ksign parity; quantize->dequantize round trips through the
 * product's independent block packers; matvec against a float64 dot within the sequential-sum
 * error bound; matmat columns against matvec; MoE top-k against numpy's stable argsort.
 */
#include <math.h>
#include <pthread.h>
#include <stdint.h>
#include <stdlib.h>
#include <string.h>

#include "le_oracle_tables.h"

enum { OR_Q4_0 = 2, OR_Q8_0 = 8, OR_Q3_K = 11, OR_Q4_K = 12, OR_Q5_K = 13, OR_Q6_K = 14, OR_IQ2_XXS = 16,
       OR_IQ3_XXS = 18, OR_IQ2_S = 22 };

/* src/quant.rs:37-49 */
float or_f16_to_f32(uint16_t h) {
    uint32_t s = (h >> 15) & 1, e = (h >> 10) & 0x1f, m = h & 0x3ff, bits;
    if (e == 0) {
        if (m == 0) {
            bits = s << 31;
        } else {
            uint32_t e2 = 113, m2 = m;
            while ((m2 & 0x400) == 0) { m2 <<= 1; e2 -= 1; }
            bits = (s << 31) | (e2 << 23) | ((m2 & 0x3ff) << 13);
        }
    } else if (e == 31) {
        bits = (s << 31) | (0xffu << 23) | (m << 13);
    } else {
        bits = (s << 31) | ((e + 112) << 23) | (m << 13);
    }
    float f;
    memcpy(&f, &bits, 4);
    return f;
}

static float hf(const uint8_t *b, size_t o) { return or_f16_to_f32((uint16_t)(b[o] | (b[o + 1] << 8))); }

/* src/quant.rs:24-31: values per block, bytes per block. Returns 0 for unsupported types. */
int or_block_info(int ty, int *values, int *bytes) {
    switch (ty) {
    case OR_Q4_0: *values = 32; *bytes = 18; return 1;
    case OR_Q8_0: *values = 32; *bytes = 34; return 1;
    case OR_Q3_K: *values = 256; *bytes = 110; return 1;
    case OR_Q4_K: *values = 256; *bytes = 144; return 1;
    case OR_Q5_K: *values = 256; *bytes = 176; return 1;
    case OR_IQ2_S: *values = 256; *bytes = 82; return 1;
    case OR_Q6_K: *values = 256; *bytes = 210; return 1;
    case OR_IQ2_XXS: *values = 256; *bytes = 66; return 1;
    case OR_IQ3_XXS: *values = 256; *bytes = 98; return 1;
    default: return 0;
    }
}

/* src/quant.rs:35 (row_header is 0 for every type here) */
size_t or_row_bytes(int ty, size_t n) {
    int v, b;
    if (!or_block_info(ty, &v, &b)) return 0;
    return n / (size_t)v * (size_t)b;
}

/* src/quant.rs:52-55 */
static void scale_min_k4(int j, const uint8_t *s, uint8_t *sc, uint8_t *m) {
    if (j < 4) {
        *sc = s[j] & 63;
        *m = s[j + 4] & 63;
    } else {
        *sc = (uint8_t)((s[j + 4] & 15) | ((s[j - 4] >> 6) << 4));
        *m = (uint8_t)((s[j + 4] >> 4) | ((s[j] >> 6) << 4));
    }
}

/* src/quant.rs:57 */
uint8_t or_ksign(int i) {
    uint32_t v = (uint32_t)i & 0x7f, pop = 0;
    for (int b = 0; b < 7; b++) pop += (v >> b) & 1;
    return (uint8_t)(v | ((pop & 1) << 7));
}

static uint32_t rd32(const uint8_t *p) { return (uint32_t)p[0] | ((uint32_t)p[1] << 8) | ((uint32_t)p[2] << 16) | ((uint32_t)p[3] << 24); }

/* src/quant.rs:59-170 for the five hot-path types. n = values in the row (multiple of the block).
 * Returns 0 on an unsupported type. */
int or_dequant_row(int ty, const uint8_t *src, float *o, size_t n) {
    switch (ty) {
    case OR_Q8_0: /* :68-71 */
        for (size_t blk = 0; blk < n / 32; blk++) {
            const uint8_t *b = src + blk * 34;
            float d = hf(b, 0);
            for (int j = 0; j < 32; j++) o[blk * 32 + j] = d * (float)(int8_t)b[2 + j];
        }
        return 1;
    case OR_Q4_0: /* :64-67 */
        for (size_t blk = 0; blk < n / 32; blk++) {
            const uint8_t *b = src + blk * 18;
            float d = hf(b, 0);
            for (int j = 0; j < 16; j++) {
                o[blk * 32 + j] = d * ((float)(b[2 + j] & 15) - 8.0f);
                o[blk * 32 + j + 16] = d * ((float)(b[2 + j] >> 4) - 8.0f);
            }
        }
        return 1;
    case OR_Q5_K: /* :83-95 */
        for (size_t blk = 0; blk < n / 256; blk++) {
            const uint8_t *b = src + blk * 176, *sc = b + 4, *qh = b + 16, *qs = b + 48;
            float d = hf(b, 0), dmin = hf(b, 2), *ob = o + blk * 256;
            for (int g = 0; g < 4; g++) {
                uint8_t s1, m1, s2, m2;
                scale_min_k4(2 * g, sc, &s1, &m1);
                scale_min_k4(2 * g + 1, sc, &s2, &m2);
                for (int l = 0; l < 32; l++) {
                    float lo = (float)(qs[g * 32 + l] & 15) + (((qh[l] >> (2 * g)) & 1) ? 16.0f : 0.0f);
                    float hi = (float)(qs[g * 32 + l] >> 4) + (((qh[l] >> (2 * g + 1)) & 1) ? 16.0f : 0.0f);
                    ob[g * 64 + l] = d * (float)s1 * lo - dmin * (float)m1;
                    ob[g * 64 + 32 + l] = d * (float)s2 * hi - dmin * (float)m2;
                }
            }
        }
        return 1;
    case OR_Q3_K: /* :113-126 */
        for (size_t blk = 0; blk < n / 256; blk++) {
            const uint8_t *b = src + blk * 110, *hm = b, *qs = b + 32, *sc = b + 96;
            float d = hf(b, 108);
            int scales[16];
            for (int i = 0; i < 16; i++) {
                int lo = i < 8 ? (sc[i] & 15) : (sc[i - 8] >> 4);
                int hi = (sc[8 + i % 4] >> (2 * (i / 4))) & 3;
                scales[i] = (lo | (hi << 4)) - 32;
            }
            for (int e = 0; e < 256; e++) {
                int c = e / 128, sh = (e % 128) / 32, l = e % 32;
                int q = ((qs[32 * c + l] >> (2 * sh)) & 3) - (((hm[l] >> (e / 32)) & 1) == 0 ? 4 : 0);
                o[blk * 256 + e] = d * (float)scales[e / 16] * (float)q;
            }
        }
        return 1;
    case OR_IQ2_S: /* :155-167 */
        for (size_t blk = 0; blk < n / 256; blk++) {
            const uint8_t *b = src + blk * 82, *qs = b + 2, *signs = b + 34, *qh = b + 66, *sc = b + 74;
            float d = hf(b, 0);
            for (int ib = 0; ib < 8; ib++) {
                float db[2] = {d * (0.5f + (float)(sc[ib] & 15)) * 0.25f, d * (0.5f + (float)(sc[ib] >> 4)) * 0.25f};
                for (int l = 0; l < 4; l++) {
                    int gi = qs[ib * 4 + l] | (((int)qh[ib] << (8 - 2 * l)) & 0x300);
                    const uint8_t *g = OR_IQ2S_GRID[gi];
                    uint8_t sgn = signs[ib * 4 + l];
                    for (int j = 0; j < 8; j++)
                        o[blk * 256 + ib * 32 + l * 8 + j] = db[l / 2] * (float)g[j] * ((sgn >> j) & 1 ? -1.0f : 1.0f);
                }
            }
        }
        return 1;
    case OR_Q4_K: /* :72-82 */
        for (size_t blk = 0; blk < n / 256; blk++) {
            const uint8_t *b = src + blk * 144, *sc = b + 4, *qs = b + 16;
            float d = hf(b, 0), dmin = hf(b, 2), *ob = o + blk * 256;
            for (int g = 0; g < 4; g++) {
                uint8_t s1, m1, s2, m2;
                scale_min_k4(2 * g, sc, &s1, &m1);
                scale_min_k4(2 * g + 1, sc, &s2, &m2);
                for (int l = 0; l < 32; l++) {
                    ob[g * 64 + l] = d * (float)s1 * (float)(qs[g * 32 + l] & 15) - dmin * (float)m1;
                    ob[g * 64 + 32 + l] = d * (float)s2 * (float)(qs[g * 32 + l] >> 4) - dmin * (float)m2;
                }
            }
        }
        return 1;
    case OR_Q6_K: /* :96-112 */
        for (size_t blk = 0; blk < n / 256; blk++) {
            const uint8_t *b = src + blk * 210;
            float d = hf(b, 208);
            for (int h = 0; h < 2; h++) {
                const uint8_t *ql = b + h * 64, *qh = b + 128 + h * 32;
                const int8_t *sc = (const int8_t *)(b + 192 + h * 8);
                float *ob = o + blk * 256 + h * 128;
                for (int l = 0; l < 32; l++) {
                    int is = l / 16;
                    int q1 = ((ql[l] & 15) | ((qh[l] & 3) << 4)) - 32;
                    int q2 = ((ql[l + 32] & 15) | (((qh[l] >> 2) & 3) << 4)) - 32;
                    int q3 = ((ql[l] >> 4) | (((qh[l] >> 4) & 3) << 4)) - 32;
                    int q4 = ((ql[l + 32] >> 4) | (((qh[l] >> 6) & 3) << 4)) - 32;
                    ob[l] = d * (float)sc[is] * (float)q1;
                    ob[l + 32] = d * (float)sc[is + 2] * (float)q2;
                    ob[l + 64] = d * (float)sc[is + 4] * (float)q3;
                    ob[l + 96] = d * (float)sc[is + 6] * (float)q4;
                }
            }
        }
        return 1;
    case OR_IQ3_XXS: /* :127-141 */
        for (size_t blk = 0; blk < n / 256; blk++) {
            const uint8_t *b = src + blk * 98, *qs = b + 2, *sg = b + 66;
            float d = hf(b, 0);
            for (int ib = 0; ib < 8; ib++) {
                uint32_t aux = rd32(sg + ib * 4);
                float db = d * (0.5f + (float)(aux >> 28)) * 0.5f;
                for (int l = 0; l < 4; l++) {
                    uint8_t sgn = or_ksign((int)((aux >> (7 * l)) & 127));
                    const uint8_t *g1 = OR_IQ3XXS_GRID[qs[ib * 8 + 2 * l]], *g2 = OR_IQ3XXS_GRID[qs[ib * 8 + 2 * l + 1]];
                    for (int j = 0; j < 4; j++) {
                        o[blk * 256 + ib * 32 + l * 8 + j] = db * (float)g1[j] * ((sgn >> j) & 1 ? -1.0f : 1.0f);
                        o[blk * 256 + ib * 32 + l * 8 + j + 4] = db * (float)g2[j] * ((sgn >> (j + 4)) & 1 ? -1.0f : 1.0f);
                    }
                }
            }
        }
        return 1;
    case OR_IQ2_XXS: /* :142-154 */
        for (size_t blk = 0; blk < n / 256; blk++) {
            const uint8_t *b = src + blk * 66, *qs = b + 2;
            float d = hf(b, 0);
            for (int ib = 0; ib < 8; ib++) {
                const uint8_t *q = qs + ib * 8;
                uint32_t aux = rd32(q + 4);
                float db = d * (0.5f + (float)(aux >> 28)) * 0.25f;
                for (int l = 0; l < 4; l++) {
                    uint8_t sgn = or_ksign((int)((aux >> (7 * l)) & 127));
                    const uint8_t *g = OR_IQ2XXS_GRID[q[l]];
                    for (int j = 0; j < 8; j++)
                        o[blk * 256 + ib * 32 + l * 8 + j] = db * (float)g[j] * ((sgn >> j) & 1 ? -1.0f : 1.0f);
                }
            }
        }
        return 1;
    default:
        return 0;
    }
}

/* Dequantize `rows` consecutive rows of `cols` values. */
int or_dequant_rows(int ty, const uint8_t *w, float *out, size_t rows, size_t cols) {
    size_t rb = or_row_bytes(ty, cols);
    if (!rb) return 0;
    for (size_t r = 0; r < rows; r++)
        if (!or_dequant_row(ty, w + r * rb, out + r * cols, cols)) return 0;
    return 1;
}

/* ---- threaded row loops (the reference uses rayon into_par_iter over rows) ---- */

typedef struct {
    int ty;
    const uint8_t *w;
    size_t rows, cols, m;
    const float *x; /* m x cols */
    float *y;       /* m x rows */
    size_t r0, r1;
} job_t;

/* One row: dequant then, for every input, the sequential f32 dot of src/cpu_ref.rs:116/273. */
static void *row_worker(void *arg) {
    job_t *j = (job_t *)arg;
    size_t rb = or_row_bytes(j->ty, j->cols);
    float *buf = (float *)malloc(j->cols * sizeof(float));
    for (size_t r = j->r0; r < j->r1; r++) {
        or_dequant_row(j->ty, j->w + r * rb, buf, j->cols);
        for (size_t t = 0; t < j->m; t++) {
            const float *x = j->x + t * j->cols;
            float acc = 0.0f;
            for (size_t c = 0; c < j->cols; c++) acc += buf[c] * x[c];
            j->y[t * j->rows + r] = acc;
        }
    }
    free(buf);
    return NULL;
}

/* out[t][r] = W[r,:] . x[t] for t < m (m = 1 is Model::matvec, m > 1 is Model::matmat). */
int or_matmat(int ty, const uint8_t *w, size_t rows, size_t cols, const float *x, size_t m, float *y, int nthreads) {
    if (!or_row_bytes(ty, cols)) return 0;
    if (nthreads < 1) nthreads = 1;
    if ((size_t)nthreads > rows) nthreads = (int)(rows ? rows : 1);
    pthread_t th[256];
    job_t jobs[256];
    if (nthreads > 256) nthreads = 256;
    size_t per = (rows + (size_t)nthreads - 1) / (size_t)nthreads;
    for (int i = 0; i < nthreads; i++) {
        job_t j = {ty, w, rows, cols, m, x, y, (size_t)i * per, (size_t)(i + 1) * per};
        if (j.r0 > rows) j.r0 = rows;
        if (j.r1 > rows) j.r1 = rows;
        jobs[i] = j;
    }
    if (nthreads == 1) {
        row_worker(&jobs[0]);
        return 1;
    }
    for (int i = 0; i < nthreads; i++) pthread_create(&th[i], NULL, row_worker, &jobs[i]);
    for (int i = 0; i < nthreads; i++) pthread_join(th[i], NULL);
    return 1;
}

int or_matvec(int ty, const uint8_t *w, size_t rows, size_t cols, const float *x, float *y, int nthreads) {
    return or_matmat(ty, w, rows, cols, x, 1, y, nthreads);
}

/* src/cpu_ref.rs:37 */
static float silu(float x) { return x / (1.0f + expf(-x)); }

/* Routing of src/cpu_ref.rs:243-250 for one token: softmax over n logits, stable sort by
 * probability descending (ties keep the lower index first), keep k, renormalise by the sum of the
 * kept probabilities. Writes idx[k] and w[k] = pr[idx]/tot. */
void or_route(const float *logits, int n, int k, int *idx, float *w) {
    float m = -3.40282347e38f; /* f32::MIN */
    for (int i = 0; i < n; i++) m = fmaxf(m, logits[i]);
    float *pr = (float *)malloc((size_t)n * sizeof(float));
    int *ord = (int *)malloc((size_t)n * sizeof(int));
    float s = 0.0f;
    for (int i = 0; i < n; i++) pr[i] = expf(logits[i] - m);
    for (int i = 0; i < n; i++) s += pr[i];
    for (int i = 0; i < n; i++) pr[i] /= s;
    /* stable insertion sort, descending */
    for (int i = 0; i < n; i++) {
        int v = i, p = i;
        while (p > 0 && pr[ord[p - 1]] < pr[v]) { ord[p] = ord[p - 1]; p--; }
        ord[p] = v;
    }
    float tot = 0.0f;
    for (int t = 0; t < k; t++) tot += pr[ord[t]];
    for (int t = 0; t < k; t++) { idx[t] = ord[t]; w[t] = pr[ord[t]] / tot; }
    free(pr);
    free(ord);
}

/* Routed part of Model::moe (src/cpu_ref.rs:242-259) for n_tok independent tokens.
 * gate/up: n_exp slabs of ff x hidden (type ty_gu); down: n_exp slabs of hidden x ff (type ty_d);
 * slab e starts at e * rows * row_bytes (src/cpu_ref.rs:110-115). h: n_tok x hidden,
 * logits: n_tok x n_exp, out: n_tok x hidden (overwritten). idx_out/w_out (n_tok x k) optional. */
int or_moe(int ty_g, int ty_u, int ty_d, const uint8_t *gate, const uint8_t *up, const uint8_t *down,
           int n_exp, int k, size_t hidden, size_t ff, const float *h, const float *logits, int n_tok,
           float *out, int *idx_out, float *w_out, int nthreads) {
    size_t rbg = or_row_bytes(ty_g, hidden), rbu = or_row_bytes(ty_u, hidden), rbd = or_row_bytes(ty_d, ff);
    if (!rbg || !rbu || !rbd || k < 1 || k > n_exp) return 0;
    float *gg = (float *)malloc(ff * sizeof(float)), *uu = (float *)malloc(ff * sizeof(float));
    float *a = (float *)malloc(ff * sizeof(float)), *r = (float *)malloc(hidden * sizeof(float));
    int *idx = (int *)malloc((size_t)k * sizeof(int));
    float *w = (float *)malloc((size_t)k * sizeof(float));
    for (int t = 0; t < n_tok; t++) {
        const float *ht = h + (size_t)t * hidden;
        float *ot = out + (size_t)t * hidden;
        or_route(logits + (size_t)t * n_exp, n_exp, k, idx, w);
        for (size_t i = 0; i < hidden; i++) ot[i] = 0.0f;
        for (int s = 0; s < k; s++) {
            int e = idx[s];
            or_matvec(ty_g, gate + (size_t)e * ff * rbg, ff, hidden, ht, gg, nthreads);
            or_matvec(ty_u, up + (size_t)e * ff * rbu, ff, hidden, ht, uu, nthreads);
            for (size_t i = 0; i < ff; i++) a[i] = silu(gg[i]) * uu[i];
            or_matvec(ty_d, down + (size_t)e * hidden * rbd, hidden, ff, a, r, nthreads);
            for (size_t i = 0; i < hidden; i++) ot[i] += w[s] * r[i];
        }
        if (idx_out)
            for (int s = 0; s < k; s++) { idx_out[t * k + s] = idx[s]; w_out[t * k + s] = w[s]; }
    }
    free(gg); free(uu); free(a); free(r); free(idx); free(w);
    return 1;
}

/* ---- int8 activation mode (reference GPU path) ---- */

/* quant_x (src/cuda/kernels.cu:15-25): per 32 values d = amax / 127, q = round-half-even(x / d)
 * computed as x * (1 / d), xs = sum q. One unit per 32 values. */
void or_quant_x(const float *x, int8_t *xq, float *xd, int32_t *xs, size_t n_units) {
    for (size_t u = 0; u < n_units; u++) {
        float a = 0.0f;
        for (int l = 0; l < 32; l++) a = fmaxf(a, fabsf(x[u * 32 + l]));
        float d = a / 127.0f, id = d > 0.0f ? 1.0f / d : 0.0f;
        int s = 0;
        for (int l = 0; l < 32; l++) {
            int q = (int)nearbyintf(x[u * 32 + l] * id);
            xq[u * 32 + l] = (int8_t)q;
            s += q;
        }
        xd[u] = d;
        xs[u] = s;
    }
}

static int dot8(const int8_t *a, const int *w) { /* w: 8 values as ints */
    int s = 0;
    for (int i = 0; i < 8; i++) s += a[i] * w[i];
    return s;
}

/* Integer weight values of 32-value unit j of block b (the q the dequant multiplies), in the
 * order the activations of that unit are laid out. */
static void unit_q(int ty, const uint8_t *b, int j, int *q) {
    switch (ty) {
    case OR_Q4_0:
        for (int l = 0; l < 16; l++) { q[l] = b[2 + l] & 15; q[l + 16] = b[2 + l] >> 4; }
        break;
    case OR_Q8_0:
        for (int l = 0; l < 32; l++) q[l] = (int8_t)b[2 + l];
        break;
    case OR_Q4_K:
        for (int l = 0; l < 32; l++) q[l] = (j & 1) ? (b[16 + (j >> 1) * 32 + l] >> 4) : (b[16 + (j >> 1) * 32 + l] & 15);
        break;
    case OR_Q5_K:
        for (int l = 0; l < 32; l++) {
            int v = (j & 1) ? (b[48 + (j >> 1) * 32 + l] >> 4) : (b[48 + (j >> 1) * 32 + l] & 15);
            q[l] = v | (((b[16 + l] >> j) & 1) << 4);
        }
        break;
    case OR_Q3_K:
        for (int l = 0; l < 32; l++)
            q[l] = ((b[32 + (j >> 2) * 32 + l] >> (2 * (j & 3))) & 3) - (((b[l] >> j) & 1) ? 0 : 4);
        break;
    case OR_Q6_K: {
        int half = j >> 2, s = j & 3;
        const uint8_t *ql = b + half * 64 + (s & 1) * 32, *qh = b + 128 + half * 32;
        for (int l = 0; l < 32; l++) q[l] = (((ql[l] >> ((s >> 1) * 4)) & 15) | (((qh[l] >> (2 * s)) & 3) << 4)) - 32;
        break;
    }
    case OR_IQ2_XXS: {
        const uint8_t *g8 = b + 2 + j * 8;
        uint32_t aux = rd32(g8 + 4);
        for (int l = 0; l < 4; l++) {
            uint8_t sg = or_ksign((int)((aux >> (7 * l)) & 127));
            for (int t = 0; t < 8; t++) q[l * 8 + t] = ((sg >> t) & 1) ? -(int)OR_IQ2XXS_GRID[g8[l]][t] : OR_IQ2XXS_GRID[g8[l]][t];
        }
        break;
    }
    case OR_IQ3_XXS: {
        const uint8_t *qs = b + 2 + j * 8;
        uint32_t aux = rd32(b + 66 + j * 4);
        for (int l = 0; l < 4; l++) {
            uint8_t sg = or_ksign((int)((aux >> (7 * l)) & 127));
            for (int t = 0; t < 8; t++) {
                int g = OR_IQ3XXS_GRID[qs[2 * l + t / 4]][t & 3];
                q[l * 8 + t] = ((sg >> t) & 1) ? -g : g;
            }
        }
        break;
    }
    case OR_IQ2_S: {
        const uint8_t *qs = b + 2 + j * 4, *sn = b + 34 + j * 4;
        int qh = b[66 + j];
        for (int l = 0; l < 4; l++) {
            int gi = qs[l] | ((qh << (8 - 2 * l)) & 0x300);
            for (int t = 0; t < 8; t++) q[l * 8 + t] = ((sn[l] >> t) & 1) ? -(int)OR_IQ2S_GRID[gi][t] : OR_IQ2S_GRID[gi][t];
        }
        break;
    }
    }
}

/* udot<ty> (src/cuda/kernels.cu:36-110): unit j of block b against int8 activations xq[32], scale
 * dx, sum sx; the integer dot is exact and the float expression keeps the reference's order. */
static float unit_dot(int ty, const uint8_t *b, int j, const int8_t *xq, float dx, int sx) {
    int q[32];
    unit_q(ty, b, j, q);
    int a0 = dot8(xq, q) + dot8(xq + 8, q + 8), a1 = dot8(xq + 16, q + 16) + dot8(xq + 24, q + 24);
    int a = a0 + a1;
    switch (ty) {
    case OR_Q4_0: return hf(b, 0) * dx * (float)(a - 8 * sx);
    case OR_Q8_0: return hf(b, 0) * dx * (float)a;
    case OR_Q4_K:
    case OR_Q5_K: {
        uint8_t sc, m;
        scale_min_k4(j, b + 4, &sc, &m);
        return dx * (hf(b, 0) * (float)sc * (float)a - hf(b, 2) * (float)m * (float)sx);
    }
    case OR_Q3_K: {
        const uint8_t *sc = b + 96;
        float r = 0.0f;
        for (int h = 0; h < 2; h++) {
            int i = 2 * j + h;
            int lo = i < 8 ? (sc[i] & 15) : (sc[i - 8] >> 4), hi = (sc[8 + (i & 3)] >> (2 * (i >> 2))) & 3;
            r += (float)(((lo | (hi << 4)) - 32) * (h ? a1 : a0));
        }
        return hf(b, 108) * dx * r;
    }
    case OR_Q6_K: {
        const int8_t *sc = (const int8_t *)(b + 192) + (j >> 2) * 8 + (j & 3) * 2;
        return hf(b, 208) * dx * (float)(sc[0] * a0 + sc[1] * a1);
    }
    case OR_IQ2_XXS: return hf(b, 0) * (0.5f + (float)(rd32(b + 2 + j * 8 + 4) >> 28)) * 0.25f * dx * (float)a;
    case OR_IQ3_XXS: return hf(b, 0) * (0.5f + (float)(rd32(b + 66 + j * 4) >> 28)) * 0.5f * dx * (float)a;
    case OR_IQ2_S: {
        int sc = b[74 + j];
        return hf(b, 0) * 0.25f * dx * ((0.5f + (float)(sc & 15)) * (float)a0 + (0.5f + (float)(sc >> 4)) * (float)a1);
    }
    }
    return 0.0f;
}

/* matvec_<ty> on int8 activations (src/cuda/kernels.cu:371-392): per row, lane li of lpr lanes
 * sums units li, li + lpr, ... in order; the lanes are then combined by the xor butterfly
 * o = lpr/2 .. 1 (lane 0's value is stored). lpr = min(32, units) as in the reference when that
 * is a power of two; otherwise (units = 24, i.e. 768 columns) the largest power of two below it,
 * since the reference's butterfly would then mix lanes of two rows. cols % 256 == 0. */
int or_matvec_q8(int ty, const uint8_t *w, size_t rows, size_t cols, const int8_t *xq, const float *xd, const int32_t *xs,
                 float *y) {
    int v, bb;
    if (!or_block_info(ty, &v, &bb) || cols % 256) return 0;
    size_t rb = or_row_bytes(ty, cols);
    int units = (int)(cols / 32), lpr = units >= 32 ? 32 : units >= 16 ? 16 : 8, ub = v / 32;
    float acc[32];
    for (size_t r = 0; r < rows; r++) {
        const uint8_t *row = w + r * rb;
        for (int li = 0; li < lpr; li++) {
            float a = 0.0f;
            for (int u = li; u < units; u += lpr)
                a += unit_dot(ty, row + (size_t)(u / ub) * bb, u % ub, xq + (size_t)u * 32, xd[u], xs[u]);
            acc[li] = a;
        }
        for (int o = lpr >> 1; o; o >>= 1) {
            float nx[32];
            for (int li = 0; li < lpr; li++) nx[li] = acc[li] + acc[li ^ o];
            memcpy(acc, nx, sizeof(float) * (size_t)lpr);
        }
        y[r] = acc[0];
    }
    return 1;
}

/* cpu_ref::rms (src/cpu_ref.rs:32-36): ss = sequential f32 sum of x*x, divided by n; r = 1 / sqrt(ss + eps);
 * o = x * r * w. */
void or_rms(const float *x, const float *w, float *o, size_t n, float eps) {
    float ss = 0.0f;
    for (size_t i = 0; i < n; i++) ss += x[i] * x[i];
    ss = ss / (float)n;
    const float r = 1.0f / sqrtf(ss + eps);
    for (size_t i = 0; i < n; i++) o[i] = x[i] * r * w[i];
}

/* SwiGLU of cpu_ref (src/cpu_ref.rs:37 silu, applied as silu(g) * u at :255): o = g / (1 + exp(-g)) * u. */
void or_swiglu(const float *g, const float *u, float *o, size_t n) {
    for (size_t i = 0; i < n; i++) o[i] = g[i] / (1.0f + expf(-g[i])) * u[i];
}
