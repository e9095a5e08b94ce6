/* HIP kernels of the GGUF quantized-matmul hot path, written for CDNA4 (gfx950, wave64).
 * Built with `hipcc --genco --offload-arch=gfx950` into code objects (one per part, see the end
 * of the file) under lastengine_amd/lib/, loaded by the
 * host library through hipModuleLoad (replacing the reference's NVRTC compile of
 * src/cuda/kernels.cu at engine start, src/gpu.rs:65-76).
 *
 * Kernels:
 *   le_dequant_<ty>            bit-exact dequant of whole rows (src/quant.rs:59-170)
 *   le_mv_<ty>_g<G>_t<T>       dequant-fused matvec / small-M matmul over `slots` weight matrices
 *                              (replaces matvec_<ty>, src/cuda/kernels.cu:371-392, and mm_<ty>,
 *                              :679-719, for T > 1 tokens)
 */
#include <hip/hip_runtime.h>
#include <stdint.h>

#include "le_formats.h"
#include "le_iq_tables.h"
#include "le_qmm_device.h"


__device__ const u32 le_iq2xxs_grid[512] = LE_IQ2XXS_GRID_WORDS;
__device__ const u32 le_iq3xxs_grid[256] = LE_IQ3XXS_GRID_WORDS;
__device__ const u32 le_iq2s_grid[2048] = LE_IQ2S_GRID_WORDS;

/* ===================================================================================== */
/* Bit-exact dequantization. One thread per 32-value unit; the arithmetic follows           */
/* src/quant.rs operation by operation with FP contraction disabled.                         */
/* ===================================================================================== */

template <int TY>
__device__ void dequant_unit(const u8 *row, int unit, float *o);

template <>
__device__ void dequant_unit<LE_TYPE_Q8_0>(const u8 *row, int unit, float *o) {
#pragma clang fp contract(off)
    const u8 *b = row + (size_t)unit * 34;
    const float d = f16_exact(b[0] | (b[1] << 8));
    for (int j = 0; j < 32; j++) o[j] = d * (float)(int8_t)b[2 + j];
}

template <>
__device__ void dequant_unit<LE_TYPE_Q4_K>(const u8 *row, int unit, float *o) {
#pragma clang fp contract(off)
    const u8 *b = row + (size_t)(unit >> 3) * 144;
    const int j = unit & 7, g = j >> 1;
    const float d = f16_exact(b[0] | (b[1] << 8)), dmin = f16_exact(b[2] | (b[3] << 8));
    const u8 *s = b + 4;
    u32 sc, m;
    if (j < 4) {
        sc = s[j] & 63;
        m = s[j + 4] & 63;
    } else {
        sc = (s[j + 4] & 15) | ((s[j - 4] >> 6) << 4);
        m = (s[j + 4] >> 4) | ((s[j] >> 6) << 4);
    }
    const u8 *qs = b + 16 + g * 32;
    for (int l = 0; l < 32; l++) {
        const u32 q = (j & 1) ? (qs[l] >> 4) : (qs[l] & 15);
        o[l] = d * (float)sc * (float)q - dmin * (float)m;
    }
}

template <>
__device__ void dequant_unit<LE_TYPE_Q6_K>(const u8 *row, int unit, float *o) {
#pragma clang fp contract(off)
    const u8 *b = row + (size_t)(unit >> 3) * 210;
    const int j = unit & 7, n = j >> 2, qd = j & 3;
    const u8 *ql = b + n * 64, *qh = b + 128 + n * 32;
    const int8_t *sc = (const int8_t *)(b + 192 + n * 8);
    const float d = f16_exact(b[208] | (b[209] << 8));
    for (int l = 0; l < 32; l++) {
        const u32 lo = (qd & 1) ? ql[l + 32] : ql[l];
        const u32 nib = (qd & 2) ? (lo >> 4) : (lo & 15);
        const int q = (int)(nib | (((qh[l] >> (2 * qd)) & 3) << 4)) - 32;
        o[l] = d * (float)sc[l / 16 + 2 * qd] * (float)q;
    }
}

template <>
__device__ void dequant_unit<LE_TYPE_IQ2_XXS>(const u8 *row, int unit, float *o) {
#pragma clang fp contract(off)
    const u8 *b = row + (size_t)(unit >> 3) * 66;
    const int ib = unit & 7;
    const u8 *q = b + 2 + ib * 8;
    const float d = f16_exact(b[0] | (b[1] << 8));
    const u32 aux = q[4] | (q[5] << 8) | (q[6] << 16) | ((u32)q[7] << 24);
    const float db = d * (0.5f + (float)(aux >> 28)) * 0.25f;
    for (int l = 0; l < 4; l++) {
        const u32 sgn = ksign_dev((aux >> (7 * l)) & 127u);
        const u32 g0 = le_iq2xxs_grid[2 * q[l]], g1 = le_iq2xxs_grid[2 * q[l] + 1];
        for (int jj = 0; jj < 8; jj++) {
            const u32 gv = ((jj < 4 ? g0 : g1) >> (8 * (jj & 3))) & 255u;
            o[l * 8 + jj] = db * (float)gv * (((sgn >> jj) & 1) ? -1.0f : 1.0f);
        }
    }
}

template <>
__device__ void dequant_unit<LE_TYPE_IQ3_XXS>(const u8 *row, int unit, float *o) {
#pragma clang fp contract(off)
    const u8 *b = row + (size_t)(unit >> 3) * 98;
    const int ib = unit & 7;
    const u8 *qs = b + 2 + ib * 8, *sg = b + 66 + ib * 4;
    const float d = f16_exact(b[0] | (b[1] << 8));
    const u32 aux = sg[0] | (sg[1] << 8) | (sg[2] << 16) | ((u32)sg[3] << 24);
    const float db = d * (0.5f + (float)(aux >> 28)) * 0.5f;
    for (int l = 0; l < 4; l++) {
        const u32 sgn = ksign_dev((aux >> (7 * l)) & 127u);
        const u32 g1 = le_iq3xxs_grid[qs[2 * l]], g2 = le_iq3xxs_grid[qs[2 * l + 1]];
        for (int jj = 0; jj < 4; jj++) {
            o[l * 8 + jj] = db * (float)((g1 >> (8 * jj)) & 255u) * (((sgn >> jj) & 1) ? -1.0f : 1.0f);
            o[l * 8 + jj + 4] = db * (float)((g2 >> (8 * jj)) & 255u) * (((sgn >> (jj + 4)) & 1) ? -1.0f : 1.0f);
        }
    }
}

/* src/quant.rs:64-67: one 18-byte block per unit, q - 8 on 4-bit codes (low nibbles: values 0-15). */
template <>
__device__ void dequant_unit<LE_TYPE_Q4_0>(const u8 *row, int unit, float *o) {
#pragma clang fp contract(off)
    const u8 *b = row + (size_t)unit * 18;
    const float d = f16_exact(b[0] | (b[1] << 8));
    for (int l = 0; l < 16; l++) {
        o[l] = d * ((float)(b[2 + l] & 15) - 8.0f);
        o[l + 16] = d * ((float)(b[2 + l] >> 4) - 8.0f);
    }
}

/* src/quant.rs:83-95: Q4_K's scales and nibbles plus a fifth bit per value in qh (bit j of qh[l]
 * for value 32j + l). */
template <>
__device__ void dequant_unit<LE_TYPE_Q5_K>(const u8 *row, int unit, float *o) {
#pragma clang fp contract(off)
    const u8 *b = row + (size_t)(unit >> 3) * 176;
    const int j = unit & 7, g = j >> 1;
    const float d = f16_exact(b[0] | (b[1] << 8)), dmin = f16_exact(b[2] | (b[3] << 8));
    const u8 *s = b + 4, *qh = b + 16, *qs = b + 48 + g * 32;
    u32 sc, m;
    if (j < 4) {
        sc = s[j] & 63;
        m = s[j + 4] & 63;
    } else {
        sc = (s[j + 4] & 15) | ((s[j - 4] >> 6) << 4);
        m = (s[j + 4] >> 4) | ((s[j] >> 6) << 4);
    }
    for (int l = 0; l < 32; l++) {
        const u32 q = ((j & 1) ? (qs[l] >> 4) : (qs[l] & 15)) + (((qh[l] >> j) & 1) ? 16u : 0u);
        o[l] = d * (float)sc * (float)q - dmin * (float)m;
    }
}

/* src/quant.rs:113-126: value e = 32j + l takes 2 bits at 2(j&3) of qs[32(j>>2) + l], minus 4 when
 * bit j of hmask[l] is clear; 16 signed 6-bit scales, one per 16 values. */
template <>
__device__ void dequant_unit<LE_TYPE_Q3_K>(const u8 *row, int unit, float *o) {
#pragma clang fp contract(off)
    const u8 *b = row + (size_t)(unit >> 3) * 110;
    const int j = unit & 7;
    const u8 *hm = b, *qs = b + 32 + (j >> 2) * 32, *sc = b + 96;
    const float d = f16_exact(b[108] | (b[109] << 8));
    int scl[2];
    for (int h = 0; h < 2; h++) {
        const int i = 2 * j + h;
        const int lo = i < 8 ? (sc[i] & 15) : (sc[i - 8] >> 4), hi = (sc[8 + (i & 3)] >> (2 * (i >> 2))) & 3;
        scl[h] = (lo | (hi << 4)) - 32;
    }
    for (int l = 0; l < 32; l++) {
        const int q = (int)((qs[l] >> (2 * (j & 3))) & 3) - (((hm[l] >> j) & 1) ? 0 : 4);
        o[l] = d * (float)scl[l >> 4] * (float)q;
    }
}

/* src/quant.rs:155-167: 10-bit grid index (qs byte, two bits of qh), an explicit sign byte per 8
 * values, a 4-bit scale per 16 values. */
template <>
__device__ void dequant_unit<LE_TYPE_IQ2_S>(const u8 *row, int unit, float *o) {
#pragma clang fp contract(off)
    const u8 *b = row + (size_t)(unit >> 3) * 82;
    const int ib = unit & 7;
    const u8 *qs = b + 2 + ib * 4, *sn = b + 34 + ib * 4;
    const u32 qh = b[66 + ib], scb = b[74 + ib];
    const float d = f16_exact(b[0] | (b[1] << 8));
    const float db[2] = {d * (0.5f + (float)(scb & 15)) * 0.25f, d * (0.5f + (float)(scb >> 4)) * 0.25f};
    for (int l = 0; l < 4; l++) {
        const u32 gi = qs[l] | ((qh << (8 - 2 * l)) & 0x300u);
        const u32 g0 = le_iq2s_grid[2 * gi], g1 = le_iq2s_grid[2 * gi + 1];
        for (int jj = 0; jj < 8; jj++) {
            const u32 gv = ((jj < 4 ? g0 : g1) >> (8 * (jj & 3))) & 255u;
            o[l * 8 + jj] = db[l >> 1] * (float)gv * (((sn[l] >> jj) & 1) ? -1.0f : 1.0f);
        }
    }
}

/* out[r*cols + c] for rows x cols; unit index over the whole matrix. */
template <int TY>
__device__ void dequant_rows(const u8 *__restrict__ w, float *__restrict__ out, int rows, int cols, size_t row_bytes) {
    const int upr = cols / 32;
    const size_t n = (size_t)rows * upr;
    for (size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x; i < n; i += (size_t)gridDim.x * blockDim.x) {
        const int r = (int)(i / upr), u = (int)(i % upr);
        float v[32];
        dequant_unit<TY>(w + (size_t)r * row_bytes, u, v);
        float4 *o = (float4 *)(out + (size_t)r * cols + (size_t)u * 32);
#pragma unroll
        for (int k = 0; k < 8; k++) o[k] = make_float4(v[4 * k], v[4 * k + 1], v[4 * k + 2], v[4 * k + 3]);
    }
}

#if defined(LE_PART_DEQ)
/* quant_x (src/cuda/kernels.cu:15-25): per 32 values d = amax / 127, q = x * (1 / d) rounded to
 * nearest even (d = 0: q = 0), xs = sum q. 32 lanes per unit, two units per wave. */
extern "C" __global__ void __launch_bounds__(256) le_quant_x(const float *x, int8_t *xq, float *xd, int *xs, int n_units) {
    const long long u = (long long)blockIdx.x * 8 + (threadIdx.x >> 5);
    const int l = threadIdx.x & 31;
    const bool ok = u < n_units;
    const float v = ok ? x[u * 32 + l] : 0.f;
    float am = fabsf(v);
#pragma unroll
    for (int o = 16; o; o >>= 1) am = fmaxf(am, __shfl_xor(am, o, 32));
    const float d = am / 127.0f, id = d > 0.f ? 1.0f / d : 0.f;
    const int q = (int)rintf(v * id);
    int s = q;
#pragma unroll
    for (int o = 16; o; o >>= 1) s += __shfl_xor(s, o, 32);
    if (ok) {
        xq[u * 32 + l] = (int8_t)q;
        if (l == 0) {
            xd[u] = d;
            xs[u] = s;
        }
    }
}
/* rms_quant (src/cuda/dense.cu:33-56): o = x * r * w with r = 1 / sqrt(sum(x^2) / n + eps) (the
 * RMSNorm of cpu_ref::rms, src/cpu_ref.rs:32-36), and o quantized as le_quant_x does, in one
 * launch. Every block forms the sum of squares over all n values (block-wide, from L2), then
 * quantizes its own 32-value units (32 lanes per unit, grid-stride). */
extern "C" __global__ void __launch_bounds__(256) le_rms_quant(const float *x, const float *w, float *o, int8_t *xq, float *xd,
                                                               int *xs, int n, float eps) {
    __shared__ float part[4];
    float s = 0.f;
    for (int i = threadIdx.x; i < n; i += 256) s += x[i] * x[i];
#pragma unroll
    for (int off = 32; off; off >>= 1) s += __shfl_xor(s, off);
    if ((threadIdx.x & 63) == 0) part[threadIdx.x >> 6] = s;
    __syncthreads();
    const float ss = (part[0] + part[1]) + (part[2] + part[3]);
    const float r = 1.0f / sqrtf(ss / (float)n + eps);
    const int l = threadIdx.x & 31, nu = n >> 5;
    for (int u = blockIdx.x * 8 + (threadIdx.x >> 5); u < nu; u += gridDim.x * 8) {
        const float v = x[u * 32 + l] * r * w[u * 32 + l];
        o[u * 32 + l] = v;
        float am = fabsf(v);
#pragma unroll
        for (int off = 16; off; off >>= 1) am = fmaxf(am, __shfl_xor(am, off, 32));
        const float d = am / 127.0f, id = d > 0.f ? 1.0f / d : 0.f;
        const int q = (int)rintf(v * id);
        int sm = q;
#pragma unroll
        for (int off = 16; off; off >>= 1) sm += __shfl_xor(sm, off, 32);
        xq[u * 32 + l] = (int8_t)q;
        if (l == 0) {
            xd[u] = d;
            xs[u] = sm;
        }
    }
}
#define LE_DEQ(TY, NAME)                                                                                   \
    extern "C" __global__ void __launch_bounds__(256) NAME(const u8 *w, float *out, int rows, int cols,     \
                                                          unsigned long long row_bytes) {                  \
        dequant_rows<TY>(w, out, rows, cols, (size_t)row_bytes);                                           \
    }
LE_DEQ(LE_TYPE_Q4_0, le_dequant_2)
LE_DEQ(LE_TYPE_Q3_K, le_dequant_11)
LE_DEQ(LE_TYPE_Q5_K, le_dequant_13)
LE_DEQ(LE_TYPE_IQ2_S, le_dequant_22)
LE_DEQ(LE_TYPE_Q8_0, le_dequant_8)
LE_DEQ(LE_TYPE_Q4_K, le_dequant_12)
LE_DEQ(LE_TYPE_Q6_K, le_dequant_14)
LE_DEQ(LE_TYPE_IQ2_XXS, le_dequant_16)
LE_DEQ(LE_TYPE_IQ3_XXS, le_dequant_18)

/* Streaming-read probe: the practical HBM read ceiling of this part at a given size, measured the
 * way the matvec reads its weights (16-byte loads, consecutive lanes on consecutive chunks). Each
 * thread keeps U loads in flight per trip of a grid-stride loop and folds every word into a
 * checksum, so no load can be dropped; one word per block is written. NT: nontemporal loads. */
template <bool NT, int U>
__device__ __forceinline__ void read_probe(const u8 *__restrict__ buf, unsigned long long n16, u32 *sink) {
    const unsigned long long stride = (unsigned long long)gridDim.x * blockDim.x;
    u32 acc = 0;
    for (unsigned long long i = (unsigned long long)blockIdx.x * blockDim.x + threadIdx.x; i < n16; i += stride * U) {
        uint4 v[U];
#pragma unroll
        for (int u = 0; u < U; u++) {
            const unsigned long long j = min(i + stride * u, n16 - 1);
            v[u] = NT ? ldg16(buf + 16 * j) : ldg16c(buf + 16 * j);
        }
#pragma unroll
        for (int u = 0; u < U; u++) acc += (v[u].x ^ v[u].y) + (v[u].z ^ v[u].w);
    }
    acc += __shfl_xor(acc, 1);
    if (threadIdx.x == 0) sink[blockIdx.x] = acc;
}
#define LE_RD(NT, U) \
    extern "C" __global__ void __launch_bounds__(512) le_read_nt##NT##_u##U(const u8 *buf, unsigned long long n16, u32 *sink) { \
        read_probe<NT, U>(buf, n16, sink);                                                              \
    }
LE_RD(0, 1) LE_RD(0, 2) LE_RD(0, 4) LE_RD(0, 8) LE_RD(1, 1) LE_RD(1, 2) LE_RD(1, 4) LE_RD(1, 8)
#endif

/* ===================================================================================== */
/* Dequant-fused matvec / small-M matmul.                                                    */
/* ===================================================================================== */

/* Launch contract (checked by the host):
 *   cols % 256 == 0; G divides cols/256; x rows 16-byte aligned; blockDim a multiple of 64;
 *   dynamic LDS = T * le_xtok_bytes(cols) + (IQ types) 4 * (256 + GRID_WORDS).
 * Grid: x = row-block workers, y = slot, z = token chunk of T tokens.
 * Slot s uses weights (ptrs ? ptrs[s] : w0 + s * w_slot_bytes), activations x + s*x_slot + t*x_tok,
 * outputs y + s*y_slot + t*y_tok, token t < ntok. */
struct MvArgs {
    const u8 *const *ptrs;
    const u8 *w0;
    unsigned long long w_slot_bytes;
    const float *x;
    long long x_slot, x_tok;
    float *y;
    long long y_slot, y_tok;
    int rows, cols, ntok;
    int swiglu; /* 1: the activation is silu(x[0, cols)) * x[cols, 2 cols) (le_matvec_swiglu) */
    /* int8 activation mode (le_matvec_q8): xq8 + s * x_slot values, xd8 + s * x_slot / 32 scales */
    const int8_t *xq8;
    const float *xd8;
};

template <int TY>
__device__ __forceinline__ void load_tables(u32 *tab) {
    if constexpr (Fmt<TY>::TABLES) {
        for (int i = threadIdx.x; i < 128; i += blockDim.x) {
            const u32 s = ksign_dev((u32)i);
            u32 m0 = 0, m1 = 0;
#pragma unroll
            for (int j = 0; j < 4; j++) {
                m0 |= ((s >> j) & 1u) ? (0xFFu << (8 * j)) : 0u;
                m1 |= ((s >> (j + 4)) & 1u) ? (0xFFu << (8 * j)) : 0u;
            }
            tab[LE_TAB_SIGN + 2 * i] = m0;
            tab[LE_TAB_SIGN + 2 * i + 1] = m1;
        }
        const u32 *src = TY == LE_TYPE_IQ2_XXS ? le_iq2xxs_grid : TY == LE_TYPE_IQ3_XXS ? le_iq3xxs_grid : le_iq2s_grid;
        for (int i = threadIdx.x; i < Fmt<TY>::GRID_WORDS; i += blockDim.x) tab[LE_TAB_GRID + i] = src[i];
    }
}

/* Dot of RW decoded rows (same columns) against one token: the LDS reads are shared by the rows.
 * The integer chain runs over the xh plane, is scaled by 128, and continues over the xl plane,
 * giving sum(q * v) with v = 128*xh + xl in one int32. */
template <int NSEG, int WPS, bool HAS_MU, int RW>
__device__ __forceinline__ void rows_dot(const Dec<NSEG, WPS> (&d)[RW], const XTok &x, int sb, int li, float (&c)[RW]) {
    const int base = 32 * sb + li, xr = sb & 3;
#pragma unroll
    for (int k = 0; k < NSEG; k++) {
        uint4 q[WPS / 2];
        float fs = 0.f, dx = 0.f;
#pragma unroll
        for (int g = 0; g < WPS / 2; g++) {
            const int pos = base + 8 * ((k * (WPS / 2) + g) ^ xr);
            q[g] = x.xq[pos];
            const float2 s = x.xs[pos];
            dx = s.x;
            if (HAS_MU) fs += s.y;
        }
#pragma unroll
        for (int i = 0; i < RW; i++) {
            int acc = 0;
#pragma unroll
            for (int g = 0; g < WPS / 2; g++) {
                acc = dot4(d[i].w[k * WPS + 2 * g], q[g].x, acc);
                acc = dot4(d[i].w[k * WPS + 2 * g + 1], q[g].y, acc);
            }
            acc <<= 7;
#pragma unroll
            for (int g = 0; g < WPS / 2; g++) {
                acc = dot4(d[i].w[k * WPS + 2 * g], q[g].z, acc);
                acc = dot4(d[i].w[k * WPS + 2 * g + 1], q[g].w, acc);
            }
            c[i] = __builtin_fmaf(d[i].sig[k], (float)acc * dx, c[i]);
            if (HAS_MU) c[i] = __builtin_fmaf(-d[i].mu[k], fs, c[i]);
        }
    }
}

/* Each wave owns row-blocks of RW*RPW rows (RPW = 8/G rows side by side, G lane groups of 8 per
 * row) and walks them in steps of CH super-blocks per lane and row. Steps are double-buffered:
 * the loads of step n+1 are in flight while step n is decoded and multiplied, and the first
 * step's loads are issued before the activation prologue so HBM latency overlaps it. */
template <int TY, int G, int T, int RW, int CH, int BLOCK, bool Q8 = false>
__device__ __forceinline__ void mv_body(const MvArgs &a) {
    using F = Fmt<TY>;
    using D = Dec<F::NSEG, F::WPS>;
    using Raw = typename F::Raw;
    extern __shared__ uint4 smem[];
    const int K = a.cols, nsb = K >> 8, ng = K >> 3;
    const int slot = blockIdx.y, t0 = blockIdx.z * T;
    const int nt = min(T, a.ntok - t0);
    const u8 *W = a.ptrs ? a.ptrs[slot] : a.w0 + (size_t)slot * a.w_slot_bytes;
    const size_t rb = (size_t)nsb * F::SB;
    constexpr int nwave = BLOCK / 64;
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    constexpr int RPW = 8 / G;
    const int li = lane & 7, g = (lane >> 3) % G, rsub = lane / (8 * G);
    const int S = nsb / G, nch = (S + CH - 1) / CH;
    const int nrb = (a.rows + RPW * RW - 1) / (RPW * RW);
    const int rstride = gridDim.x * nwave;

    auto issue = [&](Raw (&raw)[RW][CH], int rbk, int c) {
#pragma unroll
        for (int i = 0; i < RW; i++) {
            const int row = min((rbk * RW + i) * RPW + rsub, a.rows - 1);
            const u8 *wr = W + (size_t)row * rb;
#pragma unroll
            for (int u = 0; u < CH; u++) {
                const int s = c * CH + u;
                if (s < S) raw[i][u] = F::load(wr + (size_t)(g + G * s) * F::SB, li);
            }
        }
    };

    Raw ra[RW][CH], rb2[RW][CH];
    int rbk = blockIdx.x * nwave + wave, c = 0;

    /* LDS: T token images, then the IQ tables. For one token whose groups fit in registers
     * (K/8 <= 4 * blockDim), the activation loads go out before the weight loads. */
    XTok xt[T];
    uint4 *xq = smem;
    float2 *xs = (float2 *)(smem + T * ng);
#pragma unroll
    for (int t = 0; t < T; t++) {
        xt[t].xq = xq + t * ng;
        xt[t].xs = xs + t * ng;
    }
    constexpr int XR = 16384 / 8 / BLOCK; /* register-staged activations up to K = 16384 */
    if constexpr (Q8) {
        const int8_t *xq8 = a.xq8 + a.x_slot * slot;
        const float *xd8 = a.xd8 + (a.x_slot >> 5) * slot;
        if (ng <= XR * BLOCK) {
            XLoadQ8<BLOCK, XR> xl;
            xl.load(xq8, xd8, K);
            if (rbk < nrb) issue(ra, rbk, 0);
            xl.template store<F::XL>(K, xq, xs);
        } else {
            if (rbk < nrb) issue(ra, rbk, 0);
            le_q8_x_lds<F::XL>(xq8, xd8, K, xq, xs);
        }
    } else if (T == 1 && ng <= XR * BLOCK) {
        XLoad<BLOCK, XR> xl;
        const float *x0 = a.x + a.x_slot * slot + a.x_tok * t0;
        xl.load(x0, K, a.swiglu ? x0 + K : nullptr);
        if (rbk < nrb) issue(ra, rbk, 0);
        xl.template store<F::XL>(K, xq, xs);
    } else {
        if (rbk < nrb) issue(ra, rbk, 0);
        for (int t = 0; t < nt; t++) {
            const float *xt_ = a.x + a.x_slot * slot + a.x_tok * (t0 + t);
            le_quant_x_lds<F::XL>(xt_, K, xq + t * ng, xs + t * ng, a.swiglu ? xt_ + K : nullptr);
        }
    }
    u32 *tab = (u32 *)((float2 *)(smem + T * ng) + T * ng);
    load_tables<TY>(tab);
    __syncthreads();

    float acc[T][RW];
#pragma unroll
    for (int t = 0; t < T; t++)
#pragma unroll
        for (int i = 0; i < RW; i++) acc[t][i] = 0.f;

    auto consume = [&](Raw (&raw)[RW][CH], int rbk, int c) {
#pragma unroll
        for (int u = 0; u < CH; u++) {
            const int s = c * CH + u;
            if (s < S) {
                D d[RW];
#pragma unroll
                for (int i = 0; i < RW; i++) F::decode(raw[i][u], li, g + G * s, tab, d[i]);
#pragma unroll
                for (int t = 0; t < T; t++)
                    if (t < nt) rows_dot<F::NSEG, F::WPS, F::HAS_MU, RW>(d, xt[t], g + G * s, li, acc[t]);
            }
        }
        if (c == nch - 1) {
#pragma unroll
            for (int t = 0; t < T; t++)
#pragma unroll
                for (int i = 0; i < RW; i++) acc[t][i] = group_sum<8 * G>(acc[t][i]);
            if ((lane & (8 * G - 1)) == 0) {
#pragma unroll
                for (int i = 0; i < RW; i++) {
                    const int row = (rbk * RW + i) * RPW + rsub;
                    if (row < a.rows) {
#pragma unroll
                        for (int t = 0; t < T; t++)
                            if (t < nt) a.y[a.y_slot * slot + a.y_tok * (t0 + t) + row] = acc[t][i];
                    }
                }
            }
#pragma unroll
            for (int t = 0; t < T; t++)
#pragma unroll
                for (int i = 0; i < RW; i++) acc[t][i] = 0.f;
        }
    };

    /* ping-pong over the wave's (row-block, step) sequence */
    while (rbk < nrb) {
        int r1 = rbk, c1 = c + 1;
        if (c1 == nch) { c1 = 0; r1 += rstride; }
        if (r1 < nrb) issue(rb2, r1, c1);
        consume(ra, rbk, c);
        rbk = r1;
        c = c1;
        if (rbk >= nrb) break;
        int r2 = rbk, c2 = c + 1;
        if (c2 == nch) { c2 = 0; r2 += rstride; }
        if (r2 < nrb) issue(ra, r2, c2);
        consume(rb2, rbk, c);
        rbk = r2;
        c = c2;
    }
}

#define LE_MV(TY, G, T, RW, CH, BLOCK)                                                                        \
    extern "C" __global__ void __launch_bounds__(BLOCK) le_mv_##TY##_g##G##_t##T##_r##RW##_c##CH##_b##BLOCK(   \
        MvArgs a) {                                                                                           \
        mv_body<TY, G, T, RW, CH, BLOCK>(a);                                                                  \
    }
/* T = 1 (decode): four (rows, steps) shapes at 512 and 1024 threads; T > 1: two shapes at 256. */
#define LE_MV_T1B(TY, G, B) LE_MV(TY, G, 1, 1, 2, B) LE_MV(TY, G, 1, 2, 1, B) LE_MV(TY, G, 1, 2, 2, B) LE_MV(TY, G, 1, 4, 1, B)
#define LE_MV_T1(TY, G) LE_MV_T1B(TY, G, 512) LE_MV_T1B(TY, G, 1024)
#define LE_MV_TN(TY, G, T) LE_MV(TY, G, T, 2, 2, 256) LE_MV(TY, G, T, 4, 1, 256)
#define LE_MV_G(TY, G) LE_MV_T1(TY, G) LE_MV_TN(TY, G, 2) LE_MV_TN(TY, G, 4) LE_MV_TN(TY, G, 8)
#define LE_MV_ALL(TY) LE_MV_G(TY, 1) LE_MV_G(TY, 2) LE_MV_G(TY, 4) LE_MV_G(TY, 8) LE_MVQ8_ALL(TY)
/* int8 activation mode: T = 1, the shapes of the decode matvec */
#define LE_MVQ8(TY, G, RW, CH, BLOCK)                                                                       \
    extern "C" __global__ void __launch_bounds__(BLOCK) le_mv_##TY##_g##G##_t1_r##RW##_c##CH##_b##BLOCK##_q8( \
        MvArgs a) {                                                                                           \
        mv_body<TY, G, 1, RW, CH, BLOCK, true>(a);                                                            \
    }
#define LE_MVQ8_B(TY, G, B) LE_MVQ8(TY, G, 1, 2, B) LE_MVQ8(TY, G, 2, 1, B) LE_MVQ8(TY, G, 2, 2, B) LE_MVQ8(TY, G, 4, 1, B)
#define LE_MVQ8_G(TY, G) LE_MVQ8_B(TY, G, 512) LE_MVQ8_B(TY, G, 1024)
#define LE_MVQ8_ALL(TY) LE_MVQ8_G(TY, 1) LE_MVQ8_G(TY, 2) LE_MVQ8_G(TY, 4) LE_MVQ8_G(TY, 8)

/* ===================================================================================== */
/* MFMA matvec (decode, one token).                                                          */
/* ===================================================================================== */
/* v_mfma_i32_16x16x64_i8 computes D[16x16] += A[16x64] . B[64x16]; lane l holds A row l%16 and B
 * column l%16 over K-slice l/16 (16 int8 each), and D[4*(l/16)+i][l%16] for i < 4. The matvec
 * uses B = 16 weight rows (one tile) and A rows m = (plane p, sub-block j), m = 8p + j, holding
 * the activation plane p (0: xh, 1: xl) only in the K-slices that belong to sub-block j and zero
 * elsewhere. Four MFMAs cover a 256-value super-block and leave D[(p,j)][n] = sum over sub-block
 * j of q * x_p for every row n, so the per-sub-block scales are applied once per super-block in a
 * short epilogue instead of per weight.
 *
 * Q4_K K-slices: lane (n, s) loads qs bytes 16s..16s+15 (load 0) and 64+16s.. (load 1) of its
 * row's super-block. MFMA b uses the low nibbles (b even) or high nibbles (b odd) of load b/2, so
 * slice s of MFMA b is sub-block j(b,s) = 4*(b>>1) + 2*(s>>1) + (b&1), positions 16*(s&1)..+15. */
typedef int le_v4i __attribute__((ext_vector_type(4)));

__device__ __forceinline__ int mq_j(int b, int s) { return 4 * (b >> 1) + 2 * (s >> 1) + (b & 1); }

/* LDS activation image of the MFMA path, per super-block: 16 records of 32 B (record 4b+s holds
 * slice s of MFMA b: 16 B xh, 16 B xl), then dxp[16] (m = 8p+j: dx_j * (p ? 1 : 128)) and fs[8]
 * (dx_j * sum v over sub-block j). */
__host__ __device__ inline int le_mq_x_bytes(int K) { return (K / 256) * (512 + 64 + 32); }

/* Segment e = 16 activations: load, then quantize (partner segments e, e^1 share a sub-block). */
__device__ __forceinline__ void mq_load_seg(const float *__restrict__ x, int e, float4 (&v4)[4]) {
    const LE_GLOBAL float4 *xg = (const LE_GLOBAL float4 *)x;
#pragma unroll
    for (int i = 0; i < 4; i++) v4[i] = xg[4 * e + i];
}
/* A decode kernel's activation segment: x itself, or with `swiglu` silu(gate) * up from a
 * gate | up vector (gate at x[0, K), up at x[K, 2K)); the flag is uniform over the launch. The
 * second load is issued either way (without swiglu it re-reads the segment from cache), so the
 * kernels' wait counts do not depend on the flag. */
__device__ __forceinline__ void mq_load_seg_a(const float *__restrict__ x, int e, int K, bool swiglu, float4 (&v4)[4]) {
    float4 u[4];
    mq_load_seg(x, e, v4);
    mq_load_seg(x + (swiglu ? K : 0), e, u);
    if (swiglu) {
#pragma unroll
        for (int i = 0; i < 4; i++) v4[i] = le_silu_mul4(v4[i], u[i]);
    }
}
/* MAP 0 (Q4_K): slice s of MFMA b is sub-block j(b,s) = 4*(b>>1) + 2*(s>>1) + (b&1), positions
 * 16*(s&1)..; MAP 1 (Q6_K): MFMA b = (half b>>1, 16-value index b&1), slice s = quarter, so
 * sub-block j = 4*(b>>1) + s, positions 16*(b&1)... */
/* Store helpers: COH = device-coherent stores (written through to where every XCD reads), for
 * data another block reads in the same launch. */
template <bool COH>
__device__ __forceinline__ void st_u4(uint4 *p, uint4 v) {
    if constexpr (COH) {
        u32 *q = (u32 *)p;
        __hip_atomic_store(q, v.x, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        __hip_atomic_store(q + 1, v.y, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        __hip_atomic_store(q + 2, v.z, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        __hip_atomic_store(q + 3, v.w, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    } else {
        *p = v;
    }
}
template <bool COH>
__device__ __forceinline__ void st_f(float *p, float v) {
    if constexpr (COH)
        __hip_atomic_store(p, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    else
        *p = v;
}

template <int MAP = 0, bool COH = false>
__device__ __forceinline__ void mq_quant_seg(int e, bool store, const float4 (&v4)[4], uint4 *rec, float *dxp, float *fsv) {
    float am = fmaxf(amax8(v4[0], v4[1]), amax8(v4[2], v4[3]));
    am = fmaxf(am, __shfl_xor(am, 1));
    const float inv = am > 0.f ? LE_XSPLIT / am : 0.f;
    const float d = am / LE_XSPLIT;
    u32 hw[4] = {0, 0, 0, 0}, lw[4] = {0, 0, 0, 0};
    int sum = 0;
#pragma unroll
    for (int i = 0; i < 16; i++) {
        const float xv = i % 4 == 0 ? v4[i / 4].x : i % 4 == 1 ? v4[i / 4].y : i % 4 == 2 ? v4[i / 4].z : v4[i / 4].w;
        const int v = (int)rintf(xv * inv);
        const int h = (v + 64) >> 7;
        const int lo = v - (h << 7);
        hw[i >> 2] |= ((u32)h & 255u) << (8 * (i & 3));
        lw[i >> 2] |= ((u32)lo & 255u) << (8 * (i & 3));
        sum += v;
    }
    sum += __shfl_xor(sum, 1);
    if (!store) return;
    const int sb = e >> 4, j = (e & 15) >> 1, c = e & 1;
    const int b = MAP ? 2 * (j >> 2) + c : 2 * (j >> 2) + (j & 1), s = MAP ? (j & 3) : 2 * ((j & 3) >> 1) + c;
    const int r = (sb * 16 + b * 4 + s) * 2;
    st_u4<COH>(rec + r, make_uint4(hw[0], hw[1], hw[2], hw[3]));
    st_u4<COH>(rec + r + 1, make_uint4(lw[0], lw[1], lw[2], lw[3]));
    if (c == 0) {
        st_f<COH>(dxp + sb * 16 + j, d * 128.0f);
        st_f<COH>(dxp + sb * 16 + 8 + j, d);
        st_f<COH>(fsv + sb * 8 + j, d * (float)sum);
    }
}
/* mq_quant_seg for int8 activations (le_matvec_q8): the 16 values of segment e are the caller's
 * xq (|v| <= 127) with its block scale d = xd, split as v = 128 h + lo exactly. */
template <int MAP = 0>
__device__ __forceinline__ void mq_quant_seg_q8(int e, bool store, uint4 q, float d, uint4 *rec, float *dxp, float *fsv) {
    const u32 qw[4] = {q.x, q.y, q.z, q.w};
    u32 hw[4] = {0, 0, 0, 0}, lw[4] = {0, 0, 0, 0};
    int sum = 0;
#pragma unroll
    for (int i = 0; i < 16; i++) {
        const int v = (int)(int8_t)((qw[i >> 2] >> (8 * (i & 3))) & 255u);
        const int h = (v + 64) >> 7;
        const int lo = v - (h << 7);
        hw[i >> 2] |= ((u32)h & 255u) << (8 * (i & 3));
        lw[i >> 2] |= ((u32)lo & 255u) << (8 * (i & 3));
        sum += v;
    }
    sum += __shfl_xor(sum, 1);
    if (!store) return;
    const int sb = e >> 4, j = (e & 15) >> 1, c = e & 1;
    const int b = MAP ? 2 * (j >> 2) + c : 2 * (j >> 2) + (j & 1), s = MAP ? (j & 3) : 2 * ((j & 3) >> 1) + c;
    const int r = (sb * 16 + b * 4 + s) * 2;
    rec[r] = make_uint4(hw[0], hw[1], hw[2], hw[3]);
    rec[r + 1] = make_uint4(lw[0], lw[1], lw[2], lw[3]);
    if (c == 0) {
        dxp[sb * 16 + j] = d * 128.0f;
        dxp[sb * 16 + 8 + j] = d;
        fsv[sb * 8 + j] = d * (float)sum;
    }
}
__device__ __forceinline__ void mq_quant_x(const float *__restrict__ x, int K, uint4 *rec, float *dxp, float *fsv) {
    const int nseg = K >> 4; /* even: partners share trips */
    for (int e = threadIdx.x; e < nseg; e += blockDim.x) {
        float4 v4[4];
        mq_load_seg(x, e, v4);
        mq_quant_seg(e, true, v4, rec, dxp, fsv);
    }
}

/* One block = NW waves on one 16-row tile at a time; wave w takes super-blocks w, w+NW, ... (U
 * per step) and the block sums the waves' partial rows through LDS. */
template <int NW, int U>
__device__ __forceinline__ void mq_q4k_body(const MvArgs &a) {
    extern __shared__ uint4 smem[];
    const int K = a.cols, nsb = K >> 8;
    const int slot = blockIdx.y;
    const u8 *W = a.ptrs ? a.ptrs[slot] : a.w0 + (size_t)slot * a.w_slot_bytes;
    const size_t rb = (size_t)nsb * 144;
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const int n = lane & 15, sq = lane >> 4;
    uint4 *rec = smem;
    float *dxp = (float *)(smem + nsb * 32);
    float *fsv = dxp + nsb * 16;
    float *red = fsv + nsb * 8; /* NW * 16 partial rows */
    const int ntile = (a.rows + 15) >> 4;

    mq_quant_x(a.x + a.x_slot * slot, K, rec, dxp, fsv);
    __syncthreads();

    /* exec-masked A operands: lane (m = l%16, s = l/16) of MFMA b is live iff m%8 == j(b, s) */
    const int m = lane & 15, p = m >> 3, jm = m & 7;
    bool live[4];
#pragma unroll
    for (int b = 0; b < 4; b++) live[b] = jm == mq_j(b, sq);
    le_v4i A[4];
#pragma unroll
    for (int b = 0; b < 4; b++) A[b] = (le_v4i){0, 0, 0, 0};

    const int pe = sq >> 1, jb = 4 * (sq & 1);
    for (int tile = blockIdx.x; tile < ntile; tile += gridDim.x) {
        const int row = min(tile * 16 + n, a.rows - 1);
        const u8 *wr = W + (size_t)row * rb;
        float y = 0.f;
        for (int s0 = wave; s0 < nsb; s0 += NW * U) {
            uint4 hd[U], l0[U], l1[U];
#pragma unroll
            for (int u = 0; u < U; u++) {
                const int sb = min(s0 + u * NW, nsb - 1);
                const u8 *pb = wr + (size_t)sb * 144;
                hd[u] = ldg16c(pb);
                l0[u] = ldg16(pb + 16 + 16 * sq);
                l1[u] = ldg16(pb + 80 + 16 * sq);
            }
#pragma unroll
            for (int u = 0; u < U; u++) {
                const int sb = s0 + u * NW;
                if (sb < nsb) {
#pragma unroll
                    for (int b = 0; b < 4; b++)
                        if (live[b]) {
                            const uint4 v = rec[(sb * 16 + b * 4 + sq) * 2 + p];
                            A[b] = (le_v4i){(int)v.x, (int)v.y, (int)v.z, (int)v.w};
                        }
                    const le_v4i B0 = {(int)(l0[u].x & 0x0F0F0F0Fu), (int)(l0[u].y & 0x0F0F0F0Fu),
                                       (int)(l0[u].z & 0x0F0F0F0Fu), (int)(l0[u].w & 0x0F0F0F0Fu)};
                    const le_v4i B1 = {(int)((l0[u].x >> 4) & 0x0F0F0F0Fu), (int)((l0[u].y >> 4) & 0x0F0F0F0Fu),
                                       (int)((l0[u].z >> 4) & 0x0F0F0F0Fu), (int)((l0[u].w >> 4) & 0x0F0F0F0Fu)};
                    const le_v4i B2 = {(int)(l1[u].x & 0x0F0F0F0Fu), (int)(l1[u].y & 0x0F0F0F0Fu),
                                       (int)(l1[u].z & 0x0F0F0F0Fu), (int)(l1[u].w & 0x0F0F0F0Fu)};
                    const le_v4i B3 = {(int)((l1[u].x >> 4) & 0x0F0F0F0Fu), (int)((l1[u].y >> 4) & 0x0F0F0F0Fu),
                                       (int)((l1[u].z >> 4) & 0x0F0F0F0Fu), (int)((l1[u].w >> 4) & 0x0F0F0F0Fu)};
                    le_v4i D = __builtin_amdgcn_mfma_i32_16x16x64_i8(A[0], B0, (le_v4i){0, 0, 0, 0}, 0, 0, 0);
                    D = __builtin_amdgcn_mfma_i32_16x16x64_i8(A[1], B1, D, 0, 0, 0);
                    D = __builtin_amdgcn_mfma_i32_16x16x64_i8(A[2], B2, D, 0, 0, 0);
                    D = __builtin_amdgcn_mfma_i32_16x16x64_i8(A[3], B3, D, 0, 0, 0);
                    /* epilogue: lane (n, sq) holds D[(pe, jb+i)][n], i < 4 */
                    const u32 sy = hd[u].y, sz = hd[u].z, sw = hd[u].w;
                    const u32 tsc = (sq & 1) ? ((sw & 0x0F0F0F0Fu) | ((sy >> 2) & 0x30303030u)) : (sy & 0x3F3F3F3Fu);
                    const u32 tm = (sq & 1) ? (((sw >> 4) & 0x0F0F0F0Fu) | ((sz >> 2) & 0x30303030u)) : (sz & 0x3F3F3F3Fu);
                    const float4 dq = *(const float4 *)(dxp + sb * 16 + pe * 8 + jb);
                    const float t = (float)(tsc & 255u) * dq.x * (float)D[0] + (float)((tsc >> 8) & 255u) * dq.y * (float)D[1] +
                                    (float)((tsc >> 16) & 255u) * dq.z * (float)D[2] + (float)(tsc >> 24) * dq.w * (float)D[3];
                    const float2 f2 = *(const float2 *)(fsv + sb * 8 + jb + 2 * pe);
                    const u32 mm = tm >> (16 * pe);
                    const float mt = (float)(mm & 255u) * f2.x + (float)((mm >> 8) & 255u) * f2.y;
                    y += h2f(hd[u].x & 0xFFFFu) * t - h2f(hd[u].x >> 16) * mt;
                }
            }
        }
        /* sum the four slices of row n, then the NW waves */
        y = row4_sum(y);
        if (lane < 16) red[wave * 16 + lane] = y;
        __syncthreads();
        if (wave == 0 && lane < 16) {
            float acc = 0.f;
#pragma unroll
            for (int w = 0; w < NW; w++) acc += red[w * 16 + lane];
            const int r = tile * 16 + lane;
            if (r < a.rows) a.y[a.y_slot * slot + r] = acc;
        }
        __syncthreads();
    }
}

/* Block barrier that waits for this wave's LDS traffic only: global loads in flight (weight
 * prefetch) stay in flight, unlike __syncthreads, which is a workgroup fence and waits for all
 * of them. For data exchanged through LDS. */
__device__ __forceinline__ void le_lds_barrier() {
    __asm__ volatile("" ::: "memory");
    __builtin_amdgcn_s_waitcnt(0xC07F); /* lgkmcnt(0) */
    __builtin_amdgcn_s_barrier();
    __asm__ volatile("" ::: "memory");
}

/* Per-super-block MFMA step of the staged kernels, shared by the decode matvec and the MoE
 * kernels. Lane (row n = lane&15, slice sq = lane>>4); A[b] holds the activation image slice of
 * MFMA b for the lane's A row m = lane&15 (plane m>>3, sub-block m&7) where that row is live, and
 * zero elsewhere. Returns the lane's share of row n's dot product over the super-block (the four
 * sq lanes of a row are summed by the caller). */
struct MsLane {
    int sq, p, pe, jb;
    bool live[4];
};
template <int MAP>
__device__ __forceinline__ MsLane ms_lane(int lane) {
    MsLane L;
    const int m = lane & 15;
    L.sq = lane >> 4;
    L.p = m >> 3;
    L.pe = L.sq >> 1;
    L.jb = 4 * (L.sq & 1);
#pragma unroll
    for (int b = 0; b < 4; b++) L.live[b] = (m & 7) == (MAP ? 4 * (b >> 1) + L.sq : mq_j(b, L.sq));
    return L;
}
__device__ __forceinline__ void ms_load_a(const uint4 *rec_sb, const MsLane &L, le_v4i (&A)[4]) {
#pragma unroll
    for (int b = 0; b < 4; b++)
        if (L.live[b]) {
            const uint4 v = rec_sb[(b * 4 + L.sq) * 2 + L.p];
            A[b] = (le_v4i){(int)v.x, (int)v.y, (int)v.z, (int)v.w};
        }
}
/* Q4_K: sbp = the row's staged super-block (header chunk, then 8 quant chunks). */
__device__ __forceinline__ float ms_sb_q4k(const uint4 *sbp, const le_v4i (&A)[4], const float *dxp_sb, const float *fsv_sb,
                                           const MsLane &L) {
    const int sq = L.sq;
    const uint4 hd = sbp[0], l0 = sbp[1 + sq], l1 = sbp[5 + sq];
    const le_v4i B0 = {(int)(l0.x & 0x0F0F0F0Fu), (int)(l0.y & 0x0F0F0F0Fu), (int)(l0.z & 0x0F0F0F0Fu), (int)(l0.w & 0x0F0F0F0Fu)};
    const le_v4i B1 = {(int)((l0.x >> 4) & 0x0F0F0F0Fu), (int)((l0.y >> 4) & 0x0F0F0F0Fu), (int)((l0.z >> 4) & 0x0F0F0F0Fu),
                       (int)((l0.w >> 4) & 0x0F0F0F0Fu)};
    const le_v4i B2 = {(int)(l1.x & 0x0F0F0F0Fu), (int)(l1.y & 0x0F0F0F0Fu), (int)(l1.z & 0x0F0F0F0Fu), (int)(l1.w & 0x0F0F0F0Fu)};
    const le_v4i B3 = {(int)((l1.x >> 4) & 0x0F0F0F0Fu), (int)((l1.y >> 4) & 0x0F0F0F0Fu), (int)((l1.z >> 4) & 0x0F0F0F0Fu),
                       (int)((l1.w >> 4) & 0x0F0F0F0Fu)};
    le_v4i D = __builtin_amdgcn_mfma_i32_16x16x64_i8(A[0], B0, (le_v4i){0, 0, 0, 0}, 0, 0, 0);
    D = __builtin_amdgcn_mfma_i32_16x16x64_i8(A[1], B1, D, 0, 0, 0);
    D = __builtin_amdgcn_mfma_i32_16x16x64_i8(A[2], B2, D, 0, 0, 0);
    D = __builtin_amdgcn_mfma_i32_16x16x64_i8(A[3], B3, D, 0, 0, 0);
    const u32 sy = hd.y, sz = hd.z, sw = hd.w;
    const u32 tsc = (sq & 1) ? ((sw & 0x0F0F0F0Fu) | ((sy >> 2) & 0x30303030u)) : (sy & 0x3F3F3F3Fu);
    const u32 tm = (sq & 1) ? (((sw >> 4) & 0x0F0F0F0Fu) | ((sz >> 2) & 0x30303030u)) : (sz & 0x3F3F3F3Fu);
    const float4 dq = *(const float4 *)(dxp_sb + L.pe * 8 + L.jb);
    const float t = (float)(tsc & 255u) * dq.x * (float)D[0] + (float)((tsc >> 8) & 255u) * dq.y * (float)D[1] +
                    (float)((tsc >> 16) & 255u) * dq.z * (float)D[2] + (float)(tsc >> 24) * dq.w * (float)D[3];
    const float2 f2 = *(const float2 *)(fsv_sb + L.jb + 2 * L.pe);
    const u32 mm = tm >> (16 * L.pe);
    const float mt = (float)(mm & 255u) * f2.x + (float)((mm >> 8) & 255u) * f2.y;
    return h2f(hd.x & 0xFFFFu) * t - h2f(hd.x >> 16) * mt;
}

/* Q5_K (src/quant.rs:83-95): the Q4_K header chunk, qh in chunks 1-2, the nibbles in chunks 3-10 in
 * Q4_K's order; the code of sub-block j at position l is its nibble + 16 * bit j of qh[l]. Lane
 * sq reads qh bytes 16 (sq & 1) .. of its half, MFMA b takes bit mq_j(b, sq). */
__device__ __forceinline__ float ms_sb_q5k(const uint4 *sbp, const le_v4i (&A)[4], const float *dxp_sb, const float *fsv_sb,
                                           const MsLane &L) {
    const int sq = L.sq, j0 = 2 * (sq >> 1);
    const uint4 hd = sbp[0], qh = sbp[1 + (sq & 1)], l0 = sbp[3 + sq], l1 = sbp[7 + sq];
    auto hb = [&](u32 h, int j) { return ((h >> j) & 0x01010101u) << 4; };
    const le_v4i B0 = {(int)((l0.x & 0x0F0F0F0Fu) | hb(qh.x, j0)), (int)((l0.y & 0x0F0F0F0Fu) | hb(qh.y, j0)),
                       (int)((l0.z & 0x0F0F0F0Fu) | hb(qh.z, j0)), (int)((l0.w & 0x0F0F0F0Fu) | hb(qh.w, j0))};
    const le_v4i B1 = {(int)(((l0.x >> 4) & 0x0F0F0F0Fu) | hb(qh.x, j0 + 1)), (int)(((l0.y >> 4) & 0x0F0F0F0Fu) | hb(qh.y, j0 + 1)),
                       (int)(((l0.z >> 4) & 0x0F0F0F0Fu) | hb(qh.z, j0 + 1)), (int)(((l0.w >> 4) & 0x0F0F0F0Fu) | hb(qh.w, j0 + 1))};
    const le_v4i B2 = {(int)((l1.x & 0x0F0F0F0Fu) | hb(qh.x, j0 + 4)), (int)((l1.y & 0x0F0F0F0Fu) | hb(qh.y, j0 + 4)),
                       (int)((l1.z & 0x0F0F0F0Fu) | hb(qh.z, j0 + 4)), (int)((l1.w & 0x0F0F0F0Fu) | hb(qh.w, j0 + 4))};
    const le_v4i B3 = {(int)(((l1.x >> 4) & 0x0F0F0F0Fu) | hb(qh.x, j0 + 5)), (int)(((l1.y >> 4) & 0x0F0F0F0Fu) | hb(qh.y, j0 + 5)),
                       (int)(((l1.z >> 4) & 0x0F0F0F0Fu) | hb(qh.z, j0 + 5)), (int)(((l1.w >> 4) & 0x0F0F0F0Fu) | hb(qh.w, j0 + 5))};
    le_v4i D = __builtin_amdgcn_mfma_i32_16x16x64_i8(A[0], B0, (le_v4i){0, 0, 0, 0}, 0, 0, 0);
    D = __builtin_amdgcn_mfma_i32_16x16x64_i8(A[1], B1, D, 0, 0, 0);
    D = __builtin_amdgcn_mfma_i32_16x16x64_i8(A[2], B2, D, 0, 0, 0);
    D = __builtin_amdgcn_mfma_i32_16x16x64_i8(A[3], B3, D, 0, 0, 0);
    const u32 sy = hd.y, sz = hd.z, sw = hd.w;
    const u32 tsc = (sq & 1) ? ((sw & 0x0F0F0F0Fu) | ((sy >> 2) & 0x30303030u)) : (sy & 0x3F3F3F3Fu);
    const u32 tm = (sq & 1) ? (((sw >> 4) & 0x0F0F0F0Fu) | ((sz >> 2) & 0x30303030u)) : (sz & 0x3F3F3F3Fu);
    const float4 dq = *(const float4 *)(dxp_sb + L.pe * 8 + L.jb);
    const float t = (float)(tsc & 255u) * dq.x * (float)D[0] + (float)((tsc >> 8) & 255u) * dq.y * (float)D[1] +
                    (float)((tsc >> 16) & 255u) * dq.z * (float)D[2] + (float)(tsc >> 24) * dq.w * (float)D[3];
    const float2 f2 = *(const float2 *)(fsv_sb + L.jb + 2 * L.pe);
    const u32 mm = tm >> (16 * L.pe);
    const float mt = (float)(mm & 255u) * f2.x + (float)((mm >> 8) & 255u) * f2.y;
    return h2f(hd.x & 0xFFFFu) * t - h2f(hd.x >> 16) * mt;
}

/* Q4_K for NT tiles that share the activation (rows sbp + ti * tstride chunks): the MFMAs of the
 * tiles are interleaved, so NT accumulation chains are in flight instead of one. */
template <int NT>
__device__ __forceinline__ void ms_sb_q4k_n(const uint4 *sbp, int tstride, const le_v4i (&A)[4], const float *dxp_sb,
                                            const float *fsv_sb, const MsLane &L, float (&y)[NT]) {
    const int sq = L.sq;
    uint4 hd[NT], l0[NT], l1[NT];
#pragma unroll
    for (int t = 0; t < NT; t++) {
        const uint4 *p = sbp + t * tstride;
        hd[t] = p[0];
        l0[t] = p[1 + sq];
        l1[t] = p[5 + sq];
    }
    le_v4i D[NT];
#pragma unroll
    for (int b = 0; b < 4; b++) {
#pragma unroll
        for (int t = 0; t < NT; t++) {
            const uint4 w = b < 2 ? l0[t] : l1[t];
            const int sh = (b & 1) * 4;
            const le_v4i B = {(int)((w.x >> sh) & 0x0F0F0F0Fu), (int)((w.y >> sh) & 0x0F0F0F0Fu), (int)((w.z >> sh) & 0x0F0F0F0Fu),
                              (int)((w.w >> sh) & 0x0F0F0F0Fu)};
            D[t] = __builtin_amdgcn_mfma_i32_16x16x64_i8(A[b], B, b ? D[t] : (le_v4i){0, 0, 0, 0}, 0, 0, 0);
        }
    }
    const float4 dq = *(const float4 *)(dxp_sb + L.pe * 8 + L.jb);
    const float2 f2 = *(const float2 *)(fsv_sb + L.jb + 2 * L.pe);
#pragma unroll
    for (int t = 0; t < NT; t++) {
        const u32 sy = hd[t].y, sz = hd[t].z, sw = hd[t].w;
        const u32 tsc = (sq & 1) ? ((sw & 0x0F0F0F0Fu) | ((sy >> 2) & 0x30303030u)) : (sy & 0x3F3F3F3Fu);
        const u32 tm = (sq & 1) ? (((sw >> 4) & 0x0F0F0F0Fu) | ((sz >> 2) & 0x30303030u)) : (sz & 0x3F3F3F3Fu);
        const float tt = (float)(tsc & 255u) * dq.x * (float)D[t][0] + (float)((tsc >> 8) & 255u) * dq.y * (float)D[t][1] +
                         (float)((tsc >> 16) & 255u) * dq.z * (float)D[t][2] + (float)(tsc >> 24) * dq.w * (float)D[t][3];
        const u32 mm = tm >> (16 * L.pe);
        const float mt = (float)(mm & 255u) * f2.x + (float)((mm >> 8) & 255u) * f2.y;
        y[t] += h2f(hd[t].x & 0xFFFFu) * tt - h2f(hd[t].x >> 16) * mt;
    }
}

/* Q6_K on the staged MFMA design. A super-block (210 B: ql[128], qh[64], sc[16] int8, d f16,
 * src/quant.rs:96-112) is staged as 14 unaligned 16-byte chunks into a 224-byte LDS slot, so its
 * fields are 16-byte aligned there. MFMA b = (half n = b>>1, 16-value index is = b&1); slice s of
 * lane (row, s) is quarter s of the half: values 128n + 32s + 16is + (0..15), with
 *     q = ((ql[64n + 32(s&1) + 16is + l] >> 4(s>>1)) & 15) | ((qh[32n + 16is + l] >> 2s) & 3) << 4
 * and the int8 code q - 32 (exact, by a bytewise subtraction that cannot borrow across bytes).
 * Sub-block j = 4n + s of 32 values has the two scales sc[2j], sc[2j+1] (its 16-value halves), so
 * the MFMAs of is = 0 and is = 1 accumulate separately and the epilogue adds
 *     d * sum_j dx_j (sc[2j] D0[j] + sc[2j+1] D1[j]). */
__device__ __forceinline__ u32 q6_code(u32 ql, u32 qh, int s) {
    const u32 q = ((ql >> (4 * (s >> 1))) & 0x0F0F0F0Fu) | (((qh >> (2 * s)) & 0x03030303u) << 4);
    return ((q | 0x80808080u) - 0x20202020u) ^ 0x80808080u; /* q - 32 per byte */
}

/* Q6_K: sbp = the row's staged super-block (14 chunks: ql 0-7, qh 8-11, sc 12, d 13). A[b] is the
 * image slice under the Q6_K map (MAP 1). */
/* Byte offset of staged chunk c of a 210-byte Q6_K super-block: chunks 0-12 at 16 c, chunk 13 at
 * 194 (bytes 194-209, ending with d) so no load reads past the super-block, nor past the end of
 * the last row. */
__device__ __forceinline__ int q6_goff(int c) { return c == 13 ? 194 : 16 * c; }
__device__ __forceinline__ float ms_sb_q6k(const uint4 *sbp, const le_v4i (&A)[4], const float *dxp_sb, const MsLane &L) {
    const int sq = L.sq;
    le_v4i D0 = {0, 0, 0, 0}, D1 = {0, 0, 0, 0};
#pragma unroll
    for (int b = 0; b < 4; b++) {
        const int hn = b >> 1, is = b & 1;
        const uint4 l = sbp[4 * hn + 2 * (sq & 1) + is], h = sbp[8 + 2 * hn + is];
        const le_v4i B = {(int)q6_code(l.x, h.x, sq), (int)q6_code(l.y, h.y, sq), (int)q6_code(l.z, h.z, sq),
                          (int)q6_code(l.w, h.w, sq)};
        if (is)
            D1 = __builtin_amdgcn_mfma_i32_16x16x64_i8(A[b], B, D1, 0, 0, 0);
        else
            D0 = __builtin_amdgcn_mfma_i32_16x16x64_i8(A[b], B, D0, 0, 0, 0);
    }
    /* lane: row n, plane pe, sub-blocks jb..jb+3 -> scales sc[2j], sc[2j+1] */
    const uint4 scv = sbp[12];
    const u32 s0w = (sq & 1) ? scv.z : scv.x, s1w = (sq & 1) ? scv.w : scv.y;
    const float4 dq = *(const float4 *)(dxp_sb + L.pe * 8 + L.jb);
    const float dqa[4] = {dq.x, dq.y, dq.z, dq.w};
    float t = 0.f;
#pragma unroll
    for (int i = 0; i < 4; i++) {
        const u32 sw = i < 2 ? s0w : s1w;
        const int sa = (int)(signed char)((sw >> (16 * (i & 1))) & 255u);
        const int sbb = (int)(signed char)((sw >> (16 * (i & 1) + 8)) & 255u);
        t += dqa[i] * ((float)sa * (float)D0[i] + (float)sbb * (float)D1[i]);
    }
    return h2f(sbp[13].w >> 16) * t; /* d: bytes 208-209, the last two of chunk 13 */
}

/* Q3_K (src/quant.rs:113-126), 110 bytes: hm[32], qs[64], 6-bit scales packed in 12 bytes, d. Value
 * e = 128 c + 32 s + l has code ((qs[32 c + l] >> 2 s) & 3) - 4 (hm bit 4 c + s of byte l clear)
 * and scale e / 16 = 8 c + 2 s + l / 16: the Q6_K layout of halves, quarters and 16-value scales,
 * so the Q6_K kernel's map applies. Staged as 7 chunks, the last one at byte 94 (bytes 94-109:
 * the scales from its byte 2, d in its last two), so no load reads past the super-block. */
__device__ __forceinline__ int q3_goff(int c) { return c == 6 ? 94 : 16 * c; }
__device__ __forceinline__ float ms_sb_q3k(const uint4 *sbp, const le_v4i (&A)[4], const float *dxp_sb, const MsLane &L) {
    const int sq = L.sq;
    le_v4i D0 = {0, 0, 0, 0}, D1 = {0, 0, 0, 0};
#pragma unroll
    for (int b = 0; b < 4; b++) {
        const int hn = b >> 1, is = b & 1, hs = 4 * hn + sq, qsft = 2 * sq;
        const uint4 q = sbp[2 + 2 * hn + is], h = sbp[is];
        const u32 w[4] = {q.x, q.y, q.z, q.w}, m[4] = {h.x, h.y, h.z, h.w};
        int o[4];
#pragma unroll
        for (int k = 0; k < 4; k++) /* (code | high bit << 2) - 4 bytewise: (v + 0x7C) ^ 0x80, no carries */
            o[k] = (int)(((((w[k] >> qsft) & 0x03030303u) | (((m[k] >> hs) & 0x01010101u) << 2)) + 0x7C7C7C7Cu) ^ 0x80808080u);
        const le_v4i B = {o[0], o[1], o[2], o[3]};
        if (is)
            D1 = __builtin_amdgcn_mfma_i32_16x16x64_i8(A[b], B, D1, 0, 0, 0);
        else
            D0 = __builtin_amdgcn_mfma_i32_16x16x64_i8(A[b], B, D0, 0, 0, 0);
    }
    /* lane: sub-blocks jb + i (jb = 4 (sq & 1)), scales 2 (jb + i) + is */
    const uint4 c6 = sbp[6];
    const u32 s0 = __builtin_amdgcn_alignbit(c6.y, c6.x, 16), s1 = __builtin_amdgcn_alignbit(c6.z, c6.y, 16),
              s2 = __builtin_amdgcn_alignbit(c6.w, c6.z, 16);
    const int hi = sq & 1;
    const float4 dq = *(const float4 *)(dxp_sb + L.pe * 8 + L.jb);
    const float dqa[4] = {dq.x, dq.y, dq.z, dq.w};
    float t = 0.f;
#pragma unroll
    for (int i = 0; i < 4; i++) {
        int sc[2];
#pragma unroll
        for (int is = 0; is < 2; is++) {
            const int k = 2 * i + is; /* scale index 8 hi + k: low 4 bits in byte k (nibble hi), high 2 in byte 8 + k % 4 */
            const u32 lo = ((k < 4 ? s0 : s1) >> (8 * (k & 3) + 4 * hi)) & 15u;
            const u32 hb = (s2 >> (8 * (k & 3) + 2 * (2 * hi + (i >> 1)))) & 3u;
            sc[is] = (int)(lo | (hb << 4)) - 32;
        }
        t += dqa[i] * ((float)sc[0] * (float)D0[i] + (float)sc[1] * (float)D1[i]);
    }
    return h2f(c6.w >> 16) * t;
}

/* IQ2_S (src/quant.rs:155-167), 82 bytes: d, qs[32] (grid index low bits), signs[32], qh[8] (index
 * high bits), scales[8] (4 bits per 16 values). Sub-block ib is one 32-value block with one scale
 * per 16 values, so the Q6_K kernel's map (two accumulators per sub-block) applies with sub-block
 * j = 4 (b >> 1) + sq and values 16 (b & 1) ... Staged as 6 chunks, the last one at byte 66
 * (bytes 66-81: qh, then the scales), so no load reads past the super-block; slot bytes 0-79 are
 * the super-block's, 80-87 qh, 88-95 the scales. */
__device__ __forceinline__ int i2s_goff(int c) { return c == 5 ? 66 : 16 * c; }
__device__ __forceinline__ float ms_sb_iq2s(const uint4 *sbp, const le_v4i (&A)[4], const float *dxp_sb, const MsLane &L,
                                            const u32 *tab) {
    const int sq = L.sq;
    const u32 *w32 = (const u32 *)sbp, *grid = tab + LE_TAB_GRID;
    le_v4i D0 = {0, 0, 0, 0}, D1 = {0, 0, 0, 0};
#pragma unroll
    for (int b = 0; b < 4; b++) {
        const int hn = b >> 1, is = b & 1, j = 4 * hn + sq;
        /* qs bytes 2 + 4j + 2is, +1 and sign bytes 34 + 4j + 2is, +1 (2 mod 4 aligned) */
        const u32 q16 = is ? (w32[j + 1] & 0xFFFFu) : (w32[j] >> 16);
        const u32 s16 = is ? (w32[9 + j] & 0xFFFFu) : (w32[8 + j] >> 16);
        const u32 qh = (w32[20 + (j >> 2)] >> (8 * (j & 3))) & 255u;
        u32 o[4];
#pragma unroll
        for (int l = 0; l < 2; l++) {
            const int g = 2 * is + l; /* 8-value group of the 32 */
            const u32 gi = ((q16 >> (8 * l)) & 255u) | ((qh << (8 - 2 * g)) & 0x300u);
            const u32 sg = (s16 >> (8 * l)) & 255u;
            const uint2 gv = *(const uint2 *)(grid + 2 * gi);
            o[2 * l] = apply_sign(gv.x, nib_mask(sg & 15u));
            o[2 * l + 1] = apply_sign(gv.y, nib_mask(sg >> 4));
        }
        const le_v4i B = {(int)o[0], (int)o[1], (int)o[2], (int)o[3]};
        if (is)
            D1 = __builtin_amdgcn_mfma_i32_16x16x64_i8(A[b], B, D1, 0, 0, 0);
        else
            D0 = __builtin_amdgcn_mfma_i32_16x16x64_i8(A[b], B, D0, 0, 0, 0);
    }
    /* lane: sub-blocks jb + i (jb = 4 (sq & 1)), 16-value scales 2 ls + 1 (d / 8 outside) */
    const u32 scw = w32[22 + (sq & 1)];
    const float4 dq = *(const float4 *)(dxp_sb + L.pe * 8 + L.jb);
    const float dqa[4] = {dq.x, dq.y, dq.z, dq.w};
    float t = 0.f;
#pragma unroll
    for (int i = 0; i < 4; i++) {
        const u32 sc = (scw >> (8 * i)) & 255u;
        t += dqa[i] * ((float)(2 * (sc & 15u) + 1) * (float)D0[i] + (float)(2 * (sc >> 4) + 1) * (float)D1[i]);
    }
    return h2f(w32[0] & 0xFFFFu) * 0.125f * t;
}

/* Staged variant: each wave streams its tile's P super-blocks per row as consecutive 16-byte
 * chunks (consecutive lanes take consecutive chunks of a row, so every load instruction reads
 * long contiguous runs), prefetched into registers one item ahead and written to a wave-private
 * LDS buffer where one pad chunk per row keeps the 16 rows of a read in distinct banks. MFMA
 * operands then come from LDS. Barriers wait on LDS traffic only, so weight loads in flight are
 * not drained at a barrier. */
template <int P, int NW, bool Q8, int TY = LE_TYPE_Q4_K>
__device__ __forceinline__ void ms_q4k_body(const MvArgs &a) {
    extern __shared__ uint4 smem[];
    constexpr int CPS = TY == LE_TYPE_Q5_K ? 11 : 9; /* 16-byte chunks per super-block (Q4_K, Q5_K) */
    constexpr int CPR = CPS * P + 1, NCH = 16 * CPR, NI = (NCH + 63) / 64;
    const int K = a.cols, nsb = K >> 8;
    const int slot = blockIdx.y;
    const u8 *W = a.ptrs ? a.ptrs[slot] : a.w0 + (size_t)slot * a.w_slot_bytes;
    const size_t rb = (size_t)nsb * (16 * CPS);
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const int n = lane & 15, sq = lane >> 4;
    /* wave-private LDS: the activation image of this wave's super-blocks (local index ls, global
     * super-block (ls/P)*NW*P + wave*P + ls%P), then the staging buffer; the host guarantees
     * nsb % (NW*P) == 0 */
    const int nsbw = nsb / NW;
    uint4 *rec = smem + wave * (nsbw * 38 + NI * 64);
    float *dxp = (float *)(rec + nsbw * 32);
    float *fsv = dxp + nsbw * 16;
    uint4 *wb = (uint4 *)(fsv + nsbw * 8);
    float *red = (float *)(smem + NW * (nsbw * 38 + NI * 64)); /* [2][NW][16] */
    const int ntile = (a.rows + 15) >> 4;

    /* chunk i of this lane: row ri[i] of the tile, byte cb[i] of the row's P-super-block run */
    int ri[NI], cb[NI];
#pragma unroll
    for (int i = 0; i < NI; i++) {
        const int c = min(64 * i + lane, NCH - 1);
        const int col = c % CPR;
        ri[i] = c / CPR;
        cb[i] = (col == CPS * P ? 0 : col) * 16;
    }
    /* register staging: the chunks of the next item are loaded while the current one computes */
    uint4 R[NI];
    auto issue = [&](int tile, int s0) {
#pragma unroll
        for (int i = 0; i < NI; i++) {
            const int row = min(tile * 16 + ri[i], a.rows - 1);
            R[i] = ldg16(W + (size_t)row * rb + (size_t)s0 * (16 * CPS) + cb[i]);
        }
    };
    const int sfirst = wave * P, sstep = NW * P;
    const bool active = sfirst < nsb;
    /* activations of the first segment round go out first (clamped, unpredicated), then the
     * first weight item, so the quantization waits only for the activations */
    const float *xs = a.x + a.x_slot * slot;
    const int nsegw = nsbw * 16;
    auto gseg = [&](int el) { /* local segment -> global segment */
        const int ls = el >> 4;
        return ((ls / P) * sstep + sfirst + ls % P) * 16 + (el & 15);
    };
    if constexpr (Q8) { /* int8 mode (the _q8 kernels): the image holds the caller's xq, scale xd per 32 values (exact) */
        issue(min((int)blockIdx.x, ntile - 1), active ? sfirst : 0); /* unpredicated: exact wait counts */
        const int8_t *xq8 = a.xq8 + a.x_slot * slot;
        const float *xd8 = a.xd8 + (a.x_slot >> 5) * slot;
        for (int el0 = 0; el0 < nsegw; el0 += 64) {
            const int el = el0 + lane, ge = gseg(min(el, nsegw - 1));
            mq_quant_seg_q8<0>(el, el < nsegw, ldg16u((const u8 *)(xq8 + 16 * ge)), xd8[ge >> 1], rec, dxp, fsv);
        }
    } else {
    float4 xv[4];
    mq_load_seg_a(xs, gseg(min(lane, nsegw - 1)), a.cols, a.swiglu, xv);
    issue(min((int)blockIdx.x, ntile - 1), active ? sfirst : 0); /* unpredicated: exact wait counts */
    mq_quant_seg(lane, lane < nsegw, xv, rec, dxp, fsv);
    for (int el = lane + 64; el < nsegw; el += 64) {
        mq_load_seg_a(xs, gseg(el), a.cols, a.swiglu, xv);
        mq_quant_seg(el, true, xv, rec, dxp, fsv);
    }
    }

    const MsLane L = ms_lane<0>(lane);
    le_v4i A[4];
#pragma unroll
    for (int b = 0; b < 4; b++) A[b] = (le_v4i){0, 0, 0, 0};

    int par = 0;
    for (int tile = blockIdx.x; tile < ntile; tile += gridDim.x) {
        float y = 0.f;
        if (active) {
            for (int s0 = sfirst, lb = 0; s0 < nsb; s0 += sstep, lb += P) {
                int nt = tile, ns = s0 + sstep;
                if (ns >= nsb) { ns = sfirst; nt += gridDim.x; }
#pragma unroll
                for (int i = 0; i < NI; i++) wb[64 * i + lane] = R[i];
                if (nt < ntile) issue(nt, ns);
#pragma unroll
                for (int q = 0; q < P; q++) {
                    const int sb = lb + q; /* local super-block of this wave's image */
                    ms_load_a(rec + sb * 32, L, A);
                    if constexpr (TY == LE_TYPE_Q5_K)
                        y += ms_sb_q5k(wb + n * CPR + CPS * q, A, dxp + sb * 16, fsv + sb * 8, L);
                    else
                        y += ms_sb_q4k(wb + n * CPR + CPS * q, A, dxp + sb * 16, fsv + sb * 8, L);
                }
            }
        }
        y = row4_sum(y);
        float *rp = red + par * (NW * 16);
        if (lane < 16) rp[wave * 16 + lane] = y;
        __builtin_amdgcn_s_waitcnt(0xC07F);
        __builtin_amdgcn_s_barrier();
        if (wave == 0 && lane < 16) {
            float acc = 0.f;
#pragma unroll
            for (int w = 0; w < NW; w++) acc += rp[w * 16 + lane];
            const int r = tile * 16 + lane;
            if (r < a.rows) a.y[a.y_slot * slot + r] = acc;
        }
        par ^= 1;
    }
}

/* Q4_K for T tokens on one staged super-block. Token t's image slice of super-block sb is the
 * 33-slot record img[(sb T + t) 33 ..]: slots 0-31 as in the single-token image, slot 32 zero; the
 * scales are token-major per super-block (dxv[(sb T + t) 16 + j], fsv[(sb T + t) 8 + j]). Every
 * token's operand is then one immediate offset (528 B per token) from a shared address, the live
 * lanes of a read stay in adjacent slots (no bank conflicts), and a lane whose A row is not live
 * in MFMA b reads the zero slot (cs[b], fixed per lane). B fragments and row scales are decoded
 * once for all tokens. */
template <int T>
__device__ __forceinline__ void ms_sb_q4k_t(const uint4 *sbp, const uint4 *img, const float *dxv, const float *fsv, int sb,
                                            const int (&cs)[4], const MsLane &L, float (&y)[T]) {
    const int sq = L.sq;
    const uint4 hd = sbp[0], l0 = sbp[1 + sq], l1 = sbp[5 + sq];
    le_v4i D[T];
#pragma unroll
    for (int b = 0; b < 4; b++) {
        const uint4 w = b < 2 ? l0 : l1;
        const int sh = (b & 1) * 4;
        const le_v4i B = {(int)((w.x >> sh) & 0x0F0F0F0Fu), (int)((w.y >> sh) & 0x0F0F0F0Fu), (int)((w.z >> sh) & 0x0F0F0F0Fu),
                          (int)((w.w >> sh) & 0x0F0F0F0Fu)};
        const uint4 *ap = img + sb * T * 33 + cs[b];
#pragma unroll
        for (int t = 0; t < T; t++) {
            const uint4 v = ap[33 * t];
            D[t] = __builtin_amdgcn_mfma_i32_16x16x64_i8((le_v4i){(int)v.x, (int)v.y, (int)v.z, (int)v.w}, B,
                                                         b ? D[t] : (le_v4i){0, 0, 0, 0}, 0, 0, 0);
        }
    }
    const u32 sy = hd.y, sz = hd.z, sw = hd.w;
    const u32 tsc = (sq & 1) ? ((sw & 0x0F0F0F0Fu) | ((sy >> 2) & 0x30303030u)) : (sy & 0x3F3F3F3Fu);
    const u32 tm = (sq & 1) ? (((sw >> 4) & 0x0F0F0F0Fu) | ((sz >> 2) & 0x30303030u)) : (sz & 0x3F3F3F3Fu);
    const float d = h2f(hd.x & 0xFFFFu), dmin = h2f(hd.x >> 16);
    /* d * sc_j and dmin * m_j folded once for all tokens */
    const float c0 = d * (float)(tsc & 255u), c1 = d * (float)((tsc >> 8) & 255u), c2 = d * (float)((tsc >> 16) & 255u),
                c3 = d * (float)(tsc >> 24);
    const u32 mm = tm >> (16 * L.pe);
    const float m0 = dmin * (float)(mm & 255u), m1 = dmin * (float)((mm >> 8) & 255u);
    const float *dq0 = dxv + sb * T * 16 + L.pe * 8 + L.jb, *f0 = fsv + sb * T * 8 + L.jb + 2 * L.pe;
#pragma unroll
    for (int t = 0; t < T; t++) {
        const float4 dq = *(const float4 *)(dq0 + 16 * t);
        const float2 f2 = *(const float2 *)(f0 + 8 * t);
        float acc = y[t] - m0 * f2.x;
        acc = __builtin_fmaf(-m1, f2.y, acc);
        acc = __builtin_fmaf(c0 * dq.x, (float)D[t][0], acc);
        acc = __builtin_fmaf(c1 * dq.y, (float)D[t][1], acc);
        acc = __builtin_fmaf(c2 * dq.z, (float)D[t][2], acc);
        y[t] = __builtin_fmaf(c3 * dq.w, (float)D[t][3], acc);
    }
}

/* The activation split of mq_quant_seg (16 values of one sub-block half, partner lane e^1 holds
 * the other half) stored in the token-interleaved layout of ms_sb_q4k_t (Q4_K slice map). */
template <int T>
__device__ __forceinline__ void mq_quant_seg_t(int e, int t, bool store, const float4 (&v4)[4], uint4 *img, float *dxv,
                                               float *fsv) {
    float am = fmaxf(amax8(v4[0], v4[1]), amax8(v4[2], v4[3]));
    am = fmaxf(am, __shfl_xor(am, 1));
    const float inv = am > 0.f ? LE_XSPLIT / am : 0.f;
    const float d = am / LE_XSPLIT;
    u32 hw[4] = {0, 0, 0, 0}, lw[4] = {0, 0, 0, 0};
    int sum = 0;
#pragma unroll
    for (int i = 0; i < 16; i++) {
        const float xv = i % 4 == 0 ? v4[i / 4].x : i % 4 == 1 ? v4[i / 4].y : i % 4 == 2 ? v4[i / 4].z : v4[i / 4].w;
        const int v = (int)rintf(xv * inv);
        const int h = (v + 64) >> 7;
        const int lo = v - (h << 7);
        hw[i >> 2] |= ((u32)h & 255u) << (8 * (i & 3));
        lw[i >> 2] |= ((u32)lo & 255u) << (8 * (i & 3));
        sum += v;
    }
    sum += __shfl_xor(sum, 1);
    if (!store) return;
    const int sb = e >> 4, j = (e & 15) >> 1, c = e & 1;
    const int b = 2 * (j >> 2) + (j & 1), s = 2 * ((j & 3) >> 1) + c;
    const int r = (sb * 16 + b * 4 + s) * 2;
    uint4 *rt = img + (sb * T + t) * 33;
    rt[r - sb * 32] = make_uint4(hw[0], hw[1], hw[2], hw[3]);
    rt[r - sb * 32 + 1] = make_uint4(lw[0], lw[1], lw[2], lw[3]);
    if (c == 0) {
        dxv[(sb * T + t) * 16 + j] = d * 128.0f;
        dxv[(sb * T + t) * 16 + 8 + j] = d;
        fsv[(sb * T + t) * 8 + j] = d * (float)sum;
    }
}

/* The staged Q4_K matvec for T tokens at once (tokens T*blockIdx.z .. +T-1, clamped to ntok - 1,
 * of which only real ones are stored): the weight stream is the single-token kernel's, each wave
 * keeps T activation images, and every decoded weight fragment feeds T MFMA chains. */
template <int P, int NW, int T>
__device__ __forceinline__ void ms_q4k_t_body(const MvArgs &a) {
    extern __shared__ uint4 smem[];
    constexpr int CPR = 9 * P + 1, NCH = 16 * CPR, NI = (NCH + 63) / 64;
    const int K = a.cols, nsb = K >> 8;
    const int slot = blockIdx.y, tok0 = T * blockIdx.z;
    const u8 *W = a.ptrs ? a.ptrs[slot] : a.w0 + (size_t)slot * a.w_slot_bytes;
    const size_t rb = (size_t)nsb * 144;
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const int n = lane & 15;
    /* wave-private LDS: the T token-interleaved images of this wave's super-blocks, T zero slots,
     * the scales and sums, then the staging buffer */
    const int nsbw = nsb / NW, wsz = nsbw * 39 * T;
    uint4 *img = smem + wave * (wsz + NI * 64);
    float *dxv = (float *)(img + nsbw * T * 33), *fsv = dxv + nsbw * T * 16;
    uint4 *wb = img + wsz;
    float *red = (float *)(smem + NW * (wsz + NI * 64)); /* [2][NW][T][16] */
    for (int i = lane; i < nsbw * T; i += 64) img[33 * i + 32] = make_uint4(0u, 0u, 0u, 0u);
    const int ntile = (a.rows + 15) >> 4;

    int ri[NI], cb[NI];
#pragma unroll
    for (int i = 0; i < NI; i++) {
        const int c = min(64 * i + lane, NCH - 1);
        const int col = c % CPR;
        ri[i] = c / CPR;
        cb[i] = (col == 9 * P ? 0 : col) * 16;
    }
    uint4 R[NI];
    auto issue = [&](int tile, int s0) {
#pragma unroll
        for (int i = 0; i < NI; i++) {
            const int row = min(tile * 16 + ri[i], a.rows - 1);
            R[i] = ldg16(W + (size_t)row * rb + (size_t)s0 * 144 + cb[i]);
        }
    };
    const int sfirst = wave * P, sstep = NW * P;
    const bool active = sfirst < nsb;
    issue(min((int)blockIdx.x, ntile - 1), active ? sfirst : 0);
    /* the T tokens' images: element el = (token el / nsegw, local segment el % nsegw); the two
     * segments of a sub-block sit in partner lanes */
    const int nsegw = nsbw * 16, nel = T * nsegw;
    constexpr int QB = 4; /* element rounds whose loads are in flight together */
    for (int base = 0; base < nel; base += 64 * QB) {
        float4 xv[QB][4];
#pragma unroll
        for (int u = 0; u < QB; u++) {
            const int el = min(base + 64 * u + lane, nel - 1);
            const int t = el / nsegw, e = el - t * nsegw, ls = e >> 4;
            const float *xs = a.x + a.x_slot * slot + a.x_tok * min(tok0 + t, a.ntok - 1);
            mq_load_seg(xs, ((ls / P) * sstep + sfirst + ls % P) * 16 + (e & 15), xv[u]);
        }
#pragma unroll
        for (int u = 0; u < QB; u++) {
            if (base + 64 * u >= nel) break; /* wave-uniform */
            const int el = base + 64 * u + lane, elc = min(el, nel - 1);
            const int t = elc / nsegw, e = elc - t * nsegw;
            mq_quant_seg_t<T>(e, t, el < nel, xv[u], img, dxv, fsv);
        }
    }

    const MsLane L = ms_lane<0>(lane);
    int cs[4]; /* the lane's slot in a record for MFMA b: its image slice, or the zero slot */
#pragma unroll
    for (int b = 0; b < 4; b++) cs[b] = L.live[b] ? (b * 4 + L.sq) * 2 + L.p : 32;
    int par = 0;
    for (int tile = blockIdx.x; tile < ntile; tile += gridDim.x) {
        float y[T];
#pragma unroll
        for (int t = 0; t < T; t++) y[t] = 0.f;
        if (active) {
            for (int s0 = sfirst, lb = 0; s0 < nsb; s0 += sstep, lb += P) {
                int nt = tile, ns = s0 + sstep;
                if (ns >= nsb) { ns = sfirst; nt += gridDim.x; }
#pragma unroll
                for (int i = 0; i < NI; i++) wb[64 * i + lane] = R[i];
                if (nt < ntile) issue(nt, ns);
#pragma unroll
                for (int q = 0; q < P; q++) ms_sb_q4k_t<T>(wb + n * CPR + 9 * q, img, dxv, fsv, lb + q, cs, L, y);
            }
        }
        float *rp = red + par * (NW * T * 16);
#pragma unroll
        for (int t = 0; t < T; t++) {
            float v = y[t];
            v = row4_sum(v);
            if (lane < 16) rp[(wave * T + t) * 16 + lane] = v;
        }
        __builtin_amdgcn_s_waitcnt(0xC07F);
        __builtin_amdgcn_s_barrier();
        if (wave == 0) {
#pragma unroll
            for (int o = lane; o < T * 16; o += 64) {
                const int t = o >> 4, r = tile * 16 + (o & 15);
                float acc = 0.f;
#pragma unroll
                for (int w = 0; w < NW; w++) acc += rp[(w * T + t) * 16 + (o & 15)];
                if (r < a.rows && tok0 + t < a.ntok) a.y[a.y_slot * slot + a.y_tok * (tok0 + t) + r] = acc;
            }
        }
        par ^= 1;
    }
}

template <int P, int NW, bool Q8, int TY = LE_TYPE_Q6_K>
__device__ __forceinline__ void ms_q6k_body(const MvArgs &a) {
    extern __shared__ uint4 smem[];
    constexpr bool Q3 = TY == LE_TYPE_Q3_K, S2 = TY == LE_TYPE_IQ2_S;
    constexpr int CPS = Q3 ? 7 : S2 ? 6 : 14, SBB = Q3 ? 110 : S2 ? 82 : 210, CPR = CPS * P + 1, NCH = 16 * CPR, NI = (NCH + 63) / 64;
    const int K = a.cols, nsb = K >> 8;
    const int slot = blockIdx.y;
    const u8 *W = a.ptrs ? a.ptrs[slot] : a.w0 + (size_t)slot * a.w_slot_bytes;
    const size_t rb = (size_t)nsb * SBB;
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const int n = lane & 15, sq = lane >> 4;
    const int nsbw = nsb / NW;
    uint4 *rec = smem + wave * (nsbw * 38 + NI * 64);
    float *dxp = (float *)(rec + nsbw * 32);
    float *fsv = dxp + nsbw * 16;
    uint4 *wb = (uint4 *)(fsv + nsbw * 8);
    float *red = (float *)(smem + NW * (nsbw * 38 + NI * 64)); /* [2][NW][16] */
    const int ntile = (a.rows + 15) >> 4;
    __shared__ u32 tab[S2 ? LE_TAB_GRID + 2048 : 1]; /* IQ2_S: sign masks and the 1024-entry grid */
    if constexpr (S2) {
        load_tables<TY>(tab);
        __syncthreads();
    }

    /* chunk i of this lane: row ri[i] of the tile, global byte gb[i] and LDS chunk index of the
     * row's P-super-block run (the pad chunk re-reads chunk 0) */
    int ri[NI], gb[NI];
#pragma unroll
    for (int i = 0; i < NI; i++) {
        const int c = min(64 * i + lane, NCH - 1);
        const int col = c % CPR, cc = col == CPS * P ? 0 : col;
        ri[i] = c / CPR;
        gb[i] = (cc / CPS) * SBB + (Q3 ? q3_goff(cc % CPS) : S2 ? i2s_goff(cc % CPS) : q6_goff(cc % CPS));
    }
    uint4 R[NI];
    auto issue = [&](int tile, int s0) {
#pragma unroll
        for (int i = 0; i < NI; i++) {
            const int row = min(tile * 16 + ri[i], a.rows - 1);
            R[i] = ldg16u(W + (size_t)row * rb + (size_t)s0 * SBB + gb[i]);
        }
    };
    const int sfirst = wave * P, sstep = NW * P;
    const bool active = sfirst < nsb;
    const float *xs = a.x + a.x_slot * slot;
    const int nsegw = nsbw * 16;
    auto gseg = [&](int el) {
        const int ls = el >> 4;
        return ((ls / P) * sstep + sfirst + ls % P) * 16 + (el & 15);
    };
    if constexpr (Q8) { /* int8 mode (the _q8 kernels): the image holds the caller's xq, scale xd per 32 values (exact) */
        issue(min((int)blockIdx.x, ntile - 1), active ? sfirst : 0);
        const int8_t *xq8 = a.xq8 + a.x_slot * slot;
        const float *xd8 = a.xd8 + (a.x_slot >> 5) * slot;
        for (int el0 = 0; el0 < nsegw; el0 += 64) {
            const int el = el0 + lane, ge = gseg(min(el, nsegw - 1));
            mq_quant_seg_q8<1>(el, el < nsegw, ldg16u((const u8 *)(xq8 + 16 * ge)), xd8[ge >> 1], rec, dxp, fsv);
        }
    } else {
    float4 xv[4];
    mq_load_seg_a(xs, gseg(min(lane, nsegw - 1)), a.cols, a.swiglu, xv);
    issue(min((int)blockIdx.x, ntile - 1), active ? sfirst : 0);
    mq_quant_seg<1>(lane, lane < nsegw, xv, rec, dxp, fsv);
    for (int el = lane + 64; el < nsegw; el += 64) {
        mq_load_seg_a(xs, gseg(el), a.cols, a.swiglu, xv);
        mq_quant_seg<1>(el, true, xv, rec, dxp, fsv);
    }
    }

    const MsLane L = ms_lane<1>(lane);
    le_v4i A[4];
#pragma unroll
    for (int b = 0; b < 4; b++) A[b] = (le_v4i){0, 0, 0, 0};

    int par = 0;
    for (int tile = blockIdx.x; tile < ntile; tile += gridDim.x) {
        float y = 0.f;
        if (active) {
            for (int s0 = sfirst, lb = 0; s0 < nsb; s0 += sstep, lb += P) {
                int nt = tile, ns = s0 + sstep;
                if (ns >= nsb) { ns = sfirst; nt += gridDim.x; }
#pragma unroll
                for (int i = 0; i < NI; i++) wb[64 * i + lane] = R[i];
                if (nt < ntile) issue(nt, ns);
#pragma unroll
                for (int q = 0; q < P; q++) {
                    const int sb = lb + q;
                    ms_load_a(rec + sb * 32, L, A);
                    if constexpr (Q3)
                        y += ms_sb_q3k(wb + n * CPR + CPS * q, A, dxp + sb * 16, L);
                    else if constexpr (S2)
                        y += ms_sb_iq2s(wb + n * CPR + CPS * q, A, dxp + sb * 16, L, tab);
                    else
                        y += ms_sb_q6k(wb + n * CPR + CPS * q, A, dxp + sb * 16, L);
                }
            }
        }
        y = row4_sum(y);
        float *rp = red + par * (NW * 16);
        if (lane < 16) rp[wave * 16 + lane] = y;
        __builtin_amdgcn_s_waitcnt(0xC07F);
        __builtin_amdgcn_s_barrier();
        if (wave == 0 && lane < 16) {
            float acc = 0.f;
#pragma unroll
            for (int w = 0; w < NW; w++) acc += rp[w * 16 + lane];
            const int r = tile * 16 + lane;
            if (r < a.rows) a.y[a.y_slot * slot + r] = acc;
        }
        par ^= 1;
    }
}

#define LE_MS14(P, NW)                                                                                     \
    extern "C" __global__ void __launch_bounds__(NW * 64) le_ms_14_p##P##_w##NW(MvArgs a) { ms_q6k_body<P, NW, false>(a); } \
    extern "C" __global__ void __launch_bounds__(NW * 64) le_ms_14_p##P##_w##NW##_q8(MvArgs a) { ms_q6k_body<P, NW, true>(a); }

/* IQ2_XXS / IQ3_XXS on the staged MFMA design, under the Q4_K slice map (slice s of MFMA b is
 * sub-block j = 4*(b>>1) + 2*(s>>1) + (b&1), values 16*(s&1)..+15). A super-block is staged from
 * byte 2 (its quant bytes then start 16-byte aligned in LDS) plus one chunk from byte 0 holding d:
 *   IQ2_XXS (66 B, src/quant.rs:142-154): chunks 0-3 = per sub-block j the grid indices (4 bytes at
 *     8j) and aux (u32 at 8j+4: four 7-bit ksign indices, scale aux>>28); chunk 4 = d.
 *   IQ3_XXS (98 B, src/quant.rs:127-141): chunks 0-3 = grid indices (8 per sub-block at 8j), chunks
 *     4-5 = aux words (u32 at 64+4j), chunk 6 = d.
 * The lane's 16 values are grid magnitudes from the LDS tables with the ksign masks applied, and
 * the sub-block scale d * (2s+1) / 8 (IQ2) or / 4 (IQ3) comes in the epilogue. */
template <int TY>
struct MsIq;
template <>
struct MsIq<LE_TYPE_IQ2_XXS> {
    static constexpr int CPS = 5, SBB = 66;
    static constexpr float SCALE = 0.125f;
    static __device__ __forceinline__ int goff(int c) { return c < 4 ? 2 + 16 * c : 0; }
    /* B words of sub-block j, values 16h..16h+15 */
    static __device__ __forceinline__ le_v4i bfrag(const u8 *sb, int j, int h, const u32 *tab) {
        const uint2 q = *(const uint2 *)(sb + 8 * j);
        const u32 *grid = tab + LE_TAB_GRID, *sg = tab + LE_TAB_SIGN;
        u32 w[4];
#pragma unroll
        for (int l = 0; l < 2; l++) {
            const int g = 2 * h + l;
            const u32 gi = (q.x >> (8 * g)) & 255u, si = (q.y >> (7 * g)) & 127u;
            const uint2 gv = *(const uint2 *)(grid + 2 * gi);
            const uint2 m = *(const uint2 *)(sg + 2 * si);
            w[2 * l] = apply_sign(gv.x, m.x);
            w[2 * l + 1] = apply_sign(gv.y, m.y);
        }
        return (le_v4i){(int)w[0], (int)w[1], (int)w[2], (int)w[3]};
    }
    static __device__ __forceinline__ u32 aux(const u8 *sb, int j) { return *(const u32 *)(sb + 8 * j + 4); }
    static __device__ __forceinline__ float sscale(const u8 *sb, int j) { return (float)(2 * (aux(sb, j) >> 28) + 1); }
    static __device__ __forceinline__ float d(const u8 *sb) { return h2f(*(const u32 *)(sb + 64) & 0xFFFFu); }
};
template <>
struct MsIq<LE_TYPE_IQ3_XXS> {
    static constexpr int CPS = 7, SBB = 98;
    static constexpr float SCALE = 0.25f;
    static __device__ __forceinline__ int goff(int c) { return c < 6 ? 2 + 16 * c : 0; }
    static __device__ __forceinline__ le_v4i bfrag(const u8 *sb, int j, int h, const u32 *tab) {
        const u32 q = *(const u32 *)(sb + 8 * j + 4 * h), ax = *(const u32 *)(sb + 64 + 4 * j);
        const u32 *grid = tab + LE_TAB_GRID, *sg = tab + LE_TAB_SIGN;
        const uint2 m0 = *(const uint2 *)(sg + 2 * ((ax >> (14 * h)) & 127u));
        const uint2 m1 = *(const uint2 *)(sg + 2 * ((ax >> (14 * h + 7)) & 127u));
        return (le_v4i){(int)apply_sign(grid[q & 255u], m0.x), (int)apply_sign(grid[(q >> 8) & 255u], m0.y),
                        (int)apply_sign(grid[(q >> 16) & 255u], m1.x), (int)apply_sign(grid[q >> 24], m1.y)};
    }
    static __device__ __forceinline__ u32 aux(const u8 *sb, int j) { return *(const u32 *)(sb + 64 + 4 * j); }
    static __device__ __forceinline__ float sscale(const u8 *sb, int j) { return (float)(2 * (aux(sb, j) >> 28) + 1); }
    static __device__ __forceinline__ float d(const u8 *sb) { return h2f(*(const u32 *)(sb + 96) & 0xFFFFu); }
};

/* 16 bytes at a 2-byte-aligned LDS address: five aligned words, funnel-shifted */
__device__ __forceinline__ uint4 lds16_a2(const u8 *p) {
    const u32 *w = (const u32 *)(p - ((size_t)p & 3)); /* pointer arithmetic keeps the LDS address space */
    const u32 sh = (u32)((size_t)p & 3) * 8u;
    const u32 w0 = w[0], w1 = w[1], w2 = w[2], w3 = w[3], w4 = w[4];
    return make_uint4(__builtin_amdgcn_alignbit(w1, w0, sh), __builtin_amdgcn_alignbit(w2, w1, sh),
                      __builtin_amdgcn_alignbit(w3, w2, sh), __builtin_amdgcn_alignbit(w4, w3, sh));
}
__device__ __forceinline__ float lds_h2f_a2(const u8 *p) {
    const u32 w = *(const u32 *)(p - ((size_t)p & 3));
    return h2f((w >> (((size_t)p & 2) * 8)) & 0xFFFFu);
}
/* Q8_0 on the same staged design: a "super-block" is 8 consecutive 32-value blocks (272 bytes,
 * 16-byte aligned in a row of K/256 of them, staged as 17 chunks), sub-block j is block j, its
 * codes are the int8 q (src/quant.rs:68-71) and its scale is the block's d in the epilogue. (Q4_0
 * the same way measured slower than its vector kernel: 14.5 against 12.5 us at 14336x4096.) */
template <>
struct MsIq<LE_TYPE_Q8_0> {
    static constexpr int CPS = 17, SBB = 272;
    static constexpr float SCALE = 1.f;
    static __device__ __forceinline__ int goff(int c) { return 16 * c; }
    static __device__ __forceinline__ le_v4i bfrag(const u8 *sb, int j, int h, const u32 *) {
        const uint4 q = lds16_a2(sb + 34 * j + 2 + 16 * h);
        return (le_v4i){(int)q.x, (int)q.y, (int)q.z, (int)q.w};
    }
    static __device__ __forceinline__ float sscale(const u8 *sb, int j) { return lds_h2f_a2(sb + 34 * j); }
    static __device__ __forceinline__ float d(const u8 *) { return 1.f; }
};
/* Q4_0 the same way: eight 18-byte blocks (144 bytes, 9 chunks), codes the nibbles minus 8
 * (src/quant.rs:64-67: value i < 16 the low nibble of byte i, 16 + i the high one) */
template <>
struct MsIq<LE_TYPE_Q4_0> {
    static constexpr int CPS = 9, SBB = 144;
    static constexpr float SCALE = 1.f;
    static __device__ __forceinline__ int goff(int c) { return 16 * c; }
    static __device__ __forceinline__ le_v4i bfrag(const u8 *sb, int j, int h, const u32 *) {
        const uint4 q = lds16_a2(sb + 18 * j + 2);
        const u32 w[4] = {q.x, q.y, q.z, q.w};
        int o[4];
#pragma unroll
        for (int i = 0; i < 4; i++) /* nibble - 8 bytewise: (n + 0x78) ^ 0x80, no carries */
            o[i] = (int)((((h ? w[i] >> 4 : w[i]) & 0x0F0F0F0Fu) + 0x78787878u) ^ 0x80808080u);
        return (le_v4i){o[0], o[1], o[2], o[3]};
    }
    static __device__ __forceinline__ float sscale(const u8 *sb, int j) { return lds_h2f_a2(sb + 18 * j); }
    static __device__ __forceinline__ float d(const u8 *) { return 1.f; }
};

template <int TY>
__device__ __forceinline__ float ms_sb_iq(const u8 *sb, const le_v4i (&A)[4], const float *dxp_sb, const MsLane &L, const u32 *tab) {
    using F = MsIq<TY>;
    const int sq = L.sq;
    le_v4i D = {0, 0, 0, 0};
#pragma unroll
    for (int b = 0; b < 4; b++) D = __builtin_amdgcn_mfma_i32_16x16x64_i8(A[b], F::bfrag(sb, mq_j(b, sq), sq & 1, tab), D, 0, 0, 0);
    const float4 dq = *(const float4 *)(dxp_sb + L.pe * 8 + L.jb);
    const float dqa[4] = {dq.x, dq.y, dq.z, dq.w};
    float t = 0.f;
#pragma unroll
    for (int i = 0; i < 4; i++) t += F::sscale(sb, L.jb + i) * dqa[i] * (float)D[i];
    return F::d(sb) * F::SCALE * t;
}

template <int TY, int P, int NW, bool Q8>
__device__ __forceinline__ void ms_iq_body(const MvArgs &a) {
    using F = MsIq<TY>;
    extern __shared__ uint4 smem[];
    constexpr int CPS = F::CPS, CPR = CPS * P + 1, NCH = 16 * CPR, NI = (NCH + 63) / 64;
    __shared__ u32 tab[256 + 512];
    load_tables<TY>(tab);
    const int K = a.cols, nsb = K >> 8;
    const int slot = blockIdx.y;
    const u8 *W = a.ptrs ? a.ptrs[slot] : a.w0 + (size_t)slot * a.w_slot_bytes;
    const size_t rb = (size_t)nsb * F::SBB;
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const int n = lane & 15;
    const int nsbw = nsb / NW;
    uint4 *rec = smem + wave * (nsbw * 38 + NI * 64);
    float *dxp = (float *)(rec + nsbw * 32);
    float *fsv = dxp + nsbw * 16;
    uint4 *wb = (uint4 *)(fsv + nsbw * 8);
    float *red = (float *)(smem + NW * (nsbw * 38 + NI * 64)); /* [2][NW][16] */
    const int ntile = (a.rows + 15) >> 4;
    int ri[NI], gb[NI];
#pragma unroll
    for (int i = 0; i < NI; i++) {
        const int c = min(64 * i + lane, NCH - 1);
        const int col = c % CPR, cc = col == CPS * P ? 0 : col;
        ri[i] = c / CPR;
        gb[i] = (cc / CPS) * F::SBB + F::goff(cc % CPS);
    }
    uint4 R[NI];
    auto issue = [&](int tile, int s0) {
#pragma unroll
        for (int i = 0; i < NI; i++) {
            const int row = min(tile * 16 + ri[i], a.rows - 1);
            R[i] = ldg16u(W + (size_t)row * rb + (size_t)s0 * F::SBB + gb[i]);
        }
    };
    const int sfirst = wave * P, sstep = NW * P;
    const bool active = sfirst < nsb;
    const float *xs = a.x + a.x_slot * slot;
    const int nsegw = nsbw * 16;
    auto gseg = [&](int el) {
        const int ls = el >> 4;
        return ((ls / P) * sstep + sfirst + ls % P) * 16 + (el & 15);
    };
    if constexpr (Q8) { /* int8 mode (the _q8 kernels): the image holds the caller's xq, scale xd per 32 values (exact) */
        issue(min((int)blockIdx.x, ntile - 1), active ? sfirst : 0);
        const int8_t *xq8 = a.xq8 + a.x_slot * slot;
        const float *xd8 = a.xd8 + (a.x_slot >> 5) * slot;
        for (int el0 = 0; el0 < nsegw; el0 += 64) {
            const int el = el0 + lane, ge = gseg(min(el, nsegw - 1));
            mq_quant_seg_q8<0>(el, el < nsegw, ldg16u((const u8 *)(xq8 + 16 * ge)), xd8[ge >> 1], rec, dxp, fsv);
        }
    } else {
    float4 xv[4];
    mq_load_seg_a(xs, gseg(min(lane, nsegw - 1)), a.cols, a.swiglu, xv);
    issue(min((int)blockIdx.x, ntile - 1), active ? sfirst : 0);
    mq_quant_seg<0>(lane, lane < nsegw, xv, rec, dxp, fsv);
    for (int el = lane + 64; el < nsegw; el += 64) {
        mq_load_seg_a(xs, gseg(el), a.cols, a.swiglu, xv);
        mq_quant_seg<0>(el, true, xv, rec, dxp, fsv);
    }
    }
    __syncthreads(); /* the tables */
    const MsLane L = ms_lane<0>(lane);
    le_v4i A[4];
#pragma unroll
    for (int b = 0; b < 4; b++) A[b] = (le_v4i){0, 0, 0, 0};
    int par = 0;
    for (int tile = blockIdx.x; tile < ntile; tile += gridDim.x) {
        float y = 0.f;
        if (active) {
            for (int s0 = sfirst, lb = 0; s0 < nsb; s0 += sstep, lb += P) {
                int nt = tile, ns = s0 + sstep;
                if (ns >= nsb) { ns = sfirst; nt += gridDim.x; }
#pragma unroll
                for (int i = 0; i < NI; i++) wb[64 * i + lane] = R[i];
                if (nt < ntile) issue(nt, ns);
#pragma unroll
                for (int q = 0; q < P; q++) {
                    const int sb = lb + q;
                    ms_load_a(rec + sb * 32, L, A);
                    y += ms_sb_iq<TY>((const u8 *)(wb + n * CPR + CPS * q), A, dxp + sb * 16, L, tab);
                }
            }
        }
        y = row4_sum(y);
        float *rp = red + par * (NW * 16);
        if (lane < 16) rp[wave * 16 + lane] = y;
        __builtin_amdgcn_s_waitcnt(0xC07F);
        __builtin_amdgcn_s_barrier();
        if (wave == 0 && lane < 16) {
            float acc = 0.f;
#pragma unroll
            for (int w = 0; w < NW; w++) acc += rp[w * 16 + lane];
            const int r = tile * 16 + lane;
            if (r < a.rows) a.y[a.y_slot * slot + r] = acc;
        }
        par ^= 1;
    }
}

#define LE_MSIQ_(TY, P, NW)                                                                                \
    extern "C" __global__ void __launch_bounds__(NW * 64) le_ms_##TY##_p##P##_w##NW(MvArgs a) { ms_iq_body<TY, P, NW, false>(a); } \
    extern "C" __global__ void __launch_bounds__(NW * 64) le_ms_##TY##_p##P##_w##NW##_q8(MvArgs a) { ms_iq_body<TY, P, NW, true>(a); }
#define LE_MSIQ(TY, P, NW) LE_MSIQ_(TY, P, NW) /* expands TY before pasting */

#define LE_MS12(P, NW)                                                                                     \
    extern "C" __global__ void __launch_bounds__(NW * 64) le_ms_12_p##P##_w##NW(MvArgs a) { ms_q4k_body<P, NW, false>(a); } \
    extern "C" __global__ void __launch_bounds__(NW * 64) le_ms_12_p##P##_w##NW##_q8(MvArgs a) { ms_q4k_body<P, NW, true>(a); }

#define LE_MS12T(P, NW, T)                                                                                 \
    extern "C" __global__ void __launch_bounds__(NW * 64) le_ms_12_p##P##_w##NW##_t##T(MvArgs a) { ms_q4k_t_body<P, NW, T>(a); }

#define LE_MQ12(NW, U)                                                                                     \
    extern "C" __global__ void __launch_bounds__(NW * 64) le_mq_12_w##NW##_u##U(MvArgs a) { mq_q4k_body<NW, U>(a); }

/* Each code object carries the kernels of one part (the build compiles this file once per part,
 * in parallel): LE_PART_DEQ, or LE_PART_MV=<type id>. */
#if defined(LE_PART_MV)
LE_MV_ALL(LE_PART_MV)
#if LE_PART_MV == 12
LE_MQ12(4, 1) LE_MQ12(4, 2) LE_MQ12(4, 4) LE_MQ12(8, 1) LE_MQ12(8, 2) LE_MQ12(8, 4) LE_MQ12(2, 1) LE_MQ12(2, 2) LE_MQ12(2, 4)
LE_MS12(2, 12) LE_MS12(2, 14) LE_MS12(2, 16) LE_MS12(1, 1) LE_MS12(1, 2) LE_MS12(1, 4) LE_MS12(1, 8) LE_MS12(2, 1) LE_MS12(2, 2) LE_MS12(2, 4) LE_MS12(2, 8) LE_MS12(4, 1) LE_MS12(4, 2) LE_MS12(4, 4)
LE_MS12T(1, 4, 2) LE_MS12T(1, 4, 4) LE_MS12T(1, 4, 8) LE_MS12T(1, 8, 2) LE_MS12T(1, 8, 4) LE_MS12T(1, 8, 8)
LE_MS12T(2, 4, 2) LE_MS12T(2, 4, 4) LE_MS12T(2, 4, 8) LE_MS12T(2, 2, 2) LE_MS12T(2, 2, 4) LE_MS12T(2, 2, 8)
#endif
#if LE_PART_MV == 13
#define LE_MS13(P, NW)                                                                                     \
    extern "C" __global__ void __launch_bounds__(NW * 64) le_ms_13_p##P##_w##NW(MvArgs a) { ms_q4k_body<P, NW, false, LE_TYPE_Q5_K>(a); } \
    extern "C" __global__ void __launch_bounds__(NW * 64) le_ms_13_p##P##_w##NW##_q8(MvArgs a) { ms_q4k_body<P, NW, true, LE_TYPE_Q5_K>(a); }
LE_MS13(2, 12) LE_MS13(2, 14) LE_MS13(2, 16) LE_MS13(1, 1) LE_MS13(1, 2) LE_MS13(1, 4) LE_MS13(1, 8) LE_MS13(2, 1) LE_MS13(2, 2) LE_MS13(2, 4) LE_MS13(2, 8) LE_MS13(4, 1) LE_MS13(4, 2) LE_MS13(4, 4)
#endif
#if LE_PART_MV == 11
#define LE_MS11(P, NW)                                                                                     \
    extern "C" __global__ void __launch_bounds__(NW * 64) le_ms_11_p##P##_w##NW(MvArgs a) { ms_q6k_body<P, NW, false, LE_TYPE_Q3_K>(a); } \
    extern "C" __global__ void __launch_bounds__(NW * 64) le_ms_11_p##P##_w##NW##_q8(MvArgs a) { ms_q6k_body<P, NW, true, LE_TYPE_Q3_K>(a); }
LE_MS11(2, 12) LE_MS11(2, 14) LE_MS11(2, 16) LE_MS11(1, 1) LE_MS11(1, 2) LE_MS11(1, 4) LE_MS11(1, 8) LE_MS11(2, 1) LE_MS11(2, 2) LE_MS11(2, 4) LE_MS11(2, 8) LE_MS11(4, 1) LE_MS11(4, 2) LE_MS11(4, 4)
#endif
#if LE_PART_MV == 22
#define LE_MS22(P, NW)                                                                                     \
    extern "C" __global__ void __launch_bounds__(NW * 64) le_ms_22_p##P##_w##NW(MvArgs a) { ms_q6k_body<P, NW, false, LE_TYPE_IQ2_S>(a); } \
    extern "C" __global__ void __launch_bounds__(NW * 64) le_ms_22_p##P##_w##NW##_q8(MvArgs a) { ms_q6k_body<P, NW, true, LE_TYPE_IQ2_S>(a); }
LE_MS22(2, 12) LE_MS22(2, 14) LE_MS22(2, 16) LE_MS22(1, 1) LE_MS22(1, 2) LE_MS22(1, 4) LE_MS22(1, 8) LE_MS22(2, 1) LE_MS22(2, 2) LE_MS22(2, 4) LE_MS22(2, 8) LE_MS22(4, 1) LE_MS22(4, 2) LE_MS22(4, 4)
#endif
#if LE_PART_MV == 14
LE_MS14(1, 1) LE_MS14(1, 2) LE_MS14(1, 4) LE_MS14(1, 8) LE_MS14(2, 1) LE_MS14(2, 2) LE_MS14(2, 4) LE_MS14(2, 8) LE_MS14(4, 1) LE_MS14(4, 2)
#endif
#if LE_PART_MV == 16 || LE_PART_MV == 18 || LE_PART_MV == 8 || LE_PART_MV == 2
LE_MSIQ(LE_PART_MV, 1, 1) LE_MSIQ(LE_PART_MV, 1, 2) LE_MSIQ(LE_PART_MV, 1, 4) LE_MSIQ(LE_PART_MV, 2, 1) LE_MSIQ(LE_PART_MV, 2, 2)
LE_MSIQ(LE_PART_MV, 2, 4) LE_MSIQ(LE_PART_MV, 4, 1) LE_MSIQ(LE_PART_MV, 4, 2) LE_MSIQ(LE_PART_MV, 4, 4)
LE_MSIQ(LE_PART_MV, 1, 8) LE_MSIQ(LE_PART_MV, 2, 8)
#if LE_PART_MV == 18 || LE_PART_MV == 16 || LE_PART_MV == 2 /* down-projection shapes: one row tile per block, K split over 12-16 waves */
LE_MSIQ(LE_PART_MV, 2, 12) LE_MSIQ(LE_PART_MV, 2, 14) LE_MSIQ(LE_PART_MV, 2, 16)
#endif
#endif
#endif

/* ===================================================================================== */
/* MoE expert layer: routing, grouped gate/up + SwiGLU, grouped down + weighted combine.    */
/* ===================================================================================== */
#if defined(LE_PART_MOE)
/* Semantics of the routed part of cpu_ref::moe (src/cpu_ref.rs:242-259) for n_tok tokens:
 * softmax over the router logits, top-k (ties keep the lower expert first), weights renormalised
 * over the selected k, out = sum_s w_s * down_e(silu(gate_e h) * up_e h).
 *
 * Two launches instead of the reference's per-layer chain of router_topk, host read-back of the
 * indices (src/gpu.rs:579), build_ptrs, fused gate+up matvec, swiglu, quant_x, down matvec and
 * moe_combine (src/gpu.rs:560-597). Every block recomputes the routing from the logits (a few
 * hundred values), so nothing crosses to the host. (token, expert) pairs are grouped by expert:
 * group z is the z-th selected expert in ascending id order, its members the tokens that chose it
 * in ascending order, so each expert's weights are read once per launch whatever the batch.
 *   le_moe_gu_*:   grid (ff/32, groups). Gate and up rows of one 32-row unit for all members,
 *                  SwiGLU, and the down projection's activation image of that unit written to the
 *                  workspace already quantized (pair p = token*k + slot).
 *   le_moe_down_*: grid (hidden/8). The block's 8 output rows for every group; waves take groups
 *                  round-robin and the four partial sums are added in a fixed order. */
struct MoeArgs {
    const u8 *gate, *up, *down;
    const float *logits, *h;
    float *out;
    u8 *ws; /* the caller's workspace after its barrier area (images, then the routing record) */
    int *idx_out;
    float *w_out;
    int n_tok, n_exp, k, hidden, ff;
    unsigned int spin_limit;  /* bounded waits of the one-launch barrier; 0 makes it fail */
    u8 *bar;                  /* the caller's workspace start: barrier area (LE_MOE_BAR_BYTES) */
    /* per-expert weight pointers (an expert-cache arena), or null: expert e's slab at
     * e * rows * row_bytes of gate / up / down */
    const u8 *const *gptr, *const *uptr, *const *dptr;
};
/* Expert e's weights: its pointer-table entry, or its slab in the 3D tensor. */
/* Expert e's weights: slab e of a 3D tensor, or entry e of a device pointer table. e is uniform
 * over the wave at every call site, so the table entry is read with a scalar load: a vector load
 * there made the compiler wait for every vector load in flight (activations, images) before the
 * weight loads could be issued, on the slab path as well. */
__device__ __forceinline__ const u8 *moe_w(const u8 *slab, const u8 *const *ptrs, int e, size_t expert_bytes) {
    if (!ptrs) return slab + (size_t)e * expert_bytes;
    typedef const u8 *wptr;
    return ((const __attribute__((address_space(4))) wptr *)ptrs)[__builtin_amdgcn_readfirstlane(e)];
}
/* Barrier area at the start of the workspace: a status word (sticky, nonzero after a wait gave
 * up; read and cleared by le_moe_check), the generation word, then one arrival flag per block. */
#define LE_MOE_BAR_STATUS 0
#define LE_MOE_BAR_FAILED 0x5EAD0001u /* status word value after a give-up (any other value: none) */
#define LE_MOE_BAR_GEN 64
#define LE_MOE_BAR_FLAGS 128
#define LE_MOE_MAXTOK 64
#define LE_MOE_MAXK 16
#define LE_MOE_MAXEXP 256

/* Block barrier for data exchanged through LDS only: waits for this wave's LDS (and scalar)
 * operations, not for its global loads in flight (__syncthreads waits for those too). */
__device__ __forceinline__ void moe_sync() {
    __asm__ volatile("" ::: "memory");
    __builtin_amdgcn_s_waitcnt(0xC07F);
    __builtin_amdgcn_s_barrier();
    __asm__ volatile("" ::: "memory");
}

/* LDS routing state shared by both kernels. */
struct MoeRoute {
    int topi[LE_MOE_MAXTOK * LE_MOE_MAXK];
    float topw[LE_MOE_MAXTOK * LE_MOE_MAXK];
    unsigned long long mask[LE_MOE_MAXEXP];
    int grp_e[LE_MOE_MAXEXP];
    int U;
#ifdef LE_MOE_TRACE
    unsigned long long tr[8];
#endif
};
#ifdef LE_MOE_TRACE
#define MOE_RT(i) if (threadIdx.x == 0) R.tr[i] = __builtin_amdgcn_s_memrealtime()
#else
#define MOE_RT(i)
#endif

/* Wave-wide max / sum: DPP within 16-lane rows, then the four row results through readlane, so the
 * result is uniform (no LDS-routed shuffles on the routing critical path). */
__device__ __forceinline__ float wave_max(float v) {
    v = fmaxf(v, dpp_f<0xB1>(v));
    v = fmaxf(v, dpp_f<0x4E>(v));
    v = fmaxf(v, dpp_f<0x141>(v));
    v = fmaxf(v, dpp_f<0x140>(v));
    const int b = __builtin_bit_cast(int, v);
    return fmaxf(fmaxf(__builtin_bit_cast(float, __builtin_amdgcn_readlane(b, 0)), __builtin_bit_cast(float, __builtin_amdgcn_readlane(b, 16))),
                 fmaxf(__builtin_bit_cast(float, __builtin_amdgcn_readlane(b, 32)), __builtin_bit_cast(float, __builtin_amdgcn_readlane(b, 48))));
}
__device__ __forceinline__ float wave_sum(float v) {
    v += dpp_f<0xB1>(v);
    v += dpp_f<0x4E>(v);
    v += dpp_f<0x141>(v);
    v += dpp_f<0x140>(v);
    const int b = __builtin_bit_cast(int, v);
    return (__builtin_bit_cast(float, __builtin_amdgcn_readlane(b, 0)) + __builtin_bit_cast(float, __builtin_amdgcn_readlane(b, 16))) +
           (__builtin_bit_cast(float, __builtin_amdgcn_readlane(b, 32)) + __builtin_bit_cast(float, __builtin_amdgcn_readlane(b, 48)));
}

/* Order-preserving 32-bit key of a float (-0 as +0, so the two tie as the float compare has
 * them). */
__device__ __forceinline__ u32 f2key(float v) {
    const u32 b = __builtin_bit_cast(u32, v == 0.f ? 0.f : v);
    return (b & 0x80000000u) ? ~b : (b | 0x80000000u);
}
/* One token, at most 128 experts, blocks of 8 waves: wave w compares experts 16 w .. 16 w + 15 */
__device__ __forceinline__ bool moe_route_is_one(const MoeArgs &a) {
    return a.n_tok == 1 && a.n_exp <= 128 && a.k <= 64 && blockDim.x == 512;
}
/* One token, at most 128 experts, every wave of the block: the rank of expert e (the number of
 * experts before it in the stable descending sort of src/cpu_ref.rs:248) is counted directly.
 * Wave w takes the logits of experts 16w .. 16w + 15 as scalars and compares each with the two
 * experts of every lane (e = lane, lane + 64) through 64-bit keys (order-preserving logit bits
 * above the inverted index, so "larger, or equal and lower index" is one compare); the waves'
 * counts are added in LDS (rk[128], zero on entry). Then wave 0: rank < k selects, the selection is
 * written in rank order, the weights are ex / sum(ex) with ex = exp(logit - top logit) summed in
 * rank order (as the other paths), and the groups are the selected experts in ascending order
 * (prefix counts of the two selection ballots). R.mask must be zero for every expert. */
__device__ __forceinline__ unsigned long long moe_key2(float v, int e) {
    return ((unsigned long long)f2key(v) << 32) | (u32)(0xFFFFFFFFu - (u32)e);
}
__device__ __forceinline__ void moe_route_one(const MoeArgs &a, MoeRoute &R, float *sx, int *rk, float lv0, float lv1,
                                              const float (&lj)[16]) {
    const int lane = threadIdx.x & 63, w = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int e0 = lane, e1 = lane + 64;
    const unsigned long long my0 = moe_key2(lv0, e0), my1 = moe_key2(lv1, e1);
    const int j0 = 16 * w;
    if (j0 < a.n_exp) {
        int c0 = 0, c1 = 0;
#pragma unroll
        for (int i = 0; i < 16; i++) {
            /* an expert past n_exp gets key 0, below every real key: it is never counted */
            const unsigned long long kj = j0 + i < a.n_exp ? moe_key2(lj[i], j0 + i) : 0ull;
            c0 += kj > my0;
            c1 += kj > my1;
        }
        if (e0 < a.n_exp) atomicAdd(&rk[e0], c0);
        if (e1 < a.n_exp) atomicAdd(&rk[e1], c1);
    }
    moe_sync();
    if (threadIdx.x < 64) {
        const int r0 = e0 < a.n_exp ? rk[e0] : 0x7FFFFFFF, r1 = e1 < a.n_exp ? rk[e1] : 0x7FFFFFFF;
        const bool s0 = r0 < a.k, s1 = r1 < a.k;
        if (s0) { R.topi[r0] = e0; sx[r0] = lv0; R.mask[e0] = 1ull; }
        if (s1) { R.topi[r1] = e1; sx[r1] = lv1; R.mask[e1] = 1ull; }
        const unsigned long long b0 = __ballot(s0), b1 = __ballot(s1);
        const unsigned long long below = (1ull << lane) - 1ull;
        if (s0) R.grp_e[__popcll(b0 & below)] = e0;
        if (s1) R.grp_e[__popcll(b0) + __popcll(b1 & below)] = e1;
        __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
        __builtin_amdgcn_wave_barrier();
        __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
        const bool sel = lane < a.k;
        const float v = sel ? sx[lane] : 0.f, top = sx[0];
        const float ex = sel ? expf(v - top) : 0.f;
        float tot = 0.f;
        for (int r = 0; r < a.k; r++) tot += __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, ex), r));
        if (sel) R.topw[lane] = ex / tot;
        if (lane == 0) R.U = a.k;
    }
}

/* All threads: route every token (one wave per token), then list the groups. Lane l holds
 * experts l*per .. l*per+per-1 (per <= 4), so among lanes tied on the best logit the lowest lane
 * holds the lowest expert index: the ballot's first set bit is the winner (the stable descending
 * sort of src/cpu_ref.rs:248 keeps the lower index first). */
__device__ void moe_route(const MoeArgs &a, MoeRoute &R) {
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6, nwave = blockDim.x >> 6;
    const int per = (a.n_exp + 63) >> 6;
    for (int t = wave; t < a.n_tok; t += nwave) {
        const float *lg = a.logits + (size_t)t * a.n_exp;
        float v[4];
        bool taken[4];
#pragma unroll
        for (int j = 0; j < 4; j++) {
            const int e = lane * per + j;
            const bool ok = j < per && e < a.n_exp;
            v[j] = ok ? lg[e] : -INFINITY;
            taken[j] = !ok;
        }
        const float m = wave_max(fmaxf(fmaxf(v[0], v[1]), fmaxf(v[2], v[3])));
        float ls = 0.f;
#pragma unroll
        for (int j = 0; j < 4; j++) ls += taken[j] ? 0.f : expf(v[j] - m);
        const float s = wave_sum(ls);
        float tot = 0.f;
        for (int r = 0; r < a.k; r++) {
            float bv = -INFINITY;
            int bj = -1;
#pragma unroll
            for (int j = 0; j < 4; j++)
                if (!taken[j] && (bj < 0 || v[j] > bv)) { bv = v[j]; bj = j; }
            const float mx = wave_max(bj >= 0 ? bv : -INFINITY);
            const unsigned long long cand = __ballot(bj >= 0 && bv == mx);
            const int wl = __ffsll((long long)cand) - 1;
            const int wj = __builtin_amdgcn_readlane(bj, wl);
            if (lane == wl) {
#pragma unroll
                for (int j = 0; j < 4; j++)
                    if (j == wj) taken[j] = true;
            }
            const float pr = expf(mx - m) / s;
            tot += pr;
            if (lane == 0) {
                R.topi[t * a.k + r] = wl * per + wj;
                R.topw[t * a.k + r] = pr;
            }
        }
        if (lane == 0)
            for (int r = 0; r < a.k; r++) R.topw[t * a.k + r] /= tot;
    }
    moe_sync();
    /* expert masks from the top-k table (no atomics, no zeroing pass) */
    const int nsel = a.n_tok * a.k;
    for (int e = threadIdx.x; e < a.n_exp; e += blockDim.x) {
        unsigned long long msk = 0ull;
        for (int i = 0; i < nsel; i++)
            if (R.topi[i] == e) msk |= 1ull << (i / a.k);
        R.mask[e] = msk;
    }
    moe_sync();
    if (wave == 0) {
        int base = 0;
        for (int c = 0; c < a.n_exp; c += 64) {
            const int e = c + lane;
            const bool nz = e < a.n_exp && R.mask[e] != 0ull;
            const unsigned long long bal = __ballot(nz);
            if (nz) R.grp_e[base + __popcll(bal & ((1ull << lane) - 1ull))] = e;
            base += __popcll(bal);
        }
        if (lane == 0) R.U = base;
    }
    moe_sync();
}

/* Parallel routing for the decode-shaped kernels (n_exp <= 256): one thread per (token, expert).
 * Each logit becomes a 64-bit key, the float's order-preserving bits above the inverted expert
 * index, so "larger logit, or equal logit and lower index" is one unsigned compare. An expert's
 * rank (the number of larger keys) is its position in the stable descending sort of
 * src/cpu_ref.rs:248; rank < k selects it. With ex = exp(logit - top logit), the renormalised
 * weight pr/sum(pr over the k) equals ex/sum(ex over the k) (the softmax denominator cancels); the
 * k-sum runs in selection order. */
__device__ __forceinline__ unsigned long long moe_key(float v, int e) {
    u32 b = __float_as_uint(v == 0.f ? 0.f : v); /* -0 ties with +0, as the float compare does */
    b = (b & 0x80000000u) ? ~b : (b | 0x80000000u);
    return ((unsigned long long)b << 32) | (u32)(0xFFFFFFFFu - (u32)e);
}

/* Lane geometry of moe_route_par: C lanes share one (token, expert); lane c of the group compares
 * against key pairs c, c + C, ... (adjacent lanes read adjacent 16 bytes); C shrinks as tokens
 * grow so that one pass covers as many tokens as the block has threads for. */
struct MoeRouteGeom {
    int tpt, C, tpp, npass;
};
__device__ __forceinline__ MoeRouteGeom moe_route_geom(const MoeArgs &a) {
    MoeRouteGeom g;
    g.tpt = a.n_exp <= 128 ? 128 : 256;
    g.C = 8;
    while (g.C > 1 && g.C * g.tpt * a.n_tok > (int)blockDim.x) g.C >>= 1;
    g.tpp = blockDim.x / (g.tpt * g.C); /* tokens per pass */
    g.npass = (a.n_tok + g.tpp - 1) / g.tpp;
    return g;
}
/* This thread's logits of the first MOE_LPASS passes, loaded before anything else the kernel
 * loads (loads complete in order, so routing then waits for these alone). */
#define MOE_LPASS 4
struct MoeLogits {
    float v[MOE_LPASS];
    float j[16]; /* single-token ranking: this wave's 16 compared logits (scalar loads) */
};
/* 2..(waves) tokens, at most 256 experts: one wave selects each token's top-k (k rounds of a
 * wave-wide max; lane l holds experts l*per .. l*per+per-1) instead of ranking every key. One
 * token keeps the ranking, spread over eight lanes per expert (measured faster there). */
__device__ __forceinline__ bool moe_route_by_wave(const MoeArgs &a) {
    return a.n_tok >= 1 && a.n_tok <= (int)(blockDim.x >> 6) && a.n_exp <= 256;
}
__device__ __forceinline__ MoeLogits moe_route_load(const MoeArgs &a) {
    MoeLogits L;
    if (moe_route_is_one(a)) { /* every lane: experts lane and lane + 64 */
        const int lane = threadIdx.x & 63;
        L.v[0] = a.logits[min(lane, a.n_exp - 1)];
        L.v[1] = a.logits[min(lane + 64, a.n_exp - 1)];
        L.v[2] = L.v[3] = 0.f;
        const int j0 = 16 * __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
#pragma unroll
        for (int i = 0; i < 16; i++) /* wave-uniform, read-only for the kernel: scalar loads */
            L.j[i] = ((const __attribute__((address_space(4))) float *)a.logits)[min(j0 + i, a.n_exp - 1)];
        return L;
    }
    if (moe_route_by_wave(a)) {
        const int lane = threadIdx.x & 63, t = threadIdx.x >> 6, per = (a.n_exp + 63) >> 6;
#pragma unroll
        for (int j = 0; j < MOE_LPASS; j++) {
            const int e = lane * per + j;
            L.v[j] = t < a.n_tok && j < per && e < a.n_exp ? a.logits[(size_t)t * a.n_exp + e] : 0.f;
        }
        return L;
    }
    const MoeRouteGeom g = moe_route_geom(a);
    const int t1 = threadIdx.x / (g.tpt * g.C), e = (threadIdx.x / g.C) % g.tpt;
#pragma unroll
    for (int p = 0; p < MOE_LPASS; p++) {
        const int t = p * g.tpp + t1;
        L.v[p] = t < a.n_tok && e < a.n_exp ? a.logits[(size_t)t * a.n_exp + e] : 0.f;
    }
    return L;
}

__device__ __forceinline__ void moe_route_par(const MoeArgs &a, MoeRoute &R, unsigned long long *lv /* [n_tok][n_exp] LDS */,
                                              float *sx /* [n_tok][k] */, const MoeLogits &L) {
    const MoeRouteGeom g = moe_route_geom(a);
    const int tpt = g.tpt, C = g.C, tpp = g.tpp;
    /* n_tok <= 64 on every caller, so a token's bit fits the 64-bit expert mask; the first
     * barrier orders this clear before the atomics below */
    for (int e = threadIdx.x; e < a.n_exp; e += blockDim.x) R.mask[e] = 0ull;
    const int c = threadIdx.x % C;
    auto rank_of = [&](int t, int e, float v, unsigned long long key) {
        int rank = 0;
        if (t < a.n_tok && e < a.n_exp) {
            const ulonglong2 *row = (const ulonglong2 *)(lv + t * a.n_exp);
            const int npair = a.n_exp >> 1;
            /* eight reads issued before any compare, so LDS latency is paid once per batch */
            for (int j0 = c; j0 < npair; j0 += 8 * C) {
                ulonglong2 u[8];
#pragma unroll
                for (int q = 0; q < 8; q++) u[q] = row[min(j0 + q * C, npair - 1)];
#pragma unroll
                for (int q = 0; q < 8; q++)
                    if (j0 + q * C < npair) rank += (int)(u[q].x > key) + (int)(u[q].y > key);
            }
        }
        for (int o = 1; o < C; o <<= 1) rank += __shfl_xor(rank, o); /* groups are lane-aligned */
        if (t < a.n_tok && e < a.n_exp && c == 0 && rank < a.k) {
            R.topi[t * a.k + rank] = e;
            sx[t * a.k + rank] = v;
            atomicOr(&R.mask[e], 1ull << t);
        }
    };
    const int t1 = threadIdx.x / (tpt * C), e1 = (threadIdx.x / C) % tpt;
    if (moe_route_is_one(a)) {
        int *rk = (int *)lv;
        for (int e = threadIdx.x; e < 128; e += blockDim.x) rk[e] = 0;
        moe_sync(); /* the mask and count clears above, before the counts and the selection */
        MOE_RT(1);
        moe_route_one(a, R, sx, rk, L.v[0], L.v[1], L.j);
        MOE_RT(2);
        moe_sync();
        return;
    }
    if (moe_route_by_wave(a)) {
        moe_sync(); /* the mask clear above, before the atomics */
        MOE_RT(1);
        const int lane = threadIdx.x & 63, t = threadIdx.x >> 6, per = (a.n_exp + 63) >> 6;
        if (t < a.n_tok) {
            /* k rounds of a wave-wide max with no branch: round r's winner (the lowest lane among
             * equal values, whose lowest untaken index is the lowest expert: expert = lane * per
             * + j) ends up in lane r's registers, and all k are written to LDS at the end */
            float vv[MOE_LPASS];
#pragma unroll
            for (int j = 0; j < MOE_LPASS; j++) vv[j] = j < per && lane * per + j < a.n_exp ? L.v[j] : -INFINITY;
            int my_e = 0;
            float my_v = 0.f;
            for (int r = 0; r < a.k; r++) {
                float bv = vv[0];
                int bj = 0;
#pragma unroll
                for (int j = 1; j < MOE_LPASS; j++) {
                    const bool gt = vv[j] > bv; /* strict: the lower index of equal values stays */
                    bv = gt ? vv[j] : bv;
                    bj = gt ? j : bj;
                }
                const float mx = wave_max(bv);
                const int wl = __ffsll((long long)__ballot(bv == mx)) - 1;
                const int wj = __builtin_amdgcn_readlane(bj, wl);
#pragma unroll
                for (int j = 0; j < MOE_LPASS; j++) vv[j] = lane == wl && j == wj ? -INFINITY : vv[j];
                my_e = lane == r ? wl * per + wj : my_e;
                my_v = lane == r ? mx : my_v;
            }
            if (lane < a.k) {
                R.topi[t * a.k + lane] = my_e;
                sx[t * a.k + lane] = my_v;
                atomicOr(&R.mask[my_e], 1ull << t);
            }
        }
        MOE_RT(2);
        if (a.n_tok == 1) {
            /* one token: wave 0 holds the k selections; it writes the renormalised weights and
             * the groups (the k experts in ascending order) itself, with no further LDS pass */
            if (threadIdx.x < 64) {
                __builtin_amdgcn_wave_barrier();
                __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
                __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
                const bool sel = lane < a.k;
                const float v = sel ? sx[lane] : -INFINITY, top = sx[0];
                const int e = sel ? R.topi[lane] : 0x7FFFFFFF;
                /* sum of the k exponentials in selection order (as the general path adds them) */
                const float ex = sel ? expf(v - top) : 0.f;
                float tot = 0.f;
                for (int r = 0; r < a.k; r++) tot += __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, ex), r));
                int rank = 0;
                for (int r = 0; r < a.k; r++) rank += __builtin_amdgcn_readlane(e, r) < e;
                if (sel) {
                    R.topw[lane] = ex / tot;
                    R.grp_e[rank] = e;
                }
                if (lane == 0) R.U = a.k;
            }
                moe_sync();
            return;
        }
        moe_sync();
    } else if (g.npass <= MOE_LPASS) {
        /* every pass's keys in LDS, one barrier, every pass ranked, one barrier */
#pragma unroll
        for (int p = 0; p < MOE_LPASS; p++) {
            const int t = p * tpp + t1;
            if (p < g.npass && t < a.n_tok && e1 < a.n_exp && c == 0) lv[t * a.n_exp + e1] = moe_key(L.v[p], e1);
        }
        moe_sync();
#pragma unroll
        for (int p = 0; p < MOE_LPASS; p++) {
            if (p >= g.npass) break;
            const int t = p * tpp + t1;
            rank_of(t, e1, L.v[p], moe_key(L.v[p], e1));
        }
        MOE_RT(1);
        moe_sync();
        MOE_RT(2);
    } else {
        for (int t0 = 0; t0 < a.n_tok; t0 += tpp) {
            const int t = t0 + t1;
            const bool ok = t < a.n_tok && e1 < a.n_exp;
            const float v = ok ? a.logits[(size_t)t * a.n_exp + e1] : 0.f;
            const unsigned long long key = moe_key(v, e1);
            if (ok && c == 0) lv[t * a.n_exp + e1] = key;
            moe_sync();
            rank_of(t, e1, v, key);
            moe_sync();
        }
    }
    const int lane = threadIdx.x & 63, nsel = a.n_tok * a.k;
    if (threadIdx.x < 64) {
        /* wave 0: list the experts with members in ascending order */
        int base = 0;
        for (int c = 0; c < a.n_exp; c += 64) {
            const int e = c + lane;
            const bool nz = e < a.n_exp && R.mask[e] != 0ull;
            const unsigned long long bal = __ballot(nz);
            if (nz) R.grp_e[base + __popcll(bal & ((1ull << lane) - 1ull))] = e;
            base += __popcll(bal);
        }
        if (lane == 0) R.U = base;
    } else {
        /* the other waves: renormalised weights, summed in selection order */
        for (int i = threadIdx.x - 64; i < nsel; i += blockDim.x - 64) {
            const int t = i / a.k;
            const float top = sx[t * a.k];
            float tot = 0.f, mine = 0.f;
            for (int r = 0; r < a.k; r++) {
                const float ex = expf(sx[t * a.k + r] - top);
                tot += ex;
                if (t * a.k + r == i) mine = ex;
            }
            R.topw[i] = mine / tot;
        }
    }
    moe_sync();
}

/* Member i (token order) of group z: its token, pair index and routing weight. */
__device__ __forceinline__ void moe_member(const MoeArgs &a, const MoeRoute &R, int e, int i, int &t, int &pair, float &w) {
    unsigned long long msk = R.mask[e];
    for (int q = 0; q < i; q++) msk &= msk - 1ull;
    t = __ffsll((long long)msk) - 1;
    int s = 0;
    while (R.topi[t * a.k + s] != e) s++;
    pair = t * a.k + s;
    w = R.topw[pair];
}

/* Routing record in the workspace, after the pair images (offset from the host): written by the
 * gate/up launch, read by the down launch instead of routing again.
 *   int U, 3 x pad; int grp_e[256]; u64 group mask[256]; int topi[1024]; float topw[1024] */
#define LE_MOE_REC_BYTES (16 + 256 * 4 + 256 * 8 + 1024 * 4 + 1024 * 4)
__device__ __forceinline__ void moe_rec_write(const MoeArgs &a, const MoeRoute &R, u8 *rec) {
    const int nsel = a.n_tok * a.k;
    int *ri = (int *)rec;
    unsigned long long *rm = (unsigned long long *)(rec + 16 + 256 * 4);
    int *rt = (int *)(rec + 16 + 256 * 12);
    float *rw = (float *)(rec + 16 + 256 * 12 + 1024 * 4);
    if (threadIdx.x == 0) ri[0] = R.U;
    for (int z = threadIdx.x; z < R.U; z += blockDim.x) {
        ri[4 + z] = R.grp_e[z];
        rm[z] = R.mask[R.grp_e[z]];
    }
    for (int i = threadIdx.x; i < nsel; i += blockDim.x) {
        rt[i] = R.topi[i];
        rw[i] = R.topw[i];
    }
}
__device__ __forceinline__ void moe_rec_read(const MoeArgs &a, MoeRoute &R, const u8 *rec) {
    const int nsel = a.n_tok * a.k;
    const int *ri = (const int *)rec;
    const unsigned long long *rm = (const unsigned long long *)(rec + 16 + 256 * 4);
    const int *rt = (const int *)(rec + 16 + 256 * 12);
    const float *rw = (const float *)(rec + 16 + 256 * 12 + 1024 * 4);
    /* every load issued at once (the record's arrays have fixed sizes: no load depends on U) */
    const int z = threadIdx.x;
    const int U = *(const LE_GLOBAL int *)ri;
    const int zc = min(z, 255), sc = min(z, 1023);
    const int ge = *(const LE_GLOBAL int *)(ri + 4 + zc);
    const unsigned long long gm = *(const LE_GLOBAL unsigned long long *)(rm + zc);
    const int ti = *(const LE_GLOBAL int *)(rt + sc);
    const float tw = *(const LE_GLOBAL float *)(rw + sc);
    if (z == 0) R.U = U;
    if (z < U) {
        R.grp_e[z] = ge;
        R.mask[ge] = gm;
    }
    if (z < nsel) {
        R.topi[z] = ti;
        R.topw[z] = tw;
    }
    __syncthreads();
}

/* Launch 1: gate/up rows of unit blockIdx.x (32 rows) of group blockIdx.y for up to 8 members at
 * a time; block of 4 waves, wave w owns rows 8w..8w+7 of the unit. */
template <int TG, int TD, int G>
__device__ void moe_gu_body(const MoeArgs &a) {
    using F = Fmt<TG>;
    using D = Dec<F::NSEG, F::WPS>;
    __shared__ MoeRoute R;
    __shared__ float asv[8][32];
    __shared__ u32 tab[F::TABLES ? 256 + 512 : 1];
    extern __shared__ uint4 smem[];
    load_tables<TG>(tab);
    moe_route(a, R);
    const int z = blockIdx.y;
    if (z >= R.U) return; /* uniform across the block */
    const int e = R.grp_e[z];
    const int nmem = __popcll(R.mask[e]);
    if (blockIdx.x == 0 && z == 0) { /* routing outputs */
        for (int i = threadIdx.x; i < a.n_tok * a.k; i += blockDim.x) {
            if (a.idx_out) a.idx_out[i] = R.topi[i];
            if (a.w_out) a.w_out[i] = R.topw[i];
        }
    }
    const int K = a.hidden, nsb = K >> 8, ng = K >> 3;
    const size_t rbg = (size_t)nsb * F::SB;
    const u8 *Wg = moe_w(a.gate, a.gptr, e, (size_t)a.ff * rbg), *Wu = moe_w(a.up, a.uptr, e, (size_t)a.ff * rbg);
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    constexpr int RPW = 8 / G;
    const int li = lane & 7, g = (lane >> 3) % G, rsub = lane / (8 * G);
    const int S = nsb / G;
    const int ux = blockIdx.x;
    const int ngd = a.ff >> 3; /* groups of the down image */
    const int img_bytes = le_xtok_bytes(a.ff);
    for (int m0 = 0; m0 < nmem; m0 += 8) {
        const int nt = min(8, nmem - m0);
        XTok xt[8];
        for (int i = 0; i < nt; i++) {
            int t, pair;
            float w;
            moe_member(a, R, e, m0 + i, t, pair, w);
            le_quant_x_lds<F::XL>(a.h + (size_t)t * K, K, smem + i * ng, (float2 *)(smem + 8 * ng) + i * ng);
        }
#pragma unroll
        for (int i = 0; i < 8; i++) {
            xt[i].xq = smem + i * ng;
            xt[i].xs = (float2 *)(smem + 8 * ng) + i * ng;
        }
        __syncthreads();
        for (int st = 0; st < 8 / RPW; st++) {
            const int rl = 8 * wave + st * RPW + rsub; /* row within the 32-row unit */
            const int row = 32 * ux + rl;
            float ag[8], au[8];
#pragma unroll
            for (int i = 0; i < 8; i++) ag[i] = au[i] = 0.f;
            for (int s = 0; s < S; s++) {
                const int sb = g + G * s;
                D d[2];
                F::decode(F::load(Wg + (size_t)row * rbg + (size_t)sb * F::SB, li), li, sb, tab, d[0]);
                F::decode(F::load(Wu + (size_t)row * rbg + (size_t)sb * F::SB, li), li, sb, tab, d[1]);
#pragma unroll
                for (int i = 0; i < 8; i++) {
                    if (i < nt) {
                        float c[2] = {0.f, 0.f};
                        rows_dot<F::NSEG, F::WPS, F::HAS_MU, 2>(d, xt[i], sb, li, c);
                        ag[i] += c[0];
                        au[i] += c[1];
                    }
                }
            }
#pragma unroll
            for (int i = 0; i < 8; i++) {
                if (i < nt) {
                    const float gg = group_sum<8 * G>(ag[i]), uu = group_sum<8 * G>(au[i]);
                    if ((lane & (8 * G - 1)) == 0) asv[i][rl] = gg / (1.0f + __expf(-gg)) * uu;
                }
            }
        }
        __syncthreads();
        /* quantize each member's 32 values into its pair image: 4 threads per member */
        if (threadIdx.x < 4 * 8) {
            const int i = threadIdx.x >> 2, gw = threadIdx.x & 3;
            const bool ok = i < nt;
            float4 va = make_float4(0.f, 0.f, 0.f, 0.f), vb = va;
            if (ok) {
                va = make_float4(asv[i][8 * gw], asv[i][8 * gw + 1], asv[i][8 * gw + 2], asv[i][8 * gw + 3]);
                vb = make_float4(asv[i][8 * gw + 4], asv[i][8 * gw + 5], asv[i][8 * gw + 6], asv[i][8 * gw + 7]);
            }
            float am = amax8(va, vb);
            am = fmaxf(am, __shfl_xor(am, 1));
            am = fmaxf(am, __shfl_xor(am, 2));
            if (ok) {
                int t, pair;
                float w;
                moe_member(a, R, e, m0 + i, t, pair, w);
                uint4 *img = (uint4 *)(a.ws + (size_t)pair * img_bytes);
                le_quant_group(va, vb, am, img, (float2 *)(img + ngd), le_xpos<Fmt<TD>::XL>(4 * ux + gw));
            }
        }
        __syncthreads();
    }
}

/* Launch 2: output rows 8*blockIdx.x .. +7 (one row per 8-lane group) over all groups. */
template <int TD>
__device__ void moe_down_body(const MoeArgs &a) {
    using F = Fmt<TD>;
    using D = Dec<F::NSEG, F::WPS>;
    __shared__ MoeRoute R;
    __shared__ float red[4][LE_MOE_MAXTOK][8];
    __shared__ u32 tab[F::TABLES ? 256 + 512 : 1];
    load_tables<TD>(tab);
    moe_route(a, R);
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    for (int i = threadIdx.x; i < 4 * LE_MOE_MAXTOK * 8; i += blockDim.x) (&red[0][0][0])[i] = 0.f;
    __syncthreads();
    const int K = a.ff, nsb = K >> 8, ng = K >> 3;
    const size_t rbd = (size_t)nsb * F::SB;
    const int li = lane & 7, rr = lane >> 3, row = 8 * blockIdx.x + rr;
    const int img_bytes = le_xtok_bytes(K);
    for (int z = wave; z < R.U; z += 4) {
        const int e = R.grp_e[z];
        const int nmem = __popcll(R.mask[e]);
        const u8 *Wd = moe_w(a.down, a.dptr, e, (size_t)a.hidden * rbd) + (size_t)row * rbd;
        for (int m0 = 0; m0 < nmem; m0 += 8) {
            const int nt = min(8, nmem - m0);
            XTok xt[8];
            int tt[8];
            float ww[8];
#pragma unroll
            for (int i = 0; i < 8; i++) {
                int pair = 0;
                tt[i] = 0;
                ww[i] = 0.f;
                if (i < nt) moe_member(a, R, e, m0 + i, tt[i], pair, ww[i]);
                const uint4 *img = (const uint4 *)(a.ws + (size_t)pair * img_bytes);
                xt[i].xq = img;
                xt[i].xs = (const float2 *)(img + ng);
            }
            float acc[8];
#pragma unroll
            for (int i = 0; i < 8; i++) acc[i] = 0.f;
            for (int sb = 0; sb < nsb; sb++) {
                D d[1];
                F::decode(F::load(Wd + (size_t)sb * F::SB, li), li, sb, tab, d[0]);
#pragma unroll
                for (int i = 0; i < 8; i++) {
                    if (i < nt) {
                        float c[1] = {0.f};
                        rows_dot<F::NSEG, F::WPS, F::HAS_MU, 1>(d, xt[i], sb, li, c);
                        acc[i] += c[0];
                    }
                }
            }
#pragma unroll
            for (int i = 0; i < 8; i++) {
                if (i < nt) {
                    const float v = group_sum<8>(acc[i]);
                    if (li == 0) red[wave][tt[i]][rr] += ww[i] * v;
                }
            }
        }
    }
    __syncthreads();
    for (int i = threadIdx.x; i < a.n_tok * 8; i += blockDim.x) {
        const int t = i >> 3, r = i & 7;
        a.out[(size_t)t * a.hidden + 8 * blockIdx.x + r] = ((red[0][t][r] + red[1][t][r]) + red[2][t][r]) + red[3][t][r];
    }
}

/* Decode-shaped fast paths (n_tok <= 8): every wave issues all of its weight loads at once, the
 * activations and router logits go out before anything waits, and the down projection reads the
 * quantized SwiGLU images from LDS when they fit. */
#define LE_MOE_FAST_TOK 8
template <int TG, int TD, int G>
__device__ void moe_gu_fast(const MoeArgs &a) {
    using F = Fmt<TG>;
    using D = Dec<F::NSEG, F::WPS>;
    using Raw = typename F::Raw;
    constexpr int NW = 16, RPW = 8 / G, JS = (32 / RPW + NW - 1) / NW, XR = 4;
    __shared__ MoeRoute R;
    __shared__ float asv[8][32];
    __shared__ __attribute__((aligned(16))) unsigned long long lv[LE_MOE_FAST_TOK * LE_MOE_MAXEXP];
    __shared__ float sx[LE_MOE_FAST_TOK * LE_MOE_MAXK];
    __shared__ u32 tab[F::TABLES ? 256 + 512 : 1];
    extern __shared__ uint4 smem[];
    const int K = a.hidden, nsb = K >> 8, ng = K >> 3;
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    /* 1. every token's activations (n_tok * ng <= XR * 1024 groups), clamped and unpredicated */
    const MoeLogits lgt = moe_route_load(a); /* first, so routing waits for these loads alone */
    float4 ha[XR], hb[XR];
    const int ngt = a.n_tok * ng;
#pragma unroll
    for (int r = 0; r < XR; r++) {
        const int gp = min((int)threadIdx.x + 1024 * r, ngt - 1);
        const float *src = a.h + (size_t)(gp / ng) * K + 8 * (gp % ng);
        ha[r] = *(const LE_GLOBAL float4 *)src;
        hb[r] = *(const LE_GLOBAL float4 *)(src + 4);
    }
    load_tables<TG>(tab);
    moe_route_par(a, R, lv, sx, lgt);
    const int z = blockIdx.y;
    if (z >= R.U) return;
    const int e = R.grp_e[z];
    const int nmem = __popcll(R.mask[e]);
    if (blockIdx.x == 0 && z == 0) {
        for (int i = threadIdx.x; i < a.n_tok * a.k; i += blockDim.x) {
            if (a.idx_out) a.idx_out[i] = R.topi[i];
            if (a.w_out) a.w_out[i] = R.topw[i];
        }
    }
    /* 2. weight loads of this wave's rows: wave-step ws = wave + NW*j covers rows ws*RPW .. */
    const size_t rbg = (size_t)nsb * F::SB;
    const u8 *Wg = moe_w(a.gate, a.gptr, e, (size_t)a.ff * rbg), *Wu = moe_w(a.up, a.uptr, e, (size_t)a.ff * rbg);
    const int li = lane & 7, g = (lane >> 3) % G, rsub = lane / (8 * G);
    const int S = nsb / G; /* <= 2 on this path */
    const int ux = blockIdx.x;
    Raw rg[JS][2], ru[JS][2];
#pragma unroll
    for (int j = 0; j < JS; j++) {
        const int rl = min((wave + NW * j) * RPW + rsub, 31);
        const size_t ro = (size_t)(32 * ux + rl) * rbg;
#pragma unroll
        for (int s = 0; s < 2; s++) {
            const int sb = g + G * min(s, S - 1);
            rg[j][s] = F::load(Wg + ro + (size_t)sb * F::SB, li);
            ru[j][s] = F::load(Wu + ro + (size_t)sb * F::SB, li);
        }
    }
    /* 3. quantize the activations into token images */
    uint4 *xq = smem;
    float2 *xs = (float2 *)(smem + LE_MOE_FAST_TOK * ng);
#pragma unroll
    for (int r = 0; r < XR; r++) {
        const int gp = (int)threadIdx.x + 1024 * r;
        if (r * 1024 >= ngt) break;
        float am = amax8(ha[r], hb[r]);
        am = fmaxf(am, __shfl_xor(am, 1));
        am = fmaxf(am, __shfl_xor(am, 2));
        if (gp < ngt) {
            const int t = gp / ng, p = gp % ng;
            le_quant_group(ha[r], hb[r], am, xq + t * ng, xs + t * ng, le_xpos<F::XL>(p));
        }
    }
    int tokm[8], pairm[8];
    float wm[8];
#pragma unroll
    for (int i = 0; i < 8; i++) {
        tokm[i] = 0;
        pairm[i] = 0;
        if (i < nmem) moe_member(a, R, e, i, tokm[i], pairm[i], wm[i]);
    }
    __syncthreads();
    /* 4. gate and up rows for every member; the wave's JS rows go through one dot so their
     * chains interleave */
    float ag[JS][8], au[JS][8];
#pragma unroll
    for (int j = 0; j < JS; j++)
#pragma unroll
        for (int i = 0; i < 8; i++) ag[j][i] = au[j][i] = 0.f;
#pragma unroll
    for (int s = 0; s < 2; s++) {
        if (s < S) {
            const int sb = g + G * s;
            D d[2 * JS];
#pragma unroll
            for (int j = 0; j < JS; j++) {
                F::decode(rg[j][s], li, sb, tab, d[2 * j]);
                F::decode(ru[j][s], li, sb, tab, d[2 * j + 1]);
            }
#pragma unroll
            for (int i = 0; i < 8; i++) {
                if (i < nmem) {
                    XTok xt;
                    xt.xq = xq + tokm[i] * ng;
                    xt.xs = xs + tokm[i] * ng;
                    float c[2 * JS];
#pragma unroll
                    for (int q = 0; q < 2 * JS; q++) c[q] = 0.f;
                    rows_dot<F::NSEG, F::WPS, F::HAS_MU, 2 * JS>(d, xt, sb, li, c);
#pragma unroll
                    for (int j = 0; j < JS; j++) {
                        ag[j][i] += c[2 * j];
                        au[j][i] += c[2 * j + 1];
                    }
                }
            }
        }
    }
#pragma unroll
    for (int j = 0; j < JS; j++) {
        const int wsj = wave + NW * j;
        if (wsj * RPW >= 32) break; /* wave-uniform */
        const int rl = wsj * RPW + rsub;
#pragma unroll
        for (int i = 0; i < 8; i++) {
            if (i < nmem) {
                const float gg = group_sum<8 * G>(ag[j][i]), uu = group_sum<8 * G>(au[j][i]);
                if ((lane & (8 * G - 1)) == 0) asv[i][rl] = gg / (1.0f + __expf(-gg)) * uu;
            }
        }
    }
    __syncthreads();
    /* 5. the unit's SwiGLU values, quantized into each member's down image */
    if (threadIdx.x < 32) {
        const int i = threadIdx.x >> 2, gw = threadIdx.x & 3;
        const bool ok = i < nmem;
        float4 va = make_float4(0.f, 0.f, 0.f, 0.f), vb = va;
        if (ok) {
            va = make_float4(asv[i][8 * gw], asv[i][8 * gw + 1], asv[i][8 * gw + 2], asv[i][8 * gw + 3]);
            vb = make_float4(asv[i][8 * gw + 4], asv[i][8 * gw + 5], asv[i][8 * gw + 6], asv[i][8 * gw + 7]);
        }
        float am = amax8(va, vb);
        am = fmaxf(am, __shfl_xor(am, 1));
        am = fmaxf(am, __shfl_xor(am, 2));
        if (ok) {
            const int pair = pairm[0] * 0 + (i == 0 ? pairm[0] : i == 1 ? pairm[1] : i == 2 ? pairm[2] : i == 3 ? pairm[3]
                                              : i == 4 ? pairm[4] : i == 5 ? pairm[5] : i == 6 ? pairm[6] : pairm[7]);
            uint4 *img = (uint4 *)(a.ws + (size_t)pair * le_xtok_bytes(a.ff));
            le_quant_group(va, vb, am, img, (float2 *)(img + (a.ff >> 3)), le_xpos<Fmt<TD>::XL>(4 * ux + gw));
        }
    }
}

/* Launch 2 fast path: 8 output rows per block, 8 waves take the groups round-robin (one group in
 * flight per wave, the next one prefetched); ff <= 1024 so a lane's row needs at most 4
 * super-blocks. */
template <int TD>
__device__ void moe_down_fast(const MoeArgs &a) {
    using F = Fmt<TD>;
    using D = Dec<F::NSEG, F::WPS>;
    using Raw = typename F::Raw;
    constexpr int NW = 8, SM = 4;
    __shared__ MoeRoute R;
    __shared__ float red[NW][LE_MOE_FAST_TOK][8];
    __shared__ __attribute__((aligned(16))) unsigned long long lv[LE_MOE_FAST_TOK * LE_MOE_MAXEXP];
    __shared__ float sx[LE_MOE_FAST_TOK * LE_MOE_MAXK];
    __shared__ u32 tab[F::TABLES ? 256 + 512 : 1];
    extern __shared__ uint4 smem[];
    const MoeLogits lgt = moe_route_load(a);
    load_tables<TD>(tab);
    moe_route_par(a, R, lv, sx, lgt);
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const int K = a.ff, nsb = K >> 8, ng = K >> 3;
    const int img_bytes = le_xtok_bytes(K);
    const int npair = a.n_tok * a.k;
    const bool in_lds = (size_t)npair * img_bytes <= 49152;
    if (in_lds) {
        const int n16 = npair * img_bytes / 16;
        const LE_GLOBAL uint4 *src = (const LE_GLOBAL uint4 *)a.ws;
        for (int i = threadIdx.x; i < n16; i += blockDim.x) smem[i] = src[i];
    }
    for (int i = threadIdx.x; i < NW * LE_MOE_FAST_TOK * 8; i += blockDim.x) (&red[0][0][0])[i] = 0.f;
    __syncthreads();
    const size_t rbd = (size_t)nsb * F::SB;
    const int li = lane & 7, rr = lane >> 3, row = 8 * blockIdx.x + rr;
    Raw ra[SM], rb2[SM];
    auto issue = [&](int z, Raw (&r)[SM]) {
        const u8 *Wd = moe_w(a.down, a.dptr, R.grp_e[z], (size_t)a.hidden * rbd) + (size_t)row * rbd;
#pragma unroll
        for (int s = 0; s < SM; s++) r[s] = F::load(Wd + (size_t)min(s, nsb - 1) * F::SB, li);
    };
    /* img0 is either LDS or the workspace; each call site passes one of them, so the image reads
     * compile to LDS or global loads (a pointer that could be either becomes a flat load, which
     * also waits on the LDS counter) */
    auto consume = [&](int z, Raw (&r)[SM], const u8 *img0) {
        const int e = R.grp_e[z];
        const int nmem = __popcll(R.mask[e]);
        int tt[8];
        float ww[8];
        XTok xt[8];
#pragma unroll
        for (int i = 0; i < 8; i++) {
            int pair = 0;
            tt[i] = 0;
            ww[i] = 0.f;
            if (i < nmem) moe_member(a, R, e, i, tt[i], pair, ww[i]);
            const uint4 *img = (const uint4 *)(img0 + (size_t)pair * img_bytes);
            xt[i].xq = img;
            xt[i].xs = (const float2 *)(img + ng);
        }
        float acc[8];
#pragma unroll
        for (int i = 0; i < 8; i++) acc[i] = 0.f;
#pragma unroll
        for (int s = 0; s < SM; s++) {
            if (s < nsb) {
                D d[1];
                F::decode(r[s], li, s, tab, d[0]);
#pragma unroll
                for (int i = 0; i < 8; i++) {
                    if (i < nmem) {
                        float c[1] = {0.f};
                        rows_dot<F::NSEG, F::WPS, F::HAS_MU, 1>(d, xt[i], s, li, c);
                        acc[i] += c[0];
                    }
                }
            }
        }
#pragma unroll
        for (int i = 0; i < 8; i++) {
            if (i < nmem) {
                const float v = group_sum<8>(acc[i]);
                if (li == 0) red[wave][tt[i]][rr] += ww[i] * v;
            }
        }
    };
    auto groups = [&](const u8 *img0) {
        int z = wave;
        if (z < R.U) issue(z, ra);
        while (z < R.U) {
            if (z + NW < R.U) issue(z + NW, rb2);
            consume(z, ra, img0);
            z += NW;
            if (z >= R.U) break;
            if (z + NW < R.U) issue(z + NW, ra);
            consume(z, rb2, img0);
            z += NW;
        }
    };
    if (in_lds)
        groups((const u8 *)smem);
    else
        groups(a.ws);
    __syncthreads();
    for (int i = threadIdx.x; i < a.n_tok * 8; i += blockDim.x) {
        const int t = i >> 3, r = i & 7;
        float acc = 0.f;
#pragma unroll
        for (int w = 0; w < NW; w++) acc += red[w][t][r];
        a.out[(size_t)t * a.hidden + 8 * blockIdx.x + r] = acc;
    }
}

/* ===================== MoE on the staged MFMA kernels (decode-shaped: n_tok <= 8) =====================
 * Launch 1 (le_moe_gum_12_<td>_p<P>): grid (ff/32, groups), four waves. Each block routes, builds the
 * MFMA activation image of every token's h in LDS (one shared copy), and streams its expert's
 * 32-row unit of gate and of up as four 16-row tiles; wave w owns super-blocks wP..wP+P-1 of each
 * row (hidden = 1024 P). The SwiGLU values of the unit are one 32-value sub-block of the down
 * projection's input, quantized straight into each member's down image in the workspace (the
 * image format of the staged kernels, under the down type's slice map).
 * Launch 2 (le_moe_dnm_<td>_p<P>): grid (hidden/16), four waves taking the expert groups
 * round-robin; per group the 16 rows x P super-blocks (ff = 256 P) are staged like the matvec, the
 * members' images are copied into the wave's LDS, and each member's dot is weighted and added to
 * its token's rows. The waves' sums are added in a fixed order. */
#define LE_MOE_IMG(K) ((K) / 256 * 608) /* bytes of one token's MFMA activation image */
#ifdef LE_MOE_TRACE /* timing builds only: per-block timestamps after the workspace's first MiB */
#define MOE_T(i) (tr_[i] = __builtin_amdgcn_s_memrealtime())
#define MOE_T_DECL unsigned long long tr_[8] = {0, 0, 0, 0, 0, 0, 0, 0}
#define MOE_T_OUT(base)                                                                              \
    if (threadIdx.x == 0) {                                                                          \
        unsigned long long *o_ = (unsigned long long *)(a.bar + (1 << 20)) + (base) + 8 * (blockIdx.x + gridDim.x * blockIdx.y); \
        for (int i_ = 0; i_ < 8; i_++) o_[i_] = tr_[i_];                                             \
    }
#else
#define MOE_T(i)
#define MOE_T_DECL
#define MOE_T_OUT(base)
#endif

/* LDS layout of the staged MoE kernels: the routing keys (needed only until routing is done)
 * share their bytes with the weight staging that follows. */
#define LE_MOE_LV_BYTES (LE_MOE_FAST_TOK * LE_MOE_MAXEXP * 8)

template <int TD, int NW, int P>
__device__ __forceinline__ void moe_gum_body(const MoeArgs &a) {
    constexpr int CPR = 9 * P + 1, NCH = 4 * 16 * CPR, NI = (NCH + 63) / 64, MAPD = TD == LE_TYPE_Q6_K ? 1 : 0;
    constexpr int K = 256 * NW * P, NSB = NW * P, SEGT = K / 16, NT = 64 * NW; /* segments of 16 values per token */
    constexpr int XR = (LE_MOE_FAST_TOK * SEGT + NT - 1) / NT;
    __shared__ MoeRoute R;
    __shared__ float sx[LE_MOE_FAST_TOK * LE_MOE_MAXK];
    __shared__ float red[NW][LE_MOE_FAST_TOK][64];
    __shared__ __attribute__((aligned(16))) float act[LE_MOE_FAST_TOK][32];
    __shared__ int mtok[LE_MOE_FAST_TOK], mpair[LE_MOE_FAST_TOK];
    extern __shared__ uint4 smem[];
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6, n = lane & 15;
    uint4 *img = smem;                                          /* [n_tok][image] */
    uint4 *stg = smem + LE_MOE_FAST_TOK * LE_MOE_IMG(K) / 16;  /* [NW][NI*64] staging; routing keys first */
    uint4 *wb = stg + wave * NI * 64;
    MOE_T_DECL;
    MOE_T(0);
    const MoeLogits lgt = moe_route_load(a); /* first, so routing waits for these loads alone */
    /* 1. every token's activations, 16 values per (thread, r), clamped and unpredicated */
    const int nseg = a.n_tok * SEGT;
    float4 hv[XR][4];
#pragma unroll
    for (int r = 0; r < XR; r++) {
        const int e = min((int)threadIdx.x + NT * r, nseg - 1);
        mq_load_seg(a.h + (size_t)(e / SEGT) * K, e % SEGT, hv[r]);
    }
    moe_route_par(a, R, (unsigned long long *)stg, sx, lgt);
    MOE_T(1);
#ifdef LE_MOE_TRACE
    tr_[2] = R.tr[1]; tr_[3] = R.tr[2];
#endif
    const int z = blockIdx.y;
    if (z >= R.U) return; /* uniform over the block */
    const int e = R.grp_e[z];
    const int nmem = __popcll(R.mask[e]);
    /* 2. the four tiles of this wave's super-blocks (gate rows 32ux.., +16, up rows 32ux.., +16),
     * packed: chunk c = (tile, row, column) of 4 x 16 x CPR, all in flight at once */
    const size_t rb = (size_t)NSB * 144;
    const u8 *Wg = moe_w(a.gate, a.gptr, e, (size_t)a.ff * rb), *Wu = moe_w(a.up, a.uptr, e, (size_t)a.ff * rb);
    const int ux = blockIdx.x;
    uint4 Rg[NI];
#pragma unroll
    for (int i = 0; i < NI; i++) {
        const int c = min(64 * i + lane, NCH - 1), ti = c / (16 * CPR), rem = c % (16 * CPR), col = rem % CPR;
        Rg[i] = ldg16((ti < 2 ? Wg : Wu) + (size_t)(32 * ux + 16 * (ti & 1) + rem / CPR) * rb + (size_t)wave * P * 144 +
                      (col == 9 * P ? 0 : col) * 16);
    }
    /* block (0,0) also writes the routing outputs and record, and clears the output (the down
     * launch may split a row tile over two blocks that add into it), after issuing its weights so
     * those stores do not delay them */
    if (blockIdx.x == 0 && z == 0) {
        for (int i = threadIdx.x; i < a.n_tok * a.k; i += blockDim.x) {
            if (a.idx_out) a.idx_out[i] = R.topi[i];
            if (a.w_out) a.w_out[i] = R.topw[i];
        }
        moe_rec_write(a, R, a.ws + (size_t)a.n_tok * a.k * LE_MOE_IMG(a.ff));
        for (int i = threadIdx.x; i < a.n_tok * a.hidden; i += blockDim.x) a.out[i] = 0.f;
    }
    /* 3. token images (the Q4_K slice map) and the group's members */
#pragma unroll
    for (int r = 0; r < XR; r++) {
        const int eg = (int)threadIdx.x + NT * r;
        if (r * NT >= nseg) break;
        const int t = min(eg, nseg - 1) / SEGT, el = min(eg, nseg - 1) % SEGT;
        uint4 *rec = img + t * (LE_MOE_IMG(K) / 16);
        float *dxp = (float *)(rec + NSB * 32), *fsv = dxp + NSB * 16;
        mq_quant_seg<0>(el, eg < nseg, hv[r], rec, dxp, fsv);
    }
    if (threadIdx.x < nmem) {
        int t, pair;
        float w;
        moe_member(a, R, e, threadIdx.x, t, pair, w);
        mtok[threadIdx.x] = t;
        mpair[threadIdx.x] = pair;
    }
    
#pragma unroll
    for (int i = 0; i < NI; i++) wb[64 * i + lane] = Rg[i];
    
    moe_sync();
    
    /* 4. per member (a runtime loop: the code stays small), four tiles x this wave's super-blocks */
    const MsLane L = ms_lane<0>(lane);
    le_v4i A[4];
#pragma unroll
    for (int b = 0; b < 4; b++) A[b] = (le_v4i){0, 0, 0, 0};
#pragma unroll 1
    for (int i = 0; i < nmem; i++) {
        const uint4 *rec = img + mtok[i] * (LE_MOE_IMG(K) / 16);
        const float *dxp = (const float *)(rec + NSB * 32), *fsv = dxp + NSB * 16;
        float y[4] = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
        for (int q = 0; q < P; q++) {
            const int sb = wave * P + q;
            ms_load_a(rec + sb * 32, L, A);
            ms_sb_q4k_n<4>(wb + n * CPR + 9 * q, 16 * CPR, A, dxp + sb * 16, fsv + sb * 8, L, y);
        }
#pragma unroll
        for (int ti = 0; ti < 4; ti++) {
            float v = y[ti];
            v = row4_sum(v);
            if (lane < 16) red[wave][i][16 * ti + lane] = v;
        }
    }
    
    moe_sync();
    /* 5. SwiGLU of the unit's 32 values = sub-block ux of the down input: thread (member i, row r)
     * adds the waves for gate and up; then lanes 2i, 2i+1 of wave 0 quantize member i's two
     * 16-value segments into its down image */
    if (threadIdx.x < 32 * LE_MOE_FAST_TOK) {
        const int i = threadIdx.x >> 5, r = threadIdx.x & 31;
        if (i < nmem) {
            float g = 0.f, u = 0.f;
#pragma unroll
            for (int w = 0; w < NW; w++) {
                g += red[w][i][r];
                u += red[w][i][32 + r];
            }
            act[i][r] = g / (1.0f + __expf(-g)) * u;
        }
    }
    moe_sync();
    if (wave == 0 && lane < 2 * LE_MOE_FAST_TOK) {
        const int i = lane >> 1, c = lane & 1;
        const bool ok = i < nmem;
        const float4 *av = (const float4 *)&act[ok ? i : 0][16 * c];
        float4 v4[4];
#pragma unroll
        for (int q = 0; q < 4; q++) v4[q] = av[q];
        const int nsbd = a.ff >> 8;
        uint4 *rec = (uint4 *)(a.ws + (size_t)mpair[ok ? i : 0] * LE_MOE_IMG(a.ff));
        float *dxp = (float *)(rec + nsbd * 32), *fsv = dxp + nsbd * 16;
        mq_quant_seg<MAPD>(2 * ux + c, ok, v4, rec, dxp, fsv);
    }
    MOE_T(6);
    MOE_T_OUT(0);
}

#define LE_MOE_DN_IMGS 16 /* pair images the down kernel keeps in LDS */
template <int TD, int NW, int P>
__device__ __forceinline__ void moe_dnm_body(const MoeArgs &a) {
    constexpr int MAPD = TD == LE_TYPE_Q6_K ? 1 : 0, CPS = TD == LE_TYPE_Q6_K ? 14 : 9, SBB = TD == LE_TYPE_Q6_K ? 210 : 144;
    constexpr int CPR = CPS * P + 1, NCH = 16 * CPR, NI = (NCH + 63) / 64, IMG = LE_MOE_IMG(256 * P), IMGC = IMG / 16;
    constexpr int SLOTS = LE_MOE_DN_IMGS / NW; /* image slots per wave when the pairs do not all fit */
    __shared__ MoeRoute R;
    __shared__ float sx[LE_MOE_FAST_TOK * LE_MOE_MAXK];
    __shared__ float red[NW][LE_MOE_FAST_TOK][16];
    __shared__ int mtok[NW][LE_MOE_FAST_TOK], mpair[NW][LE_MOE_FAST_TOK];
    __shared__ float mw[NW][LE_MOE_FAST_TOK];
    extern __shared__ uint4 smem[];
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6, n = lane & 15;
    uint4 *imgs = smem;                          /* LE_MOE_DN_IMGS images */
    uint4 *stg = smem + LE_MOE_DN_IMGS * IMGC;   /* [NW][NI*64] staging; routing keys first */
    uint4 *wb = stg + wave * NI * 64;
    MOE_T_DECL;
    MOE_T(0);
    for (int i = threadIdx.x; i < NW * LE_MOE_FAST_TOK * 16; i += blockDim.x) (&red[0][0][0])[i] = 0.f;
    const int npair = a.n_tok * a.k;
    const bool all_in = npair <= LE_MOE_DN_IMGS;
    /* every pair's down image (written by the gate/up launch; needs no routing), issued before
     * the routing record is read so the two round trips overlap */
    uint4 iv[2][4];
    static_assert(LE_MOE_DN_IMGS * IMGC <= 8 * 64 * NW, "the image preload covers every image chunk");
    const int nci = npair * IMGC;
    if (all_in) { /* only the rounds that hold image chunks (uniform over the block): clamped
                     * re-reads of the last chunk had queued 4.5x the image bytes at one token
                     * ahead of the weight loads */
#pragma unroll
        for (int u = 0; u < 2; u++)
#pragma unroll
            for (int q = 0; q < 4; q++)
                if (64 * NW * (4 * u + q) < nci) iv[u][q] = ldg16c(a.ws + 16 * (size_t)min((int)threadIdx.x + 64 * NW * (4 * u + q), nci - 1));
    }
    /* the routing of the gate/up launch (n_tok * k <= 64 <= blockDim.x, groups <= 64) */
    moe_rec_read(a, R, a.ws + (size_t)a.n_tok * a.k * IMG);
    MOE_T(1);
    const size_t rb = (size_t)P * SBB;
    /* H blocks per 16-row tile (grid = H * hidden / 16): block hh of a tile takes the expert groups
     * z = hh (mod H) and, with H = 2, adds into the output the gate/up launch zeroed (every
     * element is 0 + a + b in either order: the same bits) */
    const int ntile = a.hidden >> 4, H = gridDim.x / ntile, hh = blockIdx.x / ntile;
    const int row0 = 16 * (blockIdx.x % ntile);
    int roff[NI];
#pragma unroll
    for (int i = 0; i < NI; i++) {
        const int c = min(64 * i + lane, NCH - 1), col = c % CPR, cc = col == CPS * P ? 0 : col;
        roff[i] = (row0 + c / CPR) * (int)rb + (TD == LE_TYPE_Q6_K ? (cc / 14) * 210 + q6_goff(cc % 14) : cc * 16);
    }
    /* weights of two groups in flight: R0 is the next group to compute, R1 the one after */
    uint4 R0[NI], R1[NI];
    auto issue = [&](int zz, uint4 (&r)[NI]) {
        const u8 *W = moe_w(a.down, a.dptr, R.grp_e[zz], (size_t)a.hidden * rb);
#pragma unroll
        for (int i = 0; i < NI; i++) r[i] = TD == LE_TYPE_Q6_K ? ldg16u(W + roff[i]) : ldg16(W + roff[i]);
    };
    if (hh + H * wave < R.U) issue(hh + H * wave, R0);
    if (hh + H * (wave + NW) < R.U) issue(hh + H * (wave + NW), R1);
    if (all_in) { /* the images loaded above (LE_MOE_DN_IMGS * IMGC <= 8 * 64 * NW chunks) */
#pragma unroll
        for (int u = 0; u < 2; u++)
#pragma unroll
            for (int q = 0; q < 4; q++) {
                const int c = (int)threadIdx.x + 64 * NW * (4 * u + q);
                if (c < nci) imgs[c] = iv[u][q];
            }
    }
    moe_sync(); /* the images, and the routing keys are no longer read before staging reuses them */
    MOE_T(2);
    const MsLane L = ms_lane<MAPD>(lane);
    le_v4i A[4];
#pragma unroll
    for (int b = 0; b < 4; b++) A[b] = (le_v4i){0, 0, 0, 0};
    uint4 *wimg = imgs + wave * SLOTS * IMGC;
#pragma unroll 1
    for (int z = hh + H * wave; z < R.U; z += H * NW) {
        const int e = R.grp_e[z];
        const int nmem = __popcll(R.mask[e]);
        if (lane < nmem) {
            int t, pair;
            float w;
            moe_member(a, R, e, lane, t, pair, w);
            mtok[wave][lane] = t;
            mpair[wave][lane] = pair;
            mw[wave][lane] = w;
        }
#pragma unroll
        for (int i = 0; i < NI; i++) {
            wb[64 * i + lane] = R0[i];
            R0[i] = R1[i];
        }
        if (z + 2 * H * NW < R.U) issue(z + 2 * H * NW, R1);
#pragma unroll 1
        for (int i = 0; i < nmem; i++) {
            const uint4 *rec;
            if (all_in) {
                rec = imgs + mpair[wave][i] * IMGC;
            } else { /* this member's image into one of the wave's slots */
                uint4 *slot = wimg + (i % SLOTS) * IMGC;
                const int pr = mpair[wave][i];
                for (int o = lane; o < IMGC; o += 64) slot[o] = ldg16c(a.ws + (size_t)pr * IMG + 16 * o);
                rec = slot;
            }
            const float *dxp = (const float *)(rec + P * 32), *fsv = dxp + P * 16;
            float y = 0.f;
#pragma unroll
            for (int q = 0; q < P; q++) {
                ms_load_a(rec + q * 32, L, A);
                if constexpr (TD == LE_TYPE_Q6_K)
                    y += ms_sb_q6k(wb + n * CPR + CPS * q, A, dxp + q * 16, L);
                else
                    y += ms_sb_q4k(wb + n * CPR + CPS * q, A, dxp + q * 16, fsv + q * 8, L);
            }
            y = row4_sum(y);
            if (lane < 16) red[wave][mtok[wave][i]][lane] += mw[wave][i] * y;
        }
        MOE_T(3);
    }
    MOE_T(4);
    moe_sync();
    MOE_T(5);
    for (int i = threadIdx.x; i < a.n_tok * 16; i += blockDim.x) {
        const int t = i >> 4, r = i & 15;
        float acc = 0.f;
#pragma unroll
        for (int w = 0; w < NW; w++) acc += red[w][t][r];
        if (H == 2)
            atomicAdd(a.out + (size_t)t * a.hidden + row0 + r, acc);
        else
            a.out[(size_t)t * a.hidden + row0 + r] = acc;
    }
    MOE_T(6);
    MOE_T_OUT(4096);
}

/* ===================== MoE in one launch: gate/up, a device-wide barrier, down =====================
 * A persistent grid (the host launches no more blocks than fit on the device at once) of 8-wave
 * blocks. Every block routes. Phase 1: blocks take the (32-row unit, expert group) items of the
 * gate/up projection round-robin, as in le_moe_gum (hidden 2048). Before that, each block issues
 * the weight loads of its first down group (they depend on the routing only), so they arrive
 * while phase 1 runs. A barrier over all blocks separates the phases. Phase 2: row tile b mod
 * ntile of the down projection as in le_moe_dnm; when the grid has at least two blocks per tile,
 * blocks b and b + ntile split the tile's expert groups and add into the output (zeroed in
 * phase 1).
 *
 * Barrier. Its state lives in the caller's workspace (so launches with different workspaces never
 * share it): per block an arrival flag, one generation word and a status word. Each launch
 * takes its epoch from the device: every block reads the generation word before it arrives, and
 * nothing changes that word until every block has arrived, so all blocks read the same value g
 * and use g + 1 (top bit cleared). Launches on one workspace therefore count up one by one,
 * also when a HIP graph replays the same kernel arguments, and a flag or generation left by an
 * earlier launch (or a late block of a launch that gave up) never matches. Block 0 polls every flag and then
 * publishes either the epoch or, if a wait gave up, the epoch with the top bit set; every other
 * block waits for one of the two. Every wait is bounded (spin_limit polls); a block whose wait
 * gave up, or that sees the failure generation, sets the status word (to LE_MOE_BAR_FAILED, a
 * value an uninitialised workspace holds with probability 2^-32) and writes NaN to all of
 * its outputs, so a failed launch is visible in the output and through le_moe_check. Launches
 * that share one workspace must not overlap (two streams), and the grid assumes it is resident
 * by itself: a concurrent kernel that occupies CUs can make the waits give up. */
#define LE_MOE_MAXGRID 1024

/* Arrival is a plain store of the epoch to the block's own flag, so no arrival contends with
 * another; block 0 polls all flags in parallel. Callers store what other blocks read after the
 * barrier with device-coherent stores (mq_quant_seg<.., true>). Returns false when a wait gave up
 * or block 0 published a failure. */
template <class F>
__device__ __forceinline__ bool moe_grid_barrier(const MoeArgs &a, unsigned int nblocks, F &&after_arrival) {
    __shared__ int ok_s;
    unsigned int *status = (unsigned int *)(a.bar + LE_MOE_BAR_STATUS);
    unsigned long long *gen = (unsigned long long *)(a.bar + LE_MOE_BAR_GEN);
    unsigned long long *flag = (unsigned long long *)(a.bar + LE_MOE_BAR_FLAGS);
    __shared__ unsigned long long ep_s;
    if (threadIdx.x == 0) /* before this block's arrival: no block can publish a new generation yet */
        ep_s = (__hip_atomic_load(gen, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) & ~(1ull << 63)) + 1;
    __builtin_amdgcn_s_waitcnt(0x0F70); /* vmcnt(0): this thread's coherent stores have completed */
    __syncthreads();
    const unsigned long long ep = ep_s & ~(1ull << 63), fail = ep | (1ull << 63);
    if (threadIdx.x == 0) {
        ok_s = a.spin_limit > 0; /* a zero limit is the host's way to make the barrier fail */
        /* the data other blocks read was stored device-coherently and has completed (the block
         * barrier above waits for it), so the arrival needs no L2 writeback */
        __hip_atomic_store(&flag[blockIdx.x], ep, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    }
    __syncthreads();
    after_arrival(); /* work that must not delay the arrival (its loads are not waited for above) */
    if (blockIdx.x == 0) {
        for (unsigned int i = threadIdx.x; i < nblocks; i += blockDim.x) {
            unsigned int spins = 0;
            /* relaxed polls (an acquire per poll would invalidate L2 every time); one acquire after */
            while (__hip_atomic_load(&flag[i], __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) != ep) {
                if (spins++ >= a.spin_limit) { /* give up instead of hanging */
                    ok_s = 0;
                    break;
                }
                __builtin_amdgcn_s_sleep(1);
            }
        }
        __syncthreads();
        if (threadIdx.x == 0) {
            if (!ok_s) __hip_atomic_store(status, LE_MOE_BAR_FAILED, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
            __hip_atomic_store(gen, ok_s ? ep : fail, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        }
    } else if (threadIdx.x == 0) {
        unsigned int spins = 0;
        unsigned long long g;
        while ((g = __hip_atomic_load(gen, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT)) != ep && g != fail) {
            if (spins++ >= a.spin_limit) break;
            __builtin_amdgcn_s_sleep(1);
        }
        if (g != ep) {
            ok_s = 0;
            __hip_atomic_store(status, LE_MOE_BAR_FAILED, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        }
    }
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "agent");
    __syncthreads();
    return ok_s != 0;
}

template <int TD, int PD>
__device__ __forceinline__ void moe_fus_body(const MoeArgs &a) {
    constexpr int NW = 8, P = 1, CPR = 9 * P + 1, NCH = 4 * 16 * CPR, NI = (NCH + 63) / 64, MAPD = TD == LE_TYPE_Q6_K ? 1 : 0;
    constexpr int K = 2048, NSB = 8, SEGT = K / 16, NT = 512;
    constexpr int XR = (LE_MOE_FAST_TOK * SEGT + NT - 1) / NT;
    constexpr int DCPS = TD == LE_TYPE_Q6_K ? 14 : 9, DSBB = TD == LE_TYPE_Q6_K ? 210 : 144;
    constexpr int DCPR = DCPS * PD + 1, DNCH = 16 * DCPR, DNI = (DNCH + 63) / 64, IMG = LE_MOE_IMG(256 * PD), IMGC = IMG / 16;
    constexpr int SLOTS = LE_MOE_DN_IMGS / NW;
    __shared__ MoeRoute R;
    __shared__ float sx[LE_MOE_FAST_TOK * LE_MOE_MAXK];
    __shared__ float red[NW][LE_MOE_FAST_TOK][64];
    __shared__ __attribute__((aligned(16))) float act[LE_MOE_FAST_TOK][32];
    __shared__ int mtok[NW][LE_MOE_FAST_TOK], mpair[NW][LE_MOE_FAST_TOK];
    __shared__ float mw[NW][LE_MOE_FAST_TOK];
    extern __shared__ uint4 smem[];
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6, n = lane & 15;
    uint4 *img = smem;                                         /* phase 1: [n_tok][image] */
    uint4 *stg = smem + LE_MOE_FAST_TOK * LE_MOE_IMG(K) / 16; /* phase 1: [NW][NI*64] staging; routing keys first */
    uint4 *wb = stg + wave * NI * 64;
    const MoeLogits lgt = moe_route_load(a); /* first, so routing waits for these loads alone */
    /* every token's activations */
    const int nseg = a.n_tok * SEGT;
    float4 hv[XR][4];
#pragma unroll
    for (int r = 0; r < XR; r++) {
        const int e = min((int)threadIdx.x + NT * r, nseg - 1);
        mq_load_seg(a.h + (size_t)(e / SEGT) * K, e % SEGT, hv[r]);
    }
    moe_route_par(a, R, (unsigned long long *)stg, sx, lgt);
    const int ngu = (a.ff >> 5) * R.U, ntile = a.hidden >> 4;
    const int b = blockIdx.x, G = gridDim.x;
    /* phase 2: row tile tb of the down projection, by H blocks that split its expert groups
     * (groups z = hh mod H); with H = 2 both add into the output that phase 1 zeroed, so every
     * element is 0 + a + b in either order: the same bits */
    const int H = G >= 2 * ntile ? 2 : 1, tb = b % ntile, hh = b / ntile;
    if (b == 0)
        for (int i = threadIdx.x; i < a.n_tok * a.k; i += blockDim.x) {
            if (a.idx_out) a.idx_out[i] = R.topi[i];
            if (a.w_out) a.w_out[i] = R.topw[i];
        }
    const size_t drb = (size_t)PD * DSBB;
    int roff[DNI];
#pragma unroll
    for (int i = 0; i < DNI; i++) {
        const int c = min(64 * i + lane, DNCH - 1), col = c % DCPR, cc = col == DCPS * PD ? 0 : col;
        roff[i] = (16 * tb + c / DCPR) * (int)drb + (TD == LE_TYPE_Q6_K ? (cc / 14) * 210 + q6_goff(cc % 14) : cc * 16);
    }
    uint4 R0[DNI];
    auto dissue = [&](int zz, uint4 (&r)[DNI]) {
        const u8 *W = moe_w(a.down, a.dptr, R.grp_e[zz], (size_t)a.hidden * drb);
#pragma unroll
        for (int i = 0; i < DNI; i++) r[i] = TD == LE_TYPE_Q6_K ? ldg16u(W + roff[i]) : ldg16(W + roff[i]);
    };
    /* ---- phase 1: gate/up items ---- */
    if (b < ngu) {
#pragma unroll
        for (int r = 0; r < XR; r++) { /* token images (the Q4_K slice map) */
            const int eg = (int)threadIdx.x + NT * r;
            if (r * NT >= nseg) break;
            const int t = min(eg, nseg - 1) / SEGT, el = min(eg, nseg - 1) % SEGT;
            uint4 *rec = img + t * (LE_MOE_IMG(K) / 16);
            float *dxp = (float *)(rec + NSB * 32), *fsv = dxp + NSB * 16;
            mq_quant_seg<0>(el, eg < nseg, hv[r], rec, dxp, fsv);
        }
    }
    const size_t rb = (size_t)NSB * 144;
    const MsLane L0 = ms_lane<0>(lane);
    le_v4i A[4];
#pragma unroll
    for (int q = 0; q < 4; q++) A[q] = (le_v4i){0, 0, 0, 0};
    /* the weights of item it (4 tiles: gate rows 32ux.., +16, up rows 32ux.., +16) into Rg; the
     * next item's loads are issued as soon as the current one is in LDS, so they arrive during its
     * MFMAs, SwiGLU and quantization (a load past the last item re-reads it: unconditional loads
     * keep the compiler's waits exact) */
    uint4 Rg[NI];
    auto gissue = [&](int it) {
        it = min(it, ngu - 1);
        const int ux = it % (a.ff >> 5), e = R.grp_e[it / (a.ff >> 5)];
        const u8 *Wg = moe_w(a.gate, a.gptr, e, (size_t)a.ff * rb), *Wu = moe_w(a.up, a.uptr, e, (size_t)a.ff * rb);
#pragma unroll
        for (int i = 0; i < NI; i++) {
            const int c = min(64 * i + lane, NCH - 1), ti = c / (16 * CPR), rem = c % (16 * CPR), col = rem % CPR;
            Rg[i] = ldg16((ti < 2 ? Wg : Wu) + (size_t)(32 * ux + 16 * (ti & 1) + rem / CPR) * rb + (size_t)wave * P * 144 +
                          (col == 9 * P ? 0 : col) * 16);
        }
    };
    if (b < ngu) gissue(b);
#pragma unroll 1
    for (int it = b; it < ngu; it += G) {
        const int ux = it % (a.ff >> 5), z = it / (a.ff >> 5);
        const int e = R.grp_e[z];
        const int nmem = __popcll(R.mask[e]);
        if (threadIdx.x < nmem) {
            int t, pair;
            float w;
            moe_member(a, R, e, threadIdx.x, t, pair, w);
            mtok[0][threadIdx.x] = t;
            mpair[0][threadIdx.x] = pair;
        }
        le_lds_barrier(); /* the previous item's readers of wb / act are done; images and members ready */
#pragma unroll
        for (int i = 0; i < NI; i++) wb[64 * i + lane] = Rg[i];
        gissue(it + G);
#pragma unroll 1
        for (int i = 0; i < nmem; i++) {
            const uint4 *rec = img + mtok[0][i] * (LE_MOE_IMG(K) / 16);
            const float *dxp = (const float *)(rec + NSB * 32), *fsv = dxp + NSB * 16;
            float y[4] = {0.f, 0.f, 0.f, 0.f};
            const int sb = wave;
            ms_load_a(rec + sb * 32, L0, A);
            ms_sb_q4k_n<4>(wb + n * CPR, 16 * CPR, A, dxp + sb * 16, fsv + sb * 8, L0, y);
#pragma unroll
            for (int ti = 0; ti < 4; ti++) {
                float v = y[ti];
                v = row4_sum(v);
                if (lane < 16) red[wave][i][16 * ti + lane] = v;
            }
        }
        le_lds_barrier();
        if (threadIdx.x < 32 * LE_MOE_FAST_TOK) {
            const int i = threadIdx.x >> 5, r = threadIdx.x & 31;
            if (i < nmem) {
                float g = 0.f, u = 0.f;
#pragma unroll
                for (int w = 0; w < NW; w++) {
                    g += red[w][i][r];
                    u += red[w][i][32 + r];
                }
                act[i][r] = g / (1.0f + __expf(-g)) * u;
            }
        }
        le_lds_barrier();
        if (wave == 0 && lane < 2 * LE_MOE_FAST_TOK) {
            const int i = lane >> 1, c = lane & 1;
            const bool ok = i < nmem;
            const float4 *av = (const float4 *)&act[ok ? i : 0][16 * c];
            float4 v4[4];
#pragma unroll
            for (int q = 0; q < 4; q++) v4[q] = av[q];
            uint4 *rec = (uint4 *)(a.ws + (size_t)mpair[0][ok ? i : 0] * IMG);
            float *dxp = (float *)(rec + PD * 32), *fsv = dxp + PD * 16;
            mq_quant_seg<MAPD, true>(2 * ux + c, ok, v4, rec, dxp, fsv); /* read by other blocks after the barrier */
        }
    }
    if (H == 2 && b < ntile) /* device-coherent, ordered before the other half's adds by the barrier */
        for (int i = threadIdx.x; i < a.n_tok * 16; i += blockDim.x)
            st_f<true>(a.out + (size_t)(i >> 4) * a.hidden + 16 * b + (i & 15), 0.f);
    /* ---- every down image written ---- */
    /* the first down group of this block's tile is issued after the arrival, so its loads are in
     * flight through the wait */
    const bool ok = moe_grid_barrier(a, G, [&]() {
        if (b < H * ntile && hh + H * wave < R.U) dissue(hh + H * wave, R0);
    });
    if (b >= H * ntile) return;
    /* ---- phase 2: row tile tb of the down projection, expert groups hh mod H ---- */
    uint4 *imgs = smem;                        /* LE_MOE_DN_IMGS images */
    uint4 *dwb = smem + LE_MOE_DN_IMGS * IMGC + wave * DNI * 64;
    for (int i = threadIdx.x; i < NW * LE_MOE_FAST_TOK * 16; i += blockDim.x) (&red[0][0][0])[i] = 0.f;
    const int npair = a.n_tok * a.k;
    const bool all_in = npair <= LE_MOE_DN_IMGS;
    if (all_in) {
        const int nc = npair * IMGC;
#pragma unroll 1
        for (int c0 = threadIdx.x; c0 < nc; c0 += 4 * 512) {
            uint4 v[4];
#pragma unroll
            for (int q = 0; q < 4; q++) v[q] = ldg16c(a.ws + 16 * (size_t)min(c0 + 512 * q, nc - 1));
#pragma unroll
            for (int q = 0; q < 4; q++)
                if (c0 + 512 * q < nc) imgs[c0 + 512 * q] = v[q];
        }
    }
    __syncthreads();
    const MsLane L = ms_lane<MAPD>(lane);
    /* the down map's dead A lanes must be zero: phase 1 filled the lanes live under the Q4_K map */
#pragma unroll
    for (int q = 0; q < 4; q++) A[q] = (le_v4i){0, 0, 0, 0};
    uint4 *wimg = imgs + wave * SLOTS * IMGC;
    float *redd = &red[0][0][0]; /* [NW][8][16] */
#pragma unroll 1
    for (int z = hh + H * wave; z < R.U; z += H * NW) {
        const int e = R.grp_e[z];
        const int nmem = __popcll(R.mask[e]);
        if (lane < nmem) {
            int t, pair;
            float w;
            moe_member(a, R, e, lane, t, pair, w);
            mtok[wave][lane] = t;
            mpair[wave][lane] = pair;
            mw[wave][lane] = w;
        }
#pragma unroll
        for (int i = 0; i < DNI; i++) dwb[64 * i + lane] = R0[i];
        if (z + H * NW < R.U) dissue(z + H * NW, R0);
#pragma unroll 1
        for (int i = 0; i < nmem; i++) {
            const uint4 *rec;
            if (all_in) {
                rec = imgs + mpair[wave][i] * IMGC;
            } else {
                uint4 *slot = wimg + (i % SLOTS) * IMGC;
                const int pr = mpair[wave][i];
                for (int o = lane; o < IMGC; o += 64) slot[o] = ldg16c(a.ws + (size_t)pr * IMG + 16 * o);
                rec = slot;
            }
            const float *dxp = (const float *)(rec + PD * 32), *fsv = dxp + PD * 16;
            float y = 0.f;
#pragma unroll
            for (int q = 0; q < PD; q++) {
                ms_load_a(rec + q * 32, L, A);
                if constexpr (TD == LE_TYPE_Q6_K)
                    y += ms_sb_q6k(dwb + n * DCPR + DCPS * q, A, dxp + q * 16, L);
                else
                    y += ms_sb_q4k(dwb + n * DCPR + DCPS * q, A, dxp + q * 16, fsv + q * 8, L);
            }
            y = row4_sum(y);
            if (lane < 16) redd[(wave * LE_MOE_FAST_TOK + mtok[wave][i]) * 16 + lane] += mw[wave][i] * y;
        }
    }
    __syncthreads();
    for (int i = threadIdx.x; i < a.n_tok * 16; i += blockDim.x) {
        const int t = i >> 4, r = i & 15;
        float acc = 0.f;
#pragma unroll
        for (int w = 0; w < NW; w++) acc += redd[(w * LE_MOE_FAST_TOK + t) * 16 + r];
        float *o = a.out + (size_t)t * a.hidden + 16 * tb + r;
        if (H == 2)
            __hip_atomic_fetch_add(o, ok ? acc : __builtin_nanf(""), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        else
            *o = ok ? acc : __builtin_nanf("");
    }
}

#define LE_MOE_FUS(TD, PD)                                                                                  \
    extern "C" __global__ void __launch_bounds__(512) le_moe_fus_12_##TD##_p##PD(MoeArgs a) { moe_fus_body<TD, PD>(a); }
LE_MOE_FUS(14, 1) LE_MOE_FUS(14, 2) LE_MOE_FUS(14, 3) LE_MOE_FUS(12, 1) LE_MOE_FUS(12, 2) LE_MOE_FUS(12, 3)


#define LE_MOE_GUM(TD, NW, P)                                                                               \
    extern "C" __global__ void __launch_bounds__(64 * NW) le_moe_gum_12_##TD##_w##NW##_p##P(MoeArgs a) {  \
        moe_gum_body<TD, NW, P>(a);                                                                        \
    }
#define LE_MOE_DNM(TD, NW, P)                                                                               \
    extern "C" __global__ void __launch_bounds__(64 * NW) le_moe_dnm_##TD##_w##NW##_p##P(MoeArgs a) {      \
        moe_dnm_body<TD, NW, P>(a);                                                                        \
    }
LE_MOE_GUM(14, 8, 1) LE_MOE_GUM(14, 4, 1) LE_MOE_GUM(14, 4, 3) LE_MOE_GUM(12, 8, 1) LE_MOE_GUM(12, 4, 1) LE_MOE_GUM(12, 4, 3)
LE_MOE_DNM(14, 8, 1) LE_MOE_DNM(14, 8, 2) LE_MOE_DNM(14, 8, 3) LE_MOE_DNM(12, 8, 1) LE_MOE_DNM(12, 8, 2) LE_MOE_DNM(12, 8, 3)

#define LE_MOE(TG, TD)                                                                                       \
    extern "C" __global__ void __launch_bounds__(256) le_moe_gu_##TG##_##TD##_g8(MoeArgs a) { moe_gu_body<TG, TD, 8>(a); } \
    extern "C" __global__ void __launch_bounds__(256) le_moe_gu_##TG##_##TD##_g1(MoeArgs a) { moe_gu_body<TG, TD, 1>(a); } \
    extern "C" __global__ void __launch_bounds__(1024) le_moe_guf_##TG##_##TD##_g8(MoeArgs a) { moe_gu_fast<TG, TD, 8>(a); } \
    extern "C" __global__ void __launch_bounds__(1024) le_moe_guf_##TG##_##TD##_g1(MoeArgs a) { moe_gu_fast<TG, TD, 1>(a); }
#define LE_MOE_DOWN(TD) \
    extern "C" __global__ void __launch_bounds__(256) le_moe_down_##TD(MoeArgs a) { moe_down_body<TD>(a); } \
    extern "C" __global__ void __launch_bounds__(512) le_moe_downf_##TD(MoeArgs a) { moe_down_fast<TD>(a); }
LE_MOE(12, 14) LE_MOE(12, 12) LE_MOE(14, 14) LE_MOE(8, 8) LE_MOE(16, 18) LE_MOE(16, 16) LE_MOE(18, 18)
LE_MOE_DOWN(8) LE_MOE_DOWN(12) LE_MOE_DOWN(14) LE_MOE_DOWN(16) LE_MOE_DOWN(18)
/* ===================== MoE prefill: routing and grouping for the grouped matmul =====================
 * For prefill-sized token counts (the reference's TMAX = 2048 per chunk, src/gpu/prefill.rs:6) the
 * layer runs as: le_moe_route_tok (top-k and weights per token) -> le_moe_group (pairs grouped by
 * expert, each expert's pairs in token order: the host grouping of src/gpu/prefill.rs:153-214 on
 * the device) -> grouped matmul gate and up (one launch) -> grouped matmul down on silu(gate) * up ->
 * le_moe_combine (weighted sum in selection order, src/cpu_ref.rs:242-259). */
struct MoePre {
    const float *logits;
    int *topi;     /* [n_tok * k] */
    float *topw;   /* [n_tok * k] */
    int *off;      /* [n_exp + 1] */
    int *in_idx;   /* [n_tok * k]: the token of each grouped pair */
    int *out_idx;  /* [n_tok * k]: the pair (t * k + s) of each grouped pair */
    int *idx_out;  /* optional copies of the selection */
    float *w_out;
    int n_tok, n_exp, k, pad;
};

/* Routing of one token by one wave: k rounds of a wave-wide max (ties keep the lower expert),
 * weights exp(v - top) / sum in selection order, as the decode kernels compute them. Lane s < k
 * ends with selection s's expert; the loads are split from the rounds so a wave can issue several
 * tokens' loads first. */
__device__ __forceinline__ void moe_route_load(const MoePre &a, int t, int lane, float (&vv)[MOE_LPASS]) {
    const int per = (a.n_exp + 63) >> 6;
#pragma unroll
    for (int j = 0; j < MOE_LPASS; j++) {
        const int e = lane * per + j;
        vv[j] = j < per && e < a.n_exp ? a.logits[(size_t)t * a.n_exp + e] : -INFINITY;
    }
}
__device__ __forceinline__ int moe_route_pick(const MoePre &a, int t, int lane, float (&vv)[MOE_LPASS]) {
    const int per = (a.n_exp + 63) >> 6;
    int my_e = 0;
    float my_v = 0.f;
    for (int r = 0; r < a.k; r++) {
        float bv = vv[0];
        int bj = 0;
#pragma unroll
        for (int j = 1; j < MOE_LPASS; j++) {
            const bool gt = vv[j] > bv;
            bv = gt ? vv[j] : bv;
            bj = gt ? j : bj;
        }
        const float mx = wave_max(bv);
        const int wl = __ffsll((long long)__ballot(bv == mx)) - 1;
        const int wj = __builtin_amdgcn_readlane(bj, wl);
#pragma unroll
        for (int j = 0; j < MOE_LPASS; j++) vv[j] = lane == wl && j == wj ? -INFINITY : vv[j];
        my_e = lane == r ? wl * per + wj : my_e;
        my_v = lane == r ? mx : my_v;
    }
    const float top = __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, my_v), 0));
    const float ex = lane < a.k ? expf(my_v - top) : 0.f;
    float tot = 0.f;
    for (int r = 0; r < a.k; r++) tot += __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, ex), r));
    if (lane < a.k) {
        const int i = t * a.k + lane;
        a.topi[i] = my_e;
        a.topw[i] = ex / tot;
        if (a.idx_out) a.idx_out[i] = my_e;
        if (a.w_out) a.w_out[i] = ex / tot;
    }
    return my_e;
}

/* One wave per token. */
extern "C" __global__ void __launch_bounds__(512) le_moe_route_tok(MoePre a) {
    const int lane = threadIdx.x & 63, t = blockIdx.x * 8 + (threadIdx.x >> 6);
    if (t >= a.n_tok) return; /* uniform over the wave */
    float vv[MOE_LPASS];
    moe_route_load(a, t, lane, vv);
    (void)moe_route_pick(a, t, lane, vv);
}

/* Routing and grouping in one block of 16 waves for up to 64 tokens and 1024 pairs: wave w routes
 * tokens w, w + 16, ... (all their logits loaded first), then thread p takes pair p: its rank
 * among the pairs of its expert is the count of that expert in lower waves (per-wave histograms
 * in LDS) plus the lower lanes of its own wave holding the same expert, so each expert's pairs
 * come out in pair order, as le_moe_group orders them. */
extern "C" __global__ void __launch_bounds__(1024) le_moe_route_group(MoePre a) {
    __shared__ int hist[16][64 * MOE_LPASS];
    __shared__ int sel[1024], base_e[64 * MOE_LPASS];
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int ne = a.n_exp, np = a.n_tok * a.k;
    for (int i = tid; i < 16 * 64 * MOE_LPASS; i += 1024) (&hist[0][0])[i] = 0;
    {
        float vv[4][MOE_LPASS];
#pragma unroll
        for (int i = 0; i < 4; i++)
            if (wave + 16 * i < a.n_tok) moe_route_load(a, wave + 16 * i, lane, vv[i]);
#pragma unroll
        for (int i = 0; i < 4; i++) {
            const int t = wave + 16 * i;
            if (t < a.n_tok) {
                const int e = moe_route_pick(a, t, lane, vv[i]);
                if (lane < a.k) sel[t * a.k + lane] = e;
            }
        }
    }
    __syncthreads();
    const int e = tid < np ? sel[tid] : -1;
    int below = 0; /* lower lanes of this wave on the same expert */
    for (int j = 0; j < 64; j++) below += j < lane && __builtin_amdgcn_readlane(e, j) == e ? 1 : 0;
    if (e >= 0) atomicAdd(&hist[wave][e], 1);
    __syncthreads();
    if (wave == 0) { /* per-expert totals, exclusive scan over the experts, 4 per lane */
        int c[MOE_LPASS], s = 0;
#pragma unroll
        for (int j = 0; j < MOE_LPASS; j++) {
            const int x = lane * MOE_LPASS + j;
            c[j] = 0;
            if (x < ne)
                for (int w = 0; w < 16; w++) c[j] += hist[w][x];
            s += c[j];
        }
        int incl = s;
#pragma unroll
        for (int o = 1; o < 64; o <<= 1) {
            const int y = __shfl_up(incl, o);
            if (lane >= o) incl += y;
        }
        int run = incl - s;
#pragma unroll
        for (int j = 0; j < MOE_LPASS; j++) {
            const int x = lane * MOE_LPASS + j;
            if (x < ne) {
                base_e[x] = run;
                a.off[x] = run;
            }
            run += c[j];
        }
        if (lane == 63) a.off[ne] = incl;
    }
    __syncthreads();
    if (e >= 0) {
        int q = base_e[e] + below;
        for (int w = 0; w < wave; w++) q += hist[w][e];
        a.in_idx[q] = tid / a.k;
        a.out_idx[q] = tid;
    }
}

/* One block per expert e: its offset (the number of pairs routed to lower experts) and its own
 * pairs in pair (= token) order, so the grouping is deterministic. A round covers 256 J pairs
 * (J = ceil(pairs / 256), at most 64), 64 J per wave, the lane reading pair 64 j + lane of its
 * wave's run at step j (coalesced), so that pair order is (wave, j, lane) order and a match's rank
 * is a ballot's popcount below its lane. With more than 16384 pairs the offset takes a pass of its
 * own first. The block for the last expert also writes off[n_exp]. */
extern "C" __global__ void __launch_bounds__(256) le_moe_group(MoePre a) {
    __shared__ int wsum[4], wcnt[4];
    const int e = blockIdx.x, lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const int npair = a.n_tok * a.k;
    const int J = min((npair + 255) >> 8, 64), R = 256 * J;
    const bool one = npair <= R;
    int low = 0;
    if (!one)
        for (int p = threadIdx.x; p < npair; p += 256) low += a.topi[p] < e;
    const unsigned long long lt = (1ull << lane) - 1ull;
    int off = 0, base = 0;
    for (int r0 = 0; r0 < npair; r0 += R) {
        const int pw = r0 + 64 * J * wave + lane;
        unsigned long long m = 0;
#pragma unroll 16
        for (int j = 0; j < J; j++) {
            const int p = pw + 64 * j;
            const int v = p < npair ? a.topi[p] : 0x7fffffff;
            if (one) low += v < e;
            m |= (unsigned long long)(v == e) << j;
        }
        int c = __popcll(m);
        for (int o = 32; o > 0; o >>= 1) c += __shfl_xor(c, o);
        if (r0 == 0)
            for (int o = 32; o > 0; o >>= 1) low += __shfl_xor(low, o);
        if (lane == 0) {
            wcnt[wave] = c;
            if (r0 == 0) wsum[wave] = low;
        }
        __syncthreads();
        if (r0 == 0) {
            off = wsum[0] + wsum[1] + wsum[2] + wsum[3];
            if (threadIdx.x == 0) a.off[e] = off;
        }
        int r = off + base;
        for (int w = 0; w < wave; w++) r += wcnt[w];
        for (int j = 0; j < J; j++) {
            const bool hit = (m >> j) & 1ull;
            const unsigned long long bj = __ballot(hit);
            if (bj == 0ull) continue; /* uniform */
            if (hit) {
                const int p = pw + 64 * j, q = r + __popcll(bj & lt);
                a.in_idx[q] = p / a.k;
                a.out_idx[q] = p;
            }
            r += __popcll(bj);
        }
        base += wcnt[0] + wcnt[1] + wcnt[2] + wcnt[3];
        __syncthreads();
    }
    if (e == a.n_exp - 1 && threadIdx.x == 0) a.off[a.n_exp] = off + base;
}

/* out[t][c] = sum over s < k of w[t k + s] * d[t k + s][c], added in selection order. Block
 * (t, b) covers columns [1024 b, 1024 b + 1024) of token t, four per thread (as a float4 when the
 * rows are 16-byte aligned). */
extern "C" __global__ void __launch_bounds__(256) le_moe_combine(const float *d, const float *w, float *out, int n_tok, int k,
                                                                 int hidden) {
    const int nb = (hidden + 1023) >> 10;
    const int t = (int)blockIdx.x / nb, c0 = ((int)blockIdx.x - t * nb) * 1024 + 4 * (int)threadIdx.x;
    if (t >= n_tok || c0 >= hidden) return;
    const float *wt = w + (size_t)t * k;
    const float *dt = d + (size_t)t * k * hidden;
    float *o = out + (size_t)t * hidden;
    if ((hidden & 3) == 0 && (((size_t)d | (size_t)out) & 15) == 0) {
        float4 acc = make_float4(0.f, 0.f, 0.f, 0.f);
        for (int s = 0; s < k; s++) {
            const float ws = wt[s];
            const float4 v = *(const float4 *)(dt + (size_t)s * hidden + c0);
            acc.x += ws * v.x;
            acc.y += ws * v.y;
            acc.z += ws * v.z;
            acc.w += ws * v.w;
        }
        *(float4 *)(o + c0) = acc;
    } else {
        for (int c = c0; c < c0 + 4 && c < hidden; c++) {
            float acc = 0.f;
            for (int s = 0; s < k; s++) acc += wt[s] * dt[(size_t)s * hidden + c];
            o[c] = acc;
        }
    }
}
#endif /* LE_PART_MOE */
