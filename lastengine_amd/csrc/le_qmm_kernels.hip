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

/* ===================================================================================== */
/* Bit-exact dequantization. One thread per 32-value unit; the arithmetic follows           */
/* src/quant.rs operation by operation with FP contraction disabled.                         */
/* ===================================================================================== */

/* src/quant.rs:37-49, in integer arithmetic (also reproduces NaN payloads bit for bit). */
__device__ float f16_exact(u32 h) {
    const u32 s = (h >> 15) & 1u, e = (h >> 10) & 0x1fu, m = h & 0x3ffu;
    u32 bits;
    if (e == 0) {
        if (m == 0) {
            bits = s << 31;
        } else {
            const int lz = __builtin_clz(m) - 21; /* shifts until bit 10 is set */
            bits = (s << 31) | ((u32)(113 - lz) << 23) | (((m << lz) & 0x3ffu) << 13);
        }
    } else if (e == 31) {
        bits = (s << 31) | (0xffu << 23) | (m << 13);
    } else {
        bits = (s << 31) | ((e + 112) << 23) | (m << 13);
    }
    return __builtin_bit_cast(float, bits);
}

__device__ __forceinline__ u32 ksign_dev(u32 i) { return (i & 0x7fu) | ((__builtin_popcount(i & 0x7fu) & 1u) << 7); }

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
#define LE_DEQ(TY, NAME)                                                                                   \
    extern "C" __global__ void __launch_bounds__(256) NAME(const u8 *w, float *out, int rows, int cols,     \
                                                          unsigned long long row_bytes) {                  \
        dequant_rows<TY>(w, out, rows, cols, (size_t)row_bytes);                                           \
    }
LE_DEQ(LE_TYPE_Q8_0, le_dequant_8)
LE_DEQ(LE_TYPE_Q4_K, le_dequant_12)
LE_DEQ(LE_TYPE_Q6_K, le_dequant_14)
LE_DEQ(LE_TYPE_IQ2_XXS, le_dequant_16)
LE_DEQ(LE_TYPE_IQ3_XXS, le_dequant_18)
#endif

/* ===================================================================================== */
/* Dequant-fused matvec / small-M matmul.                                                    */
/* ===================================================================================== */

/* Launch contract (checked by the host):
 *   cols % 256 == 0; G divides cols/256; x rows 16-byte aligned; blockDim = 256 (4 waves);
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
    int rows, cols, ntok, pad;
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
        const u32 *src = TY == LE_TYPE_IQ2_XXS ? le_iq2xxs_grid : le_iq3xxs_grid;
        for (int i = threadIdx.x; i < Fmt<TY>::GRID_WORDS; i += blockDim.x) tab[LE_TAB_GRID + i] = src[i];
    }
}

template <int TY, int G, int T>
__device__ __forceinline__ void mv_body(const MvArgs &a) {
    using F = Fmt<TY>;
    extern __shared__ uint4 smem[];
    const int K = a.cols, nsb = K >> 8, ng = K >> 3, nu = K >> 5;
    const int slot = blockIdx.y, t0 = blockIdx.z * T;
    const int nt = min(T, a.ntok - t0);
    const u8 *W = a.ptrs ? a.ptrs[slot] : a.w0 + (size_t)slot * a.w_slot_bytes;
    const size_t rb = (size_t)nsb * F::SB;

    /* LDS carve-up: T token images, then the IQ tables */
    XTok xt[T];
    {
        uint4 *xq = smem;
        float *fs = (float *)(smem + T * ng);
        float *dx = fs + T * ng;
#pragma unroll
        for (int t = 0; t < T; t++) {
            xt[t].xq = xq + t * ng;
            xt[t].fs = fs + t * ng;
            xt[t].dx = dx + t * nu;
            if (t < nt)
                le_quant_x_lds(a.x + a.x_slot * slot + a.x_tok * (t0 + t), K, xq + t * ng, fs + t * ng, dx + t * nu);
        }
    }
    u32 *tab = (u32 *)((float *)(smem + T * ng) + T * ng + T * nu);
    load_tables<TY>(tab);
    __syncthreads();

    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    constexpr int RPW = 8 / G; /* rows per wave per step */
    const int li = lane & 7, g = (lane >> 3) % G, rsub = lane / (8 * G);
    const int S = nsb / G; /* super-blocks per lane per row */
    const int nrb = (a.rows + RPW - 1) / RPW;
    constexpr int U = 4;
    for (int rbk = blockIdx.x * 4 + wave; rbk < nrb; rbk += gridDim.x * 4) {
        const int row = rbk * RPW + rsub;
        const bool rok = row < a.rows;
        const u8 *wr = W + (size_t)(rok ? row : a.rows - 1) * rb;
        float acc[T];
#pragma unroll
        for (int t = 0; t < T; t++) acc[t] = 0.f;
        for (int s0 = 0; s0 < S; s0 += U) {
            typename F::Raw raw[U];
#pragma unroll
            for (int u = 0; u < U; u++) {
                const int s = min(s0 + u, S - 1);
                raw[u] = F::load(wr + (size_t)(g + G * s) * F::SB, li);
            }
#pragma unroll
            for (int u = 0; u < U; u++) {
                if (s0 + u < S) {
                    Dec d;
                    F::decode(raw[u], li, g + G * (s0 + u), tab, d);
#pragma unroll
                    for (int t = 0; t < T; t++) {
                        if (t < nt) {
                            float c = 0.f;
#pragma unroll
                            for (int k = 0; k < 4; k++) c += group_dot<F::HAS_MU>(d, k, xt[t]);
                            acc[t] += c;
                        }
                    }
                }
            }
        }
#pragma unroll
        for (int t = 0; t < T; t++) {
#pragma unroll
            for (int off = 1; off < 8 * G; off <<= 1) acc[t] += __shfl_xor(acc[t], off);
        }
        if (rok && (lane & (8 * G - 1)) == 0) {
#pragma unroll
            for (int t = 0; t < T; t++)
                if (t < nt) a.y[a.y_slot * slot + a.y_tok * (t0 + t) + row] = acc[t];
        }
    }
}

#define LE_MV(TY, G, T)                                                                                    \
    extern "C" __global__ void __launch_bounds__(256) le_mv_##TY##_g##G##_t##T(MvArgs a) { mv_body<TY, G, T>(a); }
#define LE_MV_G(TY, G) LE_MV(TY, G, 1) LE_MV(TY, G, 2) LE_MV(TY, G, 4) LE_MV(TY, G, 8)
#define LE_MV_ALL(TY) LE_MV_G(TY, 1) LE_MV_G(TY, 2) LE_MV_G(TY, 4) LE_MV_G(TY, 8)
/* Each code object carries the kernels of one part (the build compiles this file once per part,
 * in parallel): LE_PART_DEQ, or LE_PART_MV=<type id>. */
#if defined(LE_PART_MV)
LE_MV_ALL(LE_PART_MV)
#endif
