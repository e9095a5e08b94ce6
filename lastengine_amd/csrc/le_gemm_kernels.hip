/* Small-M quantized GEMM on the matrix cores (gfx950): Y[t, r] = W[r, :] . X[t, :].
 *
 * Replaces the int8 MMA kernels mmq*_<ty> behind DenseGpu::bmm (src/cuda/kernels.cu:965-1223,
 * src/gpu/dense.rs:181-199); CPU twin cpu_ref::matmat (src/cpu_ref.rs:266-276).
 *
 * Numerics. Every supported format is, per super-block of 256 values and row r,
 *     w_k = d_r * c_k  -  dmin_r * m_{j(k)}
 * with small integer codes c_k (Q4_K: sc_j * q_k <= 945; the sub-block of value k is j(k)) and
 * integer offsets m_j. Integers below 2048 are exact in fp16, so the weight operand is the fp16
 * code c_k, built in LDS from the raw GGUF bytes. The activations are split x = xh + xl into two
 * fp16 halves (xh = fp16(x), xl = fp16(x - xh), 22 significant bits). v_mfma_f32_16x16x32_f16
 * multiplies both halves by the codes with fp32 accumulation, so per super-block
 *     D1[t, r] = sum_k c_k (xh_k + xl_k)          D2[t, r] = sum_j m_j S_j(t)
 * (S_j = fp32 sum of x over sub-block j, also split into fp16 halves for a second MFMA) and
 *     Y[t, r] += d_r * D1 - dmin_r * D2
 * in fp32. The only roundings are the activation split (|x - xh - xl| <= 2^-22 |x|) and fp32
 * accumulation; activations must stay inside the fp16 range (|x| < 65504).
 *
 * Tiling. A block of four waves computes 32*TM tokens x 128*TN rows; every wave owns 32*TN
 * rows for all the block's tokens, as TM x TN tiles of v_mfma_f32_32x32x16_f16 (this shape runs
 * near the f16 peak with one wave per SIMD). K advances one super-block per step. Staging is
 * coalesced: consecutive lanes load consecutive 16-byte chunks of a weight row's super-block and
 * consecutive float4s of a token's 256 activations, into registers one step ahead, then into LDS.
 * The weights stay raw in LDS (row stride 152 bytes: the 32-row fragment reads are free of bank
 * conflicts); each lane unpacks its own B fragment from 8 quant bytes just before the MFMAs, the
 * low nibbles giving one K slice and the high nibbles the slice 32 values further on. Blocks that
 * share weight rows (same row tile, different token tiles) get the same blockIdx % 8, so they run
 * on one XCD and share its L2. Within every aligned group of four K positions both operands are
 * stored in the order 0, 2, 1, 3 (what the nibble unpacking produces); the dot product does not
 * depend on the order.
 */
#include "le_qmm_device.h"

typedef _Float16 le_h2 __attribute__((ext_vector_type(2)));
typedef _Float16 le_v8h __attribute__((ext_vector_type(8)));
typedef float le_v4f __attribute__((ext_vector_type(4)));

struct GmArgs {
    const u8 *w;
    const float *x;
    float *y;
    int rows, cols, m;
};


/* Diagnostic builds (-DLE_TRACE) accumulate per-phase s_memrealtime deltas in registers and write
 * them per block to le_gm_trace[block * 8 + i]; compiled out otherwise. */
#if defined(LE_TRACE)
__device__ unsigned long long le_gm_trace[1 << 16];
#define GM_T(v) unsigned long long v = __builtin_amdgcn_s_memrealtime()
#define GM_ADD(i, a, b) tr[i] += (b) - (a)
#else
#define GM_T(v) do { } while (0)
#define GM_ADD(i, a, b) do { } while (0)
#endif

__device__ __forceinline__ void gm_barrier() {
    __asm__ volatile("" ::: "memory");
    __builtin_amdgcn_s_waitcnt(0xC07F); /* LDS only: the prefetch loads stay in flight */
    __builtin_amdgcn_s_barrier();
    __asm__ volatile("" ::: "memory");
}

__device__ __forceinline__ le_h2 as_h2(u32 v) { return __builtin_bit_cast(le_h2, v); }
__device__ __forceinline__ u32 as_u32(le_h2 v) { return __builtin_bit_cast(u32, v); }

/* fp32 -> (hi, lo) fp16 halves of two values, packed. */
__device__ __forceinline__ void gm_split2(float a, float b, u32 &hi, u32 &lo) {
    const _Float16 ha = (_Float16)a, hb = (_Float16)b;
    const le_h2 h = {ha, hb};
    const le_h2 l = {(_Float16)(a - (float)ha), (_Float16)(b - (float)hb)};
    hi = as_u32(h);
    lo = as_u32(l);
}

/* Q4_K: 8 quant bytes (values l..l+7 of a 64-value group in the low nibbles, l+32.. in the high
 * nibbles) -> two B fragments of fp16 codes q*sc in the order 0,2,1,3 within each four. The
 * nibble at bits 0-3 (4-7) of a 16-bit half becomes fp16 1024+q (1024+16q) by the exponent
 * trick; one packed fma with (sc, -1024 sc) (or (sc/16, -64 sc)) gives q*sc exactly. */
__device__ __forceinline__ void gm_q4k_frag(uint2 w, uint4 k, le_v8h &lo, le_v8h &hi) {
    const le_h2 slo = as_h2(k.x), clo = as_h2(k.y), shi = as_h2(k.z), chi = as_h2(k.w);
    u32 l[4], h[4];
    const u32 ws[2] = {w.x, w.y};
#pragma unroll
    for (int i = 0; i < 2; i++) {
        const u32 a = ws[i], a8 = a >> 8;
        l[2 * i] = as_u32(__builtin_elementwise_fma(as_h2((a & 0x000F000Fu) | 0x64006400u), slo, clo));
        l[2 * i + 1] = as_u32(__builtin_elementwise_fma(as_h2((a8 & 0x000F000Fu) | 0x64006400u), slo, clo));
        h[2 * i] = as_u32(__builtin_elementwise_fma(as_h2((a & 0x00F000F0u) | 0x64006400u), shi, chi));
        h[2 * i + 1] = as_u32(__builtin_elementwise_fma(as_h2((a8 & 0x00F000F0u) | 0x64006400u), shi, chi));
    }
    lo = __builtin_bit_cast(le_v8h, make_uint4(l[0], l[1], l[2], l[3]));
    hi = __builtin_bit_cast(le_v8h, make_uint4(h[0], h[1], h[2], h[3]));
}

#define GM_WS 152 /* LDS bytes per raw weight row: 144 + 8 (conflict-free 8-byte fragment reads) */
#define GM_AS 264 /* fp16 per activation row: 256 + 8 */

template <int TM, int TN>
__device__ __forceinline__ void gm_q4k_body(const GmArgs &a) {
    constexpr int BM = 32 * TM, BN = 128 * TN, NWC = BN * 9 / 256 + (BN * 9 % 256 ? 1 : 0), NXC = BM / 4;
    typedef float v16f __attribute__((ext_vector_type(16)));
    extern __shared__ uint4 smem[];
    u8 *Wr = (u8 *)smem;                          /* [BN][GM_WS] raw super-block bytes */
    uint4 *Wk = (uint4 *)(Wr + BN * GM_WS);       /* [BN][4] fragment constants per 64-value group */
    uint4 *Bm = Wk + BN * 4;                      /* [BN] offsets m_0..7 (fp16) */
    float2 *Dd = (float2 *)(Bm + BN);             /* [BN] (d, dmin) */
    _Float16 *Ah = (_Float16 *)(Dd + BN);         /* [BM][GM_AS] activation high halves */
    _Float16 *Al = Ah + BM * GM_AS;               /* [BM][GM_AS] low halves */
    float *Sf = (float *)(Al + BM * GM_AS);       /* [BM][8] sub-block sums */

    const int K = a.cols, nsb = K >> 8, M = a.m;
    const int NT = (a.rows + BN - 1) / BN, MT = (M + BM - 1) / BM;
    const int id = blockIdx.x, j = id >> 3;
    const int mt = j % MT, nt = (j / MT) * 8 + (id & 7);
    if (nt >= NT) return; /* uniform over the block */
    const int nb = nt * BN, mb = mt * BM;
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const size_t rb = (size_t)nsb * 144;

    /* staging: weight chunk c = tid + 256 i is (row c/9, 16-byte column c%9) of the super-block;
     * activation float4 f = tid + 256 i is (token f/64, column f%64) */
    uint4 wr[NWC];
    float4 xr[NXC];
    auto issue = [&](int sb) {
#pragma unroll
        for (int i = 0; i < NWC; i++) {
            const int c = min(tid + 256 * i, BN * 9 - 1), row = c / 9, col = c - 9 * row;
            wr[i] = ldg16(a.w + (size_t)min(nb + row, a.rows - 1) * rb + (size_t)sb * 144 + 16 * col);
        }
#pragma unroll
        for (int i = 0; i < NXC; i++) {
            const int t = (tid >> 6) + 4 * i;
            xr[i] = *(const LE_GLOBAL float4 *)(a.x + (size_t)min(mb + t, M - 1) * K + 256 * sb + 4 * lane);
        }
    };
    auto stage = [&]() {
#pragma unroll
        for (int i = 0; i < NWC; i++) {
            const int c = tid + 256 * i;
            if (NWC * 256 > BN * 9 && c >= BN * 9) break;
            const int row_ = c / 9;
            uint2 *d = (uint2 *)(Wr + row_ * GM_WS + 16 * (c - 9 * row_));
            d[0] = make_uint2(wr[i].x, wr[i].y);
            d[1] = make_uint2(wr[i].z, wr[i].w);
            if (c % 9 == 0) { /* the row's header: fragment constants, offsets, (d, dmin) */
                const int row = c / 9;
                const u32 sy = wr[i].y, sz = wr[i].z, sw = wr[i].w;
                const u32 sc0 = sy & 0x3F3F3F3Fu, sc1 = (sw & 0x0F0F0F0Fu) | ((sy >> 2) & 0x30303030u);
                const u32 m0 = sz & 0x3F3F3F3Fu, m1 = ((sw >> 4) & 0x0F0F0F0Fu) | ((sz >> 2) & 0x30303030u);
#pragma unroll
                for (int g = 0; g < 4; g++) {
                    const u32 scw = (g < 2 ? sc0 : sc1) >> (16 * (g & 1));
                    const float sl = (float)(scw & 255u), sh = (float)((scw >> 8) & 255u);
                    const le_h2 v0 = {(_Float16)sl, (_Float16)sl}, v1 = {(_Float16)(-1024.f * sl), (_Float16)(-1024.f * sl)};
                    const le_h2 v2 = {(_Float16)(0.0625f * sh), (_Float16)(0.0625f * sh)}, v3 = {(_Float16)(-64.f * sh), (_Float16)(-64.f * sh)};
                    Wk[row * 4 + g] = make_uint4(as_u32(v0), as_u32(v1), as_u32(v2), as_u32(v3));
                }
                u32 mw[4];
#pragma unroll
                for (int q = 0; q < 4; q++) {
                    const u32 mm = (q < 2 ? m0 : m1) >> (16 * (q & 1));
                    const le_h2 v = {(_Float16)(float)(mm & 255u), (_Float16)(float)((mm >> 8) & 255u)};
                    mw[q] = as_u32(v);
                }
                Bm[row] = make_uint4(mw[0], mw[1], mw[2], mw[3]);
                Dd[row] = make_float2(h2f(wr[i].x & 0xFFFFu), h2f(wr[i].x >> 16));
            }
        }
#pragma unroll
        for (int i = 0; i < NXC; i++) {
            const int f = tid + 256 * i, t = f >> 6, c4 = f & 63;
            float4 v = xr[i];
            if (mb + t >= M) v = make_float4(0.f, 0.f, 0.f, 0.f);
            u32 h0, h1, l0, l1;
            gm_split2(v.x, v.z, h0, l0);
            gm_split2(v.y, v.w, h1, l1);
            *(uint2 *)(Ah + t * GM_AS + 4 * c4) = make_uint2(h0, h1);
            *(uint2 *)(Al + t * GM_AS + 4 * c4) = make_uint2(l0, l1);
            /* sub-block sum over the 8 lanes holding its 32 values */
            const float sum = group_sum<8>((v.x + v.y) + (v.z + v.w)); /* DPP, no LDS round trips */
            if ((c4 & 7) == 0) Sf[t * 8 + (c4 >> 3)] = sum;
        }
    };

    v16f acc[TM][TN], d1[TM][TN];
#pragma unroll
    for (int i = 0; i < TM; i++)
#pragma unroll
        for (int k = 0; k < TN; k++) acc[i][k] = d1[i][k] = (v16f){};

    const int r32 = lane & 31, hs = lane >> 5;
    int brow[TN];
#pragma unroll
    for (int k = 0; k < TN; k++) brow[k] = 32 * (wave * TN + k) + r32;
#if defined(LE_TRACE)
    unsigned long long tr[8] = {};
#endif
    GM_T(t_start);
    issue(0);
    for (int sb = 0; sb < nsb; sb++) {
        GM_T(ta);
        gm_barrier(); /* the previous super-block's operand reads are done */
        GM_T(tb);
        stage();
        GM_T(tc);
        if (sb + 1 < nsb) issue(sb + 1);
        GM_T(td);
        gm_barrier();
        GM_T(te);
        GM_ADD(0, ta, tb);
        GM_ADD(1, tb, tc);
        GM_ADD(2, tc, td);
        GM_ADD(3, td, te);
#pragma unroll 1
        for (int g = 0; g < 4; g++) {
            uint4 kc[TN];
#pragma unroll
            for (int k = 0; k < TN; k++) kc[k] = Wk[brow[k] * 4 + g];
#pragma unroll
            for (int c = 0; c < 2; c++) {
                /* K slice: values 64g + 16c + 8hs .. +8 (low nibbles) and 64g + 32 + ... (high) */
                le_v8h blo[TN], bhi[TN];
#pragma unroll
                for (int k = 0; k < TN; k++) {
                    const uint2 w = *(const uint2 *)(Wr + brow[k] * GM_WS + 16 + 32 * g + 16 * c + 8 * hs);
                    gm_q4k_frag(w, kc[k], blo[k], bhi[k]);
                }
#pragma unroll
                for (int half = 0; half < 2; half++) {
                    const int ko = 64 * g + 32 * half + 16 * c + 8 * hs;
                    le_v8h ah[TM], al[TM];
#pragma unroll
                    for (int i = 0; i < TM; i++) {
                        ah[i] = __builtin_bit_cast(le_v8h, *(const uint4 *)(Ah + (32 * i + r32) * GM_AS + ko));
                        al[i] = __builtin_bit_cast(le_v8h, *(const uint4 *)(Al + (32 * i + r32) * GM_AS + ko));
                    }
#pragma unroll
                    for (int i = 0; i < TM; i++)
#pragma unroll
                        for (int k = 0; k < TN; k++)
                            d1[i][k] = __builtin_amdgcn_mfma_f32_32x32x16_f16(ah[i], half ? bhi[k] : blo[k], d1[i][k], 0, 0, 0);
#pragma unroll
                    for (int i = 0; i < TM; i++)
#pragma unroll
                        for (int k = 0; k < TN; k++)
                            d1[i][k] = __builtin_amdgcn_mfma_f32_32x32x16_f16(al[i], half ? bhi[k] : blo[k], d1[i][k], 0, 0, 0);
                }
            }
        }
        /* super-block epilogue: Y += d * D1 - dmin * D2 with D2 = sum_j m_j S_j from one more MFMA
         * (K slice 0 carries the high halves of S_0..7, slice 1 the low halves, both against m) */
        le_v8h a2[TM];
#pragma unroll
        for (int i = 0; i < TM; i++) {
            const float4 s0 = *(const float4 *)(Sf + (32 * i + r32) * 8), s1 = *(const float4 *)(Sf + (32 * i + r32) * 8 + 4);
            const float sv[8] = {s0.x, s0.y, s0.z, s0.w, s1.x, s1.y, s1.z, s1.w};
            u32 pw[4];
#pragma unroll
            for (int q = 0; q < 4; q++) {
                u32 hh, ll;
                gm_split2(sv[2 * q], sv[2 * q + 1], hh, ll);
                pw[q] = hs ? ll : hh;
            }
            a2[i] = __builtin_bit_cast(le_v8h, make_uint4(pw[0], pw[1], pw[2], pw[3]));
        }
#pragma unroll
        for (int k = 0; k < TN; k++) {
            const le_v8h b2 = __builtin_bit_cast(le_v8h, Bm[brow[k]]);
            const float2 dm = Dd[brow[k]];
#pragma unroll
            for (int i = 0; i < TM; i++) {
                const v16f d2 = __builtin_amdgcn_mfma_f32_32x32x16_f16(a2[i], b2, (v16f){}, 0, 0, 0);
#pragma unroll
                for (int e = 0; e < 16; e++) {
                    acc[i][k][e] = __builtin_fmaf(dm.x, d1[i][k][e], acc[i][k][e]);
                    acc[i][k][e] = __builtin_fmaf(-dm.y, d2[e], acc[i][k][e]);
                }
                d1[i][k] = (v16f){};
            }
        }
        GM_T(tf);
        GM_ADD(4, te, tf);
    }
#if defined(LE_TRACE)
    GM_T(t_end);
    tr[5] = t_end - t_start;
    if (tid == 0)
        for (int i = 0; i < 8; i++) le_gm_trace[blockIdx.x * 8 + i] = tr[i];
#endif
    /* D lane l element e: token 8*(e/4) + 4*(l/32) + e%4 of the tile, weight row l%32 */
#pragma unroll
    for (int i = 0; i < TM; i++)
#pragma unroll
        for (int k = 0; k < TN; k++) {
            const int r = nb + brow[k];
#pragma unroll
            for (int e = 0; e < 16; e++) {
                const int t = mb + 32 * i + 8 * (e >> 2) + 4 * hs + (e & 3);
                if (t < M && r < a.rows) a.y[(size_t)t * a.rows + r] = acc[i][k][e];
            }
        }
}

#define LE_GM(TM, TN)                                                                                      \
    extern "C" __global__ void __launch_bounds__(256) le_gm_12_m##TM##_n##TN(GmArgs a) { gm_q4k_body<TM, TN>(a); }

LE_GM(1, 1) LE_GM(1, 2) LE_GM(2, 1) LE_GM(2, 2)
