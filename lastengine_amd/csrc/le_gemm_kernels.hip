/* Small-M quantized GEMM on the matrix cores (gfx950): Y[t, r] = W[r, :] . X[t, :].
 *
 * Replaces the int8 MMA kernels mmq*_<ty> behind DenseGpu::bmm (src/cuda/kernels.cu:965-1223,
 * src/gpu/dense.rs:181-199); CPU twin cpu_ref::matmat (src/cpu_ref.rs:266-276).
 *
 * Numerics. Every supported format is, per super-block of 256 values and row r,
 *     w_k = d_r * c_k  -  dmin_r * m_{j(k)}
 * with small integer codes c_k (Q4_K: sc_j * q_k <= 945; the sub-block of value k is j(k)) and
 * integer offsets m_j. Integers below 2048 are exact in fp16, so the weight operand is the fp16
 * code c_k, built in registers from the raw GGUF bytes. The activations enter as xh = fp16(x)
 * (relative error 2^-11), or, under the split option, as two fp16 halves x = xh + xl (xl =
 * fp16(x - xh), 22 significant bits). The MFMAs multiply them by the codes with fp32
 * accumulation, so per super-block
 *     D1[t, r] = sum_k c_k (xh_k [+ xl_k])        D2[t, r] = sum_j m_j S_j(t)
 * (S_j = fp32 sum of x over sub-block j, split into fp16 halves for one more MFMA) and
 *     Y[t, r] += d_r * D1 - dmin_r * D2
 * in fp32. Activations must stay inside the fp16 range (|x| < 65504).
 *
 * GEMM tiling (M >= 9). A block of four MFMA waves (plus four staging waves in the
 * producer/consumer form) computes 32*TM tokens x 128*TN rows; every MFMA wave owns 32*TN rows
 * for all the block's tokens, as TM x TN tiles of v_mfma_f32_32x32x16_f16 (this shape runs near
 * the f16 peak with one wave per SIMD). K advances half a super-block per step. Staging is
 * coalesced: consecutive lanes load consecutive 16-byte chunks of a weight row's super-block and
 * consecutive float4s of a token's 256 activations, into registers one step ahead, then into LDS.
 * The weights stay raw in LDS (row stride 152 bytes: the 32-row fragment reads are free of bank
 * conflicts); each lane unpacks its own B fragment from 8 quant bytes just before the MFMAs, the
 * low nibbles giving one K slice and the high nibbles the slice 32 values further on. Blocks that
 * share weight rows (same row tile, different token tiles) get the same blockIdx % 8, so they run
 * on one XCD and share its L2. Within every aligned group of four K positions both operands are
 * stored in the order 0, 2, 1, 3 (what the nibble unpacking produces); the dot product does not
 * depend on the order.
 *
 * Few tokens (M = 3..8, le_mh_*): the staged matvec's weight stream with the tokens as the rows
 * of v_mfma_f32_16x16x32_f16 (described at mh_q4k_body).
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
    int ksplit; /* K slices (blockIdx.y); with more than one, the slices add into y, which the
                   pre-pass clears */
    int split;  /* 1: activations as fp16 high and low halves; 0: the high half only */
};



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
/* (x & m) | c in one v_and_or_b32 (a VOP3 instruction cannot carry the two literal constants, so
 * the compiler would otherwise emit an and and an or); m and c stay in registers */
__device__ __forceinline__ u32 gm_and_or(u32 x, u32 m, u32 c) {
    u32 r;
    __asm__("v_and_or_b32 %0, %1, %2, %3" : "=v"(r) : "v"(x), "v"(m), "v"(c));
    return r;
}
__device__ __forceinline__ void gm_q4k_frag(uint2 w, uint4 k, le_v8h &lo, le_v8h &hi) {
    const le_h2 slo = as_h2(k.x), clo = as_h2(k.y), shi = as_h2(k.z), chi = as_h2(k.w);
    const u32 mlo = 0x000F000Fu, mhi = 0x00F000F0u, c1024 = 0x64006400u;
    u32 l[4], h[4];
    const u32 ws[2] = {w.x, w.y};
#pragma unroll
    for (int i = 0; i < 2; i++) {
        const u32 a = ws[i], a8 = a >> 8;
        l[2 * i] = as_u32(__builtin_elementwise_fma(as_h2(gm_and_or(a, mlo, c1024)), slo, clo));
        l[2 * i + 1] = as_u32(__builtin_elementwise_fma(as_h2(gm_and_or(a8, mlo, c1024)), slo, clo));
        h[2 * i] = as_u32(__builtin_elementwise_fma(as_h2(gm_and_or(a, mhi, c1024)), shi, chi));
        h[2 * i + 1] = as_u32(__builtin_elementwise_fma(as_h2(gm_and_or(a8, mhi, c1024)), shi, chi));
    }
    lo = __builtin_bit_cast(le_v8h, make_uint4(l[0], l[1], l[2], l[3]));
    hi = __builtin_bit_cast(le_v8h, make_uint4(h[0], h[1], h[2], h[3]));
}

#define GM_WS 72  /* LDS bytes per row of a half super-block's quants: 64 + 8 */
#define GM_AS 136 /* fp16 per activation row of a half super-block: 128 + 8 */
#define GM_PD 2 /* producer register sets (steps of loads in flight + 1), one-half form */

/* Activation pre-pass: X fp32 [M][K] -> workspace planes Xh, Xl fp16 [M][K] (x = xh + xl, order
 * 0,2,1,3 within each four) and per (token, super-block) a 32-byte record of the eight sub-block
 * sums S_j as fp16 high halves then low halves. One wave per (token, super-block). */
extern "C" __global__ void __launch_bounds__(256) le_gm_xprep(GmArgs a, u8 *ws) {
    const int K = a.cols, nsb = K >> 8;
    if (a.ksplit > 1) { /* the K slices of the main pass add into y; the host sizes the grid to
                           cover y in a few trips */
        const size_t ny = (size_t)a.m * a.rows;
        for (size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x; i < ny; i += (size_t)gridDim.x * blockDim.x) a.y[i] = 0.f;
    }
    const int wid = blockIdx.x * 4 + (threadIdx.x >> 6); /* the host keeps m * nsb below 2^31 */
    if (wid >= a.m * nsb) return;
    const int lane = threadIdx.x & 63;
    const int t = wid / nsb, sb = wid - t * nsb;
    const size_t e = (size_t)t * K + 256 * sb + 4 * lane;
    const float4 v = *(const LE_GLOBAL float4 *)(a.x + e);
    u32 h0, h1, l0, l1;
    gm_split2(v.x, v.z, h0, l0);
    gm_split2(v.y, v.w, h1, l1);
    _Float16 *Xh = (_Float16 *)ws, *Xl = Xh + (size_t)a.m * K;
    *(LE_GLOBAL uint2 *)(Xh + e) = make_uint2(h0, h1);
    if (a.split) *(LE_GLOBAL uint2 *)(Xl + e) = make_uint2(l0, l1);
    /* without the low plane the MFMA sees only the high halves: sum those, so the mins term
     * cancels their rounding in the scale term */
    const le_h2 a0 = __builtin_bit_cast(le_h2, h0), a1 = __builtin_bit_cast(le_h2, h1);
    const float sum = group_sum<8>(a.split ? (v.x + v.y) + (v.z + v.w)
                                           : ((float)a0.x + (float)a1.x) + ((float)a0.y + (float)a1.y));
    const int si = __builtin_bit_cast(int, sum);
    /* the lane reads run on the whole wave, outside the single-lane store below (a reduction
     * moved under that branch would see inactive lanes) */
    float sv[8];
#pragma unroll
    for (int q = 0; q < 8; q++) sv[q] = __builtin_bit_cast(float, __builtin_amdgcn_readlane(si, 8 * q));
    __builtin_amdgcn_wave_barrier();
    if (lane == 0) {
        u32 hh[4], ll[4];
#pragma unroll
        for (int q = 0; q < 4; q++) gm_split2(sv[2 * q], sv[2 * q + 1], hh[q], ll[q]);
        uint4 *rec = (uint4 *)(ws + (size_t)a.m * K * 4) + 2 * wid;
        *(LE_GLOBAL uint4 *)rec = make_uint4(hh[0], hh[1], hh[2], hh[3]);
        *(LE_GLOBAL uint4 *)(rec + 1) = make_uint4(ll[0], ll[1], ll[2], ll[3]);
    }
}

template <int TM, int TN, bool SPLIT>
struct GmLds {
    static constexpr int BM = 32 * TM, BN = 128 * TN;
    /* one pipeline buffer: the half super-block's quants, fragment constants of its two groups,
     * offsets m_j, (d, dmin), activation high halves, low halves (SPLIT only) */
    static constexpr int W_OFF = 0, K_OFF = BN * GM_WS, M_OFF = K_OFF + BN * 32, D_OFF = M_OFF + BN * 16,
                         AH_OFF = D_OFF + BN * 8, AL_OFF = AH_OFF + BM * GM_AS * 2,
                         BUF = AL_OFF + (SPLIT ? BM * GM_AS * 2 : 0);
    static constexpr int S_OFF = 2 * BUF, BYTES = S_OFF + 2 * BM * 32; /* + sum records [2][BM][32 B] */
};

/* PC = producer/consumer blocks of 8 waves: waves 0-3 only compute (MFMAs, epilogues), waves
 * 4-7 only load and stage the next step, so the staging work overlaps the MFMAs on other waves
 * instead of alternating with them; otherwise 4 waves do both. */
template <int TM, int TN, bool PC, bool SPLIT = true>
__device__ __forceinline__ void gm_q4k_body(const GmArgs &a, const u8 *ws) {
    using L = GmLds<TM, TN, SPLIT>;
    constexpr int BM = L::BM, BN = L::BN;
    constexpr int NQC = BN * 4 / 256, NHC = BN / 256 > 0 ? BN / 256 : 1, NXC = BM * (SPLIT ? 32 : 16) / 256;
    typedef float v16f __attribute__((ext_vector_type(16)));
    extern __shared__ uint4 smem[];
    u8 *lds = (u8 *)smem;
    uint4 *Sx = (uint4 *)(lds + L::S_OFF);

    const int K = a.cols, nsb = K >> 8, M = a.m;
    const int NT = (a.rows + BN - 1) / BN, MT = (M + BM - 1) / BM;
    const int id = blockIdx.x, j = id >> 3;
    const int mt = j % MT, nt = (j / MT) * 8 + (id & 7);
    if (nt >= NT) return; /* uniform over the block */
    const int nb = nt * BN, mb = mt * BM;
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const bool producer = PC && wave >= 4;
    const int st = PC ? (tid & 255) : tid; /* staging thread index */
    const size_t rb = (size_t)nsb * 144;
    /* K slice blockIdx.y: super-blocks sb0..sb1-1 (the host makes nsb a multiple of ksplit) */
    const int sb0 = blockIdx.y * (nsb / a.ksplit), sb1 = sb0 + nsb / a.ksplit;
    const int nstep = 2 * sb1;
    const _Float16 *Xh = (const _Float16 *)ws, *Xl = Xh + (size_t)M * K;
    const uint4 *Xs = (const uint4 *)(ws + (size_t)M * K * 4);

    /* staging of step s (super-block s/2, half s&1), all copies of 16 bytes:
     *   header of row tid (+256 i), decoded by this thread;
     *   quant chunk c = tid + 256 i: row c/4, 16-byte column c%4 of the half's 64 bytes;
     *   activation chunk c = tid + 256 i: token c/32, plane (c/16)&1, 8-value column c%16
     *   (two halves), or token c/16, column c%16 (high half only);
     *   sum record chunk tid < 2*BM: token tid/2, half tid&1 (staged once per super-block) */
    struct Set {
        uint4 wh[NHC], wq[NQC], xa[NXC], xs;
    };
    /* every load is unconditional and wave-uniform in count, so the compiler's wait before
     * staging step s+1 counts only that step's loads and the later steps stay in flight; a step
     * past the slice (prefetch tail) re-reads the last one */
    auto issue = [&](int s_, Set &R) {
        const int s = min(s_, nstep - 1), sb = s >> 1, h = s & 1;
        const u8 *w0 = a.w + (size_t)sb * 144;
#pragma unroll
        for (int i = 0; i < NHC; i++) R.wh[i] = ldg16(w0 + (size_t)min(nb + st + 256 * i, a.rows - 1) * rb);
#pragma unroll
        for (int i = 0; i < NQC; i++) {
            const int c = st + 256 * i, row = c >> 2;
            R.wq[i] = ldg16(w0 + (size_t)min(nb + row, a.rows - 1) * rb + 16 + 64 * h + 16 * (c & 3));
        }
#pragma unroll
        for (int i = 0; i < NXC; i++) {
            const int c = st + 256 * i;
            /* SPLIT: token c/32, plane (c/16)&1; otherwise token c/16 of the high plane */
            const int t = min(mb + (SPLIT ? c >> 5 : c >> 4), M - 1);
            const _Float16 *src = (SPLIT && ((c >> 4) & 1) ? Xl : Xh) + (size_t)t * K + 256 * sb + 128 * h + 8 * (c & 15);
            R.xa[i] = ldg16c((const u8 *)src);
        }
        R.xs = ldg16c((const u8 *)(Xs + 2 * ((size_t)min(mb + (st >> 1), M - 1) * nsb + sb) + (st & 1)));
    };
    auto stage = [&](int s, const Set &R) {
        const int sb = s >> 1, h = s & 1;
        u8 *B = lds + (s & 1) * L::BUF;
#pragma unroll
        for (int i = 0; i < NHC; i++) {
            const int row = st + 256 * i;
            if (row >= BN) break;
            const u32 sy = R.wh[i].y, sz = R.wh[i].z, sw = R.wh[i].w;
            const u32 scw = h ? ((sw & 0x0F0F0F0Fu) | ((sy >> 2) & 0x30303030u)) : (sy & 0x3F3F3F3Fu);
            uint4 *kc = (uint4 *)(B + L::K_OFF) + 2 * row;
#pragma unroll
            for (int g = 0; g < 2; g++) {
                const float sl = (float)((scw >> (16 * g)) & 255u), sh = (float)((scw >> (16 * g + 8)) & 255u);
                const le_h2 v0 = {(_Float16)sl, (_Float16)sl}, v1 = {(_Float16)(-1024.f * sl), (_Float16)(-1024.f * sl)};
                const le_h2 v2 = {(_Float16)(0.0625f * sh), (_Float16)(0.0625f * sh)}, v3 = {(_Float16)(-64.f * sh), (_Float16)(-64.f * sh)};
                kc[g] = make_uint4(as_u32(v0), as_u32(v1), as_u32(v2), as_u32(v3));
            }
            const u32 m0 = sz & 0x3F3F3F3Fu, m1 = ((sw >> 4) & 0x0F0F0F0Fu) | ((sz >> 2) & 0x30303030u);
            u32 mw[4];
#pragma unroll
            for (int q = 0; q < 4; q++) {
                const u32 mm = (q < 2 ? m0 : m1) >> (16 * (q & 1));
                const le_h2 v = {(_Float16)(float)(mm & 255u), (_Float16)(float)((mm >> 8) & 255u)};
                mw[q] = as_u32(v);
            }
            ((uint4 *)(B + L::M_OFF))[row] = make_uint4(mw[0], mw[1], mw[2], mw[3]);
            ((float2 *)(B + L::D_OFF))[row] = make_float2(h2f(R.wh[i].x & 0xFFFFu), h2f(R.wh[i].x >> 16));
        }
#pragma unroll
        for (int i = 0; i < NQC; i++) {
            const int c = st + 256 * i;
            uint2 *d = (uint2 *)(B + L::W_OFF + (c >> 2) * GM_WS + 16 * (c & 3));
            d[0] = make_uint2(R.wq[i].x, R.wq[i].y);
            d[1] = make_uint2(R.wq[i].z, R.wq[i].w);
        }
#pragma unroll
        for (int i = 0; i < NXC; i++) {
            const int c = st + 256 * i;
            if constexpr (SPLIT)
                *(uint4 *)(B + ((c >> 4) & 1 ? L::AL_OFF : L::AH_OFF) + ((c >> 5) * GM_AS + 8 * (c & 15)) * 2) = R.xa[i];
            else
                *(uint4 *)(B + L::AH_OFF + ((c >> 4) * GM_AS + 8 * (c & 15)) * 2) = R.xa[i];
        }
        if (h == 0 && st < 2 * BM) Sx[((sb & 1) * BM + (st >> 1)) * 2 + (st & 1)] = R.xs;
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

    if (producer) {
        constexpr int PD = SPLIT ? 2 : GM_PD; /* the two-half form has no registers to spare */
        /* a ring of PD register sets: while the consumers work on step s, the loads of steps
         * s+2 .. s+PD are in flight; the loop is unrolled by PD so the sets are registers */
        Set R[PD];
        const int s0 = 2 * sb0;
        issue(s0, R[0]);
        stage(s0, R[0]);
#pragma unroll
        for (int u = 1; u < PD; u++) issue(s0 + u, R[u]);
        /* whole groups of PD steps without early exits (an exit merging into the loop would
         * make the compiler wait for every load), then the remaining steps */
        int s = s0;
        for (; s + PD <= nstep; s += PD) {
#pragma unroll
            for (int u = 0; u < PD; u++) {
                gm_barrier(); /* step s+u is staged; the consumers are done with step s+u-1's buffer */
                if (s + u + 1 < nstep) stage(s + u + 1, R[(u + 1) % PD]);
                issue(s + u + PD, R[u]);
            }
        }
#pragma unroll
        for (int u = 0; u < PD - 1; u++) {
            if (s + u >= nstep) break;
            gm_barrier();
            if (s + u + 1 < nstep) stage(s + u + 1, R[(u + 1) % PD]);
        }
        return;
    }
    Set R0;
    if (!PC) {
        issue(2 * sb0, R0);
        stage(2 * sb0, R0);
        issue(2 * sb0 + 1, R0);
    }
    for (int sb = sb0; sb < sb1; sb++) {
#pragma unroll
        for (int h = 0; h < 2; h++) {
            const int s = 2 * sb + h;
            gm_barrier(); /* step s is staged; every wave is done with step s-1's buffer */
            const u8 *B = lds + h * L::BUF; /* s & 1 == h */
            const _Float16 *Ah = (const _Float16 *)(B + L::AH_OFF), *Al = (const _Float16 *)(B + L::AL_OFF);
#pragma unroll
            for (int gl = 0; gl < 2; gl++) {
                uint4 kc[TN];
#pragma unroll
                for (int k = 0; k < TN; k++) kc[k] = ((const uint4 *)(B + L::K_OFF))[2 * brow[k] + gl];
#pragma unroll
                for (int c = 0; c < 2; c++) {
                    /* K slice: values 64gl + 16c + 8hs .. +8 (low nibbles) and 32 further (high) */
                    le_v8h blo[TN], bhi[TN];
#pragma unroll
                    for (int k = 0; k < TN; k++) {
                        const uint2 w = *(const uint2 *)(B + L::W_OFF + brow[k] * GM_WS + 32 * gl + 16 * c + 8 * hs);
                        gm_q4k_frag(w, kc[k], blo[k], bhi[k]);
                    }
#pragma unroll
                    for (int half = 0; half < 2; half++) {
                        const int ko = 64 * gl + 32 * half + 16 * c + 8 * hs;
                        le_v8h ah[TM], al[TM];
#pragma unroll
                        for (int i = 0; i < TM; i++) {
                            ah[i] = __builtin_bit_cast(le_v8h, *(const uint4 *)(Ah + (32 * i + r32) * GM_AS + ko));
                            if constexpr (SPLIT) al[i] = __builtin_bit_cast(le_v8h, *(const uint4 *)(Al + (32 * i + r32) * GM_AS + ko));
                        }
                        /* the super-block's first MFMA starts from zero: no clearing pass */
                        const bool first = h == 0 && gl == 0 && c == 0 && half == 0;
#pragma unroll
                        for (int i = 0; i < TM; i++)
#pragma unroll
                            for (int k = 0; k < TN; k++)
                                d1[i][k] = __builtin_amdgcn_mfma_f32_32x32x16_f16(ah[i], half ? bhi[k] : blo[k],
                                                                                  first ? (v16f){} : d1[i][k], 0, 0, 0);
                        if constexpr (SPLIT) {
#pragma unroll
                            for (int i = 0; i < TM; i++)
#pragma unroll
                                for (int k = 0; k < TN; k++)
                                    d1[i][k] = __builtin_amdgcn_mfma_f32_32x32x16_f16(al[i], half ? bhi[k] : blo[k], d1[i][k], 0, 0, 0);
                        }
                    }
                }
                /* the next step's staging and the loads two steps ahead run under this step's MFMAs */
                if (!PC && gl == 0) {
                    if (s + 1 < nstep) stage(s + 1, R0);
                    if (s + 2 < nstep) issue(s + 2, R0);
                }
            }
        }
        /* super-block epilogue: Y += d * D1 - dmin * D2, D2 = sum_j m_j S_j by one more MFMA per
         * tile (K slice 0: high halves of S_0..7, slice 1: low halves, both against m); all D2
         * MFMAs are issued before their results are read */
        {
            const u8 *B = lds + L::BUF; /* the super-block's second half wrote m and (d, dmin) too */
            le_v8h a2[TM];
#pragma unroll
            for (int i = 0; i < TM; i++) a2[i] = __builtin_bit_cast(le_v8h, Sx[((sb & 1) * BM + 32 * i + r32) * 2 + hs]);
            v16f d2[TM][TN];
#pragma unroll
            for (int k = 0; k < TN; k++) {
                const le_v8h b2 = __builtin_bit_cast(le_v8h, ((const uint4 *)(B + L::M_OFF))[brow[k]]);
#pragma unroll
                for (int i = 0; i < TM; i++) d2[i][k] = __builtin_amdgcn_mfma_f32_32x32x16_f16(a2[i], b2, (v16f){}, 0, 0, 0);
            }
#pragma unroll
            for (int k = 0; k < TN; k++) {
                const float2 dm = ((const float2 *)(B + L::D_OFF))[brow[k]];
#pragma unroll
                for (int i = 0; i < TM; i++)
#pragma unroll
                    for (int e = 0; e < 16; e++) {
                        acc[i][k][e] = __builtin_fmaf(dm.x, d1[i][k][e], acc[i][k][e]);
                        acc[i][k][e] = __builtin_fmaf(-dm.y, d2[i][k][e], acc[i][k][e]);
                    }
            }
        }
    }
    /* D lane l element e: token 8*(e/4) + 4*(l/32) + e%4 of the tile, weight row l%32 */
#pragma unroll
    for (int i = 0; i < TM; i++)
#pragma unroll
        for (int k = 0; k < TN; k++) {
            const int r = nb + brow[k];
#pragma unroll
            for (int e = 0; e < 16; e++) {
                const int t = mb + 32 * i + 8 * (e >> 2) + 4 * hs + (e & 3);
                if (t < M && r < a.rows) {
                    if (a.ksplit > 1)
                        unsafeAtomicAdd(a.y + (size_t)t * a.rows + r, acc[i][k][e]);
                    else
                        a.y[(size_t)t * a.rows + r] = acc[i][k][e];
                }
            }
        }
}

/* ===================== few tokens (M <= 8): the matvec's weight stream on f16 MFMAs =====================
 * The staged matvec layout (16-row tiles, each wave streaming P super-blocks per row as
 * consecutive 16-byte chunks, one item ahead in registers, into wave-private LDS), with the
 * tokens as the rows of v_mfma_f32_16x16x32_f16: one MFMA per sub-block covers every token, its
 * K slice is the sub-block's 32 values, and B holds the exact fp16 codes sc_j * q (gm_q4k_frag),
 * so the sub-block scales need no per-token work. D2 = sum_j m_j S_j(t) is one more MFMA of the
 * sum records (high halves in K 0-7, low halves in K 8-15) against the mins. Each wave builds
 * the fp16 activations and sub-block sums of its super-blocks of all T tokens in LDS once per
 * block, each (token, super-block) scaled by the power of two 2^s that puts its largest |x| in
 * [512, 1024) (so every value keeps 11 significant bits down to 2^-14 of that maximum and a
 * 32-value sum stays below 32768 at any input magnitude); 2^-s multiplies the super-block's
 * d D1 - dmin D2. MFMA rows past T repeat token rows (finite, never stored). */
struct MhArgs {
    const u8 *w;
    const float *x;
    float *y;
    int rows, cols, m;
    int groups; /* token groups of T: block b takes group (b / 8) % groups and every
                 * (gridDim.x / groups)-th row tile from ((b / 8) / groups) * 8 + b % 8, so the groups
                 * of a tile stream its weights at the same time on one XCD (the host makes
                 * gridDim.x / groups a multiple of 8 when groups > 1) */
};

template <int P, int NW, int T>
__device__ __forceinline__ void mh_q4k_body(const MhArgs &a) {
    typedef float v4f __attribute__((ext_vector_type(4)));
    extern __shared__ uint4 smem[];
    /* CPR: 16-byte slots per staged row, odd so that the 16 rows of a read fall into distinct
     * banks; IMS: slots per (token, sub-block) image record, 5 so that the 8 tokens of a read do */
    constexpr int CPR = (9 * P + 1) | 1, NCH = 16 * CPR, NI = (NCH + 63) / 64, IMS = 5;
    const int K = a.cols, nsb = K >> 8, M = a.m;
    /* token group and row-tile block: blocks b and b + 8 run on the same XCD (blocks go to the
     * XCDs round-robin), so the groups of a row tile are blocks 8 apart and share that XCD's L2 */
    const int G = max(a.groups, 1), rnd = (int)blockIdx.x >> 3;
    const int tok0 = T * (rnd % G), bx = (rnd / G) * 8 + (int)(blockIdx.x & 7), gx = max((int)gridDim.x / G, 1);
    const size_t rb = (size_t)nsb * 144;
    const int lane = threadIdx.x & 63, wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6); /* wave-uniform */
    const int n = lane & 15, kq = lane >> 4;
    const int nsbw = nsb / NW;
    /* wave-private LDS: the image [local sb][sub-block j][token][4 x 16 B], the sum records
     * [local sb][token][2 x 16 B], the inverse scales [local sb][MFMA row 0..15] (float), then
     * the weight staging */
    const int wsz = nsbw * 8 * T * IMS + nsbw * T * 2 + nsbw * 4;
    uint4 *img = smem + wave * (wsz + NI * 64);
    uint4 *srec = img + nsbw * 8 * T * IMS;
    float *isc = (float *)(srec + nsbw * T * 2);
    uint4 *wb = img + wsz;
    float *red = (float *)(smem + NW * (wsz + NI * 64)); /* [NW][16 tokens][16 rows] */
    const int ntile = (a.rows + 15) >> 4;
    const int sfirst = wave * P, sstep = NW * P;
    const bool active = sfirst < nsb;
    auto gsb = [&](int l) { return (l / P) * sstep + sfirst + l % P; }; /* local -> global super-block */

    int ri[NI], cb[NI];
#pragma unroll
    for (int i = 0; i < NI; i++) {
        const int c = min(64 * i + lane, NCH - 1);
        const int col = c % CPR;
        ri[i] = c / CPR;
        cb[i] = (col >= 9 * P ? 0 : col) * 16; /* pad slots re-read chunk 0 (never past the super-block) */
    }
    uint4 R[NI];
    auto issue = [&](int tile, int s0) {
#pragma unroll
        for (int i = 0; i < NI; i++) {
            const int row = min(tile * 16 + ri[i], a.rows - 1);
            R[i] = ldg16(a.w + (size_t)row * rb + (size_t)s0 * 144 + cb[i]);
        }
    };
    /* the wave's activations, built here: 64-lane row k of its chunks holds (local sb l, token t)
     * = (q / T, q % T) for q = 2k + lane / 32 and the 8-value column lane % 32 of the 256 ->
     * 16 bytes of fp16 in the order 0,2,1,3 within each four (the order of the B fragments);
     * the four lanes of a 32-value sub-block add their sums, which go into the token's record as
     * fp16 high and low halves. The first XP rows are loaded before the first weight item: the
     * memory wait counter retires in issue order, so activations loaded after the weights could
     * not be used before the weights had landed. */
    constexpr int LT = T == 4 ? 2 : T == 8 ? 3 : 4, XP = 8;
    /* every wave has super-blocks: the host launches only shapes with nsb % (NW P) == 0 */
    const int nk = nsbw * T / 2, hs32 = lane >> 5, col = lane & 31;
    auto xsrc = [&](int k) {
        const int q = 2 * k + hs32, l = q >> LT, t = q & (T - 1);
        return a.x + (min(tok0 + t, M - 1) * K + 256 * gsb(l) + 8 * col);
    };
    /* the largest magnitude of a (token, super-block) as an integer maximum of the bit patterns
     * without sign (the float order for every non-NaN value); over the 32 lanes by DPP within
     * each row of 16 and one swizzle (xor 16) across */
    auto amax = [&](const float4 &v0, const float4 &v1) {
        const u32 am = 0x7FFFFFFFu;
        u32 mx = max(max(__float_as_uint(v0.x) & am, __float_as_uint(v0.y) & am), __float_as_uint(v0.z) & am);
        mx = max(max(mx, __float_as_uint(v0.w) & am), __float_as_uint(v1.x) & am);
        mx = max(max(mx, __float_as_uint(v1.y) & am), __float_as_uint(v1.z) & am);
        mx = max(mx, __float_as_uint(v1.w) & am);
        mx = max(mx, (u32)__builtin_amdgcn_update_dpp(0, (int)mx, 0xB1, 0xF, 0xF, true));  /* quad_perm [1,0,3,2] */
        mx = max(mx, (u32)__builtin_amdgcn_update_dpp(0, (int)mx, 0x4E, 0xF, 0xF, true));  /* quad_perm [2,3,0,1] */
        mx = max(mx, (u32)__builtin_amdgcn_update_dpp(0, (int)mx, 0x141, 0xF, 0xF, true)); /* row_half_mirror */
        mx = max(mx, (u32)__builtin_amdgcn_update_dpp(0, (int)mx, 0x140, 0xF, 0xF, true)); /* row_mirror */
        return max(mx, (u32)__builtin_amdgcn_ds_swizzle((int)mx, 0x401F));
    };
    typedef _Float16 h2v __attribute__((ext_vector_type(2)));
    auto emit = [&](int k, const float4 &v0, const float4 &v1, u32 mx) {
        const int q = 2 * k + hs32, l = q >> LT, t = q & (T - 1);
        /* biased exponent b of the maximum: x 2^(136 - b) puts it in [512, 1024); the factor is
         * kept within 2^-118 .. 2^126 (zero or subnormal maxima, inf / NaN) */
        const int sx = min(max(136 - (int)(mx >> 23), -118), 126);
        const float sc = __uint_as_float((u32)(127 + sx) << 23);
        if (col < 16 / T) isc[l * 16 + t + T * col] = __uint_as_float((u32)(127 - sx) << 23); /* MFMA rows t, t + T, ... */
        const h2v e0 = {(_Float16)(v0.x * sc), (_Float16)(v0.z * sc)}, e1 = {(_Float16)(v0.y * sc), (_Float16)(v0.w * sc)};
        const h2v e2 = {(_Float16)(v1.x * sc), (_Float16)(v1.z * sc)}, e3 = {(_Float16)(v1.y * sc), (_Float16)(v1.w * sc)};
        img[((l * 8 + (col >> 2)) * T + t) * IMS + (col & 3)] =
            make_uint4(__builtin_bit_cast(u32, e0), __builtin_bit_cast(u32, e1), __builtin_bit_cast(u32, e2), __builtin_bit_cast(u32, e3));
        /* sums of the fp16-rounded values, so the mins term cancels the rounding the scale term
         * sees (the error then scales with sum |w x|) */
        const h2v one = {(_Float16)1.f, (_Float16)1.f};
        float sm = __builtin_amdgcn_fdot2(e0, one, 0.f, false);
        sm = __builtin_amdgcn_fdot2(e1, one, sm, false);
        sm = __builtin_amdgcn_fdot2(e2, one, sm, false);
        sm = __builtin_amdgcn_fdot2(e3, one, sm, false);
        sm += dpp_f<0xB1>(sm);
        sm += dpp_f<0x4E>(sm);
        if ((col & 3) == 0) {
            const _Float16 hi = (_Float16)sm, lo = (_Float16)(sm - (float)hi);
            _Float16 *rec = (_Float16 *)(srec + (l * T + t) * 2);
            rec[col >> 2] = hi;
            rec[8 + (col >> 2)] = lo;
        }
    };
    {
        float4 v[XP][2];
#pragma unroll
        for (int k = 0; k < XP; k++) {
            const float *src = xsrc(min(k, nk - 1));
            v[k][0] = *(const LE_GLOBAL float4 *)src;
            v[k][1] = *(const LE_GLOBAL float4 *)(src + 4);
        }
        issue(min(bx, ntile - 1), active ? sfirst : 0);
        __builtin_amdgcn_sched_barrier(0); /* the weight loads go out before any activation wait */
        /* every row's maximum first, so the rows' cross-lane reductions overlap */
        u32 mx[XP];
#pragma unroll
        for (int k = 0; k < XP; k++) mx[k] = amax(v[k][0], v[k][1]);
#pragma unroll
        for (int k = 0; k < XP; k++)
            if (k < nk) emit(k, v[k][0], v[k][1], mx[k]); /* wave-uniform */
    }
    for (int k0 = XP; k0 < nk; k0 += 4) { /* T = 16, or more than 2 local super-blocks at T = 8: the rest, after the weights */
        float4 v[4][2];
#pragma unroll
        for (int u = 0; u < 4; u++) {
            const float *src = xsrc(min(k0 + u, nk - 1));
            v[u][0] = *(const LE_GLOBAL float4 *)src;
            v[u][1] = *(const LE_GLOBAL float4 *)(src + 4);
        }
        u32 mx[4];
#pragma unroll
        for (int u = 0; u < 4; u++) mx[u] = amax(v[u][0], v[u][1]);
#pragma unroll
        for (int u = 0; u < 4; u++)
            if (k0 + u < nk) emit(k0 + u, v[u][0], v[u][1], mx[u]);
    }
    const int ta = n % T; /* this lane's A row (token); rows past T repeat earlier tokens */
    int par = 0;
    for (int tile = bx; tile < ntile; tile += gx) {
        v4f y = {0.f, 0.f, 0.f, 0.f};
        if (active) {
            for (int s0 = sfirst, lb = 0; s0 < nsb; s0 += sstep, lb += P) {
                int nt = tile, ns = s0 + sstep;
                if (ns >= nsb) { ns = sfirst; nt += gx; }
#pragma unroll
                for (int i = 0; i < NI; i++) wb[64 * i + lane] = R[i];
                if (nt < ntile) issue(nt, ns);
#pragma unroll
                for (int q = 0; q < P; q++) {
                    const int l = lb + q;
                    const uint4 *sbp = wb + n * CPR + 9 * q;
                    const uint4 hd = sbp[0];
                    const u32 sy = hd.y, sz = hd.z, sw = hd.w;
                    const u32 scw[2] = {sy & 0x3F3F3F3Fu, (sw & 0x0F0F0F0Fu) | ((sy >> 2) & 0x30303030u)};
                    const u32 mw[2] = {sz & 0x3F3F3F3Fu, ((sw >> 4) & 0x0F0F0F0Fu) | ((sz >> 2) & 0x30303030u)};
                    v4f d1 = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
                    for (int g = 0; g < 4; g++) {
                        const uint2 w = *(const uint2 *)((const u8 *)(sbp + 1) + 32 * g + 8 * kq);
                        const u32 sc2 = scw[g >> 1] >> (16 * (g & 1));
                        const float sl = (float)(sc2 & 255u), sh = (float)((sc2 >> 8) & 255u);
                        const le_h2 v0 = {(_Float16)sl, (_Float16)sl}, v1 = {(_Float16)(-1024.f * sl), (_Float16)(-1024.f * sl)};
                        const le_h2 v2 = {(_Float16)(0.0625f * sh), (_Float16)(0.0625f * sh)}, v3 = {(_Float16)(-64.f * sh), (_Float16)(-64.f * sh)};
                        le_v8h blo, bhi;
                        gm_q4k_frag(w, make_uint4(as_u32(v0), as_u32(v1), as_u32(v2), as_u32(v3)), blo, bhi);
                        const le_v8h alo = __builtin_bit_cast(le_v8h, img[((l * 8 + 2 * g) * T + ta) * IMS + kq]);
                        const le_v8h ahi = __builtin_bit_cast(le_v8h, img[((l * 8 + 2 * g + 1) * T + ta) * IMS + kq]);
                        d1 = __builtin_amdgcn_mfma_f32_16x16x32_f16(alo, blo, d1, 0, 0, 0);
                        d1 = __builtin_amdgcn_mfma_f32_16x16x32_f16(ahi, bhi, d1, 0, 0, 0);
                    }
                    /* D2: K 0-7 = high halves of S_0..7 against m_0..7, K 8-15 = low halves; the
                     * other K slices multiply zero mins */
                    u32 mb[4];
#pragma unroll
                    for (int qq = 0; qq < 4; qq++) {
                        const u32 mm = mw[qq >> 1] >> (16 * (qq & 1));
                        const le_h2 v = {(_Float16)(float)(mm & 255u), (_Float16)(float)((mm >> 8) & 255u)};
                        mb[qq] = kq < 2 ? as_u32(v) : 0u;
                    }
                    const le_v8h b2 = __builtin_bit_cast(le_v8h, make_uint4(mb[0], mb[1], mb[2], mb[3]));
                    const le_v8h a2 = __builtin_bit_cast(le_v8h, srec[(l * T + ta) * 2 + (kq & 1)]);
                    const v4f d2 = __builtin_amdgcn_mfma_f32_16x16x32_f16(a2, b2, (v4f){0.f, 0.f, 0.f, 0.f}, 0, 0, 0);
                    const float dd = h2f(hd.x & 0xFFFFu), dm = h2f(hd.x >> 16);
                    const float4 iv = *(const float4 *)(isc + l * 16 + 4 * kq);
                    const float ivs[4] = {iv.x, iv.y, iv.z, iv.w};
#pragma unroll
                    for (int e = 0; e < 4; e++) y[e] = __builtin_fmaf(ivs[e], __builtin_fmaf(dd, d1[e], -dm * d2[e]), y[e]);
                }
            }
        }
        /* D lane l element e: token 4*kq + e, row n; the waves' K shares add in a fixed order */
        float *rp = red + par * (NW * 256);
#pragma unroll
        for (int e = 0; e < 4; e++) rp[wave * 256 + (4 * kq + e) * 16 + n] = y[e];
        __builtin_amdgcn_s_waitcnt(0xC07F);
        __builtin_amdgcn_s_barrier();
        if (wave == 0) {
#pragma unroll
            for (int o = lane; o < T * 16; o += 64) {
                const int t = o >> 4, r = tile * 16 + (o & 15);
                float acc = 0.f;
#pragma unroll
                for (int w = 0; w < NW; w++) acc += rp[w * 256 + o];
                if (r < a.rows && tok0 + t < M) a.y[(size_t)(tok0 + t) * a.rows + r] = acc;
            }
        }
        par ^= 1;
    }
}

#define LE_MH(P, NW, T)                                                                                    \
    extern "C" __global__ void __launch_bounds__(NW * 64) le_mh_12_p##P##_w##NW##_t##T(MhArgs a) {        \
        mh_q4k_body<P, NW, T>(a);                                                                          \
    }
LE_MH(1, 4, 4) LE_MH(1, 4, 8) LE_MH(2, 4, 4) LE_MH(2, 4, 8) LE_MH(1, 8, 4) LE_MH(1, 8, 8) LE_MH(2, 2, 4) LE_MH(2, 2, 8)
LE_MH(1, 4, 16) LE_MH(2, 4, 16) LE_MH(1, 8, 16) LE_MH(2, 2, 16)

#define LE_GM(TM, TN)                                                                                      \
    extern "C" __global__ void __launch_bounds__(256) le_gm_12_m##TM##_n##TN(GmArgs a, const u8 *ws) {    \
        gm_q4k_body<TM, TN, false>(a, ws);                                                                 \
    }
/* producer/consumer forms, with both activation halves (_pc) or the high half only (_pc1); the
 * 64 x 256 tile has none, as it does not fit the registers */
#define LE_GM_PC(TM, TN)                                                                                     \
    extern "C" __global__ void __launch_bounds__(512) le_gm_12_m##TM##_n##TN##_pc(GmArgs a, const u8 *ws) {  \
        gm_q4k_body<TM, TN, true>(a, ws);                                                                    \
    }                                                                                                        \
    extern "C" __global__ void __launch_bounds__(512) le_gm_12_m##TM##_n##TN##_pc1(GmArgs a, const u8 *ws) { \
        gm_q4k_body<TM, TN, true, false>(a, ws);                                                             \
    }

LE_GM(1, 1) LE_GM(1, 2) LE_GM(2, 1) LE_GM(2, 2)
LE_GM_PC(1, 1) LE_GM_PC(1, 2) LE_GM_PC(2, 1)
