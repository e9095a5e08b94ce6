/* Quantized GEMM on the matrix cores for every supported type (gfx950):
 *     Y[t, r] = W[r, :] . X[t, :],  t < M tokens, r < N rows, K = cols.
 *
 * Replaces the int8 MMA kernels mmq*_<ty> / mmq128r_<ty> behind DenseGpu::bmm and prefill::dense
 * (src/cuda/kernels.cu:965-1235, src/gpu/dense.rs:181-199, src/gpu/prefill.rs:44-60); CPU twin
 * cpu_ref::matmat (src/cpu_ref.rs:266-276).
 *
 * Operands. v_mfma_f32_32x32x16_f16 with the tokens as A (32 x 16) and the weight rows as B
 * (16 x 32), fp32 accumulation. Lane l of a fragment holds token / row l % 32 and the eight K
 * positions 8 (l / 32) .. +8 of the 16-value K chunk, stored in the order P8 = 0,2,1,3,4,6,5,7
 * (what the byte-pair fp16 conversion below produces; the dot product does not depend on the
 * order as long as A and B agree).
 *
 * Activations (pre-pass le_gq_xprep_*). Token t is scaled by 2^-e_t, e_t chosen so that
 * max|x_t| 2^-e_t lies in [64, 128) (exact: a power of two), and rounded to fp16 (relative error
 * 2^-11; values below 2^-24 of the token's maximum flush towards zero). The result is written in
 * fragment order, [32-token tile][K/16 chunk][8-lane half][token][8 halves], so a block copies
 * each step's activations as contiguous 8 KB runs and every A fragment is one conflict-free
 * 16-byte LDS read per lane. Q4_K and Q5_K also get per-super-block sub-block sums S_j (per 32
 * values, as fp16 high + low halves) for their offset term. The final store multiplies by
 * 2^e_t, so the result does not depend on the activations' magnitude.
 *
 * Weights. Raw GGUF rows (src/gpu.rs:79-83), read in half super-blocks (128 values) per pipeline
 * step: each row's bytes for the step are copied as 16-byte chunks (coalesced: consecutive lanes
 * take consecutive chunks of a row) into a 16-byte-aligned LDS slot of F::SLOT bytes, then each
 * lane builds its B fragments from them:
 *   Q4_K   code sc_j * q (<= 945, exact), offset term D2 = sum_j m_j S_j (one more MFMA per
 *          super-block), epilogue  acc += d * D1 - dmin * D2                 (src/quant.rs:72-82)
 *   Q6_K   code (q6 - 32) * sc_u / 64 (exact where (q6 - 32) sc_u has at most 11 significant
 *          bits, else rounded once to fp16), epilogue acc += 64 d * D1           (:96-112)
 *   IQ2_XXS code (2s+1) * grid * sign (<= 1333, exact), epilogue acc += d/8 * D1   (:142-154)
 *   IQ3_XXS code (2s+1) * grid * sign (<= 1922, exact), epilogue acc += d/4 * D1   (:127-141)
 *   Q5_K   as Q4_K with the fifth bit from qh, code sc_j * q (<= 1953, exact)     (:83-95)
 *   Q3_K   code (q3 - 4) * (sc6 - 32) (|.| <= 128, exact), epilogue acc += d * D1 (:113-126)
 *   IQ2_S  code (2s+1) * grid * sign, 1024-entry grid, explicit sign bytes, epilogue acc += d/8 * D1
 *                                                                                  (:155-167)
 *   Q8_0, Q4_0  per-32 scale d_b inside the code: fp16(q * d_b 2^S) (one rounding, 2^-11
 *          relative), S a per-row power of two that only decreases (the accumulator is rescaled
 *          when it does) and keeps every code inside the fp16 range, final * 2^-S  (:64-71)
 * Integer byte -> fp16 conversion: a byte u placed under the fp16 exponent of 1024 (v_perm_b32)
 * is the half 1024 + u exactly; one packed fma (u+1024)*c - 1024*c gives u*c rounded once.
 *
 * Tiling. A block of WM x WN waves computes BM = 32 TM WM tokens x BN = 32 TN WN rows; a wave
 * owns TM x TN 32x32 tiles. Steps are double-buffered in LDS; every thread holds two further
 * steps of loads in registers (issued two steps before they are written to LDS), so the loads of
 * steps s+2 and s+3 are in flight while step s computes. Blocks that share weight rows (same row
 * tile, other token tiles or K slices) get the same blockIdx % 8 and therefore the same XCD and
 * L2. With fewer than 8 row tiles, row tiles vary fastest instead, so the blocks
 * spread over all XCDs. K may be split over blockIdx.y; the slices' partial results are then
 * summed by le_gq_ksum (or, without room for them, added into Y atomically after the pre-pass
 * cleared it).
 */
#include "le_qmm_device.h"
#include "le_iq_tables.h"

typedef _Float16 le_h2 __attribute__((ext_vector_type(2)));
typedef _Float16 le_v8h __attribute__((ext_vector_type(8)));
typedef float le_v16f __attribute__((ext_vector_type(16)));

__device__ const u32 le_gq_iq2_grid[512] = LE_IQ2XXS_GRID_WORDS;
__device__ const u32 le_gq_iq3_grid[256] = LE_IQ3XXS_GRID_WORDS;
__device__ const u32 le_gq_iq2s_grid[2048] = LE_IQ2S_GRID_WORDS;

struct GqArgs {
    const u8 *w;
    const float *x;
    float *y;
    int rows, cols, m;
    int mp;     /* tokens rounded up to the largest token tile (the pre-pass pads with zeros) */
    int ksplit; /* K slices (blockIdx.y); > 1: partial sums into part (then le_gq_ksum), or, with no
                 * part buffer, atomic adds into y, cleared by the pre-pass */
    /* grouped form (le_mm_grouped): slot s multiplies weight ptrs[s] (or w + s * w_slot_bytes)
     * with the activation rows in_idx[i] of its pairs i in off[s] .. off[s+1], writing output rows
     * out_idx[i]; the plan kernel lists (slot, first pair) token tiles of bm pairs in the workspace */
    const u8 *const *ptrs;
    unsigned long long w_slot_bytes;
    const int *off, *in_idx, *out_idx;
    int nslot, maxt, bm, npair; /* grouped form: npair pairs (the pre-pass's grid) */
    float *part; /* [ksplit][m][rows] partial results of the K slices, or null */
    /* grouped form, dual: a second weight set (ptrs2 or w2, same type and shape) applied to the same
     * pairs, written to y2 (the MoE gate and up projections in one launch) */
    const u8 *const *ptrs2;
    const u8 *w2;
    float *y2;
    int dual, pad2;
    const float *up; /* non-null: the activation rows are silu(x) * up (the MoE down input) */
};

/* Workspace layout: A planes (mp * K halves), S records (mp/32 * nsb * SREC bytes), token scales
 * (mp floats). */
__host__ __device__ inline size_t gq_s_off(int mp, int K) { return (size_t)mp * K * 2; }
__host__ __device__ inline size_t gq_t_off(int mp, int K, int srec) { return gq_s_off(mp, K) + (size_t)(mp / 32) * (K / 256) * srec; }

/* Tiles of the grouped form: slot s has off[s+1] - off[s] pairs, split into tiles of bm, listed
 * slot by slot. Each wave derives what it needs from off itself (no planning launch): the slots'
 * counts are loaded 256 at a time, all in flight together, then scanned across the wave. */
__device__ __forceinline__ int gq_wave_scan(int v) { /* inclusive prefix sum over the wave, by DPP */
    v += __builtin_amdgcn_update_dpp(0, v, 0x111, 0xF, 0xF, true); /* row_shr:1 (rows of 16 lanes) */
    v += __builtin_amdgcn_update_dpp(0, v, 0x112, 0xF, 0xF, true); /* row_shr:2 */
    v += __builtin_amdgcn_update_dpp(0, v, 0x114, 0xF, 0xF, true); /* row_shr:4 */
    v += __builtin_amdgcn_update_dpp(0, v, 0x118, 0xF, 0xF, true); /* row_shr:8 */
    v += __builtin_amdgcn_update_dpp(0, v, 0x142, 0xA, 0xF, false); /* row_bcast:15 into rows 1, 3 */
    v += __builtin_amdgcn_update_dpp(0, v, 0x143, 0xC, 0xF, false); /* row_bcast:31 into rows 2, 3 */
    return v;
}
/* Walk the slots 256 at a time (every load of a round in flight together), each lane holding one
 * slot's first pair o0, its tile count c and the number of tiles before it; stop at the first
 * slot for which hit(o0, o1, first, c) holds on some lane. Returns that slot (or -1) and, through
 * the references, its first pair and first tile. Uniform over the wave. */
template <class Hit>
__device__ __forceinline__ int gq_slot_walk(const int *__restrict__ off, int nslot, int bm, Hit hit, int &o0_out, int &first_out) {
    const int lane = threadIdx.x & 63;
    int base = 0;
    for (int s0 = 0; s0 < nslot; s0 += 256) {
        int o0[4], o1[4];
#pragma unroll
        for (int q = 0; q < 4; q++) {
            const int s = min(s0 + 64 * q + lane, nslot - 1);
            o0[q] = off[s];
            o1[q] = off[s + 1];
        }
#pragma unroll
        for (int q = 0; q < 4; q++) {
            const bool in = s0 + 64 * q + lane < nslot;
            const int c = in ? (max(o1[q] - o0[q], 0) + bm - 1) / bm : 0, inc = gq_wave_scan(c), first = base + inc - c;
            const unsigned long long h = __ballot(in && c > 0 && hit(o0[q], o1[q], first, c));
            if (h) {
                const int l = __ffsll((long long)h) - 1;
                o0_out = __shfl(o0[q], l);
                first_out = __shfl(first, l);
                return s0 + 64 * q + l;
            }
            base += __shfl(inc, 63);
        }
    }
    return -1;
}
/* tile mt: its slot and first pair (false past the last tile) */
__device__ __forceinline__ bool gq_tile_of(const int *__restrict__ off, int nslot, int bm, int mt, int &slot, int &pair0) {
    int o0, first;
    slot = gq_slot_walk(off, nslot, bm, [mt](int, int, int f, int c) { return mt >= f && mt < f + c; }, o0, first);
    pair0 = o0 + (mt - first) * bm;
    return slot >= 0;
}

__device__ __forceinline__ le_h2 as_h2(u32 v) { return __builtin_bit_cast(le_h2, v); }
__device__ __forceinline__ u32 as_u32(le_h2 v) { return __builtin_bit_cast(u32, v); }
__device__ __forceinline__ le_v8h as_v8h(uint4 v) { return __builtin_bit_cast(le_v8h, v); }

/* bytes 0 and 2 (lo) or 1 and 3 (hi) of w, each under the fp16 exponent of 1024 */
__device__ __forceinline__ u32 h1024_02(u32 w) { return __builtin_amdgcn_perm(0x64646464u, w, 0x04020400u); }
__device__ __forceinline__ u32 h1024_13(u32 w) { return __builtin_amdgcn_perm(0x64646464u, w, 0x04030401u); }
/* byte i of w duplicated into both halves under the exponent of 1024 */
__device__ __forceinline__ u32 h1024_dup(u32 w, int i) {
    const u32 sel = 0x04000400u | (u32)(i * 0x00010001);
    return __builtin_amdgcn_perm(0x64646464u, w, sel);
}
/* (x & m) | c in one instruction: the compiler otherwise emits an and and an or, because a VOP3
 * instruction cannot carry the two literal constants; m and c stay in registers */
__device__ __forceinline__ u32 and_or(u32 x, u32 m, u32 c) {
    u32 r;
    __asm__("v_and_or_b32 %0, %1, %2, %3" : "=v"(r) : "v"(x), "v"(m), "v"(c));
    return r;
}
__device__ __forceinline__ u32 pk_fma(u32 a, u32 b, u32 c) {
    return as_u32(__builtin_elementwise_fma(as_h2(a), as_h2(b), as_h2(c)));
}
__device__ __forceinline__ u32 pk_add(u32 a, u32 b) { return as_u32(as_h2(a) + as_h2(b)); }
__device__ __forceinline__ u32 pk_mul(u32 a, u32 b) { return as_u32(as_h2(a) * as_h2(b)); }
__device__ __forceinline__ u32 h2dup(float f) {
    const _Float16 h = (_Float16)f;
    return as_u32((le_h2){h, h});
}

__device__ __forceinline__ void gq_barrier() {
    __asm__ volatile("" ::: "memory");
    __builtin_amdgcn_s_waitcnt(0xC07F); /* LDS only: the loads of later steps stay in flight */
    __builtin_amdgcn_s_barrier();
    __asm__ volatile("" ::: "memory");
}

template <int TM, int TN>
__device__ __forceinline__ void gq_mma(le_v16f (&d)[TM][TN], const le_v8h (&A)[TM], const le_v8h (&B)[TN], bool zero) {
#pragma unroll
    for (int i = 0; i < TM; i++)
#pragma unroll
        for (int k = 0; k < TN; k++) d[i][k] = __builtin_amdgcn_mfma_f32_32x32x16_f16(A[i], B[k], zero ? (le_v16f){} : d[i][k], 0, 0, 0);
}

/* ============================ per-type formats ============================
 * SBB: bytes per super-block; NCH 16-byte chunks per row and step, chunk k of half h read from
 * byte goff(k, h) of the super-block into byte loff(k) of the row's slot; SREC: bytes of sum
 * records per (32-token tile, super-block); EPI: 1 if the per-super-block epilogue is used. */
template <int TY>
struct GqF;

template <>
struct GqF<LE_TYPE_Q4_K> { /* slot: [0,16) header, [16,80) this half's 64 quant bytes */
    static constexpr int SBB = 144, NCH = 5, SLOT = 80, SREC = 1024, EPI = 1, TAB = 0;
    static constexpr bool ALIGNED = true;
    __device__ static int goff(int k, int h) { return k == 0 ? 0 : 16 + 64 * h + 16 * (k - 1); }
    __device__ static int loff(int k) { return 16 * k; }
};
template <>
struct GqF<LE_TYPE_Q6_K> { /* slot: [0,64) ql half, [64,96) qh half, [96,112) sc[16], [112,128) bytes 194..209 (d at 126);
                             * 144-byte stride: at 128 the 32 rows of a fragment read fell into two bank groups */
    static constexpr int SBB = 210, NCH = 8, SLOT = 144, SREC = 0, EPI = 1, TAB = 0;
    static constexpr bool ALIGNED = false;
    __device__ static int goff(int k, int h) {
        return k < 4 ? 64 * h + 16 * k : k < 6 ? 128 + 32 * h + 16 * (k - 4) : k == 6 ? 192 : 194;
    }
    __device__ static int loff(int k) { return 16 * k; }
};
template <>
struct GqF<LE_TYPE_Q5_K> { /* slot: [0,16) header, [16,48) qh (all 32 bytes), [48,112) this half's 64 quant bytes */
    static constexpr int SBB = 176, NCH = 7, SLOT = 112, SREC = 1024, EPI = 1, TAB = 0;
    static constexpr bool ALIGNED = true;
    __device__ static int goff(int k, int h) { return k < 3 ? 16 * k : 48 + 64 * h + 16 * (k - 3); }
    __device__ static int loff(int k) { return 16 * k; }
};
template <>
struct GqF<LE_TYPE_Q3_K> { /* slot: [0,32) the half's 32 quant bytes, [32,64) hmask, [64,80) bytes 94..109 (scales at
                             * 66..77, d at 78) */
    static constexpr int SBB = 110, NCH = 5, SLOT = 80, SREC = 0, EPI = 1, TAB = 0;
    static constexpr bool ALIGNED = false;
    __device__ static int goff(int k, int h) { return k < 2 ? 32 + 32 * h + 16 * k : k < 4 ? 16 * (k - 2) : 94; }
    __device__ static int loff(int k) { return 16 * k; }
};
template <>
struct GqF<LE_TYPE_IQ2_S> { /* slot: [0,16) the half's grid index bytes, [16,32) its sign bytes, [32,48) bytes 66..81
                             * (qh[8], scales[8]), [48,64) bytes 0..15 (d at 48) */
    static constexpr int SBB = 82, NCH = 4, SLOT = 80, SREC = 0, EPI = 1, TAB = 16384 + 4096;
    static constexpr bool ALIGNED = false;
    __device__ static int goff(int k, int h) { return k == 0 ? 2 + 16 * h : k == 1 ? 34 + 16 * h : k == 2 ? 66 : 0; }
    __device__ static int loff(int k) { return 16 * k; }
};
template <>
struct GqF<LE_TYPE_Q4_0> { /* 8 blocks of 18 bytes form a 144-byte super-block; slot: [16b, 16b+16) quant bytes of block b
                            * of the half, [64 + 16b] chunk starting at d_b; 144-byte stride */
    static constexpr int SBB = 144, NCH = 8, SLOT = 144, SREC = 0, EPI = 2, TAB = 0;
    static constexpr bool ALIGNED = false;
    __device__ static int goff(int k, int h) { return k < 4 ? 72 * h + 18 * k + 2 : 72 * h + 18 * (k - 4); }
    __device__ static int loff(int k) { return 16 * k; }
};
template <>
struct GqF<LE_TYPE_Q8_0> { /* slot: [32b, 32b+32) quants of block b of the half, [128 + 16b] chunk starting at d_b */
    static constexpr int SBB = 272, NCH = 12, SLOT = 192, SREC = 0, EPI = 2, TAB = 0;
    static constexpr bool ALIGNED = false;
    __device__ static int goff(int k, int h) {
        return k < 8 ? 136 * h + 34 * (k >> 1) + 2 + 16 * (k & 1) : 136 * h + 34 * (k - 8);
    }
    __device__ static int loff(int k) { return 16 * k; }
};
template <>
struct GqF<LE_TYPE_IQ2_XXS> { /* slot: [0,32) the half's four 8-byte block records, [32,48) bytes 0..15 (d at 32) */
    static constexpr int SBB = 66, NCH = 3, SLOT = 48, SREC = 0, EPI = 1, TAB = 4096 + 2048;
    static constexpr bool ALIGNED = false;
    __device__ static int goff(int k, int h) { return k < 2 ? 2 + 32 * h + 16 * k : 0; }
    __device__ static int loff(int k) { return 16 * k; }
};
template <>
struct GqF<LE_TYPE_IQ3_XXS> { /* slot: [0,32) the half's grid indices, [32,48) its four aux words, [48,64) bytes 0..15 (d at 48);
                                * 80-byte stride, as Q6_K's */
    static constexpr int SBB = 98, NCH = 4, SLOT = 80, SREC = 0, EPI = 1, TAB = 2048 + 2048;
    static constexpr bool ALIGNED = false;
    __device__ static int goff(int k, int h) { return k < 2 ? 2 + 32 * h + 16 * k : k == 2 ? 66 + 16 * h : 0; }
    __device__ static int loff(int k) { return 16 * k; }
};

/* IQ tables in LDS, in fragment order: grid entries as fp16 magnitudes (IQ2_XXS, IQ2_S: 8 per
 * entry, P8 order; IQ3_XXS: 4 per entry, order 0,2,1,3), then for each 7-bit sign index the 8 half
 * masks of ksign (src/quant.rs:57), or for IQ2_S for each sign byte its 8 bits (src/quant.rs:155-167),
 * 0x8000 where the value is negative, P8 order. */
template <int TY>
__device__ __forceinline__ void gq_tables(u8 *tab) {
    if constexpr (TY == LE_TYPE_IQ2_XXS || TY == LE_TYPE_IQ3_XXS || TY == LE_TYPE_IQ2_S) {
        constexpr int NG = TY == LE_TYPE_IQ2_S ? 1024 : 256, GB = TY == LE_TYPE_IQ3_XXS ? 8 : 16;
        for (int i = threadIdx.x; i < NG; i += blockDim.x) {
            if constexpr (TY != LE_TYPE_IQ3_XXS) {
                const u32 *gw = TY == LE_TYPE_IQ2_S ? le_gq_iq2s_grid : le_gq_iq2_grid;
                const u32 w0 = gw[2 * i], w1 = gw[2 * i + 1];
                *(uint4 *)(tab + GB * i) = make_uint4(pk_add(h1024_02(w0), 0xE400E400u), pk_add(h1024_13(w0), 0xE400E400u),
                                                      pk_add(h1024_02(w1), 0xE400E400u), pk_add(h1024_13(w1), 0xE400E400u));
            } else {
                const u32 w0 = le_gq_iq3_grid[i];
                *(uint2 *)(tab + GB * i) = make_uint2(pk_add(h1024_02(w0), 0xE400E400u), pk_add(h1024_13(w0), 0xE400E400u));
            }
        }
        /* IQ2_S stores its 8 sign bits explicitly: 256 entries indexed by the sign byte */
        constexpr int NS = TY == LE_TYPE_IQ2_S ? 256 : 128;
        u8 *sg = tab + NG * GB;
        for (int i = threadIdx.x; i < NS; i += blockDim.x) {
            const u32 ks = NS == 256 ? (u32)i : (u32)i | ((__builtin_popcount((u32)i) & 1u) << 7);
            u32 m[4];
#pragma unroll
            for (int p = 0; p < 4; p++) { /* halves 2p, 2p+1 hold values P8(2p), P8(2p+1) */
                const int v0 = (p & 2) * 2 + (p & 1), v1 = v0 + 2;
                m[p] = (((ks >> v0) & 1u) << 15) | (((ks >> v1) & 1u) << 31);
            }
            *(uint4 *)(sg + 16 * i) = make_uint4(m[0], m[1], m[2], m[3]);
        }
    }
}

/* ============================ activation pre-pass ============================ */
/* pre-pass: group g (8 values 8g..8g+7 = chunk g / 2, half g & 1) of padded token t, scaled by sc,
 * into the fp16 fragments A and (SK) the sum records S. The 2 or 4 lanes of one sum are g's
 * neighbours in the same wave, all inside or all outside the row (K % 256 == 0). */
template <int SK>
__device__ __forceinline__ void gq_xconvert(int g, float4 p, float4 q, float sc, int t, int K, _Float16 *A, u8 *S) {
    constexpr int SREC = SK == 1 ? 1024 : 2048;
    const int nsb = K >> 8, tile = t >> 5, tl = t & 31;
    float v[8] = {p.x * sc, p.y * sc, p.z * sc, p.w * sc, q.x * sc, q.y * sc, q.z * sc, q.w * sc};
    const le_h2 h0 = {(_Float16)v[0], (_Float16)v[2]}, h1 = {(_Float16)v[1], (_Float16)v[3]};
    const le_h2 h2 = {(_Float16)v[4], (_Float16)v[6]}, h3 = {(_Float16)v[5], (_Float16)v[7]};
    const size_t off = ((((size_t)tile * (K / 16) + (g >> 1)) * 2 + (g & 1)) * 32 + tl) * 8;
    *(LE_GLOBAL uint4 *)(A + off) = make_uint4(as_u32(h0), as_u32(h1), as_u32(h2), as_u32(h3));
    if constexpr (SK != 0) {
        /* g runs over consecutive lanes, so the groups of one sum are neighbouring lanes */
        /* sums of the fp16-rounded values the MFMA sees, so that the mins term cancels the
         * scale term's share of the rounding exactly: the result is then sum w * x~ with
         * error relative to sum |w x|, not to sum |sc q x| */
        float r[8];
#pragma unroll
        for (int i = 0; i < 8; i++) r[i] = (float)(_Float16)v[i];
        float s = ((r[0] + r[1]) + (r[2] + r[3])) + ((r[4] + r[5]) + (r[6] + r[7]));
        s += __shfl_xor(s, 1);
        if constexpr (SK == 1) s += __shfl_xor(s, 2);
        const int span = SK == 1 ? 4 : 2;
        if ((g & (span - 1)) == 0) {
            const int sb = g >> 5, j = (g & 31) / span; /* sum index within the super-block */
            const _Float16 hi = (_Float16)s, lo = (_Float16)(s - (float)hi);
            _Float16 *rec = (_Float16 *)(S + ((size_t)tile * nsb + sb) * SREC);
            /* position P8(j % 8) (P8 is its own inverse), the order of the B2 operand */
            const int pj = (j & 4) | ((j & 1) << 1) | ((j >> 1) & 1);
            if constexpr (SK == 1) { /* [hs][token][8]: hs 0 high halves, hs 1 low halves */
                rec[tl * 8 + pj] = hi;
                rec[256 + tl * 8 + pj] = lo;
            } else { /* [f][hs][token][8]: f 0 high, f 1 low; hs = j / 8 */
                rec[((j >> 3) * 32 + tl) * 8 + pj] = hi;
                rec[512 + ((j >> 3) * 32 + tl) * 8 + pj] = lo;
            }
        }
    }
}


/* One block of 256 threads per (padded) token, or per pair in the grouped form. SK: 0 no sums, 1 per-32 sums (Q4_K), 2 per-16
 * sums (Q6_K). */
template <int SK, bool GR = false>
__device__ __forceinline__ void gq_xprep_body(const GqArgs &a, u8 *ws) {
    __shared__ float red[4];
    const int K = a.cols, nsb = K >> 8, tid = threadIdx.x, lane = tid & 63;
    int t = blockIdx.x; /* padded token (grouped form: the pair's tile position, below) */
    if (!GR && a.ksplit > 1 && !a.part) { /* the slices add into y */
        const size_t ny = (size_t)a.m * a.rows, st = (size_t)gridDim.x * blockDim.x;
        size_t i = (size_t)blockIdx.x * blockDim.x + tid;
        if ((ny & 3) == 0 && ((size_t)a.y & 15) == 0)
            for (; i < ny / 4; i += st) ((float4 *)a.y)[i] = make_float4(0.f, 0.f, 0.f, 0.f);
        else
            for (; i < ny; i += st) a.y[i] = 0.f;
    }
    bool live = t < a.m;
    size_t src = t;
    if constexpr (GR) {
        /* one block per pair p (the grid is npair blocks): its slot s (off[s] <= p < off[s+1]),
         * then its position first_tile(s) * bm + (p - off[s]) among the tiles; the pair's token
         * index loads with the slots' offsets */
        const int p = blockIdx.x;
        const int srcp = a.in_idx[p];
        live = false;
        int o0, first;
        const int lo = gq_slot_walk(a.off, a.nslot, a.bm, [p](int b, int e, int, int) { return p >= b && p < e; }, o0, first);
        if (lo >= 0) {
            const int j = p - o0, tile = first + j / a.bm;
            if (tile < a.maxt) {
                live = true;
                t = tile * a.bm + j % a.bm;
                src = (size_t)srcp;
            }
        }
    }
    /* grouped form: a tile position without a pair writes nothing. Its activation rows, sums and
     * scale are never combined with a valid row (an MFMA output row depends on its own A row
     * only) and its outputs are not stored, so whatever the workspace holds there is harmless. */
    if (GR && !live) return;
    const LE_GLOBAL float *xr = (const LE_GLOBAL float *)(a.x + (live ? src : 0) * K);
    /* up to K = 16384 every thread keeps its groups' values in registers between the max and the
     * conversion: one read of the token, all of a thread's loads in flight at once */
    constexpr int XG = 8;
    const int ng = K / 8;
    const bool inreg = ng <= 256 * XG;
    float4 P[XG], Q[XG];
    float am = 0.f;
    if (inreg) {
#pragma unroll
        for (int i = 0; i < XG; i++) {
            const int g = tid + 256 * i;
            if (live && g < ng) {
                P[i] = ((const LE_GLOBAL float4 *)xr)[2 * g];
                Q[i] = ((const LE_GLOBAL float4 *)xr)[2 * g + 1];
                if (a.up) {
                    const LE_GLOBAL float4 *ur = (const LE_GLOBAL float4 *)(a.up + src * K);
                    P[i] = le_silu_mul4(P[i], ur[2 * g]);
                    Q[i] = le_silu_mul4(Q[i], ur[2 * g + 1]);
                }
            } else {
                P[i] = Q[i] = make_float4(0.f, 0.f, 0.f, 0.f);
            }
        }
#pragma unroll
        for (int i = 0; i < XG; i++) am = fmaxf(am, amax8(P[i], Q[i]));
    } else if (live) {
        for (int i = tid; i < K / 4; i += 256) {
            float4 v = ((const LE_GLOBAL float4 *)xr)[i];
            if (a.up) v = le_silu_mul4(v, ((const LE_GLOBAL float4 *)(a.up + src * K))[i]);
            am = fmaxf(am, fmaxf(fmaxf(fabsf(v.x), fabsf(v.y)), fmaxf(fabsf(v.z), fabsf(v.w))));
        }
    }
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) am = fmaxf(am, __shfl_xor(am, o));
    if (lane == 0) red[tid >> 6] = am;
    __syncthreads();
    am = fmaxf(fmaxf(red[0], red[1]), fmaxf(red[2], red[3]));
    int ex = 0;
    if (am > 0.f && am <= 3.0e38f) {
        (void)frexpf(am, &ex); /* am = f 2^ex, f in [0.5, 1) */
        ex = max(ex - 7, -100);
    }
    const float sc = live ? ldexpf(1.f, -ex) : 0.f;
    _Float16 *A = (_Float16 *)ws;
    u8 *S = ws + gq_s_off(a.mp, K);
    auto convert = [&](int g, float4 p, float4 q) { gq_xconvert<SK>(g, p, q, sc, t, K, A, S); };
    if (inreg) {
#pragma unroll
        for (int i = 0; i < XG; i++) {
            const int g = tid + 256 * i;
            if (g < ng) convert(g, P[i], Q[i]);
        }
    } else {
        for (int g = tid; g < ng; g += 256) {
            float4 p = make_float4(0.f, 0.f, 0.f, 0.f), q = p;
            if (live) {
                p = ((const LE_GLOBAL float4 *)xr)[2 * g];
                q = ((const LE_GLOBAL float4 *)xr)[2 * g + 1];
                if (a.up) {
                    const LE_GLOBAL float4 *ur = (const LE_GLOBAL float4 *)(a.up + src * K);
                    p = le_silu_mul4(p, ur[2 * g]);
                    q = le_silu_mul4(q, ur[2 * g + 1]);
                }
            }
            convert(g, p, q);
        }
    }
    if (tid == 0) {
        constexpr int srec = SK == 0 ? 0 : SK == 1 ? 1024 : 2048;
        ((float *)(ws + gq_t_off(a.mp, K, srec)))[t] = live ? ldexpf(1.f, ex) : 0.f;
    }
}

/* Grouped form, K <= 4096: one wave per pair (four per block), each lane holding up to 8 groups of
 * the pair's row; the largest magnitude by a wave reduction (no block barrier), then the same
 * conversion as gq_xprep_body, so the same bits. */
template <int SK>
__device__ __forceinline__ void gq_xprepw_body(const GqArgs &a, u8 *ws) {
    const int K = a.cols, lane = threadIdx.x & 63;
    const int p = (int)blockIdx.x * 4 + (int)(threadIdx.x >> 6);
    if (p >= a.npair) return; /* wave-uniform; no block barrier below */
    const int srcp = a.in_idx[p]; /* loads with the slots' offsets */
    int o0, first;
    const int lo = gq_slot_walk(a.off, a.nslot, a.bm, [p](int b, int e, int, int) { return p >= b && p < e; }, o0, first);
    if (lo < 0) return;
    const int j = p - o0, tile = first + j / a.bm;
    if (tile >= a.maxt) return;
    const int t = tile * a.bm + j % a.bm;
    const LE_GLOBAL float *xr = (const LE_GLOBAL float *)(a.x + (size_t)srcp * K);
    constexpr int XW = 8;
    const int ng = K / 8;
    float4 P[XW], Q[XW];
    float am = 0.f;
#pragma unroll
    for (int i = 0; i < XW; i++) {
        const int g = lane + 64 * i;
        if (g < ng) {
            P[i] = ((const LE_GLOBAL float4 *)xr)[2 * g];
            Q[i] = ((const LE_GLOBAL float4 *)xr)[2 * g + 1];
            if (a.up) {
                const LE_GLOBAL float4 *ur = (const LE_GLOBAL float4 *)(a.up + (size_t)srcp * K);
                P[i] = le_silu_mul4(P[i], ur[2 * g]);
                Q[i] = le_silu_mul4(Q[i], ur[2 * g + 1]);
            }
        } else {
            P[i] = Q[i] = make_float4(0.f, 0.f, 0.f, 0.f);
        }
        am = fmaxf(am, amax8(P[i], Q[i]));
    }
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) am = fmaxf(am, __shfl_xor(am, o));
    int ex = 0;
    if (am > 0.f && am <= 3.0e38f) {
        (void)frexpf(am, &ex); /* am = f 2^ex, f in [0.5, 1) */
        ex = max(ex - 7, -100);
    }
    const float sc = ldexpf(1.f, -ex);
    _Float16 *A = (_Float16 *)ws;
    u8 *S = ws + gq_s_off(a.mp, K);
#pragma unroll
    for (int i = 0; i < XW; i++) {
        const int g = lane + 64 * i;
        if (g < ng) gq_xconvert<SK>(g, P[i], Q[i], sc, t, K, A, S); /* ng % 32 == 0: a sum's lanes are all in or all out */
    }
    if (lane == 0) {
        constexpr int srec = SK == 0 ? 0 : SK == 1 ? 1024 : 2048;
        ((float *)(ws + gq_t_off(a.mp, K, srec)))[t] = ldexpf(1.f, ex);
    }
}

/* Direct-to-LDS loads (gfx950 global_load_lds_dwordx4): the load unit writes lane l's 16 bytes
 * at M0 + 16 l, so a wave's 64 chunks land as one contiguous 1 KB run with no registers held
 * while in flight. Issued from inline assembly so the compiler does not wait for them before
 * every LDS read; the kernel waits for them explicitly (the memory counter retires loads in
 * issue order). */
#pragma clang diagnostic push
#pragma clang diagnostic ignored "-Winline-asm"
__device__ __forceinline__ void gq_lds_dma16(const u8 *g, u32 lds_addr) {
    asm volatile("s_mov_b32 m0, %1\n\tglobal_load_lds_dwordx4 %0, off" ::"v"(g), "s"(lds_addr) : "memory", "m0");
}
#pragma clang diagnostic pop
template <int N>
__device__ __forceinline__ void gq_vm_wait() {
    static_assert(N >= 0 && N < 64, "vmcnt range");
    asm volatile("s_waitcnt vmcnt(%0)" ::"n"(N) : "memory");
}
__device__ __forceinline__ u32 gq_lds_addr(const void *p) { return (u32)(size_t)(const __attribute__((address_space(3))) void *)p; }

/* ============================ main kernel ============================ */
/* NA > 0: the activation fragments go straight to LDS, a ring of NA step slots (2: loaded one
 * step ahead, issued as the step starts, in the LDS the register-staged form uses for them; 3:
 * two steps ahead, with the weights' loads) instead of through registers; the weights keep the
 * register staging. Every launched kernel uses NA = 2 (measured against registers at M=512: Q4_K
 * 109 -> 95 us, Q6_K 147 -> 114, Q8_0 252 -> 230, IQ2_XXS 98 -> 92; the three-slot ring 100 us for
 * Q4_K); the results are the same bits in every form. */
template <int TY, int WM, int WN, int TM, int TN, bool GR = false, int NA = 0>
__device__ __forceinline__ void gq_body(const GqArgs &a, const u8 *ws) {
    using F = GqF<TY>;
    constexpr bool AD = NA > 0;
    static_assert(NA == 0 || NA == 2 || NA == 3, "activation ring of 2 or 3 slots");
    constexpr int BM = 32 * TM * WM, BN = 32 * TN * WN, NT = 64 * WM * WN;
    constexpr int WB = BN * F::SLOT, AB = BM * 256, BUF = AD ? WB : WB + AB;
    constexpr int SBYTES = F::SREC ? (BM / 32) * F::SREC : 0; /* per super-block */
    constexpr int NWC = (BN * F::NCH + NT - 1) / NT, NAC = AB / 16 / NT, NSC = (SBYTES / 16 + NT - 1) / NT;
    static_assert(AB / 16 % NT == 0, "activation chunks must divide over the threads");
    extern __shared__ uint4 smem[];
    u8 *lds = (u8 *)smem;
    u8 *Aring = lds + 2 * BUF;          /* NA > 0: [NA][AB] activation step slots */
    u8 *Sl = lds + 2 * BUF + NA * AB;  /* [2][SBYTES] sum records, by super-block parity */
    u8 *tab = Sl + 2 * SBYTES;          /* IQ tables */

    const int K = a.cols, nsb = K >> 8;
    const int NTR1 = (a.rows + BN - 1) / BN, NTR = GR && a.dual ? 2 * NTR1 : NTR1, MT = GR ? a.maxt : (a.m + BM - 1) / BM;
    /* 8 or more row tiles: blocks of one row tile (its token tiles) share blockIdx % 8, the XCD
     * and its L2; fewer: row tiles vary fastest, so consecutive blocks spread over every XCD */
    const int id = blockIdx.x, j = id >> 3;
    const int mt = NTR >= 8 ? j % MT : id / NTR, nt = NTR >= 8 ? (j / MT) * 8 + (id & 7) : id % NTR;
    if (nt >= NTR || mt >= MT) return; /* uniform over the block */
    const bool second = nt >= NTR1; /* dual grouped form: a row tile of the second weight set */
    const int nb = (second ? nt - NTR1 : nt) * BN, mb = mt * BM;
    /* tokens of this tile: M = all tokens (plain), or the tile's pairs (grouped: rows of its slot) */
    int M = a.m, pair0 = 0;
    const u8 *Wsrc = a.w;
    if constexpr (GR) {
        int sl;
        if (!gq_tile_of(a.off, a.nslot, a.bm, mt, sl, pair0)) return; /* uniform: past the last tile */
        M = mb + min(BM, a.off[sl + 1] - pair0); /* token t of the tile is valid while t < M */
        if (second)
            Wsrc = a.ptrs2 ? a.ptrs2[sl] : a.w2 + (size_t)sl * a.w_slot_bytes;
        else
            Wsrc = a.ptrs ? a.ptrs[sl] : a.w + (size_t)sl * a.w_slot_bytes;
    }
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int wm = wave / WN, wn = wave % WN;
    const size_t rb = (size_t)nsb * F::SBB;
    const int sb0 = blockIdx.y * (nsb / a.ksplit), sb1 = sb0 + nsb / a.ksplit;
    const int nstep = 2 * sb1;
    const u8 *Ag = ws;
    const u8 *Sg = ws + gq_s_off(a.mp, K);
    const float *tsc = (const float *)(ws + gq_t_off(a.mp, K, F::SREC));

    if constexpr (F::TAB > 0) gq_tables<TY>(tab);

    struct Set {
        uint4 w[NWC], x[AD ? 1 : NAC], s[NSC > 0 ? NSC : 1];
    };
    /* every load is unconditional (addresses clamped) so the waits before staging count exactly
     * the loads of the step being staged; steps past the slice re-read the last one. Even steps
     * (first halves of super-blocks, always set RB) also bring the super-block's sum records. */
    /* per-thread 32-bit load offsets, computed once (the host keeps a slice's weights and the
     * activation planes below 4 GiB): so each load is a scalar base plus one of these */
    u32 wo0[NWC], wo1[NWC], xo[NAC], so[NSC > 0 ? NSC : 1];
    bool xlive[NAC];
#pragma unroll
    for (int i = 0; i < NWC; i++) {
        const int c = min(tid + NT * i, BN * F::NCH - 1), row = c / F::NCH, k = c - row * F::NCH;
        const u32 base = (u32)min(nb + row, a.rows - 1) * (u32)rb;
        wo0[i] = base + F::goff(k, 0);
        wo1[i] = base + F::goff(k, 1);
    }
#pragma unroll
    for (int i = 0; i < NAC; i++) {
        const int c = tid + NT * i, tl = c >> 9, off = c & 511; /* 512 chunks = 8 KB per 32-token tile */
        xo[i] = (u32)(mb / 32 + tl) * (u32)(K / 16) * 1024u + 16u * off;
        xlive[i] = mb + 32 * tl + (off & 31) < M; /* fragment lane l holds token l % 32 */
    }
#pragma unroll
    for (int i = 0; i < (NSC > 0 ? NSC : 1); i++) {
        const int c = min(tid + NT * i, SBYTES > 0 ? SBYTES / 16 - 1 : 0), tl = c / (F::SREC > 0 ? F::SREC / 16 : 1);
        const int off = c - tl * (F::SREC > 0 ? F::SREC / 16 : 1);
        so[i] = (u32)(mb / 32 + tl) * (u32)nsb * (u32)F::SREC + 16u * off;
    }
    auto issue = [&](int s_, Set &R, bool even) {
        const int s = min(s_, nstep - 1), sb = s >> 1, h = s & 1;
        const u8 *w0 = Wsrc + (size_t)sb * F::SBB;
#pragma unroll
        for (int i = 0; i < NWC; i++) {
            const u8 *p = w0 + (h ? wo1[i] : wo0[i]);
            R.w[i] = F::ALIGNED ? ldg16c(p) : ldg16u(p); /* cached: the next step reads the same lines */
        }
        if constexpr (!AD) {
            const u8 *x0 = Ag + (size_t)(sb * 16 + 8 * h) * 1024;
#pragma unroll
            for (int i = 0; i < NAC; i++) R.x[i] = ldg16c(x0 + xo[i]);
        }
        if (SBYTES > 0 && even) {
            const u8 *s0p = Sg + (size_t)sb * F::SREC;
#pragma unroll
            for (int i = 0; i < NSC; i++) R.s[i] = ldg16c(s0p + so[i]);
        }
    };
    auto stage = [&](int s, const Set &R, bool even) {
        const int sb = s >> 1, h = s & 1;
        u8 *B = lds + h * BUF;
#pragma unroll
        for (int i = 0; i < NWC; i++) {
            const int c = tid + NT * i;
            if (NWC * NT > BN * F::NCH && c >= BN * F::NCH) break;
            const int row = c / F::NCH, k = c - row * F::NCH;
            *(uint4 *)(B + row * F::SLOT + F::loff(k)) = R.w[i];
        }
        if constexpr (!AD) {
#pragma unroll
            for (int i = 0; i < NAC; i++) ((uint4 *)(B + WB))[tid + NT * i] = R.x[i];
        }
        if constexpr (SBYTES > 0) {
            if (even) {
#pragma unroll
                for (int i = 0; i < NSC; i++) {
                    const int c = tid + NT * i;
                    if (NSC * NT > SBYTES / 16 && c >= SBYTES / 16) break;
                    ((uint4 *)(Sl + (sb & 1) * SBYTES))[c] = R.s[i];
                }
            }
        }
    };

    /* NA > 0: step s_'s activation fragments into ring slot s_ % NA (steps past the slice re-read
     * the last one into a slot that is no longer read) */
    auto dma = [&](int s_) {
        if constexpr (AD) {
            const int s = min(s_, nstep - 1), sb = s >> 1, h = s & 1;
            const u8 *x0 = Ag + (size_t)(sb * 16 + 8 * h) * 1024;
            u8 *dst = Aring + (s_ % (NA > 0 ? NA : 1)) * AB + 64 * 16 * wave;
#pragma unroll
            for (int i = 0; i < NAC; i++) { /* the LDS address is uniform over the wave (M0) */
                const u32 la = __builtin_amdgcn_readfirstlane(gq_lds_addr(dst + NT * 16 * i));
                /* lanes of tokens past the tile's last one load nothing: their LDS bytes only
                 * reach output rows that are never stored, and a 128-byte line holds 8 tokens,
                 * so a sparse tile (grouped form) fetches a quarter of the lines per valid 8 */
                if (xlive[i]) gq_lds_dma16(x0 + xo[i], la);
            }
        }
    };

    le_v16f acc[TM][TN], d1[TM][TN];
#pragma unroll
    for (int i = 0; i < TM; i++)
#pragma unroll
        for (int k = 0; k < TN; k++) acc[i][k] = d1[i][k] = (le_v16f){};

    const int n = lane & 31, hs = lane >> 5;
    int rowS[TN]; /* Q8_0 / Q4_0: the accumulator holds the row's sum times 2^rowS */
#pragma unroll
    for (int k = 0; k < TN; k++) rowS[k] = 127;
    Set RA, RB; /* RA holds odd (h = 1) steps, RB even ones */
    const int s0 = 2 * sb0;
    /* the loads must reach the memory pipeline in step order (RA's before RB's, as in the loop),
     * or the wait at the loop head would have to cover both sets: no reordering across issues */
    issue(s0, RB, true);
    dma(s0);
    stage(s0, RB, true);
    issue(s0 + 1, RA, false);
    __builtin_amdgcn_sched_barrier(0);
    if constexpr (NA == 3) dma(s0 + 1);
    issue(s0 + 2, RB, true);
    __builtin_amdgcn_sched_barrier(0);

    for (int sb = sb0; sb < sb1; sb++) {
#pragma unroll
        for (int h = 0; h < 2; h++) {
            const int s = 2 * sb + h;
            /* this step's activations: younger are the loads of steps s + 2 (weights) and, with
             * three slots, s + 1 (activations) */
            if constexpr (NA == 3) {
                if (h == 0) gq_vm_wait<NWC + NAC + (SBYTES > 0 ? NSC : 0)>();
                else gq_vm_wait<NWC + NAC>();
            } else if constexpr (NA == 2) {
                if (h == 0) gq_vm_wait<NWC + (SBYTES > 0 ? NSC : 0)>();
                else gq_vm_wait<NWC>();
            }
            gq_barrier(); /* step s is staged; every wave is done with step s-1's buffer */
            if constexpr (NA == 2) dma(s + 1); /* slot (s + 1) % 2 was last read in step s - 1 */
            const u8 *Wb = lds + h * BUF, *Ab = (AD ? Aring + (s % (NA > 0 ? NA : 1)) * AB : Wb + WB) + (wm * TM) * 8192;
            const u8 *rs[TN];
#pragma unroll
            for (int k = 0; k < TN; k++) rs[k] = Wb + (wn * TN * 32 + 32 * k + n) * F::SLOT;
            /* A fragment of tile i, chunk c */
            auto afrag = [&](int c, le_v8h (&A)[TM]) {
#pragma unroll
                for (int i = 0; i < TM; i++) A[i] = as_v8h(*(const uint4 *)(Ab + i * 8192 + c * 1024 + lane * 16));
            };
            /* stage the next step and issue the loads two steps ahead once this step's first
             * fragments are under way */
            auto pipe = [&]() {
                /* unconditional (a branch here would make the compiler wait for every load in
                 * flight): past the slice's end this stages a re-read into the buffer that is
                 * no longer read */
                if (h) stage(s + 1, RB, true);
                else stage(s + 1, RA, false);
                __builtin_amdgcn_sched_barrier(0);
                if (h) issue(s + 3, RB, true);
                else issue(s + 3, RA, false);
                if constexpr (NA == 3) dma(s + 2); /* slot (s + 2) % 3 was last read in step s - 1 */
                __builtin_amdgcn_sched_barrier(0);
            };
            if constexpr (TY == LE_TYPE_Q4_K) {
                const u32 mlo = 0x000F000Fu, mhi = 0x00F000F0u, c1024 = 0x64006400u;
                uint4 hd[TN];
                u32 scw[TN];
#pragma unroll
                for (int k = 0; k < TN; k++) {
                    hd[k] = *(const uint4 *)rs[k];
                    scw[k] = h ? ((hd[k].w & 0x0F0F0F0Fu) | ((hd[k].y >> 2) & 0x30303030u)) : (hd[k].y & 0x3F3F3F3Fu);
                }
#pragma unroll
                for (int g = 0; g < 2; g++) {
                    uint4 kc[TN]; /* (sc_lo, -1024 sc_lo, sc_hi / 16, -64 sc_hi) as duplicated halves */
#pragma unroll
                    for (int k = 0; k < TN; k++) {
                        const u32 slo = pk_add(h1024_dup(scw[k], 2 * g), 0xE400E400u);
                        const u32 shi = pk_add(h1024_dup(scw[k], 2 * g + 1), 0xE400E400u);
                        kc[k] = make_uint4(slo, pk_mul(slo, 0xE400E400u), pk_mul(shi, 0x2C002C00u), pk_mul(shi, 0xD400D400u));
                    }
#pragma unroll
                    for (int c1 = 0; c1 < 2; c1++) {
                        const int c = 4 * g + c1;
                        le_v8h blo[TN], bhi[TN];
#pragma unroll
                        for (int k = 0; k < TN; k++) {
                            const uint2 q = *(const uint2 *)(rs[k] + 16 + 32 * g + 16 * c1 + 8 * hs);
                            const u32 ws_[2] = {q.x, q.y};
                            u32 l[4], hh[4];
#pragma unroll
                            for (int e = 0; e < 2; e++) {
                                const u32 x = ws_[e], x8 = x >> 8;
                                l[2 * e] = pk_fma(and_or(x, mlo, c1024), kc[k].x, kc[k].y);
                                l[2 * e + 1] = pk_fma(and_or(x8, mlo, c1024), kc[k].x, kc[k].y);
                                hh[2 * e] = pk_fma(and_or(x, mhi, c1024), kc[k].z, kc[k].w);
                                hh[2 * e + 1] = pk_fma(and_or(x8, mhi, c1024), kc[k].z, kc[k].w);
                            }
                            blo[k] = as_v8h(make_uint4(l[0], l[1], l[2], l[3]));
                            bhi[k] = as_v8h(make_uint4(hh[0], hh[1], hh[2], hh[3]));
                        }
                        le_v8h A[TM];
                        afrag(c, A);
                        gq_mma(d1, A, blo, h == 0 && c == 0);
                        afrag(c + 2, A);
                        gq_mma(d1, A, bhi, false);
                        if (g == 0 && c1 == 0) pipe();
                    }
                }
            } else if constexpr (TY == LE_TYPE_Q6_K) {
                /* chunk c of half h uses sc[8h + c], as sc / 64 duplicated (exact) */
                u32 sp[TN][8];
#pragma unroll
                for (int k = 0; k < TN; k++) {
                    const uint2 sv = *(const uint2 *)(rs[k] + 96 + 8 * h);
                    const u32 sw[2] = {sv.x ^ 0x80808080u, sv.y ^ 0x80808080u};
#pragma unroll
                    for (int c = 0; c < 8; c++)
                        sp[k][c] = pk_mul(pk_add(h1024_dup(sw[c >> 2], c & 3), 0xE480E480u), 0x24002400u); /* (byte - 1152) / 64 */
                }
#pragma unroll
                for (int c1 = 0; c1 < 2; c1++) {
                    const int l0 = 16 * c1 + 8 * hs;
                    uint2 qa[TN], qb[TN], qh[TN];
#pragma unroll
                    for (int k = 0; k < TN; k++) {
                        qa[k] = *(const uint2 *)(rs[k] + l0);
                        qb[k] = *(const uint2 *)(rs[k] + 32 + l0);
                        qh[k] = *(const uint2 *)(rs[k] + 64 + l0);
                    }
#pragma unroll
                    for (int q = 0; q < 4; q++) {
                        const int c = 2 * q + c1;
                        le_v8h B[TN];
#pragma unroll
                        for (int k = 0; k < TN; k++) {
                            const uint2 src = q & 1 ? qb[k] : qa[k];
                            const u32 sx = src.x >> (4 * (q >> 1)), sy = src.y >> (4 * (q >> 1));
                            const u32 hx = q < 2 ? (qh[k].x << (4 - 2 * q)) : (qh[k].x >> (2 * q - 4));
                            const u32 hy = q < 2 ? (qh[k].y << (4 - 2 * q)) : (qh[k].y >> (2 * q - 4));
                            const u32 vx = and_or(sx, 0x0F0F0F0Fu, hx & 0x30303030u);
                            const u32 vy = and_or(sy, 0x0F0F0F0Fu, hy & 0x30303030u);
                            /* (1024 + q6) - 1056 = q6 - 32 exactly, then one rounding by sc / 64 */
                            const u32 sc = sp[k][c];
                            B[k] = as_v8h(make_uint4(pk_mul(pk_add(h1024_02(vx), 0xE420E420u), sc), pk_mul(pk_add(h1024_13(vx), 0xE420E420u), sc),
                                                     pk_mul(pk_add(h1024_02(vy), 0xE420E420u), sc), pk_mul(pk_add(h1024_13(vy), 0xE420E420u), sc)));
                        }
                        le_v8h A[TM];
                        afrag(c, A);
                        gq_mma(d1, A, B, h == 0 && c == 0);
                        if (c1 == 0 && q == 0) pipe();
                    }
                }
            } else if constexpr (TY == LE_TYPE_Q8_0 || TY == LE_TYPE_Q4_0) {
                /* per-32 scales inside the codes: fp16(q * d_b 2^S) (one rounding), with a power of two
                 * 2^S per row that keeps every code inside the fp16 range whatever the scales are:
                 * S only decreases, to the value that puts the step's largest |d_b| 2^S in
                 * [128, 256) (|q| <= 128) when that is below the current one, and the accumulator
                 * is then rescaled (a wave-uniform branch, taken at the first step and
                 * otherwise only when a row's scales grow); the result is multiplied by 2^-S */
                constexpr int DO = TY == LE_TYPE_Q8_0 ? 128 : 64, QB = TY == LE_TYPE_Q8_0 ? 32 : 16;
                u32 r[TN][4];
                bool grow = false;
                int sn[TN];
#pragma unroll
                for (int k = 0; k < TN; k++) {
                    u32 dv[4], mx = 0;
#pragma unroll
                    for (int b = 0; b < 4; b++) {
                        dv[b] = *(const u32 *)(rs[k] + DO + 16 * b) & 0xFFFFu;
                        mx = max(mx, dv[b] & 0x7FFFu);
                    }
                    const int e = max((int)(mx >> 10), 1); /* biased fp16 exponent of the largest |d_b| */
                    sn[k] = min(rowS[k], 22 - e);
                    grow |= sn[k] != rowS[k];
                    const float up_ = __builtin_bit_cast(float, (u32)(127 + sn[k]) << 23);
#pragma unroll
                    for (int b = 0; b < 4; b++) r[k][b] = h2dup(h2f(dv[b]) * up_);
                }
                if (__any(grow)) {
#pragma unroll
                    for (int k = 0; k < TN; k++) {
                        const float f = ldexpf(1.f, sn[k] - rowS[k]);
                        rowS[k] = sn[k];
#pragma unroll
                        for (int i = 0; i < TM; i++)
#pragma unroll
                            for (int e = 0; e < 16; e++) acc[i][k][e] *= f;
                    }
                }
#pragma unroll
                for (int b = 0; b < 4; b++) {
#pragma unroll
                    for (int c1 = 0; c1 < 2; c1++) {
                        const int c = 2 * b + c1;
                        le_v8h B[TN];
#pragma unroll
                        for (int k = 0; k < TN; k++) {
                            if constexpr (TY == LE_TYPE_Q8_0) {
                                const uint2 q = *(const uint2 *)(rs[k] + QB * b + 16 * c1 + 8 * hs);
                                const u32 x = q.x ^ 0x80808080u, y = q.y ^ 0x80808080u; /* q + 128 */
                                B[k] = as_v8h(make_uint4(pk_mul(pk_add(h1024_02(x), 0xE480E480u), r[k][b]), pk_mul(pk_add(h1024_13(x), 0xE480E480u), r[k][b]),
                                                         pk_mul(pk_add(h1024_02(y), 0xE480E480u), r[k][b]), pk_mul(pk_add(h1024_13(y), 0xE480E480u), r[k][b])));
                            } else { /* value j < 16: low nibble of byte j; j >= 16: high nibble of byte j - 16 */
                                const uint2 q = *(const uint2 *)(rs[k] + QB * b + 8 * hs);
                                const u32 x = (q.x >> (4 * c1)) & 0x0F0F0F0Fu, y = (q.y >> (4 * c1)) & 0x0F0F0F0Fu;
                                B[k] = as_v8h(make_uint4(pk_mul(pk_add(h1024_02(x), 0xE408E408u), r[k][b]), pk_mul(pk_add(h1024_13(x), 0xE408E408u), r[k][b]),
                                                         pk_mul(pk_add(h1024_02(y), 0xE408E408u), r[k][b]), pk_mul(pk_add(h1024_13(y), 0xE408E408u), r[k][b])));
                            }
                        }
                        le_v8h A[TM];
                        afrag(c, A);
                        gq_mma(acc, A, B, false);
                        if (c == 0) pipe();
                    }
                }
            } else if constexpr (TY == LE_TYPE_Q5_K) {
                /* the Q4_K decode with the fifth bit of each code from qh: bit 2G (low nibbles of group
                 * G) and 2G + 1 (high nibbles) of byte l (src/quant.rs:83-95); codes sc * q <= 1953 */
                u32 scw[TN];
#pragma unroll
                for (int k = 0; k < TN; k++) {
                    const uint4 hd = *(const uint4 *)rs[k];
                    scw[k] = h ? ((hd.w & 0x0F0F0F0Fu) | ((hd.y >> 2) & 0x30303030u)) : (hd.y & 0x3F3F3F3Fu);
                }
#pragma unroll
                for (int g = 0; g < 2; g++) {
                    const int G = 2 * h + g;
                    uint4 kc[TN]; /* (sc_lo, -1024 sc_lo, sc_hi, -1024 sc_hi) as duplicated halves */
#pragma unroll
                    for (int k = 0; k < TN; k++) {
                        const u32 slo = pk_add(h1024_dup(scw[k], 2 * g), 0xE400E400u);
                        const u32 shi = pk_add(h1024_dup(scw[k], 2 * g + 1), 0xE400E400u);
                        kc[k] = make_uint4(slo, pk_mul(slo, 0xE400E400u), shi, pk_mul(shi, 0xE400E400u));
                    }
#pragma unroll
                    for (int c1 = 0; c1 < 2; c1++) {
                        const int c = 4 * g + c1;
                        le_v8h blo[TN], bhi[TN];
#pragma unroll
                        for (int k = 0; k < TN; k++) {
                            const uint2 q = *(const uint2 *)(rs[k] + 48 + 32 * g + 16 * c1 + 8 * hs);
                            const uint2 qh = *(const uint2 *)(rs[k] + 16 + 16 * c1 + 8 * hs);
                            const u32 lx = and_or(q.x, 0x0F0F0F0Fu, ((qh.x >> (2 * G)) << 4) & 0x10101010u);
                            const u32 ly = and_or(q.y, 0x0F0F0F0Fu, ((qh.y >> (2 * G)) << 4) & 0x10101010u);
                            const u32 hx = and_or(q.x >> 4, 0x0F0F0F0Fu, ((qh.x >> (2 * G + 1)) << 4) & 0x10101010u);
                            const u32 hy = and_or(q.y >> 4, 0x0F0F0F0Fu, ((qh.y >> (2 * G + 1)) << 4) & 0x10101010u);
                            blo[k] = as_v8h(make_uint4(pk_fma(h1024_02(lx), kc[k].x, kc[k].y), pk_fma(h1024_13(lx), kc[k].x, kc[k].y),
                                                       pk_fma(h1024_02(ly), kc[k].x, kc[k].y), pk_fma(h1024_13(ly), kc[k].x, kc[k].y)));
                            bhi[k] = as_v8h(make_uint4(pk_fma(h1024_02(hx), kc[k].z, kc[k].w), pk_fma(h1024_13(hx), kc[k].z, kc[k].w),
                                                       pk_fma(h1024_02(hy), kc[k].z, kc[k].w), pk_fma(h1024_13(hy), kc[k].z, kc[k].w)));
                        }
                        le_v8h A[TM];
                        afrag(c, A);
                        gq_mma(d1, A, blo, h == 0 && c == 0);
                        afrag(c + 2, A);
                        gq_mma(d1, A, bhi, false);
                        if (g == 0 && c1 == 0) pipe();
                    }
                }
            } else if constexpr (TY == LE_TYPE_Q3_K) {
                /* value 128h + 32s + l: code ((qs[32h + l] >> 2s) & 3) - (hm[l] bit 4h + s ? 0 : 4), scale
                 * 8h + c of the sixteen signed 6-bit scales (src/quant.rs:113-126); |code * scale| <= 128, exact */
                u32 sp[TN][8];
#pragma unroll
                for (int k = 0; k < TN; k++) {
                    const uint4 sw = *(const uint4 *)(rs[k] + 64); /* scale byte i at slot byte 66 + i */
                    const u32 s0 = __builtin_amdgcn_alignbyte(sw.y, sw.x, 2), s1 = __builtin_amdgcn_alignbyte(sw.z, sw.y, 2);
                    const u32 s2 = __builtin_amdgcn_alignbyte(sw.w, sw.z, 2);
                    /* scale i = 8h + c: low 4 bits from byte c (h = 0) or its high nibble (h = 1), bits 4-5
                     * from byte 8 + c % 4 at bit 2 (2h + c / 4) */
                    const u32 v0 = ((s0 >> (4 * h)) & 0x0F0F0F0Fu) | (((s2 >> (4 * h)) & 0x03030303u) << 4);
                    const u32 v1 = ((s1 >> (4 * h)) & 0x0F0F0F0Fu) | (((s2 >> (4 * h + 2)) & 0x03030303u) << 4);
#pragma unroll
                    for (int c = 0; c < 8; c++) sp[k][c] = pk_add(h1024_dup(c < 4 ? v0 : v1, c & 3), 0xE420E420u); /* byte - 32 */
                }
                uint2 qa[TN][2], hm[TN][2];
#pragma unroll
                for (int k = 0; k < TN; k++)
#pragma unroll
                    for (int p = 0; p < 2; p++) {
                        qa[k][p] = *(const uint2 *)(rs[k] + 16 * p + 8 * hs);
                        hm[k][p] = *(const uint2 *)(rs[k] + 32 + 16 * p + 8 * hs);
                    }
#pragma unroll
                for (int c = 0; c < 8; c++) {
                    const int sub = c >> 1, p = c & 1;
                    le_v8h B[TN];
#pragma unroll
                    for (int k = 0; k < TN; k++) {
                        const u32 vx = and_or(qa[k][p].x >> (2 * sub), 0x03030303u, ((hm[k][p].x >> (4 * h + sub)) & 0x01010101u) << 2);
                        const u32 vy = and_or(qa[k][p].y >> (2 * sub), 0x03030303u, ((hm[k][p].y >> (4 * h + sub)) & 0x01010101u) << 2);
                        const u32 sc = sp[k][c];
                        B[k] = as_v8h(make_uint4(pk_mul(pk_add(h1024_02(vx), 0xE404E404u), sc), pk_mul(pk_add(h1024_13(vx), 0xE404E404u), sc),
                                                 pk_mul(pk_add(h1024_02(vy), 0xE404E404u), sc), pk_mul(pk_add(h1024_13(vy), 0xE404E404u), sc)));
                    }
                    le_v8h A[TM];
                    afrag(c, A);
                    gq_mma(d1, A, B, h == 0 && c == 0);
                    if (c == 0) pipe();
                }
            } else if constexpr (TY == LE_TYPE_IQ2_S) {
                /* block 4h + b, 8-value group l: grid index qs[4b + l] | bits 2l, 2l+1 of qh[b] as bits 8-9,
                 * signs = byte 4b + l, factor 2 s + 1 of the block's nibble l / 2 (src/quant.rs:155-167) */
                const u8 *sgt = tab + 1024 * 16;
                u32 qhw[TN], scw[TN];
#pragma unroll
                for (int k = 0; k < TN; k++) {
                    qhw[k] = *(const u32 *)(rs[k] + 32 + 4 * h);
                    scw[k] = *(const u32 *)(rs[k] + 40 + 4 * h);
                }
#pragma unroll
                for (int b = 0; b < 4; b++) {
                    u32 qi[TN], sg[TN];
#pragma unroll
                    for (int k = 0; k < TN; k++) {
                        qi[k] = *(const u32 *)(rs[k] + 4 * b);
                        sg[k] = *(const u32 *)(rs[k] + 16 + 4 * b);
                    }
#pragma unroll
                    for (int c1 = 0; c1 < 2; c1++) {
                        const int c = 2 * b + c1, l = 2 * c1 + hs;
                        le_v8h B[TN];
#pragma unroll
                        for (int k = 0; k < TN; k++) {
                            const u32 qhb = (qhw[k] >> (8 * b)) & 0xFFu;
                            const u32 gi = ((qi[k] >> (8 * l)) & 255u) | ((qhb << (8 - 2 * l)) & 0x300u);
                            const u32 f = pk_add(h1024_dup(2u * ((scw[k] >> (8 * b + 4 * c1)) & 15u) + 1u, 0), 0xE400E400u);
                            const uint4 g = *(const uint4 *)(tab + 16 * gi);
                            const uint4 m = *(const uint4 *)(sgt + 16 * ((sg[k] >> (8 * l)) & 255u));
                            B[k] = as_v8h(make_uint4(pk_mul(g.x, f) ^ m.x, pk_mul(g.y, f) ^ m.y, pk_mul(g.z, f) ^ m.z, pk_mul(g.w, f) ^ m.w));
                        }
                        le_v8h A[TM];
                        afrag(c, A);
                        gq_mma(d1, A, B, h == 0 && c == 0);
                        if (c == 0) pipe();
                    }
                }
            } else if constexpr (TY == LE_TYPE_IQ2_XXS || TY == LE_TYPE_IQ3_XXS) {
                constexpr int GB = TY == LE_TYPE_IQ2_XXS ? 16 : 8;
                const u8 *sgt = tab + 256 * GB;
#pragma unroll
                for (int b = 0; b < 4; b++) {
                    uint2 rec[TN];
                    u32 aux[TN], f[TN];
#pragma unroll
                    for (int k = 0; k < TN; k++) {
                        if constexpr (TY == LE_TYPE_IQ2_XXS) {
                            rec[k] = *(const uint2 *)(rs[k] + 8 * b);
                            aux[k] = rec[k].y;
                        } else {
                            rec[k] = *(const uint2 *)(rs[k] + 8 * b);
                            aux[k] = *(const u32 *)(rs[k] + 32 + 4 * b);
                        }
                        f[k] = pk_add(h1024_dup(2u * (aux[k] >> 28) + 1u, 0), 0xE400E400u); /* (2s+1) */
                    }
#pragma unroll
                    for (int c1 = 0; c1 < 2; c1++) {
                        const int c = 2 * b + c1, l = 2 * c1 + hs;
                        le_v8h B[TN];
#pragma unroll
                        for (int k = 0; k < TN; k++) {
                            const uint4 m = *(const uint4 *)(sgt + 16 * ((aux[k] >> (7 * l)) & 127u));
                            uint4 g;
                            if constexpr (TY == LE_TYPE_IQ2_XXS) {
                                g = *(const uint4 *)(tab + GB * ((rec[k].x >> (8 * l)) & 255u));
                            } else {
                                const u32 iw = l < 2 ? rec[k].x : rec[k].y, sh = 16 * (l & 1);
                                const uint2 g0 = *(const uint2 *)(tab + GB * ((iw >> sh) & 255u));
                                const uint2 g1 = *(const uint2 *)(tab + GB * ((iw >> (sh + 8)) & 255u));
                                g = make_uint4(g0.x, g0.y, g1.x, g1.y);
                            }
                            B[k] = as_v8h(make_uint4(pk_mul(g.x, f[k]) ^ m.x, pk_mul(g.y, f[k]) ^ m.y, pk_mul(g.z, f[k]) ^ m.z,
                                                     pk_mul(g.w, f[k]) ^ m.w));
                        }
                        le_v8h A[TM];
                        afrag(c, A);
                        gq_mma(d1, A, B, h == 0 && c == 0);
                        if (c == 0) pipe();
                    }
                }
            }
        }
        /* super-block epilogue (the h = 1 buffer holds this super-block's second half) */
        if constexpr (F::EPI == 1) {
            const u8 *Wb = lds + BUF;
            const u8 *Sb = Sl + (sb & 1) * SBYTES + (wm * TM) * F::SREC;
#pragma unroll
            for (int k = 0; k < TN; k++) {
                const u8 *r = Wb + (wn * TN * 32 + 32 * k + n) * F::SLOT;
                if constexpr (TY == LE_TYPE_Q4_K || TY == LE_TYPE_Q5_K) {
                    const uint4 hd = *(const uint4 *)r;
                    const u32 m0 = hd.z & 0x3F3F3F3Fu, m1 = ((hd.w >> 4) & 0x0F0F0F0Fu) | ((hd.z >> 2) & 0x30303030u);
                    const le_v8h b2 = as_v8h(make_uint4(pk_add(h1024_02(m0), 0xE400E400u), pk_add(h1024_13(m0), 0xE400E400u),
                                                        pk_add(h1024_02(m1), 0xE400E400u), pk_add(h1024_13(m1), 0xE400E400u)));
                    const float dd = h2f(hd.x & 0xFFFFu), dm = h2f(hd.x >> 16);
#pragma unroll
                    for (int i = 0; i < TM; i++) {
                        const le_v8h a2 = as_v8h(*(const uint4 *)(Sb + i * 1024 + lane * 16));
                        const le_v16f d2 = __builtin_amdgcn_mfma_f32_32x32x16_f16(a2, b2, (le_v16f){}, 0, 0, 0);
#pragma unroll
                        for (int e = 0; e < 16; e++) acc[i][k][e] = __builtin_fmaf(dd, d1[i][k][e], __builtin_fmaf(-dm, d2[e], acc[i][k][e]));
                    }
                } else if constexpr (TY == LE_TYPE_Q6_K) {
                    const float d64 = 64.f * h2f(*(const uint16_t *)(r + 126));
#pragma unroll
                    for (int i = 0; i < TM; i++)
#pragma unroll
                        for (int e = 0; e < 16; e++) acc[i][k][e] = __builtin_fmaf(d64, d1[i][k][e], acc[i][k][e]);
                } else if constexpr (TY == LE_TYPE_Q3_K) {
                    const float dd = h2f(*(const uint16_t *)(r + 78));
#pragma unroll
                    for (int i = 0; i < TM; i++)
#pragma unroll
                        for (int e = 0; e < 16; e++) acc[i][k][e] = __builtin_fmaf(dd, d1[i][k][e], acc[i][k][e]);
                } else {
                    const float dd = h2f(*(const uint16_t *)(r + (TY == LE_TYPE_IQ2_XXS ? 32 : 48))) *
                                     (TY == LE_TYPE_IQ3_XXS ? 0.25f : 0.125f);
#pragma unroll
                    for (int i = 0; i < TM; i++)
#pragma unroll
                        for (int e = 0; e < 16; e++) acc[i][k][e] = __builtin_fmaf(dd, d1[i][k][e], acc[i][k][e]);
                }
            }
        }
    }
    if constexpr (AD) gq_vm_wait<0>(); /* no activation load may still be writing LDS */
    /* D lane l element e: token 8 (e / 4) + 4 (l / 32) + e % 4 of the tile, row l % 32; the
     * token scales of the padded tile are all loaded first (one memory round trip) */
    if constexpr (F::EPI == 2) {
#pragma unroll
        for (int k = 0; k < TN; k++) {
            const float f = ldexpf(1.f, -rowS[k]);
#pragma unroll
            for (int i = 0; i < TM; i++)
#pragma unroll
                for (int e = 0; e < 16; e++) acc[i][k][e] *= f;
        }
    }
    float ts[TM][16];
#pragma unroll
    for (int i = 0; i < TM; i++)
#pragma unroll
        for (int e = 0; e < 16; e++) ts[i][e] = tsc[mb + (wm * TM + i) * 32 + 4 * hs + 8 * (e >> 2) + (e & 3)];
    if (!GR && a.ksplit > 1 && !a.part) { /* K slices without a partial-result buffer: atomic adds */
#pragma unroll
        for (int i = 0; i < TM; i++) {
            const int t0 = mb + (wm * TM + i) * 32 + 4 * hs;
#pragma unroll
            for (int k = 0; k < TN; k++) {
                const int r = nb + (wn * TN + k) * 32 + n;
#pragma unroll
                for (int e = 0; e < 16; e++) {
                    const int t = t0 + 8 * (e >> 2) + (e & 3);
                    if (t < M && r < a.rows) unsafeAtomicAdd(a.y + (size_t)t * a.rows + r, acc[i][k][e] * ts[i][e]);
                }
            }
        }
        return;
    }
    /* Stores through LDS, one 32-token tile of every wave row at a time: the waves place their
     * results as [token][row] (row stride BN + 8 floats: the two 4-token halves of a fragment fall
     * on different banks), then each token's BN outputs leave as 16-byte stores of consecutive
     * rows (a wave covers 1 KB of one output row) instead of 4-byte stores 32 to a row. */
    float *dst = (!GR && a.ksplit > 1) ? a.part + (size_t)blockIdx.y * a.m * a.rows : second ? a.y2 : a.y;
    constexpr int TS = BN + 8, NQ = BN / 4;
    static_assert((size_t)WM * 32 * TS * 4 <= (size_t)2 * BUF + (size_t)NA * AB, "output staging must fit the step buffers");
    float *T = (float *)lds;
    const bool vec = (a.rows & 3) == 0 && ((size_t)dst & 15) == 0;
#pragma unroll
    for (int i = 0; i < TM; i++) {
        __syncthreads(); /* the step buffers (or the previous round) are no longer read */
#pragma unroll
        for (int k = 0; k < TN; k++) {
            const int rl = (wn * TN + k) * 32 + n;
#pragma unroll
            for (int e = 0; e < 16; e++)
                T[(wm * 32 + 4 * hs + 8 * (e >> 2) + (e & 3)) * TS + rl] = acc[i][k][e] * ts[i][e];
        }
        __syncthreads();
        for (int c = tid; c < WM * 32 * NQ; c += NT) {
            const int tl = c / NQ, q = c - tl * NQ;
            const int t = mb + ((tl >> 5) * TM + i) * 32 + (tl & 31), r = nb + 4 * q;
            if (t >= M || r >= a.rows) continue;
            int o = t;
            if constexpr (GR) o = a.out_idx[pair0 + t - mb];
            const float4 v = *(const float4 *)(T + tl * TS + 4 * q);
            float *yp = dst + (size_t)o * a.rows + r;
            if (vec && r + 3 < a.rows) {
                *(float4 *)yp = v;
            } else {
                const float vv[4] = {v.x, v.y, v.z, v.w};
                for (int u = 0; u < 4 && r + u < a.rows; u++) yp[u] = vv[u];
            }
        }
    }
}

#define LE_GQX(TY, SK) \
    extern "C" __global__ void __launch_bounds__(256) le_gq_xprep_##TY(GqArgs a, u8 *ws) { gq_xprep_body<SK>(a, ws); } \
    extern "C" __global__ void __launch_bounds__(256) le_gq_xprepg_##TY(GqArgs a, u8 *ws) { gq_xprep_body<SK, true>(a, ws); } \
    extern "C" __global__ void __launch_bounds__(256) le_gq_xprepw_##TY(GqArgs a, u8 *ws) { gq_xprepw_body<SK>(a, ws); }
/* two code objects, compiled in parallel: the five types of the reference's mmq kernels, and the
 * four formats added beside them (LE_GQ_SET=2) */
#if LE_GQ_SET == 2
LE_GQX(2, 0) LE_GQX(11, 0) LE_GQX(13, 1) LE_GQX(22, 0)
#else
LE_GQX(8, 0) LE_GQX(12, 1) LE_GQX(14, 0) LE_GQX(16, 0) LE_GQX(18, 0)
#endif

/* Sum of the K slices' partial results: y[e] = part[0][e] + part[1][e] + ... in slice order
 * (deterministic, unlike atomic adds). */
#if LE_GQ_SET != 2
extern "C" __global__ void __launch_bounds__(256) le_gq_ksum(GqArgs a) {
    const size_t n = (size_t)a.m * a.rows, st = (size_t)gridDim.x * blockDim.x;
    size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x;
    const int ks = a.ksplit;
    if ((n & 3) == 0 && ((size_t)a.y & 15) == 0) { /* part is 256-byte aligned in the workspace */
        const size_t n4 = n / 4;
        const float4 *p = (const float4 *)a.part;
        for (; i < n4; i += st) {
            float4 s = p[i];
            for (int q = 1; q < ks; q++) {
                const float4 v = p[q * n4 + i];
                s.x += v.x;
                s.y += v.y;
                s.z += v.z;
                s.w += v.w;
            }
            ((float4 *)a.y)[i] = s;
        }
    } else {
        for (; i < n; i += st) {
            float s = a.part[i];
            for (int q = 1; q < ks; q++) s += a.part[q * n + i];
            a.y[i] = s;
        }
    }
}

#endif

#define LE_GQ_(TY, WM, WN, TM, TN)                                                                                     \
    extern "C" __global__ void __launch_bounds__(WM * WN * 64) le_gq_##TY##_w##WM##WN##_t##TM##TN(GqArgs a, const u8 *ws) { \
        gq_body<TY, WM, WN, TM, TN, false, 2>(a, ws);                                                                  \
    }
#define LE_GQG_(TY, WM, WN, TM, TN)                                                                                     \
    extern "C" __global__ void __launch_bounds__(WM * WN * 64) le_gqg_##TY##_w##WM##WN##_t##TM##TN(GqArgs a, const u8 *ws) { \
        gq_body<TY, WM, WN, TM, TN, true, 2>(a, ws);                                                                     \
    }
#define LE_GQ(TY) LE_GQ_(TY, 1, 4, 1, 2) LE_GQ_(TY, 1, 4, 2, 2) LE_GQ_(TY, 1, 4, 4, 2) LE_GQ_(TY, 2, 2, 2, 2) \
    LE_GQ_(TY, 1, 8, 2, 1) LE_GQ_(TY, 1, 8, 4, 1) LE_GQ_(TY, 1, 8, 1, 1) LE_GQ_(TY, 1, 4, 2, 1) LE_GQ_(TY, 1, 4, 1, 1) LE_GQ_(TY, 1, 4, 4, 1) LE_GQG_(TY, 1, 8, 2, 1) LE_GQG_(TY, 1, 8, 4, 1) LE_GQG_(TY, 2, 2, 2, 2) LE_GQG_(TY, 1, 8, 1, 1) LE_GQG_(TY, 1, 4, 1, 1)
#if LE_GQ_SET == 2
LE_GQ(2) LE_GQ(11) LE_GQ(13) LE_GQ(22)
#else
LE_GQ(8) LE_GQ(12) LE_GQ(14) LE_GQ(16) LE_GQ(18)
LE_GQ_(12, 2, 4, 2, 2) LE_GQ_(12, 2, 4, 2, 1)
#endif
