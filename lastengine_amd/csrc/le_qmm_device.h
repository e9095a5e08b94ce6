/* Device-side building blocks of the quantized matmul kernels (gfx950, wave64).
 *
 * Work decomposition. Every type is handled in 256-value super-blocks (one K-quant/IQ block, or
 * eight Q8_0 blocks). Eight lanes cooperate on one super-block; each lane owns 32 of its values.
 * A lane decodes its 32 weights into eight packed int8x4 words organised as NSEG segments of
 * WPS words (4*WPS consecutive activation positions sharing one weight scale). Per segment the
 * lane holds a float weight scale `sig` and, for K-quants with an offset, a float offset scale
 * `mu`, so that
 *
 *     sum_{segment} w * x  ==  sig * dx * sum(q * v)  -  mu * sum(dx * v)
 *
 * where x ~= dx * v is the activation held in LDS as a 15-bit integer v = 128*xh + xl split into
 * two int8 planes (xh, xl), with one fp32 scale dx per 32 values. The integer dot is exact
 * (v_dot4_i32_i8 on both planes), so the only approximation is the activation rounding,
 * |x - dx*v| <= dx/2 with dx = amax32 / 16256 (3.1e-5 of the 32-value block maximum).
 *
 * Weight bytes are read straight from the raw GGUF rows (the reference uploads raw GGUF bytes,
 * src/gpu.rs:79-83) through global-address-space loads: Q4_K super-blocks are 16-byte aligned and
 * use 128-bit loads; the other types are only 2-byte aligned and use unaligned 32/64/128-bit
 * loads, which gfx950 serves in one request per cache line.
 */
#pragma once
#include <hip/hip_runtime.h>
#include <stdint.h>

#include "le_formats.h"

typedef uint8_t u8;
typedef uint32_t u32;

#if defined(__HIP_DEVICE_COMPILE__)
#define LE_GLOBAL __attribute__((address_space(1)))
#else
#define LE_GLOBAL /* host pass of a mixed host/device translation unit */
#endif
#define LE_XSPLIT 16256.0f /* 127 * 128: |v| <= 16256 so xh = (v+64)>>7 in [-127,127], xl in [-64,63] */

typedef u32 __attribute__((aligned(2))) le_u32_a2;
typedef u32 le_v4u __attribute__((ext_vector_type(4)));
typedef u32 le_v2u __attribute__((ext_vector_type(2)));
/* 2-byte aligned native vectors: a load of the HIP struct types uint4 / uint2 at this alignment is
 * split into scalar loads through a generic pointer, which the backend re-merges as a flat load */
typedef le_v4u __attribute__((aligned(2))) le_v4u_a2;
typedef le_v2u __attribute__((aligned(2))) le_v2u_a2;

/* Global loads (never flat: flat loads also count against the LDS wait counter). */
__device__ __forceinline__ uint4 ldg16(const u8 *p) { /* 16-byte aligned, streamed once */
    const le_v4u v = __builtin_nontemporal_load((const LE_GLOBAL le_v4u *)p);
    return make_uint4(v.x, v.y, v.z, v.w);
}
__device__ __forceinline__ uint4 ldg16c(const u8 *p) { /* 16-byte aligned, cached (shared by 8 lanes) */
    const le_v4u v = *(const LE_GLOBAL le_v4u *)p;
    return make_uint4(v.x, v.y, v.z, v.w);
}
__device__ __forceinline__ uint4 ldg16u(const u8 *p) { /* 2-byte aligned */
    const le_v4u v = *(const LE_GLOBAL le_v4u_a2 *)p;
    return make_uint4(v.x, v.y, v.z, v.w);
}
__device__ __forceinline__ uint2 ldg8u(const u8 *p) {
    const le_v2u v = *(const LE_GLOBAL le_v2u_a2 *)p;
    return make_uint2(v.x, v.y);
}
__device__ __forceinline__ u32 ldg4u(const u8 *p) { return *(const LE_GLOBAL le_u32_a2 *)p; }
__device__ __forceinline__ u32 ldg2(const u8 *p) { return *(const LE_GLOBAL uint16_t *)p; }

/* Sum over lanes l, l ^ 16, l ^ 32 and l ^ 48 (the four 16-lane rows of the wave), in every lane:
 * xor 16 by a swizzle, xor 32 by the gfx950 permlane32 swap on the VALU (no LDS round trip for
 * that half): (v_l + v_l^16) + (same)^32, the same bits in every lane as a swizzle/shuffle
 * butterfly (each step adds the same two values). */
__device__ __forceinline__ float row4_sum(float v) {
    const float s = v + __builtin_bit_cast(float, __builtin_amdgcn_ds_swizzle(__builtin_bit_cast(int, v), 0x401F));
    /* the swap's operands as two distinct values (the compiler would otherwise treat a swap of a
     * value with itself as a no-op); after it p[0] holds s of lanes 0-31 in both halves, p[1] s of
     * lanes 32-63 */
    u32 hi;
    __asm__("v_mov_b32 %0, %1" : "=v"(hi) : "v"(s));
    const auto p = __builtin_amdgcn_permlane32_swap(__builtin_bit_cast(u32, s), hi, false, false);
    return __builtin_bit_cast(float, (u32)p[0]) + __builtin_bit_cast(float, (u32)p[1]);
}

__device__ __forceinline__ float h2f(u32 bits16) {
    return (float)__builtin_bit_cast(_Float16, (uint16_t)bits16);
}

/* src/quant.rs:37-49, in integer arithmetic (also reproduces NaN payloads bit for bit). */
__device__ inline float f16_exact(u32 h) {
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

__device__ __forceinline__ int dot4(u32 a, u32 b, int c) {
    return __builtin_amdgcn_sdot4((int)a, (int)b, c, false);
}

/* LDS image of one token's activations: per 8-value group p, xq[p] = {xh word0, xh word1,
 * xl word0, xl word1} and xs[p] = {dx of the group's 32-value unit, dx * sum(v) over the group}. */
struct XTok {
    const uint4 *xq;
    const float2 *xs;
};

/* Bytes of LDS for one token's activation image of K values. */
__host__ __device__ inline int le_xtok_bytes(int K) { return (K / 8) * (16 + 8); }

/* LDS record order of the activation image. Lane li of a super-block's 8-lane group reads its
 * c-th 8-value group (c = 0..3, segment-major) from record 32*sb + 8*(c ^ (sb & 3)) + li, so
 * each 8-lane read touches 8 distinct 16-byte bank groups and neighbouring super-blocks differ in
 * bits 3-4. The per-type maps from a natural group (unit uu of the super-block, group gw of the
 * unit) to (li, c) follow each format's lane split:
 *   XL_Q4K: li = 2*(uu>>1) + (gw>>1), c = 2*(uu&1) + (gw&1)
 *   XL_Q6K: li = 4*(uu>>2) + gw,      c = uu & 3
 *   XL_ROW: li = uu,                  c = gw          (Q8_0, IQ2_XXS, IQ3_XXS) */
#define XL_ROW 0
#define XL_Q4K 1
#define XL_Q6K 2
template <int XL>
__device__ __forceinline__ int le_xpos(int p) {
    const int u = p >> 2, gw = p & 3, sb = u >> 3, uu = u & 7;
    int li, c;
    if (XL == XL_Q4K) { li = 2 * (uu >> 1) + (gw >> 1); c = 2 * (uu & 1) + (gw & 1); }
    else if (XL == XL_Q6K) { li = 4 * (uu >> 2) + gw; c = uu & 3; }
    else { li = uu; c = gw; }
    return 32 * sb + 8 * (c ^ (sb & 3)) + li;
}

/* Quantize 8 activations (one group) given the amax of their 32-value unit; record q. */
__device__ __forceinline__ void le_quant_group(float4 a, float4 b, float am, uint4 *xq, float2 *xs, int p) {
    const float inv = am > 0.f ? LE_XSPLIT / am : 0.f;
    const float d = am / LE_XSPLIT;
    const int v[8] = {(int)rintf(a.x * inv), (int)rintf(a.y * inv), (int)rintf(a.z * inv), (int)rintf(a.w * inv),
                      (int)rintf(b.x * inv), (int)rintf(b.y * inv), (int)rintf(b.z * inv), (int)rintf(b.w * inv)};
    u32 hw[2] = {0, 0}, lw[2] = {0, 0};
    int s = 0;
#pragma unroll
    for (int i = 0; i < 8; i++) {
        const int h = (v[i] + 64) >> 7;
        const int l = v[i] - (h << 7);
        hw[i >> 2] |= ((u32)h & 255u) << (8 * (i & 3));
        lw[i >> 2] |= ((u32)l & 255u) << (8 * (i & 3));
        s += v[i];
    }
    xq[p] = make_uint4(hw[0], hw[1], lw[0], lw[1]);
    xs[p] = make_float2(d, d * (float)s);
}

__device__ __forceinline__ float amax8(float4 a, float4 b) {
    return fmaxf(fmaxf(fmaxf(fabsf(a.x), fabsf(a.y)), fmaxf(fabsf(a.z), fabsf(a.w))),
                 fmaxf(fmaxf(fabsf(b.x), fabsf(b.y)), fmaxf(fabsf(b.z), fabsf(b.w))));
}

/* Quantize one token's K activations (K % 32 == 0) into the LDS image. Called by all threads of
 * the block; 4 consecutive threads share a 32-value unit. */
/* silu(g) * u per component (the reference's swiglu, src/cuda/kernels.cu:7,428) */
__device__ __forceinline__ float4 le_silu_mul4(float4 g, float4 u) {
    return make_float4(g.x / (1.0f + __expf(-g.x)) * u.x, g.y / (1.0f + __expf(-g.y)) * u.y, g.z / (1.0f + __expf(-g.z)) * u.z,
                       g.w / (1.0f + __expf(-g.w)) * u.w);
}

/* up != nullptr: the activation is silu(x) * up (le_matvec_swiglu). */
template <int XL>
__device__ __forceinline__ void le_quant_x_lds(const float *__restrict__ x, int K, uint4 *xq, float2 *xs,
                                               const float *__restrict__ up = nullptr) {
    const int ng = K >> 3;
    const LE_GLOBAL float *xg = (const LE_GLOBAL float *)x;
    for (int p = threadIdx.x; p < ((ng + 3) & ~3); p += blockDim.x) {
        const bool ok = p < ng;
        float4 a = make_float4(0.f, 0.f, 0.f, 0.f), b = a;
        if (ok) {
            a = *(const LE_GLOBAL float4 *)(xg + 8 * p);
            b = *(const LE_GLOBAL float4 *)(xg + 8 * p + 4);
            if (up) {
                a = le_silu_mul4(a, *(const LE_GLOBAL float4 *)(up + 8 * p));
                b = le_silu_mul4(b, *(const LE_GLOBAL float4 *)(up + 8 * p + 4));
            }
        }
        float am = amax8(a, b);
        am = fmaxf(am, __shfl_xor(am, 1));
        am = fmaxf(am, __shfl_xor(am, 2));
        if (ok) le_quant_group(a, b, am, xq, xs, le_xpos<XL>(p));
    }
}

/* The same in two phases for one token with a compile-time block of BLOCK threads and at most
 * XR groups per thread: load() issues the activation loads (before the weight loads, so they
 * return first; addresses are clamped instead of predicated so the wait counters stay exact),
 * store() quantizes into LDS. */
template <int BLOCK, int XR>
struct XLoad {
    float4 a[XR], b[XR];
    /* up != nullptr: the activation is silu(x) * up, formed at load (le_matvec_swiglu) */
    __device__ __forceinline__ void load(const float *__restrict__ x, int K, const float *__restrict__ up = nullptr) {
        const int ng = K >> 3;
        const LE_GLOBAL float *xg = (const LE_GLOBAL float *)x;
#pragma unroll
        for (int r = 0; r < XR; r++) {
            const int p = min((int)threadIdx.x + r * BLOCK, ng - 1);
            a[r] = *(const LE_GLOBAL float4 *)(xg + 8 * p);
            b[r] = *(const LE_GLOBAL float4 *)(xg + 8 * p + 4);
        }
        /* issued either way (without up: a cached re-read of x), so the wait counts of the
         * kernel do not depend on the mode */
        const LE_GLOBAL float *ug = (const LE_GLOBAL float *)(up ? up : x);
        float4 ua[XR], ub[XR];
#pragma unroll
        for (int r = 0; r < XR; r++) {
            const int p = min((int)threadIdx.x + r * BLOCK, ng - 1);
            ua[r] = *(const LE_GLOBAL float4 *)(ug + 8 * p);
            ub[r] = *(const LE_GLOBAL float4 *)(ug + 8 * p + 4);
        }
        if (up) {
#pragma unroll
            for (int r = 0; r < XR; r++) {
                a[r] = le_silu_mul4(a[r], ua[r]);
                b[r] = le_silu_mul4(b[r], ub[r]);
            }
        }
    }
    template <int XL>
    __device__ __forceinline__ void store(int K, uint4 *xq, float2 *xs) {
        const int ng = K >> 3;
#pragma unroll
        for (int r = 0; r < XR; r++) {
            if (r * BLOCK >= ng) break;
            const int p = threadIdx.x + r * BLOCK;
            float am = amax8(a[r], b[r]);
            am = fmaxf(am, __shfl_xor(am, 1));
            am = fmaxf(am, __shfl_xor(am, 2));
            if (p < ng) le_quant_group(a[r], b[r], am, xq, xs, le_xpos<XL>(p));
        }
    }
};

/* One lane's decoded share of a super-block: NSEG segments of WPS int8x4 words each; the lane's
 * activation groups c = 0..3 are taken in segment order (segment k owns groups
 * k*WPS/2 .. (k+1)*WPS/2 - 1). */
template <int NSEG, int WPS>
struct Dec {
    u32 w[NSEG * WPS];
    float sig[NSEG];
    float mu[NSEG];
};

/* Sum over aligned groups of N lanes (N = 8, 16, 32 or 64) with DPP / swizzle; the full sum is
 * valid in the first lane of each group. */
template <int CTRL>
__device__ __forceinline__ float dpp_f(float x) {
    return __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, x), CTRL, 0xF, 0xF, true));
}

template <int N>
__device__ __forceinline__ float group_sum(float v) {
    v += dpp_f<0xB1>(v);  /* quad_perm [1,0,3,2] */
    v += dpp_f<0x4E>(v);  /* quad_perm [2,3,0,1] */
    v += dpp_f<0x141>(v); /* row_half_mirror: 8-lane sums */
    if constexpr (N >= 16) v += dpp_f<0x140>(v); /* row_mirror: 16-lane sums */
    if constexpr (N >= 32) /* xor 16 within each 32 lanes */
        v += __builtin_bit_cast(float, __builtin_amdgcn_ds_swizzle(__builtin_bit_cast(int, v), 0x401F));
    if constexpr (N >= 64) v += __shfl_xor(v, 32);
    return v;
}

template <int TY>
struct Fmt;

/* ---------------- Q4_K: 144 B = d f16, dmin f16, 12 B packed 6-bit scales/mins, 128 B nibbles.
 * Lane li: pair g = li>>1 of 64 values (low nibbles -> sub-block 2g, high -> 2g+1, per
 * src/quant.rs:74-80), half hh = li&1 of the 32 nibble bytes -> two 16-value segments. */
template <>
struct Fmt<LE_TYPE_Q4_K> {
    static constexpr int SB = LE_SB_BYTES_Q4_K;
    static constexpr bool HAS_MU = true;
    static constexpr bool TABLES = false;
    static constexpr int NSEG = 2, WPS = 4, XL = XL_Q4K;
    struct Raw {
        uint4 h, q;
    };
    __device__ static __forceinline__ Raw load(const u8 *p, int li) {
        Raw r;
        r.h = ldg16c(p);
        r.q = ldg16(p + 16 + 16 * li);
        return r;
    }
    __device__ static __forceinline__ void decode(const Raw &r, int li, int sb, const u32 *, Dec<NSEG, WPS> &d) {
        const int g = li >> 1, hh = li & 1;
        const u32 q[4] = {r.q.x, r.q.y, r.q.z, r.q.w};
#pragma unroll
        for (int i = 0; i < 4; i++) {
            d.w[i] = q[i] & 0x0F0F0F0Fu;            /* segment 0: low nibbles, sub-block 2g */
            d.w[4 + i] = (q[i] >> 4) & 0x0F0F0F0Fu; /* segment 1: high nibbles, sub-block 2g+1 */
        }
        /* scale_min_k4 (src/quant.rs:52-55): lane li decodes sub-block j = li, then the pair
         * (2g, 2g+1) it needs comes from lanes li&~1 and li|1 of its quad. */
        const int sh8 = 8 * (li & 3);
        const u32 a = r.h.y >> sh8, b = r.h.z >> sh8, c = r.h.w >> sh8;
        const u32 sc = li < 4 ? (a & 63u) : ((c & 15u) | ((a >> 2) & 0x30u));
        const u32 mn = li < 4 ? (b & 63u) : (((c >> 4) & 15u) | ((b >> 2) & 0x30u));
        const float sj = h2f(r.h.x & 0xFFFFu) * (float)sc, mj = h2f(r.h.x >> 16) * (float)mn;
        d.sig[0] = dpp_f<0xA0>(sj); /* quad_perm [0,0,2,2] */
        d.sig[1] = dpp_f<0xF5>(sj); /* quad_perm [1,1,3,3] */
        d.mu[0] = dpp_f<0xA0>(mj);
        d.mu[1] = dpp_f<0xF5>(mj);
    }
};

/* ---------------- Q6_K: 210 B = ql[128], qh[64], int8 scales[16], d f16 (src/quant.rs:96-112).
 * Lane li: half n = li>>2 (128 values), l-range [8t, 8t+8) with t = li&3, all four quadrants
 * (four 8-value segments). The stored 6-bit code q is used unsigned; the -32 offset goes into
 * mu = 32*d*sc. */
template <>
struct Fmt<LE_TYPE_Q6_K> {
    static constexpr int SB = LE_SB_BYTES_Q6_K;
    static constexpr bool HAS_MU = true;
    static constexpr bool TABLES = false;
    static constexpr int NSEG = 4, WPS = 2, XL = XL_Q6K;
    struct Raw {
        uint2 la, lb, qh, sc;
        u32 d;
    };
    __device__ static __forceinline__ Raw load(const u8 *p, int li) {
        const int n = li >> 2, t = li & 3;
        Raw r;
        r.la = ldg8u(p + n * 64 + 8 * t);
        r.lb = ldg8u(p + n * 64 + 32 + 8 * t);
        r.qh = ldg8u(p + 128 + n * 32 + 8 * t);
        r.sc = ldg8u(p + 192 + n * 8);
        r.d = ldg2(p + 208);
        return r;
    }
    __device__ static __forceinline__ void decode(const Raw &r, int li, int sb, const u32 *, Dec<NSEG, WPS> &d) {
        const int n = li >> 2, t = li & 3, is = t >> 1;
        const u32 la[2] = {r.la.x, r.la.y}, lb[2] = {r.lb.x, r.lb.y}, qh[2] = {r.qh.x, r.qh.y};
#pragma unroll
        for (int k = 0; k < 2; k++) {
            d.w[0 + k] = (la[k] & 0x0F0F0F0Fu) | ((qh[k] << 4) & 0x30303030u);
            d.w[2 + k] = (lb[k] & 0x0F0F0F0Fu) | ((qh[k] << 2) & 0x30303030u);
            d.w[4 + k] = ((la[k] >> 4) & 0x0F0F0F0Fu) | (qh[k] & 0x30303030u);
            d.w[6 + k] = ((lb[k] >> 4) & 0x0F0F0F0Fu) | ((qh[k] >> 2) & 0x30303030u);
        }
        const float dd = h2f(r.d);
        /* quadrant qd uses sc[is + 2*qd] of this half: bytes is, is+2 of word x and of word y */
        const u32 sx = r.sc.x >> (8 * is), sy = r.sc.y >> (8 * is);
        d.sig[0] = dd * (float)(int)(int8_t)(sx & 255u);
        d.sig[1] = dd * (float)(int)(int8_t)((sx >> 16) & 255u);
        d.sig[2] = dd * (float)(int)(int8_t)(sy & 255u);
        d.sig[3] = dd * (float)(int)(int8_t)((sy >> 16) & 255u);
#pragma unroll
        for (int k = 0; k < 4; k++) d.mu[k] = 32.0f * d.sig[k];
    }
};

/* ---------------- Q8_0 (8 blocks of 34 B = d f16 + 32 int8 per 256 values, src/quant.rs:68-71).
 * Lane li owns block li of the super-block: one 32-value segment. */
template <>
struct Fmt<LE_TYPE_Q8_0> {
    static constexpr int SB = LE_SB_BYTES_Q8_0;
    static constexpr bool HAS_MU = false;
    static constexpr bool TABLES = false;
    static constexpr int NSEG = 1, WPS = 8, XL = XL_ROW;
    struct Raw {
        uint4 a, b;
        u32 d;
    };
    __device__ static __forceinline__ Raw load(const u8 *p, int li) {
        const u8 *bp = p + 34 * li;
        Raw r;
        r.d = ldg2(bp);
        r.a = ldg16u(bp + 2);
        r.b = ldg16u(bp + 18);
        return r;
    }
    __device__ static __forceinline__ void decode(const Raw &r, int li, int sb, const u32 *, Dec<NSEG, WPS> &d) {
        d.w[0] = r.a.x; d.w[1] = r.a.y; d.w[2] = r.a.z; d.w[3] = r.a.w;
        d.w[4] = r.b.x; d.w[5] = r.b.y; d.w[6] = r.b.z; d.w[7] = r.b.w;
        d.sig[0] = h2f(r.d);
        d.mu[0] = 0.f;
    }
};

/* Sign handling for the IQ types: the LDS sign table holds, for each 7-bit sign index s, the byte
 * masks of ksign(s) (src/quant.rs:57): word 2s covers values 0-3, word 2s+1 values 4-7, 0xFF
 * where the value is negative. Negating a byte magnitude g (1..127) is (g ^ 0xFF) + 1, which never
 * carries into the next byte, so a whole word is signed with one xor and one add. */
__device__ __forceinline__ u32 apply_sign(u32 g, u32 m) { return (g ^ m) + (m & 0x01010101u); }

/* LDS table layout for IQ kernels: [0,256) sign masks, then the grid words. */
#define LE_TAB_SIGN 0
#define LE_TAB_GRID 256

/* ---------------- IQ2_XXS: 66 B = d f16 + 8 x (4 grid indices, u32 signs/scale) (src/quant.rs:142-154).
 * Lane li owns 32-value sub-block ib = li. */
template <>
struct Fmt<LE_TYPE_IQ2_XXS> {
    static constexpr int SB = LE_SB_BYTES_IQ2_XXS;
    static constexpr bool HAS_MU = false;
    static constexpr bool TABLES = true;
    static constexpr int GRID_WORDS = 512;
    static constexpr int NSEG = 1, WPS = 8, XL = XL_ROW;
    struct Raw {
        uint2 q;
        u32 d;
    };
    __device__ static __forceinline__ Raw load(const u8 *p, int li) {
        Raw r;
        r.d = ldg2(p);
        r.q = ldg8u(p + 2 + 8 * li);
        return r;
    }
    __device__ static __forceinline__ void decode(const Raw &r, int li, int sb, const u32 *tab, Dec<NSEG, WPS> &d) {
        const u32 aux = r.q.y;
        const u32 *grid = tab + LE_TAB_GRID, *sg = tab + LE_TAB_SIGN;
#pragma unroll
        for (int l = 0; l < 4; l++) {
            const u32 gi = (r.q.x >> (8 * l)) & 255u, si = (aux >> (7 * l)) & 127u;
            const uint2 g = *(const uint2 *)(grid + 2 * gi);
            const uint2 m = *(const uint2 *)(sg + 2 * si);
            d.w[2 * l] = apply_sign(g.x, m.x);
            d.w[2 * l + 1] = apply_sign(g.y, m.y);
        }
        d.sig[0] = h2f(r.d) * (0.5f + (float)(aux >> 28)) * 0.25f;
        d.mu[0] = 0.f;
    }
};

/* ---------------- IQ3_XXS: 98 B = d f16, qs[64] grid indices, 8 x u32 signs/scale (src/quant.rs:127-141). */
template <>
struct Fmt<LE_TYPE_IQ3_XXS> {
    static constexpr int SB = LE_SB_BYTES_IQ3_XXS;
    static constexpr bool HAS_MU = false;
    static constexpr bool TABLES = true;
    static constexpr int GRID_WORDS = 256;
    static constexpr int NSEG = 1, WPS = 8, XL = XL_ROW;
    struct Raw {
        uint2 q;
        u32 aux, d;
    };
    __device__ static __forceinline__ Raw load(const u8 *p, int li) {
        Raw r;
        r.d = ldg2(p);
        r.q = ldg8u(p + 2 + 8 * li);
        r.aux = ldg4u(p + 66 + 4 * li);
        return r;
    }
    __device__ static __forceinline__ void decode(const Raw &r, int li, int sb, const u32 *tab, Dec<NSEG, WPS> &d) {
        const u32 aux = r.aux;
        const u32 *grid = tab + LE_TAB_GRID, *sg = tab + LE_TAB_SIGN;
        const u32 qw[2] = {r.q.x, r.q.y};
#pragma unroll
        for (int l = 0; l < 4; l++) {
            const u32 q = qw[l >> 1] >> (16 * (l & 1));
            const u32 si = (aux >> (7 * l)) & 127u;
            const uint2 m = *(const uint2 *)(sg + 2 * si);
            d.w[2 * l] = apply_sign(grid[q & 255u], m.x);
            d.w[2 * l + 1] = apply_sign(grid[(q >> 8) & 255u], m.y);
        }
        d.sig[0] = h2f(r.d) * (0.5f + (float)(aux >> 28)) * 0.5f;
        d.mu[0] = 0.f;
    }
};

/* Byte masks of a 4-bit sign nibble: byte i is 0xFF where bit i is set (bit i moved to bit 8i by
 * shifts that never overlap, then spread over the byte). */
__device__ __forceinline__ u32 nib_mask(u32 n) { return ((n * 0x00204081u) & 0x01010101u) * 0xFFu; }

/* ---------------- Q4_0 (8 blocks of 18 B = d f16 + 16 nibble bytes per 256 values, src/quant.rs:64-67).
 * Lane li owns block li: low nibbles are values 0-15, high nibbles 16-31; q - 8 through mu = 8 d. */
template <>
struct Fmt<LE_TYPE_Q4_0> {
    static constexpr int SB = LE_SB_BYTES_Q4_0;
    static constexpr bool HAS_MU = true;
    static constexpr bool TABLES = false;
    static constexpr int NSEG = 1, WPS = 8, XL = XL_ROW;
    struct Raw {
        uint4 q;
        u32 d;
    };
    __device__ static __forceinline__ Raw load(const u8 *p, int li) {
        const u8 *bp = p + 18 * li;
        Raw r;
        r.d = ldg2(bp);
        r.q = ldg16u(bp + 2);
        return r;
    }
    __device__ static __forceinline__ void decode(const Raw &r, int li, int sb, const u32 *, Dec<NSEG, WPS> &d) {
        const u32 q[4] = {r.q.x, r.q.y, r.q.z, r.q.w};
#pragma unroll
        for (int i = 0; i < 4; i++) {
            d.w[i] = q[i] & 0x0F0F0F0Fu;
            d.w[4 + i] = (q[i] >> 4) & 0x0F0F0F0Fu;
        }
        d.sig[0] = h2f(r.d);
        d.mu[0] = 8.0f * d.sig[0];
    }
};

/* ---------------- Q5_K: 176 B = d, dmin, 12 B scales/mins (as Q4_K), qh[32], qs[128]
 * (src/quant.rs:83-95). Lane li as Q4_K (pair g = li>>1, half hh = li&1); the fifth bit of value
 * 64g + l (l < 32) is bit 2g of qh[l], of value 64g + 32 + l bit 2g+1. */
template <>
struct Fmt<LE_TYPE_Q5_K> {
    static constexpr int SB = LE_SB_BYTES_Q5_K;
    static constexpr bool HAS_MU = true;
    static constexpr bool TABLES = false;
    static constexpr int NSEG = 2, WPS = 4, XL = XL_Q4K;
    struct Raw {
        uint4 h, q, qh;
    };
    __device__ static __forceinline__ Raw load(const u8 *p, int li) {
        Raw r;
        r.h = ldg16c(p);
        r.qh = ldg16c(p + 16 + 16 * (li & 1));
        r.q = ldg16(p + 48 + 16 * li);
        return r;
    }
    __device__ static __forceinline__ void decode(const Raw &r, int li, int sb, const u32 *, Dec<NSEG, WPS> &d) {
        const int g = li >> 1;
        const u32 q[4] = {r.q.x, r.q.y, r.q.z, r.q.w}, h[4] = {r.qh.x, r.qh.y, r.qh.z, r.qh.w};
#pragma unroll
        for (int i = 0; i < 4; i++) {
            d.w[i] = (q[i] & 0x0F0F0F0Fu) | (((h[i] >> (2 * g)) & 0x01010101u) << 4);
            d.w[4 + i] = ((q[i] >> 4) & 0x0F0F0F0Fu) | (((h[i] >> (2 * g + 1)) & 0x01010101u) << 4);
        }
        const int sh8 = 8 * (li & 3);
        const u32 a = r.h.y >> sh8, b = r.h.z >> sh8, c = r.h.w >> sh8;
        const u32 sc = li < 4 ? (a & 63u) : ((c & 15u) | ((a >> 2) & 0x30u));
        const u32 mn = li < 4 ? (b & 63u) : (((c >> 4) & 15u) | ((b >> 2) & 0x30u));
        const float sj = h2f(r.h.x & 0xFFFFu) * (float)sc, mj = h2f(r.h.x >> 16) * (float)mn;
        d.sig[0] = dpp_f<0xA0>(sj);
        d.sig[1] = dpp_f<0xF5>(sj);
        d.mu[0] = dpp_f<0xA0>(mj);
        d.mu[1] = dpp_f<0xF5>(mj);
    }
};

/* ---------------- Q3_K: 110 B = hmask[32], qs[64], 12 B of 6-bit scales, d f16 (src/quant.rs:113-126).
 * Lane li: half c = li>>2 (128 values), l-range [8t, 8t+8) with t = li&3, four quadrants s (the Q6_K
 * lane split). Value 128c + 32s + l has the 2-bit code (qs[32c+l] >> 2s) & 3 and high bit
 * (hmask[l] >> (4c+s)) & 1; the code u = q2 | 4h is used unsigned and the -4 goes into mu = 4 sig.
 * Scale i (one per 16 values, stored + 32): low nibble from byte i (i < 8) or the high nibble of
 * byte i-8, top two bits at 2(i>>2) of byte 8 + (i&3). */
template <>
struct Fmt<LE_TYPE_Q3_K> {
    static constexpr int SB = LE_SB_BYTES_Q3_K;
    static constexpr bool HAS_MU = true;
    static constexpr bool TABLES = false;
    static constexpr int NSEG = 4, WPS = 2, XL = XL_Q6K;
    struct Raw {
        uint2 hm, qs, sa;
        u32 sb4, d;
    };
    __device__ static __forceinline__ Raw load(const u8 *p, int li) {
        const int c = li >> 2, t = li & 3;
        Raw r;
        r.hm = ldg8u(p + 8 * t);
        r.qs = ldg8u(p + 32 + 32 * c + 8 * t);
        r.sa = ldg8u(p + 96);
        r.sb4 = ldg4u(p + 104);
        r.d = ldg2(p + 108);
        return r;
    }
    __device__ static __forceinline__ void decode(const Raw &r, int li, int sb, const u32 *, Dec<NSEG, WPS> &d) {
        const int c = li >> 2, t = li & 3;
        const u32 hm[2] = {r.hm.x, r.hm.y}, qs[2] = {r.qs.x, r.qs.y};
#pragma unroll
        for (int s = 0; s < 4; s++)
#pragma unroll
            for (int k = 0; k < 2; k++)
                d.w[2 * s + k] = ((qs[k] >> (2 * s)) & 0x03030303u) | (((hm[k] >> (4 * c + s)) & 0x01010101u) << 2);
        const float dd = h2f(r.d);
#pragma unroll
        for (int s = 0; s < 4; s++) {
            const int i = 8 * c + 2 * s + (t >> 1);
            const int lb = i & 7;
            const u32 lw = lb < 4 ? r.sa.x : r.sa.y;
            const u32 lo = ((lw >> (8 * (lb & 3))) >> (c ? 4 : 0)) & 15u;
            const u32 hi = (r.sb4 >> (8 * (i & 3) + 2 * (i >> 2))) & 3u;
            d.sig[s] = dd * (float)((int)(lo | (hi << 4)) - 32);
            d.mu[s] = 4.0f * d.sig[s];
        }
    }
};

/* ---------------- IQ2_S: 82 B = d f16, qs[32], signs[32], qh[8], scales[8] (src/quant.rs:155-167).
 * Lane li owns 32-value sub-block ib = li: grid index qs[4ib+l] | ((qh[ib] << (8-2l)) & 0x300) of
 * the 1024-entry grid (LDS), an explicit sign byte per 8 values, the scale nibble of its first (low)
 * and second (high) 16 values. */
template <>
struct Fmt<LE_TYPE_IQ2_S> {
    static constexpr int SB = LE_SB_BYTES_IQ2_S;
    static constexpr bool HAS_MU = false;
    static constexpr bool TABLES = true;
    static constexpr int GRID_WORDS = 2048;
    static constexpr int NSEG = 2, WPS = 4, XL = XL_ROW;
    struct Raw {
        u32 qs, sn, qh2, sc2, d;
    };
    __device__ static __forceinline__ Raw load(const u8 *p, int li) {
        Raw r;
        r.d = ldg2(p);
        r.qs = ldg4u(p + 2 + 4 * li);
        r.sn = ldg4u(p + 34 + 4 * li);
        r.qh2 = ldg2(p + 66 + (li & 6));
        r.sc2 = ldg2(p + 74 + (li & 6));
        return r;
    }
    __device__ static __forceinline__ void decode(const Raw &r, int li, int sb, const u32 *tab, Dec<NSEG, WPS> &d) {
        const u32 *grid = tab + LE_TAB_GRID;
        const u32 qh = (r.qh2 >> (8 * (li & 1))) & 255u, sc = (r.sc2 >> (8 * (li & 1))) & 255u;
#pragma unroll
        for (int l = 0; l < 4; l++) {
            const u32 gi = ((r.qs >> (8 * l)) & 255u) | ((qh << (8 - 2 * l)) & 0x300u);
            const u32 sg = (r.sn >> (8 * l)) & 255u;
            const uint2 g = *(const uint2 *)(grid + 2 * gi);
            d.w[2 * l] = apply_sign(g.x, nib_mask(sg & 15u));
            d.w[2 * l + 1] = apply_sign(g.y, nib_mask(sg >> 4));
        }
        const float dd = h2f(r.d);
        d.sig[0] = dd * (0.5f + (float)(sc & 15u)) * 0.25f;
        d.sig[1] = dd * (0.5f + (float)(sc >> 4)) * 0.25f;
        d.mu[0] = d.mu[1] = 0.f;
    }
};

/* Activation image from the reference's int8 activations (quant_x output: xq per value, xd per 32
 * values): the xl plane carries xq, the xh plane is zero, dx = xd, and the group sum is formed from
 * xq. The vector kernels then compute exactly the reference's integer dot per unit times its
 * scales (udot<ty>, src/cuda/kernels.cu:36-110). Same two-phase shape as XLoad. */
__device__ __forceinline__ void le_q8_group(uint2 w, float d, uint4 *xq, float2 *xs, int p) {
    int s = 0;
#pragma unroll
    for (int i = 0; i < 4; i++) s += (int)(int8_t)((w.x >> (8 * i)) & 255u) + (int)(int8_t)((w.y >> (8 * i)) & 255u);
    xq[p] = make_uint4(0u, 0u, w.x, w.y);
    xs[p] = make_float2(d, d * (float)s);
}
template <int BLOCK, int XR>
struct XLoadQ8 {
    uint2 w[XR];
    float d[XR];
    __device__ __forceinline__ void load(const int8_t *__restrict__ xq, const float *__restrict__ xd, int K) {
        const int ng = K >> 3;
#pragma unroll
        for (int r = 0; r < XR; r++) {
            const int p = min((int)threadIdx.x + r * BLOCK, ng - 1);
            w[r] = *(const LE_GLOBAL uint2 *)(xq + 8 * p);
            d[r] = *(const LE_GLOBAL float *)(xd + (p >> 2));
        }
    }
    template <int XL>
    __device__ __forceinline__ void store(int K, uint4 *xq, float2 *xs) {
        const int ng = K >> 3;
#pragma unroll
        for (int r = 0; r < XR; r++) {
            const int p = threadIdx.x + r * BLOCK;
            if (p < ng) le_q8_group(w[r], d[r], xq, xs, le_xpos<XL>(p));
        }
    }
};
template <int XL>
__device__ __forceinline__ void le_q8_x_lds(const int8_t *__restrict__ xqg, const float *__restrict__ xd, int K, uint4 *xq,
                                            float2 *xs) {
    for (int p = threadIdx.x; p < (K >> 3); p += blockDim.x)
        le_q8_group(*(const LE_GLOBAL uint2 *)(xqg + 8 * p), xd[p >> 2], xq, xs, le_xpos<XL>(p));
}
