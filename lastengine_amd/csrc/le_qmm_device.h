/* Device-side building blocks of the quantized matmul kernels (gfx950, wave64).
 *
 * Work decomposition. Every type is handled in 256-value super-blocks (one K-quant/IQ block, or
 * eight Q8_0 blocks). Eight lanes cooperate on one super-block; each lane owns 32 of its values,
 * split into four groups of 8 consecutive activation positions. A lane decodes its 32 weights into
 * eight packed int8x4 words plus, per group, a float weight scale `sig` and (K-quants with an
 * offset) a float offset scale `mu`, so that
 *
 *     sum_{8 values} w * x  ==  sig * (dx * sum q*v) - mu * (dx * sum v)
 *
 * where x ~= dx * v is the activation held in LDS as a 15-bit integer v = 128*xh + xl split into
 * two int8 planes (xh, xl) with one fp32 scale dx per 32 values. The integer dot is exact
 * (v_dot4_i32_i8 on both planes), so the only approximation is the activation rounding,
 * |x - dx*v| <= dx/2 with dx = amax32 / 16256 (relative 3e-5 of the 32-value block maximum).
 *
 * Weight bytes are read straight from the raw GGUF rows (the reference uploads raw GGUF bytes,
 * src/gpu.rs:79-83): Q4_K super-blocks are 16-byte aligned and are read with 128-bit loads; the
 * other types are only 2-byte aligned and use unaligned 64/128-bit loads.
 */
#pragma once
#include <hip/hip_runtime.h>
#include <stdint.h>

#include "le_formats.h"

typedef uint8_t u8;
typedef uint32_t u32;

#define LE_XSPLIT 16256.0f /* 127 * 128: |v| <= 16256 so xh = (v+64)>>7 in [-127,127], xl in [-64,63] */

template <typename T>
__device__ __forceinline__ T ldu(const u8 *p) {
    T v;
    __builtin_memcpy(&v, p, sizeof(T));
    return v;
}

__device__ __forceinline__ float h2f(u32 bits16) {
    return (float)__builtin_bit_cast(_Float16, (uint16_t)bits16);
}

__device__ __forceinline__ int dot4(u32 a, u32 b, int c) {
    return __builtin_amdgcn_sdot4((int)a, (int)b, c, false);
}

/* LDS image of one token's activations: per 8-value group p, xq[p] = {xh word0, xh word1,
 * xl word0, xl word1}, fs[p] = dx * sum(v); per 32-value unit u, dx[u]. */
struct XTok {
    const uint4 *xq;
    const float *fs;
    const float *dx;
};

/* Bytes of LDS needed for one token's activation image of K values. */
__host__ __device__ inline int le_xtok_bytes(int K) { return (K / 8) * 16 + (K / 8) * 4 + (K / 32) * 4; }

/* Quantize one token's K activations (K % 32 == 0) into the LDS image. Called by all threads of
 * the block; 4 consecutive threads share a 32-value unit. */
__device__ __forceinline__ void le_quant_x_lds(const float *__restrict__ x, int K, uint4 *xq, float *fs, float *dx) {
    const int ng = K >> 3;
    for (int p = threadIdx.x; p < ((ng + 3) & ~3); p += blockDim.x) {
        const bool ok = p < ng;
        float4 a = make_float4(0.f, 0.f, 0.f, 0.f), b = a;
        if (ok) {
            a = *(const float4 *)(x + 8 * p);
            b = *(const float4 *)(x + 8 * p + 4);
        }
        float am = fmaxf(fmaxf(fmaxf(fabsf(a.x), fabsf(a.y)), fmaxf(fabsf(a.z), fabsf(a.w))),
                         fmaxf(fmaxf(fabsf(b.x), fabsf(b.y)), fmaxf(fabsf(b.z), fabsf(b.w))));
        am = fmaxf(am, __shfl_xor(am, 1));
        am = fmaxf(am, __shfl_xor(am, 2));
        const float inv = am > 0.f ? LE_XSPLIT / am : 0.f;
        const float d = am / LE_XSPLIT;
        int v[8] = {(int)rintf(a.x * inv), (int)rintf(a.y * inv), (int)rintf(a.z * inv), (int)rintf(a.w * inv),
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
        if (ok) {
            xq[p] = make_uint4(hw[0], hw[1], lw[0], lw[1]);
            fs[p] = d * (float)s;
            if ((p & 3) == 0) dx[p >> 2] = d;
        }
    }
}

/* One lane's decoded share of a super-block: 8 int8x4 words (group k uses w[2k], w[2k+1]),
 * the activation group index p[k], and the scales of each group. */
struct Dec {
    u32 w[8];
    int p[4];
    float sig[4];
    float mu[4];
};

/* Integer dot of one decoded group against one token's LDS image, returned already scaled. */
template <bool HAS_MU>
__device__ __forceinline__ float group_dot(const Dec &d, int k, const XTok &x) {
    const uint4 q = x.xq[d.p[k]];
    const int hi = dot4(d.w[2 * k], q.x, dot4(d.w[2 * k + 1], q.y, 0));
    const int lo = dot4(d.w[2 * k], q.z, dot4(d.w[2 * k + 1], q.w, 0));
    const float a = (float)((hi << 7) + lo) * x.dx[d.p[k] >> 2];
    if (HAS_MU) return d.sig[k] * a - d.mu[k] * x.fs[d.p[k]];
    return d.sig[k] * a;
}

template <int TY>
struct Fmt;

/* ---------------- Q4_K: 144 B = d f16, dmin f16, 12 B packed 6-bit scales/mins, 128 B nibbles.
 * Lane li: pair g = li>>1 of 64 values (low nibbles -> sub-block 2g, high -> 2g+1, per
 * src/quant.rs:74-80), half hh = li&1 of the 32 nibble bytes. */
template <>
struct Fmt<LE_TYPE_Q4_K> {
    static constexpr int SB = LE_SB_BYTES_Q4_K;
    static constexpr bool HAS_MU = true;
    static constexpr bool TABLES = false;
    struct Raw {
        uint4 h, q;
    };
    __device__ static __forceinline__ Raw load(const u8 *p, int li) {
        Raw r;
        r.h = *(const uint4 *)p;
        r.q = *(const uint4 *)(p + 16 + 16 * li);
        return r;
    }
    __device__ static __forceinline__ void decode(const Raw &r, int li, int sb, const u32 *, Dec &d) {
        const int g = li >> 1, hh = li & 1;
        const u32 q[4] = {r.q.x, r.q.y, r.q.z, r.q.w};
#pragma unroll
        for (int i = 0; i < 4; i++) {
            d.w[i] = q[i] & 0x0F0F0F0Fu;              /* groups 0,1: low nibbles */
            d.w[4 + i] = (q[i] >> 4) & 0x0F0F0F0Fu;   /* groups 2,3: high nibbles */
        }
        /* scale_min_k4 (src/quant.rs:52-55) for j = 2g, 2g+1, four bytes at a time */
        const u32 sy = r.h.y, sz = r.h.z, sw = r.h.w;
        const u32 tsc = g < 2 ? sy : ((sw & 0x0F0F0F0Fu) | ((sy >> 2) & 0x30303030u));
        const u32 tm = g < 2 ? sz : (((sw >> 4) & 0x0F0F0F0Fu) | ((sz >> 2) & 0x30303030u));
        const int sh = (g & 1) * 16;
        const float dd = h2f(r.h.x & 0xFFFFu), dm = h2f(r.h.x >> 16);
        const float sa = dd * (float)((tsc >> sh) & 63u), sb2 = dd * (float)((tsc >> (sh + 8)) & 63u);
        const float ma = dm * (float)((tm >> sh) & 63u), mb = dm * (float)((tm >> (sh + 8)) & 63u);
        const int pa = (sb * 8 + 2 * g) * 4 + 2 * hh;
        d.p[0] = pa; d.p[1] = pa + 1; d.p[2] = pa + 4; d.p[3] = pa + 5;
        d.sig[0] = sa; d.sig[1] = sa; d.sig[2] = sb2; d.sig[3] = sb2;
        d.mu[0] = ma; d.mu[1] = ma; d.mu[2] = mb; d.mu[3] = mb;
    }
};

/* ---------------- Q6_K: 210 B = ql[128], qh[64], int8 scales[16], d f16 (src/quant.rs:96-112).
 * Lane li: half n = li>>2 (128 values), l-range [8t, 8t+8) with t = li&3, all four quadrants.
 * The stored 6-bit code q is used unsigned; the -32 offset goes into mu = 32*d*sc. */
template <>
struct Fmt<LE_TYPE_Q6_K> {
    static constexpr int SB = LE_SB_BYTES_Q6_K;
    static constexpr bool HAS_MU = true;
    static constexpr bool TABLES = false;
    struct Raw {
        uint2 la, lb, qh, sc;
        u32 d;
    };
    __device__ static __forceinline__ Raw load(const u8 *p, int li) {
        const int n = li >> 2, t = li & 3;
        Raw r;
        r.la = ldu<uint2>(p + n * 64 + 8 * t);
        r.lb = ldu<uint2>(p + n * 64 + 32 + 8 * t);
        r.qh = ldu<uint2>(p + 128 + n * 32 + 8 * t);
        r.sc = ldu<uint2>(p + 192 + n * 8);
        r.d = ldu<uint16_t>(p + 208);
        return r;
    }
    __device__ static __forceinline__ void decode(const Raw &r, int li, int sb, const u32 *, Dec &d) {
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
        const u32 scw = is ? (r.sc.x >> 8) | (r.sc.y << 24) : r.sc.x; /* bytes is, is+1, ... */
        const u32 scw2 = is ? (r.sc.y >> 8) : r.sc.y;
        /* quadrant qd uses sc[is + 2*qd]: qd 0,1 -> scw bytes 0,2; qd 2,3 -> scw2 bytes 0,2 */
        const int s0 = (int)(int8_t)(scw & 255u), s1 = (int)(int8_t)((scw >> 16) & 255u);
        const int s2 = (int)(int8_t)(scw2 & 255u), s3 = (int)(int8_t)((scw2 >> 16) & 255u);
        const int ub = sb * 8 + n * 4;
#pragma unroll
        for (int k = 0; k < 4; k++) d.p[k] = (ub + k) * 4 + t;
        d.sig[0] = dd * (float)s0; d.sig[1] = dd * (float)s1; d.sig[2] = dd * (float)s2; d.sig[3] = dd * (float)s3;
#pragma unroll
        for (int k = 0; k < 4; k++) d.mu[k] = 32.0f * d.sig[k];
    }
};

/* ---------------- Q8_0 (8 blocks of 34 B = d f16 + 32 int8 per 256 values, src/quant.rs:68-71).
 * Lane li owns block li of the super-block. */
template <>
struct Fmt<LE_TYPE_Q8_0> {
    static constexpr int SB = LE_SB_BYTES_Q8_0;
    static constexpr bool HAS_MU = false;
    static constexpr bool TABLES = false;
    struct Raw {
        uint4 a, b;
        u32 d;
    };
    __device__ static __forceinline__ Raw load(const u8 *p, int li) {
        const u8 *bp = p + 34 * li;
        Raw r;
        r.d = ldu<uint16_t>(bp);
        r.a = ldu<uint4>(bp + 2);
        r.b = ldu<uint4>(bp + 18);
        return r;
    }
    __device__ static __forceinline__ void decode(const Raw &r, int li, int sb, const u32 *, Dec &d) {
        d.w[0] = r.a.x; d.w[1] = r.a.y; d.w[2] = r.a.z; d.w[3] = r.a.w;
        d.w[4] = r.b.x; d.w[5] = r.b.y; d.w[6] = r.b.z; d.w[7] = r.b.w;
        const float dd = h2f(r.d);
        const int u = sb * 8 + li;
#pragma unroll
        for (int k = 0; k < 4; k++) { d.p[k] = u * 4 + k; d.sig[k] = dd; d.mu[k] = 0.f; }
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
    struct Raw {
        uint2 q;
        u32 d;
    };
    __device__ static __forceinline__ Raw load(const u8 *p, int li) {
        Raw r;
        r.d = ldu<uint16_t>(p);
        r.q = ldu<uint2>(p + 2 + 8 * li);
        return r;
    }
    __device__ static __forceinline__ void decode(const Raw &r, int li, int sb, const u32 *tab, Dec &d) {
        const u32 aux = r.q.y;
        const float db = h2f(r.d) * (0.5f + (float)(aux >> 28)) * 0.25f;
        const u32 *grid = tab + LE_TAB_GRID, *sg = tab + LE_TAB_SIGN;
#pragma unroll
        for (int l = 0; l < 4; l++) {
            const u32 gi = (r.q.x >> (8 * l)) & 255u, si = (aux >> (7 * l)) & 127u;
            const uint2 g = *(const uint2 *)(grid + 2 * gi);
            const uint2 m = *(const uint2 *)(sg + 2 * si);
            d.w[2 * l] = apply_sign(g.x, m.x);
            d.w[2 * l + 1] = apply_sign(g.y, m.y);
        }
        const int u = sb * 8 + li;
#pragma unroll
        for (int k = 0; k < 4; k++) { d.p[k] = u * 4 + k; d.sig[k] = db; d.mu[k] = 0.f; }
    }
};

/* ---------------- IQ3_XXS: 98 B = d f16, qs[64] grid indices, 8 x u32 signs/scale (src/quant.rs:127-141). */
template <>
struct Fmt<LE_TYPE_IQ3_XXS> {
    static constexpr int SB = LE_SB_BYTES_IQ3_XXS;
    static constexpr bool HAS_MU = false;
    static constexpr bool TABLES = true;
    static constexpr int GRID_WORDS = 256;
    struct Raw {
        uint2 q;
        u32 aux, d;
    };
    __device__ static __forceinline__ Raw load(const u8 *p, int li) {
        Raw r;
        r.d = ldu<uint16_t>(p);
        r.q = ldu<uint2>(p + 2 + 8 * li);
        r.aux = ldu<u32>(p + 66 + 4 * li);
        return r;
    }
    __device__ static __forceinline__ void decode(const Raw &r, int li, int sb, const u32 *tab, Dec &d) {
        const u32 aux = r.aux;
        const float db = h2f(r.d) * (0.5f + (float)(aux >> 28)) * 0.5f;
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
        const int u = sb * 8 + li;
#pragma unroll
        for (int k = 0; k < 4; k++) { d.p[k] = u * 4 + k; d.sig[k] = db; d.mu[k] = 0.f; }
    }
};
