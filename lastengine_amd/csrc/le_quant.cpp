/* CPU quantizers and the seeded normal generator declared in include/le_quant.h.
 *
 * The reference ships no quantizer (src/quant.rs only dequantizes), so these are written from the
 * block layouts that src/quant.rs:59-170 decodes:
 *   Q8_0    per 32: d = amax/127 (f16), q = round(x/d)
 *   Q4_K    per 32 sub-block: scale = (max-min)/15, min = -min(0,min); the eight scales and mins
 *           are coded as 6-bit multiples of per-block f16 d and dmin and packed as scale_min_k4
 *           reads them (src/quant.rs:52-55); q = round((x + dmin*m) / (d*sc)) in [0,15]
 *   Q6_K    per 16 values: scale = amax/31 coded as int8 multiples of an f16 d; q in [-32,31]+32
 *   IQ2_XXS per 32: db = amax/43 coded as d*(0.5+s)/4 (4-bit s); each 8 values -> the grid entry
 *           nearest to their magnitudes (found through a 3^8 ternary lookup), signs with even
 *           parity (the smallest-magnitude value absorbs an odd sign count)
 *   IQ3_XXS per 32: db = amax/62 coded as d*(0.5+s)/2; each 4 values -> nearest grid entry
 *           (8^4 lookup), signs per 8 values with even parity
 */
#include <cmath>
#include <cstdint>
#include <cstring>
#include <mutex>
#include <thread>
#include <vector>

#include "../../include/le_qmm.h"
#include "../../include/le_quant.h"
#include "le_formats.h"
#include "le_iq_tables.h"

namespace {

const uint32_t kIq2Words[512] = LE_IQ2XXS_GRID_WORDS;
const uint32_t kIq3Words[256] = LE_IQ3XXS_GRID_WORDS;

inline uint64_t mix64(uint64_t z) {
    z = (z ^ (z >> 30)) * 0xBF58476D1CE4E5B9ull;
    z = (z ^ (z >> 27)) * 0x94D049BB133111EBull;
    return z ^ (z >> 31);
}

float f16_to_f32(uint16_t h) {
    const uint32_t s = (h >> 15) & 1u, e = (h >> 10) & 0x1fu, m = h & 0x3ffu;
    uint32_t bits;
    if (e == 0) {
        if (m == 0) {
            bits = s << 31;
        } else {
            uint32_t e2 = 113, m2 = m;
            while ((m2 & 0x400u) == 0) { m2 <<= 1; e2--; }
            bits = (s << 31) | (e2 << 23) | ((m2 & 0x3ffu) << 13);
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

inline int nearest_int(float v) { return (int)std::lrintf(v); }
inline int clampi(int v, int lo, int hi) { return v < lo ? lo : v > hi ? hi : v; }
inline void put16(uint8_t *p, uint16_t v) { p[0] = (uint8_t)v; p[1] = (uint8_t)(v >> 8); }
inline void put32(uint8_t *p, uint32_t v) { for (int i = 0; i < 4; i++) p[i] = (uint8_t)(v >> (8 * i)); }

void q8_0_block(const float *x, uint8_t *b) {
    float amax = 0.f;
    for (int i = 0; i < 32; i++) amax = std::fmax(amax, std::fabs(x[i]));
    const uint16_t dh = le_f32_to_f16(amax / 127.f);
    const float d = f16_to_f32(dh), id = d != 0.f ? 1.f / d : 0.f;
    put16(b, dh);
    for (int i = 0; i < 32; i++) b[2 + i] = (uint8_t)(int8_t)clampi(nearest_int(x[i] * id), -127, 127);
}

void q4_k_block(const float *x, uint8_t *b) {
    float scale[8], mins[8];
    for (int j = 0; j < 8; j++) {
        float mn = x[32 * j], mx = x[32 * j];
        for (int i = 1; i < 32; i++) { mn = std::fmin(mn, x[32 * j + i]); mx = std::fmax(mx, x[32 * j + i]); }
        if (mn > 0.f) mn = 0.f;
        scale[j] = (mx - mn) / 15.f;
        mins[j] = -mn;
    }
    float ms = 0.f, mm = 0.f;
    for (int j = 0; j < 8; j++) { ms = std::fmax(ms, scale[j]); mm = std::fmax(mm, mins[j]); }
    const uint16_t dh = le_f32_to_f16(ms / 63.f), mh = le_f32_to_f16(mm / 63.f);
    const float d = f16_to_f32(dh), dmin = f16_to_f32(mh);
    uint8_t sc[8], m[8];
    for (int j = 0; j < 8; j++) {
        sc[j] = (uint8_t)(d > 0.f ? clampi(nearest_int(scale[j] / d), 0, 63) : 0);
        m[j] = (uint8_t)(dmin > 0.f ? clampi(nearest_int(mins[j] / dmin), 0, 63) : 0);
    }
    put16(b, dh);
    put16(b + 2, mh);
    uint8_t *s = b + 4;
    memset(s, 0, 12);
    for (int j = 0; j < 8; j++) {
        if (j < 4) {
            s[j] |= sc[j] & 63;
            s[j + 4] |= m[j] & 63;
        } else {
            s[j + 4] = (uint8_t)((sc[j] & 15) | ((m[j] & 15) << 4));
            s[j - 4] |= (uint8_t)((sc[j] >> 4) << 6);
            s[j] |= (uint8_t)((m[j] >> 4) << 6);
        }
    }
    uint8_t q[256];
    for (int j = 0; j < 8; j++) {
        const float ds = d * (float)sc[j], dm = dmin * (float)m[j];
        for (int i = 0; i < 32; i++)
            q[32 * j + i] = (uint8_t)(ds > 0.f ? clampi(nearest_int((x[32 * j + i] + dm) / ds), 0, 15) : 0);
    }
    uint8_t *qs = b + 16;
    for (int g = 0; g < 4; g++)
        for (int l = 0; l < 32; l++) qs[g * 32 + l] = (uint8_t)(q[g * 64 + l] | (q[g * 64 + 32 + l] << 4));
}

void q6_k_block(const float *x, uint8_t *b) {
    float scale[16], ms = 0.f;
    for (int s = 0; s < 16; s++) {
        float amax = 0.f;
        for (int i = 0; i < 16; i++) amax = std::fmax(amax, std::fabs(x[16 * s + i]));
        scale[s] = amax / 31.f;
        ms = std::fmax(ms, scale[s]);
    }
    const uint16_t dh = le_f32_to_f16(ms / 127.f);
    const float d = f16_to_f32(dh);
    memset(b, 0, 210);
    int8_t sc[16];
    for (int s = 0; s < 16; s++) sc[s] = (int8_t)(d > 0.f ? clampi(nearest_int(scale[s] / d), -128, 127) : 0);
    for (int p = 0; p < 256; p++) {
        const float ds = d * (float)sc[p / 16];
        const int q = (ds != 0.f ? clampi(nearest_int(x[p] / ds), -32, 31) : 0) + 32;
        const int n = p / 128, r = p % 128, qd = r / 32, l = r % 32;
        uint8_t &ql = b[n * 64 + l + 32 * (qd & 1)];
        ql |= (uint8_t)((qd & 2) ? ((q & 15) << 4) : (q & 15));
        b[128 + n * 32 + l] |= (uint8_t)(((q >> 4) & 3) << (2 * qd));
    }
    for (int s = 0; s < 16; s++) b[192 + s] = (uint8_t)sc[s];
    put16(b + 208, dh);
}

/* Nearest-grid lookups: IQ2_XXS magnitudes {8,25,43} per value -> ternary code (3^8 = 6561);
 * IQ3_XXS magnitudes {4,12,...,52,62} -> octal code (8^4 = 4096). Each code maps to the grid
 * entry nearest (L2) to the code's magnitude vector. */
struct IqLut {
    std::vector<uint8_t> iq2, iq3;
    IqLut() : iq2(6561), iq3(4096) {
        static const int lev2[3] = {8, 25, 43};
        for (int c = 0; c < 6561; c++) {
            int v[8], t = c;
            for (int i = 0; i < 8; i++) { v[i] = lev2[t % 3]; t /= 3; }
            long best = -1; int bi = 0;
            for (int g = 0; g < 256; g++) {
                long e = 0;
                for (int i = 0; i < 8; i++) {
                    const int gv = (int)((kIq2Words[2 * g + (i >> 2)] >> (8 * (i & 3))) & 255u);
                    e += (long)(gv - v[i]) * (gv - v[i]);
                }
                if (best < 0 || e < best) { best = e; bi = g; }
            }
            iq2[c] = (uint8_t)bi;
        }
        static const int lev3[8] = {4, 12, 20, 28, 36, 44, 52, 62};
        for (int c = 0; c < 4096; c++) {
            int v[4];
            for (int i = 0; i < 4; i++) v[i] = lev3[(c >> (3 * i)) & 7];
            long best = -1; int bi = 0;
            for (int g = 0; g < 256; g++) {
                long e = 0;
                for (int i = 0; i < 4; i++) {
                    const int gv = (int)((kIq3Words[g] >> (8 * i)) & 255u);
                    e += (long)(gv - v[i]) * (gv - v[i]);
                }
                if (best < 0 || e < best) { best = e; bi = g; }
            }
            iq3[c] = (uint8_t)bi;
        }
    }
};

const IqLut &lut() {
    static IqLut l;
    return l;
}

int nearest_level(float a, const int *lev, int n) {
    int bi = 0;
    float be = std::fabs(a - (float)lev[0]);
    for (int i = 1; i < n; i++) {
        const float e = std::fabs(a - (float)lev[i]);
        if (e < be) { be = e; bi = i; }
    }
    return bi;
}

/* Seven stored sign bits of 8 values, forcing an even count of negatives. */
uint32_t signs7(const float *x) {
    uint32_t s = 0;
    int neg = 0, smallest = 0;
    for (int i = 0; i < 8; i++) {
        if (x[i] < 0.f) { s |= 1u << i; neg++; }
        if (std::fabs(x[i]) < std::fabs(x[smallest])) smallest = i;
    }
    if (neg & 1) s ^= 1u << smallest;
    return s & 127u;
}

void iq2_xxs_block(const float *x, uint8_t *b) {
    static const int lev[3] = {8, 25, 43};
    const IqLut &L = lut();
    float dbs[8], mdb = 0.f;
    for (int ib = 0; ib < 8; ib++) {
        float amax = 0.f;
        for (int i = 0; i < 32; i++) amax = std::fmax(amax, std::fabs(x[32 * ib + i]));
        dbs[ib] = amax / 43.f;
        mdb = std::fmax(mdb, dbs[ib]);
    }
    const uint16_t dh = le_f32_to_f16(mdb / (15.5f * 0.25f));
    const float d = f16_to_f32(dh);
    put16(b, dh);
    for (int ib = 0; ib < 8; ib++) {
        const float *xs = x + 32 * ib;
        const int s = d > 0.f ? clampi(nearest_int(dbs[ib] / (d * 0.25f) - 0.5f), 0, 15) : 0;
        const float db = d * (0.5f + (float)s) * 0.25f, idb = db > 0.f ? 1.f / db : 0.f;
        uint8_t *q = b + 2 + 8 * ib;
        uint32_t aux = (uint32_t)s << 28;
        for (int l = 0; l < 4; l++) {
            int code = 0;
            for (int i = 7; i >= 0; i--) code = code * 3 + nearest_level(std::fabs(xs[8 * l + i]) * idb, lev, 3);
            q[l] = L.iq2[code];
            aux |= signs7(xs + 8 * l) << (7 * l);
        }
        put32(q + 4, aux);
    }
}

void iq3_xxs_block(const float *x, uint8_t *b) {
    static const int lev[8] = {4, 12, 20, 28, 36, 44, 52, 62};
    const IqLut &L = lut();
    float dbs[8], mdb = 0.f;
    for (int ib = 0; ib < 8; ib++) {
        float amax = 0.f;
        for (int i = 0; i < 32; i++) amax = std::fmax(amax, std::fabs(x[32 * ib + i]));
        dbs[ib] = amax / 62.f;
        mdb = std::fmax(mdb, dbs[ib]);
    }
    const uint16_t dh = le_f32_to_f16(mdb / (15.5f * 0.5f));
    const float d = f16_to_f32(dh);
    put16(b, dh);
    for (int ib = 0; ib < 8; ib++) {
        const float *xs = x + 32 * ib;
        const int s = d > 0.f ? clampi(nearest_int(dbs[ib] / (d * 0.5f) - 0.5f), 0, 15) : 0;
        const float db = d * (0.5f + (float)s) * 0.5f, idb = db > 0.f ? 1.f / db : 0.f;
        uint32_t aux = (uint32_t)s << 28;
        for (int k = 0; k < 8; k++) {
            int code = 0;
            for (int i = 0; i < 4; i++) code |= nearest_level(std::fabs(xs[4 * k + i]) * idb, lev, 8) << (3 * i);
            b[2 + 8 * ib + k] = L.iq3[code];
        }
        for (int l = 0; l < 4; l++) aux |= signs7(xs + 8 * l) << (7 * l);
        put32(b + 66 + 4 * ib, aux);
    }
}

template <typename Fn>
void parallel_rows(size_t rows, int nthreads, Fn fn) {
    if (nthreads < 1) nthreads = 1;
    if ((size_t)nthreads > rows) nthreads = (int)(rows ? rows : 1);
    if (nthreads == 1) {
        fn((size_t)0, rows);
        return;
    }
    std::vector<std::thread> th;
    const size_t per = (rows + nthreads - 1) / nthreads;
    for (int t = 0; t < nthreads; t++) {
        const size_t r0 = std::min(rows, t * per), r1 = std::min(rows, (t + 1) * per);
        th.emplace_back([=] { fn(r0, r1); });
    }
    for (auto &t : th) t.join();
}

}  // namespace

extern "C" {

uint16_t le_f32_to_f16(float f) {
    uint32_t x;
    memcpy(&x, &f, 4);
    const uint32_t sign = (x >> 16) & 0x8000u;
    const uint32_t ax = x & 0x7fffffffu;
    if (ax >= 0x7f800000u) return (uint16_t)(sign | (ax > 0x7f800000u ? 0x7e00u : 0x7c00u));
    if (ax >= 0x477ff000u) return (uint16_t)(sign | 0x7c00u); /* rounds to >= 65520 -> inf */
    if (ax < 0x38800000u) {                                   /* half subnormal or zero */
        if (ax < 0x33000000u) return (uint16_t)sign;          /* < 2^-25 rounds to 0 */
        const uint32_t e = ax >> 23, m = (ax & 0x7fffffu) | 0x800000u;
        const int shift = 126 - (int)e; /* 14..24 */
        uint32_t r = m >> shift;
        const uint32_t rem = m & ((1u << shift) - 1), half = 1u << (shift - 1);
        if (rem > half || (rem == half && (r & 1))) r++;
        return (uint16_t)(sign | r);
    }
    uint32_t r = ((ax >> 13) - (112u << 10));
    const uint32_t rem = ax & 0x1fffu;
    if (rem > 0x1000u || (rem == 0x1000u && (r & 1))) r++;
    return (uint16_t)(sign | r);
}

void le_fill_normal(float *dst, size_t n, uint64_t seed, uint64_t offset, double mean, double std, int nthreads) {
    const uint64_t gamma = 0x9E3779B97F4A7C15ull;
    parallel_rows((n + 4095) / 4096, nthreads, [&](size_t c0, size_t c1) {
        for (size_t c = c0; c < c1; c++) {
            const size_t i0 = c * 4096, i1 = std::min(n, i0 + 4096);
            for (size_t i = i0; i < i1; i++) {
                const uint64_t k = offset + i, j = k >> 1;
                const uint64_t a = mix64(seed + (2 * j + 1) * gamma), bb = mix64(seed + (2 * j + 2) * gamma);
                const double u1 = (double)((a >> 11) + 1) * (1.0 / 9007199254740992.0);
                const double u2 = (double)(bb >> 11) * (1.0 / 9007199254740992.0);
                const double r = std::sqrt(-2.0 * std::log(u1)), th = 6.283185307179586 * u2;
                const double z = (k & 1) ? r * std::sin(th) : r * std::cos(th);
                dst[i] = (float)(mean + std * z);
            }
        }
    });
}

int le_quantize_rows(int ty, const float *src, void *dst, size_t rows, size_t cols, int nthreads) {
    int v, bytes;
    if (!le_block_geometry(ty, &v, &bytes)) return LE_ERR_TYPE;
    if (!src || !dst) return LE_ERR_ARG;
    if (cols % (size_t)v) return LE_ERR_SHAPE;
    if (ty == LE_TYPE_IQ2_XXS || ty == LE_TYPE_IQ3_XXS) (void)lut();
    const size_t rb = cols / v * bytes;
    uint8_t *out = (uint8_t *)dst;
    parallel_rows(rows, nthreads, [&](size_t r0, size_t r1) {
        for (size_t r = r0; r < r1; r++)
            for (size_t blk = 0; blk < cols / v; blk++) {
                const float *x = src + r * cols + blk * v;
                uint8_t *b = out + r * rb + blk * bytes;
                switch (ty) {
                case LE_TYPE_Q8_0: q8_0_block(x, b); break;
                case LE_TYPE_Q4_K: q4_k_block(x, b); break;
                case LE_TYPE_Q6_K: q6_k_block(x, b); break;
                case LE_TYPE_IQ2_XXS: iq2_xxs_block(x, b); break;
                case LE_TYPE_IQ3_XXS: iq3_xxs_block(x, b); break;
                }
            }
    });
    return LE_OK;
}

}  // extern "C"
