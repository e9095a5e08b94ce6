/* Host side of the C ABI in include/le_qmm.h.
 *
 * The context owns the gfx950 code objects (hipModuleLoad) and a name -> hipFunction_t table,
 * the MI355X counterpart of the reference's NVRTC module and kernel map (src/gpu.rs:65-76).
 * Launch policy (grid, LDS, kernel variant) mirrors the role of Gpu::mv_ptrs / prefill::mm /
 * DenseGpu::bmm (src/gpu.rs:228-237, src/gpu/prefill.rs:44-56, src/gpu/dense.rs:181-199), with
 * the shapes chosen for 256 CUs and wave64 instead of 32-lane warps.
 */
#include <dlfcn.h>
#include <hip/hip_runtime.h>

#include <cstdarg>
#include <cstdio>
#include <algorithm>
#include <atomic>
#include <cstring>
#include <map>
#include <string>
#include <vector>

#include "../../include/le_qmm.h"
#include "le_formats.h"

namespace {

const char *kParts[] = {"le_qmm_deq", "le_qmm_moe", "le_qmm_mv8", "le_qmm_mv12", "le_qmm_mv14", "le_qmm_mv16", "le_qmm_mv18", "le_qmm_gm",
                        "le_qmm_gq", "le_qmm_gq2", "le_qmm_mv2", "le_qmm_mv11", "le_qmm_mv13", "le_qmm_mv22"};

/* Kernel argument block of le_mv_* (mirrors MvArgs in le_qmm_kernels.hip). */
struct MvArgs {
    const void *const *ptrs;
    const void *w0;
    unsigned long long w_slot_bytes;
    const float *x;
    long long x_slot, x_tok;
    float *y;
    long long y_slot, y_tok;
    int rows, cols, ntok, swiglu;
    const int8_t *xq8;
    const float *xd8;
};

int xtok_bytes(int K) { return (K / 8) * 24; }

/* Kernel argument block of le_moe_* (mirrors MoeArgs in le_qmm_kernels.hip). */
struct MoeArgs {
    const void *gate, *up, *down;
    const float *logits, *h;
    float *out;
    void *ws;
    int *idx_out;
    float *w_out;
    int n_tok, n_exp, k, hidden, ff;
    unsigned int spin_limit;
    void *bar;
    const void *const *gptr, *const *uptr, *const *dptr;
};
/* Barrier area at the start of an MoE workspace (status word, generation word, one 8-byte arrival
 * flag per block of the one-launch kernel, LE_MOE_MAXGRID = 1024 blocks). */
constexpr size_t kMoeBarBytes = 128 + 8 * 1024;
#define LE_MOE_MAX_TOK 65536
int table_bytes(int ty) {
    if (ty == LE_TYPE_IQ2_XXS) return 4 * (256 + 512);
    if (ty == LE_TYPE_IQ3_XXS) return 4 * (256 + 256);
    if (ty == LE_TYPE_IQ2_S) return 4 * (256 + 2048);
    return 0;
}

}  // namespace

/* le_noalloc.hip: device address of the per-GPU GEMM scratch array */
int le_scratch_attach(int device);

struct le_ctx {
    int device = 0;
    int cus = 256;
    size_t lds_limit = 65536;
    /* launch-policy options (le_set_option) */
    int mv_block = 1024;      /* threads per decode (T = 1) matvec block: 512 or 1024 */
    int mv_blocks_per_cu = 1; /* grid cap = CUs * this */
    int mv_shape = 0;        /* (rows, steps) per lane: 0 auto, 1 (1,2), 2 (2,1), 3 (2,2), 4 (4,1) */
    int mq = 1;              /* decode matvec on MFMA where available */
    int mq_waves_auto = 1;   /* double mq_waves for grids smaller than the chip */
    int mq_waves = 4, mq_steps = 2, mq_blocks_per_cu = 2;
    int ms = 1, ms_p = 2;    /* staged MFMA variant and its super-blocks per row and step */
    int rd_nt = 1, rd_u = 4, rd_blocks_per_cu = 1, rd_block = 512; /* le_stream_read probe shape */
    int ms_t = 1;            /* Q4_K with 2..8 tokens per pass on the staged MFMA kernel */
    int gm_mh = 1;           /* le_gemm, Q4_K, 3..8 tokens: the staged f16 MFMA kernel */
    int gm_mh_max = 16;      /* ... up to this many tokens (8 or 16; 16 only where K fits its LDS) */
    int gm_mh_shape = 0;     /* ... its (P, NW) as 10 * P + NW: 0 auto, 14, 18, 24, 22 */
    /* Q8_0 and Q4_0 batch-1 matvec on the staged MFMA kernels, with ms_p80 / ms_p40 super-blocks per
     * item (Q8_0 32000x4096: 29.7 us against the vector kernel's 36.5; Q4_0 14336x4096: 10.7 against
     * 12.6, 4096x4096: 5.4 against 11.1) */
    int ms80 = 1, ms_p80 = 1, ms40 = 1, ms_p40 = 2;
    int ms_wide = 1;         /* down shapes on 12-16 waves, every type but Q6_K and Q8_0 (below) */
    int ms2s = 1, ms_p2s = 1; /* IQ2_S on the Q6_K kernel's map (14336x4096: 13.0 us against the vector kernel's 13.9, 4096x4096: 6.2 against 8.7) */
    int ms3k = 1, ms_p3k = 2; /* Q3_K on the Q6_K kernel's map (14336x4096: 11.7 us against the vector kernel's 15.7, 4096x4096: 5.4 against 9.5) */
    int ms5k = 1, ms_p5k = 1; /* Q5_K the same way (the Q4_K kernel with the fifth bit from qh; 14336x4096: 11.1 us against the vector kernel's 14.5, 4096x4096: 4.9 against 8.5) */
    int mq_q8 = 1;           /* int8 mode on the staged MFMA kernels: Q4_K 14336x4096 13.1 -> 9.9 us, Q6_K 4096x14336
                                27.7 -> 15.3, IQ3_XXS 16.6 -> 15.7 against the vector kernels (IQ2_XXS stays
                                there: 10.5 against 11.3) */
    int mq6 = 1, ms_p6 = 1;  /* Q6_K decode matvec on the staged MFMA kernels, super-blocks per step (1: 1024x4096 5.6 -> 5.0 us,
                                4096x4096 6.3 -> 5.5, 14336x4096 14.8 -> 14.2 against 2) */
    int mqiq = 1, ms_piq = 2; /* IQ2_XXS / IQ3_XXS likewise */
    int moe_fast = 1;        /* decode-shaped MoE kernels */
    int moe_chunk = 1;       /* decode-form MoE above 8 tokens: consecutive calls of at most 8 tokens */
    int moe_mfma = 1;        /* decode-shaped MoE on the staged MFMA kernels where the types allow */
    int moe_fused = 1;       /* ... in one launch with a device-wide barrier where the grid fits */
    int moe_fused_min_tok = 5; /* ... from this many tokens on (config 4, two launches against one: 3 / 4 tokens
                                  41.5 / 47.1 us against 43.0 / 48.3, 5 tokens 61.2 against 55.1) */
    unsigned int moe_spin_limit = 1u << 20; /* polls before a barrier wait gives up (about a second); 0 fails it */
    int moe_prefill = 1;        /* grouped matrix-core form for larger token counts (forced above 64) */
    int moe_prefill_min_tok = 11; /* ... from this many tokens, when the workspace is sized for it (config 4, 8-token
                                     decode calls against the grouped form: 10 tokens 99.6 / 102.3 us, 12 tokens
                                     116.8 / 109.0, 14 tokens 128.5 / 112.9, 16 tokens 117.7 / 116.8) */
    int moe_dn_split = 0;    /* down launch blocks per row tile: 0 auto, 1, 2 */
    std::map<std::string, int> occ; /* resident blocks per CU, by kernel name and LDS bytes */
    int gm_min_m = 5;        /* le_gemm uses the MFMA GEMM from this many tokens on (below: the
                                staged matvec with 2..4 tokens per pass, faster there) */
    int gm_tile = 0;         /* MFMA GEMM tile: 0 auto, else 10*TM + TN (TM, TN in 1..2) */
    int gm_ksplit = 0;       /* MFMA GEMM K slices: 0 auto, else 1, 2, 4, 8 */
    int gm_pc = 1;           /* MFMA GEMM with producer/consumer waves */
    int gm_split = 0;        /* 1: activations as two fp16 halves (22 bits); 0: one fp16 value (11 bits) */
    int gm_mh_t16 = 0;       /* 9..16 tokens: one 16-token group instead of two 8-token groups */
    int gq = 1;              /* Q4_K GEMM on the generic kernels (le_gq_*) instead of le_gm_12_* */
    int gq_min_m = 9;        /* other types: smallest M on the matrix-core GEMM (below: vector kernels) */
    int gq_cfg = 0;          /* generic GEMM block shape (tokens x rows, waves): 0 auto, 1 (32x256, 4), 2 (64x256, 4),
                                3 (128x256, 4), 4 (128x128, 4), 5 (64x256, 8), 6 (128x256, 8), 7 (32x256, 8),
                                8 (64x128, 4), 9 (32x128, 4), 10 (128x128, 4); Q4_K only: 11 (128x256, 2x4
                                waves of 64x64), 12 (128x128, 2x4 waves of 64x32) */
    int gq_ksplit = 0;       /* generic GEMM K slices: 0 auto, else 1, 2, 4, 8 */
    int moe_route1 = 1;      /* grouped MoE up to 32 tokens: routing and grouping in one block */
    int mmg_w4 = 1;          /* grouped 32-pair tiles: 4-wave 32 x 128 blocks where 8-wave ones fill half the LDS */
    int mmg_xw = 1;          /* grouped pre-pass: one wave per pair (K <= 4096) instead of one block */
    std::vector<hipModule_t> mods;
    std::map<std::string, hipFunction_t> fns;
    std::string err;

    int fail(int code, const char *fmt, ...) {
        char buf[512];
        va_list ap;
        va_start(ap, fmt);
        vsnprintf(buf, sizeof buf, fmt, ap);
        va_end(ap);
        err = buf;
        return code;
    }
    int hip(hipError_t e, const char *what) {
        if (e == hipSuccess) return LE_OK;
        return fail(LE_ERR_HIP, "%s: %s", what, hipGetErrorString(e));
    }
    hipFunction_t fn(const std::string &name) {
        auto it = fns.find(name);
        if (it != fns.end()) return it->second;
        for (hipModule_t m : mods) {
            hipFunction_t f = nullptr;
            const hipError_t e = hipModuleGetFunction(&f, m, name.c_str());
            /* a miss in one module must not leave a sticky error behind for the caller */
            (void)hipGetLastError();
            if (e == hipSuccess && f) {
                fns[name] = f;
                return f;
            }
        }
        return nullptr;
    }
    /* resident blocks per CU of kernel `name` at this block size and dynamic LDS (0 if unknown) */
    int blocks_per_cu(const std::string &name, int block, size_t lds) {
        const std::string key = name + "/" + std::to_string(block) + "/" + std::to_string(lds);
        auto it = occ.find(key);
        if (it != occ.end()) return it->second;
        hipFunction_t f = fn(name);
        int per_cu = 0;
        if (!f || hipModuleOccupancyMaxActiveBlocksPerMultiprocessor(&per_cu, f, block, lds) != hipSuccess) {
            (void)hipGetLastError();
            per_cu = 0;
        }
        occ[key] = per_cu;
        return per_cu;
    }
    int launch(const std::string &name, dim3 grid, int block, size_t lds, hipStream_t st, void **args) {
        hipFunction_t f = fn(name);
        if (!f) return fail(LE_ERR_MODULE, "kernel %s not found in the loaded code objects", name.c_str());
        return hip(hipModuleLaunchKernel(f, grid.x, grid.y, grid.z, block, 1, 1, (unsigned)lds, st, args, nullptr),
                   name.c_str());
    }
};

namespace {

/* The five types of the decode-shaped MoE kernels. */
bool supported(int ty) {
    return ty == LE_TYPE_Q8_0 || ty == LE_TYPE_Q4_K || ty == LE_TYPE_Q6_K || ty == LE_TYPE_IQ2_XXS ||
           ty == LE_TYPE_IQ3_XXS;
}
/* ... plus Q4_0, Q3_K, Q5_K and IQ2_S: the nine types of dequant, matvec, the matrix-core GEMM, the
 * grouped matmul and the MoE layer (other type pairs than the decode kernels' through its grouped form). */
bool supported_mv(int ty) {
    return supported(ty) || ty == LE_TYPE_Q4_0 || ty == LE_TYPE_Q3_K || ty == LE_TYPE_Q5_K || ty == LE_TYPE_IQ2_S;
}
int sb_bytes(int ty) {
    switch (ty) {
    case LE_TYPE_Q8_0: return LE_SB_BYTES_Q8_0;
    case LE_TYPE_Q4_K: return LE_SB_BYTES_Q4_K;
    case LE_TYPE_Q6_K: return LE_SB_BYTES_Q6_K;
    case LE_TYPE_IQ2_XXS: return LE_SB_BYTES_IQ2_XXS;
    case LE_TYPE_IQ3_XXS: return LE_SB_BYTES_IQ3_XXS;
    case LE_TYPE_Q4_0: return LE_SB_BYTES_Q4_0;
    case LE_TYPE_Q3_K: return LE_SB_BYTES_Q3_K;
    case LE_TYPE_Q5_K: return LE_SB_BYTES_Q5_K;
    case LE_TYPE_IQ2_S: return LE_SB_BYTES_IQ2_S;
    }
    return 0;
}
bool al16(const void *p) { return ((uintptr_t)p & 15) == 0; }

std::string lib_dir_of_this_so() {
    Dl_info info;
    if (dladdr((void *)&lib_dir_of_this_so, &info) && info.dli_fname) {
        std::string p = info.dli_fname;
        size_t s = p.rfind('/');
        if (s != std::string::npos) return p.substr(0, s);
    }
    return ".";
}

/* Lanes per row: G groups of 8 lanes share a row; G is the largest of 8,4,2,1 dividing the
 * super-block count, so every lane group gets the same number of super-blocks. */
int pick_g(int nsb) {
    for (int g = 8; g > 1; g >>= 1)
        if (nsb % g == 0) return g;
    return 1;
}

/* MFMA decode matvec (Q4_K, Q6_K): one block of mq_waves waves per 16-row tile at a time. */
int mq_launch(le_ctx *c, int ty, const void *const *ptrs, const void *w, const float *x, long long x_slot, float *y,
              long long y_slot, int rows, int cols, int slots, hipStream_t st, int swiglu = 0, const int8_t *xq8 = nullptr,
              const float *xd8 = nullptr) {
    const long long ntile = (rows + 15) / 16;
    const int nsb = cols / 256, U = c->mq_steps;
    /* when the row tiles alone leave CUs idle, split K over twice the waves (shorter chains) */
    const int NW = c->mq_waves_auto && ntile * slots <= c->cus && c->mq_waves < 8 ? 2 * c->mq_waves : c->mq_waves;
    long long gx = ntile, cap = (long long)c->cus * c->mq_blocks_per_cu;
    if (gx > cap) {
        const long long it = (gx + cap - 1) / cap;
        gx = (gx + it - 1) / it;
    }
    MvArgs a{};
    a.ptrs = ptrs;
    a.w0 = w;
    a.w_slot_bytes = (unsigned long long)rows * nsb * sb_bytes(ty);
    a.x = x;
    a.x_slot = x_slot;
    a.y = y;
    a.y_slot = y_slot;
    a.rows = rows;
    a.cols = cols;
    a.ntok = 1;
    a.swiglu = swiglu;
    a.xq8 = xq8; /* int8 mode: the staged kernels build their image from xq / xd */
    a.xd8 = xd8;
    void *args[] = {&a};
    char name[64];
    size_t lds = (size_t)nsb * 608 + (size_t)NW * 64;
    /* staged variant: P super-blocks per row and item, NWs waves splitting K evenly */
    int P = ty == LE_TYPE_Q6_K ? c->ms_p6 : ty == LE_TYPE_Q4_K ? c->ms_p : ty == LE_TYPE_Q8_0 ? c->ms_p80 : ty == LE_TYPE_Q4_0 ? c->ms_p40 : ty == LE_TYPE_Q5_K ? c->ms_p5k : ty == LE_TYPE_Q3_K ? c->ms_p3k : ty == LE_TYPE_IQ2_S ? c->ms_p2s : c->ms_piq, NWs = NW;
    while (P > 1 && nsb % P) P >>= 1;
    /* keep the waves and give up super-blocks per item when both do not divide K (4096 x 14336, 56
     * super-blocks, P=1 on 8 waves against P=2 on 4: Q6_K 14.1 against 16.0 us, Q4_K 10.6 / 12.1,
     * Q4_0 13.6 / 14.0, Q3_K 13.4 / 14.0, IQ2_S 12.7 / 16.1); IQ3_XXS keeps P (15.4 against 20.0
     * us; its down shapes take the wider split below) */
    if (ty != LE_TYPE_IQ3_XXS && nsb % (NWs * P) && nsb % NWs == 0) P = 1;
    /* with no more row tiles than CUs and K of 48 super-blocks or more (a down projection: one tile
     * per block), K is split over 12-16 waves of two super-blocks each: 4096 x 14336 IQ3_XXS 15.5
     * -> 12.8 us, IQ2_XXS 12.1 -> 10.9, IQ2_S 13.2 -> 12.5, Q4_0 13.9 -> 10.8, Q4_K 10.6 -> 9.8,
     * Q5_K 12.4 -> 11.7, Q3_K 13.6 -> 12.4; IQ3_XXS 4096 x 12288 11.9 -> 11.0 (2048 x 8192, 32
     * super-blocks: 8.2 -> 8.8, so not there); Q6_K 14.3 -> 14.8 and Q8_0 17.0 -> 28.4 lose */
    if (ty != LE_TYPE_Q6_K && ty != LE_TYPE_Q8_0 && c->ms_wide && (rows + 15) / 16 * (long long)slots <= c->cus && nsb >= 48 && nsb % 2 == 0)
        for (const int w : {16, 14, 12})
            if ((nsb / 2) % w == 0) { NWs = w; P = 2; break; }
    while (NWs > 1 && nsb % (NWs * P)) NWs >>= 1;
    /* only some (P, NWs) pairs are instantiated (e.g. no P = 4 with 8 waves): lower P until the
     * kernel exists, else fall through to the unstaged or vector kernels */
    while (c->ms && P > 1 && !c->fn(std::string("le_ms_") + std::to_string(ty) + "_p" + std::to_string(P) + "_w" +
                                    std::to_string(NWs) + (xq8 ? "_q8" : "")))
        P >>= 1;
    if (c->ms && nsb % (NWs * P) == 0 &&
        c->fn(std::string("le_ms_") + std::to_string(ty) + "_p" + std::to_string(P) + "_w" + std::to_string(NWs) + (xq8 ? "_q8" : ""))) {
        const int cps = ty == LE_TYPE_Q6_K ? 14 : ty == LE_TYPE_IQ2_XXS ? 5 : ty == LE_TYPE_IQ3_XXS ? 7 : ty == LE_TYPE_Q8_0 ? 17 : ty == LE_TYPE_Q5_K ? 11 : ty == LE_TYPE_Q3_K ? 7 : ty == LE_TYPE_IQ2_S ? 6 : 9;
        const int cpr = cps * P + 1, ni = (16 * cpr + 63) / 64;
        snprintf(name, sizeof name, "le_ms_%d_p%d_w%d%s", ty, P, NWs, xq8 ? "_q8" : "");
        lds = (size_t)NWs * ((size_t)(nsb / NWs) * 608 + (size_t)ni * 1024) + (size_t)NWs * 128;
        if (lds <= c->lds_limit)
            return c->launch(name, dim3((unsigned)gx, (unsigned)slots), NWs * 64, lds, st, args);
        lds = (size_t)nsb * 608 + (size_t)NW * 64;
    }
    /* no unstaged MFMA variant for the other types, nor one that forms silu(gate) * up: the caller
     * falls back to the vector kernels */
    if (ty != LE_TYPE_Q4_K || swiglu || xq8) return 1;
    snprintf(name, sizeof name, "le_mq_12_w%d_u%d", NW, U);
    return c->launch(name, dim3((unsigned)gx, (unsigned)slots), NW * 64, lds, st, args);
}

/* Q4_K for 2..8 tokens (per pass) on the staged MFMA kernel: grid (row-tile workers, slots,
 * token groups of T). Returns 1 when no instantiated shape fits (the caller falls back). */
int ms_t_launch(le_ctx *c, const void *const *ptrs, const void *w, const float *x, long long x_slot, long long x_tok,
                float *y, long long y_slot, long long y_tok, int rows, int cols, int ntok, int slots, hipStream_t st) {
    const long long ntile = (rows + 15) / 16;
    const int nsb = cols / 256;
    const int T = ntok <= 2 ? 2 : ntok <= 4 ? 4 : 8;
    const long long groups = (ntok + T - 1) / T;
    const bool wide = c->mq_waves_auto && ntile * slots * groups <= c->cus;
    /* (P, NW) shapes that are instantiated, in order of preference */
    static const int kWide[4][2] = {{1, 8}, {1, 4}, {2, 4}, {2, 2}}, kStd[3][2] = {{1, 4}, {2, 4}, {2, 2}};
    const int(*cand)[2] = wide ? kWide : kStd;
    const int ncand = wide ? 4 : 3;
    for (int i = 0; i < ncand; i++) {
        const int P = cand[i][0], NW = cand[i][1];
        if (P > c->ms_p || nsb % (NW * P)) continue;
        const int ni = (16 * (9 * P + 1) + 63) / 64;
        const size_t lds = (size_t)NW * ((size_t)T * (nsb / NW) * 624 + (size_t)ni * 1024) + (size_t)NW * T * 128;
        if (lds > c->lds_limit) continue;
        char name[64];
        snprintf(name, sizeof name, "le_ms_12_p%d_w%d_t%d", P, NW, T);
        /* every block quantizes its tokens once, so the grid is what stays resident (blocks then
         * loop over row tiles) */
        const int per_cu = c->blocks_per_cu(name, NW * 64, lds);
        long long gx = ntile, cap = (long long)c->cus * (per_cu > 0 ? per_cu : 1);
        const long long per_slot = (cap + slots * groups - 1) / (slots * groups);
        if (gx > per_slot) {
            const long long it = (gx + per_slot - 1) / per_slot;
            gx = (gx + it - 1) / it;
        }
        MvArgs a{};
        a.ptrs = ptrs;
        a.w0 = w;
        a.w_slot_bytes = (unsigned long long)rows * nsb * sb_bytes(LE_TYPE_Q4_K);
        a.x = x;
        a.x_slot = x_slot;
        a.x_tok = x_tok;
        a.y = y;
        a.y_slot = y_slot;
        a.y_tok = y_tok;
        a.rows = rows;
        a.cols = cols;
        a.ntok = ntok;
        void *args[] = {&a};
        return c->launch(name, dim3((unsigned)gx, (unsigned)slots, (unsigned)groups), NW * 64, lds, st, args);
    }
    return 1;
}

/* Matvec/matmul launcher: T tokens per pass, grid (workers, slots, ceil(ntok/T)). */
int mv_launch(le_ctx *c, int ty, const void *const *ptrs, const void *w, const float *x, long long x_slot,
              long long x_tok, float *y, long long y_slot, long long y_tok, int rows, int cols, int ntok, int slots,
              hipStream_t st,
              const int8_t *xq8 = nullptr, const float *xd8 = nullptr, int swiglu = 0) {
    if (!supported_mv(ty)) return c->fail(LE_ERR_TYPE, "no kernel for type %d", ty);
    if (rows <= 0 || cols <= 0 || ntok <= 0 || slots <= 0) return c->fail(LE_ERR_SHAPE, "empty shape");
    if (cols % 256) return c->fail(LE_ERR_SHAPE, "cols=%d is not a multiple of 256", cols);
    const bool q8 = xq8 != nullptr;
    if (q8) {
        if (!xd8 || !y || (!ptrs && !w)) return c->fail(LE_ERR_ARG, "null pointer");
        if (((uintptr_t)xq8 & 7) || ((uintptr_t)xd8 & 3) || (x_slot % 32) || ntok != 1)
            return c->fail(LE_ERR_ALIGN, "xq must be 8-byte aligned and xstride a multiple of 32");
    } else {
        if (!x || !y || (!ptrs && !w)) return c->fail(LE_ERR_ARG, "null pointer");
        if (!al16(x) || (x_slot % 4) || (x_tok % 4)) return c->fail(LE_ERR_ALIGN, "activations must be 16-byte aligned");
    }
    const int nsb = cols / 256, G = pick_g(nsb), S = nsb / G;
    const bool iq = ty == LE_TYPE_IQ2_XXS || ty == LE_TYPE_IQ3_XXS;
    const bool q80 = (ty == LE_TYPE_Q8_0 && c->ms80) || (ty == LE_TYPE_Q4_0 && c->ms40) || (ty == LE_TYPE_Q5_K && c->ms5k) ||
                     (ty == LE_TYPE_Q3_K && c->ms3k) || (ty == LE_TYPE_IQ2_S && c->ms2s);
    if ((ty == LE_TYPE_Q4_K || (ty == LE_TYPE_Q6_K && c->mq6) || (iq && c->mqiq) || q80) && ntok == 1 && c->mq &&
        (!q8 || (c->mq_q8 && ty != LE_TYPE_IQ2_XXS)) && (size_t)nsb * 608 + 1024 <= c->lds_limit) {
        const int rc = mq_launch(c, ty, ptrs, w, x, x_slot, y, y_slot, rows, cols, slots, st, swiglu, xq8, xd8);
        if (rc != 1) return rc;
    }
    if (!q8 && ty == LE_TYPE_Q4_K && ntok >= 2 && c->mq && c->ms && c->ms_t) {
        const int rc = ms_t_launch(c, ptrs, w, x, x_slot, x_tok, y, y_slot, y_tok, rows, cols, ntok, slots, st);
        if (rc != 1) return rc;
    }
    const int xb = xtok_bytes(cols), tb = table_bytes(ty);
    int T = 1;
    const int want = ntok >= 8 ? 8 : ntok >= 4 ? 4 : ntok >= 2 ? 2 : 1;
    for (int t = want; t >= 1; t >>= 1)
        if ((size_t)(t * xb + tb) <= c->lds_limit) { T = t; break; }
    if ((size_t)(xb + tb) > c->lds_limit) return c->fail(LE_ERR_SHAPE, "cols=%d exceeds the LDS activation budget", cols);
    static const int kRW[5] = {0, 1, 2, 2, 4}, kCH[5] = {0, 2, 1, 2, 1};
    /* default (rows, steps) per lane: measured best at 14336 x 4096 (T = 1) for each type; the
     * formats with three 16-byte loads per super-block and lane (Q5_K, Q3_K, IQ2_S) lose occupancy
     * at 2 x 2 */
    int shape = c->mv_shape;
    if (!shape) {
        if (ty == LE_TYPE_Q5_K || ty == LE_TYPE_Q3_K || ty == LE_TYPE_IQ2_S) shape = 2;
        else if (ty == LE_TYPE_Q4_0) shape = 4;
        else shape = S == 1 ? 4 : 3;
    }
    if (T > 1 && shape < 3) shape = 3;
    const int RW = kRW[shape], CH = kCH[shape];
    const int block = T == 1 ? c->mv_block : 256;
    const int nwave = block / 64;
    const int rpw = 8 / G;
    const long long nrb = (rows + rpw * RW - 1) / (rpw * RW);
    const long long need = (nrb + nwave - 1) / nwave;
    const long long cap = (long long)c->cus * c->mv_blocks_per_cu;
    long long gx = need;
    if (need > cap) {
        const long long iters = (need + cap - 1) / cap;
        gx = (need + iters - 1) / iters;
    }
    MvArgs a{};
    a.ptrs = ptrs;
    a.w0 = w;
    a.w_slot_bytes = (unsigned long long)rows * (unsigned long long)nsb * sb_bytes(ty);
    a.x = x;
    a.x_slot = x_slot;
    a.x_tok = x_tok;
    a.y = y;
    a.y_slot = y_slot;
    a.y_tok = y_tok;
    a.rows = rows;
    a.cols = cols;
    a.ntok = ntok;
    void *args[] = {&a};
    char name[96];
    a.xq8 = xq8;
    a.xd8 = xd8;
    a.swiglu = swiglu;
    snprintf(name, sizeof name, "le_mv_%d_g%d_t%d_r%d_c%d_b%d%s", ty, G, T, RW, CH, block, q8 ? "_q8" : "");
    return c->launch(name, dim3((unsigned)gx, (unsigned)slots, (unsigned)((ntok + T - 1) / T)), block,
                     (size_t)(T * xb + tb), st, args);
}

}  // namespace

extern "C" {

int le_block_info(int ty, int *values, int *bytes) {
    int v, b;
    if (!le_block_geometry(ty, &v, &b)) return LE_ERR_TYPE;
    if (values) *values = v;
    if (bytes) *bytes = b;
    return LE_OK;
}

size_t le_row_bytes(int ty, size_t n) {
    int v, b;
    if (!le_block_geometry(ty, &v, &b)) return 0;
    return n / (size_t)v * (size_t)b;
}

const char *le_status_str(int s) {
    switch (s) {
    case LE_OK: return "ok";
    case LE_ERR_ARG: return "invalid argument";
    case LE_ERR_TYPE: return "unsupported quant type";
    case LE_ERR_SHAPE: return "unsupported shape";
    case LE_ERR_ALIGN: return "misaligned pointer or stride";
    case LE_ERR_HIP: return "HIP runtime error";
    case LE_ERR_MODULE: return "code object missing or device unsupported";
    case LE_ERR_WORKSPACE: return "workspace too small";
    case LE_ERR_TIMEOUT: return "a bounded device-side wait gave up";
    }
    return "unknown status";
}

int le_init(const char *lib_dir, le_ctx **out) {
    if (!out) return LE_ERR_ARG;
    *out = nullptr;
    le_ctx *c = new le_ctx();
    int dev = 0;
    if (hipGetDevice(&dev) != hipSuccess) {
        delete c;
        return LE_ERR_HIP;
    }
    c->device = dev;
    hipDeviceProp_t prop;
    if (hipGetDeviceProperties(&prop, dev) != hipSuccess) {
        delete c;
        return LE_ERR_HIP;
    }
    if (strncmp(prop.gcnArchName, "gfx950", 6) != 0) {
        delete c;
        return LE_ERR_MODULE;
    }
    c->cus = prop.multiProcessorCount;
    c->lds_limit = prop.sharedMemPerBlock;

    const std::string dir = lib_dir ? lib_dir : lib_dir_of_this_so();
    for (const char *part : kParts) {
        hipModule_t m = nullptr;
        const std::string path = dir + "/" + part + ".hsaco";
        if (hipModuleLoad(&m, path.c_str()) != hipSuccess) {
            for (hipModule_t mm : c->mods) (void)hipModuleUnload(mm);
            delete c;
            return LE_ERR_MODULE;
        }
        c->mods.push_back(m);
    }
    if (le_scratch_attach(dev) != LE_OK) {
        for (hipModule_t mm : c->mods) (void)hipModuleUnload(mm);
        delete c;
        return LE_ERR_HIP;
    }
    *out = c;
    return LE_OK;
}

void le_destroy(le_ctx *c) {
    if (!c) return;
    for (hipModule_t m : c->mods) (void)hipModuleUnload(m);
    delete c;
}

const char *le_last_error(const le_ctx *c) { return c ? c->err.c_str() : "null context"; }

int le_set_option(le_ctx *c, const char *name, int value) {
    if (!c || !name) return LE_ERR_ARG;
    const std::string n = name;
    if (n == "mv_block") {
        if (value != 512 && value != 1024) return c->fail(LE_ERR_ARG, "mv_block must be 512 or 1024");
        c->mv_block = value;
    } else if (n == "mv_blocks_per_cu") {
        if (value < 1 || value > 64) return c->fail(LE_ERR_ARG, "mv_blocks_per_cu must be 1..64");
        c->mv_blocks_per_cu = value;
    } else if (n == "mq_waves_auto") {
        c->mq_waves_auto = value ? 1 : 0;
    } else if (n == "mq") {
        c->mq = value ? 1 : 0;
    } else if (n == "mqiq") {
        c->mqiq = value ? 1 : 0;
    } else if (n == "ms_piq") {
        if (value != 1 && value != 2 && value != 4) return c->fail(LE_ERR_ARG, "ms_piq must be 1, 2 or 4");
        c->ms_piq = value;
    } else if (n == "mq6") {
        c->mq6 = value ? 1 : 0;
    } else if (n == "ms_p6") {
        if (value != 1 && value != 2) return c->fail(LE_ERR_ARG, "ms_p6 must be 1 or 2");
        c->ms_p6 = value;
    } else if (n == "gm_split") {
        if (value != 0 && value != 1) return c->fail(LE_ERR_ARG, "gm_split must be 0 or 1");
        c->gm_split = value;
    } else if (n == "rd_nt") {
        c->rd_nt = value ? 1 : 0;
    } else if (n == "rd_u") {
        if (value != 1 && value != 2 && value != 4 && value != 8) return c->fail(LE_ERR_ARG, "rd_u must be 1, 2, 4 or 8");
        c->rd_u = value;
    } else if (n == "rd_blocks_per_cu") {
        if (value < 1 || value > 16) return c->fail(LE_ERR_ARG, "rd_blocks_per_cu must be 1..16");
        c->rd_blocks_per_cu = value;
    } else if (n == "rd_block") {
        if (value != 256 && value != 512) return c->fail(LE_ERR_ARG, "rd_block must be 256 or 512");
        c->rd_block = value;
    } else if (n == "gm_mh_t16") {
        c->gm_mh_t16 = value ? 1 : 0;
    } else if (n == "gq") {
        c->gq = value ? 1 : 0;
    } else if (n == "gq_min_m") {
        if (value < 1) return c->fail(LE_ERR_ARG, "gq_min_m must be >= 1");
        c->gq_min_m = value;
    } else if (n == "gq_cfg") {
        if (value < 0 || value > 12) return c->fail(LE_ERR_ARG, "gq_cfg must be 0..12");
        c->gq_cfg = value;
    } else if (n == "moe_route1") {
        c->moe_route1 = value ? 1 : 0;
    } else if (n == "mmg_w4") {
        c->mmg_w4 = value ? 1 : 0;
    } else if (n == "mmg_xw") {
        c->mmg_xw = value ? 1 : 0;
    } else if (n == "gq_ksplit") {
        if (value != 0 && value != 1 && value != 2 && value != 4 && value != 8)
            return c->fail(LE_ERR_ARG, "gq_ksplit must be 0, 1, 2, 4 or 8");
        c->gq_ksplit = value;
    } else if (n == "gm_pc") {
        c->gm_pc = value ? 1 : 0;
    } else if (n == "gm_ksplit") {
        if (value != 0 && value != 1 && value != 2 && value != 4 && value != 8)
            return c->fail(LE_ERR_ARG, "gm_ksplit must be 0, 1, 2, 4 or 8");
        c->gm_ksplit = value;
    } else if (n == "gm_tile") {
        if (value && (value / 10 < 1 || value / 10 > 2 || value % 10 < 1 || value % 10 > 2))
            return c->fail(LE_ERR_ARG, "gm_tile must be 0, 11, 12, 21 or 22");
        c->gm_tile = value;
    } else if (n == "gm_min_m") {
        c->gm_min_m = value;
    } else if (n == "moe_fused_min_tok") {
        c->moe_fused_min_tok = value;
    } else if (n == "moe_spin_limit") {
        if (value < 0) return c->fail(LE_ERR_ARG, "moe_spin_limit must be >= 0");
        c->moe_spin_limit = (unsigned int)value;
    } else if (n == "moe_prefill") {
        c->moe_prefill = value ? 1 : 0;
    } else if (n == "moe_prefill_min_tok") {
        if (value < 1) return c->fail(LE_ERR_ARG, "moe_prefill_min_tok must be >= 1");
        c->moe_prefill_min_tok = value;
    } else if (n == "moe_dn_split") {
        if (value < 0 || value > 2) return c->fail(LE_ERR_ARG, "moe_dn_split must be 0, 1 or 2");
        c->moe_dn_split = value;
    } else if (n == "moe_fused") {
        c->moe_fused = value ? 1 : 0;
    } else if (n == "moe_mfma") {
        c->moe_mfma = value ? 1 : 0;
    } else if (n == "ms_wide") {
        c->ms_wide = value ? 1 : 0;
    } else if (n == "ms_p2s") {
        if (value != 1 && value != 2 && value != 4) return c->fail(LE_ERR_ARG, "ms_p2s must be 1, 2 or 4");
        c->ms_p2s = value;
    } else if (n == "ms2s") {
        c->ms2s = value ? 1 : 0;
    } else if (n == "ms_p3k") {
        if (value != 1 && value != 2 && value != 4) return c->fail(LE_ERR_ARG, "ms_p3k must be 1, 2 or 4");
        c->ms_p3k = value;
    } else if (n == "ms3k") {
        c->ms3k = value ? 1 : 0;
    } else if (n == "ms_p5k") {
        if (value != 1 && value != 2 && value != 4) return c->fail(LE_ERR_ARG, "ms_p5k must be 1, 2 or 4");
        c->ms_p5k = value;
    } else if (n == "ms5k") {
        c->ms5k = value ? 1 : 0;
    } else if (n == "ms_p40") {
        if (value != 1 && value != 2 && value != 4) return c->fail(LE_ERR_ARG, "ms_p40 must be 1, 2 or 4");
        c->ms_p40 = value;
    } else if (n == "ms40") {
        c->ms40 = value ? 1 : 0;
    } else if (n == "ms_p80") {
        if (value != 1 && value != 2 && value != 4) return c->fail(LE_ERR_ARG, "ms_p80 must be 1, 2 or 4");
        c->ms_p80 = value;
    } else if (n == "ms80") {
        c->ms80 = value ? 1 : 0;
    } else if (n == "mq_q8") {
        c->mq_q8 = value ? 1 : 0;
    } else if (n == "moe_chunk") {
        c->moe_chunk = value ? 1 : 0;
    } else if (n == "moe_fast") {
        c->moe_fast = value ? 1 : 0;
    } else if (n == "ms") {
        c->ms = value ? 1 : 0;
    } else if (n == "gm_mh_shape") {
        if (value != 0 && value != 14 && value != 18 && value != 24 && value != 22)
            return c->fail(LE_ERR_ARG, "gm_mh_shape must be 0, 14, 18, 24 or 22");
        c->gm_mh_shape = value;
    } else if (n == "gm_mh_max") {
        if (value != 8 && value != 16) return c->fail(LE_ERR_ARG, "gm_mh_max must be 8 or 16");
        c->gm_mh_max = value;
    } else if (n == "gm_mh") {
        c->gm_mh = value ? 1 : 0;
    } else if (n == "ms_t") {
        c->ms_t = value ? 1 : 0;
    } else if (n == "ms_p") {
        if (value != 1 && value != 2 && value != 4) return c->fail(LE_ERR_ARG, "ms_p must be 1, 2 or 4");
        c->ms_p = value;
    } else if (n == "mq_waves") {
        if (value != 2 && value != 4 && value != 8) return c->fail(LE_ERR_ARG, "mq_waves must be 2, 4 or 8");
        c->mq_waves = value;
    } else if (n == "mq_steps") {
        if (value != 1 && value != 2 && value != 4) return c->fail(LE_ERR_ARG, "mq_steps must be 1, 2 or 4");
        c->mq_steps = value;
    } else if (n == "mq_blocks_per_cu") {
        if (value < 1 || value > 32) return c->fail(LE_ERR_ARG, "mq_blocks_per_cu must be 1..32");
        c->mq_blocks_per_cu = value;
    } else if (n == "mv_shape") {
        if (value < 0 || value > 4) return c->fail(LE_ERR_ARG, "mv_shape must be 0..4");
        c->mv_shape = value;
    } else {
        return c->fail(LE_ERR_ARG, "unknown option %s", name);
    }
    return LE_OK;
}

int le_dequant_rows(le_ctx *c, int ty, const void *w, float *out, int rows, int cols, le_stream_t stream) {
    if (!c) return LE_ERR_ARG;
    if (!supported_mv(ty)) return c->fail(LE_ERR_TYPE, "no kernel for type %d", ty);
    if (!w || !out) return c->fail(LE_ERR_ARG, "null pointer");
    int v = 1, b = 0;
    le_block_geometry(ty, &v, &b);
    if (rows <= 0 || cols <= 0 || cols % v || cols % 32) return c->fail(LE_ERR_SHAPE, "bad shape %dx%d", rows, cols);
    if (!al16(out) || (cols % 4)) return c->fail(LE_ERR_ALIGN, "output must be 16-byte aligned");
    unsigned long long rb = (unsigned long long)(cols / v) * b;
    const long long units = (long long)rows * (cols / 32);
    long long blocks = (units + 255) / 256;
    if (blocks > (long long)c->cus * 16) blocks = (long long)c->cus * 16;
    char name[32];
    snprintf(name, sizeof name, "le_dequant_%d", ty);
    void *args[] = {(void *)&w, (void *)&out, (void *)&rows, (void *)&cols, (void *)&rb};
    return c->launch(name, dim3((unsigned)blocks), 256, 0, (hipStream_t)stream, args);
}

int le_matvec(le_ctx *c, int ty, const void *const *ptrs, const void *w, const float *x, long long xstride, float *y,
              int rows, int cols, int slots, le_stream_t stream) {
    if (!c) return LE_ERR_ARG;
    return mv_launch(c, ty, ptrs, w, x, xstride, 0, y, (long long)rows, 0, rows, cols, 1, slots, (hipStream_t)stream);
}

int le_matvec_swiglu(le_ctx *c, int ty, const void *const *ptrs, const void *w, const float *gu, long long xstride,
                     float *y, int rows, int cols, int slots, le_stream_t stream) {
    if (!c) return LE_ERR_ARG;
    if (slots > 1 && xstride != 0 && xstride < 2LL * cols)
        return c->fail(LE_ERR_SHAPE, "xstride must be 0 or at least 2 * cols (gate and up of one slot)");
    return mv_launch(c, ty, ptrs, w, gu, xstride, 0, y, (long long)rows, 0, rows, cols, 1, slots, (hipStream_t)stream,
                     nullptr, nullptr, 1);
}

int le_quant_x(le_ctx *c, const float *x, int8_t *xq, float *xd, int32_t *xs, int n_units, le_stream_t stream) {
    if (!c) return LE_ERR_ARG;
    if (!x || !xq || !xd || !xs) return c->fail(LE_ERR_ARG, "null pointer");
    if (n_units <= 0) return c->fail(LE_ERR_SHAPE, "n_units must be positive");
    const unsigned blocks = (unsigned)((n_units + 7) / 8);
    void *args[] = {(void *)&x, (void *)&xq, (void *)&xd, (void *)&xs, (void *)&n_units};
    return c->launch("le_quant_x", dim3(blocks), 256, 0, (hipStream_t)stream, args);
}

int le_rms_quant(le_ctx *c, const float *x, const float *w, float *o, int8_t *xq, float *xd, int32_t *xs, int n, float eps,
                 le_stream_t stream) {
    if (!c) return LE_ERR_ARG;
    if (!x || !w || !o || !xq || !xd || !xs) return c->fail(LE_ERR_ARG, "null pointer");
    if (n <= 0 || n % 32) return c->fail(LE_ERR_SHAPE, "n=%d is not a positive multiple of 32", n);
    int blocks = (n / 32 + 7) / 8;
    if (blocks > 64) blocks = 64;
    void *args[] = {(void *)&x, (void *)&w, (void *)&o, (void *)&xq, (void *)&xd, (void *)&xs, (void *)&n, (void *)&eps};
    return c->launch("le_rms_quant", dim3((unsigned)blocks), 256, 0, (hipStream_t)stream, args);
}

int le_matvec_q8(le_ctx *c, int ty, const void *const *ptrs, const void *w, const int8_t *xq, const float *xd,
                 const int32_t *xs, long long xstride, float *y, int rows, int cols, int slots, le_stream_t stream) {
    (void)xs; /* the kernels form the group sums they need from xq */
    if (!c) return LE_ERR_ARG;
    if (!xq) return c->fail(LE_ERR_ARG, "null pointer");
    return mv_launch(c, ty, ptrs, w, nullptr, xstride, 0, y, (long long)rows, 0, rows, cols, 1, slots, (hipStream_t)stream,
                     xq, xd);
}

size_t le_moe_workspace_size(int n_tok, int k, int ff) {
    if (n_tok <= 0 || k <= 0 || ff <= 0) return 0;
    /* per (token, slot) the down projection's activation image, then (staged path) a routing record */
    const size_t img = (size_t)xtok_bytes(ff) > (size_t)(ff / 256) * 608 ? (size_t)xtok_bytes(ff) : (size_t)(ff / 256) * 608;
    return kMoeBarBytes + (size_t)n_tok * (size_t)k * img + 16 + 256 * 4 + 256 * 8 + 1024 * 4 + 1024 * 4;
}

int le_moe_check(le_ctx *c, const void *ws, le_stream_t stream) {
    if (!c) return LE_ERR_ARG;
    if (!ws) return c->fail(LE_ERR_ARG, "null workspace");
    int rc = c->hip(hipStreamSynchronize((hipStream_t)stream), "le_moe_check: stream synchronize");
    if (rc) return rc;
    unsigned int st = 0;
    rc = c->hip(hipMemcpy(&st, ws, sizeof st, hipMemcpyDeviceToHost), "le_moe_check: status read");
    if (rc) return rc;
    if (st != 0x5EAD0001u) return LE_OK; /* the value the one-launch kernel stores after a give-up */
    const unsigned int zero = 0;
    rc = c->hip(hipMemcpy((void *)ws, &zero, sizeof zero, hipMemcpyHostToDevice), "le_moe_check: status clear");
    if (rc) return rc;
    return c->fail(LE_ERR_TIMEOUT, "a one-launch MoE layer on this workspace gave up at its device-wide barrier "
                                   "(its outputs are NaN): the grid was not resident at once");
}

/* Prefill form of the MoE layer (routing, grouping by expert, grouped matmuls): workspace layout. */
struct MoePreLayout {
    size_t topi, topw, off, in_idx, out_idx, g, u, d, gemm, total;
};
static MoePreLayout moe_pre_layout(int n_tok, int k, int n_exp, int hidden, int ff) {
    auto al = [](size_t x) { return (x + 255) / 256 * 256; };
    const size_t np = (size_t)n_tok * k;
    MoePreLayout L{};
    size_t o = 0;
    L.topi = o; o += al(np * 4);
    L.topw = o; o += al(np * 4);
    L.off = o; o += al(((size_t)n_exp + 1) * 4);
    L.in_idx = o; o += al(np * 4);
    L.out_idx = o; o += al(np * 4);
    L.g = o; o += al(np * ff * 4);
    L.u = o; o += al(np * ff * 4);
    L.d = o; o += al(np * hidden * 4);
    L.gemm = o;
    /* the grouped matmuls' workspace for the larger of the two K (Q4_K's, which has sum records) */
    const size_t g1 = le_mm_grouped_workspace_size(LE_TYPE_Q4_K, n_exp, (int)np, hidden);
    const size_t g2 = le_mm_grouped_workspace_size(LE_TYPE_Q4_K, n_exp, (int)np, ff);
    o += al(g1 > g2 ? g1 : g2);
    L.total = o;
    return L;
}

/* Kernel argument block of the prefill routing / grouping kernels (mirrors MoePre). */
struct MoePreArgs {
    const float *logits;
    int *topi;
    float *topw;
    int *off, *in_idx, *out_idx, *idx_out;
    float *w_out;
    int n_tok, n_exp, k, pad;
};

static int mm_grouped(le_ctx *c, int ty, const void *const *ptrs, const void *w, const void *const *ptrs2, const void *w2,
                      const int *off, const int *in_idx, const int *out_idx, int nslot, int npair, const float *x, float *y,
                      float *y2, int rows, int cols, void *ws, size_t ws_bytes, hipStream_t stream, const float *up = nullptr);

static int moe_prefill(le_ctx *c, int ty_gate, int ty_down, const void *gate, const void *up, const void *down,
                       const void *const *gptr, const void *const *uptr, const void *const *dptr, int n_exp, int k,
                       int hidden, int ff, const float *logits, const float *h, int n_tok, float *out, int *idx_out,
                       float *w_out, void *ws, hipStream_t st) {
    const MoePreLayout L = moe_pre_layout(n_tok, k, n_exp, hidden, ff);
    char *b = (char *)ws;
    const int np = n_tok * k;
    int *topi = (int *)(b + L.topi), *off = (int *)(b + L.off), *in_idx = (int *)(b + L.in_idx), *out_idx = (int *)(b + L.out_idx);
    float *topw = (float *)(b + L.topw), *G = (float *)(b + L.g), *U = (float *)(b + L.u), *D = (float *)(b + L.d);
    void *gws = b + L.gemm;
    const size_t gws_bytes = L.total - L.gemm;
    MoePreArgs a{logits, topi, topw, off, in_idx, out_idx, idx_out, w_out, n_tok, n_exp, k, 0};
    void *args[] = {&a};
    int rc;
    /* one block routes and groups up to 32 tokens (two per wave: 12 / 16 tokens 113.6 -> 110.1,
     * 122.2 -> 118.9 us a layer; at 64 tokens its serial routing costs 8 us more than two launches) */
    if (n_tok <= 32 && np <= 1024 && c->moe_route1)
        rc = c->launch("le_moe_route_group", dim3(1), 1024, 0, st, args);
    else {
        rc = c->launch("le_moe_route_tok", dim3((unsigned)((n_tok + 7) / 8)), 512, 0, st, args);
        if (!rc) rc = c->launch("le_moe_group", dim3((unsigned)n_exp), 256, 0, st, args);
    }
    /* gate and up in one grouped launch (one plan and one activation pre-pass for both) */
    if (!rc) rc = mm_grouped(c, ty_gate, gptr, gate, uptr, up, off, in_idx, out_idx, n_exp, np, h, G, U, ff, hidden, gws, gws_bytes, st);
    if (rc) return rc;
    /* down: the activation rows are the pairs themselves, in the same grouped order, each formed
     * as silu(gate) * up by the down matmul's pre-pass */
    rc = mm_grouped(c, ty_down, dptr, down, nullptr, nullptr, off, out_idx, out_idx, n_exp, np, G, D, nullptr, hidden, ff, gws,
                    gws_bytes, st, U);
    if (rc) return rc;
    const unsigned blocks = (unsigned)n_tok * (unsigned)((hidden + 1023) / 1024); /* (token, 1024 columns) */
    const float *Dc = D, *Wc = topw;
    void *cargs[] = {&Dc, &Wc, &out, &n_tok, &k, &hidden};
    return c->launch("le_moe_combine", dim3(blocks), 256, 0, st, cargs);
}

size_t le_moe_prefill_workspace_size(int n_tok, int k, int n_exp, int hidden, int ff) {
    if (n_tok <= 0 || k <= 0 || n_exp <= 0 || hidden <= 0 || ff <= 0 || hidden % 256 || ff % 256) return 0;
    return moe_pre_layout(n_tok, k, n_exp, hidden, ff).total;
}

/* The MoE layer over expert slabs (gate/up/down) or per-expert pointer tables (gptr/uptr/dptr). */
static int moe_layer_impl(le_ctx *c, int ty_gate, int ty_up, int ty_down, const void *gate, const void *up, const void *down,
                          const void *const *gptr, const void *const *uptr, const void *const *dptr, int n_exp, int k,
                          int hidden, int ff, const float *logits, const float *h, int n_tok, float *out, int *idx_out,
                          float *w_out, void *ws, size_t ws_bytes, hipStream_t stream) {
    const bool tables = gptr || uptr || dptr;
    if (tables ? !(gptr && uptr && dptr) : !(gate && up && down)) return c->fail(LE_ERR_ARG, "null weight pointer or table");
    if (!logits || !h || !out || !ws) return c->fail(LE_ERR_ARG, "null pointer");
    if (ty_gate != ty_up) return c->fail(LE_ERR_TYPE, "gate and up must share a type");
    if (!supported_mv(ty_gate) || !supported_mv(ty_down)) return c->fail(LE_ERR_TYPE, "no kernel for types %d/%d", ty_gate, ty_down);
    /* type pairs of the decode-shaped kernels; every other pair of the nine types runs the grouped
     * (prefill) form at any token count */
    static const int combos[][2] = {{12, 14}, {12, 12}, {14, 14}, {8, 8}, {16, 18}, {16, 16}, {18, 18}};
    bool have = false;
    for (auto &cb : combos) have |= cb[0] == ty_gate && cb[1] == ty_down;
    if (n_tok <= 0 || n_tok > LE_MOE_MAX_TOK || k <= 0 || k > 16 || n_exp <= 0 || n_exp > 256 || k > n_exp)
        return c->fail(LE_ERR_SHAPE, "MoE limits: n_tok <= %d, k <= 16, k <= n_exp <= 256", LE_MOE_MAX_TOK);
    if (hidden <= 0 || ff <= 0 || hidden % 256 || ff % 256) return c->fail(LE_ERR_SHAPE, "hidden and ff must be multiples of 256");
    /* prefill-sized token counts: routing, grouping by expert and grouped matrix-core matmuls (each
     * expert's weights streamed once per tile of its pairs); up to 64 tokens the decode kernels
     * take the call when the workspace is sized for them only */
    if (!have || n_tok > 64 || (c->moe_prefill && n_tok >= c->moe_prefill_min_tok &&
                       ws_bytes >= le_moe_prefill_workspace_size(n_tok, k, n_exp, hidden, ff))) {
        if (ws_bytes < le_moe_prefill_workspace_size(n_tok, k, n_exp, hidden, ff))
            return c->fail(LE_ERR_WORKSPACE, "workspace needs %zu bytes (le_moe_prefill_workspace_size)",
                           le_moe_prefill_workspace_size(n_tok, k, n_exp, hidden, ff));
        if (!al16(h) || !al16(ws)) return c->fail(LE_ERR_ALIGN, "h and ws must be 16-byte aligned");
        return moe_prefill(c, ty_gate, ty_down, gate, up, down, gptr, uptr, dptr, n_exp, k, hidden, ff, logits, h, n_tok, out,
                           idx_out, w_out, ws, stream);
    }
    if (ws_bytes < le_moe_workspace_size(n_tok, k, ff)) return c->fail(LE_ERR_WORKSPACE, "workspace needs %zu bytes", le_moe_workspace_size(n_tok, k, ff));
    if (!al16(h) || !al16(ws)) return c->fail(LE_ERR_ALIGN, "h and ws must be 16-byte aligned");
    /* 9..64 tokens in the decode form: stream-ordered calls of at most 8 tokens, each on the
     * decode kernels' fast paths (config 4, 16 tokens: 442 -> 136 us against one call on the
     * member-chunk kernels; 12 tokens 313 -> 115 us); each call reuses the workspace after the previous one */
    if (n_tok > 8 && c->moe_chunk) {
        for (int t0 = 0; t0 < n_tok; t0 += 8) {
            const int nt = n_tok - t0 < 8 ? n_tok - t0 : 8;
            const int rc = moe_layer_impl(c, ty_gate, ty_up, ty_down, gate, up, down, gptr, uptr, dptr, n_exp, k, hidden, ff,
                                          logits + (size_t)t0 * n_exp, h + (size_t)t0 * hidden, nt, out + (size_t)t0 * hidden,
                                          idx_out ? idx_out + (size_t)t0 * k : nullptr, w_out ? w_out + (size_t)t0 * k : nullptr,
                                          ws, ws_bytes, stream);
            if (rc) return rc;
        }
        return LE_OK;
    }
    const size_t lds = (size_t)8 * xtok_bytes(hidden);
    if (lds + 16384 > c->lds_limit) return c->fail(LE_ERR_SHAPE, "hidden=%d exceeds the LDS budget", hidden);
    MoeArgs a{gate, up, down, logits, h, out, (char *)ws + kMoeBarBytes, idx_out, w_out, n_tok, n_exp, k, hidden, ff,
              c->moe_spin_limit, ws, gptr, uptr, dptr};
    void *args[] = {&a};
    char name[64];
    const int nsb = hidden / 256, g8 = nsb % 8 == 0;
    const int S = g8 ? nsb / 8 : nsb;
    const int groups = n_tok * k < n_exp ? n_tok * k : n_exp;
    /* one launch with a device-wide barrier (hidden 2048): only with a grid that is resident at once */
    if (c->moe_fused && n_tok >= c->moe_fused_min_tok && ty_gate == LE_TYPE_Q4_K &&
        (ty_down == LE_TYPE_Q6_K || ty_down == LE_TYPE_Q4_K) && n_tok <= 8 &&
        hidden == 2048 && ff % 256 == 0 && ff / 256 >= 1 && ff / 256 <= 3) {
        const int pd = ff / 256, cps = ty_down == LE_TYPE_Q6_K ? 14 : 9, nid = (16 * (cps * pd + 1) + 63) / 64;
        const size_t lds1 = 8 * (size_t)8 * 608 + 8 * (size_t)10 * 1024, lds2 = 16 * (size_t)pd * 608 + 8 * (size_t)nid * 1024;
        const size_t lds = lds1 > lds2 ? lds1 : lds2;
        snprintf(name, sizeof name, "le_moe_fus_12_%d_p%d", ty_down, pd);
        hipFunction_t f = c->fn(name);
        const int per_cu = f ? c->blocks_per_cu(name, 512, lds) : 0;
        const long long resident = (long long)c->cus * per_cu, ntile = hidden / 16;
        const long long items = (long long)(ff / 32) * groups;
        if (f && resident >= ntile && ntile <= 1024) { /* 1024: the kernel's arrival flags */
            long long g = items > ntile ? (items < resident ? items : resident) : ntile;
            if (g > 1024) g = 1024;
            return c->launch(name, dim3((unsigned)g), 512, lds, (hipStream_t)stream, args);
        }
    }
    /* decode-shaped staged-MFMA path: Q4_K gate/up, Q4_K or Q6_K down; gate/up blocks of 8 waves
     * (hidden 2048) or 4 waves (hidden 1024, 3072), down blocks of 8 waves (ff 256, 512, 768) */
    const int gw = hidden == 2048 ? 8 : 4, gp = hidden / (256 * gw), dp = ff / 256;
    if (c->moe_mfma && ty_gate == LE_TYPE_Q4_K && (ty_down == LE_TYPE_Q6_K || ty_down == LE_TYPE_Q4_K) && n_tok <= 8 &&
        (hidden == 1024 || hidden == 2048 || hidden == 3072) && dp >= 1 && dp <= 3) {
        const int nig = 9 * gp + 1, cps = ty_down == LE_TYPE_Q6_K ? 14 : 9, nid = (16 * (cps * dp + 1) + 63) / 64;
        const size_t img_g = (size_t)hidden / 256 * 608, img_d = (size_t)dp * 608;
        const size_t lds_g = 8 * img_g + (size_t)gw * nig * 1024, lds_d = 16 * img_d + 8 * (size_t)nid * 1024;
        /* dynamic LDS plus the kernels' static routing/reduction state (< 40 KB) must fit */
        if (lds_g + 40960 <= c->lds_limit && lds_d + 40960 <= c->lds_limit) {
            snprintf(name, sizeof name, "le_moe_gum_12_%d_w%d_p%d", ty_down, gw, gp);
            int rc = c->launch(name, dim3((unsigned)(ff / 32), (unsigned)groups), 64 * gw, lds_g, (hipStream_t)stream, args);
            if (rc) return rc;
            snprintf(name, sizeof name, "le_moe_dnm_%d_w8_p%d", ty_down, dp);
            /* two blocks per row tile when the tiles alone leave CUs idle (each adds its half of the
             * expert groups into the output the gate/up launch zeroed) */
            const int hsplit = c->moe_dn_split == 2 || (c->moe_dn_split == 0 && hidden / 16 * 2 <= c->cus) ? 2 : 1;
            return c->launch(name, dim3((unsigned)(hsplit * hidden / 16)), 512, lds_d, (hipStream_t)stream, args);
        }
    }
    /* decode-shaped fast paths: few tokens, short rows */
    const bool fast_gu = c->moe_fast && n_tok <= 8 && S <= 2 && n_tok * (hidden / 8) <= 4096;
    const bool fast_dn = c->moe_fast && n_tok <= 8 && ff <= 1024;
    snprintf(name, sizeof name, fast_gu ? "le_moe_guf_%d_%d_g%d" : "le_moe_gu_%d_%d_g%d", ty_gate, ty_down, g8 ? 8 : 1);
    int rc = c->launch(name, dim3((unsigned)(ff / 32), (unsigned)groups), fast_gu ? 1024 : 256, lds,
                       (hipStream_t)stream, args);
    if (rc) return rc;
    snprintf(name, sizeof name, fast_dn ? "le_moe_downf_%d" : "le_moe_down_%d", ty_down);
    return c->launch(name, dim3((unsigned)(hidden / 8)), fast_dn ? 512 : 256, fast_dn ? 49152 : 0, (hipStream_t)stream, args);
}

int le_moe_layer(le_ctx *c, int ty_gate, int ty_up, int ty_down, const void *gate, const void *up, const void *down,
                 int n_exp, int k, int hidden, int ff, const float *logits, const float *h, int n_tok, float *out,
                 int *idx_out, float *w_out, void *ws, size_t ws_bytes, le_stream_t stream) {
    if (!c) return LE_ERR_ARG;
    return moe_layer_impl(c, ty_gate, ty_up, ty_down, gate, up, down, nullptr, nullptr, nullptr, n_exp, k, hidden, ff,
                          logits, h, n_tok, out, idx_out, w_out, ws, ws_bytes, (hipStream_t)stream);
}

int le_moe_layer_ptrs(le_ctx *c, int ty_gate, int ty_up, int ty_down, const void *const *gate_ptrs,
                      const void *const *up_ptrs, const void *const *down_ptrs, int n_exp, int k, int hidden, int ff,
                      const float *logits, const float *h, int n_tok, float *out, int *idx_out, float *w_out, void *ws,
                      size_t ws_bytes, le_stream_t stream) {
    if (!c) return LE_ERR_ARG;
    if (!gate_ptrs || !up_ptrs || !down_ptrs) return c->fail(LE_ERR_ARG, "null pointer table");
    return moe_layer_impl(c, ty_gate, ty_up, ty_down, nullptr, nullptr, nullptr, gate_ptrs, up_ptrs, down_ptrs, n_exp, k,
                          hidden, ff, logits, h, n_tok, out, idx_out, w_out, ws, ws_bytes, (hipStream_t)stream);
}

/* Q4_K with 3..8 (or 16) tokens: the staged f16 MFMA kernel, T = 4, 8 or 16 tokens per weight
 * pass (it builds its fp16 activations itself). Returns 1 when no instantiated shape fits. */
static int mh_launch(le_ctx *c, const void *w, const float *x, int m, float *y, int rows, int cols, hipStream_t st) {
    const long long ntile = (rows + 15) / 16;
    /* above 8 tokens: groups of 8 tokens whose blocks stream the same row tiles side by side
     * (option gm_mh_t16 = 1: one 16-token group, whose images need 128 KB of LDS at K = 4096) */
    const int nsb = cols / 256, T = m <= 4 ? 4 : m <= 8 || !c->gm_mh_t16 ? 8 : 16, G = (m + T - 1) / T;
    /* (P, NW) in order of preference, measured on 14336 x 4096 (T=4, 3..4 tokens: 12.8 us with
     * (1,8) against 13.2 with (2,4), 13.5 with (1,4); T=8: 14.0 us with (1,8)) */
    static const int k4[4][2] = {{1, 8}, {2, 4}, {1, 4}, {2, 2}}, k8[4][2] = {{1, 8}, {2, 4}, {1, 4}, {2, 2}};
    static const int k16[4][2] = {{1, 4}, {1, 8}, {2, 4}, {2, 2}};
    const int(*cand)[2] = T == 4 ? k4 : T == 8 ? k8 : k16;
    const int ncand = 4;
    for (int i = 0; i < ncand; i++) {
        const int P = c->gm_mh_shape ? c->gm_mh_shape / 10 : cand[i][0], NW = c->gm_mh_shape ? c->gm_mh_shape % 10 : cand[i][1];
        if (P > c->ms_p || nsb % (NW * P)) continue;
        /* per wave: per super-block T records of 8 x 5 16-byte image slots and 2 sum slots, 64 bytes
         * of scales; the staging of 16 rows x (9P + 1, made odd) slots; the reduction area */
        const int ni = (16 * ((9 * P + 1) | 1) + 63) / 64;
        const size_t lds = (size_t)NW * ((size_t)(nsb / NW) * (T * 672 + 64) + (size_t)ni * 1024) + (size_t)NW * 2048;
        if (lds > c->lds_limit) continue;
        char name[48];
        snprintf(name, sizeof name, "le_mh_12_p%d_w%d_t%d", P, NW, T);
        /* every block builds its activation image once: the grid is what stays resident */
        const int per_cu = c->blocks_per_cu(name, NW * 64, lds);
        long long gx = ntile, cap = (long long)c->cus * (per_cu > 0 ? per_cu : 1) / G;
        if (cap < 1) cap = 1;
        if (gx > cap) {
            const long long it = (gx + cap - 1) / cap;
            gx = (gx + it - 1) / it;
        }
        if (G > 1) gx = (gx + 7) / 8 * 8; /* the kernel's group / row-tile mapping */
        struct {
            const void *w;
            const float *x;
            float *y;
            int rows, cols, m, groups;
        } a{w, x, y, rows, cols, m, G};
        void *args[] = {&a};
        return c->launch(name, dim3((unsigned)(gx * G), 1, 1), NW * 64, lds, st, args);
    }
    return 1;
}

/* Generic matrix-core GEMM (le_gq_*): workspace = fp16 activation fragments for the tokens rounded
 * up to 128, per-super-block sum records (Q4_K: 1 KB per 32 tokens), token scales. */
static int gq_srec(int ty) { return ty == LE_TYPE_Q4_K || ty == LE_TYPE_Q5_K ? 1024 : 0; }
static size_t gq_ws_bytes(int ty, int m, int cols) {
    const size_t mp = ((size_t)m + 127) / 128 * 128;
    return mp * cols * 2 + mp / 32 * (cols / 256) * gq_srec(ty) + mp * 4;
}
/* K-slice partial results follow at the next 256-byte boundary: [ks][m][rows] floats, ks <= 8. A
 * launch splits K only while (row tiles) x (token tiles) x 2 fits the resident blocks, at most 512
 * on gfx950, and its tiles hold at least 256 rows x 128 tokens when that count is smallest, so a
 * shape with more than 256 such tiles never splits. */
static size_t gq_part_off(int ty, int m, int cols) { return (gq_ws_bytes(ty, m, cols) + 255) / 256 * 256; }
static bool gq_may_split(int m, int rows) { return (long long)((rows + 255) / 256) * ((m + 127) / 128) <= 256; }
/* Kernel arguments of le_gq_* (GqArgs in le_gq_kernels.hip). */
struct GqHostArgs {
    const void *w;
    const float *x;
    float *y;
    int rows, cols, m, mp, ksplit;
    const void *const *ptrs;
    unsigned long long w_slot_bytes;
    const int *off, *in_idx, *out_idx;
    int nslot, maxt, bm, npair;
    float *part;
    const void *const *ptrs2;
    const void *w2;
    float *y2;
    int dual, pad2;
    const float *up;
};
static int gq_slot(int ty) {
    switch (ty) {
    case LE_TYPE_Q4_K: return 80;
    case LE_TYPE_Q6_K: return 144;
    case LE_TYPE_Q8_0: return 192;
    case LE_TYPE_IQ2_XXS: return 48;
    case LE_TYPE_IQ3_XXS: return 80;
    case LE_TYPE_Q4_0: return 144;
    case LE_TYPE_Q3_K: return 80;
    case LE_TYPE_Q5_K: return 112;
    case LE_TYPE_IQ2_S: return 80;
    }
    return 0;
}
static int gq_tab(int ty) {
    return ty == LE_TYPE_IQ2_XXS ? 6144 : ty == LE_TYPE_IQ3_XXS ? 4096 : ty == LE_TYPE_IQ2_S ? 16384 + 4096 : 0;
}

static int gq_launch(le_ctx *c, int ty, const void *w, const float *x, int m, float *y, int rows, int cols, void *ws,
                     size_t ws_bytes, hipStream_t st) {
    /* block shapes: (WM, WN, TM, TN) -> BM = 32 TM WM tokens, BN = 32 TN WN rows */
    static const int cfgs[12][4] = {{1, 4, 1, 2}, {1, 4, 2, 2}, {1, 4, 4, 2}, {2, 2, 2, 2}, {1, 8, 2, 1}, {1, 8, 4, 1}, {1, 8, 1, 1}, {1, 4, 2, 1}, {1, 4, 1, 1}, {1, 4, 4, 1}, {2, 4, 2, 2}, {2, 4, 2, 1}};
    /* block shape by token count and type, from sweeps of every type at its config shape
     * (14336 x 4096; Q6_K and IQ3_XXS 4096 x 14336, Q8_0 32000 x 4096), activations loaded straight
     * into LDS: up to 32 tokens 32 x 128 tiles on 4 waves; 33..64 tokens 64 x 128 on 4 waves for
     * Q6_K and IQ3_XXS, 64 x 256 on 8 waves otherwise; 65..128 tokens 128 x 128 on 4 waves for
     * Q6_K (M=128 47.6 -> 46.3 us against 64 x 256), 64 x 256 on 8 waves for Q4_K, Q5_K and
     * IQ3_XXS (M=128 against 128 x 256: Q4_K 44.8 -> 40.9, Q5_K 46.1 -> 43.0); 129..256 tokens
     * 64 x 256 on 8 waves for Q4_K and Q5_K; everything else 128 x 256 on 8 waves (Q6_K M=256 72.8
     * -> 66.0 us and M=512 126.5 -> 107.8 against 64 x 256) */
    int ci = 5;
    const bool k45 = ty == LE_TYPE_Q4_K || ty == LE_TYPE_Q5_K;
    if (m <= 32) ci = 8;
    else if (m <= 64) ci = (ty == LE_TYPE_Q6_K || ty == LE_TYPE_IQ3_XXS) ? 7 : 4;
    else if (m <= 128 && ty == LE_TYPE_Q6_K) ci = 9;
    else if (m <= 128 && (k45 || ty == LE_TYPE_IQ3_XXS)) ci = 4;
    else if (m <= 256 && k45) ci = 4;
    if (c->gq_cfg) ci = c->gq_cfg - 1;
    const int nsb = cols / 256, srec = gq_srec(ty);
    auto lds_of = [&](int i) {
        const int BM = 32 * cfgs[i][0] * cfgs[i][2], BN = 32 * cfgs[i][1] * cfgs[i][3];
        return (size_t)2 * (BN * gq_slot(ty) + BM * 256) + (size_t)2 * (BM / 32) * srec + gq_tab(ty);
    };
    if (lds_of(ci) > c->lds_limit && (ci == 2 || ci == 5)) ci = 3;
    const size_t lds = lds_of(ci);
    if (lds > c->lds_limit) return c->fail(LE_ERR_SHAPE, "GEMM tile does not fit the LDS");
    const int WM = cfgs[ci][0], WN = cfgs[ci][1], TM = cfgs[ci][2], TN = cfgs[ci][3];
    const int BM = 32 * TM * WM, BN = 32 * TN * WN, nthr = 64 * WM * WN;
    char name[48];
    snprintf(name, sizeof name, "le_gq_%d_w%d%d_t%d%d", ty, WM, WN, TM, TN);
    if (!c->fn(name)) return c->fail(LE_ERR_SHAPE, "GEMM kernel %s is not built", name);
    const long long ntr = (rows + BN - 1) / BN, mt = (m + BM - 1) / BM;
    const long long grid = (ntr >= 8 ? (ntr + 7) / 8 * 8 : ntr) * mt; /* block order: le_gq_kernels.hip */
    if (grid > 0x7FFFFFFFLL) return c->fail(LE_ERR_SHAPE, "GEMM grid too large");
    int ks = 1;
    if (c->gq_ksplit > 0) {
        ks = c->gq_ksplit;
    } else {
        /* K slices while the grid stays within the resident blocks (one wave of blocks); the
         * 4-wave tiles stop at one block per CU (measured best: Q4_K 14336x4096 M=17, 32x128
         * tiles: 26.2 us at 224 blocks, 29.7 at 448) */
        const int per_cu = nthr == 256 ? 1 : c->blocks_per_cu(name, nthr, lds);
        const long long cap = (long long)c->cus * (per_cu > 0 ? per_cu : 1);
        while (ks < 8 && ntr * mt * 2 * ks <= cap && nsb % (2 * ks) == 0) ks *= 2;
    }
    if (nsb % ks) return c->fail(LE_ERR_SHAPE, "gq_ksplit=%d does not divide the %d super-blocks", ks, nsb);
    const int mp = (m + 127) / 128 * 128;
    /* the kernels address the weights and the activation planes with 32-bit offsets */
    if ((unsigned long long)rows * le_row_bytes(ty, cols) >= (1ull << 32) || (unsigned long long)mp * cols * 2 >= (1ull << 32))
        return c->fail(LE_ERR_SHAPE, "GEMM weights or activation planes of 4 GiB or more");
    /* K slices sum their partial results in a second pass when the workspace holds them (a
     * deterministic sum; le_gemm_workspace_size_rows), else add into y atomically */
    float *part = nullptr;
    const size_t poff = gq_part_off(ty, m, cols);
    if (ks > 1 && ws_bytes >= poff + (size_t)ks * m * rows * 4) part = (float *)((char *)ws + poff);
    GqHostArgs a{w, x, y, rows, cols, m, mp, ks, nullptr, 0, nullptr, nullptr, nullptr, 0, 0, 0, 0, part, nullptr, nullptr, nullptr, 0, 0, nullptr};
    void *args[] = {&a, &ws};
    char pname[32];
    snprintf(pname, sizeof pname, "le_gq_xprep_%d", ty);
    int rc = c->launch(pname, dim3((unsigned)mp), 256, 0, st, args);
    if (rc) return rc;
    rc = c->launch(name, dim3((unsigned)grid, (unsigned)ks), nthr, lds, st, args);
    if (rc || !part) return rc;
    const size_t n4 = ((size_t)m * rows + 3) / 4;
    const unsigned sg = (unsigned)std::min<size_t>((n4 + 255) / 256, (size_t)c->cus * 8);
    void *sargs[] = {&a};
    return c->launch("le_gq_ksum", dim3(sg), 256, 0, st, sargs);
}

/* Grouped form (le_mm_grouped): token tiles of bm pairs (32 up to 16 pairs per slot on average, 64
 * up to 64, else 128; 32 at 40 per slot measured slower: slots then span several tiles),
 * at most nslot + npair / bm of them. */
static int mmg_cfg(int nslot, int npair) {
    return (long long)npair <= 16LL * nslot ? 6 : (long long)npair <= 64LL * nslot ? 4 : 5;
}
static int mmg_bm(int nslot, int npair) { const int c = mmg_cfg(nslot, npair); return c == 6 ? 32 : c == 4 ? 64 : 128; }
static int mmg_maxt(int nslot, int npair) { const int bm = mmg_bm(nslot, npair); return nslot + (npair + bm - 1) / bm; }

size_t le_mm_grouped_workspace_size(int ty, int nslot, int npair, int cols) {
    if (!supported_mv(ty) || nslot <= 0 || npair < 0 || cols <= 0 || cols % 256) return 0;
    const size_t maxt = (size_t)mmg_maxt(nslot, npair), mp = maxt * mmg_bm(nslot, npair);
    return mp * cols * 2 + mp / 32 * (cols / 256) * gq_srec(ty) + mp * 4;
}

/* Grouped matmul; with a second weight set (ptrs2 or w2, same type and shape) the same pairs are
 * also multiplied by it into y2, in the same launches (one plan, one pre-pass, one grid). */
static int mm_grouped(le_ctx *c, int ty, const void *const *ptrs, const void *w, const void *const *ptrs2, const void *w2,
                      const int *off, const int *in_idx, const int *out_idx, int nslot, int npair, const float *x, float *y,
                      float *y2, int rows, int cols, void *ws, size_t ws_bytes, hipStream_t stream, const float *up) {
    const bool dual = ptrs2 || w2;
    if (dual && !y2) return c->fail(LE_ERR_ARG, "null second output");
    if (!supported_mv(ty)) return c->fail(LE_ERR_TYPE, "no kernel for type %d", ty);
    if ((!ptrs && !w) || !off || !in_idx || !out_idx || !x || !y || !ws) return c->fail(LE_ERR_ARG, "null pointer");
    if (nslot <= 0 || npair < 0 || rows <= 0 || cols <= 0) return c->fail(LE_ERR_SHAPE, "empty shape");
    if (cols % 256) return c->fail(LE_ERR_SHAPE, "cols=%d is not a multiple of 256", cols);
    if (!al16(x) || !al16(ws)) return c->fail(LE_ERR_ALIGN, "x and ws must be 16-byte aligned");
    const size_t need = le_mm_grouped_workspace_size(ty, nslot, npair, cols);
    if (ws_bytes < need) return c->fail(LE_ERR_WORKSPACE, "workspace needs %zu bytes", need);
    if (npair == 0) return LE_OK;
    static const int cfgs[8][4] = {{1, 4, 1, 2}, {1, 4, 2, 2}, {1, 4, 4, 2}, {2, 2, 2, 2}, {1, 8, 2, 1}, {1, 8, 4, 1}, {1, 8, 1, 1}, {1, 4, 1, 1}};
    int ci = mmg_cfg(nslot, npair);
    const int srec = gq_srec(ty);
    auto lds_of = [&](int i) {
        const int BM = 32 * cfgs[i][0] * cfgs[i][2], BN = 32 * cfgs[i][1] * cfgs[i][3];
        return (size_t)2 * (BN * gq_slot(ty) + BM * 256) + (size_t)2 * (BM / 32) * srec + gq_tab(ty);
    };
    if (lds_of(ci) > c->lds_limit) ci = 3; /* 128 x 128 on 4 waves */
    /* 32-pair tiles whose 8-wave block would hold more than half the LDS (Q6_K, Q8_0: one block
     * per CU): 32 x 128 on 4 waves, several blocks per CU */
    if (ci == 6 && c->mmg_w4 && 2 * lds_of(6) > c->lds_limit) ci = 7;
    const int WM = cfgs[ci][0], WN = cfgs[ci][1], TM = cfgs[ci][2], TN = cfgs[ci][3];
    const int BM = 32 * TM * WM, BN = 32 * TN * WN, nthr = 64 * WM * WN;
    if (BM != mmg_bm(nslot, npair) && !(ci == 3 && mmg_bm(nslot, npair) == 128))
        return c->fail(LE_ERR_SHAPE, "grouped GEMM tile does not fit the LDS");
    const int maxt = mmg_maxt(nslot, npair), mp = maxt * BM;
    const long long ntr = (rows + BN - 1) / BN * (dual ? 2 : 1), grid = (ntr >= 8 ? (ntr + 7) / 8 * 8 : ntr) * (long long)maxt;
    if (grid > 0x7FFFFFFFLL || (unsigned long long)mp * cols * 2 >= (1ull << 32) ||
        (unsigned long long)rows * le_row_bytes(ty, cols) >= (1ull << 32))
        return c->fail(LE_ERR_SHAPE, "grouped GEMM too large (32-bit weight or activation offsets)");
    GqHostArgs a{w, x, y, rows, cols, mp, mp, 1, ptrs, (unsigned long long)rows * le_row_bytes(ty, cols), off, in_idx,
                 out_idx, nslot, maxt, BM, npair, nullptr, ptrs2, w2, y2, dual ? 1 : 0, 0, up};
    /* the tiles (slots split into BM pairs, slot by slot) are derived from off inside the two
     * launches, each block finding its own */
    void *args[] = {&a, &ws};
    char name[48];
    /* from 256 pairs and up to K = 4096, one wave per pair (four pairs per block: 512 tokens
     * 262 -> 248 us, 2048 tokens 668 -> 626 us a layer); else one block per pair, whose wider
     * spread is ~1 us faster at 128 pairs */
    int rc;
    if (cols <= 4096 && npair >= 256 && c->mmg_xw) {
        snprintf(name, sizeof name, "le_gq_xprepw_%d", ty);
        rc = c->launch(name, dim3((unsigned)((npair + 3) / 4)), 256, 0, (hipStream_t)stream, args);
    } else {
        snprintf(name, sizeof name, "le_gq_xprepg_%d", ty);
        rc = c->launch(name, dim3((unsigned)npair), 256, 0, (hipStream_t)stream, args);
    }
    if (rc) return rc;
    snprintf(name, sizeof name, "le_gqg_%d_w%d%d_t%d%d", ty, WM, WN, TM, TN);
    return c->launch(name, dim3((unsigned)grid), nthr, lds_of(ci), (hipStream_t)stream, args);
}

int le_mm_grouped(le_ctx *c, int ty, const void *const *ptrs, const void *w, const int *off, const int *in_idx,
                  const int *out_idx, int nslot, int npair, const float *x, float *y, int rows, int cols, void *ws,
                  size_t ws_bytes, le_stream_t stream) {
    if (!c) return LE_ERR_ARG;
    return mm_grouped(c, ty, ptrs, w, nullptr, nullptr, off, in_idx, out_idx, nslot, npair, x, y, nullptr, rows, cols, ws,
                      ws_bytes, (hipStream_t)stream);
}

size_t le_gemm_workspace_size(int ty, int m, int cols) {
    if (!supported_mv(ty) || m <= 0 || cols <= 0 || cols % 256) return 0;
    const size_t g = gq_ws_bytes(ty, m, cols);
    if (ty != LE_TYPE_Q4_K) return g;
    /* the Q4_K GEMM of the split-activation option: two fp16 planes and 32-byte sum records */
    const size_t o = (size_t)m * cols * 4 + (size_t)m * (cols / 256) * 32;
    return g > o ? g : o;
}

size_t le_gemm_workspace_size_rows(int ty, int m, int rows, int cols) {
    const size_t base = le_gemm_workspace_size(ty, m, cols);
    if (!base || rows <= 0 || !gq_may_split(m, rows)) return base;
    const size_t full = gq_part_off(ty, m, cols) + (size_t)8 * m * rows * 4;
    return full > base ? full : base;
}

int le_gemm(le_ctx *c, int ty, const void *w, const float *x, int m, float *y, int rows, int cols, void *ws,
            size_t ws_bytes, le_stream_t stream) {
    if (!c) return LE_ERR_ARG;
    if (!supported_mv(ty)) return c->fail(LE_ERR_TYPE, "no kernel for type %d", ty);
    /* Q4_K, 3..16 tokens: the staged f16 kernel (2 tokens: the int8 multi-token matvec is faster);
     * shapes whose activations do not fit its LDS, and gm_split=1 (two fp16 halves, which only
     * the le_gm GEMM carries), go to a GEMM */
    const bool few = ty == LE_TYPE_Q4_K && c->gm_mh && !c->gm_split && m >= 3 && m <= c->gm_mh_max;
    const bool gemm = ty == LE_TYPE_Q4_K ? (m >= c->gm_min_m || few) : m >= c->gq_min_m;
    if (gemm && m > 0 && rows > 0 && cols > 0 && cols % 256 == 0 && w && x && y) {
        if (!ws) return c->fail(LE_ERR_ARG, "null workspace");
        if (ws_bytes < le_gemm_workspace_size(ty, m, cols))
            return c->fail(LE_ERR_WORKSPACE, "workspace needs %zu bytes", le_gemm_workspace_size(ty, m, cols));
        if (!al16(x) || !al16(ws)) return c->fail(LE_ERR_ALIGN, "x and ws must be 16-byte aligned");
        if (few) {
            const int rc = mh_launch(c, w, x, m, y, rows, cols, (hipStream_t)stream);
            if (rc != 1) return rc;
        }
        if (ty != LE_TYPE_Q4_K || (c->gq && !c->gm_split))
            return gq_launch(c, ty, w, x, m, y, rows, cols, ws, ws_bytes, (hipStream_t)stream);
        /* tiles: 32*TM tokens x 128*TN rows: 32 x 256 up to 64 tokens, 64 x 128 above (the
         * producer/consumer kernel of 64 x 256 tiles does not fit its registers) */
        int TM = m > 64 ? 2 : 1, TN = m > 64 && c->gm_pc ? 1 : 2;
        if (c->gm_tile) {
            TM = c->gm_tile / 10;
            TN = c->gm_tile % 10;
        }
        const bool pc = c->gm_pc && !(TM == 2 && TN == 2);
        const int split = pc ? c->gm_split : 1; /* only the producer/consumer kernel has a one-half form */
        const int BM = 32 * TM, BN = 128 * TN, nsb = cols / 256;
        const long long nt = (rows + BN - 1) / BN, mt = (m + BM - 1) / BM;
        const long long grid = (nt + 7) / 8 * 8 * mt;
        /* two pipeline buffers of BN*(72+32+16+8) + BM*136*2 bytes per activation half, plus
         * [2][BM] 32-byte sum records */
        const size_t lds = 2 * ((size_t)BN * 128 + (size_t)BM * 272 * (split ? 2 : 1)) + (size_t)BM * 64;
        char name[48];
        snprintf(name, sizeof name, "le_gm_12_m%d_n%d%s", TM, TN, pc ? (split ? "_pc" : "_pc1") : "");
        const int nthr = pc ? 512 : 256;
        /* K slices: the most that keep the grid within one block per CU (measured best on
         * 14336 x 4096 for M = 4..512; more blocks, even resident ones, cost more in clears, atomics
         * and shared CUs than the slices gain) */
        int ks = 1;
        if (c->gm_ksplit > 0) {
            ks = c->gm_ksplit;
        } else {
            while (ks < 8 && nt * mt * 2 * ks <= c->cus && nsb % (2 * ks) == 0) ks *= 2;
        }
        if (nsb % ks) return c->fail(LE_ERR_SHAPE, "gm_ksplit=%d does not divide the %d super-blocks", ks, nsb);
        struct {
            const void *w;
            const float *x;
            float *y;
            int rows, cols, m, ksplit, split;
        } a{w, x, y, rows, cols, m, ks, split};
        /* pass 1: activation halves and sub-block sums into the workspace, one wave per
         * (token, super-block); clears y when K is split */
        void *pargs[] = {&a, &ws};
        const long long waves = (long long)m * (cols / 256);
        if (waves > 0x7FFFFFFFLL) return c->fail(LE_ERR_SHAPE, "GEMM activation size too large");
        long long pblocks = (waves + 3) / 4;
        if (ks > 1) {
            const long long yb = ((long long)m * rows + 1023) / 1024;
            if (yb > pblocks) pblocks = yb < 8192 ? yb : 8192;
        }
        int rc = c->launch("le_gm_xprep", dim3((unsigned)pblocks), 256, 0, (hipStream_t)stream, pargs);
        if (rc) return rc;
        /* pass 2: the row tiles are padded to a multiple of 8 so that the token tiles of one row
         * tile share blockIdx % 8 (one XCD); blockIdx.y is the K slice */
        if (grid > 0x7FFFFFFFLL) return c->fail(LE_ERR_SHAPE, "GEMM grid too large");
        void *args[] = {&a, &ws};
        return c->launch(name, dim3((unsigned)grid, (unsigned)ks), nthr, lds, (hipStream_t)stream, args);
    }
    return mv_launch(c, ty, nullptr, w, x, 0, cols, y, 0, rows, rows, cols, m, 1, (hipStream_t)stream);
}

int le_stream_read(le_ctx *c, const void *buf, size_t bytes, void *sink, le_stream_t stream) {
    if (!c) return LE_ERR_ARG;
    if (!buf || !sink || bytes < 16 || bytes % 16) return c->fail(LE_ERR_ARG, "buf, sink and a size that is a multiple of 16 bytes");
    if (!al16(buf)) return c->fail(LE_ERR_ALIGN, "buf must be 16-byte aligned");
    const unsigned blocks = (unsigned)c->cus * c->rd_blocks_per_cu;
    unsigned long long n16 = bytes / 16;
    void *args[] = {(void *)&buf, &n16, &sink};
    char name[32];
    snprintf(name, sizeof name, "le_read_nt%d_u%d", c->rd_nt, c->rd_u);
    return c->launch(name, dim3(blocks), c->rd_block, 0, (hipStream_t)stream, args);
}

int le_stream_read_sink_bytes(le_ctx *c) { return c ? c->cus * 16 * 4 : 0; }

}  // extern "C"

/* Context accessors for le_noalloc.hip. */
int le_ctx_device(const le_ctx *c) { return c ? c->device : -1; }
int le_ctx_fail(le_ctx *c, int code, const char *msg) { return c ? c->fail(code, "%s", msg) : code; }
