/*
 * le_qmm.h -- C ABI of the MI355X-native GGUF quantized-matmul hot path.
 *
 * This is the drop-in boundary for the reference's quantized-matmul launch surface: the named
 * kernel table `f: HashMap<&str, CudaFunction>` of src/gpu.rs:30,70-75 reached through
 * Gpu::qx/mv_ptrs/mv (src/gpu.rs:223-238), prefill::mm/dense (src/gpu/prefill.rs:44-60) and
 * DenseGpu::mvq/bmm (src/gpu/dense.rs:150-199). A Rust host binds these functions through an
 * `extern "C"` FFI block.
 *
 * Conventions
 *   - Every entry returns an int status: LE_OK (0) or a negative LE_ERR_* code. The reference
 *     panics on the same conditions (src/gpu.rs:221,233); a binding maps codes to its own errors.
 *   - All pointers named w, x, y, out, logits, h, ws, ptrs, off, in_idx, out_idx are DEVICE
 *     pointers owned by the caller. Weights are raw GGUF row bytes (src/gpu.rs:79-83), row-major:
 *     `rows` rows of le_row_bytes(ty, cols) bytes; an expert slab e of a 3D tensor starts at
 *     e * rows * row_bytes (src/cpu_ref.rs:110-115).
 *   - `stream` is a hipStream_t (NULL = the null stream). Calls are asynchronous on it.
 *   - A context is thread-compatible, not thread-safe: use one per host thread or lock around
 *     it, as the reference drives one engine from one thread (src/local.rs:20,217).
 *   - No entry allocates device memory; entries that need scratch take a caller-sized workspace.
 *   - Activations are fp32; results are fp32 with fp32 accumulation. Inside the kernels each
 *     32-value activation block is held as a 15-bit integer split into two int8 planes with an
 *     fp32 scale (error <= 3.1e-5 of the block maximum per value); weight codes are exact.
 *
 * Supported types (GGML ids, src/quant.rs:13-20): Q8_0=8, Q4_K=12, Q6_K=14, IQ2_XXS=16, IQ3_XXS=18,
 * and Q4_0=2, Q3_K=11, Q5_K=13, IQ2_S=22 (src/quant.rs:64-67,83-95,113-126,155-167; the reference's
 * matvec_2/_11/_13/_22, mmq128r_2/_11/_13 and mm_22/mmq_22, src/cuda/kernels.cu:391,719,1225-1234),
 * on every entry point. The MoE layer's decode-shaped kernels take the type pairs listed there;
 * every other pair runs its grouped form.
 */
#ifndef LE_QMM_H
#define LE_QMM_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

typedef struct le_ctx le_ctx;
typedef void *le_stream_t; /* hipStream_t */

enum le_type {
    LE_Q4_0 = 2, LE_Q8_0 = 8, LE_Q3_K = 11, LE_Q4_K = 12, LE_Q5_K = 13, LE_Q6_K = 14, LE_IQ2_XXS = 16, LE_IQ3_XXS = 18,
    LE_IQ2_S = 22
};

enum le_status {
    LE_OK = 0,
    LE_ERR_ARG = -1,    /* null pointer / bad count */
    LE_ERR_TYPE = -2,   /* unsupported quant type (reference: panic!("no kernel for type"), src/gpu.rs:233) */
    LE_ERR_SHAPE = -3,  /* cols not a multiple of 256, or rows/cols out of range */
    LE_ERR_ALIGN = -4,  /* activation/output pointer or stride not 16-byte aligned */
    LE_ERR_HIP = -5,    /* a HIP runtime call failed (reference: .expect("launch"), src/gpu.rs:221) */
    LE_ERR_MODULE = -6, /* code object missing / unloadable, or device is not gfx950 */
    LE_ERR_WORKSPACE = -7, /* workspace too small */
    LE_ERR_TIMEOUT = -8    /* a bounded device-side wait gave up (le_moe_check) */
};

/* ---- geometry (src/quant.rs:24-35) ---- */

/* Values and bytes per block of `ty`; returns LE_OK or LE_ERR_TYPE. (src/quant.rs:24-31) */
int le_block_info(int ty, int *values, int *bytes);
/* Bytes of one row of n values, 0 for an unsupported type. (src/quant.rs:35) */
size_t le_row_bytes(int ty, size_t n);
/* Human-readable text for a status code. */
const char *le_status_str(int status);

/* ---- context / module load (replaces the NVRTC compile + module load, src/gpu.rs:65-76) ---- */

/* Loads the gfx950 code objects from `lib_dir` (NULL = the directory holding this library) on the
 * current HIP device. */
int le_init(const char *lib_dir, le_ctx **out);
void le_destroy(le_ctx *ctx);
/* Text of the last error raised on ctx (HIP error string or argument check). */
const char *le_last_error(const le_ctx *ctx);
/* Launch-policy knobs (the counterpart of the reference's LE_MMQ* / LE_TMAX env switches,
 * src/gpu/dense.rs:182-192). Defaults are the measured best on MI355X; results do not depend on
 * them beyond fp32 summation order, except "gm_split". Unknown names or values give LE_ERR_ARG.
 *   decode matvec, vector path:  "mv_block" threads per block (512, 1024), "mv_blocks_per_cu" grid
 *     cap, "mv_shape" rows x super-blocks in flight per lane (0 auto, 1: 1x2, 2: 2x1, 3: 2x2, 4: 4x1)
 *   decode matvec, matrix cores: "mq" (0/1), "ms" staged variant (0/1), "mq_waves" (2, 4, 8),
 *     "mq_waves_auto" (0/1: twice the waves when the row tiles do not fill the chip),
 *     "mq_steps", "mq_blocks_per_cu", super-blocks per row and step "ms_p" (Q4_K), "ms_p6" (Q6_K),
 *     "ms_piq" (IQ2_XXS, IQ3_XXS), "ms_p80" (Q8_0), "ms_p40" (Q4_0), "ms_p5k" (Q5_K), "ms_p3k"
 *     (Q3_K), "ms_p2s" (IQ2_S), and "mq6" / "mqiq" / "ms80" / "ms40" / "ms5k" / "ms3k" / "ms2s"
 *     (0/1) for the Q6_K / IQ / Q8_0 / Q4_0 / Q5_K / Q3_K / IQ2_S staged kernels (0: vector kernels);
 *     "ms_wide" (0/1) down shapes (row tiles <= CUs, K >= 48 super-blocks) on 12-16 waves, every
 *     type but Q6_K and Q8_0; "mq_q8" (0/1) int8 mode on
 *     the staged kernels;
 *     "ms_t" (0/1): Q4_K with 2..8 tokens per pass on the staged kernel (one weight stream, 8 tokens
 *     per MFMA pass), used by le_gemm below "gm_min_m" tokens
 *   GEMM: "gq" (0/1) Q4_K on the generic matrix-core GEMM (default) or the older le_gm kernels,
 *     "gq_min_m" smallest M of the other types on the matrix-core GEMM (below: vector kernels that
 *     read the weights once per 8 tokens), "gq_cfg" its block shape (0 auto; 1..10: 32x256, 64x256,
 *     128x256, 128x128 tokens x rows on 4 waves, 64x256, 128x256, 32x256 on 8 waves, 64x128, 32x128,
 *     128x128 on 4 waves; Q4_K only, 2 x 4 waves: 11 128x256, 12 128x128), "gq_ksplit" its K
 *     slices (0 auto, 1, 2, 4, 8); "mmg_xw" (0/1) the grouped form's activation pre-pass one wave
 *     per pair from 256 pairs when K <= 4096 (default) or one block per pair (same results);
 *     "mmg_w4" (0/1) grouped 32-pair tiles of Q6_K / Q8_0 / Q4_0 on 4-wave 32x128 blocks (default)
 *     or 8-wave 32x256 ones (same results);
 *     "moe_route1" (0/1) the grouped MoE's routing and grouping in one block up to 32 tokens
 *     (default) or two launches (same results);
 *     "gm_mh" (0/1) Q4_K with 3..16 tokens on the staged f16 MFMA kernel (tokens as MFMA rows),
 *     "gm_mh_max" its largest M (16, the default, where K <= 4096 fits its LDS; or 8),
 *     "gm_mh_shape" its (super-blocks per step, waves) as 10 P + NW (0 auto, 14, 18, 24, 22),
 *     "gm_min_m" smallest Q4_K M on a GEMM, "gm_tile" (0 auto, 11, 12, 21, 22), "gm_ksplit" K
 *     slices (0 auto, 1, 2, 4, 8), "gm_pc" producer/consumer waves (0/1) of the le_gm kernels,
 *     "gm_split" 1: Q4_K activations as two fp16 halves (about 2^-22 per value) on the le_gm
 *     kernels, which then also take 3..16 tokens (the le_gm kernels, selected by "gq" 0 or
 *     "gm_split" 1, take activations unscaled: |x| and 32-value sums below 65504)
 *   MoE: "moe_mfma" staged kernels (0/1), "moe_fused" single launch (0/1), "moe_fused_min_tok",
 *     "moe_fast" decode-shaped vector kernels (0/1) */
int le_set_option(le_ctx *ctx, const char *name, int value);

/* ---- bit-exact dequantization (the device twin of quant::dequant_row, src/quant.rs:59-170) ---- */

/* out[r * cols + c] = dequant(W[r])[c] for r < rows. */
int le_dequant_rows(le_ctx *ctx, int ty, const void *w, float *out, int rows, int cols, le_stream_t stream);

/* ---- batch-1 decode matvec (replaces matvec_<ty> + Gpu::mv_ptrs, src/cuda/kernels.cu:371-392,
 *      src/gpu.rs:228-237) ----
 * For slot s < slots: y[s * rows + r] = W_s[r,:] . x_s with W_s = ptrs[s] (device array of
 * `slots` weight pointers) or, when ptrs is NULL, w + s * rows * row_bytes; x_s = x + s * xstride
 * (xstride = 0 shares one activation, as the fused gate+up launch of src/gpu.rs:589 does). */
int le_matvec(le_ctx *ctx, int ty, const void *const *ptrs, const void *w, const float *x, long long xstride,
              float *y, int rows, int cols, int slots, le_stream_t stream);

/* ---- SwiGLU fused into the down projection (replaces swiglu_gu + quant_x + matvec_<ty>,
 *      src/cuda/kernels.cu:430-435, DenseGpu's FFN tail src/gpu/dense.rs:309-312, and swiglu + the
 *      down mv_ptrs of the MoE block src/gpu.rs:594-597) ----
 * le_matvec with the activation of slot s formed inside the kernel from a gate | up vector:
 * a[c] = silu(gu[c]) * gu[cols + c] for c < cols, gu = gu_base + s * xstride (xstride 0 shares one
 * vector, else >= 2 * cols), silu(g) = g / (1 + exp(-g)). gu is exactly the output of the
 * concatenated gate+up matvec (rows 0..cols-1 gate, cols..2 cols-1 up), so the FFN's middle
 * vector is never written. Same types, limits and numerics as le_matvec. */
int le_matvec_swiglu(le_ctx *ctx, int ty, const void *const *ptrs, const void *w, const float *gu, long long xstride,
                     float *y, int rows, int cols, int slots, le_stream_t stream);

/* ---- int8 activation mode: the reference's own GPU numerics (optional; not the fp32-parity path) ----
 * le_quant_x replaces quant_x (src/cuda/kernels.cu:15-25) as launched by Gpu::qx (src/gpu.rs:223-226):
 * for u < n_units, xd[u] = max|x[32u..32u+31]| / 127, xq[32u+l] = x[32u+l] * (1 / xd[u]) rounded to
 * nearest even (0 when xd[u] = 0), xs[u] = sum of the unit's xq.
 * le_matvec_q8 replaces matvec_<ty> on those activations (src/cuda/kernels.cu:371-392, udot<ty>
 * :36-110; Gpu::mv_ptrs src/gpu.rs:228-237): for slot s < slots, y[s * rows + r] = sum over units u
 * of W_s[r, unit u] . (xd[u'] * xq[32u' ..]) with u' = s * xstride / 32 + u, i.e. the reference's
 * exact integer dot per 32-value unit times its scales, summed in fp32. xq/xd/xs of slot s start
 * at s * xstride values (xstride % 32 == 0; 0 shares one vector); xq 8-byte aligned. xs is
 * accepted for the reference's signature and may be NULL (the kernels form the sums from xq).
 * Per value the activation error is up to xd / 2 (about 4e-3 relative at K = 4096, as on the
 * reference's GPU path), so results differ from cpu_ref by more than le_matvec's. */
int le_quant_x(le_ctx *ctx, const float *x, int8_t *xq, float *xd, int32_t *xs, int n_units, le_stream_t stream);
/* rms_quant (src/cuda/dense.cu:33-56, launched by DenseGpu::rms_q, src/gpu/dense.rs:143): RMSNorm
 * and int8 quantization of the result in one launch. o[i] = x[i] * r * w[i] with
 * r = 1 / sqrt(sum(x^2) / n + eps) (cpu_ref::rms, src/cpu_ref.rs:32-36; the sum is reduced in a
 * different order, so r agrees to a few ulp), and xq/xd/xs = le_quant_x(o) exactly. n % 32 == 0. */
int le_rms_quant(le_ctx *ctx, const float *x, const float *w, float *o, int8_t *xq, float *xd, int32_t *xs, int n, float eps,
                 le_stream_t stream);
int le_matvec_q8(le_ctx *ctx, int ty, const void *const *ptrs, const void *w, const int8_t *xq, const float *xd,
                 const int32_t *xs, long long xstride, float *y, int rows, int cols, int slots, le_stream_t stream);

/* ---- small-M GEMM for speculative verify / prefill (replaces mmq*_<ty> / mmq128r_<ty> + DenseGpu::bmm,
 *      src/cuda/kernels.cu:965-1235, src/gpu/dense.rs:181-199; CPU twin cpu_ref::matmat,
 *      src/cpu_ref.rs:266-276) ----
 * Y[t * rows + r] = W[r,:] . X[t * cols ...] for t < m. ws: device workspace of
 * le_gemm_workspace_size(ty, m, cols) bytes, the counterpart of the reference's pre-quantized
 * activation buffers (xqb/xdb/xsb, src/gpu.rs:210). Every type runs on the matrix cores from 17
 * tokens (Q4_K: 3..16 tokens on a staged f16 MFMA kernel, 2 on the staged int8 matvec; other types:
 * from "gq_min_m" = 9 tokens, vector kernels below). On the matrix cores each token is scaled by
 * its own power of two and rounded to fp16 (relative error 2^-11 per value at any magnitude up to
 * 2^127); Q8_0 and Q4_0 weights enter as fp16(q * d_b * 2^S), one rounding, with a power of two per
 * row that keeps every code inside the fp16 range for any finite scales; the other types as exact
 * integer codes (Q6_K: rounded to fp16 where (q - 32) * sc has more than 11 significant bits). The
 * 3..16-token Q4_K kernel scales each token's 256-value super-block by its own power of two
 * instead (the same 2^-11 at any magnitude). */
size_t le_gemm_workspace_size(int ty, int m, int cols);
/* Workspace with room for the K slices' partial results as well (no counterpart in the reference,
 * whose GEMM never splits K): shapes with few row and token tiles are split along K to fill the
 * GPU, and with this much workspace the slices are summed in a second pass in a fixed order
 * (bit-reproducible), instead of adding into y atomically. At least le_gemm_workspace_size. */
size_t le_gemm_workspace_size_rows(int ty, int m, int rows, int cols);
int le_gemm(le_ctx *ctx, int ty, const void *w, const float *x, int m, float *y, int rows, int cols, void *ws,
            size_t ws_bytes, le_stream_t stream);

/* ---- streaming-read probe (no counterpart in the reference; a measurement helper) ----
 * Reads `bytes` (a multiple of 16) of device memory at buf the way the matvec kernels read weights
 * (16-byte loads, consecutive lanes on consecutive chunks) and writes a checksum word per block to
 * sink (le_stream_read_sink_bytes(ctx) bytes). Its time is the practical HBM read ceiling for that
 * size; options "rd_nt", "rd_u", "rd_blocks_per_cu", "rd_block" choose the load form. */
int le_stream_read(le_ctx *ctx, const void *buf, size_t bytes, void *sink, le_stream_t stream);
int le_stream_read_sink_bytes(le_ctx *ctx);

/* ---- grouped matmul (replaces mm_<ty> / mm_impl, src/cuda/kernels.cu:679-719, launched by
 *      prefill::mm, src/gpu/prefill.rs:44-56, over the host pair grouping of prefill.rs:153-214) ----
 * For each slot s < nslot and each pair i in off[s] .. off[s+1] - 1:
 *     y[out_idx[i] * rows + r] = W_s[r,:] . x[in_idx[i] * cols ...]   for r < rows,
 * with W_s = ptrs[s] (device array of nslot weight pointers, like build_ptrs' tables) or, when
 * ptrs is NULL, w + s * rows * row_bytes (expert slab s of a 3D tensor). off (nslot + 1 ints),
 * in_idx and out_idx (npair ints) are device arrays; npair = off[nslot] - off[0] is the caller's
 * bound on the pairs (the reference's host-side grouping knows it). Runs on the matrix cores for
 * every type, each slot's weights streamed once per tile of 32, 64 or 128 of its pairs, with the
 * same activation numerics as le_gemm. Output rows of different pairs must differ. ws: device
 * workspace of le_mm_grouped_workspace_size(ty, nslot, npair, cols) bytes. */
size_t le_mm_grouped_workspace_size(int ty, int nslot, int npair, int cols);
int le_mm_grouped(le_ctx *ctx, int ty, const void *const *ptrs, const void *w, const int *off, const int *in_idx,
                  const int *out_idx, int nslot, int npair, const float *x, float *y, int rows, int cols, void *ws,
                  size_t ws_bytes, le_stream_t stream);

/* ---- le_gemm without a workspace argument (no counterpart in the reference) ----
 * For callers that cannot allocate device memory: code under HIP graph capture, tight serving
 * loops, harnesses that forbid hipMalloc. Same result as le_gemm (same kernels), with the
 * workspace taken from a device array the library holds per GPU for the life of the process
 * (LE_GEMM_SCRATCH_BYTES). Allocates nothing. Returns LE_ERR_WORKSPACE when
 * le_gemm_workspace_size(ty, m, cols) exceeds LE_GEMM_SCRATCH_BYTES (about m * cols <= 8M
 * values). Every call on one GPU shares that array: calls that overlap on one GPU (two streams or
 * two host threads) race and must be serialized by the caller. */
#define LE_GEMM_SCRATCH_BYTES (32u << 20)
int le_gemm_noalloc(le_ctx *ctx, int ty, const void *w, const float *x, int m, float *y, int rows, int cols,
                    le_stream_t stream);

/* ---- MoE expert layer, routed part (replaces the decode chain router_topk -> host read-back ->
 *      build_ptrs -> matvec gate/up -> swiglu -> quant_x -> matvec down -> moe_combine,
 *      src/gpu.rs:560-597, and the prefill expert grouping of src/gpu/prefill.rs:153-215; CPU twin
 *      cpu_ref::moe, src/cpu_ref.rs:242-259) ----
 * For each token t < n_tok: softmax over logits[t*n_exp ...], top-k (ties keep the lower expert),
 * weights renormalised over the k, out[t*hidden ...] = sum_s w_s * down_e(silu(gate_e h_t) * up_e h_t).
 * gate/up: n_exp slabs of ff x hidden (types ty_gate, ty_up), down: n_exp slabs of hidden x ff
 * (ty_down), slab e at e * rows * row_bytes. Routing and grouping by expert run on the device
 * (no host synchronisation); each routed expert's weights are read once per call (for 9..10
 * tokens once per 8-token chunk; in the grouped form once per tile of its pairs). idx_out/w_out
 * (n_tok*k, optional) receive the selection. ws: device workspace of le_moe_workspace_size bytes
 * (type pairs other than (Q4_K, Q6_K), (Q4_K, Q4_K), (Q6_K, Q6_K), (Q8_0, Q8_0), (IQ2_XXS, IQ3_XXS),
 * (IQ2_XXS, IQ2_XXS), (IQ3_XXS, IQ3_XXS) run the grouped form below at every token count and need
 * le_moe_prefill_workspace_size bytes).
 * Limits: n_tok <= 65536, k <= 16, n_exp <= 256, hidden and ff multiples of 256.
 * Prefill-sized calls (more than 64 tokens; from 11 tokens when ws holds
 * le_moe_prefill_workspace_size bytes) route every token, group the (token, expert) pairs by
 * expert on the device (token order within an expert) and run the three projections as grouped
 * matrix-core matmuls (le_mm_grouped), so each expert's weights are streamed once per tile of up
 * to 128 of its pairs; ws must then hold le_moe_prefill_workspace_size bytes. Decode-sized calls
 * need le_moe_workspace_size bytes; 9..10 tokens (or up to 64 without the grouped form's workspace)
 * run as consecutive calls of at most 8 tokens, each of which streams its own routed experts.
 * For 5..8 tokens at hidden 2048 the layer runs as one launch with a device-wide barrier between
 * gate/up and down. That launch sizes its grid to the blocks that fit on the device at once and
 * assumes nothing else occupies it: a concurrent kernel on another stream can make its bounded
 * waits (about a second, option "moe_spin_limit") give up, and the launch then writes NaN to out
 * and sets a status word in ws that le_moe_check reports. The barrier state lives in ws, so calls
 * with different workspaces are independent; calls that share a workspace must not overlap.
 * Zero-fill ws once when it is allocated (it is then fully rewritten by every call). */
size_t le_moe_workspace_size(int n_tok, int k, int ff);
size_t le_moe_prefill_workspace_size(int n_tok, int k, int n_exp, int hidden, int ff);
int le_moe_layer(le_ctx *ctx, int ty_gate, int ty_up, int ty_down, const void *gate, const void *up,
                 const void *down, int n_exp, int k, int hidden, int ff, const float *logits, const float *h,
                 int n_tok, float *out, int *idx_out, float *w_out, void *ws, size_t ws_bytes,
                 le_stream_t stream);
/* le_moe_layer with per-expert weight pointer tables (device arrays of n_exp pointers, one slab
 * of ff x hidden / hidden x ff rows each) instead of contiguous 3D tensors: the layout of an
 * expert-cache arena, whose per-expert table the reference turns into per-slot pointers with
 * build_ptrs (src/cuda/kernels.cu:458-468, src/gpu.rs:587-596). Same semantics and workspace. */
int le_moe_layer_ptrs(le_ctx *ctx, int ty_gate, int ty_up, int ty_down, const void *const *gate_ptrs,
                      const void *const *up_ptrs, const void *const *down_ptrs, int n_exp, int k, int hidden, int ff,
                      const float *logits, const float *h, int n_tok, float *out, int *idx_out, float *w_out,
                      void *ws, size_t ws_bytes, le_stream_t stream);
/* Status of the MoE layer calls made with workspace ws (no counterpart in the reference, which
 * has no device-side waits): synchronizes `stream`, returns LE_ERR_TIMEOUT (and clears the status)
 * if a one-launch layer on ws gave up at its barrier since the last check, else LE_OK. Not for use
 * under graph capture. */
int le_moe_check(le_ctx *ctx, const void *ws, le_stream_t stream);

#ifdef __cplusplus
}
#endif
#endif /* LE_QMM_H */
