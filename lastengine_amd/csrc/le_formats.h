/* GGUF block geometry shared by the host library and the HIP kernels.
 *
 * Type ids and (values, bytes) per block follow the reference's src/quant.rs:10-31; row bytes =
 * cols / values * bytes (src/quant.rs:35). Matrices are row-major GGUF tensors: dims[0] = cols (K),
 * dims[1] = rows (N); expert slab e of a 3D tensor starts at e * rows * row_bytes
 * (src/cpu_ref.rs:110-115).
 */
#pragma once

#define LE_TYPE_Q4_0 2
#define LE_TYPE_Q8_0 8
#define LE_TYPE_Q3_K 11
#define LE_TYPE_Q4_K 12
#define LE_TYPE_Q5_K 13
#define LE_TYPE_Q6_K 14
#define LE_TYPE_IQ2_XXS 16
#define LE_TYPE_IQ3_XXS 18
#define LE_TYPE_IQ2_S 22

/* Every type is processed in "super-blocks" of 256 values: one K-quant/IQ block, or eight
 * consecutive Q8_0 / Q4_0 blocks. Bytes per 256-value super-block: */
#define LE_SB_BYTES_Q4_0 144
#define LE_SB_BYTES_Q8_0 272
#define LE_SB_BYTES_Q3_K 110
#define LE_SB_BYTES_Q5_K 176
#define LE_SB_BYTES_IQ2_S 82
#define LE_SB_BYTES_Q4_K 144
#define LE_SB_BYTES_Q6_K 210
#define LE_SB_BYTES_IQ2_XXS 66
#define LE_SB_BYTES_IQ3_XXS 98

static inline int le_block_geometry(int ty, int *values, int *bytes) {
    switch (ty) {
    case LE_TYPE_Q4_0: *values = 32; *bytes = 18; return 1;
    case LE_TYPE_Q8_0: *values = 32; *bytes = 34; return 1;
    case LE_TYPE_Q3_K: *values = 256; *bytes = 110; return 1;
    case LE_TYPE_Q5_K: *values = 256; *bytes = 176; return 1;
    case LE_TYPE_IQ2_S: *values = 256; *bytes = 82; return 1;
    case LE_TYPE_Q4_K: *values = 256; *bytes = 144; return 1;
    case LE_TYPE_Q6_K: *values = 256; *bytes = 210; return 1;
    case LE_TYPE_IQ2_XXS: *values = 256; *bytes = 66; return 1;
    case LE_TYPE_IQ3_XXS: *values = 256; *bytes = 98; return 1;
    default: return 0;
    }
}
