"""MI355X-native GGUF quantized-matmul hot path (Q8_0, Q4_K, Q6_K, IQ2_XXS, IQ3_XXS; dequant/matvec also Q4_0, Q3_K, Q5_K, IQ2_S).

The product is the C-ABI library lastengine_amd/lib/lible_qmm.so plus its gfx950 code objects
(include/le_qmm.h, include/le_quant.h). This package is the Python-side binding used by the tests
and the benchmark; see lastengine_amd.qmm.
"""
from .qmm import (LeError, Engine, TYPES, MV_TYPES, Q4_0, Q8_0, Q3_K, Q4_K, Q5_K, Q6_K, IQ2_XXS, IQ3_XXS, IQ2_S,
                  block_info, row_bytes,
                  fill_normal, quantize_rows, f32_to_f16, library_path)

__all__ = ["LeError", "Engine", "TYPES", "MV_TYPES", "Q4_0", "Q8_0", "Q3_K", "Q4_K", "Q5_K", "Q6_K", "IQ2_XXS",
           "IQ3_XXS", "IQ2_S", "block_info",
           "row_bytes", "fill_normal", "quantize_rows", "f32_to_f16", "library_path"]
