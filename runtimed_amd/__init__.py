"""MI355X-native (gfx950) quantized linear layers for runtimed.

librq.so holds the HIP kernels behind the C ABI of include/rq.h; `rq` binds it
with ctypes, `synth` makes seeded GGUF inputs.  Build with
``python -m runtimed_amd.build``.
"""
from .rq import (BF16, F16, F32, F8E4M3, FP8_PER_TOKEN, FP8_UNSCALED, GEOMETRY, Q4_0, Q4_K, Q5_0,
                 Q5_K, Q6_K, Q8_0, QTYPES, QWeight, RqError, dequant_tensor, fp8_gemm, fp8_gemm_q,
                 fp8_quantize, lib)

__all__ = ["BF16", "F16", "F32", "F8E4M3", "FP8_PER_TOKEN", "FP8_UNSCALED", "GEOMETRY", "Q4_0",
           "Q4_K", "Q5_0", "Q5_K", "Q6_K", "Q8_0", "QTYPES", "QWeight", "RqError", "dequant_tensor",
           "fp8_gemm", "fp8_gemm_q", "fp8_quantize", "lib"]
