"""MI355X-native MTP speculative-decode verify step for Cubic-quantized models.

Two halves, both hand-written HIP for gfx950 behind a C ABI
(include/cubic_mi355x.h), loaded through ctypes:

* ``linear``   -- Cubic non-uniform-codebook weight-only GEMM (WNA16) with the
  reference's packed-linear operator API (PackedLinearOperators, bind_linear,
  bind_linear_group, the Cubic extension hooks).
* ``sampling`` -- acceptance: candidate preparation, K1 p/q verification,
  accepted-prefix merge, and the fused single-pass verify-from-logits plan.
"""
from .quantization import (  # noqa: F401
    CUBIC_FORMAT,
    QuantizationError,
    QuantizationScheme,
    QuantizedMatrix,
    parse_group,
    payload_headers,
    quantize_cubic,
)

__version__ = "0.1.0"
