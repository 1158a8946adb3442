"""Block-scaled FP8 GEMM for AMD Instinct MI355X (gfx950), with explicit model profiles.

Drop-in for the reference package fp8_gemm_h20 (its __init__.py:1-5):
`matmul(A, B, As, Bs, profile=...)`, `select`, `supports`,
`available_profiles`, plus `config.get_profile`; `quantize_act` and
`linear` add the activation quantiser and the adapter's dense linear, and
`shuffle_weight` an optional weight layout for faster small-M loads.  The kernels are
hand-written HIP for gfx950 in csrc/fp8bg.hip behind the C ABI of
include/fp8bg.h; nothing is loaded until the first matmul.
"""
from .dispatch import matmul, quantize_act, linear, shuffle_weight
from .config import available_profiles, select, supports

__all__ = ["matmul", "quantize_act", "linear", "shuffle_weight", "available_profiles", "select",
           "supports"]
