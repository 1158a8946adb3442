"""One kernel registry shared by all profiles (reference fp8_gemm_h20/engine.py:5-19).

`KERNELS[impl] = (module, function)`; the function is imported on first use,
so importing the package and selecting configs neither loads libfp8bg.so nor
touches the GPU.  `run(entry, args)` calls fn(A, B, As, Bs, dict(config)).

gfx950-native impls written by this package's tables:
  tiled   LDS-tiled MFMA kernel, optional tail or full split-K
  skinny  small-M kernel: operands straight to registers, waves split K
  ring    large-tile kernel: direct-to-LDS ring, one barrier per K group
  shortk  K == 256 kernel, no K loop (also accepts the reference's BM/BN keys)
Reference H20 impl names, accepted so reference tables keep working; each
runs on the gfx950 kernels (see kernels.py):
  triton, gluon, v2, scale_tma
"""
from functools import lru_cache
from importlib import import_module

KERNELS = {
    "tiled": ("kernels", "tiled"),
    "skinny": ("kernels", "skinny"),
    "ring": ("kernels", "ring"),
    "shortk": ("kernels", "shortk"),
    "triton": ("kernels", "triton"),
    "gluon": ("kernels", "gluon"),
    "v2": ("kernels", "v2"),
    "scale_tma": ("kernels", "scale_tma"),
}

# impls whose config uses this package's gfx950 keys
NATIVE = ("tiled", "skinny", "ring", "shortk")


@lru_cache(maxsize=None)
def kernel(name):
    module, function = KERNELS[name]
    return getattr(import_module(f".{module}", __package__), function)


def run(entry, args, **epilogue):
    return kernel(entry["impl"])(*args, dict(entry["config"]), **epilogue)
