"""Opt-in runtime patch that routes SGLang's block-FP8 dense linear on ROCm to this package.

The ROCm counterpart of the reference's adapter (sgl_patch/fp8mm_sglang_patch.py:1-96).
On a gfx950 GPU SGLang's `dispatch_w8a8_block_fp8_linear()` hands out either
aiter's or Triton's block-FP8 linear.  Once
`sglang.srt.layers.quantization.fp8_utils` has been imported, this module
wraps that dispatcher.  Eligible calls then run `linear()`: the gfx950
activation quantiser, then the GEMM with the bias fused in the epilogue, with
no host sync.  Every other call falls through to the function SGLang chose.
No SGLang source is edited.

Environment (the reference's names, so existing launch scripts keep working):
  FP8MM_ENABLE=1          install the patch when this module is imported
  FP8MM_PROFILE=35b_tp1   or 122b_tp4: the measured shape/config profile
  FP8MM_HOME=/path        prepended to sys.path (where this package lives)
  FP8MM_SHUFFLE_WEIGHTS=1 also keep each weight in the shuffled layout
                          (`shuffle_weight`; faster small-M loads, bitwise
                          the same results, one more copy of the weights)

Loading it into every SGLang process: put a `sitecustomize.py` containing
`import fp8_gemm_h20.sglang_patch` on PYTHONPATH (the reference's
sgl_patch/sitecustomize.py does the same for its adapter), or import this
module before SGLang builds its model.  Importing it does not import torch
or load the HIP library; both wait for the first patched call.
"""
import importlib.abc
import importlib.machinery
import os
import warnings
import sys

TARGET = "sglang.srt.layers.quantization.fp8_utils"

# Functions the ROCm build of SGLang may hand out for block-FP8 weights; the
# patch replaces only these (the reference replaces only the DeepGEMM path,
# fp8mm_sglang_patch.py:63-66).
ROCM_LINEARS = ("aiter_w8a8_block_fp8_linear", "triton_w8a8_block_fp8_linear")


def eligible(profile, input, weight, block_size, weight_scale, input_scale, bias):
    """True when `linear()` computes this call; mirrors the reference's
    predicate (fp8mm_sglang_patch.py:36-46) for gfx950: OCP e4m3fn weights
    with 128x128 fp32 scales, bf16 activations on the weight's GPU, no static
    input scale, a bf16 [N] bias if any, and a shape the profile covers."""
    import torch
    from . import supports
    if weight.ndim != 2 or input.ndim < 1:
        return False
    n, k = weight.shape
    if input.shape[-1] != k or input.numel() == 0:
        return False
    return (input_scale is None
            and input.dtype == torch.bfloat16
            and input.is_cuda and input.device == weight.device
            and weight.dtype == torch.float8_e4m3fn and weight.is_contiguous()
            and weight_scale.dtype == torch.float32 and weight_scale.device == weight.device
            and tuple(weight_scale.shape) == (n // 128, k // 128)
            and list(block_size) == [128, 128]
            and (bias is None or (bias.dtype == torch.bfloat16 and tuple(bias.shape) == (n,)
                                  and bias.device == weight.device))
            and supports(profile, input.numel() // k, n, k))


_OOM_WARNED = []


def shuffled_copy(weight):
    """The weight in the shuffled layout, made on its first eligible call
    and kept on the tensor (made again after an in-place change of the
    weight, which bumps its version counter); the row-major weight stays for
    SGLang's own paths.  None while a CUDA graph is being captured: a copy
    made there would live in the graph's memory pool, so a weight first seen
    during capture runs row-major until an eager call makes its copy.

    The copies double the weights' memory (about 35 GB for the 35B model),
    allocated during SGLang's warm-up, after it has sized its KV-cache pool
    from the free memory: lower --mem-fraction-static by the weights' share
    when enabling them.  A copy that does not fit is not made: that weight
    runs row-major (the same C bit for bit), with one warning per process."""
    import torch
    from . import shuffle_weight
    held = getattr(weight, "_fp8mm_shuffled", None)
    if held is not None and held[0] == weight._version:
        return held[1]
    if held is not None and held[1] is None:
        return None                          # no room for this weight's copy
    if torch.cuda.is_current_stream_capturing():
        return None
    try:
        copy = shuffle_weight(weight)
    except torch.cuda.OutOfMemoryError:
        if not _OOM_WARNED:
            _OOM_WARNED.append(True)
            warnings.warn("fp8mm: no memory for a shuffled weight copy (FP8MM_SHUFFLE_WEIGHTS=1); "
                          "such weights run row-major.  Lower SGLang's --mem-fraction-static by the "
                          "FP8 weights' share to make room for the copies.", RuntimeWarning)
        weight._fp8mm_shuffled = (weight._version, None)
        return None
    held = (weight._version, copy)
    weight._fp8mm_shuffled = held
    return held[1]


def make_linear(orig_linear, profile, shuffle_weights=False):
    """Wrap one of SGLang's block-FP8 linears; `.fp8mm_stats` counts the
    calls taken here ("ours") and passed through ("fallback").  With
    shuffle_weights the GEMM reads each weight's shuffled copy."""
    stats = {"ours": 0, "fallback": 0}

    def fp8mm_w8a8_block_fp8_linear(input, weight, block_size, weight_scale, input_scale=None,
                                    bias=None):
        if not eligible(profile, input, weight, block_size, weight_scale, input_scale, bias):
            stats["fallback"] += 1
            return orig_linear(input, weight, block_size, weight_scale, input_scale, bias)
        from . import linear
        stats["ours"] += 1
        w = shuffled_copy(weight) if shuffle_weights else None
        return linear(input, weight if w is None else w, weight_scale, profile=profile,
                      bias=None if bias is None else bias.contiguous())

    fp8mm_w8a8_block_fp8_linear.fp8mm_stats = stats
    fp8mm_w8a8_block_fp8_linear.fp8mm_wrapped = orig_linear
    return fp8mm_w8a8_block_fp8_linear


def patch_module(mod, profile=None, shuffle_weights=None):
    """Install the wrapper into an imported fp8_utils module (idempotent).
    shuffle_weights None: from FP8MM_SHUFFLE_WEIGHTS."""
    if getattr(mod.dispatch_w8a8_block_fp8_linear, "fp8mm_patched", False):
        return
    profile = profile or os.environ.get("FP8MM_PROFILE", "35b_tp1")
    if shuffle_weights is None:
        shuffle_weights = os.environ.get("FP8MM_SHUFFLE_WEIGHTS") == "1"
    from .config import get_profile
    get_profile(profile)                       # unknown profile: fail at install, not mid-serve
    orig_dispatch = mod.dispatch_w8a8_block_fp8_linear
    wrapped = {}

    def patched_dispatch(*args, **kwargs):
        orig = orig_dispatch(*args, **kwargs)
        if not any(orig is getattr(mod, name, None) for name in ROCM_LINEARS):
            return orig
        if orig not in wrapped:
            wrapped[orig] = make_linear(orig, profile, shuffle_weights)
        return wrapped[orig]

    patched_dispatch.fp8mm_patched = True
    patched_dispatch.fp8mm_profile = profile
    patched_dispatch.fp8mm_shuffle_weights = shuffle_weights
    mod.dispatch_w8a8_block_fp8_linear = patched_dispatch
    print(f"[fp8mm] patched {TARGET}.dispatch_w8a8_block_fp8_linear (profile={profile}"
          f"{', shuffled weights' if shuffle_weights else ''})", file=sys.stderr, flush=True)


class _PatchingLoader(importlib.abc.Loader):
    """Runs the real loader, then patches the freshly executed module."""

    def __init__(self, inner, profile, shuffle_weights):
        self.inner = inner
        self.profile = profile
        self.shuffle_weights = shuffle_weights

    def create_module(self, spec):
        return self.inner.create_module(spec)

    def exec_module(self, module):
        self.inner.exec_module(module)
        patch_module(module, self.profile, self.shuffle_weights)


class PatchFinder(importlib.abc.MetaPathFinder):
    """Meta-path hook that intercepts the import of TARGET."""

    def __init__(self, profile=None, shuffle_weights=None):
        self.profile = profile
        self.shuffle_weights = shuffle_weights

    def find_spec(self, name, path, target=None):
        if name != TARGET:
            return None
        spec = importlib.machinery.PathFinder.find_spec(name, path)
        if spec is None or spec.loader is None:
            return None
        spec.loader = _PatchingLoader(spec.loader, self.profile, self.shuffle_weights)
        return spec


def install(profile=None, shuffle_weights=None):
    """Patch TARGET now if it is already imported, else when it is imported.
    Returns the meta-path finder (None when the module was patched in place)."""
    if TARGET in sys.modules:
        patch_module(sys.modules[TARGET], profile, shuffle_weights)
        return None
    finder = PatchFinder(profile, shuffle_weights)
    sys.meta_path.insert(0, finder)
    return finder


def uninstall(finder):
    """Remove a finder returned by install() (modules already patched stay so)."""
    if finder is not None and finder in sys.meta_path:
        sys.meta_path.remove(finder)


if os.environ.get("FP8MM_ENABLE") == "1":
    if os.environ.get("FP8MM_HOME"):
        sys.path.insert(0, os.environ["FP8MM_HOME"])
    install()
