"""ctypes binding of libfp8bg.so (declared in include/fp8bg.h).

Loading is lazy: importing the package or selecting configs never loads the
library or touches the GPU (reference docs/configuration.md:36).  A missing
library is an error, never a silent fallback.
"""
import ctypes
import os
import threading
from pathlib import Path

LIB_NAME = "libfp8bg.so"
LIB_PATH = Path(__file__).resolve().with_name(LIB_NAME)
ABI_VERSION = 12

OK = 0
ERR_SHAPE = 1
ERR_CONFIG = 2
ERR_WORKSPACE = 3
ERR_ALIGN = 4
ERR_LAUNCH = 5
ERR_DEVICE = 6
ERR_NULL = 7
ERR_SCRATCH = 8

# fp32 elements of fp8bg_gemm_noalloc's static split-K scratch (FP8BG_SCRATCH_ELEMS)
SCRATCH_ELEMS = 1 << 22

KIND_TILED = 0
KIND_SKINNY = 1
KIND_RING = 2

SPLIT_NONE = 0
SPLIT_TAIL = 1
SPLIT_FULL = 2
SPLIT_LAST = 3
SPLIT_STREAM = 4

# uint32 tile counters at the start of every split-K workspace (FP8BG_COUNTERS)
COUNTERS = 4096

FLAG_SCALE_LDS = 0x1
FLAG_XCD_REMAP = 0x2
FLAG_SWZ8 = 0x4
FLAG_SWZPAIR = 0x8
FLAG_B_SHUFFLED = 0x10

# Every symbol include/fp8bg.h declares.
EXPORTS = (
    "fp8bg_version",
    "fp8bg_num_cus",
    "fp8bg_make_plan",
    "fp8bg_config_supported",
    "fp8bg_gemm",
    "fp8bg_gemm_noalloc",
    "fp8bg_gemm_bf16a",
    "fp8bg_quant_act",
    "fp8bg_shuffle_b",
    "fp8bg_e4m3_encode_host",
    "fp8bg_e4m3_encode_device",
    "fp8bg_calib_mfma",
    "fp8bg_calib_mfma_promoted",
    "fp8bg_calib_read",
    "fp8bg_calib_write",
    "fp8bg_calib_launch",
    "fp8bg_strerror",
)


class Config(ctypes.Structure):
    """struct fp8bg_config."""
    _fields_ = [
        ("kind", ctypes.c_int32),
        ("block_w", ctypes.c_int32),
        ("block_t", ctypes.c_int32),
        ("waves_w", ctypes.c_int32),
        ("waves_t", ctypes.c_int32),
        ("waves_k", ctypes.c_int32),
        ("unroll", ctypes.c_int32),
        ("stages", ctypes.c_int32),
        ("split", ctypes.c_int32),
        ("split_mode", ctypes.c_int32),
        ("group_t", ctypes.c_int32),
        ("flags", ctypes.c_int32),
        ("k_fixed", ctypes.c_int32),
    ]


class Plan(ctypes.Structure):
    """struct fp8bg_plan."""
    _fields_ = [
        ("tiles_w", ctypes.c_int32),
        ("tiles_t", ctypes.c_int32),
        ("tiles", ctypes.c_int32),
        ("split", ctypes.c_int32),
        ("n_dp", ctypes.c_int32),
        ("n_split", ctypes.c_int32),
        ("grid", ctypes.c_int32),
        ("launches", ctypes.c_int32),
        ("ws_elems", ctypes.c_int64),
        ("lds_bytes", ctypes.c_int32),
        ("threads", ctypes.c_int32),
        ("kernel_id", ctypes.c_int32),
        ("stream_units", ctypes.c_int32),
    ]


class Fp8bgError(RuntimeError):
    """Nonzero return code from libfp8bg."""

    def __init__(self, code, msg):
        super().__init__(f"fp8bg error {code}: {msg}")
        self.code = code


_lock = threading.Lock()
_lib = None


def _declare(lib):
    i32, i64, vp = ctypes.c_int32, ctypes.c_int64, ctypes.c_void_p
    lib.fp8bg_version.argtypes = []
    lib.fp8bg_version.restype = ctypes.c_int
    lib.fp8bg_num_cus.argtypes = [ctypes.c_int, ctypes.POINTER(i32)]
    lib.fp8bg_num_cus.restype = ctypes.c_int
    lib.fp8bg_make_plan.argtypes = [i32, i32, i32, ctypes.POINTER(Config), i32, ctypes.POINTER(Plan)]
    lib.fp8bg_make_plan.restype = ctypes.c_int
    lib.fp8bg_config_supported.argtypes = [ctypes.POINTER(Config)]
    lib.fp8bg_config_supported.restype = ctypes.c_int
    lib.fp8bg_gemm.argtypes = [
        vp, vp,                 # A, B
        vp, i64, i64,           # As, strides
        vp, i64, i64,           # Bs, strides
        vp,                     # bias (bf16 [N] or NULL)
        vp, i32, i32, i32,      # C, M, N, K
        ctypes.POINTER(Config), i32,
        vp, i64,                # ws, ws_elems
        vp,                     # stream
    ]
    lib.fp8bg_gemm.restype = ctypes.c_int
    lib.fp8bg_gemm_noalloc.argtypes = lib.fp8bg_gemm.argtypes[:15] + [vp]
    lib.fp8bg_gemm_noalloc.restype = ctypes.c_int
    lib.fp8bg_gemm_bf16a.argtypes = [
        vp, i64, ctypes.c_float,  # X, row stride, eps
        vp, vp, i64, i64,       # B, Bs, strides
        vp,                     # bias (bf16 [N] or NULL)
        vp, i32, i32, i32,      # C, M, N, K
        ctypes.POINTER(Config), i32,
        vp, i64,                # ws, ws_elems
        vp, vp, i64, i64,       # q_out, s_out, s strides (or NULLs)
        vp,                     # stream
    ]
    lib.fp8bg_gemm_bf16a.restype = ctypes.c_int
    lib.fp8bg_quant_act.argtypes = [vp, i64, vp, vp, i64, i64, i32, i32, ctypes.c_float, vp]
    lib.fp8bg_quant_act.restype = ctypes.c_int
    lib.fp8bg_shuffle_b.argtypes = [vp, i64, vp, i32, i32, vp]
    lib.fp8bg_shuffle_b.restype = ctypes.c_int
    lib.fp8bg_e4m3_encode_host.argtypes = [vp, vp, i64]
    lib.fp8bg_e4m3_encode_host.restype = ctypes.c_int
    lib.fp8bg_e4m3_encode_device.argtypes = [vp, vp, i64, vp]
    lib.fp8bg_e4m3_encode_device.restype = ctypes.c_int
    lib.fp8bg_calib_mfma.argtypes = [vp, vp, i32, i32, vp]
    lib.fp8bg_calib_mfma.restype = ctypes.c_int
    lib.fp8bg_calib_mfma_promoted.argtypes = [vp, vp, vp, i32, i32, vp]
    lib.fp8bg_calib_mfma_promoted.restype = ctypes.c_int
    lib.fp8bg_calib_read.argtypes = [vp, i64, vp, i32, vp]
    lib.fp8bg_calib_read.restype = ctypes.c_int
    lib.fp8bg_calib_write.argtypes = [vp, i64, ctypes.c_uint32, i32, i32, vp]
    lib.fp8bg_calib_write.restype = ctypes.c_int
    lib.fp8bg_calib_launch.argtypes = [i32, vp]
    lib.fp8bg_calib_launch.restype = ctypes.c_int
    lib.fp8bg_strerror.argtypes = [ctypes.c_int]
    lib.fp8bg_strerror.restype = ctypes.c_char_p


def lib():
    """Load libfp8bg.so once (thread-safe); raise if it is not built."""
    global _lib
    if _lib is not None:
        return _lib
    with _lock:
        if _lib is None:
            path = os.environ.get("FP8BG_LIB", str(LIB_PATH))
            if not os.path.exists(path):
                raise RuntimeError(
                    f"fp8_gemm_h20: HIP library {path} is not built; run "
                    "`python -c 'import __graft_entry__ as g; g.build()'` or "
                    "`python -m fp8_gemm_h20.build` first")
            handle = ctypes.CDLL(path)
            _declare(handle)
            ver = handle.fp8bg_version()
            if ver != ABI_VERSION:
                raise RuntimeError(f"{path}: ABI version {ver}, expected {ABI_VERSION}; rebuild it")
            _lib = handle
    return _lib


def strerror(code):
    return lib().fp8bg_strerror(code).decode()


def check(code):
    if code != OK:
        raise Fp8bgError(code, strerror(code))


def make_plan(m, n, k, cfg, num_cus):
    plan = Plan()
    check(lib().fp8bg_make_plan(m, n, k, ctypes.byref(cfg), num_cus, ctypes.byref(plan)))
    return plan


def num_cus(device_index):
    out = ctypes.c_int32(0)
    check(lib().fp8bg_num_cus(device_index, ctypes.byref(out)))
    return out.value
