"""fp8bg_gemm_noalloc (static split-K scratch) against fp8bg_gemm (caller's
workspace), through the C ABI.

Both run the same kernels in the same fixed summation order, so C must be
bitwise equal; it must also meet the parity bar against the oracle.  Each
case makes two calls in a row, the second with fewer rows, so the second
call runs over the first call's leftover partials (and, for the in-kernel
reductions, its counters) in the shared scratch.  The entry point exists for
callers that cannot allocate, such as code under hipGraph capture: its calls
are also captured on a side stream and replayed, and a fresh process makes
its first call of the entry point under capture (the call that looks up the
scratch's device address).
"""
import ctypes
import subprocess
import sys
from pathlib import Path

import numpy as np
import pytest
import torch

from fp8_gemm_h20 import _lib, kernels, quant
from oracle import blockfp8 as ob

pytestmark = pytest.mark.gpu

TOL = 1e-2
COS = 0.99999

# (N, K, first M, second M, impl, config): every one splits K, so the
# scratch carries the partials
CASES = [
    # a two-kernel ring split whose workspace (3.7 Mi elements) nearly fills
    # the scratch
    (2048, 4096, 97, 40, "ring", dict(BLOCK_W=128, BLOCK_T=32, WAVES_W=4, WAVES_T=1, STAGES=4,
                                      GROUP_SIZE_M=8, K_UNROLL=2, SPLIT=4, SPLIT_MODE="full")),
    # the ring's in-kernel reduction: per-wave counters in the scratch's
    # counter words, reused by the second call
    (3072, 2048, 37, 20, "ring", dict(BLOCK_W=64, BLOCK_T=64, WAVES_W=4, WAVES_T=1, STAGES=4,
                                      SPLIT=4, SPLIT_MODE="last")),
    # stream-K: runs' partial slots and per-wave tile counters in the scratch
    (1024, 2048, 100, 40, "ring", dict(BLOCK_W=64, BLOCK_T=64, WAVES_W=4, WAVES_T=1, STAGES=8,
                                       K_UNROLL=4, GROUP_SIZE_M=8, XCD_REMAP=True, SPLIT_MODE="stream")),
    (12288, 2048, 8, 3, "skinny", dict(BLOCK_W=16, BLOCK_T=16, WAVES_K=4, UNROLL=2, SPLIT=4,
                                       SPLIT_MODE="last")),
    (12288, 2048, 64, 3, "skinny", dict(BLOCK_W=16, BLOCK_T=64, WAVES_K=4, UNROLL=2, SPLIT=4,
                                        SPLIT_MODE="full")),
    (3072, 2048, 960, 300, "tiled", dict(BLOCK_W=64, BLOCK_T=64, SPLIT=2, SPLIT_MODE="tail",
                                          GROUP_SIZE_M=4)),
    (512, 3072, 160, 37, "ring", dict(BLOCK_W=64, BLOCK_T=64, WAVES_W=4, WAVES_T=1, STAGES=8,
                                      K_UNROLL=2, WAVES_K=2, SPLIT=2, SPLIT_MODE="full")),
]


def cstruct(impl, cfg):
    if impl == "ring":
        return kernels.ring_struct(cfg)
    if impl == "skinny":
        return kernels.skinny_struct(cfg)
    return kernels.tiled_struct(cfg)


def call(lib, entry, A, B, As, Bs, c, noalloc, bias=None):
    m, k = A.shape
    n = B.shape[0]
    cus = _lib.num_cus(0)
    C = torch.full((m, n), float("nan"), dtype=torch.bfloat16, device="cuda")
    stream = torch.cuda.current_stream().cuda_stream
    common = (A.data_ptr(), B.data_ptr(), As.data_ptr(), As.stride(0), As.stride(1),
              Bs.data_ptr(), Bs.stride(0), Bs.stride(1),
              None if bias is None else bias.data_ptr(), C.data_ptr(), m, n, k, ctypes.byref(c), cus)
    if noalloc:
        _lib.check(lib.fp8bg_gemm_noalloc(*common, stream))
    else:
        plan = _lib.make_plan(m, n, k, c, cus)
        # zero: the in-kernel reductions' counters must start at zero
        ws = torch.zeros(max(plan.ws_elems, 1), dtype=torch.float32, device="cuda")
        _lib.check(lib.fp8bg_gemm(*common, ws.data_ptr(), ws.numel(), stream))
        torch.cuda.synchronize()
    return C


@pytest.mark.parametrize("n,k,m1,m2,impl,cfg", CASES, ids=lambda v: str(v) if not isinstance(v, dict) else "")
def test_noalloc_matches_gemm_with_workspace(n, k, m1, m2, impl, cfg):
    lib = _lib.lib()
    c = cstruct(impl, cfg)
    cus = _lib.num_cus(0)
    print(f"noalloc {impl} N={n} K={k} M={m1},{m2}", flush=True)
    for m in (m1, m2):
        plan = _lib.make_plan(m, n, k, c, cus)
        assert plan.n_split > 0 and plan.ws_elems <= _lib.SCRATCH_ELEMS, (m, plan.ws_elems)
        assert cfg.get("SPLIT_MODE") != "stream" or plan.stream_units > 0
        A, B, As, Bs = quant.make_inputs(m, n, k, seed=m + 7, device="cuda")
        got = call(lib, impl, A, B, As, Bs, c, noalloc=True)
        want = call(lib, impl, A, B, As, Bs, c, noalloc=False)
        torch.cuda.synchronize()
        assert torch.equal(got.view(torch.int16), want.view(torch.int16)), (impl, m)
        ref = ob.dequant_matmul(A.cpu().view(torch.uint8).numpy(), B.cpu().view(torch.uint8).numpy(),
                                As.cpu().numpy(), Bs.cpu().numpy())
        g = got.float().cpu().numpy()
        assert np.isfinite(g).all()
        assert ob.error(g, ref) <= TOL and ob.cosine(g, ref) >= COS, (impl, m)


def test_noalloc_without_split_and_with_bias():
    # a plan without split tiles never touches the scratch; the bias path and
    # column-major As go through unchanged
    lib = _lib.lib()
    m, n, k = 200, 3072, 2048
    c = kernels.ring_struct(dict(BLOCK_W=128, BLOCK_T=64, WAVES_W=4, WAVES_T=1, STAGES=6))
    A, B, As, Bs = quant.make_inputs(m, n, k, device="cuda")
    As_cm = As.T.contiguous().T
    bias = torch.randn(n, generator=torch.Generator().manual_seed(3)).to(torch.bfloat16).cuda()
    got = call(lib, "ring", A, B, As_cm, Bs, c, noalloc=True, bias=bias)
    want = call(lib, "ring", A, B, As, Bs, c, noalloc=False, bias=bias)
    torch.cuda.synchronize()
    assert torch.equal(got.view(torch.int16), want.view(torch.int16))


def test_noalloc_rejects_oversized_plan_on_the_gpu():
    lib = _lib.lib()
    m, n, k = 16384, 12288, 2048
    c = kernels.tiled_struct(dict(BLOCK_W=256, BLOCK_T=128, SPLIT=16, SPLIT_MODE="full"))
    A = torch.empty(m, k, dtype=torch.float8_e4m3fn, device="cuda")
    B = torch.empty(n, k, dtype=torch.float8_e4m3fn, device="cuda")
    As = torch.ones(m, k // 128, device="cuda")
    Bs = torch.ones(n // 128, k // 128, device="cuda")
    C = torch.empty(m, n, dtype=torch.bfloat16, device="cuda")
    rc = lib.fp8bg_gemm_noalloc(A.data_ptr(), B.data_ptr(), As.data_ptr(), As.stride(0), 1,
                                Bs.data_ptr(), Bs.stride(0), 1, None, C.data_ptr(), m, n, k,
                                ctypes.byref(c), _lib.num_cus(0),
                                torch.cuda.current_stream().cuda_stream)
    assert rc == _lib.ERR_SCRATCH


def capture_cases():
    return [(3072, 2048, 37, "ring", dict(BLOCK_W=64, BLOCK_T=64, WAVES_W=4, WAVES_T=1, STAGES=4,
                                         SPLIT=4, SPLIT_MODE="full")),
            (12288, 2048, 8, "skinny", dict(BLOCK_W=16, BLOCK_T=16, WAVES_K=4, UNROLL=2, SPLIT=4,
                                            SPLIT_MODE="last")),
            (1024, 2048, 100, "ring", dict(BLOCK_W=64, BLOCK_T=64, WAVES_W=4, WAVES_T=1, STAGES=8,
                                           K_UNROLL=4, GROUP_SIZE_M=8, SPLIT_MODE="stream"))]


def test_noalloc_calls_captured_in_a_graph_replay_bitwise():
    # split noalloc calls captured on a side stream, replayed with eager work
    # and synchronisations between the replays: every replay equals the
    # workspace entry point's result
    lib = _lib.lib()
    cus = _lib.num_cus(0)
    work = []
    for n, k, m, impl, cfg in capture_cases():
        c = cstruct(impl, cfg)
        A, B, As, Bs = quant.make_inputs(m, n, k, seed=m + 11, device="cuda")
        want = call(lib, impl, A, B, As, Bs, c, noalloc=False)
        work.append((A, B, As, Bs, c, want))
    torch.cuda.synchronize()
    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    outs = []
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g, stream=s):
        for A, B, As, Bs, c, want in work:
            m, k = A.shape
            n = B.shape[0]
            C = torch.empty((m, n), dtype=torch.bfloat16, device="cuda")
            _lib.check(lib.fp8bg_gemm_noalloc(A.data_ptr(), B.data_ptr(), As.data_ptr(), As.stride(0),
                                              As.stride(1), Bs.data_ptr(), Bs.stride(0), Bs.stride(1),
                                              None, C.data_ptr(), m, n, k, ctypes.byref(c), cus,
                                              s.cuda_stream))
            outs.append(C)
    for r in range(6):
        with torch.cuda.stream(s):
            g.replay()
        torch.cuda.synchronize()
        for C, (_, _, _, _, _, want) in zip(outs, work):
            assert torch.equal(C.view(torch.int16), want.view(torch.int16)), r
        # eager calls of the same entry point between the replays
        for A, B, As, Bs, c, want in work:
            got = call(lib, "", A, B, As, Bs, c, noalloc=True)
            torch.cuda.synchronize()
            assert torch.equal(got.view(torch.int16), want.view(torch.int16)), r


CHILD = r"""
import ctypes, sys
sys.path.insert(0, sys.argv[1])
import torch
from fp8_gemm_h20 import _lib, kernels, quant
lib = _lib.lib()
cus = _lib.num_cus(0)
m, n, k = 37, 3072, 2048
c = kernels.ring_struct(dict(BLOCK_W=64, BLOCK_T=64, WAVES_W=4, WAVES_T=1, STAGES=4, SPLIT=4,
                             SPLIT_MODE="last"))
A, B, As, Bs = quant.make_inputs(m, n, k, seed=5, device="cuda")
plan = _lib.make_plan(m, n, k, c, cus)
ws = torch.zeros(plan.ws_elems, dtype=torch.float32, device="cuda")
want = torch.empty((m, n), dtype=torch.bfloat16, device="cuda")
args = (A.data_ptr(), B.data_ptr(), As.data_ptr(), As.stride(0), As.stride(1), Bs.data_ptr(),
        Bs.stride(0), Bs.stride(1), None)
_lib.check(lib.fp8bg_gemm(*args, want.data_ptr(), m, n, k, ctypes.byref(c), cus, ws.data_ptr(),
                          ws.numel(), torch.cuda.current_stream().cuda_stream))
torch.cuda.synchronize()
print("child: reference done; first noalloc call under capture", flush=True)
s = torch.cuda.Stream()
s.wait_stream(torch.cuda.current_stream())
C = torch.empty((m, n), dtype=torch.bfloat16, device="cuda")
g = torch.cuda.CUDAGraph()
with torch.cuda.graph(g, stream=s):
    rc = lib.fp8bg_gemm_noalloc(*args, C.data_ptr(), m, n, k, ctypes.byref(c), cus, s.cuda_stream)
assert rc == 0, _lib.strerror(rc)
for r in range(5):
    C.fill_(float("nan"))
    torch.cuda.synchronize()
    with torch.cuda.stream(s):
        g.replay()
    torch.cuda.synchronize()
    assert torch.equal(C.view(torch.int16), want.view(torch.int16)), r
print("child: ok", flush=True)
"""


def test_first_noalloc_call_of_a_process_under_capture():
    # a fresh process whose first fp8bg_gemm_noalloc call (the one that
    # looks up the scratch address on the device) is made inside a graph
    # capture; the child exits with the test's status
    root = str(Path(__file__).resolve().parents[1])
    res = subprocess.run([sys.executable, "-c", CHILD, root], capture_output=True, text=True, timeout=300)
    print(res.stdout[-2000:], res.stderr[-2000:], flush=True)
    assert res.returncode == 0 and "child: ok" in res.stdout
