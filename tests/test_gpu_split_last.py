"""The in-kernel split-K reduction (SPLIT_MODE "last") of the skinny and ring kernels.

Each split workgroup stores its partial tile with device-scope stores and
counts it in the tile's counter; the workgroup that completes the count sums
the partials in split order and writes C.  The summation order is the
two-kernel full split's, so the result must be bitwise that of
SPLIT_MODE "full", on every call: a partial read before it was visible (the
writer may run on another XCD, with its own L2) would show up as a
difference.  The counters must be left at zero, so repeated calls, hipGraph
replays and calls that share the workspace with the two-kernel splits keep
giving the same result.
"""
import ctypes

import numpy as np
import pytest
import torch

from fp8_gemm_h20 import _lib, kernels, quant
from oracle import blockfp8 as ob

pytestmark = pytest.mark.gpu

TOL = 1e-2
COS = 0.99999

# (M, N, K, config): few weight tiles and long K, split over the CUs
CASES = [
    (16, 512, 3072, dict(BLOCK_W=16, BLOCK_T=16, WAVES_K=4, UNROLL=2, SPLIT=8)),
    (32, 512, 3072, dict(BLOCK_W=16, BLOCK_T=16, WAVES_K=4, UNROLL=2, SPLIT=4)),
    (1, 1024, 2048, dict(BLOCK_W=16, BLOCK_T=16, WAVES_K=4, UNROLL=4, SPLIT=4)),
    (37, 2048, 4096, dict(BLOCK_W=32, BLOCK_T=16, WAVES_K=4, UNROLL=2, SPLIT=4, XCD_REMAP=True)),
    (5, 3072, 2048, dict(BLOCK_W=16, BLOCK_T=16, WAVES_K=8, UNROLL=1, SPLIT=2)),
    (50, 512, 3072, dict(BLOCK_W=16, BLOCK_T=64, WAVES_K=4, UNROLL=2, SPLIT=8)),
]


def oracle_ref(A, B, As, Bs):
    return ob.dequant_matmul(A.cpu().view(torch.uint8).numpy(), B.cpu().view(torch.uint8).numpy(),
                             As.cpu().numpy(), Bs.cpu().numpy())


def check(out, ref, what):
    got = out.float().cpu().numpy()
    assert np.isfinite(got).all(), what
    assert ob.error(got, ref) <= TOL and ob.cosine(got, ref) >= COS, what


@pytest.mark.parametrize("m,n,k,cfg", CASES, ids=lambda v: str(v) if not isinstance(v, dict) else "")
def test_in_kernel_split_is_bitwise_the_two_kernel_split(m, n, k, cfg):
    print(f"split last M={m} N={n} K={k} {cfg}", flush=True)
    last = dict(cfg, SPLIT_MODE="last")
    full = dict(cfg, SPLIT_MODE="full")
    inputs = [quant.make_inputs(m, n, k, seed=s, device="cuda") for s in (1, 2)]
    bias = torch.randn(n, generator=torch.Generator().manual_seed(9)).to(torch.bfloat16).cuda()
    want = [kernels.skinny(*x, full) for x in inputs]
    want_b = [kernels.skinny(*x, full, bias=bias) for x in inputs]
    for x, w in zip(inputs, want):
        check(w, oracle_ref(*x), (m, n, k, "full"))
    # alternate the two input sets (and the two-kernel split on the same
    # workspace) so that a stale partial or a counter left non-zero shows
    for i in range(24):
        j = i % 2
        got = kernels.skinny(*inputs[j], last)
        assert torch.equal(got.view(torch.int16), want[j].view(torch.int16)), (i, m, n, k)
        if i % 3 == 0:
            assert torch.equal(kernels.skinny(*inputs[j], full), want[j])
        if i % 4 == 1:
            got_b = kernels.skinny(*inputs[j], last, bias=bias)
            assert torch.equal(got_b.view(torch.int16), want_b[j].view(torch.int16)), (i, "bias")
    torch.cuda.synchronize()


def test_in_kernel_split_graph_replays_and_two_streams():
    # counters reset inside the kernel: many replays of graphs on two streams
    # (each with its own workspace) stay bitwise equal to the eager result
    m, n, k = 16, 512, 3072
    cfg = dict(BLOCK_W=16, BLOCK_T=16, WAVES_K=4, UNROLL=2, SPLIT=8, SPLIT_MODE="last")
    args = [quant.make_inputs(m, n, k, seed=s, device="cuda") for s in (3, 4)]
    eager = [kernels.skinny(*a, dict(cfg, SPLIT_MODE="full")) for a in args]
    streams = [torch.cuda.Stream(), torch.cuda.Stream()]
    graphs, outs = [], []
    for s, a in zip(streams, args):
        s.wait_stream(torch.cuda.current_stream())
        with torch.cuda.stream(s):
            for _ in range(2):
                kernels.skinny(*a, cfg)
    torch.cuda.synchronize()
    for s, a in zip(streams, args):
        g = torch.cuda.CUDAGraph()
        with torch.cuda.graph(g, stream=s):
            o = [kernels.skinny(*a, cfg) for _ in range(8)]
        graphs.append(g)
        outs.append(o)
    for r in range(30):
        for s, g in zip(streams, graphs):
            with torch.cuda.stream(s):
                g.replay()
        if r % 10 == 9:
            torch.cuda.synchronize()
            for o, e in zip(outs, eager):
                for x in o:
                    assert torch.equal(x.view(torch.int16), e.view(torch.int16)), r
    torch.cuda.synchronize()


def test_in_kernel_split_fused_quantiser_and_no_alloc():
    # the fused-quantiser linear and the allocation-free entry point run the
    # same reduction: bitwise equal to their two-kernel split
    lib = _lib.lib()
    m, n, k = 8, 512, 3072
    x = torch.randn(m, k, generator=torch.Generator().manual_seed(5)).to(torch.bfloat16).cuda()
    _, B, _, Bs = quant.make_inputs(m, n, k, device="cuda")
    base = dict(BLOCK_W=16, BLOCK_T=16, WAVES_K=4, UNROLL=2, SPLIT=8)
    f_full = kernels.linear_fused(x, B, Bs, dict(base, SPLIT_MODE="full"), 1e-10)
    for _ in range(4):
        f_last = kernels.linear_fused(x, B, Bs, dict(base, SPLIT_MODE="last"), 1e-10)
        assert torch.equal(f_last.view(torch.int16), f_full.view(torch.int16))
    A, B, As, Bs = quant.make_inputs(16, n, k, device="cuda")
    want = kernels.skinny(A, B, As, Bs, dict(base, SPLIT_MODE="full"))
    c = kernels.skinny_struct(dict(base, SPLIT_MODE="last"))
    for _ in range(4):
        C = torch.full((16, n), float("nan"), dtype=torch.bfloat16, device="cuda")
        _lib.check(lib.fp8bg_gemm_noalloc(A.data_ptr(), B.data_ptr(), As.data_ptr(), As.stride(0),
                                          As.stride(1), Bs.data_ptr(), Bs.stride(0), Bs.stride(1),
                                          None, C.data_ptr(), 16, n, k, ctypes.byref(c),
                                          _lib.num_cus(0), torch.cuda.current_stream().cuda_stream))
        torch.cuda.synchronize()
        assert torch.equal(C.view(torch.int16), want.view(torch.int16))


# ring instances with token tiles up to 64 (fp8bg_ring_last): each wave of a
# split tile counts its own part, the last one sums it in split order
RING_CASES = [
    (37, 3072, 2048, dict(BLOCK_W=64, BLOCK_T=64, WAVES_W=4, WAVES_T=1, STAGES=4, SPLIT=4)),
    (64, 4608, 3072, dict(BLOCK_W=64, BLOCK_T=64, WAVES_W=4, WAVES_T=1, STAGES=8, K_UNROLL=4, WAVES_K=2,
                          SPLIT=2)),
    (32, 12288, 2048, dict(BLOCK_W=128, BLOCK_T=32, WAVES_W=4, WAVES_T=1, STAGES=4, SPLIT=2)),
    (50, 512, 3072, dict(BLOCK_W=64, BLOCK_T=64, WAVES_W=2, WAVES_T=2, STAGES=8, K_UNROLL=4, SPLIT=2)),
    (100, 3072, 2048, dict(BLOCK_W=192, BLOCK_T=64, WAVES_W=6, WAVES_T=2, STAGES=4, SPLIT=2)),
    (37, 2048, 4096, dict(BLOCK_W=64, BLOCK_T=64, WAVES_W=4, WAVES_T=1, STAGES=8, K_UNROLL=4, WAVES_K=4,
                          SPLIT=2)),
    (7, 1024, 2048, dict(BLOCK_W=128, BLOCK_T=64, WAVES_W=4, WAVES_T=1, STAGES=6, K_UNROLL=2, WAVES_K=2,
                         SPLIT=4, XCD_REMAP=True)),
]


@pytest.mark.parametrize("m,n,k,cfg", RING_CASES, ids=lambda v: str(v) if not isinstance(v, dict) else "")
def test_ring_in_kernel_split_is_bitwise_the_two_kernel_split(m, n, k, cfg):
    print(f"ring split last M={m} N={n} K={k} {cfg}", flush=True)
    last = dict(cfg, SPLIT_MODE="last")
    full = dict(cfg, SPLIT_MODE="full")
    inputs = [quant.make_inputs(m, n, k, seed=s, device="cuda") for s in (5, 6)]
    bias = torch.randn(n, generator=torch.Generator().manual_seed(8)).to(torch.bfloat16).cuda()
    want = [kernels.ring(*x, full) for x in inputs]
    want_b = [kernels.ring(*x, full, bias=bias) for x in inputs]
    for x, w in zip(inputs, want):
        check(w, oracle_ref(*x), (m, n, k, "ring full"))
    for i in range(16):
        j = i % 2
        got = kernels.ring(*inputs[j], last)
        assert torch.equal(got.view(torch.int16), want[j].view(torch.int16)), (i, m, n, k)
        if i % 3 == 0:
            assert torch.equal(kernels.ring(*inputs[j], full), want[j])
        if i % 4 == 1:
            got_b = kernels.ring(*inputs[j], last, bias=bias)
            assert torch.equal(got_b.view(torch.int16), want_b[j].view(torch.int16)), (i, "bias")
    torch.cuda.synchronize()


def test_ring_in_kernel_split_graph_replays():
    m, n, k = 37, 3072, 2048
    cfg = dict(BLOCK_W=64, BLOCK_T=64, WAVES_W=4, WAVES_T=1, STAGES=8, K_UNROLL=4, WAVES_K=2, SPLIT=4,
               SPLIT_MODE="last")
    args = quant.make_inputs(m, n, k, seed=9, device="cuda")
    eager = kernels.ring(*args, dict(cfg, SPLIT_MODE="full"))
    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(s):
        for _ in range(2):
            kernels.ring(*args, cfg)
    torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g, stream=s):
        outs = [kernels.ring(*args, cfg) for _ in range(6)]
    for r in range(20):
        with torch.cuda.stream(s):
            g.replay()
        if r % 5 == 4:
            torch.cuda.synchronize()
            for o in outs:
                assert torch.equal(o.view(torch.int16), eager.view(torch.int16)), r
    torch.cuda.synchronize()


def test_in_kernel_split_beyond_the_counters_takes_two_launches():
    # 384 split tiles of 192 x 64 with 12 waves need 4608 counters, more than
    # FP8BG_COUNTERS: the plan falls back to the two-kernel reduction, and the
    # entry still gives the full split's C bit for bit (a table entry of this
    # mode tuned at a smaller M stays usable at any M)
    m, n, k = 384, 12288, 2048
    cfg = dict(BLOCK_W=192, BLOCK_T=64, WAVES_W=6, WAVES_T=2, STAGES=4, SPLIT=2)
    plan = _lib.make_plan(m, n, k, kernels.ring_struct(dict(cfg, SPLIT_MODE="last")), 256)
    assert (plan.n_split, plan.launches) == (384, 2)
    print(f"ring split last beyond counters M={m} N={n} K={k}", flush=True)
    args = quant.make_inputs(m, n, k, seed=3, device="cuda")
    want = kernels.ring(*args, dict(cfg, SPLIT_MODE="full"))
    check(want, oracle_ref(*args), "ring full, 384 split tiles")
    got = kernels.ring(*args, dict(cfg, SPLIT_MODE="last"))
    assert torch.equal(got.view(torch.int16), want.view(torch.int16))
    torch.cuda.synchronize()
