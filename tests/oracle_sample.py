"""The numpy oracle on a sampled block of a product too large for it whole.

Where M*N*K is too large for the oracle (oracle/blockfp8.py) to finish in
seconds, the GPU tests compare the whole C with a torch fp32 dequant-matmul,
and `pin` checks that torch C against the oracle on a block: the first and last 8 rows and
columns and an even spread between them, enough that every 256-row and every
128-column tile of C contributes.  The block's columns are weight rows, so
they are dequantised with their own block scales, `Bs[col // 128]`, through
the oracle's per-row-group dequantiser; `test_oracle.py` checks that this
equals the oracle's full product at the same rows and columns.
"""
import numpy as np
import torch

from oracle import blockfp8 as ob

ROWS = 80          # at most 80 sampled rows: 64 spread + 16 edge rows
COLS = 272         # at most 272 sampled columns: 256 spread + 16 edge columns


def spread(n, count):
    """Sorted unique indices in [0, n): the first and last 8 and `count - 16` evenly spaced."""
    if n <= count:
        return np.arange(n, dtype=np.int64)
    mid = np.linspace(8, n - 9, count - 16).round().astype(np.int64)
    return np.unique(np.concatenate([np.arange(8), mid, np.arange(n - 8, n)]))


def _u8(t):
    return t.detach().cpu().contiguous().view(torch.uint8).numpy()


def oracle_block(A, B, As, Bs, rows, cols):
    """Oracle C[rows][:, cols] from fp8 A [M,K], B [N,K] and fp32 As [M,K/128], Bs [N/128,K/128]."""
    r = torch.as_tensor(rows, device=A.device)
    c = torch.as_tensor(cols, device=B.device)
    a = ob.dequant_a(_u8(A.index_select(0, r)), As.index_select(0, r).float().cpu().numpy())
    cb = torch.as_tensor(np.asarray(cols) // 128, device=Bs.device)
    b = ob.dequant_a(_u8(B.index_select(0, c)), Bs.index_select(0, cb).float().cpu().numpy())
    return a @ b.T


PIN_TOL = 1e-4     # two fp32 sums of the same terms in different orders


def pin(ref, A, B, As, Bs, what=""):
    """Check a full fp32 reference C (numpy array or torch tensor) against the
    oracle on the sampled block: NaN at the same places, elsewhere within
    PIN_TOL of the block's largest magnitude."""
    m, n = ref.shape
    rows, cols = spread(m, ROWS), spread(n, COLS)
    if isinstance(ref, torch.Tensor):
        blk = ref.index_select(0, torch.as_tensor(rows, device=ref.device))
        blk = blk.index_select(1, torch.as_tensor(cols, device=ref.device)).double().cpu().numpy()
    else:
        blk = np.asarray(ref)[rows][:, cols].astype(np.float64)
    with np.errstate(invalid="ignore"):
        want = oracle_block(A, B, As, Bs, rows, cols).astype(np.float64)
    nan = np.isnan(want)
    assert np.array_equal(nan, np.isnan(blk)), ("NaN places", what)
    if nan.all():
        return 0.0
    den = float(np.abs(want[~nan]).max())
    diff = float(np.abs(blk[~nan] - want[~nan]).max())
    assert diff <= PIN_TOL * den or diff == 0.0, (what, diff, den)
    return diff / den if den else 0.0
