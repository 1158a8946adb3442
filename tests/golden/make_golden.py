"""Regenerate the golden GEMM fixtures: `python tests/golden/make_golden.py`.

Inputs come from the package's seeded recipe (fp8_gemm_h20.quant.sample,
CPU torch.Generator) quantised by the oracle's numpy quantiser; expected
outputs are the float64 dequant-matmul of the quantised operands (exact
products, float64 sums), stored rounded to float32 plus the bf16 bits
of that value.  The float64 value pins both the fp32 oracle and the GPU kernel
within their tolerances.
"""
import hashlib
import json
import sys
from pathlib import Path

import numpy as np

HERE = Path(__file__).resolve().parent
ROOT = HERE.parents[1]
sys.path.insert(0, str(ROOT))

from fp8_gemm_h20 import quant  # noqa: E402
from oracle import blockfp8 as ob  # noqa: E402

CASES = [
    # (M, N, K, mode, seed)
    (1, 128, 128, "normal", 1),
    (3, 256, 256, "normal", 2),
    (5, 128, 256, "zero", 3),
    (17, 384, 512, "outlier_rows", 4),
    (37, 256, 1152, "normal", 5),
    (64, 512, 384, "skew", 6),
    (100, 256, 640, "outlier_cols", 7),
    (130, 384, 768, "normal", 8),
]


def make_case(m, n, k, mode, seed):
    a, b = quant.sample(m, n, k, seed, mode)
    A, As = ob.quantize_act(a.numpy())
    B, Bs = ob.quantize_weight(b.numpy())
    c64 = ob.dequant_matmul(A, B, As, Bs, dtype=np.float64)
    return dict(A=A, B=B, As=As, Bs=Bs, C=c64.astype(np.float32), Cbf16=ob.bf16_bits(c64.astype(np.float32)))


def digest(*arrays):
    h = hashlib.sha256()
    for x in arrays:
        h.update(np.ascontiguousarray(x).tobytes())
    return h.hexdigest()


def main():
    out = {}
    index = []
    for i, (m, n, k, mode, seed) in enumerate(CASES):
        c = make_case(m, n, k, mode, seed)
        for key, v in c.items():
            out[f"c{i}_{key}"] = v
        index.append(dict(case=i, M=m, N=n, K=k, mode=mode, seed=seed,
                          inputs_sha256=digest(c["A"], c["B"], c["As"], c["Bs"])))
    np.savez_compressed(HERE / "gemm_cases.npz", **out)
    # config 0: too large to store; keep input digests
    # and float64 output statistics.
    m, n, k = 200, 3072, 2048
    a, b = quant.sample(m, n, k, m + n + k + 113, "normal")
    A, As = ob.quantize_act(a.numpy())
    B, Bs = ob.quantize_weight(b.numpy())
    c64 = ob.dequant_matmul(A, B, As, Bs, dtype=np.float64)
    rs = np.random.RandomState(0)
    idx = [(int(rs.randint(m)), int(rs.randint(n))) for _ in range(64)]
    cfg0 = dict(M=m, N=n, K=k, seed=m + n + k + 113, mode="normal",
                inputs_sha256=digest(A, B, As, Bs),
                c_absmax=float(np.abs(c64).max()), c_sum=float(c64.sum()),
                c_abs_sum=float(np.abs(c64).sum()),
                samples=[[i, j, float(c64[i, j])] for i, j in idx])
    (HERE / "gemm_cases.json").write_text(json.dumps(dict(cases=index, config0=cfg0), indent=1) + "\n")
    print("wrote", HERE / "gemm_cases.npz", HERE / "gemm_cases.json")


if __name__ == "__main__":
    main()
