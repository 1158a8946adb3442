"""bench.py's command-line contract and host-side arithmetic, without a GPU."""
import json
import subprocess
import sys
from pathlib import Path

import pytest

ROOT = Path(__file__).resolve().parents[1]
sys.path.insert(0, str(ROOT))
import bench  # noqa: E402


def test_more_than_one_gpu_exits_with_a_message():
    r = subprocess.run([sys.executable, str(ROOT / "bench.py"), "--gpus", "2", "--steps", "1"],
                       capture_output=True, text=True, timeout=120)
    assert r.returncode != 0
    assert "one GPU" in (r.stderr + r.stdout) or "1 GPU" in (r.stderr + r.stdout)


def test_algorithmic_counts():
    # algorithmic units: flops 2MNK; bytes A + B + As + Bs + C (bf16)
    m, n, k = 200, 3072, 2048
    assert bench.flops(m, n, k) == 2 * m * n * k
    assert bench.algo_bytes(m, n, k) == m * k + n * k + 4 * m * (k // 128) + 4 * (n // 128) * (k // 128) + 2 * m * n


def test_traffic_record_matches_the_packaged_table():
    # the committed HBM measurement is reported only for the kernel and config
    # the table selects; the packaged table and the record must agree
    rec = json.loads((ROOT / "profiles" / "hbm_traffic.json").read_text())
    for key, r in rec.items():
        if key.startswith("_"):
            continue
        m, n, k = (int(x) for x in key.split(","))
        assert bench.measured_traffic(m, n, k, "35b_tp1") == r["bytes"]
        assert (ROOT / r["summary"]).exists()


@pytest.mark.parametrize("workload", sorted(bench.WORKLOADS))
def test_workload_grids_are_covered_by_their_profiles(workload):
    from fp8_gemm_h20 import supports
    nks, ms = bench.WORKLOADS[workload]
    for n, k in nks:
        for m in ms:
            assert supports(workload, m, n, k), (workload, m, n, k)


def test_kernel_names_follow_the_built_kernels():
    # bench.kernel_name names fp8bg_ring_dp for unsplit ring entries exactly
    # where the library builds one (the launcher then runs it)
    import re
    import shutil
    import subprocess
    from fp8_gemm_h20 import _lib, kernels
    if shutil.which("nm") is None or not _lib.LIB_PATH.exists():
        pytest.skip("nm or the built library is not available")
    syms = subprocess.run(["nm", "-C", str(_lib.LIB_PATH)], capture_output=True, text=True).stdout
    built = {tuple(int(v) for v in m.split(", "))
             for m in re.findall(r"fp8bg_ring_dp<([0-9, ]+)>\(", syms)}
    named = set()
    for tw, tt, ww, wt, st, kf, ku, wk in kernels.RING:
        cfg = dict(BLOCK_W=tw, BLOCK_T=tt, WAVES_W=ww, WAVES_T=wt, STAGES=st, K_FIXED=kf,
                   K_UNROLL=ku, WAVES_K=wk)
        if bench.kernel_name({"impl": "ring", "config": cfg}).startswith("fp8bg_ring_dp<"):
            named.add((tw, tt, ww, wt, st, kf, ku, wk))
    assert built and built == named
