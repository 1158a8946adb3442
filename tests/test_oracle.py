"""Pin the CPU oracle (oracle/blockfp8.py) before trusting it as the checker.

Each oracle function is checked against something other than itself:
library routines (torch's float8_e4m3fn / bfloat16 casts), the OCP e4m3
definition, a float64 brute-force loop, closed forms and exact invariants.
"""
import json

import numpy as np
import pytest
import torch

from oracle import blockfp8 as ob
from fp8_gemm_h20 import quant


# ---------------------------------------------------------------- e4m3 / bf16
def test_e4m3_decode_matches_torch_for_all_codes():
    codes = np.arange(256, dtype=np.uint8)
    ref = torch.from_numpy(codes).view(torch.float8_e4m3fn).float().numpy()
    got = ob.e4m3_decode(codes)
    assert np.array_equal(np.isnan(ref), np.isnan(got))
    ok = ~np.isnan(ref)
    assert np.array_equal(ref[ok], got[ok])


def test_e4m3_ocp_special_values():
    d = ob.e4m3_decode(np.array([0x7E, 0x08, 0x01, 0x07, 0x38, 0x80, 0xFE], np.uint8))
    assert d[0] == 448.0                 # max normal S.1111.110
    assert d[1] == 2.0 ** -6             # min normal
    assert d[2] == 2.0 ** -9             # min subnormal
    assert d[3] == 7 * 2.0 ** -9         # max subnormal
    assert d[4] == 1.0                   # exponent bias 7
    assert d[5] == 0.0 and np.signbit(d[5])
    assert d[6] == -448.0
    assert np.isnan(ob.e4m3_decode(np.array([0x7F, 0xFF], np.uint8))).all()
    # 126 distinct positive finite magnitudes + zero: no infinities in "fn"
    pos = ob.e4m3_decode(np.arange(0x7F, dtype=np.uint8))
    assert np.isfinite(pos).all() and len(np.unique(pos)) == 127


def test_e4m3_encode_matches_torch_on_dense_sweep_and_ties():
    d = ob.e4m3_decode(np.arange(256, dtype=np.uint8))
    d = d[~np.isnan(d)]
    mids = (np.sort(d)[1:] + np.sort(d)[:-1]) / 2          # exact ties between neighbours
    x = np.concatenate([
        np.linspace(-500, 500, 100001, dtype=np.float32),
        (np.random.RandomState(0).randn(50000) * 30).astype(np.float32),
        d, mids.astype(np.float32),
        np.nextafter(mids.astype(np.float32), np.float32(np.inf)),
        np.nextafter(mids.astype(np.float32), np.float32(-np.inf)),
        np.float32([464, 465, 463.99, 480, 1e6, -464, 2 ** -10, 3 * 2 ** -11, 2 ** -11, -0.0, 0.0,
                    np.inf, -np.inf, 3.4e38, -3.4e38]),
    ]).astype(np.float32)
    ref = torch.from_numpy(x).to(torch.float8_e4m3fn).view(torch.uint8).numpy()
    assert np.array_equal(ob.e4m3_encode(x), ref)


def test_e4m3_roundtrip_is_identity_on_codes():
    codes = np.array([c for c in range(256) if c not in (0x7F, 0xFF)], np.uint8)
    assert np.array_equal(ob.e4m3_encode(ob.e4m3_decode(codes)), codes)


def test_bf16_rounding_matches_torch():
    rs = np.random.RandomState(1)
    x = np.concatenate([
        (rs.randn(200000) * 1000).astype(np.float32),
        # exact ties: low 16 bits == 0x8000 with both parities of bit 16
        (rs.randint(0, 1 << 15, 1000).astype(np.uint32) << 17 | 0x8000).view(np.float32),
        (rs.randint(0, 1 << 15, 1000).astype(np.uint32) << 17 | 0x18000).view(np.float32),
        np.float32([np.inf, -np.inf, 3.3895314e38, -0.0, 1e-40]),
    ]).astype(np.float32)
    x = x[np.isfinite(x) | np.isinf(x)]
    ref = torch.from_numpy(x).to(torch.bfloat16).view(torch.int16).numpy().view(np.uint16)
    assert np.array_equal(ob.bf16_bits(x), ref)
    assert ob.bf16_bits(np.float32([np.nan]))[0] == 0x7FC0


# ---------------------------------------------------------------- GEMM math
def _rand_case(m, n, k, seed, mode="normal"):
    a, b = quant.sample(m, n, k, seed, mode)
    A, As = ob.quantize_act(a.numpy())
    B, Bs = ob.quantize_weight(b.numpy())
    return A, B, As, Bs


@pytest.mark.parametrize("m,n,k", [(1, 128, 128), (3, 256, 128), (2, 128, 256)])
def test_dequant_matmul_matches_brute_force(m, n, k):
    A, B, As, Bs = _rand_case(m, n, k, seed=m * 7 + n + k)
    ref = ob.brute_force(A, B, As, Bs)
    got = ob.dequant_matmul(A, B, As, Bs)
    assert np.abs(got - ref).max() <= 1e-5 * np.abs(ref).max()


def test_one_hot_weights_select_dequantised_activations():
    # B row n = e4m3(1.0) at column k_n, zero elsewhere; Bs = 1 -> C[:, n] = dequant(A)[:, k_n]
    m, n, k = 5, 256, 384
    A, _, As, _ = _rand_case(m, n, k, seed=11)
    cols = np.random.RandomState(3).randint(0, k, n)
    B = np.zeros((n, k), np.uint8)
    B[np.arange(n), cols] = 0x38
    Bs = np.ones((n // 128, k // 128), np.float32)
    C = ob.dequant_matmul(A, B, As, Bs)
    want = ob.dequant_a(A, As)[:, cols]
    assert np.array_equal(C, want)


def test_zero_activations_give_zero():
    A, B, As, Bs = _rand_case(4, 256, 256, seed=5, mode="zero")
    assert not A.any()
    assert not ob.dequant_matmul(A, B, As, Bs).any()


def test_power_of_two_scale_linearity_is_exact():
    # Doubling As[m, g] doubles only row m's group-g contribution; scaling a
    # whole As row or a Bs block-row by 2 scales the output exactly.
    A, B, As, Bs = _rand_case(6, 384, 512, seed=9)
    C = ob.dequant_matmul(A, B, As, Bs)
    As2 = As.copy()
    As2[2] *= 2
    C2 = ob.dequant_matmul(A, B, As2, Bs)
    assert np.array_equal(C2[2], 2 * C[2])
    assert np.array_equal(np.delete(C2, 2, 0), np.delete(C, 2, 0))
    Bs2 = Bs.copy()
    Bs2[1] *= 0.5
    C3 = ob.dequant_matmul(A, B, As, Bs2)
    assert np.array_equal(C3[:, 128:256], 0.5 * C[:, 128:256])
    assert np.array_equal(C3[:, :128], C[:, :128]) and np.array_equal(C3[:, 256:], C[:, 256:])


def test_group_scale_applies_to_its_own_k_group_only():
    # Zero out As[:, 1] -> equals the GEMM with K-group 1 of A zeroed.
    A, B, As, Bs = _rand_case(3, 128, 384, seed=21)
    As0 = As.copy()
    As0[:, 1] = 0
    A0 = A.copy()
    A0[:, 128:256] = 0
    C = ob.dequant_matmul(A, B, As0, Bs)
    Cb = ob.brute_force(A0, B, As, Bs)
    assert np.abs(C - Cb).max() <= 1e-5 * np.abs(Cb).max()


def test_row_independence():
    A, B, As, Bs = _rand_case(8, 256, 256, seed=13)
    C = ob.dequant_matmul(A, B, As, Bs)
    C5 = ob.dequant_matmul(A[5:6], B, As[5:6], Bs)
    assert np.allclose(C5[0], C[5], rtol=0, atol=1e-6 * np.abs(C).max())


def test_sampled_oracle_block_equals_the_full_product_there():
    # the GPU tests check a sampled block of a product too large for the
    # oracle; the block's weight rows take their own block scales
    from tests import oracle_sample as osm
    A, B, As, Bs = _rand_case(300, 640, 256, seed=21)
    rows, cols = osm.spread(300, 40), osm.spread(640, 48)
    t = lambda x: torch.from_numpy(np.ascontiguousarray(x))
    got = osm.oracle_block(t(A).view(torch.float8_e4m3fn), t(B).view(torch.float8_e4m3fn), t(As), t(Bs),
                           rows, cols)
    full = ob.dequant_matmul(A, B, As, Bs)[rows][:, cols]
    assert np.abs(got - full).max() <= 1e-6 * np.abs(full).max()
    # operands bitwise: the per-row-group dequantiser with Bs[col // 128]
    # is the block dequantiser on those rows
    assert np.array_equal(ob.dequant_a(B[cols], Bs[cols // 128]), ob.dequant_b(B, Bs)[cols])
    # a wrong block scale index (col // 64) is caught
    assert not np.array_equal(ob.dequant_a(B[cols], Bs[np.minimum(cols // 64, len(Bs) - 1)]),
                              ob.dequant_b(B, Bs)[cols])


def test_sample_spread_covers_every_tile():
    from tests import oracle_sample as osm
    for n in (1, 16, 80, 85, 777, 4097, 16384):
        s = osm.spread(n, osm.ROWS)
        assert s[0] == 0 and s[-1] == n - 1 and np.all(np.diff(s) > 0)
        assert len(s) == min(n, osm.ROWS) or (n > osm.ROWS and len(s) <= osm.ROWS)
        assert set(range(min(n, 8))) <= set(s.tolist())
        assert len(set((s // 256).tolist())) == (n + 255) // 256
    for n in (512, 2048, 12288):
        c = osm.spread(n, osm.COLS)
        assert len(set((c // 128).tolist())) == n // 128


def test_nonsquare_shapes_reject_transposed_operand():
    # A wrong orientation (B instead of B^T, or scale index n//128 vs n) cannot
    # satisfy brute force on a non-square, multi-block case.
    A, B, As, Bs = _rand_case(2, 256, 384, seed=17, mode="skew")
    ref = ob.brute_force(A, B, As, Bs)
    got = ob.dequant_matmul(A, B, As, Bs)
    assert got.shape == (2, 256)
    assert np.abs(got - ref).max() <= 1e-5 * np.abs(ref).max()
    wrong = ob.dequant_matmul(A, B, As, Bs[::-1].copy())
    assert np.abs(wrong - ref).max() > 1e-2 * np.abs(ref).max()


def test_error_and_cosine_metrics():
    ref = np.array([[1.0, -2.0], [4.0, 0.5]])
    out = ref + np.array([[0.0, 0.04], [0.0, 0.0]])
    assert ob.error(out, ref) == pytest.approx(0.01)
    assert ob.error(np.zeros(3), np.zeros(3)) == 0.0
    assert ob.cosine(ref, ref) == pytest.approx(1.0)
    assert ob.cosine(ref, -ref) == pytest.approx(-1.0)


# ---------------------------------------------------------------- quantisation recipe
@pytest.mark.parametrize("mode", quant.MODES)
def test_torch_quantisers_match_numpy_restatement(mode):
    m, n, k = 33, 256, 384
    a, b = quant.sample(m, n, k, seed=123, mode=mode)
    A, As = quant.quantize_per_token_group(a)
    B, Bs = quant.quantize_per_block(b)
    nA, nAs = ob.quantize_act(a.numpy())
    nB, nBs = ob.quantize_weight(b.numpy())
    assert np.array_equal(A.view(torch.uint8).numpy(), nA)
    assert np.array_equal(B.view(torch.uint8).numpy(), nB)
    assert np.array_equal(As.numpy(), nAs) and np.array_equal(Bs.numpy(), nBs)
    # amax/448 recipe: every group's largest code is +-448 unless the group is zero
    dA = ob.e4m3_decode(nA).reshape(m, k // 128, 128)
    big = np.abs(dA).max(-1)
    assert np.all((big == 448.0) | (big == 0.0))


def test_outlier_rows_recipe():
    m, k = 200, 256
    a, _ = quant.sample(m, 128, k, seed=7, mode="outlier_rows")
    base, _ = quant.sample(m, 128, k, seed=7, mode="normal")
    ratio = (a / base.where(base != 0, torch.ones_like(base))).abs()
    scaled = ((ratio - 50).abs() < 1e-3).all(dim=1)
    assert int(scaled.sum()) == 2                   # max(1, round(0.01*200))


# ---------------------------------------------------------------- golden fixtures
def test_golden_fixtures_reproduce(golden_dir):
    meta = json.loads((golden_dir / "gemm_cases.json").read_text())
    data = np.load(golden_dir / "gemm_cases.npz")
    from tests.golden.make_golden import digest
    for case in meta["cases"]:
        i = case["case"]
        A, B, As, Bs = (data[f"c{i}_{x}"] for x in ("A", "B", "As", "Bs"))
        # the recipe still produces the stored inputs
        a, b = quant.sample(case["M"], case["N"], case["K"], case["seed"], case["mode"])
        qa, sa = quant.quantize_per_token_group(a)
        qb, sb = quant.quantize_per_block(b)
        assert digest(qa.view(torch.uint8).numpy(), qb.view(torch.uint8).numpy(),
                      sa.numpy(), sb.numpy()) == case["inputs_sha256"]
        # the fp32 oracle agrees with the stored float64 result
        ref = data[f"c{i}_C"].astype(np.float64)
        got = ob.dequant_matmul(A, B, As, Bs)
        scale = max(np.abs(ref).max(), 1e-30)
        assert np.abs(got - ref).max() <= 1e-5 * scale
        if case["mode"] == "zero":
            assert not data[f"c{i}_Cbf16"].any()


def test_config0_fixture_reproduces(golden_dir):
    cfg = json.loads((golden_dir / "gemm_cases.json").read_text())["config0"]
    from tests.golden.make_golden import digest
    a, b = quant.sample(cfg["M"], cfg["N"], cfg["K"], cfg["seed"], cfg["mode"])
    A, As = ob.quantize_act(a.numpy())
    B, Bs = ob.quantize_weight(b.numpy())
    assert digest(A, B, As, Bs) == cfg["inputs_sha256"]
    C = ob.dequant_matmul(A, B, As, Bs)
    assert abs(np.abs(C).max() - cfg["c_absmax"]) <= 1e-5 * cfg["c_absmax"]
    for i, j, v in cfg["samples"]:
        assert abs(C[i, j] - v) <= 1e-5 * cfg["c_absmax"]


def test_reciprocal_quantiser_differs_from_division_only_at_rounding_boundaries():
    # The fused GEMM's recipe e4m3(x * (1/s)) against quantize_act's e4m3(x / s):
    # identical scales; codes equal except where the two fp32 quotients fall on
    # opposite sides of an e4m3 rounding boundary, and then one step apart.
    rng = np.random.default_rng(11)
    x = (rng.standard_normal((64, 4096)) * 3).astype(np.float32)
    q1, s1 = ob.quantize_act(x, eps=1e-10)
    q2, s2 = ob.quantize_act_reciprocal(x, eps=1e-10)
    assert np.array_equal(s1, s2)
    d = q1 != q2
    assert d.mean() < 2e-3
    v1 = ob.e4m3_decode(q1[d]).astype(np.float64)
    v2 = ob.e4m3_decode(q2[d]).astype(np.float64)
    codes = np.sort(ob.e4m3_decode(np.arange(256, dtype=np.uint8))[~np.isnan(ob.e4m3_decode(np.arange(256, dtype=np.uint8)))])
    i1 = np.searchsorted(codes, v1)
    i2 = np.searchsorted(codes, v2)
    assert np.all(np.abs(i1 - i2) == 1)
    # a power-of-two scale makes both quotients exact: every code comes back
    vals = ob.e4m3_decode(np.arange(0, 127, dtype=np.uint8)).astype(np.float32)   # 0 .. 448
    row = np.concatenate([vals, -vals[1:2]]) * np.float32(2.0 ** -3)             # amax 56: s = 1/8
    q1, s1 = ob.quantize_act(row[None, :], eps=1e-10)
    q2, s2 = ob.quantize_act_reciprocal(row[None, :], eps=1e-10)
    assert s1[0, 0] == s2[0, 0] == np.float32(0.125)
    assert np.array_equal(q1, q2) and np.array_equal(q1[0, :127], np.arange(0, 127, dtype=np.uint8))


def test_torch_cpu_baseline_matches_the_numpy_oracle():
    # the bench's CPU baseline (torch restatement of validate.py:32-34 plus the
    # bf16 cast) equals the numpy oracle up to fp32 summation order, and a
    # transposed weight operand fails the same check
    import torch
    from fp8_gemm_h20 import quant
    from oracle import torch_cpu
    for m, n, k in [(1, 256, 128), (37, 384, 512), (200, 512, 1024)]:
        A, B, As, Bs = quant.make_inputs(m, n, k, device="cpu")
        got = torch_cpu.dequant_matmul_bf16(A, B, As, Bs)
        assert got.dtype == torch.bfloat16 and got.shape == (m, n)
        ref = ob.dequant_matmul(A.view(torch.uint8).numpy(), B.view(torch.uint8).numpy(),
                                As.numpy(), Bs.numpy())
        assert ob.error(got.float().numpy(), ref) <= 2 ** -8
        assert ob.cosine(got.float().numpy(), ref) > 0.99999
    A, B, As, Bs = quant.make_inputs(64, 256, 256, device="cpu")
    bad = torch_cpu.dequant_matmul_bf16(A, B.view(2, 128, 2, 128).transpose(1, 3).reshape(256, 256)
                                        .contiguous(), As, Bs)
    ref = ob.dequant_matmul(A.view(torch.uint8).numpy(), B.view(torch.uint8).numpy(), As.numpy(), Bs.numpy())
    assert ob.error(bad.float().numpy(), ref) > 0.1
