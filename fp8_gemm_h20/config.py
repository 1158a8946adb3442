"""CPU-only profile loading, schema validation and deterministic M -> entry selection.

Same public functions and behaviour as the reference's fp8_gemm_h20/config.py:
available_profiles, token_tile, validate_config, get_profile, supports, select
(config.py:13-105, policy prose in docs/configuration.md:26-38).  No torch,
no GPU: only json/math/copy/functools.

Differences, all additive:
* Packaged tables (configs/*.json) are gfx950 tables whose entries use the
  native impls "tiled"/"skinny"/"shortk".  Their tile rule is widened: a
  native entry must name a kernel instance compiled into libfp8bg.so (e.g. a
  256-row tiled tile spans two 128-row weight-scale blocks).  Entries with
  the reference's impl names keep the reference's rule (BLOCK_W divides 128,
  power-of-two token tile), so the reference's own H20 tables validate and
  route unchanged.
* `select_in(data, M, N, K)` / `supports_in(...)` apply the policy to any
  validated table dict, e.g. a table loaded with `load_profile(path)`.
* An optional `fused_entries` section ({"N,K": {"M": entry}}, M the decode
  anchors) names, per anchor, the skinny configuration of the fused
  quantiser + GEMM launch that `linear()` takes for bf16 activations, with
  its measured time ("anchor_us"), the two-kernel time ("two_kernel_us") and
  whether the fused launch is used by default ("use").  `select_fused`
  routes M to the log-nearest anchor, or to no fused entry above the largest.
"""
import copy
import json
import math
from functools import lru_cache
from pathlib import Path

from .engine import KERNELS, NATIVE

_CONFIG_DIR = Path(__file__).with_name("configs")
_PROFILES = ("35b_tp1", "122b_tp4")
_POLICIES = ("log_nearest", "nearby_equal_tiles")
_SPLIT_MODES = ("none", "tail", "full")     # ring and tiled ("last": skinny, small-token ring)


def available_profiles():
    return _PROFILES


def token_tile(entry):
    """Token (M) tile of an entry, whatever the impl's key spelling (config.py:19-21)."""
    c = entry["config"]
    for key in ("BLOCK_T", "BLOCK_SIZE_M", "BM", "BT"):
        if key in c:
            return c[key]
    return None


def weight_tile(entry):
    c = entry["config"]
    for key in ("BLOCK_W", "BLOCK_SIZE_N", "BN"):
        if key in c:
            return c[key]
    return None


def _native_ok(impl, c, k):
    """A gfx950-native entry names a compiled kernel instance."""
    from .kernels import TILED, SKINNY_TILES, RING, RING_SK
    tw, tt = c.get("BLOCK_W"), c.get("BLOCK_T")
    if c.get("LDS_SWIZZLE", "row16") not in ("row8", "row16", "pair"):
        return False
    if impl == "ring":
        c = {key: v for key, v in c.items() if key not in ("M_SPLIT", "TAIL")}
        kf = c.get("K_FIXED", 0)
        ku = c.get("K_UNROLL", 1)
        split = c.get("SPLIT", 1) if c.get("SPLIT_MODE", "none") != "none" else 1
        inst = (tw, tt, c.get("WAVES_W"), c.get("WAVES_T"), c.get("STAGES"), kf, ku, c.get("WAVES_K", 1))
        # SPLIT_MODE "last": the instances with the in-kernel reduction
        # (RING_LAST); "stream": those with a stream-K kernel (RING_SK)
        modes = _SPLIT_MODES + (("last",) if tt is not None and tt <= 64 and kf == 0 else ()) + \
            (("stream",) if inst in RING_SK else ())
        return (c.get("SPLIT_MODE", "none") in modes and (kf == 0 or k == 256 * kf // 2) and
                inst in RING and
                (k // 128 // (split if (k // 128) % split == 0 else 1)) % ku == 0)
    if impl == "skinny":
        mode = c.get("SPLIT_MODE", "none")
        return (mode in ("none", "full", "last") and
                (tw, tt, c.get("WAVES_K", 8), c.get("UNROLL", 1)) in SKINNY_TILES)
    kf = 2 if impl == "shortk" else 0
    if c.get("SPLIT_MODE", "full") not in _SPLIT_MODES:
        return False
    waves = (c.get("WAVES_W"), c.get("WAVES_T"))
    if waves == (None, None):
        return any((w, t, f) == (tw, tt, kf) for w, t, _, _, f in TILED)
    return (tw, tt, waves[0], waves[1], kf) in TILED


def _check_entry(field, nk, k, m, entry, policy):
    where = f"{nk}/{m}"
    if not 1 <= int(m) <= 16384 or entry.get("impl") not in KERNELS:
        raise ValueError(f"Invalid entry: {where}")
    c = entry["config"]
    bt, bw = token_tile(entry), weight_tile(entry)
    if entry["impl"] in NATIVE and "BLOCK_W" in c:
        if not _native_ok(entry["impl"], c, k):
            raise ValueError(f"Invalid tile: {where}")
    elif not bt or bt & (bt - 1) or not bw or 128 % bw:
        raise ValueError(f"Invalid tile: {where}")
    if c.get("SPLIT", c.get("SPLIT_K", 1)) < 1:
        raise ValueError(f"Invalid split-K: {where}")
    if "M_SPLIT" in c or "TAIL" in c:
        # gfx950 ring entry whose last rows run on a second configuration
        tail = c.get("TAIL")
        m1 = c.get("M_SPLIT")
        if (entry["impl"] != "ring" or not isinstance(m1, int) or m1 < 1 or m1 % c["BLOCK_T"]
                or not isinstance(tail, dict) or tail.get("impl") not in NATIVE
                or "M_SPLIT" in tail.get("config", {})
                or not _native_ok(tail["impl"], tail.get("config", {}), k)):
            raise ValueError(f"Invalid row split: {where}")
    if entry["impl"] == "shortk" and k != 256:
        raise ValueError("shortk requires K=256")
    if c.get("MODE") == 3 and (c["NUM_STAGES"] < 4 or (k // 128) % (4 * c.get("SPLIT", 1))):
        raise ValueError("MODE=3 needs complete groups of four K tiles")
    if field == "entries" and policy["kind"] == "nearby_equal_tiles":
        us = entry.get("anchor_us")
        if not isinstance(us, (int, float)) or not math.isfinite(us) or us <= 0:
            raise ValueError("Measured anchor latency must be positive")


def validate_config(data):
    """Raise ValueError unless `data` is a well-formed schema-v1 profile (config.py:23-59)."""
    if data.get("schema_version") != 1 or data.get("block_size") != [128, 128]:
        raise ValueError("Unsupported schema or quantization block size")
    if data.get("m_range") != [1, 16384]:
        raise ValueError("Profiles must declare the validated M=1..16384 range")
    shapes = {f"{s['N']},{s['K']}" for s in data["shapes"]}
    if set(data["entries"]) != shapes:
        raise ValueError("Shape inventory and dispatch entries disagree")
    policy = data["policy"]
    if policy.get("kind") not in _POLICIES:
        raise ValueError("Unsupported dispatch policy")
    if policy["kind"] == "nearby_equal_tiles":
        if policy["max_distance"] < 0 or set(data.get("fallback_entries", {})) != shapes:
            raise ValueError("Incomplete bounded interpolation/fallback policy")
    for field in ("entries", "fallback_entries"):
        for nk, table in data.get(field, {}).items():
            n, k = (int(x) for x in nk.split(","))
            if n % 128 or k % 128 or not table:
                raise ValueError(f"Invalid shape/table: {nk}")
            for m, entry in table.items():
                _check_entry(field, nk, k, m, entry, policy)
    for nk, table in data.get("fused_entries", {}).items():
        if nk not in shapes or not table:
            raise ValueError(f"Invalid fused shape/table: {nk}")
        for m, entry in table.items():
            _check_fused_entry(nk, m, entry)


def _check_fused_entry(nk, m, entry):
    from .kernels import SKINNY_QA
    where = f"fused {nk}/{m}"
    if not 1 <= int(m) <= 16384 or entry.get("impl") != "skinny" or not isinstance(entry.get("use"), bool):
        raise ValueError(f"Invalid entry: {where}")
    c = entry.get("config", {})
    try:
        inst = (c["BLOCK_W"] // 16, c["BLOCK_T"] // 16, c.get("WAVES_K", 8), c.get("UNROLL", 1))
    except (KeyError, TypeError):
        raise ValueError(f"Invalid tile: {where}") from None
    if (c["BLOCK_W"] % 16 or c["BLOCK_T"] % 16 or inst not in SKINNY_QA
            or c.get("SPLIT_MODE", "none") not in ("none", "full", "last") or c.get("SPLIT", 1) < 1):
        raise ValueError(f"Invalid tile: {where}")
    for key in ("anchor_us", "two_kernel_us"):
        us = entry.get(key)
        if not isinstance(us, (int, float)) or not math.isfinite(us) or us <= 0:
            raise ValueError(f"Measured latency must be positive: {where}")


def load_profile(path):
    """Read and validate a profile JSON from any path."""
    data = json.loads(Path(path).read_text())
    validate_config(data)
    return data


@lru_cache(maxsize=None)
def _profile(name):
    if name not in _PROFILES:
        raise ValueError(f"Unknown profile {name!r}; choose one of {_PROFILES}")
    return load_profile(_CONFIG_DIR / f"{name}.json")


def get_profile(name):
    return copy.deepcopy(_profile(name))


def supports_in(data, m, n, k):
    lo, hi = data["m_range"]
    return lo <= m <= hi and f"{n},{k}" in data["entries"]


def supports(profile, m, n, k):
    return supports_in(_profile(profile), m, n, k)


def _log_nearest(table, m):
    # First minimum in JSON insertion order wins ties (config.py:100).
    return min(table, key=lambda a: abs(math.log(int(a) / m)))


def _split_fits(entry, m, anchor):
    """Whether a row-split entry (gfx950 extension: rows [M_SPLIT, M) run on
    TAIL) is used at M: its TAIL was chosen for the anchor's tail rows, so it
    takes tails up to that many rows rounded up to its own token tile; past
    that (M routed from far off the anchor), the entry runs whole on its own
    tile, as a fallback entry does."""
    c = entry["config"]
    tt = token_tile(c["TAIL"])
    return m - c["M_SPLIT"] <= -(-(anchor - c["M_SPLIT"]) // tt) * tt


def _routed(entry, m, anchor):
    """The entry as it runs at M when routed from `anchor`.  Two gfx950
    structures are fitted to the anchor's own tile count and run only where
    they still fit, elsewhere the entry's plain tile runs: a row split
    (_split_fits), and a tail split of the last, partial wave of tiles
    (SPLIT_MODE "tail"), kept only at M with the anchor's number of token-tile
    rows (routed further, its leftover tiles and their split-K workspace grow
    with M)."""
    c = entry["config"]
    if "M_SPLIT" in c and not _split_fits(entry, m, anchor):
        return dict(entry, config={key: v for key, v in c.items() if key not in ("M_SPLIT", "TAIL")})
    if (entry["impl"] in NATIVE and c.get("SPLIT_MODE") == "tail" and c.get("SPLIT", 1) > 1
            and -(-m // c["BLOCK_T"]) != -(-anchor // c["BLOCK_T"])):
        return dict(entry, config={key: v for key, v in c.items() if key not in ("SPLIT", "SPLIT_MODE")})
    return entry


def select_in(data, m, n, k):
    """Policy of config.py:76-101 applied to a validated table dict.

    Returns (entry, {"method": ..., "anchor": int}), the table's own entry
    (not a copy) except where a row split or tail split fitted to the anchor
    does not fit M, which comes without it (_routed).
    """
    if not supports_in(data, m, n, k):
        raise ValueError(f"{data.get('profile', 'profile')} does not cover M,N,K={m},{n},{k}")
    nk = f"{n},{k}"
    table = data["entries"][nk]
    if str(m) in table:
        return table[str(m)], {"method": "exact", "anchor": m}
    policy = data["policy"]
    if policy["kind"] == "nearby_equal_tiles":
        best = None
        for a, entry in table.items():
            if entry["impl"] in policy["exact_only"]:
                continue
            anchor, bt = int(a), token_tile(entry)
            if abs(m - anchor) > policy["max_distance"]:
                continue
            if -(-m // bt) != -(-anchor // bt):
                continue
            rank = (entry["anchor_us"], abs(math.log(m / anchor)), anchor)
            if best is None or rank < best[0]:
                best = (rank, anchor, entry)
        if best is not None:
            return _routed(best[2], m, best[1]), {"method": "equal_tile_count", "anchor": best[1]}
        table = data["fallback_entries"][nk]
        method = "baseline_fallback"
    else:
        method = "log_nearest"
    anchor = _log_nearest(table, m)
    return _routed(table[anchor], m, int(anchor)), {"method": method, "anchor": int(anchor)}


def select_fused_in(data, m, n, k):
    """The fused-quantiser entry for (M, N, K): the log-nearest anchor of the
    shape's fused_entries, None above the largest anchor or where the
    profile has no fused table for the shape."""
    table = data.get("fused_entries", {}).get(f"{n},{k}")
    if not table or m > max(int(a) for a in table):
        return None
    return table[str(m)] if str(m) in table else table[_log_nearest(table, m)]


def _has_fused_table(profile, n, k):
    return f"{n},{k}" in _profile(profile).get("fused_entries", {})


@lru_cache(maxsize=4096)
def _select_fused(profile, m, n, k):
    return select_fused_in(_profile(profile), m, n, k)


def select_fused(profile, m, n, k):
    """Return a copy of the fused entry for (M, N, K), or None."""
    return copy.deepcopy(_select_fused(profile, m, n, k))


@lru_cache(maxsize=4096)
def _select(profile, m, n, k):
    return select_in(_profile(profile), m, n, k)


def select(profile, m, n, k):
    """Return a copy of the selected entry and its routing explanation."""
    return copy.deepcopy(_select(profile, m, n, k))
