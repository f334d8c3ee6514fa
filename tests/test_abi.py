"""The C-ABI library: it loads, exports every declared symbol, and its host-only
entry points (plans, workspace sizes, argument checks) behave. No GPU needed:
nothing here launches a kernel."""

from __future__ import annotations

import ctypes
import re
from pathlib import Path

import numpy as np
import pytest

ROOT = Path(__file__).resolve().parents[1]

from ssalaad_amd import _lib, _runtime  # noqa: E402


def _declared_symbols() -> set[str]:
    text = (ROOT / "include" / "ssalaad_amd.h").read_text()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return set(re.findall(r"\b(ssl_[a-z0-9_]+)\s*\(", text))


def test_library_exports_every_declared_symbol():
    lib = _lib.load()
    declared = _declared_symbols()
    assert declared, "no declarations parsed"
    assert declared == set(_lib.exported_symbols())
    for name in declared:
        assert getattr(lib, name) is not None


def test_library_is_built_for_gfx950_only():
    data = _lib.LIB_PATH.read_bytes()
    assert b"gfx950" in data
    for other in (b"gfx942", b"gfx90a", b"gfx1100"):
        assert other not in data


def test_single_hip_runtime_in_process():
    _lib.load()
    maps = Path("/proc/self/maps").read_text()
    paths = {ln.split()[-1] for ln in maps.splitlines() if "libamdhip64" in ln}
    assert len({Path(p).resolve() for p in paths}) <= 1


def test_version():
    assert _lib.load().ssl_version() == 1


# ------------------------------------------------------------------ plans --


def _plan(crow, rows=None, q=64, lr=0, target=0):
    table, n, s = _runtime.build_plan(np.asarray(crow, np.int32),
                                      None if rows is None else np.asarray(rows, np.int32),
                                      q, lr, target)
    return table, n, s


def test_plan_covers_every_unit_once():
    rng = np.random.default_rng(0)
    counts = rng.integers(0, 40, 50)
    crow = np.concatenate([[0], np.cumsum(counts)])
    lr = 8
    for target in (0, 64, 200, 1000):
        table, n, slots = _plan(crow, q=64, lr=lr, target=target)
        seen = {}
        for row, ub, ue, seq, nseq, slot, nblk, blk0 in table:
            assert nblk == counts[row] and blk0 == crow[row]
            assert 0 <= ub < ue <= nblk + lr
            seen.setdefault(row, []).append((seq, nseq, ub, ue, slot))
        assert sorted(seen) == list(range(50))  # every row has units (lr > 0)
        used_slots = set()
        for row, parts in seen.items():
            parts.sort()
            k = parts[0][1]
            assert [p[0] for p in parts] == list(range(k))
            assert parts[0][2] == 0 and parts[-1][3] == counts[row] + lr
            for a, b in zip(parts, parts[1:]):
                assert a[3] == b[2]  # consecutive, no gap or overlap
            if k > 1:
                base = parts[0][4]
                assert all(p[4] == base for p in parts)
                for j in range(k):
                    assert base + j not in used_slots
                    used_slots.add(base + j)
        assert len(used_slots) == slots


def test_plan_splits_long_rows_evenly():
    crow = [0, 4, 4 + 400, 404 + 10]
    table, n, slots = _plan(crow, q=64, lr=0, target=64 * 8)
    per_row = {}
    for row, ub, ue, *_ in table:
        per_row.setdefault(row, []).append(ue - ub)
    assert len(per_row[0]) == 1
    assert len(per_row[1]) == 50 and set(per_row[1]) == {8}
    assert len(per_row[2]) == 2
    assert 1 not in per_row or True


def test_plan_with_row_list_skips_unlisted_and_empty_rows():
    crow = [0, 3, 3, 7, 9]
    table, n, _ = _plan(crow, rows=[0, 1, 3], q=16)
    assert [int(r) for r in table[:, 0]] == [0, 3]


def test_plan_rejects_bad_structures():
    with pytest.raises(ValueError):
        _plan([1, 2, 3])
    with pytest.raises(ValueError):
        _plan([0, 5, 3])
    with pytest.raises(ValueError):
        _plan([0, 1, 2], rows=[1, 0])
    with pytest.raises(ValueError):
        _plan([0, 1, 2], rows=[2])


def test_plan_target_cost_policy():
    assert _runtime.plan_target_cost(10**6, 64, 2, M=65) == 0  # several token tiles: no split
    small = _runtime.plan_target_cost(100, 64, 2, M=1)
    assert small == 16384 // 128
    big = _runtime.plan_target_cost(5504 * 64 + 172 * 8 * 32, 64, 2, M=16)
    assert big == -(-(5504 * 64 + 172 * 8 * 32) // 512)


# ---------------------------------------------------- workspace / checks --


def test_workspace_sizes_are_aligned_and_monotone():
    lib = _lib.load()
    a = lib.ssl_slr_workspace_size(16, 172, 64, 256, 4096, 0, _lib.SSL_BF16)
    b = lib.ssl_slr_workspace_size(16, 172, 64, 256, 4096, 100, _lib.SSL_BF16)
    c = lib.ssl_slr_workspace_size(2048, 172, 64, 256, 4096, 0, _lib.SSL_BF16)
    assert a % 256 == 0 and b > a and c > a
    assert lib.ssl_slr_counter_bytes(16, 172, 256, 4096) <= a
    assert lib.ssl_bsr_addmm_counter_bytes(16, 172) % 256 == 0
    assert lib.ssl_bsr_addmm_workspace_size(16, 172, 64, 10) > lib.ssl_bsr_addmm_counter_bytes(16, 172)


def test_entry_points_reject_bad_arguments_before_any_launch():
    lib = _lib.load()
    # unsupported block shape
    rc = lib.ssl_bsr_addmm_inplace(1, 64, 1, 64, 1, 1, 1, 1, 0, 1, 64, 64, 1, 8, 8,
                                   _lib.SSL_BF16, None, 0, None)
    assert rc == _lib.SSL_ERR_UNSUPPORTED and b"square" in lib.ssl_last_error()
    # N inconsistent with NB·p
    rc = lib.ssl_bsr_addmm_inplace(1, 64, 1, 64, 1, 1, 1, 1, 0, 1, 60, 64, 1, 64, 64,
                                   _lib.SSL_BF16, None, 0, None)
    assert rc == _lib.SSL_ERR_INVALID
    # bad dtype
    rc = lib.ssl_slr_forward(1, 64, 1, 64, 1, 1, None, 1, 1, 1, 1, 0, 1, 64, 64, 1, 64, 64, 64,
                             7, None, 0, None)
    assert rc == _lib.SSL_ERR_UNSUPPORTED
    # r_pad not a multiple of 64
    rc = lib.ssl_slr_forward(1, 64, 1, 64, 1, 1, None, 1, 1, 1, 1, 0, 1, 64, 64, 1, 48, 64, 64,
                             _lib.SSL_BF16, None, 0, None)
    assert rc == _lib.SSL_ERR_INVALID
    # missing workspace
    rc = lib.ssl_slr_forward(16, 64, 16, 64, 16, 16, None, 16, 16, 16, 1, 0, 1, 64, 64, 1, 64, 64,
                             64, _lib.SSL_BF16, None, 0, None)
    assert rc == _lib.SSL_ERR_WORKSPACE
    with pytest.raises(ValueError):
        _lib.check(_lib.SSL_ERR_INVALID, "x")
    with pytest.raises(TypeError):
        _lib.check(_lib.SSL_ERR_UNSUPPORTED, "x")
    with pytest.raises(RuntimeError):
        _lib.check(_lib.SSL_ERR_HIP, "x")


def test_encoder_rejects_bad_arguments():
    lib = _lib.load()
    rc = lib.ssl_bsr_encode_count(1, 10, 2, 2, 16, 16, _lib.SSL_BF16, 1, 1, 1, 1, None)
    assert rc == _lib.SSL_ERR_INVALID  # lds < NBK·q
    rc = lib.ssl_bsr_encode_count(None, 32, 0, 2, 16, 16, 9, None, 1, None, 1, None)
    assert rc == _lib.SSL_ERR_UNSUPPORTED
