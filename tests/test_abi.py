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
    assert _lib.load().ssl_version() == 3


# ------------------------------------------------------------------ plans --


def _cols(crow):
    """Valid column indices for a structure whose columns do not matter."""
    return np.zeros(max(int(np.asarray(crow)[-1]), 0), np.int32)


def _plan(crow, rows=None, q=64, lr=0, target=0, col=None, NBK=1):
    col = _cols(crow) if col is None else np.asarray(col, np.int32)
    table, n, s = _runtime.build_plan(np.asarray(crow, np.int32), col, NBK,
                                      None if rows is None else np.asarray(rows, np.int32),
                                      q, lr, target)
    return table, n, s


def _check_plan(crow, lr, table, n, slots):
    """Every block and low-rank unit of every row is covered exactly once, chunks
    of a row share one slot base, and finalisers (chunks with low-rank units)
    come after every other chunk."""
    rows = {}
    for idx, (row, bb, be, lb, le, seq, nseq, slot) in enumerate(table):
        assert crow[row] <= bb <= be <= crow[row + 1]
        assert 0 <= lb <= le <= lr
        rows.setdefault(int(row), []).append((seq, nseq, bb, be, lb, le, slot, idx))
    used = set()
    last_plain = max([i for *_, lb, le, _s, i in
                      ((p[0], p[1], p[2], p[3], p[4], p[5], p[6], p[7]) for v in rows.values() for p in v)
                      if le == lb] + [-1])
    for row, parts in rows.items():
        parts.sort()
        k = parts[0][1]
        assert [p[0] for p in parts] == list(range(k)) and all(p[1] == k for p in parts)
        assert parts[0][2] == crow[row] and parts[-1][3] == crow[row + 1]
        for a, b in zip(parts, parts[1:]):
            assert a[3] == b[2]
        if lr:
            fin = parts[-1]
            assert (fin[4], fin[5]) == (0, lr)                 # finaliser holds every unit
            assert all(p[4] == p[5] for p in parts[:-1])        # others hold none
            assert fin[7] > last_plain                          # listed after all others
        if k > 1:
            base = parts[0][6]
            assert all(p[6] == base for p in parts)
            for j in range(k):
                assert base + j not in used
                used.add(base + j)
    assert len(used) == slots
    return rows


def test_plan_covers_every_unit_once():
    rng = np.random.default_rng(0)
    counts = rng.integers(0, 40, 50)
    crow = np.concatenate([[0], np.cumsum(counts)])
    for lr in (0, 8):
        for target in (0, 64, 200, 1000):
            table, n, slots = _plan(crow, q=64, lr=lr, target=target)
            rows = _check_plan(crow, lr, table, n, slots)
            expect = set(range(50)) if lr else {i for i in range(50) if counts[i]}
            assert set(rows) == expect


def test_plan_splits_long_rows_evenly():
    crow = [0, 4, 4 + 400, 404 + 10]
    table, n, slots = _plan(crow, q=64, lr=0, target=64 * 8)
    per_row = {}
    for row, bb, be, *_ in table:
        per_row.setdefault(int(row), []).append(int(be - bb))
    assert per_row[0] == [4]
    assert len(per_row[1]) == 50 and set(per_row[1]) == {8}
    assert per_row[2] == [5, 5]
    assert slots == 52


def test_plan_finaliser_takes_the_low_rank_units():
    crow = np.array([0, 30, 30, 100], np.int32)
    table, n, slots = _plan(crow, q=32, lr=8, target=300)
    rows = _check_plan(crow, 8, table, n, slots)
    # a row without blocks is a lone finaliser; a single-chunk row is its own finaliser
    assert [(p[2], p[3], p[4], p[5]) for p in rows[1]] == [(30, 30, 0, 8)]
    table1, n1, s1 = _plan(crow, q=32, lr=8, target=0)
    assert n1 == 3 and s1 == 0 and all(int(r[6]) == 1 for r in table1)


def test_partial_split_plan_covers_every_unit_once():
    """Equal rows (2:4 storage), the last 4 of 10 split in two: every block and
    low-rank unit once, each split row's finaliser after its other chunk, two
    partial slots per split row."""
    crow = np.arange(0, 11 * 12, 12, dtype=np.int32)
    table, n, slots = _runtime.partial_split_plan(crow, _cols(crow), 1, 32, 8, 4)
    assert n == 6 + 8 and slots == 8
    seen_blocks, per_row = [], {}
    for idx, (row, bb, be, lb, le, seq, nseq, slot) in enumerate(table[:n]):
        seen_blocks += list(range(bb, be))
        per_row.setdefault(int(row), []).append((seq, nseq, lb, le, slot, idx))
    assert sorted(seen_blocks) == list(range(crow[-1]))
    for row, parts in per_row.items():
        parts.sort()
        assert len(parts) == (2 if row >= 6 else 1)
        assert sum(le - lb for _, _, lb, le, _, _ in parts) == 8    # every unit once
        fin = parts[-1]
        assert (fin[2], fin[3]) == (0, 8) and fin[5] == max(p[5] for p in parts)
    # a row's chunks share a slot base; chunk `seq` uses base + seq
    split_slots = sorted(p[4] + p[0] for r, ps in per_row.items() if r >= 6 for p in ps)
    assert split_slots == list(range(8))


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


@pytest.mark.parametrize("bad", [-1, 4, 1 << 30])
def test_plans_reject_column_indices_out_of_range(bad):
    """The library checks every block's column before any kernel can index x
    or the values with it (both planners)."""
    crow = [0, 2, 3]
    with pytest.raises(ValueError, match="col"):
        _plan(crow, col=[0, bad, 1], NBK=4)
    with pytest.raises(ValueError, match="col"):
        _pf_plan(crow, [0, bad, 1], NBK=4)
    _plan(crow, col=[0, 3, 1], NBK=4)        # in range: accepted
    _pf_plan(crow, [0, 3, 1], NBK=4)
    with pytest.raises(ValueError, match="col"):
        _runtime.build_plan(np.asarray(crow, np.int32), np.zeros(0, np.int32), 4, None, 16, 0, 0)


def _pf_plan(crow, col, rows=None, group=1, NBK=None, p=64, step_cols=64):
    col = np.asarray(col, np.int32)
    if NBK is None:
        NBK = int(col.max()) + 1 if col.size else 1
    return _runtime.build_prefill_plan(np.asarray(crow, np.int32), col, NBK,
                                       None if rows is None else np.asarray(rows, np.int32), p,
                                       group, step_cols)


def _steps_to_entries(steps, s0, s1, p, G, step_cols=64):
    """The union entries (col_block, {slot: blk}) a group's step records hold,
    in order, checking each step's mask against its blocks on the way. A record
    holds, per wave w of the row kernel and load i, the block indices of slot
    8·(w + 4i) / p: every copy of a slot's index must agree."""
    E, IB, half = step_cols // p, G * p // 32, step_cols // 2
    out = []
    for rec in steps[s0:s1]:
        mask, cols = rec[0], rec[1:1 + E]
        W = rec[1 + E:1 + E + 4 * IB * E].reshape(4, IB, E)
        blks = np.full((E, G), -2, np.int64)
        for w in range(4):
            for i in range(IB):
                g = 8 * (w + 4 * i) // p
                assert (blks[:, g] == -2).all() or (blks[:, g] == W[w, i]).all()
                blks[:, g] = W[w, i]
        assert (blks != -2).all()  # every slot has its words
        want = 0
        for e in range(E):
            if cols[e] < 0:
                assert (blks[e] < 0).all()
                continue
            assert cols[e] % p == 0
            out.append((cols[e] // p, {g: int(blks[e, g]) for g in range(G) if blks[e, g] >= 0}))
            for g in range(G):
                if blks[e, g] >= 0:
                    for h in range(2):  # halves of the step the entry covers
                        if e * p < half * (h + 1) and (e + 1) * p > half * h:
                            want |= 1 << (h * G + g)
        assert int(mask) & 0xffffffff == want
        assert (rec[1 + E + 4 * IB * E:] == -1).all()  # padding
    return out


@pytest.mark.parametrize("p,step_cols", [(16, 64), (32, 64), (64, 64), (16, 32), (32, 32)])
def test_prefill_plan_merges_each_groups_columns(p, step_cols):
    """Every block of every listed row appears exactly once, in its row's slot,
    entries of a group ascend by column, E = step_cols/p entries per step, and
    the masks match the slots present in each half of a step."""
    rng = np.random.default_rng(1)
    NB, NBK = 23, 17
    counts = rng.integers(0, NBK + 1, NB)
    crow = np.concatenate([[0], np.cumsum(counts)]).astype(np.int32)
    col = np.concatenate([np.sort(rng.choice(NBK, c, replace=False)) for c in counts]).astype(np.int32)
    lib = _lib.load()
    for rows in (None, [0, 2, 3, 7, 11, 12, 20, 22]):
        for G in (64 // p,):  # the row kernel's tiles are 64 features wide
            groups, steps, ng = _pf_plan(crow, col, rows, G, p=p, step_cols=step_cols)
            assert steps.shape[1] == lib.ssl_prefill_step_ints(p, G, step_cols)
            assert steps.shape[1] % 4 == 0
            listed = list(range(NB)) if rows is None else rows
            assert ng == -(-len(listed) // G)
            seen = []
            for gi in range(ng):
                s0, s1 = groups[gi, 0], groups[gi, 1]
                grows = groups[gi, 2:]
                assert list(grows[grows >= 0]) == listed[gi * G:(gi + 1) * G]
                ents = _steps_to_entries(steps, s0, s1, p, G, step_cols)
                assert s1 - s0 == -(-len(ents) // (step_cols // p))
                cols = [c for c, _ in ents]
                assert np.all(np.diff(cols) > 0)
                for c, blks in ents:
                    for g, b in blks.items():
                        assert crow[grows[g]] <= b < crow[grows[g] + 1] and col[b] == c
                        seen.append(b)
            want = [b for r in listed for b in range(crow[r], crow[r + 1])]
            assert sorted(seen) == sorted(want)


def test_prefill_plan_repeated_column_gets_its_own_entry():
    crow, col = [0, 3], [5, 5, 2]
    groups, steps, ng = _pf_plan(crow, col, None, 1, p=64)
    ents = _steps_to_entries(steps, groups[0, 0], groups[0, 1], 64, 1)
    assert ng == 1 and ents == [(2, {0: 2}), (5, {0: 0}), (5, {0: 1})]


def test_prefill_step_ints():
    lib = _lib.load()
    sc = lib.ssl_prefill_step_ints
    # 1 + E + 4·IB·E words rounded up to 4 (E = step_cols/p entries, IB = 2
    # loads of 8 weight rows per wave)
    assert sc(64, 1, 64) == 12 and sc(32, 2, 64) == 20 and sc(16, 4, 64) == 40
    assert sc(32, 2, 32) == 12 and sc(16, 4, 32) == 20  # fp32: 32-column steps
    # only the row kernel's tiles (group·p = 64) and whole blocks per step
    assert sc(48, 2, 64) == 0 and sc(16, 17, 64) == 0
    assert sc(64, 2, 64) == 0 and sc(16, 8, 64) == 0
    assert sc(64, 1, 32) == 0 and sc(32, 2, 48) == 0
    assert lib.ssl_prefill_step_cols(_lib.SSL_F32) == 32
    assert lib.ssl_prefill_step_cols(_lib.SSL_BF16) == 64


def test_plan_target_cost_policy():
    assert _runtime.plan_target_cost(10**6, 64, 2, M=65) == 0  # several token tiles: no split
    # rows are split beyond 512 KiB of weights: 4096 cost units of a 64-row bf16 block
    assert _runtime.plan_target_cost(100, 64, 2, M=1) == 4096
    assert _runtime.plan_target_cost(10**7, 16, 4, M=16) == 512 * 1024 // 64


# ---------------------------------------------------- workspace / checks --


def test_workspace_sizes_are_aligned_and_monotone():
    lib = _lib.load()
    a = lib.ssl_slr_workspace_size(16, 172, 64, 256, 4096, 0, _lib.SSL_BF16)
    b = lib.ssl_slr_workspace_size(16, 172, 64, 256, 4096, 100, _lib.SSL_BF16)
    c = lib.ssl_slr_workspace_size(2048, 172, 64, 256, 4096, 10, _lib.SSL_BF16)
    # workspace: fp32 latent partials (up to 8 K chunks at decode), the final
    # latent (activation dtype), then the fp32 partial tiles of split rows
    # ([MG][slots][16·MT][p]); each part 256-byte aligned
    assert a == 8 * 16 * 256 * 4 + 16 * 256 * 2
    assert b == a + 100 * 16 * 64 * 4
    # 2048 rows: the final latent, the split-row partials and room for the
    # latent's K chunks when the row groups run whole (4096 in_features, 64
    # steps, in chunks of at least 16, at most twice the CUs' worth: 4 chunks
    # of 32 token tiles × 4 rank tiles, 64 × 64 fp32 each)
    assert c == 2048 * 256 * 2 + 32 * 10 * 64 * 64 * 4 + 4 * 32 * 4 * 64 * 64 * 4
    # 256 rows of 4096×11008 (64 block-rows): room for the split row groups'
    # partial tiles (up to 4 parts of 64-row tiles, at most 4 per CU, 128 × 64
    # fp32 each) and the latent's K chunks (172 steps in 11 chunks of 16, 16
    # tiles of 64 × 64 fp32); calls whose tall grid fills the device reserve none
    d = lib.ssl_slr_workspace_size(256, 64, 64, 256, 11008, 0, _lib.SSL_BF16)
    assert d == 256 * 256 * 2 + 1024 * 128 * 64 * 4 + 11 * 16 * 64 * 64 * 4
    assert lib.ssl_slr_workspace_size(8192, 64, 64, 256, 4096, 0, _lib.SSL_BF16) == 8192 * 256 * 2
    # counters: one per (token tile, block-row); from 128 rows (the prefill
    # kernels) then, 128-aligned, 4 slots of 128 per 64 rows: the latent tiles
    # written and the waiters passed, zero at rest like the row counters
    assert lib.ssl_slr_counter_count(16, 172) == 172
    assert lib.ssl_slr_counter_count(64, 172) == 172
    # (and one arrival word per (64-row token tile, block-row) for the parts of
    # split row groups)
    assert lib.ssl_slr_counter_count(2048, 172) == 5504 + 32 * 4 * 128 + 32 * 172
    assert lib.ssl_slr_counter_count(256, 172) == 4 * 172 + 80 + 4 * 4 * 128 + 4 * 172
    # exchange: the plan's uint64 handshake words (status, then per token tile
    # the latent-ready and ticket words and one arrival word per 16-rank
    # tile), 256-byte aligned
    # handshake words 8·(1 + MG·(2 + r/16)) rounded up to 256 bytes, then 16
    # copies of 512 bytes per token tile of the final-latent count
    assert lib.ssl_slr_exchange_size(16, 256, 4096, _lib.SSL_BF16) == 256 + 8192
    assert lib.ssl_slr_exchange_size(2048, 256, 4096, _lib.SSL_BF16) == 4864 + 32 * 8192
    assert lib.ssl_slr_exchange_size(16, 0, 4096, _lib.SSL_BF16) == 256
    assert lib.ssl_bsr_addmm_counter_count(16, 172) == 172
    assert lib.ssl_bsr_addmm_counter_count(65, 172) == 2 * 172
    assert lib.ssl_bsr_addmm_workspace_size(16, 172, 64, 0) == 0
    assert lib.ssl_bsr_addmm_workspace_size(16, 172, 64, 10) == 10 * 16 * 64 * 4


def test_entry_points_reject_bad_arguments_before_any_launch():
    lib = _lib.load()
    P = 256

    def op(**kw):
        a = dict(out=P, ldo=64, x=P, ldx=64, col=P, values=P, nnz=1, plan=P, n_chunks=1, n_slots=0,
                 values_pq=None, pf_groups=None, pf_entries=None, pf_n_groups=0, pf_group=0, M=1, N=64, K=64, NB=1,
                 p=64, q=64, dtype=_lib.SSL_BF16, counters=None, n_counters=0, workspace=None,
                 workspace_bytes=0, stream=None)
        a.update(kw)
        return lib.ssl_bsr_addmm_inplace(*a.values())

    # unsupported block shapes: sides not multiples of 16, tiles wider than 64,
    # blocks deeper than 256 (the Python layer cuts those into sub-blocks first)
    for p, q in ((8, 8), (16, 8), (80, 16), (128, 64), (64, 272), (64, 0)):
        assert op(p=p, q=q, N=p, K=max(q, 16)) == _lib.SSL_ERR_UNSUPPORTED, (p, q)
        assert b"output features" in lib.ssl_last_error()
    # every supported shape gets past the shape check (then stops at N ≠ NB·p)
    for p in (16, 32, 48, 64):
        for q in (16, 32, 48, 64, 96, 256):
            assert op(p=p, q=q, N=p + 1, K=q) == _lib.SSL_ERR_INVALID, (p, q)
    # N inconsistent with NB·p
    assert op(N=60) == _lib.SSL_ERR_INVALID
    # missing counters
    assert op(M=16) == _lib.SSL_ERR_WORKSPACE
    # prefill-sized call without a prefill plan
    big = dict(M=4096, counters=P, n_counters=1 << 20)
    assert op(**big) == _lib.SSL_ERR_INVALID and b"prefill plan" in lib.ssl_last_error()
    assert lib.ssl_prefill_min_rows() == 128
    # 16-bit fused calls: streaming below 128 rows, and at 128 rows for at
    # most 2048 output features (block-rows × p); the tiled kernels otherwise,
    # 16×16 blocks included
    tp = lambda M, rows, p, dt=_lib.SSL_BF16, q=None: lib.ssl_slr_takes_prefill(
        M, rows, p, p if q is None else q, dt)
    assert tp(127, 500, 64) == 0 and tp(128, 172, 64) == 1 and tp(128, 64, 64) == 1
    assert tp(128, 32, 64) == 0 and tp(128, 64, 32) == 0 and tp(128, 65, 32) == 1
    assert tp(128, 128, 16) == 0 and tp(128, 129, 16) == 1 and tp(129, 64, 32) == 1
    assert tp(512, 500, 32) == 1 and tp(511, 64, 32) == 1 and tp(300, 500, 32) == 1
    assert tp(128, 500, 32) == 1 and tp(512, 500, 16) == 1 and tp(300, 500, 16) == 1
    assert tp(2048, 64, 32) == 1 and tp(4096, 500, 64, _lib.SSL_F32) == 0
    # fp32: when the short (64-row) tiles' grid fills the device (LLaMA-60M
    # 512-wide projections at 2048 rows: 32 token tiles × 8 groups of two
    # 32-row block-rows)
    F32 = _lib.SSL_F32
    assert tp(2048, 16, 32, F32) == 1 and tp(1024, 16, 32, F32) == 0 and tp(1024, 43, 32, F32) == 1
    assert lib.ssl_prefill_group(4096, 172, 64, 64) == 1  # 64 output features per row tile
    # the prefill kernels take square 16/32/64 blocks; other shapes stream
    assert tp(2048, 500, 32, q=64) == 0 and tp(2048, 500, 48) == 0
    # the op: from 128 rows, except one token tile whose short-tile grid (64/p
    # block-rows a group) fills at most a quarter of 256 CUs with 32/64-wide blocks
    ap = lambda M, rows, p, q, dt=_lib.SSL_BF16: lib.ssl_bsr_addmm_takes_prefill(M, rows, p, q, dt)
    assert ap(128, 172, 64, 64) == 1 and ap(127, 172, 64, 64) == 0 and ap(4096, 500, 32, 64) == 0
    assert ap(4096, 500, 64, 64, _lib.SSL_F32) == 0 and ap(129, 1, 64, 64) == 1
    assert ap(128, 64, 64, 64) == 0 and ap(128, 65, 64, 64) == 1 and ap(128, 128, 32, 32) == 0
    assert ap(128, 129, 32, 32) == 1 and ap(128, 1, 16, 16) == 1

    # ssl_slr_forward with fake, aligned device pointers (every case below is
    # rejected on the host before any launch)
    P = 256

    def slr(**kw):
        a = dict(y=P, ldy=64, x=P, ldx=64, A=P, B=P, bias=None, col=P, values=P, plan=P,
                 n_chunks=1, n_slots=0, lr_wgs=1, M=1, m=64, m_pad=64, NB=1, r_pad=64, p=64,
                 q=64, dtype=_lib.SSL_BF16, counters=None, n_counters=0, exchange=None,
                 exchange_bytes=0, workspace=None, workspace_bytes=0, stream=None)
        a.update(kw)
        return lib.ssl_slr_forward(*a.values())

    assert slr(dtype=7) == _lib.SSL_ERR_UNSUPPORTED
    assert slr(p=80, q=48) == _lib.SSL_ERR_UNSUPPORTED
    # lr_wgs inconsistent with r_pad, or more consuming workgroups than chunks
    assert slr(lr_wgs=0) == _lib.SSL_ERR_INVALID and b"lr_wgs" in lib.ssl_last_error()
    assert slr(lr_wgs=2) == _lib.SSL_ERR_INVALID and b"lr_wgs" in lib.ssl_last_error()
    # r_pad not a multiple of 64; misaligned x
    assert slr(r_pad=48) == _lib.SSL_ERR_INVALID
    assert slr(x=P + 2) == _lib.SSL_ERR_INVALID and b"x rows" in lib.ssl_last_error()
    # missing workspace / counters / exchange area
    assert slr(M=16) == _lib.SSL_ERR_WORKSPACE and b"workspace" in lib.ssl_last_error()
    assert slr(M=16, workspace=P, workspace_bytes=1 << 20) == _lib.SSL_ERR_WORKSPACE
    assert b"counters" in lib.ssl_last_error()
    assert slr(M=16, workspace=P, workspace_bytes=1 << 20, counters=P,
               n_counters=1) == _lib.SSL_ERR_WORKSPACE
    assert b"exchange" in lib.ssl_last_error()
    # M = 0 is a no-op
    assert slr(M=0) == _lib.SSL_OK
    # a call that ssl_slr_takes_prefill sends to the prefill kernels needs the
    # prefill plans, which only the group entry point carries: an fp32 call
    # whose 64-row tiles fill the device (2048 rows × 16 block-rows of 32)
    M2, NB2, F32 = 2048, 16, _lib.SSL_F32
    assert tp(M2, NB2, 32, F32) == 1
    big = dict(M=M2, m=512, m_pad=512, ldx=512, ldy=512, NB=NB2, p=32, q=32, dtype=F32,
               workspace=P, workspace_bytes=lib.ssl_slr_workspace_size(M2, NB2, 32, 64, 512, 0, F32),
               counters=P, n_counters=lib.ssl_slr_counter_count(M2, NB2),
               exchange=P, exchange_bytes=lib.ssl_slr_exchange_size(M2, 64, 512, F32))
    assert slr(**big) == _lib.SSL_ERR_INVALID and b"prefill plan" in lib.ssl_last_error()
    # the same call with a 16-bit dtype and with a row count the kernels stream
    assert tp(M2, NB2, 32) == 1
    assert slr(**{**big, "dtype": _lib.SSL_BF16}) == _lib.SSL_ERR_INVALID
    assert b"prefill plan" in lib.ssl_last_error()
    assert tp(1024, NB2, 32, F32) == 0
    # the group entry point: 1..4 members
    members = (_lib.SlrMember * 5)()
    rc = lib.ssl_slr_forward_group(P, 64, 1, 64, 64, 64, 64, _lib.SSL_BF16, members, 5, None)
    assert rc == _lib.SSL_ERR_INVALID and b"1 to 4" in lib.ssl_last_error()
    rc = lib.ssl_slr_forward_group(P, 64, 1, 64, 64, 64, 64, _lib.SSL_BF16, members, 0, None)
    assert rc == _lib.SSL_ERR_INVALID
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


def test_block_topk_rejects_bad_arguments_before_any_launch():
    lib = _lib.load()
    fake = 256  # never dereferenced: every call below fails its argument checks first
    ws = lib.ssl_block_topk_workspace_size(4)
    assert ws >= 4096 and ws % 256 == 0 and lib.ssl_block_topk_workspace_size(0) == 0
    assert lib.ssl_block_topk(fake, 64, 2, 2, 0, 32, _lib.SSL_F32, 1, fake, fake, None, 0, fake, ws, None) == 1
    assert lib.ssl_block_topk(fake, 32, 2, 2, 32, 32, _lib.SSL_F32, 1, fake, fake, None, 0, fake, ws, None) == 1
    assert lib.ssl_block_topk(fake, 64, 2, 2, 32, 32, 7, 1, fake, fake, None, 0, fake, ws, None) == 2
    assert lib.ssl_block_topk(None, 64, 2, 2, 32, 32, _lib.SSL_BF16, 1, fake, fake, None, 0, fake, ws, None) == 1
    assert lib.ssl_block_topk(fake, 64, 2, 2, 32, 32, _lib.SSL_BF16, 1, fake, fake, fake, 16, fake, ws, None) == 1
    assert b"ldo" in lib.ssl_last_error()
    # the select's workspace: missing, short, misaligned
    assert lib.ssl_block_topk(fake, 64, 2, 2, 32, 32, _lib.SSL_BF16, 1, fake, fake, None, 0, None, ws, None) == 3
    assert lib.ssl_block_topk(fake, 64, 2, 2, 32, 32, _lib.SSL_BF16, 1, fake, fake, None, 0, fake, ws - 4, None) == 3
    assert lib.ssl_block_topk(fake, 64, 2, 2, 32, 32, _lib.SSL_BF16, 1, fake, fake, None, 0, fake + 4, ws, None) == 3
    assert b"workspace" in lib.ssl_last_error()
    assert lib.ssl_block_topk(fake, 64, 0, 2, 32, 32, _lib.SSL_BF16, 1, None, None, None, 0, None, 0, None) == 0


def test_decode_entry_points_reject_bad_arguments_before_any_launch():
    lib = _lib.load()
    fake = 256  # never dereferenced: every call below fails its argument checks first
    bf = _lib.SSL_BF16
    # add_rmsnorm: unknown dtype, leading dimension below hidden, null weight
    assert lib.ssl_add_rmsnorm(fake, 64, None, 0, fake, fake, 64, 2, 64, 1e-6, 9, None) == 1
    assert lib.ssl_add_rmsnorm(fake, 32, None, 0, fake, fake, 64, 2, 64, 1e-6, bf, None) == 1
    assert lib.ssl_add_rmsnorm(fake, 64, None, 0, None, fake, 64, 2, 64, 1e-6, bf, None) == 1
    assert lib.ssl_add_rmsnorm(None, 64, None, 0, None, None, 64, 0, 64, 1e-6, bf, None) == 0
    assert lib.ssl_add_rmsnorm(fake, 9000, None, 0, fake, fake, 9000, 2, 9000, 1e-6, bf, None) == 2
    # embed_rmsnorm: no vocabulary, narrow table, null tokens
    assert lib.ssl_embed_rmsnorm(fake, 64, 0, fake, fake, 64, fake, fake, 64, 2, 64, 1e-6, bf, None) == 1
    assert lib.ssl_embed_rmsnorm(fake, 32, 9, fake, fake, 64, fake, fake, 64, 2, 64, 1e-6, bf, None) == 1
    assert lib.ssl_embed_rmsnorm(fake, 64, 9, None, fake, 64, fake, fake, 64, 2, 64, 1e-6, bf, None) == 1
    # rope: heads not a multiple of kv_heads, odd or too wide heads, narrow rows
    args = [fake, 512, fake, 128, fake, 128, fake, fake, None, None, 1e-6, fake, fake, fake, fake, 2]
    assert lib.ssl_rope_kv_append(*args, 4, 3, 128, 16, bf, None) == 1
    assert lib.ssl_rope_kv_append(*args, 4, 1, 127, 16, bf, None) == 2
    assert lib.ssl_rope_kv_append(*args, 4, 1, 512, 16, bf, None) == 2
    assert lib.ssl_rope_kv_append(*args, 8, 1, 128, 16, bf, None) == 1
    # attention: head_dim without a kernel, too many splits, small workspace, misalignment
    a = [fake, fake, fake, fake, fake, 512, 2, 4, 4]
    cn = lib.ssl_decode_attention_counter_count(2, 4, 4)
    assert cn == 2 * 4 and lib.ssl_decode_attention_counter_count(2, 16, 1) == 2 * 2
    assert lib.ssl_decode_attention(*a, 96, 16, 0.1, 1, fake, 1 << 20, fake, cn, bf, None) == 2
    assert lib.ssl_decode_attention(*a, 128, 16, 0.1, 300, fake, 1 << 20, fake, cn, bf, None) == 1
    need = lib.ssl_decode_attention_workspace_size(2, 4, 128, 3)
    assert need == 2 * 4 * 3 * 130 * 4
    assert lib.ssl_decode_attention(*a, 128, 16, 0.1, 3, fake, need - 1, fake, cn, bf, None) == 3
    assert lib.ssl_decode_attention(*a, 128, 16, 0.1, 3, fake, need, fake, cn - 1, bf, None) == 3
    assert lib.ssl_decode_attention(fake + 2, *a[1:], 128, 16, 0.1, 3, fake, need, fake, cn, bf,
                                    None) == 1
    # rope + attention in one launch: the attention checks, plus the projections'
    # widths and 16-byte rows
    r = [fake, 512, fake, 512, fake, 512, fake, fake, None, None, 1e-6, fake, fake, fake, fake,
         512, 2, 4, 4]
    tail = [16, 0.1, 3, fake, need, fake, cn, bf, None]
    assert lib.ssl_decode_rope_attention(*r, 96, *tail) == 2
    assert lib.ssl_decode_rope_attention(*r, 128, 16, 0.1, 3, fake, need - 1, fake, cn, bf,
                                         None) == 3
    assert lib.ssl_decode_rope_attention(*r[:1], 256, *r[2:], 128, *tail) == 1  # ldq < 4·128
    assert lib.ssl_decode_rope_attention(*r[:1], 516, *r[2:], 128, *tail) == 1  # 1032-byte rows
    assert lib.ssl_decode_rope_attention(*r[:2], fake + 2, *r[3:], 128, *tail) == 1  # k misaligned
    assert lib.ssl_decode_rope_attention(*r[:6], None, *r[7:], 128, *tail) == 1  # no cos table
    assert lib.ssl_decode_rope_attention(*r[:16], 0, *r[17:], 128, *tail) == 0  # no rows
    # silu_mul: leading dimension below n
    assert lib.ssl_silu_mul(fake, 8, fake, 16, fake, 16, 2, 16, bf, None) == 1
    assert lib.ssl_silu_mul(None, 8, None, 16, None, 16, 0, 16, bf, None) == 0


def test_decode_attention_split_policy():
    lib = _lib.load()
    # about 1024 workgroups, slices of at least 128 positions, at most 64 slices
    assert lib.ssl_decode_attention_splits(1, 16, 16, 1024) == 8
    assert lib.ssl_decode_attention_splits(16, 16, 16, 1024) == 4
    assert lib.ssl_decode_attention_splits(1, 32, 8, 100000) == 64
    assert lib.ssl_decode_attention_splits(64, 32, 32, 4096) == 1
    assert lib.ssl_decode_attention_splits(1, 4, 4, 10) == 1


def test_balanced_target_splits_only_the_longest_rows():
    """The decode balancing target (p = 64 rows, one workgroup per compute unit):
    the chunk count fits the slots a minimal latent leaves free, only rows above
    the target split, and short rows or a full device get no target."""
    rng = np.random.default_rng(0)
    blocks = rng.binomial(64, 0.5, size=172)
    costs = blocks.astype(np.int64) * 64 + 8 * 32
    lat_min = _runtime._BALANCE_LATENT_MIN
    t = _runtime.balanced_target(costs, 128, 256, 16)
    assert 0 < t < costs.max()
    chunks = np.ceil(costs / t).sum()
    assert costs.size < chunks <= 256 - lat_min * 16
    assert np.ceil(costs / (t - 1)).sum() > 256 - lat_min * 16  # the smallest such target
    assert _runtime.balanced_target(costs, 16, 256, 16) == 0  # rows under 128 KiB
    assert _runtime.balanced_target(np.full(400, 2304), 128, 256, 16) == 0  # no free slots
    # the plan built with it covers every unit once
    crow = np.concatenate([[0], np.cumsum(blocks)]).astype(np.int32)
    table, n_chunks, _ = _runtime.build_plan(crow, _cols(crow), 1, None, 64, 8, t)
    assert n_chunks == chunks
    for row in range(172):
        mine = table[table[:, 0] == row]
        spans = sorted((int(b), int(e)) for b, e in mine[:, 1:3])
        assert spans[0][0] == crow[row] and spans[-1][1] == crow[row + 1]
        assert all(spans[i][1] == spans[i + 1][0] for i in range(len(spans) - 1))
        assert (len(mine) > 1) == (costs[row] > t)
        assert sum(int(e - b) for b, e in mine[:, 3:5]) == 8


def test_chain_fragment_copy_sizes():
    """Room for a chained stage's input in fragment order: 1 KiB per 16 token
    rows (whole tiles of the call's tile height) and 32 features, rounded up."""
    lib = _lib.load()
    assert lib.ssl_slr_chain_frag_bytes(16, 2048) == 64 * 1024
    assert lib.ssl_slr_chain_frag_bytes(1, 2048) == 64 * 1024  # one 16-row tile
    assert lib.ssl_slr_chain_frag_bytes(16, 5472) == 171 * 1024
    assert lib.ssl_slr_chain_frag_bytes(16, 5461) == 171 * 1024  # 32-feature units, rounded up
    tiles = lib.ssl_slr_chain_frag_bytes(40, 256) // (8 * 1024)
    assert tiles >= 3 and tiles * 8 * 1024 == lib.ssl_slr_chain_frag_bytes(40, 256)
    assert lib.ssl_slr_chain_frag_bytes(0, 2048) == 0
    assert lib.ssl_slr_chain_frag_bytes(16, 0) == 0


def test_balanced_target_extra_chunks_for_64_wide_rows():
    """With 64-wide blocks the decode balancing may use an eighth of the
    compute units beyond the free slots: more rows split than without."""
    rng = np.random.default_rng(1)
    costs = rng.binomial(64, 0.5, size=172).astype(np.int64) * 64 + 8 * 32
    base = _runtime.balanced_target(costs, 128, 256, 16)
    wide = _runtime.balanced_target(costs, 128, 256 + 256 // _runtime._BALANCE_EXTRA_P64, 16)
    assert 0 < wide < base
    assert np.ceil(costs / wide).sum() <= 256 + 32 - _runtime._BALANCE_LATENT_MIN * 16


def _parts(groups, group):
    return _runtime.build_prefill_parts(np.asarray(groups, np.int32), len(groups), group)


def _groups_of(steps, group=1):
    """A group table whose group g holds steps[g] steps (rows are placeholders)."""
    b = np.concatenate([[0], np.cumsum(steps)])
    return [[b[g], b[g + 1]] + [g] * group for g in range(len(steps))]


def test_part_table_cuts_only_the_long_groups_of_a_skewed_plan():
    """Parts of about the mean group's steps (at least 32): every step of every
    group exactly once, parts in group and step order, near-equal parts, the
    split groups' partial tiles numbered contiguously in part order."""
    rng = np.random.default_rng(3)
    steps = np.concatenate([[172, 150, 100], rng.integers(0, 30, 61)])
    for group in (1, 2, 4):
        table, n_parts, split = _parts(_groups_of(steps, group), group)
        mean = -(-int(steps.sum()) // len(steps))
        target = max(32, mean)
        covered = {}
        nxt = 0
        for g, b0, b1, k, nk, first, z0, z1 in table:
            assert (z0, z1) == (0, 0)
            covered.setdefault(int(g), []).append((int(k), int(nk), int(b0), int(b1), int(first)))
        for g, recs in covered.items():
            recs.sort()
            nk = recs[0][1]
            assert [r[0] for r in recs] == list(range(nk)) and all(r[1] == nk for r in recs)
            b = int(np.sum(steps[:g]))
            assert recs[0][2] == b and recs[-1][3] == b + steps[g]
            for r0, r1 in zip(recs, recs[1:]):
                assert r0[3] == r1[2]
            lens = [r[3] - r[2] for r in recs]
            assert nk == max(1, -(-int(steps[g]) // target)) or nk == 16
            if nk > 1:
                assert max(lens) - min(lens) <= max(lens) // 2 + 1
                assert recs[0][4] == nxt and all(r[4] == nxt for r in recs)
                nxt += nk
        assert sorted(covered) == list(range(len(steps)))
        assert n_parts == len(table) and split == nxt
        assert [int(r[0]) for r in table] == sorted(int(r[0]) for r in table)  # group order


def test_part_table_is_empty_for_even_plans_and_checks_its_input():
    assert _parts(_groups_of([40, 41, 39, 80]), 1) is None            # longest ≤ 2 · mean
    assert _parts(_groups_of([5, 6, 60]), 1) is None                   # ≤ 2 · 32
    assert _parts([], 1) is None
    t = _parts(_groups_of([0, 0, 0, 200], 2), 2)
    assert t is not None and t[1] == 3 + 4 and t[2] == 4               # 200 in parts of the mean, 50
    bad = _groups_of([10, 200])
    bad[1][0] += 1                                                      # a gap between groups
    with pytest.raises(ValueError, match="tile"):
        _parts(bad, 1)
    assert _lib.load().ssl_prefill_parts_bytes(2048, 10) == 10 * 2048 * 64 * 4
    assert _lib.load().ssl_prefill_parts_bytes(300, 3) == 3 * 384 * 64 * 4
    assert _lib.load().ssl_prefill_parts_bytes(300, 0) == 0
