"""Pin the CPU oracle (oracle/slr_oracle.py, oracle/bsr_addmm_port.c).

Every oracle function is checked against something other than its own formula:
the reference AVX2 kernel's stored outputs (tests/golden), torch's own BSR
conversion, closed forms computed along a different path, brute-force loops, and
the special cases of the L1 keep rule. A last group plants mistakes in copies of
the oracle and shows that these checks catch them.
"""

from __future__ import annotations

import ctypes
import subprocess
import sys
from pathlib import Path

import numpy as np
import pytest
import torch

ROOT = Path(__file__).resolve().parents[1]
sys.path.insert(0, str(ROOT / "tests" / "golden"))

from golden_inputs import CASES, make_case  # noqa: E402
from oracle import slr_oracle as orc  # noqa: E402

GOLDEN = np.load(ROOT / "tests" / "golden" / "bsr_addmm_avx2.npz")


def _oracle_lib():
    lib_path = ROOT / "oracle" / "liboracle.so"
    if not lib_path.exists():
        subprocess.run(["make", "-C", str(ROOT / "oracle"), "liboracle.so"], check=True,
                       capture_output=True)
    lib = ctypes.CDLL(str(lib_path))
    f = lib.oracle_bsr_addmm_port
    f.restype = ctypes.c_int
    f.argtypes = [ctypes.c_void_p] * 6 + [ctypes.c_int64] * 5 + [ctypes.c_int]
    return f


def _port(out, x, crow, col, values_t, active, block, threads=2):
    out = np.ascontiguousarray(out, dtype=np.float32).copy()
    x = np.ascontiguousarray(x, dtype=np.float32)
    f = _oracle_lib()
    rc = f(out.ctypes.data, x.ctypes.data, crow.ctypes.data, col.ctypes.data,
           values_t.ctypes.data, active.ctypes.data, out.shape[0], x.shape[1],
           len(crow) - 1, len(active), block, threads)
    assert rc == 0
    return out


# ------------------------------------------------- golden (reference AVX2) --


@pytest.mark.parametrize("name", CASES)
def test_oracle_bsr_addmm_matches_reference_kernel_outputs(name):
    c = make_case(name)
    ref = GOLDEN[f"{name}__out"]
    got = orc.bsr_addmm_inplace(c["out"], c["x"], c["crow"], c["col"], c["values_t"], c["active"])
    scale = max(1.0, float(np.abs(ref).max()))
    assert np.max(np.abs(got - ref)) <= 1e-5 * scale


@pytest.mark.parametrize("name", CASES)
def test_c_port_is_bit_exact_with_reference_kernel_outputs(name):
    c = make_case(name)
    got = _port(c["out"], c["x"], c["crow"], c["col"], c["values_t"], c["active"], c["block"])
    assert np.array_equal(got.view(np.uint32), GOLDEN[f"{name}__out"].view(np.uint32))


def test_c_port_matches_live_reference_build_when_present():
    ref_dir = ROOT / "oracle" / "_ref"
    if not any(ref_dir.glob("bsr_ref_avx2*.so")):
        pytest.skip("oracle/_ref not built (reference tree absent)")
    sys.path.insert(0, str(ref_dir))
    import bsr_ref_avx2

    rng = np.random.default_rng(5)
    for block in (8, 16, 32, 64):
        NB, NBK, M = 5, 7, 13
        slots = np.sort(rng.permutation(NB * NBK)[:17])
        S = np.zeros((NB * block, NBK * block), np.float32)
        for s in slots:
            br, bc = divmod(int(s), NBK)
            S[br * block:(br + 1) * block, bc * block:(bc + 1) * block] = rng.standard_normal(
                (block, block), dtype=np.float32)
        crow, col, vals = orc.dense_to_bsr(S, block, block)
        crow32, col32, vt, act = orc.module_buffers(crow, col, vals)
        vt = vt.astype(np.float32)
        x = rng.standard_normal((M, NBK * block), dtype=np.float32)
        out = rng.standard_normal((M, NB * block), dtype=np.float32)
        ref = torch.from_numpy(out.copy())
        bsr_ref_avx2.bsr_addmm_avx2_(ref, torch.from_numpy(x), torch.from_numpy(crow32),
                                     torch.from_numpy(col32), torch.from_numpy(vt),
                                     torch.from_numpy(act))
        got = _port(out, x, crow32, col32, vt, act, block, threads=3)
        assert np.array_equal(got, ref.numpy())


# -------------------------------------------- reference tests restated --


@pytest.mark.parametrize("p,q", [(8, 8), (16, 16), (32, 32), (64, 64), (16, 32), (32, 16),
                                 (48, 48), (48, 16), (64, 48), (128, 32), (16, 512)])
def test_oracle_bsr_addmm_matches_a_dense_matmul(p, q):
    """tests/test_ssalaad.py:320-327, with torch's to_sparse_bsr building the
    buffers: square blocks as the reference test has them, and the non-square
    (p, q) blocks the reference's GPU op takes (addmm_inplace.py:59-63, 96-97:
    values (nnz, q, p), p and q read separately). A transposed block, swapped
    p/q or a wrong column stride fails the closed form x·Sᵀ."""
    g = torch.Generator().manual_seed(0)
    S = torch.zeros(p * 4, q * 6)
    for br, bc in [(0, 1), (1, 0), (1, 3), (2, 5), (3, 2)]:
        S[br * p:(br + 1) * p, bc * q:(bc + 1) * q] = torch.randn(p, q, generator=g)
    x = torch.randn(5, q * 6, generator=g)
    bsr = S.to_sparse_bsr(blocksize=(p, q))
    crow = bsr.crow_indices().to(torch.int32)
    got = orc.bsr_addmm_inplace(
        np.zeros((5, p * 4)), x.numpy(), crow.numpy(), bsr.col_indices().to(torch.int32).numpy(),
        bsr.values().transpose(1, 2).contiguous().numpy(),
        (crow[1:] - crow[:-1]).nonzero().squeeze(-1).to(torch.int32).numpy())
    np.testing.assert_allclose(got, (x @ S.T).numpy(), rtol=0, atol=1e-4)


def test_oracle_bsr_addmm_skips_empty_block_rows():
    """tests/test_ssalaad.py:330-337: rows of inactive block-rows stay untouched."""
    c = make_case("untouched_b16")
    got = orc.bsr_addmm_inplace(c["out"], c["x"], c["crow"], c["col"], c["values_t"], c["active"])
    assert np.array_equal(got[:, :32], np.full((3, 32), 7.0))
    assert not np.array_equal(got[:, 32:], np.full((3, 16), 7.0))


def test_oracle_bsr_addmm_honours_the_active_row_list():
    """A block-row missing from active_rows is skipped even if it holds blocks
    (addmm_inplace.py:65-69 iterates active_rows only)."""
    c = make_case("random_b16_m7")
    act = c["active"][1:]
    got = orc.bsr_addmm_inplace(c["out"], c["x"], c["crow"], c["col"], c["values_t"], act)
    skipped = int(c["active"][0])
    assert np.array_equal(got[:, skipped * 16:(skipped + 1) * 16],
                          c["out"][:, skipped * 16:(skipped + 1) * 16])


def test_oracle_bsr_addmm_equals_brute_force_loops():
    rng = np.random.default_rng(3)
    block, NB, NBK, M = 4, 3, 4, 2
    S = np.zeros((NB * block, NBK * block))
    for br, bc in [(0, 0), (0, 3), (2, 1)]:
        S[br * block:(br + 1) * block, bc * block:(bc + 1) * block] = rng.standard_normal((block, block))
    crow, col, vals = orc.dense_to_bsr(S, block, block)
    crow32, col32, vt, act = orc.module_buffers(crow, col, vals)
    x = rng.standard_normal((M, NBK * block))
    out0 = rng.standard_normal((M, NB * block))
    got = orc.bsr_addmm_inplace(out0, x, crow32, col32, vt, act)
    want = out0.copy()
    for i in range(M):
        for r in range(NB * block):
            if (r // block) not in act:
                continue
            s = 0.0
            for k in range(NBK * block):
                s += x[i, k] * S[r, k]
            want[i, r] += s
    np.testing.assert_allclose(got, want, rtol=1e-12, atol=1e-12)


# ---------------------------------------------------------- structure --


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
@pytest.mark.parametrize("pq", [(16, 16), (32, 32), (8, 16), (64, 32)])
def test_dense_to_bsr_matches_torch_to_sparse_bsr(dtype, pq):
    p, q = pq
    rng = np.random.default_rng(p * 100 + q)
    NB, NBK = 5, 6
    S = np.zeros((NB * p, NBK * q), dtype=np.float32)
    for s in rng.permutation(NB * NBK)[:13]:
        br, bc = divmod(int(s), NBK)
        S[br * p:(br + 1) * p, bc * q:(bc + 1) * q] = rng.standard_normal((p, q))
    S_t = torch.from_numpy(S).to(dtype)
    bsr = S_t.to_sparse_bsr(blocksize=(p, q))
    crow, col, vals = orc.dense_to_bsr(S_t.float().numpy(), p, q)
    assert np.array_equal(crow, bsr.crow_indices().numpy())
    assert np.array_equal(col, bsr.col_indices().numpy())
    assert np.array_equal(vals, bsr.values().float().numpy())


def test_dense_to_bsr_keep_rule_special_values():
    """L1-sum rule (artifact.py:28-29): a NaN anywhere drops the block; ±0 blocks
    are dropped; inf and subnormal entries keep it."""
    p = q = 4
    S = np.zeros((p, 6 * q), dtype=np.float32)
    S[0, 0 * q] = np.nan            # block 0: NaN -> dropped (L1 = NaN)
    S[1, 0 * q + 1] = 5.0
    S[:, 1 * q:2 * q] = -0.0        # block 1: only negative zeros -> dropped
    S[2, 2 * q] = np.inf            # block 2: inf -> kept
    S[3, 3 * q + 3] = np.float32(1e-45)  # block 3: smallest subnormal -> kept
    S[0, 4 * q] = np.inf            # block 4: inf and -inf -> |.| sums to inf -> kept
    S[1, 4 * q] = -np.inf
    crow, col, _ = orc.dense_to_bsr(S, p, q)  # block 5: all zero -> dropped
    assert crow.tolist() == [0, 3]
    assert col.tolist() == [2, 3, 4]


def test_dense_to_bsr_rejects_indivisible_shapes():
    with pytest.raises(ValueError, match="not divisible"):
        orc.dense_to_bsr(np.zeros((10, 16)), 4, 4)


def test_module_buffers_match_the_reference_conversion():
    """ls_linear.py:89-97 via torch ops, as the reference's test helper does (:307-317)."""
    rng = np.random.default_rng(11)
    S = np.zeros((64, 96), dtype=np.float32)
    for br, bc in [(0, 1), (2, 0), (2, 5), (3, 2)]:
        S[br * 16:(br + 1) * 16, bc * 16:(bc + 1) * 16] = rng.standard_normal((16, 16))
    bsr = torch.from_numpy(S).to_sparse_bsr(blocksize=(16, 16))
    crow = bsr.crow_indices()
    crow32, col32, vt, act = orc.module_buffers(*orc.dense_to_bsr(S, 16, 16))
    assert crow32.dtype == np.int32 and col32.dtype == np.int32 and act.dtype == np.int32
    assert np.array_equal(crow32, crow.to(torch.int32).numpy())
    assert np.array_equal(col32, bsr.col_indices().to(torch.int32).numpy())
    assert np.array_equal(vt, bsr.values().transpose(1, 2).contiguous().numpy())
    assert np.array_equal(act, (crow[1:] - crow[:-1]).nonzero().squeeze(-1).to(torch.int32).numpy())
    assert act.tolist() == [0, 2, 3]


# --------------------------------------------------------- arithmetic --


def _random_slr(rng, n, m, r, block, density, bias=True):
    NB, NBK = n // block, m // block
    rows, cols = orc.random_block_structure(NB, NBK, density, rng)
    vals = rng.standard_normal((len(rows), block, block)) * 0.02
    crow, col, vals = orc.structure_to_bsr(rows, cols, NB, vals)
    A = rng.standard_normal((n, r)) * 0.02
    B = rng.standard_normal((r, m)) * 0.02
    b = rng.standard_normal(n) if bias else None
    return A, B, crow, col, vals, b


@pytest.mark.parametrize("pq", [(16, 16), (32, 16), (16, 48)])
def test_bsr_to_dense_matches_torch_bsr_to_dense(pq):
    """The oracle's densification against torch.sparse_bsr_tensor(...).to_dense()
    on a structure with empty block-rows, a full block-row and repeated values."""
    p, q = pq
    rng = np.random.default_rng(p * 100 + q)
    NB, NBK = 9, 7
    counts = np.array([0, 3, 7, 0, 1, 5, 2, 0, 4])
    crow = np.concatenate([[0], np.cumsum(counts)])
    col = np.concatenate([np.sort(rng.permutation(NBK)[:c]) for c in counts]).astype(np.int64)
    vals = rng.standard_normal((int(crow[-1]), p, q))
    vals[2] = vals[1]
    want = torch.sparse_bsr_tensor(torch.from_numpy(crow), torch.from_numpy(col),
                                   torch.from_numpy(vals), size=(NB * p, NBK * q)).to_dense()
    np.testing.assert_array_equal(orc.bsr_to_dense(crow, col, vals, NB * p, NBK * q), want.numpy())


def test_slr_linear_matches_the_densified_weight():
    """y = x·(A·B + S)ᵀ + b with S densified independently (the bundle test's formula)."""
    rng = np.random.default_rng(21)
    n, m, r, block = 96, 128, 8, 16
    A, B, crow, col, vals, b = _random_slr(rng, n, m, r, block, 0.5)
    x = rng.standard_normal((7, m))
    S_dense = orc.bsr_to_dense(crow, col, vals, n, m)
    want = x @ (A @ B + S_dense).T + b
    crow32, col32, vt, act = orc.module_buffers(crow, col, vals)
    np.testing.assert_allclose(orc.slr_linear(x, A, B, S_dense, b), want, rtol=1e-12, atol=1e-12)
    np.testing.assert_allclose(orc.slr_linear_bsr(x, A, B, crow32, col32, vt, act, b), want,
                               rtol=1e-12, atol=1e-12)


def test_reference_rounding_emulation_is_exact_on_representable_values():
    """With small integers every intermediate is exact in bf16, so the emulation of
    the reference's four rounding points must equal the closed form exactly."""
    rng = np.random.default_rng(4)
    n, m, r, block = 32, 32, 2, 16
    NB = NBK = 2
    A = rng.integers(-1, 2, (n, r)).astype(np.float64)
    B = rng.integers(-1, 2, (r, m)).astype(np.float64)
    vals = rng.integers(-1, 2, (3, block, block)).astype(np.float64)
    crow, col, vals = orc.structure_to_bsr(np.array([0, 0, 1]), np.array([0, 1, 1]), NB, vals)
    x = rng.integers(-2, 3, (3, m)).astype(np.float64)
    b = rng.integers(-3, 4, n).astype(np.float64)
    crow32, col32, vt, act = orc.module_buffers(crow, col, vals)
    emu = orc.slr_linear_ref_rounding(x, A, B, crow32, col32, vt, act, b)
    exact = orc.slr_linear(x, A, B, orc.bsr_to_dense(crow, col, vals, n, m), b)
    assert np.array_equal(emu, exact)


def test_reference_rounding_emulation_stays_within_bf16_tolerance():
    rng = np.random.default_rng(8)
    n, m, r, block = 128, 128, 32, 32
    A, B, crow, col, vals, b = _random_slr(rng, n, m, r, block, 0.5)
    A, B, vals = orc.bf16_round(A), orc.bf16_round(B), orc.bf16_round(vals)
    b = orc.bf16_round(b)
    x = orc.bf16_round(rng.standard_normal((16, m)))
    crow32, col32, vt, act = orc.module_buffers(crow, col, vals)
    emu = orc.slr_linear_ref_rounding(x, A, B, crow32, col32, vt, act, b)
    exact = orc.slr_linear_bsr(x, A, B, crow32, col32, vt, act, b)
    err = orc.max_abs_normalised_error(emu, exact)
    assert 0 < err <= 1e-2


def test_bf16_round_known_values():
    v = np.array([1.0, 1.0 + 2**-8, 1.0 + 2**-7 + 2**-9, -3.5, 65280.0, 1e-40], dtype=np.float32)
    got = orc.bf16_round(v)
    # 1+2^-8 is a tie -> even (1.0); 1+2^-7+2^-9 rounds down to 1+2^-7
    assert got.tolist()[:4] == [1.0, 1.0, 1.0 + 2**-7, -3.5]
    assert np.array_equal(orc.bf16_round(got), got)
    t = torch.from_numpy(v).to(torch.bfloat16).float().numpy()
    assert np.array_equal(got, t)


def test_factor_from_svd_preserves_a_low_rank_matrix():
    """tests/test_ssalaad.py:276-283."""
    rng = np.random.default_rng(0)
    matrix = rng.standard_normal((16, 3)) @ rng.standard_normal((3, 32))
    U, s, Vh = np.linalg.svd(matrix, full_matrices=False)
    A, B = orc.factor_from_svd(U, s, Vh, 3)
    np.testing.assert_allclose(A @ B, matrix, atol=1e-10)
    A0, B0 = orc.factor_from_svd(U, s, Vh, 0)
    assert A0.shape == (16, 0) and B0.shape == (0, 32)


# ------------------------------------------------------ synthetic data --


def test_zipf_structure_hits_density_and_cap():
    rng = np.random.default_rng(1)
    for d in (0.1, 0.5, 0.9):
        rows, cols = orc.zipf_block_structure(64, 172, d, rng)
        assert len(rows) == round(d * 64 * 172)
        counts = np.bincount(rows, minlength=64)
        assert counts.max() <= 172
        key = rows * 172 + cols
        assert np.all(np.diff(key) > 0)  # sorted row-major, no duplicates
        if d <= 0.1:
            assert counts.max() > 3 * counts.mean()  # skewed
        elif d <= 0.5:
            assert counts.max() == 172 and counts.std() > 0.3 * counts.mean()


# ------------------------------------------------------ planted mistakes --


def test_planted_mistakes_are_caught_by_the_golden_vectors():
    """Variants of the oracle with a plausible mistake fail the golden check."""
    c = make_case("random_b16_m7")
    ref = GOLDEN["random_b16_m7__out"]

    def close(got):
        return np.max(np.abs(got - ref)) <= 1e-5 * max(1.0, np.abs(ref).max())

    good = orc.bsr_addmm_inplace(c["out"], c["x"], c["crow"], c["col"], c["values_t"], c["active"])
    assert close(good)
    # untransposed values (the (nnz, p, q) BSR layout fed where (nnz, q, p) belongs)
    wrong_t = np.ascontiguousarray(c["values_t"].transpose(0, 2, 1))
    assert not close(orc.bsr_addmm_inplace(c["out"], c["x"], c["crow"], c["col"], wrong_t, c["active"]))
    # accumulator not initialised from out
    assert not close(orc.bsr_addmm_inplace(np.zeros_like(c["out"]), c["x"], c["crow"], c["col"],
                                           c["values_t"], c["active"]))
    # off-by-one block column
    col_shift = np.minimum(c["col"] + 1, 4).astype(np.int32)
    assert not close(orc.bsr_addmm_inplace(c["out"], c["x"], c["crow"], col_shift, c["values_t"],
                                           c["active"]))


# ------------------------------------------------- block projection (_project_S) --


def _torch_project(M, n_keep, p, q):
    """The reference's selection (egar.py:296-317), written with the routines it calls."""
    M_f = torch.from_numpy(np.asarray(M, np.float32))
    n, m = M_f.shape
    rb, cb = n // p, m // q
    n_keep = min(max(n_keep, 0), rb * cb)
    keep = torch.zeros(rb * cb, dtype=torch.bool)
    if n_keep:
        blk = M_f.reshape(rb, p, cb, q).permute(0, 2, 1, 3)
        _, order = blk.pow(2).sum(dim=(2, 3)).flatten().topk(n_keep, largest=True)
        keep[order] = True
    return keep.reshape(rb, cb).numpy()


def _separated_blocks(n, m, p, q, seed):
    """Random blocks whose Frobenius norms differ by ≥ 0.1% (no near ties)."""
    rng = np.random.default_rng(seed)
    rb, cb = n // p, m // q
    M = rng.standard_normal((n, m)).astype(np.float32)
    blk = M.reshape(rb, p, cb, q)
    norms = np.sqrt((blk.astype(np.float64) ** 2).sum(axis=(1, 3)))
    target = 1.0 + 1e-3 * rng.permutation(rb * cb).reshape(rb, cb)
    blk *= (target / norms)[:, None, :, None].astype(np.float32)
    return blk.reshape(n, m)


def test_project_blocks_reference_case():
    """tests/test_ssalaad.py:215-221: the larger of two 4×4 blocks survives."""
    M = np.zeros((8, 8), np.float32)
    M[0:4, 0:4] = 3.0
    M[4:8, 4:8] = 1.0
    kept, keep = orc.project_blocks(M, 1, 4, 4)
    assert np.array_equal(kept[0:4, 0:4], M[0:4, 0:4])
    assert float(np.abs(kept[4:8, 4:8]).max()) == 0.0
    assert keep.tolist() == [[True, False], [False, False]]


@pytest.mark.parametrize("shape", [(64, 96, 16, 16), (128, 64, 32, 32), (24, 40, 4, 8), (6, 10, 1, 1)])
def test_project_blocks_matches_torch_topk_without_ties(shape):
    n, m, p, q = shape
    M = _separated_blocks(n, m, p, q, seed=n + m)
    total = (n // p) * (m // q)
    for n_keep in (1, total // 3, total // 2, total - 1):
        kept, keep = orc.project_blocks(M, n_keep, p, q)
        assert np.array_equal(keep, _torch_project(M, n_keep, p, q))
        mask = np.repeat(np.repeat(keep, p, 0), q, 1)
        assert np.array_equal(kept, np.where(mask, M, 0).astype(np.float32))


def test_project_blocks_maximises_the_kept_energy_by_brute_force():
    from itertools import combinations

    M = _separated_blocks(6, 6, 2, 3, seed=3)   # 3 × 2 = 6 blocks
    blk = M.astype(np.float64).reshape(3, 2, 2, 3)
    norms = (blk ** 2).sum(axis=(1, 3)).reshape(-1)
    for n_keep in range(7):
        best = max(combinations(range(6), n_keep), key=lambda s: sum(norms[list(s)]))
        _, keep = orc.project_blocks(M, n_keep, 2, 3)
        assert sorted(np.flatnonzero(keep.reshape(-1)).tolist()) == sorted(best)


def test_project_blocks_clamps_n_keep_and_breaks_ties_by_block_order():
    M = np.ones((4, 6), np.float32)                # six equal 2×2 blocks
    for n_keep, want in ((-2, 0), (0, 0), (3, 3), (6, 6), (9, 6)):
        kept, keep = orc.project_blocks(M, n_keep, 2, 2)
        assert int(keep.sum()) == want
        assert np.flatnonzero(keep.reshape(-1)).tolist() == list(range(want))  # lowest first
        assert kept.dtype == np.float32 and float(kept.sum()) == 4.0 * want


def test_project_blocks_counts_nan_and_inf_blocks_as_largest_like_torch():
    M = _separated_blocks(8, 8, 2, 2, seed=5)
    M[2, 3] = np.nan                               # block (1, 1)
    M[6, 0] = np.inf                               # block (3, 0)
    for n_keep in (1, 2, 3):
        _, keep = orc.project_blocks(M, n_keep, 2, 2)
        assert np.array_equal(keep, _torch_project(M, n_keep, 2, 2))
    _, keep = orc.project_blocks(M, 2, 2, 2)
    assert keep[1, 1] and keep[3, 0]


# ------------------------------------------------------- N:M projection --


def _torch_project_nm(R, nm_n, nm_m):
    """The routine egar.py:284-292 calls: |R| top-k per group, scatter, multiply."""
    R3 = torch.from_numpy(np.asarray(R, np.float32)).view(R.shape[0], -1, nm_m)
    _, top = R3.abs().topk(nm_n, dim=-1)
    mask = torch.zeros_like(R3, dtype=torch.bool)
    mask.scatter_(-1, top, True)
    return (R3 * mask.float()).view(R.shape).numpy(), mask.view(R.shape).numpy()


def _tie_free(n, m, seed):
    """Entries with distinct magnitudes (a permutation of spaced values, random signs)."""
    rng = np.random.default_rng(seed)
    mag = (1.0 + rng.permutation(n * m) * 1e-3).astype(np.float32)
    return (mag * rng.choice([-1.0, 1.0], n * m)).astype(np.float32).reshape(n, m)


def test_project_nm_reference_case():
    """tests/test_ssalaad.py:222-223."""
    R = np.array([[4.0, 1.0, 3.0, 2.0, 0.5, 9.0, 0.1, 7.0]], np.float32)
    out, mask = orc.project_nm(R, 2, 4)
    assert out[0].tolist() == [4, 0, 3, 0, 0, 9, 0, 7]
    assert mask[0].tolist() == [True, False, True, False, False, True, False, True]


@pytest.mark.parametrize("nm_n,nm_m", [(2, 4), (1, 4), (3, 4), (4, 8), (1, 2), (8, 16), (5, 7)])
def test_project_nm_matches_torch_topk_without_ties(nm_n, nm_m):
    R = _tie_free(6, 4 * nm_m, seed=nm_m)
    out, mask = orc.project_nm(R, nm_n, nm_m)
    want, wmask = _torch_project_nm(R, nm_n, nm_m)
    assert np.array_equal(mask, wmask)
    assert np.array_equal(out.view(np.uint32), want.view(np.uint32))  # bits, −0 included


def test_project_nm_keeps_the_largest_subset_by_brute_force():
    from itertools import combinations

    R = _tie_free(3, 10, seed=4)
    for nm_n in range(6):
        _, mask = orc.project_nm(R, nm_n, 5)
        for row in range(3):
            for g in range(2):
                vals = np.abs(R[row, 5 * g:5 * g + 5].astype(np.float64))
                best = max(combinations(range(5), nm_n), key=lambda s: sum(vals[list(s)]))
                assert sorted(np.flatnonzero(mask[row, 5 * g:5 * g + 5]).tolist()) == sorted(best)


def test_project_nm_closed_forms_and_special_values():
    R = np.array([[-1.0, 2.0, -0.0, np.inf, np.nan, -3.0, 0.5, 0.25]], np.float32)
    out, mask = orc.project_nm(R, 4, 4)           # keep all: R·1
    assert mask.all() and np.array_equal(out.view(np.uint32), (R * np.float32(1)).view(np.uint32))
    out, mask = orc.project_nm(R, 0, 4)           # keep none: R·0 (−0, NaN for inf and NaN)
    assert not mask.any()
    assert np.array_equal(np.isnan(out), np.isnan(R * np.float32(0)))
    assert np.signbit(out[0, 0]) and not np.signbit(out[0, 1])
    out, mask = orc.project_nm(R, 1, 4)           # NaN counts as the largest magnitude
    assert mask[0].tolist() == [False, False, False, True, True, False, False, False]
    ties = np.array([[1.0, -1.0, 1.0, 1.0]], np.float32)
    assert orc.project_nm(ties, 2, 4)[1][0].tolist() == [True, True, False, False]  # lower index
    with pytest.raises(ValueError):
        orc.project_nm(R, 2, 3)                   # m not a multiple of nm_m
    with pytest.raises(ValueError):
        orc.project_nm(R, 5, 4)
