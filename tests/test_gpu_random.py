"""Seeded random sweeps against the oracle: the fused SLR linear, the device
encoder (dense -> BSR, bit-exact structure and values) and the block projection.

Each case draws its shape (feature counts that need not be block multiples),
rank, block size, density, row structure (uniform or Zipf), dtype, bias and
token count (decode and prefill paths alike) from one seed, builds one to three
linears that read the same x, runs them as a group and one by one, and checks:
  * every output against the float64 oracle (fp32 1e-5, 16-bit 1e-2);
  * the grouped outputs equal the single-linear outputs bit for bit;
  * no latent wait gave up.
A failure names its seed; the case can be rebuilt alone with `_case(seed)`.
The encoder and projection sweeps draw block shapes from 1 to 64 (not square
too) and compare structure, values and keep masks exactly; the in-place op
sweep checks active block-rows against the oracle and every other row's bits.
"""

from __future__ import annotations

import sys
from pathlib import Path

import numpy as np
import pytest
import torch

sys.path.insert(0, str(Path(__file__).resolve().parent))
from slr_cases import TOL, err, make_problem, make_x, oracle_y, sparse_bsr_tensor, to_dev  # noqa: E402

import ssalaad_amd  # noqa: E402
from oracle import slr_oracle as orc  # noqa: E402
from ssalaad_amd import LRSLinear  # noqa: E402
from ssalaad_amd.ls_linear import latent_wait_status  # noqa: E402

pytestmark = pytest.mark.gpu

DTYPES = (torch.float32, torch.bfloat16, torch.float16)


SIDES_P = [16, 32, 48, 64, 96, 128]
SIDES_Q = [16, 32, 48, 64, 80, 96, 320]


def _block(rng) -> tuple[int, int]:
    """Square 16/32/64 half the time (the shapes the prefill kernels take),
    else any (p, q) with sides multiples of 16, including tiles wider than 64
    and blocks deeper than 256 (cut into sub-blocks by the kernel view)."""
    if rng.integers(2):
        p = int(rng.choice([16, 32, 64]))
        return p, p
    return int(rng.choice(SIDES_P)), int(rng.choice(SIDES_Q))


def _case(seed: int) -> dict:
    rng = np.random.default_rng(1000 + seed)
    p, q = _block(rng)
    dtype = DTYPES[int(rng.integers(3))]
    m = int(rng.integers(1, 40)) * 16 + int(rng.choice([0, 0, 5, 11]))
    M = int(rng.choice([1, 2, 7, 16, 33, 64, 100, 130, 257]))
    members = []
    for _ in range(int(rng.integers(1, 4))):
        n = int(rng.integers(1, 30)) * 16 + int(rng.choice([0, 0, 3, 9]))
        members.append(dict(n=n, r=int(rng.choice([8, 32, 64, 96, 256])),
                            d=float(rng.choice([0.1, 0.3, 0.5, 0.9])),
                            skew=bool(rng.integers(2)), bias=bool(rng.integers(2))))
    return dict(p=p, q=q, dtype=dtype, m=m, M=M, members=members, seed=seed)


def _module(prob, dev, bias):
    dt = prob["dtype"]
    return LRSLinear(
        to_dev(prob["A"], dt, dev), to_dev(prob["B"], dt, dev), sparse_bsr_tensor(prob, dev),
        in_features=prob["m"], out_features=prob["n"],
        bias=to_dev(prob["bias"], dt, dev) if bias else None, block_p=prob["p"],
        block_q=prob["q"],
    )


@pytest.mark.parametrize("seed", range(64))
def test_random_slr_linears_match_the_oracle(seed, gpu_device):
    c = _case(seed)
    probs = [make_problem(mb["n"], c["m"], mb["r"], c["p"], mb["d"], c["dtype"],
                          seed=seed * 7 + i, skew=mb["skew"], bias=mb["bias"], pad=True, q=c["q"])
             for i, mb in enumerate(c["members"])]
    mods = [_module(pr, gpu_device, mb["bias"]) for pr, mb in zip(probs, c["members"])]
    x = make_x(probs[0], c["M"], seed=seed)
    xt = to_dev(x, c["dtype"], gpu_device)
    singles = [mod(xt) for mod in mods]
    # an S with no stored block makes a low-rank-only linear, whose output tile
    # differs from the block linears': such members are not grouped
    groupable = len({mod._kernel_block for mod in mods}) == 1
    grouped = ssalaad_amd.LRSLinearGroup(*mods)(xt) if groupable else singles
    torch.cuda.synchronize()
    for y, yg, pr in zip(singles, grouped, probs):
        assert y.shape == (c["M"], pr["n"])
        assert err(y, oracle_y(pr, x)) <= TOL[c["dtype"]], c
        assert torch.equal(y, yg), c
    assert latent_wait_status(gpu_device) == 0, c


# ------------------------------------------------ encoder and projection --

_BITS = {torch.float32: torch.int32, torch.bfloat16: torch.int16, torch.float16: torch.int16}
_SIZES = (1, 2, 4, 8, 16, 32, 64)


def _random_dense(rng, rb, cb, p, q, dtype) -> torch.Tensor:
    """Blocks drawn as zero, dense, one non-zero, -0.0, NaN, inf or subnormal."""
    S = np.zeros((rb * p, cb * q), np.float32)
    kinds = rng.choice(7, size=(rb, cb), p=[0.35, 0.3, 0.1, 0.05, 0.07, 0.06, 0.07])
    tiny = {torch.float32: 1e-40, torch.bfloat16: 1e-40, torch.float16: 1e-7}[dtype]
    for r in range(rb):
        for c in range(cb):
            blk = S[r * p:(r + 1) * p, c * q:(c + 1) * q]
            i, j = rng.integers(p), rng.integers(q)
            k = kinds[r, c]
            if k == 1:
                blk[:] = rng.standard_normal((p, q))
            elif k == 2:
                blk[i, j] = rng.standard_normal()
            elif k == 3:
                blk[:] = -0.0
            elif k == 4:
                blk[i, j] = np.nan
            elif k == 5:
                blk[i, j] = np.inf * rng.choice([-1, 1])
            elif k == 6:
                blk[i, j] = tiny
    return torch.from_numpy(S).to(dtype)


@pytest.mark.parametrize("seed", range(24))
def test_random_encoder_structure_is_bit_exact(seed, gpu_device):
    rng = np.random.default_rng(5000 + seed)
    p, q = int(rng.choice(_SIZES)), int(rng.choice(_SIZES))
    rb, cb = int(rng.integers(1, 13)), int(rng.integers(1, 13))
    dtype = DTYPES[int(rng.integers(3))]
    S = _random_dense(rng, rb, cb, p, q, dtype)
    crow, col, vals = orc.dense_to_bsr(S.float().numpy(), p, q)
    crow32, col32, _, act = orc.module_buffers(crow, col, vals)
    k_crow, k_col, k_vt, k_act = ssalaad_amd.encode_for_kernels(S.to(gpu_device), p, q)
    bsr = ssalaad_amd.dense_to_bsr(S.to(gpu_device), p, q)
    torch.cuda.synchronize()
    case = (seed, p, q, rb, cb, dtype)
    assert np.array_equal(k_crow.cpu().numpy(), crow32), case
    assert np.array_equal(k_col.cpu().numpy(), col32), case
    assert np.array_equal(k_act.cpu().numpy(), act), case
    assert np.array_equal(bsr.crow_indices().cpu().numpy(), crow), case
    assert np.array_equal(bsr.col_indices().cpu().numpy(), col), case
    bits = _BITS[dtype]
    S_bits = S.view(bits).numpy()
    rows = np.repeat(np.arange(rb), np.diff(crow))
    want = (np.stack([S_bits[r * p:(r + 1) * p, c * q:(c + 1) * q] for r, c in zip(rows, col)])
            if len(col) else np.zeros((0, p, q), S_bits.dtype))
    assert np.array_equal(bsr.values().cpu().view(bits).numpy(), want), case
    assert np.array_equal(k_vt.cpu().view(bits).numpy(), want.transpose(0, 2, 1)), case


@pytest.mark.parametrize("seed", range(24))
def test_random_block_projection_matches_the_oracle(seed, gpu_device):
    """Block norms separated by construction (each block scaled by a distinct
    power of 1.05), so the top-k selection is the same in fp32 and float64."""
    rng = np.random.default_rng(7000 + seed)
    p, q = int(rng.choice(_SIZES)), int(rng.choice(_SIZES))
    rb, cb = int(rng.integers(1, 17)), int(rng.integers(1, 17))
    dtype = (torch.float32, torch.bfloat16)[int(rng.integers(2))]
    M = rng.standard_normal((rb * p, cb * q))
    M /= np.sqrt((M.reshape(rb, p, cb, q) ** 2).sum(axis=(1, 3)))[:, None, :, None].repeat(
        p, 1).repeat(q, 3).reshape(rb * p, cb * q)
    scale = 1.05 ** rng.permutation(rb * cb).reshape(rb, cb)
    M *= np.repeat(np.repeat(scale, p, axis=0), q, axis=1)
    Md = torch.from_numpy(M.astype(np.float32)).to(dtype)
    total = rb * cb
    n_keep = int(rng.integers(-2, total + 3))
    out, keep, _ = ssalaad_amd.block_topk(Md.to(gpu_device), n_keep, p, q)
    torch.cuda.synchronize()
    want, want_keep = orc.project_blocks(Md.float().numpy(), n_keep, p, q)
    case = (seed, p, q, rb, cb, dtype, n_keep)
    assert np.array_equal(keep.cpu().numpy(), want_keep), case
    assert np.array_equal(out.cpu().numpy(), want), case


# ------------------------------------------------------- in-place op --


@pytest.mark.parametrize("seed", range(40))
def test_random_inplace_op_matches_the_oracle(seed, gpu_device):
    """torch.ops.ssalaad.tilelang_bsr_addmm_inplace_dense_ on random shapes,
    block sizes, dtypes and token counts (decode and prefill kernels), with
    `active_rows` a random subset of the block-rows that hold blocks: active
    rows match the oracle, every other row keeps its bits."""
    import ssalaad_amd.addmm_inplace  # noqa: F401  (registers the op)

    rng = np.random.default_rng(9000 + seed)
    p, q = _block(rng)
    dtype = DTYPES[int(rng.integers(3))]
    NB, NBK = int(rng.integers(1, 13)), int(rng.integers(1, 13))
    M = int(rng.choice([1, 5, 16, 64, 65, 130, 300]))
    prob = make_problem(NB * p, NBK * q, 4, p, float(rng.choice([0.2, 0.5, 0.9])), dtype,
                        seed=seed, skew=bool(rng.integers(2)), q=q)
    crow32, col32, vt, act_all = orc.module_buffers(prob["crow"], prob["col"], prob["vals"])
    act = np.sort(rng.permutation(act_all)[: int(rng.integers(0, len(act_all) + 1))]).astype(np.int32)
    x = make_x(prob, M, seed=seed)
    out0 = torch.from_numpy(rng.standard_normal((M, NB * p))).to(dtype).double().numpy()
    want = orc.bsr_addmm_inplace(out0, x, crow32, col32, vt, act)
    dev = gpu_device
    out = to_dev(out0, dtype, dev)
    torch.ops.ssalaad.tilelang_bsr_addmm_inplace_dense_(
        out, to_dev(x, dtype, dev), torch.from_numpy(crow32).to(dev),
        torch.from_numpy(col32).to(dev), to_dev(vt, dtype, dev), torch.from_numpy(act).to(dev))
    torch.cuda.synchronize()
    case = (seed, p, q, dtype, NB, NBK, M, len(act))
    got = out.double().cpu().numpy()
    cols = np.zeros(NB * p, bool)
    for by in act:
        cols[by * p:(by + 1) * p] = True
    if cols.any():
        assert err(out[:, torch.from_numpy(cols).to(dev)], want[:, cols]) <= TOL[dtype], case
    assert np.array_equal(got[:, ~cols], out0[:, ~cols]), case
