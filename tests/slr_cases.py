"""Seeded SLR-linear problems for the parity tests: NumPy master copies (for the
oracle) and matching torch tensors (for the HIP path)."""

from __future__ import annotations

import numpy as np
import torch

from oracle import slr_oracle as orc

TOL = {torch.float32: 1e-5, torch.bfloat16: 1e-2, torch.float16: 1e-2}


def round_to(a: np.ndarray, dtype: torch.dtype) -> np.ndarray:
    """Values exactly representable in `dtype`, as float64."""
    return torch.from_numpy(np.asarray(a, dtype=np.float32)).to(dtype).double().numpy()


def make_problem(n, m, r, p, density, dtype, seed=0, skew=False, bias=True, pad=False, q=None):
    """A random SLR linear with (p, q) blocks (q = p by default). With pad=True,
    n and m need not be multiples of the block: S is stored at the padded shape
    (ceil(n/p)·p, ceil(m/q)·q) with zero padding."""
    q = p if q is None else q
    rng = np.random.default_rng(seed)
    NB, NBK = -(-n // p), -(-m // q)
    if not pad:
        assert n % p == 0 and m % q == 0
    if skew:
        rows, cols = orc.zipf_block_structure(NB, NBK, density, rng)
    else:
        rows, cols = orc.random_block_structure(NB, NBK, density, rng)
    vals = rng.standard_normal((len(rows), p, q)) * 0.02
    # zero the padded rows/columns of edge blocks
    for k, (br, bc) in enumerate(zip(rows, cols)):
        if (br + 1) * p > n:
            vals[k, n - br * p:, :] = 0
        if (bc + 1) * q > m:
            vals[k, :, m - bc * q:] = 0
    vals = round_to(vals, dtype)
    crow, col, vals = orc.structure_to_bsr(rows, cols, NB, vals)
    A = round_to(rng.standard_normal((n, r)) * 0.02, dtype)
    B = round_to(rng.standard_normal((r, m)) * 0.02, dtype)
    b = round_to(rng.standard_normal(n) * 0.1, dtype) if bias else None
    return dict(n=n, m=m, r=r, p=p, q=q, NB=NB, NBK=NBK, crow=crow, col=col, vals=vals, A=A,
                B=B, bias=b, dtype=dtype, rng=rng)


def s_dense(prob) -> np.ndarray:
    full = orc.bsr_to_dense(prob["crow"], prob["col"], prob["vals"], prob["NB"] * prob["p"],
                            prob["NBK"] * prob["q"])
    return full[: prob["n"], : prob["m"]]


def sparse_bsr_tensor(prob, device) -> torch.Tensor:
    p = prob["p"]
    return torch.sparse_bsr_tensor(
        torch.from_numpy(prob["crow"]).to(device),
        torch.from_numpy(prob["col"]).to(device),
        torch.from_numpy(prob["vals"]).to(device=device, dtype=prob["dtype"]),
        size=(prob["NB"] * p, prob["NBK"] * prob["q"]),
    )


def make_x(prob, M, seed=1) -> np.ndarray:
    rng = np.random.default_rng(seed)
    return round_to(rng.standard_normal((M, prob["m"])), prob["dtype"])


def oracle_y(prob, x) -> np.ndarray:
    return orc.slr_linear(x, prob["A"], prob["B"], s_dense(prob), prob["bias"])


def to_dev(a, dtype, device):
    return torch.from_numpy(np.ascontiguousarray(a)).to(device=device, dtype=dtype)


def err(y_gpu: torch.Tensor, y_ref: np.ndarray) -> float:
    return orc.max_abs_normalised_error(y_gpu.double().cpu().numpy(), y_ref)


def make_module(prob, dev, bias=True):
    """The package's LRSLinear for a problem (BSR S on the device)."""
    from ssalaad_amd import LRSLinear

    dt = prob["dtype"]
    S = sparse_bsr_tensor(prob, dev)
    return LRSLinear(
        to_dev(prob["A"], dt, dev), to_dev(prob["B"], dt, dev), S,
        in_features=prob["m"], out_features=prob["n"],
        bias=to_dev(prob["bias"], dt, dev) if (bias and prob["bias"] is not None) else None,
        block_p=prob["p"], block_q=prob["q"],
    )
