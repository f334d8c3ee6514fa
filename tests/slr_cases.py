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
    if n % p:
        vals[np.asarray(rows) == NB - 1, n % p:, :] = 0
    if m % q:
        vals[np.asarray(cols) == NBK - 1, :, m % q:] = 0
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


def nm24_matrix(n, m, seed, dtype) -> np.ndarray:
    """Random 2:4 S (0, 1 or 2 non-zeros in every group of four input features)."""
    rng = np.random.default_rng(seed)
    count = rng.choice(3, size=(n, m // 4), p=[0.15, 0.25, 0.6])        # kept per group
    rank = np.argsort(rng.random((n, m // 4, 4)), axis=-1).argsort(axis=-1)  # random order
    keep = rank < count[..., None]
    S = (rng.standard_normal((n, m // 4, 4)) * 0.05 * keep).reshape(n, m)
    return torch.from_numpy(S).to(dtype).double().numpy()


def make_nm_module(n, m, r, dtype, dev, seed, bias=True):
    """The package's LRSLinear with a 2:4 S, and its (A, B, S, bias) master copies."""
    from ssalaad_amd import LRSLinear

    rng = np.random.default_rng(seed + 1)
    A = rng.standard_normal((n, r)) * 0.05
    B = rng.standard_normal((r, m)) * 0.05
    b = rng.standard_normal(n) * 0.1 if bias else None
    A, B = (torch.from_numpy(t).to(dtype).double().numpy() for t in (A, B))
    if b is not None:
        b = torch.from_numpy(b).to(dtype).double().numpy()
    S = nm24_matrix(n, m, seed, dtype)
    mod = LRSLinear(to_dev(A, dtype, dev), to_dev(B, dtype, dev), to_dev(S, dtype, dev),
                    in_features=m, out_features=n,
                    bias=None if b is None else to_dev(b, dtype, dev), nm_n=2, nm_m=4)
    return mod, (A, B, S, b)
