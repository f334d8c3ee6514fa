"""Seeded random sweep of the fused SLR linear against the oracle.

Each case draws its shape (feature counts that need not be block multiples),
rank, block size, density, row structure (uniform or Zipf), dtype, bias and
token count (decode and prefill paths alike) from one seed, builds one to three
linears that read the same x, runs them as a group and one by one, and checks:
  * every output against the float64 oracle (fp32 1e-5, 16-bit 1e-2);
  * the grouped outputs equal the single-linear outputs bit for bit;
  * no latent wait gave up.
A failure names its seed; the case can be rebuilt alone with `_case(seed)`.
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
from ssalaad_amd import LRSLinear  # noqa: E402
from ssalaad_amd.ls_linear import latent_wait_status  # noqa: E402

pytestmark = pytest.mark.gpu

DTYPES = (torch.float32, torch.bfloat16, torch.float16)


def _case(seed: int) -> dict:
    rng = np.random.default_rng(1000 + seed)
    p = int(rng.choice([16, 32, 64]))
    dtype = DTYPES[int(rng.integers(3))]
    m = int(rng.integers(1, 40)) * 16 + int(rng.choice([0, 0, 5, 11]))
    M = int(rng.choice([1, 2, 7, 16, 33, 64, 100, 130, 257]))
    members = []
    for _ in range(int(rng.integers(1, 4))):
        n = int(rng.integers(1, 30)) * 16 + int(rng.choice([0, 0, 3, 9]))
        members.append(dict(n=n, r=int(rng.choice([8, 32, 64, 96, 256])),
                            d=float(rng.choice([0.1, 0.3, 0.5, 0.9])),
                            skew=bool(rng.integers(2)), bias=bool(rng.integers(2))))
    return dict(p=p, dtype=dtype, m=m, M=M, members=members, seed=seed)


def _module(prob, dev, bias):
    dt = prob["dtype"]
    return LRSLinear(
        to_dev(prob["A"], dt, dev), to_dev(prob["B"], dt, dev), sparse_bsr_tensor(prob, dev),
        in_features=prob["m"], out_features=prob["n"],
        bias=to_dev(prob["bias"], dt, dev) if bias else None, block_p=prob["p"],
        block_q=prob["p"],
    )


@pytest.mark.parametrize("seed", range(48))
def test_random_slr_linears_match_the_oracle(seed, gpu_device):
    c = _case(seed)
    probs = [make_problem(mb["n"], c["m"], mb["r"], c["p"], mb["d"], c["dtype"],
                          seed=seed * 7 + i, skew=mb["skew"], bias=mb["bias"], pad=True)
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
