"""The benchmark workloads at full size, every output row against the oracle.

Each case is one SLR linear y = x·Bᵀ·Aᵀ + x·Sᵀ + b (the forward of
ssalaad/efficient/ls_linear.py:124-137) built by LRSLinear and called as a
user calls it: the library picks streaming or tiled kernels, the row tile and
the K parts itself. bf16, x ~ N(0, 1), A, B, S values ~ N(0, 0.02), seeded.

  * LLaMA-1B projections: q/k/v/o 2048×2048, gate/up 5461×2048, down
    2048×5461 (S stored at the 32-multiple padded shape), rank 256, 32×32
    blocks at 50%, 1 / 4 / 16 / 2048 tokens;
  * LLaMA-7B layer set: 4096×4096, 11008×4096 and 4096×11008, rank 256, 64×64
    blocks at 30 / 50 / 70% density, 1 / 16 / 256 / 2048 tokens;
  * skewed structures: 4096×11008, rank 128, 16/32/64 blocks whose per-row
    block counts follow Zipf(1.2) at 10 / 50 / 90% mean density, 1 and 2048
    tokens.

One weight set and one 2048-row oracle output per (shape, block, density),
kept while its token counts run; smaller calls take the first rows.
"""

from __future__ import annotations

import zlib

import pytest
import torch

from slr_cases import TOL, err, make_module, make_problem, make_x, oracle_y, round_to, to_dev

from ssalaad_amd import _runtime
from ssalaad_amd.ls_linear import latent_wait_status

pytestmark = pytest.mark.gpu

_CACHE: dict = {}


def _setup(key, n, m, r, p, density, skew, dev):
    """(problem, module, x [2048, m], y_ref [2048, n]) for a weight set, built
    once; the previous set is dropped."""
    if key not in _CACHE:
        _CACHE.clear()
        torch.cuda.empty_cache()
        seed = zlib.crc32(repr(key).encode())
        prob = make_problem(n, m, r, p, density, torch.bfloat16, seed=seed, skew=skew,
                            pad=(n % p != 0 or m % p != 0))
        x = make_x(prob, 2048, seed=seed + 1)
        _CACHE[key] = (prob, make_module(prob, dev), x, oracle_y(prob, x))
    return _CACHE[key]


def _check(key, n, m, r, p, density, skew, M, dev):
    prob, mod, x, want = _setup(key, n, m, r, p, density, skew, dev)
    print(f"[config] {key} M={M}", flush=True)
    y = mod(to_dev(x[:M], torch.bfloat16, dev))
    torch.cuda.synchronize()
    assert y.shape == (M, n)
    e = err(y, want[:M])
    assert e <= TOL[torch.bfloat16], (key, M, e)
    assert latent_wait_status(dev) == 0
    assert all(int(buf.abs().max()) == 0 for (idx, _), buf in _runtime._COUNTERS.items()
               if idx == dev.index)


_1B = [(n, m) for n, m in ((2048, 2048), (5461, 2048), (2048, 5461))]


@pytest.mark.parametrize("shape,M", [(s, M) for s in _1B for M in (1, 4, 16, 2048)],
                         ids=[f"{n}x{m}-M{M}" for n, m in _1B for M in (1, 4, 16, 2048)])
def test_llama1b_projections(shape, M, gpu_device):
    n, m = shape
    _check(("1b", n, m), n, m, 256, 32, 0.5, False, M, gpu_device)


_7B = [(n, m, d) for n, m in ((4096, 4096), (11008, 4096), (4096, 11008)) for d in (0.3, 0.5, 0.7)]


@pytest.mark.parametrize("case,M", [(c, M) for c in _7B for M in (1, 16, 256, 2048)],
                         ids=[f"{n}x{m}-d{d}-M{M}" for n, m, d in _7B for M in (1, 16, 256, 2048)])
def test_llama7b_layer_set(case, M, gpu_device):
    n, m, d = case
    _check(("7b", n, m, d), n, m, 256, 64, d, False, M, gpu_device)


_SKEW = [(p, d) for p in (16, 32, 64) for d in (0.1, 0.5, 0.9)]


@pytest.mark.parametrize("case,M", [(c, M) for c in _SKEW for M in (1, 2048)],
                         ids=[f"p{p}-zipf{d}-M{M}" for p, d in _SKEW for M in (1, 2048)])
def test_skewed_structures(case, M, gpu_device):
    p, d = case
    _check(("skew", p, d), 4096, 11008, 128, p, d, True, M, gpu_device)



@pytest.mark.parametrize("M", [128, 256, 2048])
def test_low_rank_only_llama7b_ffn(M, gpu_device):
    """S = 0 (the low-rank-only module, ssalaad/efficient/ls_linear.py:47-54) at
    the 7B FFN shape: the latent over 4096 in_features is the rows' whole wait,
    so it splits into K chunks whose fp32 partials are summed in chunk order."""
    import numpy as np

    from oracle import slr_oracle as orc
    from ssalaad_amd import LRSLinear

    n, m, r = 11008, 4096, 256
    rng = np.random.default_rng(M)
    A = round_to(rng.standard_normal((n, r)) * 0.02, torch.bfloat16)
    B = round_to(rng.standard_normal((r, m)) * 0.02, torch.bfloat16)
    b = round_to(rng.standard_normal(n) * 0.1, torch.bfloat16)
    x = round_to(rng.standard_normal((M, m)), torch.bfloat16)
    dev = gpu_device
    mod = LRSLinear(to_dev(A, torch.bfloat16, dev), to_dev(B, torch.bfloat16, dev),
                    torch.zeros(n, m, dtype=torch.bfloat16, device=dev), in_features=m,
                    out_features=n, bias=to_dev(b, torch.bfloat16, dev))
    assert mod.kind == "lr_only"
    print(f"[config] lr-only 11008x4096 r256 M={M}", flush=True)
    y1, y2 = mod(to_dev(x, torch.bfloat16, dev)), mod(to_dev(x, torch.bfloat16, dev))
    torch.cuda.synchronize()
    want = orc.slr_linear(x, A, B, np.zeros((n, m)), b)
    assert err(y1, want) <= TOL[torch.bfloat16]
    assert torch.equal(y1, y2)
    assert latent_wait_status(dev) == 0
    assert all(int(buf.abs().max()) == 0 for (idx, _), buf in _runtime._COUNTERS.items()
               if idx == dev.index)
