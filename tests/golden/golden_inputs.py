"""Deterministic inputs of the golden cases (NumPy PCG64, seeded per case).

Shared by make_golden.py (which runs the reference kernel on them) and the
tests (which rebuild the same inputs and compare against the stored outputs).
The BSR buffers follow the module conversion of ssalaad/efficient/ls_linear.py:89-97:
int32 crow/col, values transposed per block to (nnz, q, p), active block-rows.
"""

from __future__ import annotations

import numpy as np

REF_TEST_COORDS = [(0, 1), (1, 0), (1, 3), (2, 5), (3, 2)]

CASES = [
    "reftest_b8", "reftest_b16", "reftest_b32", "reftest_b64",
    "untouched_b16",
    "random_b16_m7", "random_b32_m1", "random_b64_m64", "random_b8_m9",
    "slr512_b32_m64",
]


def _bsr_from_coords(n, m, block, coords, rng):
    S = np.zeros((n, m), dtype=np.float32)
    for br, bc in coords:
        S[br * block:(br + 1) * block, bc * block:(bc + 1) * block] = rng.standard_normal(
            (block, block), dtype=np.float32)
    return S


def _to_kernel_buffers(S, block):
    n, m = S.shape
    rb, cb = n // block, m // block
    blocks = S.reshape(rb, block, cb, block).transpose(0, 2, 1, 3)
    mask = np.abs(blocks.astype(np.float64)).reshape(rb, cb, -1).sum(-1) > 0
    crow = np.concatenate([[0], np.cumsum(mask.sum(1))]).astype(np.int32)
    r, c = np.nonzero(mask)
    values_t = np.ascontiguousarray(blocks[r, c].transpose(0, 2, 1)).astype(np.float32)
    active = np.nonzero(np.diff(crow))[0].astype(np.int32)
    return crow, c.astype(np.int32), values_t, active


def make_case(name: str) -> dict:
    seed = CASES.index(name) + 1000
    rng = np.random.default_rng(seed)
    if name.startswith("reftest_b"):
        block = int(name[len("reftest_b"):])
        S = _bsr_from_coords(block * 4, block * 6, block, REF_TEST_COORDS, rng)
        x = rng.standard_normal((5, block * 6), dtype=np.float32)
        out = np.zeros((5, block * 4), dtype=np.float32)
    elif name == "untouched_b16":
        block = 16
        S = _bsr_from_coords(block * 3, block * 3, block, [(2, 0)], rng)
        x = rng.standard_normal((3, block * 3), dtype=np.float32)
        out = np.full((3, block * 3), 7.0, dtype=np.float32)
    elif name.startswith("random_b"):
        block = int(name.split("_")[1][1:])
        M = int(name.split("_")[2][1:])
        NB, NBK = 6, 5
        slots = np.sort(rng.permutation(NB * NBK)[: (NB * NBK) // 2])
        coords = [(s // NBK, s % NBK) for s in slots]
        S = _bsr_from_coords(NB * block, NBK * block, block, coords, rng)
        x = rng.standard_normal((M, NBK * block), dtype=np.float32)
        out = rng.standard_normal((M, NB * block), dtype=np.float32)
    elif name == "slr512_b32_m64":
        block, NB = 32, 16
        slots = np.sort(rng.permutation(NB * NB)[:128])
        coords = [(s // NB, s % NB) for s in slots]
        S = _bsr_from_coords(512, 512, block, coords, rng) * np.float32(0.02)
        x = rng.standard_normal((64, 512), dtype=np.float32)
        out = np.zeros((64, 512), dtype=np.float32)
    else:
        raise KeyError(name)
    crow, col, values_t, active = _to_kernel_buffers(S, block)
    return dict(S=S, x=x, out=out, crow=crow, col=col, values_t=values_t, active=active,
                block=block)
