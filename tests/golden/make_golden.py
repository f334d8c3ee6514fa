"""Write golden vectors of the reference AVX2 BSR kernel.

Runs the reference kernel ssalaad/cpu_sparse/bsr_addmm_avx2.cpp, compiled from
its own source into oracle/_ref by `make -C oracle ref` (the source is never
copied into this repository), on seeded inputs and stores inputs' seeds and
shapes plus the kernel's fp32 outputs in bsr_addmm_avx2.npz.

Inputs are regenerated from the seeds by tests/golden/golden_inputs.py with
NumPy's PCG64 generator, so only small arrays are stored. Cases:
  * blocks 8/16/32/64 with the block pattern of the reference's own test
    (tests/test_ssalaad.py:320-327: S of (4·B, 6·B), blocks
    (0,1),(1,0),(1,3),(2,5),(3,2), x of 5 rows, out zero);
  * the untouched-rows case of tests/test_ssalaad.py:330-337 (out filled with 7);
  * random structures at 50% density with non-zero `out`, M = 1, 7, 64;
  * the fp32 single-SLR-linear shape (512×512, 32×32 blocks, 50%) at M = 64 rows.
Run: python tests/golden/make_golden.py   (needs oracle/_ref built)
"""

from __future__ import annotations

import sys
from pathlib import Path

import numpy as np

HERE = Path(__file__).resolve().parent
ROOT = HERE.parents[1]
sys.path.insert(0, str(HERE))
sys.path.insert(0, str(ROOT / "oracle" / "_ref"))

import torch  # noqa: E402

from golden_inputs import CASES, make_case  # noqa: E402


def main() -> None:
    import bsr_ref_avx2  # built by `make -C oracle ref`

    arrays = {}
    for name in CASES:
        c = make_case(name)
        out = torch.from_numpy(c["out"].copy())
        bsr_ref_avx2.bsr_addmm_avx2_(
            out,
            torch.from_numpy(c["x"]),
            torch.from_numpy(c["crow"]),
            torch.from_numpy(c["col"]),
            torch.from_numpy(c["values_t"]),
            torch.from_numpy(c["active"]),
        )
        arrays[f"{name}__out"] = out.numpy()
    np.savez_compressed(HERE / "bsr_addmm_avx2.npz", **arrays)
    print(f"wrote {len(arrays)} golden outputs to {HERE / 'bsr_addmm_avx2.npz'}")


if __name__ == "__main__":
    main()
