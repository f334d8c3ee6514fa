"""The N:M projection on the GPU (ssalaad/inference/egar.py:284-292,
_project_S_nm) against the oracle, bit for bit: kept values, dropped values
(R·0, so −0 and NaN as the reference's multiply leaves them) and the mask.
On inputs without equal magnitudes in a group it is also checked against the
reference's own routine (|R|.topk per group, scatter, multiply) run by torch on
the same device. Equal magnitudes go to the lower index in both the oracle and
the kernel; which of them torch.topk keeps is unspecified (parity unpinned)."""

from __future__ import annotations

import numpy as np
import pytest
import torch

from oracle import slr_oracle as orc

import ssalaad_amd

pytestmark = pytest.mark.gpu


def _bits_equal(a: np.ndarray, b: np.ndarray) -> bool:
    """Equal bits, except that any NaN equals any NaN."""
    a = np.asarray(a, np.float32)
    b = np.asarray(b, np.float32)
    nan = np.isnan(a)
    return bool(np.array_equal(nan, np.isnan(b))
                and np.array_equal(a[~nan].view(np.uint32), b[~nan].view(np.uint32)))


def _torch_reference(R: torch.Tensor, nm_n: int, nm_m: int) -> torch.Tensor:
    n, m = R.shape
    R3 = R.float().view(n, m // nm_m, nm_m)
    _, top = R3.abs().topk(nm_n, dim=-1)
    mask = torch.zeros_like(R3, dtype=torch.bool)
    mask.scatter_(dim=-1, index=top, value=True)
    return (R3 * mask.float()).view(n, m).contiguous()


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16, torch.float16],
                         ids=["f32", "bf16", "f16"])
@pytest.mark.parametrize("nm_n,nm_m", [(2, 4), (1, 4), (3, 4), (4, 8), (1, 2), (8, 16), (5, 7),
                                       (16, 32), (0, 4), (4, 4), (1, 1)])
def test_project_nm_matches_the_oracle(dtype, nm_n, nm_m, gpu_device):
    rng = np.random.default_rng(nm_m * 31 + nm_n)
    n, m = 37, 9 * nm_m
    R = torch.from_numpy(rng.standard_normal((n, m)).astype(np.float32)).to(dtype)
    # a few exact ties and special values
    R[0, : min(4, m)] = 1.0
    R[1, 0] = -0.0
    R[2, 0] = float("nan")
    R[3, 0] = float("inf")
    R[4, 0] = -float("inf")
    out, keep = ssalaad_amd.project_nm(R.to(gpu_device), nm_n, nm_m)
    torch.cuda.synchronize()
    want, wmask = orc.project_nm(R.float().numpy(), nm_n, nm_m)
    assert np.array_equal(keep.cpu().numpy(), wmask)
    assert _bits_equal(out.cpu().numpy(), want)


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16], ids=["f32", "bf16"])
def test_project_nm_at_the_llama7b_ffn_shape_matches_torch_topk(dtype, gpu_device):
    """11008×4096, 2:4: the kernel equals the reference routine on the device
    when no group holds equal magnitudes, and the oracle in every case."""
    # each group: a random order of four distinct magnitudes (exact in bf16),
    # random signs, and a per-row power-of-two scale
    g = torch.Generator().manual_seed(2)
    order = torch.rand(11008, 1024, 4, generator=g).argsort(-1).float()
    signs = torch.randint(0, 2, (11008, 1024, 4), generator=g).float() * 2 - 1
    scale = 2.0 ** torch.randint(-6, 6, (11008, 1, 1), generator=g).float()
    R = ((1.0 + order / 4.0) * signs * scale).reshape(11008, 4096).to(dtype)
    Rd = R.to(gpu_device)
    out = ssalaad_amd.project_S_nm(Rd, 2, 4)
    ref = _torch_reference(Rd, 2, 4)
    torch.cuda.synchronize()
    assert torch.equal(out, ref)
    rows = slice(0, 512)  # the oracle on a slice (it is slow at full size)
    assert _bits_equal(out[rows].cpu().numpy(), orc.project_nm(R[rows].float().numpy(), 2, 4)[0])


def test_project_nm_reference_case_and_strided_input(gpu_device):
    R = torch.tensor([[4.0, 1.0, 3.0, 2.0, 0.5, 9.0, 0.1, 7.0]], device=gpu_device)
    assert ssalaad_amd.project_S_nm(R, 2, 4)[0].tolist() == [4, 0, 3, 0, 0, 9, 0, 7]
    big = torch.randn(20, 48, device=gpu_device)
    view = big[:, 8:40]                      # rows with a stride of 48
    out = ssalaad_amd.project_S_nm(view, 2, 4)
    want, _ = orc.project_nm(view.cpu().numpy(), 2, 4)
    assert _bits_equal(out.cpu().numpy(), want)


@pytest.mark.parametrize("nm_n,nm_m", [(2, 4), (4, 8), (8, 16)])
def test_project_nm_misaligned_rows_take_the_scalar_path(nm_n, nm_m, gpu_device):
    """Groups that start 8 bytes past a 16-byte boundary (an fp32 view from
    column 2, rows of 3·nm_m + 6 columns) take the per-element path, with the
    same results."""
    big = torch.randn(33, 3 * nm_m + 6, device=gpu_device)
    view = big[:, 2:2 + 3 * nm_m]
    assert view.data_ptr() % 16 != 0
    out, keep = ssalaad_amd.project_nm(view, nm_n, nm_m)
    want, wmask = orc.project_nm(view.cpu().numpy(), nm_n, nm_m)
    assert np.array_equal(keep.cpu().numpy(), wmask)
    assert _bits_equal(out.cpu().numpy(), want)


def test_project_nm_rejects_what_the_reference_rejects(gpu_device):
    R = torch.randn(4, 10, device=gpu_device)
    with pytest.raises(RuntimeError, match="invalid for input of size"):
        ssalaad_amd.project_S_nm(R, 2, 4)     # 10 is not a multiple of 4
    with pytest.raises(RuntimeError, match="out of range"):
        ssalaad_amd.project_S_nm(R, 3, 2)
    empty = ssalaad_amd.project_S_nm(torch.empty(0, 8, device=gpu_device), 2, 4)
    assert empty.shape == (0, 8)
