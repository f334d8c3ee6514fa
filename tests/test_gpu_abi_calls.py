"""Fused calls made directly through the C ABI with arguments the Python layer
never sends, checked against the oracle.

A linear with no low-rank factor (r_pad 0, lr_wgs 0, A and B null) is a valid
ssl_slr_member: y = x·Sᵀ + b. It has no latent tiles and no latent tile
counters, so on the prefill kernels its row workgroups must neither wait for
a latent nor count themselves out of one. Each case checks every output row,
that the call took the kernels it names, and that the zero-at-rest counters
are zero again. The forward is ssalaad/efficient/ls_linear.py:124-137 with
the low-rank term absent (the reference's S-only linear is its op alone,
ssalaad/tilelang_sparse/addmm_inplace.py:41-82, plus the bias).
"""

from __future__ import annotations

import numpy as np
import pytest
import torch

from oracle import slr_oracle as orc
from slr_cases import TOL, err, make_module, make_nm_module, make_problem, make_x, s_dense, to_dev

from ssalaad_amd import _lib, _runtime
from ssalaad_amd.ls_linear import _members

pytestmark = pytest.mark.gpu


def _s_only_call(mod, x: torch.Tensor, prefill: bool) -> torch.Tensor:
    """One ssl_slr_forward_group call of `mod`'s S and bias alone."""
    lib = _lib.load()
    st = mod._kernel()
    M = x.shape[0]
    nm = st.s_format == 1
    takes = (lib.ssl_nm24_takes_prefill(M, st.NB, st.dtype_code) if nm
             else lib.ssl_slr_takes_prefill(M, st.NB, st.p, st.q, st.dtype_code))
    assert bool(takes) == prefill
    G = int(lib.ssl_prefill_group(M, st.NB, st.p, st.q)) if prefill else 0
    y = torch.empty(M, st.n_pad, dtype=x.dtype, device=x.device)
    members, _ = _members([st], [y], M, G)
    # a plan without low-rank units, and no factor
    table, n_chunks, n_slots = _runtime.build_plan(st.crow_h, st.col_h, st.NBK, None, st.block_q,
                                                   0, 0)
    plan = _runtime.DevicePlan(table, n_chunks, n_slots, x.device)
    mb = members[0]
    mb.plan, mb.n_chunks, mb.n_slots, mb.lr_wgs = plan.table.data_ptr(), n_chunks, n_slots, 0
    mb.r_pad = 0
    mb.A = mb.B = None
    xch = plan.exchange(lib.ssl_slr_exchange_size(M, 0, st.m_pad, st.dtype_code))
    mb.exchange, mb.exchange_bytes = xch.data_ptr(), xch.numel()
    print(f"[s-only] n={st.n_pad} m={st.m} p={st.p} M={M} nm={nm} prefill={prefill}", flush=True)
    rc = lib.ssl_slr_forward_group(x.data_ptr(), x.stride(0), M, st.m, st.m_pad, st.p, st.q,
                                   st.dtype_code, members, 1, _lib.stream_ptr(x.device))
    _lib.check(rc, "ssl_slr_forward_group")
    torch.cuda.synchronize()
    del plan
    return y


def _counters_at_rest(dev) -> bool:
    torch.cuda.synchronize()
    return all(int(buf.abs().max()) == 0 for (idx, _), buf in _runtime._COUNTERS.items()
               if idx == dev.index)


@pytest.mark.parametrize("dtype,p,M,prefill", [
    (torch.bfloat16, 32, 16, False),
    (torch.bfloat16, 32, 256, True),
    (torch.bfloat16, 64, 600, True),
    (torch.float16, 16, 300, True),
    (torch.float32, 32, 2048, True),
], ids=["bf16-p32-16", "bf16-p32-256", "bf16-p64-600", "f16-p16-300", "f32-p32-2048"])
def test_member_without_low_rank_factor(dtype, p, M, prefill, gpu_device):
    n, m = (1024, 512) if dtype == torch.float32 else (1536, 1024)
    prob = make_problem(n, m, 64, p, 0.5, dtype, seed=p + M)
    assert np.all(np.diff(prob["crow"]) > 0)  # every block-row holds blocks
    mod = make_module(prob, gpu_device)
    _runtime.reset_status(gpu_device)
    for rows in (M, M - 3):
        x_np = make_x(prob, rows, seed=rows)
        y = _s_only_call(mod, to_dev(x_np, dtype, gpu_device), prefill)
        want = orc.slr_linear(x_np, np.zeros((n, 1)), np.zeros((1, m)), s_dense(prob), prob["bias"])
        assert err(y[:, :n], want) <= TOL[dtype], rows
        assert _counters_at_rest(gpu_device), rows
    assert _runtime.read_status(gpu_device) == 0


@pytest.mark.parametrize("M,prefill", [(16, False), (256, True)])
def test_nm24_member_without_low_rank_factor(M, prefill, gpu_device):
    dtype = torch.bfloat16
    n, m = 1024, 2048
    mod, (_, _, S, b) = make_nm_module(n, m, 64, dtype, gpu_device, seed=M)
    _runtime.reset_status(gpu_device)
    x_np = np.random.default_rng(M).standard_normal((M, m))
    x_np = torch.from_numpy(x_np).to(dtype).double().numpy()
    y = _s_only_call(mod, to_dev(x_np, dtype, gpu_device), prefill)
    want = orc.slr_linear(x_np, np.zeros((n, 1)), np.zeros((1, m)), S, b)
    assert err(y[:, :n], want) <= TOL[dtype]
    assert _counters_at_rest(gpu_device)
    assert _runtime.read_status(gpu_device) == 0
