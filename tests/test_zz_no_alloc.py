"""ssl_slr_forward_noalloc (the fused SLR linear with its scratch in a static
device array) against ssl_slr_forward (caller scratch from the torch
allocator), both called through the C ABI with the same plan: bit-identical
outputs, and each within the parity bar of the oracle. Two calls in a row,
the second with fewer token rows (another exchange layout), then a call with
a different plan, then the capacity limit."""

from __future__ import annotations

import pytest
import torch

from slr_cases import TOL, err, make_module, make_problem, make_x, oracle_y, to_dev

from ssalaad_amd import _lib, _runtime

pytestmark = pytest.mark.gpu


def _args(mod, x, y, pl):
    st = mod._kernel()
    return [y.data_ptr(), y.stride(0), x.data_ptr(), x.stride(0), st.A.data_ptr(),
            st.B.data_ptr(), _lib.ptr(st.bias), st.col.data_ptr(), st.values.data_ptr(),
            pl.table.data_ptr(), pl.n_chunks, pl.n_slots, pl.lr_wgs, x.shape[0], st.m, st.m_pad,
            st.NB, st.r_pad, st.p, st.p, st.dtype_code]


def _with_scratch(mod, x):
    """The existing entry point, scratch from the torch allocator."""
    lib, st = _lib.load(), mod._kernel()
    M = x.shape[0]
    pl = st.plan(M)
    y = torch.empty(M, st.n_pad, dtype=x.dtype, device=x.device)
    ws = lib.ssl_slr_workspace_size(M, st.NB, st.p, st.r_pad, st.m_pad, pl.n_slots, st.dtype_code)
    nc = lib.ssl_slr_counter_count(M, st.NB)
    xb = lib.ssl_slr_exchange_size(M, st.r_pad, st.m_pad, st.dtype_code)
    w = torch.empty(max(ws, 256), dtype=torch.uint8, device=x.device)
    c = torch.zeros(max(nc, 1), dtype=torch.int32, device=x.device)
    e = torch.zeros(max(xb, 256), dtype=torch.uint8, device=x.device)
    rc = lib.ssl_slr_forward(*_args(mod, x, y, pl), c.data_ptr(), nc, e.data_ptr(), e.numel(),
                             w.data_ptr(), w.numel(), _lib.stream_ptr(x.device))
    _lib.check(rc, "ssl_slr_forward")
    return y, (w, c, e)


def _no_alloc(mod, x):
    lib, st = _lib.load(), mod._kernel()
    M = x.shape[0]
    pl = st.plan(M)
    y = torch.empty(M, st.n_pad, dtype=x.dtype, device=x.device)
    rc = lib.ssl_slr_forward_noalloc(*_args(mod, x, y, pl), _lib.stream_ptr(x.device))
    _lib.check(rc, "ssl_slr_forward_noalloc")
    return y


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float32], ids=["bf16", "f32"])
def test_no_alloc_entry_point_matches_the_scratch_entry_point(dtype, gpu_device, monkeypatch):
    # small chunks: split rows, so the counters, partial tiles and finaliser
    # waits are all in play
    monkeypatch.setattr(_runtime, "_CHUNK_BYTES", 16 * 1024)
    dev = gpu_device
    big = make_problem(1024, 2048, 160, 32, 0.5, dtype, seed=3, skew=True)
    small = make_problem(384, 2048, 64, 32, 0.4, dtype, seed=4)
    mb, ms = make_module(big, dev), make_module(small, dev)
    cases = [(mb, big, 48), (mb, big, 3), (ms, small, 20), (mb, big, 16)]
    for mod, prob, M in cases:
        x_np = make_x(prob, M, seed=M)
        x = to_dev(x_np, dtype, dev)
        want_y, keep = _with_scratch(mod, x)
        got = _no_alloc(mod, x)
        torch.cuda.synchronize()
        assert torch.equal(got, want_y), (prob["n"], M)
        assert err(got[:, : prob["n"]], oracle_y(prob, x_np)) <= TOL[dtype]
        del keep


def test_no_alloc_entry_point_rejects_calls_beyond_its_scratch(gpu_device):
    lib = _lib.load()
    assert lib.ssl_slr_noalloc_scratch_bytes() == 16 << 20
    # 64 token rows of a rank-65536 latent need far more than 15.25 MiB of
    # workspace; the call is refused before any pointer is used or any launch
    R = 1 << 16
    assert lib.ssl_slr_workspace_size(64, 4, 32, R, 8192, 0, _lib.SSL_BF16) > (16 << 20)
    y = torch.empty(64, 128, dtype=torch.bfloat16, device=gpu_device)
    x = torch.empty(64, 8192, dtype=torch.bfloat16, device=gpu_device)
    rc = lib.ssl_slr_forward_noalloc(y.data_ptr(), 128, x.data_ptr(), 8192, x.data_ptr(),
                                     x.data_ptr(), None, x.data_ptr(), x.data_ptr(), x.data_ptr(),
                                     4, 0, 4, 64, 8192, 8192, 4, R, 32, 32, _lib.SSL_BF16,
                                     _lib.stream_ptr(gpu_device))
    assert rc == _lib.SSL_ERR_CAPACITY
    assert b"no-allocation" in lib.ssl_last_error()
