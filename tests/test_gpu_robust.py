"""Failure handling and state consistency of the fused kernels, on the GPU.

  * a bounded wait that gives up (forced from the host with the test hooks, so
    every workgroup still ends normally) is reported in the device's status
    word, leaves the row counters at zero, and later calls are exact again;
  * the decode engine raises on the step after such a launch;
  * a module whose buffers change in place after its first forward uses the
    new weights (the reference module reads its buffers on every forward,
    ssalaad/efficient/ls_linear.py:124-137);
  * a HIP graph captured before the workspace pool grew still replays into
    live memory and still computes the right output;
  * factor_from_svd (ssalaad/efficient/artifact.py:7-17) on device tensors.
"""

from __future__ import annotations

import numpy as np
import pytest
import torch

from slr_cases import TOL, err, make_module, make_problem, make_x, oracle_y, round_to, to_dev

import ssalaad_amd
from ssalaad_amd import _lib, _runtime
from ssalaad_amd.ls_linear import latent_wait_status

pytestmark = pytest.mark.gpu


@pytest.fixture
def knobs():
    lib = _lib.load()

    def set_(knob, value):
        _lib.check(lib.ssl_debug_set(knob, value), "ssl_debug_set")

    yield set_
    set_(_lib.DEBUG_WAIT_POLLS, 0)
    set_(_lib.DEBUG_WAIT_UNREACHABLE, 0)


def _counters_at_rest(dev) -> bool:
    torch.cuda.synchronize()
    return all(int(buf.abs().max()) == 0 for (idx, _), buf in _runtime._COUNTERS.items()
               if idx == dev.index)


@pytest.mark.parametrize("M", [1, 16, 40, 600])
def test_wait_give_up_is_reported_and_counters_net_to_zero(M, knobs, gpu_device, monkeypatch):
    """Every unit its own chunk: each row's finaliser waits for its other chunks
    and for the latent. With unreachable targets every wait gives up after 64
    polls; the status word says so, the late chunks' arrivals bring every row
    counter back to zero, and the next normal calls are exact. At 600 rows the
    call runs the prefill kernels, whose row workgroups wait for the latent
    tiles of the same launch: the same give-up, the same recovery."""
    monkeypatch.setattr(_runtime, "_CHUNK_BYTES", 1)
    dtype = torch.bfloat16
    prob = make_problem(256, 1024, 96, 32, 0.4, dtype, seed=M, skew=True)
    mod = make_module(prob, gpu_device)
    x = to_dev(make_x(prob, M), dtype, gpu_device)
    want = oracle_y(prob, make_x(prob, M))
    _runtime.reset_status(gpu_device)
    knobs(_lib.DEBUG_WAIT_POLLS, 64)
    knobs(_lib.DEBUG_WAIT_UNREACHABLE, 1)
    for _ in range(3):  # give-ups on consecutive calls with one plan
        mod(x)
        assert latent_wait_status(gpu_device) == 1
        assert _counters_at_rest(gpu_device)
        # the module refuses to run again until the status is cleared
        with pytest.raises(RuntimeError, match="gave up waiting"):
            mod(x)
        ssalaad_amd.clear_wait_status(gpu_device)
    knobs(_lib.DEBUG_WAIT_POLLS, 0)
    knobs(_lib.DEBUG_WAIT_UNREACHABLE, 0)
    _runtime.reset_status(gpu_device)
    ys = [mod(x) for _ in range(3)]
    torch.cuda.synchronize()
    for y in ys:
        assert err(y, want) <= TOL[dtype]
    assert latent_wait_status(gpu_device) == 0
    assert _counters_at_rest(gpu_device)


def test_every_entry_point_raises_while_a_give_up_is_reported(knobs, gpu_device):
    """A give-up forced on one module call (it still returns): once its store
    has landed, the next call of any module, group, chain or the in-place op
    on the device raises RuntimeError before launching anything, without the
    caller synchronising or asking. After clear_wait_status every one of them
    runs again and is exact."""
    dtype = torch.bfloat16
    prob = make_problem(256, 512, 64, 32, 0.5, dtype, seed=21)
    mod, other = make_module(prob, gpu_device), make_module(prob, gpu_device)
    nxt = make_module(make_problem(128, 256, 64, 32, 0.5, dtype, seed=22), gpu_device)
    group = ssalaad_amd.LRSLinearGroup(mod, other)
    chain = ssalaad_amd.LRSLinearChain([[mod], [nxt]], [mod])
    x_np = make_x(prob, 4)
    x = to_dev(x_np, dtype, gpu_device)
    want = oracle_y(prob, x_np)
    crow = torch.from_numpy(prob["crow"].astype(np.int32)).to(gpu_device)
    col = torch.from_numpy(prob["col"].astype(np.int32)).to(gpu_device)
    vt = mod.S_values
    act = mod.S_active_rows
    out = torch.zeros(4, 256, dtype=dtype, device=gpu_device)
    calls = {
        "module": lambda: mod(x),
        "group": lambda: group(x),
        "chain": lambda: chain(x),
        "op": lambda: torch.ops.ssalaad.tilelang_bsr_addmm_inplace_dense_(out, x, crow, col, vt, act),
    }
    ssalaad_amd.clear_wait_status(gpu_device)
    knobs(_lib.DEBUG_WAIT_POLLS, 16)
    knobs(_lib.DEBUG_WAIT_UNREACHABLE, 1)
    mod(x)  # returns; its workgroups gave up
    knobs(_lib.DEBUG_WAIT_POLLS, 0)
    knobs(_lib.DEBUG_WAIT_UNREACHABLE, 0)
    torch.cuda.synchronize()  # only so that the store has surely landed
    for name, call in calls.items():
        with pytest.raises(RuntimeError, match="gave up waiting"):
            call()
    ssalaad_amd.clear_wait_status(gpu_device)
    for name, call in calls.items():
        call()
    torch.cuda.synchronize()
    assert err(mod(x), want) <= TOL[dtype]
    assert err(group(x)[1], want) <= TOL[dtype]
    assert latent_wait_status(gpu_device) == 0
    assert _counters_at_rest(gpu_device)


def test_decode_engine_raises_after_a_wait_gave_up(knobs, gpu_device):
    from test_gpu_decode import _slr_pair

    from ssalaad_amd import DecodeEngine

    model, _ = _slr_pair("llama", torch.bfloat16, 2, gpu_device, layers=1)
    eng = DecodeEngine(model, max_batch=2, max_context=8, use_graphs=False)
    _runtime.reset_status(gpu_device)
    eng.step([1, 2], [0, 0])
    knobs(_lib.DEBUG_WAIT_POLLS, 16)
    knobs(_lib.DEBUG_WAIT_UNREACHABLE, 1)
    with pytest.raises(RuntimeError, match="gave up waiting"):
        # its launches give up: an eager step's later launch may already see
        # the report; the next step sees it at the latest
        try:
            eng.step([3, 4], [1, 1])
        finally:
            knobs(_lib.DEBUG_WAIT_POLLS, 0)
            knobs(_lib.DEBUG_WAIT_UNREACHABLE, 0)
        torch.cuda.synchronize()
        eng.step([5, 6], [2, 2])
    eng.clear_status()
    eng.step([5, 6], [2, 2])
    eng.step([7, 8], [3, 3])


def test_module_uses_weights_updated_after_the_first_forward(gpu_device):
    """Rank 100 (A and B padded to 128 inside the kernel view): forward, then
    load_state_dict with other factors, S values and bias, then in-place
    copy_ into B: each forward follows the module's current buffers."""
    dtype = torch.float32
    p1 = make_problem(192, 320, 100, 32, 0.5, dtype, seed=1)
    rng = np.random.default_rng(2)
    p2 = dict(p1, **{k: round_to(rng.standard_normal(p1[k].shape) * 0.02, dtype)
                     for k in ("vals", "A", "B", "bias")})   # same structure, new values
    m1, m2 = make_module(p1, gpu_device), make_module(p2, gpu_device)
    x_np = make_x(p1, 5)
    x = to_dev(x_np, dtype, gpu_device)
    assert err(m1(x), oracle_y(p1, x_np)) <= TOL[dtype]
    m1.load_state_dict(m2.state_dict())
    assert err(m1(x), oracle_y(p2, x_np)) <= TOL[dtype]
    B3 = round_to(rng.standard_normal((100, 320)) * 0.02, dtype)
    with torch.no_grad():
        m1.B.copy_(torch.from_numpy(B3))
    assert err(m1(x), oracle_y(dict(p2, B=B3), x_np)) <= TOL[dtype]


def test_graph_replay_after_the_workspace_pool_grew(gpu_device):
    """A graph captured at one token row holds the pool's buffers; a later call
    with many rows outgrows the pool. The old buffers must stay alive: the
    replay, after the freed memory has been handed out and overwritten, still
    equals the oracle."""
    dtype = torch.bfloat16
    prob = make_problem(2048, 4096, 1024, 64, 0.5, dtype, seed=4)
    mod = make_module(prob, gpu_device)
    x1_np = make_x(prob, 1, seed=2)
    x1 = to_dev(x1_np, dtype, gpu_device)
    s = torch.cuda.Stream(gpu_device)
    s.wait_stream(torch.cuda.current_stream(gpu_device))
    with torch.cuda.stream(s):
        mod(x1)  # warm plans and pools on the capture stream
        g = torch.cuda.CUDAGraph()
        with torch.cuda.graph(g, stream=s):
            y_graph = mod(x1)
    torch.cuda.current_stream(gpu_device).wait_stream(s)
    before = {k: v.data_ptr() for k, v in _runtime._WORKSPACES.items()}
    with torch.cuda.stream(s):
        xbig = to_dev(make_x(prob, 700, seed=3), dtype, gpu_device)
        mod(xbig)  # prefill-sized workspace: the pool grows
    torch.cuda.synchronize()
    assert {k: v.data_ptr() for k, v in _runtime._WORKSPACES.items()} != before
    torch.cuda.empty_cache()
    junk = [torch.full((1 << 20,), 7, dtype=torch.int32, device=gpu_device) for _ in range(64)]
    want = oracle_y(prob, x1_np)
    for _ in range(3):
        with torch.cuda.stream(s):
            g.replay()
        torch.cuda.synchronize()
        assert err(y_graph, want) <= TOL[dtype]
    del junk


def test_factor_from_svd_on_device(gpu_device):
    """tests/test_ssalaad.py:276-283 on device tensors: the factors of a rank-3
    matrix rebuild it, rank 0 gives empty factors, the rank is clamped to the
    spectrum, and √σ is split evenly (A's columns and B's rows share norms
    σ_i^½ when U and Vh are orthonormal)."""
    g = torch.Generator().manual_seed(0)
    matrix = (torch.randn(16, 3, generator=g) @ torch.randn(3, 32, generator=g)).to(gpu_device)
    U, S, Vh = torch.linalg.svd(matrix, full_matrices=False)
    A, B = ssalaad_amd.factor_from_svd(U, S, Vh, 3)
    assert A.is_cuda and B.is_cuda and A.shape == (16, 3) and B.shape == (3, 32)
    torch.testing.assert_close(A @ B, matrix, atol=1e-4, rtol=1e-4)
    torch.testing.assert_close(A.norm(dim=0), S[:3].sqrt(), atol=1e-5, rtol=1e-5)
    torch.testing.assert_close(B.norm(dim=1), S[:3].sqrt(), atol=1e-5, rtol=1e-5)
    A0, B0 = ssalaad_amd.factor_from_svd(U, S, Vh, 0)
    assert A0.shape == (16, 0) and B0.shape == (0, 32)
    Aall, Ball = ssalaad_amd.factor_from_svd(U, S, Vh, 99)
    assert Aall.shape == (16, 16) and Ball.shape == (16, 32)
