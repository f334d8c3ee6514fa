"""Chained launches (LRSLinearChain -> ssl_slr_forward_chain): a decoder layer's
projections q,k,v -> o -> gate,up -> down in ONE launch, each later stage
reading an earlier member's output as it is written inside the launch.

Stage 0's outputs must equal the grouped launch's bit for bit; later stages
compute their latent t = x·Bᵀ in one workgroup per rank tile (another fp32
summation order than a standalone launch), so every stage is checked against
the float64 oracle on the input it actually read, and repeated calls must agree
bit for bit. Calls the chain does not take (prefill sizes) run the stages one
by one and equal them exactly. The forward
each member computes is ssalaad/efficient/ls_linear.py:124-137; the stage
order is the reference model's per-layer module order
(ssalaad/efficient/model.py:41-57).
"""

from __future__ import annotations

import numpy as np
import pytest
import torch

from slr_cases import TOL, err, make_module, make_problem, make_x, oracle_y, to_dev

import ssalaad_amd
from ssalaad_amd import _lib, _runtime
from ssalaad_amd.ls_linear import latent_wait_status

pytestmark = pytest.mark.gpu

NAMES = ["q", "k", "v", "o", "gate", "up", "down"]


def _layer(h, f, r, p, dtype, dev, seed, pad=False, density=0.5):
    shapes = [(h, h), (h, h), (h, h), (h, h), (f, h), (f, h), (h, f)]
    probs = {nm: make_problem(n, m, r, p, density, dtype, seed=seed + i, pad=pad)
             for i, (nm, (n, m)) in enumerate(zip(NAMES, shapes))}
    return probs, {nm: make_module(probs[nm], dev) for nm in NAMES}


def _chain(mods):
    return ssalaad_amd.LRSLinearChain(
        [[mods["q"], mods["k"], mods["v"]], [mods["o"]], [mods["gate"], mods["up"]],
         [mods["down"]]],
        sources=[mods["q"], mods["o"], mods["gate"]])


def _flat(outs):
    return [y for stage in outs for y in stage]


def _one_by_one(mods, x):
    q, k, v = ssalaad_amd.LRSLinearGroup(mods["q"], mods["k"], mods["v"])(x)
    o = mods["o"](q)
    g, u = ssalaad_amd.LRSLinearGroup(mods["gate"], mods["up"])(o)
    d = mods["down"](g)
    return [q, k, v, o, g, u, d]


def _inputs(x, ys):
    """The input each member read: x for q,k,v; q for o; o for gate,up; gate for down."""
    return [x, x, x, ys[0], ys[3], ys[3], ys[4]]


def _words_at_rest(dev) -> bool:
    """Every row counter and stage word is back at zero."""
    torch.cuda.synchronize()
    return all(int(buf.abs().max()) == 0 for (idx, _), buf in _runtime._COUNTERS.items()
               if idx == dev.index)


def _check_against_oracle(probs, x, ys, dtype):
    for nm, xin, y in zip(NAMES, _inputs(x, ys), ys):
        xin64 = xin.double().cpu().numpy()
        assert err(y, oracle_y(probs[nm], xin64)) <= TOL[dtype], nm


def _check_chain(chain, mods, probs, x, dtype):
    """Stage 0 bit for bit against the grouped launch, every stage against the
    oracle on its own input, and a second call equal to the first."""
    ys = _flat(chain(x))
    again = _flat(chain(x))
    q, k, v = ssalaad_amd.LRSLinearGroup(mods["q"], mods["k"], mods["v"])(x)
    torch.cuda.synchronize()
    for nm, y, w in zip(NAMES[:3], ys[:3], (q, k, v)):
        assert y.shape == w.shape and torch.equal(y, w), nm
    for nm, y, w in zip(NAMES, ys, again):
        assert torch.equal(y, w), nm
    if probs is not None:
        _check_against_oracle(probs, x, ys, dtype)
    return ys


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16], ids=["bf16", "f16"])
@pytest.mark.parametrize("p", [16, 32, 64])
@pytest.mark.parametrize("M", [1, 7, 16, 33, 100])
def test_chain_matches_the_oracle_stage_by_stage(dtype, p, M, gpu_device):
    """A layer with a ragged FFN (688 features: the last block-row of gate and
    up is cut, and down reads a ragged last K unit), one to two token tiles."""
    probs, mods = _layer(256, 688, 64, p, dtype, gpu_device, seed=3 * p + M, pad=True)
    x = to_dev(make_x(probs["q"], M), dtype, gpu_device)
    chain = _chain(mods)
    assert chain._chained([[m._kernel() for m in g.members] for g in chain.groups], M)
    _check_chain(chain, mods, probs, x, dtype)
    assert latent_wait_status(gpu_device) == 0
    assert _words_at_rest(gpu_device)


@pytest.mark.parametrize("M", [1, 16])
def test_chain_llama1b_layer(M, gpu_device):
    """The LLaMA-1B layer (hidden 2048, FFN 5461, rank 256, 32×32 blocks at
    50%): the benchmark's chained launch, against the stages one by one and
    the oracle."""
    dtype = torch.bfloat16
    probs, mods = _layer(2048, 5461, 256, 32, dtype, gpu_device, seed=90 + M, pad=True)
    x = to_dev(make_x(probs["q"], M), dtype, gpu_device)
    _check_chain(_chain(mods), mods, probs, x, dtype)
    assert latent_wait_status(gpu_device) == 0


def test_chain_calls_of_changing_size_keep_the_sync_words_at_rest(gpu_device):
    """Calls of 1, 16, 5, 33, 100 and 1 token rows in a row (one and two token
    tiles, three tile heights): each exact; the stage words net to zero."""
    dtype = torch.bfloat16
    probs, mods = _layer(256, 512, 64, 32, dtype, gpu_device, seed=5)
    chain = _chain(mods)
    for M in (1, 16, 5, 33, 100, 1):
        x = to_dev(make_x(probs["q"], M, seed=M), dtype, gpu_device)
        _check_chain(chain, mods, probs, x, dtype)
    assert _words_at_rest(gpu_device)


def test_chain_graph_replays(gpu_device):
    """The chained launch captured in a HIP graph, replayed three times with new
    inputs and eager work in between: every replay equals the eager chain."""
    dtype = torch.bfloat16
    probs, mods = _layer(256, 688, 64, 32, dtype, gpu_device, seed=17, pad=True)
    chain = _chain(mods)
    M = 16
    x_static = to_dev(make_x(probs["q"], M, seed=0), dtype, gpu_device)
    s = torch.cuda.Stream(gpu_device)
    s.wait_stream(torch.cuda.current_stream(gpu_device))
    with torch.cuda.stream(s):
        chain(x_static)
        torch.cuda.synchronize()
        g = torch.cuda.CUDAGraph()
        with torch.cuda.graph(g, stream=s):
            outs = _flat(chain(x_static))
    torch.cuda.synchronize()
    for rep in range(3):
        x_new = to_dev(make_x(probs["q"], M, seed=rep + 1), dtype, gpu_device)
        x_static.copy_(x_new)
        torch.cuda.synchronize()
        with torch.cuda.stream(s):
            g.replay()
        torch.cuda.synchronize()
        want = _flat(chain(x_new))
        torch.cuda.synchronize()
        for nm, y, w in zip(NAMES, outs, want):
            assert torch.equal(y, w), (rep, nm)


def _nm24_module(n, m, r, dtype, dev, seed):
    rng = np.random.default_rng(seed)
    count = rng.choice(3, size=(n, m // 4), p=[0.15, 0.25, 0.6])
    rank = np.argsort(rng.random((n, m // 4, 4)), axis=-1).argsort(axis=-1)
    S = (rng.standard_normal((n, m // 4, 4)) * 0.05 * (rank < count[..., None])).reshape(n, m)
    A = rng.standard_normal((n, r)) * 0.05
    B = rng.standard_normal((r, m)) * 0.05
    b = rng.standard_normal(n) * 0.1
    mod = ssalaad_amd.LRSLinear(to_dev(A, dtype, dev), to_dev(B, dtype, dev),
                                to_dev(S, dtype, dev), in_features=m, out_features=n,
                                bias=to_dev(b, dtype, dev), nm_n=2, nm_m=4)
    return mod


@pytest.mark.parametrize("M", [1, 16, 40])
def test_chain_nm24_layer(M, gpu_device):
    """Every projection with 2:4 S (hidden 256, FFN 704): equal to the stages
    one by one."""
    dtype = torch.bfloat16
    h, f = 256, 704
    shapes = [(h, h), (h, h), (h, h), (h, h), (f, h), (f, h), (h, f)]
    mods = {nm: _nm24_module(n, m, 64, dtype, gpu_device, seed=200 + i)
            for i, (nm, (n, m)) in enumerate(zip(NAMES, shapes))}
    x = to_dev(np.random.default_rng(M).standard_normal((M, h)), dtype, gpu_device)
    ys = _check_chain(_chain(mods), mods, None, x, dtype)
    # against the modules called one by one on the same inputs (the 2:4 path's
    # own oracle tests pin the modules)
    for nm, xin, y in zip(NAMES, _inputs(x, ys), ys):
        assert err(y, mods[nm](xin).double().cpu().numpy()) <= TOL[dtype], nm
    assert latent_wait_status(gpu_device) == 0


def test_chain_prefill_sized_call_runs_the_stages_one_by_one(gpu_device):
    """600 token rows take the prefill kernels: the chain runs its stages as
    grouped launches, with the same data flow and results."""
    dtype = torch.bfloat16
    probs, mods = _layer(256, 512, 64, 32, dtype, gpu_device, seed=8)
    chain = _chain(mods)
    M = 600
    assert not chain._chained([[m._kernel() for m in g.members] for g in chain.groups], M)
    x = to_dev(make_x(probs["q"], M), dtype, gpu_device)
    ys = _flat(chain(x))
    want = _one_by_one(mods, x)
    torch.cuda.synchronize()
    for nm, y, w in zip(NAMES, ys, want):
        assert torch.equal(y, w), nm


@pytest.fixture
def knobs():
    lib = _lib.load()

    def set_(knob, value):
        _lib.check(lib.ssl_debug_set(knob, value), "ssl_debug_set")

    yield set_
    set_(_lib.DEBUG_WAIT_POLLS, 0)
    set_(_lib.DEBUG_WAIT_UNREACHABLE, 0)
    set_(_lib.DEBUG_CHAIN_FRAG, 0)


@pytest.mark.parametrize("p", [32, 64, "nm24"])
@pytest.mark.parametrize("M", [3, 16])
def test_chain_fragment_order_inputs_equal_row_order(p, M, knobs, gpu_device):
    """A later stage of 32- or 64-wide blocks reads its input either by row
    segments or from the copy in MFMA-fragment order its source writes (the
    library picks by token rows; forced both ways here, at a size where it
    picks each): the same bits either way, and the oracle's values."""
    dtype = torch.bfloat16
    if p == "nm24":
        h, f = 256, 704
        shapes = [(h, h), (h, h), (h, h), (h, h), (f, h), (f, h), (h, f)]
        mods = {nm: _nm24_module(n, m, 64, dtype, gpu_device, seed=300 + i)
                for i, (nm, (n, m)) in enumerate(zip(NAMES, shapes))}
        probs = None
        x = to_dev(np.random.default_rng(M).standard_normal((M, h)), dtype, gpu_device)
    else:
        probs, mods = _layer(256, 688, 64, p, dtype, gpu_device, seed=7 * p + M, pad=True)
        x = to_dev(make_x(probs["q"], M), dtype, gpu_device)
    chain = _chain(mods)
    outs = {}
    for mode in (1, 2, 0):  # rows, fragments, the library's choice
        knobs(_lib.DEBUG_CHAIN_FRAG, mode)
        outs[mode] = _check_chain(chain, mods, probs, x, dtype)
    for nm, a, b, c in zip(NAMES, outs[1], outs[2], outs[0]):
        assert torch.equal(a, b) and torch.equal(a, c), nm
    if probs is None:
        for nm, xin, y in zip(NAMES, _inputs(x, outs[0]), outs[0]):
            assert err(y, mods[nm](xin).double().cpu().numpy()) <= TOL[dtype], nm
    assert latent_wait_status(gpu_device) == 0
    assert _words_at_rest(gpu_device)


@pytest.mark.parametrize("M", [1, 40])
def test_chain_wait_give_up_is_reported_and_words_net_to_zero(M, knobs, gpu_device):
    """With unreachable targets every wait (the stages' waits for their input,
    the latent waits) gives up after 64 polls: the status word says so, every
    counter and stage word is back at zero, and the next normal calls are
    exact."""
    dtype = torch.bfloat16
    probs, mods = _layer(256, 512, 64, 32, dtype, gpu_device, seed=11)
    chain = _chain(mods)
    x = to_dev(make_x(probs["q"], M), dtype, gpu_device)
    _runtime.reset_status(gpu_device)
    knobs(_lib.DEBUG_WAIT_POLLS, 64)
    knobs(_lib.DEBUG_WAIT_UNREACHABLE, 1)
    for _ in range(3):  # give-ups on consecutive launches with the same words
        chain(x)
        assert latent_wait_status(gpu_device) == 1
        assert _words_at_rest(gpu_device)
        with pytest.raises(RuntimeError, match="gave up waiting"):
            chain(x)
        _runtime.reset_status(gpu_device)
    knobs(_lib.DEBUG_WAIT_POLLS, 0)
    knobs(_lib.DEBUG_WAIT_UNREACHABLE, 0)
    _runtime.reset_status(gpu_device)
    for _ in range(2):
        _check_chain(chain, mods, probs, x, dtype)
    assert latent_wait_status(gpu_device) == 0


def test_chain_rejects_bad_stages(gpu_device):
    dtype = torch.bfloat16
    probs, mods = _layer(256, 512, 64, 32, dtype, gpu_device, seed=12)
    with pytest.raises(ValueError):
        ssalaad_amd.LRSLinearChain([[mods["q"]], [mods["o"]]], sources=[mods["k"]])
    with pytest.raises(ValueError):  # down reads 512 features; q writes 256
        ssalaad_amd.LRSLinearChain([[mods["q"]], [mods["down"]]], sources=[mods["q"]])
    with pytest.raises(ValueError):  # q already feeds o
        ssalaad_amd.LRSLinearChain([[mods["q"]], [mods["o"]], [mods["k"]]],
                                   sources=[mods["q"], mods["q"]])


# ------------------------------------------ many stages: descriptor table --


def _stack(layers):
    """Every layer's four stages in one chain; layer l's q,k,v read layer l-1's
    down output."""
    stages, sources = [], []
    for li, mods in enumerate(layers):
        if li > 0:
            sources.append(layers[li - 1]["down"])
        stages += [[mods["q"], mods["k"], mods["v"]], [mods["o"]], [mods["gate"], mods["up"]],
                   [mods["down"]]]
        sources += [mods["q"], mods["o"], mods["gate"]]
    return ssalaad_amd.LRSLinearChain(stages, sources)


@pytest.mark.parametrize("M", [1, 16, 40])
def test_stack_of_layers_in_one_launch(M, gpu_device):
    """Three layers (12 stages, 21 linears) in one launch with the descriptor
    table: every linear against the oracle on the input it read; forward (table
    uploaded per call) and a prepared chain agree bit for bit; repeated runs
    agree; the stage words net to zero."""
    dtype = torch.bfloat16
    layers = [_layer(256, 688, 64, 32, dtype, gpu_device, seed=300 + 10 * li, pad=True)
              for li in range(3)]
    chain = _stack([mods for _, mods in layers])
    x = to_dev(make_x(layers[0][0]["q"], M), dtype, gpu_device)
    ys = _flat(chain(x))
    assert len(ys) == 21
    x_p = x.clone()
    prep = chain.prepare(x_p)
    ys_p = _flat(prep.run(check=True))
    ys_p2 = [y.clone() for y in ys_p]
    _flat(prep.run())
    torch.cuda.synchronize()
    for i, (a, b, c) in enumerate(zip(ys, ys_p2, ys_p)):
        assert torch.equal(a, b) and torch.equal(b, c), i
    xin = x
    for li, (probs, _) in enumerate(layers):
        part = ys[7 * li:7 * li + 7]
        _check_against_oracle(probs, xin, part, dtype)
        xin = part[-1]
    q, k, v = ssalaad_amd.LRSLinearGroup(*[layers[0][1][n] for n in ("q", "k", "v")])(x)
    torch.cuda.synchronize()
    assert torch.equal(ys[0], q) and torch.equal(ys[1], k) and torch.equal(ys[2], v)
    assert latent_wait_status(gpu_device) == 0
    assert _words_at_rest(gpu_device)


def test_prepared_stack_graph_replays(gpu_device):
    """A prepared two-layer stack captured in a HIP graph and replayed with new
    input contents: every replay equals the chain's forward on that input."""
    dtype = torch.bfloat16
    layers = [_layer(256, 512, 64, 32, dtype, gpu_device, seed=400 + 10 * li) for li in range(2)]
    chain = _stack([mods for _, mods in layers])
    M = 16
    x_static = to_dev(make_x(layers[0][0]["q"], M, seed=0), dtype, gpu_device)
    prep = chain.prepare(x_static)
    s = torch.cuda.Stream(gpu_device)
    s.wait_stream(torch.cuda.current_stream(gpu_device))
    with torch.cuda.stream(s):
        prep.run()
        torch.cuda.synchronize()
        g = torch.cuda.CUDAGraph()
        with torch.cuda.graph(g, stream=s):
            outs = _flat(prep.run())
    torch.cuda.synchronize()
    for rep in range(3):
        x_new = to_dev(make_x(layers[0][0]["q"], M, seed=rep + 1), dtype, gpu_device)
        x_static.copy_(x_new)
        torch.cuda.synchronize()
        with torch.cuda.stream(s):
            g.replay()
        torch.cuda.synchronize()
        want = _flat(chain(x_new))
        torch.cuda.synchronize()
        for i, (y, w) in enumerate(zip(outs, want)):
            assert torch.equal(y, w), (rep, i)
    assert _words_at_rest(gpu_device)


def test_prepare_rejects_prefill_sized_calls(gpu_device):
    dtype = torch.bfloat16
    probs, mods = _layer(256, 512, 64, 32, dtype, gpu_device, seed=12)
    x = to_dev(make_x(probs["q"], 600), dtype, gpu_device)
    with pytest.raises(ValueError):
        _chain(mods).prepare(x)
