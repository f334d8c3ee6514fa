"""Block shapes beyond square 16/32/64, on the GPU, against the oracle.

The reference's GPU module and op take any block whose sides are multiples of
16, square or not (ssalaad/efficient/ls_linear.py:114-117,
ssalaad/tilelang_sparse/addmm_inplace.py:59-63, 96-97), and its compressor
writes whatever `--block-size P Q` asks for (ssalaad/inference/egar.py:51-56,
501-502). Here: every (p, q) in {16, 32, 48, 64}², blocks wider than the
kernels' tiles (p = 96, 128) and deeper than 256 (q = 512), through the fused
module (decode and many-token calls), the grouped launch, the in-place op and
a bundle written with 16×32 blocks.
"""

from __future__ import annotations

import numpy as np
import pytest
import torch

from oracle import slr_oracle as orc
from slr_cases import TOL, err, make_module, make_problem, make_x, oracle_y, to_dev

import ssalaad_amd
from ssalaad_amd import _runtime, bundle

pytestmark = pytest.mark.gpu

SIDES = [16, 32, 48, 64]
ALL_PQ = [(p, q) for p in SIDES for q in SIDES]
WIDE_PQ = [(96, 32), (128, 64), (32, 512), (128, 320)]


def _prob(p, q, dtype, seed, skew=False, pad=False, bias=True):
    n = 5 * p + (p // 2 if pad else 0)
    m = 7 * q + (q // 2 if pad else 0)
    return make_problem(n, m, 40, p, 0.5, dtype, seed=seed, skew=skew, pad=pad, q=q, bias=bias)


@pytest.mark.parametrize("p,q", ALL_PQ + WIDE_PQ)
@pytest.mark.parametrize("M", [1, 16, 37, 200])
def test_module_bf16_every_block_shape(p, q, M, gpu_device):
    dtype = torch.bfloat16
    prob = _prob(p, q, dtype, seed=p * 1000 + q + M, skew=(M == 37))
    mod = make_module(prob, gpu_device)
    x = make_x(prob, M)
    y = mod(to_dev(x, dtype, gpu_device))
    y2 = mod(to_dev(x, dtype, gpu_device))
    torch.cuda.synchronize()
    assert y.shape == (M, prob["n"])
    assert err(y, oracle_y(prob, x)) <= TOL[dtype]
    assert torch.equal(y, y2)


@pytest.mark.parametrize("dtype", [torch.float32, torch.float16], ids=["f32", "f16"])
@pytest.mark.parametrize("p,q", [(16, 32), (32, 16), (48, 48), (64, 16), (48, 64), (128, 32)])
@pytest.mark.parametrize("M", [3, 64, 130])
def test_module_other_dtypes(dtype, p, q, M, gpu_device):
    prob = _prob(p, q, dtype, seed=7 * p + q + M)
    mod = make_module(prob, gpu_device)
    x = make_x(prob, M)
    y = mod(to_dev(x, dtype, gpu_device))
    torch.cuda.synchronize()
    assert err(y, oracle_y(prob, x)) <= TOL[dtype]


@pytest.mark.parametrize("p,q", [(16, 48), (48, 32), (64, 32), (96, 32)])
def test_module_ragged_features_no_bias(p, q, gpu_device):
    prob = _prob(p, q, torch.bfloat16, seed=p + q, pad=True, bias=False)
    mod = make_module(prob, gpu_device, bias=False)
    x = make_x(prob, 9)
    y = mod(to_dev(x, torch.bfloat16, gpu_device))
    torch.cuda.synchronize()
    assert y.shape == (9, prob["n"])
    assert err(y, oracle_y(prob, x)) <= 1e-2


@pytest.mark.parametrize("p,q", [(16, 32), (48, 48), (64, 48)])
@pytest.mark.parametrize("M", [1, 40])
def test_module_split_rows(p, q, M, gpu_device, monkeypatch):
    """Every unit its own chunk: the partial-tile exchange with non-square and
    48-wide tiles (the 3-wide lane map)."""
    monkeypatch.setattr(_runtime, "_CHUNK_BYTES", 1)
    prob = make_problem(4 * p, 20 * q, 96, p, 0.4, torch.bfloat16, seed=M + p, skew=True, q=q)
    mod = make_module(prob, gpu_device)
    x = make_x(prob, M)
    ys = [mod(to_dev(x, torch.bfloat16, gpu_device)) for _ in range(2)]
    torch.cuda.synchronize()
    assert err(ys[0], oracle_y(prob, x)) <= 1e-2
    assert torch.equal(ys[0], ys[1])


@pytest.mark.parametrize("p,q", [(16, 32), (48, 64), (128, 64)])
@pytest.mark.parametrize("M", [1, 24, 150])
def test_group_non_square(p, q, M, gpu_device):
    probs = [make_problem(n, 6 * q, r, p, d, torch.bfloat16, seed=M + i, skew=(i == 1), q=q)
             for i, (n, r, d) in enumerate([(4 * p, 64, 0.5), (2 * p, 96, 0.3), (3 * p, 32, 0.7)])]
    grp = ssalaad_amd.LRSLinearGroup(*[make_module(pr, gpu_device) for pr in probs])
    x = make_x(probs[0], M)
    ys = grp(to_dev(x, torch.bfloat16, gpu_device))
    torch.cuda.synchronize()
    for y, pr in zip(ys, probs):
        assert err(y, oracle_y(pr, x)) <= 1e-2


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16], ids=["f32", "bf16"])
@pytest.mark.parametrize("p,q", ALL_PQ + WIDE_PQ)
@pytest.mark.parametrize("M", [5, 150])
def test_op_every_block_shape_keeps_inactive_rows(dtype, p, q, M, gpu_device):
    prob = make_problem(9 * p, 6 * q, 4, p, 0.3, dtype, seed=p + 3 * q + M, skew=True, q=q)
    crow32, col32, vt, act = orc.module_buffers(prob["crow"], prob["col"], prob["vals"])
    x = make_x(prob, M, seed=2)
    rng = np.random.default_rng(M)
    out0 = torch.from_numpy(rng.standard_normal((M, prob["n"]))).to(dtype).double().numpy()
    want = orc.bsr_addmm_inplace(out0, x, crow32, col32, vt, act)
    dev = gpu_device
    out = to_dev(out0, dtype, dev)
    torch.ops.ssalaad.tilelang_bsr_addmm_inplace_dense_(
        out, to_dev(x, dtype, dev), torch.from_numpy(crow32).to(dev),
        torch.from_numpy(col32).to(dev), to_dev(vt, dtype, dev), torch.from_numpy(act).to(dev))
    torch.cuda.synchronize()
    assert err(out, want) <= TOL[dtype]
    got = out.double().cpu().numpy()
    for by in sorted(set(range(prob["NB"])) - set(act.tolist())):
        assert np.array_equal(got[:, by * p:(by + 1) * p], out0[:, by * p:(by + 1) * p])


def test_module_rejects_sides_not_divisible_by_16(gpu_device):
    A = torch.zeros(64, 4, device=gpu_device)
    B = torch.zeros(4, 64, device=gpu_device)
    S = torch.zeros(64, 64, device=gpu_device)
    S[:8, :8] = 1
    with pytest.raises(ValueError, match="divisible by 16"):
        ssalaad_amd.LRSLinear(A, B, S.to_sparse_bsr((8, 8)), in_features=64, out_features=64,
                              block_p=8, block_q=8)


def test_bundle_with_16x32_blocks_matches_the_dense_model(tmp_path, gpu_device):
    """A bundle whose projections were compressed with --block-size 16 32
    loads onto the HIP modules and reproduces the dense model (fp32)."""
    cfg = {"model_type": "llama", "hidden_size": 128, "intermediate_size": 192,
           "num_hidden_layers": 1, "num_attention_heads": 4, "num_key_value_heads": 4,
           "vocab_size": 256, "max_position_embeddings": 64, "rms_norm_eps": 1e-6,
           "hidden_act": "silu", "tie_word_embeddings": False}
    torch.manual_seed(3)
    gen = torch.Generator().manual_seed(3)
    dense = bundle.build_model_from_config(cfg).eval()
    layers = {}
    for proj in ("self_attn.q_proj", "self_attn.k_proj", "self_attn.v_proj", "self_attn.o_proj",
                 "mlp.gate_proj", "mlp.up_proj", "mlp.down_proj"):
        name = f"model.layers.0.{proj}"
        lin = dense.get_submodule(name)
        n, m = lin.out_features, lin.in_features
        p, q, r = 16, 32, 16
        A = torch.randn(n, r, generator=gen) * 0.05
        B = torch.randn(r, m, generator=gen) * 0.05
        keep = (torch.rand(n // p, m // q, generator=gen) < 0.5).float()
        S = torch.randn(n, m, generator=gen) * 0.05 * keep.repeat_interleave(p, 0).repeat_interleave(q, 1)
        with torch.no_grad():
            lin.weight.copy_(A @ B + S)
        layers[name] = {"A": A, "B": B, "S": S.to_sparse_bsr((p, q)), "block_p": p, "block_q": q}
    path = tmp_path / "b1632.pt"
    bundle.save_artifact(path, layers, {"mode": "egar"}, model=dense, model_config=cfg)
    model, _, _ = bundle.build_efficient_model(path, device=gpu_device, dtype=torch.float32)
    assert model.get_submodule("model.layers.0.mlp.up_proj").block_q == 32
    ids = torch.randint(0, 256, (2, 12), generator=gen)
    with torch.no_grad():
        want = dense.to(gpu_device)(input_ids=ids.to(gpu_device)).logits.double()
        got = model(input_ids=ids.to(gpu_device)).logits.double()
    torch.cuda.synchronize()
    assert float((got - want).abs().max() / want.abs().max()) <= 1e-5


# ----------------------------------------- many tokens: the square tiles --
# The tiled kernels of many-token calls run square 16/32/64 blocks (fp32:
# 16/32). Other blocks run on the same matrix cut into the widest square
# blocks that tile them; every tile forced in turn, every row checked.

PF_PQ = [(16, 32), (32, 16), (48, 48), (64, 32), (32, 64), (128, 320)]
SQUARE = {(16, 32): 16, (32, 16): 16, (48, 48): 16, (64, 32): 32, (32, 64): 32, (128, 320): 32}


@pytest.fixture
def tile():
    from ssalaad_amd import _lib

    lib = _lib.load()

    def force(mode):
        _lib.check(lib.ssl_debug_set(_lib.DEBUG_PREFILL_TILE, mode), "ssl_debug_set")

    yield force
    force(0)


@pytest.mark.parametrize("p,q", PF_PQ)
@pytest.mark.parametrize("mode", [0, 1, 2, 3], ids=["auto", "narrow", "tall", "short"])
@pytest.mark.parametrize("M", [300, 600])
def test_module_many_tokens_runs_square_tiles(p, q, mode, M, tile, gpu_device):
    tile(mode)
    dtype = torch.bfloat16
    prob = make_problem(12 * p, 10 * q, 64, p, 0.5, dtype, seed=p + q + M + mode, q=q,
                        skew=(mode == 2))
    mod = make_module(prob, gpu_device)
    view = mod._kernel().prefill_view()
    assert view is not None and view.p == view.q == SQUARE[(p, q)]
    assert view.takes_prefill(M, view.NB)
    x = make_x(prob, M, seed=M)
    print(f"[square] {p}x{q} as {view.p} tile={mode} M={M}", flush=True)
    y1, y2 = mod(to_dev(x, dtype, gpu_device)), mod(to_dev(x, dtype, gpu_device))
    torch.cuda.synchronize()
    assert err(y1, oracle_y(prob, x)) <= TOL[dtype]
    assert torch.equal(y1, y2)


@pytest.mark.parametrize("mode", [0, 1, 3], ids=["auto", "narrow", "short"])
def test_module_fp32_64x64_runs_32x32_tiles(mode, tile, gpu_device):
    """fp32 steps are 32 columns: 64×64 blocks run as four 32×32 blocks."""
    tile(mode)
    dtype = torch.float32
    prob = make_problem(20 * 64, 8 * 64, 64, 64, 0.5, dtype, seed=5 + mode)
    mod = make_module(prob, gpu_device)
    view = mod._kernel().prefill_view()
    assert view is not None and view.p == 32
    M = 2048 if mode == 0 else 300
    assert view.takes_prefill(M, view.NB)
    x = make_x(prob, M, seed=M)
    y = mod(to_dev(x, dtype, gpu_device))
    torch.cuda.synchronize()
    assert err(y, oracle_y(prob, x)) <= TOL[dtype]


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16], ids=["bf16", "f16"])
@pytest.mark.parametrize("p,q", [(16, 32), (48, 48), (64, 32), (128, 320)])
@pytest.mark.parametrize("mode", [0, 1, 3], ids=["auto", "narrow", "short"])
def test_op_many_tokens_runs_square_tiles(dtype, p, q, mode, tile, gpu_device):
    tile(mode)
    M = 600
    prob = make_problem(9 * p, 6 * q, 4, p, 0.4, dtype, seed=p + q + mode, skew=True, q=q)
    crow32, col32, vt, act = orc.module_buffers(prob["crow"], prob["col"], prob["vals"])
    x = make_x(prob, M, seed=2)
    rng = np.random.default_rng(M)
    out0 = torch.from_numpy(rng.standard_normal((M, prob["n"]))).to(dtype).double().numpy()
    want = orc.bsr_addmm_inplace(out0, x, crow32, col32, vt, act)
    dev = gpu_device
    out = to_dev(out0, dtype, dev)
    values = to_dev(vt, dtype, dev)
    torch.ops.ssalaad.tilelang_bsr_addmm_inplace_dense_(
        out, to_dev(x, dtype, dev), torch.from_numpy(crow32).to(dev),
        torch.from_numpy(col32).to(dev), values, torch.from_numpy(act).to(dev))
    torch.cuda.synchronize()
    assert err(out, want) <= TOL[dtype]
    s = SQUARE[(p, q)]
    assert any(pq == (s, s) for pq in getattr(values, "_ssl_kernel_view", {}))  # the square view ran
    got = out.double().cpu().numpy()
    for by in sorted(set(range(prob["NB"])) - set(act.tolist())):
        assert np.array_equal(got[:, by * p:(by + 1) * p], out0[:, by * p:(by + 1) * p])
