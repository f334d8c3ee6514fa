"""Bundles (format_version 1) and model loading onto the HIP modules.

CPU tests: the file layout, the metadata and config filters, and the loader's
checks (ssalaad/efficient/artifact.py:78-118, ssalaad/train/model.py:63-94).
GPU tests: the reference's bundle test (tests/test_ssalaad.py:228-259) restated,
and model-level parity at the LLaMA-60M shape with every projection an SLR
linear (fp32, 8 × 256 tokens): logits of build_efficient_model vs the same
model with dense weights W = A·B + S.
"""

from __future__ import annotations

import pytest
import torch

from ssalaad_amd import bundle

TINY = {
    "model_type": "llama", "hidden_size": 32, "intermediate_size": 64, "num_hidden_layers": 1,
    "num_attention_heads": 4, "num_key_value_heads": 4, "vocab_size": 128,
    "max_position_embeddings": 128, "rms_norm_eps": 1e-6, "hidden_act": "silu",
    "bos_token_id": 1, "eos_token_id": 2, "pad_token_id": 0, "tie_word_embeddings": False,
}
PROJ = ["self_attn.q_proj", "self_attn.k_proj", "self_attn.v_proj", "self_attn.o_proj",
        "mlp.gate_proj", "mlp.up_proj", "mlp.down_proj"]


def _bsr_cpu(S: torch.Tensor, p: int) -> torch.Tensor:
    """Dense → BSR on the CPU with torch's own routine (the bundle test's layout)."""
    return S.to_sparse_bsr((p, p))


def test_save_and_load_keep_the_format(tmp_path):
    model = bundle.build_model_from_config(TINY)
    name = "model.layers.0.self_attn.q_proj"
    layer = {"A": torch.zeros(32, 4, dtype=torch.bfloat16), "B": torch.zeros(4, 32, dtype=torch.bfloat16),
             "S": _bsr_cpu(torch.zeros(32, 32, dtype=torch.bfloat16), 16), "block_p": 16, "block_q": 16}
    cfg = dict(TINY, tokenizer_id="/abs/local/tokenizer", run_name="x")
    path = tmp_path / "b" / "model.pt"
    bundle.save_artifact(path, {name: layer},
                         {"mode": "egar", "trace": "/private/source", "hostname": "h", "param_count": 7},
                         model=model, model_config=cfg)
    got = bundle.load_artifact(path)
    assert got["format_version"] == 1
    assert got["meta"] == {"mode": "egar", "param_count": 7}
    assert "tokenizer_id" not in got["model_config"] and "run_name" not in got["model_config"]
    assert got["model_config"]["hidden_size"] == 32
    assert name + ".weight" not in got["base_state_dict"]
    assert set(got["base_state_dict"]) == set(model.state_dict()) - {name + ".weight"}
    assert got["layers"][name]["block_p"] == 16


def test_load_rejects_partial_and_future_bundles(tmp_path):
    p = tmp_path / "x.pt"
    torch.save({"layers": {}}, p)
    with pytest.raises(ValueError, match="complete model bundle"):
        bundle.load_artifact(p)
    torch.save([1, 2], p)
    with pytest.raises(ValueError, match="complete model bundle"):
        bundle.load_artifact(p)
    torch.save({"format_version": 2, "layers": {}, "base_state_dict": {}, "model_config": {},
                "meta": {}}, p)
    with pytest.raises(ValueError, match="Unsupported model bundle version"):
        bundle.load_artifact(p)


def test_model_config_rules():
    m = bundle.build_model_from_config(dict(TINY, max_sequence_length=64,
                                            max_position_embeddings=None) | {"max_position_embeddings": 99})
    assert m.config.max_position_embeddings == 99
    cfg = {k: v for k, v in TINY.items() if k != "max_position_embeddings"} | {"max_sequence_length": 64}
    assert bundle.build_model_from_config(cfg).config.max_position_embeddings == 64
    with pytest.raises(ValueError, match="Unsupported model type"):
        bundle.build_model_from_config(dict(TINY, model_type="gpt2"))


def test_gpu_loader_refuses_the_cpu(tmp_path):
    with pytest.raises(ValueError, match="GPU"):
        bundle.build_efficient_model(tmp_path / "none.pt", device="cpu")


@pytest.mark.gpu
@pytest.mark.parametrize("layout", ["bsr", "zero", "dense"])
def test_bundle_reproduces_the_dense_model(tmp_path, layout, gpu_device):
    """tests/test_ssalaad.py:228-259 on the GPU modules (bf16, same tolerance)."""
    torch.manual_seed(7)
    model = bundle.build_model_from_config(TINY).eval()
    name = "model.layers.0.self_attn.q_proj"
    A, B = torch.randn(32, 4) * 0.01, torch.randn(4, 32) * 0.01
    S = torch.zeros(32, 32)
    if layout != "zero":
        S[:16, :16] = torch.randn(16, 16) * 0.01
    with torch.no_grad():
        model.get_submodule(name).weight.copy_(A @ B + S)
    ids = torch.tensor([[1, 3, 4, 5]])
    expected = model(input_ids=ids).logits
    if layout == "dense":
        layer = {"W": (A @ B + S).to(torch.bfloat16)}
    else:
        layer = {"A": A.to(torch.bfloat16), "B": B.to(torch.bfloat16),
                 "S": _bsr_cpu(S.to(torch.bfloat16), 16), "block_p": 16, "block_q": 16}
    path = tmp_path / "model.pt"
    bundle.save_artifact(path, {name: layer}, {"mode": "egar"}, model=model, model_config=TINY)
    # the bundle holds bf16 factors, as the reference's does; the restored model
    # runs in fp32 so that no bf16 attention product runs on the GPU
    restored, _, meta = bundle.build_efficient_model(path, device=gpu_device, dtype=torch.float32)
    assert meta == {"mode": "egar"}
    got = restored(input_ids=ids.to(gpu_device)).logits.float().cpu()
    torch.testing.assert_close(got, expected, atol=0.1, rtol=0.1)


@pytest.mark.gpu
def test_llama60m_every_projection_slr_matches_dense_weights(tmp_path, gpu_device):
    """8 layers, hidden 512, 8 heads, FFN 1376, vocab 32000; every q/k/v/o/gate/up/down
    an SLR linear (rank dim/4, 32×32 blocks at 50%, N(0, 0.02)); fp32 forward of
    8 × 256 tokens (each projection a 2048-row call: the fp32 prefill kernels).
    Bundle → build_efficient_model(fp32) against the float64 oracle's forward of
    the same weights (W = A·B + S), within the fp32 bar of 1e-5."""
    import numpy as np

    from oracle import decode_oracle as dor

    cfg = dict(TINY, hidden_size=512, intermediate_size=1376, num_hidden_layers=8,
               num_attention_heads=8, num_key_value_heads=8, vocab_size=32000,
               max_position_embeddings=256)
    torch.manual_seed(0)
    gen = torch.Generator().manual_seed(0)
    dense = bundle.build_model_from_config(cfg).eval()
    layers = {}
    for li in range(8):
        for proj in PROJ:
            name = f"model.layers.{li}.{proj}"
            lin = dense.get_submodule(name)
            n, m = lin.out_features, lin.in_features
            r, p = min(n, m) // 4, 32
            A = torch.randn(n, r, generator=gen) * 0.02
            B = torch.randn(r, m, generator=gen) * 0.02
            NB, NBK = n // p, m // p
            keep = torch.randperm(NB * NBK, generator=gen)[: NB * NBK // 2]
            mask = torch.zeros(NB * NBK)
            mask[keep] = 1
            S = torch.randn(n, m, generator=gen) * 0.02 * mask.view(NB, 1, NBK, 1).expand(
                NB, p, NBK, p).reshape(n, m)
            with torch.no_grad():
                lin.weight.copy_(A @ B + S)
            layers[name] = {"A": A, "B": B, "S": _bsr_cpu(S, p), "block_p": p, "block_q": p}
    path = tmp_path / "m60.pt"
    bundle.save_artifact(path, layers, {"mode": "egar"}, model=dense, model_config=cfg)
    model, _, _ = bundle.build_efficient_model(path, device=gpu_device, dtype=torch.float32)
    ids = torch.randint(3, 32000, (8, 256), generator=gen)
    with torch.no_grad():
        got = model(input_ids=ids.to(gpu_device)).logits.double().cpu().numpy()
    torch.cuda.synchronize()
    assert type(model.get_submodule("model.layers.3.mlp.down_proj")).__name__.startswith("_LRSLinear")
    want = dor.forward(dor.params_from_hf(dense.double()), ids.numpy())
    err = float(np.abs(got - want).max() / np.abs(want).max())
    print(f"[llama60m] fp32 logits vs float64 oracle: {err:.2e}")
    assert err <= 1e-5, err


@pytest.mark.gpu
def test_bundle_then_generate_matches_the_recompute_loop(tmp_path, gpu_device):
    """A bundle loaded by build_efficient_model (fp32) generates, with the cached
    decode step, the tokens the reference's loop picks by recomputing the prefix
    with the same model (generate.py:12-26). Two layers; q/k/v/gate/up/down are
    SLR linears (32x32 blocks at 50%), o_proj of layer 0 a plain dense layer."""
    from ssalaad_amd import generate

    cfg = dict(TINY, hidden_size=256, intermediate_size=352, num_hidden_layers=2,
               num_attention_heads=4, num_key_value_heads=2, vocab_size=300)
    torch.manual_seed(1)
    gen = torch.Generator().manual_seed(1)
    dense = bundle.build_model_from_config(cfg).eval()
    with torch.no_grad():
        for name, prm in dense.named_parameters():
            if "norm" not in name:
                prm.copy_(torch.randn(prm.shape, generator=gen) * (1.0 if "embed" in name else 0.08))
    layers = {}
    for li in range(2):
        for proj in PROJ:
            name = f"model.layers.{li}.{proj}"
            lin = dense.get_submodule(name)
            if li == 0 and proj == "self_attn.o_proj":
                layers[name] = {"W": lin.weight.detach().clone()}
                continue
            n, m = lin.out_features, lin.in_features
            r, p = 32, 32
            A = torch.randn(n, r, generator=gen) * 0.1
            B = torch.randn(r, m, generator=gen) * 0.1
            NB, NBK = n // p, m // p
            keep = torch.randperm(NB * NBK, generator=gen)[: NB * NBK // 2]
            mask = torch.zeros(NB * NBK)
            mask[keep] = 1
            S = torch.randn(n, m, generator=gen) * 0.05 * mask.view(NB, 1, NBK, 1).expand(
                NB, p, NBK, p).reshape(n, m)
            with torch.no_grad():
                lin.weight.copy_(A @ B + S)
            layers[name] = {"A": A, "B": B, "S": _bsr_cpu(S, p), "block_p": p, "block_q": p}
    path = tmp_path / "gen.pt"
    bundle.save_artifact(path, layers, {"mode": "egar"}, model=dense, model_config=cfg)
    model, _, _ = bundle.build_efficient_model(path, device=gpu_device, dtype=torch.float32)
    prompt = torch.randint(3, 300, (2, 6), generator=gen)
    out = generate(model, prompt, 10)
    seq = prompt.to(gpu_device)
    with torch.no_grad():
        for _ in range(10):
            logits = model(input_ids=seq, use_cache=False).logits[:, -1]
            seq = torch.cat((seq, logits.argmax(-1, keepdim=True)), dim=1)
    assert torch.equal(out, seq.cpu())
