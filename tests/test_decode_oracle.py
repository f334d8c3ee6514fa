"""The decode-step oracle pinned against transformers' own forward (CPU only).

The oracle (oracle/decode_oracle.py) restates, token by token from a cache,
what the Hugging Face causal LM computes over a whole sequence. Each test
builds a small random model in float64 and checks the oracle's logits at every
position against the library's full-sequence forward. transformers computes
RMSNorm and the rotary tables in fp32 even in a float64 model, so the bound is
a few fp32 ulps (TOL), far below what any wrong term, sign or index gives.
"""

from __future__ import annotations

import numpy as np
import pytest
import torch

from oracle import decode_oracle as dor

TOL = 2e-6


def tiny_model(model_type="llama", kv_heads=4, bias=False, seed=0, vocab=97, layers=2):
    from ssalaad_amd.bundle import build_model_from_config

    cfg = {"model_type": model_type, "hidden_size": 64, "intermediate_size": 96,
           "num_hidden_layers": layers, "num_attention_heads": 4, "num_key_value_heads": kv_heads,
           "head_dim": 16, "vocab_size": vocab, "max_position_embeddings": 64,
           "rms_norm_eps": 1e-6, "rope_theta": 10000.0, "hidden_act": "silu",
           "tie_word_embeddings": False, "attention_bias": bias}
    torch.manual_seed(seed)
    model = build_model_from_config(cfg, attn_implementation="eager").double().eval()
    with torch.no_grad():
        for name, prm in model.named_parameters():
            if "norm" in name:
                prm.copy_(1.0 + 0.1 * torch.randn_like(prm))
            elif name.endswith("bias"):
                prm.copy_(0.1 * torch.randn_like(prm))
            else:
                prm.copy_(0.2 * torch.randn_like(prm))
    return model


@pytest.mark.parametrize("model_type,kv_heads,bias", [
    ("llama", 4, False), ("llama", 2, False), ("llama", 1, True), ("qwen3", 2, False),
])
def test_decode_steps_reproduce_the_full_sequence_forward(model_type, kv_heads, bias):
    model = tiny_model(model_type, kv_heads, bias)
    P = dor.params_from_hf(model)
    B, T = 2, 9
    ids = torch.randint(0, 97, (B, T), generator=torch.Generator().manual_seed(1))
    with torch.no_grad():
        want = model(input_ids=ids, use_cache=False).logits.numpy()
    cache = dor.KVCache.empty(len(P.layers), B, P.kv_heads, T, P.head_dim)
    for t in range(T):
        got = dor.decode_step(P, cache, ids[:, t].numpy(), [t] * B)
        err = np.abs(got - want[:, t]).max() / np.abs(want[:, t]).max()
        assert err < TOL, (t, err)


@pytest.mark.parametrize("model_type,kv_heads,bias", [
    ("llama", 4, False), ("llama", 2, True), ("qwen3", 2, False),
])
def test_whole_sequence_forward_matches_transformers_and_decode_steps(model_type, kv_heads, bias):
    model = tiny_model(model_type, kv_heads, bias, seed=3)
    P = dor.params_from_hf(model)
    B, T = 2, 9
    ids = torch.randint(0, 97, (B, T), generator=torch.Generator().manual_seed(4))
    with torch.no_grad():
        want = model(input_ids=ids, use_cache=False).logits.numpy()
    got = dor.forward(P, ids.numpy())
    assert np.abs(got - want).max() / np.abs(want).max() < TOL
    cache = dor.KVCache.empty(len(P.layers), B, P.kv_heads, T, P.head_dim)
    for t in range(T):
        step = dor.decode_step(P, cache, ids[:, t].numpy(), [t] * B)
        assert np.abs(got[:, t] - step).max() / np.abs(step).max() < 1e-12


def test_ragged_positions_match_per_sequence_runs():
    """Sequences at different positions in one step give their own logits."""
    model = tiny_model("llama", 2)
    P = dor.params_from_hf(model)
    ids = torch.randint(0, 97, (2, 6), generator=torch.Generator().manual_seed(2)).numpy()
    with torch.no_grad():
        want0 = model(input_ids=torch.from_numpy(ids[:1, :6])).logits.numpy()[0, 5]
        want1 = model(input_ids=torch.from_numpy(ids[1:, :3])).logits.numpy()[0, 2]
    cache = dor.KVCache.empty(len(P.layers), 2, P.kv_heads, 6, P.head_dim)
    for t in range(3):
        dor.decode_step(P, cache, ids[:, t], [t, t])
    for t in range(3, 5):  # sequence 1 waits at position 2
        c1 = dor.KVCache([k[:1] for k in cache.k], [v[:1] for v in cache.v])
        dor.decode_step(P, c1, ids[:1, t], [t])
    got = dor.decode_step(P, cache, [ids[0, 5], ids[1, 2]], [5, 2])
    assert np.abs(got[0] - want0).max() < TOL * np.abs(want0).max()
    assert np.abs(got[1] - want1).max() < TOL * np.abs(want1).max()


def test_greedy_matches_the_recompute_loop():
    """The cached greedy loop picks the same tokens as the reference's loop, which
    recomputes the prefix with the full forward (generate.py:12-26)."""
    model = tiny_model("llama", 4)
    P = dor.params_from_hf(model)
    prompt = torch.randint(0, 97, (2, 4), generator=torch.Generator().manual_seed(3))
    seq = prompt
    with torch.no_grad():
        for _ in range(5):
            logits = model(input_ids=seq, use_cache=False).logits[:, -1]
            seq = torch.cat((seq, logits.argmax(-1, keepdim=True)), dim=1)
    assert np.array_equal(dor.greedy(P, prompt.numpy(), 5), seq.numpy())


def test_rms_norm_and_rotation_closed_forms():
    rng = np.random.default_rng(0)
    x = rng.standard_normal((3, 16))
    y = dor.rms_norm(x, np.ones(16), 0.0)
    assert np.allclose(np.sqrt((y * y).mean(-1)), 1.0)
    inv = 1.0 / 10000 ** (np.arange(0, 16, 2) / 16)
    cos, sin = dor.rope_tables(inv, [7])
    r = dor.rotate(x, cos[0], sin[0])
    # a rotation of each (j, j + 8) pair: norms kept, position 0 is the identity
    assert np.allclose(np.linalg.norm(r, axis=-1), np.linalg.norm(x, axis=-1))
    c0, s0 = dor.rope_tables(inv, [0])
    assert np.allclose(dor.rotate(x, c0[0], s0[0]), x)
    # relative-position property: <R_a q, R_b k> depends on a - b only
    q, k = x[0], x[1]
    ca, sa = dor.rope_tables(inv, [5, 9, 2, 6])
    d1 = dor.rotate(q, ca[1], sa[1]) @ dor.rotate(k, ca[0], sa[0])
    d2 = dor.rotate(q, ca[3], sa[3]) @ dor.rotate(k, ca[2], sa[2])
    assert abs(d1 - d2) < 1e-12
