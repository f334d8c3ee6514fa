"""CPU oracle for the KV-cached decode step of a LLaMA / Qwen3 decoder.

TEST INFRASTRUCTURE ONLY. This module is the checker: only tests/ may import
it, and never as the thing measured or shipped. The product path
(ssalaad_amd.decode) never calls it.

The reference has no cached decode: its greedy generation recomputes the whole
prefix each step with the Hugging Face forward (ssalaad/inference/generate.py:
1-26) of the model that build_efficient_model returns (ssalaad/efficient/
model.py:11-60). The arithmetic of that forward lives in the third-party
package transformers (unpinned in the reference's pyproject.toml:14; this image
has 5.15.0). This module restates it in NumPy float64, one token per sequence
per step, from a key/value cache:

  rms_norm        transformers/models/llama/modeling_llama.py:53-70 (LlamaRMSNorm)
  rope_tables     modeling_llama.py:73-127 (LlamaRotaryEmbedding, default rope)
  rotate          modeling_llama.py:130-160 (rotate_half, apply_rotary_pos_emb)
  attention       modeling_llama.py:191-214 (eager_attention_forward; causal,
                  so a decode query sees every cached position up to its own)
  forward         the same forward over whole sequences at once (every position's
                  logits, causal attention), for prefill-sized model checks
  decode_step     modeling_llama.py:217-325 (LlamaAttention, LlamaDecoderLayer),
                  :163-177 (LlamaMLP with silu), :347-418 (LlamaModel.forward),
                  :421-493 (LlamaForCausalLM: logits = lm_head(norm(h)));
                  Qwen3 adds a per-head RMSNorm of q and k before the rotation
                  (transformers/models/qwen3/modeling_qwen3.py:211-280,
                  Qwen3Attention, :252-253).

Pinned by tests/test_decode_oracle.py against the library routine itself:
decode_step, run token by token from an empty cache, reproduces the logits of
transformers' LlamaForCausalLM / Qwen3ForCausalLM full-sequence forward in
a float64 model at every position, for MHA and grouped-query attention, with
and without projection biases. The bound is 2e-6 (normalised): transformers
evaluates RMSNorm and the rotary tables in fp32 even in a float64 model.
forward is pinned the same way and against decode_step at every position.
rms_norm and rotate are also checked against their closed forms (unit RMS,
norm preservation of the rotation).
"""

from __future__ import annotations

from dataclasses import dataclass, field

import numpy as np


@dataclass
class DecoderParams:
    """Float64 weights of a decoder. Linear weights are [out, in] (y = W x + b)."""

    embed: np.ndarray
    layers: list[dict]
    norm: np.ndarray
    lm_head: np.ndarray
    inv_freq: np.ndarray
    eps: float
    heads: int
    kv_heads: int
    head_dim: int
    attention_scaling: float = 1.0
    qk_norm: bool = False


@dataclass
class KVCache:
    """Per layer and sequence, keys and values [kv_heads, max_ctx, head_dim]."""

    k: list = field(default_factory=list)
    v: list = field(default_factory=list)

    @classmethod
    def empty(cls, n_layers: int, batch: int, kv_heads: int, max_ctx: int, head_dim: int):
        shape = (batch, kv_heads, max_ctx, head_dim)
        return cls([np.zeros(shape) for _ in range(n_layers)],
                    [np.zeros(shape) for _ in range(n_layers)])


def params_from_hf(model) -> DecoderParams:
    """Read a transformers Llama/Qwen3 causal LM whose projections are nn.Linear."""
    cfg = model.config
    f = lambda t: t.detach().to("cpu").double().numpy()  # noqa: E731
    hd = getattr(cfg, "head_dim", None) or cfg.hidden_size // cfg.num_attention_heads
    qk_norm = cfg.model_type == "qwen3"
    layers = []
    for layer in model.model.layers:
        at, mlp = layer.self_attn, layer.mlp
        d = {"in_norm": f(layer.input_layernorm.weight),
             "post_norm": f(layer.post_attention_layernorm.weight)}
        for name, mod in (("q", at.q_proj), ("k", at.k_proj), ("v", at.v_proj), ("o", at.o_proj),
                          ("gate", mlp.gate_proj), ("up", mlp.up_proj), ("down", mlp.down_proj)):
            d[name] = f(mod.weight)
            d[name + "_bias"] = f(mod.bias) if mod.bias is not None else None
        if qk_norm:
            d["q_norm"], d["k_norm"] = f(at.q_norm.weight), f(at.k_norm.weight)
        layers.append(d)
    rot = model.model.rotary_emb
    return DecoderParams(
        embed=f(model.model.embed_tokens.weight), layers=layers, norm=f(model.model.norm.weight),
        lm_head=f(model.lm_head.weight), inv_freq=f(rot.inv_freq), eps=float(cfg.rms_norm_eps),
        heads=cfg.num_attention_heads, kv_heads=cfg.num_key_value_heads, head_dim=hd,
        attention_scaling=float(getattr(rot, "attention_scaling", 1.0)), qk_norm=qk_norm)


def rms_norm(x: np.ndarray, w: np.ndarray, eps: float) -> np.ndarray:
    """w · x / sqrt(mean(x²) + eps) over the last axis."""
    return w * (x / np.sqrt(np.mean(x * x, axis=-1, keepdims=True) + eps))


def rope_tables(inv_freq: np.ndarray, positions, scaling: float = 1.0):
    """cos, sin [len(positions), head_dim]: angles pos·inv_freq, repeated twice."""
    ang = np.outer(np.asarray(positions, dtype=np.float64), inv_freq)
    emb = np.concatenate([ang, ang], axis=-1)
    return np.cos(emb) * scaling, np.sin(emb) * scaling


def rotate(x: np.ndarray, cos: np.ndarray, sin: np.ndarray) -> np.ndarray:
    """x·cos + rotate_half(x)·sin, rotate_half(x) = (-x2, x1) over the last axis."""
    half = x.shape[-1] // 2
    rh = np.concatenate([-x[..., half:], x[..., :half]], axis=-1)
    return x * cos + rh * sin


def attention(q: np.ndarray, k: np.ndarray, v: np.ndarray, scale: float) -> np.ndarray:
    """q [heads, hd]; k, v [kv_heads, T, hd] -> [heads, hd]; head h reads kv head
    h // (heads // kv_heads)."""
    heads, kvh = q.shape[0], k.shape[0]
    rep = heads // kvh
    out = np.empty_like(q)
    for h in range(heads):
        kh = h // rep
        s = k[kh] @ q[h] * scale
        p = np.exp(s - s.max())
        out[h] = (p / p.sum()) @ v[kh]
    return out


def _linear(d: dict, name: str, x: np.ndarray) -> np.ndarray:
    y = d[name] @ x
    if d.get(name + "_bias") is not None:
        y = y + d[name + "_bias"]
    return y


def decode_step(P: DecoderParams, cache: KVCache, tokens, positions) -> np.ndarray:
    """Logits [batch, vocab] for one new token per sequence; appends to `cache`.

    Sequence b's token `tokens[b]` sits at `positions[b]`; its cache must hold
    the keys and values of positions 0 .. positions[b]-1.
    """
    hd, H, KH = P.head_dim, P.heads, P.kv_heads
    out = []
    for b, (tok, pos) in enumerate(zip(tokens, positions)):
        cos, sin = rope_tables(P.inv_freq, [pos], P.attention_scaling)
        h = P.embed[int(tok)].copy()
        for li, d in enumerate(P.layers):
            x = rms_norm(h, d["in_norm"], P.eps)
            q = _linear(d, "q", x).reshape(H, hd)
            k = _linear(d, "k", x).reshape(KH, hd)
            v = _linear(d, "v", x).reshape(KH, hd)
            if P.qk_norm:
                q = rms_norm(q, d["q_norm"], P.eps)
                k = rms_norm(k, d["k_norm"], P.eps)
            q, k = rotate(q, cos[0], sin[0]), rotate(k, cos[0], sin[0])
            cache.k[li][b, :, pos] = k
            cache.v[li][b, :, pos] = v
            a = attention(q, cache.k[li][b, :, : pos + 1], cache.v[li][b, :, : pos + 1],
                          hd ** -0.5)
            h = h + _linear(d, "o", a.reshape(-1))
            x = rms_norm(h, d["post_norm"], P.eps)
            g = _linear(d, "gate", x)
            u = _linear(d, "up", x)
            h = h + _linear(d, "down", g / (1.0 + np.exp(-g)) * u)
        out.append(P.lm_head @ rms_norm(h, P.norm, P.eps))
    return np.stack(out)


def forward(P: DecoderParams, ids) -> np.ndarray:
    """Logits [batch, T, vocab] of whole sequences ids [batch, T] (positions
    0 .. T−1, causal attention): decode_step's arithmetic on every position at once."""
    ids = np.asarray(ids)
    Bn, T = ids.shape
    hd, H, KH = P.head_dim, P.heads, P.kv_heads
    cos, sin = rope_tables(P.inv_freq, range(T), P.attention_scaling)  # [T, hd]
    causal = np.triu(np.full((T, T), -np.inf), 1)

    def lin(d, name, x):
        y = x @ d[name].T
        if d.get(name + "_bias") is not None:
            y = y + d[name + "_bias"]
        return y

    h = P.embed[ids].astype(np.float64)                                # [B, T, hidden]
    for d in P.layers:
        x = rms_norm(h, d["in_norm"], P.eps)
        q = lin(d, "q", x).reshape(Bn, T, H, hd).transpose(0, 2, 1, 3)   # [B, H, T, hd]
        k = lin(d, "k", x).reshape(Bn, T, KH, hd).transpose(0, 2, 1, 3)
        v = lin(d, "v", x).reshape(Bn, T, KH, hd).transpose(0, 2, 1, 3)
        if P.qk_norm:
            q = rms_norm(q, d["q_norm"], P.eps)
            k = rms_norm(k, d["k_norm"], P.eps)
        q, k = rotate(q, cos, sin), rotate(k, cos, sin)
        rep = H // KH
        k = np.repeat(k, rep, axis=1)
        v = np.repeat(v, rep, axis=1)
        s = q @ k.transpose(0, 1, 3, 2) * hd ** -0.5 + causal             # [B, H, T, T]
        pr = np.exp(s - s.max(axis=-1, keepdims=True))
        a = (pr / pr.sum(axis=-1, keepdims=True)) @ v                     # [B, H, T, hd]
        h = h + lin(d, "o", a.transpose(0, 2, 1, 3).reshape(Bn, T, H * hd))
        x = rms_norm(h, d["post_norm"], P.eps)
        g = lin(d, "gate", x)
        h = h + lin(d, "down", g / (1.0 + np.exp(-g)) * lin(d, "up", x))
    return rms_norm(h, P.norm, P.eps) @ P.lm_head.T


def greedy(P: DecoderParams, prompt: np.ndarray, max_new_tokens: int) -> np.ndarray:
    """The reference's greedy loop (generate.py:12-26) on the cached step:
    prompt [batch, T] -> [batch, T + max_new_tokens]."""
    B, T = prompt.shape
    cache = KVCache.empty(len(P.layers), B, P.kv_heads, T + max_new_tokens, P.head_dim)
    seq = [list(map(int, r)) for r in prompt]
    logits = None
    for t in range(T):
        logits = decode_step(P, cache, prompt[:, t], [t] * B)
    for t in range(T, T + max_new_tokens):
        nxt = logits.argmax(-1)
        for b in range(B):
            seq[b].append(int(nxt[b]))
        if t + 1 < T + max_new_tokens:
            logits = decode_step(P, cache, nxt, [t] * B)
    return np.array(seq, dtype=np.int64)
