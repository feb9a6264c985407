"""CPU oracle of Llama decoding over the paged cache — TEST INFRASTRUCTURE ONLY.

Only ``tests/`` (and ``__graft_entry__.smoke()`` / ``bench.py``'s CPU leg)
may use this module, as the checker; the product path never does.

A numpy float32 full-sequence causal forward of a Llama decoder, the
reference's correctness oracle for its paged Llama runner (the eager
full-sequence path of hf_benchmark.py:764-823) restated without
Transformers. One forward over ``prompt + generated[:-1]`` gives, at
position p, the logits that choose token p + 1 — all of a run's
teacher-forced decode logits at once.

Arithmetic (hf_benchmark.py:408-454 for the per-layer step; the Llama
architecture of the Transformers model the reference loads):

* ``rmsnorm``: ``x / sqrt(mean(x^2) + eps) * w``;
* ``rope``: rotate-half RoPE, ``inv_freq = theta^(-2i/D)``, angle = p * inv_freq
  repeated over both halves; ``x * cos + rotate_half(x) * sin``;
* attention: per query head h the kv head ``h // (H / Hkv)``, scale
  ``D^-0.5``, causal softmax in float32;
* MLP: ``down(silu(gate(x)) * up(x))``; residual adds around both blocks;
  final norm, then ``lm_head``.

``round_to="bfloat16"`` (or ``"float16"``) restates a model run in that
dtype: every op's output is rounded to it where torch's ops on such tensors
round (linear layers, RMSNorm's normalised rows and its weight product, the
RoPE tables and each term and sum of the rotation, the attention output,
residual adds, SiLU and the gate product, the logits); the attention itself
stays float32, as the paged kernels compute it.

Parity pins (tests/test_llama_oracle.py): Transformers' ``LlamaForCausalLM``
(eager attention, float32, CPU) on the same weights; a zero-layer model is
``lm_head(norm(embedding))``; RoPE is norm-preserving, the identity at
position 0 and relative (q(m).k(n) depends on m - n only); causality (later
tokens never change earlier logits).
"""

from __future__ import annotations

import numpy as np

from oracle.paged_oracle import bf16_bits_to_f32, f32_to_bf16_bits


def weights_from_model(model) -> dict:
    """float32 numpy copies of a Llama model's parameters (exact for bf16/fp16)."""
    return {name: p.detach().float().cpu().numpy() for name, p in model.named_parameters()}


def rounder(dtype: str | None):
    """x -> x rounded to `dtype` and widened back to float32 (identity for None / float32)."""
    if dtype in (None, "float32"):
        return lambda x: np.asarray(x, dtype=np.float32)
    if dtype == "bfloat16":
        return lambda x: bf16_bits_to_f32(f32_to_bf16_bits(np.asarray(x, dtype=np.float32)))
    if dtype == "float16":
        return lambda x: np.asarray(x, dtype=np.float32).astype(np.float16).astype(np.float32)
    raise ValueError(f"unsupported dtype: {dtype}")


def rmsnorm(x: np.ndarray, w: np.ndarray, eps: float, r=rounder(None)) -> np.ndarray:
    """Normalised in float32, rounded, then the weight product rounded."""
    x = x.astype(np.float32)
    return r(w * r(x / np.sqrt(np.mean(x * x, axis=-1, keepdims=True) + np.float32(eps))))


def rope_tables(positions: np.ndarray, head_dim: int, theta: float, r=rounder(None)):
    """float32 cos / sin [T, D]. The inverse frequencies pass through `r`:
    a model converted to a 16-bit dtype holds them in that dtype (they are a
    floating-point buffer of the module), and its angles are float32
    products of those rounded values."""
    inv = r(1.0 / (theta ** (np.arange(0, head_dim, 2, dtype=np.float32) / head_dim)))
    ang = positions.astype(np.float32)[:, None] * inv.astype(np.float32)[None, :]
    ang = np.concatenate([ang, ang], axis=-1)
    return np.cos(ang).astype(np.float32), np.sin(ang).astype(np.float32)


def rope(x: np.ndarray, cos: np.ndarray, sin: np.ndarray, r=rounder(None)) -> np.ndarray:
    """x [T, heads, D]; cos/sin [T, D] (already in the run's dtype)."""
    half = x.shape[-1] // 2
    rot = np.concatenate([-x[..., half:], x[..., :half]], axis=-1)
    return r(r(x * cos[:, None, :]) + r(rot * sin[:, None, :]))


def causal_attention(q: np.ndarray, k: np.ndarray, v: np.ndarray) -> np.ndarray:
    """q [T, H, D], k/v [T, Hkv, D] -> [T, H, D]; position t sees 0..t."""
    t, h, d = q.shape
    group = h // k.shape[1]
    kk = np.repeat(k, group, axis=1).transpose(1, 2, 0)  # [H, D, T]
    vv = np.repeat(v, group, axis=1).transpose(1, 0, 2)  # [H, T, D]
    s = np.matmul(q.transpose(1, 0, 2), kk) * np.float32(d ** -0.5)  # [H, T, T]
    s = np.where(np.tril(np.ones((t, t), dtype=bool))[None], s, -np.inf)
    s = s - s.max(axis=-1, keepdims=True)
    p = np.exp(s)
    p /= p.sum(axis=-1, keepdims=True)
    return np.matmul(p, vv).transpose(1, 0, 2).astype(np.float32)


def full_sequence_logits(w: dict, config, token_ids, round_to: str | None = None) -> np.ndarray:
    """float32 logits [T, vocab] of a causal forward over `token_ids`
    (with `round_to`, of a run in that dtype)."""
    r = rounder(round_to)
    ids = np.asarray(token_ids, dtype=np.int64)
    h_heads, kv_heads = int(config.num_attention_heads), int(config.num_key_value_heads)
    d = int(getattr(config, "head_dim", None) or config.hidden_size // h_heads)
    eps = float(config.rms_norm_eps)
    cos, sin = rope_tables(np.arange(len(ids)), d, float(config.rope_theta), r)
    cos, sin = r(cos), r(sin)
    x = r(w["model.embed_tokens.weight"][ids])
    for i in range(int(config.num_hidden_layers)):
        p = f"model.layers.{i}."
        a = rmsnorm(x, w[p + "input_layernorm.weight"], eps, r)
        q = r(a @ w[p + "self_attn.q_proj.weight"].T).reshape(len(ids), h_heads, d)
        k = r(a @ w[p + "self_attn.k_proj.weight"].T).reshape(len(ids), kv_heads, d)
        v = r(a @ w[p + "self_attn.v_proj.weight"].T).reshape(len(ids), kv_heads, d)
        o = r(causal_attention(rope(q, cos, sin, r), rope(k, cos, sin, r), v))
        x = r(x + r(o.reshape(len(ids), h_heads * d) @ w[p + "self_attn.o_proj.weight"].T))
        m = rmsnorm(x, w[p + "post_attention_layernorm.weight"], eps, r)
        g = r(m @ w[p + "mlp.gate_proj.weight"].T)
        act = r(r(g / (1.0 + np.exp(-g))) * r(m @ w[p + "mlp.up_proj.weight"].T))
        x = r(x + r(act @ w[p + "mlp.down_proj.weight"].T))
    x = rmsnorm(x, w["model.norm.weight"], eps, r)
    return r(x @ w["lm_head.weight"].T).astype(np.float32)


def teacher_forced_logits(w: dict, config, prompt, generated, round_to: str | None = None) -> np.ndarray:
    """[len(generated), vocab]: row j = logits that choose generated[j]."""
    seq = list(prompt) + list(generated[:-1])
    logits = full_sequence_logits(w, config, seq, round_to)
    return logits[len(prompt) - 1:]
