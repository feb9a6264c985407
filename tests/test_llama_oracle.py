"""Pins of the Llama oracle (oracle/llama_oracle.py) on the CPU: the
Transformers LlamaForCausalLM the reference's correctness check runs
(hf_benchmark.py:764-823), closed forms and invariants."""

import numpy as np
import pytest
import torch

from inferkernellab_amd.llama import LlamaConfig, random_llama
from oracle import llama_oracle as lo

TINY = dict(vocab_size=97, hidden_size=64, intermediate_size=128, num_hidden_layers=2,
            num_attention_heads=4, num_key_value_heads=2, rope_theta=10000.0, rms_norm_eps=1e-6)


def _tiny(**kw):
    cfg = LlamaConfig(**{**TINY, **kw})
    return cfg, random_llama(cfg, seed=3, device="cpu", dtype=torch.float32)


def test_oracle_matches_transformers_llama():
    transformers = pytest.importorskip("transformers")
    cfg, model = _tiny()
    hf_cfg = transformers.LlamaConfig(
        vocab_size=cfg.vocab_size, hidden_size=cfg.hidden_size, intermediate_size=cfg.intermediate_size,
        num_hidden_layers=cfg.num_hidden_layers, num_attention_heads=cfg.num_attention_heads,
        num_key_value_heads=cfg.num_key_value_heads, rope_theta=cfg.rope_theta, rms_norm_eps=cfg.rms_norm_eps,
        max_position_embeddings=64, attention_bias=False, mlp_bias=False, tie_word_embeddings=False)
    hf_cfg._attn_implementation = "eager"
    hf = transformers.LlamaForCausalLM(hf_cfg).float().eval()
    missing, unexpected = hf.load_state_dict(model.state_dict(), strict=False)
    assert not unexpected and all("rotary" in k for k in missing)
    ids = [5, 17, 3, 96, 0, 44, 44, 12, 8, 61, 2, 70]
    with torch.no_grad():
        ref = hf(torch.tensor([ids]), use_cache=False).logits[0].numpy()
    ours = lo.full_sequence_logits(lo.weights_from_model(model), cfg, ids)
    assert np.abs(ours - ref).max() < 1e-4


def test_zero_layer_model_is_head_of_normed_embedding():
    cfg, model = _tiny(num_hidden_layers=0)
    w = lo.weights_from_model(model)
    ids = [1, 2, 3]
    x = w["model.embed_tokens.weight"][ids]
    x = x / np.sqrt((x * x).mean(-1, keepdims=True) + 1e-6)
    np.testing.assert_allclose(lo.full_sequence_logits(w, cfg, ids), x @ w["lm_head.weight"].T, atol=1e-5)


def test_rope_is_a_relative_rotation():
    gen = np.random.default_rng(0)
    d = 16
    q = gen.standard_normal((1, 1, d)).astype(np.float32)
    k = gen.standard_normal((1, 1, d)).astype(np.float32)
    c0, s0 = lo.rope_tables(np.array([0]), d, 10000.0)
    np.testing.assert_allclose(lo.rope(q, c0, s0), q, atol=1e-6)  # position 0: identity

    def dot(m, n):
        cm, sm = lo.rope_tables(np.array([m]), d, 10000.0)
        cn, sn = lo.rope_tables(np.array([n]), d, 10000.0)
        return float((lo.rope(q, cm, sm) * lo.rope(k, cn, sn)).sum())

    assert abs(dot(7, 3) - dot(24, 20)) < 1e-4 and abs(dot(7, 3) - dot(4, 0)) < 1e-4
    c, s = lo.rope_tables(np.array([13]), d, 10000.0)
    assert abs(np.linalg.norm(lo.rope(q, c, s)) - np.linalg.norm(q)) < 1e-5


def test_causal_logits_ignore_later_tokens():
    cfg, model = _tiny()
    w = lo.weights_from_model(model)
    a = lo.full_sequence_logits(w, cfg, [4, 9, 1, 33, 7])
    b = lo.full_sequence_logits(w, cfg, [4, 9, 1, 80, 80])
    np.testing.assert_array_equal(a[:3], b[:3])
    assert np.abs(a[3:] - b[3:]).max() > 1e-3


def test_teacher_forced_rows_line_up_with_generated_tokens():
    cfg, model = _tiny()
    w = lo.weights_from_model(model)
    prompt, gen = [3, 1, 4], [1, 5, 9]
    tf = lo.teacher_forced_logits(w, cfg, prompt, gen)
    full = lo.full_sequence_logits(w, cfg, prompt + gen[:-1])
    assert tf.shape == (3, cfg.vocab_size)
    np.testing.assert_array_equal(tf[0], full[2])
    np.testing.assert_array_equal(tf[2], full[4])


def test_planted_rope_sign_mistake_is_caught(monkeypatch):
    transformers = pytest.importorskip("transformers")
    cfg, model = _tiny()
    hf_cfg = transformers.LlamaConfig(
        vocab_size=cfg.vocab_size, hidden_size=cfg.hidden_size, intermediate_size=cfg.intermediate_size,
        num_hidden_layers=cfg.num_hidden_layers, num_attention_heads=cfg.num_attention_heads,
        num_key_value_heads=cfg.num_key_value_heads, rope_theta=cfg.rope_theta, rms_norm_eps=cfg.rms_norm_eps,
        max_position_embeddings=64, attention_bias=False, mlp_bias=False, tie_word_embeddings=False)
    hf_cfg._attn_implementation = "eager"
    hf = transformers.LlamaForCausalLM(hf_cfg).float().eval()
    hf.load_state_dict(model.state_dict(), strict=False)
    ids = [5, 17, 3, 96, 0, 44]
    with torch.no_grad():
        ref = hf(torch.tensor([ids]), use_cache=False).logits[0].numpy()

    def wrong_rope(x, cos, sin, r=lo.rounder(None)):
        half = x.shape[-1] // 2
        rot = np.concatenate([x[..., half:], x[..., :half]], axis=-1)  # sign dropped
        return r(r(x * cos[:, None, :]) + r(rot * sin[:, None, :]))

    monkeypatch.setattr(lo, "rope", wrong_rope)
    ours = lo.full_sequence_logits(lo.weights_from_model(model), cfg, ids)
    assert np.abs(ours - ref).max() > 1e-3


def _torch_forward(model, ids):
    """The runner's op sequence on the CPU in the model's dtype: every torch
    op rounds its output to that dtype; attention in float32."""
    from inferkernellab_amd.llama import rotate_half

    m, cfg = model.model, model.config
    h, kv, d = cfg.num_attention_heads, cfg.num_key_value_heads, cfg.head_dim
    t = len(ids)
    x = m.embed_tokens(torch.tensor(ids))
    cos, sin = m.rotary_emb(x, torch.arange(t))
    cos, sin = cos.unsqueeze(1), sin.unsqueeze(1)
    causal = torch.ones(t, t, dtype=torch.bool).tril()
    for layer in m.layers:
        a = layer.input_layernorm(x)
        at = layer.self_attn
        q, k = at.q_proj(a).view(t, h, d), at.k_proj(a).view(t, kv, d)
        v = at.v_proj(a).view(t, kv, d)
        q, k = q * cos + rotate_half(q) * sin, k * cos + rotate_half(k) * sin
        qf = q.float().transpose(0, 1)
        kf = k.float().repeat_interleave(h // kv, dim=1).permute(1, 2, 0)
        vf = v.float().repeat_interleave(h // kv, dim=1).transpose(0, 1)
        s = (qf @ kf) * d ** -0.5
        o = (torch.softmax(s.masked_fill(~causal, float("-inf")), -1) @ vf).transpose(0, 1).to(x.dtype)
        x = x + at.o_proj(o.reshape(t, h * d))
        b = layer.post_attention_layernorm(x)
        x = x + layer.mlp.down_proj(layer.mlp.act_fn(layer.mlp.gate_proj(b)) * layer.mlp.up_proj(b))
    return model.lm_head(m.norm(x)).float().numpy()


@pytest.mark.parametrize("dtype,name", [(torch.bfloat16, "bfloat16"), (torch.float16, "float16")])
def test_rounded_mode_matches_the_modules_run_in_that_dtype(dtype, name, monkeypatch):
    """round_to restates a run in that dtype: against the same modules run
    in it by torch on the CPU (each op rounding its output), the logits
    agree to a unit in the last place at most, and on average far closer
    than the float32 oracle on the same (exactly representable) weights.
    Two planted mistakes are caught: float32 RoPE frequencies (the module's
    buffer is converted with its weights) and an unrounded RMSNorm row."""
    cfg, model = _tiny(num_hidden_layers=3)
    gen = torch.Generator().manual_seed(7)
    with torch.no_grad():
        for pname, p in model.named_parameters():
            if pname.endswith("norm.weight"):  # off 1.0, so that both norm roundings show
                p.copy_(1.0 + 0.3 * torch.randn(p.shape, generator=gen))
    model = model.to(dtype)
    ids = [5, 17, 3, 96, 0, 44, 44, 12, 8, 61, 2, 70, 9, 9, 31, 1]
    with torch.no_grad():
        ref = _torch_forward(model, ids)
    w = lo.weights_from_model(model)
    ulp = np.abs(ref).max() * (2.0 ** -8 if name == "bfloat16" else 2.0 ** -11)
    ours = lo.full_sequence_logits(w, cfg, ids, round_to=name)
    exact = lo.full_sequence_logits(w, cfg, ids)
    err, mean_err, mean32 = np.abs(ours - ref).max(), np.abs(ours - ref).mean(), np.abs(exact - ref).mean()
    assert err <= ulp and mean_err * 4 < mean32, (err, ulp, mean_err, mean32)

    tables = lo.rope_tables
    monkeypatch.setattr(lo, "rope_tables", lambda pos, d, theta, r=None: tables(pos, d, theta))
    planted = lo.full_sequence_logits(w, cfg, ids, round_to=name)
    monkeypatch.setattr(lo, "rope_tables", tables)
    assert np.abs(planted - ref).mean() > 2 * mean_err + 1e-6

    def unrounded_norm(x, wt, eps, r=lo.rounder(None)):
        x = x.astype(np.float32)
        return r(wt * (x / np.sqrt(np.mean(x * x, axis=-1, keepdims=True) + np.float32(eps))))

    monkeypatch.setattr(lo, "rmsnorm", unrounded_norm)
    planted = lo.full_sequence_logits(w, cfg, ids, round_to=name)
    assert np.abs(planted - ref).mean() > 2 * mean_err + 1e-6
