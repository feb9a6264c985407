"""The callers of the paged path on the GPU: the synthetic decoder
(decode.py:151-592) and the Llama runner (hf_benchmark.py:131-700) with the
HIP append and attention operators, checked against the CPU oracles.

Synthetic decoder: the same runner with attention computed by the numpy
oracle (paged_reference) on a host copy of the cache and the torch append,
token for token, logits within 1e-4 (fp32) — the reference's
paged_reference vs paged_sdpa check (tests/test_decode.py:24-36). Llama:
teacher-forced logits of the numpy full-sequence oracle (the reference's
eager-Transformers check, hf_benchmark.py:764-823): max-abs 1e-3 and every
greedy token equal in fp32; in bf16 against the oracle run with bf16
rounding, a stated logit bound and every greedy flip within twice it."""

import numpy as np
import pytest
import torch

pytestmark = pytest.mark.gpu


def _oracle_runner_class():
    from inferkernellab_amd.decode import SyntheticDecodeRunner
    from oracle import paged_oracle as po

    class OracleAttentionRunner(SyntheticDecodeRunner):
        """Attention through the CPU oracle on a host copy of the cache."""

        def _attention(self, query, tables, lens, requests, context_lengths):
            dtype = {torch.float32: "float32", torch.float16: "float16", torch.bfloat16: "bfloat16"}[query.dtype]
            oc = po.OracleCache.__new__(po.OracleCache)
            oc.num_layers, oc.num_blocks, oc.block_size = 1, self.cache.layout.num_blocks, self.cache.layout.block_size
            oc.num_kv_heads, oc.head_dim, oc.dtype = self.cache.layout.num_kv_heads, self.cache.layout.head_dim, dtype

            def host(t):
                t = t.detach().cpu()
                return t.view(torch.int16).numpy().view(np.uint16) if t.dtype == torch.bfloat16 else t.numpy()

            oc.k, oc.v = host(self.cache.k), host(self.cache.v)
            q = po.to_f32(host(query), dtype)
            out = po.paged_decode_attention(q, oc, [r.block_table for r in requests], list(context_lengths))
            return torch.from_numpy(out).to(device=query.device, dtype=query.dtype)

    return OracleAttentionRunner


def _synthetic(num_kv_heads, backend="hip_paged", append="hip", runner=None, **kw):
    from inferkernellab_amd.decode import SyntheticDecodeRunner, SyntheticDecoderConfig

    prompts = kw.pop("prompts", None) or [[1, 2, 3], [7, 8, 9, 10]]
    cfg = dict(vocab_size=32, num_heads=4, num_kv_heads=num_kv_heads, head_dim=16, block_size=4,
               dtype=torch.float32, device="cuda", seed=19, backend=backend, append_backend=append,
               max_num_seqs=2, max_num_batched_tokens=4)
    cfg.update(kw)
    return (runner or SyntheticDecodeRunner)(SyntheticDecoderConfig(**cfg), prompts, max_new_tokens=3).run()


@pytest.mark.parametrize("backend", ["hip_paged", "hip_paged_grouped"])
@pytest.mark.parametrize("num_kv_heads", [4, 2, 1])
def test_synthetic_decoder_matches_oracle_attention(num_kv_heads, backend):
    print(f"synthetic decoder kv={num_kv_heads} backend={backend}", flush=True)
    hip = _synthetic(num_kv_heads, backend=backend)
    ref = _synthetic(num_kv_heads, append="torch", runner=_oracle_runner_class())
    assert hip.generated_tokens == ref.generated_tokens
    assert len(hip.logits) == len(ref.logits) == 3
    for a, b in zip(hip.logits, ref.logits):
        assert torch.allclose(a, b, atol=1e-4, rtol=1e-4)
    assert hip.used_blocks_peak > 0


def test_synthetic_gqa_bf16_mfma_matches_oracle_attention():
    """GQA 32/8, head_dim 128, block 16: the MFMA kernel inside the decoder."""
    print("synthetic decoder bf16 gqa32x8 hd128", flush=True)
    kw = dict(vocab_size=64, num_heads=32, head_dim=128, block_size=16, dtype=torch.bfloat16,
              max_num_seqs=4, max_num_batched_tokens=64,
              prompts=[[i % 64 for i in range(40)], [3] * 17, [5, 6] * 30, [1]])
    hip = _synthetic(8, **kw)
    ref = _synthetic(8, append="torch", runner=_oracle_runner_class(), **kw)
    # the first step sees identical caches: its logits agree to bf16 rounding
    assert (hip.logits[0] - ref.logits[0]).abs().max().item() < 2e-2
    assert hip.generated_tokens[0][0] == ref.generated_tokens[0][0]


@pytest.mark.parametrize("num_kv_heads", [4, 1])
def test_synthetic_token_and_batched_prefill_match(num_kv_heads):
    common = dict(max_num_batched_tokens=5, prompts=[[1, 2, 3, 4, 5], [7, 8, 9]])
    token = _synthetic(num_kv_heads, prefill_mode="token", **common)
    batched = _synthetic(num_kv_heads, prefill_mode="batched", **common)
    assert batched.generated_tokens == token.generated_tokens
    assert batched.prefill_batch_count == token.prefill_batch_count
    for a, b in zip(token.logits, batched.logits):
        assert torch.allclose(a, b, atol=1e-5, rtol=1e-5)


def test_synthetic_decoder_tables_blocks_and_single_run():
    from inferkernellab_amd.decode import SyntheticDecodeRunner, SyntheticDecoderConfig

    cfg = SyntheticDecoderConfig(vocab_size=16, num_heads=2, num_kv_heads=1, head_dim=16, block_size=4,
                                 dtype=torch.float32, device="cuda", seed=3, max_num_seqs=2,
                                 max_num_batched_tokens=8)
    runner = SyntheticDecodeRunner(cfg, [[1, 2, 3, 4, 5], [5, 6, 7, 8, 9, 10]], max_new_tokens=4)
    assert all(len(r.block_table) > 1 and any(b - a != 1 for a, b in zip(r.block_table, r.block_table[1:]))
               for r in runner.requests)
    result = runner.run()
    assert all(len(t) == 4 for t in result.generated_tokens)
    assert runner.runtime.stats().used_blocks == 0 and runner.runtime.stats().finished == 2
    assert result.tpot_wall_ms > 0 and result.tpot_device_ms > 0
    with pytest.raises(RuntimeError, match="only be run once"):
        runner.run()


# ------------------------------------------------------------------ Llama
def _llama(dtype, **kw):
    from inferkernellab_amd.llama import LlamaConfig, random_llama

    cfg = LlamaConfig(**{**dict(vocab_size=128, hidden_size=256, intermediate_size=512, num_hidden_layers=2,
                                num_attention_heads=4, num_key_value_heads=2), **kw})
    return cfg, random_llama(cfg, seed=2026, device="cuda", dtype=dtype)


def _check_llama(cfg, model, result, prompts, *, tol, margin_check):
    from oracle import llama_oracle as lo

    w = lo.weights_from_model(model)
    worst = 0.0
    for i, (prompt, gen) in enumerate(zip(prompts, result.generated_tokens)):
        ref = lo.teacher_forced_logits(w, cfg, prompt, gen)
        ours = torch.stack([step[i] for step in result.decode_logits]).numpy()
        assert ours.shape == ref.shape
        bound = tol * (1.0 if not margin_check else float(np.abs(ref).max()))
        err = float(np.abs(ours - ref).max())
        worst = max(worst, err)
        assert err <= bound, f"request {i}: logits max err {err} > {bound}"
        top2 = np.sort(ref, axis=-1)[:, -2:]
        clear = (top2[:, 1] - top2[:, 0]) > 2 * bound
        assert (np.asarray(gen)[clear] == ref.argmax(-1)[clear]).all(), f"request {i}: greedy token mismatch"
    return worst


@pytest.mark.parametrize("num_kv_heads,layers", [(4, 1), (2, 2)])
def test_llama_runner_fp32_matches_full_sequence_oracle(num_kv_heads, layers):
    from inferkernellab_amd.llama import LlamaPagedDecodeRunner

    print(f"llama fp32 kv={num_kv_heads} layers={layers}", flush=True)
    cfg, model = _llama(torch.float32, num_key_value_heads=num_kv_heads, num_hidden_layers=layers)
    prompts = [[(3 * i + 1) % 128 for i in range(21)], [(7 * i) % 128 for i in range(9)]]
    runner = LlamaPagedDecodeRunner(model, prompts, max_new_tokens=5, backend="hip_paged", block_size=4)
    result = runner.run()
    assert result.cache_released and runner.runtime.stats().used_blocks == 0
    _check_llama(cfg, model, result, prompts, tol=1e-3, margin_check=False)
    assert all(g == tuple(torch.stack(result.decode_logits)[:, i].argmax(-1).tolist())
               for i, g in enumerate(result.generated_tokens))


@pytest.mark.parametrize("prefill_mode", ["token", "batched"])
def test_llama_prefill_modes_match_oracle(prefill_mode):
    from inferkernellab_amd.llama import LlamaPagedDecodeRunner

    cfg, model = _llama(torch.float32)
    prompts = [[1, 2, 3, 4, 5], [6, 7, 8]]
    result = LlamaPagedDecodeRunner(model, prompts, max_new_tokens=3, block_size=4, max_num_batched_tokens=6,
                                    prefill_mode=prefill_mode).run()
    assert result.prefill_mode == prefill_mode and result.prefill_tokens == 8 and result.cache_released
    _check_llama(cfg, model, result, prompts, tol=1e-3, margin_check=False)


def test_llama_ragged_batched_prefill_over_nan_cache():
    """tests/test_hf_benchmark.py:101-123: NaN in every unwritten slot."""
    from inferkernellab_amd.llama import LlamaPagedDecodeRunner

    cfg, model = _llama(torch.float32)
    prompts = [[1, 2, 3, 4, 5], [6, 7, 8]]
    runner = LlamaPagedDecodeRunner(model, prompts, max_new_tokens=2, block_size=4, max_num_batched_tokens=8)
    runner.cache.k.fill_(float("nan"))
    runner.cache.v.fill_(float("nan"))
    result = runner.run()
    assert result.prefill_padding_tokens > 0 and result.cache_released
    _check_llama(cfg, model, result, prompts, tol=1e-3, margin_check=False)


def test_llama_bf16_gqa_hd128_matches_oracle():
    """16 query / 4 KV heads, head_dim 128 (the MFMA kernel), block 16."""
    from inferkernellab_amd.llama import LlamaPagedDecodeRunner

    print("llama bf16 16/4 hd128", flush=True)
    cfg, model = _llama(torch.bfloat16, hidden_size=2048, intermediate_size=1024, num_attention_heads=16,
                        num_key_value_heads=4, vocab_size=512, num_hidden_layers=2)
    gen = np.random.default_rng(7)
    prompts = [gen.integers(0, 512, size=n).tolist() for n in (70, 33, 129, 16)]
    result = LlamaPagedDecodeRunner(model, prompts, max_new_tokens=6, block_size=16,
                                    max_num_batched_tokens=128).run()
    assert result.cache_released
    _check_llama(cfg, model, result, prompts, tol=3e-2, margin_check=True)


@pytest.mark.parametrize("dtype,tol", [(torch.float32, 1e-4), (torch.bfloat16, 3e-2)])
def test_llama_hip_prefill_matches_torch_prefix_attention(dtype, tol):
    """The batched prefill with ikl_paged_prefill_attention (+ fused RoPE
    append) against the runner's torch gather + fp32 attention on the same
    model: chunked prompts (a 48-token budget splits them, so later chunks
    start past 0) and padding rows."""
    from inferkernellab_amd.llama import LlamaPagedDecodeRunner

    cfg, model = _llama(dtype, hidden_size=512, intermediate_size=512, num_attention_heads=8,
                        num_key_value_heads=2, vocab_size=256, num_hidden_layers=2)
    gen = np.random.default_rng(3)
    prompts = [gen.integers(0, 256, size=n).tolist() for n in (70, 33, 5)]
    kw = dict(max_new_tokens=4, block_size=16, max_num_batched_tokens=48)
    hip = LlamaPagedDecodeRunner(model, prompts, **kw).run()
    ref = LlamaPagedDecodeRunner(model, prompts, prefill_attention="torch", append_backend="torch", **kw).run()
    assert hip.prefill_batch_count > 1
    scale = float(ref.prompt_logits.float().abs().max())
    err = float((hip.prompt_logits.float() - ref.prompt_logits.float()).abs().max())
    assert err <= tol * scale, (err, scale)
    for a, b in zip(hip.decode_logits, ref.decode_logits):
        assert float((a.float() - b.float()).abs().max()) <= 2 * tol * scale


def test_llama_fp8_kv_cache_matches_its_torch_path_and_stays_near_bf16():
    """kv_cache_dtype=float8_e4m3fn: the HIP path (fused RoPE append into the
    FP8 cache, FP8 prefill and decode kernels) against the runner's torch
    path over the same quantised cache (torch quantiser + dequantised fp32
    prefix attention), and the FP8 run's logits near the bf16-cache run."""
    from inferkernellab_amd.llama import LlamaPagedDecodeRunner

    cfg, model = _llama(torch.bfloat16, hidden_size=512, intermediate_size=512, num_attention_heads=8,
                        num_key_value_heads=2, vocab_size=256, num_hidden_layers=2)
    gen = np.random.default_rng(11)
    prompts = [gen.integers(0, 256, size=n).tolist() for n in (70, 33, 5)]
    kw = dict(max_new_tokens=4, block_size=16, max_num_batched_tokens=48)
    fp8 = LlamaPagedDecodeRunner(model, prompts, kv_cache_dtype=torch.float8_e4m3fn, **kw).run()
    ref = LlamaPagedDecodeRunner(model, prompts, kv_cache_dtype=torch.float8_e4m3fn, prefill_attention="torch",
                                 append_backend="torch", **kw).run()
    bf16 = LlamaPagedDecodeRunner(model, prompts, **kw).run()
    scale = float(ref.prompt_logits.float().abs().max())
    err = float((fp8.prompt_logits.float() - ref.prompt_logits.float()).abs().max())
    assert err <= 3e-2 * scale, (err, scale)
    for a, b in zip(fp8.decode_logits, ref.decode_logits):
        assert float((a.float() - b.float()).abs().max()) <= 6e-2 * scale
    q_err = float((fp8.prompt_logits.float() - bf16.prompt_logits.float()).abs().max())
    print(f"FP8 vs bf16 KV cache: prompt logits max abs diff {q_err:.4f} (logit scale {scale:.3f})")
    assert q_err <= 0.15 * scale


def test_llama_sampling_is_seeded_and_eos_stops():
    from inferkernellab_amd.llama import LlamaPagedDecodeRunner

    cfg, model = _llama(torch.float32)
    prompts = [[1, 2, 3], [4, 5]]
    a = LlamaPagedDecodeRunner(model, prompts, max_new_tokens=4, temperature=0.8, top_p=0.9, seed=5).run()
    b = LlamaPagedDecodeRunner(model, prompts, max_new_tokens=4, temperature=0.8, top_p=0.9, seed=5).run()
    assert a.generated_tokens == b.generated_tokens
    assert all(len(lp) == 4 for lp in a.token_logprobs)
    greedy = LlamaPagedDecodeRunner(model, prompts, max_new_tokens=4).run()
    eos = greedy.generated_tokens[0][1]
    stopped = LlamaPagedDecodeRunner(model, prompts, max_new_tokens=4, eos_token_ids=[eos]).run()
    first = greedy.generated_tokens[0].index(eos)
    assert stopped.finish_reasons[0] == "eos"
    assert stopped.generated_tokens[0] == greedy.generated_tokens[0][:first + 1]
    assert stopped.cache_released


def _e2e_setup(dtype):
    from inferkernellab_amd.llama import LlamaConfig, random_llama

    cfg = LlamaConfig(vocab_size=32000, hidden_size=2048, intermediate_size=5632, num_hidden_layers=8,
                      num_attention_heads=16, num_key_value_heads=4, rope_theta=10000.0)
    model = random_llama(cfg, seed=0, device="cuda", dtype=dtype)
    gen = torch.Generator().manual_seed(0)
    prompts = torch.randint(0, 32000, (16, 512), generator=gen).tolist()
    return cfg, model, prompts


def _e2e_run(model, prompts):
    from inferkernellab_amd.llama import LlamaPagedDecodeRunner

    result = LlamaPagedDecodeRunner(model, prompts, max_new_tokens=64, block_size=16,
                                    max_num_batched_tokens=4096).run()
    print(f"prefill batches {result.prefill_batch_count} prefill {result.prefill_wall_ms:.1f} ms "
          f"tpot p50 {result.decode_p50_ms:.2f} ms", flush=True)
    assert result.prefill_batch_count == 2 and result.cache_released
    assert all(len(g) == 64 for g in result.generated_tokens)
    return result


def test_llama_e2e_fp32_greedy_tokens_equal_cpu_oracle():
    """The end-to-end configuration (8 layers, hidden 2048, 16 / 4 heads of
    128, intermediate 5632, vocab 32000, seed-0 weights; 16 prompts of 512
    random ids, batched prefill under 4096 tokens = 2 batches of 8, 64
    greedy steps) in fp32: at every step of every request the generated
    token is the argmax of the CPU oracle's teacher-forced logits, so a
    greedy CPU run produces the same 16 x 64 tokens."""
    from oracle import llama_oracle as lo

    print("llama e2e fp32 8x2048 b16 p512 n64", flush=True)
    cfg, model, prompts = _e2e_setup(torch.float32)
    result = _e2e_run(model, prompts)
    w = lo.weights_from_model(model)
    worst = 0.0
    for i, (prompt, gen) in enumerate(zip(prompts, result.generated_tokens)):
        ref = lo.teacher_forced_logits(w, cfg, prompt, gen)
        ours = torch.stack([step[i] for step in result.decode_logits]).numpy()
        worst = max(worst, float(np.abs(ours - ref).max()))
        assert list(gen) == ref.argmax(-1).tolist(), f"request {i}: greedy tokens differ from the CPU oracle"
    assert worst < 1e-3
    print(f"fp32 e2e: 1024/1024 tokens equal, logits max err {worst:.2e}", flush=True)


def test_llama_e2e_bf16_greedy_tokens_against_cpu_oracle():
    """The end-to-end configuration in bf16 against the CPU oracle run in
    bf16: the numpy forward of the same weights with every op's output
    rounded to bf16 where the bf16 modules round (round_to="bfloat16"; the
    attention in float32, as the kernels compute it), teacher-forced on all
    16 requests along the tokens the GPU run generated.

    The two runs round the same values at the same points; they part only
    where a float32 sum, accumulated in another order (GEMMs, softmax),
    lands on the other side of a bf16 rounding boundary, and 8 random-weight
    layers amplify those last-bit differences. The test states the result as
    BOUND on every logit of every step. A greedy token can then differ from
    the oracle's argmax only where the oracle's top logit leads the
    generated token's logit by at most 2 * BOUND; every flip is printed with
    that margin and must satisfy it, and at least 95 % of all greedy tokens
    agree (measured: logits within 0.086, 986 / 1024 tokens, every flip a
    near-tie within 0.047). The float32 oracle's agreement is reported
    beside it: a bf16 run cannot follow it (180 / 256 measured; its own
    rounding moves the prompt logits already by several tenths)."""
    from oracle import llama_oracle as lo

    bound = 0.12
    print("llama e2e bf16 8x2048 b16 p512 n64 vs cpu oracle (bf16 rounding)", flush=True)
    cfg, model, prompts = _e2e_setup(torch.bfloat16)
    result = _e2e_run(model, prompts)
    w = lo.weights_from_model(model)
    worst, worst0, flips, agree32 = 0.0, 0.0, [], 0
    for i, (prompt, gen) in enumerate(zip(prompts, result.generated_tokens)):
        ref = lo.teacher_forced_logits(w, cfg, prompt, gen, round_to="bfloat16")
        ours = torch.stack([step[i] for step in result.decode_logits]).float().numpy()
        err = np.abs(ours - ref).max(-1)
        worst, worst0 = max(worst, float(err.max())), max(worst0, float(err[0]))
        best = ref.argmax(-1)
        for j in np.nonzero(np.asarray(gen) != best)[0]:
            flips.append((i, int(j), int(gen[j]), int(best[j]), float(ref[j, best[j]] - ref[j, gen[j]])))
        if i % 4 == 0:
            agree32 += int((np.asarray(gen) == lo.teacher_forced_logits(w, cfg, prompt, gen).argmax(-1)).sum())
    for i, j, got, want, margin in flips:
        print(f"  flip request {i} step {j}: generated {got}, oracle argmax {want}, oracle margin {margin:.4f}")
    total = sum(len(g) for g in result.generated_tokens)
    print(f"bf16 e2e vs cpu oracle in bf16: logits max err {worst:.4f} (prompt logits {worst0:.4f}), "
          f"greedy agreement {total - len(flips)}/{total}, largest flip margin "
          f"{max((f[4] for f in flips), default=0.0):.4f} (allowed {2 * bound}); against the float32 "
          f"oracle (requests 0, 4, 8, 12): {agree32}/{4 * 64}", flush=True)
    assert worst <= bound
    assert all(margin <= 2 * bound for *_, margin in flips)
    assert total - len(flips) >= 0.95 * total


def eager_logits(model, tokens) -> torch.Tensor:
    """Dense full-sequence forward of the same modules (same dtype, same
    linear layers), causal attention in fp32: float32 logits [T, vocab]."""
    from inferkernellab_amd.llama import rotate_half

    m = model.model
    cfg = model.config
    h, kv, d = cfg.num_attention_heads, cfg.num_key_value_heads, cfg.head_dim
    ids = torch.tensor([tokens], device="cuda")
    t = ids.shape[1]
    x = m.embed_tokens(ids)
    cos, sin = m.rotary_emb(x, torch.arange(t, device="cuda").view(1, -1))
    cos, sin = cos.unsqueeze(2), sin.unsqueeze(2)
    mask = torch.ones(t, t, dtype=torch.bool, device="cuda").tril()
    for layer in m.layers:
        a = layer.input_layernorm(x)
        at = layer.self_attn
        q = at.q_proj(a).view(1, t, h, d)
        k = at.k_proj(a).view(1, t, kv, d)
        q, k = q * cos + rotate_half(q) * sin, k * cos + rotate_half(k) * sin
        v = at.v_proj(a).view(1, t, kv, d)
        qf = q[0].float().permute(1, 0, 2).contiguous()
        kf = k[0].float().repeat_interleave(h // kv, dim=1).permute(1, 2, 0).contiguous()
        vf = v[0].float().repeat_interleave(h // kv, dim=1).permute(1, 0, 2).contiguous()
        s = torch.matmul(qf, kf) * d ** -0.5
        o = torch.matmul(torch.softmax(s.masked_fill(~mask, float("-inf")), -1), vf)
        x = x + at.o_proj(o.permute(1, 0, 2).reshape(1, t, h * d).to(x.dtype))
        b = layer.post_attention_layernorm(x)
        x = x + layer.mlp.down_proj(layer.mlp.act_fn(layer.mlp.gate_proj(b)) * layer.mlp.up_proj(b))
    return model.lm_head(m.norm(x))[0].float()


def test_llama_e2e_bf16_matches_same_dtype_eager():
    """The same configuration in bf16 against a dense full-sequence forward
    of the same bf16 modules on the GPU (the reference's own check,
    hf_benchmark.py:764-823), teacher-forced on four requests.

    Bound: 0.1 on logits of std ~0.9. Both sides round every linear layer's
    output to bf16, but at different GEMM shapes (the runner's decode steps
    multiply 16 rows, the eager pass 575), so their outputs differ in the
    last bf16 bit and 8 random-weight layers amplify that. The prompt
    logits (step 0: batched prefill, before any paged decode step) already
    differ at the same level, which this test reports. Every greedy token
    whose eager top-2 margin exceeds 0.2 must match, and at least 95 % of
    all greedy tokens agree."""
    print("llama e2e bf16 8x2048 b16 p512 n64", flush=True)
    cfg, model, prompts = _e2e_setup(torch.bfloat16)
    result = _e2e_run(model, prompts)
    bound = 0.1
    worst, worst0, matched, total = 0.0, 0.0, 0, 0
    with torch.no_grad():
        for i in (0, 7, 8, 15):
            gen = result.generated_tokens[i]
            ref = eager_logits(model, list(prompts[i]) + list(gen[:-1]))[len(prompts[i]) - 1:].cpu().numpy()
            ours = torch.stack([step[i] for step in result.decode_logits]).numpy()
            err = np.abs(ours - ref).max(-1)
            worst, worst0 = max(worst, float(err.max())), max(worst0, float(err[0]))
            top2 = np.sort(ref, axis=-1)[:, -2:]
            clear = (top2[:, 1] - top2[:, 0]) > 2 * bound
            assert (np.asarray(gen)[clear] == ref.argmax(-1)[clear]).all(), f"request {i}: greedy token mismatch"
            matched += int((np.asarray(gen) == ref.argmax(-1)).sum())
            total += len(gen)
    print(f"bf16 e2e vs same-dtype eager: logits max err {worst:.4f} (prompt logits {worst0:.4f}), "
          f"greedy agreement {matched}/{total}", flush=True)
    assert worst <= bound and matched >= 0.95 * total


def test_llama_graph_decode_equals_eager_decode():
    """use_graph (the greedy step replayed as one HIP graph) gives the eager
    step's logits and tokens bit for bit."""
    from inferkernellab_amd.llama import LlamaPagedDecodeRunner

    cfg, model = _llama(torch.bfloat16, hidden_size=512, intermediate_size=1024, num_attention_heads=8,
                        num_key_value_heads=2, vocab_size=256, head_dim=64)
    gen = np.random.default_rng(9)
    prompts = [gen.integers(0, 256, size=n).tolist() for n in (40, 17, 95)]
    runs = [LlamaPagedDecodeRunner(model, prompts, max_new_tokens=20, block_size=16, use_graph=g).run()
            for g in (True, False)]
    assert runs[0].generated_tokens == runs[1].generated_tokens
    for a, b in zip(runs[0].decode_logits, runs[1].decode_logits):
        assert torch.equal(a, b)
    assert runs[0].cache_released
