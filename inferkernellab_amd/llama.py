"""Llama decoding over the paged KV cache with the HIP operators.

``LlamaPagedDecodeRunner`` is the caller of the paged path for a Llama
model (hf_benchmark.py:131-700). Per decode step and layer it computes
q/k/v for one token per request, rotates q and k (rotate-half RoPE) and
writes the rotated k and v into the paged cache in one fused HIP launch
(ikl_rope_append_kv; with ``append_backend="torch"``: torch RoPE and the
cache's index_put), runs the HIP paged decode attention over the request's
whole context (the current token included) and finishes the layer (o_proj +
residual, SwiGLU MLP + residual). Batched
prefill writes a whole prompt chunk per request, then attends causally over
the gathered paged prefix.

The runner reads the model through the attribute layout of a Transformers
``LlamaForCausalLM`` (``model.embed_tokens``, ``model.layers[i].self_attn.
q_proj`` ..., ``model.norm``, ``lm_head``, ``config``), so it accepts either
that class or :class:`LlamaForCausalLM` below, a dependency-free module with
the same layout and arithmetic (RMSNorm in fp32, RoPE tables in fp32 cast
to the activation dtype) for seeded random-weight models.
"""

from __future__ import annotations

import math
import time
from dataclasses import dataclass
from typing import Any, Sequence

import torch
from torch import nn

from . import ops
from .cache import PagedKVCache
from .decode import ATTENTION_BACKENDS, APPEND_BACKENDS, DecodeMetadata, percentile
from .runtime import InferenceRuntime
from .scheduler import InferenceRequest, TokenBudgetScheduler


# ---------------------------------------------------------------- the model
@dataclass
class LlamaConfig:
    vocab_size: int = 32000
    hidden_size: int = 2048
    intermediate_size: int = 5632
    num_hidden_layers: int = 8
    num_attention_heads: int = 16
    num_key_value_heads: int = 4
    head_dim: int | None = None
    rope_theta: float = 10000.0
    rms_norm_eps: float = 1e-6
    max_position_embeddings: int = 4096

    def __post_init__(self) -> None:
        if self.head_dim is None:
            self.head_dim = self.hidden_size // self.num_attention_heads


class RMSNorm(nn.Module):
    def __init__(self, size: int, eps: float):
        super().__init__()
        self.weight = nn.Parameter(torch.ones(size))
        self.variance_epsilon = eps

    def forward(self, x: torch.Tensor) -> torch.Tensor:
        x32 = x.float()
        x32 = x32 * torch.rsqrt(x32.pow(2).mean(-1, keepdim=True) + self.variance_epsilon)
        return self.weight * x32.to(x.dtype)


class RotaryEmbedding(nn.Module):
    """cos / sin tables of rotate-half RoPE for integer positions."""

    def __init__(self, head_dim: int, theta: float):
        super().__init__()
        inv = 1.0 / (theta ** (torch.arange(0, head_dim, 2, dtype=torch.float32) / head_dim))
        self.register_buffer("inv_freq", inv, persistent=False)

    def forward(self, x: torch.Tensor, position_ids: torch.Tensor):
        angles = position_ids.float().unsqueeze(-1) * self.inv_freq.to(x.device)
        emb = torch.cat((angles, angles), dim=-1)
        return emb.cos().to(x.dtype), emb.sin().to(x.dtype)


def rotate_half(x: torch.Tensor) -> torch.Tensor:
    half = x.shape[-1] // 2
    return torch.cat((-x[..., half:], x[..., :half]), dim=-1)


class _Attention(nn.Module):
    def __init__(self, c: LlamaConfig):
        super().__init__()
        self.q_proj = nn.Linear(c.hidden_size, c.num_attention_heads * c.head_dim, bias=False)
        self.k_proj = nn.Linear(c.hidden_size, c.num_key_value_heads * c.head_dim, bias=False)
        self.v_proj = nn.Linear(c.hidden_size, c.num_key_value_heads * c.head_dim, bias=False)
        self.o_proj = nn.Linear(c.num_attention_heads * c.head_dim, c.hidden_size, bias=False)


class _MLP(nn.Module):
    def __init__(self, c: LlamaConfig):
        super().__init__()
        self.gate_proj = nn.Linear(c.hidden_size, c.intermediate_size, bias=False)
        self.up_proj = nn.Linear(c.hidden_size, c.intermediate_size, bias=False)
        self.down_proj = nn.Linear(c.intermediate_size, c.hidden_size, bias=False)
        self.act_fn = nn.SiLU()


class _DecoderLayer(nn.Module):
    def __init__(self, c: LlamaConfig):
        super().__init__()
        self.input_layernorm = RMSNorm(c.hidden_size, c.rms_norm_eps)
        self.self_attn = _Attention(c)
        self.post_attention_layernorm = RMSNorm(c.hidden_size, c.rms_norm_eps)
        self.mlp = _MLP(c)


class _LlamaModel(nn.Module):
    def __init__(self, c: LlamaConfig):
        super().__init__()
        self.embed_tokens = nn.Embedding(c.vocab_size, c.hidden_size)
        self.layers = nn.ModuleList(_DecoderLayer(c) for _ in range(c.num_hidden_layers))
        self.norm = RMSNorm(c.hidden_size, c.rms_norm_eps)
        self.rotary_emb = RotaryEmbedding(c.head_dim, c.rope_theta)


class LlamaForCausalLM(nn.Module):
    """Llama decoder weights in the Transformers attribute layout."""

    def __init__(self, config: LlamaConfig):
        super().__init__()
        self.config = config
        self.model = _LlamaModel(config)
        self.lm_head = nn.Linear(config.hidden_size, config.vocab_size, bias=False)


def random_llama(config: LlamaConfig, *, seed: int = 0, device="cuda",
                 dtype: torch.dtype = torch.bfloat16) -> LlamaForCausalLM:
    """Seeded random model: linear and embedding weights ~ N(0, 0.02^2)
    drawn on the CPU in module order, norms = 1."""
    model = LlamaForCausalLM(config)
    gen = torch.Generator().manual_seed(seed)
    with torch.no_grad():
        for name, p in model.named_parameters():
            if name.endswith("layernorm.weight") or name.endswith("norm.weight"):
                p.fill_(1.0)
            else:
                p.copy_(torch.randn(p.shape, generator=gen) * 0.02)
    model = model.to(device=device, dtype=dtype).eval()
    for p in model.parameters():
        p.requires_grad_(False)
    return model


# --------------------------------------------------------------- the runner
@dataclass
class _StepBuffers:
    """Static device buffers of one captured decode step."""

    ids: torch.Tensor
    logits: torch.Tensor
    pos: torch.Tensor
    tok: torch.Tensor
    lens: torch.Tensor
    slots: torch.Tensor
    used: torch.Tensor | None = None
    graph: torch.cuda.CUDAGraph | None = None


@dataclass(frozen=True)
class LlamaPagedRunResult:
    """Outcome and timing of a Llama run (fields of hf_benchmark.py:88-128)."""

    backend: str
    append_backend: str
    prompt_lengths: tuple[int, ...]
    max_new_tokens: int
    generated_tokens: tuple[tuple[int, ...], ...]
    prompt_logits: torch.Tensor
    decode_logits: tuple[torch.Tensor, ...]
    prefill_wall_ms: float
    decode_step_wall_ms: tuple[float, ...]
    ttft_wall_ms: float
    tpot_wall_ms: float
    peak_memory_allocated_bytes: int
    peak_kv_memory_bytes: int
    used_blocks_peak: int
    cache_released: bool
    prefill_step_wall_ms: tuple[float, ...] = ()
    prefill_mode: str = "token"
    prefill_batch_count: int = 0
    prefill_tokens: int = 0
    prefill_padding_tokens: int = 0
    token_logprobs: tuple[tuple[float, ...], ...] = ()
    sampling_logprobs: tuple[tuple[float, ...], ...] = ()
    finish_reasons: tuple[str, ...] = ()

    @property
    def decode_p50_ms(self) -> float:
        return percentile(self.decode_step_wall_ms, 0.50)

    @property
    def decode_p95_ms(self) -> float:
        return percentile(self.decode_step_wall_ms, 0.95)

    @property
    def prefill_p50_ms(self) -> float:
        return percentile(self.prefill_step_wall_ms, 0.50)

    @property
    def prefill_p95_ms(self) -> float:
        return percentile(self.prefill_step_wall_ms, 0.95)


class LlamaPagedDecodeRunner:
    """Runs a Llama model one token per request per step over the paged cache."""

    def __init__(self, model: Any, prompts: Sequence[Sequence[int]], *, max_new_tokens: int,
                 backend: str = "hip_paged_grouped", block_size: int = 16, append_backend: str = "hip",
                 max_num_batched_tokens: int = 2048, prefill_mode: str = "batched",
                 temperature: float = 0.0, top_p: float = 1.0, seed: int = 2026,
                 eos_token_ids: Sequence[int] | None = None, use_graph: bool = True,
                 prefill_attention: str = "hip", kv_cache_dtype: torch.dtype | None = None) -> None:
        if not prompts:
            raise ValueError("at least one prompt is required")
        if max_new_tokens <= 0:
            raise ValueError("max_new_tokens must be positive")
        if block_size <= 0 or max_num_batched_tokens <= 0:
            raise ValueError("block-size and max-num-batched-tokens must be positive")
        if backend not in ATTENTION_BACKENDS:
            raise ValueError(f"unsupported backend: {backend}")
        if append_backend not in APPEND_BACKENDS:
            raise ValueError(f"unsupported append backend: {append_backend}")
        if prefill_mode not in ("batched", "token"):
            raise ValueError("prefill_mode must be batched or token")
        if prefill_attention not in ("hip", "torch"):
            raise ValueError("prefill_attention must be hip or torch")
        if not (math.isfinite(temperature) and temperature >= 0 and math.isfinite(top_p) and 0 < top_p <= 1):
            raise ValueError("temperature must be non-negative and top_p must be in (0, 1]")
        param = next(model.parameters())
        self.model, self.device, self.dtype = model, param.device, param.dtype
        if self.device.type != "cuda":
            raise ValueError(f"{backend} requires a GPU (torch 'cuda') device")
        cfg = model.config
        self.prompts = tuple(tuple(int(t) for t in p) for p in prompts)
        if any(len(p) == 0 for p in self.prompts):
            raise ValueError("prompts must be non-empty")
        if any(not 0 <= t < int(cfg.vocab_size) for p in self.prompts for t in p):
            raise ValueError("prompt token is outside the configured vocabulary")
        self.eos_token_ids = set(eos_token_ids or ())
        if any(not 0 <= t < int(cfg.vocab_size) for t in self.eos_token_ids):
            raise ValueError("EOS token id is outside the configured vocabulary")
        ops._require_backend()
        self.backend, self.append_backend, self.prefill_mode = backend, append_backend, prefill_mode
        self.prefill_attention = prefill_attention
        self.max_new_tokens, self.temperature, self.top_p = max_new_tokens, temperature, top_p
        self._attend = ATTENTION_BACKENDS[backend]
        self.num_layers = int(cfg.num_hidden_layers)
        self.num_heads = int(cfg.num_attention_heads)
        self.num_kv_heads = int(cfg.num_key_value_heads)
        self.head_dim = int(getattr(cfg, "head_dim", None) or cfg.hidden_size // cfg.num_attention_heads)
        if self.num_heads % self.num_kv_heads != 0:
            raise ValueError("num_attention_heads must be divisible by num_key_value_heads")
        self.prompt_lengths = tuple(len(p) for p in self.prompts)
        width = max(-(-(n + max_new_tokens) // block_size) for n in self.prompt_lengths)
        total_blocks = sum(-(-(n + max_new_tokens) // block_size) for n in self.prompt_lengths)
        # kv_cache_dtype=torch.float8_e4m3fn: the FP8 KV format (E4M3 codes,
        # one power-of-two scale per token and head) under fp16/bf16 models
        fp8 = kv_cache_dtype == torch.float8_e4m3fn
        if kv_cache_dtype not in (None, self.dtype) and not fp8:
            raise ValueError("kv_cache_dtype must be None, the model dtype or torch.float8_e4m3fn")
        if fp8 and self.dtype not in (torch.float16, torch.bfloat16):
            raise ValueError("the FP8 KV cache needs an fp16 or bf16 model")
        self.cache = PagedKVCache(total_blocks, block_size, self.num_kv_heads, self.head_dim,
                                  num_layers=self.num_layers, dtype=kv_cache_dtype if fp8 else self.dtype,
                                  act_dtype=self.dtype if fp8 else None, device=self.device)
        batched = prefill_mode == "batched"
        self.runtime = InferenceRuntime(
            self.cache,
            TokenBudgetScheduler(max_num_seqs=len(self.prompts), max_num_batched_tokens=max_num_batched_tokens),
            prefill_fn=None if batched else self._prefill,
            prefill_batch_fn=self._prefill_batch if batched else None,
            decode_fn=self._decode,
        )
        self.requests = [self.runtime.submit(i, len(p), max_new_tokens) for i, p in enumerate(self.prompts)]
        self.metadata = DecodeMetadata(len(self.requests), width, self.device)
        self._prompt_logits: dict[int, torch.Tensor] = {}
        self._next_logits: dict[int, torch.Tensor] = {}
        self._decode_logits: list[torch.Tensor] = []
        self._padding = 0
        self._generated = {r.request_id: [] for r in self.requests}
        self._token_logprobs = {r.request_id: [] for r in self.requests}
        self._sampling_logprobs = {r.request_id: [] for r in self.requests}
        self._finish = {r.request_id: "length" for r in self.requests}
        self._generators = {r.request_id: torch.Generator(device=self.device).manual_seed(seed + r.request_id)
                            for r in self.requests}
        self.use_graph = use_graph
        self._graphs: dict[tuple[int, ...], _StepBuffers] = {}
        self._max_ctx = max(self.prompt_lengths) + max_new_tokens
        self._has_run = False

    # ------------------------------------------------------------ helpers
    def _rope(self, x: torch.Tensor, cos: torch.Tensor, sin: torch.Tensor) -> torch.Tensor:
        return x * cos + rotate_half(x) * sin

    def _append(self, layer: int, slots: torch.Tensor, key: torch.Tensor, value: torch.Tensor) -> None:
        if self.append_backend == "torch":
            self.cache.write_slots(layer, slots, key, value, validate_slots=False)
        else:
            ops.append_kv_hip(key.contiguous(), value.contiguous(), self.cache, slots, layer=layer)

    def _mlp_residual(self, layer, hidden: torch.Tensor) -> torch.Tensor:
        x = layer.post_attention_layernorm(hidden)
        return hidden + layer.mlp.down_proj(layer.mlp.act_fn(layer.mlp.gate_proj(x)) * layer.mlp.up_proj(x))

    # ------------------------------------------------------- decode forward
    def _forward_decode(self, token_ids: torch.Tensor, requests, positions) -> torch.Tensor:
        """Logits [B, vocab] after one token per request at `positions`."""
        pos = torch.tensor(list(positions), dtype=torch.long, device=self.device)
        tables, lens = self.metadata.for_batch(requests, [p + 1 for p in positions])
        slots = self.metadata.slots(requests, positions, self.cache.layout.block_size)
        return self._decode_layers(token_ids.to(device=self.device, dtype=torch.long), pos, tables, lens, slots,
                                   validate=True)

    def _decode_layers(self, token_ids, pos, tables, lens, slots, *, validate: bool) -> torch.Tensor:
        """The decode forward on device metadata: token_ids / pos [n] long,
        tables [n, W] int32, lens / slots [n] int32 (no host synchronisation
        unless `validate`, so it can be captured in a graph)."""
        m = self.model.model
        n = token_ids.shape[0]
        hidden = m.embed_tokens(token_ids)
        cos, sin = m.rotary_emb(hidden.unsqueeze(1), pos.view(n, 1))  # [n, 1, D]: broadcasts over heads
        fused = self.append_backend != "torch"
        if fused:
            cos2, sin2 = cos.reshape(n, self.head_dim).contiguous(), sin.reshape(n, self.head_dim).contiguous()
        for li, layer in enumerate(m.layers):
            x = layer.input_layernorm(hidden)
            att = layer.self_attn
            q = att.q_proj(x).view(n, self.num_heads, self.head_dim)
            k = att.k_proj(x).view(n, self.num_kv_heads, self.head_dim)
            v = att.v_proj(x).view(n, self.num_kv_heads, self.head_dim)
            if fused:  # RoPE of q and k + append of rope(k), v: one launch (q rotated in place)
                ops.rope_append_kv_hip(q, k, v, cos2, sin2, self.cache, slots, layer=li)
            else:
                q, k = self._rope(q, cos, sin), self._rope(k, cos, sin)
                self._append(li, slots, k, v)
            o = self._attend(q.contiguous(), self.cache, tables, lens, layer=li, validate_inputs=validate and li == 0,
                             max_context_len=self._max_ctx)
            hidden = hidden + att.o_proj(o.reshape(n, self.num_heads * self.head_dim))
            hidden = self._mlp_residual(layer, hidden)
        return self.model.lm_head(m.norm(hidden))

    # ------------------------------------------------------ prefill forward
    def _prefix_attention(self, q: torch.Tensor, layer: int, tables: torch.Tensor, starts, ends) -> torch.Tensor:
        """Causal attention of prompt chunk rows q [B, T, H, D] (row t of
        request b sits at position starts[b] + t) over the request's paged
        prefix [0, ends[b]); fp32 softmax. Rows past a chunk are padding."""
        b, t = q.shape[0], q.shape[1]
        bs = self.cache.layout.block_size
        span = max(ends)
        kpos = torch.arange(span, device=self.device)
        blocks = tables[:, kpos // bs].to(torch.long)
        k = self.cache.k[layer][blocks, kpos % bs]  # [B, L, Hkv, D]
        v = self.cache.v[layer][blocks, kpos % bs]
        if self.cache.fp8:  # dequantise: codes times their row scales
            k = k.float() * self.cache.k_scale[layer][blocks, :, kpos % bs].unsqueeze(-1)
            v = v.float() * self.cache.v_scale[layer][blocks, :, kpos % bs].unsqueeze(-1)
        end_t = torch.tensor(list(ends), device=self.device).view(b, 1)
        start_t = torch.tensor(list(starts), device=self.device).view(b, 1)
        kvalid = kpos.view(1, -1) < end_t  # [B, L]
        k = k.float().masked_fill(~kvalid[..., None, None], 0.0)
        v = v.float().masked_fill(~kvalid[..., None, None], 0.0)
        rep = self.num_heads // self.num_kv_heads
        k = k.repeat_interleave(rep, dim=2).permute(0, 2, 3, 1).contiguous()  # [B, H, D, L]
        v = v.repeat_interleave(rep, dim=2).permute(0, 2, 1, 3).contiguous()  # [B, H, L, D]
        qf = q.float().permute(0, 2, 1, 3).contiguous()  # [B, H, T, D]
        scores = torch.matmul(qf, k) * (self.head_dim ** -0.5)  # [B, H, T, L]
        qpos = start_t + torch.arange(t, device=self.device).view(1, -1)  # [B, T]
        allow = (kpos.view(1, 1, -1) <= qpos.unsqueeze(-1)) & kvalid.unsqueeze(1)  # [B, T, L]
        allow = allow | (kpos.view(1, 1, -1) == 0)  # padding rows keep one key (never NaN)
        scores = scores.masked_fill(~allow.unsqueeze(1), float("-inf"))
        out = torch.matmul(torch.softmax(scores, dim=-1), v)  # [B, H, T, D]
        return out.permute(0, 2, 1, 3).to(q.dtype)

    def _forward_prefill(self, token_ids: torch.Tensor, requests, starts, ends) -> torch.Tensor:
        """Logits [B, T, vocab] of prompt chunks token_ids [B, T] (padded).

        With the HIP backends (the default) each layer runs two kernels
        around its projections: the fused RoPE + append over the batch's
        tokens (padding rows rotate but are not appended: their slot is -1)
        and the paged prefill attention (ikl_paged_prefill_attention), which
        reads the chunk's prefix straight from the cache — the role of
        paged_prefill_attention_sdpa at hf_benchmark.py:491-498."""
        m = self.model.model
        b, t = token_ids.shape
        spans = [e - s for s, e in zip(starts, ends)]
        hidden = m.embed_tokens(token_ids)
        pos = torch.tensor(list(starts), device=self.device).view(-1, 1) + torch.arange(t, device=self.device)
        cos, sin = m.rotary_emb(hidden, pos)
        tables, _ = self.metadata.for_batch(requests, list(ends))
        fused = self.append_backend != "torch"
        if fused:
            slot_rows = torch.full((b, t), -1, dtype=torch.int32)
            for i, (r, s_, n) in enumerate(zip(requests, starts, spans)):
                slot_rows[i, :n] = torch.as_tensor(self.cache.slot_mapping(r.block_table, s_, n), dtype=torch.int32)
            slots = slot_rows.reshape(-1).to(self.device)
            cos2, sin2 = cos.reshape(b * t, self.head_dim).contiguous(), sin.reshape(b * t, self.head_dim).contiguous()
        else:
            slots = torch.cat([self.cache.slot_mapping(r.block_table, s_, n)
                               for r, s_, n in zip(requests, starts, spans)]).to(torch.int32)
            cos, sin = cos.unsqueeze(2), sin.unsqueeze(2)
        prefill = None
        if self.prefill_attention == "hip":
            prefill = ops.PreparedPagedPrefill(self.cache, tables, list(starts), list(ends),
                                               num_heads=self.num_heads, query_width=t)
        for li, layer in enumerate(m.layers):
            x = layer.input_layernorm(hidden)
            att = layer.self_attn
            q = att.q_proj(x).view(b, t, self.num_heads, self.head_dim)
            k = att.k_proj(x).view(b, t, self.num_kv_heads, self.head_dim)
            v = att.v_proj(x).view(b, t, self.num_kv_heads, self.head_dim)
            if fused:  # q rotated in place; padding rows of k / v are skipped (slot -1)
                ops.rope_append_kv_hip(q.view(b * t, self.num_heads, self.head_dim),
                                       k.reshape(b * t, self.num_kv_heads, self.head_dim),
                                       v.reshape(b * t, self.num_kv_heads, self.head_dim),
                                       cos2, sin2, self.cache, slots, layer=li)
            else:
                q, k = self._rope(q, cos, sin), self._rope(k, cos, sin)
                self._append(li, slots, torch.cat([k[i, :n] for i, n in enumerate(spans)]),
                             torch.cat([v[i, :n] for i, n in enumerate(spans)]))
            if prefill is not None:
                o = torch.empty_like(q)  # [B, T, H, D]; the kernel writes its [B, H, T, D] view
                prefill(q.transpose(1, 2), li, out=o.transpose(1, 2))
            else:
                o = self._prefix_attention(q, li, tables, starts, ends)
            hidden = hidden + att.o_proj(o.reshape(b, t, self.num_heads * self.head_dim))
            hidden = self._mlp_residual(layer, hidden)
        return self.model.lm_head(m.norm(hidden))

    # -------------------------------------------------------------- hooks
    def _prefill(self, request: InferenceRequest, start: int, end: int) -> None:
        self._prefill_batch((request,), (start,), (end,))

    def _prefill_batch(self, requests, starts, ends) -> None:
        spans = [e - s for s, e in zip(starts, ends)]
        if not requests or any(n <= 0 for n in spans):
            raise ValueError("prefill batch must contain non-empty ranges")
        width = max(spans)
        ids = torch.zeros((len(requests), width), dtype=torch.long)
        for row, (r, s, e) in enumerate(zip(requests, starts, ends)):
            ids[row, : e - s] = torch.tensor(self.prompts[r.request_id][s:e])
        self._padding += len(requests) * width - sum(spans)
        logits = self._forward_prefill(ids.to(self.device), requests, starts, ends)
        for row, (r, e, n) in enumerate(zip(requests, ends, spans)):
            if e == len(self.prompts[r.request_id]):
                self._prompt_logits[r.request_id] = logits[row, n - 1].detach()
                self._next_logits[r.request_id] = logits[row, n - 1].detach()

    def _sample(self, logits: torch.Tensor, gen: torch.Generator):
        """(token, policy log-prob, sampling log-prob) as hf_benchmark.py:578-606."""
        x = logits.float()
        if self.temperature > 0:
            x = x / self.temperature
        policy = torch.log_softmax(x, dim=-1)
        if self.top_p < 1.0:
            order = torch.argsort(x, descending=True)
            probs = torch.softmax(x[order], dim=-1)
            drop = probs.cumsum(-1) - probs > self.top_p
            x = torch.full_like(x, float("-inf")).scatter(-1, order, x[order].masked_fill(drop, float("-inf")))
        logp = torch.log_softmax(x, dim=-1)
        if self.temperature == 0:
            tok = x.argmax(dim=-1)
        else:
            tok = torch.multinomial(logp.exp(), 1, generator=gen).squeeze(-1)
        return tok, policy[tok], logp[tok]

    # ------------------------------------------------- graph-captured steps
    def _decode_graphed(self, requests: tuple[InferenceRequest, ...]) -> None:
        """Greedy decode step as one HIP graph replay per batch composition.

        The graph holds the whole step on static device buffers: argmax of
        the previous logits, lens = pos + 1 and slots from the table buffer
        on the device, the layers (fused RoPE + append, paged attention),
        lm_head, and pos += 1. The host only publishes new table entries and
        reads the tokens back. A batch's first step runs eagerly (it is that
        step's execution) and is then captured."""
        key = tuple(r.request_id for r in requests)
        self.metadata.sync_tables(requests)
        st = self._graphs.get(key)
        if st is None:
            n = len(requests)
            st = _StepBuffers(
                ids=torch.tensor(key, dtype=torch.long, device=self.device),
                logits=torch.stack([self._next_logits[r.request_id] for r in requests]).contiguous(),
                pos=torch.tensor([r.prompt_tokens + r.generated_tokens for r in requests], dtype=torch.long,
                                 device=self.device),
                tok=torch.zeros(n, dtype=torch.long, device=self.device),
                lens=torch.zeros(n, dtype=torch.int32, device=self.device),
                slots=torch.zeros(n, dtype=torch.int32, device=self.device),
            )
            st.used = torch.empty_like(st.logits)
            side = torch.cuda.Stream(self.device)
            side.wait_stream(torch.cuda.current_stream(self.device))
            with torch.cuda.stream(side):
                self._graph_body(st)  # this step's execution
            torch.cuda.current_stream(self.device).wait_stream(side)
            st.graph = torch.cuda.CUDAGraph()
            with torch.cuda.graph(st.graph):
                self._graph_body(st)
            self._graphs[key] = st
        else:
            st.graph.replay()
        self._decode_logits.append(st.used.float().cpu())
        toks = st.tok.tolist()
        for i, r in enumerate(requests):
            self._generated[r.request_id].append(int(toks[i]))
            self._next_logits[r.request_id] = st.logits[i]

    def _graph_body(self, st: "_StepBuffers") -> None:
        bs = self.cache.layout.block_size
        st.used.copy_(st.logits)
        st.tok.copy_(st.used.argmax(dim=-1))
        st.lens.copy_(st.pos + 1)
        tables = self.metadata.tables.index_select(0, st.ids)
        # The runtime reserves every decoded position inside the table's
        # width; the clamp keeps a stray replay (positions past the run) from
        # indexing outside the table buffer.
        col = (st.pos // bs).clamp(max=self.metadata.width - 1)
        blocks = tables.gather(1, col.view(-1, 1)).view(-1).to(torch.long)
        st.slots.copy_(blocks * bs + st.pos % bs)
        st.logits.copy_(self._decode_layers(st.tok, st.pos, tables, st.lens, st.slots, validate=False))
        st.pos.add_(1)

    def _decode(self, requests: tuple[InferenceRequest, ...]) -> None:
        if self.use_graph and self.temperature == 0 and not self.eos_token_ids:
            self._decode_graphed(requests)
            return
        used = torch.stack([self._next_logits[r.request_id] for r in requests])
        sampled = None
        if self.temperature == 0 and not self.eos_token_ids:
            next_tokens = used.argmax(dim=-1)
        else:
            sampled = [self._sample(used[i], self._generators[r.request_id]) for i, r in enumerate(requests)]
            next_tokens = torch.stack([s[0] for s in sampled])
        positions = [r.prompt_tokens + r.generated_tokens for r in requests]
        logits = self._forward_decode(next_tokens, requests, positions)
        self._decode_logits.append(used.float().cpu())
        toks = next_tokens.tolist()
        for i, r in enumerate(requests):
            self._generated[r.request_id].append(int(toks[i]))
            if sampled is not None:
                self._token_logprobs[r.request_id].append(float(sampled[i][1]))
                self._sampling_logprobs[r.request_id].append(float(sampled[i][2]))
            if toks[i] in self.eos_token_ids:
                self._finish[r.request_id] = "eos"
                r.max_new_tokens = r.generated_tokens + 1
            self._next_logits[r.request_id] = logits[i].detach()

    # ---------------------------------------------------------------- run
    def run(self) -> LlamaPagedRunResult:
        if self._has_run:
            raise RuntimeError("a LlamaPagedDecodeRunner instance can only be run once")
        self._has_run = True
        torch.cuda.reset_peak_memory_stats(self.device)
        prefill_steps, decode_steps = [], []
        peak_blocks = self.cache.allocator.num_used_blocks
        # no_grad, not inference_mode: the decode graph captured below would
        # otherwise create torch's graph-safe generator state as inference
        # tensors, and any later capture in the process outside inference
        # mode would fail on it
        with torch.no_grad():
            while self.runtime.scheduler.waiting or self.runtime.scheduler.running:
                t0 = time.perf_counter()
                batch = self.runtime.step()
                torch.cuda.synchronize(self.device)
                ms = (time.perf_counter() - t0) * 1e3
                peak_blocks = max(peak_blocks, self.cache.allocator.num_used_blocks)
                if batch.phase == "prefill":
                    prefill_steps.append(ms)
                elif batch.phase == "decode":
                    decode_steps.append(ms)
                else:
                    raise RuntimeError("scheduler became idle before all requests finished")
        if len(self._prompt_logits) != len(self.requests):
            raise RuntimeError("prefill did not produce one final logits tensor per request")
        generated = tuple(tuple(self._generated[r.request_id]) for r in self.requests)
        if any(not g or len(g) > self.max_new_tokens for g in generated):
            raise RuntimeError("decoder finished with an invalid generated sequence length")
        layout = self.cache.layout
        kv_bytes = (peak_blocks * layout.block_size * layout.num_layers * layout.num_kv_heads
                    * layout.head_dim * 2 * self.cache.k.element_size())
        return LlamaPagedRunResult(
            backend=self.backend,
            append_backend=self.append_backend,
            prompt_lengths=self.prompt_lengths,
            max_new_tokens=self.max_new_tokens,
            generated_tokens=generated,
            prompt_logits=torch.stack([self._prompt_logits[r.request_id] for r in self.requests]).float().cpu(),
            decode_logits=tuple(self._decode_logits),
            prefill_wall_ms=sum(prefill_steps),
            decode_step_wall_ms=tuple(decode_steps),
            ttft_wall_ms=sum(prefill_steps) + decode_steps[0],
            tpot_wall_ms=sum(decode_steps) / len(decode_steps),
            peak_memory_allocated_bytes=int(torch.cuda.max_memory_allocated(self.device)),
            peak_kv_memory_bytes=kv_bytes,
            used_blocks_peak=peak_blocks,
            cache_released=self.cache.allocator.num_used_blocks == 0,
            prefill_step_wall_ms=tuple(prefill_steps),
            prefill_mode=self.prefill_mode,
            prefill_batch_count=len(prefill_steps),
            prefill_tokens=sum(self.prompt_lengths),
            prefill_padding_tokens=self._padding,
            token_logprobs=tuple(tuple(self._token_logprobs[r.request_id]) for r in self.requests),
            sampling_logprobs=tuple(tuple(self._sampling_logprobs[r.request_id]) for r in self.requests),
            finish_reasons=tuple(self._finish[r.request_id] for r in self.requests),
        )
