"""Paged-KV decode benchmark on one MI355X.

A step is one decode step of the paged-KV path over one batch: split-context
paged decode attention (partition kernel + log-sum-exp reduce) over every
request's context, followed by a one-token KV append per request — the
order of the reference's decode step (decode.py:480-487).

Default workload (the GQA decode shape): batch 32, 32 query heads / 8 KV
heads, head_dim 128, bf16, block size 16, ragged context lengths uniform in
[4096, 8192] (seeded), block tables drawn by random permutation from a pool
of 20,000 physical blocks, K/V/q ~ N(0,1). The split is the library's
automatic choice (on the MFMA family: the balanced split, one equal run of
tiles per resident workgroup, here one wave each, merged by the reduce
kernel); ``--partition-size
512`` selects fixed 512-token partitions instead. Inputs are resident in HBM
before the timed region.

Prints ONE JSON line. ``value`` is the algorithmic HBM bytes of a step
divided by its wall time (GB/s); ``roofline`` times the attention partition
kernel with HIP events recorded around it on its stream; ``cpu_baseline``
times the CPU oracle (a numpy restatement of paged_reference) on a bounded
sample of the same requests.

Workloads whose step K/V is below 384 MiB (1.5x the 256 MB MALL) could be
served in part from the MALL when steps run back to back, so by default
(``--mall-flush auto``) a 512 MiB buffer is read before every timed sample
of those (a read, so that no dirty lines are left to write back during the
sample): outside the HIP-event brackets of the kernels, and its own
event-timed duration is taken out of the eager steps' wall time. Their
graph-timed step is a graph of the K steps, each behind the flush, less a
graph of the K flushes alone, so that neither the flush nor a replay's
start-up counts as step time. Above that the
steps run back to back with no flush: the GQA decode shape over the FP8
cache (414 MB of K/V) measured its attention kernel at 75.7-77.1 us back to
back and 72.9-73.0 us with a flush before every step, so the MALL serves it
nothing.

``--workload prefill_*`` measures the paged prefill attention kernel
instead (one causal launch over a batch of prompt chunks): ``value`` and
``roofline`` in TFLOP/s of algorithmic flops against the dense bf16 MFMA
peak, with the reference's gather + masked SDPA path timed on the same GPU
beside it.
"""

from __future__ import annotations

import argparse
import ctypes
import json
import math
import os
import sys
import time
from pathlib import Path

import torch

ROOT = Path(__file__).resolve().parent
PEAK_HBM_GBPS = 8000.0
PEAK_MFMA_TFLOPS = 2500.0  # MI355X dense bf16 / fp16 matrix peak
METRIC = "paged decode attn µs/step + HBM GB/s (% peak), GQA 32/8 hd128 bf16"

WORKLOADS = {
    # name: (batch, heads, kv_heads, head_dim, dtype, ctx_lo, ctx_hi, pool, kv_scale, partition[, cache])
    "gqa32x8_hd128_bf16_b32_ctx4k-8k": (32, 32, 8, 128, torch.bfloat16, 4096, 8192, 20000, 1.0, None),
    "mha32_hd128_fp16_b16_ctx512": (16, 32, 32, 128, torch.float16, 512, 512, None, 1.0, None),
    "mqa32x1_hd128_bf16_b64_ctx1k-4k": (64, 32, 1, 128, torch.bfloat16, 1024, 4096, None, 0.5, None),
    # the GQA decode shape over the FP8 (E4M3, per-row scale) cache format
    "gqa32x8_hd128_fp8kv_b32_ctx4k-8k": (32, 32, 8, 128, torch.bfloat16, 4096, 8192, 20000, 1.0, None, "fp8"),
    # one GPU's share of that GQA 32/8 decode shape when its KV heads are split over 8 and 2 GPUs
    # (same lengths and tables; each GPU attends its KV heads and their query heads)
    "gqa4x1_hd128_bf16_b32_ctx4k-8k": (32, 4, 1, 128, torch.bfloat16, 4096, 8192, 20000, 1.0, None),
    "gqa16x4_hd128_bf16_b32_ctx4k-8k": (32, 16, 4, 128, torch.bfloat16, 4096, 8192, 20000, 1.0, None),
    # the shapes the reference publishes its Triton kernel's A100 timings on (head_dim 64, block 16,
    # uniform contexts; docs/benchmark_report.md:45-52)
    "gqa32x8_hd64_fp16_b4_ctx512": (4, 32, 8, 64, torch.float16, 512, 512, None, 1.0, None),
    "gqa32x8_hd64_fp16_b16_ctx2k": (16, 32, 8, 64, torch.float16, 2048, 2048, None, 1.0, None),
    "gqa32x8_hd64_bf16_b16_ctx2k": (16, 32, 8, 64, torch.bfloat16, 2048, 2048, None, 1.0, None),
    "mha32_hd64_fp16_b16_ctx2k": (16, 32, 32, 64, torch.float16, 2048, 2048, None, 1.0, None),
    "mqa32x1_hd64_bf16_b16_ctx2k": (16, 32, 1, 64, torch.bfloat16, 2048, 2048, None, 1.0, None),
}
DEFAULT_WORKLOAD = "gqa32x8_hd128_bf16_b32_ctx4k-8k"


# Steps whose K/V is below this many bytes get a MALL flush before every
# timed sample (1.5x the 256 MB MALL; see the module docstring).
MALL_FLUSH_BELOW = 384 << 20


class HipEvents:
    """Raw hipEvent_t handles from the HIP runtime torch already loaded."""

    def __init__(self):
        self.lib = ctypes.CDLL("libamdhip64.so.7")
        self.lib.hipEventCreate.argtypes = [ctypes.POINTER(ctypes.c_void_p)]
        self.lib.hipEventElapsedTime.argtypes = [ctypes.POINTER(ctypes.c_float), ctypes.c_void_p,
                                                 ctypes.c_void_p]
        self.lib.hipEventDestroy.argtypes = [ctypes.c_void_p]

    def create(self) -> int:
        handle = ctypes.c_void_p()
        rc = self.lib.hipEventCreate(ctypes.byref(handle))
        if rc != 0:
            raise RuntimeError(f"hipEventCreate failed: {rc}")
        return handle.value

    def elapsed_ms(self, start: int, end: int) -> float:
        out = ctypes.c_float()
        rc = self.lib.hipEventElapsedTime(ctypes.byref(out), ctypes.c_void_p(start), ctypes.c_void_p(end))
        if rc != 0:
            raise RuntimeError(f"hipEventElapsedTime failed: {rc}")
        return float(out.value)

    def destroy(self, handle: int) -> None:
        self.lib.hipEventDestroy(ctypes.c_void_p(handle))


class MallFlush:
    """Evicts the 256 MB MALL (and the L2s) before a timed sample by READING
    a 512 MiB buffer (one reduction over it), so that the flush leaves no
    dirty lines whose write-back could compete with the sample's own reads
    (on a read-only probe of the MQA workload's 90 MB of K/V tiles, a 512 MiB
    hipMemsetAsync before each launch doubled its time, 19 -> 37 µs, against
    the read flush); a decode step's attention follows reads of other
    layers' K/V and weights, not bulk writes."""

    def __init__(self, device: torch.device):
        self.buf = torch.zeros((512 << 20) // 4, dtype=torch.float32, device=device)
        self.sink = torch.empty((), dtype=torch.float32, device=device)

    def __call__(self) -> None:
        torch.sum(self.buf, dim=0, out=self.sink)


class ProbeFlush:
    """The same eviction as MallFlush, made with the library's read probe
    (ikl_hbm_read_probe) over its own 512 MiB buffer: one kernel launch that
    records nothing but itself into a HIP graph (torch's sum over many
    blocks also records a memset node). Measured on the MQA 32/1 hd128 bf16
    B64 x U[1024, 4096] step: 29.5 us median after it against 29.6 us after
    MallFlush, so its streaming loads evict the MALL alike."""

    def __init__(self, device: torch.device):
        from inferkernellab_amd import _lib

        self.lib = _lib.load()
        self.check = _lib.check
        self.buf = torch.ones((512 << 20) // 4, dtype=torch.int32, device=device)
        self.sink = torch.zeros(1 << 14, dtype=torch.int32, device=device)
        self.device = device

    def __call__(self) -> None:
        stream = torch.cuda.current_stream(self.device).cuda_stream
        self.check(self.lib.ikl_hbm_read_probe(ctypes.c_void_p(self.buf.data_ptr()), self.buf.numel() * 4,
                                               ctypes.c_void_p(self.sink.data_ptr()), self.sink.numel() * 4,
                                               ctypes.c_void_p(stream)), "MALL flush (read probe)")


def build_workload(name: str, device: torch.device, seed: int = 0, head_major: bool | None = None):
    from inferkernellab_amd import PagedKVCache

    batch, heads, kv_heads, head_dim, dtype, lo, hi, pool, kv_scale, _ = WORKLOADS[name][:10]
    fp8 = len(WORKLOADS[name]) > 10 and WORKLOADS[name][10] == "fp8"
    block_size = 16
    gen = torch.Generator().manual_seed(seed)
    lengths = torch.randint(lo, hi + 1, (batch,), generator=gen).tolist()
    need = [-(-(n + 1) // block_size) for n in lengths]  # room for the appended token
    pool = pool or sum(need) + 8
    perm = torch.randperm(pool, generator=gen).tolist()
    tables, used = [], 0
    for n in need:
        tables.append(perm[used : used + n])
        used += n
    width = max(need)
    padded = [t + [0] * (width - len(t)) for t in tables]
    dgen = torch.Generator(device=device).manual_seed(seed + 1)
    if fp8:
        from inferkernellab_amd.cache import quantize_rows_e4m3

        cache = PagedKVCache(pool, block_size, kv_heads, head_dim, dtype=torch.float8_e4m3fn, act_dtype=dtype,
                             device=device, head_major=head_major)
        step = 1024  # blocks quantised per chunk
        for codes, scales in ((cache.k, cache.k_scale), (cache.v, cache.v_scale)):
            for b0 in range(0, pool, step):
                n = min(step, pool - b0)
                rows = torch.randn(n, block_size, kv_heads, head_dim, generator=dgen, device=device) * kv_scale
                c, sc = quantize_rows_e4m3(rows.to(dtype))
                codes[0, b0 : b0 + n] = c
                scales[0, b0 : b0 + n] = sc.transpose(1, 2)
    else:
        cache = PagedKVCache(pool, block_size, kv_heads, head_dim, dtype=dtype, device=device,
                             head_major=head_major)
        for t in (cache.k, cache.v):
            t.normal_(0.0, kv_scale, generator=dgen)
    query = torch.randn(batch, heads, head_dim, generator=dgen, device=device, dtype=torch.float32).to(dtype)
    new_k = (torch.randn(batch, kv_heads, head_dim, generator=dgen, device=device) * kv_scale).to(dtype)
    new_v = (torch.randn(batch, kv_heads, head_dim, generator=dgen, device=device) * kv_scale).to(dtype)
    slots = [tables[b][n // block_size] * block_size + n % block_size for b, n in enumerate(lengths)]
    return {
        "cache": cache,
        "query": query,
        "tables": torch.tensor(padded, dtype=torch.int32, device=device),
        "tables_list": tables,
        "lengths": lengths,
        "lens": torch.tensor(lengths, dtype=torch.int32, device=device),
        "new_k": new_k,
        "new_v": new_v,
        "slots": torch.tensor(slots, dtype=torch.int32, device=device),
        "dtype": dtype,
        "fp8": fp8,
        "heads": heads,
        "kv_heads": kv_heads,
        "head_dim": head_dim,
        "block_size": block_size,
        "pool": pool,
    }


def attention_bytes(lengths, heads: int, kv_heads: int, head_dim: int, elem_bytes: int,
                    block_size: int, idx_bytes: int = 4, fp8: bool = False) -> int:
    """Algorithmic HBM bytes of one paged decode attention launch: the K+V
    rows of every context token (the reference's estimated_kv_read_bytes,
    benchmark.py:271-278, summed over ragged lengths), the q and out rows,
    the block-table entries and the context lengths read. With the FP8
    cache a row is head_dim one-byte codes plus its 4-byte scale."""
    row = head_dim + 4 if fp8 else head_dim * elem_bytes
    kv = sum(lengths) * kv_heads * row * 2
    q_out = 2 * len(lengths) * heads * head_dim * elem_bytes
    table = sum(-(-n // block_size) for n in lengths) * idx_bytes
    return kv + q_out + table + len(lengths) * idx_bytes


def step_bytes(w) -> tuple[int, int]:
    """(attention algorithmic bytes, append algorithmic bytes) of one step."""
    eb = torch.tensor([], dtype=w["dtype"]).element_size()
    attn = attention_bytes(w["lengths"], w["heads"], w["kv_heads"], w["head_dim"], eb, w["block_size"],
                           fp8=w["fp8"])
    batch = len(w["lengths"])
    written = w["head_dim"] + 4 if w["fp8"] else w["head_dim"] * eb  # per row: codes + scale, or the row
    append = 2 * batch * w["kv_heads"] * (w["head_dim"] * eb + written) + batch * 4  # K,V read + write, slots
    return attn, append


# Tolerances of this path against the fp32 oracle (max-abs), plus half an
# ulp of the output dtype at |expected| for the output's own rounding.
TOLERANCE = {torch.float16: 2e-3, torch.bfloat16: 1e-2, torch.float32: 1e-4}
_SIGNIFICAND_BITS = {torch.float16: 11, torch.bfloat16: 8, torch.float32: 24}


def host_threads() -> int:
    try:
        from threadpoolctl import threadpool_info

        return max([info.get("num_threads", 1) for info in threadpool_info()] or [1])
    except Exception:  # pragma: no cover
        return os.cpu_count() or 1


def cpu_model() -> str:
    try:
        for line in Path("/proc/cpuinfo").read_text().splitlines():
            if line.startswith("model name"):
                return line.split(":", 1)[1].strip()
    except OSError:
        pass
    return "unknown"


def oracle_view(w):
    """(OracleCache over a host copy of the workload's cache, fp32 query) for
    the CPU oracle. The FP8 cache is attended dequantised (codes x scales,
    exact in fp32)."""
    import numpy as np
    from oracle import paged_oracle as po

    cache = w["cache"]
    dtype = {torch.bfloat16: "bfloat16", torch.float16: "float16", torch.float32: "float32"}[w["dtype"]]

    def host(t):
        t = t.detach().cpu()
        return t.view(torch.int16).numpy().view(np.uint16) if t.dtype == torch.bfloat16 else t.numpy()

    if w["fp8"]:
        k = (cache.k.float() * cache.k_scale.transpose(2, 3).unsqueeze(-1)).cpu().numpy()
        v = (cache.v.float() * cache.v_scale.transpose(2, 3).unsqueeze(-1)).cpu().numpy()
        oc = po.OracleCache.wrap(k, v, "float32")
    else:
        oc = po.OracleCache.wrap(host(cache.k), host(cache.v), dtype)
    return oc, po.to_f32(host(w["query"]), dtype)


def oracle_step(view, w):
    """The oracle's paged_reference over every request of the step: fp32 [B, H, D]."""
    from oracle import paged_oracle as po

    oc, q = view
    return po.paged_decode_attention(q, oc, w["tables_list"], w["lengths"])


def parity(out: torch.Tensor, expected, dtype: torch.dtype) -> dict:
    """Max-abs error of the kernel output against the oracle and the largest
    excess over the tolerance (<= 0 passes): |out - expected| <= tol + half
    an ulp of the output dtype at |expected|."""
    import numpy as np

    got = out.detach().float().cpu().numpy()
    err = np.abs(got - expected)
    _, e = np.frexp(np.abs(expected).astype(np.float64))
    half_ulp = np.ldexp(1.0, e - _SIGNIFICAND_BITS[dtype] - 1)
    excess = float(np.max(err - (TOLERANCE[dtype] + half_ulp))) if err.size else 0.0
    return {
        "max_abs_err": float(np.max(err)) if err.size else 0.0,
        "tolerance": TOLERANCE[dtype],
        "max_excess": excess,
        "nan": bool(np.isnan(got).any()),
        "passed": bool(excess <= 0 and not np.isnan(got).any()),
    }


def cpu_baseline(w, view, budget_s: float, first_step_s: float) -> dict:
    """Times the CPU oracle (numpy paged_reference) over whole decode steps of
    the same workload — every request of the batch per step — until about
    budget_s of CPU work; the parity check's step is the first sample."""
    samples = [first_step_s]
    while sum(samples) < budget_s:
        t0 = time.perf_counter()
        oracle_step(view, w)
        samples.append(time.perf_counter() - t0)
    step_s = sum(samples) / len(samples)
    kv_bytes = sum(w["lengths"]) * w["kv_heads"] * w["head_dim"] * 2 * w["cache"].k.element_size()
    return {
        "value": round(step_s * 1e6, 1),
        "unit": "us/step",
        "gbps": round(kv_bytes / step_s / 1e9, 3),
        "cores": host_threads(),
        "cpu": cpu_model(),
        "logical_cpus": os.cpu_count(),
        "kind": "port",
        "sample": f"oracle paged_reference (numpy fp32 per-request loop): {len(samples)} whole steps "
                  f"of all {len(w['lengths'])} requests ({sum(w['lengths'])} context tokens each, "
                  f"{sum(samples):.1f} s), mean per step",
    }


def mfma_figures(w, attn, kernel_ms: float, workload: str) -> dict | None:
    """Matrix-core use of the decode kernel (MFMA family only): the flops
    the attention needs (QK^T and PV, 4 * head_dim per context token and
    query head), the flops the MFMA instructions issue (16-token tiles x
    16-head groups, PV twice for bf16 P with its residual), both as rates
    over the kernel time against the dense bf16/fp16 peak, and the MFMA
    busy share measured by rocprofv3 counters when a profile of the
    workload holds it."""
    if attn.path != "mfma_grouped":
        return None
    lengths, d = w["lengths"], w["head_dim"]
    heads_per_kv = w["heads"] // w["kv_heads"]
    group = attn.launch["group_size"]
    units = w["kv_heads"] * -(-heads_per_kv // group)
    ng = 1 if group <= 16 else 2
    tiles = units * sum(-(-n // 16) for n in lengths)
    pv_passes = 2 if (w["dtype"] == torch.bfloat16 and not w["fp8"]) else 1
    issued = tiles * (2 * 16 * 16 * ng * d) * (1 + pv_passes)
    needed = 4 * d * w["heads"] * sum(lengths)
    secs = kernel_ms * 1e-3
    out = {
        "peak_tflops": PEAK_MFMA_TFLOPS,
        "algorithmic_tflops": round(needed / secs / 1e12, 2),
        "issued_tflops": round(issued / secs / 1e12, 2),
        "frac_issued_of_peak": round(issued / secs / 1e12 / PEAK_MFMA_TFLOPS, 4),
        "busy_frac": None,
    }
    prof = ROOT / "profiles" / f"mfma_{workload}.json"
    if prof.exists():
        try:
            out["busy_frac"] = json.loads(prof.read_text()).get("mfma_busy_frac")
        except (OSError, ValueError):
            pass
    return out


# ------------------------------------------------------------------ prefill
PREFILL_METRIC = "paged prefill attention TFLOP/s (causal, algorithmic flops), bf16"
PREFILL_WORKLOADS = {
    # name: (batch, heads, kv_heads, head_dim, dtype, chunk start, chunk end) — every request
    # runs the chunk [start, end) of a prompt whose positions [0, start) are already cached
    "prefill_gqa32x8_hd128_bf16_b8_4k": (8, 32, 8, 128, torch.bfloat16, 0, 4096),
    "prefill_chunk_gqa32x8_hd128_bf16_b8_3k+1k": (8, 32, 8, 128, torch.bfloat16, 3072, 4096),
    "prefill_gqa16x4_hd128_bf16_b8_512": (8, 16, 4, 128, torch.bfloat16, 0, 512),
    # the 4k prompts over the FP8 (E4M3 + per-row scale) cache
    "prefill_gqa32x8_hd128_fp8kv_b8_4k": (8, 32, 8, 128, torch.bfloat16, 0, 4096, "fp8"),
}


def build_prefill_workload(name: str, device: torch.device, seed: int = 0):
    from inferkernellab_amd import PagedKVCache

    batch, heads, kv_heads, head_dim, dtype, start, end = PREFILL_WORKLOADS[name][:7]
    fp8 = PREFILL_WORKLOADS[name][7:] == ("fp8",)
    block_size = 16
    gen = torch.Generator().manual_seed(seed)
    need = -(-end // block_size)
    pool = batch * need + 8
    perm = torch.randperm(pool, generator=gen).tolist()
    tables = [perm[b * need : (b + 1) * need] for b in range(batch)]
    dgen = torch.Generator(device=device).manual_seed(seed + 1)
    if fp8:
        from inferkernellab_amd.cache import quantize_rows_e4m3

        cache = PagedKVCache(pool, block_size, kv_heads, head_dim, dtype=torch.float8_e4m3fn, act_dtype=dtype,
                             device=device)
        for codes, scales in ((cache.k, cache.k_scale), (cache.v, cache.v_scale)):
            for b0 in range(0, pool, 1024):
                n = min(1024, pool - b0)
                rows = torch.randn(n, block_size, kv_heads, head_dim, generator=dgen, device=device)
                c, sc = quantize_rows_e4m3(rows.to(dtype))
                codes[0, b0 : b0 + n] = c
                scales[0, b0 : b0 + n] = sc.transpose(1, 2)
    else:
        cache = PagedKVCache(pool, block_size, kv_heads, head_dim, dtype=dtype, device=device)
        for t in (cache.k, cache.v):
            t.normal_(0.0, 1.0, generator=dgen)
    width = end - start
    query = torch.randn(batch, heads, width, head_dim, generator=dgen, device=device).to(dtype)
    return {
        "cache": cache, "query": query, "tables_list": tables,
        "tables": torch.tensor(tables, dtype=torch.int32, device=device),
        "starts": [start] * batch, "ends": [end] * batch, "dtype": dtype, "heads": heads,
        "kv_heads": kv_heads, "head_dim": head_dim, "block_size": block_size, "pool": pool, "fp8": fp8,
    }


def dequantized_kv(cache):
    """(K, V) of an FP8 cache as code x row scale in fp32 (exact), [layers, blocks, block_size, kv_heads, D]."""
    k = cache.k.float() * cache.k_scale.transpose(2, 3).unsqueeze(-1)
    v = cache.v.float() * cache.v_scale.transpose(2, 3).unsqueeze(-1)
    return k, v


def prefill_pairs(starts, ends) -> int:
    """Attended (query row, key) pairs per head: row t of a chunk [s, e) sees s + t + 1 keys."""
    return sum((e - s) * s + (e - s) * (e - s + 1) // 2 for s, e in zip(starts, ends))


def prefill_flops(w) -> int:
    """Algorithmic flops of one prefill attention launch: QK^T and PV, 2 * head_dim
    each per attended (row, key) pair and query head."""
    return prefill_pairs(w["starts"], w["ends"]) * w["heads"] * 4 * w["head_dim"]


def torch_gather_sdpa(w):
    """The reference's prefill path restated on the same GPU (attention.py:289-321):
    gather the whole prefix through the block table, zero the unread slots,
    build the boolean causal mask and call torch SDPA. An FP8 cache is read
    through a dequantized copy in the query dtype (exact: codes carry 4
    significant bits), made once per workload."""
    import torch.nn.functional as F

    cache, q = w["cache"], w["query"]
    if w.get("fp8"):
        if "dequantized" not in w:
            k, v = dequantized_kv(cache)
            w["dequantized"] = (k.to(q.dtype), v.to(q.dtype))
        k_all, v_all = w["dequantized"]
    else:
        k_all, v_all = cache.k, cache.v
    bs = w["block_size"]
    span = max(w["ends"])
    kpos = torch.arange(span, device=q.device)
    phys = w["tables"].long()[:, kpos // bs]
    key = k_all[0][phys, (kpos % bs).unsqueeze(0)]
    value = v_all[0][phys, (kpos % bs).unsqueeze(0)]
    lengths = torch.tensor(w["ends"], device=q.device).view(-1, 1, 1)
    starts = torch.tensor(w["starts"], device=q.device).view(-1, 1, 1)
    key_ok = kpos.view(1, 1, -1) < lengths
    valid = key_ok.squeeze(1).unsqueeze(-1).unsqueeze(-1)
    key = key.masked_fill(~valid, 0)
    value = value.masked_fill(~valid, 0)
    qpos = torch.arange(q.shape[2], device=q.device)
    valid_query = qpos.view(1, -1, 1) < (lengths - starts).view(-1, 1, 1)
    allow = (valid_query & key_ok & (kpos.view(1, 1, -1) <= starts + qpos.view(1, -1, 1))) | (
        (~valid_query) & (kpos.view(1, 1, -1) == 0))
    return F.scaled_dot_product_attention(q, key.permute(0, 2, 1, 3), value.permute(0, 2, 1, 3),
                                          attn_mask=allow.unsqueeze(1), enable_gqa=True)


def prefill_oracle_view(w):
    """(OracleCache over a host copy of the prefill workload's cache, fp32 query)."""
    import numpy as np
    from oracle import paged_oracle as po

    dtype = {torch.bfloat16: "bfloat16", torch.float16: "float16"}[w["dtype"]]

    def host(t):
        t = t.detach().cpu()
        return t.view(torch.int16).numpy().view(np.uint16) if t.dtype == torch.bfloat16 else t.numpy()

    if w.get("fp8"):  # the FP8 cache is attended dequantised (codes x scales, exact in fp32)
        k, v = dequantized_kv(w["cache"])
        oc = po.OracleCache.wrap(k.cpu().numpy(), v.cpu().numpy(), "float32")
    else:
        oc = po.OracleCache.wrap(host(w["cache"].k), host(w["cache"].v), dtype)
    return oc, po.to_f32(host(w["query"]), dtype)


def prefill_parity(w, out: torch.Tensor, rows: int = 64) -> dict:
    """The kernel's output against the oracle on a bounded sample: for every
    request, the first and the last `rows` query rows of its chunk (the
    shortest and the longest prefixes), all heads."""
    import numpy as np
    from oracle import paged_oracle as po

    oc, q = prefill_oracle_view(w)
    worst = {"max_abs_err": 0.0, "tolerance": TOLERANCE[w["dtype"]], "max_excess": -1.0, "nan": False,
             "passed": True}
    checked = 0
    for b in range(q.shape[0]):
        span = w["ends"][b] - w["starts"][b]
        for r0 in sorted({0, max(0, span - rows)}):
            r1 = min(span, r0 + rows)
            s = w["starts"][b] + r0
            exp = po.paged_prefill_attention(q[b : b + 1, :, r0:r1], oc, [w["tables_list"][b]], [s],
                                             [w["starts"][b] + r1])
            res = parity(out[b : b + 1, :, r0:r1], exp, w["dtype"])
            worst["max_abs_err"] = max(worst["max_abs_err"], res["max_abs_err"])
            worst["max_excess"] = max(worst["max_excess"], res["max_excess"])
            worst["nan"] = worst["nan"] or res["nan"]
            worst["passed"] = worst["passed"] and res["passed"]
            checked += r1 - r0
    worst["checked"] = f"{checked} query rows x {q.shape[1]} heads (first and last {rows} rows of every chunk)"
    return worst


def prefill_cpu_baseline(w, budget_s: float) -> dict:
    """Times the CPU oracle's paged_prefill_attention on 256-row slices of the
    workload's chunks (cycling through requests and slices) for ~budget_s,
    then scales per attended (row, key) pair to the whole launch."""
    from oracle import paged_oracle as po

    oc, q = prefill_oracle_view(w)
    batch, width = q.shape[0], q.shape[2]
    rows = min(256, width)
    slices = [(b, r0) for r0 in range(0, width, rows) for b in range(batch)]
    done, elapsed, pairs = 0, 0.0, 0
    while elapsed < budget_s and done < 4 * len(slices):
        b, r0 = slices[(len(slices) - 1 - done) % len(slices)]  # longest rows first
        s = w["starts"][b] + r0
        e = min(s + rows, w["ends"][b])
        t0 = time.perf_counter()
        po.paged_prefill_attention(q[b : b + 1, :, r0 : r0 + (e - s)], oc, [w["tables_list"][b]], [s], [e])
        elapsed += time.perf_counter() - t0
        pairs += prefill_pairs([s], [e])
        done += 1
    step_s = elapsed / pairs * prefill_pairs(w["starts"], w["ends"])
    return {
        "value": round(step_s * 1e6, 1),
        "unit": "us/step",
        "cores": host_threads(),
        "cpu": cpu_model(),
        "logical_cpus": os.cpu_count(),
        "kind": "port",
        "sample": f"oracle paged_prefill_attention (numpy fp32), {done} slices of <= {rows} rows "
                  f"({pairs} attended row-key pairs per head, {elapsed:.1f} s), scaled per attended "
                  f"pair to the full launch",
    }


def run_prefill(args, device) -> int:
    from inferkernellab_amd import PreparedPagedPrefill

    w = build_prefill_workload(args.workload, device, args.seed)
    q = w["query"]
    prep = PreparedPagedPrefill(w["cache"], w["tables"], w["starts"], w["ends"], num_heads=w["heads"],
                                query_width=q.shape[2])
    out = torch.empty_like(q)
    events = HipEvents()
    k_steps, warmup = args.steps, args.warmup
    ev = [[events.create() for _ in range(2)] for _ in range(k_steps)]
    # correctness gate before timing (the reference's harness raises on a
    # mismatch before it times, benchmark.py:225-268)
    prep(q, 0, out=out)
    torch.cuda.synchronize()
    check = prefill_parity(w, out)
    if not check["passed"]:
        print(json.dumps({"error": "prefill kernel output differs from the oracle", "parity": check}))
        return 3
    for _ in range(warmup):
        prep(q, 0, out=out)
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    for i in range(k_steps):
        prep(q, 0, out=out, events=ev[i])
    torch.cuda.synchronize()
    wall_s = time.perf_counter() - t0
    kernel_ms = [events.elapsed_ms(e[0], e[1]) for e in ev]
    for pair in ev:
        for h in pair:
            events.destroy(h)
    flops = prefill_flops(w)
    ms_per_step = wall_s * 1e3 / k_steps
    kern_ms = sum(kernel_ms) / len(kernel_ms)
    achieved = flops / (kern_ms * 1e-3) / 1e12

    # the reference's gather + masked SDPA on the same GPU, for comparison
    sdpa_ms = None
    scores_bytes = q.shape[0] * q.shape[1] * q.shape[2] * max(w["ends"]) * 4
    if scores_bytes < (48 << 30):
        ref = torch_gather_sdpa(w)
        err = float((ref.float() - out.float()).abs().max())
        del ref
        start, stop = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        torch.cuda.synchronize()
        start.record()
        for _ in range(3):
            torch_gather_sdpa(w)
        stop.record()
        torch.cuda.synchronize()
        sdpa_ms = start.elapsed_time(stop) / 3
    else:
        err = None

    traffic = None
    traffic_file = ROOT / "profiles" / f"traffic_{args.workload}.json"
    if traffic_file.exists():
        try:
            traffic = json.loads(traffic_file.read_text()).get("hbm_bytes_per_launch")
        except (OSError, ValueError):
            traffic = None
    cpu = None if args.no_cpu_baseline else prefill_cpu_baseline(w, args.cpu_budget_s)
    value = flops / (ms_per_step * 1e-3) / 1e12
    record = {
        "metric": PREFILL_METRIC,
        "value": round(value, 1),
        "unit": "TFLOP/s",
        "n_gpus": 1,
        "steps": k_steps,
        "warmup": warmup,
        "ms_per_step": round(ms_per_step, 4),
        "us_per_step": round(ms_per_step * 1e3, 1),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": {torch.bfloat16: "bf16", torch.float16: "fp16"}[w["dtype"]],
        "data": "synthetic (seeded N(0,1) K/V/q, random-permutation block tables)",
        "config": {
            "workload": args.workload,
            "batch": q.shape[0],
            "num_heads": w["heads"],
            "num_kv_heads": w["kv_heads"],
            "head_dim": w["head_dim"],
            "block_size": w["block_size"],
            "chunk": [w["starts"][0], w["ends"][0]],
            "kv_cache": "fp8 e4m3 codes + one fp32 scale per (token, kv head)" if w["fp8"] else "same as dtype",
            "step": "one paged prefill attention launch over the batch's chunks (causal)",
            "parallelism": "single GPU",
        },
        "prefill_kernel_us": round(kern_ms * 1e3, 2),
        "algorithmic_flops_per_launch": flops,
        "torch_gather_sdpa_us": round(sdpa_ms * 1e3, 1) if sdpa_ms is not None else None,
        "max_abs_diff_vs_torch_sdpa": err,
        "parity": check,
        "roofline": {
            "bound": "mfma",
            "achieved": round(achieved, 1),
            "peak": PEAK_MFMA_TFLOPS,
            "unit": "TFLOP/s",
            "frac": round(achieved / PEAK_MFMA_TFLOPS, 4),
            "traffic": traffic,
            "kernel": prep.kernel_name(),
            "algorithmic_flops_per_launch": flops,
        },
        "cpu_baseline": cpu,
    }
    print(json.dumps(record))
    return 0


# ------------------------------------------------------------------ sweep
# The reference's attention sweep (docs/benchmark_report.md:28-34; cases
# built by benchmark.py:73-123): batch {1, 4, 16} x context {128, 512, 2048}
# x KV heads {32, 8, 1} (MHA / GQA / MQA) x {fp16, bf16}, 32 query heads,
# head_dim 64, block 16, warmup 10, 50 event-timed samples.
SWEEP_BATCHES = (1, 4, 16)
SWEEP_CONTEXTS = (128, 512, 2048)
SWEEP_KV_HEADS = (32, 8, 1)
SWEEP_DTYPES = (("fp16", torch.float16), ("bf16", torch.bfloat16))

# Published A100-SXM4-40GB means (µs) of the reference's triton_paged kernel
# and of its paged gather + SDPA path on each sweep shape, one line of
# docs/benchmark_results/a100_cuda13_triton36.jsonl each (lines 1-54).
A100_SWEEP_US = {
    ("fp16", 1, 128, 32): (101.3, 184.7), ("bf16", 1, 128, 32): (101.2, 186.2),
    ("fp16", 1, 128, 8): (102.0, 192.5), ("bf16", 1, 128, 8): (100.6, 191.5),
    ("fp16", 1, 128, 1): (101.8, 194.9), ("bf16", 1, 128, 1): (101.0, 189.1),
    ("fp16", 1, 512, 32): (102.5, 196.4), ("bf16", 1, 512, 32): (101.5, 194.9),
    ("fp16", 1, 512, 8): (102.6, 201.7), ("bf16", 1, 512, 8): (102.4, 204.3),
    ("fp16", 1, 512, 1): (103.9, 203.3), ("bf16", 1, 512, 1): (102.0, 202.4),
    ("fp16", 1, 2048, 32): (157.5, 238.4), ("bf16", 1, 2048, 32): (162.1, 238.7),
    ("fp16", 1, 2048, 8): (146.5, 203.9), ("bf16", 1, 2048, 8): (145.6, 204.3),
    ("fp16", 1, 2048, 1): (145.5, 204.0), ("bf16", 1, 2048, 1): (146.6, 200.7),
    ("fp16", 4, 128, 32): (104.2, 224.0), ("bf16", 4, 128, 32): (101.3, 223.8),
    ("fp16", 4, 128, 8): (101.3, 230.8), ("bf16", 4, 128, 8): (100.3, 230.2),
    ("fp16", 4, 128, 1): (100.2, 230.2), ("bf16", 4, 128, 1): (99.7, 229.3),
    ("fp16", 4, 512, 32): (101.7, 270.0), ("bf16", 4, 512, 32): (102.2, 267.9),
    ("fp16", 4, 512, 8): (101.4, 239.6), ("bf16", 4, 512, 8): (100.8, 237.2),
    ("fp16", 4, 512, 1): (101.8, 240.4), ("bf16", 4, 512, 1): (101.2, 242.6),
    ("fp16", 4, 2048, 32): (213.6, 549.9), ("bf16", 4, 2048, 32): (214.1, 606.0),
    ("fp16", 4, 2048, 8): (164.2, 257.6), ("bf16", 4, 2048, 8): (162.5, 263.4),
    ("fp16", 4, 2048, 1): (158.0, 240.4), ("bf16", 4, 2048, 1): (156.6, 243.0),
    ("fp16", 16, 128, 32): (100.7, 271.5), ("bf16", 16, 128, 32): (100.9, 272.2),
    ("fp16", 16, 128, 8): (100.7, 233.0), ("bf16", 16, 128, 8): (102.2, 233.7),
    ("fp16", 16, 128, 1): (101.1, 232.7), ("bf16", 16, 128, 1): (105.5, 232.9),
    ("fp16", 16, 512, 32): (141.0, 617.3), ("bf16", 16, 512, 32): (141.7, 615.1),
    ("fp16", 16, 512, 8): (117.0, 271.0), ("bf16", 16, 512, 8): (112.3, 270.9),
    ("fp16", 16, 512, 1): (111.8, 240.0), ("bf16", 16, 512, 1): (112.1, 238.4),
    ("fp16", 16, 2048, 32): (296.0, 1645.3), ("bf16", 16, 2048, 32): (295.5, 1648.8),
    ("fp16", 16, 2048, 8): (216.6, 526.5), ("bf16", 16, 2048, 8): (216.6, 525.6),
    ("fp16", 16, 2048, 1): (190.4, 242.3), ("bf16", 16, 2048, 1): (192.4, 239.8),
}


def build_sweep_case(batch: int, ctx: int, kv_heads: int, dtype: torch.dtype, device: torch.device,
                     seed: int = 0, heads: int = 32, head_dim: int = 64, block_size: int = 16):
    """One sweep case with the reference's block-table layout
    (benchmark.py:85-95): logical block j of request r is physical block
    j * (B + 1) + r — requests interleaved, one reserved block between
    rounds — in a pool of exactly the blocks that allocation touches."""
    from inferkernellab_amd import PagedKVCache

    need = -(-ctx // block_size)
    pool = batch * need + need - 1
    tables = [[j * (batch + 1) + r for j in range(need)] for r in range(batch)]
    cache = PagedKVCache(pool, block_size, kv_heads, head_dim, dtype=dtype, device=device)
    gen = torch.Generator(device=device).manual_seed(seed)
    for t in (cache.k, cache.v):
        t.normal_(0.0, 1.0, generator=gen)
    query = torch.randn(batch, heads, head_dim, generator=gen, device=device, dtype=torch.float32).to(dtype)
    return {
        "cache": cache, "query": query, "tables_list": tables, "lengths": [ctx] * batch,
        "tables": torch.tensor(tables, dtype=torch.int64, device=device),
        "lens": torch.tensor([ctx] * batch, dtype=torch.int32, device=device),
        "dtype": dtype, "fp8": False, "heads": heads, "kv_heads": kv_heads, "head_dim": head_dim,
        "block_size": block_size, "pool": pool,
    }


def _percentile(values, q: float) -> float:
    """Linear-interpolated percentile, as the reference reports (benchmark.py:36-44)."""
    v = sorted(values)
    pos = (len(v) - 1) * q
    lo, hi = math.floor(pos), math.ceil(pos)
    return v[lo] if lo == hi else v[lo] * (hi - pos) + v[hi] * (pos - lo)


def run_sweep(args, device) -> int:
    """Every sweep shape: one checked launch against the oracle (all
    requests and heads; a mismatch stops the sweep, as the reference's
    harness raises, benchmark.py:225-268), then warmup and event-timed
    samples of the whole attention operation (split kernel + reduce) on
    prevalidated inputs, as the reference times its kernel with
    validate_inputs=False (benchmark.py:251-262). A 512 MiB MALL flush (a
    read) runs before every sample, outside the event bracket, unless --mall-flush off.
    One JSON line per shape goes to --sweep-out (and stderr); stdout gets one
    summary line."""
    import statistics

    from inferkernellab_amd import ops

    flush_buf = MallFlush(device) if args.mall_flush != "off" else None
    rows = []
    out_file = open(args.sweep_out, "w") if args.sweep_out else None
    for name, dtype in SWEEP_DTYPES:
        for batch in SWEEP_BATCHES:
            for ctx in SWEEP_CONTEXTS:
                for kv in SWEEP_KV_HEADS:
                    w = build_sweep_case(batch, ctx, kv, dtype, device, args.seed)
                    attn = ops.PreparedPagedAttention(w["query"], w["cache"], w["tables"], w["lens"],
                                                      max_context_len=ctx)
                    attn()
                    torch.cuda.synchronize()
                    check = parity(attn.out, oracle_step(oracle_view(w), w), dtype)
                    shape = {"dtype": name, "batch": batch, "context_len": ctx, "num_heads": 32,
                             "num_kv_heads": kv, "head_dim": 64, "block_size": 16, "num_blocks": w["pool"]}
                    if not check["passed"]:
                        print(json.dumps({"error": "sweep case differs from the oracle", "case": shape,
                                          "parity": check}))
                        return 3
                    for _ in range(args.warmup):
                        attn()
                    samples = []
                    start, stop = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
                    for i in range(args.steps):
                        if flush_buf is not None:
                            flush_buf()
                        start.record()
                        attn()
                        stop.record()
                        stop.synchronize()
                        samples.append(start.elapsed_time(stop) * 1e3)
                    mean_us = sum(samples) / len(samples)
                    a100_triton, a100_sdpa = A100_SWEEP_US[(name, batch, ctx, kv)]
                    kv_bytes = 2 * batch * ctx * kv * 64 * 2  # the reference's estimated_kv_read_bytes
                    row = {
                        "case": shape, "path": attn.path,
                        "split": "balanced" if attn.balanced_split else (
                            f"fixed {attn.partition_size}" if attn.partition_size > 0 else "none"),
                        "mean_us": round(mean_us, 2), "p50_us": round(_percentile(samples, 0.5), 2),
                        "p95_us": round(_percentile(samples, 0.95), 2),
                        "kv_gbps": round(kv_bytes / (mean_us * 1e-6) / 1e9, 1),
                        "max_abs_err": check["max_abs_err"], "tolerance": check["tolerance"],
                        "a100_triton_us": a100_triton, "a100_paged_sdpa_us": a100_sdpa,
                        "speedup_vs_a100_triton": round(a100_triton / mean_us, 2),
                    }
                    rows.append(row)
                    line = json.dumps(row)
                    print(line, file=sys.stderr, flush=True)
                    if out_file:
                        out_file.write(line + "\n")
                    del attn, w
    if out_file:
        out_file.close()
    ratios = [r["speedup_vs_a100_triton"] for r in rows]
    print(json.dumps({
        "sweep": "reference attention matrix: batch {1,4,16} x context {128,512,2048} x kv heads "
                 "{32,8,1} x {fp16,bf16}; 32 heads, head_dim 64, block 16",
        "cases": len(rows),
        "all_within_tolerance": True,
        "max_abs_err": {n: max(r["max_abs_err"] for r in rows if r["case"]["dtype"] == n) for n, _ in SWEEP_DTYPES},
        "median_speedup_vs_a100_triton": round(statistics.median(ratios), 2),
        "min_speedup_vs_a100_triton": min(ratios),
        "max_speedup_vs_a100_triton": max(ratios),
        "mall_flush": flush_buf is not None,
        "samples": args.steps, "warmup": args.warmup,
    }))
    return 0


# ------------------------------------------------------------------ llama
LLAMA_E2E_METRIC = "tiny Llama end-to-end paged decode: tokens/s, TPOT ms, bf16"


def measure_llama_e2e(device: torch.device, *, check_requests: int, seed: int = 0) -> dict:
    """The end-to-end configuration: a random-init Llama (8 layers, hidden
    2048, 16 / 4 heads of 128, intermediate 5632, vocab 32000, RMSNorm, RoPE
    theta 1e4, seed-0 weights) in bf16; 16 prompts of 512 random ids
    (seeded), batched prefill under max_num_batched_tokens 4096 (2 batches
    of 8), then 64 greedy decode steps through the paged runtime (HIP fused
    RoPE + append, paged prefill and decode kernels, one HIP graph per
    decode step). A 4-token run warms the kernels and the allocator first;
    the second run is timed. The first `check_requests` requests are
    teacher-forced through the CPU oracle (numpy forward rounding to bf16
    where the bf16 modules round, hf_benchmark.py:764-823's role): greedy
    agreement, flips with the oracle's margin, and the largest logit error."""
    import numpy as np
    from oracle import llama_oracle as lo

    from inferkernellab_amd.llama import LlamaConfig, LlamaPagedDecodeRunner, random_llama

    cfg = LlamaConfig(vocab_size=32000, hidden_size=2048, intermediate_size=5632, num_hidden_layers=8,
                      num_attention_heads=16, num_key_value_heads=4, rope_theta=10000.0)
    model = random_llama(cfg, seed=0, device=device, dtype=torch.bfloat16)
    gen = torch.Generator().manual_seed(seed)
    prompts = torch.randint(0, 32000, (16, 512), generator=gen).tolist()
    kw = dict(block_size=16, max_num_batched_tokens=4096)
    LlamaPagedDecodeRunner(model, prompts, max_new_tokens=4, **kw).run()
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    result = LlamaPagedDecodeRunner(model, prompts, max_new_tokens=64, **kw).run()
    wall_s = time.perf_counter() - t0
    steps = list(result.decode_step_wall_ms)
    new_tokens = sum(len(g) for g in result.generated_tokens)
    decode_s = sum(steps) / 1e3
    w = lo.weights_from_model(model) if check_requests > 0 else None
    checked = flips = 0
    worst, margins = 0.0, []
    for i in range(min(check_requests, len(prompts))):
        gen_i = result.generated_tokens[i]
        ref = lo.teacher_forced_logits(w, cfg, prompts[i], gen_i, round_to="bfloat16")
        ours = torch.stack([step[i] for step in result.decode_logits]).float().numpy()
        worst = max(worst, float(np.abs(ours - ref).max()))
        best = ref.argmax(-1)
        for j in np.nonzero(np.asarray(gen_i) != best)[0]:
            flips += 1
            margins.append(float(ref[j, best[j]] - ref[j, gen_i[j]]))
        checked += len(gen_i)
    del w
    return {
        "prefill_ms": round(result.prefill_wall_ms, 2),
        "prefill_batches": result.prefill_batch_count,
        "prefill_tokens": result.prefill_tokens,
        "prefill_tokens_per_s": round(result.prefill_tokens / (result.prefill_wall_ms * 1e-3), 1),
        "ttft_ms": round(result.ttft_wall_ms, 2),
        "tpot_mean_ms": round(result.tpot_wall_ms, 3),
        "tpot_p50_ms": round(_percentile(steps, 0.5), 3),
        "tpot_p95_ms": round(_percentile(steps, 0.95), 3),
        "decode_tokens_per_s": round(new_tokens / decode_s, 1),
        "end_to_end_tokens_per_s": round(new_tokens / wall_s, 1),
        "wall_s": round(wall_s, 3),
        "generated_tokens": new_tokens,
        "greedy_checked_tokens": checked,
        "greedy_agreement": (checked - flips) / checked if checked else None,
        "greedy_flips": flips,
        "largest_flip_margin": round(max(margins), 4) if margins else 0.0,
        "logits_max_abs_err": round(worst, 4),
        "peak_memory_allocated_bytes": result.peak_memory_allocated_bytes,
    }


def llama_e2e_entry(device: torch.device, *, check_requests: int, seed: int = 0) -> dict:
    entry = {"spec": "tiny random Llama end-to-end, bf16: 8 layers, hidden 2048, 16 / 4 heads of 128, "
                     "intermediate 5632, vocab 32000; B16 x 512-token prompts, batched prefill (4096 "
                     "tokens), 64 greedy decode steps, graph decode"}
    entry.update(measure_llama_e2e(device, check_requests=check_requests, seed=seed))
    torch.cuda.empty_cache()
    return entry


def run_llama_e2e(args, device) -> int:
    t0 = time.perf_counter()
    e = measure_llama_e2e(device, check_requests=args.check_requests, seed=args.seed)
    record = {
        "metric": LLAMA_E2E_METRIC,
        "value": e["decode_tokens_per_s"],
        "unit": "tokens/s",
        "n_gpus": 1,
        "steps": 64,
        "warmup": 1,
        "ms_per_step": e["tpot_mean_ms"],
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "bf16",
        "data": "synthetic (seed-0 random weights, seeded random prompt ids)",
        "config": {"workload": "llama_e2e", "layers": 8, "hidden": 2048, "num_heads": 16, "num_kv_heads": 4,
                   "head_dim": 128, "intermediate": 5632, "vocab": 32000, "batch": 16, "prompt_len": 512,
                   "max_num_batched_tokens": 4096, "new_tokens": 64, "parallelism": "single GPU"},
        **{k: v for k, v in e.items()},
        "greedy_criterion": "teacher-forced against the CPU oracle in bf16 rounding; a flip is a token "
                            "whose oracle logit trails the oracle's argmax by the printed margin",
    }
    record["environment"] = environment(sys.argv)
    record["bench_wall_s"] = round(time.perf_counter() - t0, 1)
    print(json.dumps(record))
    return 0


# ------------------------------------------------------------------ decode
class BenchFailure(Exception):
    """A correctness gate failed: `record` is the JSON line to print."""

    def __init__(self, record: dict):
        super().__init__(record.get("error", "bench failure"))
        self.record = record


def append_matches(w) -> bool:
    """Whether the step's 1-token append left exactly the new K/V rows at
    each request's slot: bit for bit for a 16-bit cache, the codes and
    scales quantize_rows_e4m3 gives for the FP8 cache."""
    cache, bs = w["cache"], w["block_size"]
    # k / v are [layers, blocks, block_size, kv_heads, D] views whatever the
    # storage order; the FP8 scales are [layers, blocks, kv_heads, block_size]
    assert tuple(cache.k.shape[1:3]) == (w["pool"], bs)
    slots = w["slots"].long().cpu()
    blk, off = slots // bs, slots % bs
    assert int(blk.max()) < w["pool"] and int(off.max()) < bs
    blk, off = blk.to(cache.k.device), off.to(cache.k.device)
    if w["fp8"]:
        from inferkernellab_amd.cache import quantize_rows_e4m3

        assert tuple(cache.k_scale.shape[1:]) == (w["pool"], w["kv_heads"], bs)
        ok = True
        for new, codes, scales in ((w["new_k"], cache.k, cache.k_scale), (w["new_v"], cache.v, cache.v_scale)):
            c, sc = quantize_rows_e4m3(new)
            ok = ok and torch.equal(codes[0][blk, off].view(torch.uint8), c.view(torch.uint8))
            ok = ok and torch.equal(scales[0][blk, :, off], sc)
        return bool(ok)
    views = []
    for new, t in ((w["new_k"], cache.k), (w["new_v"], cache.v)):
        views.append(torch.equal(t[0][blk, off].view(torch.int16), new.view(torch.int16)))
    return all(views)


def measure_decode(workload: str, device: torch.device, *, steps: int, warmup: int, seed: int = 0,
                   partition: int | None = None, head_major: bool | None = None, separate_append: bool = False,
                   graph: bool = True, mall_flush: str = "auto", cpu_budget_s: float | None = None) -> dict:
    """One decode-step workload, measured: the correctness gate (every
    request against the oracle, and the appended rows), then `steps` timed
    steps eagerly with HIP events around the split kernel and the reduce,
    then as HIP graph replays. Returns the figures (raises BenchFailure when
    the gate fails)."""
    from inferkernellab_amd import ops

    w = build_workload(workload, device, seed, head_major=head_major)
    partition = partition or WORKLOADS[workload][9]
    attn = ops.PreparedPagedAttention(
        w["query"], w["cache"], w["tables"], w["lens"], validate_inputs=True,
        partition_size=partition, max_context_len=max(w["lengths"]),
    )
    append = ops.PreparedAppend(w["new_k"], w["new_v"], w["cache"], w["slots"])
    step = ops.PreparedDecodeStep(attn, append)

    def run_step(events=None) -> None:
        """Attention then the 1-token append: one library call (the append
        rides on the split reduce kernel when it can), or, separately, the
        two operators launched one after the other."""
        if separate_append:
            attn(events=events)
            append()
        else:
            step(events=events)

    events = HipEvents()
    ev = [[events.create() for _ in range(3)] for _ in range(steps)]
    attn_bytes, append_bytes = step_bytes(w)
    flush = mall_flush == "on" or (mall_flush == "auto" and attn_bytes < MALL_FLUSH_BELOW)
    flush_buf = MallFlush(device) if flush else None
    flush_marks = []

    def flush_mall() -> None:
        """512 MiB of reads (evicts the MALL and the L2s), bracketed by
        events so that the step time can leave it out."""
        if flush_buf is not None:
            e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
            e0.record()
            flush_buf()
            e1.record()
            flush_marks.append((e0, e1))

    def flush_seconds() -> float:
        t = sum(a.elapsed_time(b) for a, b in flush_marks) / 1e3
        flush_marks.clear()
        return t

    # Correctness gate before timing, like the reference's harness
    # (benchmark.py:225-268, which raises when the kernel differs from its
    # PyTorch reference): one eager step, every request against the oracle,
    # and the appended rows against the new K/V. It runs the timed steps'
    # own launches; the append writes past each context, where the oracle
    # does not read, and the timed steps rewrite the same rows.
    run_step()
    torch.cuda.synchronize()
    view = oracle_view(w)
    t_oracle = time.perf_counter()
    expected = oracle_step(view, w)
    first_oracle_s = time.perf_counter() - t_oracle
    check = parity(attn.out, expected, w["dtype"])
    check["checked"] = f"all {len(w['lengths'])} requests x {w['heads']} heads of one eager step"
    check["append_exact"] = append_matches(w)
    if not check["passed"]:
        raise BenchFailure({"error": "decode attention output differs from the oracle", "workload": workload,
                            "parity": check})
    if not check["append_exact"]:
        raise BenchFailure({"error": "the step's KV append differs from the new rows", "workload": workload,
                            "parity": check})
    checked_out = attn.out.clone()
    del expected

    for _ in range(warmup):
        run_step()
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    for i in range(steps):
        flush_mall()
        run_step(events=ev[i])
    torch.cuda.synchronize()
    wall_s = eager_wall_s = time.perf_counter() - t0 - flush_seconds()
    step_mode = "eager launches"
    single_graph_us = None
    if graph:
        # HIP graphs: a decode loop's launch pattern, without the host's
        # per-kernel dispatch. Inside a graph the reduce starts as the split
        # kernel ends, but every replay costs several µs before its first
        # kernel. A model's decode graph holds one attention step per layer,
        # so that cost is shared by all of them: the K timed steps are
        # captured back to back in one graph and replayed once (exactly K
        # steps). Workloads that flush the MALL before every step capture
        # the flush in front of each step of that graph, and a second graph
        # of the K flushes alone; the step time is their difference over K.
        # The one-step-per-replay rate is reported beside it.
        def capture(n: int, body=None) -> torch.cuda.CUDAGraph:
            body = body or run_step
            side = torch.cuda.Stream(device)
            side.wait_stream(torch.cuda.current_stream(device))
            with torch.cuda.stream(side):
                body()
            torch.cuda.current_stream(device).wait_stream(side)
            g = torch.cuda.CUDAGraph()
            with torch.cuda.graph(g):
                for _ in range(n):
                    body()
            return g

        def replay_s(g: torch.cuda.CUDAGraph) -> float:
            torch.cuda.synchronize()
            t = time.perf_counter()
            g.replay()
            torch.cuda.synchronize()
            return time.perf_counter() - t

        one = capture(1)
        for _ in range(warmup):
            one.replay()
        torch.cuda.synchronize()
        t0 = time.perf_counter()
        for i in range(steps):
            flush_mall()
            one.replay()
        torch.cuda.synchronize()
        single_s = time.perf_counter() - t0 - flush_seconds()
        single_graph_us = single_s * 1e6 / steps
        wall_s = single_s
        step_mode = "hip graph replay, one step per replay"
        if flush_buf is None:
            many = capture(steps)
            many.replay()  # warm
            wall_s = replay_s(many)
            step_mode = "hip graph of the K steps back to back, replayed once"
            del many
        else:
            probe = ProbeFlush(device)

            def flushed_step() -> None:
                probe()
                run_step()

            both, flushes = capture(steps, flushed_step), capture(steps, probe)
            both.replay()  # warm
            flushes.replay()
            # median of 5 interleaved pairs of replays
            diffs = sorted(replay_s(both) - replay_s(flushes) for _ in range(5))
            wall_s = diffs[len(diffs) // 2]
            step_mode = ("hip graph of the K steps, each behind a 512 MiB MALL flush read, minus a graph of the "
                         "K flushes alone (median of 5 pairs of replays)")
            del both, flushes, probe
        del one
    torch.cuda.synchronize()
    # every timed step recomputes the checked output (same inputs; the
    # append writes past each context): the last one must equal it bit for bit
    same = torch.equal(attn.out.view(torch.int16) if attn.out.element_size() == 2 else attn.out,
                       checked_out.view(torch.int16) if checked_out.element_size() == 2 else checked_out)
    check["timed_steps_equal_checked_step"] = bool(same)
    if not same:
        raise BenchFailure({"error": "timed steps changed the attention output", "workload": workload,
                            "parity": check})
    kernel_ms = [events.elapsed_ms(e[0], e[1]) for e in ev]
    reduce_ms = [events.elapsed_ms(e[1], e[2]) for e in ev]
    both_ms = [events.elapsed_ms(e[0], e[2]) for e in ev]
    for trio in ev:
        for h in trio:
            events.destroy(h)

    traffic = None
    traffic_file = ROOT / "profiles" / f"traffic_{workload}.json"
    if traffic_file.exists():
        try:
            traffic = json.loads(traffic_file.read_text()).get("hbm_bytes_per_launch")
        except (OSError, ValueError):
            traffic = None
    cpu = cpu_baseline(w, view, cpu_budget_s, first_oracle_s) if cpu_budget_s is not None else None
    kern_avg_ms = sum(kernel_ms) / len(kernel_ms)
    m = {
        "workload": workload,
        "w": {k: w[k] for k in ("lengths", "dtype", "fp8", "heads", "kv_heads", "head_dim", "block_size", "pool")},
        "head_major": w["cache"].head_major,
        "attn": attn,
        "step": step,
        "separate_append": separate_append,
        "flush": flush,
        "steps": steps,
        "warmup": warmup,
        "wall_s": wall_s,
        "eager_wall_s": eager_wall_s,
        "single_graph_us": single_graph_us,
        "step_mode": step_mode,
        "kernel_ms": kernel_ms,
        "reduce_ms": reduce_ms,
        "both_ms": both_ms,
        "kern_avg_ms": kern_avg_ms,
        "attn_bytes": attn_bytes,
        "append_bytes": append_bytes,
        "check": check,
        "traffic": traffic,
        "cpu": cpu,
        "mfma": mfma_figures(w, attn, kern_avg_ms, workload),
    }
    del w, view
    return m


def split_name(m) -> str:
    attn, step = m["attn"], m["step"]
    if attn.balanced_split:
        return "balanced (equal tile runs per resident workgroup)"
    if attn.launch["split"] != "none":
        return f"fixed partitions of {attn.partition_size} tokens"
    if attn.launch["path"] != "mfma_grouped" and attn.launch["num_warps"] > 1:
        return "none: up to 4 partitions per request folded into one multi-wave workgroup"
    return "none"


def decode_record(m) -> dict:
    """The headline JSON record of one measured decode workload."""
    w, attn, step = m["w"], m["attn"], m["step"]
    k_steps = m["steps"]
    ms_per_step = m["wall_s"] * 1e3 / k_steps
    step_gbps = (m["attn_bytes"] + m["append_bytes"]) / (ms_per_step * 1e-3) / 1e9
    kern_avg_ms = m["kern_avg_ms"]
    # Algorithmic bytes of the partition kernel: K/V + q + tables + lengths
    # (+ its fp32 partial writes are workspace traffic, not algorithmic).
    achieved = m["attn_bytes"] / (kern_avg_ms * 1e-3) / 1e9
    return {
        "metric": METRIC,
        "value": round(step_gbps, 1),
        "unit": "GB/s",
        "n_gpus": 1,
        "steps": k_steps,
        "warmup": m["warmup"],
        "ms_per_step": round(ms_per_step, 4),
        "us_per_step": round(ms_per_step * 1e3, 1),
        "step_mode": m["step_mode"],
        "step_timing": (("wall clock around the graph of the K flushed steps minus that around the graph of "
                         "the K flushes, each synchronized on both sides" if m["single_graph_us"] is not None
                         else "wall clock around the K steps, synchronized on both sides, minus the "
                              "event-timed 512 MiB MALL flush read before each step") if m["flush"]
                        else "wall clock around the K steps, synchronized on both sides"),
        "eager_us_per_step": round(m["eager_wall_s"] * 1e6 / k_steps, 1),
        "one_step_graph_us_per_step": (round(m["single_graph_us"], 1) if m["single_graph_us"] is not None
                                       else None),
        "pct_of_peak_hbm": round(100 * step_gbps / PEAK_HBM_GBPS, 1),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": {torch.bfloat16: "bf16", torch.float16: "fp16", torch.float32: "fp32"}[w["dtype"]],
        "data": "synthetic (seeded N(0,1) K/V/q, random-permutation block tables)",
        "config": {
            "workload": m["workload"],
            "batch": len(w["lengths"]),
            "num_heads": w["heads"],
            "num_kv_heads": w["kv_heads"],
            "head_dim": w["head_dim"],
            "block_size": w["block_size"],
            "num_blocks": w["pool"],
            "context_tokens": sum(w["lengths"]),
            "kv_cache": "fp8 e4m3 codes + one fp32 scale per (token, kv head)" if w["fp8"] else "same as dtype",
            "kv_block_layout": "[kv_heads, block_size, D]" if m["head_major"] else "[block_size, kv_heads, D]",
            "partition_size": attn.partition_size,
            "split": split_name(m),
            "step": ("paged attention then a 1-token KV append per request: "
                     + ("two operator launches" if m["separate_append"]
                        else "one library call, the append carried by the reduce kernel" if step.fused
                        else "one library call, the attention then the append kernel")),
            "kernels": ([n for n in attn.kernel_names() if n] + ["append_kv_kernel"] if m["separate_append"]
                        else list(step.kernel_names())),
            "parallelism": "single GPU",
        },
        "attention_kernel_us": round(kern_avg_ms * 1e3, 2),
        "attention_kernel_p50_us": round(_percentile(m["kernel_ms"], 0.5) * 1e3, 2),
        "attention_kernel_p95_us": round(_percentile(m["kernel_ms"], 0.95) * 1e3, 2),
        "reduce_kernel_us": round(sum(m["reduce_ms"]) / len(m["reduce_ms"]) * 1e3, 2),
        "reduce_carries_append": bool(step.fused and not m["separate_append"]),
        "algorithmic_bytes_per_step": m["attn_bytes"] + m["append_bytes"],
        "roofline": {
            "bound": "hbm",
            "achieved": round(achieved, 1),
            "peak": PEAK_HBM_GBPS,
            "unit": "GB/s",
            "frac": round(achieved / PEAK_HBM_GBPS, 4),
            "traffic": m["traffic"],
            "kernel": attn.kernel_names()[0],
            "algorithmic_bytes_per_launch": m["attn_bytes"],
        },
        "mfma": m["mfma"],
        "parity": m["check"],
        "cpu_baseline": m["cpu"],
    }


def config_entry(m, spec: str) -> dict:
    """One measured decode workload, compact, for the default line's
    `configs` block: parity, kernel / reduce / step times and the kernel's
    roofline fraction."""
    rec = decode_record(m)
    kernel_us = rec["attention_kernel_us"]
    both_us = sum(m["both_ms"]) / len(m["both_ms"]) * 1e3
    step_bytes_ = m["attn_bytes"] + m["append_bytes"]
    return {
        "spec": spec,
        "workload": m["workload"],
        "dtype": rec["dtype"],
        "kv_cache": rec["config"]["kv_cache"],
        "split": rec["config"]["split"],
        "partition_size": rec["config"]["partition_size"],
        "step": rec["config"]["step"],
        "kernels": rec["config"]["kernels"],
        "max_abs_err": m["check"]["max_abs_err"],
        "tolerance": m["check"]["tolerance"],
        "parity_passed": m["check"]["passed"],
        "append_exact": m["check"]["append_exact"],
        "kernel_us": kernel_us,
        "kernel_p50_us": rec["attention_kernel_p50_us"],
        "reduce_us": rec["reduce_kernel_us"],
        "kernel_plus_reduce_us": round(both_us, 2),
        "step_us": rec["us_per_step"],
        "step_mode": rec["step_mode"],
        "mall_flushed": m["flush"],
        "algorithmic_bytes_per_launch": m["attn_bytes"],
        "algorithmic_bytes_per_step": step_bytes_,
        "roofline_frac": rec["roofline"]["frac"],
        "kernel_plus_reduce_frac": round(step_bytes_ / (both_us * 1e-6) / 1e9 / PEAK_HBM_GBPS, 4),
        "step_frac": round(rec["pct_of_peak_hbm"] / 100, 4),
    }


def c1_cpu_reference(device: torch.device, samples: int = 10, warmup: int = 2) -> dict:
    """The CPU decode configuration: batch 4, context 512, GQA 32 / 8, head_dim
    64, fp32, block 16, 159 physical blocks. q, k and v come from seed 0 in
    the order the reference's case builder draws them (benchmark.py:73-110:
    per request a key then a value tensor, then the query); each request's
    table is a slice of one random permutation (seed 1) of the 159 blocks;
    the cache is filled by appending every context token through
    slot_mapping (the oracle's write_slots, cache.py:156-189, and the HIP
    append into the device cache, compared bit for bit). The oracle's
    paged_reference is timed over `samples` whole steps after `warmup`
    (warmup plus at least 10 samples); the HIP kernel runs on the
    same inputs beside it."""
    import numpy as np
    from oracle import paged_oracle as po

    from inferkernellab_amd import PagedKVCache, ops

    B, L, H, HKV, D, BS, NB = 4, 512, 32, 8, 64, 16, 159
    gen_state = torch.random.get_rng_state()
    torch.manual_seed(0)
    keys, values = [], []
    for _ in range(B):
        k = torch.randn(L, HKV, D, dtype=torch.float32)
        keys.append(k)
        values.append(torch.randn_like(k))
    query = torch.randn(B, H, D, dtype=torch.float32)
    torch.random.set_rng_state(gen_state)
    perm = torch.randperm(NB, generator=torch.Generator().manual_seed(1)).tolist()
    per = L // BS
    tables = [perm[b * per:(b + 1) * per] for b in range(B)]
    oc = po.OracleCache(NB, BS, HKV, D, dtype="float32", fill=np.nan)
    slots = [oc.slot_mapping(t, 0, L) for t in tables]
    for b in range(B):
        oc.write_slots(0, slots[b], keys[b].numpy(), values[b].numpy())
    q = query.numpy()
    times = []
    for i in range(warmup + samples):
        t0 = time.perf_counter()
        expected = po.paged_decode_attention(q, oc, tables, [L] * B)
        if i >= warmup:
            times.append(time.perf_counter() - t0)
    mean_s = sum(times) / len(times)
    kv_bytes = B * L * HKV * D * 2 * 4

    # the HIP path on the same inputs: append every token, then attend
    cache = PagedKVCache(NB, BS, HKV, D, dtype=torch.float32, device=device)
    cache.k.fill_(float("nan"))
    cache.v.fill_(float("nan"))
    dev_slots = torch.tensor(np.concatenate(slots), dtype=torch.int32, device=device)
    ops.append_kv_hip(torch.cat(keys).to(device), torch.cat(values).to(device), cache, dev_slots)
    torch.cuda.synchronize()
    append_exact = bool(np.array_equal(cache.k.cpu().numpy(), oc.k, equal_nan=True)
                        and np.array_equal(cache.v.cpu().numpy(), oc.v, equal_nan=True))
    tables_d = torch.tensor(tables, dtype=torch.int32, device=device)
    lens_d = torch.full((B,), L, dtype=torch.int32, device=device)
    attn = ops.PreparedPagedAttention(query.to(device), cache, tables_d, lens_d, max_context_len=L)
    attn()
    torch.cuda.synchronize()
    err = float(np.max(np.abs(attn.out.cpu().numpy() - expected)))
    for _ in range(5):
        attn()
    start, stop = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    start.record()
    for _ in range(20):
        attn()
    stop.record()
    stop.synchronize()
    hip_us = start.elapsed_time(stop) * 1e3 / 20
    return {
        "spec": "CPU paged_reference decode attention, fp32: B4 x ctx 512, GQA 32/8, head_dim 64, block 16, "
                "159 blocks; seed-0 q/k/v, seed-1 permutation tables, cache filled by append",
        "cpu_paged_reference_us": round(mean_s * 1e6, 1),
        "cpu_p50_us": round(_percentile(times, 0.5) * 1e6, 1),
        "cpu_p95_us": round(_percentile(times, 0.95) * 1e6, 1),
        "cpu_gbps": round(kv_bytes / mean_s / 1e9, 3),
        "samples": samples,
        "warmup": warmup,
        "cores": host_threads(),
        "kind": "port",
        "cpu_sample": "oracle paged_reference (numpy fp32 per-request loop), whole steps of all 4 requests",
        "hip_append_exact": append_exact,
        "hip_kernel_us": round(hip_us, 2),
        "hip_path": attn.path,
        "hip_max_abs_err": err,
        "tolerance": TOLERANCE[torch.float32],
        "hip_parity_passed": bool(err <= TOLERANCE[torch.float32]),
    }


def read_ceiling(device: torch.device, nbytes: int = 512 << 20, samples: int = 5) -> dict:
    """Event-timed plain-stream read of a contiguous 512 MiB buffer
    (ikl_hbm_read_probe), best and median of `samples` launches after one
    warm launch: the HBM read rate the device delivers in this run."""
    from inferkernellab_amd import _lib

    lib = _lib.load()
    buf = torch.ones(nbytes // 4, dtype=torch.int32, device=device)
    sink = torch.zeros(1 << 14, dtype=torch.int32, device=device)
    stream = torch.cuda.current_stream(device).cuda_stream

    def launch():
        _lib.check(lib.ikl_hbm_read_probe(ctypes.c_void_p(buf.data_ptr()), nbytes, ctypes.c_void_p(sink.data_ptr()),
                                          sink.numel() * 4, ctypes.c_void_p(stream)), "read probe")

    launch()
    times = []
    for _ in range(samples):
        start, stop = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        start.record()
        launch()
        stop.record()
        stop.synchronize()
        times.append(start.elapsed_time(stop) * 1e-3)
    best = min(times)
    med = sorted(times)[len(times) // 2]
    del buf
    return {
        "read_ceiling_gbps": round(nbytes / best / 1e9, 1),
        "read_median_gbps": round(nbytes / med / 1e9, 1),
        "bytes": nbytes,
        "samples": samples,
        "kernel": "hbm_read_probe_kernel (one contiguous chunk per one-wave workgroup, 16-byte non-temporal "
                  "loads, 8 waves per CU)",
    }


def environment(argv) -> dict:
    """Where and from what the line was measured (the reference records
    its environment beside every result: benchmark.py:154-163,
    hf_benchmark.py:847-871)."""
    import hashlib
    import platform

    from inferkernellab_amd import _lib
    from inferkernellab_amd.build import source_hash

    props = torch.cuda.get_device_properties(0)
    lib = _lib.load()
    version = lib.ikl_version().decode()
    so_hash = hashlib.sha256(_lib.LIB_PATH.read_bytes()).hexdigest()[:16]
    built = dict(part.split(":", 1) for part in version.split()[-1].split(",") if ":" in part)
    rocm = None
    try:
        rocm = Path("/opt/rocm/.info/version").read_text().strip()
    except OSError:
        pass
    return {
        "gpu": props.name,
        "gcn_arch": getattr(props, "gcnArchName", None),
        "compute_units": props.multi_processor_count,
        "hbm_bytes": props.total_memory,
        "torch": torch.__version__,
        "hip": torch.version.hip,
        "rocm": rocm,
        "library": version,
        "library_sha256_16": so_hash,
        "library_abi_version": lib.ikl_abi_version(),
        "built_from_git": built.get("git"),
        "built_source_hash": built.get("src"),
        "library_matches_sources": built.get("src") == source_hash(),
        "host_cpu": cpu_model(),
        "host_logical_cpus": os.cpu_count(),
        "python": platform.python_version(),
        "command": " ".join([Path(sys.executable).name, *argv]),
    }


# The default line's configurations beyond the headline: (key, workload,
# partition, spec). The fixed-512 entry is the GQA configuration exactly as
# written (512-token partitions + reduce), beside the automatic split the
# headline times.
DEFAULT_CONFIGS = (
    ("mha_fp16_append", "mha32_hd128_fp16_b16_ctx512", None,
     "MHA paged decode + KV append, fp16: B16 x 512, 32 = 32 heads, head_dim 128, block 16"),
    ("mqa_bf16", "mqa32x1_hd128_bf16_b64_ctx1k-4k", None,
     "MQA paged decode, bf16: B64, 32 / 1 heads, head_dim 128, ragged U[1024, 4096], K/V 0.5 N(0,1)"),
    ("gqa_bf16_fixed512", DEFAULT_WORKLOAD, 512,
     "GQA 32/8 hd128 bf16 B32 x U[4096, 8192] with split-context partitions of 512 tokens + reduce"),
    ("gqa_fp8kv", "gqa32x8_hd128_fp8kv_b32_ctx4k-8k", None,
     "the GQA decode configuration over the FP8 (E4M3, per-row scale) KV cache"),
    ("gqa_kv_heads_over_8_gpus", "gqa4x1_hd128_bf16_b32_ctx4k-8k", None,
     "one GPU's share of the GQA 32/8 hd128 bf16 B32 x U[4096, 8192] step when its KV heads are split over 8 "
     "GPUs: 4 / 1 heads, the same lengths and tables"),
    ("gqa_kv_heads_over_2_gpus", "gqa16x4_hd128_bf16_b32_ctx4k-8k", None,
     "one GPU's share of the same step over 2 GPUs: 16 / 4 heads"),
)


def main() -> int:
    parser = argparse.ArgumentParser(description=__doc__.splitlines()[0])
    parser.add_argument("--gpus", type=int, default=1)
    parser.add_argument("--steps", type=int, default=50)
    parser.add_argument("--warmup", type=int, default=10)
    parser.add_argument("--workload", default=DEFAULT_WORKLOAD,
                        choices=sorted(WORKLOADS) + sorted(PREFILL_WORKLOADS) + ["llama_e2e"])
    parser.add_argument("--partition-size", type=int, default=None,
                        help="tokens per fixed split partition (default: the library's automatic split)")
    parser.add_argument("--cpu-budget-s", type=float, default=15.0)
    parser.add_argument("--no-cpu-baseline", action="store_true")
    parser.add_argument("--no-configs", action="store_true",
                        help="the headline workload only: no configs block, read ceiling or CPU decode case")
    parser.add_argument("--seed", type=int, default=0)
    parser.add_argument("--kv-layout", choices=("default", "token-major", "head-major"), default="default",
                        help="cache block layout: [block_size, kv_heads, D] (the reference's, default for "
                             "16-bit caches) or [kv_heads, block_size, D] (default for the FP8 cache)")
    parser.add_argument("--separate-append", action="store_true",
                        help="launch the append as its own kernel after the attention instead of "
                             "letting the split reduce kernel carry it (same result)")
    parser.add_argument("--no-graph", action="store_true",
                        help="time eager launches instead of HIP graph replays of the step")
    parser.add_argument("--mall-flush", choices=("auto", "on", "off"), default="auto",
                        help="read a 512 MiB buffer before every timed sample so that the K/V of "
                             "the step is not served from the 256 MB MALL (auto: when the step's "
                             "K/V is below 384 MiB, 1.5x the MALL)")
    parser.add_argument("--copy-calibration", action="store_true",
                        help="run only a plain 512 MiB device copy (torch copy_) three times: the "
                             "known-size reference for scaling FETCH_SIZE / WRITE_SIZE counters")
    parser.add_argument("--sweep", action="store_true",
                        help="run the reference's 54-shape attention sweep (each shape checked against "
                             "the oracle, then timed; --steps samples after --warmup launches)")
    parser.add_argument("--sweep-out", default=None, help="JSONL file for the sweep's per-shape records")
    parser.add_argument("--check-requests", type=int, default=16,
                        help="llama_e2e: requests whose greedy tokens are checked against the CPU oracle")
    args = parser.parse_args()

    if args.gpus != 1:
        print(json.dumps({"error": "this benchmark runs on exactly one GPU: the paged decode path "
                                   "is measured on one GPU's share; --gpus must be 1"}))
        return 2
    if not torch.cuda.is_available():
        print(json.dumps({"error": "no GPU visible"}))
        return 2

    device = torch.device("cuda", 0)
    torch.cuda.set_device(device)
    if args.copy_calibration:
        nbytes = 512 << 20
        src = torch.ones(nbytes // 4, dtype=torch.int32, device=device)
        dst = torch.empty_like(src)
        for _ in range(3):
            dst.copy_(src)
        torch.cuda.synchronize()
        print(json.dumps({"copy_calibration": {"bytes_read": nbytes, "bytes_written": nbytes, "launches": 3}}))
        return 0

    if args.sweep:
        return run_sweep(args, device)
    if args.workload in PREFILL_WORKLOADS:
        return run_prefill(args, device)
    if args.workload == "llama_e2e":
        return run_llama_e2e(args, device)

    t_start = time.perf_counter()
    head_major = {"default": None, "token-major": False, "head-major": True}[args.kv_layout]
    try:
        m = measure_decode(args.workload, device, steps=args.steps, warmup=args.warmup, seed=args.seed,
                           partition=args.partition_size, head_major=head_major,
                           separate_append=args.separate_append, graph=not args.no_graph,
                           mall_flush=args.mall_flush,
                           cpu_budget_s=None if args.no_cpu_baseline else args.cpu_budget_s)
        record = decode_record(m)
        del m
        if args.workload == DEFAULT_WORKLOAD and not args.no_configs:
            configs = {"cpu_decode_fp32": c1_cpu_reference(device)}
            for key, workload, partition, spec in DEFAULT_CONFIGS:
                cm = measure_decode(workload, device, steps=args.steps, warmup=args.warmup, seed=args.seed,
                                    partition=partition, graph=not args.no_graph, mall_flush=args.mall_flush)
                configs[key] = config_entry(cm, spec)
                del cm
                torch.cuda.empty_cache()
            configs["llama_e2e"] = llama_e2e_entry(device, check_requests=2, seed=args.seed)
            record["configs"] = configs
            record["read_ceiling"] = read_ceiling(device)
            record["roofline"]["frac_of_read_ceiling"] = round(
                record["roofline"]["achieved"] / record["read_ceiling"]["read_ceiling_gbps"], 4)
    except BenchFailure as exc:
        print(json.dumps(exc.record))
        return 3
    record["environment"] = environment(sys.argv)
    record["bench_wall_s"] = round(time.perf_counter() - t_start, 1)
    print(json.dumps(record))
    return 0


if __name__ == "__main__":
    sys.exit(main())
