"""CPU oracle of the paged-KV decode path — TEST INFRASTRUCTURE ONLY.

Only ``tests/``, ``__graft_entry__.smoke()`` and the ``cpu_baseline`` leg of
``bench.py`` may import this module, and only as the checker (or as the
timed CPU baseline); the product path (``inferkernellab_amd``) never routes
through it.

It restates, in numpy, the reference's algorithm for this path:

* ``OracleCache.slot_mapping``   — cache.py:113-129
* ``OracleCache.write_slots``    — cache.py:156-189 (torch index_put semantics)
* ``OracleCache.write``          — cache.py:131-154
* ``OracleCache.read``           — cache.py:191-200
* ``expand_kv``                  — attention.py:9-15 (repeat_interleave)
* ``dense_decode_attention``     — attention.py:18-36 (fp32 einsum/softmax/einsum)
* ``paged_decode_attention``     — attention.py:134-175 (= backend ``paged_reference``)
* ``rope_rows``                  — hf_benchmark.py:69-85 (rotate-half RoPE before the append)
* ``paged_prefill_attention``    — attention.py:230-321 (gather + causal masked SDPA of a
  ragged prompt-chunk batch)
* ``e4m3_encode`` / ``e4m3_decode`` / ``quantize_rows_e4m3`` — the FP8 KV format (no
  counterpart in the reference): OCP E4M3 codes with round-to-nearest-even,
  saturated to +-448, and one power-of-two fp32 scale per (token, kv head)
  row, scale = 2^ceil(log2(amax / 448)), code = e4m3(x / scale)

Storage keeps the cache's own element type: float16 and float32 as numpy
arrays of that type, bfloat16 as raw ``uint16`` bit patterns (numpy has no
bfloat16), so append results can be compared bit for bit. Attention upcasts
to float32 exactly like ``query.float()`` / ``key.float()`` in the reference
and returns float32 (the tolerance reference); ``cast_output`` applies the
reference's final ``.to(query.dtype)``.

Parity pins (each checked in tests/test_oracle.py):
* slot_mapping / write / read / allocator: the known answers of the
  reference's tests (tests/golden/known_answers.json, transcribed from
  tests/test_cache.py:8-84 and tests/test_attention.py:129-144);
* attention: float64 brute force on tiny inputs, closed forms (context 1 ->
  v, equal keys -> mean of v, one dominant key -> its v), MHA == GQA after
  explicit head expansion, block-table permutation invariance, and torch's
  own softmax/einsum on the same data;
* rope_rows: torch's own elementwise ops on the same storage, bit for bit,
  in the three dtypes; position 0 (cos 1, sin 0) is the identity;
* paged_prefill_attention: every attending row equals the (pinned) decode
  attention over its own prefix — the check of the reference's test
  (tests/test_attention.py:90-116), run on that test's tables and ranges —
  plus a float64 causal brute force and torch SDPA under the reference's
  mask construction (padding rows included);
* e4m3_encode: bit-for-bit against torch's float -> float8_e4m3fn conversion
  on random values, ties, subnormals, signed zeros and the +-448 ends;
  e4m3_decode: every one of the 256 codes against torch's decode;
  quantize_rows_e4m3: closed forms (power-of-two scales, the row maximum
  lands in (224, 448], zero rows keep scale 1, dequantised rows within half
  an e4m3 step).
"""

from __future__ import annotations

import math

import numpy as np

DTYPES = ("float16", "bfloat16", "float32")


# ------------------------------------------------------------ element types
def bf16_bits_to_f32(bits: np.ndarray) -> np.ndarray:
    """Exact bfloat16 -> float32 widening of raw uint16 bit patterns."""
    return (np.asarray(bits, dtype=np.uint16).astype(np.uint32) << 16).view(np.float32)


def f32_to_bf16_bits(x: np.ndarray) -> np.ndarray:
    """float32 -> bfloat16 bits, round to nearest even (NaN stays NaN)."""
    u = np.asarray(x, dtype=np.float32).view(np.uint32).astype(np.uint64)
    nan = (u & 0x7FFFFFFF) > 0x7F800000
    rounded = ((u + 0x7FFF + ((u >> 16) & 1)) >> 16).astype(np.uint16)
    return np.where(nan, np.uint16(0x7FC0), rounded).astype(np.uint16)


def to_f32(storage: np.ndarray, dtype: str) -> np.ndarray:
    if dtype == "bfloat16":
        return bf16_bits_to_f32(storage)
    return np.asarray(storage).astype(np.float32)


def storage_dtype(dtype: str):
    return {"float16": np.float16, "bfloat16": np.uint16, "float32": np.float32}[dtype]


def cast_output(x: np.ndarray, dtype: str) -> np.ndarray:
    """The reference's ``.to(query.dtype)`` (attention.py:36), as storage."""
    if dtype == "bfloat16":
        return f32_to_bf16_bits(x)
    return np.asarray(x, dtype=np.float32).astype(storage_dtype(dtype))


# ------------------------------------------------------------------- rope
def rope_rows(x: np.ndarray, cos: np.ndarray, sin: np.ndarray, dtype: str) -> np.ndarray:
    """Rotate-half RoPE on storage arrays, with the rounding of the
    reference's torch ops (hf_benchmark.py:69-85): ``x * cos`` and
    ``rotate_half(x) * sin`` each rounded to ``dtype``, then their sum
    rounded. x ``[..., D]``; cos / sin broadcast against x. Returns storage."""
    half = x.shape[-1] // 2
    xf, cf, sf = to_f32(x, dtype), to_f32(cos, dtype), to_f32(sin, dtype)
    rot = np.concatenate([-xf[..., half:], xf[..., :half]], axis=-1)

    def rnd(v):  # one elementwise op's result in `dtype`
        return to_f32(cast_output(v, dtype), dtype)

    return cast_output(rnd(xf * cf) + rnd(rot * sf), dtype)


# -------------------------------------------------------------------- cache
class OracleCache:
    """Storage ``[layers, blocks, block_size, kv_heads, head_dim]`` (cache.py:90)."""

    def __init__(self, num_blocks, block_size, num_kv_heads, head_dim, *, num_layers=1,
                 dtype="float32", fill=np.nan):
        if min(num_layers, num_blocks, block_size, num_kv_heads, head_dim) <= 0:
            raise ValueError("cache dimensions must be positive")
        if dtype not in DTYPES:
            raise ValueError(f"unsupported dtype {dtype}")
        self.num_layers = num_layers
        self.num_blocks = num_blocks
        self.block_size = block_size
        self.num_kv_heads = num_kv_heads
        self.head_dim = head_dim
        self.dtype = dtype
        shape = (num_layers, num_blocks, block_size, num_kv_heads, head_dim)
        sd = storage_dtype(dtype)
        if dtype == "bfloat16":
            init = f32_to_bf16_bits(np.float32(fill))
        else:
            init = sd(fill)
        self.k = np.full(shape, init, dtype=sd)
        self.v = np.full(shape, init, dtype=sd)

    @classmethod
    def wrap(cls, k: np.ndarray, v: np.ndarray, dtype: str) -> "OracleCache":
        """A cache over existing storage arrays ``[layers, blocks, block_size,
        kv_heads, head_dim]`` (no copy), e.g. a device cache copied to host."""
        if k.shape != v.shape or k.ndim != 5:
            raise ValueError("k/v must share a [L, NB, bs, Hkv, D] shape")
        if dtype not in DTYPES or k.dtype != storage_dtype(dtype) or v.dtype != k.dtype:
            raise ValueError(f"storage arrays do not hold {dtype}")
        self = cls.__new__(cls)
        self.num_layers, self.num_blocks, self.block_size, self.num_kv_heads, self.head_dim = k.shape
        self.dtype = dtype
        self.k, self.v = k, v
        return self

    def slot_mapping(self, block_table, start: int, length: int) -> np.ndarray:
        """slot(p) = table[p // bs] * bs + p % bs for p in [start, start+length)."""
        if start < 0 or length < 0:
            raise ValueError("start and length must be non-negative")
        table = list(block_table)
        if any(not isinstance(b, (int, np.integer)) or not 0 <= int(b) < self.num_blocks for b in table):
            raise ValueError("block_table contains an invalid physical block id")
        if length and (start + length - 1) // self.block_size >= len(table):
            raise ValueError("block_table is shorter than the requested range")
        out = np.empty(length, dtype=np.int64)
        for i, p in enumerate(range(start, start + length)):
            out[i] = int(table[p // self.block_size]) * self.block_size + p % self.block_size
        return out

    def write_slots(self, layer: int, slots, key: np.ndarray, value: np.ndarray, *,
                    validate_slots: bool = True) -> None:
        """k[layer, slot // bs, slot % bs, :, :] = key[t] for every token t."""
        key = np.asarray(key)
        value = np.asarray(value)
        slots = np.asarray(slots, dtype=np.int64).reshape(-1)
        if key.shape != value.shape or key.ndim != 3:
            raise ValueError("key/value must have the same [T, H, D] shape")
        if slots.shape[0] != key.shape[0]:
            raise ValueError("slots must have one entry per key/value token")
        if key.shape[1:] != (self.num_kv_heads, self.head_dim):
            raise ValueError("key/value shape does not match cache layout")
        if not 0 <= layer < self.num_layers:
            raise IndexError("layer is out of range")
        limit = self.num_blocks * self.block_size
        if validate_slots and slots.size and (slots.min() < 0 or slots.max() >= limit):
            raise ValueError("slots contain an invalid physical cache position")
        # numpy fancy assignment: with duplicate slots the last row wins (the
        # reference's torch index_put leaves that order unspecified)
        blocks, offsets = slots // self.block_size, slots % self.block_size
        self.k[layer, blocks, offsets] = key
        self.v[layer, blocks, offsets] = value

    def write(self, layer: int, block_table, start: int, key, value) -> None:
        key = np.asarray(key)
        if key.ndim != 3:
            raise ValueError("key/value must have the same [T, H, D] shape")
        slots = self.slot_mapping(block_table, start, key.shape[0])
        self.write_slots(layer, slots, key, value, validate_slots=False)

    def read(self, layer: int, block_table, length: int):
        """First ``length`` logical tokens in order, as storage arrays."""
        if length < 0:
            raise ValueError("length must be non-negative")
        slots = self.slot_mapping(block_table, 0, length)
        if not 0 <= layer < self.num_layers:
            raise IndexError("layer is out of range")
        blocks = slots // self.block_size
        offsets = slots % self.block_size
        return self.k[layer, blocks, offsets], self.v[layer, blocks, offsets]


# ---------------------------------------------------------------- attention
def expand_kv(x: np.ndarray, num_heads: int) -> np.ndarray:
    """[T, Hkv, D] -> [T, H, D]; query head h reads kv head h // (H // Hkv)."""
    if x.shape[1] == num_heads:
        return x
    if num_heads % x.shape[1] != 0:
        raise ValueError("num_heads must be divisible by num_kv_heads")
    return np.repeat(x, num_heads // x.shape[1], axis=1)


def dense_decode_attention(query: np.ndarray, key: np.ndarray, value: np.ndarray, *,
                           scale: float | None = None) -> np.ndarray:
    """fp32 softmax(q.k * scale) @ v for q [B,H,D], k/v [T,Hkv,D] -> [B,H,D] fp32."""
    if query.ndim != 3 or key.ndim != 3 or value.ndim != 3:
        raise ValueError("query must be [B,H,D], key/value must be [T,Hkv,D]")
    if key.shape != value.shape or query.shape[2] != key.shape[2]:
        raise ValueError("incompatible attention shapes")
    q = np.asarray(query, dtype=np.float32)
    k = expand_kv(np.asarray(key, dtype=np.float32), q.shape[1]).transpose(1, 0, 2)  # [H,T,D]
    v = expand_kv(np.asarray(value, dtype=np.float32), q.shape[1]).transpose(1, 0, 2)
    scores = np.einsum("bhd,htd->bht", q, k, optimize=True).astype(np.float32)
    scores *= np.float32(scale if scale is not None else q.shape[-1] ** -0.5)
    scores -= scores.max(axis=-1, keepdims=True)
    probs = np.exp(scores, dtype=np.float32)
    probs /= probs.sum(axis=-1, keepdims=True)
    return np.einsum("bht,htd->bhd", probs, v, optimize=True).astype(np.float32)


def paged_decode_attention(query_f32: np.ndarray, cache: OracleCache, block_tables,
                           context_lens, *, scale: float | None = None,
                           layer: int = 0) -> np.ndarray:
    """Per-request loop: gather the first ctx tokens through the block table,
    then dense fp32 attention (attention.py:134-175). Returns fp32 [B,H,D]."""
    query_f32 = np.asarray(query_f32, dtype=np.float32)
    if query_f32.ndim != 3:
        raise ValueError("query must be [B,H,D]")
    batch, num_heads, head_dim = query_f32.shape
    if head_dim != cache.head_dim:
        raise ValueError("query head_dim does not match cache")
    if num_heads % cache.num_kv_heads != 0:
        raise ValueError("num_heads must be divisible by num_kv_heads")
    lengths = [int(x) for x in np.asarray(context_lens).reshape(-1)]
    tables = [list(map(int, row)) for row in block_tables]
    if len(lengths) != batch:
        raise ValueError("context_lens must have one entry per query")
    if len(tables) != batch:
        raise ValueError("block_tables must have one row per query")
    outputs = np.empty((batch, num_heads, head_dim), dtype=np.float32)
    for index, length in enumerate(lengths):
        if length <= 0:
            raise ValueError("context lengths must be positive")
        k_raw, v_raw = cache.read(layer, tables[index], length)
        k = to_f32(k_raw, cache.dtype)
        v = to_f32(v_raw, cache.dtype)
        outputs[index] = dense_decode_attention(query_f32[index:index + 1], k, v, scale=scale)[0]
    return outputs


def brute_force_attention_f64(query, keys, values, *, scale=None):
    """Pure-Python float64 attention for tiny inputs: q [H][D], keys/values
    [T][Hkv][D] nested lists; returns [H][D]. Independent of numpy."""
    num_heads = len(query)
    num_kv = len(keys[0])
    group = num_heads // num_kv
    head_dim = len(query[0])
    s = scale if scale is not None else head_dim ** -0.5
    out = []
    for h in range(num_heads):
        kvh = h // group
        scores = [s * sum(query[h][d] * keys[t][kvh][d] for d in range(head_dim)) for t in range(len(keys))]
        mx = max(scores)
        weights = [math.exp(x - mx) for x in scores]
        z = sum(weights)
        out.append([sum(weights[t] * values[t][kvh][d] for t in range(len(keys))) / z
                    for d in range(head_dim)])
    return out


def causal_allow(positions: np.ndarray, num_keys: int) -> np.ndarray:
    """[n, num_keys] mask: the row at position p may attend keys 0..p
    (attention.py:301-303)."""
    return np.arange(num_keys)[None, :] <= np.asarray(positions)[:, None]


def paged_prefill_attention(query_f32: np.ndarray, cache: OracleCache, block_tables, query_starts,
                            context_lens, *, scale: float | None = None, layer: int = 0) -> np.ndarray:
    """Causal attention of a ragged prompt-chunk batch (attention.py:230-321).

    ``query_f32`` is [B, H, T, D]; row t of request b sits at position
    starts[b] + t. Rows t < ends[b] - starts[b] attend positions
    [0, starts[b] + t] in fp32; the remaining (padding) rows are allowed only
    position 0 by the reference's mask (attention.py:305), so they equal the
    value there. Returns fp32 [B, H, T, D].
    """
    q = np.asarray(query_f32, dtype=np.float32)
    if q.ndim != 4:
        raise ValueError("query must be [B,H,T,D]")
    batch, num_heads, width, head_dim = q.shape
    if head_dim != cache.head_dim:
        raise ValueError("query head_dim does not match cache")
    if num_heads % cache.num_kv_heads != 0:
        raise ValueError("num_heads must be divisible by num_kv_heads")
    starts = [int(x) for x in np.asarray(query_starts).reshape(-1)]
    ends = [int(x) for x in np.asarray(context_lens).reshape(-1)]
    tables = [list(map(int, row)) for row in block_tables]
    if len(starts) != batch or len(ends) != batch:
        raise ValueError("query_starts and context_lens must have one entry per query batch")
    spans = [e - s for s, e in zip(starts, ends)]
    if any(s < 0 or n <= 0 for s, n in zip(starts, spans)):
        raise ValueError("prefill ranges must be non-empty and non-negative")
    if max(spans) > width:
        raise ValueError("query width is smaller than a prefill range")
    sc = np.float32(scale if scale is not None else head_dim ** -0.5)
    out = np.empty(q.shape, dtype=np.float32)
    for b in range(batch):
        k_raw, v_raw = cache.read(layer, tables[b], ends[b])
        k = expand_kv(to_f32(k_raw, cache.dtype), num_heads).transpose(1, 0, 2)  # [H, L, D]
        v = expand_kv(to_f32(v_raw, cache.dtype), num_heads).transpose(1, 0, 2)
        n = spans[b]
        scores = np.matmul(q[b, :, :n], k.transpose(0, 2, 1)) * sc  # [H, n, L]
        allow = causal_allow(starts[b] + np.arange(n), ends[b])  # [n, L]
        scores = np.where(allow[None], scores, -np.inf).astype(np.float32)
        scores -= scores.max(axis=-1, keepdims=True)
        probs = np.exp(scores, dtype=np.float32)
        probs /= probs.sum(axis=-1, keepdims=True)
        out[b, :, :n] = np.matmul(probs, v)
        out[b, :, n:] = v[:, :1, :]  # padding rows: position 0
    return out


def brute_force_prefill_f64(query, keys, values, start: int, *, scale=None):
    """Pure-Python float64 causal attention for tiny inputs: query [H][n][D]
    (row t at position start + t), keys/values [L][Hkv][D]; returns [H][n][D]."""
    out = []
    for h in range(len(query)):
        rows = []
        for t, qrow in enumerate(query[h]):
            pos = start + t
            rows.append(brute_force_attention_f64([qrow], [[kv[h * len(keys[0]) // len(query)]]
                                                           for kv in keys[: pos + 1]],
                                                  [[vv[h * len(values[0]) // len(query)]]
                                                   for vv in values[: pos + 1]], scale=scale)[0])
        out.append(rows)
    return out


# ------------------------------------------------------------- FP8 KV format
E4M3_MAX = 448.0


def e4m3_decode(codes: np.ndarray) -> np.ndarray:
    """OCP E4M3 (e4m3fn) codes -> float32: sign, 4 exponent bits (bias 7), 3
    mantissa bits; exponent 0 is subnormal (m * 2^-9); 0x7f / 0xff are NaN."""
    c = np.asarray(codes, dtype=np.uint8).astype(np.int32)
    sign = np.where(c & 0x80, -1.0, 1.0)
    e = (c >> 3) & 0xF
    m = c & 0x7
    mag = np.where(e == 0, m * 2.0 ** -9, (1.0 + m / 8.0) * 2.0 ** (e - 7))
    out = (sign * mag).astype(np.float32)
    out[(c & 0x7F) == 0x7F] = np.nan
    return out


_E4M3_POS = e4m3_decode(np.arange(0x7F, dtype=np.uint8)).astype(np.float64)  # codes 0..0x7e, ascending


def e4m3_encode(x: np.ndarray) -> np.ndarray:
    """float32 -> OCP E4M3 codes, round to nearest (ties to the even code),
    magnitudes above 448 saturated to 448 (code 0x7e); NaN -> 0x7f."""
    x = np.asarray(x, dtype=np.float32)
    a = np.minimum(np.abs(x).astype(np.float64), E4M3_MAX)
    hi = np.clip(np.searchsorted(_E4M3_POS, a, side="left"), 0, 0x7E)
    lo = np.clip(hi - 1, 0, 0x7E)
    d_lo, d_hi = a - _E4M3_POS[lo], _E4M3_POS[hi] - a
    pick_hi = (d_hi < d_lo) | ((d_hi == d_lo) & (hi % 2 == 0))
    code = np.where(pick_hi, hi, lo).astype(np.uint8)
    code = np.where(np.signbit(x), code | 0x80, code).astype(np.uint8)
    return np.where(np.isnan(x), np.uint8(0x7F), code).astype(np.uint8)


def pow2_scale(amax: np.ndarray) -> np.ndarray:
    """Power-of-two scale of rows with maximum magnitude amax:
    2^ceil(log2(t)) for t = amax / 448 (one correctly rounded fp32 division),
    read off t's bits (at least 2^-126); 1 for amax == 0 or non-finite."""
    amax = np.asarray(amax, dtype=np.float32)
    ok = (amax > 0) & np.isfinite(amax)
    t = np.where(ok, amax, np.float32(448)).astype(np.float32) / np.float32(E4M3_MAX)
    bits = t.astype(np.float32).view(np.int32)
    e = ((bits >> 23) & 0xFF) - 127 + ((bits & 0x7FFFFF) != 0)
    e = np.clip(e, -126, 127)
    scale = ((e + 127).astype(np.int32) << 23).view(np.float32)
    return np.where(ok, scale, np.float32(1.0)).astype(np.float32)


def quantize_rows_e4m3(rows: np.ndarray) -> tuple[np.ndarray, np.ndarray]:
    """[..., D] float rows -> (codes [..., D] uint8, scale [...] float32):
    scale = pow2_scale(max |x| over the row), codes = e4m3(x / scale), an
    exact scaling (a power of two) followed by one rounding."""
    x = np.asarray(rows, dtype=np.float32)
    scale = pow2_scale(np.abs(x).max(axis=-1))
    y = np.clip(x / scale[..., None], -E4M3_MAX, E4M3_MAX).astype(np.float32)
    return e4m3_encode(y), scale


def dequantize_rows_e4m3(codes: np.ndarray, scale: np.ndarray) -> np.ndarray:
    return (e4m3_decode(codes) * np.asarray(scale, np.float32)[..., None]).astype(np.float32)
