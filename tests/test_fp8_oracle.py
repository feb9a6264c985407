"""Pins of the oracle's FP8 KV format (E4M3 codes, one fp32 scale per
(token, KV head) row) and of the package's torch quantiser.

e4m3_encode / e4m3_decode are checked bit for bit against torch's own
float8_e4m3fn conversion (values, ties, subnormals, signed zeros, both
ends of the range, all 256 codes); quantize_rows_e4m3 by its closed forms.
A planted rounding mistake (ties away from zero) must be caught."""

import numpy as np
import pytest
import torch

from oracle import paged_oracle as po


def _torch_codes(x: np.ndarray) -> np.ndarray:
    return torch.from_numpy(np.ascontiguousarray(x, dtype=np.float32)).to(torch.float8_e4m3fn).view(torch.uint8).numpy()


def _probe_values(seed=0):
    rng = np.random.default_rng(seed)
    pos = po.e4m3_decode(np.arange(0x7F, dtype=np.uint8)).astype(np.float64)
    mids = ((pos[:-1] + pos[1:]) / 2).astype(np.float32)  # every tie
    edges = np.array([0.0, -0.0, 448.0, -448.0, 2.0**-9, -(2.0**-9), 2.0**-10, 1.5 * 2.0**-9, 2.0**-6,
                      0.5 * 2.0**-6], dtype=np.float32)
    return np.concatenate([rng.standard_normal(50000).astype(np.float32) * np.float32(40),
                           rng.uniform(-448, 448, 50000).astype(np.float32),
                           (rng.standard_normal(20000) * 1e-3).astype(np.float32), mids, -mids, edges])


def test_e4m3_encode_matches_torch_bit_for_bit():
    x = _probe_values()
    assert np.array_equal(po.e4m3_encode(x), _torch_codes(x))


def test_e4m3_decode_matches_torch_for_all_codes():
    codes = np.arange(256, dtype=np.uint8)
    ref = torch.from_numpy(codes).view(torch.float8_e4m3fn).float().numpy()
    assert np.array_equal(po.e4m3_decode(codes), ref, equal_nan=True)
    assert po.e4m3_decode(np.array([0x7E], np.uint8))[0] == 448.0
    assert np.isnan(po.e4m3_decode(np.array([0x7F, 0xFF], np.uint8))).all()


def test_e4m3_round_trip_of_every_code():
    codes = np.array([c for c in range(256) if c & 0x7F != 0x7F], dtype=np.uint8)
    assert np.array_equal(po.e4m3_encode(po.e4m3_decode(codes)), codes)


def test_e4m3_saturates_past_448():
    x = np.array([449.0, 1e6, -500.0], np.float32)
    assert po.e4m3_encode(x).tolist() == [0x7E, 0x7E, 0xFE]


def test_quantize_rows_closed_forms():
    rng = np.random.default_rng(1)
    rows = rng.standard_normal((64, 8, 128)).astype(np.float32) * 3
    rows[0, 0] = 0.0
    codes, scale = po.quantize_rows_e4m3(rows)
    amax = np.abs(rows).max(-1)
    assert scale[0, 0] == 1.0 and not codes[0, 0].any()
    nz = amax > 0
    # scales are powers of two: the smallest with amax / scale <= 448
    mant, _ = np.frexp(scale[nz])
    assert (mant == 0.5).all()
    ratio = amax[nz].astype(np.float64) / scale[nz]
    assert (ratio <= 448).all() and (ratio > 224).all()
    # scaling by a power of two is exact: the codes are those of x / scale
    assert np.array_equal(codes, po.e4m3_encode(np.clip(rows / scale[..., None], -448, 448)))
    # dequantised values within half an E4M3 step (relative 2^-4) of the input, plus the subnormal floor
    back = po.dequantize_rows_e4m3(codes, scale)
    assert (np.abs(back - rows) <= np.abs(rows) * 2.0**-4 + scale[..., None] * 2.0**-10 + 1e-12).all()


@pytest.mark.parametrize("seed", [25, 0, 1, 2])
def test_torch_quantiser_matches_the_oracle(seed):
    """Random rows over several magnitudes; seed 25 is the case that once
    separated a reciprocal-then-multiply from a correctly rounded division."""
    from inferkernellab_amd.cache import quantize_rows_e4m3

    torch.manual_seed(seed)
    x = torch.randn(300, 4, 96) * 5
    x[3, 1] = 0
    codes, scale = quantize_rows_e4m3(x)
    oc, os_ = po.quantize_rows_e4m3(x.numpy())
    assert np.array_equal(codes.view(torch.uint8).numpy(), oc)
    assert np.array_equal(scale.numpy(), os_)


def test_fp8_cache_torch_write_read_round_trip():
    from inferkernellab_amd import PagedKVCache

    cache = PagedKVCache(12, 16, 2, 64, dtype=torch.float8_e4m3fn)
    assert cache.fp8 and cache.act_dtype == torch.bfloat16 and cache.k_scale.shape == (1, 12, 2, 16)
    table = cache.allocate_request(0, 40)
    k = torch.randn(40, 2, 64)
    v = torch.randn(40, 2, 64)
    cache.write(0, table, 0, k, v)
    kr, vr = cache.read(0, table, 40)
    codes, scale = po.quantize_rows_e4m3(k.numpy())
    assert np.array_equal(kr.numpy(), po.dequantize_rows_e4m3(codes, scale))
    codes, scale = po.quantize_rows_e4m3(v.numpy())
    assert np.array_equal(vr.numpy(), po.dequantize_rows_e4m3(codes, scale))


def test_planted_rounding_mistake_is_caught(monkeypatch):
    """Ties rounded away from zero instead of to the even code fail the
    torch pin."""
    real = po.e4m3_encode

    def away(x):
        x = np.asarray(x, np.float32)
        a = np.minimum(np.abs(x).astype(np.float64), 448.0)
        pos = po._E4M3_POS
        hi = np.clip(np.searchsorted(pos, a, side="left"), 0, 0x7E)
        lo = np.clip(hi - 1, 0, 0x7E)
        code = np.where(pos[hi] - a <= a - pos[lo], hi, lo).astype(np.uint8)
        return np.where(np.signbit(x), code | 0x80, code).astype(np.uint8)

    monkeypatch.setattr(po, "e4m3_encode", away)
    x = _probe_values(3)
    assert not np.array_equal(po.e4m3_encode(x), _torch_codes(x))
    monkeypatch.setattr(po, "e4m3_encode", real)
    assert np.array_equal(po.e4m3_encode(x), _torch_codes(x))


@pytest.mark.parametrize("act", [torch.float16, torch.bfloat16])
def test_fp8_cache_checks(act):
    from inferkernellab_amd import PagedKVCache

    cache = PagedKVCache(4, 16, 1, 32, dtype=torch.float8_e4m3fn, act_dtype=act)
    assert cache.act_dtype == act and cache.numel_bytes == 2 * 4 * 16 * 32 + 2 * 4 * 16 * 4
    with pytest.raises(ValueError, match="act_dtype"):
        PagedKVCache(4, 16, 1, 32, dtype=torch.float16, act_dtype=torch.bfloat16)
