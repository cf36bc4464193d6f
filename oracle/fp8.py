"""Oracle of the fp8 formats (test infrastructure only: imported by tests, the smoke check and the
CPU baseline, never by the product path).

Formats restated here:
  * OCP 8-bit floating point, E4M3 "fn" variant (OCP OFP8 specification v1.0, section 5.3):
    1 sign bit, 4 exponent bits with bias 7, 3 mantissa bits; exponent 0 is subnormal
    (m / 8 * 2^-6); no infinities; 0x7f and 0xff are NaN; largest finite value 448.
    Encoding rounds to nearest, ties to even, after clamping to [-448, 448].
  * Expert weights with one fp32 scale per 128 x 128 block (w = value(q) * scale), the
    "fp8 e4m3 with block scales" weight format of the quantized Ling-mini-2.0 experts that
    TTNNExperts.from_torch (ttnn_moe.py:1055-1078) would take in place of bf16.
  * A paged KV cache in e4m3fn with one fp32 scale per (block, kv head) (pools laid out as
    TTNNPagedAttentionKVCache, ttnn_attention.py:116-137). The reference keeps its cache in
    bf16, so the scale rule is this library's (power-of-two scales that grow as a block fills);
    it is stated by `kv_block_append`.

Every function works on numpy arrays with float32 arithmetic in a fixed order, so a kernel that
does the same float32 operations produces the same bytes.
"""
from __future__ import annotations

import numpy as np

FP8_MAX = np.float32(448.0)
BLOCK = 128


def _decode_table() -> np.ndarray:
    """Value of each of the 256 e4m3fn codes (NaN for 0x7f, 0xff), from the format's definition."""
    vals = np.empty(256, dtype=np.float32)
    for code in range(256):
        s = -1.0 if code & 0x80 else 1.0
        e = (code >> 3) & 0xF
        m = code & 0x7
        if e == 0xF and m == 0x7:
            vals[code] = np.nan
        elif e == 0:
            vals[code] = s * (m / 8.0) * 2.0 ** -6
        else:
            vals[code] = s * (1.0 + m / 8.0) * 2.0 ** (e - 7)
    return vals


E4M3_VALUES = _decode_table()
# the 127 finite non-negative values in code order (codes 0x00 .. 0x7e), increasing
_POS = E4M3_VALUES[:127].astype(np.float64)


def decode_e4m3(codes: np.ndarray) -> np.ndarray:
    """e4m3fn bytes -> float32 values (exact)."""
    return E4M3_VALUES[np.asarray(codes, dtype=np.uint8)]


def encode_e4m3(x: np.ndarray) -> np.ndarray:
    """float32 -> e4m3fn bytes: clamp to [-448, 448], then round to nearest, ties to the even
    code (consecutive codes are one unit in the last place apart, so "even code" is "even
    mantissa"). -0.0 and negative values that round to zero keep the sign bit (0x80)."""
    x = np.asarray(x, dtype=np.float32)
    a = np.minimum(np.abs(x).astype(np.float64), float(FP8_MAX))
    hi = np.searchsorted(_POS, a, side="left")          # first value >= a
    hi = np.minimum(hi, 126)
    lo = np.maximum(hi - 1, 0)
    d_lo = a - _POS[lo]
    d_hi = _POS[hi] - a
    pick_hi = (d_hi < d_lo) | ((d_hi == d_lo) & (hi % 2 == 0))
    code = np.where(pick_hi, hi, lo).astype(np.uint8)
    code = np.where(a == _POS[hi], hi, code).astype(np.uint8)
    neg = np.signbit(x)
    return (code | np.where(neg, 0x80, 0).astype(np.uint8)).astype(np.uint8)


def dequant_blocks(q: np.ndarray, scale: np.ndarray) -> np.ndarray:
    """[..., N, K] e4m3fn bytes and [..., N/128, K/128] fp32 scales -> float32 weights
    w[n, k] = value(q[n, k]) * scale[n // 128, k // 128] (one float32 product per element)."""
    vals = decode_e4m3(q)
    s = np.repeat(np.repeat(np.asarray(scale, np.float32), BLOCK, axis=-2), BLOCK, axis=-1)
    return (vals * s).astype(np.float32)


def quantize_blocks(w: np.ndarray):
    """Per 128 x 128 block: scale = amax / 448 (1 for an all-zero block), q = e4m3(w / scale)."""
    w = np.asarray(w, dtype=np.float32)
    *lead, n, k = w.shape
    wb = w.reshape(*lead, n // BLOCK, BLOCK, k // BLOCK, BLOCK)
    amax = np.abs(wb).max(axis=(-3, -1))
    scale = np.where(amax > 0, (amax / FP8_MAX).astype(np.float32), np.float32(1.0))
    scale = scale.astype(np.float32)
    q = encode_e4m3(wb / scale[..., :, None, :, None])
    return q.reshape(*lead, n, k), scale


def pow2_ceil(y) -> np.float32:
    """Smallest power of two >= y for float32 y > 0 (2^-126 for y below that; 0 for y == 0),
    by exponent arithmetic on the float32 bits."""
    y = np.float32(y)
    if y == 0:
        return np.float32(0.0)
    if y < np.float32(2.0 ** -126):
        return np.float32(2.0 ** -126)
    bits = np.array([y], np.float32).view(np.uint32)[0]
    if bits & 0x7FFFFF == 0:
        return y
    return np.array([(bits & 0x7F800000) + 0x00800000], np.uint32).view(np.float32)[0]


def kv_block_append(codes: np.ndarray, scale: float, n_old: int, new: np.ndarray):
    """Append tokens to one (block, kv head) of an fp8 KV pool.

    codes [block_size, D] uint8 holds the block; its first n_old rows are valid and `scale`
    is their scale (ignored when n_old == 0). new [n, D] float32 are the next n tokens (the
    bf16 values the bf16 cache would hold). Rule:
      s_new = max(s_old, pow2_ceil(amax(new) / 448))      (s_old = 0 for an empty block)
      if n_old > 0 and s_new > s_old: every old code c becomes e4m3(value(c) * (s_old / s_new))
      new codes = e4m3(x / s_new)  (0 when s_new == 0)
    Scales are powers of two, so they only grow while a block fills, requantising an old code
    is an exact exponent shift (rounding only where it becomes subnormal), dividing by the scale
    is exact, and no value is clamped. Returns (codes, s_new); rows n_old .. n_old+n-1 are
    written.
    """
    codes = np.array(codes, dtype=np.uint8, copy=True)
    new = np.asarray(new, dtype=np.float32)
    n = new.shape[0]
    s_old = np.float32(scale) if n_old > 0 else np.float32(0.0)
    amax = np.float32(np.abs(new).max()) if n > 0 else np.float32(0.0)
    s_new = np.maximum(s_old, pow2_ceil(np.float32(amax / FP8_MAX)))
    if n_old > 0 and s_new > s_old:
        r = np.float32(s_old / s_new)
        codes[:n_old] = encode_e4m3((decode_e4m3(codes[:n_old]) * r).astype(np.float32))
    if s_new > 0:
        codes[n_old:n_old + n] = encode_e4m3((new / s_new).astype(np.float32))
    else:
        codes[n_old:n_old + n] = 0
    return codes, np.float32(s_new)


def kv_dequant(codes: np.ndarray, scale) -> np.ndarray:
    """Values of a block (or a stack of blocks with per-block scales broadcast)."""
    return (decode_e4m3(codes) * np.asarray(scale, np.float32)).astype(np.float32)
