"""Pins of the fp8 oracle (CPU).

  * e4m3fn decode table vs torch.float8_e4m3fn (a library implementation of the OCP format), all
    256 codes;
  * encode vs torch's float -> float8_e4m3fn conversion on every tie between adjacent values,
    values just either side of each tie, subnormals, the clamp boundary and random inputs; and vs
    a brute-force nearest-value search written independently;
  * 128 x 128 block quantisation: the product's weight intake (tt_symbiote_amd.hip_ops
    .quantize_block_fp8, torch) produces the oracle's bytes and scales; dequant(quant(w)) is
    within half a unit in the last place of w; exactly representable blocks round-trip;
  * KV block append: scale = the power of two at or above amax / 448 of everything appended so
    far, old codes untouched when the scale does not grow, each new value within half a unit in
    the last place, and token-by-token appends (with their requantisations) equal the one-shot
    encoding on every value that stays normal.
"""
import numpy as np
import pytest
import torch

from oracle.fp8 import (E4M3_VALUES, FP8_MAX, decode_e4m3, dequant_blocks, encode_e4m3,
                        kv_block_append, kv_dequant, pow2_ceil, quantize_blocks)


def _torch_encode(x: np.ndarray) -> np.ndarray:
    t = torch.from_numpy(np.asarray(x, np.float32)).to(torch.float8_e4m3fn)
    return t.view(torch.uint8).numpy()


def test_decode_table_matches_torch():
    codes = torch.arange(256, dtype=torch.int32).to(torch.uint8)
    ref = codes.view(torch.float8_e4m3fn).float().numpy()
    nan = np.isnan(ref)
    assert np.array_equal(nan, np.isnan(E4M3_VALUES))
    assert set(np.nonzero(nan)[0].tolist()) == {0x7F, 0xFF}
    assert np.array_equal(ref[~nan], E4M3_VALUES[~nan])
    assert E4M3_VALUES[0x7E] == 448.0 and E4M3_VALUES[0x01] == 2.0 ** -9


def _tie_points():
    pos = E4M3_VALUES[:127].astype(np.float64)
    mids = (pos[:-1] + pos[1:]) / 2
    eps = np.abs(mids) * 2.0 ** -20 + 1e-12
    pts = np.concatenate([mids, mids - eps, mids + eps, pos])
    return np.concatenate([pts, -pts]).astype(np.float32)


def test_encode_matches_torch_on_ties_and_neighbours():
    x = _tie_points()
    assert np.array_equal(encode_e4m3(x), _torch_encode(x))


def test_encode_matches_torch_random_and_clamped():
    rng = np.random.default_rng(0)
    x = np.concatenate([
        rng.standard_normal(20000) * s for s in (1e-3, 0.02, 1.0, 30.0, 300.0)
    ]).astype(np.float32)
    xc = np.clip(x, -448.0, 448.0)
    assert np.array_equal(encode_e4m3(xc), _torch_encode(xc))
    # clamping: anything beyond 448 in magnitude encodes as +-448
    big = np.array([448.0, 449.0, 470.0, 1e6, -500.0], np.float32)
    assert decode_e4m3(encode_e4m3(big)).tolist() == [448.0, 448.0, 448.0, 448.0, -448.0]


def test_encode_matches_brute_force():
    rng = np.random.default_rng(1)
    x = np.concatenate([rng.uniform(-448, 448, 3000), rng.uniform(-0.02, 0.02, 3000),
                        _tie_points()[::7]]).astype(np.float32)
    finite = [(c, float(E4M3_VALUES[c])) for c in range(256) if not np.isnan(E4M3_VALUES[c])]
    got = encode_e4m3(x)
    for xi, ci in zip(x.tolist(), got.tolist()):
        best = None
        for c, v in finite:
            if (v < 0) != (np.signbit(np.float32(xi))) and v != 0.0:
                continue
            d = abs(xi - v)
            if best is None or d < best[0] - 0.0 or (d == best[0] and (c & 1) == 0 and
                                                     (best[1] & 1) == 1):
                best = (d, c)
        assert float(decode_e4m3(np.uint8(ci))) == float(E4M3_VALUES[best[1]]), (xi, ci, best)


def test_block_quant_roundtrip_bound_and_exact_blocks():
    rng = np.random.default_rng(2)
    w = (rng.standard_normal((2, 256, 384)) * 0.02).astype(np.float32)
    w[0, :128, :128] = 0.0                                    # all-zero block -> scale 1
    q, s = quantize_blocks(w)
    assert q.shape == w.shape and s.shape == (2, 2, 3)
    assert s[0, 0, 0] == 1.0
    d = dequant_blocks(q, s)
    # |err| <= half an ulp of the fp8 grid at the value's binade (2^-4 relative for normals,
    # half the subnormal step scale * 2^-10 absolute)
    sb = np.repeat(np.repeat(s, 128, axis=-2), 128, axis=-1)
    bound = np.maximum(np.abs(w) * 2.0 ** -4, sb * 2.0 ** -10) * 1.0001
    assert np.all(np.abs(d - w) <= bound)
    # a block of exactly representable values (times a power of two) is reproduced exactly
    codes = rng.integers(0, 0x7E, size=(128, 128)).astype(np.uint8)
    codes[0, 0] = 0x7E                                        # amax = 448 -> scale = 2^-3
    exact = decode_e4m3(codes) * np.float32(2.0 ** -3)
    q2, s2 = quantize_blocks(exact)
    assert s2.item() == 2.0 ** -3
    assert np.array_equal(dequant_blocks(q2, s2), exact)


def test_product_weight_intake_matches_oracle():
    from tt_symbiote_amd.hip_ops import quantize_block_fp8

    g = torch.Generator().manual_seed(3)
    w = torch.randn(3, 256, 512, generator=g) * 0.05
    w[1, 128:, :128] = 0.0
    qt = quantize_block_fp8(w.to(torch.bfloat16))
    q, s = quantize_blocks(w.to(torch.bfloat16).float().numpy())
    assert np.array_equal(qt.scale.numpy(), s)
    assert np.array_equal(qt.q.view(torch.uint8).numpy(), q)


def _ulp(v):
    """Spacing of the fp8 grid at |v| (subnormal spacing below 2^-6)."""
    a = np.maximum(np.abs(v), 2.0 ** -6)
    return 2.0 ** (np.floor(np.log2(a)) - 3)


def test_pow2_ceil():
    assert pow2_ceil(0.0) == 0.0
    assert pow2_ceil(1.0) == 1.0 and pow2_ceil(1.0000001) == 2.0 and pow2_ceil(0.75) == 1.0
    assert pow2_ceil(2.0 ** -130) == 2.0 ** -126
    rng = np.random.default_rng(6)
    for y in (rng.uniform(0, 1, 500) * 10.0 ** rng.integers(-30, 30, 500)).astype(np.float32):
        p = pow2_ceil(y)
        assert p >= y and p / 2 < y and np.log2(p) == np.round(np.log2(p))


def test_kv_append_scale_rule_and_bounds():
    rng = np.random.default_rng(4)
    bs, D = 32, 128
    codes = rng.integers(0, 255, size=(bs, D)).astype(np.uint8)   # stale bytes of a reused block
    toks = rng.standard_normal((bs, D)).astype(np.float32)
    toks[5] *= 4.0                                                # a token that grows the scale
    toks[20] *= 40.0
    s = np.float32(123.0)                                         # stale scale, ignored (n_old=0)
    grew = 0
    for t in range(bs):
        prev_codes, prev_s = codes.copy(), s
        codes, s = kv_block_append(codes, s, t, toks[t:t + 1])
        amax = np.abs(toks[:t + 1]).max()
        assert s == pow2_ceil(np.float32(np.float32(amax) / FP8_MAX))
        if t > 0 and s == prev_s:
            assert np.array_equal(codes[:t], prev_codes[:t])
        grew += int(t > 0 and s > prev_s)
        # the new token: within half an ulp (in units of the scale)
        err_new = np.abs(kv_dequant(codes[t], s) - toks[t])
        assert np.all(err_new <= 0.5 * _ulp(toks[t] / s) * s * 1.0001)
    assert grew >= 2
    # requantisation by a power of two is exact except where a value becomes subnormal:
    # token-by-token equals one-shot encode(x / s) on every value that is normal at the end
    c1, s1 = kv_block_append(np.zeros((bs, D), np.uint8), 0.0, 0, toks)
    assert s1 == s
    assert np.array_equal(c1, encode_e4m3((toks / s1).astype(np.float32)))
    normal = np.abs(toks / s) >= 2.0 ** -6
    assert np.array_equal(codes[normal], c1[normal])
    sub = ~normal
    assert np.all(np.abs(kv_dequant(codes[sub], s) - kv_dequant(c1[sub], s)) <= 2.0 ** -9 * s)


def test_kv_append_zero_block_and_partial_start():
    bs, D = 16, 128
    z = np.zeros((3, D), np.float32)
    c, s = kv_block_append(np.full((bs, D), 0x55, np.uint8), 7.0, 0, z)
    assert s == 0.0 and np.all(c[:3] == 0) and np.all(c[3:] == 0x55)
    # appending into a block that already has rows keeps their scale when it suffices
    rng = np.random.default_rng(5)
    first = rng.standard_normal((4, D)).astype(np.float32)
    c, s = kv_block_append(np.zeros((bs, D), np.uint8), 0.0, 0, first)
    small = first[:2] * 0.5
    c2, s2 = kv_block_append(c, s, 4, small)
    assert s2 == s and np.array_equal(c2[:4], c[:4])
    assert np.array_equal(c2[4:6], encode_e4m3((small / s).astype(np.float32)))
