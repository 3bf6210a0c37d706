"""Pins the oracle's scalar formats and MXFP8/MXFP4 arithmetic against
independent definitions: OCP MX tables, torch's float8_e4m3fn / bfloat16
conversions, and brute-force restatements in numpy. A plausible oracle mistake
(nibble order, bias, rounding direction, scale exponent off by one) fails one
of these."""
import math

import numpy as np
import pytest
import torch

import oracle as O


def test_e2m1_table():
    # OCP MX v1.0: E2M1 = 1 sign, 2 exponent bits (bias 1), 1 mantissa bit.
    for code in range(16):
        s, e, m = code >> 3, (code >> 1) & 3, code & 1
        v = (m * 0.5) if e == 0 else (1 + m * 0.5) * 2.0 ** (e - 1)
        assert O.lib().oracle_e2m1(code) == (-v if s else v)


def test_e8m0_all_codes():
    for e in range(256):
        v = O.lib().oracle_e8m0(e)
        if e == 255:
            assert math.isnan(v)
        else:
            assert v == 2.0 ** (e - 127)  # e == 0 -> 2^-127, an fp32 subnormal


def test_e4m3_decode_matches_torch():
    codes = torch.arange(256, dtype=torch.uint8)
    ref = codes.view(torch.float8_e4m3fn).float().numpy()
    got = np.array([O.lib().oracle_e4m3(c) for c in range(256)], np.float32)
    both_nan = np.isnan(ref) & np.isnan(got)
    assert np.all(both_nan | (ref == got))


def test_e4m3_encode_matches_torch_all_bf16_in_range():
    bits = np.arange(65536, dtype=np.uint32)
    vals = (bits << 16).view(np.float32)
    vals = vals[np.isfinite(vals) & (np.abs(vals) <= 448.0)]
    ref = torch.from_numpy(vals).to(torch.float8_e4m3fn).view(torch.uint8).numpy()
    got = np.array([O.lib().oracle_e4m3_from_f32(float(v)) for v in vals], np.uint8)
    assert np.array_equal(ref, got)


def test_e4m3_encode_random_fp32_and_saturation():
    rng = np.random.default_rng(7)
    vals = (rng.standard_normal(20000) * rng.choice([1e-4, 1e-2, 1, 30, 300], 20000)).astype(np.float32)
    vals = np.clip(vals, -448, 448)
    ref = torch.from_numpy(vals).to(torch.float8_e4m3fn).view(torch.uint8).numpy()
    got = np.array([O.lib().oracle_e4m3_from_f32(float(v)) for v in vals], np.uint8)
    assert np.array_equal(ref, got)
    # satfinite: beyond 448 saturates (torch's conversion would give NaN there)
    assert O.lib().oracle_e4m3_from_f32(460.0) == 0x7E
    assert O.lib().oracle_e4m3_from_f32(-1e9) == 0xFE
    assert O.lib().oracle_e4m3_from_f32(float("inf")) == 0x7E
    assert O.lib().oracle_e4m3_from_f32(-0.0) == 0x80


def test_bf16_rounding_matches_torch():
    rng = np.random.default_rng(3)
    vals = np.concatenate([rng.standard_normal(5000).astype(np.float32),
                           (rng.integers(0, 2**32, 5000, dtype=np.uint64).astype(np.uint32)).view(np.float32)])
    vals = vals[np.isfinite(vals)]
    ref = torch.from_numpy(vals).to(torch.bfloat16).view(torch.int16).numpy().view(np.uint16)
    assert np.array_equal(O.bf16_bits(vals), ref)


def test_dequant_exhaustive_codes_and_scales():
    # every nibble code at both nibble positions x every scale byte
    n, k = 256, 32
    w = np.zeros((n, k // 2), np.uint8)
    for c in range(16):
        w[:, c] = c | (((c + 5) % 16) << 4)
    s = np.arange(256, dtype=np.uint8).reshape(n, 1)
    out = O.dequant_mxfp4(w, s, n, k)
    table = [0, .5, 1, 1.5, 2, 3, 4, 6]
    for e in (0, 1, 100, 127, 131, 254, 255):
        for c in range(16):
            lo = (-1 if c & 8 else 1) * table[c & 7]
            hi_code = (c + 5) % 16
            hi = (-1 if hi_code & 8 else 1) * table[hi_code & 7]
            scale = 2.0 ** (e - 127)
            if e == 255:
                assert math.isnan(out[e, 2 * c]) and math.isnan(out[e, 2 * c + 1])
            else:
                assert out[e, 2 * c] == np.float32(lo * scale)      # low nibble = even element
                assert out[e, 2 * c + 1] == np.float32(hi * scale)


def _numpy_mxfp8(x_f32):
    """Independent restatement of mxfp4.cu:12-22 with numpy float32 and torch's RNE e4m3."""
    rows, cols = x_f32.shape
    g = x_f32.reshape(rows, cols // 32, 32)
    amax = np.nanmax(np.where(np.isnan(g), -np.inf, np.abs(g)), axis=2).astype(np.float32)
    amax = np.maximum(amax, np.float32(1e-4))
    t = (amax * np.float32(1.0 / 448.0)).astype(np.float32)
    mant, ex = np.frexp(t.astype(np.float64))          # t = mant * 2^ex, mant in [0.5, 1)
    e = np.where(mant == 0.5, ex - 1, ex) + 127          # ceil to a power of two
    scale = np.ldexp(np.float32(1), (e - 127)).astype(np.float32)
    v = np.clip(g / scale[..., None], -448, 448).astype(np.float32)
    q = torch.from_numpy(np.ascontiguousarray(v)).to(torch.float8_e4m3fn).view(torch.uint8).numpy()
    return q.reshape(rows, cols), e.astype(np.uint8)


@pytest.mark.parametrize("seed", [0, 1, 2])
def test_quantize_mxfp8_vs_numpy(seed):
    rng = np.random.default_rng(seed)
    x = (rng.standard_normal((8, 1024)) * rng.choice([1e-6, 1e-3, 1, 100, 1e4], (8, 1))).astype(np.float32)
    bits = O.bf16_bits(x)
    q, s = O.quantize_mxfp8(bits)
    qr, sr = _numpy_mxfp8(O.bf16_to_f32(bits))
    assert np.array_equal(s, sr)
    assert np.array_equal(q, qr)


def test_quantize_mxfp8_edges():
    x = np.zeros((4, 64), np.float32)
    x[1, :32] = 448.0 * 2.0 ** 3          # exact power-of-two multiple of 448: no ceil bump
    x[1, 32:] = np.linspace(-3, 3, 32)
    x[2, 5] = 1e-30                         # below the 1e-4 floor
    x[3, :] = -0.0
    bits = O.bf16_bits(x)
    q, s = O.quantize_mxfp8(bits)
    qr, sr = _numpy_mxfp8(O.bf16_to_f32(bits))
    assert np.array_equal(q, qr) and np.array_equal(s, sr)
    assert s[1, 0] == 127 + 3 and np.all(q[1, :32] == 0x7E)
    # all-zero group: scale from the 1e-4 floor
    floor_e = int(np.frexp(np.float64(np.float32(np.float32(1e-4) * np.float32(1 / 448))))[1]) + 127
    assert s[0, 0] == floor_e
    assert np.all(q[3] == 0x80)  # -0 keeps its sign


def test_quantize_mxfp8_bruteforce_one_group_all_bf16_magnitudes():
    # every finite bf16 value as the lone nonzero of a group, at a fixed amax partner
    vals = (np.arange(0, 0x7F80, 1, dtype=np.uint32) << 16).view(np.float32)
    vals = vals[::7]
    n = len(vals) // 31 * 31
    x = np.zeros((n // 31, 32), np.float32)
    x[:, :31] = vals[:n].reshape(-1, 31)
    x[:, 31] = -vals[:n].reshape(-1, 31)[:, -1]
    bits = O.bf16_bits(x)
    q, s = O.quantize_mxfp8(bits)
    qr, sr = _numpy_mxfp8(O.bf16_to_f32(bits))
    assert np.array_equal(q, qr) and np.array_equal(s, sr)
