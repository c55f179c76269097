"""Pin the oracle's scalar numerics against library conversions (CPU only).

Every 16-bit and 8-bit code is checked exhaustively against torch / numpy,
which are implementations independent of oracle/cbq_oracle.c. A plausible
mistake (round-half-up instead of half-even, a wrong exponent bias, a missing
saturation, a flushed subnormal) fails at least one of these.
"""
import numpy as np
import pytest
import torch

import oracle

pytestmark = pytest.mark.filterwarnings("ignore::RuntimeWarning")

ALL16 = np.arange(65536, dtype=np.uint32).astype(np.uint16)


def _nan_aware_equal_f32(a: np.ndarray, b: np.ndarray) -> bool:
    a = np.asarray(a, np.float32)
    b = np.asarray(b, np.float32)
    both_nan = np.isnan(a) & np.isnan(b)
    same = a.view(np.uint32) == b.view(np.uint32)
    return bool(np.all(both_nan | same))


def _codes_equal_nan_aware(a, b, nan_mask):
    a = np.asarray(a)
    b = np.asarray(b)
    return bool(np.all((a == b) | nan_mask))


def test_decode_fp16_exhaustive_vs_numpy():
    ref = ALL16.view(np.float16).astype(np.float32)
    assert _nan_aware_equal_f32(oracle.to_f32(ALL16, oracle.F16), ref)


def test_decode_bf16_exhaustive_vs_torch():
    ref = torch.from_numpy(ALL16.view(np.int16)).view(torch.bfloat16).float().numpy()
    assert _nan_aware_equal_f32(oracle.to_f32(ALL16, oracle.BF16), ref)


def test_decode_e4m3_exhaustive_vs_torch():
    codes = np.arange(256, dtype=np.uint8)
    ref = torch.from_numpy(codes).view(torch.float8_e4m3fn).float().numpy()
    assert _nan_aware_equal_f32(oracle.decode_e4m3(codes), ref)
    # closed-form spot values of OCP E4M3
    got = oracle.decode_e4m3(np.array([0x7E, 0x08, 0x01, 0x38, 0xFE, 0x7F], np.uint8))
    assert got[0] == 448.0 and got[1] == 2.0 ** -6 and got[2] == 2.0 ** -9
    assert got[3] == 1.0 and got[4] == -448.0 and np.isnan(got[5])


def _probe_floats() -> np.ndarray:
    """Float32 values that stress 16-bit and 8-bit rounding: every fp16 and
    bf16 value, their midpoints and neighbours, and random floats."""
    f16 = ALL16.view(np.float16).astype(np.float32)
    bf = (ALL16.astype(np.uint32) << 16).view(np.float32)
    base = np.concatenate([f16, bf])
    base = base[np.isfinite(base)]
    u = base.view(np.uint32)
    mids16 = ((u[: len(u) // 2] + (1 << 12)) & 0xFFFFFFFF).astype(np.uint32).view(np.float32)
    midsbf = ((u + (1 << 15)) & 0xFFFFFFFF).astype(np.uint32).view(np.float32)
    nb = np.concatenate([(u + 1).view(np.float32), (u - 1).view(np.float32)])
    rng = np.random.default_rng(7)
    rnd = (rng.standard_normal(200_000) * np.exp(rng.uniform(-30, 15, 200_000))).astype(np.float32)
    specials = np.array([0.0, -0.0, np.inf, -np.inf, np.nan, 65504, 65519.99, 65520,
                         448, 464, 463.99, 480, 2 ** -10, 2 ** -25, 3 * 2 ** -26],
                        np.float32)
    out = np.concatenate([base, mids16, midsbf, nb, rnd, specials])
    return out


PROBE = _probe_floats()


def test_encode_f16_vs_numpy():
    ref = PROBE.astype(np.float16).view(np.uint16)
    got = oracle.from_f32(PROBE, oracle.F16)
    assert _codes_equal_nan_aware(got, ref, np.isnan(PROBE))
    assert np.all(np.isnan(got.view(np.float16)) == np.isnan(PROBE))


def test_encode_bf16_vs_torch():
    ref = torch.from_numpy(PROBE).to(torch.bfloat16).view(torch.int16).numpy().view(np.uint16)
    got = oracle.from_f32(PROBE, oracle.BF16)
    nan = np.isnan(PROBE)
    assert _codes_equal_nan_aware(got, ref, nan)
    got_f = (got.astype(np.uint32) << 16).view(np.float32)
    assert np.all(np.isnan(got_f) == nan)


@pytest.mark.parametrize("inv", [1.0, 56.0, 448.0 / 3.1, 7.13e3, 3.3e-3, 4.48e14])
def test_encode_e4m3_satfinite_vs_torch(inv):
    v = (PROBE * np.float32(inv)).astype(np.float32)
    ref = (torch.from_numpy(v).clamp(-448.0, 448.0).to(torch.float8_e4m3fn)
           .view(torch.uint8).numpy())
    got = oracle.cast_e4m3(v)
    nan = np.isnan(v)
    assert _codes_equal_nan_aware(got, ref, nan)
    assert np.all(((got & 0x7F) == 0x7F) == nan)


def test_encode_e4m3_every_midpoint():
    """Midpoints between adjacent E4M3 values must round to the even code."""
    codes = np.arange(0, 0x7E, dtype=np.uint8)
    lo = oracle.decode_e4m3(codes).astype(np.float64)
    hi = oracle.decode_e4m3(codes + 1).astype(np.float64)
    mid = ((lo + hi) / 2).astype(np.float32)
    got = oracle.cast_e4m3(mid)
    want = np.where(codes % 2 == 0, codes, codes + 1).astype(np.uint8)
    assert np.array_equal(got, want)
    assert np.array_equal(oracle.cast_e4m3(-mid), want | 0x80)


def test_round_clamp_int8_vs_torch():
    rng = np.random.default_rng(3)
    halves = (np.arange(-300, 301) / 2.0).astype(np.float32)
    v = np.concatenate([halves, (rng.standard_normal(100_000) * 100).astype(np.float32),
                        np.array([np.inf, -np.inf, 1e30, -1e30, 126.5, -126.5, 127.5,
                                  -127.5, 0.49999997, -0.49999997], np.float32)])
    ref = torch.round(torch.from_numpy(v)).clamp(-127, 127).to(torch.int8).numpy()
    assert np.array_equal(oracle.cast_int8(v), ref)
    # half-to-even closed forms and NaN -> 0 (PTX cvt.rni semantics)
    assert list(oracle.cast_int8(np.array([0.5, 1.5, 2.5, -2.5, np.nan], np.float32))) == \
        [0, 2, 2, -2, 0]


def test_inv_scale_is_correctly_rounded_division():
    """fp32 127/a and 448/a must equal the float64 quotient narrowed once
    (the reference computes in double then narrows: quantize_int8.cu:120-126)."""
    rng = np.random.default_rng(11)
    amax = np.abs(rng.standard_normal(20000) * np.exp(rng.uniform(-20, 20, 20000))).astype(np.float32)
    for q in (127.0, 448.0):
        for a in amax[:2000]:
            inv = oracle.inv_scale(float(a), 1e-12, q)
            assert inv == np.float32(q / np.float64(a))
            assert oracle.scale_from_inv(float(inv)) == np.float32(1.0 / np.float64(inv))
    # eps floor
    assert oracle.inv_scale(0.0, 1e-12, 127.0) == np.float32(127.0 / np.float64(np.float32(1e-12)))


def test_amax_vs_numpy_and_nan_dropped():
    rng = np.random.default_rng(5)
    x = rng.standard_normal(100_001).astype(np.float32)
    x[777] = -91.5
    b = torch.from_numpy(x).to(torch.bfloat16).view(torch.int16).numpy().view(np.uint16)
    assert oracle.amax(b, oracle.BF16) == np.abs(oracle.to_f32(b, oracle.BF16)).max() == 91.5
    xn = x.copy()
    xn[5] = np.nan
    assert oracle.amax(xn, oracle.F32) == np.nanmax(np.abs(xn))
    assert oracle.amax(np.zeros(0, np.float32), oracle.F32) == 0.0


def test_planted_rounding_mistake_is_detected():
    """Guard on the checks themselves: a round-half-away int8 cast (a plausible
    restatement mistake) disagrees with the library reference used above."""
    v = (np.arange(-300, 301) / 2.0).astype(np.float32)
    wrong = np.clip(np.sign(v) * np.floor(np.abs(v) + 0.5), -127, 127).astype(np.int8)
    ref = torch.round(torch.from_numpy(v)).clamp(-127, 127).to(torch.int8).numpy()
    assert not np.array_equal(wrong, ref)
    assert np.array_equal(oracle.cast_int8(v), ref)
