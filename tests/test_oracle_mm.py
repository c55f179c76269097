"""Pins the oracle's GEMM restatement (oracle.mm_int8 / oracle.mm_float, the
checker of the HIP GEMM; reference kernels/cuda/wmma.cu:29-261) on the CPU:

- against numpy's int64 / float64 matmul (a library routine) reduced the
  way the reference's accumulators are (int32 wrap-around);
- closed forms: identity and permutation operands, all-equal operands
  (C = K * a * b), the int32 wrap of a sum that passes 2^31;
- the uint8 offset identity the HIP path relies on,
  sum ua ub = sum sa sb + 128 (sum sa + sum sb) + 16384 K with s = u - 128;
- a pure-Python triple loop on tiny inputs;
- both storages of B ([K, N] and [N, K]).
The reference ships no golden vectors for this kernel (its example compares
against torch.matmul, examples/kernels/wmma_simple.py:57-80).
"""
from __future__ import annotations

import numpy as np
import pytest

import oracle


def wrap32(v: np.ndarray) -> np.ndarray:
    return (np.asarray(v, np.int64) & 0xFFFFFFFF).astype(np.uint32).view(np.int32)


@pytest.mark.parametrize("dt", [np.int8, np.uint8])
@pytest.mark.parametrize("M,N,K", [(1, 1, 1), (3, 5, 7), (16, 32, 48), (33, 17, 129)])
def test_mm_int8_matches_numpy(dt, M, N, K):
    rng = np.random.default_rng(M * 100 + N * 10 + K)
    info = np.iinfo(dt)
    a = rng.integers(info.min, info.max + 1, (M, K)).astype(dt)
    b = rng.integers(info.min, info.max + 1, (K, N)).astype(dt)
    want = wrap32(a.astype(np.int64) @ b.astype(np.int64))
    np.testing.assert_array_equal(oracle.mm_int8(a, b), want)
    np.testing.assert_array_equal(oracle.mm_int8(a, np.ascontiguousarray(b.T), b_nk=True), want)


def test_mm_int8_closed_forms():
    K = 64
    eye = np.eye(K, dtype=np.int8)
    b = np.arange(K * 8, dtype=np.int64).reshape(K, 8).astype(np.int8)
    np.testing.assert_array_equal(oracle.mm_int8(eye, b), b.astype(np.int32))
    perm = np.random.default_rng(0).permutation(K)
    p = eye[perm]
    np.testing.assert_array_equal(oracle.mm_int8(p, b), b[perm].astype(np.int32))
    # all-equal operands: C = K * a * b
    for av, bv in [(-128, -128), (127, -128), (-1, 3)]:
        a = np.full((4, K), av, np.int8)
        bb = np.full((K, 4), bv, np.int8)
        np.testing.assert_array_equal(oracle.mm_int8(a, bb), np.full((4, 4), K * av * bv, np.int32))
    # uint8 all 255: 65025 K
    a = np.full((2, K), 255, np.uint8)
    np.testing.assert_array_equal(oracle.mm_int8(a, np.full((K, 2), 255, np.uint8)),
                                  np.full((2, 2), 65025 * K, np.int32))


def test_mm_int8_wraps_like_int32_accumulators():
    # (-128)^2 * 2^17 = 2^31: one past INT32_MAX wraps to INT32_MIN
    K = 1 << 17
    a = np.full((1, K), -128, np.int8)
    b = np.full((K, 1), -128, np.int8)
    assert oracle.mm_int8(a, b)[0, 0] == -(1 << 31)
    # 255^2 * 2^16 = 4261478400 wraps to 4261478400 - 2^32
    K = 1 << 16
    a = np.full((1, K), 255, np.uint8)
    assert oracle.mm_int8(a, np.full((K, 1), 255, np.uint8))[0, 0] == 4261478400 - (1 << 32)


@pytest.mark.parametrize("K", [16, 64, 1000])
def test_uint8_offset_identity(K):
    """The HIP uint8 path multiplies s = u ^ 0x80 (= u - 128) as int8 and
    adds 128 (rowsum(sa) + colsum(sb)) + 16384 K; the identity holds exactly
    modulo 2^32."""
    rng = np.random.default_rng(K)
    ua = rng.integers(0, 256, (7, K)).astype(np.uint8)
    ub = rng.integers(0, 256, (K, 9)).astype(np.uint8)
    sa = (ua ^ 0x80).view(np.int8)
    sb = (ub ^ 0x80).view(np.int8)
    assert np.array_equal(sa.astype(np.int64), ua.astype(np.int64) - 128)
    core = oracle.mm_int8(sa, sb).astype(np.int64)
    fix = 128 * (sa.astype(np.int64).sum(1)[:, None] + sb.astype(np.int64).sum(0)[None, :]) \
        + 16384 * K
    np.testing.assert_array_equal(wrap32(core + fix), oracle.mm_int8(ua, ub))


def test_mm_int8_brute_force_tiny():
    rng = np.random.default_rng(5)
    a = rng.integers(-128, 128, (2, 3)).astype(np.int8)
    b = rng.integers(-128, 128, (3, 4)).astype(np.int8)
    want = [[sum(int(a[m, k]) * int(b[k, n]) for k in range(3)) for n in range(4)]
            for m in range(2)]
    np.testing.assert_array_equal(oracle.mm_int8(a, b), np.array(want, np.int32))


@pytest.mark.parametrize("code", [oracle.F16, oracle.BF16])
def test_mm_float_matches_numpy(code):
    rng = np.random.default_rng(code)
    a32 = rng.standard_normal((9, 40)).astype(np.float32)
    b32 = rng.standard_normal((40, 11)).astype(np.float32)
    a = oracle.from_f32(a32, code)
    b = oracle.from_f32(b32, code)
    want = oracle.to_f32(a, code).astype(np.float64) @ oracle.to_f32(b, code).astype(np.float64)
    np.testing.assert_allclose(oracle.mm_float(a, b, code), want, rtol=1e-12, atol=1e-12)
    np.testing.assert_allclose(oracle.mm_float(a, np.ascontiguousarray(b.T), code, b_nk=True),
                               want, rtol=1e-12, atol=1e-12)
    # identity: exact
    eye = oracle.from_f32(np.eye(40, dtype=np.float32), code)
    np.testing.assert_array_equal(oracle.mm_float(eye, b, code), oracle.to_f32(b, code))
