"""GPU parity of the dense GEMM (cbq_mm through cublade_amd.bindings.hip.wmma,
the replacement of the reference's wmma_gemm, kernels/cuda/wmma.cu:29-261)
against the CPU oracle.

Bar: int8 / uint8 -> int32 bit-exact (int32 wrap-around included); fp16 /
bf16 within the fp32-accumulation error bound
|C - ref| <= K * 2^-24 * sum_k |a_k b_k| (+ the final rounding to fp16,
2^-11 |ref| + 2^-24, for fp16 outputs), with ref the oracle's double sum.
Covers both storages of B ([K, N] and the [N, K] weight layout read in
place), K that is not a multiple of 64 bytes (padded staging), partial
tiles, both tile sizes (256 and 128) with and without a K split, and the
reference's argument errors.
"""
from __future__ import annotations

import numpy as np
import pytest
import torch

import oracle
from tests._util import bits

pytestmark = pytest.mark.gpu

DEV = "cuda"


def H():
    from cublade_amd.bindings.hip import wmma
    return wmma


def rand_int(shape, dt, seed):
    g = torch.Generator().manual_seed(seed)
    if dt == torch.int8:
        return torch.randint(-128, 128, shape, generator=g, dtype=torch.int16).to(torch.int8)
    return torch.randint(0, 256, shape, generator=g, dtype=torch.int16).to(torch.uint8)


def np_of(t: torch.Tensor) -> np.ndarray:
    return t.cpu().numpy()


INT_SHAPES = [(16, 16, 16), (256, 256, 64), (128, 272, 48), (272, 528, 1040), (512, 512, 512),
              (64, 1024, 4096), (1024, 256, 256), (32, 48, 80)]


@pytest.mark.parametrize("dt", [torch.int8, torch.uint8])
@pytest.mark.parametrize("M,N,K", INT_SHAPES)
@pytest.mark.parametrize("layout", ["kn", "nk"])
def test_mm_int_bit_exact(dt, M, N, K, layout):
    print(f"[mm] {dt} M={M} N={N} K={K} B={layout}", flush=True)
    A = rand_int((M, K), dt, seed=M + 7 * N + 13 * K)
    if layout == "kn":
        B = rand_int((K, N), dt, seed=3 * M + N + K)
        Bd = B.to(DEV)
        want = oracle.mm_int8(np_of(A), np_of(B))
    else:
        W = rand_int((N, K), dt, seed=3 * M + N + K)
        Bd = W.to(DEV).t()                       # [K, N] view of the [N, K] weight
        want = oracle.mm_int8(np_of(A), np_of(W), b_nk=True)
    C = H().wmma_gemm(A.to(DEV), Bd)
    assert C.dtype == torch.int32 and tuple(C.shape) == (M, N)
    np.testing.assert_array_equal(np_of(C), want)


def test_mm_int8_extremes_and_wrap():
    """All -128 operands at K = 2^17 (16 x 16 tiles): every sum is 2^31 and
    wraps to INT32_MIN, as int32 accumulators do; all 255 uint8 at K = 2^16."""
    K = 1 << 17
    A = torch.full((16, K), -128, dtype=torch.int8, device=DEV)
    C = H().wmma_gemm(A, torch.full((K, 16), -128, dtype=torch.int8, device=DEV))
    assert bool((C == -(1 << 31)).all())
    K = 1 << 16
    A = torch.full((16, K), 255, dtype=torch.uint8, device=DEV)
    C = H().wmma_gemm(A, torch.full((K, 16), 255, dtype=torch.uint8, device=DEV))
    assert bool((C == 4261478400 - (1 << 32)).all())


def test_mm_int8_bench_shape_rows():
    """The benchmark shape (8192^3, weight layout): 16 rows and all columns
    against the oracle, bit-exact."""
    M = N = K = 8192
    A = rand_int((M, K), torch.int8, seed=1)
    W = rand_int((N, K), torch.int8, seed=2)
    C = H().wmma_gemm(A.to(DEV), W.to(DEV).t())
    rows = np.random.default_rng(0).choice(M, 16, replace=False)
    want = oracle.mm_int8(np_of(A)[rows], np_of(W), b_nk=True)
    np.testing.assert_array_equal(np_of(C)[rows], want)


def float_bound(a64: np.ndarray, b64: np.ndarray, K: int, f16_out: bool, ref: np.ndarray):
    bound = K * 2.0 ** -24 * (np.abs(a64) @ np.abs(b64)) + 1e-30
    if f16_out:
        bound = bound + 2.0 ** -11 * np.abs(ref) + 2.0 ** -24
    return bound


@pytest.mark.parametrize("dt,out", [(torch.float16, torch.float32), (torch.float16, torch.float16),
                                    (torch.bfloat16, torch.float32)])
@pytest.mark.parametrize("M,N,K", [(16, 16, 16), (272, 528, 1040), (256, 256, 512), (48, 32, 16)])
@pytest.mark.parametrize("layout", ["kn", "nk"])
def test_mm_float_within_bound(dt, out, M, N, K, layout):
    print(f"[mm] {dt}->{out} M={M} N={N} K={K} B={layout}", flush=True)
    code = oracle.F16 if dt == torch.float16 else oracle.BF16
    g = torch.Generator().manual_seed(M + N + K)
    A = torch.randn(M, K, generator=g).to(dt)
    W = torch.randn(N, K, generator=g).to(dt)          # B = W^T
    if layout == "kn":
        Bd = W.t().contiguous().to(DEV)
    else:
        Bd = W.to(DEV).t()
    C = H().wmma_gemm(A.to(DEV), Bd, out)
    assert C.dtype == out and tuple(C.shape) == (M, N)
    ref = oracle.mm_float(bits(A), bits(W), code, b_nk=True)
    a64 = oracle.to_f32(bits(A), code).astype(np.float64)
    b64 = oracle.to_f32(bits(W), code).astype(np.float64).T
    err = np.abs(C.float().cpu().numpy().astype(np.float64) - ref)
    bound = float_bound(a64, b64, K, out == torch.float16, ref)
    assert (err <= bound).all(), float((err / bound).max())


def test_mm_noncontiguous_b_and_default_acc():
    """A B that is neither [K, N] nor a transposed [N, K] is copied; defaults
    follow the reference's precision table (int8 -> int32, fp16 -> fp32)."""
    A = rand_int((64, 96), torch.int8, seed=3).to(DEV)
    Bfull = rand_int((96, 256), torch.int8, seed=4).to(DEV)
    Bv = Bfull[:, ::2]                                  # [96, 128], strided
    C = H().wmma_gemm(A, Bv)
    want = oracle.mm_int8(np_of(A), np.ascontiguousarray(np_of(Bv)))
    np.testing.assert_array_equal(np_of(C), want)
    Ah = torch.randn(32, 32, device=DEV).half()
    assert H().wmma_gemm(Ah, Ah).dtype == torch.float32


def test_mm_reference_errors():
    w = H().wmma_gemm
    a = torch.zeros(16, 16, dtype=torch.int8, device=DEV)
    with pytest.raises(RuntimeError, match="CUDA tensors"):
        w(a.cpu(), a)
    with pytest.raises(RuntimeError, match="2D"):
        w(a.view(16, 16, 1), a)
    with pytest.raises(RuntimeError, match="incompatible"):
        w(a, torch.zeros(32, 16, dtype=torch.int8, device=DEV))
    with pytest.raises(RuntimeError, match="same dtype"):
        w(a, a.to(torch.uint8))
    with pytest.raises(RuntimeError, match="multiples of 16"):
        w(torch.zeros(24, 16, dtype=torch.int8, device=DEV), a)
    with pytest.raises(RuntimeError, match="int32 accumulator"):
        w(a, a, torch.float32)
    with pytest.raises(RuntimeError, match="float32 accumulator"):
        w(a.to(torch.bfloat16), a.to(torch.bfloat16), torch.float16)
    with pytest.raises(RuntimeError, match="Unsupported dtype"):
        w(a.float(), a.float())


@pytest.mark.parametrize("dt,out", [(torch.int8, torch.int32), (torch.uint8, torch.int32),
                                    (torch.float16, torch.float16), (torch.bfloat16, torch.float32)])
def test_mm_empty_contraction(dt, out):
    """K == 0 is a multiple of 16: C = 0 (the reference's zero-filled
    accumulators are stored); M == 0 gives an empty C."""
    C = H().wmma_gemm(torch.empty(32, 0, dtype=dt, device=DEV),
                      torch.empty(0, 48, dtype=dt, device=DEV), out)
    assert C.dtype == out and tuple(C.shape) == (32, 48) and bool((C == 0).all())
    C = H().wmma_gemm(torch.empty(0, 16, dtype=dt, device=DEV),
                      torch.zeros(16, 48, dtype=dt, device=DEV), out)
    assert tuple(C.shape) == (0, 48)


@pytest.mark.parametrize("M,N,K,dt,path", [
    (4096, 4096, 128, torch.int8, "256 tiles"),
    (256, 8192, 16384, torch.int8, "256 tiles, K in 8 ranges"),
    (1024, 1024, 1024, torch.int8, "128 tiles"),
    (16, 11008, 4096, torch.int8, "128 tiles, K in 5 ranges"),
    (64, 1024, 4096, torch.uint8, "128 tiles, K in 16 ranges"),
    (2048, 4096, 4096, torch.float16, "256 tiles, K in 2 ranges"),
    (1024, 4096, 4096, torch.float16, "128 tiles"),
])
def test_mm_tile_and_split_paths(M, N, K, dt, path):
    """Each tile size with and without a K split (the host's time model picks
    them per shape), B in the weight layout; sampled rows against an exact
    numpy product: int64 reduced modulo 2^32 for integers, the fp32
    accumulation bound for fp16."""
    print(f"[mm] {dt} M={M} N={N} K={K} ({path})", flush=True)
    if dt == torch.float16:
        g = torch.Generator().manual_seed(M + N)
        A, W = torch.randn(M, K, generator=g).half(), torch.randn(N, K, generator=g).half()
    else:
        A, W = rand_int((M, K), dt, seed=M + K), rand_int((N, K), dt, seed=N + K)
    C = H().wmma_gemm(A.to(DEV), W.to(DEV).t())
    rows = np.unique(np.array([0, 1, M // 3, M // 2, M - 1]))
    if dt == torch.float16:
        a64 = A.numpy()[rows].astype(np.float64)
        b64 = W.numpy().astype(np.float64).T
        ref = a64 @ b64
        err = np.abs(np_of(C)[rows].astype(np.float64) - ref)
        assert (err <= float_bound(a64, b64, K, False, ref)).all()
    else:
        ref = (np_of(A)[rows].astype(np.int64) @ np_of(W).astype(np.int64).T) % (1 << 32)
        got = np_of(C)[rows].astype(np.int64) % (1 << 32)
        np.testing.assert_array_equal(got, ref)


@pytest.mark.parametrize("M,N,K,dt", [
    (4096, 4096, 128, torch.int8), (256, 8192, 16384, torch.int8), (1024, 1024, 1024, torch.int8),
    (16, 11008, 4096, torch.int8), (256, 1040, 512, torch.int8), (2048, 4096, 4096, torch.float16),
    (1024, 4096, 4096, torch.float16), (256, 1040, 512, torch.float16), (512, 768, 1024, torch.bfloat16),
])
def test_mm_kn_in_place_paths(M, N, K, dt):
    """B given as a contiguous [K, N] with K filling whole 64-byte k-steps is
    read in place (transposing LDS reads, no staging pass) on each tile and
    split path, including column tiles past N: sampled rows against an exact
    numpy product (int64 modulo 2^32, or the fp32 accumulation bound)."""
    print(f"[mm] {dt} M={M} N={N} K={K} (B [K, N] in place)", flush=True)
    if dt in (torch.float16, torch.bfloat16):
        g = torch.Generator().manual_seed(M + N + K)
        A, B = torch.randn(M, K, generator=g).to(dt), torch.randn(K, N, generator=g).to(dt)
    else:
        A, B = rand_int((M, K), dt, seed=M + K), rand_int((K, N), dt, seed=N + K)
    C = H().wmma_gemm(A.to(DEV), B.to(DEV))
    rows = np.unique(np.array([0, 1, M // 3, M // 2, M - 1]))
    if dt in (torch.float16, torch.bfloat16):
        a64 = A[rows].float().numpy().astype(np.float64)
        b64 = B.float().numpy().astype(np.float64)
        ref = a64 @ b64
        err = np.abs(np_of(C)[rows].astype(np.float64) - ref)
        assert (err <= float_bound(a64, b64, K, False, ref)).all()
    else:
        ref = (np_of(A)[rows].astype(np.int64) @ np_of(B).astype(np.int64)) % (1 << 32)
        got = np_of(C)[rows].astype(np.int64) % (1 << 32)
        np.testing.assert_array_equal(got, ref)


def test_mm_repeated_calls_share_workspace():
    """Back-to-back calls with different staging needs on one workspace."""
    wm = H().wmma_gemm
    for M, N, K, dt in [(512, 256, 1040, torch.uint8), (64, 64, 64, torch.int8),
                        (256, 512, 80, torch.uint8), (128, 128, 128, torch.int8)]:
        A = rand_int((M, K), dt, seed=M + K)
        B = rand_int((K, N), dt, seed=N + K)
        C = wm(A.to(DEV), B.to(DEV))
        np.testing.assert_array_equal(np_of(C), oracle.mm_int8(np_of(A), np_of(B)))
