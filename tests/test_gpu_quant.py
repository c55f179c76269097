"""GPU parity of the quant / dequant kernels (HIP C ABI via the bindings and
the public API) against the CPU oracle and the committed golden vectors.

Bar: bit-exact FP8 / INT8 codes, bit-exact fp32 scales, bit-exact fp16 /
bf16 dequantized outputs (any NaN matches any NaN). Covers every kernel
shape the dispatcher selects (row lengths 8..16384 and odd lengths, vector
and unaligned scalar paths, tails), exhaustive 16-bit and 8-bit code spaces,
special values (NaN, inf, zeros, subnormals), repeated calls sharing one
workspace, a non-default stream, and the BASELINE configurations at full
size.
"""
from __future__ import annotations

import numpy as np
import pytest
import torch

import oracle
from tests import _golden as G
from tests._util import (CODE_OF, DTYPE_OF, assert_array_equal, assert_bits_equal_16,
                         assert_fp8_equal, assert_scales_equal, bits, from_bits)

pytestmark = pytest.mark.gpu

DEV = "cuda"


def _lib():
    from cublade_amd import _abi
    return _abi.lib()


@pytest.fixture(scope="module", autouse=True)
def _loaded():
    _lib()  # the HIP library must load; there is no fallback


def hip():
    from cublade_amd.bindings import hip as H
    return H


# ---------------------------------------------------------------------------
# checkers: run the HIP path on bits `x` and compare with the oracle
# ---------------------------------------------------------------------------
def check_fp8_tensor(x, code, shape=None, what=""):
    xt = from_bits(x, code, DEV)
    if shape is not None:
        xt = xt.view(shape)
    q, s = hip().quantize_per_tensor_fp8(xt)
    qo, so = oracle.quant_fp8_tensor(x, code)
    assert_fp8_equal(bits(q), qo, what + " q")
    assert_scales_equal(bits(s).reshape(-1), np.array([so]), what)
    for out in (torch.float16, torch.bfloat16):
        y = hip().dequantize_per_tensor_fp8(q, s, out)
        assert_bits_equal_16(bits(y), oracle.dequant_fp8_tensor(qo, so, CODE_OF[out]),
                             CODE_OF[out], what + f" y {out}")


def check_int8_tensor(x, code, what=""):
    xt = from_bits(x, code, DEV)
    q, s = hip().quantize_per_tensor_int8(xt)
    qo, so = oracle.quant_int8_tensor(x, code)
    assert_array_equal(bits(q), qo, what + " q")
    assert_scales_equal(bits(s).reshape(-1), np.array([so]), what)
    for out in (torch.float16, torch.bfloat16):
        y = hip().dequantize_per_tensor_int8(q, s, out)
        assert_bits_equal_16(bits(y), oracle.dequant_int8_tensor(qo, so, CODE_OF[out]),
                             CODE_OF[out], what + f" y {out}")


def check_int8_channel(x2, code, axis, what=""):
    rows, cols = x2.shape
    xt = from_bits(x2.reshape(-1), code, DEV).view(rows, cols)
    q, s = hip().quantize_per_channel_int8(xt, axis=axis)
    qo, so = oracle.quant_int8_channel(x2, code, axis=axis)
    assert_array_equal(bits(q), qo, what + " q")
    assert_scales_equal(bits(s), so, what)
    out = torch.bfloat16 if code != oracle.F16 else torch.float16
    y = hip().dequantize_per_channel_int8(q, s, out, axis=axis)
    assert_bits_equal_16(bits(y), oracle.dequant_int8_channel(qo, so, CODE_OF[out], axis=axis),
                         CODE_OF[out], what + " y")


def check_int8_group(x2, code, gs, what=""):
    xt = from_bits(x2.reshape(-1), code, DEV).view(-1, gs)
    q, s = hip().quantize_per_group_int8(xt, gs)
    qo, so = oracle.quant_int8_group(x2, code, gs)
    assert_array_equal(bits(q), qo, what + " q")
    assert_scales_equal(bits(s), so, what)
    for out in (torch.float16, torch.bfloat16):
        y = hip().dequantize_per_group_int8(q, s, gs, out)
        assert_bits_equal_16(bits(y), oracle.dequant_int8_group(qo, so, gs, CODE_OF[out]),
                             CODE_OF[out], what + f" y {out}")


def rand_bits(shape, code, seed, scale=1.0, rowfac=False):
    g = torch.Generator().manual_seed(seed)
    v = torch.randn(*shape, generator=g) * scale
    if rowfac and len(shape) == 2:
        v = v * (0.1 + 9.9 * torch.rand(shape[0], 1, generator=g))
    return bits(v.to(DTYPE_OF[code]))


# ---------------------------------------------------------------------------
# golden vectors
# ---------------------------------------------------------------------------
@pytest.mark.parametrize("meta,arr", G.cases("fp8_tensor"), ids=G.ids("fp8_tensor"))
def test_golden_fp8_tensor(meta, arr):
    x = arr["x"].reshape(-1)
    xt = from_bits(x, meta["dtype"], DEV).view(meta["shape"])
    q, s = hip().quantize_per_tensor_fp8(xt)
    assert_fp8_equal(bits(q), arr["q"], meta["name"])
    assert_scales_equal(bits(s).reshape(-1), arr["scale"], meta["name"])
    for out in (torch.float16, torch.bfloat16):
        y = hip().dequantize_per_tensor_fp8(q, s, out)
        assert_bits_equal_16(bits(y), arr[f"y{CODE_OF[out]}"], CODE_OF[out], meta["name"])


@pytest.mark.parametrize("meta,arr", G.cases("int8_tensor"), ids=G.ids("int8_tensor"))
def test_golden_int8_tensor(meta, arr):
    xt = from_bits(arr["x"].reshape(-1), meta["dtype"], DEV).view(meta["shape"])
    q, s = hip().quantize_per_tensor_int8(xt)
    assert_array_equal(bits(q), arr["q"], meta["name"])
    assert_scales_equal(bits(s).reshape(-1), arr["scale"], meta["name"])
    for out in (torch.float16, torch.bfloat16):
        y = hip().dequantize_per_tensor_int8(q, s, out)
        assert_bits_equal_16(bits(y), arr[f"y{CODE_OF[out]}"], CODE_OF[out], meta["name"])


@pytest.mark.parametrize("meta,arr", G.cases("int8_channel"), ids=G.ids("int8_channel"))
def test_golden_int8_channel(meta, arr):
    from cublade_amd.quantization import dequantize_tensor, quantize_tensor
    xt = from_bits(arr["x"].reshape(-1), meta["dtype"], DEV).view(meta["shape"])
    rows = meta["shape"][0]
    cols = int(np.prod(meta["shape"][1:])) if len(meta["shape"]) > 1 else 1
    q, s = hip().quantize_per_channel_int8(xt.view(rows, cols), axis=meta["axis"])
    assert_array_equal(bits(q), arr["q"], meta["name"])
    assert_scales_equal(bits(s), arr["scale"], meta["name"])
    for out in (torch.float16, torch.bfloat16):
        y = hip().dequantize_per_channel_int8(q, s, out, axis=meta["axis"])
        assert_bits_equal_16(bits(y), arr[f"y{CODE_OF[out]}"], CODE_OF[out], meta["name"])
    if meta["dtype"] != oracle.F32 and (meta["axis"] == 0 or len(meta["shape"]) == 2):
        qt = quantize_tensor(xt, dtype=torch.int8, mode="channel", ch_axis=meta["axis"])
        assert_array_equal(bits(qt.data), arr["q"], meta["name"] + " api")
        y = dequantize_tensor(qt)
        assert_bits_equal_16(bits(y), arr[f"y{meta['dtype']}"], meta["dtype"],
                             meta["name"] + " api")


@pytest.mark.parametrize("meta,arr", G.cases("int8_group"), ids=G.ids("int8_group"))
def test_golden_int8_group(meta, arr):
    gs = meta["group_size"]
    xt = from_bits(arr["x"].reshape(-1), meta["dtype"], DEV).view(-1, gs)
    q, s = hip().quantize_per_group_int8(xt, gs)
    assert_array_equal(bits(q), arr["q"], meta["name"])
    assert_scales_equal(bits(s), arr["scale"], meta["name"])
    for out in (torch.float16, torch.bfloat16):
        y = hip().dequantize_per_group_int8(q, s, gs, out)
        assert_bits_equal_16(bits(y), arr[f"y{CODE_OF[out]}"], CODE_OF[out], meta["name"])


# ---------------------------------------------------------------------------
# known answers (closed form)
# ---------------------------------------------------------------------------
def test_fp8_toy_known_answer():
    from cublade_amd.quantization import dequantize_tensor, quantize_tensor
    x = torch.arange(1, 9, dtype=torch.bfloat16, device=DEV)
    qt = quantize_tensor(x, dtype=torch.float8_e4m3fn, mode="tensor")
    assert bits(qt.data).tolist() == [0x66, 0x6E, 0x72, 0x76, 0x79, 0x7A, 0x7C, 0x7E]
    assert bits(qt.scale).view(np.uint32).item() == 0x3C924925
    assert bits(dequantize_tensor(qt)).tolist() == [0x3F80, 0x4000, 0x4037, 0x4080, 0x40A5,
                                                     0x40B7, 0x40DB, 0x4100]


def test_int8_linspace_known_answer():
    from cublade_amd.quantization import quantize_tensor
    x = torch.linspace(-1.0, 1.0, 256, dtype=torch.bfloat16).to(DEV)
    qt = quantize_tensor(x, dtype=torch.int8, mode="tensor")
    q = bits(qt.data)
    assert q[:10].tolist() == list(range(-127, -117))
    assert q[123:133].tolist() == [-4, -3, -2, -1, 0, 0, 1, 2, 3, 4]
    assert np.float32(qt.scale.item()) == np.float32(1.0) / np.float32(127.0)


# ---------------------------------------------------------------------------
# exhaustive code spaces
# ---------------------------------------------------------------------------
ALL16 = np.arange(65536, dtype=np.uint32).astype(np.uint16)


@pytest.mark.parametrize("code", [oracle.BF16, oracle.F16])
def test_exhaustive_fp8_cast_unit_inverse(code):
    """All finite 16-bit inputs with |x| <= 448, plus 448 so that inv == 1:
    the kernel's cast is then the bare E4M3 conversion of every such value
    (ties, subnormals, signed zeros)."""
    v = oracle.to_f32(ALL16, code)
    keep = ALL16[np.isfinite(v) & (np.abs(v) <= 448.0)]
    x = np.concatenate([keep, oracle.from_f32(np.array([448.0], np.float32), code)])
    check_fp8_tensor(x, code, what="exhaustive unit")


@pytest.mark.parametrize("code", [oracle.BF16, oracle.F16])
@pytest.mark.parametrize("amax", [1.0, 3.0, 0.01, 1000.0, 65504.0])
def test_exhaustive_fp8_cast_scaled(code, amax):
    """Every finite 16-bit input with |x| <= amax (amax present), so the
    multiply by a non-power-of-two inv and saturation paths are exercised."""
    v = oracle.to_f32(ALL16, code)
    keep = ALL16[np.isfinite(v) & (np.abs(v) <= amax)]
    x = np.concatenate([keep, oracle.from_f32(np.array([amax], np.float32), code)])
    check_fp8_tensor(x, code, what=f"exhaustive amax={amax}")


@pytest.mark.parametrize("code", [oracle.BF16, oracle.F16, oracle.F32])
@pytest.mark.parametrize("amax", [127.0, 1.0, 300.0])
def test_exhaustive_int8_cast(code, amax):
    if code == oracle.F32:
        rng = np.random.default_rng(1)
        v = np.concatenate([(np.arange(-254 * 4, 254 * 4 + 1) / 8.0),
                            rng.uniform(-amax, amax, 200_000)]).astype(np.float32)
        v = np.concatenate([v[np.abs(v) <= amax], np.array([amax], np.float32)])
        x = v
    else:
        v = oracle.to_f32(ALL16, code)
        keep = ALL16[np.isfinite(v) & (np.abs(v) <= amax)]
        x = np.concatenate([keep, oracle.from_f32(np.array([amax], np.float32), code)])
    check_int8_tensor(x, code, what=f"exhaustive int8 amax={amax}")


@pytest.mark.parametrize("scale", [1.0, 0.017857144, 3.5e-5, 7.77e3, 1e-30, 2.0 ** -20])
def test_exhaustive_dequant_codes(scale):
    """All 256 FP8 codes and all 256 INT8 codes (-128 included) times a scale."""
    s = torch.tensor(scale, dtype=torch.float32, device=DEV)
    codes8 = np.arange(256, dtype=np.uint8)
    q8 = torch.from_numpy(np.tile(codes8, 3)).view(torch.float8_e4m3fn).to(DEV)
    sc = np.float32(scale)
    for out in (torch.float16, torch.bfloat16):
        y = hip().dequantize_per_tensor_fp8(q8, s, out)
        assert_bits_equal_16(bits(y), oracle.dequant_fp8_tensor(np.tile(codes8, 3), sc,
                                                                 CODE_OF[out]),
                             CODE_OF[out], f"fp8 codes x {scale}")
        qi = torch.from_numpy(np.tile(codes8.view(np.int8), 3)).to(DEV)
        y = hip().dequantize_per_tensor_int8(qi, s, out)
        assert_bits_equal_16(bits(y), oracle.dequant_int8_tensor(np.tile(codes8.view(np.int8), 3),
                                                                 sc, CODE_OF[out]),
                             CODE_OF[out], f"int8 codes x {scale}")


def test_special_values_per_tensor():
    """NaN is ignored by amax and encodes as NaN (FP8) / 0 (INT8); inf
    saturates FP8 to 448 when amax is finite... and forces inv = 0 when it is
    the maximum."""
    for code in (oracle.BF16, oracle.F16):
        base = np.array([1.0, -2.5, 0.0, -0.0, 3.0, np.nan, 1e-8, -1e-8], np.float32)
        x = oracle.from_f32(np.tile(base, 37), code)
        check_fp8_tensor(x, code, what="nan")
        check_int8_tensor(x, code, what="nan")
        xi = oracle.from_f32(np.tile(np.array([1.0, np.inf, -3.0, 0.5], np.float32), 9), code)
        check_fp8_tensor(xi, code, what="inf")
        check_int8_tensor(xi, code, what="inf")
        z = oracle.from_f32(np.zeros(100, np.float32), code)
        check_fp8_tensor(z, code, what="zeros")
        check_int8_tensor(z, code, what="zeros")


# ---------------------------------------------------------------------------
# every kernel shape, tails, unaligned views
# ---------------------------------------------------------------------------
@pytest.mark.parametrize("n", [1, 7, 8, 9, 15, 16, 17, 2047, 2049, 4096 * 3 + 5, 1 << 20,
                               (1 << 21) + 13])
@pytest.mark.parametrize("code", [oracle.BF16, oracle.F16])
def test_tensor_sizes(n, code):
    x = rand_bits((n,), code, seed=n, scale=3.0)
    check_fp8_tensor(x, code, what=f"fp8 n={n}")
    check_int8_tensor(x, code, what=f"int8 n={n}")


@pytest.mark.parametrize("n", [(1 << 25) - 8, (1 << 25) + 13])
def test_tensor_sizes_dequant_chunking(n):
    """Either side of the size where the per-tensor dequant switches from 4
    to 2 chunks of 8 codes per thread (2^25 codes), with a ragged tail."""
    x = rand_bits((n,), oracle.BF16, seed=n, scale=3.0)
    check_fp8_tensor(x, oracle.BF16, what=f"fp8 n={n}")
    check_int8_tensor(x, oracle.BF16, what=f"int8 n={n}")


@pytest.mark.parametrize("n", [5, 1000, 65537])
def test_tensor_fp32_int8(n):
    check_int8_tensor(rand_bits((n,), oracle.F32, seed=n, scale=2.0), oracle.F32, what="f32")


ROW_LENGTHS = [8, 16, 32, 64, 128, 256, 512, 1024, 2048, 4096, 8192, 16384,   # fast shapes
               24, 40, 56, 96, 112, 136, 224, 448, 896, 1000, 1792, 2040, 2056,  # masked slots
               3000, 3584,
               4104, 5120, 11008, 14336, 28672, 65536,                           # one workgroup
               1, 3, 7, 33, 100, 129, 1001, 2047,                                # element loads
               3004, 65544]                                                      # generic


@pytest.mark.parametrize("L", ROW_LENGTHS)
@pytest.mark.parametrize("code", [oracle.BF16, oracle.F16, oracle.F32])
def test_rows_every_length(L, code):
    rows = max(3, min(257, (1 << 19) // L))
    x = rand_bits((rows, L), code, seed=L * 7 + code, rowfac=True)
    check_int8_channel(x, code, 0, what=f"channel rows={rows} L={L}")
    if L <= 4096:
        check_int8_group(x, code, L, what=f"group G={L}")


# Few long rows (per-channel axis 0): each row is cut into slices spread over
# the CUs and the slices' maxima combined; an outlier planted at a different
# position of each row lands in different slices.
@pytest.mark.parametrize("shape", [(1, 1 << 20), (4, 1 << 17), (5, 20000), (16, 16384),
                                   (3, 3 * 65536 + 8), (300, 65544)])
@pytest.mark.parametrize("code", [oracle.BF16, oracle.F16, oracle.F32])
def test_rows_split(shape, code):
    R, L = shape
    x = rand_bits(shape, code, seed=R + L + code, rowfac=True)
    v = oracle.to_f32(x.reshape(shape), code)
    for r in range(R):
        v[r, (r * 7919 * 8 + L - 1) % L] *= 30.0
    x2 = oracle.from_f32(v, code).reshape(shape) if code != oracle.F32 else v
    check_int8_channel(x2, code, 0, what=f"split rows {shape}")


@pytest.mark.parametrize("shape,axis", [((6, 1 << 17), 0), ((40000, 64), 1)])
def test_split_and_narrow_special_values(shape, axis):
    """NaN, +-inf, all-zero and subnormal rows / columns through the split-row
    path (few long rows, axis 0) and the narrow-column path (axis 1),
    bit-exact against the oracle for codes, scales and the dequant."""
    v = torch.randn(*shape, generator=torch.Generator().manual_seed(12)).bfloat16()
    if axis == 0:
        v[0, 70000] = float("nan")          # one NaN in a late slice
        v[1, 5] = float("inf")
        v[1, 130000] = -float("inf")
        v[2, :] = 0.0
        v[3, :] = 1e-39                      # bf16 subnormal
        v[4, 100000:] = float("nan")         # a whole slice of NaN
    else:
        v[7, 3] = float("nan")
        v[30000, 9] = float("inf")
        v[39999, 9] = -float("inf")
        v[:, 20] = 0.0
        v[:, 21] = 1e-39
        v[:20000, 40] = float("nan")
    check_int8_channel(bits(v), oracle.BF16, axis, what=f"special {shape} axis {axis}")


def test_rows_split_needs_its_workspace():
    """Through the C ABI: with only the control block as workspace the
    few-long-rows call takes the one-workgroup-per-row path, with the
    workspace its size query names it takes the split path; both give the
    oracle's codes and scales."""
    from cublade_amd import _abi
    L = _abi.lib()
    R, Lr = 4, 1 << 17
    code = oracle.BF16
    x = rand_bits((R, Lr), code, seed=77, rowfac=True)
    xt = from_bits(x.reshape(-1), code, DEV)
    qo, so = oracle.quant_int8_channel(x.reshape(R, Lr), code, axis=0)
    need = L.cbq_quant_int8_channel_ws_bytes(R, Lr, 0)
    assert need > _abi.WS_CTRL_BYTES
    h = torch.cuda.current_stream().cuda_stream
    for nbytes in (_abi.WS_CTRL_BYTES, need):
        ws = torch.zeros(nbytes, dtype=torch.uint8, device=DEV)
        q = torch.empty(R * Lr, dtype=torch.int8, device=DEV)
        sc = torch.empty(R, dtype=torch.float32, device=DEV)
        rc = L.cbq_quant_int8_channel(xt.data_ptr(), code, R, Lr, 0, 1e-12, ws.data_ptr(),
                                      ws.numel(), q.data_ptr(), sc.data_ptr(), h)
        assert rc == 0, L.cbq_last_error()
        torch.cuda.synchronize()
        assert_array_equal(bits(q).reshape(R, Lr), qo, f"ws {nbytes} q")
        assert_scales_equal(bits(sc), so, f"ws {nbytes}")


@pytest.mark.parametrize("shape", [(5, 8), (37, 29), (64, 2048), (1000, 24), (3, 16384),
                                   (4097, 136), (300, 1),
                                   # narrow rows (cols / 8 <= 128 chunks): several rows
                                   # per workgroup pass, 2 .. 32 threads per chunk
                                   (20000, 64), (4096, 256), (3000, 1000), (50000, 8),
                                   (7, 64), (10001, 24), (2048, 40), (1000, 1016),
                                   (70000, 16),
                                   # narrow rows without 16-byte loads: one element per
                                   # thread, several rows per workgroup pass
                                   (20000, 60), (5000, 37), (3000, 127), (70000, 5), (9, 100)])
@pytest.mark.parametrize("code", [oracle.BF16, oracle.F16, oracle.F32])
def test_columns(shape, code):
    x = rand_bits(shape, code, seed=sum(shape) + code)
    x2 = x.reshape(shape)
    # a few planted column outliers
    v = oracle.to_f32(x2, code)
    v[:, :: max(1, shape[1] // 3)] *= 20.0
    x2 = oracle.from_f32(v, code).reshape(shape) if code != oracle.F32 else v
    check_int8_channel(x2, code, 1, what=f"cols {shape}")


@pytest.mark.parametrize("offset", [1, 2, 3, 4, 5, 8])
def test_unaligned_views(offset):
    """Contiguous views that start off a 16-byte boundary take the scalar paths."""
    code = oracle.BF16
    n = 4096
    base = rand_bits((n + offset,), code, seed=99 + offset, scale=2.0)
    xt = from_bits(base, code, DEV)[offset:]
    x = base[offset:]
    q, s = hip().quantize_per_tensor_fp8(xt)
    qo, so = oracle.quant_fp8_tensor(x, code)
    assert_fp8_equal(bits(q), qo, "unaligned fp8")
    q, s = hip().quantize_per_tensor_int8(xt)
    qo, so = oracle.quant_int8_tensor(x, code)
    assert_array_equal(bits(q), qo, "unaligned int8")
    y = hip().dequantize_per_tensor_int8(q[offset:], s, torch.bfloat16)
    assert_bits_equal_16(bits(y), oracle.dequant_int8_tensor(qo[offset:], so, code), code,
                         "unaligned dequant")
    rows, L = 31, 128
    xt2 = xt[: rows * L].view(rows, L)
    x2 = x[: rows * L].reshape(rows, L)
    q, s = hip().quantize_per_group_int8(xt2, L)
    qo, so = oracle.quant_int8_group(x2, code, L)
    assert_array_equal(bits(q), qo, "unaligned group")
    qb = torch.zeros(rows * L + offset, dtype=torch.int8, device=DEV)
    qb[offset:].copy_(q.reshape(-1))
    y = hip().dequantize_per_group_int8(qb[offset:].view(rows, L), s, L, torch.bfloat16)
    assert_bits_equal_16(bits(y), oracle.dequant_int8_group(qo, so, L, oracle.BF16),
                         oracle.BF16, "unaligned group dequant")
    q, s = hip().quantize_per_channel_int8(xt2, axis=1)
    qo, so = oracle.quant_int8_channel(x2, code, axis=1)
    assert_array_equal(bits(q), qo, "unaligned cols")


def test_workspace_reuse_many_calls():
    """The per-tensor control block is reset by every call: a sequence of
    calls on one stream with different maxima gives each its own scale."""
    code = oracle.BF16
    for i, amp in enumerate([1.0, 1000.0, 1e-3, 5.0, 5.0, 0.0, 77.0] * 3):
        x = rand_bits((3000 + 100 * i,), code, seed=500 + i, scale=amp)
        check_int8_tensor(x, code, what=f"call {i}")
        check_fp8_tensor(x, code, what=f"call {i}")


def test_side_stream():
    code = oracle.F16
    x = rand_bits((1 << 16,), code, seed=3)
    s = torch.cuda.Stream()
    with torch.cuda.stream(s):
        xt = from_bits(x, code, DEV)
        q, sc = hip().quantize_per_tensor_fp8(xt)
        y = hip().dequantize_per_tensor_fp8(q, sc, torch.float16)
    s.synchronize()
    qo, so = oracle.quant_fp8_tensor(x, code)
    assert_fp8_equal(bits(q), qo, "stream q")
    assert_bits_equal_16(bits(y), oracle.dequant_fp8_tensor(qo, so, code), code, "stream y")


def test_stream_handle_is_torchs_current_stream():
    """The launch stream the bindings pass is torch's current stream, on the
    default stream and inside a side stream."""
    from cublade_amd import _abi
    dev = torch.device(DEV, torch.cuda.current_device())
    assert _abi.stream_handle(dev) == torch.cuda.current_stream(dev).cuda_stream
    s = torch.cuda.Stream()
    with torch.cuda.stream(s):
        assert _abi.stream_handle(dev) == s.cuda_stream
        assert _abi.stream_handle(torch.device(DEV)) == s.cuda_stream
    assert _abi.stream_handle(dev) == torch.cuda.current_stream(dev).cuda_stream


# ---------------------------------------------------------------------------
# public API
# ---------------------------------------------------------------------------
def test_api_group_non_last_axis_and_nd():
    from cublade_amd.quantization import dequantize_tensor, quantize_tensor
    code = oracle.BF16
    x = rand_bits((64, 6, 32), code, seed=11)
    xt = from_bits(x.reshape(-1), code, DEV).view(64, 6, 32)
    qt = quantize_tensor(xt, dtype=torch.int8, mode="group", group_size=32, ch_axis=0)
    moved = np.ascontiguousarray(np.moveaxis(x.reshape(64, 6, 32), 0, -1))
    qo, so = oracle.quant_int8_group(moved, code, 32)
    assert_array_equal(bits(qt.data), np.moveaxis(qo.reshape(6, 32, 64), -1, 0), "group axis 0")
    y = dequantize_tensor(qt)
    yo = oracle.dequant_int8_group(qo, so, 32, code).reshape(6, 32, 64)
    assert_bits_equal_16(bits(y), np.moveaxis(yo, -1, 0), code, "group axis 0 y")
    qt = quantize_tensor(xt, dtype=torch.int8, mode="channel", ch_axis=-1)
    qo, so = oracle.quant_int8_channel(x.reshape(-1, 32), code, axis=1)
    assert_array_equal(bits(qt.data), qo, "channel last axis")
    assert tuple(qt.scale.shape) == (32,)
    assert_bits_equal_16(bits(dequantize_tensor(qt)),
                         oracle.dequant_int8_channel(qo, so, code, axis=1), code, "channel last y")


def test_api_errors():
    from cublade_amd.quantization import QuantizedTensor, dequantize_tensor, quantize_tensor
    x = torch.randn(16, 32, device=DEV).bfloat16()
    with pytest.raises(NotImplementedError):
        quantize_tensor(x, scheme="asymmetric")
    with pytest.raises(ValueError):
        quantize_tensor(x, dtype=torch.float8_e4m3fn, mode="channel")
    with pytest.raises(ValueError):
        quantize_tensor(x.float(), dtype=torch.float8_e4m3fn)
    with pytest.raises(ValueError):
        quantize_tensor(x.t(), dtype=torch.int8)
    with pytest.raises(ValueError):
        quantize_tensor(x, dtype=torch.int8, mode="group", group_size=5, ch_axis=-1)
    with pytest.raises(RuntimeError):
        quantize_tensor(torch.randn(2, 5000, device=DEV).bfloat16().view(-1, 5000),
                        dtype=torch.int8, mode="group", group_size=5000, ch_axis=-1)
    with pytest.raises(IndexError):
        quantize_tensor(torch.randn(4, 5, 6, device=DEV), dtype=torch.int8, mode="channel",
                        ch_axis=3)
    with pytest.raises(ValueError):
        quantize_tensor(torch.randn(4, 6, 5, device=DEV), dtype=torch.int8, mode="group",
                        group_size=4, ch_axis=1)
    qt = quantize_tensor(x, dtype=torch.float8_e4m3fn)
    bad = QuantizedTensor(qt.data, qt.scale, qt.zero_point, "channel", 0, 32, qt.dtype,
                          torch.bfloat16)
    with pytest.raises(NotImplementedError):
        dequantize_tensor(bad)
    bad = QuantizedTensor(qt.data, qt.scale, qt.zero_point, "tensor", 0, 32, qt.dtype,
                          torch.float32)
    with pytest.raises(ValueError):
        dequantize_tensor(bad)


def test_empty_inputs():
    from cublade_amd.quantization import dequantize_tensor, quantize_tensor
    e = torch.zeros(0, dtype=torch.bfloat16, device=DEV)
    for dt in (torch.float8_e4m3fn, torch.int8):
        qt = quantize_tensor(e, dtype=dt)
        assert qt.data.numel() == 0 and qt.scale.item() == 0.0
        assert dequantize_tensor(qt).numel() == 0
    q, s = hip().quantize_per_channel_int8(torch.zeros(0, 8, device=DEV))
    assert q.shape == (0, 8) and s.shape == (0,)
    q, s = hip().quantize_per_group_int8(torch.zeros(0, 32, device=DEV), 32)
    assert q.shape == (0, 32) and s.shape == (0,)


# ---------------------------------------------------------------------------
# BASELINE configurations at full size (bit-exact against the oracle)
# ---------------------------------------------------------------------------
def test_config1_fp8_full():
    g = torch.Generator().manual_seed(0)
    x = torch.randn(4096, 4096, generator=g).bfloat16()
    check_fp8_tensor(bits(x).reshape(-1), oracle.BF16, shape=(4096, 4096), what="C1")


def test_config2_int8_tensor_full():
    g = torch.Generator().manual_seed(1)
    shape = (8192, 8192)
    z = torch.randn(*shape, generator=g)
    c = [torch.randn(*shape, generator=g) for _ in range(3)]
    t = z / torch.sqrt((c[0] ** 2 + c[1] ** 2 + c[2] ** 2) / 3)
    x = (0.5 * t).half()
    assert torch.isfinite(x).all()
    check_int8_tensor(bits(x).reshape(-1), oracle.F16, what="C2")


@pytest.mark.parametrize("axis", [0, 1])
def test_config3_int8_channel_full(axis):
    g = torch.Generator().manual_seed(2)
    w = 0.02 * torch.randn(28672, 8192, generator=g)
    cols = torch.randperm(8192, generator=g)[:8]
    w[:, cols] *= 20
    x = bits(w.bfloat16())
    del w
    check_int8_channel(x, oracle.BF16, axis, what=f"C3 axis {axis}")


def test_config4_int8_group_full():
    g = torch.Generator().manual_seed(3)
    x = torch.randn(16384, 14336, generator=g)
    x *= (0.1 + 9.9 * torch.rand(16384, 1, generator=g))
    xb = bits(x.bfloat16())
    del x
    check_int8_group(xb.reshape(-1, 128), oracle.BF16, 128, what="C4")


# ---------------------------------------------------------------------------
# N-D axes without transposing copies (channel on any axis, groups along any
# axis): bit-exact against the oracle applied to the moved tensor
# ---------------------------------------------------------------------------
@pytest.mark.parametrize("code", [oracle.BF16, oracle.F16, oracle.F32])
@pytest.mark.parametrize("shape,axis", [
    # inner < 512: column maxima per row block over the [outer, C * inner] view
    ((6, 40, 24), 1), ((3, 5, 7, 8), 2), ((3, 5, 7, 8), 1), ((64, 3, 5), 1), ((2, 300, 3), 1),
    ((5, 1, 9), 1),
    # inner >= 512: one wave per contiguous segment (vector and scalar loads)
    ((3, 17, 512), 1), ((2, 5, 1000), 1), ((4, 3, 1001), 1), ((3, 2, 600, 2), 1),
    ((9, 2, 8192), 1),
    # 512 .. 8192 chunks of 8 per channel: one workgroup per channel, held in
    # registers (1, 2, 3 -> 4, 14 -> 16 and 16 chunks per thread)
    ((2, 8, 2048), 1), ((2, 64, 4096), 1), ((3, 10, 2048), 1), ((2, 9, 3, 1600), 1),
    ((7, 6, 8192), 1), ((16, 3, 4096), 1),
    # leading axis with few long channels: rows cut into slices over the CUs
    ((4, 64, 1024), 0), ((2, 3, 70000), 0),
    # narrow [outer, C * inner] views: several rows per workgroup pass
    ((64, 30, 64), 2), ((100, 4, 16), 1), ((3000, 2, 8), 1), ((500, 8, 3), 1),
    ((400, 5, 3), 1), ((2000, 13), 1)])
def test_channel_any_axis(code, shape, axis):
    from cublade_amd.quantization import dequantize_tensor, quantize_tensor
    x = rand_bits(shape, code, seed=sum(shape) + axis)
    xt = from_bits(x.reshape(-1), code, DEV).view(*shape)
    qt = quantize_tensor(xt, dtype=torch.int8, mode="channel", ch_axis=axis)
    C = shape[axis]
    moved = np.ascontiguousarray(np.moveaxis(x.reshape(shape), axis, 0)).reshape(C, -1)
    qo, so = oracle.quant_int8_channel(moved, code, axis=0)
    mshape = (C,) + tuple(d for i, d in enumerate(shape) if i != axis)
    assert_array_equal(bits(qt.data), np.moveaxis(qo.reshape(mshape), 0, axis), "channel nd q")
    assert tuple(qt.scale.shape) == (C,)
    assert_array_equal(bits(qt.scale).view(np.uint32), np.asarray(so, np.float32).view(np.uint32),
                       "channel nd scale")
    out = oracle.BF16 if code == oracle.F32 else code
    qt.original_dtype = DTYPE_OF[out]
    y = dequantize_tensor(qt)
    yo = oracle.dequant_int8_channel(qo, so, out, axis=0).reshape(mshape)
    assert_bits_equal_16(bits(y), np.moveaxis(yo, 0, axis), out, "channel nd y")


@pytest.mark.parametrize("code", [oracle.BF16, oracle.F16, oracle.F32])
@pytest.mark.parametrize("shape,axis,G", [
    # inner % 8 != 0: one thread per group
    ((6, 64, 3), 1, 32), ((4, 128, 100), 1, 128), ((2, 8, 6, 5), 2, 2), ((96, 7), 0, 32),
    ((2, 4096, 2), 1, 4096),
    # inner == 1: contiguous rows
    ((3, 256, 1), 1, 64),
    # tiled: 8 / 4 / 2 / 1 waves per group, groups held in registers (<= 16
    # positions per wave) or read twice, partial inner tiles
    ((256, 64), 0, 32), ((6, 96, 520), 1, 96), ((512, 1024), 0, 128), ((2, 384, 16), 1, 384),
    ((136, 8), 0, 136), ((3, 10, 24), 1, 5), ((4, 36, 8), 1, 6), ((2, 12, 1032), 1, 12),
    # group-major scale scratch with 8 waves per group and a walk that is not a
    # power of two (3 and 12 positions, clamped to 4 and 16), partial inner tile
    ((3, 48, 8), 1, 24), ((2, 192, 520), 1, 96), ((5, 64, 16), 1, 8),
    # 16 waves per group (G > 128): held in registers up to 256, read twice beyond
    ((512, 520), 0, 256), ((2, 480, 24), 1, 160), ((1024, 64), 0, 512)])
def test_group_any_axis(code, shape, axis, G):
    from cublade_amd.quantization import dequantize_tensor, quantize_tensor
    x = rand_bits(shape, code, seed=sum(shape) * 3 + axis + G)
    xt = from_bits(x.reshape(-1), code, DEV).view(*shape)
    qt = quantize_tensor(xt, dtype=torch.int8, mode="group", group_size=G, ch_axis=axis)
    moved = np.ascontiguousarray(np.moveaxis(x.reshape(shape), axis, -1))
    qo, so = oracle.quant_int8_group(moved.reshape(-1, G), code, G)
    assert_array_equal(bits(qt.data), np.moveaxis(qo.reshape(moved.shape), -1, axis), "group nd q")
    assert_array_equal(bits(qt.scale).view(np.uint32), np.asarray(so, np.float32).view(np.uint32),
                       "group nd scale")
    out = oracle.BF16 if code == oracle.F32 else code
    qt.original_dtype = DTYPE_OF[out]
    y = dequantize_tensor(qt)
    yo = oracle.dequant_int8_group(qo, so, G, out).reshape(moved.shape)
    assert_bits_equal_16(bits(y), np.moveaxis(yo, -1, axis), out, "group nd y")


@pytest.mark.parametrize("shape,axis,G", [
    ((256, 64), 0, 32), ((6, 96, 520), 1, 32), ((512, 1024), 0, 128), ((2, 12, 1032), 1, 4),
    ((3, 70, 136), 1, 7), ((4, 200, 72), 1, 2)])
def test_group_nd_scale_scratch_and_direct_agree(shape, axis, G):
    """The tiled group quant kernels write the scales either through group-major
    workspace scratch and a transposing pass (the API's path) or, without a
    workspace, directly in the movedim order: same codes and scale bits. The
    first path is pinned to the oracle by test_group_any_axis."""
    from cublade_amd import _abi
    from cublade_amd.bindings.hip.quantize_int8 import quantize_per_group_int8_nd
    x = rand_bits(shape, oracle.BF16, seed=sum(shape) + G)
    xt = from_bits(x.reshape(-1), oracle.BF16, DEV).view(*shape)
    print(f"[group scratch] shape={shape} axis={axis} G={G}", flush=True)
    q1, s1 = quantize_per_group_int8_nd(xt, axis, G)
    outer = int(np.prod(shape[:axis], dtype=np.int64))
    inner = int(np.prod(shape[axis + 1:], dtype=np.int64))
    L = _abi.lib()
    assert L.cbq_quant_int8_group_nd_ws_bytes(outer, shape[axis], inner, G) > _abi.WS_CTRL_BYTES
    q2 = torch.empty_like(q1)
    s2 = torch.empty_like(s1)
    rc = L.cbq_quant_int8_group_nd(_abi.ptr(xt), _abi.DTYPE_CODE[torch.bfloat16], outer,
                                   shape[axis], inner, G, 1e-12, None, 0, _abi.ptr(q2),
                                   _abi.ptr(s2), _abi.stream_handle(xt.device))
    _abi.check(rc, "group nd without workspace")
    # with the workspace again, the scales written one float past a 16-byte
    # boundary (the transposing pass's 4-byte store path)
    q3 = torch.empty_like(q1)
    s3 = torch.empty(s1.numel() + 1, dtype=torch.float32, device=xt.device)
    nb = L.cbq_quant_int8_group_nd_ws_bytes(outer, shape[axis], inner, G)
    ws = torch.zeros(nb, dtype=torch.uint8, device=xt.device)
    rc = L.cbq_quant_int8_group_nd(_abi.ptr(xt), _abi.DTYPE_CODE[torch.bfloat16], outer,
                                   shape[axis], inner, G, 1e-12, _abi.ptr(ws), nb, _abi.ptr(q3),
                                   _abi.ptr(s3) + 4, _abi.stream_handle(xt.device))
    _abi.check(rc, "group nd, unaligned scales")
    torch.cuda.synchronize()
    assert torch.equal(q1, q2) and torch.equal(q1, q3)
    assert torch.equal(s1.view(torch.int32), s2.view(torch.int32))
    assert torch.equal(s1.view(torch.int32), s3[1:].view(torch.int32))
    # the group dequant: scales transposed into workspace scratch (the API's
    # path), read in place without a workspace, and from unaligned scales
    from cublade_amd.bindings.hip.dequantize_int8 import dequantize_per_group_int8_nd
    y1 = dequantize_per_group_int8_nd(q1, s1, axis, G, torch.bfloat16)
    assert L.cbq_dequant_int8_group_nd_ws_bytes(outer, shape[axis], inner, G) == nb
    y2, y3 = torch.empty_like(y1), torch.empty_like(y1)
    bf = _abi.DTYPE_CODE[torch.bfloat16]
    rc = L.cbq_dequant_int8_group_nd(_abi.ptr(q1), _abi.ptr(s1), outer, shape[axis], inner, G,
                                     None, 0, _abi.ptr(y2), bf, _abi.stream_handle(xt.device))
    _abi.check(rc, "group nd dequant without workspace")
    rc = L.cbq_dequant_int8_group_nd(_abi.ptr(q1), _abi.ptr(s3) + 4, outer, shape[axis], inner,
                                     G, _abi.ptr(ws), nb, _abi.ptr(y3), bf,
                                     _abi.stream_handle(xt.device))
    _abi.check(rc, "group nd dequant, unaligned scales")
    torch.cuda.synchronize()
    assert torch.equal(y1.view(torch.int16), y2.view(torch.int16))
    assert torch.equal(y1.view(torch.int16), y3.view(torch.int16))


@pytest.mark.parametrize("mode,axis", [("group", 0), ("channel", 1)])
def test_any_axis_unaligned_view(mode, axis):
    """A view whose data pointer is not 16-byte aligned takes the scalar
    kernels; codes and scales match those of an aligned copy bit for bit."""
    from cublade_amd.quantization import dequantize_tensor, quantize_tensor
    shape = (64, 4, 520)
    n = int(np.prod(shape))
    base = torch.randn(n + 1, generator=torch.Generator().manual_seed(9)).half().to(DEV)
    xv = base[1:].view(shape)
    xa = xv.clone()
    kw = dict(dtype=torch.int8, mode=mode, ch_axis=axis)
    if mode == "group":
        kw["group_size"] = 32
    qv, qa = quantize_tensor(xv, **kw), quantize_tensor(xa, **kw)
    assert_array_equal(bits(qv.data), bits(qa.data), "unaligned q")
    assert_array_equal(bits(qv.scale).view(np.uint32), bits(qa.scale).view(np.uint32),
                       "unaligned scale")
    assert_array_equal(bits(dequantize_tensor(qv)), bits(dequantize_tensor(qa)), "unaligned y")


@pytest.mark.parametrize("mode,axis,G", [("group", 0, 32), ("group", 0, 8), ("channel", 1, None)])
def test_any_axis_special_values(mode, axis, G):
    """NaN, +-inf, all-zero and subnormal columns through the tiled group
    kernels and the segment-max channel path, bit-exact against the oracle."""
    from cublade_amd.quantization import dequantize_tensor, quantize_tensor
    shape = (64, 520) if mode == "group" else (3, 4, 640)
    v = torch.randn(*shape, generator=torch.Generator().manual_seed(11)).bfloat16()
    if mode == "group":
        v[3, 5] = float("nan")
        v[40, 7] = float("inf")
        v[41, 7] = -float("inf")
        v[:, 9] = 0.0
        v[:, 10] = 1e-39          # bf16 subnormal
        v[:32, 11] = float("nan")
    else:
        v[1, 2, 5] = float("nan")
        v[2, 0, 600] = -float("inf")
        v[:, 3, :] = 0.0
        v[:, 1, :] = 1e-39
    x = bits(v)
    xt = from_bits(x.reshape(-1), oracle.BF16, DEV).view(*shape)
    if mode == "group":
        qt = quantize_tensor(xt, dtype=torch.int8, mode="group", group_size=G, ch_axis=axis)
        moved = np.ascontiguousarray(np.moveaxis(x, axis, -1))
        qo, so = oracle.quant_int8_group(moved.reshape(-1, G), oracle.BF16, G)
        qo = np.moveaxis(qo.reshape(moved.shape), -1, axis)
        yo = np.moveaxis(oracle.dequant_int8_group(np.moveaxis(qo, axis, -1).reshape(-1, G), so, G,
                                                   oracle.BF16).reshape(moved.shape), -1, axis)
    else:
        qt = quantize_tensor(xt, dtype=torch.int8, mode="channel", ch_axis=axis)
        C = shape[axis]
        mshape = (C,) + tuple(d for i, d in enumerate(shape) if i != axis)
        moved = np.ascontiguousarray(np.moveaxis(x, axis, 0)).reshape(C, -1)
        qo, so = oracle.quant_int8_channel(moved, oracle.BF16, axis=0)
        yo = np.moveaxis(oracle.dequant_int8_channel(qo, so, oracle.BF16, axis=0).reshape(mshape),
                         0, axis)
        qo = np.moveaxis(qo.reshape(mshape), 0, axis)
    assert_array_equal(bits(qt.data), qo, "special q")
    assert_array_equal(bits(qt.scale).view(np.uint32), np.asarray(so, np.float32).view(np.uint32),
                       "special scale")
    assert_bits_equal_16(bits(dequantize_tensor(qt)), yo, oracle.BF16, "special y")
