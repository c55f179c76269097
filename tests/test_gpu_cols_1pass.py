"""The one-launch per-column (axis 1) quant, against the oracle, bit for bit.

k_quant_cols_1pass takes rows of 8192, 16384 or 32768 elements (x of 2^22
elements up to 480 MiB, 16-byte aligned; larger x takes the two-pass path,
which the full config-3 test covers): the per-tensor one-launch step layout
(grid-wide steps of 2^23 elements on 256 CUs; the last HS steps of each
thread held in registers, the first LS streamed ones parked in LDS, the
others read again after the exchange) with per-column running maxima, then
two grid-wide exchanges (partial column maxima; the multipliers of each
workgroup's slice of columns). Random data puts each column's maximum in a
random row, so across the columns every part of the layout holds some
column's maximum; explicit outlier columns are added in the parked, re-read,
first held and last held parts. Codes, scales and the dequantized outputs are
compared bit for bit with the oracle, through the public API
(quantize_tensor(..., mode="channel", ch_axis=1)) and through the C ABI.

Sizes (hold steps HS / parked LS per row length and dtype): one partial step
(fewer workgroups with data than CUs), held only, held + parked, and held +
parked + re-read with a ragged last step, for each row length; fp32 as well.
"""
from __future__ import annotations

import gc

import numpy as np
import pytest
import torch

import oracle
from tests._util import (CODE_OF, assert_array_equal, assert_bits_equal_16, assert_scales_equal,
                         bits, from_bits)

pytestmark = pytest.mark.gpu

TORCH = {oracle.F32: torch.float32, oracle.F16: torch.float16, oracle.BF16: torch.bfloat16}
HOLD = {(2, 1): 6, (2, 2): 5, (2, 4): 3, (4, 1): 3, (4, 2): 2, (4, 4): 1}   # (bytes, CPT) -> HS
PARK = {2: 2, 4: 1}


@pytest.fixture(autouse=True)
def _free():
    yield
    gc.collect()
    torch.cuda.empty_cache()


def _grid() -> int:
    cus = torch.cuda.get_device_properties(0).multi_processor_count
    g = 1
    while 2 * g <= cus and 2 * g <= 1920:
        g *= 2
    return g


def layout(rows: int, cols: int, code: int) -> dict[str, tuple[int, int]]:
    """Row ranges [lo, hi) of each part of the step layout that exists."""
    eb = 4 if code == oracle.F32 else 2
    cpt = cols // 8192
    step_rows = _grid() * 4096 * 8 // cols
    steps = -(-rows // step_rows)
    held0 = max(steps - HOLD[(eb, cpt)], 0)
    parked = min(held0, PARK[eb])
    out = {"held_first": (held0 * step_rows, min((held0 + 1) * step_rows, rows)),
           "held_last": ((steps - 1) * step_rows, rows)}
    if parked:
        out["parked"] = (0, parked * step_rows)
    if held0 > parked:
        out["reread"] = (parked * step_rows, held0 * step_rows)
    return out


def make_x(rows: int, cols: int, code: int, seed: int) -> np.ndarray:
    g = torch.Generator().manual_seed(seed)
    x = torch.randn(rows, cols, generator=g) * 0.05
    # columns whose maximum sits in a chosen part of the layout
    for k, (lo, hi) in enumerate(layout(rows, cols, code).values()):
        for j in range(3):
            c = (977 * (3 * k + j) + 13) % cols
            r = lo + (hi - lo) * (j + 1) // 4
            x[r, c] = (-1) ** j * (30.0 + k + j)
    return bits(x.to(TORCH[code]))


def check(rows: int, cols: int, code: int, seed: int, via_api: bool):
    from cublade_amd import _abi
    from cublade_amd.quantization import dequantize_tensor, quantize_tensor
    xb = make_x(rows, cols, code, seed)
    print(f"[cols1] rows={rows} cols={cols} code={code} api={via_api} parts="
          f"{sorted(layout(rows, cols, code))}", flush=True)
    qo, so = oracle.quant_int8_channel(xb.reshape(rows, cols), code, axis=1)
    xt = from_bits(xb.reshape(-1), code, "cuda").view(rows, cols)
    if via_api:
        qt = quantize_tensor(xt, dtype=torch.int8, mode="channel", ch_axis=1)
        q, s = qt.data, qt.scale
    else:
        L = _abi.lib()
        ws = torch.zeros(L.cbq_quant_int8_channel_ws_bytes(rows, cols, 1), dtype=torch.uint8,
                         device="cuda")
        q = torch.empty(rows, cols, dtype=torch.int8, device="cuda")
        s = torch.empty(cols, dtype=torch.float32, device="cuda")
        import ctypes
        for _ in range(2):   # the second call reuses the control block
            _abi.check(L.cbq_quant_int8_channel(xt.data_ptr(), _abi.DTYPE_CODE[TORCH[code]], rows,
                                                cols, 1, ctypes.c_float(1e-12), ws.data_ptr(),
                                                ws.numel(), q.data_ptr(), s.data_ptr(),
                                                _abi.stream_handle(torch.device("cuda"))),
                       "channel axis 1")
    assert_array_equal(bits(q), qo, f"codes rows={rows} cols={cols}")
    assert_scales_equal(bits(s), so, f"scales rows={rows} cols={cols}")
    if via_api and code != oracle.F32:   # dequant outputs fp16 / bf16 only
        out = TORCH[code]
        y = dequantize_tensor(qt)
        assert y.dtype == out
        assert_bits_equal_16(bits(y), oracle.dequant_int8_channel(qo, so, CODE_OF[out], axis=1),
                             CODE_OF[out], "dequant")


CASES = [
    # cols 8192 (one 1024-row grid step on 256 CUs), 2-byte: HS 6, LS 2
    (512, 8192, oracle.BF16),          # one partial step
    (6144, 8192, oracle.F16),          # held only
    (8192, 8192, oracle.BF16),         # held + parked (128 MiB: all on chip)
    (13000, 8192, oracle.BF16),        # + re-read steps, ragged last step
    # cols 16384 (512-row steps): HS 5
    (2048, 16384, oracle.F16),
    (4100, 16384, oracle.BF16),
    # cols 32768 (256-row steps): HS 3
    (1024, 32768, oracle.BF16),
    (2049, 32768, oracle.F16),
    # fp32: HS 3 / 2 / 1, LS 1
    (5000, 8192, oracle.F32),
    (2600, 16384, oracle.F32),
    (1300, 32768, oracle.F32),
]


@pytest.mark.parametrize("rows,cols,code", CASES)
def test_cols_1pass_api(rows, cols, code):
    check(rows, cols, code, seed=rows + cols, via_api=True)


@pytest.mark.parametrize("rows,cols,code", [(13000, 8192, oracle.BF16), (2049, 32768, oracle.F16)])
def test_cols_1pass_abi_repeated(rows, cols, code):
    check(rows, cols, code, seed=7 * rows + cols, via_api=False)


@pytest.mark.parametrize("code", [oracle.BF16, oracle.F16, oracle.F32])
def test_cols_1pass_special_values(code):
    """NaN (ignored by the column maxima, encoded as 0), +-inf (a column
    with inf gets scale inf and codes 0 / +-127 as the oracle defines), an
    all-zero column (amax = 0: the eps floor), all-NaN and subnormal columns,
    and -0, through the one-launch path ([2048, 8192]: 16M elements, held
    steps only for 2-byte input, held + parked for fp32)."""
    rows, cols = 2048, 8192
    g = torch.Generator().manual_seed(77)
    v = torch.randn(rows, cols, generator=g) * 0.1
    v[5, 3] = float("nan")
    v[1000, 3] = 2.0                       # the column's maximum despite the NaN
    v[7, 11] = float("inf")
    v[1500, 12] = -float("inf")
    v[:, 20] = 0.0                         # all zero
    v[:, 21] = float("nan")                # all NaN
    v[:, 22] = 1e-7 if code == oracle.F16 else 1e-39   # subnormal in the input dtype
    v[:, 23] = -0.0
    v[2047, 8191] = -40.0                  # last element of x
    xb = bits(v.to(TORCH[code]))
    qo, so = oracle.quant_int8_channel(xb.reshape(rows, cols), code, axis=1)
    from cublade_amd.quantization import quantize_tensor
    qt = quantize_tensor(from_bits(xb.reshape(-1), code, "cuda").view(rows, cols),
                         dtype=torch.int8, mode="channel", ch_axis=1)
    assert_array_equal(bits(qt.data), qo, "codes")
    assert_scales_equal(bits(qt.scale), so, "scales")


def _random_cases(n=6, seed=2024):
    """Seeded random shapes that take the one-launch path: width 8192 /
    16384 / 32768, a row count giving 2^22 elements up to ~320 MiB, any
    dtype."""
    rng = np.random.default_rng(seed)
    cases = []
    for _ in range(n):
        cols = int(rng.choice([8192, 16384, 32768]))
        code = int(rng.choice([oracle.BF16, oracle.F16, oracle.F32]))
        eb = 4 if code == oracle.F32 else 2
        lo, hi = (1 << 22) // cols, (320 << 20) // (cols * eb)
        cases.append((int(rng.integers(lo, hi)), cols, code, int(rng.integers(1 << 30))))
    return cases


@pytest.mark.parametrize("rows,cols,code,seed", _random_cases())
def test_cols_1pass_random(rows, cols, code, seed):
    g = torch.Generator().manual_seed(seed)
    x = torch.randn(rows, cols, generator=g) * torch.exp(torch.randn(1, cols, generator=g))
    k = max(1, cols // 1000)                # a few outlier columns at random rows
    oc = torch.randperm(cols, generator=g)[:k]
    orow = torch.randint(0, rows, (k,), generator=g)
    x[orow, oc] *= 50.0
    xb = bits(x.to(TORCH[code]))
    print(f"[cols1 random] rows={rows} cols={cols} code={code} seed={seed}", flush=True)
    qo, so = oracle.quant_int8_channel(xb.reshape(rows, cols), code, axis=1)
    from cublade_amd.quantization import quantize_tensor
    qt = quantize_tensor(from_bits(xb.reshape(-1), code, "cuda").view(rows, cols),
                         dtype=torch.int8, mode="channel", ch_axis=1)
    assert_array_equal(bits(qt.data), qo, "codes")
    assert_scales_equal(bits(qt.scale), so, "scales")
