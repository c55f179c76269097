"""Every part of the one-launch per-tensor quant's step layout, on random data.

k_quant_tensor_1pass (x >= 2^20 elements) reads x in grid-wide steps of
grid * 4096 chunks of 8 elements (2^23 elements on 256 CUs). Of a thread's
steps, the last HS stay in registers ("held"), the first LS streamed ones are
parked in LDS ("parked"), and any others are read again after the exchange
("re-read"): HS = 6, LS = 2 for 2-byte inputs, HS = 3, LS = 1 for fp32.
Each case below puts the tensor's maximum in one of those parts (or in the
ragged tail of fewer than 8 elements) and compares codes, scale and the
dequantized outputs bit for bit with the oracle, so that a part that is
skipped in the maximum, or cast from the wrong chunk, fails.

Sizes: fp32 with 1 step (held only, fewer workgroups than CUs), 3 (held
only), 4 (held + parked) and 6 steps (held + parked + two re-read steps);
fp16 [10240, 8192] (10 steps: 160 MiB, past the 128 MiB that registers and
LDS hold) through INT8 and FP8.
"""
from __future__ import annotations

import gc

import pytest
import torch

import oracle
from tests._util import bits
from tests.test_gpu_quant import check_fp8_tensor, check_int8_tensor

pytestmark = pytest.mark.gpu

HOLD = {oracle.F32: 3, oracle.F16: 6, oracle.BF16: 6}
PARK = {oracle.F32: 1, oracle.F16: 2, oracle.BF16: 2}
TORCH = {oracle.F32: torch.float32, oracle.F16: torch.float16, oracle.BF16: torch.bfloat16}


@pytest.fixture(autouse=True)
def _free():
    yield
    gc.collect()
    torch.cuda.empty_cache()


def _cus() -> int:
    return torch.cuda.get_device_properties(0).multi_processor_count


def step_elems(n: int) -> int:
    """Elements per grid step of the one-launch kernel for n elements."""
    chunks = n // 8
    grid = min(-(-chunks // 4096), _cus())
    return grid * 4096 * 8


def parts(n: int, code: int) -> dict[str, tuple[int, int]]:
    """Element ranges [lo, hi) of each part of the step layout that exists."""
    se = step_elems(n)
    steps = -(-(n // 8) // (se // 8))
    held0 = max(steps - HOLD[code], 0)
    parked = min(held0, PARK[code])
    out = {"held_first": (held0 * se, min((held0 + 1) * se, n)),
           "held_last": ((steps - 1) * se, (n // 8) * 8)}
    if parked:
        out["parked"] = (0, parked * se)
    if held0 > parked:
        out["reread"] = (parked * se, held0 * se)
    if n % 8:
        out["tail"] = ((n // 8) * 8, n)
    return out


_base: dict[tuple[int, int], torch.Tensor] = {}


def base(n: int, code: int) -> torch.Tensor:
    key = (n, code)
    if key not in _base:
        _base.clear()
        g = torch.Generator().manual_seed(n % 100003)
        _base[key] = (torch.randn(n, generator=g) * 2.0).to(TORCH[code])
    return _base[key]


def run_case(n: int, code: int, where: str, fp8: bool):
    p = parts(n, code)
    if where not in p:
        pytest.skip(f"no {where} part at n={n}")
    lo, hi = p[where]
    x = base(n, code).clone()
    pos = lo + (hi - lo) * 7 // 11
    x[pos] = -40.0 if where != "held_last" else 40.0
    print(f"[1pass] n={n} code={code} {where} at {pos} steps of {step_elems(n)}", flush=True)
    xb = bits(x)
    del x
    if fp8:
        check_fp8_tensor(xb, code, what=f"fp8 n={n} max in {where}")
    else:
        check_int8_tensor(xb, code, what=f"int8 n={n} max in {where}")


WHERE = ["parked", "reread", "held_first", "held_last", "tail"]

# (n, parts present on 256 CUs): n in multiples of the 2^23-element step,
# with ragged tails
F32_CASES = [((1 << 20) + 13, ["held_first", "tail"]),   # one step, fewer workgroups than CUs
             (3 * (1 << 23) - 1000, ["held_first", "held_last"]),   # held only
             (4 * (1 << 23) - 5, ["parked", "held_first", "held_last", "tail"]),
             (6 * (1 << 23) + 3, WHERE)]                 # held + parked + two re-read steps


@pytest.mark.parametrize("n,where", [(n, w) for n, ws in F32_CASES for w in ws])
def test_fp32_int8_step_layout(n, where):
    run_case(n, oracle.F32, where, fp8=False)


@pytest.mark.parametrize("fp8", [False, True])
@pytest.mark.parametrize("where", WHERE)
def test_fp16_past_128mib(where, fp8):
    # [10240, 8192] fp16 = 160 MiB; one more odd element gives the tail case
    n = 10240 * 8192 + (3 if where == "tail" else 0)
    run_case(n, oracle.F16, where, fp8=fp8)
