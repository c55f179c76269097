"""The allocation-free entry point cbq_quant_fp8_tensor_noalloc, called
through the C ABI, against cbq_quant_fp8_tensor (the same kernels with a
caller-owned workspace) on consecutive calls that share the library's static
scratch: a large input (one-launch path), a smaller one (two-pass path, the
scratch still holding the previous call's state), and a large one again.
Codes and scale must be bit-identical; both are also checked against the CPU
oracle."""
from __future__ import annotations

import ctypes

import numpy as np
import pytest
import torch

import oracle
from tests._util import assert_fp8_equal, bits

pytestmark = pytest.mark.gpu

DEV = "cuda"


def _quant(fn_name, x, use_ws):
    from cublade_amd import _abi
    L = _abi.lib()
    q = torch.empty(x.shape, dtype=torch.uint8, device=x.device)
    scale = torch.empty((), dtype=torch.float32, device=x.device)
    code = _abi.DTYPE_CODE[x.dtype]
    stream = _abi.stream_handle(x.device)
    if use_ws:
        ws = torch.zeros(L.cbq_quant_tensor_ws_bytes(), dtype=torch.uint8, device=x.device)
        rc = getattr(L, fn_name)(x.data_ptr(), code, x.numel(), ctypes.c_float(1e-12),
                                 ws.data_ptr(), ws.numel(), q.data_ptr(), scale.data_ptr(), stream)
        _abi.check(rc, fn_name)
        torch.cuda.synchronize()
        del ws
    else:
        rc = getattr(L, fn_name)(x.data_ptr(), code, x.numel(), ctypes.c_float(1e-12),
                                 q.data_ptr(), scale.data_ptr(), stream)
        _abi.check(rc, fn_name)
        torch.cuda.synchronize()
    return bits(q), np.float32(scale.item())


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16])
def test_noalloc_matches_workspace_entry_point(dtype):
    g = torch.Generator().manual_seed(11)
    sizes = [(3 << 20) + 5, 1000, 16_777_216]
    for i, n in enumerate(sizes):
        print(f"[no-alloc] call {i}: n={n} dtype={dtype}", flush=True)
        x = (torch.randn(n, generator=g) * (1 + i)).to(dtype)
        x[n // 2] = 50.0 * (i + 1)
        xd = x.to(DEV)
        q_na, s_na = _quant("cbq_quant_fp8_tensor_noalloc", xd, use_ws=False)
        q_ws, s_ws = _quant("cbq_quant_fp8_tensor", xd, use_ws=True)
        assert_fp8_equal(q_na, q_ws, f"call {i} codes")
        assert s_na.view(np.uint32) == s_ws.view(np.uint32), (i, s_na, s_ws)
        code = oracle.BF16 if dtype == torch.bfloat16 else oracle.F16
        qo, so = oracle.quant_fp8_tensor(bits(x), code)
        assert_fp8_equal(q_na, qo, f"call {i} codes vs oracle")
        assert s_na.view(np.uint32) == np.float32(so).view(np.uint32)
