"""Failure handling of the one-launch per-tensor quant, forced from the host.

k_quant_tensor_1pass exchanges workgroup maxima through tagged slots and
gives up after a bounded number of polls. CBQ_TENSOR_SPIN_LIMIT=0 (read by
the library at its first call) makes every workgroup give up after its first
poll, so the early finishers time out while every kernel still ends
normally. A child process (fresh library state) checks that:
  * the call sets the sticky status word of the workspace's control block
    (byte offset 512) to 1;
  * the next call on that workspace is poisoned: every code is NaN (FP8) or
    0 (INT8) and the scale is NaN, with no exchange;
  * a fresh, zero-filled workspace in a normal process gives exact results
    (covered by every other per-tensor test).
"""
from __future__ import annotations

import os
import subprocess
import sys
import textwrap
from pathlib import Path

import pytest

pytestmark = pytest.mark.gpu

ROOT = Path(__file__).resolve().parents[1]

CHILD = textwrap.dedent("""
    import ctypes, sys
    sys.path.insert(0, {root!r})
    import torch
    from cublade_amd import _abi
    L = _abi.lib()
    dev = torch.device("cuda:0")
    g = torch.Generator().manual_seed(5)
    n = 16 * 1024 * 1024
    x = torch.randn(n, generator=g).to(torch.bfloat16).to(dev)
    ws = torch.zeros(L.cbq_quant_tensor_ws_bytes(), dtype=torch.uint8, device=dev)
    def call(fp8):
        q = torch.empty(n, dtype=torch.uint8, device=dev)
        s = torch.empty((), dtype=torch.float32, device=dev)
        fn = L.cbq_quant_fp8_tensor if fp8 else L.cbq_quant_int8_tensor
        rc = fn(x.data_ptr(), _abi.BF16, n, ctypes.c_float(1e-12), ws.data_ptr(), ws.numel(),
                q.data_ptr(), s.data_ptr(), _abi.stream_handle(dev))
        _abi.check(rc, "quant")
        torch.cuda.synchronize()
        return q, s
    call(True)
    status = int(ws[512:516].view(torch.int32).item())
    print("status after forced timeout:", status, flush=True)
    assert status == 1, status
    q, s = call(True)
    assert torch.isnan(s).item(), s
    assert bool(((q & 0x7F) == 0x7F).all()), "poisoned FP8 codes must all be NaN"
    q, s = call(False)
    assert torch.isnan(s).item(), s
    assert bool((q == 0).all()), "poisoned INT8 codes must all be 0"
    print("POISON_OK", flush=True)
""")


def test_forced_exchange_timeout_sets_status_and_poisons():
    env = dict(os.environ, CBQ_TENSOR_SPIN_LIMIT="0", CUBLADE_SKIP_WARMUP="1")
    print("[timeout] child with CBQ_TENSOR_SPIN_LIMIT=0", flush=True)
    proc = subprocess.run([sys.executable, "-c", CHILD.format(root=str(ROOT))], env=env,
                          capture_output=True, text=True, timeout=120)
    print(proc.stdout[-2000:], proc.stderr[-2000:], flush=True)
    assert proc.returncode == 0, proc.stderr[-2000:]
    assert "POISON_OK" in proc.stdout
