"""Failure handling of the one-launch per-tensor quant, forced from the host.

k_quant_tensor_1pass exchanges workgroup maxima through tagged slots and
gives up after a bounded number of polls. A spin limit of 0
(cbq_set_tensor_spin_limit) makes every workgroup that does not find all the
others at its first poll give up, so the early finishers time out while every
kernel still ends normally. A child process (fresh library state) checks, for
the workspace entry points (FP8 and INT8) and for the allocation-free entry:
  * a call made with the limit at 0 sets the sticky status word to 1;
  * that call's outputs are never quietly wrong: its scale is NaN, or its
    scale and every code equal the oracle's;
  * the next calls, with the default limit restored, are bit-exact against
    the oracle on the same workspace, with no reset (twice, the second on a
    smaller tensor, so that slots beyond the smaller grid stay stale);
  * the status word stays 1 until cbq_tensor_quant_status_clear, then reads 0
    and stays 0 over exact calls;
  * through the public API with CUBLADE_CHECK_EXCHANGE=1, a timed-out call
    raises RuntimeError naming the timeout, and the next call is exact.
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
    sys.path.insert(0, {root!r} + "/tests")
    import numpy as np
    import torch
    import oracle
    from cublade_amd import _abi
    from _util import bits
    L = _abi.lib()
    dev = torch.device("cuda:0")
    stream = _abi.stream_handle(dev)
    g = torch.Generator().manual_seed(5)
    N_BIG = 16 * 1024 * 1024
    N_SMALL = 3 * 1024 * 1024 + 5
    xs = {{}}
    for n in (N_BIG, N_SMALL):
        x = torch.randn(n, generator=g).to(torch.bfloat16)
        x[n // 3] = 17.5                     # a maximum away from the first workgroup's part
        xs[n] = (x.to(dev), bits(x))
    ws = torch.zeros(L.cbq_quant_tensor_ws_bytes(), dtype=torch.uint8, device=dev)
    want = {{}}
    def expect(n, fp8):
        key = (n, fp8)
        if key not in want:
            xb = xs[n][1]
            want[key] = (oracle.quant_fp8_tensor(xb, oracle.BF16) if fp8
                         else oracle.quant_int8_tensor(xb, oracle.BF16))
        return want[key]
    def call(entry, n):
        x = xs[n][0]
        q = torch.empty(n, dtype=torch.uint8, device=dev)
        s = torch.empty((), dtype=torch.float32, device=dev)
        if entry == "noalloc":
            rc = L.cbq_quant_fp8_tensor_noalloc(x.data_ptr(), _abi.BF16, n, ctypes.c_float(1e-12),
                                                q.data_ptr(), s.data_ptr(), stream)
        else:
            fn = L.cbq_quant_fp8_tensor if entry == "fp8" else L.cbq_quant_int8_tensor
            rc = fn(x.data_ptr(), _abi.BF16, n, ctypes.c_float(1e-12), ws.data_ptr(),
                    ws.numel(), q.data_ptr(), s.data_ptr(), stream)
        _abi.check(rc, entry)
        torch.cuda.synchronize()
        return q.cpu().numpy(), np.float32(s.item())
    def status(entry):
        st = ctypes.c_int(-1)
        _abi.check(L.cbq_tensor_quant_status(None if entry == "noalloc" else ws.data_ptr(),
                                             stream, ctypes.byref(st)), "status")
        return st.value
    def clear(entry):
        _abi.check(L.cbq_tensor_quant_status_clear(None if entry == "noalloc" else ws.data_ptr(),
                                                   stream), "clear")
        torch.cuda.synchronize()
    def exact(entry, n, q, s):
        wq, ws_ = expect(n, entry != "int8")
        return (np.float32(s).view(np.uint32) == np.float32(ws_).view(np.uint32)
                and np.array_equal(q, np.asarray(wq).view(np.uint8)))
    default = _abi.set_tensor_spin_limit(0)
    _abi.set_tensor_spin_limit(default)
    print("default spin limit", default, flush=True)
    for entry in ("fp8", "int8", "noalloc"):
        print("[timeout] entry", entry, flush=True)
        assert status(entry) == 0, "status must start at 0"
        q, s = call(entry, N_BIG)                 # a normal call first: exact
        assert exact(entry, N_BIG, q, s), "exact before the timeout"
        _abi.set_tensor_spin_limit(0)
        forced = 0
        for _ in range(3):
            q, s = call(entry, N_BIG)
            if status(entry) == 1:
                forced += 1
            assert np.isnan(s) or exact(entry, N_BIG, q, s), "a finite scale with wrong codes"
        _abi.set_tensor_spin_limit(default)
        print("  forced calls that set status:", forced, flush=True)
        assert forced >= 1, "limit 0 never timed out"
        assert status(entry) == 1
        for n in (N_BIG, N_SMALL, N_BIG):
            q, s = call(entry, n)
            assert exact(entry, n, q, s), f"call after the timeout not exact (n={{n}})"
        assert status(entry) == 1, "status is sticky until cleared"
        clear(entry)
        assert status(entry) == 0
        q, s = call(entry, N_SMALL)
        assert exact(entry, N_SMALL, q, s) and status(entry) == 0
        # the workspace entries share one control block: start the next entry clean
        clear(entry)
    # the public API: with CUBLADE_CHECK_EXCHANGE=1 a timed-out call raises
    import os
    from cublade_amd.quantization import quantize_tensor
    os.environ["CUBLADE_CHECK_EXCHANGE"] = "1"
    x = xs[N_BIG][0]
    _abi.set_tensor_spin_limit(0)
    raised = 0
    for _ in range(3):
        try:
            quantize_tensor(x, dtype=torch.int8, mode="tensor")
        except RuntimeError as e:
            assert "timed out" in str(e), e
            raised += 1
    _abi.set_tensor_spin_limit(default)
    print("  public-API calls that raised:", raised, flush=True)
    assert raised >= 1
    qt = quantize_tensor(x, dtype=torch.int8, mode="tensor")   # exact, no raise
    wq, wsc = expect(N_BIG, False)
    assert np.array_equal(qt.data.cpu().numpy(), wq)
    assert np.float32(qt.scale.item()).view(np.uint32) == np.float32(wsc).view(np.uint32)
    print("RECOVERY_OK", flush=True)
""")


def test_forced_exchange_timeout_recovers_exactly():
    print("[timeout] child process with the spin limit forced to 0", flush=True)
    proc = subprocess.run([sys.executable, "-c", CHILD.format(root=str(ROOT))],
                          env={**os.environ, "CUBLADE_SKIP_WARMUP": "1"},
                          capture_output=True, text=True, timeout=180)
    print(proc.stdout[-3000:], proc.stderr[-3000:], flush=True)
    assert proc.returncode == 0, proc.stderr[-3000:]
    assert "RECOVERY_OK" in proc.stdout


CHILD_COLS = textwrap.dedent("""
    import ctypes, sys
    sys.path.insert(0, {root!r})
    sys.path.insert(0, {root!r} + "/tests")
    import numpy as np
    import torch
    import oracle
    from cublade_amd import _abi
    from _util import bits
    L = _abi.lib()
    dev = torch.device("cuda:0")
    stream = _abi.stream_handle(dev)
    g = torch.Generator().manual_seed(11)
    R, C = 13000, 8192
    x = (torch.randn(R, C, generator=g) * 0.05)
    x[7, 5], x[12000, 6000] = 30.0, -25.0
    x = x.to(torch.bfloat16)
    qo, so = oracle.quant_int8_channel(bits(x), oracle.BF16, axis=1)
    qo = np.asarray(qo).reshape(R, C)
    so_bits = np.asarray(so, np.float32).view(np.uint32)
    xd = x.to(dev)
    ws = torch.zeros(L.cbq_quant_int8_channel_ws_bytes(R, C, 1), dtype=torch.uint8, device=dev)
    def call():
        q = torch.empty(R, C, dtype=torch.int8, device=dev)
        s = torch.empty(C, dtype=torch.float32, device=dev)
        _abi.check(L.cbq_quant_int8_channel(xd.data_ptr(), _abi.BF16, R, C, 1, ctypes.c_float(1e-12),
                                            ws.data_ptr(), ws.numel(), q.data_ptr(), s.data_ptr(),
                                            stream), "channel axis 1")
        torch.cuda.synchronize()
        return q.cpu().numpy(), s.cpu().numpy()
    def status():
        st = ctypes.c_int(-1)
        _abi.check(L.cbq_tensor_quant_status(ws.data_ptr(), stream, ctypes.byref(st)), "status")
        return st.value
    q, s = call()
    assert np.array_equal(q, qo) and np.array_equal(s.view(np.uint32), so_bits), "exact first"
    default = _abi.set_tensor_spin_limit(0)
    forced = 0
    for _ in range(3):
        q, s = call()
        forced += status() == 1
        finite = ~np.isnan(s)
        # a column whose scale is not NaN has its exact scale and codes
        assert np.array_equal(s.view(np.uint32)[finite], so_bits[finite]), "finite scale differs"
        assert np.array_equal(q[:, finite], qo[:, finite]), "codes of a finite-scale column differ"
    _abi.set_tensor_spin_limit(default)
    print("  forced column calls that set status:", forced, flush=True)
    assert status() == 1
    for _ in range(2):
        q, s = call()
        assert np.array_equal(q, qo) and np.array_equal(s.view(np.uint32), so_bits), "after timeout"
    _abi.check(L.cbq_tensor_quant_status_clear(ws.data_ptr(), stream), "clear")
    assert status() == 0
    print("COLS_RECOVERY_OK", flush=True)
""")


def test_forced_column_exchange_timeout_recovers_exactly():
    """The one-launch per-column quant (two grid-wide exchanges) under a spin
    limit of 0: the status word is set, every column whose scale is not NaN
    has exact codes and scale, and the calls after it are exact."""
    print("[timeout] column child process with the spin limit forced to 0", flush=True)
    proc = subprocess.run([sys.executable, "-c", CHILD_COLS.format(root=str(ROOT))],
                          env={**os.environ, "CUBLADE_SKIP_WARMUP": "1"},
                          capture_output=True, text=True, timeout=180)
    print(proc.stdout[-3000:], proc.stderr[-3000:], flush=True)
    assert proc.returncode == 0, proc.stderr[-3000:]
    assert "COLS_RECOVERY_OK" in proc.stdout
