"""First-import warm-up (reference: cublade/_post_install.py:22-50): build
(if needed) and load the HIP library so the first kernel call does not pay
for hipcc. Silent when no GPU is visible or the build is current.

    python -m cublade_amd._post_install
"""
import sys
import time


def main() -> int:
    try:
        import torch
    except ImportError:
        print("[cublade] PyTorch not importable; skipping kernel warm-up.", file=sys.stderr)
        return 0
    if not torch.cuda.is_available():
        print("[cublade] No GPU visible; skipping kernel warm-up.", file=sys.stderr)
        return 0
    from cublade_amd import _abi

    t0 = time.perf_counter()
    _abi.lib()
    elapsed = time.perf_counter() - t0
    if elapsed > 1.0:
        print(f"[cublade] kernels compiled in {elapsed:.0f}s on {torch.cuda.get_device_name(0)}",
              file=sys.stderr)
    return 0


if __name__ == "__main__":
    sys.exit(main())
