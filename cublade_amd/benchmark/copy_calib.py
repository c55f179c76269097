"""Known-size device copy for calibrating rocprofv3 byte counters.

Copies a 256 MiB buffer into another ten times (the runtime's device copy
kernel), each after a read-only sweep of 512 MiB. Under
``rocprofv3 --pmc FETCH_SIZE`` (then ``WRITE_SIZE``) each dispatch should
read (write) 262,144 KiB; the ratio of the measured value to that is the
counter's scale factor on this GPU, applied to the kernels of interest.

    rocprofv3 --pmc FETCH_SIZE --kernel-trace -d DIR -o calib -- python -m cublade_amd.benchmark.copy_calib
"""
import torch

NBYTES = 256 << 20


def main() -> None:
    src = torch.ones(NBYTES // 4, dtype=torch.int32, device="cuda")
    dst = torch.empty_like(src)
    flush = torch.zeros(512 << 20 >> 2, dtype=torch.float32, device="cuda")
    sink = torch.zeros((), dtype=torch.float32, device="cuda")
    for _ in range(10):
        torch.sum(flush, dim=0, out=sink)
        dst.copy_(src)
    torch.cuda.synchronize()
    print(f"copied {NBYTES} bytes x 10", flush=True)


if __name__ == "__main__":
    main()
