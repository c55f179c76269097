"""hipcc build-and-load for the cublade_amd HIP library (gfx950).

Mirrors the reference loader (``cublade/_loader.py:47-125``): a module is
built on first use, memoised in-process by name, and a failed build is
remembered and re-raised without retrying. Differences, by design:

* the compiler is ``hipcc --offload-arch=gfx950`` and the product is a plain
  C-ABI shared library loaded with :mod:`ctypes` (no torch extension, no
  pybind);
* the library is built IN-TREE under ``cublade_amd/_build/`` and keyed by a
  hash of its sources, headers and flags, so a library built ahead of time
  (``__graft_entry__.build()``) is loaded as-is wherever the tree is copied;
* fast math is never used: every quantization kernel needs IEEE division and
  no FMA contraction (``-ffp-contract=off``) to be bit-exact. The
  ``use_fast_math`` argument is accepted for signature compatibility and
  ignored.
"""
from __future__ import annotations

import ctypes
import hashlib
import os
import shutil
import subprocess
import threading
from pathlib import Path
from typing import Sequence

PKG = Path(__file__).resolve().parent
CSRC: Path = PKG / "csrc"
INCLUDE: Path = PKG.parent / "include"
BUILD: Path = PKG / "_build"

DEFAULT_ARCH = "gfx950"

# hipcc flags for every build. -Xclang -target-feature -Xclang -packed-fp32-ops
# keeps the compiler from emitting packed fp32 VALU ops.
BASE_FLAGS = (
    "-O3", "-std=c++17", "-fPIC", "-shared", "-ffp-contract=off",
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
)

_loaded: dict[str, ctypes.CDLL] = {}
_failed: dict[str, str] = {}
_lock = threading.Lock()


def hipcc() -> str:
    exe = shutil.which("hipcc") or "/opt/rocm/bin/hipcc"
    if not Path(exe).exists():
        raise RuntimeError("hipcc not found: cannot build the cublade_amd HIP library")
    return exe


def _command(sources, out: Path, arch: str, extra_cflags, extra_includes, extra_ldflags):
    inc = [f"-I{INCLUDE}", f"-I{CSRC}", *(f"-I{p}" for p in extra_includes)]
    return [hipcc(), f"--offload-arch={arch}", *BASE_FLAGS, *inc, *extra_cflags,
            *(str(s) for s in sources), "-o", str(out), *extra_ldflags]


def _stamp(sources, arch, extra_cflags, extra_includes, extra_ldflags) -> str:
    h = hashlib.sha256()
    files = [Path(s) for s in sources]
    for d in (CSRC, INCLUDE, *(Path(p) for p in extra_includes)):
        if d.is_dir():
            files += sorted(d.glob("*.h"))
    for f in files:
        h.update(str(f.name).encode())
        h.update(f.read_bytes())
    h.update(repr((arch, BASE_FLAGS, tuple(extra_cflags), tuple(extra_ldflags))).encode())
    return h.hexdigest()


def library_path(name: str) -> Path:
    return BUILD / f"lib{name}.so"


def build_module(name: str, sources: Sequence[Path | str], *, arch: str | None = None,
                 extra_cflags: Sequence[str] = (), extra_includes: Sequence[Path | str] = (),
                 extra_ldflags: Sequence[str] = (), force: bool = False,
                 verbose: bool = False) -> Path:
    """Compile ``sources`` into ``_build/lib<name>.so`` unless an up-to-date
    build (same source/header/flag hash) is already there."""
    arch = arch or DEFAULT_ARCH
    out = library_path(name)
    stamp_file = out.with_suffix(".so.stamp")
    stamp = _stamp(sources, arch, extra_cflags, extra_includes, extra_ldflags)
    if not force and out.exists() and stamp_file.exists() and stamp_file.read_text() == stamp:
        return out
    BUILD.mkdir(parents=True, exist_ok=True)
    tmp = out.with_name(f"{out.name}.tmp{os.getpid()}")
    cmd = _command(sources, tmp, arch, extra_cflags, extra_includes, extra_ldflags)
    proc = subprocess.run(cmd, capture_output=True, text=True)
    if verbose or proc.returncode != 0:
        msg = "\n".join(line for line in (proc.stdout + proc.stderr).splitlines()
                        if "packed-fp32-ops" not in line)
        if proc.returncode != 0:
            tmp.unlink(missing_ok=True)
            raise RuntimeError(f"hipcc failed for {name} (exit {proc.returncode}):\n{msg}")
        print(msg)
    os.replace(tmp, out)
    stamp_file.write_text(stamp)
    return out


def load_hip_module(name: str, sources: Sequence[Path | str], *, arch: str | None = None,
                    extra_cflags: Sequence[str] = (), extra_includes: Sequence[Path | str] = (),
                    extra_ldflags: Sequence[str] = (), use_fast_math: bool = False,
                    verbose: bool = False) -> ctypes.CDLL:
    """Build (if needed) and load a HIP C-ABI library, memoised by ``name``.

    Raises RuntimeError if a previous attempt for ``name`` failed, like the
    reference (``_loader.py:84-88``).
    """
    del use_fast_math  # never used: see module docstring
    with _lock:
        cached = _loaded.get(name)
        if cached is not None:
            return cached
        prior = _failed.get(name)
        if prior is not None:
            raise RuntimeError(f"cublade kernel '{name}' failed to compile earlier: {prior}")
        try:
            path = build_module(name, sources, arch=arch, extra_cflags=extra_cflags,
                                extra_includes=extra_includes, extra_ldflags=extra_ldflags,
                                verbose=verbose)
            lib = ctypes.CDLL(str(path))
        except Exception as exc:
            _failed[name] = str(exc)
            raise
        _loaded[name] = lib
        return lib


# Reference name (cublade/_loader.py:47).
load_cuda_module = load_hip_module


def is_loaded(name: str) -> bool:
    return name in _loaded


def load_error(name: str) -> str | None:
    return _failed.get(name)
