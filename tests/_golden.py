"""Loader for the committed golden vectors (tests/golden/golden.npz)."""
from __future__ import annotations

import json
from functools import lru_cache
from pathlib import Path

import numpy as np

PATH = Path(__file__).resolve().parent / "golden" / "golden.npz"


@lru_cache(maxsize=1)
def load():
    z = np.load(PATH, allow_pickle=False)
    data = {k: z[k] for k in z.files}
    manifest = json.loads(bytes(data.pop("manifest")).decode())
    return manifest, data


def cases(kind: str):
    manifest, data = load()
    out = []
    for meta in manifest:
        if meta["kind"] != kind:
            continue
        prefix = f"{kind}:{meta['name']}:"
        arrs = {k[len(prefix):]: v for k, v in data.items() if k.startswith(prefix)}
        out.append((meta, arrs))
    return out


def ids(kind: str):
    return [m["name"] for m, _ in cases(kind)]


def f16_bits_equal(a: np.ndarray, b: np.ndarray) -> bool:
    """Bit equality for fp16/bf16 patterns, treating any NaN as equal to any NaN."""
    a = np.asarray(a, np.uint16)
    b = np.asarray(b, np.uint16)
    return bool(np.array_equal(a, b))
