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
