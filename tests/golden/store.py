"""Reading and writing the golden fixtures of the hot path.

One compressed ``<case>.npz`` per case, holding ``in_<name>`` input arrays
and ``out_<name>`` expected outputs, all float32: the 16-bit inputs are
exact in float32, and the expected outputs are the float64 oracle values
rounded once to float32 (1e-7 relative, far below every parity bar).
``manifest.json`` records per case the seed, the scalar parameters, each
input's dtype and every shape, and the sha256 of the ``.npz`` file.

This module imports nothing from ``oracle/``: the GPU test of the fixtures
reads the stored vectors through it and runs no oracle code.
"""

from __future__ import annotations

import hashlib
import json
import os

import numpy as np
import torch

HERE = os.path.dirname(os.path.abspath(__file__))
MANIFEST = os.path.join(HERE, "manifest.json")


def path(name: str) -> str:
    return os.path.join(HERE, name + ".npz")


def sha256(p: str) -> str:
    with open(p, "rb") as f:
        return hashlib.sha256(f.read()).hexdigest()


def manifest() -> dict:
    with open(MANIFEST) as f:
        return json.load(f)


def save(name: str, seed: int, x: dict, out: dict) -> dict:
    """Write ``<name>.npz`` from inputs ``x`` (tensors plus ``"params"``) and
    expected outputs ``out``; returns the case's manifest entry."""
    arrays, dtypes, in_shapes, out_shapes = {}, {}, {}, {}
    for n, t in x.items():
        if n == "params":
            continue
        arrays["in_" + n] = t.detach().to(torch.float32).numpy()
        dtypes[n] = str(t.dtype).replace("torch.", "")
        in_shapes[n] = list(t.shape)
    for n, t in out.items():
        arrays["out_" + n] = t.detach().to(torch.float32).numpy()
        out_shapes[n] = list(t.shape)
    np.savez_compressed(path(name), **arrays)
    return {"seed": seed, "params": x["params"], "dtypes": dtypes, "inputs": in_shapes,
            "outputs": out_shapes, "sha256": sha256(path(name))}


def load(name: str, entry: dict | None = None):
    """``(inputs, outputs)`` of a stored case: inputs as CPU tensors in their
    recorded dtype plus ``"params"``, outputs as float64 CPU tensors."""
    entry = entry if entry is not None else manifest()[name]
    with np.load(path(name), allow_pickle=False) as z:
        arrs = {k: z[k] for k in z.files}
    x = {"params": entry["params"]}
    for n, dt in entry["dtypes"].items():
        x[n] = torch.from_numpy(arrs["in_" + n]).to(getattr(torch, dt))
    out = {n[4:]: torch.from_numpy(a).to(torch.float64) for n, a in arrs.items() if n.startswith("out_")}
    return x, out
