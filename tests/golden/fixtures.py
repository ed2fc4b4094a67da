"""Loader of the golden model fixtures written by make_model_fixtures.py.

Checks every array against the SHA-256 in the manifest before handing it out,
so an edited or truncated fixture fails loudly instead of moving the bar."""
from __future__ import annotations

import functools
import hashlib
import json
from pathlib import Path

import numpy as np
import torch

HERE = Path(__file__).resolve().parent


@functools.lru_cache(maxsize=1)
def load() -> tuple[dict, dict]:
    manifest = json.loads((HERE / "model_fixtures.json").read_text())
    with np.load(HERE / "model_fixtures.npz", allow_pickle=False) as z:
        arrays = {k: z[k] for k in z.files}
    want = manifest["sha256"]
    if set(want) != set(arrays):
        raise AssertionError("fixture arrays and manifest disagree")
    for k, v in arrays.items():
        got = hashlib.sha256(np.ascontiguousarray(v).tobytes()).hexdigest()
        if got != want[k]:
            raise AssertionError(f"fixture array {k} does not match its checksum")
    return arrays, manifest["meta"]


def group(tag: str, dtype=torch.float64) -> dict[str, torch.Tensor]:
    """Arrays of one fixture group as tensors, floating ones in ``dtype``."""
    arrays, _ = load()
    out = {}
    pre = tag + "/"
    for k, v in arrays.items():
        if k.startswith(pre):
            t = torch.from_numpy(v.copy())
            out[k[len(pre):]] = t.to(dtype) if t.is_floating_point() else t
    return out


def state_dict(tag: str, strip: str = "", dtype=torch.float64) -> dict[str, torch.Tensor]:
    """The parameters of a fixture group (everything but its inputs/outputs),
    keys with ``strip`` removed from the front."""
    io = {"ids", "out", "x", "prefix", "labels", "logits", "loss", "logits_chunked", "loss_chunked",
          "hidden", "loss_fused", "grad_hidden", "grad_weight", "block0_out", "block1_out", "w"}
    return {k[len(strip):]: v for k, v in group(tag, dtype).items()
            if k not in io and not k.startswith("grad/") and k.startswith(strip)}


def grads(tag: str, dtype=torch.float64) -> dict[str, torch.Tensor]:
    """Parameter gradients stored with a fixture group (``grad/<name>``)."""
    return {k[len("grad/"):]: v for k, v in group(tag, dtype).items() if k.startswith("grad/")}


def meta(tag: str):
    return load()[1][tag]
