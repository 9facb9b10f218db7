"""Loaders of the committed fixtures (written by make_golden.py)."""
from __future__ import annotations

from pathlib import Path

import numpy as np

HERE = Path(__file__).resolve().parent


def load_blocks():
    """[(ggml type, raw bytes, expected FP32 bits, expected FP16 bits)]."""
    z = np.load(HERE / "blocks.npz")
    return [(t, z[f"raw_{t}"].tobytes(), z[f"f32_{t}"], z[f"f16_{t}"]) for t in (8, 12, 14)]


def load_model_small() -> dict:
    z = np.load(HERE / "model_small.npz")
    d = {k: z[k] for k in z.files}
    d["sha256"] = bytes(d["sha256"]).hex()
    return d
