"""Writes the committed fixtures of tests/golden/ (run from the repo root:
`python tests/golden/make_golden.py`).

blocks.npz   raw GGUF blocks of Q8_0 / Q4_K / Q6_K made by the independent
             element-wise encoder (tests/spec_blocks.py) from known integers,
             with the FP32 values of the published formula (float64, rounded
             once) and their binary16 RNE rounding (numpy).  Pins the block
             decoders of the oracle and of the device.
model_small.npz
             the oracle's greedy continuation (32 tokens, with top-2 margins)
             and last-row logits for the small synthetic Qwen3 of
             tests/conftest.py (SMALL) on the bench prompt recipe
             (std::mt19937_64(42) % vocab, tools/bench_decode.cpp:208-213),
             plus a hash of the synthetic checkpoint bytes so a change in the
             generator is told apart from a change in the decoder.
The reference has no numeric fixtures for this path (its quant tests check
finiteness against downloaded checkpoints only), so these are the vectors.
"""
from __future__ import annotations

import hashlib
import sys
import tempfile
from pathlib import Path

import numpy as np

HERE = Path(__file__).resolve().parent
TESTS = HERE.parent
ROOT = TESTS.parent
sys.path[:0] = [str(ROOT), str(TESTS)]

import spec_blocks as sb  # noqa: E402

PROMPT_LEN = 24
N_NEW = 32


def make_blocks() -> dict:
    rng = np.random.default_rng(20261201)
    out = {}
    for t, nb in ((8, 96), (12, 24), (14, 24)):
        raw, val = sb.random_blocks(rng, t, nb, extremes=True)
        out[f"raw_{t}"] = np.frombuffer(raw, np.uint8)
        out[f"f32_{t}"] = val.view(np.uint32)
        out[f"f16_{t}"] = val.astype(np.float16).view(np.uint16)
    return out


def checkpoint_digest(path: Path) -> str:
    return hashlib.sha256(path.read_bytes()).hexdigest()


def make_model_fixture(tmp: Path) -> dict:
    import brolm_amd as ba
    import oracle
    from conftest import SMALL, write_synth

    path = write_synth(tmp, SMALL, "small_q4k")
    prompt = ba.prompt_ids(PROMPT_LEN, SMALL["vocab"], seed=42)
    m = oracle.Model(str(path))
    m.allocate_cache(PROMPT_LEN + N_NEW + 1)
    last = m.forward(prompt, last_only=True)[0]
    m2 = oracle.Model(str(path))
    toks, margins = m2.generate_greedy(prompt, N_NEW)
    return {"prompt": np.asarray(prompt, np.int32), "tokens": np.asarray(toks, np.int32),
            "margins": margins.astype(np.float32), "last_logits": last.astype(np.float32),
            "sha256": np.frombuffer(bytes.fromhex(checkpoint_digest(path)), np.uint8)}


def main() -> None:
    np.savez_compressed(HERE / "blocks.npz", **make_blocks())
    with tempfile.TemporaryDirectory() as td:
        np.savez_compressed(HERE / "model_small.npz", **make_model_fixture(Path(td)))
    print("wrote", HERE / "blocks.npz", HERE / "model_small.npz")


if __name__ == "__main__":
    main()
