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
model_full.npz
             full-depth greedy fixtures at BASELINE.json shapes, each with the
             oracle's per-step top-2 logit margins and the checkpoint hash:
             "q4k" Qwen3-1.7B (28 layers, Q4_K with Q6_K v / down / output,
             untied; configs[2]'s format mix), 32-token prompt, 32 tokens;
             "bf16" Qwen3-0.6B random-init BF16, tied, 32-token
             prompt, 128 tokens.  Prompts: std::mt19937_64(42) % vocab.
model_full_logits.npz
             the 28-layer Qwen3-1.7B of "q4k" at two contexts,
             a 32-token prompt and a 1024-token prompt (the bench context):
             for each of 32 teacher-forced steps on the oracle's own greedy
             tokens, the oracle's logits at every 37th vocabulary id and at
             its 16 largest ids, its argmax and top-2 margin.
model_8b_width.npz
             Qwen3-8B widths (hidden 4096, FFN 12288, 32 / 8 heads of 128,
             vocab 151936; all-Q4_K layers, Q6_K output: configs[4]'s mix)
             over 2 layers: the oracle's logits at every 37th vocabulary id,
             argmax and top-2 margin after a 2048-token prefill and after
             each of 8 greedy steps (the oracle's prefill takes about a minute
             on 8 cores, too slow to rerun inside a GPU test).
model_full_depth_widths.npz
             the other BASELINE.json shapes at full depth, teacher-forced on
             the oracle's own greedy tokens: "q8" configs[1] (Qwen3-0.6B
             widths, 28 layers, all-Q8_0, tied FP16 lm_head clone) after a
             512-token prompt, 32 steps; "w8b" configs[4] (Qwen3-8B widths,
             36 layers, Q4_K with Q6_K output) after a 256-token prompt
             (the oracle's 36-layer prefill of configs[4]'s 2048 tokens
             would take most of an hour here), 16 steps.  Per step the
             oracle's logits at every 37th id and at its 16 largest ids,
             its argmax and top-2 margin.
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


# Full-depth shapes of BASELINE.json (synthetic, seeded): name -> (spec, prompt, new tokens)
FULL = {
    "q4k": (dict(vocab=151936, hidden=2048, intermediate=6144, layers=28, n_q=16, n_kv=8, head_dim=128,
                 tied=False, embed="Q4_K", q="Q4_K", k="Q4_K", v="Q6_K", o="Q4_K", gate="Q4_K", up="Q4_K",
                 down="Q6_K", output="Q6_K", seed=0), 32, 32),
    "bf16": (dict(vocab=151936, hidden=1024, intermediate=3072, layers=28, n_q=16, n_kv=8, head_dim=128,
                  tied=True, embed="BF16", q="BF16", k="BF16", v="BF16", o="BF16", gate="BF16", up="BF16",
                  down="BF16", output="BF16", seed=0), 32, 128),
}


def make_full_fixture(tmp: Path) -> dict:
    import brolm_amd as ba
    import oracle
    from conftest import write_synth

    out = {}
    for name, (spec, n_prompt, n_new) in FULL.items():
        path = write_synth(tmp, spec, f"full_{name}")
        prompt = ba.prompt_ids(n_prompt, spec["vocab"], seed=42)
        m = oracle.Model(str(path))
        toks, margins = m.generate_greedy(prompt, n_new)
        out[f"{name}_prompt"] = np.asarray(prompt, np.int32)
        out[f"{name}_tokens"] = np.asarray(toks, np.int32)
        out[f"{name}_margins"] = margins.astype(np.float32)
        out[f"{name}_sha256"] = np.frombuffer(bytes.fromhex(checkpoint_digest(path)), np.uint8)
        print(name, "margins min", float(margins.min()), "tokens", toks[:8], flush=True)
        del m
        path.unlink()
    return out


FL_STEPS, FL_STRIDE, FL_TOP = 32, 37, 16
FL_CONTEXTS = (32, 1024)


def make_full_logits_fixture(tmp: Path) -> dict:
    import brolm_amd as ba
    import oracle
    from conftest import write_synth

    spec, _, _ = FULL["q4k"]
    path = write_synth(tmp, spec, "full_q4k")
    out = {"sha256": np.frombuffer(bytes.fromhex(checkpoint_digest(path)), np.uint8)}
    m = oracle.Model(str(path))
    for ctx in FL_CONTEXTS:
        prompt = ba.prompt_ids(ctx, spec["vocab"], seed=42)
        m.allocate_cache(ctx + FL_STEPS + 1)
        lg = m.forward(prompt, last_only=True)[0]
        rows, top_ids, top_vals, toks, margins = [], [], [], [], []
        for step in range(FL_STEPS):
            order = np.argsort(lg, kind="stable")[::-1]
            rows.append(lg[::FL_STRIDE].copy())
            top_ids.append(order[:FL_TOP].astype(np.int32))
            top_vals.append(lg[order[:FL_TOP]].copy())
            tok, _ = oracle.argmax(lg)
            toks.append(tok)
            margins.append(float(lg[order[0]] - lg[order[1]]))
            if step + 1 < FL_STEPS:
                lg = m.forward([tok], last_only=True)[0]
        out[f"c{ctx}_prompt"] = np.asarray(prompt, np.int32)
        out[f"c{ctx}_rows"] = np.stack(rows).astype(np.float32)
        out[f"c{ctx}_top_ids"] = np.stack(top_ids)
        out[f"c{ctx}_top_vals"] = np.stack(top_vals).astype(np.float32)
        out[f"c{ctx}_tokens"] = np.asarray(toks, np.int32)
        out[f"c{ctx}_margins"] = np.asarray(margins, np.float32)
        print(ctx, "tokens", toks[:8], "min margin", min(margins), flush=True)
    return out


W8B = dict(vocab=151936, hidden=4096, intermediate=12288, layers=2, n_q=32, n_kv=8, head_dim=128, tied=False,
           embed="Q4_K", q="Q4_K", k="Q4_K", v="Q4_K", o="Q4_K", gate="Q4_K", up="Q4_K", down="Q4_K",
           output="Q6_K", seed=5)
W8B_PROMPT, W8B_STEPS, W8B_STRIDE = 2048, 8, 37


def make_8b_width_fixture(tmp: Path) -> dict:
    import brolm_amd as ba
    import oracle
    from conftest import write_synth

    path = write_synth(tmp, W8B, "w8b")
    prompt = ba.prompt_ids(W8B_PROMPT, W8B["vocab"], seed=42)
    m = oracle.Model(str(path))
    m.allocate_cache(W8B_PROMPT + W8B_STEPS + 1)
    rows, arg, marg, toks = [], [], [], []
    lg = m.forward(prompt, last_only=True)[0]
    for step in range(W8B_STEPS + 1):
        top = np.argsort(lg)[::-1][:2]
        rows.append(lg[::W8B_STRIDE].copy())
        arg.append(int(top[0]))
        marg.append(float(lg[top[0]] - lg[top[1]]))
        if step == W8B_STEPS:
            break
        toks.append(int(top[0]))
        lg = m.forward([toks[-1]], last_only=True)[0]
    return {"logits": np.stack(rows).astype(np.float32), "argmax": np.asarray(arg, np.int32),
            "margins": np.asarray(marg, np.float32), "tokens": np.asarray(toks, np.int32),
            "sha256": np.frombuffer(bytes.fromhex(checkpoint_digest(path)), np.uint8)}


# Full-depth widths of configs[1] and configs[4]: name -> (spec, prompt tokens, teacher-forced steps)
FULL_WIDTHS = {
    "q8": (dict(vocab=151936, hidden=1024, intermediate=3072, layers=28, n_q=16, n_kv=8, head_dim=128, tied=True,
                embed="Q8_0", q="Q8_0", k="Q8_0", v="Q8_0", o="Q8_0", gate="Q8_0", up="Q8_0", down="Q8_0",
                output="Q8_0", seed=9), 512, 32),
    "w8b": (dict(W8B, layers=36), 256, 16),
}


def teacher_forced(m, prompt, steps: int) -> dict:
    """The oracle's logits rows (every FL_STRIDE-th id), top-FL_TOP ids and
    values, argmax tokens and top-2 margins over `steps` teacher-forced steps
    on its own greedy tokens after `prompt`."""
    import oracle

    m.allocate_cache(len(prompt) + steps + 1)
    lg = m.forward(prompt, last_only=True)[0]
    rows, top_ids, top_vals, toks, margins = [], [], [], [], []
    for step in range(steps):
        order = np.argsort(lg, kind="stable")[::-1]
        rows.append(lg[::FL_STRIDE].copy())
        top_ids.append(order[:FL_TOP].astype(np.int32))
        top_vals.append(lg[order[:FL_TOP]].copy())
        tok, _ = oracle.argmax(lg)
        toks.append(tok)
        margins.append(float(lg[order[0]] - lg[order[1]]))
        if step + 1 < steps:
            lg = m.forward([tok], last_only=True)[0]
    return {"prompt": np.asarray(prompt, np.int32), "rows": np.stack(rows).astype(np.float32),
            "top_ids": np.stack(top_ids), "top_vals": np.stack(top_vals).astype(np.float32),
            "tokens": np.asarray(toks, np.int32), "margins": np.asarray(margins, np.float32)}


def make_full_widths_fixture(tmp: Path) -> dict:
    import brolm_amd as ba
    import oracle
    from conftest import write_synth

    out = {}
    for name, (spec, n_prompt, steps) in FULL_WIDTHS.items():
        path = write_synth(tmp, spec, f"fw_{name}")
        out[f"{name}_sha256"] = np.frombuffer(bytes.fromhex(checkpoint_digest(path)), np.uint8)
        m = oracle.Model(str(path))
        for k, v in teacher_forced(m, ba.prompt_ids(n_prompt, spec["vocab"], seed=42), steps).items():
            out[f"{name}_{k}"] = v
        print(name, "tokens", out[f"{name}_tokens"][:8], "min margin", float(out[f"{name}_margins"].min()),
              flush=True)
        del m
        path.unlink()
    return out


def main() -> None:
    which = sys.argv[1:] or ["blocks", "small", "full", "w8b", "full_logits", "full_widths"]
    if "blocks" in which:
        np.savez_compressed(HERE / "blocks.npz", **make_blocks())
    with tempfile.TemporaryDirectory() as td:
        if "small" in which:
            np.savez_compressed(HERE / "model_small.npz", **make_model_fixture(Path(td)))
        if "full" in which:
            np.savez_compressed(HERE / "model_full.npz", **make_full_fixture(Path(td)))
        if "w8b" in which:
            np.savez_compressed(HERE / "model_8b_width.npz", **make_8b_width_fixture(Path(td)))
        if "full_logits" in which:
            np.savez_compressed(HERE / "model_full_logits.npz", **make_full_logits_fixture(Path(td)))
        if "full_widths" in which:
            np.savez_compressed(HERE / "model_full_depth_widths.npz", **make_full_widths_fixture(Path(td)))
    print("wrote", which)


if __name__ == "__main__":
    main()
