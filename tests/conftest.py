"""Shared fixtures.  `gpu`-marked tests need a gfx950 device and call the
native libraries through their C ABI; everything else runs on the CPU."""
from __future__ import annotations

import sys
from pathlib import Path

import pytest

ROOT = Path(__file__).resolve().parents[1]
TESTS = Path(__file__).resolve().parent
for p in (str(ROOT), str(TESTS)):
    if p not in sys.path:
        sys.path.insert(0, p)

# Small Qwen3 shape used by the model-level tests: the BASELINE 1.7B format mix
# (Q4_K with Q6_K v/down/output, untied) at toy widths.
SMALL = dict(vocab=1000, hidden=256, intermediate=768, layers=2, n_q=4, n_kv=2, head_dim=64, tied=False,
             embed="Q4_K", q="Q4_K", k="Q4_K", v="Q6_K", o="Q4_K", gate="Q4_K", up="Q4_K", down="Q6_K",
             output="Q6_K", seed=7)
# BASELINE configs[1] format mix (all Q8_0, tied): the lm_head is the FP16 clone of the embedding.
SMALL_Q8 = dict(vocab=768, hidden=512, intermediate=1024, layers=2, n_q=8, n_kv=4, head_dim=64, tied=True,
                embed="Q8_0", q="Q8_0", k="Q8_0", v="Q8_0", o="Q8_0", gate="Q8_0", up="Q8_0", down="Q8_0",
                output="Q8_0", seed=11)

# Mistral 3.1 text shape in miniature: no QK-norm, untied, GQA 4:1, head_dim
# (128) != hidden / heads (64), Mistral's eps and rope theta; the FFN width
# is Qwen3-1.7B's, so single-token steps run the persistent-step
# instantiation of that model's format mix.
SMALL_M3 = dict(vocab=1000, hidden=256, intermediate=6144, layers=2, n_q=4, n_kv=1, head_dim=128, tied=False,
                eps=1e-5, theta=1e9, context=131072, embed="Q4_K", q="Q4_K", k="Q4_K", v="Q6_K", o="Q4_K",
                gate="Q4_K", up="Q4_K", down="Q6_K", output="Q6_K", seed=23)


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (gfx950) device; calls the HIP path")


def _ensure_built():
    lib = ROOT / "brolm_amd" / "lib"
    if not (lib / "libbrolm_hip.so").exists() or not (lib / "libbrolm.so").exists():
        from brolm_amd import build
        build.build_all()


@pytest.fixture(scope="session")
def native():
    _ensure_built()
    from brolm_amd import _native
    _native.lib()
    return _native


def write_synth(tmpdir: Path, spec: dict, name: str, arch: str = "qwen3") -> Path:
    _ensure_built()
    import brolm_amd as ba
    path = tmpdir / f"{name}.gguf"
    if not path.exists():
        write = ba.write_synth_qwen3 if arch == "qwen3" else ba.write_synth_mistral3
        write(ba.SynthSpec(**spec), str(path))
    return path


@pytest.fixture(scope="session")
def small_gguf(tmp_path_factory) -> Path:
    return write_synth(tmp_path_factory.mktemp("synth"), SMALL, "small_q4k")


@pytest.fixture(scope="session")
def small_q8_gguf(tmp_path_factory) -> Path:
    return write_synth(tmp_path_factory.mktemp("synth8"), SMALL_Q8, "small_q8")


@pytest.fixture(scope="session")
def small_m3_gguf(tmp_path_factory) -> Path:
    return write_synth(tmp_path_factory.mktemp("synth_m3"), SMALL_M3, "small_m3", arch="mistral3")
