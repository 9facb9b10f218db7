"""Reloading weights into a model that already ran: everything derived from
the old weights must go (DenseDecoder::load_weights, the reference's
src/detail/dense_decoder.cpp:121-191 uploads into the same model object).
Derived state here: the captured graphs of batched steps (they hold the old
weight pointers) and the FP16 layer copies a pass of 512+ rows makes.  After a
reload the model must give the bits a fresh model of the new weights gives on
the same inputs; stale graphs or copies would give the old model's values (or
read freed memory)."""
from __future__ import annotations

import numpy as np
import pytest

from conftest import SMALL, write_synth

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def ba():
    import brolm_amd
    brolm_amd.init()
    return brolm_amd


@pytest.fixture(scope="module")
def other_gguf(tmp_path_factory):
    """The small Q4_K model's shape with other weights (another seed)."""
    return write_synth(tmp_path_factory.mktemp("synth_reload"), dict(SMALL, seed=8), "small_q4k_seed8")


def _fresh(ba, path):
    m = ba.Qwen3Model(ba.Qwen3Config.from_gguf(str(path)))
    m.load_weights(str(path))
    return m


def _batched(m, rng_seed, V):
    """Prefill four slots, then three 4-row batched steps (the first captures
    the row count's graph, the others replay it); returns every step's logits."""
    rng = np.random.default_rng(rng_seed)
    out = []
    for s in range(4):
        out.append(m.prefill_slot(s, rng.integers(0, V, 5 + 3 * s).tolist()))
    for _ in range(3):
        out.append(m.forward_batch(rng.integers(0, V, 4).tolist(), [0, 1, 2, 3]))
    return out


def test_reload_after_batched_steps_matches_fresh_model(ba, small_gguf, other_gguf):
    print("[reload] batched steps", flush=True)
    m = _fresh(ba, small_gguf)
    V = m.cfg.vocab_size
    m.allocate_batch(4, 64)
    before = _batched(m, 1, V)
    m.load_weights(str(other_gguf))
    for s in range(4):   # the slots' keys came from the old weights; prefill_slot appends
        m.truncate_slot(s, 0)
    after = _batched(m, 2, V)
    f = _fresh(ba, other_gguf)
    f.allocate_batch(4, 64)
    want = _batched(f, 2, V)
    for i, (a, b) in enumerate(zip(after, want)):
        assert np.array_equal(a, b), f"step {i}: reloaded model differs from a fresh one"
    # the reload changed the model (the test is not vacuous)
    assert not np.array_equal(before[-1], after[-1])
    for x in (m, f):
        x.close()


def test_reload_after_long_prefill_matches_fresh_model(ba, small_gguf, other_gguf):
    """A 600-token pass makes the FP16 layer copies; after a reload the next
    600-token pass must use the new weights."""
    print("[reload] long prefill", flush=True)
    rng = np.random.default_rng(3)
    m = _fresh(ba, small_gguf)
    V = m.cfg.vocab_size
    m.allocate_cache(1024)
    p1 = rng.integers(0, V, 600).tolist()
    first = m.forward_last(p1)
    m.load_weights(str(other_gguf))
    m.reset_cache()
    p2 = rng.integers(0, V, 600).tolist()
    got = m.forward_last(p2)
    f = _fresh(ba, other_gguf)
    f.allocate_cache(1024)
    want = f.forward_last(p2)
    assert np.array_equal(got, want)
    assert not np.array_equal(first, got)
    for x in (m, f):
        x.close()
