"""Bidirectional encode on the MI355X against the oracle: LLM2Vec's Encoder
(encode, encode_pooled) and DenseDecoder::forward_encode on Qwen3 (QK-norm)
and Mistral-style (no QK-norm) weights; the reference's invariants from
tests/test_llm2vec.cpp:163-251."""
from __future__ import annotations

import numpy as np
import pytest

import oracle

pytestmark = pytest.mark.gpu
HIDDEN_TOL = 3e-2


@pytest.fixture(scope="module")
def ba():
    import brolm_amd
    brolm_amd.init()
    return brolm_amd


def _encoder(ba, path):
    t = ba.Mistral3Config.from_gguf(str(path)).text
    cfg = ba.Llm2VecConfig(t.vocab_size, t.hidden_size, t.intermediate_size, t.num_hidden_layers,
                           t.num_attention_heads, t.num_key_value_heads, t.head_dim, t.rms_norm_eps, t.rope_theta)
    e = ba.Llm2VecEncoder(cfg)
    e.load_weights(str(path))
    return e


@pytest.mark.parametrize("L", [4, 37, 300])
def test_encode_vs_oracle(ba, small_m3_gguf, L):
    print(f"[llm2vec] encode L={L}", flush=True)
    e = _encoder(ba, small_m3_gguf)
    ids = ba.prompt_ids(L, e.cfg.vocab_size, seed=L)
    got = e.encode(ids)
    want = oracle.Model(str(small_m3_gguf)).forward_encode(ids)
    assert got.shape == (L, e.cfg.hidden_size) and np.isfinite(got).all()
    assert np.abs(got - want).max() <= HIDDEN_TOL * max(1.0, np.abs(want).max())
    assert np.array_equal(got, e.encode(ids))       # deterministic


def test_encode_is_bidirectional_and_pools(ba, small_m3_gguf):
    e = _encoder(ba, small_m3_gguf)
    seq, seq_b = [5, 17, 2, 31], [5, 17, 2, 9]
    h, hb = e.encode(seq), e.encode(seq_b)
    assert np.abs(h[0] - hb[0]).max() > 1e-3        # row 0 sees the last token
    pooled = e.encode_pooled(seq)
    assert pooled.shape == (e.cfg.hidden_size,)
    assert np.abs(pooled - h.mean(axis=0)).max() < 5e-3
    pooled2 = e.encode_pooled(seq, [1.0, 1.0, 0.0, 0.0])
    assert np.abs(pooled2 - 0.5 * (h[0] + h[1])).max() < 5e-3
    assert np.array_equal(e.encode_pooled(seq, [0.0] * 4), np.zeros(e.cfg.hidden_size, np.float32))
    with pytest.raises(ValueError):
        e.encode_pooled(seq, [1.0, 1.0])


def test_forward_encode_on_qwen3_leaves_the_cache(ba, small_gguf):
    """QK-norm weights, and the KV cache is untouched: a decode that runs
    around an encode matches one that does not."""
    a = ba.Qwen3Model(ba.Qwen3Config.from_gguf(str(small_gguf)))
    a.load_weights(str(small_gguf))
    ids = [1, 2, 3, 4, 900, 17, 512]
    want = oracle.Model(str(small_gguf)).forward_encode(ids)
    got = a.forward_encode(ids)                     # no cache allocated yet
    assert np.abs(got - want).max() <= HIDDEN_TOL * max(1.0, np.abs(want).max())
    a.allocate_cache(64)
    b = ba.Qwen3Model(ba.Qwen3Config.from_gguf(str(small_gguf)))
    b.load_weights(str(small_gguf))
    b.allocate_cache(64)
    la, lb = a.forward([7, 8, 9]), b.forward([7, 8, 9])
    a.forward_encode([44, 45, 46, 47, 48])
    assert a.cache_len() == 3
    assert np.array_equal(a.forward_last([10]), b.forward_last([10]))
    assert np.array_equal(la, lb)
