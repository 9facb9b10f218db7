"""Mistral 3.1 text decoder on the MI355X against the oracle: prefill (op
path), single-token steps (persistent step, graph step and eager step, all
with QK-norm off), greedy tokens, and the reference's model invariants
(tests/test_mistral3_text.cpp)."""
from __future__ import annotations

import os

import numpy as np
import pytest

import oracle

pytestmark = pytest.mark.gpu
LOGIT_TOL = 2e-2


@pytest.fixture(scope="module")
def ba():
    import brolm_amd
    brolm_amd.init()
    return brolm_amd


@pytest.mark.timeout(600)
def test_llama3_8b_widths_persistent_vs_oracle(ba, tmp_path_factory):
    """Two layers at Llama-3-8B widths (H 4096, F 14336, 32 / 8 heads of 128,
    no QK-norm, vocab 128256; Q4_K with Q6_K v / down / output): the persistent
    step's instantiation for these widths, a 256-token prefill and 8 greedy
    steps against the oracle."""
    from conftest import write_synth
    spec = dict(vocab=128256, hidden=4096, intermediate=14336, layers=2, n_q=32, n_kv=8, head_dim=128,
                tied=False, eps=1e-5, theta=5e5, context=8192, embed="Q4_K", q="Q4_K", k="Q4_K", v="Q6_K",
                o="Q4_K", gate="Q4_K", up="Q4_K", down="Q6_K", output="Q6_K", seed=31)
    path = write_synth(tmp_path_factory.mktemp("wl8"), spec, "wl8", arch="mistral3")
    print("[mistral3] Llama-3-8B-width checkpoint written", flush=True)
    m = _load(ba, path, cap=1024)
    assert m.decode_mode() == "persistent"
    om = oracle.Model(str(path))
    om.allocate_cache(1024)
    prompt = ba.prompt_ids(256, spec["vocab"], seed=42)
    a = m.forward_last(prompt)
    b = om.forward(prompt, last_only=True)[0]
    print(f"[mistral3] Llama-3-8B widths prefill max diff {np.abs(a - b).max():.3e}", flush=True)
    assert np.abs(a - b).max() <= LOGIT_TOL
    tok = int(b.argmax())
    for step in range(8):
        a = m.forward_last([tok])
        b = om.forward([tok], last_only=True)[0]
        print(f"[mistral3] Llama-3-8B widths step {step} max diff {np.abs(a - b).max():.3e}", flush=True)
        assert np.abs(a - b).max() <= LOGIT_TOL
        tok = int(b.argmax())
    m.close()


@pytest.mark.timeout(600)
def test_mistral_24b_widths_graph_step_vs_oracle(ba, tmp_path_factory):
    """Two layers at Mistral-Small-3.1-24B widths (H 5120 > the persistent
    step's 4096, so the graph step; F 32768: the down projection takes the
    one-row GEMV with K split over each workgroup's wavefronts, adding into the
    FP32 residual), vocab cut to 8192: a 64-token prefill and 6 single-token
    steps against the oracle."""
    from conftest import write_synth
    spec = dict(vocab=8192, hidden=5120, intermediate=32768, layers=2, n_q=32, n_kv=8, head_dim=128,
                tied=False, eps=1e-5, theta=1e9, context=131072, embed="Q4_K", q="Q4_K", k="Q4_K", v="Q6_K",
                o="Q4_K", gate="Q4_K", up="Q4_K", down="Q6_K", output="Q6_K", seed=37)
    path = write_synth(tmp_path_factory.mktemp("wm24"), spec, "wm24", arch="mistral3")
    print("[mistral3] 24B-width checkpoint written", flush=True)
    m = _load(ba, path, cap=256)
    assert m.decode_mode() == "graph"
    om = oracle.Model(str(path))
    om.allocate_cache(256)
    prompt = ba.prompt_ids(64, spec["vocab"], seed=42)
    a = m.forward_last(prompt)
    b = om.forward(prompt, last_only=True)[0]
    assert np.abs(a - b).max() <= LOGIT_TOL
    tok = int(b.argmax())
    for step in range(6):
        a = m.forward_last([tok])
        b = om.forward([tok], last_only=True)[0]
        print(f"[mistral3] 24B widths step {step} max diff {np.abs(a - b).max():.3e}", flush=True)
        assert np.abs(a - b).max() <= LOGIT_TOL
        tok = int(b.argmax())
    m.close()


def _load(ba, path, cap=128, env=None):
    m = ba.Mistral3TextModel(ba.Mistral3Config.from_gguf(str(path)).text)
    m.load_weights(str(path))
    m.allocate_cache(cap)
    if env is not None:
        saved = {k: os.environ.get(k) for k in env}
        os.environ.update(env)
        try:
            m.decode_mode()    # the step session reads the switches when it is created
        finally:
            for k, v in saved.items():
                if v is None:
                    os.environ.pop(k, None)
                else:
                    os.environ[k] = v
    return m


@pytest.mark.parametrize("env,mode", [({}, "persistent"), ({"BROLM_NO_PERSIST": "1"}, "graph"),
                                      ({"BROLM_NO_GRAPH": "1"}, "eager")])
def test_prefill_and_steps_vs_oracle(ba, small_m3_gguf, env, mode):
    print(f"[mistral3] mode {mode}", flush=True)
    m = _load(ba, small_m3_gguf, env=env)
    assert m.decode_mode() == mode
    om = oracle.Model(str(small_m3_gguf))
    om.allocate_cache(128)
    V = m.cfg.vocab_size
    ids = [5, 17, 2, 31, V - 1, 0, 640]
    got = m.forward(ids)
    want = om.forward(ids)
    assert got.shape == (len(ids), V) and np.isfinite(got).all()
    assert np.abs(got - want).max() <= LOGIT_TOL
    for t in (9, V - 2, 44, 0, 11, 500, 3, 3):
        a = m.forward_last([t])
        b = om.forward([t], last_only=True)[0]
        assert np.abs(a - b).max() <= LOGIT_TOL
    assert m.cache_len() == len(ids) + 8


def test_long_context_steps_vs_oracle(ba, small_m3_gguf):
    """Past one 64-key tile: several attention splits per KV head."""
    m = _load(ba, small_m3_gguf, cap=600)
    assert m.decode_mode() == "persistent"
    om = oracle.Model(str(small_m3_gguf))
    om.allocate_cache(600)
    prompt = ba.prompt_ids(520, m.cfg.vocab_size, seed=5)
    m.forward_last(prompt)
    tok = int(om.forward(prompt, last_only=True)[0].argmax())
    for _ in range(5):
        a = m.forward_last([tok])
        b = om.forward([tok], last_only=True)[0]
        assert np.abs(a - b).max() <= LOGIT_TOL
        tok = int(b.argmax())


def test_greedy_tokens_match_oracle(ba, small_m3_gguf):
    """Device greedy decode (mistral3::generate with greedy sampling) against
    the oracle, teacher-forced: at every step whose oracle top-2 gap exceeds
    twice the logit tolerance the argmaxes agree."""
    m = _load(ba, small_m3_gguf)
    prompt = [1, 50, 7, 300, 42]
    opts = ba.GenerateOptions(max_new_tokens=24, sampling=ba.SamplingParams(temperature=0.0), stop_on_eos=False)
    toks = ba.generate(m, prompt, -1, opts)
    assert len(toks) == 24
    om = oracle.Model(str(small_m3_gguf))
    om.allocate_cache(64)
    lg = om.forward(prompt, last_only=True)[0]
    checked = 0
    for t in toks:
        top2 = np.sort(lg)[-2:]
        if top2[1] - top2[0] > 2 * LOGIT_TOL:
            assert t == int(lg.argmax())
            checked += 1
        lg = om.forward([t], last_only=True)[0]
    assert checked >= 12
    opts.device_greedy = False
    assert ba.generate(m, prompt, -1, opts) == toks


def test_model_invariants(ba, small_m3_gguf):
    """tests/test_mistral3_text.cpp:183-270: determinism, prefill == streamed
    decode, embed_tokens + forward_embeds == forward."""
    ids = [5, 17, 2, 31]
    a, b = _load(ba, small_m3_gguf, cap=16), _load(ba, small_m3_gguf, cap=16)
    la = a.forward(ids)
    assert np.array_equal(la, b.forward(ids))
    a.reset_cache()
    step = np.stack([a.forward_last([t]) for t in ids])
    assert a.cache_len() == len(ids)
    assert np.abs(step[-1] - la[-1]).max() <= LOGIT_TOL
    c = _load(ba, small_m3_gguf, cap=16)
    emb = c.embed_tokens(ids)
    assert emb.shape == (len(ids), c.cfg.hidden_size)
    assert np.array_equal(c.forward_embeds(emb), la)


def test_untied_without_output_weight_raises(ba, small_m3_gguf, tmp_path):
    """tests/test_mistral3_text.cpp:272-312: a config that says untied and a
    checkpoint without output.weight is a load error."""
    from conftest import SMALL_M3
    p = tmp_path / "tied.gguf"
    ba.write_synth_mistral3(ba.SynthSpec(**{**SMALL_M3, "tied": True}), str(p))
    cfg = ba.Mistral3Config.from_gguf(str(p)).text
    assert cfg.tie_word_embeddings is True
    cfg.tie_word_embeddings = False
    m = ba.Mistral3TextModel(cfg)
    with pytest.raises(Exception):
        m.load_weights(str(p))
    # tied as the file says: loads and matches the oracle
    t = _load(ba, p)
    om = oracle.Model(str(p))
    om.allocate_cache(128)
    assert np.abs(t.forward([3, 4, 5]) - om.forward([3, 4, 5])).max() <= LOGIT_TOL
