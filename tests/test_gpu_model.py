"""Model-level parity on the device through the C ABI of libbrolm.so
(brolm_qwen3_*), against the CPU oracle and the committed greedy fixture, plus
the reference's own model invariants (tests/test_qwen.cpp,
tests/test_qwen_generate.cpp).  Logit tolerance: max-abs 2e-2 against the
oracle's FP32 logits (FP16 activations and weights on the device)."""
from __future__ import annotations

import os

import numpy as np
import pytest

import oracle
from conftest import SMALL, write_synth

pytestmark = pytest.mark.gpu
LOGIT_TOL = 2e-2


@pytest.fixture(scope="module")
def ba():
    import brolm_amd
    brolm_amd.init()
    return brolm_amd


def _load(ba, path, cap=128):
    m = ba.Qwen3Model(ba.Qwen3Config.from_gguf(str(path)))
    m.load_weights(str(path))
    m.allocate_cache(cap)
    return m


@pytest.mark.parametrize("which", ["small_gguf", "small_q8_gguf"])
def test_prefill_and_decode_logits_vs_oracle(ba, which, request):
    path = request.getfixturevalue(which)
    print(f"[model] {which}", flush=True)
    m = _load(ba, path)
    om = oracle.Model(str(path))
    om.allocate_cache(128)
    V = m.cfg.vocab_size
    ids = [1, 2, 3, 4, V - 1, 17, 0, 300]
    assert m.decode_mode() == "persistent"
    got = m.forward(ids)
    want = om.forward(ids)
    assert got.shape == (len(ids), V) and np.isfinite(got).all()
    assert np.abs(got - want).max() <= LOGIT_TOL
    assert m.cache_len() == len(ids)
    # single-token steps: the fused, graph-captured decode step
    for t in (5, 9, V - 2, 44, 11, 0):
        a = m.forward_last([t])
        b = om.forward([t], last_only=True)[0]
        assert np.abs(a - b).max() <= LOGIT_TOL
    assert m.cache_len() == len(ids) + 6


def test_greedy_32_tokens_match_golden(ba, small_gguf):
    from golden import load_model_small
    fx = load_model_small()
    m = _load(ba, small_gguf)
    opts = ba.GenerateOptions(max_new_tokens=32, sampling=ba.SamplingParams(temperature=0.0), stop_on_eos=False)
    toks = ba.generate(m, fx["prompt"].tolist(), -1, opts)
    assert toks == fx["tokens"].tolist(), (toks, fx["tokens"].tolist(), fx["margins"].tolist())
    # the host loop (logits download + host argmax, generate.h:78-123) agrees
    opts.device_greedy = False
    assert ba.generate(m, fx["prompt"].tolist(), -1, opts) == toks


def test_prefill_equals_streamed_decode(ba, small_gguf):
    """tests/test_qwen.cpp:214-248 (FP16 tolerance instead of FP32 rel 1e-4)."""
    ids = [11, 250, 3, 999, 42, 7, 600, 5, 5, 81]
    m = _load(ba, small_gguf)
    full = m.forward(ids)
    m.reset_cache()
    step = np.stack([m.forward_last([t]) for t in ids])
    assert np.abs(full - step).max() <= LOGIT_TOL


def test_bitwise_determinism(ba, small_gguf):
    """tests/test_qwen.cpp:203-211."""
    ids = [9, 8, 7, 6, 5]
    a = _load(ba, small_gguf)
    b = _load(ba, small_gguf)
    assert np.array_equal(a.forward(ids), b.forward(ids))
    assert np.array_equal(a.forward_last([3]), b.forward_last([3]))
    assert a.decode_greedy(4, 16) == b.decode_greedy(4, 16)


def test_forward_embeds_splice_identity(ba, small_gguf):
    """tests/test_qwen.cpp:250-283: forward(ids) == forward_embeds(embed_tokens(ids)) bitwise."""
    ids = [1, 500, 2, 999, 3]
    m = _load(ba, small_gguf)
    la, ha = m.forward(ids, want_hidden=True)
    m.reset_cache()
    lb, hb = m.forward_embeds(m.embed_tokens(ids), want_hidden=True)
    assert np.array_equal(la, lb) and np.array_equal(ha, hb)
    om = oracle.Model(str(small_gguf))
    om.allocate_cache(16)
    _, ho = om.forward(ids, want_hidden=True)
    assert np.abs(ha - ho).max() <= LOGIT_TOL * max(1.0, np.abs(ho).max())


def test_truncate_cache_replays_bitwise(ba, small_gguf):
    """tests/test_qwen.cpp:285-338: speculative draft, rollback, replay."""
    m = _load(ba, small_gguf)
    m.forward([1, 2, 3, 4, 5])
    anchor = m.cache_len()
    draft = [m.forward_last([t]) for t in (9, 8, 7)]
    assert m.cache_len() == anchor + 3
    m.truncate_cache(anchor)
    assert m.cache_len() == anchor
    replay = [m.forward_last([t]) for t in (9, 8, 7)]
    assert all(np.array_equal(a, b) for a, b in zip(draft, replay))


def test_teacher_forced_argmax_equals_greedy(ba, small_gguf):
    """tests/test_qwen_generate.cpp:282-323 on the device."""
    prompt = [5, 17, 2, 31]
    m = _load(ba, small_gguf)
    opts = ba.GenerateOptions(max_new_tokens=10, sampling=ba.SamplingParams(temperature=0.0), stop_on_eos=False)
    toks = ba.generate(m, prompt, -1, opts)
    m2 = _load(ba, small_gguf)
    lg = m2.forward(prompt + toks[:-1])
    tf = [int(lg[len(prompt) - 1 + k].argmax()) for k in range(len(toks))]
    om = oracle.Model(str(small_gguf))
    om.allocate_cache(32)
    margins = [oracle.argmax(r)[1] for r in om.forward(prompt + toks[:-1])[len(prompt) - 1:]]
    # prefill (GEMM) and decode (GEMV) round differently: compare where the oracle's top-2 gap is resolvable
    assert all(a == b for a, b, g in zip(tf, toks, margins) if g > 2 * LOGIT_TOL)


def test_generate_lengths_eos_and_sampling(ba, small_gguf):
    """tests/test_qwen_generate.cpp:245-280 plus the EOS stop of generate.h:106-119."""
    m = _load(ba, small_gguf)
    prompt = [5, 17, 2, 31]
    opts = ba.GenerateOptions(max_new_tokens=12, sampling=ba.SamplingParams(temperature=0.0), stop_on_eos=False)
    out = ba.generate(m, prompt, -1, opts)
    assert len(out) == 12 and all(0 <= t < m.cfg.vocab_size for t in out)
    eos = out[3]
    opts.stop_on_eos = True
    stopped = ba.generate(m, prompt, eos, opts)
    assert stopped == out[:out.index(eos)]  # the EOS id itself is not returned
    opts.device_greedy = False
    assert ba.generate(m, prompt, eos, opts) == stopped
    s = ba.SamplingParams(temperature=0.8, top_k=20, top_p=0.9, seed=1234)
    o1 = ba.generate(m, prompt, -1, ba.GenerateOptions(max_new_tokens=10, sampling=s, stop_on_eos=False))
    o2 = ba.generate(m, prompt, -1, ba.GenerateOptions(max_new_tokens=10, sampling=s, stop_on_eos=False))
    assert o1 == o2 and len(o1) == 10


def test_generate_text_matches_oracle(ba, small_gguf):
    """qwen::generate_text (src/qwen_generate.cpp:19-25) on the checkpoint's own
    tokenizer: the prompt encodes to the oracle tokenizer's ids, the text is the
    decode of the greedy ids (oracle tokenizer, same bytes), and each greedy id
    is the oracle model's teacher-forced argmax wherever its top-2 gap is
    resolvable at the logit tolerance."""
    from gguf_meta import read_metadata
    from oracle import tokenizer as otok
    meta = read_metadata(str(small_gguf))
    orc_tok = otok.Tokenizer.from_lists(meta["tokenizer.ggml.tokens"], meta["tokenizer.ggml.merges"],
                                        meta["tokenizer.ggml.token_type"])
    tok = ba.Tokenizer.from_gguf(str(small_gguf))
    m = _load(ba, small_gguf)
    om = oracle.Model(str(small_gguf))
    for prompt in ("The model reads the tokens of the prompt.", "<|im_start|>user\nhi cat<|im_end|>\n"):
        ids = tok.encode(prompt)
        assert ids == orc_tok.encode(prompt)
        opts = ba.GenerateOptions(max_new_tokens=16, sampling=ba.SamplingParams(temperature=0.0))
        text = ba.generate_text(m, tok, prompt, opts)
        gen = ba.generate(m, ids, tok.eos_id(), opts)
        assert text == tok.decode(gen)
        assert tok.decode_bytes(gen) == orc_tok.decode_bytes(gen)
        om.reset_cache()
        om.allocate_cache(len(ids) + len(gen) + 1)
        rows = om.forward(ids + gen[:-1])[len(ids) - 1:]
        checked = 0
        for t, row in zip(gen, rows):
            a, _ = oracle.argmax(row)
            top2 = np.sort(row)[-2:]
            if top2[1] - top2[0] > 2 * LOGIT_TOL:
                assert t == a
                checked += 1
        assert checked >= 1


def _session(m, env: dict) -> str:
    """Create the model's step session under `env` (the switches are read when
    the session is created) and return its mode."""
    saved = {k: os.environ.get(k) for k in env}
    os.environ.update(env)
    try:
        return m.decode_mode()
    finally:
        for k, v in saved.items():
            if v is None:
                os.environ.pop(k, None)
            else:
                os.environ[k] = v


def test_graph_step_equals_eager_step(ba, small_gguf):
    """dense_decoder.cpp:335-524: the captured step replays the same kernels as
    the eager step (BROLM_NO_GRAPH), so logits agree bitwise."""
    g = _load(ba, small_gguf)
    assert _session(g, {"BROLM_NO_PERSIST": "1"}) == "graph"
    e = _load(ba, small_gguf)
    assert _session(e, {"BROLM_NO_GRAPH": "1"}) == "eager"
    ids = [3, 1, 4, 1, 5]
    g.forward(ids)
    e.forward(ids)
    for t in (9, 2, 6, 5):
        assert np.array_equal(g.forward_last([t]), e.forward_last([t]))
    assert g.decode_greedy(3, 12) == e.decode_greedy(3, 12)


@pytest.mark.parametrize("which", ["small_gguf", "small_q8_gguf"])
def test_persistent_step_matches_graph_step(ba, which, request):
    """The single-launch step computes the same step as the per-stage kernels
    (same GEMV cores; attention splits differ, so FP rounding may too)."""
    path = request.getfixturevalue(which)
    p = _load(ba, path)
    assert _session(p, {}) == "persistent"
    g = _load(ba, path)
    assert _session(g, {"BROLM_NO_PERSIST": "1"}) == "graph"
    ids = [3, 1, 4, 1, 5, 9, 2, 6]
    p.forward(ids)
    g.forward(ids)
    for t in (5, 3, 5, 8, 9, 7):
        a, b = p.forward_last([t]), g.forward_last([t])
        assert np.abs(a - b).max() <= LOGIT_TOL / 4
    assert p.decode_greedy(3, 16) == g.decode_greedy(3, 16)
    assert p.cache_len() == g.cache_len() == len(ids) + 6 + 16


def test_persistent_step_many_splits_vs_oracle(ba, small_gguf):
    """Context beyond one 64-key tile: several attention splits per KV head,
    merged by split 0 of each group, against the oracle."""
    m = _load(ba, small_gguf, cap=700)
    assert m.decode_mode() == "persistent"
    om = oracle.Model(str(small_gguf))
    om.allocate_cache(700)
    prompt = ba.prompt_ids(600, m.cfg.vocab_size, seed=42)
    m.forward_last(prompt)
    b = om.forward(prompt, last_only=True)[0]
    tok = int(b.argmax())
    for _ in range(6):
        a = m.forward_last([tok])
        b = om.forward([tok], last_only=True)[0]
        assert np.abs(a - b).max() <= LOGIT_TOL
        tok = int(b.argmax())


def test_persistent_tag_cycles_are_invisible(ba, small_gguf):
    """The hand-off words carry 16-bit tags, re-initialized every 63 launches:
    150 steps cross two cycle boundaries, at different steps in two models
    (one ran 37 extra steps first).  Greedy tokens are identical, and the
    logits after the boundaries still match the oracle."""
    a = _load(ba, small_gguf, cap=256)
    b = _load(ba, small_gguf, cap=256)
    assert a.decode_mode() == b.decode_mode() == "persistent"
    prompt = [3, 1, 4, 1, 5]
    a.forward(prompt)
    b.forward(prompt)
    b.decode_greedy(9, 37)
    b.truncate_cache(len(prompt))
    ta = a.decode_greedy(2, 150)
    tb = b.decode_greedy(2, 150)
    assert ta == tb
    got = a.forward_last([ta[-1]])
    om = oracle.Model(str(small_gguf))
    om.allocate_cache(256)
    want = om.forward(prompt + [2] + ta, last_only=True)[0]
    assert np.abs(got - want).max() <= LOGIT_TOL


def test_cache_errors_raise(ba, small_gguf):
    m = _load(ba, small_gguf, cap=8)
    with pytest.raises(Exception):
        m.forward(list(range(9)))           # beyond the cache capacity
    with pytest.raises(Exception):
        m.forward([m.cfg.vocab_size])       # id out of range
    with pytest.raises(Exception):
        m.truncate_cache(5)                 # longer than the cache holds
    m.forward([1, 2])
    assert m.cache_len() == 2


def test_real_width_layers_long_context(ba, tmp_path_factory):
    """The Qwen3-1.7B widths (hidden 2048, ffn 6144, 16/8 heads of 128, vocab
    151936, Q4_K with Q6_K v/down/output) over 2 layers: a 1024-token prefill
    (MFMA GEMM, split-K attention) then fused decode steps at context > 1024,
    against the oracle."""
    spec = dict(SMALL, vocab=151936, hidden=2048, intermediate=6144, layers=2, n_q=16, n_kv=8, head_dim=128,
                seed=3)
    path = write_synth(tmp_path_factory.mktemp("wide"), spec, "wide")
    print("[model] wide checkpoint written", flush=True)
    prompt = ba.prompt_ids(1024, 151936, seed=42)
    m = _load(ba, path, cap=1100)
    om = oracle.Model(str(path))
    om.allocate_cache(1100)
    a = m.forward_last(prompt)
    b = om.forward(prompt, last_only=True)[0]
    print(f"[model] prefill max diff {np.abs(a - b).max():.3e}", flush=True)
    assert np.abs(a - b).max() <= LOGIT_TOL
    for t in (int(b.argmax()), 7, 151935):
        a = m.forward_last([t])
        b = om.forward([t], last_only=True)[0]
        assert np.abs(a - b).max() <= LOGIT_TOL


def test_long_prompt_fp16_layer_copies_match_oracle(ba, small_gguf, monkeypatch):
    """A pass over >= 512 rows multiplies FP16 copies of the quantized layer
    matrices (made once, when HBM allows); with BROLM_PREFILL_F16=0 it runs
    the quantized tiles.  Both match the oracle to the logit tolerance, and the
    decode steps after them stay on the quantized weights."""
    print("[model] FP16 layer copies", flush=True)
    om = oracle.Model(str(small_gguf))
    om.allocate_cache(700)
    V = 1000
    rng = np.random.default_rng(21)
    prompt = rng.integers(0, V, 600).tolist()
    want = om.forward(prompt, last_only=True)[0]
    nxt = om.forward([7], last_only=True)[0]
    got = {}
    for mode in ("copies", "quantized"):
        if mode == "quantized":
            monkeypatch.setenv("BROLM_PREFILL_F16", "0")
        m = _load(ba, small_gguf, cap=700)
        got[mode] = m.forward_last(prompt)
        step = m.forward_last([7])
        monkeypatch.delenv("BROLM_PREFILL_F16", raising=False)
        assert np.abs(got[mode] - want).max() <= LOGIT_TOL, mode
        assert np.abs(step - nxt).max() <= LOGIT_TOL, mode
        assert m.decode_mode() == "persistent"
        m.close()
