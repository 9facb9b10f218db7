"""Multi-sequence batched decode on the device (brolm_qwen3_allocate_batch /
_prefill_slot / _forward_batch): every row of a batched step must give the
logits that sequence gets alone.  The checker is one CPU oracle model per
sequence (the reference's one-sequence DenseDecoder semantics,
src/detail/dense_decoder.cpp:231-329, 526-681), fed the same tokens.
Logit tolerance: max-abs 2e-2 against the oracle's FP32 logits, as for the
one-sequence model tests."""
from __future__ import annotations

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


def _model(ba, path, arch):
    if arch == "mistral3":
        m = ba.Mistral3TextModel(ba.Mistral3Config.from_gguf(str(path)).text)
    else:
        m = ba.Qwen3Model(ba.Qwen3Config.from_gguf(str(path)))
    m.load_weights(str(path))
    return m


def _oracles(path, n, cap):
    out = []
    for _ in range(n):
        om = oracle.Model(str(path))
        om.allocate_cache(cap)
        out.append(om)
    return out


@pytest.mark.parametrize("which,arch", [("small_gguf", "qwen3"), ("small_q8_gguf", "qwen3"),
                                        ("small_m3_gguf", "mistral3")])
def test_batched_steps_match_each_sequence_alone(ba, which, arch, request):
    """Ragged prompts in non-contiguous slots, then steps over changing
    subsets of the slots in shuffled row order (M from 1 to 5), then all 8."""
    path = request.getfixturevalue(which)
    print(f"[batch] {which}", flush=True)
    cap = 64
    m = _model(ba, path, arch)
    m.allocate_batch(8, cap)
    V = m.cfg.vocab_size
    rng = np.random.default_rng(5)
    slots = [0, 2, 3, 5, 7]
    lens = [1, 7, 3, 19, 12]
    om = dict(zip(slots, _oracles(path, len(slots), cap)))
    for s, n in zip(slots, lens):
        prompt = rng.integers(0, V, n).tolist()
        got = m.prefill_slot(s, prompt)
        want = om[s].forward(prompt, last_only=True)[0]
        assert np.abs(got - want).max() <= LOGIT_TOL, f"prefill slot {s}"
        assert m.slot_len(s) == n
    steps = [[0, 2, 3, 5, 7], [7, 0, 3], [5], [2, 7, 5, 0], [3, 2, 0, 7, 5], [0, 5]]
    # then every slot: 8 rows (the residual norms carried by the GEMV launches)
    for s in (1, 4, 6):
        prompt = rng.integers(0, V, 4 + s).tolist()
        m.prefill_slot(s, prompt)
        om[s] = _oracles(path, 1, cap)[0]
        om[s].forward(prompt, last_only=True)
        lens.append(4 + s)
        slots.append(s)
    steps += [[6, 1, 0, 3, 5, 2, 7, 4], [0, 1, 2, 3, 4, 5, 6, 7]]
    for step in steps:
        ids = rng.integers(0, V, len(step)).tolist()
        got = m.forward_batch(ids, step)
        assert got.shape == (len(step), V) and np.isfinite(got).all()
        for r, (s, t) in enumerate(zip(step, ids)):
            want = om[s].forward([t], last_only=True)[0]
            err = np.abs(got[r] - want).max()
            assert err <= LOGIT_TOL, f"step {step} row {r} slot {s}: {err}"
    for s, n in zip(slots, lens):
        assert m.slot_len(s) == n + sum(s in st for st in steps[6 if s in (1, 4, 6) else 0:])
    m.close()


def test_sixteen_rows_and_long_slots(ba, small_gguf):
    """M = 16 (the widest MFMA-GEMV row count) with slots past several
    attention splits; then a truncated slot replays bit-for-bit."""
    print("[batch] 16 rows", flush=True)
    cap = 640
    m = _model(ba, small_gguf, "qwen3")
    m.allocate_batch(16, cap)
    V = m.cfg.vocab_size
    rng = np.random.default_rng(9)
    lens = [int(x) for x in rng.integers(1, 600, 16)]
    oms = _oracles(small_gguf, 16, cap)
    for s in range(16):
        prompt = rng.integers(0, V, lens[s]).tolist()
        m.prefill_slot(s, prompt)
        oms[s].forward(prompt, last_only=True)
    order = rng.permutation(16).tolist()
    ids = rng.integers(0, V, 16).tolist()
    got = m.forward_batch(ids, order)
    for r, s in enumerate(order):
        want = oms[s].forward([ids[r]], last_only=True)[0]
        assert np.abs(got[r] - want).max() <= LOGIT_TOL, f"row {r} slot {s}"
    # drop the step from every slot and repeat it: identical logits
    for s in range(16):
        m.truncate_slot(s, lens[s])
    again = m.forward_batch(ids, order)
    assert np.array_equal(got, again)
    m.close()


def test_batch_leaves_the_single_sequence_cache_alone(ba, small_gguf):
    print("[batch] isolation", flush=True)
    m = _model(ba, small_gguf, "qwen3")
    m.allocate_cache(64)
    m.allocate_batch(4, 64)
    V = m.cfg.vocab_size
    a = m.forward([3, 4, 5, 6])
    m.prefill_slot(1, [9, 8, 7])
    m.forward_batch([1, 2], [1, 3])
    assert m.cache_len() == 4
    b = m.forward_last([10])
    om = oracle.Model(str(small_gguf))
    om.allocate_cache(64)
    om.forward([3, 4, 5, 6])
    assert np.abs(b - om.forward([10], last_only=True)[0]).max() <= LOGIT_TOL
    assert a.shape == (4, V)
    m.close()


def test_batch_errors_raise(ba, small_gguf):
    print("[batch] errors", flush=True)
    m = _model(ba, small_gguf, "qwen3")
    with pytest.raises(ba._native.NativeError, match="not allocated"):
        m.forward_batch([1], [0])
    m.allocate_batch(3, 8)
    with pytest.raises(ba._native.NativeError, match="appears twice"):
        m.forward_batch([1, 2], [1, 1])
    with pytest.raises(ba._native.NativeError, match="out of range"):
        m.forward_batch([1], [3])
    with pytest.raises(ba._native.NativeError, match="token id out of range"):
        m.forward_batch([m.cfg.vocab_size], [0])
    with pytest.raises(ba._native.NativeError, match="M must be"):
        m.forward_batch([1, 2, 3, 4], [0, 1, 2, 0])
    with pytest.raises(ba._native.NativeError, match="exceeds"):
        m.prefill_slot(0, list(range(9)))
    m.prefill_slot(0, list(range(8)))
    with pytest.raises(ba._native.NativeError, match="slot is full"):
        m.forward_batch([1], [0])
    with pytest.raises(ba._native.NativeError, match="truncate_slot"):
        m.truncate_slot(1, 1)
    m.truncate_slot(0, 7)
    assert m.slot_len(0) == 7
    m.forward_batch([1], [0])
    assert m.slot_len(0) == 8
    m.close()


def test_batched_graph_replays_equal_eager(ba, small_gguf, monkeypatch):
    """The second step of a given M is captured into a hipGraph and later steps
    replay it; every replay must equal the eager step bit for bit, also with
    other device work (a prefill into another slot, single-sequence steps) and
    host synchronisation between the replays."""
    print("[batch] graph vs eager", flush=True)
    models = {}
    for mode in ("graph", "eager"):
        if mode == "eager":
            monkeypatch.setenv("BROLM_NO_GRAPH", "1")
        m = _model(ba, small_gguf, "qwen3")
        m.allocate_cache(32)
        m.allocate_batch(10, 48)
        monkeypatch.delenv("BROLM_NO_GRAPH", raising=False)
        models[mode] = m
    V = models["graph"].cfg.vocab_size
    rng = np.random.default_rng(3)
    for s, n in zip(range(8), (3, 9, 1, 5, 2, 7, 4, 6)):
        prompt = rng.integers(0, V, n).tolist()
        for m in models.values():
            m.prefill_slot(s, prompt)
    # 4 rows (norms on their own) and 8 rows (norms carried by the GEMVs)
    for step in range(6):
        M = 4 if step % 2 == 0 else 8
        ids = rng.integers(0, V, M).tolist()
        order = rng.permutation(M).tolist()
        out = {k: m.forward_batch(ids, order) for k, m in models.items()}
        assert np.array_equal(out["graph"], out["eager"]), f"step {step}"
        # unrelated device work between replays
        for m in models.values():
            m.prefill_slot(9, [int(step) + 1])
            m.forward_last([7])
    for m in models.values():
        m.close()


@pytest.mark.parametrize("hd,norm", [(128, True), (64, True), (256, True), (128, False)])
def test_qk_rope_kv_rows_equals_separate_ops(hd, norm):
    """bx_qk_rope_kv_rows_f16 (the per-head stage of a batched step in one
    launch) gives exactly the bits of its three separate launches: head
    rms_norm of q and k (when gains are given), rope_rows at each row's own
    position, kv_append_rows into scattered cache rows; cache rows not written
    stay as they were."""
    from gpu_util import call, dev, f16_dev, host, ptr, stream, torch
    import ctypes as C
    print(f"[batch] qk_rope_kv hd={hd} norm={norm}", flush=True)
    rng = np.random.default_rng(hd + norm)
    M, n_q, n_kv, cap, tab = 7, 8, 2, 50, 64
    width = n_kv * hd
    q = rng.standard_normal((M, n_q * hd)) * 3
    k = rng.standard_normal((M, width)) * 3
    v = rng.standard_normal((M, width))
    qg = rng.uniform(0.5, 1.5, hd) if norm else None
    kg = rng.uniform(0.5, 1.5, hd) if norm else None
    pos = np.array([0, 5, 63, 17, 1, 40, 33], np.int32)
    dst = np.array([3, 49, 0, 20, 7, 31, 12], np.int64)
    cos_t = np.empty((tab, hd // 2), np.float32)
    sin_t = np.empty((tab, hd // 2), np.float32)
    import brolm_amd._native as nat
    nat.hip().bx_rope_table_host(cos_t.ctypes.data_as(nat.P_f32), sin_t.ctypes.data_as(nat.P_f32), tab, hd, 1e6)
    cs, sn = dev(cos_t), dev(sin_t)
    pos_d, dst_d = dev(pos), dev(dst)
    fill = rng.integers(0, 2 ** 15, (cap, width)).astype(np.uint16)
    eps = 1e-6
    # fused
    qf = f16_dev(q)
    Kf, Vf = dev(fill), dev(fill)
    gq = f16_dev(qg) if norm else None
    gk = f16_dev(kg) if norm else None
    kd, vd = f16_dev(k), f16_dev(v)
    call("bx_qk_rope_kv_rows_f16", ptr(qf), ptr(kd), ptr(vd), M, hd, n_q, n_kv, ptr(gq), ptr(gk), C.c_float(eps),
         ptr(pos_d), ptr(cs), ptr(sn), tab, ptr(dst_d), ptr(Kf), ptr(Vf), cap, ptr(qf), stream())
    # separate
    qs, ks = f16_dev(q), f16_dev(k)
    if norm:
        call("bx_rms_norm", ptr(qs), 0, ptr(gq), C.c_float(eps), ptr(qs), M * n_q, hd, stream())
        call("bx_rms_norm", ptr(ks), 0, ptr(gk), C.c_float(eps), ptr(ks), M * n_kv, hd, stream())
    call("bx_rope_rows_f16", ptr(qs), ptr(qs), M, hd, n_q, ptr(pos_d), ptr(cs), ptr(sn), tab, stream())
    call("bx_rope_rows_f16", ptr(ks), ptr(ks), M, hd, n_kv, ptr(pos_d), ptr(cs), ptr(sn), tab, stream())
    Ks, Vs = dev(fill), dev(fill)
    call("bx_kv_append_rows_f16", ptr(ks), ptr(vd), M, width, ptr(dst_d), ptr(Ks), ptr(Vs), cap, stream())
    assert np.array_equal(host(qf), host(qs))
    assert np.array_equal(host(Kf), host(Ks)) and np.array_equal(host(Vf), host(Vs))
    untouched = np.setdiff1d(np.arange(cap), dst)
    assert np.array_equal(host(Kf).reshape(cap, width)[untouched], fill[untouched])


@pytest.mark.parametrize("hd,n_q,n_kv,norm,cap", [(128, 8, 4, True, 300), (64, 8, 2, False, 200),
                                                  (256, 2, 2, True, 150), (128, 16, 2, True, 700)])
def test_batch_attention_fused(hd, n_q, n_kv, norm, cap):
    """bx_batch_attention_f16 (q / k norm + RoPE + k / v cache write + split
    attention + merge in one launch): the cache rows it writes have exactly the
    bits of bx_qk_rope_kv_rows_f16, the output matches a float64 softmax over
    each row's own keys (atol 3e-3, as the single-sequence kernel), for ragged
    rows in scattered slots across several key tiles and splits (one row with a
    single key); a second launch gives the same bits (its counters are back at
    zero)."""
    from gpu_util import call, dev, f16_dev, f16_host, host, ptr, stream, torch
    import ctypes as C
    import brolm_amd._native as nat
    print(f"[batch] fused attention hd={hd} n_q={n_q} n_kv={n_kv} norm={norm} cap={cap}", flush=True)
    rng = np.random.default_rng(hd * 7 + n_q + cap)
    slots = [3, 0, 5, 1, 4]
    lens = [cap, 1, cap // 2 + 7, 129, 64]
    M, n_slots, width = len(slots), 6, n_kv * hd
    rows_total = n_slots * cap
    q = rng.standard_normal((M, n_q * hd))
    k = rng.standard_normal((M, width))
    v = rng.standard_normal((M, width))
    qg = rng.uniform(0.5, 1.5, hd) if norm else None
    kg = rng.uniform(0.5, 1.5, hd) if norm else None
    cache_k = (rng.standard_normal((rows_total, width)) * 0.5).astype(np.float16)
    cache_v = rng.standard_normal((rows_total, width)).astype(np.float16)
    cos_t = np.empty((cap, hd // 2), np.float32)
    sin_t = np.empty((cap, hd // 2), np.float32)
    nat.hip().bx_rope_table_host(cos_t.ctypes.data_as(nat.P_f32), sin_t.ctypes.data_as(nat.P_f32), cap, hd, 1e6)
    cs, sn = dev(cos_t), dev(sin_t)
    base = np.array([s * cap for s in slots], np.int64)
    lens_a = np.array(lens, np.int32)
    pos = lens_a - 1
    dst = base + pos
    gq = f16_dev(qg) if norm else None
    gk = f16_dev(kg) if norm else None
    qd, kd, vd = f16_dev(q), f16_dev(k), f16_dev(v)
    # the separate q / k stage (reference for the cache rows and the roped q)
    qs = f16_dev(q)
    Ks, Vs = dev(cache_k.view(np.uint16)), dev(cache_v.view(np.uint16))
    call("bx_qk_rope_kv_rows_f16", ptr(qs), ptr(kd), ptr(vd), M, hd, n_q, n_kv, ptr(gq), ptr(gk), C.c_float(1e-6),
         ptr(dev(pos)), ptr(cs), ptr(sn), cap, ptr(dev(dst)), ptr(Ks), ptr(Vs), rows_total, ptr(qs), stream())
    # fused
    Kf, Vf = dev(cache_k.view(np.uint16)), dev(cache_v.view(np.uint16))
    wsb = nat.hip().bx_batch_attention_workspace_bytes(M, n_q, n_kv, hd, cap)
    ws = torch().zeros(wsb, dtype=torch().uint8, device="cuda")
    outs = []
    for _ in range(2):
        out = torch().empty(M * n_q * hd, dtype=torch().int16, device="cuda")
        call("bx_batch_attention_f16", ptr(qd), ptr(kd), ptr(vd), M, hd, n_q, n_kv, ptr(gq), ptr(gk),
             C.c_float(1e-6), ptr(dev(lens_a)), ptr(dev(base)), cap, ptr(cs), ptr(sn), cap, ptr(Kf), ptr(Vf),
             rows_total, ptr(out), ptr(ws), stream())
        outs.append(host(out))
    assert np.array_equal(outs[0], outs[1])
    assert np.array_equal(host(Kf), host(Ks)) and np.array_equal(host(Vf), host(Vs))
    Kh = host(Ks).view(np.float16).reshape(rows_total, width)
    Vh = host(Vs).view(np.float16).reshape(rows_total, width)
    qr = f16_host(qs).reshape(M, n_q * hd)
    got = outs[0].view(np.float16).astype(np.float32).reshape(M, n_q * hd)
    G = n_q // n_kv
    for r in range(M):
        keys = np.arange(base[r], base[r] + lens[r])
        for h in range(n_q):
            g = h // G
            sc = Kh[keys, g * hd:(g + 1) * hd].astype(np.float64) @ qr[r, h * hd:(h + 1) * hd].astype(np.float64)
            w = np.exp(sc / np.sqrt(hd) - (sc / np.sqrt(hd)).max())
            ref = (w / w.sum()) @ Vh[keys, g * hd:(g + 1) * hd].astype(np.float64)
            np.testing.assert_allclose(got[r, h * hd:(h + 1) * hd], ref, atol=3e-3, err_msg=f"row {r} head {h}")
    assert not host(ws)[:256].any()   # counters back at zero
