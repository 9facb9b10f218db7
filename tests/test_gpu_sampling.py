"""Device top-k / top-p sampling (bx_sample_f16 through
brolm_sample_token_device) against the oracle's sampler (the reference's
sample_token, src/detail/generate.cpp:68-142) on the same FP16 logits and the
same std::mt19937_64 draw.

Criterion: the device id equals the oracle's, except (a) an id of equal
logit (the reference's std::sort leaves the order of equal probabilities
unspecified) or (b) a draw within 1e-5 of the kept mass from the boundary of
the oracle's interval (FP32 / FP64 summation order moves boundaries by ~1e-7);
(b) is counted and printed.  At a top-k cut both keep exactly k ids, ties
ordered by ascending id (the oracle's sort and the device agree on that
order), so ties at the cut need no exception."""
from __future__ import annotations

import ctypes as C

import numpy as np
import pytest

import oracle
from mt64 import first_uniform

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def env():
    import torch
    import brolm_amd
    from brolm_amd import _native
    brolm_amd.init()
    return torch, _native


def _distinct_fp16(rng, n, lo, hi):
    """n distinct FP16 values in [lo, hi), shuffled."""
    cand = np.unique(rng.uniform(lo, hi, 8 * n).astype(np.float16))
    assert cand.size >= n
    return rng.permutation(cand)[:n]


@pytest.mark.parametrize("V", [1000, 151936])
def test_device_sampler_matches_oracle(env, V):
    torch, nat = env
    lib = nat.lib()
    rng = np.random.default_rng(V)
    cases = [(1.0, 0, 1.0), (0.7, 50, 1.0), (1.0, 0, 0.9), (1.3, 40, 0.8), (0.5, 5, 0.5), (1.0, 0, 0.01),
             (2.0, 1000, 0.95)]
    near = total = 0
    for scale in (0.5, 3.0, 8.0):
        if V <= 2000:
            lg16 = _distinct_fp16(rng, V, -scale * 3, scale * 3)
        else:
            # the top 4000 distinct (every cut above falls among them), the
            # rest below them, FP16 ties allowed there
            lg16 = np.empty(V, np.float16)
            top = rng.choice(V, 4000, replace=False)
            rest = np.setdiff1d(np.arange(V), top)
            bits = rng.choice(np.arange(0x3C00, 0x4C40, dtype=np.uint16), 4000, replace=False)  # [1, 17)
            lg16[top] = bits.view(np.float16)
            lg16[rest] = np.minimum(rng.uniform(-scale * 3, 0.99, rest.size), 0.99).astype(np.float16)
        lg32 = lg16.astype(np.float32)
        dev = torch.from_numpy(lg16.view(np.uint16).astype(np.int16)).cuda()
        for T, k, p in cases:
            for seed in range(6):
                print(f"[sample] V={V} scale={scale} T={T} k={k} p={p} seed={seed}", flush=True)
                want, margin = oracle.sample_token(lg32, T, k, p, first_uniform(seed))
                got = lib.brolm_sample_token_device(C.c_void_p(dev.data_ptr()), V, T, k, p, seed)
                assert got >= 0, nat.lib().brolm_last_error()
                total += 1
                if got == want or lg32[got] == lg32[want]:
                    continue
                assert margin < 1e-5, (T, k, p, seed, want, got, margin)
                near += 1
    print(f"[sample] V={V}: {total} draws, {near} within 1e-5 of an interval boundary", flush=True)
    assert near <= 2


def test_device_sampler_ties_at_the_cut(env):
    """Logits from 40 FP16 values over 151936 ids, so every top-k / top-p cut
    and most draws fall inside groups of equal probability.  The oracle orders
    equal probabilities by ascending id, as the device does, so the id must be
    the oracle's exactly (draws within 1e-5 of an interval boundary aside).
    k = 6000 leaves more candidates above the histogram floor than the gathered
    path takes, so the draw over all ids runs there."""
    torch, nat = env
    lib = nat.lib()
    V = 151936
    rng = np.random.default_rng(11)
    levels = _distinct_fp16(rng, 40, -4.0, 6.0)
    lg16 = levels[rng.integers(0, levels.size, V)]
    lg32 = lg16.astype(np.float32)
    dev = torch.from_numpy(lg16.view(np.uint16).astype(np.int16)).cuda()
    near = total = 0
    for T, k, p in [(1.0, 40, 1.0), (0.8, 100, 0.9), (1.0, 0, 0.3), (1.0, 6000, 1.0), (1.5, 6000, 0.5),
                    (0.6, 2500, 0.95)]:
        for seed in range(5):
            print(f"[sample] ties T={T} k={k} p={p} seed={seed}", flush=True)
            want, margin = oracle.sample_token(lg32, T, k, p, first_uniform(seed))
            got = lib.brolm_sample_token_device(C.c_void_p(dev.data_ptr()), V, T, k, p, seed)
            assert got >= 0, nat.lib().brolm_last_error()
            total += 1
            if got != want:
                assert margin < 1e-5, (T, k, p, seed, want, got, margin)
                near += 1
    print(f"[sample] ties: {total} draws, {near} within 1e-5 of an interval boundary", flush=True)
    assert near <= 2


def test_sampled_generation_on_device_matches_host(env, small_gguf):
    """generate() with temperature sampling: the device sampler (default) and
    the host path draw, from the same seed, ids of equal probability (this
    model's logits are small, so FP16 ties are common and the reference's
    tie order is unspecified)."""
    import brolm_amd as ba
    m = ba.Qwen3Model(ba.Qwen3Config.from_gguf(str(small_gguf)))
    m.load_weights(str(small_gguf))
    prompt = [1, 2, 3]
    m.allocate_cache(8)
    lg = np.asarray(m.forward_last(prompt)).reshape(-1)
    same = 0
    for seed in range(12):
        sp = ba.SamplingParams(temperature=0.8, top_k=40, top_p=0.9, seed=seed)
        a = ba.generate(m, prompt, -1, ba.GenerateOptions(max_new_tokens=1, sampling=sp, stop_on_eos=False))
        b = ba.generate(m, prompt, -1, ba.GenerateOptions(max_new_tokens=1, sampling=sp, stop_on_eos=False,
                                                          device_sampling=False))
        assert len(a) == len(b) == 1
        assert lg[a[0]] == lg[b[0]], (seed, a, b)
        same += a == b
    sp = ba.SamplingParams(temperature=0.8, top_k=40, top_p=0.9, seed=7)
    assert len(ba.generate(m, prompt, -1, ba.GenerateOptions(max_new_tokens=24, sampling=sp,
                                                             stop_on_eos=False))) == 24


def _tie_at_cut(lg, T, k, p):
    """Whether the logit where the top-k / top-p kept set ends is shared with
    the first logit left out (float64 probabilities, enough to find the cut)."""
    srt = np.sort(lg.astype(np.float64))[::-1]
    n = srt.size if k <= 0 else min(k, srt.size)
    if n < srt.size and srt[n - 1] == srt[n]:
        return True
    pr = np.exp((srt[:n] - srt[0]) / T)
    c = np.cumsum(pr / pr.sum())
    m = min(int(np.searchsorted(c, p)) + 1, n)
    return m < srt.size and srt[m - 1] == srt[m]


@pytest.mark.parametrize("cap,op", [(64, False), (33000, False), (64, True)])
def test_device_sampled_decode_matches_per_token_sampling(env, small_gguf, monkeypatch, cap, op):
    """decode_sampled (the fused step and the device sampler back to back, no
    host round trip; with BROLM_OP_STEP=1, the op path and the sampler per
    token) picks, at every step, the oracle sampler's id for that step's own
    logits and draw (a second model fed the same tokens gives the logits), up
    to the first draw within 1e-5 of an interval boundary (criteria as above);
    an FP16 tie where the kept set ends is checked like any other step."""
    import brolm_amd as ba
    print(f"[sample] decode_sampled cap={cap} op={op}", flush=True)
    if op:
        monkeypatch.setenv("BROLM_OP_STEP", "1")
    mods = []
    for _ in range(2):
        m = ba.Qwen3Model(ba.Qwen3Config.from_gguf(str(small_gguf)))
        m.load_weights(str(small_gguf))
        m.allocate_cache(cap)
        mods.append(m)
    a, b = mods
    prompt = [5, 9, 2, 7]
    rng = np.random.default_rng(cap)
    T, k, p = 0.7, 50, 0.9
    for m in mods:
        m.forward_last(prompt)
    first = 11
    n = 32
    u = rng.random(n)
    got = a.decode_sampled(first, u, T, k, p)
    assert len(got) == n
    checked = ties = 0
    for i in range(n):
        lg = np.asarray(b.forward_last([first if i == 0 else got[i - 1]]), dtype=np.float32).reshape(-1)
        want, margin = oracle.sample_token(lg, T, k, p, float(u[i]))
        if margin < 1e-5:
            continue  # boundary draw
        assert got[i] == want, (i, got[i], want, bool(_tie_at_cut(lg, T, k, p)))
        ties += bool(_tie_at_cut(lg, T, k, p))
        checked += 1
    print(f"[sample] {checked} of {n} steps checked, {ties} with an FP16 tie at the cut", flush=True)
    assert checked >= n // 3
    assert a.cache_len() == len(prompt) + n
    for m in mods:
        m.close()
