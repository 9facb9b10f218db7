"""Pins of the CPU oracle (oracle/oracle.c) against mathematics and an
independent encoder.  Each check is chosen so a plausible slip in the oracle
(a swapped nibble, a wrong scale index, a dropped term, a transposed operand)
fails it."""
from __future__ import annotations

import numpy as np
import pytest

import oracle
import spec_blocks as sb


# ----------------------------------------------------------------- binary16 / bfloat16

def test_f16_to_f32_exhaustive():
    bits = np.arange(65536, dtype=np.uint32).astype(np.uint16)
    got = oracle.f16_to_f32(bits)
    want = bits.view(np.float16).astype(np.float32)
    nan = np.isnan(want)
    assert np.array_equal(np.isnan(got), nan)
    assert np.array_equal(got[~nan].view(np.uint32), want[~nan].view(np.uint32))


def test_f16_roundtrip_exhaustive():
    bits = np.arange(65536, dtype=np.uint32).astype(np.uint16)
    f = bits.view(np.float16).astype(np.float32)
    back = oracle.f32_to_f16(f)
    ok = ~np.isnan(f)
    assert np.array_equal(back[ok], bits[ok])
    assert np.all(np.isnan(back[~ok].view(np.float16)))


def test_f32_to_f16_rne_with_subnormals_and_ties():
    rng = np.random.default_rng(0)
    # random magnitudes across the whole binary16 range, incl. subnormals and overflow
    x = (rng.standard_normal(200000) * np.exp2(rng.uniform(-30, 18, 200000))).astype(np.float32)
    # exact halfway points between neighbouring binary16 values (ties -> even)
    h = np.arange(0, 0x7BFF, 7, dtype=np.uint16)
    lo = h.view(np.float16).astype(np.float64)
    hi = (h + 1).view(np.float16).astype(np.float64)
    mids = ((lo + hi) / 2).astype(np.float32)
    x = np.concatenate([x, mids, -mids])
    with np.errstate(over="ignore"):  # values beyond 65504 round to +-inf on both sides
        want = x.astype(np.float16).view(np.uint16)
    assert np.array_equal(oracle.f32_to_f16(x), want)


def _bf16_rne(x: np.ndarray) -> np.ndarray:
    """Nearest bfloat16 by comparing the two candidate truncations in float64."""
    b = x.view(np.uint32)
    lo = (b & 0xFFFF0000).view(np.float32).astype(np.float64)
    hi_bits = (b & 0xFFFF0000) + 0x10000
    hi = hi_bits.view(np.float32).astype(np.float64)
    xd = x.astype(np.float64)
    dlo, dhi = np.abs(xd - lo), np.abs(hi - xd)
    pick_hi = (dhi < dlo) | ((dhi == dlo) & (((b >> 16) & 1) == 1))
    return np.where(pick_hi, hi_bits >> 16, b >> 16).astype(np.uint16)


def test_bf16_conversions():
    lib = oracle.lib()
    rng = np.random.default_rng(1)
    x = (rng.standard_normal(20000) * np.exp2(rng.uniform(-20, 20, 20000))).astype(np.float32)
    want = _bf16_rne(x)
    got = np.array([lib.or_f32_to_bf16(float(v)) for v in x], np.uint16)
    assert np.array_equal(got, want)
    back = np.array([lib.or_bf16_to_f32(int(v)) for v in want[:2000]], np.float32)
    assert np.array_equal(back.view(np.uint32), want[:2000].astype(np.uint32) << 16)


# ----------------------------------------------------------------- Q4_K 6-bit scales

def test_scale_min_k4_is_the_spec_bijection():
    """Every one of the 96 scale bits lands in exactly one (j, sc|m, bit) slot,
    the same slot the element-wise packer puts it in."""
    seen = {}
    for bit in range(96):
        s = bytearray(12)
        s[bit // 8] = 1 << (bit % 8)
        hits = []
        for j in range(8):
            sc, m = oracle.scale_min_k4(j, bytes(s))
            for field, v in (("sc", sc), ("m", m)):
                if v:
                    assert v & (v - 1) == 0, "a single input bit produced several output bits"
                    hits.append((j, field, v.bit_length() - 1))
        assert len(hits) == 1, f"scale bit {bit} maps to {hits}"
        seen[hits[0]] = bit
    assert len(seen) == 96
    for (j, field, b), bit in seen.items():
        sc = np.zeros(8, np.uint8)
        m = np.zeros(8, np.uint8)
        (sc if field == "sc" else m)[j] = 1 << b
        packed = sb.pack_scales_k4(sc, m)
        assert packed[bit // 8] == 1 << (bit % 8) and packed.sum() == packed[bit // 8]


def test_scale_min_k4_random_roundtrip():
    rng = np.random.default_rng(2)
    for _ in range(500):
        sc = rng.integers(0, 64, 8).astype(np.uint8)
        m = rng.integers(0, 64, 8).astype(np.uint8)
        s = sb.pack_scales_k4(sc, m).tobytes()
        for j in range(8):
            assert oracle.scale_min_k4(j, s) == (sc[j], m[j])


# ----------------------------------------------------------------- block dequant

@pytest.mark.parametrize("t", [oracle.T_Q8_0, oracle.T_Q4_K, oracle.T_Q6_K])
def test_dequant_matches_independent_encoder(t):
    rng = np.random.default_rng(t)
    raw, want = sb.random_blocks(rng, t, 400, extremes=True)
    got = oracle.dequant(t, raw, want.size)
    assert np.array_equal(got.view(np.uint32), want.view(np.uint32))


@pytest.mark.parametrize("t", [oracle.T_Q8_0, oracle.T_Q4_K, oracle.T_Q6_K])
def test_dequant_zero_blocks(t):
    n = sb.QK[t] * 3
    got = oracle.dequant(t, bytes(sb.BB[t] * 3), n)
    assert np.all(got == 0)


def test_dequant_q4k_subnormal_scales_and_zero_d():
    rng = np.random.default_rng(3)
    nb = 64
    d = sb.random_f16(rng, nb, lo_exp=-14, hi_exp=-14, sign=False) * np.float16(1 / 256)  # subnormal
    dmin = sb.random_f16(rng, nb, lo_exp=-14, hi_exp=-14, sign=False) * np.float16(1 / 64)
    d[:8] = 0
    dmin[8:16] = 0
    sc = rng.integers(0, 64, (nb, 8))
    m = rng.integers(0, 64, (nb, 8))
    q = rng.integers(0, 16, (nb, 256))
    raw = sb.enc_q4_k(d, dmin, sc, m, q)
    want = sb.val_q4_k(d, dmin, sc, m, q)
    got = oracle.dequant(oracle.T_Q4_K, raw, want.size)
    assert np.array_equal(got.view(np.uint32), want.view(np.uint32))


def test_dequant_golden_fixture():
    """Committed vectors (tests/golden/make_golden.py): raw blocks plus the FP32
    and FP16 bit patterns the decoder must produce."""
    from golden import load_blocks
    for t, raw, f32_bits, f16_bits in load_blocks():
        got = oracle.dequant(t, raw, f32_bits.size)
        assert np.array_equal(got.view(np.uint32), f32_bits)
        assert np.array_equal(oracle.f32_to_f16(got), f16_bits)


# ----------------------------------------------------------------- FP32 ops vs float64 closed forms

def test_rms_norm_closed_form():
    rng = np.random.default_rng(4)
    x = rng.standard_normal((7, 384)).astype(np.float32) * 3
    g = rng.uniform(0.5, 1.5, 384).astype(np.float32)
    xd = x.astype(np.float64)
    want = xd / np.sqrt((xd * xd).mean(1, keepdims=True) + 1e-6) * g
    np.testing.assert_allclose(oracle.rms_norm(x, g, 1e-6), want, rtol=2e-6, atol=1e-6)


def _rope_hf_rotate_half(x, hd, n_heads, pos0, theta):
    """HF Qwen3 rotary embedding (rotate_half form) in float64."""
    L = x.shape[0]
    inv = theta ** (-np.arange(0, hd, 2, dtype=np.float64) / hd)
    ang = (pos0 + np.arange(L, dtype=np.float64))[:, None] * inv[None, :]
    cos = np.concatenate([np.cos(ang), np.cos(ang)], 1)[:, None, :]
    sin = np.concatenate([np.sin(ang), np.sin(ang)], 1)[:, None, :]
    v = x.astype(np.float64).reshape(L, n_heads, hd)
    rot = np.concatenate([-v[..., hd // 2:], v[..., :hd // 2]], -1)
    return (v * cos + rot * sin).reshape(L, n_heads * hd)


@pytest.mark.parametrize("hd,pos0", [(64, 0), (128, 1000), (128, 40000)])
def test_rope_interleaved_on_permuted_equals_rotate_half(hd, pos0):
    """The load-time row permute (dst rows 2i, 2i+1 <- src rows i, i+hd/2,
    include/brolm/detail/weights.h:132-148) makes the interleaved-pair RoPE
    reproduce HF's rotate_half exactly up to that permutation."""
    rng = np.random.default_rng(hd + pos0)
    n_heads, L, theta = 3, 5, 1e6
    x = rng.standard_normal((L, n_heads * hd)).astype(np.float32)
    perm = np.empty(hd, np.int64)
    perm[0::2] = np.arange(hd // 2)
    perm[1::2] = np.arange(hd // 2) + hd // 2
    xp = x.reshape(L, n_heads, hd)[..., perm].reshape(L, -1)
    got = oracle.rope(xp, hd, n_heads, pos0, theta).reshape(L, n_heads, hd)
    want = _rope_hf_rotate_half(x, hd, n_heads, pos0, theta).reshape(L, n_heads, hd)[..., perm]
    np.testing.assert_allclose(got, want, atol=2e-5 * np.abs(x).max() * max(1.0, pos0 / 1e3))


def test_linear_closed_form():
    rng = np.random.default_rng(5)
    W = rng.standard_normal((37, 512)).astype(np.float32)
    X = rng.standard_normal((3, 512)).astype(np.float32)
    want = X.astype(np.float64) @ W.astype(np.float64).T
    np.testing.assert_allclose(oracle.linear(W, X), want, rtol=1e-5, atol=1e-4)


def _attention_f64(q, K, V, L, pos0, n_q, n_kv, hd):
    out = np.zeros((L, n_q * hd))
    G = n_q // n_kv
    for r in range(L):
        p = pos0 + r
        for h in range(n_q):
            g = h // G
            qv = q[r, h * hd:(h + 1) * hd].astype(np.float64)
            k = K[:p + 1, g * hd:(g + 1) * hd].astype(np.float64)
            v = V[:p + 1, g * hd:(g + 1) * hd].astype(np.float64)
            s = k @ qv / np.sqrt(hd)
            w = np.exp(s - s.max())
            out[r, h * hd:(h + 1) * hd] = (w / w.sum()) @ v
    return out


@pytest.mark.parametrize("L,pos0,n_q,n_kv,hd", [(1, 0, 4, 2, 64), (3, 9, 8, 2, 64), (1, 130, 16, 8, 128)])
def test_attention_causal_gqa(L, pos0, n_q, n_kv, hd):
    rng = np.random.default_rng(L * 100 + pos0)
    T = pos0 + L
    q = rng.standard_normal((L, n_q * hd)).astype(np.float32)
    K = rng.standard_normal((T, n_kv * hd)).astype(np.float32)
    V = rng.standard_normal((T, n_kv * hd)).astype(np.float32)
    got = oracle.attention(q, K, V, L, pos0, n_q, n_kv, hd)
    np.testing.assert_allclose(got, _attention_f64(q, K, V, L, pos0, n_q, n_kv, hd), atol=2e-5)


def test_argmax_lowest_index_on_ties():
    x = np.zeros(100, np.float32)
    x[[17, 42, 99]] = 5.0
    x[3] = 4.0
    i, margin = oracle.argmax(x)
    assert i == 17 and margin == 0.0
    x[42] = 6.0
    i, margin = oracle.argmax(x)
    assert i == 42 and margin == 1.0


# ----------------------------------------------------------------- GGUF reader vs the product writer

def test_gguf_reader_reads_product_writer(small_gguf, native):
    import ctypes as C
    g = oracle.Gguf(str(small_gguf))
    names = g.tensor_names()
    n = C.c_int64()
    assert native.lib().brolm_gguf_tensor_count(str(small_gguf).encode(), C.byref(n)) == 0
    assert n.value == len(names) == 2 + 1 + 2 * 11
    assert g.meta_str("general.architecture") == "qwen3"
    assert g.meta_int("qwen3.block_count") == 2
    assert g.meta_int("qwen3.embedding_length") == 256
    t, dims, raw = g.tensor("blk.1.attn_v.weight")
    assert t == oracle.T_Q6_K and dims == [256, 2 * 64] and raw.size == 128 * 256 // 256 * 210
    t, dims, raw = g.tensor("output_norm.weight")
    assert t == oracle.T_F32 and dims == [256] and np.all(raw.view(np.float32) == 1.0)
