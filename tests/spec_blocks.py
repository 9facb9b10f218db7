"""Independent GGUF block packer for the tests (public ggml block formats).

The oracle and the device kernels DECODE blocks chunk by chunk; this module
ENCODES them element by element from the published layout, so a misplaced
nibble, bit pair, scale index or sign in a decoder shows up as a mismatch:

  Q8_0  34 B / 32:  {f16 d; i8 qs[32]}                      y = d*q
  Q4_K 144 B / 256: {f16 d; f16 dmin; u8 scales[12]; u8 qs[128]}
        element e: sub-block s = e//32 (6-bit sc[s], m[s]), byte qs[32*(e//64) + e%32],
        low nibble when e%64 < 32, else high nibble;  y = d*sc[s]*q - dmin*m[s]
        scales: s<4: low 6 bits of scales[s] = sc[s], of scales[s+4] = m[s];
        s>=4: scales[s+4] = (sc[s]&15) | (m[s]&15)<<4, the top two bits of
        sc[s] in bits 6-7 of scales[s-4] and of m[s] in bits 6-7 of scales[s]
  Q6_K 210 B / 256: {u8 ql[128]; u8 qh[64]; i8 scales[16]; f16 d}
        element e: half = e//128, quarter = (e%128)//32, l = e%32;
        ql byte 64*half + l + 32*(quarter&1), low nibble for quarter<2 else high;
        qh byte 32*half + l, bits 2*quarter..+1;  q = (ql4 | qh2<<4) - 32;
        y = d*scales[e//16]*q

Expected values are computed from the KNOWN integers in float64 (exact here:
every product has < 32 significant bits and the test exponents keep each
difference inside 53 bits) and rounded once to float32, which is what a
correctly rounded FP32 evaluation of the formula gives.
"""
from __future__ import annotations

import numpy as np

QK = {8: 32, 12: 256, 14: 256}
BB = {8: 34, 12: 144, 14: 210}


def f16_bits(x) -> np.ndarray:
    return np.asarray(x, np.float16).view(np.uint16)


def pack_scales_k4(sc: np.ndarray, m: np.ndarray) -> np.ndarray:
    """8 six-bit (sc, m) pairs -> the 12 scale bytes of a Q4_K block."""
    assert sc.shape == (8,) and m.shape == (8,) and sc.max() < 64 and m.max() < 64
    s = np.zeros(12, np.uint8)
    for j in range(8):
        if j < 4:
            s[j] |= sc[j]
            s[j + 4] |= m[j]
        else:
            s[j + 4] |= (sc[j] & 15) | ((m[j] & 15) << 4)
            s[j - 4] |= (sc[j] >> 4) << 6
            s[j] |= (m[j] >> 4) << 6
    return s


def enc_q8_0(d: np.ndarray, q: np.ndarray) -> bytes:
    """d: (nb,) float16; q: (nb, 32) int8 in [-128, 127]."""
    nb = d.shape[0]
    out = np.zeros((nb, 34), np.uint8)
    out[:, 0:2] = f16_bits(d).reshape(nb, 1).view(np.uint8).reshape(nb, 2)
    out[:, 2:] = q.astype(np.int8).view(np.uint8)
    return out.tobytes()


def val_q8_0(d, q) -> np.ndarray:
    return (d.astype(np.float64)[:, None] * q.astype(np.float64)).astype(np.float32).reshape(-1)


def enc_q4_k(d, dmin, sc, m, q) -> bytes:
    """d, dmin: (nb,) float16; sc, m: (nb, 8) in [0, 63]; q: (nb, 256) in [0, 15]."""
    nb = d.shape[0]
    out = np.zeros((nb, 144), np.uint8)
    out[:, 0:2] = f16_bits(d).reshape(nb, 1).view(np.uint8).reshape(nb, 2)
    out[:, 2:4] = f16_bits(dmin).reshape(nb, 1).view(np.uint8).reshape(nb, 2)
    for b in range(nb):
        out[b, 4:16] = pack_scales_k4(sc[b].astype(np.uint8), m[b].astype(np.uint8))
    q = q.astype(np.uint8)
    for e in range(256):
        byte = 16 + 32 * (e // 64) + e % 32
        out[:, byte] |= q[:, e] if e % 64 < 32 else (q[:, e] << 4)
    return out.tobytes()


def val_q4_k(d, dmin, sc, m, q) -> np.ndarray:
    s = np.arange(256) // 32
    dd = d.astype(np.float64)[:, None]
    mm = dmin.astype(np.float64)[:, None]
    y = dd * sc[:, s].astype(np.float64) * q.astype(np.float64) - mm * m[:, s].astype(np.float64)
    return y.astype(np.float32).reshape(-1)


def enc_q6_k(d, sc, q) -> bytes:
    """d: (nb,) float16; sc: (nb, 16) int8; q: (nb, 256) in [-32, 31]."""
    nb = d.shape[0]
    out = np.zeros((nb, 210), np.uint8)
    u = (q.astype(np.int32) + 32).astype(np.uint8)
    for e in range(256):
        half, quarter, l = e // 128, (e % 128) // 32, e % 32
        qlb = 64 * half + l + 32 * (quarter & 1)
        out[:, qlb] |= (u[:, e] & 15) << (0 if quarter < 2 else 4)
        out[:, 128 + 32 * half + l] |= (u[:, e] >> 4) << (2 * quarter)
    out[:, 192:208] = sc.astype(np.int8).view(np.uint8)
    out[:, 208:210] = f16_bits(d).reshape(nb, 1).view(np.uint8).reshape(nb, 2)
    return out.tobytes()


def val_q6_k(d, sc, q) -> np.ndarray:
    s = np.arange(256) // 16
    y = d.astype(np.float64)[:, None] * sc[:, s].astype(np.float64) * q.astype(np.float64)
    return y.astype(np.float32).reshape(-1)


def random_f16(rng, n, lo_exp=-14, hi_exp=-3, sign=True) -> np.ndarray:
    """Normal float16 values with exponents in [lo_exp, hi_exp]."""
    mant = rng.integers(0, 1024, n)
    e = rng.integers(lo_exp, hi_exp + 1, n)
    v = (1.0 + mant / 1024.0) * np.exp2(e.astype(np.float64))
    if sign:
        v *= rng.choice([-1.0, 1.0], n)
    return v.astype(np.float16)


def random_blocks(rng, ggml_type: int, nb: int, extremes: bool = False):
    """(raw bytes, expected float32 values) for nb random blocks."""
    if ggml_type == 8:
        d = random_f16(rng, nb)
        q = rng.integers(-128, 128, (nb, 32))
        if extremes:
            q[:, 0], q[:, 1] = -128, 127
        return enc_q8_0(d, q), val_q8_0(d, q)
    if ggml_type == 12:
        d = random_f16(rng, nb, sign=False)
        dmin = random_f16(rng, nb, sign=False)
        sc = rng.integers(0, 64, (nb, 8))
        m = rng.integers(0, 64, (nb, 8))
        q = rng.integers(0, 16, (nb, 256))
        if extremes:
            sc[:, 0], m[:, 0], sc[:, 7], m[:, 7] = 63, 63, 63, 0
            q[:, 0], q[:, 255] = 0, 15
        return enc_q4_k(d, dmin, sc, m, q), val_q4_k(d, dmin, sc, m, q)
    if ggml_type == 14:
        d = random_f16(rng, nb)
        sc = rng.integers(-128, 128, (nb, 16))
        q = rng.integers(-32, 32, (nb, 256))
        if extremes:
            sc[:, 0], sc[:, 15] = -128, 127
            q[:, 0], q[:, 255] = -32, 31
        return enc_q6_k(d, sc, q), val_q6_k(d, sc, q)
    raise ValueError(ggml_type)


def random_matrix(rng, ggml_type: int, rows: int, cols: int):
    """A (rows, cols) matrix of random blocks: (raw, float32 values (rows, cols))."""
    nb = rows * cols // QK[ggml_type]
    raw, val = random_blocks(rng, ggml_type, nb)
    return raw, val.reshape(rows, cols)
