"""BASELINE.json configs[3] at its own shapes: the quant GEMV behind
linear_forward_batched (include/brolm/detail/compute.h:54-86), bx_linear_f16
on the device, for every case of the isolated sweep (brolm_amd/sweep.py):
3 formats x 5 weight shapes [N, K] x M in {1, 2, 4, 8, 16} = 75 cases,
against the oracle's linear (FP32 accumulation in the oracle's own order)
on the exactly dequantized weights.

Weights: seeded N(0, 0.02) quantized by the synthetic generator's quantizer
(brolm_synth_quantize), as the sweep makes them; activations FP16 N(0, 1).
Tolerance (tests/test_gpu_kernels.py::_linear_tol): the FP16 output rounding
(2^-10 relative) plus 2^-14 of the absolute dot-product mass for the FP32
accumulation order.  The (151936, 2048) lm_head shape at M 4..16 runs the
matrix-core GEMV over many row tiles per wavefront; the layer shapes run the
split-K form at M >= 3."""
from __future__ import annotations

import numpy as np
import pytest

import oracle
from gpu_util import carrier, release
from test_gpu_kernels import _f16, _linear_tol, _run_linear

pytestmark = pytest.mark.gpu

SHAPES = [(3072, 1024), (1024, 3072), (6144, 2048), (2048, 6144), (151936, 2048)]
FORMATS = {"Q8_0": 8, "Q4_K": 12, "Q6_K": 14}
MS = [1, 2, 4, 8, 16]


@pytest.fixture(scope="module", autouse=True)
def _device():
    import brolm_amd as ba
    ba.init()


def _quantized(fmt: str, N: int, K: int, seed: int):
    from brolm_amd import GGML, _native
    rng = np.random.default_rng(seed)
    w = rng.standard_normal((N, K), dtype=np.float32) * 0.02
    t = FORMATS[fmt]
    be, bb = (32, 34) if t == 8 else (256, 144 if t == 12 else 210)
    raw = np.empty(N * (K // be) * bb, np.uint8)
    _native.check(_native.lib().brolm_synth_quantize(GGML[fmt], w.ctypes.data_as(_native.P_f32), w.size,
                                                     raw.ctypes.data_as(_native.P_u8)), "quantize")
    del w
    Wv = oracle.dequant(t, raw, N * K).reshape(N, K)
    return raw, Wv, rng


@pytest.mark.timeout(300)
@pytest.mark.parametrize("fmt", list(FORMATS))
@pytest.mark.parametrize("N,K", SHAPES)
def test_quant_gemv_sweep_shapes_vs_oracle(fmt, N, K):
    t = FORMATS[fmt]
    raw, Wv, rng = _quantized(fmt, N, K, seed=N * 7 + K + t)
    car = carrier(t, raw, N, K)
    for M in MS:
        print(f"[sweep] {fmt} N={N} K={K} M={M}", flush=True)
        X = _f16(rng.standard_normal((M, K)))
        got = _run_linear(t, car, X, N, K)
        ref = oracle.linear(Wv, X)
        err = np.abs(got.astype(np.float64) - ref)
        tol = _linear_tol(Wv, X, ref)
        worst = float((err / tol).max())
        print(f"[sweep] {fmt} N={N} K={K} M={M}: max err {float(err.max()):.3e}, worst err/tol {worst:.3f}",
              flush=True)
        assert np.all(err <= tol), (fmt, N, K, M, worst)
    release()
