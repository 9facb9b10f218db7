"""Kernel parity on the device, through the C ABI of libbrolm_hip.so, against
the CPU oracle and the independent block encoder.  Integer/byte work is
bit-exact; floating-point results carry the tolerance stated in each test."""
from __future__ import annotations

import ctypes as C

import numpy as np
import pytest

import oracle
import spec_blocks as sb
from gpu_util import call, carrier, dev, empty, f16_dev, f16_host, host, hip, lws, new_workspace, ptr, release, stream, torch

pytestmark = pytest.mark.gpu

QTYPES = [8, 12, 14]


@pytest.fixture(scope="module", autouse=True)
def _device():
    import brolm_amd as ba
    ba.init()
    assert hip().bx_device_ok() == 1


@pytest.fixture(autouse=True)
def _keep_buffers_until_done():
    yield
    release()


def _f16(x: np.ndarray) -> np.ndarray:
    return np.asarray(x, np.float32).astype(np.float16).astype(np.float32)


# ----------------------------------------------------------------- carriers and dequant (bit-exact)

@pytest.mark.parametrize("t", QTYPES)
@pytest.mark.parametrize("rows,cols", [(1, 256), (3, 512), (37, 1024), (5, 6144)])
def test_repack_roundtrip_and_dequant_bit_exact(t, rows, cols):
    print(f"[dequant] type={t} rows={rows} cols={cols}", flush=True)
    rng = np.random.default_rng(rows * cols + t)
    raw, want = sb.random_matrix(rng, t, rows, cols)
    assert hip().bx_carrier_bytes(t, rows, cols) == len(raw)
    car = carrier(t, raw, rows, cols)
    back = empty(len(raw))
    call("bx_unpack_carrier_rows", t, ptr(car), ptr(back), rows, cols, stream())
    assert host(back).tobytes() == raw
    f32 = torch().empty(rows * cols, dtype=torch().float32, device="cuda")
    call("bx_dequant_to_f32", t, ptr(car), ptr(f32), rows, cols, stream())
    assert np.array_equal(host(f32).view(np.uint32), want.reshape(-1).view(np.uint32))
    f16 = torch().empty(rows * cols, dtype=torch().int16, device="cuda")
    call("bx_dequant_to_f16", t, ptr(car), ptr(f16), rows, cols, stream())
    assert np.array_equal(host(f16).view(np.uint16), want.reshape(-1).astype(np.float16).view(np.uint16))


def test_dequant_golden_fixture():
    from golden import load_blocks
    for t, raw, f32_bits, f16_bits in load_blocks():
        cols = sb.QK[t] * 4
        rows = f32_bits.size // cols
        car = carrier(t, raw, rows, cols)
        f32 = torch().empty(f32_bits.size, dtype=torch().float32, device="cuda")
        call("bx_dequant_to_f32", t, ptr(car), ptr(f32), rows, cols, stream())
        assert np.array_equal(host(f32).view(np.uint32), f32_bits)
        f16 = torch().empty(f32_bits.size, dtype=torch().int16, device="cuda")
        call("bx_dequant_to_f16", t, ptr(car), ptr(f16), rows, cols, stream())
        assert np.array_equal(host(f16).view(np.uint16), f16_bits)


# ----------------------------------------------------------------- linear (GEMV M<=16, GEMM above)

def _linear_tol(W: np.ndarray, X: np.ndarray, ref: np.ndarray) -> np.ndarray:
    """FP16 output rounding (2^-11 relative, doubled) plus an FP32
    accumulation allowance of 2^-14 of the absolute dot-product mass.  For
    M > 16 the prefill GEMM feeds the MFMA dequantized weights rounded to FP16
    (relative error <= 2^-11 per product), so its bound adds 2^-11 of the mass."""
    mass = np.abs(X.astype(np.float64)) @ np.abs(W.astype(np.float64)).T
    gemm = 2.0 ** -11 if X.shape[0] > 16 else 0.0
    return 2.0 ** -10 * np.abs(ref) + (2.0 ** -14 + gemm) * mass + 1e-6


def _run_linear(t, Wdev, X, N, K, bias=None):
    M = X.shape[0]
    x = f16_dev(X)
    y = torch().empty(M * N, dtype=torch().int16, device="cuda")
    b = f16_dev(bias) if bias is not None else None
    call("bx_linear_f16", t, ptr(Wdev), ptr(b), ptr(x), ptr(y), M, N, K, *lws(), stream())
    return f16_host(y).reshape(M, N)


@pytest.mark.parametrize("t", QTYPES)
@pytest.mark.parametrize("N,K", [(1, 256), (7, 512), (96, 1024), (300, 2048), (64, 3072), (33, 6144), (40, 8192),
                                 (9, 12288)])
def test_linear_quant_vs_oracle(t, N, K):
    rng = np.random.default_rng(N * 31 + K + t)
    raw, Wv = sb.random_matrix(rng, t, N, K)
    car = carrier(t, raw, N, K)
    for M in (1, 2, 3, 4, 5, 8, 16, 17, 64, 130):
        print(f"[linear] type={t} N={N} K={K} M={M}", flush=True)
        X = _f16(rng.standard_normal((M, K)))
        got = _run_linear(t, car, X, N, K)
        ref = oracle.linear(Wv, X)
        err = np.abs(got - ref)
        tol = _linear_tol(Wv, X, ref)
        assert np.all(err <= tol), (M, float((err / tol).max()))


@pytest.mark.parametrize("t", QTYPES)
@pytest.mark.parametrize("N,K", [(16400, 2048), (5470, 6144)])
def test_linear_several_rows_lm_head_sized(t, N, K):
    """M = 2..4 over matrices of 32 M weights or more (the lm_head's class):
    the several-row kernel (M = 2 in every format, M = 3 and 4 in Q6_K and
    Q8_0) against the oracle within the linear tolerance, and each of its
    output rows bit for bit equal to a one-row launch on that activation row
    (same units per lane, same order, same lane reduction).  Q4_K at M = 3 / 4
    runs the matrix-core kernel and is held to the tolerance only.  N leaves
    a ragged last task; K 6144 keeps the activations in LDS."""
    rng = np.random.default_rng(N + K + t)
    raw, Wv = sb.random_matrix(rng, t, N, K)
    car = carrier(t, raw, N, K)
    for M in (2, 3, 4):
        print(f"[linear rows] type={t} N={N} K={K} M={M}", flush=True)
        X = _f16(rng.standard_normal((M, K)))
        got = _run_linear(t, car, X, N, K)
        ref = oracle.linear(Wv, X)
        tol = _linear_tol(Wv, X, ref)
        assert np.all(np.abs(got - ref) <= tol), (M, float((np.abs(got - ref) / tol).max()))
        if M == 2 or t != 12:
            for m in range(M):
                one = _run_linear(t, car, X[m:m + 1], N, K)
                assert np.array_equal(got[m].view(np.uint32), one[0].view(np.uint32)), (M, m)


@pytest.mark.parametrize("t", QTYPES + [1])
@pytest.mark.parametrize("N,K", [(128, 256), (300, 1024), (1024, 512), (4100, 256)])
def test_linear_big_tiles_vs_oracle(t, N, K):
    """The 256x128 / 128x128 MFMA tiles (M >= 128, K a multiple of 64):
    partial tiles in M and N, a grid above and below the CU count (both tile
    shapes), bias."""
    rng = np.random.default_rng(N * 7 + K + t)
    if t == 1:
        Wv = _f16(rng.standard_normal((N, K)) * 0.05)
        car = f16_dev(Wv)
    else:
        raw, Wv = sb.random_matrix(rng, t, N, K)
        car = carrier(t, raw, N, K)
    bias = _f16(rng.standard_normal(N))
    for M in (128, 129, 255, 256, 600):
        print(f"[linear tiles] type={t} N={N} K={K} M={M}", flush=True)
        X = _f16(rng.standard_normal((M, K)))
        got = _run_linear(t, car, X, N, K, bias)
        ref = oracle.linear(Wv, X) + bias
        tol = _linear_tol(Wv, X, ref)
        assert np.all(np.abs(got - ref) <= tol), (M, float((np.abs(got - ref) / tol).max()))


def _weights(rng, t, N, K):
    if t == 1:
        Wv = _f16(rng.standard_normal((N, K)) * 0.05)
        return f16_dev(Wv), Wv
    raw, Wv = sb.random_matrix(rng, t, N, K)
    return carrier(t, raw, N, K), Wv


@pytest.mark.parametrize("M,K,Ns", [(300, 512, (384, 128, 128)), (5, 512, (384, 136, 136)),
                                    (16, 512, (256, 120, 120)), (16, 6144, (64, 48, 48))])
@pytest.mark.parametrize("t", QTYPES + [1])
def test_fused_prefill_linears_equal_unfused_ops(t, M, K, Ns):
    """bx_linear_group / _residual / _swiglu give bit-identical results to the
    separate linear, add_inplace, silu and mul launches they replace (same
    MFMA arithmetic, same FP16 roundings): the tile GEMM at M >= 128, the MFMA
    GEMV of decode batches at 3 <= M <= 16 (partial row tiles; K = 6144 in two
    row chunks of staged activations); other M decline."""
    print(f"[fused] t={t} M={M} K={K} N={Ns}", flush=True)
    rng = np.random.default_rng(900 + t + M)
    ws = [_weights(rng, t, n, K)[0] for n in Ns]
    X = _f16(rng.standard_normal((M, K)))
    x = f16_dev(X)
    h = hip()
    # q / k / v group vs three linears
    ys = [torch().empty(M * n, dtype=torch().int16, device="cuda") for n in Ns]
    W_arr = (C.c_void_p * 3)(*[ptr(w) for w in ws])
    Y_arr = (C.c_void_p * 3)(*[ptr(y) for y in ys])
    N_arr = (C.c_int * 3)(*Ns)
    call("bx_linear_group_f16", t, 3, W_arr, Y_arr, N_arr, ptr(x), M, K, *lws(), stream())
    for w, y, n in zip(ws, ys, Ns):
        ref = torch().empty(M * n, dtype=torch().int16, device="cuda")
        call("bx_linear_f16", t, ptr(w), None, ptr(x), ptr(ref), M, n, K, *lws(), stream())
        assert np.array_equal(host(y), host(ref))
    # residual: H (FP32) += f16(X W^T)
    H0 = rng.standard_normal((M, Ns[0])).astype(np.float32)
    Hf = dev(H0)
    call("bx_linear_residual_f16", t, ptr(ws[0]), ptr(x), ptr(Hf), M, Ns[0], K, *lws(), stream())
    Hr = dev(H0)
    proj = torch().empty(M * Ns[0], dtype=torch().int16, device="cuda")
    call("bx_linear_f16", t, ptr(ws[0]), None, ptr(x), ptr(proj), M, Ns[0], K, *lws(), stream())
    call("bx_add_inplace", ptr(Hr), 1, ptr(proj), M * Ns[0], stream())
    assert np.array_equal(host(Hf).view(np.uint32), host(Hr).view(np.uint32))
    # SwiGLU: gate = ws[1], up = ws[2] (same shape)
    act = torch().empty(M * Ns[1], dtype=torch().int16, device="cuda")
    call("bx_linear_swiglu_f16", t, ptr(ws[1]), ptr(ws[2]), ptr(x), ptr(act), M, Ns[1], K, *lws(), stream())
    g = torch().empty(M * Ns[1], dtype=torch().int16, device="cuda")
    u = torch().empty(M * Ns[1], dtype=torch().int16, device="cuda")
    call("bx_linear_f16", t, ptr(ws[1]), None, ptr(x), ptr(g), M, Ns[1], K, *lws(), stream())
    call("bx_linear_f16", t, ptr(ws[2]), None, ptr(x), ptr(u), M, Ns[1], K, *lws(), stream())
    call("bx_silu_f16", ptr(g), ptr(g), M * Ns[1], stream())
    call("bx_mul_f16", ptr(g), ptr(u), M * Ns[1], stream())
    assert np.array_equal(host(act), host(g))
    # between the two paths: declined, nothing written
    assert h.bx_linear_tiles_ok(100, K) == 0 and h.bx_linear_tiles_ok(2, K) == 0 and h.bx_linear_tiles_ok(M, K) == 1
    assert h.bx_linear_residual_f16(t, ptr(ws[0]), ptr(x), ptr(Hf), 100, Ns[0], K, *lws(), stream()) == -3  # BX_EUNSUPPORTED


@pytest.mark.parametrize("t", QTYPES)
def test_linear_split_k_two_streams_own_workspaces(t):
    """16-row split-K linears on two streams at once, each stream with its own
    workspace: every launch matches the oracle, and each stream's result has
    the bits of the same launch run alone (the slice order is fixed).  A
    workspace whose counters hold a stale word of an unfinished launch (tag
    and partial count written from the host) still gives the same bits.  No
    workspace: the plain launch, still within the oracle's tolerance; the
    split-only forms return BX_EINVAL with nothing written."""
    print(f"[linear two streams] t={t}", flush=True)
    T = torch()
    h = hip()
    rng = np.random.default_rng(5150 + t)
    N, K, M, reps = 2048, 2048, 16, 6
    raw, Wv = sb.random_matrix(rng, t, N, K)
    car = carrier(t, raw, N, K)
    Xs = [_f16(rng.standard_normal((M, K))) for _ in range(2)]
    xs = [f16_dev(X) for X in Xs]
    alone = []
    for x in xs:
        y = T.empty(M * N, dtype=T.int16, device="cuda")
        call("bx_linear_f16", t, ptr(car), None, ptr(x), ptr(y), M, N, K, *lws(), stream())
        alone.append(host(y))
    wss = [new_workspace() for _ in range(2)]
    T.cuda.synchronize()
    streams = [T.cuda.Stream(), T.cuda.Stream()]
    outs = [[T.empty(M * N, dtype=T.int16, device="cuda") for _ in range(reps)] for _ in range(2)]
    for i in range(reps):
        for s in range(2):
            call("bx_linear_f16", t, ptr(car), None, ptr(xs[s]), ptr(outs[s][i]), M, N, K,
                 C.c_void_p(wss[s][0].data_ptr()), C.c_size_t(wss[s][1]), C.c_void_p(streams[s].cuda_stream))
    T.cuda.synchronize()
    for s in range(2):
        ref = oracle.linear(Wv, Xs[s])
        tol = _linear_tol(Wv, Xs[s], ref)
        for i in range(reps):
            got = host(outs[s][i])
            assert np.array_equal(got, alone[s]), (s, i)
            assert np.all(np.abs(got.view(np.float16).astype(np.float32).reshape(M, N) - ref) <= tol), (s, i)
    # a stale counter word: tag 0xdeadbeef with 3 arrivals, in every group
    buf, n = wss[0]
    stale = np.zeros(4096, np.uint64) | np.uint64((0xdeadbeef << 32) | 3)
    buf[: stale.nbytes].copy_(T.from_numpy(stale.view(np.uint8)).to("cuda"))
    y = T.empty(M * N, dtype=T.int16, device="cuda")
    call("bx_linear_f16", t, ptr(car), None, ptr(xs[0]), ptr(y), M, N, K, C.c_void_p(buf.data_ptr()), C.c_size_t(n),
         stream())
    assert np.array_equal(host(y), alone[0])
    # no workspace: the single-pass launch
    y = T.empty(M * N, dtype=T.int16, device="cuda")
    call("bx_linear_f16", t, ptr(car), None, ptr(xs[0]), ptr(y), M, N, K, None, C.c_size_t(0), stream())
    ref = oracle.linear(Wv, Xs[0])
    assert np.all(np.abs(f16_host(y).reshape(M, N) - ref) <= _linear_tol(Wv, Xs[0], ref))
    H = dev(np.zeros((M, N), np.float32))
    ss = T.zeros(h.bx_linear_ss_floats(N), dtype=T.float32, device="cuda")
    Wo = carrier(t, sb.random_matrix(rng, t, N, K)[0], N, K)
    assert h.bx_linear_residual_ss_f16(t, ptr(Wo), ptr(xs[0]), ptr(H), ptr(ss), M, N, K, None, C.c_size_t(0),
                                       stream()) == -1   # BX_EINVAL
    assert not np.any(host(H))


@pytest.mark.parametrize("t", QTYPES)
def test_linear_ffn_width_k(t):
    """K = 32768 (Mistral-Small-3.1's FFN width, the down projection) and
    24576: the one-row GEMV with K split over the workgroup's four wavefronts
    (odd row counts end a chunk on the repeated-row request), and the GEMM for
    2..16 rows; K 17408, between the split widths, takes the one-wavefront-
    per-row kernel (16 units per lane, 80 KB of staged activations)."""
    rng = np.random.default_rng(4242 + t)
    for N, K in ((320, 32768), (331, 24576), (130, 17408)):
        raw, Wv = sb.random_matrix(rng, t, N, K)
        car = carrier(t, raw, N, K)
        for M in (1, 2, 5, 17):
            print(f"[linear wide K] type={t} N={N} K={K} M={M}", flush=True)
            # activations scaled so the 32768-term sums stay well inside FP16
            X = _f16(rng.standard_normal((M, K)) * 0.05)
            got = _run_linear(t, car, X, N, K)
            ref = oracle.linear(Wv, X)
            tol = _linear_tol(Wv, X, ref)
            assert np.all(np.abs(got - ref) <= tol), (M, K)


@pytest.mark.parametrize("t", QTYPES + [1])
@pytest.mark.parametrize("N,K", [(1000, 6144), (4100, 2048), (77, 12288), (40, 768), (96, 14336), (40, 32768)])
def test_linear_split_k_repeats_bitwise(t, N, K):
    """Batched GEMV of decoder-layer size: K split over workgroups, partial
    tiles added by the last workgroup of each tile group.  Row tiles not a
    multiple of the group, slices of one to three chunks (K 768 .. 32768, up to
    43 slices),
    bias; three launches in a row give the same bits (the per-group counters
    are back at zero after every launch) and match the oracle."""
    rng = np.random.default_rng(5150 + N + t)
    if t == 1:
        Wv = _f16(rng.standard_normal((N, K)) * 0.05)
        car = f16_dev(Wv)
    else:
        raw, Wv = sb.random_matrix(rng, t, N, K)
        car = carrier(t, raw, N, K)
    bias = _f16(rng.standard_normal(N))
    for M in (3, 8, 13, 16):
        print(f"[linear split] type={t} N={N} K={K} M={M}", flush=True)
        X = _f16(rng.standard_normal((M, K)) * (0.05 if K > 12288 else 0.25 if K > 4096 else 1.0))
        outs = [_run_linear(t, car, X, N, K, bias) for _ in range(3)]
        assert all(np.array_equal(o, outs[0]) for o in outs[1:]), M
        ref = oracle.linear(Wv, X) + bias
        tol = _linear_tol(Wv, X, ref) + 2.0 ** -10 * np.abs(bias)
        assert np.all(np.abs(outs[0] - ref) <= tol), (M, float((np.abs(outs[0] - ref) / tol).max()))


@pytest.mark.parametrize("t", QTYPES + [1])
def test_linear_batched_many_tiles(t):
    """Batched GEMV with more 16-row tiles than the workgroups hold at once
    (each wavefront walks several tiles) and a last tile of one row."""
    rng = np.random.default_rng(77 + t)
    N, K = 70001, 256
    if t == 1:
        Wv = _f16(rng.standard_normal((N, K)) * 0.05)
        car = f16_dev(Wv)
    else:
        raw, Wv = sb.random_matrix(rng, t, N, K)
        car = carrier(t, raw, N, K)
    bias = _f16(rng.standard_normal(N))
    for M in (3, 5, 8, 16):
        print(f"[linear many tiles] type={t} N={N} K={K} M={M}", flush=True)
        X = _f16(rng.standard_normal((M, K)))
        got = _run_linear(t, car, X, N, K, bias)
        ref = oracle.linear(Wv, X) + bias
        tol = _linear_tol(Wv, X, ref) + 2.0 ** -10 * np.abs(bias)
        assert np.all(np.abs(got - ref) <= tol), M


@pytest.mark.parametrize("t", [1, 12])
def test_linear_bias_and_dense_f16(t):
    rng = np.random.default_rng(5)
    N, K = 200, 1024
    if t == 1:
        Wv = _f16(rng.standard_normal((N, K)) * 0.05)
        Wdev = f16_dev(Wv)
    else:
        raw, Wv = sb.random_matrix(rng, t, N, K)
        Wdev = carrier(t, raw, N, K)
    bias = _f16(rng.standard_normal(N))
    for M in (1, 4, 33):
        X = _f16(rng.standard_normal((M, K)))
        got = _run_linear(t, Wdev, X, N, K, bias)
        ref = oracle.linear(Wv, X) + bias
        assert np.all(np.abs(got - ref) <= _linear_tol(Wv, X, ref) + 2.0 ** -10 * np.abs(bias)), M


def test_linear_onehot_selects_dequantized_column():
    """X = e_k makes Y the k-th dequantized column, rounded once to FP16."""
    rng = np.random.default_rng(9)
    for t in QTYPES:
        N, K = 64, 512
        raw, Wv = sb.random_matrix(rng, t, N, K)
        car = carrier(t, raw, N, K)
        for k in (0, 31, 32, 255, 256, 511):
            X = np.zeros((1, K), np.float32)
            X[0, k] = 1.0
            got = _run_linear(t, car, X, N, K)
            assert np.array_equal(got[0], _f16(Wv[:, k])), (t, k)


# ----------------------------------------------------------------- norms, rope, kv

@pytest.mark.parametrize("x_is_f32", [0, 1])
def test_rms_norm(x_is_f32):
    rng = np.random.default_rng(11)
    rows, cols = 9, 2048
    x = rng.standard_normal((rows, cols)).astype(np.float32) * 2
    if not x_is_f32:
        x = _f16(x)
    g = _f16(rng.uniform(0.5, 1.5, cols))
    xd = dev(x) if x_is_f32 else f16_dev(x)
    y = torch().empty(rows * cols, dtype=torch().int16, device="cuda")
    call("bx_rms_norm", ptr(xd), x_is_f32, ptr(f16_dev(g)), C.c_float(1e-6), ptr(y), rows, cols, stream())
    ref = oracle.rms_norm(x, g, 1e-6)
    np.testing.assert_allclose(f16_host(y).reshape(rows, cols), ref, atol=2e-3 * np.abs(ref).max(), rtol=2 ** -10)


@pytest.mark.parametrize("hd,pos0", [(64, 0), (128, 1023), (128, 40000)])
def test_rope(hd, pos0):
    rng = np.random.default_rng(hd + pos0)
    n_heads, L, theta = 4, 3, 1e6
    cap = pos0 + L + 5
    cos = np.empty((cap, hd // 2), np.float32)
    sin = np.empty((cap, hd // 2), np.float32)
    hip().bx_rope_table_host(cos.ctypes.data_as(C.POINTER(C.c_float)), sin.ctypes.data_as(C.POINTER(C.c_float)),
                             cap, hd, C.c_float(theta))
    x = _f16(rng.standard_normal((L, n_heads * hd)))
    xd = f16_dev(x)
    call("bx_rope_f16", ptr(xd), ptr(xd), L, hd, n_heads, pos0, ptr(dev(cos)), ptr(dev(sin)), cap, stream())
    ref = oracle.rope(x, hd, n_heads, pos0, theta)
    np.testing.assert_allclose(f16_host(xd).reshape(L, -1), ref, atol=4e-3)


def test_kv_append_and_scatter_row():
    rng = np.random.default_rng(12)
    cap, cols, L, cur = 16, 256, 3, 5
    Kc = torch().zeros(cap * cols, dtype=torch().int16, device="cuda")
    Vc = torch().zeros(cap * cols, dtype=torch().int16, device="cuda")
    k = rng.integers(0, 1 << 15, (L, cols)).astype(np.uint16)
    v = rng.integers(0, 1 << 15, (L, cols)).astype(np.uint16)
    call("bx_kv_append_f16", ptr(dev(k)), ptr(dev(v)), L, cols, cur, ptr(Kc), ptr(Vc), cap, stream())
    kh, vh = host(Kc).view(np.uint16).reshape(cap, cols), host(Vc).view(np.uint16).reshape(cap, cols)
    assert np.array_equal(kh[cur:cur + L], k) and np.array_equal(vh[cur:cur + L], v)
    assert not kh[:cur].any() and not kh[cur + L:].any()
    row = rng.integers(0, 1 << 15, cols).astype(np.uint16)
    idx = dev(np.array([11], np.int32))
    call("bx_scatter_row", ptr(dev(row)), ptr(idx), ptr(Kc), cols * 2, cap, stream())
    assert np.array_equal(host(Kc).view(np.uint16).reshape(cap, cols)[11], row)


# ----------------------------------------------------------------- attention

def _attn_ref(q, K, V, L, valid, n_q, n_kv, hd, softcap=0.0, window=0, mask=None):
    """float64 softmax attention with GQA map h -> h // (n_q / n_kv)."""
    out = np.zeros((L, n_q * hd))
    G = n_q // n_kv
    for r in range(L):
        p = valid - L + r
        lo = max(0, p - window + 1) if window > 0 else 0
        keys = np.arange(lo, p + 1)
        if mask is not None:
            keys = np.nonzero(mask[:valid])[0]
        for h in range(n_q):
            g = h // G
            s = K[keys, g * hd:(g + 1) * hd].astype(np.float64) @ q[r, h * hd:(h + 1) * hd].astype(np.float64)
            s /= np.sqrt(hd)
            if softcap > 0:
                s = softcap * np.tanh(s / softcap)
            w = np.exp(s - s.max())
            out[r, h * hd:(h + 1) * hd] = (w / w.sum()) @ V[keys, g * hd:(g + 1) * hd].astype(np.float64)
    return out


@pytest.mark.parametrize("L,valid,n_q,n_kv,hd", [
    (1, 1, 4, 2, 64), (1, 5, 16, 8, 128), (1, 64, 16, 8, 128), (1, 65, 16, 8, 128), (1, 300, 8, 8, 64),
    (1, 2049, 16, 8, 128), (1, 4096, 32, 8, 128), (4, 70, 4, 2, 64), (16, 600, 16, 8, 128),
    # split-K head dims other than 64 / 128 (a partial last chunk per lane
    # quad, two dims pairs per lane) and a GQA group of 8
    (1, 300, 8, 2, 96), (2, 130, 8, 8, 256), (1, 77, 4, 1, 72), (3, 1000, 32, 4, 128), (1, 20000, 16, 8, 128),
    # L >= 16 rows: the MFMA flash-attention kernel (partial query and key
    # tiles, GQA groups 1..4, prompt-only and after a cached prefix)
    (17, 17, 4, 2, 64), (64, 64, 16, 8, 128), (65, 200, 32, 8, 128), (130, 130, 8, 8, 64),
    (300, 1000, 8, 2, 128)])
def test_attention_decode(L, valid, n_q, n_kv, hd):
    print(f"[attention] L={L} valid={valid} n_q={n_q} n_kv={n_kv} hd={hd}", flush=True)
    rng = np.random.default_rng(valid + 7 * L)
    cap = valid + 3
    q = _f16(rng.standard_normal((L, n_q * hd)))
    K = _f16(rng.standard_normal((cap, n_kv * hd)))
    V = _f16(rng.standard_normal((cap, n_kv * hd)))
    ws = empty(max(1, hip().bx_attention_workspace_bytes(L, n_q, hd, valid)))
    out = torch().empty(L * n_q * hd, dtype=torch().int16, device="cuda")
    call("bx_attention_decode_f16", ptr(f16_dev(q)), ptr(f16_dev(K)), ptr(f16_dev(V)), L, valid, n_q, n_kv, hd,
         C.c_float(0.0), 0, ptr(out), ptr(ws), stream())
    ref = _attn_ref(q, K, V, L, valid, n_q, n_kv, hd)
    np.testing.assert_allclose(f16_host(out).reshape(L, -1), ref, atol=3e-3)


@pytest.mark.parametrize("L,n_keys,causal,hd", [(16, 16, 0, 128), (100, 100, 0, 64), (77, 77, 1, 128),
                                                 (40, 90, 1, 128), (200, 200, 0, 128)])
def test_attention_gqa_encode(L, n_keys, causal, hd):
    """flash_attention_gqa_forward (dense_decoder.cpp:737-745): bidirectional
    rows see every key, causal rows the keys up to their position."""
    print(f"[attention gqa] L={L} keys={n_keys} causal={causal} hd={hd}", flush=True)
    rng = np.random.default_rng(L * 3 + n_keys + causal)
    n_q, n_kv = 8, 4
    q = _f16(rng.standard_normal((L, n_q * hd)))
    K = _f16(rng.standard_normal((n_keys, n_kv * hd)))
    V = _f16(rng.standard_normal((n_keys, n_kv * hd)))
    ws = empty(max(1, hip().bx_attention_workspace_bytes(L, n_q, hd, n_keys)))
    out = torch().empty(L * n_q * hd, dtype=torch().int16, device="cuda")
    call("bx_attention_gqa_f16", ptr(f16_dev(q)), ptr(f16_dev(K)), ptr(f16_dev(V)), L, n_keys, n_q, n_kv, hd, causal,
         ptr(out), ptr(ws), stream())
    if causal:
        ref = _attn_ref(q, K, V, L, n_keys, n_q, n_kv, hd)
    else:
        ref = np.concatenate([_attn_ref(q[r:r + 1], K, V, 1, n_keys, n_q, n_kv, hd) for r in range(L)])
    np.testing.assert_allclose(f16_host(out).reshape(L, -1), ref, atol=3e-3)


def test_attention_softcap_window_and_mask():
    rng = np.random.default_rng(3)
    L, valid, n_q, n_kv, hd = 2, 200, 8, 4, 128
    q = _f16(rng.standard_normal((L, n_q * hd)) * 3)
    K = _f16(rng.standard_normal((valid, n_kv * hd)))
    V = _f16(rng.standard_normal((valid, n_kv * hd)))
    ws = empty(hip().bx_attention_workspace_bytes(L, n_q, hd, valid))
    out = torch().empty(L * n_q * hd, dtype=torch().int16, device="cuda")
    call("bx_attention_decode_f16", ptr(f16_dev(q)), ptr(f16_dev(K)), ptr(f16_dev(V)), L, valid, n_q, n_kv, hd,
         C.c_float(5.0), 37, ptr(out), ptr(ws), stream())
    ref = _attn_ref(q, K, V, L, valid, n_q, n_kv, hd, softcap=5.0, window=37)
    np.testing.assert_allclose(f16_host(out).reshape(L, -1), ref, atol=3e-3)
    mask = (rng.random(valid) < 0.3).astype(np.float32)
    mask[0] = 1
    ws1 = empty(hip().bx_attention_workspace_bytes(1, n_q, hd, valid))
    out1 = torch().empty(n_q * hd, dtype=torch().int16, device="cuda")
    call("bx_attention_masked_f16", ptr(f16_dev(q[:1])), ptr(f16_dev(K)), ptr(f16_dev(V)), ptr(dev(mask)), valid,
         n_q, n_kv, hd, ptr(out1), ptr(ws1), stream())
    ref1 = _attn_ref(q[:1], K, V, 1, valid, n_q, n_kv, hd, mask=mask)
    np.testing.assert_allclose(f16_host(out1).reshape(1, -1), ref1, atol=3e-3)


# ----------------------------------------------------------------- elementwise, embedding, argmax

def test_elementwise_ops():
    rng = np.random.default_rng(13)
    n = 6144 * 3 + 5
    g = _f16(rng.standard_normal(n) * 4)
    u = _f16(rng.standard_normal(n))
    gd, ud = f16_dev(g), f16_dev(u)
    call("bx_silu_mul_f16", ptr(gd), ptr(ud), n, stream())
    gg = g.astype(np.float64)
    np.testing.assert_allclose(f16_host(gd), gg / (1 + np.exp(-gg)) * u, rtol=2 ** -9, atol=1e-4)
    y = torch().empty(n, dtype=torch().int16, device="cuda")
    call("bx_silu_f16", ptr(f16_dev(g)), ptr(y), n, stream())
    np.testing.assert_allclose(f16_host(y), gg / (1 + np.exp(-gg)), rtol=2 ** -9, atol=1e-4)
    a = f16_dev(g)
    call("bx_mul_f16", ptr(a), ptr(ud), n, stream())
    assert np.array_equal(f16_host(a), _f16(g.astype(np.float32) * u))
    h = rng.standard_normal(n).astype(np.float32)
    hd_ = dev(h)
    call("bx_add_inplace", ptr(hd_), 1, ptr(ud), n, stream())
    assert np.array_equal(host(hd_), h + u)
    x = (rng.standard_normal(n) * np.exp2(rng.uniform(-26, 17, n))).astype(np.float32)
    y = torch().empty(n, dtype=torch().int16, device="cuda")
    call("bx_f32_to_f16", ptr(dev(x)), ptr(y), n, stream())
    with np.errstate(over="ignore"):
        assert np.array_equal(host(y).view(np.uint16), x.astype(np.float16).view(np.uint16))


def test_embedding_gather_is_exact():
    rng = np.random.default_rng(14)
    V, H = 1000, 512
    W = rng.integers(0, 0x7C00, (V, H)).astype(np.uint16)  # every finite non-negative binary16
    W[1::2] |= 0x8000
    ids = np.array([0, 999, 5, 5, 123], np.int32)
    out = torch().empty(len(ids) * H, dtype=torch().int16, device="cuda")
    Wd = dev(W)
    call("bx_embedding_f16", ptr(Wd), V, H, ptr(dev(ids)), len(ids), ptr(out), stream())
    assert np.array_equal(host(out).view(np.uint16).reshape(-1, H), W[ids])
    out32 = torch().empty(len(ids) * H, dtype=torch().float32, device="cuda")
    call("bx_embedding_f32", ptr(Wd), V, H, ptr(dev(ids)), len(ids), ptr(out32), stream())
    assert np.array_equal(host(out32).reshape(-1, H), W[ids].view(np.float16).astype(np.float32))


@pytest.mark.parametrize("n", [1, 63, 1000, 151936, 262144 + 17])
def test_argmax_lowest_index_wins(n):
    rng = np.random.default_rng(n)
    x = _f16(rng.standard_normal(n))
    top = x.max()
    # plant ties of the maximum at several indices
    idx = np.sort(rng.choice(n, size=min(n, 5), replace=False))
    x[idx] = top + 1
    ws = empty(hip().bx_argmax_workspace_bytes(n))
    out = torch().empty(1, dtype=torch().int32, device="cuda")
    call("bx_argmax_f16", ptr(f16_dev(x)), n, ptr(out), ptr(ws), stream())
    assert int(host(out)[0]) == oracle.argmax(x)[0] == idx[0]


# ----------------------------------------------------------------- error paths (host-side checks)

def test_linear_rejects_bad_shapes_and_types():
    x = torch().zeros(256, dtype=torch().int16, device="cuda")
    y = torch().zeros(256, dtype=torch().int16, device="cuda")
    h = hip()
    assert h.bx_linear_f16(12, ptr(x), None, ptr(x), ptr(y), 1, 1, 100, *lws(), stream()) == -1   # K not a block multiple
    assert h.bx_linear_f16(2, ptr(x), None, ptr(x), ptr(y), 1, 1, 256, *lws(), stream()) == -3    # unsupported type
    assert h.bx_linear_f16(12, None, None, ptr(x), ptr(y), 1, 1, 256, *lws(), stream()) == -1     # null weight
    assert b"linear" in h.bx_last_error()


@pytest.mark.parametrize("t", [12, 14, 8])
@pytest.mark.parametrize("M", [3, 8, 16])
def test_linear_norm_carried_between_launches(t, M):
    """Decode-batch forms with the residual RMSNorm carried between launches:
    bx_linear_residual_ss_f16 updates H exactly as bx_linear_residual_f16 and
    writes partial row sums of squares adding up to each row's sum (rel 1e-5);
    bx_linear_group_norm_f16 / bx_linear_swiglu_norm_f16 on H match
    bx_rms_norm + the plain forms up to the FP16 rounding of the normalised
    input (their sum of squares is added in another order); outside the split
    GEMV (M = 2, or N beyond 32768 rows) they refuse with BX_EUNSUPPORTED and
    write nothing."""
    print(f"[linear norm] type={t} M={M}", flush=True)
    rng = np.random.default_rng(700 + t + M)
    K, Ka, F = 2048, 1024, 768
    Ns = (512, 256, 256)
    Wo, Wov = _weights(rng, t, K, Ka)
    ws = [_weights(rng, t, n, K) for n in Ns]
    wg, wu = _weights(rng, t, F, K), _weights(rng, t, F, K)
    gamma = _f16(rng.uniform(0.5, 1.5, K))
    gd = f16_dev(gamma)
    X = _f16(rng.standard_normal((M, Ka)))
    H0 = (rng.standard_normal((M, K)) * 2).astype(np.float32)
    h = hip()
    nss = h.bx_linear_ss_floats(K)
    ss = torch().zeros(nss, dtype=torch().float32, device="cuda")
    # residual with row sums vs the plain residual
    Hs, Hp = dev(H0), dev(H0)
    call("bx_linear_residual_ss_f16", t, ptr(Wo), ptr(f16_dev(X)), ptr(Hs), ptr(ss), M, K, Ka, *lws(), stream())
    call("bx_linear_residual_f16", t, ptr(Wo), ptr(f16_dev(X)), ptr(Hp), M, K, Ka, *lws(), stream())
    Hn = host(Hs).reshape(M, K)
    assert np.array_equal(Hn.view(np.uint32), host(Hp).reshape(M, K).view(np.uint32))
    rows = host(ss).reshape(-1, 16)[:, :M].sum(axis=0, dtype=np.float64)
    np.testing.assert_allclose(rows, (Hn.astype(np.float64) ** 2).sum(axis=1), rtol=1e-5)
    # separate norm -> FP16 X for the plain forms
    xn = torch().empty(M * K, dtype=torch().int16, device="cuda")
    call("bx_rms_norm", ptr(Hs), 1, ptr(gd), C.c_float(1e-6), ptr(xn), M, K, stream())
    Xn = f16_host(xn).reshape(M, K)
    ys = [torch().empty(M * n, dtype=torch().int16, device="cuda") for n in Ns]
    yr = [torch().empty(M * n, dtype=torch().int16, device="cuda") for n in Ns]
    W_arr = (C.c_void_p * 3)(*[ptr(w[0]) for w in ws])
    N_arr = (C.c_int * 3)(*Ns)
    call("bx_linear_group_norm_f16", t, 3, W_arr, (C.c_void_p * 3)(*[ptr(y) for y in ys]), N_arr, ptr(Hs), ptr(gd),
         C.c_float(1e-6), ptr(ss), M, K, *lws(), stream())
    call("bx_linear_group_f16", t, 3, W_arr, (C.c_void_p * 3)(*[ptr(y) for y in yr]), N_arr, ptr(xn), M, K, *lws(), stream())
    for (w, Wv), n, y, r in zip(ws, Ns, ys, yr):
        got, ref = f16_host(y).reshape(M, n), f16_host(r).reshape(M, n)
        # one FP16 ulp of the normalised input per element, on top of the output rounding
        tol = 2.0 ** -10 * np.abs(ref) + 2.0 ** -10 * (np.abs(Xn) @ np.abs(Wv).T) + 1e-6
        assert np.all(np.abs(got - ref) <= tol), (n, float((np.abs(got - ref) / tol).max()))
    act = torch().empty(M * F, dtype=torch().int16, device="cuda")
    act_r = torch().empty(M * F, dtype=torch().int16, device="cuda")
    call("bx_linear_swiglu_norm_f16", t, ptr(wg[0]), ptr(wu[0]), ptr(Hs), ptr(gd), C.c_float(1e-6), ptr(ss), ptr(act),
         M, F, K, *lws(), stream())
    call("bx_linear_swiglu_f16", t, ptr(wg[0]), ptr(wu[0]), ptr(xn), ptr(act_r), M, F, K, *lws(), stream())
    got, ref = f16_host(act).reshape(M, F), f16_host(act_r).reshape(M, F)
    scale = (np.abs(Xn) @ np.abs(wg[1]).T) * (np.abs(Xn) @ np.abs(wu[1]).T)
    fin = np.isfinite(ref)   # products beyond FP16 overflow the same way in both
    assert np.array_equal(np.isfinite(got), fin)
    assert np.all((np.abs(got[fin] - ref[fin]) <= (2.0 ** -9 * np.abs(ref) + 2.0 ** -9 * scale + 1e-5)[fin]))
    # refused, nothing written
    sentinel = torch().full((M * Ns[0],), 0x1234, dtype=torch().int16, device="cuda")
    rc = h.bx_linear_group_norm_f16(t, 1, W_arr, (C.c_void_p * 3)(ptr(sentinel), None, None), N_arr, ptr(Hs), ptr(gd),
                                    C.c_float(1e-6), ptr(ss), 2, K, *lws(), stream())
    assert rc == -3 and np.all(host(sentinel) == 0x1234)


@pytest.mark.parametrize("M", [3, 4, 9, 16])
def test_linear_group_two_formats_equals_own_launches(M):
    """bx_linear_group2_f16 / _norm_f16: q and k (Q4_K) with v (Q6_K) in one
    launch give each member exactly the bits of its own group launch (the K
    split depends on K alone), from FP16 X and from RMSNorm(H) with carried
    row sums; other type pairs are refused with nothing launched."""
    print(f"[linear group2] M={M}", flush=True)
    rng = np.random.default_rng(4400 + M)
    K, Ns = 2048, (512, 256, 256)
    ws = [_weights(rng, 12, Ns[0], K)[0], _weights(rng, 12, Ns[1], K)[0], _weights(rng, 14, Ns[2], K)[0]]
    X = _f16(rng.standard_normal((M, K)))
    x = f16_dev(X)
    W_arr = (C.c_void_p * 3)(*[ptr(w) for w in ws])
    N_arr = (C.c_int * 3)(*Ns)

    def outs():
        return [torch().empty(M * n, dtype=torch().int16, device="cuda") for n in Ns]

    def arr(ys):
        return (C.c_void_p * 3)(*[ptr(y) for y in ys])

    ya, yb = outs(), outs()
    call("bx_linear_group2_f16", 12, 14, 3, 2, W_arr, arr(ya), N_arr, ptr(x), M, K, *lws(), stream())
    call("bx_linear_group_f16", 12, 2, W_arr, arr(yb), N_arr, ptr(x), M, K, *lws(), stream())
    call("bx_linear_group_f16", 14, 1, (C.c_void_p * 3)(ptr(ws[2]), None, None), (C.c_void_p * 3)(ptr(yb[2]), None, None),
         (C.c_int * 3)(Ns[2], 0, 0), ptr(x), M, K, *lws(), stream())
    for a, b in zip(ya, yb):
        assert np.array_equal(host(a), host(b))
    # from RMSNorm(H), the row sums from a residual launch
    Wo, _ = _weights(rng, 12, K, 512)
    H = dev((rng.standard_normal((M, K)) * 2).astype(np.float32))
    h = hip()
    ss = torch().zeros(h.bx_linear_ss_floats(K), dtype=torch().float32, device="cuda")
    call("bx_linear_residual_ss_f16", 12, ptr(Wo), ptr(f16_dev(rng.standard_normal((M, 512)))), ptr(H), ptr(ss), M, K,
         512, *lws(), stream())
    gd = f16_dev(rng.uniform(0.5, 1.5, K))
    ya, yb = outs(), outs()
    call("bx_linear_group2_norm_f16", 12, 14, 3, 2, W_arr, arr(ya), N_arr, ptr(H), ptr(gd), C.c_float(1e-6), ptr(ss),
         M, K, *lws(), stream())
    call("bx_linear_group_norm_f16", 12, 2, W_arr, arr(yb), N_arr, ptr(H), ptr(gd), C.c_float(1e-6), ptr(ss), M, K,
         *lws(), stream())
    call("bx_linear_group_norm_f16", 14, 1, (C.c_void_p * 3)(ptr(ws[2]), None, None),
         (C.c_void_p * 3)(ptr(yb[2]), None, None), (C.c_int * 3)(Ns[2], 0, 0), ptr(H), ptr(gd), C.c_float(1e-6),
         ptr(ss), M, K, *lws(), stream())
    for a, b in zip(ya, yb):
        assert np.array_equal(host(a), host(b))
    assert h.bx_linear_group2_f16(14, 12, 3, 2, W_arr, arr(ya), N_arr, ptr(x), M, K, *lws(), stream()) == -3
