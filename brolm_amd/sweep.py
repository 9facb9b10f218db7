"""Isolated quant-GEMV sweep.

Weight matrices [N, K] in {(3072,1024), (1024,3072), (6144,2048), (2048,6144),
(151936,2048)} x {Q8_0, Q4_K, Q6_K}, FP16 activations N(0,1), batch
M in {1,2,4,8,16}.  Each timed batch rotates over distinct weight copies
totalling about --rotate-gb (2.5 GB: ten times the 256 MB Infinity Cache, so
repeats come from HBM; a row whose rotation stays under 512 MB says
"cache_resident").  Two timings per case:
  us        median of 100 launches, HIP events around each launch (includes
            the GPU-side dispatch gap, so small matrices read launch-bound);
  us_batch  100 back-to-back launches between two events / 100 (dispatch
            overlapped, the kernels' own throughput).
GB/s counts the carrier bytes + M*(K+N)*2 activation bytes.  Every row
also checks the output of its last timed launch against X W^T in FP32 on the
dequantized weights ("err_over_tol", "ok"); the run exits nonzero when a row
fails, so a fast kernel that computes the wrong thing cannot post a number.  The comparison
leg "ref_fp32_us" is the reference's FP32 route for a quantized weight
(include/brolm/detail/compute.h:77-85: dequantize to FP32, then an FP32
GEMM; here bx_dequant_to_f32 then torch.matmul in FP32) on the same case.
The first line printed is the measured device-copy bandwidth.

Device memory comes from torch (plumbing only); every GEMV runs through the
C ABI bx_linear_f16 of libbrolm_hip.so.

    python -m brolm_amd.sweep [--shapes ...] [--types ...] [--ms ...] [--json out.json]
"""
from __future__ import annotations

import argparse
import ctypes as C
import json
import statistics
import sys

import numpy as np

from . import GGML, _native

SHAPES = [(3072, 1024), (1024, 3072), (6144, 2048), (2048, 6144), (151936, 2048)]
TYPES = ["Q8_0", "Q4_K", "Q6_K"]
MS = [1, 2, 4, 8, 16]
BLOCK = {"Q8_0": (32, 34), "Q4_K": (256, 144), "Q6_K": (256, 210), "F16": (1, 2)}
HBM_PEAK = 8000.0


def carrier_bytes(t: str, n: int, k: int) -> int:
    be, bb = BLOCK[t]
    return n * (k // be) * bb


def make_weights(torch, t: str, n: int, k: int, copies: int, seed: int):
    """`copies` device carriers of one seeded N(0, 0.02) matrix at distinct
    addresses (the caches key on addresses, so identical bytes still miss)."""
    rng = np.random.default_rng(seed)
    nbytes = carrier_bytes(t, n, k)
    lib = _native.lib()
    hip = _native.hip()
    w = (rng.standard_normal((n, k), dtype=np.float32) * 0.02)
    raw = np.empty(nbytes, np.uint8)
    _native.check(lib.brolm_synth_quantize(GGML[t], w.ctypes.data_as(_native.P_f32), w.size,
                                           raw.ctypes.data_as(_native.P_u8)), "quantize")
    stage = torch.from_numpy(raw).to("cuda")
    first = torch.empty(nbytes, dtype=torch.uint8, device="cuda")
    _native.bx_check(hip.bx_repack_gguf_rows(GGML[t], C.c_void_p(stage.data_ptr()), C.c_void_p(first.data_ptr()),
                                             n, k, C.c_void_p(torch.cuda.current_stream().cuda_stream)), "repack")
    out = [first] + [first.clone() for _ in range(copies - 1)]
    torch.cuda.synchronize()
    return out


_WS: dict = {}


def workspace(torch):
    """(pointer, bytes) of the split-K workspace handed to every timed launch,
    allocated and cleared once (bx_linear_workspace_bytes / _init)."""
    if "buf" not in _WS:
        hip = _native.hip()
        n = int(hip.bx_linear_workspace_bytes())
        _WS["buf"] = torch.empty(n, dtype=torch.uint8, device="cuda")
        _WS["n"] = n
        _native.bx_check(hip.bx_linear_workspace_init(C.c_void_p(_WS["buf"].data_ptr()), C.c_size_t(n),
                                                      C.c_void_p(torch.cuda.current_stream().cuda_stream)),
                         "workspace")
    return C.c_void_p(_WS["buf"].data_ptr()), C.c_size_t(_WS["n"])


def check_output(torch, t: str, n: int, k: int, x, y, w) -> float:
    """Worst |y - ref| / tol over the launch's output, ref = X W^T in FP32 on
    the exactly dequantized weights (bx_dequant_to_f32, bit-exact to the
    block formats), tol = 2^-10 |ref| (FP16 output rounding, doubled) +
    2^-14 sum |x||w| (FP32 accumulation order) + 1e-6.  A value above 1
    means the timed kernel computed something else."""
    hip = _native.hip()
    st = torch.cuda.current_stream()
    wf = torch.empty(n, k, device="cuda", dtype=torch.float32)
    _native.bx_check(hip.bx_dequant_to_f32(GGML[t], C.c_void_p(w.data_ptr()), C.c_void_p(wf.data_ptr()), n, k,
                                           C.c_void_p(st.cuda_stream)), "dequant")
    xf = x.float()
    ref = xf @ wf.t()
    mass = xf.abs() @ wf.abs().t()
    tol = 2.0 ** -10 * ref.abs() + 2.0 ** -14 * mass + 1e-6
    worst = float(((y.float() - ref).abs() / tol).max())
    del wf, ref, mass, tol
    return worst


def time_case(torch, t: str, n: int, k: int, m: int, weights, reps: int = 100) -> dict:
    hip = _native.hip()
    st = torch.cuda.current_stream()
    x = torch.randn(m, k, device="cuda", dtype=torch.float16)
    y = torch.empty(m, n, device="cuda", dtype=torch.float16)
    wsp, wsb = workspace(torch)

    def launch(w):
        _native.bx_check(hip.bx_linear_f16(GGML[t], C.c_void_p(w.data_ptr()), None, C.c_void_p(x.data_ptr()),
                                           C.c_void_p(y.data_ptr()), m, n, k, wsp, wsb, C.c_void_p(st.cuda_stream)),
                         "linear")

    for w in weights[:4]:
        launch(w)
    torch.cuda.synchronize()
    times = []
    evs = [(torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)) for _ in range(reps)]
    for i in range(reps):
        w = weights[i % len(weights)]
        evs[i][0].record(st)
        launch(w)
        evs[i][1].record(st)
    torch.cuda.synchronize()
    times = [a.elapsed_time(b) * 1e3 for a, b in evs]  # us
    med = statistics.median(times)
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    e0.record(st)
    for i in range(reps):
        launch(weights[i % len(weights)])
    e1.record(st)
    torch.cuda.synchronize()
    batch = e0.elapsed_time(e1) * 1e3 / reps
    worst = check_output(torch, t, n, k, x, y, weights[(reps - 1) % len(weights)])
    byts = carrier_bytes(t, n, k) + m * (k + n) * 2
    return {"type": t, "N": n, "K": k, "M": m, "us": round(med, 3), "GBps": round(byts / (med * 1e-6) / 1e9, 1),
            "frac": round(byts / (med * 1e-6) / 1e9 / HBM_PEAK, 4), "us_batch": round(batch, 3),
            "GBps_batch": round(byts / (batch * 1e-6) / 1e9, 1), "bytes": byts, "err_over_tol": round(worst, 4),
            "ok": worst <= 1.0}


def time_ref_fp32(torch, t: str, n: int, k: int, m: int, w, reps: int = 20) -> float:
    """Dequantize the carrier to FP32, then X (M, K) @ W^T in FP32: the route
    the reference takes for a weight dtype without a quant kernel."""
    hip = _native.hip()
    st = torch.cuda.current_stream()
    x = torch.randn(m, k, device="cuda", dtype=torch.float32)
    wf = torch.empty(n, k, device="cuda", dtype=torch.float32)

    def run():
        _native.bx_check(hip.bx_dequant_to_f32(GGML[t], C.c_void_p(w.data_ptr()), C.c_void_p(wf.data_ptr()), n, k,
                                               C.c_void_p(st.cuda_stream)), "dequant")
        return x @ wf.t()

    run()
    torch.cuda.synchronize()
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    e0.record(st)
    for _ in range(reps):
        run()
    e1.record(st)
    torch.cuda.synchronize()
    return e0.elapsed_time(e1) * 1e3 / reps


def main(argv=None) -> int:
    ap = argparse.ArgumentParser()
    ap.add_argument("--shapes", default=",".join(f"{n}x{k}" for n, k in SHAPES))
    ap.add_argument("--types", default=",".join(TYPES))
    ap.add_argument("--ms", default=",".join(map(str, MS)))
    ap.add_argument("--rotate-gb", type=float, default=2.5)
    ap.add_argument("--json", default=None)
    ap.add_argument("--no-ref", action="store_true", help="skip the dequant + FP32 GEMM comparison leg")
    a = ap.parse_args(argv)
    import torch

    src = torch.empty(2 << 30, dtype=torch.uint8, device="cuda")
    dst = torch.empty_like(src)
    dst.copy_(src)
    torch.cuda.synchronize()
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    e0.record()
    for _ in range(10):
        dst.copy_(src)
    e1.record()
    torch.cuda.synchronize()
    print(json.dumps({"stream_copy_GBps": round(2.0 * src.numel() * 10 / (e0.elapsed_time(e1) * 1e-3) / 1e9, 1)}),
          flush=True)
    del src, dst
    torch.cuda.empty_cache()

    shapes = [tuple(int(v) for v in s.split("x")) for s in a.shapes.split(",")]
    rows = []
    for t in a.types.split(","):
        for n, k in shapes:
            nb = carrier_bytes(t, n, k)
            copies = max(2, min(4096, int(a.rotate_gb * 1e9 // nb) + 1))
            ws = make_weights(torch, t, n, k, copies, seed=n * 7 + k)
            for m in [int(v) for v in a.ms.split(",")]:
                r = time_case(torch, t, n, k, m, ws)
                r["copies"] = copies
                r["cache_resident"] = copies * nb < 512e6
                if not a.no_ref:
                    r["ref_fp32_us"] = round(time_ref_fp32(torch, t, n, k, m, ws[0]), 3)
                rows.append(r)
                print(json.dumps(r), flush=True)
            del ws
            torch.cuda.empty_cache()
    if a.json:
        with open(a.json, "w") as f:
            json.dump(rows, f, indent=1)
    bad = [r for r in rows if not r["ok"]]
    if bad:
        print(f"{len(bad)} row(s) failed the output check", file=sys.stderr)
        return 1
    return 0


if __name__ == "__main__":
    sys.exit(main())
