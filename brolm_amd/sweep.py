"""Isolated quant-GEMV sweep.

Weight matrices [N, K] in {(3072,1024), (1024,3072), (6144,2048), (2048,6144),
(151936,2048)} x {Q8_0, Q4_K, Q6_K}, FP16 activations N(0,1), batch
M in {1,2,4,8,16}.  Each timed batch rotates over enough distinct weight
copies (> 2 GB) that the 256 MB Infinity Cache cannot serve repeats; the
launch time is the median over >= 100 launches (HIP events on the launch
stream).  GB/s counts the carrier bytes + M*(K+N)*2 activation bytes.

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


def time_case(torch, t: str, n: int, k: int, m: int, weights, reps: int = 100) -> dict:
    hip = _native.hip()
    st = torch.cuda.current_stream()
    x = torch.randn(m, k, device="cuda", dtype=torch.float16)
    y = torch.empty(m, n, device="cuda", dtype=torch.float16)

    def launch(w):
        _native.bx_check(hip.bx_linear_f16(GGML[t], C.c_void_p(w.data_ptr()), None, C.c_void_p(x.data_ptr()),
                                           C.c_void_p(y.data_ptr()), m, n, k, C.c_void_p(st.cuda_stream)), "linear")

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
    byts = carrier_bytes(t, n, k) + m * (k + n) * 2
    return {"type": t, "N": n, "K": k, "M": m, "us": round(med, 3), "GBps": round(byts / (med * 1e-6) / 1e9, 1),
            "frac": round(byts / (med * 1e-6) / 1e9 / HBM_PEAK, 4), "bytes": byts}


def main(argv=None) -> int:
    ap = argparse.ArgumentParser()
    ap.add_argument("--shapes", default=",".join(f"{n}x{k}" for n, k in SHAPES))
    ap.add_argument("--types", default=",".join(TYPES))
    ap.add_argument("--ms", default=",".join(map(str, MS)))
    ap.add_argument("--rotate-gb", type=float, default=2.5)
    ap.add_argument("--json", default=None)
    a = ap.parse_args(argv)
    import torch

    shapes = [tuple(int(v) for v in s.split("x")) for s in a.shapes.split(",")]
    rows = []
    for t in a.types.split(","):
        for n, k in shapes:
            nb = carrier_bytes(t, n, k)
            copies = max(2, min(64, int(a.rotate_gb * 1e9 // nb) + 1))
            ws = make_weights(torch, t, n, k, copies, seed=n * 7 + k)
            for m in [int(v) for v in a.ms.split(",")]:
                r = time_case(torch, t, n, k, m, ws)
                r["copies"] = copies
                rows.append(r)
                print(json.dumps(r), flush=True)
            del ws
            torch.cuda.empty_cache()
    if a.json:
        with open(a.json, "w") as f:
            json.dump(rows, f, indent=1)
    return 0


if __name__ == "__main__":
    sys.exit(main())
