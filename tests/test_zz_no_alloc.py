"""bx_argmax_f16_noalloc (a fixed device array in place of the workspace)
against bx_argmax_f16 through the C ABI: two calls in a row, the second on a
smaller input, results identical (bit-exact indices) and equal to the
reference's tie rule (lowest index of the maximum, generate.cpp:38-48)."""
from __future__ import annotations

import numpy as np
import pytest

import oracle
from gpu_util import empty, f16_dev, hip, host, ptr, release, stream, torch

pytestmark = pytest.mark.gpu


def _f16(a):
    return np.asarray(a, np.float32).astype(np.float16)


def _argmax_ws(x) -> int:
    n = x.size
    ws = empty(hip().bx_argmax_workspace_bytes(n))
    out = torch().empty(1, dtype=torch().int32, device="cuda")
    assert hip().bx_argmax_f16(ptr(f16_dev(x)), n, ptr(out), ptr(ws), stream()) == 0
    return int(host(out)[0])


def _argmax_noalloc(x) -> int:
    out = torch().full((1,), -7, dtype=torch().int32, device="cuda")
    assert hip().bx_argmax_f16_noalloc(ptr(f16_dev(x)), x.size, ptr(out), stream()) == 0, hip().bx_last_error()
    return int(host(out)[0])


def test_noalloc_matches_workspace_entry_twice_second_smaller():
    rng = np.random.default_rng(2026)
    for n in (151936 + 1000, 4096 + 3):   # second call smaller: fewer partial blocks than the first wrote
        x = _f16(rng.standard_normal(n))
        top = x.max()
        idx = np.sort(rng.choice(n, size=4, replace=False))
        x[idx] = top + 1      # ties of the maximum: the lowest index wins
        a = _argmax_noalloc(x)
        b = _argmax_ws(x)
        assert a == b == oracle.argmax(x)[0] == idx[0]
    # a tiny input after the large ones (one partial block)
    x = _f16([0.5, 2.0, 2.0, -1.0])
    assert _argmax_noalloc(x) == _argmax_ws(x) == 1
    release()


def test_noalloc_rejects_bad_arguments():
    out = torch().empty(1, dtype=torch().int32, device="cuda")
    x = torch().zeros(8, dtype=torch().float16, device="cuda")
    h = hip()
    assert h.bx_argmax_f16_noalloc(None, 8, ptr(out), stream()) != 0
    assert h.bx_argmax_f16_noalloc(ptr(x), 0, ptr(out), stream()) != 0
    assert h.bx_argmax_f16_noalloc(ptr(x), 1 << 31, ptr(out), stream()) != 0
    assert b"argmax_noalloc" in h.bx_last_error()
    release()
