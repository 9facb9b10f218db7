"""Device plumbing for the GPU tests: torch allocates device memory, every
kernel is reached through the C ABI of libbrolm_hip.so (include/brolm_hip.h)."""
from __future__ import annotations

import ctypes as C

import numpy as np


def torch():
    import torch as t
    return t


def hip():
    from brolm_amd import _native
    return _native.hip()


_alive: list = []


def ptr(t) -> C.c_void_p | None:
    """Raw device pointer of a torch tensor.  The tensor is kept alive until
    release(): a temporary freed right after this call would hand its block to
    the next allocation before the kernel reading it has run."""
    if t is None:
        return None
    _alive.append(t)
    return C.c_void_p(t.data_ptr())


def release() -> None:
    torch().cuda.synchronize()
    _alive.clear()


def stream() -> C.c_void_p:
    return C.c_void_p(torch().cuda.current_stream().cuda_stream)


_ws: dict = {}


def new_workspace():
    """A fresh split-K workspace for the bx_linear_* entry points: a device
    buffer of bx_linear_workspace_bytes() bytes, counters cleared by
    bx_linear_workspace_init on the current stream.  Returns (buffer, bytes)."""
    n = int(hip().bx_linear_workspace_bytes())
    buf = torch().empty(n, dtype=torch().uint8, device="cuda")
    call("bx_linear_workspace_init", C.c_void_p(buf.data_ptr()), C.c_size_t(n), stream())
    return buf, n


def lws():
    """(pointer, bytes) of the module-wide workspace the tests hand to every
    bx_linear_* call on the default stream; made once per process."""
    if "buf" not in _ws:
        _ws["buf"], _ws["n"] = new_workspace()
    return C.c_void_p(_ws["buf"].data_ptr()), C.c_size_t(_ws["n"])


def dev(a: np.ndarray):
    return torch().from_numpy(np.ascontiguousarray(a)).to("cuda")


def empty(n: int, dtype=None):
    t = torch()
    return t.empty(n, dtype=dtype or t.uint8, device="cuda")


def host(t) -> np.ndarray:
    torch().cuda.synchronize()
    return t.cpu().numpy()


def call(name: str, *args) -> None:
    rc = getattr(hip(), name)(*args)
    if rc != 0:
        raise RuntimeError(f"{name}: code {rc}: {hip().bx_last_error().decode()}")


def carrier(ggml_type: int, raw: bytes, rows: int, cols: int):
    """GGUF bytes -> device carrier (bx_repack_gguf_rows)."""
    stage = dev(np.frombuffer(raw, np.uint8).copy())
    out = torch().empty_like(stage)
    call("bx_repack_gguf_rows", ggml_type, ptr(stage), ptr(out), rows, cols, stream())
    return out


def f16_dev(a: np.ndarray):
    return dev(np.asarray(a, np.float32).astype(np.float16).view(np.uint16))


def f16_host(t) -> np.ndarray:
    return host(t).view(np.float16).astype(np.float32)
