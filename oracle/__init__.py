"""Python handle on the CPU oracle (liboracle.so).

TEST INFRASTRUCTURE ONLY: imported by tests/, __graft_entry__.smoke() and
bench.py's cpu_baseline leg as the checker.  The product (brolm_amd/) never
imports it.  See oracle.h for what each function restates and where it is
pinned.
"""
from __future__ import annotations

import ctypes as C
import subprocess
from pathlib import Path

import numpy as np

HERE = Path(__file__).resolve().parent
_lib = None

T_F32, T_F16, T_Q8_0, T_Q4_K, T_Q6_K, T_BF16 = 0, 1, 8, 12, 14, 30
P_f32 = C.POINTER(C.c_float)
P_u16 = C.POINTER(C.c_uint16)
P_i32 = C.POINTER(C.c_int32)


class Config(C.Structure):
    _fields_ = [(n, C.c_int) for n in ("vocab_size", "hidden_size", "intermediate_size", "num_hidden_layers",
                                        "num_attention_heads", "num_key_value_heads", "head_dim")] + [
        ("rms_norm_eps", C.c_float), ("rope_theta", C.c_float), ("tie_word_embeddings", C.c_int),
        ("max_position_embeddings", C.c_int), ("use_qk_norm", C.c_int)]


def build() -> Path:
    subprocess.run(["make", "-s", "-C", str(HERE)], check=True)
    return HERE / "liboracle.so"


def lib():
    global _lib
    if _lib is None:
        path = HERE / "liboracle.so"
        if not path.exists():
            build()
        l = C.CDLL(str(path))
        sig = {
            "or_f16_to_f32": (C.c_float, [C.c_uint16]),
            "or_f32_to_f16": (C.c_uint16, [C.c_float]),
            "or_bf16_to_f32": (C.c_float, [C.c_uint16]),
            "or_f32_to_bf16": (C.c_uint16, [C.c_float]),
            "or_f32_to_f16_array": (None, [P_f32, P_u16, C.c_int64]),
            "or_f16_to_f32_array": (None, [P_u16, P_f32, C.c_int64]),
            "or_type_block_elems": (C.c_int64, [C.c_int]),
            "or_type_block_bytes": (C.c_int64, [C.c_int]),
            "or_row_bytes": (C.c_int64, [C.c_int, C.c_int64]),
            "or_get_scale_min_k4": (None, [C.c_int, C.c_void_p, C.POINTER(C.c_uint8), C.POINTER(C.c_uint8)]),
            "or_dequant": (C.c_int, [C.c_int, C.c_void_p, C.c_int64, P_f32]),
            "or_gguf_open": (C.c_void_p, [C.c_char_p]),
            "or_gguf_open_memory": (C.c_void_p, [C.c_void_p, C.c_size_t]),
            "or_gguf_close": (None, [C.c_void_p]),
            "or_gguf_error": (C.c_char_p, []),
            "or_gguf_n_tensors": (C.c_int64, [C.c_void_p]),
            "or_gguf_find_tensor": (C.c_int64, [C.c_void_p, C.c_char_p]),
            "or_gguf_tensor_name": (C.c_char_p, [C.c_void_p, C.c_int64]),
            "or_gguf_tensor_type": (C.c_int, [C.c_void_p, C.c_int64]),
            "or_gguf_tensor_ndims": (C.c_int, [C.c_void_p, C.c_int64]),
            "or_gguf_tensor_dim": (C.c_int64, [C.c_void_p, C.c_int64, C.c_int]),
            "or_gguf_tensor_data": (C.c_void_p, [C.c_void_p, C.c_int64]),
            "or_gguf_tensor_nbytes": (C.c_int64, [C.c_void_p, C.c_int64]),
            "or_gguf_meta_int": (C.c_int, [C.c_void_p, C.c_char_p, C.POINTER(C.c_int64)]),
            "or_gguf_meta_f64": (C.c_int, [C.c_void_p, C.c_char_p, C.POINTER(C.c_double)]),
            "or_gguf_meta_str": (C.c_int, [C.c_void_p, C.c_char_p, C.POINTER(C.c_char_p)]),
            "or_gguf_meta_array_len": (C.c_int, [C.c_void_p, C.c_char_p, C.POINTER(C.c_int64)]),
            "or_rms_norm": (None, [P_f32, P_f32, C.c_float, P_f32, C.c_int, C.c_int]),
            "or_rope": (None, [P_f32, C.c_int, C.c_int, C.c_int, C.c_int, C.c_float]),
            "or_linear": (None, [P_f32, P_f32, P_f32, C.c_int, C.c_int, C.c_int]),
            "or_attention": (None, [P_f32, P_f32, P_f32, C.c_int, C.c_int, C.c_int, C.c_int, C.c_int, P_f32]),
            "or_silu": (C.c_float, [C.c_float]),
            "or_model_load": (C.c_void_p, [C.c_void_p]),
            "or_model_free": (None, [C.c_void_p]),
            "or_model_config": (None, [C.c_void_p, C.POINTER(Config)]),
            "or_model_allocate_cache": (C.c_int, [C.c_void_p, C.c_int]),
            "or_model_reset_cache": (None, [C.c_void_p]),
            "or_model_truncate_cache": (C.c_int, [C.c_void_p, C.c_int]),
            "or_model_cache_len": (C.c_int, [C.c_void_p]),
            "or_model_fill_cache": (C.c_int, [C.c_void_p, C.c_int, C.c_uint64]),
            "or_model_forward": (C.c_int, [C.c_void_p, P_i32, C.c_int, C.c_int, P_f32, P_f32]),
            "or_model_forward_encode": (C.c_int, [C.c_void_p, P_i32, C.c_int, P_f32]),
            "or_model_weight": (P_f32, [C.c_void_p, C.c_int, C.c_char_p, C.POINTER(C.c_int64),
                                        C.POINTER(C.c_int64)]),
            "or_argmax": (C.c_int, [P_f32, C.c_int, P_f32]),
            "or_sample_token": (C.c_int, [P_f32, C.c_int, C.c_float, C.c_int, C.c_float, C.c_double,
                                          C.POINTER(C.c_double)]),
            "or_generate_greedy": (C.c_int, [C.c_void_p, P_i32, C.c_int, C.c_int, C.c_int, P_i32, P_f32]),
            "or_num_threads": (C.c_int, []),
        }
        for name, (res, args) in sig.items():
            fn = getattr(l, name)
            fn.restype = res
            fn.argtypes = args
        _lib = l
    return _lib


def _f32p(a):
    return a.ctypes.data_as(P_f32)


def f16_to_f32(bits: np.ndarray) -> np.ndarray:
    b = np.ascontiguousarray(bits, dtype=np.uint16)
    out = np.empty(b.shape, np.float32)
    lib().or_f16_to_f32_array(b.ctypes.data_as(P_u16), _f32p(out), b.size)
    return out


def f32_to_f16(x: np.ndarray) -> np.ndarray:
    a = np.ascontiguousarray(x, dtype=np.float32)
    out = np.empty(a.shape, np.uint16)
    lib().or_f32_to_f16_array(_f32p(a), out.ctypes.data_as(P_u16), a.size)
    return out


def dequant(ggml_type: int, raw: bytes | np.ndarray, n: int) -> np.ndarray:
    buf = np.frombuffer(bytes(raw), dtype=np.uint8) if not isinstance(raw, np.ndarray) else np.ascontiguousarray(raw)
    out = np.empty((n,), np.float32)
    rc = lib().or_dequant(ggml_type, buf.ctypes.data_as(C.c_void_p), n, _f32p(out))
    if rc != 0:
        raise ValueError("or_dequant failed")
    return out


def scale_min_k4(j: int, scales12: bytes) -> tuple[int, int]:
    b = (C.c_uint8 * 12).from_buffer_copy(bytes(scales12))
    sc, m = C.c_uint8(), C.c_uint8()
    lib().or_get_scale_min_k4(j, C.cast(b, C.c_void_p), C.byref(sc), C.byref(m))
    return sc.value, m.value


def rms_norm(x: np.ndarray, gamma: np.ndarray, eps: float) -> np.ndarray:
    x = np.ascontiguousarray(x, np.float32)
    g = np.ascontiguousarray(gamma, np.float32)
    y = np.empty_like(x)
    lib().or_rms_norm(_f32p(x), _f32p(g), eps, _f32p(y), x.shape[0], x.shape[1])
    return y


def rope(x: np.ndarray, hd: int, n_heads: int, pos0: int, theta: float) -> np.ndarray:
    y = np.ascontiguousarray(x, np.float32).copy()
    lib().or_rope(_f32p(y), y.shape[0], hd, n_heads, pos0, theta)
    return y


def linear(W: np.ndarray, X: np.ndarray) -> np.ndarray:
    W = np.ascontiguousarray(W, np.float32)
    X = np.ascontiguousarray(X, np.float32)
    Y = np.empty((X.shape[0], W.shape[0]), np.float32)
    lib().or_linear(_f32p(W), _f32p(X), _f32p(Y), X.shape[0], W.shape[0], W.shape[1])
    return Y


def attention(q, Kc, Vc, L, pos0, n_q, n_kv, hd) -> np.ndarray:
    q = np.ascontiguousarray(q, np.float32)
    Kc = np.ascontiguousarray(Kc, np.float32)
    Vc = np.ascontiguousarray(Vc, np.float32)
    out = np.empty((L, n_q * hd), np.float32)
    lib().or_attention(_f32p(q), _f32p(Kc), _f32p(Vc), L, pos0, n_q, n_kv, hd, _f32p(out))
    return out


def argmax(logits: np.ndarray) -> tuple[int, float]:
    a = np.ascontiguousarray(logits, np.float32)
    m = C.c_float()
    i = lib().or_argmax(_f32p(a), a.size, C.byref(m))
    return i, m.value


def sample_token(logits: np.ndarray, temperature: float, top_k: int, top_p: float, u: float) -> tuple[int, float]:
    """sample_token (src/detail/generate.cpp:68-142) with the uniform draw u;
    returns (token, margin of u to the chosen interval's ends / kept mass)."""
    a = np.ascontiguousarray(logits, np.float32)
    m = C.c_double()
    t = lib().or_sample_token(_f32p(a), a.size, temperature, top_k, top_p, u, C.byref(m))
    return t, m.value


class Gguf:
    """Oracle GGUF reader."""

    def __init__(self, path: str):
        self._h = lib().or_gguf_open(str(path).encode())
        if not self._h:
            raise ValueError(lib().or_gguf_error().decode())

    def close(self):
        if getattr(self, "_h", None) and _lib is not None:
            _lib.or_gguf_close(self._h)
        self._h = None

    def __del__(self):
        self.close()

    def tensor_names(self) -> list[str]:
        return [lib().or_gguf_tensor_name(self._h, i).decode() for i in range(lib().or_gguf_n_tensors(self._h))]

    def tensor(self, name: str):
        i = lib().or_gguf_find_tensor(self._h, name.encode())
        if i < 0:
            raise KeyError(name)
        nd = lib().or_gguf_tensor_ndims(self._h, i)
        dims = [lib().or_gguf_tensor_dim(self._h, i, d) for d in range(nd)]
        nb = lib().or_gguf_tensor_nbytes(self._h, i)
        ptr = lib().or_gguf_tensor_data(self._h, i)
        raw = np.frombuffer((C.c_uint8 * nb).from_address(ptr), dtype=np.uint8).copy()
        return lib().or_gguf_tensor_type(self._h, i), dims, raw

    def meta_int(self, key: str):
        v = C.c_int64()
        return v.value if lib().or_gguf_meta_int(self._h, key.encode(), C.byref(v)) == 0 else None

    def meta_f64(self, key: str):
        v = C.c_double()
        return v.value if lib().or_gguf_meta_f64(self._h, key.encode(), C.byref(v)) == 0 else None

    def meta_str(self, key: str):
        v = C.c_char_p()
        return v.value.decode() if lib().or_gguf_meta_str(self._h, key.encode(), C.byref(v)) == 0 else None


class Model:
    """FP32 Qwen3 decoder on dequantized weights (dense_decoder.cpp:526-681)."""

    def __init__(self, gguf_path: str):
        self._g = Gguf(gguf_path)
        self._h = lib().or_model_load(self._g._h)
        if not self._h:
            raise ValueError(lib().or_gguf_error().decode())
        c = Config()
        lib().or_model_config(self._h, C.byref(c))
        self.cfg = c

    def __del__(self):
        if getattr(self, "_h", None) and _lib is not None:
            _lib.or_model_free(self._h)
        self._h = None

    def allocate_cache(self, n: int) -> None:
        if lib().or_model_allocate_cache(self._h, n) != 0:
            raise ValueError("allocate_cache")

    def reset_cache(self) -> None:
        lib().or_model_reset_cache(self._h)

    def truncate_cache(self, n: int) -> None:
        if lib().or_model_truncate_cache(self._h, n) != 0:
            raise ValueError("truncate_cache")

    def fill_cache(self, n: int, seed: int = 1) -> None:
        """Benchmark helper: deterministic K / V rows [0, n), cache_len = n."""
        if lib().or_model_fill_cache(self._h, n, seed) != 0:
            raise ValueError("fill_cache")

    def cache_len(self) -> int:
        return lib().or_model_cache_len(self._h)

    def forward(self, ids, last_only=False, want_hidden=False):
        a = np.ascontiguousarray(np.asarray(ids, np.int32))
        L = a.size
        logits = np.empty((1 if last_only else L, self.cfg.vocab_size), np.float32)
        hidden = np.empty((L, self.cfg.hidden_size), np.float32) if want_hidden else None
        rc = lib().or_model_forward(self._h, a.ctypes.data_as(P_i32), L, 1 if last_only else 0, _f32p(logits),
                                    _f32p(hidden) if want_hidden else None)
        if rc != 0:
            raise ValueError(lib().or_gguf_error().decode())
        return (logits, hidden) if want_hidden else logits

    def forward_encode(self, ids) -> np.ndarray:
        """Bidirectional, cacheless (L, H) post-final-norm hidden states."""
        a = np.ascontiguousarray(np.asarray(ids, np.int32))
        out = np.empty((len(a), self.cfg.hidden_size), np.float32)
        if lib().or_model_forward_encode(self._h, a.ctypes.data_as(P_i32), len(a), _f32p(out)) != 0:
            raise RuntimeError(lib().or_gguf_error().decode())
        return out

    def weight(self, layer: int, which: str) -> np.ndarray:
        r, c = C.c_int64(), C.c_int64()
        p = lib().or_model_weight(self._h, layer, which.encode(), C.byref(r), C.byref(c))
        if not p:
            raise KeyError(which)
        return np.ctypeslib.as_array(p, shape=(r.value * c.value,)).reshape(r.value, c.value).copy()

    def generate_greedy(self, prompt, max_new: int, eos_id: int = -1):
        a = np.ascontiguousarray(np.asarray(prompt, np.int32))
        out = np.empty((max(max_new, 1),), np.int32)
        margins = np.empty((max(max_new, 1),), np.float32)
        n = lib().or_generate_greedy(self._h, a.ctypes.data_as(P_i32), a.size, max_new, eos_id,
                                     out.ctypes.data_as(P_i32), _f32p(margins))
        if n < 0:
            raise ValueError("generate failed")
        return out[:n].tolist(), margins[:n].copy()


def num_threads() -> int:
    return lib().or_num_threads()
