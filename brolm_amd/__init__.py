"""brolm_amd — MI355X-native implementation of brolm's quantized Qwen3 decode path.

Python mirror of the C++ API (reference include/brolm/qwen.h,
include/brolm/qwen_generate.h, include/brolm/detail/generate.h,
include/brolm/mistral3_text.h, include/brolm/mistral3_config.h) over the C ABI
of libbrolm.so.  All compute runs in the native libraries on a gfx950 device;
there is no Python or CPU fallback.
"""
from __future__ import annotations

import atexit
import ctypes as C
from dataclasses import dataclass, field
from typing import Optional, Sequence

import numpy as np

from . import _native
from ._native import check

GGML = {"F32": 0, "F16": 1, "Q8_0": 8, "Q4_K": 12, "Q6_K": 14, "BF16": 30}

__all__ = ["Qwen3Config", "Qwen3Model", "SamplingParams", "GenerateOptions", "generate", "sample_token",
           "qwen3_hf_to_ggml", "SynthSpec", "write_synth_qwen3", "init", "GGML", "Mistral3Config",
           "Mistral3TextConfig", "Mistral3TextModel", "mistral3_hf_to_ggml", "write_synth_mistral3",
           "Llm2VecConfig", "Llm2VecEncoder", "shutdown",
           "PROFILE_STAGES", "profile_stages", "profile_reset", "profile_report"]


def init() -> None:
    """brotensor::init(): register the gfx950 device (raises without one).
    The first call also registers shutdown() with atexit, so the runtime's
    own device buffers and stream are released while the HIP runtime is
    still whole, before the process's exit handlers run."""
    global _atexit_registered
    check(_native.lib().brolm_init(), "init")
    if not _atexit_registered:
        atexit.register(shutdown)
        _atexit_registered = True


def shutdown() -> None:
    """brotensor::shutdown(): wait for queued work, free the runtime's scratch,
    sampler buffers and profiler events, destroy the op stream.  Open models
    stay valid to close(); init() may be called again."""
    check(_native.lib().brolm_shutdown(), "shutdown")


_atexit_registered = False


def _i32(a) -> "C.Array":
    arr = np.ascontiguousarray(np.asarray(a, dtype=np.int32))
    return arr, arr.ctypes.data_as(_native.P_i32)


@dataclass
class Qwen3Config:
    """Qwen3Config (include/brolm/qwen.h:35-56)."""
    vocab_size: int = 151936
    hidden_size: int = 1024
    intermediate_size: int = 3072
    num_hidden_layers: int = 28
    num_attention_heads: int = 16
    num_key_value_heads: int = 8
    head_dim: int = 128
    rms_norm_eps: float = 1e-6
    rope_theta: float = 1000000.0
    tie_word_embeddings: bool = True
    max_position_embeddings: int = 40960

    def _c(self) -> _native.Qwen3ConfigC:
        c = _native.Qwen3ConfigC()
        for f in ("vocab_size", "hidden_size", "intermediate_size", "num_hidden_layers", "num_attention_heads",
                  "num_key_value_heads", "head_dim", "max_position_embeddings"):
            setattr(c, f, int(getattr(self, f)))
        c.rms_norm_eps = float(self.rms_norm_eps)
        c.rope_theta = float(self.rope_theta)
        c.tie_word_embeddings = 1 if self.tie_word_embeddings else 0
        return c

    @staticmethod
    def from_gguf(path: str) -> "Qwen3Config":
        c = _native.Qwen3ConfigC()
        check(_native.lib().brolm_qwen3_config_from_gguf(str(path).encode(), C.byref(c)), "from_gguf")
        return Qwen3Config(c.vocab_size, c.hidden_size, c.intermediate_size, c.num_hidden_layers,
                           c.num_attention_heads, c.num_key_value_heads, c.head_dim, c.rms_norm_eps, c.rope_theta,
                           bool(c.tie_word_embeddings), c.max_position_embeddings)


def qwen3_hf_to_ggml(hf_name: str) -> str:
    buf = C.create_string_buffer(256)
    n = _native.lib().brolm_qwen3_hf_to_ggml(hf_name.encode(), buf, 256)
    return buf.value.decode() if n > 0 else ""


class Qwen3Model:
    """Qwen3Model (include/brolm/qwen.h:58-157); logits are returned as float32
    copies of the FP16 device logits."""

    def __init__(self, cfg: Qwen3Config):
        self.cfg = cfg
        self._h = _native.lib().brolm_qwen3_create(C.byref(cfg._c()))
        if not self._h:
            raise _native.NativeError(_native.lib().brolm_last_error().decode())

    def close(self) -> None:
        """Free the device state now (weights, KV cache, decode sessions)
        rather than at garbage collection."""
        h = getattr(self, "_h", None)
        if h:
            _native.lib().brolm_qwen3_free(h)
            self._h = None

    def __del__(self):
        self.close()

    def config(self) -> Qwen3Config:
        return self.cfg

    def load_weights(self, gguf_path: str) -> None:
        check(_native.lib().brolm_qwen3_load_gguf(self._h, str(gguf_path).encode()), "load_weights")

    def allocate_cache(self, max_seq_len: int) -> None:
        check(_native.lib().brolm_qwen3_allocate_cache(self._h, int(max_seq_len)), "allocate_cache")

    def reset_cache(self) -> None:
        check(_native.lib().brolm_qwen3_reset_cache(self._h), "reset_cache")

    def truncate_cache(self, length: int) -> None:
        check(_native.lib().brolm_qwen3_truncate_cache(self._h, int(length)), "truncate_cache")

    def cache_len(self) -> int:
        return _native.lib().brolm_qwen3_cache_len(self._h)

    def forward(self, ids: Sequence[int], want_hidden: bool = False):
        arr, p = _i32(ids)
        L = arr.size
        logits = np.empty((L, self.cfg.vocab_size), np.float32)
        hidden = np.empty((L, self.cfg.hidden_size), np.float32) if want_hidden else None
        check(_native.lib().brolm_qwen3_forward(self._h, p, L, logits.ctypes.data_as(_native.P_f32),
                                                hidden.ctypes.data_as(_native.P_f32) if want_hidden else None),
              "forward")
        return (logits, hidden) if want_hidden else logits

    def forward_last(self, ids: Sequence[int]) -> np.ndarray:
        arr, p = _i32(ids)
        logits = np.empty((self.cfg.vocab_size,), np.float32)
        check(_native.lib().brolm_qwen3_forward_last(self._h, p, arr.size, logits.ctypes.data_as(_native.P_f32)),
              "forward_last")
        return logits

    def embed_tokens(self, ids: Sequence[int]) -> np.ndarray:
        arr, p = _i32(ids)
        out = np.empty((arr.size, self.cfg.hidden_size), np.float16)
        check(_native.lib().brolm_qwen3_embed_tokens(self._h, p, arr.size, out.ctypes.data_as(_native.P_u16)),
              "embed_tokens")
        return out

    def forward_embeds(self, embeds: np.ndarray, want_hidden: bool = False):
        e = np.ascontiguousarray(embeds, dtype=np.float16)
        L = e.shape[0]
        logits = np.empty((L, self.cfg.vocab_size), np.float32)
        hidden = np.empty((L, self.cfg.hidden_size), np.float32) if want_hidden else None
        check(_native.lib().brolm_qwen3_forward_embeds(self._h, e.ctypes.data_as(_native.P_u16), L,
                                                       logits.ctypes.data_as(_native.P_f32),
                                                       hidden.ctypes.data_as(_native.P_f32) if want_hidden else None),
              "forward_embeds")
        return (logits, hidden) if want_hidden else logits

    def forward_encode(self, ids: Sequence[int]) -> np.ndarray:
        """DenseDecoder::forward_encode (dense_decoder.h:157-169): bidirectional,
        cacheless; (L, hidden) post-final-norm hidden states."""
        arr, p = _i32(ids)
        out = np.empty((len(ids), self.cfg.hidden_size), np.float32)
        check(_native.lib().brolm_decoder_forward_encode(self._h, p, len(ids), out.ctypes.data_as(_native.P_f32)),
              "forward_encode")
        return out

    def decode_greedy(self, token: int, n: int, eos_id: int = -1) -> list[int]:
        out = np.empty((max(n, 1),), np.int32)
        k = check(_native.lib().brolm_qwen3_decode_greedy(self._h, int(token), int(n),
                                                          out.ctypes.data_as(_native.P_i32), int(eos_id)),
                  "decode_greedy")
        return out[:k].tolist()

    def decode_sampled(self, token: int, u: Sequence[float], temperature: float, top_k: int = 0,
                       top_p: float = 1.0, eos_id: int = -1) -> list[int]:
        """Top-k / top-p continuation on the device, step i drawing with u[i]."""
        uu = np.ascontiguousarray(np.asarray(u, dtype=np.float64))
        out = np.empty((max(uu.size, 1),), np.int32)
        k = check(_native.lib().brolm_qwen3_decode_sampled(self._h, int(token), uu.size, uu.ctypes.data_as(C.c_void_p),
                                                           float(temperature), int(top_k), float(top_p),
                                                           out.ctypes.data_as(_native.P_i32), int(eos_id)),
                  "decode_sampled")
        return out[:k].tolist()

    def time_decode_steps(self, token: int, n: int) -> float:
        ms = _native.lib().brolm_qwen3_time_decode_steps(self._h, int(token), int(n))
        if ms < 0:
            raise _native.NativeError(_native.lib().brolm_last_error().decode())
        return ms

    # -- multi-sequence batched decode (beyond the reference's one-sequence model)
    def allocate_batch(self, n_slots: int, max_seq_len: int) -> None:
        """n_slots independent sequences, each with its own KV rows."""
        check(_native.lib().brolm_qwen3_allocate_batch(self._h, int(n_slots), int(max_seq_len)), "allocate_batch")

    def slot_len(self, slot: int) -> int:
        return check(_native.lib().brolm_qwen3_slot_len(self._h, int(slot)), "slot_len")

    def truncate_slot(self, slot: int, length: int) -> None:
        check(_native.lib().brolm_qwen3_truncate_slot(self._h, int(slot), int(length)), "truncate_slot")

    def prefill_slot(self, slot: int, ids: Sequence[int]) -> np.ndarray:
        """Appends a prompt to one slot; logits of its last token."""
        arr, p = _i32(ids)
        logits = np.empty((self.cfg.vocab_size,), np.float32)
        check(_native.lib().brolm_qwen3_prefill_slot(self._h, int(slot), p, arr.size,
                                                     logits.ctypes.data_as(_native.P_f32)), "prefill_slot")
        return logits

    def forward_batch(self, ids: Sequence[int], slots: Sequence[int]) -> np.ndarray:
        """One decode step of len(ids) sequences: ids[r] joins slot slots[r];
        (M, vocab) logits."""
        a, pa = _i32(ids)
        b, pb = _i32(slots)
        if a.size != b.size:
            raise ValueError("forward_batch: ids and slots differ in length")
        logits = np.empty((a.size, self.cfg.vocab_size), np.float32)
        check(_native.lib().brolm_qwen3_forward_batch(self._h, pa, pb, a.size, logits.ctypes.data_as(_native.P_f32)),
              "forward_batch")
        return logits

    def time_forward_batch(self, ids: Sequence[int], slots: Sequence[int], n: int) -> float:
        """Wall-clock ms per batched step over n steps (logits stay on the device)."""
        a, pa = _i32(ids)
        b, pb = _i32(slots)
        if a.size != b.size:
            raise ValueError("time_forward_batch: ids and slots differ in length")
        ms = _native.lib().brolm_qwen3_time_forward_batch(self._h, pa, pb, a.size, int(n))
        if ms < 0:
            raise _native.NativeError(_native.lib().brolm_last_error().decode())
        return ms

    def decode_weight_bytes(self) -> int:
        return int(_native.lib().brolm_qwen3_decode_weight_bytes(self._h))

    def decode_mode(self) -> str:
        """Which single-token step path runs: "persistent", "graph", "eager" or
        "op" (one forward_last per token)."""
        m = check(_native.lib().brolm_qwen3_decode_mode(self._h), "decode_mode")
        return ("eager", "graph", "persistent", "op")[m]


@dataclass
class Mistral3TextConfig:
    """Mistral3Config::Text (include/brolm/mistral3_config.h:38-58); defaults
    are Mistral-Small-3.1-24B."""
    vocab_size: int = 131072
    hidden_size: int = 5120
    intermediate_size: int = 32768
    num_hidden_layers: int = 40
    num_attention_heads: int = 32
    num_key_value_heads: int = 8
    head_dim: int = 128
    rms_norm_eps: float = 1e-5
    rope_theta: float = 1.0e9
    tie_word_embeddings: bool = False
    max_position_embeddings: int = 131072
    has_sliding_window: bool = False
    sliding_window: int = 0

    _INT = ("vocab_size", "hidden_size", "intermediate_size", "num_hidden_layers", "num_attention_heads",
            "num_key_value_heads", "head_dim", "max_position_embeddings", "sliding_window")

    def _c(self) -> _native.Mistral3TextConfigC:
        c = _native.Mistral3TextConfigC()
        for f in self._INT:
            setattr(c, f, int(getattr(self, f)))
        c.rms_norm_eps = float(self.rms_norm_eps)
        c.rope_theta = float(self.rope_theta)
        c.tie_word_embeddings = 1 if self.tie_word_embeddings else 0
        c.has_sliding_window = 1 if self.has_sliding_window else 0
        return c

    @classmethod
    def _from_c(cls, c: _native.Mistral3TextConfigC) -> "Mistral3TextConfig":
        out = cls(**{f: getattr(c, f) for f in cls._INT})
        out.rms_norm_eps, out.rope_theta = c.rms_norm_eps, c.rope_theta
        out.tie_word_embeddings = bool(c.tie_word_embeddings)
        out.has_sliding_window = bool(c.has_sliding_window)
        return out


@dataclass
class Mistral3Config:
    """Mistral3Config (include/brolm/mistral3_config.h:30-143): the text
    section and the multimodal glue (no Pixtral vision section here)."""
    text: Mistral3TextConfig = field(default_factory=Mistral3TextConfig)
    image_token_index: int = 10
    spatial_merge_size: int = 2
    multimodal_projector_bias: bool = False

    @classmethod
    def _from_c(cls, c: _native.Mistral3ConfigC) -> "Mistral3Config":
        return cls(Mistral3TextConfig._from_c(c.text), c.image_token_index, c.spatial_merge_size,
                   bool(c.multimodal_projector_bias))

    @classmethod
    def from_gguf(cls, path: str) -> "Mistral3Config":
        c = _native.Mistral3ConfigC()
        check(_native.lib().brolm_mistral3_config_from_gguf(str(path).encode(), C.byref(c)), "from_gguf")
        return cls._from_c(c)

    @classmethod
    def from_json_text(cls, text: str) -> "Mistral3Config":
        c = _native.Mistral3ConfigC()
        check(_native.lib().brolm_mistral3_config_from_json(text.encode(), C.byref(c)), "from_json_text")
        return cls._from_c(c)

    @classmethod
    def load(cls, path: str) -> "Mistral3Config":
        with open(path, encoding="utf-8") as f:
            return cls.from_json_text(f.read())


def mistral3_hf_to_ggml(hf_name: str) -> str:
    buf = C.create_string_buffer(256)
    n = _native.lib().brolm_mistral3_hf_to_ggml(hf_name.encode(), buf, 256)
    return buf.value.decode() if n > 0 else ""


class Mistral3TextModel(Qwen3Model):
    """mistral3::TextModel (include/brolm/mistral3_text.h:52-131): the dense
    decoder without QK-norm, untied lm_head; same forward / cache / decode
    surface as Qwen3Model (one shared decoder handle type)."""

    def __init__(self, cfg: Mistral3TextConfig):
        self.cfg = cfg
        self._h = _native.lib().brolm_mistral3_text_create(C.byref(cfg._c()))
        if not self._h:
            raise _native.NativeError(_native.lib().brolm_last_error().decode())


@dataclass
class Llm2VecConfig:
    """llm2vec::Config (include/brolm/llm2vec.h:41-63); defaults are
    Meta-Llama-3-8B-Instruct."""
    vocab_size: int = 128256
    hidden_size: int = 4096
    intermediate_size: int = 14336
    num_hidden_layers: int = 32
    num_attention_heads: int = 32
    num_key_value_heads: int = 8
    head_dim: int = 128
    rms_norm_eps: float = 1e-5
    rope_theta: float = 5.0e5

    def _c(self) -> _native.Llm2VecConfigC:
        c = _native.Llm2VecConfigC()
        for f in ("vocab_size", "hidden_size", "intermediate_size", "num_hidden_layers", "num_attention_heads",
                  "num_key_value_heads", "head_dim"):
            setattr(c, f, int(getattr(self, f)))
        c.rms_norm_eps, c.rope_theta = float(self.rms_norm_eps), float(self.rope_theta)
        return c

    @classmethod
    def from_json_text(cls, text: str) -> "Llm2VecConfig":
        c = _native.Llm2VecConfigC()
        check(_native.lib().brolm_llm2vec_config_from_json(text.encode(), C.byref(c)), "from_json_text")
        return cls(c.vocab_size, c.hidden_size, c.intermediate_size, c.num_hidden_layers, c.num_attention_heads,
                   c.num_key_value_heads, c.head_dim, c.rms_norm_eps, c.rope_theta)

    @classmethod
    def load(cls, path: str) -> "Llm2VecConfig":
        with open(path, encoding="utf-8") as f:
            return cls.from_json_text(f.read())


class Llm2VecEncoder(Qwen3Model):
    """llm2vec::Encoder (include/brolm/llm2vec.h:65-114) over GGUF weights."""

    def __init__(self, cfg: Llm2VecConfig):
        self.cfg = cfg
        self._h = _native.lib().brolm_llm2vec_create(C.byref(cfg._c()))
        if not self._h:
            raise _native.NativeError(_native.lib().brolm_last_error().decode())

    def encode(self, ids: Sequence[int]) -> np.ndarray:
        return self.forward_encode(ids)

    def encode_pooled(self, ids: Sequence[int], pool_mask=None) -> np.ndarray:
        arr, p = _i32(ids)
        out = np.empty((self.cfg.hidden_size,), np.float32)
        m = None
        if pool_mask is not None:
            mk = np.ascontiguousarray(np.asarray(pool_mask, np.float32))
            if mk.shape != (len(ids),):
                raise ValueError("pool_mask must hold one value per token")
            m = mk.ctypes.data_as(_native.P_f32)
        check(_native.lib().brolm_llm2vec_encode_pooled(self._h, p, len(ids), m, out.ctypes.data_as(_native.P_f32)),
              "encode_pooled")
        return out


@dataclass
class SamplingParams:
    """SamplingParams (include/brolm/detail/generate.h:29-34)."""
    temperature: float = 1.0
    top_k: int = 0
    top_p: float = 1.0
    seed: int = 0


@dataclass
class GenerateOptions:
    """GenerateOptions (include/brolm/detail/generate.h:57-61)."""
    max_new_tokens: int = 64
    sampling: SamplingParams = field(default_factory=SamplingParams)
    stop_on_eos: bool = True
    device_greedy: bool = True
    device_sampling: bool = True


def generate(model: Qwen3Model, prompt_ids: Sequence[int], eos_id: int, opts: GenerateOptions) -> list[int]:
    """qwen::generate (include/brolm/qwen_generate.h:45-47): only the new ids."""
    arr, p = _i32(list(prompt_ids) if len(prompt_ids) else [0])
    n_prompt = len(prompt_ids)
    out = np.empty((max(opts.max_new_tokens, 1),), np.int32)
    s = opts.sampling
    k = check(_native.lib().brolm_qwen3_generate(model._h, p, n_prompt, int(opts.max_new_tokens), int(eos_id),
                                                 1 if opts.stop_on_eos else 0, float(s.temperature), int(s.top_k),
                                                 float(s.top_p), int(s.seed), 1 if opts.device_greedy else 0,
                                                 1 if opts.device_sampling else 0, out.ctypes.data_as(_native.P_i32)),
              "generate")
    return out[:k].tolist()


class Tokenizer:
    """qwen::Tokenizer (include/brolm/qwen_tokenizer.h): byte-level BPE, the
    reference's token ids (reference include/brolm/qwen_tokenizer.h:41-151)."""

    def __init__(self, handle):
        if not handle:
            raise _native.NativeError(f"tokenizer: {_native.lib().brolm_last_error().decode()}")
        self._h = handle

    @staticmethod
    def _extra(extra) -> bytes | None:
        return "\n".join(extra).encode() if extra else None

    @classmethod
    def load(cls, vocab_json: str, merges_txt: str, extra_special_tokens=()) -> "Tokenizer":
        return cls(_native.lib().brolm_tokenizer_load(str(vocab_json).encode(), str(merges_txt).encode(),
                                                     cls._extra(extra_special_tokens)))

    @classmethod
    def from_gguf(cls, path: str, extra_special_tokens=()) -> "Tokenizer":
        return cls(_native.lib().brolm_tokenizer_from_gguf(str(path).encode(), cls._extra(extra_special_tokens)))

    @classmethod
    def from_tokenizer_json(cls, path: str, extra_special_tokens=()) -> "Tokenizer":
        return cls(_native.lib().brolm_tokenizer_from_json(str(path).encode(), cls._extra(extra_special_tokens)))

    def close(self) -> None:
        if getattr(self, "_h", None) and _native._lib is not None:
            _native.lib().brolm_tokenizer_free(self._h)
        self._h = None

    def __del__(self):
        self.close()

    def encode(self, text: str, add_special: bool = False) -> list[int]:
        b = text.encode() if isinstance(text, str) else bytes(text)
        n = check(_native.lib().brolm_tokenizer_encode(self._h, b, len(b), 1 if add_special else 0, None, 0),
                  "tokenizer encode")
        out = np.empty((max(n, 1),), np.int32)
        check(_native.lib().brolm_tokenizer_encode(self._h, b, len(b), 1 if add_special else 0,
                                                   out.ctypes.data_as(_native.P_i32), n), "tokenizer encode")
        return out[:n].tolist()

    def decode_bytes(self, ids: Sequence[int]) -> bytes:
        arr, p = _i32(list(ids) if len(ids) else [0])
        n = check(_native.lib().brolm_tokenizer_decode(self._h, p, len(ids), None, 0), "tokenizer decode")
        buf = C.create_string_buffer(max(n, 1))
        check(_native.lib().brolm_tokenizer_decode(self._h, p, len(ids), buf, n), "tokenizer decode")
        return buf.raw[:n]

    def decode(self, ids: Sequence[int]) -> str:
        return self.decode_bytes(ids).decode("utf-8", errors="replace")

    def apply_chat_template(self, messages, add_generation_prompt: bool = True) -> str:
        roles = (C.c_char_p * max(len(messages), 1))(*[r.encode() for r, _ in messages])
        conts = (C.c_char_p * max(len(messages), 1))(*[c.encode() for _, c in messages])
        args = (self._h, roles, conts, len(messages), 1 if add_generation_prompt else 0)
        n = check(_native.lib().brolm_tokenizer_chat(*args, None, 0), "chat template")
        buf = C.create_string_buffer(max(n, 1))
        check(_native.lib().brolm_tokenizer_chat(*args, buf, n), "chat template")
        return buf.raw[:n].decode()

    def register_special_token(self, token: str, id_: int) -> None:
        check(_native.lib().brolm_tokenizer_register_special(self._h, token.encode(), int(id_)), "register special")

    def _info(self) -> list[int]:
        a = np.zeros(6, np.int64)
        check(_native.lib().brolm_tokenizer_info(self._h, a.ctypes.data_as(_native.P_i64)), "tokenizer info")
        return a.tolist()

    def vocab_count(self) -> int:
        return self._info()[0]

    def merge_count(self) -> int:
        return self._info()[1]

    def eos_id(self) -> int:
        return self._info()[2]

    def im_start_id(self) -> int:
        return self._info()[3]

    def im_end_id(self) -> int:
        return self._info()[4]

    def endoftext_id(self) -> int:
        return self._info()[5]


def generate_text(model: Qwen3Model, tok: Tokenizer, prompt: str, opts: GenerateOptions) -> str:
    """qwen::generate_text (reference src/qwen_generate.cpp:19-25)."""
    s = opts.sampling
    args = (model._h, tok._h, prompt.encode(), int(opts.max_new_tokens), 1 if opts.stop_on_eos else 0,
            float(s.temperature), int(s.top_k), float(s.top_p), int(s.seed))
    cap = 64 * max(int(opts.max_new_tokens), 1) + 4096   # one generation fills it; longer text re-runs
    while True:
        buf = C.create_string_buffer(cap)
        n = check(_native.lib().brolm_qwen3_generate_text(*args, buf, cap), "generate_text")
        if n <= cap:
            return buf.raw[:n].decode("utf-8", errors="replace")
        cap = n


def sample_token(logits: np.ndarray, params: SamplingParams, seed: int) -> int:
    """sample_token with a fresh std::mt19937_64(seed) (src/detail/generate.cpp:68-142)."""
    a = np.ascontiguousarray(logits, dtype=np.float32)
    return _native.lib().brolm_sample_token(a.ctypes.data_as(_native.P_f32), a.size, float(params.temperature),
                                            int(params.top_k), float(params.top_p), int(seed))


PROFILE_STAGES = ("embed", "idx_upload", "rms_norm", "qkv_proj", "qk_norm", "rope", "kv_append", "attention",
                  "o_proj", "mlp_proj", "swiglu", "residual_add", "final_norm", "lm_head", "logits_download",
                  "sample", "other")


def profile_stages() -> dict:
    """BROLM_PROFILE totals: {stage: (device ns, calls)} for every stage with
    calls (include/brolm/detail/profile.h:19-38 order)."""
    out = {}
    for i, name in enumerate(PROFILE_STAGES):
        ns, calls = C.c_uint64(), C.c_uint64()
        if _native.lib().brolm_profile_stage(i, C.byref(ns), C.byref(calls)) != 0:
            raise RuntimeError(f"brolm_profile_stage({i}) failed")
        if calls.value:
            out[name] = (ns.value, calls.value)
    return out


def profile_reset() -> None:
    _native.lib().brolm_profile_reset()


def profile_report() -> None:
    _native.lib().brolm_profile_report()


def prompt_ids(n: int, vocab: int, seed: int = 42) -> list[int]:
    """bench_decode's synthetic prompt: std::mt19937_64(seed)() % vocab (tools/bench_decode.cpp:208-213)."""
    out = np.empty((max(n, 1),), np.int32)
    check(_native.lib().brolm_prompt_ids(int(seed), int(n), int(vocab), out.ctypes.data_as(_native.P_i32)),
          "prompt_ids")
    return out[:n].tolist()


@dataclass
class SynthSpec:
    """Synthetic Qwen3 checkpoint (include/brolm/synth.h)."""
    vocab: int = 151936
    hidden: int = 1024
    intermediate: int = 3072
    layers: int = 28
    n_q: int = 16
    n_kv: int = 8
    head_dim: int = 128
    eps: float = 1e-6
    theta: float = 1000000.0
    context: int = 40960
    tied: bool = True
    embed: str = "Q8_0"
    q: str = "Q8_0"
    k: str = "Q8_0"
    v: str = "Q8_0"
    o: str = "Q8_0"
    gate: str = "Q8_0"
    up: str = "Q8_0"
    down: str = "Q8_0"
    output: str = "Q6_K"
    stddev: float = 0.02
    seed: int = 0
    # type of attn_v / ffn_down on llama.cpp's use_more_bits layers ("" none):
    # "Q6_K" over a Q4_K base gives a Q4_K_M-style per-layer mix
    more_bits: str = ""


def _synth_c(spec: SynthSpec) -> _native.SynthSpecC:
    s = _native.SynthSpecC()
    for f in ("vocab", "hidden", "intermediate", "layers", "n_q", "n_kv", "head_dim", "context"):
        setattr(s, f, int(getattr(spec, f)))
    s.eps, s.theta, s.stddev = float(spec.eps), float(spec.theta), float(spec.stddev)
    s.tied = 1 if spec.tied else 0
    for f in ("embed", "q", "k", "v", "o", "gate", "up", "down", "output"):
        setattr(s, f + "_type", GGML[getattr(spec, f)])
    s.seed = int(spec.seed)
    s.more_bits_type = GGML[spec.more_bits] if spec.more_bits else -1
    return s


def write_synth_qwen3(spec: SynthSpec, path: str) -> None:
    check(_native.lib().brolm_synth_qwen3_write(C.byref(_synth_c(spec)), str(path).encode()), "write_synth_qwen3")


def write_synth_mistral3(spec: SynthSpec, path: str) -> None:
    """Mistral 3.1 text checkpoint: the same tensors under general.architecture
    "llama", without per-head QK-norm gammas; untied when spec.tied is False."""
    check(_native.lib().brolm_synth_mistral3_write(C.byref(_synth_c(spec)), str(path).encode()),
          "write_synth_mistral3")
