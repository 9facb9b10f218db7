"""Whole-model pins of the oracle: HF transformers' Qwen3 in float64 on the
same dequantized weights, the committed greedy fixture, and the reference's
own model invariants (tests/test_qwen.cpp, tests/test_qwen_generate.cpp)."""
from __future__ import annotations

import numpy as np
import pytest

import oracle
from conftest import SMALL


def _dequant(g: oracle.Gguf, name: str) -> np.ndarray:
    t, dims, raw = g.tensor(name)
    return oracle.dequant(t, raw, int(np.prod(dims))).reshape(list(reversed(dims)))


def test_oracle_matches_hf_qwen3_float64(small_gguf):
    """transformers' Qwen3ForCausalLM (rotate_half RoPE on unpermuted q/k rows,
    its own RMSNorm, GQA attention and SwiGLU) in float64 on the oracle's
    dequantized weights.  Pins the load-time rope permute, the op order of
    dense_decoder.cpp:526-681 and every FP32 op of the oracle at once."""
    torch = pytest.importorskip("torch")
    tr = pytest.importorskip("transformers")
    g = oracle.Gguf(str(small_gguf))
    s = SMALL
    cfg = tr.Qwen3Config(vocab_size=s["vocab"], hidden_size=s["hidden"], intermediate_size=s["intermediate"],
                         num_hidden_layers=s["layers"], num_attention_heads=s["n_q"], num_key_value_heads=s["n_kv"],
                         head_dim=s["head_dim"], rms_norm_eps=1e-6, rope_theta=1e6, tie_word_embeddings=False,
                         max_position_embeddings=4096, attention_bias=False)
    torch.manual_seed(0)
    hf = tr.Qwen3ForCausalLM(cfg).double().eval()
    sd = {"model.embed_tokens.weight": _dequant(g, "token_embd.weight"),
          "model.norm.weight": _dequant(g, "output_norm.weight").reshape(-1),
          "lm_head.weight": _dequant(g, "output.weight")}
    names = {"self_attn.q_proj": "attn_q", "self_attn.k_proj": "attn_k", "self_attn.v_proj": "attn_v",
             "self_attn.o_proj": "attn_output", "self_attn.q_norm": "attn_q_norm", "self_attn.k_norm": "attn_k_norm",
             "input_layernorm": "attn_norm", "post_attention_layernorm": "ffn_norm", "mlp.gate_proj": "ffn_gate",
             "mlp.up_proj": "ffn_up", "mlp.down_proj": "ffn_down"}
    for l in range(s["layers"]):
        for hfn, ggn in names.items():
            w = _dequant(g, f"blk.{l}.{ggn}.weight")
            sd[f"model.layers.{l}.{hfn}.weight"] = w.reshape(-1) if w.ndim == 1 or min(w.shape) == 1 else w
    for k in list(sd):
        if "norm" in k:
            sd[k] = sd[k].reshape(-1)
    res = hf.load_state_dict({k: torch.tensor(v, dtype=torch.float64) for k, v in sd.items()}, strict=False)
    assert not res.unexpected_keys and all("rotary" in k for k in res.missing_keys)
    ids = [1, 2, 3, 4, 900, 17, 512, 999]
    with torch.no_grad():
        want = hf(torch.tensor([ids])).logits[0].numpy()
    m = oracle.Model(str(small_gguf))
    m.allocate_cache(16)
    got = m.forward(ids)
    assert np.abs(got - want).max() < 5e-5 * max(1.0, np.abs(want).max())


def test_oracle_golden_greedy(small_gguf):
    from golden import load_model_small
    fx = load_model_small()
    m = oracle.Model(str(small_gguf))
    toks, margins = m.generate_greedy(fx["prompt"].tolist(), len(fx["tokens"]))
    assert toks == fx["tokens"].tolist()
    np.testing.assert_allclose(margins, fx["margins"], atol=1e-5)
    m2 = oracle.Model(str(small_gguf))
    m2.allocate_cache(64)
    np.testing.assert_allclose(m2.forward(fx["prompt"].tolist(), last_only=True)[0], fx["last_logits"], atol=1e-5)


def test_oracle_prefill_equals_streamed_decode(small_gguf):
    """tests/test_qwen.cpp:214-248: logits of a one-shot prefill equal the
    logits of feeding the same ids one by one through the KV cache (rel 1e-4)."""
    ids = [11, 250, 3, 999, 42, 7, 600]
    m = oracle.Model(str(small_gguf))
    m.allocate_cache(16)
    full = m.forward(ids)
    m.reset_cache()
    step = np.stack([m.forward([t])[0] for t in ids])
    rel = np.abs(full - step) / np.maximum(1e-4, np.abs(full))
    assert rel.max() < 1e-4


def test_oracle_truncate_replays_identically(small_gguf):
    """tests/test_qwen.cpp:285-338: truncating the cache back to an anchor and
    re-feeding gives the same logits bitwise."""
    m = oracle.Model(str(small_gguf))
    m.allocate_cache(32)
    m.forward([1, 2, 3, 4, 5])
    a = m.forward([9, 8, 7])
    m.truncate_cache(5)
    assert m.cache_len() == 5
    b = m.forward([9, 8, 7])
    assert np.array_equal(a, b)


def test_oracle_teacher_forced_argmax_equals_greedy(small_gguf):
    """tests/test_qwen_generate.cpp:282-323."""
    prompt = [5, 17, 2, 31]
    toks, _ = oracle.Model(str(small_gguf)).generate_greedy(prompt, 10)
    m = oracle.Model(str(small_gguf))
    m.allocate_cache(32)
    lg = m.forward(prompt + toks[:-1])
    assert [oracle.argmax(lg[len(prompt) - 1 + k])[0] for k in range(len(toks))] == toks
