"""LLM2Vec encoder on the CPU: config parsing (tests/test_llm2vec.cpp:253-267)
and the oracle's bidirectional, cacheless pass (DenseDecoder::forward_encode,
src/detail/dense_decoder.cpp:296-309, :682-779) pinned by transformers'
Mistral and Qwen3 models in float64 with a full (all-visible) attention mask."""
from __future__ import annotations

import numpy as np
import pytest

import oracle
from conftest import SMALL, SMALL_M3


@pytest.fixture(scope="module")
def ba():
    import brolm_amd
    return brolm_amd


def test_config_known_answers(ba):
    c = ba.Llm2VecConfig.from_json_text(
        '{"vocab_size":128256,"hidden_size":4096,"intermediate_size":14336,"num_hidden_layers":32,'
        '"num_attention_heads":32,"num_key_value_heads":8,"rms_norm_eps":1e-05,"rope_theta":500000.0}')
    assert (c.vocab_size, c.hidden_size, c.num_key_value_heads, c.head_dim) == (128256, 4096, 8, 128)
    assert c.rope_theta == pytest.approx(5e5) and c.rms_norm_eps == pytest.approx(1e-5)
    assert ba.Llm2VecConfig.from_json_text('{"hidden_size":256,"num_attention_heads":2,"num_key_value_heads":2,"head_dim":96}').head_dim == 96
    for bad in ('{"num_attention_heads":32,"num_key_value_heads":7}', '{"head_dim":7}', '[]', '{'):
        with pytest.raises(Exception):
            ba.Llm2VecConfig.from_json_text(bad)


def _dequant(g, name):
    t, dims, raw = g.tensor(name)
    return oracle.dequant(t, raw, int(np.prod(dims))).reshape(list(reversed(dims)))


def _hf_state(g, layers, qk_norm):
    names = {"self_attn.q_proj": "attn_q", "self_attn.k_proj": "attn_k", "self_attn.v_proj": "attn_v",
             "self_attn.o_proj": "attn_output", "input_layernorm": "attn_norm",
             "post_attention_layernorm": "ffn_norm", "mlp.gate_proj": "ffn_gate", "mlp.up_proj": "ffn_up",
             "mlp.down_proj": "ffn_down"}
    if qk_norm:
        names.update({"self_attn.q_norm": "attn_q_norm", "self_attn.k_norm": "attn_k_norm"})
    sd = {"model.embed_tokens.weight": _dequant(g, "token_embd.weight"),
          "model.norm.weight": _dequant(g, "output_norm.weight").reshape(-1)}
    for l in range(layers):
        for hfn, ggn in names.items():
            w = _dequant(g, f"blk.{l}.{ggn}.weight")
            sd[f"model.layers.{l}.{hfn}.weight"] = w.reshape(-1) if "norm" in hfn else w
    return sd


@pytest.mark.parametrize("arch", ["mistral3", "qwen3"])
def test_oracle_encode_matches_hf_bidirectional_float64(arch, small_m3_gguf, small_gguf):
    """transformers' decoder stack (MistralModel / Qwen3Model) in float64 on
    the oracle's dequantized weights, fed a 4-D additive attention mask of
    zeros (every query sees every key): the post-final-norm hidden states."""
    torch = pytest.importorskip("torch")
    tr = pytest.importorskip("transformers")
    path, s = (small_m3_gguf, SMALL_M3) if arch == "mistral3" else (small_gguf, SMALL)
    eps, theta = (1e-5, 1e9) if arch == "mistral3" else (1e-6, 1e6)
    kw = dict(vocab_size=s["vocab"], hidden_size=s["hidden"], intermediate_size=s["intermediate"],
              num_hidden_layers=s["layers"], num_attention_heads=s["n_q"], num_key_value_heads=s["n_kv"],
              head_dim=s["head_dim"], rms_norm_eps=eps, rope_theta=theta, max_position_embeddings=4096)
    if arch == "mistral3":
        cfg, cls = tr.MistralConfig(sliding_window=None, **kw), tr.MistralModel
    else:
        cfg, cls = tr.Qwen3Config(**kw), tr.Qwen3Model
    cfg._attn_implementation = "eager"
    torch.manual_seed(0)
    hf = cls(cfg).double().eval()
    g = oracle.Gguf(str(path))
    sd = {k.removeprefix("model."): torch.tensor(v, dtype=torch.float64)
          for k, v in _hf_state(g, s["layers"], arch == "qwen3").items()}
    res = hf.load_state_dict(sd, strict=False)
    assert not res.unexpected_keys and all("rotary" in k for k in res.missing_keys)
    ids = [1, 2, 3, 4, 900, 17, 512, 999, 0]
    L = len(ids)
    full = torch.zeros((1, 1, L, L), dtype=torch.float64)
    with torch.no_grad():
        want = hf(input_ids=torch.tensor([ids]), attention_mask=full).last_hidden_state[0].numpy()
        causal = hf(input_ids=torch.tensor([ids])).last_hidden_state[0].numpy()
    m = oracle.Model(str(path))
    got = m.forward_encode(ids)
    tol = 5e-5 * max(1.0, np.abs(want).max())
    assert np.abs(got - want).max() < tol
    # the pin sees the mask: the causal stack differs on every row but the last
    assert np.abs(causal[0] - want[0]).max() > 100 * tol
    # and the oracle's causal forward agrees with HF's causal run
    m.allocate_cache(16)
    _, hid = m.forward(ids, want_hidden=True)
    assert np.abs(hid - causal).max() < tol
