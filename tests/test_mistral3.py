"""Mistral 3.1 text decoder on the CPU: config parsing (the reference's
known answers, tests/test_mistral3_config.cpp), GGUF config and tensor-name
map (src/mistral3_config.cpp:130-191, src/mistral3_text.cpp:70-108), and the
oracle's no-QK-norm decoder pinned by transformers' MistralForCausalLM in
float64."""
from __future__ import annotations

import json
from pathlib import Path

import numpy as np
import pytest

import oracle
from conftest import SMALL_M3
from gguf_meta import read_metadata

GOLDEN = Path(__file__).parent / "golden"


@pytest.fixture(scope="module")
def ba():
    import brolm_amd
    return brolm_amd


def test_hf_to_ggml_is_qwen3_map_without_qk_norm(ba):
    tails = ["self_attn.q_proj.weight", "self_attn.k_proj.weight", "self_attn.v_proj.weight",
             "self_attn.o_proj.weight", "input_layernorm.weight", "post_attention_layernorm.weight",
             "mlp.gate_proj.weight", "mlp.up_proj.weight", "mlp.down_proj.weight"]
    for layer in (0, 7, 39):
        for t in tails:
            hf = f"model.layers.{layer}.{t}"
            assert ba.mistral3_hf_to_ggml(hf) == ba.qwen3_hf_to_ggml(hf) != ""
        for t in ("self_attn.q_norm.weight", "self_attn.k_norm.weight"):
            assert ba.qwen3_hf_to_ggml(f"model.layers.{layer}.{t}") != ""
            assert ba.mistral3_hf_to_ggml(f"model.layers.{layer}.{t}") == ""
    assert ba.mistral3_hf_to_ggml("model.layers.12.mlp.down_proj.weight") == "blk.12.ffn_down.weight"
    assert ba.mistral3_hf_to_ggml("model.embed_tokens.weight") == "token_embd.weight"
    assert ba.mistral3_hf_to_ggml("model.norm.weight") == "output_norm.weight"
    assert ba.mistral3_hf_to_ggml("lm_head.weight") == "output.weight"
    for bad in ("", "model.layers.x.mlp.up_proj.weight", "model.layers.3", "language_model.lm_head.weight",
                "model.layers.3.mlp.up_proj.bias", "vision_tower.patch_conv.weight"):
        assert ba.mistral3_hf_to_ggml(bad) == ""


def test_config_real_json_known_answers(ba):
    """tests/test_mistral3_config.cpp:76-100 on the verbatim
    Mistral-Small-3.1-24B-Instruct-2503 config.json it embeds."""
    cfg = ba.Mistral3Config.load(str(GOLDEN / "mistral3_small_3_1_config.json"))
    assert (cfg.image_token_index, cfg.spatial_merge_size, cfg.multimodal_projector_bias) == (10, 2, False)
    t = cfg.text
    assert (t.vocab_size, t.hidden_size, t.intermediate_size, t.num_hidden_layers) == (131072, 5120, 32768, 40)
    assert (t.num_attention_heads, t.num_key_value_heads, t.head_dim) == (32, 8, 128)
    assert t.rms_norm_eps == pytest.approx(1e-5, rel=1e-6) and t.rope_theta == pytest.approx(1e9, rel=1e-6)
    assert t.max_position_embeddings == 131072
    assert t.tie_word_embeddings is False and t.has_sliding_window is False


def test_config_json_window_and_errors(ba):
    """tests/test_mistral3_config.cpp:117-154."""
    w = ba.Mistral3Config.from_json_text('{"text_config": {"sliding_window": 4096}, "vision_config": {}}')
    assert w.text.has_sliding_window and w.text.sliding_window == 4096
    for bad in ('{"vision_config": {}}',
                '{"text_config": {"num_attention_heads": 32, "num_key_value_heads": 7}, "vision_config": {}}',
                '{"text_config": {"head_dim": 127}, "vision_config": {}}',
                '{"text_config": {}}', '[1, 2]', '{"text_config": {'):
        with pytest.raises(Exception):
            ba.Mistral3Config.from_json_text(bad)


def test_config_from_gguf(ba, small_m3_gguf):
    """Arch-prefixed keys, head_dim from key_length (128, not hidden / heads),
    vocab from the token list, untied because output.weight is present; the
    file itself read back by the test-side GGUF reader."""
    meta = read_metadata(str(small_m3_gguf))
    assert meta["general.architecture"] == "llama"
    assert meta["llama.attention.key_length"] == 128 != meta["llama.embedding_length"] // meta[
        "llama.attention.head_count"]
    names = set(oracle.Gguf(str(small_m3_gguf)).tensor_names())
    assert "output.weight" in names and not any("q_norm" in n or "k_norm" in n for n in names)
    t = ba.Mistral3Config.from_gguf(str(small_m3_gguf)).text
    s = SMALL_M3
    assert (t.vocab_size, t.hidden_size, t.intermediate_size, t.num_hidden_layers) == (
        len(meta["tokenizer.ggml.tokens"]), s["hidden"], s["intermediate"], s["layers"])
    assert (t.num_attention_heads, t.num_key_value_heads, t.head_dim) == (s["n_q"], s["n_kv"], s["head_dim"])
    assert t.rms_norm_eps == pytest.approx(1e-5) and t.rope_theta == pytest.approx(1e9)
    assert t.max_position_embeddings == s["context"] and t.tie_word_embeddings is False
    # the Qwen3 loader refuses the architecture
    with pytest.raises(Exception):
        ba.Qwen3Config.from_gguf(str(small_m3_gguf))


def _dequant(g: oracle.Gguf, name: str) -> np.ndarray:
    t, dims, raw = g.tensor(name)
    return oracle.dequant(t, raw, int(np.prod(dims))).reshape(list(reversed(dims)))


def test_oracle_matches_hf_mistral_float64(small_m3_gguf):
    """transformers' MistralForCausalLM (no QK-norm, rotate_half RoPE on
    unpermuted rows, theta 1e9, head_dim 128 != hidden / heads, GQA 4:1) in
    float64 on the oracle's dequantized weights."""
    torch = pytest.importorskip("torch")
    tr = pytest.importorskip("transformers")
    g = oracle.Gguf(str(small_m3_gguf))
    s = SMALL_M3
    cfg = tr.MistralConfig(vocab_size=s["vocab"], hidden_size=s["hidden"], intermediate_size=s["intermediate"],
                           num_hidden_layers=s["layers"], num_attention_heads=s["n_q"],
                           num_key_value_heads=s["n_kv"], head_dim=s["head_dim"], rms_norm_eps=1e-5,
                           rope_theta=1e9, tie_word_embeddings=False, max_position_embeddings=4096,
                           sliding_window=None)
    torch.manual_seed(0)
    hf = tr.MistralForCausalLM(cfg).double().eval()
    sd = {"model.embed_tokens.weight": _dequant(g, "token_embd.weight"),
          "model.norm.weight": _dequant(g, "output_norm.weight").reshape(-1),
          "lm_head.weight": _dequant(g, "output.weight")}
    names = {"self_attn.q_proj": "attn_q", "self_attn.k_proj": "attn_k", "self_attn.v_proj": "attn_v",
             "self_attn.o_proj": "attn_output", "input_layernorm": "attn_norm",
             "post_attention_layernorm": "ffn_norm", "mlp.gate_proj": "ffn_gate", "mlp.up_proj": "ffn_up",
             "mlp.down_proj": "ffn_down"}
    for l in range(s["layers"]):
        for hfn, ggn in names.items():
            w = _dequant(g, f"blk.{l}.{ggn}.weight")
            sd[f"model.layers.{l}.{hfn}.weight"] = w.reshape(-1) if "norm" in hfn else w
    res = hf.load_state_dict({k: torch.tensor(v, dtype=torch.float64) for k, v in sd.items()}, strict=False)
    assert not res.unexpected_keys and all("rotary" in k for k in res.missing_keys)
    ids = [1, 2, 3, 4, 900, 17, 512, 999, 0, 33]
    with torch.no_grad():
        want = hf(torch.tensor([ids])).logits[0].numpy()
    m = oracle.Model(str(small_m3_gguf))
    assert m.cfg.use_qk_norm == 0 and m.cfg.tie_word_embeddings == 0
    m.allocate_cache(16)
    got = m.forward(ids)
    assert np.abs(got - want).max() < 5e-5 * max(1.0, np.abs(want).max())
    # the pin sees QK-norm: the same weights through Qwen3 (unit gammas) differ
    cfg_q = tr.Qwen3Config(vocab_size=s["vocab"], hidden_size=s["hidden"], intermediate_size=s["intermediate"],
                           num_hidden_layers=s["layers"], num_attention_heads=s["n_q"],
                           num_key_value_heads=s["n_kv"], head_dim=s["head_dim"], rms_norm_eps=1e-5,
                           rope_theta=1e9, tie_word_embeddings=False, max_position_embeddings=4096)
    hq = tr.Qwen3ForCausalLM(cfg_q).double().eval()
    hq.load_state_dict({k: torch.tensor(v, dtype=torch.float64) for k, v in sd.items()}, strict=False)
    with torch.no_grad():
        other = hq(torch.tensor([ids])).logits[0].numpy()
    assert np.abs(other - want).max() > 100 * 5e-5 * max(1.0, np.abs(want).max())


def test_oracle_mistral_prefill_equals_streamed_decode(small_m3_gguf):
    """tests/test_mistral3_text.cpp:218-251: four 1-token steps reproduce the
    prefill's last row."""
    ids = [5, 17, 2, 31, 800, 64]
    m = oracle.Model(str(small_m3_gguf))
    m.allocate_cache(16)
    full = m.forward(ids)
    m.reset_cache()
    step = np.stack([m.forward([t], last_only=True)[0] for t in ids])
    assert np.abs(full - step).max() <= 1e-4 * max(1.0, np.abs(full).max())


def test_synth_mistral3_is_deterministic(ba, tmp_path):
    spec = ba.SynthSpec(**{**SMALL_M3, "layers": 1, "vocab": 300})
    a, b = tmp_path / "a.gguf", tmp_path / "b.gguf"
    ba.write_synth_mistral3(spec, str(a))
    ba.write_synth_mistral3(spec, str(b))
    assert a.read_bytes() == b.read_bytes()
    # the same spec as Qwen3 carries the two extra gammas per layer
    q = tmp_path / "q.gguf"
    ba.write_synth_qwen3(spec, str(q))
    nq = set(oracle.Gguf(str(q)).tensor_names())
    nm = set(oracle.Gguf(str(a)).tensor_names())
    assert nq - nm == {"blk.0.attn_q_norm.weight", "blk.0.attn_k_norm.weight"} and nm <= nq
    assert json.dumps(read_metadata(str(a))["general.architecture"]) == '"llama"'
