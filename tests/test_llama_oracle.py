"""The Llama decode-step oracle and the host RoPE tables, pinned against independent implementations (CPU).

The reference checks its decode against transformers' LlamaForCausalLM with the same weights (llama/run.py:186-198,
``reference``); the oracle is pinned the same way here, in float64 on a small model of the same architecture: every
decode step's logits must match transformers' incremental (KV-cached) forward pass. Its parts are checked against torch's
own routines (RMSNorm, scaled-dot-product attention) and against closed forms (RoPE at position 0 is the identity and
preserves each pair's norm; attention over one position returns that value row). The RoPE tables the product computes
must equal transformers' LlamaRotaryEmbedding bit for bit (the reference exports exactly those, llama/run.py:161-163).
"""
import dataclasses

import numpy as np
import pytest
import torch

from aq import synth
from aq.llama import LlamaConfig, rope_tables
from oracle import aq_oracle as orc

SMALL = LlamaConfig(dim=256, layers=2, heads=4, kv_heads=2, head_dim=64, ffn=512, vocab=300, max_pos=64)


def _hf_config(cfg: LlamaConfig):
    from transformers import LlamaConfig as HFConfig
    scaling = None
    if cfg.rope_orig:
        scaling = dict(rope_type="llama3", factor=cfg.rope_factor, low_freq_factor=cfg.rope_low,
                       high_freq_factor=cfg.rope_high, original_max_position_embeddings=cfg.rope_orig)
    return HFConfig(vocab_size=cfg.vocab, hidden_size=cfg.dim, intermediate_size=cfg.ffn,
                    num_hidden_layers=cfg.layers, num_attention_heads=cfg.heads, num_key_value_heads=cfg.kv_heads,
                    head_dim=cfg.head_dim, rms_norm_eps=cfg.eps, rope_theta=cfg.rope_theta,
                    max_position_embeddings=131072, rope_scaling=scaling, tie_word_embeddings=False,
                    hidden_act="silu", attention_bias=False, mlp_bias=False)


@pytest.mark.parametrize("cfg", [LlamaConfig(), dataclasses.replace(LlamaConfig(), rope_orig=0, rope_theta=10000.0)],
                         ids=["llama3-scaled", "unscaled"])
def test_rope_tables_match_transformers(cfg):
    from transformers.models.llama.modeling_llama import LlamaRotaryEmbedding
    rot = LlamaRotaryEmbedding(config=_hf_config(cfg))
    cos, sin = rot(torch.zeros(1, dtype=torch.float32), torch.arange(cfg.max_pos)[None])
    c, s = rope_tables(cfg)
    np.testing.assert_array_equal(c, cos[0, :, :cfg.head_dim // 2].numpy())
    np.testing.assert_array_equal(s, sin[0, :, :cfg.head_dim // 2].numpy())
    # rotate_half duplicates the angles over the two halves
    np.testing.assert_array_equal(cos[0, :, :32].numpy(), cos[0, :, 32:].numpy())


def test_rmsnorm_vs_torch():
    rng = np.random.default_rng(0)
    x = rng.standard_normal((3, 512))
    w = rng.standard_normal(512).astype(np.float16)
    ref = torch.nn.functional.rms_norm(torch.from_numpy(x), (512,), torch.from_numpy(w.astype(np.float64)), eps=1e-5)
    np.testing.assert_allclose(orc.rmsnorm(x, w, 1e-5), ref.numpy(), rtol=1e-13, atol=1e-13)


def test_rope_closed_forms():
    rng = np.random.default_rng(1)
    v = rng.standard_normal((5, 64))
    c, s = rope_tables(SMALL)
    np.testing.assert_array_equal(orc.rope(v, c[0], s[0]), v)  # angle 0
    r = orc.rope(v, c[17], s[17])
    np.testing.assert_allclose(r[:, :32] ** 2 + r[:, 32:] ** 2, v[:, :32] ** 2 + v[:, 32:] ** 2, rtol=1e-6)
    # rotate_half as a complex product: (a + ib) * (c + is)
    z = (v[:, :32] + 1j * v[:, 32:]) * (c[17].astype(np.float64) + 1j * s[17].astype(np.float64))
    np.testing.assert_allclose(r, np.concatenate([z.real, z.imag], axis=1), rtol=1e-12, atol=1e-12)


@pytest.mark.parametrize("heads,kv", [(4, 2), (8, 8), (8, 1)])
def test_attention_vs_sdpa(heads, kv):
    rng = np.random.default_rng(heads * 10 + kv)
    n, p = 37, 64
    q = rng.standard_normal((heads, 64))
    kc = rng.standard_normal((kv, p, 64))
    vc = rng.standard_normal((kv, p, 64))
    out = orc.attention_decode(q, kc, vc, n)
    k = torch.from_numpy(kc[:, :n]).repeat_interleave(heads // kv, dim=0)
    v = torch.from_numpy(vc[:, :n]).repeat_interleave(heads // kv, dim=0)
    ref = torch.nn.functional.scaled_dot_product_attention(torch.from_numpy(q)[:, None], k, v)[:, 0]
    np.testing.assert_allclose(out, ref.numpy(), rtol=1e-12, atol=1e-12)
    # one position: the output is that position's value row
    np.testing.assert_allclose(orc.attention_decode(q, kc, vc, 1), vc[np.arange(heads) // (heads // kv), 0],
                               rtol=1e-14)


def test_argmax_first_takes_the_first_maximum():
    assert orc.argmax_first(np.array([1.0, 3.0, 2.0, 3.0])) == 1
    assert orc.argmax_first(np.array([-1.0, -1.0])) == 0


def _hf_model(cfg, arrays):
    from transformers import LlamaForCausalLM
    torch.manual_seed(0)
    model = LlamaForCausalLM(_hf_config(cfg)).to(torch.float64).eval()
    deq = lambda n: torch.from_numpy(orc.q4w_dequant(arrays[n + ".q"], arrays[n + ".s"], cfg.group)  # noqa: E731
                                     .astype(np.float64))
    f64 = lambda a: torch.from_numpy(np.asarray(a).astype(np.float64))  # noqa: E731
    hq, hk = cfg.heads * cfg.head_dim, cfg.kv_heads * cfg.head_dim
    with torch.no_grad():
        model.model.embed_tokens.weight.copy_(f64(arrays["embed"]))
        for i, layer in enumerate(model.model.layers):
            p = f"l{i}."
            qkv = deq(p + "wqkv")
            layer.self_attn.q_proj.weight.copy_(qkv[:hq])
            layer.self_attn.k_proj.weight.copy_(qkv[hq:hq + hk])
            layer.self_attn.v_proj.weight.copy_(qkv[hq + hk:])
            layer.self_attn.o_proj.weight.copy_(deq(p + "wo"))
            gu = deq(p + "wgu")
            layer.mlp.gate_proj.weight.copy_(gu[:cfg.ffn])
            layer.mlp.up_proj.weight.copy_(gu[cfg.ffn:])
            layer.mlp.down_proj.weight.copy_(deq(p + "wdown"))
            layer.input_layernorm.weight.copy_(f64(arrays[p + "attn_norm"]))
            layer.post_attention_layernorm.weight.copy_(f64(arrays[p + "mlp_norm"]))
        model.model.norm.weight.copy_(f64(arrays["final_norm"]))
        model.lm_head.weight.copy_(deq("lm"))
    return model


def test_decode_oracle_matches_transformers():
    """Eight decode steps, token by token through transformers' KV cache, against the oracle with an unrounded cache.
    A dropped residual, a swapped rotate_half sign or a wrong KV-head mapping moves the logits by O(1)."""
    from transformers import DynamicCache
    cfg = SMALL
    arrays = synth.llama_arrays(cfg, seed=11)
    arrays["embed"] = (arrays["embed"].astype(np.float32) * 0.1).astype(np.float16)
    cos, sin = rope_tables(cfg)
    oracle = orc.LlamaDecodeOracle(arrays, cfg, cos, sin, kv_dtype=None)
    model = _hf_model(cfg, arrays)
    cache = DynamicCache()
    tokens = [5, 17, 299, 0, 42, 42, 100, 7]
    with torch.no_grad():
        for pos, tok in enumerate(tokens):
            out = model(torch.tensor([[tok]]), past_key_values=cache, use_cache=True,
                        position_ids=torch.tensor([[pos]]))
            cache = out.past_key_values
            ref = out.logits[0, -1].numpy()
            got = oracle.step(tok, pos)
            # transformers' RMSNorm computes in float32 even in a float64 model: agreement to ~1e-7 of the range
            np.testing.assert_allclose(got, ref, rtol=0, atol=2e-6 * np.abs(ref).max())
            assert orc.argmax_first(got) == int(np.argmax(ref))


def test_fp16_cache_rounding_is_small():
    """The fp16 cache (what the build stores) changes the logits only slightly against the float64 cache."""
    cfg = SMALL
    arrays = synth.llama_arrays(cfg, seed=12)
    cos, sin = rope_tables(cfg)
    a = orc.LlamaDecodeOracle(arrays, cfg, cos, sin, kv_dtype=None)
    b = orc.LlamaDecodeOracle(arrays, cfg, cos, sin, kv_dtype=np.float16)
    for pos, tok in enumerate([3, 1, 4, 1, 5]):
        la, lb = a.step(tok, pos), b.step(tok, pos)
        assert np.abs(la - lb).max() <= 1e-2 * np.abs(la).max()
