"""Pin the oracle's GLM decoder layer against transformers' GlmOcrTextDecoderLayer (the container's copy, third
party; the reference pins transformers 5.9.0, uv.lock:1033-1035) on identical weights and inputs, eager attention
with an additive causal mask over a cache, in fp32. Also: the product's synthetic weight generator draws exactly
the oracle's weights."""
import numpy as np
import pytest
import torch

from oracle.attention import window_mask
from oracle.decoder import DecoderConfig, KVCache, OracleDecoder, make_weights


def hf_layer_and_rotary(cfg: DecoderConfig, w, l):
    from transformers.models.glm_ocr.configuration_glm_ocr import GlmOcrTextConfig
    from transformers.models.glm_ocr.modeling_glm_ocr import GlmOcrTextDecoderLayer, GlmOcrTextRotaryEmbedding
    half = cfg.rot_dim // 2
    sec = [half - 2 * (half // 3), half // 3, half // 3]
    hc = GlmOcrTextConfig(hidden_size=cfg.hidden, intermediate_size=cfg.ffn, num_attention_heads=cfg.n_heads,
                          num_key_value_heads=cfg.n_kv_heads, head_dim=cfg.head_dim, vocab_size=cfg.vocab,
                          num_hidden_layers=cfg.n_layers, rms_norm_eps=cfg.rms_eps,
                          rope_parameters={"rope_type": "default", "rope_theta": cfg.rope_theta,
                                           "partial_rotary_factor": cfg.partial_rotary, "mrope_section": sec})
    hc._attn_implementation = "eager"
    layer = GlmOcrTextDecoderLayer(hc, l).eval()
    sd = {"self_attn.q_proj.weight": w[f"{l}.wq"], "self_attn.k_proj.weight": w[f"{l}.wk"],
          "self_attn.v_proj.weight": w[f"{l}.wv"], "self_attn.o_proj.weight": w[f"{l}.wo"],
          "mlp.gate_up_proj.weight": w[f"{l}.w_gate_up"], "mlp.down_proj.weight": w[f"{l}.w_down"],
          "input_layernorm.weight": w[f"{l}.in_norm"], "post_self_attn_layernorm.weight": w[f"{l}.post_self_attn_norm"],
          "post_attention_layernorm.weight": w[f"{l}.post_attn_norm"],
          "post_mlp_layernorm.weight": w[f"{l}.post_mlp_norm"]}
    layer.load_state_dict(sd)
    return layer, GlmOcrTextRotaryEmbedding(hc)


@pytest.mark.parametrize("cfg", [DecoderConfig(), DecoderConfig(hidden=512, n_heads=8, n_kv_heads=2, head_dim=128,
                                                                 ffn=1024, vocab=1000)])
def test_layer_matches_transformers(cfg):
    from transformers import DynamicCache
    torch.manual_seed(0)
    w = make_weights(cfg, seed=1)
    g = torch.Generator().manual_seed(2)
    for n in ("in_norm", "post_self_attn_norm", "post_attn_norm", "post_mlp_norm"):
        w[f"0.{n}"] = 1 + 0.1 * torch.randn(cfg.hidden, generator=g)      # non-trivial norm weights
    dec = OracleDecoder(cfg, w)
    layer, rot = hf_layer_and_rotary(cfg, w, 0)
    P, W = 23, 6
    x_pre = torch.randn(P, cfg.hidden, generator=g)
    x_win = torch.randn(W, cfg.hidden, generator=g)
    # ours: prefill P rows causally, then a W-row causal window over the cache
    cache = KVCache(1)
    h1 = dec.layer(0, x_pre, torch.arange(P), cache, window_mask(0, P, P))
    h2 = dec.layer(0, x_win, torch.arange(P, P + W) + 5, cache, window_mask(P, W, W))
    # transformers: same two calls through a DynamicCache with additive masks and 3 equal M-RoPE rows
    hc = DynamicCache()
    with torch.no_grad():
        for xs, pos, m in ((x_pre, torch.arange(P), window_mask(0, P, P)),
                           (x_win, torch.arange(P, P + W) + 5, window_mask(P, W, W))):
            pid = pos[None, None, :].expand(3, 1, -1)
            pe = rot(xs[None], pid)
            add = torch.zeros(m.shape).masked_fill(torch.from_numpy(~m), torch.finfo(torch.float32).min)
            out = layer(xs[None], position_embeddings=pe, attention_mask=add[None, None], past_key_values=hc,
                        use_cache=True)
            out = out[0] if isinstance(out, tuple) else out
            if xs is x_pre:
                r1 = out[0]
            else:
                r2 = out[0]
    torch.testing.assert_close(h1, r1, rtol=1e-5, atol=1e-5)
    torch.testing.assert_close(h2, r2, rtol=1e-5, atol=1e-5)


def test_product_weights_equal_oracle_weights():
    from gravityocr_amd.model import TINY, synthetic_prompt, synthetic_weights
    from oracle.decoder import TINY as OT, make_prefix
    a, b = synthetic_weights(TINY, 0), make_weights(OT, 0)
    assert a.keys() == b.keys() and all(torch.equal(a[k], b[k]) for k in a)
    va, ia = synthetic_prompt(TINY, 256, 16, 0)
    vb, ib = make_prefix(OT, 256, 16, 0)
    assert torch.equal(va, vb) and torch.equal(ia, ib)
