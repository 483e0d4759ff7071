"""GLM-OCR text decoder, restated on the CPU in torch (fp32 by default), with a contiguous per-layer KV cache.

Test infrastructure only (see ``oracle/__init__.py``).

Layer math follows transformers' GlmOcrTextDecoderLayer as the reference calls it through ``_run_layers``
(src/fast_sampling.py:89-102; container transformers/models/glm_ocr/modeling_glm_ocr.py:58-72 RMSNorm,
:129-173 interleaved partial RoPE, :176-236 attention, :239-253 SwiGLU MLP, :256-310 sandwich norms):

    x  = input_layernorm(h);  a = o_proj(attn(rope(q_proj x), rope(k_proj x), v_proj x))
    h  = h + post_self_attn_layernorm(a)
    m  = down_proj(silu(gate) * up) of gate_up_proj(post_attention_layernorm(h))
    h  = h + post_mlp_layernorm(m)

RoPE pairs adjacent elements (2i, 2i+1) of the first ``rot = head_dim * partial_rotary`` dims with frequency
inv_freq[i] = theta^(-2i/rot); the rest pass through. With the three M-RoPE position rows equal (a text-only or
synthetic prefix), M-RoPE reduces to this 1-D RoPE (modeling_glm_ocr.py:672-692).
"""
from dataclasses import dataclass, field
from typing import Dict, List, Optional

import numpy as np
import torch


@dataclass
class DecoderConfig:
    n_layers: int = 2
    hidden: int = 256
    n_heads: int = 4
    n_kv_heads: int = 2
    head_dim: int = 64
    ffn: int = 704
    vocab: int = 4096
    rms_eps: float = 1e-5
    rope_theta: float = 10000.0
    partial_rotary: float = 0.5

    @property
    def rot_dim(self) -> int:
        return int(self.head_dim * self.partial_rotary)


TINY = DecoderConfig()
SYNTH_1536 = DecoderConfig(n_layers=16, hidden=1536, n_heads=16, n_kv_heads=2, head_dim=128, ffn=4608, vocab=59392)


def make_weights(cfg: DecoderConfig, seed: int, std: float = 0.02) -> Dict[str, torch.Tensor]:
    """Seeded N(0, std) weights in a fixed draw order (embed, per layer q,k,v,o,gate_up,down, lm_head); RMSNorm
    weights are ones. fp32 CPU tensors, nn.Linear layout [out, in]."""
    g = torch.Generator().manual_seed(seed)
    H, D = cfg.hidden, cfg.head_dim

    def draw(*shape):
        return torch.empty(*shape).normal_(0.0, std, generator=g)

    w = {"embed": draw(cfg.vocab, H)}
    for l in range(cfg.n_layers):
        w[f"{l}.wq"] = draw(cfg.n_heads * D, H)
        w[f"{l}.wk"] = draw(cfg.n_kv_heads * D, H)
        w[f"{l}.wv"] = draw(cfg.n_kv_heads * D, H)
        w[f"{l}.wo"] = draw(H, cfg.n_heads * D)
        w[f"{l}.w_gate_up"] = draw(2 * cfg.ffn, H)
        w[f"{l}.w_down"] = draw(H, cfg.ffn)
        for n in ("in_norm", "post_self_attn_norm", "post_attn_norm", "post_mlp_norm"):
            w[f"{l}.{n}"] = torch.ones(H)
    w["norm"] = torch.ones(H)
    w["lm_head"] = draw(cfg.vocab, H)
    return w


def make_prefix(cfg: DecoderConfig, n_vis: int, n_text: int, seed: int):
    """Synthetic prompt: ``n_vis`` visual embeddings ~N(0,1) then ``n_text`` token ids ~U[0, vocab)."""
    g = torch.Generator().manual_seed(seed)
    vis = torch.empty(n_vis, cfg.hidden).normal_(0.0, 1.0, generator=g)
    ids = torch.randint(0, cfg.vocab, (n_text,), generator=g)
    return vis, ids


def rms_norm(x: torch.Tensor, w: torch.Tensor, eps: float) -> torch.Tensor:
    xf = x.float()
    y = xf * torch.rsqrt(xf.pow(2).mean(-1, keepdim=True) + eps)
    return w * y.to(x.dtype)


def inv_freq(cfg: DecoderConfig) -> torch.Tensor:
    """fp32 inverse frequencies exactly as transformers computes them (modeling_glm_ocr.py:660-668)."""
    rot = cfg.rot_dim
    return 1.0 / (cfg.rope_theta ** (torch.arange(0, rot, 2, dtype=torch.int64).float() / rot))


def apply_rope(x: torch.Tensor, pos: torch.Tensor, cfg: DecoderConfig) -> torch.Tensor:
    """x [T, heads, D]; pos [T] int. Interleaved-pair rotation of the first rot_dim dims, in fp32."""
    rot = cfg.rot_dim
    freqs = pos.to(torch.float32)[:, None] * inv_freq(cfg)[None, :]         # [T, rot/2]
    c = torch.cos(freqs)[:, None, :]
    s = torch.sin(freqs)[:, None, :]
    xf = x.float()
    x0 = xf[..., 0:rot:2]
    x1 = xf[..., 1:rot:2]
    out = xf.clone()
    out[..., 0:rot:2] = x0 * c - x1 * s
    out[..., 1:rot:2] = x1 * c + x0 * s
    return out.to(x.dtype)


class KVCache:
    """Contiguous per-layer K/V [L, Hkv, D] (the reference's DynamicCache shape, without the batch axis)."""

    def __init__(self, n_layers: int):
        self.k: List[Optional[torch.Tensor]] = [None] * n_layers
        self.v: List[Optional[torch.Tensor]] = [None] * n_layers

    def length(self) -> int:
        return 0 if self.k[0] is None else self.k[0].shape[0]

    def append(self, l: int, k: torch.Tensor, v: torch.Tensor):
        self.k[l] = k if self.k[l] is None else torch.cat([self.k[l], k], 0)
        self.v[l] = v if self.v[l] is None else torch.cat([self.v[l], v], 0)

    def truncate(self, length: int):
        """src/fast_sampling.py:78-86 ``_truncate_cache``."""
        for l in range(len(self.k)):
            if self.k[l] is not None and self.k[l].shape[0] > length:
                self.k[l] = self.k[l][:length].clone()
                self.v[l] = self.v[l][:length].clone()


class OracleDecoder:
    """The synthetic GLM decoder on the CPU. ``dtype`` is the compute dtype of activations and weights."""

    def __init__(self, cfg: DecoderConfig, weights: Dict[str, torch.Tensor], dtype=torch.float32):
        self.cfg = cfg
        self.dtype = dtype
        self.w = {k: v.to(dtype) for k, v in weights.items()}

    def embed(self, ids: torch.Tensor) -> torch.Tensor:
        return self.w["embed"][ids.long()]

    def logits(self, h: torch.Tensor) -> torch.Tensor:
        return rms_norm(h, self.w["norm"], self.cfg.rms_eps) @ self.w["lm_head"].t()

    def attend(self, q, k, v, mask):
        """q [W, Hq, D], k/v [T, Hkv, D], mask [W, T] bool -> [W, Hq*D] (softmax in fp32 as transformers'
        eager path does)."""
        cfg = self.cfg
        G = cfg.n_heads // cfg.n_kv_heads
        kk = k.repeat_interleave(G, dim=1)
        vv = v.repeat_interleave(G, dim=1)
        s = torch.einsum("whd,thd->hwt", q.float(), kk.float()) * (cfg.head_dim ** -0.5)
        s = s.masked_fill(~torch.as_tensor(mask)[None], float("-inf"))
        p = torch.softmax(s, dim=-1).to(self.dtype)
        o = torch.einsum("hwt,thd->whd", p.float(), vv.float()).to(self.dtype)
        return o.reshape(q.shape[0], -1)

    def layer(self, l: int, h: torch.Tensor, pos: torch.Tensor, cache: KVCache, mask: np.ndarray) -> torch.Tensor:
        cfg, w = self.cfg, self.w
        T = h.shape[0]
        x = rms_norm(h, w[f"{l}.in_norm"], cfg.rms_eps)
        q = (x @ w[f"{l}.wq"].t()).view(T, cfg.n_heads, cfg.head_dim)
        k = (x @ w[f"{l}.wk"].t()).view(T, cfg.n_kv_heads, cfg.head_dim)
        v = (x @ w[f"{l}.wv"].t()).view(T, cfg.n_kv_heads, cfg.head_dim)
        q = apply_rope(q, pos, cfg)
        k = apply_rope(k, pos, cfg)
        cache.append(l, k, v)
        a = self.attend(q, cache.k[l], cache.v[l], mask) @ w[f"{l}.wo"].t()
        h = h + rms_norm(a, w[f"{l}.post_self_attn_norm"], cfg.rms_eps)
        x = rms_norm(h, w[f"{l}.post_attn_norm"], cfg.rms_eps)
        gu = x @ w[f"{l}.w_gate_up"].t()
        g, u = gu.chunk(2, dim=-1)
        m = (u * torch.nn.functional.silu(g)) @ w[f"{l}.w_down"].t()
        return h + rms_norm(m, w[f"{l}.post_mlp_norm"], cfg.rms_eps)

    def forward(self, emb: torch.Tensor, pos: torch.Tensor, cache: KVCache, mask: np.ndarray) -> torch.Tensor:
        """Run all layers over ``emb`` [T, H] at positions ``pos`` [T]; K/V are appended to ``cache``; ``mask`` is
        [T, cache_len + T]. Returns the last hidden states [T, H]."""
        h = emb.to(self.dtype)
        for l in range(self.cfg.n_layers):
            h = self.layer(l, h, pos, cache, mask)
        return h
