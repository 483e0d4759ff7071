"""GLM-OCR text-decoder description and a synthetic random-init model exposing the reference's model protocol.

The drop-in decode functions read a model through the handles the reference's fast_sampling reads
(src/fast_sampling.py:16-18, src/models/glm_ocr_dllm.py:139-183): ``text_model`` (embed_tokens, layers, norm),
``glm.lm_head``, ``mm_model`` (get_image_features, get_rope_index), ``processor``, ``tokenizer``, ``mask_id``,
``image_token_id``, ``bd_size``, ``_sample_top_p``. ``SyntheticGlmOcr`` implements that protocol around seeded
N(0, 0.02) weights with transformers' GlmOcrTextDecoderLayer attribute names, so weights are extracted the same way
from it and from a real GLM-OCR text decoder.
"""
from dataclasses import dataclass
from typing import Dict, Tuple

import torch


@dataclass
class GlmTextConfig:
    n_layers: int = 16
    hidden: int = 1536
    n_heads: int = 16
    n_kv_heads: int = 2
    head_dim: int = 128
    ffn: int = 4608
    vocab: int = 59392
    rms_eps: float = 1e-5
    rope_theta: float = 10000.0
    partial_rotary: float = 0.5
    mrope_section: Tuple[int, int, int] = (8, 12, 12)   # rotary frequencies taken from the (t, h, w) positions

    @property
    def rot_dim(self) -> int:
        return int(self.head_dim * self.partial_rotary)

    @property
    def qkv_dim(self) -> int:
        return (self.n_heads + 2 * self.n_kv_heads) * self.head_dim


# the two decoders of the workloads: the CPU plumbing model and the 16-layer, 1536-hidden decoder
TINY = GlmTextConfig(n_layers=2, hidden=256, n_heads=4, n_kv_heads=2, head_dim=64, ffn=704, vocab=4096)
SYNTH_1536 = GlmTextConfig()


def synthetic_weights(cfg: GlmTextConfig, seed: int, std: float = 0.02) -> Dict[str, torch.Tensor]:
    """Seeded N(0, std) fp32 CPU weights, nn.Linear layout, drawn in a fixed order (embed; per layer q, k, v, o,
    gate_up, down; lm_head). RMSNorm weights are ones."""
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


def synthetic_prompt(cfg: GlmTextConfig, n_vis: int, n_text: int, seed: int):
    """``n_vis`` visual embeddings ~N(0,1) followed by ``n_text`` token ids ~U[0, vocab)."""
    g = torch.Generator().manual_seed(seed)
    vis = torch.empty(n_vis, cfg.hidden).normal_(0.0, 1.0, generator=g)
    ids = torch.randint(0, cfg.vocab, (n_text,), generator=g)
    return vis, ids


def config_from_model(model) -> GlmTextConfig:
    """The decoder shape of a model behind the protocol: ``model.cfg`` when it is a GlmTextConfig (the synthetic
    model), else transformers' GlmOcrTextConfig on ``model.text_model.config`` (hidden_size, num_hidden_layers,
    num_attention_heads, num_key_value_heads, head_dim, intermediate_size, vocab_size, rms_norm_eps,
    rope_parameters {rope_theta, partial_rotary_factor, mrope_section})."""
    cfg = getattr(model, "cfg", None)
    if isinstance(cfg, GlmTextConfig):
        return cfg
    hc = model.text_model.config
    rp = getattr(hc, "rope_parameters", None) or {}
    heads = hc.num_attention_heads
    return GlmTextConfig(n_layers=hc.num_hidden_layers, hidden=hc.hidden_size, n_heads=heads,
                         n_kv_heads=hc.num_key_value_heads,
                         head_dim=getattr(hc, "head_dim", None) or hc.hidden_size // heads,
                         ffn=hc.intermediate_size, vocab=hc.vocab_size, rms_eps=hc.rms_norm_eps,
                         rope_theta=rp.get("rope_theta", 10000.0),
                         partial_rotary=rp.get("partial_rotary_factor", 1.0),
                         mrope_section=tuple(rp.get("mrope_section", (8, 12, 12))))


def weights_from_model(model) -> Dict[str, torch.Tensor]:
    """Extract decoder weights through the model protocol (transformers GlmOcrTextDecoderLayer attribute names)."""
    tm = model.text_model
    w = {"embed": tm.embed_tokens.weight.detach(), "norm": tm.norm.weight.detach(),
         "lm_head": model.glm.lm_head.weight.detach()}
    for l, layer in enumerate(tm.layers):
        at, mlp = layer.self_attn, layer.mlp
        w[f"{l}.wq"] = at.q_proj.weight.detach()
        w[f"{l}.wk"] = at.k_proj.weight.detach()
        w[f"{l}.wv"] = at.v_proj.weight.detach()
        w[f"{l}.wo"] = at.o_proj.weight.detach()
        w[f"{l}.w_gate_up"] = mlp.gate_up_proj.weight.detach()
        w[f"{l}.w_down"] = mlp.down_proj.weight.detach()
        w[f"{l}.in_norm"] = layer.input_layernorm.weight.detach()
        w[f"{l}.post_self_attn_norm"] = layer.post_self_attn_layernorm.weight.detach()
        w[f"{l}.post_attn_norm"] = layer.post_attention_layernorm.weight.detach()
        w[f"{l}.post_mlp_norm"] = layer.post_mlp_layernorm.weight.detach()
    return w


# ----------------------------------------------------------------------------- synthetic model protocol ---------
class _Lin(torch.nn.Module):
    def __init__(self, w):
        super().__init__()
        self.weight = torch.nn.Parameter(w, requires_grad=False)


class _Norm(torch.nn.Module):
    def __init__(self, w, eps):
        super().__init__()
        self.weight = torch.nn.Parameter(w, requires_grad=False)
        self.eps = eps

    def forward(self, x):
        h = x.float()
        h = h * torch.rsqrt(h.pow(2).mean(-1, keepdim=True) + self.eps)
        return self.weight * h.to(x.dtype)


class _Layer(torch.nn.Module):
    def __init__(self, w, l, eps):
        super().__init__()
        self.self_attn = torch.nn.Module()
        for n, k in (("q_proj", "wq"), ("k_proj", "wk"), ("v_proj", "wv"), ("o_proj", "wo")):
            setattr(self.self_attn, n, _Lin(w[f"{l}.{k}"]))
        self.mlp = torch.nn.Module()
        self.mlp.gate_up_proj = _Lin(w[f"{l}.w_gate_up"])
        self.mlp.down_proj = _Lin(w[f"{l}.w_down"])
        self.input_layernorm = _Norm(w[f"{l}.in_norm"], eps)
        self.post_self_attn_layernorm = _Norm(w[f"{l}.post_self_attn_norm"], eps)
        self.post_attention_layernorm = _Norm(w[f"{l}.post_attn_norm"], eps)
        self.post_mlp_layernorm = _Norm(w[f"{l}.post_mlp_norm"], eps)


class _Enc(dict):
    def to(self, device):
        return _Enc({k: (v.to(device) if isinstance(v, torch.Tensor) else v) for k, v in self.items()})


class _Processor:
    """Chat template + 'image' encoding of the synthetic prompt: every image becomes n_vis placeholder ids."""

    def __init__(self, owner):
        self.owner = owner

    def apply_chat_template(self, msgs, add_generation_prompt=True, tokenize=False):
        return msgs[0]["content"][1]["text"]

    def __call__(self, text=None, images=None, return_tensors="pt"):
        o = self.owner
        key = o.crop_key(images[0] if images else None)
        vis, prompt_ids = o.crop(key)
        n_vis = vis.shape[0]
        ids = torch.cat([torch.full((n_vis,), o.image_token_id, dtype=torch.long), prompt_ids])[None]
        return _Enc(input_ids=ids, mm_token_type_ids=torch.zeros_like(ids), pixel_values=torch.tensor([key]),
                    image_grid_thw=torch.tensor([[1, 1, n_vis]]))


class _Tokenizer:
    def __init__(self, eos):
        self.eos_token_id = eos
        self.pad_token_id = None

    def decode(self, ids, skip_special_tokens=True):
        return " ".join(str(int(x)) for x in torch.as_tensor(ids).reshape(-1).tolist())


class _MM:
    def __init__(self, owner):
        self.owner = owner

    def get_image_features(self, pixel_values, image_grid_thw, return_dict=True):
        class _R:
            pass
        r = _R()
        r.pooler_output = [self.owner.crop(int(pixel_values.reshape(-1)[0]))[0]]
        return r

    def get_rope_index(self, input_ids, mm_tt, image_grid_thw=None, video_grid_thw=None, attention_mask=None):
        P = input_ids.shape[1]
        return torch.arange(P, device=input_ids.device)[None, None, :].expand(3, 1, P), None


class SyntheticGlmOcr(torch.nn.Module):
    """Random-init GLM-OCR stand-in: the decoder above, a synthetic 'image' (n_vis N(0,1) embeddings) and a fixed
    prompt of token ids. Positions are 1-D (the three M-RoPE rows equal). More crops, each with its own embeddings
    and prompt ids, can be added with ``add_crop``: a PIL image whose width is a crop's key encodes as that crop,
    any other image as the default one."""

    def __init__(self, cfg: GlmTextConfig, weights, visual, prompt_ids, mask_id, bd_size, eos_id=None,
                 image_token_id=None, dtype=torch.float32):
        super().__init__()
        self.cfg = cfg
        w = {k: v.to(dtype) for k, v in weights.items()}
        tm = torch.nn.Module()
        tm.embed_tokens = torch.nn.Embedding.from_pretrained(w["embed"], freeze=True)
        tm.layers = torch.nn.ModuleList([_Layer(w, l, cfg.rms_eps) for l in range(cfg.n_layers)])
        tm.norm = _Norm(w["norm"], cfg.rms_eps)
        self.text_model = tm
        self.glm = torch.nn.Module()
        self.glm.lm_head = _Lin(w["lm_head"])
        self.visual = visual.to(dtype)
        self.n_vis = visual.shape[0]
        self.prompt_ids = prompt_ids.long()
        self.mask_id = mask_id
        self.bd_size = bd_size
        self.image_token_id = image_token_id if image_token_id is not None else cfg.vocab - 2
        self.mm_model = _MM(self)
        self.processor = _Processor(self)
        self.tokenizer = _Tokenizer(eos_id)
        self._dtype = dtype
        self.crops = {}

    def add_crop(self, key: int, visual: torch.Tensor, prompt_ids: torch.Tensor):
        """Register a crop for images of width ``key`` (> 0)."""
        if key <= 0:
            raise ValueError("crop keys are image widths > 0")
        self.crops[int(key)] = (visual.to(self._dtype), prompt_ids.long())

    def crop_key(self, image) -> int:
        w = getattr(image, "size", (0,))[0] if image is not None else 0
        return int(w) if int(w) in self.crops else 0

    def crop(self, key: int):
        """(visual embeddings, prompt ids) of crop ``key`` (0 = the default crop)."""
        if key in self.crops:
            vis, ids = self.crops[key]
            return vis.to(self.visual.device), ids
        return self.visual, self.prompt_ids

    def _sample_top_p(self, logits, top_p, temperature):
        logits = logits.float()
        if temperature > 0:
            raise NotImplementedError("the synthetic model samples greedily only")
        probs = torch.softmax(logits, dim=-1)
        return probs.argmax(dim=-1), probs
