"""Write the natcache golden vectors for the tiny CPU plumbing workload by running the reference's own
``generate_speculative_natcache`` / ``generate_speculative_prefixcache`` / ``teacher_force_argmax``
(src/fast_sampling.py) on a duck-typed model.

Why an import: the per-round acceptance sequence (k per round, draft, ar_pred, new_tokens) of natcache depends on its
round-0 seed handling, masks, token shift and truncation (src/fast_sampling.py:499-584); nothing else in the
reference pins it. The duck-typed model exposes exactly the handles the drop-in reads (text_model.embed_tokens /
layers / norm / rotary_emb, mm_model.get_image_features / get_rope_index, glm.lm_head, processor, tokenizer,
mask_id, image_token_id, bd_size, _sample_top_p); its decoder layers run the oracle's layer math, so the vectors pin
the ROUND logic of the oracle restatement (oracle/rounds.py), given the layer.

Workload (tiny CPU plumbing): 2 layers, hidden 256, 4 q / 2 kv heads, head_dim 64, FFN 704, vocab 4096,
weights N(0, 0.02) fp32 seed 0; prefix 256 visual embeddings N(0,1) + 16 text ids U[0, 4096) (prefix seed 0);
bd 4, mask id 4095, 64 new tokens, greedy.

Run from the repo root:  python tests/golden/make_golden.py   (needs the reference tree at /root/reference).
Output: tests/golden/natcache_tiny.json
"""
import hashlib
import json
import os
import sys

import numpy as np
import torch
from PIL import Image

REPO = os.path.dirname(os.path.dirname(os.path.dirname(os.path.abspath(__file__))))
sys.path.insert(0, REPO)
sys.path.insert(0, "/root/reference/src")

from oracle.attention import window_mask  # noqa: E402
from oracle.decoder import TINY, KVCache, OracleDecoder, apply_rope, make_prefix, make_weights, rms_norm  # noqa: E402

N_VIS, N_TEXT, BD, MASK_ID, IMAGE_TOKEN_ID, MAX_NEW = 256, 16, 4, 4095, 4094, 64


def weights_digest(w):
    h = hashlib.sha256()
    for k in sorted(w):
        h.update(k.encode())
        h.update(w[k].numpy().tobytes())
    return h.hexdigest()


def dense_mask(attention_mask, Q, KV):
    """BlockMask (flex) or additive float mask -> [Q, KV] bool visible."""
    if isinstance(attention_mask, torch.Tensor):
        m = attention_mask[0, 0]
        return (m == 0).numpy()
    mod = attention_mask.mask_mod
    qi = torch.arange(Q)[:, None]
    ki = torch.arange(KV)[None, :]
    return mod(torch.tensor(0), torch.tensor(0), qi, ki).expand(Q, KV).numpy().astype(bool)


class ShimLayer(torch.nn.Module):
    """One decoder layer with transformers' call signature, computing the oracle's layer math."""

    def __init__(self, dec, idx):
        super().__init__()
        self.dec, self.idx = dec, idx

    def forward(self, hidden, position_embeddings=None, attention_mask=None, past_key_values=None, use_cache=True,
                **kw):
        dec, l = self.dec, self.idx
        cfg, w = dec.cfg, dec.w
        pos = position_embeddings[0]
        h = hidden[0]
        T = h.shape[0]
        x = rms_norm(h, w[f"{l}.in_norm"], cfg.rms_eps)
        q = apply_rope((x @ w[f"{l}.wq"].t()).view(T, cfg.n_heads, cfg.head_dim), pos, cfg)
        k = apply_rope((x @ w[f"{l}.wk"].t()).view(T, cfg.n_kv_heads, cfg.head_dim), pos, cfg)
        v = (x @ w[f"{l}.wv"].t()).view(T, cfg.n_kv_heads, cfg.head_dim)
        kk, vv = past_key_values.update(k.transpose(0, 1)[None], v.transpose(0, 1)[None], l)
        kk, vv = kk[0].transpose(0, 1), vv[0].transpose(0, 1)
        mask = dense_mask(attention_mask, T, kk.shape[0])
        a = dec.attend(q, kk, vv, mask) @ w[f"{l}.wo"].t()
        h = h + rms_norm(a, w[f"{l}.post_self_attn_norm"], cfg.rms_eps)
        x = rms_norm(h, w[f"{l}.post_attn_norm"], cfg.rms_eps)
        g, u = (x @ w[f"{l}.w_gate_up"].t()).chunk(2, dim=-1)
        m = (u * torch.nn.functional.silu(g)) @ w[f"{l}.w_down"].t()
        return (h + rms_norm(m, w[f"{l}.post_mlp_norm"], cfg.rms_eps))[None]


class Rotary(torch.nn.Module):
    def forward(self, x, position_ids=None):
        return (position_ids[0, 0], None)        # the three M-RoPE rows are equal: pass the 1-D positions


class Norm(torch.nn.Module):
    def __init__(self, dec):
        super().__init__()
        self.dec = dec

    def forward(self, h):
        return rms_norm(h, self.dec.w["norm"], self.dec.cfg.rms_eps)


class Enc(dict):
    def to(self, device):
        return self


class Processor:
    def __init__(self, ids):
        self.ids = ids

    def apply_chat_template(self, msgs, add_generation_prompt=True, tokenize=False):
        return "<image>" + msgs[0]["content"][1]["text"]

    def __call__(self, text=None, images=None, return_tensors="pt"):
        P = self.ids.shape[0]
        return Enc(input_ids=self.ids[None], mm_token_type_ids=torch.zeros(1, P, dtype=torch.long),
                   pixel_values=torch.zeros(1), image_grid_thw=torch.tensor([[1, 16, 16]]))


class Tokenizer:
    eos_token_id = None
    pad_token_id = None

    def decode(self, ids, skip_special_tokens=True):
        return " ".join(str(int(x)) for x in ids.tolist())


class MM:
    def __init__(self, vis):
        self.vis = vis

    def get_image_features(self, pixel_values, image_grid_thw, return_dict=True):
        class R:
            pass
        r = R()
        r.pooler_output = [self.vis]
        return r

    def get_rope_index(self, input_ids, mm_tt, image_grid_thw=None, video_grid_thw=None, attention_mask=None):
        P = input_ids.shape[1]
        return torch.arange(P)[None, None, :].expand(3, 1, P), torch.zeros(1, 1, dtype=torch.long)


class ShimModel(torch.nn.Module):
    def __init__(self, dec, vis, ids):
        super().__init__()
        self.dummy = torch.nn.Parameter(torch.zeros(1))
        tm = torch.nn.Module()
        tm.embed_tokens = torch.nn.Embedding.from_pretrained(dec.w["embed"], freeze=True)
        tm.layers = torch.nn.ModuleList([ShimLayer(dec, l) for l in range(dec.cfg.n_layers)])
        tm.norm = Norm(dec)
        tm.rotary_emb = Rotary()
        self.text_model = tm
        self.mm_model = MM(vis)
        glm = torch.nn.Module()
        glm.lm_head = torch.nn.Linear(dec.cfg.hidden, dec.cfg.vocab, bias=False)
        glm.lm_head.weight.data.copy_(dec.w["lm_head"])
        self.glm = glm
        self.processor = Processor(ids)
        self.tokenizer = Tokenizer()
        self.mask_id = MASK_ID
        self.image_token_id = IMAGE_TOKEN_ID
        self.bd_size = BD

    def _sample_top_p(self, logits, top_p, temperature):
        logits = logits.float()
        probs = torch.softmax(logits, dim=-1)
        return probs.argmax(dim=-1), probs


def main():
    import fast_sampling as ref   # the reference's src/fast_sampling.py

    torch.set_grad_enabled(False)
    w = make_weights(TINY, seed=0)
    vis, text = make_prefix(TINY, N_VIS, N_TEXT, seed=0)
    assert not (text == IMAGE_TOKEN_ID).any(), "a text id collides with the image placeholder id"
    ids = torch.cat([torch.full((N_VIS,), IMAGE_TOKEN_ID, dtype=torch.long), text])
    dec = OracleDecoder(TINY, w)
    model = ShimModel(dec, vis, ids)
    img = Image.new("RGB", (8, 8))

    out = {"workload": "tiny GLM decoder, natcache bd 4, 64 new tokens", "weights_sha256": weights_digest(w),
           "prefix_text_ids": text.tolist(), "n_vis": N_VIS, "bd": BD, "mask_id": MASK_ID,
           "image_token_id": IMAGE_TOKEN_ID, "max_new_tokens": MAX_NEW}
    for fd in (True, False):
        trace = []
        txt, stats = ref.generate_speculative_natcache(model, img, max_new_tokens=MAX_NEW, return_stats=True,
                                                       trace=trace, full_draft=fd)
        out[f"natcache_full_draft_{int(fd)}"] = {"ids": [int(x) for x in txt.split()], "stats": stats,
                                                 "trace": trace}
    txt, stats = ref.generate_speculative_prefixcache(model, img, max_new_tokens=MAX_NEW, return_stats=True)
    out["prefixcache"] = {"ids": [int(x) for x in txt.split()], "stats": stats}
    gen = out["natcache_full_draft_1"]["ids"]
    out["teacher_force_argmax"] = ref.teacher_force_argmax(model, img, "Text Recognition:", gen)
    path = os.path.join(os.path.dirname(os.path.abspath(__file__)), "natcache_tiny.json")
    with open(path, "w") as f:
        json.dump(out, f)
    print("wrote", path, "rounds", out["natcache_full_draft_1"]["stats"])


if __name__ == "__main__":
    main()
