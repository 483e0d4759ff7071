"""Write the block-diffusion golden vectors for the tiny CPU workload by running the reference's own
``generate_cached`` (src/fast_sampling.py) and ``generate_cached_batched`` (src/fast_sampling_batched.py) on a
duck-typed model.

Why an import: the order in which threshold unmasking fills a block (the in-block token shift, the forced most
confident position, the seed taken from the commit forward, the stop rules of the batched loop) is only pinned by
the reference's own loops (src/fast_sampling.py:198-258, src/fast_sampling_batched.py:181-228). The duck-typed model
exposes the handles the samplers read; its decoder layers run the oracle's layer math for every row of a batch (per
row positions and the reference's per-row flex masks, left padding included), so the vectors pin the decode logic of
the oracle restatement (oracle/diffusion.py), given the layer.

Workload (tiny CPU plumbing): the 2-layer 256-hidden decoder of tests/golden/make_golden.py (weights seed 0, fp32);
three crops with prefixes of (visual, text) = (48, 8), (32, 12), (64, 4) tokens (prefix seeds 1, 2, 3); bd 4,
mask id 4095, image token id 4094, 24 new tokens, threshold 0.000725 (the tiny model's confidences lie around
7e-4, so some steps unmask one position and some several).

Run from the repo root:  python tests/golden/make_golden_diffusion.py   (needs the reference tree at
/root/reference). Output: tests/golden/diffusion_tiny.json
"""
import json
import os
import sys

import torch
from PIL import Image

HERE = os.path.dirname(os.path.abspath(__file__))
REPO = os.path.dirname(os.path.dirname(HERE))
sys.path.insert(0, REPO)
sys.path.insert(0, HERE)
sys.path.insert(0, "/root/reference/src")

from make_golden import Enc, Norm, weights_digest  # noqa: E402
from oracle.decoder import TINY, OracleDecoder, apply_rope, make_prefix, make_weights, rms_norm  # noqa: E402

CROPS = [(48, 8, 1), (32, 12, 2), (64, 4, 3)]       # (visual tokens, text tokens, prefix seed)
BD, MASK_ID, IMAGE_TOKEN_ID, MAX_NEW, THRESHOLD = 4, 4095, 4094, 24, 0.000725


def dense_mask_row(attention_mask, b, Q, KV):
    """BlockMask (flex) -> [Q, KV] bool visible, for batch row b."""
    mod = attention_mask.mask_mod
    qi = torch.arange(Q)[:, None]
    ki = torch.arange(KV)[None, :]
    return mod(torch.tensor(b), torch.tensor(0), qi, ki).expand(Q, KV).numpy().astype(bool)


class BatchedShimLayer(torch.nn.Module):
    """One decoder layer with transformers' call signature over a batch [bs, T, H]: the oracle's layer math per row,
    each row with its own positions and its own row of the flex mask."""

    def __init__(self, dec, idx):
        super().__init__()
        self.dec, self.idx = dec, idx

    def forward(self, hidden, position_embeddings=None, attention_mask=None, past_key_values=None, use_cache=True,
                **kw):
        dec, l = self.dec, self.idx
        cfg, w = dec.cfg, dec.w
        pos = position_embeddings[0]                      # [bs, T]
        bs, T, _ = hidden.shape
        qs, ks, vs = [], [], []
        for b in range(bs):
            x = rms_norm(hidden[b], w[f"{l}.in_norm"], cfg.rms_eps)
            qs.append(apply_rope((x @ w[f"{l}.wq"].t()).view(T, cfg.n_heads, cfg.head_dim), pos[b], cfg))
            ks.append(apply_rope((x @ w[f"{l}.wk"].t()).view(T, cfg.n_kv_heads, cfg.head_dim), pos[b], cfg))
            vs.append((x @ w[f"{l}.wv"].t()).view(T, cfg.n_kv_heads, cfg.head_dim))
        k = torch.stack(ks).transpose(1, 2)                # [bs, Hkv, T, D]
        v = torch.stack(vs).transpose(1, 2)
        kk, vv = past_key_values.update(k, v, l)
        out = []
        for b in range(bs):
            kb, vb = kk[b].transpose(0, 1), vv[b].transpose(0, 1)
            mask = dense_mask_row(attention_mask, b, T, kb.shape[0])
            a = dec.attend(qs[b], kb, vb, mask) @ w[f"{l}.wo"].t()
            h = hidden[b] + rms_norm(a, w[f"{l}.post_self_attn_norm"], cfg.rms_eps)
            x = rms_norm(h, w[f"{l}.post_attn_norm"], cfg.rms_eps)
            g, u = (x @ w[f"{l}.w_gate_up"].t()).chunk(2, dim=-1)
            m = (u * torch.nn.functional.silu(g)) @ w[f"{l}.w_down"].t()
            out.append(h + rms_norm(m, w[f"{l}.post_mlp_norm"], cfg.rms_eps))
        return torch.stack(out)


class Rotary(torch.nn.Module):
    def forward(self, x, position_ids=None):
        return (position_ids[0], None)        # the three M-RoPE rows are equal: pass the per-row 1-D positions


class Processor:
    """Maps each crop (told apart by its pixel width) to its prefix ids."""

    def __init__(self, ids_by_width):
        self.ids_by_width = ids_by_width

    def apply_chat_template(self, msgs, add_generation_prompt=True, tokenize=False):
        return "<image>" + msgs[0]["content"][1]["text"]

    def __call__(self, text=None, images=None, return_tensors="pt"):
        width = images[0].size[0]
        ids = self.ids_by_width[width]
        P = ids.shape[0]
        return Enc(input_ids=ids[None], mm_token_type_ids=torch.zeros(1, P, dtype=torch.long),
                   pixel_values=torch.tensor([width]), image_grid_thw=torch.tensor([[1, 16, 16]]))


class Tokenizer:
    def __init__(self, eos=None):
        self.eos_token_id = eos
        self.pad_token_id = None

    def decode(self, ids, skip_special_tokens=True):
        return " ".join(str(int(x)) for x in ids.tolist())


class MM:
    def __init__(self, vis_by_width):
        self.vis_by_width = vis_by_width

    def get_image_features(self, pixel_values, image_grid_thw, return_dict=True):
        class R:
            pass
        r = R()
        r.pooler_output = [self.vis_by_width[int(pixel_values[0])]]
        return r

    def get_rope_index(self, input_ids, mm_tt, image_grid_thw=None, video_grid_thw=None, attention_mask=None):
        P = input_ids.shape[1]
        return torch.arange(P)[None, None, :].expand(3, 1, P), torch.zeros(1, 1, dtype=torch.long)


class ShimModel(torch.nn.Module):
    def __init__(self, dec, vis_by_width, ids_by_width):
        super().__init__()
        self.dummy = torch.nn.Parameter(torch.zeros(1))
        tm = torch.nn.Module()
        tm.embed_tokens = torch.nn.Embedding.from_pretrained(dec.w["embed"], freeze=True)
        tm.layers = torch.nn.ModuleList([BatchedShimLayer(dec, l) for l in range(dec.cfg.n_layers)])
        tm.norm = Norm(dec)
        tm.rotary_emb = Rotary()
        self.text_model = tm
        self.mm_model = MM(vis_by_width)
        glm = torch.nn.Module()
        glm.lm_head = torch.nn.Linear(dec.cfg.hidden, dec.cfg.vocab, bias=False)
        glm.lm_head.weight.data.copy_(dec.w["lm_head"])
        self.glm = glm
        self.processor = Processor(ids_by_width)
        self.tokenizer = Tokenizer()
        self.mask_id = MASK_ID
        self.image_token_id = IMAGE_TOKEN_ID
        self.bd_size = BD

    def _sample_top_p(self, logits, top_p, temperature):
        logits = logits.float()
        probs = torch.softmax(logits, dim=-1)
        return probs.argmax(dim=-1), probs


def ids_of(txt):
    return [int(x) for x in txt.split()] if txt else []


def main():
    import fast_sampling as ref               # the reference's src/fast_sampling.py
    import fast_sampling_batched as ref_b     # the reference's src/fast_sampling_batched.py

    torch.set_grad_enabled(False)
    w = make_weights(TINY, seed=0)
    dec = OracleDecoder(TINY, w)
    vis_by_width, ids_by_width, images, crops = {}, {}, [], []
    for i, (n_vis, n_text, seed) in enumerate(CROPS):
        vis, text = make_prefix(TINY, n_vis, n_text, seed=seed)
        assert not (text == IMAGE_TOKEN_ID).any() and not (text == MASK_ID).any()
        width = 8 + i                                      # tells the crops apart
        vis_by_width[width] = vis
        ids_by_width[width] = torch.cat([torch.full((n_vis,), IMAGE_TOKEN_ID, dtype=torch.long), text])
        images.append(Image.new("RGB", (width, 8)))
        crops.append({"n_vis": n_vis, "text_ids": text.tolist(), "prefix_seed": seed})
    model = ShimModel(dec, vis_by_width, ids_by_width)

    out = {"workload": "tiny GLM decoder, block diffusion bd 4, 24 new tokens", "weights_sha256": weights_digest(w),
           "crops": crops, "bd": BD, "mask_id": MASK_ID, "image_token_id": IMAGE_TOKEN_ID, "max_new_tokens": MAX_NEW,
           "threshold": THRESHOLD}
    # generate_cached on crop 0: block-causal and token-causal commits, with the commit trace and detail
    for causal in (False, True):
        trace, detail = [], []
        txt = ref.generate_cached(model, images[0], max_new_tokens=MAX_NEW, threshold=THRESHOLD,
                                  commit_trace=trace, commit_causal=causal, commit_detail=detail)
        out[f"cached_commit_causal_{int(causal)}"] = {"ids": ids_of(txt), "commit_trace": trace,
                                                      "commit_detail": detail}
    # an EOS inside the output: the first id whose first occurrence is past the first block and not a block seed
    gen = out["cached_commit_causal_0"]["ids"]
    eos = next(t for i, t in enumerate(gen) if i >= BD + 1 and i % BD != 0 and t not in gen[:i])
    model.tokenizer = Tokenizer(eos)
    out["cached_eos"] = {"eos_id": eos, "ids": ids_of(ref.generate_cached(model, images[0], max_new_tokens=MAX_NEW,
                                                                         threshold=THRESHOLD))}
    # generate_cached_batched on the three crops: no stop ids, then a tokenizer EOS plus a generation-config stop
    model.tokenizer = Tokenizer()
    out["batched"] = {"ids": [ids_of(t) for t in ref_b.generate_cached_batched(model, images, max_new_tokens=MAX_NEW,
                                                                                threshold=THRESHOLD)]}
    rows = out["batched"]["ids"]
    stop_a, stop_b = rows[1][6], rows[2][13]
    model.tokenizer = Tokenizer(stop_a)
    model.glm.generation_config = type("GenerationConfig", (), {"eos_token_id": [stop_a, stop_b]})()
    out["batched_stops"] = {"stop_ids": [stop_a, stop_b],
                            "ids": [ids_of(t) for t in ref_b.generate_cached_batched(
                                model, images, max_new_tokens=MAX_NEW, threshold=THRESHOLD)]}
    path = os.path.join(HERE, "diffusion_tiny.json")
    with open(path, "w") as f:
        json.dump(out, f)
    print("wrote", path, {k: v["ids"] for k, v in out.items() if isinstance(v, dict) and "ids" in v})


if __name__ == "__main__":
    main()
