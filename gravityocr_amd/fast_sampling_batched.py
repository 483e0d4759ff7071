"""Drop-in ``generate_cached_batched`` with the signature of the reference's src/fast_sampling_batched.py:95-97,
running the batched block-diffusion decode on the MI355X kernels.

The reference left-pads the ragged prompts to a rectangular cache and masks the pad columns per row
(src/fast_sampling_batched.py:10-25, :150-167). Here every crop owns a slot of the paged KV pool with its own
committed length, so there is no padding: each row's attention reads exactly its own prompt and blocks, which is
what the pad mask achieves. Per-row M-RoPE positions come from the model's ``get_rope_index`` as in the reference
(prefill), and the response of row b continues at its own ``next_pos[b]``.

Rows advance block by block together; within a block the probe forwards run until every row's block is clean
(a clean row's step leaves it unchanged), as in the reference's loop (:196-211). A row stops recording at a stop id
inside its block or when its next seed is one; the stop ids are the model's generation-config EOS list plus the
tokenizer's EOS (:121-129, :219-228). Greedy only (``temperature == 0``).
"""
import re
from typing import List

import torch

from .engine import PAGE
from .fast_sampling import _argmax_rows, _check_greedy, _model_device, _prefill, _session, prepare_prompt

__all__ = ["generate_cached_batched"]


def _stop_ids(model) -> set:
    eos_id = model.tokenizer.eos_token_id
    gce = getattr(getattr(model.glm, "generation_config", None), "eos_token_id", None)
    stops = set(int(x) for x in gce) if isinstance(gce, (list, tuple)) else set()
    if eos_id is not None:
        stops.add(int(eos_id))
    return stops


@torch.no_grad()
def generate_cached_batched(model, images, prompt="Text Recognition:", max_new_tokens=512,
                            threshold=0.99, temperature=0.0, top_p=0.95, max_long_side=1344):
    """Batched block-diffusion OCR of a list of crops (src/fast_sampling_batched.py:95-234). Returns list[str], one
    per crop, in order."""
    from PIL import Image

    _check_greedy(temperature)
    if isinstance(images, Image.Image):
        images = [images]
    bs = len(images)
    if bs == 0:
        return []
    device = _model_device(model)
    bd, mask_id = int(model.bd_size), int(model.mask_id)
    stops = _stop_ids(model)
    per = [prepare_prompt(model, img, prompt, max_long_side, device) for img in images]
    lens = [p[0].shape[1] for p in per]
    num_blocks = (max_new_tokens + bd - 1) // bd
    sess = _session(model, device, max(lens) + num_blocks * bd + PAGE, bs=bs)
    eng = sess.eng
    seeds = []
    for b, (input_ids, emb, positions, next_pos) in enumerate(per):
        last = _prefill(eng, emb, positions, slot=b)
        seeds.append(int(_argmax_rows(eng, last.view(1, -1), softmax_rule=True)[0]))
    dec = sess.diffusion_decoder(bs, bd, mask_id, threshold, False)
    pos_delta = torch.tensor([p[3] - n for p, n in zip(per, lens)], dtype=torch.int32)
    dec.start(torch.tensor(seeds), pos_delta=pos_delta)

    generated: List[List[int]] = [[] for _ in range(bs)]
    done = [s in stops for s in seeds]
    for _ in range(num_blocks):
        if all(done):
            break
        blocks, seeds, _ = dec.decode_block(seeds)
        for b in range(bs):
            if done[b]:
                continue
            for t in blocks[b]:
                if t in stops:
                    done[b] = True
                    break
                generated[b].append(t)
            if not done[b] and seeds[b] in stops:
                done[b] = True

    def strip(t):
        return re.sub(r"<think>.*?</think>\s*", "", t, flags=re.S)

    return [strip(model.tokenizer.decode(torch.tensor(g, device=device), skip_special_tokens=True)) if g else ""
            for g in generated]
