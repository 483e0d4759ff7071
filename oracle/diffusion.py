"""The cached block-diffusion decode (threshold unmasking) restated on the CPU over ``OracleDecoder``.

Test infrastructure only (see ``oracle/__init__.py``). Greedy (temperature 0), positions equal to KV indices (a
synthetic prefix, so the response starts at ``next_pos`` = P; src/fast_sampling.py:181-184).

  generate_cached          src/fast_sampling.py:105-258  (bs = 1)
  generate_cached_batched  src/fast_sampling_batched.py:95-234  (rows in lockstep, each over its own cache: the
                           reference's left padding and pad mask make a row see exactly its own prefix, :15-25, :163-167)

One block: block = [seed | MASK x (bd-1)] at positions base..base+bd-1. While any position is masked, a probe
forward of the block against the frozen cache (all block rows see the cache and the whole block) gives logits; the
in-block token shift maps position j to row max(j-1, 0); x1 = argmax of the fp32 softmax, conf its probability;
masked positions with conf > threshold are unmasked, and the most confident masked position always is. A final
forward over the clean block commits its K/V (all rows bidirectional, or token-causal with ``commit_causal``), and
its last row's greedy id seeds the next block.
"""
from typing import Iterable, List, Optional

import torch

from .attention import window_mask
from .decoder import KVCache, OracleDecoder
from .rounds import greedy, prefill


def unmask_step(logits: torch.Tensor, block: torch.Tensor, mask_id: int, threshold: float):
    """One iteration of the unmask loop (src/fast_sampling.py:206-216; src/fast_sampling_batched.py:198-211).
    logits [W, V] are the block forward's rows (no shift yet); block [W] long. Returns (new block, x1 [W],
    conf [W] fp32 before masking, unmask [W] bool)."""
    shifted = torch.cat([logits[:1], logits[:-1]], 0)
    probs = torch.softmax(shifted.float(), dim=-1)
    x1 = probs.argmax(-1)
    conf = torch.gather(probs, -1, x1[:, None])[:, 0]
    mpos = block == mask_id
    c = torch.where(mpos, conf, torch.full_like(conf, float("-inf")))
    unmask = c > threshold
    unmask[c.argmax(-1)] = True
    unmask &= mpos
    new = block.clone()
    new[unmask] = x1[unmask]
    return new, x1, conf, unmask


class _Row:
    """One sequence's decode state: its cache, frozen length, next block's seed and the ids it has emitted."""

    def __init__(self, model: OracleDecoder, prefix_emb: torch.Tensor):
        self.cache, seed_logit = prefill(model, prefix_emb)
        self.P = prefix_emb.shape[0]
        self.frozen = self.P
        self.seed = int(greedy(seed_logit)[0])
        self.generated: List[int] = []
        self.done = False


def _block_forward(model: OracleDecoder, row: _Row, block: torch.Tensor, base: int, causal: bool) -> torch.Tensor:
    bd = block.shape[0]
    row.cache.truncate(row.frozen)
    mask = window_mask(row.frozen, bd, bd if causal else 0)
    return model.forward(model.embed(block), torch.arange(base, base + bd), row.cache, mask)


def cached_generate(model: OracleDecoder, prefix_emb: torch.Tensor, bd: int, mask_id: int, max_new_tokens: int,
                    threshold: float, eos_id: Optional[int] = None, commit_causal: bool = False,
                    commit_trace: Optional[list] = None, steps: Optional[list] = None) -> List[int]:
    """``generate_cached`` (src/fast_sampling.py:105-258). Returns the generated ids (cut before EOS).
    ``commit_trace`` receives the number of tokens unmasked by each probe forward (:217); ``steps`` receives one
    dict per probe forward: block index, the block before the step, x1, conf (fp32, before masking), unmask."""
    row = _Row(model, prefix_emb)
    num_blocks = (max_new_tokens + bd - 1) // bd
    for blk in range(num_blocks):
        if row.done or (eos_id is not None and row.seed == eos_id):
            break
        block = torch.full((bd,), mask_id, dtype=torch.long)
        block[0] = row.seed
        base = row.P + len(row.generated)
        while bool((block == mask_id).any()):
            h = _block_forward(model, row, block, base, causal=False)
            before = block
            block, x1, conf, unmask = unmask_step(model.logits(h), block, mask_id, threshold)
            if commit_trace is not None:
                commit_trace.append(int(unmask.sum()))
            if steps is not None:
                steps.append({"block": blk, "before": before.tolist(), "x1": x1.tolist(), "conf": conf.tolist(),
                              "unmask": unmask.tolist()})
        h = _block_forward(model, row, block, base, causal=commit_causal)
        row.frozen += bd
        row.seed = int(greedy(model.logits(h[-1:]))[0])
        for t in block.tolist():
            if eos_id is not None and t == eos_id:
                row.done = True
                break
            row.generated.append(t)
    return row.generated


def cached_batched_generate(model: OracleDecoder, prefix_embs: List[torch.Tensor], bd: int, mask_id: int,
                            max_new_tokens: int, threshold: float, stop_ids: Iterable[int] = ()) -> List[List[int]]:
    """``generate_cached_batched`` (src/fast_sampling_batched.py:95-234). Rows advance block by block in lockstep;
    within a block the probe forwards run until every row's block is clean (a clean row's step is a no-op,
    :196-197). A row stops recording at a stop id inside its block, or when its next seed is one (:219-228)."""
    stops = set(int(x) for x in stop_ids)
    rows = [_Row(model, e) for e in prefix_embs]
    for r in rows:
        if r.seed in stops:
            r.done = True
    num_blocks = (max_new_tokens + bd - 1) // bd
    for blk in range(num_blocks):
        if all(r.done for r in rows):
            break
        blocks = []
        for r in rows:
            b = torch.full((bd,), mask_id, dtype=torch.long)
            b[0] = r.seed
            blocks.append(b)
        bases = [r.P + blk * bd for r in rows]
        while any(bool((b == mask_id).any()) for b in blocks):
            for i, r in enumerate(rows):
                if not bool((blocks[i] == mask_id).any()):
                    continue                                # a clean block's step changes nothing
                h = _block_forward(model, r, blocks[i], bases[i], causal=False)
                blocks[i] = unmask_step(model.logits(h), blocks[i], mask_id, threshold)[0]
        for i, r in enumerate(rows):
            h = _block_forward(model, r, blocks[i], bases[i], causal=False)
            r.frozen += bd
            r.seed = int(greedy(model.logits(h[-1:]))[0])
        for i, r in enumerate(rows):
            if r.done:
                continue
            for t in blocks[i].tolist():
                if t in stops:
                    r.done = True
                    break
                r.generated.append(t)
            if not r.done and r.seed in stops:
                r.done = True
    return [r.generated for r in rows]
