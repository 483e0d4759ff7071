"""Pin the oracle's block-diffusion decode (oracle/diffusion.py) to the reference's golden vectors
(tests/golden/diffusion_tiny.json, written by the reference's own generate_cached / generate_cached_batched on the
tiny CPU workload; see tests/golden/make_golden_diffusion.py): ids with block-causal and token-causal commits, the
commit trace and commit detail, an EOS inside a block, the batched rows with and without stop ids. Also the unmask
rule against a brute-force reading of it on small cases, including NaN / inf rows and a seed equal to the mask id."""
import json
import math
import os

import numpy as np
import pytest
import torch

from oracle.decoder import TINY, OracleDecoder, make_prefix, make_weights
from oracle.diffusion import cached_batched_generate, cached_generate, unmask_step

GOLDEN = os.path.join(os.path.dirname(__file__), "golden", "diffusion_tiny.json")


@pytest.fixture(scope="module")
def setup():
    with open(GOLDEN) as f:
        g = json.load(f)
    torch.set_grad_enabled(False)
    dec = OracleDecoder(TINY, make_weights(TINY, 0))
    embs = []
    for c in g["crops"]:
        vis, text = make_prefix(TINY, c["n_vis"], len(c["text_ids"]), c["prefix_seed"])
        assert text.tolist() == c["text_ids"]
        embs.append(torch.cat([vis, dec.embed(text)], 0))
    return g, dec, embs


def detail_from_steps(steps, P, bd, mask_id, seeds):
    """The reference's commit_detail records (src/fast_sampling.py:185-238) rebuilt from the oracle's steps."""
    out = []
    by_block = {}
    for s in steps:
        by_block.setdefault(s["block"], []).append(s)
    for blk in sorted(set(by_block) | set(range(len(seeds)))):
        frozen = P + blk * bd
        out.append({"block": frozen // bd, "step": len(out), "pos": [frozen], "in_block_pos": [0],
                    "tok": [seeds[blk]], "conf": [1.0], "is_seed": True})
        for s in by_block.get(blk, []):
            idx = [i for i, u in enumerate(s["unmask"]) if u]
            if not idx:
                continue
            mp = [i for i, t in enumerate(s["before"]) if t == mask_id]
            out.append({"pred_all": {"pos": mp, "tok": [s["x1"][i] for i in mp],
                                     "conf": [round(s["conf"][i], 4) for i in mp]},
                        "block": frozen // bd, "step": len(out), "pos": [frozen + i for i in idx],
                        "in_block_pos": idx, "tok": [s["x1"][i] for i in idx],
                        "conf": [round(s["conf"][i], 4) for i in idx]})
    return out


@pytest.mark.parametrize("causal", [0, 1])
def test_cached_equals_golden(setup, causal):
    g, dec, embs = setup
    trace, steps = [], []
    ids = cached_generate(dec, embs[0], g["bd"], g["mask_id"], g["max_new_tokens"], g["threshold"],
                          commit_causal=bool(causal), commit_trace=trace, steps=steps)
    want = g[f"cached_commit_causal_{causal}"]
    assert ids == want["ids"]
    assert trace == want["commit_trace"]
    seeds = [d["tok"][0] for d in want["commit_detail"] if d.get("is_seed")]
    assert seeds == ids[::g["bd"]]                      # block[0] of every block is its seed
    P = embs[0].shape[0]
    assert detail_from_steps(steps, P, g["bd"], g["mask_id"], seeds) == want["commit_detail"]


def test_cached_eos_inside_a_block(setup):
    g, dec, embs = setup
    ids = cached_generate(dec, embs[0], g["bd"], g["mask_id"], g["max_new_tokens"], g["threshold"],
                          eos_id=g["cached_eos"]["eos_id"])
    assert ids == g["cached_eos"]["ids"]
    full = g["cached_commit_causal_0"]["ids"]
    assert ids == full[:full.index(g["cached_eos"]["eos_id"])]


def test_batched_equals_golden(setup):
    g, dec, embs = setup
    rows = cached_batched_generate(dec, embs, g["bd"], g["mask_id"], g["max_new_tokens"], g["threshold"])
    assert rows == g["batched"]["ids"]
    # rows never interact: each row is its own bs=1 decode
    assert rows[0] == g["cached_commit_causal_0"]["ids"]
    rows = cached_batched_generate(dec, embs, g["bd"], g["mask_id"], g["max_new_tokens"], g["threshold"],
                                   stop_ids=g["batched_stops"]["stop_ids"])
    assert rows == g["batched_stops"]["ids"]


def brute_unmask(logits, block, mask_id, threshold):
    """The unmask rule read literally, one position at a time, with Python floats (fp64) for the softmax."""
    W, V = logits.shape
    x1, conf = [], []
    for j in range(W):
        row = [float(v) for v in logits[max(j - 1, 0)]]
        if any(math.isnan(v) or v == math.inf for v in row) or all(v == -math.inf for v in row):
            x1.append(0)
            conf.append(float("nan"))
            continue
        m = max(row)
        i = row.index(m)
        x1.append(i)
        conf.append(1.0 / sum(math.exp(v - m) for v in row))
    masked = [int(block[j]) == mask_id for j in range(W)]
    best, bj = -math.inf, 0
    for j in range(W):
        c = conf[j] if masked[j] else -math.inf
        if (math.isnan(c) and not math.isnan(best)) or (not math.isnan(best) and c > best):
            best, bj = c, j
    new = [int(t) for t in block]
    unmask = [False] * W
    for j in range(W):
        if masked[j] and (conf[j] > threshold or j == bj):
            new[j] = x1[j]
            unmask[j] = True
    return new, x1, conf, unmask


@pytest.mark.parametrize("case", range(40))
def test_unmask_step_equals_brute_force(case):
    rng = np.random.default_rng(case)
    W, V, mask_id = int(rng.integers(1, 7)), int(rng.integers(2, 40)), 999
    logits = torch.from_numpy(rng.normal(0, 2, (W, V)).astype(np.float32))
    if case % 5 == 1:
        logits[rng.integers(0, W), rng.integers(0, V)] = float("nan")
    if case % 5 == 2:
        logits[rng.integers(0, W), rng.integers(0, V)] = float("inf")
    if case % 5 == 3:
        logits[rng.integers(0, W)] = float("-inf")
    if case % 7 == 0:
        logits[:, 1] = logits[:, 0]                       # ties: the lowest index wins
    block = torch.tensor([mask_id if rng.random() < 0.6 else int(rng.integers(0, V)) for _ in range(W)])
    threshold = float(rng.choice([0.0, 0.3, 0.6, 0.99, 1.0]))
    new, x1, conf, unmask = unmask_step(logits, block, mask_id, threshold)
    bn, bx, bc, bu = brute_unmask(logits, block, mask_id, threshold)
    assert x1.tolist() == bx
    np.testing.assert_allclose(conf.numpy(), np.array(bc, dtype=np.float64), rtol=1e-5, equal_nan=True)
    assert unmask.tolist() == bu
    assert new.tolist() == bn
