"""The block-diffusion decode on the GPU: gss_unmask_step against the oracle's unmask rule, the softmax argmax rule of
gss_argmax_accept, and the generate_cached / generate_cached_batched drop-ins on the reference's golden workload
(tests/golden/diffusion_tiny.json, written by the reference's own samplers).

  * unmask kernel: x1 and every unmask decision equal the oracle's rule (oracle/diffusion.py unmask_step) on the same
    logits exactly; conf within 1e-5 relative (the sum of exponentials runs in another order); decisions within
    1e-5 relative of the threshold are skipped. Edge rows: NaN, +inf, all -inf, ties, a seed equal to the mask id,
    blocks without masks, thresholds 0 and 1.
  * drop-in: every probe step of the GPU decode is replayed: its decisions are the oracle's rule applied to the GPU's
    own logits (exact), and those logits are within the bf16 tolerance of the fp32 oracle's forward of the same block
    over the same committed history; each seed is the greedy id of the commit forward's last row. commit_trace and
    commit_detail are the reference's records of those steps.
  * batched: each row of generate_cached_batched equals generate_cached of that crop alone, bit for bit (the kernels
    are batch invariant); stop ids cut each row at its first stop.
"""
import json
import os

import numpy as np
import pytest
import torch

from oracle.attention import window_mask
from oracle.decoder import TINY as O_TINY, KVCache, OracleDecoder, make_prefix
from oracle.diffusion import unmask_step as o_unmask
from oracle.rounds import causal_mask
from tests.helpers import LOGIT_ABS

pytestmark = pytest.mark.gpu

GOLDEN = os.path.join(os.path.dirname(__file__), "golden", "diffusion_tiny.json")
CONF_REL = 1e-5


def golden():
    with open(GOLDEN) as f:
        return json.load(f)


def tiny_model(dev, eos_id=None, stops=None):
    """The golden workload's model: crop i (image width 8 + i) = the i-th golden crop; the default crop is crop 0."""
    from gravityocr_amd.model import TINY, SyntheticGlmOcr, synthetic_weights
    g = golden()
    w = synthetic_weights(TINY, 0)
    crops = []
    for c in g["crops"]:
        vis, ids = make_prefix(O_TINY, c["n_vis"], len(c["text_ids"]), c["prefix_seed"])
        assert ids.tolist() == c["text_ids"]
        crops.append((vis, ids))
    m = SyntheticGlmOcr(TINY, w, crops[0][0], crops[0][1], mask_id=g["mask_id"], bd_size=g["bd"], eos_id=eos_id,
                        image_token_id=g["image_token_id"]).to(dev)
    for i, (vis, ids) in enumerate(crops):
        m.add_crop(8 + i, vis, ids)
    if stops is not None:
        m.glm.generation_config = type("GenerationConfig", (), {"eos_token_id": list(stops)})()
    return m, w, crops


def crop_image(i):
    from PIL import Image
    return Image.new("RGB", (8 + i, 8))


# ---------------------------------------------------------------------------------------------- unmask kernel ---
def check_unmask(logits, block, mask_id, threshold, out):
    """Compare the kernel's outputs (x1, conf, new block, n_unmasked, n_left, seed) for every sequence with the
    oracle's rule on the same logits (float32 of what the kernel read)."""
    x1, conf, blk, n_un, n_left, seed = out
    bs, W, V = logits.shape
    lg = logits.float().cpu()
    for b in range(bs):
        new, ox1, oconf, un = o_unmask(lg[b], block[b].long().cpu(), mask_id, threshold)
        assert x1[b].tolist() == ox1.tolist(), b
        np.testing.assert_allclose(conf[b].cpu().numpy(), oconf.numpy(), rtol=CONF_REL, equal_nan=True)
        near = torch.isfinite(oconf) & ((oconf - threshold).abs() <= CONF_REL * max(threshold, 1e-30))
        if bool(near.any()):
            continue                                       # a decision within rounding of the threshold
        assert blk[b].tolist() == new.tolist(), b
        assert int(n_un[b]) == int(un.sum())
        assert int(n_left[b]) == int((new == mask_id).sum())
        row = lg[b, -1]
        want_seed = 0 if (torch.isnan(row).any() or torch.isposinf(row).any() or torch.isneginf(row).all()) \
            else int(row.argmax())
        assert int(seed[b]) == want_seed


def run_unmask(logits, block, mask_id, threshold, ws=None):
    from gravityocr_amd.kernels import unmask_step, unmask_workspace_bytes
    bs, W, V = logits.shape
    dev = logits.device
    if ws is None:
        ws = torch.zeros(unmask_workspace_bytes(bs, W, V), dtype=torch.uint8, device=dev)
    i32 = dict(dtype=torch.int32, device=dev)
    blk = block.clone()
    x1, conf = torch.full((bs, W), -7, **i32), torch.full((bs, W), -7.0, device=dev)
    n_un, n_left, seed = torch.full((bs,), -7, **i32), torch.full((bs,), -7, **i32), torch.full((bs,), -7, **i32)
    unmask_step(logits, blk, ws, mask_id=mask_id, threshold=threshold, x1=x1, conf=conf, n_unmasked=n_un,
                n_left=n_left, seed=seed)
    torch.cuda.synchronize()
    return x1, conf, blk, n_un, n_left, seed


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
@pytest.mark.parametrize("bs,W,V", [(1, 1, 100), (1, 4, 4096), (3, 4, 4101), (2, 17, 59392), (1, 32, 59392),
                                    (4, 32, 5000)])
def test_unmask_kernel_equals_oracle(cuda, dtype, bs, W, V):
    g = torch.Generator().manual_seed(bs * 1000 + W * 10 + V)
    mask_id = V - 1
    for trial in range(4):
        logits = (torch.randn(bs, W, V, generator=g) * 3).to(dtype)
        block = torch.randint(0, V - 1, (bs, W), generator=g, dtype=torch.int32)
        masked = torch.rand(bs, W, generator=g) < 0.7
        block[masked] = mask_id
        if trial == 1:
            logits[0, 0, 5] = float("nan")                 # NaN row: argmax 0, conf NaN (forced position)
            block[0, 0] = mask_id                          # a masked seed position reads row 0
            if W > 2:
                logits[0, 1, V // 2] = float("inf")
                logits[0, 2] = float("-inf")
        if trial == 2:
            block[0] = 3                                   # a block without masks is left alone
            logits[:, :, 7] = logits[:, :, 3]              # ties in value: the lower index
        threshold = [0.5, 0.0, 0.9, 1.0][trial]
        out = run_unmask(logits.to(cuda), block.to(cuda), mask_id, threshold)
        check_unmask(logits, block, mask_id, threshold, out)


def test_unmask_kernel_reuses_its_workspace(cuda):
    """Counters are reset by the kernel: a workspace filled with garbage past the counters, then reused by calls of
    different shapes, gives the same results as a fresh one."""
    from gravityocr_amd.kernels import unmask_workspace_bytes
    ws = torch.full((unmask_workspace_bytes(3, 32, 59392),), 0xFF, dtype=torch.uint8, device=cuda)
    ws[:1024 * 9 * 128] = 0                                # the counter block
    g = torch.Generator().manual_seed(5)
    for bs, W, V in [(3, 32, 59392), (1, 4, 100), (2, 17, 9000), (3, 32, 59392)]:
        logits = torch.randn(bs, W, V, generator=g).bfloat16()
        block = torch.full((bs, W), V - 1, dtype=torch.int32)
        block[:, 0] = 1
        out = run_unmask(logits.to(cuda), block.to(cuda), V - 1, 0.002, ws=ws)
        check_unmask(logits, block, V - 1, 0.002, out)


def test_argmax_softmax_rule(cuda):
    from gravityocr_amd.kernels import ARGMAX_LAST_RAW, ARGMAX_SOFTMAX, argmax_accept, argmax_workspace_bytes
    V, W = 5000, 3
    lg = torch.randn(1, W, V)
    lg[0, 0, 17] = float("nan")
    lg[0, 1, 23] = float("inf")
    lg[0, 2, 31] = float("nan")
    lg = lg.to(cuda)
    ws = torch.zeros(argmax_workspace_bytes(1, W, V), dtype=torch.uint8, device=cuda)
    t = torch.zeros(1, W, dtype=torch.int32, device=cuda)
    results = {}
    for flags in (0, ARGMAX_SOFTMAX, ARGMAX_SOFTMAX | ARGMAX_LAST_RAW):
        argmax_accept(lg, t, ws, flags=flags)
        results[flags] = t[0].tolist()
    assert results[0] == [17, 23, 31]                               # torch.argmax of the logits: NaN, then +inf
    soft = torch.softmax(lg.float().cpu(), -1).argmax(-1)[0].tolist()
    assert results[ARGMAX_SOFTMAX] == soft == [0, 0, 0]             # argmax of an all-NaN softmax
    assert results[ARGMAX_SOFTMAX | ARGMAX_LAST_RAW] == [0, 0, 31]  # the bonus row keeps the raw rule


# ---------------------------------------------------------------------------------------------- drop-in ----------
def oracle_bf16(w):
    return OracleDecoder(O_TINY, {k: v.bfloat16().float() for k, v in w.items()})


def decode_with_steps(model, image, max_new, threshold, commit_causal=False):
    """Run the drop-in's decode loop through BlockDiffusionDecoder, recording every probe step (block before, GPU
    logits, x1, conf, block after, n_unmasked) and every block's commit logits row and seed."""
    from gravityocr_amd import fast_sampling as fs
    dev = next(model.parameters()).device
    bd, mask_id = int(model.bd_size), int(model.mask_id)
    input_ids, emb, positions, next_pos = fs.prepare_prompt(model, image, "Text Recognition:", 1344, dev)
    P = input_ids.shape[1]
    num_blocks = (max_new + bd - 1) // bd
    sess = fs._session(model, dev, P + num_blocks * bd + fs.PAGE)
    seed_logit = fs._prefill(sess.eng, emb, positions)
    seed = int(fs._argmax_rows(sess.eng, seed_logit.view(1, -1), softmax_rule=True)[0])
    dec = sess.diffusion_decoder(1, bd, mask_id, threshold, commit_causal)
    dec.start(torch.tensor([seed]), pos_delta=torch.tensor([next_pos - P]))
    blocks = []
    for blk in range(num_blocks):
        steps = []

        def on_step():
            steps.append({"before": dec.before[0].tolist(), "logits": dec.b.logits[:bd].float().cpu(),
                          "x1": dec.x1[0].tolist(), "conf": dec.conf[0].cpu(), "after": dec.block[0].tolist(),
                          "n_unmasked": int(dec.n_unmasked[0])})
        ids, seeds, n = dec.decode_block([seed], on_step)
        blocks.append({"seed": seed, "steps": steps, "ids": ids[0], "next_seed": seeds[0],
                       "commit_logits": dec.b.logits[bd - 1].float().cpu()})
        seed = seeds[0]
    return P, blocks


def replay(o, emb_pre, blocks, bd, mask_id, threshold, commit_causal=False):
    """Check every recorded step and commit against the oracle; returns the GPU's ids and the number of steps."""
    P = emb_pre.shape[0]
    cache = KVCache(o.cfg.n_layers)
    h = o.forward(emb_pre, torch.arange(P), cache, causal_mask(0, P))
    frozen = P
    n_steps = 0
    out = []
    for blk in blocks:
        pos = torch.arange(frozen, frozen + bd)
        for s in blk["steps"]:
            n_steps += 1
            # the rule, exactly, on the GPU's own logits
            new, x1, conf, un = o_unmask(s["logits"], torch.tensor(s["before"]), mask_id, threshold)
            assert s["x1"] == x1.tolist()
            np.testing.assert_allclose(s["conf"].numpy(), conf.numpy(), rtol=CONF_REL)
            near = (conf - threshold).abs() <= CONF_REL * threshold
            if not bool(near.any()):
                assert s["after"] == new.tolist() and s["n_unmasked"] == int(un.sum())
            # the GPU's logits: the fp32 oracle's forward of the same block over the same history
            cache.truncate(frozen)
            ol = o.logits(o.forward(o.embed(torch.tensor(s["before"])), pos, cache, window_mask(frozen, bd, 0)))
            assert float((ol - s["logits"]).abs().max()) <= LOGIT_ABS
        ids = blk["ids"]
        assert ids[0] == blk["seed"] and mask_id not in ids
        cache.truncate(frozen)
        hc = o.forward(o.embed(torch.tensor(ids)), pos, cache, window_mask(frozen, bd, bd if commit_causal else 0))
        ol = o.logits(hc[-1:])[0]
        assert float((ol - blk["commit_logits"]).abs().max()) <= LOGIT_ABS
        row = blk["commit_logits"]
        assert blk["next_seed"] == int(row.argmax())
        frozen += bd
        out.extend(ids)
    return out, n_steps


@pytest.mark.parametrize("causal", [False, True])
def test_cached_golden_workload_steps_match_oracle(cuda, causal):
    from gravityocr_amd.fast_sampling import generate_cached
    g = golden()
    bd, mask_id, thr, n = g["bd"], g["mask_id"], g["threshold"], g["max_new_tokens"]
    model, w, crops = tiny_model(cuda)
    P, blocks = decode_with_steps(model, crop_image(0), n, thr, commit_causal=causal)
    o = oracle_bf16(w)
    vis, ids = crops[0]
    emb_pre = torch.cat([vis.bfloat16().float(), o.embed(ids)], 0)
    gpu_ids, n_steps = replay(o, emb_pre, blocks, bd, mask_id, thr, commit_causal=causal)
    # the drop-in runs the same loop: the same ids, one trace entry per probe step, the reference's records
    trace, detail = [], []
    txt = generate_cached(model, crop_image(0), max_new_tokens=n, threshold=thr, commit_trace=trace,
                          commit_causal=causal, commit_detail=detail)
    assert [int(x) for x in txt.split()] == gpu_ids
    assert trace == [s["n_unmasked"] for b in blocks for s in b["steps"]]
    assert len(detail) == len(blocks) + sum(1 for b in blocks for s in b["steps"] if s["n_unmasked"])
    seeds = [d["tok"][0] for d in detail if d.get("is_seed")]
    assert seeds == [b["seed"] for b in blocks] == gpu_ids[::bd]
    ref = g[f"cached_commit_causal_{int(causal)}"]
    same = next((i for i, (a, b) in enumerate(zip(gpu_ids, ref["ids"])) if a != b), len(ref["ids"]))
    print(f"golden ids equal for {same} of {len(ref['ids'])} tokens; {n_steps} probe steps "
          f"(golden {len(ref['commit_trace'])})")


def test_cached_eos(cuda):
    from gravityocr_amd.fast_sampling import generate_cached
    g = golden()
    model = tiny_model(cuda)[0]
    full = [int(x) for x in generate_cached(model, crop_image(0), max_new_tokens=g["max_new_tokens"],
                                            threshold=g["threshold"]).split()]
    bd = g["bd"]
    eos = next(t for i, t in enumerate(full) if i > bd and i % bd and t not in full[:i])
    model_e = tiny_model(cuda, eos_id=eos)[0]
    txt = generate_cached(model_e, crop_image(0), max_new_tokens=g["max_new_tokens"], threshold=g["threshold"])
    assert [int(x) for x in txt.split()] == full[:full.index(eos)]
    # an EOS equal to the first block's seed ends the decode before any block
    model_s = tiny_model(cuda, eos_id=full[0])[0]
    assert generate_cached(model_s, crop_image(0), max_new_tokens=g["max_new_tokens"], threshold=g["threshold"]) == ""


def test_batched_rows_equal_single_decodes(cuda):
    from gravityocr_amd.fast_sampling import generate_cached
    from gravityocr_amd.fast_sampling_batched import generate_cached_batched
    g = golden()
    n, thr = g["max_new_tokens"], g["threshold"]
    model = tiny_model(cuda)[0]
    singles = [[int(x) for x in generate_cached(model, crop_image(i), max_new_tokens=n, threshold=thr).split()]
               for i in range(3)]
    rows = generate_cached_batched(model, [crop_image(i) for i in range(3)], max_new_tokens=n, threshold=thr)
    assert [[int(x) for x in r.split()] for r in rows] == singles
    # the same crops in another order, and a crop twice: each row is still its own decode
    rows = generate_cached_batched(model, [crop_image(2), crop_image(0), crop_image(2)], max_new_tokens=n,
                                   threshold=thr)
    assert [[int(x) for x in r.split()] for r in rows] == [singles[2], singles[0], singles[2]]
    # stop ids: a tokenizer EOS and a generation-config stop, first seen mid-row in rows 1 and 2
    s1 = next(t for i, t in enumerate(singles[1]) if i > 1 and t not in singles[1][:i])
    s2 = next(t for i, t in enumerate(singles[2]) if i > 1 and t not in singles[2][:i] and t != s1)
    model_s = tiny_model(cuda, eos_id=s1, stops=[s1, s2])[0]
    rows = generate_cached_batched(model_s, [crop_image(i) for i in range(3)], max_new_tokens=n, threshold=thr)

    def cut(r):
        stops = [k for k, t in enumerate(r) if t in (s1, s2)]
        return r[:stops[0]] if stops else r
    assert [[int(x) for x in r.split()] if r else [] for r in rows] == [cut(r) for r in singles]


def test_mid_model_steps_follow_the_rule(cuda):
    """The 1536-hidden decoder at bd 32 (the model's default block): the kernel's decisions on every probe step are
    the oracle's rule on the GPU's logits, and the decode ends every block with no mask left."""
    from gravityocr_amd.model import GlmTextConfig, SyntheticGlmOcr, synthetic_prompt, synthetic_weights
    cfg = GlmTextConfig(n_layers=4, hidden=1536, n_heads=16, n_kv_heads=2, head_dim=128, ffn=4608, vocab=59392)
    w = synthetic_weights(cfg, 7)
    vis, ids = synthetic_prompt(cfg, 700, 24, 7)
    model = SyntheticGlmOcr(cfg, w, vis, ids, mask_id=cfg.vocab - 1, bd_size=32,
                            image_token_id=cfg.vocab - 2).to(cuda)
    from PIL import Image
    # threshold 1: one position per step (bd - 1 steps per block); then the median confidence of the first step, so
    # that steps unmask several positions at once
    thr = 1.0
    for run in range(2):
        P, blocks = decode_with_steps(model, Image.new("RGB", (64, 48)), 64, thr)
        n_multi = 0
        for blk in blocks:
            assert cfg.vocab - 1 not in blk["ids"]
            for s in blk["steps"]:
                new, x1, conf, un = o_unmask(s["logits"], torch.tensor(s["before"]), cfg.vocab - 1, thr)
                assert s["x1"] == x1.tolist()
                np.testing.assert_allclose(s["conf"].numpy(), conf.numpy(), rtol=CONF_REL)
                if not bool(((conf - thr).abs() <= CONF_REL * thr).any()):
                    assert s["after"] == new.tolist()
                n_multi += s["n_unmasked"] > 1
            assert blk["next_seed"] == int(blk["commit_logits"].argmax())
        steps = [len(b["steps"]) for b in blocks]
        print(f"threshold {thr:.3g}: probe steps per block {steps}, steps unmasking > 1: {n_multi}")
        if run == 0:
            assert steps == [31, 31] and n_multi == 0
            thr = float(blocks[0]["steps"][0]["conf"][1:].median())
        else:
            assert n_multi > 0 and max(steps) < 31
