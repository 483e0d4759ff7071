"""The drop-in entry points of gravityocr_amd/fast_sampling.py on the GPU, on the reference's golden workload (tiny
decoder, natcache bd 4, 64 new tokens; tests/golden/natcache_tiny.json, written by the reference's own
generate_speculative_natcache) and on a 4-layer 1536-hidden decoder:

  * every round of the GPU decode, replayed through the fp32 oracle on the GPU's own history: each draft token and
    each ar_pred token is an argmax of the oracle's logits to within 2 x the bf16 logit tolerance, and k / new
    follow from draft and ar_pred by the accept rule exactly (src/fast_sampling.py:562-584);
  * the golden ids and trace are reproduced up to the first position where the fp32 oracle itself has a near tie;
  * the committed ids equal the engine's own AR greedy decode bit for bit, for any draft_bd (the reference's
    K-invariance, src/fast_sampling.py:436-439), with the EOS cut and the max_new_tokens overshoot rule;
  * teacher_force_argmax agrees with the oracle's teacher forcing to the same tolerance;
  * the M-RoPE prefill rotation equals transformers' GlmOcrTextRotaryEmbedding + apply_rotary_pos_emb.
"""
import json
import os

import numpy as np
import pytest
import torch

from oracle.attention import window_mask
from oracle.decoder import TINY as O_TINY, KVCache, OracleDecoder, make_prefix, make_weights
from oracle.rounds import causal_mask, teacher_force_argmax as o_teacher_force
from tests.helpers import LOGIT_ABS

pytestmark = pytest.mark.gpu

GOLDEN = os.path.join(os.path.dirname(__file__), "golden", "natcache_tiny.json")
TOL = 2 * LOGIT_ABS      # a GPU argmax may differ from the oracle's only where the oracle's top-2 gap is below this


def golden():
    with open(GOLDEN) as f:
        return json.load(f)


def tiny_model(dev, eos_id=None):
    from gravityocr_amd.model import TINY, SyntheticGlmOcr, synthetic_weights
    g = golden()
    w = synthetic_weights(TINY, 0)
    vis, ids = make_prefix(O_TINY, g["n_vis"], len(g["prefix_text_ids"]), 0)
    assert ids.tolist() == g["prefix_text_ids"]
    m = SyntheticGlmOcr(TINY, w, vis, ids, mask_id=g["mask_id"], bd_size=g["bd"], eos_id=eos_id,
                        image_token_id=g["image_token_id"]).to(dev)
    return m, w, vis, ids


def mid_model(dev, eos_id=None, bd=16):
    from gravityocr_amd.model import GlmTextConfig, SyntheticGlmOcr, synthetic_prompt, synthetic_weights
    cfg = GlmTextConfig(n_layers=4, hidden=1536, n_heads=16, n_kv_heads=2, head_dim=128, ffn=4608, vocab=59392)
    w = synthetic_weights(cfg, 7)
    vis, ids = synthetic_prompt(cfg, 700, 24, 7)
    return SyntheticGlmOcr(cfg, w, vis, ids, mask_id=cfg.vocab - 1, bd_size=bd, eos_id=eos_id,
                           image_token_id=cfg.vocab - 2).to(dev)


def image():
    from PIL import Image
    return Image.new("RGB", (64, 48))


def near_argmax(logits_row, tok):
    row = logits_row.float()
    return float(row[tok]) >= float(row.max()) - TOL


def oracle_bf16(w):
    return OracleDecoder(O_TINY, {k: v.bfloat16().float() for k, v in w.items()})


def replay_round(o, emb_pre, hist, draft, bd, mask_id):
    """The oracle's draft-row logits and verify-row logits of the natcache round that starts after the committed
    tokens ``hist`` (cache = prompt + hist[:-1], pending = hist[-1]; round 0: no pending, seed = prefill logit),
    with the verify window built from the GPU's ``draft``. Returns (draft_logits [bd+1, V], pred [bd+1, V],
    bonus_logits [V])."""
    pre = 1 if hist else 0
    ctx = torch.tensor(hist[:-1], dtype=torch.long)
    emb = torch.cat([emb_pre, o.embed(ctx)], 0) if len(ctx) else emb_pre
    clen = emb.shape[0]
    cache = KVCache(o.cfg.n_layers)
    h = o.forward(emb, torch.arange(clen), cache, causal_mask(0, clen))
    seed = o.logits(h[-1:])
    ids = torch.tensor(([hist[-1]] if pre else []) + [mask_id] * bd)
    Q = ids.shape[0]
    raw = o.logits(o.forward(o.embed(ids), torch.arange(clen, clen + Q), cache, window_mask(clen, Q, pre)))
    draft_logits = raw if pre else torch.cat([seed, raw], 0)
    cache.truncate(clen)
    ids_v = torch.tensor(([hist[-1]] if pre else []) + list(draft))
    Qv = ids_v.shape[0]
    lv = o.logits(o.forward(o.embed(ids_v), torch.arange(clen, clen + Qv), cache, window_mask(clen, Qv, Qv)))
    pred = torch.cat([lv[:1] if pre else seed, lv[:-1]], 0)[pre:]
    return draft_logits, pred, lv[-1]


def check_trace_against_oracle(o, emb_pre, trace, bd, mask_id):
    hist = []
    for t in trace:
        draft, ar_pred, new, k = t["draft"], t["ar_pred"], t["new_tokens"], t["k"]
        assert len(draft) == bd + 1 and len(ar_pred) == bd + 1 and ar_pred[0] == draft[0]
        # integer rule, exact
        mism = [j for j in range(bd + 1) if draft[j] != ar_pred[j]]
        assert k == (mism[0] if mism else bd + 1), t
        dl, pred, bonus = replay_round(o, emb_pre, hist, draft, bd, mask_id)
        for j in range(bd + 1):
            assert near_argmax(dl[j], draft[j]), (t["round"], "draft", j)
            assert near_argmax(pred[j], ar_pred[j]), (t["round"], "ar_pred", j)
        if k <= bd:
            assert new == draft[:k] + [ar_pred[k]], t
        else:
            assert new[:-1] == draft and near_argmax(bonus, new[-1]), t
        hist = hist + new
    return hist


def test_natcache_golden_workload_rounds_match_oracle(cuda):
    from gravityocr_amd.fast_sampling import generate_speculative_natcache
    g = golden()
    model, w, vis, ids = tiny_model(cuda)
    trace = []
    txt, stats = generate_speculative_natcache(model, image(), max_new_tokens=g["max_new_tokens"], return_stats=True,
                                               trace=trace)
    gen = [int(x) for x in txt.split()]
    o = oracle_bf16(w)
    emb_pre = torch.cat([vis.bfloat16().float(), o.embed(ids)], 0)
    hist = check_trace_against_oracle(o, emb_pre, trace, g["bd"], g["mask_id"])
    assert hist == gen
    assert stats["rounds"] == len(trace) and stats["resp_tokens"] == len(gen)
    assert stats["total_fwd"] == 2 * len(trace) and stats["commit_fwd"] == 0
    # the golden vectors (the reference's own function, fp32): every committed id, and, round by round, the accept
    # index k, the committed tokens and the entries that decide them (the accepted drafts d[:k] and ar_pred[:k+1])
    # until a round where a deciding entry differs. There the first differing entry must be a near tie of the
    # oracle's row for both choices (the GPU's bf16 argmax and the reference's fp32 one); past it the round
    # boundaries may shift, the ids cannot (both decodes commit AR greedy ids). Entries past a round's mismatch
    # decide nothing.
    ref = g["natcache_full_draft_1"]
    bd, mask_id = g["bd"], g["mask_id"]
    assert gen == ref["ids"] and len(gen) == 69
    assert stats["resp_tokens"] == ref["stats"]["resp_tokens"] == 69
    hist, n_equal, n_tail_diff, split = [], 0, 0, None
    for t, r in zip(trace, ref["trace"]):
        k = t["k"]
        if (t["k"], t["new_tokens"]) == (r["k"], r["new_tokens"]) and t["draft"][:k] == r["draft"][:k] and \
                t["ar_pred"][:k + 1] == r["ar_pred"][:k + 1]:
            n_tail_diff += sum(a != b for a, b in zip(t["draft"][k:] + t["ar_pred"][k + 1:],
                                                         r["draft"][k:] + r["ar_pred"][k + 1:]))
            hist += t["new_tokens"]
            n_equal += 1
            continue
        j = next(j for j in range(bd + 1) if t["draft"][j] != r["draft"][j] or t["ar_pred"][j] != r["ar_pred"][j])
        dl, pred, _ = replay_round(o, emb_pre, hist, t["draft"], bd, mask_id)
        kind, row = ("draft", dl[j]) if t["draft"][j] != r["draft"][j] else ("ar_pred", pred[j])
        ours, theirs = t[kind][j], r[kind][j]
        assert near_argmax(row, ours) and near_argmax(row, theirs), (t["round"], kind, j, ours, theirs)
        split = (t["round"], kind, j, float(row.float()[ours] - row.float()[theirs]))
        break
    if split is None:
        assert stats == ref["stats"] and len(trace) == len(ref["trace"]) == 18
    else:
        assert n_equal >= 1
    print(f"golden: all {len(gen)} ids equal; {n_equal} of {len(ref['trace'])} rounds equal in k, committed tokens and "
          f"deciding entries ({n_tail_diff} undecisive entries differ)"
          + ("" if split is None else f"; round {split[0]} {split[1]}[{split[2]}] differs at a near tie of the oracle "
                                      f"(logit difference {split[3]:+.4f}), from there the round boundaries shift"))


def test_prefixcache_golden_ids_and_stats(cuda):
    """generate_speculative_prefixcache on the golden workload: the ids of the reference's own function (its causal
    verify makes them AR greedy ids), every stats key, and trace entries with the reference's keys whose committed
    tokens and ar_pred[0] (the seed) follow the accept rule."""
    from gravityocr_amd.fast_sampling import generate_speculative_prefixcache
    g = golden()
    model = tiny_model(cuda)[0]
    trace = []
    txt, stats = generate_speculative_prefixcache(model, image(), max_new_tokens=g["max_new_tokens"],
                                                  return_stats=True, trace=trace)
    ids = [int(x) for x in txt.split()]
    ref = g["prefixcache"]
    assert ids == ref["ids"]
    assert set(stats) == set(ref["stats"]) and stats["resp_tokens"] == ref["stats"]["resp_tokens"]
    assert stats["total_fwd"] == 2 * stats["rounds"] == 2 * len(trace)
    hist = []
    for t in trace:
        assert list(t) == ["round", "k", "seed", "draft", "ar_pred", "new_tokens"]
        assert t["seed"] == t["ar_pred"][0]
        k = t["k"]
        want = t["draft"][:k] + ([t["ar_pred"][k]] if k < len(t["draft"]) else t["new_tokens"][-1:])
        assert t["new_tokens"] == want
        hist += t["new_tokens"]
    assert hist[:len(ids)] == ids
    print(f"prefixcache: {len(ids)} golden ids, stats {stats} (reference {ref['stats']})")


def engine_ar(model, n):
    """The engine's own AR greedy decode (one-row verify forwards) from the drop-in's session."""
    from gravityocr_amd import fast_sampling as fs
    sess = fs._SESSIONS[model]
    dec = sess.decoder(int(model.bd_size), int(model.mask_id))
    dev = sess.eng.device
    input_ids, emb, positions, next_pos = fs.prepare_prompt(model, image(), "Text Recognition:", 1344, dev)
    last = fs._prefill(sess.eng, emb, positions)
    a0 = fs._argmax_rows(sess.eng, last.view(1, -1))
    dec.start(a0, pos_delta=torch.zeros(1, dtype=torch.int32, device=dev))
    for _ in range(n - 1):
        dec.ar_step()
    torch.cuda.synchronize()
    return [int(a0[0])] + dec.ar_log[:n - 1, 0].cpu().tolist()


@pytest.mark.parametrize("which", ["tiny", "mid"])
def test_natcache_equals_engine_ar_for_any_draft_bd(cuda, which):
    from gravityocr_amd.fast_sampling import generate_speculative_natcache
    model = tiny_model(cuda)[0] if which == "tiny" else mid_model(cuda)
    n = 96 if which == "tiny" else 160
    outs = {}
    for bd in ([None, 2, 7] if which == "tiny" else [None, 8]):
        st = {}
        trace = []
        txt, st = generate_speculative_natcache(model, image(), max_new_tokens=n, draft_bd=bd, return_stats=True,
                                                trace=trace)
        ids = [int(x) for x in txt.split()]
        K = (bd or model.bd_size) + 2
        assert n <= len(ids) < n + K, (bd, len(ids))          # the last round may overshoot by up to bd + 1
        outs[bd] = ids
        print(which, "draft_bd", bd, st)
    ar = engine_ar(model, max(len(v) for v in outs.values()))
    for bd, ids in outs.items():
        assert ids == ar[:len(ids)], bd


def test_natcache_eos_cut(cuda):
    from gravityocr_amd.fast_sampling import generate_speculative_natcache
    model = tiny_model(cuda)[0]
    full = [int(x) for x in generate_speculative_natcache(model, image(), max_new_tokens=64).split()]
    # an EOS id that first appears mid-sequence (the latest such position within the first 40 tokens)
    firsts = [i for i in range(1, min(40, len(full))) if full[i] not in full[:i]]
    assert firsts, full
    i = firsts[-1]
    eos = full[i]
    model_e = tiny_model(cuda, eos_id=eos)[0]
    trace = []
    txt, st = generate_speculative_natcache(model_e, image(), max_new_tokens=64, return_stats=True, trace=trace)
    ids = [int(x) for x in txt.split()] if txt else []
    assert ids == full[:i]
    assert eos in trace[-1]["new_tokens"] and all(eos not in t["new_tokens"] for t in trace[:-1])
    assert st["resp_tokens"] == i


def test_teacher_force_argmax_matches_oracle(cuda):
    from gravityocr_amd.fast_sampling import generate_speculative_natcache, teacher_force_argmax
    model, w, vis, ids = tiny_model(cuda)
    gen = [int(x) for x in generate_speculative_natcache(model, image(), max_new_tokens=40).split()]
    gen[5] = (gen[5] + 17) % 4000                      # a wrong token: the AR prediction after it still follows
    tf = teacher_force_argmax(model, image(), "Text Recognition:", gen)
    assert len(tf) == len(gen)
    o = oracle_bf16(w)
    emb_pre = torch.cat([vis.bfloat16().float(), o.embed(ids)], 0)
    ref = o_teacher_force(o, emb_pre, gen)
    P, T = emb_pre.shape[0], emb_pre.shape[0] + len(gen)
    lg = o.logits(o.forward(torch.cat([emb_pre, o.embed(torch.tensor(gen))], 0), torch.arange(T),
                            KVCache(O_TINY.n_layers), causal_mask(0, T)))[P - 1:T - 1]
    for i, (a, b) in enumerate(zip(tf, ref)):
        assert a == b or near_argmax(lg[i], a), i
    assert teacher_force_argmax(model, image(), "Text Recognition:", []) == []


def test_mrope_prefill_rotation_matches_transformers(cuda):
    from transformers.models.glm_ocr.configuration_glm_ocr import GlmOcrTextConfig
    from transformers.models.glm_ocr.modeling_glm_ocr import GlmOcrTextRotaryEmbedding, apply_rotary_pos_emb
    from gravityocr_amd.kernels import rope_stage_mrope
    from gravityocr_amd.model import SYNTH_1536 as cfg
    hc = GlmOcrTextConfig(hidden_size=cfg.hidden, num_attention_heads=cfg.n_heads,
                          num_key_value_heads=cfg.n_kv_heads, head_dim=cfg.head_dim,
                          rope_parameters={"rope_type": "default", "rope_theta": cfg.rope_theta,
                                           "partial_rotary_factor": cfg.partial_rotary,
                                           "mrope_section": list(cfg.mrope_section)})
    rot = GlmOcrTextRotaryEmbedding(hc)
    g = torch.Generator().manual_seed(11)
    P, Hq, Hkv, D = 300, cfg.n_heads, cfg.n_kv_heads, cfg.head_dim
    pos = torch.stack([torch.randint(0, 40, (P,), generator=g), torch.randint(0, 60, (P,), generator=g),
                       torch.randint(0, 90, (P,), generator=g)], 1)
    pos[:50] = torch.arange(50)[:, None] + 1000                      # some text rows: all three equal
    qkv = torch.randn(P, (Hq + 2 * Hkv) * D, generator=g).bfloat16()
    x = qkv[:, :(Hq + Hkv) * D].view(P, Hq + Hkv, D)
    cos, sin = rot(x, pos.t()[:, None, :])                           # position_ids [3, 1, P]
    qh = x[:, :Hq].transpose(0, 1)[None]                              # [1, Hq, P, D]
    kh = x[:, Hq:].transpose(0, 1)[None]
    rq, rk = apply_rotary_pos_emb(qh, kh, cos, sin)
    q = torch.empty(P, Hq, D, dtype=torch.bfloat16, device=cuda)
    k = torch.empty(P, Hkv, D, dtype=torch.bfloat16, device=cuda)
    v = torch.empty_like(k)
    inv = rot.inv_freq.float().to(cuda)
    rope_stage_mrope(qkv.to(cuda), pos.to(torch.int32).to(cuda), inv, q, k, v, sections=cfg.mrope_section,
                     rot_dim=cfg.rot_dim)
    torch.cuda.synchronize()
    from tests.test_gpu_layer import ulp_close
    ulp_close(q.cpu(), rq[0].transpose(0, 1))
    ulp_close(k.cpu(), rk[0].transpose(0, 1))
    assert torch.equal(v.cpu(), qkv[:, (Hq + Hkv) * D:].view(P, Hkv, D))
