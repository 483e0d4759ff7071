"""Pin the oracle's round logic to the reference's golden vectors (tests/golden/natcache_tiny.json, written by the
reference's own generate_speculative_natcache / generate_speculative_prefixcache / teacher_force_argmax on the tiny
CPU workload; see tests/golden/make_golden.py): ids, stats and the per-round trace (k, draft, ar_pred, new_tokens)
of natcache with full_draft True and False, the prefixcache ids (= AR greedy), and teacher forcing. Also: the
serving full-draft round commits exactly the AR ids on this workload."""
import json
import os

import pytest
import torch

from oracle.decoder import TINY, OracleDecoder, make_prefix, make_weights
from oracle.rounds import ar_generate, fulldraft_generate, natcache_generate, teacher_force_argmax

GOLDEN = os.path.join(os.path.dirname(__file__), "golden", "natcache_tiny.json")


@pytest.fixture(scope="module")
def setup():
    with open(GOLDEN) as f:
        g = json.load(f)
    torch.set_grad_enabled(False)
    w = make_weights(TINY, 0)
    vis, text = make_prefix(TINY, g["n_vis"], len(g["prefix_text_ids"]), 0)
    assert text.tolist() == g["prefix_text_ids"]
    dec = OracleDecoder(TINY, w)
    emb = torch.cat([vis, dec.embed(text)], 0)
    return g, dec, emb


@pytest.mark.parametrize("full_draft", [1, 0])
def test_natcache_equals_golden(setup, full_draft):
    g, dec, emb = setup
    trace = []
    ids, stats = natcache_generate(dec, emb, g["bd"], g["mask_id"], g["max_new_tokens"], full_draft=bool(full_draft),
                                   trace=trace)
    want = g[f"natcache_full_draft_{full_draft}"]
    assert ids == want["ids"]
    assert stats == want["stats"]
    assert trace == want["trace"]


def test_ar_equals_golden_prefixcache_and_teacher_force(setup):
    g, dec, emb = setup
    n = len(g["prefixcache"]["ids"])
    ar, _ = ar_generate(dec, emb, n)
    assert ar == g["prefixcache"]["ids"]
    assert ar[:len(g["natcache_full_draft_1"]["ids"])] == g["natcache_full_draft_1"]["ids"]
    assert teacher_force_argmax(dec, emb, g["natcache_full_draft_1"]["ids"]) == g["teacher_force_argmax"]


def test_fulldraft_round_commits_ar_ids(setup):
    g, dec, emb = setup
    out, rounds = fulldraft_generate(dec, emb, g["bd"], g["mask_id"], g["max_new_tokens"])
    ar, _ = ar_generate(dec, emb, len(out))
    assert out == ar
    assert all(0 <= r["acc"] <= g["bd"] for r in rounds)
