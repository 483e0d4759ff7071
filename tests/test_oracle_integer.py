"""Pin the integer half of the oracle (argmax, chain accept, commit packing, slots, finish rules) against library
routines, the published tree-verify walk, the reference's own post-commit invariants and brute force; and check the
product's host finish rules against the oracle's per-token loop."""
import numpy as np
import torch
from hypothesis import given, settings
from hypothesis import strategies as st

from oracle.integer import (kv_meta, accept_chain, argmax_first, bf16_bits_to_f32, chain_links, committed_tokens,
                            cut_index_loop, f32_to_bf16_bits, host_commit_loop, page_slot, ss_commit,
                            verify_tree_greedy)


def brute_argmax(row):
    best = 0
    for i in range(1, len(row)):
        a, b = row[i], row[best]
        if (np.isnan(a) and not np.isnan(b)) or (not np.isnan(a) and not np.isnan(b) and a > b):
            best = i
    return best


def test_argmax_first_matches_torch_and_brute_force():
    g = np.random.default_rng(0)
    x = g.integers(-3, 4, size=(200, 37)).astype(np.float32)       # many exact ties
    x[5, 7] = np.nan
    x[6, :] = -np.inf
    x[7, [3, 9]] = np.nan
    got = argmax_first(x)
    np.testing.assert_array_equal(got, torch.from_numpy(x).argmax(-1).numpy())
    assert [brute_argmax(r) for r in x] == got.tolist()


def test_softmax_argmax_equals_raw_argmax_on_bf16():
    # the reference's greedy rule (fp32 softmax then argmax) vs the raw-logit rule the kernel implements
    g = np.random.default_rng(1)
    x = torch.from_numpy(g.standard_normal((500, 4096)).astype(np.float32) * 3).bfloat16()
    x[:50, 100] = x[:50].float().max(-1).values.bfloat16()       # planted exact ties
    sm = torch.softmax(x.float(), -1).argmax(-1).numpy()
    np.testing.assert_array_equal(sm, argmax_first(x.float().numpy()))


def test_bf16_bits_roundtrip_matches_torch():
    g = np.random.default_rng(2)
    x = np.concatenate([g.standard_normal(10000).astype(np.float32) * 1e3, [0.0, -0.0, np.inf, -np.inf, 1e-40]])
    bits = f32_to_bf16_bits(x.astype(np.float32))
    ref = torch.from_numpy(x.astype(np.float32)).bfloat16().view(torch.int16).numpy().view(np.uint16)
    np.testing.assert_array_equal(bits, ref)
    np.testing.assert_array_equal(bf16_bits_to_f32(bits), torch.from_numpy(x).bfloat16().float().numpy())


@settings(max_examples=300, deadline=None)
@given(st.integers(1, 4), st.integers(2, 9), st.integers(0, 10**6))
def test_accept_chain_equals_tree_walk(bs, K, seed):
    g = np.random.default_rng(seed)
    V = 3                                  # tiny vocab: long accepted runs and mismatches both common
    window = g.integers(0, V, (bs, K))
    target = g.integers(0, V, (bs, K))
    acc = accept_chain(window, target)
    ri, nxt, sib = chain_links(bs, K)
    predicts, acc_idx, acc_num = verify_tree_greedy(window, target.reshape(-1), ri, nxt, sib)
    np.testing.assert_array_equal(acc, acc_num)
    for b in range(bs):
        a = int(acc[b])
        assert all(target[b, r] == window[b, r + 1] for r in range(a))
        assert a == K - 1 or target[b, a] != window[b, a + 1]
        assert list(acc_idx[b, : a + 1]) == [b * K + r for r in range(a + 1)]
        assert all(v == -1 for v in acc_idx[b, a + 1:])
        # predicts at the accepted rows are the target tokens: T = [a0, t_0..t_acc]
        assert [int(predicts[b * K + r]) for r in range(a + 1)] == list(target[b, : a + 1])
        T = committed_tokens(window[b, 0], target[b], a)
        assert len(T) == a + 2


def test_tree_walk_on_a_branching_tree():
    # root(0) -> children 1 (token 5) and 2 (token 7); 2 -> 3 (token 9). target after root is 7, after node 2 is 9.
    cand = np.array([[0, 5, 7, 9]])
    target = np.array([7, 0, 9, 4])
    ri = np.array([[0, 1, 2, 3]])
    nxt = np.array([[1, -1, 3, -1]])
    sib = np.array([[-1, 2, -1, -1]])
    predicts, idx, num = verify_tree_greedy(cand, target, ri, nxt, sib)
    assert num[0] == 2 and list(idx[0, :3]) == [0, 2, 3]
    assert predicts[0] == 7 and predicts[2] == 9 and predicts[3] == 4


@settings(max_examples=200, deadline=None)
@given(st.integers(1, 6), st.integers(2, 8), st.integers(0, 10**6))
def test_ss_commit_reference_invariants(bs, K, seed):
    # the reference's post-commit checks (selfspec_fast_commit.py:454-477), restated independently
    g = np.random.default_rng(seed)
    predict = g.integers(0, 1000, bs * K + 1)
    acc = g.integers(0, K, bs)
    a0 = g.integers(0, 1000, bs)
    rpi = g.permutation(bs + 3)[:bs]
    seeds = np.zeros(bs + 3, dtype=np.int64)
    seq = g.integers(0, 5000, bs)
    loc = g.integers(0, 10**6, bs * K)
    packed, seeds2, seq2, free, out, cut = ss_commit(predict, acc, a0, rpi, seeds, seq, loc, K)
    assert cut.tolist() == (acc + 1).tolist()
    want_free = [int(loc[i * K + t]) for i in range(bs) for t in range(int(acc[i]) + 1, K)]
    assert free.tolist() == want_free
    assert len(free) == int(sum(K - 1 - acc))
    for i in range(bs):
        a = int(acc[i])
        assert packed[i, 0] == a0[i] and packed[i, 1] == a
        assert out[i] == packed[i, 2 + a] == seeds2[rpi[i]] == predict[i * K + a]
        assert seq2[i] == seq[i] + a + 1
        assert all(packed[i, 2 + j] == 0 for j in range(a + 1, K))


@settings(max_examples=100, deadline=None)
@given(st.integers(1, 9), st.integers(0, 33), st.integers(0, 10**6))
def test_kv_meta_equals_reference_host_plan_and_check(bs, extra, seed):
    # the reference's host plan (selfspec_fast_attn.py:244-253: kv_indptr = cumsum(seq_lens_cpu + n)) and its
    # SELFSPEC_CHECK comparison (:267-283: kv_indices == concatenated req_to_token rows), restated with numpy
    g = np.random.default_rng(seed)
    pool, ctx = bs + 4, 300
    r2t = g.integers(0, 10**6, (pool, ctx)).astype(np.int32)
    rpi = g.permutation(pool)[:bs]
    sl = g.integers(0, ctx - extra, bs)
    indptr, idx = kv_meta(r2t, rpi, sl, extra)
    assert indptr.tolist() == [0] + np.cumsum(sl + extra).tolist()
    assert idx.tolist() == np.concatenate([r2t[rpi[i], : sl[i] + extra] for i in range(bs)]).tolist()


def test_page_slot_is_flattened_page_order():
    g = np.random.default_rng(3)
    pt = g.permutation(40)[:12]
    flat = [p * 16 + o for p in pt for o in range(16)]     # the sequence's slots laid out page by page
    for pos in range(12 * 16):
        assert page_slot(pt, pos) == flat[pos]


@settings(max_examples=300, deadline=None)
@given(st.integers(1, 6), st.integers(2, 20), st.sampled_from([1, 4, 16]), st.integers(0, 10**6))
def test_ss_commit_paged_frees_by_page_sets(bs, K, page, seed):
    """The free list of the paged commit, against its definition as page sets: each request's slots are page-aligned
    (its own shuffled pages, position p at page_table[p // page] * page + p % page); after the cut j the kept
    positions are [0, S + j); a verify slot is freed iff its page holds no kept position. The finish rule's cut is
    checked against the per-token loop by the same function (rows with budget < 0 keep every token)."""
    g = np.random.default_rng(seed)
    n_pages = 64
    predict = g.integers(-1, 12, bs * K + 1)
    acc = g.integers(0, K, bs)
    a0 = g.integers(0, 12, bs)
    rpi = g.permutation(bs + 3)[:bs]
    seeds = np.zeros(bs + 3, dtype=np.int64)
    S = g.integers(0, 40, bs)
    pts = [g.permutation(n_pages) + 1000 * (i + 1) for i in range(bs)]   # disjoint page ids per request
    loc = np.array([pts[i][(S[i] + r) // page] * page + (S[i] + r) % page for i in range(bs) for r in range(K)])
    budgets = [int(x) for x in g.integers(-1, 2 * K, bs)]
    stops = [set(int(x) for x in g.integers(0, 12, 2)) for _ in range(bs)]
    vocabs = [int(x) for x in g.integers(5, 12, bs)]
    packed, _, seq2, free, _, cut = ss_commit(predict, acc, a0, rpi, seeds, S, loc, K, page=page,
                                              finish=(budgets, stops, vocabs))
    want_free = []
    for i in range(bs):
        a = int(acc[i])
        T = [int(a0[i])] + [int(predict[i * K + t]) for t in range(a + 1)]
        j = a + 1 if budgets[i] < 0 else cut_index_loop(T, budgets[i], stops[i], vocabs[i])
        assert cut[i] == j and seq2[i] == S[i] + j
        kept_pages = {int(pts[i][p // page]) for p in range(int(S[i]) + j)}
        want_free += [int(loc[i * K + r]) for r in range(K) if r >= j and int(loc[i * K + r]) // page not in kept_pages]
    assert free.tolist() == want_free


class _SP:
    def __init__(self, max_new):
        self.max_new_tokens, self.stop_token_ids, self.ignore_eos = max_new, [3], False
        self.stop_strs, self.stop_regex_strs = [], []


class _Req:
    """minimal request: finishes on length, stop id or vocab boundary, checked on the appended tokens."""

    def __init__(self, max_new, vocab):
        self.sampling_params, self.vocab_size = _SP(max_new), vocab
        self.output_ids, self.eos_token_ids, self.tokenizer, self.grammar, self.to_finish = [], [7], None, None, None
        self.spec_verify_ct = self.spec_accepted_tokens = 0
        self.hist, self._fin = [], False

    def finished(self):
        return self._fin

    def check_finished(self, new_accepted_len=1):
        sp = self.sampling_params
        for x in self.output_ids[-new_accepted_len:]:
            if len(self.output_ids) >= sp.max_new_tokens or x in (3, 7) or x > self.vocab_size or x < 0:
                self._fin = True

    def update_spec_acceptance_histogram(self, n):
        self.hist.append(n)


@settings(max_examples=300, deadline=None)
@given(st.lists(st.integers(-2, 12), min_size=1, max_size=10), st.integers(1, 12), st.integers(0, 5),
       st.integers(5, 11))
def test_cut_index_loop_equals_request_appends(T, max_new, prior, vocab):
    """The oracle's per-token cut against a request object that appends T one token at a time and runs its own
    finish check after each append (length, stop ids 3 and 7, vocabulary bound), starting from ``prior`` tokens."""
    req = _Req(max_new + prior, vocab)
    req.output_ids = [0] * prior
    j = len(T) - 1
    for t, x in enumerate(T):
        req.output_ids.append(x)
        req.check_finished()
        if req.finished():
            j = t
            break
    assert cut_index_loop(T, max_new, {3, 7}, vocab) == j
