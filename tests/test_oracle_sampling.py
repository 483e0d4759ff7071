"""Pins the sampled-verify oracle (oracle/sampling.py) without the reference's torch / sglang code:
the top-k / top-p filters against their definitions by brute force (ties included), the in-block penalties against
AR decode simulated token by token (the reference's own validation method, selfspec_sampling.py:1-24), the
inverse-CDF draw at its breakpoints, and speculative sampling against the identity it must satisfy: the first
committed token is distributed as AR's row 0 whatever the draft token (integrated over a grid of coins and
uniforms)."""
import numpy as np
import pytest

from oracle import sampling as S


def brute_joint(p, k, top_p):
    keep = np.array([(np.sum(p > p[q]) < k) and (p[p > p[q]].sum() < top_p or top_p >= 1.0) for q in range(len(p))])
    q = np.where(keep, p, 0.0)
    return q / q.sum()


def brute_torch(p, k, top_p, min_p):
    order = sorted(range(len(p)), key=lambda i: (-p[i], i))   # descending, equal values by index
    keep = np.zeros(len(p), dtype=bool)
    before = 0.0
    for rank, i in enumerate(order):
        keep[i] = rank < k and not (before > top_p) and not (min_p > 0 and p[i] < p[order[0]] * min_p)
        before += p[i]
    q = np.where(keep, p, 0.0)
    return q / q.sum()


@pytest.mark.parametrize("seed", range(6))
def test_filters_match_definitions(seed):
    g = np.random.default_rng(seed)
    V = 40
    logits = g.normal(size=V) * 2
    logits[g.integers(0, V, 6)] = logits[3]            # ties
    for T in (0.5, 1.0, 1.7):
        p = S.softmax_t(logits, T)
        for k in (1, 3, 7, V):
            for top_p in (0.1, 0.5, 0.9, 1.0):
                np.testing.assert_allclose(S.joint_top_k_top_p(p, k, top_p), brute_joint(p, k, top_p), rtol=0,
                                           atol=1e-12)
                for min_p in (0.0, 0.05, 0.3):
                    np.testing.assert_allclose(S.torch_backend_filter(p, k, top_p, min_p, min_p > 0),
                                               brute_torch(p, k, top_p, min_p), rtol=0, atol=1e-12)


def brute_fi_min_p(p, k, top_p, min_p):
    """The three flashinfer steps one token at a time, each on the previous step's renormalized vector."""
    def renorm(keep, x):
        y = np.array([x[i] if keep[i] else 0.0 for i in range(len(x))])
        return y / y.sum()
    q = renorm([sum(1 for v in p if v > p[i]) < k for i in range(len(p))], p)
    q = renorm([top_p >= 1.0 or sum(v for v in q if v > q[i]) < top_p for i in range(len(q))], q)
    return renorm([q[i] >= max(q) * min_p for i in range(len(q))], q)


def test_flashinfer_min_p_chain_known_answers():
    """Hand-worked rows. [0.4, 0.3, 0.2, 0.1], k = 2, top_p = 0.5: top-k leaves [4/7, 3/7]; the second token has 4/7
    above it, so top-p keeps only the first (the joint filter, which tests top-p on the unrenormalized mass 0.4, keeps
    both). [0.5, 0.3, 0.15, 0.05], k = 3, top_p = 0.9, min_p = 0.4: top-k renorm [10/19, 6/19, 3/19]; top-p keeps
    all three (16/19 < 0.9); min-p drops 3/19 < 0.4 * 10/19, leaving [5/8, 3/8]."""
    np.testing.assert_allclose(S.flashinfer_min_p_chain(np.array([0.4, 0.3, 0.2, 0.1]), 2, 0.5, 0.0),
                               [1.0, 0.0, 0.0, 0.0], rtol=0, atol=1e-15)
    np.testing.assert_allclose(S.joint_top_k_top_p(np.array([0.4, 0.3, 0.2, 0.1]), 2, 0.5),
                               [4 / 7, 3 / 7, 0.0, 0.0], rtol=0, atol=1e-15)
    np.testing.assert_allclose(S.flashinfer_min_p_chain(np.array([0.5, 0.3, 0.15, 0.05]), 3, 0.9, 0.4),
                               [0.625, 0.375, 0.0, 0.0], rtol=0, atol=1e-15)
    # min_p = 0 with neutral top-k / top-p: the untouched distribution
    p = np.array([0.25, 0.5, 0.125, 0.125])
    np.testing.assert_array_equal(S.flashinfer_min_p_chain(p, 5, 1.0, 0.0), p)


@pytest.mark.parametrize("seed", range(4))
def test_flashinfer_min_p_chain_definitions_and_reductions(seed):
    """Brute force (ties included), and the special cases that reduce to filters pinned above: no top-k / top-p ->
    the pytorch backend's min-p alone; min_p = 0 and top_p = 1 -> the joint filter's top-k; min_p = 0 and no top-k ->
    the joint filter's top-p."""
    g = np.random.default_rng(100 + seed)
    V = 32
    logits = g.normal(size=V) * 2
    logits[g.integers(0, V, 5)] = logits[7]
    for T in (0.6, 1.0, 1.5):
        p = S.softmax_t(logits, T)
        for k in (1, 4, 9, V):
            for top_p in (0.3, 0.8, 1.0):
                for min_p in (0.0, 0.1, 0.5):
                    np.testing.assert_allclose(S.flashinfer_min_p_chain(p, k, top_p, min_p),
                                               brute_fi_min_p(p, k, top_p, min_p), rtol=0, atol=1e-12)
        for min_p in (0.02, 0.2, 0.7):
            np.testing.assert_allclose(S.flashinfer_min_p_chain(p, V + 1, 1.0, min_p),
                                       S.torch_backend_filter(p, V + 1, 1.0, min_p, True), rtol=0, atol=1e-12)
        for k in (1, 3, 10):
            np.testing.assert_allclose(S.flashinfer_min_p_chain(p, k, 1.0, 0.0), S.joint_top_k_top_p(p, k, 1.0),
                                       rtol=0, atol=1e-12)
        for top_p in (0.2, 0.6, 0.95):
            np.testing.assert_allclose(S.flashinfer_min_p_chain(p, V + 1, top_p, 0.0),
                                       S.joint_top_k_top_p(p, V + 1, top_p), rtol=0, atol=1e-12)


def test_greedy_request_is_a_point_mass():
    """SGLang turns a greedy request into top_k = 1: both filters then keep only the maximum."""
    p = S.softmax_t(np.array([0.1, 2.0, -1.0, 1.5]), 1.0)
    for q in (S.joint_top_k_top_p(p, 1, 1.0), S.torch_backend_filter(p, 1, 1.0, 0.0, False)):
        np.testing.assert_array_equal(q, [0.0, 1.0, 0.0, 0.0])


def _state(g, bs, V):
    return dict(rep_cum=np.ones((bs, V), np.float32), rep_pen=g.uniform(1.05, 1.5, bs).astype(np.float32),
                pres_cum=np.zeros((bs, V), np.float32), pres_pen=g.uniform(0.1, 0.8, bs).astype(np.float32),
                freq_cum=np.zeros((bs, V), np.float32), freq_pen=g.uniform(0.05, 0.5, bs).astype(np.float32),
                len_out=g.integers(0, 6, bs).astype(np.int64), min_new=g.integers(0, 12, bs).astype(np.int64),
                stop_pen=np.where(np.arange(V)[None] % 7 == 0, -np.inf, 0.0).repeat(bs, 0).astype(np.float32),
                logit_bias=g.normal(size=(bs, V)).astype(np.float32))


@pytest.mark.parametrize("order", [(S.REPETITION, S.PRESENCE, S.FREQUENCY, S.MIN_NEW_TOKENS),
                                   (S.FREQUENCY, S.MIN_NEW_TOKENS, S.PRESENCE, S.REPETITION)])
def test_in_block_penalties_equal_ar_token_by_token(order):
    """Row r of penalize_rows == AR's penalties after committing cand[1..r] one token at a time (bit for bit)."""
    g = np.random.default_rng(1)
    bs, K, V = 3, 6, 50
    st = _state(g, bs, V)
    for b in range(bs):                                   # some committed history
        for t in g.integers(0, V, 5):
            S.cumulate(st, b, int(t))
    cand = g.integers(0, V, (bs, K))
    cand[0, 3] = cand[0, 2]                               # a repeated in-block token (frequency counts it twice)
    logits = g.normal(size=(bs * K, V)).astype(np.float32) * 3
    got = S.penalize_rows(logits, cand, st, order)
    for b in range(bs):
        for r in range(K):
            np.testing.assert_array_equal(got[b * K + r], _ar_row(logits[b * K + r], st, b, cand[b, 1:r + 1],
                                                                   order), err_msg=f"b={b} r={r}")


def _ar_row(row, st, b, inblk, order):
    """AR decode's penalties on one row after committing ``inblk`` token by token (fresh copy of the state)."""
    ar = {k: (v.copy() if isinstance(v, np.ndarray) else v) for k, v in st.items()}
    for t in inblk:
        S.cumulate(ar, b, int(t))
    out = row.astype(np.float32).copy()
    for name in order:
        if name == S.REPETITION:
            out = S.apply_scaling(out, ar["rep_cum"][b]).astype(np.float32)
        elif name == S.PRESENCE:
            out -= ar["pres_cum"][b]
        elif name == S.FREQUENCY:
            out -= ar["freq_cum"][b]
        elif name == S.MIN_NEW_TOKENS:
            if ar["len_out"][b] < ar["min_new"][b]:
                out += ar["stop_pen"][b]
    return out + ar["logit_bias"][b]


def test_inverse_cdf_breakpoints():
    g = np.random.default_rng(3)
    q = g.uniform(0, 1, 12)
    q[[2, 7]] = 0.0
    c = np.cumsum(q) / q.sum()
    for t in range(12):
        if q[t] == 0:
            continue
        lo = c[t - 1] if t else 0.0
        assert S.inverse_cdf(q, lo + 1e-9) == t
        assert S.inverse_cdf(q, c[t] - 1e-9) == t
    assert S.inverse_cdf(np.zeros(4), 0.5) == -1


@pytest.mark.parametrize("seed", range(3))
def test_speculative_sampling_first_token_is_ar_distributed(seed):
    """P(first committed token after a0 = t) = p_0(t) for every draft token d_1 (accept with p_0(d_1), else draw
    from p_0 without d_1): measured over a 400 x 400 grid of coins in (0, 1] and uniforms in [0, 1)."""
    g = np.random.default_rng(seed)
    V, K = 6, 3
    probs = np.stack([S.softmax_t(g.normal(size=V) * 1.5, 1.0) for _ in range(K)])
    n = 400
    for d1 in range(V):
        cand = np.array([0, d1, int(g.integers(0, V))])
        counts = np.zeros(V)
        for ci in range(n):
            coin = 1.0 - (ci + 0.5) / n
            for ui in range(n):
                acc, tok, targets = S.spec_sample_chain(probs, cand, np.array([coin, 1.0, 1.0]), (ui + 0.5) / n)
                counts[targets[0]] += 1
        np.testing.assert_allclose(counts / n / n, probs[0], atol=6 / n)


def test_all_accepted_draws_the_bonus_from_the_last_row():
    g = np.random.default_rng(5)
    V, K = 5, 4
    probs = np.stack([S.softmax_t(g.normal(size=V), 1.0) for _ in range(K)])
    cand = np.array([1, 2, 3, 4])
    acc, tok, targets = S.spec_sample_chain(probs, cand, np.full(K, 1e-9), 0.37)
    assert acc == K - 1 and targets[:-1] == [2, 3, 4] and tok == S.inverse_cdf(probs[K - 1], 0.37)
    acc, tok, targets = S.spec_sample_chain(probs, cand, np.array([1e-9, 1.0, 1e-9, 1e-9]), 0.37)
    q = probs[1].copy()
    q[3] = 0
    assert acc == 1 and targets == [2, tok] and tok == S.inverse_cdf(q, 0.37) and tok != 3
