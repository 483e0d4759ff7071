"""The sampled verify kernels against the oracle (oracle/sampling.py) on the same coins and uniforms:
gss_penalize_rows bit for bit (fp32, every penalizer order); gss_sample_rows' draws (sample mode, every filter,
temperatures down to the point mass) and its chain decision (verify mode: accept length, committed targets, packed
row, next seed). A draw may differ from the float64 oracle only where the uniform sits within 1e-5 of a
cumulative-probability boundary (fp32 prefix sums); the tests check that every mismatch is such a case."""
import numpy as np
import pytest
import torch

from oracle import sampling as S

pytestmark = pytest.mark.gpu

ORDERS = [("repetition", "presence", "frequency", "min_new_tokens"), ("frequency", "min_new_tokens", "presence",
                                                                      "repetition"), ("presence",), ()]


def _state_np(g, bs, V):
    st = dict(rep_cum=np.ones((bs, V), np.float32), rep_pen=g.uniform(1.05, 1.5, bs).astype(np.float32),
              pres_cum=np.zeros((bs, V), np.float32), pres_pen=g.uniform(0.1, 0.8, bs).astype(np.float32),
              freq_cum=np.zeros((bs, V), np.float32), freq_pen=g.uniform(0.05, 0.5, bs).astype(np.float32),
              len_out=g.integers(0, 6, bs).astype(np.int64), min_new=g.integers(0, 12, bs).astype(np.int64),
              stop_pen=np.where(np.arange(V)[None] % 97 == 0, -np.inf, 0.0).repeat(bs, 0).astype(np.float32),
              logit_bias=(g.normal(size=(bs, V)) * 0.5).astype(np.float32))
    for b in range(bs):
        for t in g.integers(0, V, 20):
            S.cumulate(st, b, int(t))
    return st


def _to_dev(st, cuda):
    out = {}
    for k, v in st.items():
        dt = torch.int32 if k in ("len_out", "min_new") else torch.float32
        out[k] = torch.as_tensor(np.asarray(v)).to(dt).to(cuda).contiguous()
    return out


@pytest.mark.parametrize("order", ORDERS)
@pytest.mark.parametrize("V", [4096, 59392])
def test_penalize_rows_bit_exact(cuda, order, V):
    from gravityocr_amd.kernels import penalize_rows
    print(f"penalize V={V} order={order}", flush=True)
    g = np.random.default_rng(V + len(order))
    bs, K = 3, 9
    st = _state_np(g, bs, V)
    cand = g.integers(0, V, (bs, K)).astype(np.int32)
    cand[1, 4] = cand[1, 2]
    cand[2, 1:] = g.integers(0, 40, K - 1)               # in-block tokens that also carry committed state
    logits = (g.normal(size=(bs * K, V)) * 3).astype(np.float32)
    want = S.penalize_rows(logits, cand, st, order)
    dl = torch.as_tensor(logits).to(cuda)
    penalize_rows(dl, torch.as_tensor(cand).to(cuda), _to_dev(st, cuda), order)
    torch.cuda.synchronize()
    got = dl.cpu().numpy()
    np.testing.assert_array_equal(got, want)


def _draw_ok(q, u, tok):
    want = S.inverse_cdf(q, u)
    if tok == want:
        return True
    if want < 0 or tok < 0 or q[tok] <= 0:
        return False
    c = np.cumsum(q) / q.sum()
    lo = min(tok, want)
    return abs(c[lo] - u) < 1e-5


CASES = [  # (filter, temperature, top_k, top_p, min_p)
    ("none", 1.0, 0, 1.0, 0.0), ("none", 0.7, 0, 1.0, 0.0), ("none", 0.0, 0, 1.0, 0.0),
    ("joint", 1.0, 20, 0.9, 0.0), ("joint", 0.8, 1, 1.0, 0.0), ("joint", 1.3, 0, 0.5, 0.0), ("joint", 1.0, 5, 1.0, 0.0),
    ("torch", 1.0, 50, 0.95, 0.0), ("torch", 0.9, 1, 1.0, 0.0), ("torch", 1.0, 0, 0.8, 0.05),
    ("torch", 1.2, 30, 1.0, 0.1), ("flashinfer_min_p", 1.0, 20, 0.9, 0.1), ("flashinfer_min_p", 0.8, 0, 0.7, 0.0),
    ("flashinfer_min_p", 1.2, 40, 1.0, 0.3), ("flashinfer_min_p", 1.0, 60, 0.5, 0.02)]


def _target(row, case):
    filt, T, k, tp, mp = case
    if T <= 0:
        q = np.zeros(row.shape[0])
        q[int(np.argmax(row))] = 1.0
        return q
    mode = {"none": 0, "joint": 1, "torch": 2, "flashinfer_min_p": 3}[filt]
    return S.target_probs(row, T, mode, k if k > 0 else row.shape[0] + 1, tp, mp)


@pytest.mark.parametrize("V", [4096, 12000, 59392])
@pytest.mark.parametrize("case", CASES, ids=lambda c: "-".join(map(str, c)))
def test_sample_mode_draws_match_oracle(cuda, V, case):
    from gravityocr_amd.kernels import sample_rows
    print(f"sample V={V} case={case}", flush=True)
    filt, T, k, tp, mp = case
    g = np.random.default_rng(V * 3 + len(filt))
    bs, K = 3, 4
    logits = (g.normal(size=(bs * K, V)) * 2.5).astype(np.float32)
    u = g.uniform(0, 1, (bs, K)).astype(np.float32)
    f = lambda x, dt: torch.tensor([x] * bs, dtype=dt, device=cuda)
    sampled = torch.full((bs, K), -7, dtype=torch.int32, device=cuda)
    sample_rows(torch.as_tensor(logits).to(cuda), bs, K, temperature=f(T, torch.float32), filter=filt,
                top_k=f(k, torch.int32), top_p=f(tp, torch.float32), min_p=f(mp, torch.float32),
                uniforms=torch.as_tensor(u).to(cuda), sampled=sampled)
    torch.cuda.synchronize()
    got = sampled.cpu().numpy()
    for r in range(bs * K):
        q = _target(logits[r], case)
        assert _draw_ok(q, float(u.flat[r]), int(got.flat[r])), (r, int(got.flat[r]), S.inverse_cdf(q, float(u.flat[r])))


@pytest.mark.parametrize("V", [4096, 59392])
@pytest.mark.parametrize("case", [CASES[0], CASES[3], CASES[7], CASES[9], CASES[2], CASES[11], CASES[14]],
                         ids=lambda c: "-".join(map(str, c)))
def test_verify_mode_chain_matches_oracle(cuda, V, case):
    """Speculative sampling of a draft chain: drafts are high-probability tokens of the rows (so several are
    accepted), coins spread over (0, 1]; every sequence's accept length, targets, next seed and packed row equal the
    oracle's chain on the same coins and uniform."""
    from gravityocr_amd.kernels import sample_rows, sample_workspace_bytes
    print(f"verify V={V} case={case}", flush=True)
    g = np.random.default_rng(V + 17)
    bs, K = 6, 9
    logits = (g.normal(size=(bs * K, V)) * 2.5).astype(np.float32)
    logits[np.arange(bs * K), g.integers(0, V, bs * K)] += 12.0      # a dominant token per row (often accepted)
    cand = np.zeros((bs, K), np.int32)
    probs = np.stack([_target(logits[r], case) for r in range(bs * K)]).reshape(bs, K, V)
    for b in range(bs):
        cand[b, 0] = g.integers(0, V)
        for j in range(K - 1):
            top = np.argsort(-probs[b, j])[:3]
            cand[b, j + 1] = top[g.integers(0, 3)] if g.uniform() < 0.85 else g.integers(0, V)
    coins = (1.0 - g.uniform(0, 1, (bs, K))).astype(np.float32) * 0.6
    u = g.uniform(0, 1, bs).astype(np.float32)
    f = lambda x, dt: torch.tensor([x] * bs, dtype=dt, device=cuda)
    dev = lambda a: torch.as_tensor(a).to(cuda)
    sampled = torch.full((bs, K), -7, dtype=torch.int32, device=cuda)
    target = torch.full((bs, K), -7, dtype=torch.int32, device=cuda)
    acc = torch.full((bs,), -7, dtype=torch.int32, device=cuda)
    nx = torch.full((bs,), -7, dtype=torch.int32, device=cuda)
    packed = torch.full((bs, K + 2), -7, dtype=torch.int32, device=cuda)
    ws = torch.zeros(sample_workspace_bytes(bs, K), dtype=torch.uint8, device=cuda)
    filt, T, k, tp, mp = case
    for call in range(2):   # the workspace counters reset themselves
        sample_rows(dev(logits), bs, K, temperature=f(T, torch.float32), filter=filt, top_k=f(k, torch.int32),
                    top_p=f(tp, torch.float32), min_p=f(mp, torch.float32), cand=dev(cand), coins=dev(coins),
                    uniforms=dev(u), sampled=sampled, target=target, accept_len=acc, next_x0=nx, packed=packed,
                    workspace=ws)
        torch.cuda.synchronize()
        n_acc = 0
        for b in range(bs):
            a_want, tok_want, t_want = S.spec_sample_chain(probs[b], cand[b], coins[b].astype(np.float64), float(u[b]))
            a = int(acc[b])
            if a != a_want:   # only a coin within 1e-5 of its row's draft probability may flip the decision
                j = min(a, a_want)
                assert abs(coins[b, j] - probs[b, j, cand[b, j + 1]]) < 1e-5, (b, a, a_want)
                continue
            n_acc += a
            q = probs[b, a].copy()
            if a < K - 1:
                q[cand[b, a + 1]] = 0.0
            tok = int(nx[b])
            assert _draw_ok(q, float(u[b]), tok), (b, tok, tok_want)
            assert target[b, :a].cpu().tolist() == [int(t) for t in cand[b, 1:a + 1]] and int(target[b, a]) == tok
            assert packed[b].cpu().tolist() == [int(cand[b, 0]), a] + target[b, :a + 1].cpu().tolist() + [0] * (K - 1 - a)
            assert int(sampled[b, a]) == tok
        if case[1] > 0 and case[0] != "joint":
            assert n_acc > 0   # the drafts were built to be accepted sometimes


@pytest.mark.parametrize("order", [("repetition",), ("presence", "frequency")])
def test_penalize_rows_without_min_new_tokens(cuda, order):
    """Penalizers listed without min_new_tokens: the length / stop arrays are absent (null) and never read."""
    from gravityocr_amd.kernels import penalize_rows
    g = np.random.default_rng(21)
    bs, K, V = 2, 5, 4096
    st = _state_np(g, bs, V)
    cand = g.integers(0, V, (bs, K)).astype(np.int32)
    logits = (g.normal(size=(bs * K, V)) * 3).astype(np.float32)
    st_np = {k: v for k, v in st.items() if k not in ("min_new", "stop_pen", "logit_bias")}
    want = S.penalize_rows(logits, cand, st_np, order)
    dst = _to_dev(st_np, cuda)          # len_out present, min_new / stop_pen absent
    dl = torch.as_tensor(logits).to(cuda)
    penalize_rows(dl, torch.as_tensor(cand).to(cuda), dst, order)
    torch.cuda.synchronize()
    np.testing.assert_array_equal(dl.cpu().numpy(), want)


@pytest.mark.parametrize("kind", ["peaked-top-k", "flat-top-p", "all-equal", "equal-blocks"])
def test_threshold_search_paths(cuda, kind):
    """The threshold search finishes over compacted candidates when few tokens lie near the cut (a peaked row under
    top-k 40; a flat row under top-p 0.95, after a second, narrower attempt) and by full passes when too many do (a
    row of equal logits, where every token is a candidate at any width; blocks of exactly tied values straddling the
    cut): every path draws from the oracle's distribution."""
    from gravityocr_amd.kernels import sample_rows
    print(f"threshold search {kind}", flush=True)
    g = np.random.default_rng(len(kind))
    bs, K, V = 2, 5, 59392
    if kind == "peaked-top-k":
        logits, T, k, tp = g.normal(size=(bs * K, V)) * 2.5, 0.8, 40, 0.9
    elif kind == "flat-top-p":
        logits, T, k, tp = g.normal(size=(bs * K, V)) * 0.5, 1.5, 0, 0.95
    elif kind == "all-equal":
        logits, T, k, tp = np.zeros((bs * K, V)), 1.0, 0, 0.9
    else:
        logits, T, k, tp = np.repeat(g.normal(size=(bs * K, V // 64)), 64, axis=1), 1.0, 0, 0.7
    logits = logits.astype(np.float32)
    u = g.uniform(0, 1, (bs, K)).astype(np.float32)
    f = lambda x, dt: torch.tensor([x] * bs, dtype=dt, device=cuda)
    sampled = torch.full((bs, K), -7, dtype=torch.int32, device=cuda)
    sample_rows(torch.as_tensor(logits).to(cuda), bs, K, temperature=f(T, torch.float32), filter="joint",
                top_k=f(k, torch.int32), top_p=f(tp, torch.float32), min_p=f(0.0, torch.float32),
                uniforms=torch.as_tensor(u).to(cuda), sampled=sampled)
    torch.cuda.synchronize()
    got = sampled.cpu().numpy()
    for r in range(bs * K):
        q = S.target_probs(logits[r], T, 1, k if k > 0 else V + 1, tp)
        assert _draw_ok(q, float(u.flat[r]), int(got.flat[r])), (r, int(got.flat[r]), S.inverse_cdf(q, float(u.flat[r])))
