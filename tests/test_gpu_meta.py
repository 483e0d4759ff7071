"""The serving-boundary integer kernels bit-exact against the oracle: gss_ss_commit vs oracle.integer.ss_commit
(_ss_commit_kernel, selfspec_fast_commit.py:108-147) and gss_kv_meta vs oracle.integer.kv_meta (_ss_kv_meta_kernel,
selfspec_fast_attn.py:104-132), at batch sizes 1..256 and window sizes K in {5, 17, 33, 64}, including the edge cases
of the accept length (0 and K-1), a strided a0 view, empty rows (seq_len 0) and zero extra."""
import numpy as np
import pytest
import torch

from oracle.integer import kv_meta as o_kv_meta, ss_commit as o_ss_commit

pytestmark = pytest.mark.gpu


@pytest.mark.parametrize("bs,K", [(1, 17), (8, 5), (33, 17), (64, 33), (256, 17), (7, 64)])
def test_ss_commit_matches_oracle(cuda, bs, K):
    from gravityocr_amd.kernels import ss_commit
    g = np.random.default_rng(bs * 100 + K)
    predict = g.integers(0, 59392, bs * K + 1).astype(np.int32)
    acc = g.integers(0, K, bs).astype(np.int32)
    acc[0] = 0
    acc[-1] = K - 1
    a0_full = g.integers(0, 59392, (bs, 3)).astype(np.int64)       # a0 is a strided column view
    rpi = g.permutation(bs + 5)[:bs].astype(np.int64)
    seeds = g.integers(-5, 5, bs + 5).astype(np.int64)
    seq = g.integers(0, 20000, bs).astype(np.int64)
    loc = g.integers(0, 10**7, bs * K).astype(np.int64)
    want = o_ss_commit(predict, acc, a0_full[:, 1], rpi, seeds, seq, loc, K)
    d = lambda x: torch.from_numpy(np.ascontiguousarray(x)).to(cuda)
    a0_dev = d(a0_full)[:, 1]
    seeds_d, seq_d = d(seeds), d(seq)
    packed = torch.full((bs, K + 2), -9, dtype=torch.int32, device=cuda)
    free = torch.full((bs * K,), -9, dtype=torch.int64, device=cuda)
    out = torch.full((bs,), -9, dtype=torch.int64, device=cuda)
    ss_commit(d(predict), d(acc), a0_dev, d(rpi), seeds_d, seq_d, d(loc), packed, free, out, K=K)
    torch.cuda.synchronize()
    w_packed, w_seeds, w_seq, w_free, w_out, _ = want
    np.testing.assert_array_equal(packed.cpu().numpy(), w_packed)
    np.testing.assert_array_equal(seeds_d.cpu().numpy(), w_seeds)
    np.testing.assert_array_equal(seq_d.cpu().numpy(), w_seq)
    np.testing.assert_array_equal(out.cpu().numpy(), w_out)
    n = len(w_free)
    np.testing.assert_array_equal(free[:n].cpu().numpy(), w_free)
    assert bool((free[n:] == -9).all())                               # nothing written past the list


@pytest.mark.parametrize("bs,K,page", [(1, 17, 16), (8, 5, 16), (33, 17, 16), (64, 33, 4), (130, 17, 16),
                                       (7, 64, 16), (40, 9, 1)])
def test_ss_commit_cut_rule_and_page_frees(cuda, bs, K, page):
    """gss_ss_commit with the finish rule (per-request budgets, stop ids, vocabulary bounds; some requests marked for
    the per-token path) and page-aligned slots: cut indices, lengths, packed rows, seeds and the page-granular free
    list and its count bit-exact against the oracle (its cut is the per-token loop, its frees the page rule)."""
    from gravityocr_amd.kernels import ss_commit
    g = np.random.default_rng(bs * 7 + K + page)
    V = 500
    predict = g.integers(-3, V + 20, bs * K + 1).astype(np.int32)
    acc = g.integers(0, K, bs).astype(np.int32)
    a0 = g.integers(0, V, bs).astype(np.int64)
    rpi = g.permutation(bs + 5)[:bs].astype(np.int64)
    seeds = np.zeros(bs + 5, dtype=np.int64)
    S = g.integers(0, 4000, bs).astype(np.int64)
    n_pg = (4000 + K + page - 1) // page                                     # pages that cover a request
    pts = [g.permutation(n_pg) + n_pg * i for i in range(bs)]
    loc = np.array([pts[i][(S[i] + r) // page] * page + (S[i] + r) % page for i in range(bs) for r in range(K)],
                   dtype=np.int64)
    budgets = g.integers(-1, 2 * K, bs).astype(np.int32)
    n_stop = 3
    stop_ids = g.integers(-1, V, (bs, n_stop)).astype(np.int32)
    stop_ids[:, 0] = -1                                                      # padding entries
    # make some stop ids hit: a committed token of the row
    for i in range(0, bs, 3):
        stop_ids[i, 1] = predict[i * K + min(int(acc[i]), 1)]
    vocab = g.integers(V - 5, V + 5, bs).astype(np.int32)
    stops = [set(int(x) for x in row if x >= 0) for row in stop_ids]
    w_packed, w_seeds, w_seq, w_free, w_out, w_cut = o_ss_commit(predict, acc, a0, rpi, seeds, S, loc, K, page=page,
                                                                 finish=(budgets, stops, vocab))
    d = lambda x: torch.from_numpy(np.ascontiguousarray(x)).to(cuda)
    seeds_d, seq_d = d(seeds), d(S)
    packed = torch.full((bs, K + 2), -9, dtype=torch.int32, device=cuda)
    free = torch.full((bs * K,), -9, dtype=torch.int64, device=cuda)
    out = torch.full((bs,), -9, dtype=torch.int64, device=cuda)
    cut = torch.full((bs,), -9, dtype=torch.int32, device=cuda)
    n_free = torch.full((1,), -9, dtype=torch.int32, device=cuda)
    ss_commit(d(predict), d(acc), d(a0), d(rpi), seeds_d, seq_d, d(loc), packed, free, out, K=K, page=page,
              budget=d(budgets), stop_ids=d(stop_ids), vocab=d(vocab), cut=cut, n_free=n_free)
    torch.cuda.synchronize()
    np.testing.assert_array_equal(cut.cpu().numpy(), w_cut)
    np.testing.assert_array_equal(seq_d.cpu().numpy(), w_seq)
    np.testing.assert_array_equal(packed.cpu().numpy(), w_packed)
    np.testing.assert_array_equal(seeds_d.cpu().numpy(), w_seeds)
    np.testing.assert_array_equal(out.cpu().numpy(), w_out)
    n = len(w_free)
    assert int(n_free[0]) == n
    np.testing.assert_array_equal(free[:n].cpu().numpy(), w_free)
    assert bool((free[n:] == -9).all())
    print(f"bs={bs} K={K} page={page}: cuts {np.bincount(w_cut, minlength=K + 1).tolist()}, {n} slots freed")


@pytest.mark.parametrize("bs,extra", [(1, 17), (5, 0), (32, 17), (200, 33)])
def test_kv_meta_matches_oracle(cuda, bs, extra):
    from gravityocr_amd.kernels import kv_meta
    g = np.random.default_rng(bs + extra)
    pool, ctx = bs + 7, 4096
    r2t = g.integers(0, 2**31 - 1, (pool, ctx)).astype(np.int32)
    rpi = g.permutation(pool)[:bs].astype(np.int64)
    sl = g.integers(0, ctx - extra, bs).astype(np.int64)
    sl[0] = 0                                                          # an empty committed prefix
    w_ptr, w_idx = o_kv_meta(r2t, rpi, sl, extra)
    d = lambda x: torch.from_numpy(np.ascontiguousarray(x)).to(cuda)
    ptr = torch.full((bs + 1,), -9, dtype=torch.int32, device=cuda)
    idx = torch.full((len(w_idx) + 64,), -9, dtype=torch.int32, device=cuda)
    kv_meta(d(r2t), d(rpi), d(sl), ptr, idx, extra=extra)
    torch.cuda.synchronize()
    np.testing.assert_array_equal(ptr.cpu().numpy(), w_ptr)
    np.testing.assert_array_equal(idx[:len(w_idx)].cpu().numpy(), w_idx)
    assert bool((idx[len(w_idx):] == -9).all())


def test_log_append_rows_clamp_and_counter(cuda):
    """gss_log_append writes row min(ctr, capacity - 1) of every log and advances the counter by one per call;
    calls beyond the capacity rewrite the last row."""
    from gravityocr_amd.kernels import log_append
    cap, bs, K = 4, 3, 17
    ctr = torch.zeros(1, dtype=torch.int64, device=cuda)
    logs = [torch.full((cap, bs, K + 2), -1, dtype=torch.int32, device=cuda),
            torch.full((cap, bs, K), -1, dtype=torch.int32, device=cuda),
            torch.full((cap, bs), -1, dtype=torch.int32, device=cuda)]
    want = [torch.full(t.shape, -1, dtype=torch.int32) for t in logs]
    for call in range(6):
        srcs = [torch.arange(t[0].numel(), dtype=torch.int32, device=cuda).view(t[0].shape) * 10 + call for t in logs]
        pairs = list(zip(srcs, logs))[: 1 + call % 3]
        log_append(ctr, pairs)
        for i, (src, _) in enumerate(pairs):
            want[i][min(call, cap - 1)] = src.cpu()
    torch.cuda.synchronize()
    assert int(ctr.item()) == 6
    for t, w in zip(logs, want):
        assert torch.equal(t.cpu(), w)
