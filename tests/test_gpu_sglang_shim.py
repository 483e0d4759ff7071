"""The SGLang backend shim (gravityocr_amd/sglang_shim.py) on duck-typed server objects at page size 16:
  * set_kv_buffer writes each token's K/V to its slot in the kernels' page layout (read back exactly);
  * forward_extend for both roles equals the oracle's masked attention over the request's committed prefix (read
    through req_to_token's page-aligned slots) plus the window, within the attention tolerance (1e-2 * max |ref|);
  * commit equals the oracle's _ss_commit restatement and per-token host loop: next seeds, committed tokens and j,
    seq_lens (device and host), and, at page size 16, the freed pages: exactly the pages of the verify slots that hold
    no kept token (a page-granular allocator would otherwise release committed KV);
  * the draft-ahead commit settles as the plain one, and calls the next draft's launch before the bookkeeping
    exactly in the rounds where no request can finish."""
import numpy as np
import pytest
import torch

from oracle.attention import paged_window_attention
from oracle.integer import host_commit_loop, ss_commit as o_ss_commit
from tests.test_oracle_integer import _Req

pytestmark = pytest.mark.gpu


class _NS:
    def __init__(self, **kw):
        self.__dict__.update(kw)


def _server(cuda, g, lens, K, Hkv=2, D=128, n_layers=2, ctx=2048):
    """a request pool at page size 16: whole pages handed out from a shuffled free list."""
    from gravityocr_amd.sglang_shim import PagedKVPool
    n_pages = sum((L + K + 15) // 16 + 1 for L in lens) + 4
    pool = PagedKVPool(n_layers, n_pages, Hkv, D, cuda)
    free = list(g.permutation(n_pages))
    r2t = torch.zeros(len(lens) + 2, ctx, dtype=torch.int32)
    for r, L in enumerate(lens):
        for blk in range((L + K + 15) // 16):
            pg = int(free.pop())
            r2t[r + 1, blk * 16:(blk + 1) * 16] = torch.arange(pg * 16, pg * 16 + 16, dtype=torch.int32)
    return pool, r2t.to(cuda)


@pytest.mark.parametrize("role", ["draft", "verify"])
def test_attention_backend_matches_oracle(cuda, role):
    from gravityocr_amd.sglang_shim import GssSelfSpecAttnBackend
    print(f"shim attention {role}", flush=True)
    g = np.random.default_rng(11 if role == "draft" else 12)
    lens, K, Hq, Hkv, D = [100, 1000, 37], 17, 16, 2, 128
    bs = len(lens)
    pool, r2t = _server(cuda, g, lens, K)
    rpi = torch.arange(1, bs + 1, dtype=torch.int64, device=cuda)
    layer = _NS(layer_id=1, scaling=D ** -0.5)
    # the committed prefixes: every position's K/V written through set_kv_buffer
    for r, L in enumerate(lens):
        loc = r2t[r + 1, :L].to(torch.int64)
        k = (torch.randn(L, Hkv, D, device=cuda) / D ** 0.5).bfloat16()
        v = (torch.randn(L, Hkv, D, device=cuda) / D ** 0.5).bfloat16()
        pool.set_kv_buffer(layer.layer_id, loc, k, v)
        pg, off = loc // 16, loc % 16
        assert torch.equal(pool.k[1][pg, :, off, :], k) and torch.equal(pool.v[1][pg, :, :, off], v)
    be = GssSelfSpecAttnBackend(pool, r2t, Hq, Hkv, D, max_bs=4, K=K, max_kv_len=1536)
    seq_lens = torch.tensor(lens, dtype=torch.int64, device=cuda)
    out_loc = torch.cat([r2t[r + 1, L:L + K] for r, L in enumerate(lens)]).to(torch.int64)
    fb = _NS(spec_info=_NS(selfspec_role=role, draft_token_num=K), req_pool_indices=rpi, seq_lens=seq_lens,
             out_cache_loc=out_loc)
    q = (torch.randn(bs * K, Hq * D, device=cuda) / D ** 0.5).bfloat16()
    k = (torch.randn(bs * K, Hkv * D, device=cuda) / D ** 0.5).bfloat16()
    v = (torch.randn(bs * K, Hkv * D, device=cuda) / D ** 0.5).bfloat16()
    be.init_forward_metadata(fb)
    o = be.forward_extend(q, k, v, layer, fb)
    torch.cuda.synchronize()
    # the window's K/V landed in its slots too
    pg, off = out_loc // 16, out_loc % 16
    assert torch.equal(pool.k[1][pg, :, off, :], k.view(-1, Hkv, D))
    kp, vp = pool.k[1].cpu(), pool.v[1].cpu()
    for r, L in enumerate(lens):
        pt_row = (r2t[r + 1, ::16] // 16).cpu().numpy()
        ref = paged_window_attention(q.view(bs, K, Hq, D)[r].cpu(), kp, vp, pt_row, L, k.view(bs, K, Hkv, D)[r].cpu(),
                                     v.view(bs, K, Hkv, D)[r].cpu(), 1 if role == "draft" else K, D ** -0.5)
        got = o.view(bs, K, Hq, D)[r].float().cpu()
        err = float((got.double() - ref).abs().max())
        assert err <= 1e-2 * float(ref.abs().max()), (r, err)


class _PageAlloc:
    """SGLang's paged allocator as the commit sees it: free(slots) releases the pages those slots lie in."""

    def __init__(self, page=16):
        self.page, self.freed_pages, self.calls = page, [], 0
        self.is_not_in_free_group = True

    def free(self, t):
        self.calls += 1
        self.freed_pages += sorted(set((t.cpu() // self.page).tolist()))


def _token_loop(req, T):
    """The per-token path for requests outside the cut rule: append one token, check, stop when finished."""
    for t, x in enumerate(T):
        req.output_ids.append(x)
        req.check_finished()
        if req.finished():
            return t
    return len(T) - 1


@pytest.mark.parametrize("bs,finish", [(1, False), (4, False), (4, True), (16, True)])
def test_fast_commit_pages_and_finish_rules(cuda, bs, finish):
    """GssFastCommit at page size 16 on page-aligned verify slots: next seeds, committed tokens and cut j equal the
    oracle's commit and per-token loop (stop ids 3 and 7, per-request budgets, vocabulary bound 10); every third
    request (stop strings set) goes through the injected per-token path; seq_lens (device and host) advance by j;
    the allocator is handed exactly the pages that hold no kept token (none holding a kept position), and the kv
    lengths stay page-aligned."""
    from gravityocr_amd.sglang_shim import GssFastCommit
    print(f"shim commit bs={bs} finish={finish}", flush=True)
    g = np.random.default_rng(bs * 3 + finish)
    K, vocab, pool_n, page = 17, 10, bs + 4, 16
    acc = g.integers(0, K, bs).astype(np.int32)
    predict = g.integers(0, 12, bs * K + 1).astype(np.int32)
    a0 = g.integers(0, 12, bs).astype(np.int64)
    rpi = g.permutation(pool_n)[:bs].astype(np.int64)
    seeds = g.integers(0, 100, pool_n).astype(np.int64)
    S = g.integers(10, 200, bs).astype(np.int64)
    pts = [g.permutation(64) + 64 * i for i in range(bs)]            # each request's own shuffled pages
    loc = np.array([pts[i][(S[i] + r) // page] * page + (S[i] + r) % page for i in range(bs) for r in range(K)],
                   dtype=np.int64)
    budgets = [int(x) for x in g.integers(1, 3 if finish else 60, bs)]
    reqs = [_Req(bdg, vocab) for bdg in budgets]
    slow = [i % 3 == 2 for i in range(bs)]
    for i, r in enumerate(reqs):
        r.kv_committed_len, r.kv_allocated_len = int(S[i]), int(S[i])
        if slow[i]:
            r.sampling_params.stop_strs = ["</s>"]
    dev = lambda a: torch.as_tensor(a).to(cuda)
    vi = _NS(predict=dev(predict), accept_length=dev(acc), a0=dev(a0), draft_token_num=K)
    seeds_d, sl_d = dev(seeds), dev(S)
    alloc = _PageAlloc(page)
    batch = _NS(batch_size=lambda: bs, out_cache_loc=dev(loc), req_pool_indices=dev(rpi), seq_lens=sl_d,
                seq_lens_cpu=torch.as_tensor(S.copy()), seq_lens_sum=int(S.sum()), reqs=reqs,
                token_to_kv_pool_allocator=alloc)
    fc = GssFastCommit(K, 32, cuda, page=page, token_loop=_token_loop)
    out, toks, js = fc.commit(vi, batch, seeds_d)
    torch.cuda.synchronize()
    packed, seeds_w, _, _, out_w, _ = o_ss_commit(predict, acc, a0, rpi, seeds.copy(), S.copy(), loc, K)
    otoks, ojs, oaccs = host_commit_loop(packed.tolist(), budgets, [{3, 7}] * bs, vocab)
    assert out.cpu().numpy().tolist() == out_w.tolist()
    assert np.array_equal(seeds_d.cpu().numpy(), seeds_w)
    assert toks == otoks and js == ojs
    for i, r in enumerate(reqs):
        assert r.output_ids == otoks[i]
        assert r.kv_committed_len == S[i] + js[i] + 1 and r.kv_allocated_len % page == 0
        assert r.kv_allocated_len >= r.kv_committed_len
    want_sl = S + np.array(js)
    assert np.array_equal(sl_d.cpu().numpy(), want_sl) and np.array_equal(batch.seq_lens_cpu.numpy(), want_sl)
    assert batch.seq_lens_sum == int(S.sum()) + sum(js)
    # pages: exactly those of the verify slots that hold no kept position [0, S + j)
    want_pages = []
    for i in range(bs):
        kept = {int(pts[i][p // page]) for p in range(int(S[i]) + js[i])}
        want_pages += sorted({int(loc[i * K + r]) // page for r in range(K)} - kept)
        assert not kept & set(alloc.freed_pages)
    assert sorted(alloc.freed_pages) == sorted(want_pages)
    assert alloc.calls <= 1


def _ahead_round(cuda, case, bs, seed):
    """One commit round's inputs at page size 16 (K = 17): case "clean" draws ids that are neither stop ids (3, 7)
    nor outside the vocabulary (10) and budgets beyond the round, so no request finishes; "finish" plants stop id 7
    as request 1's first accepted token; "slow" gives request 2 stop strings (outside the cut rule)."""
    g = np.random.default_rng(seed)
    K, vocab, pool_n, page = 17, 10, bs + 4, 16
    ok = np.array([0, 1, 2, 4, 5, 6, 8, 9])
    acc = g.integers(0, K, bs).astype(np.int32)
    predict = ok[g.integers(0, len(ok), bs * K + 1)].astype(np.int32)
    a0 = ok[g.integers(0, len(ok), bs)].astype(np.int64)
    if case == "finish":
        predict[1 * K] = 7
    rpi = g.permutation(pool_n)[:bs].astype(np.int64)
    seeds = g.integers(0, 100, pool_n).astype(np.int64)
    S = g.integers(10, 200, bs).astype(np.int64)
    pts = [g.permutation(64) + 64 * i for i in range(bs)]
    loc = np.array([pts[i][(S[i] + r) // page] * page + (S[i] + r) % page for i in range(bs) for r in range(K)],
                   dtype=np.int64)
    reqs = [_Req(int(b), vocab) for b in g.integers(K + 2, 100, bs)]
    for i, r in enumerate(reqs):
        r.kv_committed_len, r.kv_allocated_len = int(S[i]), int(S[i])
        if case == "slow" and i == 2:
            r.sampling_params.stop_strs = ["</s>"]
    dev = lambda a: torch.as_tensor(a).to(cuda)
    vi = _NS(predict=dev(predict), accept_length=dev(acc), a0=dev(a0), draft_token_num=K)
    alloc = _PageAlloc(page)
    batch = _NS(batch_size=lambda: bs, out_cache_loc=dev(loc), req_pool_indices=dev(rpi), seq_lens=dev(S),
                seq_lens_cpu=torch.as_tensor(S.copy()), seq_lens_sum=int(S.sum()), reqs=reqs,
                token_to_kv_pool_allocator=alloc)
    return vi, batch, dev(seeds), alloc


@pytest.mark.parametrize("case,bs", [("clean", 1), ("clean", 4), ("clean", 16), ("finish", 4), ("slow", 4)])
def test_fast_commit_draft_ahead(cuda, case, bs):
    """The draft-ahead commit against the plain one on two identical rounds: the same next seeds, seed pool,
    committed tokens, cuts, device and host lengths, freed pages and counters. ahead(inc) runs exactly when no
    request finishes in the plain commit and every request is under the cut rule: then once, with inc = the cuts
    (the length increments), after the frees and before any output_ids is extended, and the launched draft's K
    slots count in the page-aligned kv_allocated_len. Otherwise the round settles as the plain one."""
    from gravityocr_amd.sglang_shim import GssFastCommit
    K, page, seed = 17, 16, 11 * bs + len(case)
    print(f"draft-ahead commit {case} bs={bs}", flush=True)
    vi_p, b_p, seeds_p, alloc_p = _ahead_round(cuda, case, bs, seed)
    vi_a, b_a, seeds_a, alloc_a = _ahead_round(cuda, case, bs, seed)
    out_p, toks_p, js_p = GssFastCommit(K, 32, cuda, page=page, token_loop=_token_loop).commit(vi_p, b_p, seeds_p)
    calls = []

    def ahead(inc):
        calls.append((list(inc), alloc_a.calls, [list(r.output_ids) for r in b_a.reqs]))
        return True

    fc = GssFastCommit(K, 32, cuda, page=page, token_loop=_token_loop)
    out_a, toks_a, js_a = fc.commit(vi_a, b_a, seeds_a, ahead=ahead)
    torch.cuda.synchronize()
    assert torch.equal(out_a, out_p) and torch.equal(seeds_a, seeds_p)
    assert toks_a == toks_p and js_a == js_p
    assert torch.equal(b_a.seq_lens, b_p.seq_lens) and torch.equal(b_a.seq_lens_cpu, b_p.seq_lens_cpu)
    assert b_a.seq_lens_sum == b_p.seq_lens_sum
    assert alloc_a.freed_pages == alloc_p.freed_pages and alloc_a.calls == alloc_p.calls
    none_finish = not any(r.finished() for r in b_p.reqs) and case != "slow"
    assert none_finish == (case == "clean")
    assert len(calls) == (1 if none_finish else 0) and fc.n_ahead == fc.n_launched == len(calls)
    for ra, rp in zip(b_a.reqs, b_p.reqs):
        assert ra.output_ids == rp.output_ids and ra.finished() == rp.finished() and ra.hist == rp.hist
        assert ra.kv_committed_len == rp.kv_committed_len
        want = -(-(rp.kv_committed_len + (K if none_finish else 0)) // page) * page
        assert ra.kv_allocated_len == want
    if none_finish:
        inc, n_free_calls, outs = calls[0]
        assert inc == js_p == [len(t) - 1 for t in toks_p]
        assert n_free_calls == alloc_p.calls and all(o == [] for o in outs)


def test_fast_commit_without_token_loop_raises_for_slow_requests(cuda):
    from gravityocr_amd.sglang_shim import GssFastCommit
    K = 5
    req = _Req(10, 10)
    req.sampling_params.stop_strs = ["</s>"]
    req.kv_committed_len = req.kv_allocated_len = 16
    dev = lambda a: torch.as_tensor(a).to(cuda)
    vi = _NS(predict=dev(np.arange(K + 1, dtype=np.int32)), accept_length=dev(np.array([1], dtype=np.int32)),
             a0=dev(np.array([4], dtype=np.int64)), draft_token_num=K)
    batch = _NS(batch_size=lambda: 1, out_cache_loc=dev(np.arange(16, 16 + K, dtype=np.int64)),
                req_pool_indices=dev(np.array([0])), seq_lens=dev(np.array([16])),
                seq_lens_cpu=torch.tensor([16]), seq_lens_sum=16, reqs=[req], token_to_kv_pool_allocator=_PageAlloc())
    with pytest.raises(NotImplementedError):
        GssFastCommit(K, 4, cuda).commit(vi, batch, dev(np.zeros(2, dtype=np.int64)))
