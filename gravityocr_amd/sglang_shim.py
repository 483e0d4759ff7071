"""SGLang attention / commit backend for the self-spec serving round on the gfx950 kernels: the hook surface the
reference patches into SGLang (attention routed by ``spec_info.selfspec_role``, patches/sglang/
sglang_0.5.10_selfspec.patch:418-541; the planner it replaces, selfspec_fast_attn.py:168-465; the fast commit,
selfspec_fast_commit.py:291-355), written against duck-typed SGLang objects (SGLang is not importable here).

Page size. The reference runs the server at --page-size 1 (flashinfer reads one slot per token through kv_indices).
The attention kernels read 16-token pages (K [page][head][16][D], V [page][head][D][16]), so this backend runs the
server at --page-size 16: SGLang's allocator then hands out whole pages and req_to_token holds slot = page * 16 +
offset, so a request's page table is req_to_token[r, 0::16] // 16 (one device op, no host plan, nothing to copy),
and the KV pool keeps the kernels' layout (``PagedKVPool``; SGLang's set_kv_buffer(layer, loc, k, v) writes into it).

Roles: a draft forward [x0 | MASK x (K-1)] runs gss_draft_attn with its first row causal (the reference's
NON_CAUSAL mask rows + CAUSAL seed row), a verify forward gss_verify_attn (causal, bottom-right aligned); the prefix
is the request's committed length (forward_batch.seq_lens) read from the pages, the window's own K/V from the
forward's k / v. The commit (GssFastCommit) runs gss_ss_commit: packed rows, seeds, the finish cut of every
request, seq_lens and the page-granular free list in one launch, then one page-locked readback and one extend +
check_finished per request; with a draft-ahead callback (selfspec_fast_commit.py:357-440), rounds in which no request
can finish apply their lengths and frees at the readback and launch the next draft before the bookkeeping.
"""
from typing import Callable, List, Optional

import numpy as np
import torch

from . import kernels as gk

PAGE = 16
ROLE_DRAFT, ROLE_VERIFY = "draft", "verify"


class PagedKVPool:
    """The server's KV pool in the attention kernels' layout: per layer K [n_pages, Hkv, 16, D] and V
    [n_pages, Hkv, D, 16] (bf16). Slot s is token s % 16 of page s // 16 (SGLang's slot numbering at page size 16)."""

    def __init__(self, n_layers: int, n_pages: int, n_kv_heads: int, head_dim: int, device, dtype=torch.bfloat16):
        self.k = torch.zeros(n_layers, n_pages, n_kv_heads, PAGE, head_dim, dtype=dtype, device=device)
        self.v = torch.zeros(n_layers, n_pages, n_kv_heads, head_dim, PAGE, dtype=dtype, device=device)

    def set_kv_buffer(self, layer_id: int, loc: torch.Tensor, cache_k: torch.Tensor, cache_v: torch.Tensor):
        """MHATokenToKVPool.set_kv_buffer: token i's K/V [Hkv, D] into slot loc[i]."""
        loc = loc.to(torch.int64)
        page, off = loc // PAGE, loc % PAGE
        self.k[layer_id][page, :, off, :] = cache_k.to(self.k.dtype)
        self.v[layer_id][page, :, :, off] = cache_v.to(self.v.dtype)

    def get_key_buffer(self, layer_id: int) -> torch.Tensor:
        return self.k[layer_id]

    def get_value_buffer(self, layer_id: int) -> torch.Tensor:
        return self.v[layer_id]


class GssSelfSpecAttnBackend:
    """forward_extend for the self-spec draft / verify forwards (both TARGET_VERIFY forwards of K tokens per request).
    ``max_kv_len``: the capacity every request's kv length stays within (it fixes the kernels' key partition, so a
    verify row equals the AR step of the same token bit for bit)."""

    def __init__(self, pool: PagedKVPool, req_to_token: torch.Tensor, n_heads: int, n_kv_heads: int, head_dim: int,
                 max_bs: int, K: int, max_kv_len: int):
        self.pool, self.req_to_token = pool, req_to_token
        self.Hq, self.Hkv, self.D, self.K = n_heads, n_kv_heads, head_dim, K
        self.max_kv_len = max_kv_len
        self.max_pages = (max_kv_len + PAGE - 1) // PAGE
        self.ws = torch.zeros(max(1, gk.attn_workspace_bytes(max_bs, n_heads, n_kv_heads, head_dim, K, max_kv_len)),
                              dtype=torch.uint8, device=req_to_token.device)
        self.page_table = None
        self.prefix = None
        self.role = None

    def init_forward_metadata(self, forward_batch):
        """Per forward: the role, the page table of the batch's requests and their committed lengths (device ops)."""
        spec = forward_batch.spec_info
        self.role = getattr(spec, "selfspec_role", None)
        if self.role not in (ROLE_DRAFT, ROLE_VERIFY):
            raise ValueError(f"self-spec attention: unknown role {self.role!r}")
        self.K = int(getattr(spec, "draft_token_num", self.K))
        rpi = forward_batch.req_pool_indices.to(torch.int64)
        if self.req_to_token.shape[1] < self.max_pages * PAGE:
            raise ValueError("req_to_token rows are shorter than max_kv_len")
        # the kernels read at most max_kv_len prefix keys (the plan's capacity): a longer request would lose its
        # last keys, so it is an error here, where the host copy of the lengths is at hand
        sl_cpu = getattr(forward_batch, "seq_lens_cpu", None)
        if sl_cpu is not None and len(sl_cpu) and int(sl_cpu.max()) > self.max_kv_len:
            raise ValueError(f"a request's kv length {int(sl_cpu.max())} exceeds the backend's max_kv_len "
                             f"{self.max_kv_len}")
        self.page_table = (self.req_to_token[rpi, : self.max_pages * PAGE : PAGE] // PAGE).to(torch.int32).contiguous()
        self.prefix = forward_batch.seq_lens.to(torch.int32).contiguous()

    def forward_extend(self, q, k, v, layer, forward_batch, save_kv_cache: bool = True):
        """q [bs*K, Hq*D], k / v [bs*K, Hkv*D] (this forward's window) -> o [bs*K, Hq*D]. With save_kv_cache the
        window's K/V also go to their slots (forward_batch.out_cache_loc), as SGLang's backends do."""
        bs = forward_batch.req_pool_indices.shape[0]
        W = self.K
        q4 = q.view(bs, W, self.Hq, self.D).contiguous()
        kw = k.view(bs, W, self.Hkv, self.D).contiguous()
        vw = v.view(bs, W, self.Hkv, self.D).contiguous()
        if save_kv_cache:
            self.pool.set_kv_buffer(layer.layer_id, forward_batch.out_cache_loc, kw.view(-1, self.Hkv, self.D),
                                    vw.view(-1, self.Hkv, self.D))
        o = torch.empty_like(q4)
        gk.window_attention(q4, self.pool.get_key_buffer(layer.layer_id), self.pool.get_value_buffer(layer.layer_id),
                           self.page_table, self.prefix, kw, vw, o,
                           n_causal=1 if self.role == ROLE_DRAFT else None, scale=float(layer.scaling),
                           max_kv_len=self.max_kv_len, workspace=self.ws)
        return o.view(bs * W, self.Hq * self.D)


def _round_up(x: int, m: int) -> int:
    return -(-x // m) * m


def stop_ids_of(req) -> List[int]:
    """The token ids that end a request (SGLang's token-based finish check: the request's stop_token_ids, its
    eos_token_ids and the tokenizer's eos and additional stop ids), none with ignore_eos."""
    sp = req.sampling_params
    if sp.ignore_eos:
        return []
    tk = req.tokenizer
    ids = list(sp.stop_token_ids or ()) + list(req.eos_token_ids or ())
    if tk is not None:
        ids += [tk.eos_token_id] if tk.eos_token_id is not None else []
        ids += list(getattr(tk, "additional_stop_token_ids", None) or ())
    return sorted(set(int(x) for x in ids))


def cut_rule_applies(req) -> bool:
    """Whether the device cut rule decides this request's finish: only length, stop ids and the vocabulary bound
    can end it (no grammar to advance, no stop strings or regexes, no pending finish, not finished already)."""
    sp = req.sampling_params
    return (req.grammar is None and not req.to_finish and not req.finished() and not sp.stop_strs
            and not sp.stop_regex_strs and req.vocab_size is not None)


class GssFastCommit:
    """The serving round's commit on gss_ss_commit at KV page size ``page``: one launch does the packed readback
    rows, the seed pool, the cut index of every request (where its finish is decided by length, stop ids and the
    vocabulary bound), seq_lens += cut and the free list of the verify slots in pages that hold no kept token; one
    page-locked readback; then per request one extend of output_ids and one check_finished.

    Requests the cut rule does not cover (grammar, stop strings / regexes, a pending finish) go through
    ``token_loop(req, T) -> j``, the per-token append-and-check path (a deployment passes the reference's own,
    selfspec_commit_rules.commit_slow, adapted to return j); without one such a request raises. When it stops
    before the end of T, its device length and free pages are corrected on the stream (no extra sync)."""

    def __init__(self, K: int, max_bs: int, device, page: int = PAGE, max_stop: int = 16,
                 token_loop: Optional[Callable] = None):
        self.K, self.max_bs, self.device, self.page = K, max_bs, device, page
        self.max_stop = max_stop
        self.token_loop = token_loop
        i32 = dict(dtype=torch.int32)
        self.packed_dev = torch.zeros(max_bs, K + 2, device=device, **i32)
        self.cut_dev = torch.zeros(max_bs + 1, device=device, **i32)       # [bs] cut, then the free count
        self.free_dev = torch.zeros(max_bs * K, dtype=torch.int64, device=device)
        # finish-rule inputs (budget, vocabulary bound, stop ids), staged in page-locked memory and copied on the
        # stream before the launch
        self.budget_host = torch.zeros(max_bs, pin_memory=True, **i32)
        self.vocab_host = torch.zeros(max_bs, pin_memory=True, **i32)
        self.stop_host = torch.zeros(max_bs, max_stop, pin_memory=True, **i32)
        self.budget_dev = torch.zeros(max_bs, device=device, **i32)
        self.vocab_dev = torch.zeros(max_bs, device=device, **i32)
        self.stop_dev = torch.zeros(max_bs, max_stop, device=device, **i32)
        self.packed_host = torch.zeros(max_bs, K + 2, pin_memory=True, **i32)
        self.cut_host = torch.zeros(max_bs + 1, pin_memory=True, **i32)
        self.event = torch.cuda.Event()
        self.n_rounds = 0
        self.n_ahead = self.n_launched = 0   # draft-ahead: rounds settled before the bookkeeping, drafts launched

    def _stage_rules(self, reqs) -> None:
        """Host values of the finish rule for this round's requests, then their copies to the device (queued on
        the stream ahead of the commit kernel)."""
        bs = len(reqs)
        budget, vocab, stop = (t[:bs].numpy() for t in (self.budget_host, self.vocab_host, self.stop_host))
        budget.fill(-1)                                   # -1: the per-token path decides
        vocab.fill(0)
        stop.fill(-1)
        for i, req in enumerate(reqs):
            if not cut_rule_applies(req):
                continue
            ids = stop_ids_of(req)
            if len(ids) > self.max_stop:
                raise ValueError(f"request has {len(ids)} stop ids, more than the {self.max_stop} staged")
            budget[i] = max(0, req.sampling_params.max_new_tokens - len(req.output_ids))
            vocab[i] = req.vocab_size
            stop[i, :len(ids)] = ids
        for h, d in ((self.budget_host, self.budget_dev), (self.vocab_host, self.vocab_dev),
                     (self.stop_host, self.stop_dev)):
            d[:bs].copy_(h[:bs], non_blocking=True)

    def commit(self, vi, batch, seeds: torch.Tensor, ahead=None):
        """Returns (next seeds device [bs], tokens per request, j per request).

        ``ahead`` (draft-ahead serving, None = the plain round): a callable ahead(inc) -> bool that launches the next
        round's draft. When the readback shows that no request can finish this round (``_none_finish``), every cut
        is the round's full length, so the lengths and the free pages are final at the readback: they are applied
        (the frees before the next draft allocates), ahead(inc) runs with inc[i] = the length increment of request
        i, and the per-request bookkeeping follows while that draft runs on the GPU; a launched draft's K slots
        count in kv_allocated_len. Any other round settles exactly as the plain one."""
        st = self._launch(vi, batch, seeds)
        if ahead is None or not self._none_finish(st):
            return self._settle(st, batch)
        bs = st["bs"]
        inc = [int(c) for c in st["cuts"]]
        batch.seq_lens_cpu += torch.as_tensor(inc, dtype=batch.seq_lens_cpu.dtype)
        batch.seq_lens_sum += sum(inc)
        self._free(batch, [self.free_dev[:st["n_free"]]] if st["n_free"] else [])
        launched = bool(ahead(inc))
        toks, js = [], []
        for i, req in enumerate(batch.reqs):
            T, j = st["T"][i], inc[i]
            req.output_ids.extend(T)
            req.check_finished(len(T))
            if req.finished():
                raise RuntimeError(f"draft-ahead commit: request {i} finished in a round the readback showed it "
                                   f"could not finish in (tokens {T})")
            self._count(req, j, st["acc"][i])
            req.kv_committed_len += j + 1
            req.kv_allocated_len = _round_up(req.kv_committed_len + (self.K if launched else 0), self.page)
            toks.append(T)
            js.append(j)
        self.n_rounds += 1
        self.n_ahead += 1
        self.n_launched += launched
        return st["out"], toks, js

    def _launch(self, vi, batch, seeds) -> dict:
        """The commit kernel and the round's one readback; returns the host view of the round."""
        reqs = batch.reqs
        bs, K, pg = batch.batch_size(), self.K, self.page
        if vi.draft_token_num != K or bs > self.max_bs:
            raise ValueError(f"commit: window {vi.draft_token_num} / batch {bs} vs {K} / {self.max_bs}")
        loc = batch.out_cache_loc
        S = batch.seq_lens_cpu.numpy().copy()             # verify row r of request i sits at position S[i] + r
        self._stage_rules(reqs)
        out = torch.empty(bs, dtype=torch.int64, device=self.device)
        gk.ss_commit(vi.predict, vi.accept_length, vi.a0, batch.req_pool_indices, seeds, batch.seq_lens, loc,
                     self.packed_dev[:bs], self.free_dev[: bs * K], out, K=K, page=pg, budget=self.budget_dev[:bs],
                     vocab=self.vocab_dev[:bs], stop_ids=self.stop_dev[:bs], cut=self.cut_dev[:bs],
                     n_free=self.cut_dev[bs:bs + 1])
        self.packed_host[:bs].copy_(self.packed_dev[:bs], non_blocking=True)
        self.cut_host[:bs + 1].copy_(self.cut_dev[:bs + 1], non_blocking=True)
        self.event.record()
        self.event.synchronize()                          # the round's one readback
        rows = self.packed_host[:bs].numpy()
        acc = [int(rows[i, 1]) for i in range(bs)]
        # host lists: the page-locked buffers are rewritten by the next round's copies
        T = [[int(rows[i, 0])] + rows[i, 2:3 + acc[i]].tolist() for i in range(bs)]
        return dict(bs=bs, S=S, loc=loc, out=out, acc=acc, T=T, cuts=self.cut_host[:bs].numpy().tolist(),
                    n_free=int(self.cut_host[bs]), by_rule=(self.budget_host[:bs].numpy() >= 0).tolist())

    def _none_finish(self, st) -> bool:
        """True when no request of the round can finish: every request is under the cut rule, its remaining budget
        exceeds the round's token count (so length cannot fire), and none of the round's ids is one of its stop ids
        or outside [0, vocab]. Then its cut is the last token and check_finished leaves it running."""
        bs = st["bs"]
        budget, vocab, stop = (t[:bs].numpy() for t in (self.budget_host, self.vocab_host, self.stop_host))
        for i in range(bs):
            T = st["T"][i]
            if not st["by_rule"][i] or budget[i] <= len(T) or min(T) < 0 or max(T) > vocab[i]:
                return False
            ids = stop[i]
            if np.isin(T, ids[ids >= 0]).any():
                return False
        return True

    def _count(self, req, j, a):
        """acceptance counters: the verified count, or 0 when a0 itself ended the request"""
        verified = 0 if (j == 0 and req.finished()) else a + 1
        req.spec_verify_ct += 1
        req.spec_accepted_tokens += verified
        req.update_spec_acceptance_histogram(verified)

    @staticmethod
    def _free(batch, freed):
        if freed:
            fl = torch.cat(freed) if len(freed) > 1 else freed[0]
            # inside a free group the allocator keeps the tensor itself: never hand it a view of a reused buffer
            alloc = batch.token_to_kv_pool_allocator
            alloc.free(fl if getattr(alloc, "is_not_in_free_group", True) else fl.clone())

    def _settle(self, st, batch):
        """Per request: extend + check_finished (or the per-token path), counters, kv lengths; then the host and
        device lengths and the frees."""
        K, pg, S, loc = self.K, self.page, st["S"], st["loc"]
        extra_free = []
        toks, js = [], []
        for i, req in enumerate(batch.reqs):
            a, T, j = st["acc"][i], st["T"][i], st["cuts"][i]
            if st["by_rule"][i]:
                req.output_ids.extend(T[: j + 1])
                req.check_finished(j + 1)
            else:
                if self.token_loop is None:
                    raise NotImplementedError("a request outside the cut rule (grammar, stop strings) needs the "
                                              "per-token path: pass token_loop")
                jl = int(self.token_loop(req, T))
                if jl < j:
                    # stopped inside the round: the device advanced seq_lens by j = a + 1 and freed the pages past
                    # S + j; the kept rows end at S + jl, so the pages between the two page boundaries go as well
                    batch.seq_lens[i:i + 1].sub_(j - jl)
                    lo = _round_up(int(S[i]) + jl, pg) - int(S[i])
                    hi = min(K, _round_up(int(S[i]) + j, pg) - int(S[i]))
                    if hi > lo:
                        extra_free.append(loc[i * K + lo:i * K + hi])
                    j = jl
            self._count(req, j, a)
            req.kv_committed_len += j + 1
            req.kv_allocated_len = _round_up(req.kv_committed_len, pg)
            toks.append(T[: j + 1])
            js.append(j)
        batch.seq_lens_cpu += torch.as_tensor(js, dtype=batch.seq_lens_cpu.dtype)
        batch.seq_lens_sum += sum(js)
        self._free(batch, ([self.free_dev[:st["n_free"]]] if st["n_free"] else []) + extra_free)
        self.n_rounds += 1
        return st["out"], toks, js
