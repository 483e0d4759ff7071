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
forward's k / v. The commit runs gss_ss_commit (packed row, seeds, seq_lens, compacted free list) and the reference's
host bookkeeping over one page-locked readback.
"""
from typing import Optional

import torch

from . import kernels as gk
from .selfspec_commit_rules import host_commit

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


class GssFastCommit:
    """SelfSpecFastCommit.commit on gss_ss_commit: the round's device bookkeeping in one launch, one page-locked
    readback, then the reference's host bookkeeping (host_commit, lengths, frees of the rejected verify slots)."""

    def __init__(self, K: int, max_bs: int, device):
        self.K, self.max_bs, self.device = K, max_bs, device
        self.packed_dev = torch.zeros(max_bs, K + 2, dtype=torch.int32, device=device)
        self.packed_host = torch.zeros(max_bs, K + 2, dtype=torch.int32, pin_memory=True)
        self.free_dev = torch.zeros(max_bs * K, dtype=torch.int64, device=device)
        self.event = torch.cuda.Event()
        self.n_rounds = 0

    def commit(self, vi, batch, seeds: torch.Tensor, ahead=None):
        """Returns (next seeds device [bs], tokens per request, j per request)."""
        if ahead is not None:
            raise NotImplementedError("the draft-ahead commit is not built")
        bs, Kw = batch.batch_size(), self.K
        if vi.draft_token_num != Kw or bs > self.max_bs:
            raise ValueError(f"commit: window {vi.draft_token_num} / batch {bs} vs {Kw} / {self.max_bs}")
        loc = batch.out_cache_loc
        out = torch.empty(bs, dtype=torch.int64, device=self.device)
        gk.ss_commit(vi.predict, vi.accept_length, vi.a0, batch.req_pool_indices, seeds, batch.seq_lens, loc,
                    self.packed_dev[:bs], self.free_dev[: bs * Kw], out, K=Kw)
        host = self.packed_host[:bs]
        host.copy_(self.packed_dev[:bs], non_blocking=True)
        self.event.record()
        self.event.synchronize()            # the round's one readback
        rows = host.numpy().tolist()
        toks, js, accs = host_commit(batch.reqs, rows)
        sl = batch.seq_lens_cpu.numpy()
        fix, n_free = False, 0
        for i, req in enumerate(batch.reqs):
            j, a = js[i], accs[i]
            sl[i] += j
            req.kv_committed_len += j + 1
            req.kv_allocated_len = req.kv_committed_len
            n_free += Kw - 1 - a
            if j < a + 1:               # finished inside the round: the kernel advanced seq_lens by acc + 1
                batch.seq_lens[i:i + 1].sub_(a + 1 - j)
                fix = True
        batch.seq_lens_sum += sum(js)
        alloc = batch.token_to_kv_pool_allocator
        if bs == 1:
            alloc.free(loc[js[0]:])
        elif fix:
            alloc.free(torch.cat([loc[i * Kw + js[i]:(i + 1) * Kw] for i in range(bs)]))
        elif n_free:
            fl = self.free_dev[:n_free]
            alloc.free(fl if getattr(alloc, "is_not_in_free_group", True) else fl.clone())
        self.n_rounds += 1
        return out, toks, js
