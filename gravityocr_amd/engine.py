"""The self-spec round on one MI355X: GLM decoder forward over a paged KV cache through the C-ABI kernels,
with every round-to-round quantity (committed lengths, boundary tokens, accept lengths) resident on the device so a
whole round is captured once as a HIP graph and replayed.

Per layer of a window forward (rows = bs * W, any count: above 64 rows the GEMMs run a tiled kernel with the skinny
kernel's exact operation sequence, so every row is computed the same way at every batch size):
    gss_gemm_rope_stage             fused q|k|v projection, RoPE on q and k, window K/V staged (not yet in the cache)
    gss_draft_attn / gss_verify_attn   paged prefix + window, draft or verify mask, under the decoder's attention plan
    gss_gemm_parts (o_proj)         fp32 k-split partial sums
    gss_add_rmsnorm_parts           residual + post-attention sandwich norm + the MLP input norm (at <= 12 rows
                                    the same norm runs inside the gate_up GEMM's prologue instead: fuse_gate_norm,
                                    on by default)
    gss_gemm_swiglu                 gate_up projection with the SwiGLU epilogue
    gss_gemm_parts (down)           fp32 k-split partial sums
    gss_add_rmsnorm_parts           residual + post-MLP norm + the next layer's input norm
The prefill (one long prompt) runs the same GEMMs (gss_gemm, gss_gemm_swiglu), gss_rope_stage, gss_kv_commit and
the verify attention over causal chunks of the prompt.
A round (the serving full-draft round, patches/sglang/.../selfspec_diffusion_worker.py:660-961):
    draft forward [x0 | MASK x B] -> gss_argmax_accept (argmax only) -> gss_kv_commit of row 0 (x0)
    verify forward [a0, d_1..d_B] -> gss_argmax_accept (argmax + accept + bonus) -> gss_kv_commit of acc+1 rows
"""
import math
from dataclasses import dataclass, field
from typing import Dict, List, Optional, Tuple

import numpy as np
import torch

from . import kernels as K
from .model import GlmTextConfig

PAGE = K.PAGE


class _Bufs:
    """Activation buffers of one (bs, W) window shape."""

    def __init__(self, eng: "GssEngine", bs: int, W: int):
        c, dev, bf = eng.cfg, eng.device, torch.bfloat16
        rows = bs * W
        self.bs, self.W = bs, W
        self.h = torch.empty(rows, c.hidden, dtype=bf, device=dev)
        self.h2 = torch.empty(rows, c.hidden, dtype=bf, device=dev)   # residual ping-pong for the fused norms
        self.x = torch.empty(rows, c.hidden, dtype=bf, device=dev)
        self.qkv = torch.empty(rows, c.qkv_dim, dtype=bf, device=dev)
        self.q = torch.empty(bs, W, c.n_heads, c.head_dim, dtype=bf, device=dev)
        self.o = torch.empty(bs, W, c.n_heads, c.head_dim, dtype=bf, device=dev)
        self.a = torch.empty(rows, c.hidden, dtype=bf, device=dev)
        # fp32 partial sums of o_proj and down_proj (gemm_parts), summed by the norm that follows
        self.ap_o = torch.empty(K.gemm_parts_count(c.hidden, c.n_heads * c.head_dim), rows, c.hidden,
                                dtype=torch.float32, device=dev)
        self.ap_d = torch.empty(K.gemm_parts_count(c.hidden, c.ffn), rows, c.hidden, dtype=torch.float32, device=dev)
        self.gu = torch.empty(rows, 2 * c.ffn, dtype=bf, device=dev)
        self.act = torch.empty(rows, c.ffn, dtype=bf, device=dev)
        self.logits = torch.empty(rows, c.vocab, dtype=bf, device=dev)
        self.k_win = torch.empty(c.n_layers, bs, W, c.n_kv_heads, c.head_dim, dtype=bf, device=dev)
        self.v_win = torch.empty_like(self.k_win)


class GssEngine:
    """Weights, paged KV pool and kernels for up to ``max_bs`` sequences of up to ``max_len`` tokens each."""

    def __init__(self, cfg: GlmTextConfig, weights: Dict[str, torch.Tensor], *, max_bs: int, max_len: int,
                 device="cuda", page_seed: int = 0, max_win: int = 48):
        self.cfg = cfg
        # the GEMM prologue norm is bit-identical only to an unsplit GEMM; the decode path normalizes in the GEMM
        # epilogues instead, for every row count (0 = the prologue path is off)
        self.fuse_norm_rows = 0
        # sandwich norms in the o_proj / down GEMM epilogues (one launch less each) instead of gss_add_rmsnorm
        self.post_norm = False
        # the post-attention norms in the gate_up GEMM's prologue (persistent kernel: once per CU, while the first
        # weight tiles load) instead of a gss_add_rmsnorm launch; bit-identical to the separate norm, for at most 12
        # rows (one row per wave of the GEMM's 12) and a hidden size the prologue supports (a multiple of 512,
        # <= 1536); with gemm_parts, the post-MLP norms likewise in the next layer's qkv prologue and the last one in
        # the LM head's. On: with the wave reductions on lane swaps and DPP the 1-row AR step takes 715 against
        # 726 us on the 16-layer decoder with the gate_up prologue alone (the windows of a round have more rows and
        # keep the separate norms)
        self.fuse_gate_norm = True
        self.gemm_parts = True    # o_proj / down as k-split partial sums (gemm_parts + the parts norms)
        self.device = torch.device(device)
        self.max_bs, self.max_len, self.max_win = max_bs, max_len, max_win
        dev, bf = self.device, torch.bfloat16

        def up(t):
            return t.detach().to(device=dev, dtype=bf).contiguous()

        L = cfg.n_layers
        self.embed = up(weights["embed"])
        self.wqkv = [up(torch.cat([weights[f"{l}.wq"], weights[f"{l}.wk"], weights[f"{l}.wv"]], 0)) for l in range(L)]
        self.wo = [up(weights[f"{l}.wo"]) for l in range(L)]
        # gate_up rows interleaved (2i = gate_i, 2i+1 = up_i) so one GEMM tile holds both halves of a SwiGLU unit
        self.wgu = [up(weights[f"{l}.w_gate_up"].view(2, cfg.ffn, cfg.hidden).transpose(0, 1)
                       .reshape(2 * cfg.ffn, cfg.hidden)) for l in range(L)]
        self.wdown = [up(weights[f"{l}.w_down"]) for l in range(L)]
        self.n_in = [up(weights[f"{l}.in_norm"]) for l in range(L)]
        self.n_psa = [up(weights[f"{l}.post_self_attn_norm"]) for l in range(L)]
        self.n_pa = [up(weights[f"{l}.post_attn_norm"]) for l in range(L)]
        self.n_pm = [up(weights[f"{l}.post_mlp_norm"]) for l in range(L)]
        self.n_final = up(weights["norm"])
        self.lm_head = up(weights["lm_head"])
        rot = cfg.rot_dim
        self.inv_freq = (1.0 / (cfg.rope_theta ** (torch.arange(0, rot, 2, dtype=torch.int64).float() / rot))).to(dev)
        self.scale = cfg.head_dim ** -0.5

        # paged KV pool: every sequence slot owns ceil(max_len / 16) pages, drawn from a seeded permutation of the
        # pool (pages of one sequence are scattered, as a shared serving pool leaves them)
        self.pages_per_seq = (max_len + PAGE - 1) // PAGE
        n_pages = max_bs * self.pages_per_seq
        perm = np.random.default_rng(page_seed).permutation(n_pages).astype(np.int32)
        self.page_table = torch.from_numpy(perm.reshape(max_bs, self.pages_per_seq)).to(dev)
        self.k_pages = torch.zeros(L, n_pages, cfg.n_kv_heads, PAGE, cfg.head_dim, dtype=bf, device=dev)
        self.v_pages = torch.zeros(L, n_pages, cfg.n_kv_heads, cfg.head_dim, PAGE, dtype=bf, device=dev)
        self.seq_lens = torch.zeros(max_bs, dtype=torch.int32, device=dev)

        self.ws_attn = torch.zeros(max(1, K.attn_workspace_bytes(max_bs, cfg.n_heads, cfg.n_kv_heads, cfg.head_dim,
                                                                 max_win, max_len)), dtype=torch.uint8, device=dev)
        self.ws_arg = torch.zeros(K.argmax_workspace_bytes(max_bs, max_win, cfg.vocab), dtype=torch.uint8, device=dev)
        self.ws_commit = torch.zeros(K.commit_workspace_bytes(max_bs), dtype=torch.uint8, device=dev)
        rows = max_bs * max_win
        shapes = [(cfg.qkv_dim, cfg.hidden), (cfg.hidden, cfg.n_heads * cfg.head_dim), (2 * cfg.ffn, cfg.hidden),
                  (cfg.hidden, cfg.ffn), (cfg.vocab, cfg.hidden)]
        # sized at 64 rows or more: every call (the prefill's too) then fits; larger M needs no more
        self.ws_gemm = torch.zeros(max(K.gemm_workspace_bytes(max(rows, 64), n, kd) for n, kd in shapes),
                                   dtype=torch.uint8, device=dev)
        self._bufs: Dict[Tuple[int, int], _Bufs] = {}
        self._retired_ws: List[torch.Tensor] = []

    # ------------------------------------------------------------------------------------------ primitives ------
    def attn_plan(self, bs: int, max_kv_len: Optional[int] = None, **policy):
        """The attention plan of a bs-sequence batch over this cache (the library default unless policy overrides
        target_wgs / min_tiles / wide_min)."""
        return K.attn_plan(bs, self.cfg.n_kv_heads, self.max_len if max_kv_len is None else max_kv_len, **policy)

    def _attn_ws(self, bs: int, W: int, plan) -> torch.Tensor:
        """The attention workspace, grown (outside graph capture: every shape runs eagerly before it is captured)
        when a plan needs more than the engine's default."""
        c = self.cfg
        need = K.attn_workspace_bytes(bs, c.n_heads, c.n_kv_heads, c.head_dim, W, plan)
        if need > self.ws_attn.numel():
            # graphs captured earlier still hold the old buffer's address: it is kept, never freed
            self._retired_ws.append(self.ws_attn)
            self.ws_attn = torch.zeros(need, dtype=torch.uint8, device=self.device)
        return self.ws_attn

    def bufs(self, bs: int, W: int) -> _Bufs:
        key = (bs, W)
        if key not in self._bufs:
            if bs > self.max_bs or W > self.max_win:
                raise ValueError(f"window {bs}x{W} exceeds the engine's {self.max_bs}x{self.max_win}")
            self._bufs[key] = _Bufs(self, bs, W)
        return self._bufs[key]

    def forward(self, b: _Bufs, *, ids: Optional[torch.Tensor] = None, emb: Optional[torch.Tensor] = None,
                n_causal: Optional[int], seq_lens: Optional[torch.Tensor] = None,
                page_table: Optional[torch.Tensor] = None, pos_delta: Optional[torch.Tensor] = None,
                max_kv_len: Optional[int] = None, attn_plan=None, logits_f32: bool = False) -> torch.Tensor:
        """One window forward of all layers. ``ids`` int32/int64 [bs, W] or ``emb`` [bs*W, H]; n_causal None =
        verify mask. The window's K/V is left in b.k_win / b.v_win (not committed). ``attn_plan``: the attention
        plan (default: the library's for bs sequences of capacity max_kv_len). Returns logits [bs, W, V] (bf16;
        fp32 with ``logits_f32``: the LM head's sums before their bf16 rounding, for the sampled round)."""
        c = self.cfg
        bs, W = b.bs, b.W
        b.want_f32 = logits_f32
        sl = self.seq_lens[:bs] if seq_lens is None else seq_lens
        pt = self.page_table[:bs] if page_table is None else page_table
        plan = self.attn_plan(bs, max_kv_len) if attn_plan is None else attn_plan
        self._attn_ws(bs, W, plan)
        # the GEMM-prologue norm path (off by default: it would not match the split-K epilogue path bit for bit)
        fused = bs * W <= min(64, self.fuse_norm_rows) and c.hidden % 512 == 0 and c.hidden <= 1536
        if logits_f32 and fused:
            raise NotImplementedError("fp32 logits are produced by the unfused-norm decode path")
        if emb is None and ids.dtype == torch.int32 and ids.is_contiguous() and not fused:
            K.embed_rmsnorm(self.embed, ids, self.n_in[0], b.h, b.x, c.rms_eps)   # lookup + first input norm
        else:
            if emb is not None:
                b.h.copy_(emb.view(bs * W, c.hidden))
            else:
                torch.index_select(self.embed, 0, ids.reshape(-1), out=b.h)
            if fused:
                return self._forward_fused(b, n_causal, sl, pt, pos_delta, plan)
            K.rmsnorm(b.h, self.n_in[0], b.x, c.rms_eps)
        return self._forward_own(b, n_causal, sl, pt, pos_delta, plan)

    def _forward_own(self, b: _Bufs, n_causal, sl, pt, pos_delta, plan) -> torch.Tensor:
        """Decode forward on the batch-invariant GEMMs (b.x already holds the first input norm). Per layer:
        [qkv + RoPE + staging], attention (+ split merge), o_proj, residual norm, [gate_up + SwiGLU], down,
        residual norm (the norms inside the o_proj / down GEMM epilogues when post_norm is set; the post-attention
        norms inside the gate_up prologue when fuse_gate_norm is set)."""
        c = self.cfg
        bs, W = b.bs, b.W
        ws = self.ws_gemm
        h, h_alt = b.h, b.h2  # the residual stream; a GEMM prologue writes the updated one to the other buffer
        # windows of at most 12 rows: every parts norm runs in the next GEMM's prologue (gate_up, the next layer's
        # qkv, the LM head) instead of its own launch
        fuse = (self.fuse_gate_norm and self.gemm_parts and (c.hidden // 64) % 4 == 0 and not self.post_norm
                and bs * W <= 12 and c.hidden % 512 == 0 and c.hidden <= 1536)
        pending = None  # down_proj's parts and the norm weights the next prologue applies to them
        for l in range(c.n_layers):
            if pending is not None:
                K.gemm_rope_stage(None, self.wqkv[l], sl, self.inv_freq, b.q, b.k_win[l], b.v_win[l],
                                  rot_dim=c.rot_dim, pos_delta=pos_delta, workspace=ws,
                                  pro=dict(a_parts=pending[0], h_in=h, h_out=h_alt, w_post=pending[1],
                                           w_next=pending[2], eps=c.rms_eps))
                h, h_alt = h_alt, h
                pending = None
            else:
                K.gemm_rope_stage(b.x, self.wqkv[l], sl, self.inv_freq, b.q, b.k_win[l], b.v_win[l],
                                  rot_dim=c.rot_dim, pos_delta=pos_delta, workspace=ws)
            K.window_attention(b.q, self.k_pages[l], self.v_pages[l], pt, sl, b.k_win[l], b.v_win[l], b.o,
                               n_causal=n_causal, scale=self.scale, plan=plan, workspace=self.ws_attn)
            nxt = self.n_in[l + 1] if l + 1 < c.n_layers else self.n_final
            if self.post_norm:
                K.gemm(b.o.view(bs * W, -1), self.wo[l], b.a, workspace=ws,
                       post=dict(h=h, w_post=self.n_psa[l], w_next=self.n_pa[l], x=b.x, eps=c.rms_eps))
                K.gemm_swiglu(b.x, self.wgu[l], b.act, workspace=ws)
                K.gemm(b.act, self.wdown[l], b.a, workspace=ws,
                       post=dict(h=h, w_post=self.n_pm[l], w_next=nxt, x=b.x, eps=c.rms_eps))
            elif self.gemm_parts and (c.hidden // 64) % 4 == 0:
                # o_proj and down as k-split partial sums, added in split order by the norm that follows
                K.gemm_parts(b.o.view(bs * W, -1), self.wo[l], b.ap_o)
                if fuse:
                    K.gemm_swiglu(None, self.wgu[l], b.act, workspace=ws,
                                  pro=dict(a_parts=b.ap_o, h_in=h, h_out=h_alt, w_post=self.n_psa[l],
                                           w_next=self.n_pa[l], eps=c.rms_eps))
                    h, h_alt = h_alt, h
                else:
                    K.add_rmsnorm_parts(b.ap_o, self.n_psa[l], h, self.n_pa[l], b.x, c.rms_eps)
                    K.gemm_swiglu(b.x, self.wgu[l], b.act, workspace=ws)
                K.gemm_parts(b.act, self.wdown[l], b.ap_d)
                if fuse:
                    pending = (b.ap_d, self.n_pm[l], nxt)
                else:
                    K.add_rmsnorm_parts(b.ap_d, self.n_pm[l], h, nxt, b.x, c.rms_eps)
            else:
                K.gemm(b.o.view(bs * W, -1), self.wo[l], b.a, workspace=ws)
                if self.fuse_gate_norm and bs * W <= 12 and c.hidden % 512 == 0 and c.hidden <= 1536:
                    K.gemm_swiglu(None, self.wgu[l], b.act, workspace=ws,
                                  pro=dict(a=b.a, h_in=h, h_out=h_alt, w_post=self.n_psa[l], w_next=self.n_pa[l],
                                           eps=c.rms_eps))
                    h, h_alt = h_alt, h
                else:
                    K.add_rmsnorm(b.a, self.n_psa[l], h, self.n_pa[l], b.x, c.rms_eps)
                    K.gemm_swiglu(b.x, self.wgu[l], b.act, workspace=ws)
                K.gemm(b.act, self.wdown[l], b.a, workspace=ws)
                K.add_rmsnorm(b.a, self.n_pm[l], h, nxt, b.x, c.rms_eps)
        x_in, pro = b.x, None
        if pending is not None:  # the final norm in the LM head's prologue (the residual is not needed after it)
            x_in, pro = None, dict(a_parts=pending[0], h_in=h, h_out=None, w_post=pending[1], w_next=pending[2],
                                   eps=c.rms_eps)
        if getattr(b, "want_f32", False):
            if getattr(b, "logits32", None) is None:
                b.logits32 = torch.empty(bs * W, c.vocab, dtype=torch.float32, device=self.device)
            K.gemm(x_in, self.lm_head, b.logits32, pro=pro, workspace=ws)
            return b.logits32.view(bs, W, c.vocab)
        K.gemm(x_in, self.lm_head, b.logits, pro=pro, workspace=ws)
        return b.logits.view(bs, W, c.vocab)

    def _forward_fused(self, b: _Bufs, n_causal, sl, pt, pos_delta, plan) -> torch.Tensor:
        """Decode forward with the sandwich norms folded into the GEMM prologues: per layer
        [norm + qkv + RoPE], attention (+ split merge), o_proj, [norm + gate_up + SwiGLU], down."""
        c = self.cfg
        bs, W = b.bs, b.W
        eps = c.rms_eps
        h_a, h_b = b.h, b.h2
        prev = None
        for l in range(c.n_layers):
            K.gemm_rope_stage(None, self.wqkv[l], sl, self.inv_freq, b.q, b.k_win[l], b.v_win[l], rot_dim=c.rot_dim,
                              pos_delta=pos_delta,
                              pro=dict(a=prev, h_in=h_a, h_out=h_b, w_post=self.n_pm[l - 1] if prev is not None else None,
                                       w_next=self.n_in[l], eps=eps))
            K.window_attention(b.q, self.k_pages[l], self.v_pages[l], pt, sl, b.k_win[l], b.v_win[l], b.o,
                               n_causal=n_causal, scale=self.scale, plan=plan, workspace=self.ws_attn)
            K.gemm(b.o.view(bs * W, -1), self.wo[l], b.a)
            K.gemm_swiglu(None, self.wgu[l], b.act,
                          pro=dict(a=b.a, h_in=h_b, h_out=h_a, w_post=self.n_psa[l], w_next=self.n_pa[l], eps=eps))
            K.gemm(b.act, self.wdown[l], b.a)
            prev = b.a
        K.gemm(None, self.lm_head, b.logits,
               pro=dict(a=b.a, h_in=h_a, h_out=None, w_post=self.n_pm[c.n_layers - 1], w_next=self.n_final, eps=eps))
        return b.logits.view(bs, W, c.vocab)

    def commit(self, b: _Bufs, *, n_rows=None, n_add: int = 0, slots=None, seq_lens=None, page_table=None):
        bs = b.bs
        K.kv_commit(b.k_win, b.v_win, self.k_pages, self.v_pages,
                    self.page_table[:bs] if page_table is None else page_table,
                    self.seq_lens[:bs] if seq_lens is None else seq_lens, self.ws_commit, n_rows=n_rows, n_add=n_add,
                    slots=slots)

    def argmax(self, logits, target, **kw):
        K.argmax_accept(logits, target, self.ws_arg, **kw)

    # ------------------------------------------------------------------------------------------ prefill ---------
    def prefill(self, slot: int, emb: torch.Tensor, chunk: int = 64, pos_delta: Optional[torch.Tensor] = None,
                positions: Optional[torch.Tensor] = None, logits_rows: Optional[Tuple[int, int]] = None):
        """Causal prefill of one sequence slot from its prompt embeddings [P, H]. The layer runs the decode
        forward's kernels over all P rows (the tiled GEMM above 64 rows): q|k|v with the RoPE epilogue (or, with
        M-RoPE ``positions``, the plain GEMM and gss_rope_stage_mrope), o_proj and down as k-split parts with the
        parts norms, gate_up with the SwiGLU epilogue; attention runs in causal chunks of ``chunk`` rows through the
        verify kernel (prefix from the pages, chunk as the window, at most 64 rows: the widest window the kernels
        take, and the fastest of 16 / 32 / 48 / 64 for an 8192-token prompt) under the bs = 1 plan, and K/V is
        committed layer by layer. Every GEMM and norm computes a row the same way at any row count and the attention
        does not depend on where a key comes from, so a prefilled row equals the AR step of the same token bit for
        bit (at any chunk size). Row j sits at position j (+ pos_delta), or at the M-RoPE positions ``positions``
        int32 [P, 3] (t, h, w) when given.
        Returns the logits of the last prompt row [V] (bf16), or of rows [r0, r1) as [r1 - r0, V] when
        ``logits_rows`` = (r0, r1)."""
        c, dev, bf = self.cfg, self.device, torch.bfloat16
        P = emb.shape[0]
        if P > self.max_len:
            raise ValueError("prompt longer than the engine capacity")
        if positions is not None and tuple(positions.shape) != (P, 3):
            raise ValueError("positions must be [P, 3]")
        eps = c.rms_eps
        pt = self.page_table[slot:slot + 1]
        h = emb.to(device=dev, dtype=bf).contiguous().clone()
        x = torch.empty_like(h)
        q = torch.empty(1, P, c.n_heads, c.head_dim, dtype=bf, device=dev)
        o = torch.empty_like(q)
        kw = torch.empty(1, 1, P, c.n_kv_heads, c.head_dim, dtype=bf, device=dev)
        vw = torch.empty_like(kw)
        act = torch.empty(P, c.ffn, dtype=bf, device=dev)
        parts_path = self.gemm_parts and (c.hidden // 64) % 4 == 0
        if parts_path:
            np_o = K.gemm_parts_count(c.hidden, c.n_heads * c.head_dim)
            np_d = K.gemm_parts_count(c.hidden, c.ffn)
            parts = torch.empty(max(np_o, np_d), P, c.hidden, dtype=torch.float32, device=dev)
        else:
            a = torch.empty(P, c.hidden, dtype=bf, device=dev)
        qkv = None if positions is None else torch.empty(P, c.qkv_dim, dtype=bf, device=dev)
        ws_g = self.ws_gemm
        zero = torch.zeros(1, dtype=torch.int32, device=dev)
        starts = torch.arange(0, P, chunk, dtype=torch.int32, device=dev)
        lens = torch.zeros(1, dtype=torch.int32, device=dev)
        pos3 = None if positions is None else positions.to(device=dev, dtype=torch.int32).contiguous()
        plan = self.attn_plan(1)
        ws = self._attn_ws(1, min(chunk, P), plan)
        K.rmsnorm(h, self.n_in[0], x, eps)
        for l in range(c.n_layers):
            if positions is None:
                K.gemm_rope_stage(x, self.wqkv[l], zero, self.inv_freq, q, kw[0], vw[0], rot_dim=c.rot_dim,
                                  pos_delta=pos_delta, workspace=ws_g)
            else:
                K.gemm(x, self.wqkv[l], qkv, workspace=ws_g)
                K.rope_stage_mrope(qkv, pos3, self.inv_freq, q[0], kw[0, 0], vw[0, 0], sections=c.mrope_section,
                                   rot_dim=c.rot_dim)
            lens.zero_()
            K.kv_commit(kw, vw, self.k_pages[l:l + 1], self.v_pages[l:l + 1], pt, lens, self.ws_commit, n_add=P)
            for i, s0 in enumerate(range(0, P, chunk)):
                n = min(chunk, P - s0)
                K.window_attention(q[:, s0:s0 + n].contiguous(), self.k_pages[l], self.v_pages[l], pt,
                                   starts[i:i + 1], kw[0, :, s0:s0 + n].contiguous(), vw[0, :, s0:s0 + n].contiguous(),
                                   o[:, s0:s0 + n], n_causal=None, scale=self.scale, plan=plan, workspace=ws)
            nxt = self.n_in[l + 1] if l + 1 < c.n_layers else self.n_final
            if parts_path:
                K.gemm_parts(o.view(P, -1), self.wo[l], parts[:np_o])
                K.add_rmsnorm_parts(parts[:np_o], self.n_psa[l], h, self.n_pa[l], x, eps)
                K.gemm_swiglu(x, self.wgu[l], act, workspace=ws_g)
                K.gemm_parts(act, self.wdown[l], parts[:np_d])
                K.add_rmsnorm_parts(parts[:np_d], self.n_pm[l], h, nxt, x, eps)
            else:
                K.gemm(o.view(P, -1), self.wo[l], a, workspace=ws_g)
                K.add_rmsnorm(a, self.n_psa[l], h, self.n_pa[l], x, eps)
                K.gemm_swiglu(x, self.wgu[l], act, workspace=ws_g)
                K.gemm(act, self.wdown[l], a, workspace=ws_g)
                K.add_rmsnorm(a, self.n_pm[l], h, nxt, x, eps)
        self.seq_lens[slot:slot + 1].fill_(P)
        r0, r1 = logits_rows if logits_rows is not None else (P - 1, P)
        logits = torch.empty(r1 - r0, c.vocab, dtype=bf, device=dev)
        K.gemm(x[r0:r1], self.lm_head, logits, workspace=ws_g)
        return logits if logits_rows is not None else logits[0]


@dataclass
class RoundState:
    """Device state of a batch of sequences decoded with the full-draft round (K = B + 1 rows per forward)."""
    bs: int
    K: int
    x0: torch.Tensor          # int32 [bs]   boundary token (committed, its K/V not yet in the cache)
    win: torch.Tensor         # int32 [bs, K] draft window [x0 | MASK x B]
    am: torch.Tensor          # int32 [bs, K] draft argmax = verify window [a0, d_1..d_B]
    tgt: torch.Tensor         # int32 [bs, K] verify argmax
    acc: torch.Tensor         # int32 [bs]
    packed: torch.Tensor      # int32 [bs, K+2] (a0, acc, targets zeroed past acc)
    slots: torch.Tensor       # int32 [bs, K]  paged slots of the committed verify rows
    log: torch.Tensor         # int32 [max_rounds, bs, K+2] packed rows of every round
    ctr: torch.Tensor         # int64 [1] rounds logged
    graph: Optional[torch.cuda.CUDAGraph] = None


class SelfSpecDecoder:
    """The full-draft self-spec round and the AR step over a GssEngine, device resident and graph-capturable.

    The decoder owns the engine's sequence slots [slot0, slot0 + bs) (their lengths and page-table rows). Its
    attention runs under ``attn_plan`` (default: the library plan for bs sequences); a decoder given the plan of a
    larger batch computes every row exactly as that batch does, so one sequence decoded alone reproduces its rows of
    the batched decode bit for bit."""

    def __init__(self, eng: GssEngine, bd: int, mask_id: int, bs: int = 1, max_rounds: int = 4096,
                 softmax_rule: bool = False, slot0: int = 0, attn_plan=None):
        self.eng, self.bd, self.mask_id, self.bs = eng, bd, mask_id, bs
        if slot0 < 0 or slot0 + bs > eng.max_bs:
            raise ValueError(f"slots [{slot0}, {slot0 + bs}) exceed the engine's {eng.max_bs}")
        self.slot0 = slot0
        self.sl = eng.seq_lens[slot0:slot0 + bs]
        self.pt = eng.page_table[slot0:slot0 + bs]
        self.plan = eng.attn_plan(bs) if attn_plan is None else attn_plan
        # greedy rule for rows holding a NaN or +inf: the serving worker's raw argmax (NaN as the maximum), or the
        # HF path's argmax of the fp32 softmax (index 0) with the raw bonus row (src/fast_sampling.py:572-575)
        self.f_draft = K.ARGMAX_SOFTMAX if softmax_rule else 0
        self.f_verify = (K.ARGMAX_SOFTMAX | K.ARGMAX_LAST_RAW) if softmax_rule else 0
        Kw = bd + 1
        dev = eng.device
        i32 = dict(dtype=torch.int32, device=dev)
        win = torch.full((bs, Kw), mask_id, **i32)
        # at bs = 1 the boundary token lives in the draft window's first column, where the verify argmax writes it
        x0 = win[:, 0] if bs == 1 else torch.zeros(bs, **i32)
        self.st = RoundState(bs=bs, K=Kw, x0=x0, win=win,
                             am=torch.zeros(bs, Kw, **i32), tgt=torch.zeros(bs, Kw, **i32),
                             acc=torch.zeros(bs, **i32), packed=torch.zeros(bs, Kw + 2, **i32),
                             slots=torch.zeros(bs, Kw, **i32), log=torch.zeros(max_rounds, bs, Kw + 2, **i32),
                             ctr=torch.zeros(1, dtype=torch.int64, device=dev))
        self.draft_b = eng.bufs(bs, Kw)
        self.verify_b = _Bufs(eng, bs, Kw)          # separate staging from the draft's
        self.r0_b = None                            # round 0's [MASK x B] draft window, made on first use
        self.r0_ids = torch.full((bs, bd), mask_id, **i32)
        self.r0_am = torch.zeros(bs, bd, **i32)
        self.pos_delta = torch.zeros(bs, **i32)     # position - cache index of every response row (M-RoPE delta)
        self.log_am = torch.zeros(max_rounds, bs, Kw, **i32)    # every round's verify window (the draft)
        self.log_tgt = torch.zeros(max_rounds, bs, Kw, **i32)   # every round's verify argmax
        self.ar_b = eng.bufs(bs, 1)
        self.ar_tgt = torch.zeros(bs, 1, **i32)
        self.ar_ids = self.st.x0.view(bs, 1)        # the AR step's input is the boundary token itself
        self.ar_log = torch.zeros(max_rounds, bs, **i32)
        self.ar_ctr = torch.zeros(1, dtype=torch.int64, device=dev)
        self.g_round = None
        self.g_ar = None

    # ---- one round, all device-side --------------------------------------------------------------------------
    def round(self, after_draft=None):
        """One full-draft round. ``after_draft`` (optional, device ops only) runs between the x0 commit and the
        verify forward and may rewrite the verify window ``st.am[:, 1:]`` (the planted-acceptance measurement)."""
        e, s = self.eng, self.st
        if self.bs > 1:
            s.win[:, 0].copy_(s.x0)
        lg = self._fwd(self.draft_b, s.win, n_causal=1)
        e.argmax(lg, s.am, flags=self.f_draft)                              # a0, d_1..d_B
        self._commit(self.draft_b, n_add=1)                                 # x0's K/V (causal row 0): S += 1
        if after_draft is not None:
            after_draft()
        self._verify()

    def round0(self):
        """The first round of the reference's cached decode (src/fast_sampling.py:519-560 with pending = None): the
        prefill's argmax a0 (in st.x0, no K/V) seeds block[0]; the draft window is [MASK x B] at the next B
        positions, all rows bidirectional, and its rows 0..B-1 give d_1..d_B; the verify half of the round then runs
        on [a0, d_1..d_B] at positions S.. exactly as in every later round."""
        e, s = self.eng, self.st
        if self.r0_b is None:
            self.r0_b = e.bufs(self.bs, self.bd)
        lg = self._fwd(self.r0_b, self.r0_ids, n_causal=0)
        e.argmax(lg, self.r0_am, flags=self.f_draft)
        s.am[:, 0].copy_(s.x0)
        s.am[:, 1:].copy_(self.r0_am)
        self._verify()

    def _fwd(self, b, ids, n_causal, **kw):
        return self.eng.forward(b, ids=ids, n_causal=n_causal, pos_delta=self.pos_delta, seq_lens=self.sl,
                                page_table=self.pt, attn_plan=self.plan, **kw)

    def _commit(self, b, **kw):
        self.eng.commit(b, seq_lens=self.sl, page_table=self.pt, **kw)

    def _verify(self):
        e, s = self.eng, self.st
        lg = self._fwd(self.verify_b, s.am, n_causal=None)
        e.argmax(lg, s.tgt, window=s.am, accept_len=s.acc, next_x0=s.x0, packed=s.packed, flags=self.f_verify)
        self._commit(self.verify_b, n_rows=s.acc, n_add=1, slots=s.slots)   # a0, d_1..d_acc: S += acc + 1
        # the log index is clamped on the device, so rounds beyond the log's capacity rewrite its last row
        K.log_append(s.ctr, [(s.packed, s.log), (s.am, self.log_am), (s.tgt, self.log_tgt)])

    def ar_step(self):
        e = self.eng
        lg = self._fwd(self.ar_b, self.ar_ids, n_causal=None)
        # a one-row window: accept length 0, so next_x0 = the argmax itself (written over the input token)
        e.argmax(lg, self.ar_tgt, window=self.ar_ids, next_x0=self.st.x0)
        self._commit(self.ar_b, n_add=1)
        K.log_append(self.ar_ctr, [(self.ar_tgt.view(self.bs), self.ar_log)])

    def capture(self):
        """Capture one round and one AR step as HIP graphs (call after one eager warm-up of each)."""
        self.g_round = torch.cuda.CUDAGraph()
        with torch.cuda.graph(self.g_round):
            self.round()
        self.g_ar = torch.cuda.CUDAGraph()
        with torch.cuda.graph(self.g_ar):
            self.ar_step()

    def start(self, x0: torch.Tensor, pos_delta: Optional[torch.Tensor] = None):
        """Begin decoding: x0 = the token the prefill produced (committed; no K/V yet). ``pos_delta`` [bs]: the
        position of cache index i is i + pos_delta (0 when the prompt's positions are 0..P-1)."""
        self.st.x0.copy_(x0.to(torch.int32))
        if pos_delta is None:
            self.pos_delta.zero_()
        else:
            self.pos_delta.copy_(pos_delta.to(torch.int32))
        self.st.ctr.zero_()
        self.ar_ctr.zero_()

    # ---- host views -------------------------------------------------------------------------------------------
    def committed(self, n_rounds: int) -> List[List[int]]:
        """Committed ids per sequence over the first n_rounds logged rounds: [a0, t_0..t_acc] per round."""
        log = self.st.log[:n_rounds].cpu().numpy()
        out = [[] for _ in range(self.bs)]
        for r in range(n_rounds):
            for b in range(self.bs):
                a = int(log[r, b, 1])
                out[b].append(int(log[r, b, 0]))
                out[b].extend(int(x) for x in log[r, b, 2:3 + a])
        return out

    def accept_lengths(self, n_rounds: int) -> np.ndarray:
        return self.st.log[:n_rounds, :, 1].cpu().numpy()
