"""The sampled self-speculative round (requests that do not decode greedily) on the GssEngine: the serving
worker's non-plain round (selfspec_diffusion_worker.py:742-746, selfspec_fast_commit.py:150-230, 232-245).

Per round: draft forward (fp32 logits); the draft tokens d_1..d_{K-1} are the argmax of the mask rows (a
deterministic draft); a0 is drawn from the draft's causal row with the request's logits processing (penalties of
the committed tokens, logit_bias) and AR's sampler (temperature, top-k / top-p / min-p), then fed to the penalty
state; verify forward on [a0, d_1..d_{K-1}]; every verify row gets AR's penalties for its prefix
(gss_penalize_rows) and speculative sampling decides the chain against AR's target distribution
(gss_sample_rows); the accepted rows' K/V are committed and the committed tokens fed to the penalty state.
Coins are in (0, 1] (a zero-probability draft token is never accepted), uniforms in [0, 1), both from torch's
device generator, so a round can be captured into a HIP graph.

Grammar vocabulary masks and custom logit processors are host-side objects of the serving stack: a round that uses
them (``SamplingSpec.grammar`` / ``custom_logit_processor``) reads a0 and the draft back after the draft forward,
walks each grammar along [a0, d_1..] to build the verify rows' packed masks (fulldraft_bitmask,
selfspec_sampling.py:305-337), and processes the rows in the serving order (selfspec_fast_commit.py:170-194):
penalties, the grammar mask (gss_apply_vocab_mask), logit_bias, then the custom processor once per row position
with a read-only request view whose output_ids hold that row's prefix (apply_custom_rows, selfspec_sampling.py:
200-221). Such rounds synchronize with the host twice and are not captured. The flashinfer backend in a batch that
needs min_p (any min_p > 0) takes the reference's other branch for every row of the batch (selfspec_sampling.py:
278-281): top-k renorm, top-p renorm, min-p (gss_sample_rows filter 3).
"""
from dataclasses import dataclass, field
from typing import Optional, Sequence

import torch

from . import kernels as K
from .engine import SelfSpecDecoder


@dataclass
class SamplingSpec:
    """Per-sequence sampling settings (lists or scalars, broadcast over the batch). ``filter``: "joint" (the flashinfer
    backend, the serving default: joint top-k / top-p, or its renorm chain with min-p when any min_p > 0), "torch"
    (the pytorch backend, with min_p) or "none". Penalties run in
    ``order`` (the penalizer orchestrator's order); a penalizer whose parameter is absent is not applied."""
    temperature: object = 1.0
    top_k: object = 0
    top_p: object = 1.0
    min_p: object = 0.0
    filter: str = "joint"
    repetition_penalty: Optional[object] = None
    presence_penalty: Optional[object] = None
    frequency_penalty: Optional[object] = None
    min_new_tokens: Optional[object] = None
    stop_token_ids: Sequence[int] = ()
    logit_bias: Optional[torch.Tensor] = None     # [bs, V] fp32
    order: Sequence[str] = ("frequency", "min_new_tokens", "presence", "repetition")
    grammar: object = None                 # per-sequence grammar objects (None entries: no grammar) or None
    custom_logit_processor: object = None  # callable(logits_rows [n, V] fp32, params list) -> logits rows
    custom_params: Optional[Sequence] = None  # per-sequence params (a dict's "__req__" gets the row's request view)


class RequestView:
    """Read-only stand-in for a request inside a custom logit processor applied to verify row j: output_ids = the
    request's committed output ids + the tokens row j's prefix adds; every other attribute is the request's own."""

    __slots__ = ("_req", "output_ids")

    def __init__(self, req, extra):
        object.__setattr__(self, "_req", req)
        object.__setattr__(self, "output_ids", list(getattr(req, "output_ids", [])) + [int(t) for t in extra])

    def __getattr__(self, name):
        return getattr(object.__getattribute__(self, "_req"), name)

    def __setattr__(self, name, value):
        raise AttributeError("RequestView is read-only")


def _allowed(mask_row, tok: int) -> bool:
    return bool((int(mask_row[tok >> 5]) >> (tok & 31)) & 1)


def grammar_masks(grammars, cand, V: int, first_accepted: bool = True):
    """Packed int32 vocabulary masks [bs * K, ceil(V / 32)] (host) of windows cand [bs, K] (host ints): row j of
    sequence b allows what b's grammar allows after cand[b, 0..j] (with ``first_accepted`` False, after
    cand[b, 1..j]: row 0 is the grammar's current state). Each grammar accepts the window's tokens while the previous
    row allows them, fills its rows, and is rolled back to the state it came in; rows of a sequence without a
    grammar, of a terminated grammar, and past a token its previous row forbids stay all-allowed. Grammar objects
    follow the serving stack's surface: allocate_vocab_mask, fill_vocab_mask, accept_token, rollback,
    is_terminated (selfspec_sampling.py:305-337)."""
    bs, K = len(cand), len(cand[0])
    first = next(g for g in grammars if g is not None)
    mask = first.allocate_vocab_mask(vocab_size=V, batch_size=bs * K, device="cpu")
    mask.fill_(-1)
    for b, g in enumerate(grammars):
        if g is None or g.is_terminated():
            continue
        n_acc = 0
        try:
            if first_accepted:
                try:
                    g.accept_token(int(cand[b][0]))
                    n_acc += 1
                except ValueError:
                    continue
            for j in range(K):
                g.fill_vocab_mask(mask, b * K + j)
                if j + 1 >= K or g.is_terminated():
                    break
                nxt = int(cand[b][j + 1])
                if not _allowed(mask[b * K + j], nxt):
                    break
                g.accept_token(nxt)
                n_acc += 1
        finally:
            if n_acc:
                g.rollback(n_acc)
    return mask


class SampledSelfSpec:
    """Sampled rounds (and the matching AR step) over a SelfSpecDecoder's engine, buffers and logs."""

    def __init__(self, dec: SelfSpecDecoder, spec: SamplingSpec):
        self.grammars = None
        if spec.grammar is not None:
            gl = list(spec.grammar)
            if len(gl) != dec.bs:
                raise ValueError("one grammar entry per sequence")
            self.grammars = gl if any(g is not None for g in gl) else None
        self.custom = spec.custom_logit_processor
        if self.custom is not None and (spec.custom_params is None or len(spec.custom_params) != dec.bs):
            raise ValueError("custom_logit_processor needs one custom_params entry per sequence")
        self.hosted = self.grammars is not None or self.custom is not None
        if spec.filter not in ("joint", "torch", "none"):
            raise ValueError(f"filter {spec.filter!r}: 'joint' (flashinfer), 'torch' or 'none'")
        # the batch-level need_min_p_sampling flag selects the flashinfer backend's renorm chain for every row
        self.kfilter = "flashinfer_min_p" if spec.filter == "joint" and _any_positive(spec.min_p) else spec.filter
        self.dec, self.spec = dec, spec
        e, bs, Kw, V = dec.eng, dec.bs, dec.st.K, dec.eng.cfg.vocab
        dev = e.device
        f32 = dict(dtype=torch.float32, device=dev)
        i32 = dict(dtype=torch.int32, device=dev)
        vec = lambda x, kw: torch.as_tensor(x, **kw).expand(bs).contiguous() if torch.as_tensor(x).dim() == 0 \
            else torch.as_tensor(x, **kw).contiguous()
        self.temperature = vec(spec.temperature, f32)
        self.top_k = vec(spec.top_k, i32)
        self.top_p = vec(spec.top_p, f32)
        self.min_p = vec(spec.min_p, f32)
        # penalty state of the committed tokens (SGLang's penalizers' cumulated tensors)
        self.order = []
        self.state = {}
        if spec.repetition_penalty is not None:
            self.order_add("repetition")
            self.state.update(rep_cum=torch.ones(bs, V, **f32), rep_pen=vec(spec.repetition_penalty, f32))
        if spec.presence_penalty is not None:
            self.order_add("presence")
            self.state.update(pres_cum=torch.zeros(bs, V, **f32), pres_pen=vec(spec.presence_penalty, f32))
        if spec.frequency_penalty is not None:
            self.order_add("frequency")
            self.state.update(freq_cum=torch.zeros(bs, V, **f32), freq_pen=vec(spec.frequency_penalty, f32))
        if spec.min_new_tokens is not None:
            self.order_add("min_new_tokens")
            stop = torch.zeros(bs, V, **f32)
            if len(spec.stop_token_ids):
                stop[:, torch.as_tensor(list(spec.stop_token_ids), device=dev)] = float("-inf")
            self.state.update(min_new=vec(spec.min_new_tokens, i32), stop_pen=stop)
        self.state["len_out"] = torch.zeros(bs, **i32)
        if spec.logit_bias is not None:
            self.state["logit_bias"] = spec.logit_bias.to(**f32).contiguous()
        self.order = [n for n in spec.order if n in self.order]
        self.processed = bool(self.order) or spec.logit_bias is not None
        self.a0_cand = torch.zeros(bs, 1, **i32)
        self.a0_tok = torch.zeros(bs, 1, **i32)
        self.u_a0 = torch.zeros(bs, 1, **f32)
        self.coins = torch.ones(bs, Kw, **f32)
        self.u = torch.zeros(bs, **f32)
        self.sampled = torch.zeros(bs, Kw, **i32)
        self.ws = torch.zeros(K.sample_workspace_bytes(bs, Kw), dtype=torch.uint8, device=dev)
        self.ar_tok = torch.zeros(bs, 1, **i32)
        self.ar_u = torch.zeros(bs, 1, **f32)
        self.ar_cand = torch.zeros(bs, 1, **i32)
        self.keep = None   # (verify logits after processing, coins, uniform) of the last round, when asked for

    def order_add(self, name):
        self.order.append(name)

    def start(self, x0: torch.Tensor, pos_delta: Optional[torch.Tensor] = None):
        """Begin decoding after the prefill's token x0 (the first output token: it enters the penalty state)."""
        self.dec.start(x0, pos_delta)
        self._cumulate(x0.to(self.dec.st.x0.device).view(-1, 1).to(torch.int64),
                       torch.ones(self.dec.bs, 1, dtype=torch.bool, device=self.dec.st.x0.device))

    # ---- pieces ----------------------------------------------------------------------------------------------
    def _process(self, logits, cand, mask=None, cand_host=None, extra_from: int = 0):
        """AR's logits processing of rows [bs*K, V] (in place) for the prefixes cand[b, 0..r]: penalties, then (a
        hosted round) the grammar mask, logit_bias and the custom processor with the rows' request views (prefix
        tokens cand_host[b][extra_from..r])."""
        if not self.hosted:
            if self.processed:
                K.penalize_rows(logits, cand, {k: v for k, v in self.state.items()}, self.order)
            return
        bias = self.state.get("logit_bias")
        if self.order:
            st = {k: v for k, v in self.state.items() if k != "logit_bias"}
            K.penalize_rows(logits, cand, st, self.order)
        if mask is not None:
            K.apply_vocab_mask(logits, mask)
        Kr = cand.shape[1]
        if bias is not None:
            logits.add_(torch.repeat_interleave(bias, Kr, dim=0))
        if self.custom is not None:
            users = list(range(self.dec.bs))
            for j in range(Kr):
                params = []
                for b in users:
                    prm = self.spec.custom_params[b]
                    if isinstance(prm, dict) and "__req__" in prm:
                        prm = dict(prm)
                        prm["__req__"] = RequestView(prm["__req__"], cand_host[b][extra_from:j + 1])
                    params.append(prm)
                rows = torch.tensor([b * Kr + j for b in users], device=logits.device, dtype=torch.int64)
                logits[rows] = self.custom(logits[rows], params)

    def _draw(self, logits, bs, Kr, uniforms, out):
        K.sample_rows(logits, bs, Kr, temperature=self.temperature, filter=self.kfilter, top_k=self.top_k,
                      top_p=self.top_p, min_p=self.min_p, uniforms=uniforms, sampled=out)

    def _cumulate(self, tok, valid):
        """The penalizers' state after committing tok[b, i] where valid[b, i] (any order gives the same state: the
        set-type penalties write one value per request, frequency adds one equal amount per token)."""
        st = self.state
        tok = tok.to(torch.int64)
        # a token outside the vocabulary (a draw from a row without probability mass: NaN logits) is not fed
        valid = valid & (tok >= 0) & (tok < self.dec.eng.cfg.vocab)
        any_ = valid.any(1, keepdim=True)
        first = tok.gather(1, valid.to(torch.int64).argmax(1, keepdim=True))
        idx = torch.where(valid, tok, torch.where(any_, first, torch.zeros_like(first)))
        if "rep_cum" in st:
            cur = st["rep_cum"].gather(1, idx)
            st["rep_cum"].scatter_(1, idx, torch.where(any_, st["rep_pen"][:, None].expand_as(cur), cur))
        if "pres_cum" in st:
            cur = st["pres_cum"].gather(1, idx)
            st["pres_cum"].scatter_(1, idx, torch.where(any_, st["pres_pen"][:, None].expand_as(cur), cur))
        if "freq_cum" in st:
            st["freq_cum"].scatter_add_(1, idx, st["freq_pen"][:, None].expand(idx.shape) * valid)
        st["len_out"] += valid.sum(1).to(torch.int32)

    # ---- the round -------------------------------------------------------------------------------------------
    def round(self, keep: bool = False):
        if self.hosted:
            return self._round_hosted(keep)
        d, e, s = self.dec, self.dec.eng, self.dec.st
        bs, Kw = d.bs, s.K
        V = e.cfg.vocab
        if bs > 1:
            s.win[:, 0].copy_(s.x0)
        lg = d._fwd(d.draft_b, s.win, n_causal=1, logits_f32=True)
        e.argmax(lg, s.am)                                       # the deterministic draft d_1..d_{K-1}
        row0 = lg[:, 0, :]
        self._process(row0, self.a0_cand)
        self.u_a0.uniform_()
        self._draw(row0, bs, 1, self.u_a0, self.a0_tok)          # a0 ~ AR's distribution of the token after x0
        s.am[:, 0].copy_(self.a0_tok[:, 0])
        self._cumulate(self.a0_tok, torch.ones_like(self.a0_tok, dtype=torch.bool))
        d._commit(d.draft_b, n_add=1)
        lg = d._fwd(d.verify_b, s.am, n_causal=None, logits_f32=True)
        rows = lg.view(bs * Kw, V)
        self._process(rows, s.am)
        self.coins.uniform_().neg_().add_(1.0)                   # (0, 1]
        self.u.uniform_()
        if keep:
            self.keep = (rows.clone(), self.coins.clone(), self.u.clone(), s.am.clone())
        K.sample_rows(rows, bs, Kw, temperature=self.temperature, filter=self.kfilter, top_k=self.top_k,
                      top_p=self.top_p, min_p=self.min_p, cand=s.am, coins=self.coins, uniforms=self.u,
                      sampled=self.sampled, target=s.tgt, accept_len=s.acc, next_x0=s.x0, packed=s.packed,
                      workspace=self.ws)
        d._commit(d.verify_b, n_rows=s.acc, n_add=1, slots=s.slots)
        valid = torch.arange(Kw, device=s.acc.device)[None, :] <= s.acc[:, None]
        self._cumulate(s.tgt, valid)
        K.log_append(s.ctr, [(s.packed, s.log), (s.am, d.log_am), (s.tgt, d.log_tgt)])

    def _round_hosted(self, keep: bool):
        """The round with grammar masks and / or custom processors: a0's row is processed against the current
        grammar states, the verify rows against the states after [a0, d_1..d_j]; the committed tokens then advance
        the grammars."""
        d, e, s = self.dec, self.dec.eng, self.dec.st
        bs, Kw = d.bs, s.K
        V = e.cfg.vocab
        dev = s.am.device
        if bs > 1:
            s.win[:, 0].copy_(s.x0)
        lg = d._fwd(d.draft_b, s.win, n_causal=1, logits_f32=True)
        e.argmax(lg, s.am)
        row0 = lg[:, 0, :]
        m0 = None
        if self.grammars is not None:
            cur = [[0] for _ in range(bs)]
            m0 = grammar_masks(self.grammars, cur, V, first_accepted=False).to(dev)
        self._process(row0, self.a0_cand, m0, [[] for _ in range(bs)], 0)
        self.u_a0.uniform_()
        self._draw(row0, bs, 1, self.u_a0, self.a0_tok)
        s.am[:, 0].copy_(self.a0_tok[:, 0])
        self._cumulate(self.a0_tok, torch.ones_like(self.a0_tok, dtype=torch.bool))
        d._commit(d.draft_b, n_add=1)
        cand = s.am.cpu().tolist()                                 # a0, d_1..d_{K-1} (host)
        mv = None if self.grammars is None else grammar_masks(self.grammars, cand, V).to(dev)
        lg = d._fwd(d.verify_b, s.am, n_causal=None, logits_f32=True)
        rows = lg.view(bs * Kw, V)
        self._process(rows, s.am, mv, cand, 0)
        self.coins.uniform_().neg_().add_(1.0)
        self.u.uniform_()
        if keep:
            self.keep = (rows.clone(), self.coins.clone(), self.u.clone(), s.am.clone())
        K.sample_rows(rows, bs, Kw, temperature=self.temperature, filter=self.kfilter, top_k=self.top_k,
                      top_p=self.top_p, min_p=self.min_p, cand=s.am, coins=self.coins, uniforms=self.u,
                      sampled=self.sampled, target=s.tgt, accept_len=s.acc, next_x0=s.x0, packed=s.packed,
                      workspace=self.ws)
        d._commit(d.verify_b, n_rows=s.acc, n_add=1, slots=s.slots)
        valid = torch.arange(Kw, device=s.acc.device)[None, :] <= s.acc[:, None]
        self._cumulate(s.tgt, valid)
        K.log_append(s.ctr, [(s.packed, s.log), (s.am, d.log_am), (s.tgt, d.log_tgt)])
        if self.grammars is not None:                           # the committed tokens: a0, t_0..t_acc
            packed = s.packed.cpu().tolist()
            for b, g in enumerate(self.grammars):
                if g is None:
                    continue
                row = packed[b]
                for t in [row[0]] + row[2:3 + row[1]]:
                    if g.is_terminated():
                        break
                    g.accept_token(int(t))

    def ar_step(self):
        """One sampled AR decode step with the same processing (the reference distribution of the round)."""
        d, e = self.dec, self.dec.eng
        lg = d._fwd(d.ar_b, d.ar_ids, n_causal=None, logits_f32=True)
        row = lg[:, 0, :]
        m = None
        if self.grammars is not None:
            m = grammar_masks(self.grammars, [[0] for _ in range(d.bs)], e.cfg.vocab, first_accepted=False)
            m = m.to(row.device)
        self._process(row, self.ar_cand, m, [[] for _ in range(d.bs)], 0)
        self.ar_u.uniform_()
        self._draw(row, d.bs, 1, self.ar_u, self.ar_tok)
        d._commit(d.ar_b, n_add=1)
        d.st.x0.copy_(self.ar_tok[:, 0])
        self._cumulate(self.ar_tok, torch.ones_like(self.ar_tok, dtype=torch.bool))
        K.log_append(d.ar_ctr, [(self.ar_tok.view(d.bs), d.ar_log)])
        if self.grammars is not None:
            for b, (g, t) in enumerate(zip(self.grammars, self.ar_tok[:, 0].cpu().tolist())):
                if g is not None and not g.is_terminated():
                    g.accept_token(int(t))


def _any_positive(x) -> bool:
    t = torch.as_tensor(x)
    return bool((t > 0).any())
