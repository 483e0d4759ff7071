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

Not built: grammar vocabulary masks and custom logit processors (host-side objects of the serving stack), and the
flashinfer backend's min-p path (its top-k / top-p renormalizations are flashinfer's own kernels): they raise.
"""
from dataclasses import dataclass, field
from typing import Optional, Sequence

import torch

from . import kernels as K
from .engine import SelfSpecDecoder


@dataclass
class SamplingSpec:
    """Per-sequence sampling settings (lists or scalars, broadcast over the batch). ``filter``: "joint" (flashinfer's
    top-k / top-p, the serving default), "torch" (the pytorch backend, with min_p) or "none". Penalties run in
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
    grammar: object = None
    custom_logit_processor: object = None


class SampledSelfSpec:
    """Sampled rounds (and the matching AR step) over a SelfSpecDecoder's engine, buffers and logs."""

    def __init__(self, dec: SelfSpecDecoder, spec: SamplingSpec):
        if spec.grammar is not None or spec.custom_logit_processor is not None:
            raise NotImplementedError("grammar masks and custom logit processors are not built")
        if spec.filter == "joint" and _any_positive(spec.min_p):
            raise NotImplementedError("min_p with the flashinfer backend (its renorm kernels) is not built; "
                                      "use filter='torch'")
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
    def _process(self, logits, cand):
        """AR's logits processing of rows [bs*K, V] (in place) for the prefixes cand[b, 0..r]."""
        if self.processed:
            K.penalize_rows(logits, cand, {k: v for k, v in self.state.items()}, self.order)

    def _draw(self, logits, bs, Kr, uniforms, out):
        K.sample_rows(logits, bs, Kr, temperature=self.temperature, filter=self.spec.filter, top_k=self.top_k,
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
        K.sample_rows(rows, bs, Kw, temperature=self.temperature, filter=self.spec.filter, top_k=self.top_k,
                      top_p=self.top_p, min_p=self.min_p, cand=s.am, coins=self.coins, uniforms=self.u,
                      sampled=self.sampled, target=s.tgt, accept_len=s.acc, next_x0=s.x0, packed=s.packed,
                      workspace=self.ws)
        d._commit(d.verify_b, n_rows=s.acc, n_add=1, slots=s.slots)
        valid = torch.arange(Kw, device=s.acc.device)[None, :] <= s.acc[:, None]
        self._cumulate(s.tgt, valid)
        K.log_append(s.ctr, [(s.packed, s.log), (s.am, d.log_am), (s.tgt, d.log_tgt)])

    def ar_step(self):
        """One sampled AR decode step with the same processing (the reference distribution of the round)."""
        d, e = self.dec, self.dec.eng
        lg = d._fwd(d.ar_b, d.ar_ids, n_causal=None, logits_f32=True)
        row = lg[:, 0, :]
        self._process(row, self.ar_cand)
        self.ar_u.uniform_()
        self._draw(row, d.bs, 1, self.ar_u, self.ar_tok)
        d._commit(d.ar_b, n_add=1)
        d.st.x0.copy_(self.ar_tok[:, 0])
        self._cumulate(self.ar_tok, torch.ones_like(self.ar_tok, dtype=torch.bool))
        K.log_append(d.ar_ctr, [(self.ar_tok.view(d.bs), d.ar_log)])


def _any_positive(x) -> bool:
    t = torch.as_tensor(x)
    return bool((t > 0).any())
