"""The sampled round on the tiny decoder (GPU): with top-k 1 every request decodes greedily through the sampled
path, so the committed ids must equal the sampled AR decode's ids exactly, with and without penalties (the verify
rows' in-block penalties, a0's draw and the penalty state after every round all have to agree with AR token by
token for that to hold). With temperature sampling, each round's decision equals the oracle's speculative sampling
of the same processed verify logits, coins and uniform. With a grammar (masks of the rows' prefixes) or a custom
logit processor (request views of the rows' prefixes), top-1 rounds equal the sampled AR decode under the same
grammar / processor; the mask kernel equals the unpacked bits exactly."""
import numpy as np
import pytest
import torch

from oracle import sampling as S

pytestmark = pytest.mark.gpu


def _build(cuda, bd=4):
    from gravityocr_amd.engine import GssEngine, SelfSpecDecoder
    from gravityocr_amd.model import TINY, synthetic_prompt, synthetic_weights
    w = synthetic_weights(TINY, 0)
    vis, ids = synthetic_prompt(TINY, 256, 16, 0)
    emb = torch.cat([vis, w["embed"][ids]], 0)
    eng = GssEngine(TINY, w, max_bs=1, max_len=1024, device=cuda)
    dec = SelfSpecDecoder(eng, bd=bd, mask_id=TINY.vocab - 1, bs=1)
    return eng, dec, emb


PEN = dict(repetition_penalty=1.3, presence_penalty=0.4, frequency_penalty=0.3, min_new_tokens=12,
           stop_token_ids=(5, 17))


@pytest.mark.parametrize("pen", [{}, PEN], ids=["plain", "penalties"])
def test_top1_sampled_round_equals_sampled_ar(cuda, pen):
    from gravityocr_amd.sampling import SampledSelfSpec, SamplingSpec
    print(f"sampled top-1 {sorted(pen)}", flush=True)
    n = 40
    eng, dec, emb = _build(cuda)
    spec = SamplingSpec(temperature=1.0, top_k=1, filter="joint", **pen)
    ss = SampledSelfSpec(dec, spec)
    last = eng.prefill(0, emb)
    x0 = last.float().argmax().view(1)
    ss.start(x0)
    for _ in range(n):
        ss.ar_step()
    torch.cuda.synchronize()
    ar = [int(x0)] + dec.ar_log[:n, 0].cpu().tolist()

    eng, dec, emb = _build(cuda)
    ss = SampledSelfSpec(dec, spec)
    last = eng.prefill(0, emb)
    ss.start(last.float().argmax().view(1))
    rounds = 0
    while True:
        ss.round()
        rounds += 1
        torch.cuda.synchronize()
        out = [int(x0)] + dec.committed(rounds)[0]
        if len(out) > n:
            break
    assert out[:n + 1] == ar
    assert int(dec.accept_lengths(rounds).sum()) > 0


@pytest.mark.parametrize("filt,min_p,mode,pen", [("joint", 0.0, 1, {}), ("torch", 0.05, 2, PEN), ("joint", 0.05, 3, {})],
                         ids=["joint", "torch-penalties", "joint-min_p"])
def test_sampled_round_decisions_match_oracle(cuda, filt, min_p, mode, pen):
    """mode = the oracle's target distribution: the flashinfer backend with min_p > 0 in the batch is its renorm
    chain (top-k renorm, top-p renorm, min-p)."""
    from gravityocr_amd.sampling import SampledSelfSpec, SamplingSpec
    print(f"sampled decisions {filt} min_p={min_p}", flush=True)
    torch.manual_seed(3)
    eng, dec, emb = _build(cuda)
    spec = SamplingSpec(temperature=0.8, top_k=40, top_p=0.9, min_p=min_p, filter=filt, **pen)
    ss = SampledSelfSpec(dec, spec)
    last = eng.prefill(0, emb)
    ss.start(last.float().argmax().view(1))
    K = dec.st.K
    total_acc = 0
    for r in range(12):
        ss.round(keep=True)
        torch.cuda.synchronize()
        rows, coins, u, cand = (t.cpu().numpy() for t in ss.keep)
        probs = np.stack([S.target_probs(rows[j], 0.8, mode, 40, 0.9, spec.min_p)
                          for j in range(K)])
        a_want, tok_want, t_want = S.spec_sample_chain(probs, cand[0], coins[0].astype(np.float64), float(u[0]))
        a = int(dec.st.acc[0])
        packed = dec.st.packed[0].cpu().tolist()
        if a != a_want:
            j = min(a, a_want)
            assert abs(coins[0, j] - probs[j, cand[0, j + 1]]) < 1e-5
            continue
        total_acc += a
        assert packed[1] == a and packed[2:2 + a] == [int(t) for t in cand[0, 1:a + 1]]
        q = probs[a].copy()
        if a < K - 1:
            q[cand[0, a + 1]] = 0.0
        tok = packed[2 + a]
        if tok != tok_want:
            c = np.cumsum(q) / q.sum()
            assert abs(c[min(tok, tok_want)] - float(u[0])) < 1e-5
    assert total_acc >= 0


@pytest.mark.parametrize("V", [4095, 4096, 59392])
def test_vocab_mask_kernel(cuda, V):
    """gss_apply_vocab_mask: -inf exactly where the token's bit is clear, every other logit untouched."""
    from gravityocr_amd import kernels as K
    g = torch.Generator().manual_seed(V)
    rows = 17
    logits = torch.randn(rows, V, generator=g)
    words = torch.randint(-2 ** 31, 2 ** 31 - 1, (rows, (V + 31) // 32), generator=g, dtype=torch.int64).to(torch.int32)
    words[3] = -1                                              # an all-allowed row
    bits = ((words.to(torch.int64).unsqueeze(-1) >> torch.arange(32)) & 1).reshape(rows, -1)[:, :V].bool()
    want = torch.where(bits, logits, torch.full_like(logits, float("-inf")))
    got = logits.to(cuda)
    K.apply_vocab_mask(got, words.to(cuda))
    torch.cuda.synchronize()
    assert torch.equal(got.cpu(), want)


def _grammar_decode(cuda, n, spec_kw, use_round, make_grammar=None, processor=None):
    """n tokens of the tiny model's sampled decode with top-1 (greedy through the sampled path) under a grammar
    and / or a custom processor: AR steps or rounds. A request object's output_ids follow the committed tokens."""
    from gravityocr_amd.sampling import SampledSelfSpec, SamplingSpec
    eng, dec, emb = _build(cuda)
    req = type("Req", (), {})()
    gram = make_grammar() if make_grammar else None
    spec = SamplingSpec(temperature=1.0, top_k=1, filter="joint", grammar=None if gram is None else [gram],
                        custom_logit_processor=processor,
                        custom_params=None if processor is None else [{"__req__": req, "bump": 2.5}], **spec_kw)
    ss = SampledSelfSpec(dec, spec)
    last = eng.prefill(0, emb).float()
    if gram is not None:   # the first output token is drawn under the grammar too
        allowed = torch.tensor([gram.allowed(t) for t in range(last.numel())], device=last.device)
        last = torch.where(allowed, last, torch.full_like(last, float("-inf")))
    x0 = last.argmax().view(1)
    if gram is not None:
        gram.accept_token(int(x0))
    req.output_ids = [int(x0)]
    ss.start(x0)
    if not use_round:
        for i in range(n):
            ss.ar_step()
            req.output_ids.append(int(dec.ar_log[i, 0]))
        return [int(x0)] + dec.ar_log[:n, 0].cpu().tolist(), gram
    rounds = 0
    out = [int(x0)]
    while len(out) <= n:
        ss.round()
        rounds += 1
        new = dec.committed(rounds)[0][len(out) - 1:]
        out += new
        req.output_ids += new
    return out, gram


def _bump_processor(logits, params):
    """adds params' bump to the token (7 * len(output_ids)) % V of each row: depends on the row's prefix"""
    V = logits.shape[1]
    out = logits.clone()
    for r, prm in enumerate(params):
        out[r, (7 * len(prm["__req__"].output_ids)) % V] += prm["bump"]
    return out


@pytest.mark.parametrize("pen", [{}, PEN], ids=["plain", "penalties"])
def test_top1_sampled_round_with_grammar_equals_sampled_ar(cuda, pen):
    """Grammar masks (a position-dependent grammar): the rounds commit exactly the sampled AR decode's ids under
    the same grammar, every committed token is allowed by the grammar at its position, and the grammar ends in the
    committed state."""
    from tests.helpers import PositionGrammar
    from gravityocr_amd.model import TINY
    n = 40
    make = lambda: PositionGrammar(TINY.vocab)
    ar, g_ar = _grammar_decode(cuda, n, pen, False, make)
    rd, g_rd = _grammar_decode(cuda, n, pen, True, make)
    assert rd[:n + 1] == ar
    walk = PositionGrammar(TINY.vocab)
    for t in ar:
        walk.accept_token(t)                                  # raises if the decode broke the grammar
    assert g_ar.acc == ar[:len(g_ar.acc)] and g_rd.acc[:n + 1] == ar


def test_top1_sampled_round_with_custom_processor_equals_sampled_ar(cuda):
    """A custom logit processor that depends on each row's request view (its output_ids): the rounds' rows see the
    committed ids plus the row's own prefix [a0, d_1..d_j], so they commit exactly the sampled AR decode's ids."""
    n = 40
    ar, _ = _grammar_decode(cuda, n, {}, False, processor=_bump_processor)
    rd, _ = _grammar_decode(cuda, n, {}, True, processor=_bump_processor)
    plain, _ = _grammar_decode(cuda, n, {}, False)
    assert rd[:n + 1] == ar and ar != plain
