"""The sampled round on the tiny decoder (GPU): with top-k 1 every request decodes greedily through the sampled
path, so the committed ids must equal the sampled AR decode's ids exactly, with and without penalties (the verify
rows' in-block penalties, a0's draw and the penalty state after every round all have to agree with AR token by
token for that to hold). With temperature sampling, each round's decision equals the oracle's speculative sampling
of the same processed verify logits, coins and uniform."""
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


@pytest.mark.parametrize("filt,pen", [("joint", {}), ("torch", PEN)], ids=["joint", "torch-penalties"])
def test_sampled_round_decisions_match_oracle(cuda, filt, pen):
    from gravityocr_amd.sampling import SampledSelfSpec, SamplingSpec
    print(f"sampled decisions {filt}", flush=True)
    torch.manual_seed(3)
    eng, dec, emb = _build(cuda)
    spec = SamplingSpec(temperature=0.8, top_k=40, top_p=0.9, min_p=0.05 if filt == "torch" else 0.0, filter=filt,
                        **pen)
    ss = SampledSelfSpec(dec, spec)
    last = eng.prefill(0, emb)
    ss.start(last.float().argmax().view(1))
    K = dec.st.K
    total_acc = 0
    for r in range(12):
        ss.round(keep=True)
        torch.cuda.synchronize()
        rows, coins, u, cand = (t.cpu().numpy() for t in ss.keep)
        probs = np.stack([S.target_probs(rows[j], 0.8, 1 if filt == "joint" else 2, 40, 0.9, spec.min_p)
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
