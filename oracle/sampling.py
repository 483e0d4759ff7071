"""Sampled (non-greedy) verify of the serving round: per-row penalties, AR's target distribution and speculative
sampling of the deterministic draft chain, restated in numpy (float64 unless noted).

Test infrastructure only (see ``oracle/__init__.py``). Reference:
patches/sglang/python/sglang/srt/speculative/selfspec_sampling.py (S below) and selfspec_fast_commit.py (F below).

Row layout: logits [bs * K, V], row b * K + r = the verify row r of sequence b, which predicts the token after
cand[b, r] (cand = the verify ids [a0, d_1 .. d_{K-1}]); row r's draft token is cand[b, r + 1].
"""
from typing import Dict, Optional, Sequence

import numpy as np

REPETITION, PRESENCE, FREQUENCY, MIN_NEW_TOKENS = "repetition", "presence", "frequency", "min_new_tokens"


def apply_scaling(logits: np.ndarray, S: np.ndarray) -> np.ndarray:
    """SGLang's apply_scaling_penalties: positive logits divided by the penalty, the others multiplied."""
    return np.where(logits > 0, logits / S, logits * S)


def penalize_rows(logits: np.ndarray, cand: np.ndarray, state: Dict, order: Sequence[str]) -> np.ndarray:
    """S:139-198. Row r of sequence b gets the penalties AR decode applies after cand[b, 1..r]: the cumulated
    state of every committed token plus the in-block tokens cand[b, 1..r], each penalizer in ``order`` with its own
    op (repetition: apply_scaling with the penalty set to rep_pen[b] at those tokens; presence: subtract, set;
    frequency: subtract, one freq_pen[b] added per occurrence; min_new_tokens: stop penalties while the row's output
    length len_out[b] + r < min_new[b]). Then logit_bias (F:190-191). float32 like the reference's tensors."""
    out = logits.astype(np.float32).copy()
    bs, K = cand.shape
    for b in range(bs):
        for r in range(K):
            row = out[b * K + r]
            inblk = [int(t) for t in cand[b, 1:r + 1]]
            for name in order:
                if name == REPETITION:
                    S = state["rep_cum"][b].astype(np.float32).copy()
                    for t in inblk:
                        S[t] = np.float32(state["rep_pen"][b])
                    row[:] = apply_scaling(row, S)
                elif name == PRESENCE:
                    S = state["pres_cum"][b].astype(np.float32).copy()
                    for t in inblk:
                        S[t] = np.float32(state["pres_pen"][b])
                    row -= S
                elif name == FREQUENCY:
                    S = state["freq_cum"][b].astype(np.float32).copy()
                    for t in inblk:
                        S[t] = np.float32(S[t] + np.float32(state["freq_pen"][b]))
                    row -= S
                elif name == MIN_NEW_TOKENS:
                    if state["len_out"][b] + r < state["min_new"][b]:
                        row += state["stop_pen"][b].astype(np.float32)
                else:
                    raise ValueError(name)
            if state.get("logit_bias") is not None:
                row += state["logit_bias"][b].astype(np.float32)
    return out


def cumulate(state: Dict, b: int, tok: int) -> None:
    """One committed token fed to the penalizers (SGLang's cumulate_output_tokens, as S:86-125 restates it): the
    repetition and presence state at the token becomes the request's penalty, frequency adds it, the output length
    grows by one. In place."""
    state["rep_cum"][b, tok] = state["rep_pen"][b]
    state["pres_cum"][b, tok] = state["pres_pen"][b]
    state["freq_cum"][b, tok] = np.float32(state["freq_cum"][b, tok] + np.float32(state["freq_pen"][b]))
    state["len_out"][b] += 1


def softmax_t(logits: np.ndarray, temperature: float) -> np.ndarray:
    """S:273: softmax(logits / T) (float64 here)."""
    x = logits.astype(np.float64) / float(temperature)
    x = x - x.max()
    e = np.exp(x)
    return e / e.sum()


def joint_top_k_top_p(p: np.ndarray, k: int, top_p: float) -> np.ndarray:
    """S:230-244 (flashinfer's joint filter): token q kept iff #{v: p_v > p_q} < k and sum{p_v: p_v > p_q} < top_p
    (top_p >= 1 keeps every token by the second test); renormalized. Ties are kept or dropped together."""
    order = np.argsort(-p, kind="stable")
    s = p[order]
    V = p.shape[0]
    pos = np.arange(V)
    new_group = np.ones(V, dtype=bool)
    new_group[1:] = s[1:] < s[:-1]
    start = np.maximum.accumulate(np.where(new_group, pos, 0))      # count of strictly greater values
    excl = np.cumsum(s) - s
    gt_sum = excl[start]
    keep_s = (start < k) & ((gt_sum < top_p) | (top_p >= 1.0))
    keep = np.zeros(V, dtype=bool)
    keep[order] = keep_s
    q = np.where(keep, p, 0.0)
    return q / q.sum()


def torch_backend_filter(p: np.ndarray, k: int, top_p: float, min_p: float, need_min_p: bool) -> np.ndarray:
    """S:253-263 (SGLang's pytorch backend): in descending order, keep rank < k, mass before the token <= top_p, and
    (with min_p) p >= max(p) * min_p; renormalized. Equal values are ranked by index (lowest first)."""
    order = np.argsort(-p, kind="stable")
    s = p[order]
    V = p.shape[0]
    csum = np.cumsum(s)
    keep_s = np.arange(V) < k
    keep_s &= ~((csum - s) > top_p)
    if need_min_p:
        keep_s &= ~(s < s[0] * min_p)
    keep = np.zeros(V, dtype=bool)
    keep[order] = keep_s
    q = np.where(keep, p, 0.0)
    return q / q.sum()


def flashinfer_min_p_chain(p: np.ndarray, k: int, top_p: float, min_p: float) -> np.ndarray:
    """S:278-281 (the flashinfer backend when the batch needs min_p): top_k_renorm_probs, then top_p_renorm_probs on
    the renormalized result, then S:247-251's min-p cut (p >= min_p * max(p)), renormalizing after each step.

    top_k_renorm_probs and top_p_renorm_probs are flashinfer's (flashinfer-python, not vendored; the reference's
    sglang patch binds them through sglang.srt.layers.sampler). Their published behaviour, restated here: top-k keeps
    the tokens with fewer than k strictly greater probabilities, top-p keeps those whose strictly greater mass is below
    top_p (top_p >= 1 keeps every token). How flashinfer's pivot search treats tied probabilities at the cut, and its
    float32 rounding of the renormalized mass, are not restated: parity unpinned for ties and for rows whose mass sits
    within float32 rounding of top_p."""
    q = joint_top_k_top_p(p, k, 1.0)
    q = joint_top_k_top_p(q, q.shape[0] + 1, top_p)
    keep = q >= q.max() * min_p
    q = np.where(keep, q, 0.0)
    return q / q.sum()


def target_probs(logits_row: np.ndarray, temperature: float, mode: int, k: int, top_p: float,
                 min_p: float = 0.0) -> np.ndarray:
    """S:266-286 for one row: mode 0 = no filter (softmax only), 1 = flashinfer joint top-k/top-p (a batch without
    min_p), 2 = the pytorch backend (min_p applied when > 0), 3 = the flashinfer backend in a batch that needs min_p
    (top-k renorm, top-p renorm, min-p; a row whose own min_p is 0 still takes the two renorm steps)."""
    p = softmax_t(logits_row, temperature)
    if mode == 0:
        return p
    if mode == 1:
        return joint_top_k_top_p(p, k, top_p)
    if mode == 3:
        return flashinfer_min_p_chain(p, k, top_p, min_p)
    return torch_backend_filter(p, k, top_p, min_p, min_p > 0.0)


def inverse_cdf(q: np.ndarray, u: float) -> int:
    """The sampler's draw from weights q (need not sum to 1) with a uniform u in [0, 1): the smallest index whose
    inclusive prefix sum exceeds u * sum(q) (the last nonzero weight if rounding leaves none)."""
    c = np.cumsum(q.astype(np.float64))
    if c[-1] <= 0.0:
        return -1   # no mass (a residual whose only token was the draft's; that row is never chosen)
    hit = np.nonzero(c > u * c[-1])[0]
    if hit.size:
        return int(hit[0])
    return int(np.nonzero(q)[0][-1])


def spec_sample_chain(probs: np.ndarray, cand: np.ndarray, coins: np.ndarray, u_final: float):
    """F:197-230 (sgl-kernel tree_speculative_sampling_target_only on the linear chain, point-mass draft, thresholds
    1.0): row j accepts its draft token cand[j + 1] iff coins[j] <= probs[j, cand[j + 1]]; at the first rejection
    (row acc) the token is drawn from probs[acc] with the rejected token removed (relu(target - draft) with the
    draft mass set to the target's at that token), and when every draft token is accepted the bonus is drawn from
    the last row. Returns (acc, sampled token, targets t_0..t_acc)."""
    K = probs.shape[0]
    acc = 0
    while acc < K - 1 and coins[acc] <= probs[acc, int(cand[acc + 1])]:
        acc += 1
    q = probs[acc].copy()
    if acc < K - 1:
        q[int(cand[acc + 1])] = 0.0
    tok = inverse_cdf(q, u_final)
    targets = [int(cand[r + 1]) for r in range(acc)] + [tok]
    return acc, tok, targets


def residual_samples(probs: np.ndarray, cand: Optional[np.ndarray], u: float) -> np.ndarray:
    """Every row's candidate draw as the kernel computes it before the chain decision: row j < K-1 draws from
    probs[j] without cand[j + 1], the last row from probs[K-1] (cand None: every row from its full distribution)."""
    K = probs.shape[0]
    out = np.zeros(K, dtype=np.int64)
    for j in range(K):
        q = probs[j].copy()
        if cand is not None and j < K - 1:
            q[int(cand[j + 1])] = 0.0
        out[j] = inverse_cdf(q, u)
    return out
