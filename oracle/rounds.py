"""The self-speculative decode rounds and the AR baseline, restated on the CPU over ``OracleDecoder``.

Test infrastructure only (see ``oracle/__init__.py``). Greedy decoding, batch size 1 per call (batched rows never
interact: src/fast_sampling_batched.py:18-25), positions equal to KV indices (a text-only / synthetic prefix, so
the M-RoPE start position ``next_pos`` equals the prefix length P; src/fast_sampling.py:490-493).
"""
from typing import Dict, List, Optional, Tuple

import numpy as np
import torch

from .attention import window_mask
from .decoder import KVCache, OracleDecoder
from .integer import accept_chain


def greedy(logits: torch.Tensor) -> torch.Tensor:
    """``_sample_top_p`` at temperature 0: fp32 softmax, then argmax (src/models/glm_ocr_dllm.py:997-1002)."""
    return torch.softmax(logits.float(), dim=-1).argmax(-1)


def causal_mask(L_pre: int, T: int) -> np.ndarray:
    return window_mask(L_pre, T, T)


def prefill(model: OracleDecoder, prefix_emb: torch.Tensor) -> Tuple[KVCache, torch.Tensor]:
    """Causal prefill of the prompt (src/fast_sampling.py:499-502). Returns (cache, logits of the last row)."""
    P = prefix_emb.shape[0]
    cache = KVCache(model.cfg.n_layers)
    h = model.forward(prefix_emb, torch.arange(P), cache, causal_mask(0, P))
    return cache, model.logits(h[-1:])


def natcache_generate(model: OracleDecoder, prefix_emb: torch.Tensor, bd: int, mask_id: int, max_new_tokens: int,
                      eos_id: Optional[int] = None, full_draft: bool = True, trace: Optional[list] = None):
    """``generate_speculative_natcache`` (src/fast_sampling.py:425-628) with its defaults draft_steps=1,
    accept_conf=0, temperature=0. Returns (generated ids cut at EOS, stats dict).

    Round structure (pending = last committed token, not yet in the cache; round 0 has none):
      draft  : window [pending | MASK x bd] at positions clen.., pending row causal, mask rows see the whole
               window (:508-510, :538-555); token shift (:531-536); x_extra from the last row (:557-560).
      verify : window [pending | a0, d_1..d_bd] causal (:562-576); ar_pred via the same token shift with
               seed_logit for round 0; bonus = argmax of the last row.
      accept : k = first mismatch of draft vs ar_pred; new = draft[:k] + [ar_pred[k]] or draft + [bonus] (:577-584).
      commit : keep verify KV for pending + new[:m-1]; pending = new[-1] (:600-607).
    """
    P = prefix_emb.shape[0]
    next_pos = P
    cache, seed_logit = prefill(model, prefix_emb)
    clen = P
    committed: List[int] = []
    pending: Optional[int] = None
    n_draft = n_verify = n_rounds = n_acc = 0
    done = False
    while not done and len(committed) < max_new_tokens:
        n_rounds += 1
        pre = 1 if pending is not None else 0
        r0 = clen - P
        Q = pre + bd
        pos = torch.arange(next_pos + r0, next_pos + r0 + Q)
        ids = torch.tensor(([pending] if pre else []) + [mask_id] * bd)
        cache.truncate(clen)
        raw = model.logits(model.forward(model.embed(ids), pos, cache, window_mask(clen, Q, pre)))
        used = torch.cat([raw[:1], raw[:-1]], 0) if pre else torch.cat([seed_logit, raw[:-1]], 0)
        draft = greedy(used[pre:])                                        # [bd]
        n_draft += 1
        if full_draft:
            draft = torch.cat([draft, greedy(raw[-1:])])                  # [bd+1] = a0, d_1..d_bd
        cache.truncate(clen)
        if full_draft:
            Qv = Q + 1
            ids_v = torch.cat([torch.tensor([pending]) if pre else torch.empty(0, dtype=torch.long), draft])
            lv = model.logits(model.forward(model.embed(ids_v), torch.arange(next_pos + r0, next_pos + r0 + Qv),
                                            cache, window_mask(clen, Qv, Qv)))
            pred = torch.cat([lv[:1] if pre else seed_logit, lv[:-1]], 0)[pre:]
            ar_pred = greedy(pred)
            bonus = lv[-1].float().argmax(-1, keepdim=True)
            nd = draft.shape[0]
            mism = (draft != ar_pred).nonzero()
            k = int(mism[0, 0]) if mism.numel() > 0 else nd
            new = torch.cat([draft[:k], ar_pred[k:k + 1]]) if k < nd else torch.cat([draft, bonus])
        else:
            ids_f = torch.cat([torch.tensor([pending]) if pre else torch.empty(0, dtype=torch.long), draft])
            lv = model.logits(model.forward(model.embed(ids_f), pos, cache, window_mask(clen, Q, Q)))
            used_v = torch.cat([lv[:1], lv[:-1]], 0) if pre else torch.cat([seed_logit, lv[:-1]], 0)
            ar_pred = greedy(used_v[pre:])
            mism = (draft != ar_pred).nonzero()
            k = int(mism[0, 0]) if mism.numel() > 0 else bd
            new = torch.cat([draft[:k], ar_pred[k:k + 1]]) if k < bd else draft
        n_verify += 1
        m = new.shape[0]
        cache.truncate(clen + pre + m - 1)
        clen = clen + pre + m - 1
        pending = int(new[-1])
        committed.extend(int(x) for x in new)
        n_acc += m
        if trace is not None:
            trace.append({"round": n_rounds, "k": k, "draft": draft.tolist(), "ar_pred": ar_pred.tolist(),
                          "new_tokens": new.tolist()})
        if eos_id is not None and eos_id in new.tolist():
            done = True
    gen = list(committed)
    if eos_id is not None and eos_id in gen:
        gen = gen[:gen.index(eos_id)]
    fwd = n_draft + n_verify
    stats = {"rounds": n_rounds, "draft_fwd": n_draft, "verify_fwd": n_verify, "commit_fwd": 0, "total_fwd": fwd,
             "resp_tokens": len(gen), "tokens_per_fwd": round(len(gen) / max(1, fwd), 3),
             "accept_per_round": round(n_acc / max(1, n_rounds), 2)}
    return gen, stats


def fulldraft_round(model: OracleDecoder, cache: KVCache, S: int, x0: int, bd: int, mask_id: int,
                    pos_offset: int = 0, trace: Optional[list] = None, verify_window: Optional[List[int]] = None):
    """One serving full-draft round (patches/sglang/.../selfspec_diffusion_worker.py:660-961 with
    selfspec_fast_commit.py:108-147), K = bd + 1 rows per forward, AR-aligned positions (SELFSPEC_POS_OFFSET=0):
      draft  [x0 | MASK x bd] at positions S+pos_offset.. (x0 row causal, mask rows bidirectional); am = argmax.
      x0's K/V (draft row 0, causal, exact) is committed: S += 1.
      verify [a0, d_1..d_bd] = am at positions S.. (causal); t = argmax; acc = leading matches t_r == d_{r+1}.
      commit T = [a0, t_0..t_acc]; keep verify K/V rows 0..acc: S += acc + 1; x0 = t_acc.
    ``cache`` holds exactly S committed positions on entry and S' on return. Returns (S', x0', T, acc, record).
    ``verify_window`` (K ids) replaces the draft's own argmax as the verify window: the replay of another
    implementation's round from the same state (its draft argmax may differ from this one's at near ties)."""
    K = bd + 1
    ids = torch.tensor([x0] + [mask_id] * bd)
    cache.truncate(S)
    dl = model.logits(model.forward(model.embed(ids), torch.arange(S, S + K) + pos_offset, cache,
                                    window_mask(S, K, 1)))
    am = dl.float().argmax(-1)                                           # [K] = a0, d_1..d_bd
    if verify_window is not None:
        am = torch.as_tensor(list(verify_window), dtype=torch.long)
    cache.truncate(S + 1)                                                # x0 committed from draft row 0
    S1 = S + 1
    vl = model.logits(model.forward(model.embed(am), torch.arange(S1, S1 + K) + pos_offset, cache,
                                    window_mask(S1, K, K)))
    t = vl.float().argmax(-1)
    acc = int(accept_chain(am[None].numpy(), t[None].numpy())[0])
    T = [int(am[0])] + [int(x) for x in t[: acc + 1]]
    cache.truncate(S1 + acc + 1)
    if trace is not None:
        trace.append({"draft_logits": dl, "verify_logits": vl})
    rec = {"S": S, "acc": acc, "window": am.tolist(), "target": t.tolist(), "T": T}
    return S1 + acc + 1, int(t[acc]), T, acc, rec


def fulldraft_generate(model: OracleDecoder, prefix_emb: torch.Tensor, bd: int, mask_id: int, max_new_tokens: int,
                       eos_id: Optional[int] = None, pos_offset: int = 0, trace: Optional[list] = None):
    """Prefill, then full-draft rounds until max_new_tokens are committed (or EOS). The prefill emits x0 (the
    extend step's sampled token, committed). Returns (committed ids, per-round records)."""
    cache, last = prefill(model, prefix_emb)
    x0 = int(greedy(last)[0])
    S = prefix_emb.shape[0]
    out = [x0]
    rounds = []
    while len(out) < max_new_tokens and not (eos_id is not None and eos_id in out):
        S, x0, T, acc, rec = fulldraft_round(model, cache, S, x0, bd, mask_id, pos_offset, trace)
        rounds.append(rec)
        out.extend(T)
    return out, rounds


def ar_generate(model: OracleDecoder, prefix_emb: torch.Tensor, n_tokens: int, keep_logits: bool = False):
    """Greedy AR decode with a KV cache (the reference's AR baseline, src/infer_odb_ar.py:40-50)."""
    cache, last = prefill(model, prefix_emb)
    S = prefix_emb.shape[0]
    toks = [int(last.float().argmax(-1)[0])]
    logits = [last[0]] if keep_logits else None
    while len(toks) < n_tokens:
        l = model.logits(model.forward(model.embed(torch.tensor([toks[-1]])), torch.tensor([S]), cache,
                                       window_mask(S, 1, 1)))
        S += 1
        toks.append(int(l.float().argmax(-1)[0]))
        if keep_logits:
            logits.append(l[0])
    return toks, logits


def teacher_force_argmax(model: OracleDecoder, prefix_emb: torch.Tensor, gen_ids: List[int]) -> List[int]:
    """src/fast_sampling.py:631-690: one causal forward over prefix + gen_ids; the AR argmax predicting every
    generated position."""
    P = prefix_emb.shape[0]
    g = torch.tensor(list(gen_ids), dtype=torch.long)
    emb = torch.cat([prefix_emb.to(model.dtype), model.embed(g)], 0)
    T = emb.shape[0]
    cache = KVCache(model.cfg.n_layers)
    h = model.forward(emb, torch.arange(T), cache, causal_mask(0, T))
    return model.logits(h[P - 1: T - 1]).argmax(-1).tolist()
