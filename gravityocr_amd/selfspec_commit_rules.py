"""Host-side finish rules of the full-draft self-spec round, dependency free (no torch import).

Restates patches/sglang/python/sglang/srt/speculative/selfspec_commit_rules.py (names, argument meaning and error
behaviour kept) for requests that follow SGLang's Req protocol: ``output_ids``, ``sampling_params``
(max_new_tokens, stop_token_ids, ignore_eos, stop_strs, stop_regex_strs), ``eos_token_ids``, ``tokenizer``,
``grammar``, ``to_finish``, ``finished()``, ``check_finished(new_accepted_len=1)``, ``vocab_size`` and the spec
counters. A round commits T = [a0] + accepted verify tokens + bonus; the per-token loop appends one token at a time
and stops at the first of length / stop id / vocab boundary, which for "fast" requests is the closed form
j = min(budget - 1, first stop id, first out-of-vocab id, len(T) - 1).
"""
import logging
from typing import Callable, List, Optional

logger = logging.getLogger(__name__)

_abort_reason_factory: Optional[Callable[[str], object]] = None


def set_abort_reason_factory(fn: Callable[[str], object]) -> None:
    """Install the finish-reason factory used when a grammar rejects a committed token (selfspec_commit_rules.py:37-39)."""
    global _abort_reason_factory
    _abort_reason_factory = fn


def grammar_accept_or_abort(req, token: int) -> bool:
    """Feed ``token`` to the request's grammar; on rejection abort the request instead of raising
    (selfspec_commit_rules.py:42-54). Returns True when accepted."""
    try:
        req.grammar.accept_token(token)
        return True
    except ValueError as e:
        logger.error("grammar rejected token %s for request %s: %s", token, getattr(req, "rid", None), e)
        if _abort_reason_factory is None:
            raise
        req.to_finish = _abort_reason_factory(f"grammar rejected token {token}")
        req.check_finished()
        return False


def stop_set(req) -> frozenset:
    """Ids that end a request: stop_token_ids | eos_token_ids | tokenizer eos + additional stops; empty with
    ignore_eos. Cached on the request (selfspec_commit_rules.py:57-78)."""
    cached = getattr(req, "_ss_stop", None)
    if cached is not None:
        return cached
    sp = req.sampling_params
    ids = set()
    if not sp.ignore_eos:
        ids.update(sp.stop_token_ids or ())
        ids.update(req.eos_token_ids or ())
        tk = req.tokenizer
        if tk is not None:
            if tk.eos_token_id is not None:
                ids.add(tk.eos_token_id)
            ids.update(getattr(tk, "additional_stop_token_ids", None) or ())
    out = frozenset(ids)
    req._ss_stop = out
    return out


def is_fast(req) -> bool:
    """True when the finish check reduces to length / stop id / vocab boundary (selfspec_commit_rules.py:81-91)."""
    sp = req.sampling_params
    return (req.grammar is None and not req.to_finish and not req.finished() and not sp.stop_strs
            and not sp.stop_regex_strs and req.vocab_size is not None)


def cut_index(T: List[int], budget: int, stop: frozenset, vocab: int) -> int:
    """Index of the last token the per-token loop appends (selfspec_commit_rules.py:94-103)."""
    last = len(T) - 1
    if budget - 1 < last:
        last = max(budget - 1, 0)
    for t in range(last):
        x = T[t]
        if x < 0 or x > vocab or x in stop:
            return t
    return last


def cannot_finish(req, T: List[int]) -> bool:
    """True iff host_commit(req, T) appends all of T and leaves the request unfinished; always False for slow
    requests (selfspec_commit_rules.py:106-118)."""
    if not is_fast(req):
        return False
    if req.sampling_params.max_new_tokens - len(req.output_ids) <= len(T):
        return False
    s = stop_set(req)
    if s and not s.isdisjoint(T):
        return False
    return min(T) >= 0 and max(T) <= req.vocab_size


def commit_fast(req, T: List[int]) -> int:
    """One extend + one check_finished for a fast request; returns j (T[:j+1] appended)."""
    j = cut_index(T, req.sampling_params.max_new_tokens - len(req.output_ids), stop_set(req), req.vocab_size)
    req.output_ids.extend(T[: j + 1])
    req.check_finished(j + 1)
    return j


def commit_slow(req, T: List[int]):
    """The per-token loop (grammar, stop strings, pending to_finish). Returns (j, a0_finished)."""
    req.output_ids.append(T[0])
    req.check_finished()
    if req.finished():
        return 0, True
    if req.grammar is not None and not grammar_accept_or_abort(req, T[0]):
        return 0, True
    for t in range(1, len(T)):
        req.output_ids.append(T[t])
        req.check_finished()
        if req.finished():
            return t, False
        if req.grammar is not None and not grammar_accept_or_abort(req, T[t]):
            return t, False
    if req.grammar is not None and not req.finished():
        req.check_finished()
    return len(T) - 1, False


def host_commit(reqs, rows) -> tuple:
    """Commit the packed rows (a0, acc, predict row) of one round into the requests
    (selfspec_commit_rules.py:150-170). Returns (tokens per request, j per request, acc per request)."""
    toks, js, accs = [], [], []
    for req, r in zip(reqs, rows):
        a = int(r[1])
        T = [int(r[0])] + [int(x) for x in r[2: 3 + a]]
        if is_fast(req):
            j = commit_fast(req, T)
            a0_fin = j == 0 and req.finished()
        else:
            j, a0_fin = commit_slow(req, T)
        req.spec_verify_ct += 1
        verified = 0 if a0_fin else a + 1
        req.spec_accepted_tokens += verified
        req.update_spec_acceptance_histogram(verified)
        toks.append(T[: j + 1])
        js.append(j)
        accs.append(a)
    return toks, js, accs
