"""Integer half of the oracle: argmax, linear-chain accept, commit packing, KV slot indices, finish rules.

Test infrastructure only (see ``oracle/__init__.py``).
"""
from typing import Iterable, List, Sequence, Tuple

import numpy as np


def bf16_bits_to_f32(bits: np.ndarray) -> np.ndarray:
    """bf16 stored as uint16 bit patterns -> float32 (exact: bf16 is the upper half of an fp32)."""
    return (bits.astype(np.uint32) << 16).view(np.float32)


def f32_to_bf16_bits(x: np.ndarray) -> np.ndarray:
    """float32 -> bf16 bit patterns, round to nearest even (NaN kept quiet), as torch's ``.to(torch.bfloat16)``."""
    u = np.ascontiguousarray(x, dtype=np.float32).view(np.uint32)
    nan = np.isnan(x)
    rounded = ((u + 0x7FFF + ((u >> 16) & 1)) >> 16).astype(np.uint16)
    rounded[nan] = ((u[nan] >> 16) | 0x40).astype(np.uint16)
    return rounded


def argmax_first(rows: np.ndarray) -> np.ndarray:
    """Greedy token rule: index of the row maximum, the LOWEST index among exact ties, NaN counted as the maximum.

    The reference draws greedy tokens with ``F.softmax(logits.float()).argmax(-1)``
    (src/models/glm_ocr_dllm.py:997-1002), ``lv.float().argmax`` (src/fast_sampling.py:575) and, on the serving path,
    ``logits.argmax(-1)`` (patches/sglang/.../selfspec_diffusion_worker.py:742). torch.argmax returns the first
    index of the maximum; the fp32 softmax of upcast bf16 keeps distinct bf16 values distinct whenever the row
    maximum is >= 2^-14 in magnitude, so all three reduce to this rule. ``rows``: [..., V] float32.
    """
    return np.argmax(rows, axis=-1).astype(np.int64)


def verify_tree_greedy(candidates: np.ndarray, target_predict: np.ndarray, retrive_index: np.ndarray,
                       retrive_next_token: np.ndarray, retrive_next_sibling: np.ndarray):
    """The published greedy tree-verify walk of sgl-kernel's ``verify_tree_greedy`` (sglang-kernel 0.4.1, not
    vendored; called at patches/sglang/.../selfspec_fast_commit.py:159 via NgramVerifyInput._greedy_verify).

    Per request: start at the root; at each depth follow first-child / next-sibling links and accept the first
    child whose candidate token equals the target prediction of the last accepted node. Returns
    (predicts [bs*n], accept_index [bs, n] (-1 padded), accept_token_num [bs]). predicts holds, for every accepted
    node, the target token there (the last accepted node's entry is the correction / bonus).
    """
    bs, n = candidates.shape
    predicts = np.zeros(bs * n, dtype=np.int64)
    accept_index = np.full((bs, n), -1, dtype=np.int64)
    accept_num = np.zeros(bs, dtype=np.int64)
    for b in range(bs):
        last = int(retrive_index[b, 0])
        accept_index[b, 0] = last
        num = 0
        cur = 0
        for _depth in range(1, n):
            cur = int(retrive_next_token[b, cur])
            matched = False
            while cur != -1:
                draft_index = int(retrive_index[b, cur])
                if int(candidates[b, cur]) == int(target_predict[last]):
                    predicts[last] = int(target_predict[last])
                    num += 1
                    accept_index[b, num] = draft_index
                    last = draft_index
                    matched = True
                    break
                cur = int(retrive_next_sibling[b, cur])
            if not matched:
                break
        accept_num[b] = num
        predicts[last] = int(target_predict[last])
    return predicts, accept_index, accept_num


def chain_links(bs: int, n: int):
    """The constant linear-chain layout the worker builds (selfspec_diffusion_worker.py:530-548):
    retrive_index = b*n + j, next = j+1 (last -1), sibling = -1."""
    ri = np.arange(bs)[:, None] * n + np.arange(n)[None, :]
    nxt = np.tile(np.arange(1, n + 1), (bs, 1))
    nxt[:, -1] = -1
    sib = np.full((bs, n), -1)
    return ri, nxt, sib


def accept_chain(window: np.ndarray, target: np.ndarray) -> np.ndarray:
    """Linear-chain greedy accept (docs/SGLANG_SELFSPEC_IMPL.md:114-121; selfspec_diffusion_worker.py:530-548):
    acc[b] = number of leading r in [0, K-2] with target[b, r] == window[b, r+1].

    window: verify ids [bs, K] = [a0, d_1..d_{K-1}]; target: argmax of the verify rows [bs, K].
    """
    bs, K = window.shape
    acc = np.zeros(bs, dtype=np.int64)
    for b in range(bs):
        a = 0
        while a < K - 1 and int(target[b, a]) == int(window[b, a + 1]):
            a += 1
        acc[b] = a
    return acc


def committed_tokens(a0: int, target_row: Sequence[int], acc: int) -> List[int]:
    """T = [a0, t_0 .. t_acc]: a0 + the accepted draft tokens (== targets) + the correction / bonus
    (selfspec_fast_commit.py:13-20, host unpacking selfspec_commit_rules.py:155-156)."""
    return [int(a0)] + [int(t) for t in target_row[: acc + 1]]


def ss_commit(predict: np.ndarray, acc: np.ndarray, a0: np.ndarray, rpi: np.ndarray, seeds: np.ndarray,
              seq_lens: np.ndarray, loc: np.ndarray, K: int, page: int = 1, finish=None):
    """Restatement of ``_ss_commit_kernel`` (patches/sglang/.../selfspec_fast_commit.py:108-147), with the host
    commit's cut (selfspec_commit_rules.py:94-103 via ``cut_index_loop``) and page-granular frees.

    Per request i with a = acc[i] and T = [a0, predict[i*K .. i*K + a]]:
      packed[i] = (a0[i], a, predict[i*K : i*K+K] with entries past a zeroed)
      seeds[rpi[i]] = out[i] = predict[i*K + a]
      j = a + 1 without ``finish`` or for budget < 0, else cut_index_loop(T, budget, stop, vocab)
      seq_lens[i] += j
      free list: slots loc[i*K + r], r = j .. K-1, whose position seq_lens[i] + r lies at or past the first page
      boundary at or after seq_lens[i] + j (pages holding a kept token stay); rows in order. With page 1 and no
      finish rule: loc[i*K + a+1 .. i*K + K-1], the reference kernel's list.
    ``finish`` = (budgets, stops, vocabs) per request. Returns (packed [bs, K+2] int32, seeds', seq_lens',
    free int64, out [bs] int64, cut [bs])."""
    bs = acc.shape[0]
    packed = np.zeros((bs, K + 2), dtype=np.int32)
    seeds = seeds.copy()
    seq_lens = seq_lens.copy()
    out = np.zeros(bs, dtype=np.int64)
    cut = np.zeros(bs, dtype=np.int64)
    free = []
    for i in range(bs):
        a = int(acc[i])
        row = [int(predict[i * K + j]) if j <= a else 0 for j in range(K)]
        packed[i, 0] = np.int32(np.int64(a0[i]).astype(np.int32))
        packed[i, 1] = a
        packed[i, 2:] = row
        s = int(predict[i * K + a])
        seeds[int(rpi[i])] = s
        out[i] = s
        T = [int(packed[i, 0])] + row[: a + 1]
        if finish is None or finish[0][i] < 0:
            j = a + 1
        else:
            j = cut_index_loop(T, int(finish[0][i]), finish[1][i], int(finish[2][i]))
        cut[i] = j
        S = int(seq_lens[i])
        first_free = -(-(S + j) // page) * page
        free.extend(int(loc[i * K + r]) for r in range(j, K) if S + r >= first_free)
        seq_lens[i] += j
    return packed, seeds, seq_lens, np.asarray(free, dtype=np.int64), out, cut


def kv_meta(req_to_token: np.ndarray, rpi: np.ndarray, seq_lens: np.ndarray, extra: int):
    """Restatement of ``_ss_kv_meta_kernel`` (patches/sglang/python/sglang/srt/speculative/selfspec_fast_attn.py:
    104-132): sequence i contributes req_to_token[rpi[i], 0 : seq_lens[i] + extra] at offset
    kv_indptr[i] = sum_{j<i} (seq_lens[j] + extra). Returns (kv_indptr int32 [bs+1], kv_indices int32)."""
    n = [int(seq_lens[i]) + extra for i in range(len(seq_lens))]
    indptr = np.zeros(len(n) + 1, dtype=np.int32)
    rows = []
    for i, ln in enumerate(n):
        indptr[i + 1] = indptr[i] + ln
        rows.append(np.asarray(req_to_token[int(rpi[i]), :ln], dtype=np.int32))
    return indptr, (np.concatenate(rows) if rows else np.zeros(0, dtype=np.int32))


def page_slot(page_table_row: np.ndarray, pos: int, page_size: int = 16) -> int:
    """Paged-KV slot of absolute position ``pos``: page_table[pos // page] * page + pos % page.

    The reference pages with page_size 1 (selfspec_fast_attn.py:213, selfspec_diffusion_worker.py:354-355), where
    the slot IS the req_to_token entry; with 16-token pages the same mapping goes through the page table."""
    return int(page_table_row[pos // page_size]) * page_size + pos % page_size


def cut_index_loop(T: Sequence[int], budget: int, stop: Iterable[int], vocab: int) -> int:
    """The per-token finish loop the closed-form ``cut_index`` replaces
    (patches/sglang/.../selfspec_commit_rules.py:9-17, :94-103): append one token at a time, after each append
    check length (output length >= max_new_tokens, i.e. appended >= budget), then stop id, then vocab boundary
    (id > vocab or id < 0); return the index of the last appended token."""
    stop = set(stop)
    appended = 0
    for t, x in enumerate(T):
        appended += 1
        if appended >= budget:
            return t
        if x in stop or x > vocab or x < 0:
            return t
    return len(T) - 1


def host_commit_loop(rows: Sequence[Sequence[int]], budgets: Sequence[int], stops: Sequence[Iterable[int]],
                     vocab: int) -> Tuple[List[List[int]], List[int], List[int]]:
    """Per-token host commit over packed rows (a0, acc, predict row) for fast requests
    (selfspec_commit_rules.py:150-170 with commit_fast): returns (tokens appended, j, acc) per request."""
    toks, js, accs = [], [], []
    for r, budget, stop in zip(rows, budgets, stops):
        a = int(r[1])
        T = [int(r[0])] + [int(x) for x in r[2: 3 + a]]
        j = cut_index_loop(T, budget, stop, vocab)
        toks.append(T[: j + 1])
        js.append(j)
        accs.append(a)
    return toks, js, accs
