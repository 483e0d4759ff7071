"""Bit-exact parity of the fused argmax + accept + bonus kernel (c) with the oracle.

Workload: logits bf16 [batch in {1, 8, 32}] x [17] x vocab 59392 ~ N(0,1); each row's draft equals the verify
argmax up to a planted mismatch position ~ geometric(p=0.1) capped at 16; 1% of rows get a planted near-tie (a
runner-up 5e-4 below the maximum, most of which round to exact bf16 ties, decided by the lowest-index rule).
"""
import numpy as np
import pytest
import torch

from oracle.integer import accept_chain, argmax_first, committed_tokens

pytestmark = pytest.mark.gpu


def make_case(bs, W, V, seed, near_tie_frac=0.01, dtype=torch.bfloat16):
    g = np.random.default_rng(seed)
    logits = torch.from_numpy(g.standard_normal((bs, W, V)).astype(np.float32))
    rows = logits.view(-1, V)
    n_tie = max(1, int(round(near_tie_frac * rows.shape[0])))
    for r in g.choice(rows.shape[0], n_tie, replace=False):
        top = int(rows[r].argmax())
        other = int(g.integers(0, V))
        if other == top:
            other = (top + 1) % V
        rows[r, other] = rows[r, top] - 5e-4
    logits = logits.to(dtype)
    tgt = argmax_first(logits.float().numpy())
    window = np.zeros((bs, W), dtype=np.int64)
    for b in range(bs):
        m = min(int(g.geometric(0.1)) - 1, W - 1)        # number of leading matches
        window[b, 0] = g.integers(0, V)
        for r in range(W - 1):
            wrong = (tgt[b, r] + 1 + g.integers(0, V - 1)) % V if V > 1 else tgt[b, r]  # V = 1: no other id
            window[b, r + 1] = tgt[b, r] if r < m else wrong
    return logits, window, tgt


def run(dev, logits, window, with_window=True, ld_pad=0):
    from gravityocr_amd.kernels import argmax_accept, argmax_workspace_bytes
    bs, W, V = logits.shape
    lg = logits
    if ld_pad:
        big = torch.zeros(bs, W, V + ld_pad, dtype=logits.dtype)
        big[..., :V] = logits
        lg = big[..., :V]
    lg = lg.to(dev)
    ws = torch.zeros(argmax_workspace_bytes(bs, W, V), dtype=torch.uint8, device=dev)
    target = torch.full((bs, W), -7, dtype=torch.int32, device=dev)
    acc = torch.full((bs,), -7, dtype=torch.int32, device=dev)
    nx = torch.full((bs,), -7, dtype=torch.int32, device=dev)
    packed = torch.full((bs, W + 2), -7, dtype=torch.int32, device=dev)
    win = torch.as_tensor(window, dtype=torch.int32).to(dev) if with_window else None
    for _ in range(2):  # the second launch checks that the kernel left its workspace reusable
        argmax_accept(lg, target, ws, window=win, accept_len=acc if with_window else None,
                      next_x0=nx if with_window else None, packed=packed if with_window else None)
    torch.cuda.synchronize()
    return target.cpu().numpy(), acc.cpu().numpy(), nx.cpu().numpy(), packed.cpu().numpy()


@pytest.mark.parametrize("bs", [1, 8, 32])
def test_accept_config(cuda, bs):
    print(f"accept bs={bs}", flush=True)
    W, V = 17, 59392
    logits, window, tgt = make_case(bs, W, V, seed=100 + bs)
    t, acc, nx, packed = run(cuda, logits, window)
    np.testing.assert_array_equal(t, tgt)
    want_acc = accept_chain(window, tgt)
    np.testing.assert_array_equal(acc, want_acc)
    for b in range(bs):
        a = int(want_acc[b])
        assert nx[b] == tgt[b, a]
        assert packed[b, 0] == window[b, 0] and packed[b, 1] == a
        np.testing.assert_array_equal(packed[b, 2:], [tgt[b, r] if r <= a else 0 for r in range(W)])
        T = [int(packed[b, 0])] + [int(x) for x in packed[b, 2:3 + a]]
        assert T == committed_tokens(window[b, 0], tgt[b], a)


def test_exact_ties_lowest_index(cuda):
    V = 10000
    logits = torch.zeros(2, 3, V, dtype=torch.bfloat16)
    logits[0, 0, [5, 77, 9000]] = 3.0          # three-way tie -> 5
    logits[0, 1, :] = -float("inf")              # all -inf -> 0
    logits[0, 2, [4096, 4097]] = 1.0             # tie across a chunk boundary -> 4096
    logits[1, 0, 123] = float("nan")             # NaN counts as the maximum (torch.argmax)
    logits[1, 0, 5] = float("inf")
    logits[1, 1, 9999] = 0.5                     # last element
    logits[1, 2, 0] = -0.0                       # -0 == +0 tie -> 0
    want = argmax_first(logits.float().numpy())
    assert want[1, 0] == 123 and want[0, 0] == 5 and want[0, 2] == 4096 and want[1, 2] == 0
    t, *_ = run(cuda, logits, np.zeros((2, 3), dtype=np.int64), with_window=False)
    np.testing.assert_array_equal(t, want)
    assert np.array_equal(torch.from_numpy(t.astype(np.int64)).numpy(), logits.float().argmax(-1).numpy())


@pytest.mark.parametrize("V", [1, 7, 4096, 4097, 59392])
def test_vocab_sizes_and_fp32(cuda, V):
    print(f"V={V}", flush=True)
    for dtype in (torch.bfloat16, torch.float32):
        logits, window, tgt = make_case(3, 5, V, seed=V, dtype=dtype)
        t, acc, nx, _ = run(cuda, logits, window, ld_pad=24)
        np.testing.assert_array_equal(t, tgt)
        np.testing.assert_array_equal(acc, accept_chain(window, tgt))


def test_full_accept_and_no_accept(cuda):
    W, V = 17, 5000
    logits, _, tgt = make_case(2, W, V, seed=9, near_tie_frac=0)
    window = np.zeros((2, W), dtype=np.int64)
    window[0, 1:] = tgt[0, :W - 1]               # every draft matches: acc = 16, bonus = target[16]
    window[1, 1:] = (tgt[1, :W - 1] + 1) % V     # first draft wrong: acc = 0, correction = target[0]
    t, acc, nx, packed = run(cuda, logits, window)
    assert list(acc) == [W - 1, 0]
    assert nx[0] == tgt[0, W - 1] and nx[1] == tgt[1, 0]


def test_workspace_shared_across_window_sizes(cuda):
    """Regression: one workspace serving W = 17 and W = 1 calls in turn (the round's argmax and the AR step's)."""
    from gravityocr_amd.kernels import argmax_accept, argmax_workspace_bytes
    V = 59392
    ws = torch.zeros(argmax_workspace_bytes(1, 17, V), dtype=torch.uint8, device=cuda)
    for it in range(3):
        for W in (17, 1, 9, 1):
            logits, window, tgt = make_case(1, W, V, seed=50 + 10 * it + W)
            t = torch.full((1, W), -7, dtype=torch.int32, device=cuda)
            argmax_accept(logits.to(cuda), t, ws)
            torch.cuda.synchronize()
            np.testing.assert_array_equal(t.cpu().numpy(), tgt)


@pytest.mark.parametrize("bs,V,dtype,ld_pad", [(32, 59393, torch.bfloat16, 24), (32, 12345, torch.float32, 0),
                                               (8, 59392, torch.float32, 8), (1, 59392, torch.bfloat16, 0)],
                         ids=["4-pieces-misaligned", "2-pieces-ragged", "2-pieces-f32", "1-piece"])
def test_pieces_per_workgroup(cuda, bs, V, dtype, ld_pad):
    """A workgroup scans 1, 2 or 4 pieces of 4096 logits depending on the batch's size (rows x pieces): every choice
    gives the oracle's greedy ids, with ragged vocabularies (a partial last piece), misaligned rows (the scalar path),
    planted NaNs and bf16 ties."""
    print(f"pieces bs={bs} V={V} {dtype} pad={ld_pad}", flush=True)
    W = 17
    logits, window, _ = make_case(bs, W, V, seed=V + bs, dtype=dtype)
    rows = logits.view(-1, V)
    g = np.random.default_rng(V)
    for r in g.choice(rows.shape[0], max(1, rows.shape[0] // 20), replace=False):
        rows[r, int(g.integers(0, V))] = float("nan")  # NaN is the maximum; the lowest NaN index wins
    tgt = argmax_first(logits.float().numpy())
    t, acc, nx, packed = run(cuda, logits, window, ld_pad=ld_pad)
    np.testing.assert_array_equal(t, tgt)
    np.testing.assert_array_equal(acc, accept_chain(window, tgt))
