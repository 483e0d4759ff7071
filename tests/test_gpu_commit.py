"""Bit-exact parity of the KV-commit kernel (d): accepted window rows land in their paged slots, everything else
is untouched, lengths advance, slot indices follow page_table[pos // 16] * 16 + pos % 16.

Workload: 16 layers, 2 kv heads, head_dim 128, 17-row window, batch in {1, 8, 32}, committed lengths ~U[1K, 12K],
rows committed per sequence = accept length + 1 with accept ~U[0, 16], shuffled 16-token pages.
"""
import numpy as np
import pytest
import torch

from oracle.integer import page_slot
from tests.helpers import PAGE, shuffled_page_table

pytestmark = pytest.mark.gpu


@pytest.mark.parametrize("bs", [1, 8, 32])
def test_commit_config(cuda, bs):
    from gravityocr_amd.kernels import commit_workspace_bytes, kv_commit
    print(f"commit bs={bs}", flush=True)
    nl, W, Hkv, D = 16, 17, 2, 128
    g = np.random.default_rng(bs)
    S = g.integers(1024, 12288, bs).astype(np.int32)
    acc = g.integers(0, W, bs).astype(np.int32)
    ppseq = (int(S.max()) + W + PAGE) // PAGE + 1
    n_pages = bs * ppseq + 2
    pt = shuffled_page_table(bs, ppseq, n_pages, seed=bs)
    k_pages = torch.randn(nl, n_pages, Hkv, PAGE, D).bfloat16()
    v_pages = torch.randn(nl, n_pages, Hkv, D, PAGE).bfloat16()
    k_win = torch.randn(nl, bs, W, Hkv, D).bfloat16()
    v_win = torch.randn(nl, bs, W, Hkv, D).bfloat16()
    dk, dv = k_pages.cuda(), v_pages.cuda()
    sl = torch.as_tensor(S).cuda()
    slots = torch.full((bs, W), -9, dtype=torch.int32, device="cuda")
    ws = torch.zeros(commit_workspace_bytes(bs), dtype=torch.uint8, device="cuda")
    kv_commit(k_win.cuda(), v_win.cuda(), dk, dv, torch.as_tensor(pt).cuda(), sl, ws,
              n_rows=torch.as_tensor(acc).cuda(), n_add=1, slots=slots)
    torch.cuda.synchronize()
    # expected: the oracle's placement of the committed rows
    ek, ev = k_pages.clone(), v_pages.clone()
    want_slots = np.full((bs, W), -1, dtype=np.int64)
    for b in range(bs):
        for j in range(int(acc[b]) + 1):
            pos = int(S[b]) + j
            slot = page_slot(pt[b], pos, PAGE)
            want_slots[b, j] = slot
            ek[:, slot // PAGE, :, slot % PAGE, :] = k_win[:, b, j]
            ev[:, slot // PAGE, :, :, slot % PAGE] = v_win[:, b, j]
    assert torch.equal(dk.cpu(), ek)
    assert torch.equal(dv.cpu(), ev)
    np.testing.assert_array_equal(sl.cpu().numpy(), S + acc + 1)
    np.testing.assert_array_equal(slots.cpu().numpy(), want_slots)
    # a second call (n_add only) reuses the workspace counters
    kv_commit(k_win.cuda(), v_win.cuda(), dk, dv, torch.as_tensor(pt).cuda(), sl, ws, n_add=1)
    torch.cuda.synchronize()
    np.testing.assert_array_equal(sl.cpu().numpy(), S + acc + 2)


@pytest.mark.parametrize("W,n_fixed", [(1, None), (33, None), (300, 300), (16, 16)])
def test_commit_window_sizes(cuda, W, n_fixed):
    """The AR step (W = 1), the 33-row window, a prefill-sized commit (n = W = 300 rows, 20 pages) and a full
    16-row window at every page alignment of the committed length."""
    from gravityocr_amd.kernels import commit_workspace_bytes, kv_commit
    print(f"commit W={W}", flush=True)
    nl, Hkv, D = 2, 2, 128
    bs = 16
    g = np.random.default_rng(W)
    S = (np.arange(bs) * 97 + g.integers(0, 16, bs)).astype(np.int32)   # every alignment mod 16
    S[np.arange(bs) % 16 == 0] = 0
    if n_fixed is None:
        acc = g.integers(0, W, bs).astype(np.int32)
        n_add = 1
    else:
        acc = np.zeros(bs, dtype=np.int32)
        n_add = n_fixed
    ppseq = (int(S.max()) + W + PAGE) // PAGE + 1
    n_pages = bs * ppseq + 2
    pt = shuffled_page_table(bs, ppseq, n_pages, seed=W)
    k_pages = torch.randn(nl, n_pages, Hkv, PAGE, D).bfloat16()
    v_pages = torch.randn(nl, n_pages, Hkv, D, PAGE).bfloat16()
    k_win = torch.randn(nl, bs, W, Hkv, D).bfloat16()
    v_win = torch.randn(nl, bs, W, Hkv, D).bfloat16()
    dk, dv = k_pages.cuda(), v_pages.cuda()
    sl = torch.as_tensor(S).cuda()
    slots = torch.full((bs, W), -9, dtype=torch.int32, device="cuda")
    ws = torch.zeros(commit_workspace_bytes(bs), dtype=torch.uint8, device="cuda")
    kv_commit(k_win.cuda(), v_win.cuda(), dk, dv, torch.as_tensor(pt).cuda(), sl, ws,
              n_rows=torch.as_tensor(acc).cuda(), n_add=n_add, slots=slots)
    torch.cuda.synchronize()
    ek, ev = k_pages.clone(), v_pages.clone()
    want_slots = np.full((bs, W), -1, dtype=np.int64)
    n = np.minimum(acc + n_add, W)
    for b in range(bs):
        for j in range(int(n[b])):
            slot = page_slot(pt[b], int(S[b]) + j, PAGE)
            want_slots[b, j] = slot
            ek[:, slot // PAGE, :, slot % PAGE, :] = k_win[:, b, j]
            ev[:, slot // PAGE, :, :, slot % PAGE] = v_win[:, b, j]
    assert torch.equal(dk.cpu(), ek)
    assert torch.equal(dv.cpu(), ev)
    np.testing.assert_array_equal(sl.cpu().numpy(), S + n)
    np.testing.assert_array_equal(slots.cpu().numpy(), want_slots)
