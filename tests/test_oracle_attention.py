"""Pin the oracle's masked attention and window masks: against torch SDPA with an explicit boolean mask (a library
routine), against the reference's mask predicates (src/fast_sampling.py:508-514, a differently written formula),
and against closed forms (one visible key returns its value; equal scores return the mean of visible values)."""
import numpy as np
import pytest
import torch

from oracle.attention import gather_pages, masked_attention, window_mask
from tests.helpers import shuffled_page_table, to_pages


@pytest.mark.parametrize("L,W,nc", [(0, 5, 1), (13, 5, 0), (40, 17, 1), (40, 17, 17), (100, 3, 2)])
def test_window_mask_equals_reference_predicates(L, W, nc):
    m = window_mask(L, W, nc)
    q = np.arange(W)[:, None]
    kv = np.arange(L + W)[None, :]
    if nc == W:   # mask_causal(cur, Q): (kv < cur) | ((kv - cur) <= q)
        ref = (kv < L) | ((kv - L) <= q)
    else:         # draft_mask(cur, pre, Q): (kv < cur) | (q >= pre) | ((kv - cur) <= q)
        ref = (kv < L) | (q >= nc) | ((kv - L) <= q)
    np.testing.assert_array_equal(m, ref)


@pytest.mark.parametrize("seed", range(4))
def test_masked_attention_equals_sdpa(seed):
    g = torch.Generator().manual_seed(seed)
    W, Hq, Hkv, D, L = 7, 8, 2, 32, 45
    q = torch.randn(W, Hq, D, generator=g)
    k = torch.randn(L + W, Hkv, D, generator=g)
    v = torch.randn(L + W, Hkv, D, generator=g)
    for nc in (0, 1, 3, W):
        m = window_mask(L, W, nc)
        ours = masked_attention(q, k, v, m, D ** -0.5)
        kk = k.double().repeat_interleave(Hq // Hkv, 1).transpose(0, 1)
        vv = v.double().repeat_interleave(Hq // Hkv, 1).transpose(0, 1)
        ref = torch.nn.functional.scaled_dot_product_attention(q.double().transpose(0, 1), kk, vv,
                                                               attn_mask=torch.from_numpy(m)[None])
        torch.testing.assert_close(ours, ref.transpose(0, 1), rtol=1e-10, atol=1e-12)


def test_closed_forms():
    g = torch.Generator().manual_seed(9)
    W, Hq, Hkv, D, L = 4, 4, 2, 16, 10
    k = torch.randn(L + W, Hkv, D, generator=g)
    v = torch.randn(L + W, Hkv, D, generator=g)
    # q = 0: equal scores -> mean of the visible values
    q0 = torch.zeros(W, Hq, D)
    m = window_mask(L, W, W)
    out = masked_attention(q0, k, v, m, 1.0)
    for w in range(W):
        vis = torch.from_numpy(m[w])
        mean = v[vis].double().mean(0).repeat_interleave(Hq // Hkv, 0)
        torch.testing.assert_close(out[w], mean)
    # a single visible key (L = 0, row 0 of a causal window) -> that key's value
    out1 = masked_attention(torch.randn(W, Hq, D, generator=g), k[L:], v[L:], window_mask(0, W, W), 1.0)
    torch.testing.assert_close(out1[0], v[L].double().repeat_interleave(Hq // Hkv, 0))


def test_paging_roundtrip():
    g = torch.Generator().manual_seed(1)
    L, Hkv, D = 83, 2, 8
    k = torch.randn(L, Hkv, D, generator=g)
    v = torch.randn(L, Hkv, D, generator=g)
    pt = shuffled_page_table(1, 6, 20, seed=4)[0]
    kp = torch.full((20, Hkv, 16, D), float("nan"))
    vp = torch.full((20, Hkv, D, 16), float("nan"))
    to_pages(k, v, pt, kp, vp)
    assert torch.equal(gather_pages(kp, pt, L), k)
    assert torch.equal(gather_pages(vp, pt, L, v_transposed=True), v)
