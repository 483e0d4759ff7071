"""Parity of the draft (a) / verify (b) attention kernels with the oracle's explicit-mask attention.

Kernel-only workload: 1 sequence, 16 q / 2 kv heads, head_dim 128, committed prefix L in {1K, 4K, 8K, 16K} in
16-token pages in a shuffled page order, 17 window rows (boundary token + 16 masks), Q/K/V ~ N(0,1)/sqrt(128),
seed 1; draft mask (row 0 causal, rows 1.. bidirectional) and verify mask (causal). Tolerance: max |err| <=
1e-2 * max |ref| (bf16 output). Every case runs on both kernels (row-group and wide, chosen through the plan).
Unused cache slots hold NaN, so a read outside the committed prefix would show.
"""
import numpy as np
import pytest
import torch

from oracle.attention import masked_attention, window_mask
from tests.helpers import ATTN_REL, PAGE, rel_err, shuffled_page_table

pytestmark = pytest.mark.gpu


# plan policy of the current case (the attn_kernel fixture picks the kernel through wide_min)
_POLICY = {}


@pytest.fixture(autouse=True, params=["rowgroup", "wide"])
def attn_kernel(request):
    """Every case runs through both attention kernels: the row-group kernel (small batches) and the wide kernel
    (large batches), chosen by the plan's bs * Hkv threshold."""
    _POLICY.clear()
    _POLICY["wide_min"] = 1 << 30 if request.param == "rowgroup" else 1
    yield request.param
    _POLICY.clear()


def run_case(dev, Ls, W, n_causal, Hq=16, Hkv=2, D=128, seed=1, max_kv_len=None, prefix_extra=0, verify=False,
             ws_fill=0, plan=None, inputs=None):
    bs = len(Ls)
    g = torch.Generator().manual_seed(seed)
    sc = D ** -0.5
    Lmax = max(Ls) + prefix_extra
    cap = max_kv_len if max_kv_len is not None else Lmax
    ppseq = max(1, (cap + PAGE - 1) // PAGE)
    n_pages = bs * ppseq + 3
    pt = shuffled_page_table(bs, ppseq, n_pages, seed)
    k_pages = torch.full((n_pages, Hkv, PAGE, D), float("nan"), dtype=torch.bfloat16)
    v_pages = torch.full((n_pages, Hkv, D, PAGE), float("nan"), dtype=torch.bfloat16)
    q = (torch.randn(bs, W, Hq, D, generator=g) * sc).bfloat16()
    k_win = (torch.randn(bs, W, Hkv, D, generator=g) * sc).bfloat16()
    v_win = (torch.randn(bs, W, Hkv, D, generator=g) * sc).bfloat16()
    refs = []
    for b, L0 in enumerate(Ls):
        L = L0 + prefix_extra
        k = (torch.randn(L, Hkv, D, generator=g) * sc).bfloat16()
        v = (torch.randn(L, Hkv, D, generator=g) * sc).bfloat16()
        if L:
            pos = torch.arange(L)
            pg = torch.as_tensor(pt[b])[pos // PAGE].long()
            k_pages[pg, :, pos % PAGE, :] = k
            v_pages[pg, :, :, pos % PAGE] = v
        nc = W if verify else n_causal
        refs.append(masked_attention(q[b], torch.cat([k, k_win[b]]), torch.cat([v, v_win[b]]),
                                     window_mask(L, W, nc), sc))
    from gravityocr_amd.kernels import attn_plan, attn_workspace_bytes, window_attention
    if plan is None:
        plan = attn_plan(bs, Hkv, cap, **_POLICY)
    ws = torch.full((max(1, attn_workspace_bytes(bs, Hq, Hkv, D, W, plan)),), ws_fill, dtype=torch.uint8,
                    device=dev)
    out = torch.empty(bs, W, Hq, D, dtype=torch.bfloat16, device=dev)
    dv = dict(q=q.to(dev), k_pages=k_pages.to(dev), v_pages=v_pages.to(dev), pt=torch.as_tensor(pt).to(dev),
              k_win=k_win.to(dev), v_win=v_win.to(dev))
    if inputs is not None:
        inputs.update(dv)
    window_attention(dv["q"], dv["k_pages"], dv["v_pages"], dv["pt"], torch.tensor(Ls, dtype=torch.int32, device=dev),
                     dv["k_win"], dv["v_win"], out, n_causal=None if verify else n_causal, scale=sc, plan=plan,
                     workspace=ws, prefix_extra=prefix_extra)
    torch.cuda.synchronize()
    out = out.cpu()
    assert torch.isfinite(out.float()).all()
    for b in range(bs):
        e = rel_err(out[b], refs[b])
        assert e <= ATTN_REL, (b, Ls[b], e)
    return out, refs


@pytest.mark.parametrize("L", [1024, 4096, 8192, 16384])
@pytest.mark.parametrize("verify", [False, True])
def test_block_attention_config(cuda, L, verify):
    print(f"attn L={L} verify={verify}", flush=True)
    run_case(cuda, [L], 17, 1, verify=verify)


@pytest.mark.parametrize("L", [0, 1, 15, 16, 17, 63, 64, 65, 130, 1000])
@pytest.mark.parametrize("n_causal", [0, 1, 17])
def test_draft_mask_edges(cuda, L, n_causal):
    print(f"edge L={L} nc={n_causal}", flush=True)
    run_case(cuda, [L], 17, n_causal, seed=L + 7)


@pytest.mark.parametrize("W", [1, 2, 5, 9, 33, 34, 64])
def test_window_sizes(cuda, W):
    print(f"W={W}", flush=True)
    run_case(cuda, [777], W, 1, seed=W)
    run_case(cuda, [777], W, 1, seed=W, verify=True)


def test_no_grouping_and_wide_windows(cuda):
    """Hq == Hkv (one query row per window row: the wide kernel runs a single row wave of two waves) and the widest
    window (64 rows x 8 heads = 32 N-tiles: three row groups of 11)."""
    run_case(cuda, [900, 31], 17, 1, Hq=2, Hkv=2, seed=80)
    run_case(cuda, [900, 31], 64, 64, Hq=2, Hkv=2, seed=81, verify=True)
    run_case(cuda, [2000, 70], 64, 1, seed=82)


def test_many_ragged_sequences(cuda):
    """More sequences than one wave scans at a time (the wide kernel finds its unit by a prefix scan over the batch in
    chunks of 64 sequences), with empty, one-key and tile-boundary prefixes among them, on both kernels."""
    rng = np.random.default_rng(70)
    Ls = [int(x) for x in rng.integers(0, 600, size=70)]
    Ls[0], Ls[5], Ls[63], Ls[64], Ls[69] = 0, 1, 64, 0, 1199
    print(f"bs={len(Ls)}", flush=True)
    run_case(cuda, Ls, 17, 1, max_kv_len=1300, seed=70)
    run_case(cuda, Ls, 5, 1, max_kv_len=1300, seed=71, verify=True)


def test_ragged_batch_and_capacity(cuda):
    # ragged prefixes, a capacity (max_kv_len) far above the actual lengths, as a captured graph would use
    run_case(cuda, [1024, 3, 4097, 0, 12288], 17, 1, max_kv_len=16384, seed=3)
    run_case(cuda, [1024, 3, 4097, 0, 12288], 9, 1, max_kv_len=16384, seed=4, verify=True)


def test_prefix_extra(cuda):
    # verify after an in-round x0 commit: prefix = seq_len + 1
    run_case(cuda, [500, 2047], 17, 1, prefix_extra=1, verify=True, seed=5)


def test_tiny_head_dim_64(cuda):
    # the CPU plumbing decoder's shape: 4 q / 2 kv heads, head_dim 64
    run_case(cuda, [272], 5, 1, Hq=4, Hkv=2, D=64, seed=6)
    run_case(cuda, [272, 31], 6, 6, Hq=4, Hkv=2, D=64, seed=7, verify=True)


def test_deterministic(cuda):
    a, _ = run_case(cuda, [8192], 17, 1, seed=11)
    b, _ = run_case(cuda, [8192], 17, 1, seed=11)
    assert torch.equal(a, b)


@pytest.mark.parametrize("policy", [(1, 256), (4096, 1), (64, 9)])
def test_split_policies(cuda, policy):
    """One split (direct output), one tile per split (many partials, one key lane idle), and 9-tile splits (several
    stages per split, the last one half full), each a plan of its own (no process-wide state)."""
    print(f"policy={policy}", flush=True)
    _POLICY.update(target_wgs=policy[0], min_tiles=policy[1])
    run_case(cuda, [5000], 17, 1, seed=21)
    run_case(cuda, [5000, 17, 700], 17, 1, seed=22, verify=True, max_kv_len=6000)


def test_batch_plan_reproduces_rows_alone(cuda):
    """A sequence of a ragged 32-sequence batch, computed alone under the batch's plan, gives its rows of the batched
    call bit for bit (same kernel, same key partition), for the draft and the verify mask."""
    from gravityocr_amd.kernels import attn_plan, attn_workspace_bytes, window_attention
    rng = np.random.default_rng(33)
    Ls = [int(x) for x in rng.integers(1024, 12289, size=32)]
    cap = 12288
    plan = attn_plan(32, 2, cap, **_POLICY)
    for verify in (False, True):
        ins = {}
        out_b, _ = run_case(cuda, Ls, 17, 1, seed=33, max_kv_len=cap, verify=verify, plan=plan, inputs=ins)
        q, kp, vp, pt, kw, vw = (ins[k] for k in ("q", "k_pages", "v_pages", "pt", "k_win", "v_win"))
        ws = torch.zeros(max(1, attn_workspace_bytes(1, 16, 2, 128, 17, plan)), dtype=torch.uint8, device=cuda)
        for b in (0, 7, 31):
            out = torch.empty(1, 17, 16, 128, dtype=torch.bfloat16, device=cuda)
            window_attention(q[b:b + 1], kp, vp, pt[b:b + 1], torch.tensor([Ls[b]], dtype=torch.int32, device=cuda),
                             kw[b:b + 1], vw[b:b + 1], out, n_causal=None if verify else 1, scale=128 ** -0.5,
                             plan=plan, workspace=ws)
            torch.cuda.synchronize()
            assert torch.equal(out[0].cpu(), out_b[b]), (verify, b)
