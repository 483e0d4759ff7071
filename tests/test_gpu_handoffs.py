"""Replay stress of the kernels whose last-arriving workgroup finishes the others' work (chunk winners of
gss_argmax_accept, the k-split tiles of gss_gemm): each is captured once in a HIP graph and replayed many times with
fresh inputs written between replays, and every replay is checked (argmax against torch's first-index argmax and
the accept rule against numpy; the split-K GEMM against an eager call on the same inputs, bit for bit, and an fp32
reference). A handoff that read a stale partial or a stale counter would fail one of the replays; the counters
reset themselves inside the kernels, so the graphs hold no memset."""
import numpy as np
import pytest
import torch

pytestmark = pytest.mark.gpu

REPLAYS = 40


def test_argmax_accept_graph_replays(cuda):
    from gravityocr_amd.kernels import argmax_accept, argmax_workspace_bytes
    bs, W, V = 32, 17, 59392
    print(f"argmax_accept graph replays bs={bs} W={W} V={V}", flush=True)
    g = torch.Generator(device=cuda).manual_seed(11)
    logits = torch.empty(bs, W, V, dtype=torch.bfloat16, device=cuda)
    window = torch.zeros(bs, W, dtype=torch.int32, device=cuda)
    ws = torch.zeros(argmax_workspace_bytes(bs, W, V), dtype=torch.uint8, device=cuda)
    target = torch.empty(bs, W, dtype=torch.int32, device=cuda)
    acc = torch.empty(bs, dtype=torch.int32, device=cuda)
    nx = torch.empty(bs, dtype=torch.int32, device=cuda)
    packed = torch.empty(bs, W + 2, dtype=torch.int32, device=cuda)
    call = lambda: argmax_accept(logits, target, ws, window=window, accept_len=acc, next_x0=nx, packed=packed)
    logits.normal_(generator=g)
    call()  # eager warm-up outside the capture
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        call()
    rng = np.random.default_rng(11)
    for rep in range(REPLAYS):
        logits.normal_(generator=g)
        if rep % 4 == 0:  # exact ties of the maximum: the lowest index must win
            logits[:, :, V // 2] = logits.amax(-1)
        tgt = torch.argmax(logits.float(), dim=-1).to(torch.int32)  # first maximal index
        t_np = tgt.cpu().numpy()
        win = np.zeros((bs, W), dtype=np.int32)
        m = np.minimum(rng.geometric(0.15, bs) - 1, W - 1)  # leading matches per sequence
        for b in range(bs):
            win[b, 0] = rng.integers(0, V)
            for r in range(W - 1):
                win[b, r + 1] = t_np[b, r] if r < m[b] else (t_np[b, r] + 1 + rng.integers(0, V - 1)) % V
        window.copy_(torch.from_numpy(win))
        target.fill_(-7)
        acc.fill_(-7)
        graph.replay()
        torch.cuda.synchronize()
        assert torch.equal(target, tgt), rep
        a = acc.cpu().numpy()
        np.testing.assert_array_equal(a, m, err_msg=f"replay {rep}")
        p = packed.cpu().numpy()
        for b in range(bs):
            k = int(m[b])
            assert int(nx[b]) == t_np[b, k]
            assert p[b, 0] == win[b, 0] and p[b, 1] == k
            np.testing.assert_array_equal(p[b, 2:], [t_np[b, r] if r <= k else 0 for r in range(W)])


@pytest.mark.parametrize("M", [1, 17])
def test_split_k_gemm_graph_replays(cuda, M):
    from gravityocr_amd.kernels import gemm, gemm_workspace_bytes
    N, Kd = 1536, 4608  # down_proj's shape: the k-split kernel with the counter handoff
    print(f"split-K gemm graph replays M={M}", flush=True)
    g = torch.Generator(device=cuda).manual_seed(5 + M)
    x = torch.empty(M, Kd, dtype=torch.bfloat16, device=cuda)
    w = (torch.randn(N, Kd, device=cuda, generator=g) * 0.02).bfloat16()
    y = torch.empty(M, N, dtype=torch.float32, device=cuda)
    y_eager = torch.empty_like(y)
    ws = torch.zeros(gemm_workspace_bytes(M, N, Kd), dtype=torch.uint8, device=cuda)
    x.normal_(generator=g)
    gemm(x, w, y, workspace=ws)
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        gemm(x, w, y, workspace=ws)
    for rep in range(REPLAYS):
        x.normal_(generator=g)
        y.fill_(float("nan"))
        graph.replay()
        gemm(x, w, y_eager, workspace=ws)
        torch.cuda.synchronize()
        assert torch.equal(y, y_eager), rep
        r = x.float() @ w.float().t()
        assert float((y - r).abs().max()) <= 1e-4 * float(r.abs().max()) + 1e-5, rep
