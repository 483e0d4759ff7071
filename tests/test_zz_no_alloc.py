"""gss_argmax_accept_noalloc (the library's own scratch, no allocation) against gss_argmax_accept (caller workspace):
targets, accept lengths, next boundary tokens and packed rows bit-exact, on two calls in a row on one stream, the
second with a smaller batch, window and vocabulary (the scratch keeps the first call's winners and counters: the
second must not see them); bf16 and fp32 logits, both greedy rules; sizes past the limit rejected."""
import pytest
import torch

pytestmark = pytest.mark.gpu


def _planted(g, bs, W, V, dtype, cuda):
    """Logits whose argmax chain matches the window up to a random point, with exact ties and a NaN row."""
    lg = torch.randn(bs, W, V, generator=g)
    win = torch.randint(0, V, (bs, W), generator=g, dtype=torch.int32)
    for b in range(bs):
        m = int(torch.randint(0, W, (1,), generator=g))
        for r in range(W - 1):
            tok = int(win[b, r + 1]) if r < m else (int(win[b, r + 1]) + 1) % V
            lg[b, r, tok] = 9.0
        lg[b, W - 1, int(torch.randint(0, V, (1,), generator=g))] = 9.0
    lg[0, 0, 3] = lg[0, 0, 5] = 12.0                  # exact tie: the lower index wins
    if bs > 1:
        lg[1, 0, 7] = float("nan")                    # NaN row
    return lg.to(dtype).to(cuda), win.to(cuda)


def _outputs(fn, lg, win, flags, cuda, **kw):
    bs, W, _ = lg.shape
    out = dict(target=torch.full((bs, W), -5, dtype=torch.int32, device=cuda),
               accept_len=torch.full((bs,), -5, dtype=torch.int32, device=cuda),
               next_x0=torch.full((bs,), -5, dtype=torch.int32, device=cuda),
               packed=torch.full((bs, W + 2), -5, dtype=torch.int32, device=cuda))
    fn(lg, out["target"], window=win, accept_len=out["accept_len"], next_x0=out["next_x0"], packed=out["packed"],
       flags=flags, **kw)
    torch.cuda.synchronize()
    return {k: v.cpu() for k, v in out.items()}


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float32])
@pytest.mark.parametrize("flags", [0, 3])
def test_noalloc_equals_workspace_entry_point(cuda, dtype, flags):
    from gravityocr_amd.kernels import argmax_accept, argmax_accept_noalloc, argmax_workspace_bytes
    g = torch.Generator().manual_seed(17 + flags)
    for bs, W, V in ((64, 33, 59392), (5, 9, 4099)):  # two calls in a row, the second smaller
        print(f"noalloc argmax bs={bs} W={W} V={V} dtype={dtype} flags={flags}", flush=True)
        lg, win = _planted(g, bs, W, V, dtype, cuda)
        got = _outputs(argmax_accept_noalloc, lg, win, flags, cuda)
        ws = torch.zeros(argmax_workspace_bytes(bs, W, V), dtype=torch.uint8, device=cuda)
        want = _outputs(argmax_accept, lg, win, flags, cuda, workspace=ws)
        for k in want:
            assert torch.equal(got[k], want[k]), (bs, W, V, k)


def test_noalloc_rejects_sizes_past_its_scratch(cuda):
    from gravityocr_amd._lib import GssError
    from gravityocr_amd.kernels import argmax_accept_noalloc
    lg = torch.zeros(65, 2, 128, dtype=torch.bfloat16, device=cuda)
    tgt = torch.zeros(65, 2, dtype=torch.int32, device=cuda)
    with pytest.raises(GssError, match="unsupported"):
        argmax_accept_noalloc(lg, tgt)
