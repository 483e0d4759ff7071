"""The skinny decode GEMMs: parity with an fp32 torch reference at the decoder's shapes, batch invariance (a row's
result does not depend on M or on its row position: bit-identical), and the fused RoPE / SwiGLU epilogues against
the unfused kernels (bit-identical) and torch's bf16 SwiGLU."""
import pytest
import torch

pytestmark = pytest.mark.gpu

SHAPES = [(17, 2560, 1536), (17, 1536, 2048), (17, 1536, 4608), (17, 59392, 1536), (1, 1536, 4608), (64, 9216, 1536),
          (33, 2560, 1536), (5, 512, 256), (5, 256, 704), (2, 96, 64)]


def ref(x, w):
    return x.float() @ w.float().t()


@pytest.mark.parametrize("M,N,Kd", SHAPES)
def test_gemm_parity_and_fp32_out(cuda, M, N, Kd):
    from gravityocr_amd.kernels import gemm
    print(f"gemm M={M} N={N} K={Kd}", flush=True)
    g = torch.Generator().manual_seed(M * 7 + N)
    x = torch.randn(M, Kd, generator=g).bfloat16().to(cuda)
    w = (torch.randn(N, Kd, generator=g) * 0.02).bfloat16().to(cuda)
    r = ref(x, w)
    y = torch.empty(M, N, dtype=torch.bfloat16, device=cuda)
    gemm(x, w, y)
    y32 = torch.empty(M, N, dtype=torch.float32, device=cuda)
    gemm(x, w, y32)
    torch.cuda.synchronize()
    scale = float(r.abs().max())
    assert float((y32 - r).abs().max()) <= 1e-4 * scale + 1e-5
    assert float((y.float() - r).abs().max()) <= 8e-3 * scale
    assert torch.equal(y, y32.bfloat16())


@pytest.mark.parametrize("M,N,Kd", [(17, 2560, 1536), (17, 1536, 4608), (33, 59392, 1536), (64, 512, 256)])
def test_gemm_batch_invariance(cuda, M, N, Kd):
    from gravityocr_amd.kernels import gemm
    g = torch.Generator().manual_seed(3)
    x = torch.randn(M, Kd, generator=g).bfloat16().to(cuda)
    w = (torch.randn(N, Kd, generator=g) * 0.02).bfloat16().to(cuda)
    y = torch.empty(M, N, dtype=torch.bfloat16, device=cuda)
    gemm(x, w, y)
    perm = torch.randperm(M, generator=g).to(cuda)
    yp = torch.empty_like(y)
    gemm(x[perm].contiguous(), w, yp)
    for r in (0, M // 2, M - 1):
        y1 = torch.empty(1, N, dtype=torch.bfloat16, device=cuda)
        gemm(x[r:r + 1].contiguous(), w, y1)
        torch.cuda.synchronize()
        assert torch.equal(y1[0], y[r]), r
    assert torch.equal(yp, y[perm])


def test_gemm_swiglu(cuda):
    from gravityocr_amd.kernels import gemm, gemm_swiglu
    g = torch.Generator().manual_seed(4)
    M, F, Kd = 17, 4608, 1536
    x = torch.randn(M, Kd, generator=g).bfloat16().to(cuda)
    wgu = (torch.randn(2 * F, Kd, generator=g) * 0.02).bfloat16()
    wil = wgu.view(2, F, Kd).transpose(0, 1).reshape(2 * F, Kd).contiguous().to(cuda)
    act = torch.empty(M, F, dtype=torch.bfloat16, device=cuda)
    gemm_swiglu(x, wil, act)
    gu = torch.empty(M, 2 * F, dtype=torch.bfloat16, device=cuda)
    gemm(x, wgu.to(cuda), gu)                         # same rows, un-interleaved: gate | up
    torch.cuda.synchronize()
    gate, up = gu.float().cpu().bfloat16().chunk(2, -1)
    want = up * torch.nn.functional.silu(gate)        # torch bf16 ops: silu rounded, product rounded
    a, b = act.cpu().float(), want.float()
    ulp = torch.maximum(a.abs(), b.abs()).clamp_min(1e-30) * 2 ** -7
    assert bool(((a - b).abs() <= ulp * 1.01).all())
    assert float((a != b).float().mean()) < 0.01


def test_gemm_rope_stage_equals_unfused(cuda):
    from gravityocr_amd.kernels import gemm, gemm_rope_stage, rope_stage
    from gravityocr_amd.model import SYNTH_1536 as cfg
    g = torch.Generator().manual_seed(5)
    bs, W, Hq, Hkv, D, Kd = 2, 17, 16, 2, 128, 1536
    x = torch.randn(bs * W, Kd, generator=g).bfloat16().to(cuda)
    w = (torch.randn((Hq + 2 * Hkv) * D, Kd, generator=g) * 0.02).bfloat16().to(cuda)
    sl = torch.tensor([100, 8191], dtype=torch.int32, device=cuda)
    rot = cfg.rot_dim
    inv = (1.0 / (cfg.rope_theta ** (torch.arange(0, rot, 2).float() / rot))).to(cuda)
    q1 = torch.empty(bs, W, Hq, D, dtype=torch.bfloat16, device=cuda)
    k1 = torch.empty(bs, W, Hkv, D, dtype=torch.bfloat16, device=cuda)
    v1 = torch.empty_like(k1)
    gemm_rope_stage(x, w, sl, inv, q1, k1, v1, rot_dim=rot)
    qkv = torch.empty(bs * W, (Hq + 2 * Hkv) * D, dtype=torch.bfloat16, device=cuda)
    gemm(x, w, qkv)
    q2, k2, v2 = torch.empty_like(q1), torch.empty_like(k1), torch.empty_like(v1)
    rope_stage(qkv, sl, inv, q2, k2, v2, rot_dim=rot)
    torch.cuda.synchronize()
    assert torch.equal(q1, q2) and torch.equal(k1, k2) and torch.equal(v1, v2)


@pytest.mark.parametrize("M", [1, 17, 33])
def test_norm_prologue_equals_unfused(cuda, M):
    """gss_norm_prologue inside the GEMMs == gss_add_rmsnorm followed by the plain GEMM, bit for bit."""
    from gravityocr_amd.kernels import add_rmsnorm, gemm, gemm_rope_stage, gemm_swiglu, rmsnorm
    g = torch.Generator().manual_seed(10 + M)
    H, eps = 1536, 1e-5
    a = (torch.randn(M, H, generator=g) * 3).bfloat16().to(cuda)
    h = torch.randn(M, H, generator=g).bfloat16().to(cuda)
    wp = (1 + 0.1 * torch.randn(H, generator=g)).bfloat16().to(cuda)
    wn = (1 + 0.1 * torch.randn(H, generator=g)).bfloat16().to(cuda)
    w = (torch.randn(2560, H, generator=g) * 0.02).bfloat16().to(cuda)
    # unfused
    h_ref = h.clone()
    x = torch.empty_like(h)
    add_rmsnorm(a, wp, h_ref, wn, x, eps)
    y_ref = torch.empty(M, 2560, dtype=torch.bfloat16, device=cuda)
    gemm(x, w, y_ref)
    # fused
    h_out = torch.empty_like(h)
    y = torch.empty_like(y_ref)
    gemm(None, w, y, pro=dict(a=a, h_in=h, h_out=h_out, w_post=wp, w_next=wn, eps=eps))
    torch.cuda.synchronize()
    assert torch.equal(y, y_ref) and torch.equal(h_out, h_ref)
    # no residual input: x = rmsnorm(h) * w_next
    x2 = torch.empty_like(h)
    rmsnorm(h, wn, x2, eps)
    gemm(x2, w, y_ref)
    gemm(None, w, y, pro=dict(h_in=h, w_next=wn, eps=eps))
    torch.cuda.synchronize()
    assert torch.equal(y, y_ref)
    # swiglu and rope epilogues with the prologue
    wgu = (torch.randn(2 * 4608, H, generator=g) * 0.02).bfloat16().to(cuda)
    act_ref = torch.empty(M, 4608, dtype=torch.bfloat16, device=cuda)
    act = torch.empty_like(act_ref)
    gemm_swiglu(x2, wgu, act_ref)
    gemm_swiglu(None, wgu, act, pro=dict(h_in=h, w_next=wn, eps=eps))
    torch.cuda.synchronize()
    assert torch.equal(act, act_ref)
