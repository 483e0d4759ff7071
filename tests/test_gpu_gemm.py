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


@pytest.mark.parametrize("M,N,Kd", [(17, 2560, 1536), (17, 1536, 4608), (33, 59392, 1536), (64, 512, 256),
                                    (65, 2560, 1536), (544, 9216, 1536), (561, 59392, 1536), (136, 1536, 2048),
                                    (1056, 96, 64)])
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
    # the engine's fused post-attention norm: residual input a, updated residual to h_out (the persistent GEMM)
    gemm_swiglu(x, wgu, act_ref)
    h_out2 = torch.empty_like(h)
    gemm_swiglu(None, wgu, act, pro=dict(a=a, h_in=h, h_out=h_out2, w_post=wp, w_next=wn, eps=eps))
    torch.cuda.synchronize()
    assert torch.equal(act, act_ref) and torch.equal(h_out2, h_ref)


@pytest.mark.parametrize("M,N,Kd", [(17, 2560, 1536), (1, 1536, 2048), (17, 1536, 4608), (64, 1536, 4608),
                                    (544, 1536, 4608)])
def test_gemm_split_k_parity_and_invariance(cuda, M, N, Kd):
    """Split-K keeps fp32-reference parity and batch invariance (a row alone == the same row in a batch)."""
    from gravityocr_amd.kernels import gemm
    g = torch.Generator().manual_seed(M + N + Kd)
    x = torch.randn(M, Kd, generator=g).bfloat16().to(cuda)
    w = (torch.randn(N, Kd, generator=g) * 0.02).bfloat16().to(cuda)
    y = torch.empty(M, N, dtype=torch.float32, device=cuda)
    gemm(x, w, y)
    y1 = torch.empty(1, N, dtype=torch.float32, device=cuda)
    gemm(x[M - 1:].contiguous(), w, y1)
    torch.cuda.synchronize()
    r = ref(x, w)
    assert float((y - r).abs().max()) <= 1e-4 * float(r.abs().max()) + 1e-5
    assert torch.equal(y1[0], y[M - 1])


@pytest.mark.parametrize("M", [1, 17, 64])
@pytest.mark.parametrize("N,Kd", [(1536, 2048), (1536, 4608), (512, 704), (2048, 1536)])
def test_post_norm_epilogue_equals_separate_norm(cuda, M, N, Kd):
    """gss_norm_epilogue (h += rmsnorm(Y) * w_post; x = rmsnorm(h) * w_next inside the GEMM) == the plain GEMM followed
    by gss_add_rmsnorm, bit for bit, for split-K (Kd = 4608) and unsplit shapes, 1 to 4 chunks of 8 per lane."""
    from gravityocr_amd.kernels import add_rmsnorm, gemm
    g = torch.Generator().manual_seed(M * 3 + N + Kd)
    x = torch.randn(M, Kd, generator=g).bfloat16().to(cuda)
    w = (torch.randn(N, Kd, generator=g) * 0.02).bfloat16().to(cuda)
    h = torch.randn(M, N, generator=g).bfloat16().to(cuda)
    wp = (1 + 0.1 * torch.randn(N, generator=g)).bfloat16().to(cuda)
    wn = (1 + 0.1 * torch.randn(N, generator=g)).bfloat16().to(cuda)
    a_ref = torch.empty(M, N, dtype=torch.bfloat16, device=cuda)
    gemm(x, w, a_ref)
    h_ref, x_ref = h.clone(), torch.empty(M, N, dtype=torch.bfloat16, device=cuda)
    add_rmsnorm(a_ref, wp, h_ref, wn, x_ref, 1e-5)
    ws = torch.zeros(1 << 22, dtype=torch.uint8, device=cuda)
    for rep in range(3):  # the counters reset themselves: repeated calls on one workspace agree
        a, h2, x2 = torch.empty_like(a_ref), h.clone(), torch.empty_like(x_ref)
        gemm(x, w, a, workspace=ws, post=dict(h=h2, w_post=wp, w_next=wn, x=x2, eps=1e-5))
        torch.cuda.synchronize()
        assert torch.equal(a, a_ref) and torch.equal(h2, h_ref) and torch.equal(x2, x_ref), rep


def test_post_norm_epilogue_rejects_other_widths(cuda):
    from gravityocr_amd._lib import GssError
    from gravityocr_amd.kernels import gemm
    x = torch.zeros(4, 256, dtype=torch.bfloat16, device=cuda)
    w = torch.zeros(256, 256, dtype=torch.bfloat16, device=cuda)
    y, h, xo = (torch.zeros(4, 256, dtype=torch.bfloat16, device=cuda) for _ in range(3))
    one = torch.ones(256, dtype=torch.bfloat16, device=cuda)
    ws = torch.zeros(1 << 20, dtype=torch.uint8, device=cuda)
    with pytest.raises(GssError, match="unsupported"):
        gemm(x, w, y, workspace=ws, post=dict(h=h, w_post=one, w_next=one, x=xo, eps=1e-5))


def test_split_k_shapes_share_one_workspace(cuda):
    """The decoder's GEMM shapes one after another on one workspace (split and unsplit, different tile counts) give
    the results of the same calls on fresh workspaces."""
    from gravityocr_amd.kernels import gemm, gemm_workspace_bytes
    g = torch.Generator().manual_seed(77)
    shapes = [(2560, 1536), (1536, 2048), (9216, 1536), (1536, 4608), (59392, 1536)]
    M = 17
    xs = {kd: torch.randn(M, kd, generator=g).bfloat16().to(cuda) for kd in {kd for _, kd in shapes}}
    ws_all = [(torch.randn(n, kd, generator=g) * 0.02).bfloat16().to(cuda) for n, kd in shapes]
    shared = torch.zeros(max(gemm_workspace_bytes(M, n, kd) for n, kd in shapes), dtype=torch.uint8, device=cuda)
    for rep in range(2):
        for (n, kd), w in zip(shapes, ws_all):
            y1 = torch.empty(M, n, dtype=torch.bfloat16, device=cuda)
            gemm(xs[kd], w, y1, workspace=shared)
            y2 = torch.empty_like(y1)
            gemm(xs[kd], w, y2, workspace=torch.zeros(gemm_workspace_bytes(M, n, kd), dtype=torch.uint8,
                                                       device=cuda))
            torch.cuda.synchronize()
            assert torch.equal(y1, y2), (rep, n, kd)


PARTS_SHAPES = [(17, 1536, 2048), (17, 1536, 4608), (1, 1536, 2048), (1, 1536, 4608), (33, 1536, 2048),
                (5, 256, 256), (5, 256, 704), (544, 1536, 2048), (561, 1536, 4608), (100, 256, 704)]


@pytest.mark.parametrize("M,N,Kd", PARTS_SHAPES)
def test_gemm_parts_parity_and_invariance(cuda, M, N, Kd):
    """gss_gemm_parts: the fp32 partial sums add up to x @ w^T (fp32 reference, same bound as gss_gemm's fp32
    output); their bf16 sum is the same for a row alone (M = 1) and inside the batch; where gss_gemm splits k the
    same way (down_proj: 2 splits of 72 k-steps), bf16(parts[0] + parts[1]) is gss_gemm's output bit for bit."""
    from gravityocr_amd.kernels import gemm, gemm_parts, gemm_parts_count
    print(f"gemm_parts M={M} N={N} K={Kd}", flush=True)
    g = torch.Generator().manual_seed(M * 11 + Kd)
    x = torch.randn(M, Kd, generator=g).bfloat16().to(cuda)
    w = (torch.randn(N, Kd, generator=g) * 0.02).bfloat16().to(cuda)
    S = gemm_parts_count(N, Kd)
    assert 1 <= S <= 2
    parts = torch.full((S, M, N), float("nan"), dtype=torch.float32, device=cuda)
    gemm_parts(x, w, parts)
    r = ref(x, w)
    total = parts[0].clone()
    for k in range(1, S):
        total += parts[k]
    torch.cuda.synchronize()
    scale = float(r.abs().max())
    assert not torch.isnan(parts).any()
    assert float((total - r).abs().max()) <= 1e-4 * scale + 1e-5
    for row in (0, M - 1):
        p1 = torch.empty(S, 1, N, dtype=torch.float32, device=cuda)
        gemm_parts(x[row:row + 1].contiguous(), w, p1)
        torch.cuda.synchronize()
        assert torch.equal(p1[:, 0], parts[:, row]), row
    if (N, Kd) == (1536, 4608):
        y = torch.empty(M, N, dtype=torch.bfloat16, device=cuda)
        gemm(x, w, y)
        torch.cuda.synchronize()
        assert S == 2 and torch.equal(y, (parts[0] + parts[1]).bfloat16())


@pytest.mark.parametrize("n_parts", [1, 2, 3, 4])
def test_parts_norm_every_part_count(cuda, n_parts):
    """gss_add_rmsnorm_parts for each part count it is built for == gss_add_rmsnorm on a = bf16 of the parts added in
    part order (fp32), bit for bit."""
    from gravityocr_amd.kernels import add_rmsnorm, add_rmsnorm_parts
    g = torch.Generator().manual_seed(90 + n_parts)
    M, H, eps = 17, 1536, 1e-5
    parts = torch.randn(n_parts, M, H, generator=g).to(cuda)
    h = torch.randn(M, H, generator=g).bfloat16().to(cuda)
    wp = (1 + 0.1 * torch.randn(H, generator=g)).bfloat16().to(cuda)
    wn = (1 + 0.1 * torch.randn(H, generator=g)).bfloat16().to(cuda)
    a = parts[0].clone()
    for k in range(1, n_parts):
        a += parts[k]
    h_ref, x_ref = h.clone(), torch.empty_like(h)
    add_rmsnorm(a.bfloat16(), wp, h_ref, wn, x_ref, eps)
    h1, x1 = h.clone(), torch.empty_like(h)
    add_rmsnorm_parts(parts, wp, h1, wn, x1, eps)
    torch.cuda.synchronize()
    assert torch.equal(h1, h_ref) and torch.equal(x1, x_ref)


@pytest.mark.parametrize("M", [1, 5, 12, 17])
def test_norms_on_parts_equal_unfused(cuda, M):
    """gss_add_rmsnorm_parts == gss_add_rmsnorm on a = bf16(sum of the parts), and the gate_up prologue with a_parts
    == that norm followed by the plain gate_up GEMM, bit for bit (h updated, x, act)."""
    from gravityocr_amd.kernels import add_rmsnorm, add_rmsnorm_parts, gemm_parts, gemm_swiglu
    g = torch.Generator().manual_seed(40 + M)
    H, F, eps = 1536, 4608, 1e-5
    o = torch.randn(M, 2048, generator=g).bfloat16().to(cuda)
    wo = (torch.randn(H, 2048, generator=g) * 0.02).bfloat16().to(cuda)
    h = torch.randn(M, H, generator=g).bfloat16().to(cuda)
    wp = (1 + 0.1 * torch.randn(H, generator=g)).bfloat16().to(cuda)
    wn = (1 + 0.1 * torch.randn(H, generator=g)).bfloat16().to(cuda)
    wgu = (torch.randn(2 * F, H, generator=g) * 0.02).bfloat16().to(cuda)
    from gravityocr_amd.kernels import gemm_parts_count
    parts = torch.empty(gemm_parts_count(H, 2048), M, H, dtype=torch.float32, device=cuda)
    gemm_parts(o, wo, parts)
    a = parts[0].clone()
    for k in range(1, parts.shape[0]):
        a += parts[k]
    a = a.bfloat16()
    h_ref, x_ref = h.clone(), torch.empty_like(h)
    add_rmsnorm(a, wp, h_ref, wn, x_ref, eps)
    h1, x1 = h.clone(), torch.empty_like(h)
    add_rmsnorm_parts(parts, wp, h1, wn, x1, eps)
    torch.cuda.synchronize()
    assert torch.equal(h1, h_ref) and torch.equal(x1, x_ref)
    act_ref = torch.empty(M, F, dtype=torch.bfloat16, device=cuda)
    gemm_swiglu(x_ref, wgu, act_ref)
    act = torch.empty_like(act_ref)
    h_out = torch.empty_like(h)
    if M <= 12:   # the prologue form the engine uses (at most one row per wave)
        gemm_swiglu(None, wgu, act, pro=dict(a_parts=parts, h_in=h, h_out=h_out, w_post=wp, w_next=wn, eps=eps))
        torch.cuda.synchronize()
        assert torch.equal(act, act_ref) and torch.equal(h_out, h_ref)


@pytest.mark.parametrize("bs,W", [(4, 17), (32, 17), (32, 33), (8, 9)])
def test_batched_epilogues_equal_rows_alone(cuda, bs, W):
    """Windows of more than 64 rows (64-row slabs): the RoPE + staging and SwiGLU epilogues of a batch give, for every
    sequence, exactly what a one-sequence call gives (positions from each sequence's own length)."""
    from gravityocr_amd.kernels import gemm_rope_stage, gemm_swiglu
    from gravityocr_amd.model import SYNTH_1536 as cfg
    print(f"batched epilogues bs={bs} W={W}", flush=True)
    g = torch.Generator().manual_seed(bs * 100 + W)
    Hq, Hkv, D, Kd, F = 16, 2, 128, 1536, 4608
    x = torch.randn(bs * W, Kd, generator=g).bfloat16().to(cuda)
    w = (torch.randn((Hq + 2 * Hkv) * D, Kd, generator=g) * 0.02).bfloat16().to(cuda)
    wgu = (torch.randn(2 * F, Kd, generator=g) * 0.02).bfloat16().to(cuda)
    sl = torch.randint(0, 12000, (bs,), generator=g, dtype=torch.int32).to(cuda)
    pd = torch.randint(-50, 50, (bs,), generator=g, dtype=torch.int32).to(cuda)
    rot = cfg.rot_dim
    inv = (1.0 / (cfg.rope_theta ** (torch.arange(0, rot, 2).float() / rot))).to(cuda)
    q = torch.empty(bs, W, Hq, D, dtype=torch.bfloat16, device=cuda)
    k = torch.empty(bs, W, Hkv, D, dtype=torch.bfloat16, device=cuda)
    v = torch.empty_like(k)
    gemm_rope_stage(x, w, sl, inv, q, k, v, rot_dim=rot, pos_delta=pd)
    act = torch.empty(bs * W, F, dtype=torch.bfloat16, device=cuda)
    gemm_swiglu(x, wgu, act)
    for b in sorted({0, bs // 2, bs - 1}):
        xb = x[b * W:(b + 1) * W].contiguous()
        q1, k1, v1 = (torch.empty(1, *t.shape[1:], dtype=torch.bfloat16, device=cuda) for t in (q, k, v))
        gemm_rope_stage(xb, w, sl[b:b + 1], inv, q1, k1, v1, rot_dim=rot, pos_delta=pd[b:b + 1])
        a1 = torch.empty(W, F, dtype=torch.bfloat16, device=cuda)
        gemm_swiglu(xb, wgu, a1)
        torch.cuda.synchronize()
        assert torch.equal(q1[0], q[b]) and torch.equal(k1[0], k[b]) and torch.equal(v1[0], v[b]), b
        assert torch.equal(a1, act[b * W:(b + 1) * W]), b
