"""Parity of the fused decoder-layer helpers with transformers' GLM-OCR bf16 module math, restated with torch CPU
bf16 ops (each op rounds to bf16, as the reference's bf16 module does). RoPE, RMSNorm and the norm-residual-norm
step must agree bit for bit up to one bf16 ulp on isolated elements (transcendentals and reduction order differ)."""
import pytest
import torch

from oracle.decoder import DecoderConfig, inv_freq

pytestmark = pytest.mark.gpu


def ulp_close(a, b, max_frac=1e-3):
    """equal, or within one bf16 ulp on at most max_frac of the elements"""
    a, b = a.float().cpu(), b.float().cpu()
    diff = (a - b).abs()
    ulp = torch.maximum(a.abs(), b.abs()).clamp_min(1e-30) * 2 ** -7
    bad = diff > ulp * 1.01
    assert not bad.any(), f"{int(bad.sum())} elements beyond one ulp, max diff {float(diff.max())}"
    assert float((diff > 0).float().mean()) <= max_frac + 0.05


def hf_rope_bf16(x, pos, cfg):
    """transformers apply_rotary_pos_emb on bf16 tensors: cos/sin cast to bf16, interleaved pairs, partial."""
    freqs = pos.float()[:, None] * inv_freq(cfg)[None]
    emb = torch.cat([freqs, freqs], -1)
    cos, sin = emb.cos().bfloat16()[:, None, :], emb.sin().bfloat16()[:, None, :]
    cos = cos[..., : cos.shape[-1] // 2].repeat_interleave(2, -1)
    sin = sin[..., : sin.shape[-1] // 2].repeat_interleave(2, -1)
    r = cos.shape[-1]
    xr, xp = x[..., :r], x[..., r:]
    rot = torch.stack((-xr[..., 1::2], xr[..., 0::2]), -1).flatten(-2)
    return torch.cat([xr * cos + rot * sin, xp], -1)


def test_rope_stage(cuda):
    from gravityocr_amd.kernels import rope_stage
    cfg = DecoderConfig(hidden=1536, n_heads=16, n_kv_heads=2, head_dim=128)
    bs, W, Hq, Hkv, D = 3, 17, 16, 2, 128
    g = torch.Generator().manual_seed(0)
    qkv = torch.randn(bs * W, (Hq + 2 * Hkv) * D, generator=g).bfloat16()
    S = torch.tensor([0, 5000, 12000], dtype=torch.int32)
    q = torch.empty(bs, W, Hq, D, dtype=torch.bfloat16, device=cuda)
    kw = torch.empty(bs, W, Hkv, D, dtype=torch.bfloat16, device=cuda)
    vw = torch.empty_like(kw)
    rope_stage(qkv.to(cuda), S.to(cuda), inv_freq(cfg).to(cuda), q, kw, vw, pos_offset=1, rot_dim=cfg.rot_dim)
    torch.cuda.synchronize()
    pos = (S[:, None] + 1 + torch.arange(W)[None]).reshape(-1)
    x = qkv.view(bs * W, Hq + 2 * Hkv, D)
    ref_q = hf_rope_bf16(x[:, :Hq], pos, cfg).view(bs, W, Hq, D)
    ref_k = hf_rope_bf16(x[:, Hq:Hq + Hkv], pos, cfg).view(bs, W, Hkv, D)
    ulp_close(q, ref_q)
    ulp_close(kw, ref_k)
    assert torch.equal(vw.cpu(), x[:, Hq + Hkv:].reshape(bs, W, Hkv, D))


def hf_rmsnorm(x, w, eps):
    h = x.float()
    h = h * torch.rsqrt(h.pow(2).mean(-1, keepdim=True) + eps)
    return w * h.to(x.dtype)


def test_norms_and_silu(cuda):
    from gravityocr_amd.kernels import add_rmsnorm, rmsnorm, silu_mul
    g = torch.Generator().manual_seed(1)
    rows, H, F, eps = 17, 1536, 4608, 1e-5
    x = torch.randn(rows, H, generator=g).bfloat16()
    a = (torch.randn(rows, H, generator=g) * 3).bfloat16()
    w1 = (1 + 0.1 * torch.randn(H, generator=g)).bfloat16()
    w2 = (1 + 0.1 * torch.randn(H, generator=g)).bfloat16()
    out = torch.empty(rows, H, dtype=torch.bfloat16, device=cuda)
    rmsnorm(x.to(cuda), w1.to(cuda), out, eps)
    torch.cuda.synchronize()
    ulp_close(out, hf_rmsnorm(x, w1, eps))
    h = x.to(cuda).clone()
    xo = torch.empty_like(h)
    add_rmsnorm(a.to(cuda), w1.to(cuda), h, w2.to(cuda), xo, eps)
    torch.cuda.synchronize()
    h_ref = x + hf_rmsnorm(a, w1, eps)
    ulp_close(h, h_ref)
    ulp_close(xo, hf_rmsnorm(h_ref, w2, eps))
    gu = torch.randn(rows, 2 * F, generator=g).bfloat16()
    act = torch.empty(rows, F, dtype=torch.bfloat16, device=cuda)
    silu_mul(gu.to(cuda), act)
    torch.cuda.synchronize()
    gate, up = gu.chunk(2, -1)
    ulp_close(act, up * torch.nn.functional.silu(gate))


@pytest.mark.parametrize("rows,H", [(17, 1536), (1, 1536), (33, 256), (5, 64)])
def test_embed_rmsnorm_equals_lookup_then_norm(cuda, rows, H):
    """The fused lookup + first input norm equals index_select followed by gss_rmsnorm bit for bit; ids outside the
    table give zero rows (h and x)."""
    from gravityocr_amd.kernels import embed_rmsnorm, rmsnorm
    print(f"embed_rmsnorm rows={rows} H={H}", flush=True)
    g = torch.Generator().manual_seed(rows * 7 + H)
    V, eps = 4096, 1e-5
    table = torch.randn(V, H, generator=g).bfloat16().to(cuda)
    w = (1 + 0.1 * torch.randn(H, generator=g)).bfloat16().to(cuda)
    ids = torch.randint(0, V, (rows,), generator=g, dtype=torch.int32)
    ids[0] = V - 1
    if rows > 2:
        ids[1], ids[2] = -1, V          # out of range: zero rows
    ids = ids.to(cuda)
    h = torch.full((rows, H), 7.0, dtype=torch.bfloat16, device=cuda)
    x = torch.full((rows, H), 7.0, dtype=torch.bfloat16, device=cuda)
    embed_rmsnorm(table, ids, w, h, x, eps)
    valid = (ids >= 0) & (ids < V)
    h_ref = torch.zeros(rows, H, dtype=torch.bfloat16, device=cuda)
    h_ref[valid] = table[ids[valid].long()]
    x_ref = torch.empty_like(h_ref)
    rmsnorm(h_ref, w, x_ref, eps)
    torch.cuda.synchronize()
    assert torch.equal(h, h_ref)
    assert torch.equal(x, x_ref)
    assert not x[~valid].any()
