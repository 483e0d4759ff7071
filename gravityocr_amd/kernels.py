"""torch-tensor front end of the C-ABI kernels. Every function validates shapes / dtypes / devices on the host
(the kernels trust their arguments), launches on torch's current stream and raises on a non-zero status."""
import ctypes
from typing import Optional

import torch

from ._lib import AttnPlan, FinishRule, NormEpilogue, NormPrologue, Penalties, check, lib

PAGE = 16
ATTN_ROWGROUP, ATTN_WIDE = 0, 1


def _stream():
    return ctypes.c_void_p(torch.cuda.current_stream().cuda_stream)


def _ptr(t: Optional[torch.Tensor]):
    return ctypes.c_void_p(0 if t is None else t.data_ptr())


def _need(t: torch.Tensor, dtype, name: str, shape=None):
    if not t.is_cuda:
        raise ValueError(f"{name} must be a GPU tensor")
    if t.dtype != dtype:
        raise ValueError(f"{name} must be {dtype}, got {t.dtype}")
    if not t.is_contiguous():
        raise ValueError(f"{name} must be contiguous")
    if shape is not None and tuple(t.shape) != tuple(shape):
        raise ValueError(f"{name} has shape {tuple(t.shape)}, expected {tuple(shape)}")


_PLANS = {}


def attn_plan(bs: int, Hkv: int, max_kv_len: int, *, target_wgs: int = 0, min_tiles: int = 0,
              wide_min: int = 0) -> AttnPlan:
    """The attention plan (kernel + key partition) of a batch shape (gss_attn_make_plan; zeros = the defaults).
    Plans are values: two calls with the same arguments return equal plans."""
    key = (bs, Hkv, max_kv_len, target_wgs, min_tiles, wide_min)
    if key not in _PLANS:
        plan = AttnPlan()
        check(lib().gss_attn_make_plan(bs, Hkv, max_kv_len, target_wgs, min_tiles, wide_min, ctypes.byref(plan)),
              "gss_attn_make_plan")
        _PLANS[key] = plan
    return _PLANS[key]


def attn_workspace_bytes(bs, Hq, Hkv, D, W, plan) -> int:
    """Workspace of an attention call; ``plan`` is an AttnPlan or a capacity (the default plan of that capacity)."""
    if not isinstance(plan, AttnPlan):
        plan = attn_plan(bs, Hkv, int(plan))
    n = ctypes.c_size_t(0)
    check(lib().gss_attn_workspace_size(bs, Hq, Hkv, D, W, ctypes.byref(plan), ctypes.byref(n)),
          "gss_attn_workspace_size")
    return n.value


def argmax_workspace_bytes(bs, W, V) -> int:
    n = ctypes.c_size_t(0)
    check(lib().gss_argmax_workspace_size(bs, W, V, ctypes.byref(n)), "gss_argmax_workspace_size")
    return n.value


def commit_workspace_bytes(bs) -> int:
    n = ctypes.c_size_t(0)
    check(lib().gss_kv_commit_workspace_size(bs, ctypes.byref(n)), "gss_kv_commit_workspace_size")
    return n.value


def window_attention(q, k_pages, v_pages, page_table, prefix_len, k_win, v_win, out, *, n_causal: Optional[int],
                     scale: float, max_kv_len: Optional[int] = None, plan: Optional[AttnPlan] = None,
                     workspace: Optional[torch.Tensor], prefix_extra: int = 0):
    """Draft (n_causal given) or verify (n_causal None) attention. Shapes: q/out [bs, W, Hq, D] bf16,
    k_pages [n_pages, Hkv, 16, D], v_pages [n_pages, Hkv, D, 16], page_table int32 [bs, P], prefix_len int32 [bs],
    k_win/v_win [bs, W, Hkv, D]. ``plan`` (AttnPlan) fixes the kernel and key partition; without one, the default
    plan of (bs, Hkv, max_kv_len)."""
    bs, W, Hq, D = q.shape
    n_pages, Hkv = k_pages.shape[0], k_pages.shape[1]
    _need(q, torch.bfloat16, "q")
    _need(out, torch.bfloat16, "out", q.shape)
    _need(k_pages, torch.bfloat16, "k_pages", (n_pages, Hkv, PAGE, D))
    _need(v_pages, torch.bfloat16, "v_pages", (n_pages, Hkv, D, PAGE))
    _need(k_win, torch.bfloat16, "k_win", (bs, W, Hkv, D))
    _need(v_win, torch.bfloat16, "v_win", (bs, W, Hkv, D))
    _need(page_table, torch.int32, "page_table")
    _need(prefix_len, torch.int32, "prefix_len", (bs,))
    if page_table.shape[0] != bs:
        raise ValueError("page_table rows != batch")
    if plan is None:
        if max_kv_len is None:
            raise ValueError("window_attention needs a plan or a capacity (max_kv_len)")
        plan = attn_plan(bs, Hkv, int(max_kv_len))
    if plan.max_kv_len > page_table.shape[1] * PAGE:
        raise ValueError("the plan's capacity exceeds what the page table addresses")
    need = attn_workspace_bytes(bs, Hq, Hkv, D, W, plan)
    ws_bytes = 0 if workspace is None else workspace.numel() * workspace.element_size()
    if need > ws_bytes:
        raise ValueError(f"attention workspace {ws_bytes} B < {need} B")
    L = lib()
    common = (_ptr(q), _ptr(k_pages), _ptr(v_pages), _ptr(page_table), page_table.shape[1], _ptr(prefix_len),
              prefix_extra, _ptr(k_win), _ptr(v_win), _ptr(out), bs, W)
    tail = (Hq, Hkv, D, PAGE, float(scale), ctypes.byref(plan), _ptr(workspace), ws_bytes, _stream())
    if n_causal is None:
        check(L.gss_verify_attn(*common, *tail), "gss_verify_attn")
    else:
        check(L.gss_draft_attn(*common, int(n_causal), *tail), "gss_draft_attn")
    return out


ARGMAX_SOFTMAX, ARGMAX_LAST_RAW = 1, 2


def argmax_accept(logits, target, workspace, *, window=None, accept_len=None, next_x0=None, packed=None,
                  flags: int = 0):
    """logits [bs, W, V] (bf16 or fp32, rows may be strided: logits.stride(1) is the row stride, last dim dense);
    target int32 [bs, W]. With ``window`` (int32 [bs, W]) also accept_len / next_x0 [bs] and packed [bs, W+2].
    ``flags``: ARGMAX_SOFTMAX (argmax of the fp32 softmax: rows with a NaN or +inf give 0), optionally with
    ARGMAX_LAST_RAW (the last row of each sequence keeps the raw rule, NaN as the maximum)."""
    bs, W, V = logits.shape
    if not logits.is_cuda or logits.stride(2) != 1 or logits.stride(0) != W * logits.stride(1):
        raise ValueError("logits must be a GPU tensor [bs, W, V] with dense rows and a uniform row stride")
    dt = {torch.bfloat16: 0, torch.float32: 1}.get(logits.dtype)
    if dt is None:
        raise ValueError("logits must be bf16 or fp32")
    _need(target, torch.int32, "target", (bs, W))
    for name, t, shp in (("window", window, (bs, W)), ("accept_len", accept_len, (bs,)),
                         ("next_x0", next_x0, (bs,)), ("packed", packed, (bs, W + 2))):
        if t is not None:
            _need(t, torch.int32, name, shp)
    need = argmax_workspace_bytes(bs, W, V)
    if workspace.numel() * workspace.element_size() < need:
        raise ValueError("argmax workspace too small")
    check(lib().gss_argmax_accept(_ptr(logits), dt, logits.stride(1), bs, W, V, int(flags), _ptr(window), _ptr(target),
                                  _ptr(accept_len), _ptr(next_x0), _ptr(packed), _ptr(workspace),
                                  workspace.numel() * workspace.element_size(), _stream()), "gss_argmax_accept")


def argmax_accept_noalloc(logits, target, *, window=None, accept_len=None, next_x0=None, packed=None,
                          flags: int = 0):
    """argmax_accept without a workspace (gss_argmax_accept_noalloc: the library's own scratch, nothing allocated);
    bs <= 64. Same arguments and outputs as argmax_accept."""
    bs, W, V = logits.shape
    if not logits.is_cuda or logits.stride(2) != 1 or logits.stride(0) != W * logits.stride(1):
        raise ValueError("logits must be a GPU tensor [bs, W, V] with dense rows and a uniform row stride")
    dt = {torch.bfloat16: 0, torch.float32: 1}.get(logits.dtype)
    if dt is None:
        raise ValueError("logits must be bf16 or fp32")
    _need(target, torch.int32, "target", (bs, W))
    for name, t, shp in (("window", window, (bs, W)), ("accept_len", accept_len, (bs,)),
                         ("next_x0", next_x0, (bs,)), ("packed", packed, (bs, W + 2))):
        if t is not None:
            _need(t, torch.int32, name, shp)
    check(lib().gss_argmax_accept_noalloc(_ptr(logits), dt, logits.stride(1), bs, W, V, int(flags), _ptr(window),
                                          _ptr(target), _ptr(accept_len), _ptr(next_x0), _ptr(packed), _stream()),
          "gss_argmax_accept_noalloc")


def unmask_workspace_bytes(bs, W, V) -> int:
    n = ctypes.c_size_t(0)
    check(lib().gss_unmask_workspace_size(bs, W, V, ctypes.byref(n)), "gss_unmask_workspace_size")
    return n.value


def unmask_step(logits, block, workspace, *, mask_id: int, threshold: float, x1=None, conf=None, n_unmasked=None,
                n_left=None, seed=None):
    """One threshold-unmask step of the block-diffusion decode (gss_unmask_step). logits [bs, W, V] bf16 or fp32
    (uniform row stride, dense rows); block int32 [bs, W] (updated in place); optional outputs x1 int32 [bs, W],
    conf float32 [bs, W], n_unmasked / n_left / seed int32 [bs]."""
    bs, W, V = logits.shape
    if not logits.is_cuda or logits.stride(2) != 1 or logits.stride(0) != W * logits.stride(1):
        raise ValueError("logits must be a GPU tensor [bs, W, V] with dense rows and a uniform row stride")
    dt = {torch.bfloat16: 0, torch.float32: 1}.get(logits.dtype)
    if dt is None:
        raise ValueError("logits must be bf16 or fp32")
    _need(block, torch.int32, "block", (bs, W))
    for name, t, dtype, shp in (("x1", x1, torch.int32, (bs, W)), ("conf", conf, torch.float32, (bs, W)),
                                ("n_unmasked", n_unmasked, torch.int32, (bs,)), ("n_left", n_left, torch.int32, (bs,)),
                                ("seed", seed, torch.int32, (bs,))):
        if t is not None:
            _need(t, dtype, name, shp)
    if workspace.numel() * workspace.element_size() < unmask_workspace_bytes(bs, W, V):
        raise ValueError("unmask workspace too small")
    check(lib().gss_unmask_step(_ptr(logits), dt, logits.stride(1), bs, W, V, _ptr(block), int(mask_id),
                                float(threshold), _ptr(x1), _ptr(conf), _ptr(n_unmasked), _ptr(n_left), _ptr(seed),
                                _ptr(workspace), workspace.numel() * workspace.element_size(), _stream()),
          "gss_unmask_step")


def kv_commit(k_win, v_win, k_pages, v_pages, page_table, seq_lens, workspace, *, n_rows=None, n_add=0,
              slots=None):
    """k_win/v_win [n_layers, bs, W, Hkv, D]; k_pages [n_layers, n_pages, Hkv, 16, D]; v_pages
    [n_layers, n_pages, Hkv, D, 16]; seq_lens int32 [bs] (advanced in place); n_rows int32 [bs] or None;
    slots int32 [bs, W] or None."""
    nl, bs, W, Hkv, D = k_win.shape
    _need(k_win, torch.bfloat16, "k_win")
    _need(v_win, torch.bfloat16, "v_win", k_win.shape)
    _need(k_pages, torch.bfloat16, "k_pages")
    _need(v_pages, torch.bfloat16, "v_pages")
    if k_pages.shape[0] != nl or k_pages.shape[2:] != (Hkv, PAGE, D) or v_pages.shape[2:] != (Hkv, D, PAGE):
        raise ValueError("page tensors do not match the window tensors")
    _need(page_table, torch.int32, "page_table")
    _need(seq_lens, torch.int32, "seq_lens", (bs,))
    if n_rows is not None:
        _need(n_rows, torch.int32, "n_rows", (bs,))
    if slots is not None:
        _need(slots, torch.int32, "slots", (bs, W))
    wsb = workspace.numel() * workspace.element_size()
    check(lib().gss_kv_commit(_ptr(k_win), _ptr(v_win), bs * W * Hkv * D, _ptr(k_pages), _ptr(v_pages),
                              k_pages[0].numel(), _ptr(page_table), page_table.shape[1], _ptr(seq_lens),
                              _ptr(n_rows), int(n_add), _ptr(slots), bs, W, nl, Hkv, D, PAGE, _ptr(workspace), wsb,
                              _stream()), "gss_kv_commit")


def ss_commit(predict, accept_len, a0, req_pool_indices, seeds, seq_lens, loc, packed, free_slots, out, *, K: int,
              page: int = 1, budget=None, stop_ids=None, vocab=None, cut=None, n_free=None):
    """The serving round's commit bookkeeping (gss_ss_commit). predict int32 [>= bs*K]; accept_len int32 [bs];
    a0 int64 [bs] (any stride); req_pool_indices int64 [bs]; seeds int64 [pool]; seq_lens int64 [bs] (in place);
    loc int64 [bs*K]; packed int32 [bs, K+2]; free_slots int64 [bs*K]; out int64 [bs]. ``page``: the KV page size
    of the slots. The finish rule (optional, all three): budget / vocab int32 [bs], stop_ids int32 [bs, n_stop];
    cut int32 [bs] and n_free int32 [1] receive the cut index and the free-list length."""
    bs = accept_len.shape[0]
    _need(accept_len, torch.int32, "accept_len", (bs,))
    if predict.dtype != torch.int32 or not predict.is_contiguous() or predict.numel() < bs * K:
        raise ValueError("predict must be contiguous int32 with at least bs*K entries")
    if a0.dtype != torch.int64 or a0.dim() != 1 or a0.shape[0] != bs or not a0.is_cuda:
        raise ValueError("a0 must be a GPU int64 vector of length bs")
    _need(req_pool_indices, torch.int64, "req_pool_indices", (bs,))
    _need(seeds, torch.int64, "seeds")
    _need(seq_lens, torch.int64, "seq_lens", (bs,))
    _need(loc, torch.int64, "loc", (bs * K,))
    _need(packed, torch.int32, "packed", (bs, K + 2))
    _need(free_slots, torch.int64, "free_slots", (bs * K,))
    _need(out, torch.int64, "out", (bs,))
    rule = None
    if budget is not None or stop_ids is not None or vocab is not None:
        if budget is None or vocab is None or stop_ids is None:
            raise ValueError("the finish rule needs budget, stop_ids and vocab")
        _need(budget, torch.int32, "budget", (bs,))
        _need(vocab, torch.int32, "vocab", (bs,))
        _need(stop_ids, torch.int32, "stop_ids", (bs, stop_ids.shape[1]))
        rule = FinishRule(budget.data_ptr(), stop_ids.data_ptr() if stop_ids.numel() else 0, stop_ids.shape[1],
                          vocab.data_ptr())
    if cut is not None:
        _need(cut, torch.int32, "cut", (bs,))
    if n_free is not None:
        _need(n_free, torch.int32, "n_free", (1,))
    check(lib().gss_ss_commit(_ptr(predict), _ptr(accept_len), _ptr(a0), a0.stride(0), _ptr(req_pool_indices),
                              _ptr(seeds), _ptr(seq_lens), _ptr(loc), _ptr(packed), _ptr(free_slots), _ptr(out),
                              seeds.numel(), bs, K, int(page), None if rule is None else ctypes.byref(rule),
                              _ptr(cut), _ptr(n_free), _stream()), "gss_ss_commit")


def kv_meta(req_to_token, req_pool_indices, seq_lens, kv_indptr, kv_indices, *, extra: int):
    """Flattened page-size-1 KV indices of a batch (gss_kv_meta). req_to_token int32 [pool, ctx];
    req_pool_indices / seq_lens int64 [bs]; kv_indptr int32 [bs+1]; kv_indices int32 [capacity]."""
    bs = seq_lens.shape[0]
    _need(req_to_token, torch.int32, "req_to_token")
    if req_to_token.dim() != 2:
        raise ValueError("req_to_token must be 2-D")
    _need(req_pool_indices, torch.int64, "req_pool_indices", (bs,))
    _need(seq_lens, torch.int64, "seq_lens", (bs,))
    _need(kv_indptr, torch.int32, "kv_indptr", (bs + 1,))
    _need(kv_indices, torch.int32, "kv_indices")
    check(lib().gss_kv_meta(_ptr(req_to_token), req_to_token.shape[1], req_to_token.shape[0], _ptr(req_pool_indices),
                            _ptr(seq_lens), int(extra), _ptr(kv_indptr), _ptr(kv_indices), kv_indices.numel(), bs,
                            _stream()), "gss_kv_meta")


def log_append(ctr, pairs):
    """Row min(ctr, capacity - 1) of each log gets its source's contents, then ctr += 1 (gss_log_append).
    ctr int64 [1]; pairs: up to three (src int32, log int32 [capacity, *src.shape])."""
    _need(ctr, torch.int64, "ctr", (1,))
    if not 1 <= len(pairs) <= 3:
        raise ValueError("one to three logs")
    cap = pairs[0][1].shape[0]
    args = []
    for src, log in pairs:
        _need(src, torch.int32, "src")
        _need(log, torch.int32, "log", (cap,) + tuple(src.shape))
        args += [_ptr(src), _ptr(log), src.numel()]
    args += [None, None, 0] * (3 - len(pairs))
    check(lib().gss_log_append(_ptr(ctr), cap, *args, _stream()), "gss_log_append")


def rope_stage(qkv, seq_lens, inv_freq, q, k_win, v_win, *, pos_offset=0, pos_delta=None, rot_dim: int):
    """qkv [bs*W, (Hq+2Hkv)*D] bf16 (row stride qkv.stride(0)); q [bs, W, Hq, D]; k_win/v_win [bs, W, Hkv, D]."""
    bs, W, Hq, D = q.shape
    Hkv = k_win.shape[2]
    if qkv.stride(1) != 1 or qkv.shape[0] != bs * W or qkv.shape[1] < (Hq + 2 * Hkv) * D:
        raise ValueError("qkv shape")
    _need(seq_lens, torch.int32, "seq_lens", (bs,))
    _need(inv_freq, torch.float32, "inv_freq", (rot_dim // 2,))
    check(lib().gss_rope_stage(_ptr(qkv), qkv.stride(0), _ptr(seq_lens), _ptr(pos_delta), int(pos_offset),
                               _ptr(inv_freq), rot_dim, _ptr(q), _ptr(k_win), _ptr(v_win), bs, W, Hq, Hkv, D,
                               _stream()), "gss_rope_stage")


def rope_stage_mrope(qkv, positions, inv_freq, q, k_win, v_win, *, sections, rot_dim: int):
    """One sequence's rows with explicit M-RoPE positions int32 [rows, 3]; q [rows, Hq, D]; k_win/v_win
    [rows, Hkv, D]; ``sections`` = mrope_section (t, h, w) in rotary frequencies."""
    rows, Hq, D = q.shape
    Hkv = k_win.shape[1]
    if qkv.stride(1) != 1 or qkv.shape[0] != rows or qkv.shape[1] < (Hq + 2 * Hkv) * D:
        raise ValueError("qkv shape")
    _need(positions, torch.int32, "positions", (rows, 3))
    _need(inv_freq, torch.float32, "inv_freq", (rot_dim // 2,))
    check(lib().gss_rope_stage_mrope(_ptr(qkv), qkv.stride(0), _ptr(positions), int(sections[0]), int(sections[1]),
                                     _ptr(inv_freq), rot_dim, _ptr(q), _ptr(k_win), _ptr(v_win), rows, Hq, Hkv, D,
                                     _stream()), "gss_rope_stage_mrope")


def rmsnorm(x, w, out, eps):
    rows, H = x.shape
    check(lib().gss_rmsnorm(_ptr(x), _ptr(w), _ptr(out), rows, H, float(eps), _stream()), "gss_rmsnorm")


def embed_rmsnorm(table, ids, w, h, x, eps):
    """h = table[ids] (rows = ids.numel()), x = rmsnorm(h) * w; ids int32, contiguous."""
    V, H = table.shape
    _need(table, torch.bfloat16, "table")
    _need(ids, torch.int32, "ids")
    rows = ids.numel()
    _need(h, torch.bfloat16, "h", (rows, H))
    _need(x, torch.bfloat16, "x", (rows, H))
    check(lib().gss_embed_rmsnorm(_ptr(table), _ptr(ids), V, _ptr(w), _ptr(h), _ptr(x), rows, H, float(eps),
                                  _stream()), "gss_embed_rmsnorm")


def add_rmsnorm(a, w_post, h, w_next, x, eps):
    rows, H = h.shape
    check(lib().gss_add_rmsnorm(_ptr(a), _ptr(w_post), _ptr(h), _ptr(w_next), _ptr(x), rows, H, float(eps),
                                _stream()), "gss_add_rmsnorm")


def silu_mul(gu, out):
    rows, F = out.shape
    check(lib().gss_silu_mul(_ptr(gu), gu.stride(0), _ptr(out), rows, F, _stream()), "gss_silu_mul")


def _gemm_args(x, w):
    if w.dtype != torch.bfloat16 or not w.is_cuda or w.stride(1) != 1:
        raise ValueError("gemm weights must be a bf16 GPU tensor with a dense last dimension")
    if x is not None:
        if x.dtype != torch.bfloat16 or not x.is_cuda or x.stride(1) != 1:
            raise ValueError("gemm activations must be a bf16 GPU tensor with a dense last dimension")
        if x.shape[1] != w.shape[1]:
            raise ValueError(f"gemm inner dims differ: {tuple(x.shape)} x {tuple(w.shape)}^T")


def _prologue(pro, M, Kd):
    """pro = dict(h_in=..., w_next=..., eps=..., a=None, w_post=None, h_out=None, a_parts=None) -> (NormPrologue or
    None). ``a_parts`` (fp32 [n_parts, M, Kd], from gemm_parts) stands for a = bf16 of the parts' sum."""
    if pro is None:
        return None
    for k in ("h_in", "a", "h_out"):
        t = pro.get(k)
        if t is not None:
            _need(t, torch.bfloat16, f"prologue {k}", (M, Kd))
    for k in ("w_next", "w_post"):
        t = pro.get(k)
        if t is not None:
            _need(t, torch.bfloat16, f"prologue {k}", (Kd,))
    ap = pro.get("a_parts")
    if ap is not None:
        _need(ap, torch.float32, "prologue a_parts", (ap.shape[0], M, Kd))
    return NormPrologue(_ptr(pro.get("a")).value, _ptr(pro["h_in"]).value, _ptr(pro.get("h_out")).value,
                        _ptr(pro.get("w_post")).value, _ptr(pro["w_next"]).value, float(pro["eps"]), _ptr(ap).value,
                        0 if ap is None else ap.shape[0])


def _rows(x, pro):
    return (x.shape[0], x.stride(0)) if x is not None else (pro["h_in"].shape[0], 0)


def gemm_workspace_bytes(M, N, Kd) -> int:
    n = ctypes.c_size_t(0)
    check(lib().gss_gemm_workspace_size(M, N, Kd, ctypes.byref(n)), "gss_gemm_workspace_size")
    return n.value


_DEFAULT_WS = {}


def _gemm_ws(workspace, dev, M, N, Kd):
    """The caller's GEMM workspace, or (callers that do not keep one, e.g. tests) a zeroed per-device default that
    grows to the largest shape seen."""
    if workspace is not None:
        return workspace
    need = gemm_workspace_bytes(M, N, Kd)
    ws = _DEFAULT_WS.get(dev)
    if ws is None or ws.numel() < need:
        ws = torch.zeros(need, dtype=torch.uint8, device=dev)
        _DEFAULT_WS[dev] = ws
    return ws


def _epilogue(post, M, N):
    """post = dict(h=..., w_post=..., w_next=..., x=..., eps=...) -> NormEpilogue or None."""
    if post is None:
        return None
    for k in ("h", "x"):
        _need(post[k], torch.bfloat16, f"epilogue {k}", (M, N))
    for k in ("w_post", "w_next"):
        _need(post[k], torch.bfloat16, f"epilogue {k}", (N,))
    return NormEpilogue(_ptr(post["w_post"]).value, _ptr(post["h"]).value, _ptr(post["w_next"]).value,
                        _ptr(post["x"]).value, float(post["eps"]))


def gemm(x, w, y, pro=None, post=None, workspace=None):
    """y[M, N] = x[M, Kd] @ w[N, Kd]^T (bf16 or fp32 y), M <= 64, batch invariant. With ``pro`` (a dict of the
    gss_norm_prologue fields) x is rmsnorm(h_in + rmsnorm(a) * w_post) * w_next, built inside the kernel; with
    ``post`` (gss_norm_epilogue fields) the kernel finishes with h += rmsnorm(y) * w_post, x = rmsnorm(h) * w_next."""
    _gemm_args(x, w)
    Kd, N = w.shape[1], w.shape[0]
    M, ldx = _rows(x, pro)
    if y.shape[0] != M or y.shape[1] < N or y.stride(1) != 1:
        raise ValueError("gemm output shape")
    dt = {torch.bfloat16: 0, torch.float32: 1}[y.dtype]
    pr = _prologue(pro, M, Kd)
    po = _epilogue(post, M, N)
    ws = _gemm_ws(workspace, w.device, M, N, Kd)
    check(lib().gss_gemm(_ptr(x), ldx, None if pr is None else ctypes.byref(pr), _ptr(w), w.stride(0), _ptr(y),
                         y.stride(0), M, N, Kd, dt, None if po is None else ctypes.byref(po), _ptr(ws),
                         ws.numel(), _stream()), "gss_gemm")


def gemm_parts_count(N, Kd) -> int:
    n = ctypes.c_int(0)
    check(lib().gss_gemm_parts_count(N, Kd, ctypes.byref(n)), "gss_gemm_parts_count")
    return n.value


def gemm_parts(x, w, parts):
    """parts[s, :M, :N] (fp32, [n_parts, M, N] contiguous, n_parts = gemm_parts_count(N, Kd)): the k splits'
    partial sums of x @ w^T; y = bf16(parts.sum(0) in part order)."""
    _gemm_args(x, w)
    Kd, N = w.shape[1], w.shape[0]
    M = x.shape[0]
    _need(parts, torch.float32, "parts", (gemm_parts_count(N, Kd), M, N))
    check(lib().gss_gemm_parts(_ptr(x), x.stride(0), _ptr(w), w.stride(0), _ptr(parts), M, N, Kd, _stream()),
          "gss_gemm_parts")


PENALIZERS = {"repetition": 1, "presence": 2, "frequency": 3, "min_new_tokens": 4}
FILTERS = {"none": 0, "joint": 1, "torch": 2, "flashinfer_min_p": 3}


def penalize_rows(logits, cand, state, order):
    """In place on fp32 logits [bs*K, V] (dense rows): AR's penalties for every verify row (gss_penalize_rows).
    cand int32 [bs, K]; state: dict of GPU tensors rep_cum/pres_cum/freq_cum/stop_pen/logit_bias fp32 [bs, V],
    rep_pen/pres_pen/freq_pen fp32 [bs], len_out/min_new int32 [bs] (what ``order`` uses); order: penalizer names
    in the orchestrator's order."""
    bs, K = cand.shape
    V = logits.shape[1]
    _need(cand, torch.int32, "cand")
    if logits.dtype != torch.float32 or not logits.is_cuda or logits.stride(1) != 1 or logits.shape[0] != bs * K:
        raise ValueError("logits must be fp32 [bs*K, V] on the GPU with dense rows")
    shapes = dict(rep_cum=(bs, V), pres_cum=(bs, V), freq_cum=(bs, V), stop_pen=(bs, V), logit_bias=(bs, V),
                  rep_pen=(bs,), pres_pen=(bs,), freq_pen=(bs,), len_out=(bs,), min_new=(bs,))
    for k, t in state.items():
        if t is not None:
            _need(t, torch.int32 if k in ("len_out", "min_new") else torch.float32, k, shapes[k])
    pen = Penalties()
    pen.n_order = len(order)
    for i, name in enumerate(order):
        pen.order[i] = PENALIZERS[name]
    for k in shapes:
        setattr(pen, k, _ptr(state.get(k)).value)
    check(lib().gss_penalize_rows(_ptr(logits), logits.stride(0), bs, K, V, _ptr(cand), ctypes.byref(pen),
                                  _stream()), "gss_penalize_rows")


def apply_vocab_mask(logits, mask):
    """In place on fp32 logit rows [rows, V]: -inf where the packed int32 grammar mask [rows, ceil(V/32)] has the
    token's bit clear (gss_apply_vocab_mask)."""
    rows, V = logits.shape
    _need(mask, torch.int32, "mask")
    if logits.dtype != torch.float32 or logits.stride(1) != 1:
        raise ValueError("logits must be fp32 rows")
    if mask.shape[0] != rows or mask.shape[1] < (V + 31) // 32 or mask.stride(1) != 1:
        raise ValueError("mask shape")
    check(lib().gss_apply_vocab_mask(_ptr(logits), logits.stride(0), rows, V, _ptr(mask), mask.stride(0), _stream()),
          "gss_apply_vocab_mask")


def sample_workspace_bytes(bs, K) -> int:
    n = ctypes.c_size_t(0)
    check(lib().gss_sample_workspace_size(bs, K, ctypes.byref(n)), "gss_sample_workspace_size")
    return n.value


def sample_rows(logits, bs, K, *, temperature, filter="none", top_k=None, top_p=None, min_p=None, cand=None,
                coins=None, uniforms, sampled, target=None, accept_len=None, next_x0=None, packed=None,
                workspace=None):
    """gss_sample_rows on fp32 logits rows (row b*K + r at logits[b*K + r], any row stride): sample mode (cand
    None: uniforms [bs, K]) or verify mode (cand int32 [bs, K], coins fp32 [bs, K], uniforms [bs])."""
    if logits.dtype != torch.float32 or not logits.is_cuda or logits.stride(-1) != 1:
        raise ValueError("logits must be fp32 on the GPU with dense rows")
    V = logits.shape[-1]
    ld = logits.stride(-2) if logits.dim() >= 2 else V
    for name, t, dt, shp in (("temperature", temperature, torch.float32, (bs,)), ("top_k", top_k, torch.int32, (bs,)),
                             ("top_p", top_p, torch.float32, (bs,)), ("min_p", min_p, torch.float32, (bs,)),
                             ("cand", cand, torch.int32, (bs, K)), ("coins", coins, torch.float32, (bs, K)),
                             ("uniforms", uniforms, torch.float32, (bs,) if cand is not None else (bs, K)),
                             ("sampled", sampled, torch.int32, (bs, K)), ("target", target, torch.int32, (bs, K)),
                             ("accept_len", accept_len, torch.int32, (bs,)), ("next_x0", next_x0, torch.int32, (bs,)),
                             ("packed", packed, torch.int32, (bs, K + 2))):
        if t is not None:
            _need(t, dt, name, shp)
    wsb = 0 if workspace is None else workspace.numel() * workspace.element_size()
    check(lib().gss_sample_rows(_ptr(logits), ld, bs, K, V, FILTERS[filter], _ptr(temperature), _ptr(top_k),
                                _ptr(top_p), _ptr(min_p), _ptr(cand), _ptr(coins), _ptr(uniforms), _ptr(sampled),
                                _ptr(target), _ptr(accept_len), _ptr(next_x0), _ptr(packed), _ptr(workspace), wsb,
                                _stream()), "gss_sample_rows")


def add_rmsnorm_parts(parts, w_post, h, w_next, x, eps):
    """gss_add_rmsnorm with a = bf16 of the fp32 parts' sum (parts [n_parts, rows, H])."""
    rows, H = h.shape
    _need(parts, torch.float32, "parts", (parts.shape[0], rows, H))
    check(lib().gss_add_rmsnorm_parts(_ptr(parts), parts.shape[0], _ptr(w_post), _ptr(h), _ptr(w_next), _ptr(x),
                                      rows, H, float(eps), _stream()), "gss_add_rmsnorm_parts")


def gemm_swiglu(x, w_gu_il, act, pro=None, workspace=None):
    """act[M, F] = up * silu(gate) of x @ w_gu_il^T, w_gu_il [2F, Kd] with gate/up rows interleaved."""
    _gemm_args(x, w_gu_il)
    Kd, F = w_gu_il.shape[1], w_gu_il.shape[0] // 2
    M, ldx = _rows(x, pro)
    _need(act, torch.bfloat16, "act", (M, F))
    pr = _prologue(pro, M, Kd)
    ws = _gemm_ws(workspace, w_gu_il.device, M, 2 * F, Kd)
    check(lib().gss_gemm_swiglu(_ptr(x), ldx, None if pr is None else ctypes.byref(pr), _ptr(w_gu_il),
                                w_gu_il.stride(0), _ptr(act), M, F, Kd, _ptr(ws), ws.numel(), _stream()),
          "gss_gemm_swiglu")


def gemm_rope_stage(x, w_qkv, seq_lens, inv_freq, q, k_win, v_win, *, rot_dim, pos_delta=None, pro=None,
                    workspace=None):
    """q|k|v projection with RoPE and window staging fused: q [bs, W, Hq, D], k_win/v_win [bs, W, Hkv, D]."""
    _gemm_args(x, w_qkv)
    bs, W, Hq, D = q.shape
    Hkv = k_win.shape[2]
    Kd = w_qkv.shape[1]
    M, ldx = _rows(x, pro)
    if M != bs * W or w_qkv.shape[0] != (Hq + 2 * Hkv) * D:
        raise ValueError("gemm_rope_stage shapes")
    _need(seq_lens, torch.int32, "seq_lens", (bs,))
    _need(q, torch.bfloat16, "q")
    _need(k_win, torch.bfloat16, "k_win", (bs, W, Hkv, D))
    _need(v_win, torch.bfloat16, "v_win", (bs, W, Hkv, D))
    pr = _prologue(pro, M, Kd)
    ws = _gemm_ws(workspace, w_qkv.device, M, w_qkv.shape[0], Kd)
    check(lib().gss_gemm_rope_stage(_ptr(x), ldx, None if pr is None else ctypes.byref(pr), _ptr(w_qkv),
                                    w_qkv.stride(0), _ptr(seq_lens), _ptr(pos_delta), _ptr(inv_freq), rot_dim,
                                    _ptr(q), _ptr(k_win), _ptr(v_win), bs, W, Hq, Hkv, D, Kd, _ptr(ws), ws.numel(),
                                    _stream()),
          "gss_gemm_rope_stage")
