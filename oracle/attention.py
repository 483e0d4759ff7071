"""Masked GQA attention and the draft / verify masks of the self-spec round (CPU, torch fp64/fp32).

Test infrastructure only (see ``oracle/__init__.py``).

Masks (closed forms; a query row sees the committed prefix plus part of its own window):
  draft   (src/fast_sampling.py:508-510 ``draft_mask``; patches/sglang/.../selfspec_fast_attn.py:9-13):
          the first ``n_causal`` window rows are causal (row w sees window rows 0..w); every later row sees the whole
          window. natcache round 0 has n_causal = 0, rounds >= 1 and the serving draft have n_causal = 1.
  verify  (src/fast_sampling.py:512-514 ``mask_causal``; selfspec_fast_attn.py:9 CAUSAL bottom-right aligned):
          row w sees window rows 0..w.
  full    (src/fast_sampling.py:199-200, src/fast_sampling_batched.py:193-194): every row sees the whole window.
"""
import numpy as np
import torch


def window_mask(L_pre: int, W: int, n_causal: int) -> np.ndarray:
    """[W, L_pre + W] bool: keys 0..L_pre-1 are the prefix, keys L_pre.. the window. Rows < n_causal are causal,
    rows >= n_causal see the whole window. n_causal = W is the verify mask, 0 the all-bidirectional block."""
    m = np.zeros((W, L_pre + W), dtype=bool)
    m[:, :L_pre] = True
    for w in range(W):
        if w < n_causal:
            m[w, L_pre: L_pre + w + 1] = True
        else:
            m[w, L_pre:] = True
    return m


def masked_attention(q: torch.Tensor, k: torch.Tensor, v: torch.Tensor, mask: np.ndarray, scale: float,
                     dtype=torch.float64) -> torch.Tensor:
    """softmax(q k^T * scale + mask) v for GQA.

    q [W, Hq, D], k/v [T, Hkv, D], mask [W, T] bool (True = visible). Query head h reads KV head h // (Hq/Hkv)
    (transformers repeat_kv, container modeling_glm_ocr.py:91-100). Returns [W, Hq, D] in ``dtype``.
    """
    W, Hq, D = q.shape
    T, Hkv, _ = k.shape
    G = Hq // Hkv
    qd = q.to(dtype)
    kd = k.to(dtype).repeat_interleave(G, dim=1)           # [T, Hq, D]
    vd = v.to(dtype).repeat_interleave(G, dim=1)
    s = torch.einsum("whd,thd->hwt", qd, kd) * scale       # [Hq, W, T]
    mt = torch.from_numpy(mask)[None]
    s = s.masked_fill(~mt, float("-inf"))
    p = torch.softmax(s, dim=-1)
    return torch.einsum("hwt,thd->whd", p, vd)


def gather_pages(pages: torch.Tensor, page_table_row: np.ndarray, L: int, page_size: int = 16,
                 v_transposed: bool = False) -> torch.Tensor:
    """Read the first L positions of one sequence out of a paged cache.

    pages: [n_pages, Hkv, page, D] (K layout), or [n_pages, Hkv, D, page] with ``v_transposed`` (V layout).
    Returns [L, Hkv, D]."""
    n = (L + page_size - 1) // page_size
    idx = torch.as_tensor(np.asarray(page_table_row[:n], dtype=np.int64))
    blk = pages.index_select(0, idx)                        # [n, Hkv, page, D] or [n, Hkv, D, page]
    if v_transposed:
        blk = blk.transpose(2, 3)
    return blk.permute(0, 2, 1, 3).reshape(n * page_size, pages.shape[1], -1)[:L]


def paged_window_attention(q, k_pages, v_pages, page_table_row, L_pre, k_win, v_win, n_causal, scale,
                           page_size=16, v_transposed=True, dtype=torch.float64):
    """Attention of W window rows over (prefix from pages) ++ (window K/V), with ``window_mask``.

    q [W, Hq, D]; k_win / v_win [W, Hkv, D]. This is the contract of the draft (n_causal < W) and verify
    (n_causal = W) kernels."""
    W = q.shape[0]
    kp = gather_pages(k_pages, page_table_row, L_pre, page_size)
    vp = gather_pages(v_pages, page_table_row, L_pre, page_size, v_transposed=v_transposed)
    k = torch.cat([kp.to(k_win.dtype), k_win], 0)
    v = torch.cat([vp.to(v_win.dtype), v_win], 0)
    return masked_attention(q, k, v, window_mask(L_pre, W, n_causal), scale, dtype=dtype)
