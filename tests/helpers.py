"""Test-side helpers: paged-cache construction from contiguous K/V (a seeded shuffled page order), and tolerances."""
import numpy as np
import torch

PAGE = 16

# attention outputs: max |err| <= ATTN_REL * max |ref| (bf16 output, bf16 P operand)
ATTN_REL = 1e-2
# logits of a bf16 forward vs the fp32 oracle
LOGIT_ABS = 2e-2


def shuffled_page_table(bs, pages_per_seq, n_pages_total, seed):
    """Disjoint pages for every sequence, drawn from a seeded permutation of the pool."""
    g = np.random.default_rng(seed)
    perm = g.permutation(n_pages_total)[: bs * pages_per_seq]
    return perm.reshape(bs, pages_per_seq).astype(np.int32)


def to_pages(k, v, page_table_row, k_pages, v_pages):
    """Write contiguous k/v [L, Hkv, D] (torch, any dtype) into k_pages [n_pages, Hkv, 16, D] and the token-minor
    v_pages [n_pages, Hkv, D, 16] at the positions 0..L-1 of one sequence."""
    L = k.shape[0]
    for pos0 in range(0, L, PAGE):
        n = min(PAGE, L - pos0)
        pg = int(page_table_row[pos0 // PAGE])
        k_pages[pg, :, :n, :] = k[pos0:pos0 + n].transpose(0, 1).to(k_pages.dtype)
        v_pages[pg, :, :, :n] = v[pos0:pos0 + n].permute(1, 2, 0).to(v_pages.dtype)


def rel_err(out, ref):
    out = out.double().cpu()
    ref = ref.double().cpu()
    return float((out - ref).abs().max() / ref.abs().max().clamp_min(1e-30))
