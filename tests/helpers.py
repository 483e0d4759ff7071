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


class PositionGrammar:
    """A grammar object with the serving stack's surface (allocate_vocab_mask, fill_vocab_mask, accept_token,
    rollback, is_terminated) over a rule that depends on the accepted tokens: after n accepted tokens whose last is
    x, token t is allowed iff (t + n + x) % 3 != 0. Never terminates."""

    def __init__(self, V, tokens=()):
        self.V, self.acc = V, list(tokens)

    def allowed(self, t):
        last = self.acc[-1] if self.acc else 0
        return (t + len(self.acc) + last) % 3 != 0

    def allocate_vocab_mask(self, vocab_size, batch_size, device):
        import torch
        return torch.zeros(batch_size, (vocab_size + 31) // 32, dtype=torch.int32, device=device)

    def fill_vocab_mask(self, mask, idx):
        import numpy as np
        import torch
        bits = np.array([self.allowed(t) for t in range(self.V)] + [False] * (-self.V % 32), dtype=np.uint64)
        words = (bits.reshape(-1, 32) << np.arange(32, dtype=np.uint64)).sum(1).astype(np.uint32).view(np.int32)
        mask[idx] = torch.from_numpy(words)

    def accept_token(self, t):
        if not self.allowed(t):
            raise ValueError(f"token {t} not allowed")
        self.acc.append(int(t))

    def rollback(self, k):
        del self.acc[len(self.acc) - k:]

    def is_terminated(self):
        return False
