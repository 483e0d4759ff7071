"""CPU oracle for GravityOCR's self-speculative draft/verify/commit round.

TEST INFRASTRUCTURE ONLY. Only ``tests/``, ``__graft_entry__.smoke()`` and ``bench.py``'s CPU-baseline leg may
import this package, and only as the checker (or, for the baseline, as the CPU path that is timed next to the GPU
one). The product path (``gravityocr_amd``) never imports it and fails loudly when its HIP library is missing.

Each function restates the reference algorithm it names (file:line in the reference tree). Integer work (argmax,
accept, commit packing, finish rules, slot indices) is numpy / plain Python; floating-point work (masked attention,
the GLM decoder layer) is torch fp32 on the CPU.

Pinning (what each function is checked against, in ``tests/``):
  argmax_first        numpy/torch argmax contract + brute force on tiny rows (tests/test_oracle_integer.py)
  accept_chain        brute-force tree walk of the published verify_tree_greedy algorithm on random chains
  ss_commit           the reference's own post-commit invariants (seeds == predict[acc], free list == slots past acc,
                      seq_lens += acc + 1), checked independently per row
  cut_index_loop      the per-token finish loop the reference says its closed form is tested against
  masked_attention    torch SDPA with an explicit boolean mask; single-key / uniform-score closed forms
  decoder layer       transformers' GlmOcrTextDecoderLayer (container copy, third party) on the same weights
  natcache / fulldraft rounds   golden traces written by importing the reference's generate_speculative_natcache
                      (tests/golden/make_golden.py) + AR-equivalence (committed ids == greedy AR ids)
  block diffusion     golden ids / commit traces / commit details written by importing the reference's
                      generate_cached and generate_cached_batched (tests/golden/make_golden_diffusion.py); the
                      unmask rule against a brute-force fp64 reading (tests/test_oracle_diffusion.py)
  sampled verify      top-k / top-p / min-p filters against their definitions by brute force (ties included); the
                      in-block penalties against AR decode simulated token by token; speculative sampling against
                      the identity P(first committed token = t) = p_0(t) over a coin x uniform grid
                      (tests/test_oracle_sampling.py)
"""
