"""Cached block-diffusion decode (threshold unmasking) on the MI355X kernels: the ``generate_cached`` /
``generate_cached_batched`` samplers of the reference (src/fast_sampling.py:105-258,
src/fast_sampling_batched.py:95-234) over a GssEngine.

Per block of ``bd`` positions, for ``bs`` sequences in engine slots 0..bs-1 (each with its own committed length, so
ragged prompts need no padding):
    block = [seed | MASK x (bd-1)]
    probe step (until no row has a masked position):
        forward of the block against the frozen cache, all block rows bidirectional (n_causal = 0; nothing is
        committed: the block's K/V stays in the staging window)  ->  gss_unmask_step (shifted argmax, softmax
        confidence, threshold rule, block updated on the device)
    commit: forward of the clean block (bidirectional, or token-causal), gss_unmask_step for the next seed (the
        last row's greedy id), gss_kv_commit of all bd rows; the block is copied out and reset to the next seed.
The probe step and the commit are each captured once as a HIP graph and replayed; the host reads back, per step,
only the per-row counts of masked positions left (the loop condition), and per block the committed ids and seeds.
"""
from typing import Callable, List, Optional

import torch

from . import kernels as K
from .engine import GssEngine


class BlockDiffusionDecoder:
    """Block-diffusion decode state of ``bs`` sequences (engine slots 0..bs-1), device resident."""

    def __init__(self, eng: GssEngine, bd: int, mask_id: int, bs: int, threshold: float, commit_causal: bool = False):
        if bd < 1:
            raise ValueError("bd must be >= 1")
        self.eng, self.bd, self.mask_id, self.bs = eng, bd, mask_id, bs
        self.threshold, self.commit_causal = float(threshold), commit_causal
        dev = eng.device
        i32 = dict(dtype=torch.int32, device=dev)
        self.b = eng.bufs(bs, bd)
        self.block = torch.full((bs, bd), mask_id, **i32)
        self.before = torch.zeros(bs, bd, **i32)             # the block before the last probe step
        self.committed = torch.zeros(bs, bd, **i32)
        self.x1 = torch.zeros(bs, bd, **i32)
        self.conf = torch.zeros(bs, bd, dtype=torch.float32, device=dev)
        self.n_unmasked = torch.zeros(bs, **i32)
        self.n_left = torch.zeros(bs, **i32)
        self.seed = torch.zeros(bs, **i32)
        self.pos_delta = torch.zeros(bs, **i32)
        self.ws = torch.zeros(K.unmask_workspace_bytes(bs, bd, eng.cfg.vocab), dtype=torch.uint8, device=dev)
        self.g_step: Optional[torch.cuda.CUDAGraph] = None
        self.g_commit: Optional[torch.cuda.CUDAGraph] = None
        self._pin_left = torch.zeros(bs, dtype=torch.int32).pin_memory()
        self._pin_block = torch.zeros(bs, bd, dtype=torch.int32).pin_memory()
        self._pin_seed = torch.zeros(bs, dtype=torch.int32).pin_memory()
        self._ev = torch.cuda.Event()

    # ---- device work ------------------------------------------------------------------------------------------
    def _step(self):
        self.before.copy_(self.block)
        lg = self.eng.forward(self.b, ids=self.block, n_causal=0, pos_delta=self.pos_delta)
        K.unmask_step(lg, self.block, self.ws, mask_id=self.mask_id, threshold=self.threshold, x1=self.x1,
                      conf=self.conf, n_unmasked=self.n_unmasked, n_left=self.n_left)

    def _commit(self):
        lg = self.eng.forward(self.b, ids=self.block, n_causal=None if self.commit_causal else 0,
                              pos_delta=self.pos_delta)
        K.unmask_step(lg, self.block, self.ws, mask_id=self.mask_id, threshold=self.threshold, seed=self.seed)
        self.eng.commit(self.b, n_add=self.bd)                 # all bd rows: seq_lens += bd
        self.committed.copy_(self.block)
        self._reset_block()

    def _reset_block(self):
        self.block.fill_(self.mask_id)
        self.block[:, 0].copy_(self.seed)

    def _replay(self, which: str):
        """Run the probe step or the commit: eagerly the first time, then captured once and replayed."""
        g = self.g_step if which == "step" else self.g_commit
        if g is not None:
            g.replay()
            return
        fn = self._step if which == "step" else self._commit
        fn()
        # capture records the kernels without running them, so the state is unchanged by it
        g = torch.cuda.CUDAGraph()
        torch.cuda.synchronize(self.eng.device)
        with torch.cuda.graph(g):
            fn()
        if which == "step":
            self.g_step = g
        else:
            self.g_commit = g

    # ---- host loop --------------------------------------------------------------------------------------------
    def start(self, seeds: torch.Tensor, pos_delta: Optional[torch.Tensor] = None):
        """Begin with the first block's seeds (int [bs]); the position of cache index i of row b is
        i + pos_delta[b]. The slots' committed lengths (engine seq_lens) must hold the prompts already."""
        self.seed.copy_(seeds.to(device=self.seed.device, dtype=torch.int32))
        if pos_delta is None:
            self.pos_delta.zero_()
        else:
            self.pos_delta.copy_(pos_delta.to(device=self.pos_delta.device, dtype=torch.int32))
        self._reset_block()

    def decode_block(self, seeds: List[int], on_step: Optional[Callable[[], None]] = None):
        """Unmask the current block of every row and commit it. ``seeds`` are the host copies of the block seeds
        (to know whether any position is masked before the first step). ``on_step`` runs after every probe step,
        once its outputs (before, block, x1, conf, n_unmasked, n_left) are complete on the device.
        Returns (committed ids [bs][bd], next seeds [bs], probe steps taken).

        Every step unmasks at least one masked position per row that has one, so bd steps suffice unless the model
        predicts the mask id itself at a masked position (the position stays masked); the reference's loop would then
        not end, and this raises instead."""
        left = [self.bd - 1 + (1 if s == self.mask_id else 0) for s in seeds]
        n_steps = 0
        stream = torch.cuda.current_stream(self.eng.device)
        while any(n > 0 for n in left):
            if n_steps > self.bd:
                raise RuntimeError("block-diffusion step limit: the model keeps predicting the mask id at a masked "
                                   "position, so the unmask loop cannot finish")
            self._replay("step")
            n_steps += 1
            self._pin_left.copy_(self.n_left, non_blocking=True)
            self._ev.record(stream)
            self._ev.synchronize()
            if on_step is not None:
                on_step()
            left = self._pin_left.tolist()
        self._replay("commit")
        self._pin_block.copy_(self.committed, non_blocking=True)
        self._pin_seed.copy_(self.seed, non_blocking=True)
        self._ev.record(stream)
        self._ev.synchronize()
        return self._pin_block.tolist(), self._pin_seed.tolist(), n_steps
