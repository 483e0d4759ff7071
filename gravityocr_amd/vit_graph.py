"""Exact-M HIP graphs of the GLM-OCR vision tower (the ViT in front of the prefill).

An eager ViT call is hundreds of small launches plus host work per block, so for one crop its host time is many
times its GPU time (patches/sglang/python/sglang/srt/multimodal/glm_vit_graph_runner.py, header). ``VitGraphRunner``
wraps a transformers ``GlmOcrVisionModel`` (the model's own modules and weights, unchanged) and replays one HIP
graph per patch count M for calls with a single image of one temporal patch (grid (1, h, w), M = h * w <= max_m):

  * the graph holds the tower body: patch embedding, the blocks (attention over the one image: cu_seqlens [0, M]
    kept on the host, so the blocks' per-image split needs no device read), the post norm, the spatial-merge
    downsample and the merger;
  * the only (h, w)-dependent inputs, the rotary cos / sin of the patch positions, are computed eagerly by the
    tower's own rotary module and copied into the graph's static inputs with the pixel rows, so one graph per M
    serves every grid of that size;
  * every M is checked right after its capture against the eager tower on the call's own input, or that M stays
    eager. The eager tower on this stack is not bit-reproducible from call to call (repeated calls on one input
    differ in the last bits of some outputs, about 6e-5 on outputs of magnitude 1e-2), so the check bounds the
    difference at CHECK_TOL of the output's largest magnitude: a replay that read a wrong input (another grid's
    cos / sin, stale pixels) differs by the output's own size;
  * all graphs share one memory pool; outputs are cloned after the replay (a later replay reuses the pool).

Everything else (several images, t > 1, M > max_m, other keyword arguments) runs the tower eagerly. Attributes of
the tower (dtype, config, spatial_merge_size, ...) are reachable through the runner, so it can stand in for
``model.visual`` (``enable_vit_graphs``).
"""
from typing import Dict, Optional

import torch

try:
    from transformers.modeling_outputs import BaseModelOutputWithPooling
except ImportError:  # pragma: no cover - transformers is part of the image
    BaseModelOutputWithPooling = None


CHECK_TOL = 1e-2


def close(a: torch.Tensor, b: torch.Tensor, tol: float = CHECK_TOL) -> bool:
    """max |a - b| <= tol * max |b| (exact equality passes for any tol)"""
    if a.shape != b.shape:
        return False
    d = (a.float() - b.float()).abs().max().item()
    return d <= tol * b.float().abs().max().item()


class VitGraphRunner(torch.nn.Module):
    def __init__(self, visual: torch.nn.Module, max_m: int = 2048, check: bool = True):
        super().__init__()
        self.visual = visual
        self.max_m = int(max_m) // 4 * 4
        self.check = check
        self._graphs: Dict[int, tuple] = {}
        self._dropped = set()
        self._pool = None
        self.n_calls = self.n_replays = 0

    def __getattr__(self, name):
        try:
            return super().__getattr__(name)
        except AttributeError:
            return getattr(self._modules["visual"], name)

    # ---- pieces --------------------------------------------------------------------------------------------------
    def _cos_sin(self, grid_thw: torch.Tensor):
        """Rotary cos / sin [M, head_dim] of the patch positions of the grid, by the tower's own position-id helper
        and rotary module (the eager forward's first steps)."""
        from transformers.models.glm_ocr import modeling_glm_ocr as m
        v = self.visual
        pos = m.get_vision_position_ids(grid_thw, v.spatial_merge_size)
        rot = v.rotary_pos_emb(pos)
        emb = torch.cat((rot, rot), dim=-1)
        return emb.cos(), emb.sin()

    def _body(self, x, cos, sin, M: int):
        v = self.visual
        cu = torch.tensor([0, M], dtype=torch.int32)  # host: the blocks split by it without a device read
        h = v.patch_embed(x)
        for blk in v.blocks:
            h = blk(h, cu_seqlens=cu, max_seqlen=M, position_embeddings=(cos, sin))
        h = v.post_layernorm(h)
        s = v.spatial_merge_size
        h = h.view(-1, s, s, h.shape[-1]).permute(0, 3, 1, 2)
        h = v.downsample(h).view(-1, v.config.out_hidden_size)
        return h, v.merger(h)

    def _eligible(self, hidden_states, grid_thw, kwargs) -> Optional[int]:
        if grid_thw is None or grid_thw.dim() != 2 or grid_thw.shape[0] != 1 or not hidden_states.is_cuda:
            return None
        if any(k not in ("return_dict",) for k in kwargs):
            return None
        t, h, w = (int(x) for x in grid_thw[0].tolist())
        M = h * w
        if t != 1 or M > self.max_m or M != hidden_states.shape[0] or M in self._dropped:
            return None
        return M

    def _capture(self, M: int, x, cos, sin):
        sx, sc, ss = x.clone(), cos.clone(), sin.clone()
        side = torch.cuda.Stream()
        side.wait_stream(torch.cuda.current_stream())
        with torch.cuda.stream(side), torch.no_grad():
            for _ in range(2):
                self._body(sx, sc, ss, M)
        torch.cuda.current_stream().wait_stream(side)
        if self._pool is None:
            self._pool = torch.cuda.graph_pool_handle()
        g = torch.cuda.CUDAGraph()
        with torch.no_grad(), torch.cuda.graph(g, pool=self._pool):
            out = self._body(sx, sc, ss, M)
        return g, sx, sc, ss, out

    def _wrap(self, last, pooled):
        if BaseModelOutputWithPooling is None:
            return pooled
        return BaseModelOutputWithPooling(last_hidden_state=last, pooler_output=pooled)

    # ---- the call ------------------------------------------------------------------------------------------------
    def forward(self, hidden_states, grid_thw=None, **kwargs):
        self.n_calls += 1
        M = self._eligible(hidden_states, grid_thw, kwargs)
        if M is None:
            return self.visual(hidden_states, grid_thw=grid_thw, **kwargs)
        with torch.no_grad():
            cos, sin = self._cos_sin(grid_thw)
            x = hidden_states.to(next(self.visual.parameters()).dtype)
            entry = self._graphs.get(M)
            fresh = entry is None
            if fresh:
                entry = self._capture(M, x, cos, sin)
                self._graphs[M] = entry
            g, sx, sc, ss, out = entry
            sx.copy_(x)
            sc.copy_(cos)
            ss.copy_(sin)
            g.replay()
            last, pooled = out[0].clone(), out[1].clone()
            if fresh and self.check:
                ref = self.visual(hidden_states, grid_thw=grid_thw, return_dict=True)
                if not (close(pooled, ref.pooler_output) and close(last, ref.last_hidden_state)):
                    del self._graphs[M]
                    self._dropped.add(M)
                    return ref
        self.n_replays += 1
        return self._wrap(last, pooled)

    @property
    def graph_sizes(self):
        return sorted(self._graphs)


def enable_vit_graphs(model, max_m: int = 2048, check: bool = True) -> VitGraphRunner:
    """Route a GLM-OCR model's vision tower through a VitGraphRunner (model.mm_model.visual, or model.visual).
    Returns the runner; calling it again returns the installed one."""
    holder = getattr(model, "mm_model", model)
    visual = holder.visual
    if isinstance(visual, VitGraphRunner):
        return visual
    runner = VitGraphRunner(visual, max_m=max_m, check=check)
    holder.visual = runner
    return runner
