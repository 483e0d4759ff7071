"""The vision tower's exact-M HIP graphs (gravityocr_amd/vit_graph.py; glm_vit_graph_runner.py in the reference) on
a small random transformers GlmOcrVisionModel in bf16: replays equal the eager tower to within its own call-to-call
spread (1e-2 of the output's magnitude; a replay with another grid's positions is far outside it), for two grids
of the same patch count (the rotary cos / sin are graph inputs) and for a second size; calls the graphs do not
cover (two images, more patches than max_m) run eagerly and equal the eager tower too."""
import time

import pytest
import torch

pytestmark = pytest.mark.gpu


def _tower(cuda):
    from transformers.models.glm_ocr.configuration_glm_ocr import GlmOcrVisionConfig
    from transformers.models.glm_ocr.modeling_glm_ocr import GlmOcrVisionModel
    cfg = GlmOcrVisionConfig(depth=4, hidden_size=256, num_heads=4, intermediate_size=512, out_hidden_size=128,
                             patch_size=14, temporal_patch_size=2, spatial_merge_size=2)
    torch.manual_seed(0)
    return GlmOcrVisionModel(cfg).to(device=cuda, dtype=torch.bfloat16).eval()


def _eager(v, x, grid):
    with torch.no_grad():
        return v(x, grid_thw=grid, return_dict=True)


def _check(out, ref, what):
    """within the eager tower's own call-to-call spread: 1e-2 of the output's magnitude (a replay on a wrong input,
    e.g. another grid's cos / sin, is off by the output's own size); prints how many entries are bit-equal"""
    from gravityocr_amd.vit_graph import close
    for a, b, name in ((out.pooler_output, ref.pooler_output, "pooled"), (out.last_hidden_state, ref.last_hidden_state,
                                                                         "hidden")):
        eq = (a == b).float().mean().item()
        d = (a.float() - b.float()).abs().max().item()
        print(f"vit {what} {name}: {100 * eq:.2f}% bit-equal, max |diff| {d:.3g} (scale {b.float().abs().max().item():.3g})")
        assert close(a, b), (what, name, d)


def test_vit_graph_replays_equal_eager(cuda):
    from gravityocr_amd.vit_graph import VitGraphRunner
    v = _tower(cuda)
    r = VitGraphRunner(v, max_m=1024)
    g = torch.Generator(device=cuda).manual_seed(1)
    cases = [(8, 12), (12, 8), (16, 16), (8, 12)]
    for h, w in cases:
        x = torch.randn(h * w, 3 * 2 * 14 * 14, device=cuda, generator=g).bfloat16()
        grid = torch.tensor([[1, h, w]], device=cuda)
        ref = _eager(v, x, grid)
        out = r(x, grid_thw=grid, return_dict=True)
        torch.cuda.synchronize()
        _check(out, ref, (h, w))
        # a replay with another grid's positions (same M) is far off: the check can tell
        if (h, w) == (12, 8):
            from gravityocr_amd.vit_graph import close
            wrong = _eager(v, x, torch.tensor([[1, 8, 12]], device=cuda))
            assert not close(out.pooler_output, wrong.pooler_output)
    assert r.graph_sizes == [96, 256] and r.n_replays == len(cases)
    # eager fallbacks: two images; more patches than max_m
    x = torch.randn(128, 3 * 2 * 14 * 14, device=cuda, generator=g).bfloat16()
    grid = torch.tensor([[1, 8, 8], [1, 8, 8]], device=cuda)
    _check(r(x, grid_thw=grid, return_dict=True), _eager(v, x, grid), "two images")
    x = torch.randn(32 * 40, 3 * 2 * 14 * 14, device=cuda, generator=g).bfloat16()
    grid = torch.tensor([[1, 32, 40]], device=cuda)
    _check(r(x, grid_thw=grid, return_dict=True), _eager(v, x, grid), "M > max_m")
    assert r.n_replays == len(cases) and r.graph_sizes == [96, 256]
    # host time per call: eager tower vs replay (printed)
    x = torch.randn(256, 3 * 2 * 14 * 14, device=cuda, generator=g).bfloat16()
    grid = torch.tensor([[1, 16, 16]], device=cuda)
    for name, fn in (("eager", lambda: _eager(v, x, grid)), ("graph", lambda: r(x, grid_thw=grid))):
        fn()
        torch.cuda.synchronize()
        t0 = time.perf_counter()
        for _ in range(20):
            fn()
        torch.cuda.synchronize()
        print(f"vit {name}: {(time.perf_counter() - t0) / 20 * 1e3:.2f} ms per call (256 patches, 4 blocks)")


def test_enable_vit_graphs_installs_once(cuda):
    from gravityocr_amd.vit_graph import VitGraphRunner, enable_vit_graphs
    holder = type("MM", (), {})()
    holder.visual = _tower(cuda)
    model = type("Model", (), {})()
    model.mm_model = holder
    r = enable_vit_graphs(model)
    assert isinstance(holder.visual, VitGraphRunner) and enable_vit_graphs(model) is r
    assert r.spatial_merge_size == 2 and r.config.out_hidden_size == 128   # the tower's attributes, through the runner
