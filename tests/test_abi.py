"""The C-ABI library without a GPU: it loads, exports every function include/gss.h declares (and the ctypes binding
declares exactly those), and its host-side argument checks reject bad calls before anything touches a device. The
drop-in entry points keep the reference's signatures and reject what they do not implement, loudly."""
import ctypes
import inspect
import subprocess

import pytest
import torch

from gravityocr_amd import _lib

OK, ARG, UNSUPPORTED, WORKSPACE = 0, 1, 2, 3


def test_header_symbols_equal_binding():
    syms = _lib.header_symbols()
    assert len(syms) == len(set(syms)) >= 19
    assert set(syms) == set(_lib.SIGNATURES)


def test_library_exports_every_declared_symbol():
    L = _lib.lib()
    for name in _lib.header_symbols():
        assert hasattr(L, name), name
    out = subprocess.run(["nm", "-D", "--defined-only", _lib.LIB_PATH], capture_output=True, text=True,
                         check=True).stdout
    exported = {line.split()[-1] for line in out.splitlines() if " T " in line}
    assert set(_lib.header_symbols()) <= exported


def test_host_side_queries_and_status_strings():
    L = _lib.lib()
    assert L.gss_version().decode().endswith("gfx950")
    assert L.gss_status_string(OK) == b"ok"
    assert L.gss_status_string(WORKSPACE).startswith(b"workspace")
    n = ctypes.c_size_t(0)
    # argmax: arrival counters (1024 sequences x 9 lines of 128 B) + chunk winners (value, index) of ceil(V / 4096)
    # chunks per row
    ctr = 1024 * 9 * 128
    assert L.gss_argmax_workspace_size(2, 17, 59392, ctypes.byref(n)) == OK
    assert n.value == ctr + 2 * 17 * 15 * 8
    assert L.gss_argmax_workspace_size(1, 17, 131073, ctypes.byref(n)) == UNSUPPORTED
    assert L.gss_argmax_workspace_size(1, 65, 100, ctypes.byref(n)) == UNSUPPORTED
    assert L.gss_argmax_workspace_size(0, 17, 100, ctypes.byref(n)) == ARG
    plan = _lib.AttnPlan()
    assert L.gss_attn_make_plan(1, 2, 8192, 0, 0, 0, ctypes.byref(plan)) == OK
    assert L.gss_attn_workspace_size(1, 16, 2, 128, 17, ctypes.byref(plan), ctypes.byref(n)) == OK and n.value > 0
    assert L.gss_attn_workspace_size(1, 16, 3, 128, 17, ctypes.byref(plan), ctypes.byref(n)) == UNSUPPORTED  # Hq % Hkv
    assert L.gss_attn_workspace_size(1, 16, 2, 96, 17, ctypes.byref(plan), ctypes.byref(n)) == UNSUPPORTED   # head dim
    assert L.gss_attn_workspace_size(1, 16, 2, 128, 17, None, ctypes.byref(n)) == ARG
    assert L.gss_kv_commit_workspace_size(4, ctypes.byref(n)) == OK
    # unmask: the same counters + chunk (max, index, sum) of ceil(V / 4096) chunks per row, 16 B each
    assert L.gss_unmask_workspace_size(2, 32, 59392, ctypes.byref(n)) == OK
    assert n.value == ctr + 2 * 32 * 15 * 16
    assert L.gss_unmask_workspace_size(1, 65, 100, ctypes.byref(n)) == UNSUPPORTED


def test_entry_points_reject_bad_arguments_before_launch():
    L = _lib.lib()
    null = None
    # null pointers
    plan = _lib.AttnPlan()
    assert L.gss_attn_make_plan(1, 2, 8192, 0, 0, 0, ctypes.byref(plan)) == OK
    pp = ctypes.byref(plan)
    assert L.gss_draft_attn(null, null, null, null, 1, null, 0, null, null, null, 1, 17, 1, 16, 2, 128, 16, 0.1,
                            pp, null, 0, null) == ARG
    assert L.gss_argmax_accept(null, 0, 100, 1, 1, 100, 0, null, null, null, null, null, null, 0, null) == ARG
    assert L.gss_unmask_step(null, 0, 100, 1, 4, 100, null, 7, 0.9, null, null, null, null, null, null, 0, null) == ARG
    # unsupported page size / window wider than a tile: rejected before pointers are looked at
    assert L.gss_verify_attn(null, null, null, null, 1, null, 0, null, null, null, 1, 17, 16, 2, 128, 32, 0.1,
                             pp, null, 0, null) == UNSUPPORTED
    assert L.gss_verify_attn(null, null, null, null, 1, null, 0, null, null, null, 1, 65, 16, 2, 128, 16, 0.1,
                             pp, null, 0, null) == UNSUPPORTED
    # a missing plan, or one whose splits do not cover its capacity plus a window, is rejected
    bad = _lib.AttnPlan(1, 4, 2, 8192)
    for p in (None, ctypes.byref(bad)):
        assert L.gss_verify_attn(null, null, null, null, 1, null, 0, null, null, null, 1, 17, 16, 2, 128, 16, 0.1,
                                 p, null, 0, null) == ARG
    assert L.gss_attn_make_plan(1, 2, 8192, -1, 0, 0, pp) == ARG
    assert L.gss_attn_make_plan(1, 2, 8192, 0, 257, 0, pp) == ARG
    # the parts norm is built for 1..4 fp32 parts (gss_gemm_parts writes at most 2); dummy aligned pointers are
    # never dereferenced on a rejected call
    fake = ctypes.c_void_p(1 << 20)
    assert L.gss_add_rmsnorm_parts(fake, 5, fake, fake, fake, fake, 17, 1536, 1e-5, null) == UNSUPPORTED
    assert L.gss_add_rmsnorm_parts(fake, 0, fake, fake, fake, fake, 17, 1536, 1e-5, null) == ARG


REFERENCE_SIGNATURES = {
    # src/fast_sampling.py:426-429
    "generate_speculative_natcache": [
        ("model", inspect.Parameter.empty), ("image", inspect.Parameter.empty), ("prompt", "Text Recognition:"),
        ("max_new_tokens", 512), ("draft_threshold", 0.9), ("temperature", 0.0), ("top_p", 0.95),
        ("max_long_side", 1344), ("accept_conf", 0.0), ("draft_steps", 1), ("return_stats", False),
        ("trace", None), ("draft_bd", None), ("full_draft", True)],
    # src/fast_sampling.py:262-266
    "generate_speculative_prefixcache": [
        ("model", inspect.Parameter.empty), ("image", inspect.Parameter.empty), ("prompt", "Text Recognition:"),
        ("max_new_tokens", 512), ("draft_threshold", 0.9), ("temperature", 0.0), ("top_p", 0.95),
        ("max_long_side", 1344), ("accept_conf", 0.0), ("draft_steps", 1), ("return_stats", False),
        ("trace", None), ("full_draft", True)],
    # src/fast_sampling.py:631-632
    "teacher_force_argmax": [("model", inspect.Parameter.empty), ("image", inspect.Parameter.empty),
                             ("prompt", inspect.Parameter.empty), ("gen_ids", inspect.Parameter.empty),
                             ("max_long_side", 1344)],
    # src/fast_sampling.py:50
    "enable_fused_flex": [("dynamic", True)],
    # src/fast_sampling.py:105-107
    "generate_cached": [
        ("model", inspect.Parameter.empty), ("image", inspect.Parameter.empty), ("prompt", "Text Recognition:"),
        ("max_new_tokens", 512), ("threshold", 0.99), ("temperature", 0.0), ("top_p", 0.95),
        ("max_long_side", 1344), ("commit_trace", None), ("commit_causal", False), ("commit_detail", None)],
    # src/fast_sampling_batched.py:95-97
    "fast_sampling_batched.generate_cached_batched": [
        ("model", inspect.Parameter.empty), ("images", inspect.Parameter.empty), ("prompt", "Text Recognition:"),
        ("max_new_tokens", 512), ("threshold", 0.99), ("temperature", 0.0), ("top_p", 0.95),
        ("max_long_side", 1344)],
}


@pytest.mark.parametrize("name", sorted(REFERENCE_SIGNATURES))
def test_dropin_signatures_match_reference(name):
    import importlib
    mod, _, fn = name.rpartition(".")
    module = importlib.import_module("gravityocr_amd." + (mod or "fast_sampling"))
    params = inspect.signature(getattr(module, fn)).parameters
    assert [(p.name, p.default) for p in params.values()] == REFERENCE_SIGNATURES[name]


def test_dropin_rejects_unimplemented_modes_and_cpu_models():
    from gravityocr_amd.fast_sampling import generate_speculative_natcache
    from gravityocr_amd.model import TINY, SyntheticGlmOcr, synthetic_prompt, synthetic_weights
    vis, ids = synthetic_prompt(TINY, 8, 4, 0)
    m = SyntheticGlmOcr(TINY, synthetic_weights(TINY, 0), vis, ids, mask_id=4095, bd_size=4)
    for kw in (dict(temperature=0.7), dict(accept_conf=0.5), dict(draft_steps=2), dict(full_draft=False)):
        with pytest.raises(NotImplementedError):
            generate_speculative_natcache(m, None, **kw)
    with pytest.raises(RuntimeError, match="ROCm GPU"):
        generate_speculative_natcache(m, None)
    from gravityocr_amd.fast_sampling import generate_speculative_prefixcache
    for kw in (dict(temperature=0.7), dict(accept_conf=0.5), dict(draft_steps=2), dict(full_draft=False)):
        with pytest.raises(NotImplementedError):
            generate_speculative_prefixcache(m, None, **kw)
    with pytest.raises(RuntimeError, match="ROCm GPU"):
        generate_speculative_prefixcache(m, None)
    from gravityocr_amd.fast_sampling import generate_cached
    from gravityocr_amd.fast_sampling_batched import generate_cached_batched
    with pytest.raises(NotImplementedError):
        generate_cached(m, None, temperature=0.5)
    with pytest.raises(NotImplementedError):
        generate_cached_batched(m, [None], temperature=0.5)
    with pytest.raises(RuntimeError, match="ROCm GPU"):
        generate_cached(m, None)


def test_gemm_workspace_sizes_follow_the_k_split():
    """Split-K partials only for shapes whose column tiles leave CUs idle and whose splits keep at least 64 k-steps
    (the down projection of the 1536-hidden decoder, 2 splits); the counters' block is always there. The split is a
    function of the weight shape only, so the size scales with M and nothing else, up to M = 64 (larger M runs the
    tiled kernel, which folds the splits in registers)."""
    L = _lib.lib()
    n = ctypes.c_size_t(0)
    sizes = {}
    for M in (17, 544):
        for N, Kd in [(2560, 1536), (1536, 2048), (9216, 1536), (1536, 4608), (59392, 1536)]:
            assert L.gss_gemm_workspace_size(M, N, Kd, ctypes.byref(n)) == OK
            sizes[(M, N, Kd)] = n.value
    ctr = sizes[(17, 9216, 1536)]
    for M in (17, 544):
        assert sizes[(M, 9216, 1536)] == ctr
        assert sizes[(M, 59392, 1536)] == ctr                       # many column tiles: unsplit
        assert sizes[(M, 2560, 1536)] == ctr                        # 48 k-steps: too short to split
        assert sizes[(M, 1536, 2048)] == ctr                        # 64 k-steps: one split of 64
        assert sizes[(M, 1536, 4608)] == ctr + 2 * min(M, 64) * 1536 * 4  # 144 k-steps, 96 column tiles: 2 splits


def test_attn_plans_are_values_of_their_arguments():
    """gss_attn_make_plan: the default policy (about 896 / (bs * Hkv) splits of at least 4 tiles; the wide kernel
    from bs * Hkv = 16), overrides per call, and no process-wide state between calls."""
    L = _lib.lib()

    def mk(*a):
        p = _lib.AttnPlan()
        assert L.gss_attn_make_plan(*a, ctypes.byref(p)) == OK
        return p.key()

    tiles = (8192 + 64 + 63) // 64  # 129
    k1 = mk(1, 2, 8192, 0, 0, 0)
    assert k1 == (0, 4, (tiles + 3) // 4, 8192)
    k32 = mk(32, 2, 12288, 0, 0, 0)
    assert k32[0] == 1 and k32[2] * k32[1] * 64 >= 12288 + 64
    assert mk(1, 2, 8192, 0, 0, 1)[0] == 1                           # wide kernel by override
    assert mk(1, 2, 8192, 1, 256, 0)[1:3] == (256, 1)                 # one split
    assert mk(1, 2, 8192, 0, 0, 0) == k1                              # the override left nothing behind
