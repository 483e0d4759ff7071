"""ctypes binding of the C-ABI kernel library (include/gss.h). Loading fails loudly when the library is missing:
there is no CPU or eager fallback on the product path."""
import ctypes
import os
import re

HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(HERE, "lib", "libgss.so")
HEADER = os.path.join(os.path.dirname(HERE), "include", "gss.h")

_p, _i, _i64, _sz, _f = ctypes.c_void_p, ctypes.c_int, ctypes.c_int64, ctypes.c_size_t, ctypes.c_float
_psz = ctypes.POINTER(ctypes.c_size_t)

# argument types of every entry point, in header order
SIGNATURES = {
    "gss_version": ([], ctypes.c_char_p),
    "gss_status_string": ([_i], ctypes.c_char_p),
    "gss_attn_make_plan": ([_i, _i, _i, _i, _i, _i, _p], _i),
    "gss_attn_workspace_size": ([_i, _i, _i, _i, _i, _p, _psz], _i),
    "gss_draft_attn": ([_p, _p, _p, _p, _i, _p, _i, _p, _p, _p, _i, _i, _i, _i, _i, _i, _i, _f, _p, _p, _sz, _p], _i),
    "gss_verify_attn": ([_p, _p, _p, _p, _i, _p, _i, _p, _p, _p, _i, _i, _i, _i, _i, _i, _f, _p, _p, _sz, _p], _i),
    "gss_argmax_workspace_size": ([_i, _i, _i, _psz], _i),
    "gss_argmax_accept": ([_p, _i, _i64, _i, _i, _i, _i, _p, _p, _p, _p, _p, _p, _sz, _p], _i),
    "gss_argmax_accept_noalloc": ([_p, _i, _i64, _i, _i, _i, _i, _p, _p, _p, _p, _p, _p], _i),
    "gss_unmask_workspace_size": ([_i, _i, _i, _psz], _i),
    "gss_unmask_step": ([_p, _i, _i64, _i, _i, _i, _p, _i, _f, _p, _p, _p, _p, _p, _p, _sz, _p], _i),
    "gss_kv_commit_workspace_size": ([_i, _psz], _i),
    "gss_kv_commit": ([_p, _p, _i64, _p, _p, _i64, _p, _i, _p, _p, _i, _p, _i, _i, _i, _i, _i, _i, _p, _sz, _p], _i),
    "gss_ss_commit": ([_p, _p, _p, _i64, _p, _p, _p, _p, _p, _p, _p, _i64, _i, _i, _i, _p, _p, _p, _p], _i),
    "gss_kv_meta": ([_p, _i64, _i64, _p, _p, _i, _p, _p, _i64, _i, _p], _i),
    "gss_log_append": ([_p, _i, _p, _p, _i, _p, _p, _i, _p, _p, _i, _p], _i),
    "gss_penalize_rows": ([_p, _i64, _i, _i, _i, _p, _p, _p], _i),
    "gss_apply_vocab_mask": ([_p, _i64, _i, _i, _p, _i64, _p], _i),
    "gss_sample_workspace_size": ([_i, _i, _psz], _i),
    "gss_sample_rows": ([_p, _i64, _i, _i, _i, _i, _p, _p, _p, _p, _p, _p, _p, _p, _p, _p, _p, _p, _p, _sz, _p], _i),
    "gss_gemm_workspace_size": ([_i, _i, _i, _psz], _i),
    "gss_gemm": ([_p, _i64, _p, _p, _i64, _p, _i64, _i, _i, _i, _i, _p, _p, _sz, _p], _i),
    "gss_gemm_parts_count": ([_i, _i, ctypes.POINTER(ctypes.c_int)], _i),
    "gss_gemm_parts": ([_p, _i64, _p, _i64, _p, _i, _i, _i, _p], _i),
    "gss_gemm_swiglu": ([_p, _i64, _p, _p, _i64, _p, _i, _i, _i, _p, _sz, _p], _i),
    "gss_gemm_rope_stage": ([_p, _i64, _p, _p, _i64, _p, _p, _p, _i, _p, _p, _p, _i, _i, _i, _i, _i, _i, _p, _sz,
                             _p], _i),
    "gss_rope_stage": ([_p, _i64, _p, _p, _i, _p, _i, _p, _p, _p, _i, _i, _i, _i, _i, _p], _i),
    "gss_rope_stage_mrope": ([_p, _i64, _p, _i, _i, _p, _i, _p, _p, _p, _i, _i, _i, _i, _p], _i),
    "gss_rmsnorm": ([_p, _p, _p, _i, _i, _f, _p], _i),
    "gss_embed_rmsnorm": ([_p, _p, _i, _p, _p, _p, _i, _i, _f, _p], _i),
    "gss_add_rmsnorm": ([_p, _p, _p, _p, _p, _i, _i, _f, _p], _i),
    "gss_add_rmsnorm_parts": ([_p, _i, _p, _p, _p, _p, _i, _i, _f, _p], _i),
    "gss_silu_mul": ([_p, _i64, _p, _i, _i, _p], _i),
}



class AttnPlan(ctypes.Structure):
    """gss_attn_plan (include/gss.h): the attention kernel and key partition of a batch shape."""
    _fields_ = [("kernel", ctypes.c_int), ("tiles_per_split", ctypes.c_int), ("n_split", ctypes.c_int),
                ("max_kv_len", ctypes.c_int)]

    def key(self):
        return (self.kernel, self.tiles_per_split, self.n_split, self.max_kv_len)

    def __repr__(self):
        return "AttnPlan(kernel=%d, tiles_per_split=%d, n_split=%d, max_kv_len=%d)" % self.key()


class FinishRule(ctypes.Structure):
    """gss_finish_rule (include/gss.h): per-request budget, stop ids and vocabulary bound of the cut rule."""
    _fields_ = [("budget", ctypes.c_void_p), ("stop_ids", ctypes.c_void_p), ("n_stop", ctypes.c_int),
                ("vocab", ctypes.c_void_p)]


class NormEpilogue(ctypes.Structure):
    """gss_norm_epilogue (include/gss.h)."""
    _fields_ = [("w_post", ctypes.c_void_p), ("h", ctypes.c_void_p), ("w_next", ctypes.c_void_p),
                ("x", ctypes.c_void_p), ("eps", ctypes.c_float)]


class Penalties(ctypes.Structure):
    """gss_penalties (include/gss.h)."""
    _fields_ = [("n_order", ctypes.c_int), ("order", ctypes.c_int * 4)] + [
        (n, ctypes.c_void_p) for n in ("rep_cum", "rep_pen", "pres_cum", "pres_pen", "freq_cum", "freq_pen", "len_out",
                                       "min_new", "stop_pen", "logit_bias")]


class NormPrologue(ctypes.Structure):
    """gss_norm_prologue (include/gss.h)."""
    _fields_ = [("a", ctypes.c_void_p), ("h_in", ctypes.c_void_p), ("h_out", ctypes.c_void_p),
                ("w_post", ctypes.c_void_p), ("w_next", ctypes.c_void_p), ("eps", ctypes.c_float),
                ("a_parts", ctypes.c_void_p), ("n_parts", ctypes.c_int)]


_LIB = None


class GssError(RuntimeError):
    pass


def header_symbols():
    """Function names declared in include/gss.h."""
    txt = open(HEADER).read()
    txt = re.sub(r"/\*.*?\*/", "", txt, flags=re.S)
    return re.findall(r"^\s*(?:const\s+)?\w+\**\s+\**(gss_\w+)\s*\(", txt, flags=re.M)


def lib():
    """Load libgss.so once and declare the prototypes. Raises if the library has not been built."""
    global _LIB
    if _LIB is None:
        if not os.path.exists(LIB_PATH):
            raise GssError(f"{LIB_PATH} is missing: build it with `python -m gravityocr_amd.build` "
                           "(the HIP kernels have no CPU fallback)")
        L = ctypes.CDLL(LIB_PATH)
        for name, (args, res) in SIGNATURES.items():
            fn = getattr(L, name)
            fn.argtypes = args
            fn.restype = res
        _LIB = L
    return _LIB


def check(status: int, what: str):
    if status != 0:
        msg = lib().gss_status_string(status).decode()
        raise GssError(f"{what}: {msg} (status {status})")
