"""ctypes binding of libprefixlm.so (the C ABI in include/prefixlm.h).

Loading fails loudly if the library was not built: there is no fallback path.
torch is imported first so that the library binds to the HIP runtime torch
loaded (same soname), and the streams torch hands out are valid for it.
"""
from __future__ import annotations

import ctypes
import os

import torch  # noqa: F401  (must be loaded before the HIP library)

from ._build import LIB_PATH

c_i32, c_i64, c_f32, c_vp, c_sz = ctypes.c_int32, ctypes.c_int64, ctypes.c_float, ctypes.c_void_p, ctypes.c_size_t
_c_i32p = ctypes.POINTER(ctypes.c_int32)
_c_f32p = ctypes.POINTER(ctypes.c_float)

NUM_KERNELS = 8
KERNEL_NAMES = ("fwd_worklist", "fwd", "fwd_pad", "bwd_worklist", "bwd_pre", "bwd_dkdv", "bwd_pad", "bwd_dq")


class _SizedArgs(ctypes.Structure):
    """An argument struct whose first field, struct_size, the library checks against its
    own sizeof: filled in here, the other fields follow positionally or by keyword."""

    def __init__(self, *args, **kw):
        super().__init__(ctypes.sizeof(type(self)), *args, **kw)


class FwdArgs(_SizedArgs):
    _fields_ = [
        ("struct_size", ctypes.c_uint32),
        ("q", c_vp), ("k", c_vp), ("v", c_vp), ("out", c_vp), ("out_lo", c_vp), ("lse", c_vp),
        ("q_stride_t", c_i64), ("q_stride_h", c_i64),
        ("k_stride_t", c_i64), ("k_stride_h", c_i64),
        ("v_stride_t", c_i64), ("v_stride_h", c_i64),
        ("out_stride_t", c_i64), ("out_stride_h", c_i64),
        ("out_lo_stride_t", c_i64), ("out_lo_stride_h", c_i64),
        ("prefix_lens", c_vp), ("causal_lens", c_vp), ("cu_seqlens", c_vp),
        ("meta_len", c_i64),
        ("num_tokens", c_i32), ("num_heads", c_i32), ("head_dim", c_i32),
        ("total_seqlen", c_i32), ("numseqs", c_i32),
        ("max_seqlen_prefix", c_i32), ("max_seqlen_causal", c_i32), ("max_seqlen_all", c_i32),
        ("is_causal", c_i32), ("softmax_scale", c_f32),
        ("workspace", c_vp), ("workspace_bytes", c_sz),
        ("plan", c_vp), ("plan_bytes", c_sz),
        ("gate", c_vp), ("out_gated", c_vp),
        ("gate_stride_t", c_i64), ("gate_stride_h", c_i64),
        ("out_gated_stride_t", c_i64), ("out_gated_stride_h", c_i64),
        ("timer", c_vp),
        ("q_amax", c_vp),
    ]


class BwdArgs(_SizedArgs):
    _fields_ = [
        ("struct_size", ctypes.c_uint32),
        ("q", c_vp), ("k", c_vp), ("v", c_vp), ("out", c_vp), ("out_lo", c_vp), ("dout", c_vp),
        ("lse", c_vp), ("q_amax", c_vp),
        ("dq", c_vp), ("dk", c_vp), ("dv", c_vp),
        ("q_stride_t", c_i64), ("q_stride_h", c_i64),
        ("k_stride_t", c_i64), ("k_stride_h", c_i64),
        ("v_stride_t", c_i64), ("v_stride_h", c_i64),
        ("out_stride_t", c_i64), ("out_stride_h", c_i64),
        ("out_lo_stride_t", c_i64), ("out_lo_stride_h", c_i64),
        ("dout_stride_t", c_i64), ("dout_stride_h", c_i64),
        ("dq_stride_t", c_i64), ("dq_stride_h", c_i64),
        ("dk_stride_t", c_i64), ("dk_stride_h", c_i64),
        ("dv_stride_t", c_i64), ("dv_stride_h", c_i64),
        ("prefix_lens", c_vp), ("causal_lens", c_vp), ("cu_seqlens", c_vp),
        ("meta_len", c_i64),
        ("num_tokens", c_i32), ("num_heads", c_i32), ("head_dim", c_i32),
        ("total_seqlen", c_i32), ("numseqs", c_i32),
        ("max_seqlen_prefix", c_i32), ("max_seqlen_causal", c_i32), ("max_seqlen_all", c_i32),
        ("is_causal", c_i32), ("softmax_scale", c_f32),
        ("workspace", c_vp), ("workspace_bytes", c_sz),
        ("plan", c_vp), ("plan_bytes", c_sz),
        ("gate", c_vp), ("dgate", c_vp), ("dout_attn", c_vp),
        ("gate_stride_t", c_i64), ("gate_stride_h", c_i64),
        ("dgate_stride_t", c_i64), ("dgate_stride_h", c_i64),
        ("dout_attn_stride_t", c_i64), ("dout_attn_stride_h", c_i64),
        ("timer", c_vp),
        ("ds_buf", c_vp), ("ds_buf_bytes", c_sz), ("ds_blocks", c_i64),
    ]


class RopeArgs(ctypes.Structure):
    _fields_ = [
        ("x", c_vp), ("y", c_vp), ("cos", c_vp), ("sin", c_vp),
        ("x_stride_t", c_i64), ("x_stride_h", c_i64),
        ("y_stride_t", c_i64), ("y_stride_h", c_i64),
        ("cs_stride_t", c_i64),
        ("num_tokens", c_i32), ("num_heads", c_i32), ("head_dim", c_i32), ("backward", c_i32),
    ]


class KvcacheArgs(ctypes.Structure):
    _fields_ = [
        ("q", c_vp), ("k", c_vp), ("v", c_vp), ("k_cache", c_vp), ("v_cache", c_vp), ("out", c_vp),
        ("q_stride_b", c_i64), ("q_stride_s", c_i64), ("q_stride_h", c_i64),
        ("k_stride_b", c_i64), ("k_stride_s", c_i64), ("k_stride_h", c_i64),
        ("v_stride_b", c_i64), ("v_stride_s", c_i64), ("v_stride_h", c_i64),
        ("k_cache_stride_b", c_i64), ("k_cache_stride_s", c_i64), ("k_cache_stride_h", c_i64),
        ("v_cache_stride_b", c_i64), ("v_cache_stride_s", c_i64), ("v_cache_stride_h", c_i64),
        ("out_stride_b", c_i64), ("out_stride_s", c_i64), ("out_stride_h", c_i64),
        ("cache_seqlens", c_vp), ("cache_seqlen", c_i32),
        ("batch", c_i32), ("seqlen_q", c_i32), ("num_heads", c_i32), ("head_dim", c_i32),
        ("max_seqlen_cache", c_i32), ("is_causal", c_i32), ("softmax_scale", c_f32),
        ("workspace", c_vp), ("workspace_bytes", c_sz),
    ]


class SwigluArgs(ctypes.Structure):
    _fields_ = [
        ("gu", c_vp), ("dy", c_vp), ("y", c_vp), ("dgu", c_vp),
        ("gu_stride", c_i64), ("y_stride", c_i64), ("dy_stride", c_i64), ("dgu_stride", c_i64),
        ("rows", c_i64), ("cols", c_i64),
    ]


class RmsnormArgs(ctypes.Structure):
    _fields_ = [
        ("x", c_vp), ("dy", c_vp), ("y", c_vp), ("dx", c_vp), ("rstd", c_vp),
        ("x_stride", c_i64), ("y_stride", c_i64), ("dy_stride", c_i64), ("dx_stride", c_i64),
        ("rows", c_i64), ("cols", c_i32), ("eps", c_f32),
    ]


class ProjGemmArgs(ctypes.Structure):
    _fields_ = [
        ("x", c_vp), ("w", c_vp), ("y", c_vp),
        ("x_stride", c_i64), ("w_stride", c_i64), ("y_stride", c_i64),
        ("M", c_i32), ("K", c_i32), ("N", c_i32), ("swiglu", c_i32), ("norm", c_i32), ("eps", c_f32),
        ("rstd", c_vp),
    ]


# every symbol include/prefixlm.h declares, with (restype, argtypes)
SIGNATURES = {
    "prefixlm_fwd_workspace_size": (c_sz, [c_i32, c_i32, c_i32, c_i32, c_i32]),
    "prefixlm_fwd_q_amax_count": (c_sz, [c_i32, c_i32]),
    "prefixlm_bwd_workspace_size": (c_sz, [c_i32, c_i32, c_i32, c_i32, c_i32]),
    "prefixlm_bwd_ds_bytes": (c_sz, [c_i32, c_i32, c_i32, c_i32]),
    "prefixlm_bwd_ds_bytes_blocks": (c_sz, [c_i32, c_i32, c_i32, c_i64]),
    "prefixlm_plan_ds_blocks": (c_i64, [c_vp, c_sz]),
    "prefixlm_fwd": (ctypes.c_int, [ctypes.POINTER(FwdArgs), c_vp]),
    "prefixlm_bwd": (ctypes.c_int, [ctypes.POINTER(BwdArgs), c_vp]),
    "prefixlm_bwd_noalloc": (ctypes.c_int, [ctypes.POINTER(BwdArgs), c_vp]),
    "prefixlm_bwd_noalloc_max_scratch": (c_sz, []),
    "prefixlm_check_workspace": (ctypes.c_int, [c_vp, c_vp, _c_i32p]),
    "prefixlm_plan_size": (c_sz, [c_i32, c_i32]),
    "prefixlm_rope": (ctypes.c_int, [ctypes.POINTER(RopeArgs), c_vp]),
    "prefixlm_swiglu_fwd": (ctypes.c_int, [ctypes.POINTER(SwigluArgs), c_vp]),
    "prefixlm_swiglu_bwd": (ctypes.c_int, [ctypes.POINTER(SwigluArgs), c_vp]),
    "prefixlm_rmsnorm_fwd": (ctypes.c_int, [ctypes.POINTER(RmsnormArgs), c_vp]),
    "prefixlm_rmsnorm_bwd": (ctypes.c_int, [ctypes.POINTER(RmsnormArgs), c_vp]),
    "prefixlm_proj_gemm": (ctypes.c_int, [ctypes.POINTER(ProjGemmArgs), c_vp]),
    "prefixlm_kvcache_workspace_size": (c_sz, [c_i32, c_i32, c_i32, c_i32, c_i32]),
    "prefixlm_kvcache_fwd": (ctypes.c_int, [ctypes.POINTER(KvcacheArgs), c_vp]),
    "prefixlm_plan_build": (ctypes.c_int, [_c_i32p, _c_i32p, _c_i32p, c_i32, c_i32, c_i32, c_i32, c_vp, c_sz]),
    "prefixlm_last_error": (ctypes.c_char_p, []),
    "prefixlm_version": (c_i32, []),
    "prefixlm_timer_create": (c_vp, []),
    "prefixlm_timer_destroy": (None, [c_vp]),
    "prefixlm_timer_read": (ctypes.c_int, [c_vp, _c_f32p, _c_i32p]),
}

_lib = None
LIB_VERSION = 300   # include/prefixlm.h PREFIXLM_VERSION


def lib_path() -> str:
    return os.environ.get("PREFIXLM_LIB", LIB_PATH)


def load():
    """Load (once) and return the ctypes library object."""
    global _lib
    if _lib is not None:
        return _lib
    path = lib_path()
    if not os.path.exists(path):
        raise RuntimeError(
            f"{path} is missing: the HIP extension is not built. Run "
            "`python -c 'import __graft_entry__ as g; g.build()'` in the repository root.")
    lib = ctypes.CDLL(path)
    for name, (res, args) in SIGNATURES.items():
        fn = getattr(lib, name)
        fn.restype = res
        fn.argtypes = args
    # the buffers this package allocates (out_lo's element size above all) follow the
    # library's major.minor version: another build would address them differently
    got = lib.prefixlm_version()
    if got // 100 != LIB_VERSION // 100:
        raise RuntimeError(f"{path} is version {got}, this package needs {LIB_VERSION // 100}.x "
                           "(buffer layouts differ): rebuild the extension")
    _lib = lib
    return lib


def last_error() -> str:
    msg = load().prefixlm_last_error()
    return msg.decode() if msg else ""


def check(rc: int, what: str):
    if rc != 0:
        raise RuntimeError(f"{what} failed (status {rc}): {last_error()}")


class Timer:
    """A caller-owned per-kernel timer (``prefixlm_timer_create``). While it is
    active (``with timer:``), the ops pass it to every call they make, and each
    launch is bracketed by HIP events on its stream."""

    _active = None

    def __init__(self):
        self._h = load().prefixlm_timer_create()
        if not self._h:
            raise RuntimeError("prefixlm_timer_create failed")

    def __enter__(self):
        Timer._active = self
        return self

    def __exit__(self, *exc):
        Timer._active = None

    def read(self):
        """{kernel name: (total_ms, launches)} since the last read (synchronizes)."""
        ms = (ctypes.c_float * NUM_KERNELS)()
        n = (ctypes.c_int32 * NUM_KERNELS)()
        check(load().prefixlm_timer_read(ctypes.c_void_p(self._h), ms, n), "prefixlm_timer_read")
        return {KERNEL_NAMES[i]: (float(ms[i]), int(n[i])) for i in range(NUM_KERNELS)}

    def close(self):
        if self._h:
            load().prefixlm_timer_destroy(ctypes.c_void_p(self._h))
            self._h = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass


def active_timer() -> ctypes.c_void_p:
    """Handle of the timer inside a ``with Timer():`` block, else NULL."""
    t = Timer._active
    return ctypes.c_void_p(t._h if t is not None else 0)
