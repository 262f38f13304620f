"""ctypes binding of libhsd.so (the gfx950 HIP kernels behind a C ABI).

The library is built in-tree (`make` in the package root, or `__graft_entry__.build()`)
and loaded from next to this package. There is no fallback: if the library is missing
or a call fails, an exception says so.
"""
from __future__ import annotations

import contextlib
import ctypes
import gc
import os

import torch

_PKG_ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
# HSD_LIB: path of another build of the same library (e.g. a tuning variant)
LIB_PATH = os.environ.get("HSD_LIB") or os.path.join(_PKG_ROOT, "libhsd.so")

DT_BF16, DT_F16, DT_F32 = 0, 1, 2
STATUS_BAD_EXPERT, STATUS_BAD_STATE, STATUS_BAD_TOKEN = 1, 2, 4
X_BF16, X_RMS, X_GATED, X_GATED_Z = 0, 1, 2, 3
W_Q4, W_BF16 = 0, 1
Y_BF16, Y_F32, Y_RESID, Y_ARGMAX = 0, 1, 2, 3
# sequence state indices (include/hsd.h HSD_SEQ_*)
SEQ_POS, SEQ_CUR, SEQ_N, SEQ_TOK, SEQ_HEAD_POS, SEQ_R, SEQ_HEAD_POS2, SEQ_ACCEPT, SEQ_STEPS, SEQ_ACC_SUM = range(10)
SEQ_LEN = 16


@contextlib.contextmanager
def capture_guard():
    """Python's cyclic garbage collector runs one full pass, then stays off for the body
    (a stream capture). A dead object that owns a captured graph (a torch CUDAGraph held in
    a reference cycle) must not be freed while a capture runs: releasing its memory pool is
    an API call that a global-mode capture prohibits, and the error, raised in a destructor,
    aborts the process. torch.cuda.graph no longer collects on entry by default."""
    gc.collect()
    was = gc.isenabled()
    gc.disable()
    try:
        yield
    finally:
        if was:
            gc.enable()


_c_int, _c_i64, _c_size, _c_float, _vp = ctypes.c_int, ctypes.c_int64, ctypes.c_size_t, ctypes.c_float, ctypes.c_void_p

# name -> (restype, [argtypes]); every pointer is passed as void*.
_SIGS = {
    "hsd_last_error": (ctypes.c_char_p, []),
    "hsd_abi_version": (_c_int, []),
    "hsd_permute_nibbles": (_c_int, [_vp, _vp, _c_i64, _c_i64, _c_i64, _vp]),
    "hsd_transpose_u16": (_c_int, [_vp, _vp, _c_i64, _c_i64, _c_i64, _vp]),
    "hsd_sparse_down_workspace_bytes": (_c_size, [_c_i64] * 5),
    "hsd_sparse_down_decode": (_c_int, [_vp, _c_int, _vp, _vp, _vp, _vp, _vp, _vp, _vp, _vp, _vp, _c_int,
                                        _c_i64, _c_i64, _c_i64, _c_i64, _c_i64, _c_i64, _c_int, _vp, _vp,
                                        _vp, _c_size, _vp]),
    "hsd_sparse_down_decode_noalloc": (_c_int, [_vp, _c_int, _vp, _vp, _vp, _vp, _vp, _vp, _vp, _vp, _vp,
                                                _c_int, _c_i64, _c_i64, _c_i64, _c_i64, _c_i64, _c_i64,
                                                _c_int, _vp, _vp, _vp]),
    "hsd_dense_down_decode": (_c_int, [_vp, _c_int, _vp, _vp, _vp, _vp, _vp, _vp, _vp, _vp, _vp, _c_int,
                                       _c_i64, _c_i64, _c_i64, _c_i64, _c_i64, _c_i64, _vp, _vp]),
    "hsd_prefill_num_tiles": (_c_i64, [_c_i64] * 4),
    "hsd_prefill_tiles_workspace_bytes": (_c_size, [_c_i64] * 3),
    "hsd_prefill_tiles": (_c_int, [_vp, _c_i64, _c_i64, _c_i64, _c_i64, _vp, _vp, _vp, _vp, _c_size, _vp]),
    "hsd_prefill_union": (_c_int, [_vp, _c_int, _vp, _vp, _vp, _vp] + [_c_i64] * 8 + [_vp]),
    "hsd_prefill_gemm_workspace_bytes": (_c_size, [_c_i64] * 7),
    "hsd_prefill_gemm": (_c_int, [_vp] * 14 + [_c_int] + [_c_i64] * 9 + [_vp, _c_size, _vp]),
    "hsd_mamba_workspace_bytes": (_c_size, [_c_i64] * 3),
    "hsd_mamba_verify": (_c_int, [_vp, _c_i64, _vp, _c_i64, _vp, _c_i64] + [_vp] * 9 + [_c_i64, _vp, _c_int]
                         + [_c_i64] * 6 + [_c_float] * 3 + [_vp, _vp, _c_size, _vp]),
    "hsd_mamba_ssm": (_c_int, [_vp, _c_i64, _vp, _c_i64] + [_vp] * 8 + [_c_i64, _vp] + [_c_i64] * 5
                      + [_c_float] * 2 + [_vp, _vp]),
    "hsd_mamba_ssm_gated": (_c_int, [_vp, _c_i64, _vp, _c_i64, _vp, _c_i64] + [_vp] * 8 + [_c_i64, _vp, _c_i64]
                            + [_c_i64] * 5 + [_c_float] * 2 + [_vp, _vp]),
    "hsd_mamba_select_row": (_c_int, [_vp, _vp, _c_i64, _c_i64, _c_i64, _vp, _vp]),
    "hsd_greedy_accept": (_c_int, [_vp, _c_int, _c_i64, _c_i64, _vp, _vp, _vp, _vp, _vp, _vp, _c_i64, _vp]),
    "hsd_moe_up_relu2": (_c_int, [_vp, _c_int, _vp, _vp, _vp, _vp, _vp, _vp, _vp, _vp]
                         + [_c_i64] * 6 + [_vp, _vp, _vp]),
    "hsd_moe_route_up_relu2": (_c_int, [_vp, _c_int, _vp, _vp, _c_float, _c_int, _vp, _vp] + [_vp] * 7
                               + [_c_i64] * 6 + [_vp, _vp]),
    "hsd_router_topk": (_c_int, [_vp, _vp, _c_float, _c_int, _vp, _vp, _c_i64, _c_i64, _c_i64, _vp]),
    "hsd_sparse_down_residual": (_c_int, [_vp, _c_int] + [_vp] * 10 + [_c_i64] * 6 + [_c_int, _vp, _vp, _vp,
                                                                                      _c_size, _vp]),
    "hsd_linear_argmax_slots": (_c_i64, [_c_i64, _c_int]),
    "hsd_linear": (_c_int, [_vp, _c_i64, _c_int, _vp, _c_i64, _vp, _c_float, _vp, _vp, _vp, _c_int, _vp, _c_i64,
                            _c_int, _vp, _c_i64, _vp, _c_i64, _vp, _c_i64, _c_i64, _c_i64, _c_i64, _vp]),
    "hsd_argmax_keys": (_c_int, [_vp, _c_i64, _c_i64, _c_i64, _vp, _vp]),
    "hsd_attn_workspace_bytes": (_c_size, [_c_i64] * 3),
    "hsd_attn_decode": (_c_int, [_vp, _c_i64, _c_i64, _vp, _vp, _c_i64, _vp, _vp, _c_i64, _c_i64, _c_i64, _c_i64,
                                 _c_float, _vp, _vp, _c_size, _vp]),
    "hsd_embed_q4": (_c_int, [_vp, _c_i64, _vp, _vp, _vp, _c_i64, _c_i64, _vp, _c_i64, _vp, _vp]),
    "hsd_pair_norm": (_c_int, [_vp, _c_i64, _vp, _c_i64, _vp, _vp, _c_float, _c_i64, _c_i64, _vp, _c_i64, _vp]),
    "hsd_decode_advance": (_c_int, [_vp, _c_i64, _vp, _vp, _c_i64, _c_i64, _vp]),
    "hsd_spec_accept": (_c_int, [_vp, _c_i64, _c_i64, _c_i64, _vp, _vp, _vp, _c_i64, _c_i64, _vp, _vp, _vp]),
    "hsd_seq_select_row": (_c_int, [_vp, _c_i64, _vp, _vp, _c_i64, _vp]),
    "hsd_mtp_chain": (_c_int, [_vp, _c_i64, _c_i64, _vp, _c_i64, _c_i64, _vp, _vp, _vp, _vp]),
    "hsd_draft_ids": (_c_int, [_vp, _vp, _c_i64, _c_i64, _vp, _vp, _c_i64, _vp, _c_i64, _c_i64, _vp, _vp]),
    "hsd_head_input": (_c_int, [_vp, _vp, _c_i64, _vp, _vp, _vp, _c_i64, _vp, _c_i64, _vp, _vp, _c_float, _c_i64,
                                _c_i64, _vp, _vp, _vp, _c_i64, _vp, _vp]),
    "hsd_verify_input": (_c_int, [_vp, _vp, _c_i64, _c_i64, _vp, _vp, _c_i64, _vp, _c_i64, _c_i64, _vp, _vp, _vp,
                                  _c_i64, _vp, _vp, _c_i64, _vp, _vp]),
    "hsd_seq_add": (_c_int, [_vp, _c_i64, _c_i64, _vp]),
    "hsd_gather_tokens": (_c_int, [_vp, _c_i64, _vp, _c_i64, _c_i64, _vp, _vp]),
    "hsd_prefill_advance": (_c_int, [_vp, _c_i64, _c_i64, _c_i64, _vp]),
    "hsd_seq_rollback": (_c_int, [_vp, _c_i64, _c_i64, _vp]),
}

EXPORTS = tuple(_SIGS)


class HSDError(RuntimeError):
    """A libhsd entry point returned a negative status."""


_lib = None


def lib():
    """The loaded library (loaded once). Raises if it has not been built."""
    global _lib
    if _lib is None:
        if not os.path.exists(LIB_PATH):
            raise HSDError(f"libhsd.so not found at {LIB_PATH}: build it first "
                           "(make -C mlx-heimr-sparse-down_amd, or __graft_entry__.build())")
        L = ctypes.CDLL(LIB_PATH)
        for name, (res, args) in _SIGS.items():
            f = getattr(L, name)
            f.restype = res
            f.argtypes = args
        _lib = L
    return _lib


def call(name, *args):
    """Call an entry point; raise HSDError with hsd_last_error() on a negative status."""
    rc = getattr(lib(), name)(*args)
    if rc != 0:
        raise HSDError(f"{name} -> {rc}: {lib().hsd_last_error().decode(errors='replace')}")
    return rc


def ptr(t):
    """Device pointer of a tensor (None -> NULL)."""
    if t is None:
        return None
    if not t.is_cuda:
        raise HSDError("libhsd takes device tensors only (got a CPU tensor)")
    return ctypes.c_void_p(t.data_ptr())


def stream(device=None):
    """The current torch stream of `device` as a hipStream_t."""
    return ctypes.c_void_p(torch.cuda.current_stream(device).cuda_stream)


_DT = {torch.bfloat16: DT_BF16, torch.float16: DT_F16, torch.float32: DT_F32}


def dtype_tag(dt):
    try:
        return _DT[dt]
    except KeyError:
        raise HSDError(f"unsupported dtype {dt}; libhsd takes bfloat16, float16 or float32") from None


def as_words(t):
    """A packed-nibble tensor (int32 or uint32) as the int32 view the kernels read."""
    if t.dtype == torch.int32:
        return t
    if t.dtype == torch.uint32:
        return t.view(torch.int32)
    raise HSDError(f"packed 4-bit words must be int32 or uint32, got {t.dtype}")


def as_u16(t):
    """A bf16 (or any 16-bit) tensor passed by its bit pattern."""
    if t.element_size() != 2:
        raise HSDError(f"expected a 16-bit tensor, got {t.dtype}")
    return t


def contig(t):
    """Row-contiguous inputs, copied if needed (as mx.fast.metal_kernel's
    ensure_row_contiguous does for the reference's kernels, decode.py:146-153)."""
    return t if t.is_contiguous() else t.contiguous()
