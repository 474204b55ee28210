"""ctypes binding of the HIP sampling library (lib/libtachyon_sampler.so).

This is the product path: every call goes to the gfx950 kernels through the C
ABI of include/tachyon_sampler.h.  There is no CPU fallback; if the library
is missing, loading fails with an error that says how to build it.
"""
from __future__ import annotations

import ctypes
import os

HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(HERE, "lib", "libtachyon_sampler.so")

vp = ctypes.c_void_p
u32 = ctypes.c_uint32


class TsmBatch(ctypes.Structure):
    _fields_ = [
        ("logits", vp),
        ("rows", u32),
        ("row_stride", u32),
        ("usable", u32),
        ("mask_stride", u32),
        ("params", vp),
        ("hist_ids", vp),
        ("hist_offsets", vp),
        ("mask", vp),
        ("uniforms", vp),
        ("row_kinds", u32),
        ("reserved", u32),
    ]


class TsmOutputs(ctypes.Structure):
    _fields_ = [
        ("token", vp),
        ("logprob", vp),
        ("top_ids", vp),
        ("top_logprobs", vp),
        ("top_stride", u32),
        ("reserved", u32),
        ("prob", vp),
        ("keep", vp),
    ]


class TsmJsonState(ctypes.Structure):
    _fields_ = [
        ("stack", u32),
        ("depth", ctypes.c_uint8),
        ("state", ctypes.c_uint8),
        ("aux", ctypes.c_uint8),
        ("len", ctypes.c_uint8),
        ("whitespace", ctypes.c_uint8),
        ("pad", ctypes.c_uint8 * 3),
    ]


class TsmJsonFillStats(ctypes.Structure):
    _fields_ = [("rows", u32), ("distinct", u32), ("hits", u32), ("evaluated", u32)]


class TsmVocab(ctypes.Structure):
    _fields_ = [
        ("bytes", vp),
        ("offsets", vp),
        ("special", vp),
        ("n_tokens", u32),
        ("reserved", u32),
    ]


SYMBOLS = ["tsm_create", "tsm_destroy", "tsm_sample", "tsm_distribution", "tsm_status", "tsm_version",
           "tsm_row_kind", "tsm_sample_static", "tsm_json_init", "tsm_json_advance", "tsm_json_accepts",
           "tsm_json_is_complete", "tsm_json_mask", "tsm_json_masks_create", "tsm_json_masks_destroy",
           "tsm_json_masks_reset", "tsm_json_masks_fill", "tsm_lm_head_workspace", "tsm_lm_head",
           "tsm_lm_head_q8_workspace", "tsm_lm_head_q8"]
LM_SPLIT = 1
ROWKIND_SPLIT = 1
ROWKIND_WHOLE = 2
ROWKIND_LEAN = 4

_lib = None


class LibraryMissing(RuntimeError):
    pass


def lib():
    global _lib
    if _lib is None:
        if not os.path.exists(LIB_PATH):
            raise LibraryMissing(
                f"{LIB_PATH} is not built; run `python -c 'import __graft_entry__ as g; g.build()'` "
                "or `python tachyon_amd/build.py`")
        L = ctypes.CDLL(LIB_PATH)
        L.tsm_create.restype = vp
        L.tsm_create.argtypes = [ctypes.c_int, u32, u32, ctypes.c_char_p, ctypes.c_size_t]
        L.tsm_destroy.restype = None
        L.tsm_destroy.argtypes = [vp]
        L.tsm_sample.restype = ctypes.c_int
        L.tsm_sample.argtypes = [vp, vp, ctypes.POINTER(TsmBatch), ctypes.POINTER(TsmOutputs),
                                 ctypes.c_char_p, ctypes.c_size_t]
        L.tsm_distribution.restype = ctypes.c_int
        L.tsm_distribution.argtypes = [vp, vp, ctypes.POINTER(TsmBatch), vp, vp, u32, vp,
                                       ctypes.c_char_p, ctypes.c_size_t]
        L.tsm_status.restype = ctypes.c_int
        L.tsm_status.argtypes = [vp, ctypes.POINTER(u32), ctypes.c_char_p, ctypes.c_size_t]
        L.tsm_version.restype = ctypes.c_char_p
        L.tsm_version.argtypes = []
        L.tsm_sample_static.restype = ctypes.c_int
        L.tsm_sample_static.argtypes = [vp, ctypes.POINTER(TsmBatch), ctypes.POINTER(TsmOutputs), vp,
                                        ctypes.c_char_p, ctypes.c_size_t]
        L.tsm_row_kind.restype = u32
        L.tsm_row_kind.argtypes = [vp, u32, u32, ctypes.c_int]
        js = ctypes.POINTER(TsmJsonState)
        L.tsm_json_init.restype = None
        L.tsm_json_init.argtypes = [js]
        L.tsm_json_advance.restype = None
        L.tsm_json_advance.argtypes = [js, ctypes.c_char_p, ctypes.c_size_t]
        L.tsm_json_accepts.restype = ctypes.c_int
        L.tsm_json_accepts.argtypes = [js, ctypes.c_char_p, ctypes.c_size_t]
        L.tsm_json_is_complete.restype = ctypes.c_int
        L.tsm_json_is_complete.argtypes = [js]
        L.tsm_json_mask.restype = ctypes.c_int
        L.tsm_json_mask.argtypes = [vp, ctypes.POINTER(TsmVocab), vp, u32, u32, vp, u32, ctypes.c_char_p,
                                    ctypes.c_size_t]
        L.tsm_json_masks_create.restype = vp
        L.tsm_json_masks_create.argtypes = [ctypes.c_int, u32, u32, u32, ctypes.c_char_p, ctypes.c_size_t]
        L.tsm_json_masks_destroy.restype = None
        L.tsm_json_masks_destroy.argtypes = [vp]
        L.tsm_json_masks_reset.restype = None
        L.tsm_json_masks_reset.argtypes = [vp]
        L.tsm_json_masks_fill.restype = ctypes.c_int
        L.tsm_json_masks_fill.argtypes = [vp, vp, ctypes.POINTER(TsmVocab), ctypes.POINTER(TsmJsonState), u32, vp,
                                          u32, ctypes.POINTER(TsmJsonFillStats), ctypes.c_char_p, ctypes.c_size_t]
        L.tsm_lm_head_workspace.restype = ctypes.c_size_t
        L.tsm_lm_head_workspace.argtypes = [u32, u32, u32]
        L.tsm_lm_head.restype = ctypes.c_int
        L.tsm_lm_head.argtypes = [vp, vp, u32, vp, ctypes.c_float, vp, u32, u32, u32, u32, vp, ctypes.c_size_t,
                                  vp, u32, ctypes.c_char_p, ctypes.c_size_t]
        L.tsm_lm_head_q8_workspace.restype = ctypes.c_size_t
        L.tsm_lm_head_q8_workspace.argtypes = [u32, u32]
        L.tsm_lm_head_q8.restype = ctypes.c_int
        L.tsm_lm_head_q8.argtypes = [vp, vp, u32, vp, ctypes.c_float, vp, vp, u32, u32, u32, vp, ctypes.c_size_t,
                                     vp, u32, ctypes.c_char_p, ctypes.c_size_t]
        _lib = L
    return _lib


class TsmError(RuntimeError):
    pass


def _err():
    return ctypes.create_string_buffer(1024)
