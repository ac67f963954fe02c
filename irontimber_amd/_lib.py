"""ctypes binding of libit_attn.so, the C ABI declared in include/it_attn.h.

The library is the only compute path: if it is missing, loading raises instead of falling back.
"""
from __future__ import annotations

import ctypes
import os
from ctypes import c_float, c_int, c_size_t, c_uint32, c_void_p, c_char_p

LIB_PATH = os.path.join(os.path.dirname(os.path.abspath(__file__)), "lib", "libit_attn.so")

# name -> (restype, argtypes); pointers travel as c_void_p (device addresses as ints).
P = c_void_p
SIGNATURES = {
    "it_last_error": (c_char_p, []),
    "it_abi_version": (c_int, []),
    "it_kv_append_f16": (c_int, [P, P, c_int, P, P, c_int, c_int, c_int, c_int, P]),
    "it_attn_prep_f16": (c_int, [P, c_int, P, P, c_int, P, P, c_float, P, P, c_int, c_int, c_int, c_int, c_int, c_int,
                                 c_int, c_float, c_int, c_int, c_int, c_int, c_int, P]),
    "it_attn_prep_f16_q16": (c_int, [P, c_int, P, P, c_int, P, P, c_float, P, P, c_int, c_int, c_int, c_int, c_int,
                                     c_int, c_int, c_float, c_int, c_int, c_int, c_int, c_int, P, c_int, c_float, P]),
    "it_attn_f16_q16": (c_int, [P, c_int, P, c_int, P, P, c_int, c_int, c_int, c_int, c_int, c_int, c_float, P, c_int,
                                P, c_size_t, P]),
    "it_attn_prep_f32kv": (c_int, [P, c_int, P, P, c_int, P, P, c_float, P, P, c_int, c_int, c_int, c_int, c_int,
                                   c_int, c_int, c_int, c_float, c_int, c_int, c_int, c_int, P]),
    "it_attn_f32kv_scratch_bytes": (c_size_t, [c_int, c_int, c_int, c_int, c_int]),
    "it_attn_f32kv_plan": (c_int, [c_int, c_int, c_int, c_int, c_int, c_size_t, P, P]),
    "it_attn_f32kv": (c_int, [P, c_int, P, P, c_int, c_int, c_int, c_int, c_int, c_int, c_float, P, c_int, P, c_size_t,
                              P]),
    "it_attn_scratch_bytes": (c_size_t, [c_int, c_int, c_int, c_int, c_int]),
    "it_calib_mfma_f16": (c_int, [c_int, c_int, P, P]),
    "it_attn_f16": (c_int, [P, c_int, P, P, c_int, c_int, c_int, c_int, c_int, c_int, c_float, P, c_int, P, c_size_t, P]),
    "it_attn_scratch_bytes_ex": (c_size_t, [c_int, c_int, c_int, c_int, c_int, c_int, c_int]),
    "it_attn_f16_ex": (c_int, [P, c_int, P, P, c_int, c_int, c_int, c_int, c_int, c_int, c_float, P, c_int, P, c_size_t,
                               c_int, c_int, P]),
    "it_attn_partials": (c_int, [P, c_int, P, P, c_int, c_int, c_int, c_int, c_int, c_int, c_float, P, c_size_t, c_int,
                                 P]),
    "it_attn_combine": (c_int, [P, c_int, P, c_int, c_int, c_int, c_int, c_int, P, c_int, P]),
    "it_attn_partials_ex": (c_int, [P, c_int, P, P, c_int, c_int, c_int, c_int, c_int, c_int, c_float, P, c_size_t,
                                    c_int, c_int, P]),
    "it_attn_combine_ex": (c_int, [P, c_int, P, c_int, c_int, c_int, c_int, c_int, c_int, P, c_int, P]),
    "it_gdn_conv": (c_int, [P, c_int, P, P, P, c_int, c_int, c_int, c_int, P]),
    "it_l2norm_heads": (c_int, [P, c_int, c_int, c_int, c_int, c_float, P]),
    "it_gdn_conv_l2norm": (c_int, [P, c_int, P, P, P, c_int, c_int, c_int, c_int, c_int, c_float, P]),
    "it_gdn_step": (c_int, [P, c_int, P, P, c_int, P, P, P, P, c_int, c_int, c_int, c_int, c_int, P]),
    "it_gdn_decode_fused": (c_int, [P, c_int, P, c_int, P, P, P, P, c_int, P, P, P, P, c_int, c_int, c_int, c_int, c_int,
                                    c_float, P]),
    "it_gdn_decode_fused_ckpt": (c_int, [P, c_int, P, c_int, P, P, P, P, c_int, P, P, P, P, c_int, c_int, c_int, c_int,
                                         c_int, c_float, P, P, c_int, P]),
    "it_gdn_conv_ckpt": (c_int, [P, c_int, P, P, P, c_int, c_int, c_int, c_int, P, c_int, P]),
    "it_gdn_conv_l2norm_ckpt": (c_int, [P, c_int, P, P, P, c_int, c_int, c_int, c_int, c_int, c_float, P, c_int, P]),
    "it_gdn_step_ckpt": (c_int, [P, c_int, P, P, c_int, P, P, P, P, c_int, c_int, c_int, c_int, c_int, P, c_int, P]),
    "it_gdn_step_gated": (c_int, [P, c_int, P, P, c_int, P, P, P, P, c_int, c_int, c_int, c_int, c_int, P, c_int, P,
                                  c_float, P, c_int, P]),
    "it_gdn_gated_rmsnorm": (c_int, [P, c_int, P, c_int, P, c_float, P, c_int, c_int, c_int, c_int, P]),
    "it_gdn_rollback": (c_int, [P, P, c_size_t, P, P, c_size_t, P]),
    "it_gdn_chunked_scratch_bytes": (c_size_t, [c_int, c_int, c_int]),
    "it_gdn_chunked": (c_int, [P, c_int, P, P, c_int, P, P, P, P, c_int, c_int, c_int, c_int, c_int, P, c_size_t, P]),
    "it_attention_scratch_words": (c_size_t, [c_size_t, c_size_t]),
    "it_attention_dispatch_room": (c_size_t, [c_size_t, c_size_t, c_size_t]),
    "it_attention_chunk": (c_int, [c_uint32, c_uint32, c_uint32, c_size_t]),
    "it_validate_geometry": (c_int, [c_int] * 9),
    "it_attn_f16_noalloc": (c_int, [P, c_int, P, P, c_int, c_int, c_int, c_int, c_int, c_int, c_float, P, c_int, P]),
    "it_gdn_prefill_scratch_bytes": (c_size_t, [c_int, c_int, c_int, c_int]),
    "it_gdn_prefill": (c_int, [P, c_int, P, c_int, P, P, P, c_int, P, P, P, P, c_int, c_int, c_int, c_int, c_int,
                               c_float, P, c_size_t, P]),
    "it_attn_mailbox_bytes": (c_size_t, [c_int, c_int, c_int]),
    "it_attn_mailbox_init": (c_int, [P, c_size_t, P]),
    "it_attn_mailbox_would_launch": (c_int, [c_int, c_int, c_int, c_int, c_int, c_size_t]),
    "it_attn_mailbox_poisoned": (c_int, [P, P, P]),
    "it_attn_f16_mailbox": (c_int, [P, c_int, P, P, c_int, c_int, c_int, c_int, c_int, c_int, c_float, P, c_int, P,
                                    c_size_t, P, c_size_t, P]),
    "it_attn_plan": (c_int, [c_int, c_int, c_int, c_int, c_int, c_size_t, P, P, P]),
    "it_prefill_chunks": (ctypes.c_long, [c_size_t, c_size_t, P, P, c_size_t]),
}


class ItError(RuntimeError):
    """A nonzero return from the C ABI, carrying it_last_error()."""


_lib = None


def lib() -> ctypes.CDLL:
    global _lib
    if _lib is None:
        if not os.path.exists(LIB_PATH):
            raise ItError(f"{LIB_PATH} is not built; run __graft_entry__.build() (make -C irontimber_amd/csrc)")
        handle = ctypes.CDLL(LIB_PATH)
        for name, (res, args) in SIGNATURES.items():
            fn = getattr(handle, name)
            fn.restype, fn.argtypes = res, args
        _lib = handle
    return _lib


def last_error() -> str:
    return lib().it_last_error().decode()


def call(name: str, *args) -> int:
    """Call an int-returning entry point; raise ItError with the library's message on failure."""
    rc = getattr(lib(), name)(*args)
    if rc != 0:
        raise ItError(f"{name}: {last_error()}")
    return rc
