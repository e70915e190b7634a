"""ctypes view of the C-ABI in include/fable_attn_abi.h.

The structs below mirror the header field for field (tests/test_abi.py compiles the header with
gcc and compares every offset): the extended Fable* structs the binding uses, and the
reference-layout Ref* structs of the reference's own launchers. The library is loaded after torch so that the HIP runtime torch
already mapped is the one the library binds to (both carry the soname libamdhip64.so.7).
"""
import ctypes
import os

import torch  # noqa: F401  (must be imported before the HIP library is loaded)

_HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(_HERE, "libfable_attn_hip.so")

FA_F16, FA_BF16, FA_F32 = 0, 1, 2
FA_OK = 0

ABI_VERSION = 5  # FABLE_ATTN_ABI_VERSION of include/fable_attn_abi.h

c_i32, c_i64, c_u64, c_f32, c_ptr = (ctypes.c_int32, ctypes.c_int64, ctypes.c_uint64,
                                     ctypes.c_float, ctypes.c_void_p)
c_int, c_ll, c_ull = ctypes.c_int, ctypes.c_longlong, ctypes.c_ulonglong


class Strides(ctypes.Structure):
    _fields_ = [("b", c_i64), ("h", c_i64), ("s", c_i64)]


class FableFwdParams(ctypes.Structure):
    _fields_ = [("Q", c_ptr), ("K", c_ptr), ("V", c_ptr), ("O", c_ptr), ("LSE", c_ptr),
                ("sQ", Strides), ("sK", Strides), ("sV", Strides), ("sO", Strides),
                ("SQ", c_i32), ("SK", c_i32), ("HD", c_i32), ("NH", c_i32), ("gqa", c_i32),
                ("scale", c_f32), ("softcap", c_f32),
                ("win_left", c_i32), ("win_right", c_i32),
                ("alibi_slopes", c_ptr), ("causal", c_i32), ("dropout_p", c_f32),
                ("philox_seed", c_u64), ("cu_q", c_ptr), ("cu_k", c_ptr), ("batch", c_i32),
                ("attn_chunk", c_i32), ("seqused_q", c_ptr), ("seqused_k", c_ptr),
                ("lse_sb", c_i64), ("lse_sh", c_i64)]


class FableBwdParams(ctypes.Structure):
    _fields_ = [("Q", c_ptr), ("K", c_ptr), ("V", c_ptr), ("O", c_ptr), ("dO", c_ptr),
                ("dQ", c_ptr), ("dK", c_ptr), ("dV", c_ptr), ("lse", c_ptr), ("dsum", c_ptr),
                ("qs", Strides), ("ks", Strides), ("vs", Strides), ("os", Strides),
                ("dos", Strides), ("dqs", Strides), ("dks", Strides), ("dvs", Strides),
                ("B", c_i32), ("Hq", c_i32), ("Hk", c_i32), ("SQ", c_i32), ("SK", c_i32),
                ("D", c_i32), ("gqa", c_i32), ("scale", c_f32), ("softcap", c_f32),
                ("alibi", c_ptr), ("causal", c_i32), ("win_left", c_i32), ("win_right", c_i32),
                ("dropout", c_i32), ("drop_seed", c_u64), ("dropout_p", c_f32),
                ("keep_scale", c_f32), ("cu_q", c_ptr), ("cu_k", c_ptr), ("seqused_q", c_ptr),
                ("seqused_k", c_ptr), ("lse_sb", c_i64), ("lse_sh", c_i64),
                ("ds_ws", c_ptr), ("ds_ws_bytes", c_i64)]


class FableDecParams(ctypes.Structure):
    _fields_ = [("q", c_ptr), ("Kc", c_ptr), ("Vc", c_ptr), ("block_table", c_ptr),
                ("o", c_ptr), ("scratch", c_ptr), ("ctx_len", c_ptr), ("cos", c_ptr),
                ("sin", c_ptr), ("batch", c_i32), ("NH", c_i32), ("gqa", c_i32), ("HD", c_i32),
                ("page", c_i32), ("max_blocks", c_i32), ("nsplit", c_i32), ("window", c_i32),
                ("rotary", c_i32), ("scale", c_f32), ("leftpad", c_ptr), ("lse_out", c_ptr),
                ("softcap", c_f32), ("alibi", c_ptr), ("nq", c_i32), ("rotary_dim", c_i32),
                ("rotary_pos", c_ptr)]


class CombineParams(ctypes.Structure):
    _fields_ = [("out_partial", c_ptr), ("lse_partial", c_ptr), ("out", c_ptr),
                ("nsplit", c_i32), ("B", c_i32), ("S", c_i32), ("H", c_i32), ("D", c_i32),
                ("op_split", c_i64), ("op_b", c_i64), ("op_seq", c_i64), ("op_h", c_i64),
                ("lp_split", c_i64), ("lp_b", c_i64), ("lp_h", c_i64), ("lp_seq", c_i64),
                ("in_dtype", c_i32), ("out_dtype", c_i32)]


# The reference's layouts (package/csrc/fa_iface.h:9-63), taken by fa_forward_launch,
# fable_attn_backward_launch and fa_decode_launch.
class RefStrides(ctypes.Structure):
    _fields_ = [("b", c_ll), ("h", c_ll), ("s", c_ll)]


class RefFwdParams(ctypes.Structure):
    _fields_ = [("Q", c_ptr), ("K", c_ptr), ("V", c_ptr), ("O", c_ptr), ("LSE", c_ptr),
                ("sQ", RefStrides), ("sK", RefStrides), ("sV", RefStrides), ("sO", RefStrides),
                ("SQ", c_int), ("SK", c_int), ("HD", c_int), ("NH", c_int), ("gqa", c_int),
                ("scale", c_f32), ("softcap", c_f32), ("win_left", c_int), ("win_right", c_int),
                ("alibi_slopes", c_ptr), ("causal", c_int), ("dropout_p", c_f32),
                ("philox_seed", c_ull), ("cu_q", c_ptr), ("cu_k", c_ptr), ("batch", c_int),
                ("sc_q", c_f32), ("sc_k", c_f32), ("sc_v", c_f32), ("attn_chunk", c_int),
                ("seqused_q", c_ptr), ("seqused_k", c_ptr)]


class RefBwdParams(ctypes.Structure):
    _fields_ = [("Q", c_ptr), ("K", c_ptr), ("V", c_ptr), ("O", c_ptr), ("dO", c_ptr),
                ("dQ", c_ptr), ("dK", c_ptr), ("dV", c_ptr), ("lse", c_ptr), ("dsum", c_ptr),
                ("qs", RefStrides), ("ks", RefStrides), ("vs", RefStrides), ("os", RefStrides),
                ("dos", RefStrides), ("dqs", RefStrides), ("dks", RefStrides),
                ("dvs", RefStrides),
                ("B", c_int), ("Hq", c_int), ("Hk", c_int), ("SQ", c_int), ("SK", c_int),
                ("D", c_int), ("gqa", c_int), ("scale", c_f32), ("softcap", c_f32),
                ("alibi", c_ptr), ("causal", c_int), ("win_left", c_int), ("win_right", c_int),
                ("dropout", c_int), ("drop_seed", c_ull), ("dropout_p", c_f32),
                ("keep_scale", c_f32), ("shQ", c_int), ("shK", c_int), ("shV", c_int),
                ("shdO", c_int)]


class RefDecParams(ctypes.Structure):
    _fields_ = [("q", c_ptr), ("Kc", c_ptr), ("Vc", c_ptr), ("block_table", c_ptr),
                ("o", c_ptr), ("scratch", c_ptr), ("ctx_len", c_ptr), ("cos", c_ptr),
                ("sin", c_ptr), ("batch", c_int), ("NH", c_int), ("gqa", c_int), ("HD", c_int),
                ("page", c_int), ("max_blocks", c_int), ("nsplit", c_int), ("window", c_int),
                ("page_shift", c_int), ("page_mask", c_int), ("rotary", c_int),
                ("scale", c_f32), ("sc_q", c_f32), ("sc_k", c_f32), ("sc_v", c_f32),
                ("leftpad", c_ptr), ("lse_out", c_ptr), ("softcap", c_f32), ("alibi", c_ptr),
                ("nq", c_int), ("append", c_int), ("rotary_dim", c_int), ("rotary_pos", c_ptr)]


STRUCTS = {0: FableFwdParams, 1: FableBwdParams, 2: FableDecParams, 3: CombineParams,
           4: Strides, 5: RefFwdParams, 6: RefBwdParams, 7: RefDecParams}

# exported symbols of libfable_attn_hip.so (the C-ABI surface)
EXPORTS = ("fa_forward_launch", "fable_attn_backward_launch", "fa_decode_launch",
           "fable_attn_fwd", "fable_attn_fwd_ws", "fable_attn_fwd_ws_bytes", "fable_attn_bwd", "fable_attn_dec", "fable_attn_dec_noalloc",
           "fable_attn_dec_noalloc_max_floats",
           "fa_decode_num_splits", "fa_combine_launch", "fable_attn_bwd_ds_bytes",
           "fable_attn_abi_version", "fable_attn_struct_size", "fable_attn_last_error")

_lib = None


def load():
    """Load the library once; raises ImportError when it has not been built."""
    global _lib
    if _lib is not None:
        return _lib
    if not os.path.exists(LIB_PATH):
        raise ImportError(
            f"fable_attn: {LIB_PATH} is missing; build it with "
            "`python flash-attention-rdna2_amd/build.py` (no CPU fallback exists)")
    lib = ctypes.CDLL(LIB_PATH)
    lib.fable_attn_fwd.argtypes = [FableFwdParams, c_i32, c_ptr]
    lib.fable_attn_fwd_ws.argtypes = [FableFwdParams, c_i32, c_ptr, c_i64, c_ptr]
    lib.fable_attn_fwd_ws_bytes.argtypes = [FableFwdParams, c_i32]
    lib.fable_attn_fwd_ws_bytes.restype = c_i64
    lib.fable_attn_bwd.argtypes = [FableBwdParams, c_i32, c_ptr]
    lib.fable_attn_dec.argtypes = [FableDecParams, c_i32, c_ptr, c_ptr, c_ptr]
    lib.fa_decode_num_splits.argtypes = [c_i32, c_i32, c_i32, c_i32, c_i64, c_i32]
    lib.fa_combine_launch.argtypes = [CombineParams, c_ptr]
    lib.fa_forward_launch.argtypes = [RefFwdParams, c_i32, c_ptr]
    lib.fable_attn_backward_launch.argtypes = [RefBwdParams, c_i32, c_ptr]
    lib.fa_decode_launch.argtypes = [RefDecParams, c_i32, c_ptr, c_ptr, c_ptr]
    lib.fable_attn_dec_noalloc.argtypes = [FableDecParams, c_i32, c_ptr, c_ptr, c_ptr]
    lib.fable_attn_dec_noalloc_max_floats.restype = c_i64
    for f in ("fable_attn_fwd", "fable_attn_fwd_ws", "fable_attn_bwd", "fable_attn_dec", "fable_attn_dec_noalloc",
              "fa_forward_launch",
              "fable_attn_backward_launch", "fa_decode_launch",
              "fa_decode_num_splits", "fa_combine_launch", "fable_attn_abi_version"):
        getattr(lib, f).restype = c_i32
    lib.fable_attn_bwd_ds_bytes.argtypes = [FableBwdParams, c_i32]
    lib.fable_attn_bwd_ds_bytes.restype = c_i64
    lib.fable_attn_struct_size.argtypes = [c_i32]
    lib.fable_attn_struct_size.restype = ctypes.c_size_t
    lib.fable_attn_last_error.restype = ctypes.c_char_p
    if lib.fable_attn_abi_version() != ABI_VERSION:
        raise ImportError("fable_attn: ABI version mismatch between library and binding")
    for k, st in STRUCTS.items():
        if lib.fable_attn_struct_size(k) != ctypes.sizeof(st):
            raise ImportError(f"fable_attn: struct {st.__name__} size mismatch "
                              f"({lib.fable_attn_struct_size(k)} vs {ctypes.sizeof(st)})")
    _lib = lib
    return lib


def check(rc, what):
    """Raise RuntimeError carrying the library's message for a failed launch."""
    if rc != FA_OK:
        msg = _lib.fable_attn_last_error().decode(errors="replace") if _lib else ""
        raise RuntimeError(f"fable_attn: {what} failed (status {rc}): {msg}")
