"""Python side of the fp64 CPU oracle (TEST INFRASTRUCTURE ONLY).

Only tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg import this module; the
shipped library never does. It wraps oracle/liboracle.so (oracle.c, a restatement of the
reference's fp64 oracles) and, when they were built, oracle/_ref/libref.so (the reference's own
ref_attention compiled from kernels/fa_common.hpp) and oracle/_ref/librefdrop.so (the
reference's host replica of its dropout multiplier, from kernels/backward.hip), plus the dtype
rounding and the seeded input generator the reference's gates use.

Array layouts follow oracle.c: [B, H, S, D] float32 for the forward/backward,
[B, nq, H, D] / [nblocks, page, Hk, D] for decode.
"""
import ctypes
import os
import subprocess

import numpy as np

_HERE = os.path.dirname(os.path.abspath(__file__))
_LIB = None
_REF = None
_REFDROP = None


class OracleCfg(ctypes.Structure):
    _fields_ = [("B", ctypes.c_int), ("H", ctypes.c_int), ("Hk", ctypes.c_int),
                ("SQ", ctypes.c_int), ("SK", ctypes.c_int), ("D", ctypes.c_int),
                ("scale", ctypes.c_double), ("softcap", ctypes.c_double),
                ("win_left", ctypes.c_int), ("win_right", ctypes.c_int),
                ("causal", ctypes.c_int), ("attn_chunk", ctypes.c_int),
                ("alibi", ctypes.c_void_p), ("dropout_p", ctypes.c_double),
                ("seed", ctypes.c_uint64)]


class OracleDecCfg(ctypes.Structure):
    _fields_ = [("B", ctypes.c_int), ("nq", ctypes.c_int), ("H", ctypes.c_int),
                ("Hk", ctypes.c_int), ("D", ctypes.c_int), ("page", ctypes.c_int),
                ("max_blocks", ctypes.c_int), ("scale", ctypes.c_double),
                ("softcap", ctypes.c_double), ("window", ctypes.c_int),
                ("rotary", ctypes.c_int), ("rdim", ctypes.c_int), ("append", ctypes.c_int),
                ("alibi", ctypes.c_void_p), ("round_append", ctypes.c_int)]


def build():
    """Compile liboracle.so (and _ref/libref.so when the reference tree is present)."""
    subprocess.run(["make", "-s", "-C", _HERE, "all"], check=True)


def lib():
    global _LIB
    if _LIB is None:
        path = os.path.join(_HERE, "liboracle.so")
        if not os.path.exists(path):
            build()
        _LIB = ctypes.CDLL(path)
        _LIB.oracle_rel_rms.restype = ctypes.c_double
    return _LIB


def ref_lib():
    """The reference's own ref_attention, or None when it was not built (e.g. on a GPU box)."""
    global _REF
    if _REF is None:
        path = os.path.join(_HERE, "_ref", "libref.so")
        if not os.path.exists(path):
            return None
        _REF = ctypes.CDLL(path)
    return _REF


def _p(a):
    return a.ctypes.data_as(ctypes.c_void_p) if a is not None else None


def _f32(a):
    return np.ascontiguousarray(a, dtype=np.float32)


def _f32s(x):
    """Scalars reach the kernels as C float (FwdParams/DecParams); the oracle uses the same
    rounded value so both sides evaluate the same function."""
    return float(np.float32(x))


# ----------------------------------------------------------------------------- dtype rounding
def round_bf16(x):
    """Round-to-nearest-even to bf16, returned as float32 (fa_forward_gate.inc:4-6)."""
    x = _f32(x)
    u = x.view(np.uint32).astype(np.uint64)
    r = ((u + 0x7FFF + ((u >> 16) & 1)) >> 16) << 16
    out = (r & 0xFFFFFFFF).astype(np.uint32).view(np.float32)
    return np.where(np.isnan(x), x, out)


def round_to(x, dtype):
    """Round float data to the storage dtype ('f16', 'bf16' or 'f32') and back to float32."""
    if dtype in ("f16", "fp16", "float16"):
        return _f32(x).astype(np.float16).astype(np.float32)
    if dtype in ("bf16", "bfloat16"):
        return round_bf16(x)
    return _f32(x)


# ----------------------------------------------------------------------------- seeded inputs
def frand(n, seed):
    """The reference gates' LCG stream (fa_common.hpp:140-141): s = s*1664525 + 1013904223,
    value ((s >> 16) & 4095)/4096 - 0.5. Returns (values float32[n], final state)."""
    a, c, m = 1664525, 1013904223, 1 << 32
    idx = np.arange(1, n + 1, dtype=np.uint64)
    # s_k = A_k * s0 + C_k (mod 2^32), A_k = a^k, C_k = c*(a^k-1)/(a-1) built by binary powering
    A = np.ones(n, dtype=np.uint64)
    C = np.zeros(n, dtype=np.uint64)
    pa, pc = np.uint64(a), np.uint64(c)  # affine map x -> pa*x + pc applied 2^bit times
    k = idx.copy()
    mask = np.uint64(m - 1)
    while k.any():
        sel = (k & np.uint64(1)).astype(bool)
        # compose: (A, C) <- (pa*A, pa*C + pc) for selected entries
        A = np.where(sel, (A * pa) & mask, A)
        C = np.where(sel, (C * pa + pc) & mask, C)
        pc = (pa * pc + pc) & mask
        pa = (pa * pa) & mask
        k >>= np.uint64(1)
    s = (A * np.uint64(seed & 0xFFFFFFFF) + C) & mask
    vals = ((s >> np.uint64(16)) & np.uint64(4095)).astype(np.float32) / 4096.0 - 0.5
    return vals.astype(np.float32), int(s[-1]) if n else seed


def randn(shape, seed, dtype="f16"):
    """Seeded N(0,1) data rounded to dtype (the configs' distribution)."""
    g = np.random.default_rng(seed)
    return round_to(g.standard_normal(shape, dtype=np.float32), dtype)


# ----------------------------------------------------------------------------- oracles
def philox4x32_10(ctr, key):
    """Philox4x32-10 of a 4-word counter and a 2-word key (oracle.c, Salmon et al. 2011)."""
    c = (ctypes.c_uint32 * 4)(*[int(x) & 0xFFFFFFFF for x in ctr])
    k = (ctypes.c_uint32 * 2)(*[int(x) & 0xFFFFFFFF for x in key])
    out = (ctypes.c_uint32 * 4)()
    lib().oracle_philox4x32_10(c, k, out)
    return tuple(out)


def oracle_drop_mul(seed, idx, p):
    """One dropout multiplier (oracle.c oracle_drop_mul): 0 or 1/(1-p)."""
    f = lib().oracle_drop_mul
    f.restype = ctypes.c_double
    f.argtypes = [ctypes.c_uint64, ctypes.c_uint64, ctypes.c_double]
    return f(int(seed) & ((1 << 64) - 1), int(idx), float(p))


def keep_mask(seed, p, H, SQ, SK):
    """Dropout multipliers z[h, i, j] (0 or 1/(1-p)) of the reference's scheme: Philox on
    idx = (h*SQ + i)*SK + j, key = seed, kept iff (word0 >> 8) * 2^-24 >= p (fa_common.hpp:84-88)."""
    z = np.zeros((H, SQ, SK))
    lib().oracle_dropout_mask(ctypes.c_uint64(int(seed) & ((1 << 64) - 1)), ctypes.c_double(p),
                              H, SQ, SK, _p(z))
    return z


def ref_drop_lib():
    """The reference's host replica of its dropout multiplier (hdrop), or None when
    oracle/_ref/librefdrop.so was not built (e.g. on a GPU box)."""
    global _REFDROP
    if _REFDROP is None:
        path = os.path.join(_HERE, "_ref", "librefdrop.so")
        if not os.path.exists(path):
            return None
        _REFDROP = ctypes.CDLL(path)
        _REFDROP.ref_drop_mul.restype = ctypes.c_float
        _REFDROP.ref_drop_mul.argtypes = [ctypes.c_ulonglong, ctypes.c_ulonglong, ctypes.c_float,
                                          ctypes.c_float]
    return _REFDROP


def fwd(q, k, v, scale, causal=False, win_left=-1, win_right=-1, softcap=0.0, alibi=None,
        chunk=0, rows=None, want_lse=True, dropout_p=0.0, seed=0):
    """fp64 forward oracle. q [B,H,SQ,D], k/v [B,Hk,SK,D] float32 (already dtype-rounded).
    rows: optional list of query indices to evaluate (others stay 0 / -inf). dropout_p > 0
    applies the reference's Philox dropout with `seed`."""
    q, k, v = _f32(q), _f32(k), _f32(v)
    B, H, SQ, D = q.shape
    Hk, SK = k.shape[1], k.shape[2]
    o = np.zeros_like(q)
    lse = np.full((B, H, SQ), -np.inf, dtype=np.float32) if want_lse else None
    al = _f32(alibi) if alibi is not None else None
    cfg = OracleCfg(B, H, Hk, SQ, SK, D, _f32s(scale), _f32s(softcap), int(win_left),
                    int(win_right), int(bool(causal)), int(chunk),
                    al.ctypes.data if al is not None else None, _f32s(dropout_p),
                    int(seed) & ((1 << 64) - 1))
    r = np.ascontiguousarray(rows, dtype=np.int32) if rows is not None else None
    lib().oracle_fwd(_p(q), _p(k), _p(v), _p(o), _p(lse), ctypes.byref(cfg), _p(r),
                     ctypes.c_int(len(r) if r is not None else 0))
    return o, lse


def bwd(q, k, v, do, scale, causal=False, win_left=-1, win_right=-1, softcap=0.0, alibi=None,
        chunk=0, dropout_p=0.0, seed=0, model=None, stored_o=None):
    """fp64 backward oracle: returns (dq, dk, dv) float64 with the layouts of q, k, v.
    model=None gives the exact gradients. model='f16'/'bf16' gives the rounding model of a
    backward whose matrix products take 16-bit operands (oracle.c bwd_impl): O rounded before
    D = rowsum(O*dO), z*P rounded before the dV product, dS rounded before the dK/dQ products;
    its distance from the exact gradients is the floor of any such kernel. stored_o: the
    forward output [B,H,SQ,D] a kernel stored, to take D = rowsum(O*dO) from (with model=None
    the arithmetic stays exact and only D comes from stored_o)."""
    q, k, v, do = _f32(q), _f32(k), _f32(v), _f32(do)
    B, H, SQ, D = q.shape
    Hk, SK = k.shape[1], k.shape[2]
    dq = np.zeros(q.shape, dtype=np.float64)
    dk = np.zeros(k.shape, dtype=np.float64)
    dv = np.zeros(v.shape, dtype=np.float64)
    al = _f32(alibi) if alibi is not None else None
    cfg = OracleCfg(B, H, Hk, SQ, SK, D, _f32s(scale), _f32s(softcap), int(win_left),
                    int(win_right), int(bool(causal)), int(chunk),
                    al.ctypes.data if al is not None else None, _f32s(dropout_p),
                    int(seed) & ((1 << 64) - 1))
    mode = {None: 0, "f32": 0, "f16": 1, "bf16": 2}[model]
    if mode or stored_o is not None:
        so = _f32(stored_o) if stored_o is not None else None
        lib().oracle_bwd_model(_p(q), _p(k), _p(v), _p(do), _p(dq), _p(dk), _p(dv),
                               ctypes.byref(cfg), ctypes.c_int(mode), _p(so))
    else:
        lib().oracle_bwd(_p(q), _p(k), _p(v), _p(do), _p(dq), _p(dk), _p(dv), ctypes.byref(cfg))
    return dq, dk, dv


def decode(q, k_cache, v_cache, block_table, ctx_len, scale, new_k=None, new_v=None,
           rotary_cos=None, rotary_sin=None, rotary=0, rotary_dim=0, leftpad=None,
           rotary_pos=None, window=-1, softcap=0.0, alibi=None, append_dtype=None):
    """fp64 paged-decode oracle. q [B,nq,H,D]; caches [nblocks,page,Hk,D]; block_table
    [B,max_blocks] int; ctx_len [B] (length before append). append_dtype ('f16'/'bf16') rounds
    the rotated appended keys to the cache dtype, as storing them in the cache does.
    Returns (o [B,nq,H,D], lse [B,nq,H])."""
    q = _f32(q)
    kc, vc = _f32(k_cache), _f32(v_cache)
    B, nq, H, D = q.shape
    page, Hk = kc.shape[1], kc.shape[2]
    bt = np.ascontiguousarray(block_table, dtype=np.int32)
    cl = np.ascontiguousarray(ctx_len, dtype=np.int32)
    nk = _f32(new_k) if new_k is not None else None
    nv = _f32(new_v) if new_v is not None else None
    cs = _f32(rotary_cos) if rotary_cos is not None else None
    sn = _f32(rotary_sin) if rotary_sin is not None else None
    lp = np.ascontiguousarray(leftpad, dtype=np.int32) if leftpad is not None else None
    rp = np.ascontiguousarray(rotary_pos, dtype=np.int32) if rotary_pos is not None else None
    al = _f32(alibi) if alibi is not None else None
    o = np.zeros_like(q)
    lse = np.zeros((B, nq, H), dtype=np.float32)
    cfg = OracleDecCfg(B, nq, H, Hk, D, page, bt.shape[1], _f32s(scale), _f32s(softcap),
                       int(window), int(rotary), int(rotary_dim), int(nk is not None),
                       al.ctypes.data if al is not None else None,
                       {None: 0, "f32": 0, "f16": 1, "bf16": 2}[append_dtype])
    lib().oracle_decode(_p(q), _p(kc), _p(vc), _p(bt), _p(cl), _p(nk), _p(nv), _p(cs), _p(sn),
                        _p(lp), _p(rp), _p(o), _p(lse), ctypes.byref(cfg))
    return o, lse


def combine(out_partial, lse_partial):
    """LSE-weighted merge (flash_attn_interface.py:567-580) in float64.
    out_partial [nsplit,B,S,H,D], lse_partial [nsplit,B,H,S] -> [B,S,H,D]."""
    lse = np.asarray(lse_partial, dtype=np.float64)
    m = lse.max(axis=0, keepdims=True)
    m = np.where(np.isfinite(m), m, 0.0)
    w = np.exp(lse - m)
    wsum = w.sum(axis=0)
    wt = np.transpose(w, (0, 1, 3, 2))[..., None]
    acc = (np.asarray(out_partial, dtype=np.float64) * wt).sum(axis=0)
    return acc / np.maximum(np.transpose(wsum, (0, 2, 1))[..., None], 1e-30)


def reference_fwd(q, k, v, scale, causal=False, win_left=-1, win_right=-1, softcap=0.0,
                  alibi=None, chunk=0):
    """The reference's own ref_attention (kernels/fa_common.hpp:102-134) on the same inputs.
    Batch 1 only (as the reference gate). Returns (O, LSE) in oracle layouts, or None when
    oracle/_ref was not built."""
    rl = ref_lib()
    if rl is None:
        return None
    q, k, v = _f32(q), _f32(k), _f32(v)
    B, H, SQ, D = q.shape
    assert B == 1
    Hk, SK = k.shape[1], k.shape[2]
    Q = np.ascontiguousarray(q[0].transpose(1, 0, 2))  # [SQ][NH][HD]
    K = np.ascontiguousarray(k[0])                      # [NKV][SK][HD]
    V = np.ascontiguousarray(v[0])
    O = np.zeros_like(Q)
    L = np.zeros((H, SQ), dtype=np.float32)
    al = _f32(alibi) if alibi is not None else None
    rl.ref_fwd(_p(Q), _p(K), _p(V), _p(O), _p(L), SQ, SK, D, H, H // Hk,
               ctypes.c_float(scale), ctypes.c_float(softcap), win_left, win_right,
               int(bool(causal)), _p(al), chunk)
    return O.transpose(1, 0, 2)[None].copy(), L[None].copy()


def rel_rms(got, ref):
    """||got-ref||_2 / ||ref||_2 (fa_common.hpp:136-139), in float64."""
    g = np.asarray(got, dtype=np.float64).ravel()
    r = np.asarray(ref, dtype=np.float64).ravel()
    den = np.sqrt((r * r).sum())
    num = np.sqrt(((g - r) ** 2).sum())
    return float(num / den) if den > 0 else float(num)
