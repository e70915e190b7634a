"""Host glue between torch tensors and the C-ABI launchers (the reference's `_C` module).

Mirrors the functions of the reference's pybind module (package/csrc/dispatch.cpp:35-231,
bound at :239-268) with the same names, argument order and meaning:
    fwd(q, k, v, scale, causal, win_left, win_right, softcap, alibi, dropout_p, seed,
        attn_chunk=0, out=None) -> (out, lse)
    bwd(dout, q, k, v, out, lse, scale, causal, win_left, win_right, softcap, alibi,
        dropout_p, seed, ds_max_bytes=None) -> (dq, dk, dv)
    bwd_varlen(dout, q, k, v, out, lse, cu_q, cu_k, max_sq, max_sk, scale, causal, win_left,
               win_right, softcap, alibi, dropout_p, seed, seqused_q=None, seqused_k=None,
               ds_max_bytes=None)
        -> (dq, dk, dv)   (no counterpart in the reference's _C: native varlen backward)
    fwd_varlen(q, k, v, cu_q, cu_k, max_sq, max_sk, scale, causal, win_left, win_right,
               softcap, alibi, dropout_p, seed, attn_chunk=0, seqused_q=None,
               seqused_k=None, return_lse=False) -> out  (or (out, lse) when return_lse)
    dec(q, k_cache, v_cache, block_table, cache_seqlens, new_k, new_v, rotary_cos,
        rotary_sin, rotary_interleaved, scale, window, num_splits, cache_leftpad=None,
        return_lse=False, softcap=0.0, alibi=None, rotary_dim=0, rotary_pos=None) -> (out, lse)
    combine(out_partial, lse_partial, out_dtype) -> out
Tensor checks raise RuntimeError as TORCH_CHECK does there. torch only allocates outputs and
workspaces and supplies the current stream; all compute is in libfable_attn_hip.so. There is
no fallback: if the library is missing, importing this module raises ImportError.

Backward dS workspace: for fp16/bf16 at every head dim the backward can store dS once and
form dQ = dS.K from it (FableBwdParams.ds_ws) instead of recomputing S and dP in its dQ kernel. The
workspace holds 2 bytes per visible (query, key) pair of every q head, in 32x32 tiles (about half
of B*Hq*SQ*SK*2 bytes under a causal mask; packed varlen batches keep the rectangle of the longest
sequences); bwd/bwd_varlen allocate it when it is at most `ds_max_bytes` (default
BWD_DS_MAX_BYTES, 16 GiB, or the environment variable FABLE_ATTN_BWD_DS_MAX_BYTES) and fall back
to the recomputing path when the allocation fails. Both paths give the same gradients to
rounding.
"""
import contextlib
import ctypes
import os

import torch

from . import _lib
from ._lib import FableBwdParams, CombineParams, FableDecParams, FableFwdParams, Strides

_L = _lib.load()

BWD_DS_MAX_BYTES = int(os.environ.get("FABLE_ATTN_BWD_DS_MAX_BYTES", 16 << 30))


def _ds_workspace(p, dtype, device, ds_max_bytes):
    """Attach a dS workspace to FableBwdParams p when the library has a path for it and it fits the
    cap; returns the tensor (kept alive by the caller until the launch is enqueued)."""
    cap = BWD_DS_MAX_BYTES if ds_max_bytes is None else int(ds_max_bytes)
    need = int(_L.fable_attn_bwd_ds_bytes(p, dtype))
    if need <= 0 or need > cap:
        return None
    try:
        ws = torch.empty(need, dtype=torch.uint8, device=device)
    except torch.cuda.OutOfMemoryError:
        return None  # the recomputing path needs no workspace
    if ws.data_ptr() % 16:  # (the caching allocator aligns; an unaligned buffer is not used)
        return None
    p.ds_ws, p.ds_ws_bytes = ws.data_ptr(), need
    return ws


def _req(cond, msg):
    if not cond:
        raise RuntimeError("fable_attn: " + msg)


def _dt(t):
    if t.dtype == torch.float16:
        return _lib.FA_F16
    if t.dtype == torch.bfloat16:
        return _lib.FA_BF16
    if t.dtype == torch.float32:
        return _lib.FA_F32
    raise RuntimeError(f"fable_attn: dtype {t.dtype} not supported")


def _ptr(t):
    return ctypes.c_void_p(t.data_ptr()) if t is not None else None


def _on(dev):
    """The device context of a launch: a no-op when dev is already current (the common case;
    entering torch.cuda.device costs microseconds per call)."""
    if dev.index == torch.cuda.current_device():
        return contextlib.nullcontext()
    return torch.cuda.device(dev)


def _stream(t):
    """The current stream of t's device as a raw handle (the torch call that returns the handle
    directly costs a fraction of building a Stream object; the public call is the fallback)."""
    try:
        return ctypes.c_void_p(torch._C._cuda_getCurrentRawStream(t.device.index))
    except AttributeError:
        return ctypes.c_void_p(torch.cuda.current_stream(t.device).cuda_stream)


def _bhs(t):
    """(b, h, s) element strides of a [B,H,S,D] view."""
    return Strides(t.stride(0), t.stride(1), t.stride(2))


def _rows_aligned(t):
    """16-byte aligned rows with a contiguous head_dim: what the kernels' vector loads need."""
    st, el = t.stride(), t.element_size()
    if st[-1] != 1 or t.data_ptr() % 16:
        return False
    acc = 0
    for x in st[:-1]:
        acc |= x * el
    return acc % 16 == 0


def _check_index(name, t, dev, n=None, at_least=False):
    """int32 index tensor on `dev`, contiguous (the kernels read it through a raw pointer),
    with exactly (or at least) n entries."""
    _req(torch.is_tensor(t), f"{name}: tensor expected")
    _req(t.dtype == torch.int32, f"{name}: int32 expected, got {t.dtype}")
    _req(t.device == dev, f"{name}: must be on {dev}, got {t.device}")
    _req(t.is_contiguous(), f"{name}: must be contiguous")
    if n is not None:
        _req(t.numel() >= n if at_least else t.numel() == n,
             f"{name}: {'at least ' if at_least else ''}{n} entries expected, got {t.numel()}")


def _check_f32(name, t, dev, n=None):
    """float32 side input (alibi slopes, rotary tables) on `dev`, contiguous."""
    _req(torch.is_tensor(t), f"{name}: tensor expected")
    _req(t.dtype == torch.float32, f"{name}: float32 expected, got {t.dtype}")
    _req(t.device == dev, f"{name}: must be on {dev}, got {t.device}")
    _req(t.is_contiguous(), f"{name}: must be contiguous")
    if n is not None:
        _req(t.numel() == n, f"{name}: {n} entries expected, got {t.numel()}")


def _check_varlen_index(q, cu_q, cu_k, seqused_q, seqused_k):
    batch = cu_q.numel() - 1
    _req(batch >= 0, "cu_seqlens_q must have batch+1 entries")
    _check_index("cu_seqlens_q", cu_q, q.device)
    _check_index("cu_seqlens_k", cu_k, q.device, cu_q.numel())
    if seqused_q is not None:
        _check_index("seqused_q", seqused_q, q.device, batch)
    if seqused_k is not None:
        _check_index("seqused_k", seqused_k, q.device, batch)
    return batch


def _alibi(alibi, H, dev):
    """alibi slopes as float32 [H] on dev (converted, as the public API passes them)."""
    if alibi is None:
        return None
    _req(torch.is_tensor(alibi) and alibi.device == dev, f"alibi_slopes must be on {dev}")
    al = alibi.to(torch.float32).contiguous()
    _req(al.numel() == H, f"alibi_slopes: {H} entries (one per q head) expected, got {al.numel()}")
    return al


def _check_bhsd(name, t, dtype, dev):
    if t.dim() == 4 and t.dtype == dtype and t.is_cuda and t.device == dev and _rows_aligned(t):
        return  # (the common case, checked in one pass; the messages below name the failure)
    _req(t.is_cuda, f"{name}: GPU tensor required")
    _req(t.dim() == 4, f"{name}: expected [B,H,S,D]")
    _req(t.dtype == dtype, f"{name}: dtype {t.dtype} differs from q ({dtype})")
    _req(t.device == dev, f"{name}: device mismatch")
    _req(_rows_aligned(t), f"{name}: head_dim must be contiguous with 16-byte aligned rows")


def fwd(q, k, v, scale, causal, win_left, win_right, softcap, alibi, dropout_p, seed,
        attn_chunk=0, out=None):
    """q [B,Hq,SQ,D], k/v [B,Hk,SK,D] (strided views). Returns (out, lse [B,Hq,SQ] fp32).
    Reference: dispatch.cpp:35-80 (one launch here; the reference looped over the batch)."""
    B, Hq, SQ, D = q.shape
    Hk, SK = k.shape[1], k.shape[2]
    for n, t in (("q", q), ("k", k), ("v", v)):
        _check_bhsd(n, t, q.dtype, q.device)
    _req(k.shape[0] == B and v.shape == k.shape and k.shape[3] == D, "k/v shape mismatch")
    _req(Hq % Hk == 0, "Hq must be a multiple of Hk (GQA)")
    if out is None:
        out = torch.empty((B, SQ, Hq, D), dtype=q.dtype, device=q.device).transpose(1, 2)
    else:
        _req(tuple(out.shape) == tuple(q.shape), "out must have the shape of q [B,H,SQ,D]")
        _req(out.dtype == q.dtype, "out must have the dtype of q")
        _req(_rows_aligned(out), "out: head_dim must be contiguous with 16-byte aligned rows")
    lse = torch.empty((B, Hq, SQ), dtype=torch.float32, device=q.device)
    al = _alibi(alibi, Hq, q.device)
    # (one positional construction: a fraction of the host time of 30 field assignments)
    p = FableFwdParams(q.data_ptr(), k.data_ptr(), v.data_ptr(), out.data_ptr(), lse.data_ptr(),
                       _bhs(q), _bhs(k), _bhs(v), _bhs(out), SQ, SK, D, Hq, Hq // Hk,
                       float(scale), float(softcap), int(win_left), int(win_right),
                       al.data_ptr() if al is not None else None, 1 if causal else 0,
                       float(dropout_p), int(seed) & ((1 << 64) - 1), None, None, B, int(attn_chunk),
                       None, None, Hq * SQ, SQ)
    with _on(q.device):
        _launch_fwd(p, _dt(q), q.device, _stream(q))
    return out, lse


def _launch_fwd(p, dt, device, stream, ws_bytes=None):
    """fable_attn_fwd, or fable_attn_fwd_ws with a fresh workspace when the library splits this
    call's keys (a small grid); ws_bytes: the library's answer, when the caller has it cached."""
    if ws_bytes is None:
        ws_bytes = _L.fable_attn_fwd_ws_bytes(p, dt)
    if ws_bytes > 0:
        ws = torch.empty(ws_bytes, dtype=torch.uint8, device=device)
        _lib.check(_L.fable_attn_fwd_ws(p, dt, ws.data_ptr(), ws_bytes, stream), "fable_attn_fwd")
    else:
        _lib.check(_L.fable_attn_fwd(p, dt, stream), "fable_attn_fwd")


def fwd_varlen(q, k, v, cu_q, cu_k, max_sq, max_sk, scale, causal, win_left, win_right, softcap,
               alibi, dropout_p, seed, attn_chunk=0, seqused_q=None, seqused_k=None,
               return_lse=False):
    """q (total_q, Hq, D), k/v (total_k, Hk, D), cu_* int32 [batch+1]. One launch for all
    sequences; LSE [Hq, total_q] is produced on request (the reference wrote none,
    dispatch.cpp:116,139). Reference: dispatch.cpp:117-157."""
    _req(q.is_cuda and k.is_cuda and v.is_cuda, "GPU tensors required")
    _req(q.dim() == 3 and k.dim() == 3 and v.dim() == 3, "varlen expects [total, H, D]")
    Hq, D, Hk = q.shape[1], q.shape[2], k.shape[1]
    _req(Hq % Hk == 0, "Hq must be a multiple of Hk (GQA)")
    for n, t in (("q", q), ("k", k), ("v", v)):
        _req(t.dtype == q.dtype, f"{n}: dtype mismatch")
        _req(_rows_aligned(t), f"{n}: head_dim must be contiguous with 16-byte aligned rows")
    _req(k.device == q.device and v.device == q.device, "q, k, v must be on one device")
    _req(k.shape[2] == D and v.shape[:2] == k.shape[:2], "k/v shape mismatch")
    batch = _check_varlen_index(q, cu_q, cu_k, seqused_q, seqused_k)
    out = torch.zeros_like(q) if seqused_q is not None else torch.empty_like(q)
    lse = torch.empty((Hq, q.shape[0]), dtype=torch.float32, device=q.device) if return_lse else None
    al = _alibi(alibi, Hq, q.device)
    p = FableFwdParams()
    p.Q, p.K, p.V, p.O = q.data_ptr(), k.data_ptr(), v.data_ptr(), out.data_ptr()
    p.LSE = lse.data_ptr() if lse is not None else None
    p.sQ = Strides(0, q.stride(1), q.stride(0))
    p.sK = Strides(0, k.stride(1), k.stride(0))
    p.sV = Strides(0, v.stride(1), v.stride(0))
    p.sO = Strides(0, out.stride(1), out.stride(0))
    p.SQ, p.SK, p.HD, p.NH, p.gqa = int(max_sq), int(max_sk), D, Hq, Hq // Hk
    p.scale, p.softcap = float(scale), float(softcap)
    p.win_left, p.win_right = int(win_left), int(win_right)
    p.alibi_slopes = al.data_ptr() if al is not None else None
    p.causal = 1 if causal else 0
    p.dropout_p, p.philox_seed = float(dropout_p), int(seed) & ((1 << 64) - 1)
    p.cu_q, p.cu_k = cu_q.data_ptr(), cu_k.data_ptr()
    p.batch = batch
    p.attn_chunk = int(attn_chunk)
    p.seqused_q = seqused_q.data_ptr() if seqused_q is not None else None
    p.seqused_k = seqused_k.data_ptr() if seqused_k is not None else None
    p.lse_sb, p.lse_sh = 0, q.shape[0]
    with _on(q.device):
        _launch_fwd(p, _dt(q), q.device, _stream(q))
    return (out, lse) if return_lse else out


def bwd(dout, q, k, v, out, lse, scale, causal, win_left, win_right, softcap, alibi, dropout_p,
        seed, ds_max_bytes=None):
    """All tensors [B,H,S,D] views (D contiguous); lse [B,Hq,SQ] fp32. Returns (dq, dk, dv)
    with the (B,S,H,D)-dense memory of the public API, viewed as [B,H,S,D].
    Reference: dispatch.cpp:83-111 (no bf16 .item() host syncs here)."""
    B, Hq, SQ, D = q.shape
    Hk, SK = k.shape[1], k.shape[2]
    for n, t in (("dout", dout), ("q", q), ("k", k), ("v", v), ("out", out)):
        _check_bhsd(n, t, q.dtype, q.device)
    _req(lse.dtype == torch.float32 and lse.is_contiguous() and tuple(lse.shape) == (B, Hq, SQ)
         and lse.device == q.device, "lse must be contiguous fp32 [B,Hq,SQ] on q's device")
    dq = torch.empty((B, SQ, Hq, D), dtype=q.dtype, device=q.device).transpose(1, 2)
    dk = torch.empty((B, SK, Hk, D), dtype=k.dtype, device=q.device).transpose(1, 2)
    dv = torch.empty((B, SK, Hk, D), dtype=v.dtype, device=q.device).transpose(1, 2)
    dsum = torch.empty((B, Hq, SQ), dtype=torch.float32, device=q.device)
    al = _alibi(alibi, Hq, q.device)
    p = FableBwdParams()
    p.Q, p.K, p.V, p.O, p.dO = q.data_ptr(), k.data_ptr(), v.data_ptr(), out.data_ptr(), dout.data_ptr()
    p.dQ, p.dK, p.dV = dq.data_ptr(), dk.data_ptr(), dv.data_ptr()
    p.lse, p.dsum = lse.data_ptr(), dsum.data_ptr()
    p.qs, p.ks, p.vs, p.os, p.dos = _bhs(q), _bhs(k), _bhs(v), _bhs(out), _bhs(dout)
    p.dqs, p.dks, p.dvs = _bhs(dq), _bhs(dk), _bhs(dv)
    p.B, p.Hq, p.Hk, p.SQ, p.SK, p.D, p.gqa = B, Hq, Hk, SQ, SK, D, Hq // Hk
    p.scale, p.softcap = float(scale), float(softcap)
    p.alibi = al.data_ptr() if al is not None else None
    p.causal, p.win_left, p.win_right = 1 if causal else 0, int(win_left), int(win_right)
    p.dropout = 1 if dropout_p > 0 else 0
    p.drop_seed, p.dropout_p = int(seed) & ((1 << 64) - 1), float(dropout_p)
    p.keep_scale = 1.0 / (1.0 - dropout_p) if dropout_p > 0 else 1.0
    p.lse_sb, p.lse_sh = Hq * SQ, SQ
    ws = _ds_workspace(p, _dt(q), q.device, ds_max_bytes)  # noqa: F841  (alive through the launch)
    with _on(q.device):
        _lib.check(_L.fable_attn_bwd(p, _dt(q), _stream(q)), "fable_attn_bwd")
    return dq, dk, dv


def bwd_varlen(dout, q, k, v, out, lse, cu_q, cu_k, max_sq, max_sk, scale, causal, win_left,
               win_right, softcap, alibi, dropout_p, seed, seqused_q=None, seqused_k=None,
               ds_max_bytes=None):
    """Packed variable-length backward: dout/q/out (total_q, Hq, D), k/v (total_k, Hk, D),
    cu_* int32 [batch+1], lse [Hq, total_q] fp32 (fwd_varlen(..., return_lse=True)). One launch
    of each backward kernel for all sequences; the reference has none and loops over the
    sequences in Python (flash_attn_interface.py:523-540). Returns (dq, dk, dv) packed; rows
    outside every sequence (and past seqused) get zero gradient."""
    _req(q.is_cuda and k.is_cuda and v.is_cuda, "GPU tensors required")
    for n, t in (("dout", dout), ("q", q), ("k", k), ("v", v), ("out", out)):
        _req(t.dim() == 3, f"{n}: varlen expects [total, H, D]")
        _req(t.dtype == q.dtype and t.device == q.device, f"{n}: dtype/device mismatch")
        _req(_rows_aligned(t), f"{n}: head_dim must be contiguous with 16-byte aligned rows")
    Hq, D, Hk = q.shape[1], q.shape[2], k.shape[1]
    _req(Hq % Hk == 0, "Hq must be a multiple of Hk (GQA)")
    _req(dout.shape == q.shape and out.shape == q.shape and v.shape == k.shape, "shape mismatch")
    _req(lse.dtype == torch.float32 and lse.is_contiguous() and tuple(lse.shape) == (Hq, q.shape[0])
         and lse.device == q.device, "lse must be contiguous fp32 [Hq, total_q] on q's device")
    batch = _check_varlen_index(q, cu_q, cu_k, seqused_q, seqused_k)
    dq, dk, dv = torch.zeros_like(q), torch.zeros_like(k), torch.zeros_like(v)
    dsum = torch.empty((Hq, q.shape[0]), dtype=torch.float32, device=q.device)
    al = _alibi(alibi, Hq, q.device)
    row = lambda t: Strides(0, t.stride(1), t.stride(0))
    p = FableBwdParams()
    p.Q, p.K, p.V, p.O, p.dO = q.data_ptr(), k.data_ptr(), v.data_ptr(), out.data_ptr(), dout.data_ptr()
    p.dQ, p.dK, p.dV = dq.data_ptr(), dk.data_ptr(), dv.data_ptr()
    p.lse, p.dsum = lse.data_ptr(), dsum.data_ptr()
    p.qs, p.ks, p.vs, p.os, p.dos = row(q), row(k), row(v), row(out), row(dout)
    p.dqs, p.dks, p.dvs = row(dq), row(dk), row(dv)
    p.B, p.Hq, p.Hk, p.SQ, p.SK, p.D, p.gqa = batch, Hq, Hk, int(max_sq), int(max_sk), D, Hq // Hk
    p.scale, p.softcap = float(scale), float(softcap)
    p.alibi = al.data_ptr() if al is not None else None
    p.causal, p.win_left, p.win_right = 1 if causal else 0, int(win_left), int(win_right)
    p.dropout = 1 if dropout_p > 0 else 0
    p.drop_seed, p.dropout_p = int(seed) & ((1 << 64) - 1), float(dropout_p)
    p.keep_scale = 1.0 / (1.0 - dropout_p) if dropout_p > 0 else 1.0
    p.cu_q, p.cu_k = cu_q.data_ptr(), cu_k.data_ptr()
    p.seqused_q = seqused_q.data_ptr() if seqused_q is not None else None
    p.seqused_k = seqused_k.data_ptr() if seqused_k is not None else None
    p.lse_sb, p.lse_sh = 0, q.shape[0]
    ws = _ds_workspace(p, _dt(q), q.device, ds_max_bytes)  # noqa: F841  (alive through the launch)
    with _on(q.device):
        _lib.check(_L.fable_attn_bwd(p, _dt(q), _stream(q)), "fable_attn_bwd (varlen)")
    return dq, dk, dv


def num_splits(batch, nq, nheads, gqa, ctx_bound, hint):
    return int(_L.fa_decode_num_splits(batch, nq, nheads, gqa, int(ctx_bound), int(hint)))


def dec(q, k_cache, v_cache, block_table, cache_seqlens, new_k, new_v, rotary_cos, rotary_sin,
        rotary_interleaved, scale, window, num_splits=0, cache_leftpad=None, return_lse=False,
        softcap=0.0, alibi=None, rotary_dim=0, rotary_pos=None):
    """q [B,nq,Hq,D]; caches [num_blocks,page,Hk,D] contiguous; block_table [B,max_blocks]
    int32; cache_seqlens [B] int32 (length before append). Returns (out [B,nq,Hq,D],
    lse [B,nq,Hq] or an empty tensor). Reference: dispatch.cpp:162-231."""
    _req(q.is_cuda and k_cache.is_cuda and v_cache.is_cuda, "GPU tensors required")
    _req(q.dim() == 4, "decode expects q [B,nq,Hq,D]")
    _req(k_cache.dim() == 4, "k_cache expected [num_blocks, page, nheads_k, D]")
    B, NQ, Hq, D = q.shape
    page, Hk = k_cache.shape[1], k_cache.shape[2]
    _req(Hq % Hk == 0, "Hq must be a multiple of nheads_k (GQA)")
    _req(page > 0 and (page & (page - 1)) == 0, "page must be a power of two")
    dev = q.device
    for n, t in (("q", q), ("k_cache", k_cache), ("v_cache", v_cache)):
        _req(t.is_contiguous() and t.dtype == q.dtype and t.device == dev,
             f"{n}: contiguous, dtype and device of q")
        _req(t.data_ptr() % 16 == 0 and (D * t.element_size()) % 16 == 0,
             f"{n}: rows must be 16-byte aligned (base pointer and head_dim)")
    _req(v_cache.shape == k_cache.shape and k_cache.shape[3] == D,
         "k_cache/v_cache must both be [num_blocks, page, nheads_k, D] with q's D")
    _req(block_table.dim() == 2 and block_table.shape[0] == B, "block_table must be [B, max_blocks]")
    _check_index("block_table", block_table, dev)
    _check_index("cache_seqlens", cache_seqlens, dev, B)
    if cache_leftpad is not None:
        _check_index("cache_leftpad", cache_leftpad, dev, B)
    if rotary_pos is not None:
        _check_index("rotary_seqlens", rotary_pos, dev, B)
    if alibi is not None:
        _check_f32("alibi_slopes", alibi, dev, Hq)
    _req((rotary_cos is None) == (rotary_sin is None), "rotary_cos and rotary_sin go together")
    if rotary_cos is not None:
        _check_f32("rotary_cos", rotary_cos, dev)
        _check_f32("rotary_sin", rotary_sin, dev)
        _req(rotary_cos.dim() == 2 and rotary_sin.shape == rotary_cos.shape,
             "rotary_cos/rotary_sin must be [seqlen_ro, rotary_dim/2]")
        rd = int(rotary_dim) or D
        _req(rotary_cos.shape[1] * 2 == rd and rd <= D and rd % 2 == 0,
             f"rotary tables of width {rotary_cos.shape[1]} do not match rotary_dim {rd}")
    if new_k is not None:
        _req(new_v is not None, "new_k and new_v go together")
        for n, t in (("k", new_k), ("v", new_v)):
            _req(tuple(t.shape) == (B, NQ, Hk, D) and t.dtype == q.dtype and t.device == dev and
                 t.is_contiguous() and t.data_ptr() % 16 == 0,
                 f"{n}: contiguous, 16-byte aligned [B, seqlen_q, nheads_k, D] of q's dtype")
    else:
        _req(new_v is None, "new_k and new_v go together")
    ctx_bound = block_table.shape[1] * page
    nsplit = int(_L.fa_decode_num_splits(B, NQ, Hq, Hq // Hk, ctx_bound, int(num_splits or 0)))
    out = torch.empty((B, NQ, Hq, D), dtype=q.dtype, device=q.device)
    # one fp16/bf16 split writes out (and lse) from the partial kernel: no scratch then
    scratch = (torch.empty((B * NQ * Hq * nsplit * (D + 2),), dtype=torch.float32, device=q.device)
               if nsplit > 1 or q.dtype == torch.float32 else None)
    lse = (torch.empty((B, NQ, Hq), dtype=torch.float32, device=q.device) if return_lse
           else torch.empty((0,), dtype=torch.float32, device=q.device))
    p = FableDecParams()
    p.q, p.Kc, p.Vc = q.data_ptr(), k_cache.data_ptr(), v_cache.data_ptr()
    p.block_table, p.o = block_table.data_ptr(), out.data_ptr()
    p.scratch = scratch.data_ptr() if scratch is not None else None
    p.ctx_len = cache_seqlens.data_ptr()
    p.cos = rotary_cos.data_ptr() if rotary_cos is not None else None
    p.sin = rotary_sin.data_ptr() if rotary_sin is not None else None
    p.batch, p.NH, p.gqa, p.HD, p.page = B, Hq, Hq // Hk, D, page
    p.max_blocks, p.nsplit, p.window = block_table.shape[1], nsplit, int(window)
    p.rotary = (2 if rotary_interleaved else 1) if rotary_cos is not None else 0
    p.scale = float(scale)
    p.leftpad = cache_leftpad.data_ptr() if cache_leftpad is not None else None
    p.lse_out = lse.data_ptr() if return_lse else None
    p.softcap = float(softcap)
    p.alibi = alibi.data_ptr() if alibi is not None else None
    p.nq, p.rotary_dim = NQ, int(rotary_dim)
    p.rotary_pos = rotary_pos.data_ptr() if rotary_pos is not None else None
    with _on(q.device):
        _lib.check(_L.fable_attn_dec(p, _dt(q), _stream(q), _ptr(new_k), _ptr(new_v)),
                   "fable_attn_dec")
    return out, lse


def combine(out_partial, lse_partial, out_dtype):
    """out_partial [nsplit,B,S,H,D] (D contiguous), lse_partial [nsplit,B,H,S] fp32 ->
    dense [B,S,H,D] in out_dtype. Reference math: flash_attn_interface.py:567-580."""
    _req(out_partial.is_cuda and lse_partial.is_cuda, "GPU tensors required")
    _req(out_partial.dim() == 5 and lse_partial.dim() == 4, "shapes [nsplit,B,S,H,D] / [nsplit,B,H,S]")
    _req(out_partial.stride(-1) == 1, "out_partial: head_dim must be contiguous")
    ns, B, S, H, D = out_partial.shape
    _req(tuple(lse_partial.shape) == (ns, B, H, S),
         f"lse_partial must be [nsplit, B, H, S] = {(ns, B, H, S)}, got {tuple(lse_partial.shape)}")
    _req(lse_partial.device == out_partial.device, "out_partial and lse_partial on one device")
    lp = lse_partial.float()
    out = torch.empty((B, S, H, D), dtype=out_dtype, device=out_partial.device)
    c = CombineParams()
    c.out_partial, c.lse_partial, c.out = out_partial.data_ptr(), lp.data_ptr(), out.data_ptr()
    c.nsplit, c.B, c.S, c.H, c.D = ns, B, S, H, D
    c.op_split, c.op_b, c.op_seq, c.op_h = (out_partial.stride(0), out_partial.stride(1),
                                            out_partial.stride(2), out_partial.stride(3))
    c.lp_split, c.lp_b, c.lp_h, c.lp_seq = lp.stride(0), lp.stride(1), lp.stride(2), lp.stride(3)
    c.in_dtype, c.out_dtype = _dt(out_partial), _dt(out)
    with _on(out_partial.device):
        _lib.check(_L.fa_combine_launch(c, _stream(out_partial)), "fa_combine_launch")
    return out
