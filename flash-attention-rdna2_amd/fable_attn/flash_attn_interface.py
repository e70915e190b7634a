"""flash_attn API (FA-2 argument order) over the gfx950 kernels of libfable_attn_hip.so.

Public surface, argument order, defaults, return shapes, exception types and the message
substrings callers match on are the reference's (package/fable_attn/flash_attn_interface.py):
    flash_attn_func                  :378-388   flash_attn_qkvpacked_func        :391-401
    flash_attn_kvpacked_func         :404-414   flash_attn_varlen_func           :417-540
    flash_attn_varlen_qkvpacked_func :543-551   flash_attn_varlen_kvpacked_func  :554-564
    flash_attn_combine               :567-580   flash_attn_with_kvcache          :583-771

Structure. Every entry point first turns its arguments into one `_Spec`: the scalars the
kernels take (scale, mask, softcap, alibi, dropout, chunk) plus the tensors at the width the
kernels run (qv and a value head dim other than the score head dim become one widened
problem; a head dim without a kernel is zero-padded to the next one), and how many value
columns the caller gets back. Dense and packed variable-length batches then go through one
autograd function, `_Attention`, which calls the forward once (with LSE) and the backward once
for the whole batch. Decode builds the same `_Spec` and hands it to the paged kernel.
Inputs are (batch, seqlen, nheads, headdim); the kernels take [B, H, S, D] strided views, so
nothing is copied unless a row is misaligned. An unsupported configuration raises; a missing
library raises ImportError at import time. Nothing falls back to another implementation.
"""
import ctypes
import dataclasses
import math
import random
import threading
from typing import Optional

import torch

from . import _C, _lib

# Head dims the kernels take as they are: every multiple of 8 up to 256, in every dtype (rows
# move in 16-byte accesses; the kernels zero the columns up to their own width). Any other head
# dim is zero-padded to the next multiple of 8: zero columns change neither q.k nor the kept
# output columns.
MAX_HEAD_DIM = 256
_DTYPES = (torch.float16, torch.bfloat16, torch.float32)


# ----------------------------------------------------------------------------- contract
def _map_window(causal, window_size):
    """(causal, (left, right)) -> (causal_flag, win_left, win_right), reference :76-95.
    Key j is visible to query i when i+delta-left <= j <= i+delta+right (delta = SK-SQ); a
    negative (or None) bound is absent; causal pins right to 0; the flag is set whenever
    right == 0."""
    left, right = window_size
    wl = int(left) if left is not None and left >= 0 else -1
    wr = 0 if causal else (int(right) if right is not None and right >= 0 else -1)
    return int(wr == 0), wl, wr


def _reject_fp8(q_descale, k_descale, v_descale):
    """FP8 descaling is refused loudly (reference :99-107)."""
    if any(x is not None for x in (q_descale, k_descale, v_descale)):
        raise NotImplementedError(
            "fable_attn: q_descale/k_descale/v_descale (FP8) are not supported; "
            "pass fp16 or bf16 tensors")


def _accept_hints(num_splits=None, pack_gqa=None, sm_margin=None):
    """Scheduling hints change the schedule, never the result; only their types are checked
    (reference :110-128). num_splits is honoured by decode."""
    for name, val, ok in (("num_splits", num_splits, int), ("pack_gqa", pack_gqa, bool),
                          ("sm_margin", sm_margin, int)):
        if val is not None and not isinstance(val, ok):
            raise TypeError(f"fable_attn: {name} must be {ok.__name__} or None, got {type(val)}")


def _check_chunk(attention_chunk):
    """attention_chunk: None or a non-negative int (reference :131-137); 0 disables it."""
    if attention_chunk is None:
        return 0
    if not isinstance(attention_chunk, int) or attention_chunk < 0:
        raise ValueError(f"fable_attn: attention_chunk must be a non-negative int, "
                         f"got {attention_chunk!r}")
    return attention_chunk


# ----------------------------------------------------------------------------- normalisation
@dataclasses.dataclass
class _Spec:
    """One call after normalisation: tensors at kernel width and every kernel scalar."""
    q: torch.Tensor
    k: torch.Tensor
    v: torch.Tensor
    scale: float
    causal: int
    wl: int
    wr: int
    softcap: float
    alibi: Optional[torch.Tensor]
    dropout_p: float
    chunk: int
    keep: Optional[int]          # value columns returned to the caller (None: all)

    def cut(self, out):
        return out if self.keep is None else out[..., :self.keep]


def _kernel_width(d, dtype):
    """The head dim a call of head dim d runs at (None above MAX_HEAD_DIM)."""
    del dtype  # (every dtype has kernels for every multiple of 8)
    if d > MAX_HEAD_DIM:
        return None
    return -(-d // 8) * 8


def _with_width(t, d):
    """t with its last dim zero-extended to d (one allocation, autograd-aware)."""
    if t.shape[-1] == d:
        return t
    return torch.nn.functional.pad(t, (0, d - t.shape[-1]))


def _score_problem(q, k, v, qv):
    """Reduce FA-3's qv term and a value head dim dv other than the score head dim d to one
    attention whose q, k, v share a width, returning (q, k, v, value columns to keep):
      * qv given: S = q.k^T + qv.v^T is one product over the concatenated width d + dv,
        q' = [q | qv], k' = [k | v], and the values v' = [v | 0] leave P.V in the first dv
        output columns (the reference builds the same operands, :160-191);
      * dv != d without qv: S needs only q.k, so the narrower side is zero-extended to
        max(d, dv) (the reference also widened this case to d + dv)."""
    d, dv = q.shape[-1], v.shape[-1]
    if qv is None:
        if dv == d:
            return q, k, v, None
        w = max(d, dv)
        return _with_width(q, w), _with_width(k, w), _with_width(v, w), dv
    if qv.shape[-1] != dv:
        raise ValueError(f"fable_attn: qv.shape[-1]={qv.shape[-1]} must equal v.shape[-1]={dv}")
    if d + dv > MAX_HEAD_DIM:
        raise NotImplementedError(
            f"fable_attn: qv needs a score head_dim of headdim+headdim_v = {d}+{dv} = {d + dv}, "
            f"above the kernel maximum {MAX_HEAD_DIM}")
    return (torch.cat([q, qv], -1), torch.cat([k, v], -1), _with_width(v, d + dv), dv)


def _normalize(q, k, v, *, qv=None, softmax_scale=None, causal=False, window_size=(-1, -1),
               softcap=0.0, alibi_slopes=None, dropout_p=0.0, attention_chunk=0,
               descale=(None, None, None), hints=(None, None, None), head_axis=2):
    """Validate the arguments (reference :99-156) and build the _Spec of a prefill call.
    head_axis is the nheads axis of q/k (2 for (B,S,H,D), 1 for packed (total,H,D))."""
    _reject_fp8(*descale)
    _accept_hints(*hints)
    chunk = _check_chunk(attention_chunk)
    if not q.is_cuda:
        raise ValueError("fable_attn: tensors must be on the GPU (q.is_cuda == False)")
    if q.dtype not in _DTYPES:
        raise ValueError(f"fable_attn: dtype {q.dtype} is not supported; use fp16, bf16 or fp32")
    if q.shape[head_axis] % k.shape[head_axis]:
        raise ValueError(f"fable_attn: nheads_q={q.shape[head_axis]} is not a multiple of "
                         f"nheads_k={k.shape[head_axis]} (GQA)")
    d, dv = q.shape[-1], v.shape[-1]
    if softmax_scale is None:
        # the reference scales by the concatenated width whenever qv or headdim_v != headdim
        softmax_scale = (d + dv) ** -0.5 if (qv is not None or dv != d) else d ** -0.5
    q, k, v, keep = _score_problem(q, k, v, qv)
    w = _kernel_width(q.shape[-1], q.dtype)
    if w is None:
        raise ValueError(f"fable_attn: head_dim={q.shape[-1]} exceeds the maximum {MAX_HEAD_DIM}")
    if w != q.shape[-1]:
        keep = keep if keep is not None else v.shape[-1]
        q, k, v = _with_width(q, w), _with_width(k, w), _with_width(v, w)
    cflag, wl, wr = _map_window(causal, window_size)
    alibi = alibi_slopes.to(torch.float32).contiguous() if alibi_slopes is not None else None
    return _Spec(q, k, v, float(softmax_scale), cflag, wl, wr, float(softcap or 0.0), alibi,
                 float(dropout_p), chunk, keep)


def _bhsd(t):
    """(B,S,H,D) -> the [B,H,S,D] view the kernels take; a copy only when a row is not 16-byte
    aligned (the kernels move rows in 16-byte accesses). The copy is a fresh allocation: a
    contiguous tensor at a misaligned offset would stay where it is under .contiguous()."""
    v = t.transpose(1, 2)
    st, el = v.stride(), v.element_size()
    aligned = (st[-1] == 1 and v.data_ptr() % 16 == 0
               and (st[0] * el | st[1] * el | st[2] * el) % 16 == 0)
    return v if aligned else t.clone(memory_format=torch.contiguous_format).transpose(1, 2)


def _aligned(t, dense=False):
    """t itself when the kernels can read it in place (contiguous head dim, 16-byte aligned
    base and strides; with dense, also contiguous), else a fresh contiguous copy."""
    st, el = t.stride(), t.element_size()
    ok = st[-1] == 1 and t.data_ptr() % 16 == 0 and all((x * el) % 16 == 0 for x in st[:-1])
    if ok and (not dense or t.is_contiguous()):
        return t
    return t.clone(memory_format=torch.contiguous_format)



# ----------------------------------------------------------------------------- autograd
def _forward(spec, pack, q, k, v):
    """One forward launch of a dense ([B,H,S,D] views, pack None) or packed variable-length
    batch; returns (out, lse, dropout seed)."""
    seed = random.getrandbits(63) if spec.dropout_p > 0 else 0
    args = (spec.scale, bool(spec.causal), spec.wl, spec.wr, spec.softcap, spec.alibi,
            spec.dropout_p, seed)
    if pack is None:
        B, H, S, D = q.shape
        buf = torch.empty((B, S, H, D), dtype=q.dtype, device=q.device).transpose(1, 2)
        out, lse = _C.fwd(q, k, v, *args, spec.chunk, buf)
    else:
        cu_q, cu_k, mq, mk, su_q, su_k = pack
        out, lse = _C.fwd_varlen(q, k, v, cu_q, cu_k, mq, mk, *args, spec.chunk, su_q, su_k,
                                 return_lse=True)
    return out, lse, seed


def _run(spec, pack, q, k, v):
    """(out, lse) through the autograd node when a gradient can flow, else the launch alone
    (no graph node, no saved tensors: the inference path stays a few microseconds of host time)."""
    if torch.is_grad_enabled() and (q.requires_grad or k.requires_grad or v.requires_grad):
        return _Attention.apply(spec, pack, q, k, v)
    out, lse, _ = _forward(spec, pack, q, k, v)
    return out, lse


class _Attention(torch.autograd.Function):
    """Forward (with LSE) and backward of one dense or packed variable-length batch, one
    kernel launch sequence each way. `pack` is None for dense [B,H,S,D] views, else the tuple
    (cu_q, cu_k, max_q, max_k, seqused_q, seqused_k) of a packed (total, H, D) batch.
    `deterministic` needs no switch: the backward is atomic-free and always reproducible."""

    @staticmethod
    def forward(ctx, spec, pack, q, k, v):
        out, lse, seed = _forward(spec, pack, q, k, v)
        # (the scalars only: the spec's own tensors are this node's inputs)
        ctx.spec = dataclasses.replace(spec, q=None, k=None, v=None)
        ctx.pack, ctx.seed = pack, seed
        ctx.save_for_backward(q, k, v, out, lse)
        ctx.mark_non_differentiable(lse)
        return out, lse

    @staticmethod
    def backward(ctx, dout, _dlse):
        spec, pack = ctx.spec, ctx.pack
        if spec.chunk:
            raise NotImplementedError(
                "fable_attn: backward with attention_chunk is not supported (as in FA-3); "
                "run the chunked forward under torch.no_grad()")
        q, k, v, out, lse = ctx.saved_tensors
        args = (spec.scale, bool(spec.causal), spec.wl, spec.wr, spec.softcap, spec.alibi,
                spec.dropout_p, ctx.seed)
        if pack is None:
            dq, dk, dv = _C.bwd(_bhsd(dout.transpose(1, 2)), q, k, v, out, lse, *args)
        else:
            cu_q, cu_k, mq, mk, su_q, su_k = pack
            dq, dk, dv = _C.bwd_varlen(_aligned(dout), q, k, v, out, lse, cu_q, cu_k, mq, mk,
                                       *args, su_q, su_k)
        return None, None, dq, dk, dv


# ----------------------------------------------------------------------------- debug output
def _probabilities(spec, q, k, lse, delta):
    """The softmax matrix P = exp(logit - lse) of one [H, SQ, D] / [Hk, SK, D] problem, masked
    to 0 outside the visible keys: the return_attn_probs debug output, which materialises the
    SQ x SK matrix the kernels never form (it refuses above 80% of the free memory)."""
    H, SQ, _ = q.shape
    SK = k.shape[1]
    need, free = H * SQ * SK * 4, torch.cuda.mem_get_info(q.device)[0]
    if need > 0.8 * free:
        raise torch.cuda.OutOfMemoryError(
            f"fable_attn: return_attn_probs needs a {need / 2**30:.1f} GiB S x S matrix "
            f"({free / 2**30:.1f} GiB free); the kernel itself never materialises it")
    kk = k.float().repeat_interleave(H // k.shape[0], dim=0)
    s = torch.matmul(q.float(), kk.transpose(1, 2).contiguous()) * spec.scale
    if spec.softcap > 0:
        s = spec.softcap * torch.tanh(s / spec.softcap)
    i = torch.arange(SQ, device=q.device)[:, None] + delta     # query position in key space
    j = torch.arange(SK, device=q.device)[None, :]
    if spec.alibi is not None:
        s = s + spec.alibi.view(H, 1, 1) * (j - (i - delta)).float()
    hidden = torch.zeros(SQ, SK, dtype=torch.bool, device=q.device)
    if spec.causal:
        hidden |= j > i
    if spec.wl >= 0:
        hidden |= j < i - spec.wl
    if spec.wr >= 0:
        hidden |= j > i + spec.wr
    if spec.chunk:
        start = i.clamp_min(0) // spec.chunk * spec.chunk
        hidden |= (j < start) | (j >= start + spec.chunk)
    return torch.exp(s - lse[..., None]).masked_fill(hidden, 0.0)


# ----------------------------------------------------------------------------- prefill
def _dense(q, k, v, dropout_p, softmax_scale, causal, window_size, softcap, alibi_slopes,
           deterministic, return_attn_probs, qv, attention_chunk, q_descale, k_descale,
           v_descale, num_splits, pack_gqa, sm_margin):
    """Shared body of flash_attn_func and its packed variants; (B,S,H,D) in and out."""
    del deterministic
    spec = _normalize(q, k, v, qv=qv, softmax_scale=softmax_scale, causal=causal,
                      window_size=window_size, softcap=softcap, alibi_slopes=alibi_slopes,
                      dropout_p=dropout_p, attention_chunk=attention_chunk,
                      descale=(q_descale, k_descale, v_descale),
                      hints=(num_splits, pack_gqa, sm_margin))
    qh, kh, vh = _bhsd(spec.q), _bhsd(spec.k), _bhsd(spec.v)
    out, lse = _run(spec, None, qh, kh, vh)
    res = out.transpose(1, 2)
    if spec.keep is not None:
        res = res[..., :spec.keep].contiguous()
    if not return_attn_probs:
        return res
    with torch.no_grad():
        delta = kh.shape[2] - qh.shape[2]
        probs = torch.stack([_probabilities(spec, qh[b], kh[b], lse[b], delta)
                             for b in range(qh.shape[0])])
    return res, lse, probs


# ----------------------------------------------------------------------------- inference fast path
_tls = threading.local()
_MAX_PLANS = 256


def _infer_plan(q, k, v, softmax_scale, causal, window_size, softcap):
    """The launch parameters of one inference call signature, validated once: the general
    path's normalisation (which raises exactly as it does there) followed by the binding's
    layout checks. None when the signature needs the general path (a padded or widened head
    dim, rows the kernels cannot read in place). The result holds no data pointer."""
    spec = _normalize(q, k, v, softmax_scale=softmax_scale, causal=causal,
                      window_size=window_size, softcap=softcap)
    if spec.keep is not None or spec.q is not q or spec.k is not k or spec.v is not v:
        return None
    if q.dim() != 4 or k.dim() != 4 or v.dim() != 4 or k.dtype != q.dtype or v.dtype != q.dtype:
        return None
    if k.device != q.device or v.device != q.device or q.device.index is None:
        return None
    B, SQ, Hq, D = q.shape
    SK, Hk = k.shape[1], k.shape[2]
    if k.shape[0] != B or k.shape[3] != D or tuple(v.shape) != tuple(k.shape) or Hq % Hk:
        return None
    el = q.element_size()
    for t in (q, k, v):
        st = t.stride()
        if st[3] != 1 or (st[0] * el | st[1] * el | st[2] * el) % 16:
            return None
    bhs = lambda t: _lib.Strides(t.stride(0), t.stride(2), t.stride(1))   # [B,H,S,D] view
    o = _lib.Strides(SQ * Hq * D, D, Hq * D)      # the (B,S,H,D)-dense output seen as [B,H,S,D]
    p = _lib.FableFwdParams(0, 0, 0, 0, None, bhs(q), bhs(k), bhs(v), o, SQ, SK, D, Hq, Hq // Hk,
                            spec.scale, spec.softcap, spec.wl, spec.wr, None, spec.causal, 0.0, 0,
                            None, None, B, 0, None, None, 0, 0)
    dt = _C._dt(q)
    return p, dt, (B, SQ, Hq, D), int(_C._L.fable_attn_fwd_ws_bytes(p, dt))


def _infer_fast(q, k, v, softmax_scale, causal, window_size, softcap):
    """flash_attn_func's plain inference call (no gradient, dropout, alibi, qv, chunk or
    probabilities) with the per-call host work cut to what changes between calls of one
    signature: a per-thread cache maps (shapes, strides, dtype, device, mask, scale, softcap)
    to validated launch parameters, so a call allocates the output, fills four pointers and
    launches (no LSE: the caller does not get it). None sends the call to the general path,
    which gives the same result."""
    if torch.is_grad_enabled() and (q.requires_grad or k.requires_grad or v.requires_grad):
        return None
    plans = getattr(_tls, "plans", None)
    if plans is None:
        plans = _tls.plans = {}
    try:
        key = (q.shape, k.shape, v.shape, q.stride(), k.stride(), v.stride(), q.dtype, q.device,
               causal, window_size, softcap, softmax_scale)
        plan = plans.get(key, False)
    except (AttributeError, TypeError):   # not tensors, or an unhashable argument
        return None
    if plan is False:
        if len(plans) >= _MAX_PLANS:
            plans.clear()
        plan = plans[key] = _infer_plan(q, k, v, softmax_scale, causal, window_size, softcap)
    if plan is None:
        return None
    qp, kp, vp = q.data_ptr(), k.data_ptr(), v.data_ptr()
    dev = q.device.index
    if (qp | kp | vp) & 15 or dev != torch._C._cuda_getDevice():
        return None
    p, dt, shape, ws_bytes = plan
    out = torch.empty(shape, dtype=q.dtype, device=q.device)
    p.Q, p.K, p.V, p.O = qp, kp, vp, out.data_ptr()
    _C._launch_fwd(p, dt, q.device, ctypes.c_void_p(torch._C._cuda_getCurrentRawStream(dev)), ws_bytes)
    return out


def flash_attn_func(q, k, v, dropout_p=0.0, softmax_scale=None, causal=False,
                    window_size=(-1, -1), softcap=0.0, alibi_slopes=None,
                    deterministic=False, return_attn_probs=False, *,
                    qv=None, attention_chunk=0,
                    q_descale=None, k_descale=None, v_descale=None,
                    num_splits=1, pack_gqa=None, sm_margin=0):
    """q, k, v: (batch, seqlen, nheads, headdim). Returns out in the same layout (dense), or
    (out, softmax_lse, S_dmask) when return_attn_probs=True."""
    if (not dropout_p and alibi_slopes is None and qv is None and not attention_chunk
            and not return_attn_probs and q_descale is None and k_descale is None
            and v_descale is None and (num_splits is None or type(num_splits) is int)
            and (pack_gqa is None or type(pack_gqa) is bool)
            and (sm_margin is None or type(sm_margin) is int)):
        out = _infer_fast(q, k, v, softmax_scale, causal, window_size, softcap)
        if out is not None:
            return out
    return _dense(q, k, v, dropout_p, softmax_scale, causal, window_size, softcap, alibi_slopes,
                  deterministic, return_attn_probs, qv, attention_chunk, q_descale, k_descale,
                  v_descale, num_splits, pack_gqa, sm_margin)


def flash_attn_qkvpacked_func(qkv, dropout_p=0.0, softmax_scale=None, causal=False,
                              window_size=(-1, -1), softcap=0.0, alibi_slopes=None,
                              deterministic=False, return_attn_probs=False, *,
                              qv=None, attention_chunk=0,
                              q_descale=None, k_descale=None, v_descale=None,
                              num_splits=1, pack_gqa=None, sm_margin=0):
    """qkv: (batch, seqlen, 3, nheads, headdim)."""
    q, k, v = qkv.unbind(2)
    return _dense(q, k, v, dropout_p, softmax_scale, causal, window_size, softcap, alibi_slopes,
                  deterministic, return_attn_probs, qv, attention_chunk, q_descale, k_descale,
                  v_descale, num_splits, pack_gqa, sm_margin)


def flash_attn_kvpacked_func(q, kv, dropout_p=0.0, softmax_scale=None, causal=False,
                             window_size=(-1, -1), softcap=0.0, alibi_slopes=None,
                             deterministic=False, return_attn_probs=False, *,
                             qv=None, attention_chunk=0,
                             q_descale=None, k_descale=None, v_descale=None,
                             num_splits=1, pack_gqa=None, sm_margin=0):
    """q: (batch, sq, nheads, d); kv: (batch, sk, 2, nheads_k, d)."""
    k, v = kv.unbind(2)
    return _dense(q, k, v, dropout_p, softmax_scale, causal, window_size, softcap, alibi_slopes,
                  deterministic, return_attn_probs, qv, attention_chunk, q_descale, k_descale,
                  v_descale, num_splits, pack_gqa, sm_margin)


def _as_index(t, device):
    return t.to(device=device, dtype=torch.int32).contiguous()


def _pages_as_packed(k_cache, v_cache, block_table, cu_seqlens_k, seqused_k):
    """Paged K/V of a varlen prefill as a packed batch without a host round trip: every
    sequence's block-table row is gathered whole (max_blocks * page rows per sequence, one
    device gather), so sequence b starts at row b * max_blocks * page, and its true length
    becomes seqused_k. Table entries past a sequence's ceil(len / page) pages are not read:
    serving code leaves -1, stale or out-of-range values there, so they are replaced by page 0
    on the device before the gather (the rows they bring are past seqused_k and never attended).
    Returns (k, v, cu_k, seqused_k, max_seqlen_k)."""
    if k_cache.dim() != 4 or v_cache.dim() != 4:
        raise ValueError(
            "fable_attn: with block_table, k and v must be paged "
            f"(num_blocks, page_block_size, nheads_k, headdim); got k.shape={tuple(k_cache.shape)}")
    nseq = cu_seqlens_k.numel() - 1
    if block_table.dim() != 2 or block_table.shape[0] != nseq:
        raise ValueError(f"fable_attn: block_table must be (batch, max_blocks), got "
                         f"{tuple(block_table.shape)} for batch={nseq}")
    dev = k_cache.device
    page = k_cache.shape[1]
    bt = block_table.to(device=dev, dtype=torch.long)
    span = bt.shape[1] * page
    used = _as_index(seqused_k if seqused_k is not None
                     else cu_seqlens_k[1:] - cu_seqlens_k[:-1], dev)
    live = (torch.arange(bt.shape[1], device=dev)[None, :]
            < ((used.to(torch.long) + page - 1) // page)[:, None])
    bt = torch.where(live, bt, torch.zeros_like(bt))
    flat = lambda c: c[bt.reshape(-1)].reshape(nseq * span, c.shape[2], c.shape[3])
    cu = torch.arange(nseq + 1, device=dev, dtype=torch.int32) * span
    return flat(k_cache), flat(v_cache), cu, used, span


def flash_attn_varlen_func(q, k, v, cu_seqlens_q, cu_seqlens_k, max_seqlen_q, max_seqlen_k,
                           dropout_p=0.0, softmax_scale=None, causal=False,
                           window_size=(-1, -1), softcap=0.0, alibi_slopes=None,
                           deterministic=False, return_attn_probs=False, *,
                           seqused_q=None, seqused_k=None,
                           qv=None, attention_chunk=0,
                           q_descale=None, k_descale=None, v_descale=None,
                           num_splits=1, pack_gqa=None, sm_margin=0,
                           block_table=None):
    """Packed variable-length sequences: q (total_q, nheads, d), k/v (total_k, nheads_k, d),
    cu_seqlens_* int32 (batch+1). One forward launch over all sequences and, with grad, one
    launch of each backward kernel (the reference loops over the sequences in Python on the
    grad path, :523-540). With return_attn_probs: (out, [lse per sequence], [P per sequence])."""
    del deterministic
    if q.dim() != 3:
        raise ValueError(f"fable_attn: varlen expects (total, nheads, headdim), got {tuple(q.shape)}")
    if block_table is not None:
        k, v, cu_seqlens_k, seqused_k, max_seqlen_k = _pages_as_packed(
            k, v, block_table, cu_seqlens_k, seqused_k)
    spec = _normalize(q, k, v, qv=qv, softmax_scale=softmax_scale, causal=causal,
                      window_size=window_size, softcap=softcap, alibi_slopes=alibi_slopes,
                      dropout_p=dropout_p, attention_chunk=attention_chunk,
                      descale=(q_descale, k_descale, v_descale),
                      hints=(num_splits, pack_gqa, sm_margin), head_axis=1)
    dev = spec.q.device
    pack = (_as_index(cu_seqlens_q, dev), _as_index(cu_seqlens_k, dev), int(max_seqlen_q),
            int(max_seqlen_k), _as_index(seqused_q, dev) if seqused_q is not None else None,
            _as_index(seqused_k, dev) if seqused_k is not None else None)
    out, lse = _run(spec, pack, _aligned(spec.q), _aligned(spec.k), _aligned(spec.v))
    out = spec.cut(out)
    if not return_attn_probs:
        return out
    # debug path: one probability matrix per sequence (ragged shapes), host lengths needed
    cq, ck = pack[0].tolist(), pack[1].tolist()
    uq = pack[4].tolist() if pack[4] is not None else None
    uk = pack[5].tolist() if pack[5] is not None else None
    lses, probs = [], []
    with torch.no_grad():
        for z in range(len(cq) - 1):
            nq = uq[z] if uq is not None else cq[z + 1] - cq[z]
            nk = uk[z] if uk is not None else ck[z + 1] - ck[z]
            qz = spec.q[cq[z]:cq[z] + nq].transpose(0, 1)
            kz = spec.k[ck[z]:ck[z] + nk].transpose(0, 1)
            lz = lse[:, cq[z]:cq[z] + nq]
            lses.append(lz)
            probs.append(_probabilities(spec, qz, kz, lz, nk - nq))
    return out, lses, probs


def flash_attn_varlen_qkvpacked_func(qkv, cu_seqlens, max_seqlen, dropout_p=0.0,
                                     softmax_scale=None, causal=False, window_size=(-1, -1),
                                     softcap=0.0, alibi_slopes=None, deterministic=False,
                                     return_attn_probs=False, **kw):
    """qkv: (total_tokens, 3, nheads, headdim)."""
    q, k, v = qkv.unbind(1)
    return flash_attn_varlen_func(q, k, v, cu_seqlens, cu_seqlens, max_seqlen, max_seqlen,
                                  dropout_p, softmax_scale, causal, window_size, softcap,
                                  alibi_slopes, deterministic, return_attn_probs, **kw)


def flash_attn_varlen_kvpacked_func(q, kv, cu_seqlens_q, cu_seqlens_k, max_seqlen_q,
                                    max_seqlen_k, dropout_p=0.0, softmax_scale=None,
                                    causal=False, window_size=(-1, -1), softcap=0.0,
                                    alibi_slopes=None, deterministic=False,
                                    return_attn_probs=False, **kw):
    """q: (total_q, nheads, d); kv: (total_k, 2, nheads_k, d)."""
    k, v = kv.unbind(1)
    return flash_attn_varlen_func(q, k, v, cu_seqlens_q, cu_seqlens_k, max_seqlen_q,
                                  max_seqlen_k, dropout_p, softmax_scale, causal, window_size,
                                  softcap, alibi_slopes, deterministic, return_attn_probs, **kw)


def flash_attn_combine(out_partial, lse_partial, out=None, out_dtype=None):
    """Merge split-KV partials: out_partial (nsplit, B, S, H, D), lse_partial (nsplit, B, H, S)
    natural-log LSE -> (B, S, H, D). One HIP kernel (the reference used torch ops, :567-580)."""
    res = _C.combine(out_partial, lse_partial, out_dtype or out_partial.dtype)
    if out is None:
        return res
    out.copy_(res)
    return out


# ----------------------------------------------------------------------------- decode
def _cache_rows(q, k_cache, cache_seqlens, cache_batch_idx, block_table):
    """(block_table, page, cache lengths) for the paged kernel: a paged cache keeps its table; a
    dense (batch, seqlen, ...) cache is a paged one with one page per row (cache_batch_idx picks
    the rows), which needs a power-of-two seqlen."""
    B, dev = q.shape[0], q.device
    if block_table is not None:
        if cache_batch_idx is not None:
            raise ValueError("fable_attn: cache_batch_idx applies to a dense cache only; with a "
                             "paged cache the block_table selects the rows")
        table, page = _as_index(block_table, dev), k_cache.shape[1]
    else:
        page = k_cache.shape[1]
        if page & (page - 1):
            raise NotImplementedError(
                f"fable_attn: dense cache length {page} must be a power of two (or pass block_table)")
        rows = (cache_batch_idx if cache_batch_idx is not None
                else torch.arange(B, device=dev))
        table = _as_index(rows, dev).view(B, 1)
    if cache_seqlens is None:
        lens = torch.full((B,), k_cache.shape[1], dtype=torch.int32, device=dev)
    elif isinstance(cache_seqlens, int):
        lens = torch.full((B,), cache_seqlens, dtype=torch.int32, device=dev)
    else:
        lens = _as_index(cache_seqlens, dev)
    return table, page, lens


@torch.no_grad()
def flash_attn_with_kvcache(q, k_cache, v_cache, k=None, v=None, qv=None,
                            rotary_cos=None, rotary_sin=None,
                            cache_seqlens=None, cache_batch_idx=None, cache_leftpad=None,
                            block_table=None, softmax_scale=None, causal=False,
                            window_size=(-1, -1), softcap=0.0, rotary_interleaved=True,
                            alibi_slopes=None, num_splits=0, return_softmax_lse=False, *,
                            page_table=None, attention_chunk=0,
                            q_descale=None, k_descale=None, v_descale=None,
                            pack_gqa=None, sm_margin=0, scheduler_metadata=None,
                            cu_seqlens_q=None, cu_seqlens_k_new=None, max_seqlen_q=None,
                            rotary_seqlens=None):
    """Decode against a paged (k_cache/v_cache (num_blocks, page, nheads_k, d) + block_table)
    or dense ((batch, seqlen, nheads_k, d)) KV cache; split-KV kernels with an LSE combine.
    q: (batch, seqlen_q, nheads, d), or packed (total_q, nheads, d) with cu_seqlens_q; new
    token t of sequence b sits at cache_seqlens[b] + t. Without k/v every new token sees the
    cached keys [0, cache_seqlens[b]); k/v (batch, seqlen_q, nheads_k, d) are written into
    the cache first, and then token t also sees the new keys up to its own. Returns out, or
    (out, softmax_lse (batch, nheads, seqlen_q)). Reference :583-771."""
    _reject_fp8(q_descale, k_descale, v_descale)
    _accept_hints(num_splits, pack_gqa, sm_margin)
    del scheduler_metadata      # the launcher plans each call itself (fa_decode_num_splits)
    if cu_seqlens_k_new is not None:
        raise NotImplementedError(
            "fable_attn: cu_seqlens_k_new (ragged append) is not supported; append the same "
            "number of tokens to every batch element")
    if page_table is not None:
        if block_table is not None:
            raise ValueError("fable_attn: block_table and page_table are the same argument; pass one")
        block_table = page_table
    if (k is None) != (v is None):
        raise ValueError("fable_attn: k and v are appended to the cache together")
    if cu_seqlens_q is not None:
        return _kvcache_packed_q(q, k_cache, v_cache, k, qv, cu_seqlens_q, max_seqlen_q,
                                 return_softmax_lse, rotary_cos=rotary_cos,
                                 rotary_sin=rotary_sin, cache_seqlens=cache_seqlens,
                                 cache_batch_idx=cache_batch_idx, cache_leftpad=cache_leftpad,
                                 block_table=block_table, softmax_scale=softmax_scale,
                                 causal=causal, window_size=window_size, softcap=softcap,
                                 rotary_interleaved=rotary_interleaved,
                                 alibi_slopes=alibi_slopes, num_splits=num_splits,
                                 attention_chunk=attention_chunk, rotary_seqlens=rotary_seqlens)
    if q.dim() != 4:
        raise ValueError(f"fable_attn: decode expects q (batch, seqlen_q, nheads, headdim), "
                         f"got {tuple(q.shape)}")
    if not q.is_cuda:
        raise ValueError("fable_attn: tensors must be on the GPU (q.is_cuda == False)")
    if q.dtype not in _DTYPES:
        raise ValueError(f"fable_attn: dtype {q.dtype} is not supported; use fp16, bf16 or fp32")
    if softmax_scale is None:
        softmax_scale = (q.shape[-1] + (qv.shape[-1] if qv is not None else 0)) ** -0.5
    appending = k is not None
    if appending and (qv is not None or not (k_cache.is_contiguous() and v_cache.is_contiguous())):
        raise NotImplementedError(
            "fable_attn: appending k/v needs the kernel to write the caller's cache in place: "
            "not possible with qv (the cache is widened into a temporary) or with a "
            "non-contiguous cache")
    NQ = q.shape[1]
    table, page, lens = _cache_rows(q, k_cache, cache_seqlens, cache_batch_idx, block_table)
    kc, vc, keep = k_cache, v_cache, None
    if qv is not None or v_cache.shape[-1] != k_cache.shape[-1]:
        # compat path: the score problem widened over the whole cache (one temporary copy)
        q, kc, vc, keep = _score_problem(q, k_cache, v_cache, qv)
    w = _kernel_width(q.shape[-1], q.dtype)
    if w is None:
        raise ValueError(f"fable_attn: head_dim={q.shape[-1]} exceeds the maximum {MAX_HEAD_DIM}")
    if w != q.shape[-1]:
        if appending:
            raise NotImplementedError(
                f"fable_attn: appending k/v needs a head_dim the kernels take as it is (a multiple "
                f"of 8), got {q.shape[-1]}")
        keep = keep if keep is not None else vc.shape[-1]
        q, kc, vc = _with_width(q, w), _with_width(kc, w), _with_width(vc, w)
    _, wl, _ = _map_window(True, window_size)
    keys_back = wl + 1 if 0 <= wl < 2 ** 31 - 1 else -1   # the kernel's window: keys up to the query
    dev = q.device
    leftpad = _as_index(cache_leftpad, dev) if cache_leftpad is not None else None
    chunk = _check_chunk(attention_chunk)
    if chunk:
        if NQ > 1:
            raise NotImplementedError(
                "fable_attn: attention_chunk in decode is supported for one new token: "
                "several tokens would need different chunk starts")
        # the one new token sees its own chunk: keys from the chunk start, a left pad
        start = (lens.to(torch.int64) // chunk * chunk).to(torch.int32)
        leftpad = start if leftpad is None else torch.maximum(leftpad, start)
    cos = rotary_cos.to(torch.float32).contiguous() if rotary_cos is not None else None
    sin = rotary_sin.to(torch.float32).contiguous() if rotary_sin is not None else None
    alibi = alibi_slopes.to(torch.float32).contiguous() if alibi_slopes is not None else None
    rpos = _as_index(rotary_seqlens, dev) if rotary_seqlens is not None else None
    out, lse = _C.dec(_aligned(q, dense=True), kc.contiguous(), vc.contiguous(), table, lens,
                      _aligned(k, dense=True) if appending else None,
                      _aligned(v, dense=True) if appending else None,
                      cos, sin, bool(rotary_interleaved), float(softmax_scale), int(keys_back),
                      int(num_splits or 0), leftpad, bool(return_softmax_lse),
                      float(softcap or 0.0), alibi, int(cos.shape[-1] * 2) if cos is not None else 0,
                      rpos)
    if keep is not None:
        out = out[..., :keep].contiguous()
    return (out, lse.transpose(1, 2).contiguous()) if return_softmax_lse else out


def _kvcache_packed_q(q, k_cache, v_cache, k, qv, cu_seqlens_q, max_seqlen_q, return_lse,
                      **kw):
    """flash_attn_with_kvcache with packed queries q (total_q, nheads, d) and cu_seqlens_q
    (batch+1): the queries are scattered into a (batch, width, nheads, d) block on the device,
    decoded in one call (row t of sequence b at cache_seqlens[b] + t; padding rows are
    computed and dropped) and gathered back to (total_q, nheads, d). width is the longest
    sequence, read back once from the device (the reference reads cu_seqlens_q on the host and
    loops over the sequences, :636-660); a max_seqlen_q below it raises ValueError, since rows
    past it would land in the next sequence's slots."""
    if k is not None:
        raise NotImplementedError(
            "fable_attn: appending k/v with cu_seqlens_q (a ragged append) is not supported; "
            "append the same number of tokens to every batch element with a 4-D q")
    if q.dim() != 3:
        raise ValueError(f"fable_attn: with cu_seqlens_q, q must be (total_q, nheads, headdim), "
                         f"got {tuple(q.shape)}")
    dev = q.device
    cu = _as_index(cu_seqlens_q, dev).long()
    nseq, total = cu.numel() - 1, q.shape[0]
    width = int((cu[1:] - cu[:-1]).max()) if nseq > 0 else 0
    if max_seqlen_q is not None and width > int(max_seqlen_q):
        raise ValueError(f"fable_attn: max_seqlen_q={int(max_seqlen_q)} is below the longest "
                         f"sequence in cu_seqlens_q ({width})")
    row = torch.arange(total, device=dev)
    seq = torch.searchsorted(cu[1:], row, right=True)           # sequence of each packed row
    slot = seq * width + (row - cu[seq])                         # its row in the padded block
    qb = q.new_zeros((nseq * width,) + tuple(q.shape[1:]))
    qb[slot] = q
    qb = qb.view(nseq, width, q.shape[1], q.shape[2])
    qvb = None
    if qv is not None:
        qvb = qv.new_zeros((nseq * width,) + tuple(qv.shape[1:]))
        qvb[slot] = qv
        qvb = qvb.view(nseq, width, qv.shape[1], qv.shape[2])
    r = flash_attn_with_kvcache(qb, k_cache, v_cache, qv=qvb, return_softmax_lse=return_lse,
                                **kw)
    ob = r[0] if return_lse else r                               # (batch, width, nheads, dv)
    out = ob.reshape(nseq * width, ob.shape[2], ob.shape[3])[slot]
    if not return_lse:
        return out
    lse = r[1].transpose(1, 2).reshape(nseq * width, -1)[slot]   # (total_q, nheads)
    return out, lse.transpose(0, 1).contiguous()
