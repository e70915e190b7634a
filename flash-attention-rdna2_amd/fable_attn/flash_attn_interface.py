"""flash_attn API (FA-2 argument order) over the gfx950 kernels of libfable_attn_hip.so.

Same public surface, argument order, defaults, shapes and error behaviour as the reference's
package/fable_attn/flash_attn_interface.py:
    flash_attn_func                  :378-388   flash_attn_qkvpacked_func        :391-401
    flash_attn_kvpacked_func         :404-414   flash_attn_varlen_func           :417-540
    flash_attn_varlen_qkvpacked_func :543-551   flash_attn_varlen_kvpacked_func  :554-564
    flash_attn_combine               :567-580   flash_attn_with_kvcache          :583-771
Inputs are (batch, seqlen, nheads, headdim); the kernels take [B,H,S,D] strided views, so the
wrapper only transposes views. There is no silent fallback: an unsupported configuration
raises, and a missing library raises ImportError at import time.
"""
import itertools
import math
import random

import torch
import torch.nn.functional as F

from . import _C

# head_dims the kernels are instantiated for; others are zero-padded up to the next one
# (zero columns change neither q.k nor the kept output columns).
KERNEL_HEAD_DIMS = (64, 128, 256)
MAX_HEAD_DIM = KERNEL_HEAD_DIMS[-1]


def _kernel_dim(d):
    for x in KERNEL_HEAD_DIMS:
        if x >= d:
            return x
    return None


def _pad_last(t, d):
    return t if t.shape[-1] == d else F.pad(t, (0, d - t.shape[-1]))


def _map_window(causal, window_size):
    """(causal, (left, right)) -> (causal_flag, win_left, win_right), reference :76-95.
    Key j is visible to query i when i+delta-left <= j <= i+delta+right (delta = SK-SQ); a
    negative bound is absent; causal pins right to 0; the flag is set whenever right == 0."""
    left, right = window_size
    wl = int(left) if left is not None and left >= 0 else -1
    wr = int(right) if right is not None and right >= 0 else -1
    if causal:
        wr = 0
    return (1 if wr == 0 else 0), wl, wr


def _reject_fp8(q_descale, k_descale, v_descale):
    """FP8 descaling is refused loudly (reference :99-107)."""
    if q_descale is not None or k_descale is not None or v_descale is not None:
        raise NotImplementedError(
            "fable_attn: q_descale/k_descale/v_descale (FP8) are not supported; "
            "pass fp16 or bf16 tensors")


def _accept_hints(num_splits=None, pack_gqa=None, sm_margin=None):
    """Scheduling hints change the schedule, never the result; only their types are checked
    (reference :110-128). num_splits is used by decode."""
    if num_splits is not None and not isinstance(num_splits, int):
        raise TypeError(f"fable_attn: num_splits must be int, got {type(num_splits)}")
    if pack_gqa is not None and not isinstance(pack_gqa, bool):
        raise TypeError(f"fable_attn: pack_gqa must be bool or None, got {type(pack_gqa)}")
    if sm_margin is not None and not isinstance(sm_margin, int):
        raise TypeError(f"fable_attn: sm_margin must be int, got {type(sm_margin)}")


def _check_chunk(attention_chunk):
    if attention_chunk is None:
        return 0
    if not isinstance(attention_chunk, int) or attention_chunk < 0:
        raise ValueError(f"fable_attn: attention_chunk must be a non-negative int, "
                         f"got {attention_chunk!r}")
    return attention_chunk


def _check_supported(q, k):
    """Reference :140-156 (head count is axis 2 of the public layout)."""
    if not q.is_cuda:
        raise ValueError("fable_attn: tensors must be on the GPU (q.is_cuda == False)")
    if q.shape[-1] > MAX_HEAD_DIM:
        raise ValueError(f"fable_attn: head_dim={q.shape[-1]} exceeds the maximum {MAX_HEAD_DIM}")
    if q.dtype not in (torch.float16, torch.bfloat16, torch.float32):
        raise ValueError(f"fable_attn: dtype {q.dtype} is not supported; use fp16, bf16 or fp32")
    if q.shape[2] % k.shape[2] != 0:
        raise ValueError(f"fable_attn: nheads_q={q.shape[2]} is not a multiple of "
                         f"nheads_k={k.shape[2]} (GQA)")


def _fuse_qv(q, k, v, qv):
    """FA-3's qv term, S = q.k^T + qv.v^T, as one attention over concatenated head dims:
    [q | qv] . [k | v]^T, values [v | 0]; the first dv output columns are P.V (reference
    :160-191). Also covers headdim_v != headdim (qv = 0)."""
    d, dv = q.shape[-1], v.shape[-1]
    if d + dv > MAX_HEAD_DIM:
        raise NotImplementedError(
            f"fable_attn: qv / headdim_v needs a score head_dim of {d}+{dv}={d + dv}, "
            f"above the kernel maximum {MAX_HEAD_DIM}")
    if qv is None:
        qv = q.new_zeros(q.shape[:-1] + (dv,))
    elif qv.shape[-1] != dv:
        raise ValueError(f"fable_attn: qv.shape[-1]={qv.shape[-1]} must equal v.shape[-1]={dv}")
    qc = torch.cat([q, qv], dim=-1)
    kc = torch.cat([k, v], dim=-1)
    vc = torch.cat([v, torch.zeros_like(v[..., :d])], dim=-1) if d else v
    return qc, kc, vc, dv


def _needs_qv_path(q, v, qv):
    return qv is not None or v.shape[-1] != q.shape[-1]


def _kernel_view(t):
    """(B,S,H,D) -> [B,H,S,D] view the kernels accept without a copy when rows are 16-byte
    aligned; otherwise a contiguous copy."""
    v = t.transpose(1, 2)
    el = v.element_size()
    ok = (v.stride(-1) == 1 and v.data_ptr() % 16 == 0 and
          all((s * el) % 16 == 0 for s in v.stride()[:-1]))
    return v if ok else t.contiguous().transpose(1, 2)


class _FableAttnFn(torch.autograd.Function):
    """Autograd over the forward/backward kernels (reference :233-262). deterministic is a
    no-op: the backward is atomic-free and always bitwise reproducible."""

    @staticmethod
    def forward(ctx, q, k, v, scale, causal, wl, wr, softcap, alibi, dropout_p, deterministic,
                attn_chunk, out_buf):
        seed = random.getrandbits(63) if dropout_p > 0 else 0
        out, lse = _C.fwd(q, k, v, float(scale), bool(causal), int(wl), int(wr), float(softcap),
                          alibi, float(dropout_p), int(seed), int(attn_chunk), out_buf)
        ctx.save_for_backward(q, k, v, out, lse, alibi if alibi is not None else torch.empty(0))
        ctx.scale, ctx.causal, ctx.wl, ctx.wr, ctx.softcap = scale, causal, wl, wr, softcap
        ctx.dropout_p, ctx.seed, ctx.has_alibi, ctx.attn_chunk = dropout_p, seed, alibi is not None, attn_chunk
        return out, lse

    @staticmethod
    def backward(ctx, dout, dlse):
        if ctx.attn_chunk:
            raise NotImplementedError(
                "fable_attn: backward with attention_chunk is not supported (as in FA-3); "
                "run the chunked forward under torch.no_grad()")
        q, k, v, out, lse, alibi = ctx.saved_tensors
        dq, dk, dv = _C.bwd(_kernel_view(dout.transpose(1, 2)), q, k, v, out, lse,
                            float(ctx.scale), bool(ctx.causal), int(ctx.wl), int(ctx.wr),
                            float(ctx.softcap), alibi if ctx.has_alibi else None,
                            float(ctx.dropout_p), int(ctx.seed))
        return dq, dk, dv, None, None, None, None, None, None, None, None, None, None


class _FableVarlenFn(torch.autograd.Function):
    """Autograd over the packed variable-length kernels: one forward launch (with LSE) and one
    launch of each backward kernel for all sequences. The reference has no native varlen
    backward and differentiates a per-sequence Python loop (:523-540)."""

    @staticmethod
    def forward(ctx, q, k, v, cu_q, cu_k, max_sq, max_sk, scale, causal, wl, wr, softcap, alibi,
                dropout_p, attn_chunk, su_q, su_k):
        seed = random.getrandbits(63) if dropout_p > 0 else 0
        out, lse = _C.fwd_varlen(q, k, v, cu_q, cu_k, max_sq, max_sk, float(scale), bool(causal),
                                 int(wl), int(wr), float(softcap), alibi, float(dropout_p),
                                 int(seed), int(attn_chunk), su_q, su_k, return_lse=True)
        empty = torch.empty(0, device=q.device)
        ctx.save_for_backward(q, k, v, out, lse, cu_q, cu_k,
                              alibi if alibi is not None else empty,
                              su_q if su_q is not None else empty,
                              su_k if su_k is not None else empty)
        ctx.args = (max_sq, max_sk, scale, causal, wl, wr, softcap, dropout_p, seed, attn_chunk,
                    alibi is not None, su_q is not None, su_k is not None)
        return out

    @staticmethod
    def backward(ctx, dout):
        (max_sq, max_sk, scale, causal, wl, wr, softcap, dropout_p, seed, attn_chunk,
         has_alibi, has_suq, has_suk) = ctx.args
        if attn_chunk:
            raise NotImplementedError(
                "fable_attn: backward with attention_chunk is not supported (as in FA-3); "
                "run the chunked forward under torch.no_grad()")
        q, k, v, out, lse, cu_q, cu_k, alibi, su_q, su_k = ctx.saved_tensors
        dq, dk, dv = _C.bwd_varlen(dout.contiguous(), q, k, v, out, lse, cu_q, cu_k, max_sq,
                                   max_sk, float(scale), bool(causal), int(wl), int(wr),
                                   float(softcap), alibi if has_alibi else None,
                                   float(dropout_p), int(seed),
                                   su_q if has_suq else None, su_k if has_suk else None)
        return (dq, dk, dv) + (None,) * 14


def _attn_probs(q, k, lse, scale, causal, wl, wr, softcap, alibi, attn_chunk):
    """Debug path for return_attn_probs: the full [B,Hq,SQ,SK] probability matrix from the
    kernel's LSE, p = exp(s - lse) (reference :266-308). Materialises S x S."""
    B, Hq, SQ, D = q.shape
    Hk, SK = k.shape[1], k.shape[2]
    need = B * Hq * SQ * SK * 4
    free = torch.cuda.mem_get_info(q.device)[0]
    if need > free * 0.8:
        raise torch.cuda.OutOfMemoryError(
            f"fable_attn: return_attn_probs needs a {need / 2**30:.1f} GiB S x S matrix "
            f"({free / 2**30:.1f} GiB free); the kernel itself never materialises it")
    kk = k if Hk == Hq else k.repeat_interleave(Hq // Hk, dim=1)
    s = torch.matmul(q.float(), kk.float().transpose(-1, -2).contiguous())
    s = softcap * torch.tanh(s * scale / softcap) if softcap and softcap > 0 else s * scale
    delta = SK - SQ
    qi = torch.arange(SQ, device=q.device).view(-1, 1)
    ki = torch.arange(SK, device=q.device).view(1, -1)
    if alibi is not None:
        s = s + alibi.view(1, Hq, 1, 1).float() * (ki - qi).float()
    mask = torch.zeros(SQ, SK, device=q.device, dtype=torch.bool)
    if causal:
        mask |= ki > qi + delta
    if wl >= 0:
        mask |= ki < qi + delta - wl
    if wr >= 0:
        mask |= ki > qi + delta + wr
    if attn_chunk:
        cs = ((qi + delta).clamp_min(0) // attn_chunk) * attn_chunk
        mask |= (ki < cs) | (ki >= cs + attn_chunk)
    p = torch.exp(s - lse.unsqueeze(-1))
    return p.masked_fill(mask, 0.0)


def _fwd_bshd(q, k, v, dropout_p, softmax_scale, causal, window_size, softcap, alibi_slopes,
              deterministic, return_attn_probs, qv, attention_chunk,
              q_descale, k_descale, v_descale, num_splits, pack_gqa, sm_margin):
    """Shared body of flash_attn_func and the packed wrappers, input (B,S,H,D)
    (reference :312-374)."""
    _reject_fp8(q_descale, k_descale, v_descale)
    _accept_hints(num_splits, pack_gqa, sm_margin)
    chunk = _check_chunk(attention_chunk)
    dv_out = None
    if _needs_qv_path(q, v, qv):
        if softmax_scale is None:
            softmax_scale = (q.shape[-1] + v.shape[-1]) ** (-0.5)
        q, k, v, dv_out = _fuse_qv(q, k, v, qv)
    elif softmax_scale is None:
        softmax_scale = 1.0 / math.sqrt(q.shape[-1])
    _check_supported(q, k)
    cflag, wl, wr = _map_window(causal, window_size)
    d_real = q.shape[-1]
    d_ker = _kernel_dim(d_real)
    if d_ker != d_real:
        q, k, v = _pad_last(q, d_ker), _pad_last(k, d_ker), _pad_last(v, d_ker)
        if dv_out is None:
            dv_out = d_real
    B, SQ, Hq, D = q.shape
    qh, kh, vh = _kernel_view(q), _kernel_view(k), _kernel_view(v)
    out_buf = torch.empty((B, SQ, Hq, D), dtype=q.dtype, device=q.device).transpose(1, 2)
    al = alibi_slopes.float().contiguous() if alibi_slopes is not None else None
    out, lse = _FableAttnFn.apply(qh, kh, vh, softmax_scale, cflag, wl, wr, softcap, al,
                                  dropout_p, deterministic, chunk, out_buf)
    res = out.transpose(1, 2)
    if dv_out is not None:
        res = res[..., :dv_out].contiguous()
    if return_attn_probs:
        probs = _attn_probs(qh, kh, lse, softmax_scale, bool(cflag), wl, wr, softcap, al, chunk)
        return res, lse, probs
    return res


def flash_attn_func(q, k, v, dropout_p=0.0, softmax_scale=None, causal=False,
                    window_size=(-1, -1), softcap=0.0, alibi_slopes=None,
                    deterministic=False, return_attn_probs=False, *,
                    qv=None, attention_chunk=0,
                    q_descale=None, k_descale=None, v_descale=None,
                    num_splits=1, pack_gqa=None, sm_margin=0):
    """q, k, v: (batch, seqlen, nheads, headdim). Returns out in the same layout (dense), or
    (out, softmax_lse, S_dmask) when return_attn_probs=True."""
    return _fwd_bshd(q, k, v, dropout_p, softmax_scale, causal, window_size, softcap,
                     alibi_slopes, deterministic, return_attn_probs, qv, attention_chunk,
                     q_descale, k_descale, v_descale, num_splits, pack_gqa, sm_margin)


def flash_attn_qkvpacked_func(qkv, dropout_p=0.0, softmax_scale=None, causal=False,
                              window_size=(-1, -1), softcap=0.0, alibi_slopes=None,
                              deterministic=False, return_attn_probs=False, *,
                              qv=None, attention_chunk=0,
                              q_descale=None, k_descale=None, v_descale=None,
                              num_splits=1, pack_gqa=None, sm_margin=0):
    """qkv: (batch, seqlen, 3, nheads, headdim)."""
    return _fwd_bshd(qkv[:, :, 0], qkv[:, :, 1], qkv[:, :, 2], dropout_p, softmax_scale, causal,
                     window_size, softcap, alibi_slopes, deterministic, return_attn_probs, qv,
                     attention_chunk, q_descale, k_descale, v_descale, num_splits, pack_gqa,
                     sm_margin)


def flash_attn_kvpacked_func(q, kv, dropout_p=0.0, softmax_scale=None, causal=False,
                             window_size=(-1, -1), softcap=0.0, alibi_slopes=None,
                             deterministic=False, return_attn_probs=False, *,
                             qv=None, attention_chunk=0,
                             q_descale=None, k_descale=None, v_descale=None,
                             num_splits=1, pack_gqa=None, sm_margin=0):
    """q: (batch, sq, nheads, d); kv: (batch, sk, 2, nheads_k, d)."""
    return _fwd_bshd(q, kv[:, :, 0], kv[:, :, 1], dropout_p, softmax_scale, causal, window_size,
                     softcap, alibi_slopes, deterministic, return_attn_probs, qv,
                     attention_chunk, q_descale, k_descale, v_descale, num_splits, pack_gqa,
                     sm_margin)


def _unpage_varlen_kv(k, v, block_table, cu_seqlens_k, seqused_k):
    """Paged K/V for varlen prefill: gather each sequence's pages into a packed (total, H, D)
    layout (reference :438-469)."""
    if k.dim() != 4 or v.dim() != 4:
        raise ValueError(
            "fable_attn: with block_table, k and v must be paged "
            f"(num_blocks, page_block_size, nheads_k, headdim); got k.shape={tuple(k.shape)}")
    bt = block_table.to(torch.int32)
    if bt.dim() != 2 or bt.shape[0] != cu_seqlens_k.numel() - 1:
        raise ValueError(f"fable_attn: block_table must be (batch, max_blocks), got "
                         f"{tuple(bt.shape)} for batch={cu_seqlens_k.numel() - 1}")
    page = k.shape[1]
    lens = ((cu_seqlens_k[1:] - cu_seqlens_k[:-1]) if seqused_k is None else seqused_k).tolist()
    ks, vs = [], []
    for i, L in enumerate(int(x) for x in lens):
        idx = bt[i, :(L + page - 1) // page].long()
        ks.append(k[idx].reshape(-1, k.shape[2], k.shape[3])[:L])
        vs.append(v[idx].reshape(-1, v.shape[2], v.shape[3])[:L])
    cu = torch.tensor([0] + list(itertools.accumulate(int(x) for x in lens)),
                      device=k.device, dtype=torch.int32)
    return torch.cat(ks, 0).contiguous(), torch.cat(vs, 0).contiguous(), cu


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
    cu_seqlens_* int32 (batch+1). One forward launch over all sequences; with grad the
    backward is one launch of each backward kernel over all sequences as well (the reference
    loops over the sequences in Python on the grad path, :523-540)."""
    _reject_fp8(q_descale, k_descale, v_descale)
    _accept_hints(num_splits, pack_gqa, sm_margin)
    chunk = _check_chunk(attention_chunk)
    if block_table is not None:
        k, v, cu_seqlens_k = _unpage_varlen_kv(k, v, block_table, cu_seqlens_k, seqused_k)
        seqused_k = None
    dv_out = None
    if _needs_qv_path(q, v, qv):
        if softmax_scale is None:
            softmax_scale = (q.shape[-1] + v.shape[-1]) ** (-0.5)
        q, k, v, dv_out = _fuse_qv(q, k, v, qv)
    elif softmax_scale is None:
        softmax_scale = 1.0 / math.sqrt(q.shape[-1])
    need_grad = torch.is_grad_enabled() and (q.requires_grad or k.requires_grad or v.requires_grad)
    if q.dim() != 3:
        raise ValueError(f"fable_attn: varlen expects (total, nheads, headdim), got {tuple(q.shape)}")
    if q.shape[-1] > MAX_HEAD_DIM:
        raise ValueError(f"fable_attn: head_dim={q.shape[-1]} exceeds the maximum {MAX_HEAD_DIM}")
    if not q.is_cuda:
        raise ValueError("fable_attn: tensors must be on the GPU (q.is_cuda == False)")
    if q.shape[1] % k.shape[1] != 0:
        raise ValueError(f"fable_attn: GQA needs nheads_q ({q.shape[1]}) divisible by nheads_k ({k.shape[1]})")
    d_real = q.shape[-1]
    d_ker = _kernel_dim(d_real)
    if d_ker != d_real:
        q, k, v = _pad_last(q, d_ker), _pad_last(k, d_ker), _pad_last(v, d_ker)
        if dv_out is None:
            dv_out = d_real
    cflag, wl, wr = _map_window(causal, window_size)
    al = alibi_slopes.float().contiguous() if alibi_slopes is not None else None
    su_q = seqused_q.to(torch.int32).contiguous() if seqused_q is not None else None
    su_k = seqused_k.to(torch.int32).contiguous() if seqused_k is not None else None
    cu_q = cu_seqlens_q.to(torch.int32).contiguous()
    cu_k = cu_seqlens_k.to(torch.int32).contiguous()
    if need_grad:
        out = _FableVarlenFn.apply(q.contiguous(), k.contiguous(), v.contiguous(), cu_q, cu_k,
                                   int(max_seqlen_q), int(max_seqlen_k), float(softmax_scale),
                                   bool(cflag), int(wl), int(wr), float(softcap), al,
                                   float(dropout_p), int(chunk), su_q, su_k)
    else:
        seed = random.getrandbits(63) if dropout_p > 0 else 0
        out = _C.fwd_varlen(q.contiguous(), k.contiguous(), v.contiguous(), cu_q, cu_k,
                            int(max_seqlen_q), int(max_seqlen_k), float(softmax_scale),
                            bool(cflag), int(wl), int(wr), float(softcap), al, float(dropout_p),
                            int(seed), int(chunk), su_q, su_k)
    if dv_out is not None:
        out = out[..., :dv_out]
    if return_attn_probs:
        lse_l, probs_l = [], []
        with torch.no_grad():
            for i in range(cu_seqlens_q.numel() - 1):
                a, b = int(cu_seqlens_q[i]), int(cu_seqlens_q[i + 1])
                c, d = int(cu_seqlens_k[i]), int(cu_seqlens_k[i + 1])
                if seqused_q is not None:
                    b = a + int(seqused_q[i])
                if seqused_k is not None:
                    d = c + int(seqused_k[i])
                _, li, pi = flash_attn_func(q[a:b].unsqueeze(0), k[c:d].unsqueeze(0),
                                            v[c:d].unsqueeze(0), dropout_p, softmax_scale,
                                            causal, window_size, softcap, alibi_slopes,
                                            deterministic, True, attention_chunk=chunk)
                lse_l.append(li.squeeze(0))
                probs_l.append(pi.squeeze(0))
        return out, lse_l, probs_l
    return out


def flash_attn_varlen_qkvpacked_func(qkv, cu_seqlens, max_seqlen, dropout_p=0.0,
                                     softmax_scale=None, causal=False, window_size=(-1, -1),
                                     softcap=0.0, alibi_slopes=None, deterministic=False,
                                     return_attn_probs=False, **kw):
    """qkv: (total_tokens, 3, nheads, headdim)."""
    return flash_attn_varlen_func(qkv[:, 0], qkv[:, 1], qkv[:, 2], cu_seqlens, cu_seqlens,
                                  max_seqlen, max_seqlen, dropout_p, softmax_scale, causal,
                                  window_size, softcap, alibi_slopes, deterministic,
                                  return_attn_probs, **kw)


def flash_attn_varlen_kvpacked_func(q, kv, cu_seqlens_q, cu_seqlens_k, max_seqlen_q,
                                    max_seqlen_k, dropout_p=0.0, softmax_scale=None,
                                    causal=False, window_size=(-1, -1), softcap=0.0,
                                    alibi_slopes=None, deterministic=False,
                                    return_attn_probs=False, **kw):
    """q: (total_q, nheads, d); kv: (total_k, 2, nheads_k, d)."""
    return flash_attn_varlen_func(q, kv[:, 0], kv[:, 1], cu_seqlens_q, cu_seqlens_k,
                                  max_seqlen_q, max_seqlen_k, dropout_p, softmax_scale, causal,
                                  window_size, softcap, alibi_slopes, deterministic,
                                  return_attn_probs, **kw)


def flash_attn_combine(out_partial, lse_partial, out=None, out_dtype=None):
    """Merge split-KV partials: out_partial (nsplit, B, S, H, D), lse_partial (nsplit, B, H, S)
    natural-log LSE -> (B, S, H, D). One HIP kernel (the reference used torch ops, :567-580)."""
    res = _C.combine(out_partial, lse_partial, out_dtype or out_partial.dtype)
    if out is not None:
        out.copy_(res)
        return out
    return res


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
    q: (batch, seqlen_q, nheads, d); the new tokens sit at cache_seqlens .. +seqlen_q-1 and are
    causal among themselves. cache_seqlens is the length before appending k/v. Returns out, or
    (out, softmax_lse (batch, nheads, seqlen_q)). Reference :583-771."""
    _reject_fp8(q_descale, k_descale, v_descale)
    _accept_hints(num_splits, pack_gqa, sm_margin)
    if q.dim() != 4:
        raise ValueError(f"fable_attn: decode expects q (batch, seqlen_q, nheads, headdim), "
                         f"got {tuple(q.shape)}")
    if softmax_scale is None:
        softmax_scale = (q.shape[-1] + (qv.shape[-1] if qv is not None else 0)) ** -0.5
    del scheduler_metadata  # a precomputed schedule is not needed: the launcher plans per call
    if cu_seqlens_k_new is not None:
        raise NotImplementedError(
            "fable_attn: cu_seqlens_k_new (ragged append) is not supported; append the same "
            "number of tokens to every batch element")
    if cu_seqlens_q is not None:
        cu = cu_seqlens_q.to(torch.int32).cpu()
        outs, lses = [], []
        for i in range(cu.numel() - 1):
            a, b = int(cu[i]), int(cu[i + 1])
            qi = q[a:b].unsqueeze(0) if q.dim() == 3 else q[:, a:b]
            csi = cache_seqlens[i:i + 1] if torch.is_tensor(cache_seqlens) else cache_seqlens
            r = flash_attn_with_kvcache(
                qi, k_cache, v_cache, k=k, v=v, qv=qv, rotary_cos=rotary_cos,
                rotary_sin=rotary_sin, cache_seqlens=csi, cache_batch_idx=cache_batch_idx,
                cache_leftpad=cache_leftpad, block_table=block_table,
                softmax_scale=softmax_scale, causal=causal, window_size=window_size,
                softcap=softcap, rotary_interleaved=rotary_interleaved,
                alibi_slopes=alibi_slopes, num_splits=num_splits,
                return_softmax_lse=return_softmax_lse, page_table=page_table,
                attention_chunk=attention_chunk, pack_gqa=pack_gqa, sm_margin=sm_margin,
                rotary_seqlens=rotary_seqlens)
            if return_softmax_lse:
                outs.append(r[0].squeeze(0))
                lses.append(r[1])
            else:
                outs.append(r.squeeze(0))
        out = torch.cat(outs, dim=0)
        return (out, torch.cat(lses, dim=0)) if return_softmax_lse else out
    if page_table is not None:
        if block_table is not None:
            raise ValueError("fable_attn: block_table and page_table are the same argument; pass one")
        block_table = page_table
    B, NQ = q.shape[0], q.shape[1]
    dev = q.device
    d_real = q.shape[-1]
    if not q.is_cuda:
        raise ValueError("fable_attn: tensors must be on the GPU (q.is_cuda == False)")
    if q.dtype not in (torch.float16, torch.bfloat16, torch.float32):
        raise ValueError(f"fable_attn: dtype {q.dtype} is not supported; use fp16, bf16 or fp32")
    if qv is not None:
        # same concatenation as the prefill qv path, applied to the whole cache (compat path)
        if qv.shape[-1] != v_cache.shape[-1]:
            raise ValueError("fable_attn: qv.shape[-1] must equal the value head_dim")
        if d_real + qv.shape[-1] > MAX_HEAD_DIM:
            raise NotImplementedError(f"fable_attn: qv in decode needs headdim+headdim_v <= {MAX_HEAD_DIM}")
        q = torch.cat([q, qv], dim=-1)
        k_cache = torch.cat([k_cache, v_cache], dim=-1)
        v_cache = torch.cat([v_cache, torch.zeros_like(v_cache[..., :d_real])], dim=-1)
        if k is not None:
            k = torch.cat([k, v], dim=-1)
            v = torch.cat([v, torch.zeros_like(v[..., :d_real])], dim=-1)
    if cache_seqlens is None:
        seqlens = torch.full((B,), k_cache.shape[1], dtype=torch.int32, device=dev)
    elif isinstance(cache_seqlens, int):
        seqlens = torch.full((B,), cache_seqlens, dtype=torch.int32, device=dev)
    else:
        seqlens = cache_seqlens.to(device=dev, dtype=torch.int32).contiguous()
    if block_table is None:
        # dense cache: one block per batch row, page = the whole row
        page = k_cache.shape[1]
        if page & (page - 1):
            raise NotImplementedError(
                f"fable_attn: dense cache length {page} must be a power of two (or pass block_table)")
        if cache_batch_idx is None:
            bt = torch.arange(B, dtype=torch.int32, device=dev).view(B, 1)
        else:
            bt = cache_batch_idx.to(device=dev, dtype=torch.int32).contiguous().view(B, 1)
    else:
        if cache_batch_idx is not None:
            raise ValueError("fable_attn: cache_batch_idx applies to a dense cache only; with a "
                             "paged cache the block_table selects the rows")
        bt = block_table.to(device=dev, dtype=torch.int32).contiguous()
    kc, vc = k_cache, v_cache
    # decode takes the window as "number of keys back from the query position"
    _, wl, _ = _map_window(True, window_size)
    win = (wl + 1) if wl >= 0 else -1
    lp = cache_leftpad.to(device=dev, dtype=torch.int32).contiguous() if cache_leftpad is not None else None
    chunk = _check_chunk(attention_chunk)
    if chunk:
        if NQ > 1:
            raise NotImplementedError(
                "fable_attn: attention_chunk in decode is supported for one new token: "
                "several tokens would need different chunk starts")
        cl = ((seqlens.to(torch.int64) // chunk) * chunk).to(torch.int32)
        lp = cl if lp is None else torch.maximum(lp, cl)
    al = alibi_slopes.float().contiguous() if alibi_slopes is not None else None
    cos = rotary_cos.float().contiguous() if rotary_cos is not None else None
    sin = rotary_sin.float().contiguous() if rotary_sin is not None else None
    rdim = int(cos.shape[-1] * 2) if cos is not None else 0
    rpos = (rotary_seqlens.to(device=dev, dtype=torch.int32).contiguous()
            if rotary_seqlens is not None else None)
    nk = k.contiguous() if k is not None else None
    nv = v.contiguous() if v is not None else None
    if (nk is None) != (nv is None):
        raise ValueError("fable_attn: k and v are appended to the cache together")
    dq = q.shape[-1]
    d_ker = _kernel_dim(dq)
    if d_ker is None:
        raise ValueError(f"fable_attn: head_dim={dq} exceeds the maximum {MAX_HEAD_DIM}")
    dv_cut = None
    if d_ker != dq:
        if nk is not None:
            raise NotImplementedError(
                f"fable_attn: appending k/v needs a kernel head_dim; {dq} is not one of "
                f"{KERNEL_HEAD_DIMS}")
        q, kc, vc = _pad_last(q, d_ker), _pad_last(kc, d_ker), _pad_last(vc, d_ker)
        dv_cut = dq
    if qv is not None:
        dv_cut = v_cache.shape[-1] - d_real if dv_cut is None else dv_cut
    out, lse = _C.dec(q.contiguous(), kc.contiguous(), vc.contiguous(), bt, seqlens, nk, nv,
                      cos, sin, bool(rotary_interleaved), float(softmax_scale), int(win),
                      int(num_splits or 0), lp, bool(return_softmax_lse),
                      float(softcap or 0.0), al, int(rdim), rpos)
    if qv is not None:
        out = out[..., :qv.shape[-1]].contiguous()
    elif dv_cut is not None:
        out = out[..., :dv_cut].contiguous()
    if return_softmax_lse:
        return out, lse.transpose(1, 2).contiguous()
    return out
