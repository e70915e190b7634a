"""`torch.ops.fable_attn.forward`: the operator the reference registers for integrations that look
it up by name (package/fable_attn/torch_op.py:27-71, registered at import, __init__.py:29).

    forward(Tensor q, Tensor k, Tensor v, float scale, bool causal) -> Tensor

q, k, v are [B, H, S, D] (the layout of F.scaled_dot_product_attention); the result is
[B, H, S, D]. A shape or dtype the kernels cannot serve returns an EMPTY tensor instead of
raising: callers test `numel() == 0` and take their own path, so an exception here would break
their fallback (reference :27-48). fp16/bf16 head dims run as they are when they are multiples
of 8; others are zero-padded to the next multiple of 8, as in flash_attn_func. Registration is
idempotent and never raises (a failure is kept in LAST_ERROR); an operator of that name that
already exists is left alone (reference :51-71).
"""
import torch

LAST_ERROR = None
REGISTERED = False

_LIB = None


def _forward(q, k, v, scale, causal):
    from . import _C
    from .flash_attn_interface import _kernel_width, _with_width
    empty = q.new_empty(0)
    if q.dim() != 4 or k.dim() != 4 or v.dim() != 4:
        return empty
    if q.dtype not in (torch.float16, torch.bfloat16) or not q.is_cuda:
        return empty
    if k.dtype != q.dtype or v.dtype != q.dtype or not (k.is_cuda and v.is_cuda):
        return empty
    D = q.shape[-1]
    if k.shape[-1] != D or v.shape[-1] != D or D > 256:
        return empty
    if q.shape[1] % k.shape[1] or k.shape[:3] != v.shape[:3] or q.shape[0] != k.shape[0]:
        return empty
    dk = _kernel_width(D, q.dtype)
    try:
        # kernel views: [B,H,S,D] with a contiguous, 16-byte aligned head_dim
        views = []
        for t in (q, k, v):
            t = _with_width(t, dk)
            if not _C._rows_aligned(t):
                t = t.transpose(1, 2).contiguous().transpose(1, 2)
            views.append(t)
        out, _ = _C.fwd(views[0], views[1], views[2], float(scale), bool(causal), -1,
                        0 if causal else -1, 0.0, None, 0.0, 0, 0, None)
    except Exception:
        return empty
    return out if dk == D else out[..., :D]


def register():
    """Idempotent; never raises (a failed registration must not break `import fable_attn`)."""
    global _LIB, REGISTERED, LAST_ERROR
    if REGISTERED:
        return True
    try:
        ns = getattr(torch.ops, "fable_attn", None)
        if ns is not None and hasattr(ns, "forward"):
            REGISTERED = True
            return True
    except Exception:
        pass
    try:
        _LIB = torch.library.Library("fable_attn", "FRAGMENT")
        _LIB.define("forward(Tensor q, Tensor k, Tensor v, float scale, bool causal) -> Tensor")
        _LIB.impl("forward", _forward, "CUDA")
        REGISTERED = True
        return True
    except Exception as e:
        LAST_ERROR = f"{type(e).__name__}: {e}"
        return False
