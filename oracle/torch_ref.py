"""Exact fp32 torch restatement of the reference's attention test path (TEST INFRASTRUCTURE).

Semantics of lab/parity_new_api.py:36-75 (ref_attn) / lab/parity_test.py:20-44: s = q.k^T,
softcap or scale, alibi, mask, softmax, nan_to_num for empty rows, p.v. Used by bench.py as
the CPU baseline (run on CPU tensors on the GPU box's host cores) and by GPU tests as a second,
independent reference. The alibi term uses the kernel convention slope*(j - i)
(fa_common.hpp:123), not the torch gate's (j - i - delta) (parity_test.py:36).
"""
import torch


def attention_bhsd(q, k, v, scale, causal=False, win_left=-1, win_right=-1, softcap=0.0,
                   alibi=None, chunk=0):
    """q [B,H,SQ,D], k/v [B,Hk,SK,D] float32 (any device) -> [B,H,SQ,D] float32."""
    q, k, v = q.float(), k.float(), v.float()
    B, H, SQ, D = q.shape
    Hk, SK = k.shape[1], k.shape[2]
    if H != Hk:
        k = k.repeat_interleave(H // Hk, dim=1)
        v = v.repeat_interleave(H // Hk, dim=1)
    s = torch.matmul(q, k.transpose(-1, -2).contiguous())
    s = softcap * torch.tanh(s * scale / softcap) if softcap and softcap > 0 else s * scale
    qi = torch.arange(SQ, device=q.device).view(-1, 1)
    ki = torch.arange(SK, device=q.device).view(1, -1)
    delta = SK - SQ
    if alibi is not None:
        s = s + alibi.view(1, H, 1, 1).float() * (ki - qi).float()
    mask = torch.zeros(SQ, SK, device=q.device, dtype=torch.bool)
    if causal:
        mask |= ki > qi + delta
    if win_left >= 0:
        mask |= ki < qi + delta - win_left
    if win_right >= 0:
        mask |= ki > qi + delta + win_right
    if chunk:
        cs = ((qi + delta).clamp_min(0) // chunk) * chunk
        mask |= (ki < cs) | (ki >= cs + chunk)
    p = torch.nan_to_num(torch.softmax(s.masked_fill(mask, float("-inf")), dim=-1), nan=0.0)
    return torch.matmul(p, v)
