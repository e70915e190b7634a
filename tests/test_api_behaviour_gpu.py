"""Behaviour the reference's own package tests pin through the public API
(package/tests/test_fable_attn.py:142-164, 250-262, 277-293), on the GPU: dense (B,S,H,D)
output whatever the K/V layout, exact zeros for rows without a visible key, scheduler hints that
change nothing, bitwise determinism, and no S x S buffer."""
import numpy as np
import pytest

from oracle import oracle as orc
from tests.helpers import TOL, gen, log_errors, to_np

pytestmark = pytest.mark.gpu


def _bshd(a, dt):
    """[B,H,S,D] numpy -> (B,S,H,D) contiguous device tensor."""
    import torch
    from tests.helpers import torch_dtype
    return torch.from_numpy(np.ascontiguousarray(a.transpose(0, 2, 1, 3))).to("cuda", torch_dtype(dt))


def test_output_dense_and_independent_of_the_kv_layout():
    import torch

    from fable_attn import flash_attn_func
    B, S, H, D = 2, 256, 8, 128
    q, k, v = (gen((B, H, S, D), 60 + i, "f16") for i in range(3))
    tq, tk, tv = _bshd(q, "f16"), _bshd(k, "f16"), _bshd(v, "f16")
    print("[api] layout", flush=True)
    out = flash_attn_func(tq, tk, tv, causal=True)
    assert out.is_contiguous() and tuple(out.shape) == (B, S, H, D)
    out.view(B, S, H * D)  # the reshape attention blocks apply to the output
    # K/V as strided views of a [B,H,S,D] buffer instead of dense (B,S,H,D): same bits
    kh = tk.transpose(1, 2).contiguous().transpose(1, 2)
    vh = tv.transpose(1, 2).contiguous().transpose(1, 2)
    assert torch.equal(out, flash_attn_func(tq, kh, vh, causal=True))
    # the autograd path gives the same output
    og = flash_attn_func(tq.clone().requires_grad_(), tk, tv, causal=True)
    assert og.is_contiguous() and torch.equal(og.detach(), out)
    o_ref, _ = orc.fwd(q, k, v, D ** -0.5, True)
    e = orc.rel_rms(to_np(out).transpose(0, 2, 1, 3), o_ref)
    log_errors("api_layout", "causal B2 S256 D128", "f16", o=e)
    assert e <= TOL["f16"], e


@pytest.mark.parametrize("dt", ["f16", "bf16"])
def test_rows_without_a_visible_key_are_zero(dt):
    from fable_attn import flash_attn_func
    B, H, D, SQ, SK = 1, 4, 64, 256, 64
    q, k, v = gen((B, H, SQ, D), 70, dt), gen((B, H, SK, D), 71, dt), gen((B, H, SK, D), 72, dt)
    print(f"[api] empty rows {dt}", flush=True)
    out = to_np(flash_attn_func(_bshd(q, dt), _bshd(k, dt), _bshd(v, dt), causal=True))
    # bottom-right causal: query i sees keys j <= i + SK - SQ, so the first 192 rows see none
    assert (out[:, :SQ - SK] == 0).all()
    o_ref, _ = orc.fwd(q, k, v, D ** -0.5, True)
    e = orc.rel_rms(out.transpose(0, 2, 1, 3)[:, :, SQ - SK:], o_ref[:, :, SQ - SK:])
    log_errors("api_empty_rows", "SQ256 SK64 causal", dt, o=e)
    assert e <= TOL[dt], e


def test_scheduler_hints_and_repeats_change_nothing():
    import torch

    from fable_attn import flash_attn_func, flash_attn_varlen_func
    q, k, v = (_bshd(gen((1, 4, 128, 64), 80 + i, "f16"), "f16") for i in range(3))
    print("[api] hints", flush=True)
    base = flash_attn_func(q, k, v, causal=True)
    for kw in (dict(num_splits=4), dict(pack_gqa=True), dict(sm_margin=8)):
        assert torch.equal(flash_attn_func(q, k, v, causal=True, **kw), base), kw
    assert torch.equal(flash_attn_func(q, k, v, causal=True), base)
    cu = torch.tensor([0, 50, 128], dtype=torch.int32, device="cuda")
    qp, kp, vp = q[0], k[0], v[0]
    vb = flash_attn_varlen_func(qp, kp, vp, cu, cu, 78, 78, causal=True)
    for kw in (dict(num_splits=3), dict(pack_gqa=False), dict(sm_margin=4)):
        assert torch.equal(flash_attn_varlen_func(qp, kp, vp, cu, cu, 78, 78, causal=True, **kw), vb), kw


def test_no_s_by_s_buffer():
    import torch

    from fable_attn import flash_attn_func
    B, S, H, D = 2, 4096, 16, 128
    g = torch.Generator(device="cuda").manual_seed(13)
    q, k, v = (torch.randn(B, S, H, D, device="cuda", dtype=torch.float16, generator=g) for _ in range(3))
    print("[api] memory", flush=True)
    flash_attn_func(q, k, v, causal=True)  # warm (allocator, library)
    torch.cuda.synchronize()
    torch.cuda.reset_peak_memory_stats()
    base = torch.cuda.memory_allocated()
    out = flash_attn_func(q, k, v, causal=True)
    torch.cuda.synchronize()
    peak = torch.cuda.max_memory_allocated() - base
    # the output and the LSE (32 MiB + 0.5 MiB) against 2 GiB for one fp32 S x S score matrix
    assert peak <= out.numel() * out.element_size() + B * H * S * 4 + (1 << 20), peak
    assert peak < 0.05 * B * H * S * S * 4
