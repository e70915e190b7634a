"""torch.ops.fable_attn.forward on the GPU (reference package/fable_attn/torch_op.py:27-71): the
[B,H,S,D] operator gives the same bits as flash_attn_func on the transposed layout, pads head
dims without a kernel, and returns an empty tensor (never raises) for what it cannot serve."""
import pytest

pytestmark = pytest.mark.gpu


@pytest.mark.parametrize("D,causal,dt", [(64, True, "f16"), (128, False, "bf16"), (80, True, "f16")])
def test_op_matches_flash_attn_func(D, causal, dt):
    import torch

    import fable_attn  # noqa: F401  (registers the operator)
    from fable_attn import flash_attn_func
    dtype = torch.float16 if dt == "f16" else torch.bfloat16
    g = torch.Generator(device="cuda").manual_seed(D)
    B, H, Hk, S = 2, 4, 2, 150
    q = torch.randn(B, H, S, D, device="cuda", dtype=dtype, generator=g)
    k = torch.randn(B, Hk, S, D, device="cuda", dtype=dtype, generator=g)
    v = torch.randn(B, Hk, S, D, device="cuda", dtype=dtype, generator=g)
    scale = D ** -0.5
    o = torch.ops.fable_attn.forward(q, k, v, scale, causal)
    ref = flash_attn_func(q.transpose(1, 2), k.transpose(1, 2), v.transpose(1, 2),
                          softmax_scale=scale, causal=causal).transpose(1, 2)
    torch.cuda.synchronize()
    assert o.shape == (B, H, S, D)
    assert torch.equal(o, ref)


def test_op_empty_on_unsupported():
    import torch

    import fable_attn  # noqa: F401
    x = torch.randn(1, 2, 16, 64, device="cuda", dtype=torch.float16)
    op = torch.ops.fable_attn.forward
    assert op(x.float(), x.float(), x.float(), 0.125, True).numel() == 0       # fp32
    big = torch.randn(1, 2, 16, 320, device="cuda", dtype=torch.float16)
    assert op(big, big, big, 0.1, False).numel() == 0                          # head_dim > 256
    k3 = torch.randn(1, 3, 16, 64, device="cuda", dtype=torch.float16)
    assert op(x, k3, k3, 0.125, False).numel() == 0                            # 2 q heads, 3 kv
