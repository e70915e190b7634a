"""Host logic of the public API on CPU (no GPU): argument mapping and error behaviour of
flash_attn_interface, with the C-ABI layer replaced by a recording fake.

Covers the reference's contract (package/fable_attn/flash_attn_interface.py): window mapping
:76-95, FP8 rejection :99-107 (message contains "FP8"), hint type checks :110-128,
attention_chunk validation :131-137 and backward rejection :253-256, device/head_dim/GQA checks
:140-156, qv fusion and its "256" overflow message :160-191, default softmax_scale :325-326,
head_dim padding, dense output layout :360, kvcache argument handling :619-771 and the FA-3
argument order (fa3_interface.py:26-102).
"""
import math

import pytest
import torch

import fable_attn
from fable_attn import fa3_interface
from fable_attn import flash_attn_interface as fai


class FakeC:
    """Records calls; returns zero outputs of the right shapes."""

    def __init__(self):
        self.calls = []

    def fwd(self, q, k, v, scale, causal, wl, wr, softcap, alibi, dropout_p, seed, chunk=0, out=None):
        self.calls.append(("fwd", dict(shape=tuple(q.shape), kshape=tuple(k.shape), scale=scale,
                                       causal=causal, wl=wl, wr=wr, softcap=softcap, chunk=chunk)))
        B, H, S, D = q.shape
        o = out if out is not None else torch.zeros((B, S, H, D), dtype=q.dtype).transpose(1, 2)
        o.zero_()
        return o, torch.zeros((B, H, S), dtype=torch.float32)

    def bwd(self, dout, q, k, v, out, lse, *a):
        self.calls.append(("bwd", a))
        return torch.ones_like(q), torch.ones_like(k), torch.ones_like(v)

    def fwd_varlen(self, q, k, v, cu_q, cu_k, mq, mk, scale, causal, wl, wr, sc, al, dp, seed, chunk,
                   uq, uk, return_lse=False):
        self.calls.append(("fwd_varlen", dict(shape=tuple(q.shape), mq=mq, mk=mk, scale=scale,
                                              causal=causal, wl=wl, wr=wr, return_lse=return_lse)))
        out = torch.zeros_like(q)
        return (out, torch.zeros((q.shape[1], q.shape[0]))) if return_lse else out

    def bwd_varlen(self, dout, q, k, v, out, lse, cu_q, cu_k, mq, mk, scale, causal, wl, wr, sc, al,
                   dp, seed, uq=None, uk=None):
        self.calls.append(("bwd_varlen", dict(shape=tuple(q.shape), kshape=tuple(k.shape), mq=mq,
                                              mk=mk, causal=causal, lse=tuple(lse.shape))))
        return torch.full_like(q, 2.0), torch.full_like(k, 3.0), torch.full_like(v, 4.0)

    def dec(self, q, kc, vc, bt, seqlens, nk, nv, cos, sin, inter, scale, window, num_splits,
            lp=None, return_lse=False, softcap=0.0, alibi=None, rdim=0, rpos=None):
        self.calls.append(("dec", dict(q=tuple(q.shape), kc=tuple(kc.shape), bt=bt.clone(),
                                       seqlens=seqlens.clone(), window=window, scale=scale,
                                       lp=None if lp is None else lp.clone(), rdim=rdim,
                                       num_splits=num_splits, append=nk is not None)))
        B, NQ, H, D = q.shape
        return torch.zeros((B, NQ, H, D), dtype=q.dtype), torch.zeros((B, NQ, H))


@pytest.fixture
def fake(monkeypatch):
    f = FakeC()
    monkeypatch.setattr(fai, "_C", f)
    # CPU tensors stand in for GPU ones; the device check itself is tested separately
    monkeypatch.setattr(torch.Tensor, "is_cuda", property(lambda self: True))
    return f


def rnd(*s, dt=torch.float16):
    return torch.randn(*s).to(dt)


@pytest.mark.parametrize("causal,ws,expect", [
    (False, (-1, -1), (0, -1, -1)), (True, (-1, -1), (1, -1, 0)), (False, (-1, 0), (1, -1, 0)),
    (False, (32, 32), (0, 32, 32)), (True, (63, 5), (1, 63, 0)), (False, (0, -1), (0, 0, -1)),
    (False, (None, None), (0, -1, -1)),
])
def test_map_window(causal, ws, expect):
    assert fai._map_window(causal, ws) == expect


def test_rejections_before_any_launch(fake):
    q = rnd(1, 32, 2, 64)
    with pytest.raises(NotImplementedError, match="FP8"):
        fai.flash_attn_func(q, q, q, q_descale=torch.ones(1))
    with pytest.raises(TypeError):
        fai.flash_attn_func(q, q, q, num_splits=1.5)
    with pytest.raises(TypeError):
        fai.flash_attn_func(q, q, q, pack_gqa="yes")
    with pytest.raises(TypeError):
        fai.flash_attn_func(q, q, q, sm_margin=0.5)
    with pytest.raises(ValueError):
        fai.flash_attn_func(q, q, q, attention_chunk=-3)
    with pytest.raises(ValueError, match="GQA"):
        fai.flash_attn_func(rnd(1, 32, 3, 64), q, q)
    with pytest.raises(ValueError, match="head_dim"):
        big = rnd(1, 8, 2, 320)
        fai.flash_attn_func(big, big, big)
    with pytest.raises(NotImplementedError, match="256"):
        fai.flash_attn_func(rnd(1, 8, 2, 192), rnd(1, 8, 2, 192), rnd(1, 8, 2, 192), qv=rnd(1, 8, 2, 192))
    with pytest.raises(ValueError, match="dtype"):
        x = rnd(1, 8, 2, 64, dt=torch.float64)   # fp16, bf16 and fp32 are served (reference :149)
        fai.flash_attn_func(x, x, x)
    assert fake.calls == []


def test_cpu_tensors_rejected():
    q = rnd(1, 16, 2, 64)
    with pytest.raises(ValueError, match="GPU"):
        fai.flash_attn_func(q, q, q)


def test_forward_argument_mapping(fake):
    q, k, v = rnd(2, 40, 8, 64), rnd(2, 48, 2, 64), rnd(2, 48, 2, 64)
    out = fai.flash_attn_func(q, k, v, causal=True, window_size=(16, 3), softcap=5.0)
    name, a = fake.calls[-1]
    assert name == "fwd" and a["shape"] == (2, 8, 40, 64) and a["kshape"] == (2, 2, 48, 64)
    assert a["causal"] == 1 and a["wl"] == 16 and a["wr"] == 0 and a["softcap"] == 5.0
    assert math.isclose(a["scale"], 1 / 8)
    assert out.shape == (2, 40, 8, 64) and out.is_contiguous()   # dense (B,S,H,D)
    out.view(2, 40, 8 * 64)


def test_head_dim_padding_and_slicing(fake):
    """Head dims that are multiples of 8 go to the kernels as they are (every dtype); others
    are zero-padded to the next multiple of 8; the scale and the output keep the real head dim."""
    for D, dt, width in ((80, torch.float16, 80), (40, torch.bfloat16, 40), (100, torch.float16, 104),
                         (80, torch.float32, 80), (24, torch.float32, 24), (20, torch.float32, 24)):
        q = rnd(1, 16, 2, D, dt=dt)
        out = fai.flash_attn_func(q, q, q)
        assert fake.calls[-1][1]["shape"][-1] == width, (D, dt)
        assert math.isclose(fake.calls[-1][1]["scale"], D ** -0.5)   # scale of the real head_dim
        assert out.shape == (1, 16, 2, D) and out.is_contiguous()


def test_qv_fusion_shapes_and_scale(fake):
    q, k, v, qv = rnd(1, 8, 2, 64), rnd(1, 8, 2, 64), rnd(1, 8, 2, 64), rnd(1, 8, 2, 64)
    out = fai.flash_attn_func(q, k, v, qv=qv, causal=True)
    a = fake.calls[-1][1]
    assert a["shape"][-1] == 128 and math.isclose(a["scale"], 128 ** -0.5)
    assert out.shape == (1, 8, 2, 64)


def test_chunk_backward_rejected(fake):
    q, k, v = (rnd(1, 16, 2, 64).requires_grad_() for _ in range(3))
    out = fai.flash_attn_func(q, k, v, attention_chunk=8)
    with pytest.raises(NotImplementedError, match="attention_chunk"):
        out.sum().backward()


def test_backward_routes_to_bwd(fake):
    q, k, v = (rnd(1, 16, 2, 64).requires_grad_() for _ in range(3))
    fai.flash_attn_func(q, k, v, causal=True).sum().backward()
    assert fake.calls[-1][0] == "bwd" and q.grad is not None and q.grad.shape == q.shape


def test_packed_variants(fake):
    qkv = rnd(2, 24, 3, 4, 64)
    fai.flash_attn_qkvpacked_func(qkv, causal=True)
    assert fake.calls[-1][1]["shape"] == (2, 4, 24, 64)
    fai.flash_attn_kvpacked_func(rnd(2, 24, 4, 64), rnd(2, 30, 2, 2, 64))
    assert fake.calls[-1][1]["kshape"] == (2, 2, 30, 64)


def test_varlen_no_grad_single_launch(fake):
    cu = torch.tensor([0, 5, 12], dtype=torch.int32)
    q = rnd(12, 4, 64)
    fai.flash_attn_varlen_func(q, q, q, cu, cu, 7, 7, causal=True, window_size=(3, -1))
    name, a = fake.calls[-1]
    assert name == "fwd_varlen" and a["mq"] == 7 and a["causal"] == 1 and a["wl"] == 3 and a["wr"] == 0


def test_varlen_grad_is_one_native_call_each_way(fake):
    """With grad, varlen runs one forward (with LSE) and one backward over all sequences; the
    reference differentiated a per-sequence Python loop (flash_attn_interface.py:523-540)."""
    cu = torch.tensor([0, 5, 12, 20], dtype=torch.int32)
    q = rnd(20, 4, 64).requires_grad_()
    k = rnd(20, 2, 64).requires_grad_()
    v = rnd(20, 2, 64).requires_grad_()
    out = fai.flash_attn_varlen_func(q, k, v, cu, cu, 8, 8, causal=True)
    assert [c[0] for c in fake.calls] == ["fwd_varlen"] and fake.calls[0][1]["return_lse"]
    out.sum().backward()
    assert [c[0] for c in fake.calls] == ["fwd_varlen", "bwd_varlen"]
    a = fake.calls[1][1]
    assert a["shape"] == (20, 4, 64) and a["kshape"] == (20, 2, 64) and a["lse"] == (4, 20)
    assert a["causal"] is True and a["mq"] == 8
    assert torch.all(q.grad == 2) and torch.all(k.grad == 3) and torch.all(v.grad == 4)


def test_varlen_grad_padded_head_dim(fake):
    cu = torch.tensor([0, 6, 10], dtype=torch.int32)
    q, k, v = (rnd(10, 2, 76).requires_grad_() for _ in range(3))
    out = fai.flash_attn_varlen_func(q, k, v, cu, cu, 6, 6)
    assert out.shape == (10, 2, 76) and fake.calls[0][1]["shape"] == (10, 2, 80)
    out.sum().backward()
    assert q.grad.shape == (10, 2, 76) and torch.all(q.grad == 2)


def test_varlen_chunk_backward_rejected(fake):
    cu = torch.tensor([0, 8], dtype=torch.int32)
    q, k, v = (rnd(8, 2, 64).requires_grad_() for _ in range(3))
    out = fai.flash_attn_varlen_func(q, k, v, cu, cu, 8, 8, attention_chunk=4)
    with pytest.raises(NotImplementedError, match="attention_chunk"):
        out.sum().backward()


def test_kvcache_mapping(fake):
    q = rnd(3, 1, 8, 128)
    kc = rnd(10, 16, 2, 128)
    bt = torch.arange(9, dtype=torch.int32).view(3, 3)
    fai.flash_attn_with_kvcache(q, kc, kc, cache_seqlens=torch.tensor([5, 20, 40]), block_table=bt,
                                window_size=(31, 0), num_splits=4)
    a = fake.calls[-1][1]
    assert a["window"] == 32 and a["num_splits"] == 4 and a["seqlens"].dtype == torch.int32
    assert torch.equal(a["bt"], bt) and math.isclose(a["scale"], 128 ** -0.5)
    # dense cache: one block per row, cache_batch_idx picks the row
    kd = rnd(3, 64, 2, 128)
    fai.flash_attn_with_kvcache(q, kd, kd, cache_seqlens=10, cache_batch_idx=torch.tensor([2, 0, 1]))
    a = fake.calls[-1][1]
    assert a["bt"].tolist() == [[2], [0], [1]] and a["seqlens"].tolist() == [10, 10, 10]
    # attention_chunk becomes a left pad at the chunk start
    fai.flash_attn_with_kvcache(q, kd, kd, cache_seqlens=torch.tensor([10, 33, 63]), attention_chunk=16)
    assert fake.calls[-1][1]["lp"].tolist() == [0, 32, 48]


def test_kvcache_rejections(fake):
    q = rnd(1, 1, 4, 128)
    kc = rnd(4, 16, 2, 128)
    bt = torch.zeros((1, 4), dtype=torch.int32)
    with pytest.raises(NotImplementedError):
        fai.flash_attn_with_kvcache(q, kc, kc, cu_seqlens_k_new=torch.zeros(2))
    with pytest.raises(ValueError):
        fai.flash_attn_with_kvcache(q, kc, kc, block_table=bt, page_table=bt)
    with pytest.raises(ValueError):
        fai.flash_attn_with_kvcache(q, kc, kc, block_table=bt, cache_batch_idx=torch.zeros(1))
    with pytest.raises(ValueError):
        fai.flash_attn_with_kvcache(q, kc, kc, k=rnd(1, 1, 2, 128), block_table=bt)
    with pytest.raises(NotImplementedError):
        fai.flash_attn_with_kvcache(q, rnd(1, 48, 2, 128), rnd(1, 48, 2, 128))   # dense, not 2^n
    with pytest.raises(ValueError):
        fai.flash_attn_with_kvcache(rnd(1, 4, 128), kc, kc)


def test_fa3_order_and_pair(fake):
    q = rnd(1, 16, 2, 64)
    r = fa3_interface.flash_attn_func(q, q, q, 0.3, True)
    a = fake.calls[-1][1]
    assert math.isclose(a["scale"], 0.3) and a["causal"] == 1 and torch.is_tensor(r)
    assert fa3_interface.get_scheduler_metadata(1, 2, 3) is None


def test_install_as_flash_attn_names():
    fable_attn.install_as_flash_attn()
    import flash_attn
    import flash_attn_interface
    assert flash_attn.__version__.startswith("2.")
    assert flash_attn_interface.flash_attn_func is fa3_interface.flash_attn_func
    from flash_attn.flash_attn_interface import flash_attn_varlen_func  # noqa: F401


def test_combine_argument_checks():
    with pytest.raises(RuntimeError):
        fai.flash_attn_combine(rnd(2, 1, 4, 2, 64), torch.zeros(2, 1, 2, 4))   # CPU tensors


def test_torch_op_registered_and_falls_back_to_empty():
    """torch.ops.fable_attn.forward exists after import (reference torch_op.py:51-71) and answers
    shapes it cannot serve with an empty tensor, never an exception (:27-48)."""
    from fable_attn import torch_op
    assert torch_op.REGISTERED and torch_op.LAST_ERROR is None
    assert hasattr(torch.ops.fable_attn, "forward")
    assert torch_op.register()   # idempotent
    q = rnd(1, 2, 8, 64)
    assert torch_op._forward(q, q, q, 0.125, True).numel() == 0                  # CPU tensor
    assert torch_op._forward(q.float(), q.float(), q.float(), 0.125, True).numel() == 0
    assert torch_op._forward(q[0], q[0], q[0], 0.125, False).numel() == 0        # 3-D


def test_value_head_dim_runs_at_the_wider_width(fake):
    """headdim_v != headdim without qv: the score needs only q.k, so the narrower side is
    zero-extended to max(d, dv); the default scale keeps the reference's (d + dv)^-0.5."""
    q, k, v = rnd(1, 8, 2, 128), rnd(1, 8, 2, 128), rnd(1, 8, 2, 64)
    out = fai.flash_attn_func(q, k, v)
    a = fake.calls[-1][1]
    assert a["shape"][-1] == 128 and math.isclose(a["scale"], 192 ** -0.5)
    assert out.shape == (1, 8, 2, 64)


def test_paged_varlen_gathers_without_host_lengths(fake):
    """Paged varlen prefill: the block-table rows are gathered whole on the device, sequence z
    starts at z * max_blocks * page and its true length travels as seqused_k."""
    calls = []
    orig = fake.fwd_varlen

    def rec(q, k, v, cu_q, cu_k, mq, mk, *a, **kw):
        calls.append((k.shape, cu_k.clone(), mk, a[10]))   # (scale ... chunk, su_q, su_k)
        return orig(q, k, v, cu_q, cu_k, mq, mk, *a, **kw)
    fake.fwd_varlen = rec
    kc = rnd(6, 16, 2, 64)
    bt = torch.tensor([[4, 1], [0, 5]], dtype=torch.int32)
    cu_q = torch.tensor([0, 3, 7], dtype=torch.int32)
    cu_k = torch.tensor([0, 20, 45], dtype=torch.int32)
    fai.flash_attn_varlen_func(rnd(7, 4, 64), kc, kc, cu_q, cu_k, 4, 25, block_table=bt)
    kshape, cu, mk, used = calls[-1]
    assert kshape == (64, 2, 64) and cu.tolist() == [0, 32, 64] and mk == 32
    assert used.tolist() == [20, 25]


def test_paged_varlen_ignores_table_padding():
    """Block-table entries past a sequence's pages (serving code leaves -1, stale or
    out-of-range values there) are not gathered: the packed K/V rows of each sequence's real
    pages are those of the clean table, and no index error arises."""
    kc = torch.arange(6 * 4 * 1 * 8, dtype=torch.float32).view(6, 4, 1, 8)   # 6 pages of 4 rows
    cu_k = torch.tensor([0, 5, 8], dtype=torch.int32)                          # 2 and 1 pages used
    clean = torch.tensor([[3, 1, 0], [5, 0, 0]], dtype=torch.int32)
    dirty = torch.tensor([[3, 1, -1], [5, 6 + 7, -1]], dtype=torch.int32)
    k1, _, cu1, used1, span1 = fai._pages_as_packed(kc, kc, clean, cu_k, None)
    k2, _, cu2, used2, span2 = fai._pages_as_packed(kc, kc, dirty, cu_k, None)
    assert span1 == span2 == 12 and torch.equal(cu1, cu2) and used2.tolist() == [5, 3]
    for z, n in enumerate((5, 3)):
        assert torch.equal(k2[z * 12:z * 12 + n], k1[z * 12:z * 12 + n])
    assert torch.equal(k2[0:4], kc[3]) and torch.equal(k2[4:5], kc[1, :1])


def test_kvcache_packed_queries_one_call(fake):
    """cu_seqlens_q: the packed queries go to the kernel as one (batch, max_seqlen_q) block
    and come back packed, in one decode call."""
    kc = rnd(8, 16, 2, 64)
    bt = torch.arange(8, dtype=torch.int32).view(2, 4)
    q = rnd(5, 4, 64)
    cu = torch.tensor([0, 2, 5], dtype=torch.int32)
    out, lse = fai.flash_attn_with_kvcache(q, kc, kc, cache_seqlens=torch.tensor([10, 30]),
                                           block_table=bt, cu_seqlens_q=cu, max_seqlen_q=3,
                                           return_softmax_lse=True)
    decs = [c for c in fake.calls if c[0] == "dec"]
    assert len(decs) == 1 and decs[0][1]["q"] == (2, 3, 4, 64)
    assert out.shape == (5, 4, 64) and lse.shape == (4, 5)
    # a max_seqlen_q above the longest sequence pads no further; one below it is refused (its
    # rows would land in the next sequence's slots)
    fai.flash_attn_with_kvcache(q, kc, kc, cache_seqlens=torch.tensor([10, 30]), block_table=bt,
                                cu_seqlens_q=cu, max_seqlen_q=8)
    assert fake.calls[-1][1]["q"] == (2, 3, 4, 64)
    with pytest.raises(ValueError, match="max_seqlen_q"):
        fai.flash_attn_with_kvcache(q, kc, kc, cache_seqlens=torch.tensor([10, 30]),
                                    block_table=bt, cu_seqlens_q=cu, max_seqlen_q=2)
    with pytest.raises(NotImplementedError):
        fai.flash_attn_with_kvcache(q, kc, kc, k=rnd(5, 2, 64), v=rnd(5, 2, 64), block_table=bt,
                                    cu_seqlens_q=cu, max_seqlen_q=3)


def test_kvcache_append_refused_into_a_temporary(fake):
    """Appending must write the caller's cache: with qv (a widened temporary) or a
    non-contiguous cache it is refused instead of silently lost."""
    q, kc = rnd(1, 1, 4, 64), rnd(4, 16, 2, 64)
    bt = torch.zeros((1, 4), dtype=torch.int32)
    nk = rnd(1, 1, 2, 64)
    with pytest.raises(NotImplementedError):
        fai.flash_attn_with_kvcache(q, kc, kc, k=nk, v=nk, qv=rnd(1, 1, 4, 64), block_table=bt)
    with pytest.raises(NotImplementedError):
        t = kc.transpose(1, 2)
        fai.flash_attn_with_kvcache(q, t, t, k=nk, v=nk, block_table=bt)
