"""The packed and paged entry points of the flash_attn API on the GPU: each must give exactly
what the plain entry point gives on the same data (they are views / gathers in front of the same
kernels), and the plain entry point is checked against the fp64 oracle here too.
Reference: flash_attn_interface.py:391-469 (packed variants, paged varlen)."""
import itertools

import numpy as np
import pytest

from oracle import oracle as orc
from tests.helpers import TOL, gen, to_dev, to_np

pytestmark = pytest.mark.gpu


@pytest.mark.parametrize("causal", [False, True])
def test_packed_variants_equal_plain(causal):
    import torch

    from fable_attn import (flash_attn_func, flash_attn_kvpacked_func, flash_attn_qkvpacked_func,
                            flash_attn_varlen_func, flash_attn_varlen_kvpacked_func,
                            flash_attn_varlen_qkvpacked_func)
    B, S, H, D, dt = 2, 130, 4, 64, "f16"
    print(f"[packed] causal={causal}", flush=True)
    qkv = to_dev(gen((B, S, 3, H, D), 41, dt), dt)
    q, k, v = qkv.unbind(2)
    plain = flash_attn_func(q, k, v, causal=causal)
    assert torch.equal(flash_attn_qkvpacked_func(qkv, causal=causal), plain)
    assert torch.equal(flash_attn_kvpacked_func(q, qkv[:, :, 1:], causal=causal), plain)
    ref, _ = orc.fwd(*(np.ascontiguousarray(to_np(x).transpose(0, 2, 1, 3)) for x in (q, k, v)),
                     D ** -0.5, causal=causal, win_right=0 if causal else -1)
    assert orc.rel_rms(to_np(plain).transpose(0, 2, 1, 3), ref) <= TOL[dt]
    # varlen: the batch packed as two sequences of length S
    cu = torch.tensor([0, S, 2 * S], dtype=torch.int32, device="cuda")
    qkv_p = qkv.reshape(B * S, 3, H, D)
    vl = flash_attn_varlen_func(qkv_p[:, 0], qkv_p[:, 1], qkv_p[:, 2], cu, cu, S, S, causal=causal)
    assert torch.equal(flash_attn_varlen_qkvpacked_func(qkv_p, cu, S, causal=causal), vl)
    assert torch.equal(flash_attn_varlen_kvpacked_func(qkv_p[:, 0], qkv_p[:, 1:], cu, cu, S, S,
                                                       causal=causal), vl)
    assert orc.rel_rms(to_np(vl).reshape(B, S, H, D), to_np(plain)) <= TOL[dt]


def test_paged_varlen_equals_packed():
    """varlen prefill with K/V in pages (num_blocks, page, Hk, D) and a block table (a seeded
    permutation of the pages) against the same sequences packed contiguously."""
    import torch

    from fable_attn import flash_attn_varlen_func
    lens_q, lens_k, Hq, Hk, D, page, dt = [37, 64, 100], [90, 64, 230], 8, 2, 128, 16, "bf16"
    print("[paged-varlen]", flush=True)
    cq = [0] + list(itertools.accumulate(lens_q))
    ck = [0] + list(itertools.accumulate(lens_k))
    q = to_dev(gen((cq[-1], Hq, D), 51, dt), dt)
    k = to_dev(gen((ck[-1], Hk, D), 52, dt), dt)
    v = to_dev(gen((ck[-1], Hk, D), 53, dt), dt)
    cu_q = torch.tensor(cq, dtype=torch.int32, device="cuda")
    cu_k = torch.tensor(ck, dtype=torch.int32, device="cuda")
    packed = flash_attn_varlen_func(q, k, v, cu_q, cu_k, max(lens_q), max(lens_k), causal=True)
    # pages: sequence i's keys fill its pages in order; the pages sit at permuted slots
    npg = [(L + page - 1) // page for L in lens_k]
    total = sum(npg)
    perm = torch.randperm(total, generator=torch.Generator().manual_seed(5))
    kp = torch.zeros(total, page, Hk, D, dtype=k.dtype, device="cuda")
    vp = torch.zeros_like(kp)
    bt = torch.zeros(len(lens_k), max(npg), dtype=torch.int32)
    slot = 0
    for i, L in enumerate(lens_k):
        for j in range(npg[i]):
            phys = int(perm[slot])
            slot += 1
            bt[i, j] = phys
            r0, r1 = ck[i] + j * page, min(ck[i] + (j + 1) * page, ck[i + 1])
            kp[phys, :r1 - r0] = k[r0:r1]
            vp[phys, :r1 - r0] = v[r0:r1]
    paged = flash_attn_varlen_func(q, kp, vp, cu_q, cu_k, max(lens_q), max(lens_k), causal=True,
                                   block_table=bt.cuda())
    assert torch.equal(paged, packed)
    # table entries past a sequence's pages as serving code leaves them: -1 and out of range
    pad = torch.tensor([-1, total + 7], dtype=torch.int32)
    for i in range(len(lens_k)):
        bt[i, npg[i]:] = pad[i % 2]
    paged = flash_attn_varlen_func(q, kp, vp, cu_q, cu_k, max(lens_q), max(lens_k), causal=True,
                                   block_table=bt.cuda())
    assert torch.equal(paged, packed)
    # and the packed result against the oracle, per sequence
    for i in range(len(lens_q)):
        qi = to_np(q[cq[i]:cq[i + 1]]).transpose(1, 0, 2)[None]
        ki = to_np(k[ck[i]:ck[i + 1]]).transpose(1, 0, 2)[None]
        vi = to_np(v[ck[i]:ck[i + 1]]).transpose(1, 0, 2)[None]
        ref, _ = orc.fwd(np.ascontiguousarray(qi), np.ascontiguousarray(ki), np.ascontiguousarray(vi),
                         D ** -0.5, causal=True, win_right=0)
        got = to_np(packed[cq[i]:cq[i + 1]]).transpose(1, 0, 2)[None]
        assert orc.rel_rms(got, ref) <= TOL[dt], f"sequence {i}"


def test_host_checks_reject_before_launch():
    """Argument checks of the _C glue raise on the host, before any kernel is enqueued: a
    mismatched lse_partial in combine, cu_seqlens on the CPU or with too few entries, seqused
    of the wrong length, and decode side inputs of the wrong dtype or length."""
    import pytest
    import torch

    from fable_attn import _C
    dev = "cuda"
    op = torch.zeros(2, 1, 8, 4, 64, device=dev, dtype=torch.float16)
    with pytest.raises(RuntimeError, match="lse_partial"):
        _C.combine(op, torch.zeros(2, 1, 8, 4, device=dev), torch.float16)    # (S, H) swapped
    with pytest.raises(RuntimeError, match="lse_partial"):
        _C.combine(op, torch.zeros(1, 1, 4, 8, device=dev), torch.float16)    # fewer splits
    q = torch.zeros(10, 4, 64, device=dev, dtype=torch.float16)
    cu = torch.tensor([0, 4, 10], dtype=torch.int32)
    args = (q, q, q)
    with pytest.raises(RuntimeError, match="cu_seqlens_q"):
        _C.fwd_varlen(*args, cu, cu.to(dev), 6, 6, 0.1, True, -1, 0, 0.0, None, 0.0, 0)
    with pytest.raises(RuntimeError, match="cu_seqlens_k"):
        _C.fwd_varlen(*args, cu.to(dev), cu[:2].to(dev), 6, 6, 0.1, True, -1, 0, 0.0, None, 0.0, 0)
    with pytest.raises(RuntimeError, match="seqused_q"):
        _C.fwd_varlen(*args, cu.to(dev), cu.to(dev), 6, 6, 0.1, True, -1, 0, 0.0, None, 0.0, 0,
                      seqused_q=torch.tensor([1, 2, 3], dtype=torch.int32, device=dev))
    qd = torch.zeros(2, 1, 8, 64, device=dev, dtype=torch.float16)
    kc = torch.zeros(4, 16, 2, 64, device=dev, dtype=torch.float16)
    bt = torch.zeros(2, 2, dtype=torch.int32, device=dev)
    cs = torch.full((2,), 5, dtype=torch.int32, device=dev)
    with pytest.raises(RuntimeError, match="alibi"):
        _C.dec(qd, kc, kc, bt, cs, None, None, None, None, False, 0.1, -1,
               alibi=torch.zeros(8, dtype=torch.float16, device=dev))
    with pytest.raises(RuntimeError, match="cache_leftpad"):
        _C.dec(qd, kc, kc, bt, cs, None, None, None, None, False, 0.1, -1,
               cache_leftpad=torch.zeros(2, dtype=torch.int64, device=dev))
    with pytest.raises(RuntimeError, match="cache_seqlens"):
        _C.dec(qd, kc, kc, bt, cs[:1], None, None, None, None, False, 0.1, -1)
    with pytest.raises(RuntimeError, match="block_table"):
        _C.dec(qd, kc, kc, bt[:1], cs, None, None, None, None, False, 0.1, -1)


def test_inference_fast_path_matches_general_path():
    """flash_attn_func's inference calls go through a per-thread cache of validated launch
    parameters; the output must be bit for bit the general path's (the same kernel, launched
    with the same parameters), for dense and strided inputs, GQA, masks, softcap and every
    dtype; calls with gradients, unaligned rows or a padded head dim take the general path."""
    import torch

    from fable_attn import flash_attn_interface as fai
    print("[fast-path]", flush=True)
    g = torch.Generator(device="cuda").manual_seed(11)
    cases = [((2, 300, 8, 64), 8, torch.float16, dict(causal=True)),
             ((1, 257, 8, 128), 2, torch.bfloat16, dict(window_size=(40, 7), softcap=20.0)),
             ((1, 100, 4, 80), 4, torch.float32, dict(causal=True, softmax_scale=0.3)),
             ((2, 64, 4, 96), 1, torch.float16, dict())]
    for shape, hk, dt, kw in cases:
        B, S, H, D = shape
        q = torch.randn(shape, device="cuda", dtype=dt, generator=g)
        kv = torch.randn(B, S, 2, hk, D, device="cuda", dtype=dt, generator=g)
        k, v = kv.unbind(2)                      # strided views, as flash_attn_kvpacked_func makes
        fai._tls.plans = {}
        fast = fai.flash_attn_func(q, k, v, **kw)
        assert len(fai._tls.plans) == 1 and next(iter(fai._tls.plans.values())) is not None
        gen = fai._dense(q, k, v, 0.0, kw.get("softmax_scale"), kw.get("causal", False),
                         kw.get("window_size", (-1, -1)), kw.get("softcap", 0.0), None, False,
                         False, None, 0, None, None, None, 1, None, 0)
        torch.cuda.synchronize()
        assert fast.shape == shape and fast.is_contiguous()
        assert torch.equal(fast, gen), (shape, dt, kw)
        again = fai.flash_attn_func(q, k, v, **kw)      # the cached plan, new output buffer
        assert torch.equal(again, gen) and again.data_ptr() != fast.data_ptr()
    # the general path: gradients, an unaligned base pointer, a padded head dim
    q = torch.randn(1, 64, 2, 64, device="cuda", dtype=torch.float16, generator=g)
    fai._tls.plans = {}
    qg = q.clone().requires_grad_()
    fai.flash_attn_func(qg, q, q).sum().backward()
    assert qg.grad is not None and not fai._tls.plans
    buf = torch.randn(1 + 64 * 2 * 64, device="cuda", dtype=torch.float16, generator=g)
    qu = buf[1:].view(1, 64, 2, 64)                     # rows 2 bytes off 16-byte alignment
    ref = fai.flash_attn_func(qu.clone(), q, q)
    assert torch.equal(fai.flash_attn_func(qu, q, q), ref)      # copied to an aligned buffer
    q40 = torch.randn(1, 64, 2, 36, device="cuda", dtype=torch.float16, generator=g)
    fai._tls.plans = {}
    o40 = fai.flash_attn_func(q40, q40, q40)
    assert o40.shape == (1, 64, 2, 36) and list(fai._tls.plans.values()) == [None]
