"""fp32 forward and backward on the GPU (fable_attn_fwd / fable_attn_bwd with
dtype FA_F32, through fable_attn._C), against the fp64 oracle on the same inputs.

The reference serves fp32 through separate kernels (kernels/fa_forward.hip:317-400, 440-447;
backward.hip MODE BW_F32) and gates them at rel_rms 1e-5 (forward, fa_forward_gate.inc:169) and
1e-4 (backward, backward.hip:734); these tests use the same bounds, LSE within 1e-5 absolute.
Cases: the kernel widths 64, 128, 256 and head dims below them (16, 40, 80, 112, 160, 224:
the reference's fp32 head dims run in the next kernel width with zero columns inside the kernel),
causal bottom-right with SQ != SK both ways (empty rows), GQA, windows, softcap, alibi,
attention_chunk, dropout (mask bit-compatible with the fp16 path), varlen with seqused, ragged
tails; backward bitwise reproducible; autograd through flash_attn_func at head dim 80; the
reference-layout launcher fa_forward_launch at head dim 80.
"""
import math

import numpy as np
import pytest

from oracle import oracle as orc
from tests.helpers import gen, lse_err, to_dev, to_np

pytestmark = pytest.mark.gpu

FTOL, GTOL, LTOL = 1e-5, 1e-4, 1e-5
SEED = 0x1234ABCD

# name, B, Hq, Hk, SQ, SK, D, causal, wl, wr, softcap, alibi, chunk, dropout
CASES = [
    ("D64 full", 2, 4, 4, 96, 96, 64, False, -1, -1, 0.0, False, 0, 0.0),
    ("D64 causal gqa tail", 1, 8, 2, 150, 150, 64, True, -1, -1, 0.0, False, 0, 0.0),
    ("D128 causal SQ<SK", 1, 4, 4, 100, 230, 128, True, -1, -1, 0.0, False, 0, 0.0),
    ("D128 causal SQ>SK", 1, 4, 2, 200, 70, 128, True, -1, -1, 0.0, False, 0, 0.0),
    ("D128 window softcap", 1, 4, 4, 180, 180, 128, False, 40, 7, 25.0, False, 0, 0.0),
    ("D64 alibi causal", 1, 4, 4, 128, 128, 64, True, -1, -1, 0.0, True, 0, 0.0),
    ("D256 causal", 1, 2, 2, 140, 140, 256, True, -1, -1, 0.0, False, 0, 0.0),
    ("D256 full gqa", 1, 4, 2, 64, 90, 256, False, -1, -1, 0.0, False, 0, 0.0),
    ("D128 dropout", 1, 4, 4, 128, 128, 128, True, -1, -1, 0.0, False, 0, 0.2),
    # head dims below the kernel width (reference fp32 head dims, kernels/fa_forward.hip:443-447,
    # backward.hip:491-497, 508-516)
    ("D16 causal gqa", 1, 4, 2, 130, 130, 16, True, -1, -1, 0.0, False, 0, 0.0),
    ("D40 full tail", 2, 2, 2, 77, 93, 40, False, -1, -1, 0.0, False, 0, 0.0),
    ("D80 causal softcap", 1, 4, 4, 150, 150, 80, True, -1, -1, 20.0, False, 0, 0.0),
    ("D112 window alibi", 1, 4, 2, 140, 170, 112, False, 30, 10, 0.0, True, 0, 0.0),
    ("D160 causal SQ<SK", 1, 2, 2, 90, 160, 160, True, -1, -1, 0.0, False, 0, 0.0),
    ("D224 causal gqa", 1, 4, 2, 100, 100, 224, True, -1, -1, 0.0, False, 0, 0.0),
    # the 256-wide feature and dropout kernels
    ("D256 alibi window", 1, 4, 2, 120, 150, 256, False, 50, 20, 0.0, True, 0, 0.0),
    ("D192 dropout softcap", 1, 2, 2, 96, 96, 192, True, -1, -1, 15.0, False, 0, 0.15),
]
FWD_ONLY = [("D64 chunk 48", 1, 4, 4, 160, 160, 64, True, -1, -1, 0.0, False, 48, 0.0)]


def _view(a):
    return to_dev(a, "f32").transpose(1, 2).contiguous().transpose(1, 2)


def _inputs(case, seed=0):
    name, B, Hq, Hk, SQ, SK, D = case[:7]
    q = gen((B, Hq, SQ, D), seed + 1, "f32")
    k = gen((B, Hk, SK, D), seed + 2, "f32")
    v = gen((B, Hk, SK, D), seed + 3, "f32")
    do = gen((B, Hq, SQ, D), seed + 4, "f32")
    al = (-0.1 * np.arange(1, Hq + 1)).astype(np.float32) if case[11] else None
    return q, k, v, do, al


@pytest.mark.parametrize("case", CASES + FWD_ONLY, ids=[c[0] for c in CASES + FWD_ONLY])
def test_f32_forward_vs_oracle(case):
    import torch

    from fable_attn import _C
    print(f"[f32-fwd] {case[0]}", flush=True)
    name, B, Hq, Hk, SQ, SK, D, causal, wl, wr, sc, alibi, chunk, pd = case
    q, k, v, _, al = _inputs(case)
    scale = 1.0 / math.sqrt(D)
    ald = torch.from_numpy(al).cuda() if al is not None else None
    out, lse = _C.fwd(_view(q), _view(k), _view(v), scale, causal, wl, wr, sc, ald, pd, SEED, chunk)
    torch.cuda.synchronize()
    ro, rl = orc.fwd(q, k, v, scale, causal, wl, wr, sc, al, chunk, dropout_p=pd, seed=SEED)
    got = to_np(out)
    assert np.isfinite(got).all()
    e = orc.rel_rms(got, ro)
    assert e <= FTOL, f"O rel_rms {e:.3e} > {FTOL}"
    le, inf_ok = lse_err(to_np(lse), rl)
    assert inf_ok and le <= LTOL, f"LSE err {le:.3e}"
    if SQ > SK and causal:   # rows without a visible key: exactly 0 and -inf
        n = SQ - SK
        assert (got[:, :, :n] == 0).all() and np.isneginf(to_np(lse)[:, :, :n]).all()


@pytest.mark.parametrize("case", CASES, ids=[c[0] for c in CASES])
def test_f32_backward_vs_oracle(case):
    import torch

    from fable_attn import _C
    print(f"[f32-bwd] {case[0]}", flush=True)
    name, B, Hq, Hk, SQ, SK, D, causal, wl, wr, sc, alibi, chunk, pd = case
    q, k, v, do, al = _inputs(case, seed=20)
    scale = 1.0 / math.sqrt(D)
    ald = torch.from_numpy(al).cuda() if al is not None else None
    qd, kd, vd, dod = _view(q), _view(k), _view(v), _view(do)
    out, lse = _C.fwd(qd, kd, vd, scale, causal, wl, wr, sc, ald, pd, SEED)
    g1 = _C.bwd(dod, qd, kd, vd, out, lse, scale, causal, wl, wr, sc, ald, pd, SEED)
    g2 = _C.bwd(dod, qd, kd, vd, out, lse, scale, causal, wl, wr, sc, ald, pd, SEED)
    torch.cuda.synchronize()
    ref = orc.bwd(q, k, v, do, scale, causal, wl, wr, sc, al, dropout_p=pd, seed=SEED)
    for i, gname in enumerate(("dq", "dk", "dv")):
        got = to_np(g1[i])
        assert np.isfinite(got).all(), f"{gname} not finite"
        e = orc.rel_rms(got, ref[i])
        assert e <= GTOL, f"{gname} rel_rms {e:.3e} > {GTOL}"
        assert torch.equal(g1[i], g2[i]), f"{gname} differs between runs"


def test_f32_varlen_forward_backward():
    """Packed sequences with seqused: each sequence equals the oracle on its own (used) rows;
    rows past seqused get zero output and zero gradient."""
    import torch

    from fable_attn import _C
    H, Hk, D = 4, 2, 64
    lq, lk = [37, 100, 5], [60, 100, 17]
    su_q, su_k = [37, 80, 5], [60, 90, 17]
    cq = np.concatenate([[0], np.cumsum(lq)]).astype(np.int32)
    ck = np.concatenate([[0], np.cumsum(lk)]).astype(np.int32)
    q = gen((sum(lq), H, D), 31, "f32")
    k = gen((sum(lk), Hk, D), 32, "f32")
    v = gen((sum(lk), Hk, D), 33, "f32")
    do = gen((sum(lq), H, D), 34, "f32")
    dev = lambda a: to_dev(a, "f32")
    cqd, ckd = torch.from_numpy(cq).cuda(), torch.from_numpy(ck).cuda()
    uq = torch.tensor(su_q, dtype=torch.int32, device="cuda")
    uk = torch.tensor(su_k, dtype=torch.int32, device="cuda")
    scale = D ** -0.5
    qd, kd, vd, dod = dev(q), dev(k), dev(v), dev(do)
    out, lse = _C.fwd_varlen(qd, kd, vd, cqd, ckd, max(lq), max(lk), scale, True, -1, -1, 0.0, None,
                             0.0, 0, 0, uq, uk, return_lse=True)
    dq, dk, dv = _C.bwd_varlen(dod, qd, kd, vd, out, lse, cqd, ckd, max(lq), max(lk), scale, True,
                               -1, -1, 0.0, None, 0.0, 0, uq, uk)
    torch.cuda.synchronize()
    bhsd = lambda x: np.ascontiguousarray(x.transpose(1, 0, 2)[None])
    for i in range(len(lq)):
        a, c = cq[i], ck[i]
        nq, nk = su_q[i], su_k[i]
        ro, _ = orc.fwd(bhsd(q[a:a + nq]), bhsd(k[c:c + nk]), bhsd(v[c:c + nk]), scale, True)
        assert orc.rel_rms(to_np(out[a:a + nq]).transpose(1, 0, 2)[None], ro) <= FTOL, f"seq {i} O"
        ref = orc.bwd(bhsd(q[a:a + nq]), bhsd(k[c:c + nk]), bhsd(v[c:c + nk]), bhsd(do[a:a + nq]), scale, True)
        for got, r, gname in ((dq[a:a + nq], ref[0], "dq"), (dk[c:c + nk], ref[1], "dk"), (dv[c:c + nk], ref[2], "dv")):
            e = orc.rel_rms(to_np(got).transpose(1, 0, 2)[None], r)
            assert e <= GTOL, f"seq {i} {gname} rel_rms {e:.3e}"
        assert torch.count_nonzero(dq[a + nq:cq[i + 1]]) == 0
        assert torch.count_nonzero(dk[c + nk:ck[i + 1]]) == 0 and torch.count_nonzero(dv[c + nk:ck[i + 1]]) == 0


def test_f32_autograd_head_dim_80():
    """flash_attn_func in fp32 with head_dim 80 (run by the 128-wide kernels with zero columns
    past 80; the API passes it as it is): output and gradients against the oracle."""
    import torch

    from fable_attn import flash_attn_func
    B, S, H, D = 2, 77, 4, 80
    g = torch.Generator(device="cuda").manual_seed(5)
    q, k, v = (torch.randn(B, S, H, D, device="cuda", dtype=torch.float32, generator=g).requires_grad_()
               for _ in range(3))
    dout = torch.randn(B, S, H, D, device="cuda", dtype=torch.float32, generator=g)
    out = flash_attn_func(q, k, v, causal=True)
    out.backward(dout)
    torch.cuda.synchronize()
    bhsd = lambda t: to_np(t).transpose(0, 2, 1, 3)
    ro, _ = orc.fwd(bhsd(q), bhsd(k), bhsd(v), D ** -0.5, True)
    assert orc.rel_rms(bhsd(out), ro) <= FTOL
    ref = orc.bwd(bhsd(q), bhsd(k), bhsd(v), bhsd(dout), D ** -0.5, True)
    for got, r, gname in ((q.grad, ref[0], "dq"), (k.grad, ref[1], "dk"), (v.grad, ref[2], "dv")):
        e = orc.rel_rms(bhsd(got), r)
        assert e <= GTOL, f"{gname} rel_rms {e:.3e}"


def test_f32_reference_launcher_head_dim_80():
    """fa_forward_launch (the reference's own launcher and struct layout, package/csrc/fa_iface.h)
    in fp32 at head dim 80, which the reference instantiates (kernels/fa_forward.hip:443-447):
    one call per batch element as the reference's glue makes them (dispatch.cpp:61-78), LSE of
    batch element 0 only (the reference layout has no batch stride)."""
    import ctypes

    import torch

    from fable_attn import _lib
    lib = _lib.load()
    B, H, Hk, SQ, SK, D = 2, 4, 2, 120, 150, 80
    q = gen((B, H, SQ, D), 61, "f32")
    k = gen((B, Hk, SK, D), 62, "f32")
    v = gen((B, Hk, SK, D), 63, "f32")
    qd, kd, vd = _view(q), _view(k), _view(v)
    out = torch.empty((B, SQ, H, D), dtype=torch.float32, device="cuda").transpose(1, 2)
    lse = torch.empty((H, SQ), dtype=torch.float32, device="cuda")
    rs = lambda t: _lib.RefStrides(*t.stride()[:3])
    st = ctypes.c_void_p(torch.cuda.current_stream().cuda_stream)
    for b in range(B):
        p = _lib.RefFwdParams()
        p.Q = qd.data_ptr() + b * qd.stride(0) * 4
        p.K = kd.data_ptr() + b * kd.stride(0) * 4
        p.V = vd.data_ptr() + b * vd.stride(0) * 4
        p.O = out.data_ptr() + b * out.stride(0) * 4
        p.LSE = lse.data_ptr() if b == 0 else None
        p.sQ, p.sK, p.sV, p.sO = rs(qd), rs(kd), rs(vd), rs(out)
        p.SQ, p.SK, p.HD, p.NH, p.gqa = SQ, SK, D, H, H // Hk
        p.scale, p.softcap, p.win_left, p.win_right, p.causal = D ** -0.5, 0.0, -1, 0, 1
        p.batch = 1
        assert lib.fa_forward_launch(p, 2, st) == 0, lib.fable_attn_last_error()
    torch.cuda.synchronize()
    ro, rl = orc.fwd(q, k, v, D ** -0.5, True)
    assert orc.rel_rms(to_np(out), ro) <= FTOL
    le, inf_ok = lse_err(to_np(lse)[None], rl[:1])
    assert inf_ok and le <= LTOL
