"""Native variable-length backward on the GPU (fable_attn_bwd with cu_q/cu_k, through
fable_attn._C.bwd_varlen and flash_attn_varlen_func's autograd).

The reference has no varlen backward kernel: its grad path runs the dense backward once per
sequence from Python (package/fable_attn/flash_attn_interface.py:523-540). Here one launch
of each backward kernel covers every sequence. Checks, on packed ragged batches (lengths 1,
non-multiples of the tile sizes, SQ != SK, GQA):
  * every gradient against the fp64 oracle run per sequence (oracle/oracle.py bwd), at the
    backward bounds (tests/helpers.py check_grads: rel_rms <= 5e-4 fp16 / 4e-3 bf16 vs the exact
    gradients, and close to the oracle's dtype rounding model);
  * bitwise equality with the dense kernels run on each sequence separately (the work split
    per sequence is the same, so the arithmetic must be too);
  * seqused_q/k: rows past the used length get zero gradient, the rest match the shortened
    sequences;
  * bitwise reproducibility over repeated runs;
  * autograd through flash_attn_varlen_func, including a head_dim that is padded.
"""
import math

import numpy as np
import pytest

from oracle import oracle as orc
from tests.helpers import check_grads, gen, to_dev, to_np

pytestmark = pytest.mark.gpu

# name, lens_q, lens_k, Hq, Hk, D, causal, wl, wr, softcap
CASES = [
    ("ragged causal D64", [37, 128, 1, 200], None, 4, 4, 64, True, -1, -1, 0.0),
    ("ragged full gqa D128", [65, 7, 160], None, 4, 2, 128, False, -1, -1, 0.0),
    ("sq!=sk causal D128", [40, 96, 33], [64, 96, 17], 4, 4, 128, True, -1, -1, 0.0),
    ("window softcap D64", [150, 90], None, 4, 2, 64, True, 31, 0, 20.0),
    ("D256 causal", [70, 33], None, 2, 2, 256, True, -1, -1, 0.0),
    # the other kernel widths (multiples of 32; 88 runs in the 96-wide kernel)
    ("D32 ragged causal gqa", [50, 3, 97], None, 4, 2, 32, True, -1, -1, 0.0),
    ("D88 window", [120, 64], None, 2, 2, 88, False, 20, 5, 0.0),
    ("D160 ragged full", [45, 80], [60, 33], 2, 1, 160, False, -1, -1, 0.0),
    ("D192 causal softcap", [66, 31], None, 2, 2, 192, True, -1, -1, 15.0),
    ("D224 causal", [40, 70], None, 2, 2, 224, True, -1, -1, 0.0),
]


def _cu(lens):
    return np.concatenate([[0], np.cumsum(lens)]).astype(np.int32)


def _make(case, dt, seed=0):
    name, lq, lk, Hq, Hk, D, causal, wl, wr, sc = case
    lk = lk or lq
    tq, tk = sum(lq), sum(lk)
    q = gen((tq, Hq, D), seed + 1, dt)
    k = gen((tk, Hk, D), seed + 2, dt)
    v = gen((tk, Hk, D), seed + 3, dt)
    do = gen((tq, Hq, D), seed + 4, dt)
    return lq, lk, q, k, v, do


def _varlen_kernel(case, dt, lq, lk, q, k, v, do, su_q=None, su_k=None, ds_max=None):
    import torch

    from fable_attn import _C
    _, _, _, Hq, Hk, D, causal, wl, wr, sc = case
    cq = torch.from_numpy(_cu(lq)).cuda()
    ck = torch.from_numpy(_cu(lk)).cuda()
    qd, kd, vd, dod = (to_dev(x, dt) for x in (q, k, v, do))
    scale = 1.0 / math.sqrt(D)
    uq = torch.tensor(su_q, dtype=torch.int32, device="cuda") if su_q is not None else None
    uk = torch.tensor(su_k, dtype=torch.int32, device="cuda") if su_k is not None else None
    out, lse = _C.fwd_varlen(qd, kd, vd, cq, ck, max(lq), max(lk), scale, causal, wl, wr, sc,
                             None, 0.0, 0, 0, uq, uk, return_lse=True)
    grads = _C.bwd_varlen(dod, qd, kd, vd, out, lse, cq, ck, max(lq), max(lk), scale, causal,
                          wl, wr, sc, None, 0.0, 0, uq, uk, ds_max_bytes=ds_max)
    torch.cuda.synchronize()
    _varlen_kernel.last_out = out
    return grads


@pytest.mark.parametrize("ds_max", [None, 0], ids=["ds", "recompute"])
@pytest.mark.parametrize("dt", ["f16", "bf16"])
@pytest.mark.parametrize("case", CASES, ids=[c[0] for c in CASES])
def test_varlen_backward_vs_oracle_and_dense(case, dt, ds_max):
    """Both backward paths (dS workspace / recomputing dQ kernel); the dense comparison uses
    the same path."""
    import torch

    from fable_attn import _C
    print(f"[varlen-bwd] {case[0]} {dt} ds_max={ds_max}", flush=True)
    _, _, _, Hq, Hk, D, causal, wl, wr, sc = case
    lq, lk, q, k, v, do = _make(case, dt)
    dq, dk, dv = _varlen_kernel(case, dt, lq, lk, q, k, v, do, ds_max=ds_max)
    out = to_np(_varlen_kernel.last_out)
    again = _varlen_kernel(case, dt, lq, lk, q, k, v, do, ds_max=ds_max)
    for a, b in zip((dq, dk, dv), again):
        assert torch.equal(a, b), "varlen backward differs between runs"
    cq, ck = _cu(lq), _cu(lk)
    scale = 1.0 / math.sqrt(D)
    for i in range(len(lq)):
        a, b, c, d = cq[i], cq[i + 1], ck[i], ck[i + 1]
        # fp64 oracle on this sequence ([1,H,S,D] layout)
        bhsd = lambda x: np.ascontiguousarray(x.transpose(1, 0, 2)[None])
        args = (bhsd(q[a:b]), bhsd(k[c:d]), bhsd(v[c:d]), bhsd(do[a:b]), scale, causal, wl, wr, sc, None)
        ref = orc.bwd(*args)
        model = orc.bwd(*args, model=dt, stored_o=bhsd(out[a:b]))
        got = [to_np(x).transpose(1, 0, 2)[None] for x in (dq[a:b], dk[c:d], dv[c:d])]
        # a single visible key makes dq/dk exactly zero in exact arithmetic (dS = dP - D = 0);
        # the kernel's fp32 dP and D cancel to rounding level there
        check_grads("varlen_bwd_" + ("ds" if ds_max is None else "recompute"),
                    f"{case[0]} seq {i}", dt, got, ref, model, vanish_ok=True)
        # the dense kernels on the same sequence give the same bits
        view = lambda x, dtp=dt: to_dev(x, dtp)[None].transpose(1, 2)
        qs, ks, vs, dos = view(q[a:b]), view(k[c:d]), view(v[c:d]), view(do[a:b])
        o1, l1 = _C.fwd(qs, ks, vs, scale, causal, wl, wr, sc, None, 0.0, 0)
        g1 = _C.bwd(dos, qs, ks, vs, o1, l1, scale, causal, wl, wr, sc, None, 0.0, 0, ds_max_bytes=ds_max)
        torch.cuda.synchronize()
        for name, got, dense, lo, hi in (("dq", dq, g1[0], a, b), ("dk", dk, g1[1], c, d),
                                         ("dv", dv, g1[2], c, d)):
            assert torch.equal(got[lo:hi], dense[0].transpose(0, 1)), f"seq {i} {name} != dense"


def test_varlen_backward_seqused():
    import torch
    case = ("seqused", [80, 120], None, 4, 2, 64, True, -1, -1, 0.0)
    dt = "f16"
    lq, lk, q, k, v, do = _make(case, dt, seed=7)
    su = [50, 120]
    dq, dk, dv = _varlen_kernel(case, dt, lq, lk, q, k, v, do, su_q=su, su_k=su)
    # rows past the used lengths: zero gradient
    assert torch.count_nonzero(dq[50:80]) == 0 and torch.count_nonzero(dk[50:80]) == 0
    assert torch.count_nonzero(dv[50:80]) == 0
    # the used part equals the varlen backward of the shortened batch
    q2 = np.concatenate([q[:50], q[80:]])
    k2 = np.concatenate([k[:50], k[80:]])
    v2 = np.concatenate([v[:50], v[80:]])
    do2 = np.concatenate([do[:50], do[80:]])
    g2 = _varlen_kernel(case, dt, [50, 120], [50, 120], q2, k2, v2, do2)
    assert torch.equal(dq[:50], g2[0][:50]) and torch.equal(dq[80:], g2[0][50:])
    assert torch.equal(dk[:50], g2[1][:50]) and torch.equal(dv[80:], g2[2][50:])


def test_varlen_autograd_matches_dense_autograd():
    """flash_attn_varlen_func backward (native) == flash_attn_func backward per sequence, with a
    head_dim that the API pads (80 -> 128)."""
    import torch

    from fable_attn import flash_attn_func, flash_attn_varlen_func
    lens = [45, 130, 9]
    H, D = 4, 80
    g = torch.Generator(device="cuda").manual_seed(3)
    tot = sum(lens)
    q, k, v = (torch.randn(tot, H, D, device="cuda", dtype=torch.float16, generator=g).requires_grad_()
               for _ in range(3))
    cu = torch.tensor(_cu(lens), device="cuda")
    out = flash_attn_varlen_func(q, k, v, cu, cu, max(lens), max(lens), causal=True)
    dout = torch.randn_like(out)
    out.backward(dout)
    gq, gk, gv = q.grad.clone(), k.grad.clone(), v.grad.clone()
    for i, L in enumerate(lens):
        a, b = int(cu[i]), int(cu[i + 1])
        qs, ks, vs = (x.detach()[a:b][None].clone().requires_grad_() for x in (q, k, v))
        o = flash_attn_func(qs, ks, vs, causal=True)
        assert torch.equal(o[0], out[a:b]), f"seq {i} forward differs"
        o.backward(dout[a:b][None])
        for name, got, ref in (("dq", gq, qs.grad), ("dk", gk, ks.grad), ("dv", gv, vs.grad)):
            assert torch.equal(got[a:b], ref[0]), f"seq {i} {name} differs from the dense path"


# longer packed sequences, few heads: the pair dK/dV grid is one round and splits the query
# tiles of its key blocks (fp32 partials merged per key row through the sequence's offset)
SPLIT_CASES = [
    ("split causal gqa D64", [900, 1400, 600], None, 4, 2, 64, True, -1, -1, 0.0),
    ("split full seqused D128", [700, 1100], [900, 1000], 2, 2, 128, False, -1, -1, 0.0),
]


@pytest.mark.parametrize("dt", ["f16", "bf16"])
@pytest.mark.parametrize("case", SPLIT_CASES, ids=[c[0] for c in SPLIT_CASES])
def test_varlen_backward_query_split(case, dt):
    """Against the fp64 oracle per sequence (the dense per-sequence kernels split differently, so
    they agree with it to rounding, not bitwise); bitwise reproducible over two runs."""
    import torch

    from fable_attn import _C, _lib
    print(f"[varlen-bwd-split] {case[0]} {dt}", flush=True)
    _, _, _, Hq, Hk, D, causal, wl, wr, sc = case
    lq, lk, q, k, v, do = _make(case, dt)
    p = _lib.FableBwdParams()
    p.B, p.Hq, p.Hk, p.gqa, p.SQ, p.SK, p.D = len(lq), Hq, Hk, Hq // Hk, max(lq), max(lk), D
    p.causal, p.win_left, p.win_right = int(causal), wl, wr
    unsplit = _C._L.fable_attn_bwd_ds_bytes(p, 0)
    p.B = 64 * len(lq)                                  # many rounds: no split
    assert _C._L.fable_attn_bwd_ds_bytes(p, 0) // 64 < unsplit, "the case must split"
    su_q = [min(L, 600) for L in lq] if "seqused" in case[0] else None
    su_k = [min(L, 800) for L in lk] if "seqused" in case[0] else None
    dq, dk, dv = _varlen_kernel(case, dt, lq, lk, q, k, v, do, su_q=su_q, su_k=su_k)
    out = to_np(_varlen_kernel.last_out)
    again = _varlen_kernel(case, dt, lq, lk, q, k, v, do, su_q=su_q, su_k=su_k)
    for a, b in zip((dq, dk, dv), again):
        assert torch.equal(a, b), "varlen backward differs between runs"
    cq, ck = _cu(lq), _cu(lk)
    scale = 1.0 / math.sqrt(D)
    for i in range(len(lq)):
        a, c = cq[i], ck[i]
        b = a + (su_q[i] if su_q else lq[i])
        d = c + (su_k[i] if su_k else lk[i])
        bhsd = lambda x: np.ascontiguousarray(x.transpose(1, 0, 2)[None])
        args = (bhsd(q[a:b]), bhsd(k[c:d]), bhsd(v[c:d]), bhsd(do[a:b]), scale, causal, wl, wr, sc, None)
        ref = orc.bwd(*args)
        model = orc.bwd(*args, model=dt, stored_o=bhsd(out[a:b]))
        got = [to_np(x).transpose(1, 0, 2)[None] for x in (dq[a:b], dk[c:d], dv[c:d])]
        check_grads("varlen_bwd_split", f"{case[0]} seq {i}", dt, got, ref, model, vanish_ok=True)
        if su_q:   # rows past the used lengths get zero gradient
            assert not to_np(dq[b:cq[i + 1]]).any() and not to_np(dk[d:ck[i + 1]]).any()


# packed batches of many short sequences (lengths 1 .. 512 at head dim 128, 1 .. 256 at 64, GQA):
# at least two rounds of dK/dV work items with at most 16 query-tile steps each, which the
# persistent dK/dV kernel runs (each workgroup a fixed list of items)
PERSIST_CASES = [
    ("persist D128 causal 160 seqs", 160, 512, 4, 4, 128, True, -1, -1, 0.0),
    ("persist D64 causal gqa2 200 seqs", 200, 256, 4, 2, 64, True, -1, -1, 0.0),
    ("persist D128 window softcap 160 seqs", 160, 512, 4, 4, 128, True, 60, 0, 15.0),
    # the other pair-kernel widths: two (D=96) and three (D=32) workgroups per CU slot
    ("persist D96 causal 200 seqs", 200, 512, 4, 4, 96, True, -1, -1, 0.0),
    ("persist D32 full gqa2 200 seqs", 200, 256, 4, 2, 32, False, -1, -1, 0.0),
]


@pytest.mark.parametrize("dt", ["f16", "bf16"])
@pytest.mark.parametrize("case", PERSIST_CASES, ids=[c[0] for c in PERSIST_CASES])
def test_varlen_backward_persistent(case, dt):
    """Every sequence against the fp64 oracle (and its rounding model), bitwise reproducible over
    two runs; lengths include 1 and the longest allowed."""
    import torch

    print(f"[varlen-bwd-persist] {case[0]} {dt}", flush=True)
    name, nseq, lmax, Hq, Hk, D, causal, wl, wr, sc = case
    rng = np.random.default_rng(7)
    lens = rng.integers(1, lmax + 1, nseq)
    lens[0], lens[1], lens[-1] = 1, lmax, 2
    lens = [int(x) for x in lens]
    full = (name, lens, None, Hq, Hk, D, causal, wl, wr, sc)
    lq, lk, q, k, v, do = _make(full, dt)
    grads = _varlen_kernel(full, dt, lq, lk, q, k, v, do)
    out = to_np(_varlen_kernel.last_out)
    again = _varlen_kernel(full, dt, lq, lk, q, k, v, do)
    for a, b in zip(grads, again):
        assert torch.equal(a, b), "varlen backward differs between runs"
    dq, dk, dv = (to_np(x) for x in grads)
    cu = _cu(lens)
    scale = 1.0 / math.sqrt(D)
    bhsd = lambda x: np.ascontiguousarray(x.transpose(1, 0, 2)[None])
    for i in range(nseq):
        a, b = cu[i], cu[i + 1]
        args = (bhsd(q[a:b]), bhsd(k[a:b]), bhsd(v[a:b]), bhsd(do[a:b]), scale, causal, wl, wr, sc, None)
        ref = orc.bwd(*args)
        model = orc.bwd(*args, model=dt, stored_o=bhsd(out[a:b]))
        got = [x[a:b].transpose(1, 0, 2)[None] for x in (dq, dk, dv)]
        check_grads("varlen_bwd_persist", f"{name} seq {i} len {lens[i]}", dt, got, ref, model, vanish_ok=True)
