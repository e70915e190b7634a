"""Backward parity on the GPU: fable_attn_backward_launch (through fable_attn._C.bwd, the C-ABI)
vs exact fp64 gradients from the oracle, on identical seeded inputs; O and LSE come from this
library's forward as they do in training.

Cases follow the reference backward gate (kernels/backward.hip:710-735: base, causal, GQA,
ragged tails, SQ != SK both ways, windows, head dims, softcap, alibi). Bounds: rel_rms of each
gradient <= 2e-3 (fp16) / 8e-3 (bf16) — the gradients are the product of fp16/bf16-rounded
P and dS matrices and are stored in fp16/bf16, so their floor is above the forward's — and
bitwise-identical results across repeated runs (the atomic-free contract). At the full
BASELINE.json configs[2] size the kernel is checked against a float32 torch autograd
reference on the GPU for sampled heads, and for bitwise reproducibility over 3 runs.

Every case runs both backward paths at head_dim 64/128: "ds" (the dK/dV kernel stores dS in a
workspace and dQ = dS.K is formed from it, the default) and "recompute" (no workspace: the dQ
kernel recomputes S and dP); head_dim 256 has the recomputing path only.
"""
import math

import numpy as np
import pytest

from oracle import oracle as orc
from tests.helpers import gen, to_dev, to_np

pytestmark = pytest.mark.gpu

GTOL = {"f16": 2e-3, "bf16": 8e-3}

# name, B, Hq, Hk, SQ, SK, D, causal, wl, wr, softcap, alibi
CASES = [
    ("base D64", 1, 4, 4, 64, 64, 64, False, -1, -1, 0.0, False),
    ("causal D64", 1, 4, 4, 64, 64, 64, True, -1, -1, 0.0, False),
    ("causal+gqa B2", 2, 8, 2, 128, 128, 64, True, -1, -1, 0.0, False),
    ("causal tail 100", 1, 4, 4, 100, 100, 64, True, -1, -1, 0.0, False),
    ("cross SQ<SK", 1, 4, 4, 96, 128, 64, True, -1, -1, 0.0, False),
    ("cross SQ>SK", 1, 4, 4, 128, 96, 64, True, -1, -1, 0.0, False),
    ("window (47,0)", 1, 4, 4, 128, 128, 64, False, 47, 0, 0.0, False),
    ("window (24,24)", 1, 4, 4, 128, 128, 64, False, 24, 24, 0.0, False),
    ("window (-1,0)=causal", 1, 4, 4, 128, 128, 64, False, -1, 0, 0.0, False),
    ("D128 causal", 1, 4, 4, 200, 200, 128, True, -1, -1, 0.0, False),
    ("D128 full gqa4", 1, 8, 2, 160, 192, 128, False, -1, -1, 0.0, False),
    ("D256 causal", 1, 4, 4, 64, 64, 256, True, -1, -1, 0.0, False),
    ("D256 full", 1, 2, 2, 96, 80, 256, False, -1, -1, 0.0, False),
    ("softcap 30", 1, 4, 4, 128, 128, 64, False, -1, -1, 30.0, False),
    ("alibi causal", 1, 4, 4, 128, 128, 64, True, -1, -1, 0.0, True),
    ("D128 causal B2 S512", 2, 4, 4, 512, 512, 128, True, -1, -1, 0.0, False),
]


PATHS = {"ds": None, "recompute": 0}  # ds_max_bytes of _C.bwd


def run(case, dt, seed=0, repeats=1, path="ds"):
    import torch

    from fable_attn import _C
    name, B, Hq, Hk, SQ, SK, D, causal, wl, wr, sc, alibi = case
    q = gen((B, Hq, SQ, D), seed + 1, dt)
    k = gen((B, Hk, SK, D), seed + 2, dt)
    v = gen((B, Hk, SK, D), seed + 3, dt)
    do = gen((B, Hq, SQ, D), seed + 4, dt)
    al = (-0.1 * np.arange(1, Hq + 1)).astype(np.float32) if alibi else None
    scale = 1.0 / math.sqrt(D)
    # public (B,S,H,D) storage, [B,H,S,D] views
    view = lambda a: to_dev(a, dt).transpose(1, 2).contiguous().transpose(1, 2)
    qd, kd, vd, dod = view(q), view(k), view(v), view(do)
    ald = torch.from_numpy(al).cuda() if al is not None else None
    out, lse = _C.fwd(qd, kd, vd, scale, causal, wl, wr, sc, ald, 0.0, 0)
    res = [_C.bwd(dod, qd, kd, vd, out, lse, scale, causal, wl, wr, sc, ald, 0.0, 0,
                  ds_max_bytes=PATHS[path]) for _ in range(repeats)]
    torch.cuda.synchronize()
    ref = orc.bwd(q, k, v, do, scale, causal, wl, wr, sc, al)
    return res, ref


@pytest.mark.parametrize("path", list(PATHS))
@pytest.mark.parametrize("dt", ["f16", "bf16"])
@pytest.mark.parametrize("case", CASES, ids=[c[0] for c in CASES])
def test_backward_parity(case, dt, path):
    print(f"[bwd] {case[0]} {dt} {path}", flush=True)
    res, ref = run(case, dt, repeats=3, path=path)
    for i, name in enumerate(("dq", "dk", "dv")):
        got = to_np(res[0][i])
        assert np.isfinite(got).all(), f"{name} not finite"
        e = orc.rel_rms(got, ref[i])
        assert e <= GTOL[dt], f"{name} rel_rms {e:.3e} > {GTOL[dt]}"
        for r in res[1:]:
            assert torch_equal(r[i], res[0][i]), f"{name} differs between runs"


def torch_equal(a, b):
    import torch
    return bool(torch.equal(a, b))


@pytest.mark.parametrize("path", list(PATHS))
def test_backward_full_config_c3(path):
    """causal bf16, B=2, S=4096, H=32, D=128; bitwise identical over
    3 runs; sampled heads against a float32 torch autograd reference on the GPU."""
    import torch

    from fable_attn import _C
    from fable_attn.flash_attn_interface import _kernel_view
    B, S, H, D = 2, 4096, 32, 128
    g = torch.Generator(device="cuda").manual_seed(0)
    q, k, v, do = (torch.randn(B, S, H, D, device="cuda", dtype=torch.bfloat16, generator=g)
                   for _ in range(4))
    qh, kh, vh, doh = (_kernel_view(x) for x in (q, k, v, do))
    scale = D ** -0.5
    out, lse = _C.fwd(qh, kh, vh, scale, True, -1, 0, 0.0, None, 0.0, 0)
    print(f"[bwd] C3 full size {path}", flush=True)
    runs = [_C.bwd(doh, qh, kh, vh, out, lse, scale, True, -1, 0, 0.0, None, 0.0, 0,
                   ds_max_bytes=PATHS[path]) for _ in range(3)]
    torch.cuda.synchronize()
    for r in runs[1:]:
        for a, b in zip(runs[0], r):
            assert torch.equal(a, b)
    for bb, hd in ((0, 0), (1, 31)):
        qf, kf, vf = (x[bb, :, hd].float().detach().clone().requires_grad_() for x in (q, k, v))
        s = (qf @ kf.t()) * scale
        s = s.masked_fill(torch.ones(S, S, device="cuda", dtype=torch.bool).triu(1), float("-inf"))
        o = torch.softmax(s, -1) @ vf
        o.backward(do[bb, :, hd].float())
        for got, ref in ((runs[0][0][bb, hd], qf.grad), (runs[0][1][bb, hd], kf.grad), (runs[0][2][bb, hd], vf.grad)):
            e = ((got.float() - ref).norm() / ref.norm()).item()
            assert e <= GTOL["bf16"], e


def test_backward_ds_workspace_too_small_falls_back():
    """A dS workspace smaller than fable_attn_bwd_ds_bytes reports, or not 16-byte aligned,
    must be ignored (the recomputing path runs, the buffer stays untouched); a full-size one
    filled with NaN bit
    patterns must give the same gradients (tiles that are never written are never read).
    Both against the oracle, through the C-ABI with a hand-built BwdParams."""
    import torch

    from fable_attn import _C, _lib
    lib = _lib.load()
    case = ("D128 causal tail", 1, 4, 2, 150, 150, 128, True, -1, -1, 0.0, False)
    name, B, Hq, Hk, SQ, SK, D, causal, wl, wr, sc, alibi = case
    dt = "bf16"
    q = gen((B, Hq, SQ, D), 11, dt)
    k = gen((B, Hk, SK, D), 12, dt)
    v = gen((B, Hk, SK, D), 13, dt)
    do = gen((B, Hq, SQ, D), 14, dt)
    scale = D ** -0.5
    view = lambda a: to_dev(a, dt).transpose(1, 2).contiguous().transpose(1, 2)
    qd, kd, vd, dod = view(q), view(k), view(v), view(do)
    out, lse = _C.fwd(qd, kd, vd, scale, causal, wl, wr, sc, None, 0.0, 0)
    dq, dk, dv = (torch.empty_like(x) for x in (qd, kd, vd))
    dsum = torch.empty((B, Hq, SQ), dtype=torch.float32, device="cuda")
    p = _lib.BwdParams()
    p.Q, p.K, p.V, p.O, p.dO = qd.data_ptr(), kd.data_ptr(), vd.data_ptr(), out.data_ptr(), dod.data_ptr()
    p.dQ, p.dK, p.dV = dq.data_ptr(), dk.data_ptr(), dv.data_ptr()
    p.lse, p.dsum = lse.data_ptr(), dsum.data_ptr()
    bhs = lambda t: _lib.Strides(*t.stride()[:3])
    p.qs, p.ks, p.vs, p.os, p.dos = bhs(qd), bhs(kd), bhs(vd), bhs(out), bhs(dod)
    p.dqs, p.dks, p.dvs = bhs(dq), bhs(dk), bhs(dv)
    p.B, p.Hq, p.Hk, p.SQ, p.SK, p.D, p.gqa = B, Hq, Hk, SQ, SK, D, Hq // Hk
    p.scale, p.causal, p.win_left, p.win_right, p.keep_scale = scale, 1, -1, -1, 1.0
    need = lib.fable_attn_bwd_ds_bytes(p, 1)
    assert need == B * Hq * 5 * 5 * 2048
    ws = torch.full((need + 16,), 0xFF, dtype=torch.uint8, device="cuda")  # NaN bit patterns
    stream = ctypes_stream()
    # too small, then big enough but not 16-byte aligned: both ignored
    for ptr, nbytes in ((ws.data_ptr(), need - 1), (ws.data_ptr() + 8, need)):
        p.ds_ws, p.ds_ws_bytes = ptr, nbytes
        assert lib.fable_attn_backward_launch(p, 1, stream) == 0
        torch.cuda.synchronize()
        assert torch.all(ws == 0xFF), "an unusable workspace must not be written"
    p.ds_ws = ws.data_ptr()
    ref = orc.bwd(q, k, v, do, scale, causal)
    for got, r, gname in ((dq, ref[0], "dq"), (dk, ref[1], "dk"), (dv, ref[2], "dv")):
        e = orc.rel_rms(to_np(got), r)
        assert e <= GTOL[dt], f"{gname} rel_rms {e:.3e}"
    # a full-size workspace poisoned with NaN patterns: the dQ kernel reads only the tiles the
    # dK/dV kernel wrote (the causal upper-right tiles stay NaN and must not leak into dQ)
    p.ds_ws_bytes = need
    assert lib.fable_attn_backward_launch(p, 1, stream) == 0
    torch.cuda.synchronize()
    assert not torch.all(ws == 0xFF), "the workspace path was not taken"
    for got, r, gname in ((dq, ref[0], "dq"), (dk, ref[1], "dk"), (dv, ref[2], "dv")):
        assert torch.isfinite(got).all(), f"{gname} not finite"
        e = orc.rel_rms(to_np(got), r)
        assert e <= GTOL[dt], f"{gname} rel_rms {e:.3e} (poisoned workspace)"


def ctypes_stream():
    import ctypes

    import torch
    return ctypes.c_void_p(torch.cuda.current_stream().cuda_stream)
