"""Backward parity on the GPU: fable_attn_bwd (through fable_attn._C.bwd, the C-ABI) vs exact
fp64 gradients from the oracle, on identical seeded inputs; O and LSE come from this library's
forward as they do in training.

Cases follow the reference backward gate (kernels/backward.hip:710-735: base, causal, GQA,
ragged tails, SQ != SK both ways, windows, head dims, softcap, alibi). Bounds, per gradient:
  * rel_rms against the exact fp64 gradients <= 5e-4 (fp16) / 4e-3 (bf16), the BASELINE.json
    bounds (the reference's own gate allowed 2.5e-3 / 6e-3, kernels/backward.hip:734);
  * bitwise-identical results across repeated runs (the atomic-free contract).
Each case also runs the oracle's dtype rounding model (oracle.bwd(..., model=dtype,
stored_o=the kernel's O): D from the stored output, z*P and dS rounded to the dtype, as any
16-bit-operand backward must); its distance from the exact gradients is the case's floor, and
where that floor exceeds 2/3 of the bound the bound becomes 1.5x the floor (tests/helpers.py
check_grads). Every case logs its errors, its distance from the model and the floor.
At the full BASELINE.json configs[2] size sampled heads are checked against the fp64 oracle.

Every case runs both backward paths: "ds" (the dK/dV kernel stores dS in a workspace and
dQ = dS.K is formed from it, the default; small grids also split the pair dK/dV kernel's query
tiles) and "recompute" (no workspace: the dQ kernel recomputes S and dP).
"""
import math

import numpy as np
import pytest

from oracle import oracle as orc
from tests.helpers import check_grads, gen, to_dev, to_np

pytestmark = pytest.mark.gpu

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
    # every kernel width (multiples of 32), and head dims below their width (zero columns)
    ("D16 causal", 1, 4, 2, 130, 130, 16, True, -1, -1, 0.0, False),
    ("D32 causal", 1, 4, 2, 150, 150, 32, True, -1, -1, 0.0, False),
    ("D136 full gqa", 1, 4, 2, 90, 110, 136, False, -1, -1, 0.0, False),
    ("D176 causal", 1, 2, 2, 100, 100, 176, True, -1, -1, 0.0, False),
    ("D200 window (30,10)", 1, 2, 1, 90, 90, 200, False, 30, 10, 0.0, False),
    ("D48 full", 1, 4, 4, 100, 120, 48, False, -1, -1, 0.0, False),
    ("D80 causal gqa", 1, 8, 2, 160, 160, 80, True, -1, -1, 0.0, False),
    ("D96 window (40,0)", 1, 4, 4, 200, 200, 96, False, 40, 0, 0.0, False),
    ("D160 causal", 1, 2, 2, 96, 96, 160, True, -1, -1, 0.0, False),
    ("D192 full softcap", 1, 2, 1, 80, 100, 192, False, -1, -1, 20.0, False),
    ("D224 causal", 1, 2, 2, 70, 70, 224, True, -1, -1, 0.0, False),
    # small dK/dV grids whose key blocks split their query tiles over several workgroups
    # (fp32 partials summed by a merge kernel; "ds" path only)
    ("split D128 causal gqa4 S640", 1, 8, 2, 640, 640, 128, True, -1, -1, 0.0, False),
    ("split D64 full S1100x900", 1, 2, 2, 1100, 900, 64, False, -1, -1, 0.0, False),
    ("split D96 window (300,0) softcap", 1, 4, 2, 700, 700, 96, True, 300, 0, 20.0, False),
    ("split D32 causal alibi", 1, 4, 4, 1200, 1200, 32, True, -1, -1, 0.0, True),
    # grids of many short causal key blocks at head dim 128 (at least 512 work items, at most 16
    # query tiles each): the persistent dK/dV kernel, each workgroup running a list of items
    # ("ds" path only)
    ("persist D128 causal B8 S512", 8, 16, 16, 512, 512, 128, True, -1, -1, 0.0, False),
    ("persist D128 causal B8 S500 tail", 8, 16, 16, 500, 500, 128, True, -1, -1, 0.0, False),
    ("persist D128 causal gqa2 B32 S256", 32, 16, 8, 256, 256, 128, True, -1, -1, 0.0, False),
    ("persist D128 window (100,0) softcap", 8, 16, 16, 512, 512, 128, True, 100, 0, 20.0, False),
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
    model = orc.bwd(q, k, v, do, scale, causal, wl, wr, sc, al, model=dt, stored_o=to_np(out))
    return res, ref, model


@pytest.mark.parametrize("path", list(PATHS))
@pytest.mark.parametrize("dt", ["f16", "bf16"])
@pytest.mark.parametrize("case", CASES, ids=[c[0] for c in CASES])
def test_backward_parity(case, dt, path):
    print(f"[bwd] {case[0]} {dt} {path}", flush=True)
    res, ref, model = run(case, dt, repeats=3, path=path)
    for i, name in enumerate(("dq", "dk", "dv")):
        for r in res[1:]:
            assert torch_equal(r[i], res[0][i]), f"{name} differs between runs"
    check_grads("bwd_" + path, case[0], dt, res[0], ref, model)


def torch_equal(a, b):
    import torch
    return bool(torch.equal(a, b))


@pytest.mark.parametrize("path", list(PATHS))
def test_backward_full_config_c3(path):
    """causal bf16, B=2, S=4096, H=32, D=128; bitwise identical over
    3 runs; the gradients of sampled (batch, head) pairs (first, last and a middle one) against
    the fp64 oracle and its rounding model, with the bounds of the small cases."""
    import torch

    from fable_attn import _C
    from fable_attn.flash_attn_interface import _bhsd
    B, S, H, D = 2, 4096, 32, 128
    g = torch.Generator(device="cuda").manual_seed(0)
    q, k, v, do = (torch.randn(B, S, H, D, device="cuda", dtype=torch.bfloat16, generator=g)
                   for _ in range(4))
    qh, kh, vh, doh = (_bhsd(x) for x in (q, k, v, do))
    scale = D ** -0.5
    out, lse = _C.fwd(qh, kh, vh, scale, True, -1, 0, 0.0, None, 0.0, 0)
    print(f"[bwd] C3 full size {path}", flush=True)
    runs = [_C.bwd(doh, qh, kh, vh, out, lse, scale, True, -1, 0, 0.0, None, 0.0, 0,
                   ds_max_bytes=PATHS[path]) for _ in range(3)]
    torch.cuda.synchronize()
    for r in runs[1:]:
        for a, b in zip(runs[0], r):
            assert torch.equal(a, b)
    heads = ((0, 0), (1, 31), (1, 13))
    # the sampled heads as one B=1, H=3 problem (the oracle runs one thread per head)
    pick = lambda t: np.stack([to_np(t[bb, :, hd]) for bb, hd in heads])[None]
    qs, ks, vs, dos = pick(q), pick(k), pick(v), pick(do)
    ref = orc.bwd(qs, ks, vs, dos, scale, True)
    model = orc.bwd(qs, ks, vs, dos, scale, True, model="bf16",
                    stored_o=np.stack([to_np(out[bb, hd]) for bb, hd in heads])[None])
    got = [torch.stack([x[bb, hd] for bb, hd in heads])[None] for x in runs[0]]
    check_grads("bwd_full_c3_" + path, "C3 B2 S4096 H32 D128 heads (0,0),(1,31),(1,13)", "bf16",
                got, ref, model)


def test_backward_ds_workspace_too_small_falls_back():
    """A dS workspace smaller than fable_attn_bwd_ds_bytes reports, or not 16-byte aligned,
    must be ignored (the recomputing path runs, the buffer stays untouched); a full-size one
    filled with NaN bit
    patterns must give the same gradients (tiles that are never written are never read).
    Both against the oracle, through the C-ABI with a hand-built FableBwdParams."""
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
    p = _lib.FableBwdParams()
    p.Q, p.K, p.V, p.O, p.dO = qd.data_ptr(), kd.data_ptr(), vd.data_ptr(), out.data_ptr(), dod.data_ptr()
    p.dQ, p.dK, p.dV = dq.data_ptr(), dk.data_ptr(), dv.data_ptr()
    p.lse, p.dsum = lse.data_ptr(), dsum.data_ptr()
    bhs = lambda t: _lib.Strides(*t.stride()[:3])
    p.qs, p.ks, p.vs, p.os, p.dos = bhs(qd), bhs(kd), bhs(vd), bhs(out), bhs(dod)
    p.dqs, p.dks, p.dvs = bhs(dq), bhs(dk), bhs(dv)
    p.B, p.Hq, p.Hk, p.SQ, p.SK, p.D, p.gqa = B, Hq, Hk, SQ, SK, D, Hq // Hk
    p.scale, p.causal, p.win_left, p.win_right, p.keep_scale = scale, 1, -1, -1, 1.0
    need = lib.fable_attn_bwd_ds_bytes(p, 1)
    assert need == 256 + B * Hq * 15 * 2048   # table + the 15 causal tiles of a 5x5 block grid
    ws = torch.full((need + 16,), 0xFF, dtype=torch.uint8, device="cuda")  # NaN bit patterns
    stream = ctypes_stream()
    # too small, then big enough but not 16-byte aligned: both ignored
    for ptr, nbytes in ((ws.data_ptr(), need - 1), (ws.data_ptr() + 8, need)):
        p.ds_ws, p.ds_ws_bytes = ptr, nbytes
        assert lib.fable_attn_bwd(p, 1, stream) == 0
        torch.cuda.synchronize()
        assert torch.all(ws == 0xFF), "an unusable workspace must not be written"
    p.ds_ws = ws.data_ptr()
    ref = orc.bwd(q, k, v, do, scale, causal)
    model = orc.bwd(q, k, v, do, scale, causal, model=dt, stored_o=to_np(out))
    check_grads("bwd_ws_ignored", name, dt, (dq, dk, dv), ref, model)
    # a full-size workspace poisoned with NaN patterns: the dQ kernel reads only the tiles the
    # dK/dV kernel wrote (the causal upper-right tiles stay NaN and must not leak into dQ)
    p.ds_ws_bytes = need
    assert lib.fable_attn_bwd(p, 1, stream) == 0
    torch.cuda.synchronize()
    assert not torch.all(ws == 0xFF), "the workspace path was not taken"
    check_grads("bwd_ws_poisoned", name, dt, (dq, dk, dv), ref, model)


def ctypes_stream():
    import ctypes

    import torch
    return ctypes.c_void_p(torch.cuda.current_stream().cuda_stream)


def test_backward_long_causal_takes_the_ds_path():
    """The C2 shape's backward (causal bf16, B=1, S=16384, H=32, D=128): the dS workspace holds
    only the causal triangle's tiles (~8.6 GB instead of the 17 GB rectangle), fits the default
    cap, and the dS path gives the recomputing path's dV bit for bit (the same pair kernel, which
    only adds the tile stores), its dK and dQ to rounding (D = rowsum(O*dO) is summed in another
    order by the two paths), bitwise reproducibly."""
    import torch

    from fable_attn import _C, _lib
    from fable_attn.flash_attn_interface import _bhsd
    B, S, H, D = 1, 16384, 32, 128
    lib = _lib.load()
    p = _lib.FableBwdParams()
    p.B, p.Hq, p.Hk, p.gqa, p.SQ, p.SK, p.D, p.causal = B, H, H, 1, S, S, D, 1
    p.win_left, p.win_right = -1, 0
    need = lib.fable_attn_bwd_ds_bytes(p, 1)
    assert need == 2304 + B * H * (512 * 513 // 2) * 2048 and need <= _C.BWD_DS_MAX_BYTES
    g = torch.Generator(device="cuda").manual_seed(4)
    q, k, v, do = (torch.randn(B, S, H, D, device="cuda", dtype=torch.bfloat16, generator=g)
                   for _ in range(4))
    qh, kh, vh, doh = (_bhsd(x) for x in (q, k, v, do))
    scale = D ** -0.5
    out, lse = _C.fwd(qh, kh, vh, scale, True, -1, 0, 0.0, None, 0.0, 0)
    print("[bwd] S=16384 H=32 causal: dS path", flush=True)
    ds = [_C.bwd(doh, qh, kh, vh, out, lse, scale, True, -1, 0, 0.0, None, 0.0, 0) for _ in range(2)]
    torch.cuda.synchronize()
    for a, b in zip(*ds):
        assert torch.equal(a, b), "dS path differs between runs"
    print("[bwd] S=16384 H=32 causal: recomputing path", flush=True)
    rc = _C.bwd(doh, qh, kh, vh, out, lse, scale, True, -1, 0, 0.0, None, 0.0, 0, ds_max_bytes=0)
    torch.cuda.synchronize()
    assert torch.equal(ds[0][2], rc[2]), "dV differs between paths"
    for i, name in ((0, "dQ"), (1, "dK")):
        e = ((ds[0][i].float() - rc[i].float()).norm() / rc[i].float().norm()).item()
        assert torch.isfinite(ds[0][i]).all() and e <= 1e-3, f"{name} of the two paths: rel_rms {e:.3e}"


def test_backward_query_split_taken():
    """The "split" cases above take the pair kernel's query split: after their 256-byte-aligned
    dS tiles, the workspace they get holds n >= 2 shares of fp32 partial dK and dV rows."""
    from fable_attn import _C, _lib
    for case in [c for c in CASES if c[0].startswith("split")]:
        name, B, Hq, Hk, SQ, SK, D, causal, wl, wr, sc, alibi = case
        p = _lib.FableBwdParams()
        p.B, p.Hq, p.Hk, p.gqa, p.SQ, p.SK, p.D = B, Hq, Hk, Hq // Hk, SQ, SK, D
        p.causal, p.win_left, p.win_right = int(causal), wl, wr
        got = _C._L.fable_attn_bwd_ds_bytes(p, 0)
        p.B = 64                                   # many rounds of workgroups: no split
        hdr = -(-((SK + 31) // 32 + 1) * 4 // 256) * 256
        tiles = (_C._L.fable_attn_bwd_ds_bytes(p, 0) - hdr) // 64
        extra = got - -(-(hdr + B * tiles) // 256) * 256
        bk = 128 if (D + 31) // 32 * 32 == 128 else 64      # keys per pair-kernel workgroup
        share = 2 * B * Hk * -(-SK // bk) * bk * D * 4       # dK and dV rows of every work item
        assert extra > 0 and extra % share == 0 and extra // share >= 2, (name, got, extra)
