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
