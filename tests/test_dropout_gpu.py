"""Dropout on the GPU, bit-compatible with the reference's scheme: Philox4x32-10 word 0 on the
counter (idx, 0, 0) under the key `seed`, idx = (h*SQ + q)*SK + key with no batch term, kept
iff (word0 >> 8) * 2^-24 >= p, kept probabilities scaled by 1/(1-p) after the row sum
(kernels/fa_common.hpp:71-88, fa_forward.hip:255-259); backward dV = (z P)^T dO and
dS = P (z dP - D) (backward.hip:170-176).

Checks, through the C-ABI (fable_attn._C):
  * the keep mask, bit for bit: with V = identity rows, O[i, j] is zero exactly where the
    oracle's mask drops (i, j), for every head dim, GQA, a ragged SQ and packed varlen
    sequences (whose idx uses each sequence's own SQ/SK);
  * forward O against the fp64 oracle with the same seed (rel_rms <= 5e-4 fp16 / 4e-3 bf16),
    LSE that of the undropped probabilities (<= 1e-3 abs);
  * backward gradients against the fp64 oracle and its dtype rounding model (tests/helpers.py
    check_grads: rel_rms <= 5e-4 fp16 / 4e-3 bf16 vs the exact gradients) and bitwise
    reproducible;
  * flash_attn_func / flash_attn_varlen_func autograd: the backward reuses the forward's seed.
"""
import math
import random

import numpy as np
import pytest

from oracle import oracle as orc
from tests.helpers import LSE_ABS, TOL, check_grads, gen, log_errors, lse_err, to_dev, to_np

pytestmark = pytest.mark.gpu
SEED = 0x5DEECE66D1234

# name, B, Hq, Hk, SQ, SK, D, causal, p, softcap
CASES = [
    ("D64 full B2", 2, 4, 4, 96, 96, 64, False, 0.2, 0.0),
    ("D64 causal gqa", 1, 8, 2, 128, 128, 64, True, 0.1, 0.0),
    ("D128 causal SQ<SK", 1, 4, 4, 100, 160, 128, True, 0.3, 0.0),
    ("D128 softcap gqa", 1, 4, 2, 128, 128, 128, False, 0.2, 20.0),
    ("D256 causal", 1, 2, 2, 80, 80, 256, True, 0.25, 0.0),
    # dropout kernels of the other widths
    ("D32 causal", 1, 4, 2, 100, 100, 32, True, 0.15, 0.0),
    ("D96 full", 1, 2, 2, 70, 90, 96, False, 0.2, 0.0),
    ("D160 causal", 1, 2, 1, 64, 64, 160, True, 0.1, 0.0),
    ("D192 full softcap", 1, 2, 2, 60, 60, 192, False, 0.3, 10.0),
    # a grid of 512 short causal key blocks at head dim 128: the persistent dK/dV kernel
    ("D128 causal B8 S512 persistent", 8, 16, 16, 512, 512, 128, True, 0.1, 0.0),
]


def _view(a, dt):
    """public (B,S,H,D) storage, [B,H,S,D] view"""
    return to_dev(a, dt).transpose(1, 2).contiguous().transpose(1, 2)


def _inputs(case, dt, seed=0):
    name, B, Hq, Hk, SQ, SK, D, causal, p, sc = case
    q = gen((B, Hq, SQ, D), seed + 1, dt)
    k = gen((B, Hk, SK, D), seed + 2, dt)
    v = gen((B, Hk, SK, D), seed + 3, dt)
    do = gen((B, Hq, SQ, D), seed + 4, dt)
    return q, k, v, do


@pytest.mark.parametrize("D", [64, 128, 256])
def test_forward_mask_bit_exact(D):
    """V = identity: O[b,h,i,j] = z[h,i,j] P[b,h,i,j] / 1 with P > 0 everywhere (non-causal,
    finite scores), so the zeros of O are exactly the dropped entries."""
    import torch

    from fable_attn import _C
    print(f"[dropout-mask] D={D}", flush=True)
    B, Hq, Hk, SQ, SK, p = 2, 4, 2, 37, D, 0.3
    q = gen((B, Hq, SQ, D), 11, "f16") * 0.25
    k = gen((B, Hk, SK, D), 12, "f16") * 0.25
    v = np.broadcast_to(np.eye(SK, D, dtype=np.float32), (B, Hk, SK, D)).copy()
    out, _ = _C.fwd(_view(q, "f16"), _view(k, "f16"), _view(v, "f16"), 1.0 / math.sqrt(D), False,
                    -1, -1, 0.0, None, p, SEED)
    torch.cuda.synchronize()
    o = to_np(out)
    z = orc.keep_mask(SEED, float(np.float32(p)), Hq, SQ, SK)
    for b in range(B):
        dropped = o[b, :, :, :SK] == 0
        assert np.array_equal(dropped, z == 0), f"batch {b}: mask differs in {(dropped != (z == 0)).sum()} places"


def test_forward_mask_varlen_per_sequence():
    """Packed sequences: each one's idx runs over its own SQ/SK (fa_forward.hip:66-73, 258)."""
    import torch

    from fable_attn import _C
    D, H, p = 64, 2, 0.4
    lq, lk = [23, 50, 7], [64, 40, 9]
    cq = np.concatenate([[0], np.cumsum(lq)]).astype(np.int32)
    ck = np.concatenate([[0], np.cumsum(lk)]).astype(np.int32)
    q = gen((sum(lq), H, D), 21, "f16") * 0.25
    k = gen((sum(lk), H, D), 22, "f16") * 0.25
    v = np.zeros((sum(lk), H, D), np.float32)
    for i in range(len(lk)):
        v[ck[i]:ck[i + 1]] = np.eye(lk[i], D, dtype=np.float32)[:, None, :]
    out = _C.fwd_varlen(to_dev(q, "f16"), to_dev(k, "f16"), to_dev(v, "f16"),
                        torch.from_numpy(cq).cuda(), torch.from_numpy(ck).cuda(), max(lq), max(lk),
                        0.125, False, -1, -1, 0.0, None, p, SEED, 0)
    torch.cuda.synchronize()
    o = to_np(out)
    for i in range(len(lq)):
        z = orc.keep_mask(SEED, float(np.float32(p)), H, lq[i], lk[i])   # [H, SQ, SK]
        dropped = o[cq[i]:cq[i + 1], :, :lk[i]].transpose(1, 0, 2) == 0
        assert np.array_equal(dropped, z == 0), f"sequence {i}"


@pytest.mark.parametrize("dt", ["f16", "bf16"])
@pytest.mark.parametrize("case", CASES, ids=[c[0] for c in CASES])
def test_forward_dropout_vs_oracle(case, dt):
    import torch

    from fable_attn import _C
    print(f"[dropout-fwd] {case[0]} {dt}", flush=True)
    name, B, Hq, Hk, SQ, SK, D, causal, p, sc = case
    q, k, v, _ = _inputs(case, dt)
    scale = 1.0 / math.sqrt(D)
    out, lse = _C.fwd(_view(q, dt), _view(k, dt), _view(v, dt), scale, causal, -1, -1, sc, None, p, SEED)
    torch.cuda.synchronize()
    ro, rl = orc.fwd(q, k, v, scale, causal, -1, -1, sc, dropout_p=p, seed=SEED)
    e = orc.rel_rms(to_np(out), ro)
    le, inf_ok = lse_err(to_np(lse), rl)
    log_errors("dropout_fwd", name, dt, o=e, lse=le)
    assert e <= TOL[dt], f"O rel_rms {e:.3e} > {TOL[dt]}"
    assert inf_ok and le <= LSE_ABS, f"LSE err {le:.3e}"


@pytest.mark.parametrize("ds_max", [None, 0], ids=["ds", "recompute"])
@pytest.mark.parametrize("dt", ["f16", "bf16"])
@pytest.mark.parametrize("case", CASES, ids=[c[0] for c in CASES])
def test_backward_dropout_vs_oracle(case, dt, ds_max):
    """Both backward paths (dS workspace, or the dQ kernel recomputing dS) against the oracle."""
    import torch

    from fable_attn import _C
    print(f"[dropout-bwd] {case[0]} {dt} ds_max={ds_max}", flush=True)
    name, B, Hq, Hk, SQ, SK, D, causal, p, sc = case
    q, k, v, do = _inputs(case, dt, seed=10)
    scale = 1.0 / math.sqrt(D)
    qd, kd, vd, dod = (_view(x, dt) for x in (q, k, v, do))
    out, lse = _C.fwd(qd, kd, vd, scale, causal, -1, -1, sc, None, p, SEED)
    g1 = _C.bwd(dod, qd, kd, vd, out, lse, scale, causal, -1, -1, sc, None, p, SEED, ds_max_bytes=ds_max)
    g2 = _C.bwd(dod, qd, kd, vd, out, lse, scale, causal, -1, -1, sc, None, p, SEED, ds_max_bytes=ds_max)
    torch.cuda.synchronize()
    args = (q, k, v, do, scale, causal, -1, -1, sc, None)
    ref = orc.bwd(*args, dropout_p=p, seed=SEED)
    model = orc.bwd(*args, dropout_p=p, seed=SEED, model=dt, stored_o=to_np(out))
    for i, gname in enumerate(("dq", "dk", "dv")):
        assert torch.equal(g1[i], g2[i]), f"{gname} differs between runs"
    check_grads("dropout_bwd_" + ("ds" if ds_max is None else "recompute"), name, dt, g1, ref, model)


def test_autograd_reuses_forward_seed():
    """flash_attn_func draws the seed with random.getrandbits(63) (as the reference,
    flash_attn_interface.py:239) and hands it to the backward."""
    import torch

    from fable_attn import flash_attn_func
    B, S, H, D, p = 1, 96, 4, 64, 0.2
    g = torch.Generator(device="cuda").manual_seed(1)
    q, k, v = (torch.randn(B, S, H, D, device="cuda", dtype=torch.float16, generator=g).requires_grad_()
               for _ in range(3))
    dout = torch.randn(B, S, H, D, device="cuda", dtype=torch.float16, generator=g)
    random.seed(42)
    seed = random.getrandbits(63)
    random.seed(42)
    out = flash_attn_func(q, k, v, dropout_p=p, causal=True)
    out.backward(dout)
    torch.cuda.synchronize()
    bhsd = lambda t: to_np(t).transpose(0, 2, 1, 3)
    ro, _ = orc.fwd(bhsd(q), bhsd(k), bhsd(v), D ** -0.5, True, dropout_p=p, seed=seed)
    assert orc.rel_rms(bhsd(out), ro) <= TOL["f16"]
    args = (bhsd(q), bhsd(k), bhsd(v), bhsd(dout), D ** -0.5, True)
    ref = orc.bwd(*args, dropout_p=p, seed=seed)
    model = orc.bwd(*args, dropout_p=p, seed=seed, model="f16", stored_o=bhsd(out))
    check_grads("dropout_autograd", "causal D64", "f16",
                [bhsd(x.grad) for x in (q, k, v)], ref, model)


def test_varlen_autograd_dropout():
    import torch

    from fable_attn import flash_attn_varlen_func
    H, D, p = 2, 64, 0.25
    lens = [40, 75, 3]
    cu = np.concatenate([[0], np.cumsum(lens)]).astype(np.int32)
    g = torch.Generator(device="cuda").manual_seed(2)
    tot = sum(lens)
    q, k, v = (torch.randn(tot, H, D, device="cuda", dtype=torch.float16, generator=g).requires_grad_()
               for _ in range(3))
    dout = torch.randn(tot, H, D, device="cuda", dtype=torch.float16, generator=g)
    random.seed(9)
    seed = random.getrandbits(63)
    random.seed(9)
    cut = torch.from_numpy(cu).cuda()
    out = flash_attn_varlen_func(q, k, v, cut, cut, max(lens), max(lens), dropout_p=p, causal=True)
    out.backward(dout)
    torch.cuda.synchronize()
    for i in range(len(lens)):
        a, b = cu[i], cu[i + 1]
        seq = lambda t: to_np(t[a:b]).transpose(1, 0, 2)[None]
        ro, _ = orc.fwd(seq(q), seq(k), seq(v), D ** -0.5, True, dropout_p=p, seed=seed)
        assert orc.rel_rms(seq(out), ro) <= TOL["f16"], f"seq {i} O"
        args = (seq(q), seq(k), seq(v), seq(dout), D ** -0.5, True)
        ref = orc.bwd(*args, dropout_p=p, seed=seed)
        model = orc.bwd(*args, dropout_p=p, seed=seed, model="f16", stored_o=seq(out))
        check_grads("dropout_varlen_autograd", f"seq {i}", "f16",
                    [seq(x.grad) for x in (q, k, v)], ref, model, vanish_ok=True)
