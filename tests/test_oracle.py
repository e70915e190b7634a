"""Pinning the fp64 oracle (CPU only).

The oracle is trusted only after these checks:
  * forward: equal to the reference's own ref_attention (oracle/_ref, compiled from
    kernels/fa_common.hpp) on the reference gate's seeded inputs, through the committed golden
    fixture (tests/golden/fwd_golden.npz, generated and cross-checked by make_golden.py) and,
    where _ref is built, directly on fresh cases; plus closed forms (single visible key,
    diagonal window, constant scores, empty rows, softcap limit);
  * backward: torch.autograd on an fp64 CPU attention and central finite differences of an
    fp64 forward, including softcap (whose derivative a plausible bug would drop), GQA and
    windows;
  * backward rounding model (the dtype roundings of a 16-bit-operand backward, which sets the
    floor of the gradient bounds): bit-exact where one key per query makes dS vanish, the
    closed-form shift of dQ/dK (and none of dV) when the stored O moves, and a distance from
    the exact gradients that is a fraction of the unit roundoff and ~8x larger in bf16;
  * decode: the forward oracle on gathered pages (no append, append, window, leftpad, nq > 1),
    rotary against a complex-multiplication rotation, invariance under page permutation;
  * combine: merging two key halves equals attention over all keys;
  * dropout: Philox4x32-10 against the Random123 known-answer vectors, the keep mask against
    the reference's own host replica of its dropout multiplier (oracle/_ref, compiled from
    kernels/backward.hip) where that is built, the keep rate, a one-hot V that reads the mask
    back out of the forward, and finite differences of the dropout backward under a fixed mask.
"""
import math
import os

import numpy as np
import pytest

from oracle import oracle as orc
from tests.golden.make_golden import CASES as GOLDEN_CASES
from tests.golden.make_golden import gate_inputs

GOLDEN = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden", "fwd_golden.npz")


def test_frand_matches_lcg_stream():
    s = 1234567
    seq = []
    for _ in range(257):
        s = (s * 1664525 + 1013904223) & 0xFFFFFFFF
        seq.append(((s >> 16) & 4095) / 4096.0 - 0.5)
    vals, last = orc.frand(257, 1234567)
    assert np.array_equal(vals, np.array(seq, dtype=np.float32)) and last == s


def test_round_bf16_rne():
    x = np.array([1.0, 1.0 + 2 ** -8, 1.0 + 3 * 2 ** -8, -2.5, 3.0e38, 1e-40], dtype=np.float32)
    r = orc.round_bf16(x)
    # ties to even: 1+2^-8 -> 1.0, 1+3*2^-8 -> 1+2^-6
    assert r[0] == 1.0 and r[1] == 1.0 and r[2] == np.float32(1.0 + 2 ** -6) and r[3] == -2.5


@pytest.mark.parametrize("idx", range(len(GOLDEN_CASES)), ids=[c[0] for c in GOLDEN_CASES])
@pytest.mark.parametrize("dt", ["f16", "bf16"])
def test_oracle_matches_golden(idx, dt):
    name, SQ, SK, HD, NH, gqa, causal, alibi, wl, wr, sc, chunk = GOLDEN_CASES[idx]
    g = np.load(GOLDEN)
    key = f"c{idx}_{dt}"
    meta = g[key + "_meta"]
    assert list(meta) == [SQ, SK, HD, NH, gqa, int(causal), int(alibi), wl, wr, chunk]
    q, k, v = gate_inputs(SQ, SK, HD, NH, gqa, dt)
    al = (-np.float32(2.0) ** (-(8.0 * np.arange(1, NH + 1, dtype=np.float32) / NH))
          ).astype(np.float32) if alibi else None
    scale = np.float32(1.0) / np.sqrt(np.float32(HD))
    hs, rs = g[key + "_hs"], g[key + "_rs"]
    o, l = orc.fwd(q, k, v, scale, causal, wl, wr, sc, al, chunk, rows=np.unique(rs))
    lref = g[key + "_lse"]
    got = o[0, hs, rs, :]
    assert np.abs(got - g[key + "_o"]).max() <= 1e-6 * max(1.0, np.abs(g[key + "_o"]).max())
    sel = np.zeros_like(lref, dtype=bool)
    sel[:, :, np.unique(rs)] = True
    fin = np.isfinite(lref) & sel
    assert np.array_equal(np.isneginf(l[sel]), np.isneginf(lref[sel]))
    assert np.abs(l[fin] - lref[fin]).max() <= 1e-5


def _need_ref(lib):
    """Skip (inside the test body, so nothing built from the reference is loaded at collection)
    when oracle/_ref was not built, as on a GPU box without the reference tree."""
    if lib is None:
        pytest.skip("oracle/_ref not built (reference tree absent)")
    return lib


@pytest.mark.parametrize("cfg", [
    (64, 64, 64, 4, 2, True, -1, -1, 0.0, 0, False),
    (48, 80, 32, 4, 4, True, -1, -1, 0.0, 0, False),
    (80, 40, 64, 4, 1, True, -1, -1, 0.0, 0, False),
    (64, 64, 64, 4, 4, False, 8, 8, 0.0, 0, False),
    (64, 64, 64, 4, 4, True, -1, -1, 30.0, 0, True),
    (64, 96, 64, 4, 4, True, -1, -1, 0.0, 20, False),
    (33, 71, 96, 6, 3, False, 5, -1, 7.0, 0, True),
])
def test_oracle_matches_reference_directly(cfg):
    _need_ref(orc.ref_lib())
    SQ, SK, D, H, Hk, causal, wl, wr, sc, chunk, alibi = cfg
    rng = np.random.default_rng(sum(cfg[:5]))
    q = orc.round_to(rng.standard_normal((1, H, SQ, D)), "f16")
    k = orc.round_to(rng.standard_normal((1, Hk, SK, D)), "f16")
    v = orc.round_to(rng.standard_normal((1, Hk, SK, D)), "f16")
    al = (-np.float32(2.0) ** (-(8.0 * np.arange(1, H + 1) / H))).astype(np.float32) if alibi else None
    o, l = orc.fwd(q, k, v, D ** -0.5, causal, wl, wr, sc, al, chunk)
    ro, rl = orc.reference_fwd(q, k, v, np.float32(D ** -0.5), causal, wl, wr, sc, al, chunk)
    assert np.abs(o - ro).max() <= 1e-6
    assert np.array_equal(np.isneginf(l), np.isneginf(rl))
    fin = np.isfinite(rl)
    assert np.abs(l[fin] - rl[fin]).max() <= 1e-5


def _rand(shape, seed):
    return orc.round_to(np.random.default_rng(seed).standard_normal(shape), "f16")


def test_closed_form_single_key_and_diagonal():
    q, k, v = _rand((1, 2, 16, 32), 1), _rand((1, 2, 16, 32), 2), _rand((1, 2, 16, 32), 3)
    # window (0,0): only key i visible -> O = V[i], LSE = scale*q.k
    o, l = orc.fwd(q, k, v, 0.25, False, 0, 0)
    assert np.allclose(o, v, atol=1e-6)
    s = (q.astype(np.float64) * k).sum(-1) * np.float32(0.25)
    assert np.allclose(l, s, atol=1e-5)
    # SK=1, no mask: every query sees key 0 only -> O = V[0]
    o, l = orc.fwd(q, k[:, :, :1], v[:, :, :1], 0.25, False)
    assert np.allclose(o, np.broadcast_to(v[:, :, :1], o.shape), atol=1e-6)
    # SK=1 causal (bottom-right): only the last query sees key 0, the others are empty
    o, l = orc.fwd(q, k[:, :, :1], v[:, :, :1], 0.25, True)
    assert np.allclose(o[:, :, -1], v[:, :, 0], atol=1e-6) and (o[:, :, :-1] == 0).all()


def test_closed_form_constant_scores():
    # q = 0 -> all visible scores equal -> O = mean of visible V rows, LSE = ln(n)
    SQ, SK = 12, 20
    q = np.zeros((1, 1, SQ, 16), dtype=np.float32)
    k, v = _rand((1, 1, SK, 16), 4), _rand((1, 1, SK, 16), 5)
    o, l = orc.fwd(q, k, v, 1.0, True)
    delta = SK - SQ
    for i in range(SQ):
        n = i + delta + 1
        assert np.allclose(o[0, 0, i], v[0, 0, :n].astype(np.float64).mean(0), atol=1e-6)
        assert abs(l[0, 0, i] - math.log(n)) < 1e-6


def test_empty_rows_zero_and_neg_inf():
    q, k, v = _rand((1, 2, 40, 16), 6), _rand((1, 2, 8, 16), 7), _rand((1, 2, 8, 16), 8)
    o, l = orc.fwd(q, k, v, 0.25, True)
    assert (o[:, :, :32] == 0).all() and np.isneginf(l[:, :, :32]).all()
    assert np.isfinite(l[:, :, 32:]).all()


def test_softcap_limit():
    q, k, v = _rand((1, 2, 24, 32), 9), _rand((1, 2, 24, 32), 10), _rand((1, 2, 24, 32), 11)
    o1, l1 = orc.fwd(q, k, v, 0.2, True)
    o2, l2 = orc.fwd(q, k, v, 0.2, True, softcap=1e6)
    assert np.abs(o1 - o2).max() < 1e-5 and np.abs(l1 - l2).max() < 1e-5


def _np_attention(q, k, v, scale, causal, wl=-1, wr=-1, softcap=0.0, z=None):
    """fp64 numpy attention (a textbook softmax(QK^T)V with the mask contract), for finite
    differences only. z [H, SQ, SK]: fixed multipliers applied to the probabilities (dropout)."""
    H, Hk = q.shape[1], k.shape[1]
    k = np.repeat(k, H // Hk, axis=1).astype(np.float64)
    v = np.repeat(v, H // Hk, axis=1).astype(np.float64)
    s = np.einsum("bhid,bhjd->bhij", q.astype(np.float64), k) * scale
    if softcap > 0:
        s = softcap * np.tanh(s / softcap)
    SQ, SK = q.shape[2], k.shape[2]
    i = np.arange(SQ)[:, None]
    j = np.arange(SK)[None, :]
    d = SK - SQ
    m = np.zeros((SQ, SK), dtype=bool)
    if causal:
        m |= j > i + d
    if wl >= 0:
        m |= j < i + d - wl
    if wr >= 0:
        m |= j > i + d + wr
    s = np.where(m, -np.inf, s)
    mx = s.max(-1, keepdims=True)
    p = np.exp(s - mx)
    p /= p.sum(-1, keepdims=True)
    if z is not None:
        p = p * z[None]
    return np.einsum("bhij,bhjd->bhid", p, v)


@pytest.mark.parametrize("cfg", [
    (1, 4, 2, 9, 11, 8, True, -1, -1, 0.0),
    (2, 2, 2, 7, 7, 8, False, 2, 1, 0.0),
    (1, 2, 1, 6, 10, 8, True, -1, -1, 3.0),
])
def test_backward_finite_differences(cfg):
    B, H, Hk, SQ, SK, D, causal, wl, wr, sc = cfg
    rng = np.random.default_rng(3)
    q = rng.standard_normal((B, H, SQ, D)).astype(np.float32)
    k = rng.standard_normal((B, Hk, SK, D)).astype(np.float32)
    v = rng.standard_normal((B, Hk, SK, D)).astype(np.float32)
    do = rng.standard_normal((B, H, SQ, D)).astype(np.float32)
    scale = np.float32(0.37)
    dq, dk, dv = orc.bwd(q, k, v, do, scale, causal, wl, wr, sc)
    loss = lambda q_, k_, v_: (_np_attention(q_, k_, v_, float(scale), causal, wl, wr, sc) * do).sum()
    eps = 1e-3
    for name, x, g in (("q", q, dq), ("k", k, dk), ("v", v, dv)):
        for idx in [tuple(rng.integers(0, s) for s in x.shape) for _ in range(6)]:
            xp, xm = x.astype(np.float64).copy(), x.astype(np.float64).copy()
            xp[idx] += eps
            xm[idx] -= eps
            args = {"q": (q, k, v), "k": (q, k, v), "v": (q, k, v)}[name]
            ap = [a.astype(np.float64) for a in args]
            am = [a.astype(np.float64) for a in args]
            pos = "qkv".index(name)
            ap[pos], am[pos] = xp, xm
            fd = (loss(*ap) - loss(*am)) / (2 * eps)
            assert abs(fd - g[idx]) <= 1e-5 + 1e-4 * abs(fd), (name, idx, fd, g[idx])


def test_backward_matches_torch_autograd():
    import torch
    B, H, Hk, SQ, SK, D = 2, 4, 2, 17, 23, 16
    rng = np.random.default_rng(4)
    q = rng.standard_normal((B, H, SQ, D)).astype(np.float32)
    k = rng.standard_normal((B, Hk, SK, D)).astype(np.float32)
    v = rng.standard_normal((B, Hk, SK, D)).astype(np.float32)
    do = rng.standard_normal((B, H, SQ, D)).astype(np.float32)
    for causal, wl, wr, sc in ((True, -1, -1, 0.0), (False, 4, 3, 0.0), (True, -1, -1, 5.0)):
        dq, dk, dv = orc.bwd(q, k, v, do, 0.3, causal, wl, wr, sc)
        tq, tk, tv = (torch.tensor(x, dtype=torch.float64, requires_grad=True) for x in (q, k, v))
        kk = tk.repeat_interleave(H // Hk, dim=1)
        vv = tv.repeat_interleave(H // Hk, dim=1)
        s = tq @ kk.transpose(-1, -2) * float(np.float32(0.3))
        if sc:
            s = sc * torch.tanh(s / sc)
        i = torch.arange(SQ).view(-1, 1)
        j = torch.arange(SK).view(1, -1)
        m = torch.zeros(SQ, SK, dtype=torch.bool)
        if causal:
            m |= j > i + SK - SQ
        if wl >= 0:
            m |= j < i + SK - SQ - wl
        if wr >= 0:
            m |= j > i + SK - SQ + wr
        o = torch.softmax(s.masked_fill(m, float("-inf")), -1) @ vv
        (o * torch.tensor(do, dtype=torch.float64)).sum().backward()
        for a, b in ((dq, tq.grad), (dk, tk.grad), (dv, tv.grad)):
            assert np.abs(a - b.numpy()).max() <= 1e-9 * max(1.0, np.abs(b.numpy()).max())


def _pages(kseq, page, nblocks, rng):
    """Scatter per-sequence K rows [B, L, Hk, D] into a paged cache with a random table."""
    B, L, Hk, D = kseq.shape
    per = (L + page - 1) // page
    perm = rng.permutation(nblocks)[:B * per].reshape(B, per).astype(np.int32)
    cache = np.zeros((nblocks, page, Hk, D), dtype=np.float32)
    for b in range(B):
        for p in range(per):
            rows = kseq[b, p * page:(p + 1) * page]
            cache[perm[b, p], :rows.shape[0]] = rows
    return cache, perm


@pytest.mark.parametrize("nq,append,window,leftpad", [
    (1, False, -1, 0), (1, True, -1, 0), (4, True, -1, 0), (3, False, -1, 0),
    (1, False, 17, 0), (2, True, 9, 0), (1, False, -1, 13),
])
def test_decode_equals_forward_on_gathered_pages(nq, append, window, leftpad):
    rng = np.random.default_rng(nq * 7 + append + window + leftpad)
    B, H, Hk, D, page, ctx = 2, 8, 2, 32, 16, 70
    L = ctx + (nq if append else 0)
    kseq = orc.round_to(rng.standard_normal((B, L, Hk, D)), "f16")
    vseq = orc.round_to(rng.standard_normal((B, L, Hk, D)), "f16")
    q = orc.round_to(rng.standard_normal((B, nq, H, D)), "f16")
    kc, bt = _pages(kseq[:, :ctx], page, 20, rng)
    vc = np.zeros_like(kc)
    for b in range(B):
        for p in range(bt.shape[1]):
            rows = vseq[b, p * page:min((p + 1) * page, ctx)]
            vc[bt[b, p], :rows.shape[0]] = rows
    nk, nv = (kseq[:, ctx:], vseq[:, ctx:]) if append else (None, None)
    lp = np.full(B, leftpad, dtype=np.int32) if leftpad else None
    o, l = orc.decode(q, kc, vc, bt, np.full(B, ctx, np.int32), 0.2, new_k=nk, new_v=nv,
                      window=window, leftpad=lp)
    # forward over the visible keys: queries at ctx..ctx+nq-1, keys [leftpad, L)
    kk = kseq[:, leftpad:L].transpose(0, 2, 1, 3)
    vv = vseq[:, leftpad:L].transpose(0, 2, 1, 3)
    qq = q.transpose(0, 2, 1, 3)
    if append:
        fo, fl = orc.fwd(qq, kk, vv, 0.2, True, window - 1 if window > 0 else -1, 0)
    else:
        # without append the new tokens see the whole cache (no causality among them); the
        # bottom-right aligned forward puts a single query at position ctx-1, one before the
        # decode query position ctx, so a decode window w is a forward left window w-2
        assert window < 0 or nq == 1
        fo, fl = orc.fwd(qq, kk, vv, 0.2, False, window - 2 if window > 0 else -1, -1)
    assert np.abs(o - fo.transpose(0, 2, 1, 3)).max() < 1e-6
    assert np.abs(l - fl.transpose(0, 2, 1)).max() < 1e-5


def test_decode_page_permutation_invariance():
    rng = np.random.default_rng(12)
    B, H, Hk, D, page, ctx = 2, 4, 2, 16, 8, 45
    q = orc.round_to(rng.standard_normal((B, 1, H, D)), "f16")
    kseq = orc.round_to(rng.standard_normal((B, ctx, Hk, D)), "f16")
    vseq = orc.round_to(rng.standard_normal((B, ctx, Hk, D)), "f16")
    outs = []
    for s in range(2):
        r = np.random.default_rng(100 + s)
        kc, bt = _pages(kseq, page, 16, r)
        vc = np.zeros_like(kc)
        for b in range(B):
            for p in range(bt.shape[1]):
                rows = vseq[b, p * page:min((p + 1) * page, ctx)]
                vc[bt[b, p], :rows.shape[0]] = rows
        outs.append(orc.decode(q, kc, vc, bt, np.full(B, ctx, np.int32), 0.25))
    assert np.array_equal(outs[0][0], outs[1][0]) and np.array_equal(outs[0][1], outs[1][1])


@pytest.mark.parametrize("mode", [1, 2])
def test_decode_rotary_matches_complex_rotation(mode):
    rng = np.random.default_rng(20 + mode)
    B, H, Hk, D, page, ctx, nq = 1, 4, 4, 16, 16, 30, 2
    rdim = 8
    pos = np.arange(64)[:, None]
    ang = pos * (10000.0 ** (-np.arange(rdim // 2) * 2.0 / rdim))[None, :]
    cos, sin = np.cos(ang).astype(np.float32), np.sin(ang).astype(np.float32)
    q = orc.round_to(rng.standard_normal((B, nq, H, D)), "f16")
    kseq = orc.round_to(rng.standard_normal((B, ctx, Hk, D)), "f16")
    vseq = orc.round_to(rng.standard_normal((B, ctx, Hk, D)), "f16")
    nk = orc.round_to(rng.standard_normal((B, nq, Hk, D)), "f16")
    nv = orc.round_to(rng.standard_normal((B, nq, Hk, D)), "f16")
    kc = kseq.reshape(2, 15, Hk, D)[:, :, :, :]
    kc = np.concatenate([kseq, np.zeros((B, 2, Hk, D), np.float32)], 1).reshape(2, 16, Hk, D)
    vc = np.concatenate([vseq, np.zeros((B, 2, Hk, D), np.float32)], 1).reshape(2, 16, Hk, D)
    bt = np.array([[0, 1]], dtype=np.int32)
    o, _ = orc.decode(q, kc, vc, bt, np.array([ctx], np.int32), 0.3, new_k=nk, new_v=nv,
                      rotary_cos=cos, rotary_sin=sin, rotary=mode, rotary_dim=rdim)

    def rot(x, p):  # x [..., D] at position p, rotate the first rdim dims as complex numbers
        x = x.astype(np.float64).copy()
        c = np.cos(ang[p]) + 1j * np.sin(ang[p])
        if mode == 1:
            z = (x[..., :rdim // 2] + 1j * x[..., rdim // 2:rdim]) * c
            x[..., :rdim // 2], x[..., rdim // 2:rdim] = z.real, z.imag
        else:
            z = (x[..., 0:rdim:2] + 1j * x[..., 1:rdim:2]) * c
            x[..., 0:rdim:2], x[..., 1:rdim:2] = z.real, z.imag
        return x
    qr = np.stack([rot(q[:, t], ctx + t) for t in range(nq)], 1)
    kr = np.concatenate([kseq.astype(np.float64), np.stack([rot(nk[:, t], ctx + t) for t in range(nq)], 1)], 1)
    vr = np.concatenate([vseq, nv], 1)
    fo, _ = orc.fwd(qr.transpose(0, 2, 1, 3), kr.transpose(0, 2, 1, 3), vr.transpose(0, 2, 1, 3), 0.3, True)
    assert np.abs(o - fo.transpose(0, 2, 1, 3)).max() < 2e-6


def test_combine_halves_equal_full():
    q, k, v = _rand((1, 4, 16, 32), 30), _rand((1, 4, 40, 32), 31), _rand((1, 4, 40, 32), 32)
    o1, l1 = orc.fwd(q, k[:, :, :25], v[:, :, :25], 0.2)
    o2, l2 = orc.fwd(q, k[:, :, 25:], v[:, :, 25:], 0.2)
    of, lf = orc.fwd(q, k, v, 0.2)
    op = np.stack([o1, o2]).transpose(0, 1, 3, 2, 4)   # [nsplit,B,S,H,D]
    lp = np.stack([l1, l2])                               # [nsplit,B,H,S]
    got = orc.combine(op, lp)
    assert np.abs(got - of.transpose(0, 2, 1, 3)).max() < 1e-6


def test_rel_rms_known_value():
    assert orc.rel_rms([3.0, 4.0], [3.0, 4.0]) == 0.0
    assert abs(orc.rel_rms([3.0, 4.0], [0.0, 5.0]) - math.sqrt(10) / 5) < 1e-12


def test_c_rounding_matches_numpy():
    import ctypes
    rng = np.random.default_rng(40)
    x = np.concatenate([rng.standard_normal(20000) * 10.0 ** rng.integers(-9, 6, 20000),
                        [65504.0, 65519.9, 65520.0, 1e-8, 3e-8, -6.1e-5, 2.0 ** -25, 0.0]]).astype(np.float32)
    for mode, ref in ((1, x.astype(np.float16).astype(np.float32)), (2, orc.round_bf16(x))):
        y = np.empty_like(x)
        orc.lib().oracle_round(x.ctypes.data_as(ctypes.c_void_p), y.ctypes.data_as(ctypes.c_void_p),
                               ctypes.c_size_t(x.size), mode)
        assert np.array_equal(y, ref), mode


# ----------------------------------------------------------------------------- dropout
# Random123's published known-answer vectors for philox4x32_10 (kat_vectors): counter, key,
# expected output words.
PHILOX_KAT = [
    ((0, 0, 0, 0), (0, 0), (0x6627E8D5, 0xE169C58D, 0xBC57AC4C, 0x9B00DBD8)),
    ((0xFFFFFFFF,) * 4, (0xFFFFFFFF,) * 2, (0x408F276D, 0x41C83B0E, 0xA20BC7C6, 0x6D5451FD)),
    ((0x243F6A88, 0x85A308D3, 0x13198A2E, 0x03707344), (0xA4093822, 0x299F31D0),
     (0xD16CFE09, 0x94FDCCEB, 0x5001E420, 0x24126EA1)),
]


@pytest.mark.parametrize("ctr,key,want", PHILOX_KAT)
def test_philox_known_answers(ctr, key, want):
    assert orc.philox4x32_10(ctr, key) == want


def test_dropout_mask_matches_reference_replica():
    """Every multiplier equals the reference's hdrop (kernels/backward.hip:530-537) bit for bit,
    over seeds that use both key words and indices past 2^32 (both counter words)."""
    ref = _need_ref(orc.ref_drop_lib())
    for seed in (0, 777, (1 << 63) - 1, 0x123456789ABCDEF0):
        for p in (0.1, 0.2, 0.5, 0.9):
            H, SQ, SK = 3, 7, 41
            z = orc.keep_mask(seed, p, H, SQ, SK)
            pf = float(np.float32(p))
            ks = float(np.float32(1.0) / (np.float32(1.0) - np.float32(pf)))
            want = np.array([ref.ref_drop_mul(seed, i, pf, ks) for i in range(H * SQ * SK)])
            assert np.array_equal(z.reshape(-1) > 0, want > 0), (seed, p)
            assert np.allclose(z.reshape(-1)[want > 0], ks, rtol=1e-6)
        for base in (1 << 32, (1 << 40) + 12345):  # idx high word in play
            for i in range(base - 20, base + 20):
                assert (orc.oracle_drop_mul(seed, i, 0.3) > 0) == (ref.ref_drop_mul(seed, i, 0.3, 1.0) > 0)


def test_dropout_keep_rate():
    for p in (0.1, 0.5):
        z = orc.keep_mask(11, p, 4, 64, 256)
        n = z.size
        kept = (z > 0).mean()
        assert abs(kept - (1 - p)) <= 5 * math.sqrt(p * (1 - p) / n)
        assert np.allclose(z[z > 0], 1.0 / (1.0 - np.float32(p)))


def test_dropout_forward_reads_back_the_mask():
    """V = identity (one-hot rows): O[b,h,i,j] = z[h,i,j] * P[b,h,i,j] with P the undropped
    softmax, so the forward with dropout returns the mask times the probabilities; the
    multiplier has no batch term (both batches see the same mask); the row sum (and LSE) is
    that of the undropped probabilities."""
    B, H, SQ, SK = 2, 3, 9, 16
    rng = np.random.default_rng(5)
    q = rng.standard_normal((B, H, SQ, SK)).astype(np.float32)
    k = rng.standard_normal((B, H, SK, SK)).astype(np.float32)
    v = np.broadcast_to(np.eye(SK, dtype=np.float32), (B, H, SK, SK)).copy()
    seed, p = 99, 0.3
    o, lse = orc.fwd(q, k, v, 0.25, False, dropout_p=p, seed=seed)
    o0, lse0 = orc.fwd(q, k, v, 0.25, False)
    z = orc.keep_mask(seed, float(np.float32(p)), H, SQ, SK)
    assert np.allclose(o, z[None] * o0, rtol=1e-6, atol=1e-7)
    assert np.array_equal(lse, lse0)
    assert ((o == 0) == (z[None] == 0)).all()


def test_dropout_backward_finite_differences():
    B, H, Hk, SQ, SK, D = 1, 4, 2, 7, 12, 8
    rng = np.random.default_rng(6)
    q = rng.standard_normal((B, H, SQ, D)).astype(np.float32)
    k = rng.standard_normal((B, Hk, SK, D)).astype(np.float32)
    v = rng.standard_normal((B, Hk, SK, D)).astype(np.float32)
    do = rng.standard_normal((B, H, SQ, D)).astype(np.float32)
    seed, p, scale = 1234, 0.25, np.float32(0.4)
    for causal, sc in ((True, 0.0), (False, 4.0)):
        dq, dk, dv = orc.bwd(q, k, v, do, scale, causal, -1, -1, sc, dropout_p=p, seed=seed)
        z = orc.keep_mask(seed, p, H, SQ, SK)
        loss = lambda q_, k_, v_: (_np_attention(q_, k_, v_, float(scale), causal, softcap=sc, z=z) * do).sum()
        eps = 1e-3
        base = [a.astype(np.float64) for a in (q, k, v)]
        for pos, g in enumerate((dq, dk, dv)):
            for idx in [tuple(rng.integers(0, s_) for s_ in base[pos].shape) for _ in range(8)]:
                ap = [a.copy() for a in base]
                am = [a.copy() for a in base]
                ap[pos][idx] += eps
                am[pos][idx] -= eps
                fd = (loss(*ap) - loss(*am)) / (2 * eps)
                assert abs(fd - g[idx]) <= 1e-5 + 1e-4 * abs(fd), ("qkv"[pos], idx, fd, g[idx])


# ----------------------------------------------------------------------------- rounding model
# oracle.bwd(..., model=dt) is the backward in the roundings of a 16-bit-operand kernel (D from
# the stored O, z*P and dS rounded to the dtype); the GPU gradient tests raise a case's bound to
# 1.5x its distance from the exact gradients (its floor) when that floor is large. The checks
# below pin the model by what the mathematics fixes, so a misplaced or missing rounding, a D
# taken from the wrong O, or a dropped term changes a result here.
def _np_probs(q, k, scale, causal, wl=-1, wr=-1, softcap=0.0):
    """fp64 softmax probabilities P [B,H,SQ,SK] and the softcap derivative of the logit
    (1 - tanh^2, or 1), textbook numpy, GQA by head repetition."""
    H, Hk = q.shape[1], k.shape[1]
    kk = np.repeat(k, H // Hk, axis=1).astype(np.float64)
    x = np.einsum("bhid,bhjd->bhij", q.astype(np.float64), kk) * scale
    deriv = np.ones_like(x)
    if softcap > 0:
        t = np.tanh(x / softcap)
        x, deriv = softcap * t, 1.0 - t * t
    SQ, SK = q.shape[2], k.shape[2]
    i, j, d = np.arange(SQ)[:, None], np.arange(SK)[None, :], SK - SQ
    m = np.zeros((SQ, SK), dtype=bool)
    if causal:
        m |= j > i + d
    if wl >= 0:
        m |= j < i + d - wl
    if wr >= 0:
        m |= j > i + d + wr
    x = np.where(m, -np.inf, x)
    p = np.exp(x - x.max(-1, keepdims=True))
    return p / p.sum(-1, keepdims=True), deriv


def _rounded(shapes, seed, dt):
    rng = np.random.default_rng(seed)
    return [orc.round_to(rng.standard_normal(s), dt) for s in shapes]


@pytest.mark.parametrize("dt", ["f16", "bf16"])
def test_bwd_model_single_visible_key_is_exact(dt):
    """Window (0, 0) leaves each query one key: P = 1, O = that V row (already in the dtype, so
    rounding O changes nothing), dP = dO.V = D, so dS = 0 exactly and dV_j = the sum of dO over
    the query heads that see key j. The model must reproduce the exact gradients bit for bit; a
    rounding of dP but not of D (or of D's O before the sum differently) would leave dS != 0."""
    B, H, Hk, S, D = 1, 4, 2, 20, 16
    q, k, v, do = _rounded(((B, H, S, D), (B, Hk, S, D), (B, Hk, S, D), (B, H, S, D)), 11, dt)
    ex = orc.bwd(q, k, v, do, 0.25, False, 0, 0)
    md = orc.bwd(q, k, v, do, 0.25, False, 0, 0, model=dt)
    for a, b in zip(ex, md):
        assert np.array_equal(a, b)
    assert not md[0].any() and not md[1].any()
    want_dv = do.astype(np.float64).reshape(B, Hk, H // Hk, S, D).sum(2)
    assert np.array_equal(md[2], want_dv)


@pytest.mark.parametrize("model", [None, "f16", "bf16"])
def test_bwd_model_stored_o_shifts_ds(model):
    """D = rowsum(O*dO) comes from the stored O: replacing O by O + delta changes D_i by
    dO_i.delta_i, hence dS_ij by -P_ij*(dO_i.delta_i)*deriv_ij, dQ_i by scale*sum_j dS_ij K_j and
    dK_j by scale*sum_i dS_ij Q_i (GQA heads summed), and leaves dV unchanged. In exact
    arithmetic this holds to fp64 rounding; in a dtype model each dS is rounded, so the shift
    holds to a few unit roundoffs. Softcap and a causal window make deriv and the mask matter."""
    B, H, Hk, SQ, SK, D = 1, 4, 2, 24, 40, 16
    scale, sc, causal, wl = float(np.float32(0.3)), 4.0, True, 9   # the oracle takes fp32 scalars
    dt = model or "f16"
    q, k, v, do = _rounded(((B, H, SQ, D), (B, Hk, SK, D), (B, Hk, SK, D), (B, H, SQ, D)), 12, dt)
    o1, _ = orc.fwd(q, k, v, scale, causal, wl, -1, sc)
    rng = np.random.default_rng(13)
    o2 = (o1 + rng.standard_normal(o1.shape)).astype(np.float32)
    delta = o2.astype(np.float64) - o1.astype(np.float64)
    g1 = orc.bwd(q, k, v, do, scale, causal, wl, -1, sc, model=model, stored_o=o1)
    g2 = orc.bwd(q, k, v, do, scale, causal, wl, -1, sc, model=model, stored_o=o2)
    p, deriv = _np_probs(q, k, scale, causal, wl, -1, sc)
    dD = (do.astype(np.float64) * delta).sum(-1)                 # [B,H,SQ]
    dds = -p * dD[..., None] * deriv                              # [B,H,SQ,SK]
    kk = np.repeat(k, H // Hk, axis=1).astype(np.float64)
    want_dq = scale * np.einsum("bhij,bhjd->bhid", dds, kk)
    want_dk = (scale * np.einsum("bhij,bhid->bhjd", dds, q.astype(np.float64))
               ).reshape(B, Hk, H // Hk, SK, D).sum(2)
    assert np.array_equal(g1[2], g2[2])
    tol = 1e-9 if model is None else 2 * {"f16": 2.0 ** -11, "bf16": 2.0 ** -8}[dt]  # measured 0.5u
    assert orc.rel_rms(g2[0] - g1[0], want_dq) <= tol
    assert orc.rel_rms(g2[1] - g1[1], want_dk) <= tol
    if model is None:   # D from the forward's own O: the stored-O form equals the exact gradients
        ex = orc.bwd(q, k, v, do, scale, causal, wl, -1, sc)
        for a, b in zip(g1, ex):
            assert orc.rel_rms(a, b) <= 1e-6


@pytest.mark.parametrize("causal,wl,wr,sc", [(False, -1, -1, 0.0), (True, -1, -1, 5.0),
                                             (False, 6, 3, 0.0)])
def test_bwd_model_floor_scales_with_unit_roundoff(causal, wl, wr, sc):
    """The model differs from the exact gradients only by roundings to the dtype, so its
    distance (the floor) is a fraction of the unit roundoff u (2^-11 fp16, 2^-8 bf16) and the
    bf16 floor is about 8x the fp16 one on the same inputs. A dropped term would make the floor
    O(1); a rounding to the wrong dtype would make the ratio 1 (or 1/8); no rounding at all
    would make the floor ~1e-16."""
    B, H, Hk, SQ, SK, D = 1, 4, 2, 48, 64, 32
    q, k, v, do = _rounded(((B, H, SQ, D), (B, Hk, SK, D), (B, Hk, SK, D), (B, H, SQ, D)), 14, "f16")
    ex = orc.bwd(q, k, v, do, 0.3, causal, wl, wr, sc)
    floor = {}
    for dt, u in (("f16", 2.0 ** -11), ("bf16", 2.0 ** -8)):
        md = orc.bwd(q, k, v, do, 0.3, causal, wl, wr, sc, model=dt)
        floor[dt] = [orc.rel_rms(a, b) for a, b in zip(md, ex)]
        for f in floor[dt]:
            assert 0.2 * u <= f <= 1.5 * u, (dt, floor[dt])
    for f16, bf16 in zip(floor["f16"], floor["bf16"]):
        assert 5.0 <= bf16 / f16 <= 12.0, (floor["f16"], floor["bf16"])
