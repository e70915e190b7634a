"""flash_attn_combine (one HIP kernel, csrc/combine.hip) and return_attn_probs on the GPU.

- The combine kernel against the float64 oracle merge (oracle.combine, which restates
  flash_attn_interface.py:567-580), with empty splits (LSE -inf) and rows whose every split is
  empty (0 here; the reference's torch expression gives NaN there, a documented difference).
- The split-KV identity: attention over two key halves, merged by their LSEs, equals attention
  over all keys (the reference's own check, test_fable_attn.py:232-240), at the fp16 bound.
- return_attn_probs (flash_attn_interface.py:370-374): the probability matrix against the fp64
  oracle's softmax; every row that sees a key sums to one.
- The qv term and a value head dim below the score head dim (flash_attn_interface.py:160-191),
  forward and autograd backward, against the oracle on the concatenated problem.
"""
import numpy as np
import pytest

from oracle import oracle as orc
from tests.helpers import GTOL, LSE_ABS, TOL, gen, log_errors, lse_err, to_dev, to_np

pytestmark = pytest.mark.gpu

# nsplit, B, S, H, D, partial dtype, output dtype
CASES = [
    (1, 1, 5, 2, 64, "f32", "f32"),
    (2, 2, 7, 3, 128, "f32", "f32"),
    (3, 2, 7, 3, 128, "f32", "bf16"),
    (4, 1, 9, 4, 256, "f16", "f16"),
    (5, 2, 3, 2, 64, "bf16", "f32"),
]


@pytest.mark.parametrize("case", CASES, ids=lambda c: "ns{}_B{}_S{}_H{}_D{}_{}_to_{}".format(*c))
def test_combine_vs_oracle(case):
    import torch

    from fable_attn import flash_attn_combine
    from tests.helpers import torch_dtype
    ns, B, S, H, D, idt, odt = case
    print(f"[combine] {case}", flush=True)
    rng = np.random.default_rng(ns * 1000 + D)
    op = gen((ns, B, S, H, D), ns * 7 + D, idt)
    lp = (3.0 * rng.standard_normal((ns, B, H, S))).astype(np.float32)
    lp[0, 0, 0, 0] = -np.inf               # one empty split of a row
    empty = None
    if S > 1:
        lp[:, B - 1, H - 1, 1] = -np.inf   # a row with every split empty
        empty = (B - 1, 1, H - 1)
    got = flash_attn_combine(to_dev(op, idt), torch.from_numpy(lp).cuda(),
                             out_dtype=torch_dtype(odt))
    got = to_np(got)
    ref = orc.combine(op, lp)
    assert np.all(np.isfinite(got))
    rel = orc.rel_rms(got, ref)
    log_errors("combine", str(case), odt, o=rel)
    assert rel <= TOL[odt], f"rel_rms {rel:.3e} > {TOL[odt]}"
    if empty is not None:
        b, s, h = empty
        assert np.all(got[b, s, h] == 0.0), "a row whose every split is empty must be 0"


@pytest.mark.parametrize("causal", [False, True])
def test_combine_halves_equal_full(causal):
    """Two forward passes over the key halves (with their LSEs), merged by the combine kernel,
    against one pass over all keys and the fp64 oracle."""
    import torch

    from fable_attn import _C, flash_attn_combine
    B, SQ, SK, H, D, dt = 2, 192, 384, 4, 128, "f16"
    print(f"[combine-halves] causal={causal}", flush=True)
    q = gen((B, H, SQ, D), 11, dt)
    k = gen((B, H, SK, D), 12, dt)
    v = gen((B, H, SK, D), 13, dt)
    scale = D ** -0.5
    qd, kd, vd = to_dev(q, dt), to_dev(k, dt), to_dev(v, dt)
    wr = 0 if causal else -1
    parts = []
    for k0, k1 in ((0, SK // 2), (SK // 2, SK)):
        # causal (bottom-right): query i sees key j iff j <= i + SK - SQ. Every key of the
        # first half is below SK - SQ, so it runs unmasked; the second half, of length SQ, is
        # causal with its own alignment (delta 0), which is the same mask.
        c = causal and k1 == SK
        o, l = _C.fwd(qd, kd[:, :, k0:k1], vd[:, :, k0:k1], scale, c, -1, 0 if c else -1,
                      0.0, None, 0.0, 0)
        parts.append((o.transpose(1, 2).float(), l))
    op = torch.stack([p[0] for p in parts])            # [2, B, SQ, H, D]
    lp = torch.stack([p[1] for p in parts])            # [2, B, H, SQ]
    got = to_np(flash_attn_combine(op, lp, out_dtype=torch.float16)).transpose(0, 2, 1, 3)
    full, _ = _C.fwd(qd, kd, vd, scale, causal, -1, wr, 0.0, None, 0.0, 0)
    ref, _ = orc.fwd(q, k, v, scale, causal=causal, win_right=wr)
    assert SK // 2 - 1 < SK - SQ, "first half fully visible to every query"
    rel = orc.rel_rms(got, ref)
    assert rel <= TOL[dt], f"combined halves vs oracle rel_rms {rel:.3e}"
    rel_full = orc.rel_rms(got, to_np(full))
    assert rel_full <= TOL[dt], f"combined halves vs one pass rel_rms {rel_full:.3e}"


@pytest.mark.parametrize("causal,window", [(True, (-1, -1)), (False, (16, 8))])
def test_return_attn_probs(causal, window):
    import torch

    from fable_attn import flash_attn_func
    B, S, H, D, dt = 1, 96, 4, 64, "f16"
    print(f"[probs] causal={causal} window={window}", flush=True)
    q = gen((B, S, H, D), 21, dt)
    k = gen((B, S, H, D), 22, dt)
    v = gen((B, S, H, D), 23, dt)
    scale = D ** -0.5
    out, lse, probs = flash_attn_func(to_dev(q, dt), to_dev(k, dt), to_dev(v, dt), causal=causal,
                                      window_size=window, return_attn_probs=True)
    qh, kh, vh = (x.transpose(0, 2, 1, 3) for x in (q, k, v))
    wl, wr = window
    if causal:
        wr = 0
    ref_o, ref_lse = orc.fwd(qh, kh, vh, scale, causal=causal, win_left=wl, win_right=wr)
    # fp64 probabilities from the same scores and the oracle's LSE
    s = np.einsum("bhqd,bhkd->bhqk", qh.astype(np.float64), kh.astype(np.float64)) * scale
    i = np.arange(S)[:, None]
    j = np.arange(S)[None, :]
    vis = np.ones((S, S), dtype=bool)
    if causal:
        vis &= j <= i
    if wl >= 0:
        vis &= j >= i - wl
    if wr >= 0:
        vis &= j <= i + wr
    ref_p = np.where(vis, np.exp(s - ref_lse[..., None].astype(np.float64)), 0.0)
    got_p = to_np(probs)
    assert got_p.shape == (B, H, S, S)
    assert np.abs(got_p - ref_p).max() <= 2e-3
    sums = got_p.sum(-1)
    assert np.abs(sums - 1.0).max() <= 2e-3
    lerr, inf_ok = lse_err(to_np(lse), ref_lse)
    assert inf_ok and lerr <= LSE_ABS
    rel = orc.rel_rms(to_np(out).transpose(0, 2, 1, 3), ref_o)
    assert rel <= TOL[dt]


@pytest.mark.parametrize("kind", ["qv", "headdim_v"])
def test_qv_forward_backward(kind):
    """FA-3's qv term (S = q.k^T + qv.v^T, reference flash_attn_interface.py:160-191) and a value
    head dim below the score head dim, through flash_attn_func and autograd, against the fp64
    oracle on the concatenated problem [q | qv] . [k | v]^T with values [v | 0]; gradients split
    back (dv gets both its value and its key part)."""
    import torch

    from fable_attn import flash_attn_func
    from tests.helpers import torch_dtype
    B, S, H, D, dt = 1, 160, 4, 64, "f16"
    Dk = D if kind == "qv" else 2 * D         # score head dim of q and k
    print(f"[qv] {kind}", flush=True)
    q = gen((B, S, H, Dk), 31, dt)
    k = gen((B, S, H, Dk), 32, dt)
    v = gen((B, S, H, D), 33, dt)
    qv = gen((B, S, H, D), 34, dt) if kind == "qv" else None
    do = gen((B, S, H, D), 35, dt)
    scale = 0.1
    ts = [to_dev(x, dt).requires_grad_() for x in (q, k, v)]
    tqv = to_dev(qv, dt).requires_grad_() if qv is not None else None
    out = flash_attn_func(*ts, softmax_scale=scale, causal=True, qv=tqv)
    out.backward(to_dev(do, dt))
    # the concatenated fp64 problem
    z = np.zeros((B, S, H, D), dtype=np.float32)
    qc = np.concatenate([q, qv if qv is not None else z], -1)
    kc = np.concatenate([k, v], -1)
    vc = np.concatenate([v, np.zeros((B, S, H, qc.shape[-1] - D), np.float32)], -1)
    doc = np.concatenate([do, np.zeros_like(vc[..., D:])], -1)
    th = lambda x: np.ascontiguousarray(x.transpose(0, 2, 1, 3))
    ref_o, _ = orc.fwd(th(qc), th(kc), th(vc), scale, causal=True, win_right=0)
    args = (th(qc), th(kc), th(vc), th(doc), scale)
    grads = orc.bwd(*args, causal=True, win_right=0)
    grads_m = orc.bwd(*args, causal=True, win_right=0, model=dt)
    ref_o = ref_o[..., :D]
    rel = orc.rel_rms(to_np(out).transpose(0, 2, 1, 3), ref_o)
    assert rel <= TOL[dt], f"out rel_rms {rel:.3e}"
    split = lambda g: {"dq": g[0][..., :Dk], "dk": g[1][..., :Dk],
                       "dv": g[1][..., Dk:] + g[2][..., :D], "dqv": g[0][..., Dk:]}
    ref_g, mod_g = split(grads), split(grads_m)
    got_g = {"dq": ts[0].grad, "dk": ts[1].grad, "dv": ts[2].grad}
    if qv is not None:
        got_g["dqv"] = tqv.grad
    errs = {"o": rel}
    for name, g in got_g.items():
        gn = to_np(g).transpose(0, 2, 1, 3)
        errs[name] = orc.rel_rms(gn, ref_g[name])
        errs[name + "_model"] = orc.rel_rms(gn, mod_g[name])
    log_errors("qv", kind, dt, **errs)
    for name in got_g:
        assert errs[name] <= GTOL[dt], f"{name} rel_rms {errs[name]:.3e}"
