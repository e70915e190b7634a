"""The reference-layout launchers on the GPU: fa_forward_launch, fable_attn_backward_launch and
fa_decode_launch called through ctypes with structs laid out exactly as the reference's
package/csrc/fa_iface.h:9-63, filled the way the reference's glue fills them
(package/csrc/dispatch.cpp:35-80, 83-111, 162-231: one forward call per batch element with
batch-offset pointers and LSE [H][SQ], dense backward with dsum, paged decode with scratch),
against the fp64 oracle at the BASELINE.json tolerances."""
import ctypes
import math

import numpy as np
import pytest

from oracle import oracle as orc
from tests.helpers import LSE_ABS, TOL, gen, lse_err, log_errors, to_dev, to_np

pytestmark = pytest.mark.gpu

GRAD_TOL = {"f16": 5e-4, "bf16": 4e-3}


def _stream():
    import torch
    return ctypes.c_void_p(torch.cuda.current_stream().cuda_stream)


def _rs(t, lib):
    return lib.RefStrides(*t.stride()[:3])


@pytest.mark.parametrize("dt", ["f16", "bf16"])
def test_reference_forward_and_backward_layout(dt):
    import torch

    from fable_attn import _lib
    lib = _lib.load()
    code = {"f16": 0, "bf16": 1}[dt]
    B, H, Hk, SQ, SK, D = 2, 8, 2, 200, 200, 128
    q, k, v, do = (gen(s, i + 40, dt) for i, s in enumerate(
        [(B, H, SQ, D), (B, Hk, SK, D), (B, Hk, SK, D), (B, H, SQ, D)]))
    scale = 1.0 / math.sqrt(D)
    view = lambda a: to_dev(a, dt).transpose(1, 2).contiguous().transpose(1, 2)
    qd, kd, vd, dod = view(q), view(k), view(v), view(do)
    out = torch.empty((B, SQ, H, D), dtype=qd.dtype, device="cuda").transpose(1, 2)
    lse = torch.empty((B, H, SQ), dtype=torch.float32, device="cuda")
    esz = qd.element_size()
    print(f"[ref-abi] forward {dt}", flush=True)
    for b in range(B):  # dispatch.cpp:61-78: one launch per batch element
        p = _lib.RefFwdParams()
        p.Q = qd.data_ptr() + b * qd.stride(0) * esz
        p.K = kd.data_ptr() + b * kd.stride(0) * esz
        p.V = vd.data_ptr() + b * vd.stride(0) * esz
        p.O = out.data_ptr() + b * out.stride(0) * esz
        p.LSE = lse.data_ptr() + b * H * SQ * 4
        p.sQ, p.sK, p.sV, p.sO = _rs(qd, _lib), _rs(kd, _lib), _rs(vd, _lib), _rs(out, _lib)
        p.SQ, p.SK, p.HD, p.NH, p.gqa = SQ, SK, D, H, H // Hk
        p.scale, p.softcap, p.win_left, p.win_right, p.causal = scale, 0.0, -1, 0, 1
        p.batch = 1
        p.sc_q = p.sc_k = p.sc_v = 0.0     # reference: 0 => 1 (ignored here)
        assert lib.fa_forward_launch(p, code, _stream()) == 0, lib.fable_attn_last_error()
    torch.cuda.synchronize()
    o_ref, l_ref = orc.fwd(q, k, v, scale, True)
    e = orc.rel_rms(to_np(out), o_ref)
    le, inf_ok = lse_err(to_np(lse), l_ref)
    log_errors("ref_abi_fwd", "causal B2 GQA4 D128", dt, o=e, lse=le)
    assert e <= TOL[dt] and le <= LSE_ABS and inf_ok, (e, le)

    print(f"[ref-abi] backward {dt}", flush=True)
    dq, dk, dv = (torch.empty_like(x) for x in (qd, kd, vd))
    dsum = torch.empty((B, H, SQ), dtype=torch.float32, device="cuda")
    r = _lib.RefBwdParams()
    r.Q, r.K, r.V, r.O, r.dO = qd.data_ptr(), kd.data_ptr(), vd.data_ptr(), out.data_ptr(), dod.data_ptr()
    r.dQ, r.dK, r.dV = dq.data_ptr(), dk.data_ptr(), dv.data_ptr()
    r.lse, r.dsum = lse.data_ptr(), dsum.data_ptr()
    r.qs, r.ks, r.vs, r.os, r.dos = (_rs(t, _lib) for t in (qd, kd, vd, out, dod))
    r.dqs, r.dks, r.dvs = (_rs(t, _lib) for t in (dq, dk, dv))
    r.B, r.Hq, r.Hk, r.SQ, r.SK, r.D, r.gqa = B, H, Hk, SQ, SK, D, H // Hk
    r.scale, r.causal, r.win_left, r.win_right, r.keep_scale = scale, 1, -1, 0, 1.0
    r.shQ = r.shK = r.shV = r.shdO = 3   # the reference's bf16 shifts: ignored
    assert lib.fable_attn_backward_launch(r, code, _stream()) == 0, lib.fable_attn_last_error()
    torch.cuda.synchronize()
    ref = orc.bwd(q, k, v, do, scale, True)
    errs = {n: orc.rel_rms(to_np(g), rr) for n, g, rr in zip(("dq", "dk", "dv"), (dq, dk, dv), ref)}
    log_errors("ref_abi_bwd", "causal B2 GQA4 D128", dt, **errs)
    for n, e in errs.items():
        assert e <= GRAD_TOL[dt], f"{n} rel_rms {e:.3e}"


def test_reference_decode_layout():
    import torch

    from fable_attn import _lib
    lib = _lib.load()
    dt, B, H, Hk, D, page, ctx = "f16", 3, 32, 8, 128, 16, [333, 1, 200]
    maxb = (max(ctx) + page - 1) // page
    rng = np.random.default_rng(5)
    nblk = B * maxb + 2
    bt = rng.permutation(nblk)[:B * maxb].reshape(B, maxb).astype(np.int32)
    kc, vc = gen((nblk, page, Hk, D), 51, dt), gen((nblk, page, Hk, D), 52, dt)
    q = gen((B, 1, H, D), 53, dt)
    scale = D ** -0.5
    nsplit = 3
    qd, kcd, vcd = to_dev(q, dt), to_dev(kc, dt), to_dev(vc, dt)
    btd = torch.from_numpy(bt).cuda()
    ctxd = torch.tensor(ctx, dtype=torch.int32, device="cuda")
    o = torch.empty_like(qd)
    scratch = torch.empty(B * H * nsplit * (D + 2), dtype=torch.float32, device="cuda")
    lse = torch.empty((B, 1, H), dtype=torch.float32, device="cuda")
    p = _lib.RefDecParams()
    p.q, p.Kc, p.Vc, p.block_table = qd.data_ptr(), kcd.data_ptr(), vcd.data_ptr(), btd.data_ptr()
    p.o, p.scratch, p.ctx_len = o.data_ptr(), scratch.data_ptr(), ctxd.data_ptr()
    p.batch, p.NH, p.gqa, p.HD, p.page = B, H, H // Hk, D, page
    p.max_blocks, p.nsplit, p.window, p.scale = maxb, nsplit, -1, scale
    p.page_shift, p.page_mask, p.append = 99, 99, 1   # derived by the launcher: ignored
    p.sc_q = p.sc_k = p.sc_v = 1.0
    p.lse_out, p.nq = lse.data_ptr(), 1
    print("[ref-abi] decode", flush=True)
    assert lib.fa_decode_launch(p, 0, _stream(), None, None) == 0, lib.fable_attn_last_error()
    torch.cuda.synchronize()
    o_ref, l_ref = orc.decode(q, kc, vc, bt, np.array(ctx, np.int32), scale)
    e = orc.rel_rms(to_np(o), o_ref)
    le, inf_ok = lse_err(to_np(lse), l_ref)
    log_errors("ref_abi_dec", "paged GQA4 ragged", dt, o=e, lse=le)
    assert e <= TOL[dt] and le <= LSE_ABS and inf_ok, (e, le)
