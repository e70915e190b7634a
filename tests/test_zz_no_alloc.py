"""fable_attn_dec_noalloc through the C-ABI: the decode entry point that allocates nothing (its
split partials live in a fixed device array owned by the library) must give exactly what
fable_attn_dec gives with a caller-allocated scratch, on two calls in a row (the second with a
smaller input, so stale partials of the first would show), and must reject a call whose
partials exceed the array before any device work."""
import ctypes

import numpy as np
import pytest

from tests.helpers import gen, to_dev

pytestmark = pytest.mark.gpu


def _params(lib_mod, q, kc, vc, bt, ctx, out, scratch, nsplit, lse=None):
    p = lib_mod.FableDecParams()
    B, nq, H, D = q.shape
    p.q, p.Kc, p.Vc, p.block_table = q.data_ptr(), kc.data_ptr(), vc.data_ptr(), bt.data_ptr()
    p.o, p.ctx_len = out.data_ptr(), ctx.data_ptr()
    p.scratch = scratch.data_ptr() if scratch is not None else None
    p.batch, p.NH, p.gqa, p.HD, p.page = B, H, H // kc.shape[2], D, kc.shape[1]
    p.max_blocks, p.nsplit, p.window, p.scale = bt.shape[1], nsplit, -1, D ** -0.5
    p.lse_out = lse.data_ptr() if lse is not None else None
    p.nq = nq
    return p


def _case(B, H, Hk, D, page, ctxs, seed, dt="f16"):
    import torch
    maxb = max(1, max((c + page - 1) // page for c in ctxs))
    nblk = B * maxb + 1
    rng = np.random.default_rng(seed)
    bt = torch.from_numpy(rng.permutation(nblk)[:B * maxb].reshape(B, maxb).astype(np.int32)).cuda()
    kc, vc = to_dev(gen((nblk, page, Hk, D), seed + 1, dt), dt), to_dev(gen((nblk, page, Hk, D), seed + 2, dt), dt)
    q = to_dev(gen((B, 1, H, D), seed + 3, dt), dt)
    ctx = torch.tensor(ctxs, dtype=torch.int32, device="cuda")
    return q, kc, vc, bt, ctx


def test_noalloc_decode_matches_allocating_entry_point():
    import torch

    from fable_attn import _lib
    lib = _lib.load()
    st = ctypes.c_void_p(torch.cuda.current_stream().cuda_stream)
    # the larger call first, then a smaller one: the array keeps the first call's partials
    for B, H, Hk, D, page, ctxs, nsplit, seed in ((6, 32, 8, 128, 64, [3000, 17, 900, 2048, 1, 555], 8, 1),
                                                  (2, 16, 4, 64, 16, [40, 300], 3, 2)):
        print(f"[noalloc] B={B} H={H} D={D} nsplit={nsplit}", flush=True)
        q, kc, vc, bt, ctx = _case(B, H, Hk, D, page, ctxs, seed)
        out_a, out_b = torch.empty_like(q), torch.empty_like(q)
        lse_a = torch.empty((B, 1, H), dtype=torch.float32, device="cuda")
        lse_b = torch.empty_like(lse_a)
        scratch = torch.empty(B * H * nsplit * (D + 2), dtype=torch.float32, device="cuda")
        pa = _params(_lib, q, kc, vc, bt, ctx, out_a, scratch, nsplit, lse_a)
        assert lib.fable_attn_dec(pa, 0, st, None, None) == 0, lib.fable_attn_last_error()
        pb = _params(_lib, q, kc, vc, bt, ctx, out_b, None, nsplit, lse_b)
        assert lib.fable_attn_dec_noalloc(pb, 0, st, None, None) == 0, lib.fable_attn_last_error()
        torch.cuda.synchronize()
        assert torch.equal(out_a, out_b), "outputs differ from fable_attn_dec"
        assert torch.equal(lse_a, lse_b), "LSE differs from fable_attn_dec"
        assert torch.isfinite(out_b).all()


def test_noalloc_decode_rejects_oversized_partials():
    import torch

    from fable_attn import _lib
    lib = _lib.load()
    cap = lib.fable_attn_dec_noalloc_max_floats()
    assert cap == 4 << 20
    q, kc, vc, bt, ctx = _case(1, 8, 8, 128, 16, [32], 5)
    out = torch.zeros_like(q)
    st = ctypes.c_void_p(torch.cuda.current_stream().cuda_stream)
    # two splits: partials one batch element past the array (the tensors hold one element; the
    # size check rejects the call before anything is launched)
    p = _params(_lib, q, kc, vc, bt, ctx, out, None, 2)
    p.batch = cap // (8 * 2 * 130) + 1
    assert lib.fable_attn_dec_noalloc(p, 0, st, None, None) == 3
    assert b"exceed" in lib.fable_attn_last_error()
    # fp32 always combines through the array, one split included
    p = _params(_lib, q, kc, vc, bt, ctx, out, None, 1)
    p.batch = cap // (8 * 130) + 1
    assert lib.fable_attn_dec_noalloc(p, 2, st, None, None) == 3
    assert b"exceed" in lib.fable_attn_last_error()
    # a bad head count or split count names itself
    p = _params(_lib, q, kc, vc, bt, ctx, out, None, 1)
    p.NH = 0
    assert lib.fable_attn_dec_noalloc(p, 0, st, None, None) == 3
    assert b"NH=0" in lib.fable_attn_last_error()
    p = _params(_lib, q, kc, vc, bt, ctx, out, None, 0)
    assert lib.fable_attn_dec_noalloc(p, 0, st, None, None) == 3
    assert b"nsplit=0" in lib.fable_attn_last_error()
    torch.cuda.synchronize()
    assert torch.count_nonzero(out) == 0, "nothing may run after a rejected call"


def test_noalloc_single_split_has_no_size_limit():
    """One fp16 split writes the output from the partial kernel and never touches the array,
    so a call whose partials would exceed it runs, and equals fable_attn_dec (which needs no
    scratch either at one split)."""
    import torch

    from fable_attn import _lib
    lib = _lib.load()
    cap = lib.fable_attn_dec_noalloc_max_floats()
    B, H, Hk, D = 1040, 32, 8, 128
    assert B * H * (D + 2) > cap
    print(f"[noalloc] single split B={B}", flush=True)
    q, kc, vc, bt, ctx = _case(B, H, Hk, D, 16, [20] * B, 7)
    out_a, out_b = torch.empty_like(q), torch.empty_like(q)
    st = ctypes.c_void_p(torch.cuda.current_stream().cuda_stream)
    pa = _params(_lib, q, kc, vc, bt, ctx, out_a, None, 1)
    assert lib.fable_attn_dec(pa, 0, st, None, None) == 0, lib.fable_attn_last_error()
    pb = _params(_lib, q, kc, vc, bt, ctx, out_b, None, 1)
    assert lib.fable_attn_dec_noalloc(pb, 0, st, None, None) == 0, lib.fable_attn_last_error()
    torch.cuda.synchronize()
    assert torch.equal(out_a, out_b) and torch.isfinite(out_b).all()
    # with two splits fable_attn_dec needs its scratch
    pa = _params(_lib, q, kc, vc, bt, ctx, out_a, None, 2)
    assert lib.fable_attn_dec(pa, 0, st, None, None) == 3
    assert b"scratch" in lib.fable_attn_last_error()
