"""Paged-KV decode parity on the GPU: fable_attn_dec (through fable_attn._C.dec, the C-ABI)
vs the fp64 decode oracle on identical seeded inputs.

Cases follow the reference decode gate (kernels/fa_decode_gate.inc:159-191: GQA, rotary
neox/interleaved, window, append, leftpad, softcap, alibi, several new tokens, head dims) with
random page permutations, ragged batches, several page sizes and forced split counts, plus the
full BASELINE.json configs[3] shape (batch 16, ctx 32768, page 256) checked on sampled
sequences. Bounds: rel_rms <= 5e-4 (fp16) / 4e-3 (bf16) / 1e-5 (fp32, the reference forward
gate's fp32 bound), LSE within 1e-3 absolute.
"""
import numpy as np
import pytest

from oracle import oracle as orc
from tests.helpers import LSE_ABS, TOL, gen, log_errors, to_dev, to_np

pytestmark = pytest.mark.gpu

# name, HD, NH, gqa, ctx(list per batch), window, rotary, append, leftpad, nq, softcap, alibi, page
CASES = [
    ("paged GQA4 ctx333", 128, 32, 4, [333], -1, 0, False, 0, 1, 0.0, False, 16),
    ("paged GQA1 ctx200", 128, 8, 1, [200], -1, 0, False, 0, 1, 0.0, False, 16),
    ("rotary neox ctx256", 128, 32, 4, [256], -1, 1, False, 0, 1, 0.0, False, 16),
    ("rotary interleaved ctx256", 128, 32, 4, [256], -1, 2, False, 0, 1, 0.0, False, 16),
    ("window 64 ctx500", 128, 32, 4, [500], 64, 0, False, 0, 1, 0.0, False, 16),
    ("append+rotary ctx257", 128, 32, 4, [257], -1, 1, True, 0, 1, 0.0, False, 16),
    ("leftpad 100 ctx400", 128, 32, 4, [400], -1, 0, False, 100, 1, 0.0, False, 16),
    ("leftpad 37 GQA1 ctx333", 128, 8, 1, [333], -1, 0, False, 37, 1, 0.0, False, 16),
    ("leftpad+window ctx500", 128, 32, 4, [500], 64, 0, False, 50, 1, 0.0, False, 16),
    ("softcap 30 ctx333", 128, 32, 4, [333], -1, 0, False, 0, 1, 30.0, False, 16),
    ("softcap 50 append", 128, 32, 4, [257], -1, 0, True, 0, 1, 50.0, False, 16),
    ("alibi ctx333", 128, 32, 4, [333], -1, 0, False, 0, 1, 0.0, True, 16),
    ("alibi+window ctx500", 128, 32, 4, [500], 128, 0, False, 0, 1, 0.0, True, 16),
    ("nq4 no append", 128, 32, 4, [300], -1, 0, False, 0, 4, 0.0, False, 16),
    ("nq4 append", 128, 32, 4, [300], -1, 0, True, 0, 4, 0.0, False, 16),
    ("nq8 append+rotary", 128, 32, 4, [257], -1, 1, True, 0, 8, 0.0, False, 16),
    ("nq5 GQA1 window append", 128, 8, 1, [400], 96, 0, True, 0, 5, 0.0, False, 16),
    ("nq3 softcap+alibi append", 128, 32, 4, [300], -1, 0, True, 0, 3, 30.0, True, 16),
    ("HD64 ctx300", 64, 32, 4, [300], -1, 0, False, 0, 1, 0.0, False, 16),
    ("HD256 ctx300", 256, 8, 4, [300], -1, 0, False, 0, 1, 0.0, False, 16),
    ("GQA8 batch3 ragged page64", 128, 64, 8, [1000, 37, 513], -1, 0, False, 0, 1, 0.0, False, 64),
    ("GQA32 two head groups", 128, 64, 32, [700, 300], -1, 0, False, 0, 1, 0.0, False, 32),
    ("batch4 page256 append", 128, 32, 4, [4000, 255, 256, 1], -1, 1, True, 0, 1, 0.0, False, 256),
    ("empty context", 128, 32, 4, [0, 50], -1, 0, False, 0, 1, 0.0, False, 16),
    # pages under 16 rows (the per-lane block-table path)
    ("page8 window GQA2 batch2", 128, 16, 2, [300, 45], 70, 0, False, 0, 1, 0.0, False, 8),
    ("page4 leftpad HD64", 64, 8, 4, [200], -1, 0, False, 13, 1, 0.0, False, 4),
    ("page1 append+rotary nq2", 128, 8, 4, [40, 3], -1, 1, True, 0, 2, 0.0, False, 1),
]


def make_case(case, dt, seed=0, shuffle=True):
    name, HD, NH, gqa, ctxs, window, rotary, append, leftpad, nq, sc, alibi, page = case
    B, Hk = len(ctxs), NH // gqa
    rng = np.random.default_rng(seed + 17)
    total = [c + (nq if append else 0) for c in ctxs]
    maxb = max(1, max((t + page - 1) // page for t in total))
    nblk = B * maxb + 3
    perm = rng.permutation(nblk) if shuffle else np.arange(nblk)
    bt = perm[:B * maxb].reshape(B, maxb).astype(np.int32)
    kc = gen((nblk, page, Hk, HD), seed + 1, dt)
    vc = gen((nblk, page, Hk, HD), seed + 2, dt)
    q = gen((B, nq, NH, HD), seed + 3, dt)
    nk = gen((B, nq, Hk, HD), seed + 4, dt) if append else None
    nv = gen((B, nq, Hk, HD), seed + 5, dt) if append else None
    seqro = max(total) + 16
    ang = np.arange(seqro)[:, None] * (10000.0 ** (-2.0 * np.arange(HD // 2) / HD))[None, :]
    cos = np.cos(ang).astype(np.float32) if rotary else None
    sin = np.sin(ang).astype(np.float32) if rotary else None
    al = (-np.float32(2.0) ** (-(8.0 * np.arange(1, NH + 1) / NH))).astype(np.float32) if alibi else None
    lp = np.full(B, leftpad, np.int32) if leftpad else None
    return dict(q=q, kc=kc, vc=vc, bt=bt, ctx=np.array(ctxs, np.int32), nk=nk, nv=nv, cos=cos,
                sin=sin, rotary=rotary, window=window, lp=lp, sc=sc, al=al, scale=HD ** -0.5)


def run_kernel(c, dt, num_splits=0, return_lse=True):
    import torch

    from fable_attn import _C
    dev = lambda a: to_dev(a, dt) if a is not None else None
    kc, vc = dev(c["kc"]), dev(c["vc"])
    f32 = lambda a: torch.from_numpy(a).cuda() if a is not None else None
    out, lse = _C.dec(dev(c["q"]), kc, vc, torch.from_numpy(c["bt"]).cuda(),
                      torch.from_numpy(c["ctx"]).cuda(), dev(c["nk"]), dev(c["nv"]),
                      f32(c["cos"]), f32(c["sin"]), c["rotary"] == 2, c["scale"], c["window"],
                      num_splits, f32(c["lp"]), return_lse, c["sc"], f32(c["al"]), 0, None)
    torch.cuda.synchronize()
    return to_np(out), (to_np(lse) if return_lse else None), kc, vc


def run_oracle(c, dt):
    """The appended keys are rounded to the cache dtype after rotation, as storing them does."""
    return orc.decode(c["q"], c["kc"], c["vc"], c["bt"], c["ctx"], c["scale"], new_k=c["nk"],
                      new_v=c["nv"], rotary_cos=c["cos"], rotary_sin=c["sin"],
                      rotary=c["rotary"], leftpad=c["lp"], window=c["window"], softcap=c["sc"],
                      alibi=c["al"], append_dtype=dt)


def check(o, l, o_ref, l_ref, dt, case="decode"):
    rel = orc.rel_rms(o, o_ref)
    fin = np.isfinite(l_ref)
    err = float(np.abs(l[fin] - l_ref[fin]).max()) if fin.any() else 0.0
    log_errors("decode", case, dt, o=rel, lse=err)
    assert np.isfinite(o).all()
    assert rel <= TOL[dt], f"rel_rms {rel:.3e} > {TOL[dt]}"
    assert np.array_equal(np.isneginf(l), np.isneginf(l_ref))
    assert err <= LSE_ABS, f"LSE err {err:.3e}"


@pytest.mark.parametrize("dt", ["f16", "bf16", "f32"])
@pytest.mark.parametrize("case", CASES, ids=[c[0] for c in CASES])
def test_decode_parity(case, dt):
    print(f"[decode] {case[0]} {dt}", flush=True)
    c = make_case(case, dt)
    o, l, kc, vc = run_kernel(c, dt)
    o_ref, l_ref = run_oracle(c, dt)
    check(o, l, o_ref, l_ref, dt, case[0])
    if c["nk"] is not None:
        # the appended V rows were written into the cache at positions ctx..ctx+nq-1
        vcn = to_np(vc)
        page = c["kc"].shape[1]
        for b, cx in enumerate(c["ctx"]):
            for t in range(c["q"].shape[1]):
                pos = cx + t
                blk = c["bt"][b, pos // page]
                assert np.array_equal(vcn[blk, pos % page], c["nv"][b, t])


# head dims other than 64/128/256: fp16/bf16 kernels of every width that is a multiple of 32
# from 64 up, fp32 kernels of width 64, 128 and 256, zero columns past the head dim (rows in the
# cache are the real head dim long), with append and rotary
DIM_CASES = [
    ("HD32 append+rotary", 32, 8, 4, [70, 200], -1, 1, True, 0, 2, 0.0, False, 16),
    ("HD80 append+rotary interleaved", 80, 16, 4, [300], -1, 2, True, 0, 1, 0.0, False, 16),
    ("HD96 GQA8 window", 96, 16, 8, [500, 77], 64, 0, False, 0, 1, 0.0, False, 32),
    ("HD112 softcap append nq3", 112, 8, 2, [200], -1, 0, True, 0, 3, 30.0, False, 16),
    ("HD160 append", 160, 8, 4, [300], -1, 1, True, 0, 1, 0.0, False, 16),
    ("HD192 leftpad alibi", 192, 8, 8, [400], -1, 0, False, 37, 1, 0.0, True, 16),
    ("HD200 append rotary", 200, 4, 2, [130], -1, 1, True, 0, 2, 0.0, False, 16),
    ("HD224 GQA4 window", 224, 8, 4, [260, 33], 100, 0, False, 0, 1, 0.0, False, 16),
    ("HD136 page8 append", 136, 4, 2, [90], -1, 0, True, 0, 1, 0.0, False, 8),
    ("HD88 page4 softcap", 88, 8, 4, [150], -1, 0, False, 0, 2, 20.0, False, 4),
]


@pytest.mark.parametrize("dt", ["f16", "bf16", "f32"])
@pytest.mark.parametrize("case", DIM_CASES, ids=[c[0] for c in DIM_CASES])
def test_decode_head_dims(case, dt):
    test_decode_parity(case, dt)


@pytest.mark.parametrize("nsplit", [1, 3, 16, 64])
def test_decode_split_counts_agree(nsplit):
    c = make_case(("splits", 128, 32, 4, [3000, 1111], -1, 0, False, 0, 1, 0.0, False, 64), "f16")
    o, l, _, _ = run_kernel(c, "f16", num_splits=nsplit)
    o_ref, l_ref = run_oracle(c, "f16")
    check(o, l, o_ref, l_ref, "f16", f"nsplit {nsplit}")


def test_decode_page_permutation_bitwise():
    case = ("perm", 128, 32, 4, [2000, 900], -1, 0, False, 0, 1, 0.0, False, 32)
    c1 = make_case(case, "f16", seed=3, shuffle=False)
    c2 = dict(c1)
    rng = np.random.default_rng(99)
    nblk = c1["kc"].shape[0]
    perm = rng.permutation(nblk)            # physical page i moves to slot perm[i]
    kc2 = np.empty_like(c1["kc"])
    vc2 = np.empty_like(c1["vc"])
    kc2[perm] = c1["kc"]
    vc2[perm] = c1["vc"]
    c2.update(kc=kc2, vc=vc2, bt=perm[c1["bt"]].astype(np.int32))
    o1, l1, _, _ = run_kernel(c1, "f16", num_splits=8)
    o2, l2, _, _ = run_kernel(c2, "f16", num_splits=8)
    assert np.array_equal(o1, o2) and np.array_equal(l1, l2)


def test_decode_full_config_sampled():
    """BASELINE.json configs[3] at full size (batch 16, 32/8 heads, D=128, ctx 32768, page 256,
    block_table a seeded permutation); the oracle checks sequences 0, 7 and 15 on their own
    pages."""
    import torch

    from fable_attn import flash_attn_with_kvcache
    batch, Hq, Hk, D, ctx, page = 16, 32, 8, 128, 32768, 256
    nblk = batch * ctx // page
    g = torch.Generator(device="cuda").manual_seed(0)
    kc = torch.randn(nblk, page, Hk, D, device="cuda", dtype=torch.float16, generator=g)
    vc = torch.randn(nblk, page, Hk, D, device="cuda", dtype=torch.float16, generator=g)
    q = torch.randn(batch, 1, Hq, D, device="cuda", dtype=torch.float16, generator=g)
    bt = torch.randperm(nblk, generator=torch.Generator().manual_seed(0)).view(batch, ctx // page).int().cuda()
    cs = torch.full((batch,), ctx, dtype=torch.int32, device="cuda")
    out, lse = flash_attn_with_kvcache(q, kc, vc, cache_seqlens=cs, block_table=bt,
                                       return_softmax_lse=True)
    torch.cuda.synchronize()
    for b in (0, 7, 15):
        pages = bt[b].long()
        kb = kc[pages].float().cpu().numpy()
        vb = vc[pages].float().cpu().numpy()
        tb = np.arange(ctx // page, dtype=np.int32)[None]
        o_ref, l_ref = orc.decode(q[b:b + 1].float().cpu().numpy(), kb, vb, tb,
                                  np.array([ctx], np.int32), D ** -0.5)
        check(to_np(out[b:b + 1]), to_np(lse[b:b + 1]).transpose(0, 2, 1), o_ref, l_ref, "f16",
              f"C4 full size sequence {b}")
