"""Forward parity on the GPU: HIP kernels (through the C-ABI via fable_attn._C) vs the fp64
oracle on identical seeded inputs.

Cases follow the reference forward gate (kernels/fa_forward_gate.inc:170-211: causal, GQA,
SQ != SK bottom-right, empty rows, windows, softcap, alibi, head dims, attention_chunk, varlen
+/- seqused) at the BASELINE.json tolerances: rel_rms <= 5e-4 (fp16) / 4e-3 (bf16), LSE within
1e-3 absolute, empty rows exactly O = 0 and LSE = -inf.
"""
import math

import numpy as np
import pytest

from oracle import oracle as orc
from tests.helpers import LSE_ABS, TOL, gen, log_errors, lse_err, to_dev, to_np

pytestmark = pytest.mark.gpu

# name, B, SQ, SK, D, H, gqa, causal, wl, wr, softcap, alibi, chunk
CASES = [
    ("C1 d64 full S1024 H8", 1, 1024, 1024, 64, 8, 1, False, -1, -1, 0.0, False, 0),
    ("d128 causal GQA4", 1, 256, 256, 128, 32, 4, True, -1, -1, 0.0, False, 0),
    ("d128 causal GQA1 B2", 2, 256, 256, 128, 8, 1, True, -1, -1, 0.0, False, 0),
    ("d128 full", 1, 192, 192, 128, 16, 4, False, -1, -1, 0.0, False, 0),
    ("d128 SQ<SK bottom-right", 1, 128, 320, 128, 16, 4, True, -1, -1, 0.0, False, 0),
    ("d128 SQ>SK empty rows", 1, 256, 64, 128, 16, 4, True, -1, -1, 0.0, False, 0),
    ("window (63,0)", 1, 256, 256, 128, 16, 4, True, 63, 0, 0.0, False, 0),
    ("window (32,32)", 1, 256, 256, 128, 16, 4, False, 32, 32, 0.0, False, 0),
    ("window (0,0) diagonal", 1, 256, 256, 128, 16, 4, False, 0, 0, 0.0, False, 0),
    ("window (0,-1)", 1, 256, 256, 128, 16, 4, False, 0, -1, 0.0, False, 0),
    ("window (16,48)", 1, 192, 192, 128, 16, 4, False, 16, 48, 0.0, False, 0),
    ("window (32,32) SQ<SK", 1, 128, 320, 128, 16, 4, False, 32, 32, 0.0, False, 0),
    ("softcap 30", 1, 200, 200, 128, 16, 4, True, -1, -1, 30.0, False, 0),
    ("alibi", 1, 200, 200, 128, 16, 4, True, -1, -1, 0.0, True, 0),
    # the 8-wave shape's four-stage K/V ring over one and three tiles
    ("alibi one tile", 1, 64, 64, 128, 16, 4, True, -1, -1, 0.0, True, 0),
    ("alibi SQ<SK three tiles", 1, 100, 150, 128, 16, 2, False, -1, -1, 0.0, True, 0),
    ("d64 causal ragged", 1, 200, 200, 64, 16, 4, True, -1, -1, 0.0, False, 0),
    ("d256 causal", 1, 160, 160, 256, 8, 4, True, -1, -1, 0.0, False, 0),
    ("d256 full SQ<SK", 1, 96, 200, 256, 8, 2, False, -1, -1, 0.0, False, 0),
    ("chunk 64 causal", 1, 256, 256, 128, 16, 4, True, -1, -1, 0.0, False, 64),
    ("chunk 100 causal", 1, 256, 256, 128, 16, 4, True, -1, -1, 0.0, False, 100),
    ("chunk 128 full", 1, 256, 256, 128, 16, 4, False, -1, -1, 0.0, False, 128),
    ("chunk 64 SQ<SK", 1, 128, 320, 128, 16, 4, True, -1, -1, 0.0, False, 64),
    ("d256 window+softcap (C5 features)", 1, 300, 300, 256, 16, 1, True, 64, 0, 30.0, False, 0),
    # workgroup shapes of the launcher: wide windows / chunks (>= 2048 keys) and alibi run on the
    # plain shape's feature kernel, narrow masks on the short shape, softcap on its own shape
    ("d128 wide window (2100,0)", 1, 2400, 2400, 128, 4, 1, True, 2100, 0, 0.0, False, 0),
    ("d64 wide window (2050,9) GQA", 1, 2300, 2300, 64, 4, 2, False, 2050, 9, 0.0, False, 0),
    ("d256 chunk 2048 causal", 1, 2200, 2200, 256, 2, 1, True, -1, -1, 0.0, False, 2048),
    ("d256 window (32,32) alibi SQ<SK", 1, 200, 230, 256, 8, 2, False, 32, 32, 0.0, True, 0),
    ("d256 window (40,0) SQ>SK empty rows", 1, 200, 120, 256, 8, 4, True, 40, 0, 0.0, False, 0),
    ("d256 window (300,0) softcap B2", 2, 700, 700, 256, 4, 2, True, 300, 0, 30.0, False, 0),
    # the one-wave loop's ordered PV/transform steps with both transforms, and on the 64-key
    # softcap shape (two 32-key blocks per tile)
    ("d256 causal softcap alibi", 1, 230, 230, 256, 8, 2, True, -1, -1, 30.0, True, 0),
    ("d256 causal softcap (64-key tiles)", 1, 330, 330, 256, 8, 2, True, -1, -1, 30.0, False, 0),
    ("d128 wide window + alibi", 1, 2300, 2300, 128, 4, 1, True, 2048, 0, 0.0, True, 0),
    ("d128 narrow window + softcap", 1, 300, 300, 128, 8, 2, True, 100, 0, 20.0, False, 0),
    ("d64 narrow window + alibi", 1, 300, 300, 64, 8, 1, False, 40, 40, 0.0, True, 0),
    # head dims other than 64/128/256: kernels of width 32, 96, 160, 192, 224, and dims that
    # are not multiples of 32 (zero columns inside the kernel); the 8-wave and 4-wave shapes
    # whose loaders leave threads idle in the last round (width 32 and 96)
    ("d32 causal", 1, 300, 300, 32, 8, 2, True, -1, -1, 0.0, False, 0),
    ("d16 full", 1, 200, 200, 16, 4, 1, False, -1, -1, 0.0, False, 0),
    ("d48 window (40,0)", 1, 250, 250, 48, 8, 4, True, 40, 0, 0.0, False, 0),
    ("d80 causal GQA", 1, 330, 330, 80, 16, 4, True, -1, -1, 0.0, False, 0),
    ("d96 full SQ<SK", 1, 160, 270, 96, 8, 2, False, -1, -1, 0.0, False, 0),
    ("d96 causal 8-wave grid", 2, 1100, 1100, 96, 16, 1, True, -1, -1, 0.0, False, 0),
    ("d112 softcap", 1, 200, 200, 112, 8, 1, True, -1, -1, 30.0, False, 0),
    ("d160 causal", 1, 200, 200, 160, 8, 2, True, -1, -1, 0.0, False, 0),
    ("d192 full alibi", 1, 150, 170, 192, 4, 1, False, -1, -1, 0.0, True, 0),
    ("d200 window (64,0) softcap", 1, 260, 260, 200, 4, 2, True, 64, 0, 20.0, False, 0),
    ("d224 causal chunk 96", 1, 230, 230, 224, 4, 1, True, -1, -1, 0.0, False, 96),
    ("d40 causal ragged", 1, 77, 77, 40, 4, 1, True, -1, -1, 0.0, False, 0),
]


def _alibi(H):
    return (-np.float32(2.0) ** (-(8.0 * np.arange(1, H + 1) / H))).astype(np.float32)


def run_case(case, dt, seed=0):
    import torch

    from fable_attn import _C
    name, B, SQ, SK, D, H, gqa, causal, wl, wr, sc, alibi, chunk = case
    Hk = H // gqa
    q = gen((B, H, SQ, D), seed + 1, dt)
    k = gen((B, Hk, SK, D), seed + 2, dt)
    v = gen((B, Hk, SK, D), seed + 3, dt)
    al = _alibi(H) if alibi else None
    scale = 1.0 / math.sqrt(D)
    o_ref, l_ref = orc.fwd(q, k, v, scale, causal, wl, wr, sc, al, chunk)
    # kernel: BSHD storage (the public API layout), [B,H,S,D] views
    qd = to_dev(q, dt).transpose(1, 2).contiguous().transpose(1, 2)
    kd = to_dev(k, dt).transpose(1, 2).contiguous().transpose(1, 2)
    vd = to_dev(v, dt).transpose(1, 2).contiguous().transpose(1, 2)
    ald = torch.from_numpy(al).cuda() if al is not None else None
    out, lse = _C.fwd(qd, kd, vd, scale, causal, wl, wr, sc, ald, 0.0, 0, chunk)
    torch.cuda.synchronize()
    return to_np(out), to_np(lse), o_ref, l_ref


@pytest.mark.parametrize("dt", ["f16", "bf16"])
@pytest.mark.parametrize("case", CASES, ids=[c[0] for c in CASES])
def test_forward_parity(case, dt):
    print(f"[fwd] {case[0]} {dt}", flush=True)
    o, l, o_ref, l_ref = run_case(case, dt)
    rel = orc.rel_rms(o, o_ref)
    lerr, inf_ok = lse_err(l, l_ref)
    log_errors("fwd", case[0], dt, o=rel, lse=lerr)
    empty = np.isneginf(l_ref)
    assert np.isfinite(o).all(), "non-finite output"
    assert rel <= TOL[dt], f"rel_rms {rel:.3e} > {TOL[dt]}"
    assert inf_ok, "empty-row LSE (-inf) pattern differs"
    assert lerr <= LSE_ABS, f"LSE abs err {lerr:.3e}"
    if empty.any():
        rows = np.broadcast_to(empty[..., None], o.shape)
        assert (o[rows] == 0).all(), "empty rows must be exactly zero"


def test_forward_deterministic():
    case = CASES[1]
    a = run_case(case, "f16", seed=5)
    b = run_case(case, "f16", seed=5)
    assert np.array_equal(a[0], b[0]) and np.array_equal(a[1], b[1])


def _varlen(dt, lens, used_q=None, used_k=None, D=128, H=8, gqa=4, causal=True, wl=-1, wr=-1,
            sc=0.0, seed=11):
    import torch

    from fable_attn import _C
    Hk = H // gqa
    tot = sum(lens)
    cu = np.concatenate([[0], np.cumsum(lens)]).astype(np.int32)
    q = gen((tot, H, D), seed + 1, dt)
    k = gen((tot, Hk, D), seed + 2, dt)
    v = gen((tot, Hk, D), seed + 3, dt)
    scale = 1.0 / math.sqrt(D)
    o_ref = np.zeros_like(q)
    l_ref = np.full((H, tot), -np.inf, dtype=np.float32)
    for i, L in enumerate(lens):
        lq = used_q[i] if used_q else L
        lk = used_k[i] if used_k else L
        a = int(cu[i])
        qs = q[a:a + lq].transpose(1, 0, 2)[None]
        ks = k[a:a + lk].transpose(1, 0, 2)[None]
        vs = v[a:a + lk].transpose(1, 0, 2)[None]
        o, l = orc.fwd(qs, ks, vs, scale, causal, wl, wr, sc)
        o_ref[a:a + lq] = o[0].transpose(1, 0, 2)
        l_ref[:, a:a + lq] = l[0]
    cut = torch.from_numpy(cu).cuda()
    uq = torch.tensor(used_q, dtype=torch.int32).cuda() if used_q else None
    uk = torch.tensor(used_k, dtype=torch.int32).cuda() if used_k else None
    out, lse = _C.fwd_varlen(to_dev(q, dt), to_dev(k, dt), to_dev(v, dt), cut, cut, max(lens),
                             max(lens), scale, causal, wl, wr, sc, None, 0.0, 0, 0, uq, uk,
                             return_lse=True)
    torch.cuda.synchronize()
    o, l = to_np(out), to_np(lse)
    if used_q:
        for i, L in enumerate(lens):   # rows past seqused_q are not part of the result
            a = int(cu[i])
            l[:, a + used_q[i]:a + L] = -np.inf
    return o, l, o_ref, l_ref


def _varlen_split_bytes(lens, H, gqa, D, causal, dt):
    """fable_attn_fwd_ws_bytes of a packed varlen call (a query: the sequence table is not read)."""
    import ctypes

    from fable_attn import _C, _lib
    tot = sum(lens)
    p = _lib.FableFwdParams()
    p.sQ = _lib.Strides(0, D, H * D)
    p.sK = p.sV = _lib.Strides(0, D, H // gqa * D)
    p.sO = p.sQ
    p.SQ, p.SK, p.HD, p.NH, p.gqa = max(lens), max(lens), D, H, gqa
    p.scale, p.causal, p.win_left, p.win_right = D ** -0.5, int(causal), -1, -1
    p.cu_q = p.cu_k = ctypes.c_void_p(16)
    p.batch, p.lse_sb, p.lse_sh = len(lens), 0, tot
    return _C._L.fable_attn_fwd_ws_bytes(p, 0 if dt == "f16" else 1)


@pytest.mark.parametrize("dt", ["f16", "bf16"])
@pytest.mark.parametrize("kind", ["plain", "seqused", "window_softcap_d256", "split", "split_seqused",
                                  "split_full_d128", "split_ragged", "short_rows_d128", "short_rows_d64"])
def test_varlen_parity(kind, dt):
    print(f"[varlen] {kind} {dt}", flush=True)
    if kind == "plain":
        r = _varlen(dt, [100, 64, 200])
    elif kind == "seqused":
        r = _varlen(dt, [100, 64, 200], used_q=[70, 64, 150], used_k=[90, 30, 180])
    elif kind == "window_softcap_d256":
        r = _varlen(dt, [300, 77, 512, 129], D=256, H=16, gqa=1, wl=64, wr=0, sc=30.0)
    elif kind == "split":              # few heads: the keys of each query tile are split
        assert _varlen_split_bytes([700, 1300, 900], 2, 1, 64, True, dt) > 0
        r = _varlen(dt, [700, 1300, 900], D=64, H=2, gqa=1)
    elif kind == "split_seqused":
        r = _varlen(dt, [700, 1300, 900], used_q=[650, 1300, 700], used_k=[700, 1250, 880], D=64, H=2, gqa=1)
    elif kind == "split_full_d128":
        assert _varlen_split_bytes([900, 1500], 2, 2, 128, False, dt) > 0
        r = _varlen(dt, [900, 1500], D=128, H=2, gqa=2, causal=False)
    elif kind == "split_ragged":       # empty and one-row sequences among split ones
        assert _varlen_split_bytes([700, 0, 1300, 1, 900], 2, 1, 64, True, dt) > 0
        r = _varlen(dt, [700, 0, 1300, 1, 900], D=64, H=2, gqa=1)
    else:                              # many short causal sequences: the short-row shape (a grid
        # of 128 sequences x 8 heads, one 256-row tile each, at least 4 workgroups per CU)
        lens = np.random.default_rng(12).integers(1, 257, 128).tolist()
        lens[5], lens[77] = 0, 1
        r = _varlen(dt, lens, D=128 if kind.endswith("d128") else 64, H=8, gqa=2)
    o, l, o_ref, l_ref = r
    rel = orc.rel_rms(o, o_ref)
    lerr, inf_ok = lse_err(l, l_ref)
    log_errors("fwd_varlen", kind, dt, o=rel, lse=lerr)
    assert rel <= TOL[dt], f"rel_rms {rel:.3e}"
    assert inf_ok and lerr <= LSE_ABS, f"LSE err {lerr:.3e} inf_ok={inf_ok}"


def _sample_rows(S, tile_edges=(32, 64, 128, 256), n_random=48, seed=0):
    """First and last rows, rows on both sides of tile boundaries at several tile sizes, and
    seeded random rows."""
    rows = {0, 1, S - 2, S - 1}
    for t in tile_edges:
        for e in (t, S // 2 // t * t, (S - 1) // t * t):
            rows.update(r for r in (e - 1, e) if 0 <= r < S)
    rows.update(np.random.default_rng(seed).integers(0, S, n_random).tolist())
    return np.array(sorted(rows), dtype=np.int32)


def _check_rows(test, case, dt, got_o, got_lse, o_ref, l_ref, rows):
    """rel_rms over the sampled rows of O, max |LSE error| over them; log and assert."""
    o, r = got_o[..., rows, :], o_ref[..., rows, :]
    e = orc.rel_rms(o, r)
    le, inf_ok = lse_err(got_lse[..., rows], l_ref[..., rows])
    log_errors(test, case, dt, o=e, lse=le, rows=len(rows))
    assert np.isfinite(o).all(), "non-finite output"
    assert e <= TOL[dt], f"O rel_rms {e:.3e} > {TOL[dt]}"
    assert inf_ok and le <= LSE_ABS, f"LSE err {le:.3e}"


@pytest.mark.parametrize("cfg", [
    ("C2 causal fp16 B1 S16384 H32", 1, 16384, 32, True, "f16"),
    ("C2 causal fp16 B1 S8192 H32", 1, 8192, 32, True, "f16"),
    ("C2 causal fp16 B1 S4096 H32", 1, 4096, 32, True, "f16"),
    ("full bf16 B2 S8192 H32", 2, 8192, 32, False, "bf16"),
    # one round of causal workgroups with long rows: keys split in two
    ("key split causal fp16 B1 S8192 H6", 1, 8192, 6, True, "f16"),
    ("key split causal bf16 B1 S16384 H4", 1, 16384, 4, True, "bf16"),
    # short causal rows on grids of at least 4 workgroups per CU: 2-wave workgroups of 64 rows
    ("D128 short rows causal fp16 B16 S1024 H32", 16, 1024, 32, True, "f16", 128),
    ("D96 short rows causal bf16 B64 S512 H32", 64, 512, 32, True, "bf16", 96),
    ("D64 short rows causal fp16 B16 S1024 H32", 16, 1024, 32, True, "f16", 64),
    ("D32 short rows causal bf16 B64 S512 H32", 64, 512, 32, True, "bf16", 32),
    # head dim 96 runs the same shape on non-causal short rows
    ("D96 short rows full fp16 B64 S512 H32", 64, 512, 32, False, "f16", 96),
    ("D96 short rows full bf16 B16 S1024 H32", 16, 1024, 32, False, "bf16", 96),
    # head dims 64 and 32 on long rows: 4-wave workgroups at three waves per SIMD
    ("D64 long rows full fp16 B2 S4096 H32", 2, 4096, 32, False, "f16", 64),
    ("D64 long rows causal bf16 B1 S8192 H32", 1, 8192, 32, True, "bf16", 64),
    ("D32 long rows full fp16 B8 S1024 H16", 8, 1024, 16, False, "f16", 32),
    ("D32 long rows causal bf16 B1 S16384 H16", 1, 16384, 16, True, "bf16", 32),
], ids=lambda c: c[0])
def test_forward_full_size_sampled_rows(cfg):
    """BASELINE.json configs[1] at its full size and its S=8192 / S=4096 variants (and a
    non-causal bf16 grid of the same scale): grids that run the widest workgroup shapes.
    Sampled (batch, head) pairs and, in them, sampled query rows (first, last, both sides of
    tile boundaries, random) against the fp64 oracle, at the fp16/bf16 tolerances; LSE within
    1e-3. Head dims 64 and 32 on grids of long rows that take their long-row shape."""
    import torch

    from fable_attn import _C
    name, B, S, H, causal, dt, *width = cfg
    D = width[0] if width else 128
    print(f"[fwd-full] {name}", flush=True)
    tdt = torch.float16 if dt == "f16" else torch.bfloat16
    g = torch.Generator(device="cuda").manual_seed(3)
    q, k, v = (torch.randn(B, S, H, D, device="cuda", dtype=tdt, generator=g) for _ in range(3))
    qh, kh, vh = (x.transpose(1, 2) for x in (q, k, v))
    scale = D ** -0.5
    out, lse = _C.fwd(qh, kh, vh, scale, causal, -1, 0 if causal else -1, 0.0, None, 0.0, 0)
    torch.cuda.synchronize()
    heads = ((0, 0), (B - 1, H - 1), (B // 2, H // 2))
    pick = lambda t: np.stack([to_np(t[bb, hd]) for bb, hd in heads])[None]   # [1, 3, S, D]
    rows = _sample_rows(S)
    o_ref, l_ref = orc.fwd(pick(qh), pick(kh), pick(vh), scale, causal, rows=rows)
    got_l = np.stack([to_np(lse[bb, hd]) for bb, hd in heads])[None]
    _check_rows("fwd_full", name, dt, pick(out), got_l, o_ref, l_ref, rows)


def test_varlen_full_config_c5_sampled():
    """BASELINE.json configs[4] at its full size: 8 packed sequences with seeded lengths in
    [512, 8192], H=16, D=256, bf16, causal + window (512, 0) + softcap 30, one varlen launch.
    Sampled (sequence, head) pairs and sampled rows in them against the fp64 oracle, at the
    bf16 tolerance; LSE within 1e-3."""
    import itertools

    import torch

    from fable_attn import _C
    H, D, W, CAP = 16, 256, 512, 30.0
    lens = torch.randint(512, 8193, (8,), generator=torch.Generator().manual_seed(0)).tolist()
    offs = [0] + list(itertools.accumulate(lens))
    print(f"[fwd-full] C5 varlen lens {lens}", flush=True)
    cu = torch.tensor(offs, dtype=torch.int32, device="cuda")
    g = torch.Generator(device="cuda").manual_seed(0)
    q, k, v = (torch.randn(offs[-1], H, D, device="cuda", dtype=torch.bfloat16, generator=g) for _ in range(3))
    scale = D ** -0.5
    out, lse = _C.fwd_varlen(q, k, v, cu, cu, max(lens), max(lens), scale, True, W, 0, CAP, None,
                             0.0, 0, return_lse=True)
    torch.cuda.synchronize()
    for z, hd in ((0, 0), (3, 7), (7, H - 1), (int(np.argmax(lens)), 5)):
        a, L = offs[z], lens[z]
        seq = lambda t: to_np(t[a:a + L, hd])[None, None]                    # [1, 1, L, D]
        rows = _sample_rows(L, seed=z)
        o_ref, l_ref = orc.fwd(seq(q), seq(k), seq(v), scale, True, W, 0, CAP, rows=rows)
        got_l = to_np(lse[hd, a:a + L])[None, None]
        _check_rows("fwd_full_c5", f"C5 seq {z} (L={L}) head {hd}", "bf16", seq(out), got_l,
                    o_ref, l_ref, rows)


# The D=256 softcap loop computes tanh by a polynomial on |scale*s/softcap| <= 0.4 and switches
# a whole 32-key block of one wave to the exact form when any of its scores is outside that
# range. name, B, S, H, gqa, window left, softcap, alibi, key rows scaled by 8 (None: none)
SOFTCAP_RANGE = [
    ("narrow: some blocks outside the range", 1, 300, 8, 2, 64, 30.0, False, (96, 128)),
    ("64-key tiles: some blocks outside the range", 1, 330, 8, 2, -1, 30.0, False, (160, 224)),
    ("64-key tiles + alibi: every block outside", 1, 230, 8, 2, -1, 2.0, True, None),
    ("narrow: every block outside", 1, 260, 4, 1, 100, 1.5, False, None),
]


@pytest.mark.parametrize("dt", ["f16", "bf16"])
@pytest.mark.parametrize("case", SOFTCAP_RANGE, ids=[c[0] for c in SOFTCAP_RANGE])
def test_softcap_polynomial_range(case, dt):
    import torch

    from fable_attn import _C
    name, B, S, H, gqa, wl, sc, alibi, big = case
    print(f"[fwd-softcap-range] {name} {dt}", flush=True)
    D, Hk = 256, H // gqa
    q = gen((B, H, S, D), 41, dt)
    k = gen((B, Hk, S, D), 42, dt)
    v = gen((B, Hk, S, D), 43, dt)
    if big is not None:
        k[:, :, big[0]:big[1]] *= 8.0          # exact in fp16/bf16: a power of two
    al = _alibi(H) if alibi else None
    scale = 1.0 / math.sqrt(D)
    o_ref, l_ref = orc.fwd(q, k, v, scale, True, wl, 0, sc, al, 0)
    dev = lambda a: to_dev(a, dt).transpose(1, 2).contiguous().transpose(1, 2)
    ald = torch.from_numpy(al).cuda() if al is not None else None
    out, lse = _C.fwd(dev(q), dev(k), dev(v), scale, True, wl, 0, sc, ald, 0.0, 0)
    torch.cuda.synchronize()
    o, l = to_np(out), to_np(lse)
    rel = orc.rel_rms(o, o_ref)
    lerr, inf_ok = lse_err(l, l_ref)
    log_errors("fwd_softcap_range", name, dt, o=rel, lse=lerr)
    assert np.isfinite(o).all()
    assert rel <= TOL[dt], f"rel_rms {rel:.3e} > {TOL[dt]}"
    assert inf_ok and lerr <= LSE_ABS, f"LSE abs err {lerr:.3e}"


# bf16 softcap kernels with a cap of at most 33 (no alibi) subtract the fixed bound
# softcap*log2(e) from every logit instead of a running row max, so the probabilities reach
# down to 2^-95 of the largest possible one. "negative": every query is near +30 u and every
# key near -30 u (u a unit vector), so scale*q.k is about -56 and every logit sits near -softcap
# (the smallest probabilities the offset produces, and every block on the exact-form path);
# a cap above 33 takes the running max. name, S, D, window left, softcap, negative
SOFTCAP_FIXED = [
    ("d256 narrow, logits near -30", 300, 256, 64, 30.0, True),
    ("d256 64-key tiles, logits near -33 (largest fixed cap)", 330, 256, -1, 33.0, True),
    ("d256 narrow, cap 40 (running max)", 300, 256, 64, 40.0, True),
    ("d128 causal, logits near -30", 260, 128, -1, 30.0, True),
    ("d128 causal, random scores", 260, 128, -1, 20.0, False),
]


@pytest.mark.parametrize("dt", ["f16", "bf16"])
@pytest.mark.parametrize("case", SOFTCAP_FIXED, ids=[c[0] for c in SOFTCAP_FIXED])
def test_softcap_fixed_offset(case, dt):
    import torch

    from fable_attn import _C
    name, S, D, wl, sc, neg = case
    print(f"[fwd-softcap-fixed] {name} {dt}", flush=True)
    B, H, Hk = 1, 4, 2
    q = gen((B, H, S, D), 51, dt)
    k = gen((B, Hk, S, D), 52, dt)
    v = gen((B, Hk, S, D), 53, dt)
    if neg:
        u = orc.randn((D,), 54, "f32").astype(np.float64)
        u /= np.linalg.norm(u)
        q = orc.round_to(30.0 * u + 0.5 * q, dt)
        k = orc.round_to(-30.0 * u + 0.5 * k, dt)
    scale = 1.0 / math.sqrt(D)
    o_ref, l_ref = orc.fwd(q, k, v, scale, True, wl, 0, sc, None, 0)
    if neg:
        assert l_ref[np.isfinite(l_ref)].max() < -0.8 * sc + math.log(S)  # logits near -softcap
    dev = lambda a: to_dev(a, dt).transpose(1, 2).contiguous().transpose(1, 2)
    out, lse = _C.fwd(dev(q), dev(k), dev(v), scale, True, wl, 0, sc, None, 0.0, 0)
    torch.cuda.synchronize()
    o, l = to_np(out), to_np(lse)
    rel = orc.rel_rms(o, o_ref)
    lerr, inf_ok = lse_err(l, l_ref)
    log_errors("fwd_softcap_fixed", name, dt, o=rel, lse=lerr)
    assert np.isfinite(o).all()
    assert rel <= TOL[dt], f"rel_rms {rel:.3e} > {TOL[dt]}"
    assert inf_ok and lerr <= LSE_ABS, f"LSE abs err {lerr:.3e}"


# Small grids whose keys the library splits over several workgroups per query tile (fp32
# partials merged by a second kernel): causal with splits that see no key, SQ < SK and SQ > SK
# (empty rows), GQA, alibi, softcap on the one-wave D=256 loop, a right-only window, head dims
# that leave zero columns. Same case layout as CASES.
SPLIT_CASES = [
    ("split d128 causal", 1, 1500, 1500, 128, 2, 1, True, -1, -1, 0.0, False, 0),
    ("split d64 full SQ<SK GQA", 1, 100, 3000, 64, 4, 2, False, -1, -1, 0.0, False, 0),
    ("split d256 causal softcap", 1, 700, 700, 256, 2, 1, True, -1, -1, 30.0, False, 0),
    ("split d96 causal SQ<SK alibi", 1, 200, 900, 96, 2, 2, True, -1, -1, 0.0, True, 0),
    ("split d128 window (-1,40)", 1, 1200, 1200, 128, 1, 1, False, -1, 40, 0.0, False, 0),
    ("split d64 causal SQ>SK empty rows B2", 2, 600, 520, 64, 2, 1, True, -1, -1, 0.0, False, 0),
    ("split d80 full", 1, 300, 2100, 80, 3, 1, False, -1, -1, 0.0, False, 0),
]


def _split_bytes(case, dt):
    from fable_attn import _C, _lib
    name, B, SQ, SK, D, H, gqa, causal, wl, wr, sc, alibi, chunk = case
    s = lambda S, Hh: _lib.Strides(S * Hh * D, D, Hh * D)
    p = _lib.FableFwdParams(None, None, None, None, None, s(SQ, H), s(SK, H // gqa), s(SK, H // gqa),
                            s(SQ, H), SQ, SK, D, H, gqa, D ** -0.5, sc, wl, wr, None, 1 if causal else 0,
                            0.0, 0, None, None, B, chunk, None, None, H * SQ, SQ)
    return _C._L.fable_attn_fwd_ws_bytes(p, 0 if dt == "f16" else 1)


@pytest.mark.parametrize("dt", ["f16", "bf16"])
@pytest.mark.parametrize("case", SPLIT_CASES, ids=[c[0] for c in SPLIT_CASES])
def test_forward_key_split_parity(case, dt):
    print(f"[fwd-split] {case[0]} {dt}", flush=True)
    assert _split_bytes(case, dt) > 0, "the case must take the key split"
    o, l, o_ref, l_ref = run_case(case, dt)
    rel = orc.rel_rms(o, o_ref)
    lerr, inf_ok = lse_err(l, l_ref)
    log_errors("fwd_split", case[0], dt, o=rel, lse=lerr)
    assert np.isfinite(o).all(), "non-finite output"
    assert rel <= TOL[dt], f"rel_rms {rel:.3e} > {TOL[dt]}"
    assert inf_ok, "empty-row LSE (-inf) pattern differs"
    assert lerr <= LSE_ABS, f"LSE abs err {lerr:.3e}"
    empty = np.isneginf(l_ref)
    if empty.any():
        rows = np.broadcast_to(empty[..., None], o.shape)
        assert (o[rows] == 0).all(), "empty rows must be exactly zero"


def test_forward_key_split_matches_unsplit():
    """The split and the unsplit kernels on the same inputs (a workspace that is too small
    runs the call unsplit): equal to fp32 summation order."""
    import torch

    from fable_attn import _C, _lib
    case = SPLIT_CASES[0]
    name, B, SQ, SK, D, H, gqa, causal, wl, wr, sc, alibi, chunk = case
    q, k, v = (to_dev(gen((B, H, n, D), 7 + i, "f16"), "f16") for i, n in enumerate((SQ, SK, SK)))
    outs = []
    for split in (True, False):
        out = torch.empty_like(q)
        lse = torch.empty((B, H, SQ), dtype=torch.float32, device="cuda")
        s = lambda t: _lib.Strides(t.stride(0), t.stride(1), t.stride(2))
        p = _lib.FableFwdParams(q.data_ptr(), k.data_ptr(), v.data_ptr(), out.data_ptr(), lse.data_ptr(),
                                s(q), s(k), s(v), s(out), SQ, SK, D, H, gqa, D ** -0.5, 0.0, -1, -1, None,
                                1, 0.0, 0, None, None, B, 0, None, None, H * SQ, SQ)
        need = _C._L.fable_attn_fwd_ws_bytes(p, 0)
        assert need > 0
        ws = torch.empty(need if split else need - 256, dtype=torch.uint8, device="cuda")
        _lib.check(_C._L.fable_attn_fwd_ws(p, 0, ws.data_ptr(), ws.numel(), None), "fable_attn_fwd_ws")
        torch.cuda.synchronize()
        outs.append((to_np(out), to_np(lse)))
    assert np.abs(outs[0][0] - outs[1][0]).max() <= 2e-3
    assert np.abs(outs[0][1] - outs[1][1]).max() <= 1e-5
