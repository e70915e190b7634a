"""C-ABI checks that need no GPU: the header compiles as C, every struct field offset in the
ctypes binding equals the compiler's, the library loads and exports every function the header
declares, and argument validation fails cleanly before any device work."""
import ctypes
import os
import re
import subprocess

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
HEADER = os.path.join(ROOT, "include", "fable_attn_abi.h")


def _declared_functions():
    src = open(HEADER).read()
    src = re.sub(r"/\*.*?\*/", "", src, flags=re.S)
    return sorted(set(re.findall(r"^\s*(?:int|int64_t|size_t|const char\*)\s+(\w+)\s*\(", src, flags=re.M)))


REF_IFACE = "/root/reference/package/csrc/fa_iface.h"


def _struct_table():
    from fable_attn import _lib
    return (("fa_strides", _lib.Strides), ("FableFwdParams", _lib.FableFwdParams),
            ("FableBwdParams", _lib.FableBwdParams), ("FableDecParams", _lib.FableDecParams),
            ("CombineParams", _lib.CombineParams), ("Strides", _lib.RefStrides),
            ("FwdParams", _lib.RefFwdParams), ("BwdParams", _lib.RefBwdParams),
            ("DecParams", _lib.RefDecParams))


def _offsets(tmp_path, header, structs, compiler):
    """sizeof and offsetof of every field of `structs` (name, ctypes mirror) as the compiler
    lays them out from `header`."""
    lines = ['#include <stdio.h>', '#include <stddef.h>', f'#include "{header}"', "int main(void){"]
    for name, st in structs:
        lines.append(f'printf("{name} sizeof %zu\\n", sizeof({name}));')
        for f, _ in st._fields_:
            lines.append(f'printf("{name} {f} %zu\\n", offsetof({name}, {f}));')
    lines.append("return 0;}")
    src = tmp_path / ("abi.c" if compiler == "gcc" else "abi.cpp")
    src.write_text("\n".join(lines))
    exe = tmp_path / ("abi_" + compiler)
    std = "-std=c11" if compiler == "gcc" else "-std=c++17"
    subprocess.run([compiler, std, "-Wall", "-Werror", "-o", str(exe), str(src)], check=True)
    out = subprocess.run([str(exe)], check=True, capture_output=True, text=True).stdout
    return {tuple(l.split()[:2]): int(l.split()[2]) for l in out.splitlines()}


def _check_layout(got, structs):
    for name, st in structs:
        assert got[(name, "sizeof")] == ctypes.sizeof(st), name
        for f, _ in st._fields_:
            assert got[(name, f)] == getattr(st, f).offset, (name, f)


def test_struct_layout_matches_header(tmp_path):
    """Both struct families of the header, compiled as C and as C++, against the binding."""
    from fable_attn import _lib
    structs = _struct_table()
    _check_layout(_offsets(tmp_path, HEADER, structs, "gcc"), structs)
    _check_layout(_offsets(tmp_path, HEADER, structs, "g++"), structs)
    # every header field is mirrored (nothing missing on the Python side)
    assert len(_lib.FableFwdParams._fields_) == 30
    assert len(_lib.RefFwdParams._fields_) == 31 and len(_lib.RefDecParams._fields_) == 32


def test_reference_layout_matches_reference_header(tmp_path):
    """The reference-layout structs are bit-for-bit the reference's own fa_iface.h:9-63 (every
    field's offset and the size), so its compiled glue can pass them by value to this library.
    Needs the reference tree (skipped where it is absent, e.g. on a GPU box)."""
    if not os.path.exists(REF_IFACE):
        pytest.skip("reference tree absent")
    from fable_attn import _lib
    ref = (("Strides", _lib.RefStrides), ("Str", _lib.RefStrides), ("FwdParams", _lib.RefFwdParams),
           ("BwdParams", _lib.RefBwdParams), ("DecParams", _lib.RefDecParams))
    _check_layout(_offsets(tmp_path, REF_IFACE, ref, "g++"), ref)
    # and the library's own compiled sizes agree
    lib = _lib.load()
    assert lib.fable_attn_struct_size(5) == ctypes.sizeof(_lib.RefFwdParams)
    assert lib.fable_attn_struct_size(6) == ctypes.sizeof(_lib.RefBwdParams)
    assert lib.fable_attn_struct_size(7) == ctypes.sizeof(_lib.RefDecParams)


def test_library_exports_every_declared_function():
    from fable_attn import _lib
    lib = _lib.load()
    declared = _declared_functions()
    assert set(declared) == set(_lib.EXPORTS), declared
    for f in declared:
        assert hasattr(lib, f), f
    assert lib.fable_attn_abi_version() == _lib.ABI_VERSION == 5
    for k, st in _lib.STRUCTS.items():
        assert lib.fable_attn_struct_size(k) == ctypes.sizeof(st)


def test_launchers_validate_before_device_work():
    from fable_attn import _lib
    lib = _lib.load()
    p = _lib.FableFwdParams()          # null tensors
    assert lib.fable_attn_fwd(p, 0, None) == 3
    assert b"null" in lib.fable_attn_last_error()
    p.Q = p.K = p.V = p.O = 16    # never dereferenced: rejected on head_dim first
    p.NH, p.gqa, p.batch, p.SQ, p.SK, p.HD = 4, 1, 1, 8, 8, 100
    assert lib.fable_attn_fwd(p, 0, None) == 2
    assert b"head_dim=100" in lib.fable_attn_last_error()
    p.HD = 64
    assert lib.fable_attn_fwd(p, 7, None) == 1          # unknown dtype
    p.dropout_p = 1.0                                      # keeps nothing: rejected
    assert lib.fable_attn_fwd(p, 0, None) == 3
    assert b"dropout_p" in lib.fable_attn_last_error()
    c = _lib.CombineParams()
    assert lib.fa_combine_launch(c, None) == 3


def test_reference_launchers_validate_before_device_work():
    """The reference-layout launchers reject bad arguments with a status (and print it) before
    any device work, through the same checks as the extended entry points."""
    from fable_attn import _lib
    lib = _lib.load()
    r = _lib.RefFwdParams()
    assert lib.fa_forward_launch(r, 0, None) == 3          # null tensors
    r.Q = r.K = r.V = r.O = 16
    r.NH, r.gqa, r.batch, r.SQ, r.SK, r.HD = 4, 1, 1, 8, 8, 100
    assert lib.fa_forward_launch(r, 0, None) == 2          # head_dim 100 is not a multiple of 8
    r.HD, r.batch, r.LSE = 64, 2, 16                       # LSE without a batch stride
    assert lib.fa_forward_launch(r, 0, None) == 3
    assert b"batch == 1" in lib.fable_attn_last_error()
    b = _lib.RefBwdParams()
    assert lib.fable_attn_backward_launch(b, 1, None) == 3
    d = _lib.RefDecParams()
    assert lib.fa_decode_launch(d, 0, None, None, None) == 3


@pytest.mark.parametrize("hint,expect", [(4, 4), (1000, 512), (-1, None)])
def test_decode_split_plan(hint, expect):
    from fable_attn import _lib
    lib = _lib.load()
    n = lib.fa_decode_num_splits(16, 1, 32, 4, 32768, hint)
    if expect is not None:
        assert n == expect
    else:
        assert 1 <= n <= 512


@pytest.mark.parametrize("batch,ctx,expect", [
    (16, 32768, 2),     # C4: one full round of 256 workgroups, the model's choice
    (1, 32768, 32),     # 8 groups: the round filled (1024 keys per split)
    (4, 32768, 8),
    (1, 8192, 21),      # filling would leave 256 keys per split: the model's choice stays
    (64, 4096, 1),
])
def test_decode_split_count(batch, ctx, expect):
    """The automatic split count (Hq 32, Hk 8): the workgroup-round model, and a round that
    would leave CUs idle filled while each split keeps at least 512 keys."""
    from fable_attn import _lib
    lib = _lib.load()
    assert lib.fa_decode_num_splits(batch, 1, 32, 4, ctx, 0) == expect


def _visible_tiles(SQ, SK, causal, wl=-1, wr=-1):
    """(32-key, 32-query) blocks holding at least one visible pair, counted by brute force over
    the mask of every (query, key) pair (the reference's visibility rule, bottom-right aligned)."""
    import numpy as np
    q = np.arange(SQ)[:, None] + (SK - SQ)
    k = np.arange(SK)[None, :]
    vis = np.ones((SQ, SK), bool)
    if causal:
        vis &= k <= q
    if wl >= 0:
        vis &= k >= q - wl
    if wr >= 0:
        vis &= k <= q + wr
    nqb, nkb = (SQ + 31) // 32, (SK + 31) // 32
    pad = np.zeros((nqb * 32, nkb * 32), bool)
    pad[:SQ, :SK] = vis
    return int(pad.reshape(nqb, 32, nkb, 32).any(axis=(1, 3)).sum())


def test_bwd_ds_workspace_size():
    """fable_attn_bwd_ds_bytes: a 256-byte-padded table of ceil(SK/32)+1 ints, then 2 KiB per
    (32-query, 32-key) tile that holds a visible pair, for every (batch, q head), for the
    fp16/bf16 head dims (every multiple of 8 up to 256); 0 elsewhere (host-only call).
    The tile count is checked against a brute-force count over the pair mask."""
    from fable_attn import _lib
    lib = _lib.load()
    p = _lib.FableBwdParams()
    hdr = lambda SK: -(-((SK + 31) // 32 + 1) * 4 // 256) * 256
    p.B, p.Hq, p.Hk, p.gqa, p.SQ, p.SK, p.D = 2, 8, 2, 4, 100, 65, 128
    p.win_left, p.win_right = -1, -1
    want = hdr(65) + 2 * 8 * 4 * 3 * 2048                   # no mask: the whole rectangle
    assert lib.fable_attn_bwd_ds_bytes(p, 0) == want and lib.fable_attn_bwd_ds_bytes(p, 1) == want
    p.D = 64
    assert lib.fable_attn_bwd_ds_bytes(p, 1) == want
    p.D = 80                                                 # any multiple of 8 up to 128
    assert lib.fable_attn_bwd_ds_bytes(p, 1) == want
    assert lib.fable_attn_bwd_ds_bytes(p, 2) == 0      # fp32 recomputes
    for d in (8, 16, 32, 96, 120):                         # widths 32 and 96 have the path too
        p.D = d
        assert lib.fable_attn_bwd_ds_bytes(p, 1) == want, d
    for d in (136, 160, 192, 224, 256):                    # the one-wave-per-SIMD widths too
        p.D = d
        assert lib.fable_attn_bwd_ds_bytes(p, 0) == want, d
    p.D = 264                                               # past 256: no kernel at all
    assert lib.fable_attn_bwd_ds_bytes(p, 0) == 0
    p.D, p.SQ = 128, 0
    assert lib.fable_attn_bwd_ds_bytes(p, 0) == 0
    # causal and windowed: only the tiles with a visible pair
    for SQ, SK, causal, wl, wr in ((4096, 4096, 1, -1, 0), (150, 150, 1, -1, -1), (96, 300, 1, -1, -1),
                                   (300, 96, 1, -1, -1), (1000, 1000, 0, 100, 0), (500, 700, 0, 64, 64),
                                   (700, 500, 1, 37, -1), (64, 64, 0, 5000, -1)):
        # (64 batches: grids of more than one round, so the dK/dV kernel does not split)
        p.B, p.Hq, p.Hk, p.gqa = 64, 3, 3, 1
        p.SQ, p.SK, p.causal, p.win_left, p.win_right = SQ, SK, causal, wl, wr
        got = lib.fable_attn_bwd_ds_bytes(p, 0)
        assert got == hdr(SK) + 64 * 3 * _visible_tiles(SQ, SK, causal, wl, wr) * 2048, (SQ, SK, causal, wl, wr)


def test_bwd_query_split_workspace():
    """A dK/dV grid of one round splits the query tiles of each key block; the workspace then
    ends, after the 256-byte-aligned tiles, with the fp32 partial dK and dV rows of every share."""
    from fable_attn import _lib
    lib = _lib.load()
    hdr = lambda SK: -(-((SK + 31) // 32 + 1) * 4 // 256) * 256
    tiles = lambda S: _visible_tiles(S, S, 1)
    p = _lib.FableBwdParams()
    p.win_left, p.win_right, p.causal, p.D = -1, -1, 1, 128
    # B1 H8 S4096 causal: 256 dK/dV workgroups (one round), key block 0 takes 128 steps -> 2 shares
    p.B, p.Hq, p.Hk, p.gqa, p.SQ, p.SK = 1, 8, 8, 1, 4096, 4096
    tiles_end = -(-(hdr(4096) + 8 * tiles(4096) * 2048) // 256) * 256
    assert lib.fable_attn_bwd_ds_bytes(p, 1) == tiles_end + 2 * 2 * 8 * 4096 * 128 * 4
    # a quarter of the CUs (64 workgroups at D=64, 64-key blocks): up to 4 shares of >= 16 steps
    p.D, p.Hq, p.Hk, p.SQ, p.SK = 64, 2, 2, 2048, 2048
    tiles_end = -(-(hdr(2048) + 2 * tiles(2048) * 2048) // 256) * 256
    assert lib.fable_attn_bwd_ds_bytes(p, 0) == tiles_end + 4 * 2 * 2 * 2048 * 64 * 4
    # C3 (2048 workgroups) and the one-wave widths never split
    p.D, p.B, p.Hq, p.Hk, p.SQ, p.SK = 128, 2, 32, 32, 4096, 4096
    assert lib.fable_attn_bwd_ds_bytes(p, 0) == hdr(4096) + 2 * 32 * tiles(4096) * 2048
    p.D, p.B, p.Hq, p.Hk = 256, 1, 8, 8
    assert lib.fable_attn_bwd_ds_bytes(p, 0) == hdr(4096) + 8 * tiles(4096) * 2048


def _fwd_params(B, H, SQ, SK, D, gqa=1, causal=False, wl=-1, wr=-1, softcap=0.0, chunk=0,
                dropout=0.0, varlen=False):
    """FableFwdParams of a dense [B,H,S,D] call, tensor pointers left null (a workspace query
    reads none)."""
    from fable_attn import _lib
    s = lambda S, Hh: _lib.Strides(S * Hh * D, D, Hh * D)
    cu = ctypes.c_void_p(16) if varlen else None
    return _lib.FableFwdParams(None, None, None, None, None, s(SQ, H), s(SK, H // gqa), s(SK, H // gqa),
                               s(SQ, H), SQ, SK, D, H, gqa, D ** -0.5, softcap, wl, wr, None,
                               1 if causal else 0, dropout, 0, cu, cu, B, chunk, None, None, H * SQ, SQ)


def test_forward_key_split_workspace_query():
    """fable_attn_fwd_ws_bytes: the key split of small grids (host logic only, no launch). C1
    (64 query tiles of 128 rows on 256 CUs) splits in 4: fp32 partial O and LSE of every row per
    split; the large grids, left windows, chunks, dropout and fp32 never split; an
    invalid call answers -1."""
    from fable_attn import _lib
    lib = _lib.load()
    q = lambda dt=0, **kw: lib.fable_attn_fwd_ws_bytes(_fwd_params(**kw), dt)
    rows = 1 * 8 * 1024
    assert q(B=1, H=8, SQ=1024, SK=1024, D=64) == (4 * rows * 64 * 4 + 255) // 256 * 256 + 4 * rows * 4
    assert q(1, B=1, H=8, SQ=1024, SK=1024, D=64) > 0                      # bf16 alike
    assert q(B=1, H=32, SQ=16384, SK=16384, D=128, causal=True) == 0       # C2: a full grid
    assert q(B=2, H=32, SQ=4096, SK=4096, D=128, causal=True) == 0
    assert q(B=1, H=2, SQ=1500, SK=1500, D=128, causal=True) > 0
    # one round of causal workgroups: split in two only with rows of 128 key tiles or more
    two = lambda S, H: (2 * H * S * 128 * 4 + 255) // 256 * 256 + 2 * H * S * 4
    assert q(B=1, H=6, SQ=8192, SK=8192, D=128, causal=True) == two(8192, 6)
    assert q(B=1, H=8, SQ=8192, SK=8192, D=128, causal=True) == two(8192, 8)
    assert q(B=1, H=12, SQ=4096, SK=4096, D=128, causal=True) == 0            # 64-tile rows
    assert q(B=1, H=16, SQ=8192, SK=8192, D=128, causal=False) == 0           # not causal
    assert q(B=1, H=16, SQ=8192, SK=8192, D=128, causal=True) == 0            # two rounds
    assert q(B=1, H=8, SQ=1024, SK=1024, D=64, wl=100) == 0                # left window
    assert q(B=1, H=8, SQ=1024, SK=1024, D=64, chunk=256) == 0
    assert q(B=1, H=8, SQ=1024, SK=1024, D=64, dropout=0.1) == 0
    assert q(B=1, H=8, SQ=1024, SK=1024, D=64, varlen=True) == q(B=1, H=8, SQ=1024, SK=1024, D=64)  # packed alike
    assert q(2, B=1, H=8, SQ=1024, SK=1024, D=64) == 0                     # fp32
    assert q(B=1, H=8, SQ=256, SK=256, D=64) == 0                          # too few key tiles
    assert q(B=1, H=8, SQ=1024, SK=1024, D=60) == -1                       # no kernel for D=60
    assert b"head_dim=60" in lib.fable_attn_last_error()
