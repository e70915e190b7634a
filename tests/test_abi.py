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


def _offsets_from_gcc(tmp_path):
    from fable_attn import _lib
    lines = ['#include <stdio.h>', '#include <stddef.h>', f'#include "{HEADER}"', "int main(void){"]
    for name, st in (("fa_strides", _lib.Strides), ("FwdParams", _lib.FwdParams),
                     ("BwdParams", _lib.BwdParams), ("DecParams", _lib.DecParams),
                     ("CombineParams", _lib.CombineParams)):
        lines.append(f'printf("{name} sizeof %zu\\n", sizeof({name}));')
        for f, _ in st._fields_:
            lines.append(f'printf("{name} {f} %zu\\n", offsetof({name}, {f}));')
    lines.append("return 0;}")
    c = tmp_path / "abi.c"
    c.write_text("\n".join(lines))
    exe = tmp_path / "abi"
    subprocess.run(["gcc", "-std=c11", "-Wall", "-Werror", "-o", str(exe), str(c)], check=True)
    out = subprocess.run([str(exe)], check=True, capture_output=True, text=True).stdout
    return {tuple(l.split()[:2]): int(l.split()[2]) for l in out.splitlines()}


def test_struct_layout_matches_header(tmp_path):
    from fable_attn import _lib
    got = _offsets_from_gcc(tmp_path)
    for name, st in (("fa_strides", _lib.Strides), ("FwdParams", _lib.FwdParams),
                     ("BwdParams", _lib.BwdParams), ("DecParams", _lib.DecParams),
                     ("CombineParams", _lib.CombineParams)):
        assert got[(name, "sizeof")] == ctypes.sizeof(st), name
        for f, _ in st._fields_:
            assert got[(name, f)] == getattr(st, f).offset, (name, f)
    # every header field is mirrored (nothing missing on the Python side)
    assert len(_lib.FwdParams._fields_) == 30


def test_library_exports_every_declared_function():
    from fable_attn import _lib
    lib = _lib.load()
    declared = _declared_functions()
    assert set(declared) == set(_lib.EXPORTS), declared
    for f in declared:
        assert hasattr(lib, f), f
    assert lib.fable_attn_abi_version() == _lib.ABI_VERSION == 3
    for k, st in _lib.STRUCTS.items():
        assert lib.fable_attn_struct_size(k) == ctypes.sizeof(st)


def test_launchers_validate_before_device_work():
    from fable_attn import _lib
    lib = _lib.load()
    p = _lib.FwdParams()          # null tensors
    assert lib.fa_forward_launch(p, 0, None) == 3
    assert b"null" in lib.fable_attn_last_error()
    p.Q = p.K = p.V = p.O = 16    # never dereferenced: rejected on head_dim first
    p.NH, p.gqa, p.batch, p.SQ, p.SK, p.HD = 4, 1, 1, 8, 8, 72
    assert lib.fa_forward_launch(p, 0, None) == 2
    assert b"head_dim=72" in lib.fable_attn_last_error()
    p.HD = 64
    assert lib.fa_forward_launch(p, 7, None) == 1          # unknown dtype
    p.dropout_p = 1.0                                      # keeps nothing: rejected
    assert lib.fa_forward_launch(p, 0, None) == 3
    assert b"dropout_p" in lib.fable_attn_last_error()
    c = _lib.CombineParams()
    assert lib.fa_combine_launch(c, None) == 3


@pytest.mark.parametrize("hint,expect", [(4, 4), (1000, 512), (-1, None)])
def test_decode_split_plan(hint, expect):
    from fable_attn import _lib
    lib = _lib.load()
    n = lib.fa_decode_num_splits(16, 1, 32, 4, 32768, hint)
    if expect is not None:
        assert n == expect
    else:
        assert 1 <= n <= 512


def test_bwd_ds_workspace_size():
    """fable_attn_bwd_ds_bytes: 2 KiB per (32-query, 32-key) tile of every (batch, q head) for
    the fp16/bf16 head dims with a dS-workspace path (64, 128); 0 elsewhere (host-only call)."""
    from fable_attn import _lib
    lib = _lib.load()
    p = _lib.BwdParams()
    p.B, p.Hq, p.Hk, p.gqa, p.SQ, p.SK, p.D = 2, 8, 2, 4, 100, 65, 128
    want = 2 * 8 * 4 * 3 * 2048
    assert lib.fable_attn_bwd_ds_bytes(p, 0) == want and lib.fable_attn_bwd_ds_bytes(p, 1) == want
    p.D = 64
    assert lib.fable_attn_bwd_ds_bytes(p, 1) == want
    assert lib.fable_attn_bwd_ds_bytes(p, 2) == 0      # fp32 recomputes
    p.D = 256
    assert lib.fable_attn_bwd_ds_bytes(p, 0) == 0
    p.D, p.SQ = 128, 0
    assert lib.fable_attn_bwd_ds_bytes(p, 0) == 0
