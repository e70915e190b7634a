"""Generate the golden forward fixtures in tests/golden/fwd_golden.npz.

Inputs follow the reference forward gate exactly (kernels/fa_forward_gate.inc:33-47): the LCG
stream frand (fa_common.hpp:140-141) seeded with 1234567 + HD*7 + NH + SQ + dt*13, Q then K then V
drawn in the gate's layouts (Q [SQ][NH][HD], K/V [NKV][SK][HD]), rounded to the dtype, alibi
slopes -2^(-8(h+1)/NH). Expected outputs are computed by the reference's own ref_attention
(oracle/_ref/libref.so, built from kernels/fa_common.hpp) and must agree with this repository's
restatement (oracle/oracle.c) before anything is written. Run in the development container,
where /root/reference exists:

    make -C oracle && python tests/golden/make_golden.py
"""
import os
import sys

import numpy as np

ROOT = os.path.dirname(os.path.dirname(os.path.dirname(os.path.abspath(__file__))))
sys.path.insert(0, ROOT)
from oracle import oracle as orc  # noqa: E402

# (name, SQ, SK, HD, NH, gqa, causal, alibi, wl, wr, softcap, chunk) — a subset of the gate's
# table (fa_forward_gate.inc:170-205) at its own sizes
CASES = [
    ("d128 causal GQA4", 256, 256, 128, 32, 4, True, False, -1, -1, 0.0, 0),
    ("d128 full", 192, 192, 128, 16, 4, False, False, -1, -1, 0.0, 0),
    ("d128 SQ<SK", 128, 320, 128, 16, 4, True, False, -1, -1, 0.0, 0),
    ("d128 SQ>SK empty", 256, 64, 128, 16, 4, True, False, -1, -1, 0.0, 0),
    ("win (63,0)", 256, 256, 128, 16, 4, True, False, 63, 0, 0.0, 0),
    ("win (32,32)", 256, 256, 128, 16, 4, False, False, 32, 32, 0.0, 0),
    ("win (0,0)", 256, 256, 128, 16, 4, False, False, 0, 0, 0.0, 0),
    ("softcap 30", 200, 200, 128, 16, 4, True, False, -1, -1, 30.0, 0),
    ("alibi", 200, 200, 128, 16, 4, True, True, -1, -1, 0.0, 0),
    ("d64", 200, 200, 64, 16, 4, True, False, -1, -1, 0.0, 0),
    ("d256", 160, 160, 256, 8, 4, True, False, -1, -1, 0.0, 0),
    ("chunk 100", 256, 256, 128, 16, 4, True, False, -1, -1, 0.0, 100),
]
DTS = {"f16": 0, "bf16": 1}


def gate_inputs(SQ, SK, HD, NH, gqa, dt):
    nkv = NH // gqa
    seed = 1234567 + HD * 7 + NH + SQ + DTS[dt] * 13
    n_q, n_k = SQ * NH * HD, nkv * SK * HD
    vals, _ = orc.frand(n_q + 2 * n_k, seed)
    q = orc.round_to(vals[:n_q].reshape(SQ, NH, HD), dt)
    k = orc.round_to(vals[n_q:n_q + n_k].reshape(nkv, SK, HD), dt)
    v = orc.round_to(vals[n_q + n_k:].reshape(nkv, SK, HD), dt)
    # oracle layout [B,H,S,D]
    return q.transpose(1, 0, 2)[None].copy(), k[None].copy(), v[None].copy()


def main():
    if orc.ref_lib() is None:
        sys.exit("oracle/_ref/libref.so is missing: run `make -C oracle` with /root/reference present")
    out = {}
    for i, (name, SQ, SK, HD, NH, gqa, causal, alibi, wl, wr, sc, chunk) in enumerate(CASES):
        for dt in DTS:
            q, k, v = gate_inputs(SQ, SK, HD, NH, gqa, dt)
            al = (-np.float32(2.0) ** (-(8.0 * np.arange(1, NH + 1, dtype=np.float32) / NH))
                  ).astype(np.float32) if alibi else None
            scale = np.float32(1.0) / np.sqrt(np.float32(HD))
            o_ref, l_ref = orc.reference_fwd(q, k, v, scale, causal, wl, wr, sc, al, chunk)
            o, l = orc.fwd(q, k, v, scale, causal, wl, wr, sc, al, chunk)
            assert np.abs(o - o_ref).max() <= 1e-6 * max(1.0, np.abs(o_ref).max()), name
            fin = np.isfinite(l_ref)
            assert np.array_equal(fin, np.isfinite(l)) and np.abs(l[fin] - l_ref[fin]).max() <= 1e-5, name
            key = f"c{i}_{dt}"
            out[key + "_meta"] = np.array([SQ, SK, HD, NH, gqa, int(causal), int(alibi), wl, wr,
                                           chunk], dtype=np.int64)
            out[key + "_softcap"] = np.array([sc], dtype=np.float32)
            # inputs are regenerated from the gate seed (gate_inputs); the fixture keeps the full
            # LSE and O at 64 sampled (head, row) pairs, always including the first/last rows
            rng = np.random.default_rng(1000 + i)
            hs = rng.integers(0, NH, 64)
            rs = rng.integers(0, SQ, 64)
            rs[:4] = [0, SQ - 1, min(63, SQ - 1), min(64, SQ - 1)]
            out[key + "_hs"] = hs.astype(np.int32)
            out[key + "_rs"] = rs.astype(np.int32)
            out[key + "_o"] = o_ref[0, hs, rs, :].astype(np.float32)
            out[key + "_lse"] = l_ref.astype(np.float32)
    path = os.path.join(os.path.dirname(os.path.abspath(__file__)), "fwd_golden.npz")
    np.savez_compressed(path, **out)
    print(f"wrote {path} ({os.path.getsize(path) / 1e6:.1f} MB, {len(CASES) * len(DTS)} cases)")


if __name__ == "__main__":
    main()
