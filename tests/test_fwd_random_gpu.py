"""Seeded random forward cases on the GPU against the fp64 oracle: head dims (multiples of 8 up
to 256, so every kernel width and its zero columns), ragged SQ/SK, GQA, causal, windows,
softcap, alibi and attention chunks in combinations the fixed cases of test_fwd_gpu.py do not
list. The case list is fixed by its seed, so a failure names a reproducible case; the bounds
are the same as the fixed cases' (rel_rms 5e-4 fp16 / 4e-3 bf16, LSE within 1e-3, empty rows
exactly zero)."""
import numpy as np
import pytest

from oracle import oracle as orc
from tests.helpers import LSE_ABS, TOL, log_errors, lse_err
from tests.test_fwd_gpu import run_case

pytestmark = pytest.mark.gpu


def _cases(n=24, seed=20261202):
    rng = np.random.default_rng(seed)
    out = []
    for i in range(n):
        D = int(rng.integers(1, 33)) * 8
        gqa = int(rng.choice([1, 2, 4]))
        H = gqa * int(rng.choice([1, 2, 4]))
        B = int(rng.choice([1, 2]))
        SQ, SK = (int(x) for x in rng.integers(1, 385, 2))
        causal = bool(rng.random() < 0.5)
        wl = wr = -1
        chunk = 0
        r = rng.random()
        if r < 0.3:  # a window: left bound, and a right one unless causal fixes it at 0
            wl = int(rng.integers(0, 300))
            wr = 0 if causal else int(rng.choice([-1, int(rng.integers(0, 300))]))
        elif r < 0.45:
            chunk = int(rng.integers(16, 301))
        sc = float(rng.choice([10.0, 30.0])) if rng.random() < 0.3 else 0.0
        alibi = bool(rng.random() < 0.2)
        name = (f"r{i} B{B} SQ{SQ} SK{SK} D{D} H{H}/{gqa} {'causal' if causal else 'full'}"
                f" w({wl},{wr}) sc{sc:g} al{int(alibi)} ch{chunk}")
        out.append((name, B, SQ, SK, D, H, gqa, causal, wl, wr, sc, alibi, chunk))
    return out


CASES = _cases()


@pytest.mark.parametrize("dt", ["f16", "bf16"])
@pytest.mark.parametrize("case", CASES, ids=[c[0] for c in CASES])
def test_forward_random(case, dt):
    print(f"[fwd-random] {case[0]} {dt}", flush=True)
    o, l, o_ref, l_ref = run_case(case, dt, seed=7)
    rel = orc.rel_rms(o, o_ref)
    lerr, inf_ok = lse_err(l, l_ref)
    log_errors("fwd_random", case[0], dt, o=rel, lse=lerr)
    assert np.isfinite(o).all(), "non-finite output"
    assert rel <= TOL[dt], f"rel_rms {rel:.3e} > {TOL[dt]}"
    assert inf_ok, "empty-row LSE (-inf) pattern differs"
    assert lerr <= LSE_ABS, f"LSE abs err {lerr:.3e}"
    empty = np.isneginf(l_ref)
    if empty.any():
        rows = np.broadcast_to(empty[..., None], o.shape)
        assert (o[rows] == 0).all(), "empty rows must be exactly zero"
