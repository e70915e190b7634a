"""Seeded random backward cases on the GPU against the fp64 oracle: head dims (multiples of 8 up
to 256), ragged SQ/SK, GQA, causal, windows, softcap and alibi in combinations the fixed cases
of test_bwd_gpu.py do not list, on both backward paths (dS workspace and recompute). The case
list is fixed by its seed; the bounds and the rounding-model floors are the fixed cases'
(tests/helpers.py check_grads), and repeated runs must agree bitwise."""
import numpy as np
import pytest

from tests.helpers import check_grads
from tests.test_bwd_gpu import PATHS, run, torch_equal

pytestmark = pytest.mark.gpu


def _cases(n=16, seed=1202):
    rng = np.random.default_rng(seed)
    out = []
    for i in range(n):
        D = int(rng.integers(1, 33)) * 8
        gqa = int(rng.choice([1, 2, 4]))
        Hk = int(rng.choice([1, 2]))
        B = int(rng.choice([1, 2]))
        SQ, SK = (int(x) for x in rng.integers(1, 257, 2))
        causal = bool(rng.random() < 0.5)
        wl = wr = -1
        if rng.random() < 0.3:
            wl = int(rng.integers(0, 200))
            wr = 0 if causal else int(rng.choice([-1, int(rng.integers(0, 200))]))
        sc = float(rng.choice([10.0, 30.0])) if rng.random() < 0.25 else 0.0
        alibi = bool(rng.random() < 0.2)
        name = (f"r{i} B{B} SQ{SQ} SK{SK} D{D} H{Hk * gqa}/{gqa} {'causal' if causal else 'full'}"
                f" w({wl},{wr}) sc{sc:g} al{int(alibi)}")
        out.append((name, B, Hk * gqa, Hk, SQ, SK, D, causal, wl, wr, sc, alibi))
    return out


CASES = _cases()


@pytest.mark.parametrize("path", list(PATHS))
@pytest.mark.parametrize("dt", ["f16", "bf16"])
@pytest.mark.parametrize("case", CASES, ids=[c[0] for c in CASES])
def test_backward_random(case, dt, path):
    print(f"[bwd-random] {case[0]} {dt} {path}", flush=True)
    res, ref, model = run(case, dt, seed=11, repeats=2, path=path)
    for i, name in enumerate(("dq", "dk", "dv")):
        assert torch_equal(res[1][i], res[0][i]), f"{name} differs between runs"
    check_grads("bwd_random_" + path, case[0], dt, res[0], ref, model)
