"""Seeded random paged-decode cases on the GPU against the fp64 decode oracle: head dims
(multiples of 8 up to 256), GQA ratios, ragged batches, page sizes, several new tokens with
append and rotary, windows, leftpad, softcap and alibi, in combinations the fixed cases of
test_decode_gpu.py do not list. The case list is fixed by its seed; the bounds are the fixed
cases' (rel_rms 5e-4 fp16 / 4e-3 bf16, LSE within 1e-3)."""
import numpy as np
import pytest

from tests.test_decode_gpu import check, make_case, run_kernel, run_oracle

pytestmark = pytest.mark.gpu


def _cases(n=16, seed=3202):
    rng = np.random.default_rng(seed)
    out = []
    for i in range(n):
        HD = int(rng.integers(1, 33)) * 8
        gqa = int(rng.choice([1, 2, 4, 8, 16]))
        NH = gqa * int(rng.choice([1, 2, 4]))
        page = int(rng.choice([16, 32, 64, 256]))
        ctxs = [int(x) for x in rng.integers(0, 1500, int(rng.integers(1, 5)))]
        nq = int(rng.choice([1, 1, 2, 4]))
        append = bool(rng.random() < 0.4)
        rotary = int(rng.choice([0, 0, 1, 2])) if HD % 2 == 0 else 0
        window = int(rng.integers(1, 400)) if rng.random() < 0.3 else -1
        leftpad = int(rng.integers(1, 64)) if rng.random() < 0.2 and min(ctxs) >= 64 else 0
        sc = float(rng.choice([20.0, 50.0])) if rng.random() < 0.25 else 0.0
        alibi = bool(rng.random() < 0.2)
        name = (f"r{i} HD{HD} H{NH}/{gqa} ctx{'-'.join(map(str, ctxs))} p{page} nq{nq}"
                f" app{int(append)} rot{rotary} w{window} lp{leftpad} sc{sc:g} al{int(alibi)}")
        out.append((name, HD, NH, gqa, ctxs, window, rotary, append, leftpad, nq, sc, alibi, page))
    return out


CASES = _cases()


@pytest.mark.parametrize("dt", ["f16", "bf16"])
@pytest.mark.parametrize("case", CASES, ids=[c[0] for c in CASES])
def test_decode_random(case, dt):
    print(f"[decode-random] {case[0]} {dt}", flush=True)
    c = make_case(case, dt, seed=5)
    o, l, _, _ = run_kernel(c, dt)
    o_ref, l_ref = run_oracle(c, dt)
    check(o, l, o_ref, l_ref, dt, case[0])
