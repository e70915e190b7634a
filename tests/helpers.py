"""Shared helpers for the parity tests: seeded inputs, dtype maps, comparisons, and the
measured-error log (one JSON line per checked case)."""
import json
import os

import numpy as np

from oracle import oracle as orc

# rel_rms bounds vs the fp64 oracle (fp32 as the reference's gate,
# kernels/fa_forward_gate.inc:169)
TOL = {"f16": 5e-4, "bf16": 4e-3, "f32": 1e-5}
LSE_ABS = 1e-3                       # LSE absolute bound
# Gradients: rel_rms vs the exact fp64 gradients <= the BASELINE.json bounds GTOL (the
# reference's own gate allowed 2.5e-3 / 6e-3, kernels/backward.hip:734). Each case also runs the
# oracle's dtype rounding model (oracle.bwd(..., model=dt, stored_o=the kernel's O): D from the
# stored forward output, z*P and dS rounded to the dtype, as every 16-bit-operand backward that
# reads the stored O must compute them); its distance from the exact gradients is the case's
# floor. Where that floor exceeds 2/3 of GTOL (short causal rows, whose D carries the forward
# output's rounding into every dS of the row), the bound is FLOOR_MARGIN x the floor instead.
# Every case logs its error, its distance from the model and the floor.
GTOL = {"f16": 5e-4, "bf16": 4e-3}
FLOOR_MARGIN = 1.5


def torch_dtype(name):
    import torch
    return {"f16": torch.float16, "bf16": torch.bfloat16, "f32": torch.float32}[name]


def gen(shape, seed, dt):
    """N(0,1) data rounded to dt, as float32 numpy."""
    return orc.randn(shape, seed, dt)


def to_dev(a, dt, device="cuda"):
    import torch
    return torch.from_numpy(np.ascontiguousarray(a)).to(device=device, dtype=torch_dtype(dt))


def to_np(t):
    return t.detach().float().cpu().numpy()


def lse_err(got, ref):
    """max |got-ref| over finite entries; infinite entries must agree exactly (empty rows)."""
    got = np.asarray(got, dtype=np.float64)
    ref = np.asarray(ref, dtype=np.float64)
    inf_ok = bool(np.array_equal(np.isneginf(got), np.isneginf(ref)))
    fin = np.isfinite(ref)
    err = float(np.abs(got[fin] - ref[fin]).max()) if fin.any() else 0.0
    return err, inf_ok


_ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
ERROR_LOG = os.environ.get("FABLE_PARITY_LOG",
                           os.path.join(_ROOT, "gpurun_out", "parity_errors.jsonl"))


def log_errors(test, case, dtype, **errs):
    """Append the measured errors of one checked case (rel_rms of O / gradients, max |LSE|
    error, ...) as one JSON line to ERROR_LOG, so every run records the actual margins to the
    bounds, not only pass/fail."""
    rec = {"test": test, "case": case, "dtype": dtype}
    rec.update({k: (float(v) if v is not None else None) for k, v in errs.items()})
    os.makedirs(os.path.dirname(ERROR_LOG), exist_ok=True)
    with open(ERROR_LOG, "a") as f:
        f.write(json.dumps(rec) + "\n")


def check_grads(test, case_name, dt, got, ref, model, vanish_ok=False):
    """Assert the gradient bound above (vs the exact gradients `ref`, with the floor of the
    rounding model `model`) on (dq, dk, dv) and log the measured errors. `got` holds
    tensors or arrays in the layout of ref. With vanish_ok, a gradient that is exactly zero in
    exact arithmetic (a single visible key: dS = dP - D = 0) must only be tiny."""
    errs = {}
    for name, g, r, m in zip(("dq", "dk", "dv"), got, ref, model):
        g = g if isinstance(g, np.ndarray) else to_np(g)
        assert np.isfinite(g).all(), f"{name} not finite"
        if vanish_ok and not np.abs(r).max() > 0:
            assert np.abs(g).max() <= 1e-3, f"{name} should vanish"
            continue
        errs[name] = orc.rel_rms(g, r)
        errs[name + "_model"] = orc.rel_rms(g, m)
        errs[name + "_floor"] = orc.rel_rms(m, r)
    log_errors(test, case_name, dt, **errs)
    for name in ("dq", "dk", "dv"):
        if name not in errs:
            continue
        bound = max(GTOL[dt], FLOOR_MARGIN * errs[name + "_floor"])
        assert errs[name] <= bound, \
            f"{name} rel_rms {errs[name]:.3e} > {bound:.3e} (floor {errs[name + '_floor']:.3e})"
    return errs
