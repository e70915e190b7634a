"""Shared helpers for the parity tests: seeded inputs, dtype maps, comparisons."""
import numpy as np

from oracle import oracle as orc

# rel_rms bounds vs the fp64 oracle (fp32 as the reference's gate,
# kernels/fa_forward_gate.inc:169)
TOL = {"f16": 5e-4, "bf16": 4e-3, "f32": 1e-5}
LSE_ABS = 1e-3                       # LSE absolute bound


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
