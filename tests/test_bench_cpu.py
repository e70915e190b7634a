"""bench.py's host logic on the CPU: the committed PMC tables under profiles/ cover the kernels
each benched workload reports traffic for, the summary modes parse what the GPU runs write,
and the multi-GPU refusal."""
import json
import os
import subprocess
import sys

import bench

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))


def test_profiles_cover_the_benched_kernels():
    # every workload whose roofline carries `traffic` finds its kernels in the committed tables
    for res in (bench.FWD_C2_KERNEL, bench.FWD_C1_KERNEL, bench.BWD_C3_KERNELS, bench.DEC_C4_KERNELS,
                bench.VARLEN_C5_KERNEL):
        t = bench.profiled_traffic(res)
        assert t is not None and t > 0, res
    # the forward's bytes cover at least Q, K, V read and O written once
    assert bench.profiled_traffic(bench.FWD_C2_KERNEL) >= 4 * 16384 * 32 * 128 * 2
    assert bench.profiled_traffic(bench.DEC_C4_KERNELS) >= 2 * 16 * 32768 * 8 * 128 * 2


def test_forward_traffic_only_for_profiled_shapes():
    assert bench._fwd_traffic(1, 16384, 32, 128, True) is not None
    assert bench._fwd_traffic(1, 1024, 8, 64, False) >= 4 * 1024 * 8 * 64 * 2   # C1
    assert bench._fwd_traffic(1, 8192, 32, 128, True) is None
    assert bench._fwd_traffic(1, 4096, 32, 128, True) is None


def test_roofline_fields():
    r = bench.roofline("mfma", 2.199e12, 2.2, 1.1e9)
    assert r["bound"] == "mfma" and r["unit"] == "TFLOP/s" and r["peak"] == 2500.0
    assert abs(r["frac"] - r["achieved"] / r["peak"]) < 1e-3 and r["traffic"] == 1.1e9
    h = bench.roofline("hbm", 2.147e9, 0.36)
    assert h["unit"] == "GB/s" and h["peak"] == 8000.0 and h["traffic"] is None


def test_parity_summary(tmp_path):
    f = tmp_path / "p.jsonl"
    rows = [{"test": "fwd", "case": "a", "dtype": "f16", "o": 2e-4, "lse": 1e-6},
            {"test": "bwd", "case": "b", "dtype": "bf16", "dq": 3e-3, "dq_model": 1e-4, "dq_floor": 2e-3,
             "dk": 1e-3, "dk_model": 1e-4, "dk_floor": 3e-3, "dv": 1e-3, "dv_model": 1e-4, "dv_floor": 1e-3}]
    f.write_text("".join(json.dumps(r) + "\n" for r in rows))
    t = bench.summarize_parity(str(f))
    assert "| fwd | f16 | 1 | 2.00e-04 (5e-04)" in t
    # dk's floor 3e-3 > 2/3 of 4e-3, so its bound is 1.5 x 3e-3 = 4.5e-3: 1e-3 is 22% of it
    assert "1.00e-03 (worst 22% of its bound)" in t
    assert "3.00e-03 (worst 75% of its bound)" in t
    # the raised bound is listed case by case, with whether the error exceeds the flat bound
    assert "Gradients held to 1.5x their floor instead of the flat bound: 1 (of 3" in t
    assert "| bwd | b | bf16 | dk | 1.00e-03 | 3.00e-03 | 4.50e-03 | no (4e-03) |" in t


def test_more_than_one_gpu_is_refused():
    r = subprocess.run([sys.executable, os.path.join(ROOT, "bench.py"), "--gpus", "2"],
                       capture_output=True, text=True, timeout=120)
    assert r.returncode != 0 and "one GPU" in r.stderr
