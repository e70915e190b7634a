"""Benchmark of the hot path on one MI355X (driver contract: one JSON line on stdout).

    python bench.py [--gpus 1] [--steps K] [--warmup W] [--no-cpu] [--extras fwd,bwd,decode,varlen,gemm]

(--extras: fwd = C2 at S=4096/8192 and C1; c2sizes and c1 name those parts alone; gemm = the fp16
GEMM calibration of the MFMA roofline, gemm_random its random-operand half alone.)

A step is one pass of the hot path over one batch of synthetic input:
  headline (`value`): BASELINE.json configs[1], causal fp16 forward through flash_attn_func,
  B=1, S=16384, H=32, D=128, q/k/v ~ N(0,1) resident in HBM before timing.
  TFLOP/s counts the causal half only: 2*B*H*S^2*D (reference convention,
  lab/bench_e2e.py:137-138).
`roofline` reports the dominant kernel (the forward kernel): algorithmic FLOP per launch divided
by its average duration, measured with HIP events on the stream the kernel is launched on
(torch's current stream), against the dense fp16 MFMA peak of 2.5 PFLOP/s; `traffic` is its HBM
bytes per launch from the calibrated rocprofv3 PMC tables under profiles/.
`cpu_baseline` times the exact fp32 torch reference (oracle/torch_ref.py) on the host cores over
a bounded sample of the same workload and scales to the metric's unit with the same numerator.
`extra` holds the other BASELINE.json configs (C1, C2 at S=4096/8192, C3 backward, C4 paged
decode, C5 varlen), each measured the same way (at least 3 untimed steps and 150 ms of untimed
load, then 20 timed steps; mean and median of the per-step HIP-event times) and each with its
own `roofline` block (over the whole step's kernels) and `cpu_baseline` (the same torch
reference path on CPU tensors: per-head autograd for C3, pages gathered per sequence for C4,
per sequence and head for C5); they are not the headline. `extra.gemm_fp16_calibration` is the
vendor GEMM (torch.matmul) on fp16 8192^3 with random and with constant operands: what a dense fp16
product sustains on the same box, since the chip holds a lower clock for random operands.
"""
import argparse
import json
import math
import os
import re
import sys
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path[:0] = [ROOT, os.path.join(ROOT, "flash-attention-rdna2_amd")]

PEAK_MFMA_TFLOPS = 2500.0   # MI355X dense fp16/bf16 MFMA
PEAK_HBM_GBS = 8000.0       # MI355X HBM3E
METRIC = "fwd/bwd TFLOP/s (% MFMA peak), paged decode GB/s (% HBM peak), 1×MI355X"


def log(*a):
    print(*a, file=sys.stderr, flush=True)


def time_steps(fn, steps, warmup, per_step=None, warm_ms=0.0):
    """Returns (wall ms/step, HIP-event ms/step) over exactly `steps` calls after `warmup`
    untimed calls, and after that as many more untimed calls as it takes to fill `warm_ms` of
    wall time (the clocks of an idle MI355X take ~40 ms of load to settle: a 20-step window
    right after idle read C5 at 363 -> 457 TFLOP/s and S=8192 at 805 -> 976 over its first
    50 ms). With a list as `per_step`, also appends each step's own HIP-event time to it (an
    event pair per step, recorded on the same stream, for medians)."""
    import torch
    t_warm = time.perf_counter()
    for _ in range(warmup):
        fn()
    torch.cuda.synchronize()
    while (time.perf_counter() - t_warm) * 1e3 < warm_ms:
        fn()
        torch.cuda.synchronize()
    st = torch.cuda.current_stream()
    ev_all = [torch.cuda.Event(enable_timing=True) for _ in range(steps + 1)]
    t0 = time.perf_counter()
    ev_all[0].record(st)
    for i in range(steps):
        fn()
        ev_all[i + 1].record(st)
    torch.cuda.synchronize()
    wall = (time.perf_counter() - t0) * 1e3 / steps
    ev = ev_all[0].elapsed_time(ev_all[-1]) / steps
    if per_step is not None:
        per_step += [ev_all[i].elapsed_time(ev_all[i + 1]) for i in range(steps)]
    return wall, ev


EXTRA_WARM_MS = 150.0   # untimed warm time of each extra config (not the headline)


def _median(x):
    x = sorted(x)
    return 0.5 * (x[(len(x) - 1) // 2] + x[len(x) // 2])


def roofline(bound, work, ms, traffic=None):
    """Roofline block of one step: algorithmic work (FLOP, or bytes for an HBM-bound step) over
    the step's HIP-event time, against the MI355X peak; traffic = calibrated HBM bytes per step
    from the committed PMC tables (None when no table covers the step's kernels)."""
    if bound == "mfma":
        ach, peak, unit = work / (ms * 1e-3) / 1e12, PEAK_MFMA_TFLOPS, "TFLOP/s"
    else:
        ach, peak, unit = work / (ms * 1e-3) / 1e9, PEAK_HBM_GBS, "GB/s"
    return {"bound": bound, "achieved": round(ach, 2), "peak": peak, "unit": unit,
            "frac": round(ach / peak, 4), "traffic": traffic}


def _cpu_threads():
    import torch
    cores = os.cpu_count() or 1
    torch.set_num_threads(cores)
    return cores


def bench_fwd(S, steps, warmup, causal=True, H=32, D=128, B=1, dtype="fp16", seed=0, warm_ms=0.0):
    import torch
    from fable_attn import flash_attn_func
    dt = torch.float16 if dtype == "fp16" else torch.bfloat16
    g = torch.Generator(device="cuda").manual_seed(seed)
    q = torch.randn(B, S, H, D, device="cuda", dtype=dt, generator=g)
    k = torch.randn(B, S, H, D, device="cuda", dtype=dt, generator=g)
    v = torch.randn(B, S, H, D, device="cuda", dtype=dt, generator=g)
    flops = 4.0 * B * H * S * S * D / (2 if causal else 1)
    per = []
    wall, ev = time_steps(lambda: flash_attn_func(q, k, v, causal=causal), steps, warmup, per, warm_ms)
    res = {"S": S, "H": H, "D": D, "B": B, "causal": causal, "dtype": dtype, "flops": flops,
           "ms": wall, "kernel_ms": ev, "tflops": flops / (wall * 1e-3) / 1e12,
           "kernel_tflops": flops / (ev * 1e-3) / 1e12, "kernel_ms_median": _median(per),
           "tflops_median": flops / (_median(per) * 1e-3) / 1e12,
           "roofline": roofline("mfma", flops, ev, _fwd_traffic(B, S, H, D, causal))}
    return res, (q, k, v)


def _fwd_traffic(B, S, H, D, causal):
    """Profiled HBM bytes per launch of a forward workload: only the profiled shapes (C2 at
    S=16384 and C1) have them; other sizes share a kernel symbol but not its bytes."""
    if (B, S, H, D, causal) == (1, 16384, 32, 128, True):
        return profiled_traffic(FWD_C2_KERNEL)
    if (B, S, H, D, causal) == (1, 1024, 8, 64, False):
        return profiled_traffic(FWD_C1_KERNEL)
    return None


def bench_gemm(steps, warmup, n=8192, seed=0, warm_ms=EXTRA_WARM_MS, kinds=("random", "constant")):
    """Calibration of the MFMA roofline on the box: the vendor GEMM (torch.matmul, hipBLASLt)
    on fp16 n x n x n, with N(0, 1) operands like the attention workloads and with constant
    ones. The matrix cores draw more power on random operands, and the chip holds a lower clock
    for them (measured ~1.8 GHz against ~2.3 GHz for constant operands): the random-operand rate
    is what a dense fp16 product sustains here, against the 2.5 PFLOP/s nameplate (2.4 GHz)."""
    import torch
    g = torch.Generator(device="cuda").manual_seed(seed)
    flops = 2.0 * n ** 3
    res = {"n": n, "dtype": "fp16", "flops": flops}
    for kind in kinds:
        if kind == "random":
            a = torch.randn(n, n, device="cuda", dtype=torch.float16, generator=g)
            b = torch.randn(n, n, device="cuda", dtype=torch.float16, generator=g)
        else:
            a = torch.full((n, n), 0.001, device="cuda", dtype=torch.float16)
            b = a.clone()
        per = []
        _, ev = time_steps(lambda: a @ b, steps, warmup, per, warm_ms)
        res[f"{kind}_tflops"] = flops / (_median(per) * 1e-3) / 1e12
        res[f"{kind}_frac"] = round(res[f"{kind}_tflops"] / PEAK_MFMA_TFLOPS, 4)
        del a, b
    return res


def bench_bwd(steps, warmup, B=2, S=4096, H=32, D=128, seed=0, warm_ms=EXTRA_WARM_MS, cpu_heads=0):
    """C3: causal bf16 backward, timed without the forward; bitwise-identical check over 3 runs."""
    import torch
    from fable_attn import _C
    from fable_attn.flash_attn_interface import _bhsd
    dt = torch.bfloat16
    g = torch.Generator(device="cuda").manual_seed(seed)
    q, k, v, do = (torch.randn(B, S, H, D, device="cuda", dtype=dt, generator=g) for _ in range(4))
    qh, kh, vh, doh = (_bhsd(x) for x in (q, k, v, do))
    scale = D ** -0.5
    out, lse = _C.fwd(qh, kh, vh, scale, True, -1, 0, 0.0, None, 0.0, 0)

    def step():
        return _C.bwd(doh, qh, kh, vh, out, lse, scale, True, -1, 0, 0.0, None, 0.0, 0)
    ref = step()
    same = all(all(torch.equal(a, b) for a, b in zip(ref, step())) for _ in range(2))
    per = []
    wall, ev = time_steps(step, steps, warmup, per, warm_ms)
    flops = 2.5 * 4.0 * B * H * S * S * D / 2
    res = {"B": B, "S": S, "H": H, "D": D, "dtype": "bf16", "flops": flops, "ms": wall,
           "kernel_ms": ev, "tflops": flops / (wall * 1e-3) / 1e12,
           "kernel_ms_median": _median(per), "tflops_median": flops / (_median(per) * 1e-3) / 1e12,
           "bitwise_identical_x3": bool(same),
           "roofline": roofline("mfma", flops, ev, profiled_traffic(BWD_C3_KERNELS))}
    if cpu_heads:
        res["cpu_baseline"] = cpu_bwd(q, k, v, do, cpu_heads)
    return res


def cpu_bwd(q, k, v, do, heads):
    """C3 on the CPU: torch autograd through the exact fp32 reference on the run's own inputs
    (copied to the host once, untimed), one (batch, head) at a time, `heads` of the B*H heads;
    the rate uses C3's numerator (2.5x the causal forward)."""
    from oracle.torch_ref import attention_bhsd
    cores = _cpu_threads()
    B, S, H, D = q.shape
    pairs = [(b, h) for b in range(B) for h in range(H)][:heads]
    # the sampled heads of the run's tensors, [1, 1, S, D] fp32 each (host copies, untimed)
    host = [tuple(x[b, :, h].float().cpu()[None, None] for x in (q, k, v, do)) for b, h in pairs]
    t0 = time.perf_counter()
    for qh, kh, vh, doh in host:
        qs, ks, vs = (x.clone().requires_grad_() for x in (qh, kh, vh))
        attention_bhsd(qs, ks, vs, D ** -0.5, causal=True).backward(doh)
    dt = time.perf_counter() - t0
    flops = 2.5 * 4.0 * len(pairs) * S * S * D / 2
    return {"value": flops / dt / 1e12, "unit": "TFLOP/s", "cores": cores, "kind": "port",
            "sample": f"{len(pairs)} of {B * H} (batch, head) pairs of the run's own causal S={S} "
                      f"D={D} inputs (forward + autograd of the fp32 torch reference on CPU "
                      f"tensors), {dt:.1f} s; extrapolated linearly to all heads"}


def bench_decode(steps, warmup, batch=16, Hq=32, Hk=8, D=128, ctx=32768, page=256, seed=0,
                 cpu_seqs=0):
    """C4: paged-KV decode fp16, block_table = seeded permutation of the physical pages."""
    import torch
    from fable_attn import flash_attn_with_kvcache
    dt = torch.float16
    nblk = batch * ctx // page
    g = torch.Generator(device="cuda").manual_seed(seed)
    kc = torch.randn(nblk, page, Hk, D, device="cuda", dtype=dt, generator=g)
    vc = torch.randn(nblk, page, Hk, D, device="cuda", dtype=dt, generator=g)
    q = torch.randn(batch, 1, Hq, D, device="cuda", dtype=dt, generator=g)
    cg = torch.Generator().manual_seed(seed)
    bt = torch.randperm(nblk, generator=cg).view(batch, ctx // page).int().cuda()
    cs = torch.full((batch,), ctx, dtype=torch.int32, device="cuda")
    f = lambda: flash_attn_with_kvcache(q, kc, vc, cache_seqlens=cs, block_table=bt)
    per = []
    wall, ev = time_steps(f, steps, warmup, per, EXTRA_WARM_MS)
    nbytes = 2.0 * batch * ctx * Hk * D * 2
    res = {"batch": batch, "Hq": Hq, "Hk": Hk, "D": D, "ctx": ctx, "page": page, "bytes": nbytes,
           "ms": wall, "kernel_ms": ev, "GBs": nbytes / (wall * 1e-3) / 1e9,
           "kernel_ms_median": _median(per), "GBs_median": nbytes / (_median(per) * 1e-3) / 1e9,
           "frac_hbm": nbytes / (wall * 1e-3) / 1e9 / PEAK_HBM_GBS,
           "roofline": roofline("hbm", nbytes, ev, profiled_traffic(DEC_C4_KERNELS))}
    if cpu_seqs:
        res["cpu_baseline"] = cpu_decode(q, kc, vc, bt, ctx, page, cpu_seqs, nbytes / batch)
    return res


def cpu_decode(q, kc, vc, bt, ctx, page, seqs, bytes_per_seq):
    """C4 on the CPU: for `seqs` sequences, their pages are gathered into dense K/V (untimed,
    as a CPU cache would hold them) and the exact fp32 torch reference attends one query token
    over the ctx keys; the rate uses C4's numerator (K+V bytes in fp16)."""
    import torch
    from oracle.torch_ref import attention_bhsd
    cores = _cpu_threads()
    Hq, D = q.shape[2], q.shape[3]
    dt = 0.0
    for b in range(seqs):
        pages = bt[b].long()
        kb = kc[pages].reshape(-1, kc.shape[2], D)[:ctx].float().cpu().transpose(0, 1)[None]
        vb = vc[pages].reshape(-1, vc.shape[2], D)[:ctx].float().cpu().transpose(0, 1)[None]
        qb = q[b].float().cpu().transpose(0, 1)[None]                  # [1, Hq, 1, D]
        t0 = time.perf_counter()
        attention_bhsd(qb, kb, vb, D ** -0.5)
        dt += time.perf_counter() - t0
    return {"value": bytes_per_seq * seqs / dt / 1e9, "unit": "GB/s", "cores": cores,
            "kind": "port",
            "sample": f"{seqs} of {bt.shape[0]} sequences (ctx {ctx}, {Hq} q heads, D={D}), pages "
                      f"gathered to dense fp32 K/V untimed, fp32 torch reference on CPU tensors, "
                      f"{dt:.2f} s; GB/s of the fp16 K/V bytes those sequences read"
                      + ("; extrapolated linearly to all sequences" if seqs < bt.shape[0] else "")}


def bench_varlen(steps, warmup, H=16, D=256, seed=0, cpu_heads=0):
    """C5: varlen bf16, 8 sequences with lengths ~U[512, 8192] (seeded), window (512,0) +
    causal, softcap 30; FLOP counts exact unmasked pairs."""
    import torch
    from fable_attn import flash_attn_varlen_func
    cg = torch.Generator().manual_seed(seed)
    lens = torch.randint(512, 8193, (8,), generator=cg).tolist()
    cu = torch.tensor([0] + list(__import__("itertools").accumulate(lens)), dtype=torch.int32, device="cuda")
    T = sum(lens)
    g = torch.Generator(device="cuda").manual_seed(seed)
    q, k, v = (torch.randn(T, H, D, device="cuda", dtype=torch.bfloat16, generator=g) for _ in range(3))
    f = lambda: flash_attn_varlen_func(q, k, v, cu, cu, max(lens), max(lens), causal=True,
                                       window_size=(512, 0), softcap=30.0, softmax_scale=D ** -0.5)
    per = []
    wall, ev = time_steps(f, steps, warmup, per, EXTRA_WARM_MS)
    pairs = sum(sum(min(i, 512) + 1 for i in range(L)) for L in lens)
    flops = 4.0 * D * H * pairs
    res = {"lens": lens, "H": H, "D": D, "flops": flops, "ms": wall, "kernel_ms": ev,
           "tflops": flops / (wall * 1e-3) / 1e12, "kernel_ms_median": _median(per),
           "tflops_median": flops / (_median(per) * 1e-3) / 1e12,
           "roofline": roofline("mfma", flops, ev, profiled_traffic(VARLEN_C5_KERNEL))}
    if cpu_heads:
        res["cpu_baseline"] = cpu_varlen(q, k, v, lens, cpu_heads, H, D)
    return res


def cpu_varlen(q, k, v, lens, heads, H, D):
    """C5 on the CPU: every sequence, `heads` of its H heads, through the exact fp32 torch
    reference (window (512, 0), causal, softcap 30) on CPU tensors; the rate uses C5's
    numerator (exact visible pairs), extrapolated from the sampled heads to all H."""
    import torch
    from oracle.torch_ref import attention_bhsd
    cores = _cpu_threads()
    dt, pairs, a = 0.0, 0, 0
    for L in lens:
        sl = lambda t: t[a:a + L, :heads].float().cpu().transpose(0, 1)[None]  # [1, heads, L, D]
        qs, ks, vs = sl(q), sl(k), sl(v)
        t0 = time.perf_counter()
        attention_bhsd(qs, ks, vs, D ** -0.5, causal=True, win_left=512, win_right=0, softcap=30.0)
        dt += time.perf_counter() - t0
        pairs += sum(min(i, 512) + 1 for i in range(L))
        a += L
    flops = 4.0 * D * heads * pairs
    return {"value": flops / dt / 1e12, "unit": "TFLOP/s", "cores": cores, "kind": "port",
            "sample": f"all {len(lens)} sequences, {heads} of {H} heads (D={D}, window 512 + causal "
                      f"+ softcap 30), fp32 torch reference on CPU tensors, {dt:.1f} s; "
                      f"extrapolated linearly to all heads"}


# ---- rocprofv3 summaries (CPU only: they read the CSV files rocprofv3 wrote) ----------------

PROFILES = os.path.join(ROOT, "profiles")
COPY_KERNEL = "__amd_rocclr_copyBuffer"
COPY_CALIB_BYTES = 1 << 30   # --copy-calib copies 1 GiB device to device


def _rocprof_rows(d, suffix):
    import csv
    import glob
    rows = []
    for f in sorted(glob.glob(os.path.join(d, "**", "*" + suffix), recursive=True)):
        with open(f, newline="") as fh:
            rows += list(csv.DictReader(fh))
    if not rows:
        raise SystemExit(f"no *{suffix} under {d}")
    return rows


def summarize_pmc(fetch_dir, write_dir, kernel_re=None):
    """Markdown table of FETCH_SIZE / WRITE_SIZE per dispatch (KiB, averaged per kernel) from
    two `rocprofv3 --pmc` runs of `bench.py --copy-calib`, and HBM bytes per dispatch scaled by
    what each counter reads for the 1 GiB calibration copy (its largest copyBuffer dispatch)."""
    per = {}
    factor = {}
    for d, ctr in ((fetch_dir, "FETCH_SIZE"), (write_dir, "WRITE_SIZE")):
        vals = {}
        for r in _rocprof_rows(d, "counter_collection.csv"):
            if r["Counter_Name"] == ctr:
                vals.setdefault(r["Kernel_Name"], []).append(float(r["Counter_Value"]))
        copy = max(vals.get(COPY_KERNEL, [0.0]))
        if copy <= 0:
            raise SystemExit(f"{d}: no {COPY_KERNEL} dispatch (run bench.py with --copy-calib)")
        factor[ctr] = COPY_CALIB_BYTES / (copy * 1024.0)
        for k, v in vals.items():
            per.setdefault(k, {})[ctr] = (len(v), sum(v) / len(v))
    out = ["| kernel | dispatches | FETCH_SIZE KiB/dispatch | WRITE_SIZE KiB/dispatch | "
           "HBM bytes/dispatch (calibrated) |", "|---|---|---|---|---|"]
    for k, c in sorted(per.items(), key=lambda kv: -kv[1].get("FETCH_SIZE", (0, 0.0))[1]):
        if "FETCH_SIZE" not in c or "WRITE_SIZE" not in c or k == COPY_KERNEL:
            continue
        if kernel_re and not re.search(kernel_re, k):
            continue
        f, w = c["FETCH_SIZE"][1], c["WRITE_SIZE"][1]
        hbm = f * 1024 * factor["FETCH_SIZE"] + w * 1024 * factor["WRITE_SIZE"]
        out.append(f"| `{k}` | {c['FETCH_SIZE'][0]} | {f:.1f} | {w:.1f} | {hbm:.0f} |")
    out.append("")
    out.append(f"Calibration (1 GiB `{COPY_KERNEL}`): FETCH_SIZE x{factor['FETCH_SIZE']:.4f}, "
               f"WRITE_SIZE x{factor['WRITE_SIZE']:.4f} (bytes per KiB-count / 1024).")
    return "\n".join(out)


def summarize_mfma(d, kernel_re=None):
    """Markdown table of matrix-core utilisation per kernel from a `rocprofv3 --pmc
    SQ_VALU_MFMA_BUSY_CYCLES GRBM_GUI_ACTIVE` run. SQ_VALU_MFMA_BUSY_CYCLES sums the busy
    cycles of every SIMD's matrix core; GRBM_GUI_ACTIVE sums the active cycles of every XCD, so
    GRBM_GUI_ACTIVE / Num_Xcc / duration is the dispatch's mean clock. Utilisation at that
    clock = busy / (Simd_Count x active cycles per XCD); at the peak clock = busy /
    (Simd_Count x duration x Max_Engine_Clk_Fcompute)."""
    agent = [r for r in _rocprof_rows(d, "agent_info.csv") if int(r.get("Simd_Count") or 0) > 0][0]
    simds, nxcc = int(agent["Simd_Count"]), int(agent["Num_Xcc"])
    fmax_ghz = float(agent["Max_Engine_Clk_Fcompute"]) / 1e3
    disp = {}
    for r in _rocprof_rows(d, "counter_collection.csv"):
        if kernel_re and not re.search(kernel_re, r["Kernel_Name"]):
            continue
        e = disp.setdefault((r["Kernel_Name"], r["Dispatch_Id"]), {})
        e[r["Counter_Name"]] = float(r["Counter_Value"])
        e["ns"] = int(r["End_Timestamp"]) - int(r["Start_Timestamp"])
    per = {}
    for (k, _), e in disp.items():
        if "SQ_VALU_MFMA_BUSY_CYCLES" in e and e.get("GRBM_GUI_ACTIVE", 0) > 0 and e["ns"] > 0:
            per.setdefault(k, []).append(e)
    out = [f"| kernel | dispatches | average us | mean clock GHz | MFMA busy at that clock | "
           f"MFMA busy at {fmax_ghz:.1f} GHz |", "|---|---|---|---|---|---|"]
    for k, es in sorted(per.items(), key=lambda kv: -sum(e["ns"] for e in kv[1])):
        busy = sum(e["SQ_VALU_MFMA_BUSY_CYCLES"] for e in es)
        cyc = sum(e["GRBM_GUI_ACTIVE"] for e in es) / nxcc
        ns = sum(e["ns"] for e in es)
        out.append(f"| `{k}` | {len(es)} | {ns / len(es) / 1e3:.1f} | {cyc / ns:.2f} | "
                   f"{busy / (simds * cyc):.1%} | {busy / (simds * ns * fmax_ghz):.1%} |")
    out.append("")
    out.append(f"Agent: {simds} SIMDs, {nxcc} XCDs, peak engine clock {fmax_ghz:.1f} GHz.")
    return "\n".join(out)


def summarize_counters(dirs, kernel_re):
    """Markdown table of every counter of one or more `rocprofv3 --pmc` runs, averaged per
    dispatch of the kernels matching `kernel_re`, with the ratios used to rank what limits a
    kernel: mean clock, matrix-core busy share, VALU-and-MFMA co-execution share, instructions
    per MFMA, and the wave-cycle shares spent waiting."""
    agent = [r for r in _rocprof_rows(dirs[0], "agent_info.csv") if int(r.get("Simd_Count") or 0) > 0][0]
    simds, nxcc = int(agent["Simd_Count"]), int(agent["Num_Xcc"])
    acc, ns = {}, {}
    for d in dirs:
        for r in _rocprof_rows(d, "counter_collection.csv"):
            if not re.search(kernel_re, r["Kernel_Name"]):
                continue
            acc.setdefault(r["Counter_Name"], []).append(float(r["Counter_Value"]))
            ns.setdefault((d, r["Dispatch_Id"]), int(r["End_Timestamp"]) - int(r["Start_Timestamp"]))
    avg = {c: sum(v) / len(v) for c, v in acc.items()}
    out = ["| counter | average per dispatch |", "|---|---|"]
    out += [f"| {c} | {v:.4g} |" for c, v in sorted(avg.items())]
    out += ["", "| derived | value |", "|---|---|"]
    t = sum(ns.values()) / len(ns)
    g = avg.get("GRBM_GUI_ACTIVE")
    if g:
        cyc = g / nxcc
        out.append(f"| mean clock (GRBM_GUI_ACTIVE per XCD / duration) | {cyc / t:.2f} GHz |")
        for c, label in (("SQ_VALU_MFMA_BUSY_CYCLES", "matrix cores busy"),
                         ("SQ_VALU_MFMA_COEXEC_CYCLES", "VALU and matrix cores busy together")):
            if c in avg:
                out.append(f"| {label} (share of SIMD cycles) | {avg[c] / (simds * cyc):.1%} |")
    m = avg.get("SQ_INSTS_MFMA")
    if m:
        for c in ("SQ_INSTS_VALU", "SQ_INSTS_VALU_TRANS_F32", "SQ_INSTS_LDS", "SQ_INSTS_SALU"):
            if c in avg:
                out.append(f"| {c} per MFMA instruction | {avg[c] / m:.2f} |")
    w = avg.get("SQ_WAVE_CYCLES")
    if w:
        for c in ("SQ_WAIT_ANY", "SQ_WAIT_INST_ANY", "SQ_WAIT_INST_LDS", "SQ_ACTIVE_INST_VALU",
                  "SQ_ACTIVE_INST_LDS"):
            if c in avg:
                out.append(f"| {c} / SQ_WAVE_CYCLES | {avg[c] / w:.1%} |")
    out.append("")
    out.append(f"Agent: {simds} SIMDs, {nxcc} XCDs; {len(ns)} dispatches, {t / 1e3:.1f} us average "
               f"(counter collection slows a dispatch; read the ratios).")
    return "\n".join(out)


def summarize_stats(d, kernel_re=None, skip=0, last=0):
    """Markdown table of the `rocprofv3 --kernel-trace --stats` kernel statistics, with the
    average over the dispatches after the first `skip` of each kernel (bench.py's warmup calls),
    or over the last `last` dispatches of each (bench.py's timed steps come last), from the
    kernel trace: the dispatches bench.py's HIP-event average covers."""
    trace = {}
    for r in _rocprof_rows(d, "kernel_trace.csv"):
        trace.setdefault(r["Kernel_Name"], []).append(
            (int(r["Start_Timestamp"]), int(r["End_Timestamp"]) - int(r["Start_Timestamp"])))
    col = f"average us of the last {last}" if last else f"average us after {skip}"
    out = [f"| kernel | calls | average us | min us | max us | % of GPU time | {col} |",
           "|---|---|---|---|---|---|---|"]
    for r in _rocprof_rows(d, "kernel_stats.csv"):
        if kernel_re and not re.search(kernel_re, r["Name"]):
            continue
        ds = [t for _, t in sorted(trace.get(r["Name"], []))]
        ds = ds[-last:] if last else ds[skip:]
        after = f"{sum(ds) / len(ds) / 1e3:.1f}" if ds else "-"
        out.append(f"| `{r['Name']}` | {r['Calls']} | {float(r['AverageNs']) / 1e3:.1f} | "
                   f"{float(r['MinNs']) / 1e3:.1f} | {float(r['MaxNs']) / 1e3:.1f} | "
                   f"{float(r['Percentage']):.2f} | {after} |")
    return "\n".join(out)


# kernel symbols of the measured workloads, as regexes over the mangled names in the PMC
# tables (the headline's kernel; the kernels of one C3, C4 or C5 step)
FWD_C2_KERNEL = r"_ZN2fa10fwd_kernelIDF16_NS_6FwdCfgILi128ELi64ELi8ELi2ELi1EEELb1ELb0ELb0EEEv14FableFwdParamsiNS_8FwdSplitE"
# C1 takes the key split: the split kernel, then the merge of its partials
FWD_C1_KERNEL = (r"_ZN2fa10fwd_kernelIDF16_NS_6FwdCfgILi64E.*ELb0ELb0ELb0EEEv14FableFwdParamsiNS_8FwdSplitE",
                 r"_ZN2fa24fwd_split_combine_kernelIDF16_Li[0-9]+EEEv14FableFwdParamsNS_8FwdSplitE")
BWD_C3_KERNELS = (r"_ZN2fa15bwd_dsum_kernelIDF16b.*", r"_ZN2fa20bwd_dkdv_pair_kernelIDF16b.*",
                  r"_ZN2fa16bwd_dq_ds_kernelIDF16b.*")
DEC_C4_KERNELS = (r"_ZN2fa18dec_partial_kernelIDF16_Li128ELb0ELb1EEEv14FableDecParamsiii",
                  r"_ZN2fa18dec_combine_kernelIDF16_Li128ELi[0-9]+EEEv14FableDecParams")
VARLEN_C5_KERNEL = r"_ZN2fa10fwd_kernelIDF16bNS_6FwdCfgILi256E.*ELb1ELb1ELb0EEEv14FableFwdParamsiNS_8FwdSplitE"


def summarize_parity(path):
    """Markdown table of the measured parity errors that the GPU tests log (one JSON line per
    checked case, tests/helpers.py:log_errors), grouped by test and dtype: cases, the largest
    rel_rms of O, the largest |LSE| error, and per gradient the largest rel_rms with the bound
    it was held to (the BASELINE.json bound, or 1.5x the case's rounding-model floor where that
    floor exceeds 2/3 of it) and the largest floor."""
    import json
    tol = {"f16": 5e-4, "bf16": 4e-3, "f32": 1e-5}
    gtol = {"f16": 5e-4, "bf16": 4e-3, "f32": 1e-4}
    groups = {}
    for line in open(path):
        line = line.strip()
        if line:
            r = json.loads(line)
            groups.setdefault((r["test"], r["dtype"]), []).append(r)

    def worst(rs, key):
        v = [r[key] for r in rs if r.get(key) is not None]
        return max(v) if v else None

    def fmt(x):
        return "-" if x is None else f"{x:.2e}"

    out = ["| test | dtype | cases | O rel_rms (bound) | LSE abs (bound 1e-3) | dQ | dK | dV | "
           "largest gradient floor |", "|---|---|---|---|---|---|---|---|---|"]
    for (test, dt), rs in sorted(groups.items()):
        o = worst(rs, "o")
        ocol = "-" if o is None else f"{o:.2e} ({tol.get(dt, 0):.0e})"
        cols = []
        for g in ("dq", "dk", "dv"):
            e = [(r[g], max(gtol[dt], 1.5 * r[g + "_floor"]) if (r.get(g + "_floor") or 0) > gtol[dt] * 2 / 3
                  else gtol[dt]) for r in rs if r.get(g) is not None]
            if not e:
                cols.append("-")
                continue
            m = max(e, key=lambda t: t[0] / t[1])
            cols.append(f"{max(x for x, _ in e):.2e} (worst {m[0] / m[1]:.0%} of its bound)")
        fl = [r[g + "_floor"] for r in rs for g in ("dq", "dk", "dv") if r.get(g + "_floor") is not None]
        out.append(f"| {test} | {dt} | {len(rs)} | {ocol} | {fmt(worst(rs, 'lse'))} | "
                   + " | ".join(cols) + f" | {fmt(max(fl) if fl else None)} |")
    # every gradient whose bound is not the flat one (floor above 2/3 of it)
    raised = []
    for (test, dt), rs in sorted(groups.items()):
        for r in rs:
            for g in ("dq", "dk", "dv"):
                f = r.get(g + "_floor")
                if r.get(g) is not None and f is not None and f > gtol[dt] * 2 / 3:
                    raised.append((test, r.get("case", ""), dt, g, r[g], f, 1.5 * f, gtol[dt]))
    out += ["", f"Gradients held to 1.5x their floor instead of the flat bound: {len(raised)} "
            f"(of {sum(1 for rs in groups.values() for r in rs for g in ('dq', 'dk', 'dv') if r.get(g) is not None)} "
            "checked gradients).", ""]
    if raised:
        out += ["| test | case | dtype | gradient | rel_rms | floor | bound (1.5x floor) | "
                "above the flat bound |", "|---|---|---|---|---|---|---|---|"]
        for test, case, dt, g, e, f, b, flat in raised:
            out.append(f"| {test} | {case} | {dt} | {g} | {e:.2e} | {f:.2e} | {max(b, flat):.2e} | "
                       f"{'yes' if e > flat else 'no'} ({flat:.0e}) |")
    return "\n".join(out)


def profiled_traffic(kernel_res):
    """Calibrated HBM bytes per step summed over the kernels matching `kernel_res` (one regex or
    a tuple, one kernel each) from the PMC tables committed under profiles/; None if a kernel
    is in no table (each table comes from one run of this bench.py)."""
    import glob
    res = (kernel_res,) if isinstance(kernel_res, str) else tuple(kernel_res)
    rows = []
    for f in sorted(glob.glob(os.path.join(PROFILES, "*pmc*.md"))):
        for line in open(f):
            m = re.match(r"\| `([^`]+)` \| \d+ \| [\d.]+ \| [\d.]+ \| (\d+) \|", line)
            if m:
                rows.append((m.group(1), int(m.group(2))))
    total = 0
    for r in res:
        hit = [b for name, b in rows if re.fullmatch(r, name)]
        if not hit:
            return None
        total += hit[0]
    return total


def cpu_baseline(inputs, heads=32, causal=True):
    """Exact fp32 torch reference on the host cores over the run's own inputs (q, k, v of
    batch element 0, copied to the host once, untimed), `heads` of the H heads of the forward
    workload, one head at a time to bound memory, scaled to the full workload's FLOP rate (the
    causal half for causal, as the GPU figure)."""
    from oracle.torch_ref import attention_bhsd
    cores = _cpu_threads()
    q, k, v = inputs
    B, S, H, D = q.shape
    heads = min(heads, H)
    host = [tuple(x[0, :, h].float().cpu()[None, None] for x in (q, k, v)) for h in range(heads)]
    qh, kh, vh = host[0]
    attention_bhsd(qh[:, :, :256], kh[:, :, :256], vh[:, :, :256], D ** -0.5, causal=causal)  # warm
    t0 = time.perf_counter()
    for qh, kh, vh in host:
        attention_bhsd(qh, kh, vh, D ** -0.5, causal=causal)
    dt = time.perf_counter() - t0
    flops = 4.0 * heads * S * S * D / (2 if causal else 1)
    return {"value": flops / dt / 1e12, "unit": "TFLOP/s", "cores": cores, "kind": "port",
            "sample": f"{heads} of {B * H} heads of the run's own {'causal' if causal else 'non-causal'} "
                      f"S={S} D={D} forward inputs, fp32 torch reference on CPU tensors, {dt:.1f} s"
                      + ("; extrapolated linearly to all heads" if heads < B * H else "")}


# shapes of the rate sweep: (B, S, Hq, Hk, D, causal); the forward in fp16, the backward in bf16
SWEEP_FWD = [(1, 1024, 8, 8, 64, False), (1, 2048, 8, 8, 128, True), (1, 4096, 8, 8, 128, True),
             (1, 8192, 4, 4, 128, True), (1, 4096, 32, 32, 128, True), (1, 8192, 32, 32, 128, True),
             (1, 16384, 32, 32, 128, True), (4, 2048, 16, 16, 128, False), (1, 16384, 8, 8, 128, False),
             (2, 2048, 16, 16, 64, True), (1, 4096, 16, 16, 256, True), (1, 8192, 32, 8, 128, True),
             (2, 4096, 32, 32, 64, False), (1, 16384, 32, 32, 64, True), (8, 1024, 16, 16, 64, False),
             (2, 4096, 32, 32, 32, False), (2, 4096, 32, 32, 96, True), (8, 2048, 32, 32, 128, True),
             (8, 2048, 32, 32, 96, True), (8, 2048, 32, 32, 32, True), (4, 4096, 32, 32, 64, True),
             (64, 512, 32, 32, 128, True)]
# paged decode: (batch, ctx, page); (1, 32768, 32) is the shape of the reference's published decode
# figure, (16, 32768, 256) is C4
SWEEP_DEC = [(1, 32768, 32), (1, 32768, 256), (1, 131072, 256), (4, 32768, 256), (16, 32768, 256),
             (64, 8192, 256), (128, 2048, 16)]
SWEEP_BWD = [(2, 4096, 32, 32, 128, True), (1, 4096, 8, 8, 128, True), (1, 4096, 32, 8, 128, True),
             (1, 8192, 8, 8, 128, True), (2, 2048, 16, 16, 128, False), (1, 2048, 16, 16, 64, True),
             (1, 4096, 16, 16, 256, True), (2, 2048, 16, 16, 192, False), (2, 4096, 32, 32, 64, True),
             (2, 4096, 32, 32, 64, False), (2, 4096, 32, 32, 32, True), (2, 4096, 32, 32, 96, True),
             (64, 512, 32, 32, 128, True), (16, 1024, 32, 32, 128, True), (16, 2048, 32, 32, 128, True)]


def sweep(reps=5, inner=10):
    """Markdown tables of forward (fp16) and backward (bf16, dS workspace) rates through the
    binding the public API uses (fable_attn._C.fwd / bwd), per shape: the median of `reps`
    HIP-event timings of `inner` back-to-back calls, and whether the small-grid split applies
    (forward: key split; backward: query split of the dK/dV kernel); and of paged decode
    (flash_attn_with_kvcache) from graph replays."""
    import torch
    from fable_attn import _C, _lib

    def timed(fn):
        for _ in range(3):
            fn()
        ts = []
        for _ in range(reps):
            e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
            e0.record()
            for _ in range(inner):
                fn()
            e1.record()
            torch.cuda.synchronize()
            ts.append(e0.elapsed_time(e1) / inner)
        return _median(ts)

    g = torch.Generator(device="cuda").manual_seed(0)
    out = ["| pass | B | S | Hq / Hk | D | causal | dtype | ms per call | TFLOP/s | split |",
           "|---|---|---|---|---|---|---|---|---|---|"]
    for pas, shapes, dt in (("forward", SWEEP_FWD, torch.float16), ("backward", SWEEP_BWD, torch.bfloat16)):
        for B, S, Hq, Hk, D, causal in shapes:
            mk = lambda H: torch.randn(B, S, H, D, device="cuda", dtype=dt, generator=g).transpose(1, 2)
            q, k, v = mk(Hq), mk(Hk), mk(Hk)
            sc = D ** -0.5
            fl = 4.0 * B * Hq * S * S * D * (0.5 if causal else 1.0)
            st = lambda t: _lib.Strides(t.stride(0), t.stride(1), t.stride(2))
            if pas == "forward":
                p = _lib.FableFwdParams(None, None, None, None, None, st(q), st(k), st(v), st(q), S, S, D, Hq,
                                        Hq // Hk, sc, 0.0, -1, -1, None, int(causal), 0.0, 0, None, None, B,
                                        0, None, None, Hq * S, S)
                split = _C._L.fable_attn_fwd_ws_bytes(p, 0) > 0
                ms = timed(lambda: _C.fwd(q, k, v, sc, causal, -1, -1, 0.0, None, 0.0, 0))
            else:
                fl *= 2.5
                do = mk(Hq)
                o, lse = _C.fwd(q, k, v, sc, causal, -1, -1, 0.0, None, 0.0, 0)
                p = _lib.FableBwdParams()
                p.B, p.Hq, p.Hk, p.gqa, p.SQ, p.SK, p.D = B, Hq, Hk, Hq // Hk, S, S, D
                p.causal, p.win_left, p.win_right = int(causal), -1, -1
                need = _C._L.fable_attn_bwd_ds_bytes(p, 1)
                hdr = ((S + 31) // 32 + 1) * 4 + 255 >> 8 << 8
                p.B = 64 * B                            # many rounds of workgroups: the tiles alone
                tiles = (_C._L.fable_attn_bwd_ds_bytes(p, 1) - hdr) // 64
                split = need > hdr + tiles + 255        # the split's partials follow the tiles
                ms = timed(lambda: _C.bwd(do, q, k, v, o, lse, sc, causal, -1, -1, 0.0, None, 0.0, 0))
                del do, o, lse
            out.append(f"| {pas} | {B} | {S} | {Hq} / {Hk} | {D} | {'yes' if causal else 'no'} | "
                       f"{str(dt)[6:]} | {ms:.4f} | {fl / (ms * 1e-3) / 1e12:.0f} | {'yes' if split else 'no'} |")
            del q, k, v
    # paged decode through flash_attn_with_kvcache, timed as replays of a captured HIP graph of
    # `inner` calls: at small batch a call's kernels take less time than the host needs to issue
    # it, and back-to-back calls would time the host
    from fable_attn.flash_attn_interface import flash_attn_with_kvcache
    out += ["", "| pass | batch | ctx | page | Hq / Hk | D | dtype | us per call | GB/s (K+V once) | % of 8 TB/s | splits |",
            "|---|---|---|---|---|---|---|---|---|---|---|"]
    for B, ctx, page in SWEEP_DEC:
        Hq, Hk, D = 32, 8, 128
        nb = B * (ctx // page)
        kc = torch.randn(nb, page, Hk, D, device="cuda", dtype=torch.float16, generator=g)
        vc = torch.randn(nb, page, Hk, D, device="cuda", dtype=torch.float16, generator=g)
        bt = torch.randperm(nb, generator=torch.Generator().manual_seed(1)).view(B, ctx // page).int().cuda()
        lens = torch.full((B,), ctx, dtype=torch.int32, device="cuda")
        q = torch.randn(B, 1, Hq, D, device="cuda", dtype=torch.float16, generator=g)
        call = lambda: flash_attn_with_kvcache(q, kc, vc, cache_seqlens=lens, block_table=bt, causal=True)
        side = torch.cuda.Stream()
        side.wait_stream(torch.cuda.current_stream())
        with torch.cuda.stream(side):
            for _ in range(3):
                call()
        torch.cuda.current_stream().wait_stream(side)
        graph = torch.cuda.CUDAGraph()
        with torch.cuda.graph(graph):
            for _ in range(inner):
                call()
        ms = timed(graph.replay) / inner
        byts = 2.0 * B * ctx * Hk * D * 2
        out.append(f"| decode | {B} | {ctx} | {page} | {Hq} / {Hk} | {D} | float16 | {ms * 1e3:.1f} | "
                   f"{byts / (ms * 1e-3) / 1e9:.0f} | {byts / (ms * 1e-3) / 8e12 * 100:.0f}% | "
                   f"{_C.num_splits(B, 1, Hq, Hq // Hk, ctx, 0)} |")
        del graph, kc, vc
    return "\n".join(out)


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=20)
    # 30 untimed headline steps (~65 ms) bring an idle GPU's clocks to their loaded level
    ap.add_argument("--warmup", type=int, default=30)
    ap.add_argument("--no-cpu", action="store_true")
    ap.add_argument("--cpu-heads", type=int, default=32)
    ap.add_argument("--extras", default="fwd,bwd,decode,varlen,gemm")
    ap.add_argument("--copy-calib", action="store_true",
                    help="also run a 1 GiB device copy (calibrates rocprof FETCH/WRITE_SIZE)")
    ap.add_argument("--summarize-pmc", nargs=2, metavar=("FETCH_DIR", "WRITE_DIR"),
                    help="print the calibrated PMC table of two rocprofv3 --pmc runs and exit")
    ap.add_argument("--summarize-stats", metavar="DIR",
                    help="print the rocprofv3 --stats kernel table and exit")
    ap.add_argument("--summarize-mfma", metavar="DIR",
                    help="print the matrix-core utilisation table of a rocprofv3 --pmc "
                         "SQ_VALU_MFMA_BUSY_CYCLES GRBM_GUI_ACTIVE run and exit")
    ap.add_argument("--summarize-counters", nargs="+", metavar="DIR",
                    help="print every counter of rocprofv3 --pmc runs for --kernel-filter and exit")
    ap.add_argument("--summarize-parity", metavar="JSONL",
                    help="print the table of the parity errors the GPU tests logged and exit")
    ap.add_argument("--sweep", action="store_true",
                    help="print a markdown table of forward and backward rates over a grid of shapes and exit")
    ap.add_argument("--kernel-filter", default=None, help="regex on kernel symbols (summaries)")
    ap.add_argument("--skip", type=int, default=0, help="leading dispatches to skip (summaries)")
    ap.add_argument("--last", type=int, default=0, help="average only the last N dispatches (summaries)")
    a = ap.parse_args()
    if a.summarize_pmc:
        print(summarize_pmc(*a.summarize_pmc, kernel_re=a.kernel_filter))
        return
    if a.summarize_stats:
        print(summarize_stats(a.summarize_stats, a.kernel_filter, a.skip, a.last))
        return
    if a.summarize_mfma:
        print(summarize_mfma(a.summarize_mfma, a.kernel_filter))
        return
    if a.summarize_counters:
        print(summarize_counters(a.summarize_counters, a.kernel_filter or "."))
        return
    if a.summarize_parity:
        print(summarize_parity(a.summarize_parity))
        return
    if a.gpus != 1 or int(os.environ.get("WORLD_SIZE", "1")) > 1:
        print("bench.py: this build measures one GPU only (the reference has no multi-GPU "
              "path); run with --gpus 1", file=sys.stderr)
        sys.exit(2)
    import torch
    if not torch.cuda.is_available():
        print("bench.py: no GPU visible", file=sys.stderr)
        sys.exit(2)

    if a.sweep:
        print(sweep())
        return
    log("[bench] headline: causal fp16 forward S=16384 H=32 D=128")
    head, head_inputs = bench_fwd(16384, a.steps, a.warmup)
    log(f"[bench] fwd S=16384: {head['ms']:.3f} ms  {head['tflops']:.1f} TFLOP/s")
    cpu_on = not a.no_cpu
    extra = {}
    for name in [x for x in a.extras.split(",") if x]:
        try:
            if name in ("fwd", "c2sizes"):
                for S in (4096, 8192):
                    r, ins = bench_fwd(S, max(a.steps, 20), max(3, a.warmup), warm_ms=EXTRA_WARM_MS)
                    if cpu_on:
                        r["cpu_baseline"] = cpu_baseline(ins)
                    extra[f"fwd_causal_S{S}"] = r
                    del ins
            if name in ("fwd", "c1"):
                r, ins = bench_fwd(1024, 20, 3, causal=False, H=8, D=64, warm_ms=EXTRA_WARM_MS)
                if cpu_on:
                    r["cpu_baseline"] = cpu_baseline(ins, heads=8, causal=False)
                extra["fwd_C1_S1024_D64_noncausal"] = r
                del ins
            if name == "bwd":
                extra["bwd_C3"] = bench_bwd(max(20, a.steps), max(3, a.warmup),
                                            cpu_heads=32 if cpu_on else 0)
            elif name == "decode":
                extra["decode_C4"] = bench_decode(max(a.steps, 20), max(3, a.warmup),
                                                  cpu_seqs=16 if cpu_on else 0)
            elif name == "varlen":
                extra["varlen_C5"] = bench_varlen(max(20, a.steps), max(3, a.warmup),
                                                  cpu_heads=4 if cpu_on else 0)
            elif name in ("gemm", "gemm_random"):
                # (gemm_random: the random operands alone, for a counter run of one kind)
                extra["gemm_fp16_calibration"] = bench_gemm(max(20, a.steps), max(3, a.warmup),
                                                            kinds=("random",) if name == "gemm_random"
                                                            else ("random", "constant"))
            log(f"[bench] extra {name} done")
        except RuntimeError as e:
            extra[name] = {"error": str(e)[:300]}
            log(f"[bench] extra {name}: {e}")
    if a.copy_calib:
        x = torch.empty(1 << 29, dtype=torch.float16, device="cuda")
        y = torch.empty_like(x)
        for _ in range(3):
            y.copy_(x)
        torch.cuda.synchronize()
        extra["copy_calib_bytes_each_way"] = x.numel() * 2
    cpu = None
    if not a.no_cpu:
        log("[bench] cpu baseline")
        cpu = cpu_baseline(head_inputs, heads=a.cpu_heads)
        log(f"[bench] cpu: {cpu['value']:.4f} TFLOP/s on {cpu['cores']} cores")
    ach = head["kernel_tflops"]
    line = {
        "metric": METRIC,
        "value": round(head["tflops"], 2),
        "unit": "TFLOP/s",
        "n_gpus": 1,
        "steps": a.steps,
        "warmup": a.warmup,
        "ms_per_step": round(head["ms"], 4),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "fp16",
        "data": "synthetic",
        "config": {"workload": "flash_attn_func causal fp16 forward (BASELINE.json configs[1])",
                   "batch": 1, "seq_len": 16384, "heads": 32, "head_dim": 128,
                   "causal": True, "flop_per_step": head["flops"]},
        "roofline": {"bound": "mfma", "achieved": round(ach, 2), "peak": PEAK_MFMA_TFLOPS,
                     "unit": "TFLOP/s", "frac": round(ach / PEAK_MFMA_TFLOPS, 4),
                     "traffic": profiled_traffic(FWD_C2_KERNEL)},
        "cpu_baseline": cpu,
        "extra": extra,
    }
    print(json.dumps(line))


if __name__ == "__main__":
    main()
