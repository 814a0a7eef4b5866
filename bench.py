#!/usr/bin/env python3
"""Benchmark: HelixML SSM forward hot path on one MI355X.

Metric: Mamba selective-scan fwd tokens/s + achieved HBM GB/s (% of peak), 1 GPU.
Default workload = BASELINE config 2: fused selective scan, batch 8 x L 2048 x d_inner 1536 x
d_state 16, fp32, inputs resident in HBM, 3 rotating input sets (1.2 GB) so the 256 MB MALL
cannot serve a step from the previous one. A "step" is one hx_selective_scan_fwd call over one
batch. Prints ONE JSON line.

  python bench.py [--steps K] [--warmup W]
                  [--workload c1|c2|c2bf16|c3|c4|c4s4|c4s4exact|c4s4d|c5|c5dec|copy|gemm] [--no-cpu]

Timing: an untimed clock-settle phase (the step back to back for SETTLE_S seconds) and W untimed
warmup steps, then exactly K timed steps with a HIP event between consecutive steps; ms_per_step
is the median step time ("timing" holds the mean, min, max and the settle phase).

Rooflines on the config-2 line: "roofline" = algorithmic bytes per launch / live launch time
against 8 TB/s, with "traffic" the HBM bytes per launch rocprofv3 measured (profiles/traffic.json);
"issue_roofline" = the kernel's VALU-busy issue slots per launch (rocprofv3 SQ_ACTIVE_INST_VALU,
profiles/issue.json) / live launch time, against 1024 SIMDs x 2.4 GHz / 4 cycles per slot.

c1 = BASELINE config 1 (README SSM example shapes): exported MambaBlock MLP + S4Block, fp32.

c3 = BASELINE config 3, the full Mamba block (in_proj, conv1d+SiLU, x_proj, dt_proj, fused scan,
out_proj) at batch 4 x L 4096 x d_model 2048, bf16 storage; reported separately from the metric.
c4s4 / c4s4exact / c4s4d = BASELINE config 4's S4 recurrence (d 2048, N 16, L 65536): reference
mode time-parallel, reference mode bit-exact, and the S4D diagonal complex form.
gemm = the block's and the LM's projection shapes, here and through the vendor library.
c5 / c5dec = BASELINE config 5's byte LM (12 x (RMSNorm + Mamba), d_model 512): prefill of
16 x 8192 tokens, and one recurrent decode step at batch 256 (after a 64-token prefill).
"""
from __future__ import annotations

import argparse
import json
import os
import sys
import time

import numpy as np
import torch

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, ROOT)

from helixml_amd import _ffi, ssm  # noqa: E402

PEAK_HBM_GBS = 8000.0  # MI355X HBM3E, published
# the kernel the automatic dispatch runs for config 2 (the name rocprofv3 reports)
SCAN_KERNEL = "scan_ws2_kernel<float, 3, true, true>"


def scan_bytes(bt, L, dim, N, es, with_z=True, with_D=True):
    """Algorithmic HBM bytes of one fused scan: read u, delta, (z), B, C once, write out once,
    plus A (and D). State never leaves registers."""
    streams = 3 + (1 if with_z else 0)  # u, delta, out, z
    return streams * bt * L * dim * es + 2 * bt * L * N * es + dim * N * 4 + (dim * 4 if with_D else 0)


def make_scan_inputs(bt, L, dim, N, gen, dev, dtype):
    """BASELINE config-2 distributions."""
    f = torch.float32
    u = torch.randn((bt, L, dim), generator=gen, device=dev, dtype=f)
    delta = torch.randn((bt, L, dim), generator=gen, device=dev, dtype=f) * 0.5 - 4.0
    z = torch.randn((bt, L, dim), generator=gen, device=dev, dtype=f)
    B = torch.randn((bt, L, N), generator=gen, device=dev, dtype=f)
    C = torch.randn((bt, L, N), generator=gen, device=dev, dtype=f)
    A = -torch.exp(torch.log(torch.arange(1, N + 1, device=dev, dtype=f))).repeat(dim, 1).contiguous()
    D = torch.randn((dim,), generator=gen, device=dev, dtype=f)
    cast = lambda t: t.to(dtype).contiguous()
    return dict(u=cast(u), delta=cast(delta), A=A, B=cast(B), C=cast(C), D=D, z=cast(z))


SETTLE_S = 0.25  # untimed clock-settle phase before the warmup steps (seconds of launches)
LAST_TIMING = {}


def time_steps(fn, sets, steps, warmup, settle_s=SETTLE_S):
    """Times exactly `steps` steps after `warmup` untimed ones, rotating over `sets` input sets.

    Before the warmup the step runs back to back, untimed, for `settle_s` seconds: the GPU's
    power management raises the shader clock over the first tens of milliseconds of load, so
    steps timed from an idle GPU measure that ramp rather than the kernel (MI355X: config 2
    takes 165-170 us per step in the first ~10 ms, 141-142 us after). The timed region is the
    `steps` steps only, bracketed by synchronisation; a HIP event on the launch stream (torch's
    current stream, the stream handed to the C ABI) separates every step, and the median step
    time is returned (the mean is kept in LAST_TIMING)."""
    n_settle = 0
    if settle_s > 0:
        t_end = time.perf_counter() + settle_s
        while time.perf_counter() < t_end:
            for _ in range(8):
                fn(n_settle % sets)
                n_settle += 1
            torch.cuda.synchronize()
    for i in range(warmup):
        fn(i % sets)
    torch.cuda.synchronize()
    ev = [torch.cuda.Event(enable_timing=True) for _ in range(steps + 1)]
    ev[0].record()
    for i in range(steps):
        fn(i % sets)
        ev[i + 1].record()
    torch.cuda.synchronize()
    per = [ev[i].elapsed_time(ev[i + 1]) for i in range(steps)]
    LAST_TIMING.clear()
    LAST_TIMING.update(median_ms=float(np.median(per)), mean_ms=float(np.mean(per)),
                       min_ms=float(np.min(per)), max_ms=float(np.max(per)),
                       total_ms=float(ev[0].elapsed_time(ev[-1])),
                       clock_settle={"seconds": settle_s, "untimed_steps": n_settle})
    return float(np.median(per))


def host_info():
    """The host the CPU baselines run on: nproc, lscpu model name, the OpenMP thread count used
    (OMP_NUM_THREADS, the per-GPU CPU share on the GPU box) and OMP_PROC_BIND."""
    model = None
    try:
        with open("/proc/cpuinfo") as f:
            for line in f:
                if line.startswith("model name"):
                    model = line.split(":", 1)[1].strip()
                    break
    except OSError:
        pass
    import oracle  # test/bench infrastructure only
    return {"nproc": os.cpu_count(), "lscpu_model": model, "omp_threads": oracle.max_threads(),
            "OMP_NUM_THREADS": os.environ.get("OMP_NUM_THREADS"),
            "OMP_PROC_BIND": os.environ.get("OMP_PROC_BIND")}


def cpu_baseline_scan(x_dev, sample_batches):
    """The CPU oracle (C restatement, port of the reference's CPU arithmetic) on a bounded
    sample of the same workload: the first `sample_batches` batch rows of input set 0."""
    import oracle  # test/bench infrastructure only
    host = {k: (v[:sample_batches].float().cpu().numpy() if v.dim() == 3 else v.float().cpu().numpy())
            for k, v in x_dev.items()}
    bt, L, dim = host["u"].shape
    t0 = time.perf_counter()
    out1 = oracle.selective_scan(**host)
    t1 = time.perf_counter()
    threads = oracle.max_threads()  # OMP_NUM_THREADS: the host's CPU share for this GPU
    t2 = time.perf_counter()
    oracle.selective_scan_omp(**host, threads=threads)
    t3 = time.perf_counter()
    toks = bt * L
    return dict(value=toks / (t1 - t0), unit="tokens/s", cores=1, kind="port",
                sample=f"batch rows 0..{bt - 1} of config 2 input set 0 ({bt}x{L}x{dim}x16), "
                       f"single-threaded C oracle, {t1 - t0:.2f} s",
                host=host_info(),
                omp=dict(value=toks / (t3 - t2), threads=threads, seconds=round(t3 - t2, 3))), out1


def fit_time(run, sizes, warm=True):
    """Times run(n) once at each sample size n and fits T(n) = a + b*n through the points (the
    fixed part a: weight transposes and allocations that do not grow with n; one point or a
    non-increasing pair: T = b*n). warm: one untimed call at the smallest size first (it starts the
    OpenMP pool and faults in the pages). Returns (a, b, [[n, seconds], ...])."""
    if warm:
        run(sizes[0])
    pts = []
    for n in sizes:
        t0 = time.perf_counter()
        run(n)
        pts.append([n, time.perf_counter() - t0])
    if len(pts) >= 2 and pts[-1][1] > pts[0][1]:
        (n0, t0), (n1, t1) = pts[0], pts[-1]
        b = (t1 - t0) / (n1 - n0)
        a = max(t0 - b * n0, 0.0)
    else:
        a, b = 0.0, pts[-1][1] / pts[-1][0]
    return a, b, pts


def cpu_leg(run, sizes, full, units_full, unit, cores, sample, warm=True, **extra):
    """A CPU baseline leg: run(n) at the sample sizes, extrapolated linearly to `full` (the size
    of the GPU step, in the same units as the sizes); value = units_full / T(full)."""
    a, b, pts = fit_time(run, sizes, warm)
    t_full = a + b * full
    return dict(value=units_full / t_full, unit=unit, cores=cores, kind="port", sample=sample,
                extrapolated={"model": "T(n) = a + b*n, linear in n", "n_full": full,
                              "a_s": a, "b_s_per_n": b, "samples_n_s": pts, "t_full_s": t_full},
                host=host_info(), **extra)


def norm_err(g, r):
    g, r = np.asarray(g, np.float64), np.asarray(r, np.float64)
    return float(np.linalg.norm(g - r) / max(np.linalg.norm(r), 1e-30))


PEAK_BF16_TFLOPS = 2500.0  # MI355X dense bf16 MFMA, published


def bench_block(args, dev):
    """full Mamba block forward, bf16 storage / fp32 arithmetic. The step is one
    hx_mamba_block_fwd call; a per-stage breakdown times each kernel on its own (same operands)."""
    bt, L, dm, di, N, r, k = 4, 4096, 2048, 4096, 16, 128, 4
    M = bt * L
    gen = torch.Generator().manual_seed(0x48454C49)
    bf = torch.bfloat16

    def nrm(shape, fan):
        return (torch.randn(shape, generator=gen) * (2.0 / fan) ** 0.5).to(dev, bf)

    dt0 = torch.exp(torch.rand(di, generator=gen) * (np.log(0.1) - np.log(1e-3)) + np.log(1e-3))
    prm = dict(w_in=nrm((2 * di, dm), dm),
               conv_w=((torch.rand((di, k), generator=gen) * 2 - 1) / k ** 0.5).to(dev),
               conv_b=((torch.rand(di, generator=gen) * 2 - 1) / k ** 0.5).to(dev),
               w_x=nrm((r + 2 * N, di), di), w_dt=nrm((di, r), r),
               dt_bias=(dt0 + torch.log(-torch.expm1(-dt0))).to(dev),
               A=(-torch.arange(1, N + 1, dtype=torch.float32)).repeat(di, 1).to(dev),
               D=torch.randn(di, generator=gen).to(dev), w_out=nrm((dm, di), di))
    nsets = 2
    xs = [torch.randn((bt, L, dm), generator=gen).to(dev, bf) for _ in range(nsets)]
    outs = [torch.empty_like(x) for x in xs]
    ws = torch.empty(ssm.mamba_block_workspace_size(bt, L, di, r, N), device=dev, dtype=torch.uint8)

    def step(i):
        ssm.mamba_block_fwd(xs[i], **prm, workspace=ws, out=outs[i])

    ms = time_steps(step, nsets, args.steps, args.warmup)
    timing = dict(LAST_TIMING)
    # the GEMM kernels' products; dt_proj's runs inside the scan kernel (hx_selective_scan_dtproj_fwd)
    flops = {"in_proj": 2 * M * 2 * di * dm, "x_proj": 2 * M * (r + 2 * N) * di,
             "out_proj": 2 * M * dm * di}
    dtproj_flops = 2 * M * di * r
    # per-stage breakdown on the block's own intermediates
    x2 = xs[0].view(M, dm)
    xz = ssm.gemm_bf16(x2, prm["w_in"], splits=(di,))
    xc = ssm.conv1d_silu(xz[0].view(bt, L, di), prm["conv_w"], prm["conv_b"])
    dbc = ssm.gemm_bf16(xc.view(M, di), prm["w_x"], splits=(r, r + N))
    Bm, Cm = dbc[1].view(bt, L, N), dbc[2].view(bt, L, N)
    y = torch.empty((bt, L, di), device=dev, dtype=bf)
    stages = {
        "in_proj": lambda i: ssm.gemm_bf16(x2, prm["w_in"], splits=(di,)),
        "conv1d_silu": lambda i: ssm.conv1d_silu(xz[0].view(bt, L, di), prm["conv_w"], prm["conv_b"], out=xc),
        # narrow and long: the automatic choice is the 64-row narrow kernel, as in the block
        "x_proj": lambda i: ssm.gemm_bf16(xc.view(M, di), prm["w_x"], splits=(r, r + N)),
        # dt_proj on the matrix core inside the scan, as the block runs it
        "scan_dtproj": lambda i: ssm.selective_scan_dtproj_fwd(
            xc, dbc[0].view(bt, L, r), prm["w_dt"], prm["A"], Bm, Cm, prm["D"], xz[1].view(bt, L, di),
            prm["dt_bias"], out=y),
        "out_proj": lambda i: ssm.gemm_bf16(y.view(M, di), prm["w_out"]),
    }
    breakdown = {}
    for name, fn in stages.items():
        sms = time_steps(fn, 1, max(args.steps // 2, 3), 2, settle_s=0.02)
        e = {"ms": sms}
        if name in flops:
            e["tflops"] = flops[name] / (sms * 1e-3) / 1e12
        breakdown[name] = e
    # the fused scan reads dt_lo [M, r] and w_dt [di, r] instead of delta [M, di]
    scan_bytes_ = scan_bytes(bt, L, di, N, 2) - M * di * 2 + M * r * 2 + di * r * 2
    breakdown["scan_dtproj"]["hbm_gbs"] = scan_bytes_ / (breakdown["scan_dtproj"]["ms"] * 1e-3) / 1e9
    breakdown["scan_dtproj"]["dtproj_tflops"] = dtproj_flops / (breakdown["scan_dtproj"]["ms"] * 1e-3) / 1e12
    breakdown["conv1d_silu"]["hbm_gbs"] = 2 * M * di * 2 / (breakdown["conv1d_silu"]["ms"] * 1e-3) / 1e9
    gemm_flops = sum(flops.values())
    total_flops = gemm_flops + dtproj_flops
    gemm_ms = sum(breakdown[n]["ms"] for n in flops)
    cpu = None
    if not args.no_cpu:
        # (O): the block over OpenMP (blocked products, 16-channel scan tasks), f32 throughout,
        # on batch row 0 of input set 0 at two prefix lengths; (R): the reference's Linear
        # execution shape (transpose copy, ijk matmul, broadcast add, one thread) for the four
        # projections, the sequential C conv and scan beside it, at two short prefixes. Both are
        # extrapolated linearly in tokens to the step's 4 x 4096 (the block is causal and its
        # cost per token does not depend on the position).
        import oracle  # test/bench infrastructure only
        th = oracle.max_threads()
        hp = {k: v.float().cpu().numpy() for k, v in prm.items()}
        x0 = xs[0][:1].float().cpu().numpy()
        got = {}

        def run_o(n):
            got["y"] = oracle.mamba_block(x0[:, :n], **hp, dt_rank=r, bf16=False, impl="omp", threads=th)

        def run_r(n):
            oracle.mamba_block(x0[:, :n], **hp, dt_rank=r, bf16=False, impl="ref")

        no, nr = (1024, 2048), (16, 48)
        cpu = cpu_leg(run_o, no, M, M, "tokens/s", th,
                      f"OpenMP block (oracle/hx_oracle_omp.c, f32) on batch row 0 of input set 0, "
                      f"prefixes of {no[0]} and {no[1]} tokens", kind_note="(O) optimised, all host cores")
        # the GPU's bf16-storage output against the f32 CPU block on the same tokens
        cpu["gpu_vs_cpu_normwise_err"] = norm_err(outs[0][0, :no[-1]].float().cpu().numpy(), got["y"][0])
        cpu["reference_shape"] = cpu_leg(
            run_r, nr, M, M, "tokens/s", 1,
            f"the block with the reference's Linear execution shape (oracle/hx_oracle_ref.c), one "
            f"thread, on batch row 0 of input set 0, prefixes of {nr[0]} and {nr[1]} tokens",
            warm=False, kind_note="(R) reference-faithful, 1 core, linearly extrapolated")
    rec = {
        "metric": "Mamba block fwd tokens/s (config 3), 1 GPU",
        "value": M * 1e3 / ms, "unit": "tokens/s", "n_gpus": 1, "steps": args.steps,
        "warmup": args.warmup, "ms_per_step": ms, "higher_is_better": True, "scaling": "weak",
        "vs_baseline": None, "dtype": "bf16-storage/fp32-compute",
        "data": "synthetic (config-3 distributions, random-init weights, seeded)",
        "config": {"workload": "mamba_block_fwd config3 (batch 4, L 4096, d_model 2048, d_inner 4096, "
                               "d_state 16, dt_rank 128, conv 4)", "batch": bt, "seq_len": L,
                   "d_model": dm, "d_inner": di, "d_state": N, "dt_rank": r, "d_conv": k},
        "block_tflops": total_flops / (ms * 1e-3) / 1e12,
        # the GEMM kernels (in_proj, x_proj, out_proj) together: their products over their time
        "roofline": {"bound": "mfma", "achieved": gemm_flops / (gemm_ms * 1e-3) / 1e12,
                     "peak": PEAK_BF16_TFLOPS, "unit": "TFLOP/s",
                     "frac": gemm_flops / (gemm_ms * 1e-3) / 1e12 / PEAK_BF16_TFLOPS,
                     "traffic": None, "algorithmic_flops": gemm_flops, "kernel_ms": gemm_ms},
        "breakdown": breakdown,
        "timing": timing,
        "cpu_baseline": cpu,
    }
    print(json.dumps(rec))


def bench_s4(args, dev):
    """BASELINE config 4, S4 recurrence at d_model 2048, N 16, L 65536, fp32: A_real = -0.5,
    A_imag = pi*n, dt = 0.1; B, C ~ N(0, 0.1); D ~ N(0, 1); x ~ N(0, 1). Algorithmic bytes: x read
    once, y written once (1.074 GB)."""
    M, N, L = 2048, 16, 65536
    gen = torch.Generator(device=dev)
    gen.manual_seed(0x53345334)
    f = torch.float32
    nbytes = 2 * M * L * 4
    if args.workload in ("c4s4", "c4s4exact"):
        xs = [torch.randn((M, L), generator=gen, device=dev, dtype=f) for _ in range(2)]
        prm = dict(a_real=torch.full((N,), -0.5, device=dev),
                   a_imag=torch.pi * torch.arange(N, device=dev, dtype=f),
                   B=torch.randn((N, M), generator=gen, device=dev) * 0.1,
                   C=torch.randn((M, N), generator=gen, device=dev) * 0.1,
                   D=torch.randn((M,), generator=gen, device=dev))
        par = args.workload == "c4s4"
        # discretize(dt) once (host libm, hx_s4_discretize) and one workspace: no host round
        # trip and no allocation inside the timed steps
        a_disc = ssm.s4_discretize(prm["a_real"], prm["a_imag"], 0.1, device=dev)
        fn = _ffi.lib().hx_s4_ref_parallel_workspace_size if par else _ffi.lib().hx_s4_ref_workspace_size
        ws = torch.empty(int(fn(M, N, L)), device=dev, dtype=torch.uint8)

        def step(i):
            ssm.s4_ref_fwd(xs[i], **prm, parallel=par, a=a_disc, workspace=ws)

        workload = ("S4Block::forward_ssm reference mode, " + ("time-parallel" if par else "bit-exact")
                    + " (d_model 2048, N 16, L 65536, A = -0.5 + i*pi*n, dt 0.1)")
    else:
        xs = [torch.randn((1, L, M), generator=gen, device=dev, dtype=f) for _ in range(2)]
        prm = dict(dt=torch.full((M,), 0.1, device=dev), a_re=torch.full((M, N), -0.5, device=dev),
                   a_im=(torch.pi * torch.arange(N, device=dev, dtype=f)).repeat(M, 1).contiguous(),
                   B_re=torch.randn((M, N), generator=gen, device=dev) * 0.1,
                   B_im=torch.randn((M, N), generator=gen, device=dev) * 0.1,
                   C_re=torch.randn((M, N), generator=gen, device=dev) * 0.1,
                   C_im=torch.randn((M, N), generator=gen, device=dev) * 0.1,
                   D=torch.randn((M,), generator=gen, device=dev))

        def step(i):
            return ssm.s4d_complex_fwd(xs[i], **prm)

        workload = "S4D diagonal complex recurrence (batch 1, L 65536, d 2048, N 16, A = -0.5 + i*pi*n)"
    ms = time_steps(step, 2, args.steps, args.warmup)
    timing = dict(LAST_TIMING)
    gbs = nbytes / (ms * 1e-3) / 1e9
    cpu = None
    if not args.no_cpu and args.workload in ("c4s4", "c4s4exact"):
        # (R): S4Block::forward_ssm in the reference's execution shape (allocation per op, a
        # copied column slice per step, single thread) on the first `ls` steps of input set 0;
        # its cost per step does not depend on t, so tokens/s extrapolates to the full L
        import oracle  # test/bench infrastructure only
        ls = 4096
        xh = xs[0][:, :ls].contiguous().cpu().numpy()
        hp = {k: v.cpu().numpy() for k, v in prm.items()}
        t0 = time.perf_counter()
        yr = oracle.r_s4_forward_ssm(xh, hp["a_real"], hp["a_imag"], hp["B"], hp["C"], hp["D"])
        t1 = time.perf_counter()
        ref = oracle.s4_ref_fwd(xh, hp["a_real"], hp["a_imag"], hp["B"], hp["C"], hp["D"])
        th = oracle.max_threads()
        oracle.s4_ref_fwd_omp(xh[:, :256], hp["a_real"], hp["a_imag"], hp["B"], hp["C"], hp["D"], threads=th)
        t2 = time.perf_counter()
        yo = oracle.s4_ref_fwd_omp(xh, hp["a_real"], hp["a_imag"], hp["B"], hp["C"], hp["D"], threads=th)
        t3 = time.perf_counter()
        cpu = dict(value=ls / (t1 - t0), unit="tokens/s", cores=1, kind="port",
                   sample=f"first {ls} of {L} steps of input set 0 (d_model {M}, N {N}): "
                          f"S4Block::forward_ssm restated op by op with the reference's per-op "
                          f"allocation (oracle/hx_oracle_ref.c), {t1 - t0:.2f} s",
                   kind_note="(R) reference-faithful, 1 core",
                   host=host_info(), bit_identical_to_oracle=bool(np.array_equal(yr, ref)),
                   omp=dict(value=ls / (t3 - t2), unit="tokens/s", cores=th, seconds=round(t3 - t2, 3),
                            kind_note="(O) projection and readout over OpenMP (oracle/hx_oracle_omp.c), "
                                      "same sample",
                            bit_identical_to_oracle=bool(np.array_equal(yo, ref))))
    if not args.no_cpu and args.workload == "c4s4d":
        # (O): the S4D recurrence in f32 over OpenMP (16-channel tasks) on the first 256 and 512
        # channels of input set 0, full length; the cost is linear in channels
        import oracle  # test/bench infrastructure only
        th = oracle.max_threads()
        hp = {k: v.cpu().numpy() for k, v in prm.items()}
        got = {}
        host = {n: (xs[0][:, :, :n].contiguous().cpu().numpy(),
                    {k: np.ascontiguousarray(v[:n]) for k, v in hp.items()}) for n in (256, 512)}

        def run_o(n):
            got["y"] = oracle.s4d_complex_omp(host[n][0], **host[n][1], threads=th)

        y_gpu = step(0)
        torch.cuda.synchronize()
        cpu = cpu_leg(run_o, (256, 512), M, L, "tokens/s", th,
                      f"S4D f32 recurrence over OpenMP (oracle/hx_oracle_omp.c) on channels 0..255 and "
                      f"0..511 of input set 0, all {L} steps", kind_note="(O) optimised, all host cores")
        cpu["gpu_vs_cpu_normwise_err"] = norm_err(y_gpu[:, :, :512].cpu().numpy(), got["y"])
    print(json.dumps({
        "metric": "S4 recurrence tokens/s (config 4), 1 GPU", "value": L * 1e3 / ms, "unit": "tokens/s",
        "n_gpus": 1, "steps": args.steps, "warmup": args.warmup, "ms_per_step": ms,
        "higher_is_better": True, "scaling": "weak", "vs_baseline": None, "dtype": "fp32",
        "data": "synthetic (config-4 S4 parameters, seeded)",
        "config": {"workload": workload, "d_model": M, "d_state": N, "seq_len": L},
        "roofline": {"bound": "hbm", "achieved": gbs, "peak": PEAK_HBM_GBS, "unit": "GB/s",
                     "frac": gbs / PEAK_HBM_GBS, "traffic": None, "algorithmic_bytes": nbytes,
                     "kernel_ms": ms},
        "timing": timing,
        "cpu_baseline": cpu}))


def bench_c1(args, dev):
    """BASELINE config 1, the README SSM example's shapes: the exported MambaBlock::forward_mamba
    (Linear -> SiLU -> Linear, d_model 64, expand 2, crates/nn/src/lib.rs:888-906) on x [100, 64]
    ~ U(-1, 1), and ssm::S4Block::forward_ssm (d_model 64, N 16) on x^T [64, 100], weights from the
    reference's init distributions (seeded). A step is both forwards (latency-bound: three small
    kernels plus the S4 chain). CPU baseline (R): the same two forwards restated in the
    reference's execution shape (per-op allocation, oracle/hx_oracle_ref.c), one thread."""
    import oracle  # test/bench infrastructure only
    rng = np.random.default_rng(0x48454C49_00000001)
    R, dm, di, N = 100, 64, 128, 16
    f = np.float32
    X = rng.uniform(-1, 1, (R, dm)).astype(f)
    Wg = (rng.standard_normal((di, dm)) * np.sqrt(2 / dm)).astype(f)
    Wo = (rng.standard_normal((dm, di)) * np.sqrt(2 / di)).astype(f)
    bg, bo = np.zeros(di, f), np.zeros(dm, f)
    ar, ai = np.zeros(N, f), rng.standard_normal(N).astype(f)
    B = (rng.standard_normal((N, dm)) * 0.1).astype(f)
    C = (rng.standard_normal((dm, N)) * 0.1).astype(f)
    D = np.zeros(dm, f)
    xs = np.ascontiguousarray(X.T)
    d = lambda a: torch.from_numpy(np.ascontiguousarray(a)).to(dev)  # noqa: E731
    gX, gWg, gWo, gbg, gbo, gxs, gB, gC, gD = map(d, (X, Wg, Wo, bg, bo, xs, B, C, D))
    gar, gai = d(ar), d(ai)
    a_disc = ssm.s4_discretize(gar, gai, 0.1, device=dev)
    ws = torch.empty(int(_ffi.lib().hx_s4_ref_workspace_size(dm, N, R)), device=dev, dtype=torch.uint8)
    out = {}

    def step(i):
        h = ssm.linear(gX, gWg, gbg, act=1)
        out["mlp"] = ssm.linear(h, gWo, gbo)
        out["s4"] = ssm.s4_ref_fwd(gxs, gar, gai, gB, gC, gD, a=a_disc, workspace=ws)

    ms = time_steps(step, 1, args.steps, args.warmup)
    timing = dict(LAST_TIMING)
    torch.cuda.synchronize()
    ref_mlp = oracle.mamba_mlp(X, Wg, bg, Wo, bo)
    ref_s4 = oracle.s4_ref_fwd(xs, ar, ai, B, C, D)
    g_mlp, g_s4 = out["mlp"].cpu().numpy(), out["s4"].cpu().numpy()
    floor = lambda r: 1e-3 * np.abs(r).max()  # noqa: E731
    err_mlp = float((np.abs(g_mlp - ref_mlp) / np.maximum(np.abs(ref_mlp), floor(ref_mlp))).max())
    cpu = None
    if not args.no_cpu:
        reps = 200
        t0 = time.perf_counter()
        for _ in range(reps):
            oracle.r_mamba_mlp(X, Wg, bg, Wo, bo)
            oracle.r_s4_forward_ssm(xs, ar, ai, B, C, D)
        t1 = time.perf_counter()
        th = oracle.max_threads()
        oracle.linear_omp(oracle.linear_omp(X, Wg, bg, 1, th), Wo, bo, 0, th)
        t2 = time.perf_counter()
        for _ in range(reps):
            oracle.linear_omp(oracle.linear_omp(X, Wg, bg, 1, th), Wo, bo, 0, th)
            oracle.s4_ref_fwd_omp(xs, ar, ai, B, C, D, threads=th)
        t3 = time.perf_counter()
        cpu = dict(value=R * reps / (t1 - t0), unit="tokens/s", cores=1, kind="port",
                   sample=f"{reps} repetitions of both config-1 forwards in the reference's "
                          f"execution shape (oracle/hx_oracle_ref.c), {t1 - t0:.2f} s",
                   kind_note="(R) reference-faithful, 1 core", host=host_info(),
                   omp=dict(value=R * reps / (t3 - t2), unit="tokens/s", cores=th, seconds=round(t3 - t2, 3),
                            kind_note="(O) the same forwards over OpenMP (oracle/hx_oracle_omp.c), "
                                      f"{reps} repetitions"))
    print(json.dumps({
        "metric": "config-1 forwards (exported MambaBlock MLP [100, 64] + S4Block::forward_ssm "
                  "[64, 100]) tokens/s, 1 GPU",
        "value": R * 1e3 / ms, "unit": "tokens/s", "n_gpus": 1, "steps": args.steps,
        "warmup": args.warmup, "ms_per_step": ms, "higher_is_better": True, "scaling": "weak",
        "vs_baseline": None, "dtype": "fp32",
        "data": "synthetic (x ~ U(-1,1), the reference's init distributions, seeded)",
        "config": {"workload": "config1: MambaBlock MLP d_model 64 expand 2 on [100, 64] + "
                               "S4Block d_model 64 N 16 on [64, 100]"},
        "parity": {"mlp_max_rel_err": err_mlp, "s4_bit_exact": bool(np.array_equal(g_s4, ref_s4))},
        "timing": timing, "cpu_baseline": cpu}))


def bench_lm(args, dev):
    """byte-level LM, 12 x (RMSNorm + Mamba), d_model 512, d_state 16,
    expand 2, dt_rank 32, conv 4, vocab 256; tokens uniform bytes (seeded)."""
    from helixml_amd.lm import ByteLM
    m = ByteLM(device=dev)
    gen = torch.Generator(device=dev)
    gen.manual_seed(0x48454C49 + 5)
    if args.workload == "c5":
        bt, L = 16, 8192
        toks = [torch.randint(0, 256, (bt, L), generator=gen, device=dev, dtype=torch.int32)
                for _ in range(2)]
        states = [m.new_state(bt) for _ in range(2)]

        def step(i):
            m.prefill(toks[i], states[i])

        steps = max(2, min(args.steps, 10))
        ms = time_steps(step, 2, steps, min(args.warmup, 2))
        tokens = bt * L
        d, N, r, di = m.d_model, m.d_state, m.dt_rank, m.d_inner
        flops = m.n_layers * 2 * tokens * (2 * di * d + (r + 2 * N) * di + di * r + d * di) \
            + 2 * tokens * m.vocab * d
        workload = "byte LM prefill, 12 x (RMSNorm + Mamba) d_model 512, batch 16 x L 8192"
        extra = {"tflops": flops / (ms * 1e-3) / 1e12, "algorithmic_flops": flops}
        extra["timing"] = dict(LAST_TIMING)
        if not args.no_cpu:
            # (O): the LM over OpenMP (f32 throughout) on sequence 0 of token set 0 at two
            # prefix lengths; (R): the reference's Linear execution shape, one thread, at two
            # short prefixes; both extrapolated linearly in tokens to the step's 16 x 8192
            import oracle  # test/bench infrastructure only
            th = oracle.max_threads()
            P = m.host_params()
            t0 = toks[0][:1].cpu().numpy()
            got = {}

            def run_o(n):
                got["lg"] = oracle.lm_prefill(t0[:, :n], P, m.dt_rank, m.eps, bf16=False, impl="omp",
                                              threads=th)[0]

            def run_r(n):
                oracle.lm_prefill(t0[:, :n], P, m.dt_rank, m.eps, bf16=False, impl="ref")

            no, nr = (1024, 2048), (16, 48)
            cpu = cpu_leg(run_o, no, tokens, tokens, "tokens/s", th,
                          f"OpenMP LM (oracle/hx_oracle_omp.c, f32) on sequence 0 of token set 0, "
                          f"prefixes of {no[0]} and {no[1]} tokens", kind_note="(O) optimised, all host cores")
            g, _ = m.prefill(toks[0][:1, :no[-1]].contiguous())
            cpu["gpu_vs_cpu_normwise_err"] = norm_err(g.cpu().numpy(), got["lg"])
            cpu["reference_shape"] = cpu_leg(
                run_r, nr, tokens, tokens, "tokens/s", 1,
                f"the LM with the reference's Linear execution shape (oracle/hx_oracle_ref.c), one "
                f"thread, on sequence 0 of token set 0, prefixes of {nr[0]} and {nr[1]} tokens",
                warm=False, kind_note="(R) reference-faithful, 1 core, linearly extrapolated")
            extra["cpu_baseline"] = cpu
    else:
        bt = 256
        pre = torch.randint(0, 256, (bt, 64), generator=gen, device=dev, dtype=torch.int32)
        _, state = m.prefill(pre)
        saved = [(a.clone(), c.clone()) for a, c in state]  # the state the timed steps start from
        toks = [torch.randint(0, 256, (bt,), generator=gen, device=dev, dtype=torch.int32)
                for _ in range(4)]
        graph_step = m.decode_graph(state)  # the step captured as a HIP graph

        def step(i):
            graph_step(toks[i])

        steps = args.steps
        ms = time_steps(step, 4, steps, args.warmup)
        tokens = bt
        workload = "byte LM recurrent decode step (HIP graph), 12 layers d_model 512, batch 256"
        extra = {"timing": dict(LAST_TIMING)}
        if not args.no_cpu:
            # (O): one decode step of all 256 sequences over OpenMP (f32 throughout) from the
            # state the timed steps start from (the 64-token prefill's, copied to the host)
            import oracle  # test/bench infrastructure only
            th = oracle.max_threads()
            P = m.host_params()
            st_h = [(a.cpu().numpy(), c.cpu().numpy()) for a, c in saved]
            t0 = toks[0].cpu().numpy()
            got = {}

            def run_o(n):
                got["lg"] = oracle.lm_decode_step(t0[:n], P, [(a[:n], c[:n]) for a, c in st_h], m.dt_rank,
                                                  m.eps, bf16=False, impl="omp", threads=th)[0]

            cpu = cpu_leg(run_o, (bt,), bt, bt, "tokens/s", th,
                          f"one OpenMP decode step (oracle/hx_oracle_omp.c, f32) of all {bt} sequences "
                          f"from the timed steps' starting state", kind_note="(O) optimised, all host cores")
            g = m.decode_step(toks[0], [(a.clone(), c.clone()) for a, c in saved])
            cpu["gpu_vs_cpu_normwise_err"] = norm_err(g.cpu().numpy(), got["lg"])
            extra["cpu_baseline"] = cpu
    rec = {
        "metric": ("byte LM prefill tokens/s (config 5), 1 GPU" if args.workload == "c5"
                   else "byte LM decode tokens/s (config 5, one step at batch 256), 1 GPU"),
        "value": tokens * 1e3 / ms, "unit": "tokens/s", "n_gpus": 1, "steps": steps,
        "warmup": args.warmup, "ms_per_step": ms, "higher_is_better": True, "scaling": "weak",
        "vs_baseline": None, "dtype": "bf16-storage/fp32-compute",
        "data": "synthetic (uniform byte tokens, random-init weights, seeded)",
        "config": {"workload": workload, "layers": m.n_layers, "d_model": m.d_model,
                   "d_inner": m.d_inner, "d_state": m.d_state, "vocab": m.vocab},
        "cpu_baseline": None, **extra}
    print(json.dumps(rec))


def bench_gemm(args, dev):
    """The block's and the LM's projection shapes through hx_gemm_bf16 (automatic kernel choice)
    and through the vendor library (torch.nn.functional.linear, hipBLASLt) in the same process on
    the same random bf16 operands (X ~ N(0, 1), W ~ N(0, 1/K)); best of three rounds of 10 calls
    each, rounds interleaved. One JSON line per shape."""
    shapes = {"config3 in_proj": (16384, 2048, 8192), "config3 out_proj": (16384, 4096, 2048),
              "config3 x_proj": (16384, 4096, 160), "config3 dt_proj": (16384, 128, 4096),
              "config5 in_proj": (131072, 512, 2048), "config5 x_proj": (131072, 1024, 64),
              "config5 dt_proj": (131072, 32, 1024), "config5 head": (131072, 512, 256)}
    gen = torch.Generator(device=dev)
    gen.manual_seed(1)

    def timed(fn, n=10):
        for _ in range(3):
            fn()
        torch.cuda.synchronize()
        ev = [torch.cuda.Event(enable_timing=True) for _ in range(2)]
        ev[0].record()
        for _ in range(n):
            fn()
        ev[1].record()
        torch.cuda.synchronize()
        return ev[0].elapsed_time(ev[1]) / n * 1e3

    for name, (M, K, N) in shapes.items():
        x = torch.randn(M, K, device=dev, generator=gen).to(torch.bfloat16)
        w = (torch.randn(N, K, device=dev, generator=gen) / K ** 0.5).to(torch.bfloat16)
        here, vendor = [], []
        for _ in range(3):
            here.append(timed(lambda: ssm.gemm_bf16(x, w)))
            vendor.append(timed(lambda: torch.nn.functional.linear(x, w)))
        print(json.dumps({"metric": "bf16 GEMM time, here vs vendor library", "shape": name, "M": M,
                          "K": K, "N": N, "here_us": min(here), "vendor_us": min(vendor),
                          "here_rounds_us": here, "vendor_rounds_us": vendor,
                          "here_tflops": 2 * M * N * K / min(here) / 1e6,
                          "higher_is_better": False}))
        del x, w


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=50)
    ap.add_argument("--warmup", type=int, default=10)
    ap.add_argument("--workload", default="c2",
                    choices=["c1", "c2", "c2bf16", "c4", "c3", "c4s4", "c4s4exact", "c4s4d", "c5",
                             "c5dec", "copy", "gemm"],
                    help="copy = plain device copy of 512 MiB (HBM ceiling and counter calibration)")
    ap.add_argument("--variant", type=int, default=0, help="scan kernel variant (hx_set_scan_variant)")
    ap.add_argument("--no-cpu", action="store_true", help="skip the CPU baseline leg")
    args = ap.parse_args()

    world = int(os.environ.get("WORLD_SIZE", "1"))
    if args.gpus != 1 or world != 1:
        print(json.dumps({"error": "this build runs on one GPU only: the scan would shard by channel "
                                   "with no exchange; multi-GPU runs are not part of it",
                          "n_gpus": args.gpus}))
        sys.exit(2)

    dev = torch.device("cuda:0")
    _ffi.call("hx_init", 0)
    if args.variant:
        ssm.set_scan_variant(args.variant)

    if args.workload == "c1":
        bench_c1(args, dev)
        return
    if args.workload == "gemm":
        bench_gemm(args, dev)
        return
    if args.workload == "copy":
        n = 512 * 2**20 // 4
        src = [torch.randn(n, device=dev) for _ in range(2)]
        dst = [torch.empty_like(x) for x in src]
        ms = time_steps(lambda i: dst[i].copy_(src[i]), 2, args.steps, args.warmup)
        gbs = 2 * n * 4 / (ms * 1e-3) / 1e9
        print(json.dumps({"metric": "device copy GB/s (read + write)", "value": gbs, "unit": "GB/s",
                          "n_gpus": 1, "steps": args.steps, "warmup": args.warmup, "ms_per_step": ms,
                          "higher_is_better": True, "bytes_per_step": 2 * n * 4,
                          "frac_of_8TBs": gbs / PEAK_HBM_GBS}))
        return
    if args.workload == "c3":
        bench_block(args, dev)
        return
    if args.workload in ("c4s4", "c4s4exact", "c4s4d"):
        bench_s4(args, dev)
        return
    if args.workload in ("c5", "c5dec"):
        bench_lm(args, dev)
        return
    if args.workload in ("c2", "c2bf16"):
        bt, L, dim, N = 8, 2048, 1536, 16
        dtype = torch.bfloat16 if args.workload == "c2bf16" else torch.float32
        workload = "selective_scan_fwd config2 (batch 8, L 2048, d_inner 1536, d_state 16)"
    else:
        bt, L, dim, N = 1, 65536, 2048, 16
        dtype = torch.float32
        workload = "selective_scan_fwd config4 scan (batch 1, L 65536, d_inner 2048, d_state 16)"
    es = 2 if dtype == torch.bfloat16 else 4
    gen = torch.Generator(device=dev)
    gen.manual_seed(0x48454C49)
    nsets = 3 if bt * L * dim * es * 4 < 2**31 else 2
    sets = [make_scan_inputs(bt, L, dim, N, gen, dev, dtype) for _ in range(nsets)]
    outs = [torch.empty_like(s["u"]) for s in sets]

    def step(i):
        ssm.selective_scan_fwd(**sets[i], out=outs[i])

    ms = time_steps(step, nsets, args.steps, args.warmup)
    timing = dict(LAST_TIMING)
    tokens = bt * L
    nbytes = scan_bytes(bt, L, dim, N, es)
    achieved = nbytes / (ms * 1e-3) / 1e9

    cpu = None
    parity = None
    if not args.no_cpu and args.workload == "c4":
        # (O): the OpenMP scan (16-channel tasks, oracle/hx_oracle_omp.c) on the first 256 and 512
        # channels of input set 0 over the full 65536 steps; the cost is linear in channels
        import oracle  # test/bench infrastructure only
        th = oracle.max_threads()
        step(0)
        torch.cuda.synchronize()
        got, x = {}, sets[0]
        host = {n: {k: v.contiguous().cpu().numpy() for k, v in
                    dict(u=x["u"][:, :, :n], delta=x["delta"][:, :, :n], z=x["z"][:, :, :n],
                         A=x["A"][:n], D=x["D"][:n], B=x["B"], C=x["C"]).items()}
                for n in (256, 512)}

        def run_o(n):
            got["y"] = oracle.selective_scan_omp(**host[n], threads=th)

        cpu = cpu_leg(run_o, (256, 512), dim, tokens, "tokens/s", th,
                      f"OpenMP scan on channels 0..255 and 0..511 of input set 0, all {L} steps",
                      kind_note="(O) optimised, all host cores",
                      note="no reference implementation of the selective scan exists "
                           "(crates/nn/src/ssm.rs:474-483 delegates to the S4 recurrence): the "
                           "port restates the textbook scan with the reference's discretisation")
        g = outs[0][:, :, :512].float().cpu().numpy()
        cpu["gpu_vs_cpu_normwise_err"] = norm_err(g, got["y"])
    if not args.no_cpu and args.workload in ("c2", "c2bf16"):
        step(0)
        torch.cuda.synchronize()
        sample = 8
        cpu, ref = cpu_baseline_scan(sets[0], sample)
        g = outs[0][:sample].float().cpu().numpy()
        r = ref.astype(np.float64)
        floor = 1e-3 * np.abs(r).max()
        parity = float((np.abs(g - r) / np.maximum(np.abs(r), floor)).max())

    copy_ceiling = None
    if args.workload in ("c2", "c2bf16"):
        # the measured HBM ceiling beside the 8 TB/s spec: a plain device copy (read + write) of
        # two 512 MiB buffers in rotation, timed the same way
        n = 512 * 2**20 // 4
        src = [torch.randn(n, device=dev) for _ in range(2)]
        dst = [torch.empty_like(v) for v in src]
        cms = time_steps(lambda i: dst[i].copy_(src[i]), 2, 20, 5, settle_s=0.05)
        cgbs = 2 * n * 4 / (cms * 1e-3) / 1e9
        copy_ceiling = {"gbs": cgbs, "frac_of_8TBs": cgbs / PEAK_HBM_GBS, "bytes_per_step": 2 * n * 4,
                        "scan_frac_of_copy": achieved / cgbs}
        del src, dst

    traffic = None
    issue = None
    tfile = os.path.join(ROOT, "profiles", "traffic.json")
    tkey = {"c2": SCAN_KERNEL + "@config2", "c4": "selective_scan_fwd@config4"}.get(args.workload)
    if tkey and args.variant == 0 and os.path.exists(tfile):
        # measured HBM bytes per launch (rocprofv3 FETCH_SIZE/WRITE_SIZE, copy-calibrated)
        rec_t = json.load(open(tfile)).get(tkey)
        traffic = rec_t["traffic_bytes"] if rec_t else None
    ifile = os.path.join(ROOT, "profiles", "issue.json")
    if args.workload == "c2" and args.variant == 0 and os.path.exists(ifile):
        # VALU issue roofline: the kernel's VALU-busy issue slots per launch (rocprofv3
        # SQ_ACTIVE_INST_VALU, 4-cycle units; a transcendental holds 2) over the slots 1024 SIMDs
        # offer in this launch's live duration at the published peak engine clock (and at the
        # clock the profiling run measured)
        rec_i = json.load(open(ifile)).get(SCAN_KERNEL + "@config2")
        if rec_i:
            slots = rec_i["valu_busy_slots"]
            pl = rec_i["per_launch"]
            clk = pl["SQ_BUSY_CYCLES"] / rec_i["shader_engines"] / (pl["duration_us"] * 1e-6) / 1e9
            peak = rec_i["simds"] * rec_i["peak_clock_ghz"] / 4  # G slots/s
            got = slots / (ms * 1e-3) / 1e9
            issue = {"bound": "valu-issue", "achieved": got, "peak": peak, "unit": "G VALU slots/s",
                     "frac": got / peak, "slots_per_launch": slots,
                     "valu_insts_per_launch": pl["SQ_INSTS_VALU"],
                     "trans_insts_per_launch": pl["SQ_INSTS_VALU_TRANS_F32"],
                     "measured_clock_ghz": clk,
                     "frac_at_measured_clock": got / (rec_i["simds"] * clk / 4)}

    rec = {
        "metric": "Mamba selective-scan fwd tokens/s + achieved HBM GB/s (% of peak), 1 GPU",
        "value": tokens * 1e3 / ms,
        "unit": "tokens/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": ms,
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "fp32" if dtype == torch.float32 else "bf16-storage/fp32-compute",
        "data": "synthetic (BASELINE config distributions, seeded torch generator)",
        "config": {"workload": workload, "batch": bt, "seq_len": L, "d_inner": dim, "d_state": N,
                   "storage": "fp32" if es == 4 else "bf16", "input_sets": nsets},
        "hbm_gbs": achieved,
        "roofline": {"bound": "hbm", "achieved": achieved, "peak": PEAK_HBM_GBS, "unit": "GB/s",
                     "frac": achieved / PEAK_HBM_GBS, "traffic": traffic,
                     "algorithmic_bytes": nbytes, "kernel_ms": ms},
        "issue_roofline": issue,
        "copy_ceiling": copy_ceiling,
        "timing": timing,
        "cpu_baseline": cpu,
        "parity_max_rel_err": parity,
    }
    print(json.dumps(rec))


if __name__ == "__main__":
    main()
