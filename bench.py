"""Benchmark of the Prometheus hot path on one MI355X.

A *step* is one launch of the fp32 MFMA SGEMM C = A @ B at 4096^3 (BASELINE.json
configs[1], the configuration the headline metric is quoted on) with A, B
already resident in HBM.  ``value`` is TFLOP/s from the wall clock around
exactly ``--steps`` launches bracketed by device synchronisation;
``roofline.achieved`` is from HIP events recorded on the reactor's own stream
around the same launches.  Secondary figures (reductions in GB/s, the 1024^3
case, bf16, GEMV) ride along under ``"secondary"``.

Usage: python bench.py [--gpus 1] [--steps K] [--warmup W]
"""
from __future__ import annotations

import argparse
import json
import os
import sys
import time
from pathlib import Path

import numpy as np

REPO = Path(__file__).resolve().parent
sys.path.insert(0, str(REPO))

PEAK_FP32_MFMA_TFLOPS = 157.3
PEAK_BF16_MFMA_TFLOPS = 2500.0
PEAK_HBM_GBS = 8000.0
# One NoiseRefiner layer: 2*T*D*(3D + D + 3F) projection flops + 4*T^2*D attention flops,
# T = 1024, D = 3840, F = 10240.
NOISE_REFINER_FLOP = 2.0 * 1024 * 3840 * (3 * 3840 + 3840 + 3 * 10240) + 4.0 * 1024 * 1024 * 3840


def _settle(rt, launch, settle_ms: float) -> int:
    """Untimed launches for at least ``settle_ms`` of wall time, so that the GPU
    clock has left its idle ramp (per-launch time at 4096^3 falls from 1.17 to
    0.93 ms over the first ~30 launches of a fresh process) before the warm-up
    and timed launches.  Returns the number of launches made."""
    if settle_ms <= 0:
        return 0
    launches, t0 = 0, time.perf_counter()
    while (time.perf_counter() - t0) * 1e3 < settle_ms:
        for _ in range(8):
            launch()
        rt.synchronize()
        launches += 8
    return launches


def _timed_launches(rt, launch, steps: int, warmup: int, settle_ms: float = 0.0):
    """Returns (wall_ms_per_step, event_ms_per_step).  ``settle_ms`` of untimed
    launches come first (see ``_settle``): a secondary leg follows seconds of host
    work (input generation, uploads) during which the clock falls back."""
    _settle(rt, launch, settle_ms)
    for _ in range(warmup):
        launch()
    rt.synchronize()
    t0 = time.perf_counter()
    rt.event_record(0)
    for _ in range(steps):
        launch()
    rt.event_record(1)
    rt.synchronize()
    t1 = time.perf_counter()
    ev = rt.event_elapsed_ms(0, 1)
    return (t1 - t0) * 1e3 / steps, ev / steps


def _traffic_from_profiles(name: str):
    path = REPO / "profiles" / "traffic.json"
    if not path.exists():
        return None
    try:
        return json.loads(path.read_text()).get(name)
    except (OSError, ValueError):
        return None


class _OneCore:
    """Pins this process to one of the cores it may use (Oct's CPU `@` is single-threaded)."""

    def __enter__(self):
        self.prev = os.sched_getaffinity(0)
        self.core = min(self.prev)
        os.sched_setaffinity(0, {self.core})
        return self

    def __exit__(self, *exc):
        os.sched_setaffinity(0, self.prev)


def cpu_baseline_sgemm(a32: np.ndarray, b32: np.ndarray, gpu_rows: dict, seconds: float):
    """Oct's compiled CPU `@` (__octMatMulMM restatement, binary64 ijk, one thread pinned to
    one core) on a row sample of the benchmark's own operands; also checks the GPU's output
    rows against the oracle."""
    import oracle

    n = a32.shape[0]
    parity = max(oracle.normwise_rel_err(row, oracle.matmul_f64(a32, b32, rows=(r, r + 1))[r])
                 for r, row in gpu_rows.items())
    a = a32.astype(np.float64)
    b = b32.astype(np.float64)
    rows = 0
    with _OneCore() as pin:
        t0 = time.perf_counter()
        while rows < n:
            oracle.matmul_compiled_f64(a, b, rows=(rows, rows + 1))
            rows += 1
            if time.perf_counter() - t0 >= seconds:
                break
        dt = time.perf_counter() - t0
    flops = 2.0 * rows * n * n
    return parity, {
        "value": round(flops / dt / 1e12, 6),
        "unit": "TFLOP/s",
        "cores": 1,
        "kind": "port",
        "sample": f"rows 0..{rows - 1} of the {n}^3 product ({rows}/{n} rows, {dt:.1f} s): "
                  f"__octMatMulMM (emit_go_runtime.go:168-205) restated in C, binary64 ijk, 1 thread pinned "
                  f"to core {pin.core}; host has {len(pin.prev)} usable logical CPUs",
    }


def _blas_threads() -> int:
    try:
        from threadpoolctl import threadpool_info

        return max((i.get("num_threads", 1) for i in threadpool_info() if i.get("user_api") == "blas"), default=1)
    except Exception:  # noqa: BLE001 - informational only
        return 1


def cpu_baseline_secondary(seconds: float):
    """CPU timings of the oracles for the secondary rows (bounded samples).

    Reductions: the reference's prom_reduction_cpu_reference / RMSNorm CPU
    oracle restated in C (scalar, one thread) over the full [8192, 4096]
    input.  Decoder layer: the binary64 numpy restatement of the C4 layer
    (BLAS threads as reported)."""
    import oracle
    from oracle import blocks

    out = {}
    # C1 in full: 1024^3 through the __octMatMulMM restatement on one pinned core
    a1 = oracle.uniform(1, (1024, 1024)).astype(np.float64)
    b1 = oracle.uniform(2, (1024, 1024)).astype(np.float64)
    with _OneCore():
        t0 = time.perf_counter()
        oracle.matmul_compiled_f64(a1, b1)
        dt = time.perf_counter() - t0
    out["sgemm_1024_full_s"] = round(dt, 3)
    out["sgemm_1024_full_tflops"] = round(2.0 * 1024 ** 3 / dt / 1e12, 6)
    out["sgemm_1024_cores"] = 1
    del a1, b1
    rows, width = 8192, 4096
    x = oracle.normal(77, (rows, width))
    for op, name, nbytes in ((3, "softmax", 2 * x.nbytes), (1, "row_sum", x.nbytes + rows * 4),
                             (2, "row_max", x.nbytes + rows * 4)):
        reps, t0 = 0, time.perf_counter()
        while True:
            oracle.reduction_reference(x, op)
            reps += 1
            dt = time.perf_counter() - t0
            if dt >= min(2.0, seconds / 4) or reps >= 20:
                break
        out[f"{name}_8192x4096_gbs"] = round(nbytes * reps / dt / 1e9, 3)
    w = (1.0 + oracle.normal(89, (width,), 0.0, 0.02)).astype(np.float32)
    reps, t0 = 0, time.perf_counter()
    while True:
        oracle.rmsnorm_reference(x, w, 1e-6)
        reps += 1
        dt = time.perf_counter() - t0
        if dt >= min(2.0, seconds / 4) or reps >= 20:
            break
    out["rmsnorm_8192x4096_gbs"] = round((2 * x.nbytes + w.nbytes + rows * 4) * reps / dt / 1e9, 3)
    out["reductions_cores"] = 1
    del x
    T, D, Hq, hd, F = 512, 2048, 8, 256, 16384
    xx, wl = blocks.make_decoder_layer(4, T, D, Hq, hd, F)
    t0 = time.perf_counter()
    blocks.decoder_layer_f32(xx, wl, Hq, hd)
    out["gemma2b_layer_f64_t512_ms"] = round((time.perf_counter() - t0) * 1e3, 1)
    out["gemma2b_layer_cores"] = _blas_threads()
    # C5: the binary64 block oracle on a row subset of the full 4224-token input
    grid, text, heads, F5, C = (64, 64), 128, 30, 10240, 256
    T5 = grid[0] * grid[1] + text
    x5, cond5, w5 = blocks.make_dit_block(5, T5, heads * 128, F5, C)
    coords5 = blocks.joint_coordinates(grid[0], grid[1], text)
    sub = np.arange(0, T5, T5 // 64)[:64]
    t0 = time.perf_counter()
    blocks.dit_block_bf16(x5, coords5, cond5, w5, heads, rows=sub)
    out["dit_block_bf16_t4224_rows64_f64_ms"] = round((time.perf_counter() - t0) * 1e3, 1)
    out["dit_block_cores"] = _blas_threads()
    del x5, w5
    xf = oracle.normal(31, (2 << 20,)).astype(np.float64).view(np.complex128)
    reps, t0 = 0, time.perf_counter()
    while True:
        oracle.fft64(xf)
        reps += 1
        dt = time.perf_counter() - t0
        if dt >= min(2.0, seconds / 4) or reps >= 20:
            break
    out["fft64_2p20_us"] = round(dt / reps * 1e6, 1)
    out["kind"] = "port"
    out["sample"] = ("sgemm_1024: the full C1 product, __octMatMulMM restated in C, binary64, one pinned core; "
                     "reductions: one full [8192,4096] pass per repetition (C oracle, fp32 data, binary64 sums); "
                     "layer: one full T=512 Gemma-2B-shaped layer in binary64 numpy; "
                     "dit_block: the C5 block in binary64 numpy for 64 of the 4224 output tokens (Q, attention "
                     "and FFN for those rows; K and V projected for all tokens), BLAS threads as dit_block_cores; "
                     "fft64: internal/fft/fft.go's radix-2 restated in C, one thread, 2^20 points (twiddles included)")
    return out


def main() -> int:
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=50)
    ap.add_argument("--warmup", type=int, default=20)
    ap.add_argument("--cpu-seconds", type=float, default=12.0)
    ap.add_argument("--settle-ms", type=float, default=150.0,
                    help="untimed headline launches before the warm-up, so the clock has ramped (reported); "
                         "each secondary leg settles for a third of it")
    ap.add_argument("--no-secondary", action="store_true")
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--copy-calibration-mib", type=int, default=0,
                    help="first run a plain device copy of this many MiB (10 launches) so that rocprofv3 "
                         "FETCH_SIZE/WRITE_SIZE can be scaled against known bytes")
    args = ap.parse_args()
    world = int(os.environ.get("WORLD_SIZE", "1"))
    if args.gpus != 1 or world != 1:
        print("bench.py measures one MI355X: this build runs every configuration on a single GPU "
              "(no collectives); run it with --gpus 1", file=sys.stderr)
        return 2

    from oct_amd import prometheus as p
    from oct_amd import synthetic as syn

    if args.copy_calibration_mib:
        import torch

        src = torch.ones(args.copy_calibration_mib << 18, dtype=torch.float32, device="cuda:0")
        dst = torch.empty_like(src)
        for _ in range(10):
            dst.copy_(src)
        torch.cuda.synchronize()
        print(f"copy calibration: 10 x {args.copy_calibration_mib} MiB read + written", file=sys.stderr)

    rt = p.NativeRuntime()
    rt.require_hardware_gpu()
    diag = rt.device_diagnostics()

    # ---- headline: fp32 SGEMM 4096^3 ------------------------------------------
    n = 4096
    a = syn.uniform(11, (n, n))
    b = syn.uniform(12, (n, n))
    da, db, dc = rt.alloc(a.nbytes), rt.alloc(b.nbytes), rt.alloc(a.nbytes)
    rt.upload(da, a)
    rt.upload(db, b)
    headline = lambda: rt.sgemm_device(da, db, dc, n, n, n)  # noqa: E731
    settle_launches = _settle(rt, headline, args.settle_ms)
    wall_ms, ev_ms = _timed_launches(rt, headline, args.steps, args.warmup)
    flops = 2.0 * n * n * n
    value = flops / (wall_ms * 1e-3) / 1e12
    achieved = flops / (ev_ms * 1e-3) / 1e12
    line = {
        "metric": "SGEMM fp32 TFLOP/s @4096^3 (% MFMA peak)",
        "value": round(value, 3),
        "unit": "TFLOP/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "settle_ms": args.settle_ms,
        "settle_launches": settle_launches,
        "ms_per_step": round(wall_ms, 4),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "f32",
        "data": "synthetic: A,B ~ U[-1,1] (numpy PCG64 seeds 11,12), fp32 row-major, resident in HBM",
        "config": {"workload": "sgemm_f32 C=A@B M=N=K=4096 row-major (BASELINE configs[1])", "m": n, "n": n, "k": n,
                   "kernel": "sgemm_f32_dl128w8_kernel (v_mfma_f32_32x32x2_f32, 128x128x16 tiles loaded HBM->LDS directly, 8 waves of 32x64, 3 workgroups per CU)"},
        "roofline": {
            "bound": "mfma",
            "achieved": round(achieved, 3),
            "peak": PEAK_FP32_MFMA_TFLOPS,
            "unit": "TFLOP/s",
            "frac": round(achieved / PEAK_FP32_MFMA_TFLOPS, 4),
            "traffic": _traffic_from_profiles("sgemm_f32_4096"),
            "algorithmic_flop_per_launch": flops,
            "event_ms_per_launch": round(ev_ms, 5),
        },
        "device": {"name": diag.device_name.decode(), "arch": diag.gcn_arch_name.decode(),
                   "cus": diag.compute_units, "clock_mhz": diag.clock_khz // 1000},
    }
    # rows of the measured output, checked against the oracle in the CPU-baseline leg
    out_all = rt.download(np.empty((n, n), np.float32), dc)
    gpu_rows = {r: out_all[r].copy() for r in (0, 1777, n - 1)}
    del out_all
    for d in (da, db, dc):
        rt.free(d)
    if not args.no_secondary:
        # the reference's synchronous host-pointer contract: copies in and out over PCIe included
        for _ in range(2):
            rt.sgemm(n, n, n, a, b)
        t0 = time.perf_counter()
        for _ in range(3):
            rt.sgemm(n, n, n, a, b)
        e2e = (time.perf_counter() - t0) / 3
        line["host_pointer_e2e"] = {"ms": round(e2e * 1e3, 3), "tflops": round(flops / e2e / 1e12, 2),
                                    "note": "prometheus_reactor_runtime_sgemm with host A, B, C (H2D 128 MiB, "
                                            "D2H 64 MiB included); not the headline value"}

    if not args.no_secondary:
        sec = {}
        leg_settle = args.settle_ms / 3
        # fp32 1024^3
        m1 = 1024
        a1, b1 = syn.uniform(1, (m1, m1)), syn.uniform(2, (m1, m1))
        d1 = [rt.alloc(a1.nbytes) for _ in range(3)]
        rt.upload(d1[0], a1)
        rt.upload(d1[1], b1)
        _, ev = _timed_launches(rt, lambda: rt.sgemm_device(d1[0], d1[1], d1[2], m1, m1, m1), 50, 5, leg_settle)
        sec["sgemm_f32_1024_tflops"] = round(2.0 * m1 ** 3 / (ev * 1e-3) / 1e12, 3)
        for d in d1:
            rt.free(d)
        # ragged and GEMV
        for (m, nn, k, key) in ((1000, 1000, 1000, "sgemm_f32_1000_tflops"),
                                (4097, 3001, 513, "sgemm_f32_4097x3001x513_tflops")):
            aa, bb = syn.uniform(3, (m, k)), syn.uniform(4, (k, nn))
            dd = [rt.alloc(aa.nbytes), rt.alloc(bb.nbytes), rt.alloc(m * nn * 4)]
            rt.upload(dd[0], aa)
            rt.upload(dd[1], bb)
            _, ev = _timed_launches(rt, lambda: rt.sgemm_device(dd[0], dd[1], dd[2], m, nn, k), 30, 5, leg_settle)
            sec[key] = round(2.0 * m * nn * k / (ev * 1e-3) / 1e12, 3)
            for d in dd:
                rt.free(d)
        m, k = 8192, 4096
        aa, xx = syn.uniform(7, (m, k)), syn.uniform(8, (k, 1))
        dd = [rt.alloc(aa.nbytes), rt.alloc(xx.nbytes), rt.alloc(m * 4)]
        rt.upload(dd[0], aa)
        rt.upload(dd[1], xx)
        _, ev = _timed_launches(rt, lambda: rt.sgemm_device(dd[0], dd[1], dd[2], m, 1, k), 100, 10, leg_settle)
        sec["gemv_f32_8192x4096_gbs"] = round((m * k + k + m) * 4 / (ev * 1e-3) / 1e9, 1)
        for d in dd:
            rt.free(d)
        # bf16 4096^3
        ab, bbf = syn.to_bf16(syn.uniform(41, (n, n))), syn.to_bf16(syn.uniform(42, (n, n)))
        dd = [rt.alloc(ab.nbytes), rt.alloc(bbf.nbytes), rt.alloc(n * n * 4)]
        rt.upload(dd[0], ab)
        rt.upload(dd[1], bbf)
        _, ev = _timed_launches(rt, lambda: rt.gemm_bf16_device(dd[0], dd[1], dd[2], n, n, n), 30, 5, leg_settle)
        tf = flops / (ev * 1e-3) / 1e12
        sec["gemm_bf16_4096_tflops"] = round(tf, 2)
        sec["gemm_bf16_4096_frac"] = round(tf / PEAK_BF16_MFMA_TFLOPS, 4)
        for d in dd:
            rt.free(d)
        # reductions on [8192, 4096]
        rows, width = 8192, 4096
        x = syn.normal(77, (rows, width))
        dx, dy = rt.alloc(x.nbytes), rt.alloc(x.nbytes)
        rt.upload(dx, x)
        for op, name, nbytes in ((p.OP_SOFTMAX, "softmax", 2 * x.nbytes), (p.OP_SUM, "row_sum", x.nbytes + rows * 4),
                                 (p.OP_MAX, "row_max", x.nbytes + rows * 4)):
            _, ev = _timed_launches(rt, lambda: rt.reduction_device(dx, dy, rows, width, op), 100, 10, leg_settle)
            gbs = nbytes / (ev * 1e-3) / 1e9
            sec[f"{name}_8192x4096_gbs"] = round(gbs, 1)
            sec[f"{name}_8192x4096_frac"] = round(gbs / PEAK_HBM_GBS, 4)
        w = syn.normal(89, (width,), 1.0, 0.02)
        dw, dinv = rt.alloc(w.nbytes), rt.alloc(rows * 4)
        rt.upload(dw, w)
        _, ev = _timed_launches(rt, lambda: rt.rmsnorm_device(dx, dw, dy, dinv, rows, width, width, 1e-6), 100, 10, leg_settle)
        gbs = (2 * x.nbytes + w.nbytes + rows * 4) / (ev * 1e-3) / 1e9
        sec["rmsnorm_8192x4096_gbs"] = round(gbs, 1)
        sec["rmsnorm_8192x4096_frac"] = round(gbs / PEAK_HBM_GBS, 4)
        for d in (dx, dy, dw, dinv):
            rt.free(d)
        # transformer layers, weights resident
        T, D, Hq, hd, F = 512, 2048, 8, 256, 16384
        ptrs = syn.decoder_layer(4, T, D, Hq, hd, F)
        dptr = {k: rt.upload_new(np.ascontiguousarray(v, np.float32)) for k, v in ptrs.items()}
        dptr["output"] = rt.alloc(T * D * 4)
        req = rt.decoder_layer_request(T, D, Hq, hd, F, dptr)
        _, ev = _timed_launches(rt, lambda: rt.decoder_layer_f32_device(req), 10, 3, leg_settle)
        sec["gemma2b_layer_f32_t512_ms"] = round(ev, 4)
        sec["gemma2b_layer_f32_t512_tflops"] = round(1.149e11 / (ev * 1e-3) / 1e12, 2)
        for d in dptr.values():
            rt.free(d)
        del ptrs
        grid, text, heads, F5, C = (64, 64), 128, 30, 10240, 256
        T5 = grid[0] * grid[1] + text
        D5 = heads * 128
        arrs = syn.dit_block(5, T5, D5, F5, C, syn.joint_coordinates(grid[0], grid[1], text))
        dptr = {k: rt.upload_new(v) for k, v in arrs.items()}
        dptr["output"] = rt.alloc(T5 * D5 * 4)
        req = rt.dit_block_request(T5, D5, heads, F5, C, dptr)
        _, ev = _timed_launches(rt, lambda: rt.dit_block_bf16_device(req), 10, 3, leg_settle)
        sec["dit_block_bf16_t4224_ms"] = round(ev, 4)
        sec["dit_block_bf16_t4224_tflops"] = round(1.769e12 / (ev * 1e-3) / 1e12, 2)
        for d in dptr.values():
            rt.free(d)
        # binary64 FFT, 2^20 points (device entry: two four-step passes)
        nf = 1 << 20
        xf = syn.normal(31, (2 * nf,)).astype(np.float64).view(np.complex128)
        dfi, dfo = rt.upload_new(xf.view(np.float64)), rt.alloc(xf.nbytes)
        _, ev = _timed_launches(rt, lambda: rt.fft64_device(dfi, dfo, nf), 100, 10, leg_settle)
        sec["fft64_2p20_us"] = round(ev * 1e3, 2)
        gbs = 2 * xf.nbytes / (ev * 1e-3) / 1e9
        sec["fft64_2p20_gbs"] = round(gbs, 1)
        sec["fft64_2p20_frac"] = round(gbs / PEAK_HBM_GBS, 4)
        for d in (dfi, dfo):
            rt.free(d)
        # resident model block: one Z-Image NoiseRefiner layer (1024 tokens, fp32 on
        # resident FP16-widened weights), chained on its own resident output
        from oct_amd import model_block as mb

        mrt = p.NativeRuntime()
        model = mb.ResidentModel(mrt)
        wz = syn.zimage_weights(1)
        rc, bid, _ = model.noise_refiner_create(wz)
        x_bits = syn.to_bf16(syn.normal(2, (1024, 3840)))
        t_bits = syn.to_bf16(syn.normal(3, (256,)))
        ok = (rc == p.PROM_OK and model.noise_refiner_execute(bid, x_bits, t_bits)[0] == p.PROM_OK
              and model.noise_refiner_rebind(bid, wz)[0] == p.PROM_OK)
        if ok:
            times = []
            for _ in range(13):
                rc, ev = model.noise_refiner_resident(bid, 1)
                times.append(ev.gpu_compute_ns / 1e6)
            ms = float(np.median(times[3:]))
            sec["zimage_noise_refiner_f32_ms"] = round(ms, 4)
            sec["zimage_noise_refiner_f32_tflops"] = round(NOISE_REFINER_FLOP / (ms * 1e-3) / 1e12, 2)
            sec["zimage_noise_refiner_f32_frac"] = round(NOISE_REFINER_FLOP / (ms * 1e-3) / 1e12 /
                                                         PEAK_FP32_MFMA_TFLOPS, 4)
        mrt.close()
        del wz
        line["secondary"] = sec

    rt.close()
    line["cpu_baseline"] = None
    if not args.no_cpu_baseline:
        parity, line["cpu_baseline"] = cpu_baseline_sgemm(a, b, gpu_rows, args.cpu_seconds)
        line["parity_rows_normwise_max"] = float(parity)
    if not args.no_cpu_baseline and not args.no_secondary:
        line["secondary_cpu_baseline"] = cpu_baseline_secondary(args.cpu_seconds)
    print(json.dumps(line), flush=True)
    return 0


if __name__ == "__main__":
    sys.exit(main())
