"""Fixed launch loops of one reactor entry point, for profiler runs.

A rocprofv3 counter pass wants a short program whose dispatches are the
kernel of interest, on inputs resident in device memory.  Each subcommand
uploads synthetic inputs once, runs a few launches, then `--launches` more
bracketed by device events, and prints one line with the event time.

    python3 oct_amd/workload.py gemm-bf16 4096 4096 4096 [--launches 12] [--torch]
    python3 oct_amd/workload.py dit-block [--launches 6]

`--torch` also runs torch's bf16 matmul on the same shape (hipBLASLt on
ROCm), with bf16 and with fp32 output, as a comparison under the same
counters; it is never part of the reactor's own path.
"""
from __future__ import annotations

import argparse
import os
import sys

sys.path.insert(0, os.path.abspath(os.path.join(os.path.dirname(__file__), "..")))

from oct_amd import prometheus as p  # noqa: E402
from oct_amd import synthetic as syn  # noqa: E402


def _time(rt, fn, launches: int, warm: int = 3) -> float:
    for _ in range(warm):
        fn()
    rt.synchronize()
    rt.event_record(0)
    for _ in range(launches):
        fn()
    rt.event_record(1)
    rt.synchronize()
    return rt.event_elapsed_ms(0, 1) / launches


def gemm_bf16(rt, m: int, n: int, k: int, launches: int, with_torch: bool) -> None:
    a, b = syn.to_bf16(syn.uniform(41, (m, k))), syn.to_bf16(syn.uniform(42, (k, n)))
    da, db, dc = rt.upload_new(a), rt.upload_new(b), rt.alloc(m * n * 4)
    ms = _time(rt, lambda: rt.gemm_bf16_device(da, db, dc, m, n, k), launches)
    print(f"reactor gemm_bf16 {m}x{n}x{k} fp32 out: {ms * 1e3:.1f} us {2 * m * n * k / ms / 1e9:.1f} TFLOP/s",
          flush=True)
    for d in (da, db, dc):
        rt.free(d)
    if not with_torch:
        return
    import torch

    ta = torch.from_numpy(a.view("int16")).view(torch.bfloat16).to("cuda")
    tb = torch.from_numpy(b.view("int16")).view(torch.bfloat16).to("cuda")
    for label, fn in (("bf16 out", lambda: ta @ tb), ("fp32 out", lambda: torch.mm(ta, tb, out_dtype=torch.float32))):
        for _ in range(3):
            fn()
        torch.cuda.synchronize()
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        e0.record()
        for _ in range(launches):
            fn()
        e1.record()
        torch.cuda.synchronize()
        ms = e0.elapsed_time(e1) / launches
        print(f"torch mm {m}x{n}x{k} {label}: {ms * 1e3:.1f} us {2 * m * n * k / ms / 1e9:.1f} TFLOP/s", flush=True)


def dit_block(rt, launches: int) -> None:
    grid, text, heads, ffn, cond = (64, 64), 128, 30, 10240, 256
    tokens, hidden = grid[0] * grid[1] + text, heads * 128
    arrs = syn.dit_block(5, tokens, hidden, ffn, cond, syn.joint_coordinates(grid[0], grid[1], text))
    ptrs = {name: rt.upload_new(v) for name, v in arrs.items()}
    ptrs["output"] = rt.alloc(tokens * hidden * 4)
    req = rt.dit_block_request(tokens, hidden, heads, ffn, cond, ptrs)
    ms = _time(rt, lambda: rt.dit_block_bf16_device(req), launches)
    print(f"reactor dit_block_bf16 T={tokens}: {ms:.4f} ms", flush=True)
    for d in ptrs.values():
        rt.free(d)


def main(argv=None) -> int:
    ap = argparse.ArgumentParser(description=__doc__, formatter_class=argparse.RawDescriptionHelpFormatter)
    sub = ap.add_subparsers(dest="what", required=True)
    g = sub.add_parser("gemm-bf16")
    g.add_argument("m", type=int)
    g.add_argument("n", type=int)
    g.add_argument("k", type=int)
    g.add_argument("--launches", type=int, default=12)
    g.add_argument("--torch", action="store_true")
    d = sub.add_parser("dit-block")
    d.add_argument("--launches", type=int, default=6)
    args = ap.parse_args(argv)
    if getattr(args, "torch", False):
        # torch brings its own HIP runtime library; it initialises only when
        # loaded before the reactor's
        import torch  # noqa: F401
    rt = p.NativeRuntime()
    rt.require_hardware_gpu()
    if args.what == "gemm-bf16":
        gemm_bf16(rt, args.m, args.n, args.k, args.launches, args.torch)
    else:
        dit_block(rt, args.launches)
    return 0


if __name__ == "__main__":
    sys.exit(main())
