"""Decode throughput of the gfx950 BF16 weight decoder on one MI355X.

Workload: one 5120x17408 bf16 weight (N(0, 0.02) with 0.1% N(0, 0.5)
outliers, seed 2), compressed with a per-tensor canonical-Huffman exponent
codebook in chunks of 65536 symbols (1360 chunks). Its compressed form
(bitstreams, chunk offsets/lengths, sign/mantissa bytes, decode table) is
resident in HBM before timing starts. One step = one kernel launch that
rebuilds the whole bf16 tensor in HBM. Prints one JSON line.

    python bench.py [--steps K] [--warmup W] [--gpus 1] [--no-cpu-baseline]
"""
from __future__ import annotations

import argparse
import ctypes
import json
import os
import sys
import time
from pathlib import Path

import numpy as np
import torch

ROOT = Path(__file__).resolve().parent
METRIC = "decompressed BF16 GB/s per MI355X (+% HBM roofline); bit-exact vs reference"
HBM_PEAK_GBS = 8000.0
TRAFFIC_FILE = ROOT / "profiles" / "decode_bf16_5120x17408_traffic.json"


def _log(msg: str) -> None:
    print("[bench] " + msg, file=sys.stderr, flush=True)


def _cpu_baseline(layer, max_threads: int) -> dict:
    """The reference's CPU decode path (chunk decode + recombine), restated in
    C/OpenMP in oracle/, timed on this host's cores on a bounded sample."""
    import oracle

    oracle.build()
    threads = max(1, min(max_threads, oracle.max_threads()))
    sm = layer.sign_mantissa.numpy()
    enc = layer.encoded
    # Sample: the whole tensor, repeated until ~10 s of work at `threads`.
    res = oracle.time_cpu_decode(enc, sm, threads, min_seconds=10.0, max_reps=40)
    n = enc.n_symbols
    # One thread on a 40-chunk slice of the same tensor (reported as context).
    from afterimage_amd.runtime.compressed_store import _slice_encoded

    sub = _slice_encoded(enc, 0, 40)
    one = oracle.time_cpu_decode(sub, sm[: sub.n_symbols], 1, min_seconds=2.0, max_reps=5)
    return {
        "value": round(2 * n / res["median_s"] / 1e9, 3),
        "unit": "GB/s",
        "cores": threads,
        "kind": "port",
        "sample": "whole 5120x17408 tensor x%d reps, chunk decode + recombine, median rep"
                  % res["reps"],
        "exponent_bytes_gbs": round(n / res["median_s"] / 1e9, 3),
        "one_thread_gbs": round(2 * sub.n_symbols / one["median_s"] / 1e9, 3),
        "one_thread_sample": "chunks 0..39 of the same tensor (2.6M symbols)",
    }


def _traffic(config_key: str):
    if not TRAFFIC_FILE.exists():
        return None
    try:
        rec = json.loads(TRAFFIC_FILE.read_text())
    except ValueError:
        return None
    if rec.get("config_key") != config_key:
        return None
    return rec.get("hbm_bytes_per_launch")


def _copy_calibration(mib: int, steps: int, warmup: int) -> int:
    """Copy mib MiB device-to-device `steps` times: each launch reads and
    writes exactly mib MiB, which calibrates FETCH_SIZE / WRITE_SIZE."""
    dev = torch.device("cuda", 0)
    n = mib << 20
    src = torch.randint(0, 255, (n,), dtype=torch.uint8, device=dev)
    dst = torch.empty_like(src)
    for _ in range(warmup):
        dst.copy_(src)
    torch.cuda.synchronize(dev)
    t0 = time.perf_counter()
    for _ in range(steps):
        dst.copy_(src)
    torch.cuda.synchronize(dev)
    dt = (time.perf_counter() - t0) / steps
    print(json.dumps({"copy_bytes_per_launch": n, "steps": steps,
                      "us_per_copy": round(dt * 1e6, 2),
                      "gbs_read_plus_write": round(2 * n / dt / 1e9, 1)}), flush=True)
    return 0


def main() -> int:
    ap = argparse.ArgumentParser(description=__doc__.split("\n\n")[0])
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=200)
    ap.add_argument("--warmup", type=int, default=20)
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--cpu-threads", type=int, default=16)
    ap.add_argument("--copy-mib", type=int, default=0,
                    help="instead of decoding, time a plain device copy of this many MiB "
                         "(the reference kernel for scaling HBM byte counters)")
    args = ap.parse_args()
    world = int(os.environ.get("WORLD_SIZE", "1"))
    if args.gpus != 1 or world != 1:
        print("bench.py measures one GPU only: this build has no multi-GPU decode path "
              "(chunks would shard by range with no exchange step). Run with --gpus 1.",
              file=sys.stderr)
        return 2
    if args.steps < 1 or args.warmup < 0:
        print("--steps must be >= 1 and --warmup >= 0", file=sys.stderr)
        return 2

    if args.copy_mib:
        return _copy_calibration(args.copy_mib, args.steps, args.warmup)

    from afterimage_amd import _native, workloads
    from afterimage_amd.runtime.device import DeviceTensor, _descriptor

    dev = torch.device("cuda", 0)
    torch.cuda.set_device(dev)
    seed = 2
    t0 = time.perf_counter()
    W, layer = workloads.single_layer(seed=seed)
    enc = layer.encoded
    _log("workload built in %.1fs: %d chunks, packed %.2f MB"
         % (time.perf_counter() - t0, enc.n_chunks, enc.packed.nbytes / 1e6))
    dt = DeviceTensor.from_encoded(enc, layer.sign_mantissa, dev)
    n = enc.n_symbols
    out = torch.empty(n, dtype=torch.bfloat16, device=dev)
    desc = (_native.AimgTensor * 1)()
    desc[0] = _descriptor(dt, out, n)
    lib = _native.lib()
    stream = torch.cuda.current_stream(dev)
    handle = ctypes.c_void_p(stream.cuda_stream)
    decode = lib.aimg_decode_bf16

    def step():
        rc = decode(desc, 1, handle)
        if rc:
            _native.check(rc)

    for _ in range(args.warmup):
        step()
    torch.cuda.synchronize(dev)
    # Bit-exactness of the benchmarked output (outside the timed region).
    ok = torch.equal(out.view(torch.int16).cpu(), W.reshape(-1).view(torch.int16))
    if not ok:
        print("decoded output differs from the original weights", file=sys.stderr)
        return 1
    _log("warmup done, output bit-exact")

    ev0 = torch.cuda.Event(enable_timing=True)
    ev1 = torch.cuda.Event(enable_timing=True)
    torch.cuda.synchronize(dev)
    t_start = time.perf_counter()
    ev0.record(stream)
    for _ in range(args.steps):
        step()
    ev1.record(stream)
    torch.cuda.synchronize(dev)
    wall = time.perf_counter() - t_start
    kernel_s = ev0.elapsed_time(ev1) / 1e3 / args.steps
    _log("timed %d steps: wall %.3f ms/step, events %.1f us/launch"
         % (args.steps, wall * 1e3 / args.steps, kernel_s * 1e6))

    chunk_bytes = int(enc.chunk_nbytes.astype(np.int64).sum())
    # bitstreams + offsets and lengths + sign/mantissa + window table + bf16 write
    algo_bytes = chunk_bytes + 8 * enc.n_chunks + n + 6 * 4096 + 2 * n
    achieved = algo_bytes / kernel_s / 1e9
    value = 2 * n * args.steps / wall / 1e9
    config_key = "5120x17408/seed%d/chunk65536/outliers1e-3" % seed
    traffic = _traffic(config_key)
    rec = {
        "metric": METRIC,
        "value": round(value, 2),
        "unit": "GB/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(wall * 1e3 / args.steps, 5),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "u8",
        "data": "synthetic",
        "config": {
            "workload": "bf16 5120x17408 weight decode, N(0,0.02) + 0.1% N(0,0.5) outliers "
                        "(seed 2), per-tensor Huffman exponent codebook, 65536-symbol "
                        "chunks (1360), inputs resident in HBM, one launch per step",
            "config_key": config_key,
            "n_weights": n,
            "packed_exponent_bytes": chunk_bytes,
            "bits_per_exponent": round(8 * chunk_bytes / n, 4),
            "bit_exact": ok,
        },
        "roofline": {
            "bound": "hbm",
            "achieved": round(achieved, 1),
            "peak": HBM_PEAK_GBS,
            "unit": "GB/s",
            "frac": round(achieved / HBM_PEAK_GBS, 4),
            "traffic": traffic,
            "algorithmic_bytes_per_launch": algo_bytes,
            "kernel_us": round(kernel_s * 1e6, 2),
        },
        "cpu_baseline": None,
    }
    if not args.no_cpu_baseline:
        _log("timing the CPU baseline (~15 s)")
        rec["cpu_baseline"] = _cpu_baseline(layer, args.cpu_threads)
    print(json.dumps(rec), flush=True)
    return 0


if __name__ == "__main__":
    sys.exit(main())
