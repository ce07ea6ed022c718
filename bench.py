"""Decode throughput of the gfx950 BF16 weight decoder on one MI355X.

Headline (value and roofline of the default run): one 5120x17408 bf16 weight
(N(0, 0.02) with 0.1% N(0, 0.5) outliers, seed 2), compressed with a
per-tensor canonical-Huffman exponent codebook in chunks of 65536 symbols
(1360 chunks), its store-format arrays (bitstreams, chunk offsets/lengths,
sign/mantissa bytes) and decode table in HBM before timing starts, and
nothing else: no derived data. One step = one kernel launch that rebuilds the
whole bf16 tensor in HBM, the decode decompress_layer_gpu and the streamed
ring run. The same launches over three copies of the layer in turn
("cold_inputs") read their inputs from HBM rather than the last-level cache.

The default run ("suite") adds, as extra keys of the same line, each timed in
this run: the layer at the reference store's default 1024-symbol chunks; the
layer with a prebuilt segment index (the compressed-resident tier, with its
build time); a small 1024x3072 layer; a 14B-class block in one launch; 40
streamed blocks through a 2-slot ring; the fused decode->GEMV at batch 1 and
4 and the fused decode->GEMM at 8 and 16 rows of x, at both chunk sizes; and
the 151936x5120 lm_head at 8 tokens, blocked against fused. Prints one JSON
line.

    python bench.py [--steps K] [--warmup W] [--gpus 1]
                    [--workload suite|layer|block|gemv|ring|api|head|resync]
                    [--chunk-size N] [--batch B] [--slice-rows R] [--index] [--no-cold]
                    [--no-cpu-baseline] [--cpu-threads T]
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


def _host_cpu() -> dict:
    """This host's CPU as the baseline ran on it: model name, online CPUs,
    the CPUs this process may use, and OpenMP's thread count (which
    follows OMP_NUM_THREADS, the host's CPU share for one GPU)."""
    model = ""
    try:
        for line in open("/proc/cpuinfo"):
            if line.startswith("model name"):
                model = line.split(":", 1)[1].strip()
                break
    except OSError:
        pass
    try:
        usable = len(os.sched_getaffinity(0))
    except AttributeError:
        usable = os.cpu_count() or 1
    return {"model": model, "nproc": os.cpu_count(), "usable_cpus": usable,
            "omp_num_threads": os.environ.get("OMP_NUM_THREADS")}


def _cpu_baseline(layers, max_threads: int, what: str) -> dict:
    """The reference's CPU decode path (chunk decode + recombine), restated in
    C/OpenMP in oracle/, timed on this host's cores on a bounded sample: at
    OpenMP's thread count (every CPU this process is given) unless
    --cpu-threads asks for fewer, and on one thread."""
    import oracle

    oracle.build()
    threads = oracle.max_threads() if max_threads <= 0 else max(1, min(max_threads,
                                                                    oracle.max_threads()))
    total_s = 0.0
    reps = []
    n = 0
    # Sample: every tensor of the workload, each repeated until ~10 s of work
    # in all at `threads`.
    per_tensor = 10.0 / len(layers)
    for layer in layers:
        res = oracle.time_cpu_decode(layer.encoded, layer.sign_mantissa.numpy(), threads,
                                     min_seconds=per_tensor, max_reps=40)
        total_s += res["median_s"]
        reps.append(res["reps"])
        n += layer.encoded.n_symbols
    # One thread on a 40-chunk slice of the largest tensor (reported as context).
    from afterimage_amd.runtime.compressed_store import _slice_encoded

    big = max(layers, key=lambda l: l.encoded.n_symbols)
    sub = _slice_encoded(big.encoded, 0, min(40, big.encoded.n_chunks))
    one = oracle.time_cpu_decode(sub, big.sign_mantissa.numpy()[: sub.n_symbols], 1,
                                 min_seconds=2.0, max_reps=5)
    return {
        "value": round(2 * n / total_s / 1e9, 3),
        "unit": "GB/s",
        "cores": threads,
        "kind": "port",
        "sample": "%s: each tensor decoded whole (chunk decode + recombine), %s reps, "
                  "median rep per tensor" % (what, "/".join(str(r) for r in reps)),
        "exponent_bytes_gbs": round(n / total_s / 1e9, 3),
        "one_thread_gbs": round(2 * sub.n_symbols / one["median_s"] / 1e9, 3),
        "one_thread_sample": "first %d chunks of the largest tensor (%d symbols)"
                             % (sub.n_chunks, sub.n_symbols),
        "host": _host_cpu(),
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


def _bench_ring(args) -> int:
    rec = _ring(args)
    if rec is None:
        return 1
    print(json.dumps(rec), flush=True)
    return 0


def _ring(args, blocks=None) -> dict | None:
    """Streamed 14B-class blocks: two distinct compressed blocks in pinned host
    memory, cycled through `--layers` layers per step; H2D on a side stream,
    decode on the compute stream, 2-slot ring under a 4 GiB device budget.
    Returns the JSON record, or None when a decoded layer is not bit-exact."""
    from afterimage_amd import workloads
    from afterimage_amd.runtime.stream_ring import HostBlock, LayerRing

    dev = torch.device("cuda", 0)
    torch.cuda.set_device(dev)
    t0 = time.perf_counter()
    if blocks is None:
        blocks = [workloads.block_14b(seed=s) for s in (3, 4)]
    hbs = [HostBlock([l for _, _, l in blk]) for blk in blocks]
    _log("2 blocks built and pinned in %.1fs: %.1f MB compressed each"
         % (time.perf_counter() - t0, hbs[0].nbytes / 1e6))
    ring = LayerRing(hbs, device=dev, slots=2, vram_budget=4 << 30)
    refs = [[w.reshape(-1).view(torch.int16) for _, w, _ in blk] for blk in blocks]
    # Warmup pass, with a bit-exact check of each distinct block.
    ok = True
    for k, tensors in ring.stream(max(2, min(args.warmup, args.layers))):
        if k < 2:
            ok = ok and all(torch.equal(t.reshape(-1).view(torch.int16).cpu(), r)
                            for t, r in zip(tensors, refs[k % 2]))
    torch.cuda.synchronize(dev)
    if not ok:
        print("streamed decode differs from the original weights", file=sys.stderr)
        return None
    ring.timing = True
    walls = []
    dec_s = []
    for _ in range(args.steps):
        torch.cuda.synchronize(dev)
        t_start = time.perf_counter()
        for _k, _t in ring.stream(args.layers):
            pass
        torch.cuda.synchronize(dev)
        walls.append(time.perf_counter() - t_start)
        dec_s.append(sum(a.elapsed_time(b) for a, b in ring.decode_events) / 1e3)
    wall = sorted(walls)[len(walls) // 2]
    decode = sorted(dec_s)[len(dec_s) // 2]
    # Pinned H2D alone, for context.
    s = torch.cuda.Stream(dev)
    slot = torch.empty(hbs[0].nbytes, dtype=torch.uint8, device=dev)
    e0 = torch.cuda.Event(enable_timing=True)
    e1 = torch.cuda.Event(enable_timing=True)
    with torch.cuda.stream(s):
        e0.record(s)
        for _ in range(4):
            slot.copy_(hbs[0].buf, non_blocking=True)
        e1.record(s)
    torch.cuda.synchronize(dev)
    h2d_gbs = 4 * hbs[0].nbytes / (e0.elapsed_time(e1) / 1e3) / 1e9
    decoded = sum(hb.decoded_nbytes for hb in hbs) / len(hbs)
    rec = {
        "metric": "streamed 14B-class blocks: end-to-end layers/s (H2D + decode)",
        "value": round(args.layers / wall, 2),
        "unit": "layers/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(wall * 1e3, 3),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "bf16",
        "data": "synthetic",
        "config": {"workload": "%d layers of the 14B-class block (2 distinct blocks, seeds 3/4, "
                               "cycled), compressed in pinned host memory, H2D on a side stream, "
                               "2-slot ring" % args.layers,
                   "ring_device_bytes": ring.ring_bytes, "vram_budget": 4 << 30,
                   "compressed_bytes_per_layer": hbs[0].nbytes,
                   "decoded_bytes_per_layer": int(decoded), "bit_exact": ok},
        "decode_only_gbs": round(args.layers * decoded / decode / 1e9, 1),
        "h2d_pinned_gbs": round(h2d_gbs, 1),
        "h2d_bound_layers_per_s": round(h2d_gbs * 1e9 / hbs[0].nbytes, 2),
        "roofline": None,
        "cpu_baseline": None,
    }
    del ring, hbs, slot
    return rec


def _bench_gemv(args) -> int:
    rec = _gemv(args)
    if rec is None:
        return 1
    print(json.dumps(rec), flush=True)
    return 0


def _gemv(args, W=None, layer=None) -> dict | None:
    """Fused decode->GEMV: y[b] = W x[b] for the 5120x17408 weight, W decoded
    in the kernel and never written (batch 1..4; 5..16 rows of x take the
    fused GEMM on the matrix cores). One step = zero y + one launch; the
    roofline figures come from the launches alone, timed in a second loop.
    With --index the layer's segment index is built first (the
    compressed-resident tier; the GEMM ignores it); without it the product
    decodes speculatively, as decompress_matvec_gpu does. Returns the JSON
    record, or None when y is outside the tolerance."""
    from afterimage_amd import workloads
    from afterimage_amd.runtime.device import GEMV_MAX_BATCH, DeviceTensor, decode_gemm
    from afterimage_amd.runtime.device import decode_gemv as _gemv_call

    dev = torch.device("cuda", 0)
    torch.cuda.set_device(dev)
    if W is None:
        W, layer = workloads.single_layer(seed=2, chunk_size=args.chunk_size)
    rows, cols = W.shape
    b = args.batch
    g = np.random.default_rng(23)
    x = torch.from_numpy(g.standard_normal((b, cols), dtype=np.float32)).to(torch.bfloat16).to(dev)
    t = DeviceTensor.from_encoded(layer.encoded, layer.sign_mantissa, dev)
    if getattr(args, "index", False):
        t.build_index()  # the resident layer's segment index, built once
    y = torch.zeros((b, rows), dtype=torch.float32, device=dev)
    decode_gemv = _gemv_call if b <= GEMV_MAX_BATCH else decode_gemm
    kind = "GEMV" if b <= GEMV_MAX_BATCH else "GEMM"

    def step():
        y.zero_()
        decode_gemv(t, x, rows, cols, y)

    for _ in range(args.warmup):
        step()
    torch.cuda.synchronize(dev)
    ref = torch.matmul(x.float(), W.to(dev).float().t().contiguous())
    yb = y.to(torch.bfloat16).float()
    ok = bool(((yb - ref).abs() <= 1e-3 + 1e-2 * ref.abs()).all())
    if not ok:
        print("fused %s differs from decode-then-matmul beyond rel 1e-2 / abs 1e-3" % kind,
              file=sys.stderr)
        return None
    stream = torch.cuda.current_stream(dev)
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
    # The GEMV launches alone, for the kernel's own duration: y keeps
    # accumulating (its value was checked above).
    ev2 = torch.cuda.Event(enable_timing=True)
    ev3 = torch.cuda.Event(enable_timing=True)
    ev2.record(stream)
    for _ in range(args.steps):
        decode_gemv(t, x, rows, cols, y)
    ev3.record(stream)
    torch.cuda.synchronize(dev)
    step_s = ev2.elapsed_time(ev3) / 1e3 / args.steps
    # The decode kernel's own symbol rate on the same tensor (exponent bytes
    # out, its smallest output): what the fused GEMV's decode loop is bound by.
    from afterimage_amd.runtime.device import decode_u8

    ex = torch.empty(layer.encoded.n_symbols, dtype=torch.uint8, device=dev)
    for _ in range(args.warmup):
        decode_u8([t], outs=[ex])
    ev4 = torch.cuda.Event(enable_timing=True)
    ev5 = torch.cuda.Event(enable_timing=True)
    ev4.record(stream)
    for _ in range(args.steps):
        decode_u8([t], outs=[ex])
    ev5.record(stream)
    torch.cuda.synchronize(dev)
    u8_s = ev4.elapsed_time(ev5) / 1e3 / args.steps
    enc = layer.encoded
    n = enc.n_symbols
    chunk_bytes = int(enc.chunk_nbytes.astype(np.int64).sum())
    # bitstreams + offsets/lengths + sign/mantissa + table + x read + y
    # read/write (+ the segment index read)
    algo_bytes = (chunk_bytes + 8 * enc.n_chunks + n + (5 * 4096 + 256) + 2 * b * cols
                  + 8 * b * rows + t.index_bytes_read)
    rec = {
        "metric": "fused decode->%s weight GB/s (bf16 bytes consumed per second)" % kind,
        "value": round(2 * n * args.steps / wall / 1e9, 2),
        "unit": "GB/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(wall * 1e3 / args.steps, 5),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "bf16",
        "data": "synthetic",
        "config": {"workload": "fused decode->%s, 5120x17408 bf16 weight (seed 2, 0.1%% "
                               "outliers, %d-symbol chunks) x bf16 activation [%d, 17408] N(0,1) "
                               "(seed 23), fp32 accumulate -> bf16" % (kind, enc.chunk_size, b),
                   "batch": b, "within_tolerance": ok, "tolerance": "rel 1e-2, abs 1e-3",
                   "flops_per_step": 2 * n * b, "chunk_size": enc.chunk_size,
                   "segment_index": t.index is not None},
        # The GEMV moves 2.5x fewer bytes than the decode but runs its decode
        # loop: its bound is the decode's symbol rate, measured here on the
        # same tensor with exponent-byte output (the decode's smallest output).
        "roofline": {"bound": "decode", "achieved": round(n / step_s / 1e9, 2),
                     "peak": round(n / u8_s / 1e9, 2), "unit": "Gsymbols/s",
                     "frac": round(u8_s / step_s, 4), "traffic": None,
                     "kernel_us": round(step_s * 1e6, 2),
                     "decode_u8_us": round(u8_s * 1e6, 2),
                     "hbm_gbs": round(algo_bytes / step_s / 1e9, 1),
                     "hbm_frac": round(algo_bytes / step_s / 1e9 / HBM_PEAK_GBS, 4),
                     "algorithmic_bytes_per_launch": algo_bytes},
        "cpu_baseline": None,
    }
    del t, ex, y
    return rec


def _bench_head(args) -> int:
    rec = _head(args)
    if rec is None:
        return 1
    print(json.dumps(rec), flush=True)
    return 0


def _head(args) -> dict | None:
    """The output projection of a 14B-class model (lm_head 151936x5120 bf16,
    resident compressed in HBM at the reference store's default 1024-symbol
    chunks) applied to x [1, tokens, 5120]. One step = one blocked forward
    as the reference's chunked head computes it: 8192-row blocks, each
    decoded into one staging buffer and multiplied by the GEMM library,
    outputs concatenated (no index unless --index). Also timed: the fused
    product that decodes no weight to memory (GEMV up to 4 tokens, GEMM on
    the matrix cores for 5..16), both as its kernel alone and as the API
    call decompress_linear_gpu(fused=True) on the resident layer; the whole
    head decoded at once then one F.linear; and F.linear on the decoded
    weight alone. Returns the record, or None when a check fails."""
    import torch.nn.functional as F

    from afterimage_amd import workloads
    from afterimage_amd.runtime.compressed_store import (CompressedLayer, compress_layer,
                                                         decompress_linear_gpu)
    from afterimage_amd.runtime.device import (GEMM_MAX_ROWS, GEMV_MAX_BATCH, DeviceTensor,
                                               decode_bf16, decode_gemm, decode_gemv,
                                               decode_linear, row_blocks)
    from afterimage_amd.runtime.huffman_chunked import ChunkedEncoded

    dev = torch.device("cuda", 0)
    torch.cuda.set_device(dev)
    rows, cols, slice_rows, tokens = 151936, 5120, args.slice_rows, args.batch
    t0 = time.perf_counter()
    W = workloads.bf16_normal((rows, cols), 5, 0.02, outlier_frac=1e-3)
    layer = compress_layer(W, chunk_size=args.chunk_size)
    _log("head built in %.1fs: %d chunks, packed %.1f MB"
         % (time.perf_counter() - t0, layer.encoded.n_chunks, layer.encoded.packed.nbytes / 1e6))
    enc = layer.encoded
    n = enc.n_symbols
    t = DeviceTensor.from_encoded(enc, layer.sign_mantissa, dev)
    if args.index:
        t.build_index()
    # The same layer with its arrays resident on the GPU, for the API call.
    resident = CompressedLayer(
        sign_mantissa=t.sign_mantissa, shape=layer.shape,
        encoded=ChunkedEncoded(packed=t.packed, chunk_offsets=t.chunk_offsets,
                               chunk_nbytes=t.chunk_nbytes, sym_lut=enc.sym_lut,
                               len_lut=enc.len_lut, max_bits=enc.max_bits,
                               chunk_size=enc.chunk_size, n_symbols=n, shape=enc.shape))
    g = np.random.default_rng(29)
    x = torch.from_numpy(g.standard_normal((1, tokens, cols), dtype=np.float32)) \
        .to(torch.bfloat16).to(dev)
    blocks = row_blocks(rows, cols, enc.chunk_size, enc.n_chunks, slice_rows)
    need = max(min(n, c1 * enc.chunk_size) - c0 * enc.chunk_size for _, _, c0, c1 in blocks)
    staging = torch.empty(need, dtype=torch.bfloat16, device=dev)
    whole = torch.empty(n, dtype=torch.bfloat16, device=dev)
    y_fused = torch.zeros((tokens, rows), dtype=torch.float32, device=dev)
    fused_ok = tokens <= GEMM_MAX_ROWS
    fused_fn = decode_gemv if tokens <= GEMV_MAX_BATCH else decode_gemm

    def blocked():
        return decode_linear(t, x, rows, cols, slice_rows, staging=staging)

    def unblocked():
        decode_bf16([t], [whole])
        return F.linear(x, whole.view(rows, cols))

    def fused():
        y_fused.zero_()
        fused_fn(t, x.reshape(tokens, cols), rows, cols, y_fused)

    def api():
        return decompress_linear_gpu(resident, x, fused=True)

    # Parity before timing: the decoded head is the original bit for bit,
    # and the blocked forward is the reference's blocked F.linear calls on
    # those weights (block views at the same offsets, so the same GEMMs).
    y_blocked = blocked()
    unblocked()
    torch.cuda.synchronize(dev)
    Wd = W.to(dev)
    bit_exact = torch.equal(whole.view(rows, cols).view(torch.int16), Wd.view(torch.int16))
    ref = []
    flat = Wd.reshape(-1)
    for r0, r1, c0, c1 in blocks:
        base = c0 * enc.chunk_size
        buf = flat[base: min(n, c1 * enc.chunk_size)].clone()
        ref.append(F.linear(x, buf[r0 * cols - base: r1 * cols - base].view(r1 - r0, cols)))
    same_as_reference = torch.equal(y_blocked, torch.cat(ref, dim=-1))
    del ref, buf, flat
    if not bit_exact:
        print("decoded head differs from the original weights", file=sys.stderr)
        return None
    fused_within = None
    if fused_ok:
        fused()
        yf = torch.matmul(x.reshape(tokens, cols).float(), Wd.float().t().contiguous())
        yb = y_fused.to(torch.bfloat16).float()
        ya = api().reshape(tokens, rows).float()
        fused_within = bool(((yb - yf).abs() <= 1e-3 + 1e-2 * yf.abs()).all()) and \
            bool(((ya - yf).abs() <= 1e-3 + 1e-2 * yf.abs()).all())
        del yf, yb, ya
    del Wd
    stream = torch.cuda.current_stream(dev)

    def timed(fn):
        for _ in range(args.warmup):
            fn()
        e0 = torch.cuda.Event(enable_timing=True)
        e1 = torch.cuda.Event(enable_timing=True)
        torch.cuda.synchronize(dev)
        e0.record(stream)
        for _ in range(args.steps):
            fn()
        e1.record(stream)
        torch.cuda.synchronize(dev)
        return e0.elapsed_time(e1) / 1e3 / args.steps

    wall0 = time.perf_counter()
    blocked_s = timed(blocked)
    wall = (time.perf_counter() - wall0) / (args.steps + args.warmup)
    unblocked_s = timed(unblocked)
    decode_s = timed(lambda: decode_bf16([t], [whole]))
    gemm_s = timed(lambda: F.linear(x, whole.view(rows, cols)))
    fused_s = timed(fused) if fused_ok else None
    api_s = timed(api) if fused_ok else None
    return {
        "metric": "blocked lm_head forward: decompressed BF16 GB/s (decode + GEMM per block)",
        "value": round(2 * n / blocked_s / 1e9, 2),
        "unit": "GB/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(blocked_s * 1e3, 4),
        "wall_ms_per_step": round(wall * 1e3, 4),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "bf16",
        "data": "synthetic",
        "config": {"workload": "lm_head 151936x5120 bf16 (seed 5, 0.1%% outliers, %d-symbol "
                               "chunks) resident compressed, x [1, %d, 5120] bf16 N(0,1) "
                               "(seed 29), %d-row blocks, %s"
                               % (enc.chunk_size, tokens, slice_rows,
                                  WITH_INDEX if args.index else NO_INDEX),
                   "tokens": tokens, "slice_rows": slice_rows, "chunk_size": enc.chunk_size,
                   "blocks": len(blocks), "staging_bytes": 2 * need,
                   "segment_index": t.index is not None,
                   "weights_bit_exact": bit_exact,
                   "blocked_equals_reference_forward": same_as_reference,
                   "fused_within_tolerance": fused_within,
                   "fused_kind": ("GEMV" if tokens <= GEMV_MAX_BATCH else "GEMM (MFMA)")
                   if fused_ok else None,
                   "tolerance": "fused: rel 1e-2, abs 1e-3 against the fp32 product"},
        "paths_us": {
            "blocked_decode_and_gemm": round(blocked_s * 1e6, 1),
            "whole_decode_then_gemm": round(unblocked_s * 1e6, 1),
            "whole_decode_alone": round(decode_s * 1e6, 1),
            "gemm_alone_on_decoded_weight": round(gemm_s * 1e6, 1),
            "fused_kernel": None if fused_s is None else round(fused_s * 1e6, 1),
            "fused_api_decompress_linear_gpu": None if api_s is None else round(api_s * 1e6, 1),
        },
        "roofline": None,
        "cpu_baseline": None,
    }


def _bench_resync(args) -> int:
    """Exponent-byte decode of 16,777,216 symbols whose speculative segment
    starts are all wrong (eight equiprobable symbols, 3-bit codes: every
    168-bit segment starts inside a codeword and a guess never finds the
    boundary), with and without the segment index, beside the exponents of a
    bf16 weight of the same size. Both decodes are checked equal."""
    from afterimage_amd import workloads
    from afterimage_amd.runtime.device import DeviceTensor, decode_u8
    from afterimage_amd.runtime.huffman_chunked import encode_chunked

    dev = torch.device("cuda", 0)
    torch.cuda.set_device(dev)
    n = 1 << 24
    rng = np.random.default_rng(8)
    W = workloads.bf16_normal((1024, n // 1024), 2, 0.02, outlier_frac=1e-3)
    exps = ((W.view(torch.int16).to(torch.int32) & 0xFFFF) >> 7 & 0xFF).reshape(-1)
    cases = [("all segment guesses wrong (3-bit codes)",
              encode_chunked(torch.from_numpy(rng.integers(0, 8, n)), chunk_size=65536)),
             ("bf16 exponents of a 1024x16384 weight", encode_chunked(exps, chunk_size=65536))]
    stream = torch.cuda.current_stream(dev)

    def timed(t, out):
        for _ in range(args.warmup):
            decode_u8([t], outs=[out])
        e0 = torch.cuda.Event(enable_timing=True)
        e1 = torch.cuda.Event(enable_timing=True)
        torch.cuda.synchronize(dev)
        e0.record(stream)
        for _ in range(args.steps):
            decode_u8([t], outs=[out])
        e1.record(stream)
        torch.cuda.synchronize(dev)
        return e0.elapsed_time(e1) * 1e3 / args.steps

    res = []
    for name, enc in cases:
        t = DeviceTensor.from_encoded(enc, None, dev)
        a = torch.empty(n, dtype=torch.uint8, device=dev)
        b = torch.empty(n, dtype=torch.uint8, device=dev)
        plain_us = timed(t, a)
        t.build_index()
        index_us = timed(t, b)
        same = torch.equal(a, b)
        if not same:
            print("%s: decodes with and without the index differ" % name, file=sys.stderr)
            return 1
        res.append({"stream": name, "symbols": n,
                    "bits_per_symbol": round(8 * int(np.asarray(enc.chunk_nbytes).sum()) / n, 3),
                    "no_index_us": round(plain_us, 1), "with_index_us": round(index_us, 1),
                    "index_usable": t.index is not None, "outputs_equal": same})
    rec = {
        "metric": "exponent-byte decode time of streams that never resynchronise",
        "value": res[0]["no_index_us"], "unit": "us", "n_gpus": 1, "steps": args.steps,
        "warmup": args.warmup, "higher_is_better": False, "vs_baseline": None, "dtype": "u8",
        "data": "synthetic",
        "config": {"workload": "16,777,216 symbols in 65536-symbol chunks, aimg_decode_u8"},
        "cases": res, "roofline": None, "cpu_baseline": None,
    }
    print(json.dumps(rec), flush=True)
    return 0


def _bench_api(args) -> int:
    """The reference API path: decompress_layer_gpu on the 5120x17408 layer
    from host arrays, as the reference engine calls it (pageable H2D of the
    compressed arrays, decode table from the content-keyed cache, decode).
    One step = one call; the value includes the PCIe copies."""
    from afterimage_amd import workloads
    from afterimage_amd.runtime.compressed_store import decompress_layer_gpu

    dev = torch.device("cuda", 0)
    torch.cuda.set_device(dev)
    W, layer = workloads.single_layer(seed=2, chunk_size=args.chunk_size)
    enc = layer.encoded

    def step():
        return decompress_layer_gpu(layer, device="cuda:0", reuse_decode_tables=True)

    for _ in range(args.warmup):
        out = step()
    torch.cuda.synchronize(dev)
    ok = torch.equal(out.view(torch.int16).cpu(), W.view(torch.int16))
    if not ok:
        print("API decode differs from the original weights", file=sys.stderr)
        return 1
    del out
    torch.cuda.synchronize(dev)
    t_start = time.perf_counter()
    for _ in range(args.steps):
        step()
    torch.cuda.synchronize(dev)
    wall = (time.perf_counter() - t_start) / args.steps
    h2d = int(enc.packed.nbytes + layer.sign_mantissa.numel() + 8 * enc.n_chunks)
    n = enc.n_symbols
    rec = {
        "metric": "decompress_layer_gpu from host arrays: decompressed BF16 GB/s (H2D included)",
        "value": round(2 * n / wall / 1e9, 2),
        "unit": "GB/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(wall * 1e3, 4),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "bf16",
        "data": "synthetic",
        "config": {"workload": "decompress_layer_gpu(layer, 'cuda:0', reuse_decode_tables=True) "
                               "on the 5120x17408 weight (seed 2, 0.1%% outliers, %d-symbol "
                               "chunks) held in host numpy arrays; default 2^25-element slices"
                               % enc.chunk_size,
                   "h2d_bytes_per_call": h2d, "bit_exact": ok, "chunk_size": enc.chunk_size},
        "h2d_inclusive_gbs_compressed": round(h2d / wall / 1e9, 2),
        "roofline": None,
        "cpu_baseline": None,
    }
    print(json.dumps(rec), flush=True)
    return 0


def main() -> int:
    ap = argparse.ArgumentParser(description=__doc__.split("\n\n")[0])
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=200)
    ap.add_argument("--warmup", type=int, default=400)
    ap.add_argument("--workload",
                    choices=["suite", "layer", "block", "gemv", "ring", "api", "head", "resync"],
                    default="suite",
                    help="suite (default): the headline layer and every other configuration "
                         "as extra keys of one line; layer: one 5120x17408 weight (the "
                         "headline alone); block: a whole "
                         "14B-class decoder block in one launch; gemv: fused decode->GEMV "
                         "of the 5120x17408 weight with a [batch, 17408] activation; ring: 40 "
                         "streamed blocks from pinned host memory through a 2-slot ring; api: "
                         "decompress_layer_gpu from host arrays, H2D included; head: a 151936x5120 "
                         "lm_head applied to [1, batch, 5120] in row blocks (the reference's "
                         "chunked head); resync: streams whose segment guesses are all wrong, "
                         "with and without the index")
    ap.add_argument("--layers", type=int, default=40, help="ring: layers streamed per step")
    ap.add_argument("--batch", type=int, default=1,
                    help="gemv: rows of x (1..4: fused GEMV; 5..16: fused GEMM); head: tokens of x")
    ap.add_argument("--slice-rows", type=int, default=8192, help="head: rows per block")
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--index", action="store_true",
                    help="layer/block/gemv: build each tensor's segment index before timing "
                         "(the compressed-resident tier; the default decodes from the "
                         "store-format arrays alone, as the drop-in API does)")
    ap.add_argument("--no-cold", action="store_true",
                    help="suite/layer: skip the cold-input launches (kernel traces of the "
                         "timed loop)")
    ap.add_argument("--cpu-threads", type=int, default=0,
                    help="CPU-baseline threads (0: OpenMP's count, i.e. every CPU given)")
    ap.add_argument("--chunk-size", type=int, default=None,
                    help="layer / gemv / api: symbols per chunk of the 5120x17408 weight "
                         "(default 65536); head: of the lm_head (default 1024)")
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
    if args.chunk_size is None:
        args.chunk_size = 1024 if args.workload == "head" else 65536

    if args.copy_mib:
        return _copy_calibration(args.copy_mib, args.steps, args.warmup)
    if args.workload == "gemv":
        return _bench_gemv(args)
    if args.workload == "ring":
        return _bench_ring(args)
    if args.workload == "api":
        return _bench_api(args)
    if args.workload == "head":
        return _bench_head(args)
    if args.workload == "resync":
        return _bench_resync(args)

    if args.workload == "suite":
        return _suite(args)
    return _single(args)


LAYER_WORKLOAD = ("bf16 5120x17408 weight decode, N(0,0.02) + 0.1%% N(0,0.5) outliers (seed 2), "
                  "per-tensor Huffman exponent codebook, %d-symbol chunks (%d), inputs resident "
                  "in HBM, one launch per step, %s")
BLOCK_WORKLOAD = ("bf16 14B-class decoder block (q,o 5120x5120; k,v 1024x5120; gate,up 17408x5120; "
                  "down 5120x17408; 2 RMSNorm 5120), N(0,0.02) weights, norms N(1,0.05) (seed %d), "
                  "one exponent codebook per role, 65536-symbol chunks (%d), inputs resident in "
                  "HBM, all 9 tensors in one launch per step, %s")
NO_INDEX = "decoded from the store-format arrays alone (no derived data), as decompress_layer_gpu does"
WITH_INDEX = ("each tensor's segment index (derived data, built once when the compressed tensor "
              "becomes resident in HBM; a tier the reference does not have) prebuilt")


def _decode(items, steps: int, warmup: int, index: bool = False, cold: bool = False) -> dict:
    """aimg_decode_bf16 over the items' tensors, one launch per step, inputs
    resident in HBM: launches timed with HIP events on the launch stream,
    the loop by the host clock; bit-exactness checked against the original
    weights before timing. index: build each tensor's segment index first
    (its build time is reported). cold: also three copies decoded in turn,
    so that the inputs come from HBM rather than the last-level cache."""
    from afterimage_amd import _native
    from afterimage_amd.runtime.device import DeviceTensor, _descriptor

    dev = torch.device("cuda", 0)
    layers = [layer for _, _, layer in items]
    dts = [DeviceTensor.from_encoded(l.encoded, l.sign_mantissa, dev) for l in layers]
    outs = [torch.empty(l.encoded.n_symbols, dtype=torch.bfloat16, device=dev) for l in layers]
    lib = _native.lib()
    stream = torch.cuda.current_stream(dev)
    handle = ctypes.c_void_p(stream.cuda_stream)
    decode = lib.aimg_decode_bf16
    index_info = None
    if index:
        e0 = torch.cuda.Event(enable_timing=True)
        e1 = torch.cuda.Event(enable_timing=True)
        torch.cuda.synchronize(dev)
        e0.record(stream)
        for dt in dts:
            dt.build_index()
        e1.record(stream)
        torch.cuda.synchronize(dev)
        ix_bytes = sum(dt.index.numel() for dt in dts if dt.index is not None)
        comp = sum(dt.packed.numel() + dt.sign_mantissa.numel() for dt in dts)
        index_info = {"build_us": round(e0.elapsed_time(e1) * 1e3, 1), "bytes": ix_bytes,
                      "bytes_read_per_launch": sum(dt.index_bytes_read for dt in dts),
                      "frac_of_compressed": round(ix_bytes / comp, 4)}

    def descriptors(ts, os_):
        d = (_native.AimgTensor * len(ts))()
        for j, (dt, o) in enumerate(zip(ts, os_)):
            d[j] = _descriptor(dt, o, o.numel())
        return d

    def exact(os_) -> bool:
        torch.cuda.synchronize(dev)
        return all(torch.equal(o.view(torch.int16).cpu(), W.reshape(-1).view(torch.int16))
                   for (_, W, _), o in zip(items, os_))

    def launches(d, k: int) -> float:
        e0 = torch.cuda.Event(enable_timing=True)
        e1 = torch.cuda.Event(enable_timing=True)
        torch.cuda.synchronize(dev)
        e0.record(stream)
        for j in range(k):
            rc = decode(d[j % len(d)], len(dts), handle)
            if rc:
                _native.check(rc)
        e1.record(stream)
        torch.cuda.synchronize(dev)
        return e0.elapsed_time(e1) / 1e3 / k

    desc = descriptors(dts, outs)
    launches([desc], 1)
    ok = exact(outs)
    if not ok:
        raise RuntimeError("decoded output differs from the original weights")
    # The warmup launches come after the check, right before the timed ones:
    # the GPU idles while the host compares, and its clocks take some tens of
    # milliseconds of work to come back up (the first launches after an idle
    # spell ran 5-10% slower).
    if warmup > 0:
        launches([desc], warmup)
    t_start = time.perf_counter()
    kernel_s = launches([desc], steps)
    wall = time.perf_counter() - t_start
    n = sum(l.encoded.n_symbols for l in layers)
    n_chunks = sum(l.encoded.n_chunks for l in layers)
    chunk_bytes = sum(int(l.encoded.chunk_nbytes.astype(np.int64).sum()) for l in layers)
    n_tables = len({dt.tables.key for dt in dts})
    # bitstreams + chunk offsets and lengths + sign/mantissa + window tables
    # + bf16 write (+ the segment index read, when there is one)
    algo = chunk_bytes + 8 * n_chunks + n + (5 * 4096 + 256) * n_tables + 2 * n
    if index_info:
        algo += index_info["bytes_read_per_launch"]
    res = {"kernel_us": round(kernel_s * 1e6, 2), "wall_s": wall, "steps": steps,
           "decompressed_gbs": round(2 * n / kernel_s / 1e9, 1),
           "achieved_gbs": round(algo / kernel_s / 1e9, 1),
           "frac": round(algo / kernel_s / 1e9 / HBM_PEAK_GBS, 4),
           "algorithmic_bytes_per_launch": algo, "n_weights": n, "n_chunks": n_chunks,
           "n_tensors": len(items), "decode_tables": n_tables,
           "packed_exponent_bytes": chunk_bytes,
           "bits_per_exponent": round(8 * chunk_bytes / n, 4), "bit_exact": ok,
           "segment_index": index_info}
    if cold:
        import dataclasses

        copies = [(dts, outs)]
        for _ in range(2):
            c_dts = [dataclasses.replace(
                dt, packed=dt.packed.clone(), chunk_offsets=dt.chunk_offsets.clone(),
                chunk_nbytes=dt.chunk_nbytes.clone(), sign_mantissa=dt.sign_mantissa.clone(),
                index=None if dt.index is None else dt.index.clone()) for dt in dts]
            copies.append((c_dts, [torch.empty_like(o) for o in outs]))
        c_desc = [descriptors(c_dts, c_outs) for c_dts, c_outs in copies]
        k_cold = 3 * max(1, min(steps // 3, 40))
        launches(c_desc, 6)
        cold_s = launches(c_desc, k_cold)
        cold_ok = all(exact(c_outs) for _, c_outs in copies)
        res["cold_inputs"] = {
            "kernel_us": round(cold_s * 1e6, 2), "launches": k_cold, "bit_exact": cold_ok,
            "decompressed_gbs": round(2 * n / cold_s / 1e9, 1),
            "frac": round(algo / cold_s / 1e9 / HBM_PEAK_GBS, 4),
            "inputs_bytes": 3 * sum(dt.packed.numel() + dt.sign_mantissa.numel() for dt in dts),
            "what": "three copies decoded in turn (inputs read from HBM, not from the "
                    "last-level cache)"}
        del copies, c_desc
    del dts, outs
    torch.cuda.empty_cache()
    return res


def _record(args, res: dict, workload: str, config_key: str, layers, what: str) -> dict:
    """The driver's JSON line for a decode measurement (value: decompressed
    GB/s over the host-clocked loop)."""
    n = res["n_weights"]
    rec = {
        "metric": METRIC,
        "value": round(2 * n * res["steps"] / res["wall_s"] / 1e9, 2),
        "unit": "GB/s",
        "n_gpus": 1,
        "steps": res["steps"],
        "warmup": args.warmup,
        "ms_per_step": round(res["wall_s"] * 1e3 / res["steps"], 5),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "bf16",
        "data": "synthetic",
        "config": {"workload": workload, "config_key": config_key,
                   **{k: res[k] for k in ("n_tensors", "n_weights", "n_chunks", "decode_tables",
                                          "packed_exponent_bytes", "bits_per_exponent",
                                          "bit_exact", "segment_index")}},
        "roofline": {
            "bound": "hbm",
            "achieved": res["achieved_gbs"],
            "peak": HBM_PEAK_GBS,
            "unit": "GB/s",
            "frac": res["frac"],
            "traffic": _traffic(config_key),
            "algorithmic_bytes_per_launch": res["algorithmic_bytes_per_launch"],
            "kernel_us": res["kernel_us"],
        },
        "cold_inputs": res.get("cold_inputs"),
        "cpu_baseline": None,
    }
    if not args.no_cpu_baseline:
        _log("timing the CPU baseline (~15 s)")
        rec["cpu_baseline"] = _cpu_baseline(layers, args.cpu_threads, what)
    return rec


def _single(args) -> int:
    """--workload layer | block: one decode measurement, without the segment
    index unless --index."""
    from afterimage_amd import workloads

    torch.cuda.set_device(0)
    t0 = time.perf_counter()
    tier = WITH_INDEX if args.index else NO_INDEX
    if args.workload == "layer":
        W, layer = workloads.single_layer(seed=2, chunk_size=args.chunk_size)
        items = [("layer", W, layer)]
        key = "5120x17408/seed2/chunk%d/outliers1e-3" % args.chunk_size
        desc = LAYER_WORKLOAD % (args.chunk_size, layer.encoded.n_chunks, tier)
    else:
        items = workloads.block_14b(seed=3)
        key = "block14b/seed3/chunk65536/per-role"
        desc = BLOCK_WORKLOAD % (3, sum(l.encoded.n_chunks for _, _, l in items), tier)
    if args.index:
        key += "/index"
    _log("workload built in %.1fs" % (time.perf_counter() - t0))
    res = _decode(items, args.steps, args.warmup, index=args.index,
                  cold=args.workload == "layer" and not args.no_cold)
    rec = _record(args, res, desc, key, [l for _, _, l in items], "the whole " + args.workload)
    print(json.dumps(rec), flush=True)
    return 0


def _suite(args) -> int:
    """The default run: the headline (the 5120x17408 layer in
    65536-symbol chunks decoded without an index, as decompress_layer_gpu and
    the streamed ring decode it) as value and roofline, and the other
    configurations as extra keys, each timed in this same run."""
    import types

    from afterimage_amd import workloads
    from afterimage_amd.runtime.compressed_store import compress_layer

    torch.cuda.set_device(0)
    t0 = time.perf_counter()
    W, layer = workloads.single_layer(seed=2, chunk_size=65536)
    items = [("layer", W, layer)]
    _log("layer built in %.1fs" % (time.perf_counter() - t0))
    head = _decode(items, args.steps, args.warmup, cold=not args.no_cold)
    key = "5120x17408/seed2/chunk65536/outliers1e-3"
    rec = _record(args, head, LAYER_WORKLOAD % (65536, layer.encoded.n_chunks, NO_INDEX), key,
                  [layer], "the whole layer")
    _log("headline: %.2f us per launch, %.4f of HBM roofline" % (head["kernel_us"], head["frac"]))
    short = min(args.steps, 100)
    extra = {}

    def brief(res: dict) -> dict:
        out = {k: res[k] for k in ("kernel_us", "decompressed_gbs", "achieved_gbs", "frac",
                                   "algorithmic_bytes_per_launch", "n_weights", "n_chunks",
                                   "bit_exact")}
        if res.get("cold_inputs"):
            out["cold_inputs"] = {k: res["cold_inputs"][k]
                                  for k in ("kernel_us", "decompressed_gbs", "frac", "bit_exact")}
        if res.get("segment_index"):
            out["segment_index"] = res["segment_index"]
        return out

    # The same layer at the reference store's default 1024-symbol chunks
    # (afterimage compress, cli.py:1117 / config.py:361), no index.
    l1024 = compress_layer(W, chunk_size=1024)
    extra["chunk1024"] = dict(brief(_decode([("layer", W, l1024)], short, args.warmup, cold=True)),
                              what="the same layer in 1024-symbol chunks, no index")
    del l1024
    # The compressed-resident tier: the layer's segment index built once,
    # then decodes that use it (no reference counterpart).
    ix = _decode(items, short, args.warmup, index=True)
    extra["index_tier"] = dict(
        brief(ix), what="the layer with its segment index prebuilt: derived data built once "
                        "per resident compressed tensor, for a tier that keeps tensors "
                        "compressed in HBM (the reference has none); build_us + kernel_us is "
                        "the one-shot cost")
    # A small layer: 1024x3072 at 4096-symbol chunks.
    Ws, small = workloads.small_layer(seed=1)
    extra["small_layer_1024x3072"] = dict(
        brief(_decode([("small", Ws, small)], short, args.warmup)),
        what="bf16 1024x3072, 4096-symbol chunks, one launch, no index (launch-bound)")
    # The fused decode->GEMV at batch 1 and 4, speculative decode
    # (no index) as decompress_matvec_gpu runs it, at both chunk sizes.
    gargs = types.SimpleNamespace(steps=short, warmup=args.warmup, index=False, chunk_size=65536)
    for b in (1, 4):
        gargs.batch = b
        g = _gemv(gargs, W, layer)
        extra["gemv_b%d" % b] = None if g is None else dict(
            g["roofline"], within_tolerance=g["config"]["within_tolerance"],
            what="fused decode->GEMV, 5120x17408 x [%d, 17408], 65536-symbol chunks, no index; "
                 "frac: the exponent-byte decode's time over the GEMV's" % b)
    # The fused decode->GEMM (matrix cores) at speculative-verify widths.
    for b in (8, 16):
        gargs.batch = b
        g = _gemv(gargs, W, layer)
        extra["gemm_t%d" % b] = None if g is None else dict(
            g["roofline"], within_tolerance=g["config"]["within_tolerance"],
            what="fused decode->GEMM, 5120x17408 x [%d, 17408], 65536-symbol chunks, no index; "
                 "frac: the exponent-byte decode's time over the GEMM's" % b)
    l1024 = compress_layer(W, chunk_size=1024)
    gargs.chunk_size = 1024
    for b in (1, 4, 8):
        gargs.batch = b
        g = _gemv(gargs, W, l1024)
        extra[("gemv_b%d_chunk1024" if b <= 4 else "gemm_t%d_chunk1024") % b] = \
            None if g is None else dict(g["roofline"],
                                        within_tolerance=g["config"]["within_tolerance"],
                                        what="the same at 1024-symbol chunks")
    del l1024
    # The chunked lm_head at 8 tokens (a speculative-verify width), no index:
    # the reference's blocked forward against the fused GEMM.
    hargs = types.SimpleNamespace(slice_rows=8192, batch=8, chunk_size=1024, index=False,
                                  steps=5, warmup=2)
    h = _head(hargs)
    extra["head_t8"] = None if h is None else dict(
        paths_us=h["paths_us"], weights_bit_exact=h["config"]["weights_bit_exact"],
        blocked_equals_reference_forward=h["config"]["blocked_equals_reference_forward"],
        fused_within_tolerance=h["config"]["fused_within_tolerance"],
        what="lm_head 151936x5120 bf16, 1024-symbol chunks, resident compressed, no index, "
             "x [1, 8, 5120]: blocked decode + F.linear per 8192 rows (the reference's chunked "
             "head) against the fused decode->GEMM (kernel alone, and through "
             "decompress_linear_gpu(fused=True))")
    torch.cuda.empty_cache()
    # A 14B-class block in one launch, no index.
    t0 = time.perf_counter()
    blk3 = workloads.block_14b(seed=3)
    _log("block built in %.1fs" % (time.perf_counter() - t0))
    extra["block_14b"] = dict(
        brief(_decode(blk3, short, args.warmup)),
        what="the 14B-class block (9 tensors, 5 codebooks, 65536-symbol chunks) in one launch, "
             "no index")
    # 40 streamed blocks through a 2-slot ring under 4 GiB.
    blk4 = workloads.block_14b(seed=4)
    rargs = types.SimpleNamespace(layers=40, steps=3, warmup=2)
    r = _ring(rargs, [blk3, blk4])
    extra["ring_40_blocks"] = None if r is None else {
        "layers_per_s": r["value"], "ms_per_40_layers": r["ms_per_step"],
        "decode_only_gbs": r["decode_only_gbs"], "h2d_pinned_gbs": r["h2d_pinned_gbs"],
        "h2d_bound_layers_per_s": r["h2d_bound_layers_per_s"], "bit_exact": r["config"]["bit_exact"],
        "what": r["config"]["workload"]}
    rec["extra"] = extra
    print(json.dumps(rec), flush=True)
    return 0


if __name__ == "__main__":
    sys.exit(main())
