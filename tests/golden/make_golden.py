"""Write tests/golden/codec_vectors.npz from the reference codec.

Run in the build container, where the reference checkout is mounted:

    python tests/golden/make_golden.py [/root/reference]

It imports the reference's pure-Python codec modules
(afterimage/runtime/huffman.py, huffman_chunked.py, compressed_store.py) and
records, for seeded inputs, what they produce: code lengths, LUTs, packed
chunk bytes, offsets, and decoded outputs. The file holds data only (inputs
and expected outputs); nothing from the reference's source is stored. The
tests compare this package's encoder and the oracle's decoders against it.

The reference's encoder needs numba for its fast packer; without numba it
packs each chunk with ``pack_bits``, which it states is byte-identical.
"""
from __future__ import annotations

import sys
from pathlib import Path

import numpy as np
import torch

HERE = Path(__file__).resolve().parent
OUT = HERE / "codec_vectors.npz"


def _bf16_exponents(rng: np.random.Generator, n: int, scale: float, outlier_p: float = 0.0):
    w = rng.standard_normal(n).astype(np.float32) * scale
    if outlier_p:
        m = rng.random(n) < outlier_p
        w[m] = rng.standard_normal(int(m.sum())).astype(np.float32) * 0.5
    bits = torch.from_numpy(w).to(torch.bfloat16).view(torch.int16).numpy().view(np.uint16)
    return ((bits >> 7) & 0xFF).astype(np.uint8)


def cases():
    out = []
    rng = np.random.default_rng(0)
    out.append(("skewed_2sym", rng.choice([3, 9], size=2000, p=[0.95, 0.05]), 64, 16))
    rng = np.random.default_rng(1)
    out.append(("uniform16", rng.integers(0, 16, size=1000), 100, 16))
    rng = np.random.default_rng(2)
    out.append(("uniform256", rng.integers(0, 256, size=8000), 256, 16))
    for seed in range(10):
        rng = np.random.default_rng(100 + seed)
        k = int(rng.integers(2, 200))
        probs = rng.dirichlet(np.ones(k) * rng.uniform(0.1, 3.0))
        data = rng.choice(k, size=int(rng.integers(2000, 8000)), p=probs)
        out.append(("dirichlet_%d" % seed, data, int(rng.choice([64, 128, 256, 512])), 16))
    fib = [1, 1]
    while len(fib) < 40:
        fib.append(fib[-1] + fib[-2])
    probs = np.array(fib, dtype=np.float64) / sum(fib)
    rng = np.random.default_rng(3)
    out.append(("fibonacci40_mb6", rng.choice(40, size=20000, p=probs), 1000, 6))
    out.append(("bf16_n002", _bf16_exponents(np.random.default_rng(4), 131072, 0.02), 512, 16))
    out.append(("bf16_outliers_64k", _bf16_exponents(np.random.default_rng(5), 4 * 65536, 0.02,
                                                       1e-3), 65536, 16))
    out.append(("single_symbol", np.full(500, 7), 64, 16))
    for cs in (32, 128, 1024):
        for mb in (8, 12):
            out.append(("bf16_cs%d_mb%d" % (cs, mb),
                        _bf16_exponents(np.random.default_rng(cs + mb), 20000, 0.02), cs, mb))
    rng = np.random.default_rng(6)
    out.append(("nondivide_7777_333", rng.integers(0, 200, size=7777), 333, 16))
    rng = np.random.default_rng(7)
    out.append(("chunk16_2000", rng.integers(50, 80, size=2000), 16, 16))
    out.append(("scales_3p0", _bf16_exponents(np.random.default_rng(8), 16384, 3.0), 1024, 16))
    out.append(("scales_0p001", _bf16_exponents(np.random.default_rng(9), 16384, 0.001), 1024, 16))
    return out


def main(ref_root: str) -> None:
    sys.path.insert(0, ref_root)
    from afterimage.runtime import compressed_store as cs
    from afterimage.runtime import huffman as hf
    from afterimage.runtime import huffman_chunked as hc

    arrays: dict[str, np.ndarray] = {}
    names = []
    for name, data, chunk_size, max_bits in cases():
        sym = np.asarray(data).astype(np.uint8)
        enc = hc.encode_chunked(torch.from_numpy(sym.astype(np.int64)), chunk_size=chunk_size,
                                max_bits=max_bits)
        dec = hc.decode_chunked_cpu_reference(enc)
        assert np.array_equal(dec, sym), name
        counts = np.bincount(sym, minlength=256)
        freqs = {int(s): int(c) for s, c in enumerate(counts) if c > 0}
        lengths = hf.build_lengths(freqs, max_bits=max_bits)
        lens = np.zeros(256, dtype=np.int8)
        for s, ln in lengths.items():
            lens[s] = ln
        p = "case/%s/" % name
        arrays[p + "symbols"] = sym
        arrays[p + "params"] = np.array([chunk_size, max_bits, enc.max_bits, enc.n_symbols],
                                        dtype=np.int64)
        arrays[p + "lengths"] = lens
        arrays[p + "packed"] = np.asarray(enc.packed, dtype=np.uint8)
        arrays[p + "chunk_offsets"] = np.asarray(enc.chunk_offsets, dtype=np.int32)
        arrays[p + "chunk_nbytes"] = np.asarray(enc.chunk_nbytes, dtype=np.int32)
        arrays[p + "sym_lut"] = np.asarray(enc.sym_lut, dtype=np.int32)
        arrays[p + "len_lut"] = np.asarray(enc.len_lut, dtype=np.int8)
        # Decode of a chunk-range slice whose last chunk is partial: the
        # reference decodes whole chunks, so this records what it yields at
        # positions past the real symbols.
        if enc.n_chunks >= 2 and enc.n_symbols % chunk_size:
            c0 = max(0, enc.n_chunks - 3)
            sub = cs._slice_encoded(enc, c0, enc.n_chunks)
            arrays[p + "slice_tail"] = np.array([c0, enc.n_chunks], dtype=np.int64)
            arrays[p + "slice_tail_decoded"] = np.asarray(
                hc.decode_chunked_cpu_reference(sub), dtype=np.int32).astype(np.uint8)
        names.append(name)

    # build_lengths on the Fibonacci frequencies themselves (package-merge).
    fib = [1, 1]
    while len(fib) < 40:
        fib.append(fib[-1] + fib[-2])
    for mb in (6, 8, 16):
        lens = hf.build_lengths({s: f for s, f in enumerate(fib)}, max_bits=mb)
        arrays["fib_lengths/mb%d" % mb] = np.array([lens[s] for s in range(40)], dtype=np.int8)

    # Single-stream packing and both single-stream decoders of huffman.py.
    rng = np.random.default_rng(11)
    data = rng.choice(12, size=3000, p=rng.dirichlet(np.ones(12) * 0.7))
    et = hf.encode_exponents(torch.from_numpy(data.astype(np.int64)), max_bits=16)
    arrays["stream/symbols"] = data.astype(np.uint8)
    arrays["stream/packed"] = np.frombuffer(et.packed, dtype=np.uint8).copy()
    arrays["stream/decode_reference"] = hf.decode_reference(
        et.packed, et.table, et.codes, et.n_symbols).astype(np.int32)
    arrays["stream/decode_lut_cpu"] = hf.decode_lut_cpu(
        et.packed, et.sym_lut, et.len_lut, et.table.max_bits, et.n_symbols).astype(np.int32)

    # BF16 known answers through compress_layer + the CPU reference decode.
    kat = torch.tensor([0, -32768, 32640, -128, 32705, -63, 1, 127, 128, 16256, -16512, 32767],
                       dtype=torch.int16).reshape(3, 4)
    special = torch.tensor([0.0, -0.0, 1.0, -1.0, 1e-30, -1e-30, 1e30, -1e30, 3.14159],
                           dtype=torch.bfloat16).reshape(3, 3)
    torch.manual_seed(0)
    real = (torch.randn(128, 512) * 0.02).to(torch.bfloat16)
    for name, w, chunk in (("kat_int16", kat.view(torch.bfloat16), 5),
                           ("special_values", special, 9),
                           ("randn_128x512", real, 256)):
        layer = cs.compress_layer(w, chunk_size=chunk)
        recon = cs.decompress_layer_cpu_reference(layer)
        p = "bf16/%s/" % name
        arrays[p + "bits"] = w.contiguous().view(torch.int16).numpy().reshape(-1).copy()
        arrays[p + "shape"] = np.array(w.shape, dtype=np.int64)
        arrays[p + "chunk_size"] = np.array([chunk], dtype=np.int64)
        arrays[p + "sign_mantissa"] = layer.sign_mantissa.numpy().copy()
        arrays[p + "packed"] = np.asarray(layer.encoded.packed, dtype=np.uint8)
        arrays[p + "chunk_nbytes"] = np.asarray(layer.encoded.chunk_nbytes, dtype=np.int32)
        arrays[p + "decoded_bits"] = recon.contiguous().view(torch.int16).numpy().reshape(-1).copy()

    arrays["case_names"] = np.array(names)
    np.savez_compressed(OUT, **arrays)
    print("wrote %s (%d bytes, %d cases)" % (OUT, OUT.stat().st_size, len(names)))


if __name__ == "__main__":
    main(sys.argv[1] if len(sys.argv) > 1 else "/root/reference")
