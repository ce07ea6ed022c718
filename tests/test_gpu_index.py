"""Segment index (aimg_build_index) on the GPU: its entries against a CPU walk
of the codeword starts, and decodes with it against decodes without it and
against the known weights / exponents.

The index has no counterpart in the reference (its decoder runs one chunk per
lane and needs none); these tests pin it to the reference's decode results,
which the decodes without the index already equal (test_gpu_decode.py).
"""
import numpy as np
import pytest
import torch

from afterimage_amd import workloads
from afterimage_amd.runtime.compressed_store import compress_layer, compress_group
from afterimage_amd.runtime.device import (
    DeviceTensor,
    TABLES,
    decode_bf16,
    decode_gemv,
    decode_u8,
    segment_bits,
)
from afterimage_amd.runtime.huffman_chunked import encode_chunked
from tests.distributions import many_escape_windows

pytestmark = pytest.mark.gpu

DEV = "cuda"


def _starts(enc, c):
    """Bit offsets of the codewords that start inside chunk c, walking from
    its first bit (bits past the chunk read as zero, and a window the LUT has
    no codeword for takes the shortest code length), then the end of the
    last of them."""
    off, nb = int(enc.chunk_offsets[c]), int(enc.chunk_nbytes[c])
    data = np.frombuffer(np.asarray(enc.packed, np.uint8)[off: off + nb].tobytes() + b"\0" * 4,
                         np.uint8)
    mb = int(enc.max_bits)
    lens = np.asarray(enc.len_lut, np.int64)
    min_len = int(lens[lens > 0].min())
    out, p, end = [], 0, 8 * nb
    while p < end:
        b = p >> 3
        w = (int(data[b]) << 16 | int(data[b + 1]) << 8 | int(data[b + 2])) >> (8 - (p & 7))
        idx = (w >> (16 - mb)) & ((1 << mb) - 1)
        ln = int(lens[idx]) or min_len
        out.append(p)
        p += ln
    out.append(p)
    return np.asarray(out, np.int64)


def _expected_index(enc, seg):
    """(bases, rends, raw entries) of the index: per chunk, per segment of seg
    bits, the first boundary's offset from the segment start | count << 4,
    where count takes only the codewords before the chunk's real end (the
    end of its lim-th codeword, lim its output elements)."""
    bases, rends, entries = [], [], []
    n_jobs = -(-int(enc.n_symbols) // int(enc.chunk_size))
    for c in range(len(enc.chunk_offsets)):
        bases.append(len(entries))
        if c >= n_jobs:
            rends.append(None)
            continue
        lim = min(int(enc.chunk_size), int(enc.n_symbols) - c * int(enc.chunk_size))
        bounds = _starts(enc, c)
        st = bounds[:-1]
        rend = int(bounds[lim])  # end of the lim-th codeword
        rends.append(rend)
        nseg = -(-8 * int(enc.chunk_nbytes[c]) // seg)
        for k in range(nseg):
            lo = k * seg
            inside = st[(st >= lo) & (st < lo + seg) & (st < rend)]
            f = int(bounds[bounds >= lo][0]) - lo
            entries.append(f | (len(inside) << 4))
    bases.append(len(entries))
    return np.asarray(bases, np.uint32), rends, np.asarray(entries, np.uint16)


def _layout(t, seg):
    """Byte offsets of the index arrays (header, bases, real ends, entries,
    round starts)."""
    n = t.n_chunks
    cap = -(-8 * int(t.packed.numel()) // seg) + n
    base = 64
    rend = base + 4 * (n + 1)
    entries = (rend + 4 * n + 15) & ~15
    rounds = (entries + 4 * cap + 15) & ~15
    return base, rend, entries, cap, rounds


def _index_arrays(t, seg):
    ix = t.index.cpu().numpy()
    hdr = ix[:64].view(np.uint32)
    n = t.n_chunks
    base, rend, entries, cap, rounds = _layout(t, seg)
    return (hdr, ix[base: base + 4 * (n + 1)].view(np.uint32), ix[rend: rend + 4 * n].view(np.uint32),
            ix[entries: entries + 4 * cap].view(np.uint32),
            ix[rounds: rounds + 16 * (cap // 512 + 2)].view(np.uint32).reshape(-1, 4))


def _final_entries(bases, raw):
    """The entries as decodes read them: offset | jj << 4 | excl << 10, with
    jj the segment's chunk minus its round's first chunk (at most 63: segment
    runs take chunks of 1024 symbols or more, at most 40 to a round) and excl
    the counts of its round's segments before it (rounds: 512 segments)."""
    counts = raw.astype(np.int64) >> 4
    out = np.zeros(len(raw), np.uint32)
    for g0 in range(0, len(raw), 512):
        c0 = int(np.searchsorted(bases, g0, side="right")) - 1
        excl = 0
        for g in range(g0, min(g0 + 512, len(raw))):
            c = int(np.searchsorted(bases, g, side="right")) - 1
            out[g] = (int(raw[g]) & 15) | (min(c - c0, 63) << 4) | (excl << 10)
            excl += int(counts[g])
    return out


def _expected_rounds(enc, seg, bases, entries):
    """Round starts: for segment g = 512 m, its chunk c, the output element
    of its first codeword (c * chunk_size + the counts of the chunk's
    segments before g), its packed byte and the chunk's first segment."""
    out = []
    counts = entries.astype(np.int64) >> 4
    for g in range(0, len(entries), 512):
        c = int(np.searchsorted(bases, g, side="right")) - 1
        el = c * int(enc.chunk_size) + int(counts[bases[c]: g].sum())
        byte = int(enc.chunk_offsets[c]) + (g - int(bases[c])) * (seg // 8)
        out.append((c, el, byte, int(bases[c])))
    return np.asarray(out, np.int64).reshape(-1, 4)


@pytest.mark.parametrize("kind,chunk", [("skewed", 64), ("skewed", 1024), ("bf16", 4096),
                                        ("bf16", 65536), ("escapes", 4096)])
def test_index_entries_equal_a_cpu_walk_of_the_codeword_starts(kind, chunk):
    if kind == "skewed":
        torch.manual_seed(0)
        exps = torch.randint(100, 140, (9000,))
    elif kind == "escapes":
        exps = torch.as_tensor(many_escape_windows(seed=5, n=30000))
    else:
        W = workloads.bf16_normal((64, 4500), 3, 0.02, outlier_frac=1e-3)
        exps = ((W.view(torch.int16).to(torch.int32) & 0xFFFF) >> 7 & 0xFF).reshape(-1)
    enc = encode_chunked(exps, chunk_size=chunk)
    t = DeviceTensor.from_encoded(enc, None, DEV).build_index()
    seg = segment_bits(t.tables.host_blob)
    hdr, bases, rends, entries, rounds = _index_arrays(t, seg)
    want_b, want_r, want_e = _expected_index(enc, seg)
    assert hdr[2] == seg and hdr[4] == 1, "header: seg_bits %d ok %d" % (hdr[2], hdr[4])
    assert hdr[6] == len(want_e), "segments %d, want %d" % (hdr[6], len(want_e))
    assert np.array_equal(bases, want_b)
    assert [int(r) for r, w in zip(rends, want_r) if w is not None] == \
        [w for w in want_r if w is not None]
    got = entries[: len(want_e)]
    want_f = _final_entries(want_b, want_e)
    bad = np.nonzero(got != want_f)[0]
    assert bad.size == 0, "entries differ at %s: %s vs %s" % (bad[:5], got[bad[:5]], want_f[bad[:5]])
    want_rs = _expected_rounds(enc, seg, want_b, want_e)
    assert np.array_equal(rounds[: len(want_rs)].astype(np.int64), want_rs)
    # After the last round, the tensor's end.
    assert int(rounds[len(want_rs)][1]) == int(enc.n_symbols)
    assert np.array_equal(decode_u8([t])[0].cpu().numpy(), exps.numpy().astype(np.uint8))


@pytest.mark.parametrize("chunk", [16, 64, 256, 1024, 4096, 16384, 65536])
def test_u8_decode_with_index_equals_the_exponents(chunk):
    torch.manual_seed(chunk)
    exps = torch.randint(60, 130, (50000,))
    enc = encode_chunked(exps, chunk_size=chunk)
    t = DeviceTensor.from_encoded(enc, None, DEV)
    plain = decode_u8([t])[0].cpu().numpy()
    t.build_index()
    got = decode_u8([t])[0].cpu().numpy()
    assert np.array_equal(plain, exps.numpy().astype(np.uint8))
    assert np.array_equal(got, plain)


def test_full_alphabet_and_ragged_tail_with_index():
    torch.manual_seed(1)
    exps = torch.randint(0, 256, (7777,))
    enc = encode_chunked(exps, chunk_size=333)
    t = DeviceTensor.from_encoded(enc, None, DEV).build_index()
    assert np.array_equal(decode_u8([t])[0].cpu().numpy(), exps.numpy().astype(np.uint8))


def test_bf16_full_layer_with_index_is_bit_exact():
    W = workloads.bf16_normal((5120, 17408), 2, 0.02, outlier_frac=1e-3)
    layer = compress_layer(W, chunk_size=65536)
    t = DeviceTensor.from_encoded(layer.encoded, layer.sign_mantissa, DEV).build_index()
    out = decode_bf16([t])[0]
    assert torch.equal(out.view(torch.int16).cpu(), W.reshape(-1).view(torch.int16))
    # Index size: 4 bytes per 168-bit segment (2.6 bits per exponent), about
    # 4.7% of the compressed layer.
    comp = t.packed.numel() + t.sign_mantissa.numel()
    assert t.index.numel() < 0.05 * comp


def test_block_with_and_without_indexes_in_one_launch():
    blk = workloads.block_14b(scale=0.01, chunk_size=65536)
    ts = [DeviceTensor.from_encoded(l.encoded, l.sign_mantissa, DEV) for _, _, l in blk]
    for k, t in enumerate(ts):
        if k % 2 == 0:
            t.build_index()
    outs = decode_bf16(ts)
    for (name, w, _), o in zip(blk, outs):
        assert torch.equal(o.view(torch.int16).cpu(), w.reshape(-1).view(torch.int16)), name


def test_index_of_another_codebook_is_ignored():
    ws = [workloads.bf16_normal((300, 2000), s, 0.02 * (s + 1), outlier_frac=1e-3) for s in (1, 2)]
    la, lb = (compress_layer(w, chunk_size=4096) for w in ws)
    ta = DeviceTensor.from_encoded(la.encoded, la.sign_mantissa, DEV).build_index()
    tb = DeviceTensor.from_encoded(lb.encoded, lb.sign_mantissa, DEV)
    # tb's bytes decoded with ta's index: the index records ta's table, so
    # the decoder must not use it (different checksum).
    tb.index = ta.index
    assert not np.array_equal(la.encoded.sym_lut, lb.encoded.sym_lut) or \
        not np.array_equal(la.encoded.len_lut, lb.encoded.len_lut)
    out = decode_bf16([tb])[0]
    assert torch.equal(out.view(torch.int16).cpu(), ws[1].reshape(-1).view(torch.int16))


def test_shared_codebook_tensors_each_with_an_index():
    ws = [workloads.bf16_normal((256, 3000), s, 0.02, outlier_frac=1e-3) for s in (4, 5, 6)]
    layers = compress_group(ws, chunk_size=2048)
    ts = [DeviceTensor.from_encoded(l.encoded, l.sign_mantissa, DEV).build_index() for l in layers]
    assert len({id(t.tables) for t in ts}) == 1
    for w, o in zip(ws, decode_bf16(ts)):
        assert torch.equal(o.view(torch.int16).cpu(), w.reshape(-1).view(torch.int16))


def test_an_index_too_small_is_marked_unusable_and_ignored():
    W = workloads.bf16_normal((200, 3000), 7, 0.02, outlier_frac=1e-3)
    layer = compress_layer(W, chunk_size=4096)
    t = DeviceTensor.from_encoded(layer.encoded, layer.sign_mantissa, DEV)
    t.index = torch.zeros(t.index_nbytes - 16, dtype=torch.uint8, device=DEV)
    from afterimage_amd import _native
    from afterimage_amd.runtime.device import _descriptor, _stream_handle
    d = (_native.AimgTensor * 1)()
    d[0] = _descriptor(t, None, t.n_symbols)
    _native.check(_native.lib().aimg_build_index(d, 1, _stream_handle(DEV)))
    hdr = t.index[:64].cpu().numpy().view(np.uint32)
    assert hdr[4] == 0
    out = decode_bf16([t])[0]
    assert torch.equal(out.view(torch.int16).cpu(), W.reshape(-1).view(torch.int16))


@pytest.mark.parametrize("batch", [1, 4])
def test_gemv_with_index_matches_without(batch):
    W = workloads.bf16_normal((1024, 4096), 8, 0.02, outlier_frac=1e-3)
    layer = compress_layer(W, chunk_size=65536)
    t = DeviceTensor.from_encoded(layer.encoded, layer.sign_mantissa, DEV)
    g = torch.Generator().manual_seed(9)
    x = torch.randn((batch, 4096), generator=g).to(torch.bfloat16).to(DEV)
    y0 = decode_gemv(t, x, 1024, 4096)
    t.build_index()
    y1 = decode_gemv(t, x, 1024, 4096)
    want = (x.double().cpu() @ W.double().t()).float()
    assert torch.allclose(y1.cpu(), want, rtol=1e-2, atol=1e-3)
    assert torch.allclose(y1, y0, rtol=1e-4, atol=1e-4)


@pytest.mark.parametrize("strided", ["1", "0"])
@pytest.mark.parametrize("chunk", [1024, 2048, 65536])
def test_segment_runs_split_chunks_over_the_grid(chunk, strided, monkeypatch):
    # Large enough for a full grid: every workgroup's rounds (in turn, or a
    # contiguous range with AIMG_RUN_STRIDED=0) start and end inside chunks.
    monkeypatch.setenv("AIMG_RUN_STRIDED", strided)
    W = workloads.bf16_normal((2048, 8192), 16, 0.02, outlier_frac=1e-3)
    layer = compress_layer(W, chunk_size=chunk)
    t = DeviceTensor.from_encoded(layer.encoded, layer.sign_mantissa, DEV).build_index()
    out = decode_bf16([t])[0]
    assert torch.equal(out.view(torch.int16).cpu(), W.reshape(-1).view(torch.int16))


def test_chunks_not_back_to_back_make_the_index_unusable():
    # Same bytes, chunk 1 moved to the end of the buffer: still a valid
    # compressed tensor, but its chunks do not follow one another.
    W = workloads.bf16_normal((64, 4096), 17, 0.02, outlier_frac=1e-3)
    layer = compress_layer(W, chunk_size=4096)
    enc = layer.encoded
    packed = np.asarray(enc.packed, np.uint8)
    offs = np.asarray(enc.chunk_offsets, np.int32).copy()
    nbs = np.asarray(enc.chunk_nbytes, np.int32)
    moved = packed[offs[1]: offs[1] + nbs[1]].copy()
    packed2 = np.concatenate([packed, moved])
    offs[1] = len(packed)
    t = DeviceTensor.from_encoded(enc, layer.sign_mantissa, DEV)
    t.packed = torch.from_numpy(packed2).to(DEV)
    t.chunk_offsets = torch.from_numpy(offs).to(DEV)
    t.build_index(keep_unusable=True)
    assert not t.index_usable
    out = decode_bf16([t])[0]
    assert torch.equal(out.view(torch.int16).cpu(), W.reshape(-1).view(torch.int16))


def test_packed_buffer_past_512_mib_with_and_without_the_index():
    # 95 copies of a 1024x17408 layer's chunks (each chunk is its own
    # stream, so the copies form a valid tensor): 1.69e9 weights, about 550 MB
    # of packed bits, so bit positions in the packed buffer pass 2^32. The
    # decoders keep positions within a chunk or a round; with absolute bit
    # numbers in 32 bits, segments past the wrap would be dropped.
    import types
    W, layer = workloads.single_layer(seed=9, rows=1024, cols=17408, chunk_size=65536)
    enc = layer.encoded
    k = 95
    nb = np.asarray(enc.chunk_nbytes, np.int64)
    used = int(nb.sum())
    offs = np.asarray(enc.chunk_offsets, np.int64)
    packed = np.concatenate([np.tile(np.asarray(enc.packed, np.uint8)[:used], k),
                             np.zeros(8, np.uint8)])
    big = types.SimpleNamespace(
        packed=packed,
        chunk_offsets=np.concatenate([offs + j * used for j in range(k)]).astype(np.int32),
        chunk_nbytes=np.tile(nb, k).astype(np.int32), sym_lut=enc.sym_lut, len_lut=enc.len_lut,
        max_bits=enc.max_bits, chunk_size=enc.chunk_size, n_symbols=k * enc.n_symbols,
        shape=(k * enc.n_symbols,))
    assert 8 * used * k > 1 << 32 and big.n_symbols < 1 << 31
    sm = np.tile(layer.sign_mantissa.reshape(-1).numpy(), k)
    t = DeviceTensor.from_encoded(big, sm, DEV)
    del packed, sm
    want = W.reshape(-1).to(DEV).view(torch.int16)
    n_small = enc.n_symbols

    def check(out):
        o = out.view(torch.int16)
        for j in range(k):
            assert torch.equal(o[j * n_small:(j + 1) * n_small], want), "copy %d" % j

    out = decode_bf16([t])[0]
    check(out)
    t.build_index()
    assert t.index is not None
    out.zero_()
    decode_bf16([t], [out])
    check(out)
