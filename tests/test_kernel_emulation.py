"""The decode kernel's own source, compiled for the host under AddressSanitizer
(tests/kernel_emulation/hip/hip_runtime.h stands in for the HIP device
subset it uses) and run on small cases of every kernel variant: the scalar
and vector store paths, 16..512 threads per chunk, two-round 64Ki chunks,
escape blocks beyond the LDS share, and the tiny-buffer kernel.

This checks memory safety on the CPU before any GPU run: each device buffer
is a heap block of exactly its size, so an access past any of them, or past
the kernel's LDS block, fails the run with the offending source line. The
outputs are compared with the known weights / exponents as well; the fused
GEMV's y within the GPU tests' tolerance of a float64 product (the stand-in
gives true wave ballots, readlane and DPP).
"""
import os
import re
import shutil
import subprocess

import numpy as np
import pytest
import torch

from afterimage_amd import workloads
from afterimage_amd.runtime.compressed_store import compress_layer
from afterimage_amd.runtime.huffman_chunked import encode_chunked
from tests.distributions import many_escape_windows

HERE = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(HERE)
CXX = "/opt/rocm/llvm/bin/clang++"

pytestmark = pytest.mark.skipif(not os.path.exists(CXX), reason="needs ROCm's clang++ for the host build")
# The long cases (most of the emulator's time: a host thread per work-item,
# several thousand per launch) run with AIMG_EMULATION_FULL=1; the default
# run keeps a representative set of each path (chunk by chunk, whole and
# sub-group chunks, segment runs with an index, speculative runs, the fused
# GEMV and GEMM) within a few minutes.
full = pytest.mark.skipif(os.environ.get("AIMG_EMULATION_FULL") != "1",
                          reason="long emulation case: AIMG_EMULATION_FULL=1 runs it")


@pytest.fixture(scope="module")
def emu(tmp_path_factory):
    d = tmp_path_factory.mktemp("kernel_emulation")
    src = open(os.path.join(ROOT, "afterimage_amd", "csrc", "aimg_decode.hip")).read()
    # Host spelling of three device-only constructs: address-space qualifiers,
    # VGPR asm operands, and LDS offsets taken from generic pointers (a host
    # pointer keeps all its bits).
    src = re.sub(r"__attribute__\(\(address_space\(\d+\)\)\)", "", src)
    src = src.replace('"+v"', '"+r"').replace('::"v"', '::"r"')
    assert "using LdsOff = uint32_t;" in src
    src = src.replace("using LdsOff = uint32_t;", "using LdsOff = uintptr_t;")
    (d / "aimg_decode_emu.cpp").write_text(src)
    flags = ["-std=c++20", "-g", "-O1", "-fsanitize=address", "-fno-omit-frame-pointer",
             "-I", os.path.join(HERE, "kernel_emulation"), "-I", os.path.join(ROOT, "include"),
             "-I", os.path.join(ROOT, "afterimage_amd", "csrc"), "-w"]
    objs = []
    for s in (str(d / "aimg_decode_emu.cpp"), os.path.join(ROOT, "afterimage_amd", "csrc", "aimg_host.cpp"),
              os.path.join(HERE, "kernel_emulation", "driver.cpp")):
        o = str(d / (os.path.basename(s) + ".o"))
        subprocess.run([CXX, *flags, "-c", s, "-o", o], check=True)
        objs.append(o)
    exe = str(d / "emu")
    subprocess.run([CXX, "-fsanitize=address", "-o", exe, *objs, "-lpthread"], check=True)
    yield exe, d
    shutil.rmtree(d, ignore_errors=True)


def _write(d, enc, expect, sm=None):
    os.makedirs(d, exist_ok=True)
    np.asarray(enc.packed, np.uint8).tofile(os.path.join(d, "packed.bin"))
    np.asarray(enc.chunk_offsets, np.int32).tofile(os.path.join(d, "offsets.bin"))
    np.asarray(enc.chunk_nbytes, np.int32).tofile(os.path.join(d, "nbytes.bin"))
    np.asarray(enc.sym_lut, np.int32).tofile(os.path.join(d, "sym_lut.bin"))
    np.asarray(enc.len_lut, np.int8).tofile(os.path.join(d, "len_lut.bin"))
    np.ascontiguousarray(expect).view(np.uint8).tofile(os.path.join(d, "expect.bin"))
    if sm is not None:
        np.asarray(sm, np.uint8).tofile(os.path.join(d, "sm.bin"))
    with open(os.path.join(d, "meta.txt"), "w") as f:
        f.write("%d %d %d %d\n" % (enc.max_bits, enc.chunk_size, enc.n_symbols, len(enc.chunk_offsets)))


def _run(emu, name, mode, index="", runs=None, strided=None, cus=None, copies=None, spec=None):
    exe, d = emu
    env = dict(os.environ, ASAN_OPTIONS="detect_leaks=0:abort_on_error=0")
    env.pop("AIMG_SEGMENT_RUNS", None)
    env.pop("AIMG_RUN_STRIDED", None)
    env.pop("AIMG_EMU_CUS", None)
    env.pop("AIMG_EMU_COPIES", None)
    env.pop("AIMG_SPEC_RUNS", None)
    env.pop("AIMG_CHUNK_SPLIT", None)
    if spec is not None:
        # "0": tensors without an index decode chunk by chunk; "1": in
        # speculative runs whatever their chunk size
        env["AIMG_SPEC_RUNS"] = spec
    if cus is not None:
        env["AIMG_EMU_CUS"] = str(cus)  # a grid of 2 * cus workgroups
    if copies is not None:
        env["AIMG_EMU_COPIES"] = str(copies)  # the tensor decoded this many times in one launch
    if runs is not None:
        env["AIMG_SEGMENT_RUNS"] = runs
    if strided is not None:
        env["AIMG_RUN_STRIDED"] = strided
    args = [exe, str(d / name), mode] + ([index] if index else [])
    r = subprocess.run(args, capture_output=True, text=True, env=env, timeout=1800)
    assert r.returncode == 0 and ": ok" in r.stdout, (r.stdout + r.stderr)[-4000:]


def _u8(emu, name, exps, chunk_size, index="", cus=None, spec=None):
    exps = np.asarray(exps)
    enc = encode_chunked(torch.as_tensor(exps), chunk_size=chunk_size)
    _write(emu[1] / name, enc, exps.astype(np.uint8))
    _run(emu, name, "u8", index, cus=cus, spec=spec)


def _bf16(emu, name, W, chunk_size, index="", runs=None, strided=None, cus=None, copies=None,
          spec=None):
    layer = compress_layer(W, chunk_size=chunk_size)
    _write(emu[1] / name, layer.encoded, W.reshape(-1).view(torch.int16).numpy(),
           layer.sign_mantissa.numpy())
    _run(emu, name, "bf16", index, runs, strided, cus, copies, spec)


def _gemv(emu, name, rows, cols, chunk_size, batch, seed, index="", runs=None, cus=None, spec=None,
          mode="gemv"):
    W = workloads.bf16_normal((rows, cols), seed, 0.02, outlier_frac=1e-3)
    layer = compress_layer(W, chunk_size=chunk_size)
    g = np.random.default_rng(seed + 1)
    x = torch.from_numpy(g.standard_normal((batch, cols), dtype=np.float32)).to(torch.bfloat16)
    want = (x.double() @ W.double().t()).float()
    d = emu[1] / name
    _write(d, layer.encoded, np.zeros(1, np.uint8), layer.sign_mantissa.numpy())
    x.view(torch.int16).numpy().tofile(os.path.join(d, "x.bin"))
    want.numpy().tofile(os.path.join(d, "expect_y.bin"))
    with open(os.path.join(d, "gemv.txt"), "w") as f:
        f.write("%d %d %d\n" % (rows, cols, batch))
    _run(emu, name, mode, index, runs, cus=cus, spec=spec)


@pytest.mark.parametrize("batch", [1, 4])
def test_gemv_16_thread_chunks_spanning_rows(emu, batch):
    # 64-symbol chunks of 40-column rows: several chunks, and rows, per wave step.
    _gemv(emu, "gemv16_b%d" % batch, 96, 40, 64, batch, 3)


@pytest.mark.parametrize("batch", [1, 4])
def test_gemv_512_thread_chunks_with_row_crossings(emu, batch):
    # 32768-symbol chunks (512 threads) over 1000-column rows: wave steps of
    # 512 elements cross a row boundary about every other step.
    _gemv(emu, "gemv512_b%d" % batch, 70, 1000, 32768, batch, 5)


def test_gemv_512_thread_chunks_rows_shorter_than_a_wave_step(emu):
    _gemv(emu, "gemv512_short", 300, 200, 32768, 2, 7)


def test_u8_small_chunks_16_threads_per_chunk(emu):
    torch.manual_seed(0)
    _u8(emu, "skewed64", torch.randint(100, 140, (2000,)).numpy(), 64)


@pytest.mark.parametrize("chunk_size", [32, 256, 1024])
def test_u8_chunk_sizes(emu, chunk_size):
    torch.manual_seed(3)
    _u8(emu, "sizes%d" % chunk_size, torch.randint(50, 90, (10000,)).numpy(), chunk_size)


def test_u8_full_alphabet(emu):
    torch.manual_seed(1)
    _u8(emu, "uniform256", torch.randint(0, 256, (8000,)).numpy(), 256)


@full
def test_u8_escape_blocks_beyond_the_lds_share(emu):
    _u8(emu, "escapes", many_escape_windows(seed=5, n=30000), 4096)


def test_u8_tiny_packed_buffer(emu):
    _u8(emu, "tiny", np.array([7, 7, 7], np.uint8), 64)


@full
@pytest.mark.parametrize("spec", ["1", "0"])
def test_bf16_vector_path(emu, spec):
    # 64-thread chunks: speculative runs, and 8 chunks a workgroup.
    torch.manual_seed(2)
    _bf16(emu, "bf16_vec%s" % spec, (torch.randn(256, 1024) * 0.02).to(torch.bfloat16), 4096, cus=2,
          spec=spec)


def test_bf16_scalar_path_ragged(emu):
    torch.manual_seed(4)
    _bf16(emu, "bf16_ragged", (torch.randn(300, 333) * 0.02).to(torch.bfloat16), 1000)


def test_bf16_whole_workgroup_chunks(emu):
    # Three 65536-symbol chunks, each a workgroup's (interleaved slots, one
    # record barrier per round), two rounds each, the last chunk ragged.
    W = workloads.bf16_normal((23, 8192), 12, 0.02, outlier_frac=1e-3)
    _bf16(emu, "bf16_whole", W, 65536)


def test_bf16_whole_workgroup_chunks_several_per_workgroup(emu):
    # Seven 65536-symbol chunks on a 1-CU grid (2 workgroups): each workgroup
    # goes from item to item, its next item's job prepared during the
    # current one; a 1024-symbol tensor in the same launch (two tables).
    W = workloads.bf16_normal((27, 16384), 13, 0.02, outlier_frac=1e-3)
    _bf16(emu, "bf16_whole_items", W, 65536, cus=1, spec="0")


def test_bf16_split_chunks_hand_over_or_decode_whole(emu):
    # Seven 65536-symbol chunks on a grid of 4 workgroups: the last pass
    # would hold 3 chunks, so those are split in halves (rounds 0 and 1). The
    # emulator runs workgroups one after another: the second half of chunk 4
    # (workgroup 3) takes the record its first half (workgroup 0) wrote; those
    # of chunks 5 and 6 (workgroups 0 and 1) wait for first halves of later
    # workgroups, give up and decode their chunks whole, and those first
    # halves then find their records given up and empty them.
    W = workloads.bf16_normal((27, 16384), 14, 0.02, outlier_frac=1e-3)
    _bf16(emu, "bf16_split", W, 65536, cus=2, spec="0")


@pytest.mark.parametrize("shape", [(40, 4096), (30,)])
def test_bf16_whole_workgroup_chunks_without_slack_bytes(emu, shape):
    # The packed buffer ends at the last chunk's last byte: the last words
    # are loaded from the buffer's last whole word and shifted back.
    import dataclasses
    W = workloads.bf16_normal(shape, 123, 0.02)
    layer = compress_layer(W, chunk_size=65536)
    enc = layer.encoded
    used = int(enc.chunk_offsets[-1]) + int(enc.chunk_nbytes[-1])
    trimmed = dataclasses.replace(enc, packed=np.asarray(enc.packed)[:used].copy())
    name = "bf16_noslack_%d" % W.numel()
    _write(emu[1] / name, trimmed, W.reshape(-1).view(torch.int16).numpy(), layer.sign_mantissa.numpy())
    _run(emu, name, "bf16", spec="0")


def test_u8_split_chunks_across_tensors(emu):
    # Three copies of a 7-chunk tensor (21 chunks) on a grid of 12: the last
    # 9 chunks (two of the second tensor, seven of the third) are split.
    # Exponent bytes carry partial 16-byte groups between the halves.
    rng = np.random.default_rng(15)
    exps = np.clip(np.rint(rng.normal(120, 2.0, 7 * 65536 - 3000)), 100, 140).astype(np.int64)
    enc = encode_chunked(torch.as_tensor(exps), chunk_size=65536)
    _write(emu[1] / "u8_split", enc, exps.astype(np.uint8))
    _run(emu, "u8_split", "u8", cus=6, copies=3, spec="0")


@full
def test_bf16_two_round_64k_chunks_with_outliers(emu):
    W = workloads.bf16_normal((64, 17408), 2, 0.02, outlier_frac=1e-3)
    _bf16(emu, "bf16_64k", W, 65536)


@full
def test_u8_segment_guesses_all_wrong(emu):
    # Eight equiprobable symbols get 3-bit codes; segment starts are multiples
    # of 168 bits, and the 32-bit lead-in before each lands one bit past a
    # codeword boundary, which fixed-length codes never leave. Every thread
    # but the first is wrong on its first pass, so the result rests entirely
    # on the re-decode from the predecessor's end.
    # The 65536-symbol chunk (a whole workgroup's) holds 6000 symbols: 108
    # segments, each found on its own pass; the 4096-symbol chunks (two, in
    # speculative runs) 73 segments each.
    rng = np.random.default_rng(8)
    _u8(emu, "guess4096", rng.integers(0, 8, 4096 + 700), 4096, cus=2)
    _u8(emu, "guess65536", rng.integers(0, 8, 6000), 65536)


# Decoding with the segment index (aimg_build_index): the index is built by
# the chunk kernel's build mode and the round and finish steps, then tensors
# whose chunks hold 1024 symbols or more decode in segment runs, each segment
# from its recorded start straight into place (smaller chunks and the
# element-wise path ignore the index); the result must equal the weights /
# exponents.

@pytest.mark.parametrize("chunk_size", [64, 1024, 4096])
def test_u8_with_index(emu, chunk_size):
    torch.manual_seed(11)
    _u8(emu, "ix_u8_%d" % chunk_size, torch.randint(100, 140, (12000,)).numpy(), chunk_size,
        index="index")


def test_u8_full_alphabet_with_index(emu):
    torch.manual_seed(1)
    _u8(emu, "ix_uniform256", torch.randint(0, 256, (8000,)).numpy(), 256, index="index")


def test_u8_escape_blocks_beyond_the_lds_share_with_index(emu):
    _u8(emu, "ix_escapes", many_escape_windows(seed=5, n=30000), 4096, index="index")


def test_u8_tiny_packed_buffer_with_index(emu):
    _u8(emu, "ix_tiny", np.array([7, 7, 7], np.uint8), 64, index="index")


@full
def test_u8_index_built_where_every_guess_is_wrong(emu):
    rng = np.random.default_rng(8)
    _u8(emu, "ix_guess", rng.integers(0, 8, 6000), 65536, index="index")


@full
def test_bf16_vector_path_with_index(emu):
    torch.manual_seed(2)
    _bf16(emu, "ix_bf16_vec", (torch.randn(256, 1024) * 0.02).to(torch.bfloat16), 4096,
          index="index")


@full
def test_bf16_scalar_path_ragged_with_index(emu):
    torch.manual_seed(4)
    _bf16(emu, "ix_bf16_ragged", (torch.randn(300, 333) * 0.02).to(torch.bfloat16), 1000,
          index="index")


@full
def test_bf16_two_round_64k_chunks_with_index(emu):
    W = workloads.bf16_normal((64, 17408), 2, 0.02, outlier_frac=1e-3)
    _bf16(emu, "ix_bf16_64k", W, 65536, index="index")


@pytest.mark.parametrize("mode", ["index-small", "index-foreign"])
def test_unusable_index_is_ignored(emu, mode):
    W = workloads.bf16_normal((40, 5000), 6, 0.02, outlier_frac=1e-3)
    _bf16(emu, "ix_%s" % mode, W, 4096, index=mode)


@pytest.mark.parametrize("batch", [1, 4])
def test_gemv_with_index(emu, batch):
    _gemv(emu, "ix_gemv512_b%d" % batch, 70, 1000, 32768, batch, 5, index="index")


@full
def test_gemv_16_thread_chunks_with_index(emu):
    _gemv(emu, "ix_gemv16", 96, 40, 64, 2, 3, index="index")


@full
@pytest.mark.parametrize("strided", ["1", "0"])
def test_bf16_segment_runs_cross_chunk_and_workgroup_boundaries(emu, strided):
    # 1024-symbol chunks over 768K weights: about 20 segments of 168 bits a
    # chunk, and the launch's 24 rounds on a 4-CU grid of 8 workgroups, 3
    # rounds each (strided: rounds in turn; "0": a contiguous range of rounds
    # per workgroup, the partial group carried from round to round), so
    # rounds start and end inside chunks and inside vector groups, and each
    # workgroup goes from round to round.
    W = workloads.bf16_normal((96, 8192), 12, 0.02, outlier_frac=1e-3)
    _bf16(emu, "ix_runs1024_s%s" % strided, W, 1024, index="index", strided=strided, cus=4)


@full
@pytest.mark.parametrize("strided", ["1", "0"])
def test_bf16_segment_runs_of_several_tensors_in_one_launch(emu, strided):
    # The tensor three times in one launch on a 4-CU grid: each workgroup
    # takes rounds of every copy (a piece per tensor), in turn or as
    # contiguous ranges that cross tensor boundaries.
    W = workloads.bf16_normal((48, 8192), 19, 0.02, outlier_frac=1e-3)
    _bf16(emu, "ix_runs_multi_s%s" % strided, W, 1024, index="index", strided=strided, cus=4,
          copies=3)


@full
def test_u8_segment_runs_of_a_ragged_tensor(emu):
    # The last chunk holds 700 of its 2048 symbols; a 2-CU grid of 4
    # workgroups takes several rounds each.
    rng = np.random.default_rng(13)
    _u8(emu, "ix_runs_ragged", rng.integers(90, 135, 2048 * 150 + 700), 2048, index="index",
        cus=2)


@full
def test_gemv_segment_runs_at_chunk_1024(emu):
    # A 2-CU grid: each workgroup's contiguous range holds several rounds.
    _gemv(emu, "ix_gemv1024", 128, 2048, 1024, 2, 14, index="index", cus=2)


@full
def test_unusable_index_fallback_over_several_workgroups(emu):
    W = workloads.bf16_normal((96, 8192), 15, 0.02, outlier_frac=1e-3)
    _bf16(emu, "ix_fallback_many", W, 1024, index="index-foreign", cus=2)


# The same tensors with AIMG_SEGMENT_RUNS=0, which decodes every tensor chunk
# by chunk and ignores its index, and with =1 (segment runs, the default).

@full
@pytest.mark.parametrize("runs", ["0", "1"])
def test_bf16_two_round_64k_chunks_with_index_both_paths(emu, runs):
    W = workloads.bf16_normal((64, 17408), 2, 0.02, outlier_frac=1e-3)
    _bf16(emu, "ix_64k_paths%s" % runs, W, 65536, index="index", runs=runs)


@full
@pytest.mark.parametrize("runs", ["0", "1"])
def test_bf16_1024_chunks_with_index_both_paths(emu, runs):
    W = workloads.bf16_normal((48, 8192), 18, 0.02, outlier_frac=1e-3)
    _bf16(emu, "ix_1024_paths%s" % runs, W, 1024, index="index", runs=runs, cus=2)


def test_gemv_with_index_ignored_chunk_by_chunk(emu):
    _gemv(emu, "ix_gemv512_items", 70, 1000, 32768, 4, 5, index="index", runs="0")


@full
def test_foreign_index_ignored_chunk_by_chunk(emu):
    W = workloads.bf16_normal((40, 5000), 6, 0.02, outlier_frac=1e-3)
    _bf16(emu, "ix_foreign_items", W, 4096, index="index-foreign", runs="0")


# Speculative segment runs (no index): tensors whose chunks hold 1024 symbols
# or more decode in rounds of 512 segments across chunk boundaries over a
# contiguous chunk range per workgroup. Small CU counts give each workgroup
# many rounds (and, on a full grid, workgroups b and b + grid/2 split a CU's
# share), so rounds start inside chunks, carry codeword ranks and partial
# vector groups, and switch table sets; "0" decodes the same inputs chunk by
# chunk.

@full
@pytest.mark.parametrize("spec", ["1", "0"])
def test_spec_runs_bf16_1024_chunks_many_rounds(emu, spec):
    W = workloads.bf16_normal((96, 8192), 21, 0.02, outlier_frac=1e-3)
    _bf16(emu, "sp1024_%s" % spec, W, 1024, cus=2, spec=spec)


@full
def test_spec_runs_u8_share_above_a_round_table(emu):
    # One tensor of 1100 1024-symbol chunks on one CU: the share is more
    # chunks than a workgroup has threads, so the two workgroups split it at
    # its middle chunk instead of by segment counts.
    rng = np.random.default_rng(27)
    _u8(emu, "sp_wide", rng.integers(90, 135, 1024 * 1100), 1024, cus=1)


def test_spec_runs_shares_of_two_or_three_chunks(emu):
    # 16 and 17 chunks on 8 CUs (a full grid of 16 workgroups): CU shares of
    # two chunks and of three, the smallest a full grid has.
    W = workloads.bf16_normal((16, 1024), 28, 0.02, outlier_frac=1e-2)
    _bf16(emu, "sp_two", W, 1024, cus=8)
    W = workloads.bf16_normal((17, 1024), 29, 0.02, outlier_frac=1e-2)
    _bf16(emu, "sp_three", W, 1024, cus=8)


def test_spec_runs_bf16_64k_chunks_across_chunk_boundaries(emu):
    # 6 chunks of 65536 on a 2-CU grid, forced into speculative runs (such
    # chunks decode chunk by chunk unless forced): rounds of a workgroup
    # cross from one large chunk into the next.
    W = workloads.bf16_normal((24, 16384), 22, 0.02, outlier_frac=1e-3)
    _bf16(emu, "sp64k", W, 65536, cus=2, spec="1")


@full
def test_spec_runs_several_tensors_in_one_launch(emu):
    W = workloads.bf16_normal((48, 8192), 23, 0.02, outlier_frac=1e-3)
    _bf16(emu, "sp_multi", W, 2048, cus=2, copies=3)


@full
def test_spec_runs_u8_ragged_last_chunk(emu):
    rng = np.random.default_rng(24)
    _u8(emu, "sp_ragged", rng.integers(90, 135, 2048 * 150 + 700), 2048, cus=2)


def test_spec_runs_u8_one_bit_codes(emu):
    # Two symbols: 1-bit codes, 80-bit segments, 13 segments a 1024-symbol chunk.
    rng = np.random.default_rng(25)
    _u8(emu, "sp_onebit", rng.integers(0, 2, 1024 * 90 + 33), 1024, cus=2)


@full
def test_spec_runs_every_guess_wrong(emu):
    # 3-bit fixed-length codes: every speculative start is wrong, the result
    # rests on the re-decodes from the predecessors' ends.
    rng = np.random.default_rng(26)
    _u8(emu, "sp_guess1024", rng.integers(0, 8, 1024 * 12), 1024, cus=2)
    _u8(emu, "sp_guess4k", rng.integers(0, 8, 4096 * 8 + 300), 4096, cus=2, spec="1")


def test_spec_runs_escape_blocks_beyond_the_lds_share(emu):
    _u8(emu, "sp_escapes", many_escape_windows(seed=27, n=60000), 4096, cus=2)


@full
@pytest.mark.parametrize("batch", [1, 4])
def test_spec_runs_gemv(emu, batch):
    _gemv(emu, "sp_gemv1024_b%d" % batch, 128, 2048, 1024, batch, 28, cus=2)
    _gemv(emu, "sp_gemv32k_b%d" % batch, 70, 1000, 32768, batch, 29, cus=2, spec="1")


def test_spec_runs_sliced_stream(emu):
    # Whole-chunk decode of chunks [3, 40) of a stream: the slice's own
    # n_symbols, and 8 slack bytes past its last chunk.
    from afterimage_amd.runtime.compressed_store import _slice_encoded
    rng = np.random.default_rng(30)
    exps = rng.integers(100, 130, 1024 * 48)
    enc = encode_chunked(torch.as_tensor(exps), chunk_size=1024)
    sub = _slice_encoded(enc, 3, 40)
    _write(emu[1] / "sp_slice", sub, exps[3 * 1024: 40 * 1024].astype(np.uint8))
    _run(emu, "sp_slice", "u8", cus=2)


class _Enc:
    """A ChunkedEncoded's fields, for encodings edited by hand."""

    def __init__(self, enc, **kw):
        for k in ("packed", "chunk_offsets", "chunk_nbytes", "sym_lut", "len_lut", "max_bits",
                  "chunk_size", "n_symbols"):
            setattr(self, k, kw.get(k, getattr(enc, k)))

    @property
    def n_chunks(self):
        return len(self.chunk_offsets)


def _malformed(emu, name, enc):
    # On a 2-CU grid (workgroups of several chunks fall back to the exact
    # path when one of their chunks is short) and one chunk per workgroup
    # (the chunks that hold their output count decode speculatively).
    import oracle
    want = oracle.decode_chunks(enc)[: int(enc.n_symbols)]
    _write(emu[1] / name, enc, want.astype(np.uint8))
    _run(emu, name, "u8", cus=2)
    _run(emu, name, "u8", cus=12)
    _run(emu, name, "u8", cus=2, spec="0")


@full
def test_spec_runs_truncated_chunks_take_the_exact_path(emu):
    # Chunks cut short (the bounded reader reads zeros past their end): a
    # chunk in the middle (the chunks are then not back to back) and the last
    # chunk (its codewords run out before its output count).
    rng = np.random.default_rng(31)
    enc = encode_chunked(torch.as_tensor(rng.integers(100, 140, 1024 * 24)), chunk_size=1024)
    nb = np.array(enc.chunk_nbytes, np.int32)
    nb[11] -= 40
    _malformed(emu, "sp_trunc_mid", _Enc(enc, chunk_nbytes=nb))
    nb = np.array(enc.chunk_nbytes, np.int32)
    nb[-1] -= 60
    _malformed(emu, "sp_trunc_last", _Enc(enc, chunk_nbytes=nb))


@full
def test_spec_runs_last_codeword_cut_by_the_chunk_end(emu):
    # Each chunk loses its last byte but the chunks stay back to back (the
    # stream is re-packed): codewords that run past a chunk's end read zeros
    # there, not the next chunk's bits (about half the chunks still hold
    # their output count and decode speculatively, the last window cleared
    # past the chunk end; without that, bytes of the output differ).
    rng = np.random.default_rng(32)
    enc = encode_chunked(torch.as_tensor(rng.integers(100, 140, 1024 * 24)), chunk_size=1024)
    packed = np.asarray(enc.packed, np.uint8)
    offs = np.asarray(enc.chunk_offsets, np.int64)
    nb = np.asarray(enc.chunk_nbytes, np.int64) - 1
    parts = [packed[o: o + n] for o, n in zip(offs, nb)]
    new_off = np.concatenate([[0], np.cumsum(nb)[:-1]]).astype(np.int32)
    new_packed = np.concatenate(parts + [np.zeros(8, np.uint8)])
    _malformed(emu, "sp_cut", _Enc(enc, packed=new_packed, chunk_offsets=new_off,
                                   chunk_nbytes=nb.astype(np.int32)))


@full
def test_spec_runs_chunks_out_of_order_and_empty(emu):
    rng = np.random.default_rng(33)
    enc = encode_chunked(torch.as_tensor(rng.integers(100, 140, 1024 * 20)), chunk_size=1024)
    offs = np.array(enc.chunk_offsets, np.int32)
    nb = np.array(enc.chunk_nbytes, np.int32)
    offs[[5, 6]] = offs[[6, 5]]
    nb[[5, 6]] = nb[[6, 5]]
    _malformed(emu, "sp_order", _Enc(enc, chunk_offsets=offs, chunk_nbytes=nb))
    nb = np.array(enc.chunk_nbytes, np.int32)
    nb[9] = 0
    _malformed(emu, "sp_empty", _Enc(enc, chunk_nbytes=nb))


# Fused decode -> GEMM on the matrix cores (speculative runs, pieces of a
# round written to LDS as bf16, 16-row tiles summed across waves when the
# tile changes): several x rows, rows of W longer and shorter than a piece's
# padding threshold, a last 32-column slice cut short (cols % 32 != 0), tiles
# that continue across rounds and workgroups (2 CUs), and 64Ki-symbol chunks.

@pytest.mark.parametrize("rows,cols,chunk,n_x", [
    (70, 1024, 1024, 5),
    (40, 5120, 4096, 16),
    (300, 200, 1024, 8),
    (24, 16384, 65536, 3),
])
def test_fused_gemm(emu, rows, cols, chunk, n_x):
    _gemv(emu, "gemm_%d_%d_%d_%d" % (rows, cols, chunk, n_x), rows, cols, chunk, n_x, 40 + n_x,
          cus=2, mode="gemm")
