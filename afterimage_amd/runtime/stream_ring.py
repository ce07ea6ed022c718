"""Streamed decoder blocks: compressed blocks in pinned host memory, copied to
the GPU on a side stream while the previous block decodes on the compute
stream, through a double-buffered ring under a VRAM budget.

This is the hot loop of the reference's streamed-layer engine
(streaming_engine.py:1743-1846: load layer, decompress each tensor, run it),
whose copies are synchronous and pageable (gpu_decode_v2.py:97-99,
compressed_store.py:222, :236). Here one block is one host buffer, one
asynchronous H2D copy and one decode launch.

    ring = LayerRing([block_a, block_b], device="cuda")
    for k, tensors in ring.stream(n_layers):   # tensors: bf16, on the GPU
        ...                                       # use them on the current stream
"""
from __future__ import annotations

import dataclasses

import numpy as np
import torch

from .compressed_store import CompressedLayer
from .device import TABLES, DeviceTensor, decode_bf16

ALIGN = 256  # byte alignment of every array inside a block buffer


def _aligned(n: int) -> int:
    return (n + ALIGN - 1) // ALIGN * ALIGN


@dataclasses.dataclass(frozen=True)
class TensorLayout:
    """Where one tensor's compressed arrays sit inside its block's buffer."""

    packed: tuple[int, int]         # (byte offset, byte count)
    chunk_offsets: tuple[int, int]  # (byte offset, entries), int32
    chunk_nbytes: tuple[int, int]   # (byte offset, entries), int32
    sign_mantissa: tuple[int, int]  # (byte offset, byte count)
    chunk_size: int
    n_symbols: int
    shape: tuple[int, ...]
    sym_lut: np.ndarray
    len_lut: np.ndarray
    max_bits: int


@dataclasses.dataclass(frozen=True)
class BlockPlan:
    """Byte positions of a block's arrays in its buffer: per tensor
    (sign_mantissa, packed, chunk_offsets, chunk_nbytes). Each tensor's
    sign/mantissa bytes start ALIGN-aligned with its bitstream right after
    them, and its chunk offsets start ALIGN-aligned with the lengths right
    after them, so that a store reader fills each pair with one read."""

    spans: tuple
    sizes: tuple  # (sign_mantissa bytes, packed bytes, chunks) per tensor
    nbytes: int


class HostBlock:
    """One decoder block's compressed tensors packed into one pinned host
    buffer (a single H2D copy per block)."""

    def __init__(self, layers: list[CompressedLayer], pin: bool = True):
        arrays = []
        for layer in layers:
            enc = layer.encoded
            arrays.append((np.ascontiguousarray(layer.sign_mantissa.numpy(), dtype=np.uint8),
                           np.ascontiguousarray(enc.packed, dtype=np.uint8),
                           np.ascontiguousarray(enc.chunk_offsets, dtype=np.int32),
                           np.ascontiguousarray(enc.chunk_nbytes, dtype=np.int32)))
        plan = self.plan([(a[0].nbytes, a[1].nbytes, a[2].shape[0]) for a in arrays])
        self._init_buffer(plan, pin)
        host = self.buf.numpy()
        for span, group in zip(plan.spans, arrays):
            for at, a in zip(span, group):
                host[at: at + a.nbytes] = a.reshape(-1).view(np.uint8)
        self.describe([(int(l.encoded.chunk_size), int(l.encoded.n_symbols), tuple(l.shape))
                       for l in layers],
                      [(l.encoded.sym_lut, l.encoded.len_lut, int(l.encoded.max_bits))
                       for l in layers])

    @staticmethod
    def plan(sizes: list[tuple[int, int, int]]) -> BlockPlan:
        """Layout for tensors of (sign/mantissa bytes, packed bytes, chunks)."""
        spans = []
        pos = 0
        for n_sm, n_packed, n_chunks in sizes:
            sm_at = pos
            packed_at = sm_at + n_sm
            offs_at = _aligned(packed_at + n_packed)
            nbytes_at = offs_at + 4 * n_chunks
            pos = _aligned(nbytes_at + 4 * n_chunks)
            spans.append((sm_at, packed_at, offs_at, nbytes_at))
        return BlockPlan(spans=tuple(spans), sizes=tuple(tuple(x) for x in sizes),
                         nbytes=max(pos, ALIGN))

    @classmethod
    def allocate(cls, plan: BlockPlan, pin: bool = True) -> "HostBlock":
        """An empty block with ``plan``'s buffer, to be filled (for example by
        a store reader) and then described."""
        self = cls.__new__(cls)
        self._init_buffer(plan, pin)
        return self

    def _init_buffer(self, plan: BlockPlan, pin: bool) -> None:
        self.plan_ = plan
        self.nbytes = plan.nbytes
        self.buf = torch.empty(self.nbytes, dtype=torch.uint8, pin_memory=pin)

    def describe(self, metas: list[tuple[int, int, tuple]], luts: list) -> None:
        """Record each tensor's (chunk_size, n_symbols, shape) and LUTs
        (sym_lut, len_lut, max_bits) against the buffer layout."""
        layout = []
        for span, size, (chunk_size, n_symbols, shape), (sym, ln, mb) in zip(
                self.plan_.spans, self.plan_.sizes, metas, luts):
            sm_at, packed_at, offs_at, nbytes_at = span
            n_sm, n_packed, n_chunks = size
            layout.append(TensorLayout(
                packed=(packed_at, n_packed), chunk_offsets=(offs_at, n_chunks),
                chunk_nbytes=(nbytes_at, n_chunks), sign_mantissa=(sm_at, n_sm),
                chunk_size=int(chunk_size), n_symbols=int(n_symbols), shape=tuple(shape),
                sym_lut=sym, len_lut=ln, max_bits=int(mb)))
        self.layout = layout

    @property
    def decoded_nbytes(self) -> int:
        """Bytes of the decoded bf16 tensors, each starting 16-byte aligned."""
        return 2 * sum(_out_span(t.n_symbols) for t in self.layout)


def _out_span(n: int) -> int:
    return (n + 7) // 8 * 8  # elements, so the next tensor starts 16-byte aligned


def _device_tensors(slot: torch.Tensor, block: HostBlock, tables) -> list[DeviceTensor]:
    out = []
    for t, tb in zip(block.layout, tables):
        p0, pn = t.packed
        o0, on = t.chunk_offsets
        b0, bn = t.chunk_nbytes
        s0, sn = t.sign_mantissa
        out.append(DeviceTensor(
            packed=slot[p0:p0 + pn],
            chunk_offsets=slot[o0:o0 + 4 * on].view(torch.int32),
            chunk_nbytes=slot[b0:b0 + 4 * bn].view(torch.int32),
            sign_mantissa=slot[s0:s0 + sn],
            tables=tb,
            chunk_size=t.chunk_size, n_symbols=t.n_symbols, shape=t.shape))
    return out


class LayerRing:
    """Double-buffered ring: slot k % slots receives block k's compressed bytes
    on a copy stream while block k - 1 decodes on the compute stream. Each
    slot has its own decoded-output buffer. Ring memory (compressed slots plus
    decoded outputs) must fit ``vram_budget`` bytes."""

    def __init__(self, blocks: list[HostBlock], device="cuda", slots: int = 2,
                 vram_budget: int = 4 << 30):
        if not blocks:
            raise ValueError("LayerRing needs at least one block")
        if slots < 2:
            raise ValueError("a ring needs at least 2 slots to overlap copy and decode")
        dev = torch.device(device)
        if dev.type != "cuda":
            raise RuntimeError("LayerRing streams to a GPU; got %s" % dev)
        if dev.index is None:
            dev = torch.device("cuda", torch.cuda.current_device())
        self.device = dev
        self.blocks = blocks
        self.slots = slots
        slot_bytes = max(b.nbytes for b in blocks)
        out_bytes = max(b.decoded_nbytes for b in blocks)
        self.ring_bytes = slots * (slot_bytes + out_bytes)
        if self.ring_bytes > vram_budget:
            raise ValueError("ring needs %.2f GB of device memory, budget %.2f GB"
                             % (self.ring_bytes / 1e9, vram_budget / 1e9))
        self._slot = [torch.empty(slot_bytes, dtype=torch.uint8, device=dev) for _ in range(slots)]
        self._out = [torch.empty(out_bytes // 2, dtype=torch.bfloat16, device=dev)
                     for _ in range(slots)]
        # Device decode tables, one per codebook, resolved once per block.
        self._tables = [[TABLES.get(t.sym_lut, t.len_lut, t.max_bits, dev) for t in b.layout]
                        for b in blocks]
        self.copy_stream = torch.cuda.Stream(dev)  # default priority
        self._copied = [torch.cuda.Event() for _ in range(slots)]
        self._decoded = [torch.cuda.Event() for _ in range(slots)]
        # Per-layer timing (enable_timing events) for decode-only rates.
        self.timing = False

    def _outputs(self, j: int, block: HostBlock) -> list[torch.Tensor]:
        outs = []
        pos = 0
        for t in block.layout:
            outs.append(self._out[j][pos:pos + t.n_symbols])
            pos += _out_span(t.n_symbols)
        return outs

    def _copy(self, k: int) -> None:
        j = k % self.slots
        block = self.blocks[k % len(self.blocks)]
        with torch.cuda.stream(self.copy_stream):
            # The slot's previous block must be decoded before it is overwritten.
            self.copy_stream.wait_event(self._decoded[j])
            self._slot[j][: block.nbytes].copy_(block.buf, non_blocking=True)
            self._copied[j].record(self.copy_stream)

    def stream(self, n_layers: int):
        """Yield (k, [bf16 tensors of block k % len(blocks), shaped]) for k <
        n_layers. Tensors are on the current stream's timeline: work the caller
        queues on that stream before asking for the next layer is ordered
        before the slot is reused."""
        comp = torch.cuda.current_stream(self.device)
        for j in range(self.slots):
            self._decoded[j].record(comp)  # slots start free
        self.decode_events = []
        ahead = min(self.slots - 1, n_layers)
        for k in range(ahead):
            self._copy(k)
        for k in range(n_layers):
            if k + ahead < n_layers:
                self._copy(k + ahead)
            j = k % self.slots
            block = self.blocks[k % len(self.blocks)]
            comp.wait_event(self._copied[j])
            dts = _device_tensors(self._slot[j], block, self._tables[k % len(self.blocks)])
            outs = self._outputs(j, block)
            if self.timing:
                e0 = torch.cuda.Event(enable_timing=True)
                e1 = torch.cuda.Event(enable_timing=True)
                e0.record(comp)
            decode_bf16(dts, outs)
            if self.timing:
                e1.record(comp)
                self.decode_events.append((e0, e1))
            yield k, [o.view(t.shape) for o, t in zip(outs, block.layout)]
            # Whatever the caller queued on the compute stream is ordered
            # before the slot's next copy.
            self._decoded[j].record(comp)
