"""Length-limited canonical Huffman code construction for exponent bytes.

Same interface and the same code lengths, codes and LUT as the reference codec
(afterimage/runtime/huffman.py:30-150), so stores written by either side decode
on the other:

* ``build_lengths``: plain Huffman lengths from a binary heap whose ties break
  on (frequency, insertion index); when the longest code exceeds ``max_bits``,
  package-merge (Larmore & Hirschberg 1990) over ``max_bits`` levels with
  items ordered by (weight, symbol list). Tie order decides which of several
  optimal length assignments comes out, so both orders are kept exactly.
* ``canonical_codes``: symbols sorted by (length, symbol), consecutive code
  values, shifted left whenever the length grows.
* ``build_decode_lut``: flat LUT of ``2**max_bits`` windows, each code's entry
  repeated over every window that starts with it.

Only the encoder lives here. Decoding is done on the GPU by
``libafterimage_decode``; the CPU decoders used to check it are in ``oracle/``.
"""
from __future__ import annotations

import dataclasses
import heapq

import numpy as np


@dataclasses.dataclass
class HuffmanTable:
    """Canonical code description (afterimage/runtime/huffman.py:30-38)."""

    symbols: list[int]   # symbol values in canonical order
    lengths: list[int]   # code length per entry of ``symbols``
    max_bits: int        # longest code length (the LUT width)

    @property
    def n_symbols(self) -> int:
        return len(self.symbols)


def _natural_lengths(freqs: dict[int, int]) -> dict[int, int]:
    """Huffman code length per symbol with non-zero frequency.

    Follows huffman.py:41-61: nodes are ``(weight, order, symbols)``; leaves
    take their position in ``freqs`` as order, merged nodes take increasing
    orders starting after the leaf count, and every merge adds one bit to all
    symbols under both popped nodes. A lone symbol gets a 1-bit code.
    """
    nodes = []
    for order, (sym, f) in enumerate(freqs.items()):
        if f > 0:
            nodes.append((f, order, (sym,)))
    if not nodes:
        return {}
    if len(nodes) == 1:
        return {nodes[0][2][0]: 1}
    heapq.heapify(nodes)
    depth = {sym: 0 for _, _, (sym,) in nodes}
    next_order = len(nodes)
    while len(nodes) > 1:
        w0, _, s0 = heapq.heappop(nodes)
        w1, _, s1 = heapq.heappop(nodes)
        for sym in s0 + s1:
            depth[sym] += 1
        heapq.heappush(nodes, (w0 + w1, next_order, s0 + s1))
        next_order += 1
    return depth


def _package_merge_limit(freqs: dict[int, int], max_bits: int) -> dict[int, int]:
    """Optimal code lengths bounded by ``max_bits`` (huffman.py:64-96).

    Level 0 is the leaf list; each further level is the leaves merged with the
    pairwise packages of the level below, ordered by (weight, symbol tuple).
    The cheapest ``2(n-1)`` items of the last level are chosen, and a symbol's
    length is how many times it occurs in them.
    """
    leaves = sorted((f, s) for s, f in freqs.items() if f > 0)
    n = len(leaves)
    if n == 0:
        return {}
    if n == 1:
        return {leaves[0][1]: 1}
    base = [(f, (s,)) for f, s in leaves]
    level = list(base)
    for _ in range(1, max_bits):
        pairs = [(level[i][0] + level[i + 1][0], level[i][1] + level[i + 1][1])
                 for i in range(0, len(level) - 1, 2)]
        level = sorted(base + pairs)
    length = {s: 0 for _, s in leaves}
    for _, syms in level[: 2 * (n - 1)]:
        for s in syms:
            length[s] += 1
    return length


def build_lengths(freqs: dict[int, int], max_bits: int = 16) -> dict[int, int]:
    """Huffman lengths, length-limited only when needed (huffman.py:99-103)."""
    lengths = _natural_lengths(freqs)
    if not lengths or max(lengths.values()) <= max_bits:
        return lengths
    return _package_merge_limit(freqs, max_bits)


def canonical_codes(lengths: dict[int, int]) -> tuple[HuffmanTable, dict[int, int]]:
    """Canonical code assignment (huffman.py:106-125)."""
    ordered = sorted(lengths.items(), key=lambda kv: (kv[1], kv[0]))
    symbols = [s for s, _ in ordered]
    lens = [ln for _, ln in ordered]
    codes: dict[int, int] = {}
    value = 0
    width = lens[0] if lens else 0
    for sym, ln in ordered:
        value <<= ln - width
        width = ln
        codes[sym] = value
        value += 1
    table = HuffmanTable(symbols=symbols, lengths=lens, max_bits=max(lens) if lens else 0)
    return table, codes


def build_decode_lut(table: HuffmanTable, codes: dict[int, int]) -> tuple[np.ndarray, np.ndarray]:
    """Flat decode LUT (huffman.py:128-150): int32 symbols, int8 lengths."""
    size = 1 << table.max_bits
    sym_lut = np.zeros(size, dtype=np.int32)
    len_lut = np.zeros(size, dtype=np.int8)
    for sym, ln in zip(table.symbols, table.lengths):
        shift = table.max_bits - ln
        lo = codes[sym] << shift
        sym_lut[lo: lo + (1 << shift)] = sym
        len_lut[lo: lo + (1 << shift)] = ln
    return sym_lut, len_lut


def code_arrays(codes: dict[int, int], lengths: dict[int, int]) -> tuple[np.ndarray, np.ndarray]:
    """Per-byte-symbol code value and length arrays for the native packer."""
    code_of = np.zeros(256, dtype=np.uint32)
    len_of = np.zeros(256, dtype=np.uint8)
    for s, c in codes.items():
        if not 0 <= s <= 255:
            raise ValueError("symbols must be bytes (0..255), got %d" % s)
        code_of[s] = c
        len_of[s] = lengths[s]
    return code_of, len_of
