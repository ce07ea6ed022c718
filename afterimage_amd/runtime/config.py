"""Codec settings of the reference's EngineConfig (afterimage/runtime/config.py:360-383),
with the same names, defaults and validation (config.py:412-440, :467-469), and its
is_lossless (config.py:575-580) as far as these settings decide it."""
from __future__ import annotations

import dataclasses


@dataclasses.dataclass
class CodecConfig:
    chunk_size: int = 1024
    block_chunks: int = 32
    max_bits: int = 16
    decode_slice_elems: int = 1 << 25
    reuse_decode_tables: bool = False
    # Rows of a 2-D output projection per block (decompress_linear_gpu), or 0
    # to decode the whole tensor first.
    lm_head_slice_rows: int = 0

    def __post_init__(self) -> None:
        if self.block_chunks & (self.block_chunks - 1) != 0:
            raise ValueError(
                "block_chunks must be a power of 2 (Triton tl.arange), got %d"
                % self.block_chunks)
        if not (1 <= self.max_bits <= 16):
            raise ValueError("max_bits must be in [1, 16], got %d" % self.max_bits)
        if self.chunk_size < 1:
            raise ValueError("chunk_size must be >= 1, got %d" % self.chunk_size)
        if self.decode_slice_elems < 1:
            raise ValueError("decode_slice_elems must be >= 1, got %d"
                             % self.decode_slice_elems)
        if self.lm_head_slice_rows < 0:
            raise ValueError("lm_head_slice_rows must be >= 0 (0 disables), got %d"
                             % self.lm_head_slice_rows)

    @property
    def is_lossless(self) -> bool:
        """Bit-identical outputs: a blocked output projection adds its
        blocks' products in another order than one whole product."""
        return self.lm_head_slice_rows == 0
