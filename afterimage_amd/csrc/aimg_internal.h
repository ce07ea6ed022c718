// Layout shared by the host table builder and the gfx950 kernels.
#ifndef AIMG_INTERNAL_H
#define AIMG_INTERNAL_H

#include <cstddef>
#include <cstdint>
#include <string>

namespace aimg {

constexpr int kAbiVersion = 9;
constexpr uint32_t kTableMagic = 0x474D4941u;  // "AIMG"

// Window table: for each 12-bit window, the codewords that lie wholly inside
// it when read one after another from its first bit (at most
// kMaxSymsPerWindow), in two arrays:
//   syms (uint32): the symbols, symbol j in bits 8j..8j+7 (unused bytes zero)
//   meta (uint8):  bits 0..4 total bits those codewords take (at most 12),
//                  bits 5..7 their number (1..4)
// Meta 0 marks an escape window, whose first codeword is longer than 12
// bits or unused; its syms entry then holds the index of its escape block,
// or kUnusedBlock when the stored LUT has no codeword there.
// A 256-entry table gives each symbol's code length (every symbol of the
// stored LUT has one length), from which the codeword boundaries inside a
// window are rebuilt where a segment ends.
constexpr int kWinBits = 12;
constexpr int kWinEntries = 1 << kWinBits;
constexpr int kMaxSymsPerWindow = 4;
constexpr uint32_t kUnusedBlock = 0xFFFFu;

// Escape blocks: 16 entries of 16 bits (symbol | length << 8), indexed by
// the 4 bits that follow the 12-bit window (codewords of 13..16 bits).
constexpr int kEscBlockEntries = 16;
// A byte alphabet has at most 256 codewords, hence at most 256 windows
// whose first codeword is longer than 12 bits.
constexpr int kMaxEscBlocks = 256;

struct TableHeader {
    uint32_t magic;
    uint32_t version;
    uint32_t max_bits;      // width of the stored LUT
    uint32_t min_len;       // shortest code length (>= 1)
    uint32_t sym0;          // sym_lut[0]: what an all-zero window decodes to
    uint32_t len0;          // len_lut[0]
    uint32_t n_esc_blocks;  // escape blocks that follow the window table
    uint32_t checksum;      // FNV-1a of every byte after the header
    uint32_t reserved[8];
};
static_assert(sizeof(TableHeader) == 64, "header is 64 bytes");

constexpr size_t kSymsOffset = 64;
constexpr size_t kMetaOffset = kSymsOffset + sizeof(uint32_t) * kWinEntries;
constexpr size_t kLenOffset = kMetaOffset + sizeof(uint8_t) * kWinEntries;
constexpr size_t kEscOffset = kLenOffset + 256;

// Fixed blob size: room for the largest possible escape-block count.
inline size_t table_nbytes() {
    return kEscOffset + sizeof(uint16_t) * kEscBlockEntries * kMaxEscBlocks;
}

// Segment index of one tensor (aimg_build_index): for every segment of
// seg_bits bits of every chunk (segment k of chunk c covers chunk bits
// [k * seg_bits, (k + 1) * seg_bits)), the first codeword boundary at or
// after the segment start, as an offset 0..15 from it, and the number of
// codewords that start inside the segment, in one uint16:
//   offset | count << 4.
// Layout: the header, uint32 base[n_chunks + 1] (entry of segment 0 of
// chunk c; base[n_chunks] = entries used), then uint16 entries[capacity].
// seg_bits and the table checksum tie the index to the table it was built
// with; ok is 1 when every chunk's entries fit the capacity.
constexpr uint32_t kIndexMagic = 0x58444941u;  // "AIDX"

struct IndexHeader {
    uint32_t magic;
    uint32_t version;
    uint32_t seg_bits;
    uint32_t table_checksum;
    uint32_t ok;
    uint32_t n_chunks;
    uint32_t capacity;  // entries
    uint32_t reserved[9];
};
static_assert(sizeof(IndexHeader) == 64, "index header is 64 bytes");

// Offset of the entries of an index over n_chunks chunks (16-byte aligned).
constexpr size_t index_entries_offset(int64_t n_chunks) {
    return (sizeof(IndexHeader) + sizeof(uint32_t) * static_cast<size_t>(n_chunks + 1) + 15) &
           ~static_cast<size_t>(15);
}

// Segment length for a code whose shortest codeword has min_len bits: at
// most kSegCodewords codewords start in a segment, and it is at most
// kMaxSegBits bits and a whole number of bytes.
constexpr uint32_t kSegCodewords = 84;
constexpr uint32_t kMaxSegBits = 168;
constexpr uint32_t segment_bits(uint32_t min_len) {
    const uint32_t s = kSegCodewords * (min_len >= 1 ? min_len : 1u);
    return (s < kMaxSegBits ? s : kMaxSegBits) & ~7u;
}

int fail(int code, const std::string& msg);

}  // namespace aimg

#endif  // AIMG_INTERNAL_H
