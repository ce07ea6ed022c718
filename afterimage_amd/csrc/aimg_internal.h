// Layout shared by the host table builder and the gfx950 kernels.
#ifndef AIMG_INTERNAL_H
#define AIMG_INTERNAL_H

#include <cstddef>
#include <cstdint>
#include <string>

namespace aimg {

constexpr int kAbiVersion = 11;
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

// Segment index of one tensor (aimg_build_index). Segment k of chunk c
// covers chunk bits [k * seg_bits, (k + 1) * seg_bits); the chunk's
// segments are numbered base[c] .. base[c + 1] - 1 in one sequence over the
// tensor (its chunks that hold output elements, n_jobs of them). A
// segment's count is the number of codewords that start inside it and
// before the chunk's real end rend[c], the end of its lim-th codeword (lim:
// the chunk's output elements). Codewords past rend[c] (the zero bits that
// pad a chunk to whole bytes) are not counted, so a chunk's counts add up
// to lim and the tensor's symbols run on from chunk to chunk. The
// segments fall in rounds of 512 (segments 512 m .. 512 m + 511, across
// chunk boundaries), and each has one uint32 entry:
//   offset | jj << 4 | excl << 10
// offset: the first codeword boundary at or after the segment start, 0..15
// bits past it; jj: its chunk minus the chunk of its round's first segment
// (below 64 for chunks of 1024 symbols or more); excl: the counts of its
// round's segments before it (at most 511 * 84). While the index is built
// an entry holds offset | count << 4.
// Layout (index_layout): the header, uint32 base[n_chunks + 1] (entries
// past n_jobs repeat the total), uint32 rend[n_chunks], uint32
// entries[capacity], and RoundStart rounds[n_rounds]: where each round
// starts, and after the last round (m = ceil(n_segments / 512)) a
// sentinel whose element is the tensor's symbol count. The index is usable
// (ok == 1) only when the chunks lie back to back in the packed buffer,
// every chunk holds its lim codewords within its bytes, and everything
// fits; seg_bits and the table checksum tie it to the table it was built
// with.
constexpr uint32_t kIndexMagic = 0x32444941u;  // "AID2"

struct IndexHeader {
    uint32_t magic;
    uint32_t version;
    uint32_t seg_bits;
    uint32_t table_checksum;
    uint32_t ok;
    uint32_t n_chunks;
    uint32_t n_segments;  // base[n_jobs]: the tensor's segments
    uint32_t n_jobs;
    uint32_t reserved[8];
};
static_assert(sizeof(IndexHeader) == 64, "index header is 64 bytes");

struct IndexLayout {
    uint64_t base, rend, entries, rounds, total;
    uint64_t capacity, n_rounds;
};

// Segment 512 * m of a tensor (m < n_segments / 512): its chunk, the output
// element of its first codeword, the packed byte where its bits start, and
// the chunk's first segment.
struct RoundStart {
    uint32_t chunk;
    uint32_t element;
    uint32_t byte;
    uint32_t chunk_base;
};
static_assert(sizeof(RoundStart) == 16, "round start is 16 bytes");

// Segments between two round starts (one round of a whole workgroup).
constexpr uint32_t kIndexBlock = 512;
// Fields of a finished entry (offset in bits 0..3).
constexpr uint32_t kEntryJjShift = 4;
constexpr uint32_t kEntryExclShift = 10;

// Byte offsets of the real ends and the entries of an index over n_chunks
// chunks (they do not depend on the segment count).
constexpr uint64_t index_rend_at(int64_t n_chunks) {
    return sizeof(IndexHeader) + 4 * static_cast<uint64_t>(n_chunks > 0 ? n_chunks + 1 : 1);
}
constexpr uint64_t index_entries_at(int64_t n_chunks) {
    return (index_rend_at(n_chunks) + 4 * static_cast<uint64_t>(n_chunks > 0 ? n_chunks : 0) + 15) &
           ~uint64_t{15};
}

// Byte offsets of an index's arrays for a tensor of packed_nbytes packed
// bytes in n_chunks chunks and segments of seg_bits: room for the segments
// of chunks that lie back to back, ceil(8 * packed_nbytes / seg_bits) plus
// one partial segment per chunk.
constexpr IndexLayout index_layout(int64_t packed_nbytes, int64_t n_chunks, uint32_t seg_bits) {
    IndexLayout l{};
    const uint64_t pb = packed_nbytes > 0 ? static_cast<uint64_t>(packed_nbytes) : 0u;
    const uint64_t nc = n_chunks > 0 ? static_cast<uint64_t>(n_chunks) : 0u;
    const uint64_t s = seg_bits > 0 ? seg_bits : 1u;
    l.capacity = (8 * pb + s - 1) / s + nc;
    l.n_rounds = l.capacity / kIndexBlock + 2;
    l.base = sizeof(IndexHeader);
    l.rend = index_rend_at(n_chunks);
    l.entries = index_entries_at(n_chunks);
    l.rounds = (l.entries + 4 * l.capacity + 15) & ~uint64_t{15};
    l.total = l.rounds + sizeof(RoundStart) * l.n_rounds;
    return l;
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
