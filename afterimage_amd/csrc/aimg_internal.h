// Layout shared by the host table builder and the gfx950 kernels.
#ifndef AIMG_INTERNAL_H
#define AIMG_INTERNAL_H

#include <cstddef>
#include <cstdint>
#include <string>

namespace aimg {

constexpr int kAbiVersion = 8;
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
    uint32_t reserved[9];
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

int fail(int code, const std::string& msg);

}  // namespace aimg

#endif  // AIMG_INTERNAL_H
