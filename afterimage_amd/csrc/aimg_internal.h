// Layout shared by the host table builder and the gfx950 kernels.
#ifndef AIMG_INTERNAL_H
#define AIMG_INTERNAL_H

#include <cstddef>
#include <cstdint>
#include <string>

namespace aimg {

constexpr int kAbiVersion = 1;
constexpr uint32_t kTableMagic = 0x474D4941u;  // "AIMG"

// Window table: 2^kWinBits entries of 64 bits, each
//   bits  0..12  boundary mask (bit k: a codeword boundary at bit offset k)
//   bits 16..63  up to kMaxSymsPerWindow symbols, symbol j in bits 16+8j..23+8j
constexpr int kWinBits = 12;
constexpr int kWinEntries = 1 << kWinBits;
constexpr int kMaxSymsPerWindow = 6;

struct TableHeader {
    uint32_t magic;
    uint32_t version;
    uint32_t max_bits;      // width of the stored LUT
    uint32_t min_len;       // shortest code length (>= 1)
    uint32_t sym0;          // sym_lut[0]: what an all-zero window decodes to
    uint32_t len0;          // len_lut[0]
    uint32_t glut_entries;  // 2^max_bits
    uint32_t reserved[9];
};
static_assert(sizeof(TableHeader) == 64, "header is 64 bytes");

constexpr size_t kWinOffset = 64;
constexpr size_t kGlutOffset = kWinOffset + sizeof(uint64_t) * kWinEntries;

inline size_t table_nbytes(int max_bits) {
    return kGlutOffset + sizeof(uint16_t) * (size_t(1) << max_bits);
}

int fail(int code, const std::string& msg);

}  // namespace aimg

#endif  // AIMG_INTERNAL_H
