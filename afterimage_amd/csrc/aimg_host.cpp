// Host half of libafterimage_decode: decode-table construction, the chunk
// packer, and the thread-local error channel shared with aimg_decode.hip.
#include <cstdint>
#include <cstring>
#include <string>

#include "afterimage_decode.h"
#include "aimg_internal.h"

namespace aimg {

static thread_local std::string g_last_error;

int fail(int code, const std::string& msg) {
    g_last_error = msg;
    return code;
}

}  // namespace aimg

using aimg::fail;

extern "C" int aimg_abi_version(void) { return aimg::kAbiVersion; }

extern "C" const char* aimg_last_error(void) { return aimg::g_last_error.c_str(); }

extern "C" int aimg_table_nbytes(int max_bits, size_t* nbytes) {
    if (nbytes == nullptr) return fail(AIMG_ERR_INVALID_ARGUMENT, "nbytes is null");
    if (max_bits < 1 || max_bits > 16)
        return fail(AIMG_ERR_INVALID_ARGUMENT,
                    "max_bits must be in 1..16, got " + std::to_string(max_bits));
    *nbytes = aimg::table_nbytes();
    return AIMG_OK;
}

// The stored LUT is the flat table of build_decode_lut (huffman.py:128-150):
// entry i holds the symbol and code length of the codeword that the
// max_bits-wide window i starts with, replicated over every window sharing
// that codeword's prefix; windows no codeword covers hold (0, 0).
//
// The blob derived here serves the decoder in two levels (layout in
// aimg_internal.h): a 12-bit window table listing the codewords that lie
// wholly inside each window, and 16-entry escape blocks for windows whose
// first codeword is 13..16 bits long. Reading a codeword through either level
// gives exactly the (symbol, length) that the stored LUT gives for the same
// bits, which is what the reference bit reader computes
// (huffman_chunked.py:237-244).
extern "C" int aimg_build_table(const int32_t* sym_lut, const int8_t* len_lut, int max_bits,
                                void* out, size_t out_nbytes) {
    if (sym_lut == nullptr || len_lut == nullptr || out == nullptr)
        return fail(AIMG_ERR_INVALID_ARGUMENT, "null pointer passed to aimg_build_table");
    if (max_bits < 1 || max_bits > 16)
        return fail(AIMG_ERR_INVALID_ARGUMENT,
                    "max_bits must be in 1..16, got " + std::to_string(max_bits));
    const size_t need = aimg::table_nbytes();
    if (out_nbytes < need)
        return fail(AIMG_ERR_INVALID_ARGUMENT,
                    "table buffer too small: " + std::to_string(out_nbytes) + " < " +
                        std::to_string(need));
    const uint32_t size = 1u << max_bits;

    for (uint32_t i = 0; i < size; ++i) {
        const int32_t s = sym_lut[i];
        const int32_t l = len_lut[i];
        if (s < 0 || s > 255)
            return fail(AIMG_ERR_BAD_TABLE,
                        "decoder output is uint8; symbol alphabet must fit in a byte "
                        "(sym_lut[" + std::to_string(i) + "] = " + std::to_string(s) + ")");
        if (l < 0 || l > max_bits)
            return fail(AIMG_ERR_BAD_TABLE, "len_lut[" + std::to_string(i) + "] = " +
                                                std::to_string(l) + " is outside 0..max_bits");
    }
    // Walk the spans: an entry of length l starts an aligned run of
    // 2^(max_bits - l) identical entries (the windows sharing its prefix).
    uint32_t min_len = 0;
    uint8_t len_of[256] = {0};
    for (uint32_t i = 0; i < size;) {
        const uint32_t l = static_cast<uint32_t>(len_lut[i]);
        if (l == 0) {
            ++i;
            continue;
        }
        const uint32_t span = 1u << (max_bits - l);
        if (i % span != 0)
            return fail(AIMG_ERR_BAD_TABLE, "LUT entry " + std::to_string(i) +
                                                " starts a misaligned prefix span "
                                                "(not a prefix-code LUT)");
        for (uint32_t j = i + 1; j < i + span; ++j)
            if (sym_lut[j] != sym_lut[i] || len_lut[j] != len_lut[i])
                return fail(AIMG_ERR_BAD_TABLE,
                            "LUT entry " + std::to_string(j) +
                                " breaks the prefix span of entry " + std::to_string(i) +
                                " (not a prefix-code LUT)");
        if (min_len == 0 || l < min_len) min_len = l;
        const uint32_t sym = static_cast<uint32_t>(sym_lut[i]);
        if (len_of[sym] != 0 && len_of[sym] != l)
            return fail(AIMG_ERR_BAD_TABLE, "symbol " + std::to_string(sym) +
                                                " has codes of two lengths (a Huffman LUT "
                                                "gives each symbol one codeword)");
        len_of[sym] = static_cast<uint8_t>(l);
        i += span;
    }

    auto* blob = static_cast<uint8_t*>(out);
    std::memset(blob, 0, need);
    auto* wsyms = reinterpret_cast<uint32_t*>(blob + aimg::kSymsOffset);
    auto* wmeta = blob + aimg::kMetaOffset;
    std::memcpy(blob + aimg::kLenOffset, len_of, sizeof(len_of));
    auto* esc = reinterpret_cast<uint16_t*>(blob + aimg::kEscOffset);
    // (symbol, length) of the codeword starting at the first bit of `bits`
    // (MSB-first, zeros past the window).
    auto lut_at = [&](uint32_t bits, uint32_t* sym, uint32_t* len) {
        const uint32_t idx = bits >> (32 - max_bits);
        *sym = static_cast<uint32_t>(sym_lut[idx]) & 0xFFu;
        *len = static_cast<uint32_t>(len_lut[idx]);
    };
    uint32_t n_blocks = 0;
    for (uint32_t w = 0; w < static_cast<uint32_t>(aimg::kWinEntries); ++w) {
        const uint32_t bits = w << (32 - aimg::kWinBits);
        uint32_t pos = 0, k = 0;
        uint32_t syms = 0;
        while (k < static_cast<uint32_t>(aimg::kMaxSymsPerWindow)) {
            uint32_t s, l;
            lut_at(bits << pos, &s, &l);
            if (l == 0 || pos + l > static_cast<uint32_t>(aimg::kWinBits)) break;
            syms |= s << (8 * k);
            ++k;
            pos += l;
        }
        if (k > 0) {
            wsyms[w] = syms;
            wmeta[w] = static_cast<uint8_t>(pos | (k << 5));
            continue;
        }
        // Escape window: one entry per value of the next four bits.
        uint16_t block[aimg::kEscBlockEntries];
        bool any = false;
        for (uint32_t e4 = 0; e4 < static_cast<uint32_t>(aimg::kEscBlockEntries); ++e4) {
            uint32_t s, l;
            lut_at(bits | (e4 << (32 - aimg::kWinBits - 4)), &s, &l);
            block[e4] = static_cast<uint16_t>(s | (l << 8));
            any = any || l != 0;
        }
        wmeta[w] = 0;
        if (!any) {
            wsyms[w] = aimg::kUnusedBlock;
            continue;
        }
        if (n_blocks >= static_cast<uint32_t>(aimg::kMaxEscBlocks))
            return fail(AIMG_ERR_BAD_TABLE, "more than 256 windows start with a codeword "
                                            "longer than 12 bits");
        std::memcpy(esc + n_blocks * aimg::kEscBlockEntries, block, sizeof(block));
        wsyms[w] = n_blocks++;
    }

    aimg::TableHeader hdr{};
    hdr.magic = aimg::kTableMagic;
    hdr.version = aimg::kAbiVersion;
    hdr.max_bits = static_cast<uint32_t>(max_bits);
    hdr.min_len = min_len == 0 ? 1 : min_len;
    hdr.sym0 = static_cast<uint32_t>(sym_lut[0]);
    hdr.len0 = static_cast<uint32_t>(len_lut[0]);
    hdr.n_esc_blocks = n_blocks;
    // FNV-1a over the tables: a segment index records the checksum of the
    // table it was built with, and is used only with a table that matches.
    uint32_t h = 2166136261u;
    for (size_t k = sizeof(hdr); k < need; ++k) h = (h ^ blob[k]) * 16777619u;
    hdr.checksum = h;
    std::memcpy(blob, &hdr, sizeof(hdr));
    return AIMG_OK;
}

extern "C" int aimg_index_nbytes(const void* host_table, int64_t packed_nbytes, int32_t n_chunks,
                                 size_t* nbytes) {
    if (host_table == nullptr || nbytes == nullptr)
        return fail(AIMG_ERR_INVALID_ARGUMENT, "null pointer passed to aimg_index_nbytes");
    if (packed_nbytes < 0 || n_chunks < 0)
        return fail(AIMG_ERR_INVALID_ARGUMENT, "packed_nbytes and n_chunks must be >= 0");
    aimg::TableHeader hdr;
    std::memcpy(&hdr, host_table, sizeof(hdr));
    if (hdr.magic != aimg::kTableMagic || hdr.version != static_cast<uint32_t>(aimg::kAbiVersion))
        return fail(AIMG_ERR_BAD_TABLE, "table blob has a wrong magic or version "
                                        "(build it with aimg_build_table)");
    const aimg::IndexLayout l =
        aimg::index_layout(packed_nbytes, n_chunks, aimg::segment_bits(hdr.min_len));
    if (l.capacity >= UINT32_MAX)
        return fail(AIMG_ERR_UNSUPPORTED, "index of 2^32 - 1 or more segments");
    *nbytes = static_cast<size_t>(l.total);
    return AIMG_OK;
}

// MSB-first chunk packer with the byte layout of _pack_chunked_kernel
// (huffman_chunked.py:41-78): each chunk starts on a byte boundary, codes are
// appended most-significant bit first, and a chunk's last partial byte is
// zero-padded.
extern "C" int aimg_pack_chunked(const uint8_t* symbols, int64_t n, const uint32_t* code_of,
                                 const uint8_t* len_of, int32_t chunk_size, uint8_t* out,
                                 int64_t out_cap, int32_t* chunk_nbytes, int64_t* total) {
    if ((n > 0 && symbols == nullptr) || code_of == nullptr || len_of == nullptr ||
        chunk_nbytes == nullptr || total == nullptr || (out == nullptr && out_cap > 0))
        return fail(AIMG_ERR_INVALID_ARGUMENT, "null pointer passed to aimg_pack_chunked");
    if (n < 0 || chunk_size < 1)
        return fail(AIMG_ERR_INVALID_ARGUMENT, "n must be >= 0 and chunk_size >= 1");
    for (int s = 0; s < 256; ++s)
        if (len_of[s] > 16)
            return fail(AIMG_ERR_INVALID_ARGUMENT, "code lengths must be <= 16");
    const int64_t n_chunks = (n + chunk_size - 1) / chunk_size;
    int64_t pos = 0;
    for (int64_t c = 0; c < n_chunks; ++c) {
        const int64_t start = c * chunk_size;
        const int64_t end = start + chunk_size < n ? start + chunk_size : n;
        const int64_t cstart = pos;
        uint64_t acc = 0;  // pending bits, left-aligned at bit 63
        uint32_t nbits = 0;
        for (int64_t i = start; i < end; ++i) {
            const uint8_t s = symbols[i];
            const uint32_t ln = len_of[s];
            if (ln == 0)
                return fail(AIMG_ERR_INVALID_ARGUMENT,
                            "symbol " + std::to_string(s) + " has no code");
            acc |= static_cast<uint64_t>(code_of[s] & ((1u << ln) - 1)) << (64 - nbits - ln);
            nbits += ln;
            while (nbits >= 8) {
                if (pos >= out_cap)
                    return fail(AIMG_ERR_INVALID_ARGUMENT, "pack output buffer too small");
                out[pos++] = static_cast<uint8_t>(acc >> 56);
                acc <<= 8;
                nbits -= 8;
            }
        }
        if (nbits > 0) {
            if (pos >= out_cap)
                return fail(AIMG_ERR_INVALID_ARGUMENT, "pack output buffer too small");
            out[pos++] = static_cast<uint8_t>(acc >> 56);
        }
        const int64_t nb = pos - cstart;
        if (nb > INT32_MAX) return fail(AIMG_ERR_INVALID_ARGUMENT, "chunk exceeds 2 GiB");
        chunk_nbytes[c] = static_cast<int32_t>(nb);
    }
    *total = pos;
    return AIMG_OK;
}
