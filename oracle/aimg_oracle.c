/*
 * CPU oracle for the Afterimage BF16 decode path -- TEST INFRASTRUCTURE.
 *
 * Only tests/, __graft_entry__.smoke() and bench.py's CPU-baseline leg may
 * load this library, and only as the reference that the GPU decoder's
 * outputs are compared with, or as the timed CPU baseline. The product
 * (afterimage_amd) never calls it.
 *
 * Each function restates one piece of the reference algorithm:
 *   oracle_decode_chunks    bounded 32-bit MSB-aligned bit reader, one chunk
 *                           at a time, parallel over chunks with OpenMP:
 *                           afterimage/runtime/cpu_decode.py:67-113
 *                           (_decode_numba / decode_chunks_numba), which is
 *                           the same reader as ChunkedBitReader
 *                           (afterimage/runtime/huffman_chunked.py:210-267).
 *   oracle_recombine        bf16 = ((sm & 0x80) << 8) | (e << 7) | (sm & 0x7F):
 *                           afterimage/runtime/compressed_store.py:94-114.
 *   oracle_decode_bitwise   bit-by-bit canonical decode of one stream:
 *                           afterimage/runtime/huffman.py:195-217.
 *   oracle_pack_bitwise     MSB-first per-chunk packing written bit by bit:
 *                           afterimage/runtime/huffman_chunked.py:41-78,
 *                           huffman.py:153-192.
 *
 * Build: make -C oracle (gcc -O2 -fopenmp), output oracle/liboracle.so.
 */
#include <stdint.h>
#include <string.h>

#ifdef _OPENMP
#include <omp.h>
#endif

/*
 * Decode chunks [chunk_lo, chunk_hi) into out[(c - chunk_lo) * chunk_size + i],
 * i < chunk_size. Reads never leave [offset, offset + nbytes) of a chunk; bits
 * past the chunk end read as zero. Returns 0, or -1 on bad arguments.
 */
int oracle_decode_chunks(const uint8_t* packed, int64_t packed_len, const int32_t* offsets,
                         const int32_t* nbytes, int64_t chunk_lo, int64_t chunk_hi,
                         const int32_t* sym_lut, const int8_t* len_lut, int max_bits,
                         int64_t chunk_size, uint8_t* out, int n_threads) {
    if (max_bits < 1 || max_bits > 16 || chunk_size < 1 || chunk_lo < 0 || chunk_hi < chunk_lo)
        return -1;
    for (int64_t c = chunk_lo; c < chunk_hi; ++c)
        if (offsets[c] < 0 || nbytes[c] < 0 || (int64_t)offsets[c] + nbytes[c] > packed_len)
            return -1;
    const uint32_t mask = (1u << max_bits) - 1u;
#ifdef _OPENMP
    if (n_threads < 1) n_threads = omp_get_max_threads();
#pragma omp parallel for schedule(dynamic, 8) num_threads(n_threads)
#endif
    for (int64_t c = chunk_lo; c < chunk_hi; ++c) {
        int64_t pos = offsets[c];
        const int64_t end = pos + nbytes[c];
        uint32_t buf = 0;
        int32_t nbits = 0;
        uint8_t* dst = out + (c - chunk_lo) * chunk_size;
        for (int64_t i = 0; i < chunk_size; ++i) {
            while (nbits < max_bits && pos < end) {
                buf |= (uint32_t)packed[pos++] << (24 - nbits);
                nbits += 8;
            }
            const uint32_t window = (buf >> (32 - max_bits)) & mask;
            const uint32_t len = (uint32_t)(uint8_t)len_lut[window];
            dst[i] = (uint8_t)sym_lut[window];
            buf = len < 32 ? buf << len : 0u;
            nbits -= (int32_t)len;
        }
    }
    (void)n_threads;
    return 0;
}

void oracle_recombine(const uint8_t* exponent, const uint8_t* sign_mantissa, uint16_t* out,
                      int64_t n, int n_threads) {
#ifdef _OPENMP
    if (n_threads < 1) n_threads = omp_get_max_threads();
#pragma omp parallel for schedule(static) num_threads(n_threads)
#endif
    for (int64_t i = 0; i < n; ++i) {
        const uint32_t sm = sign_mantissa[i];
        out[i] = (uint16_t)(((sm & 0x80u) << 8) | ((uint32_t)exponent[i] << 7) | (sm & 0x7Fu));
    }
    (void)n_threads;
}

/*
 * Bit-by-bit decode of one MSB-first stream of n_symbols codewords, given the
 * canonical code as parallel arrays (symbol, length, code) of n_codes entries.
 * At each codeword, bits are taken one at a time and the accumulated value is
 * compared with every code of the current length. Returns 0, or the 1-based
 * index of the first symbol with no matching code (a corrupt stream).
 */
int64_t oracle_decode_bitwise(const uint8_t* packed, int64_t packed_len, const int32_t* symbols,
                              const int32_t* lengths, const uint32_t* codes, int n_codes,
                              int max_bits, int64_t n_symbols, int32_t* out) {
    int64_t bitpos = 0;
    for (int64_t i = 0; i < n_symbols; ++i) {
        uint32_t value = 0;
        int found = 0;
        for (int len = 1; len <= max_bits && !found; ++len) {
            const int64_t byte = bitpos >> 3;
            const uint32_t bit =
                byte < packed_len ? (packed[byte] >> (7 - (bitpos & 7))) & 1u : 0u;
            value = (value << 1) | bit;
            ++bitpos;
            for (int k = 0; k < n_codes; ++k) {
                if (lengths[k] == len && codes[k] == value) {
                    out[i] = symbols[k];
                    found = 1;
                    break;
                }
            }
        }
        if (!found) return i + 1;
    }
    return 0;
}

/*
 * Pack symbols chunk by chunk, one bit at a time, MSB first; each chunk
 * starts on a byte boundary and its last byte is zero-padded. Writes
 * chunk_nbytes and returns the total byte count, or -1 if out_cap is too
 * small or a symbol has no code.
 */
int64_t oracle_pack_bitwise(const uint8_t* symbols, int64_t n, const uint32_t* code_of,
                            const uint8_t* len_of, int64_t chunk_size, uint8_t* out,
                            int64_t out_cap, int32_t* chunk_nbytes) {
    int64_t byte = 0;
    const int64_t n_chunks = chunk_size > 0 ? (n + chunk_size - 1) / chunk_size : 0;
    for (int64_t c = 0; c < n_chunks; ++c) {
        const int64_t start = c * chunk_size;
        const int64_t end = start + chunk_size < n ? start + chunk_size : n;
        int64_t bit = 0;  /* bits written in this chunk */
        const int64_t first = byte;
        for (int64_t i = start; i < end; ++i) {
            const uint32_t len = len_of[symbols[i]];
            const uint32_t code = code_of[symbols[i]];
            if (len == 0) return -1;
            for (int32_t j = (int32_t)len - 1; j >= 0; --j) {
                const int64_t at = first + (bit >> 3);
                if (at >= out_cap) return -1;
                if ((bit & 7) == 0) out[at] = 0;
                out[at] |= (uint8_t)(((code >> j) & 1u) << (7 - (bit & 7)));
                ++bit;
            }
        }
        byte = first + (bit + 7) / 8;
        chunk_nbytes[c] = (int32_t)(byte - first);
    }
    return byte;
}

int oracle_max_threads(void) {
#ifdef _OPENMP
    return omp_get_max_threads();
#else
    return 1;
#endif
}
