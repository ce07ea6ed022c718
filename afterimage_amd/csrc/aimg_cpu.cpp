// Host decode path of libafterimage_decode: the same chunked canonical-Huffman
// exponent decode and BF16 recombine as the gfx950 kernels, on CPU threads.
//
// It serves callers that run the engine without a GPU: the reference decodes
// on the CPU when its device is "cpu" (afterimage/runtime/compressed_store.py:
// 171-180, afterimage/runtime/cpu_decode.py:67-113, numba over chunks). Here
// each chunk is decoded sequentially through the table blob of
// aimg_build_table (a 12-bit window table giving up to four codewords per
// lookup, escape blocks for 13..16-bit codewords), so the host and the GPU
// decoders read one validated description of the code and agree on every
// input, malformed ones included: bits past a chunk's bytes read as zero, and
// bits that start no codeword decode to sym_lut[0] and take the shortest code
// length.
#include <algorithm>
#include <atomic>
#include <cstdint>
#include <cstring>
#include <string>
#include <thread>
#include <vector>

#include "afterimage_decode.h"
#include "aimg_internal.h"

namespace aimg {
namespace {

struct HostTable {
    const uint32_t* syms;
    const uint8_t* meta;
    const uint16_t* esc;
    uint32_t n_esc;
    uint32_t sym0;
    uint32_t min_len;
};

int host_table(const void* blob, HostTable* tb) {
    TableHeader hdr;
    std::memcpy(&hdr, blob, sizeof(hdr));
    if (hdr.magic != kTableMagic || hdr.version != static_cast<uint32_t>(kAbiVersion))
        return fail(AIMG_ERR_BAD_TABLE, "table blob has a wrong magic or version "
                                        "(build it with aimg_build_table)");
    if (hdr.n_esc_blocks > static_cast<uint32_t>(kMaxEscBlocks) || hdr.sym0 > 255u)
        return fail(AIMG_ERR_BAD_TABLE, "table blob header is corrupt");
    const auto* b = static_cast<const uint8_t*>(blob);
    tb->syms = reinterpret_cast<const uint32_t*>(b + kSymsOffset);
    tb->meta = b + kMetaOffset;
    tb->esc = reinterpret_cast<const uint16_t*>(b + kEscOffset);
    tb->n_esc = hdr.n_esc_blocks;
    tb->sym0 = hdr.sym0;
    tb->min_len = hdr.min_len >= 1 ? hdr.min_len : 1u;
    return AIMG_OK;
}

inline uint64_t load_be64(const uint8_t* p) {
    uint64_t v;
    std::memcpy(&v, p, 8);
    return __builtin_bswap64(v);
}

// Decode `lim` exponent symbols of one chunk whose bitstream is the nb bytes
// at p into dst (room for lim + 3 bytes: a lookup stores its four symbol
// bytes whole). The reader keeps the next bits MSB-aligned in acc, nbits of
// them valid; bits past the chunk's bytes are zero.
void decode_chunk(const HostTable& tb, const uint8_t* p, uint32_t nb, uint32_t lim,
                  uint8_t* dst) {
    uint64_t acc = 0;
    int64_t nbits = 0;
    uint32_t pos = 0;
    uint32_t k = 0;
    while (k < lim) {
        if (nbits < 16 && pos < nb) {
            if (pos + 8 <= nb) {
                // Eight whole bytes inside the chunk: OR them in below the
                // valid bits and count the bytes that fitted whole. Bits of
                // a byte that only partly fitted are the stream's own, so
                // ORing that byte in again at the next refill changes nothing.
                acc |= load_be64(p + pos) >> nbits;
                const uint32_t take = static_cast<uint32_t>(63 - nbits) >> 3;
                pos += take;
                nbits += 8 * take;
            } else {
                while (nbits <= 56 && pos < nb) {
                    acc |= static_cast<uint64_t>(p[pos++]) << (56 - nbits);
                    nbits += 8;
                }
            }
        }
        const uint32_t idx = static_cast<uint32_t>(acc >> (64 - kWinBits));
        const uint32_t m = tb.meta[idx];
        uint32_t adv;
        if (m != 0) {
            const uint32_t s = tb.syms[idx];
            std::memcpy(dst + k, &s, 4);
            k += m >> 5;
            adv = m & 31u;
        } else {
            const uint32_t blk = tb.syms[idx] & 0xFFFFu;
            uint32_t sym = tb.sym0, len = tb.min_len;
            if (blk != kUnusedBlock && blk < tb.n_esc) {
                const uint32_t v = tb.esc[blk * kEscBlockEntries +
                                          static_cast<uint32_t>((acc >> (60 - kWinBits)) & 15u)];
                if ((v >> 8) != 0) {
                    sym = v & 0xFFu;
                    len = v >> 8;
                }
            }
            dst[k++] = static_cast<uint8_t>(sym);
            adv = len;
        }
        acc <<= adv;
        nbits -= adv;
    }
}

inline uint16_t bf16_bits(uint8_t sm, uint8_t e) {
    return static_cast<uint16_t>(((sm & 0x80u) << 8) | (static_cast<uint32_t>(e) << 7) |
                                 (sm & 0x7Fu));
}

void recombine(const uint8_t* e, const uint8_t* sm, uint16_t* out, int64_t n) {
    for (int64_t i = 0; i < n; ++i) out[i] = bf16_bits(sm[i], e[i]);
}

struct HostJob {
    const aimg_tensor* t;
    HostTable tb;
    int64_t n_jobs;     // chunks holding output elements
    int64_t first;      // first unit of this tensor in the call
    int64_t per_unit;   // chunks per unit of work
};

int validate(const aimg_tensor& t, int i, bool need_sm) {
    const std::string who = "tensor " + std::to_string(i) + ": ";
    if (t.chunk_size < 1) return fail(AIMG_ERR_INVALID_ARGUMENT, who + "chunk_size must be >= 1");
    if (t.n_chunks < 0 || t.n_symbols < 0 || t.packed_nbytes < 0)
        return fail(AIMG_ERR_INVALID_ARGUMENT, who + "negative size");
    if (t.n_symbols > static_cast<int64_t>(t.n_chunks) * t.chunk_size)
        return fail(AIMG_ERR_INVALID_ARGUMENT, who + "n_symbols exceeds n_chunks * chunk_size");
    if (t.n_symbols == 0) return AIMG_OK;
    if ((t.packed == nullptr && t.packed_nbytes > 0) || t.chunk_offsets == nullptr ||
        t.chunk_nbytes == nullptr || t.out == nullptr || t.table == nullptr ||
        (need_sm && t.sign_mantissa == nullptr))
        return fail(AIMG_ERR_INVALID_ARGUMENT, who + "null pointer");
    return AIMG_OK;
}

// Decode (and, for bf16, recombine) every tensor, units of whole chunks
// handed to n_threads threads through one counter.
template <bool kBf16>
int host_decode(const aimg_tensor* ts, int n, int n_threads) {
    if (ts == nullptr && n > 0) return fail(AIMG_ERR_INVALID_ARGUMENT, "tensors is null");
    if (n < 0) return fail(AIMG_ERR_INVALID_ARGUMENT, "n_tensors must be >= 0");
    std::vector<HostJob> jobs;
    int64_t units = 0;
    int32_t max_chunk = 0;
    int64_t total_syms = 0;
    for (int i = 0; i < n; ++i) {
        const aimg_tensor& t = ts[i];
        const int rc = validate(t, i, kBf16);
        if (rc != AIMG_OK) return rc;
        if (t.n_symbols == 0) continue;
        HostJob j;
        j.t = &t;
        const int trc = host_table(t.table, &j.tb);
        if (trc != AIMG_OK) return trc;
        j.n_jobs = (t.n_symbols + t.chunk_size - 1) / t.chunk_size;
        // About 64 Ki symbols per unit: small chunks are grouped.
        j.per_unit = std::max<int64_t>(1, (int64_t{1} << 16) / t.chunk_size);
        j.first = units;
        units += (j.n_jobs + j.per_unit - 1) / j.per_unit;
        max_chunk = std::max(max_chunk, t.chunk_size);
        total_syms += t.n_symbols;
        jobs.push_back(j);
    }
    if (units == 0) return AIMG_OK;
    int threads = n_threads > 0 ? n_threads : static_cast<int>(std::thread::hardware_concurrency());
    threads = static_cast<int>(std::max<int64_t>(1, std::min<int64_t>(threads, units)));

    std::atomic<int64_t> next{0};
    auto worker = [&]() {
        std::vector<uint8_t> ebuf(static_cast<size_t>(max_chunk) + 8);
        size_t ji = 0;
        for (;;) {
            const int64_t u = next.fetch_add(1, std::memory_order_relaxed);
            if (u >= units) return;
            while (ji + 1 < jobs.size() && u >= jobs[ji + 1].first) ++ji;
            while (ji > 0 && u < jobs[ji].first) --ji;
            const HostJob& J = jobs[ji];
            const aimg_tensor& t = *J.t;
            const int64_t c0 = (u - J.first) * J.per_unit;
            const int64_t c1 = std::min(J.n_jobs, c0 + J.per_unit);
            for (int64_t c = c0; c < c1; ++c) {
                int64_t off = t.chunk_offsets[c], nb = t.chunk_nbytes[c];
                off = std::min<int64_t>(std::max<int64_t>(off, 0), t.packed_nbytes);
                nb = std::min<int64_t>(std::max<int64_t>(nb, 0), t.packed_nbytes - off);
                const int64_t base = c * t.chunk_size;
                const uint32_t lim =
                    static_cast<uint32_t>(std::min<int64_t>(t.chunk_size, t.n_symbols - base));
                // Decoded into the chunk buffer, whose slack takes the whole
                // four-byte stores of the last lookups.
                decode_chunk(J.tb, t.packed + off, static_cast<uint32_t>(nb), lim, ebuf.data());
                if (kBf16)
                    recombine(ebuf.data(), t.sign_mantissa + base,
                              static_cast<uint16_t*>(t.out) + base, lim);
                else
                    std::memcpy(static_cast<uint8_t*>(t.out) + base, ebuf.data(), lim);
            }
        }
    };
    if (threads == 1 || total_syms < (int64_t{1} << 16)) {
        worker();
        return AIMG_OK;
    }
    std::vector<std::thread> pool;
    pool.reserve(static_cast<size_t>(threads - 1));
    try {
        for (int k = 1; k < threads; ++k) pool.emplace_back(worker);
    } catch (const std::exception&) {
        // Fewer threads than asked for: the ones running (and this one) finish the work.
    }
    worker();
    for (auto& th : pool) th.join();
    return AIMG_OK;
}

}  // namespace
}  // namespace aimg

extern "C" int aimg_cpu_decode_bf16(const aimg_tensor* tensors, int n_tensors, int n_threads) {
    return aimg::host_decode<true>(tensors, n_tensors, n_threads);
}

extern "C" int aimg_cpu_decode_u8(const aimg_tensor* tensors, int n_tensors, int n_threads) {
    return aimg::host_decode<false>(tensors, n_tensors, n_threads);
}

extern "C" int aimg_cpu_recombine_bf16(const uint8_t* exponent, const uint8_t* sign_mantissa,
                                       void* out, int64_t n) {
    if (n < 0) return aimg::fail(AIMG_ERR_INVALID_ARGUMENT, "n must be >= 0");
    if (n > 0 && (exponent == nullptr || sign_mantissa == nullptr || out == nullptr))
        return aimg::fail(AIMG_ERR_INVALID_ARGUMENT, "null pointer passed to aimg_cpu_recombine_bf16");
    aimg::recombine(exponent, sign_mantissa, static_cast<uint16_t*>(out), n);
    return AIMG_OK;
}
