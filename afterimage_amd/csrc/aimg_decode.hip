// gfx950 kernels of libafterimage_decode: chunked canonical-Huffman exponent
// decode fused with the BF16 recombine.
//
// One workgroup decodes one chunk. The chunk's bitstream is walked in rounds;
// a round gives each of the 256 threads one segment of S bits (S a multiple
// of 32, at most 256) and runs four phases:
//   1. stage the round's bytes in LDS as big-endian 32-bit words;
//   2. count: every thread parses its segment and records where its first
//      codeword boundary at or after the segment start lies (f) and where the
//      first boundary at or after the segment end lies (e), plus how many
//      codewords start in between. Thread 0 starts from the true boundary
//      carried over from the previous round; every other thread starts
//      speculatively 32 bits early, which Huffman codes of weight exponents
//      resynchronise within in practice. Segment t is right iff its f equals
//      segment t-1's e; any thread for which that fails re-parses from its
//      predecessor's e until all agree, so the result never depends on
//      resynchronisation happening;
//   3. a workgroup prefix sum of the counts places each segment's symbols;
//      threads re-parse from their true starts and write exponent bytes to an
//      LDS staging buffer;
//   4. the staged exponents are combined with the sign/mantissa bytes and
//      written with 16-byte stores (8 bf16 or 16 uint8 per store).
// Codewords are read through a 12-bit window table (up to 6 codewords per
// lookup); codewords longer than 12 bits go to the stored LUT in global memory.
#include <hip/hip_runtime.h>

#include <cstdint>
#include <string>

#include "afterimage_decode.h"
#include "aimg_internal.h"

namespace aimg {
namespace {

constexpr int kThreads = 256;
constexpr int kWaves = kThreads / 64;
constexpr uint32_t kOverlapBits = 32;
constexpr uint32_t kMaxSegBits = 256;
constexpr uint32_t kMinSegBits = 64;
constexpr uint32_t kStageBody = 32768;  // exponent bytes one round may stage
constexpr uint32_t kStagePad = 64;      // carried lead (< 16) and slack
constexpr uint32_t kTileWords = kThreads * kMaxSegBits / 32 + 4;

struct DevTensor {
    const uint8_t* packed;
    const int32_t* offsets;
    const int32_t* nbytes;
    const uint8_t* sm;
    void* out;
    const uint8_t* table;
    int64_t packed_nbytes;
    int64_t n_symbols;
    int64_t job_begin;  // index of this tensor's first chunk in the launch
    int32_t chunk_size;
    int32_t n_chunks;
};

struct LaunchArgs {
    DevTensor t[AIMG_MAX_TENSORS];
    int32_t n_tensors;
};

struct Adv {
    uint32_t p;
    uint32_t n;
};

// 32 bits of the staged stream starting at bit q (MSB-first).
__device__ __forceinline__ uint32_t peek32(const uint32_t* tile, uint32_t q) {
    const uint32_t k = q >> 5;
    const uint64_t v = (static_cast<uint64_t>(tile[k]) << 32) | tile[k + 1];
    return static_cast<uint32_t>((v << (q & 31)) >> 32);
}

// Parse codewords from boundary p until the first boundary at or after x.
// Returns that boundary and the number of codewords that start before x.
__device__ __forceinline__ Adv advance(const uint32_t* tile, const uint64_t* win,
                                       const uint16_t* glut, uint32_t gshift, uint32_t p,
                                       uint32_t x) {
    uint32_t n = 0;
    while (p < x) {
        const uint32_t w = peek32(tile, p);
        const uint64_t ent = win[w >> (32 - kWinBits)];
        const uint32_t m = static_cast<uint32_t>(ent) & 0x1FFFu;
        if (m == 1u) {
            const uint32_t l = glut[w >> gshift] >> 8;
            p += l ? l : 1u;
            n += 1;
            continue;
        }
        const uint32_t rel = x - p;
        const uint32_t total = 31u - __clz(m);
        const uint32_t low = rel > static_cast<uint32_t>(kWinBits) ? 0x1FFFu : ((1u << rel) - 1u);
        n += __popc(m & low & ~(1u << total));
        p += total < rel ? total : static_cast<uint32_t>(__ffs(m & ~low) - 1);
    }
    return {p, n};
}

// Parse from true boundary p to true boundary x, writing each codeword's
// symbol to stage[pos++] while pos < lim.
__device__ __forceinline__ void emit(const uint32_t* tile, const uint64_t* win,
                                     const uint16_t* glut, uint32_t gshift, uint32_t p,
                                     uint32_t x, uint8_t* stage, uint32_t pos, uint32_t lim) {
    while (p < x) {
        const uint32_t w = peek32(tile, p);
        const uint64_t ent = win[w >> (32 - kWinBits)];
        const uint32_t m = static_cast<uint32_t>(ent) & 0x1FFFu;
        if (m == 1u) {
            const uint32_t g = glut[w >> gshift];
            const uint32_t l = g >> 8;
            if (pos < lim) stage[pos] = static_cast<uint8_t>(g);
            ++pos;
            p += l ? l : 1u;
            continue;
        }
        const uint32_t rel = x - p;
        const uint32_t total = 31u - __clz(m);
        const uint32_t low = rel > static_cast<uint32_t>(kWinBits) ? 0x1FFFu : ((1u << rel) - 1u);
        const uint32_t cnt = __popc(m & low & ~(1u << total));
        const uint64_t syms = ent >> 16;
#pragma unroll
        for (uint32_t j = 0; j < static_cast<uint32_t>(kMaxSymsPerWindow); ++j)
            if (j < cnt && pos + j < lim) stage[pos + j] = static_cast<uint8_t>(syms >> (8 * j));
        pos += cnt;
        p += total < rel ? total : rel;
    }
}

// 4 stream bytes starting at byte b of a chunk of nb bytes, as a big-endian
// word; bytes at or past nb read as zero and are never fetched.
__device__ __forceinline__ uint32_t load_be_word(const uint8_t* cbytes, int64_t nb, int64_t b) {
    if (b >= nb) return 0u;
    const uintptr_t addr = reinterpret_cast<uintptr_t>(cbytes + b);
    const uintptr_t al = addr & ~static_cast<uintptr_t>(3);
    const uint32_t sh = static_cast<uint32_t>(addr & 3) * 8u;
    uint32_t v = *reinterpret_cast<const uint32_t*>(al) >> sh;
    if (sh != 0u && b + (4 - sh / 8) < nb) v |= *reinterpret_cast<const uint32_t*>(al + 4) << (32u - sh);
    const int64_t left = nb - b;
    if (left < 4) v &= (1u << (8 * left)) - 1u;
    return __builtin_bswap32(v);
}

__device__ __forceinline__ uint32_t block_scan_excl(uint32_t v, uint32_t* s_wsum, uint32_t* total) {
    const int lane = threadIdx.x & 63;
    const int w = threadIdx.x >> 6;
    uint32_t x = v;
#pragma unroll
    for (int d = 1; d < 64; d <<= 1) {
        const uint32_t y = __shfl_up(x, d, 64);
        if (lane >= d) x += y;
    }
    if (lane == 63) s_wsum[w] = x;
    __syncthreads();
    uint32_t pre = 0, tot = 0;
#pragma unroll
    for (int i = 0; i < kWaves; ++i) {
        const uint32_t s = s_wsum[i];
        pre += i < w ? s : 0u;
        tot += s;
    }
    __syncthreads();
    *total = tot;
    return pre + x - v;
}

// bf16 bits of two elements from two sign/mantissa bytes and two exponents:
// ((sm & 0x80) << 8) | (e << 7) | (sm & 0x7F), the closed form of _recombine
// (compressed_store.py:94-114). x holds e<<8|sm in each 16-bit half.
__device__ __forceinline__ uint32_t bf16_pair(uint32_t x) {
    return ((x >> 1) & 0x7F807F80u) | (x & 0x007F007Fu) | ((x & 0x00800080u) << 8);
}

__device__ __forceinline__ uint16_t bf16_one(uint32_t sm, uint32_t e) {
    return static_cast<uint16_t>(((sm & 0x80u) << 8) | (e << 7) | (sm & 0x7Fu));
}

template <bool kBf16>
__device__ __forceinline__ void store_one(const DevTensor& T, int64_t el, uint32_t e) {
    if (kBf16) {
        static_cast<uint16_t*>(T.out)[el] = bf16_one(T.sm[el], e);
    } else {
        static_cast<uint8_t*>(T.out)[el] = static_cast<uint8_t>(e);
    }
}

// kGroup: elements per store (8 for bf16 / 16 for uint8 with 16-byte
// stores, 1 for the element-wise path used when alignment does not allow).
template <bool kBf16, int kGroup>
__global__ __launch_bounds__(kThreads) void decode_kernel(LaunchArgs args) {
    __shared__ uint64_t s_win[kWinEntries];
    __shared__ uint32_t s_tile[kTileWords];
    __shared__ __attribute__((aligned(16))) uint8_t s_stage[kStageBody + kStagePad];
    __shared__ uint32_t s_f[kThreads];
    __shared__ uint32_t s_e[kThreads];
    __shared__ uint32_t s_wsum[kWaves];

    const int tid = threadIdx.x;
    const int64_t job = blockIdx.x;
    int d = 0;
    while (d + 1 < args.n_tensors && job >= args.t[d + 1].job_begin) ++d;
    const DevTensor& T = args.t[d];
    const int64_t c = job - T.job_begin;

    const TableHeader* hdr = reinterpret_cast<const TableHeader*>(T.table);
    const uint32_t gshift = 32u - hdr->max_bits;
    const uint32_t min_len = hdr->min_len;
    const uint32_t sym0 = hdr->sym0;
    const uint16_t* glut = reinterpret_cast<const uint16_t*>(T.table + kGlutOffset);
    {
        const uint4* src = reinterpret_cast<const uint4*>(T.table + kWinOffset);
        uint4* dst = reinterpret_cast<uint4*>(s_win);
        for (int i = tid; i < kWinEntries / 2; i += kThreads) dst[i] = src[i];
    }

    int64_t off = T.offsets[c];
    int64_t nb = T.nbytes[c];
    off = off < 0 ? 0 : (off > T.packed_nbytes ? T.packed_nbytes : off);
    nb = nb < 0 ? 0 : (nb > T.packed_nbytes - off ? T.packed_nbytes - off : nb);
    const uint8_t* cbytes = T.packed + off;
    const int64_t chunk_bits = nb * 8;
    const int64_t chunk_base = c * T.chunk_size;
    int64_t lim = T.n_symbols - chunk_base;
    lim = lim < 0 ? 0 : (lim > T.chunk_size ? T.chunk_size : lim);

    uint32_t smax = (kStageBody * min_len) / kThreads;
    smax = (smax > kMaxSegBits ? kMaxSegBits : smax) & ~31u;
    const int64_t per_round_max = static_cast<int64_t>(kThreads) * smax;
    const int64_t nr = (chunk_bits + per_round_max - 1) / per_round_max;
    uint32_t S = kMinSegBits;
    if (nr > 0) {
        const int64_t per_thread = (chunk_bits + kThreads * nr - 1) / (kThreads * nr);
        S = static_cast<uint32_t>((per_thread + 31) & ~int64_t(31));
        S = S < kMinSegBits ? kMinSegBits : S;
    }
    const uint32_t round_bits = kThreads * S;

    uint32_t p0 = 0;      // true start of the next round, relative to its first bit
    int64_t ob = 0;       // chunk-local symbols produced so far
    uint32_t lead = 0;    // staged symbols carried from the previous round
    uint32_t tail_at = 0; // stage index of those carried symbols after the loop
    for (int64_t r = 0; r < nr; ++r) {
        const int64_t R0 = r * round_bits;
        const int64_t left_bits = chunk_bits - R0;
        const uint32_t RB = left_bits < round_bits ? static_cast<uint32_t>(left_bits) : round_bits;
        const uint32_t nw = (RB + 31) / 32 + 2;
        for (uint32_t j = tid; j < nw; j += kThreads)
            s_tile[j] = load_be_word(cbytes, nb, R0 / 8 + 4 * static_cast<int64_t>(j));
        __syncthreads();

        const uint32_t seg_lo = tid * S;
        const bool active = seg_lo < RB;
        const uint32_t seg_hi = active ? (seg_lo + S < RB ? seg_lo + S : RB) : 0u;
        uint32_t f = 0, e = 0, cnt = 0;
        if (active) {
            f = tid == 0 ? p0 : advance(s_tile, s_win, glut, gshift, seg_lo - kOverlapBits, seg_lo).p;
            const Adv a = advance(s_tile, s_win, glut, gshift, f, seg_hi);
            e = a.p;
            cnt = a.n;
        }
        s_f[tid] = f;
        s_e[tid] = e;
        __syncthreads();
        for (;;) {
            const bool bad = active && tid > 0 && s_f[tid] != s_e[tid - 1];
            const uint32_t nf = bad ? s_e[tid - 1] : 0u;
            if (!__syncthreads_or(bad)) break;
            if (bad) {
                f = nf;
                const Adv a = advance(s_tile, s_win, glut, gshift, f, seg_hi);
                e = a.p;
                cnt = a.n;
                s_f[tid] = f;
                s_e[tid] = e;
            }
            __syncthreads();
        }

        uint32_t total;
        const uint32_t o = block_scan_excl(cnt, s_wsum, &total);
        const int64_t room = lim - ob;
        uint32_t take = total < room ? total : static_cast<uint32_t>(room);
        if (take > kStageBody) take = kStageBody;  // only malformed streams get here
        if (active && cnt > 0)
            emit(s_tile, s_win, glut, gshift, f, e, s_stage, lead + o, lead + take);
        const uint32_t n_active = (RB + S - 1) / S;
        const uint32_t e_last = s_e[n_active - 1];
        __syncthreads();

        const int64_t a0 = chunk_base + ob - lead;
        const uint32_t avail = lead + take;
        const uint32_t nfull = avail / kGroup;
        for (uint32_t g = tid; g < nfull; g += kThreads) {
            const int64_t el = a0 + static_cast<int64_t>(g) * kGroup;
            if (kGroup == 1) {
                store_one<kBf16>(T, el, s_stage[g]);
            } else if (kBf16) {
                const uint2 smv = *reinterpret_cast<const uint2*>(T.sm + el);
                const uint2 ev = *reinterpret_cast<const uint2*>(s_stage + g * kGroup);
                uint4 o4;
                o4.x = bf16_pair(__builtin_amdgcn_perm(ev.x, smv.x, 0x05010400u));
                o4.y = bf16_pair(__builtin_amdgcn_perm(ev.x, smv.x, 0x07030602u));
                o4.z = bf16_pair(__builtin_amdgcn_perm(ev.y, smv.y, 0x05010400u));
                o4.w = bf16_pair(__builtin_amdgcn_perm(ev.y, smv.y, 0x07030602u));
                *reinterpret_cast<uint4*>(static_cast<uint16_t*>(T.out) + el) = o4;
            } else {
                *reinterpret_cast<uint4*>(static_cast<uint8_t*>(T.out) + el) =
                    *reinterpret_cast<const uint4*>(s_stage + g * kGroup);
            }
        }
        ob += take;
        const uint32_t rem = avail - nfull * kGroup;
        if (r + 1 < nr) {
            __syncthreads();
            const uint8_t carry = tid < static_cast<int>(rem) ? s_stage[nfull * kGroup + tid] : 0;
            __syncthreads();
            if (tid < static_cast<int>(rem)) s_stage[tid] = carry;
            tail_at = 0;
        } else {
            tail_at = nfull * kGroup;
        }
        lead = rem;
        p0 = e_last - RB;
    }

    // Symbols carried out of the last round, then positions no codeword of
    // the chunk reached: those decode from zero bits, i.e. to sym_lut[0].
    const int64_t t0 = chunk_base + ob - lead;
    const int64_t n_tail = lim - (ob - lead);
    for (int64_t i = tid; i < n_tail; i += kThreads) {
        const uint32_t e = i < lead ? s_stage[tail_at + i] : sym0;
        store_one<kBf16>(T, t0 + i, e);
    }
}

template <bool kBf16>
int launch(const aimg_tensor* ts, int n, void* stream) {
    if (ts == nullptr && n > 0) return fail(AIMG_ERR_INVALID_ARGUMENT, "tensors is null");
    if (n < 0 || n > AIMG_MAX_TENSORS)
        return fail(AIMG_ERR_INVALID_ARGUMENT,
                    "n_tensors must be in 0.." + std::to_string(AIMG_MAX_TENSORS));
    LaunchArgs args{};
    int64_t jobs = 0;
    bool vec = true;
    const int group = kBf16 ? 8 : 16;
    int m = 0;
    for (int i = 0; i < n; ++i) {
        const aimg_tensor& t = ts[i];
        const std::string who = "tensor " + std::to_string(i) + ": ";
        if (t.chunk_size < 1) return fail(AIMG_ERR_INVALID_ARGUMENT, who + "chunk_size must be >= 1");
        if (t.n_chunks < 0 || t.n_symbols < 0 || t.packed_nbytes < 0)
            return fail(AIMG_ERR_INVALID_ARGUMENT, who + "negative size");
        if (t.n_symbols > static_cast<int64_t>(t.n_chunks) * t.chunk_size)
            return fail(AIMG_ERR_INVALID_ARGUMENT, who + "n_symbols exceeds n_chunks * chunk_size");
        if (t.n_symbols == 0) continue;
        if (t.packed == nullptr || t.chunk_offsets == nullptr || t.chunk_nbytes == nullptr ||
            t.out == nullptr || t.table == nullptr || (kBf16 && t.sign_mantissa == nullptr))
            return fail(AIMG_ERR_INVALID_ARGUMENT, who + "null device pointer");
        if (reinterpret_cast<uintptr_t>(t.table) % 16 != 0)
            return fail(AIMG_ERR_INVALID_ARGUMENT, who + "table must be 16-byte aligned");
        if (reinterpret_cast<uintptr_t>(t.out) % 16 != 0 || t.chunk_size % group != 0 ||
            (kBf16 && reinterpret_cast<uintptr_t>(t.sign_mantissa) % 8 != 0))
            vec = false;
        DevTensor& dt = args.t[m++];
        dt.packed = t.packed;
        dt.offsets = t.chunk_offsets;
        dt.nbytes = t.chunk_nbytes;
        dt.sm = t.sign_mantissa;
        dt.out = t.out;
        dt.table = static_cast<const uint8_t*>(t.table);
        dt.packed_nbytes = t.packed_nbytes;
        dt.n_symbols = t.n_symbols;
        dt.chunk_size = t.chunk_size;
        dt.n_chunks = t.n_chunks;
        dt.job_begin = jobs;
        // Chunks past the last output element hold nothing to write.
        jobs += (t.n_symbols + t.chunk_size - 1) / t.chunk_size;
    }
    args.n_tensors = m;
    if (jobs == 0) return AIMG_OK;
    if (jobs > 0x7FFFFFFF) return fail(AIMG_ERR_UNSUPPORTED, "more than 2^31-1 chunks in one launch");
    const hipStream_t s = static_cast<hipStream_t>(stream);
    const dim3 grid(static_cast<uint32_t>(jobs)), block(kThreads);
    if (vec) {
        hipLaunchKernelGGL((decode_kernel<kBf16, kBf16 ? 8 : 16>), grid, block, 0, s, args);
    } else {
        hipLaunchKernelGGL((decode_kernel<kBf16, 1>), grid, block, 0, s, args);
    }
    const hipError_t err = hipGetLastError();
    if (err != hipSuccess)
        return fail(AIMG_ERR_HIP, std::string("kernel launch failed: ") + hipGetErrorString(err));
    return AIMG_OK;
}

}  // namespace
}  // namespace aimg

extern "C" int aimg_decode_bf16(const aimg_tensor* tensors, int n_tensors, void* stream) {
    return aimg::launch<true>(tensors, n_tensors, stream);
}

extern "C" int aimg_decode_u8(const aimg_tensor* tensors, int n_tensors, void* stream) {
    return aimg::launch<false>(tensors, n_tensors, stream);
}
