// gfx950 kernels of libafterimage_decode: chunked canonical-Huffman exponent
// decode fused with the BF16 recombine.
//
// Work layout. A workgroup has 512 threads (8 waves) and uses under 80 KB
// of LDS, so two are resident per CU and one's memory phases overlap the
// other's decoding. The grid is persistent and walks "items". An item is a
// batch of chunks of one tensor: the workgroup splits into 512/TPC sub-groups
// of TPC threads (TPC = 16..512, chosen per tensor from its chunk size), and
// each sub-group decodes one chunk.
//
// A sub-group walks its chunk's bitstream in rounds. A round gives each
// thread one segment of S bits, with S at most kSlotCap times the shortest
// code length, so no segment holds more than kSlotCap codeword starts. A
// round runs:
//   1. stage the round's bytes in LDS as big-endian 32-bit words;
//   2. decode: each thread parses its segment once, writing the symbols of
//      every table lookup into its own LDS slot, and records the first
//      codeword boundary at or after the segment start (f), the first at or
//      after the segment end (e), and the codewords in between. Thread 0
//      starts from the boundary carried over from the previous round; every
//      other thread starts 32 bits early on a guess, which Huffman codes of
//      weight exponents resynchronise within in practice. Segment t is right
//      iff its f equals segment t-1's e; threads for which that fails decode
//      again from their predecessor's e until all agree, so the result never
//      depends on resynchronisation happening;
//   3. a workgroup prefix sum of the counts places each segment's symbols;
//   4. compaction: each thread reads its slot into registers and, after a
//      barrier, writes its symbols at their place in the same LDS area
//      (whole aligned words, single bytes at the two ends);
//   5. the staged exponents are combined with the sign/mantissa bytes and
//      written with 16-byte stores (8 bf16 or 16 uint8 per store); the last
//      partial vector group moves to the front for the next round.
//
// Codewords are read through a 12-bit window table of up to 4 codewords per
// lookup (LDS); codewords of 13..16 bits go through 16-entry escape blocks
// (LDS for the first 48 blocks, global memory beyond).
#include <hip/hip_runtime.h>

#include <atomic>
#include <cstdint>
#include <cstdlib>
#include <mutex>
#include <string>

#include "afterimage_decode.h"
#include "aimg_internal.h"

namespace aimg {
namespace {

constexpr int kThreads = 512;
constexpr int kBlocksPerCu = 2;
// Waves each SIMD must hold for kBlocksPerCu resident workgroups (4 SIMDs
// per CU); bounds the registers a thread may use.
constexpr int kWavesPerSimd = kBlocksPerCu * (kThreads / 64) / 4;
constexpr int kWaves = kThreads / 64;
constexpr uint32_t kLgThreads = 9;
static_assert(kThreads == 1 << kLgThreads, "kLgThreads");
constexpr int kMinTpc = 16;
constexpr int kMaxGroups = kThreads / kMinTpc;
// A segment's start is guessed by decoding the kOverlapBits before it from an
// arbitrary bit (prefix codes resynchronise): the longer the run-in, the fewer
// guesses the agreement check sends back to decode again (5120x17408 layer:
// 16 bits 79.9 us, 32 bits 67.2, 48 bits 65.9, 64 bits 67.3; 1024-symbol
// chunks 81.5, 70.1, 69.2, 70.4). Segments are at least 80 bits long.
constexpr uint32_t kOverlapBits = 48;
static_assert(kOverlapBits < segment_bits(1), "a segment's run-in starts inside the round");
// Per-thread slot for one segment's symbols: at most kSlotCap of them. A
// lookup's symbols go into the aligned word holding the first and the word
// after it, which may lie past the cap. Slots are kSlotBytes apart, an odd
// number of words, so the lanes of a wave writing at similar counts hit
// different LDS banks. 168-bit segments at the 2-bit shortest code of bf16
// weights make a 64Ki-symbol chunk (about 171K bits) two rounds of 512
// segments.
constexpr uint32_t kSlotCap = kSegCodewords;
constexpr uint32_t kSlotWords = kSlotCap / 4;  // compaction reads these and one more
constexpr uint32_t kSlotRows = kSlotWords + 1;  // a slot's words: kSlotCap symbols and the word after
constexpr uint32_t kSlotBytes = 92;
static_assert(kSlotCap % 4 == 0 && kSlotBytes >= kSlotCap + 4, "slot room for the word after the cap");
static_assert(kSlotBytes % 4 == 0 && (kSlotBytes / 4) % 2 == 1, "slot stride: an odd number of words");
constexpr uint32_t kLeadBytes = 16;  // room for a carried partial vector group
constexpr uint32_t kTileSlackWords = 4;
constexpr uint32_t kTileWords = kThreads * kMaxSegBits / 32 + kTileSlackWords * kMaxGroups;
constexpr uint32_t kStageBytes = kThreads * kSlotBytes + kLeadBytes * kMaxGroups;
static_assert(kStageBytes % (16 * kMaxGroups) == 0, "stage regions stay 16-byte aligned");
static_assert(kTileWords % kMaxGroups == 0, "tile regions split evenly");
constexpr int kLdsEscBlocks = 48;
// Stream words a thread fetches per round: a round has at most
// tpc * kMaxSegBits / 32 + 3 words.
constexpr uint32_t kTileBatch = kMaxSegBits / 32 + 1;
// Output vector groups a thread stores per round: a round places at most
// kSlotCap symbols per thread, plus a carried partial group.
constexpr uint32_t kStoreBatch = (kSlotCap * kMinTpc + 15 + 8 * kMinTpc - 1) / (8 * kMinTpc);
static_assert(kStoreBatch * 8 * kMinTpc >= kSlotCap * kMinTpc + 15, "one store batch covers a round");
// Interleaved slots of a whole-workgroup chunk (word j of lane l of wave w at
// row j, column l of the wave's block).
constexpr uint32_t kWholeSlotBytes = kWaves * kSlotRows * 64 * 4;
static_assert(kLeadBytes + kWholeSlotBytes <= kStageBytes, "the interleaved slots fit the stage");
constexpr uint32_t kStagePadded =
    (kStageBytes + 16 > kStoreBatch * kThreads * 8 ? kStageBytes + 16 : kStoreBatch * kThreads * 8);
// Of those, the groups whose sign/mantissa bytes are requested while the round
// decodes: all of them (a round of bf16 weights fills about 8 groups per
// thread, up to kStoreBatch). With fewer, the store loop carries a branch
// that loads the rest; 9 groups (36,864 symbols per round) decoded the
// 5120x17408 layer 3.8% slower, 7 groups 7%.
constexpr uint32_t kSmAhead = kStoreBatch;
// Cache-policy operand of the bf16 output stores: non-temporal (streamed
// past the caches' normal retention). The output is written once; 4.5%
// faster on the 5120x17408 layer than the default policy, while the same
// policy on the stream-word or sign/mantissa loads was 2.5% slower.
constexpr int kCachePolicyNT = 2;
// s_sleep argument (units of 64 clocks) of each of the two sleeps that delay
// the second workgroup of a CU in the chunk kernel: 2 x 80 x 64 = 10240
// clocks, about 4.3 us at 2.4 GHz.
constexpr int kStaggerSleep = 80;
static_assert(kSmAhead <= kStoreBatch, "kSmAhead");

struct DevTensor {
    const uint8_t* packed;
    const int32_t* offsets;
    const int32_t* nbytes;
    const uint8_t* sm;
    void* out;
    const uint8_t* table;
    int64_t packed_nbytes;
    int64_t n_symbols;
    int64_t item_begin;  // first item of this tensor in the launch
    int64_t n_jobs;      // chunks that hold output elements
    int32_t chunk_size;
    int32_t tpc;         // threads per chunk (power of two, 16..512)
    uint32_t packed_n32;  // packed_nbytes, capped at 2^32 - 1 (buffer loads)
    uint8_t* index;       // segment index, or null
    uint32_t index_n32;   // index bytes, capped at 2^32 - 1
    int32_t n_chunks;
};

// What a launch makes of the decoded exponents.
enum Mode : int {
    kModeU8 = 0,    // the exponent bytes themselves
    kModeBf16 = 1,  // bf16 weights
    kModeGemv = 2,  // y += W x with W decoded on the fly and never written
    kModeGemv1 = 3, // kModeGemv for one x vector (batch 1)
    kModeIndex = 4, // the segment index: each segment's first boundary and codewords
    kModeGemm = 5,      // Y += X W^T for up to 16 rows of X, W decoded on the fly (MFMA)
    kModeGemmRows = 6,  // kModeGemm for rows of more than kGemmPieceMaxCols columns
};
constexpr bool is_gemm(int mode) { return mode == kModeGemm || mode == kModeGemmRows; }
// Modes that combine the exponents with sign/mantissa bytes.
constexpr bool needs_sm(int mode) { return mode != kModeU8 && mode != kModeIndex; }
// Job::ib of a chunk decoded without the index.
constexpr uint32_t kNoIndex = 0xFFFFFFFFu;
constexpr int kGemvMaxBatch = 4;
// Rows of x (tokens) of the fused decode -> GEMM: one MFMA tile's 16.
constexpr int kGemmMaxRows = 16;
// Steps ahead of use that x is requested with up to kGemvMaxBatch x vectors
// (with one, 3). Measured on the 5120x17408 layer at batch 4: 2 steps
// ahead 7% slower than 1, 3 steps 39% slower.
constexpr uint32_t kGemvXAhead = 1;

struct GemvArgs {
    const uint16_t* x;  // bf16 [batch][cols] (GEMM: [rows of x][cols])
    float* y;           // fp32 [batch][rows], accumulated
    uint32_t rows;
    uint32_t cols;
    int32_t batch;
    uint32_t step_rows;  // 4096 elements (8 per thread of a 512-thread chunk)
    uint32_t step_cols;  // = step_rows rows + step_cols columns
};

struct LaunchArgs {
    DevTensor t[AIMG_MAX_TENSORS];
    int64_t total_items;  // speculative runs: the tensors' elements
    int32_t n_tensors;
    // Segment runs: workgroup w takes rounds w, w + grid, ... Speculative
    // runs: a full grid, whose workgroups b and b + grid / 2 split a CU's share.
    int32_t strided;
    GemvArgs gemv;  // kModeGemv only (one tensor)
    // Chunk by chunk, whole-workgroup chunks: the last n_split chunks (from
    // chunk item split_first on) are split in two halves of their rounds.
    // Items 0 .. n_split - 1 are their first halves, the grid's first items;
    // then come the other chunks, then the second halves. Split chunk k hands
    // over through record k of `handoff`, tagged with `tag`. n_split 0: no
    // chunk is split.
    int64_t split_first;
    int64_t n_split;
    uint64_t* handoff;
    uint32_t tag;
    // bf16 and exponent-byte decodes chunk by chunk on a full grid (two
    // workgroups per CU, workgroups w and w + grid / 2 sharing one): the
    // second half of the grid starts later.
    int32_t stagger;
};

// Read-only launch data that every thread of a workgroup reads at the same
// address (table header, a workgroup's own chunk offset and length): loaded
// through the constant address space, i.e. with scalar loads, which do not
// queue behind the workgroup's outstanding vector stores.
template <typename T>
__device__ __forceinline__ T load_uniform(const T* p) {
    return *(const __attribute__((address_space(4))) T*)(p);
}

// Values the same in every lane, moved to scalar registers: the compiler
// cannot always prove it, and loads through a pointer it takes for divergent
// become vector loads, whose waits also wait for the stores issued before.
// The builtin takes and returns int: each half goes back through uint32_t so
// that a low word with its top bit set is not sign-extended into the high one.
__device__ __forceinline__ uint32_t uniform(uint32_t v) {
    return static_cast<uint32_t>(__builtin_amdgcn_readfirstlane(static_cast<int>(v)));
}

template <typename P>
__device__ __forceinline__ P* uniform(P* p) {
    const uint64_t v = reinterpret_cast<uintptr_t>(p);
    const uint64_t lo = uniform(static_cast<uint32_t>(v));
    const uint64_t hi = uniform(static_cast<uint32_t>(v >> 32));
    return reinterpret_cast<P*>((hi << 32) | lo);
}

__device__ __forceinline__ const __attribute__((address_space(4))) TableHeader* header_of(
    const uint8_t* table) {
    return (const __attribute__((address_space(4))) TableHeader*)(table);
}

typedef uint32_t v4u32 __attribute__((ext_vector_type(4)));

// A generic pointer to LDS holds the LDS offset in its low 32 bits. Reads
// through the LDS-typed pointer built from that offset let the compiler fold
// constant offsets into the LDS instructions (it does not for generic
// pointers whose offset it cannot prove in range).
using LdsOff = uint32_t;
template <typename T>
__device__ __forceinline__ const __attribute__((address_space(3))) T* lds_ptr(const T* p) {
    return (const __attribute__((address_space(3))) T*)(uintptr_t)static_cast<LdsOff>(
        reinterpret_cast<uintptr_t>(p));
}

// Buffer resource over `nbytes` bytes at `base` (raw, stride 0): loads past
// the end return zero and stores past it are dropped, instead of touching
// memory outside the buffer.
__device__ __forceinline__ __amdgpu_buffer_rsrc_t buffer_of(const void* base, uint32_t nbytes) {
    return __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(base), 0, static_cast<int>(nbytes),
                                             0x00020000);
}

struct Tables {
    const uint32_t* syms;    // LDS window table: symbols / escape block
    const uint8_t* meta;     // LDS window table: total | count << 5
    const uint8_t* len;      // LDS code length of each symbol
    const uint16_t* esc;     // LDS escape blocks (first kLdsEscBlocks)
    const __attribute__((address_space(1))) uint16_t* gesc;  // all escape blocks, global memory
    uint32_t sym0;
    uint32_t min_len;  // shortest code length
};

// Bit reader over the staged stream. A sub-group's tile holds its round's
// stream words in reverse order (word j at top[-j]), so one 8-byte LDS read
// at top - k - 1 returns words k+1 and k as the low and high halves of the
// 64-bit pair that starts at word k. `pair` holds the words from bit
// p - sh (a multiple of 32, sh <= 47); a step reads at most 16 bits, all
// inside the pair. While a step's table lookup is in flight, the reader
// already fetches the pair starting at the word that contains p, which
// holds the next step's bits, so each step waits for one LDS round trip.
//
// `below` is the LDS byte address of top - 1: the pair whose first word
// starts at bit m (a multiple of 32) is at below - m / 8.
typedef const __attribute__((address_space(3))) uint8_t* TileRef;
typedef const __attribute__((address_space(3))) uint32_t* TileWords;

struct Reader {
    TileRef below;
    uint32_t p;
    uint32_t sh;
    uint64_t pair;
};

__device__ __forceinline__ uint64_t load_pair(TileRef below, uint32_t m) {
    const TileWords w = reinterpret_cast<TileWords>(below - (m >> 3));
    return static_cast<uint64_t>(w[0]) | (static_cast<uint64_t>(w[1]) << 32);
}

__device__ __forceinline__ Reader reader_at(TileRef below, uint32_t p) {
    return {below, p, p & 31u, load_pair(below, p & ~31u)};
}

// The 32 bits at the reader's position (bits past the pair read as zero;
// only the first 16 are used).
__device__ __forceinline__ uint32_t reader_bits(const Reader& rd) {
    return static_cast<uint32_t>((rd.pair << rd.sh) >> 32);
}

// Move the reader forward by n bits (n <= 16), using the pair prefetched at
// the old position (first word at bit m = old p & ~31).
__device__ __forceinline__ void reader_skip(Reader& rd, uint64_t next_pair, uint32_t m, uint32_t n) {
    rd.p += n;
    rd.sh = rd.p - m;
    rd.pair = next_pair;
}

// (symbol, length) of an escape window's first codeword; w holds the window
// in bits 31..20 and the next four bits in 19..16. Bits that start no
// codeword of the stored LUT (only a malformed stream has them) decode to
// sym_lut[0] and take the shortest code length, so every lookup consumes
// at least that many bits per codeword, whatever the input.
// kGlobalEsc: the table has escape blocks beyond the ones held in LDS. Only
// then does the loop carry a global load, whose wait would also wait for
// every prefetch in flight, so tables without such blocks use loops that
// have none.
template <bool kGlobalEsc>
__device__ __forceinline__ uint32_t escape(const Tables& tb, uint32_t ent, uint32_t w,
                                           uint32_t* len) {
    const uint32_t blk = ent & 0xFFFFu;
    if (blk == kUnusedBlock) {
        *len = tb.min_len;
        return tb.sym0;
    }
    const uint32_t at = blk * kEscBlockEntries + ((w >> 16) & 15u);
    uint32_t v;
    if (!kGlobalEsc || blk < static_cast<uint32_t>(kLdsEscBlocks)) {
        v = tb.esc[at];
    } else {
        v = tb.gesc[at];
    }
    const uint32_t l = v >> 8;
    *len = l ? l : tb.min_len;
    return l ? v & 0xFFu : tb.sym0;
}

// Escape windows are rare: the wave branches to them only when one of its
// lanes has one.
__device__ __forceinline__ bool any_lane(bool v) { return __builtin_amdgcn_ballot_w64(v) != 0; }

struct Adv {
    uint32_t p;
    uint32_t n;
};

// A window that ends at or past x, starting at P < x with c codewords
// (symbols: the bytes of syms): its codewords that start at or after x are
// cut off. Returns the first codeword boundary at or after x (`end`, the
// window's end, if none starts inside) and sets *kept to the codewords that
// start before x. Boundaries come from the symbols' code lengths.
__device__ __forceinline__ uint32_t cut_window(const Tables& tb, uint32_t P, uint32_t end,
                                               uint32_t syms, uint32_t c, uint32_t x,
                                               uint32_t* kept) {
    uint32_t st = P, e = end, k = c;
#pragma unroll
    for (uint32_t j = 0; j + 1 < static_cast<uint32_t>(kMaxSymsPerWindow); ++j) {
        if (j + 1 < c) {
            st += tb.len[(syms >> (8 * j)) & 0xFFu];
            if (st >= x && k == c) {
                e = st;
                k = j + 1;
            }
        }
    }
    *kept = k;
    return e;
}

// One table lookup: the window at the reader's position, its meta and (for
// decode) symbols, and the pair the following step reads, prefetched from the
// word holding the position (first word at bit m).
struct Step {
    uint32_t p;      // window start
    uint32_t w;      // window bits (31..20) and the next four (19..16)
    uint32_t idx;    // window table index
    uint32_t meta;
    uint32_t syms;
    uint32_t m;
    uint64_t next;
};

template <bool kSyms>
__device__ __forceinline__ Step lookup(TileRef below, const Tables& tb, uint32_t p, uint32_t sh,
                                       uint64_t pair) {
    Step s;
    s.p = p;
    s.w = static_cast<uint32_t>((pair << sh) >> 32);
    s.idx = s.w >> (32 - kWinBits);
    s.meta = tb.meta[s.idx];
    s.m = p & ~31u;
    s.next = load_pair(below, s.m);
    s.syms = kSyms ? tb.syms[s.idx] : 0u;
    return s;
}

// A lookup's symbols, bits and codewords; an escape window (rare: the wave
// branches only when one of its lanes has one) takes its first codeword from
// the escape block.
template <bool kGlobalEsc>
__device__ __forceinline__ void take(const Tables& tb, const Step& s, uint32_t* syms, uint32_t* adv,
                                     uint32_t* c) {
    *syms = s.syms;
    *adv = s.meta & 31u;
    *c = s.meta >> 5;
    if (__builtin_expect(any_lane(*adv == 0), 0)) {
        if (*adv == 0) {
            *syms = escape<kGlobalEsc>(tb, tb.syms[s.idx], s.w, adv);
            *c = 1;
        }
    }
}

// The first codeword boundary at or after x, parsing from boundary p < x.
// Each step takes a whole window; the step whose window reaches x is cut
// there, once, after the loop. Steps are software-pipelined: as soon as a
// step's length is known, the next step's lookup is issued.
template <bool kGlobalEsc>
__device__ __forceinline__ uint32_t advance(TileRef below, const Tables& tb, uint32_t p,
                                            uint32_t x) {
    const Reader rd = reader_at(below, p);
    Step s = lookup<false>(below, tb, rd.p, rd.sh, rd.pair);
    uint32_t syms, adv, c;
    take<kGlobalEsc>(tb, s, &syms, &adv, &c);
    uint32_t pn = s.p + adv;
    while (pn < x) {
        s = lookup<false>(below, tb, pn, pn - s.m, s.next);
        take<kGlobalEsc>(tb, s, &syms, &adv, &c);
        pn = s.p + adv;
    }
    const uint32_t sp = pn - adv;  // s.p, from pn (see decode_run_il)
    uint32_t kept;
    return cut_window(tb, sp, pn, c > 1 ? tb.syms[s.idx] : 0u, c, x, &kept);
}

// Before a segment is decoded into a slot, its first word is zero.
__device__ __forceinline__ void start_slot(uint8_t* slot) { *reinterpret_cast<uint32_t*>(slot) = 0u; }

// Place the symbols of one lookup (bytes of syms, zero above the lookup's
// count) at q (inside a slot, which is word-aligned): OR them into the word
// holding q and write the word after it whole. Invariant: the word holding q
// is zero from q up, since it was either the slot's first word or the last
// whole word written, whose bytes from q up are zero bytes of syms.
__device__ __forceinline__ void slot_put(uint8_t* q, uint32_t syms) {
    const uint32_t b = static_cast<uint32_t>(reinterpret_cast<uintptr_t>(q)) & 3u;
    const uint64_t v = static_cast<uint64_t>(syms) << (8 * b);
    uint32_t* w = reinterpret_cast<uint32_t*>(q - b);
    __hip_atomic_fetch_or(w, static_cast<uint32_t>(v), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP);
    w[1] = static_cast<uint32_t>(v >> 32);
}

// Parse codewords from true boundary p while they start before x, placing
// their symbols in the slot (first word zero). Returns the first boundary at
// or after x and the number of codewords. Every codeword (or unused window)
// takes at least min_len bits, so a segment of at most kSlotCap * min_len
// bits never holds more than kSlotCap codewords, and every write stays
// inside the slot. The last lookup's symbols that start at or after x are
// masked off before it is placed.
template <bool kGlobalEsc>
__device__ __forceinline__ Adv decode_run(TileRef below, const Tables& tb, uint32_t p,
                                          uint32_t x, uint8_t* slot) {
    if (p >= x) return {p, 0u};
    uint8_t* q = slot;
    const Reader rd = reader_at(below, p);
    Step s = lookup<true>(below, tb, rd.p, rd.sh, rd.pair);
    uint32_t syms, adv, c;
    take<kGlobalEsc>(tb, s, &syms, &adv, &c);
    uint32_t pn = s.p + adv;
    while (pn < x) {
        // The next step's meta and pair go out before this step's symbols
        // are placed, its symbols after.
        Step t = lookup<false>(below, tb, pn, pn - s.m, s.next);
        slot_put(q, syms);
        q += c;
        t.syms = tb.syms[t.idx];
        s = t;
        take<kGlobalEsc>(tb, s, &syms, &adv, &c);
        pn = s.p + adv;
    }
    uint32_t kept;  // 1..4
    const uint32_t e = cut_window(tb, s.p, s.p + adv, syms, c, x, &kept);
    slot_put(q, syms & (0xFFFFFFFFu >> (32u - 8u * kept)));
    return {e, static_cast<uint32_t>(q - slot) + kept};
}

__device__ __forceinline__ void lds_or(uint32_t* w, uint32_t v) {
    __hip_atomic_fetch_or(w, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP);
}

// OR one lookup's symbols (bytes of syms, zero above its count) into the
// word holding q, together with `carry`, the bytes the previous lookup put
// past its own word, which belong at the start of this word. Returns this
// lookup's bytes past the word (zero unless it crosses into the next one),
// the next call's carry.
__device__ __forceinline__ uint32_t stage_or(uint8_t* q, uint32_t syms, uint32_t carry) {
    const uint32_t b = static_cast<uint32_t>(reinterpret_cast<uintptr_t>(q)) & 3u;
    const uint64_t v = static_cast<uint64_t>(syms) << (8 * b);
    lds_or(reinterpret_cast<uint32_t*>(q - b), static_cast<uint32_t>(v) | carry);
    return static_cast<uint32_t>(v >> 32);
}

// Decode the segment from true boundary p while codewords start before x,
// placing its symbols from q on in a stage area that is zero where nothing
// is placed. Neighbouring segments share the words at their ends, so every
// write is an atomic OR: one per lookup, a lookup's bytes that spill into
// the next word going out with the next lookup's word, and the last spill
// at the end. Dense placement puts the lanes of a wave at effectively
// random LDS banks, so every write pays bank conflicts: on the 5120x17408
// layer one write per lookup is 9% faster than two (the word and the word
// after it), and as fast as the same writes to conflict-free addresses; a
// byte-aligned 4-byte store per lookup with no atomics is 29% slower.
template <bool kGlobalEsc>
__device__ __forceinline__ void decode_placed(TileRef below, const Tables& tb, uint32_t p,
                                              uint32_t x, uint8_t* q) {
    if (p >= x) return;
    const Reader rd = reader_at(below, p);
    Step s = lookup<true>(below, tb, rd.p, rd.sh, rd.pair);
    uint32_t syms, adv, c;
    take<kGlobalEsc>(tb, s, &syms, &adv, &c);
    uint32_t carry = 0;
    uint32_t pn = s.p + adv;
    while (pn < x) {
        Step t = lookup<false>(below, tb, pn, pn - s.m, s.next);
        carry = stage_or(q, syms, carry);
        q += c;
        t.syms = tb.syms[t.idx];
        s = t;
        take<kGlobalEsc>(tb, s, &syms, &adv, &c);
        pn = s.p + adv;
    }
    uint32_t kept;
    cut_window(tb, s.p, s.p + adv, syms, c, x, &kept);
    const uint32_t spill = stage_or(q, syms & (0xFFFFFFFFu >> (32u - 8u * kept)), carry);
    if (spill != 0u)
        lds_or(reinterpret_cast<uint32_t*>((q - (reinterpret_cast<uintptr_t>(q) & 3u)) + 4), spill);
}

// A lane's interleaved slot: word j of lane l of wave w at byte
// wblk + 256 j + 4 l of `slots` (wblk = w * kSlotRows * 256, a multiple of 256).
struct IlSlot {
    uint8_t* slots;
    uint32_t wblk;
    uint32_t lane4;  // 4 l
};

// One lookup's symbols into an interleaved slot at qa = wblk + 64 q, for
// slot byte q, as slot_put does it: word q / 4 is at (qa & ~255) | lane4
// and the byte within it is (qa >> 6) & 3 (one AND-OR for the address).
__device__ __forceinline__ void slot_put_il(const IlSlot& sl, uint32_t qa, uint32_t syms) {
    const uint64_t v = static_cast<uint64_t>(syms) << ((qa >> 3) & 24u);
    uint32_t* w = reinterpret_cast<uint32_t*>(sl.slots + ((qa & ~255u) | sl.lane4));
    lds_or(w, static_cast<uint32_t>(v));
    w[64] = static_cast<uint32_t>(v >> 32);
}

// decode_run into an interleaved slot. cend: the bit where the segment's
// chunk ends, when the tile holds the next chunk's bits after it (speculative
// runs; the chunk kernel's tile is zero past its chunk and passes
// 0xFFFFFFFF). The bounded reader reads zeros there, and only the last window
// can meet them (every earlier codeword ends before x <= cend), so that
// window is looked up again with the bits from cend on cleared when it
// reaches past cend.
template <bool kGlobalEsc>
__device__ __forceinline__ Adv decode_run_il(TileRef below, const Tables& tb, uint32_t p,
                                             uint32_t x, uint32_t cend, const IlSlot& sl) {
    *reinterpret_cast<uint32_t*>(sl.slots + (sl.wblk | sl.lane4)) = 0u;
    if (p >= x) return {p, 0u};
    uint32_t qa = sl.wblk;
    const Reader rd = reader_at(below, p);
    Step s = lookup<true>(below, tb, rd.p, rd.sh, rd.pair);
    uint32_t syms, adv, c;
    take<kGlobalEsc>(tb, s, &syms, &adv, &c);
    uint32_t pn = s.p + adv;
    while (pn < x) {
        Step t = lookup<false>(below, tb, pn, pn - s.m, s.next);
        slot_put_il(sl, qa, syms);
        qa += c << 6;
        // c's last use in this step: the next step's c can take its register.
        asm volatile("" : "+v"(qa), "+v"(c));
        t.syms = tb.syms[t.idx];
        s = t;
        take<kGlobalEsc>(tb, s, &syms, &adv, &c);
        pn = s.p + adv;
    }
    // The last window's start, from pn (s.p itself is then not needed past
    // the loop, and pn and s.p share a register in it).
    const uint32_t sp = pn - adv;
    if (cend - sp < 16u) {
        const uint32_t w = s.w & ~(0xFFFFFFFFu >> (cend - sp));
        const uint32_t idx = w >> (32 - kWinBits);
        const uint32_t meta = tb.meta[idx];
        syms = tb.syms[idx];
        adv = meta & 31u;
        c = meta >> 5;
        if (adv == 0) {
            syms = escape<kGlobalEsc>(tb, syms, w, &adv);
            c = 1;
        }
    }
    uint32_t kept;  // 1..4
    const uint32_t e = cut_window(tb, sp, sp + adv, syms, c, x, &kept);
    slot_put_il(sl, qa, syms & (0xFFFFFFFFu >> (32u - 8u * kept)));
    return {e, ((qa - sl.wblk) >> 6) + kept};
}

// Where to load the 4 bytes from packed-buffer byte A (A below the buffer
// size): A itself, or the last whole word of the buffer (`last` = size - 4)
// when A is within 3 bytes of its end; the word is then shifted right by
// A - word_at(A) bytes.
__device__ __forceinline__ uint32_t word_at(uint32_t A, uint32_t last) {
    return A < last ? A : last;
}

__device__ __forceinline__ uint32_t load_u32(const uint8_t* p) {
    uint32_t v;
    __builtin_memcpy(&v, p, 4);  // unaligned 4-byte load
    return v;
}

// Bytes b..b+3 of a chunk read one by one (zero at or past its end), for a
// packed buffer of fewer than 4 bytes.
__device__ __forceinline__ uint32_t load_bytes(const uint8_t* cbytes, int64_t nb, int64_t b) {
    uint32_t v = 0;
    for (int64_t k = 0; k < 4 && b + k < nb; ++k) v |= static_cast<uint32_t>(cbytes[b + k]) << (8 * k);
    return v;
}

// Big-endian stream word with the bytes at or past the chunk end zeroed.
// (Chunk byte offsets and lengths are below 2^31.)
__device__ __forceinline__ uint32_t be_word(uint32_t v, uint32_t nb, uint32_t b) {
    if (b >= nb) return 0u;
    const uint32_t left = nb - b;
    if (left < 4) v &= (1u << (8 * left)) - 1u;
    return __builtin_bswap32(v);
}

// One sub-group's share of an item: which chunk, where its bytes are, how
// many output symbols it has and in how many rounds it is decoded.
struct Job {
    int32_t d;     // tensor; -1 past the last item
    uint32_t lg;   // log2 of threads per chunk
    uint32_t S;    // segment bits
    int64_t c;     // chunk index
    uint32_t off;  // chunk byte offset in the packed buffer
    uint32_t nb;   // chunk bytes
    uint32_t lim;  // output symbols of the chunk
    uint32_t nr;   // rounds
    uint32_t ib;   // index build: the chunk's first segment, or kNoIndex
    uint32_t r0;   // the item's rounds: r0 .. r1 - 1 of the chunk's
    uint32_t r1;
    int32_t half;  // kWholeChunk, or which half of a split chunk (LaunchArgs)
    uint32_t slot; // a split chunk's handoff record
};

// Job::half.
enum Half : int32_t {
    kWholeChunk = 0,
    kFirstHalf = 1,   // rounds 0 .. nr/2 - 1; hands its state over at the end
    kSecondHalf = 2,  // rounds nr/2 .. nr - 1; takes the state over first
    kNoHalf = 3,      // second half of a chunk of fewer than 2 rounds: nothing
};

// Index build: whether the plan step gave tensor T's index its chunk bases
// and found room for every entry (entries are written only then). The same
// for every sub-group of an item.
__device__ __forceinline__ bool index_build_ready(const DevTensor& T) {
    const uint8_t* ix = uniform(T.index);
    if (ix == nullptr) return false;
    const auto* h = (const __attribute__((address_space(4))) IndexHeader*)(ix);
    return h->magic == kIndexMagic && h->ok == 1u;
}

// kLg > 0: every tensor of the launch has 1 << kLg threads per chunk.
template <int kMode, uint32_t kLg>
__device__ __forceinline__ Job make_job(const LaunchArgs& args, int64_t item, uint32_t tid) {
    Job J{-1, 0u, kMaxSegBits, 0, 0u, 0u, 0u, 0u, kNoIndex, 0u, 0u, kWholeChunk, 0u};
    if (item >= args.total_items) return J;
    // Split chunk k (chunk item split_first + k): its first half is item k,
    // its second half item split_first + n_split + k; the chunk items before
    // split_first are items n_split .. split_first + n_split - 1.
    if (args.n_split > 0) {
        if (item < args.n_split) {
            J.half = kFirstHalf;
            J.slot = static_cast<uint32_t>(item);
            item += args.split_first;
        } else if (item < args.split_first + args.n_split) {
            item -= args.n_split;
        } else {
            J.half = kSecondHalf;
            J.slot = static_cast<uint32_t>(item - args.split_first - args.n_split);
            item = args.split_first + J.slot;
        }
    }
    int d = 0;
    while (d + 1 < args.n_tensors && item >= args.t[d + 1].item_begin) ++d;
    const DevTensor& T = args.t[d];
    J.d = d;
    J.lg = kLg > 0 ? kLg : static_cast<uint32_t>(__ffs(T.tpc) - 1);
    const uint32_t n_groups = kThreads >> J.lg;
    J.c = (item - T.item_begin) * n_groups + (tid >> J.lg);
    // Segment length: at most kSlotCap codewords of the shortest length.
    J.S = segment_bits(header_of(uniform(T.table))->min_len);
    // Decodes never use the index here (segment runs do).
    const bool use_ix = kMode == kModeIndex && index_build_ready(T);
    const uint8_t* const ixp = use_ix ? uniform(T.index) : nullptr;
    const __attribute__((address_space(4))) uint32_t* ix_base =
        (const __attribute__((address_space(4))) uint32_t*)(ixp + sizeof(IndexHeader));
    // A wave holds 64 >> lg sub-groups (one when lg >= 6), on consecutive
    // chunks. Their offsets and lengths come through scalar loads, so no wait
    // for them waits for the vector stores in flight; each lane keeps its own.
    const int64_t c_wave = (item - T.item_begin) * n_groups + (uniform(tid & ~63u) >> J.lg);
    const uint32_t per_wave = J.lg >= 6 ? 1u : 64u >> J.lg;
    int64_t off = 0, nb = 0;
    uint32_t ib = 0;
#pragma unroll
    for (uint32_t k = 0; k < 64 / kMinTpc; ++k) {
        if (k < per_wave && c_wave + k < T.n_jobs) {
            const int64_t o = load_uniform(T.offsets + c_wave + k);
            const int64_t n = load_uniform(T.nbytes + c_wave + k);
            const uint32_t b = use_ix ? ix_base[c_wave + k] : 0u;
            if (J.c == c_wave + k) {
                off = o;
                nb = n;
                ib = b;
            }
        }
    }
    // kNoIndex marks "no index" for the whole item, so no entry may equal it.
    J.ib = use_ix ? (ib < kNoIndex ? ib : kNoIndex - 1u) : kNoIndex;
    if (J.c < T.n_jobs) {
        off = off < 0 ? 0 : (off > T.packed_nbytes ? T.packed_nbytes : off);
        nb = nb < 0 ? 0 : (nb > T.packed_nbytes - off ? T.packed_nbytes - off : nb);
        int64_t lim = T.n_symbols - J.c * T.chunk_size;
        lim = lim < 0 ? 0 : (lim > T.chunk_size ? T.chunk_size : lim);
        J.off = static_cast<uint32_t>(off);
        J.nb = static_cast<uint32_t>(nb);
        J.lim = static_cast<uint32_t>(lim);
        const int64_t round_bits = static_cast<int64_t>(J.S) << J.lg;
        J.nr = static_cast<uint32_t>((static_cast<int64_t>(nb) * 8 + round_bits - 1) / round_bits);
    }
    J.r1 = J.nr;
    if (J.half != kWholeChunk) {
        // A chunk of fewer than 2 rounds is not split: its first half takes it whole.
        const uint32_t h = J.nr / 2;
        if (h == 0) {
            if (J.half == kFirstHalf) {
                J.half = kWholeChunk;
            } else {
                J.half = kNoHalf;
                J.r0 = J.nr;
            }
        } else if (J.half == kFirstHalf) {
            J.r1 = h;
        } else {
            J.r0 = h;
        }
    }
    return J;
}

// Bits of round r of a job (0 when the job has no round r).
__device__ __forceinline__ uint32_t round_len(const Job& J, uint32_t r) {
    if (r >= J.nr) return 0u;
    const int64_t round_bits = static_cast<int64_t>(J.S) << J.lg;
    const int64_t left = static_cast<int64_t>(J.nb) * 8 - r * round_bits;
    return static_cast<uint32_t>(left < round_bits ? left : round_bits);
}

// A thread's stream words of one round, in flight in registers until they
// are written to the LDS tile: words k * tpc + i of the round.
struct Fetch {
    uint32_t raw[kTileBatch];
};

// The part of tensor T's index at [at, at + n) as a buffer (reads past it
// return 0, writes past it are dropped).
__device__ __forceinline__ __amdgpu_buffer_rsrc_t index_part(const DevTensor& T, uint64_t at,
                                                             uint64_t n) {
    const uint64_t lim = T.index_n32;
    const uint64_t a = at < lim ? at : lim;
    const uint64_t m = n < lim - a ? n : lim - a;
    return buffer_of(T.index + a, static_cast<uint32_t>(m));
}

// Word 0 of sub-group g's tile (the tile is filled downwards, see Reader).
__device__ __forceinline__ uint32_t* tile_top(uint32_t* s_tile, uint32_t g, uint32_t lg) {
    const uint32_t words = kTileWords >> (kLgThreads - lg);
    return s_tile + g * words + words - 1;
}

// Packed-buffer byte offsets fit 32 bits: chunk offsets and sizes are int32.
__device__ __forceinline__ uint32_t last_word(const DevTensor& T) {
    return T.packed_n32 - 4;  // packed_nbytes >= 4 outside the tiny-buffer kernel
}

// kTiny: the packed buffer has fewer than 4 bytes, so its words are read
// byte by byte. Such tensors go to a kernel of their own, which keeps these
// loads and their waits out of every other kernel's round loop.
// kLg: threads per chunk as the kernel's (0: the job's own).
template <int kMode, bool kTiny, uint32_t kLg>
__device__ __forceinline__ void fetch_issue(Fetch& F, const LaunchArgs& args, const Job& J,
                                            uint32_t r, uint32_t tid) {
    if (round_len(J, r) == 0) return;
    const DevTensor& T = args.t[J.d];
    const uint32_t lg = kLg > 0 ? kLg : J.lg;
    const uint32_t tpc = 1u << lg;
    const uint32_t b0 = ((r * J.S) << lg) / 8 + 4 * (tid & (tpc - 1));
    // All words are requested before any is used; words past the chunk read
    // an in-buffer word and are zeroed when written.
    if (!kTiny) {
        const __amdgpu_buffer_rsrc_t rs = buffer_of(T.packed, T.packed_n32);
        const uint32_t last = last_word(T);
        const uint32_t A0 = J.off + b0;
#pragma unroll
        for (uint32_t k = 0; k < kTileBatch; ++k)
            F.raw[k] = __builtin_amdgcn_raw_buffer_load_b32(rs, word_at(A0 + 4 * k * tpc, last), 0, 0);
    } else {
#pragma unroll
        for (uint32_t k = 0; k < kTileBatch; ++k)
            F.raw[k] = load_bytes(T.packed + J.off, J.nb, b0 + 4 * k * tpc);
    }
}

// Marks v as used here, so every load into it has completed by this point
// on every path. The vector-memory counter is in order: a load still pending
// when its register is loaded again next round would make that round wait
// for every store issued in between.
__device__ __forceinline__ void consume(uint32_t v) { asm volatile("" ::"v"(v)); }

template <bool kTiny, uint32_t kLg>
__device__ __forceinline__ void fetch_commit(const Fetch& F, const LaunchArgs& args, const Job& J,
                                             uint32_t r, uint32_t tid, uint32_t* s_tile) {
#pragma unroll
    for (uint32_t k = 0; k < kTileBatch; ++k) consume(F.raw[k]);
    const uint32_t RB = round_len(J, r);
    if (RB == 0) return;
    const DevTensor& T = args.t[J.d];
    const uint32_t lg = kLg > 0 ? kLg : J.lg;
    const uint32_t tpc = 1u << lg;
    const uint32_t i = tid & (tpc - 1);
    uint32_t* top = tile_top(s_tile, tid >> lg, lg);
    const uint32_t last = last_word(T);
    const uint32_t b0 = ((r * J.S) << lg) / 8;
    const uint32_t nw = (RB + 31) / 32 + 3;
    // Words below nin lie wholly inside the chunk (b0 + 4 j + 4 <= nb).
    const uint32_t nin = J.nb > b0 ? (J.nb - b0) / 4 : 0u;
#pragma unroll
    for (uint32_t k = 0; k < kTileBatch; ++k) {
        const uint32_t j = k * tpc + i;
        if (j >= nw) continue;
        const uint32_t b = b0 + 4 * j;
        uint32_t v = F.raw[k];
        // A word wholly inside the chunk was loaded from its own address
        // (A + 4 <= off + nb <= buffer size): only its byte order changes.
        if (j < nin) {
            *(top - j) = __builtin_bswap32(v);
            continue;
        }
        if (!kTiny) {
            // Within the chunk A - word_at(A, last) is 0..3; words at or past
            // its end are zeroed below, whatever the shift.
            const uint32_t A = J.off + b;
            v >>= 8 * ((A - word_at(A, last)) & 3u);
        }
        *(top - j) = be_word(v, J.nb, b);
    }
}

// Cross-lane moves through DPP (data-parallel primitives: the VALU reads a
// neighbour lane's operand), with no LDS round trip. Lanes whose source lies
// outside the pattern, or whose row is masked off, read 0. Controls:
// row_shr:n = 0x110 + n (within rows of 16 lanes), wave_shr:1 = 0x138,
// row_bcast:15 = 0x142 (lane 15 of each row to the next row), row_bcast:31 =
// 0x143 (lane 31 to rows 2 and 3).
template <int kCtrl, int kRowMask = 0xF>
__device__ __forceinline__ uint32_t dpp(uint32_t v) {
    return static_cast<uint32_t>(
        __builtin_amdgcn_update_dpp(0, static_cast<int>(v), kCtrl, kRowMask, 0xF, true));
}

// Inclusive prefix sum of v over the wave (every lane active).
__device__ __forceinline__ uint32_t wave_scan_incl(uint32_t v) {
    uint32_t x = v;
    x += dpp<0x111>(x);
    x += dpp<0x112>(x);
    x += dpp<0x114>(x);
    x += dpp<0x118>(x);
    x += dpp<0x142, 0xA>(x);
    x += dpp<0x143, 0xC>(x);
    return x;
}

// Inclusive prefix sum over the wave of the fp32 value with bits v (every
// lane active); lane 63 ends with the total.
__device__ __forceinline__ uint32_t wave_scan_incl_f32(uint32_t v) {
    float x = __uint_as_float(v);
    x += __uint_as_float(dpp<0x111>(__float_as_uint(x)));
    x += __uint_as_float(dpp<0x112>(__float_as_uint(x)));
    x += __uint_as_float(dpp<0x114>(__float_as_uint(x)));
    x += __uint_as_float(dpp<0x118>(__float_as_uint(x)));
    x += __uint_as_float(dpp<0x142, 0xA>(__float_as_uint(x)));
    x += __uint_as_float(dpp<0x143, 0xC>(__float_as_uint(x)));
    return __float_as_uint(x);
}

// v of the lane below (0 in lane 0; every lane active).
__device__ __forceinline__ uint32_t lane_below(uint32_t v) { return dpp<0x138>(v); }

__device__ __forceinline__ uint32_t block_scan_excl(uint32_t v, uint32_t* s_wsum) {
    const int lane = threadIdx.x & 63;
    const int w = threadIdx.x >> 6;
    const uint32_t x = wave_scan_incl(v);
    if (lane == 63) s_wsum[w] = x;
    __syncthreads();
    uint32_t pre = 0;
#pragma unroll
    for (int i = 0; i < kWaves; ++i) pre += i < w ? s_wsum[i] : 0u;
    return pre + x - v;
}

// bf16 bits ((sm & 0x80) << 8) | (e << 7) | (sm & 0x7F), the closed form of
// _recombine (compressed_store.py:94-114), for the four elements whose
// sign/mantissa and exponent bytes are the bytes of `sm4` and `e4`: elements
// 0 and 1 in .x, 2 and 3 in .y. A bf16's low byte is e's bit 0 over sm's bits
// 6..0, its high byte sm's bit 7 over e's bits 7..1: both for all four
// elements with one shift and one bit select each, then one byte permutation
// per pair interleaves them (six instructions; a pair at a time took eight).
__device__ __forceinline__ uint2 bf16_quad(uint32_t sm4, uint32_t e4) {
    const uint32_t lo = ((e4 << 7) & 0x80808080u) | (sm4 & 0x7F7F7F7Fu);  // low bytes
    const uint32_t hi = (sm4 & 0x80808080u) | ((e4 >> 1) & 0x7F7F7F7Fu);  // high bytes
    // {hi, lo} as bytes 7..0: element j's low byte is byte j, its high byte j + 4.
    return make_uint2(__builtin_amdgcn_perm(hi, lo, 0x05010400u), __builtin_amdgcn_perm(hi, lo, 0x07030602u));
}

__device__ __forceinline__ uint16_t bf16_one(uint32_t sm, uint32_t e) {
    return static_cast<uint16_t>(((sm & 0x80u) << 8) | (e << 7) | (sm & 0x7Fu));
}

__device__ __forceinline__ float bf16_to_f32(uint32_t bits16) {
    return __uint_as_float(bits16 << 16);
}

// Output element el from its exponent e (elements past the tensor are
// dropped).
template <int kMode>
__device__ __forceinline__ void store_one(const DevTensor& T, const GemvArgs& G, int64_t el,
                                          uint32_t e) {
    if (el < 0 || el >= T.n_symbols) return;
    if (kMode == kModeU8) {
        static_cast<uint8_t*>(T.out)[el] = static_cast<uint8_t>(e);
    } else if (kMode == kModeBf16) {
        static_cast<uint16_t*>(T.out)[el] = bf16_one(T.sm[el], e);
    } else if (kMode == kModeGemv || kMode == kModeGemv1 || is_gemm(kMode)) {
        const float w = bf16_to_f32(bf16_one(T.sm[el], e));
        const uint32_t row = static_cast<uint32_t>(el / G.cols);
        const uint32_t col = static_cast<uint32_t>(el - static_cast<int64_t>(row) * G.cols);
        for (int b = 0; b < G.batch; ++b)
            atomicAdd(G.y + static_cast<int64_t>(b) * G.rows + row,
                      w * bf16_to_f32(G.x[static_cast<int64_t>(b) * G.cols + col]));
    }
}

// Sign/mantissa bytes of the vector groups a thread stores in one round
// (groups k * tpc + i of the round), requested ahead of use.
template <int kMode>
struct SmBatch {
    uint2 v[needs_sm(kMode) && kMode != kModeGemmRows ? kSmAhead : 1];
};

// Buffer loads (zero past the tensor's last byte), so the batch needs no
// clamping and is issued back to back; the batch offset is a scalar.
template <int kMode, int kGroup>
// `limit`: no byte at or past it is needed (the loads there return zero
// without reading memory).
__device__ __forceinline__ void sm_issue(SmBatch<kMode>& B, const DevTensor& T, int64_t a0,
                                         uint32_t i, uint32_t tpc, uint32_t limit = 0xFFFFFFFFu) {
    // (kModeGemmRows reads them where its matrix tiles want them.)
    if (!needs_sm(kMode) || kMode == kModeGemmRows || kGroup == 1) return;
    const uint32_t n = static_cast<uint32_t>(T.n_symbols);
    const __amdgpu_buffer_rsrc_t rs = buffer_of(T.sm, n < limit ? n : limit);
    const uint32_t v0 = static_cast<uint32_t>(a0) + i * kGroup;
#pragma unroll
    for (uint32_t k = 0; k < kSmAhead; ++k) {
        const auto d = __builtin_amdgcn_raw_buffer_load_b64(rs, v0, k * tpc * kGroup, 0);
        B.v[k] = make_uint2(d[0], d[1]);
    }
}

typedef __bf16 bf16x2 __attribute__((ext_vector_type(2)));

// c + the products of 8 bf16 weights and 8 bf16 x values, in fp32
// (v_dot2c_f32_bf16: two products per instruction).
__device__ __forceinline__ float dot8_acc(const uint4& w, const uint4& x, float c) {
    c = __builtin_amdgcn_fdot2_f32_bf16(__builtin_bit_cast(bf16x2, w.x),
                                        __builtin_bit_cast(bf16x2, x.x), c, false);
    c = __builtin_amdgcn_fdot2_f32_bf16(__builtin_bit_cast(bf16x2, w.y),
                                        __builtin_bit_cast(bf16x2, x.y), c, false);
    c = __builtin_amdgcn_fdot2_f32_bf16(__builtin_bit_cast(bf16x2, w.z),
                                        __builtin_bit_cast(bf16x2, x.z), c, false);
    return __builtin_amdgcn_fdot2_f32_bf16(__builtin_bit_cast(bf16x2, w.w),
                                           __builtin_bit_cast(bf16x2, x.w), c, false);
}

// Add the wave's per-lane sums s[b] (b < nb) to y[b][row]: one wave sum and
// one atomic (from lane 63) per batch row.
template <int kB>
__device__ __forceinline__ void gemv_flush_lanes(const GemvArgs& G, int nb, const float (&s)[kB],
                                                 uint32_t row) {
#pragma unroll
    for (int b = 0; b < kB; ++b) {
        if (b >= nb) break;
        const float t = __uint_as_float(wave_scan_incl_f32(__float_as_uint(s[b])));
        if ((threadIdx.x & 63) == 63 && t != 0.0f)
            atomicAdd(G.y + static_cast<int64_t>(b) * G.rows + row, t);
    }
}

// Adds each live lane's products p[b] (b < nb) to y[b][row of the lane] with
// one wave sum and one atomic per distinct row, instead of one atomic per
// lane. Called with every lane of the wave; dead lanes pass live = false.
template <int kB>
__device__ __forceinline__ void gemv_rows_add(const GemvArgs& G, int nb, const float (&p)[kB],
                                              bool live, uint32_t row) {
    uint64_t left = __ballot(live);  // live lanes whose products are not yet added
    while (left != 0) {
        const uint32_t rr = __builtin_amdgcn_readlane(row, __builtin_ctzll(left));
        const bool mine = live && row == rr;
        left &= ~__ballot(mine);
#pragma unroll
        for (int b = 0; b < kB; ++b) {
            if (b >= nb) break;
            const float sum = __uint_as_float(wave_scan_incl_f32(__float_as_uint(mine ? p[b] : 0.0f)));
            if ((threadIdx.x & 63) == 63 && sum != 0.0f)
                atomicAdd(G.y + static_cast<int64_t>(b) * G.rows + rr, sum);
        }
    }
}

// Column col moved on by step elements of a row of cols.
__device__ __forceinline__ void advance_col(uint32_t& col, uint32_t step, uint32_t cols) {
    col += step;
    while (col >= cols) col -= cols;
}

// The 8 x values at column col of each batch row b < kB (col < cols, and
// col % 8 == 0 with a 16-byte-aligned x, so the reads are aligned). The
// buffer ends after the nb rows of x, so rows b >= nb read as zero. Every
// load is issued on every path: the compiler then counts them exactly, and
// a wait for one x vector's words does not become a wait for every load in
// flight.
template <int kB>
__device__ __forceinline__ void gemv_load_x(uint4 (&dst)[kB], const GemvArgs& G, int nb,
                                            uint32_t col) {
    if constexpr (kB == 1) {  // one x vector: a plain load (measured 1% faster)
        dst[0] = *reinterpret_cast<const uint4*>(G.x + col);
        return;
    }
    const uint32_t row_bytes = 2u * G.cols;
    const __amdgpu_buffer_rsrc_t rs = buffer_of(G.x, static_cast<uint32_t>(nb) * row_bytes);
#pragma unroll
    for (int b = 0; b < kB; ++b) {
        const auto d = __builtin_amdgcn_raw_buffer_load_b128(rs, 2u * col, b * row_bytes, 0);
        dst[b] = make_uint4(d[0], d[1], d[2], d[3]);
    }
}

// (row, col) of an element moved on by 4096 elements (step_rows rows and
// step_cols columns, step_cols < cols): one add and at most one wrap.
__device__ __forceinline__ void step_rc(uint32_t& row, uint32_t& col, const GemvArgs& G) {
    row += G.step_rows;
    col += G.step_cols;
    const bool wrap = col >= G.cols;
    col = wrap ? col - G.cols : col;
    row += wrap ? 1u : 0u;
}

// Fused GEMV over one staged round when the workgroup is one chunk (or a
// segment run). Thread i holds group i + 512 k, so at each step k wave w's
// 64 groups are the 512 consecutive elements from a0 + 8 (64 w + 512 k).
// Their first row and column are tracked for the whole wave as scalars,
// each lane's own as registers, both by step_rc (no division past the first
// step). Each lane keeps one fp32 sum per x vector and adds its 8 products
// with four v_dot2c_f32_bf16; the sums are reduced over the wave (DPP) and
// added to y with one atomic per x vector when the row changes. A step that
// crosses a row boundary (about 512 / cols of them) flushes the lanes of the
// first row and starts the next row's sums with the others. Only rows
// shorter than 512 elements take per-lane atomics. Dead lanes' products are
// dropped (not multiplied by zero), so an infinite x cannot make a NaN. x is
// requested kXAhead steps ahead of use for every x vector, and every
// vector's loads and products are unconditional (see gemv_load_x); G's x and
// y are those of the nb <= kB x vectors of this pass.
template <int kMode, int kGroup, int kB>
__device__ __forceinline__ void gemv_round_whole(const uint2 (&sm)[kStoreBatch], const GemvArgs& G,
                                                 int nb, const uint8_t* stage, uint32_t a0,
                                                 uint32_t nfull, uint32_t i, uint32_t v_lo) {
    static_assert(kThreads * kGroup == 4096, "step_rows / step_cols are for 4096 elements");
    constexpr uint32_t kXAhead = kB == 1 ? 3 : kGemvXAhead;
    constexpr uint32_t kSpan = 64 * kGroup;  // elements a wave holds at one step
    const uint32_t cols = G.cols;
    const uint32_t lane = i & 63;
    const uint32_t wave_first = uniform(i - lane);  // first thread of this wave
    const uint32_t wave_el = uniform(a0 + wave_first * kGroup);
    uint32_t er = wave_el / cols;  // row and column of the wave's first element
    uint32_t ec = wave_el - er * cols;
    const uint32_t lane_el = wave_el + lane * kGroup;
    uint32_t lr = lane_el / cols;  // row and column of this lane's group
    uint32_t lc = lane_el - lr * cols;
    uint32_t lr_ld = lr, lc_ld = lc;  // the same for the next step whose x is requested
    uint4 xq[kXAhead + 1][kB];
#pragma unroll
    for (uint32_t k = 0; k < kXAhead && k < kStoreBatch; ++k) {
        if (k > 0) step_rc(lr_ld, lc_ld, G);
        gemv_load_x<kB>(xq[k], G, nb, lc_ld);
    }
    float acc[kB];
#pragma unroll
    for (int b = 0; b < kB; ++b) acc[b] = 0.0f;
    uint32_t acc_row = 0xFFFFFFFFu;
#pragma unroll
    for (uint32_t k = 0; k < kStoreBatch; ++k) {
        if (k + kXAhead < kStoreBatch) {
            if (k + kXAhead > 0) step_rc(lr_ld, lc_ld, G);
            gemv_load_x<kB>(xq[(k + kXAhead) % (kXAhead + 1)], G, nb, lc_ld);
        }
        if (k > 0) {
            step_rc(er, ec, G);
            step_rc(lr, lc, G);
        }
        if (k * kThreads + wave_first >= nfull) break;  // this wave's groups are done
        const uint4(&xc)[kB] = xq[k % (kXAhead + 1)];
        const uint32_t v = k * kThreads + i;
        const bool live = v < nfull && v >= v_lo;
        const uint2 e = *reinterpret_cast<const uint2*>(stage + v * kGroup);
        uint4 w;
        const uint2 pa = bf16_quad(sm[k].x, e.x);
        const uint2 pb = bf16_quad(sm[k].y, e.y);
        w.x = pa.x;
        w.y = pa.y;
        w.z = pb.x;
        w.w = pb.y;
        if (ec + kSpan <= cols) {
            if (er != acc_row) {
                if (acc_row != 0xFFFFFFFFu) {
                    gemv_flush_lanes<kB>(G, nb, acc, acc_row);
#pragma unroll
                    for (int b = 0; b < kB; ++b) acc[b] = 0.0f;
                }
                acc_row = er;
            }
#pragma unroll
            for (int b = 0; b < kB; ++b) {
                const float t = dot8_acc(w, xc[b], acc[b]);
                acc[b] = live ? t : acc[b];
            }
        } else if (cols >= kSpan) {
            // Two rows: lanes below the boundary finish row er, the rest
            // start row er + 1.
            if (er != acc_row) {
                if (acc_row != 0xFFFFFFFFu) {
                    gemv_flush_lanes<kB>(G, nb, acc, acc_row);
#pragma unroll
                    for (int b = 0; b < kB; ++b) acc[b] = 0.0f;
                }
                acc_row = er;
            }
            const bool lo = lr == er;
            float p[kB];
#pragma unroll
            for (int b = 0; b < kB; ++b) {
                const float t = dot8_acc(w, xc[b], 0.0f);
                p[b] = live ? t : 0.0f;
                acc[b] += lo ? p[b] : 0.0f;
            }
            gemv_flush_lanes<kB>(G, nb, acc, er);
#pragma unroll
            for (int b = 0; b < kB; ++b) acc[b] = lo ? 0.0f : p[b];
            acc_row = er + 1;
        } else if (live) {
            // Rows shorter than a wave's 512 elements: per-lane atomics.
#pragma unroll
            for (int b = 0; b < kB; ++b) {
                if (b >= nb) break;
                atomicAdd(G.y + static_cast<int64_t>(b) * G.rows + lr, dot8_acc(w, xc[b], 0.0f));
            }
        }
    }
    if (acc_row != 0xFFFFFFFFu) gemv_flush_lanes<kB>(G, nb, acc, acc_row);
}

// ---------------------------------------------------------------------------
// Fused decode -> GEMM (kModeGemm, kModeGemmRows; whole-workgroup rounds):
// Y[t][r] += sum_c X[t][c] W[r][c] for t < G.batch <= 16, on
// v_mfma_f32_16x16x32_bf16. One MFMA takes a 16 x 32 tile of X (A: lane l
// holds X[l & 15][8 (l >> 4) .. + 7]) and the 32 x 16 tile of W^T over the
// same 32 columns and 16 rows of W (B: lane l holds W[row l & 15][the same 8
// columns]) and adds to a 16 x 16 tile of Y^T (D: lane l holds Y[4 (l >> 4)
// + k][row l & 15], k < 4). A round's weights are in natural order, a row of
// W after another, while the B operand wants 16 rows at the same columns;
// the waves take the 32-column slices of each 16-row tile of W the round
// touches, X from L2, and X is read once per slice for the rows of the tile
// the pass holds. Two ways to get there:
// - kModeGemm (rows of up to 8192 columns): each piece of 4 store steps
//   (2048 groups) is written to LDS as bf16 (sign/mantissa bytes requested
//   during the decode, one padding group per row so that the 16 rows a read
//   meets fall in different banks), then read as B operands: a pass per
//   piece, which holds 2 to 16 rows of W.
// - kModeGemmRows (longer rows, of which a piece holds one or two): one pass
//   per round, each lane reading its group's exponents from the stage and
//   their sign/mantissa bytes from memory (on the 5120x17408 layer, 8 rows of
//   x: 258 us against 379 us in pieces; on the 151936x5120 lm_head, 1157 us
//   against 990 us).
// Every wave keeps its partial D of the current 16-row tile in registers
// across passes and rounds; the waves' partials of a complete tile are summed
// in LDS and added to Y with one atomic per (row, x row).
// ---------------------------------------------------------------------------

typedef __bf16 bf16x8_t __attribute__((ext_vector_type(8)));
typedef float f32x4_t __attribute__((ext_vector_type(4)));

constexpr uint32_t kNoTile = 0xFFFFFFFFu;
constexpr uint32_t kGemmUnroll = 4;  // slices whose loads go out together
// Rows of more columns than this take kModeGemmRows.
constexpr int64_t kGemmPieceMaxCols = 8192;
constexpr uint32_t kGemmPieceSteps = 4;  // store steps a piece holds
constexpr uint32_t kGemmPieceGroups = kGemmPieceSteps * kThreads;
// Padding groups of a piece: one per row it touches, for rows of 64 groups
// or more (a row of fewer takes none: the reads then meet bank conflicts).
constexpr uint32_t kGemmPadMinGroups = 64;
constexpr uint32_t kGemmPieceBytes = 16 * (kGemmPieceGroups + kGemmPieceGroups / kGemmPadMinGroups + 2);
// The cross-wave sum of the partial tiles, after a piece in the stage.
constexpr uint32_t kGemmRedOffset = (kGemmPieceBytes + 255) / 256 * 256;
constexpr uint32_t kGemmRedBytes = kWaves * 64 * 16;

struct GemmAcc {
    f32x4_t d;       // this wave's partial sums of 16-row tile `tile`
    f32x4_t dp;      // those of tile `ptile`, complete, not yet added to Y
    uint32_t tile;   // kNoTile: none
    uint32_t ptile;  // kNoTile: none
};

__device__ __forceinline__ void gemm_acc_init(GemmAcc& A) {
    A.d = f32x4_t{0.0f, 0.0f, 0.0f, 0.0f};
    A.dp = A.d;
    A.tile = kNoTile;
    A.ptile = kNoTile;
}

// Partial sums d of tile `tile`, this wave's alone, to Y (one atomic per
// entry; rows no weight of the wave met hold exactly zero and are skipped).
__device__ __forceinline__ void gemm_add_wave(const f32x4_t& d, uint32_t tile, const GemvArgs& G) {
    const uint32_t lane = threadIdx.x & 63u;
    const uint32_t row = 16 * tile + (lane & 15u);
#pragma unroll
    for (uint32_t k = 0; k < 4; ++k) {
        const uint32_t t = 4 * (lane >> 4) + k;
        if (t < static_cast<uint32_t>(G.batch) && row < G.rows && d[k] != 0.0f)
            atomicAdd(G.y + static_cast<int64_t>(t) * G.rows + row, d[k]);
    }
}

// The waves' partial sums d of tile `tile`, summed in LDS, to Y; every
// thread calls it (it holds barriers), with the stage's kGemmRedBytes bytes
// from kGemmRedOffset free.
__device__ __forceinline__ void gemm_add_block(const f32x4_t& d, uint32_t tile, const GemvArgs& G,
                                               uint8_t* stage) {
    const uint32_t tid = threadIdx.x;
    const uint32_t lane = tid & 63u, w = tid >> 6;
    f32x4_t* const red = reinterpret_cast<f32x4_t*>(stage + kGemmRedOffset);
    red[w * 64 + lane] = d;
    __syncthreads();
    if (tid < 256) {
        // Entry k of lane l2 of every wave: Y[4 (l2 >> 4) + k][16 tile + (l2 & 15)].
        const uint32_t l2 = tid >> 2, k = tid & 3u;
        const float* const f = reinterpret_cast<const float*>(red) + tid;
        float sum = 0.0f;
#pragma unroll
        for (uint32_t v = 0; v < static_cast<uint32_t>(kWaves); ++v) sum += f[v * 256];
        const uint32_t t = 4 * (l2 >> 4) + k;
        const uint32_t row = 16 * tile + (l2 & 15u);
        if (t < static_cast<uint32_t>(G.batch) && row < G.rows && sum != 0.0f)
            atomicAdd(G.y + static_cast<int64_t>(t) * G.rows + row, sum);
    }
    __syncthreads();  // the sums are read before the area is written again
}

// The tile the wave's partial sums belong to, when the workgroup's elements
// end (every thread calls it).
__device__ __forceinline__ void gemm_finish(GemmAcc& A, const GemvArgs& G, uint8_t* stage) {
    if (A.ptile != kNoTile) gemm_add_block(A.dp, A.ptile, G, stage);
    if (A.tile != kNoTile) gemm_add_block(A.d, A.tile, G, stage);
    gemm_acc_init(A);
}

// kModeGemm: one round's groups [0, nfull) (W groups a0 / 8 ...), their
// sign/mantissa bytes in sm (group k * kThreads + tid at k), exponents in the
// stage, written to LDS as bf16 a piece of kGemmPieceSteps store steps at a
// time. The stage is overwritten but for the bytes past the round's groups,
// which the caller carries into the next round: those are put back.
__device__ __forceinline__ void gemm_round_pieces(const uint2 (&sm)[kStoreBatch], const GemvArgs& G,
                                                  uint8_t* stage, uint32_t a0, uint32_t nfull,
                                                  uint32_t tid, GemmAcc& A) {
    const uint32_t cols = G.cols;
    const uint32_t cg = cols / 8;  // groups a row
    const uint32_t lane = tid & 63u, w = tid >> 6;
    const uint32_t nb = static_cast<uint32_t>(G.batch);
    uint2 ev[kStoreBatch];
#pragma unroll
    for (uint32_t k = 0; k < kStoreBatch; ++k)
        ev[k] = *reinterpret_cast<const uint2*>(stage + (k * kThreads + tid) * 8);
    const uint2 keep0 = reinterpret_cast<const uint2*>(stage + nfull * 8)[0];
    const uint2 keep1 = reinterpret_cast<const uint2*>(stage + nfull * 8)[1];
    __syncthreads();  // every exponent is read before the first piece is written
    const uint32_t pad = cg >= kGemmPadMinGroups ? 1u : 0u;
    const uint32_t g0 = a0 / 8;
    const uint32_t ns = (cg + 3) / 4;  // 32-column slices a row
    const __amdgpu_buffer_rsrc_t xr = buffer_of(G.x, nb * cols * 2u);
    const uint32_t q = lane >> 4, n = lane & 15u;
#pragma unroll
    for (uint32_t p = 0; p < (kStoreBatch + kGemmPieceSteps - 1) / kGemmPieceSteps; ++p) {
        const uint32_t vb = p * kGemmPieceGroups;
        if (vb >= nfull) break;
        const uint32_t ve = nfull - vb < kGemmPieceGroups ? nfull : vb + kGemmPieceGroups;
        const uint32_t rb = (g0 + vb) / cg;      // the piece's first row
        const uint32_t re = (g0 + ve - 1) / cg;  // and last
        // The piece's weights to LDS, bf16, group v at v - vb plus the rows
        // before its own.
#pragma unroll
        for (uint32_t kk = 0; kk < kGemmPieceSteps; ++kk) {
            const uint32_t k = p * kGemmPieceSteps + kk;
            if (k >= kStoreBatch) break;
            const uint32_t v = k * kThreads + tid;
            if (v < ve) {
                uint4 wv;
                const uint2 pa = bf16_quad(sm[k].x, ev[k].x);
                const uint2 pb = bf16_quad(sm[k].y, ev[k].y);
                wv.x = pa.x;
                wv.y = pa.y;
                wv.z = pb.x;
                wv.w = pb.y;
                const uint32_t row = (g0 + v) / cg;
                *reinterpret_cast<uint4*>(stage + 16 * (v - vb + pad * (row - rb))) = wv;
            }
        }
        __syncthreads();
        for (uint32_t t = rb / 16; t <= re / 16; ++t) {
            if (t != A.tile) {
                if (A.tile != kNoTile) gemm_add_block(A.d, A.tile, G, stage);
                A.d = f32x4_t{0.0f, 0.0f, 0.0f, 0.0f};
                A.tile = t;
            }
            const uint32_t row = 16 * t + n;
            // Slices s = w, w + kWaves, ... of this tile, kGemmUnroll at a time.
            for (uint32_t s0 = w; s0 < ns; s0 += kGemmUnroll * kWaves) {
                uint4 xa[kGemmUnroll], wb[kGemmUnroll];
#pragma unroll
                for (uint32_t u = 0; u < kGemmUnroll; ++u) {
                    const uint32_t sl = s0 + u * kWaves;
                    const uint32_t j = 4 * sl + q;  // the lane's column group
                    const bool col_ok = sl < ns && j < cg;
                    // X row n (zero past the batch: out of the buffer's range).
                    const uint32_t xo = col_ok && n < nb ? n * cols * 2u + 16u * j : 0xFFFFFFF0u;
                    const auto xv = __builtin_amdgcn_raw_buffer_load_b128(xr, xo, 0, 0);
                    xa[u] = make_uint4(xv[0], xv[1], xv[2], xv[3]);
                    const uint32_t gv = row * cg + j;  // W group of this lane (rows * cols < 2^31)
                    const bool ok = col_ok && gv >= g0 + vb && gv < g0 + ve;
                    const uint32_t lo = ok ? 16u * (gv - g0 - vb + pad * (row - rb)) : 0u;
                    const uint4 bv = *reinterpret_cast<const uint4*>(stage + lo);
                    wb[u] = ok ? bv : make_uint4(0u, 0u, 0u, 0u);
                }
#pragma unroll
                for (uint32_t u = 0; u < kGemmUnroll; ++u)
                    A.d = __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(bf16x8_t, xa[u]),
                                                                  __builtin_bit_cast(bf16x8_t, wb[u]),
                                                                  A.d, 0, 0, 0);
            }
        }
        __syncthreads();  // the piece is read before the next one (or the carry) is written
    }
    if (tid == 0) {
        reinterpret_cast<uint2*>(stage + nfull * 8)[0] = keep0;
        reinterpret_cast<uint2*>(stage + nfull * 8)[1] = keep1;
    }
    __syncthreads();
}

// kModeGemmRows: one round's groups [0, nfull) (W groups a0 / 8 ...),
// exponents in the stage, read where the B operand wants them, with their
// sign/mantissa bytes from memory: X is read once per slice of the round
// (pieces would read it once per piece, and a piece of long rows holds one
// or two). Bytes past the round's groups (the partial group carried into the
// next round) are kept.
__device__ __forceinline__ void gemm_round_rows(const DevTensor& T, const GemvArgs& G, uint8_t* stage,
                                                uint32_t a0, uint32_t nfull, uint32_t tid, GemmAcc& A) {
    const uint32_t cols = G.cols;
    const uint32_t cg = cols / 8;  // groups a row
    const uint32_t lane = tid & 63u, w = tid >> 6;
    const uint32_t nb = static_cast<uint32_t>(G.batch);
    const uint32_t q = lane >> 4, n = lane & 15u;
    const uint32_t g0 = a0 / 8, ge = g0 + nfull;
    const uint32_t ns = (cg + 3) / 4;  // 32-column slices a row
    const __amdgpu_buffer_rsrc_t xr = buffer_of(G.x, nb * cols * 2u);
    const __amdgpu_buffer_rsrc_t sr = buffer_of(T.sm, static_cast<uint32_t>(T.n_symbols));
    if (nfull != 0) {
        const uint32_t t_lo = g0 / cg / 16, t_hi = (ge - 1) / cg / 16;
        for (uint32_t t = t_lo; t <= t_hi; ++t) {
            if (t != A.tile) {
                if (A.tile != kNoTile) {
                    // The wave's tile is complete: it waits for the block sum
                    // at the round's end (one waiting already: added now).
                    if (A.ptile != kNoTile) gemm_add_wave(A.dp, A.ptile, G);
                    A.dp = A.d;
                    A.ptile = A.tile;
                }
                A.d = f32x4_t{0.0f, 0.0f, 0.0f, 0.0f};
                A.tile = t;
            }
            const uint32_t row = 16 * t + n;
            // Slices s = w, w + kWaves, ... of this tile, kGemmUnroll at a
            // time; the loads of the next kGemmUnroll go out before this
            // step's products (X and the sign/mantissa bytes come from L2).
            auto issue = [&](uint32_t s0, uint4 (&xa)[kGemmUnroll], uint2 (&sm)[kGemmUnroll],
                             uint2 (&ex)[kGemmUnroll]) {
#pragma unroll
                for (uint32_t u = 0; u < kGemmUnroll; ++u) {
                    const uint32_t sl = s0 + u * kWaves;
                    const uint32_t j = 4 * sl + q;  // the lane's column group
                    const bool col_ok = sl < ns && j < cg;
                    // X row n (zero past the batch or the row: out of the buffer's range).
                    const uint32_t xo = col_ok && n < nb ? n * cols * 2u + 16u * j : 0xFFFFFFF0u;
                    const auto xv = __builtin_amdgcn_raw_buffer_load_b128(xr, xo, 0, 0);
                    xa[u] = make_uint4(xv[0], xv[1], xv[2], xv[3]);
                    const uint32_t gv = row * cg + j;  // W group of this lane (rows * cols < 2^31)
                    const bool ok = col_ok && gv >= g0 && gv < ge;
                    const auto sv = __builtin_amdgcn_raw_buffer_load_b64(sr, ok ? 8u * gv : 0xFFFFFFF8u, 0, 0);
                    sm[u] = make_uint2(sv[0], sv[1]);
                    const uint2 e = *reinterpret_cast<const uint2*>(stage + (ok ? 8u * (gv - g0) : 0u));
                    ex[u] = ok ? e : make_uint2(0u, 0u);
                }
            };
            for (uint32_t s0 = w; s0 < ns; s0 += kGemmUnroll * kWaves) {
                uint4 xa[kGemmUnroll];
                uint2 sm[kGemmUnroll], ex[kGemmUnroll];
                issue(s0, xa, sm, ex);
#pragma unroll
                for (uint32_t u = 0; u < kGemmUnroll; ++u) {
                    uint4 wb;
                    const uint2 pa = bf16_quad(sm[u].x, ex[u].x);
                    const uint2 pb = bf16_quad(sm[u].y, ex[u].y);
                    wb.x = pa.x;
                    wb.y = pa.y;
                    wb.z = pb.x;
                    wb.w = pb.y;
                    A.d = __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(bf16x8_t, xa[u]),
                                                                  __builtin_bit_cast(bf16x8_t, wb),
                                                                  A.d, 0, 0, 0);
                }
            }
        }
    }
    // Complete tiles to Y, summed over the waves in the stage once every
    // wave is done with it: the one waiting, and the current one when the
    // next round (which starts at group ge) begins past it.
    const bool done_cur = A.tile != kNoTile && ge / cg >= 16 * (A.tile + 1);
    if (A.ptile == kNoTile && !done_cur) return;
    const uint2 keep0 = reinterpret_cast<const uint2*>(stage + nfull * 8)[0];
    const uint2 keep1 = reinterpret_cast<const uint2*>(stage + nfull * 8)[1];
    __syncthreads();
    if (A.ptile != kNoTile) {
        gemm_add_block(A.dp, A.ptile, G, stage);
        A.ptile = kNoTile;
    }
    if (done_cur) {
        gemm_add_block(A.d, A.tile, G, stage);
        A.d = f32x4_t{0.0f, 0.0f, 0.0f, 0.0f};
        A.tile = kNoTile;
    }
    if (tid == 0) {
        reinterpret_cast<uint2*>(stage + nfull * 8)[0] = keep0;
        reinterpret_cast<uint2*>(stage + nfull * 8)[1] = keep1;
    }
    __syncthreads();
}

// Vector groups [0, nfull) of the staged round to output elements a0...;
// thread i of a sub-group of tpc takes groups i, i + tpc, ... kWhole: the
// sub-group is the whole workgroup, whose stage area is readable for every
// group a store batch can name, so the staged reads need no clamping.
// skip: group 0's first `skip` elements are another piece of work's (a
// segment run that starts inside a vector group); group 0's other elements
// are stored one by one, and the vector paths start at group 1.
template <int kMode, int kGroup, bool kWhole>
__device__ __forceinline__ void store_round(const SmBatch<kMode>& B, const DevTensor& T,
                                            const GemvArgs& G, const uint8_t* stage, int64_t a0,
                                            uint32_t nfull, uint32_t i, uint32_t tpc,
                                            uint32_t skip = 0, GemmAcc* gacc = nullptr) {
    if constexpr (kMode == kModeGemmRows) {
        // Whole-workgroup rounds without skipped elements only (the
        // speculative runs).
        static_assert(kWhole && kGroup == 8, "the fused GEMM takes whole-workgroup rounds");
        gemm_round_rows(T, G, const_cast<uint8_t*>(stage), static_cast<uint32_t>(a0), nfull, i, *gacc);
        return;
    }
    if (kGroup == 1) {
        for (uint32_t v = i; v < nfull; v += tpc) store_one<kMode>(T, G, a0 + v, stage[v]);
        return;
    }
    if (skip != 0 && nfull != 0 && i >= skip && i < static_cast<uint32_t>(kGroup))
        store_one<kMode>(T, G, a0 + i, stage[i]);
    const uint32_t v_lo = skip != 0 ? 1u : 0u;
    if (kMode == kModeU8) {
        for (uint32_t v = i < v_lo ? i + tpc : i; v < nfull; v += tpc)
            // Non-temporal, like the bf16 stores (2.8% faster on the layer).
            __builtin_nontemporal_store(
                *reinterpret_cast<const v4u32*>(stage + v * kGroup),
                reinterpret_cast<v4u32*>(static_cast<uint8_t*>(T.out) + a0 + static_cast<int64_t>(v) * kGroup));
        return;
    }
#pragma unroll
    for (uint32_t k = 0; k < kSmAhead; ++k) {
        consume(B.v[k].x);
        consume(B.v[k].y);
    }
    // Sign/mantissa of groups past the requested ones, for waves that have any.
    uint2 sm[kStoreBatch];
#pragma unroll
    for (uint32_t k = 0; k < kSmAhead; ++k) sm[k] = B.v[k];
    if (__ballot(kSmAhead * tpc + i < nfull) != 0) {
        const __amdgpu_buffer_rsrc_t rs = buffer_of(T.sm, static_cast<uint32_t>(T.n_symbols));
        const uint32_t v0 = static_cast<uint32_t>(a0) + i * kGroup;
#pragma unroll
        for (uint32_t k = kSmAhead; k < kStoreBatch; ++k) {
            const auto d = __builtin_amdgcn_raw_buffer_load_b64(rs, v0, k * tpc * kGroup, 0);
            sm[k] = make_uint2(d[0], d[1]);
        }
        // Waited for here, before any store is issued: a wait after the
        // stores would wait for them too.
#pragma unroll
        for (uint32_t k = kSmAhead; k < kStoreBatch; ++k) {
            consume(sm[k].x);
            consume(sm[k].y);
        }
    } else {
#pragma unroll
        for (uint32_t k = kSmAhead; k < kStoreBatch; ++k) sm[k] = make_uint2(0u, 0u);
    }
    if constexpr (kMode == kModeGemm) {
        static_assert(kWhole && kGroup == 8, "the fused GEMM takes whole-workgroup rounds");
        gemm_round_pieces(sm, G, const_cast<uint8_t*>(stage), static_cast<uint32_t>(a0), nfull, i, *gacc);
        return;
    }
    // All staged exponents are read (from always valid offsets) before any
    // is combined, so the LDS reads overlap.
    uint2 ev[kStoreBatch];
#pragma unroll
    for (uint32_t k = 0; k < kStoreBatch; ++k) {
        const uint32_t v = k * tpc + i;
        ev[k] = *reinterpret_cast<const uint2*>(stage + (kWhole || v < nfull ? v : 0u) * kGroup);
    }
    if (kMode == kModeBf16) {
        // Buffer stores: per-lane offset 2 * a0 + 16 i, the batch step as a
        // scalar offset (outputs are below 2^31 elements).
        const __amdgpu_buffer_rsrc_t rs =
            buffer_of(T.out, static_cast<uint32_t>(T.n_symbols) * 2u);
        const uint32_t vo = static_cast<uint32_t>(a0) * 2u + 16u * i;
#pragma unroll
        for (uint32_t k = 0; k < kStoreBatch; ++k) {
            const uint32_t v = k * tpc + i;
            if (v >= nfull || v < v_lo) continue;
            v4u32 o4;
            const uint2 pa = bf16_quad(sm[k].x, ev[k].x);
            const uint2 pb = bf16_quad(sm[k].y, ev[k].y);
            o4[0] = pa.x;
            o4[1] = pa.y;
            o4[2] = pb.x;
            o4[3] = pb.y;
            __builtin_amdgcn_raw_buffer_store_b128(o4, rs, vo, 16u * k * tpc, kCachePolicyNT);
        }
        return;
    }
    if constexpr (kWhole && (kMode == kModeGemv || kMode == kModeGemv1)) {
        constexpr int kB = kMode == kModeGemv1 ? 1 : kGemvMaxBatch;
        gemv_round_whole<kMode, kGroup, kB>(sm, G, kMode == kModeGemv1 ? 1 : G.batch, stage,
                                            static_cast<uint32_t>(a0), nfull, i, v_lo);
        return;
    }
    // Fused GEMV: each group's 8 weights (one matrix row, as cols % 8 == 0)
    // meet the 8 x values of their columns. When a wave's live groups at one
    // k lie in one row (the usual case), each lane adds its products to its
    // own fp32 sum per x vector (v_dot2c_f32_bf16), and the sums are reduced
    // over the wave and added to y when the row changes. A step whose live
    // groups span several rows adds one wave sum per distinct row. x is
    // requested kXAhead groups ahead of use (a group's column is always below
    // cols, so every read is in bounds, live group or not); loads and
    // products are unconditional for every x vector (see gemv_load_x).
    constexpr int kB = kMode == kModeGemv1 ? 1 : kGemvMaxBatch;
    constexpr uint32_t kXAhead = kMode == kModeGemv1 ? 3 : kGemvXAhead;
    const int nb = kMode == kModeGemv1 ? 1 : G.batch;
    const uint32_t cols = G.cols;
    const uint32_t el = static_cast<uint32_t>(a0) + i * kGroup;  // element of group k = 0
    uint32_t row = el / cols;
    uint32_t col = el - row * cols;
    const uint32_t step = tpc * kGroup;
    uint4 xq[kXAhead + 1][kB];
    uint32_t col_ld = col;  // column of the next group whose x is requested
#pragma unroll
    for (uint32_t k = 0; k < kXAhead && k < kStoreBatch; ++k) {
        if (k > 0) advance_col(col_ld, step, cols);
        gemv_load_x<kB>(xq[k], G, nb, col_ld);
    }
    float acc[kB];
#pragma unroll
    for (int b = 0; b < kB; ++b) acc[b] = 0.0f;
    uint32_t acc_row = 0xFFFFFFFFu;
#pragma unroll
    for (uint32_t k = 0; k < kStoreBatch; ++k) {
        if (k + kXAhead < kStoreBatch) {
            if (k + kXAhead > 0) advance_col(col_ld, step, cols);
            gemv_load_x<kB>(xq[(k + kXAhead) % (kXAhead + 1)], G, nb, col_ld);
        }
        if (k > 0) {
            col += step;
            while (col >= cols) {
                col -= cols;
                ++row;
            }
        }
        const uint4(&xc)[kB] = xq[k % (kXAhead + 1)];
        const uint32_t v = k * tpc + i;
        const bool live = v < nfull && v >= v_lo;
        const uint64_t lm = __ballot(live);
        if (lm == 0) continue;
        // Staged exponents read here rather than all at once: registers.
        const uint2 e = *reinterpret_cast<const uint2*>(stage + (kWhole || live ? v : 0u) * kGroup);
        uint4 w;
        const uint2 pa = bf16_quad(sm[k].x, e.x);
        const uint2 pb = bf16_quad(sm[k].y, e.y);
        w.x = pa.x;
        w.y = pa.y;
        w.z = pb.x;
        w.w = pb.y;
        const uint32_t r0 = __builtin_amdgcn_readlane(row, __builtin_ctzll(lm));
        if (__ballot(live && row != r0) == 0) {
            if (r0 != acc_row) {
                if (acc_row != 0xFFFFFFFFu) {
                    gemv_flush_lanes<kB>(G, nb, acc, acc_row);
#pragma unroll
                    for (int b = 0; b < kB; ++b) acc[b] = 0.0f;
                }
                acc_row = r0;
            }
#pragma unroll
            for (int b = 0; b < kB; ++b) {
                const float t = dot8_acc(w, xc[b], acc[b]);
                acc[b] = live ? t : acc[b];
            }
        } else {
            // Several rows: one wave sum and one atomic per distinct row
            // instead of one atomic per lane (small chunks put several
            // chunks, and often several rows, in one wave step).
            float p[kB];
#pragma unroll
            for (int b = 0; b < kB; ++b) {
                const float t = dot8_acc(w, xc[b], 0.0f);
                p[b] = live ? t : 0.0f;
            }
            gemv_rows_add<kB>(G, nb, p, live, row);
        }
    }
    if (acc_row != 0xFFFFFFFFu) gemv_flush_lanes<kB>(G, nb, acc, acc_row);
}

// Window table and the first kLdsEscBlocks escape blocks of a table blob to LDS.
__device__ __forceinline__ void load_table(const uint8_t* table, uint32_t tid, uint32_t* s_wsyms,
                                           uint8_t* s_wmeta, uint8_t* s_len, uint16_t* s_esc) {
    const uint4* src = reinterpret_cast<const uint4*>(table + kSymsOffset);
    uint4* dst = reinterpret_cast<uint4*>(s_wsyms);
    for (uint32_t j = tid; j < kWinEntries / 4; j += kThreads) dst[j] = src[j];
    const uint4* msrc = reinterpret_cast<const uint4*>(table + kMetaOffset);
    uint4* mdst = reinterpret_cast<uint4*>(s_wmeta);
    for (uint32_t j = tid; j < kWinEntries / 16; j += kThreads) mdst[j] = msrc[j];
    const uint4* lsrc = reinterpret_cast<const uint4*>(table + kLenOffset);
    for (uint32_t j = tid; j < 256 / 16; j += kThreads) reinterpret_cast<uint4*>(s_len)[j] = lsrc[j];
    const uint32_t n_blocks = header_of(table)->n_esc_blocks;
    const uint32_t n_esc = n_blocks < static_cast<uint32_t>(kLdsEscBlocks) ? n_blocks : kLdsEscBlocks;
    const uint16_t* gesc = reinterpret_cast<const uint16_t*>(table + kEscOffset);
    for (uint32_t j = tid; j < n_esc * kEscBlockEntries; j += kThreads) s_esc[j] = gesc[j];
}

// A workgroup's LDS, in one block so that the small tables sit at the lowest
// addresses, where their bases fit the LDS instructions' 16-bit offsets.
struct __attribute__((aligned(16))) Lds {
    uint8_t wmeta[kWinEntries];
    uint8_t len[256];
    uint16_t esc[kLdsEscBlocks * kEscBlockEntries];
    uint32_t wsyms[kWinEntries];
    uint32_t wsum[kWaves];
    uint32_t gpre[kMaxGroups + 1];
    uint32_t wbad[kWaves];  // some thread of the wave disagrees with its predecessor
    uint32_t gval[kMaxGroups];
    uint32_t ewave[kWaves];      // segment end of each wave's last lane
    uint32_t glast[kMaxGroups];  // segment end of each sub-group's last active thread
    uint32_t hand[8];            // a split chunk's handoff as its second half took it
    uint32_t tile[kTileWords];
    // Past the slots: the word read or zero-ORed past the last slot, and the
    // groups an unclamped store batch of a whole-workgroup chunk reads.
    __attribute__((aligned(16))) uint8_t stage[kStagePadded];
};

// Handoff records of split chunks (LaunchArgs::split_first): kHandoffWords
// 64-bit words each, every word the launch's tag above a 32-bit value. Word 0
// is the record's state: 0 empty; p0 (where the second half's first round
// starts) once the first half has written the record; kHandoffGaveUp once the
// second half has stopped waiting for it. Words 1..6: the symbols placed so
// far, the carried symbols, and their bytes. A record is empty again at the
// end of a launch: the second half empties a record it reads, and a first
// half that finds its second half gone empties it. Tags keep launches that
// overlap on one GPU from reading each other's records (they then fall back
// to whole chunks). Every access to a record is a device-scope atomic (it
// bypasses the XCD's L2, whose contents other XCDs do not see), so no
// fence has to write back or invalidate the L2 for it: the first half waits
// for its word writes to complete before it publishes word 0, and the second
// half reads the words only after it has seen word 0.
constexpr uint32_t kHandoffWords = 8;
constexpr uint32_t kHandoffSlots = 1024;
constexpr uint32_t kHandoffGaveUp = 0xFFFFFFFFu;
// Polls of a record (each an L2-bypassing load and a short sleep) before the
// second half decodes its chunk whole. First halves are the grid's first
// items and second halves its last, so the record is normally written long
// before it is read.
constexpr uint32_t kHandoffPolls = 64;

// The first half's state at its end: thread 0 writes the record's words,
// then publishes it in word 0 (release).
__device__ __forceinline__ void give_handoff(const LaunchArgs& args, uint32_t slot, uint32_t p0,
                                          uint32_t ob, uint32_t lead, const uint8_t* stage) {
    uint64_t* const rec = args.handoff + static_cast<uint64_t>(slot) * kHandoffWords;
    const uint64_t tg = static_cast<uint64_t>(args.tag) << 32;
    uint32_t b[4] = {0u, 0u, 0u, 0u};
    for (uint32_t k = 0; k < lead && k < 16u; ++k)
        b[k >> 2] |= static_cast<uint32_t>(stage[k]) << (8 * (k & 3u));
    __hip_atomic_store(rec + 1, tg | ob, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    __hip_atomic_store(rec + 2, tg | lead, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    for (uint32_t k = 0; k < 4; ++k)
        __hip_atomic_store(rec + 3 + k, tg | b[k], __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    // The words above are complete (device-scope writes) before word 0 is.
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "workgroup");
    uint64_t seen = 0;
    if (!__hip_atomic_compare_exchange_strong(rec, &seen, tg | p0, __ATOMIC_RELAXED, __ATOMIC_RELAXED,
                                              __HIP_MEMORY_SCOPE_AGENT) &&
        seen == (tg | kHandoffGaveUp))
        __hip_atomic_store(rec, uint64_t{0}, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

// The second half's wait (thread 0): out[0] 1 when the record was taken,
// then p0, the symbols placed, the carried symbols (< kGroup), their bytes.
// A record whose values cannot come from its chunk is not taken.
__device__ __forceinline__ void take_handoff(const LaunchArgs& args, uint32_t slot, uint32_t group,
                                          uint32_t lim, uint32_t* out) {
    uint64_t* const rec = args.handoff + static_cast<uint64_t>(slot) * kHandoffWords;
    const uint64_t tg = static_cast<uint64_t>(args.tag) << 32;
    uint64_t v = 0;
    bool ok = false;
    for (uint32_t k = 0; k < kHandoffPolls; ++k) {
        v = __hip_atomic_load(rec, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        ok = (v >> 32) == args.tag && static_cast<uint32_t>(v) != kHandoffGaveUp;
        if (ok) break;
        __builtin_amdgcn_s_sleep(16);
    }
    if (!ok) {
        uint64_t seen = 0;
        if (!__hip_atomic_compare_exchange_strong(rec, &seen, tg | kHandoffGaveUp, __ATOMIC_RELAXED,
                                                  __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) &&
            (seen >> 32) == args.tag && static_cast<uint32_t>(seen) != kHandoffGaveUp) {
            v = seen;
            ok = true;
        }
    }
    uint32_t w[6] = {0u, 0u, 0u, 0u, 0u, 0u};
    if (ok) {
        for (uint32_t k = 0; k < 6; ++k) {
            const uint64_t x = __hip_atomic_load(rec + 1 + k, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
            ok = ok && (x >> 32) == args.tag;
            w[k] = static_cast<uint32_t>(x);
        }
        __hip_atomic_store(rec, uint64_t{0}, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        // p0 lies within the longest codeword past its round's start.
        ok = ok && static_cast<uint32_t>(v) < 64u && w[0] <= lim && w[1] < group && w[1] <= w[0];
    }
    out[0] = ok ? 1u : 0u;
    out[1] = static_cast<uint32_t>(v);
    for (uint32_t k = 0; k < 6; ++k) out[2 + k] = w[k];
}

// kLg > 0 fixes the threads per chunk at 1 << kLg for the whole launch, so
// that sub-group geometry and the per-thread offsets derived from it are
// compile-time constants.
template <int kMode, int kGroup, bool kTiny, uint32_t kLg>
__global__ __launch_bounds__(kThreads, kWavesPerSimd) void decode_kernel(const LaunchArgs args) {
    __shared__ Lds lds;
    uint32_t* const s_wsyms = lds.wsyms;
    uint8_t* const s_wmeta = lds.wmeta;
    uint8_t* const s_len = lds.len;
    uint16_t* const s_esc = lds.esc;
    uint32_t* const s_tile = lds.tile;
    uint8_t* const s_stage = lds.stage;
    uint32_t* const s_ewave = lds.ewave;
    uint32_t* const s_glast = lds.glast;
    uint32_t* const s_wsum = lds.wsum;
    uint32_t* const s_gpre = lds.gpre;
    uint32_t* const s_wbad = lds.wbad;
    uint32_t* const s_gval = lds.gval;
    // Whole-workgroup chunks (the index build aside) take the fast path; its
    // record of each wave's lane 0 (start, whether it is checked) reuses the
    // sub-group prefix table, which that path does not need.
    constexpr bool kWhole = kLg == kLgThreads && kMode != kModeIndex;
    // Whole-workgroup chunks of bf16 or exponent-byte launches may be split.
    constexpr bool kSplit = kWhole && (kMode == kModeBf16 || kMode == kModeU8);
    uint32_t* const s_f0 = lds.gpre;
    uint32_t* const s_chk0 = lds.gpre + kWaves;

    const uint32_t tid = threadIdx.x;
    // A CU's two workgroups start together and would go through their rounds
    // in step, decoding at the same time and loading and storing at the same
    // time. The second starts two sleeps of kStaggerSleep later (about 4 us,
    // near a workgroup's start-up), so that their phases alternate from the
    // first round on: 5120x17408 layer 71.4 -> 68.4 us (2 x 60: 68.6, 2 x
    // 120: 69.0, 2 x 40: 70.2; the 14B block unchanged). AIMG_STAGGER=0
    // turns it off.
    if (args.stagger != 0 && blockIdx.x >= gridDim.x / 2) {
        __builtin_amdgcn_s_sleep(kStaggerSleep);
        __builtin_amdgcn_s_sleep(kStaggerSleep);
    }
    const uint8_t* loaded = nullptr;
    Tables tb;
    tb.syms = s_wsyms;
    tb.meta = s_wmeta;
    tb.len = s_len;
    tb.esc = s_esc;

    // Software pipeline: the stream words of the next round (or of the next
    // item's first round) are in flight while the current round decodes.
    // The first item's words and table load together.
    Job cur = make_job<kMode, kLg>(args, blockIdx.x, tid);
    Fetch F;
    fetch_issue<kMode, kTiny, kLg>(F, args, cur, cur.r0, tid);
    loaded = uniform(args.t[uniform(static_cast<uint32_t>(cur.d))].table);
    load_table(loaded, tid, s_wsyms, s_wmeta, s_len, s_esc);
    fetch_commit<kTiny, kLg>(F, args, cur, cur.r0, tid, s_tile);

    for (int64_t item = blockIdx.x; item < args.total_items; item += gridDim.x) {
        const DevTensor& T = args.t[uniform(static_cast<uint32_t>(cur.d))];
        const uint8_t* const table = uniform(T.table);
        const uint32_t lg = kLg > 0 ? kLg : uniform(cur.lg);
        const uint32_t tpc = 1u << lg;
        const uint32_t g = tid >> lg;
        const uint32_t i_item = tid & (tpc - 1);
        const uint32_t n_groups = kThreads >> lg;
        const uint32_t S = uniform(cur.S);
        const Job nxt = make_job<kMode, kLg>(args, item + gridDim.x, tid);

        const auto* hdr = header_of(table);
        tb.sym0 = hdr->sym0;
        tb.min_len = hdr->min_len >= 1 ? hdr->min_len : 1u;
        tb.gesc = (const __attribute__((address_space(1))) uint16_t*)(table + kEscOffset);
        const bool global_esc = hdr->n_esc_blocks > static_cast<uint32_t>(kLdsEscBlocks);
        __syncthreads();  // the previous item is done with LDS; its tile writes are visible
        const bool reload = table != loaded;
        if (reload) {
            loaded = table;
            load_table(table, tid, s_wsyms, s_wmeta, s_len, s_esc);
        }

        const int64_t chunk_base = cur.c * T.chunk_size;
        const int64_t lim = cur.lim;
        // Laundered: the tile base then stays one register, not a base plus
        // a constant added in every step of the decode loops.
        TileRef below = (TileRef)(tile_top(s_tile, g, lg) - 1);
        asm volatile("" : "+v"(below));
        const uint32_t region = kStageBytes >> (kLgThreads - lg);
        uint8_t* stage = s_stage + g * region;
        uint8_t* slot = stage + kLeadBytes + i_item * kSlotBytes;

        // Rounds of the item: the most any of its chunks needs (a whole-workgroup
        // chunk's own, without a barrier unless the table was just loaded).
        uint32_t NR = 0;
        if (kLg == kLgThreads && !reload) {
            NR = uniform(cur.nr);
        } else {
            if (i_item == 0) s_gval[g] = cur.nr;
            __syncthreads();
            for (uint32_t k = 0; k < n_groups; ++k) NR = NR > s_gval[k] ? NR : s_gval[k];
            NR = uniform(NR);
        }

        int64_t ob = 0;     // chunk-local symbols placed so far
        uint32_t lead = 0;  // placed symbols still staged at the front of the region
        uint32_t p0 = 0;    // true start of the next round, relative to its first bit
        uint32_t r_begin = 0, r_end = NR;
        if constexpr (kSplit) {
            r_begin = uniform(cur.r0);
            r_end = uniform(cur.r1);
            if (uniform(static_cast<uint32_t>(cur.half)) == kSecondHalf) {
                // The first half's state: where round r_begin starts, the
                // symbols placed before it and the carried ones. Without it
                // (the first half did not hand over in time), the chunk is
                // decoded whole from round 0.
                if (tid == 0) take_handoff(args, cur.slot, kGroup, cur.lim, lds.hand);
                __syncthreads();
                if (lds.hand[0] != 0u) {
                    p0 = lds.hand[1];
                    ob = lds.hand[2];
                    lead = lds.hand[3];
                    if (tid < lead) stage[tid] = static_cast<uint8_t>(lds.hand[4 + (tid >> 2)] >> (8 * (tid & 3u)));
                } else {
                    r_begin = 0;
                    fetch_issue<kMode, kTiny, kLg>(F, args, cur, 0, tid);
                    fetch_commit<kTiny, kLg>(F, args, cur, 0, tid, s_tile);
                }
                __syncthreads();
            }
        }
        for (uint32_t r = r_begin; r < r_end; ++r) {
            // Offsets derived from the thread index are cheap to recompute;
            // keeping them live across the round costs registers.
            uint32_t i = i_item;
            asm volatile("" : "+v"(i));
            // Next words: this item's round r + 1, or the next item's first.
            const bool last = r + 1 == r_end;
            const Job& fj = last ? nxt : cur;
            const uint32_t fr = last ? uniform(nxt.r0) : r + 1;
            // Wave priorities by phase: the two workgroups of a CU overlap best
            // when issuing loads comes first, stores and compaction next, the
            // agreement check and scan after, and the decode loops last (each
            // setting measured; 6.5% faster than equal priorities).
            __builtin_amdgcn_s_setprio(3);
            fetch_issue<kMode, kTiny, kLg>(F, args, fj, fr, tid);
            // Sign/mantissa bytes of every group this round can fill (its
            // output starts at a known element; its length is known only
            // after decoding), requested now so the store never waits.
            SmBatch<kMode> smb;
            // (A whole-workgroup chunk's: none past the chunk's last element.)
            sm_issue<kMode, kGroup>(smb, T, chunk_base + ob - lead, i, tpc,
                                    kWhole ? uniform(static_cast<uint32_t>(chunk_base + lim)) : 0xFFFFFFFFu);
            const uint32_t RB = round_len(cur, r);
            const bool g_active = RB != 0;

            const uint32_t seg_lo = i * S;
            const bool active = seg_lo < RB;
            const uint32_t seg_hi = active ? (seg_lo + S < RB ? seg_lo + S : RB) : 0u;
            uint32_t f = 0, e = 0, cnt = 0;
            // What the compaction hands to the store.
            int64_t a0;
            uint32_t want, avail, nfull, e_last;
            if constexpr (kWhole) {
                // A whole-workgroup chunk: slots interleaved by lane (no bank
                // conflicts), one record barrier for the agreement check and
                // the scan, and branch-free compaction writes.
                const uint32_t lane = tid & 63u;
                const uint32_t w = uniform(tid >> 6);
                uint32_t* const slot_il =
                    reinterpret_cast<uint32_t*>(stage + kLeadBytes) + w * kSlotRows * 64 + lane;
                const IlSlot sl{stage + kLeadBytes, w * kSlotRows * 256u, lane * 4u};
                __builtin_amdgcn_s_setprio(0);
                if (active) {
                    Adv a;
                    if (global_esc) {
                        f = i == 0 ? p0 : advance<true>(below, tb, seg_lo - kOverlapBits, seg_lo);
                        a = decode_run_il<true>(below, tb, f, seg_hi, 0xFFFFFFFFu, sl);
                    } else {
                        f = i == 0 ? p0 : advance<false>(below, tb, seg_lo - kOverlapBits, seg_lo);
                        a = decode_run_il<false>(below, tb, f, seg_hi, 0xFFFFFFFFu, sl);
                    }
                    e = a.p;
                    cnt = a.n;
                }
                __builtin_amdgcn_s_setprio(1);
                // Each wave checks its lanes against the lane below and scans
                // its counts; its last lane leaves the wave's count, end and
                // disagreement, lane 0 its start, and after one barrier every
                // wave checks the waves' first lanes and finds its prefix.
                uint32_t incl;
                const bool checked = active && i > 0;
                for (;;) {
                    const uint32_t ep0 = lane_below(e);
                    incl = wave_scan_incl(cnt);
                    const bool wbad = __ballot(checked && lane != 0 && f != ep0) != 0;
                    if (lane == 63) {
                        s_wsum[w] = incl;
                        s_ewave[w] = e;
                        s_wbad[w] = wbad ? 1u : 0u;
                    }
                    if (lane == 0) {
                        s_f0[w] = f;
                        s_chk0[w] = checked ? 1u : 0u;
                    }
                    __syncthreads();
                    const uint32_t lw = lane & (kWaves - 1);
                    const bool xbad = lw > 0 && s_chk0[lw] != 0u && s_f0[lw] != s_ewave[lw - 1];
                    if (__ballot(lane < kWaves && (s_wbad[lw] != 0u || xbad)) == 0) break;
                    // Rare: threads whose start disagrees with their
                    // predecessor's end decode again from it (thread 0 is
                    // always right, so pass k puts thread k right at the latest).
                    const uint32_t ep = lane == 0 ? (w > 0 ? s_ewave[w - 1] : 0u) : ep0;
                    const bool redo = checked && f != ep;
                    __syncthreads();  // the records are read before they are written again
                    if (redo) {
                        f = ep;
                        const Adv a = global_esc
                                          ? decode_run_il<true>(below, tb, f, seg_hi, 0xFFFFFFFFu, sl)
                                          : decode_run_il<false>(below, tb, f, seg_hi, 0xFFFFFFFFu, sl);
                        e = a.p;
                        cnt = a.n;
                    }
                }
                uint32_t pre = 0, gtot = 0;
#pragma unroll
                for (uint32_t k = 0; k < kWaves; ++k) {
                    const uint32_t v = s_wsum[k];
                    pre += k < w ? v : 0u;
                    gtot += v;
                }
                const uint32_t o = pre + incl - cnt;
                const int64_t still = lim - ob;
                want = g_active ? (gtot < still ? gtot : static_cast<uint32_t>(still)) : 0u;
                avail = lead + want;
                nfull = avail / kGroup;
                a0 = chunk_base + ob - lead;
                // The last active thread (its segment ends the round), or
                // thread 0 of an empty round, leaves its end.
                if (g_active ? active && seg_hi == RB : i == 0) s_glast[0] = e;
                __builtin_amdgcn_s_setprio(2);
                // Compaction: the slot into registers (the dense area overlaps
                // the slots), a barrier, then the symbols to their place.
                const uint32_t m = want > o ? (cnt < want - o ? cnt : want - o) : 0u;
                const uint32_t dpos = lead + o;
                const uint32_t head0 = (4u - (dpos & 3u)) & 3u;
                const uint32_t hb = head0 < m ? head0 : m;
                const uint32_t nbody = (m - hb) >> 2;
                const uint32_t ntail = m - hb - 4 * nbody;
                uint32_t rw[kSlotRows];
                {
                    const auto* sl = lds_ptr(slot_il);
#pragma unroll
                    for (uint32_t j = 0; j < kSlotRows; ++j) rw[j] = sl[j * 64];
                }
                const uint32_t tv = __builtin_amdgcn_alignbyte(
                    slot_il[(nbody + 1 < kSlotRows ? nbody + 1 : kSlotRows - 1) * 64], slot_il[nbody * 64], hb);
                __syncthreads();
                e_last = s_glast[0];
                uint8_t* dst = stage + dpos;
                if (hb & 1u) dst[0] = static_cast<uint8_t>(rw[0]);
                if (hb >= 2) *reinterpret_cast<uint16_t*>(dst + hb - 2) = static_cast<uint16_t>(rw[0] >> (8 * (hb - 2)));
                // Body words, each under its own lane mask at a constant
                // offset from the first (writing every word to a place clamped
                // to the last took an address computation each, 0.8% slower).
                uint32_t* const body = reinterpret_cast<uint32_t*>(dst + hb);
#pragma unroll
                for (uint32_t j = 0; j + 1 < kSlotRows; ++j)
                    if (j < nbody) body[j] = __builtin_amdgcn_alignbyte(rw[j + 1], rw[j], hb);
                uint8_t* tl = dst + hb + 4 * nbody;
                if (ntail >= 2) *reinterpret_cast<uint16_t*>(tl) = static_cast<uint16_t>(tv);
                if (ntail & 1u) tl[ntail - 1] = static_cast<uint8_t>(tv >> (8 * (ntail - 1)));
                // Every thread is past its decode, so the tile takes the next words.
                fetch_commit<kTiny, kLg>(F, args, fj, fr, tid, s_tile);
                __syncthreads();
            } else {
            __builtin_amdgcn_s_setprio(0);
            if (active) {
                start_slot(slot);
                Adv a;
                if (global_esc) {
                    f = i == 0 ? p0 : advance<true>(below, tb, seg_lo - kOverlapBits, seg_lo);
                    a = decode_run<true>(below, tb, f, seg_hi, slot);
                } else {
                    f = i == 0 ? p0 : advance<false>(below, tb, seg_lo - kOverlapBits, seg_lo);
                    a = decode_run<false>(below, tb, f, seg_hi, slot);
                }
                e = a.p;
                cnt = a.n;
            }
            __builtin_amdgcn_s_setprio(1);
            // A segment is right when it starts where its predecessor's last
            // codeword ends. The predecessor's end comes from the lane below;
            // a wave's lane 0 reads the previous wave's lane 63 through LDS.
            // Whether any thread disagrees goes through one flag per wave.
            const uint32_t lane = tid & 63u;
            const uint32_t w = tid >> 6;
            const uint32_t wprev = (w - 1u) & (kWaves - 1u);
            for (;;) {
                uint32_t ep = lane_below(e);
                if (lane == 63) s_ewave[w] = e;
                __syncthreads();
                if (lane == 0) ep = s_ewave[wprev];
                const bool bad = active && i > 0 && f != ep;
                const bool wave_bad = __ballot(bad) != 0;
                if (lane == 0) s_wbad[w] = wave_bad;
                __syncthreads();
                bool any_bad = false;
#pragma unroll
                for (uint32_t k = 0; k < kWaves; ++k) any_bad |= s_wbad[k] != 0;
                if (!any_bad) break;
                if (bad) {
                    f = ep;
                    start_slot(slot);
                    const Adv a = global_esc ? decode_run<true>(below, tb, f, seg_hi, slot)
                                             : decode_run<false>(below, tb, f, seg_hi, slot);
                    e = a.p;
                    cnt = a.n;
                }
            }
            if (g_active ? active && seg_hi == RB : i == 0) s_glast[g] = e;
            if constexpr (kMode == kModeIndex) {
                // Index build: each segment's first boundary (0..15 bits
                // past its start) and codeword count; no output.
                if (active && cur.ib != kNoIndex) {
                    const IndexLayout L = index_layout(T.packed_nbytes, T.n_chunks, S);
                    __builtin_amdgcn_raw_buffer_store_b32(
                        (cnt << 4) | (f - seg_lo), index_part(T, L.entries, 4 * L.capacity),
                        4u * (cur.ib + r * tpc + i), 0, 0);
                }
                fetch_commit<kTiny, kLg>(F, args, fj, fr, tid, s_tile);
                __syncthreads();
                if (g_active) p0 = s_glast[g] - RB;
                continue;
            }

            const uint32_t excl = block_scan_excl(cnt, s_wsum);
            if (i == 0) s_gpre[g] = excl;
            if (tid == kThreads - 1) s_gpre[n_groups] = excl + cnt;
            __syncthreads();
            e_last = s_glast[g];
            const uint32_t o = excl - s_gpre[g];
            const uint32_t gtot = s_gpre[g + 1] - s_gpre[g];
            const int64_t still = lim - ob;
            want = g_active ? (gtot < still ? gtot : static_cast<uint32_t>(still)) : 0u;
            avail = lead + want;
            nfull = avail / kGroup;
            a0 = chunk_base + ob - lead;

            __builtin_amdgcn_s_setprio(2);
            // Compaction. The dense area overlaps the slots, so every slot is
            // in registers before any symbol moves.
            const uint32_t m = want > o ? (cnt < want - o ? cnt : want - o) : 0u;
            const uint32_t dpos = lead + o;
            const uint32_t head0 = (4u - (dpos & 3u)) & 3u;
            const uint32_t head = head0 < m ? head0 : m;  // bytes before the first aligned word
            const uint32_t nbody = (m - head) >> 2;       // whole words
            const uint32_t ntail = m - head - 4 * nbody;  // bytes after them
            // One word past the cap (still inside the slot), for the byte
            // shift of the last whole word.
            uint32_t rw[kSlotWords + 1];
            const uint32_t* slot_w = reinterpret_cast<const uint32_t*>(slot);
            {
                // Read through an LDS-typed pointer: one address register,
                // the word offsets folded into the reads.
                const auto* sl = lds_ptr(slot_w);
#pragma unroll
                for (uint32_t j = 0; j < kSlotWords + 1; ++j) rw[j] = sl[j];
            }
            const uint32_t tv = __builtin_amdgcn_alignbyte(slot_w[nbody + 1], slot_w[nbody], head);
            __syncthreads();
            uint8_t* dst = stage + dpos;
#pragma unroll
            for (uint32_t k = 0; k < 3; ++k)
                if (k < head) dst[k] = static_cast<uint8_t>(rw[0] >> (8 * k));
            uint32_t* body = reinterpret_cast<uint32_t*>(dst + head);
#pragma unroll
            for (uint32_t j = 0; j < kSlotWords; ++j)
                if (j < nbody) body[j] = __builtin_amdgcn_alignbyte(rw[j + 1], rw[j], head);
            uint8_t* tl = dst + head + 4 * nbody;
#pragma unroll
            for (uint32_t k = 0; k < 3; ++k)
                if (k < ntail) tl[k] = static_cast<uint8_t>(tv >> (8 * k));
            // Every thread is past its decode, so the tile takes the next words.
            fetch_commit<kTiny, kLg>(F, args, fj, fr, tid, s_tile);
            __syncthreads();
            }

            store_round<kMode, kGroup, kLg == kLgThreads>(smb, T, args.gemv, stage, a0, nfull, i, tpc);
            ob += want;
            // The partial vector group moves to the front for the next round.
            const uint32_t rem = avail - nfull * kGroup;
            const uint8_t keep = i < rem ? stage[nfull * kGroup + i] : 0;
            __syncthreads();
            if (i < rem) stage[i] = keep;
            lead = rem;
            if (g_active) p0 = e_last - RB;
        }
        if (r_begin == r_end) {
            fetch_issue<kMode, kTiny, kLg>(F, args, nxt, nxt.r0, tid);
            fetch_commit<kTiny, kLg>(F, args, nxt, nxt.r0, tid, s_tile);
        }

        // Symbols carried out of the last round, then positions no codeword
        // of the chunk reached: those decode from zero bits, i.e. to sym_lut[0].
        // A first half hands them over instead; a chunk's empty second half
        // has none.
        __syncthreads();
        [[maybe_unused]] bool tail = true;
        if constexpr (kSplit) {
            const uint32_t half = uniform(static_cast<uint32_t>(cur.half));
            if (half == kFirstHalf && tid == 0)
                give_handoff(args, cur.slot, p0, static_cast<uint32_t>(ob), lead, stage);
            tail = half == kWholeChunk || half == kSecondHalf;
        }
        if constexpr (kMode != kModeIndex) {
            if (tail) {
            const int64_t t0 = chunk_base + ob - lead;
            const int64_t n_tail = lim - (ob - lead);
            for (int64_t k = i_item; k < n_tail; k += tpc) {
                const uint32_t ex = k < lead ? stage[k] : tb.sym0;
                store_one<kMode>(T, args.gemv, t0 + k, ex);
            }
            }
        }
        cur = nxt;
    }
}

// ---------------------------------------------------------------------------
// Segment index build (aimg_build_index): plan, entries, finish.
// ---------------------------------------------------------------------------

typedef const __attribute__((address_space(4))) uint32_t* ConstU32;

// A chunk's byte range, clamped to the packed buffer as the decoders clamp it.
__device__ __forceinline__ void chunk_range(const DevTensor& T, int64_t c, int64_t* off, int64_t* nb) {
    int64_t o = T.offsets[c], n = T.nbytes[c];
    o = o < 0 ? 0 : (o > T.packed_nbytes ? T.packed_nbytes : o);
    n = n < 0 ? 0 : (n > T.packed_nbytes - o ? T.packed_nbytes - o : n);
    *off = o;
    *nb = n;
}

// Plan, one workgroup per tensor: chunk c (c < n_jobs) gets segments
// base[c] .. base[c] + ceil(8 * nbytes / S) - 1, and the header the segment
// length, the table's checksum,
// and ok = 1 when the chunks lie back to back and the layout fits the index
// (the entries step writes only then; the finish step may clear ok).
__global__ __launch_bounds__(kThreads) void index_plan_kernel(const LaunchArgs args) {
    __shared__ uint32_t s_wsum[kWaves];
    __shared__ uint32_t s_bad;
    const DevTensor& T = args.t[blockIdx.x];
    uint8_t* const ix = T.index;
    if (ix == nullptr) return;
    const auto* th = header_of(T.table);
    const uint32_t S = segment_bits(th->min_len);
    const IndexLayout L = index_layout(T.packed_nbytes, T.n_chunks, S);
    const bool fits = L.total <= T.index_n32 && L.capacity < kNoIndex;
    if (threadIdx.x == 0) s_bad = fits ? 0u : 1u;
    __syncthreads();
    uint32_t* const base = reinterpret_cast<uint32_t*>(ix + L.base);
    uint64_t run = 0;
    // kPlanChunks consecutive chunks per thread and step: their segment
    // counts are summed in the thread, the sums scanned over the workgroup.
    constexpr int kPlanChunks = 4;
    for (int64_t c0 = 0; c0 < T.n_chunks; c0 += kPlanChunks * kThreads) {
        const int64_t cb = c0 + kPlanChunks * static_cast<int64_t>(threadIdx.x);
        uint32_t nseg[kPlanChunks];
        uint32_t mine = 0;
#pragma unroll
        for (int j = 0; j < kPlanChunks; ++j) {
            const int64_t c = cb + j;
            nseg[j] = 0;
            if (c < T.n_jobs) {
                int64_t off, nb;
                chunk_range(T, c, &off, &nb);
                nseg[j] = static_cast<uint32_t>((nb * 8 + S - 1) / S);
                // Back to back: the next chunk starts where this one ends.
                if (c + 1 < T.n_jobs && T.offsets[c + 1] != off + nb) s_bad = 1u;
            }
            mine += nseg[j];
        }
        const uint32_t excl = block_scan_excl(mine, s_wsum);
        uint32_t tot = 0;
#pragma unroll
        for (int w = 0; w < kWaves; ++w) tot += s_wsum[w];
        uint64_t at = run + excl;
#pragma unroll
        for (int j = 0; j < kPlanChunks; ++j) {
            const int64_t c = cb + j;
            if (fits && c < T.n_chunks) base[c] = static_cast<uint32_t>(at < kNoIndex ? at : kNoIndex - 1u);
            at += nseg[j];
        }
        run += tot;
        __syncthreads();  // s_wsum is written again by the next step's scan
    }
    if (threadIdx.x == 0) {
        if (fits) {
            base[T.n_chunks] = static_cast<uint32_t>(run < kNoIndex ? run : kNoIndex - 1u);
            // After the last round: the tensor's end (segment runs take a
            // round's symbol count from the next round's first element).
            const uint64_t m = (run + kIndexBlock - 1) / kIndexBlock;
            if (m < L.n_rounds) {
                RoundStart end;
                end.chunk = static_cast<uint32_t>(T.n_jobs > 0 ? T.n_jobs - 1 : 0);
                end.element = static_cast<uint32_t>(T.n_symbols);
                end.byte = static_cast<uint32_t>(T.packed_nbytes);
                end.chunk_base = static_cast<uint32_t>(run);
                reinterpret_cast<RoundStart*>(ix + L.rounds)[m] = end;
            }
        }
        IndexHeader h{};
        h.magic = kIndexMagic;
        h.version = static_cast<uint32_t>(kAbiVersion);
        h.seg_bits = S;
        h.table_checksum = th->checksum;
        h.ok = s_bad == 0u && run <= L.capacity ? 1u : 0u;
        h.n_chunks = static_cast<uint32_t>(T.n_chunks);
        h.n_segments = static_cast<uint32_t>(run < kNoIndex ? run : kNoIndex - 1u);
        h.n_jobs = static_cast<uint32_t>(T.n_jobs);
        *reinterpret_cast<IndexHeader*>(ix) = h;
    }
}

constexpr uint32_t kFinishThreads = 256;
constexpr uint32_t kWalkBytes = 32;  // a segment's bytes and the 32 bits read past its last start

// The first `keep` codewords from bit q of `seg` (a segment's bytes staged in
// LDS, zero past the chunk's end): the bit where the last of them ends,
// relative to seg. Whole windows are taken while they hold no more
// codewords than are left; the last window's codewords are counted one by
// one from their code lengths. These are the boundaries of reading one
// codeword at a time (escape windows, and windows no codeword starts, take
// their first codeword only): a window holds the codewords that lie wholly
// inside it, read one after another from its first bit.
__device__ __forceinline__ uint32_t walk_codewords(const uint8_t* seg, uint32_t q, uint32_t keep,
                                                   const uint32_t* wsyms, const uint8_t* wmeta,
                                                   const uint8_t* len, const uint16_t* esc,
                                                   const uint8_t* table) {
    const auto* hdr = header_of(table);
    const uint32_t min_len = hdr->min_len >= 1 ? hdr->min_len : 1u;
    const uint32_t n_esc = hdr->n_esc_blocks;
    const uint16_t* gesc = reinterpret_cast<const uint16_t*>(table + kEscOffset);
    uint32_t left = keep;
    while (left > 0) {
        // Only an index that does not describe its stream reads past the
        // segment's bytes; the clamp keeps it in the buffer.
        const uint32_t b = (q >> 3) < kWalkBytes - 4 ? (q >> 3) : kWalkBytes - 4;
        uint32_t w = (static_cast<uint32_t>(seg[b]) << 24) | (static_cast<uint32_t>(seg[b + 1]) << 16) |
                     (static_cast<uint32_t>(seg[b + 2]) << 8) | seg[b + 3];
        w <<= (q & 7u);
        const uint32_t idx = w >> (32 - kWinBits);
        const uint32_t meta = wmeta[idx];
        const uint32_t ent = wsyms[idx];
        if (meta != 0) {
            const uint32_t cnt = meta >> 5;
            if (left >= cnt) {
                q += meta & 31u;
                left -= cnt;
            } else {
                for (uint32_t j = 0; j < left; ++j) q += len[(ent >> (8 * j)) & 0xFFu];
                left = 0;
            }
        } else {
            const uint32_t blk = ent & 0xFFFFu;
            uint32_t l = min_len;
            if (blk != kUnusedBlock && blk < n_esc) {
                const uint32_t at = blk * kEscBlockEntries + ((w >> (28 - kWinBits)) & 15u);
                const uint16_t v = blk < static_cast<uint32_t>(kLdsEscBlocks) ? esc[at] : gesc[at];
                l = (v >> 8) ? (v >> 8) : min_len;
            }
            q += l;
            --left;
        }
    }
    return q;
}

// Finish, one wave per chunk (c < n_jobs): the chunk's lim-th codeword is
// found from the entries' counts; its end is the chunk's real end rend,
// that segment keeps only the codewords up to it and later segments none.
// A chunk with fewer than lim codewords, or whose lim-th codeword runs past
// its bytes, makes the index unusable. The round starts (segments 512 m)
// that fall in the chunk are written too: with the counts so fixed, the
// codewords before segment g of the chunk are min(raw count before g, lim).
// A wave goes through its chunk's segments 64 at a time with wave scans, so
// the waves of a workgroup finish four chunks at once with no barrier. The
// walk reads the decode table from LDS (the table of the tensor of each
// group of four chunks' first chunk; a wave whose tensor has another table
// reads it from global memory).
constexpr uint32_t kFinishWaves = kFinishThreads / 64;

template <bool kLdsTable>
__device__ __forceinline__ void finish_chunk(const LaunchArgs& args, int64_t item, uint32_t lane,
                                             uint8_t* seg, const uint32_t* f_wsyms,
                                             const uint8_t* f_wmeta, const uint8_t* f_len,
                                             const uint16_t* f_esc) {
    int d = 0;
    while (d + 1 < args.n_tensors && item >= args.t[d + 1].item_begin) ++d;
    const DevTensor& T = args.t[d];
    const int64_t c = item - T.item_begin;
    uint8_t* const ix = T.index;
    const auto* h = reinterpret_cast<const IndexHeader*>(ix);
    if (h->magic != kIndexMagic || h->ok != 1u) return;
    const uint32_t S = h->seg_bits;
    const IndexLayout L = index_layout(T.packed_nbytes, T.n_chunks, S);
    const uint32_t* base = reinterpret_cast<const uint32_t*>(ix + L.base);
    uint32_t* rend = reinterpret_cast<uint32_t*>(ix + L.rend);
    uint32_t* ent = reinterpret_cast<uint32_t*>(ix + L.entries);
    RoundStart* rounds = reinterpret_cast<RoundStart*>(ix + L.rounds);
    const uint32_t b0 = base[c], b1 = base[c + 1];
    int64_t off, nb;
    chunk_range(T, c, &off, &nb);
    int64_t lim = T.n_symbols - c * T.chunk_size;
    lim = lim > T.chunk_size ? T.chunk_size : lim;
    uint32_t found = 0;  // 1: this lane walked to the lim-th codeword's end within the chunk
    uint32_t pre = 0;    // codewords of the chunk before this block of segments
    for (uint32_t g0 = b0; g0 < b1; g0 += 64) {
        const uint32_t g = g0 + lane;
        const uint32_t e = g < b1 ? ent[g] : 0u;
        const uint32_t cnt = (e >> 4) & 127u;
        const uint32_t x = wave_scan_incl(cnt);
        const uint32_t tot = __builtin_amdgcn_readlane(x, 63);
        const uint32_t excl = pre + x - cnt;  // codewords before segment g
        if (g < b1 && g % kIndexBlock == 0 && g / kIndexBlock < L.n_rounds) {
            RoundStart rs;
            rs.chunk = static_cast<uint32_t>(c);
            rs.element = static_cast<uint32_t>(c * T.chunk_size +
                                               (excl < static_cast<uint64_t>(lim) ? excl : lim));
            rs.byte = static_cast<uint32_t>(off + (g - b0) * (S / 8));
            rs.chunk_base = b0;
            rounds[g / kIndexBlock] = rs;
        }
        if (g < b1) {
            if (excl < static_cast<uint64_t>(lim) && excl + cnt >= static_cast<uint64_t>(lim)) {
                // The lim-th codeword is in this segment: walk to its end
                // over the segment's bytes.
                const uint32_t keep = static_cast<uint32_t>(lim - excl);
                const uint32_t lo = (g - b0) * S;  // a whole byte
                const uint8_t* bytes = T.packed + off;
                const uint32_t blo = lo >> 3;
#pragma unroll
                for (uint32_t k = 0; k < kWalkBytes; ++k)
                    seg[k] = blo + k < static_cast<uint64_t>(nb) ? bytes[blo + k] : 0u;
                uint32_t q;
                if (kLdsTable) {
                    q = walk_codewords(seg, e & 15u, keep, f_wsyms, f_wmeta, f_len, f_esc, T.table);
                } else {
                    q = walk_codewords(seg, e & 15u, keep,
                                       reinterpret_cast<const uint32_t*>(T.table + kSymsOffset),
                                       T.table + kMetaOffset, T.table + kLenOffset,
                                       reinterpret_cast<const uint16_t*>(T.table + kEscOffset),
                                       T.table);
                }
                const uint32_t p = lo + q;
                rend[c] = p;
                ent[g] = (e & 15u) | (keep << 4);
                found = p <= 8 * nb ? 1u : 2u;
            } else if (excl >= static_cast<uint64_t>(lim)) {
                ent[g] = e & 15u;  // past the real end
            }
        }
        pre += tot;
    }
    // Every lane of the wave is here (the item test is per wave).
    const bool ok = __ballot(found == 1u) != 0 && __ballot(found == 2u) == 0;
    if (lane == 0 && !ok) reinterpret_cast<IndexHeader*>(ix)->ok = 0u;
}

__global__ __launch_bounds__(kFinishThreads) void index_finish_kernel(const LaunchArgs args,
                                                                      int64_t total) {
    __shared__ uint32_t f_wsyms[kWinEntries];
    __shared__ uint8_t f_wmeta[kWinEntries];
    __shared__ uint8_t f_len[256];
    __shared__ uint16_t f_esc[kLdsEscBlocks * kEscBlockEntries];
    __shared__ __attribute__((aligned(16))) uint8_t f_seg[kFinishWaves][kWalkBytes];
    const uint32_t lane = threadIdx.x & 63u, wv = threadIdx.x >> 6;
    const uint8_t* loaded = nullptr;
    for (int64_t first = static_cast<int64_t>(blockIdx.x) * kFinishWaves; first < total;
         first += static_cast<int64_t>(gridDim.x) * kFinishWaves) {
        int d0 = 0;
        while (d0 + 1 < args.n_tensors && first >= args.t[d0 + 1].item_begin) ++d0;
        const uint8_t* const table = args.t[d0].table;
        if (table != loaded) {
            __syncthreads();  // every wave is done with the previous table
            loaded = table;
            const uint4* src = reinterpret_cast<const uint4*>(table + kSymsOffset);
            for (uint32_t j = threadIdx.x; j < kWinEntries / 4; j += kFinishThreads)
                reinterpret_cast<uint4*>(f_wsyms)[j] = src[j];
            const uint4* msrc = reinterpret_cast<const uint4*>(table + kMetaOffset);
            for (uint32_t j = threadIdx.x; j < kWinEntries / 16; j += kFinishThreads)
                reinterpret_cast<uint4*>(f_wmeta)[j] = msrc[j];
            const uint4* lsrc = reinterpret_cast<const uint4*>(table + kLenOffset);
            for (uint32_t j = threadIdx.x; j < 256 / 16; j += kFinishThreads)
                reinterpret_cast<uint4*>(f_len)[j] = lsrc[j];
            const uint32_t nb_esc = header_of(table)->n_esc_blocks;
            const uint32_t n_esc = nb_esc < static_cast<uint32_t>(kLdsEscBlocks) ? nb_esc : kLdsEscBlocks;
            const uint16_t* gesc = reinterpret_cast<const uint16_t*>(table + kEscOffset);
            for (uint32_t j = threadIdx.x; j < n_esc * kEscBlockEntries; j += kFinishThreads)
                f_esc[j] = gesc[j];
            __syncthreads();
        }
        const int64_t item = first + wv;
        if (item >= total) continue;
        int d = d0;
        while (d + 1 < args.n_tensors && item >= args.t[d + 1].item_begin) ++d;
        if (args.t[d].table == loaded) {
            finish_chunk<true>(args, item, lane, f_seg[wv], f_wsyms, f_wmeta, f_len, f_esc);
        } else {
            finish_chunk<false>(args, item, lane, f_seg[wv], f_wsyms, f_wmeta, f_len, f_esc);
        }
    }
}

// ---------------------------------------------------------------------------
// Segment runs: decode of tensors that carry a usable segment index.
//
// The index makes every segment's start and output place known, and its
// counts run on from chunk to chunk, so a tensor's segments form one
// sequence that any workgroup can take a slice of: the launch's segments
// (of every tensor it decodes this way) are split evenly over the grid,
// whatever the chunk size, and a round is any 512 consecutive segments,
// chunk boundaries included. Each thread decodes its segment from its true
// start up to the segment's end or its chunk's real end, whichever comes
// first, and ORs the symbols straight into place in the stage area.
// ---------------------------------------------------------------------------

// Chunks of at least this many symbols decode in segment runs when they have
// a usable index: such chunks have at least 13 segments, so a round of 512
// segments meets at most kRunChunks chunks.
constexpr int32_t kRunMinChunk = 1024;
constexpr uint32_t kRunChunks = 64;
constexpr uint32_t kRunTileWords = kThreads * kMaxSegBits / 32 + kTileSlackWords;
// The symbols of a round (at most kSlotCap per segment) after a carried
// partial group, and every group a store batch names.
constexpr uint32_t kRunStageBytes =
    (kLeadBytes + kThreads * kSlotCap + 4 + 15) / 16 * 16 > kStoreBatch * kThreads * 8
        ? (kLeadBytes + kThreads * kSlotCap + 4 + 15) / 16 * 16
        : kStoreBatch * kThreads * 8;

// Rounds, one workgroup per round of 512 segments (items numbered per
// tensor from item_begin): each entry's count becomes its place in the
// round (the counts of the round's segments before it, a block scan) and
// its chunk's place in the round's chunk table (from the chunk bases).
// Runs after the finish step, so the counts are final.
__global__ __launch_bounds__(kThreads) void index_rounds_kernel(const LaunchArgs args,
                                                                int64_t total) {
    __shared__ uint32_t s_wsum[kWaves];
    __shared__ uint32_t s_base[kRunChunks + 1];
    const uint32_t tid = threadIdx.x;
    for (int64_t item = blockIdx.x; item < total; item += gridDim.x) {
        int d = 0;
        while (d + 1 < args.n_tensors && item >= args.t[d + 1].item_begin) ++d;
        const DevTensor& T = args.t[d];
        const uint64_t m = static_cast<uint64_t>(item - T.item_begin);
        uint8_t* const ix = T.index;
        const auto* h = reinterpret_cast<const IndexHeader*>(ix);
        const uint32_t G = h->n_segments;
        if (h->magic != kIndexMagic || h->ok != 1u || m * kIndexBlock >= G) continue;
        const IndexLayout L = index_layout(T.packed_nbytes, T.n_chunks, h->seg_bits);
        const uint32_t* base = reinterpret_cast<const uint32_t*>(ix + L.base);
        uint32_t* ent = reinterpret_cast<uint32_t*>(ix + L.entries);
        const RoundStart* rounds = reinterpret_cast<const RoundStart*>(ix + L.rounds);
        const uint32_t c0 = rounds[m].chunk;
        if (tid <= kRunChunks)
            s_base[tid] = c0 + tid <= static_cast<uint32_t>(T.n_chunks) ? base[c0 + tid] : kNoIndex;
        const uint32_t g = static_cast<uint32_t>(m * kIndexBlock) + tid;
        const uint32_t e = g < G ? ent[g] : 0u;
        const uint32_t excl = block_scan_excl(g < G ? (e >> 4) & 127u : 0u, s_wsum);
        // The last chunk of the table that starts at or before g (bases do
        // not decrease; chunks without segments share their successor's).
        uint32_t jj = 0;
#pragma unroll
        for (uint32_t step = kRunChunks / 2; step >= 1; step >>= 1)
            if (jj + step < kRunChunks && s_base[jj + step] <= g) jj += step;
        if (g < G)
            ent[g] = (e & 15u) | (jj << kEntryJjShift) |
                     ((excl < (kThreads - 1) * kSlotCap ? excl : (kThreads - 1) * kSlotCap)
                      << kEntryExclShift);
        __syncthreads();  // s_base and s_wsum are written again by the next item
    }
}

struct __attribute__((aligned(16))) RunLds {
    uint8_t wmeta[kWinEntries];
    uint8_t len[256];
    uint16_t esc[kLdsEscBlocks * kEscBlockEntries];
    uint32_t wsyms[kWinEntries];
    // Chunks c0 .. c0 + kRunChunks - 1 of a round (c0: the chunk of its
    // first segment): first segment, byte offset, real end in bits. Two
    // sets, the current round's and the next one's.
    uint32_t cbase[2][kRunChunks];
    uint32_t coff[2][kRunChunks];
    uint32_t crend[2][kRunChunks];
    uint32_t segs[AIMG_MAX_TENSORS];  // run_segments of each tensor of the launch
    uint32_t tile[kRunTileWords];
    __attribute__((aligned(16))) uint8_t stage[kRunStageBytes];
};

// Tensor T's segment count when its index is usable with its table: built
// for this table (segment length, checksum), complete, and laid out for
// this tensor. 0 otherwise. (Read by one thread per tensor.)
__device__ __forceinline__ uint32_t run_segments(const DevTensor& T) {
    const uint8_t* ix = T.index;
    if (ix == nullptr) return 0u;
    const auto* h = reinterpret_cast<const IndexHeader*>(ix);
    const auto* th = reinterpret_cast<const TableHeader*>(T.table);
    const uint32_t S = segment_bits(th->min_len);
    if (h->magic != kIndexMagic || h->version != static_cast<uint32_t>(kAbiVersion) ||
        h->ok != 1u || h->seg_bits != S || h->table_checksum != th->checksum ||
        h->n_chunks != static_cast<uint32_t>(T.n_chunks) ||
        h->n_jobs != static_cast<uint32_t>(T.n_jobs))
        return 0u;
    if (index_layout(T.packed_nbytes, T.n_chunks, S).total > T.index_n32) return 0u;
    return h->n_segments;
}

// In flight for the next round: its stream words, each thread's index
// entry, and (threads below kRunChunks) one chunk of its chunk table.
struct RunFetch {
    uint32_t raw[kTileBatch];
    uint32_t ent;
    uint32_t cb, co, cr;
    v4u32 rn;   // the round start after the fetched round (its end)
    v4u32 rnx;  // the start of the workgroup's round after it
};

struct RunPos {
    uint32_t c0;   // chunk of the round's first segment
    uint32_t g0;   // the round's first segment
    uint32_t A0;   // byte of the packed buffer where its bits start
    uint32_t el;   // output element of its first symbol
};

// A round start (RoundStart) as the position of a round.
__device__ __forceinline__ RunPos run_pos(v4u32 rs, uint32_t g0, uint32_t n_jobs) {
    RunPos P;
    P.c0 = uniform(rs[0] < n_jobs ? rs[0] : n_jobs - 1u);
    P.g0 = g0;
    P.A0 = uniform(rs[2]);
    P.el = uniform(rs[1]);
    return P;
}

// Requests the words of the round at P, each thread's entry, the round's
// chunk table and the next round's start.
__device__ __forceinline__ void run_fetch_issue(RunFetch& F, const DevTensor& T,
                                                const IndexLayout& L, const RunPos& P,
                                                uint32_t s_hi, uint32_t stride, uint32_t tid) {
    const __amdgpu_buffer_rsrc_t rs = buffer_of(T.packed, T.packed_n32);
    const uint32_t last = last_word(T);
#pragma unroll
    for (uint32_t k = 0; k < kTileBatch; ++k) {
        const uint32_t A = P.A0 + 4 * (k * kThreads + tid);
        F.raw[k] = __builtin_amdgcn_raw_buffer_load_b32(rs, word_at(A, last), 0, 0);
    }
    const uint32_t g = P.g0 + tid;
    F.ent = g < s_hi ? __builtin_amdgcn_raw_buffer_load_b32(
                           index_part(T, L.entries, 4 * L.capacity), 4 * g, 0, 0)
                     : 0u;
    // Every wave loads the table (each lane one chunk, the same addresses in
    // every wave), so each wave has the same loads in flight and the waits
    // for them stay exact; the entries past the last chunk are replaced at
    // the commit. Buffer loads throughout: a flat load would also count
    // against the LDS wait counter, and the decode loop's first LDS wait
    // would wait for it.
    const uint32_t c = P.c0 + (tid & (kRunChunks - 1));
    F.cb = __builtin_amdgcn_raw_buffer_load_b32(index_part(T, L.base, 4 * (T.n_chunks + 1)),
                                                4 * c, 0, 0);
    F.cr = __builtin_amdgcn_raw_buffer_load_b32(index_part(T, L.rend, 4 * T.n_chunks), 4 * c, 0, 0);
    F.co = __builtin_amdgcn_raw_buffer_load_b32(
        buffer_of(T.offsets, static_cast<uint32_t>(4 * T.n_chunks)), 4 * c, 0, 0);
    const __amdgpu_buffer_rsrc_t rr = index_part(T, L.rounds, sizeof(RoundStart) * L.n_rounds);
    F.rn = __builtin_amdgcn_raw_buffer_load_b128(
        rr, static_cast<uint32_t>(sizeof(RoundStart)) * (P.g0 / kIndexBlock + 1), 0, 0);
    F.rnx = __builtin_amdgcn_raw_buffer_load_b128(
        rr, static_cast<uint32_t>(sizeof(RoundStart)) * (P.g0 / kIndexBlock + stride), 0, 0);
}

// The fetched words into the tile (big-endian, bytes past the packed
// buffer zero), and the chunk table of the round into set `b`.
__device__ __forceinline__ void run_fetch_commit(const RunFetch& F, const DevTensor& T,
                                                 const RunPos& P, uint32_t tid, RunLds& lds,
                                                 uint32_t b) {
#pragma unroll
    for (uint32_t k = 0; k < kTileBatch; ++k) consume(F.raw[k]);
    consume(F.ent);
    consume(F.cb);
    consume(F.co);
    consume(F.cr);
#pragma unroll
    for (uint32_t k = 0; k < 4; ++k) {
        consume(F.rn[k]);
        consume(F.rnx[k]);
    }
    const uint32_t last = last_word(T);
    uint32_t* const top = lds.tile + kRunTileWords - 1;
#pragma unroll
    for (uint32_t k = 0; k < kTileBatch; ++k) {
        const uint32_t j = k * kThreads + tid;
        if (j >= kRunTileWords) continue;
        const uint32_t A = P.A0 + 4 * j;
        uint32_t v = F.raw[k];
        v >>= 8 * ((A - word_at(A, last)) & 3u);
        *(top - j) = A < T.packed_n32 ? be_word(v, T.packed_n32 - A, 0) : 0u;
    }
    if (tid < kRunChunks) {
        const bool real = P.c0 + tid < static_cast<uint32_t>(T.n_jobs);
        lds.cbase[b][tid] = real ? F.cb : kNoIndex;
        lds.coff[b][tid] = F.co;
        lds.crend[b][tid] = F.cr;
    }
}

// Rounds m0, m0 + stride, ... (n_rounds of them) of tensor T, whose
// segments number G (usable index). With stride 1 the rounds are one run
// and a round's last partial vector group carries into the next; otherwise
// each round stores its own partial groups element by element.
template <int kMode, int kGroup>
__device__ void run_piece(RunLds& lds, const Tables& tb, bool global_esc, const LaunchArgs& args,
                          const DevTensor& T, uint32_t m0, uint32_t n_rounds, uint32_t stride,
                          uint32_t G, const uint8_t* table) {
    const uint32_t s_lo = m0 * kThreads;
    const uint32_t tid = threadIdx.x;
    const uint32_t S = segment_bits(tb.min_len);
    const IndexLayout L = index_layout(T.packed_nbytes, T.n_chunks, S);
    const uint8_t* const ix = uniform(T.index);
    const uint32_t n_jobs = static_cast<uint32_t>(T.n_jobs);
    // Where the piece starts (s_lo is a round start, a multiple of 512): its
    // chunk, the output element of its first symbol and its packed byte.
    static_assert(sizeof(RoundStart) == sizeof(v4u32), "a round start is one 16-byte load");
    const v4u32 rs = load_uniform(reinterpret_cast<const v4u32*>(ix + L.rounds) + s_lo / kIndexBlock);
    RunPos P = run_pos(rs, s_lo, n_jobs);
    // The first round's words are requested first; the table (when this
    // piece's differs from the one in LDS) and the cleared stage are
    // written while they arrive.
    RunFetch F;
    const uint32_t s_hi0 = s_lo + kThreads < G ? s_lo + kThreads : G;
    run_fetch_issue(F, T, L, P, s_hi0, stride, tid);
    if (table != nullptr) {
        __syncthreads();  // every thread is done with the previous table
        load_table(table, tid, lds.wsyms, lds.wmeta, lds.len, lds.esc);
    }
    // The stage is zero wherever nothing is placed.
    for (uint32_t j = tid; j < kRunStageBytes / 16; j += kThreads)
        reinterpret_cast<uint4*>(lds.stage)[j] = make_uint4(0u, 0u, 0u, 0u);
    run_fetch_commit(F, T, P, tid, lds, 0);

    TileRef below = (TileRef)(lds.tile + kRunTileWords - 2);
    asm volatile("" : "+v"(below));
    uint8_t* const stage = lds.stage;
    uint32_t lead = P.el & (kGroup - 1);  // symbols staged before the round's
    uint32_t skip = lead;  // of those, the ones another piece writes
    for (uint32_t r = 0; r < n_rounds; ++r) {
        const uint32_t b = r & 1u;
        const uint32_t g0 = P.g0;
        const uint32_t s_hi = g0 + kThreads < G ? g0 + kThreads : G;
        // This round's entry, its end and the workgroup's next round's start
        // (all fetched with this round's words): the next round's words are
        // requested first.
        const uint32_t ent = F.ent;
        const uint32_t end_el = uniform(F.rn[1]);
        const uint32_t gn = g0 + stride * kThreads;
        const bool more = r + 1 < n_rounds;
        const RunPos N = run_pos(F.rnx, gn, n_jobs);
        __builtin_amdgcn_s_setprio(3);
        if (more) run_fetch_issue(F, T, L, N, gn + kThreads < G ? gn + kThreads : G, stride, tid);
        const int64_t a0 = static_cast<int64_t>(P.el) - lead;
        SmBatch<kMode> smb;
        // Only this round's bytes: the next round's are another workgroup's
        // when rounds are strided (reading them here cost 3% more traffic).
        sm_issue<kMode, kGroup>(smb, T, a0, tid, kThreads, (end_el + kGroup - 1) & ~(kGroup - 1u));
        const uint32_t g = g0 + tid;
        const bool active = g < s_hi;
        // Entries above the round's room only come from an index that does
        // not describe the tensor; the clamps keep every access in bounds.
        const uint32_t ex = ent >> kEntryExclShift;
        const uint32_t excl = ex < (kThreads - 1) * kSlotCap ? ex : (kThreads - 1) * kSlotCap;
        const uint32_t jj = (ent >> kEntryJjShift) & (kRunChunks - 1);
        const uint32_t gtot0 = end_el - P.el;
        const uint32_t gtot = gtot0 < kThreads * kSlotCap ? gtot0 : kThreads * kSlotCap;
        const uint32_t avail = lead + gtot;
        // Whole groups, never past the tensor's end (only an index that does
        // not describe the tensor could place symbols there).
        const int64_t room = (T.n_symbols - a0) / kGroup;
        const uint32_t nfull = room < static_cast<int64_t>(avail / kGroup)
                                   ? static_cast<uint32_t>(room > 0 ? room : 0)
                                   : avail / kGroup;
        __syncthreads();  // the stage is clear; the tile and chunk table hold this round's
        // This thread's segment: chunk c0 + jj, segment g - base of it.
        const uint32_t cbase = lds.cbase[b][jj];
        const uint32_t coff = lds.coff[b][jj];
        const uint32_t crend = lds.crend[b][jj];
        // Compared within the chunk (chunk bits), then moved to tile bits by
        // the chunk's byte offset from the round's first byte: absolute bit
        // numbers of the packed buffer would pass 2^32 in buffers of 512 MiB.
        const uint32_t seg_lo = (g - cbase) * S;
        const uint32_t seg_hi = seg_lo + S < crend ? seg_lo + S : crend;
        const uint32_t rel = 8u * (coff - P.A0);  // tile bit of the chunk's bit 0 (mod 2^32)
        const uint32_t lo = rel + seg_lo;
        const uint32_t hi = rel + seg_hi;
        __builtin_amdgcn_s_setprio(0);
        if (active && seg_lo < crend) {
            uint8_t* dst = stage + lead + excl;
            if (global_esc) {
                decode_placed<true>(below, tb, lo + (ent & 15u), hi, dst);
            } else {
                decode_placed<false>(below, tb, lo + (ent & 15u), hi, dst);
            }
        }
        __syncthreads();  // the round is placed; the tile takes the next words
        if (more) run_fetch_commit(F, T, N, tid, lds, b ^ 1u);
        __builtin_amdgcn_s_setprio(2);
        store_round<kMode, kGroup, true>(smb, T, args.gemv, stage, a0, nfull, tid, kThreads, skip);
        const uint32_t rem0 = avail - nfull * kGroup;
        // (The fused GEMV's rounds are never strided; compiling the path for
        // it spills its registers to scratch.)
        if (kMode != kModeGemv && kMode != kModeGemv1 && stride != 1) {
            // Rounds of other workgroups follow: the partial group goes out
            // element by element (the elements before `skip` of a round's
            // first group are the previous round's).
            const uint32_t t = nfull * kGroup + tid;
            if (tid < rem0 && t >= skip) store_one<kMode>(T, args.gemv, a0 + t, stage[t]);
            const uint32_t placed = (lead + gtot + 4 + 15) & ~15u;
            const uint32_t zend = placed < kRunStageBytes ? placed : kRunStageBytes;
            __syncthreads();
            for (uint32_t z = 16 * tid; z < zend; z += 16 * kThreads)
                *reinterpret_cast<uint4*>(stage + z) = make_uint4(0u, 0u, 0u, 0u);
            lead = N.el & (kGroup - 1);
            skip = lead;
            P = N;
            continue;
        }
        if (nfull != 0) skip = 0;
        // The partial vector group (rem < 16 bytes at a multiple of kGroup)
        // moves to the front; all else placed is cleared.
        const uint32_t rem = rem0 < static_cast<uint32_t>(kGroup) ? rem0 : kGroup - 1u;
        uint2 k0 = make_uint2(0u, 0u), k1 = make_uint2(0u, 0u);
        if (tid == 0 && rem != 0) {
            const uint2* src = reinterpret_cast<const uint2*>(stage + nfull * kGroup);
            k0 = src[0];
            k1 = src[1];
            const uint64_t a = static_cast<uint64_t>(k0.x) | static_cast<uint64_t>(k0.y) << 32;
            const uint64_t bb = static_cast<uint64_t>(k1.x) | static_cast<uint64_t>(k1.y) << 32;
            const uint64_t am = rem >= 8 ? a : a & ((uint64_t{1} << (8 * rem)) - 1);
            const uint64_t bm = rem <= 8 ? 0 : bb & ((uint64_t{1} << (8 * (rem - 8))) - 1);
            k0 = make_uint2(static_cast<uint32_t>(am), static_cast<uint32_t>(am >> 32));
            k1 = make_uint2(static_cast<uint32_t>(bm), static_cast<uint32_t>(bm >> 32));
        }
        const uint32_t placed = (lead + gtot + 4 + 15) & ~15u;
        const uint32_t zend = placed < kRunStageBytes ? placed : kRunStageBytes;
        __syncthreads();
        for (uint32_t z = 16 + 16 * tid; z < zend; z += 16 * kThreads)
            *reinterpret_cast<uint4*>(stage + z) = make_uint4(0u, 0u, 0u, 0u);
        if (tid == 0) {
            reinterpret_cast<uint2*>(stage)[0] = k0;
            reinterpret_cast<uint2*>(stage)[1] = k1;
        }
        lead = rem;
        P = N;
    }
    // The symbols still staged (those of the piece's first group that
    // another piece writes excepted).
    __syncthreads();
    if (tid >= skip && tid < lead)
        store_one<kMode>(T, args.gemv, static_cast<int64_t>(P.el) - lead + tid, stage[tid]);
    __syncthreads();
}

// Chunks [c_lo, c_hi) of tensor T whose index is not usable: one thread per
// chunk decodes it whole, codeword by codeword, as the reference does (table
// in LDS). Correct for any input, slow; decoders take this path only when a
// caller passes an index that does not match the tensor's table.
// el_from: elements below it are left alone (the fused GEMV must not add a
// product twice).
template <int kMode>
__device__ void run_fallback(const Tables& tb, const LaunchArgs& args, const DevTensor& T,
                             int64_t c_lo, int64_t c_hi, int64_t el_from = 0) {
    for (int64_t c = c_lo + threadIdx.x; c < c_hi; c += kThreads) {
        int64_t off, nb;
        chunk_range(T, c, &off, &nb);
        const uint8_t* bytes = T.packed + off;
        int64_t lim = T.n_symbols - c * T.chunk_size;
        lim = lim > T.chunk_size ? T.chunk_size : lim;
        uint64_t p = 0;
        for (int64_t k = 0; k < lim; ++k) {
            uint32_t w = 0;
            const uint64_t b0 = p >> 3;
#pragma unroll
            for (uint32_t j = 0; j < 4; ++j)
                w = (w << 8) | (b0 + j < static_cast<uint64_t>(nb) ? bytes[b0 + j] : 0u);
            w <<= (p & 7u);
            const uint32_t idx = w >> (32 - kWinBits);
            uint32_t sym, len;
            if (tb.meta[idx] != 0) {
                sym = tb.syms[idx] & 0xFFu;
                len = tb.len[sym];
            } else {
                sym = escape<true>(tb, tb.syms[idx], w, &len);
            }
            if (c * T.chunk_size + k >= el_from) store_one<kMode>(T, args.gemv, c * T.chunk_size + k, sym);
            p += len;
        }
    }
}

template <int kMode, int kGroup>
__global__ __launch_bounds__(kThreads, kWavesPerSimd) void run_kernel(const LaunchArgs args) {
    __shared__ RunLds lds;
    const uint32_t tid = threadIdx.x;
    Tables tb;
    tb.syms = lds.wsyms;
    tb.meta = lds.wmeta;
    tb.len = lds.len;
    tb.esc = lds.esc;
    const uint8_t* loaded = nullptr;
    // The launch's work in rounds (512 consecutive segments of one tensor).
    // Strided (the default): workgroup w takes rounds w, w + grid, ... of
    // the launch's round sequence. Otherwise contiguous ranges of whole
    // rounds, the first `extra` workgroups taking one more (workgroups b
    // and b + 256 share a CU, so no CU takes two extra rounds while another
    // takes none; an even split of segments instead gives every workgroup a
    // last, mostly empty round).
    if (tid < static_cast<uint32_t>(args.n_tensors)) lds.segs[tid] = run_segments(args.t[tid]);
    __syncthreads();
    uint64_t units = 0;
    for (int d = 0; d < args.n_tensors; ++d)
        units += (static_cast<uint64_t>(lds.segs[d]) + kThreads - 1) / kThreads;
    const uint64_t per = units / gridDim.x, extra = units % gridDim.x;
    const uint64_t lo = blockIdx.x * per + (blockIdx.x < extra ? blockIdx.x : extra);
    const uint64_t hi = lo + per + (blockIdx.x < extra ? 1 : 0);
    uint64_t at = 0;  // rounds of the tensors before d
    for (int d = 0; d < args.n_tensors; ++d) {
        const DevTensor& T = args.t[d];
        const uint32_t G = uniform(lds.segs[d]);
        const uint64_t U = (static_cast<uint64_t>(G) + kThreads - 1) / kThreads;
        const uint64_t ua = lo > at ? lo : at;
        const uint64_t ub = hi < at + U ? hi : at + U;
        // Segments of this tensor's rounds [ua - at, ub - at).
        const uint64_t a = (ua - at) * kThreads;
        const uint64_t b0 = (ub - at) * kThreads;
        const uint64_t b = ua < ub ? (b0 < G ? b0 : G) : a;
        // Tensors without a usable index: an even share of their chunks.
        const int64_t c_lo = G != 0 ? 0 : T.n_jobs * static_cast<int64_t>(blockIdx.x) / gridDim.x;
        const int64_t c_hi = G != 0 ? 0 : T.n_jobs * static_cast<int64_t>(blockIdx.x + 1) / gridDim.x;
        const bool work = G != 0 ? (args.strided || a < b) : c_lo < c_hi;
        if (!work) {
            at += U;
            continue;
        }
        const uint8_t* const table = uniform(T.table);
        const auto* hdr = header_of(table);
        tb.sym0 = hdr->sym0;
        tb.min_len = hdr->min_len >= 1 ? hdr->min_len : 1u;
        tb.gesc = (const __attribute__((address_space(1))) uint16_t*)(table + kEscOffset);
        const bool global_esc = hdr->n_esc_blocks > static_cast<uint32_t>(kLdsEscBlocks);
        if (kMode != kModeGemv && kMode != kModeGemv1 && G != 0 && args.strided) {
            // Rounds u = blockIdx.x + k * grid of the launch's round sequence.
            const uint64_t first = at + (blockIdx.x + gridDim.x - at % gridDim.x) % gridDim.x;
            if (first < at + U) {
                const uint32_t n = static_cast<uint32_t>((at + U - 1 - first) / gridDim.x + 1);
                run_piece<kMode, kGroup>(lds, tb, global_esc, args, T,
                                         static_cast<uint32_t>(first - at), n, gridDim.x, G,
                                         table != loaded ? table : nullptr);
                loaded = table;
            }
        } else if (G != 0 && a < b) {
            // The piece loads the table itself, once its first words are
            // requested.
            run_piece<kMode, kGroup>(lds, tb, global_esc, args, T,
                                     static_cast<uint32_t>(a / kThreads),
                                     static_cast<uint32_t>((b - a + kThreads - 1) / kThreads), 1u,
                                     G, table != loaded ? table : nullptr);
            loaded = table;
        } else if (G == 0 && c_lo < c_hi) {
            if (table != loaded) {
                __syncthreads();  // every thread is done with the previous table
                loaded = table;
                load_table(table, tid, lds.wsyms, lds.wmeta, lds.len, lds.esc);
                __syncthreads();
            }
            run_fallback<kMode>(tb, args, T, c_lo, c_hi);
        }
        at += U;
    }
}

// ---------------------------------------------------------------------------
// Speculative segment runs: decode without an index of tensors whose chunks
// hold kRunMinChunk symbols or more (vector path).
//
// A workgroup takes a contiguous range of the launch's chunks and walks it in
// rounds of 512 segments that run across chunk boundaries: segment k of a
// chunk covers its bits [k S, (k + 1) S) (its last segment is shorter), and a
// round is any 512 consecutive segments of the range. A chunk's first
// segment starts at a known codeword boundary (the chunk's first bit), and
// so does a round's first segment (the end of the previous round's last);
// every other thread starts 32 bits early on a guess and is checked against
// its predecessor's end, as in decode_kernel. Each codeword gets its rank in
// its chunk (a scan over the round that restarts at each chunk's first
// segment and carries on from round to round): the symbol of rank r of chunk
// c is element c * chunk_size + r, and ranks at or past the chunk's output
// count (the zero bits that pad a chunk to whole bytes) are dropped. A
// round's output is therefore one run of elements, compacted in LDS and
// stored whole, as the segment runs with an index store theirs.
//
// The threads' slots are interleaved by lane: word j of lane l of wave w sits
// at row j, column l of the wave's block, so the lanes of a wave write and
// read their slots in 64 different banks whatever their positions.
// ---------------------------------------------------------------------------

constexpr uint32_t kSpecChunks = 64;            // chunks a round's table holds
constexpr uint32_t kSpecSlotBytes = kWaves * kSlotRows * 64 * 4;
constexpr uint32_t kSpecStageBytes = kLeadBytes + kSpecSlotBytes;
// Dense stage limit: a carried partial group and kSlotCap symbols a segment.
constexpr uint32_t kSpecDense = kLeadBytes + kThreads * kSlotCap;
static_assert(kSpecStageBytes >= kSpecDense + 4, "a dense round fits the stage");
static_assert(kSpecStageBytes >= kStoreBatch * kThreads * 8, "store batches read inside the stage");
static_assert(kSpecStageBytes >= kStoreBatch * kThreads * 16 / 2, "u8 store batches too");
static_assert(kSpecStageBytes >= kGemmRedOffset + kGemmRedBytes, "a GEMM piece and its sums fit the stage");
static_assert(kSpecStageBytes >= kSpecDense + 16, "the GEMM round keeps the carried bytes");
// A chunk of this many bytes or more makes its table unusable (the exact
// fallback decodes it): segment counts come from a multiply-high that is
// exact below it, and its bit count fits 32 bits.
constexpr int64_t kSpecMaxChunkBytes = int64_t{1} << 26;

struct __attribute__((aligned(16))) SpecLds {
    uint8_t wmeta[kWinEntries];
    uint8_t len[256];
    uint16_t esc[kLdsEscBlocks * kEscBlockEntries];
    uint32_t wsyms[kWinEntries];
    // A round's table: the chunk of its first segment and the next ones, two
    // sets (this round's and the next one's). cseg: a chunk's first segment
    // counted from the round's first ([kSpecChunks]: the end of the table's
    // segments); coff: byte offset ([kSpecChunks]: the table's last byte + 1);
    // cbits: bits.
    int32_t cseg[2][kSpecChunks + 1];
    uint32_t coff[2][kSpecChunks + 1];
    uint32_t cbits[2][kSpecChunks];
    // Per wave, from its last lane: codewords, the wave-exclusive count of its
    // last chunk head + 1 (0: none), that lane's end, disagreement inside the
    // wave. From lane 0: its start and whether that start is known.
    uint32_t rec[kWaves][4];
    uint32_t rec0[kWaves][2];
    // The round's last segment: its end (chunk bit), its chunk's codewords up
    // to its end, the stage byte after the round's symbols.
    uint32_t last[4];
    uint32_t bad;  // a chunk of the round does not hold its symbols
    uint32_t tile[kRunTileWords];
    __attribute__((aligned(16))) uint8_t stage[kSpecStageBytes];
};

// Inclusive max over the wave (every lane active).
__device__ __forceinline__ uint32_t umax(uint32_t a, uint32_t b) { return a > b ? a : b; }

__device__ __forceinline__ uint32_t wave_scan_max(uint32_t v) {
    uint32_t x = v;
    x = umax(x, dpp<0x111>(x));
    x = umax(x, dpp<0x112>(x));
    x = umax(x, dpp<0x114>(x));
    x = umax(x, dpp<0x118>(x));
    x = umax(x, dpp<0x142, 0xA>(x));
    x = umax(x, dpp<0x143, 0xC>(x));
    return x;
}

// OR of v over the wave, in every lane (every lane active).
__device__ __forceinline__ uint32_t wave_or(uint32_t v) {
    uint32_t x = v;
    x |= dpp<0x111>(x);
    x |= dpp<0x112>(x);
    x |= dpp<0x114>(x);
    x |= dpp<0x118>(x);
    x |= dpp<0x142, 0xA>(x);
    x |= dpp<0x143, 0xC>(x);
    return static_cast<uint32_t>(__builtin_amdgcn_readlane(static_cast<int>(x), 63));
}

// One chunk per lane (chunk c0 + lane) of a round's table, in flight.
struct SpecTabFetch {
    uint32_t co, cn;
};

__device__ __forceinline__ void spec_tab_issue(SpecTabFetch& F, const DevTensor& T, uint32_t c0,
                                               uint32_t lane) {
    const uint64_t n4 = 4 * static_cast<uint64_t>(T.n_chunks);
    const uint32_t lim = n4 < 0xFFFFFFFFull ? static_cast<uint32_t>(n4) : 0xFFFFFFFCu;
    const uint32_t at = 4 * (c0 + lane);
    F.co = __builtin_amdgcn_raw_buffer_load_b32(buffer_of(T.offsets, lim), at, 0, 0);
    F.cn = __builtin_amdgcn_raw_buffer_load_b32(buffer_of(T.nbytes, lim), at, 0, 0);
}

// (All fields 32-bit: a copy of a struct with padding bytes became a copy
// through scratch memory, whose loads wait for every vector memory access.)
struct SpecTab {
    uint32_t n_tab;  // chunks of the table (those below the piece's end)
    uint32_t ns;     // segments of the round (at most 512: those of the table's chunks)
    uint32_t bad;    // 1: chunks not back to back, empty, or too large
    uint32_t off0;   // byte offset of the table's first chunk
    // The next round: its first segment is segment ns of this one, in table
    // chunk `done` (n_tab: the chunk after the table), at segment k0n of it,
    // whose bytes start at offn.
    uint32_t done, k0n, offn;
};

// ceil(a / d) for a < kSpecMaxChunkBytes and d <= 21 (segment bytes), with
// m = ceil(2^32 / d): a multiply-high is exact there (a (m d - 2^32) < 2^32).
__device__ __forceinline__ uint32_t div_ceil_seg(uint32_t a, uint32_t d, uint32_t m) {
    const uint32_t q = __umulhi(a, m);
    return q + (q * d < a ? 1u : 0u);
}

// The fetched chunks into table set `set` (written by one wave; every wave
// computes the same result). k0: the round's first segment in chunk c0;
// first_off: where chunk c0 must start (the previous table's view of it).
// *jj: the table chunk of the calling thread's segment (thread 64 w + lane),
// found in registers: the chunks that start before the wave's first segment,
// and a mask of those that start inside the wave.
__device__ __forceinline__ SpecTab spec_tab_commit(const SpecTabFetch& F, const DevTensor& T,
                                                   SpecLds& lds, uint32_t set, uint32_t c0,
                                                   uint32_t cb, uint32_t k0, uint32_t first_off,
                                                   bool check_first, uint32_t S, uint32_t smagic,
                                                   uint32_t lane, uint32_t w, uint32_t* jj) {
    consume(F.co);
    consume(F.cn);
    const uint32_t c = c0 + lane;
    const bool valid = c < cb;
    int64_t off = static_cast<int32_t>(F.co), nb = static_cast<int32_t>(F.cn);
    off = off < 0 ? 0 : (off > T.packed_nbytes ? T.packed_nbytes : off);
    nb = nb < 0 ? 0 : (nb > T.packed_nbytes - off ? T.packed_nbytes - off : nb);
    const bool huge = nb >= kSpecMaxChunkBytes;
    const uint32_t nbv = valid && !huge ? static_cast<uint32_t>(nb) : 0u;
    const uint32_t offv = static_cast<uint32_t>(off);
    const uint32_t nseg = div_ceil_seg(nbv, S / 8, smagic);
    const int64_t lim = T.n_symbols - static_cast<int64_t>(c) * T.chunk_size;
    const uint32_t incl = wave_scan_incl(nseg);
    const uint32_t prev_end = lane_below(offv + nbv);
    const bool bad = valid && (huge || (nseg == 0 && lim > 0) ||
                               (lane > 0 && offv != prev_end) ||
                               (lane == 0 && check_first && offv != first_off));
    const uint64_t vm = __ballot(valid);
    const uint32_t n_tab = static_cast<uint32_t>(__builtin_popcountll(vm));  // lanes 0 .. n_tab - 1
    const uint32_t total = static_cast<uint32_t>(__builtin_amdgcn_readlane(static_cast<int>(incl), 63));
    const uint32_t end_off = static_cast<uint32_t>(__builtin_amdgcn_readlane(
        static_cast<int>(offv + nbv), static_cast<int>(n_tab > 0 ? n_tab - 1 : 0)));
    const bool any_bad = __ballot(bad) != 0;
    const uint32_t off0 = static_cast<uint32_t>(__builtin_amdgcn_readlane(static_cast<int>(offv), 0));
    const int32_t first = static_cast<int32_t>(incl - nseg) - static_cast<int32_t>(k0);
    const int32_t end = static_cast<int32_t>(total) - static_cast<int32_t>(k0);
    const uint32_t ns = end <= 0 ? 0u : (end < static_cast<int32_t>(kThreads) ? static_cast<uint32_t>(end) : kThreads);
    const uint32_t done = static_cast<uint32_t>(__builtin_popcountll(
        __ballot(valid && static_cast<int32_t>(incl) - static_cast<int32_t>(k0) <= static_cast<int32_t>(ns))));
    const uint32_t k0n = done < n_tab ? ns - static_cast<uint32_t>(__builtin_amdgcn_readlane(
                                                 static_cast<int>(first), static_cast<int>(done)))
                                      : 0u;
    const uint32_t offn = done < n_tab ? static_cast<uint32_t>(__builtin_amdgcn_readlane(
                                             static_cast<int>(offv), static_cast<int>(done)))
                                       : end_off;
    const int32_t rel = first - static_cast<int32_t>(64 * w);
    const uint32_t before = static_cast<uint32_t>(__builtin_popcountll(__ballot(valid && rel < 0)));
    const bool inside = valid && rel >= 0 && rel < 64;
    const uint64_t bit = inside ? uint64_t{1} << rel : 0u;
    const uint64_t heads = static_cast<uint64_t>(wave_or(static_cast<uint32_t>(bit))) |
                           static_cast<uint64_t>(wave_or(static_cast<uint32_t>(bit >> 32))) << 32;
    const uint64_t upto = lane == 63 ? ~uint64_t{0} : (uint64_t{2} << lane) - 1;
    const uint32_t cnt = before + static_cast<uint32_t>(__builtin_popcountll(heads & upto));
    *jj = cnt > 0 ? cnt - 1 : 0u;
    if (w == 0) {
        lds.cseg[set][lane] = first;
        lds.coff[set][lane] = valid ? offv : end_off;
        lds.cbits[set][lane] = 8 * nbv;
        if (lane == 0) {
            lds.cseg[set][kSpecChunks] = static_cast<int32_t>(total) - static_cast<int32_t>(k0);
            lds.coff[set][kSpecChunks] = end_off;
        }
    }
    return {n_tab, uniform(ns), any_bad || ns == 0 ? 1u : 0u, uniform(off0), uniform(done),
            uniform(k0n), uniform(offn)};
}

__device__ __forceinline__ void spec_tile_issue(uint32_t (&raw)[kTileBatch], const DevTensor& T,
                                                uint32_t A0, uint32_t tid) {
    const __amdgpu_buffer_rsrc_t rs = buffer_of(T.packed, T.packed_n32);
    const uint32_t last = last_word(T);
#pragma unroll
    for (uint32_t k = 0; k < kTileBatch; ++k) {
        const uint32_t A = A0 + 4 * (k * kThreads + tid);
        raw[k] = __builtin_amdgcn_raw_buffer_load_b32(rs, word_at(A, last), 0, 0);
    }
}

__device__ __forceinline__ void spec_tile_commit(const uint32_t (&raw)[kTileBatch], const DevTensor& T,
                                                 uint32_t A0, uint32_t tid, uint32_t* tile) {
#pragma unroll
    for (uint32_t k = 0; k < kTileBatch; ++k) consume(raw[k]);
    const uint32_t last = last_word(T);
    uint32_t* const top = tile + kRunTileWords - 1;
#pragma unroll
    for (uint32_t k = 0; k < kTileBatch; ++k) {
        const uint32_t j = k * kThreads + tid;
        if (j >= kRunTileWords) continue;
        const uint32_t A = A0 + 4 * j;
        uint32_t v = raw[k];
        v >>= 8 * ((A - word_at(A, last)) & 3u);
        *(top - j) = A < T.packed_n32 ? be_word(v, T.packed_n32 - A, 0) : 0u;
    }
}

// Chunks [ca, cb) of tensor T (all of them below n_jobs).
template <int kMode, int kGroup>
__device__ void spec_piece(SpecLds& lds, const Tables& tb, bool global_esc, const LaunchArgs& args,
                           const DevTensor& T, uint32_t ca, uint32_t cb, const uint8_t* table,
                           uint32_t pre_c0 = 0xFFFFFFFFu) {
    const uint32_t tid = threadIdx.x;
    const uint32_t lane = tid & 63u, w = uniform(tid >> 6);
    const uint32_t S = segment_bits(tb.min_len);
    const uint32_t smagic = static_cast<uint32_t>(((uint64_t{1} << 32) + S / 8 - 1) / (S / 8));
    const int64_t cs = T.chunk_size;
    // The piece's first table and words; the decode table (when it changes)
    // loads while they arrive. Chunks from pre_c0 on, when set: their offsets
    // and lengths are in the stage already (those of the piece's chunks).
    SpecTabFetch TF;
    if (pre_c0 != 0xFFFFFFFFu) {
        const uint32_t* const pre = reinterpret_cast<const uint32_t*>(lds.stage);
        const uint32_t j = ca - pre_c0 + lane;
        TF.co = j < kThreads ? pre[j] : 0u;
        TF.cn = j < kThreads ? pre[kThreads + j] : 0u;
    } else {
        spec_tab_issue(TF, T, ca, lane);
    }
    if (table != nullptr) {
        __syncthreads();  // every thread is done with the previous table
        load_table(table, tid, lds.wsyms, lds.wmeta, lds.len, lds.esc);
    }
    uint32_t b = 0;
    uint32_t jj = 0;
    SpecTab tab = spec_tab_commit(TF, T, lds, b, ca, cb, 0u, 0u, false, S, smagic, lane, w, &jj);
    uint32_t c0 = ca;     // chunk of the round's first segment
    uint32_t p0 = 0;      // chunk bit where its first codeword starts (k0 > 0)
    GemmAcc gacc;         // fused GEMM: this wave's partial sums
    gemm_acc_init(gacc);
    uint32_t rank0 = 0;   // codewords of chunk c0 before the round
    uint32_t lead = 0;    // carried symbols at the front of the stage
    int64_t a0 = static_cast<int64_t>(ca) * cs;  // element of stage byte 0
    uint32_t A0 = tab.off0;  // packed byte of the round's first segment
    int64_t fall_from = tab.bad != 0u ? a0 : -1;  // the first element the exact fallback writes
    uint32_t raw[kTileBatch];
    if (fall_from < 0) spec_tile_issue(raw, T, A0, tid);
    if (tid == 0) lds.bad = 0u;
    __syncthreads();  // table set 0 is written
    if (fall_from < 0) spec_tile_commit(raw, T, A0, tid, lds.tile);
    __syncthreads();  // the first round's words are in the tile

    TileRef below = (TileRef)(lds.tile + kRunTileWords - 2);
    asm volatile("" : "+v"(below));
    uint8_t* const stage = lds.stage;
    uint32_t* const slot = reinterpret_cast<uint32_t*>(lds.stage + kLeadBytes) + w * kSlotRows * 64 + lane;
    const IlSlot sl{lds.stage + kLeadBytes, w * kSlotRows * 256u, lane * 4u};
    const int64_t piece_end = static_cast<int64_t>(cb) * cs < T.n_symbols ? static_cast<int64_t>(cb) * cs
                                                                         : T.n_symbols;
    while (fall_from < 0) {
        const uint32_t ns = tab.ns;
        // The next round (found when this round's table was committed).
        const uint32_t c0n = c0 + tab.done;
        const bool more = c0n < cb;
        const uint32_t k0n = tab.k0n;
        const uint32_t offn = tab.offn;
        const uint32_t A0n = offn + k0n * (S / 8);
        __builtin_amdgcn_s_setprio(3);
        if (more) {
            spec_tile_issue(raw, T, A0n, tid);
            spec_tab_issue(TF, T, c0n, lane);
        }
        SmBatch<kMode> smb;
        sm_issue<kMode, kGroup>(smb, T, a0, tid, kThreads, static_cast<uint32_t>(piece_end));

        // Chunk c0's output count and the stage's first place in it.
        const uint32_t lim0 = static_cast<uint32_t>(
            T.n_symbols - static_cast<int64_t>(c0) * cs < cs ? T.n_symbols - static_cast<int64_t>(c0) * cs : cs);
        const uint32_t base0 = rank0 < lim0 ? rank0 : lim0;
        // This thread's segment: segment kseg of chunk c0 + jj.
        const bool active = tid < ns;
        const int32_t kseg = static_cast<int32_t>(tid) - lds.cseg[b][jj];
        const uint32_t rel = 8u * (lds.coff[b][jj] - A0);  // tile bit of the chunk's bit 0 (mod 2^32)
        const uint32_t cbits = lds.cbits[b][jj];
        const uint32_t lo_c = static_cast<uint32_t>(kseg) * S;
        const uint32_t hi_c = lo_c + S < cbits ? lo_c + S : cbits;
        const uint32_t lo = rel + lo_c, hi = rel + hi_c, cend = rel + cbits;
        const bool known = !active || kseg == 0 || tid == 0;
        uint32_t f = 0, e = 0, cnt = 0;
        __builtin_amdgcn_s_setprio(0);
        if (active) {
            Adv a;
            if (global_esc) {
                f = kseg == 0 ? lo : tid == 0 ? rel + p0 : advance<true>(below, tb, lo - kOverlapBits, lo);
                a = decode_run_il<true>(below, tb, f, hi, cend, sl);
            } else {
                f = kseg == 0 ? lo : tid == 0 ? rel + p0 : advance<false>(below, tb, lo - kOverlapBits, lo);
                a = decode_run_il<false>(below, tb, f, hi, cend, sl);
            }
            e = a.p;
            cnt = a.n;
        }
        __builtin_amdgcn_s_setprio(1);
        // Agreement and scans. Each wave checks its lanes against the lane
        // below and scans its counts; its last lane and lane 0 leave a record,
        // from which, after one barrier, every wave checks the waves' first
        // lanes and finds its codewords' ranks.
        const bool head = active && kseg == 0;
        uint32_t incl, hm;
        for (;;) {
            const uint32_t ep0 = lane_below(e);
            incl = wave_scan_incl(cnt);
            hm = wave_scan_max(head ? incl - cnt + 1u : 0u);
            const bool wbad = __ballot(!known && lane != 0 && f != ep0) != 0;
            if (lane == 63) {
                lds.rec[w][0] = incl;
                lds.rec[w][1] = hm;
                lds.rec[w][2] = e;
                lds.rec[w][3] = wbad ? 1u : 0u;
            }
            if (lane == 0) {
                lds.rec0[w][0] = f;
                lds.rec0[w][1] = known ? 1u : 0u;
            }
            __syncthreads();
            const uint32_t lw = lane & (kWaves - 1);
            const bool xbad = lw > 0 && lds.rec0[lw][1] == 0u && lds.rec0[lw][0] != lds.rec[lw - 1][2];
            if (__ballot(lane < kWaves && (lds.rec[lw][3] != 0u || xbad)) == 0) break;
            // Rare: threads whose start disagrees with their predecessor's
            // end decode again from it. Thread 0 and chunk starts are always
            // right, so pass k puts thread k right at the latest.
            const uint32_t ep = lane == 0 ? (w > 0 ? lds.rec[w - 1][2] : 0u) : ep0;
            const bool redo = !known && f != ep;
            __syncthreads();  // the records are read before they are written again
            if (redo) {
                f = ep;
                const Adv a = global_esc ? decode_run_il<true>(below, tb, f, hi, cend, sl)
                                         : decode_run_il<false>(below, tb, f, hi, cend, sl);
                e = a.p;
                cnt = a.n;
            }
        }
        // Codewords of this lane's chunk before it: from its last head in the
        // wave, or carried from the waves before (and the rounds before).
        const uint32_t r_tot = lds.rec[lane & (kWaves - 1)][0];
        const uint32_t r_hm = lds.rec[lane & (kWaves - 1)][1];
        uint32_t carry = 0;
        bool found = false;
        for (int32_t v = static_cast<int32_t>(w) - 1; v >= 0; --v) {
            const uint32_t tv = static_cast<uint32_t>(__builtin_amdgcn_readlane(static_cast<int>(r_tot), v));
            const uint32_t hv = static_cast<uint32_t>(__builtin_amdgcn_readlane(static_cast<int>(r_hm), v));
            if (hv != 0u) {
                carry += tv - (hv - 1u);
                found = true;
                break;
            }
            carry += tv;
        }
        if (!found) carry += rank0;
        const uint32_t xw = incl - cnt;
        const uint32_t rank = hm != 0u ? xw - (hm - 1u) : carry + xw;
        // Stage place: chunk jj's element r is stage byte
        // lead + jj cs + r - min(rank0, lim of chunk c0). (32-bit: elements
        // below 2^31, chunk_size below 2^24 and jj below 64.)
        const uint32_t cs32 = static_cast<uint32_t>(cs);
        const uint32_t n32 = static_cast<uint32_t>(T.n_symbols);
        const uint32_t left = n32 - (c0 + jj) * cs32;
        const uint32_t lim = left < cs32 ? left : cs32;
        const uint32_t kept = rank < lim ? (cnt < lim - rank ? cnt : lim - rank) : 0u;
        const uint32_t pos = lead + jj * cs32 + (rank < lim ? rank : lim) - base0;
        const bool at_end = hi_c == cbits;  // the chunk's last segment
        const bool broken = active && ((at_end && rank + cnt < lim) || pos > kSpecDense ||
                                       kept > kSpecDense - pos);
        if (broken) lds.bad = 1u;
        const uint32_t dpos = broken ? 0u : pos;
        if (active && tid == ns - 1) {
            lds.last[0] = e - rel;
            lds.last[1] = rank + cnt;
            lds.last[2] = dpos + kept;
        }
        // Compaction, part 1: the slot into registers (the dense stage
        // overlaps the slots).
        const uint32_t m = active && !broken ? kept : 0u;
        const uint32_t head0 = (4u - (dpos & 3u)) & 3u;
        const uint32_t hb = head0 < m ? head0 : m;  // bytes before the first aligned word
        const uint32_t nbody = (m - hb) >> 2;
        const uint32_t ntail = m - hb - 4 * nbody;
        uint32_t rw[kSlotRows];
        {
            const auto* sl = lds_ptr(slot);
#pragma unroll
            for (uint32_t j = 0; j < kSlotRows; ++j) rw[j] = sl[j * 64];
        }
        const uint32_t tv = __builtin_amdgcn_alignbyte(
            slot[(nbody + 1 < kSlotRows ? nbody + 1 : kSlotRows - 1) * 64], slot[nbody * 64], hb);
        // Every thread is past its decode: the next round's words and table.
        SpecTab tabn = tab;
        uint32_t jjn = 0;
        if (more) {
            spec_tile_commit(raw, T, A0n, tid, lds.tile);
            tabn = spec_tab_commit(TF, T, lds, b ^ 1u, c0n, cb, k0n, offn, true, S, smagic, lane, w,
                                   &jjn);
        }
        __syncthreads();  // B: slots read; the next table and words written
        const bool bad_round = lds.bad != 0u;
        const uint32_t avail = uniform(lds.last[2]);
        const uint32_t p0n = uniform(lds.last[0]);
        const uint32_t rank0n = uniform(lds.last[1]);
        if (!bad_round) {
            // Head: the last hb bytes of a word (a byte at an odd address,
            // then an aligned pair); body: whole words; tail: the first
            // ntail bytes of a word (an aligned pair, then a byte).
            uint8_t* dst = stage + dpos;
            if (hb & 1u) dst[0] = static_cast<uint8_t>(rw[0]);
            if (hb >= 2) *reinterpret_cast<uint16_t*>(dst + hb - 2) = static_cast<uint16_t>(rw[0] >> (8 * (hb - 2)));
            // Body words, each under its own lane mask at a constant offset
            // from the first.
            uint32_t* const body = reinterpret_cast<uint32_t*>(dst + hb);
#pragma unroll
            for (uint32_t j = 0; j + 1 < kSlotRows; ++j)
                if (j < nbody) body[j] = __builtin_amdgcn_alignbyte(rw[j + 1], rw[j], hb);
            uint8_t* tl = dst + hb + 4 * nbody;
            if (ntail >= 2) *reinterpret_cast<uint16_t*>(tl) = static_cast<uint16_t>(tv);
            if (ntail & 1u) tl[ntail - 1] = static_cast<uint8_t>(tv >> (8 * (ntail - 1)));
        }
        __syncthreads();  // C: the round's symbols are in place
        if (bad_round) {
            fall_from = a0;
            break;
        }
        // Whole vector groups, never past the piece's end.
        const int64_t room = (piece_end - a0) / kGroup;
        const uint32_t nfull0 = avail / kGroup;
        const uint32_t nfull = room < static_cast<int64_t>(nfull0) ? static_cast<uint32_t>(room > 0 ? room : 0)
                                                                  : nfull0;
        __builtin_amdgcn_s_setprio(2);
        store_round<kMode, kGroup, true>(smb, T, args.gemv, stage, a0, nfull, tid, kThreads, 0, &gacc);
        // The partial vector group moves to the front.
        const uint32_t rem0 = avail - nfull * kGroup;
        const uint32_t rem = rem0 < static_cast<uint32_t>(kGroup) ? rem0 : kGroup - 1u;
        uint2 keep0 = make_uint2(0u, 0u), keep1 = make_uint2(0u, 0u);
        if (tid == 0 && rem != 0) {
            const uint2* src = reinterpret_cast<const uint2*>(stage + nfull * kGroup);
            keep0 = src[0];
            keep1 = src[1];
        }
        __syncthreads();  // D: the round is stored
        if (tid == 0) {
            reinterpret_cast<uint2*>(stage)[0] = keep0;
            reinterpret_cast<uint2*>(stage)[1] = keep1;
            lds.bad = 0u;
        }
        a0 += static_cast<int64_t>(nfull) * kGroup;
        lead = rem;
        if (!more) break;
        if (tabn.bad != 0u) {
            fall_from = a0;
            break;
        }
        // The next round continues chunk c0n at segment k0n (> 0), or starts it.
        rank0 = k0n > 0 ? rank0n : 0u;
        p0 = k0n > 0 ? p0n : 0u;
        c0 = c0n;
        A0 = A0n;
        b ^= 1u;
        tab = tabn;
        jj = jjn;
    }
    __syncthreads();  // the carried symbols are at the front
    if (fall_from < 0) {
        if (tid < lead) store_one<kMode>(T, args.gemv, a0 + tid, stage[tid]);
    } else {
        // A chunk that does not hold its symbols, or chunks not back to back:
        // from fall_from on, each chunk is decoded by one thread codeword by
        // codeword (exact on any input).
        run_fallback<kMode>(tb, args, T, fall_from / cs, cb, fall_from);
    }
    if constexpr (is_gemm(kMode)) gemm_finish(gacc, args.gemv, stage);
    __syncthreads();  // LDS is free for the next piece
}

// floor(a b / c) for a < 2^31, b < 2^16 and c >= 1: the products stay below
// 2^47, where the rounded double quotient is within one of the true one.
__device__ __forceinline__ uint32_t mul_div(uint32_t a, uint32_t b, uint32_t c) {
    const uint64_t x = static_cast<uint64_t>(a) * b;
    uint64_t q = static_cast<uint64_t>(static_cast<double>(x) / static_cast<double>(c));
    if (q * c > x)
        --q;
    else if ((q + 1) * c <= x)
        ++q;
    return static_cast<uint32_t>(q);
}

// How a CU's chunks [ca, cb) of one tensor split between its two
// workgroups: the first takes the first k of them (returned), the second the
// rest. Rounds hold 512 segments (a chunk's may straddle two), so at the
// middle both workgroups would often end in a partial round, R + 1 rounds for
// the CU where R would do. The second workgroup takes instead the last chunks
// that fit in floor(R / 2) whole rounds, the first the rest (its last round
// partial). Shares of at most kThreads chunks (the 5120x17408 layer at
// 1024-symbol chunks: 340 a CU); larger ones split at the middle. Every
// thread of both workgroups finds the same k.
// The chunks' offsets and lengths, loaded here, stay in the stage
// (pre[0 .. kThreads) and pre[kThreads ..), chunk *pre_c0 first) for the
// piece's first round table, and the tensor's decode table is loaded into
// LDS while they arrive (*pre_c0 = 0xFFFFFFFF: neither was done).
// Every wave of both workgroups runs this once, before the rounds: its
// instructions count (a thousand a wave: about 2 us on the layer's grid).
__device__ uint32_t spec_split(const DevTensor& T, uint32_t ca, uint32_t cb, SpecLds& lds,
                               uint32_t* pre_c0) {
    *pre_c0 = 0xFFFFFFFFu;
    const uint32_t n = cb - ca;
    if (n < 2 || n > static_cast<uint32_t>(kThreads)) return n / 2;
    const uint32_t tid = threadIdx.x;
    SpecTabFetch F;  // chunk ca + tid (0 past the chunk count)
    {
        const uint64_t n4 = 4 * static_cast<uint64_t>(T.n_chunks);
        const uint32_t lim = n4 < 0xFFFFFFFFull ? static_cast<uint32_t>(n4) : 0xFFFFFFFCu;
        F.co = __builtin_amdgcn_raw_buffer_load_b32(buffer_of(T.offsets, lim), 4 * (ca + tid), 0, 0);
        F.cn = __builtin_amdgcn_raw_buffer_load_b32(buffer_of(T.nbytes, lim), 4 * (ca + tid), 0, 0);
    }
    const uint8_t* const table = uniform(T.table);
    load_table(table, tid, lds.wsyms, lds.wmeta, lds.len, lds.esc);
    consume(F.co);
    consume(F.cn);
    uint32_t* const pre = reinterpret_cast<uint32_t*>(lds.stage);
    pre[tid] = F.co;
    pre[kThreads + tid] = F.cn;
    // Segments of the chunk, as the round table counts them.
    const uint32_t S = segment_bits(header_of(table)->min_len);
    const uint32_t smagic = static_cast<uint32_t>(((uint64_t{1} << 32) + S / 8 - 1) / (S / 8));
    int64_t off = static_cast<int32_t>(F.co), nb = static_cast<int32_t>(F.cn);
    off = off < 0 ? 0 : (off > T.packed_nbytes ? T.packed_nbytes : off);
    nb = nb < 0 ? 0 : (nb > T.packed_nbytes - off ? T.packed_nbytes - off : nb);
    const uint32_t nseg = tid < n && nb < kSpecMaxChunkBytes
                              ? div_ceil_seg(static_cast<uint32_t>(nb), S / 8, smagic)
                              : 0u;
    uint32_t* const s_wsum = &lds.rec[0][0];  // free until the first round
    if (tid == 0) lds.last[0] = 0u;
    const uint32_t excl = block_scan_excl(nseg, s_wsum);
    uint32_t total = 0;
#pragma unroll
    for (int k = 0; k < kWaves; ++k) total += s_wsum[k];
    const uint32_t rounds = (total + kThreads - 1) / kThreads;
    // The first workgroup's chunks: those that start before its share ends,
    // a prefix of the share (its segment counts only grow); the thread of
    // its last chunk writes their number (an atomic maximum over all of them
    // took 2.5 us: the LDS serialises updates of one word).
    const uint32_t first_share = total - rounds / 2 * kThreads;
    const bool mine = tid < n && excl < first_share;
    const bool next = tid + 1 < n && excl + nseg < first_share;
    if (mine && !next) lds.last[0] = tid + 1;
    __syncthreads();
    const uint32_t k = uniform(lds.last[0]);
    __syncthreads();  // read before the rounds use these words
    *pre_c0 = ca;
    return k;
}

// The launch's tensors in one sequence of elements; each workgroup takes the
// chunks whose first element lies in its share. On a full grid (args.strided
// set) workgroups b and b + grid / 2 are taken to share a CU and split one
// CU's share; a launch of one tensor there shares out chunks instead
// (n_jobs b / (grid / 2) on), split by spec_split.
template <int kMode, int kGroup>
__global__ __launch_bounds__(kThreads, kWavesPerSimd) void spec_kernel(const LaunchArgs args) {
    __shared__ SpecLds lds;
    Tables tb;
    tb.syms = lds.wsyms;
    tb.meta = lds.wmeta;
    tb.len = lds.len;
    tb.esc = lds.esc;
    const uint32_t G = gridDim.x;
    const uint32_t P = args.strided != 0 && G % 2 == 0 ? G / 2 : G;
    const uint32_t s = blockIdx.x % P, h = blockIdx.x / P;
    // (One call of spec_piece below: a second copy of it made the batch-4
    // GEMV's registers spill to scratch memory, 4x slower.)
    const bool by_chunks = P != G && args.n_tensors == 1;
    uint32_t pre_c0 = 0xFFFFFFFFu;
    uint32_t ca_w = 0, cb_w = 0;  // by_chunks: this workgroup's chunks
    int64_t lo = 0, hi = 0;       // otherwise: its share of the elements
    if (by_chunks) {
        const DevTensor& T = args.t[0];
        const uint32_t nj = static_cast<uint32_t>(T.n_jobs);
        const uint32_t ca_cu = mul_div(nj, s, P), cb_cu = mul_div(nj, s + 1, P);
        const uint32_t k = spec_split(T, ca_cu, cb_cu, lds, &pre_c0);
        ca_w = h == 0 ? ca_cu : ca_cu + k;
        cb_w = h == 0 ? ca_cu + k : cb_cu;
    } else {
        const int64_t N = args.total_items;
        const int64_t L = N * s / P, R = N * (s + 1) / P;
        const int64_t mid = (L + R) / 2;
        lo = P == G ? L : (h == 0 ? L : mid);
        hi = P == G ? R : (h == 0 ? mid : R);
    }
    const uint8_t* loaded = pre_c0 != 0xFFFFFFFFu ? uniform(args.t[0].table) : nullptr;
    int64_t O = 0;  // first element of tensor d in the sequence
    for (int d = 0; d < args.n_tensors; ++d) {
        const DevTensor& T = args.t[d];
        const int64_t cs = T.chunk_size;
        int64_t ca = ca_w, cb = cb_w;
        if (!by_chunks) {
            ca = lo - O <= 0 ? 0 : (lo - O + cs - 1) / cs;
            cb = hi - O <= 0 ? 0 : (hi - O + cs - 1) / cs;
            ca = ca < T.n_jobs ? ca : T.n_jobs;
            cb = cb < T.n_jobs ? cb : T.n_jobs;
        }
        O += T.n_symbols;
        if (ca >= cb) continue;
        const uint8_t* const table = uniform(T.table);
        const auto* hdr = header_of(table);
        tb.sym0 = hdr->sym0;
        tb.min_len = hdr->min_len >= 1 ? hdr->min_len : 1u;
        tb.gesc = (const __attribute__((address_space(1))) uint16_t*)(table + kEscOffset);
        const bool global_esc = hdr->n_esc_blocks > static_cast<uint32_t>(kLdsEscBlocks);
        spec_piece<kMode, kGroup>(lds, tb, global_esc, args, T, static_cast<uint32_t>(ca),
                                  static_cast<uint32_t>(cb), table != loaded ? table : nullptr,
                                  d == 0 ? pre_c0 : 0xFFFFFFFFu);
        loaded = table;
    }
}

// The handoff records of split chunks, one array per GPU (zero when the
// library loads; every launch leaves its records empty). Kernels take its
// device address, found once per device with that device current.
__device__ __attribute__((aligned(256))) uint64_t scratch[kHandoffSlots * kHandoffWords];

int handoff_records(uint64_t** out) {
    static std::mutex mu;
    static uint64_t* ptr[64] = {};
    int dev = 0;
    const hipError_t ge = hipGetDevice(&dev);
    if (ge != hipSuccess) return fail(AIMG_ERR_HIP, std::string("hipGetDevice: ") + hipGetErrorString(ge));
    if (dev < 0 || dev >= 64) {
        *out = nullptr;  // no records: chunks are not split
        return AIMG_OK;
    }
    std::lock_guard<std::mutex> lock(mu);
    if (ptr[dev] == nullptr) {
        void* p = nullptr;
        const hipError_t e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
        if (e != hipSuccess || p == nullptr)
            return fail(AIMG_ERR_HIP, std::string("hipGetSymbolAddress (chunk handoff records): ") +
                                          hipGetErrorString(e));
        ptr[dev] = static_cast<uint64_t*>(p);
    }
    *out = ptr[dev];
    return AIMG_OK;
}

// A launch's record tag: never 0, so that a written record is never 0.
uint32_t next_tag() {
    static std::atomic<uint32_t> n{0};
    uint32_t t = 0;
    while (t == 0) t = n.fetch_add(1, std::memory_order_relaxed) + 1;
    return t;
}

int cu_count() {
    static std::once_flag once;
    static int n = 0;
    std::call_once(once, [] {
        int dev = 0;
        if (hipGetDevice(&dev) != hipSuccess ||
            hipDeviceGetAttribute(&n, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess)
            n = 0;
    });
    return n > 0 ? n : 256;
}

uint32_t threads_per_chunk(int32_t chunk_size) {
    uint32_t t = kMinTpc;
    while (t < static_cast<uint32_t>(kThreads) &&
           static_cast<int64_t>(t) * kSlotCap < chunk_size)
        t <<= 1;
    return t;
}

// Tensors of one launch: those whose packed buffer has fewer than 4 bytes go
// to a kernel of their own (see fetch_issue).
struct Batch {
    LaunchArgs args{};
    int64_t items = 0;
    int m = 0;
    bool vec = true;
    bool full = true;  // every tensor has kThreads threads per chunk
};

// Whole-workgroup chunks of bf16 and exponent-byte launches: when the grid's
// last pass over the chunks has more of them than half the grid (1360 chunks
// on 512 workgroups: 336), the CUs that decode two of the last chunks finish
// a chunk's rounds later than the rest. Those chunks are split in two halves
// of their rounds: the first halves go first in the grid, the second halves
// last, so that every workgroup has 5 or 6 rounds and every CU 10 or 11
// (instead of 10 or 12), and a second half finds its record long written.
// Each first half hands its state (where the next round starts, the symbols
// placed, the carried partial group) to its second half through a record.
// AIMG_CHUNK_SPLIT=0 turns this off.
// The most rounds any CU decodes (2 a chunk, 1 a half; the grid's
// workgroups w and w + slots / 2 share a CU) when the last `rest` of n chunks
// are split (rest 0: none).
int64_t max_cu_rounds(int64_t n, int64_t rest, int64_t slots) {
    const int64_t items = n + rest;
    auto wg = [&](int64_t w) {
        int64_t r = 0;
        for (int64_t i = w; i < items; i += slots) r += i < rest || i >= n ? 1 : 2;
        return r;
    };
    int64_t m = 0;
    for (int64_t c = 0; c < slots / 2; ++c) {
        const int64_t r = wg(c) + wg(c + slots / 2);
        m = r > m ? r : m;
    }
    return m;
}

int plan_split(LaunchArgs& a, int64_t n, int64_t slots) {
    a.n_split = 0;
    a.split_first = n;
    const char* e = std::getenv("AIMG_CHUNK_SPLIT");
    if (e != nullptr && e[0] == '0') return AIMG_OK;
    if (n <= slots || slots % 2 != 0) return AIMG_OK;
    const int64_t rest = n % slots;
    if (2 * rest <= slots || rest > static_cast<int64_t>(kHandoffSlots)) return AIMG_OK;
    // Only where it lowers the busiest CU's rounds (the 14B block's 5042
    // chunks already spread to 40 or 38 rounds a CU: no split).
    if (max_cu_rounds(n, rest, slots) >= max_cu_rounds(n, 0, slots)) return AIMG_OK;
    uint64_t* rec = nullptr;
    const int rc = handoff_records(&rec);
    if (rc != AIMG_OK || rec == nullptr) return rc;
    a.n_split = rest;
    a.split_first = n - rest;
    a.total_items = n + rest;
    a.handoff = rec;
    a.tag = next_tag();
    return AIMG_OK;
}

template <int kMode>
int launch_batch(Batch& B, hipStream_t s, bool tiny) {
    B.args.n_tensors = B.m;
    B.args.total_items = B.items;
    B.args.n_split = 0;
    if (B.items == 0) return AIMG_OK;
    const int64_t slots = static_cast<int64_t>(cu_count()) * kBlocksPerCu;
    if constexpr (kMode == kModeBf16 || kMode == kModeU8) {
        if (!tiny && B.vec && B.full) {
            const int rc = plan_split(B.args, B.items, slots);
            if (rc != AIMG_OK) return rc;
        }
    }
    const int64_t grid = B.args.total_items < slots ? B.args.total_items : slots;
    // (Decodes only: the fused GEMV at batch 1 and 4 was 4.5% slower staggered.)
    const char* stag = std::getenv("AIMG_STAGGER");
    B.args.stagger = (kMode == kModeBf16 || kMode == kModeU8) && grid == slots && slots % 2 == 0 &&
                             !(stag != nullptr && stag[0] == '0')
                         ? 1
                         : 0;
    const dim3 gdim(static_cast<uint32_t>(grid)), bdim(kThreads);
    constexpr int kVecGroup = kMode == kModeU8 ? 16 : 8;
    if constexpr (kMode == kModeIndex) {
        // No output: one kernel per sub-group geometry.
        if (tiny)
            hipLaunchKernelGGL((decode_kernel<kMode, 1, true, 0>), gdim, bdim, 0, s, B.args);
        else if (B.full)
            hipLaunchKernelGGL((decode_kernel<kMode, 1, false, kLgThreads>), gdim, bdim, 0, s, B.args);
        else
            hipLaunchKernelGGL((decode_kernel<kMode, 1, false, 0>), gdim, bdim, 0, s, B.args);
    } else {
    if (tiny) {
        hipLaunchKernelGGL((decode_kernel<kMode, 1, true, 0>), gdim, bdim, 0, s, B.args);
    } else if (B.vec && B.full) {
        hipLaunchKernelGGL((decode_kernel<kMode, kVecGroup, false, kLgThreads>), gdim, bdim, 0, s, B.args);
    } else if (B.vec) {
        hipLaunchKernelGGL((decode_kernel<kMode, kVecGroup, false, 0>), gdim, bdim, 0, s, B.args);
    } else {
        hipLaunchKernelGGL((decode_kernel<kMode, 1, false, 0>), gdim, bdim, 0, s, B.args);
    }
    }
    const hipError_t err = hipGetLastError();
    if (err != hipSuccess)
        return fail(AIMG_ERR_HIP, std::string("kernel launch failed: ") + hipGetErrorString(err));
    return AIMG_OK;
}

// Validate tensor i and add it to the normal or the tiny-buffer batch.
// The segment-run kernel over the batch's tensors: a full grid, whose
// workgroups split the tensors' segments evenly among themselves.
template <int kMode>
int launch_run(Batch& B, hipStream_t s) {
    if (B.m == 0) return AIMG_OK;
    B.args.n_tensors = B.m;
    B.args.total_items = 0;
    // Rounds go to workgroups in turn (workgroup w takes rounds w, w + grid,
    // ...), so the grid works through a window of consecutive rounds: with
    // inputs read from HBM, 9% faster on a 5120x17408 layer and 5% on a 14B
    // block than contiguous ranges of rounds per workgroup, which are 3%
    // faster when the inputs are still in the last-level cache from the
    // previous launch. The fused GEMV keeps contiguous ranges: its per-row
    // atomics would all land on the few cache lines of y that a window of
    // rounds covers (batch 4 was 6x slower strided). AIMG_RUN_STRIDED=0
    // selects contiguous ranges for the decodes too.
    const char* st = std::getenv("AIMG_RUN_STRIDED");
    B.args.strided =
        (kMode == kModeGemv || kMode == kModeGemv1) || (st != nullptr && st[0] == '0') ? 0 : 1;
    int64_t bits = 0;
    for (int d = 0; d < B.m; ++d) bits += 8 * B.args.t[d].packed_nbytes;
    // A workgroup per round (of 168-bit segments) up to a full grid: each
    // workgroup pays its start-up once, and its rounds follow one another.
    const int64_t slots = static_cast<int64_t>(cu_count()) * kBlocksPerCu;
    const int64_t want = bits / (static_cast<int64_t>(kThreads) * kMaxSegBits) + 1;
    const dim3 gdim(static_cast<uint32_t>(want < slots ? want : slots)), bdim(kThreads);
    constexpr int kVecGroup = kMode == kModeU8 ? 16 : 8;
    hipLaunchKernelGGL((run_kernel<kMode, kVecGroup>), gdim, bdim, 0, s, B.args);
    const hipError_t err = hipGetLastError();
    if (err != hipSuccess)
        return fail(AIMG_ERR_HIP, std::string("kernel launch failed: ") + hipGetErrorString(err));
    return AIMG_OK;
}

// The speculative segment-run kernel over the batch's tensors: each workgroup
// takes the chunks whose first element lies in its share of the tensors'
// elements (a grid of one workgroup per chunk up to two per CU).
template <int kMode>
int launch_spec(Batch& B, hipStream_t s) {
    if (B.m == 0) return AIMG_OK;
    B.args.n_tensors = B.m;
    int64_t elements = 0, chunks = 0;
    for (int d = 0; d < B.m; ++d) {
        elements += B.args.t[d].n_symbols;
        chunks += B.args.t[d].n_jobs;
    }
    B.args.total_items = elements;
    const int64_t slots = static_cast<int64_t>(cu_count()) * kBlocksPerCu;
    const int64_t grid = chunks < slots ? chunks : slots;
    // A full grid: workgroups b and b + grid / 2 share a CU and split its share.
    B.args.strided = grid == slots ? 1 : 0;
    constexpr int kVecGroup = kMode == kModeU8 ? 16 : 8;
    hipLaunchKernelGGL((spec_kernel<kMode, kVecGroup>), dim3(static_cast<uint32_t>(grid)), dim3(kThreads), 0,
                       s, B.args);
    const hipError_t err = hipGetLastError();
    if (err != hipSuccess)
        return fail(AIMG_ERR_HIP, std::string("kernel launch failed: ") + hipGetErrorString(err));
    return AIMG_OK;
}

// Tensors with a segment index (chunks of kRunMinChunk symbols or more, the
// vector path's alignment) go to `run`, the segment-run kernel, when `run`
// is given; tensors without one that meet the same conditions go to `spec`,
// the speculative segment-run kernel, when `spec` is given; the others decode
// chunk by chunk.
constexpr uint32_t kSpecMaxTpc = 128;

template <int kMode>
int add_tensor(const aimg_tensor& t, int i, Batch& normal, Batch& tiny, Batch* run = nullptr,
               Batch* spec = nullptr, bool spec_all = false) {
    const std::string who = "tensor " + std::to_string(i) + ": ";
    if (t.chunk_size < 1) return fail(AIMG_ERR_INVALID_ARGUMENT, who + "chunk_size must be >= 1");
    if (t.n_chunks < 0 || t.n_symbols < 0 || t.packed_nbytes < 0)
        return fail(AIMG_ERR_INVALID_ARGUMENT, who + "negative size");
    if (t.n_symbols > static_cast<int64_t>(t.n_chunks) * t.chunk_size)
        return fail(AIMG_ERR_INVALID_ARGUMENT, who + "n_symbols exceeds n_chunks * chunk_size");
    if (t.n_symbols == 0) return AIMG_OK;
    if (t.n_symbols > INT32_MAX)
        return fail(AIMG_ERR_UNSUPPORTED, who + "more than 2^31 - 1 symbols");
    const bool need_sm = needs_sm(kMode);
    const bool need_out = kMode == kModeU8 || kMode == kModeBf16;
    if (t.packed == nullptr || t.chunk_offsets == nullptr || t.chunk_nbytes == nullptr ||
        (need_out && t.out == nullptr) || t.table == nullptr ||
        (need_sm && t.sign_mantissa == nullptr))
        return fail(AIMG_ERR_INVALID_ARGUMENT, who + "null device pointer");
    if (reinterpret_cast<uintptr_t>(t.table) % 16 != 0)
        return fail(AIMG_ERR_INVALID_ARGUMENT, who + "table must be 16-byte aligned");
    const int group = kMode == kModeU8 ? 16 : 8;
    const bool vec_layout = !((need_out && reinterpret_cast<uintptr_t>(t.out) % 16 != 0) ||
                              t.chunk_size % group != 0 ||
                              (need_sm && reinterpret_cast<uintptr_t>(t.sign_mantissa) % 8 != 0));
    // An index smaller than its header, or misaligned, is not one.
    const bool has_index = t.index != nullptr && t.index_nbytes >= static_cast<int64_t>(sizeof(IndexHeader)) &&
                           reinterpret_cast<uintptr_t>(t.index) % 16 == 0;
    // Decodes use the index only in segment runs; the index build is the
    // chunk kernel's (kModeIndex) and is the one other user.
    const bool to_run = run != nullptr && has_index && t.chunk_size >= kRunMinChunk &&
                        t.packed_nbytes >= 4 && vec_layout;
    // (The speculative runs keep byte offsets within a round below 2^32,
    // and chunk sizes below 2^24 keep their stage arithmetic in 32 bits.)
    // Unless forced, only chunks of 128 threads or fewer: a chunk of a whole
    // workgroup (or half of one) decodes faster chunk by chunk, where no
    // round crosses a chunk boundary (5120x17408 bf16 weights on MI355X,
    // speculative runs against chunk by chunk: 64Ki-, 32Ki- and 16Ki-symbol
    // chunks 6%, 13% and 5% slower; 8Ki and 4Ki 3% and 11% faster).
    const bool spec_size = spec_all || threads_per_chunk(t.chunk_size) <= kSpecMaxTpc;
    const bool to_spec = !to_run && spec != nullptr && t.chunk_size >= kRunMinChunk &&
                         t.chunk_size <= (1 << 24) && spec_size &&
                         t.packed_nbytes >= 4 && t.packed_nbytes < (int64_t{1} << 32) - (int64_t{1} << 20) &&
                         vec_layout;
    const bool keep_index = has_index && (to_run || kMode == kModeIndex);
    Batch& B = to_run ? *run : to_spec ? *spec : (t.packed_nbytes < 4 ? tiny : normal);
    if (!vec_layout) B.vec = false;
    DevTensor& dt = B.args.t[B.m++];
    dt.packed = t.packed;
    dt.offsets = t.chunk_offsets;
    dt.nbytes = t.chunk_nbytes;
    dt.sm = t.sign_mantissa;
    dt.out = t.out;
    dt.table = static_cast<const uint8_t*>(t.table);
    dt.packed_nbytes = t.packed_nbytes;
    dt.packed_n32 = t.packed_nbytes > static_cast<int64_t>(UINT32_MAX)
                        ? UINT32_MAX : static_cast<uint32_t>(t.packed_nbytes);
    dt.n_symbols = t.n_symbols;
    dt.chunk_size = t.chunk_size;
    dt.n_chunks = t.n_chunks;
    dt.index = keep_index ? static_cast<uint8_t*>(t.index) : nullptr;
    dt.index_n32 = !keep_index ? 0u
                   : t.index_nbytes > static_cast<int64_t>(UINT32_MAX) ? UINT32_MAX
                   : static_cast<uint32_t>(t.index_nbytes);
    dt.tpc = static_cast<int32_t>(threads_per_chunk(t.chunk_size));
    if (dt.tpc != kThreads) B.full = false;
    // Chunks past the last output element hold nothing to write.
    dt.n_jobs = (t.n_symbols + t.chunk_size - 1) / t.chunk_size;
    dt.item_begin = B.items;
    const int64_t per_item = kThreads / dt.tpc;
    B.items += (dt.n_jobs + per_item - 1) / per_item;
    return AIMG_OK;
}

// vec_ok false selects the element-wise kernel whatever the tensors' layout.
template <int kMode>
int launch(const aimg_tensor* ts, int n, const GemvArgs& gemv, bool vec_ok, void* stream) {
    if (ts == nullptr && n > 0) return fail(AIMG_ERR_INVALID_ARGUMENT, "tensors is null");
    if (n < 0 || n > AIMG_MAX_TENSORS)
        return fail(AIMG_ERR_INVALID_ARGUMENT,
                    "n_tensors must be in 0.." + std::to_string(AIMG_MAX_TENSORS));
    Batch normal, tiny, run, spec;
    normal.args.gemv = gemv;
    tiny.args.gemv = gemv;
    run.args.gemv = gemv;
    spec.args.gemv = gemv;
    normal.vec = vec_ok;
    // Tensors with an index and chunks of at least kRunMinChunk symbols
    // decode in segment runs; such tensors without an index in speculative
    // segment runs when their chunks are small enough; the others chunk by
    // chunk. AIMG_SEGMENT_RUNS=0 ignores every index, AIMG_SPEC_RUNS=0 turns
    // the speculative runs off and AIMG_SPEC_RUNS=1 takes them for every
    // chunk size they support (tests and benchmarks use these to check and
    // time each path on the same inputs).
    const char* force = std::getenv("AIMG_SEGMENT_RUNS");
    const bool no_runs = force != nullptr && force[0] == '0';
    const char* force_spec = std::getenv("AIMG_SPEC_RUNS");
    const bool no_spec = force_spec != nullptr && force_spec[0] == '0';
    const bool spec_all = force_spec != nullptr && force_spec[0] == '1';
    const hipStream_t s = static_cast<hipStream_t>(stream);
    if constexpr (is_gemm(kMode)) {
        // The fused GEMM runs in speculative segment runs only, whatever the
        // chunk size (an index is not used).
        for (int i = 0; i < n; ++i) {
            const int rc = add_tensor<kMode>(ts[i], i, normal, tiny, nullptr, vec_ok ? &spec : nullptr, true);
            if (rc != AIMG_OK) return rc;
        }
        if (normal.m != 0 || tiny.m != 0)
            return fail(AIMG_ERR_UNSUPPORTED,
                        "fused GEMM: needs chunk_size a multiple of 8 and >= " + std::to_string(kRunMinChunk) +
                            ", at most 2^24, 8-byte aligned sign_mantissa, 4 or more packed bytes and below "
                            "4 GiB - 1 MiB");
        return launch_spec<kMode>(spec, s);
    } else {
    Batch* const to_run = vec_ok && !no_runs ? &run : nullptr;
    Batch* const to_spec = vec_ok && !no_spec ? &spec : nullptr;
    for (int i = 0; i < n; ++i) {
        const int rc = add_tensor<kMode>(ts[i], i, normal, tiny, to_run, to_spec, spec_all);
        if (rc != AIMG_OK) return rc;
    }
    int rc = launch_run<kMode>(run, s);
    if (rc != AIMG_OK) return rc;
    rc = launch_spec<kMode>(spec, s);
    if (rc != AIMG_OK) return rc;
    rc = launch_batch<kMode>(normal, s, false);
    if (rc != AIMG_OK) return rc;
    return launch_batch<kMode>(tiny, s, true);
    }
}

// Recombine of already-decoded exponents: out[i] = bf16 bits of (sm[i], e[i]).
// kVec: the three pointers are 16-byte aligned, and each thread takes 16
// elements per step (two 16-byte loads, two 16-byte stores); otherwise one
// element per step.
template <bool kVec>
__global__ __launch_bounds__(256) void recombine_kernel(const uint8_t* e, const uint8_t* sm,
                                                        uint16_t* out, int64_t n) {
    const int64_t stride = static_cast<int64_t>(gridDim.x) * blockDim.x;
    const int64_t t0 = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x;
    int64_t done = 0;
    if (kVec) {
        const int64_t nvec = n / 16;
        for (int64_t v = t0; v < nvec; v += stride) {
            const uint4 ev = reinterpret_cast<const uint4*>(e)[v];
            const uint4 sv = reinterpret_cast<const uint4*>(sm)[v];
            const uint32_t ew[4] = {ev.x, ev.y, ev.z, ev.w};
            const uint32_t sw[4] = {sv.x, sv.y, sv.z, sv.w};
            v4u32 o[2];
#pragma unroll
            for (int q = 0; q < 4; ++q) {
                const uint2 qq = bf16_quad(sw[q], ew[q]);
                o[q / 2][2 * (q % 2)] = qq.x;
                o[q / 2][2 * (q % 2) + 1] = qq.y;
            }
            v4u32* dst = reinterpret_cast<v4u32*>(out + 16 * v);
            __builtin_nontemporal_store(o[0], dst);
            __builtin_nontemporal_store(o[1], dst + 1);
        }
        done = nvec * 16;
    }
    for (int64_t i = done + t0; i < n; i += stride) out[i] = bf16_one(sm[i], e[i]);
}

}  // namespace
}  // namespace aimg

extern "C" int aimg_recombine_bf16(const uint8_t* exponent, const uint8_t* sign_mantissa,
                                   void* out, int64_t n, void* stream) {
    using aimg::fail;
    if (n < 0) return fail(AIMG_ERR_INVALID_ARGUMENT, "n must be >= 0");
    if (n == 0) return AIMG_OK;
    if (exponent == nullptr || sign_mantissa == nullptr || out == nullptr)
        return fail(AIMG_ERR_INVALID_ARGUMENT, "null pointer passed to aimg_recombine_bf16");
    const bool vec = (reinterpret_cast<uintptr_t>(exponent) | reinterpret_cast<uintptr_t>(sign_mantissa) |
                      reinterpret_cast<uintptr_t>(out)) % 16 == 0;
    const int64_t per_thread = vec ? 16 : 1;
    const int64_t want = (n / per_thread + 255) / 256;
    const int64_t cap = static_cast<int64_t>(aimg::cu_count()) * 8;
    const dim3 grid(static_cast<uint32_t>(want < 1 ? 1 : (want < cap ? want : cap))), block(256);
    const hipStream_t s = static_cast<hipStream_t>(stream);
    auto* o = static_cast<uint16_t*>(out);
    if (vec)
        hipLaunchKernelGGL((aimg::recombine_kernel<true>), grid, block, 0, s, exponent, sign_mantissa, o, n);
    else
        hipLaunchKernelGGL((aimg::recombine_kernel<false>), grid, block, 0, s, exponent, sign_mantissa, o, n);
    const hipError_t err = hipGetLastError();
    if (err != hipSuccess)
        return fail(AIMG_ERR_HIP, std::string("kernel launch failed: ") + hipGetErrorString(err));
    return AIMG_OK;
}

extern "C" int aimg_build_index(const aimg_tensor* tensors, int n_tensors, void* stream) {
    using aimg::fail;
    if (tensors == nullptr && n_tensors > 0) return fail(AIMG_ERR_INVALID_ARGUMENT, "tensors is null");
    if (n_tensors < 0 || n_tensors > AIMG_MAX_TENSORS)
        return fail(AIMG_ERR_INVALID_ARGUMENT,
                    "n_tensors must be in 0.." + std::to_string(AIMG_MAX_TENSORS));
    // Tensors that have an index; each must hold at least its header.
    // Tensors with no symbols have nothing to index.
    aimg::Batch normal, tiny;
    aimg::LaunchArgs plan{};
    int n_plan = 0;
    int64_t chunks = 0;
    for (int i = 0; i < n_tensors; ++i) {
        const aimg_tensor& t = tensors[i];
        if (t.index == nullptr) continue;
        if (t.index_nbytes < static_cast<int64_t>(sizeof(aimg::IndexHeader)))
            return fail(AIMG_ERR_INVALID_ARGUMENT, "tensor " + std::to_string(i) +
                                                       ": index_nbytes is below aimg_index_nbytes");
        if (reinterpret_cast<uintptr_t>(t.index) % 16 != 0)
            return fail(AIMG_ERR_INVALID_ARGUMENT,
                        "tensor " + std::to_string(i) + ": index must be 16-byte aligned");
        const int n0 = normal.m, t0 = tiny.m;
        const int rc = aimg::add_tensor<aimg::kModeIndex>(t, i, normal, tiny);
        if (rc != AIMG_OK) return rc;
        aimg::DevTensor* dt = normal.m > n0 ? &normal.args.t[normal.m - 1]
                              : tiny.m > t0 ? &tiny.args.t[tiny.m - 1] : nullptr;
        if (dt == nullptr) continue;
        plan.t[n_plan] = *dt;
        plan.t[n_plan].item_begin = chunks;  // the finish step's chunk numbering
        chunks += dt->n_jobs;
        ++n_plan;
    }
    const hipStream_t s = static_cast<hipStream_t>(stream);
    if (n_plan == 0) return AIMG_OK;
    plan.n_tensors = n_plan;
    hipLaunchKernelGGL(aimg::index_plan_kernel, dim3(static_cast<uint32_t>(n_plan)),
                       dim3(aimg::kThreads), 0, s, plan);
    hipError_t err = hipGetLastError();
    if (err != hipSuccess)
        return fail(AIMG_ERR_HIP, std::string("kernel launch failed: ") + hipGetErrorString(err));
    int rc = aimg::launch_batch<aimg::kModeIndex>(normal, s, false);
    if (rc != AIMG_OK) return rc;
    rc = aimg::launch_batch<aimg::kModeIndex>(tiny, s, true);
    if (rc != AIMG_OK) return rc;
    // The finish step: a wave per chunk, four per workgroup.
    const int64_t slots = static_cast<int64_t>(aimg::cu_count()) * 8;
    const int64_t groups = (chunks + aimg::kFinishWaves - 1) / aimg::kFinishWaves;
    hipLaunchKernelGGL(aimg::index_finish_kernel,
                       dim3(static_cast<uint32_t>(groups < slots ? groups : slots)),
                       dim3(aimg::kFinishThreads), 0, s, plan, chunks);
    err = hipGetLastError();
    if (err != hipSuccess)
        return fail(AIMG_ERR_HIP, std::string("kernel launch failed: ") + hipGetErrorString(err));
    // Rounds: items numbered per tensor, room for every round its index can
    // hold (the kernel skips those past the tensor's segments).
    aimg::LaunchArgs rounds = plan;
    int64_t n_round_items = 0;
    for (int k = 0; k < n_plan; ++k) {
        const aimg::DevTensor& t = plan.t[k];
        rounds.t[k].item_begin = n_round_items;
        // The segment length is only known on the device (from the table);
        // the shortest possible one (a 1-bit shortest code) bounds the rounds.
        const aimg::IndexLayout L =
            aimg::index_layout(t.packed_nbytes, t.n_chunks, aimg::segment_bits(1u));
        n_round_items += static_cast<int64_t>(L.capacity / aimg::kIndexBlock + 1);
    }
    const int64_t rslots = static_cast<int64_t>(aimg::cu_count()) * aimg::kBlocksPerCu;
    hipLaunchKernelGGL(aimg::index_rounds_kernel,
                       dim3(static_cast<uint32_t>(n_round_items < rslots ? n_round_items : rslots)),
                       dim3(aimg::kThreads), 0, s, rounds, n_round_items);
    err = hipGetLastError();
    if (err != hipSuccess)
        return fail(AIMG_ERR_HIP, std::string("kernel launch failed: ") + hipGetErrorString(err));
    return AIMG_OK;
}

extern "C" int aimg_decode_bf16(const aimg_tensor* tensors, int n_tensors, void* stream) {
    return aimg::launch<aimg::kModeBf16>(tensors, n_tensors, aimg::GemvArgs{}, true, stream);
}

extern "C" int aimg_decode_u8(const aimg_tensor* tensors, int n_tensors, void* stream) {
    return aimg::launch<aimg::kModeU8>(tensors, n_tensors, aimg::GemvArgs{}, true, stream);
}

extern "C" int aimg_decode_gemv_bf16(const aimg_tensor* t, int64_t rows, int64_t cols,
                                     const void* x, int batch, float* y, void* stream) {
    using aimg::fail;
    if (t == nullptr) return fail(AIMG_ERR_INVALID_ARGUMENT, "tensor is null");
    if (rows < 1 || cols < 1 || rows > INT32_MAX || cols > INT32_MAX ||
        rows * cols != t->n_symbols)
        return fail(AIMG_ERR_INVALID_ARGUMENT, "rows * cols must equal n_symbols (both >= 1)");
    if (batch < 1 || batch > aimg::kGemvMaxBatch)
        return fail(AIMG_ERR_INVALID_ARGUMENT,
                    "batch must be in 1.." + std::to_string(aimg::kGemvMaxBatch));
    if (x == nullptr || y == nullptr) return fail(AIMG_ERR_INVALID_ARGUMENT, "null x or y");
    const uint32_t step = aimg::kThreads * 8;  // elements between a thread's groups
    const aimg::GemvArgs g{static_cast<const uint16_t*>(x), y, static_cast<uint32_t>(rows),
                           static_cast<uint32_t>(cols), batch,
                           step / static_cast<uint32_t>(cols), step % static_cast<uint32_t>(cols)};
    // The 8-weight groups take 16-byte x loads: they must lie inside one row
    // (cols % 8 == 0) and x must be 16-byte aligned.
    const bool vec_ok = cols % 8 == 0 && reinterpret_cast<uintptr_t>(x) % 16 == 0;
    if (batch == 1) return aimg::launch<aimg::kModeGemv1>(t, 1, g, vec_ok, stream);
    return aimg::launch<aimg::kModeGemv>(t, 1, g, vec_ok, stream);
}

extern "C" int aimg_decode_gemm_bf16(const aimg_tensor* t, int64_t rows, int64_t cols,
                                     const void* x, int n_x, float* y, void* stream) {
    using aimg::fail;
    if (t == nullptr) return fail(AIMG_ERR_INVALID_ARGUMENT, "tensor is null");
    if (rows < 1 || cols < 1 || rows > INT32_MAX || cols > INT32_MAX ||
        rows * cols != t->n_symbols)
        return fail(AIMG_ERR_INVALID_ARGUMENT, "rows * cols must equal n_symbols (both >= 1)");
    if (n_x < 1 || n_x > aimg::kGemmMaxRows)
        return fail(AIMG_ERR_INVALID_ARGUMENT, "n_x must be in 1.." + std::to_string(aimg::kGemmMaxRows));
    if (x == nullptr || y == nullptr) return fail(AIMG_ERR_INVALID_ARGUMENT, "null x or y");
    if (cols % 8 != 0 || reinterpret_cast<uintptr_t>(x) % 16 != 0 ||
        static_cast<int64_t>(n_x) * cols * 2 > int64_t{0xFFFFFFFF})
        return fail(AIMG_ERR_UNSUPPORTED,
                    "fused GEMM: needs cols % 8 == 0, a 16-byte aligned x and n_x * cols * 2 below 2^32");
    const aimg::GemvArgs g{static_cast<const uint16_t*>(x), y, static_cast<uint32_t>(rows),
                           static_cast<uint32_t>(cols), n_x, 0u, 0u};
    if (cols > aimg::kGemmPieceMaxCols) return aimg::launch<aimg::kModeGemmRows>(t, 1, g, true, stream);
    return aimg::launch<aimg::kModeGemm>(t, 1, g, true, stream);
}
