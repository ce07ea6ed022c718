// CPU stand-in for the HIP device subset used by aimg_decode.hip, so that the
// kernel source can be compiled for the host under AddressSanitizer and run
// on small inputs: every out-of-bounds access of a global buffer or of the
// LDS block is then reported with its source line. Test infrastructure only.
//
// Model: a block runs as one std::thread per work-item; blocks run one after
// another; __shared__ data are function statics (one block at a time).
// __syncthreads is a block barrier. Wave shuffles, DPP, readlane and HIP's
// __ballot exchange values through a per-wave buffer between per-wave
// barriers, so they must be reached by all 64 lanes (the kernel calls them in
// uniform control flow only). The compiler builtin ballot returns the calling
// lane's own bit: the kernel uses it only inside divergent loops, as "does
// any lane need this?", for which the per-lane answer gives the same
// results.
#pragma once
#include <barrier>
#include <cstdint>
#include <cstdlib>
#include <cstring>
#include <thread>
#include <vector>

#define __global__
#define __device__
#define __host__
#define __forceinline__ inline
#define __launch_bounds__(...)
#define __shared__ static

struct dim3 {
    unsigned x, y, z;
    dim3(unsigned a = 1, unsigned b = 1, unsigned c = 1) : x(a), y(b), z(c) {}
};
struct EmuIdx {
    unsigned x, y, z;
};
inline thread_local EmuIdx threadIdx{0, 0, 0};
inline thread_local EmuIdx blockIdx{0, 0, 0};
inline EmuIdx gridDim{1, 1, 1};
inline EmuIdx blockDim{1, 1, 1};

typedef int hipError_t;
enum { hipSuccess = 0 };
typedef void* hipStream_t;
enum hipDeviceAttribute_t { hipDeviceAttributeMultiprocessorCount = 0 };
inline hipError_t hipGetDevice(int* d) { *d = 0; return hipSuccess; }
// 256 CUs, or AIMG_EMU_CUS of them: a small count gives each workgroup of a
// persistent grid several items and rounds.
inline hipError_t hipDeviceGetAttribute(int* v, hipDeviceAttribute_t, int) {
    const char* e = std::getenv("AIMG_EMU_CUS");
    *v = e != nullptr && std::atoi(e) > 0 ? std::atoi(e) : 256;
    return hipSuccess;
}
inline hipError_t hipGetLastError() { return hipSuccess; }
inline const char* hipGetErrorString(hipError_t) { return "cpu"; }

namespace emu {
struct Block {
    unsigned n;
    std::barrier<> bar;
    std::vector<std::barrier<>*> wave;
    std::vector<uint64_t> xbuf;
    std::vector<uint64_t> mbuf;  // MFMA operands: 4 words a lane
    std::vector<int> flags;
    explicit Block(unsigned n_) : n(n_), bar(n_), xbuf(n_), mbuf(4 * n_), flags(n_) {
        for (unsigned w = 0; w * 64 < n; ++w)
            wave.push_back(new std::barrier<>(n - 64 * w < 64 ? n - 64 * w : 64));
    }
    ~Block() {
        for (auto* b : wave) delete b;
    }
};
inline Block* g_block = nullptr;
inline unsigned lane() { return threadIdx.x & 63u; }

template <typename T>
inline T wave_xchg(T v, unsigned src) {
    Block& B = *g_block;
    const unsigned w = threadIdx.x >> 6;
    uint64_t bits = 0;
    std::memcpy(&bits, &v, sizeof(T));
    B.wave[w]->arrive_and_wait();
    B.xbuf[threadIdx.x] = bits;
    B.wave[w]->arrive_and_wait();
    const uint64_t r = B.xbuf[w * 64 + src];
    B.wave[w]->arrive_and_wait();
    T out;
    std::memcpy(&out, &r, sizeof(T));
    return out;
}
}  // namespace emu

inline void __syncthreads() { emu::g_block->bar.arrive_and_wait(); }
inline int __syncthreads_or(int p) {
    emu::Block& B = *emu::g_block;
    B.bar.arrive_and_wait();
    B.flags[threadIdx.x] = p != 0;
    B.bar.arrive_and_wait();
    int r = 0;
    for (unsigned k = 0; k < B.n; ++k) r |= B.flags[k];
    B.bar.arrive_and_wait();
    return r;
}
template <typename T>
inline T __shfl_up(T v, unsigned d, int = 64) {
    const unsigned l = emu::lane();
    const T r = emu::wave_xchg(v, l >= d ? l - d : l);
    return l >= d ? r : v;
}
template <typename T>
inline T __shfl_xor(T v, int m, int = 64) { return emu::wave_xchg(v, emu::lane() ^ (unsigned)m); }
template <typename T>
inline T __shfl(T v, int src, int = 64) { return emu::wave_xchg(v, (unsigned)src & 63u); }

// DPP move, for the controls the kernel uses: row_shr:1..15 (0x111..0x11F),
// wave_shr:1 (0x138), row_bcast:15 (0x142), row_bcast:31 (0x143).
inline int __builtin_amdgcn_update_dpp(int old, int src, int ctrl, int row_mask, int, bool bound_ctrl) {
    const int l = (int)emu::lane(), row = l >> 4;
    int from = -1;
    if (ctrl >= 0x111 && ctrl <= 0x11F) from = (l & 15) >= ctrl - 0x110 ? l - (ctrl - 0x110) : -1;
    else if (ctrl == 0x138) from = l - 1;
    else if (ctrl == 0x142) from = row >= 1 ? 16 * row - 1 : -1;
    else if (ctrl == 0x143) from = row >= 2 ? 31 : -1;
    else __builtin_trap();
    const int v = emu::wave_xchg(src, from >= 0 ? (unsigned)from : (unsigned)l);
    if (!((row_mask >> row) & 1)) return old;
    if (from < 0) return bound_ctrl ? 0 : old;
    return v;
}

// HIP's wave ballot, used by the kernel where every lane of the wave takes
// part: the real OR over the wave's lanes.
inline unsigned long long __ballot(int p) {
    uint64_t m = 0;
    for (unsigned k = 0; k < 64; ++k) m |= (uint64_t)(emu::wave_xchg(p != 0 ? 1 : 0, k) != 0) << k;
    return m;
}

// The raw builtin is used by the kernel only inside divergent code (the
// escape branch of the decode loop), where lanes that have left the loop do
// not meet at a wave barrier: each lane sees its own bit, so a lane without
// an escape skips the branch in which it would do nothing.
inline uint64_t __builtin_amdgcn_ballot_w64(bool p) { return p ? (1ull << emu::lane()) : 0ull; }
// Same signatures as the compiler builtins (int in, int out). readfirstlane
// is applied to wave-uniform values only, so the lane's own value is it.
inline int __builtin_amdgcn_readfirstlane(int v) { return v; }
inline int __builtin_amdgcn_readlane(int v, int l) { return emu::wave_xchg(v, (unsigned)l & 63u); }
inline uint32_t __builtin_amdgcn_alignbyte(uint32_t a, uint32_t b, uint32_t s) {
    return (uint32_t)((((uint64_t)a << 32) | b) >> (8 * (s & 3)));
}
// v_perm_b32: selector bytes 0..7 pick a byte of {a, b} (b is bytes 0..3),
// 8..11 replicate the top bit of byte 1, 3, 5 or 7, 12 gives 0x00, 13.. 0xFF.
inline uint32_t __builtin_amdgcn_perm(uint32_t a, uint32_t b, uint32_t sel) {
    const uint64_t x = ((uint64_t)a << 32) | b;
    uint32_t r = 0;
    for (int k = 0; k < 4; ++k) {
        const uint32_t s = (sel >> (8 * k)) & 0xFF;
        uint32_t byte;
        if (s < 8) byte = (x >> (8 * s)) & 0xFF;
        else if (s < 12) byte = ((x >> (16 * (s - 8) + 15)) & 1) ? 0xFF : 0x00;
        else if (s == 12) byte = 0;
        else byte = 0xFF;
        r |= byte << (8 * k);
    }
    return r;
}
// Raw buffer resource: loads at or past num_records bytes read as zero.
struct __amdgpu_buffer_rsrc_t {
    const uint8_t* base;
    uint32_t n;
};
inline __amdgpu_buffer_rsrc_t __builtin_amdgcn_make_buffer_rsrc(void* p, short, int n, int) {
    return {static_cast<const uint8_t*>(p), (uint32_t)n};
}
inline uint32_t emu_dword(const __amdgpu_buffer_rsrc_t& r, uint64_t off) {
    if (off + 4 > r.n) return 0;
    uint32_t v;
    std::memcpy(&v, r.base + off, 4);
    return v;
}
inline uint32_t __builtin_amdgcn_raw_buffer_load_b32(__amdgpu_buffer_rsrc_t r, uint32_t vo, uint32_t so, int) {
    return emu_dword(r, (uint64_t)vo + so);
}
inline void __builtin_amdgcn_raw_buffer_store_b32(uint32_t v, __amdgpu_buffer_rsrc_t r, uint32_t vo, uint32_t so,
                                                  int) {
    const uint64_t off = (uint64_t)vo + so;
    if (off + 4 <= r.n) std::memcpy(const_cast<uint8_t*>(r.base) + off, &v, 4);
}
typedef uint32_t emu_u32x2 __attribute__((ext_vector_type(2)));
inline emu_u32x2 __builtin_amdgcn_raw_buffer_load_b64(__amdgpu_buffer_rsrc_t r, uint32_t vo, uint32_t so, int) {
    const uint64_t off = (uint64_t)vo + so;
    emu_u32x2 v;
    v[0] = off + 8 > r.n ? 0u : emu_dword(r, off);
    v[1] = off + 8 > r.n ? 0u : emu_dword(r, off + 4);
    return v;
}
typedef uint32_t emu_u32x4 __attribute__((ext_vector_type(4)));
inline emu_u32x4 __builtin_amdgcn_raw_buffer_load_b128(__amdgpu_buffer_rsrc_t r, uint32_t vo, uint32_t so,
                                                       int) {
    const uint64_t off = (uint64_t)vo + so;
    emu_u32x4 v;
    for (int k = 0; k < 4; ++k) v[k] = emu_dword(r, off + 4 * k);
    return v;
}
// Stores: each dword past num_records is dropped.
inline void __builtin_amdgcn_raw_buffer_store_b128(emu_u32x4 v, __amdgpu_buffer_rsrc_t r, uint32_t vo,
                                                   uint32_t so, int) {
    const uint64_t off = (uint64_t)vo + so;
    for (int k = 0; k < 4; ++k)
        if (off + 4 * k + 4 <= r.n) {
            const uint32_t d = v[k];
            std::memcpy(const_cast<uint8_t*>(r.base) + off + 4 * k, &d, 4);
        }
}
#ifndef __HIP_MEMORY_SCOPE_WORKGROUP
#define __HIP_MEMORY_SCOPE_WORKGROUP 3
#endif
struct uint2 {
    uint32_t x, y;
};
struct __attribute__((aligned(16))) uint4 {
    uint32_t x, y, z, w;
};
inline uint2 make_uint2(uint32_t a, uint32_t b) { return {a, b}; }
inline uint4 make_uint4(uint32_t a, uint32_t b, uint32_t c, uint32_t d) { return {a, b, c, d}; }
inline uint32_t __float_as_uint(float f) {
    uint32_t v;
    std::memcpy(&v, &f, 4);
    return v;
}
inline float __uint_as_float(uint32_t v) {
    float f;
    std::memcpy(&f, &v, 4);
    return f;
}
inline float atomicAdd(float* p, float v) {
    uint32_t* q = reinterpret_cast<uint32_t*>(p);
    uint32_t o = __atomic_load_n(q, __ATOMIC_RELAXED);
    for (;;) {
        float f;
        std::memcpy(&f, &o, 4);
        const float g = f + v;
        uint32_t n;
        std::memcpy(&n, &g, 4);
        if (__atomic_compare_exchange_n(q, &o, n, false, __ATOMIC_RELAXED, __ATOMIC_RELAXED)) return f;
    }
}
inline int __ffs(int x) { return __builtin_ffs(x); }
inline uint32_t __umulhi(uint32_t a, uint32_t b) { return (uint32_t)(((uint64_t)a * b) >> 32); }
inline void __builtin_amdgcn_s_setprio(int) {}  // wave issue priority: no effect here
// A wave's short sleep: blocks run one after another here, so a wait for a
// later block only passes its poll count.
inline void __builtin_amdgcn_s_sleep(int) { std::this_thread::yield(); }
inline void __builtin_amdgcn_fence(int, const char*) { __atomic_thread_fence(__ATOMIC_SEQ_CST); }
#ifndef __HIP_MEMORY_SCOPE_AGENT
#define __HIP_MEMORY_SCOPE_AGENT 4
#endif
// Device globals are host globals here.
#define HIP_SYMBOL(x) (&(x))
inline hipError_t hipGetSymbolAddress(void** p, const void* sym) {
    *p = const_cast<void*>(sym);
    return hipSuccess;
}
// v_dot2c_f32_bf16: c + a.lo b.lo + a.hi b.hi in fp32 (bf16 products are exact
// in fp32).
typedef __bf16 emu_bf16x2 __attribute__((ext_vector_type(2)));
inline float __builtin_amdgcn_fdot2_f32_bf16(emu_bf16x2 a, emu_bf16x2 b, float c, bool) {
    uint16_t x[2], y[2];
    std::memcpy(x, &a, 4);
    std::memcpy(y, &b, 4);
    return c + (__uint_as_float((uint32_t)x[0] << 16) * __uint_as_float((uint32_t)y[0] << 16) +
                __uint_as_float((uint32_t)x[1] << 16) * __uint_as_float((uint32_t)y[1] << 16));
}
// v_mfma_f32_16x16x32_bf16 on a whole wave: A[i][k] is element k % 8 of
// lane 16 (k / 8) + i, B[k][j] element k % 8 of lane 16 (k / 8) + j, and
// lane 16 (i / 4) + j gets D[i][j] + C in element i % 4 (the layout the
// hardware was checked to use). Products and sums in fp32, k in order.
typedef __bf16 emu_bf16x8 __attribute__((ext_vector_type(8)));
typedef float emu_f32x4 __attribute__((ext_vector_type(4)));
inline emu_f32x4 __builtin_amdgcn_mfma_f32_16x16x32_bf16(emu_bf16x8 a, emu_bf16x8 b, emu_f32x4 c, int, int,
                                                         int) {
    emu::Block& B = *emu::g_block;
    const unsigned w = threadIdx.x >> 6, l = emu::lane();
    B.wave[w]->arrive_and_wait();
    std::memcpy(&B.mbuf[4 * threadIdx.x], &a, 16);
    std::memcpy(&B.mbuf[4 * threadIdx.x + 2], &b, 16);
    B.wave[w]->arrive_and_wait();
    auto el = [&](unsigned ln, unsigned half, unsigned e) {
        uint16_t v;
        std::memcpy(&v, reinterpret_cast<const uint8_t*>(&B.mbuf[4 * (64 * w + ln) + 2 * half]) + 2 * e, 2);
        return __uint_as_float((uint32_t)v << 16);
    };
    emu_f32x4 d;
    for (unsigned r = 0; r < 4; ++r) {
        const unsigned i = 4 * (l >> 4) + r, j = l & 15;
        float s = c[r];
        for (unsigned k = 0; k < 32; ++k) s += el(16 * (k / 8) + i, 0, k % 8) * el(16 * (k / 8) + j, 1, k % 8);
        d[r] = s;
    }
    B.wave[w]->arrive_and_wait();
    return d;
}

template <typename K, typename... A>
inline void emu_launch(K kernel, dim3 g, dim3 b, A... args) {
    gridDim = {g.x, 1, 1};
    blockDim = {b.x, 1, 1};
    for (unsigned blk = 0; blk < g.x; ++blk) {
        emu::Block B(b.x);
        emu::g_block = &B;
        std::vector<std::thread> th;
        th.reserve(b.x);
        for (unsigned t = 0; t < b.x; ++t)
            th.emplace_back([=] {
                threadIdx = {t, 0, 0};
                blockIdx = {blk, 0, 0};
                kernel(args...);
            });
        for (auto& x : th) x.join();
        emu::g_block = nullptr;
    }
}
#define hipLaunchKernelGGL(K, G, B, SH, S, ...) emu_launch(K, G, B, __VA_ARGS__)
