/*
 * afterimage_decode.h -- C ABI of the MI355X (gfx950) lossless BF16 weight decoder.
 *
 * The decoder rebuilds BF16 tensors from Afterimage's compressed-store format:
 *   - a raw sign/mantissa byte per weight: (sign << 7) | mantissa
 *     (afterimage/runtime/compressed_store.py:78-88);
 *   - the exponent byte, canonical-Huffman coded in fixed-symbol-count chunks.
 *     Each chunk is its own MSB-first byte-aligned bitstream, located by
 *     chunk_offsets / chunk_nbytes (afterimage/runtime/huffman_chunked.py:151-207).
 *     The code is described by the stored flat LUT: sym_lut[2^max_bits] and
 *     len_lut[2^max_bits] (afterimage/runtime/huffman.py:128-150).
 *
 * The reference has no C layer; its decode API is Python
 * (afterimage/runtime/gpu_decode_v2.py, afterimage/runtime/compressed_store.py).
 * Each entry point below names the Python function whose work it replaces.
 * An FFI binding (ctypes) calls these with plain pointers and sizes.
 *
 * Conventions:
 *   - Every function returns AIMG_OK (0) or a positive AIMG_ERR_* code.
 *     aimg_last_error() returns the calling thread's last message.
 *   - Pointers named "device" are HIP device pointers. Streams are hipStream_t
 *     passed as void* (NULL = the null stream). Launches are asynchronous and
 *     ordered on the given stream. Nothing here synchronises the device.
 *   - No entry point allocates device memory. bf16 and exponent-byte decodes of
 *     chunks of 65536 symbols or more may split the launch's last chunks in two
 *     halves that hand over through a static 64 KiB device array (one per GPU,
 *     held until the process ends); launches that overlap on one GPU stay exact.
 *   - Functions are re-entrant.
 */
#ifndef AFTERIMAGE_DECODE_H
#define AFTERIMAGE_DECODE_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define AIMG_OK 0
#define AIMG_ERR_INVALID_ARGUMENT 1 /* bad size, null pointer, too many tensors */
#define AIMG_ERR_BAD_TABLE 2        /* LUT is not a prefix-code table with byte symbols */
#define AIMG_ERR_HIP 3              /* a HIP runtime call failed */
#define AIMG_ERR_UNSUPPORTED 4      /* valid request that this build does not serve */

/* Most tensors one aimg_decode_* call accepts (kernel-argument descriptors). */
#define AIMG_MAX_TENSORS 32

/* Library ABI version (bumped on any signature or table-layout change). */
int aimg_abi_version(void);

/* Message for the last non-OK status returned on this thread. */
const char* aimg_last_error(void);

/* ------------------------------------------------------------------------- */
/* Decode tables.                                                            */
/* Replaces prepare_decode_tables (afterimage/runtime/gpu_decode_v2.py:71-76), */
/* which copies sym_lut / len_lut to the device as two int32 tensors. Here    */
/* the stored LUT is turned on the host into one self-contained table blob:  */
/* a 4096-entry multi-symbol window table (up to 4 codewords per 12-bit      */
/* window) plus 16-entry escape blocks for codewords of 13..16 bits. The     */
/* caller copies the blob to device memory once per codebook and may share   */
/* it across every tensor with the same codebook.                            */
/* ------------------------------------------------------------------------- */

/* Size in bytes of the table blob for a LUT of 2^max_bits entries (1..16). */
int aimg_table_nbytes(int max_bits, size_t* nbytes);

/*
 * Build the table blob into host memory `out` (out_nbytes >= aimg_table_nbytes).
 * sym_lut: int32[2^max_bits], len_lut: int8[2^max_bits], as stored by
 * build_decode_lut (afterimage/runtime/huffman.py:128-150).
 * Fails with AIMG_ERR_BAD_TABLE when a symbol is outside 0..255 (the
 * reference asserts this, gpu_decode_v2.py:73-74), a length is outside
 * 0..max_bits, or an entry is not replicated over its whole prefix span.
 */
int aimg_build_table(const int32_t* sym_lut, const int8_t* len_lut, int max_bits,
                     void* out, size_t out_nbytes);

/* ------------------------------------------------------------------------- */
/* Decode.                                                                   */
/* ------------------------------------------------------------------------- */

/* One tensor's device-resident compressed form (a ChunkedEncoded plus its
 * sign/mantissa stream, huffman_chunked.py:135-148, compressed_store.py:28-42). */
typedef struct aimg_tensor {
    const uint8_t* packed;         /* device: chunk bitstreams, as stored       */
    const int32_t* chunk_offsets;  /* device: byte offset of each chunk         */
    const int32_t* chunk_nbytes;   /* device: byte length of each chunk         */
    const uint8_t* sign_mantissa;  /* device: n_symbols bytes (bf16 only)       */
    void* out;                     /* device: uint16 bf16 bits, or uint8        */
    const void* table;             /* device: blob from aimg_build_table        */
    void* index;                   /* device: segment index, or NULL (below)    */
    int64_t index_nbytes;          /* bytes at `index`                          */
    int64_t packed_nbytes;         /* bytes readable at `packed`                */
    int64_t n_symbols;             /* elements to write (below 2^31)            */
    int32_t chunk_size;            /* symbols per chunk                         */
    int32_t n_chunks;              /* chunks described by offsets / nbytes      */
} aimg_tensor;

/*
 * Decode n_tensors tensors to BF16 in one launch: the Huffman decode of
 * decode_gpu_v2 (gpu_decode_v2.py:79-117) fused with _recombine
 * (compressed_store.py:94-114). out[i] = ((sm[i] & 0x80) << 8) | (exp[i] << 7)
 * | (sm[i] & 0x7F) for i < n_symbols, where n_symbols <= n_chunks*chunk_size.
 * Replaces the body of decompress_layer_gpu (compressed_store.py:186-240) for
 * device-resident inputs; one call covers a whole decoder block of tensors.
 * A tensor of 2^31 or more symbols fails with AIMG_ERR_UNSUPPORTED.
 */
int aimg_decode_bf16(const aimg_tensor* tensors, int n_tensors, void* stream);

/*
 * Decode n_tensors exponent streams to uint8 symbols: decode_gpu_v2
 * (gpu_decode_v2.py:79-117). sign_mantissa is ignored. Positions past a
 * chunk's coded symbols decode as if the chunk's bytes were followed by zero
 * bits, as the bounded CPU reader does (huffman_chunked.py:230-235).
 */
int aimg_decode_u8(const aimg_tensor* tensors, int n_tensors, void* stream);

/*
 * Fused decode -> GEMV: y[b][r] += sum_c W[r][c] * x[b][c] in fp32 for the
 * rows x cols row-major bf16 matrix W held compressed in *t
 * (t->n_symbols == rows * cols) and b < batch (1..4). W is never written;
 * t->out is ignored. x: bf16 [batch][cols] (device). y: float [batch][rows]
 * (device), which the caller zeroes first: the kernel adds to it with
 * atomics, so the order of the fp32 additions is not fixed. The reference
 * computes this as decompress_rows_gpu (compressed_store.py:254-303) followed
 * by a matmul in its chunked lm_head (streaming_engine.py:2271-2335).
 * cols % 8 == 0 with a 16-byte-aligned x takes the vector path; other
 * shapes are correct but add every product with its own atomic.
 */
int aimg_decode_gemv_bf16(const aimg_tensor* t, int64_t rows, int64_t cols, const void* x,
                          int batch, float* y, void* stream);

/*
 * Fused decode -> GEMM for 1..16 rows of x: y[t][r] += sum_c W[r][c] * x[t][c]
 * in fp32 for t < n_x, W as in aimg_decode_gemv_bf16 (never written; t->out
 * ignored), on the matrix cores (bf16 products, fp32 sums). x: bf16
 * [n_x][cols], 16-byte aligned (device); y: float [n_x][rows] (device),
 * zeroed by the caller and added to with atomics (the order of the fp32
 * additions is not fixed). This is the chunked lm_head's speculative-verify
 * forward (streaming_engine.py:2307-2332, called with step_k + 1 positions
 * at :2554-2556: decompress_rows_gpu per row block, then F.linear) in one
 * launch that writes no weights. Needs cols % 8 == 0, chunk_size a multiple
 * of 8 in 1024 .. 2^24 and n_x * cols * 2 < 2^32; other shapes fail with
 * AIMG_ERR_UNSUPPORTED (the caller then takes the blocked decode and GEMM).
 */
int aimg_decode_gemm_bf16(const aimg_tensor* t, int64_t rows, int64_t cols, const void* x,
                          int n_x, float* y, void* stream);

/*
 * out[i] = ((sm[i] & 0x80) << 8) | (exponent[i] << 7) | (sm[i] & 0x7F) for
 * i < n, on the GPU (all three pointers device memory; out is uint16 bf16
 * bits). Replaces recombine_exponent_and_sign_mantissa and _recombine
 * (afterimage/runtime/compressed_store.py:94-130) for device tensors: one
 * kernel instead of a chain of elementwise torch kernels. 16-byte aligned
 * pointers take the vector path; any alignment is correct.
 */
int aimg_recombine_bf16(const uint8_t* exponent, const uint8_t* sign_mantissa, void* out,
                        int64_t n, void* stream);

/* ------------------------------------------------------------------------- */
/* Segment index (optional; no counterpart in the reference, whose decoder    */
/* runs one chunk per lane and needs none).                                  */
/* The decode kernels split each chunk into segments of a fixed number of     */
/* bits, one per thread, and find where each segment's first codeword starts */
/* by decoding ahead of it and checking agreement with the thread before.    */
/* A segment index records, once per resident tensor, each segment's first   */
/* codeword boundary, its chunk and where its symbols go in a round of 512   */
/* segments (4 bytes per segment of 168 bits for bf16 exponent codes: about  */
/* 4.7% of a compressed layer). A decode given the index runs in rounds of   */
/* 512 segments across chunk boundaries with no look-ahead, agreement check, */
/* scan or compaction, and writes each segment's symbols straight to their   */
/* place. It is used for tensors whose chunks hold 1024 symbols or more and  */
/* that take the vector path (16-byte aligned output, chunk_size % 8 == 0);  */
/* other tensors decode without it. Decoding without an index (index ==      */
/* NULL) gives the same result.                                              */
/* An index describes one tensor's packed bytes, chunk offsets and lengths   */
/* and table: the decoders use it only with the table it was built with      */
/* (checked by checksum) and otherwise ignore it; with other packed bytes or */
/* offsets than it was built from the output is unspecified (memory stays    */
/* in bounds).                                                               */
/* ------------------------------------------------------------------------- */

/*
 * Bytes of the segment index for a tensor of packed_nbytes packed bytes in
 * n_chunks chunks whose chunks lie back to back in `packed` (as the
 * encoder writes them, huffman_chunked.py:204-205), for the table whose
 * host blob (from aimg_build_table) is host_table.
 */
int aimg_index_nbytes(const void* host_table, int64_t packed_nbytes, int32_t n_chunks,
                      size_t* nbytes);

/*
 * Build the segment index of each tensor into its `index` (device memory of
 * index_nbytes >= aimg_index_nbytes bytes; tensors with a NULL index are
 * skipped; index must be 16-byte aligned). Four launches on `stream`
 * (segment numbering, the raw entries, a walk that fixes each chunk's
 * counts at its real end and writes the round starts, then each round's
 * chunk numbers and output places); the decoders that follow on the stream
 * use the index. When the chunks' segments do not fit index_nbytes (chunks
 * not back to back) or a chunk does not hold its symbols, the index is
 * marked unusable and decoders ignore it. Other fields as for
 * aimg_decode_u8.
 */
int aimg_build_index(const aimg_tensor* tensors, int n_tensors, void* stream);

/* ------------------------------------------------------------------------- */
/* Host decode (CPU threads).                                                */
/* Replaces the reference's CPU path: _decode_exponent with device "cpu"     */
/* (afterimage/runtime/compressed_store.py:161-183) over decode_chunks_numba */
/* (afterimage/runtime/cpu_decode.py:67-113), and _recombine on the CPU.     */
/* Every pointer of the aimg_tensor descriptors is HOST memory here, and     */
/* `table` is the host blob of aimg_build_table. The result equals the GPU   */
/* entry points' on every input. n_threads <= 0 uses every hardware thread.  */
/* The call returns when the work is done.                                   */
/* ------------------------------------------------------------------------- */

/* BF16 rebuild, as aimg_decode_bf16 (no size limit on n_symbols). */
int aimg_cpu_decode_bf16(const aimg_tensor* tensors, int n_tensors, int n_threads);

/* Exponent bytes only, as aimg_decode_u8. */
int aimg_cpu_decode_u8(const aimg_tensor* tensors, int n_tensors, int n_threads);

/* Host recombine, as aimg_recombine_bf16 (one thread). */
int aimg_cpu_recombine_bf16(const uint8_t* exponent, const uint8_t* sign_mantissa, void* out,
                            int64_t n);

/* ------------------------------------------------------------------------- */
/* Encoder support (host).                                                   */
/* ------------------------------------------------------------------------- */

/*
 * Pack symbols[0..n) chunk by chunk into MSB-first byte-aligned bitstreams:
 * the packer of encode_chunked (huffman_chunked.py:41-78, :101-109).
 * code_of[256] / len_of[256] give each symbol's canonical code and length
 * (lengths 1..16; symbols that occur must have len_of > 0).
 * Writes chunk_nbytes[ceil(n/chunk_size)] and the packed bytes into out
 * (capacity out_cap); *total receives the packed byte count (no slack tail).
 */
int aimg_pack_chunked(const uint8_t* symbols, int64_t n, const uint32_t* code_of,
                      const uint8_t* len_of, int32_t chunk_size, uint8_t* out,
                      int64_t out_cap, int32_t* chunk_nbytes, int64_t* total);

#ifdef __cplusplus
}
#endif

#endif /* AFTERIMAGE_DECODE_H */
