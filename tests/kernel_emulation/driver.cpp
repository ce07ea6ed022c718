// Runs the CPU build of the decode kernel on one case directory written by
// tests/test_kernel_emulation.py: decode <dir> <u8|bf16|gemv> [index mode].
// Every device buffer is a heap block of exactly its size, so
// AddressSanitizer reports any access past it.
//
// Index modes: "index" builds the segment index (aimg_build_index, exact
// size) and decodes with it, after checking that the build marked it
// usable; "index-small" gives the build room for the chunk bases only (the
// index must come out marked unusable, and decoding ignores it);
// "index-foreign" changes the table checksum the index records after the
// build (decoding must ignore it). AIMG_EMU_COPIES=n decodes the tensor n
// times in one launch (n descriptors sharing its inputs and index, each with
// an output of its own), so that workgroups go from tensor to tensor.
#include <cstdio>
#include <cstdlib>
#include <cstring>
#include <string>
#include <vector>
#include "afterimage_decode.h"

static std::vector<uint8_t> readf(const std::string& p) {
    FILE* f = fopen(p.c_str(), "rb");
    if (!f) { fprintf(stderr, "missing %s\n", p.c_str()); exit(2); }
    std::vector<uint8_t> v;
    uint8_t buf[65536];
    size_t n;
    while ((n = fread(buf, 1, sizeof buf, f)) > 0) v.insert(v.end(), buf, buf + n);
    fclose(f);
    return v;
}
template <typename T> static T* exact(const std::vector<uint8_t>& v, size_t align = 16) {
    void* p = nullptr;
    if (posix_memalign(&p, align, v.size() ? v.size() : 1)) exit(3);
    if (!v.empty()) memcpy(p, v.data(), v.size());
    return static_cast<T*>(p);
}
int main(int argc, char** argv) {
    const std::string d = argv[1];
    const bool bf16 = std::string(argv[2]) == "bf16";
    long long meta[4];
    FILE* m = fopen((d + "/meta.txt").c_str(), "r");
    if (fscanf(m, "%lld %lld %lld %lld", &meta[0], &meta[1], &meta[2], &meta[3]) != 4) return 2;
    fclose(m);
    const int max_bits = (int)meta[0], chunk_size = (int)meta[1];
    const long long n_symbols = meta[2], n_chunks = meta[3];
    auto packed = readf(d + "/packed.bin"), offs = readf(d + "/offsets.bin"), nbs = readf(d + "/nbytes.bin");
    auto slut = readf(d + "/sym_lut.bin"), llut = readf(d + "/len_lut.bin"), expect = readf(d + "/expect.bin");
    size_t tn = 0;
    if (aimg_table_nbytes(max_bits, &tn)) return 4;
    void* table = nullptr;
    if (posix_memalign(&table, 256, tn)) return 3;
    if (aimg_build_table((const int32_t*)slut.data(), (const int8_t*)llut.data(), max_bits, table, tn)) {
        fprintf(stderr, "build_table: %s\n", aimg_last_error());
        return 5;
    }
    aimg_tensor t{};
    t.packed = exact<uint8_t>(packed);
    t.chunk_offsets = exact<int32_t>(offs);
    t.chunk_nbytes = exact<int32_t>(nbs);
    t.table = table;
    t.packed_nbytes = (int64_t)packed.size();
    t.n_symbols = n_symbols;
    t.chunk_size = chunk_size;
    t.n_chunks = (int32_t)n_chunks;
    const std::string ix_mode = argc > 3 ? argv[3] : "";
    if (!ix_mode.empty()) {
        size_t ixn = 0;
        if (aimg_index_nbytes(table, t.packed_nbytes, t.n_chunks, &ixn)) {
            fprintf(stderr, "index_nbytes: %s\n", aimg_last_error());
            return 8;
        }
        // index-small: the header and chunk bases, and room for one entry.
        if (ix_mode == "index-small") ixn = ((64 + 4 * (n_chunks + 1) + 15) & ~15ull) + 2;
        std::vector<uint8_t> ixv(ixn, 0x5A);
        t.index = exact<uint8_t>(ixv);
        t.index_nbytes = (int64_t)ixn;
        if (aimg_build_index(&t, 1, nullptr)) {
            fprintf(stderr, "build_index: %s\n", aimg_last_error());
            return 9;
        }
        uint32_t hdr[7];
        memcpy(hdr, t.index, sizeof hdr);
        const bool ok = hdr[4] == 1;
        if (ok != (ix_mode != "index-small") && n_symbols > 0) {
            fprintf(stderr, "index ok flag %u in mode %s\n", hdr[4], ix_mode.c_str());
            return 10;
        }
        if (ix_mode == "index-foreign") {
            hdr[3] ^= 1u;
            memcpy(t.index, hdr, sizeof hdr);
        }
    }
    const bool gemm = std::string(argv[2]) == "gemm";
    if (std::string(argv[2]) == "gemv" || gemm) {
        // y += W x for the rows x cols bf16 weight W (gemm: on the matrix
        // cores, up to 16 x vectors), checked against expect_y.bin within
        // rel 1e-2 / abs 1e-3 (the GPU tests' bar).
        long long rows = 0, cols = 0, batch = 0;
        FILE* g = fopen((d + "/gemv.txt").c_str(), "r");
        if (!g || fscanf(g, "%lld %lld %lld", &rows, &cols, &batch) != 3) return 2;
        fclose(g);
        auto sm = readf(d + "/sm.bin"), xv = readf(d + "/x.bin"), ey = readf(d + "/expect_y.bin");
        t.sign_mantissa = exact<uint8_t>(sm);
        std::vector<uint8_t> yv(4 * batch * rows);
        float* y = exact<float>(yv);
        const void* x = exact<uint8_t>(xv);
        const int rc = gemm ? aimg_decode_gemm_bf16(&t, rows, cols, x, (int)batch, y, nullptr)
                            : aimg_decode_gemv_bf16(&t, rows, cols, x, (int)batch, y, nullptr);
        if (rc) { fprintf(stderr, "%s rc=%d: %s\n", argv[2], rc, aimg_last_error()); return 6; }
        const float* want = reinterpret_cast<const float*>(ey.data());
        size_t bad = 0;
        for (long long k = 0; k < batch * rows; ++k) {
            const double diff = y[k] > want[k] ? y[k] - want[k] : want[k] - y[k];
            const double aw = want[k] < 0 ? -want[k] : want[k];
            bad += diff > 1e-3 + 1e-2 * aw;
        }
        printf("%s %s: %s (%zu of %lld outside tolerance)\n", d.c_str(), argv[2], bad ? "MISMATCH" : "ok",
               bad, batch * rows);
        return bad ? 1 : 0;
    }
    const char* ce = getenv("AIMG_EMU_COPIES");
    const int copies = ce != nullptr && atoi(ce) > 1 ? atoi(ce) : 1;
    std::vector<uint8_t> outv(n_symbols * (bf16 ? 2 : 1));
    if (bf16) {
        auto sm = readf(d + "/sm.bin");
        t.sign_mantissa = exact<uint8_t>(sm);
    }
    std::vector<aimg_tensor> ts(copies, t);
    std::vector<void*> outs(copies);
    for (int c = 0; c < copies; ++c) {
        outs[c] = exact<uint8_t>(outv);
        memset(outs[c], 0xAB, outv.size());
        ts[c].out = outs[c];
    }
    const int rc = bf16 ? aimg_decode_bf16(ts.data(), copies, nullptr)
                        : aimg_decode_u8(ts.data(), copies, nullptr);
    if (rc) { fprintf(stderr, "decode rc=%d: %s\n", rc, aimg_last_error()); return 6; }
    if (expect.size() != outv.size()) { fprintf(stderr, "size mismatch\n"); return 7; }
    size_t bad = 0;
    for (int c = 0; c < copies; ++c)
        for (size_t k = 0; k < outv.size(); ++k) bad += ((const uint8_t*)outs[c])[k] != expect[k];
    printf("%s %s %s: %s (%zu bad bytes of %zu)\n", d.c_str(), argv[2], ix_mode.c_str(),
           bad ? "MISMATCH" : "ok", bad, outv.size() * copies);
    return bad ? 1 : 0;
}
