// for_shim.cpp -- extern "C" access to the REFERENCE's group frame-of-reference
// encoder (prototypes/for_delta_encoding/for_encoding_bench.cpp, ForCodec<G>),
// compiled in place from /root/reference by oracle/Makefile into
// oracle/_ref/libfor_ref.so.  TEST INFRASTRUCTURE ONLY: it pins the oracle's
// restatement of the FOR format (and through it the device's derived FOR
// index).  The prototype's own benchmark entry point is renamed so the file
// links as a library; nothing of its source is copied here.
#define main for_encoding_bench_main
#include "for_encoding_bench.cpp"
#undef main

#include <cstddef>
#include <cstdint>

extern "C" {

// One row's column deltas (first delta from 0) -> the prototype's FOR bytes
// for group size G in {8, 16, 32, 64}; returns the byte count (or -1 when cap
// is too small / G unsupported).
int64_t ref_for_encode(const uint32_t *deltas, int64_t n, int G, uint8_t *out, int64_t cap) {
    std::vector<uint32_t> d(deltas, deltas + n);
    std::vector<uint8_t> b;
    switch (G) {
        case 8: b = ForCodec<8>::encode(d); break;
        case 16: b = ForCodec<16>::encode(d); break;
        case 32: b = ForCodec<32>::encode(d); break;
        case 64: b = ForCodec<64>::encode(d); break;
        default: return -1;
    }
    if ((int64_t)b.size() > cap) return -1;
    for (size_t i = 0; i < b.size(); ++i) out[i] = b[i];
    return (int64_t)b.size();
}

}  // extern "C"
