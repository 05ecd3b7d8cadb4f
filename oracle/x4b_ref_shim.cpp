// x4b_ref_shim.cpp -- C entry points over the reference's own host-side X4b
// arithmetic (cuda/volta_x4b.cuh, compiled unchanged from /root/reference by
// oracle/Makefile's `ref` target into oracle/_ref/libx4b_ref.so).
//
// TEST INFRASTRUCTURE ONLY: it lets tests/ and tests/golden/ check the oracle's
// X4 restatement against the reference implementation itself.  Nothing here
// is product code and the product never loads it.
#include <cstddef>
#include <cstdint>

#include "volta_x4b.cuh"

using volta_x4b::Fp2;

extern "C" {

// root_of_unity(bits) (volta_x4b.cuh:177-181); out = (c0, c1).
void ref_x4_root_of_unity(uint32_t bits, uint64_t* out) {
    const Fp2 r = volta_x4b::root_of_unity(bits);
    out[0] = r.c0;
    out[1] = r.c1;
}

// fp2_mul / fp2_inv (volta_x4b.cuh:149-175) on (c0, c1) pairs.
void ref_fp2_mul(const uint64_t* a, const uint64_t* b, uint64_t* out) {
    const Fp2 r = volta_x4b::fp2_mul(Fp2{a[0], a[1]}, Fp2{b[0], b[1]});
    out[0] = r.c0;
    out[1] = r.c1;
}

void ref_fp2_inv(const uint64_t* a, uint64_t* out) {
    const Fp2 r = volta_x4b::fp2_inv(Fp2{a[0], a[1]});
    out[0] = r.c0;
    out[1] = r.c1;
}

// direct_fold_reference (volta_x4b.cuh:203-218): input of len Fp2, output of
// len/2; returns 0 on success, -1 when the reference rejects the geometry.
int ref_x4_direct_fold(const uint64_t* input, size_t len, uint64_t c0, uint64_t c1, uint64_t* output) {
    return volta_x4b::direct_fold_reference(reinterpret_cast<const Fp2*>(input), len, Fp2{c0, c1},
                                            reinterpret_cast<Fp2*>(output))
               ? 0
               : -1;
}

}  // extern "C"
