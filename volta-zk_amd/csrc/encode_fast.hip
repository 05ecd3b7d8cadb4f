// encode_fast.hip -- specialised Ligero encode kernels (placeholder: the
// generic transform in ntt.hip handles every shape until this path lands).
#include "kernels.hpp"

namespace vmx {

int encode_i16_fast(Context*, const int16_t*, size_t, size_t, size_t, uint64_t*, const uint64_t*) { return 1; }

}  // namespace vmx
