// Instantiations of the large-tile codebook GEMM for 2-bit weights.
#include "gemm_big.h"

namespace dimq {
int launch_big_b2(const GemmArgs& p, int xt, int tile, hipStream_t s) { return launch_big_bits<2>(p, xt, tile, s); }
}  // namespace dimq
