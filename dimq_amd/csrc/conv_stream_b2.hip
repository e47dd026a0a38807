// Instantiations of the row-streaming conv kernel for 2-bit weights.
#include "conv_stream.h"

namespace dimq {
int launch_stream_b2(const HaloArgs& p, int stride, dim3 grid, size_t lds, hipStream_t s) {
  return launch_stream_bits<2>(p, stride, grid, lds, s);
}
}  // namespace dimq
