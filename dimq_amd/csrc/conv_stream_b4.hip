// Instantiations of the row-streaming conv kernel for 4-bit weights.
#include "conv_stream.h"

namespace dimq {
int launch_stream_b4(const HaloArgs& p, int stride, dim3 grid, size_t lds, hipStream_t s) {
  return launch_stream_bits<4>(p, stride, grid, lds, s);
}
}  // namespace dimq
