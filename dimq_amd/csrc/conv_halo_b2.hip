// Instantiations of the LDS-halo conv kernels for 2-bit weights.
#include "conv_halo.h"

namespace dimq {
int launch_halo_b2(const HaloArgs& p, int CC16, int stride, int mode, hipStream_t s) {
  return launch_halo_cc<2>(p, CC16, stride, mode, s);
}
}  // namespace dimq
