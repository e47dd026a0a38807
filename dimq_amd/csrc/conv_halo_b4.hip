// Instantiations of the LDS-halo and band conv kernels for 4-bit weights.
#include "conv_halo.h"

namespace dimq {
int launch_halo_b4(const HaloArgs& p, int CC16, int stride, int mode, hipStream_t s) {
  return launch_halo_cc<4>(p, CC16, stride, mode, s);
}
int launch_band_b4(const HaloArgs& p, int mode, hipStream_t s) { return launch_band_bits<4>(p, mode, s); }
}  // namespace dimq
