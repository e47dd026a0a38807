// Instantiations of the band conv kernel (conv_band.h) for 2-, 3- and 4-bit
// weights, in a compile unit of their own.
#include "conv_halo.h"
#include "conv_band.h"

namespace dimq {
int launch_band_b2(const HaloArgs& p, int mode, hipStream_t s) { return launch_band_bits<2>(p, mode, s); }
int launch_band_b3(const HaloArgs& p, int mode, hipStream_t s) { return launch_band_bits<3>(p, mode, s); }
int launch_band_b4(const HaloArgs& p, int mode, hipStream_t s) { return launch_band_bits<4>(p, mode, s); }
}  // namespace dimq
