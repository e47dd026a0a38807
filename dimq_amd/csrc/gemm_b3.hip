// Instantiations of the codebook GEMM for 3-bit indices.
#include "gemm_kernel.h"

namespace dimq {

template <int BITS, int XT, bool A4>
int launch_gemm_tile(const GemmArgs& p, int tile, hipStream_t s) {
  const unsigned gz = static_cast<unsigned>(p.groups > 0 ? p.groups : 1);
  const unsigned gy16 = static_cast<unsigned>((p.M + 15) / 16);
  const unsigned gy64 = static_cast<unsigned>((p.M + 63) / 64);
  const unsigned gy128 = static_cast<unsigned>((p.M + 127) / 128);
  if constexpr (BITS == 8) {
    const unsigned gx = static_cast<unsigned>((p.N + 63) / 64);
    if (tile == kTile128x64) hipLaunchKernelGGL((gemm_cb8_kernel<128, 16, XT>), dim3(gx, gy128, gz), dim3(256), 0, s, p);
    else if (tile == kTile64x32) hipLaunchKernelGGL((gemm_cb8_kernel<64, 16, XT>), dim3(gx, gy64, gz), dim3(256), 0, s, p);
    else hipLaunchKernelGGL((gemm_cb8_kernel<16, 16, XT>), dim3(gx, gy16, gz), dim3(256), 0, s, p);
  } else if constexpr (A4) {
    hipLaunchKernelGGL((gemm_cb_kernel<BITS, 64, 32, XT, true>), dim3((unsigned)((p.N + 127) / 128), gy64, gz),
                       dim3(256), 0, s, p);
  } else {
    if (tile == kTile128x64)
      hipLaunchKernelGGL((gemm_cb_kernel<BITS, 128, 64, XT, false>), dim3((unsigned)((p.N + 255) / 256), gy128, gz),
                         dim3(256), 0, s, p);
    else if (tile == kTile64x32)
      hipLaunchKernelGGL((gemm_cb_kernel<BITS, 64, 32, XT, false>), dim3((unsigned)((p.N + 127) / 128), gy64, gz),
                         dim3(256), 0, s, p);
    else
      hipLaunchKernelGGL((gemm_cb_kernel<BITS, 16, 16, XT, false>), dim3((unsigned)((p.N + 63) / 64), gy16, gz),
                         dim3(256), 0, s, p);
  }
  return check_launch("linear_codebook");
}

template int launch_gemm_tile<3, DIMQ_F32, false>(const GemmArgs&, int, hipStream_t);
template int launch_gemm_tile<3, DIMQ_F16, false>(const GemmArgs&, int, hipStream_t);
template int launch_gemm_tile<3, DIMQ_BF16, false>(const GemmArgs&, int, hipStream_t);
}  // namespace dimq
