// Instantiations of the codebook GEMM for 3-bit indices.
#include "gemm_kernel.h"

namespace dimq {

template <int BITS, int XT, bool A4>
int launch_gemm_tile(const GemmArgs& p, int tile, hipStream_t s) {
  const unsigned gz = static_cast<unsigned>(p.groups > 0 ? p.groups : 1);
  const int64_t gy16 = (p.M + 15) / 16;
  const int64_t gy64 = (p.M + 63) / 64;
  const int64_t gy128 = (p.M + 127) / 128;
  auto g1 = [&](int64_t mt, int64_t bn) { return dim3(static_cast<unsigned>(mt * ((p.N + bn - 1) / bn)), 1, gz); };
  if constexpr (BITS == 8) {
    if (tile == kTile128x64) hipLaunchKernelGGL((gemm_cb8_kernel<128, 16, XT>), g1(gy128, 64), dim3(256), 0, s, p);
    else if (tile == kTile64x32) hipLaunchKernelGGL((gemm_cb8_kernel<64, 16, XT>), g1(gy64, 64), dim3(256), 0, s, p);
    else hipLaunchKernelGGL((gemm_cb8_kernel<16, 16, XT>), g1(gy16, 64), dim3(256), 0, s, p);
  } else if constexpr (A4) {
    if (tile == kTileFast64x32)
      hipLaunchKernelGGL((gemm_fast_kernel<BITS, 64, 32, XT, true>), g1(gy64, 128), dim3(256), 0, s, p);
    else
      hipLaunchKernelGGL((gemm_cb_kernel<BITS, 64, 32, XT, true>), g1(gy64, 128),
                         dim3(256), 0, s, p);
  } else {
    if (tile == kTileFast128x64)
      hipLaunchKernelGGL((gemm_fast_kernel<BITS, 128, 64, XT, false>), g1(gy128, 256), dim3(256), 0, s, p);
    else if (tile == kTileFast64x32)
      hipLaunchKernelGGL((gemm_fast_kernel<BITS, 64, 32, XT, false>), g1(gy64, 128), dim3(256), 0, s, p);
    else if (tile == kTileFast128x32)
      hipLaunchKernelGGL((gemm_fast_kernel<BITS, 128, 32, XT, false>), g1(gy128, 128), dim3(256), 0, s, p);
    else if (tile == kTileFast64x64)
      hipLaunchKernelGGL((gemm_fast_kernel<BITS, 64, 64, XT, false>), g1(gy64, 256), dim3(256), 0, s, p);
    else if (tile == kTileGemv)
      hipLaunchKernelGGL((gemv_cb_kernel<BITS, XT, 16>), dim3(static_cast<unsigned>((p.N + 15) / 16)), dim3(1024), 0,
                         s, p);
    else if (tile == kTile128x64)
      hipLaunchKernelGGL((gemm_cb_kernel<BITS, 128, 64, XT, false>), g1(gy128, 256),
                         dim3(256), 0, s, p);
    else if (tile == kTile64x32)
      hipLaunchKernelGGL((gemm_cb_kernel<BITS, 64, 32, XT, false>), g1(gy64, 128),
                         dim3(256), 0, s, p);
    else
      hipLaunchKernelGGL((gemm_cb_kernel<BITS, 16, 16, XT, false>), g1(gy16, 64),
                         dim3(256), 0, s, p);
  }
  return check_launch("linear_codebook");
}

template int launch_gemm_tile<3, DIMQ_F32, false>(const GemmArgs&, int, hipStream_t);
template int launch_gemm_tile<3, DIMQ_F16, false>(const GemmArgs&, int, hipStream_t);
template int launch_gemm_tile<3, DIMQ_BF16, false>(const GemmArgs&, int, hipStream_t);
}  // namespace dimq
