// Host side of the row-streaming conv kernel (conv_stream.h): which shapes it
// runs, band height, ring depth and launch.
#include <stdlib.h>

#include <algorithm>

#include "conv_stream.h"

namespace dimq {
namespace {

constexpr int64_t kStreamCUs = 256;
constexpr size_t kStreamMaxLds = 150 * 1024;

// Ring rows for bands of `rows` output rows: the largest number of input rows
// one 128-pixel step reads, rounded up to a power of two.
int ring_rows(int rows, int OW, int stride, int KH) {
  const int P = rows * OW;
  int span = 1;
  for (int s = 0; s * kStepPx < P; ++s) {
    const int first = s * kStepPx, last = std::min(P, (s + 1) * kStepPx) - 1;
    span = std::max(span, (last / OW - first / OW) * stride + KH);
  }
  int nr = 1;
  while (nr < span) nr *= 2;
  return nr;
}

// Input rows one step adds at most (the staging area's rows).
int stage_rows(int rows, int OW, int stride, int KH) {
  const int P = rows * OW;
  int prev = ((std::min(P, kStepPx) - 1) / OW) * stride + KH - 1, most = 0;
  for (int s = 1; s * kStepPx < P; ++s) {
    const int hi = ((std::min(P, (s + 1) * kStepPx) - 1) / OW) * stride + KH - 1;
    most = std::max(most, hi - prev);
    prev = hi;
  }
  return std::max(most, 1);
}

// LDS: the input-row ring, then the fp32 output tile of one step.
size_t ring_bytes(const HaloArgs& p, int nr, int sr) {
  (void)sr;
  return (size_t)nr * p.IW_t * p.CP * sizeof(uint16_t) + kTileFloats * sizeof(float);
}

// Band height: about one work-group per CU, at least one row.
int band_rows(const HaloArgs& p) {
  const char* force = getenv("DIMQ_STREAM_ROWS");  // A/B runs
  if (force && atoi(force) > 0) return std::min(atoi(force), p.OH);
  const int64_t oc_blocks = (p.OC + 63) / 64;
  const int64_t per_image = std::max<int64_t>(1, (kStreamCUs + p.B * oc_blocks - 1) / (p.B * oc_blocks));
  const int64_t bands = std::min<int64_t>(per_image, p.OH);
  return (int)((p.OH + bands - 1) / bands);
}

}  // namespace

bool stream_supported(const HaloArgs& p, int stride, int bits) {
  if (!(bits == 2 || bits == 3 || bits == 4)) return false;
  if (stride != 1 && stride != 2) return false;
  const bool k3 = p.KH == 3 && p.KW == 3 && p.C == 64;
  const bool k1 = p.KH == 1 && p.KW == 1 && (p.C == 64 || p.C == 128);
  if (!k3 && !k1) return false;
  if (p.x_layout == DIMQ_NCHW && p.W % 8 != 0) return false;
  // full steps store 128 pixels x 64 channels with 16-byte (8-byte) stores
  if (p.OC % 64 != 0) return false;
  if (p.y_layout == DIMQ_NCHW && p.OW % 4 != 0) return false;
  if (p.CP != p.C + 8) return false;
  const int rows = band_rows(p);
  return ring_bytes(p, ring_rows(rows, p.OW, stride, p.KH), stage_rows(rows, p.OW, stride, p.KH)) <= kStreamMaxLds;
}

int launch_conv_stream(HaloArgs p, int stride, int bits, hipStream_t s) {
  p.TH = band_rows(p);
  p.tiles_h = (p.OH + p.TH - 1) / p.TH;
  p.NR = ring_rows(p.TH, p.OW, stride, p.KH);
  p.SR = stage_rows(p.TH, p.OW, stride, p.KH);
  p.IH_t = p.NR;
  const size_t lds = ring_bytes(p, p.NR, p.SR);
  const dim3 grid(static_cast<unsigned>(p.B * p.tiles_h), static_cast<unsigned>((p.OC + 63) / 64));
  switch (bits) {
    case 2: return launch_stream_b2(p, stride, grid, lds, s);
    case 3: return launch_stream_b3(p, stride, grid, lds, s);
    default: return launch_stream_b4(p, stride, grid, lds, s);
  }
}

}  // namespace dimq
