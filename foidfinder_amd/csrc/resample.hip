// One pass of Pillow's separable 8-bit resampling (libImaging/Resample.c) on uint8 RGB images, for the Haruka
// model card's letterbox on the GPU (the reference's Metal version: foidfinder/backends/mlx/kernels.py:75-186).
//
// The caller computes the fixed-point taps on the host (22 fractional bits, per output index: first input index and
// tap count). One thread per output byte of a padded canvas: bytes inside the region are sum(code * tap) + 2^21,
// shifted right by 22 and clipped to 0..255, exactly as Pillow; bytes outside are white. Every tap's source index is
// checked against the source image, so no table can make the kernel read outside it.
#include "common.h"

namespace ff {

template <int AXIS>
__global__ __launch_bounds__(256) void resample_kernel(const uint8_t* __restrict__ src, int src_h, int src_w,
                                                       const int32_t* __restrict__ kk,
                                                       const int32_t* __restrict__ bounds, int ksize, int row0,
                                                       uint8_t* __restrict__ out, int out_w, int64_t total, int top,
                                                       int left, int h, int w) {
  const int64_t i = static_cast<int64_t>(blockIdx.x) * 256 + threadIdx.x;
  if (i >= total) return;
  const int c = static_cast<int>(i % 3);
  const int64_t p = i / 3;
  const int x = static_cast<int>(p % out_w), y = static_cast<int>(p / out_w);
  const int yy = y - top, xx = x - left;
  uint8_t v = 255;
  if (yy >= 0 && yy < h && xx >= 0 && xx < w) {
    const int o = AXIS == 0 ? xx : yy;  // output index along the resampled axis
    const int first = bounds[2 * o], taps = min(bounds[2 * o + 1], ksize);
    const int32_t* k = kk + static_cast<int64_t>(o) * ksize;
    int ss = 1 << 21;
    for (int t = 0; t < taps; ++t) {
      const int sy = AXIS == 0 ? row0 + yy : row0 + first + t;
      const int sx = AXIS == 0 ? first + t : xx;
      if (sy >= 0 && sy < src_h && sx >= 0 && sx < src_w)
        ss += static_cast<int>(src[(static_cast<int64_t>(sy) * src_w + sx) * 3 + c]) * k[t];
    }
    ss >>= 22;  // arithmetic shift, as Pillow's signed accumulator
    v = static_cast<uint8_t>(ss < 0 ? 0 : (ss > 255 ? 255 : ss));
  }
  out[i] = v;
}

}  // namespace ff

using namespace ff;

extern "C" int ff_resample_u8(const uint8_t* src, int64_t src_h, int64_t src_w, int axis, const int32_t* kk,
                              const int32_t* bounds, int64_t ksize, int64_t row0, uint8_t* out, int64_t out_h,
                              int64_t out_w, int64_t top, int64_t left, int64_t h, int64_t w, void* stream) {
  clear_error();
  if (axis != 0 && axis != 1) return fail(FF_EINVAL, "resample_u8: axis must be 0 (width) or 1 (height)");
  if (src_h <= 0 || src_w <= 0 || out_h <= 0 || out_w <= 0 || h <= 0 || w <= 0 || ksize <= 0)
    return fail(FF_EINVAL, "resample_u8: sizes must be positive");
  if (src_h > 65535 || src_w > 65535 || out_h > 65535 || out_w > 65535 || ksize > 65535)
    return fail(FF_EINVAL, "resample_u8: sizes above 65535 are not supported");
  if (top < 0 || left < 0 || top + h > out_h || left + w > out_w)
    return fail(FF_EINVAL, "resample_u8: region must lie inside the output");
  if (row0 < 0 || (axis == 0 && row0 + h > src_h) || (axis == 1 && w > src_w))
    return fail(FF_EINVAL, "resample_u8: region reads outside the source");
  if (!src || !kk || !bounds || !out) return fail(FF_EINVAL, "resample_u8: null pointer");
  const int64_t total = out_h * out_w * 3;
  const dim3 grid(static_cast<unsigned>((total + 255) / 256));
  const hipStream_t st = as_stream(stream);
  if (axis == 0)
    resample_kernel<0><<<grid, 256, 0, st>>>(src, static_cast<int>(src_h), static_cast<int>(src_w), kk, bounds,
                                             static_cast<int>(ksize), static_cast<int>(row0), out,
                                             static_cast<int>(out_w), total, static_cast<int>(top),
                                             static_cast<int>(left), static_cast<int>(h), static_cast<int>(w));
  else
    resample_kernel<1><<<grid, 256, 0, st>>>(src, static_cast<int>(src_h), static_cast<int>(src_w), kk, bounds,
                                             static_cast<int>(ksize), static_cast<int>(row0), out,
                                             static_cast<int>(out_w), total, static_cast<int>(top),
                                             static_cast<int>(left), static_cast<int>(h), static_cast<int>(w));
  return check_launch("resample_u8");
}
