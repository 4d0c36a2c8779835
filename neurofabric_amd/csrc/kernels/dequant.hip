// dequant.hip — standalone Q4_0 / Q8_0 dequantization (f32 or f16 output).
//
// Serves dequant_q4_0[_f16] and dequant_q8_0[_f16] (metal_provider.mm:510-530,
// 741-759).  HBM-bound: 18 (34) bytes in per 32 elements, 128 (64) bytes out
// for f32 (f16).  One thread produces 8 consecutive elements (a quarter of a
// block), so a wave writes 64 x 32 B (f32) / 64 x 16 B (f16) contiguous
// bytes per store instruction.
#include "../launch.hpp"
#include "common.hpp"

namespace nfk {

template <class QF, typename OutT>
__global__ __launch_bounds__(256) void dequant_kernel(const uint8_t* __restrict__ w,
                                                      OutT* __restrict__ out, uint64_t count) {
  const uint64_t t = (uint64_t)blockIdx.x * blockDim.x + threadIdx.x;
  const uint64_t e0 = t * 8;
  if (e0 >= count) return;
  float v[8];
  quarter_f32<QF>(w + (t >> 2) * QF::kBytes, (int)(t & 3), v);
  OutT* o = out + e0;
  if (e0 + 8 <= count) {
    if constexpr (sizeof(OutT) == 4) {
      float4v lo = {v[0], v[1], v[2], v[3]};
      float4v hi = {v[4], v[5], v[6], v[7]};
      reinterpret_cast<float4v*>(o)[0] = lo;
      reinterpret_cast<float4v*>(o)[1] = hi;
    } else {
      half8 h;
#pragma unroll
      for (int i = 0; i < 8; ++i) h[i] = (half_t)v[i];  // round to nearest even
      *reinterpret_cast<half8*>(o) = h;
    }
  } else {
    for (uint64_t i = 0; i < count - e0; ++i) o[i] = (OutT)v[i];
  }
}

}  // namespace nfk

namespace nfhip {

hipError_t launch_dequant(QFmt q, EType out_t, const void* w, void* out, uint64_t count,
                          hipStream_t s) {
  if (count == 0) return hipSuccess;
  const uint64_t threads = (count + 7) / 8;
  const dim3 block(256);
  const dim3 grid((unsigned)((threads + 255) / 256));
  const uint8_t* wp = static_cast<const uint8_t*>(w);
  if (q == QFmt::Q4_0) {
    if (out_t == EType::F32)
      nfk::dequant_kernel<nfk::Q4_0, float><<<grid, block, 0, s>>>(wp, (float*)out, count);
    else
      nfk::dequant_kernel<nfk::Q4_0, nfk::half_t><<<grid, block, 0, s>>>(wp, (nfk::half_t*)out, count);
  } else {
    if (out_t == EType::F32)
      nfk::dequant_kernel<nfk::Q8_0, float><<<grid, block, 0, s>>>(wp, (float*)out, count);
    else
      nfk::dequant_kernel<nfk::Q8_0, nfk::half_t><<<grid, block, 0, s>>>(wp, (nfk::half_t*)out, count);
  }
  return hipGetLastError();
}

}  // namespace nfhip
