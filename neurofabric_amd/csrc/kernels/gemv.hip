// gemv.hip — decode-shaped fused dequant + matmul (small M).
//
// C[m, n] = sum_k A[m, k] * deq(W)[n, k] with fp32 accumulation; the f16
// path rounds each dequantized weight to fp16 first and rounds C to fp16
// (metal_provider.mm:1396-1468).  HBM-bound: every weight byte is read once.
//
// Work split: one wavefront per output row n; its 64 lanes stride over the
// row's 32-element blocks; a CTA of 4 waves covers 4 rows and MT activation
// rows (grid.y tiles M).  Partial sums are combined with a wave reduction.
#include "../launch.hpp"
#include "common.hpp"

namespace nfk {

template <typename AT>
__device__ __forceinline__ float dot32(const AT* __restrict__ x, const float w[32]);

template <>
__device__ __forceinline__ float dot32<float>(const float* __restrict__ x, const float w[32]) {
  const float4v* xv = reinterpret_cast<const float4v*>(x);
  float s = 0.f;
#pragma unroll
  for (int j = 0; j < 8; ++j) {
    const float4v t = xv[j];
    s = __builtin_fmaf(w[4 * j + 0], t[0], s);
    s = __builtin_fmaf(w[4 * j + 1], t[1], s);
    s = __builtin_fmaf(w[4 * j + 2], t[2], s);
    s = __builtin_fmaf(w[4 * j + 3], t[3], s);
  }
  return s;
}

template <>
__device__ __forceinline__ float dot32<half_t>(const half_t* __restrict__ x, const float w[32]) {
  const half8* xv = reinterpret_cast<const half8*>(x);
  float s = 0.f;
#pragma unroll
  for (int j = 0; j < 4; ++j) {
    const half8 t = xv[j];
#pragma unroll
    for (int i = 0; i < 8; ++i) s = __builtin_fmaf(w[8 * j + i], (float)t[i], s);
  }
  return s;
}

template <class QF, typename AT, int MT>
__global__ __launch_bounds__(256) void gemv_kernel(const AT* __restrict__ A,
                                                   const uint8_t* __restrict__ W,
                                                   AT* __restrict__ C, int M, int N, int K) {
  constexpr bool kHalfW = sizeof(AT) == 2;
  const int lane = threadIdx.x & 63;
  const int n = blockIdx.x * 4 + (threadIdx.x >> 6);
  if (n >= N) return;  // whole wave leaves; no CTA barriers below
  const int m0 = blockIdx.y * MT;
  const int nb = K >> 5;
  const uint8_t* wrow = W + (size_t)n * nb * QF::kBytes;
  float acc[MT];
#pragma unroll
  for (int m = 0; m < MT; ++m) acc[m] = 0.f;

  for (int b = lane; b < nb; b += 64) {
    float w[32];
#pragma unroll
    for (int q = 0; q < 4; ++q) quarter_f32<QF>(wrow + (size_t)b * QF::kBytes, q, &w[8 * q]);
    if constexpr (kHalfW) {
#pragma unroll
      for (int i = 0; i < 32; ++i) w[i] = (float)(half_t)w[i];
    }
#pragma unroll
    for (int m = 0; m < MT; ++m) {
      if (m0 + m < M) acc[m] += dot32<AT>(A + (size_t)(m0 + m) * K + (size_t)b * 32, w);
    }
  }
#pragma unroll
  for (int m = 0; m < MT; ++m) {
    const float v = wave_sum(acc[m]);
    if (lane == 0 && m0 + m < M) C[(size_t)(m0 + m) * N + n] = (AT)v;
  }
}

template <class QF, typename AT>
hipError_t gemv_dispatch(const void* A, const void* W, void* C, uint32_t M, uint32_t N,
                         uint32_t K, hipStream_t s) {
  const dim3 block(256);
  const int mt = M == 1 ? 1 : (M == 2 ? 2 : (M <= 4 ? 4 : 8));
  const dim3 grid((N + 3) / 4, (M + mt - 1) / mt);
  const AT* a = static_cast<const AT*>(A);
  const uint8_t* w = static_cast<const uint8_t*>(W);
  AT* c = static_cast<AT*>(C);
  switch (mt) {
    case 1: gemv_kernel<QF, AT, 1><<<grid, block, 0, s>>>(a, w, c, M, N, K); break;
    case 2: gemv_kernel<QF, AT, 2><<<grid, block, 0, s>>>(a, w, c, M, N, K); break;
    case 4: gemv_kernel<QF, AT, 4><<<grid, block, 0, s>>>(a, w, c, M, N, K); break;
    default: gemv_kernel<QF, AT, 8><<<grid, block, 0, s>>>(a, w, c, M, N, K); break;
  }
  return hipGetLastError();
}

}  // namespace nfk

namespace nfhip {

hipError_t launch_gemv(QFmt q, EType t, const void* A, const void* W, void* C, uint32_t M,
                       uint32_t N, uint32_t K, hipStream_t s) {
  if (q == QFmt::Q4_0)
    return t == EType::F32 ? nfk::gemv_dispatch<nfk::Q4_0, float>(A, W, C, M, N, K, s)
                           : nfk::gemv_dispatch<nfk::Q4_0, nfk::half_t>(A, W, C, M, N, K, s);
  return t == EType::F32 ? nfk::gemv_dispatch<nfk::Q8_0, float>(A, W, C, M, N, K, s)
                         : nfk::gemv_dispatch<nfk::Q8_0, nfk::half_t>(A, W, C, M, N, K, s);
}

}  // namespace nfhip
