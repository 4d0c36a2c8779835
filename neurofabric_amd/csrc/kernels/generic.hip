// generic.hip — fallback kernels that are correct for any shape.
//
//  * generic fused dequant+linear for K % 32 != 0: the reference indexes
//    weight element (n, k) by its flat position n*K + k, so rows may straddle
//    blocks (metal_provider.mm:1413-1420).  One thread per output element.
//  * dense linear C = A * B^T with B stored [N, K]
//    (metal_provider.mm:150-164, 899-935, 1152-1178): 16x16 LDS tiles,
//    any mix of f32/f16 operands, fp32 accumulation.
#include "../launch.hpp"
#include "common.hpp"

namespace nfk {

template <class QF, typename AT>
__global__ __launch_bounds__(256) void generic_fused_kernel(const AT* __restrict__ A,
                                                            const uint8_t* __restrict__ W,
                                                            AT* __restrict__ C, int M, int N,
                                                            int K) {
  constexpr bool kHalfW = sizeof(AT) == 2;
  const int n = blockIdx.x * blockDim.x + threadIdx.x;
  const int m = blockIdx.y;
  if (n >= N || m >= M) return;
  float acc = 0.f;
  for (int k = 0; k < K; ++k) {
    const uint64_t e = (uint64_t)n * K + k;
    const uint8_t* blk = W + (e >> 5) * QF::kBytes;
    float w = h2f_bits(*reinterpret_cast<const uint16_t*>(blk)) * (float)code_of<QF>(blk, (int)(e & 31));
    if constexpr (kHalfW) w = (float)(half_t)w;
    acc = __builtin_fmaf((float)A[(size_t)m * K + k], w, acc);
  }
  C[(size_t)m * N + n] = (AT)acc;
}

template <typename AT, typename BT, typename CT>
__global__ __launch_bounds__(256) void dense_kernel(const AT* __restrict__ A,
                                                    const BT* __restrict__ B,
                                                    CT* __restrict__ C, int M, int N, int K) {
  __shared__ float As[16][17];
  __shared__ float Bs[16][17];
  const int tx = threadIdx.x & 15, ty = threadIdx.x >> 4;
  const int row = blockIdx.y * 16 + ty;
  const int col = blockIdx.x * 16 + tx;
  const int bn = blockIdx.x * 16 + ty;  // B row loaded by this thread
  float acc = 0.f;
  for (int t = 0; t < K; t += 16) {
    As[ty][tx] = (row < M && t + tx < K) ? (float)A[(size_t)row * K + t + tx] : 0.f;
    Bs[ty][tx] = (bn < N && t + tx < K) ? (float)B[(size_t)bn * K + t + tx] : 0.f;
    __syncthreads();
#pragma unroll
    for (int k = 0; k < 16; ++k) acc = __builtin_fmaf(As[ty][k], Bs[tx][k], acc);
    __syncthreads();
  }
  if (row < M && col < N) C[(size_t)row * N + col] = (CT)acc;
}

template <typename AT, typename BT>
hipError_t dense_c(nfhip::EType c, const void* A, const void* B, void* C, uint32_t M, uint32_t N,
                   uint32_t K, hipStream_t s) {
  const dim3 block(256);
  const dim3 grid((N + 15) / 16, (M + 15) / 16);
  if (grid.y > 65535) return hipErrorInvalidConfiguration;
  if (c == nfhip::EType::F32)
    dense_kernel<AT, BT, float><<<grid, block, 0, s>>>((const AT*)A, (const BT*)B, (float*)C, M, N, K);
  else
    dense_kernel<AT, BT, half_t><<<grid, block, 0, s>>>((const AT*)A, (const BT*)B, (half_t*)C, M, N, K);
  return hipGetLastError();
}

}  // namespace nfk

namespace nfhip {

hipError_t launch_generic(QFmt q, EType t, const void* A, const void* W, void* C, uint32_t M,
                          uint32_t N, uint32_t K, hipStream_t s) {
  const dim3 block(256);
  const dim3 grid((N + 255) / 256, M);
  if (M > 65535) return hipErrorInvalidConfiguration;
  const uint8_t* w = static_cast<const uint8_t*>(W);
  if (q == QFmt::Q4_0) {
    if (t == EType::F32)
      nfk::generic_fused_kernel<nfk::Q4_0, float><<<grid, block, 0, s>>>((const float*)A, w, (float*)C, M, N, K);
    else
      nfk::generic_fused_kernel<nfk::Q4_0, nfk::half_t><<<grid, block, 0, s>>>((const nfk::half_t*)A, w, (nfk::half_t*)C, M, N, K);
  } else {
    if (t == EType::F32)
      nfk::generic_fused_kernel<nfk::Q8_0, float><<<grid, block, 0, s>>>((const float*)A, w, (float*)C, M, N, K);
    else
      nfk::generic_fused_kernel<nfk::Q8_0, nfk::half_t><<<grid, block, 0, s>>>((const nfk::half_t*)A, w, (nfk::half_t*)C, M, N, K);
  }
  return hipGetLastError();
}

hipError_t launch_dense(EType a, EType b, EType c, const void* A, const void* B, void* C,
                        uint32_t M, uint32_t N, uint32_t K, hipStream_t s) {
  // fp16 x fp16 -> fp16 with enough rows for MFMA tiles: the tiled MFMA kernel.
  if (a == EType::F16 && b == EType::F16 && c == EType::F16 && M >= 32 && K % 64 == 0 &&
      (uintptr_t)A % 16 == 0 && (uintptr_t)B % 16 == 0)
    return launch_dense_mfma_f16(A, B, C, M, N, K, s);
  if (a == EType::F32) {
    return b == EType::F32 ? nfk::dense_c<float, float>(c, A, B, C, M, N, K, s)
                           : nfk::dense_c<float, nfk::half_t>(c, A, B, C, M, N, K, s);
  }
  return b == EType::F32 ? nfk::dense_c<nfk::half_t, float>(c, A, B, C, M, N, K, s)
                         : nfk::dense_c<nfk::half_t, nfk::half_t>(c, A, B, C, M, N, K, s);
}

}  // namespace nfhip
