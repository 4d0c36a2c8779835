// gemm.hip — prefill-shaped fused dequant + matmul on CDNA4 MFMA.
//
// f16 path (metal_provider.mm:1433-1468 semantics): A f16 [M,K]; W quantized
// [N,K]; each weight is dequantized to fp16 as RNE(d*q) — the same bits
// dequant_*_f16 produces — staged in LDS, and multiplied on
// v_mfma_f32_16x16x32_f16 with fp32 accumulation; C is rounded to fp16.
//
// CTA tile 64(M) x 64(N), 4 waves each owning a 32x32 sub-tile (2x2 MFMA
// 16x16 fragments); one Q4_0/Q8_0 block (32 k) per main-loop step.
//
// MFMA 16x16x32 operand layout used here (lane l of a wave64):
//   A: row l%16, k = 8*(l/16) .. +7   (8 halves, 16 B)
//   B: col l%16, k = 8*(l/16) .. +7
//   D: col l%16, rows 4*(l/16) .. +3 (4 floats)
#include "../launch.hpp"
#include "common.hpp"

namespace nfk {

constexpr int kTile = 64;
constexpr int kLdsPad = 8;  // halves; keeps 16-B alignment of row starts

template <class QF>
__device__ __forceinline__ half8 quarter_f16(const uint8_t* blk, int quarter) {
  float v[8];
  quarter_f32<QF>(blk, quarter, v);
  half8 h;
#pragma unroll
  for (int i = 0; i < 8; ++i) h[i] = (half_t)v[i];
  return h;
}

template <class QF>
__global__ __launch_bounds__(256) void gemm_f16_kernel(const half_t* __restrict__ A,
                                                       const uint8_t* __restrict__ W,
                                                       half_t* __restrict__ C, int M, int N,
                                                       int K) {
  __shared__ __attribute__((aligned(16))) half_t As[kTile][32 + kLdsPad];
  __shared__ __attribute__((aligned(16))) half_t Ws[kTile][32 + kLdsPad];
  const int tid = threadIdx.x;
  const int wave = tid >> 6, lane = tid & 63;
  const int m_base = blockIdx.y * kTile, n_base = blockIdx.x * kTile;
  const int wm = (wave >> 1) * 32, wn = (wave & 1) * 32;
  const int nb = K >> 5;
  const int lr = tid >> 2, lq = tid & 3;  // loader: row, quarter
  float4v acc[2][2];
#pragma unroll
  for (int i = 0; i < 2; ++i)
#pragma unroll
    for (int j = 0; j < 2; ++j) acc[i][j] = float4v{0.f, 0.f, 0.f, 0.f};

  for (int b = 0; b < nb; ++b) {
    {
      const int gm = m_base + lr;
      half8 v = {};
      if (gm < M) v = *reinterpret_cast<const half8*>(A + (size_t)gm * K + (size_t)b * 32 + lq * 8);
      *reinterpret_cast<half8*>(&As[lr][lq * 8]) = v;
    }
    {
      const int gn = n_base + lr;
      half8 v = {};
      if (gn < N) v = quarter_f16<QF>(W + ((size_t)gn * nb + b) * QF::kBytes, lq);
      *reinterpret_cast<half8*>(&Ws[lr][lq * 8]) = v;
    }
    __syncthreads();
    const int r = lane & 15, kq = (lane >> 4) * 8;
    half8 af[2], bf[2];
#pragma unroll
    for (int i = 0; i < 2; ++i) af[i] = *reinterpret_cast<const half8*>(&As[wm + i * 16 + r][kq]);
#pragma unroll
    for (int j = 0; j < 2; ++j) bf[j] = *reinterpret_cast<const half8*>(&Ws[wn + j * 16 + r][kq]);
#pragma unroll
    for (int i = 0; i < 2; ++i)
#pragma unroll
      for (int j = 0; j < 2; ++j)
        acc[i][j] = __builtin_amdgcn_mfma_f32_16x16x32_f16(af[i], bf[j], acc[i][j], 0, 0, 0);
    __syncthreads();
  }

  const int col = lane & 15, row4 = (lane >> 4) * 4;
#pragma unroll
  for (int i = 0; i < 2; ++i)
#pragma unroll
    for (int j = 0; j < 2; ++j)
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        const int gm = m_base + wm + i * 16 + row4 + r;
        const int gn = n_base + wn + j * 16 + col;
        if (gm < M && gn < N) C[(size_t)gm * N + gn] = (half_t)acc[i][j][r];
      }
}

}  // namespace nfk

namespace nfhip {

hipError_t launch_gemm_mfma(QFmt q, EType t, const void* A, const void* W, void* C, uint32_t M,
                            uint32_t N, uint32_t K, hipStream_t s) {
  if (t != EType::F16) return hipErrorInvalidValue;  // f32 path uses the skinny kernels
  const dim3 block(256);
  const dim3 grid((N + nfk::kTile - 1) / nfk::kTile, (M + nfk::kTile - 1) / nfk::kTile);
  if (grid.y > 65535) return hipErrorInvalidConfiguration;
  const nfk::half_t* a = static_cast<const nfk::half_t*>(A);
  const uint8_t* w = static_cast<const uint8_t*>(W);
  nfk::half_t* c = static_cast<nfk::half_t*>(C);
  if (q == QFmt::Q4_0)
    nfk::gemm_f16_kernel<nfk::Q4_0><<<grid, block, 0, s>>>(a, w, c, M, N, K);
  else
    nfk::gemm_f16_kernel<nfk::Q8_0><<<grid, block, 0, s>>>(a, w, c, M, N, K);
  return hipGetLastError();
}

}  // namespace nfhip
