// ref_cpu.cpp — TEST INFRASTRUCTURE ONLY (bench.py's cpu_baseline leg).
//
// The reference's own CPU path for the fused Q4_0 / Q8_0 linear, timed on the
// host beside the GPU: the file-static ref_dequant_q4_0 / ref_dequant_q8_0 and
// f16_to_f32 of tests/driver/dequant_test.cpp (lines 77-128) come from that
// file, compiled where it lies under the reference tree (this file only
// includes it, renaming its main; nothing of it is copied here).  The matmul
// is the reference test's naive loop (dequant_test.cpp:313-319): for every
// output, a fp32 accumulator over k in order.  Here B is the dequantized
// weight in the [N, K] layout the kernels use, so the loop reads B[n*K + k]
// where the test reads its logical [K, N] copy.
//
// Threads split the output rows n; each thread dequantizes the weight rows it
// owns into a private fp32 row (the reference dequantizes the whole matrix
// first; per row keeps the working set in cache and does the same work).
// Built twice by oracle/Makefile: with the reference's own Release flags
// (-O3 -DNDEBUG, no -march), which bench.py times as the cpu_baseline, and
// for x86-64-v3 (AVX2 + FMA), reported beside it when the host CPU has
// those features.  The test's main refers to
// the provider's registration entry points, so the library links against
// libnf_plugin_hip.so, whose code it never calls.
#define main nf_ref_dequant_test_main
#include "tests/driver/dequant_test.cpp"
#undef main

#include <thread>

namespace {

void dequant_row(int fmt, const uint8_t* W, uint32_t n, uint32_t K, float* row) {
  const uint32_t nb = K / 32;
  if (fmt == 0) {
    const block_q4_0* b = reinterpret_cast<const block_q4_0*>(W) + (size_t)n * nb;
    for (uint32_t i = 0; i < nb; ++i) ref_dequant_q4_0(b + i, row + 32 * i);
  } else {
    const block_q8_0* b = reinterpret_cast<const block_q8_0*>(W) + (size_t)n * nb;
    for (uint32_t i = 0; i < nb; ++i) ref_dequant_q8_0(b + i, row + 32 * i);
  }
}

void rows(int fmt, const float* A, const uint8_t* W, float* C, uint32_t M, uint32_t N, uint32_t K, uint32_t n0,
          uint32_t n1) {
  std::vector<float> row(K);
  for (uint32_t n = n0; n < n1; ++n) {
    dequant_row(fmt, W, n, K, row.data());
    for (uint32_t m = 0; m < M; ++m) {
      float acc = 0.0f;
      for (uint32_t k = 0; k < K; ++k) acc += A[(size_t)m * K + k] * row[k];
      C[(size_t)m * N + n] = acc;
    }
  }
}

}  // namespace

// C[M, N] = A[M, K] . deq(W)^T, W = N*K/32 blocks of `fmt` (0 = Q4_0,
// 1 = Q8_0), K % 32 == 0; rows n0..n1-1 only, over `threads` threads.
extern "C" int nfref_cpu_fused(int fmt, const float* A, const uint8_t* W, float* C, uint32_t M, uint32_t N,
                               uint32_t K, uint32_t n0, uint32_t n1, uint32_t threads) {
  if ((fmt != 0 && fmt != 1) || K % 32 != 0 || n1 > N || n0 > n1) return -1;
  if (threads < 1) threads = 1;
  if (threads > n1 - n0) threads = n1 - n0 ? n1 - n0 : 1;
  if (threads == 1) {
    rows(fmt, A, W, C, M, N, K, n0, n1);
    return 0;
  }
  std::vector<std::thread> pool;
  const uint64_t span = n1 - n0;
  for (uint32_t t = 0; t < threads; ++t) {
    const uint32_t a = n0 + (uint32_t)(span * t / threads), b = n0 + (uint32_t)(span * (t + 1) / threads);
    pool.emplace_back(rows, fmt, A, W, C, M, N, K, a, b);
  }
  for (auto& th : pool) th.join();
  return 0;
}
