// kquant.hip — standalone dequantization of the other GGUF block formats,
// f32 or f16 output: Q4_1, Q5_0, Q5_1 (32-element blocks) and Q2_K, Q3_K,
// Q4_K, Q5_K, Q6_K (256-element super-blocks).
//
// Serves dequant_<fmt>[_f16] (metal_provider.mm:534-736 f32, 761-894 f16),
// with the reference's simplified layouts, which are not llama.cpp's
// interleaved K-quant order:
//   Q4_1 (20 B) {d, m, qs[16]}            d*nib + m
//   Q5_0 (22 B) {d, qh[4], qs[16]}        d*((nib | bit<<4) - 16)
//   Q5_1 (24 B) {d, m, qh[4], qs[16]}     d*(nib | bit<<4) + m
//       nib: low nibble of qs[i] for i < 16, high nibble of qs[i-16] above;
//       bit: bit i of qh.
//   Q2_K (84 B) {scales[16], qs[64], d, dmin}
//       sub = i/16, s = scales[sub]; (s&15)*d * q2 - (s>>4)*dmin,
//       q2 = 2-bit field i%4 of qs[i/4].
//   Q3_K (110 B) {hmask[32], qs[64], scales[12], d}
//       d * (scale6(sub) - 32) * (q2 | hbit<<2 - 4), 6-bit scales packed as
//       low/high nibbles of bytes 0..7 plus 2-bit fields of bytes 8..11.
//       dequant_q3_k_f16 (metal_provider.mm:833-848) instead takes the raw
//       byte scales[sub] - 32 for sub = 0..15 of the 12-byte array: sub 12,13
//       read d's bytes, sub 14,15 the first two bytes of the next block (read
//       as 0 past the end of the input buffer).  Reproduced as written.
//   Q4_K (144 B) {d, dmin, scales[12], qs[128]}
//   Q5_K (176 B) {d, dmin, scales[12], qs[128], qh[32]}
//       sub = i/32, 6-bit (scale, min) pairs; q = nibble (i odd: high) of
//       qs[i/2] (| bit i of qh << 4 for Q5_K); d*sc*q - dmin*mn.
//   Q6_K (210 B) {ql[128], qh[64], int8 scales[16], d}
//       (scales[i/16]*d) * (((2-bit field i%4 of qh[i/4]) << 4 | nibble of
//       ql[i/2]) - 32).
//
// Numerics: every product in these expressions is exact in fp32 (an 11-bit
// fp16 significand times integers of at most 6+5 bits), so each f32 value is
// the exact result with one final rounding of the add/subtract — identical
// whether or not the compiler fuses it into an FMA.  Q6_K's last product
// (19-bit scale times a 6-bit code) is the one inexact multiply, rounded
// once as in the reference.  f16 outputs are the round-to-nearest-even half
// of that f32 value, as the reference's half(x) conversion.
//
// Kernel: HBM-bound (output bytes dominate: 4 B or 2 B per element against
// 0.56..0.82 B in).  A workgroup of 256 threads owns 2048 consecutive
// elements.  It copies its blocks (2048/E blocks of B bytes; 2048/E*B is a
// multiple of 16, so the copy is dword-aligned when the buffer is) plus four
// bytes past them (the Q3_K f16 overrun) into LDS with coalesced dword loads,
// then each thread decodes 8 consecutive elements (all in one block and one
// sub-block) from LDS and writes them with 16-byte stores.  Input of any
// alignment is staged byte by byte instead; an output that is not 16-byte
// aligned is written element by element.
#include "../launch.hpp"
#include "common.hpp"

namespace nfk {
namespace kq {

__device__ __forceinline__ float h16(const uint8_t* p) {
  return h2f_bits((uint16_t)(p[0] | (p[1] << 8)));
}

// Nibble of element i (0..31) of a 32-element block's qs[16].
__device__ __forceinline__ int nib32(const uint8_t* qs, int i) {
  return i < 16 ? (qs[i] & 0xF) : (qs[i - 16] >> 4);
}

struct Q4_1 {
  static constexpr int kBytes = 20, kElems = 32;
  __device__ static void decode8(const uint8_t* b, int i0, float v[8]) {
    const float d = h16(b), m = h16(b + 2);
#pragma unroll
    for (int j = 0; j < 8; ++j) v[j] = d * (float)nib32(b + 4, i0 + j) + m;
  }
};

struct Q5_0 {
  static constexpr int kBytes = 22, kElems = 32;
  __device__ static void decode8(const uint8_t* b, int i0, float v[8]) {
    const float d = h16(b);
    const int qh = b[2 + i0 / 8];
#pragma unroll
    for (int j = 0; j < 8; ++j) v[j] = d * (float)((nib32(b + 6, i0 + j) | (((qh >> j) & 1) << 4)) - 16);
  }
};

struct Q5_1 {
  static constexpr int kBytes = 24, kElems = 32;
  __device__ static void decode8(const uint8_t* b, int i0, float v[8]) {
    const float d = h16(b), m = h16(b + 2);
    const int qh = b[4 + i0 / 8];
#pragma unroll
    for (int j = 0; j < 8; ++j) v[j] = d * (float)(nib32(b + 8, i0 + j) | (((qh >> j) & 1) << 4)) + m;
  }
};

struct Q2_K {
  static constexpr int kBytes = 84, kElems = 256;
  __device__ static void decode8(const uint8_t* b, int i0, float v[8]) {
    const int s = b[i0 / 16];
    const float sc = (float)(s & 0xF) * h16(b + 80);
    const float mn = (float)(s >> 4) * h16(b + 82);
    const uint8_t* qs = b + 16 + i0 / 4;
#pragma unroll
    for (int j = 0; j < 8; ++j) v[j] = sc * (float)((qs[j / 4] >> ((j % 4) * 2)) & 3) - mn;
  }
};

// Q3_K code (q2 | hbit << 2) - 4 of the 8 elements from i0.
__device__ __forceinline__ void q3_codes(const uint8_t* b, int i0, int q[8]) {
  const int hm = b[i0 / 8];
  const uint8_t* qs = b + 32 + i0 / 4;
#pragma unroll
  for (int j = 0; j < 8; ++j) q[j] = (((qs[j / 4] >> ((j % 4) * 2)) & 3) | (((hm >> j) & 1) << 2)) - 4;
}

struct Q3_K {
  static constexpr int kBytes = 110, kElems = 256;
  __device__ static void decode8(const uint8_t* b, int i0, float v[8]) {
    const uint8_t* sc = b + 96;
    const int sub = i0 / 16;
    const int lo = sub < 8 ? (sc[sub] & 0xF) : (sc[sub - 8] >> 4);
    const int s = sub & 7;
    const int hi = (sc[8 + s / 2] >> (4 * (s % 2) + (sub < 8 ? 0 : 2))) & 3;
    const float ds = h16(b + 108) * (float)((lo | (hi << 4)) - 32);
    int q[8];
    q3_codes(b, i0, q);
#pragma unroll
    for (int j = 0; j < 8; ++j) v[j] = ds * (float)q[j];
  }
};

// dequant_q3_k_f16's reading: the raw byte at offset 96 + sub of the block
// (which may lie in the next block; the caller stages it) minus 32.
struct Q3_K_RAW {
  static constexpr int kBytes = 110, kElems = 256;
  __device__ static void decode8(const uint8_t* b, int i0, float v[8]) {
    const float ds = h16(b + 108) * (float)((int)b[96 + i0 / 16] - 32);
    int q[8];
    q3_codes(b, i0, q);
#pragma unroll
    for (int j = 0; j < 8; ++j) v[j] = ds * (float)q[j];
  }
};

// 6-bit scale and min of sub-block `sub` (0..7) of the 12 packed bytes.
__device__ __forceinline__ void k_scale_min(const uint8_t* sc, int sub, int* s, int* m) {
  if (sub < 4) {
    *s = sc[sub] & 0x3F;
    *m = sc[sub + 4] & 0x3F;
  } else {
    *s = (sc[sub - 4] >> 6) | ((sc[sub + 4] & 0x0F) << 2);
    *m = (sc[sub] >> 6) | ((sc[sub + 4] >> 4) << 2);
  }
}

template <bool kHigh>
struct QK45 {
  static constexpr int kBytes = kHigh ? 176 : 144, kElems = 256;
  __device__ static void decode8(const uint8_t* b, int i0, float v[8]) {
    int s, m;
    k_scale_min(b + 4, i0 / 32, &s, &m);
    const float dsc = h16(b) * (float)s;
    const float dmn = h16(b + 2) * (float)m;
    const uint8_t* qs = b + 16 + i0 / 2;
    const int qh = kHigh ? b[144 + i0 / 8] : 0;
#pragma unroll
    for (int j = 0; j < 8; ++j) {
      const int q = ((qs[j / 2] >> ((j & 1) * 4)) & 0xF) | (((qh >> j) & 1) << 4);
      v[j] = dsc * (float)q - dmn;
    }
  }
};
using Q4_K = QK45<false>;
using Q5_K = QK45<true>;

struct Q6_K {
  static constexpr int kBytes = 210, kElems = 256;
  __device__ static void decode8(const uint8_t* b, int i0, float v[8]) {
    const float scale = (float)(int8_t)b[192 + i0 / 16] * h16(b + 208);
    const uint8_t* ql = b + i0 / 2;
    const uint8_t* qh = b + 128 + i0 / 4;
#pragma unroll
    for (int j = 0; j < 8; ++j) {
      const int lo = (ql[j / 2] >> ((j & 1) * 4)) & 0xF;
      const int hi = (qh[j / 4] >> ((j % 4) * 2)) & 3;
      v[j] = scale * (float)(((hi << 4) | lo) - 32);
    }
  }
};

constexpr int kThreads = 256;
constexpr int kElemsPerWg = kThreads * 8;
// Largest staged span: 8 Q6_K blocks (1680 B) + 4 bytes of overrun.
constexpr int kMaxStage = 1684;

template <class F, typename OutT>
__global__ __launch_bounds__(kThreads) void kquant_dequant_kernel(const uint8_t* __restrict__ w,
                                                                  uint64_t in_bytes,
                                                                  OutT* __restrict__ out,
                                                                  uint64_t count, bool vec_out) {
  constexpr int kBlocks = kElemsPerWg / F::kElems;
  constexpr int kSpan = kBlocks * F::kBytes + 4;
  static_assert(kSpan <= kMaxStage && (kBlocks * F::kBytes) % 16 == 0, "staging layout");
  __shared__ uint32_t stage[(kMaxStage + 3) / 4];
  uint8_t* sb = reinterpret_cast<uint8_t*>(stage);

  const uint64_t base = (uint64_t)blockIdx.x * (kBlocks * F::kBytes);
  // The launch covers ceil(count / 2048) workgroups and the input holds
  // ceil(count / E) blocks, so base < in_bytes.
  const uint32_t avail = (uint32_t)min((uint64_t)kSpan, in_bytes - base);
  const uint8_t* src = w + base;
  const int tid = threadIdx.x;
  if ((reinterpret_cast<uintptr_t>(src) & 3) == 0) {
    const uint32_t nd = avail / 4;
    const uint32_t* s32 = reinterpret_cast<const uint32_t*>(src);
    for (uint32_t k = tid; k < nd; k += kThreads) stage[k] = s32[k];
    for (uint32_t k = nd * 4 + tid; k < (uint32_t)kSpan; k += kThreads) sb[k] = k < avail ? src[k] : 0;
  } else {
    for (uint32_t k = tid; k < (uint32_t)kSpan; k += kThreads) sb[k] = k < avail ? src[k] : 0;
  }
  __syncthreads();

  const uint64_t e0 = (uint64_t)blockIdx.x * kElemsPerWg + (uint64_t)tid * 8;
  if (e0 >= count) return;
  const int local = tid * 8;
  float v[8];
  F::decode8(sb + (local / F::kElems) * F::kBytes, local % F::kElems, v);
  OutT* o = out + e0;
  if (e0 + 8 <= count && vec_out) {
    if constexpr (sizeof(OutT) == 4) {
      reinterpret_cast<float4v*>(o)[0] = float4v{v[0], v[1], v[2], v[3]};
      reinterpret_cast<float4v*>(o)[1] = float4v{v[4], v[5], v[6], v[7]};
    } else {
      half8 h;
#pragma unroll
      for (int i = 0; i < 8; ++i) h[i] = (half_t)v[i];  // round to nearest even
      *reinterpret_cast<half8*>(o) = h;
    }
  } else {
    const uint64_t n = min((uint64_t)8, count - e0);
    for (uint64_t i = 0; i < n; ++i) o[i] = (OutT)v[i];
  }
}

template <class F>
hipError_t launch(bool f16, const uint8_t* w, uint64_t in_bytes, void* out, uint64_t count, hipStream_t s) {
  const uint64_t wgs = (count + kElemsPerWg - 1) / kElemsPerWg;
  if (wgs > 0x7FFFFFFFull) return hipErrorInvalidValue;
  const dim3 grid((unsigned)wgs), block(kThreads);
  // 16-byte stores need a 16-byte aligned output (an imported buffer may
  // start anywhere); otherwise elements are stored one by one.
  const bool vec_out = (reinterpret_cast<uintptr_t>(out) & 15) == 0;
  if (f16)
    kquant_dequant_kernel<F, half_t><<<grid, block, 0, s>>>(w, in_bytes, (half_t*)out, count, vec_out);
  else
    kquant_dequant_kernel<F, float><<<grid, block, 0, s>>>(w, in_bytes, (float*)out, count, vec_out);
  return hipGetLastError();
}

}  // namespace kq
}  // namespace nfk

namespace nfhip {

hipError_t launch_kquant_dequant(QFmt q, EType out_t, const void* w, uint64_t in_bytes, void* out,
                                 uint64_t count, hipStream_t s) {
  if (count == 0) return hipSuccess;
  const uint64_t need = (count + block_elems(q) - 1) / block_elems(q) * block_bytes(q);
  if (in_bytes < need) return hipErrorInvalidValue;
  const bool f16 = out_t == EType::F16;
  const uint8_t* wp = static_cast<const uint8_t*>(w);
  using namespace nfk::kq;
  switch (q) {
    case QFmt::Q4_1: return launch<Q4_1>(f16, wp, in_bytes, out, count, s);
    case QFmt::Q5_0: return launch<Q5_0>(f16, wp, in_bytes, out, count, s);
    case QFmt::Q5_1: return launch<Q5_1>(f16, wp, in_bytes, out, count, s);
    case QFmt::Q2_K: return launch<Q2_K>(f16, wp, in_bytes, out, count, s);
    case QFmt::Q3_K:
      return f16 ? launch<Q3_K_RAW>(true, wp, in_bytes, out, count, s)
                 : launch<Q3_K>(false, wp, in_bytes, out, count, s);
    case QFmt::Q4_K: return launch<Q4_K>(f16, wp, in_bytes, out, count, s);
    case QFmt::Q5_K: return launch<Q5_K>(f16, wp, in_bytes, out, count, s);
    case QFmt::Q6_K: return launch<Q6_K>(f16, wp, in_bytes, out, count, s);
    default: return hipErrorInvalidValue;
  }
}

}  // namespace nfhip
