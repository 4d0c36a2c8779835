// dequant.hip — standalone dequantization of every GGUF block format the
// reference serves, f32 or f16 output: Q4_0, Q8_0, Q4_1, Q5_0, Q5_1
// (32-element blocks) and Q2_K, Q3_K, Q4_K, Q5_K, Q6_K (256-element
// super-blocks).
//
// Serves dequant_<fmt>[_f16] (metal_provider.mm:500-736 f32, 741-894 f16;
// op names :3157-3176), with the reference's layouts (its K-quants are
// simplified ones, not llama.cpp's interleaved order):
//   Q4_0 (18 B) {d, qs[16]}               d*(nib - 8)
//   Q8_0 (34 B) {d, int8 qs[32]}          d*q
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
// Kernels: HBM-bound (output bytes dominate: 4 B or 2 B per element against
// 0.33..1.06 B in).  Each thread produces 8 (f16) or 4 (f32) consecutive
// elements, all in one sub-block, and writes them with one 16-byte
// nontemporal store, so every store instruction of a wave covers 1 KiB of
// contiguous output (two 16-byte stores per lane 32 bytes apart measured
// 35-40% slower for f32; the nontemporal hint is worth 5-60% on these
// write-once streams).  Two kernels, chosen per format by measurement (see
// launch()): a direct one that reads block fields with 16-bit loads from
// global memory, and a staged one that first copies a workgroup's blocks to
// LDS.  Inputs at odd addresses run staged with byte loads; outputs that
// are not 16-byte aligned are written element by element.
#include "../launch.hpp"
#include "common.hpp"


namespace nfk {
namespace kq {

// Blocks start at even addresses (every block size is even; the launch
// checks the input pointer), and every multi-byte field below sits at an
// even offset, so fields are read with 16-bit loads from global memory or
// LDS alike.
__device__ __forceinline__ uint32_t u16at(const uint8_t* p) {
  return *reinterpret_cast<const uint16_t*>(p);
}
__device__ __forceinline__ float h16(const uint8_t* p) { return h2f_bits((uint16_t)u16at(p)); }

// N (2, 4 or 8) bytes from an even address, little-endian in a 64-bit word.
template <int N>
__device__ __forceinline__ uint64_t bytes_at(const uint8_t* p) {
  uint64_t x = 0;
#pragma unroll
  for (int k = 0; k < N / 2; ++k) x |= (uint64_t)u16at(p + 2 * k) << (16 * k);
  return x;
}

// 2-bit fields NE..: NE/4 bytes at p (NE = 8: two bytes, an even offset;
// NE = 4: one byte).
template <int NE>
__device__ __forceinline__ uint32_t crumbs_at(const uint8_t* p) {
  return NE == 8 ? u16at(p) : (uint32_t)p[0];
}

// Nibble j of the NE elements from i0 (a multiple of NE) of a 32-element
// block whose qs[16] starts at `qs`: elements i < 16 are the low nibbles of
// qs[i], elements i >= 16 the high nibbles of qs[i - 16].
template <int NE>
__device__ __forceinline__ uint64_t nibbles32(const uint8_t* qs, int i0) {
  const uint64_t x = bytes_at<NE>(qs + (i0 & 15));
  return (x >> ((i0 & 16) >> 2)) & 0x0F0F0F0F0F0F0F0Full;  // nibble j in byte j
}

// Each format's decode<NE>(b, i0, v) writes elements i0 .. i0+NE-1 of the
// block at `b`, for NE = 4 or 8 and i0 a multiple of NE: all of them lie in
// one sub-block and share their scale.

struct Q4_0 {
  static constexpr int kBytes = 18, kElems = 32;
  template <int NE>
  __device__ static void decode(const uint8_t* b, int i0, float v[NE]) {
    const float d = h16(b);
    const uint64_t q = nibbles32<NE>(b + 2, i0);
#pragma unroll
    for (int j = 0; j < NE; ++j) v[j] = d * (float)((int)((q >> (8 * j)) & 0xF) - 8);
  }
};

struct Q8_0 {
  static constexpr int kBytes = 34, kElems = 32;
  template <int NE>
  __device__ static void decode(const uint8_t* b, int i0, float v[NE]) {
    const float d = h16(b);
    const uint64_t q = bytes_at<NE>(b + 2 + i0);
#pragma unroll
    for (int j = 0; j < NE; ++j) v[j] = d * (float)(int8_t)(uint8_t)(q >> (8 * j));
  }
};

struct Q4_1 {
  static constexpr int kBytes = 20, kElems = 32;
  template <int NE>
  __device__ static void decode(const uint8_t* b, int i0, float v[NE]) {
    const float d = h16(b), m = h16(b + 2);
    const uint64_t q = nibbles32<NE>(b + 4, i0);
#pragma unroll
    for (int j = 0; j < NE; ++j) v[j] = d * (float)(int)((q >> (8 * j)) & 0xF) + m;
  }
};

struct Q5_0 {
  static constexpr int kBytes = 22, kElems = 32;
  template <int NE>
  __device__ static void decode(const uint8_t* b, int i0, float v[NE]) {
    const float d = h16(b);
    const int qh = b[2 + i0 / 8] >> (i0 & 7);
    const uint64_t q = nibbles32<NE>(b + 6, i0);
#pragma unroll
    for (int j = 0; j < NE; ++j)
      v[j] = d * (float)(((int)((q >> (8 * j)) & 0xF) | (((qh >> j) & 1) << 4)) - 16);
  }
};

struct Q5_1 {
  static constexpr int kBytes = 24, kElems = 32;
  template <int NE>
  __device__ static void decode(const uint8_t* b, int i0, float v[NE]) {
    const float d = h16(b), m = h16(b + 2);
    const int qh = b[4 + i0 / 8] >> (i0 & 7);
    const uint64_t q = nibbles32<NE>(b + 8, i0);
#pragma unroll
    for (int j = 0; j < NE; ++j) v[j] = d * (float)((int)((q >> (8 * j)) & 0xF) | (((qh >> j) & 1) << 4)) + m;
  }
};

struct Q2_K {
  static constexpr int kBytes = 84, kElems = 256;
  template <int NE>
  __device__ static void decode(const uint8_t* b, int i0, float v[NE]) {
    const int s = b[i0 / 16];
    const float sc = (float)(s & 0xF) * h16(b + 80);
    const float mn = (float)(s >> 4) * h16(b + 82);
    const uint32_t q = crumbs_at<NE>(b + 16 + i0 / 4);
#pragma unroll
    for (int j = 0; j < NE; ++j) v[j] = sc * (float)((q >> (2 * j)) & 3) - mn;
  }
};

// Q3_K codes (q2 | hbit << 2) - 4 of the NE elements from i0.
template <int NE>
__device__ __forceinline__ void q3_codes(const uint8_t* b, int i0, int q[NE]) {
  const int hm = b[i0 / 8] >> (i0 & 7);
  const uint32_t lo = crumbs_at<NE>(b + 32 + i0 / 4);
#pragma unroll
  for (int j = 0; j < NE; ++j) q[j] = (int)(((lo >> (2 * j)) & 3) | (((hm >> j) & 1) << 2)) - 4;
}

struct Q3_K {
  static constexpr int kBytes = 110, kElems = 256;
  template <int NE>
  __device__ static void decode(const uint8_t* b, int i0, float v[NE]) {
    const uint8_t* sc = b + 96;
    const int sub = i0 / 16;
    const int lo = sub < 8 ? (sc[sub] & 0xF) : (sc[sub - 8] >> 4);
    const int s = sub & 7;
    const int hi = (sc[8 + s / 2] >> (4 * (s % 2) + (sub < 8 ? 0 : 2))) & 3;
    const float ds = h16(b + 108) * (float)((lo | (hi << 4)) - 32);
    int q[NE];
    q3_codes<NE>(b, i0, q);
#pragma unroll
    for (int j = 0; j < NE; ++j) v[j] = ds * (float)q[j];
  }
};

// dequant_q3_k_f16's reading: the raw byte at offset 96 + sub of the block
// (which may lie in the next block; the caller stages it) minus 32.
struct Q3_K_RAW {
  static constexpr int kBytes = 110, kElems = 256;
  template <int NE>
  __device__ static void decode(const uint8_t* b, int i0, float v[NE]) {
    const float ds = h16(b + 108) * (float)((int)b[96 + i0 / 16] - 32);
    int q[NE];
    q3_codes<NE>(b, i0, q);
#pragma unroll
    for (int j = 0; j < NE; ++j) v[j] = ds * (float)q[j];
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
  template <int NE>
  __device__ static void decode(const uint8_t* b, int i0, float v[NE]) {
    int s, m;
    k_scale_min(b + 4, i0 / 32, &s, &m);
    const float dsc = h16(b) * (float)s;
    const float dmn = h16(b + 2) * (float)m;
    const uint64_t qs = bytes_at<NE / 2>(b + 16 + i0 / 2);  // element j: nibble j of qs
    const int qh = kHigh ? (b[144 + i0 / 8] >> (i0 & 7)) : 0;
#pragma unroll
    for (int j = 0; j < NE; ++j) {
      const int q = (int)((qs >> (4 * j)) & 0xF) | (((qh >> j) & 1) << 4);
      v[j] = dsc * (float)q - dmn;
    }
  }
};
using Q4_K = QK45<false>;
using Q5_K = QK45<true>;

struct Q6_K {
  static constexpr int kBytes = 210, kElems = 256;
  template <int NE>
  __device__ static void decode(const uint8_t* b, int i0, float v[NE]) {
    const float scale = (float)(int8_t)b[192 + i0 / 16] * h16(b + 208);
    const uint64_t ql = bytes_at<NE / 2>(b + i0 / 2);   // element j: nibble j
    const uint32_t qh = crumbs_at<NE>(b + 128 + i0 / 4);  // element j: bits 2j, 2j+1
#pragma unroll
    for (int j = 0; j < NE; ++j) {
      const int lo = (int)((ql >> (4 * j)) & 0xF);
      const int hi = (int)((qh >> (2 * j)) & 3);
      v[j] = scale * (float)(((hi << 4) | lo) - 32);
    }
  }
};

constexpr int kThreads = 256;

// Writes the NE values of `v` to o[0 .. NE): one 16-byte nontemporal store
// when the chunk is whole and the output 16-byte aligned, else one element
// at a time (n = number of valid elements).
template <typename OutT, int NE>
__device__ __forceinline__ void store_chunk(OutT* o, const float v[NE], uint64_t n, bool vec_out) {
  if (n >= (uint64_t)NE && vec_out) {
    if constexpr (NE == 4) {
      __builtin_nontemporal_store(float4v{v[0], v[1], v[2], v[3]}, reinterpret_cast<float4v*>(o));
    } else {
      half8 h;
#pragma unroll
      for (int i = 0; i < 8; ++i) h[i] = (half_t)v[i];  // round to nearest even
      __builtin_nontemporal_store(h, reinterpret_cast<half8*>(o));
    }
  } else {
    for (uint64_t i = 0; i < n && i < (uint64_t)NE; ++i) o[i] = (OutT)v[i];
  }
}

// Direct kernel: each thread reads its block fields straight from global
// memory (the lines are shared by the 4..32 threads of a block, so the
// reads after the first hit in cache) and writes NE elements.  Needs an
// even input address.
template <class F, typename OutT>
__global__ __launch_bounds__(kThreads) void dequant_direct_kernel(const uint8_t* __restrict__ w,
                                                                  OutT* __restrict__ out, uint64_t count,
                                                                  bool vec_out) {
  constexpr int NE = sizeof(OutT) == 4 ? 4 : 8;
  const uint64_t e0 = ((uint64_t)blockIdx.x * kThreads + threadIdx.x) * NE;
  if (e0 >= count) return;
  float v[NE];
  F::template decode<NE>(w + (e0 / F::kElems) * F::kBytes, (int)(e0 % F::kElems), v);
  store_chunk<OutT, NE>(out + e0, v, count - e0, vec_out);
}

// Staged kernel: a workgroup copies the blocks of its TILE elements, plus 4
// bytes past them (dequant_q3_k_f16's overrun; zeros past `in_bytes`), into
// LDS with coalesced dword loads (byte loads when the input is not 4-byte
// aligned), then decodes from LDS.
template <class F, typename OutT, int TILE>
__global__ __launch_bounds__(kThreads) void dequant_staged_kernel(const uint8_t* __restrict__ w,
                                                                  uint64_t in_bytes, OutT* __restrict__ out,
                                                                  uint64_t count, bool vec_out) {
  constexpr int kBlocks = TILE / F::kElems;
  constexpr int kSpan = kBlocks * F::kBytes + 4;
  static_assert((kBlocks * F::kBytes) % 16 == 0, "staging layout");
  __shared__ uint32_t stage[(kSpan + 3) / 4];
  uint8_t* sb = reinterpret_cast<uint8_t*>(stage);

  const uint64_t base = (uint64_t)blockIdx.x * (kBlocks * F::kBytes);
  // The launch covers ceil(count / TILE) workgroups and the input holds
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

  // Each store instruction of a wave covers 1 KiB of contiguous output (16
  // bytes per lane, lanes in address order); passes are kThreads * NE
  // elements apart.
  constexpr int NE = sizeof(OutT) == 4 ? 4 : 8;
#pragma unroll
  for (int pass = 0; pass < TILE / (kThreads * NE); ++pass) {
    const int local = pass * (kThreads * NE) + tid * NE;
    const uint64_t e0 = (uint64_t)blockIdx.x * TILE + local;
    if (e0 >= count) return;
    float v[NE];
    F::template decode<NE>(sb + (local / F::kElems) * F::kBytes, local % F::kElems, v);
    store_chunk<OutT, NE>(out + e0, v, count - e0, vec_out);
  }
}

template <class F, typename OutT, int TILE>
hipError_t launch_staged(const uint8_t* w, uint64_t in_bytes, OutT* out, uint64_t count, bool vec_out,
                         hipStream_t s) {
  const uint64_t wgs = (count + TILE - 1) / TILE;
  if (wgs > 0x7FFFFFFFull) return hipErrorInvalidValue;
  dequant_staged_kernel<F, OutT, TILE><<<dim3((unsigned)wgs), dim3(kThreads), 0, s>>>(w, in_bytes, out, count,
                                                                                      vec_out);
  return hipGetLastError();
}

// kDirect: the format's fields are few and 16-bit aligned, so the direct
// kernel wins (measured on MI355X, 11008 x 4096 elements: Q4_0, Q8_0, Q4_1,
// Q5_0, Q5_1, Q2_K, Q6_K at 6.5-7.2 TB/s); Q3_K, Q4_K and Q5_K, whose
// scales are scattered bytes, run staged (6.0-6.9 TB/s against 5.3-6.1
// direct), with 4096-element tiles for f16 and 2048 for f32.
template <class F, bool kDirect>
hipError_t launch(bool f16, const uint8_t* w, uint64_t in_bytes, void* out, uint64_t count, hipStream_t s) {
  const bool vec_out = (reinterpret_cast<uintptr_t>(out) & 15) == 0;
  if (kDirect && (reinterpret_cast<uintptr_t>(w) & 1) == 0) {
    const uint64_t per_wg = (uint64_t)kThreads * (f16 ? 8 : 4);
    const uint64_t wgs = (count + per_wg - 1) / per_wg;
    if (wgs > 0x7FFFFFFFull) return hipErrorInvalidValue;
    const dim3 grid((unsigned)wgs), block(kThreads);
    if (f16)
      dequant_direct_kernel<F, half_t><<<grid, block, 0, s>>>(w, (half_t*)out, count, vec_out);
    else
      dequant_direct_kernel<F, float><<<grid, block, 0, s>>>(w, (float*)out, count, vec_out);
    return hipGetLastError();
  }
  return f16 ? launch_staged<F, half_t, 4096>(w, in_bytes, (half_t*)out, count, vec_out, s)
             : launch_staged<F, float, 2048>(w, in_bytes, (float*)out, count, vec_out, s);
}

}  // namespace kq
}  // namespace nfk

namespace nfhip {

hipError_t launch_dequant(QFmt q, EType out_t, const void* w, uint64_t in_bytes, void* out, uint64_t count,
                          hipStream_t s) {
  if (count == 0) return hipSuccess;
  const uint64_t need = (count + block_elems(q) - 1) / block_elems(q) * block_bytes(q);
  if (in_bytes < need) return hipErrorInvalidValue;
  const bool f16 = out_t == EType::F16;
  const uint8_t* wp = static_cast<const uint8_t*>(w);
  using namespace nfk::kq;
  switch (q) {
    case QFmt::Q4_0: return launch<Q4_0, true>(f16, wp, in_bytes, out, count, s);
    case QFmt::Q8_0: return launch<Q8_0, true>(f16, wp, in_bytes, out, count, s);
    case QFmt::Q4_1: return launch<Q4_1, true>(f16, wp, in_bytes, out, count, s);
    case QFmt::Q5_0: return launch<Q5_0, true>(f16, wp, in_bytes, out, count, s);
    case QFmt::Q5_1: return launch<Q5_1, true>(f16, wp, in_bytes, out, count, s);
    case QFmt::Q2_K: return launch<Q2_K, true>(f16, wp, in_bytes, out, count, s);
    case QFmt::Q3_K:
      // The f16 op reads two bytes past its last block: staged only, where
      // those reads are bounded by in_bytes.
      return f16 ? launch<Q3_K_RAW, false>(true, wp, in_bytes, out, count, s)
                 : launch<Q3_K, false>(false, wp, in_bytes, out, count, s);
    case QFmt::Q4_K: return launch<Q4_K, false>(f16, wp, in_bytes, out, count, s);
    case QFmt::Q5_K: return launch<Q5_K, false>(f16, wp, in_bytes, out, count, s);
    case QFmt::Q6_K: return launch<Q6_K, true>(f16, wp, in_bytes, out, count, s);
    default: return hipErrorInvalidValue;
  }
}

}  // namespace nfhip
