// common.hpp — device helpers shared by the gfx950 kernels.
//
// Block formats (ggml/GGUF, 32 elements per block along K):
//   Q4_0 (18 B): u16 fp16 scale d, then qs[16]; element i < 16 is the low
//                nibble of qs[i], element i >= 16 the high nibble of
//                qs[i-16]; value = d * (nibble - 8).
//   Q8_0 (34 B): u16 fp16 scale d, then 32 int8 codes; value = d * q.
// (metal_provider.mm:500-530, dequant_test.cpp:61-128.)
//
// Numerics: the f32 value d*q is exact in fp32 (an 11-bit significand times
// an integer of at most 8 bits), so the f32 path is exact.  The f16 path
// rounds that exact product to nearest-even fp16 (metal_provider.mm:749,758),
// which is what a single IEEE fp16 conversion or an fp16 multiply of the two
// exactly-representable factors yields.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace nfk {

typedef _Float16 half_t;
typedef _Float16 half8 __attribute__((ext_vector_type(8)));
typedef _Float16 half2v __attribute__((ext_vector_type(2)));
typedef float float4v __attribute__((ext_vector_type(4)));
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));

typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef __bf16 bf16x2v __attribute__((ext_vector_type(2)));
typedef float float2s __attribute__((ext_vector_type(2)));

// Two floats -> their bf16 pair, exact when each float has <= 8 significant
// bits (upper halves of the f32 patterns).
__device__ __forceinline__ uint32_t pack_hi16(float a, float b) {
  return __builtin_amdgcn_perm(__builtin_bit_cast(uint32_t, b), __builtin_bit_cast(uint32_t, a), 0x07060302u);
}

// Two round-to-nearest bf16 pieces of 8 floats: p1 = RNE_bf16(x), p2 =
// RNE_bf16(x - p1) (x - p1 is exact in f32),
// so |p2| <= 2^-8 |x| and |x - p1 - p2| <= 2^-8 |x - p1| <= 2^-16 |x|.
__device__ __forceinline__ void split2_rne(const float (&x)[8], bf16x8& p1, bf16x8& p2) {
#pragma unroll
  for (int j = 0; j < 4; ++j) {
    const float2s v = {x[2 * j], x[2 * j + 1]};
    const bf16x2v h1 = __builtin_convertvector(v, bf16x2v);
    const float2s r1 = v - __builtin_convertvector(h1, float2s);
    const bf16x2v h2 = __builtin_convertvector(r1, bf16x2v);
    p1[2 * j] = h1[0];
    p1[2 * j + 1] = h1[1];
    p2[2 * j] = h2[0];
    p2[2 * j + 1] = h2[1];
  }
}

// Two bf16 pieces of 8 floats: p1 = x truncated to bf16 (its upper 16 bits,
// exact), p2 = the remainder x - p1 (exact in f32) rounded to nearest bf16.
// |x - p1 - p2| <= 2^-9 |x - p1| < 2^-16 |x|, so a product p * x taken as
// p * p1 + p * p2 (each exact in fp32) is within 2^-16 of p * x.
__device__ __forceinline__ void split2(const float (&x)[8], bf16x8& p1, bf16x8& p2) {
#pragma unroll
  for (int j = 0; j < 4; ++j) {
    const uint32_t u0 = __builtin_bit_cast(uint32_t, x[2 * j]) & 0xFFFF0000u;
    const uint32_t u1 = __builtin_bit_cast(uint32_t, x[2 * j + 1]) & 0xFFFF0000u;
    const float2s r = {x[2 * j] - __builtin_bit_cast(float, u0), x[2 * j + 1] - __builtin_bit_cast(float, u1)};
    const bf16x2v h2 = __builtin_convertvector(r, bf16x2v);
    const uint32_t hi = __builtin_amdgcn_perm(u1, u0, 0x07060302u);
    p1[2 * j] = __builtin_bit_cast(bf16x2v, hi)[0];
    p1[2 * j + 1] = __builtin_bit_cast(bf16x2v, hi)[1];
    p2[2 * j] = h2[0];
    p2[2 * j + 1] = h2[1];
  }
}

struct Q4_0 {
  static constexpr int kBytes = 18;
};
struct Q8_0 {
  static constexpr int kBytes = 34;
};

__device__ __forceinline__ float h2f_bits(uint16_t h) {
  return (float)__builtin_bit_cast(half_t, h);
}

// Value of element `i` (0..31) of a block starting at `blk` (2-byte aligned).
template <class QF>
__device__ __forceinline__ int code_of(const uint8_t* blk, int i);

template <>
__device__ __forceinline__ int code_of<Q4_0>(const uint8_t* blk, int i) {
  const uint8_t b = blk[2 + (i & 15)];
  return (i < 16 ? (b & 0xF) : (b >> 4)) - 8;
}

template <>
__device__ __forceinline__ int code_of<Q8_0>(const uint8_t* blk, int i) {
  return (int)(int8_t)blk[2 + i];
}

// Eight consecutive elements [8*quarter, 8*quarter+8) of one block, as exact
// f32 products d*q.  `blk` is 2-byte aligned; loads are 16-bit.
template <class QF>
__device__ __forceinline__ void quarter_f32(const uint8_t* blk, int quarter, float v[8]);

template <>
__device__ __forceinline__ void quarter_f32<Q4_0>(const uint8_t* blk, int quarter, float v[8]) {
  const uint16_t* p = reinterpret_cast<const uint16_t*>(blk);
  const float d = h2f_bits(p[0]);
  // Quarters 0/2 read qs[0..7], quarters 1/3 read qs[8..15]; quarters 2/3
  // take the high nibbles.
  const uint16_t* q = p + 1 + (quarter & 1) * 4;
  const int shift = (quarter >> 1) * 4;
#pragma unroll
  for (int j = 0; j < 4; ++j) {
    const uint32_t s = q[j];
    v[2 * j + 0] = d * (float)((int)((s >> shift) & 0xF) - 8);
    v[2 * j + 1] = d * (float)((int)((s >> (8 + shift)) & 0xF) - 8);
  }
}

template <>
__device__ __forceinline__ void quarter_f32<Q8_0>(const uint8_t* blk, int quarter, float v[8]) {
  const uint16_t* p = reinterpret_cast<const uint16_t*>(blk);
  const float d = h2f_bits(p[0]);
  const uint16_t* q = p + 1 + quarter * 4;
#pragma unroll
  for (int j = 0; j < 4; ++j) {
    const uint32_t s = q[j];
    v[2 * j + 0] = d * (float)(int)(int8_t)(s & 0xFF);
    v[2 * j + 1] = d * (float)(int)(int8_t)(s >> 8);
  }
}

// Partial tiles exchanged between the workgroups of a split-K fix-up.  The
// stores and loads carry the sc1 cache policy (buffer instructions, 16 bytes
// per lane): on this chip sc1 accesses write through to, and read from, the
// level that all XCDs share rather than an XCD's own L2.  A workgroup stores
// its partial, waits for the stores to complete (s_waitcnt vmcnt(0)), then
// bumps the tile counter with a relaxed agent-scope atomic; the workgroup
// that sees the last count reads the partials back with sc1 loads.  Every
// access to the partials is sc1, so no L2 writeback or invalidate is needed:
// an agent-scope release / acquire on the counter emits buffer_wbl2 /
// buffer_inv for the whole L2 of the XCD, which cost 10-15 % of a decode
// step of small-batch launches (TinyLlama f32 M = 16: 1291 -> 1109 us).
constexpr int kCachePolicySc1 = 0x10;

struct CoherentTile {
  __amdgpu_buffer_rsrc_t r;
  __device__ __forceinline__ CoherentTile(const void* base, uint32_t bytes)
      : r(__builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(base), (short)0, (int)bytes, 0x00020000)) {}
  __device__ __forceinline__ void store(uint32_t i16, float4v v) const {
    __builtin_amdgcn_raw_buffer_store_b128(__builtin_bit_cast(u32x4, v), r, i16 * 16u, 0, kCachePolicySc1);
  }
  __device__ __forceinline__ float4v load(uint32_t i16) const {
    return __builtin_bit_cast(float4v, __builtin_amdgcn_raw_buffer_load_b128(r, i16 * 16u, 0, kCachePolicySc1));
  }
};

__device__ __forceinline__ float wave_sum(float v) {
#pragma unroll
  for (int off = 32; off > 0; off >>= 1) v += __shfl_xor(v, off, 64);
  return v;
}

}  // namespace nfk
