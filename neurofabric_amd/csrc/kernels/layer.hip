// layer.hip — the layer ops around the linears: element-wise add / mul,
// silu, gelu, relu, the attention_prefill mock, rms_norm, rope, rope_batch,
// softmax, embedding_lookup and argmax (metal_provider.mm:44-147, 1002-1150,
// 1601-1619).  All are HBM- or latency-bound; fp32 arithmetic, f16 variants
// read and write halves (selected by the output dtype, as the reference does).
//
// Numerics: add and mul are single IEEE operations (f16: computed in half
// precision and rounded once, as half * half / half + half), so they match
// the reference bit for bit.  The transcendental ops use the device's
// accurate expf / tanhf / powf / sincosf / sqrt; row reductions (rms_norm's
// sum of squares, softmax's sum) are tree sums in fp32 rather than the
// reference's sequential loop, so those ops agree with it to rounding.
#include "../launch.hpp"
#include "common.hpp"

namespace nfk {

using EwFnK = nfhip::EwFn;

namespace layer {

constexpr int kThreads = 256;

// ---- element-wise -----------------------------------------------------------

template <EwFnK F>
__device__ __forceinline__ float unary_f(float x) {
  if constexpr (F == EwFnK::Silu) {
    return x / (1.0f + expf(-x));
  } else if constexpr (F == EwFnK::Gelu) {
    const float x3 = x * x * x;
    return 0.5f * x * (1.0f + tanhf(0.7978845608f * (x + 0.044715f * x3)));
  } else {
    return x > 0.0f ? x : 0.0f;
  }
}

// 16-byte chunks (4 f32 / 8 f16) per thread when every pointer is 16-byte
// aligned; otherwise one element per thread.
template <typename T, EwFnK F, bool VEC>
__global__ __launch_bounds__(kThreads) void binary_kernel(const T* __restrict__ a, const T* __restrict__ b,
                                                          T* __restrict__ out, uint64_t n) {
  constexpr int V = VEC ? 16 / (int)sizeof(T) : 1;
  const uint64_t i0 = ((uint64_t)blockIdx.x * kThreads + threadIdx.x) * V;
  if (i0 >= n) return;
  if (VEC && i0 + V <= n) {
    typedef T vec_t __attribute__((ext_vector_type(V)));
    const vec_t x = *reinterpret_cast<const vec_t*>(a + i0);
    const vec_t y = *reinterpret_cast<const vec_t*>(b + i0);
    *reinterpret_cast<vec_t*>(out + i0) = F == EwFnK::Add ? x + y : x * y;
  } else {
    for (uint64_t i = i0; i < n && i < i0 + V; ++i) out[i] = F == EwFnK::Add ? (T)(a[i] + b[i]) : (T)(a[i] * b[i]);
  }
}

template <typename T, EwFnK F, bool VEC>
__global__ __launch_bounds__(kThreads) void unary_kernel(const T* __restrict__ in, T* out, uint64_t n) {
  constexpr int V = VEC ? 16 / (int)sizeof(T) : 1;
  const uint64_t i0 = ((uint64_t)blockIdx.x * kThreads + threadIdx.x) * V;
  if (i0 >= n) return;
  if (VEC && i0 + V <= n) {
    typedef T vec_t __attribute__((ext_vector_type(V)));
    vec_t x = *reinterpret_cast<const vec_t*>(in + i0);
#pragma unroll
    for (int j = 0; j < V; ++j) x[j] = (T)unary_f<F>((float)x[j]);
    *reinterpret_cast<vec_t*>(out + i0) = x;
  } else {
    for (uint64_t i = i0; i < n && i < i0 + V; ++i) out[i] = (T)unary_f<F>((float)in[i]);
  }
}

// attention_prefill mock: k = x * 0.5, v = x * -0.25 (metal_provider.mm:56-66).
__global__ __launch_bounds__(kThreads) void mock_prefill_kernel(const float* __restrict__ in, float* __restrict__ k,
                                                                float* __restrict__ v, uint64_t nk, uint64_t nv) {
  const uint64_t i = (uint64_t)blockIdx.x * kThreads + threadIdx.x;
  if (i < nk) k[i] = in[i] * 0.5f;
  if (i < nv) v[i] = in[i] * -0.25f;
}

// ---- row reductions -----------------------------------------------------------

// Sum over the workgroup (256 threads = 4 waves): wave sums by shuffle, then
// the four wave sums in a fixed order.  Every thread gets the total.
__device__ __forceinline__ float block_sum(float x, float* red) {
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) x += __shfl_xor(x, o);
  const int w = threadIdx.x >> 6;
  if ((threadIdx.x & 63) == 0) red[w] = x;
  __syncthreads();
  const float t = (red[0] + red[1]) + (red[2] + red[3]);
  __syncthreads();
  return t;
}

__device__ __forceinline__ float block_max(float x, float* red) {
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) x = fmaxf(x, __shfl_xor(x, o));
  const int w = threadIdx.x >> 6;
  if ((threadIdx.x & 63) == 0) red[w] = x;
  __syncthreads();
  const float t = fmaxf(fmaxf(red[0], red[1]), fmaxf(red[2], red[3]));
  __syncthreads();
  return t;
}

// rms_norm: one workgroup per row of `dim` (metal_provider.mm:85-102, 1069-1084).
template <typename T>
__global__ __launch_bounds__(kThreads) void rms_norm_kernel(const T* __restrict__ in, const float* __restrict__ w,
                                                            T* __restrict__ out, uint32_t dim, float eps) {
  __shared__ float red[4];
  const uint64_t base = (uint64_t)blockIdx.x * dim;
  float ss = 0.0f;
  for (uint32_t j = threadIdx.x; j < dim; j += kThreads) {
    const float v = (float)in[base + j];
    ss += v * v;
  }
  ss = block_sum(ss, red);
  const float rms = 1.0f / sqrtf(ss / (float)dim + eps);
  for (uint32_t j = threadIdx.x; j < dim; j += kThreads) out[base + j] = (T)((float)in[base + j] * rms * w[j]);
}

// The same with the row held in registers: 16-byte loads (NC per thread,
// all issued before the sum; a chunk past the row re-reads the row's last
// chunk and counts 0), then 16-byte stores.  dim % (16 / sizeof(T)) == 0.
template <typename T, int NC>
__global__ __launch_bounds__(kThreads) void rms_norm_vec_kernel(const T* __restrict__ in,
                                                                const float* __restrict__ w,
                                                                T* __restrict__ out, uint32_t dim, float eps) {
  constexpr int VW = 16 / sizeof(T);
  typedef T VecT __attribute__((ext_vector_type(VW)));
  __shared__ float red[4];
  const uint64_t base = (uint64_t)blockIdx.x * dim;
  VecT v[NC];
#pragma unroll
  for (int c = 0; c < NC; ++c) {
    const uint32_t j = (c * kThreads + threadIdx.x) * VW;
    v[c] = *reinterpret_cast<const VecT*>(in + base + (j < dim ? j : dim - VW));
  }
  float ss = 0.0f;
#pragma unroll
  for (int c = 0; c < NC; ++c) {
    const uint32_t j = (c * kThreads + threadIdx.x) * VW;
    float part = 0.0f;
#pragma unroll
    for (int e = 0; e < VW; ++e) part += (float)v[c][e] * (float)v[c][e];
    ss += j < dim ? part : 0.0f;
  }
  ss = block_sum(ss, red);
  const float rms = 1.0f / sqrtf(ss / (float)dim + eps);
#pragma unroll
  for (int c = 0; c < NC; ++c) {
    const uint32_t j = (c * kThreads + threadIdx.x) * VW;
    if (j >= dim) continue;
    VecT o;
#pragma unroll
    for (int e = 0; e < VW; ++e) o[e] = (T)((float)v[c][e] * rms * w[j + e]);
    *reinterpret_cast<VecT*>(out + base + j) = o;
  }
}

// softmax over rows of `dim` (metal_provider.mm:1002-1030).
__global__ __launch_bounds__(kThreads) void softmax_kernel(const float* __restrict__ in, float* __restrict__ out,
                                                           uint32_t dim) {
  __shared__ float red[4];
  const uint64_t base = (uint64_t)blockIdx.x * dim;
  float m = -INFINITY;
  for (uint32_t j = threadIdx.x; j < dim; j += kThreads) m = fmaxf(m, in[base + j]);
  m = block_max(m, red);
  float s = 0.0f;
  for (uint32_t j = threadIdx.x; j < dim; j += kThreads) {
    const float e = expf(in[base + j] - m);
    out[base + j] = e;
    s += e;
  }
  s = block_sum(s, red);
  const float inv = 1.0f / s;
  // each thread rescales exactly the elements it wrote, so no barrier is needed
  for (uint32_t j = threadIdx.x; j < dim; j += kThreads) out[base + j] *= inv;
}

// argmax of each row (metal_provider.mm:1601-1619): the first index of the
// largest non-NaN value, or 0 when the row starts with NaN (the reference's
// strict `>` scan never leaves a NaN start).
__global__ __launch_bounds__(kThreads) void argmax_kernel(const float* __restrict__ in, int32_t* __restrict__ out,
                                                          uint32_t dim) {
  __shared__ float rv[4];
  __shared__ uint32_t ri[4];
  const uint64_t base = (uint64_t)blockIdx.x * dim;
  constexpr uint32_t kNone = 0xFFFFFFFFu;
  if (dim == 0) {  // no elements: the reference's scan returns its start, 0
    if (threadIdx.x == 0) out[blockIdx.x] = 0;
    return;
  }
  float best = -INFINITY;
  uint32_t idx = kNone;
  for (uint32_t j = threadIdx.x; j < dim; j += kThreads) {
    const float x = in[base + j];
    if (!isnan(x) && (idx == kNone || x > best)) {
      best = x;
      idx = j;
    }
  }
  auto better = [](float b2, uint32_t i2, float b1, uint32_t i1) {
    if (i2 == kNone) return false;
    if (i1 == kNone) return true;
    return b2 > b1 || (b2 == b1 && i2 < i1);
  };
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) {
    const float b2 = __shfl_xor(best, o);
    const uint32_t i2 = __shfl_xor(idx, o);
    if (better(b2, i2, best, idx)) {
      best = b2;
      idx = i2;
    }
  }
  const int w = threadIdx.x >> 6;
  if ((threadIdx.x & 63) == 0) {
    rv[w] = best;
    ri[w] = idx;
  }
  __syncthreads();
  if (threadIdx.x == 0) {
    float b = rv[0];
    uint32_t i = ri[0];
    for (int k = 1; k < 4; ++k)
      if (better(rv[k], ri[k], b, i)) {
        b = rv[k];
        i = ri[k];
      }
    out[blockIdx.x] = isnan(in[base]) ? 0 : (int32_t)i;
  }
}

// ---- wide rows: each row split over many workgroups -------------------------------
//
// A row of a 128K-entry vocabulary in one workgroup leaves most of the chip
// idle, so wide rows go in kChunk-element chunks: the first kernel reduces
// each chunk (softmax: its max and its sum of e^(x - max); argmax: its best
// value and index) into the workspace, the second merges a row's chunks in
// chunk order (deterministic) and, for softmax, writes the chunk's outputs.

constexpr uint32_t kChunk = 4096;

__global__ __launch_bounds__(kThreads) void softmax_chunk_kernel(const float* __restrict__ in, uint32_t dim,
                                                                 uint32_t chunks, float* __restrict__ part) {
  __shared__ float red[4];
  const uint32_t c = blockIdx.x, row = blockIdx.y;
  const uint64_t base = (uint64_t)row * dim;
  const uint32_t j0 = c * kChunk, j1 = min(dim, j0 + kChunk);
  float m = -INFINITY;
  for (uint32_t j = j0 + threadIdx.x; j < j1; j += kThreads) m = fmaxf(m, in[base + j]);
  m = block_max(m, red);
  float sum = 0.0f;
  for (uint32_t j = j0 + threadIdx.x; j < j1; j += kThreads) sum += expf(in[base + j] - m);
  sum = block_sum(sum, red);
  if (threadIdx.x == 0) {
    part[((uint64_t)row * chunks + c) * 2] = m;
    part[((uint64_t)row * chunks + c) * 2 + 1] = sum;
  }
}

__global__ __launch_bounds__(kThreads) void softmax_write_kernel(const float* __restrict__ in, float* __restrict__ out,
                                                                 uint32_t dim, uint32_t chunks,
                                                                 const float* __restrict__ part) {
  const uint32_t c = blockIdx.x, row = blockIdx.y;
  const float* pr = part + (uint64_t)row * chunks * 2;
  float M = -INFINITY;
  for (uint32_t k = 0; k < chunks; ++k) M = fmaxf(M, pr[2 * k]);
  float S = 0.0f;
  for (uint32_t k = 0; k < chunks; ++k) S += pr[2 * k + 1] * expf(pr[2 * k] - M);
  const float inv = 1.0f / S;
  const uint64_t base = (uint64_t)row * dim;
  const uint32_t j0 = c * kChunk, j1 = min(dim, j0 + kChunk);
  for (uint32_t j = j0 + threadIdx.x; j < j1; j += kThreads) out[base + j] = expf(in[base + j] - M) * inv;
}

constexpr uint32_t kNoIdx = 0xFFFFFFFFu;

__device__ __forceinline__ bool arg_better(float b2, uint32_t i2, float b1, uint32_t i1) {
  if (i2 == kNoIdx) return false;
  if (i1 == kNoIdx) return true;
  return b2 > b1 || (b2 == b1 && i2 < i1);
}

__global__ __launch_bounds__(kThreads) void argmax_chunk_kernel(const float* __restrict__ in, uint32_t dim,
                                                                uint32_t chunks, float* __restrict__ part) {
  __shared__ float rv[4];
  __shared__ uint32_t ri[4];
  const uint32_t c = blockIdx.x, row = blockIdx.y;
  const uint64_t base = (uint64_t)row * dim;
  const uint32_t j0 = c * kChunk, j1 = min(dim, j0 + kChunk);
  float best = -INFINITY;
  uint32_t idx = kNoIdx;
  for (uint32_t j = j0 + threadIdx.x; j < j1; j += kThreads) {
    const float x = in[base + j];
    if (!isnan(x) && (idx == kNoIdx || x > best)) {
      best = x;
      idx = j;
    }
  }
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) {
    const float b2 = __shfl_xor(best, o);
    const uint32_t i2 = __shfl_xor(idx, o);
    if (arg_better(b2, i2, best, idx)) {
      best = b2;
      idx = i2;
    }
  }
  if ((threadIdx.x & 63) == 0) {
    rv[threadIdx.x >> 6] = best;
    ri[threadIdx.x >> 6] = idx;
  }
  __syncthreads();
  if (threadIdx.x == 0) {
    float b = rv[0];
    uint32_t i = ri[0];
    for (int k = 1; k < 4; ++k)
      if (arg_better(rv[k], ri[k], b, i)) {
        b = rv[k];
        i = ri[k];
      }
    part[((uint64_t)row * chunks + c) * 2] = b;
    part[((uint64_t)row * chunks + c) * 2 + 1] = __uint_as_float(i);
  }
}

__global__ __launch_bounds__(64) void argmax_merge_kernel(const float* __restrict__ in, uint32_t dim, uint32_t chunks,
                                                          const float* __restrict__ part, int32_t* __restrict__ out) {
  const uint32_t row = blockIdx.x;
  if (threadIdx.x != 0) return;
  const float* pr = part + (uint64_t)row * chunks * 2;
  float b = -INFINITY;
  uint32_t i = kNoIdx;
  for (uint32_t k = 0; k < chunks; ++k) {
    const uint32_t ik = __float_as_uint(pr[2 * k + 1]);
    if (arg_better(pr[2 * k], ik, b, i)) {
      b = pr[2 * k];
      i = ik;
    }
  }
  out[row] = isnan(in[(uint64_t)row * dim]) ? 0 : (int32_t)i;
}

// ---- position encodings and lookups --------------------------------------------

// RoPE on rows of head_dim: pairs (p, p + head_dim/2) rotated by pos * theta^(-2p/head_dim).
// rope_batch: [seq, n_heads, head_dim], pos = token + step (metal_provider.mm:125-147);
// rope: every row at pos = step (metal_provider.mm:104-122, with the rotation
// the kernel intends for both halves of each row).
// One thread per (group of rows at one position, pair p): the rotation of
// pair p is computed once and applied to every row of the group (up to
// kRopeRows of the n_heads rows of a token for rope_batch, a divisor of
// n_heads so no group spans two tokens; kRopeRows rows for rope).  Small
// groups keep many threads in flight: each row is a dependent load / store.
constexpr uint32_t kRopeRows = 8;

template <typename T>
__global__ __launch_bounds__(kThreads) void rope_kernel(const T* __restrict__ in, T* __restrict__ out, uint64_t rows,
                                                        uint32_t head_dim, uint32_t rows_per_group,
                                                        uint32_t rows_per_pos, uint32_t step, float theta,
                                                        bool batch) {
  const uint32_t half = head_dim / 2;
  const uint64_t id = (uint64_t)blockIdx.x * kThreads + threadIdx.x;
  const uint64_t grp = id / half;
  const uint32_t pair = (uint32_t)(id % half);
  const uint64_t r0 = grp * rows_per_group;
  if (r0 >= rows) return;
  const uint64_t pos = batch ? r0 / rows_per_pos + step : step;
  const float freq = 1.0f / powf(theta, (float)(2 * pair) / (float)head_dim);
  const float angle = (float)pos * freq;
  float s, c;
  sincosf(angle, &s, &c);
  const uint64_t r1 = min(rows, r0 + rows_per_group);
  for (uint64_t r = r0; r < r1; ++r) {
    const uint64_t base = r * head_dim;
    const float x0 = (float)in[base + pair];
    const float x1 = (float)in[base + pair + half];
    out[base + pair] = (T)(x0 * c - x1 * s);
    out[base + pair + half] = (T)(x0 * s + x1 * c);
  }
}

// embedding_lookup: out[t, :] = weights[ids[t], :] for t < seq_len; a token
// id outside the table writes zeros (the reference reads out of bounds).
template <typename T>
__global__ __launch_bounds__(kThreads) void embedding_kernel(const T* __restrict__ w, uint32_t vocab,
                                                             const int32_t* __restrict__ ids, T* __restrict__ out,
                                                             uint64_t n, uint32_t dim, uint32_t seq_len) {
  const uint64_t id = (uint64_t)blockIdx.x * kThreads + threadIdx.x;
  if (id >= n) return;
  const uint64_t t = id / dim;
  if (t >= seq_len) return;
  const int32_t tok = ids[t];
  out[id] = (tok >= 0 && (uint32_t)tok < vocab) ? w[(uint64_t)tok * dim + id % dim] : (T)0.0f;
}

// The same in 16-byte chunks (rows of dim % (16 / sizeof(T)) == 0, so no
// chunk straddles two rows): a thread copies one chunk of one token's row.
template <typename T>
__global__ __launch_bounds__(kThreads) void embedding_vec_kernel(const T* __restrict__ w, uint32_t vocab,
                                                                 const int32_t* __restrict__ ids,
                                                                 T* __restrict__ out, uint64_t nchunks,
                                                                 uint32_t row_chunks, uint32_t seq_len) {
  constexpr int VW = 16 / sizeof(T);
  typedef T VecT __attribute__((ext_vector_type(VW)));
  const uint64_t id = (uint64_t)blockIdx.x * kThreads + threadIdx.x;
  if (id >= nchunks) return;
  const uint64_t t = id / row_chunks;
  if (t >= seq_len) return;
  const int32_t tok = ids[t];
  VecT v = {};
  if (tok >= 0 && (uint32_t)tok < vocab)
    v = reinterpret_cast<const VecT*>(w)[(uint64_t)tok * row_chunks + id % row_chunks];
  reinterpret_cast<VecT*>(out)[id] = v;
}

inline dim3 grid_for(uint64_t threads) { return dim3((unsigned)((threads + kThreads - 1) / kThreads)); }

inline bool a16(const void* p) { return (reinterpret_cast<uintptr_t>(p) & 15) == 0; }

template <typename T, EwFnK F>
hipError_t binary_t(const void* a, const void* b, void* out, uint64_t n, hipStream_t s) {
  constexpr int V = 16 / (int)sizeof(T);
  if (a16(a) && a16(b) && a16(out))
    binary_kernel<T, F, true><<<grid_for((n + V - 1) / V), kThreads, 0, s>>>((const T*)a, (const T*)b, (T*)out, n);
  else
    binary_kernel<T, F, false><<<grid_for(n), kThreads, 0, s>>>((const T*)a, (const T*)b, (T*)out, n);
  return hipGetLastError();
}

template <typename T, EwFnK F>
hipError_t unary_t(const void* in, void* out, uint64_t n, hipStream_t s) {
  constexpr int V = 16 / (int)sizeof(T);
  if (a16(in) && a16(out))
    unary_kernel<T, F, true><<<grid_for((n + V - 1) / V), kThreads, 0, s>>>((const T*)in, (T*)out, n);
  else
    unary_kernel<T, F, false><<<grid_for(n), kThreads, 0, s>>>((const T*)in, (T*)out, n);
  return hipGetLastError();
}

// ---- MoE (metal_provider.mm:1907-1997) ----------------------------------------
// Gating: one thread per token, the reference's sequence of operations: max
// over all n_experts logits, p_i = exp(l_i - max) summed in index order over
// the first min(n_experts, 64), p_i / sum, then an insertion into the top_k
// (<= 8) list with a strict '>' (earlier experts win ties, zero or NaN
// probabilities are never selected), renormalized by the selected sum.  p_i
// is recomputed instead of stored: the same expf of the same argument.  The
// list lives in registers: every index below is a compile-time constant.
__global__ __launch_bounds__(256) void moe_gate_kernel(const float* __restrict__ logits,
                                                       int32_t* __restrict__ ids, float* __restrict__ wts,
                                                       uint32_t batch, uint32_t n, uint32_t top_k) {
  const uint32_t b = blockIdx.x * blockDim.x + threadIdx.x;
  if (b >= batch) return;
  const float* l = logits + (size_t)b * n;
  const uint32_t ne = n < 64 ? n : 64;
  float mx = n ? l[0] : 0.f;
  for (uint32_t i = 1; i < n; ++i) mx = l[i] > mx ? l[i] : mx;
  float sum = 0.f;
  for (uint32_t i = 0; i < ne; ++i) sum = __fadd_rn(sum, expf(l[i] - mx));
  int32_t sid[8];
  float sp[8];
#pragma unroll
  for (int k = 0; k < 8; ++k) {
    sid[k] = -1;
    sp[k] = 0.f;
  }
  for (uint32_t i = 0; i < ne; ++i) {
    const float p = __fdiv_rn(expf(l[i] - mx), sum);
    int pos = (int)top_k;  // first slot p beats, or none
#pragma unroll
    for (int k = 7; k >= 0; --k)
      if (k < (int)top_k && p > sp[k]) pos = k;
    // pos is the FIRST slot whose value p exceeds: the list is kept in
    // descending order, so every slot after it is exceeded too.
#pragma unroll
    for (int k = 7; k >= 1; --k) {
      const bool shift = k > pos, here = k == pos;
      sp[k] = shift ? sp[k - 1] : (here ? p : sp[k]);
      sid[k] = shift ? sid[k - 1] : (here ? (int32_t)i : sid[k]);
    }
    if (pos == 0) {
      sp[0] = p;
      sid[0] = (int32_t)i;
    }
  }
  float ssum = 0.f;
#pragma unroll
  for (int k = 0; k < 8; ++k)
    if (k < (int)top_k) ssum = __fadd_rn(ssum, sp[k]);
#pragma unroll
  for (int k = 0; k < 8; ++k)
    if (k < (int)top_k) {
      ids[(size_t)b * top_k + k] = sid[k];
      wts[(size_t)b * top_k + k] = ssum > 0.f ? __fdiv_rn(sp[k], ssum) : 0.f;
    }
}

// Scatter-gather: out[b, d] = sum_k w[b, k] * E[ids[b, k], d] in k order,
// unfused multiply then add; ids < 0 (unfilled slots) and ids past the rows
// of E present are skipped.  Threads run along d, so each selected expert
// row is read with coalesced loads.
__global__ __launch_bounds__(256) void moe_scatter_kernel(const float* __restrict__ E, uint32_t rows,
                                                          const int32_t* __restrict__ ids,
                                                          const float* __restrict__ w, float* __restrict__ out,
                                                          uint32_t batch, uint32_t top_k, uint32_t dim) {
  // a rounded multiply, then a rounded add: never fused into one FMA
#pragma clang fp contract(off)
  const uint32_t d = blockIdx.x * blockDim.x + threadIdx.x;
  if (d >= dim) return;
  for (uint32_t b = blockIdx.y; b < batch; b += gridDim.y) {
    float v = 0.f;
    for (uint32_t k = 0; k < top_k; ++k) {
      const int32_t e = ids[(size_t)b * top_k + k];
      if (e < 0 || (uint32_t)e >= rows) continue;
      v += w[(size_t)b * top_k + k] * E[(size_t)e * dim + d];
    }
    out[(size_t)b * dim + d] = v;
  }
}

}  // namespace layer
}  // namespace nfk

namespace nfhip {

using nfk::EwFnK;
using nfk::half_t;


hipError_t launch_binary(EwFn fn, EType t, const void* a, const void* b, void* out, uint64_t n, hipStream_t s) {
  if (n == 0) return hipSuccess;
  using namespace nfk::layer;
  if (t == EType::F16)
    return fn == EwFn::Add ? binary_t<half_t, EwFnK::Add>(a, b, out, n, s) : binary_t<half_t, EwFnK::Mul>(a, b, out, n, s);
  return fn == EwFn::Add ? binary_t<float, EwFnK::Add>(a, b, out, n, s) : binary_t<float, EwFnK::Mul>(a, b, out, n, s);
}

hipError_t launch_unary(EwFn fn, EType t, const void* in, void* out, uint64_t n, hipStream_t s) {
  if (n == 0) return hipSuccess;
  using namespace nfk::layer;
  if (fn == EwFn::Relu) return unary_t<float, EwFnK::Relu>(in, out, n, s);
  if (t == EType::F16)
    return fn == EwFn::Silu ? unary_t<half_t, EwFnK::Silu>(in, out, n, s) : unary_t<half_t, EwFnK::Gelu>(in, out, n, s);
  return fn == EwFn::Silu ? unary_t<float, EwFnK::Silu>(in, out, n, s) : unary_t<float, EwFnK::Gelu>(in, out, n, s);
}

hipError_t launch_mock_prefill(const void* in, void* k, void* v, uint64_t nk, uint64_t nv, hipStream_t s) {
  const uint64_t n = nk > nv ? nk : nv;
  if (n == 0) return hipSuccess;
  nfk::layer::mock_prefill_kernel<<<nfk::layer::grid_for(n), nfk::layer::kThreads, 0, s>>>(
      (const float*)in, (float*)k, (float*)v, nk, nv);
  return hipGetLastError();
}

hipError_t launch_rms_norm(EType t, const void* in, const void* w, void* out, uint32_t rows, uint32_t dim, float eps,
                           hipStream_t s) {
  if (rows == 0) return hipSuccess;
  using namespace nfk::layer;
  // rows held in registers when they split into 16-byte chunks, at most 8
  // per thread (8192 f16 / 4096 f32 elements per 4 chunks, twice that for 8)
  const uint32_t vw = t == EType::F16 ? 8u : 4u;
  const bool aligned = ((reinterpret_cast<uintptr_t>(in) | reinterpret_cast<uintptr_t>(out)) % 16) == 0;
  const uint32_t chunks = (dim + kThreads * vw - 1) / (kThreads * vw);
  if (aligned && dim % vw == 0 && dim >= vw && chunks <= 8) {
    const int nc = chunks <= 1 ? 1 : chunks <= 2 ? 2 : chunks <= 4 ? 4 : 8;
#define NF_RMS_VEC(TT, NC)                                                                                      \
  rms_norm_vec_kernel<TT, NC><<<rows, kThreads, 0, s>>>((const TT*)in, (const float*)w, (TT*)out, dim, eps)
    if (t == EType::F16) {
      if (nc == 1) NF_RMS_VEC(half_t, 1); else if (nc == 2) NF_RMS_VEC(half_t, 2);
      else if (nc == 4) NF_RMS_VEC(half_t, 4); else NF_RMS_VEC(half_t, 8);
    } else {
      if (nc == 1) NF_RMS_VEC(float, 1); else if (nc == 2) NF_RMS_VEC(float, 2);
      else if (nc == 4) NF_RMS_VEC(float, 4); else NF_RMS_VEC(float, 8);
    }
#undef NF_RMS_VEC
    return hipGetLastError();
  }
  if (t == EType::F16)
    rms_norm_kernel<half_t><<<rows, kThreads, 0, s>>>((const half_t*)in, (const float*)w, (half_t*)out, dim, eps);
  else
    rms_norm_kernel<float><<<rows, kThreads, 0, s>>>((const float*)in, (const float*)w, (float*)out, dim, eps);
  return hipGetLastError();
}

hipError_t launch_rope(EType t, bool batch, const void* in, void* out, uint64_t n, uint32_t n_heads,
                       uint32_t head_dim, uint32_t step, float theta, hipStream_t s) {
  if (n == 0) return hipSuccess;
  using namespace nfk::layer;
  const uint64_t rows = n / head_dim;
  if (batch && n_heads == 0) return hipErrorInvalidValue;  // the planner rejects it first
  uint32_t per = kRopeRows;  // rows sharing one position and one rotation
  if (batch) {
    per = n_heads < kRopeRows ? n_heads : kRopeRows;
    while (n_heads % per) --per;
  }
  const uint64_t groups = (rows + per - 1) / per;
  const uint64_t threads = groups * (head_dim / 2);
  if (t == EType::F16)
    rope_kernel<half_t><<<grid_for(threads), kThreads, 0, s>>>((const half_t*)in, (half_t*)out, rows, head_dim, per,
                                                               n_heads, step, theta, batch);
  else
    rope_kernel<float><<<grid_for(threads), kThreads, 0, s>>>((const float*)in, (float*)out, rows, head_dim, per,
                                                              n_heads, step, theta, batch);
  return hipGetLastError();
}

// Rows wider than two chunks, with room for their partials in the
// workspace, take the chunked kernels.
static bool chunked(uint32_t rows, uint32_t dim, size_t ws_floats, uint32_t* chunks) {
  *chunks = (dim + nfk::layer::kChunk - 1) / nfk::layer::kChunk;
  return dim > 2 * nfk::layer::kChunk && (size_t)rows * *chunks * 2 <= ws_floats;
}

hipError_t launch_softmax(const void* in, void* out, uint32_t rows, uint32_t dim, float* ws, size_t ws_floats,
                          hipStream_t s) {
  if (rows == 0) return hipSuccess;
  using namespace nfk::layer;
  uint32_t chunks = 0;
  if (ws && chunked(rows, dim, ws_floats, &chunks)) {
    softmax_chunk_kernel<<<dim3(chunks, rows), kThreads, 0, s>>>((const float*)in, dim, chunks, ws);
    softmax_write_kernel<<<dim3(chunks, rows), kThreads, 0, s>>>((const float*)in, (float*)out, dim, chunks, ws);
    return hipGetLastError();
  }
  softmax_kernel<<<rows, kThreads, 0, s>>>((const float*)in, (float*)out, dim);
  return hipGetLastError();
}

hipError_t launch_argmax(const void* in, void* out, uint32_t rows, uint32_t dim, float* ws, size_t ws_floats,
                         hipStream_t s) {
  if (rows == 0) return hipSuccess;
  using namespace nfk::layer;
  uint32_t chunks = 0;
  if (ws && chunked(rows, dim, ws_floats, &chunks)) {
    argmax_chunk_kernel<<<dim3(chunks, rows), kThreads, 0, s>>>((const float*)in, dim, chunks, ws);
    argmax_merge_kernel<<<rows, 64, 0, s>>>((const float*)in, dim, chunks, ws, (int32_t*)out);
    return hipGetLastError();
  }
  argmax_kernel<<<rows, kThreads, 0, s>>>((const float*)in, (int32_t*)out, dim);
  return hipGetLastError();
}

hipError_t launch_embedding(EType t, const void* w, uint32_t vocab, const void* ids, void* out, uint64_t n,
                            uint32_t dim, uint32_t seq_len, hipStream_t s) {
  if (n == 0) return hipSuccess;
  using namespace nfk::layer;
  const uint32_t vw = t == EType::F16 ? 8u : 4u;
  if (dim % vw == 0 && n % vw == 0 && a16(w) && a16(out)) {
    const uint64_t nc = n / vw;
    if (t == EType::F16)
      embedding_vec_kernel<half_t><<<grid_for(nc), kThreads, 0, s>>>((const half_t*)w, vocab, (const int32_t*)ids,
                                                                      (half_t*)out, nc, dim / vw, seq_len);
    else
      embedding_vec_kernel<float><<<grid_for(nc), kThreads, 0, s>>>((const float*)w, vocab, (const int32_t*)ids,
                                                                     (float*)out, nc, dim / vw, seq_len);
    return hipGetLastError();
  }
  if (t == EType::F16)
    embedding_kernel<half_t><<<grid_for(n), kThreads, 0, s>>>((const half_t*)w, vocab, (const int32_t*)ids,
                                                              (half_t*)out, n, dim, seq_len);
  else
    embedding_kernel<float><<<grid_for(n), kThreads, 0, s>>>((const float*)w, vocab, (const int32_t*)ids,
                                                             (float*)out, n, dim, seq_len);
  return hipGetLastError();
}

hipError_t launch_moe_gate(const void* logits, void* ids, void* weights, uint32_t batch, uint32_t n_experts,
                           uint32_t top_k, hipStream_t s) {
  if (batch == 0 || top_k == 0) return hipSuccess;
  nfk::layer::moe_gate_kernel<<<(batch + 255) / 256, 256, 0, s>>>((const float*)logits, (int32_t*)ids,
                                                                    (float*)weights, batch, n_experts, top_k);
  return hipGetLastError();
}

hipError_t launch_moe_scatter(const void* experts, uint32_t expert_rows, const void* ids, const void* weights,
                              void* out, uint32_t batch, uint32_t top_k, uint32_t dim, hipStream_t s) {
  if (batch == 0 || dim == 0) return hipSuccess;
  const dim3 grid((dim + 255) / 256, batch < 65535u ? batch : 65535u);
  nfk::layer::moe_scatter_kernel<<<grid, 256, 0, s>>>((const float*)experts, expert_rows, (const int32_t*)ids,
                                                      (const float*)weights, (float*)out, batch, top_k, dim);
  return hipGetLastError();
}

}  // namespace nfhip
