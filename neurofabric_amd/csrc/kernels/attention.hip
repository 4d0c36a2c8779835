// attention.hip — causal softmax attention for every attention op the
// reference serves: causal_attention, causal_attention_cached,
// flash_attention_cached, flash_attention_gqa, flash_attention_paged
// (metal_provider.mm:166-498, 1273-1394, 1622-1906), f32 and f16.
//
// One kernel, parameterised by the KV addressing (AttnMode):
//   Plain   Q, K, V, out [n_heads, seq_len, head_dim]; keys 0..q
//   Cached  Q, out [seq_len, n_heads, head_dim], cache [n_kv, max_seq, head_dim];
//           keys kv_start..q (prefill) or kv_start..step (decode), with the
//           sliding window kv_start = pos - window + 1 when window > 0
//   Gqa     Q, out [n_heads, seq_len, head_dim] (decode: [n_heads, head_dim]),
//           same cache; keys 0..q / 0..step (no window)
//   Paged   Q, out [(K + seq) , n_heads, head_dim]; key p of KV head h lives at
//           pool[((table[p / bs] * n_kv + h) * bs + p % bs) * head_dim],
//           keys 0..min(q or step, n_blocks * bs - 1)
// Query head h reads KV head h * n_kv / n_heads.  The cached modes first
// append K_new / V_new to the cache in a separate kernel on the same stream,
// so every attention read sees the appended rows (the reference appends and
// reads in the same kernel without a barrier between threads).
//
// Workgroup = one (query token, head); its waves take 64-key tiles in turn.
// Per tile a lane scores one key (q from LDS, the key row with 16-byte
// loads), the wave keeps an online softmax (running max m, sum l), and the
// P·V product runs with lanes over head_dim: the tile's 64 weights are read
// out of lane registers one by one (uniform) while each lane streams its
// columns of the 64 value rows (coalesced).  The waves' (m, l, acc) merge in
// LDS at the end.  fp32 throughout; f16 variants convert on load and round
// the output once.  Mathematically the same softmax as each reference
// variant (two-pass, 32-key tiles, per-key online, per-block online); the
// results agree to fp32 rounding.
#include "../launch.hpp"
#include "common.hpp"

namespace nfk {
namespace attn {

constexpr int kMaxDim = 256;
constexpr int kTile = 64;

struct Params {
  const void* q;
  void* k;
  void* v;
  const uint32_t* table;
  void* out;
  uint32_t n_heads, n_kv, dim, seq_len, step, max_seq, window, block_size, n_blocks, q_offset;
  uint64_t pool_blocks;
  float scale;
  bool decode;
};

template <typename T>
__device__ __forceinline__ float f(T x) {
  return (float)x;
}

// Element offset of the query (and output) row of (query token qi, head h).
template <nfhip::AttnMode MODE>
__device__ __forceinline__ uint64_t q_row(const Params& p, uint32_t qi, uint32_t h) {
  const uint64_t D = p.dim;
  if constexpr (MODE == nfhip::AttnMode::Plain) return ((uint64_t)h * p.seq_len + qi) * D;
  if constexpr (MODE == nfhip::AttnMode::Cached) return p.decode ? (uint64_t)h * D : ((uint64_t)qi * p.n_heads + h) * D;
  if constexpr (MODE == nfhip::AttnMode::Gqa) return p.decode ? (uint64_t)h * D : ((uint64_t)h * p.seq_len + qi) * D;
  return ((uint64_t)(p.q_offset + qi) * p.n_heads + h) * D;  // Paged
}

// Element offset of key / value row `pos` of KV head kvh, or ~0 when the
// position has no row (paged: a physical block past the pools).
template <nfhip::AttnMode MODE>
__device__ __forceinline__ uint64_t kv_row(const Params& p, uint32_t kvh, uint32_t pos) {
  const uint64_t D = p.dim;
  if constexpr (MODE == nfhip::AttnMode::Plain) return ((uint64_t)kvh * p.seq_len + pos) * D;
  if constexpr (MODE == nfhip::AttnMode::Cached || MODE == nfhip::AttnMode::Gqa)
    return ((uint64_t)kvh * p.max_seq + pos) * D;
  const uint32_t phys = p.table[pos / p.block_size];
  if ((uint64_t)phys >= p.pool_blocks) return ~0ull;
  return (((uint64_t)phys * p.n_kv + kvh) * p.block_size + pos % p.block_size) * D;
}

template <typename T, nfhip::AttnMode MODE, int NW>
__global__ __launch_bounds__(NW * 64) void attention_kernel(Params p) {
  __shared__ float qs[kMaxDim];
  __shared__ float part_acc[NW][kMaxDim];
  __shared__ float part_m[NW], part_l[NW];

  const uint32_t qi = blockIdx.x;  // query token
  const uint32_t h = blockIdx.y;
  const uint32_t kvh = (uint32_t)((uint64_t)h * p.n_kv / p.n_heads);
  const uint32_t D = p.dim;
  const int lane = threadIdx.x & 63;
  const int wave = threadIdx.x >> 6;
  const T* Q = static_cast<const T*>(p.q);
  const T* K = static_cast<const T*>(p.k);
  const T* V = static_cast<const T*>(p.v);

  // Key range [lo, hi] of this query.
  const uint32_t pos = p.decode ? p.step : qi;
  uint32_t lo = 0, hi = pos;
  if constexpr (MODE == nfhip::AttnMode::Cached)
    if (p.window > 0 && pos >= p.window) lo = pos - p.window + 1;
  int64_t last = hi;
  if constexpr (MODE == nfhip::AttnMode::Paged) {
    const int64_t cap = (int64_t)p.n_blocks * p.block_size - 1;
    if (last > cap) last = cap;  // the block table covers fewer positions
  }

  const uint64_t qrow = q_row<MODE>(p, qi, h);
  for (uint32_t d = threadIdx.x; d < D; d += NW * 64) qs[d] = f(Q[qrow + d]);
  __syncthreads();

  constexpr int R = kMaxDim / 64;
  float acc[R];
#pragma unroll
  for (int r = 0; r < R; ++r) acc[r] = 0.0f;
  float m = -INFINITY, l = 0.0f;

  for (int64_t t0 = (int64_t)lo + (int64_t)wave * kTile; t0 <= last; t0 += (int64_t)NW * kTile) {
    // scores: lane -> key t0 + lane
    const int64_t kp = t0 + lane;
    uint64_t krow = ~0ull;
    if (kp <= last) krow = kv_row<MODE>(p, kvh, (uint32_t)kp);
    float s = -INFINITY;
    if (krow != ~0ull) {
      float dot = 0.0f;
      const T* kr = K + krow;
      uint32_t d = 0;
      if constexpr (sizeof(T) == 4) {
        if ((D & 3) == 0 && (reinterpret_cast<uintptr_t>(kr) & 15) == 0)
          for (; d + 4 <= D; d += 4) {
            const float4v x = *reinterpret_cast<const float4v*>(kr + d);
            dot += qs[d] * x[0];
            dot += qs[d + 1] * x[1];
            dot += qs[d + 2] * x[2];
            dot += qs[d + 3] * x[3];
          }
      } else {
        if ((D & 7) == 0 && (reinterpret_cast<uintptr_t>(kr) & 15) == 0)
          for (; d + 8 <= D; d += 8) {
            const half8 x = *reinterpret_cast<const half8*>(kr + d);
#pragma unroll
            for (int j = 0; j < 8; ++j) dot += qs[d + j] * (float)x[j];
          }
      }
      for (; d < D; ++d) dot += qs[d] * f(kr[d]);
      s = dot * p.scale;
    }
    float tmax = s;
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) tmax = fmaxf(tmax, __shfl_xor(tmax, o));
    if (tmax == -INFINITY) continue;  // no key of this tile has a row
    const float m_new = fmaxf(m, tmax);
    const float corr = expf(m - m_new);
    const float pw = s == -INFINITY ? 0.0f : expf(s - m_new);
    float psum = pw;
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) psum += __shfl_xor(psum, o);
    l = l * corr + psum;
    m = m_new;
#pragma unroll
    for (int r = 0; r < R; ++r) acc[r] *= corr;
    const int nk = (int)((last - t0 + 1) < kTile ? (last - t0 + 1) : kTile);
    for (int j = 0; j < nk; ++j) {
      const float pj = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(pw), j));
      if (pj == 0.0f) continue;  // uniform: masked key or underflow
      const uint64_t vrow = kv_row<MODE>(p, kvh, (uint32_t)(t0 + j));
      const T* vr = V + vrow;
#pragma unroll
      for (int r = 0; r < R; ++r) {
        const uint32_t d = lane + 64 * r;
        if (d < D) acc[r] += pj * f(vr[d]);
      }
    }
  }

  // merge the waves: out = sum_w acc_w e^(m_w - M) / sum_w l_w e^(m_w - M)
#pragma unroll
  for (int r = 0; r < R; ++r) {
    const uint32_t d = lane + 64 * r;
    if (d < D) part_acc[wave][d] = acc[r];
  }
  if (lane == 0) {
    part_m[wave] = m;
    part_l[wave] = l;
  }
  __syncthreads();
  float M = -INFINITY;
#pragma unroll
  for (int w = 0; w < NW; ++w) M = fmaxf(M, part_m[w]);
  float L = 0.0f;
  float wt[NW];
#pragma unroll
  for (int w = 0; w < NW; ++w) {
    wt[w] = part_m[w] == -INFINITY ? 0.0f : expf(part_m[w] - M);
    L += part_l[w] * wt[w];
  }
  const float inv = L > 0.0f ? 1.0f / L : 0.0f;
  T* O = static_cast<T*>(p.out);
  for (uint32_t d = threadIdx.x; d < D; d += NW * 64) {
    float o = 0.0f;
#pragma unroll
    for (int w = 0; w < NW; ++w) o += part_acc[w][d] * wt[w];
    O[qrow + d] = (T)(o * inv);
  }
}

// Append K_new / V_new rows to the caches: prefill rows 0..seq_len-1, decode
// row `step`.  Cached: K_new [tokens, n_kv, dim]; Gqa: [n_kv, tokens, dim].
template <typename T, bool HEAD_MAJOR>
__global__ __launch_bounds__(256) void append_kernel(const T* __restrict__ kn, const T* __restrict__ vn,
                                                     T* __restrict__ ck, T* __restrict__ cv, uint32_t n_kv,
                                                     uint32_t tokens, uint32_t dim, uint32_t max_seq,
                                                     uint32_t first_pos) {
  const uint64_t id = (uint64_t)blockIdx.x * 256 + threadIdx.x;
  const uint64_t n = (uint64_t)n_kv * tokens * dim;
  if (id >= n) return;
  const uint32_t d = (uint32_t)(id % dim);
  const uint64_t row = id / dim;  // (token, head) or (head, token) in the source order
  uint32_t tok, kvh;
  if (HEAD_MAJOR) {
    kvh = (uint32_t)(row / tokens);
    tok = (uint32_t)(row % tokens);
  } else {
    tok = (uint32_t)(row / n_kv);
    kvh = (uint32_t)(row % n_kv);
  }
  const uint64_t dst = ((uint64_t)kvh * max_seq + first_pos + tok) * dim + d;
  ck[dst] = kn[id];
  cv[dst] = vn[id];
}

template <typename T, nfhip::AttnMode MODE>
hipError_t run(const Params& p, uint32_t nq, hipStream_t s) {
  // decode: one query per head, so more waves per workgroup split the keys
  if (p.decode)
    attention_kernel<T, MODE, 16><<<dim3(nq, p.n_heads), 1024, 0, s>>>(p);
  else
    attention_kernel<T, MODE, 4><<<dim3(nq, p.n_heads), 256, 0, s>>>(p);
  return hipGetLastError();
}

template <typename T>
hipError_t launch_t(const nfhip::AttnArgs& a, hipStream_t s) {
  const nfhip::LayerParams& lp = a.lp;
  if (lp.noop) return hipSuccess;
  const uint32_t nq = lp.decode ? 1 : lp.seq_len;
  if (nq == 0) return hipSuccess;
  if (lp.append) {
    const uint32_t tokens = lp.decode ? 1 : lp.seq_len;
    const uint64_t n = (uint64_t)lp.n_kv * tokens * lp.head_dim;
    const dim3 grid((unsigned)((n + 255) / 256));
    const uint32_t first = lp.decode ? lp.step : 0;
    if (lp.attn == nfhip::AttnMode::Gqa)
      append_kernel<T, true><<<grid, 256, 0, s>>>((const T*)a.k_new, (const T*)a.v_new, (T*)a.k, (T*)a.v, lp.n_kv,
                                                  tokens, lp.head_dim, lp.max_seq, first);
    else
      append_kernel<T, false><<<grid, 256, 0, s>>>((const T*)a.k_new, (const T*)a.v_new, (T*)a.k, (T*)a.v, lp.n_kv,
                                                   tokens, lp.head_dim, lp.max_seq, first);
    hipError_t e = hipGetLastError();
    if (e != hipSuccess) return e;
  }
  Params p{};
  p.q = a.q;
  p.k = a.k;
  p.v = a.v;
  p.table = a.block_table;
  p.out = a.out;
  p.n_heads = lp.n_heads;
  p.n_kv = lp.n_kv;
  p.dim = lp.head_dim;
  p.seq_len = lp.seq_len;
  p.step = lp.step;
  p.max_seq = lp.max_seq;
  p.window = lp.window;
  p.block_size = lp.block_size;
  p.n_blocks = lp.n_blocks;
  p.q_offset = lp.q_offset;
  p.pool_blocks = a.pool_blocks;
  p.scale = 1.0f / sqrtf((float)lp.head_dim);
  p.decode = lp.decode;
  switch (lp.attn) {
    case nfhip::AttnMode::Plain: return run<T, nfhip::AttnMode::Plain>(p, nq, s);
    case nfhip::AttnMode::Cached: return run<T, nfhip::AttnMode::Cached>(p, nq, s);
    case nfhip::AttnMode::Gqa: return run<T, nfhip::AttnMode::Gqa>(p, nq, s);
    default: return run<T, nfhip::AttnMode::Paged>(p, nq, s);
  }
}

}  // namespace attn
}  // namespace nfk

namespace nfhip {

hipError_t launch_attention(EType t, const AttnArgs& a, hipStream_t s) {
  return t == EType::F16 ? nfk::attn::launch_t<nfk::half_t>(a, s) : nfk::attn::launch_t<float>(a, s);
}

}  // namespace nfhip
