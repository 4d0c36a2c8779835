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
#include <type_traits>

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
  // decode: the split kernel reads key / value row `step` from K_new / V_new
  // and the workgroup that owns it writes it into the cache
  const void* k_new;
  const void* v_new;
  bool fused_append;
};

template <typename T>
__device__ __forceinline__ float f(T x) {
  return (float)x;
}

// Element offset of the query (and output) row of (query token qi, head h).
template <nfhip::AttnMode MODE>
__host__ __device__ __forceinline__ uint64_t q_row(const Params& p, uint32_t qi, uint32_t h) {
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

// Workgroup -> (query head, query block) for the prefill kernels and the
// per-query kernel (grid x = query blocks, y = heads).  Workgroup L runs on XCD L % 8, and each XCD
// has its own L2: give each XCD the query blocks of whole KV heads, so its
// L2 holds those heads' K and V instead of every head's, with the heavy
// (late, most keys) blocks first.  Any other grid keeps the plain order.
__device__ __forceinline__ void prefill_block(const Params& p, uint32_t& h, uint32_t& qblk) {
  const uint32_t nqb = gridDim.x, total = nqb * gridDim.y, L = blockIdx.x + nqb * blockIdx.y;
  const uint32_t G = p.n_heads / p.n_kv;
  if (total % 8 == 0 && p.n_heads % p.n_kv == 0) {
    const uint32_t i = (L % 8) * (total / 8) + L / 8;  // a bijection of [0, total)
    const uint32_t kv_i = i / (G * nqb), rem = i % (G * nqb);
    h = kv_i * G + rem % G;
    qblk = nqb - 1 - rem / G;
  } else {
    h = blockIdx.y;
    qblk = nqb - 1 - blockIdx.x;
  }
}

constexpr int kBatch = 8;

// Columns lane + 64 r of value rows t0 + j0 .. t0 + j0 + kBatch - 1.  Every
// load is unconditional (a row past nk or without storage reads row 0, a
// column past dim reads column dim - 1, both in bounds) so the whole batch
// is in flight before the first use; ok[jj] marks the rows that count, and
// the caller discards the others with a select (not a multiply by 0, which
// would let a NaN in unused memory through).
template <typename T, nfhip::AttnMode MODE, int R>
__device__ __forceinline__ void load_v_batch(const Params& p, const T* V, uint32_t kvh, int64_t t0, int j0, int nk,
                                             int lane, T (&x)[kBatch][R], bool (&ok)[kBatch]) {
  const uint32_t D = p.dim;
#pragma unroll
  for (int jj = 0; jj < kBatch; ++jj) {
    const int j = j0 + jj;
    const uint64_t row = j < nk ? kv_row<MODE>(p, kvh, (uint32_t)(t0 + j)) : ~0ull;
    ok[jj] = row != ~0ull;
    const T* vr = V + (ok[jj] ? row : 0);
#pragma unroll
    for (int r = 0; r < R; ++r) {
      if (r * 64 >= (int)D) break;  // uniform
      const uint32_t d = lane + 64 * r;
      x[jj][r] = vr[d < D ? d : D - 1];
    }
  }
}

template <typename T, nfhip::AttnMode MODE, int NW>
__global__ __launch_bounds__(NW * 64) void attention_kernel(Params p) {
  __shared__ float qs[kMaxDim];
  __shared__ float ps[NW][kTile];  // each wave's tile weights
  __shared__ float part_acc[NW][kMaxDim];
  __shared__ float part_m[NW], part_l[NW];

  uint32_t qi, h;  // query token, head
  prefill_block(p, h, qi);
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
#pragma unroll 4
          for (; d + 4 <= D; d += 4) {
            const float4v x = *reinterpret_cast<const float4v*>(kr + d);
            dot += qs[d] * x[0];
            dot += qs[d + 1] * x[1];
            dot += qs[d + 2] * x[2];
            dot += qs[d + 3] * x[3];
          }
      } else {
        if ((D & 7) == 0 && (reinterpret_cast<uintptr_t>(kr) & 15) == 0)
#pragma unroll 4
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
    // value rows 8 at a time: the loads of a batch are all in flight before
    // its FMAs (a masked or missing row contributes 0)
    ps[wave][lane] = pw;  // read back by this wave only: LDS keeps a wave's accesses in order
    __builtin_amdgcn_wave_barrier();
    for (int j0 = 0; j0 < nk; j0 += kBatch) {
      T x[kBatch][R];
      bool ok[kBatch];
      load_v_batch<T, MODE, R>(p, V, kvh, t0, j0, nk, lane, x, ok);
#pragma unroll
      for (int jj = 0; jj < kBatch; ++jj) {
        if (!ok[jj]) continue;  // uniform
        const float pj = ps[wave][j0 + jj];
#pragma unroll
        for (int r = 0; r < R; ++r) {
          if (r * 64 >= (int)D) break;
          acc[r] += pj * f(x[jj][r]);
        }
      }
    }
    __builtin_amdgcn_wave_barrier();
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

// Prefill, many queries per workgroup: a workgroup takes kQB consecutive
// query tokens of one head, and every 64-key tile of K and V is staged once
// in LDS for all of them (f32; K transposed, Kt[d][key], so a lane scoring
// key `lane` reads consecutive words).  Each wave scores and accumulates
// kQW = 4 queries at once: per d, four K words feed 16 FMAs; per key, one
// broadcast float4 of weights feeds 4 x R FMAs.  The per-query arithmetic is
// the per-(query, head) kernel's online softmax over the same tiles.
// head_dim <= 128 and a multiple of 4; not for paged pools or decode.
constexpr int kQW = 4, kMqDim = 128;

template <typename T>
struct Vec4 {
  typedef T type __attribute__((ext_vector_type(4)));
};

template <typename T, nfhip::AttnMode MODE, int NW>
__global__ __launch_bounds__(NW * 64) void attention_mq_kernel(Params p) {
  constexpr int kQB = NW * kQW, kThreads = NW * 64;
  __shared__ float Kt[kMqDim * kTile];
  __shared__ float Vs[kTile * kMqDim];
  __shared__ float qs[kQB * kMqDim];
  __shared__ float4v ps[NW][kTile];

  typedef typename Vec4<T>::type T4;
  uint32_t h, qblk;
  prefill_block(p, h, qblk);
  const uint32_t kvh = (uint32_t)((uint64_t)h * p.n_kv / p.n_heads);
  const uint32_t D = p.dim, D4 = D / 4;
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const uint32_t q0 = qblk * kQB;
  const uint32_t q1 = q0 + kQB < p.seq_len ? q0 + kQB : p.seq_len;
  const T* Q = static_cast<const T*>(p.q);
  const T* K = static_cast<const T*>(p.k);
  const T* V = static_cast<const T*>(p.v);

  auto lo_of = [&](uint32_t pos) -> uint32_t {
    if constexpr (MODE == nfhip::AttnMode::Cached)
      if (p.window > 0 && pos >= p.window) return pos - p.window + 1;
    return 0u;
  };
  const uint32_t lo_blk = lo_of(q0), hi_blk = q1 - 1;

  for (uint32_t i = tid; i < kQB * D4; i += kThreads) {
    const uint32_t qq = i / D4, c = i % D4;
    float4v v = {0.f, 0.f, 0.f, 0.f};
    if (q0 + qq < q1) {
      const T4 x = *reinterpret_cast<const T4*>(Q + q_row<MODE>(p, q0 + qq, h) + 4 * c);
      v = float4v{f(x[0]), f(x[1]), f(x[2]), f(x[3])};
    }
    *reinterpret_cast<float4v*>(&qs[qq * kMqDim + 4 * c]) = v;
  }

  constexpr int R = kMqDim / 64;
  float acc[kQW][R], m[kQW], l[kQW];
  uint32_t qpos[kQW], qlo[kQW];
  bool qok[kQW];
#pragma unroll
  for (int i = 0; i < kQW; ++i) {
    qpos[i] = q0 + wave * kQW + i;
    qok[i] = qpos[i] < q1;
    qlo[i] = lo_of(qpos[i]);
    m[i] = -INFINITY;
    l[i] = 0.f;
#pragma unroll
    for (int r = 0; r < R; ++r) acc[i][r] = 0.f;
  }

  // The next tile's K and V are loaded into registers while the current
  // one is computed.  Every load is unconditional: a key past the block's
  // last query reads that query's row and a chunk past the row reads its
  // last chunk (both in bounds); stage() writes zeros for them instead.
  constexpr int kLd = kTile * (kMqDim / 4) / kThreads;
  T4 kr[kLd], vr[kLd];
  auto fetch = [&](int64_t t0) {
#pragma unroll
    for (int u = 0; u < kLd; ++u) {
      const uint32_t i = tid + kThreads * u;
      const uint32_t kkey = i & (kTile - 1), kc = i / kTile < D4 ? i / kTile : D4 - 1;
      const int64_t kt = t0 + kkey <= (int64_t)hi_blk ? t0 + kkey : (int64_t)hi_blk;
      kr[u] = *reinterpret_cast<const T4*>(K + kv_row<MODE>(p, kvh, (uint32_t)kt) + 4 * kc);
      const uint32_t vkey = i / D4 < (uint32_t)kTile ? i / D4 : kTile - 1, vc = i % D4;
      const int64_t vt = t0 + vkey <= (int64_t)hi_blk ? t0 + vkey : (int64_t)hi_blk;
      vr[u] = *reinterpret_cast<const T4*>(V + kv_row<MODE>(p, kvh, (uint32_t)vt) + 4 * vc);
    }
  };
  auto stage = [&](int64_t t0) {
#pragma unroll
    for (int u = 0; u < kLd; ++u) {
      const uint32_t i = tid + kThreads * u;
      if (i >= kTile * D4) break;  // uniform per unrolled step only at the tail
      const uint32_t kkey = i & (kTile - 1), kc = i / kTile;
      const bool kin = t0 + kkey <= (int64_t)hi_blk;
#pragma unroll
      for (int j = 0; j < 4; ++j) Kt[(4 * kc + j) * kTile + kkey] = kin ? f(kr[u][j]) : 0.f;
      const uint32_t vkey = i / D4, vc = i % D4;
      const bool vin = t0 + vkey <= (int64_t)hi_blk;
      *reinterpret_cast<float4v*>(&Vs[vkey * kMqDim + 4 * vc]) =
          vin ? float4v{f(vr[u][0]), f(vr[u][1]), f(vr[u][2]), f(vr[u][3])} : float4v{0.f, 0.f, 0.f, 0.f};
    }
  };

  fetch(lo_blk);
  for (int64_t t0 = lo_blk; t0 <= (int64_t)hi_blk; t0 += kTile) {
    __syncthreads();  // the previous tile's readers are done
    stage(t0);
    __syncthreads();
    if (t0 + kTile <= (int64_t)hi_blk) fetch(t0 + kTile);

    // scores of key t0 + lane for the wave's queries
    float s[kQW];
#pragma unroll
    for (int i = 0; i < kQW; ++i) s[i] = 0.f;
    const float* qw = &qs[wave * kQW * kMqDim];
    for (uint32_t d = 0; d < D; d += 4) {
      const float k0 = Kt[d * kTile + lane], k1 = Kt[(d + 1) * kTile + lane];
      const float k2 = Kt[(d + 2) * kTile + lane], k3 = Kt[(d + 3) * kTile + lane];
#pragma unroll
      for (int i = 0; i < kQW; ++i) {
        const float4v qv = *reinterpret_cast<const float4v*>(&qw[i * kMqDim + d]);
        s[i] += qv[0] * k0;
        s[i] += qv[1] * k1;
        s[i] += qv[2] * k2;
        s[i] += qv[3] * k3;
      }
    }
    const int64_t t = t0 + lane;
    float pw[kQW];
#pragma unroll
    for (int i = 0; i < kQW; ++i) {
      const bool in = qok[i] && t >= (int64_t)qlo[i] && t <= (int64_t)qpos[i];
      const float si = in ? s[i] * p.scale : -INFINITY;
      float tmax = si;
#pragma unroll
      for (int o = 32; o > 0; o >>= 1) tmax = fmaxf(tmax, __shfl_xor(tmax, o));
      if (tmax == -INFINITY) {  // no key of this tile for query i (uniform)
        pw[i] = 0.f;
        continue;
      }
      const float m_new = fmaxf(m[i], tmax);
      const float corr = expf(m[i] - m_new);
      pw[i] = in ? expf(si - m_new) : 0.f;
      float psum = pw[i];
#pragma unroll
      for (int o = 32; o > 0; o >>= 1) psum += __shfl_xor(psum, o);
      l[i] = l[i] * corr + psum;
      m[i] = m_new;
#pragma unroll
      for (int r = 0; r < R; ++r) acc[i][r] *= corr;
    }
    ps[wave][lane] = float4v{pw[0], pw[1], pw[2], pw[3]};
    __builtin_amdgcn_wave_barrier();
    // Keys past the wave's last query are no query's.  A key outside some
    // query's range (a later token, or before its window) must not touch
    // that query's sum at all, as in the per-query kernel, which never reads
    // such a value row: a non-finite value times the weight 0 would be NaN.
    // Tiles whose keys all lie inside every live query's range (all but the
    // tiles at the diagonal and at a window edge) take the plain FMA loop;
    // the others test each key against each query (the test is uniform over
    // the wave).
    const int64_t wlast = (int64_t)(qok[kQW - 1] ? qpos[kQW - 1] : hi_blk);
    const int nk = (int)((wlast - t0 + 1) < kTile ? (wlast - t0 + 1) : kTile);
    bool interior = true;
#pragma unroll
    for (int i = 0; i < kQW; ++i)
      interior = interior && (!qok[i] || (t0 >= (int64_t)qlo[i] && t0 + nk - 1 <= (int64_t)qpos[i]));
    if (interior) {
      for (int j = 0; j < nk; ++j) {
        const float4v pj = ps[wave][j];
#pragma unroll
        for (int r = 0; r < R; ++r) {
          const float v = Vs[j * kMqDim + lane + 64 * r];
#pragma unroll
          for (int i = 0; i < kQW; ++i) acc[i][r] += pj[i] * v;
        }
      }
    } else {
      for (int j = 0; j < nk; ++j) {
        const float4v pj = ps[wave][j];
        const int64_t tj = t0 + j;
#pragma unroll
        for (int r = 0; r < R; ++r) {
          const float v = Vs[j * kMqDim + lane + 64 * r];
#pragma unroll
          for (int i = 0; i < kQW; ++i)
            if (qok[i] && tj >= (int64_t)qlo[i] && tj <= (int64_t)qpos[i]) acc[i][r] += pj[i] * v;
        }
      }
    }
    __builtin_amdgcn_wave_barrier();
  }

  T* O = static_cast<T*>(p.out);
#pragma unroll
  for (int i = 0; i < kQW; ++i) {
    if (!qok[i]) continue;
    const float inv = l[i] > 0.f ? 1.0f / l[i] : 0.f;
    const uint64_t orow = q_row<MODE>(p, qpos[i], h);
#pragma unroll
    for (int r = 0; r < R; ++r) {
      const uint32_t d = lane + 64 * r;
      if (d < D) O[orow + d] = (T)(acc[i][r] * inv);
    }
  }
}

// Sum / max over the 4 lanes of an MFMA output column (lanes n, n + 16,
// n + 32, n + 48).  v_permlane16_swap / v_permlane32_swap exchange rows
// between their two registers, so with both holding v each lane ends with
// its own value and its partner's (lane ^ 16, then lane ^ 32) in the pair.
// Inline asm: the compiler's builtins for these instructions lose the second
// result; the s_nop gives the two wait states a VALU write needs before a
// permlane reads it.
template <bool ROW32>
__device__ __forceinline__ float2s lane_swap_pair(float v) {
  float a = v, b = v;
  if constexpr (ROW32)
    asm("s_nop 1\n\tv_permlane32_swap_b32 %0, %1" : "+v"(a), "+v"(b));
  else
    asm("s_nop 1\n\tv_permlane16_swap_b32 %0, %1" : "+v"(a), "+v"(b));
  return float2s{a, b};
}
__device__ __forceinline__ float col_max(float v) {
  float2s r = lane_swap_pair<false>(v);
  r = lane_swap_pair<true>(fmaxf(r[0], r[1]));
  return fmaxf(r[0], r[1]);
}
__device__ __forceinline__ float col_sum(float v) {
  float2s r = lane_swap_pair<false>(v);
  r = lane_swap_pair<true>(r[0] + r[1]);
  return r[0] + r[1];
}

// Prefill on MFMA (f16, head_dim DD = 64 or 128; not paged): flash attention
// with the matrices transposed so that every operand comes out of registers
// or LDS in the layout the next MFMA wants.  A workgroup takes 64 query
// tokens of one head, 16 per wave; per 64-key tile of K and V (staged once
// in LDS for the workgroup, both row-major):
//  * S^T[key][query] = K[key][dims] . Q^T[dims][query] on
//    v_mfma_f32_16x16x32_f16: A = 16 key rows from LDS, B = the wave's 16
//    queries (held in registers for the whole kernel);
//  * online softmax in base 2 per query (a query's 64 scores are spread over
//    the 4 lane groups of its column); the weights carry a factor 2^7
//    (folded into the exponent), which keeps the f16 pieces below out of the
//    subnormal range and is divided out with the sum at the end, and the
//    reference max is rescaled lazily (only when a score passes it by 2^8);
//  * O^T[dim][query] += V^T[dim][key] . P^T[key][query]: the softmax weights
//    of S^T's output layout are the B operand as they are (in a fixed key
//    order), each split into two f16 pieces (two MFMAs, so the products keep
//    fp32-level accuracy); the A operand is two transposing 8-byte LDS
//    reads (ds_read_b64_tr_b16) of the row-major V tile; fp32 accumulation.
// Masked scores are -inf by select.  A weight of 0 times a non-finite value
// would still be NaN inside the MFMA, so a tile that holds a non-finite
// value and a key outside some query's range (the diagonal and window-edge
// tiles) takes the vector-ALU P.V, which skips such (key, query) pairs as
// the per-query kernel does.  Tiles inside every query's range (all but the
// last one or two of a workgroup) skip the masking, the zeroing of rows past
// the range and the non-finite check: the vector-ALU work per tile is then
// about what the 48 MFMAs take.
// Workgroup order: prefill_block (2048 tokens x 32 heads x 128: 240 -> 147
// us from the L2 locality alone).
constexpr float kPLog2Scale = 7.f;  // softmax weights carry 2^7 on the f16 MFMA path
constexpr float kLazyLog2 = 8.f;    // the reference max may lag the running max by 2^8

template <nfhip::AttnMode MODE, int DD>
__global__ __launch_bounds__(256, 2) void prefill_mfma_kernel(Params p) {
  static_assert(MODE != nfhip::AttnMode::Paged, "rows of a KV head must be contiguous in position");
  typedef half_t T;
  constexpr int KSTEP = DD / 32, CPR = DD / 8, DB = DD / 16;
  constexpr int KP = DD + 8;               // padded LDS row length (halves), K and V
  constexpr int NL = 64 * CPR / 256;       // 16-byte K and V chunks per thread and tile
  __shared__ __attribute__((aligned(16))) T Ks[64 * KP];
  __shared__ __attribute__((aligned(16))) T Vs[64 * KP];
  __shared__ __attribute__((aligned(16))) float ps[4][64][16];  // weights for the vector-ALU P.V
  __shared__ int tile_bad[2];  // per tile parity: the staged V holds a non-finite value
  const uint32_t S = p.seq_len;
  uint32_t h, qblk;
  prefill_block(p, h, qblk);
  const uint32_t kvh = (uint32_t)((uint64_t)h * p.n_kv / p.n_heads);
  const int tid = threadIdx.x, lane = tid & 63;
  const int w = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int n = lane & 15, g = lane >> 4;
  const uint32_t q0 = qblk * 64;
  const uint32_t q1 = q0 + 64 < S ? q0 + 64 : S;
  const T* Q = static_cast<const T*>(p.q);
  // rows of this KV head: position pos at Kh + pos * DD
  const T* Kh = static_cast<const T*>(p.k) + kv_row<MODE>(p, kvh, 0);
  const T* Vh = static_cast<const T*>(p.v) + kv_row<MODE>(p, kvh, 0);
  auto lo_of = [&](uint32_t pos) -> uint32_t {
    if constexpr (MODE == nfhip::AttnMode::Cached)
      if (p.window > 0 && pos >= p.window) return pos - p.window + 1;
    return 0u;
  };
  const uint32_t lo_blk = lo_of(q0), hi_blk = q1 - 1;
  const uint32_t lo_last = lo_of(hi_blk);

  // this lane's query (MFMA column n of the wave's 16)
  const uint32_t qw0 = q0 + 16 * w;
  const uint32_t qpos = qw0 + n;
  const bool qok = qpos < q1;
  const uint32_t qlo = lo_of(qpos);
  half8 qb[KSTEP];
#pragma unroll
  for (int st = 0; st < KSTEP; ++st) {
    qb[st] = *reinterpret_cast<const half8*>(Q + q_row<MODE>(p, qok ? qpos : q0, h) + 32 * st + 8 * g);
    if (!qok) qb[st] = half8{};
  }
  // the wave's query range (for the tiles it can skip or take unmasked)
  const uint32_t wq_last = qw0 + 15 < q1 ? qw0 + 15 : q1 - 1;
  const bool wave_live = qw0 < q1;
  const uint32_t wlo_last = lo_of(wq_last);

  float4v ot[DB];
#pragma unroll
  for (int b = 0; b < DB; ++b) ot[b] = float4v{0.f, 0.f, 0.f, 0.f};
  float m_run = -INFINITY, l_run = 0.f;
  const float sl2 = p.scale * 1.44269504088896341f;

  // Tile loads into registers (next tile while this one computes): chunk
  // i = tid + 256u of K and of V is row i / CPR, 16-byte chunk i % CPR
  // (coalesced), staged row-major in LDS.  In the last tile, rows past the
  // block's last query read that query's row (in bounds) and are masked (K)
  // or zeroed (V) when staged.
  half8 kr[NL], vr[NL];
  auto fetch = [&](int64_t t0) {
    if (t0 + 63 <= (int64_t)hi_blk) {  // uniform: the whole tile is in range
      const T* kt = Kh + (uint64_t)t0 * DD;
      const T* vt = Vh + (uint64_t)t0 * DD;
#pragma unroll
      for (int u = 0; u < NL; ++u) {
        const int i = tid + 256 * u;
        kr[u] = *reinterpret_cast<const half8*>(kt + (i / CPR) * DD + 8 * (i % CPR));
        vr[u] = *reinterpret_cast<const half8*>(vt + (i / CPR) * DD + 8 * (i % CPR));
      }
    } else {
#pragma unroll
      for (int u = 0; u < NL; ++u) {
        const int i = tid + 256 * u;
        const int64_t row = t0 + i / CPR <= (int64_t)hi_blk ? t0 + i / CPR : (int64_t)hi_blk;
        kr[u] = *reinterpret_cast<const half8*>(Kh + (uint64_t)row * DD + 8 * (i % CPR));
        vr[u] = *reinterpret_cast<const half8*>(Vh + (uint64_t)row * DD + 8 * (i % CPR));
      }
    }
  };
  auto stage_k = [&]() {
#pragma unroll
    for (int u = 0; u < NL; ++u) {
      const int i = tid + 256 * u;
      *reinterpret_cast<half8*>(&Ks[(i / CPR) * KP + 8 * (i % CPR)]) = kr[u];
    }
  };
  auto stage_v = [&]() {
#pragma unroll
    for (int u = 0; u < NL; ++u) {
      const int i = tid + 256 * u;
      *reinterpret_cast<half8*>(&Vs[(i / CPR) * KP + 8 * (i % CPR)]) = vr[u];
    }
  };
  // rows past the range as zeros; a non-finite value marks the tile
  auto stage_v_checked = [&](int64_t t0, int par) {
    bool bad = false;
#pragma unroll
    for (int u = 0; u < NL; ++u) {
      const int i = tid + 256 * u;
      half8 x = vr[u];
      if (t0 + i / CPR > (int64_t)hi_blk) x = half8{};
#pragma unroll
      for (int e = 0; e < 8; ++e) bad = bad || !__builtin_isfinite((float)x[e]);
      *reinterpret_cast<half8*>(&Vs[(i / CPR) * KP + 8 * (i % CPR)]) = x;
    }
    if (bad) tile_bad[par] = 1;
  };
  // The P.V A operand, V^T[dim][key], from the row-major tile with
  // ds_read_b64_tr_b16: among each 16 lanes, lane i receives element
  // i % 4 of the 8 bytes that lane 4e + i / 4 addressed, as its element e.
  // Lane n (of lane group g) addresses key row 4g + n / 4 (+ the k-step's
  // base) at dims 16b + 4 (n % 4) .. + 3, so lane n receives dim 16b + n of
  // keys 4g .. 4g + 3: one half of the A piece (the other half is the keys
  // 16 further on).
  const T* const vtr = &Vs[(4 * g + n / 4) * KP + 4 * (n % 4)];
  auto v_tr = [&](int key0, int dim0) {
    typedef short short4v __attribute__((ext_vector_type(4)));
    return __builtin_bit_cast(uint2, __builtin_amdgcn_ds_read_tr16_b64_v4i16(
                                         (__attribute__((address_space(3))) short4v*)(vtr + key0 * KP + dim0)));
  };

  // One staged tile for this wave.  INTERIOR: every key in every query's
  // range (no masking; P.V always on MFMA).
  auto tile = [&](int64_t t0, int par, auto interior_c) {
    constexpr bool INTERIOR = decltype(interior_c)::value;
    // scores S^T: lane holds keys t0 + 16j + 4g + i for query qpos; the
    // operand reads of half the head_dim first, then the 4 independent
    // accumulation chains
    float4v sc[4];
#pragma unroll
    for (int j = 0; j < 4; ++j) sc[j] = float4v{0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int h2 = 0; h2 < (KSTEP + 1) / 2; ++h2) {
      constexpr int NS = KSTEP < 2 ? KSTEP : 2;
      half8 a[NS][4];
#pragma unroll
      for (int st = 0; st < NS; ++st)
#pragma unroll
        for (int j = 0; j < 4; ++j)
          a[st][j] = *reinterpret_cast<const half8*>(&Ks[(16 * j + n) * KP + 32 * (NS * h2 + st) + 8 * g]);
#pragma unroll
      for (int st = 0; st < NS; ++st)
#pragma unroll
        for (int j = 0; j < 4; ++j)
          sc[j] = __builtin_amdgcn_mfma_f32_16x16x32_f16(a[st][j], qb[NS * h2 + st], sc[j], 0, 0, 0);
      __builtin_amdgcn_sched_barrier(0);  // bounds the operand registers in flight
    }
    // base-2 scores (the scale folded into the exponent's fma); the max of
    // the raw scores times the positive scale is the max of the scaled ones
    float sr[4][4];
    float rmax = -INFINITY;
#pragma unroll
    for (int j = 0; j < 4; ++j)
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        if constexpr (INTERIOR) {
          sr[j][i] = sc[j][i];
        } else {
          const int64_t kt = t0 + 16 * j + 4 * g + i;
          const bool in = qok && kt >= (int64_t)qlo && kt <= (int64_t)qpos;
          sr[j][i] = in ? sc[j][i] : -INFINITY;
        }
        rmax = fmaxf(rmax, sr[j][i]);
      }
    rmax = col_max(rmax);
    // Lazy rescale: the reference max m_run moves (and the sum and the
    // accumulators are rescaled) only when a score of the wave exceeds it by
    // more than kLazyLog2; the weights then stay below 2^(kLazyLog2 +
    // kPLog2Scale) = 2^15, within f16 range.
    const float tmax = rmax * sl2;
    if (__builtin_amdgcn_ballot_w64(tmax > m_run + kLazyLog2) != 0) {  // uniform
      const float m_new = fmaxf(m_run, tmax);
      const float corr = m_new == -INFINITY ? 1.f : __builtin_amdgcn_exp2f(m_run - m_new);
      l_run *= corr;
#pragma unroll
      for (int b = 0; b < DB; ++b) ot[b] *= corr;
      m_run = m_new;
    }
    const float mb = m_run - kPLog2Scale;
    float pv[4][4];
    float psum = 0.f;
#pragma unroll
    for (int j = 0; j < 4; ++j)
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const float e = __builtin_amdgcn_exp2f(__builtin_fmaf(sr[j][i], sl2, -mb));
        if constexpr (INTERIOR) {
          pv[j][i] = e;
        } else {
          // a masked score is -inf: exp2 gives 0 unless the whole column is
          // masked so far (m_run = -inf, a NaN argument)
          pv[j][i] = sr[j][i] == -INFINITY ? 0.f : e;
        }
        psum += pv[j][i];
      }
    l_run += col_sum(psum);
    // P.V: unmasked for the wave, or no non-finite value: on MFMA
    if (INTERIOR || !tile_bad[par]) {
#pragma unroll
      for (int c = 0; c < 2; ++c) {
        __builtin_amdgcn_sched_barrier(0);  // bounds the operand registers in flight
        half8 av[DB];
#pragma unroll
        for (int b = 0; b < DB; ++b) {
          const uint2 lo4 = v_tr(32 * c, 16 * b);
          const uint2 hi4 = v_tr(32 * c + 16, 16 * b);
          av[b] = __builtin_bit_cast(half8, u32x4{lo4.x, lo4.y, hi4.x, hi4.y});
        }
        // each weight as two f16 pieces, hi (rounded toward zero) + lo (the
        // remainder, exact in fp32, rounded toward zero), within 2^-20 of it
        uint32_t wh[4], wl[4];
#pragma unroll
        for (int k = 0; k < 4; ++k) {
          const float a0 = pv[2 * c + (k >> 1)][2 * (k & 1)], a1 = pv[2 * c + (k >> 1)][2 * (k & 1) + 1];
          const half2v hh = __builtin_bit_cast(half2v, __builtin_amdgcn_cvt_pkrtz(a0, a1));
          const half2v ll = __builtin_bit_cast(
              half2v, __builtin_amdgcn_cvt_pkrtz(__builtin_fmaf((float)hh[0], -1.f, a0), __builtin_fmaf((float)hh[1], -1.f, a1)));
          wh[k] = __builtin_bit_cast(uint32_t, hh);
          wl[k] = __builtin_bit_cast(uint32_t, ll);
        }
        const half8 bh = __builtin_bit_cast(half8, u32x4{wh[0], wh[1], wh[2], wh[3]});
        const half8 bl = __builtin_bit_cast(half8, u32x4{wl[0], wl[1], wl[2], wl[3]});
#pragma unroll
        for (int b = 0; b < DB; ++b) ot[b] = __builtin_amdgcn_mfma_f32_16x16x32_f16(av[b], bh, ot[b], 0, 0, 0);
#pragma unroll
        for (int b = 0; b < DB; ++b) ot[b] = __builtin_amdgcn_mfma_f32_16x16x32_f16(av[b], bl, ot[b], 0, 0, 0);
      }
    } else {
      // predicated vector-ALU P.V: key kt enters query qpos only in range
#pragma unroll
      for (int j = 0; j < 4; ++j)
#pragma unroll
        for (int i = 0; i < 4; ++i) ps[w][16 * j + 4 * g + i][n] = pv[j][i];
      __builtin_amdgcn_wave_barrier();
      __builtin_amdgcn_fence(__ATOMIC_ACQ_REL, "wavefront");
      for (int k = 0; k < 64; ++k) {
        const int64_t kt = t0 + k;
        if (!(qok && kt >= (int64_t)qlo && kt <= (int64_t)qpos)) continue;
        const float pk = ps[w][k][n];
#pragma unroll
        for (int b = 0; b < DB; ++b)
#pragma unroll
          for (int i = 0; i < 4; ++i) ot[b][i] += pk * (float)Vs[k * KP + 16 * b + 4 * g + i];
      }
      __builtin_amdgcn_wave_barrier();
    }
  };

  if (tid == 0) tile_bad[0] = tile_bad[1] = 0;
  fetch(lo_blk);
  int par = 0;
  for (int64_t t0 = lo_blk; t0 <= (int64_t)hi_blk; t0 += 64, par ^= 1) {
    __syncthreads();  // the previous tile's readers are done
    // the other parity's flag was last read before this barrier and is next
    // set after the following tile's first barrier
    if (tid == 0) tile_bad[par ^ 1] = 0;
    stage_k();
    // every key of the tile in every query's range: no zeroing, no check
    // (each wave then takes the MFMA P.V)
    if (t0 + 63 <= (int64_t)q0 && t0 >= (int64_t)lo_last) stage_v();
    else stage_v_checked(t0, par);
    __syncthreads();
    if (t0 + 64 <= (int64_t)hi_blk) fetch(t0 + 64);
    if (!wave_live || t0 > (int64_t)wq_last) continue;  // no key of this tile for the wave (uniform)
    // every key of the tile in every query's range of the wave (uniform):
    // the tile body without masking, else with it
    if (t0 + 63 <= (int64_t)qw0 && t0 >= (int64_t)wlo_last) tile(t0, par, std::true_type{});
    else tile(t0, par, std::false_type{});
  }

  if (qok) {
    const float inv = l_run > 0.f ? 1.0f / l_run : 0.f;
    T* O = static_cast<T*>(p.out) + q_row<MODE>(p, qpos, h);
#pragma unroll
    for (int b = 0; b < DB; ++b) {
      half2v lo = {(T)(ot[b][0] * inv), (T)(ot[b][1] * inv)};
      half2v hi = {(T)(ot[b][2] * inv), (T)(ot[b][3] * inv)};
      *reinterpret_cast<uint2*>(O + 16 * b + 4 * g) = uint2{__builtin_bit_cast(uint32_t, lo), __builtin_bit_cast(uint32_t, hi)};
    }
  }
}

// Prefill on fp32 MFMA (f32, head_dim DD = 64 or 128; not paged): the same
// flash attention on v_mfma_f32_16x16x4_f32, whose products and sums are
// fp32 like the reference's loops.  A workgroup takes 64 query tokens of one
// head, 16 per wave, and 32-key tiles of K and V staged row-major in LDS
// (rows padded to DD + 4 floats).  The MFMA takes one value per lane per
// operand (A[i][k] from lane i + 16k, B[k][j] from lane j + 16k; lane
// j + 16k holds D[4k .. 4k + 3][j]), and the order in which the head_dim
// (scores) or the keys (P.V) are summed is free, so both products read whole
// 16-byte LDS chunks:
//  * S^T[key][query]: k-step s of lane group g takes dim DD/4 g + s, so a
//    lane reads DD/4 consecutive floats of its key row; the wave's queries
//    are the B operand (DD/4 floats per lane, in registers);
//  * O^T[dim][query] += V^T . P^T: the k-step over keys 16j + 4g + i (lane
//    group g) takes the weight the scores left in lane (query, g) as
//    element (j, i), and row m of dim block b is dim 4m + b % 4 + 64 (b / 4),
//    so a lane reads 4 (or 8) consecutive floats of one V row per k-step and
//    ends with 16 consecutive dims per 4 dim blocks for the output.
// Masking, the order of the workgroups, the lazy rescale and the vector-ALU
// P.V for a tile with a non-finite value and masked pairs are the f16
// kernel's.
template <nfhip::AttnMode MODE, int DD>
__global__ __launch_bounds__(256, 2) void prefill_f32_mfma_kernel(Params p) {
  static_assert(MODE != nfhip::AttnMode::Paged, "rows of a KV head must be contiguous in position");
  static_assert(DD == 64 || DD == 128, "head_dim 64 or 128");
  constexpr int TK = 32;              // keys per tile
  constexpr int DP = DD + 4;          // padded LDS row (floats)
  constexpr int DG = DD / 4;          // dims per lane group in the scores
  constexpr int DB = DD / 16;         // dim blocks of the output
  constexpr int NCH = TK * DD / 4 / 256;  // 16-byte chunks of K (and of V) per thread and tile
  __shared__ __attribute__((aligned(16))) float Ks[TK * DP];
  __shared__ __attribute__((aligned(16))) float Vs[TK * DP];
  __shared__ __attribute__((aligned(16))) float ps[4][TK][16];
  __shared__ int tile_bad[2];
  const uint32_t S = p.seq_len;
  uint32_t h, qblk;
  prefill_block(p, h, qblk);
  const uint32_t kvh = (uint32_t)((uint64_t)h * p.n_kv / p.n_heads);
  const int tid = threadIdx.x, lane = tid & 63;
  const int w = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int n = lane & 15, g = lane >> 4;
  const uint32_t q0 = qblk * 64;
  const uint32_t q1 = q0 + 64 < S ? q0 + 64 : S;
  const float* Q = static_cast<const float*>(p.q);
  const float* Kh = static_cast<const float*>(p.k) + kv_row<MODE>(p, kvh, 0);
  const float* Vh = static_cast<const float*>(p.v) + kv_row<MODE>(p, kvh, 0);
  auto lo_of = [&](uint32_t pos) -> uint32_t {
    if constexpr (MODE == nfhip::AttnMode::Cached)
      if (p.window > 0 && pos >= p.window) return pos - p.window + 1;
    return 0u;
  };
  const uint32_t lo_blk = lo_of(q0), hi_blk = q1 - 1;
  const uint32_t lo_last = lo_of(hi_blk);
  const uint32_t qw0 = q0 + 16 * w;
  const uint32_t qpos = qw0 + n;
  const bool qok = qpos < q1;
  const uint32_t qlo = lo_of(qpos);
  // B operand of the scores: dims DG g .. DG g + DG - 1 of this lane's query
  float qb[DG];
  {
    const float* qr = Q + q_row<MODE>(p, qok ? qpos : q0, h) + DG * g;
#pragma unroll
    for (int c = 0; c < DG / 4; ++c) {
      const float4v x = *reinterpret_cast<const float4v*>(qr + 4 * c);
#pragma unroll
      for (int e = 0; e < 4; ++e) qb[4 * c + e] = qok ? x[e] : 0.f;
    }
  }
  const uint32_t wq_last = qw0 + 15 < q1 ? qw0 + 15 : q1 - 1;
  const bool wave_live = qw0 < q1;
  const uint32_t wlo_last = lo_of(wq_last);

  float4v ot[DB];
#pragma unroll
  for (int b = 0; b < DB; ++b) ot[b] = float4v{0.f, 0.f, 0.f, 0.f};
  float m_run = -INFINITY, l_run = 0.f;
  const float sl2 = p.scale * 1.44269504088896341f;

  // tile loads: chunk u of a thread is row (tid + 256u) / (DD/4), 16-byte
  // chunk (tid + 256u) % (DD/4) (coalesced); in the last tile, rows past the
  // block's last query read that query's row and are zeroed when staged
  float4v kr[NCH], vr[NCH];
  auto fetch = [&](int64_t t0) {
#pragma unroll
    for (int u = 0; u < NCH; ++u) {
      const int i = tid + 256 * u;
      const int64_t row = t0 + i / (DD / 4) <= (int64_t)hi_blk ? t0 + i / (DD / 4) : (int64_t)hi_blk;
      kr[u] = *reinterpret_cast<const float4v*>(Kh + (uint64_t)row * DD + 4 * (i % (DD / 4)));
      vr[u] = *reinterpret_cast<const float4v*>(Vh + (uint64_t)row * DD + 4 * (i % (DD / 4)));
    }
  };
  auto stage = [&](int64_t t0, int par, bool checked) {
    bool bad = false;
#pragma unroll
    for (int u = 0; u < NCH; ++u) {
      const int i = tid + 256 * u;
      const int r = i / (DD / 4), c = i % (DD / 4);
      float4v v = vr[u];
      if (checked) {
        const bool vin = t0 + r <= (int64_t)hi_blk;
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          v[e] = vin ? v[e] : 0.f;
          bad = bad || !__builtin_isfinite(v[e]);
        }
      }
      *reinterpret_cast<float4v*>(&Ks[r * DP + 4 * c]) = kr[u];
      *reinterpret_cast<float4v*>(&Vs[r * DP + 4 * c]) = v;
    }
    if (bad) tile_bad[par] = 1;
  };

  auto tile = [&](int64_t t0, int par, auto interior_c) {
    constexpr bool INTERIOR = decltype(interior_c)::value;
    // scores S^T: lane holds keys t0 + 16j + 4g + i for query qpos
    float4v sc[2];
#pragma unroll
    for (int j = 0; j < 2; ++j) {
      float a[DG];
      const float* kr0 = &Ks[(16 * j + n) * DP + DG * g];
#pragma unroll
      for (int c = 0; c < DG / 4; ++c) {
        const float4v x = *reinterpret_cast<const float4v*>(kr0 + 4 * c);
#pragma unroll
        for (int e = 0; e < 4; ++e) a[4 * c + e] = x[e];
      }
      sc[j] = float4v{0.f, 0.f, 0.f, 0.f};
#pragma unroll
      for (int st = 0; st < DG; ++st) sc[j] = __builtin_amdgcn_mfma_f32_16x16x4f32(a[st], qb[st], sc[j], 0, 0, 0);
    }
    float sr[2][4];
    float rmax = -INFINITY;
#pragma unroll
    for (int j = 0; j < 2; ++j)
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        if constexpr (INTERIOR) {
          sr[j][i] = sc[j][i];
        } else {
          const int64_t kt = t0 + 16 * j + 4 * g + i;
          const bool in = qok && kt >= (int64_t)qlo && kt <= (int64_t)qpos;
          sr[j][i] = in ? sc[j][i] : -INFINITY;
        }
        rmax = fmaxf(rmax, sr[j][i]);
      }
    rmax = col_max(rmax);
    const float tmax = rmax * sl2;
    if (__builtin_amdgcn_ballot_w64(tmax > m_run + kLazyLog2) != 0) {  // uniform
      const float m_new = fmaxf(m_run, tmax);
      const float corr = m_new == -INFINITY ? 1.f : __builtin_amdgcn_exp2f(m_run - m_new);
      l_run *= corr;
#pragma unroll
      for (int b = 0; b < DB; ++b) ot[b] *= corr;
      m_run = m_new;
    }
    float pv[2][4];
    float psum = 0.f;
#pragma unroll
    for (int j = 0; j < 2; ++j)
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const float e = __builtin_amdgcn_exp2f(__builtin_fmaf(sr[j][i], sl2, -m_run));
        if constexpr (INTERIOR) pv[j][i] = e;
        else pv[j][i] = sr[j][i] == -INFINITY ? 0.f : e;
        psum += pv[j][i];
      }
    l_run += col_sum(psum);
    if (INTERIOR || !tile_bad[par]) {
#pragma unroll
      for (int j = 0; j < 2; ++j) {
        // V rows of the 4 k-steps (keys 16j + 4g + i), dims 4n' .. 4n' + 3
        // (+ 64) of lane row n' = n
        float4v va[4][DB / 4];
#pragma unroll
        for (int i = 0; i < 4; ++i)
#pragma unroll
          for (int hh = 0; hh < DB / 4; ++hh)
            va[i][hh] = *reinterpret_cast<const float4v*>(&Vs[(16 * j + 4 * g + i) * DP + 4 * n + 64 * hh]);
#pragma unroll
        for (int i = 0; i < 4; ++i)
#pragma unroll
          for (int b = 0; b < DB; ++b)
            ot[b] = __builtin_amdgcn_mfma_f32_16x16x4f32(va[i][b / 4][b % 4], pv[j][i], ot[b], 0, 0, 0);
      }
    } else {
#pragma unroll
      for (int j = 0; j < 2; ++j)
#pragma unroll
        for (int i = 0; i < 4; ++i) ps[w][16 * j + 4 * g + i][n] = pv[j][i];
      __builtin_amdgcn_wave_barrier();
      __builtin_amdgcn_fence(__ATOMIC_ACQ_REL, "wavefront");
      for (int k = 0; k < TK; ++k) {
        const int64_t kt = t0 + k;
        if (!(qok && kt >= (int64_t)qlo && kt <= (int64_t)qpos)) continue;
        const float pk = ps[w][k][n];
        // lane (n, g) holds O^T rows 4g + r of block b: dim 4(4g + r) + b % 4 + 64 (b / 4)
#pragma unroll
        for (int b = 0; b < DB; ++b)
#pragma unroll
          for (int r = 0; r < 4; ++r) ot[b][r] += pk * Vs[k * DP + 4 * (4 * g + r) + b % 4 + 64 * (b / 4)];
      }
      __builtin_amdgcn_wave_barrier();
    }
  };

  if (tid == 0) tile_bad[0] = tile_bad[1] = 0;
  fetch(lo_blk);
  int par = 0;
  for (int64_t t0 = lo_blk; t0 <= (int64_t)hi_blk; t0 += TK, par ^= 1) {
    __syncthreads();  // the previous tile's readers are done
    if (tid == 0) tile_bad[par ^ 1] = 0;
    // every key of the tile in every query's range: no zeroing, no check
    stage(t0, par, !(t0 + TK - 1 <= (int64_t)q0 && t0 >= (int64_t)lo_last));
    __syncthreads();
    if (t0 + TK <= (int64_t)hi_blk) fetch(t0 + TK);
    if (!wave_live || t0 > (int64_t)wq_last) continue;  // no key of this tile for the wave (uniform)
    if (t0 + TK - 1 <= (int64_t)qw0 && t0 >= (int64_t)wlo_last) tile(t0, par, std::true_type{});
    else tile(t0, par, std::false_type{});
  }

  if (qok) {
    const float inv = l_run > 0.f ? 1.0f / l_run : 0.f;
    float* O = static_cast<float*>(p.out) + q_row<MODE>(p, qpos, h);
    // lane (n, g): dims 16g + 4r + (b % 4) + 64 (b / 4) of block b, row r
#pragma unroll
    for (int hh = 0; hh < DB / 4; ++hh)
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        const float4v v = {ot[4 * hh][r] * inv, ot[4 * hh + 1][r] * inv, ot[4 * hh + 2][r] * inv,
                           ot[4 * hh + 3][r] * inv};
        *reinterpret_cast<float4v*>(O + 64 * hh + 16 * g + 4 * r) = v;
      }
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

// ---- decode: split the keys over many workgroups ----------------------------------
//
// One query token per head, so the work is the KV cache read.  Workgroup =
// one wave = (key split, KV head): it scores its keys for every query head
// that reads this KV head (up to kMaxGroup of them), so each key / value
// row is loaded once for the whole group, and writes one partial (m, l,
// acc[dim]) per query head to the workspace.  A second kernel merges the
// splits of each head in split order (deterministic).

constexpr int kMaxGroup = 8;
constexpr int kBatchDecode = 16;
constexpr int kMaxSplits = 4096;

// Dot products of the lane's key row with the G query rows in LDS.  The row
// is read in chunks of up to 8 16-byte loads, each chunk's loads all issued
// before its FMAs.  `kr` must be a readable row (the caller substitutes row
// 0 for a lane without a key and discards its score).
template <typename T, int G>
__device__ __forceinline__ void dot_rows(const T* kr, uint32_t D, const float (*qs)[kMaxDim], float (&dot)[G]) {
  constexpr int V = 16 / (int)sizeof(T);  // elements per 16-byte load
  typedef T vec_t __attribute__((ext_vector_type(V)));
#pragma unroll
  for (int g = 0; g < G; ++g) dot[g] = 0.0f;
  uint32_t d = 0;
  if ((D % V) == 0 && (reinterpret_cast<uintptr_t>(kr) & 15) == 0) {
    for (; d + 8 * V <= D; d += 8 * V) {
      vec_t x[8];
#pragma unroll
      for (int c = 0; c < 8; ++c) x[c] = *reinterpret_cast<const vec_t*>(kr + d + c * V);
#pragma unroll
      for (int c = 0; c < 8; ++c)
#pragma unroll
        for (int e = 0; e < V; ++e) {
          const float xf = (float)x[c][e];
#pragma unroll
          for (int g = 0; g < G; ++g) dot[g] += qs[g][d + c * V + e] * xf;
        }
    }
    for (; d + V <= D; d += V) {
      const vec_t x = *reinterpret_cast<const vec_t*>(kr + d);
#pragma unroll
      for (int e = 0; e < V; ++e)
#pragma unroll
        for (int g = 0; g < G; ++g) dot[g] += qs[g][d + e] * (float)x[e];
    }
  }
  for (; d < D; ++d) {
    const float xf = f(kr[d]);
#pragma unroll
    for (int g = 0; g < G; ++g) dot[g] += qs[g][d] * xf;
  }
}

template <typename T, nfhip::AttnMode MODE, int G, int R>
__global__ __launch_bounds__(64) void decode_split_kernel(Params p, uint32_t keys_per_split, uint32_t lo,
                                                          float* __restrict__ part) {
  constexpr int VEC = 16 / (int)sizeof(T);               // elements per 16-byte load
  constexpr int KREG = sizeof(T) == 2 ? 16 : 16;         // 16-byte key loads held at once
  constexpr int VB = R == 4 ? 32 : 64;                   // value rows loaded at once
  typedef T vec_t __attribute__((ext_vector_type(VEC)));
  __shared__ float qs[G][kMaxDim];
  __shared__ __attribute__((aligned(16))) float ps[kTile][G < 4 ? G : 4 * ((G + 3) / 4)];  // tile weights [key][head]
  const uint32_t split = blockIdx.x;
  const uint32_t kvh = blockIdx.y;
  const uint32_t H = p.n_heads, KV = p.n_kv, D = p.dim;
  // query heads h with h * KV / H == kvh
  const uint32_t h0 = (uint32_t)(((uint64_t)kvh * H + KV - 1) / KV);
  const uint32_t h1 = (uint32_t)(((uint64_t)(kvh + 1) * H + KV - 1) / KV);
  const int ng = (int)(h1 - h0);
  const int lane = threadIdx.x;
  const T* Q = static_cast<const T*>(p.q);
  const T* K = static_cast<const T*>(p.k);
  const T* V = static_cast<const T*>(p.v);
  // key rows are read as 16-byte vectors when every row is aligned to them
  const bool kvec = (D % VEC) == 0 && (reinterpret_cast<uintptr_t>(K) & 15) == 0 &&
                    (!p.fused_append || (reinterpret_cast<uintptr_t>(p.k_new) & 15) == 0) &&
                    (uint32_t)(D / VEC) <= (uint32_t)KREG;

  // 1. query loads (consumed after the first tile's loads are issued)
  T qraw[G][R];
#pragma unroll
  for (int g = 0; g < G; ++g)
#pragma unroll
    for (int r = 0; r < R; ++r) {
      const uint32_t h = h0 + (uint32_t)(g < ng ? g : ng - 1);
      const uint32_t d = lane + 64 * r;
      qraw[g][r] = Q[q_row<MODE>(p, 0, h) + (d < D ? d : D - 1)];
    }

  int64_t last = p.step;
  if constexpr (MODE == nfhip::AttnMode::Paged) {
    const int64_t cap = (int64_t)p.n_blocks * p.block_size - 1;
    if (last > cap) last = cap;
  }
  const int64_t k_begin = (int64_t)lo + (int64_t)split * keys_per_split;
  int64_t k_end = k_begin + keys_per_split - 1;
  if (k_end > last) k_end = last;
  if (p.fused_append && k_begin <= (int64_t)p.step && (int64_t)p.step <= k_end) {
    // this workgroup owns row `step` of KV head kvh: append it (nobody else reads it)
    const uint64_t src = (uint64_t)kvh * D, dst = ((uint64_t)kvh * p.max_seq + p.step) * D;
    for (uint32_t d = lane; d < D; d += 64) {
      static_cast<T*>(p.k)[dst + d] = static_cast<const T*>(p.k_new)[src + d];
      static_cast<T*>(p.v)[dst + d] = static_cast<const T*>(p.v_new)[src + d];
    }
  }

  float acc[G][R];
  float m[G], l[G];
#pragma unroll
  for (int g = 0; g < G; ++g) {
    m[g] = -INFINITY;
    l[g] = 0.0f;
#pragma unroll
    for (int r = 0; r < R; ++r) acc[g][r] = 0.0f;
  }

  bool first = true;
  for (int64_t t0 = k_begin; t0 <= k_end || first; t0 += kTile) {
    const bool live_tile = t0 <= k_end;
    // 2. this tile's key row (lane = key) and value rows, all loads issued
    const int64_t kp = t0 + lane;
    uint64_t krow = ~0ull;
    if (live_tile && kp <= k_end) krow = kv_row<MODE>(p, kvh, (uint32_t)kp);
    const T* kr = K + (krow != ~0ull ? krow : 0);
    if (p.fused_append && kp == (int64_t)p.step) kr = static_cast<const T*>(p.k_new) + (uint64_t)kvh * D;
    vec_t kx[KREG];
    if (kvec) {
#pragma unroll
      for (int c = 0; c < KREG; ++c)
        if (c * VEC < (int)D) kx[c] = *reinterpret_cast<const vec_t*>(kr + c * VEC);  // uniform bound
    }
    const int nk = live_tile ? (int)((k_end - t0 + 1) < kTile ? (k_end - t0 + 1) : kTile) : 0;
    T x[VB][R];
    bool ok[VB];
#pragma unroll
    for (int jj = 0; jj < VB; ++jj) {
      const int j = jj;
      const uint64_t row = j < nk ? kv_row<MODE>(p, kvh, (uint32_t)(t0 + j)) : ~0ull;
      ok[jj] = row != ~0ull;
      const T* vr = V + (ok[jj] ? row : 0);
      if (p.fused_append && t0 + j == (int64_t)p.step) vr = static_cast<const T*>(p.v_new) + (uint64_t)kvh * D;
#pragma unroll
      for (int r = 0; r < R; ++r) {
        const uint32_t d = lane + 64 * r;
        x[jj][r] = vr[d < D ? d : D - 1];
      }
    }
    if (first) {
      // 3. queries to LDS once their loads are back
#pragma unroll
      for (int g = 0; g < G; ++g)
#pragma unroll
        for (int r = 0; r < R; ++r) {
          const uint32_t d = lane + 64 * r;
          if (d < (uint32_t)kMaxDim) qs[g][d] = (g < ng && d < D) ? f(qraw[g][r]) : 0.0f;
        }
      __syncthreads();
      first = false;
    }
    if (!live_tile) break;
    // 4. scores
    float dot[G];
#pragma unroll
    for (int g = 0; g < G; ++g) dot[g] = 0.0f;
    if (kvec) {
#pragma unroll
      for (int c = 0; c < KREG; ++c) {
        if (c * VEC >= (int)D) break;
#pragma unroll
        for (int e = 0; e < VEC; ++e) {
          const float xf = (float)kx[c][e];
#pragma unroll
          for (int g = 0; g < G; ++g) dot[g] += qs[g][c * VEC + e] * xf;
        }
      }
    } else {
      dot_rows<T, G>(kr, D, qs, dot);
    }
    float s[G];
#pragma unroll
    for (int g = 0; g < G; ++g) s[g] = krow != ~0ull ? dot[g] * p.scale : -INFINITY;
    float pw[G];
    bool any = false;
#pragma unroll
    for (int g = 0; g < G; ++g) {
      float tmax = s[g];
#pragma unroll
      for (int o = 32; o > 0; o >>= 1) tmax = fmaxf(tmax, __shfl_xor(tmax, o));
      pw[g] = 0.0f;
      if (tmax == -INFINITY) continue;  // uniform
      any = true;
      const float m_new = fmaxf(m[g], tmax);
      const float corr = expf(m[g] - m_new);
      pw[g] = s[g] == -INFINITY ? 0.0f : expf(s[g] - m_new);
      float ps = pw[g];
#pragma unroll
      for (int o = 32; o > 0; o >>= 1) ps += __shfl_xor(ps, o);
      l[g] = l[g] * corr + ps;
      m[g] = m_new;
#pragma unroll
      for (int r = 0; r < R; ++r) acc[g][r] *= corr;
    }
    if (!any) continue;
    // 5. P.V: the tile's weights go through LDS (one broadcast read per key
    // and group of 4 heads); the first VB value rows are already in registers
#pragma unroll
    for (int g = 0; g < G; ++g) ps[lane][g] = pw[g];
    __syncthreads();
    for (int j0 = 0; j0 < nk; j0 += VB) {
      if (j0 > 0) {
#pragma unroll
        for (int jj = 0; jj < VB; ++jj) {
          const int j = j0 + jj;
          const uint64_t row = j < nk ? kv_row<MODE>(p, kvh, (uint32_t)(t0 + j)) : ~0ull;
          ok[jj] = row != ~0ull;
          const T* vr = V + (ok[jj] ? row : 0);
          if (p.fused_append && t0 + j == (int64_t)p.step)
            vr = static_cast<const T*>(p.v_new) + (uint64_t)kvh * D;
#pragma unroll
          for (int r = 0; r < R; ++r) {
            const uint32_t d = lane + 64 * r;
            x[jj][r] = vr[d < D ? d : D - 1];
          }
        }
      }
#pragma unroll
      for (int jj = 0; jj < VB; ++jj) {
        if (!ok[jj]) continue;  // uniform
        float pj[G];
#pragma unroll
        for (int g = 0; g < G; ++g) pj[g] = ps[j0 + jj][g];
#pragma unroll
        for (int r = 0; r < R; ++r) {
          const float xv = f(x[jj][r]);
#pragma unroll
          for (int g = 0; g < G; ++g) acc[g][r] += pj[g] * xv;
        }
      }
    }
    __syncthreads();  // ps is rewritten by the next tile
  }

  // partial of (split, head): [m, l, acc[0..D)]
  const uint32_t stride = D + 2;
#pragma unroll
  for (int g = 0; g < G; ++g) {
    if (g >= ng) break;
    float* dst = part + ((uint64_t)split * H + h0 + g) * stride;
    if (lane == 0) {
      dst[0] = m[g];
      dst[1] = l[g];
    }
#pragma unroll
    for (int r = 0; r < R; ++r) {
      const uint32_t dd = lane + 64 * r;
      if (dd < D) dst[2 + dd] = acc[g][r];
    }
  }
}

// ---- decode with the scores on MFMA --------------------------------------------
//
// One query token, f16 or f32 K/V caches, head_dim DD = 64 or 128, G <= 8
// query heads per KV head, 16-byte aligned rows.  A workgroup of NW waves
// covers one KV head and NW x TK keys, one TK-key tile per wave:
//  * scores: S[key][head] = K[key][dims] . Q[head][dims] with A = 16 key rows
//    and B = the query heads as the 16 columns: f16 on
//    v_mfma_f32_16x16x32_f16 (exact f16 products, fp32 sums; a lane's A
//    piece is 8 dims of one key row), f32 on v_mfma_f32_16x16x4_f32 (fp32
//    products and sums; k-step s of lane group kg takes dim DD/4 kg + s, so
//    a lane's pieces are DD/4 consecutive floats of its key row); each lane
//    loads its pieces with 16-byte loads straight into registers, the query
//    operand is loaded once;
//  * softmax in base 2 on the scores (scaled by scale * log2 e), per head
//    across the lanes that hold its 64 keys;
//  * P.V on the vector ALU: lane (kq, dc) holds the 16-byte chunk dc (8 f16
//    or 4 f32 dims) of the value rows RPI*i + kq, loaded with 16-byte loads
//    together with the keys, and takes the tile's weights from LDS;
//  * the NW waves' (m, l, acc) are merged in LDS and written as the split's
//    partial (m in natural-log units); decode_combine_kernel adds the
//    splits.
//    (Measured and not kept: the merge in the last-arriving workgroup of
//    each KV head, 15.7 against 11.4 us at 4096 keys: the store, counter
//    and reload round trips cost more than a second launch; a one-pass
//    combine, each thread merging its column over its splits with a running
//    maximum, 12.4 against 11.9 us.)
// Rows past the range or without storage read row 0 and drop out by select
// (score -inf, value 0), so no load is predicated and unused memory never
// reaches the sums.  Row `step` is read from K_new / V_new when the append is
// fused; the workgroup whose range holds it writes it into the cache.
template <typename T, nfhip::AttnMode MODE, int DD, int G, int TK, int NW>
__global__ __launch_bounds__(NW * 64) void decode_mfma_kernel(Params p, uint32_t keys_per_split, uint32_t lo,
                                                              float* __restrict__ part) {
  constexpr bool F16 = std::is_same<T, half_t>::value;
  static_assert(F16 || std::is_same<T, float>::value, "f16 or f32 caches");
  constexpr int EPC = 16 / (int)sizeof(T);  // elements per 16-byte chunk
  constexpr int KSTEP = F16 ? DD / 32 : DD / 4;  // MFMA k-steps per 16-key block
  constexpr int KB = TK / 16;      // 16-key blocks per tile
  constexpr int CPR = DD / EPC;    // 16-byte chunks per row
  constexpr int RPI = 64 / CPR;    // value rows per load instruction
  constexpr int NV = TK / RPI;     // value loads per lane per tile
  static_assert(TK % RPI == 0 && TK % 16 == 0, "tile");
  typedef T chunk_t __attribute__((ext_vector_type(EPC)));
  // a lane's score operand per k-step: 8 f16 dims, or one f32 dim
  typedef typename std::conditional<F16, half8, float>::type op_t;
  constexpr int NT = NW * 64;
  __shared__ __attribute__((aligned(16))) float ps[NW][TK][G];  // tile weights [wave][key][head]
  __shared__ float wm[NW][G], wl[NW][G];
  __shared__ __attribute__((aligned(16))) float wacc[NW][G][DD];
  const uint32_t split = blockIdx.x, kvh = blockIdx.y;
  const int tid = threadIdx.x, lane = tid & 63;
  const int w = __builtin_amdgcn_readfirstlane(tid >> 6);
  const uint32_t H = p.n_heads, KV = p.n_kv, D = p.dim;
  const uint32_t h0 = (uint32_t)(((uint64_t)kvh * H + KV - 1) / KV);
  const uint32_t h1 = (uint32_t)(((uint64_t)(kvh + 1) * H + KV - 1) / KV);
  const int ng = (int)(h1 - h0);
  const T* Q = static_cast<const T*>(p.q);
  const T* K = static_cast<const T*>(p.k);
  const T* V = static_cast<const T*>(p.v);

  int64_t last = p.step;
  if constexpr (MODE == nfhip::AttnMode::Paged) {
    const int64_t cap = (int64_t)p.n_blocks * p.block_size - 1;
    if (last > cap) last = cap;
  }
  const int64_t k_begin = (int64_t)lo + (int64_t)split * keys_per_split;
  int64_t k_end = k_begin + keys_per_split - 1;
  if (k_end > last) k_end = last;
  const int64_t t0 = k_begin + TK * w;  // this wave's tile
  if (p.fused_append && k_begin <= (int64_t)p.step && (int64_t)p.step <= k_end) {
    const uint64_t src = (uint64_t)kvh * D, dst = ((uint64_t)kvh * p.max_seq + p.step) * D;
    for (uint32_t d = tid; d < D; d += NT) {
      static_cast<T*>(p.k)[dst + d] = static_cast<const T*>(p.k_new)[src + d];
      static_cast<T*>(p.v)[dst + d] = static_cast<const T*>(p.v_new)[src + d];
    }
  }
  // row pointer and validity of tile key j (0..63)
  auto key_ptr = [&](const T* base, const void* fresh, int j, bool& ok) -> const T* {
    const int64_t pos = t0 + j;
    uint64_t row = ~0ull;
    if (pos <= k_end) row = kv_row<MODE>(p, kvh, (uint32_t)pos);
    ok = row != ~0ull;
    const T* r = base + (ok ? row : 0);
    if (p.fused_append && pos == (int64_t)p.step) r = static_cast<const T*>(fresh) + (uint64_t)kvh * D;
    return r;
  };

  // ---- loads: query operand, key operands, value chunks -------------------------
  const int n = lane & 15, kg = lane >> 4;  // MFMA column (head) / k-group of the lane
  // dims of k-step s in lane group kg: f16 32 s + 8 kg .. + 7, f32 DD/4 kg + s
  op_t qb[KSTEP];
  {
    const T* qr = Q + q_row<MODE>(p, 0, h0 + (uint32_t)(n < ng ? n : ng - 1));
    if constexpr (F16) {
#pragma unroll
      for (int s = 0; s < KSTEP; ++s) {
        qb[s] = *reinterpret_cast<const half8*>(qr + 32 * s + 8 * kg);
        if (n >= ng) qb[s] = half8{};
      }
    } else {
#pragma unroll
      for (int c = 0; c < KSTEP / 4; ++c) {
        const float4v x = *reinterpret_cast<const float4v*>(qr + KSTEP * kg + 4 * c);
#pragma unroll
        for (int e = 0; e < 4; ++e) qb[4 * c + e] = n < ng ? x[e] : 0.f;
      }
    }
  }
  op_t ka[KB][KSTEP];
#pragma unroll
  for (int j = 0; j < KB; ++j) {
    bool ok;
    const T* kr = key_ptr(K, p.k_new, 16 * j + n, ok);
    if constexpr (F16) {
#pragma unroll
      for (int s = 0; s < KSTEP; ++s) ka[j][s] = *reinterpret_cast<const half8*>(kr + 32 * s + 8 * kg);
    } else {
#pragma unroll
      for (int c = 0; c < KSTEP / 4; ++c) {
        const float4v x = *reinterpret_cast<const float4v*>(kr + KSTEP * kg + 4 * c);
#pragma unroll
        for (int e = 0; e < 4; ++e) ka[j][4 * c + e] = x[e];
      }
    }
  }
  const int kq = lane / CPR, dc = lane % CPR;
  chunk_t vx[NV];
  bool vok[NV];
#pragma unroll
  for (int i = 0; i < NV; ++i) {
    const T* vr = key_ptr(V, p.v_new, RPI * i + kq, vok[i]);
    vx[i] = *reinterpret_cast<const chunk_t*>(vr + EPC * dc);
  }

  // ---- scores and the tile softmax (lane: keys 16j + 4kg + i, head n) -----------
  float4v sc[KB];
#pragma unroll
  for (int j = 0; j < KB; ++j) {
    sc[j] = float4v{0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int s = 0; s < KSTEP; ++s) {
      if constexpr (F16) sc[j] = __builtin_amdgcn_mfma_f32_16x16x32_f16(ka[j][s], qb[s], sc[j], 0, 0, 0);
      else sc[j] = __builtin_amdgcn_mfma_f32_16x16x4f32(ka[j][s], qb[s], sc[j], 0, 0, 0);
    }
  }
  const float sl2 = p.scale * 1.44269504088896341f;
  float sv[KB][4];
  float tmax = -INFINITY;
#pragma unroll
  for (int j = 0; j < KB; ++j)
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const int64_t pos = t0 + 16 * j + 4 * kg + i;
      bool ok = pos <= k_end;
      if constexpr (MODE == nfhip::AttnMode::Paged)
        if (ok) ok = kv_row<MODE>(p, kvh, (uint32_t)pos) != ~0ull;
      sv[j][i] = ok ? sc[j][i] * sl2 : -INFINITY;
      tmax = fmaxf(tmax, sv[j][i]);
    }
  tmax = col_max(tmax);
  float psum = 0.f;
#pragma unroll
  for (int j = 0; j < KB; ++j)
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const float pw = sv[j][i] == -INFINITY ? 0.f : exp2f(sv[j][i] - tmax);
      psum += pw;
      if (n < G) ps[w][16 * j + 4 * kg + i][n] = pw;
    }
  psum = col_sum(psum);
  if (kg == 0 && n < G) {
    wm[w][n] = tmax;
    wl[w][n] = psum;
  }
  __syncthreads();

  // ---- P.V (lane: dims EPC dc .. EPC dc + EPC - 1 of rows RPI*i + kq) ------------
  float acc[G][EPC];
#pragma unroll
  for (int g = 0; g < G; ++g)
#pragma unroll
    for (int e = 0; e < EPC; ++e) acc[g][e] = 0.f;
#pragma unroll
  for (int i = 0; i < NV; ++i) {
    const int r = RPI * i + kq;
    float pr[G];
    if constexpr (G % 4 == 0) {
#pragma unroll
      for (int g4 = 0; g4 < G; g4 += 4) {
        const float4v t = *reinterpret_cast<const float4v*>(&ps[w][r][g4]);
        pr[g4] = t.x; pr[g4 + 1] = t.y; pr[g4 + 2] = t.z; pr[g4 + 3] = t.w;
      }
    } else {
#pragma unroll
      for (int g = 0; g < G; ++g) pr[g] = ps[w][r][g];
    }
#pragma unroll
    for (int e = 0; e < EPC; ++e) {
      const float x = vok[i] ? (float)vx[i][e] : 0.f;
#pragma unroll
      for (int g = 0; g < G; ++g) acc[g][e] = __builtin_fmaf(pr[g], x, acc[g][e]);
    }
  }
  // add the RPI row groups (lanes dc, dc + CPR, ...): xor shuffles below a
  // distance of 16 lanes, lane-row swaps (VALU, no LDS round trip) at 16 and
  // 32; each pair adds the same two values in the same order on both lanes
#pragma unroll
  for (int o = CPR; o < 16; o <<= 1)
#pragma unroll
    for (int g = 0; g < G; ++g)
#pragma unroll
      for (int e = 0; e < EPC; ++e) acc[g][e] += __shfl_xor(acc[g][e], o);
#pragma unroll
  for (int g = 0; g < G; ++g)
#pragma unroll
    for (int e = 0; e < EPC; ++e) {
      if constexpr (CPR <= 16) {
        const float2s r = lane_swap_pair<false>(acc[g][e]);
        acc[g][e] = r[0] + r[1];
      }
      const float2s r = lane_swap_pair<true>(acc[g][e]);
      acc[g][e] = r[0] + r[1];
    }
  if (kq == 0) {
#pragma unroll
    for (int g = 0; g < G; ++g) {
      float4v* dst = reinterpret_cast<float4v*>(&wacc[w][g][EPC * dc]);
#pragma unroll
      for (int c = 0; c < EPC / 4; ++c)
        dst[c] = float4v{acc[g][4 * c], acc[g][4 * c + 1], acc[g][4 * c + 2], acc[g][4 * c + 3]};
    }
  }
  __syncthreads();

  // ---- merge the 4 waves and write the split's partial per head -----------------
  const uint32_t stride = D + 2;
  for (int idx = tid; idx < ng * DD; idx += NT) {
    const int g = idx / DD, d = idx % DD;
    float M = -INFINITY;
#pragma unroll
    for (int v = 0; v < NW; ++v) M = fmaxf(M, wm[v][g]);
    float L = 0.f, A = 0.f;
#pragma unroll
    for (int v = 0; v < NW; ++v) {
      const float f = wm[v][g] == -INFINITY ? 0.f : exp2f(wm[v][g] - M);
      L += f * wl[v][g];
      A += f * wacc[v][g][d];
    }
    float* dst = part + ((uint64_t)split * H + h0 + g) * stride;
    if (d == 0) {
      dst[0] = M == -INFINITY ? -INFINITY : M * 0.69314718055994531f;  // natural-log units
      dst[1] = L;
    }
    dst[2 + d] = A;
  }
}

template <typename T>
__global__ __launch_bounds__(1024) void decode_combine_kernel(const float* __restrict__ part, uint32_t n_splits,
                                                              uint32_t H, uint32_t D, T* __restrict__ out,
                                                              uint64_t out_row0, uint64_t out_head_stride) {
  // weight of each split, e^(m_s - M) / sum_s l_s e^(m_s - M), formed in
  // LDS by wave 0 of every workgroup of the head; then column d is summed over the
  // splits by `groups` threads (split classes sp % groups) whose partials
  // add in a fixed order.  A workgroup takes 32 columns, so a head's loads
  // spread over D/32 workgroups (measured with 32 heads x 128 dims and 32
  // splits, the whole decode: 11.9 us with one workgroup per head, 15.2
  // with 256 threads, 11.0 with 64 columns and 10.9 with 32; 10.7 with
  // each thread's first column value requested at the start and the
  // splits' (m, l) kept in registers between the passes; 1.4 % less again
  // with the weights and L formed by wave 0 alone, one barrier fewer).
  __shared__ float w[kMaxSplits];
  __shared__ float red[1024];
  __shared__ float mm[2];
  const uint32_t h = blockIdx.x;
  const uint32_t stride = D + 2;
  const uint32_t t = threadIdx.x;
  // workgroup (h, y) takes columns 32y .. 32y + 31: 32 groups of 32 threads
  // (head_dim <= 256: at most 8 workgroups per head)
  constexpr uint32_t dpad = 32, groups = 1024 / dpad;
  const uint32_t grp = t / dpad, dl = t % dpad, d = blockIdx.y * dpad + dl;
  const uint64_t cstep = (uint64_t)H * stride;
  const float* src = part + (uint64_t)h * stride + 2 + (d < D ? d : 0);
  // the thread's first column value is requested before the weights are
  // formed, so its latency overlaps theirs
  const float a0 = d < D && grp < n_splits ? src[(uint64_t)grp * cstep] : 0.0f;
  // wave 0 forms the weights and L on its own: the butterfly max leaves M
  // in every lane, and lanes 0..63 keep (m, l) of split t in registers
  if (t < 64) {
    float m0 = -INFINITY, l0 = 0.0f;
    if (t < n_splits) {
      const float* r = part + ((uint64_t)t * H + h) * stride;
      m0 = r[0];
      l0 = r[1];
    }
    float m = m0;
    for (uint32_t sp = t + 64; sp < n_splits; sp += 64) m = fmaxf(m, part[((uint64_t)sp * H + h) * stride]);
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) m = fmaxf(m, __shfl_xor(m, o));
    const float M = m;
    float L = 0.0f;
    if (t < n_splits) {
      const float wt = m0 == -INFINITY ? 0.0f : expf(m0 - M);
      w[t] = wt;
      L = l0 * wt;
    }
    for (uint32_t sp = t + 64; sp < n_splits; sp += 64) {
      const float* r = part + ((uint64_t)sp * H + h) * stride;
      const float ms = r[0];
      const float wt = ms == -INFINITY ? 0.0f : expf(ms - M);
      w[sp] = wt;
      L += r[1] * wt;
    }
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) L += __shfl_xor(L, o);
    if (t == 0) mm[1] = L > 0.0f ? 1.0f / L : 0.0f;
  }
  __syncthreads();
  float o = 0.0f;
  if (d < D && grp < n_splits) {
    o += a0 * w[grp];
#pragma unroll 8
    for (uint32_t sp = grp + groups; sp < n_splits; sp += groups) o += src[sp * cstep] * w[sp];
  }
  red[t] = o;
  __syncthreads();
  if (grp == 0 && d < D) {
    float sum = 0.0f;
    for (uint32_t g = 0; g < groups; ++g) sum += red[g * dpad + dl];
    out[out_row0 + (uint64_t)h * out_head_stride + d] = (T)(sum * mm[1]);
  }
}

// Decode with the split kernels; hipErrorNotSupported when the group or the
// workspace does not fit (the caller then runs the one-workgroup-per-head kernel).
template <typename T, nfhip::AttnMode MODE>
hipError_t run_decode_split(const Params& p, float* ws, size_t ws_floats, hipStream_t s) {
  const uint32_t H = p.n_heads, KV = p.n_kv;
  const uint32_t gmax = (H + KV - 1) / KV;
  if (!ws || gmax > (uint32_t)kMaxGroup) return hipErrorNotSupported;
  uint32_t lo = 0;
  if constexpr (MODE == nfhip::AttnMode::Cached)
    if (p.window > 0 && p.step >= p.window) lo = p.step - p.window + 1;
  int64_t last = p.step;
  if constexpr (MODE == nfhip::AttnMode::Paged) {
    const int64_t cap = (int64_t)p.n_blocks * p.block_size - 1;
    if (last > cap) last = cap;
  }
  const uint64_t n_keys = last >= (int64_t)lo ? (uint64_t)(last - lo + 1) : 1;
  // about 512 workgroups, whole 64-key tiles, at most 1024 keys each
  uint64_t kps = (n_keys * KV + 511) / 512;
  kps = (kps + kTile - 1) / kTile * kTile;
  if (kps < (uint64_t)kTile) kps = kTile;
  if (kps > 1024) kps = 1024;
  const uint64_t n_splits = (n_keys + kps - 1) / kps;
  if (n_splits > (uint64_t)kMaxSplits || n_splits * H * (p.dim + 2) > ws_floats) return hipErrorNotSupported;
  const int G = gmax == 1 ? 1 : gmax == 2 ? 2 : gmax <= 4 ? 4 : 8;
  // head_dim 64 / 128 and 16-byte aligned rows: scores on MFMA, 4 waves per
  // workgroup, each over its own range of tk keys
  {
    const bool al = ((reinterpret_cast<uintptr_t>(p.q) | reinterpret_cast<uintptr_t>(p.k) |
                      reinterpret_cast<uintptr_t>(p.v) |
                      (p.fused_append ? reinterpret_cast<uintptr_t>(p.k_new) | reinterpret_cast<uintptr_t>(p.v_new)
                                      : 0)) & 15) == 0;
    if (al && (p.dim == 64 || p.dim == 128)) {
      // 4 waves of 32 keys per workgroup (measured at 4096 keys: 7.1 us
      // against 9.0 with 8 waves of 32 and 9.1 with 4 of 64; with 4 of 16,
      // twice the workgroups and partials, 13.1 against 11.7 us with the
      // combine), 64-key tiles past 8192 keys
      const uint32_t tk = n_keys <= 8192 ? 32u : 64u;
      const uint64_t ns = (n_keys + 4 * tk - 1) / (4 * tk);
      if (ns <= (uint64_t)kMaxSplits && ns * H * (p.dim + 2) <= ws_floats) {
        const dim3 g2((unsigned)ns, KV);
#define NF_DECODE_MFMA(DDD, GG)                                                                      \
  if (p.dim == DDD && G == GG) {                                                                     \
    if (tk == 32) decode_mfma_kernel<T, MODE, DDD, GG, 32, 4><<<g2, 256, 0, s>>>(p, 4 * tk, lo, ws);  \
    else decode_mfma_kernel<T, MODE, DDD, GG, 64, 4><<<g2, 256, 0, s>>>(p, 4 * tk, lo, ws);           \
  }
        NF_DECODE_MFMA(64, 1) NF_DECODE_MFMA(64, 2) NF_DECODE_MFMA(64, 4) NF_DECODE_MFMA(64, 8)
        NF_DECODE_MFMA(128, 1) NF_DECODE_MFMA(128, 2) NF_DECODE_MFMA(128, 4) NF_DECODE_MFMA(128, 8)
#undef NF_DECODE_MFMA
        hipError_t e = hipGetLastError();
        if (e != hipSuccess) return e;
        decode_combine_kernel<T><<<dim3(H, (p.dim + 31) / 32), 1024, 0, s>>>(ws, (uint32_t)ns, H, p.dim, static_cast<T*>(p.out),
                                                   q_row<MODE>(p, 0, 0), p.dim);
        return hipGetLastError();
      }
    }
  }
  const dim3 grid((unsigned)n_splits, KV);
  const int R = p.dim <= 64 ? 1 : p.dim <= 128 ? 2 : 4;
#define NF_DECODE_SPLIT(GG, RR) \
  if (G == GG && R == RR) decode_split_kernel<T, MODE, GG, RR><<<grid, 64, 0, s>>>(p, (uint32_t)kps, lo, ws);
  NF_DECODE_SPLIT(1, 1) NF_DECODE_SPLIT(1, 2) NF_DECODE_SPLIT(1, 4)
  NF_DECODE_SPLIT(2, 1) NF_DECODE_SPLIT(2, 2) NF_DECODE_SPLIT(2, 4)
  NF_DECODE_SPLIT(4, 1) NF_DECODE_SPLIT(4, 2) NF_DECODE_SPLIT(4, 4)
  NF_DECODE_SPLIT(8, 1) NF_DECODE_SPLIT(8, 2) NF_DECODE_SPLIT(8, 4)
#undef NF_DECODE_SPLIT
  hipError_t e = hipGetLastError();
  if (e != hipSuccess) return e;
  // output rows: [n_heads, dim] at the query row of token 0
  const uint64_t row0 = q_row<MODE>(p, 0, 0);
  decode_combine_kernel<T><<<dim3(H, (p.dim + 31) / 32), 1024, 0, s>>>(ws, (uint32_t)n_splits, H, p.dim, static_cast<T*>(p.out), row0,
                                             p.dim);
  return hipGetLastError();
}

template <typename T, nfhip::AttnMode MODE>
hipError_t run(const Params& p, uint32_t nq, float* ws, size_t ws_floats, hipStream_t s) {
  if (p.decode) {
    const hipError_t e = run_decode_split<T, MODE>(p, ws, ws_floats, s);
    if (e != hipErrorNotSupported) return e;
    if (p.fused_append) {  // the split kernel declined: append here first
      const uint64_t n = (uint64_t)p.n_kv * p.dim;
      append_kernel<T, MODE == nfhip::AttnMode::Gqa><<<(unsigned)((n + 255) / 256), 256, 0, s>>>(
          static_cast<const T*>(p.k_new), static_cast<const T*>(p.v_new), static_cast<T*>(p.k),
          static_cast<T*>(p.v), p.n_kv, 1, p.dim, p.max_seq, p.step);
      const hipError_t e2 = hipGetLastError();
      if (e2 != hipSuccess) return e2;
    }
  }
  // decode: one query per head, so more waves per workgroup split the keys
  if (p.decode) {
    attention_kernel<T, MODE, 16><<<dim3(nq, p.n_heads), 1024, 0, s>>>(p);
    return hipGetLastError();
  }
  if constexpr (MODE != nfhip::AttnMode::Paged && std::is_same<T, half_t>::value) {
    // f16, head_dim 64 / 128, 16-byte aligned rows: flash attention on MFMA
    const bool al16 = ((reinterpret_cast<uintptr_t>(p.q) | reinterpret_cast<uintptr_t>(p.k) |
                        reinterpret_cast<uintptr_t>(p.v) | reinterpret_cast<uintptr_t>(p.out)) & 15) == 0;
    if (al16 && (p.dim == 64 || p.dim == 128)) {
      const dim3 grid((nq + 63) / 64, p.n_heads);
      if (p.dim == 128) prefill_mfma_kernel<MODE, 128><<<grid, 256, 0, s>>>(p);
      else prefill_mfma_kernel<MODE, 64><<<grid, 256, 0, s>>>(p);
      return hipGetLastError();
    }
  }
  if constexpr (MODE != nfhip::AttnMode::Paged && std::is_same<T, float>::value) {
    // f32, head_dim 64 / 128, 16-byte aligned rows: flash attention on fp32 MFMA
    const bool al16 = ((reinterpret_cast<uintptr_t>(p.q) | reinterpret_cast<uintptr_t>(p.k) |
                        reinterpret_cast<uintptr_t>(p.v) | reinterpret_cast<uintptr_t>(p.out)) & 15) == 0;
    if (al16 && (p.dim == 64 || p.dim == 128)) {
      const dim3 grid((nq + 63) / 64, p.n_heads);
      if (p.dim == 128) prefill_f32_mfma_kernel<MODE, 128><<<grid, 256, 0, s>>>(p);
      else prefill_f32_mfma_kernel<MODE, 64><<<grid, 256, 0, s>>>(p);
      return hipGetLastError();
    }
  }
  if constexpr (MODE != nfhip::AttnMode::Paged) {
    // many queries per workgroup when the tiles fit and the rows allow
    // 4-element vector loads
    const bool aligned = ((reinterpret_cast<uintptr_t>(p.q) | reinterpret_cast<uintptr_t>(p.k) |
                           reinterpret_cast<uintptr_t>(p.v) | reinterpret_cast<uintptr_t>(p.out)) % 16) == 0;
    if (p.dim <= (uint32_t)kMqDim && p.dim % 4 == 0 && aligned && nq >= 2) {
      // 4 waves (16 queries) per workgroup: 8 waves (32 queries, one
      // workgroup per CU for the LDS) measured 13 % slower at 2048 tokens
      attention_mq_kernel<T, MODE, 4><<<dim3((nq + 4 * kQW - 1) / (4 * kQW), p.n_heads), 256, 0, s>>>(p);
      return hipGetLastError();
    }
  }
  attention_kernel<T, MODE, 4><<<dim3(nq, p.n_heads), 256, 0, s>>>(p);
  return hipGetLastError();
}

template <typename T>
hipError_t launch_t(const nfhip::AttnArgs& a, hipStream_t s) {
  const nfhip::LayerParams& lp = a.lp;
  if (lp.noop) return hipSuccess;
  const uint32_t nq = lp.decode ? 1 : lp.seq_len;
  if (nq == 0) return hipSuccess;
  // decode appends inside the split kernel when that path runs
  const bool fuse = lp.append && lp.decode && a.ws != nullptr;
  if (lp.append && !fuse) {
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
  p.k_new = a.k_new;
  p.v_new = a.v_new;
  p.fused_append = fuse;
  switch (lp.attn) {
    case nfhip::AttnMode::Plain: return run<T, nfhip::AttnMode::Plain>(p, nq, a.ws, a.ws_floats, s);
    case nfhip::AttnMode::Cached: return run<T, nfhip::AttnMode::Cached>(p, nq, a.ws, a.ws_floats, s);
    case nfhip::AttnMode::Gqa: return run<T, nfhip::AttnMode::Gqa>(p, nq, a.ws, a.ws_floats, s);
    default: return run<T, nfhip::AttnMode::Paged>(p, nq, a.ws, a.ws_floats, s);
  }
}

}  // namespace attn
}  // namespace nfk

namespace nfhip {

hipError_t launch_attention(EType t, const AttnArgs& a, hipStream_t s) {
  return t == EType::F16 ? nfk::attn::launch_t<nfk::half_t>(a, s) : nfk::attn::launch_t<float>(a, s);
}

}  // namespace nfhip
