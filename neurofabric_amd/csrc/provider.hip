// provider.hip — the "amd_hip" execution provider behind the NeuralOS C ABI.
//
// Drop-in for plugins/metal (metal_provider.mm:1999-2120, 2199-2313,
// 3154-3289) on a discrete MI355X:
//   * buffers are hipMalloc'd device memory, zero-filled at allocation, with
//     a pinned host staging copy for map/unmap (map = device->host copy
//     after all enqueued work, unmap = host->device copy on the same stream);
//   * every dispatch is validated on the host (plan.cpp) and then enqueued
//     on ONE in-order HIP stream under a mutex, so dependent ops dispatched
//     from different engine threads execute in submission order — the
//     engine treats "dispatch returned" as done (PipelineEngine.hpp:639-650);
//   * every launch records a completion event (a provider-owned ring), and
//     each buffer it writes keeps that event, so map and
//     cache_sync(INVALIDATE) block until the last dispatch that wrote the
//     buffer has finished, not until the whole stream drains (the Metal
//     fence contract, metal_provider.mm:2044-2062);
//   * unknown ops return NF_ERROR_UNSUPPORTED_OP, bad arity or sizes
//     NF_ERROR_INVALID_ARG, HIP failures NF_ERROR_DEVICE_LOST / _INTERNAL /
//     _OUT_OF_MEMORY.  Nothing falls back to the CPU.
#include <hip/hip_runtime.h>

#include <atomic>
#include <chrono>
#include <cstddef>
#include <cstdio>
#include <cstdlib>
#include <cstring>
#include <map>
#include <mutex>
#include <string>
#include <thread>

#include "launch.hpp"
#include "nf_abi.h"
#include "nf_hip_plugin.h"
#include "plan.hpp"

namespace nfhip {
namespace {

thread_local std::string t_last_error;

nf_status set_error(nf_status st, const std::string& msg) {
  t_last_error = msg;
  return st;
}

nf_status map_hip(hipError_t e, const char* where) {
  if (e == hipSuccess) return NF_OK;
  std::string msg = std::string(where) + ": " + hipGetErrorName(e) + " (" + hipGetErrorString(e) + ")";
  switch (e) {
    case hipErrorOutOfMemory:
      return set_error(NF_ERROR_OUT_OF_MEMORY, msg);
    case hipErrorInvalidValue:
    case hipErrorInvalidConfiguration:
    case hipErrorInvalidDeviceFunction:
    case hipErrorNoBinaryForGpu:
      return set_error(NF_ERROR_INTERNAL, msg);
    default:
      return set_error(NF_ERROR_DEVICE_LOST, msg);
  }
}

// Buffers at or above this size drop their host staging after unmap, so
// uploading model weights does not keep a second pinned copy alive; the
// block goes back to a provider-wide pool (at most kPoolCap bytes) that the
// next large map reuses.  Fresh pinned memory costs one CPU page fault per
// 4 KiB page on first touch (about 2.8 GB/s of memcpy into it on MI355X
// hosts, against 31 GB/s into touched pages), so reusing blocks is what
// makes the reference's map / memcpy / unmap weight upload fast.
constexpr uint64_t kKeepStagingBelow = 64ull << 20;
constexpr uint64_t kPoolCap = 2ull << 30;

struct Provider;

struct Buffer {
  std::atomic<uint32_t> refs{1};
  Provider* prov = nullptr;
  nf_tensor_desc desc{};
  void* dev = nullptr;
  uint64_t bytes = 0;  // desc.size_bytes
  uint64_t alloc_bytes = 0;
  bool owns_dev = true;
  std::mutex mu;  // guards the fields below
  void* host = nullptr;     // pinned staging
  uint64_t host_bytes = 0;  // size of the pinned block (may exceed alloc_bytes when pooled)
  // The staging copy mirrors the device contents as of write sequence
  // host_seq (valid only while host_has).  It is current iff host_seq equals
  // last_write_seq, which launches update under the provider lock in the same
  // critical section that enqueues the write, so a map on another thread
  // never mistakes a stale copy for a current one.
  bool host_has = false;
  uint64_t host_seq = 0;
  bool mapped = false;
  uint64_t map_seq = 0;     // last_write_seq when the mapping was (re)filled
  std::atomic<uint64_t> last_write_seq{0};
  // Completion event of the last launch that wrote this buffer (provider
  // lock): ring slot, and the write sequence that event covers.
  int ev_slot = -1;
  uint64_t ev_seq = 0;
  std::atomic<bool> exported{false};  // a share token was handed out
  // A launch captured into a graph wrote this buffer: every replay of that
  // graph rewrites it without passing through the provider, so reads drain
  // the launch stream and never trust the staging copy.
  std::atomic<bool> graph_written{false};
};

inline bool host_current(const Buffer* b) {
  return b->host_has && !b->graph_written.load() && b->host_seq == b->last_write_seq.load();
}

struct TimingRec {
  char op[64];
  hipEvent_t start = nullptr, stop = nullptr;
  uint8_t dtype = 0;
  uint32_t elems = 0;
};

constexpr uint32_t kTimingRing = 1024;
// Completion events, one recorded after each launch (outside graph capture)
// and reused round-robin.  A reused slot was recorded by a later launch on
// the same in-order stream, so waiting on it still covers every earlier write.
constexpr int kEventRing = 256;

struct Provider {
  std::mutex mu;  // init/shutdown and every launch
  bool initialized = false;
  int device = -1;
  hipStream_t stream = nullptr;
  hipDeviceProp_t props{};
  uint64_t issued_seq = 0;            // guarded by mu
  std::atomic<uint64_t> done_seq{0};  // all dispatches <= done_seq finished
  std::atomic<uint64_t> launch_groups{0};  // launches enqueued (a merged group counts once)
  Tuning tuning;
  Workspace ws;  // split-K partials and tile counters
  hipEvent_t done_ev[kEventRing] = {};  // guarded by mu
  int next_ev = 0;
  // Device-to-host copies of map / cache_sync / nf_hip_buffer_read, issued
  // after the host has waited for the buffer's last writer, so they do not
  // queue behind unrelated work on the launch stream.
  hipStream_t copy_stream = nullptr;
  // pinned staging blocks of released large mappings, by size
  std::mutex pool_mu;
  std::multimap<uint64_t, void*> pool;
  uint64_t pool_bytes = 0;
  // timing ring
  std::atomic<bool> timing{false};
  std::atomic<uint32_t> timing_head{0};
  bool ring_ready = false;
  TimingRec ring[kTimingRing];
};

Provider g_prov;

Provider* as_prov(nf_provider p) { return reinterpret_cast<Provider*>(p); }
Buffer* as_buf(nf_buffer b) { return reinterpret_cast<Buffer*>(b); }

// Drain the provider stream; everything issued so far is then complete.
nf_status drain(Provider* p) {
  uint64_t target;
  {
    std::lock_guard<std::mutex> lk(p->mu);
    if (!p->initialized) return NF_OK;
    target = p->issued_seq;
  }
  hipError_t e = hipStreamSynchronize(p->stream);
  if (e != hipSuccess) return map_hip(e, "hipStreamSynchronize");
  uint64_t cur = p->done_seq.load();
  while (cur < target && !p->done_seq.compare_exchange_weak(cur, target)) {
  }
  return NF_OK;
}

// Block until the last launch that wrote `b` has finished: on that launch's
// completion event when it has one, else by draining the stream.
nf_status wait_for_writes(Buffer* b) {
  Provider* p = b->prov;
  // Memory shared with another buffer handle (imported, or exported for
  // import) may be written through that handle, and a buffer a captured
  // graph writes by every replay of it on the launch stream: drain.
  if (!b->owns_dev || b->exported.load() || b->graph_written.load()) return drain(p);
  const uint64_t target = b->last_write_seq.load();
  if (target <= p->done_seq.load()) return NF_OK;
  hipEvent_t ev = nullptr;
  {
    std::lock_guard<std::mutex> lk(p->mu);
    if (!p->initialized) return NF_OK;
    if (b->ev_slot >= 0 && b->ev_seq >= target) ev = p->done_ev[b->ev_slot];
  }
  if (!ev) return drain(p);
  hipError_t e = hipEventSynchronize(ev);
  if (e != hipSuccess) return map_hip(e, "hipEventSynchronize");
  uint64_t cur = p->done_seq.load();
  while (cur < target && !p->done_seq.compare_exchange_weak(cur, target)) {
  }
  return NF_OK;
}

// Returns a pinned block to the pool, or frees it when the pool is full.
void staging_put(Provider* p, void* h, uint64_t bytes) {
  if (!h) return;
  {
    std::lock_guard<std::mutex> lk(p->pool_mu);
    if (p->pool_bytes + bytes <= kPoolCap) {
      p->pool.emplace(bytes, h);
      p->pool_bytes += bytes;
      return;
    }
  }
  (void)hipHostFree(h);
}

void destroy_events(Provider* p) {
  for (auto& ev : p->done_ev) {
    if (ev) (void)hipEventDestroy(ev);
    ev = nullptr;
  }
  p->next_ev = 0;
}

void staging_drop(Buffer* b) {
  if (!b->host) return;
  if (b->host_bytes >= kKeepStagingBelow && b->prov)
    staging_put(b->prov, b->host, b->host_bytes);
  else
    (void)hipHostFree(b->host);
  b->host = nullptr;
  b->host_bytes = 0;
  b->host_has = false;
}

void pool_release_all(Provider* p) {
  std::lock_guard<std::mutex> lk(p->pool_mu);
  for (auto& kv : p->pool) (void)hipHostFree(kv.second);
  p->pool.clear();
  p->pool_bytes = 0;
}

nf_status ensure_staging(Buffer* b) {
  if (b->host) return NF_OK;
  if (b->alloc_bytes >= kKeepStagingBelow && b->prov) {
    // The smallest pooled block that fits and wastes at most half of itself.
    Provider* p = b->prov;
    std::lock_guard<std::mutex> lk(p->pool_mu);
    auto it = p->pool.lower_bound(b->alloc_bytes);
    if (it != p->pool.end() && it->first <= 2 * b->alloc_bytes) {
      b->host = it->second;
      b->host_bytes = it->first;
      p->pool_bytes -= it->first;
      p->pool.erase(it);
      b->host_has = false;
      return NF_OK;
    }
  }
  void* h = nullptr;
  hipError_t e = hipHostMalloc(&h, b->alloc_bytes, hipHostMallocDefault);
  if (e != hipSuccess) return map_hip(e, "hipHostMalloc(staging)");
  b->host = h;
  b->host_bytes = b->alloc_bytes;
  b->host_has = false;
  return NF_OK;
}

// Device-to-host copy of bytes [off, off + n) of `b`: waits for the
// buffer's last writer, then copies on the copy stream and waits for that.
nf_status read_device(Buffer* b, uint64_t off, void* host, uint64_t n) {
  Provider* p = b->prov;
  nf_status st = wait_for_writes(b);
  if (st != NF_OK) return st;
  hipError_t e;
  {
    std::lock_guard<std::mutex> lk(p->mu);
    if (!p->initialized) return set_error(NF_ERROR_INVALID_ARG, "provider not initialised");
    e = hipMemcpyAsync(host, static_cast<const char*>(b->dev) + off, n, hipMemcpyDeviceToHost, p->copy_stream);
  }
  if (e == hipSuccess) e = hipStreamSynchronize(p->copy_stream);
  return e == hipSuccess ? NF_OK : map_hip(e, "hipMemcpyAsync(D2H)");
}

// Copy between staging and device, then wait.  Host-to-device copies go on
// the launch stream (ordered after every dispatch already issued, which may
// still read the old contents) and drain it.
nf_status copy_sync(Buffer* b, bool to_host) {
  Provider* p = b->prov;
  if (b->bytes == 0) return NF_OK;
  if (to_host) return read_device(b, 0, b->host, b->bytes);
  hipError_t e;
  {
    std::lock_guard<std::mutex> lk(p->mu);
    if (!p->initialized) return set_error(NF_ERROR_INVALID_ARG, "provider not initialised");
    e = hipMemcpyAsync(b->dev, b->host, b->bytes, hipMemcpyHostToDevice, p->stream);
  }
  if (e != hipSuccess) return map_hip(e, "hipMemcpyAsync(H2D)");
  return drain(p);
}

void free_buffer(Buffer* b) {
  Provider* p = b->prov;
  if (p && p->initialized) (void)hipStreamSynchronize(p->stream);
  if (b->owns_dev && b->dev) (void)hipFree(b->dev);
  staging_drop(b);
  delete b;
}

/* ---- nf_buffer_ops ------------------------------------------------- */

uint32_t buf_retain(nf_buffer self) {
  return as_buf(self)->refs.fetch_add(1, std::memory_order_relaxed) + 1;
}

uint32_t buf_release(nf_buffer self) {
  Buffer* b = as_buf(self);
  const uint32_t prev = b->refs.fetch_sub(1, std::memory_order_acq_rel);
  if (prev == 1) free_buffer(b);
  return prev - 1;
}

nf_status buf_map(nf_buffer self, void** out_ptr) {
  if (!self || !out_ptr) return set_error(NF_ERROR_INVALID_ARG, "map: null argument");
  Buffer* b = as_buf(self);
  std::lock_guard<std::mutex> lk(b->mu);
  if (b->mapped) return set_error(NF_ERROR_INVALID_ARG, "map: buffer already mapped");
  nf_status st = ensure_staging(b);
  if (st != NF_OK) return st;
  const uint64_t ws = b->last_write_seq.load();
  if (!host_current(b)) {
    st = copy_sync(b, /*to_host=*/true);  // ordered after every enqueued write
    if (st != NF_OK) return st;
    b->host_has = true;
    b->host_seq = ws;
  }
  b->map_seq = ws;
  b->mapped = true;
  *out_ptr = b->host;
  return NF_OK;
}

nf_status buf_unmap(nf_buffer self) {
  if (!self) return set_error(NF_ERROR_INVALID_ARG, "unmap: null buffer");
  Buffer* b = as_buf(self);
  std::lock_guard<std::mutex> lk(b->mu);
  if (!b->mapped) return NF_OK;  // unmapping an unmapped buffer is a no-op, as in Metal
  b->mapped = false;
  // Upload the host view unless a dispatch wrote the buffer while it was
  // mapped (the device contents are then newer than the staging copy).
  if (b->last_write_seq.load() == b->map_seq) {
    nf_status st = copy_sync(b, /*to_host=*/false);
    if (st != NF_OK) return st;
    b->host_has = true;
    b->host_seq = b->map_seq;
  }
  if (b->bytes >= kKeepStagingBelow) staging_drop(b);
  return NF_OK;
}

nf_status buf_cache_sync(nf_buffer self, nf_cache_op op, uint64_t, uint64_t) {
  if (!self) return set_error(NF_ERROR_INVALID_ARG, "cache_sync: null buffer");
  Buffer* b = as_buf(self);
  std::lock_guard<std::mutex> lk(b->mu);
  if ((op & NF_CACHE_FLUSH) && b->mapped) {
    // Host writes made through a live mapping become visible to the device.
    nf_status st = copy_sync(b, false);
    if (st != NF_OK) return st;
  }
  if (op & NF_CACHE_INVALIDATE) {
    nf_status st = wait_for_writes(b);
    if (st != NF_OK) return st;
    if (b->mapped) {
      // A live mapping sees the device's latest contents.
      const uint64_t ws = b->last_write_seq.load();
      st = copy_sync(b, true);
      if (st != NF_OK) return st;
      b->host_has = true;
      b->host_seq = ws;
      b->map_seq = ws;
    }
  }
  return NF_OK;
}

nf_status buf_get_info(nf_buffer self, nf_buffer_info* info) {
  if (!self || !info) return set_error(NF_ERROR_INVALID_ARG, "get_info: null argument");
  Buffer* b = as_buf(self);
  std::memset(info, 0, sizeof(*info));
  info->desc = b->desc;
  info->domain = NF_MEM_DOMAIN_DEVICE;
  info->offset_bytes = 0;
  info->share_token = reinterpret_cast<uint64_t>(b->dev);
  b->exported.store(true);
  info->refcount = b->refs.load(std::memory_order_relaxed);
  return NF_OK;
}

nf_status buf_export(nf_buffer self, uint64_t* token, nf_mem_domain* domain) {
  if (!self || !token || !domain) return set_error(NF_ERROR_INVALID_ARG, "export: null argument");
  *token = reinterpret_cast<uint64_t>(as_buf(self)->dev);
  as_buf(self)->exported.store(true);
  *domain = NF_MEM_DOMAIN_DEVICE;
  return NF_OK;
}

nf_status wrap_device_ptr(Provider* p, uint64_t token, const nf_tensor_desc* desc, nf_buffer* out);

nf_status buf_import(nf_provider provider, uint64_t token, nf_mem_domain domain,
                     const nf_tensor_desc* desc, nf_buffer* out) {
  if (domain != NF_MEM_DOMAIN_DEVICE)
    return set_error(NF_ERROR_UNSUPPORTED_OP, "import: only NF_MEM_DOMAIN_DEVICE tokens are accepted");
  return wrap_device_ptr(as_prov(provider), token, desc, out);
}

nf_buffer_ops make_ops() {
  nf_buffer_ops ops{};
  ops.retain = buf_retain;
  ops.release = buf_release;
  ops.map = buf_map;
  ops.unmap = buf_unmap;
  ops.cache_sync = buf_cache_sync;
  ops.get_info = buf_get_info;
  ops.export_handle = buf_export;
  ops.import_handle = buf_import;
  return ops;
}

/* ---- provider vtable ----------------------------------------------- */

const char* hip_get_name(nf_provider) { return "amd_hip"; }
uint32_t hip_get_abi_version(nf_provider) { return NF_ABI_VERSION; }

nf_status hip_init(nf_provider self) {
  Provider* p = as_prov(self);
  if (!p) return set_error(NF_ERROR_INVALID_ARG, "init: null provider");
  std::lock_guard<std::mutex> lk(p->mu);
  if (p->initialized) return NF_OK;
  int n = 0;
  hipError_t e = hipGetDeviceCount(&n);
  if (e != hipSuccess || n == 0)
    return set_error(NF_ERROR_DEVICE_LOST, "init: no HIP device visible");
  e = hipGetDevice(&p->device);
  if (e != hipSuccess) return map_hip(e, "hipGetDevice");
  e = hipGetDeviceProperties(&p->props, p->device);
  if (e != hipSuccess) return map_hip(e, "hipGetDeviceProperties");
  if (std::strncmp(p->props.gcnArchName, "gfx950", 6) != 0)
    return set_error(NF_ERROR_DEVICE_LOST, std::string("init: kernels are built for gfx950, device is ") +
                                               p->props.gcnArchName);
  e = hipStreamCreateWithFlags(&p->stream, hipStreamNonBlocking);
  if (e != hipSuccess) return map_hip(e, "hipStreamCreateWithFlags");
  // split-K workspace: 32 MB of partial tiles, 64 Ki tile counters (zeroed once)
  p->ws.part_floats = (size_t)8 << 20;
  p->ws.cnt_len = 1u << 16;
  e = hipMalloc(reinterpret_cast<void**>(&p->ws.part), p->ws.part_floats * sizeof(float));
  if (e == hipSuccess) e = hipMalloc(reinterpret_cast<void**>(&p->ws.cnt), p->ws.cnt_len * sizeof(uint32_t));
  if (e == hipSuccess) e = hipMemsetAsync(p->ws.cnt, 0, p->ws.cnt_len * sizeof(uint32_t), p->stream);
  if (e == hipSuccess) e = hipStreamSynchronize(p->stream);
  if (e == hipSuccess) e = hipStreamCreateWithFlags(&p->copy_stream, hipStreamNonBlocking);
  for (int i = 0; i < kEventRing && e == hipSuccess; ++i)
    e = hipEventCreateWithFlags(&p->done_ev[i], hipEventDisableTiming);
  if (e != hipSuccess) {
    (void)hipFree(p->ws.part);
    (void)hipFree(p->ws.cnt);
    p->ws = Workspace{};
    destroy_events(p);
    if (p->copy_stream) (void)hipStreamDestroy(p->copy_stream);
    p->copy_stream = nullptr;
    (void)hipStreamDestroy(p->stream);
    p->stream = nullptr;
    return map_hip(e, "init: workspace");
  }
  p->initialized = true;
  return NF_OK;
}

void hip_shutdown(nf_provider self) {
  Provider* p = as_prov(self);
  if (!p) return;
  std::lock_guard<std::mutex> lk(p->mu);
  if (!p->initialized) return;
  (void)hipStreamSynchronize(p->stream);
  p->done_seq.store(p->issued_seq);
  if (p->ring_ready) {
    for (auto& r : p->ring) {
      (void)hipEventDestroy(r.start);
      (void)hipEventDestroy(r.stop);
      r.start = r.stop = nullptr;
    }
    p->ring_ready = false;
  }
  (void)hipFree(p->ws.part);
  (void)hipFree(p->ws.cnt);
  p->ws = Workspace{};
  pool_release_all(p);
  destroy_events(p);
  (void)hipStreamDestroy(p->copy_stream);
  p->copy_stream = nullptr;
  (void)hipStreamDestroy(p->stream);
  p->stream = nullptr;
  p->initialized = false;
}

nf_status alloc_buffer(Provider* p, const nf_tensor_desc* desc, nf_buffer* out) {
  if (!p || !desc || !out) return set_error(NF_ERROR_INVALID_ARG, "alloc: null argument");
  {
    std::lock_guard<std::mutex> lk(p->mu);
    if (!p->initialized) return set_error(NF_ERROR_INVALID_ARG, "alloc: provider not initialised");
  }
  Buffer* b = new Buffer;
  b->prov = p;
  b->desc = *desc;
  b->bytes = desc->size_bytes;
  b->alloc_bytes = (desc->size_bytes + 255) & ~255ull;
  if (b->alloc_bytes == 0) b->alloc_bytes = 256;
  hipError_t e = hipMalloc(&b->dev, b->alloc_bytes);
  if (e != hipSuccess) {
    delete b;
    return map_hip(e, "hipMalloc");
  }
  // Zero-fill, as the reference does (metal_provider.mm:2277-2278).
  {
    std::lock_guard<std::mutex> lk(p->mu);
    e = hipMemsetAsync(b->dev, 0, b->alloc_bytes, p->stream);
  }
  if (e == hipSuccess) e = hipStreamSynchronize(p->stream);
  if (e != hipSuccess) {
    (void)hipFree(b->dev);
    delete b;
    return map_hip(e, "zero-fill");
  }
  *out = reinterpret_cast<nf_buffer>(b);
  return NF_OK;
}

nf_status wrap_device_ptr(Provider* p, uint64_t token, const nf_tensor_desc* desc, nf_buffer* out) {
  if (!p || !desc || !out || token == 0) return set_error(NF_ERROR_INVALID_ARG, "import: bad argument");
  Buffer* b = new Buffer;
  b->prov = p;
  b->desc = *desc;
  b->bytes = desc->size_bytes;
  b->alloc_bytes = desc->size_bytes ? desc->size_bytes : 1;
  b->dev = reinterpret_cast<void*>(token);
  b->owns_dev = false;
  *out = reinterpret_cast<nf_buffer>(b);
  return NF_OK;
}

nf_status hip_buffer_alloc(nf_provider self, const nf_tensor_desc* desc, nf_buffer* out) {
  return alloc_buffer(as_prov(self), desc, out);
}

void hip_buffer_free(nf_provider, nf_buffer buf) {
  if (buf) buf_release(buf);
}

nf_status hip_buffer_map(nf_provider, nf_buffer buf, void** out) { return buf_map(buf, out); }
nf_status hip_buffer_unmap(nf_provider, nf_buffer buf) { return buf_unmap(buf); }

bool reads_push_constants(const char* op) { return op_reads_push_constants(op); }

// The engine passes &task_desc.inputs[0]; step back to the descriptor to
// read its push constants (metal_provider.mm:2301-2307).
const nf_task_desc* enclosing_task(const nf_buffer* inputs) {
  const uint8_t* base = reinterpret_cast<const uint8_t*>(inputs) - offsetof(nf_task_desc, inputs);
  return reinterpret_cast<const nf_task_desc*>(base);
}

hipError_t run_plan(const Plan& pl, Buffer* const* in, Buffer* const* out, int gemm_tile, const Workspace& ws,
                    hipStream_t s) {
  switch (pl.path) {
    case Path::Dequant:
      return launch_dequant(pl.q, pl.c, in[0]->dev, pl.in_bytes, out[0]->dev, pl.count, s);
    case Path::Gemv:
      return launch_gemv(pl.q, pl.c, in[0]->dev, in[1]->dev, out[0]->dev, pl.M, pl.N, pl.K, s);
    case Path::Skinny: {
      if (!skinny_fits(1, pl.N, pl.K, in[0]->dev, in[1]->dev))  // odd alignment (imported buffers)
        return pl.c == EType::F16
                   ? launch_gemm_mfma(pl.q, pl.c, in[0]->dev, in[1]->dev, out[0]->dev, pl.M, pl.N, pl.K, gemm_tile, ws, s)
                   : launch_gemv(pl.q, pl.c, in[0]->dev, in[1]->dev, out[0]->dev, pl.M, pl.N, pl.K, s);
      // at most skinny_max_rows activation rows per launch
      const size_t ea = pl.a == EType::F16 ? 2 : 4, ec = pl.c == EType::F16 ? 2 : 4;
      const uint32_t rows = skinny_max_rows(pl.c);
      for (uint32_t m0 = 0; m0 < pl.M; m0 += rows) {
        const uint32_t mc = pl.M - m0 < rows ? pl.M - m0 : rows;
        const hipError_t e = launch_skinny(pl.q, pl.c, static_cast<const char*>(in[0]->dev) + (size_t)m0 * pl.K * ea,
                                           in[1]->dev, static_cast<char*>(out[0]->dev) + (size_t)m0 * pl.N * ec, mc,
                                           pl.N, pl.K, ws, s);
        if (e != hipSuccess) return e;
      }
      return hipSuccess;
    }
    case Path::GemmMfma:
      return launch_gemm_mfma(pl.q, pl.c, in[0]->dev, in[1]->dev, out[0]->dev, pl.M, pl.N, pl.K, gemm_tile, ws, s);
    case Path::Generic:
      return launch_generic(pl.q, pl.c, in[0]->dev, in[1]->dev, out[0]->dev, pl.M, pl.N, pl.K, s);
    case Path::Dense:
      return launch_dense(pl.a, pl.b, pl.c, in[0]->dev, in[1]->dev, out[0]->dev, pl.M, pl.N, pl.K, ws, s);
    case Path::Binary:
      return launch_binary(pl.lp.fn, pl.c, in[0]->dev, in[1]->dev, out[0]->dev, pl.count, s);
    case Path::Unary:  // mock_relu without an output runs in place
      return launch_unary(pl.lp.fn, pl.c, in[0]->dev, (pl.writes_inputs & 1u) ? in[0]->dev : out[0]->dev, pl.count, s);
    case Path::MockPrefill:
      return launch_mock_prefill(in[0]->dev, out[0]->dev, out[1]->dev, pl.count, pl.lp.count2, s);
    case Path::RmsNorm:
      return launch_rms_norm(pl.c, in[0]->dev, in[1]->dev, out[0]->dev, pl.lp.rows, pl.lp.dim, pl.lp.eps, s);
    case Path::Rope:
    case Path::RopeBatch:
      return launch_rope(pl.c, pl.path == Path::RopeBatch, in[0]->dev, out[0]->dev, pl.count, pl.lp.n_heads,
                         pl.lp.head_dim, pl.lp.step, pl.lp.theta, s);
    case Path::Softmax:
      return launch_softmax(in[0]->dev, out[0]->dev, pl.lp.rows, pl.lp.dim, ws.part, ws.part_floats, s);
    case Path::Embedding:
      return launch_embedding(pl.c, in[0]->dev, pl.lp.rows, in[1]->dev, out[0]->dev, pl.count, pl.lp.dim,
                              pl.lp.seq_len, s);
    case Path::MoeGate:
      return launch_moe_gate(in[0]->dev, out[0]->dev, out[1]->dev, pl.lp.rows, pl.lp.n_experts, pl.lp.top_k, s);
    case Path::MoeScatter:
      return launch_moe_scatter(in[0]->dev, pl.lp.n_experts, in[1]->dev, in[2]->dev, out[0]->dev, pl.lp.rows,
                                pl.lp.top_k, pl.lp.dim, s);
    case Path::Argmax:
      return launch_argmax(in[0]->dev, out[0]->dev, pl.lp.rows, pl.lp.dim, ws.part, ws.part_floats, s);
    case Path::Attention: {
      AttnArgs a;
      a.q = in[0]->dev;
      a.lp = pl.lp;
      a.out = out[0]->dev;
      if (pl.lp.attn == AttnMode::Plain) {
        a.k = in[1]->dev;
        a.v = in[2]->dev;
      } else if (pl.lp.attn == AttnMode::Paged) {
        a.k = in[1]->dev;
        a.v = in[2]->dev;
        a.block_table = static_cast<const uint32_t*>(in[3]->dev);
        a.pool_blocks = pl.lp.count2;
      } else {
        a.k_new = in[1]->dev;
        a.v_new = in[2]->dev;
        a.k = in[3]->dev;
        a.v = in[4]->dev;
      }
      a.ws = ws.part;
      a.ws_floats = ws.part_floats;
      return launch_attention(pl.c, a, s);
    }
  }
  return hipErrorInvalidValue;
}

void ensure_ring(Provider* p) {
  if (p->ring_ready) return;
  for (auto& r : p->ring) {
    (void)hipEventCreate(&r.start);
    (void)hipEventCreate(&r.stop);
  }
  p->ring_ready = true;
}

// A validated dispatch: its plan and buffers.
struct Prepared {
  const char* op = nullptr;
  Plan pl;
  Buffer* in[NF_MAX_TASK_INPUTS] = {};
  Buffer* out[NF_MAX_TASK_OUTPUTS] = {};
  uint32_t n_in = 0, n_out = 0;
};

nf_status prepare(Provider* p, const char* op_name, const nf_buffer* inputs, uint32_t n_in, nf_buffer* outputs,
                  uint32_t n_out, Prepared* pr) {
  if (!p || !op_name) return set_error(NF_ERROR_INVALID_ARG, "dispatch: null provider or op name");
  if (!op_known(op_name))
    return set_error(NF_ERROR_UNSUPPORTED_OP, std::string("dispatch: unsupported op '") + op_name + "'");
  if (n_in > NF_MAX_TASK_INPUTS || n_out > NF_MAX_TASK_OUTPUTS || (n_in && !inputs) || (n_out && !outputs))
    return set_error(NF_ERROR_INVALID_ARG, "dispatch: bad input/output arrays");
  const nf_tensor_desc* in_d[NF_MAX_TASK_INPUTS] = {};
  const nf_tensor_desc* out_d[NF_MAX_TASK_OUTPUTS] = {};
  pr->op = op_name;
  pr->n_in = n_in;
  pr->n_out = n_out;
  for (uint32_t i = 0; i < n_in; ++i) {
    pr->in[i] = as_buf(inputs[i]);
    if (!pr->in[i]) return set_error(NF_ERROR_INVALID_ARG, "dispatch: null input buffer");
    in_d[i] = &pr->in[i]->desc;
  }
  for (uint32_t i = 0; i < n_out; ++i) {
    pr->out[i] = as_buf(outputs[i]);
    if (!pr->out[i]) return set_error(NF_ERROR_INVALID_ARG, "dispatch: null output buffer");
    out_d[i] = &pr->out[i]->desc;
  }
  const uint8_t* pc = nullptr;
  uint32_t pc_size = 0;
  if (reads_push_constants(op_name) && n_in > 0) {
    const nf_task_desc* td = enclosing_task(inputs);
    pc_size = td->push_constants_size;
    pc = td->push_constants;
    // The reference binds the descriptor's whole 64-byte block whenever its
    // size is non-zero (metal_provider.mm:2460), so layer ops read every field.
    if (pc_size > 0 && layer_op_known(op_name)) pc_size = NF_MAX_PUSH_CONSTANTS;
  }
  std::string why;
  nf_status st = make_plan(op_name, in_d, n_in, out_d, n_out, pc, pc_size, p->tuning, &pr->pl, &why);
  if (st != NF_OK) return set_error(st, std::string("dispatch ") + op_name + ": " + why);
  return NF_OK;
}

// Enqueue prepared dispatches in order.  n > 1 only for a group that
// groupable() accepted: one grouped launch of the GEMV or small-batch kernel
// (or, if the kernel declines the group, one launch each).
nf_status launch(Provider* p, const Prepared* prs, uint32_t n) {
  hipError_t e = hipSuccess;
  {
    std::lock_guard<std::mutex> lk(p->mu);
    if (!p->initialized) return set_error(NF_ERROR_INVALID_ARG, "dispatch: provider not initialised");
    TimingRec* rec = nullptr;
    if (n == 1 && p->timing.load(std::memory_order_relaxed)) {
      ensure_ring(p);
      rec = &p->ring[p->timing_head.fetch_add(1, std::memory_order_relaxed) % kTimingRing];
      std::strncpy(rec->op, prs[0].op, 63);
      rec->op[63] = '\0';
      rec->dtype = (uint8_t)(prs[0].n_out ? prs[0].out[0] : prs[0].in[0])->desc.dtype;
      const Plan& rp = prs[0].pl;
      rec->elems = (uint32_t)((rp.op == OpKind::FusedLinear || rp.op == OpKind::DenseLinear) ? (uint64_t)rp.M * rp.N
                                                                                              : rp.count);
      (void)hipEventRecord(rec->start, p->stream);
    }
    p->launch_groups.fetch_add(1, std::memory_order_relaxed);
    if (n == 1) {
      e = run_plan(prs[0].pl, prs[0].in, prs[0].out, p->tuning.gemm_tile, p->ws, p->stream);
    } else {
      GemvJob jobs[kGemvGroupMax];
      for (uint32_t j = 0; j < n; ++j) jobs[j] = GemvJob{prs[j].in[1]->dev, prs[j].out[0]->dev, prs[j].pl.N};
      const Plan& pl = prs[0].pl;
      e = pl.path == Path::Gemv ? launch_gemv_group(pl.q, pl.c, prs[0].in[0]->dev, jobs, n, pl.M, pl.K, p->stream)
                                : launch_skinny_group(pl.q, pl.c, prs[0].in[0]->dev, jobs, n, pl.M, pl.K, p->ws,
                                                      p->stream);
      if (e == hipErrorNotSupported) {
        p->launch_groups.fetch_add(n - 1, std::memory_order_relaxed);
        e = hipSuccess;
        for (uint32_t j = 0; j < n && e == hipSuccess; ++j)
          e = run_plan(prs[j].pl, prs[j].in, prs[j].out, p->tuning.gemm_tile, p->ws, p->stream);
      }
    }
    if (rec) (void)hipEventRecord(rec->stop, p->stream);
    // The launch's completion event; none while the stream is being
    // captured into a graph (the written buffers then fall back to a drain).
    int slot = -1;
    bool captured = false;
    if (e == hipSuccess) {
      hipStreamCaptureStatus cs = hipStreamCaptureStatusNone;
      captured = hipStreamIsCapturing(p->stream, &cs) != hipSuccess || cs != hipStreamCaptureStatusNone;
      if (!captured && hipEventRecord(p->done_ev[p->next_ev], p->stream) == hipSuccess) {
        slot = p->next_ev;
        p->next_ev = (p->next_ev + 1) % kEventRing;
      }
    }
    const uint64_t last = p->issued_seq + n;
    for (uint32_t j = 0; j < n; ++j) {
      const uint64_t seq = ++p->issued_seq;
      auto wrote = [&](Buffer* b) {
        b->last_write_seq.store(seq);
        b->ev_slot = slot;
        b->ev_seq = last;
        if (captured) b->graph_written.store(true);
      };
      for (uint32_t i = 0; i < prs[j].n_out; ++i) wrote(prs[j].out[i]);
      for (uint32_t i = 0; i < prs[j].n_in; ++i)
        if (prs[j].pl.writes_inputs & (1u << i)) wrote(prs[j].in[i]);
    }
  }
  if (e != hipSuccess) return map_hip(e, (std::string("launch ") + prs[0].pl.kernel).c_str());
  return NF_OK;
}

nf_status hip_dispatch(nf_provider self, const char* op_name, const nf_buffer* inputs,
                       uint32_t n_in, nf_buffer* outputs, uint32_t n_out) {
  Provider* p = as_prov(self);
  Prepared pr;
  nf_status st = prepare(p, op_name, inputs, n_in, outputs, n_out, &pr);
  if (st != NF_OK) return st;
  return launch(p, &pr, 1);
}

nf_status hip_synchronize(nf_provider self) {
  Provider* p = as_prov(self);
  if (!p) return set_error(NF_ERROR_INVALID_ARG, "synchronize: null provider");
  return drain(p);
}

/* ---- memory vtable ------------------------------------------------- */

nf_status mem_alloc(nf_provider self, const nf_buffer_alloc_request* req, nf_buffer_ops* ops,
                    nf_buffer* buf) {
  if (!req || !ops || !buf) return set_error(NF_ERROR_INVALID_ARG, "mem alloc: null argument");
  nf_status st = alloc_buffer(as_prov(self), &req->desc, buf);
  if (st != NF_OK) return st;
  *ops = make_ops();
  return NF_OK;
}

nf_status mem_import(nf_provider self, uint64_t token, nf_mem_domain domain, const nf_tensor_desc* desc,
                     nf_buffer_ops* ops, nf_buffer* buf) {
  if (!ops) return set_error(NF_ERROR_INVALID_ARG, "mem import: null ops");
  nf_status st = buf_import(self, token, domain, desc, buf);
  if (st != NF_OK) return st;
  *ops = make_ops();
  return NF_OK;
}

nf_status mem_can_import(nf_provider, nf_mem_domain domain) {
  return domain == NF_MEM_DOMAIN_DEVICE ? NF_OK : NF_ERROR_UNSUPPORTED_OP;
}

/* ---- async DDI ----------------------------------------------------- */

struct Token {
  hipEvent_t ev = nullptr;
};

nf_status ddi_dispatch_async(nf_provider self, const char* op, const nf_buffer* in, uint32_t n_in,
                             nf_buffer* out, uint32_t n_out, nf_completion_token* token) {
  if (!token) return set_error(NF_ERROR_INVALID_ARG, "dispatch_async: null token");
  nf_status st = hip_dispatch(self, op, in, n_in, out, n_out);
  if (st != NF_OK) return st;
  Provider* p = as_prov(self);
  Token* t = new Token;
  hipError_t e = hipEventCreateWithFlags(&t->ev, hipEventDisableTiming);
  if (e == hipSuccess) {
    std::lock_guard<std::mutex> lk(p->mu);
    e = hipEventRecord(t->ev, p->stream);
  }
  if (e != hipSuccess) {
    if (t->ev) (void)hipEventDestroy(t->ev);
    delete t;
    return map_hip(e, "dispatch_async: event");
  }
  *token = reinterpret_cast<nf_completion_token>(t);
  return NF_OK;
}

// A token is consumed by the wait/poll call that observes its completion.
nf_status ddi_wait(nf_provider, nf_completion_token token, uint64_t timeout_ms) {
  Token* t = reinterpret_cast<Token*>(token);
  if (!t) return set_error(NF_ERROR_INVALID_ARG, "wait: null token");
  const auto t0 = std::chrono::steady_clock::now();
  for (;;) {
    hipError_t e = hipEventQuery(t->ev);
    if (e == hipSuccess) break;
    if (e != hipErrorNotReady) return map_hip(e, "wait: hipEventQuery");
    if (timeout_ms != UINT64_MAX &&
        std::chrono::steady_clock::now() - t0 >= std::chrono::milliseconds(timeout_ms))
      return set_error(NF_ERROR_TIMEOUT, "wait: timed out");
    std::this_thread::sleep_for(std::chrono::microseconds(20));
  }
  (void)hipEventDestroy(t->ev);
  delete t;
  return NF_OK;
}

nf_status ddi_poll(nf_provider, nf_completion_token token) {
  Token* t = reinterpret_cast<Token*>(token);
  if (!t) return set_error(NF_ERROR_INVALID_ARG, "poll: null token");
  hipError_t e = hipEventQuery(t->ev);
  if (e == hipErrorNotReady) return NF_ERROR_TIMEOUT;
  if (e != hipSuccess) return map_hip(e, "poll: hipEventQuery");
  (void)hipEventDestroy(t->ev);
  delete t;
  return NF_OK;
}

nf_status ddi_query_caps(nf_provider self, nf_driver_caps* caps) {
  Provider* p = as_prov(self);
  if (!p || !caps) return set_error(NF_ERROR_INVALID_ARG, "query_caps: null argument");
  std::memset(caps, 0, sizeof(*caps));
  caps->max_concurrent = 1;  // one in-order stream
  std::lock_guard<std::mutex> lk(p->mu);
  if (p->initialized) caps->memory_bytes = p->props.totalGlobalMem;
  caps->flops = 2516600000000000ull;  // MI355X dense fp16 MFMA peak, FLOP/s
  // f32 / f16 tensors and every block format a dequant op decodes
  caps->supported_dtypes = (1u << NF_DTYPE_F32) | (1u << NF_DTYPE_F16) | (1u << NF_DTYPE_Q4_0) |
                           (1u << NF_DTYPE_Q8_0) | (1u << NF_DTYPE_Q4_1) | (1u << NF_DTYPE_Q5_0) |
                           (1u << NF_DTYPE_Q5_1) | (1u << NF_DTYPE_Q2_K) | (1u << NF_DTYPE_Q3_K) |
                           (1u << NF_DTYPE_Q4_K) | (1u << NF_DTYPE_Q5_K) | (1u << NF_DTYPE_Q6_K);
  caps->flags = NF_CAP_ASYNC | NF_CAP_FP16 | NF_CAP_INT8;
  return NF_OK;
}

uint32_t env_u32(const char* name, uint32_t dflt) {
  const char* v = std::getenv(name);
  if (!v || !*v) return dflt;
  char* end = nullptr;
  unsigned long x = std::strtoul(v, &end, 10);
  return (end && *end == '\0') ? (uint32_t)x : dflt;
}

uint64_t env_u64(const char* name, uint64_t dflt) {
  const char* v = std::getenv(name);
  if (!v || !*v) return dflt;
  char* end = nullptr;
  unsigned long long x = std::strtoull(v, &end, 10);
  return (end && *end == '\0') ? (uint64_t)x : dflt;
}

}  // namespace
}  // namespace nfhip

using namespace nfhip;

extern "C" {

NF_API nf_status nf_plugin_register(nf_provider_vtable* vt, nf_provider* out) {
  if (!vt || !out) return NF_ERROR_INVALID_ARG;
  vt->get_name = hip_get_name;
  vt->get_abi_version = hip_get_abi_version;
  vt->init = hip_init;
  vt->shutdown = hip_shutdown;
  vt->buffer_alloc = hip_buffer_alloc;
  vt->buffer_free = hip_buffer_free;
  vt->buffer_map = hip_buffer_map;
  vt->buffer_unmap = hip_buffer_unmap;
  vt->dispatch = hip_dispatch;
  vt->synchronize = hip_synchronize;
  g_prov.tuning.gemv_max_m_f32 = env_u32("NF_HIP_GEMV_MAX_M_F32", g_prov.tuning.gemv_max_m_f32);
  g_prov.tuning.gemv_max_m_f16 = env_u32("NF_HIP_GEMV_MAX_M_F16", g_prov.tuning.gemv_max_m_f16);
  g_prov.tuning.skinny_max_m_f16 = env_u32("NF_HIP_SKINNY_MAX_M_F16", g_prov.tuning.skinny_max_m_f16);
  g_prov.tuning.skinny_max_m_f32 = env_u32("NF_HIP_SKINNY_MAX_M_F32", g_prov.tuning.skinny_max_m_f32);
  g_prov.tuning.skinny_f16_max_k = env_u32("NF_HIP_SKINNY_F16_MAX_K", g_prov.tuning.skinny_f16_max_k);
  g_prov.tuning.gemv_m2_max_stage_bytes =
      env_u32("NF_HIP_GEMV_M2_MAX_STAGE", g_prov.tuning.gemv_m2_max_stage_bytes);
  g_prov.tuning.gemv_m4_max_weight_bytes =
      env_u64("NF_HIP_GEMV_M4_MAX_WEIGHT", g_prov.tuning.gemv_m4_max_weight_bytes);
  g_prov.tuning.gemm_tile = gemm_tile_from_name(std::getenv("NF_HIP_GEMM_TILE"));
  *out = reinterpret_cast<nf_provider>(&g_prov);
  return NF_OK;
}

NF_API nf_status nf_plugin_register_mem(nf_provider_mem_vtable* mem_vt) {
  if (!mem_vt) return NF_ERROR_INVALID_ARG;
  mem_vt->alloc = mem_alloc;
  mem_vt->import_buffer = mem_import;
  mem_vt->can_import = mem_can_import;
  return NF_OK;
}

NF_API nf_status nf_plugin_register_ddi(nf_ddi_vtable* ddi) {
  if (!ddi) return NF_ERROR_INVALID_ARG;
  ddi->dispatch_async = ddi_dispatch_async;
  ddi->wait_completion = ddi_wait;
  ddi->poll_completion = ddi_poll;
  ddi->query_caps = ddi_query_caps;
  return NF_OK;
}

NF_API void nf_hip_enable_timing(bool enable) {
  g_prov.timing.store(enable, std::memory_order_relaxed);
  if (enable) g_prov.timing_head.store(0, std::memory_order_relaxed);
}

NF_API uint32_t nf_hip_get_timing_count(void) {
  const uint32_t head = g_prov.timing_head.load(std::memory_order_relaxed);
  return head > kTimingRing ? kTimingRing : head;
}

NF_API void nf_hip_get_timings_ext(char (*op_names)[64], double* gpu_ms, uint8_t* dtypes,
                                   uint32_t* elem_counts, uint32_t max_count) {
  const uint32_t head = g_prov.timing_head.load(std::memory_order_relaxed);
  uint32_t count = head > kTimingRing ? kTimingRing : head;
  if (count > max_count) count = max_count;
  const uint32_t start = head > kTimingRing ? head % kTimingRing : 0;
  for (uint32_t i = 0; i < count; ++i) {
    TimingRec& r = g_prov.ring[(start + i) % kTimingRing];
    float ms = 0.f;
    if (r.stop && hipEventSynchronize(r.stop) == hipSuccess) (void)hipEventElapsedTime(&ms, r.start, r.stop);
    if (op_names) std::strncpy(op_names[i], r.op, 64);
    if (gpu_ms) gpu_ms[i] = ms;
    if (dtypes) dtypes[i] = r.dtype;
    if (elem_counts) elem_counts[i] = r.elems;
  }
}

NF_API void nf_hip_get_timings(char (*op_names)[64], double* gpu_ms, uint32_t max_count) {
  nf_hip_get_timings_ext(op_names, gpu_ms, nullptr, nullptr, max_count);
}

// The Metal plugin's timing entry points, under their own names, so code
// that binds them by name (trace_export.hpp:20-25, benchmark_kernels.cpp,
// real_model_test.cpp) links against this library unchanged.
NF_API void nf_metal_enable_timing(bool enable) { nf_hip_enable_timing(enable); }
NF_API uint32_t nf_metal_get_timing_count(void) { return nf_hip_get_timing_count(); }
NF_API void nf_metal_get_timings(char (*op_names)[64], double* gpu_ms, uint32_t max_count) {
  nf_hip_get_timings(op_names, gpu_ms, max_count);
}
NF_API void nf_metal_get_timings_ext(char (*op_names)[64], double* gpu_ms, uint8_t* dtypes, uint32_t* elem_counts,
                                     uint32_t max_count) {
  nf_hip_get_timings_ext(op_names, gpu_ms, dtypes, elem_counts, max_count);
}

NF_API nf_status nf_hip_plan_dispatch(const char* op_name, const nf_tensor_desc* in_descs,
                                      uint32_t n_in, const nf_tensor_desc* out_descs, uint32_t n_out,
                                      const void* push_constants, uint32_t push_constants_size,
                                      nf_hip_plan* plan) {
  if (!plan) return NF_ERROR_INVALID_ARG;
  if (n_in > NF_MAX_TASK_INPUTS || n_out > NF_MAX_TASK_OUTPUTS || (n_in && !in_descs) ||
      (n_out && !out_descs))
    return set_error(NF_ERROR_INVALID_ARG, "plan: bad descriptor arrays");
  const nf_tensor_desc* in_d[NF_MAX_TASK_INPUTS] = {};
  const nf_tensor_desc* out_d[NF_MAX_TASK_OUTPUTS] = {};
  for (uint32_t i = 0; i < n_in; ++i) in_d[i] = &in_descs[i];
  for (uint32_t i = 0; i < n_out; ++i) out_d[i] = &out_descs[i];
  Plan pl;
  std::string why;
  nf_status st = make_plan(op_name, in_d, n_in, out_d, n_out,
                           static_cast<const uint8_t*>(push_constants), push_constants_size,
                           g_prov.tuning, &pl, &why);
  if (st != NF_OK) return set_error(st, why);
  std::memset(plan, 0, sizeof(*plan));
  std::strncpy(plan->kernel, pl.kernel.c_str(), 63);
  plan->M = pl.M;
  plan->N = pl.N;
  plan->K = pl.K;
  plan->count = pl.count;
  plan->weight_bytes = pl.weight_bytes;
  plan->act_bytes = pl.act_bytes;
  plan->out_bytes = pl.out_bytes;
  plan->flops = pl.flops;
  return NF_OK;
}

NF_API void nf_hip_set_gemv_max_m(uint32_t f32_path, uint32_t f16_path) {
  std::lock_guard<std::mutex> lk(g_prov.mu);
  g_prov.tuning.gemv_max_m_f32 = f32_path;
  g_prov.tuning.gemv_max_m_f16 = f16_path;
}

NF_API void nf_hip_set_gemv_row_limits(uint32_t m2_max_stage_bytes, uint64_t m34_max_weight_bytes) {
  std::lock_guard<std::mutex> lk(g_prov.mu);
  g_prov.tuning.gemv_m2_max_stage_bytes = m2_max_stage_bytes;
  g_prov.tuning.gemv_m4_max_weight_bytes = m34_max_weight_bytes;
}

NF_API void nf_hip_get_gemv_row_limits(uint32_t* m2_max_stage_bytes, uint64_t* m34_max_weight_bytes) {
  std::lock_guard<std::mutex> lk(g_prov.mu);
  if (m2_max_stage_bytes) *m2_max_stage_bytes = g_prov.tuning.gemv_m2_max_stage_bytes;
  if (m34_max_weight_bytes) *m34_max_weight_bytes = g_prov.tuning.gemv_m4_max_weight_bytes;
}

NF_API void nf_hip_set_skinny_max_m(uint32_t f16_path) {
  std::lock_guard<std::mutex> lk(g_prov.mu);
  g_prov.tuning.skinny_max_m_f16 = f16_path;
}

NF_API uint32_t nf_hip_get_skinny_max_m(void) {
  std::lock_guard<std::mutex> lk(g_prov.mu);
  return g_prov.tuning.skinny_max_m_f16;
}

NF_API void nf_hip_set_skinny_max_m_f32(uint32_t f32_path) {
  std::lock_guard<std::mutex> lk(g_prov.mu);
  g_prov.tuning.skinny_max_m_f32 = f32_path;
}

NF_API uint32_t nf_hip_get_skinny_max_m_f32(void) {
  std::lock_guard<std::mutex> lk(g_prov.mu);
  return g_prov.tuning.skinny_max_m_f32;
}

NF_API void nf_hip_set_skinny_f16_max_k(uint32_t k) {
  std::lock_guard<std::mutex> lk(g_prov.mu);
  g_prov.tuning.skinny_f16_max_k = k;
}

NF_API uint32_t nf_hip_get_skinny_f16_max_k(void) {
  std::lock_guard<std::mutex> lk(g_prov.mu);
  return g_prov.tuning.skinny_f16_max_k;
}

NF_API void nf_hip_set_gemm_tile(int32_t tile) {
  std::lock_guard<std::mutex> lk(g_prov.mu);
  g_prov.tuning.gemm_tile = (tile >= 0 && tile <= 11) ? tile : -1;
}

NF_API int32_t nf_hip_get_gemm_tile(void) {
  std::lock_guard<std::mutex> lk(g_prov.mu);
  return g_prov.tuning.gemm_tile;
}

NF_API void nf_hip_get_gemv_max_m(uint32_t* f32_path, uint32_t* f16_path) {
  std::lock_guard<std::mutex> lk(g_prov.mu);
  if (f32_path) *f32_path = g_prov.tuning.gemv_max_m_f32;
  if (f16_path) *f16_path = g_prov.tuning.gemv_max_m_f16;
}

bool overlaps(const Buffer* a, const Buffer* b) {
  const uintptr_t a0 = reinterpret_cast<uintptr_t>(a->dev), b0 = reinterpret_cast<uintptr_t>(b->dev);
  return a0 < b0 + b->alloc_bytes && b0 < a0 + a->alloc_bytes;
}

// Paths whose kernels take a group of same-input jobs in one launch: the
// decode GEMV, and the small-batch MFMA kernel while the rows fit one launch.
bool group_path(const Plan& p) {
  return p.path == Path::Gemv || (p.path == Path::Skinny && p.M <= skinny_max_rows(p.c));
}

// May `next` join the group g[0..n)?  Same kernel family, same activation
// buffer, M and K, and no hazard between the members: no output overlaps
// another member's activations, weights or output, so running them in one
// launch is the same as running them in order.
bool groupable(const Prepared* g, uint32_t n, const Prepared& next) {
  if (n >= (uint32_t)kGemvGroupMax) return false;
  const Plan& a = g[0].pl;
  const Plan& b = next.pl;
  if (!group_path(a) || a.path != b.path || a.op != b.op || a.q != b.q || a.a != b.a || a.c != b.c ||
      a.M != b.M || a.K != b.K || next.n_in < 2 || next.n_out < 1 || next.in[0] != g[0].in[0])
    return false;
  for (uint32_t j = 0; j < n; ++j) {
    if (overlaps(next.out[0], g[j].in[0]) || overlaps(next.out[0], g[j].in[1]) || overlaps(next.out[0], g[j].out[0]) ||
        overlaps(g[j].out[0], next.in[1]))
      return false;
  }
  return !overlaps(next.out[0], next.in[0]) && !overlaps(next.out[0], next.in[1]);
}

NF_API nf_status nf_hip_run_tasks(nf_provider self, const nf_task_desc* tasks, uint32_t n_tasks,
                                  uint32_t repeat) {
  Provider* p = as_prov(self);
  if (!p || (n_tasks && !tasks)) return NF_ERROR_INVALID_ARG;
  const bool group = !p->timing.load(std::memory_order_relaxed);
  Prepared prs[kGemvGroupMax + 1];
  for (uint32_t r = 0; r < repeat; ++r) {
    uint32_t i = 0;
    while (i < n_tasks) {
      const nf_task_desc& t = tasks[i];
      nf_status st = prepare(p, t.op_name, t.inputs, t.n_inputs, const_cast<nf_buffer*>(t.outputs), t.n_outputs, &prs[0]);
      if (st != NF_OK) return st;
      uint32_t n = 1;
      while (group && group_path(prs[0].pl) && i + n < n_tasks && n < (uint32_t)kGemvGroupMax) {
        const nf_task_desc& u = tasks[i + n];
        if (prepare(p, u.op_name, u.inputs, u.n_inputs, const_cast<nf_buffer*>(u.outputs), u.n_outputs, &prs[n]) !=
                NF_OK ||
            !groupable(prs, n, prs[n]))
          break;
        ++n;
      }
      st = launch(p, prs, n);
      if (st != NF_OK) return st;
      i += n;
    }
  }
  return NF_OK;
}

NF_API uint64_t nf_hip_launch_count(nf_provider self) {
  Provider* p = as_prov(self);
  return p ? p->launch_groups.load(std::memory_order_relaxed) : 0;
}

NF_API nf_status nf_hip_diag_stream_read(const void* src, uint64_t bytes, void* stream) {
  if (bytes >= 16 && (!src || (uintptr_t)src % 16 != 0))
    return set_error(NF_ERROR_INVALID_ARG, "nf_hip_diag_stream_read: src must be 16-byte aligned");
  return map_hip(launch_diag_read(src, bytes, static_cast<hipStream_t>(stream)), "nf_hip_diag_stream_read");
}

NF_API nf_status nf_hip_get_stream(nf_provider self, void** stream) {
  Provider* p = as_prov(self);
  if (!p || !stream) return NF_ERROR_INVALID_ARG;
  std::lock_guard<std::mutex> lk(p->mu);
  if (!p->initialized) return set_error(NF_ERROR_INVALID_ARG, "get_stream: provider not initialised");
  *stream = reinterpret_cast<void*>(p->stream);
  return NF_OK;
}

NF_API nf_status nf_hip_buffer_device_ptr(nf_buffer buf, void** dev_ptr) {
  if (!buf || !dev_ptr) return NF_ERROR_INVALID_ARG;
  *dev_ptr = as_buf(buf)->dev;
  as_buf(buf)->exported.store(true);  // may now be written outside the provider's launches
  return NF_OK;
}

// Copies between host memory of any kind (pageable, e.g. an mmap of a GGUF
// file, or pinned) and a byte range of a buffer, complete on return.  A
// write is ordered on the provider stream after every dispatch already
// issued; a read waits for the buffer's last writer.
static nf_status buffer_copy(nf_buffer buf, uint64_t offset, void* host, uint64_t bytes, bool to_device) {
  if (!buf || (!host && bytes)) return set_error(NF_ERROR_INVALID_ARG, "buffer copy: null argument");
  Buffer* b = as_buf(buf);
  Provider* p = b->prov;
  if (offset > b->bytes || bytes > b->bytes - offset)
    return set_error(NF_ERROR_INVALID_ARG, "buffer copy: range outside the buffer");
  if (bytes == 0) return NF_OK;
  std::lock_guard<std::mutex> bl(b->mu);
  if (b->mapped) return set_error(NF_ERROR_INVALID_ARG, "buffer copy: buffer is mapped");
  if (!to_device) return read_device(b, offset, host, bytes);
  hipError_t e;
  {
    std::lock_guard<std::mutex> lk(p->mu);
    if (!p->initialized) return set_error(NF_ERROR_INVALID_ARG, "provider not initialised");
    e = hipMemcpyAsync(static_cast<char*>(b->dev) + offset, host, bytes, hipMemcpyHostToDevice, p->stream);
    if (e == hipSuccess) {
      b->last_write_seq.store(++p->issued_seq);
      b->ev_slot = -1;  // written by a copy, not a launch: waiting on it drains
    }
  }
  if (e != hipSuccess) return map_hip(e, "hipMemcpyAsync(write)");
  return drain(p);
}

NF_API nf_status nf_hip_buffer_write(nf_buffer buf, uint64_t offset, const void* src, uint64_t bytes) {
  return buffer_copy(buf, offset, const_cast<void*>(src), bytes, true);
}

NF_API nf_status nf_hip_buffer_read(nf_buffer buf, uint64_t offset, void* dst, uint64_t bytes) {
  return buffer_copy(buf, offset, dst, bytes, false);
}

NF_API void nf_hip_release_staging(nf_provider self) {
  Provider* p = self ? as_prov(self) : &g_prov;
  pool_release_all(p);
}

NF_API const char* nf_hip_last_error(void) { return t_last_error.c_str(); }

}  // extern "C"

// ---- fused linear that allocates nothing -------------------------------------
//
// nf_hip_fused_linear_noalloc runs the fused dequant + linear of dispatch()
// on caller-owned device pointers and a caller's stream.  The split-K partial
// tiles and tile counters its kernels need live in `scratch`, a file-scope
// device array (each GPU the library runs on holds its own copy until the
// process ends), instead of the provider workspace, so the call makes no
// allocation and needs no provider init.
namespace nfhip {
namespace {

constexpr size_t kScratchPartFloats = (size_t)1 << 20;  // 4 MiB of fp32 partial tiles
constexpr uint32_t kScratchCounters = 4096;              // per-tile arrival counters
constexpr size_t kScratchWords = kScratchPartFloats + kScratchCounters;

static __device__ __align__(256) uint32_t scratch[kScratchWords];

// Counters start at zero: the array is zero-initialised when the code object
// loads, cleared again here at set-up, and every split-K launch leaves each
// counter it used back at zero.
__global__ void scratch_clear_kernel(uint32_t* p, uint32_t n) {
  const uint32_t i = blockIdx.x * blockDim.x + threadIdx.x;
  if (i < n) p[i] = 0u;
}

constexpr int kMaxDevices = 64;
std::mutex g_scratch_mu;
uint32_t* g_scratch_ptr[kMaxDevices] = {};  // device address of `scratch`, per device

// Device address of this device's `scratch`, looked up (and its counters
// cleared on `s`) the first time the device is used.
nf_status scratch_for_current_device(hipStream_t s, uint32_t** out) {
  int dev = -1;
  hipError_t e = hipGetDevice(&dev);
  if (e != hipSuccess) return map_hip(e, "hipGetDevice");
  if (dev < 0 || dev >= kMaxDevices) return set_error(NF_ERROR_INVALID_ARG, "noalloc: device index out of range");
  std::lock_guard<std::mutex> lk(g_scratch_mu);
  if (!g_scratch_ptr[dev]) {
    uint32_t* ptr = nullptr;
    e = hipGetSymbolAddress(reinterpret_cast<void**>(&ptr), HIP_SYMBOL(scratch));
    if (e != hipSuccess) return map_hip(e, "hipGetSymbolAddress(scratch)");
    scratch_clear_kernel<<<(kScratchCounters + 255) / 256, 256, 0, s>>>(ptr + kScratchPartFloats, kScratchCounters);
    e = hipGetLastError();
    if (e != hipSuccess) return map_hip(e, "noalloc: scratch clear");
    g_scratch_ptr[dev] = ptr;
  }
  *out = g_scratch_ptr[dev];
  return NF_OK;
}

}  // namespace
}  // namespace nfhip

extern "C" {

NF_API nf_status nf_hip_fused_linear_noalloc(nf_dtype wtype, const void* A, const void* W, void* C, uint32_t M,
                                             uint32_t N, uint32_t K, bool f16, void* stream) {
  if (wtype != NF_DTYPE_Q4_0 && wtype != NF_DTYPE_Q8_0)
    return set_error(NF_ERROR_INVALID_ARG, "noalloc: weight dtype must be Q4_0 or Q8_0");
  if (!A || !W || !C) return set_error(NF_ERROR_INVALID_ARG, "noalloc: null operand");
  if (M == 0 || N == 0 || K == 0) return set_error(NF_ERROR_INVALID_ARG, "noalloc: M, N and K must be non-zero");
  const char* op = wtype == NF_DTYPE_Q4_0 ? (f16 ? "dequant_q4_0_linear_f16" : "dequant_q4_0_linear")
                                          : (f16 ? "dequant_q8_0_linear_f16" : "dequant_q8_0_linear");
  // Descriptors sized exactly for M, N, K, so make_plan validates and plans
  // the call as dispatch() would plan buffers of those sizes.
  const uint64_t elt = f16 ? 2 : 4, bb = wtype == NF_DTYPE_Q4_0 ? 18 : 34;
  const uint64_t blocks = (K % 32 == 0) ? (uint64_t)N * (K / 32) : ((uint64_t)N * K + 31) / 32;
  nf_tensor_desc da{}, dw{}, dc{};
  da.dtype = dc.dtype = f16 ? NF_DTYPE_F16 : NF_DTYPE_F32;
  dw.dtype = wtype;
  da.ndim = dw.ndim = dc.ndim = 1;
  da.size_bytes = da.shape[0] = (uint64_t)M * K * elt;
  dw.size_bytes = dw.shape[0] = blocks * bb;
  dc.size_bytes = dc.shape[0] = (uint64_t)M * N * elt;
  const nf_tensor_desc* ins[2] = {&da, &dw};
  const nf_tensor_desc* outs[1] = {&dc};
  nf_push_constants pc{};
  pc.M = M;
  pc.N = N;
  pc.K = K;
  // The switch points as of this call, copied under the provider lock that
  // the nf_hip_set_* setters take.
  Tuning tuning;
  {
    std::lock_guard<std::mutex> lk(g_prov.mu);
    tuning = g_prov.tuning;
  }
  Plan pl;
  std::string why;
  nf_status st = make_plan(op, ins, 2, outs, 1, reinterpret_cast<const uint8_t*>(&pc), sizeof(pc), tuning, &pl, &why);
  if (st != NF_OK) return set_error(st, std::string("noalloc: ") + why);
  hipStream_t s = static_cast<hipStream_t>(stream);
  uint32_t* ptr = nullptr;
  st = scratch_for_current_device(s, &ptr);
  if (st != NF_OK) return st;
  Workspace ws;
  ws.part = reinterpret_cast<float*>(ptr);
  ws.part_floats = kScratchPartFloats;
  ws.cnt = ptr + kScratchPartFloats;
  ws.cnt_len = kScratchCounters;
  // Operand views for run_plan, which reads only their device addresses.
  Buffer ba, bw, bc;
  ba.dev = const_cast<void*>(A);
  bw.dev = const_cast<void*>(W);
  bc.dev = C;
  Buffer* in[2] = {&ba, &bw};
  Buffer* out[1] = {&bc};
  const hipError_t e = run_plan(pl, in, out, tuning.gemm_tile, ws, s);
  return e == hipSuccess ? NF_OK : map_hip(e, (std::string("noalloc launch ") + pl.kernel).c_str());
}

}  // extern "C"
