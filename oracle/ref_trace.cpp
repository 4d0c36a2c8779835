// ref_trace.cpp — TEST INFRASTRUCTURE ONLY.
//
// Runs the reference's Chrome-trace exporter (model/model/trace_export.hpp,
// included from where it lies) over this provider's GPU timing ring: a few
// dispatches with timing on, then nf::export_chrome_trace(path).  The
// exporter binds the Metal plugin's timing names (nf_metal_get_timing_count,
// nf_metal_get_timings_ext), which libnf_plugin_hip.so also exports.
//
// Usage: trace_export_run <out.json>; prints "trace_export_run ok <n>".
#include <cstdio>
#include <cstdlib>
#include <cstring>
#include <vector>

#include "neuralOS/ddi/neuro_buffer_abi.h"
#include "neuralOS/ddi/neuro_fabric_abi.h"
#include "neuralOS/ddi/neuro_scheduler_abi.h"
#include "model/model/trace_export.hpp"

extern "C" nf_status nf_plugin_register(nf_provider_vtable* vt, nf_provider* out);
extern "C" nf_status nf_plugin_register_mem(nf_provider_mem_vtable* mem_vt);
extern "C" void nf_metal_enable_timing(bool enable);

#define CHECK(x)                                                            \
  do {                                                                      \
    if (!(x)) {                                                             \
      std::fprintf(stderr, "CHECK failed: %s (line %d)\n", #x, __LINE__); \
      return 1;                                                             \
    }                                                                       \
  } while (0)

namespace {

struct Buf {
  nf_buffer b = nullptr;
  nf_buffer_ops ops{};
};

Buf alloc(nf_provider prov, nf_provider_mem_vtable& mem, nf_dtype dt, size_t bytes) {
  Buf r;
  nf_buffer_alloc_request req{};
  req.desc.dtype = dt;
  req.desc.ndim = 1;
  req.desc.shape[0] = bytes;
  req.desc.size_bytes = bytes;
  req.preferred = NF_MEM_DOMAIN_DEVICE;
  if (mem.alloc(prov, &req, &r.ops, &r.b) != NF_OK) r.b = nullptr;
  return r;
}

nf_status run(nf_provider_vtable& vt, nf_provider prov, const char* op, std::vector<Buf> ins, std::vector<Buf> outs,
              uint32_t M, uint32_t N, uint32_t K) {
  nf_task_desc td{};
  std::strncpy(td.op_name, op, NF_MAX_OP_NAME - 1);
  for (size_t i = 0; i < ins.size(); ++i) {
    td.inputs[i] = ins[i].b;
    td.input_ops[i] = ins[i].ops;
  }
  td.n_inputs = (uint32_t)ins.size();
  for (size_t i = 0; i < outs.size(); ++i) {
    td.outputs[i] = outs[i].b;
    td.output_ops[i] = outs[i].ops;
  }
  td.n_outputs = (uint32_t)outs.size();
  if (M) {
    uint32_t pc[12] = {};
    pc[5] = M;
    pc[6] = N;
    pc[7] = K;
    std::memcpy(td.push_constants, pc, sizeof(pc));
    td.push_constants_size = sizeof(pc);
  }
  return vt.dispatch(prov, td.op_name, td.inputs, td.n_inputs, td.outputs, td.n_outputs);
}

}  // namespace

int main(int argc, char** argv) {
  const char* path = argc > 1 ? argv[1] : "nf_trace.json";
  nf_provider_vtable vt{};
  nf_provider_mem_vtable mem{};
  nf_provider prov = nullptr;
  CHECK(nf_plugin_register(&vt, &prov) == NF_OK);
  CHECK(nf_plugin_register_mem(&mem) == NF_OK);
  CHECK(vt.init(prov) == NF_OK);
  const uint32_t M = 1, N = 4096, K = 4096;
  Buf a = alloc(prov, mem, NF_DTYPE_F32, (size_t)M * K * 4);
  Buf w = alloc(prov, mem, NF_DTYPE_Q4_0, (size_t)N * K / 32 * 18);
  Buf c = alloc(prov, mem, NF_DTYPE_F32, (size_t)M * N * 4);
  Buf d = alloc(prov, mem, NF_DTYPE_F32, (size_t)N * K * 4);
  CHECK(a.b && w.b && c.b && d.b);
  nf_metal_enable_timing(true);
  CHECK(run(vt, prov, "dequant_q4_0_linear", {a, w}, {c}, M, N, K) == NF_OK);
  CHECK(run(vt, prov, "dequant_q4_0", {w}, {d}, 0, 0, 0) == NF_OK);
  CHECK(run(vt, prov, "silu", {c}, {a}, 0, 0, 0) == NF_OK);
  CHECK(vt.synchronize(prov) == NF_OK);
  const uint32_t n = nf_metal_get_timing_count();
  CHECK(n == 3);
  CHECK(nf::export_chrome_trace(path));
  std::printf("trace_export_run ok %u\n", n);
  for (Buf* b : {&a, &w, &c, &d}) b->ops.release(b->b);
  vt.shutdown(prov);
  return 0;
}
