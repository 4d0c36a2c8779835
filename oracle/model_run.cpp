// model_run.cpp — TEST INFRASTRUCTURE ONLY (tests/test_gpu_model_layer.py).
//
// Drives this repository's model layer (neurofabric_amd/model/llama_step.hpp)
// on the reference's PipelineEngine with the HIP provider: loads a GGUF
// model, runs a prefill step over the given token ids and then one decode
// step at the next position, and prints
//   load_ops <op> ...               ops dispatched while loading
//   prefill <V values>              logits of the last prefill position
//   decode <V values>               logits of the decode step
//                                   (f32 values, or fp16 bit patterns)
//   step_ops <op> ...               every dispatch of the decode step, in
//                                   order (the provider's timing ring)
//
//   model_run <model.gguf> <fp16 0|1> <id,id,...> <decode id>
#include <cstdio>
#include <cstdlib>
#include <sstream>
#include <string>
#include <vector>

#include "neurofabric_amd/model/llama_step.hpp"

extern "C" nf_status nf_plugin_register(nf_provider_vtable* vt, nf_provider* out);
extern "C" nf_status nf_plugin_register_mem(nf_provider_mem_vtable* mem_vt);
extern "C" void nf_hip_enable_timing(bool enable);
extern "C" uint32_t nf_hip_get_timing_count(void);
extern "C" void nf_hip_get_timings(char (*op_names)[64], double* gpu_ms, uint32_t max_count);

namespace {

void print_row(const char* tag, nfhip::model::Llama& m, uint32_t row) {
  void* p = nullptr;
  if (m.logits.ops.cache_sync(m.logits.buf, NF_CACHE_INVALIDATE, 0, 0) != NF_OK ||
      m.logits.ops.map(m.logits.buf, &p) != NF_OK) {
    std::fprintf(stderr, "logits readback failed\n");
    std::exit(3);
  }
  std::printf("%s", tag);
  for (uint32_t i = 0; i < m.V; ++i) {
    if (m.fp16)  // fp16 logits as their bit patterns
      std::printf(" %u", (unsigned)static_cast<const uint16_t*>(p)[(size_t)row * m.V + i]);
    else
      std::printf(" %.9g", static_cast<const float*>(p)[(size_t)row * m.V + i]);
  }
  std::printf("\n");
  m.logits.ops.unmap(m.logits.buf);
}

void set_tokens(nfhip::model::Llama& m, const std::vector<int32_t>& ids) {
  void* p = nullptr;
  if (m.tokens.ops.map(m.tokens.buf, &p) != NF_OK) std::exit(3);
  std::memcpy(p, ids.data(), ids.size() * 4);
  m.tokens.ops.unmap(m.tokens.buf);
}

}  // namespace

int main(int argc, char** argv) {
  if (argc < 5) {
    std::fprintf(stderr, "usage: %s model.gguf fp16 id,id,... decode_id\n", argv[0]);
    return 2;
  }
  std::vector<int32_t> ids;
  {
    std::stringstream ss(argv[3]);
    std::string t;
    while (std::getline(ss, t, ',')) ids.push_back(std::atoi(t.c_str()));
  }
  const int32_t next = std::atoi(argv[4]);
  nf::GGUFModel* g = nf::gguf_open(argv[1]);
  if (!g) return 4;

  nfhip::model::Llama m;
  m.fp16 = std::atoi(argv[2]) != 0;
  if (nf_plugin_register(&m.vt, &m.prov) != NF_OK || nf_plugin_register_mem(&m.mem) != NF_OK ||
      m.vt.init(m.prov) != NF_OK)
    return 5;
  nf::PipelineEngine engine(4);
  engine.register_provider(m.prov, m.vt, NF_AFFINITY_GPU);
  engine.register_provider_mem(0, m.mem);
  m.engine = &engine;
  if (!nfhip::model::load(m, *g, 64, (uint32_t)ids.size())) {
    std::fprintf(stderr, "model load failed\n");
    return 6;
  }
  std::printf("load_ops");
  for (auto& op : m.load_ops) std::printf(" %s", op.c_str());
  std::printf("\n");

  nfhip::model::StepGraph sg = nfhip::model::build_step(m);
  nf::PipelineEngine::Session sess(engine, sg.gid);
  if (!sess.valid()) return 7;
  const uint32_t S = (uint32_t)ids.size();
  set_tokens(m, ids);
  nfhip::model::set_push_constants(m, sg, sess, S, 0);
  if (sess.step().get() != NF_OK) return 8;
  print_row("prefill", m, S - 1);

  set_tokens(m, {next});
  nfhip::model::set_push_constants(m, sg, sess, 1, S);
  nf_hip_enable_timing(true);
  if (sess.step().get() != NF_OK) return 9;
  m.vt.synchronize(m.prov);
  print_row("decode", m, 0);
  const uint32_t n = nf_hip_get_timing_count();
  std::vector<char> names((size_t)n * 64 + 64);
  std::vector<double> ms(n + 1);
  nf_hip_get_timings(reinterpret_cast<char(*)[64]>(names.data()), ms.data(), n);
  nf_hip_enable_timing(false);
  std::printf("step_ops");
  for (uint32_t i = 0; i < n; ++i) std::printf(" %s", &names[(size_t)i * 64]);
  std::printf("\n");

  nfhip::model::release(m);
  m.vt.shutdown(m.prov);
  nf::gguf_close(g);
  return 0;
}
