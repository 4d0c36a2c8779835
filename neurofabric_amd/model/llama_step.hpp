// llama_step.hpp — this provider's model layer for llama-family models.
//
// Loads a GGUF model (the reference's loader, model/model/gguf_loader.hpp)
// into provider buffers and builds the per-token step graph on the
// reference's PipelineEngine (core/include/neuralOS/kernel/PipelineEngine.hpp),
// the same graph as the reference's model layer
// (llama_dag_builder.hpp:1386-1530: embedding, per layer rms_norm, q/k/v,
// rope_batch on q and k, flash_attention_cached with the KV-cache append,
// o, residual add, rms_norm, gate/up, silu, elementwise_mul, down, residual
// add; then the final norm, the output projection and, for f32 logits,
// argmax) with the same
// push constants (:1539-1625).  What differs is the op of each projection:
// nf_hip_projection_op_name picks it from the weight's dtype, so Q4_0 and
// Q8_0 projections and a Q4_0 / Q8_0 output projection run the fused
// dequant + linear ops on the quantized blocks as loaded (the reference
// fuses Q4_0 only and always dequantizes the output projection to a dense
// fp32 copy for `linear`).  Quantized formats the provider does not fuse are
// dequantized once at load and run as `linear`, as in the reference.
//
// Header-only C++20; compile with the reference's include directories
// (core/include and the repository root, for model/gguf_loader.hpp and
// model/quant_registry.hpp) and this repository's include/, and link
// libnf_plugin_hip.so.
#pragma once

#include <cstdio>
#include <cstring>
#include <string>
#include <vector>

#include "model/gguf_loader.hpp"
#include "model/quant_registry.hpp"
#include "neuralOS/ddi/neuro_buffer_abi.h"
#include "neuralOS/ddi/neuro_fabric_abi.h"
#include "neuralOS/kernel/PipelineEngine.hpp"
#include "nf_hip_model.h"

namespace nfhip {
namespace model {

struct Buf {
  nf_buffer buf = nullptr;
  nf_buffer_ops ops{};
};

// The 48-byte push-constant block of every task (metal_provider.mm:70-83).
struct Pc {
  uint32_t seq_len = 0, n_heads = 0, head_dim = 0;
  float eps = 0.f, theta = 0.f;
  uint32_t M = 0, N = 0, K = 0, step = 0, max_seq = 0, window = 0, pad = 0;
};
static_assert(sizeof(Pc) == 48, "push-constant block");

struct Projection {
  Buf w;              // as loaded (quantized blocks) or the dense copy
  uint32_t N = 0, K = 0;
  nf_dtype wtype = NF_DTYPE_F32;  // dtype of `w`
  const char* op = "linear";
};

struct Layer {
  Buf attn_norm, ffn_norm;
  Projection q, k, v, o, gate, up, down;
  Buf k_cache, v_cache;  // [n_kv, max_seq, head_dim]
};

// Node ids of one step graph (for its push constants).
struct StepGraph {
  uint32_t gid = 0, embed = 0, final_norm = 0, lm_head = 0, argmax = 0;
  struct L {
    uint32_t attn_norm, q, k, v, q_rope, k_rope, attn, o, add1, ffn_norm, gate, up, silu, mul, down, add2;
  };
  std::vector<L> layers;
};

struct Llama {
  nf::PipelineEngine* engine = nullptr;
  nf_provider prov = nullptr;
  nf_provider_vtable vt{};
  nf_provider_mem_vtable mem{};
  bool fp16 = false;
  uint32_t D = 0, NL = 0, H = 0, KVH = 0, HD = 0, F = 0, V = 0, MS = 0, S_max = 0;
  float eps = 1e-5f, theta = 10000.f;
  Buf embed;  // dense [V, D] table
  std::vector<Layer> layers;
  Buf out_norm;
  Projection lm_head;
  std::vector<Buf> hidden;  // NL + 1 residual-stream buffers
  Buf normed, q, k, v, q_rope, k_rope, attn, proj, resid1, normed2, gate, up, silu, mul, down, final_normed;
  Buf tokens, logits, argmax;
  std::vector<std::string> load_ops;  // ops dispatched while loading (warm-up dequantization)
  std::vector<Buf> owned;
};

inline nf_dtype act_dtype(const Llama& m) { return m.fp16 ? NF_DTYPE_F16 : NF_DTYPE_F32; }
inline size_t act_elt(const Llama& m) { return m.fp16 ? 2 : 4; }

inline Buf alloc(Llama& m, nf_dtype dt, size_t bytes) {
  Buf b;
  nf_buffer_alloc_request req{};
  req.desc.dtype = dt;
  req.desc.ndim = 1;
  req.desc.shape[0] = bytes;
  req.desc.size_bytes = bytes;
  req.preferred = NF_MEM_DOMAIN_DEVICE;
  if (m.mem.alloc(m.prov, &req, &b.ops, &b.buf) != NF_OK) b.buf = nullptr;
  if (b.buf) m.owned.push_back(b);
  return b;
}

// map / memcpy / unmap, the reference's weight upload (llama_dag_builder.hpp:146-156).
inline Buf upload(Llama& m, nf_dtype dt, const void* src, size_t bytes) {
  Buf b = alloc(m, dt, bytes);
  void* dst = nullptr;
  if (!b.buf || b.ops.map(b.buf, &dst) != NF_OK) return Buf{};
  std::memcpy(dst, src, bytes);
  b.ops.unmap(b.buf);
  return b;
}

// One task through the provider, as a one-node graph would run it.
inline nf_status dispatch(Llama& m, const char* op, std::initializer_list<Buf> in, std::initializer_list<Buf> out) {
  nf_task_desc td{};
  std::strncpy(td.op_name, op, NF_MAX_OP_NAME - 1);
  uint32_t i = 0;
  for (const Buf& b : in) {
    td.inputs[i] = b.buf;
    td.input_ops[i++] = b.ops;
  }
  td.n_inputs = i;
  i = 0;
  for (const Buf& b : out) {
    td.outputs[i] = b.buf;
    td.output_ops[i++] = b.ops;
  }
  td.n_outputs = i;
  m.load_ops.push_back(op);
  return m.vt.dispatch(m.prov, td.op_name, td.inputs, td.n_inputs, td.outputs, td.n_outputs);
}

// A weight tensor as the step graph reads it: the fused op's quantized
// blocks, a dense f32 / f16 tensor as stored, or (other quantized formats)
// a dense copy made once here with the provider's dequantization op.
inline bool load_projection(Llama& m, const nf::GGUFTensorInfo& ti, uint32_t N, uint32_t K, Projection& p) {
  const nf_dtype dt = nf::nf_dtype_for_gguf(ti.gguf_dtype);
  p.N = N;
  p.K = K;
  p.op = nf_hip_projection_op_name((uint32_t)dt, m.fp16);
  if (nf::nf_is_quantized(ti.gguf_dtype) && nf_hip_projection_needs_dequant((uint32_t)dt)) {
    const Buf raw = upload(m, dt, ti.data, ti.byte_size);
    p.wtype = act_dtype(m);
    p.w = alloc(m, p.wtype, (size_t)N * K * act_elt(m));
    if (!raw.buf || !p.w.buf) return false;
    if (dispatch(m, nf_hip_dequant_op_name((uint32_t)dt, m.fp16), {raw}, {p.w}) != NF_OK) return false;
    return m.vt.synchronize(m.prov) == NF_OK;
  }
  p.wtype = dt;
  p.w = upload(m, dt, ti.data, ti.byte_size);
  return p.w.buf != nullptr;
}

inline const nf::GGUFTensorInfo* tensor(const nf::GGUFModel& g, const std::string& name) {
  auto it = g.tensors.find(name);
  if (it == g.tensors.end()) {
    std::fprintf(stderr, "[nfhip model] missing tensor %s\n", name.c_str());
    return nullptr;
  }
  return &it->second;
}

// Loads every weight, allocates the KV caches (max_seq positions) and the
// activation buffers (up to max_tokens tokens per step).
inline bool load(Llama& m, const nf::GGUFModel& g, uint32_t max_seq, uint32_t max_tokens) {
  m.D = g.dim;
  m.NL = g.n_layers;
  m.H = g.n_heads;
  m.KVH = g.n_kv_heads ? g.n_kv_heads : g.n_heads;
  m.HD = m.D / m.H;
  m.F = g.ff_dim;
  m.V = g.vocab_size;
  m.MS = max_seq;
  m.S_max = max_tokens;
  m.eps = g.rms_norm_eps;
  m.theta = g.rope_theta;
  const uint32_t KVD = m.KVH * m.HD;
  const size_t e = act_elt(m);
  // token embeddings: a dense table for embedding_lookup
  const nf::GGUFTensorInfo* te = tensor(g, "token_embd.weight");
  if (!te) return false;
  if (m.V == 0) m.V = (uint32_t)(te->n_elements / m.D);
  const nf_dtype edt = nf::nf_dtype_for_gguf(te->gguf_dtype);
  if (nf::nf_is_quantized(te->gguf_dtype)) {
    const Buf raw = upload(m, edt, te->data, te->byte_size);
    m.embed = alloc(m, act_dtype(m), (size_t)m.V * m.D * e);
    if (!raw.buf || !m.embed.buf || dispatch(m, nf_hip_dequant_op_name((uint32_t)edt, m.fp16), {raw}, {m.embed}) != NF_OK)
      return false;
  } else {
    m.embed = upload(m, edt, te->data, te->byte_size);
  }
  auto norm = [&](const std::string& name, Buf& b) {
    const nf::GGUFTensorInfo* t = tensor(g, name);
    if (!t) return false;
    b = upload(m, NF_DTYPE_F32, t->data, t->byte_size);
    return b.buf != nullptr;
  };
  m.layers.resize(m.NL);
  for (uint32_t l = 0; l < m.NL; ++l) {
    Layer& L = m.layers[l];
    const std::string b = "blk." + std::to_string(l) + ".";
    if (!norm(b + "attn_norm.weight", L.attn_norm) || !norm(b + "ffn_norm.weight", L.ffn_norm)) return false;
    struct {
      const char* name;
      Projection* p;
      uint32_t N, K;
    } projs[] = {{"attn_q", &L.q, m.D, m.D},        {"attn_k", &L.k, KVD, m.D},    {"attn_v", &L.v, KVD, m.D},
                 {"attn_output", &L.o, m.D, m.D},   {"ffn_gate", &L.gate, m.F, m.D}, {"ffn_up", &L.up, m.F, m.D},
                 {"ffn_down", &L.down, m.D, m.F}};
    for (auto& pr : projs) {
      const nf::GGUFTensorInfo* t = tensor(g, b + pr.name + ".weight");
      if (!t || !load_projection(m, *t, pr.N, pr.K, *pr.p)) return false;
    }
    L.k_cache = alloc(m, act_dtype(m), (size_t)KVD * m.MS * e);
    L.v_cache = alloc(m, act_dtype(m), (size_t)KVD * m.MS * e);
    if (!L.k_cache.buf || !L.v_cache.buf) return false;
  }
  if (!norm("output_norm.weight", m.out_norm)) return false;
  const nf::GGUFTensorInfo* to = tensor(g, "output.weight");
  if (!to || !load_projection(m, *to, m.V, m.D, m.lm_head)) return false;
  // activations (sized for max_tokens tokens)
  const size_t S = m.S_max;
  auto act = [&](size_t elems) { return alloc(m, act_dtype(m), S * elems * e); };
  m.hidden.resize(m.NL + 1);
  for (auto& h : m.hidden) h = act(m.D);
  m.normed = act(m.D), m.q = act(m.D), m.k = act(KVD), m.v = act(KVD), m.q_rope = act(m.D), m.k_rope = act(KVD);
  m.attn = act(m.D), m.proj = act(m.D), m.resid1 = act(m.D), m.normed2 = act(m.D);
  m.gate = act(m.F), m.up = act(m.F), m.silu = act(m.F), m.mul = act(m.F), m.down = act(m.D);
  m.final_normed = act(m.D), m.logits = act(m.V);
  m.tokens = alloc(m, NF_DTYPE_I32, S * 4);
  m.argmax = alloc(m, NF_DTYPE_I32, S * 4);
  return m.logits.buf && m.tokens.buf && m.argmax.buf && m.vt.synchronize(m.prov) == NF_OK;
}

inline uint32_t node(Llama& m, uint32_t gid, const char* op, std::initializer_list<Buf> in,
                     std::initializer_list<Buf> out) {
  nf_task_desc td{};
  std::strncpy(td.op_name, op, NF_MAX_OP_NAME - 1);
  uint32_t i = 0;
  for (const Buf& b : in) {
    td.inputs[i] = b.buf;
    td.input_ops[i++] = b.ops;
  }
  td.n_inputs = i;
  i = 0;
  for (const Buf& b : out) {
    td.outputs[i] = b.buf;
    td.output_ops[i++] = b.ops;
  }
  td.n_outputs = i;
  td.affinity = NF_AFFINITY_GPU;
  return m.engine->add_task(gid, td);
}

// The step graph: one token batch (prefill) or one token (decode), sizes
// and positions set per step by set_push_constants.
inline StepGraph build_step(Llama& m) {
  nf::PipelineEngine& E = *m.engine;
  StepGraph sg;
  sg.gid = E.create_graph();
  const uint32_t g = sg.gid;
  const char* rope = m.fp16 ? "rope_batch_f16" : "rope_batch";
  sg.embed = node(m, g, "embedding_lookup", {m.embed, m.tokens}, {m.hidden[0]});
  uint32_t prev = sg.embed;
  sg.layers.resize(m.NL);
  for (uint32_t l = 0; l < m.NL; ++l) {
    Layer& L = m.layers[l];
    auto& n = sg.layers[l];
    n.attn_norm = node(m, g, "rms_norm", {m.hidden[l], L.attn_norm}, {m.normed});
    E.add_edge(g, prev, n.attn_norm);
    n.q = node(m, g, L.q.op, {m.normed, L.q.w}, {m.q});
    n.k = node(m, g, L.k.op, {m.normed, L.k.w}, {m.k});
    n.v = node(m, g, L.v.op, {m.normed, L.v.w}, {m.v});
    for (uint32_t t : {n.q, n.k, n.v}) E.add_edge(g, n.attn_norm, t);
    n.q_rope = node(m, g, rope, {m.q}, {m.q_rope});
    n.k_rope = node(m, g, rope, {m.k}, {m.k_rope});
    E.add_edge(g, n.q, n.q_rope);
    E.add_edge(g, n.k, n.k_rope);
    n.attn = node(m, g, "flash_attention_cached", {m.q_rope, m.k_rope, m.v, L.k_cache, L.v_cache}, {m.attn});
    for (uint32_t t : {n.q_rope, n.k_rope, n.v}) E.add_edge(g, t, n.attn);
    n.o = node(m, g, L.o.op, {m.attn, L.o.w}, {m.proj});
    E.add_edge(g, n.attn, n.o);
    n.add1 = node(m, g, "metal_vector_add", {m.hidden[l], m.proj}, {m.resid1});
    E.add_edge(g, n.o, n.add1);
    E.add_edge(g, prev, n.add1);
    n.ffn_norm = node(m, g, "rms_norm", {m.resid1, L.ffn_norm}, {m.normed2});
    E.add_edge(g, n.add1, n.ffn_norm);
    n.gate = node(m, g, L.gate.op, {m.normed2, L.gate.w}, {m.gate});
    n.up = node(m, g, L.up.op, {m.normed2, L.up.w}, {m.up});
    E.add_edge(g, n.ffn_norm, n.gate);
    E.add_edge(g, n.ffn_norm, n.up);
    n.silu = node(m, g, "silu", {m.gate}, {m.silu});
    E.add_edge(g, n.gate, n.silu);
    n.mul = node(m, g, "elementwise_mul", {m.silu, m.up}, {m.mul});
    E.add_edge(g, n.silu, n.mul);
    E.add_edge(g, n.up, n.mul);
    n.down = node(m, g, L.down.op, {m.mul, L.down.w}, {m.down});
    E.add_edge(g, n.mul, n.down);
    n.add2 = node(m, g, "metal_vector_add", {m.resid1, m.down}, {m.hidden[l + 1]});
    E.add_edge(g, n.down, n.add2);
    E.add_edge(g, n.add1, n.add2);
    prev = n.add2;
  }
  sg.final_norm = node(m, g, "rms_norm", {m.hidden[m.NL], m.out_norm}, {m.final_normed});
  E.add_edge(g, prev, sg.final_norm);
  sg.lm_head = node(m, g, m.lm_head.op, {m.final_normed, m.lm_head.w}, {m.logits});
  E.add_edge(g, sg.final_norm, sg.lm_head);
  // argmax reads f32 logits (metal_provider.mm:1601-1619); with f16 logits
  // the reference's node would read half pairs as floats, so the f16 graph
  // leaves it out and the caller reads the logits.
  if (!m.fp16) {
    sg.argmax = node(m, g, "argmax", {m.logits}, {m.argmax});
    E.add_edge(g, sg.lm_head, sg.argmax);
  } else {
    sg.argmax = UINT32_MAX;
  }
  return sg;
}

// Push constants of a step over `seq_len` tokens starting at position
// `step` (the reference's per-node values, llama_dag_builder.hpp:1539-1625).
inline void set_push_constants(const Llama& m, const StepGraph& sg, nf::PipelineEngine::Session& s, uint32_t seq_len,
                               uint32_t step) {
  auto set = [&](uint32_t id, const Pc& pc) { s.set_push_constants_by_id(id, &pc, sizeof(pc)); };
  auto lin = [&](uint32_t N, uint32_t K) {
    Pc pc;
    pc.M = seq_len;
    pc.N = N;
    pc.K = K;
    return pc;
  };
  Pc e;
  e.seq_len = seq_len;
  e.head_dim = m.D;
  set(sg.embed, e);
  Pc norm;
  norm.seq_len = seq_len;
  norm.n_heads = m.H;
  norm.head_dim = m.D;
  norm.eps = m.eps;
  norm.theta = m.theta;
  norm.step = step;
  norm.max_seq = m.MS;
  const uint32_t KVD = m.KVH * m.HD;
  for (uint32_t l = 0; l < m.NL; ++l) {
    const auto& n = sg.layers[l];
    set(n.attn_norm, norm);
    set(n.ffn_norm, norm);
    set(n.q, lin(m.D, m.D));
    set(n.k, lin(KVD, m.D));
    set(n.v, lin(KVD, m.D));
    set(n.o, lin(m.D, m.D));
    set(n.gate, lin(m.F, m.D));
    set(n.up, lin(m.F, m.D));
    set(n.down, lin(m.D, m.F));
    Pc r;
    r.seq_len = seq_len;
    r.head_dim = m.HD;
    r.theta = m.theta;
    r.step = step;
    r.n_heads = m.H;
    set(n.q_rope, r);
    r.n_heads = m.KVH;
    set(n.k_rope, r);
    Pc a;
    a.seq_len = seq_len;
    a.n_heads = m.H;
    a.head_dim = m.HD;
    a.M = m.KVH;
    a.step = step;
    a.max_seq = m.MS;
    set(n.attn, a);
  }
  Pc fn;
  fn.seq_len = seq_len;
  fn.head_dim = m.D;
  fn.eps = m.eps;
  fn.n_heads = m.H;
  set(sg.final_norm, fn);
  set(sg.lm_head, lin(m.V, m.D));
  if (sg.argmax != UINT32_MAX) {
    Pc am;
    am.seq_len = seq_len;
    am.N = m.V;
    set(sg.argmax, am);
  }
}

inline void release(Llama& m) {
  for (Buf& b : m.owned)
    if (b.buf) b.ops.release(b.buf);
  m.owned.clear();
}

}  // namespace model
}  // namespace nfhip
