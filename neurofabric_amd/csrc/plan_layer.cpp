// plan_layer.cpp — validation and planning of the layer ops that sit around
// the linears in a transformer block: element-wise (metal_vector_add,
// elementwise_mul, silu, gelu, mock_relu, attention_prefill), rms_norm, rope,
// rope_batch, softmax, embedding_lookup, argmax and the attention family
// (causal_attention, causal_attention_cached, flash_attention_cached,
// flash_attention_gqa, flash_attention_paged).
//
// Semantics follow the reference's Metal host code (metal_provider.mm:2313-2990,
// 3034-3079): the f16 variant is picked from the OUTPUT dtype, element counts
// come from the output buffer's size, and push constants are read from the
// task descriptor's 64-byte block whenever its size is non-zero.  Where the
// reference would read or write out of bounds (a buffer smaller than the
// work it implies, a head_dim that does not divide the element count, a
// prefill longer than the cache), this planner returns NF_ERROR_INVALID_ARG.
#include <algorithm>
#include <cstring>
#include <unordered_map>

#include "plan.hpp"

namespace nfhip {
namespace {

struct LayerInfo {
  Path path;
  EwFn fn;
  AttnMode attn;
  bool reads_pc;
  bool f16_capable;  // has an f16 variant selected by the output dtype
  bool append;       // attention op that writes K_new / V_new into the cache first
};

const std::unordered_map<std::string, LayerInfo>& layer_table() {
  static const std::unordered_map<std::string, LayerInfo> t = {
      // metal_provider.mm:3180-3204
      {"metal_vector_add", {Path::Binary, EwFn::Add, AttnMode::Plain, false, true, false}},
      {"elementwise_mul", {Path::Binary, EwFn::Mul, AttnMode::Plain, false, true, false}},
      {"silu", {Path::Unary, EwFn::Silu, AttnMode::Plain, false, true, false}},
      {"gelu", {Path::Unary, EwFn::Gelu, AttnMode::Plain, false, true, false}},
      {"mock_relu", {Path::Unary, EwFn::Relu, AttnMode::Plain, false, false, false}},
      {"attention_prefill", {Path::MockPrefill, EwFn::Mul, AttnMode::Plain, false, false, false}},
      {"rms_norm", {Path::RmsNorm, EwFn::Add, AttnMode::Plain, true, true, false}},
      {"rope", {Path::Rope, EwFn::Add, AttnMode::Plain, true, false, false}},
      {"rope_batch", {Path::RopeBatch, EwFn::Add, AttnMode::Plain, true, true, false}},
      // The name the model layer emits for the f16 rope in fp16 mode
      // (arch_registry.hpp:140, 298-301; kernel metal_provider.mm:1086-1106).
      // The Metal dispatch map (metal_provider.mm:3180-3204) has no entry for
      // it, so there the fp16 rope silently does not run; here it is the f16
      // rope_batch and takes f16 buffers only.
      {"rope_batch_f16", {Path::RopeBatch, EwFn::Add, AttnMode::Plain, true, true, false}},
      {"softmax", {Path::Softmax, EwFn::Add, AttnMode::Plain, true, false, false}},
      {"embedding_lookup", {Path::Embedding, EwFn::Add, AttnMode::Plain, true, true, false}},
      {"argmax", {Path::Argmax, EwFn::Add, AttnMode::Plain, true, false, false}},
      {"causal_attention", {Path::Attention, EwFn::Add, AttnMode::Plain, true, false, false}},
      {"causal_attention_cached", {Path::Attention, EwFn::Add, AttnMode::Cached, true, false, true}},
      {"flash_attention_cached", {Path::Attention, EwFn::Add, AttnMode::Cached, true, true, true}},
      {"flash_attention_gqa", {Path::Attention, EwFn::Add, AttnMode::Gqa, true, true, true}},
      {"flash_attention_paged", {Path::Attention, EwFn::Add, AttnMode::Paged, true, false, false}},
      {"moe_top_k_gating", {Path::MoeGate, EwFn::Add, AttnMode::Plain, true, false, false}},
      {"moe_scatter_gather", {Path::MoeScatter, EwFn::Add, AttnMode::Plain, true, false, false}},
  };
  return t;
}

nf_status fail(std::string* why, const std::string& msg) {
  if (why) *why = msg;
  return NF_ERROR_INVALID_ARG;
}

struct Pc {
  uint32_t seq_len = 0, n_heads = 0, head_dim = 0;
  float eps = 0.f, theta = 0.f;
  uint32_t M = 0, N = 0, K = 0, step = 0, max_seq = 0, window = 0;
  bool present = false;
};

Pc read_pc(const uint8_t* pc, uint32_t size) {
  Pc r;
  if (!pc || size == 0) return r;
  uint8_t b[48] = {};
  std::memcpy(b, pc, size < 48 ? size : 48);
  std::memcpy(&r.seq_len, b + 0, 4);
  std::memcpy(&r.n_heads, b + 4, 4);
  std::memcpy(&r.head_dim, b + 8, 4);
  std::memcpy(&r.eps, b + 12, 4);
  std::memcpy(&r.theta, b + 16, 4);
  std::memcpy(&r.M, b + 20, 4);
  std::memcpy(&r.N, b + 24, 4);
  std::memcpy(&r.K, b + 28, 4);
  std::memcpy(&r.step, b + 32, 4);
  std::memcpy(&r.max_seq, b + 36, 4);
  std::memcpy(&r.window, b + 40, 4);
  r.present = true;
  return r;
}

const char* tname(EType t) { return t == EType::F16 ? "f16" : "f32"; }

bool fits(const nf_tensor_desc* d, uint64_t elems, uint64_t elt) {
  return elt == 0 || elems <= d->size_bytes / elt;
}

constexpr uint64_t kMaxElems = 1ull << 32;  // kernels index with 32-bit element offsets per row/head

nf_status plan_attention(const LayerInfo& info, const char* op_name, const nf_tensor_desc* const* ins,
                         uint32_t n_in, const nf_tensor_desc* const* outs, uint32_t n_out, const Pc& pc,
                         Plan* p, std::string* why) {
  LayerParams& lp = p->lp;
  lp.attn = info.attn;
  const uint32_t need_in = info.attn == AttnMode::Plain ? 3u : info.attn == AttnMode::Paged ? 4u : 5u;
  if (n_in < need_in || n_out < 1) return fail(why, std::string(op_name) + " takes " + std::to_string(need_in) +
                                                        " inputs and 1 output");
  for (uint32_t i = 0; i < need_in; ++i)
    if (!ins[i]) return fail(why, "null input descriptor");
  if (!outs[0]) return fail(why, "null output descriptor");
  if (!pc.present) return fail(why, "attention ops need push constants");
  lp.seq_len = pc.seq_len;
  lp.n_heads = pc.n_heads;
  lp.head_dim = pc.head_dim;
  lp.step = pc.step;
  lp.max_seq = pc.max_seq;
  lp.window = pc.window;
  if (lp.n_heads == 0 || lp.head_dim == 0) return fail(why, "n_heads and head_dim must be non-zero");
  if (lp.head_dim > 256) return fail(why, "head_dim above 256 is not supported");
  // GQA mapping (metal_provider.mm:227-228): pc.M carries n_kv_heads.
  lp.n_kv = (info.attn != AttnMode::Plain && pc.M > 0 && pc.M < pc.n_heads) ? pc.M : pc.n_heads;
  const uint64_t D = lp.head_dim, H = lp.n_heads, KV = lp.n_kv;
  const uint64_t elt = elt_bytes(p->c);
  lp.decode = info.attn != AttnMode::Plain && lp.step > 0;
  const uint64_t nq = lp.decode ? 1 : lp.seq_len;  // query tokens
  p->count = nq * H;                               // (query, head) pairs
  if (info.attn == AttnMode::Plain) {
    // Q, K, V, out: [n_heads, seq_len, head_dim] (metal_provider.mm:166-213)
    const uint64_t n = H * lp.seq_len * D;
    for (int i = 0; i < 3; ++i)
      if (!fits(ins[i], n, elt)) return fail(why, "Q, K and V must hold n_heads*seq_len*head_dim elements");
    if (!fits(outs[0], n, elt)) return fail(why, "output must hold n_heads*seq_len*head_dim elements");
    p->act_bytes = 3 * n * elt;
    p->out_bytes = n * elt;
  } else if (info.attn == AttnMode::Paged) {
    // metal_provider.mm:1622-1712
    lp.block_size = pc.window ? pc.window : 16;
    lp.n_blocks = pc.N;
    lp.q_offset = pc.K;
    const uint64_t rows = (uint64_t)(lp.q_offset + nq) * H * D;
    if (!fits(ins[0], rows, elt)) return fail(why, "Q must hold (K + seq) * n_heads * head_dim elements");
    if (!fits(outs[0], rows, elt)) return fail(why, "output must hold (K + seq) * n_heads * head_dim elements");
    const uint64_t max_pos = lp.decode ? lp.step : (lp.seq_len ? lp.seq_len - 1 : 0);
    const uint64_t used_blocks = std::min<uint64_t>((max_pos + lp.block_size) / lp.block_size, lp.n_blocks);
    if (!fits(ins[3], used_blocks, 4)) return fail(why, "block table holds fewer entries than the blocks used");
    // pools: whole blocks of [n_kv][block_size][head_dim]; a physical index
    // past the pools' end is skipped by the kernel.
    lp.count2 = std::min(ins[1]->size_bytes, ins[2]->size_bytes) / (elt * KV * lp.block_size * D);
    p->weight_bytes = 2 * (max_pos + 1) * KV * D * elt;
    p->act_bytes = nq * H * D * elt;
    p->out_bytes = nq * H * D * elt;
  } else {
    if (!lp.decode) {
      if (lp.seq_len > lp.max_seq) return fail(why, "prefill seq_len exceeds max_seq_len (cache overflow)");
    } else if (lp.step >= lp.max_seq) {
      lp.noop = true;  // metal_provider.mm:284: the reference kernel returns without writing
    }
    const uint64_t cache = KV * lp.max_seq * D;
    if (!fits(ins[3], cache, elt) || !fits(ins[4], cache, elt))
      return fail(why, "caches must hold n_kv * max_seq_len * head_dim elements");
    if (!fits(ins[0], nq * H * D, elt)) return fail(why, "Q is smaller than the query tokens x n_heads x head_dim");
    if (!fits(ins[1], nq * KV * D, elt) || !fits(ins[2], nq * KV * D, elt))
      return fail(why, "K_new / V_new are smaller than the tokens x n_kv x head_dim");
    if (!fits(outs[0], nq * H * D, elt)) return fail(why, "output is smaller than tokens x n_heads x head_dim");
    lp.append = !lp.noop;
    if (lp.append) p->writes_inputs = (1u << 3) | (1u << 4);
    const uint64_t kv_len = lp.decode ? lp.step + 1 : lp.seq_len;
    p->weight_bytes = 2 * kv_len * KV * D * elt;
    p->act_bytes = nq * (H + 2 * KV) * D * elt;
    p->out_bytes = nq * H * D * elt;
  }
  if (nq * H * D >= kMaxElems) return fail(why, "attention problem too large");
  p->kernel = std::string("attention_") +
              (info.attn == AttnMode::Plain ? "plain" : info.attn == AttnMode::Cached ? "cached"
                                                        : info.attn == AttnMode::Gqa  ? "gqa" : "paged") +
              (lp.decode ? "_decode_" : "_prefill_") + tname(p->c);
  return NF_OK;
}

}  // namespace

bool layer_op_known(const char* op_name) {
  return op_name && layer_table().count(op_name) != 0;
}

bool layer_op_reads_push_constants(const char* op_name) {
  if (!op_name) return false;
  auto it = layer_table().find(op_name);
  return it != layer_table().end() && it->second.reads_pc;
}

nf_status make_layer_plan(const char* op_name, const nf_tensor_desc* const* ins, uint32_t n_in,
                          const nf_tensor_desc* const* outs, uint32_t n_out, const uint8_t* pc_bytes,
                          uint32_t pc_size, Plan* plan, std::string* why) {
  auto it = layer_table().find(op_name);
  if (it == layer_table().end()) {
    if (why) *why = std::string("unsupported op '") + op_name + "'";
    return NF_ERROR_UNSUPPORTED_OP;
  }
  const LayerInfo& info = it->second;
  const Pc pc = read_pc(pc_bytes, pc_size);
  Plan p;
  p.op = OpKind::Layer;
  p.path = info.path;
  LayerParams& lp = p.lp;
  lp.fn = info.fn;
  if (!ins && n_in) return fail(why, "null input descriptors");
  if (!outs && n_out) return fail(why, "null output descriptors");
  // The f16 kernel is chosen by the output dtype, as the reference does
  // (is_f16 = out.dtype == F16); ops without one always compute in f32.
  const nf_tensor_desc* out0 = (n_out >= 1 && outs) ? outs[0] : nullptr;
  p.c = (info.f16_capable && out0 && out0->dtype == NF_DTYPE_F16) ? EType::F16 : EType::F32;
  if (std::strcmp(op_name, "rope_batch_f16") == 0 && p.c != EType::F16)
    return fail(why, "rope_batch_f16 takes an f16 output");
  p.a = p.b = p.c;
  const uint64_t elt = elt_bytes(p.c);

  switch (info.path) {
    case Path::Binary: {
      if (n_in < 2 || n_out < 1 || !ins[0] || !ins[1] || !out0) return fail(why, "takes 2 inputs and 1 output");
      p.count = out0->size_bytes / elt;
      if (!fits(ins[0], p.count, elt) || !fits(ins[1], p.count, elt))
        return fail(why, "inputs are smaller than the output");
      p.act_bytes = 2 * p.count * elt;
      p.out_bytes = p.count * elt;
      p.kernel = std::string(info.fn == EwFn::Add ? "vector_add_" : "elementwise_mul_") + tname(p.c);
      break;
    }
    case Path::Unary: {
      if (n_in < 1 || !ins[0]) return fail(why, "takes 1 input");
      // mock_relu without an output writes its input in place (metal_provider.mm:2435-2444).
      const nf_tensor_desc* dst = out0;
      if (!dst) {
        if (info.fn != EwFn::Relu) return fail(why, "takes 1 input and 1 output");
        dst = ins[0];
        p.writes_inputs = 1u;
      }
      p.count = dst->size_bytes / elt;
      if (!fits(ins[0], p.count, elt)) return fail(why, "input is smaller than the output");
      p.act_bytes = p.count * elt;
      p.out_bytes = p.count * elt;
      p.kernel = std::string(info.fn == EwFn::Silu ? "silu_" : info.fn == EwFn::Gelu ? "gelu_" : "relu_") +
                 tname(p.c);
      break;
    }
    case Path::MockPrefill: {
      // k = x * 0.5, v = x * -0.25 (metal_provider.mm:56-66, 2388-2433)
      if (n_in < 1 || n_out < 2 || !ins[0] || !outs[0] || !outs[1])
        return fail(why, "takes 1 input and 2 outputs");
      p.count = outs[0]->size_bytes / 4;
      lp.count2 = outs[1]->size_bytes / 4;
      if (!fits(ins[0], std::max(p.count, lp.count2), 4)) return fail(why, "input is smaller than the outputs");
      p.act_bytes = std::max(p.count, lp.count2) * 4;
      p.out_bytes = (p.count + lp.count2) * 4;
      p.kernel = "attention_prefill_mock_f32";
      break;
    }
    case Path::RmsNorm: {
      // out = x * rsqrt(mean(x^2) + eps) * w per row of head_dim (metal_provider.mm:85-102)
      if (n_in < 2 || n_out < 1 || !ins[0] || !ins[1] || !out0) return fail(why, "takes 2 inputs and 1 output");
      if (!pc.present || pc.head_dim == 0) return fail(why, "rms_norm needs head_dim in the push constants");
      lp.dim = pc.head_dim;
      lp.eps = pc.eps;
      p.count = out0->size_bytes / elt;
      if (p.count % lp.dim != 0) return fail(why, "output elements are not a multiple of head_dim");
      lp.rows = (uint32_t)(p.count / lp.dim);
      if (!fits(ins[0], p.count, elt)) return fail(why, "input is smaller than the output");
      if (!fits(ins[1], lp.dim, 4)) return fail(why, "weights (f32) hold fewer than head_dim elements");
      p.act_bytes = p.count * elt + lp.dim * 4;
      p.out_bytes = p.count * elt;
      p.kernel = std::string("rms_norm_") + tname(p.c);
      break;
    }
    case Path::Rope:
    case Path::RopeBatch: {
      if (n_in < 1 || n_out < 1 || !ins[0] || !out0) return fail(why, "takes 1 input and 1 output");
      if (!pc.present || pc.head_dim == 0 || pc.head_dim % 2 != 0)
        return fail(why, "rope needs an even, non-zero head_dim in the push constants");
      lp.head_dim = pc.head_dim;
      lp.theta = pc.theta;
      lp.step = pc.step;
      lp.n_heads = pc.n_heads;
      if (info.path == Path::RopeBatch && lp.n_heads == 0) return fail(why, "rope_batch needs n_heads");
      p.count = out0->size_bytes / elt;
      if (p.count % lp.head_dim != 0) return fail(why, "output elements are not a multiple of head_dim");
      if (!fits(ins[0], p.count, elt)) return fail(why, "input is smaller than the output");
      p.act_bytes = p.count * elt;
      p.out_bytes = p.count * elt;
      p.kernel = std::string(info.path == Path::Rope ? "rope_" : "rope_batch_") + tname(p.c);
      break;
    }
    case Path::Softmax: {
      // rows = seq_len (1 without push constants), width = head_dim (metal_provider.mm:1002-1030, 2717-2744)
      if (n_in < 1 || n_out < 1 || !ins[0] || !out0) return fail(why, "takes 1 input and 1 output");
      lp.rows = pc.present ? pc.seq_len : 1;
      lp.dim = pc.head_dim;
      if (lp.dim == 0) lp.rows = 0;  // rows of width 0: the reference writes nothing
      p.count = (uint64_t)lp.rows * lp.dim;
      if (!fits(ins[0], p.count, 4) || !fits(out0, p.count, 4))
        return fail(why, "buffers are smaller than seq_len * head_dim floats");
      p.act_bytes = p.count * 4;
      p.out_bytes = p.count * 4;
      p.kernel = "softmax_f32";
      break;
    }
    case Path::Embedding: {
      // out[t, :] = weights[ids[t], :] (metal_provider.mm:1054-1067, 2795-2826)
      if (n_in < 2 || n_out < 1 || !ins[0] || !ins[1] || !out0) return fail(why, "takes 2 inputs and 1 output");
      if (!pc.present || pc.head_dim == 0) return fail(why, "embedding_lookup needs head_dim in the push constants");
      lp.dim = pc.head_dim;
      lp.seq_len = pc.seq_len;
      p.count = out0->size_bytes / elt;
      const uint64_t tokens = std::min<uint64_t>(lp.seq_len, (p.count + lp.dim - 1) / lp.dim);
      if (!fits(ins[1], tokens, 4)) return fail(why, "token id buffer holds fewer than seq_len int32 ids");
      lp.rows = (uint32_t)(ins[0]->size_bytes / (elt * lp.dim));  // vocabulary rows present
      p.act_bytes = tokens * (4 + lp.dim * elt);
      p.out_bytes = std::min<uint64_t>(p.count, tokens * lp.dim) * elt;
      p.kernel = std::string("embedding_lookup_") + tname(p.c);
      break;
    }
    case Path::Argmax: {
      // one int32 per row of N floats, rows = seq_len (metal_provider.mm:1601-1619, 2828-2855)
      if (n_in < 1 || n_out < 1 || !ins[0] || !out0) return fail(why, "takes 1 input and 1 output");
      lp.rows = pc.present ? pc.seq_len : 1;
      lp.dim = pc.N;  // N = 0: the reference's scan never leaves index 0, so every row gets 0
      p.count = lp.rows;
      if (!fits(ins[0], (uint64_t)lp.rows * lp.dim, 4)) return fail(why, "input is smaller than seq_len * N floats");
      if (!fits(out0, lp.rows, 4)) return fail(why, "output holds fewer than seq_len int32");
      p.act_bytes = (uint64_t)lp.rows * lp.dim * 4;
      p.out_bytes = lp.rows * 4ull;
      p.kernel = "argmax_f32";
      break;
    }
    case Path::MoeGate: {
      // gate logits [batch, n_experts] -> expert ids (int32) and weights (f32),
      // [batch, top_k] each; batch = seq_len, n_experts = M, top_k = min(N, 8)
      // (metal_provider.mm:1907-1962, host 3080-3112)
      if (n_in < 1 || n_out < 2 || !ins[0] || !out0 || !outs[1]) return fail(why, "takes 1 input and 2 outputs");
      lp.rows = pc.present ? pc.seq_len : 1;
      lp.n_experts = pc.M;
      lp.top_k = std::min<uint32_t>(pc.N, 8);
      p.count = (uint64_t)lp.rows * lp.top_k;
      if (!fits(ins[0], (uint64_t)lp.rows * lp.n_experts, 4)) return fail(why, "logits hold fewer than seq_len * M floats");
      if (!fits(out0, p.count, 4) || !fits(outs[1], p.count, 4))
        return fail(why, "outputs hold fewer than seq_len * min(N, 8) entries");
      p.act_bytes = (uint64_t)lp.rows * lp.n_experts * 4;
      p.out_bytes = p.count * 8;
      p.kernel = "moe_top_k_gating_f32";
      break;
    }
    case Path::MoeScatter: {
      // expert outputs [rows, dim], ids and weights [batch, top_k] -> out
      // [batch, dim]; batch = seq_len, top_k = N, dim = K
      // (metal_provider.mm:1964-1997, host 3114-3150)
      if (n_in < 3 || n_out < 1 || !ins[0] || !ins[1] || !ins[2] || !out0) return fail(why, "takes 3 inputs and 1 output");
      lp.rows = pc.present ? pc.seq_len : 1;
      lp.top_k = pc.N;
      lp.dim = pc.K;
      lp.n_experts = lp.dim ? (uint32_t)std::min<uint64_t>(ins[0]->size_bytes / (4ull * lp.dim), 0xFFFFFFFFu) : 0;
      p.count = (uint64_t)lp.rows * lp.dim;
      if (!fits(ins[1], (uint64_t)lp.rows * lp.top_k, 4) || !fits(ins[2], (uint64_t)lp.rows * lp.top_k, 4))
        return fail(why, "ids / weights hold fewer than seq_len * N entries");
      if (!fits(out0, p.count, 4)) return fail(why, "output holds fewer than seq_len * K floats");
      p.act_bytes = (uint64_t)lp.rows * lp.top_k * (8 + 4ull * lp.dim);
      p.out_bytes = p.count * 4;
      p.kernel = "moe_scatter_gather_f32";
      break;
    }
    case Path::Attention: {
      nf_status st = plan_attention(info, op_name, ins, n_in, outs, n_out, pc, &p, why);
      if (st != NF_OK) return st;
      break;
    }
    default:
      return fail(why, "internal: unplanned layer op");
  }
  *plan = p;
  return NF_OK;
}

}  // namespace nfhip
