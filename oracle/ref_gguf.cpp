// oracle/ref_gguf.cpp — opens a GGUF file with the reference's own loader
// (model/model/gguf_loader.hpp) and tokenizer (model/model/tokenizer.hpp) and
// prints what they parsed, so a test can check that a synthetic model file is
// one the reference's applications accept.  Test infrastructure only.
//
//   ref_gguf <file.gguf> "<prompt>"
#include "model/model/gguf_loader.hpp"
#include "model/model/tokenizer.hpp"

#include <cstdio>

int main(int argc, char** argv) {
    if (argc < 3) { std::fprintf(stderr, "usage: ref_gguf <file> <prompt>\n"); return 2; }
    nf::GGUFModel* m = nf::gguf_open(argv[1]);
    if (!m) return 1;
    std::printf("arch=%s dim=%u layers=%u heads=%u kv_heads=%u ff=%u vocab=%u ctx=%u "
                "theta=%g eps=%g tensors=%zu\n",
                m->architecture.c_str(), m->dim, m->n_layers, m->n_heads, m->n_kv_heads,
                m->ff_dim, m->vocab_size, m->max_seq, m->rope_theta, m->rms_norm_eps,
                m->tensors.size());
    for (const auto& kv : m->tensors) {
        const auto& t = kv.second;
        std::printf("tensor %s type=%u elems=%llu bytes=%zu first=%02x\n", kv.first.c_str(),
                    t.gguf_dtype, (unsigned long long)t.n_elements, t.byte_size,
                    t.byte_size ? ((const unsigned char*)t.data)[0] : 0u);
    }
    nf::Tokenizer tok(*m);
    auto ids = tok.encode(argv[2]);
    std::printf("ids");
    for (int id : ids) std::printf(" %d", id);
    std::printf("\ndecoded=%s\n", tok.decode(ids).c_str());
    nf::gguf_close(m);
    return 0;
}
