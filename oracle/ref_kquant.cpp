// ref_kquant.cpp — TEST INFRASTRUCTURE ONLY.
//
// Exposes the reference's own CPU dequantizers, the file-static
// ref_dequant_q4_1 .. ref_dequant_q5_k of tests/driver/kquant_dequant_test.cpp
// (lines 118-224), to the oracle pins through one C entry point.  The test
// file is compiled from where it lies under the reference tree (this file
// only includes it, renaming its main); nothing of it is copied here.  Its
// main refers to the provider's registration entry points, so the library
// links against libnf_plugin_hip.so, whose code it never calls.
#define main nf_ref_kquant_dequant_test_main
#include "tests/driver/kquant_dequant_test.cpp"
#undef main

namespace {

template <typename Block, typename Fn>
int run(const uint8_t* blocks, int n_blocks, float* out, int elems, Fn fn) {
  for (int b = 0; b < n_blocks; ++b) {
    Block blk;
    std::memcpy(&blk, blocks + (size_t)b * sizeof(Block), sizeof(Block));
    fn(&blk, out + (size_t)b * elems);
  }
  return 0;
}

}  // namespace

// fmt uses the oracle's numbering: 2 q4_1, 3 q5_0, 4 q5_1, 5 q2_k, 6 q3_k,
// 7 q4_k, 8 q5_k.  Returns -1 for any other format.
extern "C" int nfref_kquant_dequant(int fmt, const uint8_t* blocks, int n_blocks, float* out) {
  switch (fmt) {
    case 2: return run<block_q4_1>(blocks, n_blocks, out, 32, ref_dequant_q4_1);
    case 3: return run<block_q5_0>(blocks, n_blocks, out, 32, ref_dequant_q5_0);
    case 4: return run<block_q5_1>(blocks, n_blocks, out, 32, ref_dequant_q5_1);
    case 5: return run<block_q2_k>(blocks, n_blocks, out, 256, ref_dequant_q2_k);
    case 6: return run<block_q3_k>(blocks, n_blocks, out, 256, ref_dequant_q3_k);
    case 7: return run<block_q4_k>(blocks, n_blocks, out, 256, ref_dequant_q4_k);
    case 8: return run<block_q5_k>(blocks, n_blocks, out, 256, ref_dequant_q5_k);
    default: return -1;
  }
}
