// ref_fused.cpp — TEST INFRASTRUCTURE ONLY.
//
// The reference's own fused-kernel test, tests/driver/fused_matmul_test.cpp,
// compiled where it lies under the reference tree and linked against this
// repository's HIP provider: four cases (M, N, K) = (4, 8, 32), (5, 7, 64),
// (64, 128, 256) with f32 activations and (64, 128, 256) with f16, each
// comparing the fused op (dequant_q4_0_linear[_f16]) with the separate
// dequant_q4_0[_f16] -> linear_tiled / linear pipeline, dispatched through the
// test's FakeTaskDesc push-constant convention (fused_matmul_test.cpp:108-126).
//
// The test was written for macOS: it defines a file-static `sync()`, which on
// Linux collides with the `sync(void)` that <unistd.h> declares (reached
// through the engine headers).  Every header the test includes is included
// here first, so their include guards make the test's own includes no-ops,
// and the test's function is renamed with a macro for the span of the
// #include.  Nothing of the test is copied or edited.
#include <unistd.h>

#include <algorithm>
#include <cassert>
#include <cmath>
#include <cstdio>
#include <cstdlib>
#include <cstring>
#include <random>
#include <vector>

#include "neuralOS/ddi/neuro_buffer_abi.h"
#include "neuralOS/ddi/neuro_fabric_abi.h"
#include "neuralOS/ddi/neuro_scheduler_abi.h"
#include "neuralOS/kernel/PipelineEngine.hpp"

#define sync nf_fused_matmul_test_sync
#include "tests/driver/fused_matmul_test.cpp"
#undef sync
