// Once-per-bank dictionary normalization as a launch of its own (the module
// forward runs the same work inside its projection launch); the work and the
// layouts are described in dict_norm.h.
#include "dict_norm.h"

namespace da {

__global__ __launch_bounds__(256) void dict_normalize_kernel(NormJob job) {
  __shared__ __attribute__((aligned(16))) char lds[kNormLdsBytes];
  normalize_block(job, static_cast<int>(blockIdx.x), lds);
}

void launch_dictionary_normalize(const void* raw_key, const void* raw_value, int in_dtype, int R,
                                 int M, float eps, void* key_t, int key_dtype, void* value,
                                 void* value_rows, hipStream_t stream) {
  const NormJob job{raw_key, raw_value, in_dtype, R, M, static_cast<int>(round_up(M, kAtomPad)), eps,
                    key_t, key_dtype, value, value_rows};
  hipLaunchKernelGGL(dict_normalize_kernel, dim3(norm_blocks(job)), dim3(256), 0, stream, job);
}

}  // namespace da
