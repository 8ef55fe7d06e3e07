// Host-side launchers of the hand-written gfx950 kernels.  All take device
// pointers and a stream, enqueue asynchronously, and return 0 / -1.
#pragma once
#include <hip/hip_runtime.h>

#include <cstdint>

namespace nship {

// gemm.hip
int launch_gemm(const float* A, const float* B, float* C, int64_t M, int64_t N, int64_t K,
                int64_t lda, int64_t ldb, int64_t ldc, bool tA, bool tB, int act, hipStream_t s);

}  // namespace nship
