// exl3_dense.h -- plain dense GEMMs through hipBLASLt, for the resident
// matrices (decoded and un-rotated weights kept in HBM).  Row-major operands:
//   Y[rows, n] = X[rows, k] @ W[k, n]   (W's rows ldw elements apart, ldw >= n)
// in one element type for X and W (f16 / bf16 / f32), Y in `ydt`, products
// summed in f32.  One handle and one workspace per (device, stream); the
// algorithm per shape is asked of hipBLASLt's heuristic once and kept.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace exl3 {

enum DenseType { DENSE_F16 = 0, DENSE_BF16 = 1, DENSE_F32 = 2 };

// Returns hipSuccess, a HIP error, or hipErrorNotSupported when hipBLASLt has
// no algorithm for the shape.  Allocates the stream's workspace at its first
// call (so that first call must not be under graph capture).
hipError_t dense_gemm(const void *x, int xdt, const void *w, int64_t ldw, void *y, int ydt,
                      int64_t rows, int64_t k, int64_t n, hipStream_t s);

}  // namespace exl3
