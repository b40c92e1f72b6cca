// SpMM (node aggregation): C = A * B with A a PowerSparseMatrixGPU.
//
// Same entry point as the reference (ParCIS/PowerSparse
// PowerSparse_SpMM/PowerSparse_SpMM.h:11-17); the CUDA stream type becomes the
// opaque ps_stream_t of the C ABI, so this header pulls in no GPU runtime.
#ifndef POWERSPARSE_SPMM_H
#define POWERSPARSE_SPMM_H

#include "matrix_utils.h"

namespace PowerSparse {

// FP32 C = A * B, with row-major B and C. Zero C before each independent call.
// Supply GroupTypeNum() streams (null is allowed for a single workset).
// Multiple worksets synchronize the device; a single workset uses the default stream.
// N must be a positive multiple of 32 with N/32 <= 65535.
void SpMM(const PowerSparseMatrixGPU& ps_matrix_gpu, int N, const float* B_gpu, float* C_gpu,
          int ps_stream_num, const ps_stream_t* ps_stream);

// Not in the reference: the same operator enqueued on one stream without the
// device synchronisation (one launch covers every workset).
void SpMMAsync(const PowerSparseMatrixGPU& ps_matrix_gpu, int N, const float* B_gpu,
               float* C_gpu, ps_stream_t stream);

}  // namespace PowerSparse

#endif  // POWERSPARSE_SPMM_H
