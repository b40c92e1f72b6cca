// SDDMM (edge messaging): out = (lhs * rhs^T) sampled at A's nonzeros, times A.
//
// Same entry point as the reference (ParCIS/PowerSparse
// PowerSparse_SDDMM/PowerSparse_SDDMM.h:11-18), with ps_stream_t for the stream.
#ifndef POWERSPARSE_SDDMM_H
#define POWERSPARSE_SDDMM_H

#include "matrix_utils.h"

namespace PowerSparse {

// FP32 sampled (lhs * rhs^T) times sparse values. Dense inputs are row-major.
// Output is in workset order, not original CSR order: sddmm_output_gpu[s] holds
// GroupNum()[s] * GROUP_SIZE(s) floats for s > 0 and ResidueOffset()[GroupNum()[0]]
// floats for s == 0. Zero every output workset before each independent call.
// Streams follow SpMM. The reference accepts N = 32 or 128; this build accepts
// any multiple of 32 up to 512 (N = 64 is used by the community-graph config).
void SDDMM(const PowerSparseMatrixGPU& ps_matrix_gpu, int N, const float* lhs_gpu,
           const float* rhs_gpu, float** sddmm_output_gpu, int ps_stream_num,
           const ps_stream_t* ps_stream);

// Not in the reference: one launch on one stream, no device synchronisation.
void SDDMMAsync(const PowerSparseMatrixGPU& ps_matrix_gpu, int N, const float* lhs_gpu,
                const float* rhs_gpu, float* const* sddmm_output_gpu, ps_stream_t stream);

// Not in the reference: SDDMM with the output in the input CSR's order,
// out_csr[p] for the p-th nonzero of the CSR arrays the matrix was built from
// (MatrixNNZ() floats, no zeroing needed; every entry is written). One launch
// on `stream`, no device synchronisation. The matrix must have been built with
// PartitionPolicy::csr_positions.
void SDDMMToCSR(const PowerSparseMatrixGPU& ps_matrix_gpu, int N, const float* lhs_gpu,
                const float* rhs_gpu, float* out_csr_gpu, ps_stream_t stream = nullptr);

// Not in the reference: moves workset-order per-nonzero values (e.g. SDDMM
// outputs) into CSR order, out_csr[WorksetCSRPosition()[s][p]] = values[s][p].
// Same matrix requirement as SDDMMToCSR.
void WorksetToCSR(const PowerSparseMatrixGPU& ps_matrix_gpu, const float* const* values_gpu,
                  float* out_csr_gpu, ps_stream_t stream = nullptr);

}  // namespace PowerSparse

#endif  // POWERSPARSE_SDDMM_H
