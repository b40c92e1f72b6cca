/*
 * TEST INFRASTRUCTURE — the CPU oracle for the PowerSparse hot path.
 *
 * This is a plain C++17 restatement of the reference algorithm, used ONLY as the
 * checker: by tests/, by __graft_entry__.smoke() and by bench.py's cpu_baseline
 * leg. The product (powersparse_amd/) never links, loads or calls it.
 *
 * Reference files restated (ParCIS/PowerSparse):
 *   utils/matrix_utils.cu:31-663   preprocessing into block/residue worksets
 *   utils/matrix_utils.h:8-10      GROUP_SIZE / CEIL / FLOOR
 *   benchmarks/benchmark.cu:64-96  CheckSpmm / CheckSddmm (double accumulation)
 *   benchmarks/benchmark_utils.h:100-104  DenseInput (std::mt19937 % 3 / 10)
 *
 * Parity pins (tests/test_oracle_*.py): hand-derived worksets for tiny CSRs,
 * an independent brute-force Python restatement on random tiny graphs, the
 * reference's own multiset invariant (benchmark.cu:45-62), closed forms for the
 * products, and the C++-standard value of mt19937's 10000th output.
 */
#ifndef POWERSPARSE_ORACLE_H
#define POWERSPARSE_ORACLE_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

typedef struct or_worksets or_worksets;

/* Runs the full preprocessing of matrix_utils.cu:470-663 for a CSR on the CPU.
 * cu_count plays the role of cudaDeviceProp::multiProcessorCount
 * (matrix_utils.cu:37-42). Returns NULL and fills err on invalid input, with
 * the reference's exception messages (matrix_utils.cu:475-488). */
or_worksets* or_preprocess(int rows, int cols, int nnz, const int* row_ptr,
                           const int* col_ind, const float* sp_data, int cu_count,
                           char* err, int err_len);
void or_free(or_worksets* w);

int or_group_type_num(const or_worksets* w);
int or_group_num(const or_worksets* w, int s);
int or_signature_len(const or_worksets* w);
/* number of nonzeros stored in workset s */
long long or_workset_len(const or_worksets* w, int s);
/* final worksets: col/val of length or_workset_len, des of length group_num */
void or_copy_workset(const or_worksets* w, int s, int* col, float* val, int* des);
/* final residue offsets (G0+1) and atomic flags (G0, 0/1 bytes) */
void or_copy_residue(const or_worksets* w, int* offset, uint8_t* atomic);

/* intermediates, for stage-by-stage parity of the GPU preprocessing */
void or_copy_col_nnz(const or_worksets* w, int* col_nnz);        /* cols */
void or_copy_ranked_pos(const or_worksets* w, int* pos);         /* nnz: CSR positions in (row, col_nnz desc) order */
void or_copy_sigbit(const or_worksets* w, int* sigbit);          /* cols */
void or_copy_initial_des(const or_worksets* w, int s, int* des); /* group_num[s], row order */
void or_copy_initial_residue(const or_worksets* w, int* offset, uint8_t* atomic);
/* signature words of workset s, word-major: sig[word * G + g], L/32 words
 * (left untouched when the workset was ordered by bit lists) */
void or_copy_signature(const or_worksets* w, int s, uint32_t* sig);
/* 1 if workset s kept its signature bitmaps (ordered by the per-word sorts) */
int or_has_signature(const or_worksets* w, int s);
/* group permutation of workset s: sorted position -> initial group id */
void or_copy_group_perm(const or_worksets* w, int s, int* perm);

/* AnalyzeMatrix (matrix_utils.cu:31-63): number of worksets S for cu_count. */
int or_analyze_group_type_num(int rows, const int* row_ptr, int cu_count);

/* GenerateSigBit, FFC mode with ffc (matrix_utils.cu:65-128). Returns L. */
int or_generate_sigbit(int cols, const int* col_nnz, int ffc, int* sigbit);

/* How or_preprocess orders groups by signature (the order of the per-word
 * stable sorts, matrix_utils.cu:588-593, either way): 0 = bitmaps unless
 * groups x L/32 exceeds 2^28 words, then bit lists; 1 = always the per-word
 * sorts of the bitmaps; 2 = always the bit lists. Process-wide. */
void or_set_signature_order(int mode);
/* Caps the workset count S of later or_preprocess calls (0: no cap). An
 * extension for the product's capped partitions; with the cap at or above S
 * the partition is the reference's. */
void or_set_max_group_types(int cap);

/* The stable descending-signature order of `groups` groups given as sets of
 * signature bits: group g's bits are bits[begin[g] .. begin[g+1]) (any order,
 * duplicates allowed). perm[k] = group at position k. */
void or_order_bit_lists(int groups, const int* begin, const int* bits, int* perm);

/* CheckSpmm (benchmark.cu:64-77): C[r,j] = sum_p double(val[p]) * B[col[p],j]
 * in double. mag (optional) receives sum_p |val[p]| * |B[col[p],j]|. */
void or_spmm(int rows, const int* row_ptr, const int* col_ind, const float* sp_data,
             int n, const float* B, double* C, double* mag, int threads);

/* CheckSddmm (benchmark.cu:79-96) for one workset given as groups with
 * destination rows and offsets: out[p] = val[p] * sum_j X[row,j] * Y[col[p],j]
 * in double. mag (optional) receives |val[p]| * sum_j |X[row,j] * Y[col[p],j]|. */
void or_sddmm(int groups, const int* des, const int* offsets, const int* col_ind,
              const float* sp_data, int k, const float* X, const float* Y,
              double* out, double* mag, int threads);

/* DenseInput (benchmark_utils.h:100-104) drawn from one std::mt19937(seed):
 * first n1 values into out1 (may be 0), then n2 values into out2 — the order
 * the reference harness draws lhs then rhs (benchmark.cu:137-140). */
void or_dense_input(unsigned seed, size_t n1, float* out1, size_t n2, float* out2);

/* raw std::mt19937 output number `index` (1-based) for a seed */
uint32_t or_mt19937_nth(unsigned seed, long long index);

/* number of OpenMP threads the checks would use */
int or_max_threads(void);

#ifdef __cplusplus
}
#endif

#endif
