/*
 * powersparse.h — C facade over the C++17 PowerSparse API, for FFI callers
 * (Python ctypes, cgo, JNI, N-API) that cannot bind C++ classes.
 *
 * Each function wraps one C++ entry point of powersparse_amd/host, which keeps
 * the reference's interface (ParCIS/PowerSparse); the citation names the
 * reference declaration it stands for. Status codes and ps_stream_t come from
 * powersparse_hip.h. C++ exceptions never cross this boundary: std::invalid_argument
 * maps to PS_ERR_INVALID, every other exception to PS_ERR_RUNTIME, and the text
 * is available from psx_last_error() on the calling thread.
 *
 * Device pointers (B, C, lhs, rhs, outputs, workset arrays) are raw device
 * addresses, e.g. from ps_malloc.
 */
#ifndef POWERSPARSE_H
#define POWERSPARSE_H

#include <stddef.h>
#include <stdint.h>

#include "powersparse_hip.h"

#ifdef __cplusplus
extern "C" {
#endif

typedef struct psx_matrix psx_matrix;
typedef struct psx_csr psx_csr;

const char* psx_last_error(void);

/* Builds the worksets on the current device.
 * Replaces: PowerSparseMatrixGPU::PowerSparseMatrixGPU (utils/matrix_utils.h:22-23).
 * cu_count == 0 uses the device's multiProcessorCount (matrix_utils.cu:37-39);
 * a positive value reproduces the partition the reference would compute on a
 * device with that many SMs/CUs. timings_ms (optional) receives 9 stage times:
 * upload, analyze, rank, groups, sigbit, signature, order, gather, total — the
 * device is synchronised between stages only when it is non-null. */
int psx_matrix_create(int rows, int cols, int nnz, const int* row_ptr, const int* col_ind,
                      const float* sp_data, int cu_count, double* timings_ms,
                      psx_matrix** out);

/* Build options of psx_matrix_create_ex. signature_order picks how groups are
 * put in signature order (both give the reference's order,
 * matrix_utils.cu:588-593): PSX_ORDER_AUTO, PSX_ORDER_BITMAP_WORDS (per-word
 * sorts of the groups x L/32 signature bitmaps) or PSX_ORDER_BIT_LISTS (sorted
 * bit lists, memory bounded by nnz). */
enum { PSX_ORDER_AUTO = 0, PSX_ORDER_BITMAP_WORDS = 1, PSX_ORDER_BIT_LISTS = 2 };
/* Tiers of the dense hub block (PowerSparse::kHubMaxTiers). */
#define PSX_HUB_MAX_TIERS 3
typedef struct psx_build_options {
  int cu_count;
  int signature_order;
  int csr_positions; /* nonzero: keep each nonzero's CSR position (psx_sddmm_csr) */
  int task_order;    /* PSX_TASK_AUTO, PSX_TASK_SIGNATURE or PSX_TASK_ROW */
  int stored_order;  /* nonzero: no locality run order (PartitionPolicy::run_order off) */
  int max_group_types; /* cap on the workset count S (0: none) */
  int parity_spmm;   /* nonzero: SpMM on the public worksets (SpmmPartition::kParity) */
  int no_hub_block;  /* nonzero: no dense hub block (HubBlock::kOff) */
  /* explicit hub block tiers (PartitionPolicy::hub_min_degree / hub_min_count):
   * the leading pairs with both values > 0, degrees decreasing */
  int hub_min_degree[PSX_HUB_MAX_TIERS];
  int hub_min_count[PSX_HUB_MAX_TIERS];
} psx_build_options;
/* Group order the operators run in (same results; TaskOrder in matrix_utils.h):
 * the public signature order, or a row-ordered execution copy kept when it
 * scores better for gather locality (AUTO) or on request (ROW). */
enum { PSX_TASK_AUTO = 0, PSX_TASK_SIGNATURE = 1, PSX_TASK_ROW = 2 };
/* psx_matrix_create with options (NULL: all defaults). No reference counterpart. */
int psx_matrix_create_ex(int rows, int cols, int nnz, const int* row_ptr, const int* col_ind,
                         const float* sp_data, const psx_build_options* options,
                         double* timings_ms, psx_matrix** out);
/* The signature order method the build used (PSX_ORDER_BITMAP_WORDS or
 * PSX_ORDER_BIT_LISTS). No reference counterpart. */
int psx_matrix_signature_order(const psx_matrix* m, int* method);
/* The task order the build chose (PSX_TASK_SIGNATURE or PSX_TASK_ROW) and the
 * locality scores compared (0 when not computed); outputs may be NULL. */
int psx_matrix_task_order(const psx_matrix* m, int* order, double* score_signature,
                          double* score_row);
/* Whether the operators run in the locality run order (RunOrderUsed()). No
 * reference counterpart. */
int psx_matrix_run_order(const psx_matrix* m, int* used);
/* The workset count of the partition SpMM runs on (the tuned one, or
 * GroupTypeNum() when SpMM runs on the public worksets). No reference
 * counterpart. */
int psx_matrix_spmm_worksets(const psx_matrix* m, int* group_type_num);
/* The dense hub block the build chose: its number of tiers (HubTiers()) and
 * tier `tier`'s rows x columns (0 x 0 beyond the last); outputs may be NULL.
 * No reference counterpart. */
int psx_matrix_hub_block(const psx_matrix* m, int* tiers, int tier, int* rows, int* cols);
/* Replaces: ~PowerSparseMatrixGPU (matrix_utils.h:24). */
int psx_matrix_destroy(psx_matrix* m);
/* Replaces: MatrixRow/MatrixCol/MatrixNNZ/GroupTypeNum/GroupFineSize (matrix_utils.h:30-34);
 * any output may be NULL. */
int psx_matrix_info(const psx_matrix* m, int* rows, int* cols, int* nnz, int* group_type_num,
                    int* fine, int* signature_len, int* cu_count);
/* Replaces: GroupNum() (matrix_utils.h:35); writes GroupTypeNum() ints. */
int psx_matrix_group_num(const psx_matrix* m, int* group_num);
/* Replaces: WorksetColInd()[s], WorksetSpData()[s], GroupDestination()[s]
 * (matrix_utils.h:36-38); device pointers, NULL for an empty workset. */
int psx_matrix_workset(const psx_matrix* m, int s, const int** col_ind, const float** sp_data,
                       const int** group_des);
/* Replaces: ResidueOffset(), ResidueAtomic() (matrix_utils.h:39-40). */
int psx_matrix_residue(const psx_matrix* m, const int** offset, const uint8_t** atomic);

/* Replaces: PowerSparse::SpMM (PowerSparse_SpMM/PowerSparse_SpMM.h:14-17). */
int psx_spmm(const psx_matrix* m, int N, const float* B, float* C, int stream_count,
             const ps_stream_t* streams);
/* One launch on `stream`, no device synchronisation (no reference counterpart). */
int psx_spmm_async(const psx_matrix* m, int N, const float* B, float* C, ps_stream_t stream);
/* Replaces: PowerSparse::SDDMM (PowerSparse_SDDMM/PowerSparse_SDDMM.h:14-18). */
int psx_sddmm(const psx_matrix* m, int N, const float* lhs, const float* rhs, float** out,
              int stream_count, const ps_stream_t* streams);
int psx_sddmm_async(const psx_matrix* m, int N, const float* lhs, const float* rhs,
                    float* const* out, ps_stream_t stream);
/* SDDMM into CSR order: out_csr holds MatrixNNZ floats, entry p for the p-th
 * nonzero of the input CSR (no zeroing needed). One launch on `stream`. Needs a
 * matrix built with csr_positions. Replaces: the caller-side permutation of the
 * reference's workset-order output (PowerSparse_SDDMM.h:11-12). */
int psx_sddmm_csr(const psx_matrix* m, int N, const float* lhs, const float* rhs,
                  float* out_csr, ps_stream_t stream);
/* Workset-order per-nonzero values (values[s], as SDDMM writes them) into CSR
 * order. Needs a matrix built with csr_positions. Same replacement. */
int psx_workset_to_csr(const psx_matrix* m, const float* const* values, float* out_csr,
                       ps_stream_t stream);
/* Device array of workset s: CSR position of each stored nonzero (NULL if the
 * matrix was built without csr_positions or the workset is empty). */
int psx_matrix_csr_position(const psx_matrix* m, int s, const int** pos);

/* ------------------------------------------------------ host CSR inputs */
/* Replaces: ReadMatrixMarket (benchmarks/matrix_market.cpp:97-134). */
int psx_csr_read_mtx(const char* path, psx_csr** out);
/* Binary CSR ("PSCSR001"); no reference counterpart. */
int psx_csr_read_binary(const char* path, psx_csr** out);
int psx_csr_write_binary(const psx_csr* csr, const char* path);
/* Seeded synthetic graphs "C0".."C4" (no reference counterpart); scale >= 1
 * divides the node count. */
int psx_csr_synth(const char* config, uint64_t seed, int scale, psx_csr** out);
int psx_csr_chung_lu(int n, double gamma, double mean_deg, double max_deg, float val_lo,
                     float val_hi, uint64_t seed, psx_csr** out);
int psx_csr_uniform_degree(int rows, int cols, int deg_lo, int deg_hi, float val_lo,
                           float val_hi, uint64_t seed, psx_csr** out);
int psx_csr_community(int communities, int block, double p_intra, double inter_mean,
                      double empty_frac, double single_frac, float val_lo, float val_hi,
                      uint64_t seed, psx_csr** out);
int psx_csr_info(const psx_csr* csr, int* rows, int* cols, int* nnz);
/* Host pointers owned by the csr handle. */
int psx_csr_arrays(const psx_csr* csr, const int** row_ptr, const int** col_ind,
                   const float** values);
int psx_csr_free(psx_csr* csr);

/* ------------------------------------------- host steps of preprocessing */
/* Replaces: GenerateSigBit, FFC mode (utils/matrix_utils.cu:65-128). */
int psx_generate_sigbit(int cols, const int* col_nnz, int ffc, int* sigbit, int* signature_len);
/* Replaces: AnalyzeMatrix's workset count (utils/matrix_utils.cu:31-63) from
 * degree_sums[s] = sum_r floor(deg_r / GROUP_SIZE(s)), s = 0..31 (entry 0 unused). */
int psx_workset_count(const unsigned long long* degree_sums, int cu_count, int* group_type_num);
/* Replaces: DenseInput (benchmarks/benchmark_utils.h:100-104): one std::mt19937(seed),
 * n1 values then n2 values of (rng() % 3) / 10. */
int psx_dense_input(unsigned seed, size_t n1, float* out1, size_t n2, float* out2);

#ifdef __cplusplus
}
#endif

#endif /* POWERSPARSE_H */
