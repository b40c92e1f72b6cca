/*
 * powersparse_hip.h — the C ABI of the MI355X (gfx950) PowerSparse engine.
 *
 * Every entry point is `extern "C"`, takes plain pointers and sizes, returns an
 * int status (PS_OK == 0) and leaves a message for ps_last_error() on failure.
 * No C++, HIP or CUDA type crosses this boundary: streams and events are opaque
 * handles, device buffers are raw device pointers obtained from ps_malloc.
 *
 * The reference (ParCIS/PowerSparse) has no C ABI: its .cu files call the CUDA
 * runtime and launch kernels directly. Each declaration below names the
 * reference code whose role it takes over (file:line in the reference tree).
 * The C++17 host library (powersparse_amd/host) is the only in-tree caller; its
 * public headers keep the reference's C++ API (PowerSparse_SpMM.h,
 * PowerSparse_SDDMM.h, matrix_utils.h).
 *
 * Threading: calls are thread-compatible, not thread-safe on the same output.
 * All launches are asynchronous on the given stream unless stated otherwise.
 */
#ifndef POWERSPARSE_HIP_H
#define POWERSPARSE_HIP_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define PS_OK 0
#define PS_ERR_INVALID 1  /* bad argument; the reference throws std::invalid_argument */
#define PS_ERR_RUNTIME 2  /* HIP runtime failure; the reference's CUDA_CALL throws std::runtime_error */

/* A null stream means the device's default (null) stream. */
typedef struct ps_stream_s* ps_stream_t;
typedef struct ps_event_s* ps_event_t;

/* Message of the last failed call on this thread ("" if none).
 * Replaces: CheckCuda's exception text (utils/cuda_utils.h:7-12). */
const char* ps_last_error(void);

/* ---------------------------------------------------------------- device */
typedef struct ps_device_props {
  char name[256];       /* marketing name */
  char arch[64];        /* gcnArchName, e.g. "gfx950:sramecc+:xnack-" */
  int cu_count;         /* multiProcessorCount */
  int major, minor;
  int lds_per_block;    /* sharedMemPerBlock, bytes */
  int l2_bytes;
  int clock_khz;
  int mem_clock_khz;
  int mem_bus_width;
  size_t global_mem;
} ps_device_props;

/* Replaces: cudaSetDevice / cudaFree(nullptr) (benchmarks/benchmark.cu:116-117). */
int ps_set_device(int device);
int ps_get_device(int* device);
int ps_device_count(int* count);
/* Replaces: cudaGetDeviceProperties (benchmark.cu:118-120, matrix_utils.cu:37-39). */
int ps_get_device_props(int device, ps_device_props* props);
/* Replaces: cudaRuntimeGetVersion / cudaDriverGetVersion (benchmark.cu:121-123). */
int ps_runtime_version(int* version);
int ps_driver_version(int* version);
/* Replaces: cudaDeviceSynchronize (spmm_solution.cu:33, sddmm_solution.cu:49). */
int ps_device_synchronize(void);

/* ---------------------------------------------------------------- memory */
/* Replaces: cudaMalloc / cudaFree (matrix_utils.cu:628-633, matrix_utils.h:43-55,
 * benchmark_utils.h:13-37). ps_free(NULL) is a no-op. */
int ps_malloc(void** ptr, size_t bytes);
int ps_free(void* ptr);
/* Debugging aid, no reference counterpart. With the environment variable
 * PS_DEVICE_GUARD set to a byte count when the library is first used, every
 * device block the library allocates (ps_malloc, and the temporaries of the
 * entry points below) is surrounded by that many bytes (rounded up to a
 * multiple of 256) of a known pattern, which ps_free checks on the host
 * before it frees the block (the device is synchronised first). Returns the
 * number of guard bytes found changed so far, freed blocks and live ones
 * (each run is also reported on stderr); -1 when guards are off, -2 when the
 * device cannot be synchronised. */
long long ps_guard_violations(void);
/* Free and total device memory of the current device, in bytes (hipMemGetInfo).
 * No reference counterpart: callers and tests use it to check that a matrix
 * releases every device allocation it made. */
int ps_mem_get_info(size_t* free_bytes, size_t* total_bytes);
/* Replaces: thrust::copy / cudaMemcpy H2D and D2H (matrix_utils.cu:495-497, 637;
 * benchmark_utils.h:30-46). Synchronous with respect to the host. */
int ps_memcpy_htod(void* dst, const void* src, size_t bytes);
int ps_memcpy_dtoh(void* dst, const void* src, size_t bytes);
int ps_memcpy_dtod_async(void* dst, const void* src, size_t bytes, ps_stream_t stream);
/* Page-locked host memory (hipHostMalloc) and asynchronous host-to-device
 * copies from it: the staging path of the CSR upload (the reference copies
 * from pageable memory with thrust, matrix_utils.cu:495-497). src of
 * ps_memcpy_htod_async must stay untouched until the copy completes. */
int ps_host_malloc(void** ptr, size_t bytes);
int ps_host_free(void* ptr);
int ps_memcpy_htod_async(void* dst, const void* src, size_t bytes, ps_stream_t stream);
/* Replaces: cudaMemset (benchmark_utils.h:29). */
int ps_memset_async(void* dst, int value, size_t bytes, ps_stream_t stream);
/* Fills count floats with a counter-based hash of (seed, index): uniform in
 * [lo, hi) when normal == 0, N(lo, hi^2) (mean lo, std hi) when normal != 0.
 * No counterpart in the reference, whose inputs come from the host
 * (benchmark_utils.h:100-104); used for the synthetic benchmark graphs (host/synth.h). */
int ps_fill_random_async(float* dst, size_t count, uint64_t seed, float lo, float hi,
                         int normal, ps_stream_t stream);

/* ------------------------------------------------------- streams, events */
/* Replaces: cudaStreamCreate / cudaStreamDestroy (benchmark_utils.h:48-66). */
int ps_stream_create(ps_stream_t* stream);
int ps_stream_destroy(ps_stream_t stream);
int ps_stream_synchronize(ps_stream_t stream);
/* Replaces: cudaEventCreate/Record/Synchronize/ElapsedTime (benchmark_utils.h:68-88). */
int ps_event_create(ps_event_t* event);
int ps_event_destroy(ps_event_t event);
int ps_event_record(ps_event_t event, ps_stream_t stream);
int ps_event_synchronize(ps_event_t event);
int ps_event_elapsed_ms(float* ms, ps_event_t start, ps_event_t stop);
/* Makes `stream` wait for `event` (used to join per-workset streams). */
int ps_stream_wait_event(ps_stream_t stream, ps_event_t event);

/* ------------------------------------------------------------- operators */
/* Maximum number of worksets (GroupTypeNum) one call accepts. */
#define PS_MAX_WORKSETS 32
/* task_chunk of the launchers: the run length of workgroups per XCD chosen
 * from the launch size (see ps_spmm_launch). */
#define PS_TASK_CHUNK_AUTO (-1)

/* One workset as the kernels read it. For s == 0 (residue) group_size is 0 and
 * the group extents come from residue_offset; for s > 0 every group holds
 * group_size = 32 * 2^(s-1) nonzeros (utils/matrix_utils.h:8).
 * order (residue workset only, may be NULL): a permutation of its group_num
 * groups giving the order in which the operators run them, e.g. to visit the
 * groups of neighbouring rows together; results do not depend on it beyond the
 * order of FP32 atomic additions. Entries outside [0, group_num) are skipped
 * (their groups are not computed). NULL runs the groups as stored.
 * No reference counterpart. */
typedef struct ps_workset {
  const int* col_ind;     /* WorksetColInd()[s]  (matrix_utils.h:36) */
  const float* sp_data;   /* WorksetSpData()[s]  (matrix_utils.h:37) */
  const int* group_des;   /* GroupDestination()[s] (matrix_utils.h:38) */
  int group_num;          /* GroupNum()[s] (matrix_utils.h:35) */
  int group_size;
  const int* order;
} ps_workset;

/* SpMM C += A * B over all worksets in ONE launch on `stream`, FP32, B (cols x N)
 * and C (rows x N) row-major. Block groups and residue groups with
 * residue_atomic[g] != 0 add atomically into C; other residue groups store
 * (overwrite) their row. N must be a positive multiple of 32; cols * N and
 * rows * N must fit in int32. B, C and the block worksets' col_ind / sp_data
 * must be 16-byte aligned (as ps_malloc returns them).
 * task_chunk (PS_TASK_CHUNK_AUTO, 0, or a power of two up to 4096; 0 and 1
 * mean the hardware's round robin of workgroups over the 8 XCDs): consecutive
 * tasks dealt to one XCD (one L2) in runs of task_chunk workgroups. Results do
 * not depend on it. Worksets whose neighbouring groups share columns (a
 * row-ordered copy of a graph with locality) run faster with runs of 64.
 * PS_TASK_CHUNK_AUTO picks the run from the launch size: the largest power of
 * two that leaves at least 128 runs in the launch (16 windows of 8 runs), at
 * most 1024 (SpMM) or 256 (SDDMM);
 * measured on signature-ordered worksets and locality run orders (C1, C3:
 * 1-5% faster than the round robin). No reference counterpart.
 * Replaces: the launch loop of PowerSparse::SpMM (PowerSparse_SpMM/spmm_solution.cu:16-31)
 * and the kernels spmm_kernel_block (spmm_kernel_block.cu:60-162) and
 * spmm_kernel_residue (spmm_kernel_residue.cu:5-82). */
int ps_spmm_launch(int workset_count, const ps_workset* worksets, const int* residue_offset,
                   const uint8_t* residue_atomic, int rows, int cols, int N, const float* B,
                   float* C, int task_chunk, ps_stream_t stream);

/* Same operator for a single workset s (s == 0: residue), so callers may keep
 * the reference's one-stream-per-workset schedule (spmm_solution.cu:16-31);
 * workgroups in the hardware's order (task_chunk 1). */
int ps_spmm_workset_launch(int s, const ps_workset* workset, const int* residue_offset,
                           const uint8_t* residue_atomic, int rows, int cols, int N,
                           const float* B, float* C, ps_stream_t stream);

/* SDDMM over all worksets in ONE launch: for every stored nonzero p of workset
 * s in group g, out[s][p] = sp_data[p] * dot(lhs[group_des[g], :], rhs[col_ind[p], :])
 * with K = N features, lhs (rows x N) and rhs (cols x N) row-major. Block
 * worksets store their outputs; the residue workset adds into out[0] (the
 * reference uses atomicAdd into a caller-zeroed buffer). N must be a positive
 * multiple of 32 and at most 512 (the reference accepts 32 and 128 only,
 * sddmm_solution.cu:10-11). lhs, rhs and the block worksets' col_ind must be
 * 16-byte aligned. task_chunk as for ps_spmm_launch (ps_sddmm_workset_launch:
 * 1).
 * Replaces: PowerSparse::SDDMM's launch loop (sddmm_solution.cu:23-48) and
 * sddmm_kernel_block_reduce{32,128} (sddmm_kernel_block.cu:92-240),
 * sddmm_kernel_residue_reduce{32,128} (sddmm_kernel_residue.cu:69-545). */
int ps_sddmm_launch(int workset_count, const ps_workset* worksets, const int* residue_offset,
                    int rows, int cols, int N, const float* lhs, const float* rhs,
                    float* const* out, int task_chunk, ps_stream_t stream);
int ps_sddmm_workset_launch(int s, const ps_workset* workset, const int* residue_offset,
                            int rows, int cols, int N, const float* lhs, const float* rhs,
                            float* out, ps_stream_t stream);

/* SDDMM with the output in the input CSR's order, in ONE launch:
 * out_csr[csr_pos[s][p]] = sp_data[p] * dot(lhs[group_des[g], :], rhs[col_ind[p], :])
 * for every stored nonzero p of workset s, csr_pos[s] being each slot's
 * position in the CSR arrays the matrix was built from (ps_pre_gather_workset's
 * out_csr_pos). Every CSR position is stored exactly once: out_csr (nnz floats)
 * needs no zeroing. Same N and shape limits, and task_chunk, as ps_sddmm_launch.
 * Replaces: the permutation a caller must apply to the reference's output,
 * which "is in workset order, not original CSR order" (PowerSparse_SDDMM.h:11-12). */
int ps_sddmm_csr_launch(int workset_count, const ps_workset* worksets, const int* residue_offset,
                        const int* const* csr_pos, int rows, int cols, int N, const float* lhs,
                        const float* rhs, float* out_csr, int task_chunk,
                        ps_stream_t stream);

/* ----------------------------------------------------------- run orders */
/* Operators of ps_task_count / ps_task_order_build. */
#define PS_OP_SPMM 0
#define PS_OP_SDDMM 1

/* Number of tasks of one fused launch of operator op at width N (for SpMM:
 * of one column slice; every slice runs the same tasks). Tasks are numbered
 * in launch order: the worksets from the largest group size down to the
 * residue (empty ones skipped); a block workset of G groups of GS nonzeros
 * gives ceil(G * GS / T) tile tasks, the residue ceil(G0 / R) tasks of
 * consecutive groups, with T = 256, R = 8 for SpMM (T = 128, R = 4 when N is
 * a multiple of 64) and T = 64, R = 8 for SDDMM. No reference counterpart. */
int ps_task_count(int op, int N, int workset_count, const ps_workset* worksets,
                  uint32_t* count);
/* The locality run order of such a launch into order[count] (device memory,
 * count = ps_task_count): the block tiles of all worksets sorted stably by
 * their first column (the smallest, groups being stored columns ascending),
 * then the residue tasks as stored, so that waves running at the same time
 * gather from one narrow range of B / Y rows. Allocates temporary device
 * memory and synchronises `stream`. No reference counterpart (the reference
 * runs each workset's groups in stored order, one kernel per workset). */
int ps_task_order_build(int op, int N, int workset_count, const ps_workset* worksets,
                        uint32_t* order, uint32_t count, ps_stream_t stream);
/* The same order with marked tiles left out: skip[s] (device,
 * ceil(group_num * group_size / 64) bytes, or NULL; ignored for the residue)
 * marks the 64-nonzero stretches of block workset s (stretch j: stored
 * positions 64 j .. 64 j + 63), and a tile whose stretches are all marked goes
 * to the end of order; *kept receives the number of tasks before them, the
 * task count to pass to ps_sddmm_launch_ordered so that only those run (an
 * SDDMM tile is one stretch). No reference counterpart. */
int ps_task_order_build_subset(int op, int N, int workset_count, const ps_workset* worksets,
                               const uint8_t* const* skip, uint32_t* order, uint32_t count,
                               uint32_t* kept, ps_stream_t stream);

/* ps_spmm_launch, ps_sddmm_launch and ps_sddmm_csr_launch with the tasks run
 * in a given order: the workgroups are dealt to the XCDs as task_chunk says,
 * and task t of that sequence runs task task_order[t] (a permutation of the
 * ps_task_count tasks; task_count must equal that count for SpMM). Every task
 * does the same work in any order: SDDMM results are bitwise those of the
 * unordered launch, SpMM's differ only in the order of FP32 atomic additions.
 * The SDDMM variants also take task_count below the launch's count: then only
 * the first task_count entries of task_order run (see
 * ps_task_order_build_subset; the outputs of the other tasks are not
 * written). */
int ps_spmm_launch_ordered(int workset_count, const ps_workset* worksets,
                           const int* residue_offset, const uint8_t* residue_atomic, int rows,
                           int cols, int N, const float* B, float* C, int task_chunk,
                           const uint32_t* task_order, uint32_t task_count, ps_stream_t stream);
int ps_sddmm_launch_ordered(int workset_count, const ps_workset* worksets,
                            const int* residue_offset, int rows, int cols, int N,
                            const float* lhs, const float* rhs, float* const* out, int task_chunk,
                            const uint32_t* task_order, uint32_t task_count, ps_stream_t stream);
int ps_sddmm_csr_launch_ordered(int workset_count, const ps_workset* worksets,
                                const int* residue_offset, const int* const* csr_pos, int rows,
                                int cols, int N, const float* lhs, const float* rhs,
                                float* out_csr, int task_chunk, const uint32_t* task_order,
                                uint32_t task_count, ps_stream_t stream);

/* SDDMM of worksets laid out in another group order than the public ones (a
 * task-order execution copy): the result of member j of group g of workset s
 * goes to out[s][out_base[s][g] + j], out[s] being the public workset-order
 * buffer (ps_pre_exec_positions gives the bases); block results are stored,
 * residue results added, exactly as ps_sddmm_launch does at the public
 * positions; task_chunk as for ps_sddmm_launch. No reference counterpart (the
 * reference runs the public layout only). */
int ps_sddmm_scatter_launch(int workset_count, const ps_workset* worksets,
                            const int* residue_offset, const int* const* out_base, int rows,
                            int cols, int N, const float* lhs, const float* rhs,
                            float* const* out, int task_chunk, ps_stream_t stream);

/* out_csr[csr_pos[s][p]] = in[s][p] for p < lengths[s]: moves per-nonzero values
 * from workset order (e.g. the outputs of ps_sddmm_launch) to CSR order.
 * Replaces: the same caller-side permutation (PowerSparse_SDDMM.h:11-12). */
int ps_workset_to_csr(int workset_count, const long long* lengths, const int* const* csr_pos,
                      const float* const* in, float* out_csr, ps_stream_t stream);

/* ------------------------------------------------------- dense hub block */
/* The hub rows (highest degree) restricted to the hot columns (most nonzeros)
 * of a matrix, run as dense FP32 products on the matrix cores (hand-written
 * v_mfma_f32_32x32x2f32 kernels). All pointers are device memory. hot_rank /
 * hub_index map a matrix column / row to its position in hot_cols / hub_rows,
 * or -1 (hot_cols and hub_rows ascending). dense (ps_hub_dense_floats(rows,
 * cols) floats, 16-byte aligned) holds the value of every slot stored exactly
 * once, 0 elsewhere (padding included), in the matrix cores' fragment order:
 * with ld = ps_hub_dense_ld(cols), slot (i, h) is element
 *   ((i / 32) * (ld / 8) + h / 8) * 256 + ((h % 8) / 4) * 128 + (i % 32) * 4 + h % 4
 * (one 8-column step of 32 rows = 256 consecutive floats, in the order the 64
 * lanes of a wave load them). stored has one bit per such slot (rows x
 * ceil(cols / 32) words, bit h % 32 of word h / 32). A slot stored more than
 * once is left out of the block (no bit, value 0), so its entries stay on the
 * sparse SpMM path. No reference counterpart. */
typedef struct ps_hub_block {
  int matrix_rows, matrix_cols;
  int rows;              /* R: hub rows */
  int cols;              /* H: hot columns */
  const int* hub_rows;   /* [R] */
  const int* hub_index;  /* [matrix_rows] */
  const int* hot_cols;   /* [H] */
  const int* hot_rank;   /* [matrix_cols] */
  const float* dense;    /* [ps_hub_dense_floats(R, H)] */
  const uint32_t* stored;
} ps_hub_block;

/* hist[32 * 32] (device, written): hist[a * 32 + b] = stored entries of rows of
 * degree in [2^a, 2^(a+1)) (degree >= 256 only) whose column count col_nnz is
 * in [2^b, 2^(b+1)); the statistics a block is chosen from. */
int ps_hub_histogram(const int* row_ptr, int rows, const int* col_ind, const int* col_nnz,
                     unsigned long long* hist, ps_stream_t stream);
/* Words of the stored bit mask. */
size_t ps_hub_stored_words(const ps_hub_block* hb);
/* Columns per dense row: cols rounded up to a multiple of 64 (0 for cols <= 0). */
size_t ps_hub_dense_ld(int cols);
/* Floats of the dense block: rows rounded up to a multiple of 64, times
 * ps_hub_dense_ld(cols) (0 for an empty block). */
size_t ps_hub_dense_floats(int rows, int cols);
/* Fills dense and stored from the matrix CSR (finite values), slots stored
 * more than once left out; the same block on every build. */
int ps_hub_dense_build(const ps_hub_block* hb, const int* row_ptr, const int* col_ind,
                       const float* sp_data, float* dense, uint32_t* stored, ps_stream_t stream);
/* counts[r] = stored entries of row r outside the block's stored slots
 * (matrix_rows values; run after ps_hub_dense_build). */
int ps_hub_kept_counts(const ps_hub_block* hb, const int* row_ptr, const int* col_ind,
                       uint32_t* counts, ps_stream_t stream);
/* The CSR without the entries of the block's stored slots (order within rows
 * kept); new_row_ptr is the exclusive scan of ps_hub_kept_counts. */
int ps_hub_compact(const ps_hub_block* hb, const int* row_ptr, const int* col_ind,
                   const float* sp_data, const uint32_t* new_row_ptr, int* new_col,
                   float* new_val, ps_stream_t stream);
/* residue_atomic[g] = 1 for every residue group g whose row (group_des[g]) is a
 * hub row (the rows of a partition without the block keep accumulating). */
int ps_hub_mark_atomic(const ps_hub_block* hb, const int* group_des, int group_num,
                       uint8_t* residue_atomic, ps_stream_t stream);
/* flags[t] = 1 when the t-th 64-nonzero stretch of a block workset of groups
 * >= 64 nonzeros (stored positions 64 t .. 64 t + 63, group_num * group_size
 * / 64 flags) lies inside the block: its group's row is a hub row and all its
 * columns are hot; else 0. */
int ps_hub_tile_flags(const ps_hub_block* hb, const ps_workset* workset, uint8_t* flags,
                      ps_stream_t stream);
/* Device workspace bytes at width N of ps_hub_spmm_launch (op PS_OP_SPMM: one
 * feature slice, up to 128, of B's hot rows in fragment order, and flags) or
 * of ps_hub_sddmm_launch (PS_OP_SDDMM: lhs[hub_rows] and rhs[hot_cols] in
 * fragment order, rows padded to 64 and 128). */
size_t ps_hub_workspace_bytes(const ps_hub_block* hb, int op, int N);
/* C[hub_rows[i], :] += sum over stored block slots (i, h) of value * B[hot_cols[h], :],
 * B (matrix_cols x N) and C (matrix_rows x N) row-major, added with float
 * atomics (other writers of C may run at the same time); Inf / NaN in B reach
 * exactly the rows that store their column. Calls overlapping on one
 * workspace race. */
int ps_hub_spmm_launch(const ps_hub_block* hb, int N, const float* B, float* C, void* workspace,
                       size_t workspace_bytes, ps_stream_t stream);
/* The SDDMM tile list of a hub block: tiles[t] = (s << 27) | j names the j-th
 * 64-nonzero tile of block workset s (groups >= 64 nonzeros, every entry
 * inside the block); codes that name no such tile, and entries outside the
 * block, are left out of the plan. The plan (ps_hub_sddmm_plan_bytes bytes of
 * device memory) groups the listed nonzeros by the dense tile (64 hub rows x
 * 128 hot columns) they fall in, each with its output position and sp_data;
 * tile_count * 64 must stay below 2^31. ps_hub_sddmm_plan allocates
 * temporaries and synchronises the stream. */
size_t ps_hub_sddmm_plan_bytes(const ps_hub_block* hb, uint32_t tile_count);
int ps_hub_sddmm_plan(const ps_hub_block* hb, int workset_count, const ps_workset* worksets,
                      const uint32_t* tiles, uint32_t tile_count, void* plan, size_t plan_bytes,
                      ps_stream_t stream);
/* For every planned nonzero p of workset s (row group_des[g], column col_ind[p]):
 * out[s][p] = sp_data[p] * dot(lhs[row, :], rhs[col, :]), the dots taken from
 * dense tiles of X[hub_rows] * Y[hot_cols]^T computed in registers (never
 * stored); with out_csr, out_csr[out_pos[s][p]] instead. tile_count is the
 * plan's list length; workspace (16-byte aligned) holds the gathered operands
 * (ps_hub_workspace_bytes(hb, PS_OP_SDDMM, N) bytes). Calls overlapping on
 * one workspace race. */
int ps_hub_sddmm_launch(const ps_hub_block* hb, int workset_count, const ps_workset* worksets,
                        const void* plan, uint32_t tile_count, int N, const float* lhs,
                        const float* rhs, float* const* out, const int* const* out_pos,
                        float* out_csr, void* workspace, size_t workspace_bytes,
                        ps_stream_t stream);

/* ---------------------------------------------------------- primitives */
/* Device-wide exclusive prefix sum of n uint32 values (out may alias in).
 * workspace: ps_scan_workspace_bytes(n) bytes of device memory.
 * Replaces: the host prefix loops of GetGroupMetaInfo and GetResidueOffset
 * (utils/matrix_utils.cu:158-208, 451-464). */
size_t ps_scan_workspace_bytes(size_t n);
int ps_exclusive_scan_u32(const uint32_t* in, uint32_t* out, size_t n, void* workspace,
                          ps_stream_t stream);
/* ps_exclusive_scan_u32 without a workspace and without any allocation: the
 * tile sums live in a 256 KiB array the library keeps in each GPU's memory
 * for the life of the process, so n is limited to what it holds
 * (268,173,312 values; larger n returns PS_ERR_INVALID). Every call on one GPU uses
 * that GPU's array: calls that overlap on one GPU (other streams, other host
 * threads) race and must be serialised by the caller. Launches kernels only
 * (no hipMalloc, hipFree or memset), so it may be captured in a HIP graph.
 * No counterpart in the reference: it is for callers that cannot allocate
 * device memory (code under HIP graph capture, tight serving loops). */
int ps_exclusive_scan_u32_noalloc(const uint32_t* in, uint32_t* out, size_t n,
                                  ps_stream_t stream);

/* Stable LSD radix sort of (key, value) pairs by key bits [begin_bit, end_bit);
 * vals and vals_alt both NULL sorts the keys alone. Bits above end_bit inside
 * the last 8-bit digit take part in that digit: keep them equal in all keys.
 * Keys and values ping-pong between the two buffer pairs; *result_in_alt is set
 * to 1 when the sorted data ended in the *_alt buffers. workspace:
 * ps_radix_workspace_bytes(n) bytes.
 * Replaces: thrust::sort of NNZPoint (matrix_utils.cu:522-524) and
 * thrust::stable_sort of group indices (matrix_utils.cu:590-592). */
size_t ps_radix_workspace_bytes(size_t n);
int ps_radix_sort_pairs_u64(uint64_t* keys, uint64_t* keys_alt, uint32_t* vals,
                            uint32_t* vals_alt, size_t n, int begin_bit, int end_bit,
                            void* workspace, int* result_in_alt, ps_stream_t stream);
int ps_radix_sort_pairs_u32(uint32_t* keys, uint32_t* keys_alt, uint32_t* vals,
                            uint32_t* vals_alt, size_t n, int begin_bit, int end_bit,
                            void* workspace, int* result_in_alt, ps_stream_t stream);

/* out[i] = i for i < n. Replaces: thrust::sequence (matrix_utils.cu:562-566). */
int ps_iota_u32(uint32_t* out, int n, ps_stream_t stream);

/* -------------------------------------------------------- preprocessing */
/* sums[s] = sum over rows of floor(deg / (32 * 2^(s-1))) for s = 1..31 (sums[0] = 0),
 * written to host memory (synchronous).
 * Replaces: the row loop of AnalyzeMatrix (utils/matrix_utils.cu:44-53). */
int ps_pre_degree_sums(const int* row_ptr, int rows, unsigned long long* sums_host,
                       ps_stream_t stream);

/* col_nnz[c] += number of nonzeros in column c (col_nnz pre-zeroed).
 * Replaces: the OpenMP histogram (matrix_utils.cu:508-514). */
int ps_pre_col_histogram(const int* col_ind, int nnz, int* col_nnz, ps_stream_t stream);

/* keys[p] = (row(p) << count_bits) | (max_count - col_nnz[col_ind[p]]), vals[p] = p:
 * the stable sort of these pairs gives each row's nonzeros by column count
 * descending, ties in CSR order.
 * Replaces: CopyCSRToNNZ + NNZPoint::operator< (matrix_utils.cu:210-223, 239-257). */
int ps_pre_rank_keys(const int* row_ptr, int rows, const int* col_ind, int nnz,
                     const int* col_nnz, int max_count, int count_bits, uint64_t* keys,
                     uint32_t* vals, ps_stream_t stream);

/* The ranking itself, row by row: writes keys / vals as the stable sort of
 * ps_pre_rank_keys' output by key would (row << count_bits | max_count -
 * col_nnz[col], CSR position), sorting only inside rows (rows arrive in
 * order): one wave per row up to 256 nonzeros, an LDS bitonic sort per row up
 * to 8192, a radix sort over the elements of longer rows. count_bits <= 32.
 * Synchronises the stream.
 * Replaces: thrust::sort of NNZPoint (matrix_utils.cu:518-524). */
int ps_pre_rank_sort(const int* row_ptr, int rows, const int* col_ind, int nnz,
                     const int* col_nnz, int max_count, int count_bits, uint64_t* keys,
                     uint32_t* vals, ps_stream_t stream);

/* Per-row group counts: counts[s * rows + r] = groups of row r in workset s
 * (s = 0 residue). Replaces: GetGroupNumArray (matrix_utils.cu:132-156). */
int ps_pre_group_counts(const int* row_ptr, int rows, int group_type_num, int fine,
                        uint32_t* counts, ps_stream_t stream);

/* Per-group metadata in initial (row) order from the exclusive prefix of the
 * counts (prefix[s * rows + r]): destination row, first ranked index, and for
 * the residue workset its length and atomic flag.
 * Replaces: GetGroupMetaInfo (matrix_utils.cu:158-208). */
int ps_pre_group_meta(const int* row_ptr, int rows, int group_type_num, int fine,
                      const uint32_t* prefix, int* const* group_des,
                      int* const* group_start, int* residue_len, uint8_t* residue_atomic,
                      ps_stream_t stream);

/* Signature bitmaps, word-major per workset: sig[s][w * G_s + g] gets bit
 * 31 - b % 32 of word b / 32 for b = sigbit[col] of every member (sig zeroed).
 * ranked_keys are the sorted keys of ps_pre_rank_keys (row in the high bits),
 * ranked_vals the CSR positions in ranked order.
 * Replaces: GetResidueSignature / GetBlockSignature (matrix_utils.cu:261-327). */
int ps_pre_signatures(const int* row_ptr, int rows, int group_type_num, int fine,
                      const uint64_t* ranked_keys, int count_bits,
                      const uint32_t* ranked_vals, int nnz, const int* col_ind,
                      const int* sigbit, const uint32_t* prefix, const int* group_num,
                      uint32_t* const* sig, ps_stream_t stream);

/* keys[k] = ~sig_word[perm[k]] (descending signature order as an ascending key).
 * Replaces: CompareDescending (matrix_utils.cu:394-401). */
int ps_pre_signature_keys(const uint32_t* sig_word, const uint32_t* perm, int n,
                          uint32_t* keys, ps_stream_t stream);

/* OR and AND of each signature word over all groups (host arrays of `words`),
 * to skip digits that cannot reorder the groups. */
int ps_pre_signature_span(const uint32_t* sig, int groups, int words, uint32_t* or_host,
                          uint32_t* and_host, ps_stream_t stream);

/* Output base of every group of a task-order execution copy (groups in their
 * initial order): out_base[perm[k]] = where public group k (signature order)
 * starts in the public workset, k * group_size for blocks (group_size > 0),
 * pub_offset[k] (the public residue offsets) for the residue workset.
 * No reference counterpart. */
int ps_pre_exec_positions(int group_size, const uint32_t* perm, int groups,
                          const int* pub_offset, int* out_base, ps_stream_t stream);

/* Gather-locality score of a task order: the concatenated column sequence
 * col_ind[0][0 .. lengths[0]), col_ind[1][...], ... is cut into windows of
 * `window` nonzeros; up to max_windows of them, evenly spaced, are sampled and
 * *score = (distinct columns per window) / window, averaged (0 when the
 * sequence is shorter than one window). Lower = more B / Y row reuse between
 * nearby tasks. Synchronises the stream. No reference counterpart. */
int ps_pre_locality_score(int count, const int* const* col_ind, const long long* lengths,
                          int window, int max_windows, double* score, ps_stream_t stream);

/* Sparse form of the signatures, for long signatures where the bitmaps of
 * ps_pre_signatures would not fit: the ascending list of distinct signature
 * bits of every group. Groups are numbered globally, workset after workset
 * (global id = group_num[0] + ... + group_num[s-1] + g); group q's list is
 * lists[list_begin[q] .. list_begin[q+1]). lists holds up to nnz entries,
 * list_begin sum(group_num) + 1. Every group must have a member. Synchronises
 * the stream. Same inputs as ps_pre_signatures.
 * Replaces: GetResidueSignature / GetBlockSignature (matrix_utils.cu:261-327). */
int ps_pre_signature_lists(const int* row_ptr, int rows, int group_type_num, int fine,
                           const uint64_t* ranked_keys, int count_bits,
                           const uint32_t* ranked_vals, int nnz, const int* col_ind,
                           const int* sigbit, int signature_len, const uint32_t* prefix,
                           const int* group_num, uint32_t* lists, uint32_t* list_begin,
                           ps_stream_t stream);

/* perm[s][k] = the group of workset s at position k of the stable descending
 * signature order, from the lists of ps_pre_signature_lists: the same order as
 * the per-word stable sorts. Ties are refined in rounds: each class of tied
 * groups is sorted by where and which way each member's list departs from
 * the class's first member, so nested prefixes separate in one round (cost
 * follows the branching of the tied lists, not the signature length).
 * Synchronises the stream.
 * Replaces: the stable_sort loop over signature words (matrix_utils.cu:588-593)
 * with CompareDescending (:394-401). */
int ps_pre_signature_order(const uint32_t* lists, const uint32_t* list_begin,
                           int group_type_num, const int* group_num, int signature_len,
                           uint32_t* const* perm, ps_stream_t stream);

/* Final metadata in sorted order: des[k] = src_des[perm[k]]; for the residue
 * workset also len[k] = src_len[perm[k]] and atomic[k] = src_atomic[perm[k]].
 * Replaces: the metadata half of GetResidueWorkset / GetBlockWorkset
 * (matrix_utils.cu:403-449). */
int ps_pre_permute_meta(const uint32_t* perm, int groups, const int* src_des, int* des,
                        const int* src_len, uint32_t* len, const uint8_t* src_atomic,
                        uint8_t* atomic, ps_stream_t stream);

/* Final nonzeros of one workset: group k (in sorted order) takes the members
 * of initial group perm[k] (ranked_vals[group_start[perm[k]] ...]) sorted by
 * column ascending, ties in ranked order, written at offset[k] (residue) or
 * k * group_size (blocks). out_csr_pos (optional, same length as out_col)
 * receives each slot's position in the input CSR arrays.
 * Replaces: GetSrc{Residue,Block}Workset + thrust::sort of NNZPoint2 +
 * Get{Residue,Block}Workset (matrix_utils.cu:329-392, 596-617, 639-656). */
int ps_pre_gather_workset(int group_size, const uint32_t* perm, int groups,
                          const int* group_start, const int* residue_offset,
                          const uint32_t* ranked_vals, const int* col_ind,
                          const float* sp_data, int* out_col, float* out_val,
                          int* out_csr_pos, ps_stream_t stream);

#ifdef __cplusplus
}
#endif

#endif /* POWERSPARSE_HIP_H */
