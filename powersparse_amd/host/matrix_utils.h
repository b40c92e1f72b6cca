// PowerSparseMatrixGPU: owns the device worksets of a CSR matrix.
//
// Same public interface as the reference (ParCIS/PowerSparse
// utils/matrix_utils.h:8-76): constructor from host CSR arrays, the accessors
// returning device pointers, ValidateDenseShape and the GROUP_SIZE / CEIL /
// FLOOR macros. The worksets are built on the GPU (HIP kernels reached through
// the C ABI in include/powersparse_hip.h) and are bit-identical to what the
// reference's preprocessing produces for the same CU count.
//
// No HIP or CUDA header is included here: device work goes through the C ABI.
#pragma once

#include <cstdint>
#include <limits>
#include <stdexcept>
#include <vector>

#include "powersparse_hip.h"

#define GROUP_SIZE(I) (32 * (1 << ((I) - 1)))
#define CEIL(X, Y) ((X) / (Y) + ((X) % (Y) != 0))
#define FLOOR(X, Y) ((X) / (Y))

namespace PowerSparse {

enum SigBitMode { PPL = 0, FFC = 1 };
enum FreqSort { FreqNoSort = 0, FreqDoSort = 1 };
enum GroupSort { GroupNoSort = 0, GroupDoSort = 1 };

// How the groups of a workset are put in signature order. Both methods give
// the order of the reference's per-word stable sorts (utils/matrix_utils.cu:
// 588-593); they differ in cost. kBitmapWords builds the signature bitmaps
// (groups x L/32 words) and sorts once per word that varies; kBitLists sorts
// each group's list of distinct signature bits and refines ties a few list
// elements at a time, in memory bounded by nnz whatever L is. kAuto takes the
// bitmaps up to kBitmapMaxWords words (one or a few radix passes), the lists
// beyond (measured faster from 22 words up: C1, C3, C4).
enum class SignatureOrder { kAuto = 0, kBitmapWords = 1, kBitLists = 2 };
constexpr int kBitmapMaxWords = 4;

// The order in which the operators run the groups (their results do not depend
// on it, beyond the order of FP32 atomic additions). kSignature runs the public
// worksets as laid out. kRow runs a row-ordered copy of them (the group
// numbering before the signature sort; ~8 more bytes per nonzero of device
// memory), which keeps rows with shared columns together when the row ids
// carry the graph's locality, as in community graphs. kAuto builds the copy,
// scores both orders by the distinct columns per window of nearby nonzeros
// (ps_pre_locality_score) and keeps the copy only if its score is below
// kRowOrderGain times the signature order's.
enum class TaskOrder { kAuto = 0, kSignature = 1, kRow = 2 };

// Which partition SpMM runs on. kParity: the public worksets (the reference's
// partition at the policy's CU count). kTuned: a second partition of the same
// matrix kept for SpMM alone, the reference's algorithm with the number of
// worksets capped at kTunedSpmmGroupTypes (largest groups of 64 nonzeros),
// groups in signature order. Its groups are popularity bands of each row
// (the row's nonzeros ranked by column count, cut into 64s), and the signature
// sort lays bands with the same hot columns side by side, so the waves
// running together gather from fewer B rows than with the hub rows' 8192-
// nonzero groups (measured on MI355X, C3: SpMM N=32 2.03 -> 1.91 ms, N=128
// 8.14 -> 7.66 ms; see the task-order notes). It is built when the parity
// partition has more worksets than the cap and the operators run in signature
// order; it shares the upload, column counts, signature bits and per-row
// ranking with the public partition and adds its own grouping, signature sort
// and gather (C3: 220 ms for both partitions, 332 when built separately) and
// about 8 bytes per nonzero. SpMM results differ from the parity partition's
// only in the FP32 summation order: rows with a single group of at most 32
// nonzeros are stored, every other row accumulates, exactly as with the public
// worksets.
enum class SpmmPartition { kParity = 0, kTuned = 1 };
constexpr int kTunedSpmmGroupTypes = 3;

// Dense hub block. On power-law graphs the rows of highest degree hold a dense
// core with the most popular columns (C3: rows of degree >= 16384 x columns
// with >= 512 nonzeros, 70 M of the 264 M nonzeros at 38% density). kAuto
// keeps that block as a dense FP32 matrix and runs it on the matrix cores
// with hand-written MFMA kernels (ps_hub_spmm_launch / ps_hub_sddmm_launch),
// the rest as before: SpMM on a tuned partition of the matrix without the
// block, SDDMM on the public worksets with the block's tiles (64 consecutive
// nonzeros of a block group) left out of the run order and their outputs
// written from dense tiles of the product computed in registers. The block
// comes in up to
// kHubMaxTiers tiers of disjoint row ranges, each with its own columns: the
// first tier is the pair of power-of-two thresholds (row degree >= 2^a,
// column count >= 2^b) that maximises block nonzeros - kHubDenseCost * rows
// * columns, kept when that gain is at least kHubMinGain of the nonzeros; the
// next tier takes the rows below 2^a the same way, kept from kHubMinTierGain
// (kHubDenseCost: the dense element's cost relative to the sparse nonzero it
// replaces, measured on MI355X). SDDMM computes a tier's dense dots whole and
// takes from it only the tiles lying inside it, so it uses a tier when those
// hold at least kHubSddmmMinFill nonzeros per dense element (C3: both tiers,
// 2526 x 72840 and rows of degree 1024..16383 x 3578 columns). It is used
// with the tuned SpMM partition and the locality run order only. Results match the sparse path within FP32 summation order;
// Inf / NaN in B reach exactly the rows that store their column; rows of the
// block accumulate into C as the reference's do (they hold more than 32
// nonzeros); a (row, column) slot stored more than once stays on the sparse
// SpMM path. Cost: 4 bytes per block element (dense), 12 bytes per planned
// SDDMM nonzero, the tuned partition's own preprocessing (it no longer
// shares the public one's), and an operator workspace allocated with the
// block (SDDMM at N = 512: 2 KiB per hub row and per hot column of the
// widest tier, padded to whole tiles).
enum class HubBlock { kAuto = 0, kOff = 1 };
constexpr int kHubMaxTiers = 3;
constexpr double kHubDenseCost = 0.12, kHubMinGain = 0.05, kHubMinTierGain = 0.02;
constexpr double kHubSddmmMinFill = 0.25;
constexpr int kHubMinRows = 256, kHubMinCols = 1024;
constexpr long long kHubMaxElements = 1LL << 29;
constexpr double kRowOrderGain = 0.85;
// Workgroup -> XCD runs (ps_spmm_launch's task_chunk) per task order: in a
// row-ordered copy neighbouring groups share columns, so runs of 64 tasks stay
// under one L2 (C4: 4% faster than 16, 10-15% faster than the hardware's round
// robin); in signature order and the locality run orders the launchers size
// the runs from the launch (PS_TASK_CHUNK_AUTO: C3 SpMM on the tuned partition
// 3-4% and SDDMM N = 128 1.4% faster than the round robin; C1 SpMM 4-5%).
constexpr int kRowOrderTaskChunk = 64, kSignatureOrderTaskChunk = PS_TASK_CHUNK_AUTO;
constexpr int kLocalityWindow = 65536, kLocalityWindows = 128;

// The worksets as the operators run them: the public ones (out_base ==
// nullptr) or the row-ordered copy, whose group g of workset s starts at
// out_base[s][g] in the public layout. csr_pos: CSR position per slot, or
// nullptr.
struct ExecutionLayout {
  const int* const* col_ind = nullptr;
  const float* const* sp_data = nullptr;
  const int* const* group_des = nullptr;
  const int* residue_offset = nullptr;
  const bool* residue_atomic = nullptr;
  const int* const* out_base = nullptr;
  const int* const* csr_pos = nullptr;
  int task_chunk = kSignatureOrderTaskChunk;
  // Run orders of the fused launches (null: tasks run as stored), indexed by
  // RunOrderSlot(): SpMM in 32-float slices, SpMM in 64-float slices, SDDMM.
  const uint32_t* run_order[3] = {nullptr, nullptr, nullptr};
  uint32_t run_order_tasks[3] = {0, 0, 0};
};

// Which run order a launch of operator op (PS_OP_SPMM / PS_OP_SDDMM) at width
// N uses: the three operator task shapes (SpMM tiles of 256 nonzeros, or of
// 128 when N is a multiple of 64 and runs in 64-float slices; SDDMM tiles of
// 64).
inline int RunOrderSlot(int op, int N) {
  return op == PS_OP_SDDMM ? 2 : (N % 64 == 0 ? 1 : 0);
}

// Partition settings. The reference hard-codes all of them except the CU
// count, which it reads from the current device (utils/matrix_utils.cu:31-63);
// cu_count == 0 means "the current device's multiProcessorCount".
struct PartitionPolicy {
  int cu_count = 0;
  SignatureOrder signature_order = SignatureOrder::kAuto;
  // Keep, for every stored nonzero, its position in the input CSR arrays
  // (4 bytes per nonzero on the device): needed by SDDMMToCSR / WorksetToCSR.
  bool csr_positions = false;
  TaskOrder task_order = TaskOrder::kAuto;
  // With the signature task order, run each operator's tasks in the locality
  // order: block tiles of every workset sorted by their first column, the
  // residue after them as stored (ps_task_order_build). Results are those of
  // the stored order (SpMM: up to the order of FP32 atomic additions).
  bool run_order = true;
  // Cap on the number of worksets S (0: none, the reference's rule alone);
  // a capped partition is not the reference's when its rule gives more.
  int max_group_types = 0;
  SpmmPartition spmm_partition = SpmmPartition::kTuned;
  HubBlock hub_block = HubBlock::kAuto;
  // Explicit tiers, whatever the cost rule says: tier k holds the rows of
  // degree >= hub_min_degree[k] (and below tier k-1's) and the columns with
  // >= hub_min_count[k] nonzeros; the leading pairs with both values > 0 are
  // used, degrees decreasing; they serve SDDMM too, whatever their fill. The
  // block is still dropped when it would hold every nonzero, or when the
  // matrix has a single workset.
  int hub_min_degree[kHubMaxTiers] = {};
  int hub_min_count[kHubMaxTiers] = {};
};

// Wall-clock milliseconds of the preprocessing stages (host timer, the stream
// synchronised at each stage boundary only when timing was requested).
struct PreprocessTimings {
  double upload_ms = 0, analyze_ms = 0, rank_ms = 0, groups_ms = 0, sigbit_ms = 0,
         signature_ms = 0, order_ms = 0, gather_ms = 0, total_ms = 0;
};

// Owns the GPU worksets built from host CSR arrays. Construct and destroy on
// the same device; complete outstanding operator calls before destruction.
class PowerSparseMatrixGPU {
 public:
  PowerSparseMatrixGPU(int row_num, int col_num, int nnz_num, const int* row_ptr,
                       const int* col_ind, const float* sp_data);
  PowerSparseMatrixGPU(int row_num, int col_num, int nnz_num, const int* row_ptr,
                       const int* col_ind, const float* sp_data, const PartitionPolicy& policy,
                       PreprocessTimings* timings = nullptr);
  ~PowerSparseMatrixGPU();
  PowerSparseMatrixGPU(const PowerSparseMatrixGPU&) = delete;
  PowerSparseMatrixGPU& operator=(const PowerSparseMatrixGPU&) = delete;
  PowerSparseMatrixGPU(PowerSparseMatrixGPU&&) = delete;
  PowerSparseMatrixGPU& operator=(PowerSparseMatrixGPU&&) = delete;

  int MatrixRow() const { return _matrix_row; }
  int MatrixCol() const { return _matrix_col; }
  int MatrixNNZ() const { return _matrix_nnz; }
  int GroupTypeNum() const { return _group_type_num; }
  int GroupFineSize() const { return _group_fine_size; }
  const int* GroupNum() const { return _group_num; }
  const int* const* WorksetColInd() const { return _workset_col_ind; }
  const float* const* WorksetSpData() const { return _workset_sp_data; }
  const int* const* GroupDestination() const { return _group_des; }
  const int* ResidueOffset() const { return _residue_offset; }
  const bool* ResidueAtomic() const { return _residue_atomic; }

  // Not in the reference: the signature length L (bits) and the CU count the
  // partition was computed for.
  int SignatureLen() const { return _signature_len; }
  int PartitionCuCount() const { return _cu_count; }
  // The signature order method the build used (never kAuto).
  SignatureOrder SignatureOrderUsed() const { return _signature_order; }
  // Position in the input CSR arrays of every stored nonzero, per workset
  // (same layout as WorksetColInd); nullptr unless the policy asked for it.
  const int* const* WorksetCSRPosition() const { return _workset_csr_pos; }
  // The task order the build chose (never kAuto) and the locality scores it
  // compared (signature order, row order; 0 when not computed).
  TaskOrder TaskOrderUsed() const { return _task_order; }
  double LocalityScore(TaskOrder order) const {
    return order == TaskOrder::kRow ? _locality[1] : _locality[0];
  }
  // Whether the operators run in the locality run order (see PartitionPolicy).
  bool RunOrderUsed() const { return _run_order[0] != nullptr || _run_order[2] != nullptr; }
  // The partition SpMM runs on: the tuned one (SpmmPartition::kTuned), or
  // this matrix itself when none was built. With a dense hub block it holds
  // the matrix without the block (SpMM adds the block's product to it).
  const PowerSparseMatrixGPU& SpmmMatrix() const { return _spmm_tuned ? *_spmm_tuned : *this; }
  // What the operators launch on.
  ExecutionLayout Execution() const;
  // The dense hub block in use (HubBlock): its tiers, each rows x columns
  // (0 x 0 beyond the last).
  bool HubBlockUsed() const { return _hub != nullptr; }
  int HubTiers() const;
  int HubRows(int tier = 0) const;
  int HubCols(int tier = 0) const;
  // The hub block's part of an operator call, enqueued on `stream` after the
  // sparse part (SpMM: C += block * B; SDDMM: the block groups' outputs, into
  // out[s] or, with csr_out, into csr_out at the CSR positions). Calls on one
  // matrix share its workspace and run one after another on the GPU; neither
  // allocates.
  void HubSpmm(int N, const float* B, float* C, ps_stream_t stream) const;
  void HubSddmm(int N, const float* lhs, const float* rhs, float* const* out, float* csr_out,
                ps_stream_t stream) const;

 private:
  // The stages that do not depend on the partition (upload, column counts,
  // signature bits, per-row ranking), shared by the partitions of one matrix.
  struct Prepared;
  struct HubState;
  struct Unbuilt {};
  // A partition of the same matrix whose Build() the caller runs.
  PowerSparseMatrixGPU(Unbuilt, int row_num, int col_num, int nnz_num, int cu_count,
                       const PartitionPolicy& policy);
  void Configure(const PartitionPolicy& policy);
  // The partition at this object's settings from the prepared stages; drops
  // the per-row ranking from `in` once it is no longer needed when
  // `last_partition` is set.
  void Build(const int* row_ptr, Prepared& in, bool last_partition);
  void Release() noexcept;
  void ReleaseExecution() noexcept;
  void BuildRunOrders();
  // Chooses and builds the dense hub block and the tuned SpMM partition of
  // the rest; false (nothing built) when no block qualifies.
  bool BuildHub(const int* row_ptr, Prepared& in, const PartitionPolicy& policy);
  std::vector<ps_workset> PublicWorksets() const;

  int _matrix_row, _matrix_col, _matrix_nnz;
  int _group_type_num = 0, _group_fine_size = 16;
  int _signature_len = 32;
  int _cu_count = 0;
  SignatureOrder _signature_order = SignatureOrder::kAuto;
  bool _keep_csr_pos = false;
  int* _group_num = nullptr;
  int** _workset_col_ind = nullptr;
  float** _workset_sp_data = nullptr;
  int** _group_des = nullptr;
  int** _workset_csr_pos = nullptr;
  int* _residue_offset = nullptr;
  TaskOrder _task_order = TaskOrder::kAuto;
  double _locality[2] = {0.0, 0.0};
  // row-ordered execution copy (TaskOrder::kRow)
  int** _exec_col_ind = nullptr;
  float** _exec_sp_data = nullptr;
  int** _exec_group_des = nullptr;
  int** _exec_out_base = nullptr;
  int** _exec_csr_pos = nullptr;
  int* _exec_residue_offset = nullptr;
  bool* _exec_residue_atomic = nullptr;
  bool* _residue_atomic = nullptr;
  // locality run orders, by RunOrderSlot()
  bool _want_run_order = true;
  uint32_t* _run_order[3] = {nullptr, nullptr, nullptr};
  uint32_t _run_order_tasks[3] = {0, 0, 0};
  int _max_group_types = 0;
  PowerSparseMatrixGPU* _spmm_tuned = nullptr;  // SpmmPartition::kTuned
  HubState* _hub = nullptr;                      // HubBlock
};

// The kernels use signed 32-bit dense element offsets (matrix_utils.h:71-76).
inline void ValidateDenseShape(int rows, int cols, int n) {
  if (n <= 0 || int64_t(rows) * n > std::numeric_limits<int>::max() ||
      int64_t(cols) * n > std::numeric_limits<int>::max())
    throw std::invalid_argument("Dense dimensions exceed the 32-bit kernel indexing range");
}

// Converts a C ABI status into the reference's exception types:
// PS_ERR_INVALID -> std::invalid_argument, anything else -> std::runtime_error.
void ThrowOnError(int status);

}  // namespace PowerSparse
