// Run order of a fused operator launch: which task each wave takes.
//
// The signature order of the worksets puts groups with similar column sets
// next to each other, but a block workset of large groups (the rows of the
// power-law hubs: 8192-nonzero groups hold half of the ~264 M nonzeros of the
// C3 graph) is still walked group after group, and a group's tiles, its
// columns ascending, each cover another stretch of the column range. Waves
// running at the same time then gather from all over B (SpMM) or Y (SDDMM).
// The locality order sorts the block tiles of all worksets together by the
// first (smallest) column of each tile, stably, and runs the residue tasks
// after them in stored order: waves running together then gather rows from
// one narrow stretch of column ids, which the L2s hold. Each task's work is
// unchanged (same tile, same groups, same output positions), so SDDMM results
// are bitwise those of the stored order and SpMM's differ only in the order
// of FP32 atomic additions.
//
// Measured on MI355X, signature-ordered worksets at 256 CUs: C3 (264 M
// nonzeros) SDDMM N=128 10.28 -> 7.78 ms, SpMM N=32 2.24 -> 2.05 ms, N=128
// 8.51 -> 8.11 ms; C1 SDDMM N=128 2.46 -> 2.29 ms, SpMM N=32 0.57 -> 0.56 ms.
#include "ps_common.hpp"

namespace ps {
namespace {

constexpr int kThreads = 256;
constexpr uint32_t kResidueKey = 0x80000000u;  // after every column id (< 2^31)
constexpr uint32_t kSkipKey = 0xFFFFFFFFu;     // after everything: tiles left out

struct TaskKeyArgs {
  const int* col_ind[PS_MAX_WORKSETS];
  const uint8_t* skip[PS_MAX_WORKSETS];  // per 64-nonzero stretch: leave it out (or null)
  uint64_t nnz[PS_MAX_WORKSETS];         // block workset: group_num * group_size
  uint32_t task_begin[PS_MAX_WORKSETS + 1];
  int residue[PS_MAX_WORKSETS];  // 1 for the residue workset
  int count;
  int tile_nnz;
  int residue_groups;
  uint32_t total;
};

// key[t] = the first column of block tile t (its nonzeros are stored columns
// ascending within each group), kResidueKey for residue tasks, kSkipKey for a
// block tile whose 64-nonzero stretches are all marked in skip; val[t] = t.
// *skipped counts the kSkipKey tiles.
__global__ __launch_bounds__(kThreads) void task_keys_kernel(TaskKeyArgs a, uint32_t* keys,
                                                             uint32_t* vals,
                                                             unsigned int* skipped) {
  for (uint32_t t = blockIdx.x * kThreads + threadIdx.x; t < a.total;
       t += gridDim.x * kThreads) {
    int q = 0;
    while (q + 1 < a.count && t >= a.task_begin[q + 1]) ++q;
    const uint32_t local = t - a.task_begin[q];
    uint32_t key = kResidueKey;
    if (!a.residue[q]) {
      const uint64_t first = uint64_t(local) * uint64_t(a.tile_nnz);
      key = uint32_t(a.col_ind[q][first]);
      if (a.skip[q]) {
        const uint64_t end = first + uint64_t(a.tile_nnz) < a.nnz[q] ? first + a.tile_nnz
                                                                       : a.nnz[q];
        bool all = true;
        for (uint64_t j = first / 64; all && j <= (end - 1) / 64; ++j) all = a.skip[q][j] != 0;
        if (all) {
          key = kSkipKey;
          atomicAdd(skipped, 1u);
        }
      }
    }
    keys[t] = key;
    vals[t] = t;
  }
}

// Task shape of an operator at width N, or false for an unknown operator.
bool shape_of(int op, int N, TaskShape* shape) {
  if (op == PS_OP_SPMM) {
    *shape = spmm_task_shape(N);
    return true;
  }
  if (op == PS_OP_SDDMM) {
    *shape = sddmm_task_shape();
    return true;
  }
  return false;
}

// The launch's tasks (launch order: worksets from the largest group size
// down to the residue, empty ones skipped), as TaskKeyArgs.
int task_table(int op, int N, int workset_count, const ps_workset* worksets, TaskKeyArgs* a) {
  PS_CHECK_ARG(workset_count >= 1 && workset_count <= PS_MAX_WORKSETS && worksets,
               "task order: invalid workset count");
  TaskShape shape;
  PS_CHECK_ARG(shape_of(op, N, &shape), "task order: unknown operator");
  PS_CHECK_ARG(N > 0 && N % 32 == 0, "task order: N must be a positive multiple of 32");
  *a = TaskKeyArgs{};
  a->tile_nnz = shape.tile_nnz;
  a->residue_groups = shape.residue_groups;
  uint64_t total = 0;
  int n = 0;
  for (int q = 0; q < workset_count; ++q) {
    const int s = workset_count - 1 - q;
    const ps_workset& w = worksets[s];
    if (w.group_num <= 0) continue;
    PS_CHECK_ARG(w.col_ind, "task order: missing workset columns");
    uint64_t t;
    if (s > 0) {
      PS_CHECK_ARG(w.group_size >= 32 && (w.group_size & (w.group_size - 1)) == 0,
                   "task order: block group size must be a power of two >= 32");
      t = (uint64_t(w.group_num) * uint64_t(w.group_size) + shape.tile_nnz - 1) /
          uint64_t(shape.tile_nnz);
    } else {
      t = (uint64_t(w.group_num) + shape.residue_groups - 1) / uint64_t(shape.residue_groups);
    }
    a->col_ind[n] = w.col_ind;
    a->nnz[n] = s > 0 ? uint64_t(w.group_num) * uint64_t(w.group_size) : 0;
    a->residue[n] = s == 0;
    a->task_begin[n] = uint32_t(total);
    total += t;
    PS_CHECK_ARG(total < (1ull << 31), "task order: too many tasks");
    ++n;
  }
  a->count = n;
  a->task_begin[n] = uint32_t(total);
  a->total = uint32_t(total);
  return PS_OK;
}

// The locality order of the launch's tasks, the skipped tiles last;
// *kept = the tasks before them (all of them without skip flags).
int build_order(int op, int N, int workset_count, const ps_workset* worksets,
                const uint8_t* const* skip, uint32_t* order, uint32_t count,
                uint32_t* kept, ps_stream_t stream) {
  TaskKeyArgs a;
  const int rc = task_table(op, N, workset_count, worksets, &a);
  if (rc != PS_OK) return rc;
  PS_CHECK_ARG(count == a.total, "ps_task_order_build: order holds " + std::to_string(count) +
                                     " tasks, the launch " + std::to_string(a.total));
  if (skip) {
    // task_table lists the non-empty worksets from the largest group size down
    int n = 0;
    for (int q = 0; q < workset_count; ++q) {
      const int s = workset_count - 1 - q;
      if (worksets[s].group_num <= 0) continue;
      a.skip[n++] = s > 0 ? skip[s] : nullptr;
    }
  }
  if (kept) *kept = a.total;
  if (a.total == 0) return PS_OK;
  PS_CHECK_ARG(order, "ps_task_order_build: null order");
  const size_t n = a.total;
  const size_t radix_ws = ps_radix_workspace_bytes(n);
  auto round = [](size_t b) { return (b + 255) & ~size_t(255); };
  const size_t bytes = 3 * round(n * 4) + round(radix_ws) + 256;
  char* base = nullptr;
  PS_HIP(ps::dev_malloc(&base, bytes));
  uint32_t* keys = reinterpret_cast<uint32_t*>(base);
  uint32_t* keys_alt = reinterpret_cast<uint32_t*>(base + round(n * 4));
  uint32_t* vals = reinterpret_cast<uint32_t*>(base + 2 * round(n * 4));
  void* ws = base + 3 * round(n * 4);
  unsigned int* skipped = reinterpret_cast<unsigned int*>(base + 3 * round(n * 4) + round(radix_ws));
  hipStream_t st = to_hip(stream);
  hipError_t e = hipMemsetAsync(skipped, 0, sizeof(unsigned int), st);
  const size_t blocks = (n + kThreads - 1) / kThreads;
  if (e == hipSuccess) {
    task_keys_kernel<<<unsigned(blocks < 65536 ? blocks : 65536), kThreads, 0, st>>>(a, keys, vals,
                                                                                    skipped);
    e = hipGetLastError();
  }
  int alt = 0;
  int r = PS_OK;
  // values sort into vals or order (the alternate buffer); stable, 32 key bits
  if (e == hipSuccess)
    r = ps_radix_sort_pairs_u32(keys, keys_alt, vals, order, n, 0, 32, ws, &alt, stream);
  if (e == hipSuccess && r == PS_OK && !alt)
    e = hipMemcpyAsync(order, vals, n * 4, hipMemcpyDeviceToDevice, st);
  unsigned int host_skipped = 0;
  if (e == hipSuccess && r == PS_OK)
    e = hipMemcpyAsync(&host_skipped, skipped, sizeof(host_skipped), hipMemcpyDeviceToHost, st);
  if (e == hipSuccess) e = hipStreamSynchronize(st);
  ps::dev_free(base);
  if (r != PS_OK) return r;
  PS_HIP(e);
  if (kept) *kept = a.total - host_skipped;
  return PS_OK;
}

}  // namespace
}  // namespace ps

extern "C" {

int ps_task_count(int op, int N, int workset_count, const ps_workset* worksets,
                  uint32_t* count) {
  PS_CHECK_ARG(count, "ps_task_count: null output");
  ps::TaskKeyArgs a;
  const int rc = ps::task_table(op, N, workset_count, worksets, &a);
  if (rc != PS_OK) return rc;
  *count = a.total;
  return PS_OK;
}

int ps_task_order_build(int op, int N, int workset_count, const ps_workset* worksets,
                        uint32_t* order, uint32_t count, ps_stream_t stream) {
  return ps::build_order(op, N, workset_count, worksets, nullptr, order, count, nullptr, stream);
}

int ps_task_order_build_subset(int op, int N, int workset_count, const ps_workset* worksets,
                               const uint8_t* const* skip, uint32_t* order, uint32_t count,
                               uint32_t* kept, ps_stream_t stream) {
  PS_CHECK_ARG(skip && kept, "ps_task_order_build_subset: null argument");
  return ps::build_order(op, N, workset_count, worksets, skip, order, count, kept, stream);
}

}  // extern "C"
