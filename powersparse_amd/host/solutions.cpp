// Operator dispatchers: argument checks of the reference, then one fused
// launch over every workset through the C ABI.
//
// The reference launches one kernel per workset on its own stream and then
// synchronises the device when there is more than one workset
// (PowerSparse_SpMM/spmm_solution.cu:7-34, PowerSparse_SDDMM/sddmm_solution.cu:7-50).
// Here every workset is covered by a single launch (ps_spmm_launch /
// ps_sddmm_launch), enqueued on the first supplied stream after the others are
// joined into it; the synchronisation contract is kept: asynchronous for one
// workset, device-synchronising for more.
#include <stdexcept>
#include <vector>

#include "PowerSparse_SDDMM.h"
#include "PowerSparse_SpMM.h"

namespace PowerSparse {
namespace {

// The worksets the kernels run: the public ones or the row-ordered copy.
std::vector<ps_workset> Worksets(const PowerSparseMatrixGPU& m, const ExecutionLayout& e) {
  std::vector<ps_workset> ws(static_cast<size_t>(m.GroupTypeNum()));
  for (int s = 0; s < m.GroupTypeNum(); ++s) {
    ws[size_t(s)].col_ind = e.col_ind[s];
    ws[size_t(s)].sp_data = e.sp_data[s];
    ws[size_t(s)].group_des = e.group_des[s];
    ws[size_t(s)].group_num = m.GroupNum()[s];
    ws[size_t(s)].group_size = s == 0 ? 0 : GROUP_SIZE(s);
    ws[size_t(s)].order = nullptr;  // groups run as stored
  }
  return ws;
}

void CheckSpmmArgs(const PowerSparseMatrixGPU& m, int N, const float* B, float* C) {
  if (N <= 0 || N % 32 != 0 || N / 32 > 65535)
    throw std::invalid_argument("SpMM requires N to be a positive multiple of 32, with N/32 <= 65535");
  ValidateDenseShape(m.MatrixRow(), m.MatrixCol(), N);
  if (!B || !C) throw std::invalid_argument("Invalid SpMM buffers or stream count");
}

void CheckSddmmArgs(const PowerSparseMatrixGPU& m, int N, const float* lhs, const float* rhs,
                    const void* out) {
  if (N <= 0 || N % 32 != 0 || N > 512)
    throw std::invalid_argument(
        "SDDMM dispatcher expects a width N that is a multiple of 32 between 32 and 512");
  ValidateDenseShape(m.MatrixRow(), m.MatrixCol(), N);
  if (!lhs || !rhs || !out) throw std::invalid_argument("Invalid SDDMM buffers or stream count");
}

// The reference runs workset s on streams[s] (spmm_solution.cu:18-26,
// sddmm_solution.cu:24-26), so work a caller queued on streams[s] before the
// call runs before that workset. The fused launch goes to streams[0]; every
// other distinct stream is joined into it first, which keeps that ordering.
// The events are released after the dispatcher's device synchronisation.
class StreamJoin {
 public:
  StreamJoin(int count, const ps_stream_t* streams) {
    for (int s = 1; s < count; ++s) {
      if (streams[s] == streams[0]) continue;
      ps_event_t e = nullptr;
      ThrowOnError(ps_event_create(&e));
      events_.push_back(e);
      ThrowOnError(ps_event_record(e, streams[s]));
      ThrowOnError(ps_stream_wait_event(streams[0], e));
    }
  }
  ~StreamJoin() {
    for (ps_event_t e : events_) ps_event_destroy(e);
  }
  StreamJoin(const StreamJoin&) = delete;
  StreamJoin& operator=(const StreamJoin&) = delete;

 private:
  std::vector<ps_event_t> events_;
};

}  // namespace

void SpMMAsync(const PowerSparseMatrixGPU& matrix, int N, const float* B, float* C,
               ps_stream_t stream) {
  CheckSpmmArgs(matrix, N, B, C);
  // the tuned partition when the matrix keeps one (SpmmPartition::kTuned)
  const PowerSparseMatrixGPU& m = matrix.SpmmMatrix();
  const ExecutionLayout e = m.Execution();
  const auto ws = Worksets(m, e);
  const int k = RunOrderSlot(PS_OP_SPMM, N);
  if (e.run_order[k])
    ThrowOnError(ps_spmm_launch_ordered(m.GroupTypeNum(), ws.data(), e.residue_offset,
                                        reinterpret_cast<const uint8_t*>(e.residue_atomic),
                                        m.MatrixRow(), m.MatrixCol(), N, B, C, e.task_chunk,
                                        e.run_order[k], e.run_order_tasks[k], stream));
  else
    ThrowOnError(ps_spmm_launch(m.GroupTypeNum(), ws.data(), e.residue_offset,
                                reinterpret_cast<const uint8_t*>(e.residue_atomic),
                                m.MatrixRow(), m.MatrixCol(), N, B, C, e.task_chunk, stream));
  // the dense hub block's rows (the tuned partition holds the rest)
  if (matrix.HubBlockUsed()) matrix.HubSpmm(N, B, C, stream);
}

void SpMM(const PowerSparseMatrixGPU& m, int N, const float* B, float* C, int stream_count,
          const ps_stream_t* streams) {
  CheckSpmmArgs(m, N, B, C);
  if (stream_count != m.GroupTypeNum() || (stream_count > 1 && !streams))
    throw std::invalid_argument("Invalid SpMM buffers or stream count");
  if (stream_count == 1) {
    SpMMAsync(m, N, B, C, nullptr);
    return;
  }
  StreamJoin join(stream_count, streams);
  SpMMAsync(m, N, B, C, streams[0]);
  ThrowOnError(ps_device_synchronize());
}

void SDDMMAsync(const PowerSparseMatrixGPU& m, int N, const float* lhs, const float* rhs,
                float* const* out, ps_stream_t stream) {
  CheckSddmmArgs(m, N, lhs, rhs, out);
  for (int s = 0; s < m.GroupTypeNum(); ++s)
    if (m.GroupNum()[s] != 0 && !out[s]) throw std::invalid_argument("Missing SDDMM output workset");
  const ExecutionLayout e = m.Execution();
  const auto ws = Worksets(m, e);
  if (e.out_base)  // row-ordered copy: results written to the public layout
    ThrowOnError(ps_sddmm_scatter_launch(m.GroupTypeNum(), ws.data(), e.residue_offset,
                                         e.out_base, m.MatrixRow(), m.MatrixCol(), N, lhs, rhs,
                                         out, e.task_chunk, stream));
  else if (e.run_order[RunOrderSlot(PS_OP_SDDMM, N)])
    ThrowOnError(ps_sddmm_launch_ordered(m.GroupTypeNum(), ws.data(), e.residue_offset,
                                         m.MatrixRow(), m.MatrixCol(), N, lhs, rhs, out,
                                         e.task_chunk, e.run_order[RunOrderSlot(PS_OP_SDDMM, N)],
                                         e.run_order_tasks[RunOrderSlot(PS_OP_SDDMM, N)],
                                         stream));
  else
    ThrowOnError(ps_sddmm_launch(m.GroupTypeNum(), ws.data(), e.residue_offset, m.MatrixRow(),
                                 m.MatrixCol(), N, lhs, rhs, out, e.task_chunk, stream));
  // the groups inside the dense hub block (left out of the run order)
  if (m.HubBlockUsed()) m.HubSddmm(N, lhs, rhs, out, nullptr, stream);
}

void SDDMMToCSR(const PowerSparseMatrixGPU& m, int N, const float* lhs, const float* rhs,
                float* out_csr, ps_stream_t stream) {
  CheckSddmmArgs(m, N, lhs, rhs, out_csr);
  if (!m.WorksetCSRPosition())
    throw std::invalid_argument(
        "SDDMMToCSR needs a matrix built with PartitionPolicy::csr_positions");
  const ExecutionLayout e = m.Execution();
  const auto ws = Worksets(m, e);
  const int k = RunOrderSlot(PS_OP_SDDMM, N);
  if (e.run_order[k])
    ThrowOnError(ps_sddmm_csr_launch_ordered(m.GroupTypeNum(), ws.data(), e.residue_offset,
                                             e.csr_pos, m.MatrixRow(), m.MatrixCol(), N, lhs,
                                             rhs, out_csr, e.task_chunk, e.run_order[k],
                                             e.run_order_tasks[k], stream));
  else
    ThrowOnError(ps_sddmm_csr_launch(m.GroupTypeNum(), ws.data(), e.residue_offset, e.csr_pos,
                                     m.MatrixRow(), m.MatrixCol(), N, lhs, rhs, out_csr,
                                     e.task_chunk, stream));
  if (m.HubBlockUsed()) m.HubSddmm(N, lhs, rhs, nullptr, out_csr, stream);
}

void WorksetToCSR(const PowerSparseMatrixGPU& m, const float* const* values, float* out_csr,
                  ps_stream_t stream) {
  if (!values || !out_csr) throw std::invalid_argument("Invalid WorksetToCSR buffers");
  if (!m.WorksetCSRPosition())
    throw std::invalid_argument(
        "WorksetToCSR needs a matrix built with PartitionPolicy::csr_positions");
  const int S = m.GroupTypeNum();
  std::vector<long long> lengths(static_cast<size_t>(S));
  for (int s = 0; s < S; ++s) {
    if (s == 0) {
      int total = 0;
      if (m.GroupNum()[0] > 0)
        ThrowOnError(ps_memcpy_dtoh(&total, m.ResidueOffset() + m.GroupNum()[0], sizeof(int)));
      lengths[0] = total;
    } else {
      lengths[size_t(s)] = (long long)m.GroupNum()[s] * GROUP_SIZE(s);
    }
  }
  ThrowOnError(ps_workset_to_csr(S, lengths.data(), m.WorksetCSRPosition(), values, out_csr,
                                 stream));
}

void SDDMM(const PowerSparseMatrixGPU& m, int N, const float* lhs, const float* rhs,
           float** out, int stream_count, const ps_stream_t* streams) {
  CheckSddmmArgs(m, N, lhs, rhs, out);
  if (stream_count != m.GroupTypeNum() || (stream_count > 1 && !streams))
    throw std::invalid_argument("Invalid SDDMM buffers or stream count");
  if (stream_count == 1) {
    SDDMMAsync(m, N, lhs, rhs, out, nullptr);
    return;
  }
  StreamJoin join(stream_count, streams);
  SDDMMAsync(m, N, lhs, rhs, out, streams[0]);
  ThrowOnError(ps_device_synchronize());
}

}  // namespace PowerSparse
