// C facade (include/powersparse.h) over the C++17 API.
#include "powersparse.h"

#include <cstring>
#include <exception>
#include <random>
#include <stdexcept>
#include <string>

#include "PowerSparse_SDDMM.h"
#include "PowerSparse_SpMM.h"
#include "matrix_market.h"
#include "preprocess_host.h"
#include "synth.h"

struct psx_matrix {
  PowerSparse::PowerSparseMatrixGPU* m = nullptr;
};
struct psx_csr {
  PowerSparse::HostCsr csr;
};

namespace {

thread_local std::string g_error;

template <typename F>
int Guard(F&& f) {
  try {
    f();
    return PS_OK;
  } catch (const std::invalid_argument& e) {
    g_error = e.what();
    return PS_ERR_INVALID;
  } catch (const std::exception& e) {
    g_error = e.what();
    return PS_ERR_RUNTIME;
  } catch (...) {
    g_error = "unknown error";
    return PS_ERR_RUNTIME;
  }
}

void Need(bool ok, const char* what) {
  if (!ok) throw std::invalid_argument(what);
}

int CsrOut(psx_csr** out, PowerSparse::HostCsr&& csr) {
  *out = new psx_csr{std::move(csr)};
  return PS_OK;
}

}  // namespace

extern "C" {

const char* psx_last_error(void) { return g_error.c_str(); }

int psx_matrix_create(int rows, int cols, int nnz, const int* row_ptr, const int* col_ind,
                      const float* sp_data, int cu_count, double* timings_ms, psx_matrix** out) {
  psx_build_options options{cu_count, PSX_ORDER_AUTO, 0, PSX_TASK_AUTO, 0, 0, 0, 0, {}, {}};
  return psx_matrix_create_ex(rows, cols, nnz, row_ptr, col_ind, sp_data, &options, timings_ms,
                              out);
}

int psx_matrix_create_ex(int rows, int cols, int nnz, const int* row_ptr, const int* col_ind,
                         const float* sp_data, const psx_build_options* options,
                         double* timings_ms, psx_matrix** out) {
  return Guard([&] {
    Need(out != nullptr, "psx_matrix_create: null output");
    *out = nullptr;
    PowerSparse::PartitionPolicy policy;
    if (options) {
      policy.cu_count = options->cu_count;
      policy.signature_order = static_cast<PowerSparse::SignatureOrder>(options->signature_order);
      policy.csr_positions = options->csr_positions != 0;
      policy.task_order = static_cast<PowerSparse::TaskOrder>(options->task_order);
      policy.run_order = options->stored_order == 0;
      policy.max_group_types = options->max_group_types;
      policy.spmm_partition = options->parity_spmm ? PowerSparse::SpmmPartition::kParity
                                                   : PowerSparse::SpmmPartition::kTuned;
      policy.hub_block = options->no_hub_block ? PowerSparse::HubBlock::kOff
                                               : PowerSparse::HubBlock::kAuto;
      for (int k = 0; k < PSX_HUB_MAX_TIERS && k < PowerSparse::kHubMaxTiers; ++k) {
        policy.hub_min_degree[k] = options->hub_min_degree[k];
        policy.hub_min_count[k] = options->hub_min_count[k];
      }
    }
    PowerSparse::PreprocessTimings t;
    auto* m = new PowerSparse::PowerSparseMatrixGPU(rows, cols, nnz, row_ptr, col_ind, sp_data,
                                                    policy, timings_ms ? &t : nullptr);
    *out = new psx_matrix{m};
    if (timings_ms) {
      const double v[9] = {t.upload_ms, t.analyze_ms, t.rank_ms,  t.groups_ms, t.sigbit_ms,
                           t.signature_ms, t.order_ms, t.gather_ms, t.total_ms};
      std::memcpy(timings_ms, v, sizeof(v));
    }
  });
}

int psx_matrix_signature_order(const psx_matrix* m, int* method) {
  return Guard([&] {
    Need(m && m->m && method, "psx_matrix_signature_order: null argument");
    *method = int(m->m->SignatureOrderUsed());
  });
}

int psx_matrix_task_order(const psx_matrix* m, int* order, double* score_signature,
                          double* score_row) {
  return Guard([&] {
    Need(m && m->m, "psx_matrix_task_order: null matrix");
    if (order) *order = int(m->m->TaskOrderUsed());
    if (score_signature) *score_signature = m->m->LocalityScore(PowerSparse::TaskOrder::kSignature);
    if (score_row) *score_row = m->m->LocalityScore(PowerSparse::TaskOrder::kRow);
  });
}

int psx_matrix_run_order(const psx_matrix* m, int* used) {
  return Guard([&] {
    Need(m && m->m && used, "psx_matrix_run_order: null argument");
    *used = m->m->RunOrderUsed() ? 1 : 0;
  });
}

int psx_matrix_spmm_worksets(const psx_matrix* m, int* group_type_num) {
  return Guard([&] {
    Need(m && m->m && group_type_num, "psx_matrix_spmm_worksets: null argument");
    *group_type_num = m->m->SpmmMatrix().GroupTypeNum();
  });
}

int psx_matrix_hub_block(const psx_matrix* m, int* tiers, int tier, int* rows, int* cols) {
  return Guard([&] {
    Need(m && m->m, "psx_matrix_hub_block: null matrix");
    if (tiers) *tiers = m->m->HubTiers();
    if (rows) *rows = m->m->HubRows(tier);
    if (cols) *cols = m->m->HubCols(tier);
  });
}

int psx_matrix_destroy(psx_matrix* m) {
  return Guard([&] {
    if (!m) return;
    delete m->m;
    delete m;
  });
}

int psx_matrix_info(const psx_matrix* m, int* rows, int* cols, int* nnz, int* group_type_num,
                    int* fine, int* signature_len, int* cu_count) {
  return Guard([&] {
    Need(m && m->m, "psx_matrix_info: null matrix");
    if (rows) *rows = m->m->MatrixRow();
    if (cols) *cols = m->m->MatrixCol();
    if (nnz) *nnz = m->m->MatrixNNZ();
    if (group_type_num) *group_type_num = m->m->GroupTypeNum();
    if (fine) *fine = m->m->GroupFineSize();
    if (signature_len) *signature_len = m->m->SignatureLen();
    if (cu_count) *cu_count = m->m->PartitionCuCount();
  });
}

int psx_matrix_group_num(const psx_matrix* m, int* group_num) {
  return Guard([&] {
    Need(m && m->m && group_num, "psx_matrix_group_num: null argument");
    std::memcpy(group_num, m->m->GroupNum(), sizeof(int) * size_t(m->m->GroupTypeNum()));
  });
}

int psx_matrix_workset(const psx_matrix* m, int s, const int** col_ind, const float** sp_data,
                       const int** group_des) {
  return Guard([&] {
    Need(m && m->m, "psx_matrix_workset: null matrix");
    Need(s >= 0 && s < m->m->GroupTypeNum(), "psx_matrix_workset: workset out of range");
    if (col_ind) *col_ind = m->m->WorksetColInd()[s];
    if (sp_data) *sp_data = m->m->WorksetSpData()[s];
    if (group_des) *group_des = m->m->GroupDestination()[s];
  });
}

int psx_matrix_residue(const psx_matrix* m, const int** offset, const uint8_t** atomic) {
  return Guard([&] {
    Need(m && m->m, "psx_matrix_residue: null matrix");
    if (offset) *offset = m->m->ResidueOffset();
    if (atomic) *atomic = reinterpret_cast<const uint8_t*>(m->m->ResidueAtomic());
  });
}

int psx_spmm(const psx_matrix* m, int N, const float* B, float* C, int stream_count,
             const ps_stream_t* streams) {
  return Guard([&] {
    Need(m && m->m, "psx_spmm: null matrix");
    PowerSparse::SpMM(*m->m, N, B, C, stream_count, streams);
  });
}

int psx_spmm_async(const psx_matrix* m, int N, const float* B, float* C, ps_stream_t stream) {
  return Guard([&] {
    Need(m && m->m, "psx_spmm_async: null matrix");
    PowerSparse::SpMMAsync(*m->m, N, B, C, stream);
  });
}

int psx_sddmm(const psx_matrix* m, int N, const float* lhs, const float* rhs, float** out,
              int stream_count, const ps_stream_t* streams) {
  return Guard([&] {
    Need(m && m->m, "psx_sddmm: null matrix");
    PowerSparse::SDDMM(*m->m, N, lhs, rhs, out, stream_count, streams);
  });
}

int psx_sddmm_async(const psx_matrix* m, int N, const float* lhs, const float* rhs,
                    float* const* out, ps_stream_t stream) {
  return Guard([&] {
    Need(m && m->m, "psx_sddmm_async: null matrix");
    PowerSparse::SDDMMAsync(*m->m, N, lhs, rhs, out, stream);
  });
}

int psx_sddmm_csr(const psx_matrix* m, int N, const float* lhs, const float* rhs,
                  float* out_csr, ps_stream_t stream) {
  return Guard([&] {
    Need(m && m->m, "psx_sddmm_csr: null matrix");
    PowerSparse::SDDMMToCSR(*m->m, N, lhs, rhs, out_csr, stream);
  });
}

int psx_workset_to_csr(const psx_matrix* m, const float* const* values, float* out_csr,
                       ps_stream_t stream) {
  return Guard([&] {
    Need(m && m->m, "psx_workset_to_csr: null matrix");
    PowerSparse::WorksetToCSR(*m->m, values, out_csr, stream);
  });
}

int psx_matrix_csr_position(const psx_matrix* m, int s, const int** pos) {
  return Guard([&] {
    Need(m && m->m && pos, "psx_matrix_csr_position: null argument");
    Need(s >= 0 && s < m->m->GroupTypeNum(), "psx_matrix_csr_position: workset out of range");
    *pos = m->m->WorksetCSRPosition() ? m->m->WorksetCSRPosition()[s] : nullptr;
  });
}

int psx_csr_read_mtx(const char* path, psx_csr** out) {
  return Guard([&] {
    Need(path && out, "psx_csr_read_mtx: null argument");
    CsrOut(out, PowerSparse::ReadMatrixMarket(path));
  });
}

int psx_csr_read_binary(const char* path, psx_csr** out) {
  return Guard([&] {
    Need(path && out, "psx_csr_read_binary: null argument");
    CsrOut(out, PowerSparse::ReadBinaryCsr(path));
  });
}

int psx_csr_write_binary(const psx_csr* csr, const char* path) {
  return Guard([&] {
    Need(csr && path, "psx_csr_write_binary: null argument");
    PowerSparse::WriteBinaryCsr(path, csr->csr);
  });
}

int psx_csr_synth(const char* config, uint64_t seed, int scale, psx_csr** out) {
  return Guard([&] {
    Need(config && out, "psx_csr_synth: null argument");
    CsrOut(out, PowerSparse::SynthConfig(config, seed, scale));
  });
}

int psx_csr_chung_lu(int n, double gamma, double mean_deg, double max_deg, float val_lo,
                     float val_hi, uint64_t seed, psx_csr** out) {
  return Guard([&] {
    Need(out != nullptr, "psx_csr_chung_lu: null output");
    CsrOut(out, PowerSparse::SynthChungLu(n, gamma, mean_deg, max_deg, val_lo, val_hi, seed));
  });
}

int psx_csr_uniform_degree(int rows, int cols, int deg_lo, int deg_hi, float val_lo,
                           float val_hi, uint64_t seed, psx_csr** out) {
  return Guard([&] {
    Need(out != nullptr, "psx_csr_uniform_degree: null output");
    CsrOut(out, PowerSparse::SynthUniformDegree(rows, cols, deg_lo, deg_hi, val_lo, val_hi, seed));
  });
}

int psx_csr_community(int communities, int block, double p_intra, double inter_mean,
                      double empty_frac, double single_frac, float val_lo, float val_hi,
                      uint64_t seed, psx_csr** out) {
  return Guard([&] {
    Need(out != nullptr, "psx_csr_community: null output");
    CsrOut(out, PowerSparse::SynthCommunity(communities, block, p_intra, inter_mean, empty_frac,
                                            single_frac, val_lo, val_hi, seed));
  });
}

int psx_csr_info(const psx_csr* csr, int* rows, int* cols, int* nnz) {
  return Guard([&] {
    Need(csr != nullptr, "psx_csr_info: null csr");
    if (rows) *rows = csr->csr.rows;
    if (cols) *cols = csr->csr.cols;
    if (nnz) *nnz = csr->csr.nnz();
  });
}

int psx_csr_arrays(const psx_csr* csr, const int** row_ptr, const int** col_ind,
                   const float** values) {
  return Guard([&] {
    Need(csr != nullptr, "psx_csr_arrays: null csr");
    if (row_ptr) *row_ptr = csr->csr.row_ptr.data();
    if (col_ind) *col_ind = csr->csr.col_ind.data();
    if (values) *values = csr->csr.values.data();
  });
}

int psx_csr_free(psx_csr* csr) {
  delete csr;
  return PS_OK;
}

int psx_generate_sigbit(int cols, const int* col_nnz, int ffc, int* sigbit, int* signature_len) {
  return Guard([&] {
    Need(cols > 0 && col_nnz && sigbit && signature_len && ffc >= 0,
         "psx_generate_sigbit: bad argument");
    *signature_len = PowerSparse::GenerateSigBitFFC(cols, col_nnz, ffc, sigbit);
  });
}

int psx_workset_count(const unsigned long long* degree_sums, int cu_count, int* group_type_num) {
  return Guard([&] {
    Need(degree_sums && group_type_num && cu_count > 0, "psx_workset_count: bad argument");
    *group_type_num = PowerSparse::WorksetCount(degree_sums, cu_count);
  });
}

int psx_dense_input(unsigned seed, size_t n1, float* out1, size_t n2, float* out2) {
  return Guard([&] {
    Need((n1 == 0 || out1) && (n2 == 0 || out2), "psx_dense_input: null output");
    std::mt19937 rng(seed);
    for (size_t i = 0; i < n1; ++i) out1[i] = float(rng() % 3) / 10.0f;
    for (size_t i = 0; i < n2; ++i) out2[i] = float(rng() % 3) / 10.0f;
  });
}

}  // extern "C"
