// The CSV benchmark harness behind powersparse_spmm / powersparse_sddmm
// (cli/main.cpp), as a library entry point (psx_bench_main,
// include/powersparse_bench.h) so that callers can also run it in process:
//
//   powersparse_{spmm,sddmm} MATRIX N DEVICE CHECK REPEATS
//   powersparse_{spmm,sddmm} --header
//
// MATRIX is a MatrixMarket file, a binary CSR (*.pscsr) or
// "synth:NAME[:SEED[:SCALE]]" (the seeded benchmark graphs). N is 32, 64 or
// 128. CHECK=1 verifies the worksets and one operator call against a CPU
// reference before timing.
//
// The contract kept from the reference harness (ParCIS/PowerSparse
// benchmarks/benchmark.cu:98-213, benchmark_utils.h:100-115, README.md:27-42),
// because scripts and the batch runner depend on it: the arguments and exit
// codes (0 success, 1 error with "Error: ..." on stderr, 2 usage or an
// unselected N), the CSV header and row, the dense inputs (one std::mt19937
// seeded 1, values (rng() % 3) / 10, SDDMM's lhs drawn before rhs), the check
// tolerance |a - e| <= 1e-3 + 1e-3 |e| against double sums, and the timing
// protocol (30 warm-up calls, then REPEATS calls between two events on the
// null stream, outputs not cleared between calls; preprocessing timed on the
// host around the constructor with device synchronisations on both sides).
// compute_capability carries the gfx architecture and cuda_runtime /
// cuda_driver the HIP runtime and driver versions.
//
// Structure: the operator under test is a Workload (SpMM or SDDMM) owning its
// device operands through the host library's DeviceArray; Bench() builds the
// matrix and drives clear / call / verify / time over the workload.
#include <algorithm>
#include <chrono>
#include <cmath>
#include <cstdint>
#include <cstring>
#include <iomanip>
#include <iostream>
#include <memory>
#include <random>
#include <sstream>
#include <stdexcept>
#include <string>
#include <vector>

#include "PowerSparse_SDDMM.h"
#include "PowerSparse_SpMM.h"
#include "device_buffer.h"
#include "matrix_market.h"
#include "powersparse_bench.h"
#include "synth.h"

namespace {

using PowerSparse::DeviceArray;
using PowerSparse::HostCsr;
using PowerSparse::PowerSparseMatrixGPU;
using PowerSparse::ThrowOnError;

constexpr int kWarmupCalls = 30;
constexpr unsigned kInputSeed = 1;
constexpr const char* kCsvHeader =
    "algorithm,operator,matrix,rows,cols,nnz,N,device,gpu,compute_capability,"
    "cuda_runtime,cuda_driver,warmup,repeats,seed,check,preprocess_ms,ms,gflops";

// ------------------------------------------------------------- arguments

// A whole-string decimal int; "Invalid NAME: TEXT" when it does not parse,
// "Invalid NAME" when characters follow the number.
int WholeInt(const char* text, const char* name) {
  const std::string s(text);
  size_t used = 0;
  int v = 0;
  try {
    v = std::stoi(s, &used);
  } catch (...) {
    throw std::invalid_argument(std::string("Invalid ") + name + ": " + s);
  }
  if (used != s.size()) throw std::invalid_argument(std::string("Invalid ") + name);
  return v;
}

struct Spec {
  std::string matrix;
  int n = 0, device = 0, repeats = 0;
  bool check = false;
};

Spec ParseSpec(char** argv) {
  Spec s;
  s.matrix = argv[1];
  s.n = WholeInt(argv[2], "N");
  s.device = WholeInt(argv[3], "DEVICE");
  const int check = WholeInt(argv[4], "CHECK");
  s.repeats = WholeInt(argv[5], "REPEATS");
  if (s.device < 0 || (check != 0 && check != 1) || s.repeats <= 0)
    throw std::invalid_argument("DEVICE must be nonnegative, CHECK 0 or 1, and REPEATS positive");
  s.check = check == 1;
  return s;
}

void PrintUsage(const char* prog) {
  std::cerr << "Usage: " << prog << " MATRIX N DEVICE CHECK REPEATS\n"
            << "MATRIX: a .mtx file, a .pscsr binary CSR, or synth:NAME[:SEED[:SCALE]]\n"
            << "CHECK: 0=skip, 1=verify preprocessing and compare with a CPU reference\n"
            << "Benchmark widths are N=32, 64 or 128.\n";
}

// "synth:NAME[:SEED[:SCALE]]", "*.pscsr" or a MatrixMarket path.
HostCsr LoadMatrix(const std::string& spec) {
  const std::string tag = "synth:";
  if (spec.compare(0, tag.size(), tag) == 0) {
    std::vector<std::string> part;
    std::stringstream in(spec.substr(tag.size()));
    for (std::string p; std::getline(in, p, ':');) part.push_back(p);
    if (part.empty() || part.size() > 3) throw std::invalid_argument("Bad synthetic matrix: " + spec);
    const uint64_t seed = part.size() > 1 ? std::stoull(part[1]) : 1;
    const int scale = part.size() > 2 ? std::stoi(part[2]) : 1;
    return PowerSparse::SynthConfig(part[0], seed, scale);
  }
  const std::string ext = ".pscsr";
  if (spec.size() > ext.size() && spec.compare(spec.size() - ext.size(), ext.size(), ext) == 0)
    return PowerSparse::ReadBinaryCsr(spec);
  return PowerSparse::ReadMatrixMarket(spec);
}

// ------------------------------------------------------------- host views

// The reference harness's dense input generator.
std::vector<float> DrawDense(std::mt19937& rng, size_t count) {
  std::vector<float> v(count);
  std::generate(v.begin(), v.end(), [&rng] { return float(rng() % 3) / 10.0f; });
  return v;
}

bool WithinTolerance(float got, double want) {
  return std::isfinite(got) && std::isfinite(want) &&
         std::fabs(double(got) - want) <= 1e-3 + 1e-3 * std::fabs(want);
}

template <typename T>
std::vector<T> ToHost(const T* device, size_t count) {
  std::vector<T> h(count);
  if (count) ThrowOnError(ps_memcpy_dtoh(h.data(), device, count * sizeof(T)));
  return h;
}

// One workset in host memory: group g owns positions [begin[g], begin[g+1])
// and writes row dest[g].
struct HostWorkset {
  std::vector<int> dest, begin, col;
  std::vector<float> val;
};

std::vector<HostWorkset> FetchWorksets(const PowerSparseMatrixGPU& m) {
  std::vector<HostWorkset> all(static_cast<size_t>(m.GroupTypeNum()));
  const int g0 = m.GroupNum()[0];
  for (int s = 0; s < m.GroupTypeNum(); ++s) {
    HostWorkset& w = all[size_t(s)];
    const int groups = m.GroupNum()[s];
    w.dest = ToHost(m.GroupDestination()[s], size_t(groups));
    if (s == 0) {
      w.begin = ToHost(m.ResidueOffset(), size_t(g0) + 1);
    } else {
      w.begin.resize(size_t(groups) + 1);
      for (int g = 0; g <= groups; ++g) w.begin[size_t(g)] = g * GROUP_SIZE(s);
    }
    w.col = ToHost(m.WorksetColInd()[s], size_t(w.begin.back()));
    w.val = ToHost(m.WorksetSpData()[s], size_t(w.begin.back()));
  }
  return all;
}

// An entry's sort key inside its row: column, then the value's bits.
uint64_t EntryKey(int col, float v) {
  uint32_t bits;
  std::memcpy(&bits, &v, sizeof(bits));
  return (uint64_t(uint32_t(col)) << 32) | bits;
}

// The worksets hold exactly the CSR's entries (the reference harness checks
// the same multiset of (row, column, value), benchmark.cu:45-62): the
// worksets' entries are bucketed by row, and each row's keys, sorted, must
// equal the CSR row's. Values compare bitwise: the preprocessing copies them.
void VerifyWorksets(const HostCsr& csr, const std::vector<HostWorkset>& ws) {
  const size_t rows = size_t(csr.rows);
  std::vector<long long> start(rows + 1, 0);
  for (const HostWorkset& w : ws)
    for (size_t g = 0; g < w.dest.size(); ++g) {
      if (w.dest[g] < 0 || size_t(w.dest[g]) >= rows)
        throw std::runtime_error("Preprocessing changed the sparse matrix");
      start[size_t(w.dest[g]) + 1] += w.begin[g + 1] - w.begin[g];
    }
  for (size_t r = 0; r < rows; ++r) {
    start[r + 1] += start[r];
    if (start[r + 1] - start[r] != csr.row_ptr[r + 1] - csr.row_ptr[r])
      throw std::runtime_error("Preprocessing changed the sparse matrix");
  }
  std::vector<uint64_t> got(size_t(start.back()));
  std::vector<long long> fill(start.begin(), start.end() - 1);
  for (const HostWorkset& w : ws)
    for (size_t g = 0; g < w.dest.size(); ++g)
      for (int p = w.begin[g]; p < w.begin[g + 1]; ++p)
        got[size_t(fill[size_t(w.dest[g])]++)] = EntryKey(w.col[size_t(p)], w.val[size_t(p)]);
  std::vector<uint64_t> want(got.size());
  for (size_t k = 0; k < want.size(); ++k) want[k] = EntryKey(csr.col_ind[k], csr.values[k]);
  for (size_t r = 0; r < rows; ++r) {
    const long long a = start[r], b = start[r + 1];
    std::sort(got.begin() + a, got.begin() + b);
    std::sort(want.begin() + a, want.begin() + b);
    if (!std::equal(got.begin() + a, got.begin() + b, want.begin() + a))
      throw std::runtime_error("Preprocessing changed the sparse matrix");
  }
}

// ------------------------------------------------------------- workloads

// One operator with its device operands and outputs.
class Workload {
 public:
  virtual ~Workload() = default;
  virtual void ClearOutputs() = 0;  // zeroes the outputs (null stream)
  virtual void Call() = 0;          // one operator call through the drop-in API
  // Compares the outputs of one call with the CPU reference; throws on mismatch.
  virtual void Verify(const HostCsr& csr, const std::vector<HostWorkset>& ws) = 0;
};

// The drop-in operators take one stream per workset (asynchronous for one
// workset, device-synchronising for more); every workset gets the same stream.
class StreamList {
 public:
  explicit StreamList(int worksets) : list_(size_t(worksets), nullptr) {
    if (worksets > 1) {
      ThrowOnError(ps_stream_create(&own_));
      std::fill(list_.begin(), list_.end(), own_);
    }
  }
  ~StreamList() { ps_stream_destroy(own_); }
  StreamList(const StreamList&) = delete;
  StreamList& operator=(const StreamList&) = delete;
  int count() const { return int(list_.size()); }
  const ps_stream_t* data() const { return list_.data(); }

 private:
  ps_stream_t own_ = nullptr;
  std::vector<ps_stream_t> list_;
};

class SpmmWorkload final : public Workload {
 public:
  SpmmWorkload(const PowerSparseMatrixGPU& m, int n, std::mt19937& rng)
      : m_(m), n_(n), streams_(m.GroupTypeNum()),
        b_host_(DrawDense(rng, size_t(m.MatrixCol()) * size_t(n))),
        b_(b_host_.size()), c_(size_t(m.MatrixRow()) * size_t(n)) {
    b_.Upload(b_host_.data(), b_host_.size());
  }
  void ClearOutputs() override { c_.Zero(nullptr); }
  void Call() override {
    PowerSparse::SpMM(m_, n_, b_.data(), c_.data(), streams_.count(), streams_.data());
  }
  void Verify(const HostCsr& csr, const std::vector<HostWorkset>&) override {
    const std::vector<float> c = ToHost(c_.data(), c_.size());
    std::vector<double> sum(static_cast<size_t>(n_));
    for (int r = 0; r < csr.rows; ++r) {
      std::fill(sum.begin(), sum.end(), 0.0);
      for (int p = csr.row_ptr[size_t(r)]; p < csr.row_ptr[size_t(r) + 1]; ++p) {
        const double a = csr.values[size_t(p)];
        const float* brow = b_host_.data() + size_t(csr.col_ind[size_t(p)]) * size_t(n_);
        for (int j = 0; j < n_; ++j) sum[size_t(j)] += a * brow[j];
      }
      const float* crow = c.data() + size_t(r) * size_t(n_);
      for (int j = 0; j < n_; ++j)
        if (!WithinTolerance(crow[j], sum[size_t(j)]))
          throw std::runtime_error("SpMM mismatch at row " + std::to_string(r) + ", feature " +
                                   std::to_string(j));
    }
  }

 private:
  const PowerSparseMatrixGPU& m_;
  int n_;
  StreamList streams_;
  std::vector<float> b_host_;
  DeviceArray<float> b_, c_;
};

class SddmmWorkload final : public Workload {
 public:
  SddmmWorkload(const PowerSparseMatrixGPU& m, int n, std::mt19937& rng)
      : m_(m), n_(n), streams_(m.GroupTypeNum()),
        lhs_host_(DrawDense(rng, size_t(m.MatrixRow()) * size_t(n))),
        rhs_host_(DrawDense(rng, size_t(m.MatrixCol()) * size_t(n))),
        lhs_(lhs_host_.size()), rhs_(rhs_host_.size()) {
    lhs_.Upload(lhs_host_.data(), lhs_host_.size());
    rhs_.Upload(rhs_host_.data(), rhs_host_.size());
    // per workset: GroupNum[s] * GROUP_SIZE(s) outputs, the residue's total for s = 0
    int residue_total = 0;
    if (m.GroupNum()[0] > 0)
      ThrowOnError(ps_memcpy_dtoh(&residue_total, m.ResidueOffset() + m.GroupNum()[0], sizeof(int)));
    for (int s = 0; s < m.GroupTypeNum(); ++s) {
      const size_t len = s == 0 ? size_t(residue_total)
                                : size_t(m.GroupNum()[s]) * size_t(GROUP_SIZE(s));
      out_.emplace_back(len);
      out_ptr_.push_back(out_.back().data());
    }
  }
  void ClearOutputs() override {
    for (DeviceArray<float>& o : out_)
      if (o.size()) o.Zero(nullptr);
  }
  void Call() override {
    PowerSparse::SDDMM(m_, n_, lhs_.data(), rhs_.data(), out_ptr_.data(), streams_.count(),
                       streams_.data());
  }
  void Verify(const HostCsr&, const std::vector<HostWorkset>& ws) override {
    for (size_t s = 0; s < ws.size(); ++s) {
      const HostWorkset& w = ws[s];
      const std::vector<float> got = ToHost(out_[s].data(), w.col.size());
      for (size_t g = 0; g < w.dest.size(); ++g) {
        const float* x = lhs_host_.data() + size_t(w.dest[g]) * size_t(n_);
        for (int p = w.begin[g]; p < w.begin[g + 1]; ++p) {
          const float* y = rhs_host_.data() + size_t(w.col[size_t(p)]) * size_t(n_);
          double dot = 0;
          for (int j = 0; j < n_; ++j) dot += double(x[j]) * y[j];
          if (!WithinTolerance(got[size_t(p)], dot * w.val[size_t(p)]))
            throw std::runtime_error("SDDMM mismatch in workset " + std::to_string(s) +
                                     ", position " + std::to_string(p));
        }
      }
    }
  }

 private:
  const PowerSparseMatrixGPU& m_;
  int n_;
  StreamList streams_;
  std::vector<float> lhs_host_, rhs_host_;
  DeviceArray<float> lhs_, rhs_;
  std::vector<DeviceArray<float>> out_;
  std::vector<float*> out_ptr_;
};

// ------------------------------------------------------------- the run

struct DeviceInfo {
  std::string name, arch;
  int runtime = 0, driver = 0;
};

DeviceInfo OpenDevice(int device) {
  ThrowOnError(ps_set_device(device));
  ps_device_props p;
  ThrowOnError(ps_get_device_props(device, &p));
  DeviceInfo d;
  d.name = p.name;
  d.arch = std::string(p.arch).substr(0, std::string(p.arch).find(':'));
  ThrowOnError(ps_runtime_version(&d.runtime));
  ThrowOnError(ps_driver_version(&d.driver));
  return d;
}

std::string Quoted(const std::string& s) {
  std::string q = "\"";
  for (char c : s) q += c == '"' ? std::string("\"\"") : std::string(1, c);
  return q + "\"";
}

// Mean milliseconds per call over `calls` back-to-back calls, between two
// events on the null stream.
double TimeCalls(Workload& w, int calls) {
  ps_event_t ev[2] = {nullptr, nullptr};
  struct Release {
    ps_event_t* e;
    ~Release() {
      ps_event_destroy(e[0]);
      ps_event_destroy(e[1]);
    }
  } release{ev};
  ThrowOnError(ps_event_create(&ev[0]));
  ThrowOnError(ps_event_create(&ev[1]));
  ThrowOnError(ps_event_record(ev[0], nullptr));
  for (int i = 0; i < calls; ++i) w.Call();
  ThrowOnError(ps_device_synchronize());
  ThrowOnError(ps_event_record(ev[1], nullptr));
  ThrowOnError(ps_event_synchronize(ev[1]));
  float ms = 0;
  ThrowOnError(ps_event_elapsed_ms(&ms, ev[0], ev[1]));
  return double(ms) / calls;
}

int Bench(const Spec& spec, bool sddmm) {
  const char* const kOpName = sddmm ? "SDDMM" : "SpMM";
  const DeviceInfo dev = OpenDevice(spec.device);
  std::cerr << kOpName << ": " << spec.matrix << ", N=" << spec.n << ", GPU=" << dev.name << " ("
            << dev.arch << ")\n";
  const HostCsr csr = LoadMatrix(spec.matrix);
  PowerSparse::ValidateDenseShape(csr.rows, csr.cols, spec.n);

  ThrowOnError(ps_device_synchronize());
  const auto t0 = std::chrono::steady_clock::now();
  const PowerSparseMatrixGPU matrix(csr.rows, csr.cols, csr.nnz(), csr.row_ptr.data(),
                                    csr.col_ind.data(), csr.values.data());
  ThrowOnError(ps_device_synchronize());
  const double preprocess_ms =
      std::chrono::duration<double, std::milli>(std::chrono::steady_clock::now() - t0).count();

  std::mt19937 rng(kInputSeed);
  std::unique_ptr<Workload> work;
  if (sddmm) work = std::make_unique<SddmmWorkload>(matrix, spec.n, rng);
  else work = std::make_unique<SpmmWorkload>(matrix, spec.n, rng);

  auto clear = [&] {
    work->ClearOutputs();
    ThrowOnError(ps_device_synchronize());
  };
  clear();
  if (spec.check) {
    const std::vector<HostWorkset> ws = FetchWorksets(matrix);
    VerifyWorksets(csr, ws);
    work->Call();
    ThrowOnError(ps_device_synchronize());
    work->Verify(csr, ws);
    std::cerr << "Preprocessing and CPU reference checks passed (atol=rtol=1e-3).\n";
    clear();
  }
  for (int i = 0; i < kWarmupCalls; ++i) work->Call();
  ThrowOnError(ps_device_synchronize());
  clear();
  const double ms = TimeCalls(*work, spec.repeats);  // outputs accumulate, as in the reference
  if (!std::isfinite(ms) || ms <= 0) throw std::runtime_error("Invalid measured latency");
  const double gflops = 2.0 * csr.nnz() * spec.n / (ms * 1e6);

  std::ostringstream row;
  row << std::setprecision(10) << "PowerSparse," << kOpName << ',' << Quoted(spec.matrix) << ','
      << csr.rows << ',' << csr.cols << ',' << csr.nnz() << ',' << spec.n << ',' << spec.device
      << ',' << Quoted(dev.name) << ',' << dev.arch << ',' << dev.runtime << ',' << dev.driver
      << ',' << kWarmupCalls << ',' << spec.repeats << ',' << kInputSeed << ','
      << (spec.check ? "passed" : "skipped") << ',' << preprocess_ms << ',' << ms << ','
      << gflops << '\n';
  std::cout << row.str() << std::flush;
  return 0;
}

}  // namespace

int psx_bench_main(int op, int argc, char** argv) {
  const bool sddmm = op == PSX_BENCH_SDDMM;
  const char* const kOpName = sddmm ? "SDDMM" : "SpMM";
  try {
    if (op != PSX_BENCH_SPMM && op != PSX_BENCH_SDDMM) {
      std::cerr << "Error: unknown benchmark operator " << op << '\n';
      return 1;
    }
    if (argc == 2 && std::strcmp(argv[1], "--header") == 0) {
      std::cout << kCsvHeader << std::endl;
      return 0;
    }
    if (argc != 6) {
      PrintUsage(argc > 0 ? argv[0] : (sddmm ? "powersparse_sddmm" : "powersparse_spmm"));
      return 2;
    }
    const int n = WholeInt(argv[2], "N");
    if (n != 32 && n != 64 && n != 128) {
      std::cerr << kOpName << " benchmark: N=" << n
                << " was not selected in main; please use N=32, 64 or 128.\n";
      return 2;
    }
    return Bench(ParseSpec(argv), sddmm);
  } catch (const std::exception& e) {
    std::cerr << "Error: " << e.what() << '\n';
    return 1;
  }
}
