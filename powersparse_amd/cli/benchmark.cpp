// powersparse_spmm / powersparse_sddmm: the reference's CSV benchmark contract
// (ParCIS/PowerSparse benchmarks/benchmark.cu:98-213, README.md:27-42):
//   powersparse_{spmm,sddmm} MATRIX N DEVICE CHECK REPEATS
//   powersparse_{spmm,sddmm} --header
// MATRIX is a MatrixMarket file, a binary CSR (*.pscsr) or "synth:NAME[:SEED[:SCALE]]"
// for the seeded synthetic configurations. N is 32, 64 or 128 (the reference
// allows 32 and 128; 64 is added for the community-graph configuration).
// Timing: 30 warm-up calls, then REPEATS calls between two events, outputs not
// cleared between timed calls; preprocessing is timed separately on the host.
// CSV columns are the reference's; compute_capability carries the gfx arch name
// and cuda_runtime / cuda_driver the HIP runtime / driver versions.
#include <algorithm>
#include <chrono>
#include <cmath>
#include <cstring>
#include <iomanip>
#include <iostream>
#include <random>
#include <stdexcept>
#include <string>
#include <tuple>
#include <vector>

#include "PowerSparse_SDDMM.h"
#include "PowerSparse_SpMM.h"
#include "matrix_market.h"
#include "powersparse.h"
#include "synth.h"

#ifndef POWERSPARSE_BENCH_SDDMM
#define POWERSPARSE_BENCH_SDDMM 0
#endif

namespace {

constexpr bool kSddmm = POWERSPARSE_BENCH_SDDMM != 0;
constexpr int kWarmup = 30;
constexpr unsigned kSeed = 1;
constexpr const char* kOperator = kSddmm ? "SDDMM" : "SpMM";

using PowerSparse::HostCsr;
using PowerSparse::PowerSparseMatrixGPU;
using PowerSparse::ThrowOnError;

template <typename T>
class DeviceBuffer {
 public:
  explicit DeviceBuffer(size_t count = 0) : count_(count) {
    if (count > size_t(-1) / sizeof(T)) throw std::overflow_error("Device allocation size overflow");
    void* p = nullptr;
    if (count) ThrowOnError(ps_malloc(&p, count * sizeof(T)));
    data_ = static_cast<T*>(p);
  }
  ~DeviceBuffer() { ps_free(data_); }
  DeviceBuffer(const DeviceBuffer&) = delete;
  DeviceBuffer& operator=(const DeviceBuffer&) = delete;
  DeviceBuffer(DeviceBuffer&& o) noexcept : data_(o.data_), count_(o.count_) {
    o.data_ = nullptr;
    o.count_ = 0;
  }
  T* data() const { return data_; }
  size_t size() const { return count_; }
  void zero() {
    if (count_) ThrowOnError(ps_memset_async(data_, 0, count_ * sizeof(T), nullptr));
  }
  void upload(const std::vector<T>& v) {
    if (v.size() != count_) throw std::invalid_argument("Upload size mismatch");
    if (count_) ThrowOnError(ps_memcpy_htod(data_, v.data(), count_ * sizeof(T)));
  }

 private:
  T* data_ = nullptr;
  size_t count_ = 0;
};

template <typename T>
std::vector<T> Download(const T* p, size_t count) {
  std::vector<T> h(count);
  if (count) ThrowOnError(ps_memcpy_dtoh(h.data(), p, count * sizeof(T)));
  return h;
}

class Streams {
 public:
  explicit Streams(int count) : s_(size_t(count), nullptr) {
    if (count > 1)
      for (auto& st : s_) ThrowOnError(ps_stream_create(&st));
  }
  ~Streams() {
    for (auto st : s_) ps_stream_destroy(st);
  }
  int size() const { return int(s_.size()); }
  const ps_stream_t* data() const { return s_.data(); }

 private:
  std::vector<ps_stream_t> s_;
};

class GpuTimer {
 public:
  GpuTimer() {
    ThrowOnError(ps_event_create(&a_));
    ThrowOnError(ps_event_create(&b_));
  }
  ~GpuTimer() {
    ps_event_destroy(a_);
    ps_event_destroy(b_);
  }
  void start() { ThrowOnError(ps_event_record(a_, nullptr)); }
  float stop() {
    ThrowOnError(ps_event_record(b_, nullptr));
    ThrowOnError(ps_event_synchronize(b_));
    float ms = 0;
    ThrowOnError(ps_event_elapsed_ms(&ms, a_, b_));
    return ms;
  }

 private:
  ps_event_t a_ = nullptr, b_ = nullptr;
};

int ParseInt(const char* text, const char* name) {
  const std::string v(text);
  size_t used = 0;
  int n;
  try {
    n = std::stoi(v, &used);
  } catch (...) {
    throw std::invalid_argument(std::string("Invalid ") + name + ": " + v);
  }
  if (used != v.size()) throw std::invalid_argument(std::string("Invalid ") + name);
  return n;
}

std::vector<float> DenseInput(size_t count, std::mt19937& rng) {
  std::vector<float> v(count);
  for (auto& x : v) x = float(rng() % 3) / 10.0f;
  return v;
}

bool Close(float actual, double expected) {  // benchmark_utils.h:106-109
  return std::isfinite(actual) && std::isfinite(expected) &&
         std::abs(double(actual) - expected) <= 1e-3 + 1e-3 * std::abs(expected);
}

std::string Csv(const std::string& s) {
  std::string r = "\"";
  for (char c : s) {
    if (c == '"') r += '"';
    r += c;
  }
  return r + '"';
}

HostCsr LoadMatrix(const std::string& path) {
  if (path.rfind("synth:", 0) == 0) {
    std::string rest = path.substr(6), name = rest;
    uint64_t seed = 1;
    int scale = 1;
    const size_t a = rest.find(':');
    if (a != std::string::npos) {
      name = rest.substr(0, a);
      const std::string tail = rest.substr(a + 1);
      const size_t b = tail.find(':');
      seed = std::stoull(tail.substr(0, b));
      if (b != std::string::npos) scale = std::stoi(tail.substr(b + 1));
    }
    return PowerSparse::SynthConfig(name, seed, scale);
  }
  if (path.size() > 6 && path.compare(path.size() - 6, 6, ".pscsr") == 0)
    return PowerSparse::ReadBinaryCsr(path);
  return PowerSparse::ReadMatrixMarket(path);
}

struct HostWorkset {
  std::vector<int> rows, offsets, cols;
  std::vector<float> values;
};

HostWorkset ReadWorkset(const PowerSparseMatrixGPU& m, int s, const std::vector<int>& residue) {
  HostWorkset w;  // benchmark.cu:29-41
  const int groups = m.GroupNum()[s];
  w.rows = Download(m.GroupDestination()[s], size_t(groups));
  if (s == 0) {
    w.offsets = residue;
  } else {
    w.offsets.resize(size_t(groups) + 1);
    for (int g = 0; g <= groups; ++g) w.offsets[size_t(g)] = g * GROUP_SIZE(s);
  }
  w.cols = Download(m.WorksetColInd()[s], size_t(w.offsets.back()));
  w.values = Download(m.WorksetSpData()[s], size_t(w.offsets.back()));
  return w;
}

void CheckPreprocessing(const HostCsr& csr, const PowerSparseMatrixGPU& m,
                        const std::vector<int>& residue) {
  using Edge = std::tuple<int, int, float>;  // benchmark.cu:45-62
  std::vector<Edge> expected, actual;
  expected.reserve(size_t(csr.nnz()));
  actual.reserve(size_t(csr.nnz()));
  for (int r = 0; r < csr.rows; ++r)
    for (int p = csr.row_ptr[size_t(r)]; p < csr.row_ptr[size_t(r) + 1]; ++p)
      expected.emplace_back(r, csr.col_ind[size_t(p)], csr.values[size_t(p)]);
  for (int s = 0; s < m.GroupTypeNum(); ++s) {
    const auto w = ReadWorkset(m, s, residue);
    for (size_t g = 0; g < w.rows.size(); ++g)
      for (int p = w.offsets[g]; p < w.offsets[g + 1]; ++p)
        actual.emplace_back(w.rows[g], w.cols[size_t(p)], w.values[size_t(p)]);
  }
  std::sort(expected.begin(), expected.end());
  std::sort(actual.begin(), actual.end());
  if (actual != expected) throw std::runtime_error("Preprocessing changed the sparse matrix");
}

void CheckSpmm(const HostCsr& csr, int n, const std::vector<float>& b, const float* output) {
  const auto actual = Download(output, size_t(csr.rows) * n);  // benchmark.cu:64-77
  std::vector<double> expected(static_cast<size_t>(n));
  for (int r = 0; r < csr.rows; ++r) {
    std::fill(expected.begin(), expected.end(), 0.0);
    for (int p = csr.row_ptr[size_t(r)]; p < csr.row_ptr[size_t(r) + 1]; ++p)
      for (int j = 0; j < n; ++j)
        expected[size_t(j)] +=
            double(csr.values[size_t(p)]) * b[size_t(csr.col_ind[size_t(p)]) * n + j];
    for (int j = 0; j < n; ++j)
      if (!Close(actual[size_t(r) * n + j], expected[size_t(j)]))
        throw std::runtime_error("SpMM mismatch at row " + std::to_string(r) + ", feature " +
                                 std::to_string(j));
  }
}

void CheckSddmm(const PowerSparseMatrixGPU& m, const std::vector<int>& residue, int n,
                const std::vector<float>& lhs, const std::vector<float>& rhs,
                const std::vector<float*>& output) {
  for (int s = 0; s < m.GroupTypeNum(); ++s) {  // benchmark.cu:79-96
    const auto w = ReadWorkset(m, s, residue);
    const auto actual = Download(output[size_t(s)], w.values.size());
    for (size_t g = 0; g < w.rows.size(); ++g)
      for (int p = w.offsets[g]; p < w.offsets[g + 1]; ++p) {
        double expected = 0;
        for (int j = 0; j < n; ++j)
          expected += double(lhs[size_t(w.rows[g]) * n + j]) * rhs[size_t(w.cols[size_t(p)]) * n + j];
        expected *= w.values[size_t(p)];
        if (!Close(actual[size_t(p)], expected))
          throw std::runtime_error("SDDMM mismatch in workset " + std::to_string(s) +
                                   ", position " + std::to_string(p));
      }
  }
}

void CsvHeader() {
  std::cout << "algorithm,operator,matrix,rows,cols,nnz,N,device,gpu,compute_capability,"
               "cuda_runtime,cuda_driver,warmup,repeats,seed,check,preprocess_ms,ms,gflops\n";
}

int Run(int argc, char** argv) {
  if (argc == 2 && std::string(argv[1]) == "--header") {
    CsvHeader();
    return 0;
  }
  if (argc != 6) {
    std::cerr << "Usage: " << argv[0] << " MATRIX N DEVICE CHECK REPEATS\n"
              << "MATRIX: a .mtx file, a .pscsr binary CSR, or synth:NAME[:SEED[:SCALE]]\n"
              << "CHECK: 0=skip, 1=verify preprocessing and compare with a CPU reference\n"
              << "Benchmark widths are N=32, 64 or 128.\n";
    return 2;
  }
  const std::string path = argv[1];
  const int n = ParseInt(argv[2], "N"), device = ParseInt(argv[3], "DEVICE");
  const int check = ParseInt(argv[4], "CHECK"), repeats = ParseInt(argv[5], "REPEATS");
  if (device < 0 || (check != 0 && check != 1) || repeats <= 0)
    throw std::invalid_argument("DEVICE must be nonnegative, CHECK 0 or 1, and REPEATS positive");
  ThrowOnError(ps_set_device(device));
  ps_device_props props;
  ThrowOnError(ps_get_device_props(device, &props));
  int runtime = 0, driver = 0;
  ThrowOnError(ps_runtime_version(&runtime));
  ThrowOnError(ps_driver_version(&driver));
  std::string arch = props.arch;
  arch = arch.substr(0, arch.find(':'));
  std::cerr << kOperator << ": " << path << ", N=" << n << ", GPU=" << props.name << " ("
            << arch << ")\n";
  const HostCsr csr = LoadMatrix(path);
  PowerSparse::ValidateDenseShape(csr.rows, csr.cols, n);

  ThrowOnError(ps_device_synchronize());
  const auto begin = std::chrono::steady_clock::now();
  const PowerSparseMatrixGPU matrix(csr.rows, csr.cols, csr.nnz(), csr.row_ptr.data(),
                                    csr.col_ind.data(), csr.values.data());
  ThrowOnError(ps_device_synchronize());
  const double preprocess_ms =
      std::chrono::duration<double, std::milli>(std::chrono::steady_clock::now() - begin).count();
  const auto residue = Download(matrix.ResidueOffset(), size_t(matrix.GroupNum()[0]) + 1);

  std::mt19937 rng(kSeed);
  std::vector<float> lhs;
  if (kSddmm) lhs = DenseInput(size_t(csr.rows) * n, rng);
  auto rhs = DenseInput(size_t(csr.cols) * n, rng);
  DeviceBuffer<float> d_lhs(lhs.size()), d_rhs(rhs.size());
  d_lhs.upload(lhs);
  d_rhs.upload(rhs);
  DeviceBuffer<float> dense_output(kSddmm ? 0 : size_t(csr.rows) * n);
  std::vector<DeviceBuffer<float>> sparse_output;
  std::vector<float*> output_ptrs;
  if (kSddmm) {
    sparse_output.reserve(size_t(matrix.GroupTypeNum()));
    for (int s = 0; s < matrix.GroupTypeNum(); ++s) {
      const size_t count = s == 0 ? size_t(residue.back())
                                  : size_t(matrix.GroupNum()[s]) * GROUP_SIZE(s);
      sparse_output.emplace_back(count);
      output_ptrs.push_back(sparse_output.back().data());
    }
  }
  Streams streams(matrix.GroupTypeNum());
  auto reset = [&] {
    dense_output.zero();
    for (auto& o : sparse_output) o.zero();
    ThrowOnError(ps_device_synchronize());
  };
  auto invoke = [&] {
    if (kSddmm)
      PowerSparse::SDDMM(matrix, n, d_lhs.data(), d_rhs.data(), output_ptrs.data(),
                         streams.size(), streams.data());
    else
      PowerSparse::SpMM(matrix, n, d_rhs.data(), dense_output.data(), streams.size(),
                        streams.data());
  };
  reset();
  if (check) {
    CheckPreprocessing(csr, matrix, residue);
    invoke();
    ThrowOnError(ps_device_synchronize());
    if (kSddmm) CheckSddmm(matrix, residue, n, lhs, rhs, output_ptrs);
    else CheckSpmm(csr, n, rhs, dense_output.data());
    std::cerr << "Preprocessing and CPU reference checks passed (atol=rtol=1e-3).\n";
    reset();
  }
  for (int i = 0; i < kWarmup; ++i) invoke();
  ThrowOnError(ps_device_synchronize());
  reset();
  GpuTimer timer;
  timer.start();
  // As in the reference harness, outputs are not cleared between timed calls.
  for (int i = 0; i < repeats; ++i) invoke();
  ThrowOnError(ps_device_synchronize());
  const double ms = double(timer.stop()) / repeats;
  if (!std::isfinite(ms) || ms <= 0) throw std::runtime_error("Invalid measured latency");
  const double gflops = 2.0 * csr.nnz() * n / (ms * 1e6);
  std::cout << std::setprecision(10) << "PowerSparse," << kOperator << ',' << Csv(path) << ','
            << csr.rows << ',' << csr.cols << ',' << csr.nnz() << ',' << n << ',' << device << ','
            << Csv(props.name) << ',' << arch << ',' << runtime << ',' << driver << ','
            << kWarmup << ',' << repeats << ',' << kSeed << ',' << (check ? "passed" : "skipped")
            << ',' << preprocess_ms << ',' << ms << ',' << gflops << '\n';
  return 0;
}

}  // namespace

int main(int argc, char** argv) {
  try {
    if (argc == 6) {
      const int n = ParseInt(argv[2], "N");
      if (n != 32 && n != 64 && n != 128) {
        std::cerr << kOperator << " benchmark: N=" << n
                  << " was not selected in main; please use N=32, 64 or 128.\n";
        return 2;
      }
    }
    return Run(argc, argv);
  } catch (const std::exception& e) {
    std::cerr << "Error: " << e.what() << '\n';
    return 1;
  }
}
