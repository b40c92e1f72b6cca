"""The drop-in C++ boundary, checked by the compiler: a translation unit
written the way the reference's callers use its API (utils/matrix_utils.h:20-40,
PowerSparse_SpMM/PowerSparse_SpMM.h:14-17, PowerSparse_SDDMM/PowerSparse_SDDMM.h:14-18,
benchmarks/benchmark.cu:21-41, 126-167) compiles against this build's public
headers and links against its libraries, and static_asserts pin the member
and function types to the reference's (cudaStream_t becomes ps_stream_t).
Nothing is run: the program needs a GPU."""
import os
import shutil
import subprocess

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
LIB = os.path.join(ROOT, "powersparse_amd", "lib")

SOURCE = r"""
#include <stdexcept>
#include <type_traits>
#include <vector>

#include "PowerSparse_SDDMM.h"
#include "PowerSparse_SpMM.h"
#include "matrix_utils.h"

using Matrix = PowerSparse::PowerSparseMatrixGPU;

// the reference's accessors, with their exact types (matrix_utils.h:30-40)
static_assert(std::is_same<decltype(&Matrix::MatrixRow), int (Matrix::*)() const>::value, "");
static_assert(std::is_same<decltype(&Matrix::MatrixCol), int (Matrix::*)() const>::value, "");
static_assert(std::is_same<decltype(&Matrix::MatrixNNZ), int (Matrix::*)() const>::value, "");
static_assert(std::is_same<decltype(&Matrix::GroupTypeNum), int (Matrix::*)() const>::value, "");
static_assert(std::is_same<decltype(&Matrix::GroupFineSize), int (Matrix::*)() const>::value, "");
static_assert(std::is_same<decltype(&Matrix::GroupNum), const int* (Matrix::*)() const>::value, "");
static_assert(std::is_same<decltype(&Matrix::WorksetColInd),
                           const int* const* (Matrix::*)() const>::value, "");
static_assert(std::is_same<decltype(&Matrix::WorksetSpData),
                           const float* const* (Matrix::*)() const>::value, "");
static_assert(std::is_same<decltype(&Matrix::GroupDestination),
                           const int* const* (Matrix::*)() const>::value, "");
static_assert(std::is_same<decltype(&Matrix::ResidueOffset), const int* (Matrix::*)() const>::value, "");
static_assert(std::is_same<decltype(&Matrix::ResidueAtomic), const bool* (Matrix::*)() const>::value, "");
// not copyable, not movable (matrix_utils.h:24-28)
static_assert(!std::is_copy_constructible<Matrix>::value && !std::is_move_constructible<Matrix>::value, "");
static_assert(!std::is_copy_assignable<Matrix>::value && !std::is_move_assignable<Matrix>::value, "");
// the constructor of host CSR arrays (matrix_utils.h:22-23)
static_assert(std::is_constructible<Matrix, int, int, int, const int*, const int*, const float*>::value, "");
// the solution entry points (PowerSparse_SpMM.h:14-17, PowerSparse_SDDMM.h:14-18)
static_assert(std::is_same<decltype(&PowerSparse::SpMM),
                           void (*)(const Matrix&, int, const float*, float*, int,
                                    const ps_stream_t*)>::value, "");
static_assert(std::is_same<decltype(&PowerSparse::SDDMM),
                           void (*)(const Matrix&, int, const float*, const float*, float**, int,
                                    const ps_stream_t*)>::value, "");

// a caller written like the reference's benchmark (benchmark.cu:126-167)
int Run(int rows, int cols, const std::vector<int>& row_ptr, const std::vector<int>& col_ind,
        const std::vector<float>& values, int n) {
  PowerSparse::ValidateDenseShape(rows, cols, n);
  Matrix matrix(rows, cols, int(col_ind.size()), row_ptr.data(), col_ind.data(), values.data());
  const int S = matrix.GroupTypeNum();
  std::vector<ps_stream_t> streams(size_t(S), nullptr);
  for (ps_stream_t& s : streams)
    if (ps_stream_create(&s) != PS_OK) throw std::runtime_error(ps_last_error());
  void* b = nullptr;
  void* c = nullptr;
  ps_malloc(&b, size_t(cols) * size_t(n) * sizeof(float));
  ps_malloc(&c, size_t(rows) * size_t(n) * sizeof(float));
  PowerSparse::SpMM(matrix, n, static_cast<const float*>(b), static_cast<float*>(c), S,
                    streams.data());
  std::vector<float*> outputs;
  for (int s = 0; s < S; ++s) {
    size_t len = size_t(matrix.GroupNum()[s]) * size_t(GROUP_SIZE(s));
    if (s == 0) {
      int total = 0;
      ps_memcpy_dtoh(&total, matrix.ResidueOffset() + matrix.GroupNum()[0], sizeof(int));
      len = size_t(total);
    }
    void* o = nullptr;
    ps_malloc(&o, len * sizeof(float));
    outputs.push_back(static_cast<float*>(o));
  }
  PowerSparse::SDDMM(matrix, n, static_cast<const float*>(c), static_cast<const float*>(b),
                     outputs.data(), S, streams.data());
  const int* first_cols = matrix.WorksetColInd()[S - 1];
  const float* first_vals = matrix.WorksetSpData()[S - 1];
  const int* dest = matrix.GroupDestination()[0];
  const bool* atomic = matrix.ResidueAtomic();
  for (float* o : outputs) ps_free(o);
  ps_free(b);
  ps_free(c);
  for (ps_stream_t s : streams) ps_stream_destroy(s);
  return (first_cols && first_vals && dest && atomic) ? matrix.MatrixNNZ() : -1;
}

int main() {
  try {
    return Run(2, 2, {0, 1, 2}, {0, 1}, {1.f, 2.f}, 32) > 0 ? 0 : 1;
  } catch (const std::invalid_argument&) {
    return 2;
  } catch (const std::exception&) {
    return 1;
  }
}
"""


def test_reference_style_caller_compiles_and_links(tmp_path):
    if not os.path.exists(os.path.join(LIB, "libpowersparse.so")):
        pytest.skip("host library not built")
    cxx = shutil.which("g++")
    if cxx is None:
        pytest.skip("no g++")
    src = tmp_path / "caller.cpp"
    src.write_text(SOURCE)
    exe = tmp_path / "caller"
    cmd = [cxx, "-std=c++17", "-Wall", "-Werror", "-I" + os.path.join(ROOT, "include"),
           "-I" + os.path.join(ROOT, "powersparse_amd", "host"), str(src), "-o", str(exe),
           "-L" + LIB, "-lpowersparse", "-lpowersparse_hip", "-Wl,-rpath," + LIB]
    r = subprocess.run(cmd, capture_output=True, text=True, timeout=300)
    assert r.returncode == 0, r.stderr
    assert exe.exists()
