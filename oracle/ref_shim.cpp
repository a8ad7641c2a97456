// extern "C" entry points over the reference's own C++ CPU kernels
// (cpp/include/cacheir/cacheir_backend.hpp:18-22, cpp/src/cacheir_backend.cpp:91-165),
// compiled from /root/reference by oracle/Makefile into oracle/_ref/.  Test
// infrastructure only: it lets the oracle's NumPy rms_norm / silu_mul / matmul be
// checked against the reference's compiled kernels.  Shapes follow the reference's
// pybind wrapper (cpp/src/pybind_module.cpp:28-68): x is rank 3, weights [out, in].
#include <cstddef>
#include <span>

#include "cacheir/cacheir_backend.hpp"

namespace {
cacheir::ConstTensorView cv(const float* p, const std::size_t* shape, std::size_t rank) {
  return cacheir::ConstTensorView{p, std::span<const std::size_t>(shape, rank)};
}
cacheir::TensorView tv(float* p, const std::size_t* shape, std::size_t rank) {
  return cacheir::TensorView{p, std::span<const std::size_t>(shape, rank)};
}
}  // namespace

extern "C" {

int cir_ref_rms_norm(const float* x, const float* w, float* out, std::size_t b, std::size_t s, std::size_t h, float eps) {
  const std::size_t xs[3] = {b, s, h};
  const std::size_t ws[1] = {h};
  try {
    cacheir::rms_norm(cv(x, xs, 3), cv(w, ws, 1), tv(out, xs, 3), eps);
  } catch (...) {
    return 1;
  }
  return 0;
}

int cir_ref_silu_mul(const float* gate, const float* up, float* out, std::size_t n) {
  const std::size_t s[1] = {n};
  try {
    cacheir::silu_mul(cv(gate, s, 1), cv(up, s, 1), tv(out, s, 1));
  } catch (...) {
    return 1;
  }
  return 0;
}

int cir_ref_matmul_out_in(const float* x, const float* w, float* out, std::size_t b, std::size_t s, std::size_t in,
                          std::size_t outf) {
  const std::size_t xs[3] = {b, s, in};
  const std::size_t ws[2] = {outf, in};
  const std::size_t os[3] = {b, s, outf};
  try {
    cacheir::matmul_out_in(cv(x, xs, 3), cv(w, ws, 2), tv(out, os, 3));
  } catch (...) {
    return 1;
  }
  return 0;
}

const char* cir_ref_simd_backend() { return cacheir::simd_backend(); }
}
