// C-callable names for the reference's own rope/softmax/rmsnorm/silu (src/tensor/ops.hpp),
// compiled from the reference sources into oracle/_ref/libref_ops.so. Test
// infrastructure: pins the oracle's restatement against the real code.
#include <cstddef>
#include <cstdint>

#include "tensor/ops.hpp"

extern "C" void ref_rope(float* x, const std::int32_t* positions, float theta, std::size_t n_heads,
                         std::size_t seq, std::size_t head_dim) {
  dbinfer::tensor::rope(x, positions, theta, n_heads, seq, head_dim);
}

extern "C" void ref_softmax(const float* in, float* out, std::size_t n) {
  dbinfer::tensor::softmax(in, out, n);
}

extern "C" void ref_rmsnorm(const float* x, const float* weight, float eps, float* out,
                            std::size_t rows, std::size_t dim) {
  dbinfer::tensor::rmsnorm(x, weight, eps, out, rows, dim);
}

extern "C" void ref_silu(const float* in, float* out, std::size_t n) {
  dbinfer::tensor::silu(in, out, n);
}
