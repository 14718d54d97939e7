// model_ops.hpp -- inference kernels for the sequence model around the KLA layers,
// for gfx950: the blocks' RMSNorm and the SwiGLU MLP's activation
// (reference src/kla/layers/common.py:45-55, :120-123). Each replaces a chain of
// torch elementwise kernels with one launch, which is what one-token decode is
// bound by. The values are torch's: fp32 arithmetic in torch's order, one
// rounding to the tensor dtype where torch rounds.
#pragma once

#include "causal_conv.hpp"

namespace kla {

constexpr int kNormThreads = 256;   // four rows per workgroup, one wave per row

// y = ((x * r) * w) in x's dtype, r = rsqrt(mean(x^2) + eps), per row of `dim`.
template <class IO>
__global__ void __launch_bounds__(kNormThreads) rms_norm_fwd_kernel(const IO *__restrict__ x,
                                                                    const float *__restrict__ w, float eps,
                                                                    IO *__restrict__ y, int64_t rows, int64_t dim) {
  const int lane = static_cast<int>(threadIdx.x) % kWave;
  const int64_t row = static_cast<int64_t>(blockIdx.x) * (kNormThreads / kWave) + threadIdx.x / kWave;
  if (row >= rows) return;   // whole waves leave together
  const IO *xr = x + row * dim;
  float ss = 0.0f;
  for (int64_t i = lane; i < dim; i += kWave) {
    const float v = io_load(xr + i);
    ss = fmaf(v, v, ss);
  }
#pragma unroll
  for (int off = kWave / 2; off > 0; off /= 2) ss += __shfl_xor(ss, off);
  const float r = rsqrtf(ss / static_cast<float>(dim) + eps);
  IO *yr = y + row * dim;
  for (int64_t i = lane; i < dim; i += kWave) io_store(yr + i, (io_load(xr + i) * r) * w[i]);
}

// out = act(gate) * up with gate = h[:, :hidden], up = h[:, hidden:2 hidden] (rows
// ld_h apart): silu(gate) rounded to the dtype, then the product rounded.
template <class IO>
__global__ void __launch_bounds__(256) swiglu_fwd_kernel(const IO *__restrict__ h, int64_t ld_h,
                                                         IO *__restrict__ out, int64_t rows, int64_t hidden) {
  const int64_t i = static_cast<int64_t>(blockIdx.x) * 256 + threadIdx.x;
  if (i >= rows * hidden) return;
  const int64_t r = i / hidden, c = i % hidden;
  const float g = io_round<IO>(activation(kActSilu, io_load(h + r * ld_h + c)));
  io_store(out + i, g * io_load(h + r * ld_h + hidden + c));
}

}  // namespace kla
