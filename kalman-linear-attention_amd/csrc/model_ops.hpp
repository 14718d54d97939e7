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

// The k, q sensors of KLALayer._project_sensors_raw (reference kla_layer.py:194-231):
//   y = clamp(l2_norm(x), -clip, clip).float(),  l2_norm(x) = x / max(||x||_2, 1e-12)
// over the S states of each row, with torch's rounding to the input dtype after
// every operation (bf16 under autocast: the norm, the clamp_min, the quotient and
// the clip each round). The backward is torch's autograd chain through the same
// operations, rounding where autograd rounds: the gradient cast back to the
// input dtype, the clamp mask (bounds cast to the input dtype, as torch compares),
// the quotient's -g ((x / n) / n) summed over the row, the clamp_min mask, the
// norm's x (g_n / n), and the two terms' sum.
// One thread per (row, s), SP lanes per row; k rows first, then q rows.
struct QkParams {
  const void *x[2];        // k, q rows, ld[i] elements apart
  int64_t ld[2];
  float *y[2];             // forward: [rows, S] dense fp32
  const float *dy[2];      // backward: gradients of y, [rows, S] dense
  void *dx[2];             // backward: [rows, S] dense, the input dtype
  int64_t rows, S;
  int norm, has_clip;
  float clip;
};

template <class IO, int SP, bool BWD>
__global__ void __launch_bounds__(256) qk_sensors_kernel(QkParams p) {
  const int64_t g = (static_cast<int64_t>(blockIdx.x) * 256 + threadIdx.x) / SP;   // row over both tensors
  const int s = static_cast<int>(threadIdx.x) % SP;
  if (g >= 2 * p.rows) return;   // whole SP-lane groups leave together
  const int which = g >= p.rows ? 1 : 0;
  const int64_t r = g - which * p.rows;
  const bool ok = s < p.S;
  const IO *xr = static_cast<const IO *>(p.x[which]) + r * p.ld[which];
  const float x = ok ? io_load(xr + s) : 0.0f;
  float n0 = 0.0f, n = 1.0f, yn = x;
  if (p.norm) {
    n0 = io_round<IO>(sqrtf(group_sum<SP>(x * x)));
    n = io_round<IO>(fmaxf(n0, 1e-12f));
    yn = io_round<IO>(x / n);
  }
  // torch's clamp backward compares with the bounds cast to the tensor's dtype.
  const bool in_clip = !p.has_clip || (yn >= io_round<IO>(-p.clip) && yn <= io_round<IO>(p.clip));
  if constexpr (!BWD) {
    const float y = p.has_clip ? io_round<IO>(fminf(fmaxf(yn, -p.clip), p.clip)) : yn;
    if (ok) p.y[which][r * p.S + s] = y;
  } else {
    float gy = ok ? io_round<IO>(p.dy[which][r * p.S + s]) : 0.0f;
    if (!in_clip) gy = 0.0f;
    float gx = gy;
    if (p.norm) {
      const float gx1 = io_round<IO>(gy / n);
      const float t = io_round<IO>(io_round<IO>(x / n) / n);
      float gn = io_round<IO>(group_sum<SP>(io_round<IO>(-gy * t)));
      if (!(n0 >= 1e-12f)) gn = 0.0f;
      const float gx2 = n0 == 0.0f ? 0.0f : io_round<IO>(x * io_round<IO>(gn / n0));
      gx = io_round<IO>(gx1 + gx2);
    }
    if (ok) io_store(static_cast<IO *>(p.dx[which]) + r * p.S + s, gx);
  }
}

// out[r, :] = [piece_0[r, :], ..., piece_{n-1}[r, :]] for dense out [rows, W]:
// the backward of splitting the last dimension (torch.split / chunk of a
// projection: autograd concatenates the pieces' gradients). A piece is rows of
// widths[i] elements ld[i] apart, or NULL for zeros. VEC elements per thread
// (one 16-byte access) when every boundary, stride and base allows it.
constexpr int kCatMaxPieces = 4;

template <class IO>
struct CatParams {
  const IO *src[kCatMaxPieces];
  int64_t ld[kCatMaxPieces];
  int64_t start[kCatMaxPieces + 1];   // column where piece i starts; start[n] = W
  int n;
  IO *out;
  int64_t rows, W;
};

template <class IO, int VEC>
__global__ void __launch_bounds__(256) cat_cols_kernel(CatParams<IO> p) {
  const int64_t r = blockIdx.y;
  const int64_t c0 = (static_cast<int64_t>(blockIdx.x) * 256 + threadIdx.x) * VEC;
  if (c0 >= p.W) return;
  int i = 0;
  while (i + 1 < p.n && c0 >= p.start[i + 1]) ++i;
  IO *dst = p.out + r * p.W + c0;
  const IO *src = p.src[i] ? p.src[i] + r * p.ld[i] + (c0 - p.start[i]) : nullptr;
  if constexpr (VEC > 1) {
    typedef uint32_t u32x4v __attribute__((ext_vector_type(4)));
    const u32x4v v = src ? *reinterpret_cast<const u32x4v *>(src) : u32x4v{0u, 0u, 0u, 0u};
    __builtin_nontemporal_store(v, reinterpret_cast<u32x4v *>(dst));
  } else {
    *dst = src ? *src : IO{};
  }
}

// out[i] = sum_{j < P} parts[j * N + i], added in j order in fp32 and rounded
// once to IO (round to nearest even for bf16): the last step of a weight
// gradient split over the token dimension into P fp32 partial products.
// Four elements per thread (16-byte partial loads) when N % 4 == 0 and the
// pointers are 16-byte aligned, else one; grid-stride over N.
template <class IO, int VEC>
__global__ void __launch_bounds__(256) sum_parts_kernel(const float *__restrict__ parts, int64_t P, int64_t N,
                                                        IO *__restrict__ out) {
  const int64_t stride = static_cast<int64_t>(gridDim.x) * 256 * VEC;
  for (int64_t i = (static_cast<int64_t>(blockIdx.x) * 256 + threadIdx.x) * VEC; i < N; i += stride) {
    if constexpr (VEC == 4) {
      typedef float f32x4v __attribute__((ext_vector_type(4)));
      f32x4v acc = __builtin_nontemporal_load(reinterpret_cast<const f32x4v *>(parts + i));
      for (int64_t j = 1; j < P; ++j)
        acc += __builtin_nontemporal_load(reinterpret_cast<const f32x4v *>(parts + j * N + i));
      io_store(out + i, acc.x);
      io_store(out + i + 1, acc.y);
      io_store(out + i + 2, acc.z);
      io_store(out + i + 3, acc.w);
    } else {
      float acc = parts[i];
      for (int64_t j = 1; j < P; ++j) acc += parts[j * N + i];
      io_store(out + i, acc);
    }
  }
}

// out[r, :] = table[ids[r], :] (the embedding lookup of one decode step,
// reference src/kla/models/sequence_model.py:157, nn.Embedding). An id outside
// [0, vocab) reads nothing and writes a row of NaN. One workgroup per row.
template <class IO>
__global__ void __launch_bounds__(256) gather_rows_kernel(const IO *__restrict__ table, int64_t ld_table,
                                                          int64_t vocab, const int64_t *__restrict__ ids,
                                                          IO *__restrict__ out, int64_t ld_out, int64_t dim) {
  const int64_t r = blockIdx.x;
  const int64_t id = ids[r];
  const bool ok = id >= 0 && id < vocab;
  const IO *src = table + (ok ? id : 0) * ld_table;
  IO *dst = out + r * ld_out;
  for (int64_t i = threadIdx.x; i < dim; i += 256)
    io_store(dst + i, ok ? io_load(src + i) : __builtin_nanf(""));
}

// (value, index) of the larger of two candidates in torch.argmax's order: NaN
// above every number, then the larger value, ties to the smaller index.
__device__ __forceinline__ bool argmax_before(float a, int64_t ia, float b, int64_t ib) {
  const bool na = a != a, nb = b != b;
  if (na || nb) return na && (!nb || ia < ib);
  return a > b || (a == b && ia < ib);
}

constexpr int kArgmaxThreads = 1024;
constexpr int kArgmaxPartThreads = 256;

// Stage 1 of a split argmax: workgroup (part, row) takes columns
// [part * chunk, (part + 1) * chunk) of its row and writes its (value, index)
// in torch.argmax's order; stage 2 (argmax_rows_kernel over the parts, VAL_IN)
// combines a row's parts in part order. Many rows' worth of workgroups keep the
// whole GPU streaming, where one workgroup per row leaves most CUs idle.
__global__ void __launch_bounds__(kArgmaxPartThreads) argmax_parts_kernel(const float *__restrict__ x, int64_t ldx,
                                                                           int64_t n, int64_t chunk,
                                                                           float *__restrict__ part_v,
                                                                           int64_t *__restrict__ part_i) {
  __shared__ float s_v[kArgmaxPartThreads / kWave];
  __shared__ int64_t s_i[kArgmaxPartThreads / kWave];
  const int tid = static_cast<int>(threadIdx.x);
  const int64_t part = blockIdx.x, row = blockIdx.y;
  const float *xr = x + row * ldx;
  const int64_t c0 = part * chunk, c1 = c0 + chunk < n ? c0 + chunk : n;
  float best = -__builtin_inff();
  int64_t bi = n;
  constexpr int U = 8;
  for (int64_t j0 = c0 + tid; j0 < c1; j0 += static_cast<int64_t>(U) * kArgmaxPartThreads) {
    float v[U];
#pragma unroll
    for (int u = 0; u < U; ++u) {
      const int64_t j = j0 + static_cast<int64_t>(u) * kArgmaxPartThreads;
      v[u] = j < c1 ? xr[j] : -__builtin_inff();
    }
#pragma unroll
    for (int u = 0; u < U; ++u) {
      const int64_t j = j0 + static_cast<int64_t>(u) * kArgmaxPartThreads;
      if (j < c1 && argmax_before(v[u], j, best, bi)) {
        best = v[u];
        bi = j;
      }
    }
  }
#pragma unroll
  for (int off = kWave / 2; off > 0; off /= 2) {
    const float ov = __shfl_xor(best, off);
    const int64_t oi = __shfl_xor(bi, off);
    if (argmax_before(ov, oi, best, bi)) {
      best = ov;
      bi = oi;
    }
  }
  if (tid % kWave == 0) {
    s_v[tid / kWave] = best;
    s_i[tid / kWave] = bi;
  }
  __syncthreads();
  if (tid == 0) {
    for (int w = 1; w < kArgmaxPartThreads / kWave; ++w)
      if (argmax_before(s_v[w], s_i[w], best, bi)) {
        best = s_v[w];
        bi = s_i[w];
      }
    part_v[row * gridDim.x + part] = best;
    part_i[row * gridDim.x + part] = bi;
  }
}

// Stage 2: out[row] = the index of the best of the row's `parts` (value, index)
// pairs, in part order (one wave per row).
__global__ void __launch_bounds__(kWave) argmax_combine_kernel(const float *__restrict__ part_v,
                                                                const int64_t *__restrict__ part_i, int64_t parts,
                                                                int64_t n, int64_t *__restrict__ out, int64_t ld_out) {
  const int lane = static_cast<int>(threadIdx.x);
  const int64_t row = blockIdx.x;
  float best = -__builtin_inff();
  int64_t bi = n;
  for (int64_t j = lane; j < parts; j += kWave)
    if (argmax_before(part_v[row * parts + j], part_i[row * parts + j], best, bi)) {
      best = part_v[row * parts + j];
      bi = part_i[row * parts + j];
    }
#pragma unroll
  for (int off = kWave / 2; off > 0; off /= 2) {
    const float ov = __shfl_xor(best, off);
    const int64_t oi = __shfl_xor(bi, off);
    if (argmax_before(ov, oi, best, bi)) {
      best = ov;
      bi = oi;
    }
  }
  if (lane == 0) out[row * ld_out] = bi;
}

// out[r] = argmax_j x[r, j] (greedy decoding over the vocabulary, reference
// SequenceModel._sample with temperature 0, logits.argmax(dim=-1)). One
// 1024-thread workgroup per row: every thread has its loads in flight at once,
// then (value, index) pairs meet in a wave and an LDS reduction.
template <bool VEC>
__global__ void __launch_bounds__(kArgmaxThreads) argmax_rows_kernel(const float *__restrict__ x, int64_t ldx,
                                                                     int64_t n, int64_t *__restrict__ out,
                                                                     int64_t ld_out) {
  __shared__ float s_v[kArgmaxThreads / kWave];
  __shared__ int64_t s_i[kArgmaxThreads / kWave];
  const int tid = static_cast<int>(threadIdx.x);
  const float *xr = x + static_cast<int64_t>(blockIdx.x) * ldx;
  float best = -__builtin_inff();
  int64_t bi = n;   // no candidate yet: above every index
  if constexpr (VEC) {
    // Batches of U vector loads per thread, all in flight before the compares.
    constexpr int U = 8;
    const int64_t n4 = n / 4;
    for (int64_t q0 = tid; q0 < n4; q0 += static_cast<int64_t>(U) * kArgmaxThreads) {
      f32x4 v[U];
#pragma unroll
      for (int u = 0; u < U; ++u) {
        const int64_t q = q0 + static_cast<int64_t>(u) * kArgmaxThreads;
        v[u] = q < n4 ? *reinterpret_cast<const f32x4 *>(xr + 4 * q) : f32x4{0.0f, 0.0f, 0.0f, 0.0f};
      }
#pragma unroll
      for (int u = 0; u < U; ++u) {
        const int64_t q = q0 + static_cast<int64_t>(u) * kArgmaxThreads;
        if (q < n4) {
          const float e[4] = {v[u].x, v[u].y, v[u].z, v[u].w};
#pragma unroll
          for (int j = 0; j < 4; ++j)
            if (argmax_before(e[j], 4 * q + j, best, bi)) {
              best = e[j];
              bi = 4 * q + j;
            }
        }
      }
    }
    for (int64_t i = 4 * n4 + tid; i < n; i += kArgmaxThreads)
      if (argmax_before(xr[i], i, best, bi)) {
        best = xr[i];
        bi = i;
      }
  } else {
    for (int64_t i = tid; i < n; i += kArgmaxThreads)
      if (argmax_before(xr[i], i, best, bi)) {
        best = xr[i];
        bi = i;
      }
  }
#pragma unroll
  for (int off = kWave / 2; off > 0; off /= 2) {
    const float ov = __shfl_xor(best, off);
    const int64_t oi = __shfl_xor(bi, off);
    if (argmax_before(ov, oi, best, bi)) {
      best = ov;
      bi = oi;
    }
  }
  if (tid % kWave == 0) {
    s_v[tid / kWave] = best;
    s_i[tid / kWave] = bi;
  }
  __syncthreads();
  if (tid == 0) {
    for (int w = 1; w < kArgmaxThreads / kWave; ++w)
      if (argmax_before(s_v[w], s_i[w], best, bi)) {
        best = s_v[w];
        bi = s_i[w];
      }
    out[static_cast<int64_t>(blockIdx.x) * ld_out] = bi;
  }
}

}  // namespace kla
