// causal_conv.hpp -- the KLA layer's short depthwise causal conv over time, for
// gfx950 (the sequence path of CausalConv1d, reference src/kla/layers/common.py:58-96):
//
//   xpad = [state (K-1 steps), x (L steps)] per (batch, channel),
//   y[t] = act(bias + sum_j w[j] xpad[t + j]),   new_state = xpad[L : L + K - 1].
//
// x, y are [B, L, D] with channels contiguous (x may be a strided view: time and
// batch strides given), state [B, D, K-1]. The reference transposes x to
// [B, D, L], concatenates the state in front (a copy of the whole input) and
// calls a library conv (on ROCm an im2col + GEMM); here one thread walks one
// channel over a chunk of time with the K-tap window in registers, so x is read
// once (plus a K-1 halo per chunk) and y written once: an HBM-bound stream.
//
// bf16 I/O follows torch autocast: the weight and bias are rounded to bf16, the
// sum is fp32, the conv output is rounded to bf16 before the activation, and the
// activation's output is rounded again.
//
// Backward (exact adjoint): g[s] = dy[s] act'(pre[s]) with pre recomputed from x;
// d xpad[p] = sum_j w[j] g[p - j] (+ d new_state[p - L] for p >= L), i.e. dx for
// p >= K-1 and d state for p < K-1; dw[j] = sum g[s] xpad[s + j], dbias = sum g,
// each summed per chunk and then over chunks in a fixed order (deterministic).
#pragma once

#include "fused_kla.hpp"

namespace kla {

constexpr int kConvThreads = 256;
constexpr int kConvT = 64;   // time steps per thread (one chunk)
constexpr int kConvMaxK = 8;
// Steps whose loads a thread issues together (one thread walks one channel, so
// a load moves 2 or 4 bytes a lane and one step's loads alone leave the stream
// latency-bound).
constexpr int kConvU = 8;

__device__ __forceinline__ float io_load(const float *p) { return *p; }
__device__ __forceinline__ float io_load(const bf16_t *p) { return to_f32(*p); }
__device__ __forceinline__ void io_store(float *p, float x) { *p = x; }
__device__ __forceinline__ void io_store(bf16_t *p, float x) { *p = from_f32<bf16_t>(x); }

// The value an IO-typed tensor holds for x: x itself in fp32, x rounded in bf16.
template <class IO>
__device__ __forceinline__ float io_round(float x) {
  if constexpr (std::is_same<IO, float>::value) return x;
  else return to_f32(from_f32<bf16_t>(x));
}

// Derivative of the activation at x (torch's silu / gelu / relu backward).
__device__ __forceinline__ float activation_grad(int act, float x) {
  if (act == kActSilu) {
    const float s = 1.0f / (1.0f + expf(-x));
    return s * (1.0f + x * (1.0f - s));
  }
  if (act == kActGelu) {
    const float cdf = 0.5f * (1.0f + erff(x * 0.70710678118654752440f));
    const float pdf = expf(-0.5f * x * x) * 0.39894228040143267794f;
    return cdf + x * pdf;
  }
  if (act == kActRelu) return x > 0.0f ? 1.0f : 0.0f;
  return 1.0f;
}

template <class IO>
struct ConvFwdParams {
  const IO *x;
  int64_t ld_t, ld_b;          // x[b, t, d] = x[b * ld_b + t * ld_t + d]
  const IO *state;             // [B, D, K-1] or NULL (zeros)
  const float *w, *bias;       // [D, K], [D] or NULL
  IO *y;                       // [B, L, D]
  IO *state_out;               // [B, D, K-1] or NULL
  int64_t B, L, D;
  int act;
  int T;                       // time steps per chunk (a workgroup's share of one sequence)
};

template <class IO>
struct ConvBwdParams {
  const IO *dy;                // [B, L, D]
  const IO *x;
  int64_t ld_t, ld_b;
  const IO *state;             // or NULL (zeros)
  const float *w, *bias;
  const IO *dstate_out;        // gradient of new_state [B, D, K-1], or NULL
  IO *dx;                      // [B, L, D]
  IO *dstate;                  // [B, D, K-1] or NULL
  float *part_w, *part_b;      // [B * n_chunks, D, K], [B * n_chunks, D]
  int64_t B, L, D;
  int act;
};

// Grid (ceil(D / 256), ceil(L / T), B); thread = channel d of chunk blockIdx.y.
// The forward has no cross-chunk sums, so its chunk length T is free: the host
// shortens it (64 down to 8 steps) until the grid has workgroups enough.
template <class IO, int K>
__global__ void __launch_bounds__(kConvThreads) causal_conv_fwd_kernel(ConvFwdParams<IO> p) {
  const int64_t d = static_cast<int64_t>(blockIdx.x) * kConvThreads + threadIdx.x;
  if (d >= p.D) return;
  const int64_t b = blockIdx.z;
  const int64_t t0 = static_cast<int64_t>(blockIdx.y) * p.T;
  const int64_t t1 = t0 + p.T < p.L ? t0 + p.T : p.L;
  const IO *xb = p.x + b * p.ld_b + d;
  const IO *st = p.state ? p.state + (b * p.D + d) * (K - 1) : nullptr;

  float w[K];
#pragma unroll
  for (int j = 0; j < K; ++j) w[j] = io_round<IO>(p.w[d * K + j]);
  const float bias = p.bias ? io_round<IO>(p.bias[d]) : 0.0f;

  // win[j] = xpad[t + j], j < K - 1, for the step t about to be computed.
  float win[K > 1 ? K - 1 : 1];
#pragma unroll
  for (int j = 0; j < K - 1; ++j) {
    const int64_t q = t0 + j;   // padded position
    win[j] = q < K - 1 ? (st ? io_load(st + q) : 0.0f) : io_load(xb + (q - (K - 1)) * p.ld_t);
  }
  IO *yb = p.y + b * p.L * p.D + d;
  auto step = [&](int64_t t, float xt) {
    float acc = 0.0f;
#pragma unroll
    for (int j = 0; j < K - 1; ++j) acc += w[j] * win[j];
    acc += w[K - 1] * xt;
    const float pre = io_round<IO>(acc + bias);
    io_store(yb + t * p.D, activation(p.act, pre));
#pragma unroll
    for (int j = 0; j + 1 < K - 1; ++j) win[j] = win[j + 1];
    if (K > 1) win[K - 2] = xt;
  };
  // kConvU steps' loads in flight before their stores (y may not be assumed apart
  // from x by the compiler, so it would not hoist them itself).
  int64_t t = t0;
  for (; t + kConvU <= t1; t += kConvU) {
    float xs[kConvU];
#pragma unroll
    for (int u = 0; u < kConvU; ++u) xs[u] = io_load(xb + (t + u) * p.ld_t);
#pragma unroll
    for (int u = 0; u < kConvU; ++u) step(t + u, xs[u]);
  }
  for (; t < t1; ++t) step(t, io_load(xb + t * p.ld_t));
  // The chunk that ends the sequence holds xpad[L : L + K - 1] in its window.
  if (p.state_out && t1 == p.L) {
    IO *so = p.state_out + (b * p.D + d) * (K - 1);
#pragma unroll
    for (int j = 0; j < K - 1; ++j) io_store(so + j, win[j]);
  }
}

template <class IO, int K>
__global__ void __launch_bounds__(kConvThreads) causal_conv_bwd_kernel(ConvBwdParams<IO> p) {
  const int64_t d = static_cast<int64_t>(blockIdx.x) * kConvThreads + threadIdx.x;
  if (d >= p.D) return;
  const int64_t b = blockIdx.z;
  const int64_t chunk = blockIdx.y;
  const int64_t n_chunks = gridDim.y;
  const int64_t t0 = chunk * kConvT;
  const int64_t t1 = t0 + kConvT < p.L ? t0 + kConvT : p.L;
  const IO *xb = p.x + b * p.ld_b + d;
  const IO *dyb = p.dy + b * p.L * p.D + d;
  const IO *st = p.state ? p.state + (b * p.D + d) * (K - 1) : nullptr;
  const IO *dso = p.dstate_out ? p.dstate_out + (b * p.D + d) * (K - 1) : nullptr;

  float w[K];
#pragma unroll
  for (int j = 0; j < K; ++j) w[j] = io_round<IO>(p.w[d * K + j]);
  const float bias = p.bias ? io_round<IO>(p.bias[d]) : 0.0f;

  float win[K > 1 ? K - 1 : 1];
#pragma unroll
  for (int j = 0; j < K - 1; ++j) {
    const int64_t q = t0 + j;
    win[j] = q < K - 1 ? (st ? io_load(st + q) : 0.0f)
                       : (q - (K - 1) < p.L ? io_load(xb + (q - (K - 1)) * p.ld_t) : 0.0f);
  }
  // acc[i] = d xpad[s + i] gathered so far, while step s is processed.
  float acc[K];
#pragma unroll
  for (int i = 0; i < K; ++i) acc[i] = 0.0f;
  float dw[K];
#pragma unroll
  for (int j = 0; j < K; ++j) dw[j] = 0.0f;
  float db = 0.0f;

  IO *dxb = p.dx + b * p.L * p.D + d;
  IO *dsb = p.dstate ? p.dstate + (b * p.D + d) * (K - 1) : nullptr;
  // Steps s in [t0, t1 + K - 1): g[s] for s < L; position s of xpad completes at
  // step s. xs = x[s], dys = dy[s] (both 0 past L, where they are not read).
  auto step = [&](int64_t s, float xs, float dys) {
    float g = 0.0f;
    if (s < p.L) {
      float a = 0.0f;
#pragma unroll
      for (int j = 0; j < K - 1; ++j) a += w[j] * win[j];
      a += w[K - 1] * xs;
      const float pre = io_round<IO>(a + bias);
      g = dys * activation_grad(p.act, pre);
      if (s < t1) {
#pragma unroll
        for (int j = 0; j < K - 1; ++j) dw[j] += g * win[j];
        dw[K - 1] += g * xs;
        db += g;
      }
#pragma unroll
      for (int j = 0; j + 1 < K - 1; ++j) win[j] = win[j + 1];
      if (K > 1) win[K - 2] = xs;
    }
#pragma unroll
    for (int i = 0; i < K; ++i) acc[i] += w[i] * g;
    // Position q = s is complete: this thread owns q in [t0 + K - 1, t1 + K - 1)
    // (x step q - K + 1), and the first chunk also owns the state positions q < K - 1.
    const int64_t q = s;
    float dq = acc[0];
    if (q >= p.L && dso) dq += io_load(dso + (q - p.L));
    if (q >= t0 + K - 1) {
      io_store(dxb + (q - (K - 1)) * p.D, dq);
    } else if (q < K - 1 && chunk == 0 && dsb) {
      io_store(dsb + q, dq);
    }
#pragma unroll
    for (int i = 0; i + 1 < K; ++i) acc[i] = acc[i + 1];
    acc[K - 1] = 0.0f;
  };
  // Groups of kConvU steps wholly inside the sequence load their x and dy first,
  // unconditionally (the stores of dx may not be assumed apart from x and dy by
  // the compiler, so it would not hoist the loads itself); the rest step by step.
  const int64_t s_end = t1 + K - 1;
  const int64_t s_in = s_end < p.L ? s_end : p.L;
  int64_t s = t0;
  for (; s + kConvU <= s_in; s += kConvU) {
    float xs[kConvU], dys[kConvU];
#pragma unroll
    for (int u = 0; u < kConvU; ++u) {
      xs[u] = io_load(xb + (s + u) * p.ld_t);
      dys[u] = io_load(dyb + (s + u) * p.D);
    }
#pragma unroll
    for (int u = 0; u < kConvU; ++u) step(s + u, xs[u], dys[u]);
  }
  for (; s < s_end; ++s) {
    float xs = 0.0f, dys = 0.0f;
    if (s < p.L) {
      xs = io_load(xb + s * p.ld_t);
      dys = io_load(dyb + s * p.D);
    }
    step(s, xs, dys);
  }
  const int64_t row = b * n_chunks + chunk;
#pragma unroll
  for (int j = 0; j < K; ++j) p.part_w[(row * p.D + d) * K + j] = dw[j];
  p.part_b[row * p.D + d] = db;
}

// dst[i] = src[i] (or 0 with src NULL), i < n: the state passthrough of an empty sequence.
template <class IO>
__global__ void copy_or_zero_kernel(const IO *__restrict__ src, IO *__restrict__ dst, int64_t n) {
  const int64_t i = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x;
  if (i < n) dst[i] = src ? src[i] : IO{};
}

}  // namespace kla
