// gate_skip.hpp -- the KLALayer output tail after the scan, for gfx950
// (reference src/kla/layers/kla_layer.py:333-337):
//
//   t = y + lambda_skip * residual        (when the layer has a lambda skip)
//   out = t * act(gate)                   (when the layer has a gate)
//
// y is fp32 [rows, M]; out is [rows, M] fp32, or bf16 when its consumer (the
// output projection under autocast) would round it to bf16 anyway; residual and
// gate are [rows, M] rows of one IO type (fp32, or bf16 under autocast), each
// with its own row stride (the gate is one half of the input projection).
// lambda_skip is a 0-dim or [M] fp32 tensor.
// torch forms this chain as four or five elementwise passes plus their backward
// passes; here it is one pass each way.
//
// The values are torch's: a 0-dim lambda_skip does not take part in type
// promotion, so with bf16 residuals lambda * residual is rounded to bf16 before
// the add; act(gate) is rounded to the gate's dtype; the gradients of bf16
// tensors are rounded where autograd casts them (d(lambda * residual) and d act
// to bf16, then d residual and d gate). d lambda is summed per column over a
// block of rows and then over the blocks in a fixed order (deterministic); for
// a 0-dim lambda the columns are then added and the total rounded to the
// residual's dtype, as torch's sum of a bf16 tensor is.
#pragma once

#include "causal_conv.hpp"

namespace kla {

constexpr int kTailThreads = 256;
constexpr int kTailRows = 16;   // rows per workgroup (one partial row of d lambda per workgroup)

template <class IO, class OUT>
struct TailParams {
  const float *y;                // [rows, M] dense
  const IO *res;                 // rows ld_res apart, or NULL (no skip)
  const IO *gate;                // rows ld_gate apart, or NULL (no gate)
  int64_t ld_res, ld_gate;
  const float *lam;              // [M] (lam_vector) or [1]; with res
  int lam_vector;
  int act;
  int64_t rows, M;
  // forward
  OUT *out;                      // [rows, M] dense
  int64_t rows_per;              // rows per workgroup of the forward
  // backward
  const OUT *dout;               // [rows, M] dense
  float *dy;                     // [rows, M] dense
  IO *dres, *dgate;              // [rows, M] dense, or NULL
  float *part_lam;               // [n_row_blocks, M]: per-block column sums of d lambda terms
};

// V consecutive elements at p (V = 1, or 8 with p 16-byte aligned), widened to fp32.
template <int V>
__device__ __forceinline__ void vload(const float *p, float (&x)[V]) {
  if constexpr (V == 8) {
    const float4 a = reinterpret_cast<const float4 *>(p)[0], b = reinterpret_cast<const float4 *>(p)[1];
    x[0] = a.x; x[1] = a.y; x[2] = a.z; x[3] = a.w;
    x[4] = b.x; x[5] = b.y; x[6] = b.z; x[7] = b.w;
  } else {
    x[0] = *p;
  }
}

template <int V>
__device__ __forceinline__ void vload(const bf16_t *p, float (&x)[V]) {
  if constexpr (V == 8) {
    const uint4 u = *reinterpret_cast<const uint4 *>(p);
    const uint32_t w[4] = {u.x, u.y, u.z, u.w};
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      x[2 * i] = __uint_as_float(w[i] << 16);
      x[2 * i + 1] = __uint_as_float(w[i] & 0xFFFF0000u);
    }
  } else {
    x[0] = to_f32(*p);
  }
}

template <int V>
__device__ __forceinline__ void vstore(float *p, const float (&x)[V]) {
  if constexpr (V == 8) {
    reinterpret_cast<float4 *>(p)[0] = float4{x[0], x[1], x[2], x[3]};
    reinterpret_cast<float4 *>(p)[1] = float4{x[4], x[5], x[6], x[7]};
  } else {
    *p = x[0];
  }
}

template <int V>
__device__ __forceinline__ void vstore(bf16_t *p, const float (&x)[V]) {
  if constexpr (V == 8) {
    *reinterpret_cast<uint4 *>(p) = uint4{pack_bf16x2(x[0], x[1]), pack_bf16x2(x[2], x[3]),
                                          pack_bf16x2(x[4], x[5]), pack_bf16x2(x[6], x[7])};
  } else {
    *p = from_f32<bf16_t>(x[0]);
  }
}

// V elements of the forward chain at row r, columns m..m+V: t (before the gate),
// the gate factor gg, and the residual and raw gate values.
template <class IO, class OUT, int V>
__device__ __forceinline__ void tail_values(const TailParams<IO, OUT> &p, int64_t r, int64_t m, const float (&y)[V],
                                            float (&t)[V], float (&gg)[V], float (&resv)[V], float (&gatev)[V]) {
#pragma unroll
  for (int v = 0; v < V; ++v) {
    t[v] = y[v];
    resv[v] = 0.0f;
    gg[v] = 1.0f;
    gatev[v] = 0.0f;
  }
  if (p.res) {
    vload<V>(p.res + r * p.ld_res + m, resv);
    float lam[V];
    if (p.lam_vector) {
      vload<V>(p.lam + m, lam);
    } else {
#pragma unroll
      for (int v = 0; v < V; ++v) lam[v] = p.lam[0];
    }
#pragma unroll
    for (int v = 0; v < V; ++v) {
      float t1 = lam[v] * resv[v];
      if (!p.lam_vector) t1 = io_round<IO>(t1);
      t[v] = y[v] + t1;
    }
  }
  if (p.gate) {
    vload<V>(p.gate + r * p.ld_gate + m, gatev);
#pragma unroll
    for (int v = 0; v < V; ++v) gg[v] = io_round<IO>(activation(p.act, gatev[v]));
  }
}

// Grid (ceil(rows / rows_per), ceil(M / (256 V))); thread = V consecutive columns
// of a row block. The forward sums nothing across rows, so its row blocks can be
// short (the host picks rows_per, 16 down to 1, to give the grid workgroups enough).
template <class IO, class OUT, int V>
__global__ void __launch_bounds__(kTailThreads) gate_skip_fwd_kernel(TailParams<IO, OUT> p) {
  const int64_t m = (static_cast<int64_t>(blockIdx.y) * kTailThreads + threadIdx.x) * V;
  if (m >= p.M) return;
  const int64_t r0 = static_cast<int64_t>(blockIdx.x) * p.rows_per;
  const int64_t r1 = r0 + p.rows_per < p.rows ? r0 + p.rows_per : p.rows;
  for (int64_t r = r0; r < r1; ++r) {
    float y[V], t[V], gg[V], resv[V], gatev[V];
    vload<V>(p.y + r * p.M + m, y);
    tail_values<IO, OUT, V>(p, r, m, y, t, gg, resv, gatev);
    if (p.gate) {
#pragma unroll
      for (int v = 0; v < V; ++v) t[v] *= gg[v];
    }
    vstore<V>(p.out + r * p.M + m, t);
  }
}

template <class IO, class OUT, int V>
__global__ void __launch_bounds__(kTailThreads) gate_skip_bwd_kernel(TailParams<IO, OUT> p) {
  const int64_t m = (static_cast<int64_t>(blockIdx.y) * kTailThreads + threadIdx.x) * V;
  if (m >= p.M) return;
  const int64_t r0 = static_cast<int64_t>(blockIdx.x) * kTailRows;
  const int64_t r1 = r0 + kTailRows < p.rows ? r0 + kTailRows : p.rows;
  float acc[V];
#pragma unroll
  for (int v = 0; v < V; ++v) acc[v] = 0.0f;
  float lam[V];
#pragma unroll
  for (int v = 0; v < V; ++v) lam[v] = 0.0f;
  if (p.res) {
    if (p.lam_vector) {
      vload<V>(p.lam + m, lam);
    } else {
#pragma unroll
      for (int v = 0; v < V; ++v) lam[v] = p.lam[0];
    }
  }
  for (int64_t r = r0; r < r1; ++r) {
    const int64_t i = r * p.M + m;
    float y[V], t[V], gg[V], resv[V], gatev[V], dout[V], dt[V];
    vload<V>(p.y + i, y);
    tail_values<IO, OUT, V>(p, r, m, y, t, gg, resv, gatev);
    vload<V>(p.dout + i, dout);
#pragma unroll
    for (int v = 0; v < V; ++v) dt[v] = dout[v];
    if (p.gate) {
      // out = t * g: d g in the gate's dtype, then through the activation.
      float dgate[V];
#pragma unroll
      for (int v = 0; v < V; ++v) {
        const float dg = io_round<IO>(dout[v] * t[v]);
        dgate[v] = activation_grad(p.act, gatev[v]) * dg;
        dt[v] = dout[v] * gg[v];
      }
      if (p.dgate) vstore<V>(p.dgate + i, dgate);
    }
    vstore<V>(p.dy + i, dt);
    if (p.res) {
      // t = y + lambda * res; with a 0-dim lambda the product (and its gradient)
      // has the residual's dtype.
      float dres[V];
#pragma unroll
      for (int v = 0; v < V; ++v) {
        const float dt1 = p.lam_vector ? dt[v] : io_round<IO>(dt[v]);
        dres[v] = dt1 * lam[v];
        acc[v] += p.lam_vector ? dt1 * resv[v] : io_round<IO>(dt1 * resv[v]);
      }
      if (p.dres) vstore<V>(p.dres + i, dres);
    }
  }
  if (p.res && p.part_lam) vstore<V>(p.part_lam + static_cast<int64_t>(blockIdx.x) * p.M + m, acc);
}

// out[0] = in[0] rounded to IO: a 0-dim lambda's gradient is summed in the
// residual's dtype.
template <class IO>
__global__ void round_scalar_kernel(const float *in, float *out) {
  if (threadIdx.x == 0) out[0] = io_round<IO>(in[0]);
}

}  // namespace kla
