// rows_linear.hpp -- y = epilogue(norm(x) W^T) for a few rows of x, on gfx950.
//
// One-token decode of the sequence model runs every linear layer on a [batch, K]
// input with batch ~16: the projections of the KLA layers, the SwiGLU MLP and
// the LM head (reference src/kla/models/sequence_model.py, src/kla/layers/
// kla_layer.py, src/kla/layers/common.py). Such a product is a stream over the
// weight matrix (K x N fp32) with a tiny amount of arithmetic per weight, so
// what it needs is many waves with their loads in flight at once, and no extra
// launches around it. This kernel fuses what surrounds the products in a block:
//
//   prologue  optional RMSNorm of the input rows (RMSNorm.forward,
//             common.py:45-55): the products take x * g and the row scale
//             r = rsqrt(mean(x^2) + eps) multiplies each sum, r * sum_k (x g)_k W[n, k],
//             which is the same value up to fp32 rounding; the sums of squares come
//             from the x slices the waves load for the products (no extra pass)
//   product   acc[m, n] = sum_k xn[m, k] W[n, k], fp32 MFMA
//             (v_mfma_f32_16x16x4f32), + bias[n]
//   epilogue  plain: y = acc
//             residual: y = res + acc (the block's x + sublayer(x))
//             swiglu: y[m, j] = silu(acc[m, j]) * acc[m, glu_off + j]
//             (MLP.forward, common.py:116-123: h = w12(x); silu(gate) * up)
//             conv: columns n < conv_n (in_proj's z half) go through one token of
//             the depthwise causal conv, y = act(sum_j w[n, j] window[j] + b[n])
//             over window = [state[m, n, :], acc], and the state shifts by one
//             (CausalConv1d.forward, common.py:70-96); other columns are plain
//
// Work split. A workgroup of 16 waves owns 16 rows and walks 16-column tiles
// (tile, tile + gridDim.x, ...; the grid is sized to the CUs); wave w takes a
// contiguous range of K in steps of 16 and issues all its loads before its
// MFMAs. The 16 partial tiles meet in LDS and are summed in wave order, so
// results do not depend on scheduling. Lane l supplies A[l % 16][l / 16]
// and B[l / 16][l % 16] of each 16x16x4 product and receives
// D[4 (l / 16) + i][l % 16], i < 4; a lane's four k of a 16-wide step (one
// 16-byte load of x and of W where rows are aligned) feed four successive
// products, which is a relabelling of k and leaves the sum unchanged.
#pragma once

#include "causal_conv.hpp"

namespace kla {

constexpr int kRowsLinWaves = 16;
constexpr int kRowsLinThreads = kRowsLinWaves * kWave;
constexpr int kRowsLinTile = 16;    // rows and columns per workgroup

enum RowsLinEpilogue { kEpiPlain = 0, kEpiResidual = 1, kEpiSwiglu = 2, kEpiConv = 3, kEpiQk = 4 };

constexpr int kRowsLinMaxConvK = 8;   // conv taps the kEpiConv epilogue supports

// 16-wide k steps a wave keeps in flight (one pass covers k <= 16 * 16 * steps):
// 6, fewer where two weight tiles (SwiGLU) and the norm weights would push the
// registers (x, two weight sets) past the 128 a 16-wave workgroup allows.
constexpr int rows_lin_steps(int epi, bool norm) {
  return epi == kEpiSwiglu ? (norm ? 3 : 4) : (norm ? 4 : 6);
}

struct RowsLinearParams {
  const float *x;        // [rows, k], row stride ldx
  const float *w;        // [n_w, k], row stride ldw
  const float *bias;     // [n_w] or NULL
  const float *norm_w;   // [k] RMSNorm weight, or NULL for no prologue
  const float *res;      // [rows, n] residual (kEpiResidual), row stride ldres
  float *y;              // [rows, n], row stride ldy
  int64_t ldx, ldw, ldres, ldy;
  int64_t rows, n, k;
  int64_t glu_off;       // kEpiSwiglu: W row of the `up` half of output column 0
  float eps;
  int k_per_wave;        // multiple of 16
  // kEpiConv: the one-token depthwise causal conv on output columns < conv_n
  // (the z half of in_proj): conv_w [conv_n, conv_k], conv_b [conv_n] or NULL,
  // window [rows, conv_n, conv_k - 1] dense; window_out may alias window.
  const float *conv_w, *conv_b, *window;
  float *window_out;
  int64_t conv_n;
  int conv_k, conv_act;
  // kEpiQk: the k, q sensors. Output columns [0, qk_seg) are k (y, row stride
  // ldy), [qk_seg, 2 qk_seg) q (y2, row stride ldy2); each row of each is
  // l2-normalised over its qk_seg columns when qk_norm, then clipped to
  // [-qk_clip, qk_clip] when qk_has_clip. qk_seg is a power of two <= 16, so a
  // segment lies within one 16-column tile.
  float *y2;
  int64_t ldy2;
  int qk_seg, qk_norm, qk_has_clip;
  float qk_clip;
};

typedef float f32x4_t __attribute__((ext_vector_type(4)));

// The four k of a 16-wide step that a lane feeds to the four products, as
// offsets from the step's start: VEC, kq = 4 (lane / 16) + {0, 1, 2, 3}, one
// dwordx4 per lane; otherwise kq = lane / 16 + {0, 4, 8, 12}, so that each of
// the four dword loads has the four lanes of a row read adjacent words. x and W
// use the same labelling, which leaves the sum over k unchanged.
template <bool VEC>
__device__ __forceinline__ int step_k0(int lane) {
  return VEC ? 4 * (lane / 16) : lane / 16;
}

// The lane's four values of a step at p = row + step start + step_k0(lane);
// those at k >= the range end (lim = end - (step start + step_k0)) read as 0.
template <bool VEC>
__device__ __forceinline__ f32x4_t load4(const float *p, int64_t lim) {
  constexpr int D = VEC ? 1 : 4;
  if constexpr (VEC) {
    if (lim >= 4) return *reinterpret_cast<const f32x4_t *>(p);
  }
  f32x4_t v = {0.0f, 0.0f, 0.0f, 0.0f};
  if (lim > 0) v.x = p[0];
  if (lim > D) v.y = p[D];
  if (lim > 2 * D) v.z = p[2 * D];
  if (lim > 3 * D) v.w = p[3 * D];
  return v;
}

// VEC: every row of x and W (and the norm weights) starts 16-byte aligned (ldx,
// ldw multiples of 4 and aligned bases), so in-range groups of four load as one
// dwordx4.
// PIPE: one pass of IT steps covers each wave's k range. The lane's slice of x
// then stays in registers for every column tile the workgroup takes, and the
// next tile's weights are loaded while the current tile's products run.
// ITS (nonzero): IT steps a pass instead of rows_lin_steps, for short k: fewer
// registers, so that two workgroups share a CU (the LM head's many tiles).
template <int EPI, bool NORM, bool VEC, bool PIPE, int ITS = 0>
__global__ void __launch_bounds__(kRowsLinThreads) rows_linear_kernel(RowsLinearParams p) {
  constexpr int NT = EPI == kEpiSwiglu ? 2 : 1;   // weight tiles per output tile
  constexpr int IT = ITS ? ITS : rows_lin_steps(EPI, NORM);   // 16-wide k steps with all their loads in flight
  __shared__ f32x4_t s_part[2][NT][kRowsLinWaves][kWave];
  __shared__ float s_ss[kRowsLinWaves][kRowsLinTile];

  const int tid = static_cast<int>(threadIdx.x);
  const int lane = tid % kWave;
  const int wv = __builtin_amdgcn_readfirstlane(tid / kWave);
  const int64_t m0 = static_cast<int64_t>(blockIdx.y) * kRowsLinTile;
  const int64_t n_tiles = (p.n + kRowsLinTile - 1) / kRowsLinTile;

  // Operands of this lane: A row m0 + lane % 16 of x, B row n0 + lane % 16 of W,
  // four k of each 16-wide step from kq on (step_k0).
  const int r16 = lane % kRowsLinTile;
  const int kq = step_k0<VEC>(lane);
  const int64_t m = m0 + r16;
  const bool m_ok = m < p.rows;
  const float *xrow = p.x + (m_ok ? m : 0) * p.ldx;
  const int64_t k_lo = static_cast<int64_t>(wv) * p.k_per_wave;
  const int64_t k_hi = k_lo + p.k_per_wave < p.k ? k_lo + p.k_per_wave : p.k;

  // Epilogue thread t < 256 owns output (4 (t/4/16) + t%4, (t/4)%16) of each tile,
  // i.e. D element i = t % 4 of lane t / 4.
  const int e_lane = tid / 4, e_i = tid % 4;
  const bool epi_thread = tid < kRowsLinTile * kRowsLinTile;
  const int64_t om = m0 + 4 * (e_lane / kRowsLinTile) + e_i;
  float rs = 1.0f;   // RMSNorm row scale of row om (epilogue threads)

  f32x4_t xa[IT];
  auto load_x = [&](int64_t kb) {
#pragma unroll
    for (int it = 0; it < IT; ++it) {
      const int64_t kk = kb + 16 * it + kq;
      const int64_t lim = (kb + 16 * it < k_hi) ? k_hi - kk : 0;
      xa[it] = m_ok ? load4<VEC>(xrow + kk, lim) : f32x4_t{0.0f, 0.0f, 0.0f, 0.0f};
    }
  };
  // x * g for the products, and this lane's share of the rows' sums of squares.
  float ss = 0.0f;
  auto prep_x = [&](int64_t kb) {
#pragma unroll
    for (int it = 0; it < IT; ++it) {
      if constexpr (NORM) {
        const int64_t kk = kb + 16 * it + kq;
        const int64_t lim = (kb + 16 * it < k_hi) ? k_hi - kk : 0;
        ss = fmaf(xa[it].x, xa[it].x, ss);
        ss = fmaf(xa[it].y, xa[it].y, ss);
        ss = fmaf(xa[it].z, xa[it].z, ss);
        ss = fmaf(xa[it].w, xa[it].w, ss);
        xa[it] = xa[it] * load4<VEC>(p.norm_w + kk, lim);
      }
    }
  };
  auto load_w = [&](int64_t tile, int64_t kb, f32x4_t (&wb)[NT][IT]) {
    const int64_t n = tile * kRowsLinTile + r16;
    const bool ok = tile < n_tiles && n < p.n;
#pragma unroll
    for (int t = 0; t < NT; ++t) {
      const float *wrow = p.w + ((ok ? n : 0) + (t ? p.glu_off : 0)) * p.ldw;
#pragma unroll
      for (int it = 0; it < IT; ++it) {
        const int64_t kk = kb + 16 * it + kq;
        const int64_t lim = (kb + 16 * it < k_hi) ? k_hi - kk : 0;
        wb[t][it] = ok ? load4<VEC>(wrow + kk, lim) : f32x4_t{0.0f, 0.0f, 0.0f, 0.0f};
      }
    }
  };
  auto mma = [&](int64_t kb, const f32x4_t (&wb)[NT][IT], f32x4_t (&acc)[NT]) {
#pragma unroll
    for (int it = 0; it < IT; ++it) {
      if (kb + 16 * it < k_hi) {
#pragma unroll
        for (int t = 0; t < NT; ++t) {
          acc[t] = __builtin_amdgcn_mfma_f32_16x16x4f32(xa[it].x, wb[t][it].x, acc[t], 0, 0, 0);
          acc[t] = __builtin_amdgcn_mfma_f32_16x16x4f32(xa[it].y, wb[t][it].y, acc[t], 0, 0, 0);
          acc[t] = __builtin_amdgcn_mfma_f32_16x16x4f32(xa[it].z, wb[t][it].z, acc[t], 0, 0, 0);
          acc[t] = __builtin_amdgcn_mfma_f32_16x16x4f32(xa[it].w, wb[t][it].w, acc[t], 0, 0, 0);
        }
      }
    }
  };

  // One column tile: its epilogue operands, the products (with `wb` holding the
  // tile's weights, loaded earlier), then the 16-wave sum and the epilogue.
  // `prefetch` runs after the epilogue operands are requested and before the
  // products, so the products wait only for `wb` and the epilogue only for its
  // own operands, never for the next tile's weights in flight.
  auto process = [&](int64_t tile, int buf, f32x4_t (&wb)[NT][IT], auto &&prefetch) {
    const int64_t n0 = tile * kRowsLinTile;
    const int64_t on = n0 + e_lane % kRowsLinTile;
    const bool out_ok = epi_thread && om < p.rows && on < p.n;
    float res = 0.0f, b0 = 0.0f, b1 = 0.0f;
    float win[EPI == kEpiConv ? kRowsLinMaxConvK : 1], cw[EPI == kEpiConv ? kRowsLinMaxConvK : 1];
    const bool conv_col = EPI == kEpiConv && out_ok && on < p.conv_n;
    if (out_ok) {
      if constexpr (EPI == kEpiResidual) res = p.res[om * p.ldres + on];
      if (p.bias) {
        b0 = p.bias[on];
        if constexpr (NT == 2) b1 = p.bias[on + p.glu_off];
      }
    }
    if constexpr (EPI == kEpiConv) {
      if (conv_col) {
        const float *st = p.window + (om * p.conv_n + on) * (p.conv_k - 1);
#pragma unroll
        for (int j = 0; j < kRowsLinMaxConvK; ++j) {
          win[j] = j < p.conv_k - 1 ? st[j] : 0.0f;
          cw[j] = j < p.conv_k ? p.conv_w[on * p.conv_k + j] : 0.0f;
        }
      }
    }
    prefetch();
    f32x4_t acc[NT];
#pragma unroll
    for (int t = 0; t < NT; ++t) acc[t] = f32x4_t{0.0f, 0.0f, 0.0f, 0.0f};
    if constexpr (PIPE) {
      mma(k_lo, wb, acc);
    } else {
      for (int64_t kb = k_lo; kb < k_hi; kb += 16 * IT) {
        load_x(kb);
        load_w(tile, kb, wb);
        if (tile == blockIdx.x) {
          prep_x(kb);
        } else if constexpr (NORM) {
          // Later tiles: x * g again, without re-adding the sums of squares.
          const float keep = ss;
          prep_x(kb);
          ss = keep;
        }
        mma(kb, wb, acc);
      }
    }
#pragma unroll
    for (int t = 0; t < NT; ++t) s_part[buf][t][wv][lane] = acc[t];
    if (NORM && tile == blockIdx.x) {
      // Row sums of squares: lanes l, l^16, l^32, l^48 hold row l % 16.
      float v = ss + __shfl_xor(ss, 16);
      v += __shfl_xor(v, 32);
      if (lane < kRowsLinTile) s_ss[wv][lane] = v;
    }
    __syncthreads();
    if (NORM && tile == blockIdx.x && epi_thread) {
      float tot = 0.0f;
#pragma unroll
      for (int u = 0; u < kRowsLinWaves; ++u) tot += s_ss[u][om - m0];
      rs = rsqrtf(tot / static_cast<float>(p.k) + p.eps);
    }
    if constexpr (EPI == kEpiQk) {
      // The 16 columns of a row lie 4 lanes apart in one wave (lane = 4 col +
      // row % 4): its segment's sum of squares is a butterfly over lane bits
      // 2 .. 2 + log2(qk_seg) - 1, run by every lane (masked columns add 0).
      float val = 0.0f;
      if (out_ok) {
        float sum = 0.0f;
#pragma unroll
        for (int u = 0; u < kRowsLinWaves; ++u) sum += s_part[buf][0][u][e_lane][e_i];
        val = sum + b0;
      }
      float out = val;
      if (p.qk_norm) {
        float ss = val * val;
        for (int off = 4; off < 4 * p.qk_seg; off <<= 1) ss += __shfl_xor(ss, off);
        out = val / fmaxf(sqrtf(ss), 1e-12f);
      }
      if (p.qk_has_clip) out = fminf(fmaxf(out, -p.qk_clip), p.qk_clip);
      if (out_ok) {
        if (on < p.qk_seg)
          p.y[om * p.ldy + on] = out;
        else
          p.y2[om * p.ldy2 + (on - p.qk_seg)] = out;
      }
    }
    if (EPI != kEpiQk && out_ok) {
      float v[NT];
#pragma unroll
      for (int t = 0; t < NT; ++t) {
        float sum = 0.0f;
#pragma unroll
        for (int u = 0; u < kRowsLinWaves; ++u) sum += s_part[buf][t][u][e_lane][e_i];
        v[t] = NORM ? rs * sum : sum;
      }
      v[0] += b0;
      if constexpr (NT == 2) v[1] += b1;
      float out;
      if constexpr (EPI == kEpiSwiglu) {
        out = activation(kActSilu, v[0]) * v[1];
      } else if constexpr (EPI == kEpiResidual) {
        out = res + v[0];
      } else if constexpr (EPI == kEpiConv) {
        out = v[0];
        if (conv_col) {
          // The conv step's order: taps over the state, then the new input, then the bias.
          const float xt = v[0];
          float a = 0.0f;
#pragma unroll
          for (int j = 0; j < kRowsLinMaxConvK - 1; ++j)
            if (j < p.conv_k - 1) a += win[j] * cw[j];
#pragma unroll
          for (int j = 0; j < kRowsLinMaxConvK; ++j)
            if (j == p.conv_k - 1) a += xt * cw[j];
          if (p.conv_b) a = a + p.conv_b[on];
          out = activation(p.conv_act, a);
          // This thread alone reads and writes its window, so window_out may alias it.
          float *so = p.window_out + (om * p.conv_n + on) * (p.conv_k - 1);
#pragma unroll
          for (int j = 0; j + 1 < kRowsLinMaxConvK - 1; ++j)
            if (j + 1 < p.conv_k - 1) so[j] = win[j + 1];
          if (p.conv_k > 1) so[p.conv_k - 2] = xt;
        }
      } else {
        out = v[0];
      }
      p.y[om * p.ldy + on] = out;
    }
  };

  // Tiles blockIdx.x, + gridDim.x, ...; with PIPE the weights ping-pong between
  // two register sets (no copy between them, which would make the products wait
  // for the next tile's loads).
  f32x4_t wa[NT][IT], wb2[NT][IT];
  const int64_t step = gridDim.x;
  int64_t tile = blockIdx.x;
  if constexpr (PIPE) {
    load_x(k_lo);
    load_w(tile, k_lo, wa);
    prep_x(k_lo);
    while (tile < n_tiles) {
      process(tile, 0, wa, [&] { load_w(tile + step, k_lo, wb2); });
      tile += step;
      if (tile >= n_tiles) break;
      process(tile, 1, wb2, [&] { load_w(tile + step, k_lo, wa); });
      tile += step;
    }
  } else {
    for (int buf = 0; tile < n_tiles; tile += step, buf ^= 1) process(tile, buf, wa, [] {});
  }
}

}  // namespace kla
