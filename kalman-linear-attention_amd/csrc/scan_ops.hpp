// scan_ops.hpp -- the four scan policies run by lookback_scan_kernel:
//
//   MobiusFwd   lam_t = (A lam_{t-1} + B) / max(C lam_{t-1} + D, EPS)
//   MobiusBwd   exact scalar adjoint of MobiusFwd (reverse in time)
//   AffineFwd   h_t = g_t h_{t-1} + u_t
//   AffineBwd   exact adjoint of AffineFwd (reverse in time)
//
// The forward formulas follow the reference's tiled Moebius / affine scans
// (src/kla/ops/kernels/triton/tiled_mobius_scan.py:44-111, :161-203) and the
// lane-serial per-step form of the Metal kernels
// (src/kla/ops/kernels/mps/lane_mobius_scan.metal:37-90); the adjoints follow
// TiledMobiusScan.backward / TiledAffineScan.backward
// (tiled_mobius_scan.py:266-279, :291-298).
//
// Both backward recurrences are localised so that a chunk never reads the
// neighbouring chunk's inputs: with w_t = gain_t * nu_t the reverse recurrence
// nu_t = dlam_t + gain_{t+1} nu_{t+1} becomes w_t = gain_t (dlam_t + w_{t+1}),
// an affine map whose coefficients come from step t alone. The carry passed
// between chunks is w, and dlam0 (dh0) is w_0.
#pragma once

#include "lookback_scan.hpp"

namespace kla {

// ---------------------------------------------------------------- element I/O

struct bf16_t {
  uint16_t bits;
};

__device__ __forceinline__ float to_f32(float x) { return x; }
__device__ __forceinline__ float to_f32(bf16_t x) {
  return __uint_as_float(static_cast<uint32_t>(x.bits) << 16);
}

template <class IO>
__device__ __forceinline__ IO from_f32(float x);

template <>
__device__ __forceinline__ float from_f32<float>(float x) {
  return x;
}

// Round to nearest, ties to even; NaN stays a (quiet) NaN.
template <>
__device__ __forceinline__ bf16_t from_f32<bf16_t>(float x) {
  uint32_t u = __float_as_uint(x);
  if ((u & 0x7FFFFFFFu) > 0x7F800000u) return bf16_t{static_cast<uint16_t>((u >> 16) | 0x0040u)};
  u += 0x7FFFu + ((u >> 16) & 1u);
  return bf16_t{static_cast<uint16_t>(u >> 16)};
}

// Scan position s of a chain maps to time t = s (forward) or steps-1-s (reverse).
__device__ __forceinline__ int64_t time_of(bool reverse, const Geom &g, int64_t s) {
  return reverse ? g.steps - 1 - s : s;
}

__device__ __forceinline__ int64_t seq_index(const Geom &g, int64_t b, int64_t t, int64_t n) {
  return (b * g.steps + t) * g.lanes + n;
}

// ------------------------------------------------------------ affine monoid
// (m, c) is the map x -> m*x + c; composing later (L) after earlier (M) gives
// (L.m * M.m, L.m * M.c + L.c).  Reference: _affine_combine, kla_ops.py:119-123.

__device__ __forceinline__ Agg<2> affine_compose(const Agg<2> &L, const Agg<2> &M) {
  return Agg<2>{{L.v[0] * M.v[0], L.v[0] * M.v[1] + L.v[1]}};
}

__device__ __forceinline__ float affine_apply(const Agg<2> &a, float x) { return a.v[0] * x + a.v[1]; }

// ------------------------------------------------------------ Moebius monoid
// [[a, b], [c, d]] acts as x -> (a x + b) / (c x + d). Composition is the 2x2
// product later * earlier. The reference divides the product by its trace
// (_mobius_combine_tracenorm, kla_ops.py:76-116); here it is scaled by the power
// of two that brings the trace into [0.5, 1), which is exact, so the entries
// are the exact product up to one common factor and stay O(1) all the same.
// Every map in this family has non-negative entries, so the trace is positive.

__device__ __forceinline__ Agg<4> mobius_compose(const Agg<4> &L, const Agg<4> &M) {
  float a = L.v[0] * M.v[0] + L.v[1] * M.v[2];
  float b = L.v[0] * M.v[1] + L.v[1] * M.v[3];
  float c = L.v[2] * M.v[0] + L.v[3] * M.v[2];
  float d = L.v[2] * M.v[1] + L.v[3] * M.v[3];
  const int e = __builtin_amdgcn_frexp_expf(a + d);
  return Agg<4>{{__builtin_amdgcn_ldexpf(a, -e), __builtin_amdgcn_ldexpf(b, -e),
                 __builtin_amdgcn_ldexpf(c, -e), __builtin_amdgcn_ldexpf(d, -e)}};
}

// lam = (a x + b) / max(c x + d, EPS): the read-out of kla_ops.py:249-251.
__device__ __forceinline__ float mobius_apply(const Agg<4> &m, float x) {
  return (m.v[0] * x + m.v[1]) / fmaxf(m.v[2] * x + m.v[3], kEps);
}

// ================================================================ MobiusFwd

template <bool HAS_D>
struct MobiusFwd {
  static constexpr int AGG = 4;
  struct Params {
    const float *A, *B, *C, *D, *lam0;
    float *lam;
    int64_t state_stride;   // lanes: state tensors are [batch, lanes]
  };
  template <int S>
  struct Regs {
    float a[S], b[S], c[S], d[HAS_D ? S : 1];
  };

  template <int S>
  __device__ static void load(const Params &p, const Geom &g, Regs<S> &r, int64_t bb, int64_t n,
                              bool ok, int64_t s0, int nvalid) {
#pragma unroll
    for (int j = 0; j < S; ++j) {
      r.a[j] = 1.0f;
      r.b[j] = 0.0f;
      r.c[j] = 0.0f;
      if (HAS_D) r.d[HAS_D ? j : 0] = 1.0f;
      if (ok && j < nvalid) {
        const int64_t i = seq_index(g, bb, s0 + j, n);
        r.a[j] = p.A[i];
        r.b[j] = p.B[i];
        r.c[j] = p.C[i];
        if (HAS_D) r.d[HAS_D ? j : 0] = p.D[i];
      }
    }
  }

  template <int S>
  __device__ static Agg<4> leaf(const Regs<S> &r, int j) {
    return Agg<4>{{r.a[j], r.b[j], r.c[j], HAS_D ? r.d[HAS_D ? j : 0] : 1.0f}};
  }

  template <int S>
  __device__ static Agg<4> reduce(const Regs<S> &r, int nvalid) {
    Agg<4> m{{1.0f, 0.0f, 0.0f, 1.0f}};
#pragma unroll
    for (int j = 0; j < S; ++j)
      if (j < nvalid) m = (j == 0) ? leaf<S>(r, 0) : mobius_compose(leaf<S>(r, j), m);
    return m;
  }

  __device__ static Agg<4> compose(const Agg<4> &L, const Agg<4> &M) { return mobius_compose(L, M); }
  __device__ static float apply(const Agg<4> &m, float x) { return mobius_apply(m, x); }
  __device__ static float initial(const Params &p, int64_t bb, int64_t n) {
    return p.lam0 ? p.lam0[bb * p.state_stride + n] : 1.0f;
  }

  template <int S>
  __device__ static void walk(const Params &p, const Geom &g, const Regs<S> &r, int64_t bb,
                              int64_t n, bool ok, int64_t s0, int nvalid, float x) {
#pragma unroll
    for (int j = 0; j < S; ++j) {
      if (j < nvalid) {
        const float d = HAS_D ? r.d[HAS_D ? j : 0] : 1.0f;
        x = (r.a[j] * x + r.b[j]) / fmaxf(r.c[j] * x + d, kEps);
        if (ok) p.lam[seq_index(g, bb, s0 + j, n)] = x;
      }
    }
  }
};

// ================================================================ MobiusBwd
// Scan order is reverse time. Per step t (reference tiled_mobius_scan.py:266-279):
//   den_t  = max(C_t lam_{t-1} + D_t, EPS)
//   gain_t = (A_t D_t - B_t C_t) / den_t^2
//   nu_t   = dlam_t + w_{t+1},   w_t = gain_t nu_t,   w_T = 0
//   q = nu_t / den_t:  dA = q lam_{t-1}, dB = q, dC = -q lam_t lam_{t-1}, dD = -q lam_t
//   dlam0 = w_0

template <bool HAS_D>
struct MobiusBwd {
  static constexpr int AGG = 2;
  struct Params {
    const float *dlam, *A, *B, *C, *D, *lam0, *lam;
    float *dA, *dB, *dC, *dD, *dlam0;
    int64_t state_stride;   // lanes: state tensors are [batch, lanes]
  };
  template <int S>
  struct Regs {
    float dl[S], den[S], gain[S], lv[S + 1];   // lv[j] = lam at step j's time, lv[j+1] = lam_{t-1}
  };

  template <int S>
  __device__ static void load(const Params &p, const Geom &g, Regs<S> &r, int64_t bb, int64_t n,
                              bool ok, int64_t s0, int nvalid) {
    const float lam_init = (ok && p.lam0) ? p.lam0[bb * p.state_stride + n] : 1.0f;
#pragma unroll
    for (int j = 0; j <= S; ++j) {
      r.lv[j] = 1.0f;
      // Step j's time is t = T-1-s0-j; lv[j] needs t >= 0, lv[j] for t == -1 is lam0.
      if (ok && j <= nvalid) {
        const int64_t t = g.steps - 1 - s0 - j;
        r.lv[j] = (t >= 0) ? p.lam[seq_index(g, bb, t, n)] : lam_init;
      }
    }
#pragma unroll
    for (int j = 0; j < S; ++j) {
      r.dl[j] = 0.0f;
      r.den[j] = 1.0f;
      r.gain[j] = 1.0f;
      if (ok && j < nvalid) {
        const int64_t i = seq_index(g, bb, g.steps - 1 - s0 - j, n);
        const float A = p.A[i], B = p.B[i], C = p.C[i];
        const float D = HAS_D ? p.D[i] : 1.0f;
        r.dl[j] = p.dlam[i];
        const float den = fmaxf(C * r.lv[j + 1] + D, kEps);
        r.den[j] = den;
        r.gain[j] = (A * D - B * C) / (den * den);
      }
    }
  }

  template <int S>
  __device__ static Agg<2> reduce(const Regs<S> &r, int nvalid) {
    Agg<2> m{{1.0f, 0.0f}};
#pragma unroll
    for (int j = 0; j < S; ++j) {
      if (j < nvalid) {
        const Agg<2> f{{r.gain[j], r.gain[j] * r.dl[j]}};
        m = (j == 0) ? f : affine_compose(f, m);
      }
    }
    return m;
  }

  __device__ static Agg<2> compose(const Agg<2> &L, const Agg<2> &M) { return affine_compose(L, M); }
  __device__ static float apply(const Agg<2> &a, float x) { return affine_apply(a, x); }
  __device__ static float initial(const Params &, int64_t, int64_t) { return 0.0f; }

  template <int S>
  __device__ static void walk(const Params &p, const Geom &g, const Regs<S> &r, int64_t bb,
                              int64_t n, bool ok, int64_t s0, int nvalid, float x) {
#pragma unroll
    for (int j = 0; j < S; ++j) {
      if (j < nvalid) {
        const int64_t t = g.steps - 1 - s0 - j;
        const int64_t i = seq_index(g, bb, t, n);
        const float nu = r.dl[j] + x;
        const float q = nu / r.den[j];
        const float lt = r.lv[j], lp = r.lv[j + 1];
        if (ok) {
          if (p.dA) p.dA[i] = q * lp;
          if (p.dB) p.dB[i] = q;
          if (p.dC) p.dC[i] = (-q * lt) * lp;
          if (HAS_D && p.dD) p.dD[i] = -q * lt;
        }
        x = r.gain[j] * nu;
        if (t == 0 && ok && p.dlam0) p.dlam0[bb * p.state_stride + n] = x;
      }
    }
  }
};

// ================================================================ AffineFwd
// h_t = g_t h_{t-1} + u_t, h_{-1} = h0 (reference tiled_mobius_scan.py:161-203).

template <class IO>
struct AffineFwd {
  static constexpr int AGG = 2;
  struct Params {
    const IO *g, *u;
    const float *h0;
    IO *h;
    int64_t state_stride;
  };
  template <int S>
  struct Regs {
    float g[S], u[S];
  };

  template <int S>
  __device__ static void load(const Params &p, const Geom &gm, Regs<S> &r, int64_t bb, int64_t n,
                              bool ok, int64_t s0, int nvalid) {
#pragma unroll
    for (int j = 0; j < S; ++j) {
      r.g[j] = 1.0f;
      r.u[j] = 0.0f;
      if (ok && j < nvalid) {
        const int64_t i = seq_index(gm, bb, s0 + j, n);
        r.g[j] = to_f32(p.g[i]);
        r.u[j] = to_f32(p.u[i]);
      }
    }
  }

  template <int S>
  __device__ static Agg<2> reduce(const Regs<S> &r, int nvalid) {
    Agg<2> m{{1.0f, 0.0f}};
#pragma unroll
    for (int j = 0; j < S; ++j) {
      if (j < nvalid) {
        const Agg<2> f{{r.g[j], r.u[j]}};
        m = (j == 0) ? f : affine_compose(f, m);
      }
    }
    return m;
  }

  __device__ static Agg<2> compose(const Agg<2> &L, const Agg<2> &M) { return affine_compose(L, M); }
  __device__ static float apply(const Agg<2> &a, float x) { return affine_apply(a, x); }
  __device__ static float initial(const Params &p, int64_t bb, int64_t n) {
    return p.h0 ? p.h0[bb * p.state_stride + n] : 0.0f;
  }

  template <int S>
  __device__ static void walk(const Params &p, const Geom &gm, const Regs<S> &r, int64_t bb,
                              int64_t n, bool ok, int64_t s0, int nvalid, float x) {
#pragma unroll
    for (int j = 0; j < S; ++j) {
      if (j < nvalid) {
        x = r.g[j] * x + r.u[j];
        if (ok) p.h[seq_index(gm, bb, s0 + j, n)] = from_f32<IO>(x);
      }
    }
  }
};

// ================================================================ AffineBwd
// Reverse in time (reference tiled_mobius_scan.py:291-298):
//   mu_t = dh_t + w_{t+1},  w_t = g_t mu_t,  w_T = 0
//   dg_t = mu_t h_{t-1} (h_{-1} = h0 or 0),  du_t = mu_t,  dh0 = w_0

template <class IO>
struct AffineBwd {
  static constexpr int AGG = 2;
  struct Params {
    const IO *dh, *g, *h;
    const float *h0;
    IO *dg, *du;
    float *dh0;
    int64_t state_stride;
  };
  template <int S>
  struct Regs {
    float dh[S], g[S], hp[S];
  };

  template <int S>
  __device__ static void load(const Params &p, const Geom &gm, Regs<S> &r, int64_t bb, int64_t n,
                              bool ok, int64_t s0, int nvalid) {
    const float h_init = (ok && p.h0) ? p.h0[bb * p.state_stride + n] : 0.0f;
#pragma unroll
    for (int j = 0; j < S; ++j) {
      r.dh[j] = 0.0f;
      r.g[j] = 1.0f;
      r.hp[j] = 0.0f;
      if (ok && j < nvalid) {
        const int64_t t = gm.steps - 1 - s0 - j;
        const int64_t i = seq_index(gm, bb, t, n);
        r.dh[j] = to_f32(p.dh[i]);
        r.g[j] = to_f32(p.g[i]);
        r.hp[j] = (t > 0) ? to_f32(p.h[i - gm.lanes]) : h_init;
      }
    }
  }

  template <int S>
  __device__ static Agg<2> reduce(const Regs<S> &r, int nvalid) {
    Agg<2> m{{1.0f, 0.0f}};
#pragma unroll
    for (int j = 0; j < S; ++j) {
      if (j < nvalid) {
        const Agg<2> f{{r.g[j], r.g[j] * r.dh[j]}};
        m = (j == 0) ? f : affine_compose(f, m);
      }
    }
    return m;
  }

  __device__ static Agg<2> compose(const Agg<2> &L, const Agg<2> &M) { return affine_compose(L, M); }
  __device__ static float apply(const Agg<2> &a, float x) { return affine_apply(a, x); }
  __device__ static float initial(const Params &, int64_t, int64_t) { return 0.0f; }

  template <int S>
  __device__ static void walk(const Params &p, const Geom &gm, const Regs<S> &r, int64_t bb,
                              int64_t n, bool ok, int64_t s0, int nvalid, float x) {
#pragma unroll
    for (int j = 0; j < S; ++j) {
      if (j < nvalid) {
        const int64_t t = gm.steps - 1 - s0 - j;
        const int64_t i = seq_index(gm, bb, t, n);
        const float mu = r.dh[j] + x;
        if (ok) {
          if (p.dg) p.dg[i] = from_f32<IO>(mu * r.hp[j]);
          if (p.du) p.du[i] = from_f32<IO>(mu);
        }
        x = r.g[j] * mu;
        if (t == 0 && ok && p.dh0) p.dh0[bb * p.state_stride + n] = x;
      }
    }
  }
};

}  // namespace kla
