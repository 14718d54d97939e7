// fused_kla.hpp -- the whole KLA scan in one pass per direction, for gfx950.
//
// Forward (reference kla_scan_torch, src/kla/ops/kla_ops.py:188-290, run per
// lane as in the Metal fused kernel src/kla/ops/kernels/mps/fused_kla_scan.metal:53-131):
//
//   phi = Lv k^2,  r = (v Lv) k                       sufficient statistics
//   a2 = max(a^2, EPS),  p' = max(p, P_MIN)
//   lam_t = (A lam' + phi) / (C lam' + 1),  A = (1 + p' phi)/a2,  C = p'/a2
//   alpha = a / max(a2 + p' lam', EPS),  eta_t = alpha eta' + r
//   var = 1/max(lam_t, EPS),  mean = eta_t var   (prior: mean = a mean, var = a2 var + p')
//   y[b,t,m] = sum_s q mean,  y_var[b,t,m] = sum_s q^2 var
//
// with lam' = lam_{t-1}, eta' = eta_{t-1}. Nothing of shape [B, L, M, S] ever
// reaches memory: HBM traffic is v, Lv, y, y_var ([B, L, M]) plus k, q
// ([B, L, S], shared by all channels), so the kernel is VALU-bound (three
// divisions per lane-step), not HBM-bound.
//
// Layout. One thread owns one (b, m, s) lane chain and walks time serially; a
// 256-thread workgroup holds CH = 256/SP channels of SP (= S rounded up to a
// power of two) state lanes, so the SP lanes of a channel are consecutive and
// the read-out sum over s is a DPP row reduction (SP <= 16) plus cross-row
// shuffles (SP = 32, 64). Padding lanes (s >= S, m >= M) carry q = 0, k = 0 and
// take part in every reduction without contributing to it. With 2^17 and more
// chains (batch * M * S) the lane-serial walk fills the machine; time is not
// split.
//
// Backward (exact adjoint, derived from the forward above; the same formulas as
// the Metal fused backward, fused_kla_scan.metal:135-324, but with the torch
// path's guards: phi is not floored, p is floored at P_MIN). The forward
// checkpoints (lam, eta) entering every kCkpt-step block; the backward walks the
// blocks in reverse, replays kCkpt steps from the checkpoint into registers and
// runs the adjoint back over them. Contractions:
//   dv, dLv   over s: DPP row sums, one lane per channel stores;
//   dk, dq    over m: a per-workgroup partial [B, L, G, S] (G = channel groups),
//             reduced by reduce_groups_kernel in a fixed order (deterministic);
//   da, dp    over (b, t): per-lane register sums -> [B, M, S] partials -> reduced
//             over b the same way.
#pragma once

#include "scan_ops.hpp"

namespace kla {

constexpr int kFusedThreads = 256;
constexpr int kCkpt = 16;   // steps per checkpoint block
constexpr int kFusedTB = 8; // steps per prefetch block in the forward

struct FusedGeom {
  int64_t batch, steps, M, S;
  int64_t groups;   // ceil(M / CH): channel groups (workgroups) per batch row
  int64_t n_ck;     // ceil(steps / kCkpt)
};

struct FusedFwdParams {
  const float *v, *lv, *k, *q, *a, *p, *lam0, *eta0;
  float *y, *yvar, *lam_fin, *eta_fin;
  float *ck_lam, *ck_eta;   // [B, n_ck, M, S] or NULL (no backward will follow)
};

struct FusedBwdParams {
  const float *dy, *dyvar, *dlam_fin, *deta_fin;   // dlam_fin, deta_fin may be NULL
  const float *v, *lv, *k, *q, *a, *p, *ck_lam, *ck_eta;
  float *dv, *dlv, *dlam0, *deta0;                 // dlam0, deta0 may be NULL
  float *part_k, *part_q;                          // [B, L, G, S]
  float *part_a, *part_p;                          // [B, M, S]
};

// ------------------------------------------------------------ lane sums

template <int CTRL>
__device__ __forceinline__ float dpp_shift(float x) {
  return __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(x), CTRL, 0xF, 0xF, false));
}

// Sum over aligned groups of SP consecutive lanes (every lane gets its group's sum).
template <int SP>
__device__ __forceinline__ float group_sum(float x) {
  if constexpr (SP >= 2) x += dpp_shift<0xB1>(x);    // quad_perm [1,0,3,2]
  if constexpr (SP >= 4) x += dpp_shift<0x4E>(x);    // quad_perm [2,3,0,1]
  if constexpr (SP >= 8) x += dpp_shift<0x141>(x);   // row_half_mirror
  if constexpr (SP >= 16) x += dpp_shift<0x140>(x);  // row_mirror
  if constexpr (SP >= 32) x += __shfl_xor(x, 16);
  if constexpr (SP >= 64) x += __shfl_xor(x, 32);
  return x;
}

// Sum over the lanes of a wave that share the lane index modulo SP.
template <int SP>
__device__ __forceinline__ float cross_group_sum(float x) {
#pragma unroll
  for (int off = SP; off < kWave; off *= 2) x += __shfl_xor(x, off);
  return x;
}

struct FusedLane {
  int64_t b, m;
  int s;
  bool active;   // s < S and m < M
};

template <int SP>
__device__ __forceinline__ FusedLane fused_lane(const FusedGeom &g) {
  constexpr int CH = kFusedThreads / SP;
  FusedLane ln;
  const int tid = static_cast<int>(threadIdx.x);
  ln.s = tid % SP;
  ln.b = static_cast<int64_t>(blockIdx.x) / g.groups;
  ln.m = (static_cast<int64_t>(blockIdx.x) % g.groups) * CH + tid / SP;
  ln.active = ln.s < g.S && ln.m < g.M;
  return ln;
}

// One step of the filter; returns lam_t and leaves the intermediates the
// backward needs in the out-parameters.
struct StepIO {
  float phi, r, A, den, Da, alpha;
};

__device__ __forceinline__ float filter_step(float lam, float &eta, float sig, float vv, float kk, float a_s,
                                             float a2, float pp, float inv_a2, float C, StepIO &io) {
  io.phi = sig * (kk * kk);
  io.r = (vv * sig) * kk;
  io.A = (1.0f + pp * io.phi) * inv_a2;
  io.den = C * lam + 1.0f;
  const float lam_t = (io.A * lam + io.phi) / io.den;
  io.Da = fmaxf(a2 + pp * lam, kEps);
  io.alpha = a_s / io.Da;
  eta = io.alpha * eta + io.r;
  return lam_t;
}

// ================================================================ forward

template <int SP, bool PRIOR>
__global__ void __launch_bounds__(kFusedThreads) fused_kla_fwd_kernel(FusedFwdParams prm, FusedGeom g) {
  const FusedLane ln = fused_lane<SP>(g);
  const int64_t M = g.M, S = g.S, L = g.steps;
  const bool mok = ln.m < M, sok = ln.s < S;
  const int64_t ms = ln.m * S + ln.s;
  const int64_t bms = ln.b * M * S + ms;

  const float a_s = ln.active ? prm.a[ms] : 1.0f;
  const float pp = fmaxf(ln.active ? prm.p[ms] : 0.0f, kEps);
  const float a2 = fmaxf(a_s * a_s, kEps);
  const float inv_a2 = 1.0f / a2;
  const float C = pp * inv_a2;
  float lam = (ln.active && prm.lam0) ? prm.lam0[bms] : 1.0f;
  float eta = (ln.active && prm.eta0) ? prm.eta0[bms] : 0.0f;

  const float *__restrict__ vrow = prm.v + ln.b * L * M + ln.m;
  const float *__restrict__ lrow = prm.lv + ln.b * L * M + ln.m;
  const float *__restrict__ krow = prm.k + ln.b * L * S + ln.s;
  const float *__restrict__ qrow = prm.q + ln.b * L * S + ln.s;
  float *yrow = prm.y + ln.b * L * M + ln.m;
  float *vyrow = prm.yvar + ln.b * L * M + ln.m;

  float cv[kFusedTB], cl[kFusedTB], ck[kFusedTB], cq[kFusedTB];
  float nv[kFusedTB], nl[kFusedTB], nk[kFusedTB], nq[kFusedTB];
  auto fetch = [&](int64_t t0, float (&fv)[kFusedTB], float (&fl)[kFusedTB], float (&fk)[kFusedTB],
                   float (&fq)[kFusedTB]) {
#pragma unroll
    for (int j = 0; j < kFusedTB; ++j) {
      const int64_t t = t0 + j;
      const bool tok = t < L;
      fv[j] = (tok && mok) ? vrow[t * M] : 0.0f;
      fl[j] = (tok && mok) ? lrow[t * M] : 0.0f;
      fk[j] = (tok && sok) ? krow[t * S] : 0.0f;
      fq[j] = (tok && sok) ? qrow[t * S] : 0.0f;
    }
  };
  fetch(0, cv, cl, ck, cq);
  for (int64_t t0 = 0; t0 < L; t0 += kFusedTB) {
    if (t0 + kFusedTB < L) fetch(t0 + kFusedTB, nv, nl, nk, nq);
#pragma unroll
    for (int j = 0; j < kFusedTB; ++j) {
      const int64_t t = t0 + j;
      if (t < L) {
        if (prm.ck_lam && (t % kCkpt) == 0 && ln.active) {
          const int64_t ci = ((ln.b * g.n_ck + t / kCkpt) * M + ln.m) * S + ln.s;
          prm.ck_lam[ci] = lam;
          prm.ck_eta[ci] = eta;
        }
        StepIO io;
        lam = filter_step(lam, eta, cl[j], cv[j], ck[j], a_s, a2, pp, inv_a2, C, io);
        const float var = 1.0f / fmaxf(lam, kEps);
        float mean = eta * var, vo = var;
        if (PRIOR) {
          mean = a_s * mean;
          vo = a2 * var + pp;
        }
        const float ys = group_sum<SP>(cq[j] * mean);
        const float vs = group_sum<SP>((cq[j] * cq[j]) * vo);
        if (ln.s == 0 && mok) {
          yrow[t * M] = ys;
          vyrow[t * M] = vs;
        }
      }
    }
#pragma unroll
    for (int j = 0; j < kFusedTB; ++j) {
      cv[j] = nv[j];
      cl[j] = nl[j];
      ck[j] = nk[j];
      cq[j] = nq[j];
    }
  }
  if (ln.active) {
    prm.lam_fin[bms] = lam;
    prm.eta_fin[bms] = eta;
  }
}

// ================================================================ backward

template <int SP, bool PRIOR>
__global__ void __launch_bounds__(kFusedThreads) fused_kla_bwd_kernel(FusedBwdParams prm, FusedGeom g) {
  constexpr int NW = kFusedThreads / kWave;
  __shared__ float s_red[2][kCkpt][NW][SP];

  const FusedLane ln = fused_lane<SP>(g);
  const int64_t M = g.M, S = g.S, L = g.steps;
  const bool mok = ln.m < M, sok = ln.s < S;
  const int64_t ms = ln.m * S + ln.s;
  const int64_t bms = ln.b * M * S + ms;
  const int tid = static_cast<int>(threadIdx.x);
  const int wave = tid / kWave, lane = tid % kWave;
  const int64_t grp = static_cast<int64_t>(blockIdx.x) % g.groups;

  const float a_s = ln.active ? prm.a[ms] : 1.0f;
  const float p_raw = ln.active ? prm.p[ms] : 0.0f;
  const float pp = fmaxf(p_raw, kEps);
  const float a2 = fmaxf(a_s * a_s, kEps);
  const float inv_a2 = 1.0f / a2;
  const float C = pp * inv_a2;

  float gl = (ln.active && prm.dlam_fin) ? prm.dlam_fin[bms] : 0.0f;   // adjoint of lam_t
  float ge = (ln.active && prm.deta_fin) ? prm.deta_fin[bms] : 0.0f;   // adjoint of eta_t
  float acc_a = 0.0f, acc_a2 = 0.0f, acc_p = 0.0f;

  const int64_t bLM = ln.b * L * M + ln.m, bLS = ln.b * L * S + ln.s;
  const float *__restrict__ V = prm.v;
  const float *__restrict__ LV = prm.lv;
  const float *__restrict__ K = prm.k;
  const float *__restrict__ Q = prm.q;
  const float *__restrict__ DY = prm.dy;
  const float *__restrict__ DYV = prm.dyvar;

  for (int64_t c = g.n_ck - 1; c >= 0; --c) {
    const int64_t t0 = c * kCkpt;
    float lh[kCkpt], eh[kCkpt];   // lam_{t-1}, eta_{t-1} over the block
    {
      const int64_t ci = ((ln.b * g.n_ck + c) * M + ln.m) * S + ln.s;
      float lam = ln.active ? prm.ck_lam[ci] : 1.0f;
      float eta = ln.active ? prm.ck_eta[ci] : 0.0f;
#pragma unroll
      for (int j = 0; j < kCkpt; ++j) {
        lh[j] = lam;
        eh[j] = eta;
        const int64_t t = t0 + j;
        if (t < L) {
          const float vv = mok ? V[bLM + t * M] : 0.0f;
          const float sig = mok ? LV[bLM + t * M] : 0.0f;
          const float kk = sok ? K[bLS + t * S] : 0.0f;
          StepIO io;
          lam = filter_step(lam, eta, sig, vv, kk, a_s, a2, pp, inv_a2, C, io);
        }
      }
    }
#pragma unroll
    for (int j = kCkpt - 1; j >= 0; --j) {
      const int64_t t = t0 + j;
      float dk_c = 0.0f, dq_c = 0.0f;
      if (t < L) {
        const float vv = mok ? V[bLM + t * M] : 0.0f;
        const float sig = mok ? LV[bLM + t * M] : 0.0f;
        const float dy = mok ? DY[bLM + t * M] : 0.0f;
        const float dyv = mok ? DYV[bLM + t * M] : 0.0f;
        const float kk = sok ? K[bLS + t * S] : 0.0f;
        const float qq = sok ? Q[bLS + t * S] : 0.0f;
        const float lp = lh[j], ep = eh[j];

        StepIO io;
        float eta_t = ep;
        const float lam_t = filter_step(lp, eta_t, sig, vv, kk, a_s, a2, pp, inv_a2, C, io);
        const float lclamp = fmaxf(lam_t, kEps);
        const float var = 1.0f / lclamp;
        const float mean = eta_t * var;
        const float mean_o = PRIOR ? a_s * mean : mean;
        const float var_o = PRIOR ? a2 * var + pp : var;

        // read-out
        const float dmo = dy * qq, dvo = dyv * (qq * qq);
        dq_c = dy * mean_o + dyv * 2.0f * qq * var_o;
        float dmean = dmo, dvar = dvo;
        if (PRIOR) {
          dmean = dmo * a_s;
          dvar = dvo * a2;
          acc_a += dmo * mean;
          acc_a2 += dvo * var;
          acc_p += dvo;
        }
        // mean = eta var, var = 1/max(lam, EPS)
        const float ge_t = ge + dmean * var;
        const float dvar_tot = dvar + dmean * eta_t;
        const float gl_t = gl + ((lam_t >= kEps) ? -dvar_tot * var * var : 0.0f);
        // eta_t = alpha eta' + r
        const float dalpha = ge_t * ep;
        const float dr = ge_t;
        ge = ge_t * io.alpha;
        // alpha = a / Da, Da = max(a2 + p' lam', EPS)
        acc_a += dalpha / io.Da;
        const float dDa = (a2 + pp * lp >= kEps) ? -dalpha * io.alpha / io.Da : 0.0f;
        acc_a2 += dDa;
        acc_p += dDa * lp;
        // lam_t = (A lam' + phi) / den, den = C lam' + 1;  d lam_t / d lam' = 1/(a2 den^2)
        const float u = gl_t / io.den;
        const float dA = u * lp;
        const float dC = -u * lam_t * lp;
        gl = gl_t * (inv_a2 / (io.den * io.den)) + dDa * pp;
        // A = (1 + p' phi)/a2, C = p'/a2
        const float dphi = u + dA * pp * inv_a2;
        acc_p += (dA * io.phi + dC) * inv_a2;
        acc_a2 -= (dA * io.A + dC * C) * inv_a2;
        // phi = Lv k^2, r = (v Lv) k
        const float dmsi = dr * kk;
        const float dsig_c = dphi * (kk * kk) + dmsi * vv;
        const float dv_c = dmsi * sig;
        dk_c = dphi * 2.0f * sig * kk + dr * (vv * sig);
        const float dv_s = group_sum<SP>(dv_c);
        const float dl_s = group_sum<SP>(dsig_c);
        if (ln.s == 0 && mok) {
          prm.dv[bLM + t * M] = dv_s;
          prm.dlv[bLM + t * M] = dl_s;
        }
      }
      // Partial sums over this workgroup's channels: across the lane groups of
      // the wave here, across the waves once the block is done.
      dk_c = cross_group_sum<SP>(dk_c);
      dq_c = cross_group_sum<SP>(dq_c);
      if (lane < SP) {
        s_red[0][j][wave][lane] = dk_c;
        s_red[1][j][wave][lane] = dq_c;
      }
    }
    __syncthreads();
    for (int i = tid; i < 2 * kCkpt * SP; i += kFusedThreads) {
      const int which = i / (kCkpt * SP);
      const int j = (i / SP) % kCkpt;
      const int s = i % SP;
      const int64_t t = t0 + j;
      if (t < L && s < S) {
        float sum = 0.0f;
#pragma unroll
        for (int w = 0; w < NW; ++w) sum += s_red[which][j][w][s];
        float *part = which == 0 ? prm.part_k : prm.part_q;
        part[((ln.b * L + t) * g.groups + grp) * S + s] = sum;
      }
    }
    __syncthreads();
  }

  if (ln.active) {
    if (prm.dlam0) prm.dlam0[bms] = gl;
    if (prm.deta0) prm.deta0[bms] = ge;
    const float da2_da = (a_s * a_s >= kEps) ? 2.0f * a_s : 0.0f;
    prm.part_a[bms] = acc_a + acc_a2 * da2_da;
    prm.part_p[bms] = (p_raw >= kEps) ? acc_p : 0.0f;
  }
}

// out[o * inner + i] = sum_{j < G} in[(o * G + j) * inner + i], for o < outer, i < inner.
__global__ void reduce_groups_kernel(const float *__restrict__ in, float *__restrict__ out, int64_t outer,
                                     int64_t G, int64_t inner) {
  const int64_t idx = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x;
  if (idx >= outer * inner) return;
  const int64_t o = idx / inner, i = idx % inner;
  const float *src = in + o * G * inner + i;
  float sum = 0.0f;
  for (int64_t j = 0; j < G; ++j) sum += src[j * inner];
  out[idx] = sum;
}

}  // namespace kla
