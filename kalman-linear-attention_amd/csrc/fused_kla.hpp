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
// power of two, at least 4, at most 256) state lanes, so the SP lanes of a
// channel are consecutive and the read-out sum over s is a DPP row reduction
// (SP <= 16) plus cross-row shuffles (SP = 32, 64). A channel of SP = 128 or
// 256 lanes spans SP/64 waves: each wave sums its 64 lanes and the waves'
// partial sums are added in wave order when the block's outputs are written. Inputs and outputs move through LDS
// in double-buffered blocks of time steps (see "block staging"). Padding lanes (s >= S, m >= M) carry q = 0, k = 0 and
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
constexpr int kFusedTB = 32; // steps per staged block in the forward

struct FusedGeom {
  int64_t batch, steps, M, S;
  int64_t groups;   // ceil(M / CH): channel groups (workgroups) per batch row
  int64_t n_ck;     // ceil(steps / kCkpt)
};

// The [B, L, M] sensor inputs v and the precision operand: rows of stride ld
// (element (b, t, m) at (b * L + t) * ld + m, so they can be column slices of
// the layer's projection), fp32 or bf16. The precision operand is Lambda^v, or
// with log_var the projection's log sigma^2, from which the kernels form
// Lambda^v = 1 / min(softplus(log sigma^2) + ov_min, ov_max) while staging (the
// layer's _project_sensors tail, reference kla_layer.py:224-230).
struct SensorIn {
  const void *v, *lv;
  int64_t ld_v, ld_lv;
  int bf16;       // v, lv -- and the gradients dv, dlv the backward writes -- are bf16
  int log_var;
  float ov_min, ov_max;
};

struct FusedFwdParams {
  SensorIn sn;
  const float *k, *q, *a, *p, *lam0, *eta0;
  float *y, *yvar, *lam_fin, *eta_fin;
  float *ck_lam, *ck_eta;   // [B, n_ck, M, S] or NULL (no backward will follow)
};

struct FusedBwdParams {
  const float *dy, *dyvar, *dlam_fin, *deta_fin;   // dlam_fin, deta_fin may be NULL
  SensorIn sn;
  const float *k, *q, *a, *p, *ck_lam, *ck_eta;
  void *dv, *dlv;                                  // dense [B, L, M] of the sensor dtype
  float *dlam0, *deta0;                            // may be NULL
  float *part_k, *part_q;                          // [B, L, G, S]
  float *part_a, *part_p;                          // [B, M, S]
};

// ------------------------------------------------------------ lane sums

// Every control used here reads a lane of the same row, so no lane's source is
// out of range and the move needs no "old" value: with none given, the
// compiler folds the move into the add that consumes it (one v_add_f32_dpp).
template <int CTRL>
__device__ __forceinline__ float dpp_shift(float x) {
  return __int_as_float(__builtin_amdgcn_mov_dpp(__float_as_int(x), CTRL, 0xF, 0xF, true));
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

// Waves a channel's SP lanes span, and the lanes of a channel within one wave.
template <int SP>
constexpr int waves_per_channel() {
  return SP > kWave ? SP / kWave : 1;
}
template <int SP>
constexpr int lanes_in_wave() {
  return SP > kWave ? kWave : SP;
}

// Sum over a channel's SP lanes (every lane of the channel gets it) for SP up
// to the workgroup size: the in-wave group sum, then for SP > 64 the channel's
// wave sums added in wave order through LDS. Every thread of the workgroup
// must make the call.
template <int SP>
__device__ __forceinline__ float channel_sum(float x) {
  if constexpr (SP <= kWave) {
    return group_sum<SP>(x);
  } else {
    constexpr int WPC = SP / kWave;
    __shared__ float part[kFusedThreads / kWave];
    x = group_sum<kWave>(x);
    const int wave = static_cast<int>(threadIdx.x) / kWave;
    __syncthreads();   // every reader of the previous call is done
    if (threadIdx.x % kWave == 0) part[wave] = x;
    __syncthreads();
    const int w0 = wave - wave % WPC;
    float t = part[w0];
#pragma unroll
    for (int i = 1; i < WPC; ++i) t += part[w0 + i];
    return t;
  }
}

// x of this lane plus x of the same lane position in the paired row (rows
// 0-1, 2-3): v_permlane16_swap with both operands x leaves x(row 0) in the
// first result and x(row 1) in the second on both rows of a pair.
__device__ __forceinline__ float row_pair_sum(float x) {
  const auto r = __builtin_amdgcn_permlane16_swap(__float_as_uint(x), __float_as_uint(x), false, false);
  return __uint_as_float(r[0]) + __uint_as_float(r[1]);
}

// x of this lane plus x of the lane 32 away (v_permlane32_swap, as above).
__device__ __forceinline__ float half_pair_sum(float x) {
  const auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(x), __float_as_uint(x), false, false);
  return __uint_as_float(r[0]) + __uint_as_float(r[1]);
}

// Sum over the lanes of a wave that share the lane index modulo SP (every lane
// gets its sum): rotations by SP within a 16-lane row, then the row pairs and
// the two wave halves.
template <int SP>
__device__ __forceinline__ float cross_group_sum(float x) {
  if constexpr (SP <= 4) x += dpp_shift<0x124>(x);   // row_ror:4
  if constexpr (SP <= 8) x += dpp_shift<0x128>(x);   // row_ror:8
  if constexpr (SP <= 16) x = row_pair_sum(x);
  if constexpr (SP <= 32) x = half_pair_sum(x);
  return x;
}

// Sums over the four 16-lane rows of a wave, for N values at once (N a multiple
// of 4): on return a lane of row r holds in w[i], i < N / 4, the sum over the
// rows of w[(N / 2)(r >> 1) + (N / 4)(r & 1) + i] at its position in the row.
// v_permlane32_swap on the pair (w[i], w[i + N/2]) leaves the low half of the
// wave both halves of w[i] and the high half both halves of w[i + N/2]; then
// v_permlane16_swap does the same for row pairs. 3 N / 4 swaps and adds in all,
// against 4 N for N separate cross_group_sum<16> calls.
template <int N>
__device__ __forceinline__ void cross_row_transpose_sum(float (&w)[N]) {
  static_assert(N % 4 == 0, "N must be a multiple of 4");
#pragma unroll
  for (int i = 0; i < N / 2; ++i) {
    const auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(w[i]), __float_as_uint(w[i + N / 2]), false, false);
    w[i] = __uint_as_float(r[0]) + __uint_as_float(r[1]);
  }
#pragma unroll
  for (int i = 0; i < N / 4; ++i) {
    const auto r = __builtin_amdgcn_permlane16_swap(__float_as_uint(w[i]), __float_as_uint(w[i + N / 4]), false, false);
    w[i] = __uint_as_float(r[0]) + __uint_as_float(r[1]);
  }
}

// One butterfly stage of transpose_sum: lanes whose bit BIT is 0 keep the lower
// half of w[0, n) and send the upper half to their partner (the lane CTRL reads,
// whose bit BIT is 1 and which does the opposite); w[0, n/2) becomes kept + received.
template <int CTRL, int BIT, int n, int N>
__device__ __forceinline__ void transpose_stage(float (&w)[N], int lane) {
  const bool hi = (lane >> BIT) & 1;
#pragma unroll
  for (int i = 0; i < n / 2; ++i) {
    const float keep = hi ? w[i + n / 2] : w[i];
    const float send = hi ? w[i] : w[i + n / 2];
    w[i] = keep + dpp_shift<CTRL>(send);
  }
}

// Group sums of N values at once (SP = 4, 8 or 16 lanes per group, N a multiple
// of SP): on return lane s of a group holds in w[r], r < N / SP, the sum over the
// group's lanes of their w[(N / SP) s + r]. The butterfly halves the values at
// each stage, 3 (N - N / SP) VALU ops in all, where N separate group_sum calls
// take N log2(SP) DPP adds plus their hazard waits, and every lane ends with
// distinct results to store. Partners per stage: lane ^ 8 (row_ror:8), the
// mirror within 8 lanes (row_half_mirror, lane ^ 7), lane ^ 2, lane ^ 1.
template <int SP, int N>
__device__ __forceinline__ void transpose_sum(float (&w)[N], int lane) {
  static_assert(SP == 4 || SP == 8 || SP == 16, "transpose_sum serves 4, 8 or 16 lanes per group");
  static_assert(N % SP == 0, "N must be a multiple of SP");
  if constexpr (SP == 16) transpose_stage<0x128, 3, N>(w, lane);
  if constexpr (SP >= 8) transpose_stage<0x141, 2, N * 8 / SP>(w, lane);
  transpose_stage<0x4E, 1, N * 4 / SP>(w, lane);
  transpose_stage<0xB1, 0, N * 2 / SP>(w, lane);
}

// The sums over a channel's lanes in this wave of kCkpt per-step values at
// once, stored to `row` (a channel's [TB + kPad] tile row in LDS) at steps
// j0 + 0 .. kCkpt - 1. Up to 16 lanes per channel, transpose_sum leaves lane s
// the sums of steps (kCkpt / SP) s + r. Wider channels take the 16-lane
// transpose_sum within each row (lane l then holds its row's sum for step l % 16)
// and add the row pair (32 lanes) and the wave halves (64 and more, where the
// wave holds 64 of the channel's lanes): lanes 0-15 of the channel in the wave
// store its 16 steps. s is the lane's state index, SG the channel's lanes in a
// wave.
template <int SP, int N>
__device__ __forceinline__ void step_sums_to_lds(float (&w)[N], int lane, int s, float *row, int j0) {
  static_assert(N == 16, "one checkpoint half of steps at a time");
  if constexpr (SP <= 16) {
    transpose_sum<SP, N>(w, lane);
#pragma unroll
    for (int r = 0; r < N / SP; ++r) row[j0 + (N / SP) * s + r] = w[r];
  } else {
    constexpr int SG = lanes_in_wave<SP>();
    transpose_sum<16, N>(w, lane);
    float x = row_pair_sum(w[0]);
    if constexpr (SP >= 64) x = half_pair_sum(x);
    if (s % SG < 16) row[j0 + s % 16] = x;
  }
}

struct FusedLane {
  int64_t b, m;
  int s;
  bool active;   // s < S and m < M
};

// The workgroup's place in the grid. Workgroups go to MI355X's 8 XCDs round
// robin (workgroup i to XCD i % 8), each XCD with its own L2. Numbering them
// (i % 8) * (n / 8) + i / 8 gives every XCD a contiguous run of channel groups,
// so the short rows of neighbouring groups' tiles (16 channels: 32 bytes of a
// bf16 row) share that L2's lines instead of every XCD fetching whole lines.
// The identity when the grid is not a multiple of 8.
constexpr int kXcds = 8;

__device__ __forceinline__ int64_t xcd_block() {
  const int64_t n = gridDim.x, i = blockIdx.x;
  if (n % kXcds) return i;
  return (i % kXcds) * (n / kXcds) + i / kXcds;
}

template <int SP>
__device__ __forceinline__ FusedLane fused_lane(const FusedGeom &g) {
  constexpr int CH = kFusedThreads / SP;
  FusedLane ln;
  const int tid = static_cast<int>(threadIdx.x);
  const int64_t blk = xcd_block();
  ln.s = tid % SP;
  ln.b = blk / g.groups;
  ln.m = (blk % g.groups) * CH + tid / SP;
  ln.active = ln.s < g.S && ln.m < g.M;
  return ln;
}

// One step of the filter (filter_step below). The fused kernels are VALU-bound,
// so quotients are formed with the hardware reciprocal (v_rcp_f32, 1 ulp) times
// the numerator instead of the ~10-instruction IEEE division: a relative error
// of ~2 ulp per step, different from step to step, which the contractive
// recurrence does not amplify.
constexpr float kInvEps = 1.0f / kEps;

__device__ __forceinline__ float rcp(float x) { return __builtin_amdgcn_rcpf(x); }

// a2 = max(a^2, EPS) as an unevaluated sum hi + lo: hi = fl(a a) and lo = a a - hi
// exactly (one fma), or (EPS, 0) where the clamp acts. Every step of the filter
// divides by a2 + p' lam; a2 rounded once and reused for every step would bias
// each step's decay by the same half ulp, and where the filter forgets slowly
// (a close to 1, small p', a time constant of ~1 / (1 - a^2 / (a2 + p' lam))
// steps) that bias adds up over the time constant instead of averaging out:
// with a ~ 0.999 the final state of a 1024-step sequence moved by ~3e-5
// relative. With lo folded in, each step's denominator is rounded once, afresh.
struct A2 {
  float hi, lo;
};

__device__ __forceinline__ A2 split_a2(float a) {
  const float hi = a * a;
  if (hi < kEps) return A2{kEps, 0.0f};
  return A2{hi, fmaf(a, a, -hi)};
}

// 1 / (a2 + p' lam), the quotient every filter step needs.
__device__ __forceinline__ float inv_den_a(const A2 &a2, float pp, float lam) {
  return rcp(fmaf(pp, lam, a2.lo) + a2.hi);
}

// 1 / den = a2 / (a2 + p' lam) from idn_a = 1 / (a2 + p' lam), with a2's low part.
__device__ __forceinline__ float inv_den_from(const A2 &a2, float idn_a) {
  return fmaf(a2.hi, idn_a, a2.lo * idn_a);
}

// One step of the filter (reference kla_step, kla_ops.py:293-331, phi not floored
// as in the scan): with idn_a = 1 / (a2 + p' lam),
//   lam_t = lam / (a2 + p' lam) + phi = lam idn_a + phi       (d lam_t / d phi = 1)
//   eta_t = alpha eta + r,  alpha = a / max(a2 + p' lam, EPS) = a min(idn_a, 1/EPS)
// which is lam_t = (A lam + phi) / den with A = (1 + p' phi)/a2, den = C lam + 1,
// C = p'/a2 (the Moebius leaf), and the gain clamp. The fused kernels are
// VALU-bound, so the quotient is the hardware reciprocal (v_rcp_f32, 1 ulp) of
// the one denominator. phi = Lv k^2 and r = (v Lv) k come in from the caller
// (from the k^2 and v Lv tiles the kernels stage per block). Returns lam_t;
// idn_a is left for the backward.
__device__ __forceinline__ float filter_step(float lam, float &eta, float phi, float r, float a_s, const A2 &a2,
                                             float pp, float &idn_a) {
  idn_a = inv_den_a(a2, pp, lam);
  eta = fmaf(a_s * fminf(idn_a, kInvEps), eta, r);
  return fmaf(lam, idn_a, phi);
}

// ------------------------------------------------------- block staging
//
// Per block of TB steps the workgroup moves its [TB, CH] tiles of the
// [B, L, M] tensors and its [TB, S] rows of the [B, L, S] tensors through LDS:
// a few coalesced global accesses per thread instead of one (broadcast) access
// per lane and step. Tiles are stored channel-major ([CH][TB + 4]) so a lane
// reads its channel's value at step j from one LDS word that all SP lanes of
// the channel share.

constexpr int kPad = 4;

// Four consecutive steps of one LDS tile row (16-byte aligned: rows are TB + 4
// floats, TB a multiple of 4), read with one ds_read_b128; pick4 takes step i % 4.
__device__ __forceinline__ float4 lds4(const float *row, int j) {
  return *reinterpret_cast<const float4 *>(row + j);
}
__device__ __forceinline__ float pick4(const float4 &v, int i) {
  return i == 0 ? v.x : i == 1 ? v.y : i == 2 ? v.z : v.w;
}

// Global -> registers: element e = tid + 256 i of the [TB, W] tile whose rows
// are `row0 + t * ld` (t < rows) and columns c < cols of a row.
template <int TB, int W>
struct TileRegs {
  static constexpr int N = (TB * W + kFusedThreads - 1) / kFusedThreads;
  float x[N];
};

template <int TB, int W>
__device__ __forceinline__ void tile_load(TileRegs<TB, W> &r, const float *__restrict__ base, int64_t ld,
                                          int64_t rows, int64_t cols) {
  const int tid = static_cast<int>(threadIdx.x);
#pragma unroll
  for (int i = 0; i < TileRegs<TB, W>::N; ++i) {
    const int e = tid + i * kFusedThreads;
    const int t = e / W, c = e % W;
    r.x[i] = (e < TB * W && t < rows && c < cols) ? __builtin_nontemporal_load(base + t * ld + c) : 0.0f;
  }
}

template <int TB, int W>
__device__ __forceinline__ void tile_to_lds(const TileRegs<TB, W> &r, float (*lds)[TB + kPad]) {
  const int tid = static_cast<int>(threadIdx.x);
#pragma unroll
  for (int i = 0; i < TileRegs<TB, W>::N; ++i) {
    const int e = tid + i * kFusedThreads;
    if (e < TB * W) lds[e % W][e / W] = r.x[i];
  }
}

// The elementwise product x * y of two staged tiles (y = x gives k^2 from k,
// y = Lv gives v Lv from v), formed once per block for all the lanes that read
// it, so the per-step work of a lane loses a multiply.
template <int TB, int W>
__device__ __forceinline__ void tile_mul_to_lds(const TileRegs<TB, W> &x, const TileRegs<TB, W> &y,
                                                float (*lds)[TB + kPad]) {
  TileRegs<TB, W> r;
#pragma unroll
  for (int i = 0; i < TileRegs<TB, W>::N; ++i) r.x[i] = x.x[i] * y.x[i];
  tile_to_lds<TB, W>(r, lds);
}

// 2 x of a staged tile (exact).
template <int TB, int W>
__device__ __forceinline__ void tile_twice_to_lds(const TileRegs<TB, W> &x, float (*lds)[TB + kPad]) {
  TileRegs<TB, W> r;
#pragma unroll
  for (int i = 0; i < TileRegs<TB, W>::N; ++i) r.x[i] = x.x[i] + x.x[i];
  tile_to_lds<TB, W>(r, lds);
}

// LDS [W][TB + 4] -> global rows `row0 + t * ld`, columns c < cols.
template <int TB, int W>
__device__ __forceinline__ void lds_to_global(const float (*lds)[TB + kPad], float *__restrict__ base, int64_t ld,
                                              int64_t rows, int64_t cols) {
  const int tid = static_cast<int>(threadIdx.x);
#pragma unroll
  for (int i = 0; i < TileRegs<TB, W>::N; ++i) {
    const int e = tid + i * kFusedThreads;
    const int t = e / W, c = e % W;
    if (e < TB * W && t < rows && c < cols) __builtin_nontemporal_store(lds[c][t], base + t * ld + c);
  }
}

// The same for P partial tiles [P][W][TB + 4] added in order p = 0, 1, ...
// (the per-wave sums of a channel that spans P waves; P = 1 is lds_to_global).
template <int TB, int W, int P>
__device__ __forceinline__ void parts_to_global(const float (*lds)[W][TB + kPad], float *__restrict__ base,
                                                int64_t ld, int64_t rows, int64_t cols) {
  const int tid = static_cast<int>(threadIdx.x);
#pragma unroll
  for (int i = 0; i < TileRegs<TB, W>::N; ++i) {
    const int e = tid + i * kFusedThreads;
    const int t = e / W, c = e % W;
    if (e < TB * W && t < rows && c < cols) {
      float x = lds[0][c][t];
#pragma unroll
      for (int p = 1; p < P; ++p) x += lds[p][c][t];
      __builtin_nontemporal_store(x, base + t * ld + c);
    }
  }
}

// ================================================================ forward

// torch's softplus (threshold 20), for the one-token decode step.
__device__ __forceinline__ float softplus_t(float x) { return x > 20.0f ? x : log1pf(expf(x)); }

// softplus(x) = max(x, 0) + log1p(e), e = exp(-|x|) in (0, 1], with log1p(e) =
// log(w) e / (w - 1), w = 1 + e rounded (and e itself where w rounds to 1): the
// log1p identity of Goldberg, "What every computer scientist should know about
// floating-point arithmetic" (1991), Theorem 4, accurate to a few ulp with the
// hardware exp2 / log2. Equals torch's x for x > 20 (the correction is below half
// an ulp of x there). Also returns e, from which sigmoid(x) follows.
__device__ __forceinline__ float softplus_fast(float x, float &e) {
  constexpr float kLog2e = 1.44269504088896340736f, kLn2 = 0.69314718055994530942f;
  e = __builtin_amdgcn_exp2f(-fabsf(x) * kLog2e);
  const float w = 1.0f + e;
  const float l = w == 1.0f ? e : (__builtin_amdgcn_logf(w) * kLn2) * (e * __builtin_amdgcn_rcpf(w - 1.0f));
  return fmaxf(x, 0.0f) + l;
}

// Lambda^v = 1 / min(softplus(x) + ov_min, ov_max) and the factor f with
// d log sigma^2 = g Lambda^2 f for the gradient g of Lambda^v: f = -sigmoid(x),
// or 0 where the clamp is active -- torch's derivatives of the reciprocal
// (-g r^2), of clamp_max (g where not above the maximum) and of softplus
// (g sigmoid(x), or g for x > 20, where sigmoid(x) rounds to 1 within 3e-9).
__device__ __forceinline__ float sensor_precision(float x, float ov_min, float ov_max, float *f = nullptr) {
  float e;
  const float obs = softplus_fast(x, e) + ov_min;
  if (f) {
    const float sig = (x >= 0.0f ? 1.0f : e) * __builtin_amdgcn_rcpf(1.0f + e);
    *f = obs > ov_max ? 0.0f : -sig;
  }
  return __builtin_amdgcn_rcpf(fminf(obs, ov_max));
}

// Sensor tile [TB, W] at `base` (row stride ld elements). bf16 elements are kept
// as raw bits in the low half of each register until widen_sensor, so no load
// has to complete before the tile is staged.
template <int TB, int W, bool BF16>
__device__ __forceinline__ void tile_load_sensor(TileRegs<TB, W> &r, const void *base, int64_t ld, int64_t rows,
                                                 int64_t cols) {
  if constexpr (!BF16) {
    tile_load<TB, W>(r, static_cast<const float *>(base), ld, rows, cols);
  } else {
    const uint16_t *p = static_cast<const uint16_t *>(base);
    const int tid = static_cast<int>(threadIdx.x);
#pragma unroll
    for (int i = 0; i < TileRegs<TB, W>::N; ++i) {
      const int e = tid + i * kFusedThreads;
      const int t = e / W, c = e % W;
      r.x[i] = __uint_as_float((e < TB * W && t < rows && c < cols)
                                   ? static_cast<uint32_t>(__builtin_nontemporal_load(p + t * ld + c))
                                   : 0u);
    }
  }
}

template <int TB, int W, bool BF16>
__device__ __forceinline__ void widen_sensor(TileRegs<TB, W> &r) {
  if constexpr (BF16) {
#pragma unroll
    for (int i = 0; i < TileRegs<TB, W>::N; ++i) r.x[i] = __uint_as_float(__float_as_uint(r.x[i]) << 16);
  }
}

// Element (row, column m0) of a sensor tensor.
template <bool BF16>
__device__ __forceinline__ const void *sensor_at(const void *base, int64_t row, int64_t m0, int64_t ld) {
  return static_cast<const char *>(base) + (row * ld + m0) * (BF16 ? 2 : 4);
}

// The sensor gradients of a flushed block from the per-(step, channel) sums over
// s of dr k (P) and d phi k^2 (Q): dv = Lambda P, d Lambda = Q + v P. Called with
// sum = P and pv = NULL for dv (scaled by lam), or with sum = Q and pv = P for
// d Lambda; with F, d Lambda is then carried to log sigma^2 (times lam^2 f).
// LDS [W][TB + 4] -> dense rows of a tensor of the sensor dtype.
// The sums come as P partial tiles (a channel spanning P waves), added in order.
template <int TB, int W, int P, bool BF16, bool F>
__device__ __forceinline__ void lds_to_global_sensor(const float (*sum)[W][TB + kPad], const float (*lam)[TB + kPad],
                                                     const float (*v)[TB + kPad], const float (*f)[TB + kPad],
                                                     void *base, int64_t ld, int64_t rows, int64_t cols,
                                                     const float (*pv)[W][TB + kPad] = nullptr) {
  const int tid = static_cast<int>(threadIdx.x);
  auto total = [&](const float (*x)[W][TB + kPad], int c, int t) {
    float a = x[0][c][t];
#pragma unroll
    for (int p = 1; p < P; ++p) a += x[p][c][t];
    return a;
  };
#pragma unroll
  for (int i = 0; i < (TB * W + kFusedThreads - 1) / kFusedThreads; ++i) {
    const int e = tid + i * kFusedThreads;
    const int t = e / W, c = e % W;
    if (e < TB * W && t < rows && c < cols) {
      float d;
      if (pv) {
        d = total(sum, c, t) + v[c][t] * total(pv, c, t);
      } else {
        d = lam[c][t] * total(sum, c, t);
      }
      if constexpr (F) {
        const float l = lam[c][t];
        d = d * (l * l) * f[c][t];
      }
      if constexpr (BF16)
        __builtin_nontemporal_store(from_f32<bf16_t>(d).bits, static_cast<uint16_t *>(base) + t * ld + c);
      else
        __builtin_nontemporal_store(d, static_cast<float *>(base) + t * ld + c);
    }
  }
}

// The precision tile as Lambda^v (formed in place when it holds log sigma^2);
// with f, also each element's log sigma^2 gradient factor, into f.
template <int TB, int W>
__device__ __forceinline__ void to_precision(TileRegs<TB, W> &r, const SensorIn &sn, TileRegs<TB, W> *f = nullptr) {
  if (!sn.log_var) return;
#pragma unroll
  for (int i = 0; i < TileRegs<TB, W>::N; ++i)
    r.x[i] = sensor_precision(r.x[i], sn.ov_min, sn.ov_max, f ? &f->x[i] : nullptr);
}

// VAR: y_var is produced (prm.yvar non-NULL); without it the variance read-out
// is skipped altogether.
// 8 to 32 lanes per channel, and 128 with bf16 sensors and no y_var (the
// training layer's case): held to three waves per SIMD (their registers fit 168
// with at most a few spilled words; measured at (4, 2048, 1024, 128) 1.08 ->
// 0.95 ms, while the fp32 y_var variant at 128 lost 2-3% to its spills).
template <int SP, bool PRIOR, bool BF16, bool VAR>
__global__ void __launch_bounds__(kFusedThreads)
    __attribute__((amdgpu_waves_per_eu((SP >= 8 && SP <= 32) || (SP == 128 && BF16 && !VAR && !PRIOR) ? 3 : 1)))
    fused_kla_fwd_kernel(FusedFwdParams prm, FusedGeom g) {
  constexpr int CH = kFusedThreads / SP;
  constexpr int WPC = waves_per_channel<SP>();
  constexpr int SG = lanes_in_wave<SP>();
  // Wide channels stage shorter blocks: the [SP, TB] k and q tiles fill the LDS.
  constexpr int TB = SP >= 128 ? kCkpt : kFusedTB;
  // s_sv holds v Lv (the information statistic's channel factor), s_l Lv.
  __shared__ __align__(16) float s_sv[2][CH][TB + kPad], s_l[2][CH][TB + kPad];
  // The [SP, TB] k and q tiles: double-buffered, except at 256 lanes per channel
  // (40 KiB a buffer), where one buffer and a barrier before it is refilled let
  // more than one workgroup share a CU.
  constexpr int KQB = SP >= 256 ? 1 : 2;
  __shared__ __align__(16) float s_k[KQB][SP][TB + kPad], s_q[KQB][SP][TB + kPad];
  // k^2 staged beside k up to 64 lanes per channel (wider channels square k per
  // step: their k tiles already fill the LDS).
  constexpr bool kK2 = SP <= kWave;
  __shared__ __align__(16) float s_k2[kK2 ? KQB : 1][kK2 ? SP : 1][TB + kPad];
  __shared__ float s_y[2][WPC][CH][TB + kPad], s_yv[2][WPC][CH][TB + kPad];

  const FusedLane ln = fused_lane<SP>(g);
  const int64_t M = g.M, S = g.S, L = g.steps;
  const int64_t m0 = (xcd_block() % g.groups) * CH;
  const int c = static_cast<int>(ln.m - m0);
  const int64_t ms = ln.m * S + ln.s;
  const int64_t bms = ln.b * M * S + ms;
  const int64_t cols_m = M - m0 < CH ? M - m0 : CH;
  const int lane = static_cast<int>(threadIdx.x) % kWave;

  const float a_s = ln.active ? prm.a[ms] : 1.0f;
  const float pp = fmaxf(ln.active ? prm.p[ms] : 0.0f, kEps);
  const A2 a2 = split_a2(a_s);
  float lam = (ln.active && prm.lam0) ? prm.lam0[bms] : 1.0f;
  float eta = (ln.active && prm.eta0) ? prm.eta0[bms] : 0.0f;

  const SensorIn &sn = prm.sn;
  const float *kbase = prm.k + ln.b * L * S;
  const float *qbase = prm.q + ln.b * L * S;
  float *ybase = prm.y + ln.b * L * M + m0;
  float *yvbase = VAR ? prm.yvar + ln.b * L * M + m0 : nullptr;

  TileRegs<TB, CH> rv, rl;
  TileRegs<TB, SP> rk, rq;
  auto load = [&](int64_t t0) {
    const int64_t rows = L - t0;
    tile_load_sensor<TB, CH, BF16>(rv, sensor_at<BF16>(sn.v, ln.b * L + t0, m0, sn.ld_v), sn.ld_v, rows, cols_m);
    tile_load_sensor<TB, CH, BF16>(rl, sensor_at<BF16>(sn.lv, ln.b * L + t0, m0, sn.ld_lv), sn.ld_lv, rows, cols_m);
    tile_load<TB, SP>(rk, kbase + t0 * S, S, rows, S);
    tile_load<TB, SP>(rq, qbase + t0 * S, S, rows, S);
  };
  auto stage = [&](int buf) {
    widen_sensor<TB, CH, BF16>(rv);
    widen_sensor<TB, CH, BF16>(rl);
    to_precision<TB, CH>(rl, sn);
    tile_mul_to_lds<TB, CH>(rv, rl, s_sv[buf]);
    tile_to_lds<TB, CH>(rl, s_l[buf]);
    tile_to_lds<TB, SP>(rk, s_k[KQB == 1 ? 0 : buf]);
    if constexpr (kK2) tile_mul_to_lds<TB, SP>(rk, rk, s_k2[KQB == 1 ? 0 : buf]);
    tile_to_lds<TB, SP>(rq, s_q[KQB == 1 ? 0 : buf]);
  };

  // Checkpoint of the state entering step t: ck[((b * n_ck + t / kCkpt) * M + m) * S + s].
  const int64_t ck_off = (ln.b * g.n_ck * M + ln.m) * S + ln.s;
  const int64_t ck_stride = M * S;
  static_assert(TB % kCkpt == 0, "checkpoints must fall on half-block boundaries");

  const int64_t nblk = (L + TB - 1) / TB;
  if (nblk > 0) {
    load(0);
    stage(0);
  }
  __syncthreads();
  for (int64_t blk = 0; blk < nblk; ++blk) {
    const int cur = static_cast<int>(blk & 1);
    const int64_t t0 = blk * TB;
    if (blk + 1 < nblk) load(t0 + TB);
    if (blk > 0) {
      parts_to_global<TB, CH, WPC>(s_y[cur ^ 1], ybase + (t0 - TB) * M, M, TB, cols_m);
      if constexpr (VAR) parts_to_global<TB, CH, WPC>(s_yv[cur ^ 1], yvbase + (t0 - TB) * M, M, TB, cols_m);
    }
    // The read-out terms of a kCkpt-step half of the block, summed over s after
    // the half (step_sums_to_lds).
    float yw[kCkpt], vw[kCkpt];
    constexpr bool kVecLds = SP >= 16;
    // One step at block position j (position jj within its half); with x4, the
    // step's tile values come from four-step LDS reads.
    float4 l4{}, v4{}, k4{}, q4{}, k24{};
    auto step = [&](int j, int jj, bool x4) {
      const int kb = KQB == 1 ? 0 : cur;
      const float sig = x4 ? pick4(l4, j % 4) : s_l[cur][c][j];
      const float sv = x4 ? pick4(v4, j % 4) : s_sv[cur][c][j];
      const float kk = x4 ? pick4(k4, j % 4) : s_k[kb][ln.s][j];
      const float k2 = !kK2 ? kk * kk : x4 ? pick4(k24, j % 4) : s_k2[kK2 ? kb : 0][kK2 ? ln.s : 0][j];
      float idn_a;
      lam = filter_step(lam, eta, sig * k2, sv * kk, a_s, a2, pp, idn_a);
      const float var = rcp(fmaxf(lam, kEps));
      float mean = eta * var, vo = var;
      if (PRIOR) {
        mean = a_s * mean;
        vo = a2.hi * var + pp;
      }
      const float qq = x4 ? pick4(q4, j % 4) : s_q[KQB == 1 ? 0 : cur][ln.s][j];
      yw[jj] = qq * mean;
      if constexpr (VAR) vw[jj] = (qq * qq) * vo;
    };
    // Checkpoints enter every kCkpt-step half of the block (TB is a multiple of kCkpt).
#pragma unroll
    for (int h = 0; h < TB / kCkpt; ++h) {
      const int64_t th = t0 + h * kCkpt;
      if (th < L) {
        if (prm.ck_lam && ln.active) {
          prm.ck_lam[ck_off + (th / kCkpt) * ck_stride] = lam;
          prm.ck_eta[ck_off + (th / kCkpt) * ck_stride] = eta;
        }
        if (th + kCkpt <= L) {
          // The whole half lies inside the sequence: no per-step bound. Four-step
          // LDS reads are issued two steps ahead of their first step.
          float4 nl4{}, nv4{}, nk4{}, nk24{}, nq4{};
          auto read4 = [&](int jb, float4 &l, float4 &v, float4 &k, float4 &k2, float4 &q) {
            asm volatile("" ::: "memory");
            l = lds4(s_l[cur][c], jb);
            v = lds4(s_sv[cur][c], jb);
            k = lds4(s_k[KQB == 1 ? 0 : cur][ln.s], jb);
            if constexpr (kK2) k2 = lds4(s_k2[kK2 && KQB == 2 ? cur : 0][kK2 ? ln.s : 0], jb);
            q = lds4(s_q[KQB == 1 ? 0 : cur][ln.s], jb);
            asm volatile("" ::: "memory");
          };
          if (kVecLds) read4(h * kCkpt, l4, v4, k4, k24, q4);
#pragma unroll
          for (int j = 0; j < kCkpt; ++j) {
            const int jb = h * kCkpt + j;
            if (kVecLds && j % 4 == 0 && j > 0) {
              l4 = nl4;
              v4 = nv4;
              k4 = nk4;
              k24 = nk24;
              q4 = nq4;
            }
            if (kVecLds && j % 4 == 2 && j + 2 < kCkpt) read4(jb + 2, nl4, nv4, nk4, nk24, nq4);
            step(jb, j, kVecLds);
          }
        } else {
          // Unrolled: the terms live in registers indexed by j.
#pragma unroll
          for (int j = 0; j < kCkpt; ++j) {
            if (th + j < L) {
              step(h * kCkpt + j, j, false);
            } else {
              yw[j] = 0.0f;
              if constexpr (VAR) vw[j] = 0.0f;
            }
          }
        }
        step_sums_to_lds<SP>(yw, lane, ln.s, s_y[cur][ln.s / SG][c], h * kCkpt);
        if constexpr (VAR) step_sums_to_lds<SP>(vw, lane, ln.s, s_yv[cur][ln.s / SG][c], h * kCkpt);
      }
    }
    if (blk + 1 < nblk) {
      if constexpr (KQB == 1) __syncthreads();   // every wave is done with this block's k, q
      stage(cur ^ 1);
    }
    __syncthreads();
  }
  if (nblk > 0) {
    const int last = static_cast<int>((nblk - 1) & 1);
    const int64_t t0 = (nblk - 1) * TB;
    parts_to_global<TB, CH, WPC>(s_y[last], ybase + t0 * M, M, L - t0, cols_m);
    if constexpr (VAR) parts_to_global<TB, CH, WPC>(s_yv[last], yvbase + t0 * M, M, L - t0, cols_m);
  }
  if (ln.active) {
    prm.lam_fin[bms] = lam;
    prm.eta_fin[bms] = eta;
  }
}

// ================================================================ backward

// VAR: a y_var gradient is given (prm.dyvar non-NULL); without it the
// variance read-out's adjoint is skipped (a zero gradient).
template <int SP, bool PRIOR, bool BF16, bool VAR>
__global__ void __launch_bounds__(kFusedThreads) __attribute__((amdgpu_waves_per_eu(SP >= 8 ? 2 : 1)))
    fused_kla_bwd_kernel(FusedBwdParams prm, FusedGeom g) {
  constexpr int CH = kFusedThreads / SP;
  constexpr int NW = kFusedThreads / kWave;
  constexpr int WPC = waves_per_channel<SP>();
  constexpr int SG = lanes_in_wave<SP>();
  constexpr int TB = kCkpt;
  __shared__ __align__(16) float s_v[2][CH][TB + kPad], s_l[2][CH][TB + kPad];
  __shared__ __align__(16) float s_dy[2][CH][TB + kPad], s_dyv[2][CH][TB + kPad];
  // The [SP, TB] k and q tiles: double-buffered, except at 256 lanes per channel
  // (40 KiB a buffer), where one buffer and a barrier before it is refilled let
  // more than one workgroup share a CU.
  constexpr int KQB = SP >= 256 ? 1 : 2;
  __shared__ __align__(16) float s_k[KQB][SP][TB + kPad], s_q[KQB][SP][TB + kPad];
  __shared__ float s_dv[2][WPC][CH][TB + kPad], s_dl[2][WPC][CH][TB + kPad];
  __shared__ float s_lf[2][CH][TB + kPad];   // log sigma^2 gradient factors (log_var sensors)
  // Per-block products of the staged tiles: v Lv and 2 Lv per channel, k^2 per
  // state lane (up to 64 lanes per channel; wider channels square k per step).
  // At 4 lanes per channel (64 channels a workgroup) 2 Lv is formed per step
  // instead, which keeps the LDS at two workgroups per CU.
  constexpr bool kK2 = SP <= kWave;
  constexpr bool kS2 = SP >= 8;
  __shared__ __align__(16) float s_sv[2][CH][TB + kPad], s_s2[kS2 ? 2 : 1][kS2 ? CH : 1][TB + kPad];
  __shared__ __align__(16) float s_k2[kK2 ? KQB : 1][kK2 ? SP : 1][TB + kPad];
  // Per-(step, s) sums of a channel slot, double-buffered like the tiles where
  // it is small; from 64 lanes per channel on (64 KiB a buffer) one buffer and a
  // barrier between the flush that reads it and the walk that refills it, which
  // halves the backward's LDS and lets two workgroups share a CU.
  constexpr int RB = SP >= kWave ? 1 : 2;
  __shared__ float s_red[RB][2][TB][NW / WPC][SP];
  // Blocks wholly inside the sequence run as one straight block of code (no
  // per-step bound) where that code still fits two waves per SIMD without
  // spills; elsewhere (4, 8, 128 or 256 lanes per channel, the prior's
  // read-out, the variance's adjoint) every block keeps the per-step bound.
  constexpr bool kFullBlocks = SP >= 16 && SP <= 64 && !PRIOR && !VAR;

  const FusedLane ln = fused_lane<SP>(g);
  const int64_t M = g.M, S = g.S, L = g.steps;
  const int64_t grp = xcd_block() % g.groups;
  const int64_t m0 = grp * CH;
  const int c = static_cast<int>(ln.m - m0);
  const int64_t ms = ln.m * S + ln.s;
  const int64_t bms = ln.b * M * S + ms;
  const int64_t cols_m = M - m0 < CH ? M - m0 : CH;
  const int tid = static_cast<int>(threadIdx.x);
  const int wave = tid / kWave, lane = tid % kWave;

  const float a_s = ln.active ? prm.a[ms] : 1.0f;
  const float p_raw = ln.active ? prm.p[ms] : 0.0f;
  const float pp = fmaxf(p_raw, kEps);
  const A2 a2s = split_a2(a_s);
  const float a2 = a2s.hi;
  const float inv_a2 = 1.0f / a2;

  float gl = (ln.active && prm.dlam_fin) ? prm.dlam_fin[bms] : 0.0f;   // adjoint of lam_t
  float ge = (ln.active && prm.deta_fin) ? prm.deta_fin[bms] : 0.0f;   // adjoint of eta_t
  float acc_a = 0.0f, acc_a2 = 0.0f, acc_p = 0.0f;

  const int64_t offM = ln.b * L * M + m0, offS = ln.b * L * S;
  const SensorIn &sn = prm.sn;
  TileRegs<TB, CH> rv, rl, rdy, rdyv;
  TileRegs<TB, SP> rk, rq;
  auto load = [&](int64_t t0) {
    const int64_t rows = L - t0;
    tile_load_sensor<TB, CH, BF16>(rv, sensor_at<BF16>(sn.v, ln.b * L + t0, m0, sn.ld_v), sn.ld_v, rows, cols_m);
    tile_load_sensor<TB, CH, BF16>(rl, sensor_at<BF16>(sn.lv, ln.b * L + t0, m0, sn.ld_lv), sn.ld_lv, rows, cols_m);
    tile_load<TB, CH>(rdy, prm.dy + offM + t0 * M, M, rows, cols_m);
    if constexpr (VAR) tile_load<TB, CH>(rdyv, prm.dyvar + offM + t0 * M, M, rows, cols_m);
    tile_load<TB, SP>(rk, prm.k + offS + t0 * S, S, rows, S);
    tile_load<TB, SP>(rq, prm.q + offS + t0 * S, S, rows, S);
  };
  auto stage = [&](int buf) {
    widen_sensor<TB, CH, BF16>(rv);
    widen_sensor<TB, CH, BF16>(rl);
    tile_to_lds<TB, CH>(rv, s_v[buf]);
    if (sn.log_var) {
      TileRegs<TB, CH> rf;
      to_precision<TB, CH>(rl, sn, &rf);
      tile_to_lds<TB, CH>(rf, s_lf[buf]);
    }
    tile_to_lds<TB, CH>(rl, s_l[buf]);
    tile_mul_to_lds<TB, CH>(rv, rl, s_sv[buf]);
    if constexpr (kS2) tile_twice_to_lds<TB, CH>(rl, s_s2[kS2 ? buf : 0]);
    tile_to_lds<TB, CH>(rdy, s_dy[buf]);
    if constexpr (VAR) tile_to_lds<TB, CH>(rdyv, s_dyv[buf]);
    tile_to_lds<TB, SP>(rk, s_k[KQB == 1 ? 0 : buf]);
    if constexpr (kK2) tile_mul_to_lds<TB, SP>(rk, rk, s_k2[KQB == 1 ? 0 : buf]);
    tile_to_lds<TB, SP>(rq, s_q[KQB == 1 ? 0 : buf]);
  };
  // Outputs of block c (buffer `buf`): dv, dLv rows, and the workgroup's
  // partial sums of dk, dq (the waves' sums added here, in wave order).
  auto flush = [&](int64_t blk, int buf) {
    const int64_t t0 = blk * TB;
    constexpr int64_t el = BF16 ? 2 : 4;
    void *dvb = static_cast<char *>(prm.dv) + (offM + t0 * M) * el;
    void *dlb = static_cast<char *>(prm.dlv) + (offM + t0 * M) * el;
    // Every pointer argument is an LDS tile, also where a call does not read it:
    // the two dLv calls share code after inlining, and a null among the pointers
    // there would turn the LDS reads into flat loads, whose wait would cover the
    // next block's tile loads still in flight.
    lds_to_global_sensor<TB, CH, WPC, BF16, false>(s_dv[buf], s_l[buf], s_v[buf], s_lf[buf], dvb, M, L - t0, cols_m);
    if (sn.log_var)
      lds_to_global_sensor<TB, CH, WPC, BF16, true>(s_dl[buf], s_l[buf], s_v[buf], s_lf[buf], dlb, M, L - t0,
                                                    cols_m, s_dv[buf]);
    else
      lds_to_global_sensor<TB, CH, WPC, BF16, false>(s_dl[buf], s_l[buf], s_v[buf], s_lf[buf], dlb, M, L - t0,
                                                     cols_m, s_dv[buf]);
    for (int i = tid; i < 2 * TB * SP; i += kFusedThreads) {
      const int which = i / (TB * SP);
      const int j = (i / SP) % TB;
      const int s = i % SP;
      const int64_t t = t0 + j;
      if (t < L && s < S) {
        float sum = 0.0f;
#pragma unroll
        for (int w = 0; w < NW / WPC; ++w) sum += s_red[RB == 1 ? 0 : buf][which][j][w][s];
        float *part = which == 0 ? prm.part_k : prm.part_q;
        part[((ln.b * L + t) * g.groups + grp) * S + s] = sum;
      }
    }
  };

  const int64_t n_ck = g.n_ck;
  // The checkpoint entering a block is read one block ahead, with the block's
  // tiles: a load issued just before the replay would make the replay wait for
  // every load still in flight (memory counters retire in order), the next
  // block's tiles included.
  float ck_l = 1.0f, ck_e = 0.0f;
  auto load_ck = [&](int64_t blk) {
    if (ln.active) {
      const int64_t ci = ((ln.b * n_ck + blk) * M + ln.m) * S + ln.s;
      ck_l = prm.ck_lam[ci];
      ck_e = prm.ck_eta[ci];
    }
  };
  if (n_ck > 0) {
    load((n_ck - 1) * TB);
    load_ck(n_ck - 1);
    stage(0);
  }
  __syncthreads();
  for (int64_t i = 0; i < n_ck; ++i) {
    const int cur = static_cast<int>(i & 1);
    const int64_t blk = n_ck - 1 - i;
    const int64_t t0 = blk * TB;
    const float lam_ck = ck_l, eta_ck = ck_e;
    if (i + 1 < n_ck) {
      load(t0 - TB);
      load_ck(blk - 1);
    }
    if (i > 0) {
      flush(blk + 1, cur ^ 1);
      if constexpr (RB == 1) __syncthreads();   // the flush has read s_red before the walk refills it
    }

    // Tile values four steps per LDS read, where the registers that hold them
    // do not cost occupancy (16 or more lanes per channel).
    constexpr bool kVecLds = SP >= 16;
    // Steps of this block inside the sequence, as a 32-bit count: the per-step
    // bound is then a scalar compare (there is no 64-bit scalar less-than).
    const int nv = static_cast<int>(L - t0 < TB ? L - t0 : TB);
    // Over the block: lam_{t-1}, eta_{t-1} (lh[TB], eh[TB]: the state after the
    // block), and each step's 1/(a2 den), kept from the replay (the posterior
    // variance 1/lam_t is formed again in the walk: 16 registers fewer).
    float lh[TB + 1], eh[TB + 1], idn[TB];
    // da, dp sum over all steps: accumulate each block apart and add the block
    // totals (two-level summation keeps fp32 rounding at ~(TB + L/TB) ulp).
    // The terms through A = (1 + p' phi)/a2 and C = p'/a2 are gathered as
    // X = sum (dA phi + dC) and Y = sum dA and applied once per block:
    // dp += X/a2, d(a2) -= (Y + p' X)/a2^2.
    float blk_a = 0.0f, blk_a2 = 0.0f, blk_p = 0.0f, blk_x = 0.0f, blk_y = 0.0f;
    const int kb = KQB == 1 ? 0 : cur;
    // Whether no clamp acts in the block: every lam of the block (the checkpoint
    // and each step's lam_t) >= EPS. Then var = 1/lam_t has its plain derivative,
    // and lam' >= 0 makes a2 + p' lam' >= a2 >= EPS, so alpha's clamp is idle too.
    bool unclamped = true;
    // The replay from the block's checkpoint. FULL: every step of the block lies
    // inside the sequence (all blocks but the sequence's last partial one), so
    // the steps need no bound and the block is one straight run of code.
    auto replay = [&](auto full_c) __attribute__((always_inline)) {
      constexpr bool FULL = decltype(full_c)::value;
      float lam = lam_ck;
      float eta = eta_ck;
      unclamped = lam >= kEps;
      // Tile values of four steps per LDS read, issued two steps before the
      // first of them (the last two values of the group in use are dead by
      // then), so that less of the reads' latency is waited for. (Compiler
      // barriers around the reads: hoisted further, they would hold more
      // registers than two waves per SIMD allow.)
      float4 l4{}, v4{}, k4{}, k24{}, nl4{}, nv4{}, nk4{}, nk24{};
      auto read4 = [&](int j, float4 &l, float4 &v, float4 &k, float4 &k2) {
        asm volatile("" ::: "memory");
        l = lds4(s_l[cur][c], j);
        v = lds4(s_sv[cur][c], j);
        k = lds4(s_k[kb][ln.s], j);
        if constexpr (kK2) k2 = lds4(s_k2[kK2 ? kb : 0][kK2 ? ln.s : 0], j);
        asm volatile("" ::: "memory");
      };
      if (kVecLds) read4(0, l4, v4, k4, k24);
#pragma unroll
      for (int j = 0; j < TB; ++j) {
        if (kVecLds && j % 4 == 0 && j > 0) {
          l4 = nl4;
          v4 = nv4;
          k4 = nk4;
          k24 = nk24;
        }
        if (kVecLds && j % 4 == 2 && j + 2 < TB) read4(j + 2, nl4, nv4, nk4, nk24);
        lh[j] = lam;
        eh[j] = eta;
        if (!FULL) idn[j] = 0.0f;
        if (FULL || j < nv) {
          const float sig = kVecLds ? pick4(l4, j % 4) : s_l[cur][c][j];
          const float sv = kVecLds ? pick4(v4, j % 4) : s_sv[cur][c][j];
          const float kk = kVecLds ? pick4(k4, j % 4) : s_k[kb][ln.s][j];
          const float k2 = !kK2 ? kk * kk : kVecLds ? pick4(k24, j % 4) : s_k2[kK2 ? kb : 0][kK2 ? ln.s : 0][j];
          lam = filter_step(lam, eta, sig * k2, sv * kk, a_s, a2s, pp, idn[j]);
          if (FULL) unclamped = unclamped && lam >= kEps;
        }
      }
      lh[TB] = lam;
      eh[TB] = eta;
    };
    // dv, dLv contributions of the block's steps, summed over s after the walk
    // (step_sums_to_lds: within the wave; from 128 lanes per channel each wave
    // writes its partial slot, which the flush adds in wave order).
    float dv_w[TB], dl_w[TB];
    // dk, dq contributions, summed over the wave's four channel rows after the
    // walk (cross_row_transpose_sum) when SP = 16.
    constexpr bool kRows = SP == 16;
    float dk_w[kRows ? TB : 1], dq_w[kRows ? TB : 1];
    // The adjoint walk over the block. CLAMPS: with the clamps' branches (the
    // general case); without, for a block where no clamp acts (the same values).
    // FULL as for the replay.
    // No implicit contraction in the walk: every fused multiply-add is written
    // as fmaf, so the four copies (with or without clamps, guarded or full)
    // round alike wherever their code differs only by a select or a branch.
    auto walk = [&](auto clamps_c, auto full_c) __attribute__((always_inline)) {
#pragma clang fp contract(off)
      constexpr bool CLAMPS = decltype(clamps_c)::value;
      constexpr bool FULL = decltype(full_c)::value;
      // (Four-step LDS reads issued two steps ahead, as in the replay.)
      float4 sv4{}, s24{}, dy4{}, k4{}, q4{}, nsv4{}, ns24{}, ndy4{}, nk4{}, nq4{};
      auto read4 = [&](int j0, float4 &sv, float4 &s2, float4 &dy, float4 &k, float4 &q) {
        asm volatile("" ::: "memory");
        sv = lds4(s_sv[cur][c], j0);
        if constexpr (kS2) s2 = lds4(s_s2[kS2 ? cur : 0][kS2 ? c : 0], j0);
        dy = lds4(s_dy[cur][c], j0);
        k = lds4(s_k[kb][ln.s], j0);
        q = lds4(s_q[kb][ln.s], j0);
        asm volatile("" ::: "memory");
      };
      if (kVecLds) read4(TB - 4, sv4, s24, dy4, k4, q4);
#pragma unroll
      for (int j = TB - 1; j >= 0; --j) {
        if (kVecLds && j % 4 == 3 && j < TB - 1) {
          sv4 = nsv4;
          s24 = ns24;
          dy4 = ndy4;
          k4 = nk4;
          q4 = nq4;
        }
        if (kVecLds && j % 4 == 1 && j >= 4) read4(j - 5, nsv4, ns24, ndy4, nk4, nq4);
        float dk_c = 0.0f, dq_c = 0.0f;
        if constexpr (!FULL) {
          dv_w[j] = 0.0f;
          dl_w[j] = 0.0f;
        }
        if (FULL || j < nv) {
          const float sv = kVecLds ? pick4(sv4, j % 4) : s_sv[cur][c][j];
          const float s2 = !kS2 ? 2.0f * s_l[cur][c][j] : kVecLds ? pick4(s24, j % 4) : s_s2[kS2 ? cur : 0][kS2 ? c : 0][j];
          const float dy = kVecLds ? pick4(dy4, j % 4) : s_dy[cur][c][j];
          const float kk = kVecLds ? pick4(k4, j % 4) : s_k[kb][ln.s][j];
          const float qq = kVecLds ? pick4(q4, j % 4) : s_q[kb][ln.s][j];
          const float lp = lh[j], ep = eh[j];
          const float lam_t = lh[j + 1], eta_t = eh[j + 1];
          const float idn_a = idn[j], var = rcp(CLAMPS ? fmaxf(lam_t, kEps) : lam_t);
          // The step's intermediates (filter_step) from the kept 1/(a2 den):
          // 1/den = a2 idn_a, and d lam_t / d lam' = 1/(a2 den^2) = idn_a / den.
          const float inv_den = inv_den_from(a2s, idn_a);
          // alpha = a / max(a2 + p' lam', EPS) = a min(idn_a, 1/EPS)
          const bool da_ok = !CLAMPS || idn_a <= kInvEps;
          const float inv_Da = CLAMPS ? fminf(idn_a, kInvEps) : idn_a;
          const float alpha = a_s * inv_Da;
          const float mean = eta_t * var;
          const float mean_o = PRIOR ? a_s * mean : mean;
          const float var_o = PRIOR ? fmaf(a2, var, pp) : var;

          // read-out
          const float dmo = dy * qq;
          float dmean = dmo;
          if (PRIOR) {
            dmean = dmo * a_s;
            blk_a = fmaf(dmo, mean, blk_a);
          }
          // t = d(loss)/d(var) var = (dvar + dmean eta_t) var = dvar var + dmean mean.
          float t;
          if constexpr (VAR) {
            const float dyv = s_dyv[cur][c][j];
            const float dvo = dyv * (qq * qq);
            dq_c = fmaf(dy, mean_o, ((dyv * 2.0f) * qq) * var_o);
            float dvar = dvo;
            if (PRIOR) {
              dvar = dvo * a2;
              blk_a2 = fmaf(dvo, var, blk_a2);
              blk_p += dvo;
            }
            t = fmaf(dmean, mean, dvar * var);
          } else {
            dq_c = dy * mean_o;
            t = dmean * mean;
          }
          // mean = eta var, var = 1/max(lam, EPS): d lam = -d(var) var^2 = -t var
          const float ge_t = fmaf(dmean, var, ge);
          float gl_t = fmaf(-t, var, gl);
          if constexpr (CLAMPS) gl_t = lam_t >= kEps ? gl_t : gl;
          // eta_t = alpha eta' + r
          const float dalpha = ge_t * ep;
          ge = ge_t * alpha;
          // alpha = a / Da, Da = max(a2 + p' lam', EPS): d a += dalpha / Da, d Da = -dalpha alpha / Da
          const float w = dalpha * inv_Da;
          blk_a += w;
          float dDa = -(w * alpha);
          if constexpr (CLAMPS) dDa = da_ok ? dDa : 0.0f;
          blk_a2 += dDa;
          blk_p = fmaf(dDa, lp, blk_p);
          // lam_t = (A lam' + phi) / den, den = C lam' + 1: dA = u lam', dC = -u lam_t lam'
          const float u = gl_t * inv_den;
          const float dA = u * lp;
          // (Explicit fmaf where a sum of two products could be contracted either
          // way, so every kernel variant rounds alike.)
          blk_x = fmaf(-dA, lp * idn_a, blk_x);   // dA phi + dC = dA (phi - lam_t), lam_t - phi = lam' idn_a
          blk_y += dA;
          gl = fmaf(u, idn_a, dDa * pp);
          // phi = Lv k^2, r = (v Lv) k, d phi = gl_t (d lam_t / d phi = 1), d r = ge_t.
          // Per lane the s-sums need only dr k and d phi k^2: dv = Lv sum(dr k),
          // dLv = sum(d phi k^2) + v sum(dr k), formed once per (step, channel)
          // when the block is flushed; d k = 2 Lv k d phi + (v Lv) d r.
          const float pk = ge_t * kk;
          const float gk = gl_t * kk;
          const float qk = gk * kk;
          dk_c = fmaf(gk, s2, ge_t * sv);
          dv_w[j] = pk;
          dl_w[j] = qk;
        }
        // Sum over this wave's channels (now, or after the walk), over the waves
        // at the flush.
        if constexpr (kRows) {
          dk_w[j] = dk_c;
          dq_w[j] = dq_c;
        } else {
          // (For SP >= 64 a wave holds one channel's lanes or part of them:
          // nothing to add within the wave, and every lane stores its s.)
          dk_c = cross_group_sum<SP>(dk_c);
          dq_c = cross_group_sum<SP>(dq_c);
          if (SP >= kWave || lane < SP) {
            s_red[RB == 1 ? 0 : cur][0][j][wave / WPC][ln.s] = dk_c;
            s_red[RB == 1 ? 0 : cur][1][j][wave / WPC][ln.s] = dq_c;
          }
        }
      }
    };
    // (Wave-uniform branches: neither the replay nor the walk holds a barrier.)
    if (kFullBlocks && nv == TB) {
      replay(std::true_type{});
      if (__all(unclamped))
        walk(std::false_type{}, std::true_type{});
      else
        walk(std::true_type{}, std::true_type{});
    } else {
      replay(std::false_type{});
      walk(std::true_type{}, std::false_type{});
    }
    if constexpr (kRows) {
      cross_row_transpose_sum<TB>(dk_w);
      cross_row_transpose_sum<TB>(dq_w);
      const int row = lane / 16;
#pragma unroll
      for (int i = 0; i < TB / 4; ++i) {
        const int j = (TB / 2) * (row >> 1) + (TB / 4) * (row & 1) + i;
        s_red[RB == 1 ? 0 : cur][0][j][wave][ln.s] = dk_w[i];
        s_red[RB == 1 ? 0 : cur][1][j][wave][ln.s] = dq_w[i];
      }
    }
    step_sums_to_lds<SP>(dv_w, lane, ln.s, s_dv[cur][ln.s / SG][c], 0);
    step_sums_to_lds<SP>(dl_w, lane, ln.s, s_dl[cur][ln.s / SG][c], 0);
    acc_a += blk_a;
    acc_a2 += fmaf(-fmaf(pp, blk_x, blk_y), inv_a2 * inv_a2, blk_a2);
    acc_p += fmaf(blk_x, inv_a2, blk_p);
    if (i + 1 < n_ck) {
      if constexpr (KQB == 1) __syncthreads();   // every wave is done with this block's k, q
      stage(cur ^ 1);
    }
    __syncthreads();
  }
  if (n_ck > 0) flush(0, static_cast<int>((n_ck - 1) & 1));

  if (ln.active) {
    if (prm.dlam0) prm.dlam0[bms] = gl;
    if (prm.deta0) prm.deta0[bms] = ge;
    const float da2_da = (a_s * a_s >= kEps) ? 2.0f * a_s : 0.0f;
    prm.part_a[bms] = acc_a + acc_a2 * da2_da;
    prm.part_p[bms] = (p_raw >= kEps) ? acc_p : 0.0f;
  }
}

// out[o * inner + i] = sum_{j < G} in[(o * G + j) * inner + i], for o < outer, i < inner.
// out[o, i] = sum_j in[o, j, i] over G rows for INNER columns (a power of two
// dividing 256): one 256-thread block per o reads the row block [G, INNER]
// with consecutive threads on consecutive floats, each thread sums every
// (256 / INNER)-th row of its column, and a fixed-order LDS tree adds those
// partials -- deterministic, and at streaming speed where reduce_groups_kernel's
// one-thread-per-output loop is latency-bound.
template <int INNER>
__global__ void __launch_bounds__(256) reduce_rows_kernel(const float *__restrict__ in, float *__restrict__ out,
                                                          int64_t G) {
  static_assert(INNER >= 1 && INNER <= 256 && 256 % INNER == 0, "INNER must divide 256");
  constexpr int R = 256 / INNER;
  __shared__ float sm[256];
  const int t = static_cast<int>(threadIdx.x);
  const int i = t % INNER, r = t / INNER;
  const float *src = in + static_cast<int64_t>(blockIdx.x) * G * INNER + i;
  float acc = 0.0f;
  for (int64_t j = r; j < G; j += R) acc += src[j * INNER];
  sm[t] = acc;
  __syncthreads();
#pragma unroll
  for (int step = R / 2; step > 0; step /= 2) {
    if (r < step) sm[t] += sm[t + step * INNER];
    __syncthreads();
  }
  if (r == 0) out[static_cast<int64_t>(blockIdx.x) * INNER + i] = sm[i];
}

// The sums of reduce_rows_kernel<INNER>, bit for bit, for INNER >= 4: one wave
// per row block o and 16-byte loads. Lane l sums columns 4 (l % Q) .. + 3
// (Q = INNER / 4 lanes per row) over the rows j = r, r + R, ... of its phase
// r = l / Q (R = 64 / Q = 256 / INNER phases, as there), then the phases are
// added pairwise R/2 apart, R/4 apart, ... -- the same additions in the same
// order -- over lanes by shuffles, with no LDS and no barrier.
template <int INNER>
__global__ void __launch_bounds__(256) reduce_rows_wave_kernel(const float *__restrict__ in, float *__restrict__ out,
                                                               int64_t outer, int64_t G) {
  static_assert(INNER >= 4 && INNER <= 256 && 256 % INNER == 0, "INNER must be 4 to 256, a power of two");
  constexpr int Q = INNER / 4;
  constexpr int R = kWave / Q;
  typedef float f32x4v __attribute__((ext_vector_type(4)));
  const int lane = static_cast<int>(threadIdx.x) % kWave;
  const int64_t o = static_cast<int64_t>(blockIdx.x) * (256 / kWave) + threadIdx.x / kWave;
  if (o >= outer) return;   // whole waves leave together
  const int q = lane % Q, r = lane / Q;
  const f32x4v *src = reinterpret_cast<const f32x4v *>(in + o * G * INNER) + q;
  f32x4v acc = {0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll 4
  for (int64_t j = r; j < G; j += R) acc += src[j * Q];
#pragma unroll
  for (int off = kWave / 2; off >= Q; off /= 2) {
    acc.x += __shfl_xor(acc.x, off);
    acc.y += __shfl_xor(acc.y, off);
    acc.z += __shfl_xor(acc.z, off);
    acc.w += __shfl_xor(acc.w, off);
  }
  if (r == 0) *reinterpret_cast<f32x4v *>(out + o * INNER + 4 * q) = acc;
}

// out[i] = sum_j in[j, i] over G rows (outer = 1): a 1024-thread block covers 64
// columns with 16 row phases, each thread summing every 16th row of its column
// (coalesced across the 64 columns), then a fixed-order LDS tree adds the 16
// phase sums. Deterministic; parallel over rows as well as columns.
__global__ void __launch_bounds__(1024) reduce_cols_kernel(const float *__restrict__ in, float *__restrict__ out,
                                                           int64_t G, int64_t inner) {
  constexpr int COLS = 64, PH = 16;
  __shared__ float sm[PH][COLS];
  const int t = static_cast<int>(threadIdx.x);
  const int c = t % COLS, ph = t / COLS;
  const int64_t col = static_cast<int64_t>(blockIdx.x) * COLS + c;
  float acc = 0.0f;
  // Unrolled so that several independent loads are in flight before the
  // (in-order) additions: a few columns over many rows is otherwise a chain of
  // cache latencies.
  if (col < inner) {
#pragma unroll 8
    for (int64_t j = ph; j < G; j += PH) acc += in[j * inner + col];
  }
  sm[ph][c] = acc;
  __syncthreads();
#pragma unroll
  for (int step = PH / 2; step > 0; step /= 2) {
    if (ph < step) sm[ph][c] += sm[ph + step][c];
    __syncthreads();
  }
  if (ph == 0 && col < inner) out[col] = sm[0][c];
}

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

// ============================================= time-split forward (inference)
//
// With few chains (batch * M * S) the lane-serial forward leaves CUs idle. For a
// forward without a backward the sequence can be cut into `chunks` equal pieces
// run side by side: a [B, L, .] tensor viewed as [B * chunks, L / chunks, .] is
// the same memory, with sequence b's chunk c at b' = b * chunks + c.
//
// The state entering each chunk comes from one pass over the chunks and one
// walk along them. In homogeneous coordinates lam = N / D, eta = W / D a step of
// filter_step is linear:
//   N' = A N + phi D,   D' = C N + D,   W' = g W + r D'      (g = a / a2)
// since lam' = (A lam + phi) / (C lam + 1), alpha = g / (C lam + 1) = g D / D'
// and eta' = alpha eta + r. So a chunk's steps compose to one 3x3 map
//   [[n0, n1, 0], [d0, d1, 0], [w0, w1, w2]]
// which needs no entering state, and the precision and information recurrences
// are carried together. (The reference's tiled Metal kernel takes two rounds
// here, composing the affine information leaves only once the precision is
// known: src/kla/ops/kernels/mps/tiled_kla_scan.metal:26-35.) The map is scaled
// after every step by the power of two that brings n0 + d1 into [0.5, 1), as
// mobius_compose does: exact, and harmless because every read-out is a ratio.

struct ChunkMapParams {
  SensorIn sn;
  const float *k, *a, *p;
  float *maps;   // [B', M, S, 8]: n0 n1 d0 d1 w0 w1 w2 (and one unused word)
};

template <int SP, bool BF16>
__global__ void __launch_bounds__(kFusedThreads) fused_chunk_map_kernel(ChunkMapParams prm, FusedGeom g) {
  constexpr int CH = kFusedThreads / SP;
  constexpr int TB = SP >= 128 ? kCkpt : kFusedTB;
  constexpr int KQB = SP >= 256 ? 1 : 2;
  constexpr bool kVecLds = SP >= 16;
  __shared__ __align__(16) float s_v[2][CH][TB + kPad], s_l[2][CH][TB + kPad];
  __shared__ __align__(16) float s_k[KQB][SP][TB + kPad];

  const FusedLane ln = fused_lane<SP>(g);
  const int64_t M = g.M, S = g.S, L = g.steps;
  const int64_t m0 = (xcd_block() % g.groups) * CH;
  const int c = static_cast<int>(ln.m - m0);
  const int64_t ms = ln.m * S + ln.s;
  const int64_t bms = ln.b * M * S + ms;
  const int64_t cols_m = M - m0 < CH ? M - m0 : CH;

  const float a_s = ln.active ? prm.a[ms] : 1.0f;
  const float pp = fmaxf(ln.active ? prm.p[ms] : 0.0f, kEps);
  const A2 a2 = split_a2(a_s);

  const SensorIn &sn = prm.sn;
  const float *kbase = prm.k + ln.b * L * S;
  TileRegs<TB, CH> rv, rl;
  TileRegs<TB, SP> rk;
  auto load = [&](int64_t t0) {
    const int64_t rows = L - t0;
    tile_load_sensor<TB, CH, BF16>(rv, sensor_at<BF16>(sn.v, ln.b * L + t0, m0, sn.ld_v), sn.ld_v, rows, cols_m);
    tile_load_sensor<TB, CH, BF16>(rl, sensor_at<BF16>(sn.lv, ln.b * L + t0, m0, sn.ld_lv), sn.ld_lv, rows, cols_m);
    tile_load<TB, SP>(rk, kbase + t0 * S, S, rows, S);
  };
  auto stage = [&](int buf) {
    widen_sensor<TB, CH, BF16>(rv);
    widen_sensor<TB, CH, BF16>(rl);
    tile_to_lds<TB, CH>(rv, s_v[buf]);
    to_precision<TB, CH>(rl, sn);
    tile_to_lds<TB, CH>(rl, s_l[buf]);
    tile_to_lds<TB, SP>(rk, s_k[KQB == 1 ? 0 : buf]);
  };

  float n0 = 1.0f, n1 = 0.0f, d0 = 0.0f, d1 = 1.0f, w0 = 0.0f, w1 = 0.0f, w2 = 1.0f;
  // The step's leaf scaled by a2 (the map is projective, so any common factor
  // is free): N' = (1 + p' phi) N + a2 phi D, D' = p' N + a2 D, W' = a W + r D'.
  // No quotient, and the decay a2 enters D' with its low part (split_a2), so
  // no rounding of a2 repeats from step to step.
  auto step = [&](float sig, float vv, float kk) {
    const float phi = sig * (kk * kk);
    const float r = (vv * sig) * kk;
    const float pphi = pp * phi, a2phi = a2.hi * phi;
    const float e0 = fmaf(a2.hi, d0, fmaf(pp, n0, a2.lo * d0)), e1 = fmaf(a2.hi, d1, fmaf(pp, n1, a2.lo * d1));
    const float m0_ = fmaf(a2phi, d0, fmaf(pphi, n0, n0)), m1_ = fmaf(a2phi, d1, fmaf(pphi, n1, n1));
    const float x0 = fmaf(a_s, w0, r * e0), x1 = fmaf(a_s, w1, r * e1), x2 = a_s * w2;
    const int e = __builtin_amdgcn_frexp_expf(m0_ + e1);
    n0 = __builtin_amdgcn_ldexpf(m0_, -e);
    n1 = __builtin_amdgcn_ldexpf(m1_, -e);
    d0 = __builtin_amdgcn_ldexpf(e0, -e);
    d1 = __builtin_amdgcn_ldexpf(e1, -e);
    w0 = __builtin_amdgcn_ldexpf(x0, -e);
    w1 = __builtin_amdgcn_ldexpf(x1, -e);
    w2 = __builtin_amdgcn_ldexpf(x2, -e);
  };

  const int64_t nblk = (L + TB - 1) / TB;
  if (nblk > 0) {
    load(0);
    stage(0);
  }
  __syncthreads();
  for (int64_t blk = 0; blk < nblk; ++blk) {
    const int cur = static_cast<int>(blk & 1);
    const int kb = KQB == 1 ? 0 : cur;
    const int64_t t0 = blk * TB;
    if (blk + 1 < nblk) load(t0 + TB);
    if (t0 + TB <= L) {
#pragma unroll
      for (int j = 0; j < TB; j += 4) {
        if constexpr (kVecLds) {
          const float4 l4 = lds4(s_l[cur][c], j), v4 = lds4(s_v[cur][c], j), k4 = lds4(s_k[kb][ln.s], j);
#pragma unroll
          for (int i = 0; i < 4; ++i) step(pick4(l4, i), pick4(v4, i), pick4(k4, i));
        } else {
#pragma unroll
          for (int i = 0; i < 4; ++i) step(s_l[cur][c][j + i], s_v[cur][c][j + i], s_k[kb][ln.s][j + i]);
        }
      }
    } else {
      const int nv = static_cast<int>(L - t0);
      for (int j = 0; j < nv; ++j) step(s_l[cur][c][j], s_v[cur][c][j], s_k[kb][ln.s][j]);
    }
    if (blk + 1 < nblk) {
      if constexpr (KQB == 1) __syncthreads();   // every wave is done with this block's k
      stage(cur ^ 1);
    }
    __syncthreads();
  }
  if (ln.active) {
    float4 *out = reinterpret_cast<float4 *>(prm.maps + bms * 8);
    out[0] = make_float4(n0, n1, d0, d1);
    out[1] = make_float4(w0, w1, w2, 0.0f);
  }
}

// The state entering each chunk, per (b, m, s) lane: from (lam0 or 1, eta0 or 0)
// the chunk maps are applied in chunk order, lam' = (n0 lam + n1) / (d0 lam + d1)
// and eta' = (w0 lam + w1 + w2 eta) / (d0 lam + d1). maps [batch, chunks, n, 8];
// lam0, eta0 [batch, n] or NULL; lam_start, eta_start [batch, chunks, n]; lam_end,
// eta_end [batch, n] (the state after the last chunk) or NULL.
//
// A step's denominator (p/a2) lam + 1 is at least 1, so the sequential filter never
// floors it and the composed map is exact. A map rescaled to a trace in [0.5, 1)
// can still carry a normal d1 far below EPS (lam0 = 0 under decay: d1 ~ a^(2 steps)
// relative to n0), so only a zero or subnormal denominator is guarded (FLT_MIN);
// an EPS floor here would replace such a d1 and lose the chunk's state.
constexpr float kMapDenMin = __FLT_MIN__;

__global__ void __launch_bounds__(256) chunk_starts_kernel(const float *__restrict__ maps,
                                                           const float *__restrict__ lam0,
                                                           const float *__restrict__ eta0,
                                                           float *__restrict__ lam_start, float *__restrict__ eta_start,
                                                           float *__restrict__ lam_end, float *__restrict__ eta_end,
                                                           int64_t batch, int64_t chunks, int64_t n) {
  const int64_t i = static_cast<int64_t>(blockIdx.x) * 256 + threadIdx.x;
  if (i >= batch * n) return;
  const int64_t b = i / n, e = i % n;
  float lam = lam0 ? lam0[i] : 1.0f;
  float eta = eta0 ? eta0[i] : 0.0f;
  for (int64_t ch = 0; ch < chunks; ++ch) {
    const int64_t row = (b * chunks + ch) * n + e;
    lam_start[row] = lam;
    eta_start[row] = eta;
    const float4 *m = reinterpret_cast<const float4 *>(maps + row * 8);
    const float4 nd = m[0], w = m[1];
    const float den = fmaxf(fmaf(nd.z, lam, nd.w), kMapDenMin);
    const float nl = fmaf(nd.x, lam, nd.y) / den;
    eta = (fmaf(w.x, lam, w.y) + w.z * eta) / den;
    lam = nl;
  }
  if (lam_end) {
    lam_end[i] = lam;
    eta_end[i] = eta;
  }
}

// ============================================== time-split backward (training)
//
// The backward's reverse walk carries the adjoint (gl, ge) of the state
// (lam_t, eta_t). Step t of fused_kla_bwd_kernel maps it, with the forward's
// trajectory fixed, as
//   ge_t = ge + c_e,   gl_t = gl + c_l        (the step's read-out terms:
//                                              c_e = dmean var, c_l = -T var, or 0
//                                              where var's clamp acts)
//   ge' = alpha ge_t,  gl' = p gl_t + q ge_t   (p = 1/(a2 den^2) = inv_den idn_a,
//                                              q = -eta' inv_Da alpha p' where the
//                                              gain's clamp is idle, else 0)
// an affine map with an upper-triangular linear part, so a chunk's steps compose
// into five numbers per lane, x -> [[P, Q], [0, A]] x + (u_l, u_e), whatever
// adjoint enters the chunk from the right. fused_adjoint_map_kernel composes
// them per chunk (replaying each 16-step block from the forward's checkpoints,
// like the backward), adjoint_ends_kernel walks the maps from the end of each
// sequence and leaves every chunk the adjoint entering it from the right, and
// fused_kla_bwd_kernel then runs on the [B * chunks, L / chunks] view with those
// as its dlam_fin, deta_fin: the view's checkpoints, sensors, gradients and
// partial sums are the same memory as the whole sequence's.

struct AdjointMapParams {
  const float *dy, *dyvar;   // dyvar NULL: no y_var gradient (VAR false)
  SensorIn sn;
  const float *k, *q, *a, *p, *ck_lam, *ck_eta;
  float *maps;   // [B', M, S, 8]: P Q A u_l u_e (and three unused words)
};

template <int SP, bool PRIOR, bool BF16, bool VAR>
__global__ void __launch_bounds__(kFusedThreads) fused_adjoint_map_kernel(AdjointMapParams prm, FusedGeom g) {
  constexpr int CH = kFusedThreads / SP;
  constexpr int TB = kCkpt;
  constexpr int KQB = SP >= 256 ? 1 : 2;
  constexpr bool kK2 = SP <= kWave;
  __shared__ __align__(16) float s_l[2][CH][TB + kPad], s_sv[2][CH][TB + kPad];
  __shared__ __align__(16) float s_dy[2][CH][TB + kPad], s_dyv[VAR ? 2 : 1][VAR ? CH : 1][TB + kPad];
  __shared__ __align__(16) float s_k[KQB][SP][TB + kPad], s_q[KQB][SP][TB + kPad];
  __shared__ __align__(16) float s_k2[kK2 ? KQB : 1][kK2 ? SP : 1][TB + kPad];

  const FusedLane ln = fused_lane<SP>(g);
  const int64_t M = g.M, S = g.S, L = g.steps;
  const int64_t m0 = (xcd_block() % g.groups) * CH;
  const int c = static_cast<int>(ln.m - m0);
  const int64_t ms = ln.m * S + ln.s;
  const int64_t bms = ln.b * M * S + ms;
  const int64_t cols_m = M - m0 < CH ? M - m0 : CH;

  const float a_s = ln.active ? prm.a[ms] : 1.0f;
  const float pp = fmaxf(ln.active ? prm.p[ms] : 0.0f, kEps);
  const A2 a2s = split_a2(a_s);
  const float a2 = a2s.hi;

  const int64_t offM = ln.b * L * M + m0, offS = ln.b * L * S;
  const SensorIn &sn = prm.sn;
  TileRegs<TB, CH> rv, rl, rdy, rdyv;
  TileRegs<TB, SP> rk, rq;
  auto load = [&](int64_t t0) {
    const int64_t rows = L - t0;
    tile_load_sensor<TB, CH, BF16>(rv, sensor_at<BF16>(sn.v, ln.b * L + t0, m0, sn.ld_v), sn.ld_v, rows, cols_m);
    tile_load_sensor<TB, CH, BF16>(rl, sensor_at<BF16>(sn.lv, ln.b * L + t0, m0, sn.ld_lv), sn.ld_lv, rows, cols_m);
    tile_load<TB, CH>(rdy, prm.dy + offM + t0 * M, M, rows, cols_m);
    if constexpr (VAR) tile_load<TB, CH>(rdyv, prm.dyvar + offM + t0 * M, M, rows, cols_m);
    tile_load<TB, SP>(rk, prm.k + offS + t0 * S, S, rows, S);
    tile_load<TB, SP>(rq, prm.q + offS + t0 * S, S, rows, S);
  };
  auto stage = [&](int buf) {
    const int kb = KQB == 1 ? 0 : buf;
    widen_sensor<TB, CH, BF16>(rv);
    widen_sensor<TB, CH, BF16>(rl);
    to_precision<TB, CH>(rl, sn);
    tile_mul_to_lds<TB, CH>(rv, rl, s_sv[buf]);
    tile_to_lds<TB, CH>(rl, s_l[buf]);
    tile_to_lds<TB, CH>(rdy, s_dy[buf]);
    if constexpr (VAR) tile_to_lds<TB, CH>(rdyv, s_dyv[VAR ? buf : 0]);
    tile_to_lds<TB, SP>(rk, s_k[kb]);
    if constexpr (kK2) tile_mul_to_lds<TB, SP>(rk, rk, s_k2[kK2 ? kb : 0]);
    tile_to_lds<TB, SP>(rq, s_q[kb]);
  };

  // The chunk's map so far (identity): the adjoint entering the chunk from the
  // right, x, becomes [[P, Q], [0, A]] x + (ul, ue) before the steps walked.
  float P = 1.0f, Q = 0.0f, A = 1.0f, ul = 0.0f, ue = 0.0f;
  const int64_t n_ck = g.n_ck;
  // Checkpoints are read one block ahead, with the block's tiles (as in
  // fused_kla_bwd_kernel: a load just before the replay waits for all in flight).
  float ck_l = 1.0f, ck_e = 0.0f;
  auto load_ck = [&](int64_t blk) {
    if (ln.active) {
      const int64_t ci = ((ln.b * n_ck + blk) * M + ln.m) * S + ln.s;
      ck_l = prm.ck_lam[ci];
      ck_e = prm.ck_eta[ci];
    }
  };
  if (n_ck > 0) {
    load((n_ck - 1) * TB);
    load_ck(n_ck - 1);
    stage(0);
  }
  __syncthreads();
  for (int64_t i = 0; i < n_ck; ++i) {
    const int cur = static_cast<int>(i & 1);
    const int kb = KQB == 1 ? 0 : cur;
    const int64_t blk = n_ck - 1 - i;
    const int64_t t0 = blk * TB;
    const float lam_ck = ck_l, eta_ck = ck_e;
    if (i + 1 < n_ck) {
      load(t0 - TB);
      load_ck(blk - 1);
    }
    const int nv = static_cast<int>(L - t0 < TB ? L - t0 : TB);
    // The block's replay and its steps composed in reverse, as the backward's
    // replay and walk (FULL: every step of the block lies inside the sequence;
    // tile values four steps per LDS read from 16 lanes per channel on).
    auto block = [&](auto full_c) __attribute__((always_inline)) {
      constexpr bool FULL = decltype(full_c)::value;
      constexpr bool X4 = SP >= 16;
      float lh[TB + 1], eh[TB + 1], idn[TB];
      {
        float lam = lam_ck;
        float eta = eta_ck;
        float4 l4{}, v4{}, k4{}, k24{};
#pragma unroll
        for (int j = 0; j < TB; ++j) {
          if (X4 && j % 4 == 0) {
            asm volatile("" ::: "memory");
            l4 = lds4(s_l[cur][c], j);
            v4 = lds4(s_sv[cur][c], j);
            k4 = lds4(s_k[kb][ln.s], j);
            if constexpr (kK2) k24 = lds4(s_k2[kK2 ? kb : 0][kK2 ? ln.s : 0], j);
          }
          lh[j] = lam;
          eh[j] = eta;
          if (!FULL) idn[j] = 0.0f;
          if (FULL || j < nv) {
            const float sig = X4 ? pick4(l4, j % 4) : s_l[cur][c][j];
            const float sv = X4 ? pick4(v4, j % 4) : s_sv[cur][c][j];
            const float kk = X4 ? pick4(k4, j % 4) : s_k[kb][ln.s][j];
            const float k2 = !kK2 ? kk * kk : X4 ? pick4(k24, j % 4) : s_k2[kK2 ? kb : 0][kK2 ? ln.s : 0][j];
            lam = filter_step(lam, eta, sig * k2, sv * kk, a_s, a2s, pp, idn[j]);
          }
        }
        lh[TB] = lam;
        eh[TB] = eta;
      }
      // The read-out terms as the backward forms them: dmean, t = d(loss)/d(var) var.
      float4 dy4{}, q4{}, dyv4{};
#pragma unroll
      for (int j = TB - 1; j >= 0; --j) {
        if (X4 && j % 4 == 3) {
          asm volatile("" ::: "memory");
          dy4 = lds4(s_dy[cur][c], j - 3);
          q4 = lds4(s_q[kb][ln.s], j - 3);
          if constexpr (VAR) dyv4 = lds4(s_dyv[VAR ? cur : 0][VAR ? c : 0], j - 3);
        }
        if (FULL || j < nv) {
          const float dy = X4 ? pick4(dy4, j % 4) : s_dy[cur][c][j];
          const float qq = X4 ? pick4(q4, j % 4) : s_q[kb][ln.s][j];
          const float ep = eh[j];
          const float lam_t = lh[j + 1], eta_t = eh[j + 1];
          const float idn_a = idn[j];
          const float inv_den = inv_den_from(a2s, idn_a);
          const bool da_ok = idn_a <= kInvEps;
          const float inv_Da = fminf(idn_a, kInvEps);
          const float alpha = a_s * inv_Da;
          const float var = rcp(fmaxf(lam_t, kEps));
          const float mean = eta_t * var;
          const float dmo = dy * qq;
          const float dmean = PRIOR ? dmo * a_s : dmo;
          float t;
          if constexpr (VAR) {
            const float dyv = X4 ? pick4(dyv4, j % 4) : s_dyv[VAR ? cur : 0][VAR ? c : 0][j];
            const float dvo = dyv * (qq * qq);
            t = fmaf(dmean, mean, (PRIOR ? dvo * a2 : dvo) * var);
          } else {
            t = dmean * mean;
          }
          const float c_e = dmean * var;
          const float c_l = lam_t >= kEps ? -(t * var) : 0.0f;
          const float p_t = inv_den * idn_a;
          const float q_t = da_ok ? -((ep * inv_Da) * alpha) * pp : 0.0f;
          const float vl = ul + c_l, ve = ue + c_e;
          Q = fmaf(p_t, Q, q_t * A);
          P = p_t * P;
          A = alpha * A;
          ul = fmaf(p_t, vl, q_t * ve);
          ue = alpha * ve;
        }
      }
    };
    if (nv == TB)
      block(std::true_type{});
    else
      block(std::false_type{});
    if (i + 1 < n_ck) {
      if constexpr (KQB == 1) __syncthreads();   // every wave is done with this block's k, q
      stage(cur ^ 1);
    }
    __syncthreads();
  }
  if (ln.active) {
    float4 *out = reinterpret_cast<float4 *>(prm.maps + bms * 8);
    out[0] = make_float4(P, Q, A, ul);
    out[1] = make_float4(ue, 0.0f, 0.0f, 0.0f);
  }
}

// The adjoint entering each chunk from the right, per (b, m, s) lane: from
// (dlam_fin or 0, deta_fin or 0) at the end of the sequence the chunk maps are
// applied from the last chunk to the first. maps [batch, chunks, n, 8]; dlam_fin,
// deta_fin [batch, n] or NULL; gl_end, ge_end [batch, chunks, n].
__global__ void __launch_bounds__(256) adjoint_ends_kernel(const float *__restrict__ maps,
                                                           const float *__restrict__ dlam_fin,
                                                           const float *__restrict__ deta_fin,
                                                           float *__restrict__ gl_end, float *__restrict__ ge_end,
                                                           int64_t batch, int64_t chunks, int64_t n) {
  const int64_t i = static_cast<int64_t>(blockIdx.x) * 256 + threadIdx.x;
  if (i >= batch * n) return;
  const int64_t b = i / n, e = i % n;
  float gl = dlam_fin ? dlam_fin[i] : 0.0f;
  float ge = deta_fin ? deta_fin[i] : 0.0f;
  for (int64_t ch = chunks - 1; ch >= 0; --ch) {
    const int64_t row = (b * chunks + ch) * n + e;
    gl_end[row] = gl;
    ge_end[row] = ge;
    const float4 *m = reinterpret_cast<const float4 *>(maps + row * 8);
    const float4 pqa = m[0], rest = m[1];
    const float gl_new = fmaf(pqa.x, gl, fmaf(pqa.y, ge, pqa.w));
    ge = fmaf(pqa.z, ge, rest.x);
    gl = gl_new;
  }
}

}  // namespace kla

namespace kla {

// ========================================================== one decode step
//
// kla_step (reference src/kla/ops/kla_ops.py:293-331) for every (b, m, s) lane:
//   phi = max(Lv k^2, EPS)  (the step floors phi, the scan does not)
//   r = (v Lv) k,  denom = max(a2 + p' lam, EPS)
//   lam <- lam/denom + phi,  eta <- (a/denom) eta + r
//   var = 1/max(lam, EPS), mean = eta var (prior: mean = a mean, var = a2 var + p')
//   y[b, m] = sum_s q mean,  y_var[b, m] = sum_s q^2 var
// Same lane layout as the fused scan. lam_out / eta_out may alias lam / eta
// (each lane reads its own element before writing it). IEEE division: the step
// is tiny and launch-bound, not VALU-bound.

struct StepParams {
  const float *v, *lv, *k, *q, *a, *p, *lam, *eta;
  float *y, *yvar, *lam_out, *eta_out;
};

template <int SP, bool PRIOR>
__global__ void __launch_bounds__(kFusedThreads) kla_step_kernel(StepParams prm, FusedGeom g) {
  const FusedLane ln = fused_lane<SP>(g);
  const int64_t M = g.M, S = g.S;
  const bool mok = ln.m < M, sok = ln.s < S;
  const int64_t ms = ln.m * S + ln.s;
  const int64_t bms = ln.b * M * S + ms;
  const float a_s = ln.active ? prm.a[ms] : 1.0f;
  const float pp = fmaxf(ln.active ? prm.p[ms] : 0.0f, kEps);
  const A2 a2s = split_a2(a_s);   // a2 + p' lam rounded once per step, as in the scan
  const float a2 = a2s.hi;
  const float vv = mok ? prm.v[ln.b * M + ln.m] : 0.0f;
  const float sig = mok ? prm.lv[ln.b * M + ln.m] : 0.0f;
  const float kk = sok ? prm.k[ln.b * S + ln.s] : 0.0f;
  const float qq = sok ? prm.q[ln.b * S + ln.s] : 0.0f;
  float lam = ln.active ? prm.lam[bms] : 1.0f;
  float eta = ln.active ? prm.eta[bms] : 0.0f;

  const float phi = fmaxf(sig * (kk * kk), kEps);
  const float r = (vv * sig) * kk;
  const float denom = fmaxf(fmaf(pp, lam, a2s.lo) + a2s.hi, kEps);
  lam = lam / denom + phi;
  eta = (a_s / denom) * eta + r;
  const float var = 1.0f / fmaxf(lam, kEps);
  float mean = eta * var, vo = var;
  if (PRIOR) {
    mean = a_s * mean;
    vo = a2 * var + pp;
  }
  const float ys = channel_sum<SP>(mean * qq);
  const float vs = channel_sum<SP>(vo * (qq * qq));
  if (ln.s == 0 && mok) {
    prm.y[ln.b * M + ln.m] = ys;
    prm.yvar[ln.b * M + ln.m] = vs;
  }
  if (ln.active) {
    prm.lam_out[bms] = lam;
    prm.eta_out[bms] = eta;
  }
}

// ----------------------------------------------------- layer decode step
//
// The whole one-token SSM step of a KLALayer in one kernel, for inference
// (fp32, no gradient): the discretisation of the static parameters
// (_continuous_params / _discretize / _compute_aq, reference kla_layer.py:164-190),
// the sensor read-out of the projection (_project_sensors after the linear maps,
// :194-231), the filter step (kla_step, kla_ops.py:293-331), the lambda skip and
// the gating of the layer's forward (:295-349). Each (b, m, s) lane recomputes
// its (a_bar, p_bar) from the [M, S] parameters, which costs a few exp / log1p
// per lane instead of ~17 separate elementwise launches per token. Operations
// follow torch's order and formulas (softplus with threshold 20, silu
// x / (1 + exp(-x)), gelu 0.5 x (1 + erf(x / sqrt 2))), so results agree with
// the torch path to a few ulp.

enum DecodeAct { kActNone = 0, kActSilu = 1, kActGelu = 2, kActRelu = 3 };

struct DecodeParams {
  const float *v, *lv, *k, *q;          // rows of the sensor projection
  const float *z, *skip, *gate;         // residual z, lambda_skip, raw gate (NULL: absent)
  int64_t ld_v, ld_lv, ld_kq, ld_z, ld_gate;
  const float *delta, *lambda_log, *pnoise;   // [M, S]
  const float *lam, *eta;               // [B, M, S] in
  float *lam_out, *eta_out, *y, *yvar;  // [B, M, S], [B, M] out
  int ou, zero_pn, qk_norm, has_clip, skip_vector, gate_act;
  float clip, ov_min, ov_max;
};

__device__ __forceinline__ float activation(int act, float x) {
  if (act == kActSilu) return x / (1.0f + expf(-x));
  if (act == kActGelu) return 0.5f * x * (1.0f + erff(x * 0.70710678118654752440f));
  if (act == kActRelu) return x > 0.0f ? x : 0.0f;
  return x;
}

// Workgroup w covers channel group w % groups of batch rows [BB (w / groups),
// + BB): each thread discretises its (m, s) once and runs the step for its BB
// rows (the discretisation is the step's costliest part: exp, softplus, expm1).
template <int SP, bool PRIOR, int BB>
__global__ void __launch_bounds__(kFusedThreads) kla_decode_step_kernel(DecodeParams prm, FusedGeom g) {
  constexpr int CH = kFusedThreads / SP;
  const int tid = static_cast<int>(threadIdx.x);
  const int sl = tid % SP;
  const int64_t b0 = (static_cast<int64_t>(blockIdx.x) / g.groups) * BB;
  const int64_t m = (static_cast<int64_t>(blockIdx.x) % g.groups) * CH + tid / SP;
  const int64_t M = g.M, S = g.S;
  const bool mok = m < M, sok = sl < S;
  const bool active = mok && sok;
  const int64_t ms = m * S + sl;

  // (a_bar, p_bar) of this (m, s).
  float a_bar = 1.0f, p_bar = 0.0f;
  if (active) {
    const float a = -expf(prm.lambda_log[ms]);
    float p = prm.pnoise[ms];
    if (prm.zero_pn) {
      p = p + 1e-12f;
    } else {
      p = fmaxf(p, 1e-7f);
      if (prm.has_clip) p = fminf(p, prm.clip);
    }
    const float delta = softplus_t(prm.delta[ms]) + 1e-7f;
    a_bar = expf(delta * a);
    if (prm.ou) {
      const float rate = fmaxf(fabsf(a), 1e-8f);
      p_bar = (p / (2.0f * rate)) * (-expm1f((-2.0f * rate) * delta));
    } else {
      p_bar = p * delta;
    }
  }
  const float a_s = a_bar;
  const float pp = fmaxf(p_bar, kEps);
  const A2 a2s = split_a2(a_s);   // a2 + p' lam rounded once per step, as in the scan
  const float a2 = a2s.hi;

#pragma unroll
  for (int bb = 0; bb < BB; ++bb) {
    const int64_t b = b0 + bb;
    if (b >= g.batch) break;   // workgroup-uniform
    const int64_t bms = b * M * S + ms;
    // Sensors: k, q (l2-normalised over the S states, clipped), Lambda^v = 1 / obs_var.
    float kk = sok ? prm.k[b * prm.ld_kq + sl] : 0.0f;
    float qq = sok ? prm.q[b * prm.ld_kq + sl] : 0.0f;
    if (prm.qk_norm) {
      kk = kk / fmaxf(sqrtf(channel_sum<SP>(kk * kk)), 1e-12f);
      qq = qq / fmaxf(sqrtf(channel_sum<SP>(qq * qq)), 1e-12f);
    }
    if (prm.has_clip) {
      kk = fminf(fmaxf(kk, -prm.clip), prm.clip);
      qq = fminf(fmaxf(qq, -prm.clip), prm.clip);
    }
    const float vv = mok ? prm.v[b * prm.ld_v + m] : 0.0f;
    float ov = (mok ? softplus_t(prm.lv[b * prm.ld_lv + m]) : 1.0f) + prm.ov_min;
    ov = fminf(ov, prm.ov_max);
    const float sig = 1.0f / ov;

    // The filter step (as kla_step_kernel).
    float lam = active ? prm.lam[bms] : 1.0f;
    float eta = active ? prm.eta[bms] : 0.0f;
    const float phi = fmaxf(sig * (kk * kk), kEps);
    const float r = (vv * sig) * kk;
    const float denom = fmaxf(fmaf(pp, lam, a2s.lo) + a2s.hi, kEps);
    lam = lam / denom + phi;
    eta = (a_s / denom) * eta + r;
    const float var = 1.0f / fmaxf(lam, kEps);
    float mean = eta * var, vo = var;
    if (PRIOR) {
      mean = a_s * mean;
      vo = a2 * var + pp;
    }
    const float ys = channel_sum<SP>(mean * qq);
    const float vs = channel_sum<SP>(vo * (qq * qq));
    if (sl == 0 && mok) {
      float yo = ys, vo2 = vs;
      if (prm.z) {
        const float lsk = prm.skip_vector ? prm.skip[m] : prm.skip[0];
        yo = yo + lsk * prm.z[b * prm.ld_z + m];
      }
      if (prm.gate) {
        const float gg = activation(prm.gate_act, prm.gate[b * prm.ld_gate + m]);
        yo = yo * gg;
        vo2 = vo2 * (gg * gg);
      }
      prm.y[b * M + m] = yo;
      prm.yvar[b * M + m] = vo2;
    }
    // This thread alone reads and writes (b, m, s): lam_out / eta_out may alias lam / eta.
    if (active) {
      prm.lam_out[bms] = lam;
      prm.eta_out[bms] = eta;
    }
  }
}

// The static dynamics of a KLA layer, per (m, s) (reference kla_layer.py:164-190,
// KLALayer._continuous_params / _discretize / _compute_aq):
//   a = -exp(lambda_log);  p = pn + 1e-12 (zero_pn) or min(max(pn, 1e-7), clip)
//   d = softplus(delta) + 1e-7;  a_bar = exp(d a)
//   OU: rate = max(|a|, 1e-8), p_bar = (p / (2 rate)) (-expm1((-2 rate) d));  ZOH: p_bar = p d
// The backward is the chain rule through those same operations, term by term as
// torch's autograd forms it (clamp gradients pass at equality, softplus's
// gradient is 1 above the threshold 20, expm1's is exp).
struct DiscParams {
  const float *delta, *lambda_log, *pnoise;
  float *a_bar, *p_bar;                 // forward outputs
  const float *g_a, *g_p;               // backward: gradients of a_bar, p_bar (NULL: zero)
  float *d_delta, *d_ll, *d_pn;         // backward outputs
  int64_t n;
  int ou, zero_pn, has_clip;
  float clip;
};

__global__ void __launch_bounds__(256) discretize_fwd_kernel(DiscParams q) {
  const int64_t i = static_cast<int64_t>(blockIdx.x) * 256 + threadIdx.x;
  if (i >= q.n) return;
  const float a = -expf(q.lambda_log[i]);
  float p = q.pnoise[i];
  if (q.zero_pn) {
    p = p + 1e-12f;
  } else {
    p = fmaxf(p, 1e-7f);
    if (q.has_clip) p = fminf(p, q.clip);
  }
  const float d = softplus_t(q.delta[i]) + 1e-7f;
  q.a_bar[i] = expf(d * a);
  if (q.ou) {
    const float rate = fmaxf(fabsf(a), 1e-8f);
    q.p_bar[i] = (p / (2.0f * rate)) * (-expm1f((-2.0f * rate) * d));
  } else {
    q.p_bar[i] = p * d;
  }
}

__global__ void __launch_bounds__(256) discretize_bwd_kernel(DiscParams q) {
  const int64_t i = static_cast<int64_t>(blockIdx.x) * 256 + threadIdx.x;
  if (i >= q.n) return;
  const float ll = q.lambda_log[i], pn = q.pnoise[i], dl = q.delta[i];
  const float g_a = q.g_a ? q.g_a[i] : 0.0f, g_p = q.g_p ? q.g_p[i] : 0.0f;
  const float a = -expf(ll);
  float p = pn, g_pmask = 1.0f;
  if (q.zero_pn) {
    p = p + 1e-12f;
  } else {
    if (!(pn >= 1e-7f)) g_pmask = 0.0f;
    p = fmaxf(p, 1e-7f);
    if (q.has_clip) {
      if (!(p <= q.clip)) g_pmask = 0.0f;
      p = fminf(p, q.clip);
    }
  }
  const float d = softplus_t(dl) + 1e-7f;
  const float a_bar = expf(d * a);
  // a_bar = exp(t), t = d a
  const float g_t = g_a * a_bar;
  float g_d = g_t * a;
  float g_ac = g_t * d;   // gradient of the continuous a
  float g_pp;             // gradient of the floored / clipped p
  if (q.ou) {
    const float absa = fabsf(a);
    const float rate = fmaxf(absa, 1e-8f);
    const float two_rate = 2.0f * rate;
    const float q1 = p / two_rate;
    const float c = -2.0f * rate;
    const float u = c * d;
    const float E = -expm1f(u);
    // p_bar = q1 E
    const float g_q1 = g_p * E;
    const float g_E = g_p * q1;
    // E = -expm1(u)
    const float g_u = -g_E * expf(u);
    // u = c d
    const float g_c = g_u * d;
    g_d += g_u * c;
    // q1 = p / two_rate
    g_pp = g_q1 / two_rate;
    const float g_two_rate = -g_q1 * p / (two_rate * two_rate);
    // two_rate = 2 rate, c = -2 rate
    const float g_rate = 2.0f * g_two_rate + -2.0f * g_c;
    // rate = max(|a|, 1e-8)
    const float g_abs = absa >= 1e-8f ? g_rate : 0.0f;
    const float sgn = a > 0.0f ? 1.0f : (a < 0.0f ? -1.0f : 0.0f);
    g_ac += g_abs * sgn;
  } else {
    g_pp = g_p * d;
    g_d += g_p * p;
  }
  // d = softplus(delta) + 1e-7 (threshold 20)
  const float z = expf(dl);
  q.d_delta[i] = dl > 20.0f ? g_d : g_d * z / (z + 1.0f);
  // a = -exp(lambda_log)
  q.d_ll[i] = g_ac * a;
  q.d_pn[i] = g_pp * g_pmask;
}

// One token of the depthwise causal conv (CausalConv1d, reference common.py:70-96):
// window = [state[b, d, :], x[b, d]], y = act(sum_j w[d, j] window[j] + bias[d]),
// new state = window[1:]. One thread per (b, d).
// state_out may alias state: each thread reads its window before writing it, and
// the shift writes position j only after reading j + 1 (no __restrict__ on either).
__global__ void conv_step_kernel(const float *__restrict__ x, int64_t ld_x, const float *state,
                                 float *state_out, const float *__restrict__ w,
                                 const float *__restrict__ bias, int act, float *__restrict__ y, int64_t batch,
                                 int64_t D, int K) {
  const int64_t i = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x;
  if (i >= batch * D) return;
  const int64_t b = i / D, d = i % D;
  const float *st = state + i * (K - 1);
  float *so = state_out + i * (K - 1);
  const float *wd = w + d * K;
  const float xt = x[b * ld_x + d];
  float acc = 0.0f;
  for (int j = 0; j < K - 1; ++j) acc += st[j] * wd[j];
  acc += xt * wd[K - 1];
  if (bias) acc = acc + bias[d];
  y[i] = activation(act, acc);
  for (int j = 0; j + 1 < K - 1; ++j) so[j] = st[j + 1];
  if (K > 1) so[K - 2] = xt;
}

}  // namespace kla
