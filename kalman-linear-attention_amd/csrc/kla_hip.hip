// kla_hip.hip -- extern "C" entry points of libkla_hip.so (declared in
// include/kla_hip.h): host-side validation, launch geometry, workspace sizing,
// and the kernel instantiations for gfx950.
//
// Validation mirrors the TORCH_CHECKs of the reference's CUDA binding
// (src/kla/ops/kernels/cuda/v2_2/kla_matmul_scan.cu:35-59): every argument is
// checked before the first HIP call, so a bad call returns a status and a
// message instead of launching anything.
#include <stdarg.h>
#include <stdio.h>

#include <algorithm>
#include <initializer_list>
#include <mutex>
#include <type_traits>

#pragma GCC visibility push(default)
#include "kla_hip.h"
#pragma GCC visibility pop

#include "gate_skip.hpp"
#include "model_ops.hpp"
#include "rows_linear.hpp"
#include "fused_kla.hpp"
#include "lookback_scan.hpp"

namespace {

using namespace kla;

constexpr int kAbiVersion = 17;

// Tile shapes: W waves x S steps per wave (chunk = W*S steps), V lanes per
// thread (tile = 64 V lanes), each chosen by timing the kernel inside the
// fwd+bwd step on MI355X (fp32 at batch 8, 4096 steps, 2048 lanes; bf16 at
// 8 x 8192 x 2048). The forward scans want a short register footprint
// (occupancy hides the look-back), the backward scans long chunks; bf16 holds
// two elements per register, so its tiles run wider (V = 2, 4) for the same
// footprint. A V > 1 shape needs lanes % V == 0 and operands aligned to V
// elements; the V = 1 shape of the same kind serves every other call.
template <class P, int W_, int S_, int V_>
struct Shape3 {
  using Policy = P;
  static constexpr int W = W_, S = S_, V = V_;
};
using MobiusFwdTile = Shape3<void, 8, 12, 1>;
// 24 steps per wave: the backward reads the saved lam once per 24 steps.
using MobiusBwdTile = Shape3<void, 12, 24, 1>;
using AffineFwdTile = Shape3<void, 16, 24, 1>;
// fp32 affine forward whose output is stored cached (it fits the memory-side cache).
using AffineFwdCachedTile = Shape3<void, 12, 24, 1>;
using AffineBwdTile = Shape3<void, 12, 32, 1>;
using AffineFwdBf16Tile = Shape3<void, 12, 24, 2>;
using AffineBwdBf16Tile = Shape3<void, 16, 16, 4>;
using AffineBf16Fallback = Shape3<void, 8, 32, 1>;

constexpr uint32_t kMaxSpin = 1u << 20;   // ~1 s of polling before a look-back wait gives up

// Batch rows per thread of the one-token SSM step (kla_decode_step_kernel): one
// (more workgroups beat discretising the dynamics fewer times, in C5 decode).
constexpr int kDecodeRows = 1;

thread_local char g_last_error[512] = "";

int fail(int code, const char *fmt, ...) {
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(g_last_error, sizeof(g_last_error), fmt, ap);
  va_end(ap);
  return code;
}

struct Shape {
  int64_t batch, steps, lanes;
};

// Workspace sizes are products of caller-given counts: they are formed with
// these saturating operations (nonnegative operands), which stop at kHuge = 2^62
// bytes or elements instead of overflowing. No device holds kHuge bytes, so a
// saturated size is a problem too large to run: the *_workspace_bytes queries
// return 0 for it and the entry points reject it before launching.
constexpr int64_t kHuge = int64_t(1) << 62;

int64_t smul(int64_t a, int64_t b) {
  int64_t r;
  return (__builtin_mul_overflow(a, b, &r) || r > kHuge) ? kHuge : r;
}

int64_t sadd(int64_t a, int64_t b) {
  int64_t r;
  return (__builtin_add_overflow(a, b, &r) || r > kHuge) ? kHuge : r;
}

int check_shape(const char *fn, Shape s) {
  if (s.batch < 0 || s.steps < 0 || s.lanes < 0)
    return fail(KLA_ERR_INVALID_ARG, "%s: negative size (batch=%lld steps=%lld lanes=%lld)", fn,
                (long long)s.batch, (long long)s.steps, (long long)s.lanes);
  // Keep every element index well inside int64 and every grid inside 2^31.
  if (s.batch > (1ll << 31) || s.steps > (1ll << 31) || s.lanes > (1ll << 31))
    return fail(KLA_ERR_INVALID_ARG, "%s: dimension above 2^31", fn);
  return KLA_OK;
}

Geom make_geom(Shape s, int W, int S, int V) {
  Geom g;
  g.batch = s.batch;
  g.steps = s.steps;
  g.lanes = s.lanes;
  const int64_t tile = static_cast<int64_t>(kWave) * V;
  g.tiles_per_batch = (s.lanes + tile - 1) / tile;
  g.n_tiles = s.batch * g.tiles_per_batch;
  const int64_t chunk = static_cast<int64_t>(W) * S;
  g.n_chunks = (s.steps + chunk - 1) / chunk;
  g.plane = g.n_tiles * tile;
  g.max_spin = kMaxSpin;
  g.carry_only = 0;
  return g;
}

// The affine forward's output h is stored cached (for the backward that reads it
// next) when the whole [batch, steps, lanes] output fits MI355X's 256 MiB
// memory-side cache; larger outputs stream. Measured in the fwd + bwd step with
// the output cached: 256 MiB outputs (8 x 4096 x 2048 fp32, 8 x 8192 x 2048
// bf16) gain 1.5-3%, a 512 MiB output (8 x 8192 x 2048 fp32) loses 2-3%.
constexpr int64_t kCachedOutputBytes = 256ll << 20;

bool output_fits_cache(Shape s, int64_t elem) { return s.batch * s.steps * s.lanes * elem <= kCachedOutputBytes; }

// First scan position from which the Moebius forward loads its `tensors` fp32
// inputs cached: the last steps whose inputs fill the memory-side cache (every
// step when they all fit). The backward starts at the end of the sequence and
// finds them there. Measured in the headline fwd + bwd step (8 x 4096 x 2048,
// 768 MiB of A, B, C, the last third cached): Moebius bwd 350 -> 332 us and the
// affine forward that follows 149 -> 139 us, for 197 -> 220 us in the Moebius
// forward; caching the last sixth or all of the inputs gains less. Re-checked
// with scalar-base addressing (three rounds): no tail / last sixth / last third
// give Moebius bwd 346 / 336 / 324 us, fwd 196 / 197 / 199 us, step 0.913-0.917
// / 0.905-0.907 / 0.896-0.897 ms.
int64_t cached_tail_from(Shape s, int64_t tensors) {
  const int64_t per_step = s.batch * s.lanes * tensors * 4;
  if (per_step <= 0) return 0;
  const int64_t tail_steps = kCachedOutputBytes / per_step;
  return tail_steps >= s.steps ? 0 : s.steps - tail_steps;
}

template <class T>
Geom make_geom(Shape s) {
  return make_geom(s, T::W, T::S, T::V);
}

// Workspace words of one tile shape: header, then K aggregate planes and one
// carry plane, each n_chunks * plane words.
int64_t words_for(Shape s, int W, int S, int V, int K) {
  const Geom g = make_geom(s, W, S, V);
  return sadd(kHeaderWords, smul(K + 1, smul(g.n_chunks, g.plane)));
}

template <class T>
int64_t words_for(Shape s, int K) {
  return words_for(s, T::W, T::S, T::V, K);
}

// Bytes of workspace a scan kind needs: the largest over the shapes it may run
// (0 for an unknown kind or a size that saturates).
size_t workspace_bytes_kind(int kind, Shape s) {
  int64_t w = 0;
  switch (kind) {
    case KLA_SCAN_MOBIUS_FWD:
      w = words_for<MobiusFwdTile>(s, 4);
      break;
    case KLA_SCAN_MOBIUS_BWD:
      w = words_for<MobiusBwdTile>(s, 2);
      break;
    case KLA_SCAN_AFFINE_FWD:
      w = std::max(std::max(words_for<AffineFwdTile>(s, 2), words_for<AffineFwdCachedTile>(s, 2)),
                   std::max(words_for<AffineFwdBf16Tile>(s, 2), words_for<AffineBf16Fallback>(s, 2)));
      break;
    case KLA_SCAN_AFFINE_BWD:
      w = std::max(words_for<AffineBwdTile>(s, 2),
                   std::max(words_for<AffineBwdBf16Tile>(s, 2), words_for<AffineBf16Fallback>(s, 2)));
      break;
    default:
      return 0;
  }
  const int64_t bytes = smul(w, sizeof(uint64_t));
  return bytes >= kHuge ? 0 : static_cast<size_t>(bytes);
}

bool empty(Shape s) { return s.batch == 0 || s.steps == 0 || s.lanes == 0; }

template <class T>
bool misaligned(const T *p) {
  return (reinterpret_cast<uintptr_t>(p) % alignof(T)) != 0;
}
bool misaligned_bytes(const void *p, size_t a) { return (reinterpret_cast<uintptr_t>(p) % a) != 0; }

int check_launch(const char *fn, int kind, Shape s, void *ws, size_t ws_bytes) {
  // The largest grid any shape of this kind launches: the V = 1 shapes have
  // the most tiles, the shortest chunks the most chunks.
  const Geom g1 = make_geom(s, 8, 8, 1);
  const int64_t blocks = smul(g1.n_tiles, g1.n_chunks);
  if (blocks >= (1ll << 31))
    return fail(KLA_ERR_INVALID_ARG, "%s: %lld workgroups exceed the grid limit", fn, (long long)blocks);
  if (ws == nullptr) return fail(KLA_ERR_WORKSPACE, "%s: workspace is NULL", fn);
  if (misaligned_bytes(ws, 256)) return fail(KLA_ERR_WORKSPACE, "%s: workspace not 256-byte aligned", fn);
  const size_t need = workspace_bytes_kind(kind, s);
  if (need == 0) return fail(KLA_ERR_INVALID_ARG, "%s: problem too large", fn);
  if (ws_bytes < need)
    return fail(KLA_ERR_WORKSPACE, "%s: workspace of %zu bytes, %zu needed", fn, ws_bytes, need);
  return KLA_OK;
}

int hip_status(const char *fn, hipError_t e) {
  if (e != hipSuccess) return fail(KLA_ERR_HIP, "%s: %s", fn, hipGetErrorString(e));
  return KLA_OK;
}

// Look-back records: carries only (no chunk aggregates) when one chunk of every
// tile together moves at least this many HBM bytes, i.e. several microseconds
// of streaming per hop of the carry chain (about 0.5 us). Measured per kernel
// (us, aggregates -> carries only): (8, 4096, 2048) Moebius fwd 197 -> 190, bwd
// 366 -> 361, affine fwd 140 -> 137, bwd 215 -> 213; at 12.6 MB per chunk row
// ((4, 4096, 2048), (8, 4096, 1024), (16, 4096, 512)) Moebius fwd 100-104 ->
// 97-99; at 6.3 MB ((2, 4096, 2048), (2, 8192, 2048)) 57-58 -> 62 and 105 -> 114,
// and (1, 65536, 64) Moebius fwd 152 -> 577, (4, 4096, 256) 33 -> 56, where the
// chain is the critical path.
constexpr int64_t kCarryOnlyRowBytes = 8ll << 20;

template <class P, class T>
int launch(const char *fn, const typename P::Params &prm, Shape s, void *ws, hipStream_t stream) {
  Geom g = make_geom<T>(s);
  const int64_t row_bytes = smul(smul(g.plane, T::W * T::S), P::BYTES);
  g.carry_only = row_bytes >= kCarryOnlyRowBytes ? 1 : 0;
  const int64_t grid = g.n_tiles * g.n_chunks;
  hipLaunchKernelGGL((lookback_scan_kernel<P, T::W, T::S, T::V>), dim3(static_cast<uint32_t>(grid)),
                     dim3(kWave * T::W), 0, stream, prm, g, static_cast<uint64_t *>(ws));
  return hip_status(fn, hipGetLastError());
}

// True when every non-NULL pointer is aligned to `bytes`.
bool all_aligned(size_t bytes, std::initializer_list<const void *> ptrs) {
  for (const void *p : ptrs)
    if (p != nullptr && misaligned_bytes(p, bytes)) return false;
  return true;
}

int zero_state(const char *fn, float *p, int64_t count, hipStream_t stream) {
  if (p == nullptr || count == 0) return KLA_OK;
  const int64_t blocks = (count + 255) / 256;
  hipLaunchKernelGGL(fill_zero_kernel, dim3(static_cast<uint32_t>(blocks)), dim3(256), 0, stream, p,
                     count);
  return hip_status(fn, hipGetLastError());
}

// ----------------------------------------------------------- fused scan

// The fused kernels and the decode steps hold a channel's S state lanes in one
// 256-thread workgroup.
constexpr int kMaxFusedState = kFusedThreads;

// State lanes per channel in the fused kernels: S rounded up to a power of two,
// at least 4 (S <= kMaxFusedState, so at most one 256-thread workgroup).
int sp_of(int64_t S) {
  int sp = 4;
  while (sp < S) sp *= 2;
  return sp;
}

FusedGeom fused_geom(int64_t batch, int64_t steps, int64_t M, int64_t S) {
  FusedGeom g;
  g.batch = batch;
  g.steps = steps;
  g.M = M;
  g.S = S;
  const int64_t ch = kFusedThreads / sp_of(S);
  g.groups = (M + ch - 1) / ch;
  g.n_ck = (steps + kCkpt - 1) / kCkpt;
  return g;
}

// Partials of the fused backward: part_k, part_q [B, L, G, S]; part_a, part_p [B, M, S]
// (kHuge when that saturates).
int64_t fused_workspace_floats(const FusedGeom &g) {
  return sadd(smul(2, smul(smul(g.batch, g.steps), smul(g.groups, g.S))), smul(2, smul(g.batch, smul(g.M, g.S))));
}

int check_fused_shape(const char *fn, int64_t batch, int64_t steps, int64_t M, int64_t S) {
  if (batch < 0 || steps < 0 || M < 0 || S < 0)
    return fail(KLA_ERR_INVALID_ARG, "%s: negative size (batch=%lld steps=%lld M=%lld S=%lld)", fn,
                (long long)batch, (long long)steps, (long long)M, (long long)S);
  if (S > kMaxFusedState)
    return fail(KLA_ERR_INVALID_ARG, "%s: d_state S=%lld above %d", fn, (long long)S, kMaxFusedState);
  if (batch > (1ll << 31) || steps > (1ll << 31) || M > (1ll << 31))
    return fail(KLA_ERR_INVALID_ARG, "%s: dimension above 2^31", fn);
  return KLA_OK;
}

// f(std::integral_constant<int, sp_of(S)>) for S validated to at most MAX_SP
// (kernels that serve at most 64 lanes per channel instantiate no wider copy).
template <int MAX_SP = kMaxFusedState, class F>
int with_sp(int64_t S, F &&f) {
  switch (sp_of(S)) {
    case 4: return f(std::integral_constant<int, 4>{});
    case 8: return f(std::integral_constant<int, 8>{});
    case 16: return f(std::integral_constant<int, 16>{});
    case 32: return f(std::integral_constant<int, 32>{});
    case 64: return f(std::integral_constant<int, 64>{});
    default: break;
  }
  if constexpr (MAX_SP >= 256) {
    if (sp_of(S) > 128) return f(std::integral_constant<int, 256>{});
  }
  if constexpr (MAX_SP >= 128) return f(std::integral_constant<int, 128>{});
  return f(std::integral_constant<int, 64>{});
}

template <class F>
int with_k(int64_t K, F &&f) {
  switch (K) {
    case 1: return f(std::integral_constant<int, 1>{});
    case 2: return f(std::integral_constant<int, 2>{});
    case 3: return f(std::integral_constant<int, 3>{});
    case 4: return f(std::integral_constant<int, 4>{});
    case 5: return f(std::integral_constant<int, 5>{});
    case 6: return f(std::integral_constant<int, 6>{});
    case 7: return f(std::integral_constant<int, 7>{});
    default: return f(std::integral_constant<int, 8>{});
  }
}

// Time chunks of the conv kernels (no overflow for any nonnegative L).
int64_t conv_chunks(int64_t L) { return L / kConvT + (L % kConvT != 0); }

int check_conv_shape(const char *fn, int dtype, int64_t B, int64_t L, int64_t D, int64_t K, int act) {
  if (dtype != KLA_DTYPE_F32 && dtype != KLA_DTYPE_BF16) return fail(KLA_ERR_DTYPE, "%s: unsupported dtype code %d", fn, dtype);
  if (B < 0 || L < 0 || D < 0) return fail(KLA_ERR_INVALID_ARG, "%s: negative size", fn);
  if (K < 1 || K > kConvMaxK) return fail(KLA_ERR_INVALID_ARG, "%s: kernel_size %lld outside [1, %d]", fn, (long long)K, kConvMaxK);
  if (B > 65535 || conv_chunks(L) > 65535 || D > (1ll << 31))
    return fail(KLA_ERR_INVALID_ARG, "%s: batch, steps / %d or channels out of range", fn, kConvT);
  if (act < kActNone || act > kActRelu)
    return fail(KLA_ERR_INVALID_ARG, "%s: activation must be 0 (none), 1 (silu), 2 (gelu) or 3 (relu)", fn);
  return KLA_OK;
}


// The row-block reduce for many short rows (outer large, inner a power of two up
// to 256); false when the shape does not suit it.
bool launch_reduce_rows(const float *in, float *out, int64_t outer, int64_t G, int64_t inner, hipStream_t stream) {
  if (outer == 1 && G >= 4 && inner < (1ll << 37)) {
    // One output row: split the rows across phases as well as the columns.
    hipLaunchKernelGGL(reduce_cols_kernel, dim3(static_cast<uint32_t>((inner + 63) / 64)), dim3(1024), 0, stream, in,
                       out, G, inner);
    return true;
  }
  if (outer < 256 || outer >= (1ll << 31)) return false;
  if (inner >= 4 && inner <= 256 && all_aligned(16, {in, out})) {
    // The same sums with one wave per row block (reduce_rows_wave_kernel).
    const dim3 wgrid(static_cast<uint32_t>((outer + 3) / 4));
    switch (inner) {
      case 4: hipLaunchKernelGGL(reduce_rows_wave_kernel<4>, wgrid, dim3(256), 0, stream, in, out, outer, G); return true;
      case 8: hipLaunchKernelGGL(reduce_rows_wave_kernel<8>, wgrid, dim3(256), 0, stream, in, out, outer, G); return true;
      case 16: hipLaunchKernelGGL(reduce_rows_wave_kernel<16>, wgrid, dim3(256), 0, stream, in, out, outer, G); return true;
      case 32: hipLaunchKernelGGL(reduce_rows_wave_kernel<32>, wgrid, dim3(256), 0, stream, in, out, outer, G); return true;
      case 64: hipLaunchKernelGGL(reduce_rows_wave_kernel<64>, wgrid, dim3(256), 0, stream, in, out, outer, G); return true;
      case 128: hipLaunchKernelGGL(reduce_rows_wave_kernel<128>, wgrid, dim3(256), 0, stream, in, out, outer, G); return true;
      case 256: hipLaunchKernelGGL(reduce_rows_wave_kernel<256>, wgrid, dim3(256), 0, stream, in, out, outer, G); return true;
      default: break;
    }
  }
  const dim3 grid(static_cast<uint32_t>(outer));
  switch (inner) {
    case 1: hipLaunchKernelGGL(reduce_rows_kernel<1>, grid, dim3(256), 0, stream, in, out, G); return true;
    case 2: hipLaunchKernelGGL(reduce_rows_kernel<2>, grid, dim3(256), 0, stream, in, out, G); return true;
    case 4: hipLaunchKernelGGL(reduce_rows_kernel<4>, grid, dim3(256), 0, stream, in, out, G); return true;
    case 8: hipLaunchKernelGGL(reduce_rows_kernel<8>, grid, dim3(256), 0, stream, in, out, G); return true;
    case 16: hipLaunchKernelGGL(reduce_rows_kernel<16>, grid, dim3(256), 0, stream, in, out, G); return true;
    case 32: hipLaunchKernelGGL(reduce_rows_kernel<32>, grid, dim3(256), 0, stream, in, out, G); return true;
    case 64: hipLaunchKernelGGL(reduce_rows_kernel<64>, grid, dim3(256), 0, stream, in, out, G); return true;
    case 128: hipLaunchKernelGGL(reduce_rows_kernel<128>, grid, dim3(256), 0, stream, in, out, G); return true;
    case 256: hipLaunchKernelGGL(reduce_rows_kernel<256>, grid, dim3(256), 0, stream, in, out, G); return true;
    default: return false;
  }
}

// f(std::bool_constant<b>...) for runtime flags b...: one instantiation per combination.
template <class F>
void with_flags(F &&f) {
  f();
}

template <class F, class... Bs>
void with_flags(F &&f, bool b, Bs... rest) {
  if (b)
    with_flags([&](auto... c) { f(std::true_type{}, c...); }, rest...);
  else
    with_flags([&](auto... c) { f(std::false_type{}, c...); }, rest...);
}

// SensorIn of dense fp32 v, lambda_v [batch, steps, M].
SensorIn dense_sensors(const float *v, const float *lambda_v, int64_t M) {
  return SensorIn{v, lambda_v, M, M, 0, 0, 0.0f, 0.0f};
}

// Checks a kla_sensors descriptor and turns it into the kernels' SensorIn.
int sensors_from(const char *fn, const kla_sensors *in, int64_t M, SensorIn *out) {
  if (!in) return fail(KLA_ERR_INVALID_ARG, "%s: sensors is NULL", fn);
  if (in->dtype != KLA_DTYPE_F32 && in->dtype != KLA_DTYPE_BF16)
    return fail(KLA_ERR_DTYPE, "%s: unsupported sensor dtype %d", fn, in->dtype);
  if (in->ld_v < M || in->ld_obs < M)
    return fail(KLA_ERR_INVALID_ARG, "%s: row strides (%lld, %lld) below M = %lld", fn,
                static_cast<long long>(in->ld_v), static_cast<long long>(in->ld_obs), static_cast<long long>(M));
  if (in->log_var && !(in->obs_var_max > 0.0f))
    return fail(KLA_ERR_INVALID_ARG, "%s: obs_var_max must be positive (+inf for none)", fn);
  const size_t el = in->dtype == KLA_DTYPE_F32 ? 4 : 2;
  if (misaligned_bytes(in->v, el) || misaligned_bytes(in->obs, el))
    return fail(KLA_ERR_ALIGN, "%s: sensor operand not aligned to its element size", fn);
  *out = SensorIn{in->v, in->obs, in->ld_v, in->ld_obs, in->dtype == KLA_DTYPE_BF16 ? 1 : 0,
                  in->log_var ? 1 : 0, in->obs_var_min, in->obs_var_max};
  return KLA_OK;
}

// Timing events of the fused kernels (kla_set_kernel_events), for the whole
// process: [KLA_KERNEL_FUSED_FWD / _BWD][start, stop]. When set, the fused
// forward or backward records `start` on its stream right before its scan
// kernel and `stop` right after it, so that the pair brackets that kernel
// alone, whichever host thread launches it (torch's autograd launches the
// backward from its own thread).
std::mutex g_events_mu;
hipEvent_t g_kernel_events[2][2] = {};

int record_kernel_event(const char *fn, int kernel, int which, hipStream_t stream) {
  hipEvent_t ev;
  {
    std::lock_guard<std::mutex> lock(g_events_mu);
    ev = g_kernel_events[kernel][which];
  }
  return ev ? hip_status(fn, hipEventRecord(ev, stream)) : KLA_OK;
}

int fused_fwd(const char *fn, const SensorIn &sn, const float *k, const float *q, const float *a, const float *p,
              const float *lam0, const float *eta0, float *y, float *y_var, float *lam_fin, float *eta_fin,
              float *ck_lam, float *ck_eta, int decode_from_prior, int64_t batch, int64_t steps, int64_t M,
              int64_t S, hipStream_t stream) {
  int rc = check_fused_shape(fn, batch, steps, M, S);
  if (rc != KLA_OK) return rc;
  if (batch == 0 || M == 0 || S == 0) return KLA_OK;
  if (!a || !p || !lam_fin || !eta_fin)
    return fail(KLA_ERR_INVALID_ARG, "%s: a, p, lam_fin and eta_fin must not be NULL", fn);
  if (steps > 0 && (!sn.v || !sn.lv || !k || !q || !y))
    return fail(KLA_ERR_INVALID_ARG, "%s: v, lambda_v, k, q and y must not be NULL", fn);
  if ((ck_lam == nullptr) != (ck_eta == nullptr))
    return fail(KLA_ERR_INVALID_ARG, "%s: pass both checkpoint buffers or neither", fn);
  if (!all_aligned(4, {k, q, a, p, lam0, eta0, y, y_var, lam_fin, eta_fin, ck_lam, ck_eta}))
    return fail(KLA_ERR_ALIGN, "%s: fp32 operand not 4-byte aligned", fn);
  const FusedGeom g = fused_geom(batch, steps, M, S);
  const int64_t grid = batch * g.groups;
  if (grid >= (1ll << 31)) return fail(KLA_ERR_INVALID_ARG, "%s: grid too large", fn);
  const FusedFwdParams prm{sn, k, q, a, p, lam0, eta0, y, y_var, lam_fin, eta_fin, ck_lam, ck_eta};
  if ((rc = record_kernel_event(fn, KLA_KERNEL_FUSED_FWD, 0, stream)) != KLA_OK) return rc;
  rc = with_sp(S, [&](auto sp) {
    constexpr int SP = decltype(sp)::value;
    auto run = [&](auto prior, auto bf16, auto var) {
      hipLaunchKernelGGL(
          (fused_kla_fwd_kernel<SP, decltype(prior)::value, decltype(bf16)::value, decltype(var)::value>),
          dim3(static_cast<uint32_t>(grid)), dim3(kFusedThreads), 0, stream, prm, g);
    };
    with_flags(run, decode_from_prior != 0, sn.bf16 != 0, y_var != nullptr);
    return hip_status(fn, hipGetLastError());
  });
  if (rc != KLA_OK) return rc;
  return record_kernel_event(fn, KLA_KERNEL_FUSED_FWD, 1, stream);
}

int fused_bwd(const char *fn, const float *dy, const float *dy_var, const float *dlam_fin, const float *deta_fin,
              const SensorIn &sn, const float *k, const float *q, const float *a, const float *p,
              const float *ck_lam, const float *ck_eta, void *dv, void *dlambda_v, float *dk, float *dq, float *da,
              float *dp, float *dlam0, float *deta0, int decode_from_prior, int64_t batch, int64_t steps, int64_t M,
              int64_t S, void *workspace, size_t workspace_bytes, hipStream_t stream) {
  int rc = check_fused_shape(fn, batch, steps, M, S);
  if (rc != KLA_OK) return rc;
  if (M == 0 || S == 0) return KLA_OK;
  if (!a || !p || !da || !dp) return fail(KLA_ERR_INVALID_ARG, "%s: a, p, da and dp must not be NULL", fn);
  if (steps > 0 && (!dy || !sn.v || !sn.lv || !k || !q || !ck_lam || !ck_eta || !dv || !dlambda_v || !dk || !dq))
    return fail(KLA_ERR_INVALID_ARG,
                "%s: dy, v, lambda_v, k, q, checkpoints, dv, dlambda_v, dk and dq must not be NULL", fn);
  if (!all_aligned(4, {dy, dy_var, dlam_fin, deta_fin, k, q, a, p, ck_lam, ck_eta, dk, dq, da, dp, dlam0, deta0}))
    return fail(KLA_ERR_ALIGN, "%s: fp32 operand not 4-byte aligned", fn);
  if (misaligned_bytes(dv, sn.bf16 ? 2 : 4) || misaligned_bytes(dlambda_v, sn.bf16 ? 2 : 4))
    return fail(KLA_ERR_ALIGN, "%s: sensor gradient not aligned to its element size", fn);
  const FusedGeom g = fused_geom(batch, steps, M, S);
  if (workspace == nullptr) return fail(KLA_ERR_WORKSPACE, "%s: workspace is NULL", fn);
  if (misaligned_bytes(workspace, 256)) return fail(KLA_ERR_WORKSPACE, "%s: workspace not 256-byte aligned", fn);
  const int64_t need_floats = fused_workspace_floats(g);
  if (need_floats >= kHuge / 4) return fail(KLA_ERR_INVALID_ARG, "%s: problem too large", fn);
  const size_t need = static_cast<size_t>(need_floats) * sizeof(float);
  if (workspace_bytes < need)
    return fail(KLA_ERR_WORKSPACE, "%s: workspace of %zu bytes, %zu needed", fn, workspace_bytes, need);
  const int64_t grid = batch * g.groups;
  if (grid >= (1ll << 31)) return fail(KLA_ERR_INVALID_ARG, "%s: grid too large", fn);

  float *ws = static_cast<float *>(workspace);
  float *part_k = ws;
  float *part_q = part_k + batch * steps * g.groups * S;
  float *part_a = part_q + batch * steps * g.groups * S;
  float *part_p = part_a + batch * M * S;
  if (batch > 0) {
    const FusedBwdParams prm{dy, dy_var, dlam_fin, deta_fin, sn, k, q, a, p, ck_lam, ck_eta,
                             dv, dlambda_v, dlam0, deta0, part_k, part_q, part_a, part_p};
    if ((rc = record_kernel_event(fn, KLA_KERNEL_FUSED_BWD, 0, stream)) != KLA_OK) return rc;
    rc = with_sp(S, [&](auto sp) {
      constexpr int SP = decltype(sp)::value;
      auto run = [&](auto prior, auto bf16, auto var) {
        hipLaunchKernelGGL(
            (fused_kla_bwd_kernel<SP, decltype(prior)::value, decltype(bf16)::value, decltype(var)::value>),
            dim3(static_cast<uint32_t>(grid)), dim3(kFusedThreads), 0, stream, prm, g);
      };
      with_flags(run, decode_from_prior != 0, sn.bf16 != 0, dy_var != nullptr);
      return hip_status(fn, hipGetLastError());
    });
    if (rc != KLA_OK) return rc;
    if ((rc = record_kernel_event(fn, KLA_KERNEL_FUSED_BWD, 1, stream)) != KLA_OK) return rc;
  }
  // Fixed-order sums of the partials: dk, dq over channel groups; da, dp over batch.
  auto reduce = [&](const float *in, float *out, int64_t outer, int64_t G, int64_t inner) {
    const int64_t n = outer * inner;
    if (n == 0) return KLA_OK;
    if (launch_reduce_rows(in, out, outer, G, inner, stream)) return hip_status(fn, hipGetLastError());
    hipLaunchKernelGGL(reduce_groups_kernel, dim3(static_cast<uint32_t>((n + 255) / 256)), dim3(256), 0, stream,
                       in, out, outer, G, inner);
    return hip_status(fn, hipGetLastError());
  };
  if (steps > 0 && batch > 0) {
    if ((rc = reduce(part_k, dk, batch * steps, g.groups, S)) != KLA_OK) return rc;
    if ((rc = reduce(part_q, dq, batch * steps, g.groups, S)) != KLA_OK) return rc;
  }
  if ((rc = reduce(part_a, da, 1, batch, M * S)) != KLA_OK) return rc;
  return reduce(part_p, dp, 1, batch, M * S);
}

int check_tail(const char *fn, int dtype, const void *res, int64_t ld_res, const void *gate, int64_t ld_gate,
               const float *lam, int act, int64_t rows, int64_t M) {
  if (rows < 0 || M < 0) return fail(KLA_ERR_INVALID_ARG, "%s: negative shape", fn);
  if (dtype != KLA_DTYPE_F32 && dtype != KLA_DTYPE_BF16)
    return fail(KLA_ERR_DTYPE, "%s: unsupported dtype %d", fn, dtype);
  if (act < kActNone || act > kActRelu) return fail(KLA_ERR_INVALID_ARG, "%s: unknown activation %d", fn, act);
  if (res && !lam) return fail(KLA_ERR_INVALID_ARG, "%s: a residual needs lambda_skip", fn);
  if ((res && ld_res < M) || (gate && ld_gate < M))
    return fail(KLA_ERR_INVALID_ARG, "%s: row stride below M", fn);
  const size_t el = dtype == KLA_DTYPE_F32 ? 4 : 2;
  if (misaligned_bytes(res, el) || misaligned_bytes(gate, el))
    return fail(KLA_ERR_ALIGN, "%s: residual or gate not aligned to its element size", fn);
  return KLA_OK;
}

template <class F>
int with_io(int dtype, F &&f) {
  if (dtype == KLA_DTYPE_F32) return f(float{});
  return f(bf16_t{});
}

dim3 tail_grid(int64_t rows, int64_t M, int V) {
  return dim3(static_cast<uint32_t>((rows + kTailRows - 1) / kTailRows),
              static_cast<uint32_t>((M + kTailThreads * V - 1) / (kTailThreads * V)));
}

// The 8-wide tail kernels need every row start 16-byte aligned: M and the row
// strides multiples of 8, and the base pointers 16-byte aligned.
bool tail_wide(int64_t M, int64_t ld_res, int64_t ld_gate, std::initializer_list<const void *> ptrs) {
  if (M % 8 || ld_res % 8 || ld_gate % 8) return false;
  for (const void *q : ptrs)
    if (q && reinterpret_cast<uintptr_t>(q) % 16) return false;
  return true;
}

// Moebius forward after argument checks: `get_ws(&ws, &bytes)` supplies the
// look-back workspace once the call is known to be valid (so an invalid call
// touches nothing, not even a first-use scratch set-up).
template <class GetWs>
int mobius_fwd(const char *fn, const float *A, const float *B, const float *C, const float *D, const float *lam0,
               float *lam, int64_t batch, int64_t steps, int64_t lanes, hipStream_t stream, GetWs &&get_ws) {
  const Shape s{batch, steps, lanes};
  int rc = check_shape(fn, s);
  if (rc != KLA_OK) return rc;
  if (empty(s)) return KLA_OK;
  if (!A || !B || !C || !lam) return fail(KLA_ERR_INVALID_ARG, "%s: A, B, C and lam must not be NULL", fn);
  if (misaligned(A) || misaligned(B) || misaligned(C) || misaligned(D) || misaligned(lam0) ||
      misaligned(lam))
    return fail(KLA_ERR_ALIGN, "%s: fp32 operand not 4-byte aligned", fn);
  void *workspace = nullptr;
  size_t workspace_bytes = 0;
  if ((rc = get_ws(&workspace, &workspace_bytes)) != KLA_OK) return rc;
  rc = check_launch(fn, KLA_SCAN_MOBIUS_FWD, s, workspace, workspace_bytes);
  if (rc != KLA_OK) return rc;
  const int64_t from = cached_tail_from(s, D ? 4 : 3);
  if (D) {
    using P = MobiusFwd<true>;
    return launch<P, MobiusFwdTile>(fn, P::Params{A, B, C, D, lam0, lam, from}, s, workspace, stream);
  }
  using P = MobiusFwd<false>;
  return launch<P, MobiusFwdTile>(fn, P::Params{A, B, C, nullptr, lam0, lam, from}, s, workspace, stream);
}

// ------------------------------------------------ allocation-free workspace
//
// kla_mobius_scan_fwd_noalloc keeps its look-back records in `scratch`, a
// file-scope device array: every GPU the library runs on holds its own copy
// until the process ends, and the entry point allocates nothing. On the host
// the array's name is only a stand-in for the device symbol (a kernel given
// it would fault), so host code uses the address hipGetSymbolAddress returns,
// looked up once per device with that device current. All calls on one GPU
// share that GPU's array: calls that overlap in time on one GPU race.
constexpr size_t kScratchBytes = 32ull << 20;
static __device__ __align__(256) uint64_t scratch[kScratchBytes / sizeof(uint64_t)];

constexpr int kMaxDevices = 64;
std::mutex g_scratch_mu;
void *g_scratch_addr[kMaxDevices] = {};

// The current device's scratch address. The first call on a device looks the
// symbol up, zero-fills the array on `stream` (the look-back records' start
// state; the kernels keep it consistent from launch to launch afterwards) and
// waits for the fill, so that no later call, on any stream, can see the array
// before it is filled. Later calls only read the address.
int scratch_address(const char *fn, hipStream_t stream, void **out) {
  int dev = -1;
  int rc = hip_status(fn, hipGetDevice(&dev));
  if (rc != KLA_OK) return rc;
  if (dev < 0 || dev >= kMaxDevices) return fail(KLA_ERR_INVALID_ARG, "%s: device %d beyond %d", fn, dev, kMaxDevices);
  std::lock_guard<std::mutex> lock(g_scratch_mu);
  if (g_scratch_addr[dev] == nullptr) {
    void *p = nullptr;
    rc = hip_status(fn, hipGetSymbolAddress(&p, HIP_SYMBOL(scratch)));
    if (rc != KLA_OK) return rc;
    if (p == nullptr || misaligned_bytes(p, 256)) return fail(KLA_ERR_HIP, "%s: bad scratch address", fn);
    const int64_t count = static_cast<int64_t>(kScratchBytes / sizeof(float));
    hipLaunchKernelGGL(fill_zero_kernel, dim3(static_cast<uint32_t>((count + 255) / 256)), dim3(256), 0, stream,
                       static_cast<float *>(p), count);
    rc = hip_status(fn, hipGetLastError());
    if (rc != KLA_OK) return rc;
    rc = hip_status(fn, hipStreamSynchronize(stream));
    if (rc != KLA_OK) return rc;
    g_scratch_addr[dev] = p;
  }
  *out = g_scratch_addr[dev];
  return KLA_OK;
}

// The current device's scratch address if a no-alloc call has set it up, else NULL.
void *scratch_address_if_set(const char *fn, int *rc) {
  int dev = -1;
  *rc = hip_status(fn, hipGetDevice(&dev));
  if (*rc != KLA_OK) return nullptr;
  if (dev < 0 || dev >= kMaxDevices) {
    *rc = fail(KLA_ERR_INVALID_ARG, "%s: device %d beyond %d", fn, dev, kMaxDevices);
    return nullptr;
  }
  std::lock_guard<std::mutex> lock(g_scratch_mu);
  return g_scratch_addr[dev];
}

}  // namespace

extern "C" {

int kla_hip_abi_version(void) { return kAbiVersion; }

const char *kla_hip_last_error(void) { return g_last_error; }

size_t kla_scan_workspace_bytes(int kind, int64_t batch, int64_t steps, int64_t lanes) {
  const Shape s{batch, steps, lanes};
  if (check_shape("kla_scan_workspace_bytes", s) != KLA_OK) return 0;
  if (kind < KLA_SCAN_MOBIUS_FWD || kind > KLA_SCAN_AFFINE_BWD) {
    fail(KLA_ERR_INVALID_ARG, "kla_scan_workspace_bytes: unknown scan kind %d", kind);
    return 0;
  }
  const size_t bytes = workspace_bytes_kind(kind, s);
  if (bytes == 0) fail(KLA_ERR_INVALID_ARG, "kla_scan_workspace_bytes: problem too large");
  return bytes;
}

int kla_set_kernel_events(int kernel, hipEvent_t start, hipEvent_t stop) {
  if (kernel != KLA_KERNEL_FUSED_FWD && kernel != KLA_KERNEL_FUSED_BWD)
    return fail(KLA_ERR_INVALID_ARG, "kla_set_kernel_events: unknown kernel %d", kernel);
  if ((start == nullptr) != (stop == nullptr))
    return fail(KLA_ERR_INVALID_ARG, "kla_set_kernel_events: pass both events or neither");
  std::lock_guard<std::mutex> lock(g_events_mu);
  g_kernel_events[kernel][0] = start;
  g_kernel_events[kernel][1] = stop;
  return KLA_OK;
}

int kla_workspace_failures(const void *workspace, hipStream_t stream, uint32_t *failures) {
  const char *fn = "kla_workspace_failures";
  if (failures == nullptr) return fail(KLA_ERR_INVALID_ARG, "%s: NULL argument", fn);
  if (workspace == nullptr) {   // the current device's static scratch (kla_mobius_scan_fwd_noalloc)
    int rc = KLA_OK;
    workspace = scratch_address_if_set(fn, &rc);
    if (rc != KLA_OK) return rc;
    if (workspace == nullptr) {   // no allocation-free call has run on this device
      *failures = 0;
      return KLA_OK;
    }
  }
  uint64_t word = 0;
  int rc = hip_status(fn, hipMemcpyAsync(&word, static_cast<const uint64_t *>(workspace) + 1, sizeof(word),
                                         hipMemcpyDeviceToHost, stream));
  if (rc != KLA_OK) return rc;
  rc = hip_status(fn, hipStreamSynchronize(stream));
  if (rc != KLA_OK) return rc;
  *failures = static_cast<uint32_t>(word > 0xFFFFFFFFull ? 0xFFFFFFFFull : word);
  return KLA_OK;
}

int kla_mobius_scan_fwd(const float *A, const float *B, const float *C, const float *D,
                        const float *lam0, float *lam, int64_t batch, int64_t steps,
                        int64_t lanes, void *workspace, size_t workspace_bytes,
                        hipStream_t stream) {
  return mobius_fwd("kla_mobius_scan_fwd", A, B, C, D, lam0, lam, batch, steps, lanes, stream,
                    [&](void **ws, size_t *bytes) {
                      *ws = workspace;
                      *bytes = workspace_bytes;
                      return KLA_OK;
                    });
}

int kla_mobius_scan_fwd_noalloc(const float *A, const float *B, const float *C, const float *D,
                                const float *lam0, float *lam, int64_t batch, int64_t steps,
                                int64_t lanes, hipStream_t stream) {
  const char *fn = "kla_mobius_scan_fwd_noalloc";
  return mobius_fwd(fn, A, B, C, D, lam0, lam, batch, steps, lanes, stream, [&](void **ws, size_t *bytes) {
    const size_t need = workspace_bytes_kind(KLA_SCAN_MOBIUS_FWD, Shape{batch, steps, lanes});
    if (need == 0 || need > kScratchBytes)
      return fail(KLA_ERR_WORKSPACE, "%s: the look-back needs %zu bytes, the static scratch holds %zu", fn, need,
                  kScratchBytes);
    *bytes = kScratchBytes;
    return scratch_address(fn, stream, ws);
  });
}

int kla_mobius_scan_bwd(const float *dlam, const float *A, const float *B, const float *C,
                        const float *D, const float *lam0, const float *lam, float *dA,
                        float *dB, float *dC, float *dD, float *dlam0, int64_t batch,
                        int64_t steps, int64_t lanes, void *workspace,
                        size_t workspace_bytes, hipStream_t stream) {
  const char *fn = "kla_mobius_scan_bwd";
  const Shape s{batch, steps, lanes};
  int rc = check_shape(fn, s);
  if (rc != KLA_OK) return rc;
  if (batch == 0 || lanes == 0) return KLA_OK;
  if (steps == 0) return zero_state(fn, dlam0, batch * lanes, stream);
  if (!dlam || !A || !B || !C || !lam)
    return fail(KLA_ERR_INVALID_ARG, "%s: dlam, A, B, C and lam must not be NULL", fn);
  if (misaligned(dlam) || misaligned(A) || misaligned(B) || misaligned(C) || misaligned(D) ||
      misaligned(lam0) || misaligned(lam) || misaligned(dA) || misaligned(dB) || misaligned(dC) ||
      misaligned(dD) || misaligned(dlam0))
    return fail(KLA_ERR_ALIGN, "%s: fp32 operand not 4-byte aligned", fn);
  rc = check_launch(fn, KLA_SCAN_MOBIUS_BWD, s, workspace, workspace_bytes);
  if (rc != KLA_OK) return rc;
  if (D) {
    using P = MobiusBwd<true>;
    return launch<P, MobiusBwdTile>(fn, P::Params{dlam, A, B, C, D, lam0, lam, dA, dB, dC, dD, dlam0},
                                    s, workspace, stream);
  }
  using P = MobiusBwd<false>;
  return launch<P, MobiusBwdTile>(fn, P::Params{dlam, A, B, C, nullptr, lam0, lam, dA, dB, dC, nullptr, dlam0},
                                  s, workspace, stream);
}

int kla_affine_scan_fwd(int dtype, const void *g, const void *u, const float *h0, void *h,
                        int64_t batch, int64_t steps, int64_t lanes, void *workspace,
                        size_t workspace_bytes, hipStream_t stream) {
  const char *fn = "kla_affine_scan_fwd";
  if (dtype != KLA_DTYPE_F32 && dtype != KLA_DTYPE_BF16)
    return fail(KLA_ERR_DTYPE, "%s: unsupported dtype code %d", fn, dtype);
  const Shape s{batch, steps, lanes};
  int rc = check_shape(fn, s);
  if (rc != KLA_OK) return rc;
  if (empty(s)) return KLA_OK;
  if (!g || !u || !h) return fail(KLA_ERR_INVALID_ARG, "%s: g, u and h must not be NULL", fn);
  const size_t el = dtype == KLA_DTYPE_F32 ? 4 : 2;
  if (misaligned_bytes(g, el) || misaligned_bytes(u, el) || misaligned_bytes(h, el) || misaligned(h0))
    return fail(KLA_ERR_ALIGN, "%s: operand not aligned to its element size", fn);
  rc = check_launch(fn, KLA_SCAN_AFFINE_FWD, s, workspace, workspace_bytes);
  if (rc != KLA_OK) return rc;
  const bool cached = output_fits_cache(s, static_cast<int64_t>(el));
  auto run = [&](auto cached_c) {
    constexpr bool CACHED = decltype(cached_c)::value;
    if (dtype == KLA_DTYPE_F32) {
      using P = AffineFwd<float, CACHED>;
      const typename P::Params prm{static_cast<const float *>(g), static_cast<const float *>(u), h0,
                                   static_cast<float *>(h)};
      using Tile = std::conditional_t<CACHED, AffineFwdCachedTile, AffineFwdTile>;
      return launch<P, Tile>(fn, prm, s, workspace, stream);
    }
    using P = AffineFwd<bf16_t, CACHED>;
    const typename P::Params prm{static_cast<const bf16_t *>(g), static_cast<const bf16_t *>(u), h0,
                                 static_cast<bf16_t *>(h)};
    constexpr int V = AffineFwdBf16Tile::V;
    if (lanes % V == 0 && all_aligned(V * el, {g, u, h}))
      return launch<P, AffineFwdBf16Tile>(fn, prm, s, workspace, stream);
    return launch<P, AffineBf16Fallback>(fn, prm, s, workspace, stream);
  };
  return cached ? run(std::true_type{}) : run(std::false_type{});
}

int kla_affine_scan_bwd(int dtype, const void *dh, const void *g, const void *h,
                        const float *h0, void *dg, void *du, float *dh0, int64_t batch,
                        int64_t steps, int64_t lanes, void *workspace,
                        size_t workspace_bytes, hipStream_t stream) {
  const char *fn = "kla_affine_scan_bwd";
  if (dtype != KLA_DTYPE_F32 && dtype != KLA_DTYPE_BF16)
    return fail(KLA_ERR_DTYPE, "%s: unsupported dtype code %d", fn, dtype);
  const Shape s{batch, steps, lanes};
  int rc = check_shape(fn, s);
  if (rc != KLA_OK) return rc;
  if (batch == 0 || lanes == 0) return KLA_OK;
  if (steps == 0) return zero_state(fn, dh0, batch * lanes, stream);
  if (!dh || !g || !h) return fail(KLA_ERR_INVALID_ARG, "%s: dh, g and h must not be NULL", fn);
  const size_t el = dtype == KLA_DTYPE_F32 ? 4 : 2;
  if (misaligned_bytes(dh, el) || misaligned_bytes(g, el) || misaligned_bytes(h, el) ||
      misaligned_bytes(dg, el) || misaligned_bytes(du, el) || misaligned(h0) || misaligned(dh0))
    return fail(KLA_ERR_ALIGN, "%s: operand not aligned to its element size", fn);
  rc = check_launch(fn, KLA_SCAN_AFFINE_BWD, s, workspace, workspace_bytes);
  if (rc != KLA_OK) return rc;
  if (dtype == KLA_DTYPE_F32) {
    using P = AffineBwd<float>;
    const P::Params prm{static_cast<const float *>(dh), static_cast<const float *>(g),
                        static_cast<const float *>(h), h0, static_cast<float *>(dg),
                        static_cast<float *>(du), dh0};
    return launch<P, AffineBwdTile>(fn, prm, s, workspace, stream);
  }
  using P = AffineBwd<bf16_t>;
  const P::Params prm{static_cast<const bf16_t *>(dh), static_cast<const bf16_t *>(g),
                      static_cast<const bf16_t *>(h), h0, static_cast<bf16_t *>(dg),
                      static_cast<bf16_t *>(du), dh0};
  constexpr int V = AffineBwdBf16Tile::V;
  if (lanes % V == 0 && all_aligned(V * el, {dh, g, h, dg, du}))
    return launch<P, AffineBwdBf16Tile>(fn, prm, s, workspace, stream);
  return launch<P, AffineBf16Fallback>(fn, prm, s, workspace, stream);
}

int64_t kla_fused_checkpoints(int64_t steps) { return steps < 0 ? 0 : (steps + kCkpt - 1) / kCkpt; }

size_t kla_fused_workspace_bytes(int64_t batch, int64_t steps, int64_t M, int64_t S) {
  if (check_fused_shape("kla_fused_workspace_bytes", batch, steps, M, S) != KLA_OK) return 0;
  const int64_t floats = fused_workspace_floats(fused_geom(batch, steps, M, S));
  if (floats >= kHuge / 4) {
    fail(KLA_ERR_INVALID_ARG, "kla_fused_workspace_bytes: problem too large");
    return 0;
  }
  return std::max<size_t>(256, static_cast<size_t>(floats) * sizeof(float));
}

int kla_fused_scan_fwd(const float *v, const float *lambda_v, const float *k, const float *q,
                       const float *a, const float *p, const float *lam0, const float *eta0, float *y,
                       float *y_var, float *lam_fin, float *eta_fin, float *ck_lam, float *ck_eta,
                       int decode_from_prior, int64_t batch, int64_t steps, int64_t M, int64_t S,
                       hipStream_t stream) {
  const char *fn = "kla_fused_scan_fwd";
  if (!all_aligned(4, {v, lambda_v})) return fail(KLA_ERR_ALIGN, "%s: fp32 operand not 4-byte aligned", fn);
  return fused_fwd(fn, dense_sensors(v, lambda_v, M), k, q, a, p, lam0, eta0, y, y_var, lam_fin, eta_fin,
                   ck_lam, ck_eta, decode_from_prior, batch, steps, M, S, stream);
}

int kla_fused_scan_sensors_fwd(const kla_sensors *sensors, const float *k, const float *q, const float *a,
                               const float *p, const float *lam0, const float *eta0, float *y, float *y_var,
                               float *lam_fin, float *eta_fin, float *ck_lam, float *ck_eta,
                               int decode_from_prior, int64_t batch, int64_t steps, int64_t M, int64_t S,
                               hipStream_t stream) {
  const char *fn = "kla_fused_scan_sensors_fwd";
  SensorIn sn;
  const int rc = sensors_from(fn, sensors, M, &sn);
  if (rc != KLA_OK) return rc;
  return fused_fwd(fn, sn, k, q, a, p, lam0, eta0, y, y_var, lam_fin, eta_fin, ck_lam, ck_eta,
                   decode_from_prior, batch, steps, M, S, stream);
}

int kla_fused_scan_bwd(const float *dy, const float *dy_var, const float *dlam_fin, const float *deta_fin,
                       const float *v, const float *lambda_v, const float *k, const float *q,
                       const float *a, const float *p, const float *ck_lam, const float *ck_eta,
                       float *dv, float *dlambda_v, float *dk, float *dq, float *da, float *dp,
                       float *dlam0, float *deta0, int decode_from_prior, int64_t batch, int64_t steps,
                       int64_t M, int64_t S, void *workspace, size_t workspace_bytes,
                       hipStream_t stream) {
  const char *fn = "kla_fused_scan_bwd";
  if (!all_aligned(4, {v, lambda_v})) return fail(KLA_ERR_ALIGN, "%s: fp32 operand not 4-byte aligned", fn);
  return fused_bwd(fn, dy, dy_var, dlam_fin, deta_fin, dense_sensors(v, lambda_v, M), k, q, a, p, ck_lam, ck_eta,
                   dv, dlambda_v, dk, dq, da, dp, dlam0, deta0, decode_from_prior, batch, steps, M, S, workspace,
                   workspace_bytes, stream);
}

int kla_fused_scan_sensors_bwd(const float *dy, const float *dy_var, const float *dlam_fin,
                               const float *deta_fin, const kla_sensors *sensors, const float *k,
                               const float *q, const float *a, const float *p, const float *ck_lam,
                               const float *ck_eta, void *dv, void *dobs, float *dk, float *dq, float *da,
                               float *dp, float *dlam0, float *deta0, int decode_from_prior, int64_t batch,
                               int64_t steps, int64_t M, int64_t S, void *workspace, size_t workspace_bytes,
                               hipStream_t stream) {
  const char *fn = "kla_fused_scan_sensors_bwd";
  SensorIn sn;
  const int rc = sensors_from(fn, sensors, M, &sn);
  if (rc != KLA_OK) return rc;
  return fused_bwd(fn, dy, dy_var, dlam_fin, deta_fin, sn, k, q, a, p, ck_lam, ck_eta, dv, dobs, dk, dq, da, dp,
                   dlam0, deta0, decode_from_prior, batch, steps, M, S, workspace, workspace_bytes, stream);
}

int kla_fused_chunk_maps(const kla_sensors *sensors, const float *k, const float *a, const float *p, float *maps,
                         int64_t batch, int64_t steps, int64_t M, int64_t S, hipStream_t stream) {
  const char *fn = "kla_fused_chunk_maps";
  int rc = check_fused_shape(fn, batch, steps, M, S);
  if (rc != KLA_OK) return rc;
  SensorIn sn;
  if ((rc = sensors_from(fn, sensors, M, &sn)) != KLA_OK) return rc;
  if (batch == 0 || M == 0 || S == 0) return KLA_OK;
  if (!a || !p || !maps) return fail(KLA_ERR_INVALID_ARG, "%s: a, p and maps must not be NULL", fn);
  if (steps > 0 && (!sn.v || !sn.lv || !k))
    return fail(KLA_ERR_INVALID_ARG, "%s: the sensors and k must not be NULL", fn);
  if (!all_aligned(4, {k, a, p})) return fail(KLA_ERR_ALIGN, "%s: fp32 operand not 4-byte aligned", fn);
  if (!all_aligned(16, {maps})) return fail(KLA_ERR_ALIGN, "%s: maps not 16-byte aligned", fn);
  const FusedGeom g = fused_geom(batch, steps, M, S);
  const int64_t grid = smul(batch, g.groups);
  if (grid >= (1ll << 31)) return fail(KLA_ERR_INVALID_ARG, "%s: grid too large", fn);
  const ChunkMapParams prm{sn, k, a, p, maps};
  return with_sp(S, [&](auto sp) {
    constexpr int SP = decltype(sp)::value;
    if (sn.bf16)
      hipLaunchKernelGGL((fused_chunk_map_kernel<SP, true>), dim3(static_cast<uint32_t>(grid)), dim3(kFusedThreads),
                         0, stream, prm, g);
    else
      hipLaunchKernelGGL((fused_chunk_map_kernel<SP, false>), dim3(static_cast<uint32_t>(grid)), dim3(kFusedThreads),
                         0, stream, prm, g);
    return hip_status(fn, hipGetLastError());
  });
}

int kla_chunk_starts(const float *maps, const float *lam0, const float *eta0, float *lam_start, float *eta_start,
                     float *lam_end, float *eta_end, int64_t batch, int64_t chunks, int64_t M, int64_t S,
                     hipStream_t stream) {
  const char *fn = "kla_chunk_starts";
  if (batch < 0 || chunks < 0 || M < 0 || S < 0) return fail(KLA_ERR_INVALID_ARG, "%s: negative size", fn);
  const int64_t n = smul(M, S);
  const int64_t lanes = smul(batch, n);
  if (lanes >= (1ll << 40) || chunks > (1ll << 31)) return fail(KLA_ERR_INVALID_ARG, "%s: problem too large", fn);
  if (lanes == 0 || chunks == 0) return KLA_OK;
  if (!maps || !lam_start || !eta_start)
    return fail(KLA_ERR_INVALID_ARG, "%s: maps, lam_start and eta_start must not be NULL", fn);
  if (!lam_end != !eta_end) return fail(KLA_ERR_INVALID_ARG, "%s: lam_end and eta_end go together", fn);
  if (!all_aligned(4, {lam0, eta0, lam_start, eta_start, lam_end, eta_end}))
    return fail(KLA_ERR_ALIGN, "%s: fp32 operand not 4-byte aligned", fn);
  if (!all_aligned(16, {maps})) return fail(KLA_ERR_ALIGN, "%s: maps not 16-byte aligned", fn);
  hipLaunchKernelGGL(chunk_starts_kernel, dim3(static_cast<uint32_t>((lanes + 255) / 256)), dim3(256), 0, stream, maps,
                     lam0, eta0, lam_start, eta_start, lam_end, eta_end, batch, chunks, n);
  return hip_status(fn, hipGetLastError());
}

int kla_fused_adjoint_maps(const float *dy, const float *dy_var, const kla_sensors *sensors, const float *k,
                           const float *q, const float *a, const float *p, const float *ck_lam, const float *ck_eta,
                           float *maps, int decode_from_prior, int64_t batch, int64_t steps, int64_t M, int64_t S,
                           hipStream_t stream) {
  const char *fn = "kla_fused_adjoint_maps";
  int rc = check_fused_shape(fn, batch, steps, M, S);
  if (rc != KLA_OK) return rc;
  SensorIn sn;
  if ((rc = sensors_from(fn, sensors, M, &sn)) != KLA_OK) return rc;
  if (batch == 0 || M == 0 || S == 0) return KLA_OK;
  if (!a || !p || !maps) return fail(KLA_ERR_INVALID_ARG, "%s: a, p and maps must not be NULL", fn);
  if (steps > 0 && (!dy || !sn.v || !sn.lv || !k || !q || !ck_lam || !ck_eta))
    return fail(KLA_ERR_INVALID_ARG, "%s: dy, the sensors, k, q and the checkpoints must not be NULL", fn);
  if (!all_aligned(4, {dy, dy_var, k, q, a, p, ck_lam, ck_eta}))
    return fail(KLA_ERR_ALIGN, "%s: fp32 operand not 4-byte aligned", fn);
  if (!all_aligned(16, {maps})) return fail(KLA_ERR_ALIGN, "%s: maps not 16-byte aligned", fn);
  const FusedGeom g = fused_geom(batch, steps, M, S);
  const int64_t grid = smul(batch, g.groups);
  if (grid >= (1ll << 31)) return fail(KLA_ERR_INVALID_ARG, "%s: grid too large", fn);
  const AdjointMapParams prm{dy, dy_var, sn, k, q, a, p, ck_lam, ck_eta, maps};
  return with_sp(S, [&](auto sp) {
    constexpr int SP = decltype(sp)::value;
    auto run = [&](auto prior, auto bf16, auto var) {
      hipLaunchKernelGGL(
          (fused_adjoint_map_kernel<SP, decltype(prior)::value, decltype(bf16)::value, decltype(var)::value>),
          dim3(static_cast<uint32_t>(grid)), dim3(kFusedThreads), 0, stream, prm, g);
    };
    with_flags(run, decode_from_prior != 0, sn.bf16 != 0, dy_var != nullptr);
    return hip_status(fn, hipGetLastError());
  });
}

int kla_adjoint_ends(const float *maps, const float *dlam_fin, const float *deta_fin, float *gl_end, float *ge_end,
                     int64_t batch, int64_t chunks, int64_t M, int64_t S, hipStream_t stream) {
  const char *fn = "kla_adjoint_ends";
  if (batch < 0 || chunks < 0 || M < 0 || S < 0) return fail(KLA_ERR_INVALID_ARG, "%s: negative size", fn);
  const int64_t n = smul(M, S);
  const int64_t lanes = smul(batch, n);
  if (lanes >= (1ll << 40) || chunks > (1ll << 31)) return fail(KLA_ERR_INVALID_ARG, "%s: problem too large", fn);
  if (lanes == 0 || chunks == 0) return KLA_OK;
  if (!maps || !gl_end || !ge_end)
    return fail(KLA_ERR_INVALID_ARG, "%s: maps, gl_end and ge_end must not be NULL", fn);
  if (!all_aligned(4, {dlam_fin, deta_fin, gl_end, ge_end}))
    return fail(KLA_ERR_ALIGN, "%s: fp32 operand not 4-byte aligned", fn);
  if (!all_aligned(16, {maps})) return fail(KLA_ERR_ALIGN, "%s: maps not 16-byte aligned", fn);
  hipLaunchKernelGGL(adjoint_ends_kernel, dim3(static_cast<uint32_t>((lanes + 255) / 256)), dim3(256), 0, stream, maps,
                     dlam_fin, deta_fin, gl_end, ge_end, batch, chunks, n);
  return hip_status(fn, hipGetLastError());
}

int kla_step_fwd(const float *v, const float *lambda_v, const float *k, const float *q, const float *a,
                 const float *p, const float *lam, const float *eta, float *y, float *y_var, float *lam_out,
                 float *eta_out, int decode_from_prior, int64_t batch, int64_t M, int64_t S, hipStream_t stream) {
  const char *fn = "kla_step_fwd";
  int rc = check_fused_shape(fn, batch, 1, M, S);
  if (rc != KLA_OK) return rc;
  if (batch == 0 || M == 0 || S == 0) return KLA_OK;
  if (!v || !lambda_v || !k || !q || !a || !p || !lam || !eta || !y || !y_var || !lam_out || !eta_out)
    return fail(KLA_ERR_INVALID_ARG, "%s: NULL operand", fn);
  if (!all_aligned(4, {v, lambda_v, k, q, a, p, lam, eta, y, y_var, lam_out, eta_out}))
    return fail(KLA_ERR_ALIGN, "%s: fp32 operand not 4-byte aligned", fn);
  const FusedGeom g = fused_geom(batch, 1, M, S);
  const int64_t grid = batch * g.groups;
  if (grid >= (1ll << 31)) return fail(KLA_ERR_INVALID_ARG, "%s: grid too large", fn);
  const StepParams prm{v, lambda_v, k, q, a, p, lam, eta, y, y_var, lam_out, eta_out};
  return with_sp(S, [&](auto sp) {
    constexpr int SP = decltype(sp)::value;
    if (decode_from_prior)
      hipLaunchKernelGGL((kla_step_kernel<SP, true>), dim3(static_cast<uint32_t>(grid)), dim3(kFusedThreads), 0,
                         stream, prm, g);
    else
      hipLaunchKernelGGL((kla_step_kernel<SP, false>), dim3(static_cast<uint32_t>(grid)), dim3(kFusedThreads), 0,
                         stream, prm, g);
    return hip_status(fn, hipGetLastError());
  });
}

int kla_decode_step_fwd(const float *v, int64_t ld_v, const float *log_var, int64_t ld_log_var, const float *k,
                        const float *q, int64_t ld_kq, const float *residual, int64_t ld_residual,
                        const float *lambda_skip, const float *gate, int64_t ld_gate, const float *delta,
                        const float *lambda_log, const float *process_noise, const float *lam, const float *eta,
                        float *lam_out, float *eta_out, float *y, float *y_var, const kla_decode_config *cfg,
                        int64_t batch, int64_t M, int64_t S, hipStream_t stream) {
  const char *fn = "kla_decode_step_fwd";
  if (!cfg) return fail(KLA_ERR_INVALID_ARG, "%s: cfg must not be NULL", fn);
  int rc = check_fused_shape(fn, batch, 1, M, S);
  if (rc != KLA_OK) return rc;
  if (batch == 0 || M == 0 || S == 0) return KLA_OK;
  if (!v || !log_var || !k || !q || !delta || !lambda_log || !process_noise || !lam || !eta || !lam_out ||
      !eta_out || !y || !y_var)
    return fail(KLA_ERR_INVALID_ARG, "%s: NULL operand", fn);
  if ((residual == nullptr) != (lambda_skip == nullptr))
    return fail(KLA_ERR_INVALID_ARG, "%s: pass both residual and lambda_skip or neither", fn);
  if (ld_v < M || ld_log_var < M || ld_kq < S || (residual && ld_residual < M) || (gate && ld_gate < M))
    return fail(KLA_ERR_INVALID_ARG, "%s: row stride below the row length", fn);
  if (cfg->discretization != 0 && cfg->discretization != 1)
    return fail(KLA_ERR_INVALID_ARG, "%s: discretization must be 0 (ou) or 1 (zoh)", fn);
  if (gate && (cfg->gate_activation < kActSilu || cfg->gate_activation > kActRelu))
    return fail(KLA_ERR_INVALID_ARG, "%s: gate_activation must be 1 (silu), 2 (gelu) or 3 (relu)", fn);
  if (!all_aligned(4, {v, log_var, k, q, residual, lambda_skip, gate, delta, lambda_log, process_noise, lam, eta,
                       lam_out, eta_out, y, y_var}))
    return fail(KLA_ERR_ALIGN, "%s: fp32 operand not 4-byte aligned", fn);
  const FusedGeom g = fused_geom(batch, 1, M, S);
  const int64_t grid = (batch + kDecodeRows - 1) / kDecodeRows * g.groups;
  if (grid >= (1ll << 31)) return fail(KLA_ERR_INVALID_ARG, "%s: grid too large", fn);
  DecodeParams prm{};
  prm.v = v;
  prm.lv = log_var;
  prm.k = k;
  prm.q = q;
  prm.z = residual;
  prm.skip = lambda_skip;
  prm.gate = gate;
  prm.ld_v = ld_v;
  prm.ld_lv = ld_log_var;
  prm.ld_kq = ld_kq;
  prm.ld_z = ld_residual;
  prm.ld_gate = ld_gate;
  prm.delta = delta;
  prm.lambda_log = lambda_log;
  prm.pnoise = process_noise;
  prm.lam = lam;
  prm.eta = eta;
  prm.lam_out = lam_out;
  prm.eta_out = eta_out;
  prm.y = y;
  prm.yvar = y_var;
  prm.ou = cfg->discretization == 0;
  prm.zero_pn = cfg->zero_process_noise != 0;
  prm.qk_norm = cfg->qk_norm != 0;
  prm.has_clip = cfg->has_clip != 0;
  prm.skip_vector = cfg->skip_vector != 0;
  prm.gate_act = gate ? cfg->gate_activation : kActNone;
  prm.clip = cfg->clip_value;
  prm.ov_min = cfg->obs_var_min;
  prm.ov_max = cfg->obs_var_max;
  return with_sp(S, [&](auto sp) {
    constexpr int SP = decltype(sp)::value;
    if (cfg->decode_from_prior)
      hipLaunchKernelGGL((kla_decode_step_kernel<SP, true, kDecodeRows>), dim3(static_cast<uint32_t>(grid)),
                         dim3(kFusedThreads), 0, stream, prm, g);
    else
      hipLaunchKernelGGL((kla_decode_step_kernel<SP, false, kDecodeRows>), dim3(static_cast<uint32_t>(grid)),
                         dim3(kFusedThreads), 0, stream, prm, g);
    return hip_status(fn, hipGetLastError());
  });
}

int kla_conv_step_fwd(const float *x, int64_t ld_x, const float *state, float *state_out, const float *weight,
                      const float *bias, int activation, float *y, int64_t batch, int64_t channels,
                      int64_t kernel_size, hipStream_t stream) {
  const char *fn = "kla_conv_step_fwd";
  if (batch < 0 || channels < 0 || kernel_size < 1 || kernel_size > 64)
    return fail(KLA_ERR_INVALID_ARG, "%s: bad size (batch=%lld channels=%lld kernel_size=%lld)", fn,
                (long long)batch, (long long)channels, (long long)kernel_size);
  if (batch * channels >= (1ll << 31)) return fail(KLA_ERR_INVALID_ARG, "%s: batch * channels above 2^31", fn);
  if (activation < kActNone || activation > kActRelu)
    return fail(KLA_ERR_INVALID_ARG, "%s: activation must be 0 (none), 1 (silu), 2 (gelu) or 3 (relu)", fn);
  if (batch == 0 || channels == 0) return KLA_OK;
  if (!x || !weight || !y || (kernel_size > 1 && (!state || !state_out)))
    return fail(KLA_ERR_INVALID_ARG, "%s: NULL operand", fn);
  if (ld_x < channels) return fail(KLA_ERR_INVALID_ARG, "%s: row stride below the row length", fn);
  if (!all_aligned(4, {x, state, state_out, weight, bias, y}))
    return fail(KLA_ERR_ALIGN, "%s: fp32 operand not 4-byte aligned", fn);
  const int64_t n = batch * channels;
  const int threads = 256;
  hipLaunchKernelGGL(conv_step_kernel, dim3(static_cast<uint32_t>((n + threads - 1) / threads)), dim3(threads), 0,
                     stream, x, ld_x, state, state_out, weight, bias, activation, y, batch, channels,
                     static_cast<int>(kernel_size));
  return hip_status(fn, hipGetLastError());
}

int kla_causal_conv_fwd(int dtype, const void *x, int64_t ld_t, int64_t ld_b, const void *state, const float *weight,
                        const float *bias, int activation, void *y, void *state_out, int64_t batch, int64_t steps,
                        int64_t channels, int64_t kernel_size, hipStream_t stream) {
  const char *fn = "kla_causal_conv_fwd";
  int rc = check_conv_shape(fn, dtype, batch, steps, channels, kernel_size, activation);
  if (rc != KLA_OK) return rc;
  if (batch == 0 || channels == 0) return KLA_OK;
  if (!weight || (steps > 0 && (!x || !y)))
    return fail(KLA_ERR_INVALID_ARG, "%s: NULL operand", fn);
  if (steps > 0 && (ld_t < channels || ld_b < (steps - 1) * ld_t + channels))
    return fail(KLA_ERR_INVALID_ARG, "%s: strides below the row length", fn);
  const size_t el = dtype == KLA_DTYPE_F32 ? 4 : 2;
  if (misaligned_bytes(x, el) || misaligned_bytes(state, el) || misaligned_bytes(y, el) ||
      misaligned_bytes(state_out, el) || !all_aligned(4, {weight, bias}))
    return fail(KLA_ERR_ALIGN, "%s: operand not aligned to its element size", fn);
  const int64_t n_state = batch * channels * (kernel_size - 1);
  auto run = [&](auto io) {
    using IO = decltype(io);
    if (steps == 0) {
      if (state_out && n_state > 0)
        hipLaunchKernelGGL(copy_or_zero_kernel<IO>, dim3(static_cast<uint32_t>((n_state + 255) / 256)), dim3(256), 0,
                           stream, static_cast<const IO *>(state), static_cast<IO *>(state_out), n_state);
      return hip_status(fn, hipGetLastError());
    }
    // Chunks of 64 steps, halved down to 8 while the grid is under 1024 workgroups.
    const int64_t col_blocks = (channels + kConvThreads - 1) / kConvThreads;
    int T = kConvT;
    while (T > 8 && col_blocks * batch * ((steps + T - 1) / T) < 1024) T /= 2;
    ConvFwdParams<IO> p{static_cast<const IO *>(x), ld_t, ld_b, static_cast<const IO *>(state), weight, bias,
                        static_cast<IO *>(y), static_cast<IO *>(state_out), batch, steps, channels, activation, T};
    const dim3 grid(static_cast<uint32_t>(col_blocks), static_cast<uint32_t>((steps + T - 1) / T),
                    static_cast<uint32_t>(batch));
    return with_k(kernel_size, [&](auto kc) {
      constexpr int K = decltype(kc)::value;
      hipLaunchKernelGGL((causal_conv_fwd_kernel<IO, K>), grid, dim3(kConvThreads), 0, stream, p);
      return hip_status(fn, hipGetLastError());
    });
  };
  return dtype == KLA_DTYPE_F32 ? run(float{}) : run(bf16_t{});
}

size_t kla_causal_conv_workspace_bytes(int64_t batch, int64_t steps, int64_t channels, int64_t kernel_size) {
  if (batch < 0 || steps < 0 || channels < 0 || kernel_size < 1 || kernel_size > kConvMaxK) {
    fail(KLA_ERR_INVALID_ARG, "kla_causal_conv_workspace_bytes: bad size");
    return 0;
  }
  const int64_t bytes = smul(smul(smul(batch, conv_chunks(steps)), channels), smul(kernel_size + 1, 4));
  if (bytes >= kHuge) {
    fail(KLA_ERR_INVALID_ARG, "kla_causal_conv_workspace_bytes: problem too large");
    return 0;
  }
  return std::max<size_t>(256, static_cast<size_t>(bytes));
}

int kla_causal_conv_bwd(int dtype, const void *dy, const void *x, int64_t ld_t, int64_t ld_b, const void *state,
                        const float *weight, const float *bias, int activation, const void *dstate_out, void *dx,
                        void *dstate, float *dweight, float *dbias, int64_t batch, int64_t steps, int64_t channels,
                        int64_t kernel_size, void *workspace, size_t workspace_bytes, hipStream_t stream) {
  const char *fn = "kla_causal_conv_bwd";
  int rc = check_conv_shape(fn, dtype, batch, steps, channels, kernel_size, activation);
  if (rc != KLA_OK) return rc;
  if (batch == 0 || channels == 0) return KLA_OK;
  if (!weight || !dweight || (steps > 0 && (!dy || !x || !dx)) || (bias && !dbias))
    return fail(KLA_ERR_INVALID_ARG, "%s: NULL operand", fn);
  if (steps > 0 && (ld_t < channels || ld_b < (steps - 1) * ld_t + channels))
    return fail(KLA_ERR_INVALID_ARG, "%s: strides below the row length", fn);
  const size_t need = kla_causal_conv_workspace_bytes(batch, steps, channels, kernel_size);
  if (steps > 0 && (!workspace || workspace_bytes < need))
    return fail(KLA_ERR_WORKSPACE, "%s: workspace of %zu bytes, %zu needed", fn, workspace_bytes, need);
  const size_t el = dtype == KLA_DTYPE_F32 ? 4 : 2;
  if (misaligned_bytes(dy, el) || misaligned_bytes(x, el) || misaligned_bytes(state, el) ||
      misaligned_bytes(dstate_out, el) || misaligned_bytes(dx, el) || misaligned_bytes(dstate, el) ||
      !all_aligned(4, {weight, bias, dweight, dbias, workspace}))
    return fail(KLA_ERR_ALIGN, "%s: operand not aligned to its element size", fn);
  const int64_t n_state = batch * channels * (kernel_size - 1);
  auto run = [&](auto io) {
    using IO = decltype(io);
    if (steps == 0) {
      // Empty sequence: d state = d new_state, no weight gradient.
      if (dstate && n_state > 0)
        hipLaunchKernelGGL(copy_or_zero_kernel<IO>, dim3(static_cast<uint32_t>((n_state + 255) / 256)), dim3(256), 0,
                           stream, static_cast<const IO *>(dstate_out), static_cast<IO *>(dstate), n_state);
      const int64_t nw = channels * kernel_size;
      hipLaunchKernelGGL(copy_or_zero_kernel<float>, dim3(static_cast<uint32_t>((nw + 255) / 256)), dim3(256), 0,
                         stream, nullptr, dweight, nw);
      if (dbias)
        hipLaunchKernelGGL(copy_or_zero_kernel<float>, dim3(static_cast<uint32_t>((channels + 255) / 256)), dim3(256),
                           0, stream, nullptr, dbias, channels);
      return hip_status(fn, hipGetLastError());
    }
    const int64_t rows = batch * conv_chunks(steps);
    float *part_w = static_cast<float *>(workspace);
    float *part_b = part_w + rows * channels * kernel_size;
    ConvBwdParams<IO> p{static_cast<const IO *>(dy), static_cast<const IO *>(x), ld_t, ld_b,
                        static_cast<const IO *>(state), weight, bias, static_cast<const IO *>(dstate_out),
                        static_cast<IO *>(dx), static_cast<IO *>(dstate), part_w, part_b, batch, steps, channels,
                        activation};
    const dim3 grid(static_cast<uint32_t>((channels + kConvThreads - 1) / kConvThreads),
                    static_cast<uint32_t>(conv_chunks(steps)), static_cast<uint32_t>(batch));
    rc = with_k(kernel_size, [&](auto kc) {
      constexpr int K = decltype(kc)::value;
      hipLaunchKernelGGL((causal_conv_bwd_kernel<IO, K>), grid, dim3(kConvThreads), 0, stream, p);
      return hip_status(fn, hipGetLastError());
    });
    if (rc != KLA_OK) return rc;
    // Sums over the (batch, chunk) rows in a fixed order.
    const int64_t nw = channels * kernel_size;
    if (!launch_reduce_rows(part_w, dweight, 1, rows, nw, stream))
      hipLaunchKernelGGL(reduce_groups_kernel, dim3(static_cast<uint32_t>((nw + 255) / 256)), dim3(256), 0, stream,
                         part_w, dweight, int64_t{1}, rows, nw);
    if (dbias && !launch_reduce_rows(part_b, dbias, 1, rows, channels, stream))
      hipLaunchKernelGGL(reduce_groups_kernel, dim3(static_cast<uint32_t>((channels + 255) / 256)), dim3(256), 0,
                         stream, part_b, dbias, int64_t{1}, rows, channels);
    return hip_status(fn, hipGetLastError());
  };
  return dtype == KLA_DTYPE_F32 ? run(float{}) : run(bf16_t{});
}


// ------------------------------------------------------- layer output tail

size_t kla_gate_skip_workspace_bytes(int64_t rows, int64_t M) {
  if (rows < 0 || M < 0) return 0;
  const int64_t nblk = rows / kTailRows + (rows % kTailRows != 0);
  const int64_t bytes = smul(sadd(smul(nblk, M), sadd(M, 1)), sizeof(float));
  if (bytes >= kHuge) {
    fail(KLA_ERR_INVALID_ARG, "kla_gate_skip_workspace_bytes: problem too large");
    return 0;
  }
  return std::max<size_t>(256, static_cast<size_t>(bytes));
}

int kla_gate_skip_fwd(int dtype, int out_dtype, const float *y, const void *residual, int64_t ld_res,
                      const void *gate, int64_t ld_gate, const float *lambda_skip, int lambda_vector, int activation,
                      void *out, int64_t rows, int64_t M, hipStream_t stream) {
  const char *fn = "kla_gate_skip_fwd";
  int rc = check_tail(fn, dtype, residual, ld_res, gate, ld_gate, lambda_skip, activation, rows, M);
  if (rc != KLA_OK) return rc;
  if (out_dtype != KLA_DTYPE_F32 && out_dtype != KLA_DTYPE_BF16)
    return fail(KLA_ERR_DTYPE, "%s: unsupported out dtype %d", fn, out_dtype);
  if (rows == 0 || M == 0) return KLA_OK;
  if (!y || !out) return fail(KLA_ERR_INVALID_ARG, "%s: y and out must not be NULL", fn);
  if (!all_aligned(4, {y, lambda_skip}) || misaligned_bytes(out, out_dtype == KLA_DTYPE_F32 ? 4 : 2))
    return fail(KLA_ERR_ALIGN, "%s: operand not aligned to its element size", fn);
  if ((rows + kTailRows - 1) / kTailRows >= (1ll << 31)) return fail(KLA_ERR_INVALID_ARG, "%s: too many rows", fn);
  return with_io(dtype, [&](auto io) {
    return with_io(out_dtype, [&](auto ov) {
      using IO = decltype(io);
      using OUT = decltype(ov);
      TailParams<IO, OUT> p{};
      p.y = y;
      p.res = static_cast<const IO *>(residual);
      p.gate = static_cast<const IO *>(gate);
      p.ld_res = ld_res;
      p.ld_gate = ld_gate;
      p.lam = lambda_skip;
      p.lam_vector = lambda_vector ? 1 : 0;
      p.act = activation;
      p.rows = rows;
      p.M = M;
      p.out = static_cast<OUT *>(out);
      const int V = tail_wide(M, ld_res, ld_gate, {y, residual, gate, lambda_vector ? lambda_skip : nullptr, out}) ? 8 : 1;
      // Row blocks of 16, halved down to 1 while the grid is under 1024 workgroups.
      const int64_t col_blocks = (M + kTailThreads * V - 1) / (kTailThreads * V);
      p.rows_per = kTailRows;
      while (p.rows_per > 1 && col_blocks * ((rows + p.rows_per - 1) / p.rows_per) < 1024) p.rows_per /= 2;
      const dim3 grid(static_cast<uint32_t>((rows + p.rows_per - 1) / p.rows_per), static_cast<uint32_t>(col_blocks));
      if (V == 8)
        hipLaunchKernelGGL((gate_skip_fwd_kernel<IO, OUT, 8>), grid, dim3(kTailThreads), 0, stream, p);
      else
        hipLaunchKernelGGL((gate_skip_fwd_kernel<IO, OUT, 1>), grid, dim3(kTailThreads), 0, stream, p);
      return hip_status(fn, hipGetLastError());
    });
  });
}

int kla_gate_skip_bwd(int dtype, int out_dtype, const void *dout, const float *y, const void *residual,
                      int64_t ld_res, const void *gate, int64_t ld_gate, const float *lambda_skip, int lambda_vector,
                      int activation, float *dy, void *dres, void *dgate, float *dlambda, int64_t rows, int64_t M,
                      void *workspace, size_t workspace_bytes, hipStream_t stream) {
  const char *fn = "kla_gate_skip_bwd";
  int rc = check_tail(fn, dtype, residual, ld_res, gate, ld_gate, lambda_skip, activation, rows, M);
  if (rc != KLA_OK) return rc;
  if (out_dtype != KLA_DTYPE_F32 && out_dtype != KLA_DTYPE_BF16)
    return fail(KLA_ERR_DTYPE, "%s: unsupported out dtype %d", fn, out_dtype);
  if (M == 0) return KLA_OK;
  if (residual && !dlambda) return fail(KLA_ERR_INVALID_ARG, "%s: a residual needs dlambda", fn);
  const int64_t nblk = (rows + kTailRows - 1) / kTailRows;
  if (nblk >= (1ll << 31)) return fail(KLA_ERR_INVALID_ARG, "%s: too many rows", fn);
  if (rows > 0 && (!dout || !y || !dy)) return fail(KLA_ERR_INVALID_ARG, "%s: dout, y and dy must not be NULL", fn);
  const size_t el = dtype == KLA_DTYPE_F32 ? 4 : 2;
  if (!all_aligned(4, {y, lambda_skip, dy, dlambda}) || misaligned_bytes(dres, el) ||
      misaligned_bytes(dgate, el) || misaligned_bytes(dout, out_dtype == KLA_DTYPE_F32 ? 4 : 2))
    return fail(KLA_ERR_ALIGN, "%s: operand not aligned to its element size", fn);
  float *ws = static_cast<float *>(workspace);
  if (residual) {
    if (!ws) return fail(KLA_ERR_WORKSPACE, "%s: workspace is NULL", fn);
    if (misaligned_bytes(workspace, 256)) return fail(KLA_ERR_WORKSPACE, "%s: workspace not 256-byte aligned", fn);
    const size_t need = kla_gate_skip_workspace_bytes(rows, M);
    if (workspace_bytes < need)
      return fail(KLA_ERR_WORKSPACE, "%s: workspace of %zu bytes, %zu needed", fn, workspace_bytes, need);
  }
  return with_io(dtype, [&](auto io) {
    using IO = decltype(io);
    float *part = ws;
    float *colsum = ws ? ws + nblk * M : nullptr;
    if (rows > 0) {
      const int st = with_io(out_dtype, [&](auto ov) {
        using OUT = decltype(ov);
        TailParams<IO, OUT> p{};
        p.y = y;
        p.res = static_cast<const IO *>(residual);
        p.gate = static_cast<const IO *>(gate);
        p.ld_res = ld_res;
        p.ld_gate = ld_gate;
        p.lam = lambda_skip;
        p.lam_vector = lambda_vector ? 1 : 0;
        p.act = activation;
        p.rows = rows;
        p.M = M;
        p.dout = static_cast<const OUT *>(dout);
        p.dy = dy;
        p.dres = static_cast<IO *>(dres);
        p.dgate = static_cast<IO *>(dgate);
        p.part_lam = part;
        if (tail_wide(M, ld_res, ld_gate,
                      {dout, y, residual, gate, lambda_vector ? lambda_skip : nullptr, dy, dres, dgate, part}))
          hipLaunchKernelGGL((gate_skip_bwd_kernel<IO, OUT, 8>), tail_grid(rows, M, 8), dim3(kTailThreads), 0,
                             stream, p);
        else
          hipLaunchKernelGGL((gate_skip_bwd_kernel<IO, OUT, 1>), tail_grid(rows, M, 1), dim3(kTailThreads), 0,
                             stream, p);
        return hip_status(fn, hipGetLastError());
      });
      if (st != KLA_OK) return st;
    }
    if (!residual) return KLA_OK;
    // d lambda: column sums over the row blocks, in a fixed order.
    float *dst = lambda_vector ? dlambda : colsum;
    if (rows == 0) {
      hipLaunchKernelGGL(fill_zero_kernel, dim3(static_cast<uint32_t>((M + 255) / 256)), dim3(256), 0, stream, dst, M);
    } else if (!launch_reduce_rows(part, dst, 1, nblk, M, stream)) {
      hipLaunchKernelGGL(reduce_groups_kernel, dim3(static_cast<uint32_t>((M + 255) / 256)), dim3(256), 0, stream,
                         part, dst, int64_t{1}, nblk, M);
    }
    int st = hip_status(fn, hipGetLastError());
    if (st != KLA_OK || lambda_vector) return st;
    // A 0-dim lambda: the columns summed in order, rounded to the residual's dtype.
    float *total = colsum + M;
    if (!launch_reduce_rows(colsum, total, 1, M, 1, stream))
      hipLaunchKernelGGL(reduce_groups_kernel, dim3(1), dim3(256), 0, stream, colsum, total, int64_t{1}, M, int64_t{1});
    hipLaunchKernelGGL(round_scalar_kernel<IO>, dim3(1), dim3(64), 0, stream, total, dlambda);
    return hip_status(fn, hipGetLastError());
  });
}

// ------------------------------------------------------- sequence-model kernels

int kla_rms_norm_fwd(int dtype, const void *x, const float *weight, float eps, void *y, int64_t rows, int64_t dim,
                     hipStream_t stream) {
  const char *fn = "kla_rms_norm_fwd";
  if (rows < 0 || dim < 0) return fail(KLA_ERR_INVALID_ARG, "%s: negative shape", fn);
  if (dtype != KLA_DTYPE_F32 && dtype != KLA_DTYPE_BF16) return fail(KLA_ERR_DTYPE, "%s: unsupported dtype %d", fn, dtype);
  if (rows == 0 || dim == 0) return KLA_OK;
  if (!x || !weight || !y) return fail(KLA_ERR_INVALID_ARG, "%s: x, weight and y must not be NULL", fn);
  const size_t el = dtype == KLA_DTYPE_F32 ? 4 : 2;
  if (misaligned_bytes(x, el) || misaligned_bytes(y, el) || misaligned(weight))
    return fail(KLA_ERR_ALIGN, "%s: operand not aligned to its element size", fn);
  const int64_t per = kNormThreads / kWave;
  if ((rows + per - 1) / per >= (1ll << 31)) return fail(KLA_ERR_INVALID_ARG, "%s: too many rows", fn);
  const dim3 grid(static_cast<uint32_t>((rows + per - 1) / per));
  if (dtype == KLA_DTYPE_F32)
    hipLaunchKernelGGL(rms_norm_fwd_kernel<float>, grid, dim3(kNormThreads), 0, stream, static_cast<const float *>(x),
                       weight, eps, static_cast<float *>(y), rows, dim);
  else
    hipLaunchKernelGGL(rms_norm_fwd_kernel<bf16_t>, grid, dim3(kNormThreads), 0, stream,
                       static_cast<const bf16_t *>(x), weight, eps, static_cast<bf16_t *>(y), rows, dim);
  return hip_status(fn, hipGetLastError());
}

int kla_swiglu_fwd(int dtype, const void *h, int64_t ld_h, void *out, int64_t rows, int64_t hidden,
                   hipStream_t stream) {
  const char *fn = "kla_swiglu_fwd";
  if (rows < 0 || hidden < 0) return fail(KLA_ERR_INVALID_ARG, "%s: negative shape", fn);
  if (dtype != KLA_DTYPE_F32 && dtype != KLA_DTYPE_BF16) return fail(KLA_ERR_DTYPE, "%s: unsupported dtype %d", fn, dtype);
  if (rows == 0 || hidden == 0) return KLA_OK;
  if (!h || !out) return fail(KLA_ERR_INVALID_ARG, "%s: h and out must not be NULL", fn);
  if (ld_h < 2 * hidden) return fail(KLA_ERR_INVALID_ARG, "%s: row stride below 2 * hidden", fn);
  const size_t el = dtype == KLA_DTYPE_F32 ? 4 : 2;
  if (misaligned_bytes(h, el) || misaligned_bytes(out, el))
    return fail(KLA_ERR_ALIGN, "%s: operand not aligned to its element size", fn);
  const int64_t n = rows * hidden;
  if ((n + 255) / 256 >= (1ll << 31)) return fail(KLA_ERR_INVALID_ARG, "%s: too many elements", fn);
  const dim3 grid(static_cast<uint32_t>((n + 255) / 256));
  if (dtype == KLA_DTYPE_F32)
    hipLaunchKernelGGL(swiglu_fwd_kernel<float>, grid, dim3(256), 0, stream, static_cast<const float *>(h), ld_h,
                       static_cast<float *>(out), rows, hidden);
  else
    hipLaunchKernelGGL(swiglu_fwd_kernel<bf16_t>, grid, dim3(256), 0, stream, static_cast<const bf16_t *>(h), ld_h,
                       static_cast<bf16_t *>(out), rows, hidden);
  return hip_status(fn, hipGetLastError());
}

}  // extern "C"

namespace {

// Validates the product part of a row-linear call, fills `p` and launches the
// kernel variant for `epi` (the caller has filled the epilogue's own fields).
int rows_linear_launch(const char *fn, int epi, RowsLinearParams &p, hipStream_t stream) {
  const int64_t rows = p.rows, n = p.n, k = p.k;
  if (rows < 0 || n < 0 || k < 0 || p.glu_off < 0) return fail(KLA_ERR_INVALID_ARG, "%s: negative size", fn);
  if (rows == 0 || n == 0) return KLA_OK;
  if (!p.y || (k > 0 && (!p.x || !p.w))) return fail(KLA_ERR_INVALID_ARG, "%s: x, w and y must not be NULL", fn);
  if (epi == kEpiResidual && !p.res) return fail(KLA_ERR_INVALID_ARG, "%s: the residual epilogue needs res", fn);
  if (epi == kEpiSwiglu && p.glu_off < n)
    return fail(KLA_ERR_INVALID_ARG, "%s: glu_off %lld below n %lld (the halves overlap)", fn,
                (long long)p.glu_off, (long long)n);
  const bool qk = epi == kEpiQk;
  if (p.ldx < k || p.ldw < k || (!qk && p.ldy < n) || (qk && (p.ldy < p.qk_seg || p.ldy2 < p.qk_seg)) ||
      (epi == kEpiResidual && p.ldres < n))
    return fail(KLA_ERR_INVALID_ARG, "%s: a row stride is below its row length", fn);
  if (p.norm_w && k == 0) return fail(KLA_ERR_INVALID_ARG, "%s: RMSNorm over zero columns", fn);
  if (misaligned(p.x) || misaligned(p.w) || misaligned(p.bias) || misaligned(p.norm_w) || misaligned(p.res) ||
      misaligned(p.y))
    return fail(KLA_ERR_ALIGN, "%s: fp32 operand not 4-byte aligned", fn);
  const int64_t tiles_n = (n + kRowsLinTile - 1) / kRowsLinTile;
  const int64_t tiles_m = (rows + kRowsLinTile - 1) / kRowsLinTile;
  if (tiles_n >= (1ll << 31) || tiles_m >= 65536) return fail(KLA_ERR_INVALID_ARG, "%s: grid too large", fn);
  // k split over the workgroup's waves in multiples of 16.
  const int64_t per = ((k + kRowsLinWaves - 1) / kRowsLinWaves + 15) / 16 * 16;
  if (per > (1 << 30)) return fail(KLA_ERR_INVALID_ARG, "%s: k too large", fn);
  p.k_per_wave = static_cast<int>(per > 0 ? per : 16);
  // Rows that start 16-byte aligned load four k at a time; a ragged last group
  // of a row (k not a multiple of 4) falls back to single loads in the kernel.
  const bool vec = p.ldx % 4 == 0 && p.ldw % 4 == 0 && all_aligned(16, {p.x, p.w, p.norm_w});
  // One workgroup per CU at most (a 1024-thread workgroup fills a CU): more
  // column tiles than that are walked by each workgroup in turn.
  int dev = 0, cus = 256;
  if (hipGetDevice(&dev) == hipSuccess) {
    int v = 0;
    if (hipDeviceGetAttribute(&v, hipDeviceAttributeMultiprocessorCount, dev) == hipSuccess && v > 0) cus = v;
  }
  const int64_t per_cu = (cus + tiles_m - 1) / tiles_m;
  // A plain product over a short k with many more tiles than CUs (the LM head:
  // 3144 tiles over k = 512) runs the two-step variant, two workgroups a CU,
  // so each CU keeps two tiles' weights in flight instead of one (the same sums:
  // the steps past k were skipped anyway). C5 graph decode 0.2955-0.2978 ->
  // 0.2920-0.2928 ms per token, A/B on one box.
  const bool two_per_cu = epi == kEpiPlain && p.k_per_wave <= 32 && tiles_n >= 4 * per_cu;
  const int64_t ctas_cap = two_per_cu ? 2 * per_cu : per_cu;
  const int64_t ctas_n = tiles_n < ctas_cap ? tiles_n : ctas_cap;
  const dim3 grid(static_cast<uint32_t>(ctas_n), static_cast<uint32_t>(tiles_m));
  const bool pipe = p.k_per_wave <= 16 * rows_lin_steps(epi, p.norm_w != nullptr);
  auto go = [&](auto epi_c, auto norm_c, auto vec_c) {
    if constexpr (decltype(epi_c)::value == kEpiPlain) {
      if (two_per_cu) {
        hipLaunchKernelGGL((rows_linear_kernel<kEpiPlain, decltype(norm_c)::value, decltype(vec_c)::value, true, 2>),
                           grid, dim3(kRowsLinThreads), 0, stream, p);
        return;
      }
    }
    if (pipe)
      hipLaunchKernelGGL((rows_linear_kernel<decltype(epi_c)::value, decltype(norm_c)::value,
                                             decltype(vec_c)::value, true>),
                         grid, dim3(kRowsLinThreads), 0, stream, p);
    else
      hipLaunchKernelGGL((rows_linear_kernel<decltype(epi_c)::value, decltype(norm_c)::value,
                                             decltype(vec_c)::value, false>),
                         grid, dim3(kRowsLinThreads), 0, stream, p);
  };
  using T = std::true_type;
  using F = std::false_type;
  auto by_vec = [&](auto epi_c, auto norm_c) { vec ? go(epi_c, norm_c, T{}) : go(epi_c, norm_c, F{}); };
  auto by_norm = [&](auto epi_c) { p.norm_w ? by_vec(epi_c, T{}) : by_vec(epi_c, F{}); };
  switch (epi) {
    case kEpiPlain:
      by_norm(std::integral_constant<int, kEpiPlain>{});
      break;
    case kEpiResidual:
      by_norm(std::integral_constant<int, kEpiResidual>{});
      break;
    case kEpiSwiglu:
      by_norm(std::integral_constant<int, kEpiSwiglu>{});
      break;
    case kEpiQk:
      by_vec(std::integral_constant<int, kEpiQk>{}, F{});
      break;
    default:
      by_norm(std::integral_constant<int, kEpiConv>{});
      break;
  }
  return hip_status(fn, hipGetLastError());
}

// Parts per row of the split argmax: about 256 workgroups in all, chunks of at
// least 2048 columns, at most 64 parts; 1 means the one-kernel path.
int64_t argmax_parts(int64_t rows, int64_t n) {
  int64_t parts = rows >= 256 ? 1 : (256 + rows - 1) / rows;
  if (parts > 64) parts = 64;
  while (parts > 1 && n / parts < 2048) --parts;
  return parts;
}

int64_t argmax_workspace_bytes(int64_t rows, int64_t n) {
  const int64_t pairs = smul(rows, argmax_parts(rows, n));
  return sadd(smul(sadd(smul(pairs, 4), 255) / 256, 256), smul(pairs, 8));
}

RowsLinearParams rows_params(const float *x, int64_t ldx, const float *w, int64_t ldw, const float *bias,
                             const float *norm_w, float eps, float *y, int64_t ldy, int64_t rows, int64_t n,
                             int64_t k) {
  RowsLinearParams p{};
  p.x = x;
  p.w = w;
  p.bias = bias;
  p.norm_w = norm_w;
  p.y = y;
  p.ldx = ldx;
  p.ldw = ldw;
  p.ldy = ldy;
  p.rows = rows;
  p.n = n;
  p.k = k;
  p.eps = eps;
  return p;
}

}  // namespace

extern "C" {

int kla_rows_linear_fwd(int epilogue, const float *x, int64_t ldx, const float *w, int64_t ldw, const float *bias,
                        const float *norm_w, float eps, const float *res, int64_t ldres, float *y, int64_t ldy,
                        int64_t rows, int64_t n, int64_t k, int64_t glu_off, hipStream_t stream) {
  const char *fn = "kla_rows_linear_fwd";
  if (epilogue != KLA_ROWS_PLAIN && epilogue != KLA_ROWS_RESIDUAL && epilogue != KLA_ROWS_SWIGLU)
    return fail(KLA_ERR_INVALID_ARG, "%s: unknown epilogue %d", fn, epilogue);
  RowsLinearParams p = rows_params(x, ldx, w, ldw, bias, norm_w, eps, y, ldy, rows, n, k);
  p.res = res;
  p.ldres = ldres;
  p.glu_off = glu_off;
  const int epi = epilogue == KLA_ROWS_PLAIN ? kEpiPlain : epilogue == KLA_ROWS_RESIDUAL ? kEpiResidual : kEpiSwiglu;
  return rows_linear_launch(fn, epi, p, stream);
}

int kla_rows_linear_qk_fwd(const float *x, int64_t ldx, const float *w, int64_t ldw, const float *bias,
                           float *k_out, float *q_out, int64_t rows, int64_t k, int64_t S, int norm, int has_clip,
                           float clip, hipStream_t stream) {
  const char *fn = "kla_rows_linear_qk_fwd";
  if (S < 1 || S > 16 || (S & (S - 1)) != 0)
    return fail(KLA_ERR_INVALID_ARG, "%s: S must be a power of two in [1, 16], got %lld", fn, (long long)S);
  if (rows > 0 && !q_out) return fail(KLA_ERR_INVALID_ARG, "%s: q_out must not be NULL", fn);
  if (misaligned(q_out)) return fail(KLA_ERR_ALIGN, "%s: fp32 operand not 4-byte aligned", fn);
  RowsLinearParams p = rows_params(x, ldx, w, ldw, bias, nullptr, 0.0f, k_out, S, rows, 2 * S, k);
  p.y2 = q_out;
  p.ldy2 = S;
  p.qk_seg = static_cast<int>(S);
  p.qk_norm = norm ? 1 : 0;
  p.qk_has_clip = has_clip ? 1 : 0;
  p.qk_clip = clip;
  return rows_linear_launch(fn, kEpiQk, p, stream);
}

int kla_rows_linear_conv_fwd(const float *x, int64_t ldx, const float *w, int64_t ldw, const float *bias,
                             const float *norm_w, float eps, float *y, int64_t ldy, int64_t rows, int64_t n,
                             int64_t k, const float *conv_w, const float *conv_b, const float *window,
                             float *window_out, int64_t conv_n, int conv_k, int activation, hipStream_t stream) {
  const char *fn = "kla_rows_linear_conv_fwd";
  if (conv_n < 0 || conv_n > n) return fail(KLA_ERR_INVALID_ARG, "%s: conv_n outside [0, n]", fn);
  if (conv_k < 1 || conv_k > kRowsLinMaxConvK)
    return fail(KLA_ERR_INVALID_ARG, "%s: conv_k %d outside [1, %d]", fn, conv_k, kRowsLinMaxConvK);
  if (activation < 0 || activation > 3) return fail(KLA_ERR_INVALID_ARG, "%s: unknown activation %d", fn, activation);
  if (rows > 0 && conv_n > 0 && (!conv_w || (conv_k > 1 && (!window || !window_out))))
    return fail(KLA_ERR_INVALID_ARG, "%s: conv_w, window and window_out must not be NULL", fn);
  if (misaligned(conv_w) || misaligned(conv_b) || misaligned(window) || misaligned(window_out))
    return fail(KLA_ERR_ALIGN, "%s: fp32 operand not 4-byte aligned", fn);
  RowsLinearParams p = rows_params(x, ldx, w, ldw, bias, norm_w, eps, y, ldy, rows, n, k);
  p.conv_w = conv_w;
  p.conv_b = conv_b;
  p.window = window;
  p.window_out = window_out;
  p.conv_n = conv_n;
  p.conv_k = conv_k;
  p.conv_act = activation;
  return rows_linear_launch(fn, kEpiConv, p, stream);
}

int kla_gather_rows(int dtype, const void *table, int64_t ld_table, int64_t vocab, const int64_t *ids, void *out,
                    int64_t ld_out, int64_t rows, int64_t dim, hipStream_t stream) {
  const char *fn = "kla_gather_rows";
  if (dtype != KLA_DTYPE_F32 && dtype != KLA_DTYPE_BF16) return fail(KLA_ERR_DTYPE, "%s: unsupported dtype %d", fn, dtype);
  if (rows < 0 || dim < 0 || vocab < 0) return fail(KLA_ERR_INVALID_ARG, "%s: negative size", fn);
  if (rows == 0 || dim == 0) return KLA_OK;
  if (!table || !ids || !out) return fail(KLA_ERR_INVALID_ARG, "%s: table, ids and out must not be NULL", fn);
  if (ld_table < dim || ld_out < dim) return fail(KLA_ERR_INVALID_ARG, "%s: a row stride is below dim", fn);
  if (rows >= (1ll << 31)) return fail(KLA_ERR_INVALID_ARG, "%s: too many rows", fn);
  const size_t el = dtype == KLA_DTYPE_F32 ? 4 : 2;
  if (misaligned_bytes(table, el) || misaligned_bytes(out, el) || misaligned_bytes(ids, 8))
    return fail(KLA_ERR_ALIGN, "%s: operand not aligned to its element size", fn);
  const dim3 grid(static_cast<uint32_t>(rows));
  if (dtype == KLA_DTYPE_F32)
    hipLaunchKernelGGL(gather_rows_kernel<float>, grid, dim3(256), 0, stream, static_cast<const float *>(table),
                       ld_table, vocab, ids, static_cast<float *>(out), ld_out, dim);
  else
    hipLaunchKernelGGL(gather_rows_kernel<bf16_t>, grid, dim3(256), 0, stream, static_cast<const bf16_t *>(table),
                       ld_table, vocab, ids, static_cast<bf16_t *>(out), ld_out, dim);
  return hip_status(fn, hipGetLastError());
}

size_t kla_argmax_workspace_bytes(int64_t rows, int64_t n) {
  if (rows <= 0 || n <= 0) return 0;
  const int64_t bytes = argmax_workspace_bytes(rows, n);
  return bytes >= kHuge ? 0 : static_cast<size_t>(bytes);
}

int kla_argmax_rows(const float *x, int64_t ldx, int64_t rows, int64_t n, int64_t *out, int64_t ld_out,
                    void *workspace, size_t workspace_bytes, hipStream_t stream) {
  const char *fn = "kla_argmax_rows";
  if (rows < 0 || n < 0) return fail(KLA_ERR_INVALID_ARG, "%s: negative size", fn);
  if (rows == 0) return KLA_OK;
  if (n == 0) return fail(KLA_ERR_INVALID_ARG, "%s: argmax over zero values", fn);
  if (!x || !out) return fail(KLA_ERR_INVALID_ARG, "%s: x and out must not be NULL", fn);
  if (ldx < n || ld_out < 1) return fail(KLA_ERR_INVALID_ARG, "%s: bad row stride", fn);
  if (rows >= (1ll << 31)) return fail(KLA_ERR_INVALID_ARG, "%s: too many rows", fn);
  if (misaligned(x) || misaligned_bytes(out, 8)) return fail(KLA_ERR_ALIGN, "%s: operand not aligned", fn);
  if (workspace && workspace_bytes >= argmax_workspace_bytes(rows, n) && argmax_parts(rows, n) > 1) {
    // Split: parts per row so that about 256 workgroups stream the rows, then a combine.
    const int64_t parts = argmax_parts(rows, n);
    const int64_t chunk = (n + parts - 1) / parts;
    float *pv = static_cast<float *>(workspace);
    int64_t *pi = reinterpret_cast<int64_t *>(static_cast<char *>(workspace) + ((rows * parts * 4 + 255) / 256) * 256);
    hipLaunchKernelGGL(argmax_parts_kernel, dim3(static_cast<uint32_t>(parts), static_cast<uint32_t>(rows)),
                       dim3(kArgmaxPartThreads), 0, stream, x, ldx, n, chunk, pv, pi);
    hipLaunchKernelGGL(argmax_combine_kernel, dim3(static_cast<uint32_t>(rows)), dim3(kWave), 0, stream, pv, pi,
                       parts, n, out, ld_out);
    return hip_status(fn, hipGetLastError());
  }
  const dim3 grid(static_cast<uint32_t>(rows));
  if (ldx % 4 == 0 && all_aligned(16, {x}))
    hipLaunchKernelGGL(argmax_rows_kernel<true>, grid, dim3(kArgmaxThreads), 0, stream, x, ldx, n, out, ld_out);
  else
    hipLaunchKernelGGL(argmax_rows_kernel<false>, grid, dim3(kArgmaxThreads), 0, stream, x, ldx, n, out, ld_out);
  return hip_status(fn, hipGetLastError());
}

int kla_discretize_fwd(const float *delta, const float *lambda_log, const float *pnoise, int64_t n, int ou,
                       int zero_process_noise, int has_clip, float clip, float *a_bar, float *p_bar,
                       hipStream_t stream) {
  const char *fn = "kla_discretize_fwd";
  if (n < 0) return fail(KLA_ERR_INVALID_ARG, "%s: negative size", fn);
  if (n == 0) return KLA_OK;
  if (!delta || !lambda_log || !pnoise || !a_bar || !p_bar)
    return fail(KLA_ERR_INVALID_ARG, "%s: NULL operand", fn);
  if (!all_aligned(4, {delta, lambda_log, pnoise, a_bar, p_bar}))
    return fail(KLA_ERR_ALIGN, "%s: fp32 operand not 4-byte aligned", fn);
  if ((n + 255) / 256 >= (1ll << 31)) return fail(KLA_ERR_INVALID_ARG, "%s: too many elements", fn);
  DiscParams q{};
  q.delta = delta;
  q.lambda_log = lambda_log;
  q.pnoise = pnoise;
  q.a_bar = a_bar;
  q.p_bar = p_bar;
  q.n = n;
  q.ou = ou != 0;
  q.zero_pn = zero_process_noise != 0;
  q.has_clip = has_clip != 0;
  q.clip = clip;
  hipLaunchKernelGGL(discretize_fwd_kernel, dim3(static_cast<uint32_t>((n + 255) / 256)), dim3(256), 0, stream, q);
  return hip_status(fn, hipGetLastError());
}

int kla_discretize_bwd(const float *delta, const float *lambda_log, const float *pnoise, int64_t n, int ou,
                       int zero_process_noise, int has_clip, float clip, const float *g_a_bar, const float *g_p_bar,
                       float *d_delta, float *d_lambda_log, float *d_pnoise, hipStream_t stream) {
  const char *fn = "kla_discretize_bwd";
  if (n < 0) return fail(KLA_ERR_INVALID_ARG, "%s: negative size", fn);
  if (n == 0) return KLA_OK;
  if (!delta || !lambda_log || !pnoise || !d_delta || !d_lambda_log || !d_pnoise)
    return fail(KLA_ERR_INVALID_ARG, "%s: NULL operand", fn);
  if (!all_aligned(4, {delta, lambda_log, pnoise, g_a_bar, g_p_bar, d_delta, d_lambda_log, d_pnoise}))
    return fail(KLA_ERR_ALIGN, "%s: fp32 operand not 4-byte aligned", fn);
  if ((n + 255) / 256 >= (1ll << 31)) return fail(KLA_ERR_INVALID_ARG, "%s: too many elements", fn);
  DiscParams q{};
  q.delta = delta;
  q.lambda_log = lambda_log;
  q.pnoise = pnoise;
  q.g_a = g_a_bar;
  q.g_p = g_p_bar;
  q.d_delta = d_delta;
  q.d_ll = d_lambda_log;
  q.d_pn = d_pnoise;
  q.n = n;
  q.ou = ou != 0;
  q.zero_pn = zero_process_noise != 0;
  q.has_clip = has_clip != 0;
  q.clip = clip;
  hipLaunchKernelGGL(discretize_bwd_kernel, dim3(static_cast<uint32_t>((n + 255) / 256)), dim3(256), 0, stream, q);
  return hip_status(fn, hipGetLastError());
}

}  // extern "C"

namespace {

int qk_sensors_launch(const char *fn, bool bwd, int dtype, QkParams &p, hipStream_t stream) {
  if (dtype != KLA_DTYPE_F32 && dtype != KLA_DTYPE_BF16) return fail(KLA_ERR_DTYPE, "%s: unsupported dtype %d", fn, dtype);
  if (p.rows < 0 || p.S < 0) return fail(KLA_ERR_INVALID_ARG, "%s: negative size", fn);
  if (p.rows == 0 || p.S == 0) return KLA_OK;
  if (p.S > 64) return fail(KLA_ERR_INVALID_ARG, "%s: S = %lld above 64", fn, (long long)p.S);
  if (p.ld[0] < p.S || p.ld[1] < p.S) return fail(KLA_ERR_INVALID_ARG, "%s: a row stride is below S", fn);
  const size_t el = dtype == KLA_DTYPE_F32 ? 4 : 2;
  for (int i = 0; i < 2; ++i) {
    if (!p.x[i] || (!bwd && !p.y[i]) || (bwd && (!p.dy[i] || !p.dx[i])))
      return fail(KLA_ERR_INVALID_ARG, "%s: NULL operand", fn);
    if (misaligned_bytes(p.x[i], el) || misaligned(p.y[i]) || misaligned(p.dy[i]) || misaligned_bytes(p.dx[i], el))
      return fail(KLA_ERR_ALIGN, "%s: operand not aligned to its element size", fn);
  }
  return with_sp<64>(p.S, [&](auto sp) {
    constexpr int SP = decltype(sp)::value;
    const int64_t threads = 2 * p.rows * SP;
    if ((threads + 255) / 256 >= (1ll << 31)) return fail(KLA_ERR_INVALID_ARG, "%s: too many rows", fn);
    const dim3 grid(static_cast<uint32_t>((threads + 255) / 256));
    auto go = [&](auto io, auto b) {
      hipLaunchKernelGGL((qk_sensors_kernel<decltype(io), SP, decltype(b)::value>), grid, dim3(256), 0, stream, p);
    };
    if (dtype == KLA_DTYPE_F32)
      bwd ? go(float{}, std::true_type{}) : go(float{}, std::false_type{});
    else
      bwd ? go(bf16_t{}, std::true_type{}) : go(bf16_t{}, std::false_type{});
    return hip_status(fn, hipGetLastError());
  });
}

}  // namespace

extern "C" {

int kla_qk_sensors_fwd(int dtype, const void *k, int64_t ld_k, const void *q, int64_t ld_q, float *yk, float *yq,
                       int64_t rows, int64_t S, int norm, int has_clip, float clip, hipStream_t stream) {
  QkParams p{};
  p.x[0] = k;
  p.x[1] = q;
  p.ld[0] = ld_k;
  p.ld[1] = ld_q;
  p.y[0] = yk;
  p.y[1] = yq;
  p.rows = rows;
  p.S = S;
  p.norm = norm != 0;
  p.has_clip = has_clip != 0;
  p.clip = clip;
  return qk_sensors_launch("kla_qk_sensors_fwd", false, dtype, p, stream);
}

int kla_qk_sensors_bwd(int dtype, const void *k, int64_t ld_k, const void *q, int64_t ld_q, const float *dyk,
                       const float *dyq, void *dk, void *dq, int64_t rows, int64_t S, int norm, int has_clip,
                       float clip, hipStream_t stream) {
  QkParams p{};
  p.x[0] = k;
  p.x[1] = q;
  p.ld[0] = ld_k;
  p.ld[1] = ld_q;
  p.dy[0] = dyk;
  p.dy[1] = dyq;
  p.dx[0] = dk;
  p.dx[1] = dq;
  p.rows = rows;
  p.S = S;
  p.norm = norm != 0;
  p.has_clip = has_clip != 0;
  p.clip = clip;
  return qk_sensors_launch("kla_qk_sensors_bwd", true, dtype, p, stream);
}

int kla_cat_cols(int dtype, int n, const void *const *pieces, const int64_t *ld, const int64_t *widths, void *out,
                 int64_t rows, hipStream_t stream) {
  const char *fn = "kla_cat_cols";
  if (dtype != KLA_DTYPE_F32 && dtype != KLA_DTYPE_BF16) return fail(KLA_ERR_DTYPE, "%s: unsupported dtype %d", fn, dtype);
  if (n < 1 || n > kCatMaxPieces) return fail(KLA_ERR_INVALID_ARG, "%s: %d pieces (1 to %d)", fn, n, kCatMaxPieces);
  if (!pieces || !ld || !widths) return fail(KLA_ERR_INVALID_ARG, "%s: NULL piece arrays", fn);
  if (rows < 0) return fail(KLA_ERR_INVALID_ARG, "%s: negative rows", fn);
  const size_t el = dtype == KLA_DTYPE_F32 ? 4 : 2;
  const int vec = static_cast<int>(16 / el);
  int64_t W = 0;
  bool can_vec = true;
  int64_t start[kCatMaxPieces + 1];
  for (int i = 0; i < n; ++i) {
    if (widths[i] < 0) return fail(KLA_ERR_INVALID_ARG, "%s: negative width", fn);
    if (pieces[i] && ld[i] < widths[i]) return fail(KLA_ERR_INVALID_ARG, "%s: piece %d stride below its width", fn, i);
    if (misaligned_bytes(pieces[i], el)) return fail(KLA_ERR_ALIGN, "%s: piece %d not aligned", fn, i);
    start[i] = W;
    W += widths[i];
    if (widths[i] % vec || (pieces[i] && (ld[i] % vec || !all_aligned(16, {pieces[i]})))) can_vec = false;
  }
  start[n] = W;
  if (rows == 0 || W == 0) return KLA_OK;
  if (!out) return fail(KLA_ERR_INVALID_ARG, "%s: NULL out", fn);
  if (misaligned_bytes(out, el)) return fail(KLA_ERR_ALIGN, "%s: out not aligned", fn);
  if (W % vec || !all_aligned(16, {out})) can_vec = false;
  if (rows >= 65536 * 32768ll) return fail(KLA_ERR_INVALID_ARG, "%s: too many rows", fn);
  auto go = [&](auto io) {
    using IO = decltype(io);
    CatParams<IO> p{};
    for (int i = 0; i < n; ++i) {
      p.src[i] = static_cast<const IO *>(pieces[i]);
      p.ld[i] = ld[i];
    }
    for (int i = 0; i <= n; ++i) p.start[i] = start[i];
    p.n = n;
    p.out = static_cast<IO *>(out);
    p.rows = rows;
    p.W = W;
    const int v = can_vec ? vec : 1;
    const int64_t per = 256ll * v;
    // rows go on grid.y (at most 65535): larger row counts take several launches.
    for (int64_t r0 = 0; r0 < rows; r0 += 65535) {
      const int64_t rr = rows - r0 < 65535 ? rows - r0 : 65535;
      CatParams<IO> q = p;
      for (int i = 0; i < n; ++i)
        if (q.src[i]) q.src[i] += r0 * q.ld[i];
      q.out += r0 * W;
      q.rows = rr;
      const dim3 grid(static_cast<uint32_t>((W + per - 1) / per), static_cast<uint32_t>(rr));
      if (can_vec)
        hipLaunchKernelGGL((cat_cols_kernel<IO, 16 / sizeof(IO)>), grid, dim3(256), 0, stream, q);
      else
        hipLaunchKernelGGL((cat_cols_kernel<IO, 1>), grid, dim3(256), 0, stream, q);
    }
    return hip_status(fn, hipGetLastError());
  };
  return dtype == KLA_DTYPE_F32 ? go(float{}) : go(bf16_t{});
}

int kla_sum_parts(int dtype, const float *parts, int64_t nparts, int64_t n, void *out, hipStream_t stream) {
  const char *fn = "kla_sum_parts";
  if (dtype != KLA_DTYPE_F32 && dtype != KLA_DTYPE_BF16) return fail(KLA_ERR_DTYPE, "%s: unsupported dtype %d", fn, dtype);
  if (nparts < 1 || n < 0) return fail(KLA_ERR_INVALID_ARG, "%s: %lld parts of %lld", fn, (long long)nparts, (long long)n);
  if (n == 0) return KLA_OK;
  if (!parts || !out) return fail(KLA_ERR_INVALID_ARG, "%s: NULL pointer", fn);
  const size_t el = dtype == KLA_DTYPE_F32 ? 4 : 2;
  if (misaligned_bytes(parts, 4) || misaligned_bytes(out, el)) return fail(KLA_ERR_ALIGN, "%s: misaligned", fn);
  const bool vec = n % 4 == 0 && all_aligned(16, {parts}) && all_aligned(4 * el, {out});
  const int64_t per = 256ll * (vec ? 4 : 1);
  // Eight workgroups per CU of 256 (MI355X) at most; each thread walks the rest.
  int64_t blocks = (n + per - 1) / per;
  if (blocks > 2048) blocks = 2048;
  const dim3 grid(static_cast<uint32_t>(blocks));
  auto go = [&](auto io) {
    using IO = decltype(io);
    if (vec)
      hipLaunchKernelGGL((sum_parts_kernel<IO, 4>), grid, dim3(256), 0, stream, parts, nparts, n, static_cast<IO *>(out));
    else
      hipLaunchKernelGGL((sum_parts_kernel<IO, 1>), grid, dim3(256), 0, stream, parts, nparts, n, static_cast<IO *>(out));
    return hip_status(fn, hipGetLastError());
  };
  return dtype == KLA_DTYPE_F32 ? go(float{}) : go(bf16_t{});
}

}  // extern "C"
