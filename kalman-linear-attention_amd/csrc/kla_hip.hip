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

#pragma GCC visibility push(default)
#include "kla_hip.h"
#pragma GCC visibility pop

#include "lookback_scan.hpp"

namespace {

using namespace kla;

constexpr int kAbiVersion = 1;

// Tile shapes: W waves x S steps per wave (chunk = W*S steps), V lanes per
// thread (tile = 64 V lanes). Chosen by measurement on MI355X at
// (batch 8, steps 4096, lanes 2048): the forward scans want a short register
// footprint (occupancy hides the look-back), the backward scans long chunks.
// A V > 1 shape needs lanes % V == 0 and operands aligned to V elements; the
// V = 1 shape of the same kind serves every other call.
template <class P, int W_, int S_, int V_>
struct Shape3 {
  using Policy = P;
  static constexpr int W = W_, S = S_, V = V_;
};
using MobiusFwdTile = Shape3<void, 8, 12, 1>;
using MobiusBwdTile = Shape3<void, 8, 32, 1>;
using AffineFwdTile = Shape3<void, 16, 24, 1>;
using AffineBwdTile = Shape3<void, 12, 32, 1>;
using AffineFwdBf16Tile = Shape3<void, 8, 24, 2>;
using AffineBwdBf16Tile = Shape3<void, 16, 8, 4>;
using AffineBf16Fallback = Shape3<void, 8, 32, 1>;

constexpr uint32_t kMaxSpin = 1u << 20;   // ~1 s of polling before a wait gives up

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
  return g;
}

template <class T>
Geom make_geom(Shape s) {
  return make_geom(s, T::W, T::S, T::V);
}

// Workspace words of one tile shape: header, then K aggregate planes and one
// carry plane, each n_chunks * plane words.
size_t words_for(Shape s, int W, int S, int V, int K) {
  const Geom g = make_geom(s, W, S, V);
  return static_cast<size_t>(kHeaderWords + (K + 1) * g.n_chunks * g.plane);
}

template <class T>
size_t words_for(Shape s, int K) {
  return words_for(s, T::W, T::S, T::V, K);
}

// Bytes of workspace a scan kind needs: the largest over the shapes it may run.
size_t workspace_bytes_kind(int kind, Shape s) {
  size_t w = 0;
  switch (kind) {
    case KLA_SCAN_MOBIUS_FWD:
      w = words_for<MobiusFwdTile>(s, 4);
      break;
    case KLA_SCAN_MOBIUS_BWD:
      w = words_for<MobiusBwdTile>(s, 2);
      break;
    case KLA_SCAN_AFFINE_FWD:
      w = std::max(words_for<AffineFwdTile>(s, 2),
                   std::max(words_for<AffineFwdBf16Tile>(s, 2), words_for<AffineBf16Fallback>(s, 2)));
      break;
    case KLA_SCAN_AFFINE_BWD:
      w = std::max(words_for<AffineBwdTile>(s, 2),
                   std::max(words_for<AffineBwdBf16Tile>(s, 2), words_for<AffineBf16Fallback>(s, 2)));
      break;
    default:
      return 0;
  }
  return w * sizeof(uint64_t);
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
  const int64_t blocks = g1.n_tiles * g1.n_chunks;
  if (blocks >= (1ll << 31))
    return fail(KLA_ERR_INVALID_ARG, "%s: %lld workgroups exceed the grid limit", fn, (long long)blocks);
  if (ws == nullptr) return fail(KLA_ERR_WORKSPACE, "%s: workspace is NULL", fn);
  if (misaligned_bytes(ws, 256)) return fail(KLA_ERR_WORKSPACE, "%s: workspace not 256-byte aligned", fn);
  const size_t need = workspace_bytes_kind(kind, s);
  if (ws_bytes < need)
    return fail(KLA_ERR_WORKSPACE, "%s: workspace of %zu bytes, %zu needed", fn, ws_bytes, need);
  return KLA_OK;
}

int hip_status(const char *fn, hipError_t e) {
  if (e != hipSuccess) return fail(KLA_ERR_HIP, "%s: %s", fn, hipGetErrorString(e));
  return KLA_OK;
}

template <class P, class T>
int launch(const char *fn, const typename P::Params &prm, Shape s, void *ws, hipStream_t stream) {
  const Geom g = make_geom<T>(s);
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

}  // namespace

extern "C" {

int kla_hip_abi_version(void) { return kAbiVersion; }

const char *kla_hip_last_error(void) { return g_last_error; }

size_t kla_scan_workspace_bytes(int kind, int64_t batch, int64_t steps, int64_t lanes) {
  const Shape s{batch, steps, lanes};
  if (check_shape("kla_scan_workspace_bytes", s) != KLA_OK) return 0;
  const size_t bytes = workspace_bytes_kind(kind, s);
  if (bytes == 0) fail(KLA_ERR_INVALID_ARG, "kla_scan_workspace_bytes: unknown scan kind %d", kind);
  return bytes;
}

int kla_workspace_failures(const void *workspace, hipStream_t stream, uint32_t *failures) {
  const char *fn = "kla_workspace_failures";
  if (workspace == nullptr || failures == nullptr) return fail(KLA_ERR_INVALID_ARG, "%s: NULL argument", fn);
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
  const char *fn = "kla_mobius_scan_fwd";
  const Shape s{batch, steps, lanes};
  int rc = check_shape(fn, s);
  if (rc != KLA_OK) return rc;
  if (empty(s)) return KLA_OK;
  if (!A || !B || !C || !lam) return fail(KLA_ERR_INVALID_ARG, "%s: A, B, C and lam must not be NULL", fn);
  if (misaligned(A) || misaligned(B) || misaligned(C) || misaligned(D) || misaligned(lam0) ||
      misaligned(lam))
    return fail(KLA_ERR_ALIGN, "%s: fp32 operand not 4-byte aligned", fn);
  rc = check_launch(fn, KLA_SCAN_MOBIUS_FWD, s, workspace, workspace_bytes);
  if (rc != KLA_OK) return rc;
  if (D) {
    using P = MobiusFwd<true>;
    return launch<P, MobiusFwdTile>(fn, P::Params{A, B, C, D, lam0, lam}, s, workspace, stream);
  }
  using P = MobiusFwd<false>;
  return launch<P, MobiusFwdTile>(fn, P::Params{A, B, C, nullptr, lam0, lam}, s, workspace, stream);
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
  if (dtype == KLA_DTYPE_F32) {
    using P = AffineFwd<float>;
    const P::Params prm{static_cast<const float *>(g), static_cast<const float *>(u), h0, static_cast<float *>(h)};
    return launch<P, AffineFwdTile>(fn, prm, s, workspace, stream);
  }
  using P = AffineFwd<bf16_t>;
  const P::Params prm{static_cast<const bf16_t *>(g), static_cast<const bf16_t *>(u), h0, static_cast<bf16_t *>(h)};
  constexpr int V = AffineFwdBf16Tile::V;
  if (lanes % V == 0 && all_aligned(V * el, {g, u, h}))
    return launch<P, AffineFwdBf16Tile>(fn, prm, s, workspace, stream);
  return launch<P, AffineBf16Fallback>(fn, prm, s, workspace, stream);
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

}  // extern "C"
