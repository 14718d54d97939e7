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

#pragma GCC visibility push(default)
#include "kla_hip.h"
#pragma GCC visibility pop

#include "scan_ops.hpp"

namespace {

using namespace kla;

constexpr int kAbiVersion = 1;

// Tile shape per scan: W waves x S steps per wave, 64 lanes per workgroup.
template <int KIND>
struct Tile;
template <>
struct Tile<KLA_SCAN_MOBIUS_FWD> {
  static constexpr int W = 4, S = 16, AGG = 4;
};
template <>
struct Tile<KLA_SCAN_MOBIUS_BWD> {
  static constexpr int W = 4, S = 16, AGG = 2;
};
template <>
struct Tile<KLA_SCAN_AFFINE_FWD> {
  static constexpr int W = 4, S = 16, AGG = 2;
};
template <>
struct Tile<KLA_SCAN_AFFINE_BWD> {
  static constexpr int W = 4, S = 16, AGG = 2;
};

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

template <int KIND>
Geom make_geom(Shape s) {
  Geom g;
  g.batch = s.batch;
  g.steps = s.steps;
  g.lanes = s.lanes;
  g.tiles_per_batch = (s.lanes + kWave - 1) / kWave;
  g.n_tiles = s.batch * g.tiles_per_batch;
  const int64_t chunk = Tile<KIND>::W * Tile<KIND>::S;
  g.n_chunks = (s.steps + chunk - 1) / chunk;
  g.plane = g.n_tiles * kWave;
  g.max_spin = kMaxSpin;
  return g;
}

template <int KIND>
size_t workspace_bytes_for(Shape s) {
  const Geom g = make_geom<KIND>(s);
  const int64_t words = kHeaderWords + (Tile<KIND>::AGG + 1) * g.n_chunks * g.plane;
  return static_cast<size_t>(words) * sizeof(uint64_t);
}

bool empty(Shape s) { return s.batch == 0 || s.steps == 0 || s.lanes == 0; }

template <class T>
bool misaligned(const T *p) {
  return (reinterpret_cast<uintptr_t>(p) % alignof(T)) != 0;
}
bool misaligned_bytes(const void *p, size_t a) { return (reinterpret_cast<uintptr_t>(p) % a) != 0; }

template <int KIND>
int check_launch(const char *fn, Shape s, void *ws, size_t ws_bytes, int64_t *grid) {
  const Geom g = make_geom<KIND>(s);
  const int64_t blocks = g.n_tiles * g.n_chunks;
  if (blocks >= (1ll << 31))
    return fail(KLA_ERR_INVALID_ARG, "%s: %lld workgroups exceed the grid limit", fn, (long long)blocks);
  if (ws == nullptr) return fail(KLA_ERR_WORKSPACE, "%s: workspace is NULL", fn);
  if (misaligned_bytes(ws, 256)) return fail(KLA_ERR_WORKSPACE, "%s: workspace not 256-byte aligned", fn);
  const size_t need = workspace_bytes_for<KIND>(s);
  if (ws_bytes < need)
    return fail(KLA_ERR_WORKSPACE, "%s: workspace of %zu bytes, %zu needed", fn, ws_bytes, need);
  *grid = blocks;
  return KLA_OK;
}

int hip_status(const char *fn, hipError_t e) {
  if (e != hipSuccess) return fail(KLA_ERR_HIP, "%s: %s", fn, hipGetErrorString(e));
  return KLA_OK;
}

template <class P, int KIND>
int launch(const char *fn, const typename P::Params &prm, Shape s, void *ws, int64_t grid,
           hipStream_t stream) {
  constexpr int W = Tile<KIND>::W, S = Tile<KIND>::S;
  const Geom g = make_geom<KIND>(s);
  hipLaunchKernelGGL((lookback_scan_kernel<P, W, S>), dim3(static_cast<uint32_t>(grid)),
                     dim3(kWave * W), 0, stream, prm, g, static_cast<uint64_t *>(ws));
  return hip_status(fn, hipGetLastError());
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
  switch (kind) {
    case KLA_SCAN_MOBIUS_FWD: return workspace_bytes_for<KLA_SCAN_MOBIUS_FWD>(s);
    case KLA_SCAN_MOBIUS_BWD: return workspace_bytes_for<KLA_SCAN_MOBIUS_BWD>(s);
    case KLA_SCAN_AFFINE_FWD: return workspace_bytes_for<KLA_SCAN_AFFINE_FWD>(s);
    case KLA_SCAN_AFFINE_BWD: return workspace_bytes_for<KLA_SCAN_AFFINE_BWD>(s);
    default:
      fail(KLA_ERR_INVALID_ARG, "kla_scan_workspace_bytes: unknown scan kind %d", kind);
      return 0;
  }
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
  int64_t grid = 0;
  rc = check_launch<KLA_SCAN_MOBIUS_FWD>(fn, s, workspace, workspace_bytes, &grid);
  if (rc != KLA_OK) return rc;
  if (D) {
    using P = MobiusFwd<true>;
    const P::Params prm{A, B, C, D, lam0, lam, lanes};
    return launch<P, KLA_SCAN_MOBIUS_FWD>(fn, prm, s, workspace, grid, stream);
  }
  using P = MobiusFwd<false>;
  const P::Params prm{A, B, C, nullptr, lam0, lam, lanes};
  return launch<P, KLA_SCAN_MOBIUS_FWD>(fn, prm, s, workspace, grid, stream);
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
  int64_t grid = 0;
  rc = check_launch<KLA_SCAN_MOBIUS_BWD>(fn, s, workspace, workspace_bytes, &grid);
  if (rc != KLA_OK) return rc;
  if (D) {
    using P = MobiusBwd<true>;
    const P::Params prm{dlam, A, B, C, D, lam0, lam, dA, dB, dC, dD, dlam0, lanes};
    return launch<P, KLA_SCAN_MOBIUS_BWD>(fn, prm, s, workspace, grid, stream);
  }
  using P = MobiusBwd<false>;
  const P::Params prm{dlam, A, B, C, nullptr, lam0, lam, dA, dB, dC, nullptr, dlam0, lanes};
  return launch<P, KLA_SCAN_MOBIUS_BWD>(fn, prm, s, workspace, grid, stream);
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
  int64_t grid = 0;
  rc = check_launch<KLA_SCAN_AFFINE_FWD>(fn, s, workspace, workspace_bytes, &grid);
  if (rc != KLA_OK) return rc;
  if (dtype == KLA_DTYPE_F32) {
    using P = AffineFwd<float>;
    const P::Params prm{static_cast<const float *>(g), static_cast<const float *>(u), h0,
                        static_cast<float *>(h), lanes};
    return launch<P, KLA_SCAN_AFFINE_FWD>(fn, prm, s, workspace, grid, stream);
  }
  using P = AffineFwd<bf16_t>;
  const P::Params prm{static_cast<const bf16_t *>(g), static_cast<const bf16_t *>(u), h0,
                      static_cast<bf16_t *>(h), lanes};
  return launch<P, KLA_SCAN_AFFINE_FWD>(fn, prm, s, workspace, grid, stream);
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
  int64_t grid = 0;
  rc = check_launch<KLA_SCAN_AFFINE_BWD>(fn, s, workspace, workspace_bytes, &grid);
  if (rc != KLA_OK) return rc;
  if (dtype == KLA_DTYPE_F32) {
    using P = AffineBwd<float>;
    const P::Params prm{static_cast<const float *>(dh), static_cast<const float *>(g),
                        static_cast<const float *>(h), h0, static_cast<float *>(dg),
                        static_cast<float *>(du), dh0, lanes};
    return launch<P, KLA_SCAN_AFFINE_BWD>(fn, prm, s, workspace, grid, stream);
  }
  using P = AffineBwd<bf16_t>;
  const P::Params prm{static_cast<const bf16_t *>(dh), static_cast<const bf16_t *>(g),
                      static_cast<const bf16_t *>(h), h0, static_cast<bf16_t *>(dg),
                      static_cast<bf16_t *>(du), dh0, lanes};
  return launch<P, KLA_SCAN_AFFINE_BWD>(fn, prm, s, workspace, grid, stream);
}

}  // extern "C"
