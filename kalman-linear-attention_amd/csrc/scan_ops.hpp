// scan_ops.hpp -- the four scan policies run by the look-back scan kernel
// (lookback_scan_kernel):
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
//
// Policy interface (P):
//   AGG                                   floats per aggregate (monoid element)
//   Params                                operand pointers
//   Raw<S, V>                             registers filled by fetch (loads only)
//   Regs<S, V>                            registers after prep (per-step coefficients)
//   fetch<S, V>(prm, g, raw, pos, s0, nvalid)  issue the loads of scan positions
//                                         [s0, s0 + nvalid) (nvalid <= S, wave-uniform)
//   prep<S, V>(raw, regs)                 turn loaded values into coefficients
//   reduce<S, V>(regs, v, nvalid) -> Agg  chunk-local aggregate of lane v, scan order
//   compose(later, earlier) -> Agg
//   apply(agg, x) -> float                act on the carried scalar
//   initial(prm, g, pos, v) -> float      carry entering scan position 0 (lane v)
//   walk<S, V>(prm, g, regs, pos, s0, nvalid, x[V])   re-walk and store
// A thread owns V consecutive lanes (V = 1, 2 or 4) and moves them with one
// vector load or store per operand and step.
// fetch only loads, so a kernel can issue the next chunk's fetch before it
// works on the current one.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include <type_traits>

namespace kla {

constexpr float kEps = 1e-12f;   // EPS = P_MIN of the reference (kla_ops.py:43-44)
constexpr int kWave = 64;

struct Geom {
  int64_t batch, steps, lanes;
  int64_t tiles_per_batch;   // ceil(lanes / (64 V)): a tile is the 64 V lanes of one workgroup
  int64_t n_tiles;           // batch * tiles_per_batch
  int64_t n_chunks;          // look-back kernel: ceil(steps / (W * S))
  int64_t plane;             // look-back kernel: record words per (plane, chunk) = n_tiles * 64 V
  uint32_t max_spin;         // look-back kernel: polls before a wait gives up
  int carry_only;            // look-back kernel: publish carries only, no chunk aggregates
};

template <int K>
struct Agg {
  float v[K];
};

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

typedef float f32x2_cvt __attribute__((ext_vector_type(2)));
typedef __bf16 bf16x2_cvt __attribute__((ext_vector_type(2)));

// Two fp32 values rounded to bf16 (to nearest, ties to even; a NaN stays a
// quiet NaN) and packed lo | hi << 16: one v_cvt_pk_bf16_f32 on gfx950.
__device__ __forceinline__ uint32_t pack_bf16x2(float lo, float hi) {
  const bf16x2_cvt b = __builtin_convertvector(f32x2_cvt{lo, hi}, bf16x2_cvt);
  return __builtin_bit_cast(uint32_t, b);
}

template <>
__device__ __forceinline__ bf16_t from_f32<bf16_t>(float x) {
  return bf16_t{static_cast<uint16_t>(pack_bf16x2(x, 0.0f))};
}

// Where one thread sits: batch b and lane tile [n0, n0 + 64 V) are wave-uniform
// (so row addresses below live in SGPRs); the thread owns lanes
// [n0 + off, n0 + off + V) with off = V * (thread index in the wave).
struct Pos {
  int64_t b;      // batch
  int64_t n0;     // first lane of the tile
  uint32_t off;   // first lane of this thread within the tile
  bool ok;        // n0 + off < lanes (lanes is a multiple of V, so all V lanes are valid)
};

// Element index of (b, t, n0): the start of a tile's row at time t, for a time
// that is wave-uniform at every call. row_index pins the result to scalar
// registers (readfirstlane of both halves: exact for a uniform value, and free
// once the value is already scalar), so that the per-step row offsets and the
// access addresses below stay scalar arithmetic; without it the compiler keeps
// the row in vector registers in some kernels (the Moebius forward).
// row_index_vreg is the plain form, for the policy that measured faster with it.
__device__ __forceinline__ int64_t row_index_vreg(const Geom &g, const Pos &q, int64_t t) {
  return (q.b * g.steps + t) * g.lanes + q.n0;
}
__device__ __forceinline__ int64_t row_index(const Geom &g, const Pos &q, int64_t t) {
  const uint64_t r = static_cast<uint64_t>(row_index_vreg(g, q, t));
  const uint32_t lo = __builtin_amdgcn_readfirstlane(static_cast<uint32_t>(r));
  const uint32_t hi = __builtin_amdgcn_readfirstlane(static_cast<uint32_t>(r >> 32));
  return static_cast<int64_t>((static_cast<uint64_t>(hi) << 32) | lo);
}

// The thread's first element in the row starting at `row` (wave-uniform at
// every call). at() makes the row start an explicit wave-uniform global
// pointer, so each access takes the scalar-base plus 32-bit lane-offset form
// (global_load v, v_off, s[base]) with no vector address arithmetic. Written as
// plain (p + row) + off -- at_vreg -- the compiler hoists p + off into a vector
// register pair per array and adds each row with a 64-bit vector add, one per
// access (194 of the Moebius backward's 1070 VALU instructions).
template <class T>
__device__ __forceinline__ T *at_vreg(T *p, int64_t row, const Pos &q) {
  return (p + row) + q.off;
}
template <class T>
__device__ __forceinline__ T *at(T *p, int64_t row, const Pos &q) {
  using Global = __attribute__((address_space(1))) T;
  const uint64_t u = reinterpret_cast<uint64_t>(p + row);
  const uint32_t lo = __builtin_amdgcn_readfirstlane(static_cast<uint32_t>(u));
  const uint32_t hi = __builtin_amdgcn_readfirstlane(static_cast<uint32_t>(u >> 32));
  Global *base = (Global *)((static_cast<uint64_t>(hi) << 32) | lo);
  return (T *)(base + q.off);
}

__device__ __forceinline__ int64_t state_index(const Geom &g, const Pos &q) {
  return q.b * g.lanes + q.n0 + q.off;
}

// Sequence tensors are streamed: every element is read once and written once,
// so their loads and stores carry the nontemporal hint (they do not displace
// reused lines from the caches). One dword / dwordx2 / dwordx4 access per
// operand and step moves the V lanes of a thread.
typedef float f32x2 __attribute__((ext_vector_type(2)));
typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef uint32_t u32x2 __attribute__((ext_vector_type(2)));

// V consecutive sequence elements, widened to fp32.
template <int V>
__device__ __forceinline__ void load_v(const float *p, float (&o)[V]) {
  if constexpr (V == 1) {
    o[0] = __builtin_nontemporal_load(p);
  } else if constexpr (V == 2) {
    const f32x2 t = __builtin_nontemporal_load(reinterpret_cast<const f32x2 *>(p));
    o[0] = t.x;
    o[1] = t.y;
  } else {
    static_assert(V == 4, "V must be 1, 2 or 4");
    const f32x4 t = __builtin_nontemporal_load(reinterpret_cast<const f32x4 *>(p));
    o[0] = t.x;
    o[1] = t.y;
    o[2] = t.z;
    o[3] = t.w;
  }
}

template <int V>
__device__ __forceinline__ void load_v(const bf16_t *p, float (&o)[V]) {
  if constexpr (V == 1) {
    const uint16_t u = __builtin_nontemporal_load(reinterpret_cast<const uint16_t *>(p));
    o[0] = __uint_as_float(static_cast<uint32_t>(u) << 16);
  } else if constexpr (V == 2) {
    const uint32_t u = __builtin_nontemporal_load(reinterpret_cast<const uint32_t *>(p));
    o[0] = __uint_as_float(u << 16);
    o[1] = __uint_as_float(u & 0xFFFF0000u);
  } else {
    static_assert(V == 4, "V must be 1, 2 or 4");
    const u32x2 u = __builtin_nontemporal_load(reinterpret_cast<const u32x2 *>(p));
    o[0] = __uint_as_float(u.x << 16);
    o[1] = __uint_as_float(u.x & 0xFFFF0000u);
    o[2] = __uint_as_float(u.y << 16);
    o[3] = __uint_as_float(u.y & 0xFFFF0000u);
  }
}

template <int V>
__device__ __forceinline__ void store_v(float *p, const float (&x)[V]) {
  if constexpr (V == 1) {
    __builtin_nontemporal_store(x[0], p);
  } else if constexpr (V == 2) {
    const f32x2 t = {x[0], x[1]};
    __builtin_nontemporal_store(t, reinterpret_cast<f32x2 *>(p));
  } else {
    static_assert(V == 4, "V must be 1, 2 or 4");
    const f32x4 t = {x[0], x[1], x[2], x[3]};
    __builtin_nontemporal_store(t, reinterpret_cast<f32x4 *>(p));
  }
}

template <int V>
__device__ __forceinline__ void store_v(bf16_t *p, const float (&x)[V]) {
  if constexpr (V == 1) {
    __builtin_nontemporal_store(from_f32<bf16_t>(x[0]).bits, reinterpret_cast<uint16_t *>(p));
  } else if constexpr (V == 2) {
    __builtin_nontemporal_store(pack_bf16x2(x[0], x[1]), reinterpret_cast<uint32_t *>(p));
  } else {
    static_assert(V == 4, "V must be 1, 2 or 4");
    const u32x2 u = {pack_bf16x2(x[0], x[1]), pack_bf16x2(x[2], x[3])};
    __builtin_nontemporal_store(u, reinterpret_cast<u32x2 *>(p));
  }
}

// The forward scans' outputs (lam, h) are read again by the backward scans, in
// reverse time order and usually right away. With CACHED (chosen per launch: the
// output fits the memory-side cache) they are stored with ordinary (cached)
// stores instead of nontemporal ones, so the backward finds the end of the
// sequence still in L2 and the memory-side cache. The choice is a template
// parameter, not a branch: the compiler merges the two stores of a branch into
// one and drops the nontemporal hint.
template <int V>
__device__ __forceinline__ void store_v_cached(float *p, const float (&x)[V]) {
  if constexpr (V == 1) {
    p[0] = x[0];
  } else if constexpr (V == 2) {
    *reinterpret_cast<f32x2 *>(p) = f32x2{x[0], x[1]};
  } else {
    static_assert(V == 4, "V must be 1, 2 or 4");
    *reinterpret_cast<f32x4 *>(p) = f32x4{x[0], x[1], x[2], x[3]};
  }
}

template <int V>
__device__ __forceinline__ void store_v_cached(bf16_t *p, const float (&x)[V]) {
  if constexpr (V == 1) {
    *reinterpret_cast<uint16_t *>(p) = from_f32<bf16_t>(x[0]).bits;
  } else if constexpr (V == 2) {
    *reinterpret_cast<uint32_t *>(p) = pack_bf16x2(x[0], x[1]);
  } else {
    static_assert(V == 4, "V must be 1, 2 or 4");
    *reinterpret_cast<u32x2 *>(p) = u32x2{pack_bf16x2(x[0], x[1]), pack_bf16x2(x[2], x[3])};
  }
}

// V consecutive sequence elements read with ordinary (cached) loads: the lines
// stay in L2 and the memory-side cache for a kernel that reads them next.
template <int V>
__device__ __forceinline__ void load_v_cached(const float *p, float (&o)[V]) {
  if constexpr (V == 1) {
    o[0] = p[0];
  } else if constexpr (V == 2) {
    const f32x2 t = *reinterpret_cast<const f32x2 *>(p);
    o[0] = t.x;
    o[1] = t.y;
  } else {
    static_assert(V == 4, "V must be 1, 2 or 4");
    const f32x4 t = *reinterpret_cast<const f32x4 *>(p);
    o[0] = t.x;
    o[1] = t.y;
    o[2] = t.z;
    o[3] = t.w;
  }
}

// V consecutive elements of a [batch, lanes] fp32 state tensor (ordinary access).
template <int V>
__device__ __forceinline__ void load_state_v(const float *p, float (&o)[V]) {
#pragma unroll
  for (int v = 0; v < V; ++v) o[v] = p[v];
}

template <int V>
__device__ __forceinline__ void store_state_v(float *p, const float (&x)[V]) {
#pragma unroll
  for (int v = 0; v < V; ++v) p[v] = x[v];
}

template <int V>
__device__ __forceinline__ void fill_v(float (&o)[V], float x) {
#pragma unroll
  for (int v = 0; v < V; ++v) o[v] = x;
}

// V consecutive sequence elements as held in registers: fp32 as V floats, bf16
// packed two to a 32-bit register and widened on read, so a bf16 tile costs
// half the VGPRs of the same tile in fp32.
template <class IO, int V>
struct Lanes;

template <int V>
struct Lanes<float, V> {
  float w[V];
  __device__ __forceinline__ float operator[](int v) const { return w[v]; }
  __device__ __forceinline__ void fill(float x) { fill_v(w, x); }
  __device__ __forceinline__ void load(const float *p) { load_v<V>(p, w); }
};

// The widening is one VALU op, issued as volatile asm at every read: the
// compiler can neither hoist it nor keep the widened copies alive between the
// reduce and the walk over the same registers, which would double the tile's
// register footprint.
__device__ __forceinline__ float bf16_lo_to_f32(uint32_t x) {
  float r;
  asm volatile("v_lshlrev_b32 %0, 16, %1" : "=v"(r) : "v"(x));
  return r;
}

__device__ __forceinline__ float bf16_hi_to_f32(uint32_t x) {
  float r;
  asm volatile("v_and_b32 %0, 0xffff0000, %1" : "=v"(r) : "v"(x));
  return r;
}

template <int V>
struct Lanes<bf16_t, V> {
  static constexpr int N = (V + 1) / 2;
  uint32_t w[N];
  __device__ __forceinline__ float operator[](int v) const {
    const uint32_t x = w[v >> 1];
    return (v & 1) ? bf16_hi_to_f32(x) : bf16_lo_to_f32(x);
  }
  // x must be exact in bf16 (the fills are 0 and 1).
  __device__ __forceinline__ void fill(float x) {
    const uint32_t b = __float_as_uint(x) >> 16;
#pragma unroll
    for (int i = 0; i < N; ++i) w[i] = b | (b << 16);
  }
  __device__ __forceinline__ void load(const bf16_t *p) {
    if constexpr (V == 1) {
      w[0] = __builtin_nontemporal_load(reinterpret_cast<const uint16_t *>(p));
    } else if constexpr (V == 2) {
      w[0] = __builtin_nontemporal_load(reinterpret_cast<const uint32_t *>(p));
    } else {
      static_assert(V == 4, "V must be 1, 2 or 4");
      const u32x2 u = __builtin_nontemporal_load(reinterpret_cast<const u32x2 *>(p));
      w[0] = u.x;
      w[1] = u.y;
    }
  }
};

// ------------------------------------------------------------ affine monoid
// (m, c) is the map x -> m*x + c; composing later (L) after earlier (M) gives
// (L.m * M.m, L.m * M.c + L.c).  Reference: _affine_combine, kla_ops.py:119-123.

__device__ __forceinline__ Agg<2> affine_compose(const Agg<2> &L, const Agg<2> &M) {
  return Agg<2>{{L.v[0] * M.v[0], L.v[0] * M.v[1] + L.v[1]}};
}

__device__ __forceinline__ float affine_apply(const Agg<2> &a, float x) { return a.v[0] * x + a.v[1]; }

// Aggregate of the affine steps (m_j, c_j), j < nvalid, in order.
template <int S, class M, class C>
__device__ __forceinline__ Agg<2> affine_reduce(M m, C c, int nvalid) {
  Agg<2> acc{{1.0f, 0.0f}};
#pragma unroll
  for (int j = 0; j < S; ++j) {
    if (j < nvalid) {
      const Agg<2> f{{m(j), c(j)}};
      acc = (j == 0) ? f : affine_compose(f, acc);
    }
  }
  return acc;
}

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

// One step of the recurrence, lam_t = (A lam_{t-1} + B) / den_t with
// den_t = max(C lam_{t-1} + D, EPS), as the forward walk computes it. The
// quotient is the numerator times the hardware reciprocal (v_rcp_f32, 1 ulp):
// ~2 ulp per step, which the contractive recurrence does not amplify, for a
// tenth of the IEEE division's instructions (the backward forms three quotients
// per step from one reciprocal). The reciprocal stays a normal float for den up
// to 2^126, within a factor 4 of float overflow. The backward recomputes lam_t
// with these same functions (explicit fmaf, the same reciprocal), so its values
// equal the forward's stored lam bit for bit.
__device__ __forceinline__ float mobius_den(float c, float d, float x) { return fmaxf(fmaf(c, x, d), kEps); }
__device__ __forceinline__ float mobius_next_inv(float a, float b, float x, float inv_den) {
  return fmaf(a, x, b) * inv_den;
}
__device__ __forceinline__ float mobius_next(float a, float b, float x, float den) {
  return mobius_next_inv(a, b, x, __builtin_amdgcn_rcpf(den));
}

// ================================================================ MobiusFwd
// The backward (MobiusBwd) walks time in reverse right after this kernel and
// reads A, B, C (D) again, starting at the end of the sequence. Scan positions
// from `cache_from` on are therefore loaded with ordinary loads, which leave
// them in the memory-side cache for the backward's first chunks; the host picks
// cache_from so that this tail fits the cache (all of it for small problems).
// Earlier positions, and lam, stream (nontemporal): the backward reads lam only
// once per S steps.

template <bool HAS_D>
struct MobiusFwd {
  static constexpr int AGG = 4;
  static constexpr int BYTES = HAS_D ? 20 : 16;   // HBM bytes per element: A, B, C (D) in, lam out
  using IO = float;
  struct Params {
    const float *A, *B, *C, *D, *lam0;
    float *lam;
    int64_t cache_from;   // first scan position whose inputs are loaded cached
  };
  template <int S, int V>
  struct Raw {
    float a[S][V], b[S][V], c[S][V], d[HAS_D ? S : 1][V];
  };
  template <int S, int V>
  using Regs = Raw<S, V>;

  template <int S, int V, bool CACHED>
  __device__ __forceinline__ static void load_steps(const Params &p, const Geom &g, Raw<S, V> &r, const Pos &q,
                                    int64_t row, int nvalid) {
#pragma unroll
    for (int j = 0; j < S; ++j) {
      if (j < nvalid) {
        const int64_t rj = row + j * g.lanes;
        if constexpr (CACHED) {
          load_v_cached<V>(at(p.A, rj, q), r.a[j]);
          load_v_cached<V>(at(p.B, rj, q), r.b[j]);
          load_v_cached<V>(at(p.C, rj, q), r.c[j]);
          if (HAS_D) load_v_cached<V>(at(p.D, rj, q), r.d[HAS_D ? j : 0]);
        } else {
          load_v<V>(at(p.A, rj, q), r.a[j]);
          load_v<V>(at(p.B, rj, q), r.b[j]);
          load_v<V>(at(p.C, rj, q), r.c[j]);
          if (HAS_D) load_v<V>(at(p.D, rj, q), r.d[HAS_D ? j : 0]);
        }
      }
    }
  }

  template <int S, int V>
  __device__ __forceinline__ static void fetch(const Params &p, const Geom &g, Raw<S, V> &r, const Pos &q, int64_t s0,
                               int nvalid) {
    const int64_t row = row_index(g, q, s0);
#pragma unroll
    for (int j = 0; j < S; ++j) {
      fill_v(r.a[j], 1.0f);
      fill_v(r.b[j], 0.0f);
      fill_v(r.c[j], 0.0f);
      if (HAS_D) fill_v(r.d[HAS_D ? j : 0], 1.0f);
    }
    if (!q.ok) return;
    // The empty asm statements are compiler barriers: without them the two
    // branches' loads, identical but for the nontemporal hint, are merged into
    // one set and the hint is lost (the branch is wave-uniform).
    if (s0 >= p.cache_from) {
      asm volatile("" ::: "memory");
      load_steps<S, V, true>(p, g, r, q, row, nvalid);
      asm volatile("" ::: "memory");
    } else {
      load_steps<S, V, false>(p, g, r, q, row, nvalid);
    }
  }

  template <int S, int V>
  __device__ __forceinline__ static void prep(const Raw<S, V> &raw, Regs<S, V> &r) {
    r = raw;
  }

  template <int S, int V>
  __device__ __forceinline__ static Agg<4> leaf(const Regs<S, V> &r, int j, int v) {
    return Agg<4>{{r.a[j][v], r.b[j][v], r.c[j][v], HAS_D ? r.d[HAS_D ? j : 0][v] : 1.0f}};
  }

  template <int S, int V>
  __device__ __forceinline__ static Agg<4> reduce(const Regs<S, V> &r, int v, int nvalid) {
    Agg<4> m{{1.0f, 0.0f, 0.0f, 1.0f}};
#pragma unroll
    for (int j = 0; j < S; ++j)
      if (j < nvalid) m = (j == 0) ? leaf<S, V>(r, 0, v) : mobius_compose(leaf<S, V>(r, j, v), m);
    return m;
  }

  __device__ __forceinline__ static Agg<4> compose(const Agg<4> &L, const Agg<4> &M) { return mobius_compose(L, M); }
  __device__ __forceinline__ static float apply(const Agg<4> &m, float x) { return mobius_apply(m, x); }
  __device__ __forceinline__ static float initial(const Params &p, const Geom &g, const Pos &q, int v) {
    return p.lam0 ? p.lam0[state_index(g, q) + v] : 1.0f;
  }

  template <int S, int V>
  __device__ __forceinline__ static void walk(const Params &p, const Geom &g, const Regs<S, V> &r, const Pos &q,
                              int64_t s0, int nvalid, float (&x)[V]) {
    const int64_t row = row_index(g, q, s0);
#pragma unroll
    for (int j = 0; j < S; ++j) {
      if (j < nvalid) {
#pragma unroll
        for (int v = 0; v < V; ++v) {
          const float d = HAS_D ? r.d[HAS_D ? j : 0][v] : 1.0f;
          x[v] = mobius_next(r.a[j][v], r.b[j][v], x[v], mobius_den(r.c[j][v], d, x[v]));
        }
        if (q.ok) store_v<V>(at(p.lam, row + j * g.lanes, q), x);
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
// Scan position s0 + j is time t = T-1-s0-j, at row `row - j * lanes`.
//
// The saved lam is read once per thread: the value entering the thread's S
// steps (lam at time T-1-s0-nvalid, or lam0 once the scan has passed time 0).
// The thread recomputes lam over its steps from A, B, C, D, which it loads for
// the adjoint anyway, with the forward walk's own step (mobius_den, the
// reciprocal, mobius_next_inv), so the values are the forward's bit for bit.
// That takes the per-element traffic from 32 to 28 bytes plus 4 / S (dlam, A,
// B, C in; dA, dB, dC out) for D = 1.
//
// Its accesses keep the compiler's vector-register addressing (at_vreg,
// row_index_vreg): with the scalar-base form it measured 325-326 us in the
// headline step against 323-324.

template <bool HAS_D>
struct MobiusBwd {
  static constexpr int AGG = 2;
  static constexpr int BYTES = HAS_D ? 36 : 28;   // dlam, A, B, C (D) in, dA, dB, dC (dD) out
  using IO = float;
  struct Params {
    const float *dlam, *A, *B, *C, *D, *lam0, *lam;
    float *dA, *dB, *dC, *dD, *dlam0;
  };
  template <int S, int V>
  struct Raw {
    // lin = lam entering the thread's steps, i.e. lam_{t-1} of its earliest step.
    float dl[S][V], a[S][V], b[S][V], c[S][V], d[HAS_D ? S : 1][V], lin[V];
  };
  template <int S, int V>
  struct Regs {
    // lv[j] = lam at step j's time t, lv[j+1] = lam_{t-1}.
    float dl[S][V], inv[S][V], gain[S][V], lv[S + 1][V];   // inv = 1 / den
  };

  template <int S, int V>
  __device__ __forceinline__ static void fetch(const Params &p, const Geom &g, Raw<S, V> &r, const Pos &q, int64_t s0,
                               int nvalid) {
    const int64_t row = row_index_vreg(g, q, g.steps - 1 - s0);
#pragma unroll
    for (int j = 0; j < S; ++j) {
      fill_v(r.dl[j], 0.0f);
      fill_v(r.a[j], 1.0f);
      fill_v(r.b[j], 0.0f);
      fill_v(r.c[j], 0.0f);
      if (HAS_D) fill_v(r.d[HAS_D ? j : 0], 1.0f);
    }
    fill_v(r.lin, 1.0f);
    if (!q.ok) return;
    if (s0 + nvalid < g.steps) {
      load_v<V>(at_vreg(p.lam, row - static_cast<int64_t>(nvalid) * g.lanes, q), r.lin);
    } else if (p.lam0) {
      load_state_v<V>(p.lam0 + state_index(g, q), r.lin);
    }
#pragma unroll
    for (int j = 0; j < S; ++j) {
      if (j < nvalid) {
        const int64_t rj = row - j * g.lanes;
        load_v<V>(at_vreg(p.dlam, rj, q), r.dl[j]);
        load_v<V>(at_vreg(p.A, rj, q), r.a[j]);
        load_v<V>(at_vreg(p.B, rj, q), r.b[j]);
        load_v<V>(at_vreg(p.C, rj, q), r.c[j]);
        if (HAS_D) load_v<V>(at_vreg(p.D, rj, q), r.d[HAS_D ? j : 0]);
      }
    }
  }

  // Recomputes lam forward in time (j from S-1 down to 0). Steps j >= nvalid
  // hold the fills A = D = 1, B = C = 0: the identity map, which carries lin
  // unchanged (lin > 0) to the earliest valid step.
  template <int S, int V>
  __device__ __forceinline__ static void prep(const Raw<S, V> &raw, Regs<S, V> &r) {
#pragma unroll
    for (int v = 0; v < V; ++v) r.lv[S][v] = raw.lin[v];
#pragma unroll
    for (int j = S - 1; j >= 0; --j) {
#pragma unroll
      for (int v = 0; v < V; ++v) {
        const float D = HAS_D ? raw.d[HAS_D ? j : 0][v] : 1.0f;
        const float inv = __builtin_amdgcn_rcpf(mobius_den(raw.c[j][v], D, r.lv[j + 1][v]));
        r.lv[j][v] = mobius_next_inv(raw.a[j][v], raw.b[j][v], r.lv[j + 1][v], inv);
        r.dl[j][v] = raw.dl[j][v];
        r.inv[j][v] = inv;
        r.gain[j][v] = (raw.a[j][v] * D - raw.b[j][v] * raw.c[j][v]) * (inv * inv);
      }
    }
  }

  template <int S, int V>
  __device__ __forceinline__ static Agg<2> reduce(const Regs<S, V> &r, int v, int nvalid) {
    return affine_reduce<S>([&](int j) { return r.gain[j][v]; },
                            [&](int j) { return r.gain[j][v] * r.dl[j][v]; }, nvalid);
  }

  __device__ __forceinline__ static Agg<2> compose(const Agg<2> &L, const Agg<2> &M) { return affine_compose(L, M); }
  __device__ __forceinline__ static float apply(const Agg<2> &a, float x) { return affine_apply(a, x); }
  __device__ __forceinline__ static float initial(const Params &, const Geom &, const Pos &, int) { return 0.0f; }

  template <int S, int V>
  __device__ __forceinline__ static void walk(const Params &p, const Geom &g, const Regs<S, V> &r, const Pos &q,
                              int64_t s0, int nvalid, float (&x)[V]) {
    const int64_t row = row_index_vreg(g, q, g.steps - 1 - s0);
#pragma unroll
    for (int j = 0; j < S; ++j) {
      if (j < nvalid) {
        const int64_t rj = row - j * g.lanes;
        float da[V], db[V], dc[V], dd[V];
#pragma unroll
        for (int v = 0; v < V; ++v) {
          const float nu = r.dl[j][v] + x[v];
          const float qv = nu * r.inv[j][v];
          const float lt = r.lv[j][v], lp = r.lv[j + 1][v];
          da[v] = qv * lp;
          db[v] = qv;
          dc[v] = (-qv * lt) * lp;
          dd[v] = -qv * lt;
          x[v] = r.gain[j][v] * nu;
        }
        if (q.ok) {
          if (p.dA) store_v<V>(at_vreg(p.dA, rj, q), da);
          if (p.dB) store_v<V>(at_vreg(p.dB, rj, q), db);
          if (p.dC) store_v<V>(at_vreg(p.dC, rj, q), dc);
          if (HAS_D && p.dD) store_v<V>(at_vreg(p.dD, rj, q), dd);
        }
      }
    }
    // The position that is time 0 closes the chain: dlam0 = w_0.
    if (s0 + nvalid == g.steps && nvalid > 0 && q.ok && p.dlam0) store_state_v<V>(p.dlam0 + state_index(g, q), x);
  }
};

// ================================================================ AffineFwd
// h_t = g_t h_{t-1} + u_t, h_{-1} = h0 (reference tiled_mobius_scan.py:161-203).

template <class IOT, bool CACHED = false>
struct AffineFwd {
  static constexpr int AGG = 2;
  static constexpr int BYTES = 3 * static_cast<int>(sizeof(IOT));   // g, u in, h out
  using IO = IOT;
  struct Params {
    const IO *g, *u;
    const float *h0;
    IO *h;
  };
  template <int S, int V>
  struct Raw {
    Lanes<IO, V> g[S], u[S];
  };
  template <int S, int V>
  using Regs = Raw<S, V>;

  template <int S, int V>
  __device__ __forceinline__ static void fetch(const Params &p, const Geom &gm, Raw<S, V> &r, const Pos &q, int64_t s0,
                               int nvalid) {
    const int64_t row = row_index(gm, q, s0);
#pragma unroll
    for (int j = 0; j < S; ++j) {
      r.g[j].fill(1.0f);
      r.u[j].fill(0.0f);
    }
    if (!q.ok) return;
#pragma unroll
    for (int j = 0; j < S; ++j) {
      if (j < nvalid) {
        const int64_t rj = row + j * gm.lanes;
        r.g[j].load(at(p.g, rj, q));
        r.u[j].load(at(p.u, rj, q));
      }
    }
  }

  template <int S, int V>
  __device__ __forceinline__ static void prep(const Raw<S, V> &raw, Regs<S, V> &r) {
    r = raw;
  }

  template <int S, int V>
  __device__ __forceinline__ static Agg<2> reduce(const Regs<S, V> &r, int v, int nvalid) {
    return affine_reduce<S>([&](int j) { return r.g[j][v]; }, [&](int j) { return r.u[j][v]; }, nvalid);
  }

  __device__ __forceinline__ static Agg<2> compose(const Agg<2> &L, const Agg<2> &M) { return affine_compose(L, M); }
  __device__ __forceinline__ static float apply(const Agg<2> &a, float x) { return affine_apply(a, x); }
  __device__ __forceinline__ static float initial(const Params &p, const Geom &gm, const Pos &q, int v) {
    return p.h0 ? p.h0[state_index(gm, q) + v] : 0.0f;
  }

  template <int S, int V>
  __device__ __forceinline__ static void walk(const Params &p, const Geom &gm, const Regs<S, V> &r, const Pos &q,
                              int64_t s0, int nvalid, float (&x)[V]) {
    const int64_t row = row_index(gm, q, s0);
#pragma unroll
    for (int j = 0; j < S; ++j) {
      if (j < nvalid) {
#pragma unroll
        for (int v = 0; v < V; ++v) x[v] = r.g[j][v] * x[v] + r.u[j][v];
        if (q.ok) {
          if constexpr (CACHED)
            store_v_cached<V>(at(p.h, row + j * gm.lanes, q), x);
          else
            store_v<V>(at(p.h, row + j * gm.lanes, q), x);
        }
      }
    }
  }
};

// ================================================================ AffineBwd
// Reverse in time (reference tiled_mobius_scan.py:291-298):
//   mu_t = dh_t + w_{t+1},  w_t = g_t mu_t,  w_T = 0
//   dg_t = mu_t h_{t-1} (h_{-1} = h0 or 0),  du_t = mu_t,  dh0 = w_0

template <class IOT>
struct AffineBwd {
  static constexpr int AGG = 2;
  static constexpr int BYTES = 5 * static_cast<int>(sizeof(IOT));   // dh, g, h in, dg, du out
  using IO = IOT;
  struct Params {
    const IO *dh, *g, *h;
    const float *h0;
    IO *dg, *du;
    float *dh0;
  };
  // bf16 registers hold h_{-1} = h0 (fp32 state) apart, so it is not rounded;
  // in fp32 it simply takes the place of h_{t-1} at time 0.
  static constexpr bool SPLIT_H0 = !std::is_same<IO, float>::value;
  template <int S, int V>
  struct Raw {
    Lanes<IO, V> dh[S], g[S], hp[S];   // hp[j] = h_{t-1} for step j's time t
    float h_init[SPLIT_H0 ? V : 1];    // h0, for the position at time 0 (bf16 only)
  };
  template <int S, int V>
  using Regs = Raw<S, V>;

  template <int S, int V>
  __device__ __forceinline__ static void fetch(const Params &p, const Geom &gm, Raw<S, V> &r, const Pos &q, int64_t s0,
                               int nvalid) {
    const int64_t row = row_index(gm, q, gm.steps - 1 - s0);
    fill_v(r.h_init, 0.0f);
    if (nvalid == S && s0 + S < gm.steps && q.n0 + kWave * V <= gm.lanes) {
      // Wave-uniform fast path: a full chunk away from time 0 with every lane
      // of the wave valid needs none of the fill values below. At C3 with bf16
      // I/O (8 x 8192 x 2048) the kernel went 285-288 -> 270-271 us (the fills
      // were 308 of its 2405 VALU instructions); fp32 is unchanged.
#pragma unroll
      for (int j = 0; j < S; ++j) {
        const int64_t rj = row - j * gm.lanes;
        r.dh[j].load(at(p.dh, rj, q));
        r.g[j].load(at(p.g, rj, q));
        r.hp[j].load(at(p.h, rj - gm.lanes, q));
      }
      return;
    }
#pragma unroll
    for (int j = 0; j < S; ++j) {
      r.dh[j].fill(0.0f);
      r.g[j].fill(1.0f);
      r.hp[j].fill(0.0f);
    }
    if (!q.ok) return;
#pragma unroll
    for (int j = 0; j < S; ++j) {
      if (j < nvalid) {
        const int64_t rj = row - j * gm.lanes;
        r.dh[j].load(at(p.dh, rj, q));
        r.g[j].load(at(p.g, rj, q));
        if (s0 + j + 1 < gm.steps) {
          r.hp[j].load(at(p.h, rj - gm.lanes, q));
        } else if (p.h0) {
          if constexpr (SPLIT_H0)
            load_state_v<V>(p.h0 + state_index(gm, q), r.h_init);
          else
            load_state_v<V>(p.h0 + state_index(gm, q), r.hp[j].w);
        }
      }
    }
  }

  template <int S, int V>
  __device__ __forceinline__ static void prep(const Raw<S, V> &raw, Regs<S, V> &r) {
    r = raw;
  }

  // Aggregate of the thread's steps j < nvalid: leaves (g, g dh), composed in
  // order (affine_reduce's arithmetic; g is read once per step, which for bf16
  // is one widening instead of two). A whole chunk runs without the per-step
  // bound, whose branches made the compiler copy the running sum at every step.
  template <int S, int V>
  __device__ __forceinline__ static Agg<2> reduce(const Regs<S, V> &r, int v, int nvalid) {
    Agg<2> acc{{1.0f, 0.0f}};
    auto step = [&](int j) __attribute__((always_inline)) {
      const float gj = r.g[j][v];
      const Agg<2> f{{gj, gj * r.dh[j][v]}};
      acc = (j == 0) ? f : affine_compose(f, acc);
    };
    if (nvalid == S) {
#pragma unroll
      for (int j = 0; j < S; ++j) step(j);
    } else {
#pragma unroll
      for (int j = 0; j < S; ++j)
        if (j < nvalid) step(j);
    }
    return acc;
  }

  __device__ __forceinline__ static Agg<2> compose(const Agg<2> &L, const Agg<2> &M) { return affine_compose(L, M); }
  __device__ __forceinline__ static float apply(const Agg<2> &a, float x) { return affine_apply(a, x); }
  __device__ __forceinline__ static float initial(const Params &, const Geom &, const Pos &, int) { return 0.0f; }

  // Scan position s0 + j is time t = T-1-s0-j; the step at time 0 (bf16) takes
  // h_{-1} = h0 from h_init. jz, the position of time 0 within the thread's
  // steps (S when they do not reach it), is a wave-uniform 32-bit value, so the
  // test is a scalar compare: written as s0 + j + 1 >= T it was a 64-bit
  // less-than, which has no scalar form, and cost vector compares, a select and
  // moves at every step (C3 bf16 backward 274 -> 261 us with the reduce above).
  // (A second, unguarded copy of the walk for whole chunks spilled 30 VGPRs
  // instead of 10 in the bf16 tile and ran slower.)
  template <int S, int V>
  __device__ __forceinline__ static void walk(const Params &p, const Geom &gm, const Regs<S, V> &r, const Pos &q,
                              int64_t s0, int nvalid, float (&x)[V]) {
    const int64_t row = row_index(gm, q, gm.steps - 1 - s0);
    const int64_t left = gm.steps - 1 - s0;
    const int jz = __builtin_amdgcn_readfirstlane(left < S ? static_cast<int>(left) : S);
#pragma unroll
    for (int j = 0; j < S; ++j) {
      if (j < nvalid) {
        const int64_t rj = row - j * gm.lanes;
        const bool first = SPLIT_H0 && j == jz;
        float dg[V], mu[V];
#pragma unroll
        for (int v = 0; v < V; ++v) {
          mu[v] = r.dh[j][v] + x[v];
          const float hp = r.hp[j][v];
          dg[v] = mu[v] * (first ? r.h_init[SPLIT_H0 ? v : 0] : hp);
          x[v] = r.g[j][v] * mu[v];
        }
        if (q.ok) {
          if (p.dg) store_v<V>(at(p.dg, rj, q), dg);
          if (p.du) store_v<V>(at(p.du, rj, q), mu);
        }
      }
    }
    if (s0 + nvalid == gm.steps && nvalid > 0 && q.ok && p.dh0) store_state_v<V>(p.dh0 + state_index(gm, q), x);
  }
};

}  // namespace kla
