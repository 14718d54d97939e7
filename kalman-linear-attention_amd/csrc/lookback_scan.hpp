// lookback_scan.hpp -- single-pass chunked scan along time with a decoupled,
// deterministic look-back across chunks, for gfx950 (CDNA4, wave64).
//
// Problem shape: `batch * lanes` independent chains, each `steps` long, stored
// as dense [batch, steps, lanes] (lanes contiguous). One workgroup owns a tile
// of 64 lanes (one lane per thread, so every wave-wide load or store touches
// 256 contiguous bytes of one time row) and a chunk of W*S consecutive steps:
// wave w holds steps [w*S, (w+1)*S) of the chunk in registers.
//
//   1. every thread loads its S steps and reduces them to a chunk-local
//      aggregate (an element of the scan's monoid: a 2x2 projective map for the
//      Moebius scan, an affine map x -> m*x + c for the affine scans);
//   2. the W wave aggregates meet in LDS; wave 0 composes them into the chunk
//      aggregate, publishes it, then looks back along its lane's chain for the
//      carry entering the chunk and publishes the carry leaving it;
//   3. every wave applies the aggregates of the waves before it to that carry
//      and re-walks its S steps from registers, writing outputs.
//
// HBM traffic is therefore the compulsory one (inputs read once, outputs
// written once) plus 8-byte records per lane per chunk.
//
// Records. Each published float travels in one 64-bit word, (tag << 32) | bits,
// written and read with relaxed agent-scope atomics: a word is valid iff its tag
// equals the launch's tag, so no fence orders a payload against a flag, and the
// L2 of another XCD is never flushed or invalidated. Tags are the workspace's
// epoch + 1; the epoch advances when the last workgroup of a launch takes its
// ticket, so the workspace is zero-filled only once, at allocation.
//
// Determinism. A chunk's carry is the scalar chain
//     carry_c = apply(Agg_{c-1}, carry_{c-1}),   carry_0 = initial state,
// and the carry a chunk publishes is apply(Agg_c, carry_c). A chunk that finds
// its predecessor's carry unpublished walks back to the nearest published one
// and re-applies the aggregates in between in the same order, which computes
// bit-for-bit the same chain. Results do not depend on scheduling.
//
// Forward progress. Workgroups take tickets from one atomic counter and map
// them chunk-major (all lane tiles of chunk 0 first), so a workgroup only waits
// on chunks whose tickets were drawn earlier by resident workgroups. The wait is
// bounded by Geom::max_spin polls; a wait that gives up yields NaN and counts a
// failure in the workspace header instead of hanging the GPU.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace kla {

constexpr float kEps = 1e-12f;   // EPS = P_MIN of the reference (kla_ops.py:43-44)
constexpr int kWave = 64;
constexpr int64_t kHeaderWords = 32;   // 256-byte workspace header

// Header word 0: (epoch << 32) | tickets drawn in the running launch.
// Header word 1: count of look-back waits that gave up.

struct Geom {
  int64_t batch, steps, lanes;
  int64_t tiles_per_batch;   // ceil(lanes / 64)
  int64_t n_tiles;           // batch * tiles_per_batch
  int64_t n_chunks;          // ceil(steps / (W * S))
  int64_t plane;             // record words per (plane, chunk) = n_tiles * 64
  uint32_t max_spin;
};

template <int K>
struct Agg {
  float v[K];
};

__device__ __forceinline__ void put_word(uint64_t *p, float v, uint32_t tag) {
  const uint64_t w = (static_cast<uint64_t>(tag) << 32) | static_cast<uint64_t>(__float_as_uint(v));
  __hip_atomic_store(p, w, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

__device__ __forceinline__ bool get_word(uint64_t *p, uint32_t tag, float &v) {
  const uint64_t w = __hip_atomic_load(p, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  v = __uint_as_float(static_cast<uint32_t>(w));
  return static_cast<uint32_t>(w >> 32) == tag;
}

// Carry entering `chunk` along one lane chain (see "Determinism" above).
template <class P>
__device__ float look_back(uint64_t *rec, uint64_t *ctl, const Geom &g, int64_t chunk,
                           int64_t slot, uint32_t tag) {
  constexpr int K = P::AGG;
  const int64_t carry_plane = K * g.n_chunks;
  int64_t j = chunk - 1;
  float base = 0.0f;
  uint32_t spins = 0;
  for (;;) {
    float v;
    if (get_word(rec + (carry_plane + j) * g.plane + slot, tag, v)) {
      base = v;
      break;
    }
    // Chunk 0 publishes only its carry, never an aggregate.
    bool ready = j > 0;
#pragma unroll
    for (int k = 0; k < K; ++k) {
      float t;
      if (ready) ready = get_word(rec + (k * g.n_chunks + j) * g.plane + slot, tag, t);
    }
    if (ready) {
      --j;
      continue;
    }
    if (++spins > g.max_spin) {
      __hip_atomic_fetch_add(ctl + 1, 1ull, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
      return __builtin_nanf("");
    }
    __builtin_amdgcn_s_sleep(1);
  }
  float x = base;
  for (int64_t i = j + 1; i < chunk; ++i) {
    Agg<K> a;
#pragma unroll
    for (int k = 0; k < K; ++k) get_word(rec + (k * g.n_chunks + i) * g.plane + slot, tag, a.v[k]);
    x = P::apply(a, x);
  }
  return x;
}

// P (a scan policy) provides:
//   AGG                       floats per aggregate
//   Params                    operand pointers
//   Regs<S>                   per-thread register file for S steps
//   load<S>(prm, g, r, b, n, lane_ok, s0, nvalid)
//   reduce<S>(r, nvalid) -> Agg        chunk-local aggregate, scan order
//   compose(later, earlier) -> Agg
//   apply(agg, x) -> float             act on the carried scalar
//   initial(prm, b, n) -> float        carry entering scan position 0
//   walk<S>(prm, g, r, b, n, lane_ok, s0, nvalid, x)   re-walk and store
template <class P, int W, int S>
__global__ void __launch_bounds__(kWave * W)
    lookback_scan_kernel(typename P::Params prm, Geom g, uint64_t *__restrict__ ws) {
  constexpr int K = P::AGG;
  __shared__ uint32_t s_ticket, s_tag;
  __shared__ float s_agg[K][W][kWave];
  __shared__ float s_carry[kWave];

  const int tid = static_cast<int>(threadIdx.x);
  const int l = tid & (kWave - 1);
  const int w = tid / kWave;
  uint64_t *ctl = ws;
  uint64_t *rec = ws + kHeaderWords;

  if (tid == 0) {
    const uint64_t old = __hip_atomic_fetch_add(ctl, 1ull, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    const uint32_t ticket = static_cast<uint32_t>(old);
    const uint32_t epoch = static_cast<uint32_t>(old >> 32);
    if (ticket == gridDim.x - 1) {
      // Last ticket of this launch: open the next epoch for the next launch.
      uint32_t next = epoch + 1;
      if (next == 0xFFFFFFFFu) next = 0;   // keep tag = epoch + 1 non-zero
      __hip_atomic_store(ctl, static_cast<uint64_t>(next) << 32, __ATOMIC_RELAXED,
                         __HIP_MEMORY_SCOPE_AGENT);
    }
    s_ticket = ticket;
    s_tag = epoch + 1;
  }
  __syncthreads();
  const uint32_t ticket = s_ticket;
  const uint32_t tag = s_tag;
  if (ticket >= gridDim.x) {
    // Header not in the state a previous launch leaves it in (e.g. a workspace
    // that was not zero-filled): count it and touch nothing else.
    if (tid == 0) __hip_atomic_fetch_add(ctl + 1, 1ull, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    return;
  }

  const int64_t chunk = static_cast<int64_t>(ticket) / g.n_tiles;
  const int64_t tile = static_cast<int64_t>(ticket) % g.n_tiles;
  const int64_t b = tile / g.tiles_per_batch;
  const int64_t n = (tile % g.tiles_per_batch) * kWave + l;
  const bool lane_ok = n < g.lanes;
  const int64_t s0 = chunk * (W * S) + static_cast<int64_t>(w) * S;
  int64_t rem = g.steps - s0;
  const int nvalid = rem <= 0 ? 0 : (rem >= S ? S : static_cast<int>(rem));

  typename P::template Regs<S> r;
  P::template load<S>(prm, g, r, b, n, lane_ok, s0, nvalid);
  const Agg<K> mine = P::template reduce<S>(r, nvalid);
#pragma unroll
  for (int k = 0; k < K; ++k) s_agg[k][w][l] = mine.v[k];
  __syncthreads();

  if (w == 0) {
    Agg<K> tot = mine;
#pragma unroll
    for (int q = 1; q < W; ++q) {
      Agg<K> a;
#pragma unroll
      for (int k = 0; k < K; ++k) a.v[k] = s_agg[k][q][l];
      tot = P::compose(a, tot);
    }
    const int64_t slot = tile * kWave + l;
    float carry = 0.0f;
    if (lane_ok) {
      if (chunk == 0) {
        carry = P::initial(prm, b, n);
      } else {
#pragma unroll
        for (int k = 0; k < K; ++k) put_word(rec + (k * g.n_chunks + chunk) * g.plane + slot, tot.v[k], tag);
        carry = look_back<P>(rec, ctl, g, chunk, slot, tag);
      }
      if (chunk + 1 < g.n_chunks)
        put_word(rec + (K * g.n_chunks + chunk) * g.plane + slot, P::apply(tot, carry), tag);
    }
    s_carry[l] = carry;
  }
  __syncthreads();

  float x = s_carry[l];
#pragma unroll
  for (int q = 0; q < W - 1; ++q) {
    if (q < w) {
      Agg<K> a;
#pragma unroll
      for (int k = 0; k < K; ++k) a.v[k] = s_agg[k][q][l];
      x = P::apply(a, x);
    }
  }
  P::template walk<S>(prm, g, r, b, n, lane_ok, s0, nvalid, x);
}

// Fills a fp32 state tensor with zeros (gradients of an empty sequence).
__global__ void fill_zero_kernel(float *p, int64_t count) {
  const int64_t i = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x;
  if (i < count) p[i] = 0.0f;
}

}  // namespace kla
