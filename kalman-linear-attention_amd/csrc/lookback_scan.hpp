// lookback_scan.hpp -- single-pass chunked scan along time with a decoupled,
// deterministic look-back across chunks, for gfx950 (CDNA4, wave64).
//
// Problem shape: `batch * lanes` independent chains, each `steps` long, stored
// as dense [batch, steps, lanes] (lanes contiguous). One workgroup owns a tile
// of 64 V lanes (V consecutive lanes per thread, moved by one vector access, so
// a wave-wide load or store touches 256 V contiguous bytes of one fp32 time
// row) and a chunk of W*S consecutive steps: wave w holds steps
// [w*S, (w+1)*S) of the chunk in registers. Workgroups are numbered
// chunk-major, so the tiles of one time chunk (adjacent pieces of the same
// rows) are in flight together.
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
// Carry-only launches (Geom::carry_only) publish no aggregates: a chunk waits
// for its predecessor's carry alone, so the carries travel the chain one chunk
// at a time (about half a microsecond a hop). That pays where one chunk of every
// tile together is a few microseconds of HBM traffic or more, so the chain hides
// under the streaming (the headline shapes: 2-4% faster, 1 record word per lane
// and chunk instead of K + 1); with few tiles along a long sequence the hop
// latency is the critical path and the aggregates let a chunk skip ahead instead.
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

#include "scan_ops.hpp"

namespace kla {

constexpr int64_t kHeaderWords = 32;   // 256-byte workspace header

// Header word 0: (epoch << 32) | tickets drawn in the running launch.
// Header word 1: count of look-back waits that gave up.

__device__ __forceinline__ void put_word(uint64_t *p, float v, uint32_t tag) {
  const uint64_t w = (static_cast<uint64_t>(tag) << 32) | static_cast<uint64_t>(__float_as_uint(v));
  __hip_atomic_store(p, w, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

__device__ __forceinline__ uint64_t load_word(uint64_t *p) {
  return __hip_atomic_load(p, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

__device__ __forceinline__ bool word_ok(uint64_t w, uint32_t tag) { return static_cast<uint32_t>(w >> 32) == tag; }
__device__ __forceinline__ float word_val(uint64_t w) { return __uint_as_float(static_cast<uint32_t>(w)); }

// Carry entering `chunk` along one lane chain (see "Determinism" above).
//
// Polls the nearest unresolved predecessor's carry word (one load per poll
// while it waits); when only its aggregate is out (never in a carry-only
// launch), the search passes on to the chunk before. The aggregates between the carry found and `chunk` are then
// applied one by one in chain order. Each chunk's K aggregate words are read
// with their loads in flight together.
template <class P>
__device__ __forceinline__ float look_back(uint64_t *rec, uint64_t *ctl, const Geom &g, int64_t chunk,
                           int64_t slot, uint32_t tag) {
  constexpr int K = P::AGG;
  const int64_t carry_plane = K * g.n_chunks;
  int64_t j = chunk - 1;
  uint32_t spins = 0;
  float x;
  for (;;) {
    const uint64_t cw = load_word(rec + (carry_plane + j) * g.plane + slot);
    if (word_ok(cw, tag)) {
      x = word_val(cw);
      break;
    }
    // Chunk 0 publishes only its carry, never an aggregate.
    bool ready = !g.carry_only && j > 0;
    if (ready) {
      uint64_t aw[K];
#pragma unroll
      for (int k = 0; k < K; ++k) aw[k] = load_word(rec + (k * g.n_chunks + j) * g.plane + slot);
#pragma unroll
      for (int k = 0; k < K; ++k) ready = ready && word_ok(aw[k], tag);
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
  for (int64_t i = j + 1; i < chunk; ++i) {
    uint64_t aw[K];
#pragma unroll
    for (int k = 0; k < K; ++k) aw[k] = load_word(rec + (k * g.n_chunks + i) * g.plane + slot);
    Agg<K> a;
#pragma unroll
    for (int k = 0; k < K; ++k) a.v[k] = word_val(aw[k]);
    x = P::apply(a, x);
  }
  return x;
}

// P is a scan policy (scan_ops.hpp). Grid: n_tiles * n_chunks workgroups of W
// waves; a workgroup covers 64 V lanes and W * S steps.
template <class P, int W, int S, int V>
__global__ void __launch_bounds__(kWave * W)
    lookback_scan_kernel(typename P::Params prm, Geom g, uint64_t *__restrict__ ws) {
  constexpr int K = P::AGG;
  constexpr int TILE = kWave * V;
  __shared__ uint32_t s_ticket, s_tag;
  __shared__ float s_agg[K][W][TILE];
  __shared__ float s_carry[TILE];

  const int tid = static_cast<int>(threadIdx.x);
  const int l = tid & (kWave - 1);
  const int w = __builtin_amdgcn_readfirstlane(tid / kWave);
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
  // Uniform by construction (one thread wrote them before the barrier); read
  // back from LDS the compiler cannot know that, so say it.
  const uint32_t ticket = __builtin_amdgcn_readfirstlane(s_ticket);
  const uint32_t tag = __builtin_amdgcn_readfirstlane(s_tag);
  if (ticket >= gridDim.x) {
    // Header not in the state a previous launch leaves it in (e.g. a workspace
    // that was not zero-filled): count it and touch nothing else.
    if (tid == 0) __hip_atomic_fetch_add(ctl + 1, 1ull, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    return;
  }

  const int64_t chunk = static_cast<int64_t>(ticket) / g.n_tiles;
  const int64_t tile = static_cast<int64_t>(ticket) % g.n_tiles;
  Pos q;
  q.b = tile / g.tiles_per_batch;
  q.n0 = (tile % g.tiles_per_batch) * TILE;
  q.off = static_cast<uint32_t>(l * V);
  q.ok = q.n0 + q.off < g.lanes;
  const int64_t s0 = chunk * (W * S) + static_cast<int64_t>(w) * S;
  const int64_t rem = g.steps - s0;
  const int nvalid = __builtin_amdgcn_readfirstlane(rem <= 0 ? 0 : (rem >= S ? S : static_cast<int>(rem)));

  typename P::template Regs<S, V> r;
  {
    typename P::template Raw<S, V> raw;
    P::template fetch<S, V>(prm, g, raw, q, s0, nvalid);
    P::template prep<S, V>(raw, r);
  }
  Agg<K> mine[V];
#pragma unroll
  for (int v = 0; v < V; ++v) {
    mine[v] = P::template reduce<S, V>(r, v, nvalid);
#pragma unroll
    for (int k = 0; k < K; ++k) s_agg[k][w][l * V + v] = mine[v].v[k];
  }
  __syncthreads();

  if (w == 0) {
#pragma unroll
    for (int v = 0; v < V; ++v) {
      Agg<K> tot = mine[v];
#pragma unroll
      for (int u = 1; u < W; ++u) {
        Agg<K> a;
#pragma unroll
        for (int k = 0; k < K; ++k) a.v[k] = s_agg[k][u][l * V + v];
        tot = P::compose(a, tot);
      }
      const int64_t slot = tile * TILE + l * V + v;
      float carry = 0.0f;
      if (q.ok) {
        if (chunk == 0) {
          carry = P::initial(prm, g, q, v);
        } else if (!g.carry_only) {
#pragma unroll
          for (int k = 0; k < K; ++k) put_word(rec + (k * g.n_chunks + chunk) * g.plane + slot, tot.v[k], tag);
        }
      }
      s_carry[l * V + v] = carry;
      mine[v] = tot;
    }
    if (q.ok && chunk > 0) {
      // Aggregates of all V lanes are out; now wait for the carries.
#pragma unroll
      for (int v = 0; v < V; ++v)
        s_carry[l * V + v] = look_back<P>(rec, ctl, g, chunk, tile * TILE + l * V + v, tag);
    }
    if (q.ok && chunk + 1 < g.n_chunks) {
#pragma unroll
      for (int v = 0; v < V; ++v)
        put_word(rec + (K * g.n_chunks + chunk) * g.plane + tile * TILE + l * V + v,
                 P::apply(mine[v], s_carry[l * V + v]), tag);
    }
  }
  __syncthreads();

  float x[V];
#pragma unroll
  for (int v = 0; v < V; ++v) {
    x[v] = s_carry[l * V + v];
#pragma unroll
    for (int u = 0; u < W - 1; ++u) {
      if (u < w) {
        Agg<K> a;
#pragma unroll
        for (int k = 0; k < K; ++k) a.v[k] = s_agg[k][u][l * V + v];
        x[v] = P::apply(a, x[v]);
      }
    }
  }
  P::template walk<S, V>(prm, g, r, q, s0, nvalid, x);
}

// Fills a fp32 state tensor with zeros (gradients of an empty sequence).
__global__ void fill_zero_kernel(float *p, int64_t count) {
  const int64_t i = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x;
  if (i < count) p[i] = 0.0f;
}

}  // namespace kla
