// One decode attention item of the one-launch decode step: the REP query
// heads of one token of a sequence over its c keys in one KV head of a paged
// cache (vllmlite/attention.py:59-98 for a sequence with one query: no
// causal mask, softmax over every key), computed by 8 wavefronts; the step
// runs one item per KV head of its sequence, and issues a chunk's loads
// before the barrier that precedes its attention phase.
//
// Keys come in chunks of 256: wavefront w of chunk t takes keys 32 (8 t + w)
// + kk, kk < 32. QK: lanes kk and kk + 32 each hold half of key kk's row
// (dims [0, D/2) and [D/2, D)) and its dot products with the query heads over
// that half; the two halves are added, low half first. Softmax: a base-2
// online softmax per wavefront (running max by DPP, every lane keeping the
// sum of its keys' weights, the low-half lane of each key adding it). PV:
// lane (pg, pc) = (lane / NC, lane % NC) takes the 16-byte chunk pc of the V
// rows of keys pg + G j (G = 64 / NC key groups, KPL keys per lane). The 8
// wavefronts are merged in LDS at the end, max-rescaled, one head at a time.
//
// Every read-modify step of the accumulations is an explicit fma, so the
// result does not depend on how the compiler would contract the source.
#pragma once

#include "vl_common.h"

namespace vl_item {

constexpr int kWaves = 8;                 // wavefronts per item
constexpr int kThreads = 64 * kWaves;     // 512
constexpr int kWaveKeys = 32;             // keys per wavefront per chunk
constexpr int kChunk = kWaves * kWaveKeys;  // 256 keys per chunk
constexpr int kMaxCtx = 2048;             // keys per sequence (block table staged in LDS)

template <typename TKV, int D, int REP>
struct Shape {
  static constexpr int VE = 16 / (int)sizeof(TKV);  // cache elements per 16 bytes
  static constexpr int NC = D / VE;                 // 16-byte chunks per head row
  static constexpr int G = 64 / NC;                 // PV key groups
  static constexpr int KPL = (kWaveKeys + G - 1) / G;  // PV keys per lane
  static constexpr int HB = D / 2 * (int)sizeof(TKV);  // bytes of a half row
  static constexpr int KPB = HB % 16 == 0 ? 16 : 8;    // bytes per K load
  static constexpr int NKP = HB / KPB;                 // K loads per lane
  static_assert(D % VE == 0 && HB % 8 == 0 && NC <= 64, "head_dim");
};

// The item's LDS, apart from its block table (which the caller keeps where
// it outlives other uses of this space).
template <typename TKV, int D, int REP>
struct Lds {
  using S = Shape<TKV, D, REP>;
  float q[REP][D];                      // query heads, pre-scaled to the log2 domain
  float p[kWaves][REP][kWaveKeys];      // per wavefront: the chunk's weights
  float red[kWaves][64][S::VE];         // per wavefront and lane: one head's PV sums
  float m[kWaves][REP], l[kWaves][REP];
};

// One lane's loads of one chunk.
template <typename TKV, int D, int REP>
struct Regs {
  using S = Shape<TKV, D, REP>;
  uint4 k[S::KPB == 16 ? S::NKP : 1];
  uint2 k8[S::KPB == 8 ? S::NKP : 1];
  uint4 v[S::KPL];
};

// What an item reads: its KV head of one layer's caches and its block
// table (in LDS, at least ceil(c / block size) entries).
template <typename TKV>
struct Src {
  const int32_t* tbl;
  const TKV* kc;
  const TKV* vc;
  KvGeom geom;
  int g;         // KV head
  int c;         // keys (context)
  int bs_log2;   // block size of the table
  __amdgpu_buffer_rsrc_t rk, rv;  // the caches, for device-scope loads
};

__device__ __forceinline__ __amdgpu_buffer_rsrc_t cache_rsrc(const void* p, int64_t bytes) {
  return __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(p), (short)0,
                                           (int)(bytes < 0x7fffffff ? bytes : 0x7fffffff),
                                           0x00020000);
}

template <typename TKV>
__device__ __forceinline__ int64_t row_of(const Src<TKV>& a, int k) {
  const int mask = (1 << a.bs_log2) - 1;
  return a.geom.at(((int64_t)a.tbl[k >> a.bs_log2] << a.bs_log2) + (k & mask), a.g);
}

// 16 / 8 bytes at element e of a cache: an ordinary load, or (dev) a
// device-scope load that misses the L1. With BUF the load goes through the
// cache's buffer descriptor with a 32-bit byte offset (one address register
// instead of two; the caller guarantees the cache is under 2 GiB); device-
// scope loads always do.
template <bool BUF, typename TKV>
__device__ __forceinline__ uint4 ld16(const TKV* base, __amdgpu_buffer_rsrc_t r, int64_t e,
                                      bool dev) {
  typedef unsigned u32x4_t __attribute__((ext_vector_type(4)));
  const int off = (int)(e * (int64_t)sizeof(TKV));
  if (dev) {
    const u32x4_t v = __builtin_amdgcn_raw_buffer_load_b128(r, off, 0, 16);
    return make_uint4(v.x, v.y, v.z, v.w);
  }
  if constexpr (BUF) {
    const u32x4_t v = __builtin_amdgcn_raw_buffer_load_b128(r, off, 0, 0);
    return make_uint4(v.x, v.y, v.z, v.w);
  } else {
    return *reinterpret_cast<const uint4*>(base + e);
  }
}
template <bool BUF, typename TKV>
__device__ __forceinline__ uint2 ld8(const TKV* base, __amdgpu_buffer_rsrc_t r, int64_t e,
                                     bool dev) {
  typedef unsigned u32x2_t __attribute__((ext_vector_type(2)));
  const int off = (int)(e * (int64_t)sizeof(TKV));
  if (dev) {
    const u32x2_t v = __builtin_amdgcn_raw_buffer_load_b64(r, off, 0, 16);
    return make_uint2(v.x, v.y);
  }
  if constexpr (BUF) {
    const u32x2_t v = __builtin_amdgcn_raw_buffer_load_b64(r, off, 0, 0);
    return make_uint2(v.x, v.y);
  } else {
    return *reinterpret_cast<const uint2*>(base + e);
  }
}

// Issue the loads of chunk t for this lane (wavefront w). Keys past the
// context load the last key (their weight is 0). The row of the key
// `fresh` (< 0: none) is loaded with device-scope loads, or left out when
// skip_fresh (load_fresh loads it later).
template <bool BUF, typename TKV, int D, int REP>
__device__ __forceinline__ void issue(Regs<TKV, D, REP>& r, const Src<TKV>& a, int t, int w,
                                      int lane, int fresh, bool skip_fresh) {
  using S = Shape<TKV, D, REP>;
  const int cb = (kWaves * t + w) * kWaveKeys;
  if (cb >= a.c) return;  // wavefront-uniform: no key of this wavefront
  const int kk = lane & 31, hh = lane >> 5;
  {
    const int key = min(cb + kk, a.c - 1);
    const bool f = key == fresh;
    if (!(f && skip_fresh)) {
      const int64_t e = row_of(a, key) + hh * (D / 2);
#pragma unroll
      for (int j = 0; j < S::NKP; ++j) {
        if constexpr (S::KPB == 16)
          r.k[j] = ld16<BUF>(a.kc, a.rk, e + j * (16 / (int)sizeof(TKV)), f);
        else
          r.k8[j] = ld8<BUF>(a.kc, a.rk, e + j * (8 / (int)sizeof(TKV)), f);
      }
    }
  }
  const int pg = lane / S::NC, pc = lane - (lane / S::NC) * S::NC;
#pragma unroll
  for (int j = 0; j < S::KPL; ++j) {
    const int key = min(cb + min(pg + S::G * j, kWaveKeys - 1), a.c - 1);
    const bool f = key == fresh;
    if (!(f && skip_fresh)) r.v[j] = ld16<BUF>(a.vc, a.rv, row_of(a, key) + pc * S::VE, f);
  }
}

// After issue(..., skip_fresh): the left-out loads of the key `fresh`,
// device-scope.
template <bool BUF, typename TKV, int D, int REP>
__device__ __forceinline__ void load_fresh(Regs<TKV, D, REP>& r, const Src<TKV>& a, int t, int w,
                                           int lane, int fresh) {
  using S = Shape<TKV, D, REP>;
  const int cb = (kWaves * t + w) * kWaveKeys;
  if (cb >= a.c) return;
  const int kk = lane & 31, hh = lane >> 5;
  if (min(cb + kk, a.c - 1) == fresh) {
    const int64_t e = row_of(a, fresh) + hh * (D / 2);
#pragma unroll
    for (int j = 0; j < S::NKP; ++j) {
      if constexpr (S::KPB == 16)
        r.k[j] = ld16<BUF>(a.kc, a.rk, e + j * (16 / (int)sizeof(TKV)), true);
      else
        r.k8[j] = ld8<BUF>(a.kc, a.rk, e + j * (8 / (int)sizeof(TKV)), true);
    }
  }
  const int pg = lane / S::NC, pc = lane - (lane / S::NC) * S::NC;
#pragma unroll
  for (int j = 0; j < S::KPL; ++j) {
    const int key = min(cb + min(pg + S::G * j, kWaveKeys - 1), a.c - 1);
    if (key == fresh) r.v[j] = ld16<BUF>(a.vc, a.rv, row_of(a, fresh) + pc * S::VE, true);
  }
}

// Running state of one lane.
template <int VE, int REP>
struct State {
  float m[REP], l[REP], acc[REP][VE];
  __device__ __forceinline__ void init() {
#pragma unroll
    for (int h = 0; h < REP; ++h) {
      m[h] = -__builtin_inff(), l[h] = 0.f;
#pragma unroll
      for (int e = 0; e < VE; ++e) acc[h][e] = 0.f;
    }
  }
};

// Chunk t of wavefront w from its loaded registers. Wavefront-uniform: a
// wavefront whose keys all lie past the context does nothing.
template <typename TKV, int D, int REP>
__device__ __forceinline__ void compute(State<Shape<TKV, D, REP>::VE, REP>& st,
                                        const Regs<TKV, D, REP>& r, Lds<TKV, D, REP>& s,
                                        int c, int t, int w, int lane) {
  using S = Shape<TKV, D, REP>;
  constexpr int VE = S::VE;
  const int cb = (kWaves * t + w) * kWaveKeys;
  if (cb >= c) return;
  const int kk = lane & 31, hh = lane >> 5;
  float kr[D / 2];
#pragma unroll
  for (int j = 0; j < S::NKP; ++j) {
    if constexpr (S::KPB == 16) {
      widen16<TKV>(r.k[j], kr + j * (16 / (int)sizeof(TKV)));
    } else {  // 8 FP8 bytes
      e4m3x4_to_f32(r.k8[j].x, kr + 8 * j);
      e4m3x4_to_f32(r.k8[j].y, kr + 8 * j + 4);
    }
  }
  const bool valid = cb + kk < c;
#pragma unroll
  for (int h = 0; h < REP; ++h) {
    float part = 0.f;
#pragma unroll
    for (int d = 0; d < D / 2; ++d) part = __builtin_fmaf(s.q[h][hh * (D / 2) + d], kr[d], part);
    const float other = __shfl_xor(part, 32, 64);
    const float dot = hh ? other + part : part + other;  // low half first
    const float sc = valid ? dot : -__builtin_inff();
    const float mn = fmaxf(st.m[h], wave_max_dpp(sc));  // finite: key cb is valid
    const float alpha = exp2_fast(st.m[h] - mn);
    const float pr = exp2_fast(sc - mn);
    st.l[h] = __builtin_fmaf(st.l[h], alpha, hh ? 0.f : pr);
#pragma unroll
    for (int e = 0; e < VE; ++e) st.acc[h][e] *= alpha;
    st.m[h] = mn;
    if (!hh) s.p[w][h][kk] = pr;
  }
  // the weights the wavefront's other lanes wrote above
  __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
  __builtin_amdgcn_wave_barrier();
  __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
  const int pg = lane / S::NC;
#pragma unroll
  for (int j = 0; j < S::KPL; ++j) {
    const int key = pg + S::G * j;
    float v[VE];
    widen16<TKV>(r.v[j], v);
#pragma unroll
    for (int h = 0; h < REP; ++h) {
      const float wt = key < kWaveKeys ? s.p[w][h][key] : 0.f;
#pragma unroll
      for (int e = 0; e < VE; ++e) st.acc[h][e] = __builtin_fmaf(wt, v[e], st.acc[h][e]);
    }
  }
  // the weights have been read before the next chunk overwrites them
  __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
  __builtin_amdgcn_wave_barrier();
  __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
}

// The wavefronts' states merged; thread it < D of the item writes dim it of
// head h to out_h(h) (a pointer to that head's D outputs). Every thread of
// the workgroup calls this (REP times two __syncthreads); only threads with
// active set take part.
template <typename TKV, int D, int REP, typename Out>
__device__ __forceinline__ void finish(State<Shape<TKV, D, REP>::VE, REP>& st,
                                       Lds<TKV, D, REP>& s, bool active, int it, int w, int lane,
                                       Out out_h) {
  using S = Shape<TKV, D, REP>;
  constexpr int VE = S::VE, NC = S::NC, G = S::G;
  if (active) {
#pragma unroll
    for (int h = 0; h < REP; ++h) st.l[h] = wave_sum_dpp(st.l[h]);
    if (lane == 0) {
#pragma unroll
      for (int h = 0; h < REP; ++h) s.m[w][h] = st.m[h], s.l[w][h] = st.l[h];
    }
  }
#pragma unroll
  for (int h = 0; h < REP; ++h) {
    if (active) {
#pragma unroll
      for (int e = 0; e < VE; ++e) s.red[w][lane][e] = st.acc[h][e];
    }
    __syncthreads();
    if (active && it < D) {
      const int dc = it / VE, de = it - (it / VE) * VE;
      float M = -__builtin_inff();
#pragma unroll
      for (int ww = 0; ww < kWaves; ++ww) M = fmaxf(M, s.m[ww][h]);
      float L = 0.f, acc = 0.f;
#pragma unroll
      for (int ww = 0; ww < kWaves; ++ww) {
        const float mw = s.m[ww][h];
        if (mw == -__builtin_inff()) continue;
        const float wt = exp2_fast(mw - M);
        float sw = 0.f;
#pragma unroll
        for (int gg = 0; gg < G; ++gg) sw += s.red[ww][gg * NC + dc][de];
        L = __builtin_fmaf(s.l[ww][h], wt, L);
        acc = __builtin_fmaf(sw, wt, acc);
      }
      out_h(h, it, L > 0.f ? acc * (1.f / L) : 0.f);
    }
    __syncthreads();
  }
}

}  // namespace vl_item
