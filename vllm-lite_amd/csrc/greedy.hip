// K5 row argmax and greedy speculative acceptance
// (vllmlite/speculative.py:86-100, vllmlite/sampling.py:56-57).
//
// The argmax follows numpy: the lowest index among equal maxima, and a NaN
// beats every number (the first NaN wins). vl_argmax_rows: one workgroup
// scans one row with 16-byte loads; vl_greedy_verify: the rows' argmaxes
// and the acceptance in one launch.
#include "vl_common.h"

namespace {

struct ArgBest {
  float v;
  int i;
};

// true when (v, i) should replace the current best (bv, bi)
__device__ __forceinline__ bool arg_better(float v, int i, float bv, int bi) {
  const bool vn = v != v, bn = bv != bv;
  if (vn || bn) return vn && (!bn || i < bi);
  return v > bv || (v == bv && i < bi);
}

// Each thread scans its elements in increasing index order, so a strict
// greater-than keeps the lowest index among its equal maxima and NaNs only
// need their first index (ni); the reduction then merges (value, index)
// pairs with arg_better, a NaN anywhere winning with its lowest index. A row
// of -inf (no thread took a value) gives index 0.
__device__ ArgBest block_argmax(const float* __restrict__ row, int vocab) {
  constexpr int kNone = 0x7fffffff;
  float bv = -__builtin_inff();
  int bi = kNone, ni = kNone;
  auto take = [&](float e, int idx) {
    if (e > bv) bv = e, bi = idx;
    if (e != e && ni == kNone) ni = idx;
  };
  const bool vec = (((uintptr_t)row) & 15) == 0;
  const int nv = vec ? vocab / 4 : 0;
  const float4* r4 = reinterpret_cast<const float4*>(row);
  const int step = blockDim.x;
  int i = threadIdx.x;
  for (; i + 3 * step < nv; i += 4 * step) {  // four 16-byte loads in flight
    float4 q[4];
#pragma unroll
    for (int u = 0; u < 4; ++u) q[u] = r4[i + u * step];
#pragma unroll
    for (int u = 0; u < 4; ++u) {
      const int base = 4 * (i + u * step);
      take(q[u].x, base), take(q[u].y, base + 1), take(q[u].z, base + 2), take(q[u].w, base + 3);
    }
  }
  // the remaining 16-byte chunks keep the per-thread index order: chunk i
  // and later ones all follow every chunk this thread has taken
  for (; i < nv; i += step) {
    const float4 q = r4[i];
    take(q.x, 4 * i), take(q.y, 4 * i + 1), take(q.z, 4 * i + 2), take(q.w, 4 * i + 3);
  }
  for (int k = 4 * nv + threadIdx.x; k < vocab; k += step) take(row[k], k);
  // wave then workgroup reduction
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) {
    const float ov = __shfl_xor(bv, o, 64);
    const int oi = __shfl_xor(bi, o, 64);
    if (arg_better(ov, oi, bv, bi)) bv = ov, bi = oi;
    ni = min(ni, __shfl_xor(ni, o, 64));
  }
  __shared__ float sv[16];
  __shared__ int si[16], sn[16];
  const int w = threadIdx.x >> 6, nw = blockDim.x >> 6;
  if ((threadIdx.x & 63) == 0) sv[w] = bv, si[w] = bi, sn[w] = ni;
  __syncthreads();
  bv = sv[0];
  bi = si[0];
  ni = sn[0];
  for (int k = 1; k < nw; ++k) {
    if (arg_better(sv[k], si[k], bv, bi)) bv = sv[k], bi = si[k];
    ni = min(ni, sn[k]);
  }
  __syncthreads();
  if (ni != kNone) return {__builtin_nanf(""), ni};
  return {bv, bi == kNone ? 0 : bi};
}

__global__ void __launch_bounds__(256) argmax_rows_kernel(const float* __restrict__ logits,
                                                          int64_t stride, int64_t rows, int vocab,
                                                          int32_t* __restrict__ out,
                                                          int32_t* __restrict__ out2) {
  for (int64_t r = blockIdx.x; r < rows; r += gridDim.x) {
    const ArgBest b = block_argmax(logits + r * stride, vocab);
    if (threadIdx.x == 0) {
      out[r] = b.i;
      if (out2) out2[r] = b.i;
    }
  }
}

// Greedy acceptance (vllmlite/speculative.py:86-100) in one launch. The
// logits rows are read by many small workgroups, so that every compute unit
// pulls its share (one compute unit alone reads ~25 GB/s): workgroup (s, j,
// c) takes chunk c of row j of sequence s (kChunkFloats floats, every 16-byte
// load issued before the first compare), reduces it to a (value, index) key
// whose unsigned order is numpy's argmax order, and folds it into keys[row]
// with one 64-bit atomic max; then it arrives at the sequence's counter. The
// sequence's last workgroup to arrive reads its rows' keys (clearing them),
// and writes the picks up to the first mismatch with the drafts (or the
// bonus row when every draft matched), -1 after, and num_accepted; it clears
// the counter. Rows past a sequence's drafts have no workgroups at work.
constexpr int kVerifyThreads = 256;
constexpr int kVerifyUnroll = 16;
constexpr int kChunkFloats = 4 * kVerifyUnroll * kVerifyThreads;  // 16384
constexpr int kNoIndex = 0x7fffffff;

// The key of value v at index idx: high word the value's order (every NaN
// above +inf, -0 as +0), low word the complement of the index (the lower
// index wins among equal values).
__device__ __forceinline__ unsigned long long verify_key(float v, int idx) {
  const unsigned b = __float_as_uint(v);
  const unsigned o = v != v ? 0xFFFFFFFFu
                     : v == 0.f ? 0x80000000u
                     : (b & 0x80000000u) ? ~b
                                         : (b | 0x80000000u);
  return ((unsigned long long)o << 32) | (0xFFFFFFFFu - (unsigned)idx);
}

__global__ void __launch_bounds__(kVerifyThreads) verify_greedy_kernel(
    const float* __restrict__ logits, int64_t stride, int vocab, int chunks,
    const int32_t* __restrict__ row_start, const int32_t* __restrict__ num_drafts,
    const int32_t* __restrict__ drafts, int max_drafts, int32_t* __restrict__ out_tokens,
    int32_t* __restrict__ num_accepted, unsigned long long* keys, unsigned* counts) {
  const int tid = threadIdx.x;
  const int c = blockIdx.x % chunks, j = (blockIdx.x / chunks) % (max_drafts + 1);
  const int s = blockIdx.x / chunks / (max_drafts + 1);
  const int nd = min(max(num_drafts[s], 0), max_drafts);
  if (j > nd) return;  // uniform: no row here
  const float* row = logits + ((int64_t)row_start[s] + j) * stride;
  const int lo = c * kChunkFloats, hi = min(vocab, lo + kChunkFloats);
  // this thread's best in index order: strict > keeps the lowest index among
  // equal values, starting from the first index it reads (a run of -inf
  // then names its first element); ni: its first NaN
  float bv = -__builtin_inff();
  int bi = kNoIndex, ni = kNoIndex;
  auto take = [&](float e, int idx) {
    if (bi == kNoIndex) bi = idx;
    if (e > bv) bv = e, bi = idx;
    if (e != e && ni == kNoIndex) ni = idx;
  };
  const int nv = (hi - lo) / 4;  // whole 16-byte chunks of the row's part
  if ((((uintptr_t)row) & 15) == 0 && (lo & 3) == 0 && nv > 0) {
    const float4* r4 = reinterpret_cast<const float4*>(row + lo);
    float4 q[kVerifyUnroll];
#pragma unroll
    for (int u = 0; u < kVerifyUnroll; ++u) q[u] = r4[max(0, min(u * kVerifyThreads + tid, nv - 1))];
    // keep every load above the first compare (the scheduler would sink each
    // load to its use and leave a few in flight)
    __builtin_amdgcn_sched_barrier(0);
#pragma unroll
    for (int u = 0; u < kVerifyUnroll; ++u) {
      const int k = u * kVerifyThreads + tid;
      if (k < nv) {
        const int e = lo + 4 * k;
        take(q[u].x, e), take(q[u].y, e + 1), take(q[u].z, e + 2), take(q[u].w, e + 3);
      }
    }
    for (int e = lo + 4 * nv + tid; e < hi; e += kVerifyThreads) take(row[e], e);
  } else {
    for (int e = lo + tid; e < hi; e += kVerifyThreads) take(row[e], e);
  }
  unsigned long long key = bi == kNoIndex ? 0ull : verify_key(ni != kNoIndex ? __builtin_nanf("") : bv,
                                                              ni != kNoIndex ? ni : bi);
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) {
    const unsigned long long other = __shfl_xor(key, o, 64);
    key = other > key ? other : key;
  }
  __shared__ unsigned long long wkey[kVerifyThreads / 64];
  __shared__ int last;
  if ((tid & 63) == 0) wkey[tid >> 6] = key;
  __syncthreads();
  if (tid == 0) {
    unsigned long long k = wkey[0];
    for (int w = 1; w < kVerifyThreads / 64; ++w) k = wkey[w] > k ? wkey[w] : k;
    const int64_t r = (int64_t)s * (max_drafts + 1) + j;
    __hip_atomic_fetch_max(keys + r, k, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    asm volatile("s_waitcnt vmcnt(0)" ::: "memory");  // the maximum is in before the arrival
    last = __hip_atomic_fetch_add(counts + s, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) ==
           (unsigned)((nd + 1) * chunks - 1);
  }
  __syncthreads();
  if (!last) return;
  // the sequence's rows are all in: thread i takes row i's key (clearing
  // it) and its draft, all at once; thread 0 then does the acceptance
  __shared__ int picks[kVerifyThreads], dr[kVerifyThreads];
  int32_t* o = out_tokens + (int64_t)s * (max_drafts + 1);
  const int32_t* d = drafts + (int64_t)s * max_drafts;
  int acc = nd;
  for (int i0 = 0; i0 <= nd; i0 += kVerifyThreads) {  // one round below 256 drafts
    const int i = i0 + tid;
    if (i <= nd) {
      const unsigned long long k = __hip_atomic_exchange(keys + (int64_t)s * (max_drafts + 1) + i,
                                                         0ull, __ATOMIC_RELAXED,
                                                         __HIP_MEMORY_SCOPE_AGENT);
      picks[tid] = (int)(0xFFFFFFFFu - (unsigned)(k & 0xFFFFFFFFull));
      dr[tid] = i < nd ? d[i] : 0;
    }
    __syncthreads();
    if (tid == 0)
      for (int u = 0; u < kVerifyThreads && i0 + u <= nd; ++u) {
        const int row = i0 + u;
        o[row] = acc < row ? -1 : picks[u];
        if (acc == nd && row < nd && picks[u] != dr[u]) acc = row;
      }
    __syncthreads();
  }
  if (tid == 0) {
    num_accepted[s] = acc;
    __hip_atomic_store(counts + s, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  }
  for (int i = nd + 1 + tid; i <= max_drafts; i += kVerifyThreads) o[i] = -1;
}

}  // namespace

extern "C" int vl_argmax_rows(const float* logits, int64_t row_stride, int64_t rows, int vocab,
                              int32_t* out, int32_t* out2, void* stream) {
  VL_CHECK_ARG(rows >= 0 && vocab > 0 && row_stride >= vocab, "bad shape");
  if (rows == 0) return VL_OK;
  VL_CHECK_ARG(logits && out, "null pointer");
  const int grid = (int)(rows < 65536 ? rows : 65536);
  argmax_rows_kernel<<<grid, 256, 0, (hipStream_t)stream>>>(logits, row_stride, rows, vocab, out,
                                                            out2);
  VL_CHECK_LAUNCH();
  return VL_OK;
}

extern "C" int vl_greedy_verify(const float* logits, int64_t row_stride, int vocab,
                                const int32_t* row_start, const int32_t* num_drafts,
                                const int32_t* drafts, int max_drafts, int32_t* out_tokens,
                                int32_t* num_accepted, int num_seqs, void* scratch,
                                int64_t scratch_bytes, void* stream) {
  VL_CHECK_ARG(num_seqs >= 0 && vocab > 0 && row_stride >= vocab && max_drafts >= 0 &&
                   max_drafts < 65535,
               "bad shape");
  if (num_seqs == 0) return VL_OK;
  VL_CHECK_ARG(logits && row_start && num_drafts && out_tokens && num_accepted && scratch &&
                   (drafts || max_drafts == 0),
               "null pointer");
  const int chunks = (vocab + kChunkFloats - 1) / kChunkFloats;
  const int64_t grid = (int64_t)num_seqs * (max_drafts + 1) * chunks;
  VL_CHECK_ARG(grid <= 0x7fffffff, "too many rows");
  const int64_t need = 8 * (int64_t)num_seqs * (max_drafts + 1) + 4 * (int64_t)num_seqs;
  VL_CHECK_ARG((((uintptr_t)scratch) & 7) == 0 && scratch_bytes >= need,
               "scratch must be 8-byte aligned and hold %lld bytes", (long long)need);
  unsigned long long* keys = static_cast<unsigned long long*>(scratch);
  unsigned* counts = reinterpret_cast<unsigned*>(keys + (int64_t)num_seqs * (max_drafts + 1));
  verify_greedy_kernel<<<(unsigned)grid, kVerifyThreads, 0, (hipStream_t)stream>>>(
      logits, row_stride, vocab, chunks, row_start, num_drafts, drafts, max_drafts, out_tokens,
      num_accepted, keys, counts);
  VL_CHECK_LAUNCH();
  return VL_OK;
}
