// K5 row argmax and greedy speculative acceptance
// (vllmlite/speculative.py:86-100, vllmlite/sampling.py:56-57).
//
// The argmax follows numpy: the lowest index among equal maxima, and a NaN
// beats every number (the first NaN wins). One workgroup scans one row with
// 16-byte loads; the acceptance pass is a per-sequence scan over <= k+1 picks.
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

// grid (num_seqs, max_drafts + 1): workgroup (s, j) writes the pick of row j
__global__ void __launch_bounds__(256) verify_pick_kernel(
    const float* __restrict__ logits, int64_t stride, int vocab,
    const int32_t* __restrict__ row_start, const int32_t* __restrict__ num_drafts,
    int max_drafts, int32_t* __restrict__ out_tokens) {
  const int s = blockIdx.x, j = blockIdx.y;
  const int nd = min(max(num_drafts[s], 0), max_drafts);
  if (j > nd) return;
  const ArgBest b = block_argmax(logits + (int64_t)(row_start[s] + j) * stride, vocab);
  if (threadIdx.x == 0) out_tokens[(int64_t)s * (max_drafts + 1) + j] = b.i;
}

__global__ void verify_accept_kernel(const int32_t* __restrict__ num_drafts,
                                     const int32_t* __restrict__ drafts, int max_drafts,
                                     int32_t* __restrict__ out_tokens,
                                     int32_t* __restrict__ num_accepted, int num_seqs) {
  const int s = blockIdx.x * blockDim.x + threadIdx.x;
  if (s >= num_seqs) return;
  const int nd = min(max(num_drafts[s], 0), max_drafts);
  int32_t* o = out_tokens + (int64_t)s * (max_drafts + 1);
  const int32_t* d = drafts + (int64_t)s * max_drafts;
  int acc = nd;
  for (int i = 0; i < nd; ++i)
    if (o[i] != d[i]) {
      acc = i;
      break;
    }
  // emitted: picks 0..acc (the mismatch, or the bonus row when all matched)
  for (int i = acc + 1; i <= max_drafts; ++i) o[i] = -1;
  num_accepted[s] = acc;
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
                                int32_t* num_accepted, int num_seqs, void* stream) {
  VL_CHECK_ARG(num_seqs >= 0 && vocab > 0 && row_stride >= vocab && max_drafts >= 0 &&
                   max_drafts < 65535,
               "bad shape");
  if (num_seqs == 0) return VL_OK;
  VL_CHECK_ARG(logits && row_start && num_drafts && out_tokens && num_accepted &&
                   (drafts || max_drafts == 0),
               "null pointer");
  VL_CHECK_ARG(num_seqs <= 0x7fffffff / 256, "too many sequences");
  hipStream_t st = (hipStream_t)stream;
  verify_pick_kernel<<<dim3(num_seqs, max_drafts + 1), 256, 0, st>>>(
      logits, row_stride, vocab, row_start, num_drafts, max_drafts, out_tokens);
  VL_CHECK_LAUNCH();
  verify_accept_kernel<<<(num_seqs + 255) / 256, 256, 0, st>>>(num_drafts, drafts, max_drafts,
                                                              out_tokens, num_accepted, num_seqs);
  VL_CHECK_LAUNCH();
  return VL_OK;
}
