// K1 reshape-and-cache, K3 copy-on-write block copy, K4b RoPE + scatter.
//
// All three are pure data movement over the paged per-layer cache, token-major
// [num_slots, num_kv_heads, head_dim] or head-major [num_blocks, num_kv_heads,
// block_size, head_dim] (KvGeom). They are HBM-bound byte copies: each
// workgroup moves whole rows with the widest aligned vector the operands allow.
#include "vl_common.h"

namespace {

// A token's row of nvec vectors lands in the cache as segments of seg_vec
// vectors: one segment at the slot's row (token-major), or one per KV head
// at that head's row (head-major).
template <typename V>
__global__ void __launch_bounds__(256) scatter_rows_kernel(
    const char* __restrict__ key, const char* __restrict__ value, int64_t key_stride_b,
    int64_t value_stride_b, char* __restrict__ kc, char* __restrict__ vc,
    const int32_t* __restrict__ slots, int64_t num_tokens, KvGeom g, int es, int seg_vec,
    int nvec) {
  for (int64_t t = blockIdx.x; t < num_tokens; t += gridDim.x) {
    const int slot = slots[t];
    if (slot < 0) continue;
    const V* ks = reinterpret_cast<const V*>(key + t * key_stride_b);
    const V* vs = reinterpret_cast<const V*>(value + t * value_stride_b);
    for (int i = threadIdx.x; i < nvec; i += blockDim.x) {
      const int seg = i / seg_vec;
      const int64_t off = g.at(slot, seg) * es + (int64_t)(i - seg * seg_vec) * sizeof(V);
      *reinterpret_cast<V*>(kc + off) = ks[i];
      *reinterpret_cast<V*>(vc + off) = vs[i];
    }
  }
}

template <typename V>
__global__ void __launch_bounds__(256) copy_blocks_kernel(char* __restrict__ kc,
                                                          char* __restrict__ vc,
                                                          const int32_t* __restrict__ pairs,
                                                          int64_t layer_stride_b, int nvec) {
  const int p = blockIdx.x;
  const int layer = blockIdx.y;
  char* base = (blockIdx.z == 0 ? kc : vc) + (int64_t)layer * layer_stride_b;
  const int64_t blk_b = (int64_t)nvec * sizeof(V);
  const V* src = reinterpret_cast<const V*>(base + (int64_t)pairs[2 * p] * blk_b);
  V* dst = reinterpret_cast<V*>(base + (int64_t)pairs[2 * p + 1] * blk_b);
  for (int i = threadIdx.x; i < nvec; i += blockDim.x) dst[i] = src[i];
}

inline bool aligned(const void* p, int64_t a) { return ((uintptr_t)p % a) == 0; }

// Interleaved-pair rotation with the reference's fp32 rounding: each product
// is rounded, then the difference/sum (vllmlite/attention.py:35-36). Contraction
// into fma is disabled so results match numpy's elementwise float32 math.
__device__ __forceinline__ void rotate_pair(float e, float o, float c, float s, float* oe,
                                            float* oo) {
#pragma clang fp contract(off)
  float ec = e * c, os = o * s, es = e * s, oc = o * c;
  *oe = ec - os;
  *oo = es + oc;
}

// TC: cache elements (float; uint16_t bf16 bits or uint8_t FP8 E4M3 bytes,
// rounded to nearest even)
template <typename TC>
__global__ void __launch_bounds__(256) rope_and_cache_kernel(
    const float* __restrict__ qkv, int64_t qkv_stride, float* __restrict__ q_out,
    TC* __restrict__ kc, TC* __restrict__ vc, const int32_t* __restrict__ positions,
    const int32_t* __restrict__ slots, const float* __restrict__ cos_t,
    const float* __restrict__ sin_t, int64_t num_tokens, int nh, int nkv, int hd, KvGeom g) {
  const int half = hd >> 1;
  const int q_pairs = nh * half;
  const int k_pairs = nkv * half;
  const int v_elems = nkv * hd;
  for (int64_t t = blockIdx.x; t < num_tokens; t += gridDim.x) {
    const float* row = qkv + t * qkv_stride;
    const int pos = positions[t];
    const int slot = slots[t];
    const float* c = cos_t + (int64_t)pos * half;
    const float* s = sin_t + (int64_t)pos * half;
    for (int i = threadIdx.x; i < q_pairs + k_pairs; i += blockDim.x) {
      const int pi = (i < q_pairs) ? i : i - q_pairs;
      const int head = pi / half, pr = pi - head * half;
      const float* src = (i < q_pairs ? row : row + nh * hd) + head * hd + 2 * pr;
      float oe, oo;
      rotate_pair(src[0], src[1], c[pr], s[pr], &oe, &oo);
      if (i < q_pairs) {
        float* dst = q_out + t * (int64_t)nh * hd + head * hd + 2 * pr;
        dst[0] = oe;
        dst[1] = oo;
      } else if (slot >= 0) {
        TC* dst = kc + g.at(slot, head) + 2 * pr;
        Elem<TC>::store(dst, 0, oe);
        Elem<TC>::store(dst, 1, oo);
      }
    }
    if (slot >= 0) {
      const float* vs = row + (nh + nkv) * hd;
      for (int i = threadIdx.x; i < v_elems; i += blockDim.x) {
        const int head = i / hd;
        Elem<TC>::store(vc + g.at(slot, head), i - head * hd, vs[i]);
      }
    }
  }
}

// Token ids of a step whose inputs include tokens the previous step chose on
// the device: an id t < 0 stands for prev_ids[-t - 1] (out of range: 0).
__global__ void __launch_bounds__(256) resolve_tokens_kernel(int32_t* __restrict__ tok, int64_t n,
                                                             const int32_t* __restrict__ prev,
                                                             int64_t num_prev) {
  const int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x;
  if (i >= n) return;
  const int32_t t = tok[i];
  if (t < 0) {
    const int64_t j = -(int64_t)t - 1;
    tok[i] = j < num_prev ? prev[j] : 0;
  }
}

}  // namespace

extern "C" int vl_reshape_and_cache(const void* key, const void* value, int64_t key_stride,
                                    int64_t value_stride, void* key_cache, void* value_cache,
                                    const int32_t* slot_mapping, int64_t num_tokens,
                                    int num_kv_heads, int head_dim, int dtype, int kv_layout,
                                    int block_size, void* stream) {
  const int es = vl_cache_elem_bytes(dtype);
  VL_CHECK_ARG(es > 0, "bad dtype %d", dtype);
  VL_CHECK_ARG(num_tokens >= 0 && num_kv_heads > 0 && head_dim > 0, "bad shape");
  KvGeom g;
  if (int rc = vl_kv_geom(kv_layout, block_size, num_kv_heads, head_dim, &g)) return rc;
  if (num_tokens == 0) return VL_OK;
  VL_CHECK_ARG(key && value && key_cache && value_cache && slot_mapping, "null pointer");
  const int64_t row_b = (int64_t)num_kv_heads * head_dim * es;
  const int64_t ks_b = key_stride * es, vs_b = value_stride * es;
  VL_CHECK_ARG(key_stride >= num_kv_heads * (int64_t)head_dim &&
                   value_stride >= num_kv_heads * (int64_t)head_dim,
               "row stride smaller than a row");
  hipStream_t st = (hipStream_t)stream;
  const int grid = (int)(num_tokens < 65536 ? num_tokens : 65536);
  // a contiguous segment: the whole row (token-major) or one head's D elements
  const int64_t seg_b = kv_layout == VL_KV_HEAD_MAJOR ? (int64_t)head_dim * es : row_b;
  auto ok = [&](int64_t a) {
    return seg_b % a == 0 && ks_b % a == 0 && vs_b % a == 0 && aligned(key, a) &&
           aligned(value, a) && aligned(key_cache, a) && aligned(value_cache, a);
  };
  if (ok(16)) {
    const int nvec = (int)(row_b / 16);
    scatter_rows_kernel<uint4><<<grid, nvec < 256 ? ((nvec + 63) / 64) * 64 : 256, 0, st>>>(
        (const char*)key, (const char*)value, ks_b, vs_b, (char*)key_cache, (char*)value_cache,
        slot_mapping, num_tokens, g, es, (int)(seg_b / 16), nvec);
  } else if (ok(4)) {
    const int nvec = (int)(row_b / 4);
    scatter_rows_kernel<uint32_t><<<grid, 256, 0, st>>>(
        (const char*)key, (const char*)value, ks_b, vs_b, (char*)key_cache, (char*)value_cache,
        slot_mapping, num_tokens, g, es, (int)(seg_b / 4), nvec);
  } else if (ok(2)) {
    const int nvec = (int)(row_b / 2);
    scatter_rows_kernel<uint16_t><<<grid, 256, 0, st>>>(
        (const char*)key, (const char*)value, ks_b, vs_b, (char*)key_cache, (char*)value_cache,
        slot_mapping, num_tokens, g, es, (int)(seg_b / 2), nvec);
  } else {
    scatter_rows_kernel<uint8_t><<<grid, 256, 0, st>>>(
        (const char*)key, (const char*)value, ks_b, vs_b, (char*)key_cache, (char*)value_cache,
        slot_mapping, num_tokens, g, es, (int)seg_b, (int)row_b);
  }
  VL_CHECK_LAUNCH();
  return VL_OK;
}

extern "C" int vl_copy_blocks(void* key_cache, void* value_cache, const int32_t* block_pairs,
                              int num_pairs, int num_layers, int64_t layer_stride,
                              int64_t block_elems, int dtype, void* stream) {
  const int es = vl_cache_elem_bytes(dtype);
  VL_CHECK_ARG(es > 0, "bad dtype %d", dtype);
  VL_CHECK_ARG(num_pairs >= 0 && num_layers > 0 && block_elems > 0 && layer_stride >= 0,
               "bad shape");
  VL_CHECK_ARG(num_layers <= 65535, "too many layers");
  if (num_pairs == 0) return VL_OK;
  VL_CHECK_ARG(key_cache && value_cache && block_pairs, "null pointer");
  const int64_t blk_b = block_elems * es, ls_b = layer_stride * es;
  hipStream_t st = (hipStream_t)stream;
  dim3 grid(num_pairs, num_layers, 2);
  if (blk_b % 16 == 0 && ls_b % 16 == 0 && aligned(key_cache, 16) && aligned(value_cache, 16)) {
    copy_blocks_kernel<uint4><<<grid, 256, 0, st>>>((char*)key_cache, (char*)value_cache,
                                                    block_pairs, ls_b, (int)(blk_b / 16));
  } else if (blk_b % 4 == 0 && ls_b % 4 == 0 && aligned(key_cache, 4) && aligned(value_cache, 4)) {
    copy_blocks_kernel<uint32_t><<<grid, 256, 0, st>>>((char*)key_cache, (char*)value_cache,
                                                       block_pairs, ls_b, (int)(blk_b / 4));
  } else if (blk_b % 2 == 0 && ls_b % 2 == 0 && aligned(key_cache, 2) && aligned(value_cache, 2)) {
    copy_blocks_kernel<uint16_t><<<grid, 256, 0, st>>>((char*)key_cache, (char*)value_cache,
                                                       block_pairs, ls_b, (int)(blk_b / 2));
  } else {
    copy_blocks_kernel<uint8_t><<<grid, 256, 0, st>>>((char*)key_cache, (char*)value_cache,
                                                      block_pairs, ls_b, (int)blk_b);
  }
  VL_CHECK_LAUNCH();
  return VL_OK;
}

extern "C" int vl_rope_and_cache(const float* qkv, int64_t qkv_stride, float* q_out,
                                 void* key_cache, void* value_cache, const int32_t* positions,
                                 const int32_t* slot_mapping, const float* cos_table,
                                 const float* sin_table, int64_t num_tokens, int num_heads,
                                 int num_kv_heads, int head_dim, int cache_dtype, int kv_layout,
                                 int block_size, void* stream) {
  VL_CHECK_ARG(vl_cache_elem_bytes(cache_dtype) > 0, "bad cache dtype %d", cache_dtype);
  VL_CHECK_ARG(num_tokens >= 0 && num_heads > 0 && num_kv_heads > 0 && head_dim > 0 &&
                   head_dim % 2 == 0,
               "bad shape");
  KvGeom g;
  if (int rc = vl_kv_geom(kv_layout, block_size, num_kv_heads, head_dim, &g)) return rc;
  VL_CHECK_ARG(qkv_stride >= (int64_t)(num_heads + 2 * num_kv_heads) * head_dim,
               "qkv row stride too small");
  if (num_tokens == 0) return VL_OK;
  VL_CHECK_ARG(qkv && q_out && key_cache && value_cache && positions && slot_mapping &&
                   cos_table && sin_table,
               "null pointer");
  const int grid = (int)(num_tokens < 65536 ? num_tokens : 65536);
  if (cache_dtype == VL_DTYPE_F32)
    rope_and_cache_kernel<float><<<grid, 128, 0, (hipStream_t)stream>>>(
        qkv, qkv_stride, q_out, (float*)key_cache, (float*)value_cache, positions, slot_mapping,
        cos_table, sin_table, num_tokens, num_heads, num_kv_heads, head_dim, g);
  else if (cache_dtype == VL_DTYPE_BF16)
    rope_and_cache_kernel<uint16_t><<<grid, 128, 0, (hipStream_t)stream>>>(
        qkv, qkv_stride, q_out, (uint16_t*)key_cache, (uint16_t*)value_cache, positions,
        slot_mapping, cos_table, sin_table, num_tokens, num_heads, num_kv_heads, head_dim, g);
  else
    rope_and_cache_kernel<uint8_t><<<grid, 128, 0, (hipStream_t)stream>>>(
        qkv, qkv_stride, q_out, (uint8_t*)key_cache, (uint8_t*)value_cache, positions,
        slot_mapping, cos_table, sin_table, num_tokens, num_heads, num_kv_heads, head_dim, g);
  VL_CHECK_LAUNCH();
  return VL_OK;
}

// One workgroup copies n int32 words; src may be pinned host memory, read
// over the bus by the kernel itself (16-byte loads when both ends allow).
__global__ void __launch_bounds__(256) copy_words_kernel(int32_t* __restrict__ dst,
                                                         const int32_t* __restrict__ src,
                                                         int64_t n) {
  const bool vec = ((((uintptr_t)dst) | ((uintptr_t)src)) & 15) == 0;
  const int64_t n4 = vec ? n / 4 : 0;
  for (int64_t i = threadIdx.x; i < n4; i += 256)
    reinterpret_cast<uint4*>(dst)[i] = reinterpret_cast<const uint4*>(src)[i];
  for (int64_t i = n4 * 4 + threadIdx.x; i < n; i += 256) dst[i] = src[i];
}

extern "C" int vl_copy_words(int32_t* dst, const int32_t* src, int64_t n, void* stream) {
  VL_CHECK_ARG(n >= 0, "bad count");
  if (n == 0) return VL_OK;
  VL_CHECK_ARG(dst && src, "null pointer");
  copy_words_kernel<<<1, 256, 0, (hipStream_t)stream>>>(dst, src, n);
  VL_CHECK_LAUNCH();
  return VL_OK;
}

extern "C" int vl_resolve_tokens(int32_t* token_ids, int64_t num_tokens, const int32_t* prev_ids,
                                 int64_t num_prev, void* stream) {
  VL_CHECK_ARG(num_tokens >= 0 && num_prev >= 0, "bad counts");
  if (num_tokens == 0) return VL_OK;
  VL_CHECK_ARG(token_ids && (prev_ids || num_prev == 0), "null pointer");
  const int64_t grid = (num_tokens + 255) / 256;
  VL_CHECK_ARG(grid < (1ll << 31), "too many tokens");
  resolve_tokens_kernel<<<(unsigned)grid, 256, 0, (hipStream_t)stream>>>(token_ids, num_tokens,
                                                                         prev_ids, num_prev);
  VL_CHECK_LAUNCH();
  return VL_OK;
}
