// Shared device/host helpers for the gfx950 kernels of the paged-attention step.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include "../../include/vllmlite_hip.h"

// ---------------------------------------------------------------- errors ----
// Every entry point returns 0, a negative VL_E* argument error, or a positive
// hipError_t; the message of the last failure on the calling thread is kept
// for vl_last_error().
void vl_set_error(const char* fmt, ...);

#define VL_CHECK_ARG(cond, ...)              \
  do {                                       \
    if (!(cond)) {                           \
      vl_set_error(__VA_ARGS__);             \
      return VL_EINVAL;                      \
    }                                        \
  } while (0)

#define VL_CHECK_HIP(expr)                                                        \
  do {                                                                            \
    hipError_t e_ = (expr);                                                       \
    if (e_ != hipSuccess) {                                                       \
      vl_set_error("%s failed: %s (%s:%d)", #expr, hipGetErrorString(e_), __FILE__, \
                   __LINE__);                                                     \
      return (int)e_;                                                             \
    }                                                                             \
  } while (0)

#define VL_CHECK_LAUNCH() VL_CHECK_HIP(hipGetLastError())

// Number of compute units of the current device (cached per device).
int vl_num_cus();

// ----------------------------------------------------------------- dtypes ---
// bf16 is carried as its raw 16 bits (uint16_t) so that copies stay bit-exact.
__device__ __forceinline__ float bf16_to_f32(uint16_t b) {
  return __uint_as_float(((uint32_t)b) << 16);
}

// Round to nearest even; NaN stays a quiet NaN.
__device__ __forceinline__ uint16_t f32_to_bf16(float f) {
  uint32_t u = __float_as_uint(f);
  if ((u & 0x7fffffffu) > 0x7f800000u) return (uint16_t)((u >> 16) | 0x40);
  u += 0x7fffu + ((u >> 16) & 1u);
  return (uint16_t)(u >> 16);
}

// Low / high bf16 of a packed pair as fp32.
__device__ __forceinline__ float bf16lo(uint32_t w) { return __uint_as_float(w << 16); }
__device__ __forceinline__ float bf16hi(uint32_t w) { return __uint_as_float(w & 0xffff0000u); }

template <typename T>
struct Elem;
template <>
struct Elem<float> {
  static __device__ __forceinline__ float load(const float* p, int64_t i) { return p[i]; }
  static __device__ __forceinline__ void store(float* p, int64_t i, float v) { p[i] = v; }
};
template <>
struct Elem<uint16_t> {
  static __device__ __forceinline__ float load(const uint16_t* p, int64_t i) {
    return bf16_to_f32(p[i]);
  }
  static __device__ __forceinline__ void store(uint16_t* p, int64_t i, float v) {
    p[i] = f32_to_bf16(v);
  }
};

// OCP FP8 E4M3 ("e4m3fn": 4 exponent bits with bias 7, 3 mantissa bits, no
// infinities, 0x7F / 0xFF NaN, largest finite 448), carried as raw bytes.
// Stores round to nearest even and saturate: finite values (and infinities)
// beyond 448 in magnitude become +-448; NaN stays NaN.
__host__ __device__ __forceinline__ uint8_t f32_to_e4m3(float f) {
  const uint32_t u = __builtin_bit_cast(uint32_t, f);
  const uint32_t sign = (u >> 24) & 0x80u;
  const uint32_t a = u & 0x7fffffffu;
  if (a > 0x7f800000u) return (uint8_t)(sign | 0x7fu);  // NaN
  if (a >= 0x43e00000u) return (uint8_t)(sign | 0x7eu);  // |f| >= 448
  if (a < 0x3c800000u) {  // below 2^-6: multiples of 2^-9 (8 is 2^-6, the first normal)
    const float m = __builtin_rintf(__builtin_bit_cast(float, a) * 512.f);
    return (uint8_t)(sign | (uint32_t)m);
  }
  // normal: round the fp32 mantissa to 3 bits (a carry moves the exponent),
  // then rebias the exponent from 127 to 7
  const uint32_t r = a + 0x7ffffu + ((a >> 20) & 1u);
  return (uint8_t)(sign | ((r >> 20) - (120u << 3)));
}

// Four FP8 E4M3 bytes (w, little-endian) to fp32, exactly, by gfx950's
// conversion instruction (v_cvt_pk_f32_fp8 reads OCP E4M3: exponent bias 7,
// 0x7f / 0xff NaN, subnormals m * 2^-9; every code of the cache is checked
// against the oracle's fp8_e4m3_decode through each attention kernel by the
// GPU tests); one instruction per two bytes
__device__ __forceinline__ void e4m3x4_to_f32(uint32_t w, float* r) {
  typedef float f32x2_t __attribute__((ext_vector_type(2)));
  const f32x2_t lo = __builtin_amdgcn_cvt_pk_f32_fp8((int)w, false);
  const f32x2_t hi = __builtin_amdgcn_cvt_pk_f32_fp8((int)w, true);
  r[0] = lo[0], r[1] = lo[1], r[2] = hi[0], r[3] = hi[1];
}

template <>
struct Elem<uint8_t> {
  static __device__ __forceinline__ float load(const uint8_t* p, int64_t i) {
    return __builtin_amdgcn_cvt_f32_fp8((int)p[i], 0);
  }
  static __device__ __forceinline__ void store(uint8_t* p, int64_t i, float v) {
    p[i] = f32_to_e4m3(v);
  }
};

// Element bytes of a VL_DTYPE_* cache dtype (0 if not a cache dtype).
inline int vl_cache_elem_bytes(int dtype) {
  return dtype == VL_DTYPE_F32 ? 4 : dtype == VL_DTYPE_BF16 ? 2 : dtype == VL_DTYPE_FP8_E4M3 ? 1 : 0;
}

// ------------------------------------------------------- wave reductions ----
// 64-lane wavefront reductions through ds_swizzle-free shuffles.
__device__ __forceinline__ float wave_max(float v) {
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) v = fmaxf(v, __shfl_xor(v, o, 64));
  return v;
}
__device__ __forceinline__ float wave_sum(float v) {
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) v += __shfl_xor(v, o, 64);
  return v;
}

__host__ __device__ __forceinline__ int64_t cdiv64(int64_t a, int64_t b) { return (a + b - 1) / b; }
__host__ __device__ __forceinline__ int cdiv(int a, int b) { return (a + b - 1) / b; }

// ----------------------------------------------------------- cache layout ---
// A paged K or V cache in one of two layouts: VL_KV_TOKEN_MAJOR, [num_slots,
// Hkv, D] with slot = block * block_size + offset, or VL_KV_HEAD_MAJOR,
// [num_blocks, Hkv, block_size, D]. A block spans the same block_size * Hkv
// * D elements in both, so block copies do not depend on the layout. The row
// of (slot, KV head h) starts at element
//   (slot >> bs_log2) * blk + (slot & (2^bs_log2 - 1)) * row + h * head
// (token-major: bs_log2 0, blk = row = Hkv * D, head = D; head-major: blk =
// 2^bs_log2 * Hkv * D, row = D, head = 2^bs_log2 * D).
struct KvGeom {
  int64_t blk, row, head;
  int bs_log2;
  __host__ __device__ __forceinline__ int64_t at(int64_t slot, int h) const {
    return (slot >> bs_log2) * blk + (slot & ((1ll << bs_log2) - 1)) * row + (int64_t)h * head;
  }
};

// Checks kv_layout (and, for head-major, that block_size is a power of two)
// and fills *g; a VL_EINVAL return carries its message.
int vl_kv_geom(int kv_layout, int block_size, int num_kv_heads, int head_dim, KvGeom* g);

// ------------------------------------------------- shared device helpers ----
// 2^x by the hardware's v_exp_f32 (about 1 ulp; results below 2^-126 may
// flush to zero, far below a softmax row sum's fp32 resolution). exp2f adds
// a range reduction for denormal results that costs six more VALU ops.
__device__ __forceinline__ float exp2_fast(float x) { return __builtin_amdgcn_exp2f(x); }

// DPP lane exchange (update_dpp with `old` kept where the row mask excludes
// the lane).
#define VL_DPP(old, v, ctrl, rmask)                                                     \
  __int_as_float(__builtin_amdgcn_update_dpp(__float_as_int(old), __float_as_int(v), ctrl, \
                                             rmask, 0xF, false))

// Max / sum over the 64 lanes of a wavefront by DPP: within each row of 16
// (quad xor 1, xor 2, half-row mirror, row mirror), then row 0 into 1 and 2
// into 3 (row_bcast:15), row 1 into 2 and 3 (row_bcast:31); lane 63 holds the
// result, which every lane reads back.
__device__ __forceinline__ float wave_max_dpp(float v) {
  v = fmaxf(v, VL_DPP(v, v, 0xB1, 0xF));
  v = fmaxf(v, VL_DPP(v, v, 0x4E, 0xF));
  v = fmaxf(v, VL_DPP(v, v, 0x141, 0xF));
  v = fmaxf(v, VL_DPP(v, v, 0x140, 0xF));
  v = fmaxf(v, VL_DPP(v, v, 0x142, 0xA));
  v = fmaxf(v, VL_DPP(v, v, 0x143, 0xC));
  return __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), 63));
}
__device__ __forceinline__ float wave_sum_dpp(float v) {
  v += VL_DPP(0.f, v, 0xB1, 0xF);
  v += VL_DPP(0.f, v, 0x4E, 0xF);
  v += VL_DPP(0.f, v, 0x141, 0xF);
  v += VL_DPP(0.f, v, 0x140, 0xF);
  v += VL_DPP(0.f, v, 0x142, 0xA);
  v += VL_DPP(0.f, v, 0x143, 0xC);
  return __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), 63));
}

// 16 bytes of T (fp32, bf16 bits or FP8 E4M3 bytes) as floats
template <typename T>
__device__ __forceinline__ void widen16(const uint4& v, float* r) {
  if constexpr (sizeof(T) == 4) {
    r[0] = __uint_as_float(v.x), r[1] = __uint_as_float(v.y);
    r[2] = __uint_as_float(v.z), r[3] = __uint_as_float(v.w);
  } else if constexpr (sizeof(T) == 1) {
    e4m3x4_to_f32(v.x, r), e4m3x4_to_f32(v.y, r + 4);
    e4m3x4_to_f32(v.z, r + 8), e4m3x4_to_f32(v.w, r + 12);
  } else {
    const uint32_t w[4] = {v.x, v.y, v.z, v.w};
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      r[2 * e] = __uint_as_float(w[e] << 16);
      r[2 * e + 1] = __uint_as_float(w[e] & 0xffff0000u);
    }
  }
}
