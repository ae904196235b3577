// K6 fp32 projections of the TinyLlama forward, with the RMSNorm before them
// and the residual add or SwiGLU gate after them fused in
// (vllmlite/model.py:96-101, 114, 116-117, 119-120). Built for few token rows
// (the decode steps: at most 16, one row tile), and taking any number of rows
// as 16-row tiles (the prefill steps); on large grids a workgroup takes 2 or 4
// row tiles in turn, so that its weights serve all of them.
//
// One workgroup computes 16 rows x 16 output columns: its kLinWaves (8)
// wavefronts split K into contiguous ranges on v_mfma_f32_16x16x4f32, each
// loading its weight operands straight into registers (all loads in flight at
// once) while the rows of x are staged in LDS and normalised there; the
// partial tiles are summed in wavefront order. hipBLASLt runs these shapes as separate launches of
// ~7 us each; here a projection and its neighbours are one.
//
// Weights come row-major ([k, n] at a row stride) or as 16-column tiles
// ([ceil(n/16), k, 16], the columns past n zero): a workgroup's 16 columns
// are then one contiguous k x 64-byte run, ordered inside so that a lane's
// B operands of 4 consecutive MFMA steps are adjacent (element (k, m), k =
// 16 g + 4 s + j, at 256 g + 4 (16 j + m) + s): a wavefront reads 1 KB per
// 16-byte load instruction (row-major, every k row is a separate 64-byte
// piece read 4 bytes per lane). These kernels run on few workgroups, where
// the number of requests each one issues sets the time.
#include "vl_common.h"

namespace {

constexpr int kRowsMax = 16;                 // rows per workgroup (one row tile)
constexpr int kRowsLimit = kRowsMax * 65535;  // rows per call (grid y)
constexpr int kCols = 16;
#ifndef VL_LIN_WAVES
#define VL_LIN_WAVES 8
#endif
// wavefronts per projection workgroup; they split K, so more of them make the
// serial MFMA chain of each shorter (the kernel is latency-bound at <= 16
// rows): 8 measured 7 % faster per TinyLlama decode step than 4, and the same
// as 16, which spills registers at K = 1024)
constexpr int kLinWaves = VL_LIN_WAVES;
static_assert(kLinWaves == 4 || kLinWaves == 8, "4 or 8 wavefronts");

typedef float f32x4_t __attribute__((ext_vector_type(4)));

// silu(g) * u with each step rounded like numpy's float32 elementwise ops
__device__ __forceinline__ float silu_times_f32(float g, float u) {
#pragma clang fp contract(off)
  const float s = g / (1.0f + expf(-g));
  return s * u;
}

// Interleaved-pair rotation with the reference's fp32 rounding (each product
// rounded, then the difference / sum; vllmlite/attention.py:35-36), as the
// RoPE kernel computes it.
__device__ __forceinline__ void rotate_pair_f32(float e, float o, float c, float s, float* oe,
                                                float* oo) {
#pragma clang fp contract(off)
  float ec = e * c, os = o * s, es = e * s, oc = o * c;
  *oe = ec - os;
  *oo = es + oc;
}

// Where MODE 3 puts the columns [q | k | v] of a fused QKV projection.
struct RopeCache {
  float* q_out;  // [rows, nh * hd]
  void* kc;      // paged cache (layout geom) of kv_dtype elements
  void* vc;
  KvGeom geom;
  const int32_t* positions;
  const int32_t* slots;
  const float* cos_t;  // [max_pos, hd / 2]
  const float* sin_t;
  int nh, nkv, hd;
  int kv_dtype;  // VL_DTYPE_F32, or VL_DTYPE_BF16 / VL_DTYPE_FP8_E4M3 (rounded to nearest even)
};

__device__ __forceinline__ void store_cache(void* cache, int64_t i, float v, int dtype) {
  if (dtype == VL_DTYPE_BF16)
    static_cast<uint16_t*>(cache)[i] = f32_to_bf16(v);
  else if (dtype == VL_DTYPE_FP8_E4M3)
    static_cast<uint8_t*>(cache)[i] = f32_to_e4m3(v);
  else
    static_cast<float*>(cache)[i] = v;
}

// MODE 0: out = f(x) @ w; 1: out += f(x) @ w; 2: out = silu(f(x) @ w[:, :n]) *
// (f(x) @ w[:, up_off : up_off + n]); 3: f(x) @ w is a [q | k | v] row: q and k
// rotated by RoPE, q to rc.q_out, k and v to the caches at the row's slot.
// f(x) = x, or with NORM the RMSNorm of x (as rms_norm_kernel computes it)
// times norm_w.
// TILES: the weight is in 16-column tiles (ldw unused; up_off counts
// elements, the start of the up tiles).
template <int MODE, bool NORM, int KMAX, bool TILES>
__global__ void __launch_bounds__(64 * kLinWaves) linear_rows_kernel(
    float* __restrict__ out, int64_t ldo, const float* __restrict__ x, int64_t ldx,
    const float* __restrict__ w, int64_t ldw, int64_t up_off, const float* __restrict__ norm_w,
    float eps, int M, int K, int N, const RopeCache rc, const int32_t* __restrict__ row_index,
    float* __restrict__ x_out, int nsub) {
  constexpr int kSlices = MODE == 2 ? 2 : 1;
  constexpr int KP = KMAX + 4;  // xs row stride: rows 4 words apart, so the
                                // 16 rows x 4 k of an A read hit 64 banks
  constexpr int kSteps = KMAX / (4 * kLinWaves);  // 16x16x4 steps per wavefront at K = KMAX
  static_assert(kSteps % 4 == 0, "whole groups of 4 steps");
  __shared__ float xs[kRowsMax * KP];
  __shared__ float red[kSlices][kLinWaves][kRowsMax * kCols];
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int c0 = blockIdx.x * kCols;
  const int m = lane & 15, j = lane >> 4;
  // wavefront w takes the spw steps of 4 k from step w spw (k in [kb, kb + 4
  // nsteps)); the last wavefronts may have fewer steps, or none
  // (spw is a multiple of 4: the tiled weights hold 4 steps per 16-byte load)
  const int spw = ((K / 4 + kLinWaves - 1) / kLinWaves + 3) / 4 * 4;
  const int kb = wave * spw * 4;
  const int nsteps = max(0, min(spw, K / 4 - wave * spw));
  // ---- the epilogue's own global reads for the row tile at r0, issued early
  // so that they arrive with the weights (tile 0) or the rows instead of
  // after the reduction: thread t writes row t / 16, column c0 + t % 16; the
  // residual it adds to (MODE 1), or its slot and its RoPE table entries
  // (MODE 3)
  const int er = tid / kCols, ec = tid - (tid / kCols) * kCols;
  const int M_all = M;  // M is the current tile's row count from here on
  float e_resid = 0.f, e_cos = 0.f, e_sin = 0.f;
  int e_slot = -1;
  auto epilogue_reads = [&](int r0) {
    const bool ok = er < min(kRowsMax, M_all - r0) && c0 + ec < N;
    if constexpr (MODE == 1) {
      if (ok) e_resid = out[(int64_t)(r0 + er) * ldo + c0 + ec];
    } else if constexpr (MODE == 3) {
      if (ok) {
        const int col = c0 + ec, qd = rc.nh * rc.hd, kd = rc.nkv * rc.hd;
        e_slot = rc.slots[r0 + er];
        if (col < qd + kd) {
          const int base = col < qd ? col : col - qd;
          const int64_t tab =
              (int64_t)rc.positions[r0 + er] * (rc.hd >> 1) + ((base % rc.hd) >> 1);
          e_cos = rc.cos_t[tab];
          e_sin = rc.sin_t[tab];
        }
      }
    }
  };
  epilogue_reads(blockIdx.y * nsub * kRowsMax);

  // ---- the B operand straight into registers: step i of wavefront w needs
  // w[kb + 4i + l/16][c0 + l%16] in lane l (columns past the end read 0);
  // every load is issued before any is used
  // (loads outside the shape read a clamped, valid element that is then
  // multiplied by 0: columns past N, and steps past this wavefront's nsteps,
  // whose A values belong to the next wavefront's range. A select would let
  // the compiler turn each load into a branch that waits for it.)
  float wb[kSlices][kSteps];
  const float colmask = c0 + m < N ? 1.f : 0.f;
#pragma unroll
  for (int s = 0; s < kSlices; ++s) {
    if constexpr (TILES) {
      // tile blockIdx.x: element (k, m), k = 16 g + 4 s + j, at 256 g + 4 (16 j
      // + m) + s, so lane l's operands of the 4 steps of group g are one
      // float4 and a wavefront reads 1 KB per load (groups clamped below K / 16;
      // kb and nsteps are multiples of 16 and 4)
      const float4* src = reinterpret_cast<const float4*>(w + (s ? up_off : 0) +
                                                          (int64_t)blockIdx.x * K * kCols) +
                          lane;
#pragma unroll
      for (int g = 0; g < kSteps / 4; ++g) {
        const float4 v = src[(int64_t)min(kb / 16 + g, K / 16 - 1) * 64];
        const float z = 4 * g < nsteps ? colmask : 0.f;
        wb[s][4 * g] = v.x * z;
        wb[s][4 * g + 1] = v.y * z;
        wb[s][4 * g + 2] = v.z * z;
        wb[s][4 * g + 3] = v.w * z;
      }
    } else {
      const float* src = w + (s ? up_off : 0) + min(c0 + m, N - 1);
#pragma unroll
      for (int i = 0; i < kSteps; ++i)
        wb[s][i] = src[(int64_t)(min(kb + 4 * i, K - 4) + j) * ldw] * (i < nsteps ? colmask : 0.f);
    }
  }
  // the norm weights of this lane's columns k = lane + 64 i (clamped loads)
  float gw[KMAX / 64];
  if constexpr (NORM) {
#pragma unroll
    for (int i = 0; i < KMAX / 64; ++i) gw[i] = norm_w[min(lane + 64 * i, K - 1)];
  }
  // row tiles blockIdx.y nsub + t (t < nsub), rows r0 .. r0 + 15 each, one
  // after the other on the weights already in registers; every row index
  // below counts from the tile's r0. The barriers of each tile also order the
  // previous tile's LDS reads (its A operands and reduction) before this
  // tile's writes.
  for (int t = 0; t < nsub; ++t) {
    const int r0 = (blockIdx.y * nsub + t) * kRowsMax;
    if (r0 >= M_all) break;  // uniform over the workgroup
    M = min(kRowsMax, M_all - r0);
    const int32_t* row_index_t = row_index ? row_index + r0 : nullptr;
    const float* x_t = row_index ? x : x + (int64_t)r0 * ldx;
    float* out_t = MODE != 3 ? out + (int64_t)r0 * ldo : out;
    float* x_out_t = x_out ? x_out + (int64_t)r0 * K : nullptr;
    float* q_out = MODE == 3 ? rc.q_out + (int64_t)r0 * rc.nh * rc.hd : nullptr;
    if (t > 0) epilogue_reads(r0);
    const bool e_ok = er < M && c0 + ec < N;
    // ---- x rows to LDS (rows >= M are zero): thread t < 256 takes row t / 16
    // and float4 columns t % 16 + 16 u; row r is x[row_index[r]] when an index
    // is given, and workgroup 0 copies the rows it read to x_out when given
    if (tid < 16 * kRowsMax) {
      const int r = tid >> 4, q = tid & 15;
      const int kq = K / 4;
      float4 xv[KMAX / 64];
      const int rr = min(r, M - 1);
      const float* xr = x_t + (int64_t)(row_index_t ? row_index_t[rr] : rr) * ldx;
#pragma unroll
      for (int u = 0; u < KMAX / 64; ++u) {
        const int k4 = q + 16 * u;
        const float z = r < M && k4 < kq ? 1.f : 0.f;  // rows past M, columns past K: 0
        const float4 v = *reinterpret_cast<const float4*>(xr + 4 * min(k4, kq - 1));
        xv[u] = make_float4(v.x * z, v.y * z, v.z * z, v.w * z);
      }
#pragma unroll
      for (int u = 0; u < KMAX / 64; ++u)
        *reinterpret_cast<float4*>(&xs[r * KP + 4 * (q + 16 * u)]) = xv[u];
      if (x_out_t && blockIdx.x == 0 && r < M) {
#pragma unroll
        for (int u = 0; u < KMAX / 64; ++u)
          if (q + 16 * u < kq)
            *reinterpret_cast<float4*>(x_out_t + (int64_t)r * K + 4 * (q + 16 * u)) = xv[u];
      }
    }
    __syncthreads();

    if constexpr (NORM) {
      // rows r = wave, wave + kLinWaves, ...: the sum of squares over k = lane +
      // 64 i in increasing i, then the wavefront sum, as rms_norm_kernel (the
      // rows of a wavefront interleaved; columns past K hold zeros)
      constexpr int kRq = kRowsMax / kLinWaves;
      float ss[kRq];
#pragma unroll
      for (int q = 0; q < kRq; ++q) ss[q] = 0.f;
#pragma unroll
      for (int i = 0; i < KMAX / 64; ++i)
#pragma unroll
        for (int q = 0; q < kRq; ++q) {
          const float a = xs[(wave + kLinWaves * q) * KP + lane + 64 * i];
          ss[q] += a * a;
        }
#pragma unroll
      for (int q = 0; q < kRq; ++q) {
        const float rms = sqrtf(wave_sum(ss[q]) / (float)K + eps);
        float* row = &xs[(wave + kLinWaves * q) * KP + lane];
#pragma unroll
        for (int i = 0; i < KMAX / 64; ++i)
          if (lane + 64 * i < K) row[64 * i] = (row[64 * i] / rms) * gw[i];
      }
      __syncthreads();
    }

    // ---- lane l supplies A[l%16][l/16] and B[l/16][l%16] of each 16x16x4 step
    // four independent accumulators per slice (steps i % 4), so consecutive
    // MFMAs do not wait for each other's results
    constexpr int kAcc = kSteps >= 4 ? 4 : 1;
    f32x4_t acc4[kSlices][kAcc];
#pragma unroll
    for (int s = 0; s < kSlices; ++s)
#pragma unroll
      for (int q = 0; q < kAcc; ++q) acc4[s][q] = (f32x4_t){0.f, 0.f, 0.f, 0.f};
    const float* arow = &xs[m * KP + kb + j];
    // all A reads first, then the MFMA chain (the reads of steps past this
    // wavefront's nsteps stay inside the row, below KMAX, and meet zero weights)
    float av[kSteps];
#pragma unroll
    for (int i = 0; i < kSteps; ++i) av[i] = arow[4 * i];
#pragma unroll
    for (int i = 0; i < kSteps; ++i)
#pragma unroll
      for (int s = 0; s < kSlices; ++s)
        acc4[s][i % kAcc] =
            __builtin_amdgcn_mfma_f32_16x16x4f32(av[i], wb[s][i], acc4[s][i % kAcc], 0, 0, 0);
    f32x4_t acc[kSlices];
#pragma unroll
    for (int s = 0; s < kSlices; ++s) {
      acc[s] = acc4[s][0];
#pragma unroll
      for (int q = 1; q < kAcc; ++q) acc[s] += acc4[s][q];
    }
    // C layout: lane l holds rows 4(l/16) + i of column l%16
#pragma unroll
    for (int s = 0; s < kSlices; ++s)
#pragma unroll
      for (int i = 0; i < 4; ++i) red[s][wave][(4 * j + i) * kCols + m] = acc[s][i];
    __syncthreads();

    const int r = er, c = ec;
    if (e_ok) {
      // the wavefronts' partial sums in wavefront order
      auto total = [&](int s, int e) {
        float t = red[s][0][e];
#pragma unroll
        for (int q = 1; q < kLinWaves; ++q) t += red[s][q][e];
        return t;
      };
      float v[kSlices];
#pragma unroll
      for (int s = 0; s < kSlices; ++s) v[s] = total(s, tid);
      if constexpr (MODE == 0) {
        out_t[(int64_t)r * ldo + c0 + c] = v[0];
      } else if constexpr (MODE == 1) {
        out_t[(int64_t)r * ldo + c0 + c] = e_resid + v[0];
      } else if constexpr (MODE == 2) {
        out_t[(int64_t)r * ldo + c0 + c] = silu_times_f32(v[0], v[1]);
      } else {
        // the pair partner of column c is c ^ 1 in the same tile (head_dim even,
        // tiles 16 columns)
        const int pt = r * kCols + (c ^ 1);
        const float partner = total(0, pt);
        const int col = c0 + c, qd = rc.nh * rc.hd, kd = rc.nkv * rc.hd;
        const int slot = e_slot;
        if (col < qd + kd) {
          const int base = col < qd ? col : col - qd;
          const bool odd = (base % rc.hd) & 1;
          float oe, oo;
          rotate_pair_f32(odd ? partner : v[0], odd ? v[0] : partner, e_cos, e_sin, &oe, &oo);
          const float val = odd ? oo : oe;
          if (col < qd)
            q_out[(int64_t)r * qd + col] = val;
          else if (slot >= 0)
            store_cache(rc.kc, rc.geom.at(slot, base / rc.hd) + base % rc.hd, val, rc.kv_dtype);
        } else if (slot >= 0) {
          const int vcol = col - qd - kd;
          store_cache(rc.vc, rc.geom.at(slot, vcol / rc.hd) + vcol % rc.hd, v[0], rc.kv_dtype);
        }
      }
    }
  }
}

#ifndef VL_LIN_SUB_MAX
#define VL_LIN_SUB_MAX 4
#endif
// Row tiles per workgroup: 1 while the grid is at most one round of two
// workgroups per CU (the kernel is latency-bound there, so tiles run side by
// side); beyond that doubled, up to VL_LIN_SUB_MAX, while the grid keeps at
// least that round, so that each workgroup's weight tile serves more rows.
inline int rows_per_workgroup(int ntile, int row_tiles) {
  const int64_t round = 2 * (int64_t)vl_num_cus();
  int nsub = 1;
  while (nsub < VL_LIN_SUB_MAX &&
         (int64_t)ntile * ((row_tiles + 2 * nsub - 1) / (2 * nsub)) >= round)
    nsub *= 2;
  return nsub;
}

template <int MODE, bool NORM, int KMAX>
int launch(float* out, int64_t ldo, const float* x, int64_t ldx, const float* w, int64_t ldw,
           bool tiles, const float* norm_w, float eps, int M, int K, int N, hipStream_t st,
           const int32_t* row_index, const RopeCache& rc = RopeCache{}, float* x_out = nullptr) {
  const int ntile = (N + kCols - 1) / kCols;
  const int row_tiles = (M + kRowsMax - 1) / kRowsMax;
  const int nsub = rows_per_workgroup(ntile, row_tiles);
  const dim3 grid(ntile, (row_tiles + nsub - 1) / nsub);
  if (tiles) {
    const int64_t up_off = MODE == 2 ? (int64_t)ntile * K * kCols : 0;
    linear_rows_kernel<MODE, NORM, KMAX, true><<<grid, 64 * kLinWaves, 0, st>>>(
        out, ldo, x, ldx, w, 0, up_off, norm_w, eps, M, K, N, rc, row_index, x_out, nsub);
  } else {
    const int64_t up_off = MODE == 2 ? N : 0;
    linear_rows_kernel<MODE, NORM, KMAX, false><<<grid, 64 * kLinWaves, 0, st>>>(
        out, ldo, x, ldx, w, ldw, up_off, norm_w, eps, M, K, N, rc, row_index, x_out, nsub);
  }
  VL_CHECK_LAUNCH();
  return VL_OK;
}

}  // namespace

extern "C" int vl_linear_rows(float* out, int64_t out_stride, const float* x, int64_t x_stride,
                              const int32_t* row_index, const float* weight,
                              int64_t weight_stride, const float* norm_weight, float eps,
                              int rows, int k, int n, int mode, void* stream) {
  VL_CHECK_ARG(rows >= 0 && rows <= kRowsLimit, "rows must be in 0..%d", kRowsLimit);
  const bool tiles = (mode & VL_LINEAR_TILES16) != 0;
  mode &= ~VL_LINEAR_TILES16;
  VL_CHECK_ARG(mode >= VL_LINEAR_STORE && mode <= VL_LINEAR_SWIGLU, "bad mode %d", mode);
  VL_CHECK_ARG(k > 0 && k % 16 == 0 && k <= 1024, "k must be a multiple of 16, at most 1024");
  VL_CHECK_ARG(n > 0, "n must be positive");
  if (rows == 0) return VL_OK;
  VL_CHECK_ARG(out && x && weight, "null pointer");
  VL_CHECK_ARG((((uintptr_t)x) & 15) == 0 && x_stride % 4 == 0,
               "x must be 16-byte aligned with a row stride that is a multiple of 4");
  VL_CHECK_ARG(x_stride >= k && out_stride >= n, "row strides too small");
  const int64_t wcols = mode == VL_LINEAR_SWIGLU ? 2 * (int64_t)n : n;
  VL_CHECK_ARG(tiles || weight_stride >= wcols, "weight row stride too small");
  VL_CHECK_ARG(!tiles || (((uintptr_t)weight) & 15) == 0, "tiled weight must be 16-byte aligned");
  hipStream_t st = (hipStream_t)stream;
  const bool nrm = norm_weight != nullptr;
  // KMAX, the unrolled depth, is the smallest of 384 / 512 / 1024 that holds k
#define VL_LINEAR_K(MODE, NORM)                                                              \
  (k <= 384 ? launch<MODE, NORM, 384>(out, out_stride, x, x_stride, weight, weight_stride,    \
                                      tiles, norm_weight, eps, rows, k, n, st, row_index)      \
   : k <= 512 ? launch<MODE, NORM, 512>(out, out_stride, x, x_stride, weight, weight_stride,  \
                                        tiles, norm_weight, eps, rows, k, n, st, row_index)    \
              : launch<MODE, NORM, 1024>(out, out_stride, x, x_stride, weight, weight_stride, \
                                         tiles, norm_weight, eps, rows, k, n, st, row_index))
  switch (mode) {
    case VL_LINEAR_STORE:
      return nrm ? VL_LINEAR_K(0, true) : VL_LINEAR_K(0, false);
    case VL_LINEAR_ACCUMULATE:
      return nrm ? VL_LINEAR_K(1, true) : VL_LINEAR_K(1, false);
    default:
      return nrm ? VL_LINEAR_K(2, true) : VL_LINEAR_K(2, false);
  }
#undef VL_LINEAR_K
}

extern "C" int vl_qkv_rope_cache(float* q_out, void* key_cache, void* value_cache,
                                 const float* x, int64_t x_stride, const int32_t* row_index,
                                 float* x_out, const float* weight,
                                 int64_t weight_stride, int weight_layout,
                                 const float* norm_weight, float eps,
                                 const int32_t* positions, const int32_t* slot_mapping,
                                 const float* cos_table, const float* sin_table, int rows, int k,
                                 int num_heads, int num_kv_heads, int head_dim, int cache_dtype,
                                 int kv_layout, int block_size, void* stream) {
  VL_CHECK_ARG(vl_cache_elem_bytes(cache_dtype) > 0, "bad cache dtype %d", cache_dtype);
  KvGeom geom;
  if (num_kv_heads > 0 && head_dim > 0)
    if (int rc = vl_kv_geom(kv_layout, block_size, num_kv_heads, head_dim, &geom)) return rc;
  VL_CHECK_ARG(rows >= 0 && rows <= kRowsLimit, "rows must be in 0..%d", kRowsLimit);
  VL_CHECK_ARG(k > 0 && k % 16 == 0 && k <= 1024, "k must be a multiple of 16, at most 1024");
  VL_CHECK_ARG(num_heads > 0 && num_kv_heads > 0 && head_dim > 0 && head_dim % 2 == 0,
               "bad head shape (head_dim even)");
  if (rows == 0) return VL_OK;
  VL_CHECK_ARG(q_out && key_cache && value_cache && x && weight && positions && slot_mapping &&
                   cos_table && sin_table,
               "null pointer");
  VL_CHECK_ARG((((uintptr_t)x) & 15) == 0 && x_stride % 4 == 0 && x_stride >= k,
               "x must be 16-byte aligned with a row stride that is a multiple of 4");
  const int n = (num_heads + 2 * num_kv_heads) * head_dim;
  VL_CHECK_ARG(weight_layout == VL_WEIGHT_ROWS || weight_layout == VL_WEIGHT_TILES16,
               "bad weight layout %d", weight_layout);
  const bool tiles = weight_layout == VL_WEIGHT_TILES16;
  VL_CHECK_ARG(tiles || weight_stride >= n, "weight row stride too small");
  VL_CHECK_ARG(!tiles || (((uintptr_t)weight) & 15) == 0, "tiled weight must be 16-byte aligned");
  RopeCache rc;
  rc.q_out = q_out, rc.kc = key_cache, rc.vc = value_cache, rc.positions = positions;
  rc.slots = slot_mapping, rc.cos_t = cos_table, rc.sin_t = sin_table;
  rc.nh = num_heads, rc.nkv = num_kv_heads, rc.hd = head_dim;
  rc.kv_dtype = cache_dtype;
  rc.geom = geom;
  hipStream_t st = (hipStream_t)stream;
  const bool nrm = norm_weight != nullptr;
#define VL_QKV(NORM, KM) \
  launch<3, NORM, KM>(nullptr, 0, x, x_stride, weight, weight_stride, tiles, norm_weight, eps, rows, \
                      k, n, st, row_index, rc, x_out)
  if (k <= 384) return nrm ? VL_QKV(true, 384) : VL_QKV(false, 384);
  if (k <= 512) return nrm ? VL_QKV(true, 512) : VL_QKV(false, 512);
  return nrm ? VL_QKV(true, 1024) : VL_QKV(false, 1024);
#undef VL_QKV
}
