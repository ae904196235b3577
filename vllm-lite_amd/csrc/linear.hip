// K6 fp32 projections of the TinyLlama forward, with the RMSNorm before them
// and the residual add or SwiGLU gate after them fused in
// (vllmlite/model.py:96-101, 114, 116-117, 119-120). Built for few token rows
// (the decode steps: at most 16, one row tile), and taking any number of rows
// as 16-row tiles (the prefill steps); on large grids a workgroup takes 2 or 4
// row tiles in turn, so that its weights serve all of them.
//
// One workgroup computes 16 rows x 16 output columns: its kLinWaves (8)
// wavefronts split K into contiguous ranges on v_mfma_f32_16x16x4f32, each
// loading its rows of x and its weights straight into operand registers (all
// loads in flight at once, no LDS stage); the RMSNorm is applied as a per-row
// scale after the product, so the partial tiles and sums of squares meet in
// LDS behind one barrier and are summed in wavefront order. These kernels run
// on few workgroups at <= 16 rows, where the dependent phases of a workgroup
// (not the bytes) set the time: an empty kernel in a graph takes 1.9 us, one
// that loads 40 KB per workgroup 2.3 us.
//
// Weights come row-major ([k, n] at a row stride) or as 16-column tiles
// ([ceil(n/16), k, 16], the columns past n zero): a workgroup's 16 columns
// are then one contiguous k x 64-byte run, ordered inside so that a lane's
// B operands of the 4 MFMA steps of a 16-k group are adjacent (element (k,
// m), k = 16 g + 4 j + s, at 256 g + 4 (16 j + m) + s): a wavefront reads 1 KB
// per 16-byte load instruction, and the same lane's A operands, x[m][16 g + 4
// j + s], are one float4 of the row.
#include "vl_common.h"

namespace {

constexpr int kRowsMax = 16;                 // rows per workgroup (one row tile)
constexpr int kRowsLimit = kRowsMax * 65535;  // rows per call (grid y)
constexpr int kCols = 16;
// wavefronts per projection workgroup; they split K, so more of them make the
// serial MFMA chain of each shorter (the kernel is latency-bound at <= 16
// rows): 8 measured 7 % faster per TinyLlama decode step than 4, and the same
// as 16, which spills registers at K = 1024
constexpr int kLinWaves = 8;
// row tiles a workgroup takes at most (see rows_per_workgroup)
constexpr int kSubMax = 4;

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
  // a record copied by the same launch (rec_n words from rec_src to rec_dst),
  // or none (rec_n 0)
  const int32_t* rec_src;
  int32_t* rec_dst;
  int64_t rec_n;
};

// Where MODE 4 puts each row's argmax (vl_linear_rows_argmax). Every
// workgroup folds its tiles' columns into keys[row] with one 64-bit atomic
// max per row and then arrives at count; the last to arrive turns the keys
// into ids and clears keys and count for the next launch.
struct ArgmaxOut {
  unsigned long long* keys;  // [rows], zero before and after a launch
  unsigned* count;           // zero before and after a launch
  int32_t* ids;
  int32_t* host_ids;  // a second copy (pinned host memory), or null
};

// A key whose unsigned order is numpy's argmax order: the high word orders
// the values (every NaN above +inf, -0 as +0), the low word prefers the
// lower column among equal values.
__device__ __forceinline__ unsigned long long argmax_key(float v, int col) {
  const unsigned b = __float_as_uint(v);
  const unsigned o = v != v ? 0xFFFFFFFFu
                     : v == 0.f ? 0x80000000u
                     : (b & 0x80000000u) ? ~b
                                         : (b | 0x80000000u);
  return ((unsigned long long)o << 32) | (0xFFFFFFFFu - (unsigned)col);
}

__device__ __forceinline__ void store_cache(void* cache, int64_t i, float v, int dtype) {
  if (dtype == VL_DTYPE_BF16)
    static_cast<uint16_t*>(cache)[i] = f32_to_bf16(v);
  else if (dtype == VL_DTYPE_FP8_E4M3)
    static_cast<uint8_t*>(cache)[i] = f32_to_e4m3(v);
  else
    static_cast<float*>(cache)[i] = v;
}

// MODE 0: out = f(x) @ w (4: and each row's argmax to am); 1: out += f(x) @
// w; 2: out = silu(f(x) @ w[:, :n]) * (f(x) @ w[:, up_off : up_off + n]); 3:
// f(x) @ w is a [q | k | v] row: q and k rotated by RoPE, q to rc.q_out, k and
// v to the caches at the row's slot (and rc's record copied, when it has one).
// f(x) = x, or with NORM the RMSNorm of x times norm_w, applied as
// ((x * norm_w) @ w) / rms(x): the per-row scale 1 / rms commutes with the
// product, so no wavefront waits for another's rows before its MFMAs.
// TILES: the weight is in 16-column tiles (ldw unused; up_off counts
// elements, the start of the up tiles).
//
// Lane l = 16 j + m of wavefront w holds, for each 16-k group g of the
// wavefront's contiguous k range, x[row m][16 g + 4 j .. +3] (one float4
// straight from global memory: no LDS stage) and the weights w[16 g + 4 j +
// s][c0 + m], s = 0..3 (one float4 of a tile); step s of group g is then one
// v_mfma_f32_16x16x4f32 with A = x[m][16 g + 4 j + s], B = w[16 g + 4 j +
// s][c0 + m]. The 8 wavefronts' partial 16 x 16 tiles (and, with NORM, each
// lane's sum of x^2 over its k) meet in LDS behind the kernel's one barrier
// and are summed in wavefront order, so every run gives the same bits.
// NP > 0: the input rows are x[r] + x_parts[r, 0] + ... + x_parts[r, NP - 1]
// (rows of K, summed in that order; vl_linear_rows_parts).
template <int MODE, bool NORM, int KMAX, bool TILES, int NP = 0>
__global__ void __launch_bounds__(64 * kLinWaves) linear_rows_kernel(
    float* __restrict__ out, int64_t ldo, const float* __restrict__ x, int64_t ldx,
    const float* __restrict__ w, int64_t ldw, int64_t up_off, const float* __restrict__ norm_w,
    float eps, int M, int K, int N, const RopeCache rc, const int32_t* __restrict__ row_index,
    const int32_t* __restrict__ prev_ids, int64_t num_prev, float* __restrict__ x_out,
    int nsub, int rt, const float* __restrict__ x_parts = nullptr,
    const ArgmaxOut am = ArgmaxOut{}) {
  constexpr int kSlices = MODE == 2 ? 2 : 1;
  constexpr int kGroups = KMAX / (16 * kLinWaves);  // 16-k groups per wavefront at K = KMAX
  static_assert(kGroups >= 1 && KMAX % (16 * kLinWaves) == 0, "whole 16-k groups");
  __shared__ float red[kSlices][kLinWaves][kRowsMax * kCols];
  __shared__ float4 ssq[kRowsMax][kLinWaves];  // row m: the 4 lanes j of each wavefront
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  // rt rows per row tile (4 or 16); lanes of rows past the tile's end load
  // nothing and feed zeros to the MFMAs
  const int c0 = blockIdx.x * kCols;
  const int m = lane & 15, j = lane >> 4;
  // wavefront w takes the gn 16-k groups from group gb (the last wavefronts may
  // have fewer, or none); loads past them read a clamped, valid group whose
  // weights are then multiplied by 0 (a select would let the compiler turn
  // each load into a branch that waits for it)
  const int ng = K / 16;
  const int gpw = (ng + kLinWaves - 1) / kLinWaves;
  const int gb = wave * gpw;
  const int gn = max(0, min(gpw, ng - gb));
  // ---- the loads of a row tile at r0, in an order that keeps dependent
  // loads from waiting for independent ones (vector loads complete in issue
  // order, so waiting for a load waits for every load issued before it):
  // first the index loads (lane m: its input row; epilogue thread t: its
  // row's slot and position), then the weights (once, for every tile), then
  // x at the indexed rows, then the epilogue's reads (the residual, or the
  // RoPE table entries at the position).
  // Input rows: x[r0 + m], or x[row_index[r0 + m]] where an index -(1 + i) <
  // 0 stands for prev_ids[i], the id the previous step chose for its row i (0
  // when i is not below num_prev). Lanes of rows past the tile's end read its
  // last row again (the same addresses: no extra traffic); their results are
  // never stored. Every load is unconditional: a load in a branch whose
  // other side sets zeros makes the compiler wait for it where the two meet.
  const int M_all = M;  // M is the current tile's row count from here on
  const int er = tid / kCols, ec = tid - (tid / kCols) * kCols;
  const bool e_col = c0 + ec < N;
  int in_row = 0, e_pos = 0, e_slot = -1;
  auto index_reads = [&](int r0, int Mt) {
    if (row_index) in_row = row_index[r0 + min(m, Mt - 1)];
    if constexpr (MODE == 3) {
      if (er < Mt && e_col) {
        e_slot = rc.slots[r0 + er];
        e_pos = rc.positions[r0 + er];
      }
    }
  };
  auto load_x = [&](float4 (&xv)[kGroups], int r0, int Mt) {
    int64_t row = r0 + min(m, Mt - 1);
    if (row_index) {
      row = in_row;
      if (prev_ids && num_prev > 0) {
        const int64_t i = -row - 1;
        const int64_t pv = prev_ids[min(max(i, (int64_t)0), num_prev - 1)];
        row = row >= 0 ? row : (i < num_prev ? pv : 0);
      } else {
        row = max(row, (int64_t)0);
      }
    }
    const float* xr = x + row * ldx;
#pragma unroll
    for (int g = 0; g < kGroups; ++g)
      xv[g] = *reinterpret_cast<const float4*>(xr + 16 * min(gb + g, ng - 1) + 4 * j);
    if constexpr (NP > 0) {
      float4 pv[NP][kGroups];  // every load issued before the first add
      const float* pr = x_parts + row * NP * K;
#pragma unroll
      for (int q = 0; q < NP; ++q)
#pragma unroll
        for (int g = 0; g < kGroups; ++g)
          pv[q][g] =
              *reinterpret_cast<const float4*>(pr + (int64_t)q * K + 16 * min(gb + g, ng - 1) + 4 * j);
#pragma unroll
      for (int g = 0; g < kGroups; ++g)
#pragma unroll
        for (int q = 0; q < NP; ++q) {
          xv[g].x += pv[q][g].x;
          xv[g].y += pv[q][g].y;
          xv[g].z += pv[q][g].z;
          xv[g].w += pv[q][g].w;
        }
    }
  };
  // thread t writes row t / 16, column c0 + t % 16
  float e_resid = 0.f, e_cos = 0.f, e_sin = 0.f;
  auto epilogue_reads = [&](int r0) {
    const bool ok = er < min(rt, M_all - r0) && e_col;
    if constexpr (MODE == 1) {
      if (ok) e_resid = out[(int64_t)(r0 + er) * ldo + c0 + ec];
    } else if constexpr (MODE == 3) {
      const int col = c0 + ec, qd = rc.nh * rc.hd, kd = rc.nkv * rc.hd;
      if (ok && col < qd + kd) {
        const int base = col < qd ? col : col - qd;
        const int64_t tab = (int64_t)e_pos * (rc.hd >> 1) + ((base % rc.hd) >> 1);
        e_cos = rc.cos_t[tab];
        e_sin = rc.sin_t[tab];
      }
    }
  };

  // ---- loads of the first row tile
  const int r00 = blockIdx.y * nsub * rt;
  index_reads(r00, min(rt, M_all - r00));
  // MODE 3 with a record: thread g of the grid copies word g (loaded here,
  // after the index reads, which may read the record's source too; stored at
  // the end) and, in records longer than the grid, words g + grid, ...
  const int64_t rec_g =
      ((int64_t)blockIdx.y * gridDim.x + blockIdx.x) * (64 * kLinWaves) + tid;
  int32_t rec_word = 0;
  if constexpr (MODE == 3) {
    if (rc.rec_n > 0) rec_word = rc.rec_src[min(rec_g, rc.rec_n - 1)];
  }
  // the B operands: lane (m, j), group g, step s needs w[16 (gb + g) + 4 j +
  // s][c0 + m]; in a tile that is one float4 at 256 (gb + g) + 4 (16 j + m)
  float4 wv[kSlices][kGroups];
  const float colmask = c0 + m < N ? 1.f : 0.f;
#pragma unroll
  for (int s = 0; s < kSlices; ++s) {
#pragma unroll
    for (int g = 0; g < kGroups; ++g) {
      const int gg = min(gb + g, ng - 1);
      float4 v;
      if constexpr (TILES) {
        v = reinterpret_cast<const float4*>(w + (s ? up_off : 0) +
                                            (int64_t)blockIdx.x * K * kCols)[gg * 64 + lane];
      } else {
        const float* src = w + (s ? up_off : 0) + min(c0 + m, N - 1) + (16 * gg + 4 * j) * ldw;
        v = make_float4(src[0], src[ldw], src[2 * ldw], src[3 * ldw]);
      }
      const float z = g < gn ? colmask : 0.f;
      wv[s][g] = make_float4(v.x * z, v.y * z, v.z * z, v.w * z);
    }
  }
  // the norm weights of the same k (16-byte aligned, checked by the host)
  float4 gq[NORM ? kGroups : 1];
  if constexpr (NORM) {
#pragma unroll
    for (int g = 0; g < kGroups; ++g)
      gq[g] = *reinterpret_cast<const float4*>(norm_w + 16 * min(gb + g, ng - 1) + 4 * j);
  }
  float4 xv[kGroups];
  load_x(xv, r00, min(rt, M_all - r00));
  epilogue_reads(r00);

  // row tiles blockIdx.y nsub + t (t < nsub), rows r0 .. r0 + 15 each, one
  // after the other on the weights already in registers; every row index
  // below counts from the tile's r0
  for (int t = 0; t < nsub; ++t) {
    const int r0 = (blockIdx.y * nsub + t) * rt;
    if (r0 >= M_all) break;  // uniform over the workgroup
    M = min(rt, M_all - r0);
    if (t > 0) {
      index_reads(r0, M);
      load_x(xv, r0, M);
      epilogue_reads(r0);
      __syncthreads();  // the previous tile's reads of red / ssq are done
    }
    float* out_t = MODE != 3 ? out + (int64_t)r0 * ldo : out;
    float* q_out = MODE == 3 ? rc.q_out + (int64_t)r0 * rc.nh * rc.hd : nullptr;
    // layer 0 writes the rows it gathered (workgroup 0 of each row tile)
    if (x_out && blockIdx.x == 0 && m < M) {
#pragma unroll
      for (int g = 0; g < kGroups; ++g)
        if (g < gn)
          *reinterpret_cast<float4*>(x_out + (int64_t)(r0 + m) * K + 16 * (gb + g) + 4 * j) = xv[g];
    }
    // ---- sum of squares of this lane's x (in k order), x * norm_w, and the
    // MFMA chain: four accumulators per slice (step s of every group), so
    // consecutive MFMAs do not wait for each other's results
    float ss = 0.f;
    f32x4_t acc4[kSlices][4];
#pragma unroll
    for (int s = 0; s < kSlices; ++s)
#pragma unroll
      for (int q = 0; q < 4; ++q) acc4[s][q] = (f32x4_t){0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int g = 0; g < kGroups; ++g) {
      float a[4] = {xv[g].x, xv[g].y, xv[g].z, xv[g].w};
      if constexpr (NORM) {
        const float b[4] = {gq[g].x, gq[g].y, gq[g].z, gq[g].w};
        float sg = 0.f;
#pragma unroll
        for (int s = 0; s < 4; ++s) sg += a[s] * a[s];
        ss += g < gn ? sg : 0.f;
#pragma unroll
        for (int s = 0; s < 4; ++s) a[s] *= b[s];
      }
#pragma unroll
      for (int s = 0; s < 4; ++s)
#pragma unroll
        for (int sl = 0; sl < kSlices; ++sl) {
          const float bw = s == 0 ? wv[sl][g].x : s == 1 ? wv[sl][g].y : s == 2 ? wv[sl][g].z : wv[sl][g].w;
          acc4[sl][s] = __builtin_amdgcn_mfma_f32_16x16x4f32(a[s], bw, acc4[sl][s], 0, 0, 0);
        }
    }
    // C layout: lane l holds rows 4(l/16) + i of column l%16
#pragma unroll
    for (int sl = 0; sl < kSlices; ++sl) {
      const f32x4_t acc = ((acc4[sl][0] + acc4[sl][1]) + acc4[sl][2]) + acc4[sl][3];
#pragma unroll
      for (int i = 0; i < 4; ++i) red[sl][wave][(4 * j + i) * kCols + m] = acc[i];
    }
    if constexpr (NORM) reinterpret_cast<float*>(&ssq[m][wave])[j] = ss;
    __syncthreads();

    const int r = er, c = ec;
    unsigned long long e_key = 0;  // MODE 4: this thread's (value, column) key
    if (er < M && e_col) {
      // the wavefronts' partial sums in wavefront order
      auto total = [&](int s, int e) {
        float v = red[s][0][e];
#pragma unroll
        for (int q = 1; q < kLinWaves; ++q) v += red[s][q][e];
        return v;
      };
      float rms = 1.f;
      if constexpr (NORM) {
        // sum of x^2 over the row: wavefronts in order, the 4 lanes of each in order
        float s2 = 0.f;
#pragma unroll
        for (int q = 0; q < kLinWaves; ++q) {
          const float4 p = ssq[r][q];
          s2 += ((p.x + p.y) + p.z) + p.w;
        }
        rms = sqrtf(s2 / (float)K + eps);
      }
      float v[kSlices];
#pragma unroll
      for (int s = 0; s < kSlices; ++s) v[s] = NORM ? total(s, tid) / rms : total(s, tid);
      if constexpr (MODE == 0 || MODE == 4) {
        out_t[(int64_t)r * ldo + c0 + c] = v[0];
        if constexpr (MODE == 4) e_key = argmax_key(v[0], c0 + c);
      } else if constexpr (MODE == 1) {
        out_t[(int64_t)r * ldo + c0 + c] = e_resid + v[0];
      } else if constexpr (MODE == 2) {
        out_t[(int64_t)r * ldo + c0 + c] = silu_times_f32(v[0], v[1]);
      } else {
        // the pair partner of column c is c ^ 1 in the same tile (head_dim even,
        // tiles 16 columns)
        const int pt = r * kCols + (c ^ 1);
        const float partner = NORM ? total(0, pt) / rms : total(0, pt);
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
    if constexpr (MODE == 4) {
      // the largest key of each row's 16 threads (lanes 16 u .. 16 u + 15 of
      // a wavefront), one atomic max per row; waves past the tile's 16 rows
      // hold none
      if (tid < kRowsMax * kCols) {
#pragma unroll
        for (int o = 8; o > 0; o >>= 1) {
          const unsigned long long other = __shfl_xor(e_key, o, 64);
          e_key = other > e_key ? other : e_key;
        }
        if (ec == 0 && e_key != 0)
          __hip_atomic_fetch_max(am.keys + r0 + er, e_key, __ATOMIC_RELAXED,
                                 __HIP_MEMORY_SCOPE_AGENT);
      }
    }
  }
  if constexpr (MODE == 4) {
    __shared__ int last;
    asm volatile("s_waitcnt vmcnt(0)" ::: "memory");  // this thread's atomics have completed
    __syncthreads();
    if (tid == 0)
      last = __hip_atomic_fetch_add(am.count, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) ==
             gridDim.x * gridDim.y - 1;
    __syncthreads();
    if (last) {  // every workgroup's maxima are in: the ids, and the keys cleared
      for (int r = tid; r < M_all; r += 64 * kLinWaves) {
        const unsigned long long k =
            __hip_atomic_exchange(am.keys + r, 0ull, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        const int32_t id = (int32_t)(0xFFFFFFFFu - (unsigned)(k & 0xFFFFFFFFull));
        am.ids[r] = id;
        if (am.host_ids) am.host_ids[r] = id;
      }
      if (tid == 0) __hip_atomic_store(am.count, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    }
  }
  if constexpr (MODE == 3) {
    if (rc.rec_n > 0) {
      if (rec_g < rc.rec_n) rc.rec_dst[rec_g] = rec_word;
      const int64_t grid_threads = (int64_t)gridDim.x * gridDim.y * (64 * kLinWaves);
      for (int64_t w = rec_g + grid_threads; w < rc.rec_n; w += grid_threads)
        rc.rec_dst[w] = rc.rec_src[w];
    }
  }
}

// Row tiles per workgroup: 1 while the grid is at most one round of two
// workgroups per CU (the kernel is latency-bound there, so tiles run side by
// side); beyond that doubled, up to kSubMax, while the grid keeps at
// least that round, so that each workgroup's weight tile serves more rows.
inline int rows_per_workgroup(int ntile, int row_tiles) {
  const int64_t round = 2 * (int64_t)vl_num_cus();
  int nsub = 1;
  while (nsub < kSubMax &&
         (int64_t)ntile * ((row_tiles + 2 * nsub - 1) / (2 * nsub)) >= round)
    nsub *= 2;
  return nsub;
}

// Rows per row tile. A step of at most 16 rows (a decode step) runs as row
// tiles of 4, a workgroup per (16 columns, 4 rows), while that grid stays
// within one round of two workgroups per CU: a workgroup then loads a quarter
// of the rows of x, and the last of its wavefronts to receive its operands,
// which sets the time, waits less (measured per TinyLlama decode layer, 16
// rows: QKV 3.55 -> 3.16 us, gate|up 3.65 -> 3.32, down 4.16 -> 3.24; rows of
// 8, or 8 columns per workgroup, were slower). Larger steps use 16-row tiles,
// several per workgroup on large grids (rows_per_workgroup).
inline int row_tile(int M, int N) {
  const int64_t ntile = (N + kCols - 1) / kCols;
  if (M <= kRowsMax && ntile * ((M + 3) / 4) <= 2 * (int64_t)vl_num_cus()) return 4;
  return kRowsMax;
}

template <int MODE, bool NORM, int KMAX, int NP = 0>
int launch(float* out, int64_t ldo, const float* x, int64_t ldx, const float* w, int64_t ldw,
           bool tiles, const float* norm_w, float eps, int M, int K, int N, hipStream_t st,
           const int32_t* row_index, const RopeCache& rc = RopeCache{}, float* x_out = nullptr,
           const int32_t* prev_ids = nullptr, int64_t num_prev = 0,
           const float* x_parts = nullptr, const ArgmaxOut& am = ArgmaxOut{}) {
  const int ntile = (N + kCols - 1) / kCols;
  const int rt = row_tile(M, N);
  const int row_tiles = (M + rt - 1) / rt;
  const int nsub = rt == kRowsMax ? rows_per_workgroup(ntile, row_tiles) : 1;
  const dim3 grid(ntile, (row_tiles + nsub - 1) / nsub);
  if (tiles) {
    const int64_t up_off = MODE == 2 ? (int64_t)ntile * K * kCols : 0;
    linear_rows_kernel<MODE, NORM, KMAX, true, NP><<<grid, 64 * kLinWaves, 0, st>>>(
        out, ldo, x, ldx, w, 0, up_off, norm_w, eps, M, K, N, rc, row_index, prev_ids, num_prev,
        x_out, nsub, rt, x_parts, am);
  } else if constexpr (NP == 0 && MODE != 4) {
    const int64_t up_off = MODE == 2 ? N : 0;
    linear_rows_kernel<MODE, NORM, KMAX, false><<<grid, 64 * kLinWaves, 0, st>>>(
        out, ldo, x, ldx, w, ldw, up_off, norm_w, eps, M, K, N, rc, row_index, prev_ids,
        num_prev, x_out, nsub, rt);
  }
  VL_CHECK_LAUNCH();
  return VL_OK;
}

template <int NP>
int launch_parts(float* out, int64_t ldo, const float* x, int64_t ldx, const float* x_parts,
                 float* x_out, const float* w, const float* norm_w, float eps, int M, int K, int N,
                 hipStream_t st) {
  const bool nrm = norm_w != nullptr;
  if (K <= 384)
    return nrm ? launch<2, true, 384, NP>(out, ldo, x, ldx, w, 0, true, norm_w, eps, M, K, N, st,
                                          nullptr, RopeCache{}, x_out, nullptr, 0, x_parts)
               : launch<2, false, 384, NP>(out, ldo, x, ldx, w, 0, true, norm_w, eps, M, K, N, st,
                                           nullptr, RopeCache{}, x_out, nullptr, 0, x_parts);
  return nrm ? launch<2, true, 512, NP>(out, ldo, x, ldx, w, 0, true, norm_w, eps, M, K, N, st,
                                        nullptr, RopeCache{}, x_out, nullptr, 0, x_parts)
             : launch<2, false, 512, NP>(out, ldo, x, ldx, w, 0, true, norm_w, eps, M, K, N, st,
                                         nullptr, RopeCache{}, x_out, nullptr, 0, x_parts);
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
  VL_CHECK_ARG((((uintptr_t)norm_weight) & 15) == 0, "norm weight must be 16-byte aligned");
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
                                 const int32_t* prev_ids, int64_t num_prev,
                                 float* x_out, const float* weight,
                                 int64_t weight_stride, int weight_layout,
                                 const float* norm_weight, float eps,
                                 const int32_t* positions, const int32_t* slot_mapping,
                                 const float* cos_table, const float* sin_table, int rows, int k,
                                 int num_heads, int num_kv_heads, int head_dim, int cache_dtype,
                                 int kv_layout, int block_size, const int32_t* record_src,
                                 int32_t* record_dst, int64_t record_words, void* stream) {
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
  VL_CHECK_ARG((((uintptr_t)norm_weight) & 15) == 0, "norm weight must be 16-byte aligned");
  VL_CHECK_ARG(num_prev >= 0 && (num_prev == 0 || (prev_ids && row_index)),
               "prev_ids needs row_index (and num_prev > 0 needs prev_ids)");
  VL_CHECK_ARG(record_words >= 0 && (record_words == 0 || (record_src && record_dst)),
               "a record needs its source and destination");
  RopeCache rc;
  rc.q_out = q_out, rc.kc = key_cache, rc.vc = value_cache, rc.positions = positions;
  rc.slots = slot_mapping, rc.cos_t = cos_table, rc.sin_t = sin_table;
  rc.nh = num_heads, rc.nkv = num_kv_heads, rc.hd = head_dim;
  rc.kv_dtype = cache_dtype;
  rc.geom = geom;
  rc.rec_src = record_src, rc.rec_dst = record_dst, rc.rec_n = record_words;
  hipStream_t st = (hipStream_t)stream;
  const bool nrm = norm_weight != nullptr;
#define VL_QKV(NORM, KM) \
  launch<3, NORM, KM>(nullptr, 0, x, x_stride, weight, weight_stride, tiles, norm_weight, eps, rows, \
                      k, n, st, row_index, rc, x_out, prev_ids, num_prev)
  if (k <= 384) return nrm ? VL_QKV(true, 384) : VL_QKV(false, 384);
  if (k <= 512) return nrm ? VL_QKV(true, 512) : VL_QKV(false, 512);
  return nrm ? VL_QKV(true, 1024) : VL_QKV(false, 1024);
#undef VL_QKV
}

extern "C" int vl_linear_rows_parts(float* out, int64_t out_stride, const float* x,
                                    int64_t x_stride, const float* x_parts, int num_parts,
                                    float* x_out, const float* weight, const float* norm_weight,
                                    float eps, int rows, int k, int n, void* stream) {
  VL_CHECK_ARG(rows >= 0 && rows <= kRowsLimit, "rows must be in 0..%d", kRowsLimit);
  VL_CHECK_ARG(k > 0 && k % 16 == 0 && k <= 512, "k must be a multiple of 16, at most 512");
  VL_CHECK_ARG(n > 0, "n must be positive");
  VL_CHECK_ARG(num_parts == 1 || num_parts == 2 || num_parts == 4 || num_parts == 8,
               "num_parts must be 1, 2, 4 or 8");
  if (rows == 0) return VL_OK;
  VL_CHECK_ARG(out && x && x_parts && weight, "null pointer");
  VL_CHECK_ARG((((uintptr_t)x) & 15) == 0 && x_stride % 4 == 0 && x_stride >= k,
               "x must be 16-byte aligned with a row stride that is a multiple of 4");
  VL_CHECK_ARG((((uintptr_t)x_parts) & 15) == 0 && (!x_out || (((uintptr_t)x_out) & 15) == 0),
               "x_parts and x_out must be 16-byte aligned");
  VL_CHECK_ARG(out_stride >= n, "row stride too small");
  VL_CHECK_ARG((((uintptr_t)weight) & 15) == 0, "tiled weight must be 16-byte aligned");
  VL_CHECK_ARG((((uintptr_t)norm_weight) & 15) == 0, "norm weight must be 16-byte aligned");
  VL_CHECK_ARG(x_out != x, "x_out must not be x (other workgroups still read x)");
  hipStream_t st = (hipStream_t)stream;
  switch (num_parts) {
    case 1: return launch_parts<1>(out, out_stride, x, x_stride, x_parts, x_out, weight, norm_weight, eps, rows, k, n, st);
    case 2: return launch_parts<2>(out, out_stride, x, x_stride, x_parts, x_out, weight, norm_weight, eps, rows, k, n, st);
    case 4: return launch_parts<4>(out, out_stride, x, x_stride, x_parts, x_out, weight, norm_weight, eps, rows, k, n, st);
    default: return launch_parts<8>(out, out_stride, x, x_stride, x_parts, x_out, weight, norm_weight, eps, rows, k, n, st);
  }
}

extern "C" int vl_linear_rows_argmax(float* out, int64_t out_stride, const float* x,
                                     int64_t x_stride, const int32_t* row_index,
                                     const float* weight, const float* norm_weight, float eps,
                                     int rows, int k, int n, int32_t* ids, int32_t* host_ids,
                                     void* scratch, int64_t scratch_bytes, void* stream) {
  VL_CHECK_ARG(rows >= 0 && rows <= kRowsLimit, "rows must be in 0..%d", kRowsLimit);
  VL_CHECK_ARG(k > 0 && k % 16 == 0 && k <= 1024, "k must be a multiple of 16, at most 1024");
  VL_CHECK_ARG(n > 0, "n must be positive");
  if (rows == 0) return VL_OK;
  VL_CHECK_ARG(out && x && weight && ids && scratch, "null pointer");
  VL_CHECK_ARG((((uintptr_t)x) & 15) == 0 && x_stride % 4 == 0 && x_stride >= k,
               "x must be 16-byte aligned with a row stride that is a multiple of 4");
  VL_CHECK_ARG(out_stride >= n, "row stride too small");
  VL_CHECK_ARG((((uintptr_t)weight) & 15) == 0, "tiled weight must be 16-byte aligned");
  VL_CHECK_ARG((((uintptr_t)norm_weight) & 15) == 0, "norm weight must be 16-byte aligned");
  VL_CHECK_ARG((((uintptr_t)scratch) & 7) == 0 && scratch_bytes >= 8 * ((int64_t)rows + 1),
               "scratch must be 8-byte aligned and hold rows + 1 8-byte words");
  ArgmaxOut am;
  am.keys = static_cast<unsigned long long*>(scratch);
  am.count = reinterpret_cast<unsigned*>(am.keys + rows);
  am.ids = ids;
  am.host_ids = host_ids;
  hipStream_t st = (hipStream_t)stream;
  const bool nrm = norm_weight != nullptr;
#define VL_ARGMAX(NORM, KM)                                                                     \
  launch<4, NORM, KM>(out, out_stride, x, x_stride, weight, 0, true, norm_weight, eps, rows, k, n, \
                      st, row_index, RopeCache{}, nullptr, nullptr, 0, nullptr, am)
  if (k <= 384) return nrm ? VL_ARGMAX(true, 384) : VL_ARGMAX(false, 384);
  if (k <= 512) return nrm ? VL_ARGMAX(true, 512) : VL_ARGMAX(false, 512);
  return nrm ? VL_ARGMAX(true, 1024) : VL_ARGMAX(false, 1024);
#undef VL_ARGMAX
}
