// K7 one TinyLlama decode step in one launch, on the compute units of one XCD
// (vllmlite/model.py:80-120 over the batch vllmlite/runner.py:62-100 builds
// when every scheduled sequence pushes one token): the embedding gather, per
// layer RMSNorm + QKV + RoPE + K/V scatter, paged attention over each
// sequence's context, x += attn @ wo, RMSNorm + gate|up + SwiGLU,
// x += act @ w_down; then the final RMSNorm, lm_head and the argmax of every
// row, written to device memory and to the caller's pinned host buffer.
//
// Why one XCD. A decode step of the 6-layer model is ~30 small dependent
// phases. As separate launches each costs 4-7 us, mostly the launch and the
// cache maintenance between kernels; a persistent grid spread over all 8 XCDs
// pays as much per phase, since data and barriers must then pass through
// memory beyond the XCDs' own L2 caches. Workgroups are dispatched to the XCDs
// round-robin (workgroup b runs on XCD (s + b) % 8, s where the dispatcher's
// rotation stands when the launch begins), so a grid of 8 * NW workgroups of
// which only those with b % 8 == 0 stay puts NW workgroups on one XCD,
// where they share one L2: a barrier and the exchange of a phase's results
// (16 rows of 384 floats) then cost ~1.7 us.
//
// Protocol between the workgroups of the launch:
//   * results a later phase reads are written with ordinary stores (the L1 is
//     write-through) and each writer waits for its stores (s_waitcnt) before
//     it arrives at the barrier;
//   * the barrier: one L2 atomic add per workgroup on an arrival counter; the
//     last arriver (it sees the count reach epoch * NW) stores the epoch to a
//     release word on another cache line; the others poll that word;
//   * every read of a buffer that is rewritten during the launch (the
//     exchange rows x, q, attn, act, rewritten every layer, and the logits)
//     and every poll is a device-scope load, which misses the CU's L1 (whose
//     lines may be older than the write) and is served by the L2. The paged
//     K/V takes ordinary loads: the lines of a layer's cache are read only in
//     that layer's attention phase, after the barrier that follows their
//     writes, so no L1 holds an older copy (the L1 starts each launch empty);
//     so do the read-only inputs (weights, the step's record);
//   * the returning atomics execute in the XCD's L2 (the L1 executes none).
// Every participant checks that it runs on the XCD of workgroup 0 (hardware
// register XCC_ID; workgroup 0 publishes its own before the first barrier);
// every wait is bounded (a wait that runs out stops waiting). Either failure
// is reported in host_ids[16] (0 when the launch was good) and the results
// are then not to be used. The last workgroup to leave resets the counters,
// so consecutive launches on one stream reuse the sync words without a
// memset.
//
// Arithmetic: the projections perform the same operations in the same order
// as this library's separate kernels (vl_qkv_rope_cache, vl_linear_rows):
// 16 x 16 tiles on v_mfma_f32_16x16x4f32 with K split over 8 wavefronts and
// their partial tiles summed in wavefront order, RMSNorm over k = lane + 64 i
// then across the wavefront, RoPE / SwiGLU rounded as numpy rounds them; the
// attention is decode_item.h's 8-wavefront item (the short-decode kernel
// sums in another order, so logits agree to ~1e-6, not bit for bit); the
// argmax follows numpy's rule as vl_argmax_rows does.
#include "vl_common.h"
#include "decode_item.h"

namespace {

constexpr int kXcds = 8;
constexpr int kThreads = 512;    // 8 wavefronts: 256 VGPRs each, one workgroup per CU
constexpr int kRows = 16;        // token rows (= sequences) of a step
constexpr int kCols = 16;        // columns of a projection tile
constexpr int kTileWaves = 8;    // wavefronts that split a tile's K
constexpr int kMaxCtx = 2048;    // context per sequence (its block table staged in LDS)
constexpr int kSc1 = 16;         // buffer-load cache policy: device scope (misses the L1)

// sync words (uint32), each on its own 128-byte line
enum : int { kArrive = 0, kRelease = 32, kExit = 64, kLmDone = 96, kXcc = 112, kSyncWords = 128 };

typedef float f32x4_t __attribute__((ext_vector_type(4)));
typedef unsigned u32x4_t __attribute__((ext_vector_type(4)));

// ------------------------------------------------------------ exchange ----
__device__ __forceinline__ unsigned l2_add(unsigned* p, unsigned v) {
  unsigned r;
  asm volatile("global_atomic_add %0, %1, %2, off sc0\n\ts_waitcnt vmcnt(0)"
               : "=v"(r)
               : "v"(p), "v"(v)
               : "memory");
  return r;
}
__device__ __forceinline__ void l2_store(unsigned* p, unsigned v) {
  __hip_atomic_store(p, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP);
}
__device__ __forceinline__ unsigned dev_load(const unsigned* p) {
  return __hip_atomic_load(p, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ float dev_loadf(const float* p) {
  return __uint_as_float(dev_load(reinterpret_cast<const unsigned*>(p)));
}
__device__ __forceinline__ void stores_done() { asm volatile("s_waitcnt vmcnt(0)" ::: "memory"); }

// A buffer of `bytes` bytes at p, for device-scope 16-byte loads.
__device__ __forceinline__ __amdgpu_buffer_rsrc_t rsrc(const void* p, uint32_t bytes) {
  return __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(p), (short)0, (int)bytes,
                                           0x00020000);
}
__device__ __forceinline__ uint4 ld16_dev(__amdgpu_buffer_rsrc_t r, uint32_t byte_off) {
  const u32x4_t v = __builtin_amdgcn_raw_buffer_load_b128(r, (int)byte_off, 0, kSc1);
  return make_uint4(v.x, v.y, v.z, v.w);
}

// threadIdx.x through an opaque move: values derived from it are recomputed
// where they are used instead of being hoisted out of the layer loop and held
// (or spilled) for the whole launch
__device__ __forceinline__ int otid() {
  int t = threadIdx.x;
  asm volatile("" : "+v"(t));
  return t;
}

struct Sync {
  unsigned* w;
  int NW;
  unsigned epoch;
  unsigned limit;
  bool bad;  // thread 0: a wait ran out
};

// Grid barrier among the NW workgroups of the XCD (see the protocol above).
// Every thread has waited for its stores of the phase before (stores_done at
// the end of each phase); the loads a workgroup issues for the next phase
// stay in flight across the barrier.
__device__ __forceinline__ void grid_sync(Sync& s) {
  __syncthreads();
  if (threadIdx.x == 0) {
    ++s.epoch;
    const unsigned prev = l2_add(s.w + kArrive, 1u);
    if (prev + 1 == s.epoch * (unsigned)s.NW) {
      l2_store(s.w + kRelease, s.epoch);
    } else if (!s.bad) {
      unsigned spins = 0;
      while (dev_load(s.w + kRelease) < s.epoch) {
        __builtin_amdgcn_s_sleep(1);
        if (++spins > s.limit) {
          s.bad = true;
          break;
        }
      }
    }
  }
  __syncthreads();
}

// ------------------------------------------------------------- params ----
// The weights of every layer: one buffer per kind, layer l at l * stride
// elements (so a phase finds its weights by arithmetic, with no dependent
// load of a pointer). Weights are 16-column tiles [ceil(n / 16), k, 16].
enum : int { kAttnNorm, kQkv, kWo, kFfnNorm, kGateUp, kDown, kWeightKinds };
//   kAttnNorm [d]; kQkv [ceil(nqkv / 16), d, 16]; kWo [d / 16, d, 16];
//   kFfnNorm [d]; kGateUp [2 dff / 16, d, 16] (the gate tiles, then the up
//   tiles); kDown [d / 16, dff, 16]
struct StepWeights {
  const float* base[kWeightKinds];
  int64_t stride[kWeightKinds];
  __device__ __forceinline__ const float* at(int kind, int l) const {
    return base[kind] + (int64_t)l * stride[kind];
  }
};

struct StepParams {
  StepWeights w;
  int n_layers;
  const float* tok_emb;     // [vocab, d]
  const float* final_norm;  // [d]
  const float* lm_head;     // [ceil(vocab / 16), d, 16]
  void* kc;                 // [n_layers] x layer_stride cache elements
  void* vc;
  int64_t layer_stride;
  KvGeom geom;
  const int32_t* tokens;     // [16]: < 0 stands for prev_ids[-t - 1]
  const int32_t* positions;  // [16]
  const int32_t* slots;      // [16], -1: no cache write
  const int32_t* seq_lens;   // [n_seqs]
  const int32_t* bt;         // [n_seqs, bt_stride]
  int bt_stride, n_seqs;
  const int32_t* prev_ids;
  int n_prev;
  const float* cos_t;  // [max_pos, hd / 2]
  const float* sin_t;
  float* x;       // [16, d]
  float* q;       // [16, H hd]
  float* attn;    // [16, H hd]
  float* act;     // [16, dff]
  float* logits;  // [16, vocab]
  int32_t* ids;       // [16]
  int32_t* host_ids;  // [17] pinned host memory: ids, then the launch's status
  unsigned* sync;     // kSyncWords words, zero before the first launch
  int d, dff, H, Hkv, vocab;
  int bs_log2;  // log2 of the block size (block tables)
  float scale_log2, eps;
  unsigned spin_limit;
};

// -------------------------------------------------- projection tiles ----
// A workgroup computes NT 16 x 16 tiles of a projection at once (tile
// u + j NW, j < NT), each with NS slices (SwiGLU: the gate and up tiles).
// Its 8 wavefronts split K: wavefront w takes the steps of 4 k from step
// w spw, for every tile and slice, its weights in registers (0 past K and
// past N columns). Tiled element (k, m), k = 16 g + 4 j + s, sits at 256 g +
// 4 (16 j + m) + s, so a lane's operands of 4 steps are one float4.
__device__ __forceinline__ int steps_per_wave(int K) {
  return ((K / 4 + kTileWaves - 1) / kTileWaves + 3) / 4 * 4;
}

template <int KMAX, int NSL>
struct TileW {
  float v[NSL][KMAX / 32];
};

// Slice sl of wb: tile `tile` of w (+ off), or zeros when not valid.
template <int KMAX, int NSL>
__device__ __forceinline__ void load_slice(TileW<KMAX, NSL>& wb, int sl, const float* w,
                                           int64_t off, int tile, int K, int N, bool valid) {
  const int t_ = otid();
  const int lane = t_ & 63, tw = t_ >> 6;
  const int m = lane & 15;
  const int spw = steps_per_wave(K), kb = tw * spw * 4;
  const int nsteps = max(0, min(spw, K / 4 - tw * spw));
  const float colmask = valid && tile * kCols + m < N ? 1.f : 0.f;
  const float4* src =
      reinterpret_cast<const float4*>(w + off + (int64_t)(valid ? tile : 0) * K * kCols) + lane;
#pragma unroll
  for (int g = 0; g < KMAX / 128; ++g) {
    const float4 v = src[(int64_t)min(kb / 16 + g, K / 16 - 1) * 64];
    const float z = 4 * g < nsteps ? colmask : 0.f;
    wb.v[sl][4 * g] = v.x * z;
    wb.v[sl][4 * g + 1] = v.y * z;
    wb.v[sl][4 * g + 2] = v.z * z;
    wb.v[sl][4 * g + 3] = v.w * z;
  }
}

// The RMSNorm weights a lane applies (k = lane + 64 i).
template <int KMAX>
__device__ __forceinline__ void load_norm(float (&gw)[KMAX / 64], const float* w, int K) {
  const int lane = otid() & 63;
#pragma unroll
  for (int i = 0; i < KMAX / 64; ++i) gw[i] = w[min(lane + 64 * i, K - 1)];
}

// 16 rows of K floats to LDS (row pitch KP), zero past K, from an exchange
// buffer [16, K] (device-scope loads); every load of a thread is issued
// before the first LDS store.
template <int KMAX, int KP>
__device__ __forceinline__ void stage_rows(float* xs, const float* src, int K) {
  constexpr int kQ = KMAX / 4;  // float4 per row
  constexpr int kPer = (kRows * kQ + kThreads - 1) / kThreads;
  const int tid = otid();
  const __amdgpu_buffer_rsrc_t r = rsrc(src, (uint32_t)(kRows * K * 4));
  float4 v[kPer];
#pragma unroll
  for (int u = 0; u < kPer; ++u) {
    const int e = tid + u * kThreads;
    const int row = e / kQ, c4 = e - row * kQ;
    v[u] = make_float4(0.f, 0.f, 0.f, 0.f);
    if (row < kRows && 4 * c4 < K) {
      const uint4 w = ld16_dev(r, (uint32_t)(row * K + 4 * c4) * 4u);
      v[u] = make_float4(__uint_as_float(w.x), __uint_as_float(w.y), __uint_as_float(w.z),
                         __uint_as_float(w.w));
    }
  }
#pragma unroll
  for (int u = 0; u < kPer; ++u) {
    const int e = tid + u * kThreads;
    const int row = e / kQ, c4 = e - row * kQ;
    if (row < kRows) *reinterpret_cast<float4*>(&xs[row * KP + 4 * c4]) = v[u];
  }
}

// The embedding rows tok_emb[token] of the 16 tokens to LDS, as stage_rows
// (token t < 0 stands for prev[-t - 1], the id the previous step chose for
// its row -t - 1; ordinary loads: the table and ids are not written in this
// launch). With x_out, the rows are also written there: the residual stream
// starts as the embeddings.
template <int KMAX, int KP>
__device__ __forceinline__ void stage_embeddings(float* xs, const float* tok_emb, int K,
                                                 const int32_t* tokens, const int32_t* prev,
                                                 int n_prev, int vocab, float* x_out) {
  constexpr int kQ = KMAX / 4;
  constexpr int kPer = (kRows * kQ + kThreads - 1) / kThreads;
  const int tid = otid();
  float4 v[kPer];
#pragma unroll
  for (int u = 0; u < kPer; ++u) {
    const int e = tid + u * kThreads;
    const int row = e / kQ, c4 = e - row * kQ;
    v[u] = make_float4(0.f, 0.f, 0.f, 0.f);
    if (row < kRows && 4 * c4 < K) {
      int t = tokens[row];
      if (t < 0) t = prev[min(-t - 1, n_prev - 1)];
      t = min(max(t, 0), vocab - 1);
      v[u] = *reinterpret_cast<const float4*>(tok_emb + (int64_t)t * K + 4 * c4);
    }
  }
#pragma unroll
  for (int u = 0; u < kPer; ++u) {
    const int e = tid + u * kThreads;
    const int row = e / kQ, c4 = e - row * kQ;
    if (row < kRows) {
      *reinterpret_cast<float4*>(&xs[row * KP + 4 * c4]) = v[u];
      if (x_out && 4 * c4 < K)
        *reinterpret_cast<float4*>(x_out + (int64_t)row * K + 4 * c4) = v[u];
    }
  }
}

// RMSNorm of the 16 staged rows in place, wavefront w on rows w and w + 8:
// the sum of squares over k = lane + 64 i in increasing i, the wavefront sum,
// then (x / rms) * g, as rms_norm_kernel computes it.
template <int KMAX, int KP>
__device__ __forceinline__ void norm_rows(float* xs, const float (&gw)[KMAX / 64], int K,
                                          float eps) {
  const int t_ = otid();
  const int lane = t_ & 63, wave = t_ >> 6;
#pragma unroll
  for (int rr = 0; rr < kRows / kTileWaves; ++rr) {
    float* row = &xs[(wave + kTileWaves * rr) * KP + lane];
    float ss = 0.f;
#pragma unroll
    for (int i = 0; i < KMAX / 64; ++i) {
      const float a = row[64 * i];
      ss += a * a;
    }
    const float rms = sqrtf(wave_sum(ss) / (float)K + eps);
#pragma unroll
    for (int i = 0; i < KMAX / 64; ++i)
      if (lane + 64 * i < K) row[64 * i] = (row[64 * i] / rms) * gw[i];
  }
}

// The products of every slice, each summed over the 8 wavefronts in order:
// thread t < 256 NT gets row (t % 256) / 16, column t % 16 of slices j NS +
// s of tile j = t / 256 in out[s]. red holds [NSL][8][256] floats.
template <int KMAX, int NT, int NS, int KP>
__device__ __forceinline__ void tile_mma(const float* xs, const TileW<KMAX, NT * NS>& wb,
                                         float* red, int K, float (&out)[NS]) {
  constexpr int NSL = NT * NS;
  constexpr int kSteps = KMAX / 32;
  constexpr int kAcc = kSteps >= 4 ? 4 : 1;
  const int t_ = otid();
  const int lane = t_ & 63, tw = t_ >> 6;
  const int m = lane & 15, j = lane >> 4;
  const int kb = tw * steps_per_wave(K) * 4;
  f32x4_t acc4[NSL][kAcc];
#pragma unroll
  for (int s = 0; s < NSL; ++s)
#pragma unroll
    for (int q = 0; q < kAcc; ++q) acc4[s][q] = (f32x4_t){0.f, 0.f, 0.f, 0.f};
  // step i = 4 g + s meets k = kb + 16 g + 4 j + s (the tile order)
  const float* arow = &xs[m * KP + kb + 4 * j];
  float av[kSteps];
#pragma unroll
  for (int i = 0; i < kSteps; ++i) av[i] = arow[16 * (i / 4) + (i % 4)];
#pragma unroll
  for (int i = 0; i < kSteps; ++i)
#pragma unroll
    for (int s = 0; s < NSL; ++s)
      acc4[s][i % kAcc] =
          __builtin_amdgcn_mfma_f32_16x16x4f32(av[i], wb.v[s][i], acc4[s][i % kAcc], 0, 0, 0);
#pragma unroll
  for (int s = 0; s < NSL; ++s) {
    f32x4_t a = acc4[s][0];
#pragma unroll
    for (int q = 1; q < kAcc; ++q) a += acc4[s][q];
#pragma unroll
    for (int i = 0; i < 4; ++i) red[(s * kTileWaves + tw) * 256 + (4 * j + i) * kCols + m] = a[i];
  }
  __syncthreads();
  if (t_ < 256 * NT) {
    const int tj = t_ >> 8, e = t_ & 255;
#pragma unroll
    for (int s = 0; s < NS; ++s) {
      const float* r = red + (tj * NS + s) * kTileWaves * 256;
      float v = r[e];
#pragma unroll
      for (int w = 1; w < kTileWaves; ++w) v += r[w * 256 + e];
      out[s] = v;
    }
  }
}

// one element of slice sl summed over the wavefronts (the RoPE pair partner)
__device__ __forceinline__ float tile_total(const float* red, int sl, int e) {
  const float* r = red + sl * kTileWaves * 256;
  float v = r[e];
#pragma unroll
  for (int w = 1; w < kTileWaves; ++w) v += r[w * 256 + e];
  return v;
}

__device__ __forceinline__ float silu_times(float g, float u) {
#pragma clang fp contract(off)
  const float s = g / (1.0f + expf(-g));
  return s * u;
}

__device__ __forceinline__ void rotate_pair(float e, float o, float c, float s, float* oe,
                                            float* oo) {
#pragma clang fp contract(off)
  float ec = e * c, os = o * s, es = e * s, oc = o * c;
  *oe = ec - os;
  *oo = es + oc;
}

// ------------------------------------------------------------ attention ----
// A workgroup takes one sequence and NH of its KV heads: one decode item
// (decode_item.h, as the short-decode kernel runs it) per head, run by the
// same 8 wavefronts chunk by chunk, both heads' loads in flight together.
// The sequence's block table is staged once per launch (it is the same in
// every layer); the heads' first chunk of K/V is loaded before the barrier
// that precedes the attention phase (this step's key, written by the QKV
// phase, after it).

// The block table of sequence i (c keys) into tbl.
__device__ __forceinline__ void stage_table(int32_t* tbl, const StepParams& p, int i, int c) {
  if (i >= p.n_seqs || c <= 0 || c > kMaxCtx) return;
  const int nblk = (c + (1 << p.bs_log2) - 1) >> p.bs_log2;
  const int32_t* table = p.bt + (int64_t)i * p.bt_stride;
  for (int b = otid(); b < nblk; b += kThreads) tbl[b] = table[b];
}

// ---------------------------------------------------------------- kernel --
template <typename TKV, int KD, int KF, int D, int REP, int NH>
struct StepLds {
  static constexpr int KPD = KD + 4, KPF = KF + 4;  // staged row pitches
  struct Proj {
    float xs[kRows * KPF];
    float red[4][kTileWaves * 256];  // slices of the tiles of one pass
  };
  union {  // the projection phases' rows and partial tiles, or the attention items
    Proj pj;
    vl_item::Lds<TKV, D, REP> at[NH];
  };
  int32_t tbl[kMaxCtx];  // the sequence's block table, kept across phases
  int flag;
};

template <typename TKV, int KD, int KF, int D, int REP, int NH>
__global__ void __launch_bounds__(kThreads) decode_step_kernel(const StepParams p) {
  using L = StepLds<TKV, KD, KF, D, REP, NH>;
  namespace it = vl_item;
  constexpr int KPD = L::KPD, KPF = L::KPF;
  static_assert(it::kMaxCtx == kMaxCtx && kThreads == it::kThreads, "item layout");
  __shared__ L s;

  if (blockIdx.x % kXcds) return;  // workgroups of the other XCDs leave at once
  const int u = blockIdx.x / kXcds, NW = gridDim.x / kXcds;
  // a phase's thread coordinates (recomputed per phase from an opaque
  // thread index): lane, wavefront, and the (row, column) of the tile
  // element a thread finishes (tile t / 256 of the pass)
#define VL_IDS                                                    \
  const int tid = otid(), lane = tid & 63, wave = tid >> 6;       \
  const int ej = tid >> 8, er = (tid & 255) / kCols, ec = tid % kCols; \
  (void)lane, (void)wave, (void)ej, (void)er, (void)ec
  Sync sy{p.sync, NW, 0u, p.spin_limit, false};
  int status = 0;
  unsigned xcc = 0;
  if (threadIdx.x == 0) {
    asm volatile("s_getreg_b32 %0, hwreg(HW_REG_XCC_ID)" : "=s"(xcc));
    xcc &= 0xf;
    if (u == 0) l2_store(p.sync + kXcc, xcc + 1);  // read after the first barrier
  }

  const int d = p.d, dff = p.dff, H = p.H, Hkv = p.Hkv;
  const int qd = H * D, kd = Hkv * D, nqkv = qd + 2 * kd;
  const int n_qkv = cdiv(nqkv, kCols), n_d = d / kCols, n_ff = dff / kCols;
  const int n_lm = cdiv(p.vocab, kCols);
  const int bs_log2 = p.bs_log2;
  // attention: workgroup u takes sequence u / (Hkv / NH), KV heads from
  // NH (u % (Hkv / NH)); a pass covers NW such units
  const int hpu = Hkv / NH;  // units per sequence
  const int n_units = p.n_seqs * hpu;
  int c_first;  // the context of this workgroup's first unit
  {
    const int i = u / hpu;
    c_first = u < n_units ? p.seq_lens[i] : 0;
    stage_table(s.tbl, p, i, c_first);
  }

  for (int l = 0; l < p.n_layers; ++l) {
    TKV* kc = static_cast<TKV*>(p.kc) + (int64_t)l * p.layer_stride;
    TKV* vc = static_cast<TKV*>(p.vc) + (int64_t)l * p.layer_stride;
    // ------------------------------------------ A: RMSNorm, QKV, RoPE ----
    {
      VL_IDS;
      constexpr int NT = 2;
      const float* wq = p.w.at(kQkv, l);
      TileW<KD, NT> wb;
      float gw[KD / 64];
#pragma unroll
      for (int j = 0; j < NT; ++j) load_slice(wb, j, wq, 0, u + j * NW, d, nqkv, u + j * NW < n_qkv);
      load_norm<KD>(gw, p.w.at(kAttnNorm, l), d);
      if (l > 0) grid_sync(sy);
      for (int base = 0; base < n_qkv; base += NT * NW) {
        if (base > 0) {
#pragma unroll
          for (int j = 0; j < NT; ++j)
            load_slice(wb, j, wq, 0, base + u + j * NW, d, nqkv, base + u + j * NW < n_qkv);
        }
        const int tile = base + u + ej * NW;
        const bool valid = ej < NT && tile < n_qkv;
        // epilogue inputs of this thread's element
        const int col = tile * kCols + ec;
        int slot = -1;
        float cs = 0.f, sn = 0.f;
        if (valid && col < qd + kd) {
          const int bcol = col < qd ? col : col - qd;
          const int64_t tab = (int64_t)p.positions[er] * (D >> 1) + ((bcol % D) >> 1);
          cs = p.cos_t[tab];
          sn = p.sin_t[tab];
        }
        if (valid) slot = p.slots[er];
        if (base == 0) {
          if (l == 0)
            stage_embeddings<KD, KPD>(s.pj.xs, p.tok_emb, d, p.tokens, p.prev_ids, p.n_prev,
                                      p.vocab, u == 0 ? p.x : nullptr);
          else
            stage_rows<KD, KPD>(s.pj.xs, p.x, d);
          __syncthreads();
          norm_rows<KD, KPD>(s.pj.xs, gw, d, p.eps);
          __syncthreads();
        }
        float v[1];
        tile_mma<KD, NT, 1, KPD>(s.pj.xs, wb, &s.pj.red[0][0], d, v);
        if (valid && col < nqkv) {
          if (col < qd + kd) {
            const float partner = tile_total(&s.pj.red[0][0], ej, (tid & 255) ^ 1);
            const int bcol = col < qd ? col : col - qd;
            const bool odd = (bcol % D) & 1;
            float oe, oo;
            rotate_pair(odd ? partner : v[0], odd ? v[0] : partner, cs, sn, &oe, &oo);
            const float val = odd ? oo : oe;
            if (col < qd)
              p.q[(int64_t)er * qd + col] = val;
            else if (slot >= 0)
              Elem<TKV>::store(kc, p.geom.at(slot, bcol / D) + bcol % D, val);
          } else if (slot >= 0) {
            const int vcol = col - qd - kd;
            Elem<TKV>::store(vc, p.geom.at(slot, vcol / D) + vcol % D, v[0]);
          }
        }
        __syncthreads();
      }
      stores_done();
    }
    // ------------------------------------------------------ B: attention ----
    {
      VL_IDS;
      it::Src<TKV> src[NH];
      const __amdgpu_buffer_rsrc_t rk = it::cache_rsrc(kc, p.layer_stride * (int64_t)sizeof(TKV));
      const __amdgpu_buffer_rsrc_t rv = it::cache_rsrc(vc, p.layer_stride * (int64_t)sizeof(TKV));
#pragma unroll
      for (int h = 0; h < NH; ++h) {
        src[h].tbl = s.tbl;
        src[h].kc = kc;
        src[h].vc = vc;
        src[h].geom = p.geom;
        src[h].bs_log2 = bs_log2;
        src[h].rk = rk;
        src[h].rv = rv;
        src[h].g = (u % hpu) * NH + h;
        src[h].c = c_first;
      }
      bool act = u < n_units && c_first > 0 && c_first <= kMaxCtx;
      // the first chunk of the first unit's first head, but for this step's
      // key (the other heads' right after the barrier: registers)
      it::Regs<TKV, D, REP> r[NH];
      if (act) it::issue<true>(r[0], src[0], 0, wave, lane, c_first - 1, true);
      grid_sync(sy);
      if (l == 0 && threadIdx.x == 0 && dev_load(p.sync + kXcc) != xcc + 1) status = 2;
#pragma unroll
      for (int h = 1; h < NH; ++h)
        if (act) it::issue<true>(r[h], src[h], 0, wave, lane, c_first - 1, false);
      for (int base = 0; base < n_units; base += NW) {
        const int unit = base + u;
        const int i = unit / hpu;
        if (base > 0) {
          const int c = unit < n_units ? p.seq_lens[i] : 0;
#pragma unroll
          for (int h = 0; h < NH; ++h) src[h].c = c, src[h].g = (unit % hpu) * NH + h;
          act = unit < n_units && c > 0 && c <= kMaxCtx;
          __syncthreads();  // the previous unit is done with the table
          stage_table(s.tbl, p, i, c);
        }
        const int c = src[0].c;
        if (act) {
#pragma unroll
          for (int h = 0; h < NH; ++h)
            for (int e = tid; e < REP * D; e += kThreads) {
              const int hh = e / D, dd = e - (e / D) * D;
              s.at[h].q[hh][dd] =
                  dev_loadf(p.q + (int64_t)i * qd + (src[h].g * REP + hh) * D + dd) *
                  p.scale_log2;
            }
        }
        __syncthreads();
        it::State<it::Shape<TKV, D, REP>::VE, REP> st[NH];
#pragma unroll
        for (int h = 0; h < NH; ++h) st[h].init();
        if (act) {
          const int nchunk = (c + it::kChunk - 1) / it::kChunk;
          for (int t = 0; t < nchunk; ++t) {
#pragma unroll
            for (int h = 0; h < NH; ++h) {
              if (t == 0 && base == 0 && h == 0)
                it::load_fresh<true>(r[h], src[h], 0, wave, lane, c - 1);
              else if (!(t == 0 && base == 0))
                it::issue<true>(r[h], src[h], t, wave, lane, c - 1, false);
            }
#pragma unroll
            for (int h = 0; h < NH; ++h) it::compute(st[h], r[h], s.at[h], c, t, wave, lane);
          }
        }
#pragma unroll
        for (int h = 0; h < NH; ++h) {
          const int g = src[h].g;
          it::finish(st[h], s.at[h], act, tid, wave, lane, [&](int hh, int dd, float v) {
            p.attn[((int64_t)i * H + g * REP + hh) * D + dd] = v;
          });
        }
      }
      if (n_units > NW) {  // the next layer starts again with the first unit
        __syncthreads();
        stage_table(s.tbl, p, u / hpu, c_first);
      }
      stores_done();
    }
    // --------------------------------------------------- W: wo + residual ----
    {
      VL_IDS;
      const float* ww = p.w.at(kWo, l);
      TileW<KD, 1> wb;
      load_slice(wb, 0, ww, 0, u, d, d, u < n_d);
      // the residual element: x was last written two barriers ago
      float xres = 0.f;
      if (ej == 0 && u < n_d) xres = dev_loadf(p.x + (int64_t)er * d + u * kCols + ec);
      grid_sync(sy);
      for (int base = 0; base < n_d; base += NW) {
        const int tile = base + u;
        const bool valid = ej == 0 && tile < n_d;
        if (base > 0) {
          load_slice(wb, 0, ww, 0, tile, d, d, tile < n_d);
          if (valid) xres = dev_loadf(p.x + (int64_t)er * d + tile * kCols + ec);
        }
        if (base == 0) {
          stage_rows<KD, KPD>(s.pj.xs, p.attn, d);
          __syncthreads();
        }
        float v[1];
        tile_mma<KD, 1, 1, KPD>(s.pj.xs, wb, &s.pj.red[0][0], d, v);
        if (valid) p.x[(int64_t)er * d + tile * kCols + ec] = xres + v[0];
        __syncthreads();
      }
      stores_done();
    }
    // --------------------------------- C: RMSNorm, gate|up, SwiGLU ----
    {
      VL_IDS;
      constexpr int NT = 2;
      const float* wg = p.w.at(kGateUp, l);
      const int64_t up_off = (int64_t)n_ff * d * kCols;
      TileW<KD, 2 * NT> wb;
      float gw[KD / 64];
#pragma unroll
      for (int j = 0; j < NT; ++j) {
        const int t = u + j * NW;
        load_slice(wb, 2 * j, wg, 0, t, d, dff, t < n_ff);
        load_slice(wb, 2 * j + 1, wg, up_off, t, d, dff, t < n_ff);
      }
      load_norm<KD>(gw, p.w.at(kFfnNorm, l), d);
      grid_sync(sy);
      for (int base = 0; base < n_ff; base += NT * NW) {
        if (base > 0) {
#pragma unroll
          for (int j = 0; j < NT; ++j) {
            const int t = base + u + j * NW;
            load_slice(wb, 2 * j, wg, 0, t, d, dff, t < n_ff);
            load_slice(wb, 2 * j + 1, wg, up_off, t, d, dff, t < n_ff);
          }
        }
        const int tile = base + u + ej * NW;
        const bool valid = ej < NT && tile < n_ff;
        if (base == 0) {
          stage_rows<KD, KPD>(s.pj.xs, p.x, d);
          __syncthreads();
          norm_rows<KD, KPD>(s.pj.xs, gw, d, p.eps);
          __syncthreads();
        }
        float v[2];
        tile_mma<KD, NT, 2, KPD>(s.pj.xs, wb, &s.pj.red[0][0], d, v);
        if (valid) p.act[(int64_t)er * dff + tile * kCols + ec] = silu_times(v[0], v[1]);
        __syncthreads();
      }
      stores_done();
    }
    // ------------------------------------------- D: down + residual ----
    {
      VL_IDS;
      const float* wd = p.w.at(kDown, l);
      TileW<KF, 1> wb;
      load_slice(wb, 0, wd, 0, u, dff, d, u < n_d);
      // x was last written by the W phase, a barrier ago
      float xres = 0.f;
      if (ej == 0 && u < n_d) xres = dev_loadf(p.x + (int64_t)er * d + u * kCols + ec);
      grid_sync(sy);
      for (int base = 0; base < n_d; base += NW) {
        const int tile = base + u;
        const bool valid = ej == 0 && tile < n_d;
        if (base > 0) {
          load_slice(wb, 0, wd, 0, tile, dff, d, tile < n_d);
          if (valid) xres = dev_loadf(p.x + (int64_t)er * d + tile * kCols + ec);
        }
        if (base == 0) {
          stage_rows<KF, KPF>(s.pj.xs, p.act, dff);
          __syncthreads();
        }
        float v[1];
        tile_mma<KF, 1, 1, KPF>(s.pj.xs, wb, &s.pj.red[0][0], dff, v);
        if (valid) p.x[(int64_t)er * d + tile * kCols + ec] = xres + v[0];
        __syncthreads();
      }
      stores_done();
    }
  }
  // ------------------------------------ L: final RMSNorm, lm_head ----
  {
    VL_IDS;
    TileW<KD, 1> wb;
    float gw[KD / 64];
    load_slice(wb, 0, p.lm_head, 0, u, d, p.vocab, u < n_lm);
    load_norm<KD>(gw, p.final_norm, d);
    grid_sync(sy);
    const bool has_tile = u < n_lm;  // workgroup-uniform
    for (int base = 0; base < n_lm; base += NW) {
      const int tile = base + u;
      if (base > 0) load_slice(wb, 0, p.lm_head, 0, tile, d, p.vocab, tile < n_lm);
      if (base == 0) {
        stage_rows<KD, KPD>(s.pj.xs, p.x, d);
        __syncthreads();
        norm_rows<KD, KPD>(s.pj.xs, gw, d, p.eps);
        __syncthreads();
      }
      float v[1];
      tile_mma<KD, 1, 1, KPD>(s.pj.xs, wb, &s.pj.red[0][0], d, v);
      const int col = tile * kCols + ec;
      if (ej == 0 && tile < n_lm && col < p.vocab)
        p.logits[(int64_t)er * p.vocab + col] = v[0];
      __syncthreads();
    }
    // the last workgroup with lm_head tiles to finish takes every row's argmax
    stores_done();
    __syncthreads();
    if (tid == 0) {
      s.flag = 0;
      if (has_tile) {
        const unsigned n_wg = (unsigned)min(NW, n_lm);
        s.flag = l2_add(p.sync + kLmDone, 1u) + 1 == n_wg;
      }
    }
    __syncthreads();
    if (s.flag) {
      // wavefront w takes rows w and w + 8: numpy's rule, the lowest index of
      // the maximum, a NaN beating every number (its first index)
      constexpr int kNone = 0x7fffffff;
#pragma unroll
      for (int rr = 0; rr < kRows / kTileWaves; ++rr) {
        const int r = wave + kTileWaves * rr;
        const float* row = p.logits + (int64_t)r * p.vocab;
        float bv = -__builtin_inff();
        int bi = kNone, ni = kNone;
        for (int c = lane; c < p.vocab; c += 64) {
          const float e = dev_loadf(row + c);
          if (e > bv) bv = e, bi = c;
          if (e != e && ni == kNone) ni = c;
        }
#pragma unroll
        for (int o = 32; o > 0; o >>= 1) {
          const float ov = __shfl_xor(bv, o, 64);
          const int oi = __shfl_xor(bi, o, 64);
          if (ov > bv || (ov == bv && oi < bi)) bv = ov, bi = oi;
          ni = min(ni, __shfl_xor(ni, o, 64));
        }
        if (lane == 0) {
          const int id = ni != kNone ? ni : (bi == kNone ? 0 : bi);
          p.ids[r] = id;
          p.host_ids[r] = id;
        }
      }
    }
  }
  // ------------------------------------------------------------- exit ----
  stores_done();
  __syncthreads();
  if (threadIdx.x == 0) {
    if (sy.bad) status = 1;
    if (status) p.host_ids[kRows] = status;
    if (l2_add(p.sync + kExit, 1u) + 1 == (unsigned)NW) {  // everyone is past every barrier
      l2_store(p.sync + kArrive, 0u);
      l2_store(p.sync + kRelease, 0u);
      l2_store(p.sync + kLmDone, 0u);
      l2_store(p.sync + kXcc, 0u);
      l2_store(p.sync + kExit, 0u);
    }
  }
#undef VL_IDS
}

template <typename TKV, int KD, int KF, int D, int REP, int NH>
int launch(const StepParams& prm, int nw, hipStream_t st) {
  decode_step_kernel<TKV, KD, KF, D, REP, NH><<<nw * kXcds, kThreads, 0, st>>>(prm);
  VL_CHECK_LAUNCH();
  return VL_OK;
}

}  // namespace

extern "C" int vl_decode_step_supported(int d_model, int num_heads, int num_kv_heads, int d_ff,
                                        int kv_dtype, int max_context) {
  if (num_heads <= 0 || num_kv_heads <= 0 || num_heads % num_kv_heads || d_model <= 0 ||
      d_model % num_heads)
    return 0;
  const int hd = d_model / num_heads, rep = num_heads / num_kv_heads;
  const bool dt = kv_dtype == VL_DTYPE_F32 || kv_dtype == VL_DTYPE_BF16 ||
                  kv_dtype == VL_DTYPE_FP8_E4M3;
  return dt && rep == 2 && (hd == 48 || hd == 16) && d_model % 64 == 0 && d_model <= 384 &&
         d_ff % 16 == 0 && d_ff <= 1024 && max_context > 0 && max_context <= kMaxCtx;
}

extern "C" int vl_decode_step(const void* const* layer_weights, const int64_t* layer_strides,
                              int n_layers, const float* tok_emb,
                              const float* final_norm, const float* lm_head, void* key_cache,
                              void* value_cache, int64_t layer_stride, int kv_dtype,
                              int kv_layout, const int32_t* token_ids, const int32_t* positions,
                              const int32_t* slot_mapping, const int32_t* seq_lens,
                              const int32_t* block_tables, int block_table_stride, int num_seqs,
                              const int32_t* prev_ids, int num_prev, const float* cos_table,
                              const float* sin_table, int d_model, int num_heads,
                              int num_kv_heads, int d_ff, int vocab, int block_size,
                              int max_context, float scale, float eps, float* x, float* q,
                              float* attn, float* act, float* logits, int32_t* out_ids,
                              int32_t* out_ids_host, uint32_t* sync, void* stream) {
  VL_CHECK_ARG(vl_decode_step_supported(d_model, num_heads, num_kv_heads, d_ff, kv_dtype,
                                        max_context),
               "decode step: shape not supported (d_model %d, heads %d / %d, d_ff %d, kv "
               "dtype %d, context %d)",
               d_model, num_heads, num_kv_heads, d_ff, kv_dtype, max_context);
  VL_CHECK_ARG(n_layers > 0 && vocab > 0 && num_seqs >= 0 && num_seqs <= kRows &&
                   block_size > 0 && (block_size & (block_size - 1)) == 0 &&
                   block_table_stride >= (max_context + block_size - 1) / block_size &&
                   num_prev > 0,
               "decode step: bad layer count, vocab, sequence count (<= %d), block size, table "
               "stride or prev_ids length",
               kRows);
  VL_CHECK_ARG(layer_weights && layer_strides && tok_emb && final_norm && lm_head && key_cache && value_cache &&
                   token_ids && positions && slot_mapping && (seq_lens || !num_seqs) &&
                   (block_tables || !num_seqs) && prev_ids && cos_table && sin_table && x && q &&
                   attn && act && logits && out_ids && out_ids_host && sync,
               "decode step: null pointer");
  const int es = vl_cache_elem_bytes(kv_dtype);
  VL_CHECK_ARG(layer_stride > 0 && layer_stride * es <= 0x7fffffff,
               "decode step: a layer of the cache must be under 2 GiB");
  VL_CHECK_ARG((((uintptr_t)key_cache | (uintptr_t)value_cache | (uintptr_t)tok_emb |
                 (uintptr_t)lm_head | (uintptr_t)x | (uintptr_t)attn | (uintptr_t)act) & 15) == 0 &&
                   ((uintptr_t)sync & 127) == 0 && (layer_stride * es) % 16 == 0,
               "decode step: caches, embeddings, lm_head and row buffers 16-byte aligned, sync "
               "words 128-byte aligned");
  const int hd = d_model / num_heads;
  StepParams p{};
  for (int k = 0; k < kWeightKinds; ++k) {
    VL_CHECK_ARG(layer_weights[k] && (((uintptr_t)layer_weights[k]) & 15) == 0 &&
                     (k == kAttnNorm || k == kFfnNorm || layer_strides[k] % 4 == 0),
                 "decode step: weight buffer %d null or misaligned", k);
    p.w.base[k] = static_cast<const float*>(layer_weights[k]);
    p.w.stride[k] = layer_strides[k];
  }
  p.n_layers = n_layers;
  p.tok_emb = tok_emb;
  p.final_norm = final_norm;
  p.lm_head = lm_head;
  p.kc = key_cache;
  p.vc = value_cache;
  p.layer_stride = layer_stride;
  int rc = vl_kv_geom(kv_layout, block_size, num_kv_heads, hd, &p.geom);
  if (rc) return rc;
  p.tokens = token_ids;
  p.positions = positions;
  p.slots = slot_mapping;
  p.seq_lens = seq_lens;
  p.bt = block_tables;
  p.bt_stride = block_table_stride;
  p.n_seqs = num_seqs;
  p.prev_ids = prev_ids;
  p.n_prev = num_prev;
  p.cos_t = cos_table;
  p.sin_t = sin_table;
  p.x = x;
  p.q = q;
  p.attn = attn;
  p.act = act;
  p.logits = logits;
  p.ids = out_ids;
  p.host_ids = out_ids_host;
  p.sync = sync;
  p.d = d_model;
  p.dff = d_ff;
  p.H = num_heads;
  p.Hkv = num_kv_heads;
  p.vocab = vocab;
  p.bs_log2 = __builtin_ctz((unsigned)block_size);
  p.scale_log2 = scale * 1.4426950408889634f;
  p.eps = eps;
  p.spin_limit = 1u << 18;
  const int nw = vl_num_cus() / kXcds;
  VL_CHECK_ARG(nw >= 1, "decode step: fewer than 8 compute units");
  hipStream_t st = (hipStream_t)stream;
#define VL_STEP_LAUNCH(T, Dh)                                                     \
  if (hd == Dh)                                                                   \
    return num_kv_heads % 2 ? launch<T, 384, 1024, Dh, 2, 1>(p, nw, st)           \
                            : launch<T, 384, 1024, Dh, 2, 2>(p, nw, st);
  if (kv_dtype == VL_DTYPE_F32) {
    VL_STEP_LAUNCH(float, 48)
    VL_STEP_LAUNCH(float, 16)
  } else if (kv_dtype == VL_DTYPE_BF16) {
    VL_STEP_LAUNCH(uint16_t, 48)
    VL_STEP_LAUNCH(uint16_t, 16)
  } else {
    VL_STEP_LAUNCH(uint8_t, 48)
    VL_STEP_LAUNCH(uint8_t, 16)
  }
#undef VL_STEP_LAUNCH
  VL_CHECK_ARG(false, "decode step: no kernel for head_dim %d", hd);
}
