// K2 ragged paged attention: decode, chunked prefill and speculative verify in
// one call (vllmlite/attention.py:59-98 applied per sequence at
// vllmlite/model.py:107-112).
//
// A call is a plan followed by a run, both on the caller's stream and without
// host synchronisation:
//  plan     one workgroup reads seq_lens / query_start_loc and writes into the
//           workspace, per sequence, its work-item offsets, its number of
//           context partitions (multi-query) or ranges (decode), where split
//           partials go, and the order in which items are handed out
//           (longest first). Partitions start at 64 tokens and ranges at the
//           smallest power of two that gives a few items per resident
//           workgroup; both double until the split partials fit the
//           workspace, so any workspace >= the minimum is correct. The plan
//           depends only on the lengths, so one plan serves every layer of a
//           step.
//  run      single-query sequences of the bf16 / head_dim 128 / 4-query-heads-
//           per-KV-head / block-16 shape go to the bandwidth kernel (a
//           workgroup per (range, KV head) item, its 4 wavefronts splitting
//           the range's blocks), which merges its own split sequences;
//           multi-query sequences go to the MFMA tile kernels (16- or 32-row
//           wavefronts) when the head dim has an instantiation, else to the
//           generic kernel (one wavefront per (sequence, query, head,
//           partition)); a batch holding both kinds runs in the one step
//           kernel. Split sequences are merged (max-rescaled log-sum-exp)
//           by the last workgroup to finish a partition of them, in the
//           bandwidth, tile and step kernels, and by the combine kernel
//           after the generic one.
//
// Softmax runs in the base-2 domain: scores are pre-multiplied by
// scale * log2(e) and exponentiated with exp2, which is the same function.
#include <algorithm>
#include <mutex>
#include <type_traits>

#include "vl_common.h"

namespace {

constexpr int kHdrInts = 64;  // [0] bandwidth-kernel items [1] generic items [2] partition len
                              // [3] split rows [4] tile items [5] full ranges [6] tail ranges
                              // [7] range length [8] bandwidth-kernel work counter
                              // [9] bandwidth-kernel workgroups finished
                              // [10] 32-row tile items
                              // [12] split sequences for the combine kernel
                              // [11] 1: bandwidth-kernel decodes and tile items
                              // together (the step kernel runs them, the
                              // decode and tile kernels exit)
                              // [16..25] step kernel: work counters of the decode
                              // queue and the 8 tile queues, workgroups finished
                              // [26..33] 16-row tile kernel: work counters of its 8
                              // queues; [34..41] the same for the 32-row kernel
                              // (zeroed by the plan, then by the claim that
                              // returns each queue's last value)
constexpr int kPlanThreads = 256;
constexpr int kMaxHeadDim = 256;
constexpr int kSplitMaxQ = 16;  // only sequences with <= this many queries split their context
constexpr int kPart0 = 64;  // first partition length tried by the planner
constexpr float kLog2e = 1.4426950408889634f;

// bandwidth-kernel shape
constexpr int kFD = 128;   // head_dim
constexpr int kFRep = 4;   // query heads per KV head
constexpr int kFBs = 16;   // block size
constexpr int kFChunk = 16;  // blocks per softmax chunk (256 tokens)
constexpr int kBK = 4;  // blocks per K load burst (decode kernel)
constexpr int kBV = 2;  // blocks per V load burst (decode kernel)
// The step kernel's decode items: a deeper V burst. A CU there typically
// holds one decode and one tile workgroup, so a decode workgroup keeps more
// bytes in flight on its own (the tile body sets the register budget
// anyway). Mixed step: bursts (K 4, V 2) 569-573 us, (4, 4) 555-564, (8, 2)
// 577-588, (8, 4) 573-576.
constexpr int kStepBK = 4;  // blocks per K load burst (step kernel's decode items)
constexpr int kStepBV = 4;  // blocks per V load burst (step kernel's decode items)

// MFMA tile-kernel shape: 4 wavefronts x 16 (token, head) rows per workgroup,
// 64 keys per LDS tile
constexpr int kTileRows = 64;
constexpr int kTileKeys = 64;
// rows of a 32-row-wavefront (bf16, > 16 queries) item: 8 wavefronts share
// each staged K/V tile (the 4-wavefront step kernel takes an item in two
// passes)
constexpr int kWideRows = 256;
constexpr int kPvLook = 2;  // 32-row PV product: V^T operands read this many MFMAs ahead

struct Layout {
  int32_t* hdr;
  int32_t* gen_off;     // [S+1] generic wavefront items
  int32_t* tile_off;    // [S+1] 16-row MFMA tile items of every partition but the last
                        // (all P keys long), in sequence order
  int32_t* tail_seq;    // [S] sequences in the order their last partitions' 16-row
                        // items are handed out (after all of the above): longest first
  int32_t* tail_off;    // [S+1] those items, by position in tail_seq (right after
                        // tail_seq: the kernels find it at tail_seq + S)
  int32_t* nparts;      // [S]
  int32_t* split_base;  // [S] first partial row, or -1
  int32_t* wide_off;    // [S+1] 32-row MFMA tile workgroup items, by position in wide_seq
  int32_t* cmb_seq;     // [S] split sequences the combine kernel merges
  int32_t* wide_seq;    // [S] sequences in the order their 32-row items are handed
                        // out: longest context first, those without such items last
  int4* desc;           // [S + cap_rows] bandwidth-kernel ranges: (sequence, range,
                        // context length, query token); full ranges in sequence
                        // order, then the short last ranges, longest first
  float2* ml;           // [cap_rows] (running max (log2 domain), running sum)
  float* po;            // [cap_rows, D] unnormalised partial outputs
  int64_t cap_rows;
};

inline size_t plan_bytes(int S) {
  size_t b = kHdrInts * 4 + (size_t)(10 * S + 4) * 4;
  return (b + 255) & ~(size_t)255;
}

// Bytes of a workspace without partial rows: the plan, S range descriptors
// and alignment padding.
inline size_t fixed_bytes(int S) { return plan_bytes(S) + (size_t)S * 16 + 768; }

// Workspace bytes per partial row: its (max, sum), D floats and a range
// descriptor (a split sequence has at least as many rows as ranges).
inline size_t row_bytes(int D) { return (size_t)(D + 2) * 4 + 16; }

inline Layout make_layout(void* ws, size_t bytes, int S, int D) {
  Layout L;
  char* p = (char*)ws;
  L.hdr = (int32_t*)p;
  L.gen_off = L.hdr + kHdrInts;
  L.tile_off = L.gen_off + S + 1;
  L.nparts = L.tile_off + S + 1;
  L.split_base = L.nparts + S;
  L.wide_off = L.split_base + S;
  L.cmb_seq = L.wide_off + S + 1;
  L.wide_seq = L.cmb_seq + S;
  L.tail_seq = L.wide_seq + S;
  L.tail_off = L.tail_seq + S;
  const size_t pb = plan_bytes(S);
  // descriptors, 8-byte (m, l) pairs and a [rows, D] float array, each
  // 256-byte aligned
  const size_t fb = fixed_bytes(S);
  const int64_t rows = bytes > fb ? (int64_t)((bytes - fb) / row_bytes(D)) : 0;
  auto align = [](size_t x) { return (x + 255) & ~(size_t)255; };
  L.cap_rows = rows;
  L.desc = (int4*)(p + pb);
  const size_t ml_at = align(pb + (size_t)(S + rows) * 16);
  L.ml = (float2*)(p + ml_at);
  L.po = (float*)(p + align(ml_at + (size_t)rows * 8));
  return L;
}

inline bool fast_shape(int dtype, int H, int Hkv, int D, int bs) {
  return dtype == VL_DTYPE_BF16 && D == kFD && bs == kFBs && Hkv % 4 == 0 && H == kFRep * Hkv;
}

// head_dims with an MFMA tile instantiation
inline bool tile_shape(int dtype, int D, int bs) {
  if (bs <= 0 || (bs & (bs - 1)) != 0) return false;  // block math is shifts and masks
  if (dtype == VL_DTYPE_BF16) return D == 64 || D == 128;
  // fp32, and fp32 queries over bf16 / FP8 E4M3 caches (widened when staged)
  return D == 16 || D == 32 || D == 48 || D == 64 || D == 128;
}

__device__ __forceinline__ int upper_bound_le(const int32_t* a, int n, int x) {
  // largest i in [0, n) with a[i] <= x (a non-decreasing, a[0] <= x)
  int lo = 0, hi = n - 1;
  while (lo < hi) {
    const int mid = (lo + hi + 1) >> 1;
    if (a[mid] <= x) lo = mid; else hi = mid - 1;
  }
  return lo;
}

// The same search done by a whole wavefront: each round the 64 lanes probe
// 64 evenly spaced entries of the remaining range and a ballot picks the
// sub-range, so n <= 4097 takes 2 rounds of (independent) loads instead of
// log2(n) dependent ones. Every lane of the wavefront must call it; all get
// the result.
__device__ __forceinline__ int wave_upper_bound_le(const int32_t* a, int n, int x) {
  const int lane = threadIdx.x & 63;
  int lo = 0, len = n;
  while (len > 1) {
    const int step = (len + 63) >> 6;
    const int off = lane * step;
    const bool le = off < len && a[lo + off] <= x;
    const uint64_t m = __ballot(le);
    const int k = 63 - __builtin_clzll(m);  // lane 0 always passes: a[lo] <= x
    lo += k * step;
    len = min(step, len - k * step);
  }
  return lo;
}

// Exclusive scan of one int64 per thread across the workgroup; returns the
// thread's offset and writes the total to *total.
// x plus the 64-bit value DPP control kCtrl moves into this lane (0 where
// it moves none, or in rows outside kRowMask)
template <int kCtrl, int kRowMask>
__device__ __forceinline__ unsigned long long dpp_add64(unsigned long long x) {
  const int lo = __builtin_amdgcn_update_dpp(0, (int)(unsigned)x, kCtrl, kRowMask, 0xF, false);
  const int hi =
      __builtin_amdgcn_update_dpp(0, (int)(unsigned)(x >> 32), kCtrl, kRowMask, 0xF, false);
  return x + (((unsigned long long)(unsigned)hi << 32) | (unsigned)lo);
}

// Inclusive prefix sum over the 64 lanes of a wavefront by DPP: within each
// row of 16 lanes by shifts of 1, 2, 4 and 8, then row 0's total into row 1
// and row 2's into row 3 (row_bcast:15), then the first two rows' total into
// rows 2 and 3 (row_bcast:31). Lanes without a source add 0.
__device__ __forceinline__ int wave_incl_scan_dpp(int x) {
  x += __builtin_amdgcn_update_dpp(0, x, 0x111, 0xF, 0xF, false);  // row_shr:1
  x += __builtin_amdgcn_update_dpp(0, x, 0x112, 0xF, 0xF, false);  // row_shr:2
  x += __builtin_amdgcn_update_dpp(0, x, 0x114, 0xF, 0xF, false);  // row_shr:4
  x += __builtin_amdgcn_update_dpp(0, x, 0x118, 0xF, 0xF, false);  // row_shr:8
  x += __builtin_amdgcn_update_dpp(0, x, 0x142, 0xA, 0xF, false);  // row_bcast:15
  x += __builtin_amdgcn_update_dpp(0, x, 0x143, 0xC, 0xF, false);  // row_bcast:31
  return x;
}

// Exclusive prefix sums over the plan workgroup of N values per thread at
// once (v is replaced by its prefix; total gets the sums): a DPP scan within
// each wavefront, then every thread adds the totals of the wavefronts before
// its own from LDS. Two barriers for all N values. The counts are item, row
// and sequence counts, which the plan stores as int32.
template <int N>
__device__ void block_exclusive_scan(int (&v)[N], int (&total)[N]) {
  constexpr int kWaves = kPlanThreads / 64;
  __shared__ int wsum[kWaves][N];  // wavefront totals
  const int t = threadIdx.x, lane = t & 63, w = t >> 6;
  int incl[N];
#pragma unroll
  for (int k = 0; k < N; ++k) incl[k] = wave_incl_scan_dpp(v[k]);
  if (lane == 63)
#pragma unroll
    for (int k = 0; k < N; ++k) wsum[w][k] = incl[k];
  __syncthreads();
  // every thread adds the totals of the wavefronts before its own
#pragma unroll
  for (int k = 0; k < N; ++k) {
    int off = 0, tot = 0;
#pragma unroll
    for (int u = 0; u < kWaves; ++u) {
      const int s = wsum[u][k];
      off += u < w ? s : 0;
      tot += s;
    }
    v[k] = off + incl[k] - v[k];
    total[k] = tot;
  }
  __syncthreads();  // wsum may be reused
}

struct SeqWork {
  int np;        // context partitions
  int64_t full;  // bandwidth kernel: ranges of exactly R tokens
  int64_t tail;  // bandwidth kernel: 1 if the last range is shorter
  int64_t tile;  // MFMA tile workgroup items (16-row wavefronts)
  int64_t wide;  // MFMA tile workgroup items (32-row wavefronts)
  int64_t gen;   // generic wavefront items
  int64_t rows;  // split partial rows
};

// Routing: single-query sequences of the bandwidth shape go to the decode
// kernel, whose context is cut into ranges of R tokens (the last one
// shorter); everything else goes to the MFMA tile kernel when the shape has
// one (one workgroup per 64-row block of (token, head-in-group) rows per KV
// head and partition of P tokens; sequences with more than kSplitMaxQ
// queries take kWideRows-row blocks of 32-row wavefronts when `wide`), else to the
// generic kernel.
__device__ __forceinline__ bool is_bw(int q, int c, bool fast) { return fast && q == 1 && c > 0; }

__device__ __forceinline__ SeqWork seq_work(int q, int c, int P, int R, int H, int Hkv, bool fast,
                                            bool tile, bool wide) {
  SeqWork w;
  const bool live = q > 0 && c > 0;
  const bool bw = is_bw(q, c, fast);
  const bool tl = !bw && tile && live;
  if (bw) {
    w.np = (c + R - 1) / R;
    w.full = c / R;
    w.tail = (c % R) != 0;
  } else {
    w.np = (q > 0 && q <= kSplitMaxQ && c > P) ? (c + P - 1) / P : 1;
    w.full = w.tail = 0;
  }
  const bool wd = tl && wide && q > kSplitMaxQ;  // never split (np == 1)
  w.tile = tl && !wd ? (int64_t)w.np * Hkv * cdiv(q * (H / Hkv), kTileRows) : 0;
  w.wide = wd ? (int64_t)Hkv * cdiv(q * (H / Hkv), kWideRows) : 0;
  w.gen = (bw || tl) ? 0 : (int64_t)max(q, 0) * H * w.np;
  // a split decode sequence also keeps one arrival counter per KV head in
  // the rows after its partials, a split 16-row tile sequence one per (KV
  // head, row block)
  w.rows = w.np > 1 ? (int64_t)q * H * w.np + (bw ? Hkv : w.tile > 0 ? w.tile / w.np : 0) : 0;
  return w;
}

constexpr int kRangeMax = 2048;       // longest decode range the planner starts with
constexpr int kItemsPerWg = 4;  // decode items aimed for per resident workgroup
constexpr int kTileItemsPerWg = 4;  // split tile items aimed for per workgroup
constexpr int kTailBuckets = 1024;
constexpr int kPlanLdsSeqs = 2048;  // batches the plan keeps per-sequence counts of in LDS
constexpr int kPlanBuckets = kTailBuckets / kPlanThreads;  // buckets owned by each plan thread
constexpr int kPlanRegSeqs = 4;  // sequences a plan thread keeps in registers (S <= 1024)
static_assert(kTailBuckets % kPlanThreads == 0, "whole tail buckets per plan thread");

// Sums of N 64-bit values over the plan workgroup. red is this call's own LDS
// slot (a later call that reuses it must come after a barrier that follows
// every thread's reads here); every thread gets the totals.
template <int N>
__device__ __forceinline__ void plan_sum(unsigned long long (&v)[N],
                                         unsigned long long (*red)[N]) {
  const int lane = threadIdx.x & 63, w = threadIdx.x >> 6;
  // the wavefront's sum in lane 63 by DPP steps on the two 32-bit halves
  // (quad and row permutes, then row_bcast:15 and row_bcast:31)
#pragma unroll
  for (int k = 0; k < N; ++k) {
    unsigned long long x = v[k];
    x = dpp_add64<0xB1, 0xF>(x);   // quad_perm [1, 0, 3, 2]
    x = dpp_add64<0x4E, 0xF>(x);   // quad_perm [2, 3, 0, 1]
    x = dpp_add64<0x141, 0xF>(x);  // row_half_mirror
    x = dpp_add64<0x140, 0xF>(x);  // row_mirror
    x = dpp_add64<0x142, 0xA>(x);  // row_bcast:15
    x = dpp_add64<0x143, 0xC>(x);  // row_bcast:31
    v[k] = x;
  }
  if (lane == 63)
#pragma unroll
    for (int k = 0; k < N; ++k) red[w][k] = v[k];
  __syncthreads();
#pragma unroll
  for (int k = 0; k < N; ++k) {
    unsigned long long s = 0;
#pragma unroll
    for (int j = 0; j < kPlanThreads / 64; ++j) s += red[j][k];
    v[k] = s;
  }
}

// A thread's contiguous chunk [s0, s1) of the sequences, with the query
// counts and context lengths in registers when the chunk has at most
// kPlanRegSeqs of them (kCached), else read again from global memory.
template <bool kCached>
struct PlanChunk {
  int s0, s1;
  int q[kPlanRegSeqs], c[kPlanRegSeqs];
  __device__ __forceinline__ PlanChunk(const int32_t* __restrict__ qsl,
                                       const int32_t* __restrict__ seq_lens, int S) {
    const int chunk = (S + kPlanThreads - 1) / kPlanThreads;
    s0 = min(S, (int)threadIdx.x * chunk);
    s1 = min(S, s0 + chunk);
    if constexpr (kCached) {
#pragma unroll
      for (int j = 0; j < kPlanRegSeqs; ++j) {
        const bool in = s0 + j < s1;
        q[j] = in ? qsl[s0 + j + 1] - qsl[s0 + j] : 0;
        c[j] = in ? seq_lens[s0 + j] : 0;
      }
    }
  }
  // f(i, q, c) for every sequence of the chunk, in order
  template <typename F>
  __device__ __forceinline__ void each(const int32_t* __restrict__ qsl,
                                       const int32_t* __restrict__ seq_lens, F&& f) const {
    if constexpr (kCached) {
#pragma unroll
      for (int j = 0; j < kPlanRegSeqs; ++j)
        if (s0 + j < s1) f(s0 + j, q[j], c[j]);
    } else {
      for (int i = s0; i < s1; ++i) f(i, qsl[i + 1] - qsl[i], seq_lens[i]);
    }
  }
};

// Adds 1 to h[key] for every active lane, the lanes whose key is `hot` (the
// bucket most sequences share) with one atomic per wavefront: same-address
// LDS atomics run one after another. With want_pos, returns the old count
// plus the lane's rank among the wavefront's hot lanes (its slot).
template <bool want_pos>
__device__ __forceinline__ int bucket_add(int* h, int key, int hot) {
  const bool is_hot = key == hot;
  const uint64_t m = __ballot(is_hot);
  int pos = 0;
  if (is_hot) {
    const int leader = __ffsll((unsigned long long)m) - 1;
    const int lane = threadIdx.x & 63;
    int base = 0;
    if (lane == leader) base = atomicAdd(&h[hot], __popcll(m));
    if constexpr (want_pos) {
      base = __shfl(base, leader, 64);
      pos = base + __popcll(m & ((1ull << lane) - 1));
    }
  } else if constexpr (want_pos) {
    pos = atomicAdd(&h[key], 1);
  } else {
    atomicAdd(&h[key], 1);
  }
  return pos;
}

// One workgroup. Chooses the bandwidth kernel's range length R (the smallest
// power of two in 64..kRangeMax that leaves at most target_items (range, KV head)
// items, i.e. a few per resident workgroup: longer ranges mean fewer split
// partials to write and merge, shorter ones keep every CU busy) and the
// multi-query partition length P (the smallest power of two from kPart0 that
// leaves about tile_target items), doubling both until the split partials fit
// the workspace. Then writes per-sequence offsets and the order
// in which the shorter last ranges are handed out: longest first, after all
// full ranges, so the kernel ends on its smallest items. The sequences with
// 32-row tile items are ordered the same way, by context length, longest
// first (their row blocks are handed out last block first, so within a
// sequence too the items come longest first). Every thread owns a contiguous
// chunk of the sequences and kPlanBuckets consecutive buckets of each
// histogram; sums are wavefront reductions, not same-address atomics.
template <bool kCached>
__global__ void __launch_bounds__(kPlanThreads) plan_kernel(
    const int32_t* __restrict__ seq_lens, const int32_t* __restrict__ qsl, int S, int H, int Hkv,
    bool fast, bool tile, bool wide, int64_t cap_rows, int target_items, int tile_target,
    int32_t* __restrict__ hdr, int32_t* __restrict__ gen_off,
    int32_t* __restrict__ tile_off, int32_t* __restrict__ nparts,
    int32_t* __restrict__ split_base, int32_t* __restrict__ wide_off,
    int32_t* __restrict__ cmb_seq, int32_t* __restrict__ wide_seq,
    int32_t* __restrict__ tail_seq, int32_t* __restrict__ tail_off, int4* __restrict__ desc,
    float2* __restrict__ ml) {
  constexpr int kWaves = kPlanThreads / 64;
  __shared__ unsigned long long red0[kWaves][2], red1[2][kWaves][1];
  __shared__ int hist[kTailBuckets], whist[kTailBuckets], thist[kTailBuckets];
  // with at most kPlanLdsSeqs sequences, the item counts of the 32-row list
  // and of the second 16-row list by position, so that their offsets need no
  // global reads
  __shared__ int wcnt[kPlanLdsSeqs], tcnt[kPlanLdsSeqs];
  const int t = threadIdx.x;
  const PlanChunk<kCached> ch(qsl, seq_lens, S);
#pragma unroll
  for (int k = 0; k < kPlanBuckets; ++k)
    hist[t * kPlanBuckets + k] = 0, whist[t * kPlanBuckets + k] = 0, thist[t * kPlanBuckets + k] = 0;
  // 0. range length from the decode tokens and the target item count; the
  // same for the partition length of the splittable multi-query sequences
  // (at most kSplitMaxQ queries), counted in (KV head, 64-row block) units
  int R = 64, P = kPart0;
  bool lpt;  // the 16-row items in two lists, the last partitions longest first
  {
    const int rep = H / Hkv;
    unsigned long long v[2] = {0, 0};
    ch.each(qsl, seq_lens, [&](int, int q, int c) {
      if (is_bw(q, c, fast))
        v[0] += (unsigned long long)c;
      else if (tile && q > 0 && q <= kSplitMaxQ && c > 0)
        v[1] += (unsigned long long)c * cdiv(q * rep, kTileRows);
    });
    plan_sum(v, red0);  // its barrier also orders the histogram clearing
    while (R < kRangeMax && v[0] * (unsigned long long)Hkv >
                                (unsigned long long)max(target_items, 1) * (unsigned long long)R)
      R *= 2;
    while (P < (1 << 20) && v[1] * (unsigned long long)Hkv >
                                (unsigned long long)max(tile_target, 1) * (unsigned long long)P)
      P *= 2;
    lpt = wide && v[1] > 0;  // bf16 16-row items (short queries over split contexts)
  }
  // 1. double P and R until the split partials fit (every thread holds the
  // same sums, so all take the same branch)
  for (int it = 0;; ++it) {
    unsigned long long need[1] = {0};
    ch.each(qsl, seq_lens, [&](int, int q, int c) {
      need[0] += seq_work(q, c, P, R, H, Hkv, fast, tile, wide).rows;
    });
    plan_sum(need, red1[it & 1]);
    if (need[0] <= (unsigned long long)cap_rows || (P >= (1 << 29) && R >= (1 << 29))) break;
    P = min(P * 2, 1 << 29), R = min(R * 2, 1 << 29);
  }
  // 2. offsets
  // tail ranges are bucketed by their length in blocks, longest first
  const int rblocks = R / kFBs;
  auto tail_key = [&](int c) {
    const int blocks = ((c % R) + kFBs - 1) / kFBs;  // 1 .. rblocks
    const int k = rblocks <= kTailBuckets ? blocks - 1
                                          : (int)((int64_t)(blocks - 1) * kTailBuckets / rblocks);
    return kTailBuckets - 1 - k;  // ascending key = descending length
  };
  // sequences with 32-row items by their context in 64-key tiles (up to
  // kTailBuckets - 2 distinct lengths), descending; the others in the last bucket
  auto wide_key = [&](int c, bool wd) {
    return wd ? kTailBuckets - 2 - min(kTailBuckets - 2, cdiv(c, kTileKeys) - 1) : kTailBuckets - 1;
  };
  // 16-row tile items come from two lists. bf16 items over split contexts
  // (lpt: HBM-bound, partitions of up to P keys): the first holds those of
  // every partition but a sequence's last (each P keys long), in sequence
  // order; the second the last partitions' items, sequences ordered by that
  // partition's length in 64-key tiles, descending (sequences without such
  // items in the last bucket), so that a launch ends on its shortest items.
  // Otherwise (fp32 items: short contexts, tiny items) the first list holds
  // them all, in sequence order.
  auto split_items = [&](const SeqWork& w) -> int64_t {
    return !lpt ? w.tile : w.tile > 0 ? w.tile / w.np * (w.np - 1) : 0;
  };
  auto last_key = [&](int c, const SeqWork& w) {
    if (w.tile == 0 || !lpt) return kTailBuckets - 1;
    const int64_t last = (int64_t)c - (int64_t)(w.np - 1) * P;  // 1 .. P keys (all of c unsplit)
    return kTailBuckets - 2 - (int)min<int64_t>(kTailBuckets - 2, cdiv64(last, kTileKeys) - 1);
  };
  int64_t f = 0, g = 0, r = 0, x = 0, xs = 0, tl = 0, wd = 0, cm = 0;
  ch.each(qsl, seq_lens, [&](int, int q, int c) {
    const SeqWork w = seq_work(q, c, P, R, H, Hkv, fast, tile, wide);
    f += w.full, g += w.gen, r += w.rows, x += w.tile, tl += w.tail, wd += w.wide;
    xs += split_items(w);
    cm += w.np > 1 && w.gen > 0;  // the combine kernel merges only the generic kernel's splits
    if (w.tail) {  // contexts are often alike: the wavefront's first key aggregated
      const int key = tail_key(c);
      bucket_add<false>(hist, key, __builtin_amdgcn_readfirstlane(key));
    }
    bucket_add<false>(whist, wide_key(c, w.wide > 0), kTailBuckets - 1);
    if (lpt) bucket_add<false>(thist, last_key(c, w), kTailBuckets - 1);
  });
  __syncthreads();
  // the thread's buckets: their counts, summed, join the same scan as the
  // per-sequence counts; the starts within the thread's buckets follow
  int hb[kPlanBuckets], wb[kPlanBuckets], lb[kPlanBuckets], hsum = 0, wsum = 0, lsum = 0;
#pragma unroll
  for (int k = 0; k < kPlanBuckets; ++k) {
    hb[k] = hsum, wb[k] = wsum, lb[k] = lsum;
    hsum += hist[t * kPlanBuckets + k], wsum += whist[t * kPlanBuckets + k];
    lsum += thist[t * kPlanBuckets + k];
  }
  int sc[11] = {(int)f,  (int)g,    (int)r, (int)xs,  (int)tl, (int)wd,
                (int)cm, hsum,      wsum,   (int)x,   lsum},
      tot[11];
  block_exclusive_scan(sc, tot);
  int64_t fo = sc[0], go = sc[1], ro = sc[2], xo = sc[3], co = sc[6];
  const int64_t tf = tot[0], tg = tot[1], tr = tot[2], txs = tot[3], ttl = tot[4], twd = tot[5],
                tcm = tot[6], tx = tot[9];
  // bucket starts (block_exclusive_scan ends on a barrier: the counts above
  // have been read by every thread)
#pragma unroll
  for (int k = 0; k < kPlanBuckets; ++k) {
    hist[t * kPlanBuckets + k] = sc[7] + hb[k], whist[t * kPlanBuckets + k] = sc[8] + wb[k];
    thist[t * kPlanBuckets + k] = sc[10] + lb[k];
  }
  __syncthreads();
  ch.each(qsl, seq_lens, [&](int i, int q, int c) {
    const SeqWork w = seq_work(q, c, P, R, H, Hkv, fast, tile, wide);
    const int qs = qsl[i];
    for (int k = 0; k < w.full; ++k) desc[fo + k] = make_int4(i, k, c, qs);
    gen_off[i] = (int32_t)go;
    tile_off[i] = (int32_t)xo;
    {
      const int p = bucket_add<true>(whist, wide_key(c, w.wide > 0), kTailBuckets - 1);
      wide_seq[p] = i;
      if (S <= kPlanLdsSeqs) wcnt[p] = (int)w.wide;
    }
    if (lpt) {
      const int p = bucket_add<true>(thist, last_key(c, w), kTailBuckets - 1);
      tail_seq[p] = i;
      if (S <= kPlanLdsSeqs) tcnt[p] = (int)(w.tile - split_items(w));
    }
    nparts[i] = w.np;
    split_base[i] = w.np > 1 ? (int32_t)ro : -1;
    if (w.tail) {
      const int key = tail_key(c);
      desc[tf + bucket_add<true>(hist, key, __builtin_amdgcn_readfirstlane(key))] =
          make_int4(i, c / R, c, qs);
    }
    if (w.np > 1 && w.gen > 0) cmb_seq[co++] = i;
    if (w.np > 1 && w.gen == 0)  // arrival counters start at 0
      for (int64_t k = (int64_t)q * H * w.np; k < w.rows; ++k)
        reinterpret_cast<int32_t*>(ml + ro + k)[0] = 0;
    fo += w.full, go += w.gen, ro += w.rows, xo += split_items(w);
  });
  // 32-row item offsets in wide_seq order and the second 16-row list's in
  // tail_seq order (every thread reads the positions of its chunk, written
  // above by any thread of the workgroup)
  __syncthreads();
  {
    const bool do_w = twd > 0, do_t = lpt && tx > 0;  // the same in every thread
    auto wide_items = [&](int p) -> int64_t {
      if (S <= kPlanLdsSeqs) return wcnt[p];
      const int i = wide_seq[p];
      return seq_work(qsl[i + 1] - qsl[i], seq_lens[i], P, R, H, Hkv, fast, tile, wide).wide;
    };
    auto last_items = [&](int p) -> int64_t {
      if (S <= kPlanLdsSeqs) return tcnt[p];
      const int i = tail_seq[p];
      const SeqWork w = seq_work(qsl[i + 1] - qsl[i], seq_lens[i], P, R, H, Hkv, fast, tile, wide);
      return w.tile - split_items(w);
    };
    int64_t mw = 0, mt = 0;
    for (int p = ch.s0; p < ch.s1; ++p) {
      if (do_w) mw += wide_items(p);
      if (do_t) mt += last_items(p);
    }
    int v2[2] = {(int)mw, (int)mt}, tot2[2];
    if (do_w || do_t) block_exclusive_scan(v2, tot2);
    int64_t a = v2[0], b = v2[1];
    for (int p = ch.s0; p < ch.s1; ++p) {
      wide_off[p] = do_w ? (int32_t)a : 0;
      tail_off[p] = do_t ? (int32_t)b : 0;
      if (do_w) a += wide_items(p);
      if (do_t) b += last_items(p);
    }
  }
  if (t == 0) {
    gen_off[S] = (int32_t)tg;
    tile_off[S] = (int32_t)txs;
    tail_off[S] = (int32_t)(tx - txs);
    wide_off[S] = (int32_t)twd;
    hdr[0] = (int32_t)((tf + ttl) * Hkv);
    hdr[1] = (int32_t)tg;
    hdr[2] = P;
    hdr[3] = (int32_t)tr;
    hdr[4] = (int32_t)tx;
    hdr[5] = (int32_t)tf;
    hdr[6] = (int32_t)ttl;
    hdr[7] = R;
    hdr[8] = 0;
    hdr[9] = 0;
    hdr[10] = (int32_t)twd;
    hdr[11] = (tf + ttl) > 0 && (tx + twd) > 0;
    hdr[12] = (int32_t)tcm;
    for (int k = 16; k < 42; ++k) hdr[k] = 0;
  }
}

// ------------------------------------------------------------ generic -----

template <typename T, typename TKV>
__global__ void __launch_bounds__(64) attend_generic_kernel(
    T* __restrict__ out, const T* __restrict__ query, int64_t q_stride, const TKV* __restrict__ kc,
    const TKV* __restrict__ vc, const int32_t* __restrict__ bt, int bt_stride,
    const int32_t* __restrict__ seq_lens, const int32_t* __restrict__ qsl, int S, int H, int Hkv,
    int D, int bs, int kv_hm, float scale_log2, const int32_t* __restrict__ hdr,
    const int32_t* __restrict__ item_off, const int32_t* __restrict__ nparts,
    const int32_t* __restrict__ split_base, float2* __restrict__ ml, float* __restrict__ po) {
  __shared__ float q_s[kMaxHeadDim];
  __shared__ float p_s[64];
  __shared__ int64_t row_s[64];
  const int lane = threadIdx.x;
  const int n_items = hdr[1];
  const int P = hdr[2];
  const int rep = H / Hkv;
  // row of (block b, offset o, KV head h): b * blk + o * row + h * head, for
  // token-major [slots, Hkv, D] or head-major [blocks, Hkv, bs, D] caches
  const int64_t blk = (int64_t)bs * Hkv * D;
  const int64_t row_stride = kv_hm ? D : (int64_t)Hkv * D;
  const int64_t head_stride = kv_hm ? (int64_t)bs * D : D;
  constexpr int kR = kMaxHeadDim / 64;
  for (int it = blockIdx.x; it < n_items; it += gridDim.x) {
    const int i = wave_upper_bound_le(item_off, S + 1, it);
    const int q_len = qsl[i + 1] - qsl[i];
    const int ctx = seq_lens[i];
    const int np = nparts[i];
    const int local = it - item_off[i];
    const int part = local % np;
    const int unit = local / np;
    const int j = unit / H, h = unit - (unit / H) * H;
    const int kvh = h / rep;
    const int tok = qsl[i] + j;
    const int qpos = ctx - q_len + j;
    int kbeg = 0, kend = min(qpos + 1, ctx);
    if (np > 1) {
      kbeg = part * P;
      kend = min(kend, kbeg + P);
    }
    const T* qrow = query + (int64_t)tok * q_stride + (int64_t)h * D;
    for (int d = lane; d < D; d += 64) q_s[d] = Elem<T>::load(qrow, d);
    __syncthreads();
    const int32_t* table = bt + (int64_t)i * bt_stride;
    float m = -__builtin_inff(), l = 0.f;
    float acc[kR];
#pragma unroll
    for (int r = 0; r < kR; ++r) acc[r] = 0.f;
    for (int k0 = kbeg; k0 < kend; k0 += 64) {
      const int key = k0 + lane;
      float s = -__builtin_inff();
      int64_t row = 0;
      if (key < kend) {
        row = (int64_t)table[key / bs] * blk + (int64_t)(key % bs) * row_stride +
              (int64_t)kvh * head_stride;
        const TKV* kr = kc + row;
        float dot = 0.f;
        for (int d = 0; d < D; ++d) dot += q_s[d] * Elem<TKV>::load(kr, d);
        s = dot * scale_log2;
      }
      const float cmax = wave_max(s);
      const float m_new = fmaxf(m, cmax);
      const float alpha = (m == -__builtin_inff()) ? 0.f : exp2f(m - m_new);
      const float p = (key < kend) ? exp2f(s - m_new) : 0.f;
      l = l * alpha + wave_sum(p);
      p_s[lane] = p;
      row_s[lane] = row;
      __syncthreads();
      const int nk = min(64, kend - k0);
#pragma unroll
      for (int r = 0; r < kR; ++r) acc[r] *= alpha;
      for (int jj = 0; jj < nk; ++jj) {
        const float pj = p_s[jj];
        const TKV* vr = vc + row_s[jj];
#pragma unroll
        for (int r = 0; r < kR; ++r) {
          const int d = lane + 64 * r;
          if (d < D) acc[r] += pj * Elem<TKV>::load(vr, d);
        }
      }
      __syncthreads();
      m = m_new;
    }
    if (np == 1) {
      const float inv = l > 0.f ? 1.f / l : 0.f;
      T* orow = out + ((int64_t)tok * H + h) * D;
#pragma unroll
      for (int r = 0; r < kR; ++r) {
        const int d = lane + 64 * r;
        if (d < D) Elem<T>::store(orow, d, acc[r] * inv);
      }
    } else {
      const int64_t prow = (int64_t)split_base[i] + (int64_t)unit * np + part;
#pragma unroll
      for (int r = 0; r < kR; ++r) {
        const int d = lane + 64 * r;
        if (d < D) po[prow * D + d] = acc[r];
      }
      if (lane == 0) ml[prow] = make_float2(m, l);
    }
    __syncthreads();
  }
}


// ----------------------------------------------------------- MFMA tiles ----
//
// Multi-query attention (chunked prefill, speculative verify) on the matrix
// cores. One workgroup item = (sequence, KV head, block of 64 rows, context
// partition); a row is a (query token j, head r of the KV head's group) pair,
// row = j * rep + r, so the query heads of a GQA group share every K/V tile.
// Wavefront w owns rows 16w..16w+15 of the block.
//
// Keys stream in tiles of 64 through one LDS buffer (K row-major, V
// transposed): while a tile is computed, the next one's K/V are already in
// flight into registers (each thread gathers its keys through the block
// table), and are written to LDS between two barriers once every wavefront
// is done with the current tile.
//   S^T[64 keys x 16 rows] = K . Q^T   four 16x16 output tiles; lane l holds
//                                      row l%16 and keys 16t + 4(l/16) + i
//   online softmax per row (a row's 64 keys of a tile sit in the 4 lanes
//   l%16 + 16g, so a row max is a register max plus two xor shuffles)
//   O^T[D x 16 rows] += V^T . P^T      the probabilities are already in the
//                                      B-operand registers: for keys 32h..,
//                                      k-slot e of lane group g is key
//                                      32h + 4g + e (e < 4) or 32h + 16 + 4g
//                                      + e - 4, and V^T is read in that order.
// bf16 uses v_mfma_f32_16x16x32_bf16 (P rounded to bf16, fp32 accumulation);
// fp32 uses v_mfma_f32_16x16x4f32, so fp32 inputs keep fp32 products.

typedef __bf16 bf16x8_t __attribute__((ext_vector_type(8)));
typedef __bf16 bf16x2_t __attribute__((ext_vector_type(2)));
typedef float f32x4_t __attribute__((ext_vector_type(4)));
typedef uint32_t u32x4_t __attribute__((ext_vector_type(4)));

// 16-byte global load as a native vector (a uint4 struct copy can become an
// aggregate memcpy that keeps a register array in scratch memory)
__device__ __forceinline__ uint4 load16(const void* p) {
  return __builtin_bit_cast(uint4, *reinterpret_cast<const u32x4_t*>(p));
}

// 4 consecutive cache elements as the bits of 4 fp32 values: fp32 as they
// are, bf16 and FP8 E4M3 widened (exactly) for the fp32 tile path
__device__ __forceinline__ uint4 load4_as_f32(const float* p) { return load16(p); }
__device__ __forceinline__ uint4 load4_as_f32(const uint16_t* p) {
  const uint2 w = *reinterpret_cast<const uint2*>(p);
  return make_uint4(w.x << 16, w.x & 0xffff0000u, w.y << 16, w.y & 0xffff0000u);
}
__device__ __forceinline__ uint4 load4_as_f32(const uint8_t* p) {
  float r[4];
  e4m3x4_to_f32(*reinterpret_cast<const uint32_t*>(p), r);
  return make_uint4(__float_as_uint(r[0]), __float_as_uint(r[1]), __float_as_uint(r[2]),
                    __float_as_uint(r[3]));
}

// The same for the K / V bytes of a tile item: a non-temporal (streaming)
// load when no other item reads them (a sequence whose rows fit one item:
// spec-verify and short chunks; measured 950 -> 870 us on the 64 x 5 verify
// batch), an ordinary one when the sequence's other row blocks re-read them
// from the cache (long prefill chunks: streaming loads there measured 281 ->
// 298 us)
// kStream: a non-temporal load (data read once). A compile-time choice: a
// runtime one puts every load in a branch of its own, and the compiler then
// cannot issue a tile's loads (and the block-id loads they need) together.
template <bool kStream>
__device__ __forceinline__ uint4 load16_kv(const void* p) {
  if constexpr (kStream)
    return __builtin_bit_cast(uint4, __builtin_nontemporal_load(reinterpret_cast<const u32x4_t*>(p)));
  return load16(p);
}

// One K/V tile in LDS. RW (rows per wavefront) sets the V^T row stride: the
// PV operand reads of a wavefront (rows l % RW, 8-byte reads) then spread
// over all 64 banks.
template <typename T, int D, int RW>
struct TileLds;
// (16-byte aligned: the K rows are read 16 bytes at a time)
template <int D, int RW>
struct alignas(16) TileLds<uint16_t, D, RW> {
  static constexpr int kRow = D + 8;  // K row stride (bf16), 16-byte aligned
  // V rows as in the cache (key-major), read transposed by ds_read_b64_tr_b16:
  // a PV operand read takes 8 bytes of each of 4 (RW 16: 8) keys per 16 dims,
  // so the row stride in dwords is 16 (RW 16: 8) modulo the 64 banks
  static constexpr int vRow = 2 * ((D / 2 + 63 - (RW == 32 ? 16 : 8)) / 64 * 64 + (RW == 32 ? 16 : 8));
  static constexpr int kChunks = D / 8;  // 16-byte chunks per head row
  // prefetch units per thread (K and V alike): (key, chunk)
  static constexpr int kUnits = kTileKeys * kChunks / 256;
  uint16_t k[kTileKeys * kRow];
  uint16_t v[kTileKeys * vRow];
  int last;  // the item's workgroup arrived last among its row block's partitions
};

// 4 bf16 of a PV operand from LDS by the transposing read: lane i of each
// 16-lane group passes the address of 4 consecutive dims (4 (i % 4) ..) of key
// i / 4 of a 4-key x 16-dim block and receives dim i of the 4 keys.
__device__ __forceinline__ uint2 lds_read_tr16(const uint16_t* p) {
  typedef short s16x4_t __attribute__((ext_vector_type(4)));
  typedef __attribute__((address_space(3))) s16x4_t lds_s16x4_t;
  const s16x4_t r = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_s16x4_t*)p);
  return __builtin_bit_cast(uint2, r);
}
template <int D, int RW>
struct alignas(16) TileLds<float, D, RW> {
  static constexpr int kRow = D + 1;
  static constexpr int vRow = D + 1;
  static constexpr int kChunks = D / 4;        // float4 chunks per head row
  static constexpr int kUnits = (kTileKeys * kChunks + 255) / 256;
  static constexpr int vUnits = 0;             // V goes with K (same key, chunk)
  float k[kTileKeys * kRow];
  float v[kTileKeys * vRow];
  int last;  // the item's workgroup arrived last among its row block's partitions
};

__device__ __forceinline__ uint32_t pack_bf16x2(float lo, float hi) {
  return (uint32_t)f32_to_bf16(lo) | ((uint32_t)f32_to_bf16(hi) << 16);
}



// Two floats to packed bf16 with the hardware conversion (v_cvt_pk_bf16_f32,
// round to nearest even, as f32_to_bf16 for every finite value).
__device__ __forceinline__ uint32_t cvt_pk_bf16(float lo, float hi) {
  const bf16x2_t v = {(__bf16)lo, (__bf16)hi};
  return __builtin_bit_cast(uint32_t, v);
}

// threadIdx.x, with kOpaque through an opaque move: values an item derives
// from it are then recomputed per item instead of being hoisted out of a
// persistent kernel's item loop, where they would stay live across the other
// item kinds.
template <bool kOpaque>
__device__ __forceinline__ int item_tid() {
  int t = threadIdx.x;
  if constexpr (kOpaque) asm volatile("" : "+v"(t));
  return t;
}

// Kernel parameters shared by the tile and decode items: the batch, the
// plan's per-sequence arrays and the decode items' range descriptors. They stay plain restrict-qualified kernel parameters so that the
// compiler reads the plan's arrays with scalar loads. K/V are not restrict:
// restrict-qualified loads are treated as invariant and may be scheduled past
// the compiler barriers that batch them.
#define VL_ATTN_PARAMS(T) VL_ATTN_PARAMS_KV(T, T)
// (TKV: the cache elements, when they differ from the query's: fp32 queries
// over bf16 or FP8 E4M3 caches)
#define VL_ATTN_PARAMS_KV(T, TKV)                                                            \
  T *__restrict__ out, const T *__restrict__ query, int64_t q_stride, const TKV *kc,        \
      const TKV *vc, const int32_t *__restrict__ bt, int bt_stride,                         \
      const int32_t *__restrict__ seq_lens, const int32_t *__restrict__ qsl, int S, int H,   \
      int Hkv, int bs_log2, int kv_hm, float scale_log2, const int4 *__restrict__ desc,      \
      const int32_t *__restrict__ nparts,                                                    \
      const int32_t *__restrict__ split_base, float2 *ml, float *po
#define VL_ATTN_ARGS \
  out, query, q_stride, kc, vc, bt, bt_stride, seq_lens, qsl, S, H, Hkv, bs_log2, kv_hm,      \
      scale_log2, desc, nparts, split_base, ml, po


// Two floats as one 64-bit word (for 8-byte device-scope stores and loads).
__device__ __forceinline__ uint64_t pack2(float lo, float hi) {
  return (uint64_t)__float_as_uint(lo) | ((uint64_t)__float_as_uint(hi) << 32);
}
__device__ __forceinline__ float lo_f(uint64_t w) { return __uint_as_float((uint32_t)w); }
__device__ __forceinline__ float hi_f(uint64_t w) { return __uint_as_float((uint32_t)(w >> 32)); }

// One output row's merge of np partitions written by other workgroups
// (device-scope loads): lane p holds partition p's (max, sum) and weight, 64
// partitions at a time; every lane sums its two dims over the partitions with
// the weights read lane by lane, four partitions' loads in flight (relaxed
// atomic loads are not batched by the compiler unless written out).
// xrow: the lane's dims of partition 0; xstride: 8-byte words between
// partitions. Returns the normalised pair.
__device__ __forceinline__ float2 merge_partitions(const uint64_t* mlw, const uint64_t* xrow,
                                                   int64_t xstride, int np, int lane) {
  auto ld = [](const uint64_t* a) {
    return __hip_atomic_load(a, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  };
  float M = -__builtin_inff();
  for (int p = lane; p < np; p += 64) M = fmaxf(M, lo_f(ld(mlw + p)));
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) M = fmaxf(M, __shfl_xor(M, o, 64));
  float L = 0.f, a0 = 0.f, a1 = 0.f;
  for (int p0 = 0; p0 < np; p0 += 64) {
    float wgt = 0.f;
    if (p0 + lane < np) {
      const uint64_t v = ld(mlw + p0 + lane);
      wgt = lo_f(v) == -__builtin_inff() ? 0.f : exp2_fast(lo_f(v) - M);
      L += hi_f(v) * wgt;
    }
    auto wt = [&](int u) {
      return __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, wgt), u));
    };
    const int cnt = min(64, np - p0);
    const uint64_t* src = xrow + (int64_t)p0 * xstride;
    int u = 0;
    for (; u + 4 <= cnt; u += 4) {
      const uint64_t x0 = ld(src + (int64_t)u * xstride);
      const uint64_t x1 = ld(src + (int64_t)(u + 1) * xstride);
      const uint64_t x2 = ld(src + (int64_t)(u + 2) * xstride);
      const uint64_t x3 = ld(src + (int64_t)(u + 3) * xstride);
      a0 += lo_f(x0) * wt(u), a1 += hi_f(x0) * wt(u);
      a0 += lo_f(x1) * wt(u + 1), a1 += hi_f(x1) * wt(u + 1);
      a0 += lo_f(x2) * wt(u + 2), a1 += hi_f(x2) * wt(u + 2);
      a0 += lo_f(x3) * wt(u + 3), a1 += hi_f(x3) * wt(u + 3);
    }
    for (; u < cnt; ++u) {
      const uint64_t x = ld(src + (int64_t)u * xstride);
      a0 += lo_f(x) * wt(u), a1 += hi_f(x) * wt(u);
    }
  }
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) L += __shfl_xor(L, o, 64);
  const float inv = L > 0.f ? 1.f / L : 0.f;
  return make_float2(a0 * inv, a1 * inv);
}

// The merged output rows r_begin .. r_end - 1 of one (sequence, KV head)
// row block (row r: query r / rep, head kvh rep + r % rep; the sequence's
// first token tok0) from its np partitions' device-scope partials at
// base: wavefront w takes rows r_begin + w, r_begin + w + kWv, ... in groups
// of kMergeRows, lane l dims 2l and 2l + 1, with every load of a group issued
// before the first sum (np <= kMergeFew; longer splits row by row). Groups of
// 5 rows take a spec-verify row block (5 queries x 4 heads) in one round on 4
// wavefronts; kernels whose item body needs fewer registers use groups of 2,
// so that the merge does not raise their register count.
constexpr int kMergeFew = 8;
template <typename T, int D, int kWv, int kMergeRows>
__device__ __forceinline__ void merge_tile_rows(T* __restrict__ out, int H, int rep, int kvh,
                                                int r_begin, int r_end, int tok0, int np,
                                                int64_t base, const float2* ml, const float* po,
                                                int wave, int lane) {
  static_assert(D % 2 == 0 && D <= 128, "dim pairs per lane");
  const bool pair_ok = 2 * lane < D;
  const int dp = pair_ok ? lane : 0;  // lanes past the row read pair 0 and store nothing
  auto ld = [](const uint64_t* a) {
    return __hip_atomic_load(a, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  };
  auto row_at = [&](int r) {  // the row's first partial row
    const int j = r / rep;
    return base + (int64_t)(j * H + kvh * rep + (r - j * rep)) * np;
  };
  auto store = [&](int r, float o0, float o1) {
    const int j = r / rep;
    T* dst = out + ((int64_t)(tok0 + j) * H + kvh * rep + (r - j * rep)) * D + 2 * lane;
    if (!pair_ok) return;
    if constexpr (sizeof(T) == 2)
      *reinterpret_cast<uint32_t*>(dst) = cvt_pk_bf16(o0, o1);
    else
      *reinterpret_cast<float2*>(dst) = make_float2(o0, o1);
  };
  if (np > kMergeFew) {
    for (int r = r_begin + wave; r < r_end; r += kWv) {
      const int64_t rb = row_at(r);
      const float2 o = merge_partitions(reinterpret_cast<const uint64_t*>(ml + rb),
                                        reinterpret_cast<const uint64_t*>(po + rb * D) + dp, D / 2,
                                        np, lane);
      store(r, o.x, o.y);
    }
    return;
  }
  for (int r0 = r_begin + wave; r0 < r_end; r0 += kWv * kMergeRows) {
    uint64_t mv[kMergeRows], xv[kMergeRows][kMergeFew];
#pragma unroll
    for (int g = 0; g < kMergeRows; ++g) {
      const int64_t rb = row_at(min(r0 + kWv * g, r_end - 1));
      mv[g] = ld(reinterpret_cast<const uint64_t*>(ml + rb) + min(lane, np - 1));
#pragma unroll
      for (int u = 0; u < kMergeFew; ++u)
        xv[g][u] = ld(reinterpret_cast<const uint64_t*>(po + (rb + min(u, np - 1)) * D) + dp);
    }
#pragma unroll
    for (int g = 0; g < kMergeRows; ++g) {
      const int r = r0 + kWv * g;
      if (r >= r_end) break;  // uniform over the wavefront
      const float m = lo_f(mv[g]);
      float M = lane < np ? m : -__builtin_inff();
#pragma unroll
      for (int o = 32; o > 0; o >>= 1) M = fmaxf(M, __shfl_xor(M, o, 64));
      const float wgt = lane < np && m != -__builtin_inff() ? exp2_fast(m - M) : 0.f;
      float L = lane < np ? hi_f(mv[g]) * wgt : 0.f;
      float a0 = 0.f, a1 = 0.f;
#pragma unroll
      for (int u = 0; u < kMergeFew; ++u) {
        if (u >= np) break;  // uniform
        const float wt =
            __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, wgt), u));
        a0 += lo_f(xv[g][u]) * wt, a1 += hi_f(xv[g][u]) * wt;
      }
#pragma unroll
      for (int o = 32; o > 0; o >>= 1) L += __shfl_xor(L, o, 64);
      const float inv = L > 0.f ? 1.f / L : 0.f;
      store(r, a0 * inv, a1 * inv);
    }
  }
}

// One workgroup item of the tile kernel (kWv wavefronts; the caller's LDS).
// item_off holds the first item of each sequence, in sequence order, or (32-row
// items) in the order of item_seq, which names the sequences; there a
// sequence's row blocks come last block first.
// RW = rows per wavefront: 16 (v_mfma_f32_16x16x32_bf16 / 16x16x4f32, 64-row
// items on 4 wavefronts; short-query sequences, which may be split into
// partitions, and fp32) or 32 (bf16 v_mfma_f32_32x32x16_bf16, 256-row items,
// for long query chunks: one pass of 8 wavefronts, or two passes of the step
// kernel's 4; each K/V tile read from LDS feeds twice the rows). With RW 32
// a lane holds row l%32; its S^T values are keys 32t + 8(r/4) + 4(l/32) + r%4
// (r < 16) and its O^T values dims 32u + 8(r/4) + 4(l/32) + r%4.
template <typename T, int D, int RW, bool kMixed, int kWv = 4, typename TKV = T>
__device__ __forceinline__ void tile_body(TileLds<T, D, RW>& lds, int it, int pass, int P,
                                          const int32_t* __restrict__ item_off,
                                          const int32_t* __restrict__ item_seq,
                                          VL_ATTN_PARAMS_KV(T, TKV)) {
  const int tid = item_tid<kMixed>();
  constexpr bool kBf16 = sizeof(T) == 2;
  constexpr bool kW = RW == 32;
  static_assert(RW == 16 || (RW == 32 && kBf16), "32-row wavefronts are bf16 only");
  static_assert(std::is_same<T, TKV>::value || (!kBf16 && RW == 16),
                "narrow caches under fp32 queries only");
  constexpr int kRows = kWv * RW;                         // rows per pass (kWv wavefronts)
  // a 32-row item spans kWideRows rows: one pass of an 8-wavefront
  // workgroup, or `pass` 0 or 1 of a 4-wavefront one (the step kernel
  // hands out the two passes as separate items)
  constexpr int kItemRows = kW ? kWideRows : kRows;
  static_assert(kItemRows % kRows == 0, "rows per item");
  // staging: the workgroup's threads as kWv / 4 groups of 256; group hg
  // stages the 16-key units hg, hg + kWv / 4, ... (wave-uniform)
  constexpr int kHalves = kWv / 4;
  const int hg = __builtin_amdgcn_readfirstlane(tid >> 8), tl = tid & 255;
  constexpr int kDT = D / (kW ? 32 : 16);                // d tiles of the output
  constexpr int kKS = kW ? D / 16 : kBf16 ? D / 32 : D / 4;  // k-steps of the QK^T product
  constexpr int kST = kTileKeys / (kW ? 32 : 16);        // key subtiles per LDS tile
  constexpr int kCV = kW ? 16 : 4;                       // accumulator values per subtile
  using Lds = TileLds<T, D, RW>;
  using AccT = float __attribute__((ext_vector_type(kCV)));
  static_assert(!kBf16 || Lds::kUnits * 256 == kTileKeys * Lds::kChunks,
                "bf16 tile staging assumes head_dim 64 or 128");
  static_assert(kHalves == 1 || (kBf16 && Lds::kUnits % kHalves == 0),
                "8-wavefront items are bf16");
  const int wave = tid >> 6;
  const int lane = tid & 63;
  const int col = lane & (RW - 1);  // the lane's row within the wave's rows
  const int grp = lane / RW;        // lane group: which keys / d chunk it holds
  const int rep = H / Hkv;
  // elements between a KV head's consecutive slots inside a block and
  // between KV heads: token-major [slots, Hkv, D] or head-major [blocks, Hkv,
  // bs, D] caches
  const int64_t slot_stride = kv_hm ? D : (int64_t)Hkv * D;
  const int64_t head_stride = kv_hm ? (int64_t)D << bs_log2 : D;

  {
    // the item's sequence i, context partition, KV head and row block: 32-row
    // items by the sequence's position in item_seq (item_off in that order);
    // 16-row items from a first list, item_off (sequence order, item_off[S]
    // items): partitions 0 .. ns - 1 of sequence i, for ns its items there
    // over its KV heads and row blocks (every partition, or all but the
    // last), then from a second list in the order of item_seq (tail_seq),
    // whose offsets follow it: the last partitions
    int i, part, kvh, rb_local, q_len;
    const bool first = !kW && it < item_off[S];
    if (kW || !first) {
      const int32_t* off = kW ? item_off : item_seq + S;
      const int t = kW ? it : it - item_off[S];
      const int pos = wave_upper_bound_le(off, S + 1, t);
      i = item_seq[pos];
      q_len = qsl[i + 1] - qsl[i];
      const int local = t - off[pos];
      part = kW ? 0 : nparts[i] - 1, kvh = local % Hkv, rb_local = local / Hkv;
    } else {
      i = wave_upper_bound_le(item_off, S + 1, it);
      q_len = qsl[i + 1] - qsl[i];
      const int local = it - item_off[i];
      const int ns = (item_off[i + 1] - item_off[i]) / (Hkv * cdiv(q_len * rep, kItemRows));
      part = local % ns, kvh = (local / ns) % Hkv, rb_local = (local / ns) / Hkv;
    }
    const int ctx = seq_lens[i];
    const int np = kW ? 1 : nparts[i];
    const int nrows = q_len * rep;
    const bool stream_kv = nrows <= kRows;  // no other pass or row block reads this K / V
    const int rb = kW ? cdiv(nrows, kItemRows) - 1 - rb_local : rb_local;
    const int rbase = rb * kItemRows + pass * kRows;  // the pass's first row
    if (rbase >= nrows) return;
    const int kbeg = np > 1 ? part * P : 0;
    const int kend = np > 1 ? min(ctx, kbeg + P) : ctx;
    // keys the block's last row can see bound the tiles the workgroup loads
    const int blk_last = min(nrows - 1, rbase + kRows - 1);
    const int kend_wg = min(kend, ctx - q_len + blk_last / rep + 1);
    const int row0 = rbase + wave * RW;
    const int wave_last = min(nrows - 1, row0 + RW - 1);
    const int kend_wave = row0 < nrows ? min(kend, ctx - q_len + wave_last / rep + 1) : kbeg;
    const int my_row = row0 + col;
    const bool row_ok = my_row < nrows;
    const int j = row_ok ? my_row / rep : 0;
    const int head = kvh * rep + (row_ok ? my_row - (my_row / rep) * rep : 0);
    const int tok = qsl[i] + j;
    const int qpos = ctx - q_len + j;
    const int qpos_wave_min = ctx - q_len + row0 / rep;  // earliest query row of the wave
    const int32_t* table = bt + (int64_t)i * bt_stride;
    const int64_t kv_off = (int64_t)kvh * head_stride;

    // Q^T operand of the QK^T product, kept in registers for the whole item
    typename std::conditional<kBf16, bf16x8_t, float>::type qop[kKS];
    {
      const T* qrow = query + (int64_t)tok * q_stride + (int64_t)head * D;
#pragma unroll
      for (int s = 0; s < kKS; ++s) {
        if constexpr (kBf16) {
          const int d0 = kW ? 16 * s + 8 * grp : 32 * s + 8 * grp;
          uint4 w = row_ok ? *reinterpret_cast<const uint4*>(qrow + d0) : make_uint4(0, 0, 0, 0);
          qop[s] = __builtin_bit_cast(bf16x8_t, w);
        } else {
          qop[s] = row_ok ? qrow[4 * s + grp] : 0.f;
        }
      }
    }
    AccT acc[kDT];
#pragma unroll
    for (int u = 0; u < kDT; ++u)
#pragma unroll
      for (int r = 0; r < kCV; ++r) acc[u][r] = 0.f;
    float m_run = -__builtin_inff();
    float l_part = 0.f;  // this lane's share of the row sum

    // ---- prefetch registers: this thread's share of one tile's K and V
    const uint32_t blk_elems = (uint32_t)(Hkv * D) << bs_log2;
    const uint32_t bs_mask = (1u << bs_log2) - 1;
    auto row_of = [&](int key) -> int64_t {  // element offset of key's head row
      const uint32_t blk = (uint32_t)table[key >> bs_log2];
      return (int64_t)((uint64_t)blk * blk_elems) +
             (int64_t)((key & bs_mask) * (uint32_t)slot_stride) + kv_off;
    };
    // 16-row bf16 items of head_dim 128 (short queries: spec-verify, HBM-bound)
    // keep three tiles' loads in flight; the others one
    constexpr bool kDeep = kBf16 && RW == 16 && D == 128;
    uint4 pk[Lds::kUnits / kHalves], pv[Lds::kUnits / kHalves];
    uint4 pk2[kDeep ? Lds::kUnits : 1], pv2[kDeep ? Lds::kUnits : 1];
    uint4 pk3[kDeep ? Lds::kUnits : 1], pv3[kDeep ? Lds::kUnits : 1];
    // bf16 staging: K unit r of a tile is keys k0 + kUnitKeys r + threadIdx / kChunks,
    // chunk threadIdx % kChunks; with blocks of >= kUnitKeys slots the unit lies
    // in one block whose id is uniform over the workgroup (tile starts are
    // multiples of 64); in a head-major cache the unit is one contiguous span.
    // Keys past the workgroup's end are masked: K reads stay in the last
    // key's block (finite or not, the score is replaced by -inf); V reads
    // re-read the last key, finite values whose weights are zero.
    constexpr int kUnitKeys = 256 / Lds::kChunks;
    const bool unit_blocks = (1 << bs_log2) >= kUnitKeys;
    const uint32_t k_thr_off =
        (uint32_t)(tl / Lds::kChunks) * (uint32_t)slot_stride + (tl % Lds::kChunks) * 8;
    // nt: std::true_type / std::false_type, non-temporal loads or not;
    // (pk, pv): the registers the tile lands in
    constexpr int kU = Lds::kUnits / kHalves;  // units this thread stages
    using Regs = uint4[kU];
    auto prefetch_as = [&](int k0, auto nt, Regs& pk, Regs& pv) {
      constexpr bool kNt = decltype(nt)::value;
      if constexpr (kBf16) {
        if (unit_blocks) {
          // the units' block ids first (scalar loads, issued together), then
          // every K and V address from them; V keys past the end re-read the
          // last key, which lies in the last unit's block, as does a unit
          // past the end (its K reads stay there too; their scores are masked)
          const int klast = (kend_wg - 1) & ~(kUnitKeys - 1);
          uint32_t blk[kU];
#pragma unroll
          for (int r = 0; r < kU; ++r)
            blk[r] = (uint32_t)table[min(k0 + kUnitKeys * (kHalves * r + hg), klast) >> bs_log2];
          const int tk = tl / Lds::kChunks, tc = (tl % Lds::kChunks) * 8;
#pragma unroll
          for (int r = 0; r < kU; ++r) {
            const int kr = min(k0 + kUnitKeys * (kHalves * r + hg), klast);
            const int64_t boff = (int64_t)((uint64_t)blk[r] * blk_elems) + kv_off;
            pk[r] = load16_kv<kNt>(kc + boff + ((uint32_t)(kr & bs_mask) * (uint32_t)slot_stride +
                                                k_thr_off));
            const int vkey = min(kr + tk, kend_wg - 1);
            pv[r] = load16_kv<kNt>(vc + boff + ((uint32_t)(vkey & bs_mask) * (uint32_t)slot_stride + tc));
          }
        } else {
#pragma unroll
          for (int r = 0; r < kU; ++r) {
            const int idx = tl + 256 * (kHalves * r + hg);
            const int kk = idx / Lds::kChunks, cc = idx - kk * Lds::kChunks;
            const int64_t off = row_of(min(k0 + kk, kend_wg - 1)) + cc * 8;
            pk[r] = load16_kv<kNt>(kc + off);
            pv[r] = load16_kv<kNt>(vc + off);
          }
        }
      } else {
#pragma unroll
        for (int r = 0; r < Lds::kUnits; ++r) {
          const int idx = tid + 256 * r;
          const int kk = idx / Lds::kChunks, c = idx - kk * Lds::kChunks;
          const int key = k0 + kk;
          const bool ok = idx < kTileKeys * Lds::kChunks && key < kend_wg;
          const int64_t off = ok ? row_of(key) + c * 4 : 0;
          pk[r] = ok ? load4_as_f32(kc + off) : make_uint4(0, 0, 0, 0);
          pv[r] = ok ? load4_as_f32(vc + off) : make_uint4(0, 0, 0, 0);
        }
      }
    };
    // one uniform branch per tile, around branch-free loads
    auto prefetch = [&](int k0, Regs& dk, Regs& dv) {
      if (stream_kv)
        prefetch_as(k0, std::true_type{}, dk, dv);
      else
        prefetch_as(k0, std::false_type{}, dk, dv);
    };
    auto stage = [&](Lds& b, const Regs& pk, const Regs& pv) {  // registers -> LDS b
      if constexpr (kBf16) {
#pragma unroll
        for (int r = 0; r < kU; ++r) {
          const int idx = tl + 256 * (kHalves * r + hg);
          const int kk = idx / Lds::kChunks, c = idx - kk * Lds::kChunks;
          *reinterpret_cast<uint4*>(&b.k[kk * Lds::kRow + c * 8]) = pk[r];
          *reinterpret_cast<uint4*>(&b.v[kk * Lds::vRow + c * 8]) = pv[r];
        }
      } else {
#pragma unroll
        for (int r = 0; r < Lds::kUnits; ++r) {
          const int idx = tid + 256 * r;
          if (idx < kTileKeys * Lds::kChunks) {
            const int kk = idx / Lds::kChunks, c = idx - kk * Lds::kChunks;
            float* kd = &b.k[kk * Lds::kRow + c * 4];
            float* vd = &b.v[kk * Lds::vRow + c * 4];
            kd[0] = __uint_as_float(pk[r].x), kd[1] = __uint_as_float(pk[r].y);
            kd[2] = __uint_as_float(pk[r].z), kd[3] = __uint_as_float(pk[r].w);
            vd[0] = __uint_as_float(pv[r].x), vd[1] = __uint_as_float(pv[r].y);
            vd[2] = __uint_as_float(pv[r].z), vd[3] = __uint_as_float(pv[r].w);
          }
        }
      }
    };
    // key of accumulator value r of subtile t for this lane
    auto key_of = [&](int k0, int t, int r) {
      return kW ? k0 + 32 * t + 8 * (r >> 2) + 4 * grp + (r & 3) : k0 + 16 * t + 4 * grp + r;
    };

    const int ntile = kend_wg > kbeg ? (kend_wg - kbeg + kTileKeys - 1) / kTileKeys : 0;
    // one tile of keys k0.. from LDS b into the running softmax and output
    auto compute = [&](const Lds& b, int k0) {
      // ---- S^T = K Q^T for the key subtiles
      AccT sc[kST];
      if constexpr (kW) {
        // every K operand of a subtile read before its MFMAs, the next
        // subtile's reads paired with them: the LDS latency is paid once per
        // subtile instead of once per two MFMAs (the compiler's own order
        // kept two reads in flight)
        uint4 kw[2][kKS];
#pragma unroll
        for (int s = 0; s < kKS; ++s)
          kw[0][s] = *reinterpret_cast<const uint4*>(&b.k[col * Lds::kRow + 16 * s + 8 * grp]);
#pragma unroll
        for (int t = 0; t < kST; ++t) {
#pragma unroll
          for (int r = 0; r < kCV; ++r) sc[t][r] = 0.f;
#pragma unroll
          for (int s = 0; s < kKS; ++s) {
            if (t + 1 < kST)
              kw[(t + 1) & 1][s] = *reinterpret_cast<const uint4*>(
                  &b.k[(32 * (t + 1) + col) * Lds::kRow + 16 * s + 8 * grp]);
            sc[t] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(__builtin_bit_cast(bf16x8_t, kw[t & 1][s]),
                                                            qop[s], sc[t], 0, 0, 0);
          }
        }
        __builtin_amdgcn_sched_group_barrier(0x100, kKS, 0);  // subtile 0's reads
#pragma unroll
        for (int i = 0; i < kKS * (kST - 1); ++i) {
          __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);  // an MFMA
          __builtin_amdgcn_sched_group_barrier(0x100, 1, 0);  // a read of the next subtile
        }
        __builtin_amdgcn_sched_group_barrier(0x008, kKS, 0);  // the last subtile's MFMAs
      }
#pragma unroll
      for (int t = 0; t < kST && !kW; ++t) {
#pragma unroll
        for (int r = 0; r < kCV; ++r) sc[t][r] = 0.f;
#pragma unroll
        for (int s = 0; s < kKS; ++s) {
          if constexpr (kW) {
          } else if constexpr (kBf16) {
            const uint4 w = *reinterpret_cast<const uint4*>(
                &b.k[(16 * t + col) * Lds::kRow + 32 * s + 8 * grp]);
            sc[t] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(bf16x8_t, w),
                                                            qop[s], sc[t], 0, 0, 0);
          } else {
            const float a = b.k[(16 * t + col) * Lds::kRow + 4 * s + grp];
            sc[t] = __builtin_amdgcn_mfma_f32_16x16x4f32(a, qop[s], sc[t], 0, 0, 0);
          }
        }
      }
      // ---- mask, online softmax (base 2). A tile every row of the wave
      // sees in full needs no per-key test (rows past the block's end only
      // feed their own, never written, lanes). The exponent reference m_run
      // moves only when a row's tile max exceeds it by more than kLazy: the
      // weights then stay below 2^kLazy (exact in fp32, relative error in
      // bf16 unchanged), so the accumulator rescale is a rare wave-uniform
      // branch instead of a multiply of every accumulator per tile.
      constexpr float kLazy = 8.f;
      float cmax = -__builtin_inff();
      const bool full = k0 + kTileKeys - 1 <= qpos_wave_min && k0 + kTileKeys <= kend;
      if (!full) {
        // value (t, r) holds key key_of(k0, t, r) = key_of(k0, 0, 0) + a constant;
        // rows past the end (row_ok false) use query 0's limit and are never written
        const int lim = min(qpos + 1, kend) - key_of(k0, 0, 0);
#pragma unroll
        for (int t = 0; t < kST; ++t)
#pragma unroll
          for (int r = 0; r < kCV; ++r)
            sc[t][r] = key_of(0, t, r) - 4 * grp < lim ? sc[t][r] : -__builtin_inff();
      }
#pragma unroll
      for (int t = 0; t < kST; ++t)
#pragma unroll
        for (int r = 0; r < kCV; ++r) cmax = fmaxf(cmax, sc[t][r]);
      if constexpr (!kW) cmax = fmaxf(cmax, __shfl_xor(cmax, 16, 64));
      if constexpr (kW) {
        // the row's other lane (l ^ 32) by a lane swap, not an LDS permute
        const auto sw = __builtin_amdgcn_permlane32_swap(__float_as_uint(cmax), __float_as_uint(cmax),
                                                         false, false);
        cmax = fmaxf(__uint_as_float(sw[0]), __uint_as_float(sw[1]));
      } else {
        cmax = fmaxf(cmax, __shfl_xor(cmax, 32, 64));
      }
      const float cm = cmax * scale_log2;
      if (__any(cm > m_run + kLazy)) {
        const float m_new = fmaxf(m_run, cm);
        const float alpha = m_new == -__builtin_inff() ? 1.f : exp2_fast(m_run - m_new);
        l_part *= alpha;
#pragma unroll
        for (int u = 0; u < kDT; ++u) acc[u] *= alpha;
        m_run = m_new;
      }
      // the first V^T operands of the 32-row PV product, read now so that
      // their LDS latency passes during the exponentials
      constexpr int kPvSteps = kST * 2 * kDT;  // (subtile t, half hh, d tile u)
      constexpr int kLook = kW ? kPvLook : 1;
      auto vread = [&](int st) {  // operand of step st: dims 32u + .., keys 32t + 16hh + ..
        if constexpr (kW) {
          // keys 32t + 16hh + 4 grp + (0..3) and + 8, dims 32u + l % 32 (16-lane
          // group: dims 32u + 16 (l / 16 % 2) + ..)
          const int t = st / (2 * kDT), hh = (st / kDT) % 2, u = st % kDT;
          const int li = lane & 15;
          const uint16_t* vp = &b.v[(32 * t + 16 * hh + 4 * grp + (li >> 2)) * Lds::vRow + 32 * u +
                                    16 * ((lane >> 4) & 1) + 4 * (li & 3)];
          const uint2 lo = lds_read_tr16(vp);
          const uint2 hi = lds_read_tr16(vp + 8 * Lds::vRow);
          return make_uint4(lo.x, lo.y, hi.x, hi.y);
        } else {
          return make_uint4(0, 0, 0, 0);
        }
      };
      uint4 vq[kLook];
      if constexpr (kW) {
#pragma unroll
        for (int i = 0; i < kLook; ++i) vq[i] = vread(i);
      }
      // masked scores are -inf and give 0; a row with nothing unmasked yet
      // keeps m_run = -inf and uses reference 0
      const float neg_ref = m_run == -__builtin_inff() ? 0.f : -m_run;
      float pr[kST][kCV];
      float psum = 0.f;
#pragma unroll
      for (int t = 0; t < kST; ++t)
#pragma unroll
        for (int r = 0; r < kCV; ++r) {
          pr[t][r] = exp2_fast(fmaf(sc[t][r], scale_log2, neg_ref));
          if constexpr (!kW) psum += pr[t][r];
        }
      if constexpr (!kW) l_part += psum;
      // ---- O^T += V^T P^T
      if constexpr (kW) {
        // 16-key k-steps: subtile t, half h covers keys 32t + 16h ..; this
        // lane's values r = 8h .. 8h+7 are exactly the B operand's k-slots.
        // Each V^T operand is read kLook steps before its MFMA.
        bf16x8_t pop;
#pragma unroll
        for (int st = 0; st < kPvSteps; ++st) {
          const int t = st / (2 * kDT), hh = (st / kDT) % 2, u = st % kDT;
          if (u == 0) {
            uint4 pw;
            pw.x = cvt_pk_bf16(pr[t][8 * hh + 0], pr[t][8 * hh + 1]);
            pw.y = cvt_pk_bf16(pr[t][8 * hh + 2], pr[t][8 * hh + 3]);
            pw.z = cvt_pk_bf16(pr[t][8 * hh + 4], pr[t][8 * hh + 5]);
            pw.w = cvt_pk_bf16(pr[t][8 * hh + 6], pr[t][8 * hh + 7]);
            pop = __builtin_bit_cast(bf16x8_t, pw);
            // the row sum of the weights as the MFMA uses them (bf16), by
            // dot products with ones: 4 VALU ops per 8 weights instead of 8
            const bf16x2_t ones = {(__bf16)1.f, (__bf16)1.f};
            psum = __builtin_amdgcn_fdot2_f32_bf16(__builtin_bit_cast(bf16x2_t, pw.x), ones, psum, false);
            psum = __builtin_amdgcn_fdot2_f32_bf16(__builtin_bit_cast(bf16x2_t, pw.y), ones, psum, false);
            psum = __builtin_amdgcn_fdot2_f32_bf16(__builtin_bit_cast(bf16x2_t, pw.z), ones, psum, false);
            psum = __builtin_amdgcn_fdot2_f32_bf16(__builtin_bit_cast(bf16x2_t, pw.w), ones, psum, false);
          }
          const uint4 vw = vq[st % kLook];
          if (st + kLook < kPvSteps) vq[st % kLook] = vread(st + kLook);
          acc[u] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(__builtin_bit_cast(bf16x8_t, vw), pop,
                                                           acc[u], 0, 0, 0);
        }
        l_part += psum;
      } else if constexpr (kBf16) {
#pragma unroll
        for (int hh = 0; hh < 2; ++hh) {
          uint4 pw;
          pw.x = cvt_pk_bf16(pr[2 * hh][0], pr[2 * hh][1]);
          pw.y = cvt_pk_bf16(pr[2 * hh][2], pr[2 * hh][3]);
          pw.z = cvt_pk_bf16(pr[2 * hh + 1][0], pr[2 * hh + 1][1]);
          pw.w = cvt_pk_bf16(pr[2 * hh + 1][2], pr[2 * hh + 1][3]);
          const bf16x8_t pop = __builtin_bit_cast(bf16x8_t, pw);
#pragma unroll
          for (int u = 0; u < kDT; ++u) {
            // keys 32hh + 4 grp + (0..3) and + 16, dims 16u + l % 16
            const int li = lane & 15;
            const uint16_t* vp =
                &b.v[(32 * hh + 4 * grp + (li >> 2)) * Lds::vRow + 16 * u + 4 * (li & 3)];
            const uint2 lo = lds_read_tr16(vp);
            const uint2 hi = lds_read_tr16(vp + 16 * Lds::vRow);
            const uint4 vw = make_uint4(lo.x, lo.y, hi.x, hi.y);
            acc[u] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(bf16x8_t, vw), pop,
                                                             acc[u], 0, 0, 0);
          }
        }
      } else {
#pragma unroll
        for (int t = 0; t < kST; ++t)
#pragma unroll
          for (int e = 0; e < 4; ++e) {
            const float* vrow = &b.v[(16 * t + 4 * grp + e) * Lds::vRow];
#pragma unroll
            for (int u = 0; u < kDT; ++u)
              acc[u] = __builtin_amdgcn_mfma_f32_16x16x4f32(vrow[16 * u + col], pr[t][e], acc[u],
                                                            0, 0, 0);
          }
      }
    };
    // one tile: stage it from registers (pk, pv), refill them with the tile
    // `ahead` tiles later, compute
    auto tile_step = [&](int ti, int ahead, Regs& pk, Regs& pv) {
      const int k0 = kbeg + ti * kTileKeys;
      __syncthreads();  // the previous tile (or item) is done with the LDS buffer
      stage(lds, pk, pv);
      __syncthreads();
      if (ti + ahead < ntile) prefetch(k0 + ahead * kTileKeys, pk, pv);  // in flight meanwhile
      if (k0 < kend_wave) compute(lds, k0);  // else every row of the wave is past its end
    };
    if constexpr (kDeep) {
      // three tiles in flight (three register sets, the loop unrolled by
      // three so each set stays in fixed registers): three times the bytes in
      // flight for the HBM-bound short-query items, within the 2-waves-per-
      // SIMD register budget (242 VGPRs). Verify step: one tile in flight
      // 857-875 us, two 831-847, three 783-860 (two boxes)
      if (ntile > 0) prefetch(kbeg, pk, pv);
      if (ntile > 1) prefetch(kbeg + kTileKeys, pk2, pv2);
      if (ntile > 2) prefetch(kbeg + 2 * kTileKeys, pk3, pv3);
      for (int ti = 0; ti < ntile; ti += 3) {
        tile_step(ti, 3, pk, pv);
        if (ti + 1 < ntile) tile_step(ti + 1, 3, pk2, pv2);
        if (ti + 2 < ntile) tile_step(ti + 2, 3, pk3, pv3);
      }
    } else {
      if (ntile > 0) prefetch(kbeg, pk, pv);
      for (int ti = 0; ti < ntile; ++ti) tile_step(ti, 1, pk, pv);
    }
    // ---- row sums over the lane groups, then write
    float l_row = l_part;
    if constexpr (!kW) l_row += __shfl_xor(l_row, 16, 64);
    l_row += __shfl_xor(l_row, 32, 64);
    if (row_ok) {
      if (np == 1) {
        const float inv = l_row > 0.f ? 1.f / l_row : 0.f;
        T* orow = out + ((int64_t)tok * H + head) * D;
#pragma unroll
        for (int u = 0; u < kDT; ++u)
#pragma unroll
          for (int b4 = 0; b4 < kCV / 4; ++b4) {
            const int d = kW ? 32 * u + 8 * b4 + 4 * grp : 16 * u + 4 * grp;
            const float x0 = acc[u][4 * b4] * inv, x1 = acc[u][4 * b4 + 1] * inv;
            const float x2 = acc[u][4 * b4 + 2] * inv, x3 = acc[u][4 * b4 + 3] * inv;
            if constexpr (kBf16) {
              *reinterpret_cast<uint2*>(orow + d) = make_uint2(cvt_pk_bf16(x0, x1), cvt_pk_bf16(x2, x3));
            } else {
              *reinterpret_cast<float4*>(orow + d) = make_float4(x0, x1, x2, x3);
            }
          }
      } else {
        // the partial at device scope (written through to the point of
        // coherence of all XCDs), for the row block's last workgroup
        const int64_t prow = (int64_t)split_base[i] + (int64_t)(j * H + head) * np + part;
        uint64_t* dst = reinterpret_cast<uint64_t*>(po + prow * D);
#pragma unroll
        for (int u = 0; u < kDT; ++u)
#pragma unroll
          for (int b4 = 0; b4 < kCV / 4; ++b4) {
            const int d = kW ? 32 * u + 8 * b4 + 4 * grp : 16 * u + 4 * grp;
            __hip_atomic_store(dst + d / 2, pack2(acc[u][4 * b4], acc[u][4 * b4 + 1]),
                               __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
            __hip_atomic_store(dst + d / 2 + 1, pack2(acc[u][4 * b4 + 2], acc[u][4 * b4 + 3]),
                               __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
          }
        if (grp == 0)
          __hip_atomic_store(reinterpret_cast<uint64_t*>(ml + prow), pack2(m_run, l_row),
                             __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
      }
    }
    if (np > 1) {  // uniform over the workgroup (32-row items are never split)
      // Split rows are merged in the kernel by the last workgroup to finish a
      // partition of the row block, as the bandwidth decode kernel merges its
      // ranges: partial stores completed, then one device-scope arrival on
      // the row block's counter (after the sequence's partial rows; the plan
      // zeroes it, the last arrival resets it); the last reads every
      // partition's partial with device-scope loads.
      asm volatile("s_waitcnt vmcnt(0)" ::: "memory");  // this thread's stores have completed
      __syncthreads();  // every thread's have
      const int nrb = cdiv(nrows, kItemRows);
      if (tid == 0) {
        int32_t* cnt = reinterpret_cast<int32_t*>(ml + split_base[i] + (int64_t)q_len * H * np +
                                                  kvh * nrb + rb);
        const int prev = __hip_atomic_fetch_add(cnt, 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        lds.last = prev == np - 1;
        if (prev == np - 1) __hip_atomic_store(cnt, 0, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
      }
      __syncthreads();
      if (lds.last) {
        asm volatile("" ::: "memory");  // no load below moves above the arrival
        merge_tile_rows<T, D, kWv, kDeep ? 5 : 2>(out, H, rep, kvh, rbase,
                                                  min(nrows, rbase + kItemRows), qsl[i], np,
                                                  (int64_t)split_base[i], ml, po, wave, lane);
      }
    }
  }
}

// The last workgroup to leave a persistent kernel (every claim of every
// workgroup has returned) zeroes the work counters counters[0..n) and the
// exit counter counters[n] for the next run.
__device__ __forceinline__ void leave_and_reset(int32_t* counters, int n) {
  if (threadIdx.x == 0) {
    const int prev =
        __hip_atomic_fetch_add(counters + n, 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    if (prev == (int)gridDim.x - 1) {
      for (int k = 0; k <= n; ++k)
        __hip_atomic_store(counters + k, 0, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    }
  }
}

constexpr int kXcds = 8;

// The item index of claim c of a persistent kernel's queue (items base,
// base + stride, ...), or n (none: the claimer stops) when it falls outside
// the n items. Computed in 64 bits, so that no counter value, whatever it
// held, gives an index that wraps to a negative int and passes an `it < n`
// test into an item body.
__device__ __forceinline__ int claimed_item(int64_t c, int stride, int base, int n) {
  const int64_t it = c * stride + base;
  return c < 0 || it >= n ? n : (int)it;
}

// RW = rows per wavefront (see tile_body). Persistent workgroups take items
// from 8 queues, queue x holding the items it with it % 8 == x: workgroup b
// serves queue b % 8 (workgroups are dispatched round-robin over the 8 XCDs,
// so that is its XCD), its first item is the queue's (b / 8)-th and the later
// ones are claimed from the queue's counter (counters[x]), each at the start
// of the item before, so the atomic's latency is hidden and a workgroup
// without items leaves at once. Consecutive items are the KV heads of one row
// block, so with 8 KV heads each XCD's L2 holds the K/V of its own KV head,
// which the sequence's other row blocks read again; the plan orders the
// items longest first, so the launch ends on short ones. The counters are
// zeroed by the plan and, at the end of every run, by the claims that return
// each queue's last value (below).
template <typename T, int D, int RW, int kWv, typename TKV = T>
__global__ void __launch_bounds__(64 * kWv) __attribute__((amdgpu_waves_per_eu(2))) attend_tile_kernel(
    VL_ATTN_PARAMS_KV(T, TKV), const int32_t* __restrict__ hdr, const int32_t* __restrict__ item_off,
    const int32_t* __restrict__ item_seq, int32_t* counters) {
  __shared__ TileLds<T, D, RW> lds;
  __shared__ int claim_lds;
  if (hdr[11]) return;  // a mixed batch: the step kernel has these items
  const int P = hdr[2];
  const int n_items = hdr[RW == 32 ? 10 : 4];
  const int xcd = blockIdx.x % kXcds;
  const int per_queue = ((int)gridDim.x + kXcds - 1 - xcd) / kXcds;  // workgroups serving it
  int it = (blockIdx.x / kXcds) * kXcds + xcd;
  // The queue's items are xcd, xcd + 8, ... below n_items (n_q of them).
  // Every item processed makes one claim, so the claims on the queue's
  // counter return 0 .. n_q - 1, and the one that returns n_q - 1 is the
  // counter's last use in this run: its claimer zeroes it for the next run.
  // (An exit count instead, every workgroup's atomic on one address at the
  // end of the launch, cost tens of microseconds.)
  const int n_q = n_items > xcd ? (n_items - xcd + kXcds - 1) / kXcds : 0;
  while (it < n_items) {
    int nxt = 0;
    if (threadIdx.x == 0) {
      const int c = atomicAdd(counters + xcd, 1);
      if (c == n_q - 1)
        __hip_atomic_store(counters + xcd, 0, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
      nxt = claimed_item(per_queue + (int64_t)c, kXcds, xcd, n_items);
    }
    tile_body<T, D, RW, false, kWv, TKV>(lds, it, 0, P, item_off, item_seq, VL_ATTN_ARGS);
    __syncthreads();  // the item is done with the LDS; claim_lds has been read
    if (threadIdx.x == 0) claim_lds = nxt;
    __syncthreads();
    it = claim_lds;
  }
}

// ---------------------------------------------------- bandwidth decode -----


__device__ __forceinline__ float dot8(const uint4& a, const uint4& b, float c) {
  c = __builtin_amdgcn_fdot2_f32_bf16(__builtin_bit_cast(bf16x2_t, a.x),
                                      __builtin_bit_cast(bf16x2_t, b.x), c, false);
  c = __builtin_amdgcn_fdot2_f32_bf16(__builtin_bit_cast(bf16x2_t, a.y),
                                      __builtin_bit_cast(bf16x2_t, b.y), c, false);
  c = __builtin_amdgcn_fdot2_f32_bf16(__builtin_bit_cast(bf16x2_t, a.z),
                                      __builtin_bit_cast(bf16x2_t, b.z), c, false);
  c = __builtin_amdgcn_fdot2_f32_bf16(__builtin_bit_cast(bf16x2_t, a.w),
                                      __builtin_bit_cast(bf16x2_t, b.w), c, false);
  return c;
}

// Reduce over lanes that share (lane & 3): xor 4, 8, 16, 32.
__device__ __forceinline__ float stride4_max(float v) {
#pragma unroll
  for (int o = 4; o < 64; o <<= 1) v = fmaxf(v, __shfl_xor(v, o, 64));
  return v;
}
__device__ __forceinline__ float stride4_sum(float v) {
#pragma unroll
  for (int o = 4; o < 64; o <<= 1) v += __shfl_xor(v, o, 64);
  return v;
}


// Transposing sum over each row of 16 lanes: lane c (= lane & 15) holds 16
// partial values v[0..15]; afterwards it returns the row's total of v[c].
// Four halving steps pair lanes whose index differs in bit 3, 2, 1, 0 (row
// mirror 15 - c, half-row mirror, quad mirror, quad swap); each lane adds
// its partner's copy of the half of the values whose index bit matches its
// own and keeps that half. 45 VALU instead of 16 separate 4-step sums.
__device__ __forceinline__ float row_transpose_sum16(const float (&v)[16], int c) {
  float w[8], x[4], y[2];
#pragma unroll
  for (int i = 0; i < 8; ++i) {
    const float lo = v[i] + VL_DPP(0.f, v[i], 0x140, 0xF);
    const float hi = v[i + 8] + VL_DPP(0.f, v[i + 8], 0x140, 0xF);
    w[i] = (c & 8) ? hi : lo;
  }
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const float lo = w[i] + VL_DPP(0.f, w[i], 0x141, 0xF);
    const float hi = w[i + 4] + VL_DPP(0.f, w[i + 4], 0x141, 0xF);
    x[i] = (c & 4) ? hi : lo;
  }
#pragma unroll
  for (int i = 0; i < 2; ++i) {
    const float lo = x[i] + VL_DPP(0.f, x[i], 0x1B, 0xF);
    const float hi = x[i + 2] + VL_DPP(0.f, x[i + 2], 0x1B, 0xF);
    y[i] = (c & 2) ? hi : lo;
  }
  const float lo = y[0] + VL_DPP(0.f, y[0], 0xB1, 0xF);
  const float hi = y[1] + VL_DPP(0.f, y[1], 0xB1, 0xF);
  return (c & 1) ? hi : lo;
}

// One workgroup item = (decode sequence, KV head, range of the context);
// the 4 wavefronts split the range's 16-token blocks (wavefront w takes
// blocks w, w + 4, ...), each for the KV head's 4 query heads, and merge
// their (max, sum, output) in LDS at the end, so an item writes one output
// row per query head, or one partial row when the sequence has several
// ranges. Items are (range, KV head) with the KV heads of a range adjacent;
// full ranges come first, then the shorter last ranges, longest first.
// Persistent workgroups claim items from a counter.
//   QK: load j (j < 4) of a block gives lane l the 16-byte chunk l&15 of
//       token 4j + (l>>4) (whole 256-byte head rows, four per instruction);
//       four v_dot2_f32_bf16 per chunk and query head give 16 partial dot
//       products per lane, which a transposing DPP sum over each 16-lane
//       row turns into one (token, head) score per lane.
//   softmax: scores through LDS, per head max over the wavefront's chunk of
//       up to 16 blocks, exponentials rounded to bf16 (the sum adds the
//       rounded values).
//   PV: lane l reads dims chunk l&15 of tokens (l>>4)+4t (t < 4); token
//       pairs (t, t + 4) become bf16 pairs for v_dot2_f32_bf16; 4 heads x 8
//       dims of fp32 accumulators per lane, summed over the 4 token groups
//       at the end.
//   Split sequences are merged in the kernel, by the last workgroup to
//   finish a range of the (sequence, KV head): every workgroup writes its
//   unnormalised partial and (max, sum) per query head with device-scope
//   stores (written through to the point of coherence of all XCDs), waits
//   until they have completed, then counts itself in the sequence's arrival
//   counter with a device-scope atomic; the one that sees the count complete
//   reads the partials with device-scope loads, merges them (max-rescaled
//   log-sum-exp) and resets the counter. No cache-wide fence is needed: a
//   device-scope release or acquire writes back / invalidates the XCD's
//   whole L2 on gfx950, which made a fenced version 3x slower.
//   The last workgroup to leave resets the work counter for the next run.
struct DecodeLds {
  float4 p[4][kFChunk * 16];  // per wave: [block][token] -> 4 heads
  uint4 q[4][kFRep * 16];     // per wave: 4 heads x 128 bf16
  float4 acc[4][8 * 64];      // per wave: accumulators between chunks, then its
                              // merged [head][dim] result
  float2 wml[4][kFRep];       // per wave: (max, sum) per head
  int last;
};

// An item's prologue: its range descriptor (sequence, range, context length,
// query token), this lane's 16 bytes of the KV head's 4 query heads, and
// (lane b < 16) block b of the wavefront's first chunk.
struct DecodeItem {
  int4 d;
  uint4 q;
  int bid0;
};

// The prologue of item `it` with descriptor d (a scalar load): the query and
// the first chunk's block ids, loaded together.
__device__ __forceinline__ DecodeItem decode_fetch(int4 d, int it, int R, int Hkv, int wave,
                                                   int lane, const uint16_t* __restrict__ query,
                                                   int64_t q_stride,
                                                   const int32_t* __restrict__ bt, int bt_stride) {
  DecodeItem x;
  x.d = d;
  const int kvh = it % Hkv;
  x.q = load16(query + (int64_t)d.w * q_stride + (int64_t)kvh * kFRep * kFD + lane * 8);
  const int kbeg = d.y * R, kend = min(d.z, kbeg + R);
  const int ublk = (kend - kbeg + kFBs - 1) / kFBs;
  const int nw = ublk > wave ? (ublk - wave + 3) >> 2 : 0;
  const int wb0 = kbeg / kFBs + wave;
  x.bid0 = lane < min(kFChunk, nw) ? bt[(int64_t)d.x * bt_stride + wb0 + 4 * lane] : 0;
  return x;
}

// 16 bytes of K or V for the decode kernel. Each step reads every byte once
// out of a pool far larger than the caches: non-temporal (streaming) loads
// measured 222-230 us against 241 us with ordinary loads for the 256-sequence
// batch (1.29 GB).
__device__ __forceinline__ uint4 load_stream16(const char* p) {
  typedef unsigned int u32x4 __attribute__((ext_vector_type(4)));
  const u32x4 v = __builtin_nontemporal_load(reinterpret_cast<const u32x4*>(p));
  return make_uint4(v.x, v.y, v.z, v.w);
}

// One item (see above) by the 256 threads of a workgroup, from its prologue
// `cur`; R from the plan header. Load j of a block's K (j < 4) reads tokens
// 4 j .. 4 j + 3 of the KV head whole (lane l: chunk l % 16 of token 4 j +
// l / 16): four 256-byte rows per instruction, one contiguous 1 KB span in a
// head-major cache. The 16 chunks' partial dot products are then summed
// across each 16-lane row by a transposing DPP sum. (Lanes reading 64 bytes
// of each of 16 tokens per instruction, completed by a quad sum, measured
// 229-233 us against 215-221 us for the 256-sequence batch.)
template <bool kMixed, int kBK, int kBV>
__device__ __forceinline__ void decode_body(DecodeLds& s, int it, const DecodeItem& cur, int R,
                                            VL_ATTN_PARAMS(uint16_t)) {
  const int tid = item_tid<kMixed>();
  const int wave = tid >> 6;
  const int lane = tid & 63;
  const int qp = lane & 3;                    // the head of the lane's scores
  const int vcn = lane & 15, vg = lane >> 4;  // PV mapping
  // H = Hkv * kFRep (the bandwidth-kernel shape). Elements between a KV
  // head's consecutive slots of a block: Hkv * 128 (token-major) or 128
  // (head-major, where a head's 16 rows are one 4 KB span)
  const int64_t tok_stride = kv_hm ? kFD : (int64_t)Hkv * kFD;
  float4* pw = s.p[wave];
  uint4* qw = s.q[wave];
  float4* stash = s.acc[wave] + lane;  // stash[64 * k]: conflict-free
  float* pf = reinterpret_cast<float*>(pw);  // [block][token][head] scores, then probabilities
  const int64_t blk_bytes = (int64_t)kFBs * Hkv * kFD * 2;
  const char* kbytes = reinterpret_cast<const char*>(kc);
  const char* vbytes = reinterpret_cast<const char*>(vc);
  {
    const int kvh = it % Hkv;
    const int i = cur.d.x, part = cur.d.y, ctx = cur.d.z, tok = cur.d.w;
    const int np = nparts[i];
    const int kbeg = part * R;
    const int kend = min(ctx, kbeg + R);
    const int32_t* table = bt + (int64_t)i * bt_stride;
    // blocks of this wavefront: kbeg/16 + wave + 4k, k < nw
    const int ublk = (kend - kbeg + kFBs - 1) / kFBs;
    const int nw = ublk > wave ? (ublk - wave + 3) >> 2 : 0;
    const int wb0 = kbeg / kFBs + wave;  // first block; stride 4

    qw[lane] = cur.q;  // query of the 4 heads to LDS: [head][16-byte chunk]
    const int64_t kv_off = (int64_t)kvh * (kv_hm ? kFBs * kFD : kFD);
    // byte offsets of this lane inside a block (a block is 16 slots x Hkv x 128 bf16)
    const uint32_t k_lane = (uint32_t)(((lane >> 4) * tok_stride + kv_off) * 2) + (lane & 15) * 16;
    const uint32_t k_jstep = (uint32_t)(4 * tok_stride * 2);
    const uint32_t v_lane = (uint32_t)((vg * tok_stride + kv_off) * 2) + vcn * 16;
    const uint32_t v_tstep = (uint32_t)(4 * tok_stride * 2);

    float m_run = -__builtin_inff();  // per head qp (lanes share qp)
    float l_run = 0.f;
    float acc[kFRep][8];  // (re)defined before each chunk's PV pass
#pragma unroll
    for (int h = 0; h < kFRep; ++h)
#pragma unroll
      for (int e = 0; e < 8; ++e) acc[h][e] = 0.f;
    // every LDS region above is private to its wavefront until the merge
    for (int c = 0; c < nw; c += kFChunk) {
      const int nblk = min(kFChunk, nw - c);
      // block ids of the chunk: lane b holds block b, broadcast with readlane
      const int my_bid = c == 0 ? cur.bid0 : lane < nblk ? table[wb0 + 4 * (c + lane)] : 0;
      const int key0 = (wb0 + 4 * c) * kFBs;  // first key of chunk block 0; block b adds 64 b
      // ---- QK: kBK blocks per step, loads issued back to back (blocks past
      // the chunk end re-read the last block and are masked)
      float cmax = -__builtin_inff();
#pragma unroll 1
      for (int g = 0; g < nblk; g += kBK) {
        // keeps the query reads below inside the loop: hoisting them would pin
        // 64 registers for the whole item and lower the occupancy
        asm volatile("" ::: "memory");
        uint4 kb[kBK][4];
#pragma unroll
        for (int u = 0; u < kBK; ++u) {
          const int bid = __builtin_amdgcn_readlane(my_bid, min(g + u, nblk - 1));
          const char* bp = kbytes + (int64_t)bid * blk_bytes + k_lane;
#pragma unroll
          for (int j = 0; j < 4; ++j) kb[u][j] = load_stream16(bp + j * k_jstep);
        }
        // all loads of the group go out before any of them is consumed
        asm volatile("" ::: "memory");
        __builtin_amdgcn_sched_barrier(0);
        // lane (tg = lane / 16, c = lane % 16) holds chunk c of tokens 4 j +
        // tg; partial v[4 j + h] = chunk c of head h's query . chunk c of K,
        // summed over the row; lane c then holds token 4 (c / 4) + tg of head
        // c % 4 = qp
        const int c = lane & 15, tg = lane >> 4;
        uint4 qh[kFRep];
#pragma unroll
        for (int h = 0; h < kFRep; ++h) qh[h] = qw[h * 16 + c];
#pragma unroll
        for (int u = 0; u < kBK; ++u) {
          float v[16];
#pragma unroll
          for (int j = 0; j < 4; ++j)
#pragma unroll
            for (int h = 0; h < kFRep; ++h) v[4 * j + h] = dot8(qh[h], kb[u][j], 0.f);
          const float sc = row_transpose_sum16(v, c);
          const int tok16 = 4 * (c >> 2) + tg;
          const int key = key0 + (g + u) * 4 * kFBs + tok16;
          const bool ok = (g + u < nblk) && key < kend;
          const float sv = ok ? sc * scale_log2 : -__builtin_inff();
          cmax = fmaxf(cmax, sv);
          pf[((g + u) * 16 + tok16) * 4 + qp] = sv;
        }
      }
      // ---- online softmax update for head qp
      cmax = stride4_max(cmax);
      const float m_new = fmaxf(m_run, cmax);
      const float alpha = m_run == -__builtin_inff() ? 0.f : exp2f(m_run - m_new);
      // exponentials, in place, two blocks per step: lane l takes head
      // qp = l & 3 of the token pair (t, t + 4), t = ((l >> 2) & 3) + 8 * ((l >> 4)
      // & 1), of block 2 * step + (l >> 5), rounds both probabilities to bf16
      // and stores them packed as word slot * 4 + qp of the block's score
      // area, slot = t % 4 + 4 * (t / 8): the PV pass then reads one pair's 4
      // heads as a uint4. The block's scores are all read before its first
      // half is overwritten (one wavefront, LDS in program order). The row
      // sum adds the rounded values, the weights PV actually uses.
      float lsum = 0.f;
      // through every block the PV pass reads (bursts of kBV); blocks past
      // the chunk end get p = 0
      const int nbp = (nblk + kBV - 1) / kBV * kBV;
      {
        const int pt = ((lane >> 2) & 3) + 8 * ((lane >> 4) & 1);
        const int pslot = ((lane >> 2) & 3) + 4 * ((lane >> 4) & 1);
        uint32_t* pf32 = reinterpret_cast<uint32_t*>(pf);
        for (int b = lane >> 5; b < nbp; b += 2) {
          const float s0 = b < nblk ? pf[(b * 16 + pt) * 4 + qp] : -__builtin_inff();
          const float s1 = b < nblk ? pf[(b * 16 + pt + 4) * 4 + qp] : -__builtin_inff();
          const uint16_t h0 = f32_to_bf16(s0 == -__builtin_inff() ? 0.f : exp2f(s0 - m_new));
          const uint16_t h1 = f32_to_bf16(s1 == -__builtin_inff() ? 0.f : exp2f(s1 - m_new));
          lsum += bf16_to_f32(h0) + bf16_to_f32(h1);
          pf32[b * 64 + pslot * 4 + qp] = (uint32_t)h0 | ((uint32_t)h1 << 16);
        }
      }
      lsum = stride4_sum(lsum);
      l_run = l_run * alpha + lsum;
      m_run = m_new;
      if (c == 0) {
#pragma unroll
        for (int h = 0; h < kFRep; ++h)
#pragma unroll
          for (int e = 0; e < 8; ++e) acc[h][e] = 0.f;
      } else {  // a later chunk: the previous chunks' accumulators, rescaled
#pragma unroll
        for (int h = 0; h < kFRep; ++h) {
          const float ah = __shfl(alpha, h, 64);
          const float4 x0 = stash[64 * (2 * h)], x1 = stash[64 * (2 * h + 1)];
          acc[h][0] = x0.x * ah, acc[h][1] = x0.y * ah, acc[h][2] = x0.z * ah, acc[h][3] = x0.w * ah;
          acc[h][4] = x1.x * ah, acc[h][5] = x1.y * ah, acc[h][6] = x1.z * ah, acc[h][7] = x1.w * ah;
        }
      }
      // ---- PV: kBV blocks per step; probabilities past the context are 0
      // and the V rows there are zeroed so poisoned slots cannot leak in (a
      // NaN times 0 would)
#pragma unroll 1
      for (int g = 0; g < nblk; g += kBV) {
        uint4 vb[kBV][4];
#pragma unroll
        for (int u = 0; u < kBV; ++u) {
          const int bid = __builtin_amdgcn_readlane(my_bid, min(g + u, nblk - 1));
          const char* bp = vbytes + (int64_t)bid * blk_bytes + v_lane;
#pragma unroll
          for (int t = 0; t < 4; ++t) vb[u][t] = load_stream16(bp + t * v_tstep);
        }
        asm volatile("" ::: "memory");
        __builtin_amdgcn_sched_barrier(0);
        // rows (vg, vg + 4) and (vg + 8, vg + 12) pair up: v_perm builds a
        // (row0, row1) bf16 pair per dim and v_dot2_f32_bf16 applies the
        // pair's probabilities, 4 heads at a time
        const uint4* pp4 = reinterpret_cast<const uint4*>(pw);
#pragma unroll
        for (int u = 0; u < kBV; ++u) {
#pragma unroll
          for (int j = 0; j < 2; ++j) {
            const int key = key0 + (g + u) * 4 * kFBs + vg + 8 * j;
            const uint32_t keep0 = (g + u < nblk && key < kend) ? 0xffffffffu : 0u;
            const uint32_t keep1 = (g + u < nblk && key + 4 < kend) ? 0xffffffffu : 0u;
            const uint4 w0 = vb[u][2 * j], w1 = vb[u][2 * j + 1];
            const uint32_t a0[4] = {w0.x & keep0, w0.y & keep0, w0.z & keep0, w0.w & keep0};
            const uint32_t a1[4] = {w1.x & keep1, w1.y & keep1, w1.z & keep1, w1.w & keep1};
            const uint4 pp = pp4[(g + u) * 16 + vg + 4 * j];
            const uint32_t ph[kFRep] = {pp.x, pp.y, pp.z, pp.w};
#pragma unroll
            for (int m = 0; m < 4; ++m) {
              const uint32_t lo = __builtin_amdgcn_perm(a1[m], a0[m], 0x05040100u);
              const uint32_t hi = __builtin_amdgcn_perm(a1[m], a0[m], 0x07060302u);
#pragma unroll
              for (int h = 0; h < kFRep; ++h) {
                acc[h][2 * m] = __builtin_amdgcn_fdot2_f32_bf16(
                    __builtin_bit_cast(bf16x2_t, ph[h]), __builtin_bit_cast(bf16x2_t, lo),
                    acc[h][2 * m], false);
                acc[h][2 * m + 1] = __builtin_amdgcn_fdot2_f32_bf16(
                    __builtin_bit_cast(bf16x2_t, ph[h]), __builtin_bit_cast(bf16x2_t, hi),
                    acc[h][2 * m + 1], false);
              }
            }
          }
        }
      }
      if (c + kFChunk < nw) {  // another chunk follows: park the accumulators
#pragma unroll
        for (int h = 0; h < kFRep; ++h) {
          stash[64 * (2 * h)] = make_float4(acc[h][0], acc[h][1], acc[h][2], acc[h][3]);
          stash[64 * (2 * h + 1)] = make_float4(acc[h][4], acc[h][5], acc[h][6], acc[h][7]);
        }
      }
    }
    // ---- sum the 4 token groups; lanes 0..15 then hold 8 dims x 4 heads
#pragma unroll
    for (int h = 0; h < kFRep; ++h)
#pragma unroll
      for (int e = 0; e < 8; ++e) {
        float a = acc[h][e];
        a += __shfl_xor(a, 16, 64);
        a += __shfl_xor(a, 32, 64);
        acc[h][e] = a;
      }
    // ---- merge the 4 wavefronts through LDS (the wave's stash area holds its
    // [head][128] result)
    float* wres = reinterpret_cast<float*>(s.acc[wave]);
    if (vg == 0) {
#pragma unroll
      for (int h = 0; h < kFRep; ++h) {
        float4* dst = reinterpret_cast<float4*>(wres + h * kFD + vcn * 8);
        dst[0] = make_float4(acc[h][0], acc[h][1], acc[h][2], acc[h][3]);
        dst[1] = make_float4(acc[h][4], acc[h][5], acc[h][6], acc[h][7]);
      }
    }
    if (lane < kFRep) s.wml[wave][lane] = make_float2(m_run, l_run);  // lane h holds head h
    __syncthreads();
    {
      // thread: head h = tid / 64, dims 2 (tid % 64), +1
      const int h = tid >> 6, d = 2 * lane;
      float M = -__builtin_inff();
#pragma unroll
      for (int w = 0; w < 4; ++w) M = fmaxf(M, s.wml[w][h].x);
      float L = 0.f, a0 = 0.f, a1 = 0.f;
#pragma unroll
      for (int w = 0; w < 4; ++w) {
        const float2 v = s.wml[w][h];
        const float wt = v.x == -__builtin_inff() ? 0.f : exp2f(v.x - M);
        const float2 x = *reinterpret_cast<const float2*>(
            reinterpret_cast<const float*>(s.acc[w]) + h * kFD + d);
        L += v.y * wt;
        a0 += x.x * wt;
        a1 += x.y * wt;
      }
      const int qh = kvh * kFRep + h;
      if (np == 1) {
        const float inv = L > 0.f ? 1.f / L : 0.f;
        reinterpret_cast<uint32_t*>(out + ((int64_t)tok * H + qh) * kFD)[lane] =
            (uint32_t)f32_to_bf16(a0 * inv) | ((uint32_t)f32_to_bf16(a1 * inv) << 16);
      } else {
        const int64_t prow = (int64_t)split_base[i] + (int64_t)qh * np + part;
        __hip_atomic_store(reinterpret_cast<uint64_t*>(po + prow * kFD + d), pack2(a0, a1),
                           __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        if (lane == 0)
          __hip_atomic_store(reinterpret_cast<uint64_t*>(ml + prow), pack2(M, L), __ATOMIC_RELAXED,
                             __HIP_MEMORY_SCOPE_AGENT);
        asm volatile("s_waitcnt vmcnt(0)" ::: "memory");  // the stores have completed
      }
    }
    if (np > 1) {  // uniform over the workgroup
      __syncthreads();  // every thread's partial stores have completed
      if (tid == 0) {
        int32_t* cnt = reinterpret_cast<int32_t*>(ml + split_base[i] + (int64_t)H * np + kvh);
        const int prev = __hip_atomic_fetch_add(cnt, 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        s.last = prev == np - 1;
        if (prev == np - 1) __hip_atomic_store(cnt, 0, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
      }
      __syncthreads();
      if (s.last) {
        asm volatile("" ::: "memory");  // no load below moves above the arrival
        const int h = tid >> 6, d = 2 * lane;
        const int qh = kvh * kFRep + h;
        const int64_t r0 = (int64_t)split_base[i] + (int64_t)qh * np;
        const float2 o = merge_partitions(
            reinterpret_cast<const uint64_t*>(ml + r0),
            reinterpret_cast<const uint64_t*>(po + r0 * kFD + d), kFD / 2, np, lane);
        reinterpret_cast<uint32_t*>(out + ((int64_t)tok * H + qh) * kFD)[lane] =
            (uint32_t)f32_to_bf16(o.x) | ((uint32_t)f32_to_bf16(o.y) << 16);
      }
    }
  }
}

__global__ void __launch_bounds__(256) attend_decode_bf16_kernel(
    VL_ATTN_PARAMS(uint16_t), const int32_t* __restrict__ hdr, int32_t* work) {
  __shared__ DecodeLds s;
  __shared__ int next_lds;
  const int n_items = hdr[0];
  const int R = hdr[7];
  const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
  // Persistent workgroups (as many as fit on the chip): the first item is
  // blockIdx.x, later ones are claimed from the work counter, the next one at
  // the start of the current item so that the atomic's latency is hidden.
  // The counter is zeroed by the plan and, after each run, by the last
  // workgroup to leave.
  int it = blockIdx.x;
  while (it < n_items) {
    int nxt = 0;
    if (threadIdx.x == 0)
      nxt = claimed_item((int64_t)gridDim.x + atomicAdd(work, 1), 1, 0, n_items);
    decode_body<false, kBK, kBV>(
        s, it, decode_fetch(desc[it / Hkv], it, R, Hkv, wave, lane, query, q_stride, bt, bt_stride),
        R, VL_ATTN_ARGS);
    if (threadIdx.x == 0) next_lds = nxt;
    __syncthreads();  // the merge has read every wavefront's LDS; next_lds is set
    it = next_lds;
  }
  leave_and_reset(work, 1);
}

// --------------------------------------------------------- short decode --

// Decode batches of short sequences (every sequence at most one query and at
// most kShortCtx tokens) for head dims up to 64: one workgroup of NW
// wavefronts per (sequence, KV head) takes the whole context, so the call
// needs no plan, no context split and no merge launch. The sequence's block
// table is staged in LDS first, so that the K and V loads of a 64 NW-key
// chunk (wavefront w takes keys 64 (NW t + w) + lane of chunk t) are issued
// together; with 8 wavefronts a context of up to 512 keys is one chunk, one
// round trip to memory:
//   QK: lane l holds key l of its wavefront's 64, its K row in registers,
//       and the dot products with the REP query heads (LDS broadcast reads);
//   softmax: per head, the wavefront max by DPP row operations (no LDS
//       round trips), merged online across chunks; each lane keeps the sum of
//       its own keys' weights until the end; the weights go to the
//       wavefront's LDS row;
//   PV: lane l = g NC + c (NC 16-byte chunks per head row, G = 64 / NC key
//       groups) sums chunk c over keys g, g + G, ... of the chunk, its V
//       chunks loaded with the K row.
// At the end each wavefront sums its key groups through its own LDS rows;
// after one workgroup barrier, thread (head, dim) merges the wavefronts
// (max-rescaled) and writes that element once. Keys past the context re-read
// the last key (finite values) and get weight 0.
constexpr int kShortCtx = 2048;
constexpr int kShortWaves = 8;  // wavefronts per short-decode workgroup

template <typename TKV, int D, int REP, int NW>
struct ShortLds {
  static constexpr int kVE = 16 / (int)sizeof(TKV);  // cache elements per 16-byte load
  static constexpr int kNC = D / kVE;                 // 16-byte chunks per head row
  // K rows staged key-major, a row padded to an odd number of 16-byte chunks
  // (the 64 lanes' reads of their own rows then meet no bank conflicts),
  // where the wavefronts' rows fit beside the rest (all but fp32 head_dim 64)
  static constexpr int kNCP = kNC + 1 + (kNC & 1);
  static constexpr bool kStageK = (size_t)NW * 64 * kNCP * 16 <= 110 * 1024;
  float q[REP][D];          // query heads, pre-scaled to the log2 domain
  float p[NW][REP][64];     // per wavefront: the chunk's weights
  float red[NW][64][kVE];   // per wavefront and lane: one head's PV sums
  float m[NW][REP], l[NW][REP];
  int32_t tbl[kShortCtx];   // the sequence's block ids
  uint4 k[kStageK ? NW : 1][kStageK ? 64 : 1][kStageK ? kNCP : 1];  // per wavefront: its keys' K rows
  float o[REP * D];         // with wo: the workgroup's merged output rows
};




// A head row of D elements of T as floats (16-byte loads).
template <typename T, int D>
__device__ __forceinline__ void load_row(const T* p, float (&r)[D]) {
  constexpr int VE = 16 / (int)sizeof(T);
#pragma unroll
  for (int c = 0; c < D / VE; ++c) {
    const uint4 v = reinterpret_cast<const uint4*>(p)[c];
    widen16<T>(v, r + VE * c);
  }
}

// T: query and output elements, TKV: cache elements; NW wavefronts.
// With wo (fp32 T only): instead of its REP output rows the workgroup writes
// parts[i, g, :] = (its REP x D outputs, as one row) @ wo[g REP D .. (g + 1)
// REP D, 0 .. wo_n) (row-major, wo_n columns): the output projection of
// vllmlite/model.py:114 split by KV head, whose wo_n-wide partial rows the
// next projection adds to its input in KV-head order. Thread t < wo_n takes
// column t; its REP D weights are loaded when the key chunks are done, so
// they arrive during the merge of the wavefronts.
template <typename T, typename TKV, int D, int REP, int NW>
__global__ void __launch_bounds__(64 * NW) attend_short_decode_kernel(
    T* __restrict__ out, const T* __restrict__ query, int64_t q_stride, const TKV* kc,
    const TKV* vc, const int32_t* __restrict__ bt, int bt_stride,
    const int32_t* __restrict__ seq_lens, const int32_t* __restrict__ qsl, int Hkv, int bs_log2,
    int kv_hm, float scale_log2, const float* __restrict__ wo, int wo_n,
    float* __restrict__ parts, int n_items, int ncg) {
  using Lds = ShortLds<TKV, D, REP, NW>;
  constexpr int VE = Lds::kVE;
  constexpr int kThreads = 64 * NW;
  static_assert(D % VE == 0 && D <= 64, "head_dim");
  constexpr int NC = D / VE;               // 16-byte chunks per head row
  constexpr int G = 64 / NC;               // PV key groups
  constexpr int KPL = (64 + G - 1) / G;    // keys per lane in the PV product
  __shared__ Lds s;
  // item (sequence i, KV head g); with wo split over ncg column groups, the
  // ncg workgroups of an item are b = 8 (ncg (item / 8) + cg) + item % 8, so
  // they run on one XCD (workgroups go to the XCDs round-robin) and its L2
  // serves the three that read the item's K/V after the first
  int item = blockIdx.x, cg = 0;
  if (ncg > 1) {
    const int r = blockIdx.x >> 3;
    item = (r / ncg) * 8 + (blockIdx.x & 7);
    cg = r - (r / ncg) * ncg;
  }
  if (item >= n_items) return;  // the grid's rounding to whole groups of 8 items
  const int i = item / Hkv, g = item - (item / Hkv) * Hkv;
  const int tid = threadIdx.x, wave = tid >> 6, lane = tid & 63;
  // the first kThreads entries of the sequence's block-table row (it has
  // bt_stride of them) are loaded with its length, not after it
  const int32_t* table = bt + (int64_t)i * bt_stride;
  const int32_t tbl0 = tid < bt_stride ? table[tid] : 0;
  const int c = seq_lens[i];
  // a sequence without exactly one query, or longer than the staged table,
  // is not this kernel's (the bounds the caller stated do not hold)
  if (qsl[i + 1] - qsl[i] != 1 || c <= 0 || c > kShortCtx) return;
  const int tok = qsl[i];
  const int bs_mask = (1 << bs_log2) - 1;
  const int nblk = (c + bs_mask) >> bs_log2;
  if (tid < nblk) s.tbl[tid] = tbl0;
  for (int b = tid + kThreads; b < nblk; b += kThreads) s.tbl[b] = table[b];
  for (int e = tid; e < REP * D; e += kThreads) {
    const int h = e / D, d = e - (e / D) * D;
    s.q[h][d] = Elem<T>::load(query, (int64_t)tok * q_stride + (int64_t)(g * REP + h) * D + d) *
                scale_log2;
  }
  __syncthreads();
  // row of key k of KV head g: block * blk + offset * row + g * head
  // (token-major: row Hkv * D, head D; head-major: row D, head bs * D)
  const int64_t blk = (int64_t)Hkv * D << bs_log2;
  const int64_t row = kv_hm ? D : (int64_t)Hkv * D;
  const TKV* kg = kc + (int64_t)g * (kv_hm ? (int64_t)D << bs_log2 : D);
  const TKV* vg = vc + (kg - kc);
  auto row_of = [&](int k) { return s.tbl[k >> bs_log2] * blk + (k & bs_mask) * row; };
  const int pg = lane / NC, pc = lane - (lane / NC) * NC;  // PV: key group, chunk
  float m[REP], lsum[REP], acc[REP][VE];
#pragma unroll
  for (int h = 0; h < REP; ++h) {
    m[h] = -__builtin_inff(), lsum[h] = 0.f;
#pragma unroll
    for (int e = 0; e < VE; ++e) acc[h][e] = 0.f;
  }
  const int nchunk = (c + kThreads - 1) / kThreads;
  for (int t = 0; t < nchunk; ++t) {
    const int base = (NW * t + wave) * 64;
    if (base >= c) break;  // wavefront-uniform; later chunks start later still
    // every load of the chunk first. K and V alike: lane (pg, pc) loads
    // 16-byte chunk pc of keys pg + G j, so each load instruction reads G
    // whole rows (a lane per key reads one chunk of 64 rows, 64 cache lines,
    // per instruction: the address work of those loads set the kernel's time)
    uint4 kraw[Lds::kStageK ? KPL : 1], vraw[KPL];
#pragma unroll
    for (int j = 0; j < KPL; ++j) {
      const int kk = min(pg + G * j, 63);  // past the chunk (or lanes past G NC): weight 0
      const int64_t ro = row_of(min(base + kk, c - 1)) + pc * VE;
      if constexpr (Lds::kStageK) kraw[j] = *reinterpret_cast<const uint4*>(kg + ro);
      vraw[j] = *reinterpret_cast<const uint4*>(vg + ro);
    }
    // the lane's key row: through the wavefront's LDS rows, or (fp32 head_dim
    // 64, whose rows do not fit) straight from the cache
    float kr[D];
    if constexpr (Lds::kStageK) {
#pragma unroll
      for (int j = 0; j < KPL; ++j) {
        const int kk = pg + G * j;
        if (pg < G && kk < 64) s.k[wave][kk][pc] = kraw[j];
      }
      __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
      __builtin_amdgcn_wave_barrier();
      __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
#pragma unroll
      for (int cc = 0; cc < NC; ++cc) widen16<TKV>(s.k[wave][lane][cc], kr + VE * cc);
    } else {
      load_row<TKV, D>(kg + row_of(min(base + lane, c - 1)), kr);
    }
    const bool valid = base + lane < c;
#pragma unroll
    for (int h = 0; h < REP; ++h) {
      float a = 0.f;
#pragma unroll
      for (int d = 0; d < D; ++d) a = __builtin_fmaf(s.q[h][d], kr[d], a);
      const float sc = valid ? a : -__builtin_inff();
      const float mn = fmaxf(m[h], wave_max_dpp(sc));  // finite: key base is valid
      const float alpha = exp2_fast(m[h] - mn);
      const float p = exp2_fast(sc - mn);
      lsum[h] = __builtin_fmaf(lsum[h], alpha, p);
#pragma unroll
      for (int e = 0; e < VE; ++e) acc[h][e] *= alpha;
      m[h] = mn;
      s.p[wave][h][lane] = p;
    }
    // the weights the wavefront's other lanes wrote above
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
    __builtin_amdgcn_wave_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
#pragma unroll
    for (int j = 0; j < KPL; ++j) {
      const int kk = pg + G * j;
      float v[VE];
      widen16<TKV>(vraw[j], v);
#pragma unroll
      for (int h = 0; h < REP; ++h) {
        const float w = kk < 64 ? s.p[wave][h][kk] : 0.f;
#pragma unroll
        for (int e = 0; e < VE; ++e) acc[h][e] = __builtin_fmaf(w, v[e], acc[h][e]);
      }
    }
    // the weights have been read before the next chunk overwrites them
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
    __builtin_amdgcn_wave_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
  }
  // with wo: the weights of this thread's products, in flight during the
  // merge below. Column sums are ((S0 + S1) + S2) + S3 over the quarters k =
  // KQ q .. KQ (q + 1) - 1 of the REP D rows, each S_q one chain in k order,
  // however the columns are split: with one column group, thread t < wo_n
  // takes column t whole; with ncg groups of cols = wo_n / ncg, thread t <
  // 4 cols takes quarter t / cols of column cg cols + t % cols.
  constexpr int KQ = REP * D / 4;
  static_assert(REP * D % 4 == 0, "whole quarters");
  float wcol[REP * D];
  const int cols = wo_n / ncg;
  const int wq = ncg > 1 ? tid / max(cols, 1) : 0;  // the thread's quarter (split columns)
  const int wc_col = ncg > 1 ? cg * cols + (tid - wq * cols) : tid;
  const bool wo_col = wo != nullptr && (ncg > 1 ? tid < 4 * cols : tid < wo_n);
  if (wo_col) {
    const float* wc = wo + (int64_t)g * REP * D * wo_n + wc_col;
    if (ncg > 1) {
#pragma unroll
      for (int k = 0; k < KQ; ++k) wcol[k] = wc[(int64_t)(wq * KQ + k) * wo_n];
    } else {
#pragma unroll
      for (int k = 0; k < REP * D; ++k) wcol[k] = wc[(int64_t)k * wo_n];
    }
  }
#pragma unroll
  for (int h = 0; h < REP; ++h) lsum[h] = wave_sum_dpp(lsum[h]);
  if (lane == 0) {
#pragma unroll
    for (int h = 0; h < REP; ++h) s.m[wave][h] = m[h], s.l[wave][h] = lsum[h];
  }
  // each wavefront sums its key groups, one head at a time through its own
  // LDS rows (no workgroup barrier): lane d < D adds dim d over the groups in
  // order into the wavefront's weight row of head h, free after the loop
#pragma unroll
  for (int h = 0; h < REP; ++h) {
#pragma unroll
    for (int e = 0; e < VE; ++e) s.red[wave][lane][e] = acc[h][e];
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
    __builtin_amdgcn_wave_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
    if (lane < D) {
      const int dc = lane / VE, de = lane - (lane / VE) * VE;
      float sw = 0.f;
#pragma unroll
      for (int gg = 0; gg < G; ++gg) sw += s.red[wave][gg * NC + dc][de];
      s.p[wave][h][lane] = sw;
    }
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
    __builtin_amdgcn_wave_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
  }
  __syncthreads();
  // thread (h, d) merges the wavefronts' sums, max-rescaled, in wavefront order
  const int H = Hkv * REP;
  for (int e = tid; e < REP * D; e += kThreads) {
    const int h = e / D, d = e - (e / D) * D;
    float M = -__builtin_inff();
#pragma unroll
    for (int w = 0; w < NW; ++w) M = fmaxf(M, s.m[w][h]);
    float L = 0.f, a = 0.f;
#pragma unroll
    for (int w = 0; w < NW; ++w) {
      const float mw = s.m[w][h];
      if (mw == -__builtin_inff()) continue;
      const float wt = exp2_fast(mw - M);
      L = __builtin_fmaf(s.l[w][h], wt, L);
      a = __builtin_fmaf(s.p[w][h][d], wt, a);
    }
    const float o = L > 0.f ? a * (1.f / L) : 0.f;
    if (wo)
      s.o[e] = o;
    else
      Elem<T>::store(out, ((int64_t)tok * H + g * REP + h) * D + d, o);
  }
  if (wo) {
    __syncthreads();
    float* prow = parts + ((int64_t)i * Hkv + g) * wo_n;
    if (ncg == 1) {
      if (wo_col) {
        float sq[4] = {0.f, 0.f, 0.f, 0.f};  // four independent chains
#pragma unroll
        for (int k = 0; k < REP * D; ++k)
          sq[k / KQ] = __builtin_fmaf(s.o[k], wcol[k], sq[k / KQ]);
        prow[tid] = ((sq[0] + sq[1]) + sq[2]) + sq[3];
      }
    } else {
      // the quarters meet in LDS (the PV sums' rows, free since the merge)
      float* sq = reinterpret_cast<float*>(s.red);
      if (wo_col) {
        float a = 0.f;
#pragma unroll
        for (int k = 0; k < KQ; ++k) a = __builtin_fmaf(s.o[wq * KQ + k], wcol[k], a);
        sq[tid] = a;  // = sq[wq cols + column]
      }
      __syncthreads();
      if (tid < cols)
        prow[cg * cols + tid] =
            ((sq[tid] + sq[cols + tid]) + sq[2 * cols + tid]) + sq[3 * cols + tid];
    }
  }
}

// ------------------------------------------------------------------ step --

// One launch for a whole batch of the bandwidth-kernel shape (bf16, head_dim
// 128, 4 query heads per KV head, 16-token blocks): decode items and MFMA
// tile items (32-row, then 16-row), each kind from its own queues. Tile
// items are dealt to 8 queues by item % 8 and a workgroup drains the queue of
// its XCD (workgroups are dispatched round-robin over the 8 XCDs, so
// blockIdx % 8 names it) before it helps the others: consecutive tile items
// are the KV heads of one row block, so each XCD's L2 holds the K/V of its
// own KV heads, which the other row blocks of the sequence read again. Half
// of the persistent workgroups start on the tile queues and half on the
// decode queue, so the compute units hold MFMA-bound and HBM-bound work at
// the same time; a workgroup whose queues have run dry moves to the others.
// The two item kinds share the LDS allocation. counters: [0] decode queue,
// [1 + x] tile queue x, [9] workgroups finished.
constexpr size_t kStepLds = std::max({sizeof(TileLds<uint16_t, kFD, 32>),
                                      sizeof(TileLds<uint16_t, kFD, 16>), sizeof(DecodeLds)});
constexpr int kStepTileFirst = 2;  // one in this many workgroups starts on the tile queues

__global__ void __launch_bounds__(256) __attribute__((amdgpu_waves_per_eu(2)))
attend_step_bf16_kernel(VL_ATTN_PARAMS(uint16_t), const int32_t* __restrict__ hdr,
                        const int32_t* __restrict__ wide_off, const int32_t* __restrict__ wide_seq,
                        const int32_t* __restrict__ tile_off, const int32_t* __restrict__ tail_seq,
                        int32_t* counters, int always) {
  __shared__ __align__(16) unsigned char smem[kStepLds];
  __shared__ int claim_lds;
  auto& tl32 = *reinterpret_cast<TileLds<uint16_t, kFD, 32>*>(smem);
  auto& tl16 = *reinterpret_cast<TileLds<uint16_t, kFD, 16>*>(smem);
  auto& dl = *reinterpret_cast<DecodeLds*>(smem);
  if (!always && !hdr[11]) return;  // not a mixed batch: the decode and tile kernels run it
  const int P = hdr[2];
  // the kWideRows-row items as two items each (pass 0 of every item, then
  // pass 1: with 8 KV heads n_wide is a multiple of 8, so both passes of an
  // item fall in its KV head's queue), then the 16-row items
  const int n_wide = hdr[10], n_tiles = 2 * n_wide + hdr[4], n_dec = hdr[0];
  const int R = hdr[7];
  const int xcd = blockIdx.x % kXcds;
  const bool tiles_first = (blockIdx.x / kXcds) % kStepTileFirst == 0;
  for (int v = 0; v <= kXcds; ++v) {  // the decode queue and the 8 tile queues, in turn
    const int qid = tiles_first ? (v < kXcds ? 1 + (xcd + v) % kXcds : 0)
                                : (v == 0 ? 0 : 1 + (xcd + v - 1) % kXcds);
    const bool tiles = qid != 0;
    const int stride = tiles ? kXcds : 1, base = tiles ? qid - 1 : 0;
    const int n = tiles ? n_tiles : n_dec;
    __syncthreads();  // every thread has read the previous queue's last claim
    if (threadIdx.x == 0) {
      // a queue seen empty is skipped without an atomic; one thread decides,
      // so the whole workgroup takes the same branch around the barriers
      const int seen = __hip_atomic_load(counters + qid, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
      claim_lds = claimed_item(seen, stride, base, n) >= n
                      ? -1
                      : claimed_item(atomicAdd(counters + qid, 1), stride, base, n);
    }
    __syncthreads();
    if (claim_lds < 0) continue;
    int it = claim_lds;
    while (it < n) {
      int nxt = 0;
      if (threadIdx.x == 0)  // the next item, claimed early
        nxt = claimed_item(atomicAdd(counters + qid, 1), stride, base, n);
      if (!tiles)
        decode_body<true, kStepBK, kStepBV>(dl, it,
                          decode_fetch(desc[it / Hkv], it, R, Hkv, threadIdx.x >> 6,
                                       threadIdx.x & 63, query, q_stride, bt, bt_stride),
                          R, VL_ATTN_ARGS);
      else if (it < 2 * n_wide)
        tile_body<uint16_t, kFD, 32, true>(tl32, it % n_wide, it / n_wide, P, wide_off, wide_seq,
                                           VL_ATTN_ARGS);
      else
        tile_body<uint16_t, kFD, 16, true>(tl16, it - 2 * n_wide, 0, P, tile_off, tail_seq,
                                           VL_ATTN_ARGS);
      __syncthreads();  // the item is done with the LDS; claim_lds has been read
      if (threadIdx.x == 0) claim_lds = nxt;
      __syncthreads();
      it = claim_lds;
    }
  }
  leave_and_reset(counters, kXcds + 1);
}

// --------------------------------------------------------------- combine --

// Merges the partitions of the split multi-query sequences (listed by the
// plan): one workgroup per (sequence, query head) item, wavefront w takes the
// sequence's query tokens w, w + 4, .... Lane p holds partition p's (max,
// sum) and weight (64 partitions at a time); the output dims lane + 64k are
// then summed over the partitions with the weights read lane by lane, so the
// partial loads are independent of each other.
constexpr int kCombineFew = 8;  // partitions whose loads a combine row issues at once

template <typename T>
__global__ void __launch_bounds__(256) combine_kernel(
    T* __restrict__ out, const int32_t* __restrict__ qsl, int H, int D,
    const int32_t* __restrict__ hdr, const int32_t* __restrict__ cmb_seq,
    const int32_t* __restrict__ nparts, const int32_t* __restrict__ split_base,
    const float2* __restrict__ ml, const float* __restrict__ po) {
  constexpr int kDk = kMaxHeadDim / 64;
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int64_t items = (int64_t)hdr[12] * H;
  for (int64_t item = blockIdx.x; item < items; item += gridDim.x) {
    const int k = (int)(item / H), h = (int)(item - (item / H) * H);
    const int i = cmb_seq[k];
    const int np = nparts[i];
    const int q = qsl[i + 1] - qsl[i];
    for (int j = wave; j < q; j += 4) {
      const int64_t row0 = (int64_t)split_base[i] + (int64_t)(j * H + h) * np;
      if (np <= kCombineFew) {
        // every load of the row issued at once (the partials do not depend on
        // the maximum); the arithmetic is the general loop's below, in the
        // same order, so the output has the same bits
        const float2 v = ml[row0 + min(lane, np - 1)];
        float xs[kCombineFew][kDk];
#pragma unroll
        for (int u = 0; u < kCombineFew; ++u)
#pragma unroll
          for (int e = 0; e < kDk; ++e)
            xs[u][e] = po[(row0 + min(u, np - 1)) * D + min(lane + 64 * e, D - 1)];
        float M = lane < np ? v.x : -__builtin_inff();
#pragma unroll
        for (int o = 32; o > 0; o >>= 1) M = fmaxf(M, __shfl_xor(M, o, 64));
        float L = 0.f, w = 0.f, acc[kDk];
#pragma unroll
        for (int e = 0; e < kDk; ++e) acc[e] = 0.f;
        if (lane < np) {
          w = v.x == -__builtin_inff() ? 0.f : exp2_fast(v.x - M);
          L += v.y * w;
        }
        auto wt = [&](int u) {
          return __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, w), u));
        };
#pragma unroll
        for (int u = 0; u + 4 <= kCombineFew; u += 4) {
          if (u + 4 > np) break;  // uniform
#pragma unroll
          for (int e = 0; e < kDk; ++e)
            if (lane + 64 * e < D)
              acc[e] += xs[u][e] * wt(u) + xs[u + 1][e] * wt(u + 1) + xs[u + 2][e] * wt(u + 2) +
                        xs[u + 3][e] * wt(u + 3);
        }
#pragma unroll
        for (int u = 0; u < kCombineFew; ++u) {
          if (u < (np & ~3) || u >= np) continue;  // uniform
#pragma unroll
          for (int e = 0; e < kDk; ++e)
            if (lane + 64 * e < D) acc[e] += xs[u][e] * wt(u);
        }
#pragma unroll
        for (int o = 32; o > 0; o >>= 1) L += __shfl_xor(L, o, 64);
        const float inv = L > 0.f ? 1.f / L : 0.f;
        T* dst = out + ((int64_t)(qsl[i] + j) * H + h) * D;
#pragma unroll
        for (int e = 0; e < kDk; ++e)
          if (lane + 64 * e < D) Elem<T>::store(dst, lane + 64 * e, acc[e] * inv);
        continue;
      }
      float M = -__builtin_inff();
      for (int p = lane; p < np; p += 64) M = fmaxf(M, ml[row0 + p].x);
#pragma unroll
      for (int o = 32; o > 0; o >>= 1) M = fmaxf(M, __shfl_xor(M, o, 64));
      float L = 0.f, acc[kDk];
#pragma unroll
      for (int e = 0; e < kDk; ++e) acc[e] = 0.f;
      for (int p0 = 0; p0 < np; p0 += 64) {
        float w = 0.f;
        if (p0 + lane < np) {
          const float2 v = ml[row0 + p0 + lane];
          w = v.x == -__builtin_inff() ? 0.f : exp2_fast(v.x - M);
          L += v.y * w;
        }
        const int cnt = min(64, np - p0);
        const float* src = po + (row0 + p0) * D;
        auto wt = [&](int u) {
          return __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, w), u));
        };
        int u = 0;
        for (; u + 4 <= cnt; u += 4) {  // four partitions' loads in flight
#pragma unroll
          for (int e = 0; e < kDk; ++e) {
            if (lane + 64 * e >= D) continue;
            const float* x = src + (int64_t)u * D + lane + 64 * e;
            const float x0 = x[0], x1 = x[D], x2 = x[2 * D], x3 = x[3 * D];
            acc[e] += x0 * wt(u) + x1 * wt(u + 1) + x2 * wt(u + 2) + x3 * wt(u + 3);
          }
        }
        for (; u < cnt; ++u)
#pragma unroll
          for (int e = 0; e < kDk; ++e)
            if (lane + 64 * e < D) acc[e] += src[(int64_t)u * D + lane + 64 * e] * wt(u);
      }
#pragma unroll
      for (int o = 32; o > 0; o >>= 1) L += __shfl_xor(L, o, 64);
      const float inv = L > 0.f ? 1.f / L : 0.f;
      T* dst = out + ((int64_t)(qsl[i] + j) * H + h) * D;
#pragma unroll
      for (int e = 0; e < kDk; ++e)
        if (lane + 64 * e < D) Elem<T>::store(dst, lane + 64 * e, acc[e] * inv);
    }
  }
}

struct Args {
  void* out;
  const void* query;
  int64_t q_stride;
  const void* kc;
  const void* vc;
  const int32_t* bt;
  int bt_stride;
  const int32_t* seq_lens;
  const int32_t* qsl;
  int S, T, H, Hkv, D, bs;
  float scale;
  int dtype;
  int kv_layout;
};

int check_args(const Args& a, const void* ws, size_t ws_bytes, bool need_kv) {
  VL_CHECK_ARG(a.dtype == VL_DTYPE_F32 || a.dtype == VL_DTYPE_BF16 ||
                   a.dtype == VL_DTYPE_F32_BF16KV || a.dtype == VL_DTYPE_F32_FP8KV,
               "bad dtype %d", a.dtype);
  VL_CHECK_ARG(a.S >= 0 && a.T >= 0, "bad batch size");
  VL_CHECK_ARG(a.H > 0 && a.Hkv > 0 && a.H % a.Hkv == 0,
               "num_heads must be a positive multiple of num_kv_heads");
  VL_CHECK_ARG(a.D > 0 && a.D <= kMaxHeadDim, "head_dim must be in 1..%d", kMaxHeadDim);
  VL_CHECK_ARG(a.bs > 0 && a.bt_stride >= 0, "bad block table");
  if (need_kv) VL_CHECK_ARG(a.q_stride >= (int64_t)a.H * a.D, "query row stride too small");
  if (a.S == 0 || a.T == 0) return VL_OK;
  VL_CHECK_ARG(a.seq_lens && a.qsl && ws, "null pointer");
  if (need_kv)
    VL_CHECK_ARG(a.out && a.query && a.kc && a.vc && a.bt, "null pointer");
  VL_CHECK_ARG(ws_bytes >= fixed_bytes(a.S), "workspace too small: %zu < %zu", ws_bytes,
               fixed_bytes(a.S));
  VL_CHECK_ARG(((uintptr_t)ws & 255) == 0, "workspace must be 256-byte aligned");
  return VL_OK;
}

// Workgroups of the bandwidth kernel that are resident at once on the
// current device (its grid is persistent), cached per device.
int decode_grid() {
  static int cached[64] = {0};
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 64) dev = 0;
  if (!cached[dev]) {
    int per_cu = 0;
    if (hipOccupancyMaxActiveBlocksPerMultiprocessor(&per_cu, attend_decode_bf16_kernel, 256, 0) !=
            hipSuccess ||
        per_cu <= 0)
      per_cu = 2;
    // at most 2 per compute unit: 3 fit (157 VGPRs, 52 KB of LDS) but
    // measured 225-230 us against 215-221 us for the 256-sequence batch (the
    // plan then also cuts the contexts into more, shorter ranges)
    cached[dev] = std::min(per_cu, 2) * vl_num_cus();
  }
  return cached[dev];
}

int step_grid() {
  static int cached[64] = {0};
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 64) dev = 0;
  if (!cached[dev]) {
    int per_cu = 0;
    if (hipOccupancyMaxActiveBlocksPerMultiprocessor(&per_cu, attend_step_bf16_kernel, 256, 0) !=
            hipSuccess ||
        per_cu <= 0)
      per_cu = 2;
    cached[dev] = per_cu * vl_num_cus();
  }
  return cached[dev];
}

// The tile items the plan aims for are kTileItemsPerWg per this many
// workgroups.
int tile_grid() { return vl_num_cus() * 4; }

int do_plan(const Args& a, void* ws, size_t ws_bytes, hipStream_t st) {
  const Layout L = make_layout(ws, ws_bytes, a.S, a.D);
  const bool fast = fast_shape(a.dtype, a.H, a.Hkv, a.D, a.bs);
  const bool tile = tile_shape(a.dtype, a.D, a.bs);
  // a few bandwidth-kernel items per resident workgroup
  const int target_items = fast ? kItemsPerWg * decode_grid() : 0;
  const int tile_target = kTileItemsPerWg * tile_grid();
  const bool wide = tile && a.dtype == VL_DTYPE_BF16;
  auto* plan = a.S <= kPlanThreads * kPlanRegSeqs ? plan_kernel<true> : plan_kernel<false>;
  plan<<<1, kPlanThreads, 0, st>>>(a.seq_lens, a.qsl, a.S, a.H, a.Hkv, fast, tile, wide,
                                   L.cap_rows, target_items, tile_target, L.hdr, L.gen_off,
                                   L.tile_off, L.nparts, L.split_base, L.wide_off, L.cmb_seq,
                                   L.wide_seq, L.tail_seq, L.tail_off, L.desc, L.ml);
  VL_CHECK_LAUNCH();
  return VL_OK;
}

// The VL_ATTN_PARAMS arguments of a launch (inside do_run / launch_tile_d).
#define VL_ATTN_LAUNCH_ARGS(T) VL_ATTN_LAUNCH_ARGS_KV(T, T)
#define VL_ATTN_LAUNCH_ARGS_KV(T, TKV)                                                          \
  (T*)a.out, (const T*)a.query, a.q_stride, (const TKV*)a.kc, (const TKV*)a.vc, a.bt,          \
      a.bt_stride,                                                                              \
      a.seq_lens, a.qsl, a.S, a.H, a.Hkv, __builtin_ctz(a.bs),                                 \
      a.kv_layout == VL_KV_HEAD_MAJOR ? 1 : 0, sl2, L.desc, L.nparts, L.split_base, L.ml, L.po

// Workgroups of a tile kernel that are resident at once on the current device
// (its grid is persistent), cached per device and instantiation.
template <typename T, int D, int RW, int kWv, typename TKV = T>
int tile_launch_grid() {
  static int cached[64] = {0};
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 64) dev = 0;
  if (!cached[dev]) {
    int per_cu = 0;
    if (hipOccupancyMaxActiveBlocksPerMultiprocessor(&per_cu, attend_tile_kernel<T, D, RW, kWv, TKV>,
                                                     64 * kWv, 0) != hipSuccess ||
        per_cu <= 0)
      per_cu = 2;
    // at most 4 per compute unit: more only add workgroups that find no item
    // in small batches
    cached[dev] = std::min(per_cu, 4) * vl_num_cus();
  }
  return cached[dev];
}

// 32-row items (kWideRows rows) by 8-wavefront workgroups: every staged K/V
// tile serves 256 rows (prefill chunks 278-300 -> 256-274 us against 4
// wavefronts); 16-row items by 4.
template <typename T, int D, int RW, typename TKV = T>
int launch_tile_d(const Args& a, const Layout& L, float sl2, hipStream_t st) {
  constexpr int kWv = RW == 32 ? 8 : 4;
  attend_tile_kernel<T, D, RW, kWv, TKV><<<tile_launch_grid<T, D, RW, kWv, TKV>(), 64 * kWv, 0,
                                           st>>>(
      VL_ATTN_LAUNCH_ARGS_KV(T, TKV), L.hdr, RW == 32 ? L.wide_off : L.tile_off,
      RW == 32 ? L.wide_seq : L.tail_seq, L.hdr + (RW == 32 ? 34 : 26));
  VL_CHECK_LAUNCH();
  return VL_OK;
}

// The 16-row tile kernel always (short-query and fp32 items); for bf16 also
// the 32-row kernel when a sequence may have more than kSplitMaxQ queries.
template <typename T, typename TKV = T>
int launch_tile(const Args& a, const Layout& L, float sl2, int max_q, hipStream_t st) {
  const bool wide = sizeof(T) == 2 && (max_q <= 0 || max_q > kSplitMaxQ);
  int rc = VL_OK;
  if constexpr (sizeof(T) == 2) {
    switch (a.D) {
      case 64:
        rc = launch_tile_d<T, 64, 16>(a, L, sl2, st);
        if (!rc && wide) rc = launch_tile_d<T, 64, 32>(a, L, sl2, st);
        return rc;
      case 128:
        rc = launch_tile_d<T, 128, 16>(a, L, sl2, st);
        if (!rc && wide) rc = launch_tile_d<T, 128, 32>(a, L, sl2, st);
        return rc;
    }
  } else {
    switch (a.D) {
      case 16: return launch_tile_d<T, 16, 16, TKV>(a, L, sl2, st);
      case 32: return launch_tile_d<T, 32, 16, TKV>(a, L, sl2, st);
      case 48: return launch_tile_d<T, 48, 16, TKV>(a, L, sl2, st);
      case 64: return launch_tile_d<T, 64, 16, TKV>(a, L, sl2, st);
      case 128: return launch_tile_d<T, 128, 16, TKV>(a, L, sl2, st);
    }
  }
  VL_CHECK_ARG(false, "no tile kernel for head_dim %d", a.D);
  return VL_EINVAL;
}

// Whether a call takes the short-decode kernel: every sequence a decode
// (max_q 1) of at most kShortCtx tokens (max_ctx), a power-of-two block size,
// head_dim 16 / 32 / 48 / 64 and 1, 2, 4 or 8 query heads per KV head.
inline bool short_decode(const Args& a, int max_q, int max_ctx) {
  if (a.Hkv <= 0 || a.H <= 0 || a.H % a.Hkv != 0) return false;
  const int rep = a.H / a.Hkv;
  return max_q == 1 && max_ctx > 0 && max_ctx <= kShortCtx && a.bs > 0 &&
         (a.bs & (a.bs - 1)) == 0 && (a.D == 16 || a.D == 32 || a.D == 48 || a.D == 64) &&
         (rep == 1 || rep == 2 || rep == 4 || rep == 8) && (int64_t)a.S * a.Hkv <= (1 << 30);
}

// Column groups of the fused output projection: 4 where the items (sequence,
// KV head) are few enough that 4 workgroups each still fit one round of the
// chip and a group's quarters fit one thread each, else 1. A workgroup's wo
// slice (REP D rows of wo_n floats, 147 KB at TinyLlama's 2 x 48 x 384) then
// streams through 4 compute units' L1s instead of one.
inline int wo_column_groups(int items, int wo_n) {
  if (wo_n % 4 == 0 && wo_n <= 64 * kShortWaves && (int64_t)items * 4 <= vl_num_cus()) return 4;
  return 1;
}

template <typename T, typename TKV, int D>
int launch_short_decode_d(const Args& a, float sl2, hipStream_t st, const float* wo = nullptr,
                          int wo_n = 0, float* parts = nullptr) {
  const int rep = a.H / a.Hkv;
  const int items = a.S * a.Hkv;
  if (items == 0) return VL_OK;
  const int ncg = wo ? wo_column_groups(items, wo_n) : 1;
  const int grid = ncg > 1 ? (items + 7) / 8 * 8 * ncg : items;
  const int bs_log2 = __builtin_ctz((unsigned)a.bs);
#define VL_SHORT(REP)                                                                        \
  attend_short_decode_kernel<T, TKV, D, REP, kShortWaves><<<grid, 64 * kShortWaves, 0, st>>>( \
      (T*)a.out, (const T*)a.query, a.q_stride, (const TKV*)a.kc, (const TKV*)a.vc, a.bt,    \
      a.bt_stride, a.seq_lens, a.qsl, a.Hkv, bs_log2, a.kv_layout == VL_KV_HEAD_MAJOR ? 1 : 0, sl2, \
      wo, wo_n, parts, items, ncg)
  switch (rep) {
    case 1: VL_SHORT(1); break;
    case 2: VL_SHORT(2); break;
    case 4: VL_SHORT(4); break;
    default: VL_SHORT(8); break;
  }
#undef VL_SHORT
  VL_CHECK_LAUNCH();
  return VL_OK;
}

template <typename T, typename TKV>
int launch_short_decode(const Args& a, float sl2, hipStream_t st, const float* wo = nullptr,
                        int wo_n = 0, float* parts = nullptr) {
  switch (a.D) {
    case 16: return launch_short_decode_d<T, TKV, 16>(a, sl2, st, wo, wo_n, parts);
    case 32: return launch_short_decode_d<T, TKV, 32>(a, sl2, st, wo, wo_n, parts);
    case 48: return launch_short_decode_d<T, TKV, 48>(a, sl2, st, wo, wo_n, parts);
    default: return launch_short_decode_d<T, TKV, 64>(a, sl2, st, wo, wo_n, parts);
  }
}

// T: query and output elements, TKV: cache elements (fp32 / fp32, bf16 /
// bf16, or fp32 / bf16; the fast and tile kernels take one type).
template <typename T, typename TKV>
int do_run(const Args& a, int max_q, int min_q, int max_ctx, void* ws, size_t ws_bytes,
           hipStream_t st) {
  const float sl2 = a.scale * kLog2e;
  if (short_decode(a, max_q, max_ctx)) return launch_short_decode<T, TKV>(a, sl2, st);  // no plan
  const Layout L = make_layout(ws, ws_bytes, a.S, a.D);
  const int ncu = vl_num_cus();
  constexpr bool one_type = std::is_same<T, TKV>::value;
  const bool fast = one_type && fast_shape(a.dtype, a.H, a.Hkv, a.D, a.bs);
  if constexpr (!one_type) {
    if (tile_shape(a.dtype, a.D, a.bs)) {
      const int rc = launch_tile<T, TKV>(a, L, sl2, max_q, st);
      if (rc) return rc;
    }
  } else if (fast) {
    if (max_q == 1) {  // every sequence is a decode
      attend_decode_bf16_kernel<<<decode_grid(), 256, 0, st>>>(VL_ATTN_LAUNCH_ARGS(uint16_t),
                                                               L.hdr, L.hdr + 8);
      VL_CHECK_LAUNCH();
      return VL_OK;
    }
    // With both bounds known the host knows the batch's kind: decodes and
    // multi-query sequences together (min 1, max > 1) run in the step kernel
    // alone; multi-query sequences only (min > 1) in the tile kernels alone.
    // A bound unknown (0): the step kernel runs a mixed batch and exits on any
    // other (the plan's flag, read on the device), the tile kernels the reverse.
    const bool known = max_q > 0 && min_q > 0;
    const bool step_all = max_q <= 0;
    if (!known || min_q == 1) {
      attend_step_bf16_kernel<<<step_grid(), 256, 0, st>>>(VL_ATTN_LAUNCH_ARGS(uint16_t), L.hdr,
                                                           L.wide_off, L.wide_seq, L.tile_off,
                                                           L.tail_seq, L.hdr + 16, step_all ? 1 : 0);
      VL_CHECK_LAUNCH();
    }
    if (!step_all && !(known && min_q == 1)) {
      const int rc = launch_tile<T>(a, L, sl2, max_q, st);
      if (rc) return rc;
    }
  } else if (tile_shape(a.dtype, a.D, a.bs)) {
    int rc = launch_tile<T>(a, L, sl2, max_q, st);
    if (rc) return rc;
  }
  if (!fast && !tile_shape(a.dtype, a.D, a.bs)) {
    attend_generic_kernel<T, TKV><<<ncu * 16, 64, 0, st>>>(
        (T*)a.out, (const T*)a.query, a.q_stride, (const TKV*)a.kc, (const TKV*)a.vc, a.bt,
        a.bt_stride, a.seq_lens, a.qsl, a.S, a.H, a.Hkv, a.D, a.bs,
        a.kv_layout == VL_KV_HEAD_MAJOR ? 1 : 0, sl2, L.hdr, L.gen_off,
        L.nparts, L.split_base, L.ml, L.po);
    VL_CHECK_LAUNCH();
    // the generic kernel's split rows; the other kernels merge their own
    // one workgroup per (split sequence, query head) item, at most S * H of them
    const int cmb_grid =
        (int)std::min<int64_t>((int64_t)ncu * 8, std::max<int64_t>((int64_t)a.S * a.H, 1));
    combine_kernel<T><<<cmb_grid, 256, 0, st>>>((T*)a.out, a.qsl, a.H, a.D, L.hdr, L.cmb_seq,
                                              L.nparts, L.split_base, L.ml, L.po);
    VL_CHECK_LAUNCH();
  }
  return VL_OK;
}

int dispatch_run(const Args& a, int max_q, int min_q, int max_ctx, void* ws, size_t ws_bytes,
                 hipStream_t st) {
  switch (a.dtype) {
    case VL_DTYPE_F32: return do_run<float, float>(a, max_q, min_q, max_ctx, ws, ws_bytes, st);
    case VL_DTYPE_BF16:
      return do_run<uint16_t, uint16_t>(a, max_q, min_q, max_ctx, ws, ws_bytes, st);
    case VL_DTYPE_F32_FP8KV:
      return do_run<float, uint8_t>(a, max_q, min_q, max_ctx, ws, ws_bytes, st);
    default: return do_run<float, uint16_t>(a, max_q, min_q, max_ctx, ws, ws_bytes, st);
  }
}

}  // namespace

extern "C" size_t vl_paged_attention_min_workspace(int num_seqs) {
  return fixed_bytes(num_seqs < 0 ? 0 : num_seqs);
}

extern "C" size_t vl_paged_attention_workspace_size(int num_seqs, int num_tokens, int num_heads,
                                                    int head_dim, int max_context_len) {
  if (num_seqs < 0 || num_tokens < 0 || num_heads <= 0 || head_dim <= 0) return 0;
  const int64_t S = num_seqs, H = num_heads;
  const int64_t ctx = max_context_len > 0 ? max_context_len : 1;
  // multi-query rows split into partitions of kPart0 tokens or more (at most 64)
  const int64_t split_tokens = num_tokens < S * kSplitMaxQ ? num_tokens : S * kSplitMaxQ;
  int64_t parts = std::min<int64_t>(std::max<int64_t>(cdiv64(ctx, kPart0), 1), 64);
  // (and a split sequence's arrival counters, at most one row per query row)
  const int64_t rows_tile = parts > 1 ? split_tokens * H * (parts + 1) : 0;
  // decode ranges: as short as 64 tokens for small batches, at most a few
  // items per resident workgroup (plus one short range per sequence) and at
  // most kRangeMax (2048) tokens long otherwise
  const int64_t rows_fast =
      std::min<int64_t>(S * H * cdiv64(ctx, 64),
                        4 * kItemsPerWg * (int64_t)decode_grid() +
                            S * H * (cdiv64(ctx, kRangeMax) + 1));
  const int64_t rows = std::max(rows_tile, rows_fast);
  return fixed_bytes(num_seqs) + (size_t)rows * row_bytes(head_dim);
}

extern "C" int vl_paged_attention_reads_plan(int num_heads, int num_kv_heads, int head_dim,
                                             int block_size, int max_query_len,
                                             int max_context_len) {
  Args a{};
  a.H = num_heads, a.Hkv = num_kv_heads, a.D = head_dim, a.bs = block_size;
  return short_decode(a, max_query_len, max_context_len) ? 0 : 1;
}

extern "C" int vl_paged_attention_plan(const int32_t* seq_lens, const int32_t* query_start_loc,
                                       int num_seqs, int num_tokens, int num_heads,
                                       int num_kv_heads, int head_dim, int block_size, int dtype,
                                       void* workspace, size_t workspace_bytes, void* stream) {
  Args a{};
  a.seq_lens = seq_lens, a.qsl = query_start_loc, a.S = num_seqs, a.T = num_tokens;
  a.H = num_heads, a.Hkv = num_kv_heads, a.D = head_dim, a.bs = block_size, a.dtype = dtype;
  int rc = check_args(a, workspace, workspace_bytes, false);
  if (rc || a.S == 0 || a.T == 0) return rc;
  return do_plan(a, workspace, workspace_bytes, (hipStream_t)stream);
}

extern "C" int vl_paged_attention_run(void* out, const void* query, int64_t query_stride,
                                      const void* key_cache, const void* value_cache,
                                      const int32_t* block_tables, int block_table_stride,
                                      const int32_t* seq_lens, const int32_t* query_start_loc,
                                      int num_seqs, int num_tokens, int num_heads,
                                      int num_kv_heads, int head_dim, int block_size, float scale,
                                      int dtype, int kv_layout, int max_query_len,
                                      int min_query_len, int max_context_len, void* workspace,
                                      size_t workspace_bytes, void* stream) {
  VL_CHECK_ARG(min_query_len >= 0 && (max_query_len <= 0 || min_query_len <= max_query_len),
               "bad query length bounds");
  VL_CHECK_ARG(max_context_len >= 0, "bad context length bound");
  Args a{out, query, query_stride, key_cache, value_cache, block_tables, block_table_stride,
         seq_lens, query_start_loc, num_seqs, num_tokens, num_heads, num_kv_heads, head_dim,
         block_size, scale, dtype, kv_layout};
  KvGeom geom;
  if (num_kv_heads > 0 && head_dim > 0)
    if (int rc = vl_kv_geom(kv_layout, block_size, num_kv_heads, head_dim, &geom)) return rc;
  int rc = check_args(a, workspace, workspace_bytes, true);
  if (rc || a.S == 0 || a.T == 0) return rc;
  if (fast_shape(dtype, num_heads, num_kv_heads, head_dim, block_size) ||
      tile_shape(dtype, head_dim, block_size))
    VL_CHECK_ARG((query_stride % 8) == 0 && ((uintptr_t)query & 15) == 0 &&
                     ((uintptr_t)out & 15) == 0 && ((uintptr_t)key_cache & 15) == 0 &&
                     ((uintptr_t)value_cache & 15) == 0,
                 "query, out and caches must be 16-byte aligned (query rows a multiple of 8 elements)");
  if (short_decode(a, max_query_len, max_context_len))
    VL_CHECK_ARG(((uintptr_t)key_cache & 15) == 0 && ((uintptr_t)value_cache & 15) == 0,
                 "caches must be 16-byte aligned");
  return dispatch_run(a, max_query_len, min_query_len, max_context_len, workspace,
                      workspace_bytes, (hipStream_t)stream);
}

extern "C" int vl_decode_attention_wo(float* parts, const float* query, int64_t query_stride,
                                      const void* key_cache, const void* value_cache,
                                      const int32_t* block_tables, int block_table_stride,
                                      const int32_t* seq_lens, const int32_t* query_start_loc,
                                      int num_seqs, int num_heads, int num_kv_heads, int head_dim,
                                      int block_size, float scale, int dtype, int kv_layout,
                                      int max_context_len, const float* wo, int d_model,
                                      void* stream) {
  Args a{parts, query, query_stride, key_cache, value_cache, block_tables, block_table_stride,
         seq_lens, query_start_loc, num_seqs, num_seqs, num_heads, num_kv_heads, head_dim,
         block_size, scale, dtype, kv_layout};
  VL_CHECK_ARG(dtype == VL_DTYPE_F32 || dtype == VL_DTYPE_F32_BF16KV || dtype == VL_DTYPE_F32_FP8KV,
               "fp32 queries required (dtype %d)", dtype);
  VL_CHECK_ARG(num_seqs >= 0 && num_kv_heads > 0 && num_heads > 0 && num_heads % num_kv_heads == 0,
               "bad head counts");
  VL_CHECK_ARG(short_decode(a, 1, max_context_len),
               "not a short-decode batch (head_dim 16/32/48/64, 1/2/4/8 query heads per KV head, "
               "power-of-two blocks, 0 < max_context_len <= %d)", kShortCtx);
  VL_CHECK_ARG(d_model > 0 && d_model <= 64 * kShortWaves, "d_model must be in 1..%d",
               64 * kShortWaves);
  VL_CHECK_ARG(query_stride >= (int64_t)num_heads * head_dim, "query row stride too small");
  KvGeom geom;
  if (int rc = vl_kv_geom(kv_layout, block_size, num_kv_heads, head_dim, &geom)) return rc;
  if (num_seqs == 0) return VL_OK;
  VL_CHECK_ARG(parts && query && key_cache && value_cache && block_tables && seq_lens &&
                   query_start_loc && wo,
               "null pointer");
  VL_CHECK_ARG(((uintptr_t)key_cache & 15) == 0 && ((uintptr_t)value_cache & 15) == 0,
               "caches must be 16-byte aligned");
  const float sl2 = scale * kLog2e;
  hipStream_t st = (hipStream_t)stream;
  switch (dtype) {
    case VL_DTYPE_F32: return launch_short_decode<float, float>(a, sl2, st, wo, d_model, parts);
    case VL_DTYPE_F32_BF16KV:
      return launch_short_decode<float, uint16_t>(a, sl2, st, wo, d_model, parts);
    default: return launch_short_decode<float, uint8_t>(a, sl2, st, wo, d_model, parts);
  }
}

extern "C" int vl_paged_attention(void* out, const void* query, int64_t query_stride,
                                  const void* key_cache, const void* value_cache,
                                  const int32_t* block_tables, int block_table_stride,
                                  const int32_t* seq_lens, const int32_t* query_start_loc,
                                  int num_seqs, int num_tokens, int num_heads, int num_kv_heads,
                                  int head_dim, int block_size, float scale, int dtype,
                                  int kv_layout, int max_query_len, int min_query_len,
                                  int max_context_len, void* workspace, size_t workspace_bytes,
                                  void* stream) {
  Args a{};
  a.S = num_seqs, a.H = num_heads, a.Hkv = num_kv_heads, a.D = head_dim, a.bs = block_size;
  if (!short_decode(a, max_query_len, max_context_len)) {  // that kernel reads no plan
    const int rc = vl_paged_attention_plan(seq_lens, query_start_loc, num_seqs, num_tokens,
                                           num_heads, num_kv_heads, head_dim, block_size, dtype,
                                           workspace, workspace_bytes, stream);
    if (rc) return rc;
  }
  return vl_paged_attention_run(out, query, query_stride, key_cache, value_cache, block_tables,
                                block_table_stride, seq_lens, query_start_loc, num_seqs,
                                num_tokens, num_heads, num_kv_heads, head_dim, block_size, scale,
                                dtype, kv_layout, max_query_len, min_query_len, max_context_len,
                                workspace, workspace_bytes, stream);
}

// ---------------------------------------------------- allocation-free call --
// The workspace of vl_paged_attention_noalloc: a file-scope device array, one
// copy per GPU, held until the process ends. Host code never passes its name
// to a kernel (the name is a host-side stand-in); it uses the per-device
// address hipGetSymbolAddress returns.
static __device__ __align__(256) unsigned char scratch[VL_NOALLOC_SCRATCH_BYTES];

namespace {

std::mutex g_scratch_mu;
void* g_scratch_ptr[64] = {};

// The current device's copy of `scratch`, looked up once per device.
int scratch_ptr(void** out) {
  int dev = 0;
  VL_CHECK_HIP(hipGetDevice(&dev));
  VL_CHECK_ARG(dev >= 0 && dev < 64, "device ordinal %d out of range", dev);
  std::lock_guard<std::mutex> lock(g_scratch_mu);
  if (!g_scratch_ptr[dev]) {
    void* p = nullptr;
    VL_CHECK_HIP(hipGetSymbolAddress(&p, HIP_SYMBOL(scratch)));
    VL_CHECK_ARG(p != nullptr && ((uintptr_t)p & 255) == 0, "bad scratch address");
    g_scratch_ptr[dev] = p;
  }
  *out = g_scratch_ptr[dev];
  return VL_OK;
}

}  // namespace

extern "C" int vl_paged_attention_noalloc(void* out, const void* query, int64_t query_stride,
                                          const void* key_cache, const void* value_cache,
                                          const int32_t* block_tables, int block_table_stride,
                                          const int32_t* seq_lens,
                                          const int32_t* query_start_loc, int num_seqs,
                                          int num_tokens, int num_heads, int num_kv_heads,
                                          int head_dim, int block_size, float scale, int dtype,
                                          int kv_layout, int max_query_len, int min_query_len,
                                          int max_context_len, void* stream) {
  VL_CHECK_ARG(num_seqs >= 0 && fixed_bytes(num_seqs) <= (size_t)VL_NOALLOC_SCRATCH_BYTES,
               "vl_paged_attention_noalloc: %d sequences need %zu bytes of plan space, more than "
               "its %zu-byte static scratch; use vl_paged_attention with a workspace",
               num_seqs, fixed_bytes(num_seqs < 0 ? 0 : num_seqs),
               (size_t)VL_NOALLOC_SCRATCH_BYTES);
  void* ws = nullptr;
  const int rc = scratch_ptr(&ws);
  if (rc) return rc;
  // the plan kernel rewrites every header field and counter the run reads,
  // so nothing left in the scratch by an earlier call is used
  return vl_paged_attention(out, query, query_stride, key_cache, value_cache, block_tables,
                            block_table_stride, seq_lens, query_start_loc, num_seqs, num_tokens,
                            num_heads, num_kv_heads, head_dim, block_size, scale, dtype,
                            kv_layout, max_query_len, min_query_len, max_context_len, ws,
                            (size_t)VL_NOALLOC_SCRATCH_BYTES, stream);
}
