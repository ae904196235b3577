// K2 ragged paged attention: decode, chunked prefill and speculative verify in
// one call (vllmlite/attention.py:59-98 applied per sequence at
// vllmlite/model.py:107-112).
//
// Three launches on the caller's stream, no host synchronisation:
//  1. plan    one workgroup reads seq_lens / query_start_loc and writes, into
//             the workspace, per-sequence work-item offsets, the number of
//             context partitions and where split partials go. The partition
//             length doubles until the split partials fit the workspace, so
//             any workspace >= the minimum is correct.
//  2. attend  a persistent grid walks the item list. Each item is one
//             (sequence, query token, head, context partition); a wavefront
//             streams the partition's keys 64 at a time through the block
//             table with an online (running max / running sum) softmax.
//  3. combine sequences whose context was split merge their partials with
//             the usual max-rescaled log-sum-exp.
#include "vl_common.h"

namespace {

constexpr int kHdrInts = 64;      // header: [0] n_items, [1] partition tokens, [2] split rows
constexpr int kPlanThreads = 1024;
constexpr int kMaxHeadDim = 256;
constexpr int kSplitMaxQ = 16;    // only sequences with <= this many queries split their context
constexpr int kPart0 = 256;       // first partition length tried by the planner

struct Layout {
  int32_t* hdr;
  int32_t* item_off;   // [S+1]
  int32_t* nparts;     // [S]
  int32_t* split_base; // [S] first partial row, or -1
  float2* ml;          // [cap_rows] (running max, running sum)
  float* po;           // [cap_rows, D] unnormalised partial outputs
  int64_t cap_rows;
};

inline size_t plan_bytes(int S) {
  size_t b = kHdrInts * 4 + (size_t)(3 * S + 1) * 4;
  return (b + 255) & ~(size_t)255;
}

inline Layout make_layout(void* ws, size_t bytes, int S, int D) {
  Layout L;
  char* p = (char*)ws;
  L.hdr = (int32_t*)p;
  L.item_off = L.hdr + kHdrInts;
  L.nparts = L.item_off + S + 1;
  L.split_base = L.nparts + S;
  const size_t pb = plan_bytes(S);
  const size_t per_row = (size_t)(D + 2) * 4;
  L.cap_rows = bytes > pb ? (int64_t)((bytes - pb) / per_row) : 0;
  L.ml = (float2*)(p + pb);
  L.po = (float*)(p + pb + (size_t)L.cap_rows * 8);
  return L;
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

// Exclusive scan of one int64 per thread across the workgroup; returns the
// thread's offset and writes the total to *total.
__device__ int64_t block_exclusive_scan(int64_t v, int64_t* total) {
  __shared__ int64_t buf[kPlanThreads];
  const int t = threadIdx.x;
  buf[t] = v;
  __syncthreads();
  for (int o = 1; o < kPlanThreads; o <<= 1) {
    const int64_t a = t >= o ? buf[t - o] : 0;
    __syncthreads();
    buf[t] += a;
    __syncthreads();
  }
  const int64_t incl = buf[t];
  *total = buf[kPlanThreads - 1];
  __syncthreads();
  return incl - v;
}

__global__ void __launch_bounds__(kPlanThreads) plan_kernel(
    const int32_t* __restrict__ seq_lens, const int32_t* __restrict__ qsl, int S, int H,
    int64_t cap_rows, int32_t* __restrict__ hdr, int32_t* __restrict__ item_off,
    int32_t* __restrict__ nparts, int32_t* __restrict__ split_base) {
  __shared__ unsigned long long need;
  __shared__ int part_len;
  const int t = threadIdx.x;
  if (t == 0) part_len = kPart0;
  __syncthreads();
  // 1. smallest power-of-two multiple of kPart0 whose split partials fit
  for (;;) {
    if (t == 0) need = 0;
    __syncthreads();
    const int P = part_len;
    unsigned long long mine = 0;
    for (int i = t; i < S; i += kPlanThreads) {
      const int q = qsl[i + 1] - qsl[i], c = seq_lens[i];
      if (q > 0 && q <= kSplitMaxQ && c > P) mine += (unsigned long long)q * H * ((c + P - 1) / P);
    }
    if (mine) atomicAdd(&need, mine);
    __syncthreads();
    const bool fits = need <= (unsigned long long)cap_rows || P >= (1 << 30);
    __syncthreads();
    if (fits) break;
    if (t == 0) part_len = P * 2;
    __syncthreads();
  }
  const int P = part_len;
  // 2. per-sequence items and split rows, contiguous chunk of sequences per thread
  const int chunk = (S + kPlanThreads - 1) / kPlanThreads;
  const int s0 = min(S, t * chunk), s1 = min(S, s0 + chunk);
  int64_t items = 0, rows = 0;
  for (int i = s0; i < s1; ++i) {
    const int q = qsl[i + 1] - qsl[i], c = seq_lens[i];
    const int np = (q > 0 && q <= kSplitMaxQ && c > P) ? (c + P - 1) / P : 1;
    items += (int64_t)max(q, 0) * H * np;
    if (np > 1) rows += (int64_t)q * H * np;
  }
  int64_t tot_items, tot_rows;
  int64_t io = block_exclusive_scan(items, &tot_items);
  int64_t ro = block_exclusive_scan(rows, &tot_rows);
  for (int i = s0; i < s1; ++i) {
    const int q = qsl[i + 1] - qsl[i], c = seq_lens[i];
    const int np = (q > 0 && q <= kSplitMaxQ && c > P) ? (c + P - 1) / P : 1;
    item_off[i] = (int32_t)io;
    nparts[i] = np;
    split_base[i] = np > 1 ? (int32_t)ro : -1;
    io += (int64_t)max(q, 0) * H * np;
    if (np > 1) ro += (int64_t)q * H * np;
  }
  if (t == 0) {
    item_off[S] = (int32_t)tot_items;
    hdr[0] = (int32_t)tot_items;
    hdr[1] = P;
    hdr[2] = (int32_t)tot_rows;
  }
}

template <typename T>
__global__ void __launch_bounds__(64) attend_generic_kernel(
    T* __restrict__ out, const T* __restrict__ query, int64_t q_stride, const T* __restrict__ kc,
    const T* __restrict__ vc, const int32_t* __restrict__ bt, int bt_stride,
    const int32_t* __restrict__ seq_lens, const int32_t* __restrict__ qsl, int S, int H, int Hkv,
    int D, int bs, float scale, const int32_t* __restrict__ hdr,
    const int32_t* __restrict__ item_off, const int32_t* __restrict__ nparts,
    const int32_t* __restrict__ split_base, float2* __restrict__ ml, float* __restrict__ po) {
  __shared__ float q_s[kMaxHeadDim];
  __shared__ float p_s[64];
  __shared__ int64_t row_s[64];
  const int lane = threadIdx.x;
  const int n_items = hdr[0];
  const int P = hdr[1];
  const int rep = H / Hkv;
  const int64_t slot_stride = (int64_t)Hkv * D;
  constexpr int kR = kMaxHeadDim / 64;
  for (int it = blockIdx.x; it < n_items; it += gridDim.x) {
    const int i = upper_bound_le(item_off, S + 1, it);
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
        const int64_t slot = (int64_t)table[key / bs] * bs + key % bs;
        row = slot * slot_stride + (int64_t)kvh * D;
        const T* kr = kc + row;
        float dot = 0.f;
        for (int d = 0; d < D; ++d) dot += q_s[d] * Elem<T>::load(kr, d);
        s = dot * scale;
      }
      const float cmax = wave_max(s);
      const float m_new = fmaxf(m, cmax);
      const float alpha = (m == -__builtin_inff()) ? 0.f : expf(m - m_new);
      const float p = (key < kend) ? expf(s - m_new) : 0.f;
      l = l * alpha + wave_sum(p);
      p_s[lane] = p;
      row_s[lane] = row;
      __syncthreads();
      const int nk = min(64, kend - k0);
#pragma unroll
      for (int r = 0; r < kR; ++r) acc[r] *= alpha;
      for (int jj = 0; jj < nk; ++jj) {
        const float pj = p_s[jj];
        const T* vr = vc + row_s[jj];
#pragma unroll
        for (int r = 0; r < kR; ++r) {
          const int d = lane + 64 * r;
          if (d < D) acc[r] += pj * Elem<T>::load(vr, d);
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

template <typename T>
__global__ void __launch_bounds__(64) combine_kernel(
    T* __restrict__ out, const int32_t* __restrict__ qsl, int S, int T_, int H, int D,
    const int32_t* __restrict__ nparts, const int32_t* __restrict__ split_base,
    const float2* __restrict__ ml, const float* __restrict__ po) {
  const int lane = threadIdx.x;
  const int64_t pairs = (int64_t)T_ * H;
  for (int64_t pr = blockIdx.x; pr < pairs; pr += gridDim.x) {
    const int tok = (int)(pr / H), h = (int)(pr - (pr / H) * H);
    const int i = upper_bound_le(qsl, S, tok);
    const int np = nparts[i];
    if (np <= 1) continue;
    const int j = tok - qsl[i];
    const int64_t row0 = (int64_t)split_base[i] + (int64_t)(j * H + h) * np;
    float M = -__builtin_inff();
    for (int p = 0; p < np; ++p) M = fmaxf(M, ml[row0 + p].x);
    float L = 0.f;
    for (int p = 0; p < np; ++p) {
      const float2 v = ml[row0 + p];
      if (v.x != -__builtin_inff()) L += v.y * expf(v.x - M);
    }
    const float inv = L > 0.f ? 1.f / L : 0.f;
    for (int d = lane; d < D; d += 64) {
      float a = 0.f;
      for (int p = 0; p < np; ++p) {
        const float2 v = ml[row0 + p];
        if (v.x != -__builtin_inff()) a += po[(row0 + p) * D + d] * expf(v.x - M);
      }
      Elem<T>::store(out + ((int64_t)tok * H + h) * D, d, a * inv);
    }
  }
}

template <typename T>
int launch_attention(void* out, const void* query, int64_t q_stride, const void* kc,
                     const void* vc, const int32_t* bt, int bt_stride, const int32_t* seq_lens,
                     const int32_t* qsl, int S, int T_, int H, int Hkv, int D, int bs,
                     float scale, const Layout& L, hipStream_t st) {
  plan_kernel<<<1, kPlanThreads, 0, st>>>(seq_lens, qsl, S, H, L.cap_rows, L.hdr, L.item_off,
                                          L.nparts, L.split_base);
  VL_CHECK_LAUNCH();
  const int grid = vl_num_cus() * 16;
  attend_generic_kernel<T><<<grid, 64, 0, st>>>(
      (T*)out, (const T*)query, q_stride, (const T*)kc, (const T*)vc, bt, bt_stride, seq_lens,
      qsl, S, H, Hkv, D, bs, scale, L.hdr, L.item_off, L.nparts, L.split_base, L.ml, L.po);
  VL_CHECK_LAUNCH();
  const int64_t pairs = (int64_t)T_ * H;
  const int cgrid = (int)(pairs < 65536 ? pairs : 65536);
  combine_kernel<T><<<cgrid, 64, 0, st>>>((T*)out, qsl, S, T_, H, D, L.nparts, L.split_base,
                                          L.ml, L.po);
  VL_CHECK_LAUNCH();
  return VL_OK;
}

}  // namespace

extern "C" size_t vl_paged_attention_min_workspace(int num_seqs) {
  return plan_bytes(num_seqs < 0 ? 0 : num_seqs);
}

extern "C" size_t vl_paged_attention_workspace_size(int num_seqs, int num_tokens, int num_heads,
                                                    int head_dim, int max_context_len) {
  if (num_seqs < 0 || num_tokens < 0 || num_heads <= 0 || head_dim <= 0) return 0;
  const int64_t split_tokens = num_tokens < (int64_t)num_seqs * kSplitMaxQ
                                   ? num_tokens
                                   : (int64_t)num_seqs * kSplitMaxQ;
  int64_t parts = (max_context_len + kPart0 - 1) / kPart0;
  if (parts < 1) parts = 1;
  if (parts > 64) parts = 64;
  const int64_t rows = parts > 1 ? split_tokens * num_heads * parts : 0;
  return plan_bytes(num_seqs) + (size_t)rows * (size_t)(head_dim + 2) * 4;
}

extern "C" int vl_paged_attention(void* out, const void* query, int64_t query_stride,
                                  const void* key_cache, const void* value_cache,
                                  const int32_t* block_tables, int block_table_stride,
                                  const int32_t* seq_lens, const int32_t* query_start_loc,
                                  int num_seqs, int num_tokens, int num_heads, int num_kv_heads,
                                  int head_dim, int block_size, float scale, int dtype,
                                  void* workspace, size_t workspace_bytes, void* stream) {
  VL_CHECK_ARG(dtype == VL_DTYPE_F32 || dtype == VL_DTYPE_BF16, "bad dtype %d", dtype);
  VL_CHECK_ARG(num_seqs >= 0 && num_tokens >= 0, "bad batch size");
  VL_CHECK_ARG(num_heads > 0 && num_kv_heads > 0 && num_heads % num_kv_heads == 0,
               "num_heads must be a positive multiple of num_kv_heads");
  VL_CHECK_ARG(head_dim > 0 && head_dim <= kMaxHeadDim, "head_dim must be in 1..%d", kMaxHeadDim);
  VL_CHECK_ARG(block_size > 0 && block_table_stride >= 0, "bad block table");
  VL_CHECK_ARG(query_stride >= (int64_t)num_heads * head_dim, "query row stride too small");
  if (num_seqs == 0 || num_tokens == 0) return VL_OK;
  VL_CHECK_ARG(out && query && key_cache && value_cache && block_tables && seq_lens &&
                   query_start_loc && workspace,
               "null pointer");
  VL_CHECK_ARG(workspace_bytes >= vl_paged_attention_min_workspace(num_seqs),
               "workspace too small: %zu < %zu", workspace_bytes,
               vl_paged_attention_min_workspace(num_seqs));
  VL_CHECK_ARG(((uintptr_t)workspace & 255) == 0, "workspace must be 256-byte aligned");
  const Layout L = make_layout(workspace, workspace_bytes, num_seqs, head_dim);
  hipStream_t st = (hipStream_t)stream;
  if (dtype == VL_DTYPE_F32)
    return launch_attention<float>(out, query, query_stride, key_cache, value_cache,
                                   block_tables, block_table_stride, seq_lens, query_start_loc,
                                   num_seqs, num_tokens, num_heads, num_kv_heads, head_dim,
                                   block_size, scale, L, st);
  return launch_attention<uint16_t>(out, query, query_stride, key_cache, value_cache, block_tables,
                                    block_table_stride, seq_lens, query_start_loc, num_seqs,
                                    num_tokens, num_heads, num_kv_heads, head_dim, block_size,
                                    scale, L, st);
}
