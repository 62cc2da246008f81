// QUEST page selection over the dual cache's page tables (gfx950).
//
// The reference's comparison baseline (src/modeling_layers.py:452-576 with
// the page bounds kept at :1333-1347 and :744-761): every global page keeps
// the elementwise min and max of its keys; at a decode step each head scores
// its full global pages by max over the grouped queries of
// sum_d q_d * (q_d >= 0 ? max_d : min_d), keeps the top pages within a token
// budget (after its local window), always keeps the trailing partial page,
// and the decode attention runs over the local pages plus the kept pages.
//
//   * quest_bounds_kernel: recompute the bounds of a head's logical global
//     pages [from/page, ceil(len/page)) from the pool (the min / max over the
//     page's valid rows, which equals the reference's incremental updates);
//   * quest_scores_kernel: the page scores of every head into the workspace;
//   * quest_select_kernel: one workgroup per head -- a 4-pass radix select
//     of the k-th largest score, then a
//     stable compaction that writes local pages, the kept full pages in page
//     order and the partial page, and the head's token count.
// Scores are fp32, or (scores_bf16) rounded as the reference's bf16 torch ops
// round them: each product q_d * bound_d to bf16, the fp32 sum over d to
// bf16.  Equal scores at the cut keep the lowest page index (the reference's
// topk leaves their order unspecified).
#include "wgkv_common.h"

namespace {

constexpr int kThreads = 256;

struct BoundsArgs {
  const uint16_t* pool_k;
  const int32_t* bt;  // block_table + layer * H * max_pages
  int max_pages, lb;  // pages per head, local pages per head
  const int32_t* len;   // global_lengths + layer * H
  const int32_t* from;  // global lengths before the update (NULL: 0)
  int H, page, D;
  uint16_t* kmin;
  uint16_t* kmax;
};

__device__ __forceinline__ float bf(uint16_t x) { return __uint_as_float((uint32_t)x << 16); }
__device__ __forceinline__ float round_bf16f(float x) { return round_to_bf16(x); }

// grid (H, groups): workgroup g of head h takes pages first+g, first+g+groups, ...
__global__ __launch_bounds__(kThreads) void quest_bounds_kernel(BoundsArgs a) {
  const int h = blockIdx.x;
  const int n = a.len[h];
  const int f = a.from ? a.from[h] : 0;
  const int first = f / a.page, last = (n + a.page - 1) / a.page;  // [first, last)
  const int32_t* bt = a.bt + (int64_t)h * a.max_pages + a.lb;
  const int per = kThreads / a.D;  // pages per pass (D <= 256)
  const int sub = threadIdx.x / a.D, d = threadIdx.x % a.D;
  if (sub >= per) return;
  for (int p = first + blockIdx.y * per + sub; p < last; p += gridDim.y * per) {
    const int rows = min(a.page, n - p * a.page);
    const int64_t pg = bt[p];
    const uint16_t* src = a.pool_k + pg * a.page * a.D + d;
    uint16_t lo = src[0], hi = src[0];
    for (int r = 1; r < rows; ++r) {
      const uint16_t x = src[(int64_t)r * a.D];
      if (bf(x) < bf(lo)) lo = x;
      if (bf(x) > bf(hi)) hi = x;
    }
    a.kmin[pg * a.D + d] = lo;
    a.kmax[pg * a.D + d] = hi;
  }
}

struct SelectArgs {
  const uint16_t* q;  // (Hq, D) of this token, stride q_sh
  int64_t q_sh;
  const int32_t* bt;   // block_table + layer * H * max_pages
  int max_pages, lb;
  const int32_t* len;  // global_lengths + layer * H
  const uint16_t* kmin;
  const uint16_t* kmax;
  int H, G, D, page, local_tokens, budget, scores_bf16;
  int32_t* sel_bt;     // (H, sel_cap)
  int sel_cap;
  int32_t* sel_len;    // (H)
  float* scores;       // workspace (H, max_pages)
};

// Page scores, grid (64, H): 16 lanes per page (8 d-values each, 16-byte
// loads of the bounds), the lane partials summed with a 16-lane row
// reduction; workgroups stride over the head's full pages.
__global__ __launch_bounds__(kThreads) void quest_scores_kernel(SelectArgs a) {
  __shared__ float s_q[8][256];
  const int h = blockIdx.y, t = threadIdx.x;
  const int full = a.len[h] / a.page;
  for (int e = t; e < a.G * a.D; e += kThreads) {
    const int g = e / a.D, d = e - g * a.D;
    s_q[g][d] = bf(a.q[(int64_t)(h * a.G + g) * a.q_sh + d]);
  }
  __syncthreads();
  const int32_t* bt = a.bt + (int64_t)h * a.max_pages + a.lb;
  float* sc = a.scores + (int64_t)h * a.max_pages;
  const int lane16 = t & 15, slot = t >> 4;  // 16 pages per pass
  const int nch = a.D / 8;                   // 8-value chunks per row (<= 32)
  for (int p0 = blockIdx.x * 16; p0 < full; p0 += gridDim.x * 16) {
    const int p = p0 + slot;
    const bool ok = p < full;
    const int64_t pg = ok ? bt[p] : 0;
    float s[8];
#pragma unroll
    for (int g = 0; g < 8; ++g) s[g] = 0.f;
    for (int c = lane16; c < nch; c += 16) {
      const u32x4_t lo = ok ? *(const u32x4_t*)(a.kmin + pg * a.D + c * 8) : (u32x4_t){0u, 0u, 0u, 0u};
      const u32x4_t hi = ok ? *(const u32x4_t*)(a.kmax + pg * a.D + c * 8) : (u32x4_t){0u, 0u, 0u, 0u};
#pragma unroll
      for (int e = 0; e < 8; ++e) {
        const float l = (e & 1) ? bf16hi(lo[e >> 1]) : bf16lo(lo[e >> 1]);
        const float u = (e & 1) ? bf16hi(hi[e >> 1]) : bf16lo(hi[e >> 1]);
        for (int g = 0; g < a.G; ++g) {
          const float qd = s_q[g][c * 8 + e];
          const float b = qd >= 0.f ? u : l;
          // a product of two bf16 values is exact in fp32; bf16 ops round it
          s[g] = a.scores_bf16 ? s[g] + round_bf16f(qd * b) : fmaf(qd, b, s[g]);
        }
      }
    }
    float best = -INFINITY;
    for (int g = 0; g < a.G; ++g) {
      const float v = row_sum16(s[g]);
      best = fmaxf(best, a.scores_bf16 ? round_bf16f(v) : v);
    }
    if (ok && lane16 == 0) sc[p] = best;
  }
}

// order-preserving map of an fp32 to uint32 (larger float -> larger key)
__device__ __forceinline__ uint32_t fkey(float f) {
  const uint32_t u = __float_as_uint(f);
  return (u & 0x80000000u) ? ~u : (u | 0x80000000u);
}

__global__ __launch_bounds__(kThreads) void quest_select_kernel(SelectArgs a) {
  __shared__ int s_hist[256];
  __shared__ int s_tmp[kThreads];
  __shared__ uint32_t s_prefix;
  __shared__ int s_need;
  const int h = blockIdx.x, t = threadIdx.x;
  const int n = a.len[h];
  const int full = n / a.page, rem = n % a.page;
  const int local_blocks = (a.local_tokens + a.page - 1) / a.page;
  const int budget_blocks = (max(a.budget - a.local_tokens, 0) + a.page - 1) / a.page;
  const int gblocks = (n + a.page - 1) / a.page;
  const int capacity = min(budget_blocks, gblocks);
  const bool partial = capacity > 0 && rem > 0;
  const int k = capacity - (rem > 0 ? 1 : 0);  // full pages to keep
  const int32_t* bt = a.bt + (int64_t)h * a.max_pages;
  int32_t* out = a.sel_bt + (int64_t)h * a.sel_cap;
  float* sc = a.scores + (int64_t)h * a.max_pages;

  for (int i = t; i < local_blocks; i += kThreads) out[i] = bt[i];
  const bool all = k >= full;
  const int keep = k <= 0 ? 0 : (all ? full : k);

  if (keep > 0 && !all) {
    // radix select of the key of the keep-th largest score
    if (t == 0) {
      s_prefix = 0;
      s_need = keep;
    }
    __syncthreads();
    for (int shift = 24; shift >= 0; shift -= 8) {
      s_hist[t] = 0;
      __syncthreads();
      const uint32_t hi_mask = shift == 24 ? 0u : (0xffffffffu << (shift + 8));
      const uint32_t prefix = s_prefix;
      for (int p = t; p < full; p += kThreads) {
        const uint32_t key = fkey(sc[p]);
        if ((key & hi_mask) == (prefix & hi_mask)) atomicAdd(&s_hist[(key >> shift) & 255], 1);
      }
      __syncthreads();
      // counts from the top bin down: thread t holds bin 255 - t
      const int c = s_hist[255 - t];
      int total = 0;
      const int above = block_exclusive_scan_256(c, s_tmp, &total);  // keys in higher bins
      const int need = s_need;
      __syncthreads();
      if (above < need && need <= above + c) {  // the bin holding the need-th key
        s_prefix = prefix | ((uint32_t)(255 - t) << shift);
        s_need = need - above;
      }
      __syncthreads();
    }
    // kept: key > T, plus the first s_need pages (in page order) with key == T;
    // thread t owns the contiguous pages [t*per, (t+1)*per)
    const uint32_t T = s_prefix;
    const int need_eq = s_need;
    const int per = (full + kThreads - 1) / kThreads;
    const int p0 = min(full, t * per), p1 = min(full, p0 + per);
    int n_eq = 0;
    for (int p = p0; p < p1; ++p) n_eq += fkey(sc[p]) == T ? 1 : 0;
    int tot = 0;
    int eq_rank = block_exclusive_scan_256(n_eq, s_tmp, &tot);
    int n_take = 0;
    {
      int r = eq_rank;
      for (int p = p0; p < p1; ++p) {
        const uint32_t key = fkey(sc[p]);
        if (key > T) ++n_take;
        else if (key == T) n_take += (r++ < need_eq) ? 1 : 0;
      }
    }
    int pos = local_blocks + block_exclusive_scan_256(n_take, s_tmp, &tot);
    for (int p = p0; p < p1; ++p) {
      const uint32_t key = fkey(sc[p]);
      bool take = key > T;
      if (key == T) take = eq_rank++ < need_eq;
      if (take) out[pos++] = bt[a.lb + p];
    }
  } else if (keep > 0) {
    for (int p = t; p < keep; p += kThreads) out[local_blocks + p] = bt[a.lb + p];
  }
  if (t == 0) {
    if (partial) out[local_blocks + keep] = bt[a.lb + full];
    a.sel_len[h] = a.local_tokens + keep * a.page + (partial ? rem : 0);
  }
}

}  // namespace

extern "C" int wgkv_quest_update_bounds(
    const void* pool_k, const int32_t* block_table, int32_t max_pages_per_head,
    const int32_t* global_lengths, const int32_t* from_lengths,
    int32_t layer, int32_t num_layers, int32_t num_kv_heads, int32_t local_window, int32_t page_size,
    int32_t head_dim, void* key_min, void* key_max, void* stream) {
  if (!pool_k || !block_table || !global_lengths || !key_min || !key_max) return WGKV_ERR_ARG;
  if (layer < 0 || layer >= num_layers || num_kv_heads <= 0 || page_size <= 0 || local_window % page_size)
    return WGKV_ERR_ARG;
  if (head_dim <= 0 || head_dim > kThreads || kThreads % head_dim) return WGKV_ERR_UNSUPPORTED;
  BoundsArgs a;
  a.pool_k = (const uint16_t*)pool_k;
  a.bt = block_table + (int64_t)layer * num_kv_heads * max_pages_per_head;
  a.max_pages = max_pages_per_head;
  a.lb = local_window / page_size;
  a.len = global_lengths + (int64_t)layer * num_kv_heads;
  a.from = from_lengths;
  a.H = num_kv_heads;
  a.page = page_size;
  a.D = head_dim;
  a.kmin = (uint16_t*)key_min;
  a.kmax = (uint16_t*)key_max;
  hipLaunchKernelGGL(quest_bounds_kernel, dim3(num_kv_heads, 64), dim3(kThreads), 0, (hipStream_t)stream, a);
  return hipGetLastError() == hipSuccess ? WGKV_OK : WGKV_ERR_HIP;
}

extern "C" size_t wgkv_quest_select_workspace_bytes(int32_t num_kv_heads, int32_t max_pages_per_head) {
  return (size_t)num_kv_heads * max_pages_per_head * sizeof(float);
}

extern "C" int wgkv_quest_select(
    const void* q, int64_t q_stride_h,
    const int32_t* block_table, int32_t max_pages_per_head, const int32_t* global_lengths,
    const void* key_min, const void* key_max,
    int32_t layer, int32_t num_layers, int32_t num_q_heads, int32_t num_kv_heads, int32_t head_dim,
    int32_t local_window, int32_t page_size, int32_t local_tokens, int32_t token_budget, int32_t scores_bf16,
    int32_t* sel_block_table, int32_t sel_cap, int32_t* sel_seqlens,
    void* workspace, size_t workspace_bytes, void* stream) {
  if (!q || !block_table || !global_lengths || !key_min || !key_max || !sel_block_table || !sel_seqlens)
    return WGKV_ERR_ARG;
  if (layer < 0 || layer >= num_layers || num_kv_heads <= 0 || num_q_heads % num_kv_heads) return WGKV_ERR_ARG;
  if (page_size <= 0 || local_window % page_size || local_tokens < 0 || local_tokens > local_window) return WGKV_ERR_ARG;
  const int G = num_q_heads / num_kv_heads;
  if (G > 8 || head_dim <= 0 || head_dim > 256 || head_dim % 8) return WGKV_ERR_UNSUPPORTED;
  if (((uintptr_t)key_min | (uintptr_t)key_max) & 15) return WGKV_ERR_UNSUPPORTED;
  const int local_blocks = (local_tokens + page_size - 1) / page_size;
  const int budget_blocks = ((token_budget > local_tokens ? token_budget - local_tokens : 0) + page_size - 1) / page_size;
  if (sel_cap < local_blocks + budget_blocks) return WGKV_ERR_ARG;
  if (!workspace || workspace_bytes < wgkv_quest_select_workspace_bytes(num_kv_heads, max_pages_per_head))
    return WGKV_ERR_WORKSPACE;
  SelectArgs a;
  a.q = (const uint16_t*)q;
  a.q_sh = q_stride_h;
  a.bt = block_table + (int64_t)layer * num_kv_heads * max_pages_per_head;
  a.max_pages = max_pages_per_head;
  a.lb = local_window / page_size;
  a.len = global_lengths + (int64_t)layer * num_kv_heads;
  a.kmin = (const uint16_t*)key_min;
  a.kmax = (const uint16_t*)key_max;
  a.H = num_kv_heads;
  a.G = G;
  a.D = head_dim;
  a.page = page_size;
  a.local_tokens = local_tokens;
  a.budget = token_budget;
  a.scores_bf16 = scores_bf16 ? 1 : 0;
  a.sel_bt = sel_block_table;
  a.sel_cap = sel_cap;
  a.sel_len = sel_seqlens;
  a.scores = (float*)workspace;
  hipStream_t st = (hipStream_t)stream;
  hipLaunchKernelGGL(quest_scores_kernel, dim3(64, num_kv_heads), dim3(kThreads), 0, st, a);
  hipLaunchKernelGGL(quest_select_kernel, dim3(num_kv_heads), dim3(kThreads), 0, st, a);
  return hipGetLastError() == hipSuccess ? WGKV_OK : WGKV_ERR_HIP;
}
