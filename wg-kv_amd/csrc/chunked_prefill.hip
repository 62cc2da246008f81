// Chunked gated prefill: cache writes around the attention of one chunk
// (gfx950).  The reference prefills the whole prompt at once
// (src/modeling_layers.py:1183-1376); a chunk [c0, c0+C) here leaves the dual
// cache exactly as a one-shot prefill of the first c0+C tokens would, up to
// page numbering:
//   * admit: the admitted positions of [c0-W, c0+C-W) -- the previous ring
//     (slot i holds position c0-W+i, flag in local_is_global) followed by the
//     chunk -- are appended in position order to each head's global cache
//     (so it stays sorted), new pages bump-allocated in head order as a head
//     crosses page boundaries;
//   * column_count of the chunk's row blocks = admitted positions below
//     max(0, r*64 - W + 1): the global length before the chunk plus a prefix
//     count over (ring flags ++ chunk mask);
//   * ring (after the chunk's attention): slot i <- position c0+C-W+i.
// Requires, for every chunk after the first, c0 >= W (a full ring) and C >= W
// (the ring then refills from the chunk alone); c0 and W multiples of 64.
#include "wgkv_common.h"

namespace {

constexpr int kThreads = 256;
constexpr int kWaves = kThreads / 64;
constexpr int kTile = 512;   // virtual positions per scan tile
constexpr int kBlk = 64;

struct ChunkArgs {
  const uint16_t* key;
  const uint16_t* value;
  int64_t kv_sh, kv_ss;
  const uint16_t* pre_key;
  int64_t pk_sh, pk_ss;
  const uint8_t* mask;  // chunk flags (H, C)
  int64_t m_sh;
  int mask_vec16;       // mask rows 16-byte aligned (16 flags per load)
  int layer, H, C, D, W, page, max_tokens_per_head, c0;
  int64_t total_pages;
  uint16_t* pool_k;
  uint16_t* pool_v;
  int32_t* block_table;
  int max_pages;
  int32_t* global_lengths;
  uint8_t* local_is_global;
  uint16_t* local_pre_key;
  int32_t* next_free;
  int32_t* status;
  int32_t* column_count;  // (H, R_chunk)
  int r0, rchunk;         // first global row block of the chunk, row blocks in the chunk
  int ntiles;             // kTile-position tiles of the virtual sequence
  // workspace, written by stage 0 and read by stage 1
  int32_t* adm;           // (H) positions admitted by the chunk
  int32_t* gl_before;     // (H) global lengths before the chunk
  int32_t* next_free_after;
  int32_t* abort_flag;
};

constexpr int kMaxHeads = 1024;

// Virtual sequence of a chunk: ring positions (c0 > 0 only) then the chunk.
__device__ __forceinline__ int vlen(const ChunkArgs& a) { return (a.c0 > 0 ? a.W : 0) + a.C; }
__device__ __forceinline__ int vring(const ChunkArgs& a) { return a.c0 > 0 ? a.W : 0; }

__device__ __forceinline__ bool vflag(const ChunkArgs& a, int h, int v) {
  const int nr = vring(a);
  if (v < nr) return a.local_is_global[((int64_t)a.layer * a.H + h) * a.W + v] != 0;
  return a.mask[(int64_t)h * a.m_sh + (v - nr)] != 0;
}

// Admitted flags among virtual positions [v, min(v + 16, lim)) of head h
// (flags are 0/1 bytes, so popcounts of the 16 bytes count them).  The ring
// length W and v are multiples of 16, so the 16 positions lie all in the
// ring or all in the chunk; reads never pass the chunk's own flags (v < lim
// <= chunk_len + ring, and lim - v < 16 only at the admission range's end,
// which lies W - 16 or more flags before the end of the chunk).
__device__ __forceinline__ int count16(const ChunkArgs& a, int h, int v, int lim) {
  const int nr = vring(a);
  const int n = min(16, lim - v);
  const uint8_t* p = v < nr ? a.local_is_global + ((int64_t)a.layer * a.H + h) * a.W + v
                            : a.mask + (int64_t)h * a.m_sh + (v - nr);
  u32x4_t w;
  if (v < nr || a.mask_vec16) {
    w = *(const u32x4_t*)p;
  } else {
    w = (u32x4_t){0u, 0u, 0u, 0u};
    for (int i = 0; i < n; ++i) w[i >> 2] |= (uint32_t)p[i] << (8 * (i & 3));
  }
  if (n < 16) {
#pragma unroll
    for (int q = 0; q < 4; ++q) {
      const int keep = min(4, max(0, n - 4 * q));  // bytes of word q inside the range
      w[q] &= keep == 4 ? ~0u : ((1u << (8 * keep)) - 1u);
    }
  }
  return __builtin_popcount(w[0]) + __builtin_popcount(w[1]) + __builtin_popcount(w[2]) + __builtin_popcount(w[3]);
}

// Admission of one chunk in one launch (workgroup = kTile virtual positions
// of one head).  Every workgroup first counts the admitted flags of every
// head and makes the same plan from them -- totals, capacity checks before
// any write, pages bump-allocated in head order -- so no workgroup waits for
// another; then it compacts its own tile into the head's pages (new pages are
// numbered arithmetically from the plan, so the block-table entries written
// here are not read back) and writes the column counts of the row blocks
// whose band starts inside its tile: the count of row block r is the number
// of admitted positions below p = 64 r - W + 1, i.e. the inclusive count at
// virtual index p - 1 - base.  The global lengths and the bump pointer are
// left to stage 1 (every workgroup here reads the lengths from before the
// chunk).  Independent loads are issued together: the tile's flags, every
// head's length and the 16-flag count loads, so the launch waits on memory
// about three times (flags and lengths, existing page ids, K/V rows).
__global__ __launch_bounds__(kThreads) void chunk_admit_kernel(ChunkArgs a) {
  constexpr int kPer = kTile / kThreads;
  constexpr int kCnt = 16;       // flags per count load
  constexpr int kLoads = 16;     // count loads per thread issued together
  __shared__ int s_tot[kMaxHeads];    // admitted positions of each head
  __shared__ int s_first[kMaxHeads];  // first new page of each head, relative to the bump pointer
  __shared__ int s_tmp[kThreads];
  __shared__ int s_wave[kWaves];
  __shared__ int s_pre, s_fail, s_total_pages, s_nf;
  __shared__ int s_src[kTile];        // virtual index
  __shared__ int64_t s_dst[kTile];    // pool row
  const int h = blockIdx.y, tile = blockIdx.x;
  const int t = threadIdx.x;
  const int lane = t & 63, wid = t >> 6;
  const int nr = vring(a);
  const int n_adm = vlen(a) - a.W;  // admission range [0, n_adm) of the virtual sequence
  const int lb = a.W / a.page;

  // this tile's flags and the lengths before the chunk
  const int v0 = tile * kTile + t * kPer;
  bool f[kPer];
#pragma unroll
  for (int k = 0; k < kPer; ++k) f[k] = v0 + k < n_adm && vflag(a, h, v0 + k);
  const int gl_t = t < a.H ? a.global_lengths[a.layer * a.H + t] : 0;
  for (int i = t; i < a.H; i += kThreads) s_tot[i] = 0;
  if (t == 0) {
    s_pre = 0;
    s_fail = 0;
    s_nf = *a.next_free;
  }
  __syncthreads();

  // ---- admitted counts of every head, and of this head before the tile ----
  const int gph = n_adm > 0 ? (n_adm + kCnt - 1) / kCnt : 0;  // count loads per head
  const int ng = a.H * gph;
  for (int g0 = t; g0 < ng; g0 += kThreads * kLoads) {
    int c[kLoads];
#pragma unroll
    for (int k = 0; k < kLoads; ++k) {
      const int g = g0 + k * kThreads;
      c[k] = g < ng ? count16(a, g / gph, (g % gph) * kCnt, n_adm) : 0;
    }
#pragma unroll
    for (int k = 0; k < kLoads; ++k) {
      const int g = g0 + k * kThreads;
      if (g < ng && c[k]) {
        const int hh = g / gph;
        atomicAdd(&s_tot[hh], c[k]);
        if (hh == h && (g % gph) * kCnt < tile * kTile) atomicAdd(&s_pre, c[k]);
      }
    }
  }
  __syncthreads();

  // ---- the plan (identical in every workgroup) ----------------------------
  if (a.H <= 64) {
    if (wid == 0) {
      int pages = 0;
      if (lane < a.H) {
        const int n = s_tot[lane];
        pages = (gl_t + n + a.page - 1) / a.page - (gl_t + a.page - 1) / a.page;
        if (n > 0 && (a.W + gl_t + n > a.max_tokens_per_head || lb + (gl_t + n + a.page - 1) / a.page > a.max_pages))
          s_fail = 1;
      }
      const int incl = wave_incl_scan(pages, lane);
      if (lane < a.H) s_first[lane] = incl - pages;
      if (lane == 63) {
        s_total_pages = incl;
        if ((int64_t)s_nf + incl > a.total_pages) s_fail = 1;
      }
    }
  } else {
    int carry = 0;
    for (int h0 = 0; h0 < a.H; h0 += kThreads) {
      const int hh = h0 + t;
      int pages = 0;
      if (hh < a.H) {
        const int n = s_tot[hh];
        const int gl = h0 == 0 ? gl_t : a.global_lengths[a.layer * a.H + hh];
        pages = (gl + n + a.page - 1) / a.page - (gl + a.page - 1) / a.page;
        if (n > 0 && (a.W + gl + n > a.max_tokens_per_head || lb + (gl + n + a.page - 1) / a.page > a.max_pages))
          atomicOr(&s_fail, 1);
      }
      int total = 0;
      const int excl = block_exclusive_scan_256(pages, s_tmp, &total);
      if (hh < a.H) s_first[hh] = carry + excl;
      carry += total;
    }
    if (t == 0) {
      s_total_pages = carry;
      if ((int64_t)s_nf + carry > a.total_pages) s_fail = 1;
    }
  }
  __syncthreads();
  const bool fail = s_fail != 0;
  int32_t* cc = a.column_count + (int64_t)h * a.rchunk;
  if (tile == 0) {
    // rows whose band starts at position 0 see no admitted column; on a
    // failure no row does (the chunk then attends to its band only)
    for (int i = t; i < a.rchunk; i += kThreads)
      if (fail || (a.r0 + i) * kBlk - a.W + 1 <= 0) cc[i] = 0;
    if (fail && h == 0 && t == 0) {
      *a.status = WGKV_ERR_CAPACITY;
      *a.abort_flag = 1;
    }
  }
  if (fail) return;  // tile 0 of each head has zeroed its column counts

  // ---- this tile: stable compaction and column counts ----------------------
  const int gl0 = a.global_lengths[a.layer * a.H + h];
  const int first_new = (gl0 + a.page - 1) / a.page;  // index of the head's first new page
  const int page0 = s_nf + s_first[h];                  // its page id
  const int32_t* bt = a.block_table + ((int64_t)a.layer * a.H + h) * a.max_pages + lb;
  if (tile == 0) {
    const int n_h = s_tot[h];
    const int pages = (gl0 + n_h + a.page - 1) / a.page - first_new;
    int32_t* row = a.block_table + ((int64_t)a.layer * a.H + h) * a.max_pages + lb;
    for (int i = t; i < pages; i += kThreads) row[first_new + i] = page0 + i;
    if (t == 0) {
      a.adm[h] = n_h;
      a.gl_before[h] = gl0;
      if (h == 0) {
        *a.next_free_after = s_nf + s_total_pages;
        *a.abort_flag = 0;
      }
    }
  }
  const int base = a.c0 > 0 ? a.c0 - a.W : 0;  // global position of virtual index 0
  int cnt = 0;
#pragma unroll
  for (int k = 0; k < kPer; ++k) cnt += f[k] ? 1 : 0;
  const int incl = wave_incl_scan(cnt, lane);
  if (lane == 63) s_wave[wid] = incl;
  __syncthreads();
  int o = incl - cnt, total = 0;
#pragma unroll
  for (int w = 0; w < kWaves; ++w) {
    o += w < wid ? s_wave[w] : 0;
    total += s_wave[w];
  }
  const int before = gl0 + s_pre;
#pragma unroll
  for (int k = 0; k < kPer; ++k) {
    const int v = v0 + k;
    if (f[k]) {
      const int j = before + o;  // logical index in the head's global cache
      const int pi = j / a.page;
      const int pg = pi < first_new ? bt[pi] : page0 + (pi - first_new);
      s_src[o] = v;
      s_dst[o] = (int64_t)pg * a.page + j % a.page;
      ++o;
    }
    // o is now the inclusive count at v within the tile
    const int pp = base + v + 1;
    if (v < n_adm && pp > 0 && (pp + a.W - 1) % kBlk == 0) {
      const int r = (pp + a.W - 1) / kBlk;
      if (r >= a.r0 && r < a.r0 + a.rchunk) cc[r - a.r0] = before + o;
    }
  }
  __syncthreads();
  const int chunks = a.D / 8;
  const int64_t ring_base = ((int64_t)a.layer * a.H + h) * a.W;
  for (int e = t; e < total * chunks; e += kThreads) {
    const int r = e / chunks, c = e - r * chunks;
    const int v = s_src[r];
    u32x4_t kv, vv;
    if (v < nr) {
      kv = *(const u32x4_t*)(a.pool_k + (ring_base + v) * a.D + c * 8);
      vv = *(const u32x4_t*)(a.pool_v + (ring_base + v) * a.D + c * 8);
    } else {
      const int64_t off = (int64_t)h * a.kv_sh + (int64_t)(v - nr) * a.kv_ss + c * 8;
      kv = *(const u32x4_t*)(a.key + off);
      vv = *(const u32x4_t*)(a.value + off);
    }
    *(u32x4_t*)(a.pool_k + s_dst[r] * a.D + c * 8) = kv;
    *(u32x4_t*)(a.pool_v + s_dst[r] * a.D + c * 8) = vv;
  }
}

// After the chunk's attention: ring slot i <- chunk position C - W + i.
// Grid (head, 64-slot group).
__global__ __launch_bounds__(kThreads) void chunk_ring_kernel(ChunkArgs a) {
  if (*a.abort_flag) return;
  const int h = blockIdx.x;
  if (blockIdx.y == 0 && threadIdx.x == 0) {
    // stage 0's admissions become the head's global length (no kernel of
    // stage 0 could, since all of them read the length from before)
    a.global_lengths[a.layer * a.H + h] = a.gl_before[h] + a.adm[h];
    if (h == 0) *a.next_free = *a.next_free_after;
  }
  const int n_loc = min(a.W, a.c0 + a.C);
  const int first = a.C - n_loc;  // chunk row of slot 0
  const int i0 = blockIdx.y * kBlk, i1 = min(n_loc, i0 + kBlk);
  if (i0 >= i1) return;
  const int64_t ring_base = ((int64_t)a.layer * a.H + h) * a.W;
  const int chunks = a.D / 8;
  for (int e = threadIdx.x; e < (i1 - i0) * chunks; e += kThreads) {
    const int i = i0 + e / chunks, c = e % chunks;
    const int64_t off = (int64_t)h * a.kv_sh + (int64_t)(first + i) * a.kv_ss + c * 8;
    *(u32x4_t*)(a.pool_k + (ring_base + i) * a.D + c * 8) = *(const u32x4_t*)(a.key + off);
    *(u32x4_t*)(a.pool_v + (ring_base + i) * a.D + c * 8) = *(const u32x4_t*)(a.value + off);
    if (a.pre_key && a.local_pre_key) {
      const int64_t po = (int64_t)h * a.pk_sh + (int64_t)(first + i) * a.pk_ss + c * 8;
      *(u32x4_t*)(a.local_pre_key + (ring_base + i) * a.D + c * 8) = *(const u32x4_t*)(a.pre_key + po);
    }
  }
  for (int i = i0 + threadIdx.x; i < i1; i += kThreads)
    a.local_is_global[ring_base + i] = a.mask[(int64_t)h * a.m_sh + first + i] ? 1 : 0;
}

bool aligned16(const void* p) { return ((uintptr_t)p & 15) == 0; }

}  // namespace

extern "C" size_t wgkv_chunk_admit_workspace_bytes(int32_t num_kv_heads, int32_t chunk_len, int32_t local_window) {
  (void)chunk_len;
  (void)local_window;
  return (2 * (size_t)(num_kv_heads > 0 ? num_kv_heads : 0) + 16) * sizeof(int32_t);
}

extern "C" int wgkv_chunk_cache_update(
    int32_t stage,
    const void* key, const void* value, int64_t kv_stride_h, int64_t kv_stride_s,
    const void* pre_key, int64_t pk_stride_h, int64_t pk_stride_s,
    const uint8_t* g_mask, int64_t gm_stride_h,
    int32_t layer, int32_t num_layers, int32_t num_kv_heads, int32_t chunk_start, int32_t chunk_len, int32_t head_dim,
    int32_t local_window, int32_t page_size, int32_t max_tokens_per_head, int64_t total_pages,
    void* pool_k, void* pool_v, int32_t* block_table, int32_t max_pages_per_head,
    int32_t* global_lengths, uint8_t* local_is_global, void* local_pre_key,
    int32_t* next_free_block, int32_t* status, int32_t* column_count,
    void* workspace, size_t workspace_bytes, void* stream) {
  if (stage != 0 && stage != 1) return WGKV_ERR_ARG;
  if (!key || !value || !g_mask || !pool_k || !pool_v || !block_table || !global_lengths || !local_is_global ||
      !next_free_block || !status)
    return WGKV_ERR_ARG;
  if (stage == 0 && !column_count) return WGKV_ERR_ARG;
  if (num_kv_heads <= 0 || num_kv_heads > 1024 || layer < 0 || layer >= num_layers) return WGKV_ERR_ARG;
  if (chunk_start < 0 || chunk_len <= 0 || local_window <= 0 || page_size <= 0) return WGKV_ERR_ARG;
  if (local_window % kBlk || chunk_start % kBlk || local_window % page_size) return WGKV_ERR_ARG;
  if (chunk_start > 0 && (chunk_len < local_window || chunk_start < local_window)) return WGKV_ERR_ARG;
  if (head_dim % 8 || head_dim <= 0) return WGKV_ERR_UNSUPPORTED;
  if (!aligned16(key) || !aligned16(value) || !aligned16(pool_k) || !aligned16(pool_v)) return WGKV_ERR_UNSUPPORTED;
  if ((kv_stride_h | kv_stride_s) & 7) return WGKV_ERR_UNSUPPORTED;
  if (pre_key && (!aligned16(pre_key) || ((pk_stride_h | pk_stride_s) & 7))) return WGKV_ERR_UNSUPPORTED;
  if (!workspace || workspace_bytes < wgkv_chunk_admit_workspace_bytes(num_kv_heads, chunk_len, local_window))
    return WGKV_ERR_WORKSPACE;
  ChunkArgs a = {};
  a.key = (const uint16_t*)key;
  a.value = (const uint16_t*)value;
  a.kv_sh = kv_stride_h;
  a.kv_ss = kv_stride_s;
  a.pre_key = (const uint16_t*)pre_key;
  a.pk_sh = pk_stride_h;
  a.pk_ss = pk_stride_s;
  a.mask = g_mask;
  a.m_sh = gm_stride_h;
  a.layer = layer;
  a.H = num_kv_heads;
  a.C = chunk_len;
  a.D = head_dim;
  a.W = local_window;
  a.page = page_size;
  a.max_tokens_per_head = max_tokens_per_head;
  a.c0 = chunk_start;
  a.total_pages = total_pages;
  a.pool_k = (uint16_t*)pool_k;
  a.pool_v = (uint16_t*)pool_v;
  a.block_table = block_table;
  a.max_pages = max_pages_per_head;
  a.global_lengths = global_lengths;
  a.local_is_global = local_is_global;
  a.local_pre_key = (uint16_t*)local_pre_key;
  a.next_free = next_free_block;
  a.status = status;
  a.column_count = column_count;
  a.r0 = chunk_start / kBlk;
  a.rchunk = (chunk_len + kBlk - 1) / kBlk;
  const int vl = (chunk_start > 0 ? local_window : 0) + chunk_len;
  a.ntiles = (vl + kTile - 1) / kTile;
  a.mask_vec16 = (((uintptr_t)g_mask | (uintptr_t)gm_stride_h) & 15) == 0;
  int32_t* ws = (int32_t*)workspace;
  a.adm = ws;
  a.gl_before = ws + num_kv_heads;
  a.next_free_after = ws + 2 * (size_t)num_kv_heads;
  a.abort_flag = a.next_free_after + 1;
  hipStream_t st = (hipStream_t)stream;
  if (stage == 0) {
    hipLaunchKernelGGL(chunk_admit_kernel, dim3(a.ntiles, num_kv_heads), dim3(kThreads), 0, st, a);
  } else {
    const int groups = (min(local_window, chunk_start + chunk_len) + kBlk - 1) / kBlk;
    hipLaunchKernelGGL(chunk_ring_kernel, dim3(num_kv_heads, groups), dim3(kThreads), 0, st, a);
  }
  return hipGetLastError() == hipSuccess ? WGKV_OK : WGKV_ERR_HIP;
}
