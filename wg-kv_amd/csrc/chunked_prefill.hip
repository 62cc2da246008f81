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
  // workspace
  int ntiles;
  int32_t* tile_cnt;
  int32_t* tile_base;
  int32_t* gl_before;
  int32_t* abort_flag;
};

// Virtual sequence of a chunk: ring positions (c0 > 0 only) then the chunk.
__device__ __forceinline__ int vlen(const ChunkArgs& a) { return (a.c0 > 0 ? a.W : 0) + a.C; }
__device__ __forceinline__ int vring(const ChunkArgs& a) { return a.c0 > 0 ? a.W : 0; }

__device__ __forceinline__ bool vflag(const ChunkArgs& a, int h, int v) {
  const int nr = vring(a);
  if (v < nr) return a.local_is_global[((int64_t)a.layer * a.H + h) * a.W + v] != 0;
  return a.mask[(int64_t)h * a.m_sh + (v - nr)] != 0;
}

__global__ __launch_bounds__(kThreads) void chunk_count_kernel(ChunkArgs a) {
  __shared__ int s_red[kThreads];
  const int h = blockIdx.y, tile = blockIdx.x;
  const int n_adm = vlen(a) - a.W;  // admission range [0, n_adm) of the virtual sequence
  int cnt = 0;
  for (int v = tile * kTile + threadIdx.x; v < min(n_adm, (tile + 1) * kTile); v += kThreads) cnt += vflag(a, h, v);
  s_red[threadIdx.x] = cnt;
  __syncthreads();
  for (int off = kThreads / 2; off > 0; off >>= 1) {
    if (threadIdx.x < off) s_red[threadIdx.x] += s_red[threadIdx.x + off];
    __syncthreads();
  }
  if (threadIdx.x == 0) a.tile_cnt[h * a.ntiles + tile] = s_red[0];
}

// One workgroup: totals, capacity, page allocation (head order), lengths.
// Everything is checked before the first write.
__global__ __launch_bounds__(kThreads) void chunk_plan_kernel(ChunkArgs a) {
  __shared__ int s_tmp[kThreads];
  __shared__ int s_n[1024];
  __shared__ int s_first[1024];
  __shared__ int s_fail;
  const int t = threadIdx.x;
  if (t == 0) s_fail = 0;
  __syncthreads();
  const int lb = a.W / a.page;
  for (int h = t; h < a.H; h += kThreads) {
    int run = 0;
    for (int tl = 0; tl < a.ntiles; ++tl) {
      a.tile_base[h * a.ntiles + tl] = run;
      run += a.tile_cnt[h * a.ntiles + tl];
    }
    s_n[h] = run;
    const int gl = a.global_lengths[a.layer * a.H + h];
    if (run > 0 && (a.W + gl + run > a.max_tokens_per_head || lb + (gl + run + a.page - 1) / a.page > a.max_pages))
      atomicOr(&s_fail, 1);
  }
  __syncthreads();
  const int nf = *a.next_free;
  int carry = 0;
  for (int h0 = 0; h0 < a.H; h0 += kThreads) {
    const int h = h0 + t;
    int pages = 0;
    if (h < a.H) {
      const int gl = a.global_lengths[a.layer * a.H + h];
      pages = (gl + s_n[h] + a.page - 1) / a.page - (gl + a.page - 1) / a.page;
    }
    int total = 0;
    const int excl = block_exclusive_scan_256(pages, s_tmp, &total);
    if (h < a.H) s_first[h] = nf + carry + excl;
    carry += total;
  }
  if (t == 0 && (int64_t)nf + carry > a.total_pages) s_fail = 1;
  __syncthreads();
  // column counts the scatter does not write: rows whose band starts at
  // position 0 and, on failure, every row (the chunk then sees no columns)
  for (int e = t; e < a.H * a.rchunk; e += kThreads) {
    const int i = e % a.rchunk;
    if (s_fail || (a.r0 + i) * kBlk - a.W + 1 <= 0) a.column_count[e] = 0;
  }
  if (s_fail) {
    if (t == 0) {
      *a.status = WGKV_ERR_CAPACITY;
      *a.abort_flag = 1;
    }
    return;
  }
  for (int h = t; h < a.H; h += kThreads) {
    const int gl = a.global_lengths[a.layer * a.H + h];
    const int first_new = (gl + a.page - 1) / a.page;
    const int pages = (gl + s_n[h] + a.page - 1) / a.page - first_new;
    int32_t* row = a.block_table + ((int64_t)a.layer * a.H + h) * a.max_pages + lb;
    for (int i = 0; i < pages; ++i) row[first_new + i] = s_first[h] + i;
    a.gl_before[h] = gl;
    a.global_lengths[a.layer * a.H + h] = gl + s_n[h];
  }
  if (t == 0) {
    *a.next_free = nf + carry;
    *a.abort_flag = 0;
  }
}

// Stable compaction of the admission range into the heads' global pages, and
// column_count of the chunk's row blocks: the count of row block r is the
// number of admitted positions below p = 64 r - W + 1, i.e. the inclusive
// count at virtual index p - 1 - base, which falls in exactly one tile.
__global__ __launch_bounds__(kThreads) void chunk_scatter_kernel(ChunkArgs a) {
  constexpr int kPer = kTile / kThreads;
  __shared__ int s_tmp[kThreads];
  __shared__ int s_src[kTile];     // virtual index
  __shared__ int64_t s_dst[kTile]; // pool row
  if (*a.abort_flag) return;
  const int h = blockIdx.y, tile = blockIdx.x;
  const int t = threadIdx.x;
  const int nr = vring(a);
  const int n_adm = vlen(a) - a.W;
  const int lb = a.W / a.page;
  const int base = a.c0 > 0 ? a.c0 - a.W : 0;  // global position of virtual index 0
  const int32_t* bt = a.block_table + ((int64_t)a.layer * a.H + h) * a.max_pages + lb;
  const int gl0 = a.gl_before[h];
  const int v0 = tile * kTile + t * kPer;
  bool f[kPer];
  int cnt = 0;
#pragma unroll
  for (int k = 0; k < kPer; ++k) {
    const int v = v0 + k;
    f[k] = v < n_adm && vflag(a, h, v);
    cnt += f[k] ? 1 : 0;
  }
  int total = 0;
  int o = block_exclusive_scan_256(cnt, s_tmp, &total);
  const int before = gl0 + a.tile_base[h * a.ntiles + tile];
  int32_t* cc = a.column_count + (int64_t)h * a.rchunk;
#pragma unroll
  for (int k = 0; k < kPer; ++k) {
    const int v = v0 + k;
    if (f[k]) {
      const int j = before + o;  // logical index in the head's global cache
      s_src[o] = v;
      s_dst[o] = (int64_t)bt[j / a.page] * a.page + j % a.page;
      ++o;
    }
    // o is now the inclusive count at v within the tile
    const int p = base + v + 1;
    if (v < n_adm && p > 0 && (p + a.W - 1) % kBlk == 0) {
      const int r = (p + a.W - 1) / kBlk;
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
  const size_t ntiles = (size_t)(chunk_len + local_window + kTile - 1) / kTile;
  return (2 * (size_t)num_kv_heads * ntiles + (size_t)num_kv_heads + 16) * sizeof(int32_t);
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
  int32_t* ws = (int32_t*)workspace;
  a.tile_cnt = ws;
  a.tile_base = ws + (size_t)num_kv_heads * a.ntiles;
  a.gl_before = ws + 2 * (size_t)num_kv_heads * a.ntiles;
  a.abort_flag = a.gl_before + num_kv_heads;
  hipStream_t st = (hipStream_t)stream;
  if (stage == 0) {
    dim3 grid(a.ntiles, num_kv_heads);
    hipLaunchKernelGGL(chunk_count_kernel, grid, dim3(kThreads), 0, st, a);
    hipLaunchKernelGGL(chunk_plan_kernel, dim3(1), dim3(kThreads), 0, st, a);
    hipLaunchKernelGGL(chunk_scatter_kernel, grid, dim3(kThreads), 0, st, a);
  } else {
    const int groups = (min(local_window, chunk_start + chunk_len) + kBlk - 1) / kBlk;
    hipLaunchKernelGGL(chunk_ring_kernel, dim3(num_kv_heads, groups), dim3(kThreads), 0, st, a);
  }
  return hipGetLastError() == hipSuccess ? WGKV_OK : WGKV_ERR_HIP;
}
