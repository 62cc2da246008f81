// Dual-cache writes of the write-gated path (gfx950): admission at prefill
// (stable per-head compaction, bump-allocated pages, local ring) and the
// decode-step append (lazy promotion of the token leaving the ring, ring
// write, decode lengths).  All bookkeeping lives on the device; capacity is
// checked for the whole call before anything is written, and a failed check
// leaves the cache untouched and sets *status = WGKV_ERR_CAPACITY.
//
// Pool layout (the reference's, src/modeling_layers.py:1209-1216): one pool
// of total_pages*page rows of D bf16 per K and V; page p holds rows
// [p*page, p*page+page).  Local pages of (layer, head) are
// [(l*H + h)*W/page, ...) -- ring slot s of (l, h) is pool row (l*H + h)*W + s.
// block_table (L, H, max_pages): local pages first, then global pages in
// allocation order; unused entries hold the sentinel total_pages-1.
#include <string.h>

#include "wgkv_common.h"

namespace {

constexpr int kThreads = 256;
constexpr int kTile = 2048;  // positions per scatter workgroup (8 per thread)

struct AdmitArgs {
  const uint16_t* key;
  const uint16_t* value;
  int64_t kv_sh, kv_ss;
  const uint16_t* pre_key;
  int64_t pk_sh, pk_ss;
  const uint8_t* mask;
  int64_t m_sh;
  int layer, L, H, S, D, W, page, max_tokens_per_head;
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
  int ntiles;
  int32_t* tile_cnt;   // [H][ntiles]
  int32_t* tile_base;  // [H][ntiles] exclusive prefix within the head
  int64_t* head_row;   // [H] first pool row of the head's new global pages
  int32_t* abort_flag;
};

// Copies `n` rows of D bf16 (src row pointers / dst pool rows from LDS lists)
// with the whole workgroup, 16 bytes per thread per step.
__device__ void copy_rows(const uint16_t* __restrict__ base, int64_t ss, const int* s_src, const int64_t* s_dst,
                          int n, int D, uint16_t* __restrict__ dst_pool) {
  const int chunks = D / 8;
  for (int e = threadIdx.x; e < n * chunks; e += kThreads) {
    const int r = e / chunks, c = e - r * chunks;
    const u32x4_t v = *(const u32x4_t*)(base + (int64_t)s_src[r] * ss + c * 8);
    *(u32x4_t*)(dst_pool + s_dst[r] * D + c * 8) = v;
  }
}

__global__ __launch_bounds__(kThreads) void admit_count_kernel(AdmitArgs a) {
  __shared__ int s_red[kThreads];
  const int h = blockIdx.y, tile = blockIdx.x;
  const int n_early = max(0, a.S - a.W);
  const uint8_t* m = a.mask + (int64_t)h * a.m_sh;
  int cnt = 0;
  for (int p = tile * kTile + threadIdx.x; p < min(n_early, (tile + 1) * kTile); p += kThreads) cnt += m[p] != 0;
  s_red[threadIdx.x] = cnt;
  __syncthreads();
  for (int off = kThreads / 2; off > 0; off >>= 1) {
    if (threadIdx.x < off) s_red[threadIdx.x] += s_red[threadIdx.x + off];
    __syncthreads();
  }
  if (threadIdx.x == 0) a.tile_cnt[h * a.ntiles + tile] = s_red[0];
}

// One workgroup: per-head totals, capacity checks, page allocation in head
// order (src/modeling_layers.py:1303-1331), block-table rows, lengths.
__global__ __launch_bounds__(kThreads) void admit_plan_kernel(AdmitArgs a) {
  __shared__ int s_tmp[kThreads];
  __shared__ int s_n[1024];
  __shared__ int s_fail;
  const int t = threadIdx.x;
  if (t == 0) s_fail = 0;
  __syncthreads();
  const int n_loc = min(a.S, a.W);
  const int lb = a.W / a.page;
  // per-head totals and within-head tile prefixes (one thread per head)
  for (int h = t; h < a.H; h += kThreads) {
    int run = 0;
    for (int tl = 0; tl < a.ntiles; ++tl) {
      a.tile_base[h * a.ntiles + tl] = run;
      run += a.tile_cnt[h * a.ntiles + tl];
    }
    s_n[h] = run;
    if (run > 0 && (n_loc + run > a.max_tokens_per_head || lb + (run + a.page - 1) / a.page > a.max_pages))
      atomicOr(&s_fail, 1);
  }
  __syncthreads();
  // exclusive scan of pages over heads (H <= 1024, one pass per 256 heads)
  const int nf = *a.next_free;
  int carry = 0;
  for (int h0 = 0; h0 < a.H; h0 += kThreads) {
    const int h = h0 + t;
    const int pages = h < a.H ? (s_n[h] + a.page - 1) / a.page : 0;
    int total = 0;
    const int excl = block_exclusive_scan_256(pages, s_tmp, &total);
    if (h < a.H) a.head_row[h] = (int64_t)(nf + carry + excl) * a.page;
    carry += total;
  }
  if (t == 0 && (int64_t)nf + carry > a.total_pages) s_fail = 1;
  __syncthreads();
  if (s_fail) {
    if (t == 0) {
      *a.status = WGKV_ERR_CAPACITY;
      *a.abort_flag = 1;
    }
    return;
  }
  for (int h = t; h < a.H; h += kThreads) {
    const int n = s_n[h];
    if (n == 0) continue;
    const int first = (int)(a.head_row[h] / a.page);
    const int pages = (n + a.page - 1) / a.page;
    int32_t* row = a.block_table + ((int64_t)a.layer * a.H + h) * a.max_pages + lb;
    for (int i = 0; i < pages; ++i) row[i] = first + i;
    a.global_lengths[a.layer * a.H + h] = n;
  }
  if (t == 0) {
    *a.next_free = nf + carry;
    *a.abort_flag = 0;
  }
}

// Stable compaction of admitted positions of [0, S-W) into the head's pages,
// and the ring write of the last min(S, W) positions.
__global__ __launch_bounds__(kThreads) void admit_scatter_kernel(AdmitArgs a) {
  __shared__ int s_tmp[kThreads];
  __shared__ int s_src[kTile];
  __shared__ int64_t s_dst[kTile];
  __shared__ int s_n;
  if (*a.abort_flag) return;
  const int h = blockIdx.y, tile = blockIdx.x;
  const int t = threadIdx.x;
  const int n_early = max(0, a.S - a.W);
  const int n_loc = min(a.S, a.W);
  const uint8_t* m = a.mask + (int64_t)h * a.m_sh;
  const int p0 = tile * kTile + t * (kTile / kThreads);
  // global part: positions p0 .. p0+7 of this thread, in order
  int cnt = 0;
  for (int k = 0; k < kTile / kThreads; ++k) {
    const int p = p0 + k;
    cnt += (p < n_early && m[p]) ? 1 : 0;
  }
  int total = 0;
  int o = block_exclusive_scan_256(cnt, s_tmp, &total);
  const int64_t base_row = a.head_row[h] + a.tile_base[h * a.ntiles + tile];
  for (int k = 0; k < kTile / kThreads; ++k) {
    const int p = p0 + k;
    if (p < n_early && m[p]) {
      s_src[o] = p;
      s_dst[o] = base_row + o;
      ++o;
    }
  }
  __syncthreads();
  copy_rows(a.key + (int64_t)h * a.kv_sh, a.kv_ss, s_src, s_dst, total, a.D, a.pool_k);
  copy_rows(a.value + (int64_t)h * a.kv_sh, a.kv_ss, s_src, s_dst, total, a.D, a.pool_v);
  __syncthreads();
  // ring part: slot i <- position S - n_loc + i (src/modeling_layers.py:1290-1300)
  const int ring0 = a.S - n_loc;
  const int lo = max(ring0, tile * kTile), hi = min(a.S, (tile + 1) * kTile);
  if (t == 0) s_n = max(0, hi - lo);
  const int64_t local_base = ((int64_t)a.layer * a.H + h) * a.W;
  for (int p = lo + t; p < hi; p += kThreads) {
    const int slot = p - ring0;
    s_src[p - lo] = p;
    s_dst[p - lo] = local_base + slot;
    a.local_is_global[local_base + slot] = m[p] ? 1 : 0;
  }
  __syncthreads();
  const int nr = s_n;
  copy_rows(a.key + (int64_t)h * a.kv_sh, a.kv_ss, s_src, s_dst, nr, a.D, a.pool_k);
  copy_rows(a.value + (int64_t)h * a.kv_sh, a.kv_ss, s_src, s_dst, nr, a.D, a.pool_v);
  if (a.pre_key && a.local_pre_key) {
    // local_pre_key is (L, H, W, D): its row index equals the pool's ring row
    copy_rows(a.pre_key + (int64_t)h * a.pk_sh, a.pk_ss, s_src, s_dst, nr, a.D, a.local_pre_key);
  }
}

// ---------------------------------------------------------------------------
struct AppendArgs {
  const uint16_t* key;
  const uint16_t* value;
  int64_t kv_sh;
  const uint16_t* pre_key;
  int64_t pk_sh;
  const uint8_t* mask;
  int layer, L, H, D, W, page, max_tokens_per_head;
  int64_t total_pages;
  int local_ptr, local_length, do_migrate, do_write;
  int32_t* ring;  // device (local_ptr, local_length, last slot written), replacing the two above when set
  uint16_t* qmin;  // QUEST page key bounds (total_pages, D) or NULL
  uint16_t* qmax;
  int32_t* free_ids;    // SnapKV free page list (ids in release order) or NULL
  int32_t* free_count;  // its length (device)
  int advance;    // with ring: advance it after this layer's write (the last layer's call)
  uint16_t* pool_k;
  uint16_t* pool_v;
  int32_t* block_table;
  int max_pages;
  int32_t* global_lengths;
  uint8_t* local_is_global;
  uint16_t* local_pre_key;
  int32_t* next_free;
  int32_t* cache_seqlens;
  int32_t* status;
};

// One workgroup.  Lazy promotion (src/modeling_layers.py:674-763) of ring slot
// local_ptr of every flagged (layer, head), pages allocated in row-major
// (layer, head) order; then the ring write of this layer's token (:1390-1407)
// and cache_seqlens = current local length + global length (:1429-1432).
__global__ __launch_bounds__(kThreads) void decode_append_kernel(AppendArgs a) {
  __shared__ int s_tmp[kThreads];
  __shared__ int s_fail;
  const int t = threadIdx.x;
  const int LH = a.L * a.H;
  const int lb = a.W / a.page;
  int local_ptr = a.local_ptr, local_length = a.local_length, do_migrate = a.do_migrate;
  if (a.ring) {
    // ring pointers on the device; promotion only once the ring is full (:1470)
    local_ptr = a.ring[0];
    local_length = a.ring[1];
    do_migrate = do_migrate && local_length == a.W;
  }
  if (t == 0) s_fail = 0;
  __syncthreads();
  if (do_migrate) {
    // pass 1: checks
    int need_total = 0;
    for (int i0 = 0; i0 < LH; i0 += kThreads) {
      const int i = i0 + t;
      int need = 0;
      if (i < LH) {
        const bool flag = a.local_is_global[(int64_t)i * a.W + local_ptr] != 0;
        const int gl = a.global_lengths[i];
        if (flag && (a.W + gl + 1 > a.max_tokens_per_head || lb + gl / a.page >= a.max_pages)) atomicOr(&s_fail, 1);
        need = (flag && gl % a.page == 0) ? 1 : 0;
      }
      int total = 0;
      block_exclusive_scan_256(need, s_tmp, &total);
      need_total += total;
    }
    const int nf = *a.next_free;
    // freed pages are reused first: the last from_free entries of the list, in
    // list order, go to the first heads that need a page (:694-712)
    const int n_free = a.free_ids ? *a.free_count : 0;
    const int from_free = min(need_total, n_free);
    if (t == 0 && (int64_t)nf + (need_total - from_free) > a.total_pages) s_fail = 1;
    __syncthreads();
    if (s_fail) {
      if (t == 0) *a.status = WGKV_ERR_CAPACITY;
      return;
    }
    // pass 2: allocate, copy, lengths
    int carry = 0;
    for (int i0 = 0; i0 < LH; i0 += kThreads) {
      const int i = i0 + t;
      bool flag = false;
      int gl = 0, need = 0;
      if (i < LH) {
        flag = a.local_is_global[(int64_t)i * a.W + local_ptr] != 0;
        gl = a.global_lengths[i];
        need = (flag && gl % a.page == 0) ? 1 : 0;
      }
      int total = 0;
      const int excl = block_exclusive_scan_256(need, s_tmp, &total);
      if (flag) {
        int32_t* bt = a.block_table + (int64_t)i * a.max_pages + lb + gl / a.page;
        int pg;
        if (need) {
          const int rank = carry + excl;
          pg = rank < from_free ? a.free_ids[n_free - from_free + rank] : nf + (rank - from_free);
          *bt = pg;
        } else {
          pg = *bt;
        }
        const int64_t src = (int64_t)i * a.W + local_ptr;
        const int64_t dst = (int64_t)pg * a.page + gl % a.page;
        for (int c = 0; c < a.D / 8; ++c) {
          const u32x4_t kv = *(const u32x4_t*)(a.pool_k + src * a.D + c * 8);
          *(u32x4_t*)(a.pool_k + dst * a.D + c * 8) = kv;
          *(u32x4_t*)(a.pool_v + dst * a.D + c * 8) = *(const u32x4_t*)(a.pool_v + src * a.D + c * 8);
          if (a.qmin) {
            // QUEST page bounds (:744-761): a new page starts at the key, else min / max with it
            u32x4_t* mn = (u32x4_t*)(a.qmin + (int64_t)pg * a.D + c * 8);
            u32x4_t* mx = (u32x4_t*)(a.qmax + (int64_t)pg * a.D + c * 8);
            if (gl % a.page == 0) {
              *mn = kv;
              *mx = kv;
            } else {
              u32x4_t lo = *mn, hi = *mx;
#pragma unroll
              for (int e = 0; e < 4; ++e) {
                uint32_t l = lo[e], hh = hi[e];
#pragma unroll
                for (int half = 0; half < 2; ++half) {
                  const uint32_t sh = 16u * half;
                  const uint32_t x = (kv[e] >> sh) & 0xffffu;
                  const float xf = __uint_as_float(x << 16);
                  if (xf < __uint_as_float(((l >> sh) & 0xffffu) << 16)) l = (l & ~(0xffffu << sh)) | (x << sh);
                  if (xf > __uint_as_float(((hh >> sh) & 0xffffu) << 16)) hh = (hh & ~(0xffffu << sh)) | (x << sh);
                }
                lo[e] = l;
                hi[e] = hh;
              }
              *mn = lo;
              *mx = hi;
            }
          }
        }
        a.global_lengths[i] = gl + 1;
      }
      carry += total;
    }
    if (t == 0) {
      *a.next_free = nf + carry - from_free;
      if (a.free_ids) *a.free_count = n_free - from_free;
    }
    __syncthreads();
  }
  if (!a.do_write) return;
  // ring write of this layer's new token
  const int slot = local_length < a.W ? local_length : local_ptr;
  const int cur = local_length < a.W ? local_length + 1 : a.W;
  const int chunks = a.D / 8;
  for (int e = t; e < a.H * chunks; e += kThreads) {
    const int h = e / chunks, c = e - h * chunks;
    const int64_t row = ((int64_t)a.layer * a.H + h) * a.W + slot;
    *(u32x4_t*)(a.pool_k + row * a.D + c * 8) = *(const u32x4_t*)(a.key + (int64_t)h * a.kv_sh + c * 8);
    *(u32x4_t*)(a.pool_v + row * a.D + c * 8) = *(const u32x4_t*)(a.value + (int64_t)h * a.kv_sh + c * 8);
    if (a.mask == nullptr && a.pre_key && a.local_pre_key)
      *(u32x4_t*)(a.local_pre_key + row * a.D + c * 8) = *(const u32x4_t*)(a.pre_key + (int64_t)h * a.pk_sh + c * 8);
  }
  for (int h = t; h < a.H; h += kThreads) {
    const int64_t row = ((int64_t)a.layer * a.H + h) * a.W + slot;
    if (a.mask) a.local_is_global[row] = a.mask[h] ? 1 : 0;
    if (a.cache_seqlens) a.cache_seqlens[h] = cur + a.global_lengths[a.layer * a.H + h];
  }
  // the slot this step wrote, for decisions later in the step (the deferred
  // gate's window refresh when it is W-1, :1402-1405); ring[0..1] are not
  // touched here, so no thread's read of them races with this store
  if (a.ring && t == 0) a.ring[2] = slot;
  if (a.ring && a.advance) {
    // every thread has read the pointers above; advance them for the next step
    // (decode_wrapper's host update after the last layer, :1409-1413)
    __syncthreads();
    if (t == 0) {
      if (local_length < a.W) a.ring[1] = local_length + 1;
      else a.ring[0] = (local_ptr + 1) % a.W;
    }
  }
}

bool aligned16(const void* p) { return ((uintptr_t)p & 15) == 0; }

}  // namespace

extern "C" size_t wgkv_prefill_admit_workspace_bytes(int32_t num_kv_heads, int32_t seq_len) {
  const size_t ntiles = (size_t)(seq_len + kTile - 1) / kTile;
  return 2 * (size_t)num_kv_heads * ntiles * sizeof(int32_t) + (size_t)num_kv_heads * sizeof(int64_t) + 64;
}

extern "C" int wgkv_prefill_admit(
    const void* key, const void* value, int64_t kv_stride_h, int64_t kv_stride_s,
    const void* pre_key, int64_t pk_stride_h, int64_t pk_stride_s,
    const uint8_t* g_mask, int64_t gm_stride_h,
    int32_t layer, int32_t num_layers, int32_t num_kv_heads, int32_t seq_len, int32_t head_dim,
    int32_t local_window, int32_t page_size, int32_t max_tokens_per_head, int64_t total_pages,
    void* pool_k, void* pool_v, int32_t* block_table, int32_t max_pages_per_head,
    int32_t* global_lengths, uint8_t* local_is_global, void* local_pre_key,
    int32_t* next_free_block, int32_t* status,
    void* workspace, size_t workspace_bytes, void* stream) {
  if (!key || !value || !g_mask || !pool_k || !pool_v || !block_table || !global_lengths || !local_is_global ||
      !next_free_block || !status)
    return WGKV_ERR_ARG;
  if (num_kv_heads <= 0 || num_kv_heads > 1024 || seq_len <= 0 || layer < 0 || layer >= num_layers) return WGKV_ERR_ARG;
  if (page_size <= 0 || local_window <= 0 || local_window % page_size) return WGKV_ERR_ARG;
  if (head_dim % 8 || head_dim <= 0) return WGKV_ERR_UNSUPPORTED;
  if (!aligned16(key) || !aligned16(value) || !aligned16(pool_k) || !aligned16(pool_v)) return WGKV_ERR_UNSUPPORTED;
  if ((kv_stride_h | kv_stride_s) & 7) return WGKV_ERR_UNSUPPORTED;
  if (pre_key && (!aligned16(pre_key) || ((pk_stride_h | pk_stride_s) & 7))) return WGKV_ERR_UNSUPPORTED;
  if (local_pre_key && !aligned16(local_pre_key)) return WGKV_ERR_UNSUPPORTED;
  if ((int64_t)num_layers * num_kv_heads * (local_window / page_size) > total_pages) return WGKV_ERR_ARG;
  if (!workspace || workspace_bytes < wgkv_prefill_admit_workspace_bytes(num_kv_heads, seq_len)) return WGKV_ERR_WORKSPACE;
  AdmitArgs a;
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
  a.L = num_layers;
  a.H = num_kv_heads;
  a.S = seq_len;
  a.D = head_dim;
  a.W = local_window;
  a.page = page_size;
  a.max_tokens_per_head = max_tokens_per_head;
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
  a.ntiles = (seq_len + kTile - 1) / kTile;
  char* ws = (char*)workspace;
  a.head_row = (int64_t*)ws;
  ws += (size_t)num_kv_heads * sizeof(int64_t);
  a.tile_cnt = (int32_t*)ws;
  ws += (size_t)num_kv_heads * a.ntiles * sizeof(int32_t);
  a.tile_base = (int32_t*)ws;
  ws += (size_t)num_kv_heads * a.ntiles * sizeof(int32_t);
  a.abort_flag = (int32_t*)ws;
  hipStream_t st = (hipStream_t)stream;
  dim3 grid(a.ntiles, num_kv_heads);
  hipLaunchKernelGGL(admit_count_kernel, grid, dim3(kThreads), 0, st, a);
  hipLaunchKernelGGL(admit_plan_kernel, dim3(1), dim3(kThreads), 0, st, a);
  hipLaunchKernelGGL(admit_scatter_kernel, grid, dim3(kThreads), 0, st, a);
  return hipGetLastError() == hipSuccess ? WGKV_OK : WGKV_ERR_HIP;
}

namespace {

int decode_append_launch(
    const void* key, const void* value, int64_t kv_stride_h,
    const void* pre_key, int64_t pk_stride_h,
    const uint8_t* g_mask,
    int32_t layer, int32_t num_layers, int32_t num_kv_heads, int32_t head_dim,
    int32_t local_window, int32_t page_size, int32_t max_tokens_per_head, int64_t total_pages,
    int32_t local_ptr, int32_t local_length, int32_t* ring_state, int32_t advance, int32_t do_migrate, int32_t do_write,
    void* pool_k, void* pool_v, int32_t* block_table, int32_t max_pages_per_head,
    int32_t* global_lengths, uint8_t* local_is_global, void* local_pre_key,
    int32_t* next_free_block, int32_t* cache_seqlens, int32_t* status,
    void* quest_key_min, void* quest_key_max, int32_t* free_ids, int32_t* free_count,
    void* stream) {
  if (do_write && (!key || !value)) return WGKV_ERR_ARG;
  if ((free_ids == nullptr) != (free_count == nullptr)) return WGKV_ERR_ARG;
  if (!pool_k || !pool_v || !block_table || !global_lengths || !local_is_global ||
      !next_free_block || !status)
    return WGKV_ERR_ARG;
  if (num_kv_heads <= 0 || layer < 0 || layer >= num_layers) return WGKV_ERR_ARG;
  if (page_size <= 0 || local_window <= 0 || local_window % page_size) return WGKV_ERR_ARG;
  if (!ring_state && (local_ptr < 0 || local_ptr >= local_window || local_length < 0 || local_length > local_window))
    return WGKV_ERR_ARG;
  if (do_write && !g_mask && (!pre_key || !local_pre_key)) return WGKV_ERR_ARG;  // deferred gating stores pre_key
  if (head_dim % 8 || head_dim <= 0) return WGKV_ERR_UNSUPPORTED;
  if (!aligned16(pool_k) || !aligned16(pool_v)) return WGKV_ERR_UNSUPPORTED;
  if (do_write && (!aligned16(key) || !aligned16(value) || (kv_stride_h & 7))) return WGKV_ERR_UNSUPPORTED;
  if (pre_key && (!aligned16(pre_key) || (pk_stride_h & 7))) return WGKV_ERR_UNSUPPORTED;
  AppendArgs a;
  a.key = (const uint16_t*)key;
  a.value = (const uint16_t*)value;
  a.kv_sh = kv_stride_h;
  a.pre_key = (const uint16_t*)pre_key;
  a.pk_sh = pk_stride_h;
  a.mask = g_mask;
  a.layer = layer;
  a.L = num_layers;
  a.H = num_kv_heads;
  a.D = head_dim;
  a.W = local_window;
  a.page = page_size;
  a.max_tokens_per_head = max_tokens_per_head;
  a.total_pages = total_pages;
  a.local_ptr = local_ptr;
  a.local_length = local_length;
  a.ring = ring_state;
  a.advance = advance;
  if ((quest_key_min == nullptr) != (quest_key_max == nullptr)) return WGKV_ERR_ARG;
  if (((uintptr_t)quest_key_min | (uintptr_t)quest_key_max) & 15) return WGKV_ERR_UNSUPPORTED;
  a.qmin = (uint16_t*)quest_key_min;
  a.qmax = (uint16_t*)quest_key_max;
  a.free_ids = free_ids;
  a.free_count = free_count;
  a.do_migrate = do_migrate;
  a.do_write = do_write;
  a.pool_k = (uint16_t*)pool_k;
  a.pool_v = (uint16_t*)pool_v;
  a.block_table = block_table;
  a.max_pages = max_pages_per_head;
  a.global_lengths = global_lengths;
  a.local_is_global = local_is_global;
  a.local_pre_key = (uint16_t*)local_pre_key;
  a.next_free = next_free_block;
  a.cache_seqlens = cache_seqlens;
  a.status = status;
  hipLaunchKernelGGL(decode_append_kernel, dim3(1), dim3(kThreads), 0, (hipStream_t)stream, a);
  return hipGetLastError() == hipSuccess ? WGKV_OK : WGKV_ERR_HIP;
}

}  // namespace

extern "C" int wgkv_decode_append(
    const void* key, const void* value, int64_t kv_stride_h,
    const void* pre_key, int64_t pk_stride_h,
    const uint8_t* g_mask,
    int32_t layer, int32_t num_layers, int32_t num_kv_heads, int32_t head_dim,
    int32_t local_window, int32_t page_size, int32_t max_tokens_per_head, int64_t total_pages,
    int32_t local_ptr, int32_t local_length, int32_t do_migrate, int32_t do_write,
    void* pool_k, void* pool_v, int32_t* block_table, int32_t max_pages_per_head,
    int32_t* global_lengths, uint8_t* local_is_global, void* local_pre_key,
    int32_t* next_free_block, int32_t* cache_seqlens, int32_t* status,
    void* quest_key_min, void* quest_key_max, int32_t* free_ids, int32_t* free_count,
    void* stream) {
  return decode_append_launch(key, value, kv_stride_h, pre_key, pk_stride_h, g_mask, layer, num_layers, num_kv_heads,
                              head_dim, local_window, page_size, max_tokens_per_head, total_pages, local_ptr,
                              local_length, nullptr, 0, do_migrate, do_write, pool_k, pool_v, block_table,
                              max_pages_per_head, global_lengths, local_is_global, local_pre_key, next_free_block,
                              cache_seqlens, status, quest_key_min, quest_key_max, free_ids, free_count, stream);
}

extern "C" int wgkv_decode_append_ring(
    const void* key, const void* value, int64_t kv_stride_h,
    const void* pre_key, int64_t pk_stride_h,
    const uint8_t* g_mask,
    int32_t layer, int32_t num_layers, int32_t num_kv_heads, int32_t head_dim,
    int32_t local_window, int32_t page_size, int32_t max_tokens_per_head, int64_t total_pages,
    int32_t* ring_state, int32_t advance, int32_t do_migrate, int32_t do_write,
    void* pool_k, void* pool_v, int32_t* block_table, int32_t max_pages_per_head,
    int32_t* global_lengths, uint8_t* local_is_global, void* local_pre_key,
    int32_t* next_free_block, int32_t* cache_seqlens, int32_t* status,
    void* quest_key_min, void* quest_key_max, int32_t* free_ids, int32_t* free_count,
    void* stream) {
  if (!ring_state) return WGKV_ERR_ARG;
  return decode_append_launch(key, value, kv_stride_h, pre_key, pk_stride_h, g_mask, layer, num_layers, num_kv_heads,
                              head_dim, local_window, page_size, max_tokens_per_head, total_pages, 0, 0, ring_state,
                              advance, do_migrate, do_write, pool_k, pool_v, block_table, max_pages_per_head,
                              global_lengths, local_is_global, local_pre_key, next_free_block, cache_seqlens, status,
                              quest_key_min, quest_key_max, free_ids, free_count, stream);
}

// ---- random admission (the reference's random_sparsity ablation) -----------
// get_random_g_scores (src/modeling_layers.py:1160-1166) draws r ~ U[0,1) per
// token and admits it iff r >= random_sparsity; the deferred refresh applies
// it to the whole window (:1177-1178).  Here the draws come from a
// counter-based generator so that a decode step can make them on the device,
// inside a captured graph, conditioned on a device flag: token (h, i) of draw
// number c takes the SplitMix64 finaliser (Steele, Lea, Flood, "Fast
// splittable pseudorandom number generators", OOPSLA 2014) of
// seed + (c * 2^32 + h * n + i + 1) * golden-ratio increment, and r is its top
// 24 bits / 2^24.  One workgroup per call: it reads the draw counter, writes
// the flags, then advances the counter, so consecutive calls draw fresh
// numbers and replays of a graph continue the same sequence as eager calls.
namespace {

__device__ __forceinline__ uint64_t splitmix64(uint64_t z) {
  z = (z ^ (z >> 30)) * 0xBF58476D1CE4E5B9ull;
  z = (z ^ (z >> 27)) * 0x94D049BB133111EBull;
  return z ^ (z >> 31);
}

__global__ __launch_bounds__(1024) void random_admission_kernel(uint8_t* flags, int64_t f_sh, int H, int n,
                                                                float cut, uint64_t seed, int32_t* counter,
                                                                const int32_t* active, int active_value) {
  if (active != nullptr && *active != active_value) return;
  __shared__ int s_c;
  if (threadIdx.x == 0) s_c = *counter;
  __syncthreads();
  const uint64_t base = seed + ((uint64_t)(uint32_t)s_c << 32);
  for (int j = threadIdx.x; j < H * n; j += blockDim.x) {
    const int h = j / n, i = j - h * n;
    const uint64_t z = splitmix64(base + (uint64_t)(j + 1) * 0x9E3779B97F4A7C15ull);
    const float r = (float)(z >> 40) * (1.0f / 16777216.0f);
    flags[(int64_t)h * f_sh + i] = r >= cut ? 1 : 0;
  }
  __syncthreads();
  if (threadIdx.x == 0) *counter = s_c + 1;
}

// Round-to-nearest-even f32 -> bf16 -> f32 on the host (finite values).
float host_bf16(float f) {
  uint32_t u;
  memcpy(&u, &f, 4);
  u += 0x7fffu + ((u >> 16) & 1u);
  u &= 0xffff0000u;
  memcpy(&f, &u, 4);
  return f;
}

}  // namespace

extern "C" int wgkv_random_admission(uint8_t* flags, int64_t flags_stride_h, int32_t num_kv_heads, int32_t n,
                                     float random_sparsity, uint64_t seed, int32_t* draw_counter,
                                     const int32_t* active_flag, int32_t active_value, void* stream) {
  if (!flags || !draw_counter || num_kv_heads <= 0 || n <= 0 || flags_stride_h < n) return WGKV_ERR_ARG;
  if (!(random_sparsity >= 0.f && random_sparsity <= 1.f)) return WGKV_ERR_ARG;
  // the reference compares its bf16 draws with the Python float, which the
  // comparison rounds to bf16
  const float cut = host_bf16(random_sparsity);
  hipLaunchKernelGGL(random_admission_kernel, dim3(1), dim3(1024), 0, (hipStream_t)stream, flags, flags_stride_h,
                     num_kv_heads, n, cut, seed, draw_counter, active_flag, active_value);
  return hipGetLastError() == hipSuccess ? WGKV_OK : WGKV_ERR_HIP;
}
