// SnapKV eviction on the device (gfx950): scoring, selection, packing and
// page release for every (layer, KV head) in four launches with no host
// synchronisation.
//
// Replaces snapkv_evict (src/modeling_layers.py:595-671) and its trigger
// (:1500-1507).  Per (layer l, KV head h) with n global tokens and
// n_evict = int(n * ratio) > 0 (heads with n_evict == 0 are skipped, :604):
//   x[g][w][i] = q(l, w, h*G + g) . k_i * scale      (bf16 logits: the
//                reference multiplies in bf16, so x = bf16(bf16(q.k) * scale))
//   p = softmax over i (fp32), s[i] = mean_w max_g p[g][w][i]
//   pooled[i] = max(s[i - k/2 .. i + k/2] within [0, n))  (max_pool1d, stride 1)
//   drop the n_evict lowest pooled scores (equal scores: lower position
//   first -- torch.topk leaves their order unspecified), pack the kept
//   tokens in order into the head's first pages, release the head's pages
//   past the kept length to the free list (heads in (layer, head) order,
//   pages in table order) and reset their table entries.
// The eviction runs only when the sum of all global lengths exceeds
// max_cached_tokens, decided on the device.
//
// Launches (one stream):
//   1 snapkv_rowstats_kernel  trigger + per query row (g, w) the softmax max
//                             and sum over the head's keys (online, MFMA)
//   2 snapkv_scores_kernel    per key: mean over w of max over g of p (MFMA)
//   3 snapkv_select_kernel    one workgroup per head: radix select of the
//                             n_evict-th smallest pooled score, tie ranks,
//                             in-place ordered compaction of K and V
//   4 snapkv_release_kernel   free-list append and table reset per head
#include "wgkv_common.h"

namespace {

constexpr float kLog2e = 1.4426950408889634f;
constexpr int kSelectThreads = 1024;
constexpr int kMoveTokens = 256;  // tokens per compaction step (4 threads each)

struct SnapArgs {
  uint16_t* pool_k;
  uint16_t* pool_v;
  int32_t* block_table;
  int32_t* global_lengths;
  int32_t* free_ids;
  int32_t* free_count;
  const uint16_t* qwin;  // (L, win, Hq, D) bf16
  int L, H, G, D, P, pshift, lb, max_pages, total_pages, mtph, win, win_pad, ksz;
  double ratio;
  float scale;
  int64_t max_cached;
  int logits_bf16;
  int32_t* state;     // [0] evicted on this call, [1] evictions so far
  float* scores_out;  // optional pooled scores (L*H, mtph)
  // workspace
  int32_t* meta;  // [0] triggered, [1] free list length before the call
  float* stats;   // (L*H, G, win_pad, 2): softmax max and 1/sum per query row
  float* base;    // (L*H, mtph): unpooled scores
  int32_t* rel;   // (L*H): pages released
  int32_t* newp;  // (L*H): global pages kept
};

// The four logits of an MFMA output fragment of fp32 product sums:
// bf16(bf16(acc) * scale) as the reference's bf16 matmul and scalar multiply
// round them (two values per conversion), or acc * scale.
__device__ __forceinline__ void logits4(const f32x4_t& c, const SnapArgs& a, float (&x)[4]) {
  if (a.logits_bf16) {
#pragma unroll
    for (int i = 0; i < 4; i += 2) {
      const uint32_t r = pack_bf16x2(c[i], c[i + 1]);
      const uint32_t y = pack_bf16x2(bf16lo(r) * a.scale, bf16hi(r) * a.scale);
      x[i] = bf16lo(y);
      x[i + 1] = bf16hi(y);
    }
  } else {
#pragma unroll
    for (int i = 0; i < 4; ++i) x[i] = c[i] * a.scale;
  }
}

__device__ __forceinline__ int n_evict_of(const SnapArgs& a, int n) { return (int)((double)n * a.ratio); }

// Pool row of logical token i of a head (pages of P = 1 << pshift tokens).
__device__ __forceinline__ int64_t row_of(const SnapArgs& a, const int32_t* bt, int i) {
  return ((int64_t)bt[a.lb + (i >> a.pshift)] << a.pshift) + (i & (a.P - 1));
}

__device__ __forceinline__ const uint16_t* key_row(const SnapArgs& a, const int32_t* bt, int i) {
  return a.pool_k + row_of(a, bt, i) * a.D;
}

// ---- 1: trigger and softmax row statistics ----------------------------------
// grid (G * win_pad / 256, L*H), 256 threads: wave w of the workgroup takes
// the 64 windows wb*256 + 64w .. +63 of group member g (four 16-row MFMA
// blocks, the A operands held in registers) and streams the head's keys in
// tiles of 64 (four 16-key column blocks, each K fragment serving the four
// row blocks), keeping per row the running max and the sum of
// exp2((x - max) * log2 e).
template <int D>
__global__ __launch_bounds__(256) void snapkv_rowstats_kernel(SnapArgs a) {
  __shared__ int64_t s_sum[4];
  const int t = threadIdx.x, lane = t & 63, wid = t >> 6;
  const int LH = a.L * a.H;
  int64_t part = 0;
  for (int i = t; i < LH; i += 256) part += a.global_lengths[i];
#pragma unroll
  for (int off = 32; off > 0; off >>= 1) part += __shfl_xor(part, off, 64);
  if (lane == 0) s_sum[wid] = part;
  __syncthreads();
  const int64_t total = (s_sum[0] + s_sum[1]) + (s_sum[2] + s_sum[3]);
  const bool trig = total > a.max_cached;
  if (blockIdx.x == 0 && blockIdx.y == 0 && t == 0) {
    a.meta[0] = trig ? 1 : 0;
    a.meta[1] = a.free_count ? *a.free_count : 0;
    a.state[0] = trig ? 1 : 0;
    if (trig) a.state[1] += 1;
  }
  if (!trig) return;
  const int lh = blockIdx.y;
  const int n = a.global_lengths[lh];
  if (n_evict_of(a, n) == 0) return;
  const int wblocks = a.win_pad / 256;
  const int g = blockIdx.x / wblocks, wb = blockIdx.x - g * wblocks;
  const int w0 = wb * 256 + wid * 64;
  if (w0 >= a.win) return;
  const int l = lh / a.H, h = lh - l * a.H;
  const int n16 = lane & 15, kg = lane >> 4;
  constexpr int KS = D / 32;
  const int32_t* bt = a.block_table + (int64_t)lh * a.max_pages;
  // A fragments of the four row blocks: query rows w0 + 16rb + n16 (rows past the window repeat the last)
  bf16x8_t q[4][KS];
#pragma unroll
  for (int rb = 0; rb < 4; ++rb) {
    const int w = min(w0 + rb * 16 + n16, a.win - 1);
    const uint16_t* qrow = a.qwin + (((int64_t)l * a.win + w) * (a.H * a.G) + h * a.G + g) * D + kg * 8;
#pragma unroll
    for (int ks = 0; ks < KS; ++ks) q[rb][ks] = __builtin_bit_cast(bf16x8_t, *(const u32x4_t*)(qrow + ks * 32));
  }
  // per lane and row: the running max over this lane's keys and the sum of
  // exp2((x - max) log2 e) over them; the 16 lanes of a row combine at the end
  float m[4][4], s[4][4];
#pragma unroll
  for (int rb = 0; rb < 4; ++rb)
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      m[rb][i] = -INFINITY;
      s[rb][i] = 0.f;
    }
  // the K fragments of the next tile are loaded while this tile computes
  u32x4_t bk[4][KS];
  auto load_tile = [&](int k0) {
#pragma unroll
    for (int kb = 0; kb < 4; ++kb) {
      const uint16_t* kr = key_row(a, bt, min(k0 + kb * 16 + n16, n - 1)) + kg * 8;
#pragma unroll
      for (int ks = 0; ks < KS; ++ks) bk[kb][ks] = *(const u32x4_t*)(kr + ks * 32);
    }
  };
  load_tile(0);
  for (int k0 = 0; k0 < n; k0 += 64) {
    f32x4_t c[4][4];  // [row block][key block]
#pragma unroll
    for (int kb = 0; kb < 4; ++kb)
#pragma unroll
      for (int rb = 0; rb < 4; ++rb) {
        c[rb][kb] = (f32x4_t){0.f, 0.f, 0.f, 0.f};
#pragma unroll
        for (int ks = 0; ks < KS; ++ks)
          c[rb][kb] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(q[rb][ks], __builtin_bit_cast(bf16x8_t, bk[kb][ks]),
                                                              c[rb][kb], 0, 0, 0);
      }
    if (k0 + 64 < n) load_tile(k0 + 64);
#pragma unroll
    for (int rb = 0; rb < 4; ++rb) {
      float x[4][4];  // [key block][row]
#pragma unroll
      for (int kb = 0; kb < 4; ++kb) {
        logits4(c[rb][kb], a, x[kb]);
        if (k0 + kb * 16 + n16 >= n)
#pragma unroll
          for (int i = 0; i < 4; ++i) x[kb][i] = -INFINITY;
      }
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const float mx = fmaxf(fmaxf(x[0][i], x[1][i]), fmaxf(x[2][i], x[3][i]));
        const float mn = fmaxf(m[rb][i], mx);
        if (mn == -INFINITY) continue;  // no valid key of this lane yet
        const float ml = mn * kLog2e;
        float e = 0.f;
#pragma unroll
        for (int kb = 0; kb < 4; ++kb) e += fast_exp2(fmaf(x[kb][i], kLog2e, -ml));
        s[rb][i] = fmaf(s[rb][i], fast_exp2(fmaf(m[rb][i], kLog2e, -ml)), e);
        m[rb][i] = mn;
      }
    }
  }
  // combine the 16 lanes of each row: M = max, S = sum of s * exp2((m - M) log2 e)
#pragma unroll
  for (int rb = 0; rb < 4; ++rb)
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const float M = row_max16(m[rb][i]);  // finite: key 0 is valid
      const float part = m[rb][i] == -INFINITY ? 0.f : s[rb][i] * fast_exp2((m[rb][i] - M) * kLog2e);
      m[rb][i] = M;
      s[rb][i] = row_sum16(part);
    }
  if (n16 == 0) {
#pragma unroll
    for (int rb = 0; rb < 4; ++rb)
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const int w = w0 + rb * 16 + 4 * kg + i;
        if (w < a.win) {
          float* st = a.stats + (((int64_t)lh * a.G + g) * a.win_pad + w) * 2;
          st[0] = m[rb][i];
          st[1] = 1.0f / s[rb][i];
        }
      }
  }
}

// ---- 2: per-key scores ------------------------------------------------------
// grid (NB, L*H), 256 threads: workgroups stride over the head's 256-key
// tiles, wave w taking keys tile*256 + 64w .. +63 as four 16-key MFMA column
// blocks (the B operands, held in registers); for each 16-window block and
// group member one A fragment (the 16 window queries) serves the four
// blocks: the logits, p = exp2((x - max) log2 e) / sum per row, the max over
// group members, and the sum over windows accumulates per lane.
template <int D>
__global__ __launch_bounds__(256) void snapkv_scores_kernel(SnapArgs a) {
  if (a.meta[0] == 0) return;
  const int lh = blockIdx.y;
  const int n = a.global_lengths[lh];
  if (n_evict_of(a, n) == 0) return;
  const int t = threadIdx.x, lane = t & 63, wid = t >> 6;
  const int l = lh / a.H, h = lh - l * a.H;
  const int n16 = lane & 15, kg = lane >> 4;
  constexpr int KS = D / 32;
  const int32_t* bt = a.block_table + (int64_t)lh * a.max_pages;
  const int Hq = a.H * a.G;
  const float inv_win = 1.0f / (float)a.win;
  for (int tile = blockIdx.x; tile * 256 < n; tile += gridDim.x) {
    const int kbase = tile * 256 + wid * 64;
    if (kbase >= n) continue;
    bf16x8_t bk[4][KS];
#pragma unroll
    for (int kb = 0; kb < 4; ++kb) {
      const uint16_t* kr = key_row(a, bt, min(kbase + kb * 16 + n16, n - 1)) + kg * 8;
#pragma unroll
      for (int ks = 0; ks < KS; ++ks) bk[kb][ks] = __builtin_bit_cast(bf16x8_t, *(const u32x4_t*)(kr + ks * 32));
    }
    float acc[4][4] = {};
    for (int w0 = 0; w0 < a.win; w0 += 16) {
      float pmax[4][4] = {};
      const int wq = min(w0 + n16, a.win - 1);
      for (int g = 0; g < a.G; ++g) {
        const uint16_t* qrow = a.qwin + (((int64_t)l * a.win + wq) * Hq + h * a.G + g) * D + kg * 8;
        bf16x8_t q[KS];
#pragma unroll
        for (int ks = 0; ks < KS; ++ks) q[ks] = __builtin_bit_cast(bf16x8_t, *(const u32x4_t*)(qrow + ks * 32));
        const float* st = a.stats + (((int64_t)lh * a.G + g) * a.win_pad + w0 + 4 * kg) * 2;
        const f32x4_t s01 = *(const f32x4_t*)st, s23 = *(const f32x4_t*)(st + 4);  // rows 4kg .. 4kg+3 (in win_pad)
        const float ml[4] = {s01[0] * kLog2e, s01[2] * kLog2e, s23[0] * kLog2e, s23[2] * kLog2e};
        const float irow[4] = {s01[1], s01[3], s23[1], s23[3]};
#pragma unroll
        for (int kb = 0; kb < 4; ++kb) {
          f32x4_t c = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
          for (int ks = 0; ks < KS; ++ks) c = __builtin_amdgcn_mfma_f32_16x16x32_bf16(q[ks], bk[kb][ks], c, 0, 0, 0);
          float x[4];
          logits4(c, a, x);
#pragma unroll
          for (int i = 0; i < 4; ++i) {
            const float p = fast_exp2(fmaf(x[i], kLog2e, -ml[i])) * irow[i];
            pmax[kb][i] = w0 + 4 * kg + i < a.win ? fmaxf(pmax[kb][i], p) : 0.f;
          }
        }
      }
#pragma unroll
      for (int kb = 0; kb < 4; ++kb)
#pragma unroll
        for (int i = 0; i < 4; ++i) acc[kb][i] += pmax[kb][i];
    }
#pragma unroll
    for (int kb = 0; kb < 4; ++kb) {
      float tot = (acc[kb][0] + acc[kb][1]) + (acc[kb][2] + acc[kb][3]);
      tot += __shfl_xor(tot, 16, 64);
      tot += __shfl_xor(tot, 32, 64);
      const int key = kbase + kb * 16 + n16;
      if (kg == 0 && key < n) a.base[(int64_t)lh * a.mtph + key] = tot * inv_win;
    }
  }
}

// ---- 3: selection and compaction --------------------------------------------
__device__ __forceinline__ uint32_t pooled_key(const SnapArgs& a, const float* base, int n, int i) {
  float v = base[i];
  const int r = a.ksz / 2;
  for (int d = 1; d <= r; ++d) {
    if (i - d >= 0) v = fmaxf(v, base[i - d]);
    if (i + d < n) v = fmaxf(v, base[i + d]);
  }
  return __float_as_uint(v);  // scores are >= +0: the bit patterns sort as the values
}

// Exclusive scan of one int per thread over the first 256 threads (waves 0-3)
// with the total; s_w holds 4 ints.  Called by all threads (barriers inside).
__device__ __forceinline__ int scan256(int v, int t, int* s_w, int* total) {
  const int lane = t & 63, wid = t >> 6;
  const int incl = wave_incl_scan(v, lane);
  if (wid < 4 && lane == 63) s_w[wid] = incl;
  __syncthreads();
  int off = 0;
#pragma unroll
  for (int w = 0; w < 4; ++w) off += (w < wid) ? s_w[w] : 0;
  *total = (s_w[0] + s_w[1]) + (s_w[2] + s_w[3]);
  __syncthreads();
  return off + incl - v;
}

template <int D>
__global__ __launch_bounds__(kSelectThreads) void snapkv_select_kernel(SnapArgs a) {
  __shared__ int s_hist[256];
  __shared__ int s_bin, s_k;
  __shared__ int s_w[4];
  __shared__ int s_dest[kMoveTokens];
  if (a.meta[0] == 0) return;
  const int lh = blockIdx.x;
  const int t = threadIdx.x, lane = t & 63, wid = t >> 6;
  const int n = a.global_lengths[lh];
  const int n_evict = n_evict_of(a, n);
  if (n_evict == 0) {
    if (t == 0) {
      a.rel[lh] = 0;
      a.newp[lh] = (n + a.P - 1) / a.P;
    }
    return;
  }
  const float* base = a.base + (int64_t)lh * a.mtph;
  const int32_t* bt = a.block_table + (int64_t)lh * a.max_pages;
  // radix select, 8 bits per pass from the top: T = the n_evict-th smallest key
  uint32_t prefix = 0, pmask = 0;
  int k = n_evict;  // rank within the keys matching prefix
  for (int shift = 24; shift >= 0; shift -= 8) {
    for (int i = t; i < 256; i += kSelectThreads) s_hist[i] = 0;
    __syncthreads();
    for (int i = t; i < n; i += kSelectThreads) {
      const uint32_t u = pooled_key(a, base, n, i);
      if (shift == 24 && a.scores_out) a.scores_out[(int64_t)lh * a.mtph + i] = __uint_as_float(u);
      if ((u & pmask) == prefix) atomicAdd(&s_hist[(u >> shift) & 255], 1);
    }
    __syncthreads();
    if (wid == 0) {
      // lane holds bins 4*lane .. 4*lane+3
      int hb[4], sum = 0;
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        hb[j] = s_hist[4 * lane + j];
        sum += hb[j];
      }
      const int excl = wave_incl_scan(sum, lane) - sum;
      int run = excl;
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        if (run < k && k <= run + hb[j]) {
          s_bin = 4 * lane + j;
          s_k = k - run;
        }
        run += hb[j];
      }
    }
    __syncthreads();
    prefix |= (uint32_t)s_bin << shift;
    pmask |= 255u << shift;
    k = s_k;
    __syncthreads();
  }
  const uint32_t T = prefix;
  const int need_ties = k;  // keys equal to T that are dropped, lowest positions first
  // ordered compaction, kMoveTokens tokens per step
  constexpr int PARTS = 4;                 // threads per token
  constexpr int VEC = D * 2 / 16 / PARTS;  // 16-byte vectors per thread and row
  int carry_tie = 0, carry_keep = 0;
  for (int c0 = 0; c0 < n; c0 += kMoveTokens) {
    const int i = c0 + t;
    const bool valid = t < kMoveTokens && i < n;
    const uint32_t u = valid ? pooled_key(a, base, n, i) : 0xffffffffu;
    const int eq = (valid && u == T) ? 1 : 0;
    int tot_eq = 0, tot_keep = 0;
    const int tie_rank = carry_tie + scan256(eq, t, s_w, &tot_eq);
    const bool drop = valid && (u < T || (eq && tie_rank < need_ties));
    const int keep = (valid && !drop) ? 1 : 0;
    const int dest = carry_keep + scan256(keep, t, s_w, &tot_keep);
    if (t < kMoveTokens) s_dest[t] = keep ? dest : -1;
    carry_tie += tot_eq;
    carry_keep += tot_keep;
    __syncthreads();
    // move: thread t copies part t % 4 of token c0 + t / 4 (K and V)
    const int tok = t / PARTS, part = t % PARTS;
    const int src_i = c0 + tok;
    const int dst_i = s_dest[tok];
    const bool move = dst_i >= 0 && dst_i != src_i;
    u32x4_t kv[2][VEC];
    int64_t dst_off = 0;
    if (move) {
      const int64_t src_off = row_of(a, bt, src_i) * D + part * VEC * 8;
      dst_off = row_of(a, bt, dst_i) * D + part * VEC * 8;
#pragma unroll
      for (int e = 0; e < VEC; ++e) {
        kv[0][e] = *(const u32x4_t*)(a.pool_k + src_off + e * 8);
        kv[1][e] = *(const u32x4_t*)(a.pool_v + src_off + e * 8);
      }
    }
    // every load of this step has returned before any thread stores: a
    // destination may be another thread's source in the same step
    __builtin_amdgcn_s_waitcnt(0);
    __syncthreads();
    if (move) {
#pragma unroll
      for (int e = 0; e < VEC; ++e) {
        *(u32x4_t*)(a.pool_k + dst_off + e * 8) = kv[0][e];
        *(u32x4_t*)(a.pool_v + dst_off + e * 8) = kv[1][e];
      }
    }
  }
  if (t == 0) {
    const int kept = carry_keep;  // n - n_evict
    const int pages = (n + a.P - 1) / a.P, kept_pages = (kept + a.P - 1) / a.P;
    a.global_lengths[lh] = kept;
    a.rel[lh] = pages - kept_pages;
    a.newp[lh] = kept_pages;
  }
}

// ---- 4: page release --------------------------------------------------------
// grid (L*H), 256 threads: the head's released pages go to the free list
// after those of the heads before it ((layer, head) order, :661-668) and
// its table entries past the kept pages are reset to the sentinel.
__global__ __launch_bounds__(256) void snapkv_release_kernel(SnapArgs a) {
  __shared__ int s_sum[4];
  if (a.meta[0] == 0) return;
  const int lh = blockIdx.x, t = threadIdx.x, lane = t & 63, wid = t >> 6;
  int part = 0;
  for (int j = t; j < lh; j += 256) part += a.rel[j];
  part = wave_sum_int(part);
  if (lane == 0) s_sum[wid] = part;
  __syncthreads();
  const int before = (s_sum[0] + s_sum[1]) + (s_sum[2] + s_sum[3]);
  const int rel = a.rel[lh], newp = a.newp[lh];
  const int at = a.meta[1] + before;
  int32_t* bt = a.block_table + (int64_t)lh * a.max_pages + a.lb + newp;
  for (int e = t; e < rel; e += 256) {
    a.free_ids[at + e] = bt[e];
    bt[e] = a.total_pages - 1;
  }
  if (lh == a.L * a.H - 1 && t == 0) *a.free_count = at + rel;
}

int64_t align256(int64_t x) { return (x + 255) / 256 * 256; }

struct Layout {
  int64_t meta, stats, base, rel, newp, total;
};

Layout layout(int L, int H, int G, int win, int mtph) {
  const int64_t LH = (int64_t)L * H, win_pad = (win + 255) / 256 * 256;
  Layout o;
  o.meta = 0;
  o.stats = 256;
  o.base = o.stats + align256(LH * G * win_pad * 2 * 4);
  o.rel = o.base + align256(LH * (int64_t)mtph * 4);
  o.newp = o.rel + align256(LH * 4);
  o.total = o.newp + align256(LH * 4);
  return o;
}

}  // namespace

extern "C" int64_t wgkv_snapkv_workspace_bytes(int32_t num_layers, int32_t num_kv_heads, int32_t num_kv_groups,
                                               int32_t window, int32_t max_tokens_per_head) {
  if (num_layers <= 0 || num_kv_heads <= 0 || num_kv_groups <= 0 || window <= 0 || max_tokens_per_head <= 0)
    return -1;
  return layout(num_layers, num_kv_heads, num_kv_groups, window, max_tokens_per_head).total;
}

extern "C" int wgkv_snapkv_evict(
    void* pool_k, void* pool_v, int32_t* block_table, int32_t* global_lengths,
    int32_t* free_ids, int32_t* free_count, const void* query_window,
    int32_t num_layers, int32_t num_kv_heads, int32_t num_kv_groups, int32_t head_dim, int32_t block_size,
    int32_t local_pages, int32_t max_pages, int32_t total_pages, int32_t max_tokens_per_head,
    int32_t window, int32_t kernel_size, double evict_ratio, float softmax_scale, int64_t max_cached_tokens,
    int32_t logits_bf16, int32_t* state, float* scores_out,
    void* workspace, int64_t workspace_bytes, void* stream) {
  if (!pool_k || !pool_v || !block_table || !global_lengths || !free_ids || !free_count || !query_window || !state ||
      !workspace)
    return WGKV_ERR_ARG;
  if (num_layers <= 0 || num_kv_heads <= 0 || num_kv_groups <= 0 || num_kv_groups > 8 || block_size <= 0 ||
      local_pages < 0 || max_pages <= local_pages || total_pages <= 0 || max_tokens_per_head <= 0 || window <= 0)
    return WGKV_ERR_ARG;
  if (kernel_size <= 0 || kernel_size % 2 == 0 || !(evict_ratio > 0.0 && evict_ratio <= 1.0)) return WGKV_ERR_ARG;
  if ((int64_t)(max_pages - local_pages) * block_size < max_tokens_per_head - (int64_t)local_pages * block_size)
    return WGKV_ERR_ARG;
  if (head_dim != 64 && head_dim != 128) return WGKV_ERR_UNSUPPORTED;
  if (block_size & (block_size - 1)) return WGKV_ERR_UNSUPPORTED;  // pages of a power of two tokens
  if ((((uintptr_t)pool_k | (uintptr_t)pool_v | (uintptr_t)query_window) & 15) != 0) return WGKV_ERR_UNSUPPORTED;
  const Layout o = layout(num_layers, num_kv_heads, num_kv_groups, window, max_tokens_per_head);
  if (workspace_bytes < o.total || ((uintptr_t)workspace & 255) != 0) return WGKV_ERR_ARG;
  char* ws = (char*)workspace;
  SnapArgs a = {};
  a.pool_k = (uint16_t*)pool_k;
  a.pool_v = (uint16_t*)pool_v;
  a.block_table = block_table;
  a.global_lengths = global_lengths;
  a.free_ids = free_ids;
  a.free_count = free_count;
  a.qwin = (const uint16_t*)query_window;
  a.L = num_layers;
  a.H = num_kv_heads;
  a.G = num_kv_groups;
  a.D = head_dim;
  a.P = block_size;
  a.pshift = __builtin_ctz((unsigned)block_size);
  a.lb = local_pages;
  a.max_pages = max_pages;
  a.total_pages = total_pages;
  a.mtph = max_tokens_per_head;
  a.win = window;
  a.win_pad = (window + 255) / 256 * 256;
  a.ksz = kernel_size;
  a.ratio = evict_ratio;
  a.scale = softmax_scale;
  a.max_cached = max_cached_tokens;
  a.logits_bf16 = logits_bf16 ? 1 : 0;
  a.state = state;
  a.scores_out = scores_out;
  a.meta = (int32_t*)(ws + o.meta);
  a.stats = (float*)(ws + o.stats);
  a.base = (float*)(ws + o.base);
  a.rel = (int32_t*)(ws + o.rel);
  a.newp = (int32_t*)(ws + o.newp);
  hipStream_t st = (hipStream_t)stream;
  const int LH = num_layers * num_kv_heads;
  const dim3 g1(num_kv_groups * (a.win_pad / 256), LH);
  // scoring workgroups per head: enough to spread a head's tiles over the chip
  const int tiles = (max_tokens_per_head + 255) / 256;
  const int nb = tiles < 32 ? tiles : 32;
  const dim3 g2(nb, LH);
  if (head_dim == 128) {
    hipLaunchKernelGGL(snapkv_rowstats_kernel<128>, g1, dim3(256), 0, st, a);
    hipLaunchKernelGGL(snapkv_scores_kernel<128>, g2, dim3(256), 0, st, a);
    hipLaunchKernelGGL(snapkv_select_kernel<128>, dim3(LH), dim3(kSelectThreads), 0, st, a);
  } else {
    hipLaunchKernelGGL(snapkv_rowstats_kernel<64>, g1, dim3(256), 0, st, a);
    hipLaunchKernelGGL(snapkv_scores_kernel<64>, g2, dim3(256), 0, st, a);
    hipLaunchKernelGGL(snapkv_select_kernel<64>, dim3(LH), dim3(kSelectThreads), 0, st, a);
  }
  hipLaunchKernelGGL(snapkv_release_kernel, dim3(LH), dim3(256), 0, st, a);
  return hipGetLastError() == hipSuccess ? WGKV_OK : WGKV_ERR_HIP;
}
