// Vertical-slash metadata of the sparse prefill (gfx950), built on the device.
//
// Replaces generate_sparse_indices / generate_block_offset /
// generate_column_index (src/modeling_layers.py:321-409), which loop over
// (batch, head) on the host with a torch.nonzero and a .item() sync each.
//
// Count blocks: block 0 is position 0 alone, block k >= 1 covers
// [1 + (k-1)*bs, 1 + k*bs) -- the grouping whose running sums give, for row
// block r >= P, the number of admitted positions below r*bs - W + 1.
// One workgroup per (b, h) walks the count blocks in tiles of 256 with a
// block-wide scan, writes column_count and compacts the admitted positions of
// the listed range (positions < 1 + bs*((S-1)/bs)) in ascending order.  One
// extra workgroup writes the band tables, which depend only on (W, S, bs).
#include "wgkv_common.h"

namespace {

constexpr int kThreads = 256;

struct MetaArgs {
  const uint8_t* mask;
  int64_t m_sb, m_sh;
  int B, H, S, W, bs, R, P;
  int32_t* block_count;
  int32_t* block_offset;
  int32_t* column_count;
  int32_t* column_index;
  int col_cap;
  int32_t* column_total;
};

__global__ __launch_bounds__(kThreads) void prefill_meta_kernel(MetaArgs a) {
  __shared__ int s_tmp[kThreads];
  const int t = threadIdx.x;
  const int BH = a.B * a.H;
  if ((int)blockIdx.x == BH) {
    // band tables (one row per row block, P+1 entries each)
    const int width = a.P + 1;
    const int last_first = max(0, (a.R - 1) * a.bs - a.W + 1);
    const int last_count = (a.S - last_first + a.bs - 1) / a.bs;
    for (int r = t; r < a.R; r += kThreads) {
      int cnt;
      if (r < a.P) {
        cnt = r + 1;
        for (int c = 0; c < width; ++c) a.block_offset[r * width + c] = c < a.P ? c * a.bs : 0;
      } else {
        cnt = a.P + 1;
        for (int c = 0; c < width; ++c) a.block_offset[r * width + c] = 1 + (r - a.P + c) * a.bs;
      }
      a.block_count[r] = r == a.R - 1 ? last_count : cnt;
    }
    return;
  }
  const int bh = blockIdx.x;
  const int b = bh / a.H, h = bh - b * a.H;
  const uint8_t* m = a.mask + (int64_t)b * a.m_sb + (int64_t)h * a.m_sh;
  int32_t* cc = a.column_count + (int64_t)bh * a.R;
  int32_t* ci = a.column_index + (int64_t)bh * a.col_cap;
  for (int r = t; r < min(a.P, a.R); r += kThreads) cc[r] = 0;

  const int nblk = a.R;  // count blocks 0 .. (S-1)/bs
  int carry = 0;
  for (int base = 0; base < nblk; base += kThreads) {
    const int k = base + t;
    int lo = 0, hi = 0;
    if (k < nblk) {
      lo = k == 0 ? 0 : 1 + (k - 1) * a.bs;
      hi = k == 0 ? 1 : min(a.S, 1 + k * a.bs);
    }
    int cnt = 0;
    for (int p = lo; p < hi; ++p) cnt += m[p] != 0;
    int total = 0;
    const int excl = block_exclusive_scan_256(cnt, s_tmp, &total);
    if (k < nblk) {
      const int incl = carry + excl + cnt;
      if (k + a.P < a.R) cc[k + a.P] = incl;
      int o = carry + excl;
      for (int p = lo; p < hi; ++p)
        if (m[p]) {
          if (o < a.col_cap) ci[o] = p;
          ++o;
        }
    }
    carry += total;
  }
  if (t == 0 && a.column_total) a.column_total[bh] = carry;
}

}  // namespace

extern "C" int wgkv_build_prefill_meta(
    const uint8_t* g_mask, int64_t gm_stride_b, int64_t gm_stride_h,
    int32_t batch, int32_t num_kv_heads, int32_t seq_len, int32_t local_window, int32_t block,
    int32_t* block_count, int32_t* block_offset,
    int32_t* column_count, int32_t* column_index, int32_t col_cap, int32_t* column_total,
    void* stream) {
  if (!g_mask || !block_count || !block_offset || !column_count || !column_index) return WGKV_ERR_ARG;
  if (batch <= 0 || num_kv_heads <= 0 || seq_len <= 0 || block <= 0 || local_window < 0 || col_cap < 0)
    return WGKV_ERR_ARG;
  if (local_window % block) return WGKV_ERR_ARG;  // the reference asserts W % bs == 0
  MetaArgs a;
  a.mask = g_mask;
  a.m_sb = gm_stride_b;
  a.m_sh = gm_stride_h;
  a.B = batch;
  a.H = num_kv_heads;
  a.S = seq_len;
  a.W = local_window;
  a.bs = block;
  a.R = (seq_len + block - 1) / block;
  a.P = min(local_window / block, a.R);
  a.block_count = block_count;
  a.block_offset = block_offset;
  a.column_count = column_count;
  a.column_index = column_index;
  a.col_cap = col_cap;
  a.column_total = column_total;
  hipLaunchKernelGGL(prefill_meta_kernel, dim3(batch * num_kv_heads + 1), dim3(kThreads), 0,
                     (hipStream_t)stream, a);
  return hipGetLastError() == hipSuccess ? WGKV_OK : WGKV_ERR_HIP;
}
