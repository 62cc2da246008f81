// Sparse (vertical-slash) causal prefill attention on bf16 MFMA (gfx950).
//
// Replaces the external sparse_attn_func the reference calls at
// src/modeling_layers.py:1366-1374 (semantics pinned by
// utils/test_sparse_attn.py:34-93): for row block r (64 query rows) of
// (batch b, KV head h) the visible keys are
//   * the admitted columns column_index[b,h,0,:column_count[b,h,r]] ("vertical"), and
//   * the band blocks [o, o+64) for o in block_offset[r,:block_count[r]],
// intersected with causality (key <= query).  Query head hq uses KV head
// hq / G.
//
// Workgroup = (row block, b*Hkv + h), 2*G waves: wave w serves query head
// h*G + w/2, rows (w%2)*32 .. +32 of the block, so each 64-key K/V tile is
// staged in LDS once for all G heads.  Scores are computed transposed,
// S^T = K Q^T on v_mfma_f32_16x16x32_bf16 (K from LDS as the A operand, the
// wave's queries held as the B operand), which leaves each lane with 4
// consecutive keys of one query row: after the online softmax those
// probabilities are already the B operand of O^T = V^T P^T, with the V^T
// operand read from the row-major V tile by LDS transpose reads
// (ds_read_b64_tr_b16).  Softmax runs in the log2 domain in fp32.
//
// K and V tiles go from global memory straight into LDS
// (global_load_lds_dwordx4: each wave instruction fills 1 KB of LDS, lane i
// at byte 16*i), so a tile is stored unpadded, D*2 bytes per key, and bank
// conflicts are avoided by permuting the 16-byte slices of each key row:
// slice c of row r sits at slice c ^ swz_k(r) in K and c ^ swz_v(r) in V.
#include "wgkv_common.h"

namespace {

constexpr int kBlk = 64;     // query rows per block and keys per tile
constexpr float kLog2e = 1.4426950408889634f;
constexpr float kRescaleSlack = 8.f;  // log2 units a row maximum may grow before O / l are rescaled

// IEEE-754-2019 maximum (v_maximum3_f32): unlike fmaxf it needs no
// canonicalisation of its operands, and -inf (masked scores) is ordered.
__device__ __forceinline__ float fmax_ieee(float x, float y) { return __builtin_elementwise_maximum(x, y); }

// max of x over lanes i and i^16 / i^32 (v_permlane16_swap / v_permlane32_swap)
__device__ __forceinline__ float xor16_max(float x) {
  const auto r = __builtin_amdgcn_permlane16_swap(__float_as_uint(x), __float_as_uint(x), false, false);
  return fmax_ieee(__uint_as_float(r[0]), __uint_as_float(r[1]));
}
__device__ __forceinline__ float xor32_max(float x) {
  const auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(x), __float_as_uint(x), false, false);
  return fmax_ieee(__uint_as_float(r[0]), __uint_as_float(r[1]));
}

typedef short v4i16_t __attribute__((ext_vector_type(4)));
typedef short v8i16_t __attribute__((ext_vector_type(8)));

// global_load_lds_dwordx4: the 16 bytes at g go to LDS at lds + 16 * lane
// (lds must be the same in every lane)
__device__ __forceinline__ void lds_dma16(const uint16_t* g, uint16_t* lds) {
  __builtin_amdgcn_global_load_lds(g, lds, 16, 0, 0);
}

// ds_read_b64_tr_b16: see the V^T operand read in the kernel for the layout
__device__ __forceinline__ v4i16_t lds_read_tr16(const uint16_t* p) {
  return __builtin_amdgcn_ds_read_tr16_b64_v4i16((v4i16_t __attribute__((address_space(3)))*)(p));
}


// LDS slice permutations of the K and V tiles (16-byte slices, D*2-byte key
// rows, no padding).  The LDS serves 256 bytes per clock: 16 lanes of a
// 16-byte read or 32 lanes of an 8-byte transpose read.  K fragment reads
// take one slice from each of 16 consecutive rows, so those rows must land
// on 16 distinct slice positions modulo 256 bytes; a transpose read takes a
// 32-byte slice pair from each of 8 consecutive rows.  The permutation only
// uses the row bits that the 16-row and 32-row fragment offsets keep.  At
// D = 32 a row is 64 bytes: rows r and r + 4 share a 256-byte window
// position, so the permutation takes bits 2-3 of the row (K: the 16 rows
// fill 4 rows x 4 slices of the window; V: the 8 rows of a transpose read
// use the two 32-byte halves alternately).
template <int D>
__device__ __forceinline__ int swz_k(int row) {
  return D == 128 ? (row & 15) : D == 64 ? ((row >> 1) & 7) : ((row >> 2) & 3);
}
template <int D>
__device__ __forceinline__ int swz_v(int row) {
  return D == 128 ? 2 * (row & 7) : D == 64 ? 2 * ((row >> 1) & 3) : 2 * ((row >> 2) & 1);
}

struct PrefillArgs {
  const uint16_t* q;
  int64_t q_sb, q_ss, q_sh;
  const uint16_t* k;
  const uint16_t* v;
  int64_t kv_sb, kv_ss, kv_sh;
  uint16_t* out;
  int64_t o_sb, o_ss, o_sh;
  const int32_t* block_count;
  const int32_t* block_offset;
  int bo_width;
  const int32_t* column_count;
  const int32_t* column_index;
  int64_t ci_sb, ci_sh;  // column_index strides (batch, head); positions contiguous
  int B, S, Hkv, R, G;
  float scale_log2;
  // chunked mode: queries/outputs and the chunk's k/v are chunk-relative rows
  // of positions c0 .. c0+C-1; S = c0 + C bounds the keys.  Admitted columns
  // are logical indices into each head's paged global cache (block table row
  // bt + h*bt_sh, already offset past the local pages), band keys below c0
  // come from the ring (pool row ring_row0 + h*W + p - (c0 - W)).
  int c0, W;
  int page_log2;  // pages of the global cache hold 1 << page_log2 tokens (16, 32 or 64)
  // one-shot mode: every key row of k/v lies within 2^31 bytes of the head's
  // base, so its byte offset fits 32 bits
  int off32;
  const uint16_t* pool_k;
  const uint16_t* pool_v;
  const int32_t* bt;
  int64_t bt_sh;
  int64_t ring_row0;
};

template <int D, int HPW, bool CHUNK>
__global__ __launch_bounds__(128 * HPW) void sparse_prefill_kernel(PrefillArgs a) {
  constexpr int NT = 128 * HPW;    // threads
  constexpr int KS = D / 32;       // k-steps over head_dim
  constexpr int DT = D / 16;       // 16-wide d tiles
  constexpr int CH = D / 8;        // 16-byte slices per row
  constexpr int NW = 2 * HPW;      // waves
  constexpr int RPB = 64 / CH;     // key rows per 1 KB LDS block (one wave load instruction)
  constexpr int NBLK = kBlk / RPB; // 1 KB blocks per K (or V) tile
  // With four heads per workgroup only waves 0-3 load tiles: they are the
  // older wave of each SIMD, win its issue arbitration and reach the tile
  // barrier first, so the load issue moves off the younger waves' path.
  constexpr int NL = HPW == 4 ? NW / 2 : NW;  // loading waves
  constexpr int KPT = NBLK / NL;   // blocks per loading wave and tile
  static_assert(NBLK % NL == 0, "every loading wave loads whole 1 KB blocks");
  // double buffers as four distinct LDS objects: the DMA into one buffer
  // provably does not alias the reads of the other, so no wait for the
  // in-flight tile is placed before them
  __shared__ __attribute__((aligned(16))) uint16_t sK0[kBlk * D];
  __shared__ __attribute__((aligned(16))) uint16_t sK1[kBlk * D];
  __shared__ __attribute__((aligned(16))) uint16_t sV0[kBlk * D];
  __shared__ __attribute__((aligned(16))) uint16_t sV1[kBlk * D];
  // block offsets are read-only metadata: scalar loads
  const int32_t __attribute__((address_space(4)))* bofs =
      (const int32_t __attribute__((address_space(4)))*)a.block_offset;

  const int t = threadIdx.x;
  const int lane = t & 63, wid = __builtin_amdgcn_readfirstlane(t >> 6);
  const int n = lane & 15, g = lane >> 4;
  // Persistent workgroups: the grid holds as many workgroups as are resident
  // at once, and workgroup w serves the items w and, in alternate rounds,
  // counting from the other end (a snake order).  Items run from the last
  // row block to the first: a row block sees at least as many admitted
  // columns and band keys as any earlier one, so the order is heaviest
  // first and the snake pairs heavy items with light ones -- no second
  // round of dispatch with a ragged tail.  Within a round consecutive items
  // are the (sequence, KV head) pairs of one row block, and workgroups are
  // dealt to the XCDs round-robin, so an XCD serves one KV head per round
  // (at B*Hkv = 8) and its L2 holds that head's K/V.
  const int nbh = a.B * a.Hkv;
  const int nbz = nbh * (a.G / HPW);
  const int n_items = a.R * nbz;
  for (int round = 0;; ++round) {
    const int w = (round & 1) ? (int)gridDim.x - 1 - (int)blockIdx.x : (int)blockIdx.x;
    const int item = round * (int)gridDim.x + w;
    if (item >= n_items) break;
    if (round) __syncthreads();  // every wave is done with the previous item's tiles
    const int rb = item / nbz, rest = item - rb * nbz;
    const int r = a.R - 1 - rb;
    const int bh = rest % nbh;
    const int b = bh / a.Hkv, h = bh - b * a.Hkv;
    const int hq = h * a.G + (rest / nbh) * HPW + (wid >> 1);
    const int lrow0 = r * kBlk + (wid & 1) * 32;   // first query row of this wave (tensor row)
    const int row0 = (CHUNK ? a.c0 : 0) + lrow0;   // its position
    const int nrows = a.S - (CHUNK ? a.c0 : 0);    // query rows in the tensors

    // queries as the B operand: lane (row n, slice g) of row tile rt, k-step j
    bf16x8_t qb[2][KS];
  #pragma unroll
    for (int rt = 0; rt < 2; ++rt) {
      const int s = min(lrow0 + rt * 16 + n, nrows - 1);
      const uint16_t* qrow = a.q + (int64_t)b * a.q_sb + (int64_t)s * a.q_ss + (int64_t)hq * a.q_sh;
  #pragma unroll
      for (int j = 0; j < KS; ++j) qb[rt][j] = __builtin_bit_cast(bf16x8_t, *(const u32x4_t*)(qrow + (j * 4 + g) * 8));
    }

    float m_run[2] = {-INFINITY, -INFINITY};
    // row sums of the (bf16) probabilities, accumulated by the matrix core as
    // ones . P^T: every entry of lsum[rt] holds the sum of query row rt*16+n
    f32x4_t lsum[2] = {(f32x4_t){0.f, 0.f, 0.f, 0.f}, (f32x4_t){0.f, 0.f, 0.f, 0.f}};
    const bf16x8_t ones = __builtin_bit_cast(bf16x8_t, (u32x4_t){0x3f803f80u, 0x3f803f80u, 0x3f803f80u, 0x3f803f80u});
    f32x4_t o[DT][2];
  #pragma unroll
    for (int dt = 0; dt < DT; ++dt)
  #pragma unroll
      for (int rt = 0; rt < 2; ++rt) o[dt][rt] = (f32x4_t){0.f, 0.f, 0.f, 0.f};

    const int nv = a.column_count[((int64_t)b * a.Hkv + h) * a.R + r];
    int nb, band_start = 0;
    if (CHUNK) {
      // band of global row block rg: [max(0, rg*64 - W + 1), rg*64 + 64) in 64-key tiles
      const int rg = a.c0 / kBlk + r;
      band_start = max(0, rg * kBlk - a.W + 1);
      nb = (min(rg * kBlk + kBlk, a.S) - band_start + kBlk - 1) / kBlk;
    } else {
      nb = a.block_count[r];
    }
    const int n_vtiles = (nv + kBlk - 1) / kBlk;
    const int ntiles = n_vtiles + nb;
    const int32_t* cidx = a.column_index + (int64_t)b * a.ci_sb + (int64_t)h * a.ci_sh;
    const uint16_t* kbase = a.k + (int64_t)b * a.kv_sb + (int64_t)h * a.kv_sh;
    const uint16_t* vbase = a.v + (int64_t)b * a.kv_sb + (int64_t)h * a.kv_sh;

    // Tile loading: loading wave w fills the 1 KB blocks w, w+NL, ... of the K
    // and of the V tile; in block q, lane i loads key row q*RPB + i/CH, slice
    // position i%CH, i.e. global slice (i%CH) ^ swz_k(row) for K and
    // (i%CH) ^ swz_v(row) for V.  The keys of the next tile are looked up two
    // tiles ahead and its rows loaded one tile ahead, so both latencies overlap
    // the current tile's arithmetic.
    int krow[KPT], kcolK[KPT], kcolV[KPT];
  #pragma unroll
    for (int i = 0; i < KPT; ++i) {
      const int row = (wid + i * NL) * RPB + lane / CH;
      krow[i] = row;
      kcolK[i] = (lane % CH) ^ swz_k<D>(row);
      kcolV[i] = (lane % CH) ^ swz_v<D>(row);
    }
    // A tile's rows are fetched in two stages.  Two tiles ahead, tile_idx
    // loads the indirections -- the admitted columns' positions or, in chunked
    // mode, the page ids of the global-cache entries (band rows need none) --
    // into registers; one tile ahead, tile_load turns them into row addresses
    // and loads the rows.  Keeping the dependent index loads a tile ahead of
    // the row loads means no wait for an index also waits for the rows issued
    // before it (memory counters retire in order).
    struct Idx {
      // per item: one-shot mode, the column or band position of the lane's
      // row; chunked mode, admitted columns, the page id of the wave's 1 KB
      // block (uniform; band rows need no index in chunked mode)
      int k[KPT];
    };
    // In chunked mode the 4 rows of a wave's 1 KB block are 4 consecutive
    // logical entries of the head's global cache, aligned to 4, so they lie in
    // one page (16, 32 or 64 tokens): the page id is one scalar load per block
    // and the row address is that page's (scalar) base plus a 32-bit lane
    // offset.
    const int32_t __attribute__((address_space(4)))* bt_h =
        CHUNK ? (const int32_t __attribute__((address_space(4)))*)(a.bt + (int64_t)h * a.bt_sh) : nullptr;
    auto tile_idx = [&](int tl, Idx& ix) __attribute__((always_inline)) {
      if (wid >= NL) return;
      if (tl < n_vtiles) {
        const int nval = min(kBlk, nv - tl * kBlk);
  #pragma unroll
        for (int i = 0; i < KPT; ++i) {
          if (CHUNK) {
            const int first = (wid + i * NL) * RPB;  // first row of the block (uniform)
            ix.k[i] = bt_h[(unsigned)(tl * kBlk + min(first, nval - 1)) >> a.page_log2];
          } else {
            ix.k[i] = cidx[tl * kBlk + min(krow[i], nval - 1)];
          }
        }
      } else if (!CHUNK) {
        const int b0 = bofs[r * a.bo_width + (tl - n_vtiles)];
  #pragma unroll
        for (int i = 0; i < KPT; ++i) ix.k[i] = min(b0 + krow[i], a.S - 1);
      }
    };
    // row start of key x of tile tl in the K (or V) source (not the chunked
    // mode's admitted columns, which tile_load addresses by page)
    auto row_ptr = [&](bool vertical, int x, const uint16_t* tensor_base, const uint16_t* pool) -> const uint16_t* {
      if (vertical) return tensor_base + (int64_t)x * a.kv_ss;
      if (CHUNK && x < a.c0) return pool + (a.ring_row0 + (int64_t)h * a.W + (x - (a.c0 - a.W))) * D;
      return tensor_base + (int64_t)(x - (CHUNK ? a.c0 : 0)) * a.kv_ss;
    };
    // Chunked mode: a tile that needs no clamping is loaded from a scalar
    // base plus a 32-bit lane offset -- within a page (admitted columns),
    // within the ring (band rows before the chunk) or within the chunk's k/v
    // (band rows of the chunk; 32-bit while 63 rows of the k/v stride fit).
    // The general path below serves the last admitted tile, the band tile
    // that straddles the chunk start and the tile that runs past the sequence
    // end.  This keeps the per-lane 64-bit address arithmetic, which held the
    // load issue of a tile at ~500 cycles per wave, off the common tiles.
    auto dma_at = [&](const void* base, uint32_t off, uint16_t* lds) __attribute__((always_inline)) {
      lds_dma16((const uint16_t*)((const char*)base + off), lds);
    };
    auto tile_load = [&](int tl, const Idx& ix, uint16_t* dK, uint16_t* dV) __attribute__((always_inline)) {
      if (wid >= NL) return;
      const bool vertical = tl < n_vtiles;
      const int nval = vertical ? min(kBlk, nv - tl * kBlk) : kBlk;
      if (!CHUNK && a.off32) {
        // one-shot mode: every row is k/v row ix.k[i] (clamped when it was looked up)
  #pragma unroll
        for (int i = 0; i < KPT; ++i) {
          const int blk = (wid + i * NL) * 512;
          int ck = kcolK[i], cv = kcolV[i];
          asm volatile("" : "+v"(ck), "+v"(cv));
          const uint32_t r = (uint32_t)ix.k[i] * (uint32_t)(a.kv_ss * 2);
          dma_at(kbase, r + ck * 16, dK + blk);
          dma_at(vbase, r + cv * 16, dV + blk);
        }
        return;
      }
      if (CHUNK) {
        const int first = band_start + (tl - n_vtiles) * kBlk;  // band tiles: first key position
        if (vertical && nval == kBlk) {
  #pragma unroll
          for (int i = 0; i < KPT; ++i) {
            const int blk = (wid + i * NL) * 512;
            const int64_t pg = ((int64_t)ix.k[i] << a.page_log2) * (D * 2);
            int kr = krow[i], ck = kcolK[i], cv = kcolV[i];
            asm volatile("" : "+v"(kr), "+v"(ck), "+v"(cv));  // recomputed here, not hoisted out of the loop
            // tl * kBlk is a multiple of the page, so the row within the page is kr mod page
            const uint32_t r = (uint32_t)(kr & ((1 << a.page_log2) - 1)) * (D * 2);
            dma_at((const char*)a.pool_k + pg, r + ck * 16, dK + blk);
            dma_at((const char*)a.pool_v + pg, r + cv * 16, dV + blk);
          }
          return;
        }
        if (!vertical && first + kBlk <= a.c0) {
          const int64_t row = a.ring_row0 + (int64_t)h * a.W + (first - (a.c0 - a.W));
  #pragma unroll
          for (int i = 0; i < KPT; ++i) {
            const int blk = (wid + i * NL) * 512;
            int kr = krow[i], ck = kcolK[i], cv = kcolV[i];
            asm volatile("" : "+v"(kr), "+v"(ck), "+v"(cv));
            const uint32_t r = (uint32_t)kr * (D * 2);
            dma_at(a.pool_k + row * D, r + ck * 16, dK + blk);
            dma_at(a.pool_v + row * D, r + cv * 16, dV + blk);
          }
          return;
        }
        if (!vertical && first >= a.c0 && first + kBlk <= a.S && a.kv_ss <= (1 << 24)) {
          const int64_t row = (int64_t)(first - a.c0) * a.kv_ss;
  #pragma unroll
          for (int i = 0; i < KPT; ++i) {
            const int blk = (wid + i * NL) * 512;
            int kr = krow[i], ck = kcolK[i], cv = kcolV[i];
            asm volatile("" : "+v"(kr), "+v"(ck), "+v"(cv));
            const uint32_t r = (uint32_t)kr * (uint32_t)(a.kv_ss * 2);
            dma_at(kbase + row, r + ck * 16, dK + blk);
            dma_at(vbase + row, r + cv * 16, dV + blk);
          }
          return;
        }
      }
  #pragma unroll
      for (int i = 0; i < KPT; ++i) {
        const int kt = min(krow[i], nval - 1);
        const int blk = (wid + i * NL) * 512;  // element offset of this wave's block (1 KB)
        if (CHUNK && vertical) {
          // tl * kBlk is a multiple of the page, so the slot is kt mod page
          const int64_t page_base = ((int64_t)ix.k[i] << a.page_log2) * D;
          const int lane_row = (kt & ((1 << a.page_log2) - 1)) * D;
          lds_dma16(a.pool_k + page_base + (lane_row + kcolK[i] * 8), dK + blk);
          lds_dma16(a.pool_v + page_base + (lane_row + kcolV[i] * 8), dV + blk);
        } else {
          const int x = CHUNK ? min(band_start + (tl - n_vtiles) * kBlk + krow[i], a.S - 1) : ix.k[i];
          lds_dma16(row_ptr(vertical, x, kbase, a.pool_k) + kcolK[i] * 8, dK + blk);
          lds_dma16(row_ptr(vertical, x, vbase, a.pool_v) + kcolV[i] * 8, dV + blk);
        }
      }
    };
    // Per-lane LDS element offsets of the fragments (the slice permutations
    // above, resolved once): K row kt*16+n, slice j*4+g sits at slice
    // (j*4+g) ^ swz_k(n); the transpose read of lane n in group g (row
    // 4g + n/4 + 16u + 32s, d slice 2*dt + (n&3)/2, half n&1) finds its slice at
    // (2*dt + (n&3)/2) ^ swz_v(4g + n/4).
    int koff[KS];
  #pragma unroll
    for (int j = 0; j < KS; ++j) koff[j] = n * D + ((j * 4 + g) ^ swz_k<D>(n)) * 8;
    const int vrow = 4 * g + (n >> 2);
    int voff[DT];
  #pragma unroll
    for (int dt = 0; dt < DT; ++dt)
      voff[dt] = vrow * D + ((2 * dt + ((n & 3) >> 1)) ^ swz_v<D>(vrow)) * 8 + (n & 1) * 4;

    Idx idx_next;
    if (ntiles > 0) {
      Idx i0;
      tile_idx(0, i0);
      tile_load(0, i0, sK0, sV0);
      if (ntiles > 1) tile_idx(1, idx_next);
    }

    // one 64-key tile: K and V of the tile in (sK, sV); the next tile's rows go to (nK, nV)
    auto step = [&](int tile, const uint16_t* sK, const uint16_t* sV, uint16_t* nK,
                    uint16_t* nV) __attribute__((always_inline)) {
      const bool vert = tile < n_vtiles;
      int band0 = 0, nvalid = kBlk;
      if (vert) nvalid = min(kBlk, nv - tile * kBlk);
      else band0 = CHUNK ? band_start + (tile - n_vtiles) * kBlk : bofs[r * a.bo_width + (tile - n_vtiles)];

      // this wave's loads of the tile (and of the next tile's indices) have
      // landed; the barrier publishes every wave's and frees the other buffer
      __builtin_amdgcn_s_waitcnt(0x0F70);  // vmcnt(0)
      __syncthreads();
      // K fragments of k-step j+1 are read while the MFMAs of k-step j run;
      // those of k-step 0 before the next tile's loads are issued
      bf16x8_t kf[2][4];
  #pragma unroll
      for (int kt = 0; kt < 4; ++kt)
        kf[0][kt] = __builtin_bit_cast(bf16x8_t, *(const u32x4_t*)(&sK[kt * 16 * D + koff[0]]));
      __builtin_amdgcn_sched_barrier(0);
      // the next tile's rows stream into the other buffer under this tile's arithmetic
      if (tile + 1 < ntiles) {
        tile_load(tile + 1, idx_next, nK, nV);
        if (tile + 2 < ntiles) tile_idx(tile + 2, idx_next);
      }

      // ---- S^T = K Q^T: key tiles kt (16 keys) x row tiles rt ------------------
      f32x4_t sc[4][2];
      // k-step outer: the 8 accumulators are independent chains, so
      // consecutive MFMAs never wait on each other
  #pragma unroll
      for (int kt = 0; kt < 4; ++kt)
  #pragma unroll
        for (int rt = 0; rt < 2; ++rt) sc[kt][rt] = (f32x4_t){0.f, 0.f, 0.f, 0.f};
  #pragma unroll
      for (int j = 0; j < KS; ++j) {
        if (j + 1 < KS)
  #pragma unroll
          for (int kt = 0; kt < 4; ++kt)
            kf[(j + 1) & 1][kt] = __builtin_bit_cast(bf16x8_t, *(const u32x4_t*)(&sK[kt * 16 * D + koff[j + 1]]));
        __builtin_amdgcn_sched_barrier(0);
  #pragma unroll
        for (int kt = 0; kt < 4; ++kt)
  #pragma unroll
          for (int rt = 0; rt < 2; ++rt)
            sc[kt][rt] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(kf[j & 1][kt], qb[rt][j], sc[kt][rt], 0, 0, 0);
      }
      // tiles whose 64 keys are all visible to all 32 rows of the wave skip masking
      const bool full = vert ? nvalid == kBlk : (band0 + kBlk - 1 <= row0 && band0 + kBlk <= a.S);
      // ---- online softmax (lane: query row rt*16+n, keys kt*16+4g+i) -------------
      // Row maxima are taken on the raw scores (the scale is positive) and the
      // scale is folded into the exponent's FMA.  The reference maximum m_run of
      // a row moves only when a tile's maximum exceeds it by more than 8 (log2
      // units), so p <= 2^8 and the O / l rescale runs on few tiles.
      float mxs[2];
  #pragma unroll
      for (int rt = 0; rt < 2; ++rt) {
        if (!full) {
          // visible keys of this row are kk < lim
          const int qrow = row0 + rt * 16 + n;
          const int lim = vert ? nvalid : min(a.S - band0, qrow - band0 + 1);
  #pragma unroll
          for (int kt = 0; kt < 4; ++kt)
  #pragma unroll
            for (int i = 0; i < 4; ++i) {
              const int kk = kt * 16 + 4 * g + i;
              sc[kt][rt][i] = kk < lim ? sc[kt][rt][i] : -INFINITY;
            }
        }
        float mx = -INFINITY;
  #pragma unroll
        for (int kt = 0; kt < 4; ++kt)
          mx = fmax_ieee(mx, fmax_ieee(fmax_ieee(sc[kt][rt][0], sc[kt][rt][1]), fmax_ieee(sc[kt][rt][2], sc[kt][rt][3])));
        mxs[rt] = mx;  // this lane's 16 keys of the row
      }
      // A row needs the rescale iff one of its four lanes' maxima exceeds
      // m_run by the slack (the scale is positive, so scaling commutes with
      // the max); only then are the row maxima reduced across the lanes.
      if (__builtin_amdgcn_ballot_w64(mxs[0] * a.scale_log2 > m_run[0] + kRescaleSlack ||
                                      mxs[1] * a.scale_log2 > m_run[1] + kRescaleSlack) != 0) {
  #pragma unroll
        for (int rt = 0; rt < 2; ++rt) mxs[rt] = xor32_max(xor16_max(mxs[rt])) * a.scale_log2;
        const bool need0 = mxs[0] > m_run[0] + kRescaleSlack;
        const bool need1 = mxs[1] > m_run[1] + kRescaleSlack;
  #pragma unroll
        for (int rt = 0; rt < 2; ++rt) {
          const bool need = rt == 0 ? need0 : need1;
          const float mnew = need ? mxs[rt] : m_run[rt];
          const float alpha = mnew == m_run[rt] ? 1.f : fast_exp2(m_run[rt] - mnew);
          m_run[rt] = mnew;
          lsum[rt] *= alpha;
  #pragma unroll
          for (int dt = 0; dt < DT; ++dt) o[dt][rt] *= alpha;
        }
      }
      bf16x8_t pb[2][2];  // [rt][k-step of 32 keys]
  #pragma unroll
      for (int rt = 0; rt < 2; ++rt) {
        const float mref = m_run[rt] == -INFINITY ? 0.f : m_run[rt];  // rows with nothing visible keep p = 0
        uint32_t pw[8];
  #pragma unroll
        for (int kt = 0; kt < 4; ++kt)
  #pragma unroll
          for (int i = 0; i < 4; i += 2) {
            const float p0 = fast_exp2(fmaf(sc[kt][rt][i], a.scale_log2, -mref));
            const float p1 = fast_exp2(fmaf(sc[kt][rt][i + 1], a.scale_log2, -mref));
            pw[kt * 2 + i / 2] = pack_bf16x2(p0, p1);
          }
        // k-step s covers key tiles 2s (slots 0-3) and 2s+1 (slots 4-7)
  #pragma unroll
        for (int s = 0; s < 2; ++s) {
          const u32x4_t w = (u32x4_t){pw[4 * s], pw[4 * s + 1], pw[4 * s + 2], pw[4 * s + 3]};
          pb[rt][s] = __builtin_bit_cast(bf16x8_t, w);
        }
      }
      // ---- O^T += V^T P^T ------------------------------------------------------
      // The A operand (lane: d = dt*16 + n, keys 32s+4g+0..3 and 32s+16+4g+0..3,
      // the key order of pb) comes from two transpose reads of the row-major V
      // tile: within each 16-lane group, lane n addresses row kb + n/4 at column
      // d0 + 4*(n%4), and receives V[kb+k][d0+n] for k = 0..3.
  #pragma unroll
      for (int s = 0; s < 2; ++s) {
  #pragma unroll
        for (int dt = 0; dt < DT; ++dt) {
          const uint16_t* vrd = sV + voff[dt] + s * 32 * D;
          const v4i16_t lo = lds_read_tr16(vrd);
          const v4i16_t hi = lds_read_tr16(vrd + 16 * D);
          const bf16x8_t vf = __builtin_bit_cast(bf16x8_t, __builtin_shufflevector(lo, hi, 0, 1, 2, 3, 4, 5, 6, 7));
  #pragma unroll
          for (int rt = 0; rt < 2; ++rt)
            o[dt][rt] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(vf, pb[rt][s], o[dt][rt], 0, 0, 0);
        }
  #pragma unroll
        for (int rt = 0; rt < 2; ++rt) lsum[rt] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(ones, pb[rt][s], lsum[rt], 0, 0, 0);
      }
    };
    for (int tile = 0; tile < ntiles; tile += 2) {
      step(tile, sK0, sV0, sK1, sV1);
      if (tile + 1 < ntiles) step(tile + 1, sK1, sV1, sK0, sV0);
    }

    // ---- normalise and store: lane holds O[row rt*16+n][dt*16 + 4g + i] -------
  #pragma unroll
    for (int rt = 0; rt < 2; ++rt) {
      const float l = lsum[rt][0];
      const float inv = l > 0.f ? 1.f / l : 0.f;
      const int s = lrow0 + rt * 16 + n;
      if (s < nrows) {
        uint16_t* orow = a.out + (int64_t)b * a.o_sb + (int64_t)s * a.o_ss + (int64_t)hq * a.o_sh;
  #pragma unroll
        for (int dt = 0; dt < DT; ++dt) {
          const uint32_t w0 = pack_bf16x2(o[dt][rt][0] * inv, o[dt][rt][1] * inv);
          const uint32_t w1 = pack_bf16x2(o[dt][rt][2] * inv, o[dt][rt][3] * inv);
          *(uint64_t*)(orow + dt * 16 + 4 * g) = (uint64_t)w0 | ((uint64_t)w1 << 32);
        }
      }
    }
  }
}

int cu_count() {
  static int cached[64] = {0};
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 64) return 256;
  if (cached[dev] == 0) {
    int n = 0;
    if (hipDeviceGetAttribute(&n, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess || n <= 0) n = 256;
    cached[dev] = n;
  }
  return cached[dev];
}

// Persistent grid: the workgroups resident at once (occupancy of the
// instance times the CUs), at most one per item.
template <int D, int HPW, bool CHUNK>
hipError_t launch_persistent(const PrefillArgs& a, hipStream_t st) {
  static int per_cu = 0;
  if (per_cu == 0) {
    int nb = 0;
    if (hipOccupancyMaxActiveBlocksPerMultiprocessor(&nb, sparse_prefill_kernel<D, HPW, CHUNK>, 128 * HPW, 0) !=
            hipSuccess ||
        nb <= 0)
      nb = 1;
    per_cu = nb;
  }
  const int64_t items = (int64_t)a.R * a.B * a.Hkv * (a.G / HPW);
  const int grid = (int)(items < (int64_t)per_cu * cu_count() ? items : (int64_t)per_cu * cu_count());
  hipLaunchKernelGGL((sparse_prefill_kernel<D, HPW, CHUNK>), dim3(grid), dim3(128 * HPW), 0, st, a);
  return hipGetLastError();
}

template <int D, int HPW>
hipError_t launch(const PrefillArgs& a, hipStream_t st, bool chunked) {
  return chunked ? launch_persistent<D, HPW, true>(a, st) : launch_persistent<D, HPW, false>(a, st);
}

// Query heads per workgroup: the largest of 4, 2, 1 that divides G and lets
// every wave load whole 1 KB blocks of a tile (2 * HPW waves, D / 8 blocks:
// at most 2 heads at D = 32).  G = 3 then takes one head per workgroup.
int heads_per_wg(int head_dim, int G) {
  const int cap = head_dim == 32 ? 2 : 4;
  for (int h = cap; h > 1; h >>= 1)
    if (G % h == 0) return h;
  return 1;
}

hipError_t launch_any(PrefillArgs& a, hipStream_t st, int head_dim, int G, bool chunked) {
  a.G = G;
  const int hpw = heads_per_wg(head_dim, G);
  if (head_dim == 128)
    return hpw == 1 ? launch<128, 1>(a, st, chunked) : hpw == 2 ? launch<128, 2>(a, st, chunked)
                    : launch<128, 4>(a, st, chunked);
  if (head_dim == 64)
    return hpw == 1 ? launch<64, 1>(a, st, chunked) : hpw == 2 ? launch<64, 2>(a, st, chunked)
                    : launch<64, 4>(a, st, chunked);
  return hpw == 1 ? launch<32, 1>(a, st, chunked) : launch<32, 2>(a, st, chunked);
}

}  // namespace

extern "C" int wgkv_sparse_prefill_attn(
    const void* q, int64_t q_sb, int64_t q_ss, int64_t q_sh,
    const void* k, const void* v, int64_t kv_sb, int64_t kv_ss, int64_t kv_sh,
    void* out, int64_t o_sb, int64_t o_ss, int64_t o_sh,
    const int32_t* block_count, const int32_t* block_offset, int32_t block_offset_width,
    const int32_t* column_count, const int32_t* column_index, int64_t ci_sb, int64_t ci_sh,
    int32_t batch, int32_t seq_len, int32_t num_q_heads, int32_t num_kv_heads, int32_t head_dim,
    int32_t block, float softmax_scale, void* stream) {
  if (!q || !k || !v || !out || !block_count || !block_offset || !column_count || !column_index) return WGKV_ERR_ARG;
  if (batch <= 0 || seq_len <= 0 || num_kv_heads <= 0 || num_q_heads % num_kv_heads) return WGKV_ERR_ARG;
  if (block != kBlk) return WGKV_ERR_UNSUPPORTED;
  const int G = num_q_heads / num_kv_heads;
  if (head_dim != 32 && head_dim != 64 && head_dim != 128) return WGKV_ERR_UNSUPPORTED;
  if (G < 1 || G > 8) return WGKV_ERR_UNSUPPORTED;
  if (((uintptr_t)q | (uintptr_t)k | (uintptr_t)v | (uintptr_t)out) & 15) return WGKV_ERR_UNSUPPORTED;
  if ((q_sb | q_ss | q_sh | kv_sb | kv_ss | kv_sh | o_sb | o_ss | o_sh) & 7) return WGKV_ERR_UNSUPPORTED;
  PrefillArgs a;
  a.q = (const uint16_t*)q;
  a.q_sb = q_sb;
  a.q_ss = q_ss;
  a.q_sh = q_sh;
  a.k = (const uint16_t*)k;
  a.v = (const uint16_t*)v;
  a.kv_sb = kv_sb;
  a.kv_ss = kv_ss;
  a.kv_sh = kv_sh;
  a.out = (uint16_t*)out;
  a.o_sb = o_sb;
  a.o_ss = o_ss;
  a.o_sh = o_sh;
  a.block_count = block_count;
  a.block_offset = block_offset;
  a.bo_width = block_offset_width;
  a.column_count = column_count;
  a.column_index = column_index;
  a.ci_sb = ci_sb;
  a.ci_sh = ci_sh;
  a.B = batch;
  a.S = seq_len;
  a.Hkv = num_kv_heads;
  a.R = (seq_len + kBlk - 1) / kBlk;
  a.scale_log2 = softmax_scale * kLog2e;
  a.c0 = 0;
  a.W = 0;
  a.page_log2 = 4;
  a.off32 = (int64_t)seq_len * kv_ss * 2 <= (int64_t)INT32_MAX;
  a.pool_k = a.pool_v = nullptr;
  a.bt = nullptr;
  a.bt_sh = 0;
  a.ring_row0 = 0;
  const hipError_t e = launch_any(a, (hipStream_t)stream, head_dim, G, false);
  return e == hipSuccess ? WGKV_OK : WGKV_ERR_HIP;
}

extern "C" int wgkv_chunk_prefill_attn(
    const void* q, int64_t q_ss, int64_t q_sh,
    const void* k, const void* v, int64_t kv_ss, int64_t kv_sh,
    void* out, int64_t o_ss, int64_t o_sh,
    const void* pool_k, const void* pool_v,
    const int32_t* block_table, int32_t max_pages_per_head,
    const int32_t* column_count,
    int32_t layer, int32_t chunk_start, int32_t chunk_len,
    int32_t num_q_heads, int32_t num_kv_heads, int32_t head_dim,
    int32_t local_window, int32_t page_size, float softmax_scale, void* stream) {
  if (!q || !k || !v || !out || !pool_k || !pool_v || !block_table || !column_count) return WGKV_ERR_ARG;
  if (chunk_len <= 0 || chunk_start < 0 || num_kv_heads <= 0 || num_q_heads % num_kv_heads) return WGKV_ERR_ARG;
  if (local_window <= 0 || local_window % kBlk || chunk_start % kBlk || page_size <= 0 || local_window % page_size)
    return WGKV_ERR_ARG;
  int page_log2;
  if (page_size == 16) page_log2 = 4;
  else if (page_size == 32) page_log2 = 5;
  else if (page_size == 64) page_log2 = 6;
  else return WGKV_ERR_UNSUPPORTED;  // pages must divide the 64-key tile
  if (chunk_start > 0 && chunk_start < local_window) return WGKV_ERR_ARG;  // the ring must be full
  const int G = num_q_heads / num_kv_heads;
  if (head_dim != 32 && head_dim != 64 && head_dim != 128) return WGKV_ERR_UNSUPPORTED;
  if (G < 1 || G > 8) return WGKV_ERR_UNSUPPORTED;
  if (((uintptr_t)q | (uintptr_t)k | (uintptr_t)v | (uintptr_t)out | (uintptr_t)pool_k | (uintptr_t)pool_v) & 15)
    return WGKV_ERR_UNSUPPORTED;
  if ((q_ss | q_sh | kv_ss | kv_sh | o_ss | o_sh) & 7) return WGKV_ERR_UNSUPPORTED;
  PrefillArgs a = {};
  a.q = (const uint16_t*)q;
  a.q_ss = q_ss;
  a.q_sh = q_sh;
  a.k = (const uint16_t*)k;
  a.v = (const uint16_t*)v;
  a.kv_ss = kv_ss;
  a.kv_sh = kv_sh;
  a.out = (uint16_t*)out;
  a.o_ss = o_ss;
  a.o_sh = o_sh;
  a.column_count = column_count;
  a.B = 1;
  a.S = chunk_start + chunk_len;
  a.Hkv = num_kv_heads;
  a.R = (chunk_len + kBlk - 1) / kBlk;
  a.scale_log2 = softmax_scale * kLog2e;
  a.c0 = chunk_start;
  a.W = local_window;
  a.page_log2 = page_log2;
  a.pool_k = (const uint16_t*)pool_k;
  a.pool_v = (const uint16_t*)pool_v;
  a.bt = block_table + ((int64_t)layer * num_kv_heads) * max_pages_per_head + local_window / page_size;
  a.bt_sh = max_pages_per_head;
  a.ring_row0 = (int64_t)layer * num_kv_heads * local_window;
  const hipError_t e = launch_any(a, (hipStream_t)stream, head_dim, G, true);
  return e == hipSuccess ? WGKV_OK : WGKV_ERR_HIP;
}
