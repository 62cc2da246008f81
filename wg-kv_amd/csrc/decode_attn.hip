// Ragged paged decode attention over the dual cache (gfx950).
//
// Work split: the logical sequence of every (batch row b, KV head h) is cut
// into 16-token sub-pages; sub-pages are grouped into chunks of `cp`
// sub-pages (chosen on the device so that the whole batch, per-head
// remainders included, gives about one chunk per resident workgroup slot).
// One workgroup owns one chunk, and its waves take 64-token "quads" (4
// sub-pages) in turn.  Every K/V byte of the cache is read exactly once, for
// all G query heads of the KV head together.  Workgroups have 4 waves (three
// per CU) or, when the batch has few heads (B*Hkv < 32, G <= 4), 8 waves
// (one per CU), so that a head is cut into ~CUs/(B*Hkv) chunks rather than
// three times as many.  (8 rather than 12 waves: the 2048 waves dispatch
// sooner, and two per SIMD keep enough K/V loads in flight -- batch 1 at
// 128K 23.6 -> 22.9 us, 8 heads of ~80K tokens 55.8 -> 53.6 us, at 32K
// 13.5 -> 13.7 us.)
//
// Per quad and wave:
//   * K is read in the MFMA B-operand layout (lane n%16 = token row, lane/16
//     = 16-byte slice of the row) and multiplied with the query heads on
//     v_mfma_f32_16x16x32_bf16 (query head 4*gi + i of group gi replicated
//     in rows 4r+i of that group's A operand);
//   * softmax runs in the log2 domain with one lazily moved running max per
//     query head, uniform over the wave, and a per-lane running denominator;
//   * P goes through a 1 KB LDS slot per wave and head group, and V is read
//     fully coalesced (consecutive 16-byte slices of consecutive rows); P V
//     runs on v_dot2_f32_bf16 over pairs of rows (P rounded to bf16, fp32
//     sums).
// At the end of a chunk the waves merge through LDS.  A single-chunk head
// writes its output directly.  Otherwise the chunk stores (m, l, acc)
// partials, which are combined with the log-sum-exp rule in a fixed chunk
// order (so the result does not depend on which chunk finishes first):
//   * 8-wave workgroups: with device-coherent stores; the chunk counts its
//     arrival on the head's counter, and the last chunk of the head to
//     arrive merges the head's ~30 partials (one round of loads) and resets
//     the counter -- one launch per call, ~2 us less at batch 1 than a
//     second launch;
//   * 4-wave workgroups: decode_merge_kernel, launched after the split
//     kernel (at batch 8 the last arriver's write-through stores and
//     arrival count cost as much as the second launch, which spreads the
//     merge over B*Hkv*G workgroups).
#include <mutex>

#include "wgkv_common.h"

namespace {

constexpr int kPlanThreads = 256;   // plan_block's block scan: 4-wave workgroups
constexpr int kMaxBH = 2048;
constexpr int kWaveBH = 64;          // B*Hkv up to this: each wave plans alone, in registers
constexpr int kMaxSlots = 1024;      // cap on CUs * resident workgroups per CU (workspace sizing)
constexpr int kMaxChunks = kMaxSlots + kMaxBH;
constexpr int kMaxG = 8;
constexpr float kLog2e = 1.4426950408889634f;
constexpr float kRescaleSlack = 8.f;  // log2 units a running maximum may lag the scores

// Resident workgroups per CU: with 4 waves, G <= 4 fits three (158 VGPRs at
// D=128, G=4), G = 8 (two head groups, 83 KB of LDS) one; an 8-wave
// workgroup (G <= 4) fills a CU alone (two waves per SIMD).
constexpr int wg_per_cu(int G, int NW) { return NW > 4 ? 1 : (G > 4 ? 1 : 3); }
constexpr int waves_per_simd(int G, int NW) { return NW > 4 ? NW / 4 : wg_per_cu(G, NW); }
// Batches with fewer heads than this (and G <= 4) take 8-wave workgroups.
constexpr int kWideBelowBH = 32;

struct DecodeArgs {
  const uint16_t* q;
  int64_t q_sb, q_sh;
  const uint16_t* kc;
  const uint16_t* vc;
  int64_t num_pages;
  int page_size, page_shift;  // page_size = 16 << page_shift
  const int32_t* seqlens;
  int64_t sl_sb;
  const int32_t* bt;
  int64_t bt_sb, bt_sh;
  int max_pages;
  uint16_t* out;
  int64_t out_sb, out_sh;
  int B, Hkv;
  float scale_log2;
  int target_chunks;  // resident workgroup slots: the plan aims at one chunk per slot
  // partials of chunk w, query head i (i < G): m at part_m[w*G+i], l at
  // part_l[w*G+i], acc at part_acc[(w*G+i)*D ..]
  float* part_m;
  float* part_l;
  float* part_acc;
  // arrival counters, one per (b, h): zero before a call, zero after it
  // (8-wave workgroups)
  int* counter;
  // [B*Hkv + 1] first chunk of each (b,h) and the chunk count, written by
  // the split kernel for decode_merge_kernel (4-wave workgroups)
  int* plan;
};

__device__ __forceinline__ int clamped_tokens(const DecodeArgs& a, int bh) {
  const int b = bh / a.Hkv, h = bh - b * a.Hkv;
  int T = a.seqlens[(int64_t)b * a.sl_sb + h];
  const int cap = a.max_pages * a.page_size;
  T = T < 0 ? 0 : (T > cap ? cap : T);
  return T;
}

// This workgroup's share of the device-side split plan (replaces the host
// planner of the reference, src/modeling_layers.py:1032-1055).
struct Plan {
  int n_chunks;  // chunks of the whole call
  int bh;        // (b, h) this workgroup serves
  int first;     // global index of that head's first chunk
  int n_bh;      // chunks of that head
  int cp;        // sub-pages per chunk
};

// Sub-pages per chunk: the total over the chunk slots, rounded up to a
// multiple of 16 (4-wave workgroups: at least one quad per wave) or of 4
// (8-wave workgroups: chunks stay quad-aligned, and the ~CU-count chunks of
// a batch-1 call fill the CUs evenly), at least 16.
template <int NW>
__device__ __forceinline__ int chunk_subpages(int total, int target) {
  const int cp = (total + target - 1) / target;
  return NW > 4 ? max(16, (cp + 3) & ~3) : max(16, (cp + 15) & ~15);
}

// B*Hkv <= 64: lane bh of every wave takes head bh; the plan is two wave
// scans in registers, no LDS and no barrier.  With 4-wave workgroups,
// workgroup 0 stores the plan (first chunk of each head, then the chunk
// count) for the merge kernel.
template <int NW>
__device__ Plan plan_wave(const DecodeArgs& a, int w) {
  const int BH = a.B * a.Hkv;
  const int lane = threadIdx.x & 63;
  const int ns = lane < BH ? (clamped_tokens(a, lane) + 15) >> 4 : 0;
  const int total = __builtin_amdgcn_readlane(wave_incl_scan(ns, lane), 63);
  int cp = chunk_subpages<NW>(total, a.target_chunks);
  int ch = lane < BH ? max(1, (ns + cp - 1) / cp) : 0;
  int incl = wave_incl_scan(ch, lane);
  if (NW > 4 && __builtin_amdgcn_readlane(incl, 63) > a.target_chunks) {
    // With one workgroup per CU a chunk beyond the slots would run in a
    // second round and double the call: size for target - BH chunks instead
    // (sum over heads of ceil(n/cp) <= total/cp + BH <= target).
    cp = chunk_subpages<NW>(total, max(1, a.target_chunks - BH));
    ch = lane < BH ? max(1, (ns + cp - 1) / cp) : 0;
    incl = wave_incl_scan(ch, lane);
  }
  const int excl = incl - ch;
  Plan p;
  p.n_chunks = __builtin_amdgcn_readlane(incl, 63);
  p.cp = cp;
  // owner of chunk w: the largest head whose first chunk is <= w
  const uint64_t own = __builtin_amdgcn_ballot_w64(lane < BH && excl <= w);
  p.bh = own ? 63 - __builtin_clzll(own) : 0;
  p.first = __builtin_amdgcn_readlane(excl, p.bh);
  p.n_bh = __builtin_amdgcn_readlane(ch, p.bh);
  if (NW == 4 && w == 0 && threadIdx.x < 64) {
    if (lane < BH) a.plan[lane] = excl;
    if (lane == 0) a.plan[BH] = p.n_chunks;
  }
  return p;
}

// B*Hkv > 64 (4-wave workgroups): block scans over the heads through LDS
// (workgroup 0 stores the plan for the merge kernel).
__device__ Plan plan_block(const DecodeArgs& a, int w, int* s_pref, int* s_tmp) {
  const int BH = a.B * a.Hkv;
  const int t = threadIdx.x;
  const int per = (BH + kPlanThreads - 1) / kPlanThreads;
  const int lo = min(BH, t * per), hi = min(BH, lo + per);
  int subs = 0;
  for (int bh = lo; bh < hi; ++bh) subs += (clamped_tokens(a, bh) + 15) >> 4;
  int total = 0;
  block_exclusive_scan_256(subs, s_tmp, &total);
  const int cp = chunk_subpages<4>(total, a.target_chunks);
  int chunks = 0;
  for (int bh = lo; bh < hi; ++bh) {
    const int ns = (clamped_tokens(a, bh) + 15) >> 4;
    chunks += max(1, (ns + cp - 1) / cp);
  }
  int n_chunks = 0;
  int run = block_exclusive_scan_256(chunks, s_tmp, &n_chunks);
  for (int bh = lo; bh < hi; ++bh) {
    s_pref[bh] = run;
    const int ns = (clamped_tokens(a, bh) + 15) >> 4;
    run += max(1, (ns + cp - 1) / cp);
  }
  if (t == 0) s_pref[BH] = n_chunks;
  __syncthreads();
  if (w == 0)
    for (int i = t; i <= BH; i += kPlanThreads) a.plan[i] = s_pref[i];
  int l = 0, h = BH - 1;  // largest bh with s_pref[bh] <= w
  while (l < h) {
    const int mid = (l + h + 1) >> 1;
    if (s_pref[mid] <= w) l = mid; else h = mid - 1;
  }
  Plan p;
  p.n_chunks = n_chunks;
  p.cp = cp;
  p.bh = l;
  p.first = s_pref[l];
  p.n_bh = s_pref[l + 1] - s_pref[l];
  return p;
}

// First pool row (token slot) of sub-page `sp` of a head; page ids outside
// the pool are clamped so that a corrupt table cannot read out of bounds.
__device__ __forceinline__ int64_t subpage_row(const DecodeArgs& a, const int32_t* bt_row, int sp) {
  int pg = bt_row[sp >> a.page_shift];
  pg = pg < 0 ? 0 : (pg >= a.num_pages ? (int)(a.num_pages - 1) : pg);
  const int within = sp & ((1 << a.page_shift) - 1);
  return (int64_t)pg * a.page_size + within * 16;
}

// K of 4 sub-pages in the MFMA B-operand layout: lane (n, g) holds row n,
// 16-byte slice j*4+g, for k-step j.  One load instruction reads 64 bytes of
// each of 16 rows, half of a 128-byte line; the other half is the next
// k-step's.  These loads therefore use the default cache policy, so the
// second half comes from L2.  As non-temporal loads the line was fetched
// again: 3.6 % slower at batch 8, 12.6 % at batch 1.
template <int D>
__device__ __forceinline__ void load_k(const DecodeArgs& a, u32x4_t (&kr)[4][D / 32], const int64_t (&off)[4],
                                       int n, int g) {
#pragma unroll
  for (int p = 0; p < 4; ++p)
#pragma unroll
    for (int j = 0; j < D / 32; ++j) kr[p][j] = *(const u32x4_t*)(a.kc + off[p] + n * D + (j * 4 + g) * 8);
}

// V of 4 sub-pages, fully coalesced: load i covers rows i*RPI .. i*RPI+RPI-1
// of the quad, lane -> (row lane/CH, 16-byte slice lane%CH).  Every line is
// read whole by one instruction and never again: non-temporal loads (the
// default policy measured 4 % slower at batch 8).
template <int D>
__device__ __forceinline__ void load_v(const DecodeArgs& a, u32x4_t (&vr)[D / 8], const int64_t (&off)[4],
                                       int lane) {
  constexpr int CH = D / 8, RPI = 64 / CH;
#pragma unroll
  for (int i = 0; i < 64 / RPI; ++i) {
    const int r = i * RPI + lane / CH;
    const int p = (i * RPI) >> 4;
    vr[i] = __builtin_nontemporal_load((const u32x4_t*)(a.vc + off[p] + (r & 15) * D + (lane % CH) * 8));
  }
}

typedef __attribute__((__vector_size__(2 * sizeof(__bf16)))) __bf16 bf16x2_t;
// c + a.lo * b.lo + a.hi * b.hi for packed bf16 pairs, fp32 accumulation
__device__ __forceinline__ float dot2_bf16(uint32_t a, uint32_t b, float c) {
  return __builtin_amdgcn_fdot2_f32_bf16(__builtin_bit_cast(bf16x2_t, a), __builtin_bit_cast(bf16x2_t, b), c, false);
}

// Device-coherent accesses to the split partials.  The stores write through
// to the point of coherence of the whole device and the loads do not return
// a line that another XCD's writes left stale in this XCD's L2 (agent-scope
// relaxed atomics: sc1 on gfx950; buffer cache-policy bit 4 for the 16-byte
// loads).  No L2 writeback or invalidation is needed then: release/acquire
// fences at device scope write back and invalidate whole L2s, which also
// drops the K lines the other workgroups of the XCD are reading.
__device__ __forceinline__ void store_coherent(float* p, float v) {
  __hip_atomic_store(p, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ float load_coherent(const float* p) {
  return __hip_atomic_load(p, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ f32x4_t load_coherent4(__amdgpu_buffer_rsrc_t r, int byte_off) {
  return __builtin_bit_cast(f32x4_t, __builtin_amdgcn_raw_buffer_load_b128(r, byte_off, 0, 16));
}

template <int D, int G, int NW>
__global__ __launch_bounds__(NW * 64) __attribute__((amdgpu_waves_per_eu(waves_per_simd(G, NW), waves_per_simd(G, NW))))
void decode_split_kernel(DecodeArgs a) {
  constexpr int kThreads = NW * 64;
  constexpr int KS = D / 32;       // MFMA k-steps per row
  constexpr int CH = D / 8;        // 16-byte slices per row
  constexpr int RPI = 64 / CH;     // rows per coalesced V load
  constexpr int NV = 64 / RPI;     // V loads per quad
  constexpr int NG = (G + 3) / 4;  // groups of 4 query heads (MFMA A operands)
  static_assert(G <= kMaxG, "query heads per KV head");
  static_assert(NW == 4 || (NW == 8 && G <= 4), "4-wave workgroups, or 8-wave ones for G <= 4");

  constexpr bool kFused = NW > 4;  // the last chunk of a head merges (see top)
  // s_buf: each wave's (RPI, G, D) accumulators, then the fused merge's
  // group partials (kThreads x (m, l, float4 acc))
  constexpr int kBufFloats = NW * RPI * G * D > (kFused ? kThreads * 6 : 0) ? NW * RPI * G * D : kThreads * 6;
  __shared__ f32x4_t s_p[NW][NG][64];
  __shared__ __attribute__((aligned(16))) float s_buf[kBufFloats];
  __shared__ float s_ml[NW][2][G];
  __shared__ int s_last;

  const int w = blockIdx.x;
  Plan pl;
  if constexpr (NW == 4) {
    __shared__ int s_pref[kMaxBH + 1];
    __shared__ int s_tmp[kPlanThreads];
    pl = a.B * a.Hkv <= kWaveBH ? plan_wave<NW>(a, w) : plan_block(a, w, s_pref, s_tmp);
  } else {
    pl = plan_wave<NW>(a, w);  // the host takes 8 waves only for B*Hkv < 32
  }
  if (w >= pl.n_chunks) return;
  const int bh = pl.bh;
  const int ci = w - pl.first;
  const int b = bh / a.Hkv, h = bh - b * a.Hkv;
  const int T = clamped_tokens(a, bh);
  const int nsub = (T + 15) >> 4;
  const int s0 = ci * pl.cp;
  const int s1 = min(nsub, s0 + pl.cp);
  const int tok_end = min(T, s1 * 16);

  // wid is wave-uniform: the quad bookkeeping, page-table reads and row
  // addresses then live in scalar registers
  const int lane = threadIdx.x & 63, wid = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int n = lane & 15, g = lane >> 4;
  const int32_t* bt_row = a.bt + (int64_t)b * a.bt_sb + (int64_t)h * a.bt_sh;

  // Query heads as the MFMA A operands: row m of group gi holds head
  // 4*gi + m%4 (zero if >= G).
  bf16x8_t qa[NG][KS];
#pragma unroll
  for (int gi = 0; gi < NG; ++gi) {
    const int qh = 4 * gi + (n & 3);
    const uint16_t* qrow = a.q + (int64_t)b * a.q_sb + (int64_t)(h * G + (qh < G ? qh : 0)) * a.q_sh;
#pragma unroll
    for (int j = 0; j < KS; ++j) {
      u32x4_t v = *(const u32x4_t*)(qrow + (j * 4 + g) * 8);
      if (qh >= G) v = (u32x4_t){0u, 0u, 0u, 0u};
      qa[gi][j] = __builtin_bit_cast(bf16x8_t, v);
    }
  }

  float m_run[G], l_lane[G], acc[G][8];
#pragma unroll
  for (int i = 0; i < G; ++i) {
    m_run[i] = -INFINITY;
    l_lane[i] = 0.f;
#pragma unroll
    for (int e = 0; e < 8; ++e) acc[i][e] = 0.f;
  }

  const int nq = (s1 - s0 + 3) >> 2;
  for (int jq = wid; jq < nq; jq += NW) {
    const int sp0 = s0 + jq * 4;
    int64_t off[4];
#pragma unroll
    for (int p = 0; p < 4; ++p) off[p] = subpage_row(a, bt_row, min(sp0 + p, s1 - 1)) * D;
    u32x4_t kr[4][KS];
    u32x4_t vr[NV];
    load_k<D>(a, kr, off, n, g);
    load_v<D>(a, vr, off, lane);

    f32x4_t c[NG][4];
#pragma unroll
    for (int gi = 0; gi < NG; ++gi)
#pragma unroll
      for (int p = 0; p < 4; ++p) {
        c[gi][p] = (f32x4_t){0.f, 0.f, 0.f, 0.f};
#pragma unroll
        for (int j = 0; j < KS; ++j)
          c[gi][p] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(qa[gi][j], __builtin_bit_cast(bf16x8_t, kr[p][j]),
                                                             c[gi][p], 0, 0, 0);
      }

    // Softmax in the log2 domain with a lazy running maximum: m_run of a
    // head moves only when a score of the quad exceeds it by more than
    // kRescaleSlack (then to the quad's maximum, rescaling l and acc), so
    // p <= 2^kRescaleSlack and most quads need neither a maximum nor a
    // rescale -- one compare and ballot per head.  Lane (n, g) holds token n
    // of sub-page g (rows 4g..4g+3 of its MFMA are the group's heads).
    const bool ok = (sp0 + g) * 16 + n < tok_end;
    float s[G], pr[NG][4];
#pragma unroll
    for (int i = 0; i < G; ++i) {
      const f32x4_t* cg = c[i / 4];
      const float x = g == 0 ? cg[0][i % 4] : g == 1 ? cg[1][i % 4] : g == 2 ? cg[2][i % 4] : cg[3][i % 4];
      s[i] = ok ? x * a.scale_log2 : -INFINITY;
    }
    uint64_t up_any = 0;
#pragma unroll
    for (int i = 0; i < G; ++i) up_any |= __builtin_amdgcn_ballot_w64(s[i] > m_run[i] + kRescaleSlack);
    if (up_any) {
#pragma unroll
      for (int i = 0; i < G; ++i) {
        if (__builtin_amdgcn_ballot_w64(s[i] > m_run[i] + kRescaleSlack) == 0) continue;
        const float mn = wave_max(s[i]);  // > m_run[i] + slack
        const float alpha = fast_exp2(m_run[i] - mn);  // 0 when m_run was -inf
        m_run[i] = mn;
        l_lane[i] *= alpha;
#pragma unroll
        for (int e = 0; e < 8; ++e) acc[i][e] *= alpha;
      }
    }
#pragma unroll
    for (int gi = 0; gi < NG; ++gi)
#pragma unroll
      for (int i = 0; i < 4; ++i) pr[gi][i] = 0.f;
#pragma unroll
    for (int i = 0; i < G; ++i) {
      // m_run is -inf only while every score seen is -inf: p = 0 then
      pr[i / 4][i % 4] = fast_exp2(s[i] - (m_run[i] == -INFINITY ? 0.f : m_run[i]));
      l_lane[i] += pr[i / 4][i % 4];
    }
#pragma unroll
    for (int gi = 0; gi < NG; ++gi)
      s_p[wid][gi][g * 16 + n] = (f32x4_t){pr[gi][0], pr[gi][1], pr[gi][2], pr[gi][3]};
    wave_lds_sync();

    // P V on v_dot2_f32_bf16: the lane's rows are paired (load i, load i+1)
    // so that one instruction adds p_r * v_r + p_r' * v_r' for one d; the
    // probabilities are rounded to bf16 for the product, as the reference's
    // kernel does (src/modeling_layers.py:930-931).
    const bool full = sp0 * 16 + 64 <= tok_end;
#pragma unroll
    for (int i = 0; i < NV; i += 2) {
      const int r0 = i * RPI + lane / CH, r1 = r0 + RPI;
      u32x4_t v0 = vr[i], v1 = vr[i + 1];
      if (!full && sp0 * 16 + r0 >= tok_end) v0 = (u32x4_t){0u, 0u, 0u, 0u};
      if (!full && sp0 * 16 + r1 >= tok_end) v1 = (u32x4_t){0u, 0u, 0u, 0u};
      uint32_t pp[G];
#pragma unroll
      for (int gi = 0; gi < NG; ++gi) {
        const f32x4_t p0 = s_p[wid][gi][r0];
        const f32x4_t p1 = s_p[wid][gi][r1];
#pragma unroll
        for (int qi = 4 * gi; qi < G && qi < 4 * gi + 4; ++qi) pp[qi] = pack_bf16x2(p0[qi % 4], p1[qi % 4]);
      }
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        // (v0.d, v1.d) for d = 2e (low halves) and d = 2e+1 (high halves)
        const uint32_t lo = __builtin_amdgcn_perm(v1[e], v0[e], 0x05040100u);
        const uint32_t hi = __builtin_amdgcn_perm(v1[e], v0[e], 0x07060302u);
#pragma unroll
        for (int qi = 0; qi < G; ++qi) {
          acc[qi][2 * e] = dot2_bf16(lo, pp[qi], acc[qi][2 * e]);
          acc[qi][2 * e + 1] = dot2_bf16(hi, pp[qi], acc[qi][2 * e + 1]);
        }
      }
    }
    wave_lds_sync();
  }

  // ---- merge the waves -----------------------------------------------------
#pragma unroll
  for (int i = 0; i < G; ++i) {
    const float lw = wave_sum(l_lane[i]);
    if (lane == 0) {
      s_ml[wid][0][i] = m_run[i];
      s_ml[wid][1][i] = lw;
    }
  }
  {
    // s_acc[wid][slot][i][d]: the RPI lanes that hold the same d summed rows
    // of different V loads
    const int slot = lane / CH, cc = lane % CH;
#pragma unroll
    for (int i = 0; i < G; ++i)
#pragma unroll
      for (int e = 0; e < 8; ++e) s_buf[((wid * RPI + slot) * G + i) * D + cc * 8 + e] = acc[i][e];
  }
  __syncthreads();

  const bool single = pl.n_bh == 1;
  for (int v = threadIdx.x; v < G * D; v += kThreads) {
    const int i = v / D, d = v - i * D;
    float M = -INFINITY;
#pragma unroll
    for (int ww = 0; ww < NW; ++ww) M = fmaxf(M, s_ml[ww][0][i]);
    float L = 0.f, A = 0.f;
#pragma unroll
    for (int ww = 0; ww < NW; ++ww) {
      const float mw = s_ml[ww][0][i];
      if (mw == -INFINITY) continue;
      const float sc = fast_exp2(mw - M);
      float sum = 0.f;
#pragma unroll
      for (int sl = 0; sl < RPI; ++sl) sum += s_buf[((ww * RPI + sl) * G + i) * D + d];
      L = fmaf(sc, s_ml[ww][1][i], L);
      A = fmaf(sc, sum, A);
    }
    if (single) {
      const float o = L > 0.f ? A / L : 0.f;
      a.out[(int64_t)b * a.out_sb + (int64_t)(h * G + i) * a.out_sh + d] = f32_to_bf16(o);
    } else if constexpr (kFused) {
      if (d == 0) {
        store_coherent(&a.part_m[w * G + i], M);
        store_coherent(&a.part_l[w * G + i], L);
      }
      store_coherent(&a.part_acc[((int64_t)w * G + i) * D + d], A);
    } else {
      if (d == 0) {
        a.part_m[w * G + i] = M;
        a.part_l[w * G + i] = L;
      }
      a.part_acc[((int64_t)w * G + i) * D + d] = A;
    }
  }
  if (single) return;
  if constexpr (!kFused) return;  // decode_merge_kernel follows

  // ---- the last chunk of the head to arrive merges its partials -------------
  // Why the partials are visible to the last arriver without release /
  // acquire fences (this is gfx950 hardware ordering, not the HIP memory
  // model, whose relaxed atomics order nothing across addresses):
  //  1. every partial is an agent-scope store (sc1): it is written through
  //     the XCD's L2 to the device's point of coherence;
  //  2. on gfx950 stores are counted by vmcnt, which drops only when the
  //     memory system acknowledges the write, so after vmcnt(0) this wave's
  //     partials are at the point of coherence;
  //  3. the barrier holds thread 0's arrival atomic until every wave of the
  //     workgroup has passed its vmcnt(0);
  //  4. the arrival counter is an agent-scope atomic, performed at the point
  //     of coherence, so the workgroup that reads n_bh - 1 comes after every
  //     other chunk's arrival, hence after all their partial stores;
  //  5. the last arriver reads the partials with sc1 loads, which are not
  //     served from a possibly stale copy in its own XCD's L2.
  // The signal fences are compiler-only barriers: they keep the compiler
  // from sinking the partial stores below the wait or hoisting the merge's
  // loads above the arrival.  A device-scope release/acquire pair would
  // write back and invalidate the whole L2 (1.7x slower in a trial).
#if defined(__HIP_DEVICE_COMPILE__) && !defined(__gfx950__)
#error "the fused decode merge relies on gfx950 store acknowledgement and sc1 ordering"
#endif
  __atomic_signal_fence(__ATOMIC_SEQ_CST);
  __builtin_amdgcn_s_waitcnt(0x0F70);  // vmcnt(0)
  __atomic_signal_fence(__ATOMIC_SEQ_CST);
  __syncthreads();
  if (threadIdx.x == 0) {
    const int prev = __hip_atomic_fetch_add(&a.counter[bh], 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    const int last = prev == pl.n_bh - 1;
    if (last) __hip_atomic_store(&a.counter[bh], 0, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    s_last = last;
  }
  __syncthreads();
  if (!s_last) return;
  __atomic_signal_fence(__ATOMIC_SEQ_CST);

  // Thread t sums the float4 quad t % NQ of the head's (G, D) output over the
  // chunks grp, grp + GROUPS, ... of the head (grp = t / NQ), all loads of a
  // batch issued before the (branch-free) online update consumes them; the
  // groups are then combined through LDS in group order.  8-wave workgroups
  // read the ~32 partials of a batch-1 head (G = 4, D = 128) in one round of
  // loads.
  constexpr int NQ = G * D / 4;
  constexpr int GROUPS = kThreads / NQ;
  constexpr int kBatch = 8;
  static_assert(GROUPS >= 1, "one float4 quad per thread at least");
  const int t = threadIdx.x;
  const int c0 = pl.first, c1 = pl.first + pl.n_bh;
  const int vq = t % NQ, grp = t / NQ;
  const int i = (vq * 4) / D;
  float M = -INFINITY, L = 0.f;
  f32x4_t A = (f32x4_t){0.f, 0.f, 0.f, 0.f};
  if (grp < GROUPS) {
    const __amdgpu_buffer_rsrc_t acc_rsrc =
        __builtin_amdgcn_make_buffer_rsrc(a.part_acc + (int64_t)c0 * G * D, (short)0, 0x7fffffff, 0x00020000);
    for (int cb = c0 + grp; cb < c1; cb += GROUPS * kBatch) {
      float mc[kBatch], lc[kBatch];
      f32x4_t ac[kBatch];
#pragma unroll
      for (int k = 0; k < kBatch; ++k) {
        const int c = min(cb + k * GROUPS, c1 - 1);
        mc[k] = load_coherent(&a.part_m[c * G + i]);
        lc[k] = load_coherent(&a.part_l[c * G + i]);
        ac[k] = load_coherent4(acc_rsrc, ((c - c0) * G * D + vq * 4) * (int)sizeof(float));
      }
#pragma unroll
      for (int k = 0; k < kBatch; ++k) {
        const bool valid = cb + k * GROUPS < c1 && mc[k] != -INFINITY;
        const float mn = valid ? fmaxf(M, mc[k]) : M;
        const float sa = M == -INFINITY ? 0.f : fast_exp2(M - mn);
        const float sb = valid ? fast_exp2(mc[k] - mn) : 0.f;
        L = L * sa + lc[k] * sb;
        A = A * sa + ac[k] * sb;
        M = mn;
      }
    }
  }
  // s_buf is free again (read before the arrival barriers): group partials
  float* s_m = s_buf;
  float* s_l = s_m + kThreads;
  f32x4_t* s_a = (f32x4_t*)(s_l + kThreads);
  s_m[t] = M;
  s_l[t] = L;
  s_a[t] = A;
  __syncthreads();
  if (t < NQ) {
    float Mx = -INFINITY;
    for (int gg = 0; gg < GROUPS; ++gg) Mx = fmaxf(Mx, s_m[gg * NQ + t]);
    float Lt = 0.f;
    f32x4_t At = (f32x4_t){0.f, 0.f, 0.f, 0.f};
    for (int gg = 0; gg < GROUPS; ++gg) {
      const float mg = s_m[gg * NQ + t];
      if (mg == -INFINITY) continue;
      const float sc = fast_exp2(mg - Mx);
      Lt += sc * s_l[gg * NQ + t];
      At += sc * s_a[gg * NQ + t];
    }
    const float inv = Lt > 0.f ? 1.f / Lt : 0.f;
    uint16_t* o = a.out + (int64_t)b * a.out_sb + (int64_t)(h * G + i) * a.out_sh + (vq * 4 - i * D);
#pragma unroll
    for (int e = 0; e < 4; ++e) o[e] = f32_to_bf16(Lt > 0.f ? At[e] * inv : 0.f);
  }
}

// Log-sum-exp merge of a head's chunk partials in one pass, one workgroup
// per (b, h, query head i): the float4 quads of head i's row are summed by
// GROUPS thread groups over disjoint chunk subsets, each thread keeping a
// running (max, sum, acc) with all loads of a batch issued before the
// (branch-free) update consumes them; the groups are then combined through
// LDS in group order.  The plan comes from the split kernel, which ran
// before on the same stream.
template <int D, int G>
__global__ __launch_bounds__(256) void decode_merge_kernel(DecodeArgs a) {
  constexpr int kThreads = 256;
  constexpr int NQ = D / 4;
  constexpr int GROUPS = kThreads / NQ;
  __shared__ f32x4_t s_a[kThreads];
  __shared__ float s_m[kThreads], s_l[kThreads];
  const int bh = blockIdx.x;
  const int c0 = a.plan[bh], c1 = a.plan[bh + 1];
  if (c1 - c0 <= 1) return;  // written directly by the split kernel
  const int b = bh / a.Hkv, h = bh - b * a.Hkv;
  const int t = threadIdx.x;
  const int i = blockIdx.y;
  const int vq = t % NQ, grp = t / NQ;
  // 16 chunks per batch and 8 groups (D = 128) read the ~80-100 chunks of
  // a head at batch 1 in one round of loads
  constexpr int kBatch = 16;
  float M = -INFINITY, L = 0.f;
  f32x4_t A = (f32x4_t){0.f, 0.f, 0.f, 0.f};
  for (int cb = c0 + grp; cb < c1; cb += GROUPS * kBatch) {
    float mc[kBatch], lc[kBatch];
    f32x4_t ac[kBatch];
#pragma unroll
    for (int k = 0; k < kBatch; ++k) {
      const int c = min(cb + k * GROUPS, c1 - 1);
      mc[k] = a.part_m[c * G + i];
      lc[k] = a.part_l[c * G + i];
      ac[k] = *(const f32x4_t*)(a.part_acc + ((int64_t)c * G + i) * D + vq * 4);
    }
#pragma unroll
    for (int k = 0; k < kBatch; ++k) {
      const bool valid = cb + k * GROUPS < c1 && mc[k] != -INFINITY;
      const float mn = valid ? fmaxf(M, mc[k]) : M;
      const float sa = M == -INFINITY ? 0.f : fast_exp2(M - mn);
      const float sb = valid ? fast_exp2(mc[k] - mn) : 0.f;
      L = L * sa + lc[k] * sb;
      A = A * sa + ac[k] * sb;
      M = mn;
    }
  }
  s_m[t] = M;
  s_l[t] = L;
  s_a[t] = A;
  __syncthreads();
  if (t < NQ) {
    float Mx = -INFINITY;
    for (int gg = 0; gg < GROUPS; ++gg) Mx = fmaxf(Mx, s_m[gg * NQ + t]);
    float Lt = 0.f;
    f32x4_t At = (f32x4_t){0.f, 0.f, 0.f, 0.f};
    for (int gg = 0; gg < GROUPS; ++gg) {
      const float mg = s_m[gg * NQ + t];
      if (mg == -INFINITY) continue;
      const float sc = fast_exp2(mg - Mx);
      Lt += sc * s_l[gg * NQ + t];
      At += sc * s_a[gg * NQ + t];
    }
    const float inv = Lt > 0.f ? 1.f / Lt : 0.f;
    uint16_t* o = a.out + (int64_t)b * a.out_sb + (int64_t)(h * G + i) * a.out_sh + vq * 4;
#pragma unroll
    for (int e = 0; e < 4; ++e) o[e] = f32_to_bf16(Lt > 0.f ? At[e] * inv : 0.f);
  }
}

// Zeroes the arrival counters of a workspace the library owns (once).
__global__ void zero_counters_kernel(int* c, int n) {
  const int i = blockIdx.x * blockDim.x + threadIdx.x;
  if (i < n) c[i] = 0;
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

template <int D, int G, int NW>
hipError_t launch_nw(DecodeArgs a, hipStream_t st) {
  const int BH = a.B * a.Hkv;
  const int slots = min(kMaxSlots, cu_count() * wg_per_cu(G, NW));
  // The plan makes at most target_chunks + BH chunks (one remainder per
  // head; 8-wave plans stay within target_chunks).  With three workgroups
  // per CU a few chunks beyond the slots only fill the first free slots
  // (aiming at slots - BH measured 0.5 % slower at batch 8).
  a.target_chunks = slots;
  hipLaunchKernelGGL((decode_split_kernel<D, G, NW>), dim3(a.target_chunks + BH), dim3(NW * 64), 0, st, a);
  const hipError_t e = hipGetLastError();
  if (NW > 4 || e != hipSuccess) return e;
  hipLaunchKernelGGL((decode_merge_kernel<D, G>), dim3(BH, G), dim3(256), 0, st, a);
  return hipGetLastError();
}

template <int D, int G>
hipError_t launch(const DecodeArgs& a, hipStream_t st) {
  if constexpr (G <= 4) {
    if (a.B * a.Hkv < kWideBelowBH) return launch_nw<D, G, 8>(a, st);
  }
  return launch_nw<D, G, 4>(a, st);
}

template <int D>
hipError_t launch_g(const DecodeArgs& a, int G, hipStream_t st) {
  switch (G) {
    case 1: return launch<D, 1>(a, st);
    case 2: return launch<D, 2>(a, st);
    case 3: return launch<D, 3>(a, st);
    case 4: return launch<D, 4>(a, st);
    case 5: return launch<D, 5>(a, st);
    case 6: return launch<D, 6>(a, st);
    case 7: return launch<D, 7>(a, st);
    default: return launch<D, 8>(a, st);
  }
}

// Workspace layout: the arrival counters (one int per (b, h), at a fixed
// offset so that calls of either head_dim share them), the partials, then
// the plan.
constexpr size_t kCounterBytes = ((size_t)kMaxBH * sizeof(int) + 255) & ~(size_t)255;
size_t part_floats(int head_dim) { return (size_t)kMaxChunks * kMaxG * (2 + (size_t)head_dim); }

// ---- scratch of the allocation-free entry point ------------------------------
// The counters and partials of the largest supported call (head_dim 128,
// G 8, B*Hkv 2048): 12.2 MiB per device, held until the process ends.  In
// host code `scratch` names a host-side stand-in; its device address is
// looked up once per device with hipGetSymbolAddress and only that address
// is used.
constexpr size_t kScratchBytes = (kCounterBytes + (size_t)kMaxChunks * kMaxG * (2 + 128) * sizeof(float) +
                                  (size_t)(kMaxBH + 1) * sizeof(int) + 255) &
                                 ~(size_t)255;
static __device__ __align__(256) unsigned char scratch[kScratchBytes];

constexpr int kMaxDevices = 64;
std::mutex g_scratch_mu;
void* g_scratch_ptr[kMaxDevices] = {};

// Device address of `scratch` on the device that owns `stream` (the current
// device for the null stream), resolved on the first call for that device
// with the device made current for the lookup; that first call also zeroes
// the arrival counters, with a kernel on `stream` (ordered before the call's
// own launch; a fill kernel rather than a memset node if the stream is being
// captured).
int scratch_for_stream(hipStream_t stream, void** out) {
  int dev = -1;
  if (stream) {
    if (hipStreamGetDevice(stream, &dev) != hipSuccess) return WGKV_ERR_HIP;
  } else if (hipGetDevice(&dev) != hipSuccess) {
    return WGKV_ERR_HIP;
  }
  if (dev < 0 || dev >= kMaxDevices) return WGKV_ERR_UNSUPPORTED;
  std::lock_guard<std::mutex> lock(g_scratch_mu);
  if (!g_scratch_ptr[dev]) {
    int cur = -1;
    if (hipGetDevice(&cur) != hipSuccess) return WGKV_ERR_HIP;
    if (cur != dev && hipSetDevice(dev) != hipSuccess) return WGKV_ERR_HIP;
    void* p = nullptr;
    const hipError_t e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
    if (cur != dev && hipSetDevice(cur) != hipSuccess) return WGKV_ERR_HIP;
    if (e != hipSuccess || !p) return WGKV_ERR_HIP;
    if (cur != dev && hipSetDevice(dev) != hipSuccess) return WGKV_ERR_HIP;
    hipLaunchKernelGGL(zero_counters_kernel, dim3((kMaxBH + 255) / 256), dim3(256), 0, stream, (int*)p, kMaxBH);
    const hipError_t ez = hipGetLastError();
    if (cur != dev && hipSetDevice(cur) != hipSuccess) return WGKV_ERR_HIP;
    if (ez != hipSuccess) return WGKV_ERR_HIP;
    g_scratch_ptr[dev] = p;
  }
  *out = g_scratch_ptr[dev];
  return WGKV_OK;
}

}  // namespace

extern "C" size_t wgkv_paged_decode_workspace_bytes(int32_t batch, int32_t num_kv_heads, int32_t head_dim) {
  (void)batch;
  (void)num_kv_heads;
  return kCounterBytes + part_floats(head_dim > 0 ? head_dim : 0) * sizeof(float) + (size_t)(kMaxBH + 1) * sizeof(int);
}

extern "C" int wgkv_paged_decode_attn(
    const void* q, int64_t q_stride_b, int64_t q_stride_h,
    const void* k_cache, const void* v_cache, int64_t num_pages, int32_t page_size,
    const int32_t* cache_seqlens, int64_t sl_stride_b,
    const int32_t* block_table, int64_t bt_stride_b, int64_t bt_stride_h, int32_t max_pages,
    void* out, int64_t out_stride_b, int64_t out_stride_h,
    int32_t batch, int32_t num_q_heads, int32_t num_kv_heads, int32_t head_dim,
    float softmax_scale,
    void* workspace, size_t workspace_bytes,
    void* stream) {
  if (!q || !k_cache || !v_cache || !cache_seqlens || !block_table || !out) return WGKV_ERR_ARG;
  if (batch <= 0 || num_kv_heads <= 0 || num_q_heads <= 0 || num_pages <= 0 || max_pages <= 0) return WGKV_ERR_ARG;
  if (num_q_heads % num_kv_heads) return WGKV_ERR_ARG;
  if ((int64_t)batch * num_kv_heads > kMaxBH) return WGKV_ERR_UNSUPPORTED;
  const int G = num_q_heads / num_kv_heads;
  if (head_dim != 64 && head_dim != 128) return WGKV_ERR_UNSUPPORTED;
  if (G < 1 || G > kMaxG) return WGKV_ERR_UNSUPPORTED;
  int shift;
  if (page_size == 16) shift = 0;
  else if (page_size == 32) shift = 1;
  else if (page_size == 64) shift = 2;
  else return WGKV_ERR_UNSUPPORTED;
  // 16-byte vector loads: rows and bases must be 16-byte aligned.
  if (((uintptr_t)q | (uintptr_t)k_cache | (uintptr_t)v_cache) & 15) return WGKV_ERR_UNSUPPORTED;
  if ((q_stride_b | q_stride_h) & 7) return WGKV_ERR_UNSUPPORTED;
  if (!workspace || workspace_bytes < wgkv_paged_decode_workspace_bytes(batch, num_kv_heads, head_dim) ||
      ((uintptr_t)workspace & 15))
    return WGKV_ERR_WORKSPACE;

  DecodeArgs a;
  a.q = (const uint16_t*)q;
  a.q_sb = q_stride_b;
  a.q_sh = q_stride_h;
  a.kc = (const uint16_t*)k_cache;
  a.vc = (const uint16_t*)v_cache;
  a.num_pages = num_pages;
  a.page_size = page_size;
  a.page_shift = shift;
  a.seqlens = cache_seqlens;
  a.sl_sb = sl_stride_b;
  a.bt = block_table;
  a.bt_sb = bt_stride_b;
  a.bt_sh = bt_stride_h;
  a.max_pages = max_pages;
  a.out = (uint16_t*)out;
  a.out_sb = out_stride_b;
  a.out_sh = out_stride_h;
  a.B = batch;
  a.Hkv = num_kv_heads;
  a.scale_log2 = softmax_scale * kLog2e;
  a.counter = (int*)workspace;
  float* ws = (float*)((char*)workspace + kCounterBytes);
  a.part_m = ws;
  a.part_l = ws + (size_t)kMaxChunks * kMaxG;
  a.part_acc = ws + (size_t)kMaxChunks * kMaxG * 2;
  a.plan = (int*)(ws + part_floats(head_dim));

  hipStream_t st = (hipStream_t)stream;
  const hipError_t e = head_dim == 128 ? launch_g<128>(a, G, st) : launch_g<64>(a, G, st);
  return e == hipSuccess ? WGKV_OK : WGKV_ERR_HIP;
}

extern "C" int wgkv_paged_decode_attn_noalloc(
    const void* q, int64_t q_stride_b, int64_t q_stride_h,
    const void* k_cache, const void* v_cache, int64_t num_pages, int32_t page_size,
    const int32_t* cache_seqlens, int64_t sl_stride_b,
    const int32_t* block_table, int64_t bt_stride_b, int64_t bt_stride_h, int32_t max_pages,
    void* out, int64_t out_stride_b, int64_t out_stride_h,
    int32_t batch, int32_t num_q_heads, int32_t num_kv_heads, int32_t head_dim,
    float softmax_scale, void* stream) {
  if (batch <= 0 || num_kv_heads <= 0 || head_dim <= 0) return WGKV_ERR_ARG;
  if ((int64_t)batch * num_kv_heads > kMaxBH || head_dim > 128) return WGKV_ERR_UNSUPPORTED;
  if (wgkv_paged_decode_workspace_bytes(batch, num_kv_heads, head_dim) > kScratchBytes) return WGKV_ERR_WORKSPACE;
  void* ws = nullptr;
  const int st = scratch_for_stream((hipStream_t)stream, &ws);
  if (st != WGKV_OK) return st;
  return wgkv_paged_decode_attn(q, q_stride_b, q_stride_h, k_cache, v_cache, num_pages, page_size, cache_seqlens,
                                sl_stride_b, block_table, bt_stride_b, bt_stride_h, max_pages, out, out_stride_b,
                                out_stride_h, batch, num_q_heads, num_kv_heads, head_dim, softmax_scale, ws,
                                kScratchBytes, stream);
}
