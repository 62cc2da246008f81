// Write-gate MLP scores and admission flags (gfx950, fp32).
//
// Replaces GatingPredictor.forward (src/modeling_layers.py:170-205) with the
// RMS norms of GatingRMSNorm (:113-131) and the threshold of :1465:
//   x  = concat(rms(pre_k)*w_pre, rms(post_k)*w_post[, rms(v)*w_v])   (n_in*D)
//   h  = act(W1[h] x + b1[h])                                        (inner)
//   g  = sigmoid(w2[h] . h + b2[h]);  conv path: g = max(g, clamp_min)
//   mask = g > threshold
// Two arithmetics (GateArgs::prec): fp32 parameters (fp32 from the normalised
// inputs on, as the reference with fp32 gate weights), or bf16 parameters
// (the reference's inference: the gate checkpoint loads in bf16) where every
// op's result is rounded to bf16 -- the norm product, the first layer's
// output (fast path: einsum output, then the bias add; conv path: one
// rounding after the bias), the activation, the second layer likewise, the
// sigmoid -- and the score is compared with bf16(threshold).
// One workgroup = 64 tokens of one (batch, KV head), heads dealt across the
// XCDs so each head's W1 stays in one L2.  The normalised inputs
// go to LDS (fp32, rows padded for conflict-free 16-byte reads); the hidden
// columns are dealt round-robin to the 4 waves in 16-column tiles, so W1[h]
// is read once per workgroup; x @ W1^T runs on v_mfma_f32_16x16x4f32 with
// each lane feeding four consecutive k from one 16-byte load; the epilogue
// applies bias, activation and w2 and reduces over columns in registers.
#include <string.h>

#include "wgkv_common.h"

namespace {

constexpr int kThreads = 256;
constexpr int kTok = 64;

struct GateArgs {
  const void* in[3];
  int64_t sb[3], sh[3], ss[3];
  int n_in, in_f32, rms;
  const float* w_norm[3];
  const float* w1;
  const float* b1;
  const float* w2;
  const float* b2;
  int B, H, S, D, inner, act;
  int prec;  // 0 fp32 parameters, 1 bf16 parameters (fast path), 2 bf16 parameters (conv path)
  float clamp_min, threshold;
  float* scores;
  int64_t sc_sb, sc_sh;
  uint8_t* mask;
  int64_t mk_sb, mk_sh;
  // few-token kernel: hidden columns split over nsplit workgroups per head;
  // partial logits part[(bh*nsplit + split)*kSmallTok + t], arrival counters
  // counter[bh] (zero between launches)
  int nsplit;
  float* part;
  int32_t* counter;
  // when set, the launch does nothing unless *active == active_value (a
  // condition decided on the device, e.g. by a captured decode step)
  const int32_t* active;
  int active_value;
};

__device__ __forceinline__ bool inactive(const GateArgs& a) {
  return a.active != nullptr && *a.active != a.active_value;
}

__device__ __forceinline__ float load_in(const GateArgs& a, int i, int b, int h, int s, int d) {
  const int64_t off = (int64_t)b * a.sb[i] + (int64_t)h * a.sh[i] + (int64_t)s * a.ss[i] + d;
  if (a.in_f32) return ((const float*)a.in[i])[off];
  return __uint_as_float((uint32_t)((const uint16_t*)a.in[i])[off] << 16);
}

__device__ __forceinline__ float round_bf16(float x) { return round_to_bf16(x); }

__device__ __forceinline__ float gelu_erf(float z) { return 0.5f * z * (1.0f + erff(z * 0.70710678118654752f)); }
__device__ __forceinline__ float silu(float z) { return z / (1.0f + expf(-z)); }

// Layer output from the fp32 accumulation and the bias, at the rounding
// points of the arithmetic prec (0: none; 1: einsum output, then the bias
// add; 2: one rounding after the bias).
__device__ __forceinline__ float layer_out(float acc, float bias, int prec) {
  if (prec == 1) return round_bf16(round_bf16(acc) + bias);
  if (prec == 2) return round_bf16(acc + bias);
  return acc + bias;
}

__device__ __forceinline__ float activation(float z, int act, int prec) {
  const float r = act ? silu(z) : gelu_erf(z);
  return prec ? round_bf16(r) : r;
}

// Normalised input element y times its norm weight (rounded with bf16 parameters).
__device__ __forceinline__ float norm_out(float w, float y, int prec) { return prec ? round_bf16(w * y) : w * y; }

// Score and admission flag from the second layer's fp32 sum z (before b2).
__device__ __forceinline__ float score_of(const GateArgs& a, float z, float b2) {
  z = layer_out(z, b2, a.prec);
  float g = 1.0f / (1.0f + expf(-z));
  if (a.prec) g = round_bf16(g);
  if (a.clamp_min > 0.f) g = fmaxf(g, a.clamp_min);
  return g;
}

// End of a 64-token tile: lane (n, kq) holds partial logits of tokens
// mt*16 + 4*kq + i over its columns; sum over the 16 lanes of each row, then
// over the 4 waves, and apply b2, sigmoid, clamp and threshold.
__device__ __forceinline__ void finish_tile(const GateArgs& a, const float (&logit)[4][4], float (*s_part)[kTok],
                                            int lane, int wid, int b, int h, int s0) {
  const int n = lane & 15, kq = lane >> 4;
#pragma unroll
  for (int mt = 0; mt < 4; ++mt)
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const float v = row_sum16(logit[mt][i]);
      if (n == 0) s_part[wid][mt * 16 + 4 * kq + i] = v;
    }
  __syncthreads();
  if (threadIdx.x < kTok) {
    const int m = threadIdx.x;
    const int s = s0 + m;
    if (s < a.S) {
      const float g = score_of(a, (s_part[0][m] + s_part[1][m]) + (s_part[2][m] + s_part[3][m]), a.b2[h]);
      if (a.scores) a.scores[(int64_t)b * a.sc_sb + (int64_t)h * a.sc_sh + s] = g;
      if (a.mask) a.mask[(int64_t)b * a.mk_sb + (int64_t)h * a.mk_sh + s] = g > a.threshold ? 1 : 0;
    }
  }
}

template <int K>  // n_in * D
__global__ __launch_bounds__(kThreads) void gate_kernel(GateArgs a) {
  constexpr int LDX = K + 4;  // padded row (floats)
  __shared__ float xs[kTok * LDX];
  __shared__ float s_part[4][kTok];
  if (inactive(a)) return;
  const int lane = threadIdx.x & 63, wid = threadIdx.x >> 6;
  // XCD-aware order: workgroups are dealt to the 8 XCDs round-robin by linear
  // id, so taking (batch, head) = id mod B*H keeps each head's workgroups on
  // few XCDs and its W1 resident in their L2
  const int nbh = a.B * a.H;
  const int lid = blockIdx.x + blockIdx.y * gridDim.x;
  const int bh = lid % nbh, tile = lid / nbh;
  const int b = bh / a.H, h = bh - b * a.H;
  const int s0 = tile * kTok;
  const int D = a.D;

  // ---- normalised inputs -> LDS: wave w handles tokens w*16 .. w*16+15 ----
  // Four tokens at a time: all their input loads are issued before the first
  // reduction, so the load latency is paid four times per wave, not sixteen.
  constexpr int kGroup = 4;
  for (int tt0 = 0; tt0 < 16; tt0 += kGroup) {
    float v[kGroup][3][2];
#pragma unroll
    for (int u = 0; u < kGroup; ++u) {
      const int s = min(s0 + wid * 16 + tt0 + u, a.S - 1);  // rows past S are computed and discarded
#pragma unroll
      for (int i = 0; i < 3; ++i)
#pragma unroll
        for (int e = 0; e < 2; ++e) {
          const int d = lane + e * 64;
          v[u][i][e] = (i < a.n_in && d < D) ? load_in(a, i, b, h, s, d) : 0.f;
        }
    }
#pragma unroll
    for (int u = 0; u < kGroup; ++u) {
      const int m = wid * 16 + tt0 + u;
#pragma unroll
      for (int i = 0; i < 3; ++i) {
        if (i >= a.n_in) break;
        float scale = 1.f;
        if (a.rms) {
          const float var = wave_sum(v[u][i][0] * v[u][i][0] + v[u][i][1] * v[u][i][1]) / (float)D;
          scale = 1.0f / sqrtf(var + 1e-6f);
        }
#pragma unroll
        for (int e = 0; e < 2; ++e) {
          const int d = lane + e * 64;
          if (d < D) {
            float y = a.rms ? v[u][i][e] * scale : v[u][i][e];
            if (a.rms && !a.in_f32) y = round_bf16(y);  // cast back to the input dtype (:128)
            xs[m * LDX + i * D + d] = a.rms ? norm_out(a.w_norm[i][d], y, a.prec) : y;
          }
        }
      }
    }
  }
  __syncthreads();

  // ---- x @ W1[h]^T on fp32 MFMA, epilogue act(. + b1) . w2 ----------------
  const int n = lane & 15, kq = lane >> 4;
  const int ntot = a.inner / 16;  // 16-column tiles of the hidden layer
  const float* w1h = a.w1 + (int64_t)h * a.inner * K;
  const float* b1h = a.b1 + (int64_t)h * a.inner;
  const float* w2h = a.w2 + (int64_t)h * a.inner;
  float logit[4][4];  // [m-tile][row i] partial logits of tokens mt*16 + 4*kq + i
#pragma unroll
  for (int mt = 0; mt < 4; ++mt)
#pragma unroll
    for (int i = 0; i < 4; ++i) logit[mt][i] = 0.f;

  for (int t0 = wid; t0 < ntot; t0 += 16) {  // up to 4 column tiles t0, t0+4, t0+8, t0+12
    f32x4_t c[4][4];
#pragma unroll
    for (int mt = 0; mt < 4; ++mt)
#pragma unroll
      for (int j = 0; j < 4; ++j) c[mt][j] = (f32x4_t){0.f, 0.f, 0.f, 0.f};
    int cols[4];
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const int tj = t0 + 4 * j;
      cols[j] = (tj < ntot ? tj : t0) * 16 + n;  // out-of-range tiles recompute tile t0 and are skipped below
    }
    // W1 slices of the next k-step are loaded while this step's MFMAs run
    f32x4_t bw[4];
#pragma unroll
    for (int j = 0; j < 4; ++j) bw[j] = *(const f32x4_t*)(w1h + (int64_t)cols[j] * K + 4 * kq);
#pragma unroll 1
    for (int k0 = 0; k0 < K; k0 += 16) {
      f32x4_t bwn[4], ax[4];
      if (k0 + 16 < K)
#pragma unroll
        for (int j = 0; j < 4; ++j) bwn[j] = *(const f32x4_t*)(w1h + (int64_t)cols[j] * K + k0 + 16 + 4 * kq);
#pragma unroll
      for (int mt = 0; mt < 4; ++mt) ax[mt] = *(const f32x4_t*)(&xs[(mt * 16 + n) * LDX + k0 + 4 * kq]);
#pragma unroll
      for (int e = 0; e < 4; ++e)
#pragma unroll
        for (int mt = 0; mt < 4; ++mt)
#pragma unroll
          for (int j = 0; j < 4; ++j)
            c[mt][j] = __builtin_amdgcn_mfma_f32_16x16x4f32(ax[mt][e], bw[j][e], c[mt][j], 0, 0, 0);
      if (k0 + 16 < K)
#pragma unroll
        for (int j = 0; j < 4; ++j) bw[j] = bwn[j];
    }
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      if (t0 + 4 * j >= ntot) break;
      const float bias = b1h[cols[j]], wo = w2h[cols[j]];
#pragma unroll
      for (int mt = 0; mt < 4; ++mt)
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          const float z = layer_out(c[mt][j][i], bias, a.prec);
          logit[mt][i] = fmaf(wo, activation(z, a.act, a.prec), logit[mt][i]);
        }
    }
  }
  finish_tile(a, logit, s_part, lane, wid, b, h, s0);
}

// Few tokens (decode steps, S <= kSmallTok).  The hidden columns of a head
// are split over nsplit workgroups of 4 waves, 64 columns each, so a head's
// W1 streams through many CUs at once; within a wave the lanes split the K
// dimension (each W1 row is one coalesced load per wave) and the wave takes
// 16 columns.  Per column the lane partials are summed over the wave; lane
// i < 16 then applies bias, activation and w2 for column i.  Each workgroup
// stores its partial logits; the last workgroup of the head to arrive (a
// device-scope counter, reset to zero by that workgroup) adds the partials in
// split order and applies sigmoid, clamp and threshold, so results do not
// depend on arrival order.  Without a workspace (nsplit = 1) one workgroup
// takes all columns.
// Sums over the wave of 16 per-lane values at once (a transposing
// butterfly: at each exchange a lane keeps half of its values and adds the
// partner's copy of that half).  Returns, in lane l, the wave-wide sum of
// v[(l >> 2) & 15].
__device__ __forceinline__ float reduce16_columns(const float (&v)[16], int lane) {
  float a8[8], a4[4], a2[2];
  const bool b5 = lane & 32, b4 = lane & 16, b3 = lane & 8, b2 = lane & 4;
#pragma unroll
  for (int i = 0; i < 8; ++i) a8[i] = (b5 ? v[8 + i] : v[i]) + __shfl_xor(b5 ? v[i] : v[8 + i], 32);
#pragma unroll
  for (int i = 0; i < 4; ++i) a4[i] = (b4 ? a8[4 + i] : a8[i]) + __shfl_xor(b4 ? a8[i] : a8[4 + i], 16);
#pragma unroll
  for (int i = 0; i < 2; ++i) a2[i] = (b3 ? a4[2 + i] : a4[i]) + __shfl_xor(b3 ? a4[i] : a4[2 + i], 8);
  float r = (b2 ? a2[1] : a2[0]) + __shfl_xor(b2 ? a2[0] : a2[1], 4);
  r += __shfl_xor(r, 2);
  r += __shfl_xor(r, 1);
  return r;
}

constexpr int kSmallTok = 4;
#ifndef WGKV_GATE_SMALL_WAVES
#define WGKV_GATE_SMALL_WAVES 4
#endif
constexpr int kSmallWaves = WGKV_GATE_SMALL_WAVES;
constexpr int kSplitCols = 16 * kSmallWaves;  // hidden columns per workgroup and pass

template <int K>
__global__ __launch_bounds__(64 * kSmallWaves) void gate_small_kernel(GateArgs a) {
  constexpr int KC = K / 4;                 // float4 chunks of an input row
  constexpr int CPL = (KC + 63) / 64;       // chunks per lane
  __shared__ __attribute__((aligned(16))) float xs[kSmallTok][K];
  __shared__ float s_part[kSmallWaves][kSmallTok];
  if (inactive(a)) return;  // before any arrival is counted
  const int lane = threadIdx.x & 63, wid = threadIdx.x >> 6;
  const int split = blockIdx.x, bh = blockIdx.y;
  const int b = bh / a.H, h = bh - b * a.H;
  const int nt = a.S;  // <= kSmallTok
  const int D = a.D;
  // sigmoid, clamp, threshold and the stores of token s's logit z (before b2)
  auto finish = [&](int s, float z) {
    const float g = score_of(a, z, a.b2[h]);
    if (a.scores) a.scores[(int64_t)b * a.sc_sb + (int64_t)h * a.sc_sh + s] = g;
    if (a.mask) a.mask[(int64_t)b * a.mk_sb + (int64_t)h * a.mk_sh + s] = g > a.threshold ? 1 : 0;
  };

  // The first W1 rows of this wave do not depend on the inputs: their loads
  // are issued first, so their latency overlaps the input normalisation.
  const float* w1h = a.w1 + (int64_t)h * a.inner * K;
  constexpr int JB = CPL > 1 ? 8 : 16;  // W1 rows in flight per wave (two input chunks per lane: 8)
  f32x4_t wrow[JB][CPL];
  auto load_rows = [&](int c0) {
#pragma unroll
    for (int j = 0; j < JB; ++j)
#pragma unroll
      for (int c = 0; c < CPL; ++c) {
        const int kc = lane + c * 64;
        wrow[j][c] = kc < KC ? *(const f32x4_t*)(w1h + (int64_t)(c0 + j) * K + kc * 4) : (f32x4_t){0.f, 0.f, 0.f, 0.f};
      }
  };
  const int c_first = split * kSplitCols + wid * 16;
  if (c_first < a.inner) load_rows(c_first);

  // normalised inputs -> LDS: wave w handles tokens w, w + waves, ...; all its input loads
  // are issued before the first reduction
  for (int s = wid; s < nt; s += kSmallWaves) {
    float v[3][2];
#pragma unroll
    for (int i = 0; i < 3; ++i)
#pragma unroll
      for (int e = 0; e < 2; ++e) {
        const int d = lane + e * 64;
        v[i][e] = (i < a.n_in && d < D) ? load_in(a, i, b, h, s, d) : 0.f;
      }
#pragma unroll
    for (int i = 0; i < 3; ++i) {
      if (i >= a.n_in) break;
      float scale = 1.f;
      if (a.rms) {
        const float var = wave_sum(v[i][0] * v[i][0] + v[i][1] * v[i][1]) / (float)D;
        scale = 1.0f / sqrtf(var + 1e-6f);
      }
#pragma unroll
      for (int e = 0; e < 2; ++e) {
        const int d = lane + e * 64;
        if (d < D) {
          float y = a.rms ? v[i][e] * scale : v[i][e];
          if (a.rms && !a.in_f32) y = round_bf16(y);  // cast back to the input dtype (:128)
          xs[s][i * D + d] = a.rms ? norm_out(a.w_norm[i][d], y, a.prec) : y;
        }
      }
    }
  }
  __syncthreads();

  // this lane's slices of the inputs
  f32x4_t xr[kSmallTok][CPL];
#pragma unroll
  for (int t = 0; t < kSmallTok; ++t)
#pragma unroll
    for (int c = 0; c < CPL; ++c) {
      const int kc = lane + c * 64;
      xr[t][c] = (t < nt && kc < KC) ? *(const f32x4_t*)(&xs[t][kc * 4]) : (f32x4_t){0.f, 0.f, 0.f, 0.f};
    }
  const float* b1h = a.b1 + (int64_t)h * a.inner;
  const float* w2h = a.w2 + (int64_t)h * a.inner;
  float logit[kSmallTok];
#pragma unroll
  for (int t = 0; t < kSmallTok; ++t) logit[t] = 0.f;
  // after the column reduction lane l holds column (l >> 2) & 15 of the
  // wave's 16 (four lanes per column)
  const int my_col = (lane >> 2) & 15;
  for (int c0 = c_first; c0 < a.inner; c0 += kSplitCols * a.nsplit) {
    float dot[kSmallTok][16];
#pragma unroll
    for (int j0 = 0; j0 < 16; j0 += JB) {
      if (c0 != c_first || j0 != 0) load_rows(c0 + j0);
#pragma unroll
      for (int j = 0; j < JB; ++j)
#pragma unroll
        for (int t = 0; t < kSmallTok; ++t) {
          float acc = 0.f;
#pragma unroll
          for (int c = 0; c < CPL; ++c)
#pragma unroll
            for (int e = 0; e < 4; ++e) acc = fmaf(wrow[j][c][e], xr[t][c][e], acc);
          dot[t][j0 + j] = acc;
        }
    }
    const float bias = b1h[c0 + my_col], wo = w2h[c0 + my_col];
#pragma unroll
    for (int t = 0; t < kSmallTok; ++t) {
      if (t >= nt) break;
      const float z = layer_out(reduce16_columns(dot[t], lane), bias, a.prec);
      const float y = wo * activation(z, a.act, a.prec);  // one activation per lane
      logit[t] += (lane & 3) == 0 ? y : 0.f;
    }
  }
  // sum the wave's partial logits over its lanes, then over the waves
#pragma unroll
  for (int t = 0; t < kSmallTok; ++t) {
    if (t >= nt) break;
    const float v = wave_sum(logit[t]);
    if (lane == 0) s_part[wid][t] = v;
  }
  __syncthreads();
  const int t = threadIdx.x;
  if (a.nsplit > 1) {
    // thread 0 publishes this workgroup's partials and counts its arrival
    // (acquire-release at device scope); the last to arrive sums the
    // partials in split order and resets the counter
    if (t != 0) return;
    float* part = a.part + (int64_t)bh * a.nsplit * kSmallTok;
    for (int tt = 0; tt < nt; ++tt) {
      float zz = 0.f;
#pragma unroll
      for (int w = 0; w < kSmallWaves; ++w) zz += s_part[w][tt];
      part[split * kSmallTok + tt] = zz;
    }
    const int prev = __hip_atomic_fetch_add(&a.counter[bh], 1, __ATOMIC_ACQ_REL, __HIP_MEMORY_SCOPE_AGENT);
    if (prev != a.nsplit - 1) return;
    __hip_atomic_store(&a.counter[bh], 0, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    for (int tt = 0; tt < nt; ++tt) {
      float z = 0.f;
      for (int sp = 0; sp < a.nsplit; ++sp) z += part[sp * kSmallTok + tt];
      finish(tt, z);
    }
    return;
  }
  float z = 0.f;
  if (t < nt) {
#pragma unroll
    for (int w = 0; w < kSmallWaves; ++w) z += s_part[w][t];
  }
  if (t < nt) finish(t, z);
}

// ---- bf16 inputs on the bf16 matrix core --------------------------------
// With bf16 inputs each normalised row y = bf16(x * rsqrt(mean(x^2) + eps))
// is exact in bf16, and the first layer is sum_d y_d * (w_norm_d * W1[j][d]).
// The folded fp32 weights f = w_norm * W1 are split once into three bf16
// planes, f = hi + mid + lo, each the round-to-nearest-even bf16 of what the
// previous planes leave (the remainders are exact in fp32, so the planes
// carry all 24 significand bits of f); a product y_d * plane is exact in
// fp32 and the matrix core accumulates the three products in fp32, so the
// layer costs three bf16 MFMAs where fp32 MFMAs would take eight times the
// cycles of one.
// With bf16 parameters W1 is itself bf16 and the norm product is rounded on
// its own, so the packing is one plane holding W1 and the norm weight is
// applied to the inputs.
// Packed layout, bf16: [head][16-column tile][32-input k-step][plane][lane][8]
// -- the B operand of v_mfma_f32_16x16x32_bf16, lane kg*16 + n holding
// column n and inputs 8*kg .. 8*kg+7 -- so one wave load reads 1 KB.
constexpr int kPlanes = 3;

__host__ __device__ constexpr int planes_of(int prec) { return prec ? 1 : kPlanes; }

// With bf16 parameters the activation's input h is a bf16 value and its
// result is rounded to bf16, so act is a function of h's 16 bits.  The pack
// step tabulates bf16(act(h)) -- computed by activation() itself, so the
// table holds exactly what the kernel would compute -- for |h| in
// [2^-16, 16) (20 binades x 128 mantissas x 2 signs), one table for GELU
// and one for SiLU after the weight plane; the kernel reads it from LDS and
// computes the (rare) values outside the range.
constexpr int kActE0 = 127 - 16;  // biased exponent of 2^-16
constexpr int kActBinades = 20;
constexpr int kActTab = 2 * kActBinades * 128;  // entries per activation
// Entry (sign, binade e, 7 mantissa bits m) sits at sign * kActBinades * 128 +
// e * 128 + m, so for a bf16 value with bits b the byte offset within the
// sign's half is 2 * ((b & 0x7fff) - (kActE0 << 7)): in [0, kActBytes)
// exactly for the table's range (in 16-bit arithmetic it wraps past it for
// smaller magnitudes, zero included), plus kActBytes for b < 0.
constexpr int kActBytes = kActBinades * 128 * 2;
constexpr int kActBias2 = (kActE0 << 7) * 2;
typedef unsigned short u16x2_t __attribute__((ext_vector_type(2)));

// Two f32 -> a bf16 pair (round to nearest even) in one v_cvt_pk_bf16_f32.
__device__ __forceinline__ uint32_t cvt_pk_bf16(float lo, float hi) {
  typedef float f32x2_t __attribute__((ext_vector_type(2)));
  typedef __bf16 bf16x2_t __attribute__((ext_vector_type(2)));
  return __builtin_bit_cast(uint32_t, __builtin_convertvector((f32x2_t){lo, hi}, bf16x2_t));
}

__global__ void gate_act_table_kernel(uint16_t* __restrict__ tab) {
  const int i = blockIdx.x * blockDim.x + threadIdx.x;
  if (i >= 2 * kActTab) return;
  const int act = i / kActTab, j = i - act * kActTab;
  const int sgn = j / (kActBinades * 128), r = j - sgn * (kActBinades * 128);
  const uint32_t bits = ((uint32_t)sgn << 31) | ((uint32_t)(kActE0 + r / 128) << 23) | ((uint32_t)(r % 128) << 16);
  tab[i] = (uint16_t)(__float_as_uint(activation(__uint_as_float(bits), act, 1)) >> 16);
}

__global__ void gate_pack_kernel(const float* __restrict__ w1, const float* wn0, const float* wn1,
                                 const float* wn2, int H, int inner, int D, int n_in, int np,
                                 u32x4_t* __restrict__ packed) {
  const int K = n_in * D, NT = inner / 16, KS = K / 32;
  const int64_t total = (int64_t)H * NT * KS * 64;
  for (int64_t id = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; id < total; id += (int64_t)gridDim.x * blockDim.x) {
    const int lane = (int)(id % 64);
    int64_t rest = id / 64;
    const int ks = (int)(rest % KS);
    rest /= KS;
    const int nt = (int)(rest % NT);
    const int h = (int)(rest / NT);
    const int col = nt * 16 + (lane & 15), k0 = ks * 32 + (lane >> 4) * 8;
    uint32_t w[kPlanes][4];
#pragma unroll
    for (int e = 0; e < 8; e += 2) {
      uint16_t pl[kPlanes][2];
#pragma unroll
      for (int u = 0; u < 2; ++u) {
        const int k = k0 + e + u, i = k / D, d = k - i * D;
        const float* wn = np == 1 ? nullptr : i == 0 ? wn0 : i == 1 ? wn1 : wn2;
        const float f = w1[((int64_t)h * inner + col) * K + k] * (wn ? wn[d] : 1.f);
        const uint16_t hi = f32_to_bf16(f);
        const float r1 = f - bf16lo(hi);
        const uint16_t mid = f32_to_bf16(r1);
        const uint16_t lo = f32_to_bf16(r1 - bf16lo(mid));
        pl[0][u] = hi;
        pl[1][u] = mid;
        pl[2][u] = lo;
      }
#pragma unroll
      for (int p = 0; p < kPlanes; ++p) w[p][e / 2] = (uint32_t)pl[p][0] | ((uint32_t)pl[p][1] << 16);
    }
    u32x4_t* dst = packed + (((int64_t)(h * NT + nt) * KS + ks) * np) * 64 + lane;
    for (int p = 0; p < np; ++p) dst[p * 64] = (u32x4_t){w[p][0], w[p][1], w[p][2], w[p][3]};
  }
}

// One workgroup = 64 tokens of one (batch, KV head), as gate_kernel.  The
// inputs are read 16 bytes per lane (a wave load covers 64 / (D/8) rows), the
// row norms reduced over the D/8 lanes of a row, and y goes to LDS as bf16
// (rows padded by 16 bytes: the 16 rows of a fragment read start 16 bytes
// apart modulo 256).  Wave w takes 16-column tiles w, w+4, ... in groups of
// four; per 32-input k-step it reads the four 64-token A fragments from LDS
// and the 4 x 3 packed B fragments of the next k-step from global memory.
// Two waves per SIMD (two workgroups per CU) hide each other's loads and
// GELU epilogues.  fp32 parameters only (PREC 0, three planes); bf16
// parameters run gate_bf16p_kernel.
template <int D, int NIN, int PREC>
__global__ __launch_bounds__(kThreads) __attribute__((amdgpu_waves_per_eu(2, 2))) void gate_bf16_kernel(GateArgs a, const u32x4_t* __restrict__ packed) {
  static_assert(PREC == 0, "three planes: fp32 parameters (bf16 parameters run gate_bf16p_kernel)");
  constexpr int NP = planes_of(PREC);
  constexpr int K = NIN * D;
  constexpr int KS = K / 32;
  constexpr int LDY = K + 8;     // LDS row stride (bf16)
  constexpr int LPR = D / 8;     // lanes per input row
  constexpr int RPL = 64 / LPR;  // rows per wave load
  constexpr int NLD = 16 / RPL;  // wave loads per input for the wave's 16 tokens
  __shared__ __attribute__((aligned(16))) uint16_t ys[kTok * LDY];
  __shared__ float s_part[4][kTok];
  if (inactive(a)) return;
  const int lane = threadIdx.x & 63, wid = threadIdx.x >> 6;
  const int nbh = a.B * a.H;
  const int lid = blockIdx.x + blockIdx.y * gridDim.x;  // XCD-aware order, as gate_kernel
  const int bh = lid % nbh, tile = lid / nbh;
  const int b = bh / a.H, h = bh - b * a.H;
  const int s0 = tile * kTok;

  // ---- normalised inputs -> LDS (bf16) ------------------------------------
  {
    const int c = lane % LPR;
    u32x4_t v[NIN][NLD];
#pragma unroll
    for (int i = 0; i < NIN; ++i)
#pragma unroll
      for (int u = 0; u < NLD; ++u) {
        const int s = min(s0 + wid * 16 + u * RPL + lane / LPR, a.S - 1);  // rows past S are computed and discarded
        const uint16_t* row = (const uint16_t*)a.in[i] + (int64_t)b * a.sb[i] + (int64_t)h * a.sh[i] + (int64_t)s * a.ss[i];
        v[i][u] = *(const u32x4_t*)(row + c * 8);
      }
#pragma unroll
    for (int i = 0; i < NIN; ++i)
#pragma unroll
      for (int u = 0; u < NLD; ++u) {
        u32x4_t y = v[i][u];
        if (a.rms) {
          float f[8];
#pragma unroll
          for (int e = 0; e < 4; ++e) {
            f[2 * e] = bf16lo(y[e]);
            f[2 * e + 1] = bf16hi(y[e]);
          }
          float ss = 0.f;
#pragma unroll
          for (int e = 0; e < 8; ++e) ss = fmaf(f[e], f[e], ss);
          ss += dpp_f32<WGKV_DPP_QP_1032>(ss);
          ss += dpp_f32<WGKV_DPP_QP_2301>(ss);
          ss += dpp_f32<WGKV_DPP_ROW_HALF_MIRROR>(ss);
          if (LPR == 16) ss += dpp_f32<WGKV_DPP_ROW_MIRROR>(ss);
          const float scale = 1.0f / sqrtf(ss / (float)D + 1e-6f);
#pragma unroll
          for (int e = 0; e < 4; ++e) y[e] = pack_bf16x2(f[2 * e] * scale, f[2 * e + 1] * scale);  // cast back to bf16 (:128)
        }
        const int m = wid * 16 + u * RPL + lane / LPR;
        *(u32x4_t*)(&ys[m * LDY + i * D + c * 8]) = y;
      }
  }
  __syncthreads();

  // ---- y @ (w_norm * W1[h])^T: three bf16 MFMAs per k-step and tile pair --
  const int n = lane & 15, kg = lane >> 4;
  const int ntot = a.inner / 16;
  const u32x4_t* ph = packed + (int64_t)h * ntot * KS * NP * 64 + lane;
  const float* b1h = a.b1 + (int64_t)h * a.inner;
  const float* w2h = a.w2 + (int64_t)h * a.inner;
  float logit[4][4];
#pragma unroll
  for (int mt = 0; mt < 4; ++mt)
#pragma unroll
    for (int i = 0; i < 4; ++i) logit[mt][i] = 0.f;
  for (int t0 = wid; t0 < ntot; t0 += 16) {
    int tj[4];
#pragma unroll
    for (int j = 0; j < 4; ++j) tj[j] = t0 + 4 * j < ntot ? t0 + 4 * j : t0;  // out-of-range tiles recompute t0, skipped below
    f32x4_t c[4][4];
#pragma unroll
    for (int mt = 0; mt < 4; ++mt)
#pragma unroll
      for (int j = 0; j < 4; ++j) c[mt][j] = (f32x4_t){0.f, 0.f, 0.f, 0.f};
    {
    u32x4_t bw[4][NP];
#pragma unroll
    for (int j = 0; j < 4; ++j)
#pragma unroll
      for (int p = 0; p < NP; ++p) bw[j][p] = ph[((int64_t)tj[j] * KS * NP + p) * 64];
#pragma unroll 2
    for (int ks = 0; ks < KS; ++ks) {
      u32x4_t bn[4][NP];
      if (ks + 1 < KS)
#pragma unroll
        for (int j = 0; j < 4; ++j)
#pragma unroll
          for (int p = 0; p < NP; ++p) bn[j][p] = ph[(((int64_t)tj[j] * KS + ks + 1) * NP + p) * 64];
      bf16x8_t ax[4];
#pragma unroll
      for (int mt = 0; mt < 4; ++mt)
        ax[mt] = __builtin_bit_cast(bf16x8_t, *(const u32x4_t*)(&ys[(mt * 16 + n) * LDY + ks * 32 + kg * 8]));
#pragma unroll
      for (int p = NP - 1; p >= 0; --p)  // smallest plane first
#pragma unroll
        for (int mt = 0; mt < 4; ++mt)
#pragma unroll
          for (int j = 0; j < 4; ++j)
            c[mt][j] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(ax[mt], __builtin_bit_cast(bf16x8_t, bw[j][p]), c[mt][j], 0, 0, 0);
      if (ks + 1 < KS)
#pragma unroll
        for (int j = 0; j < 4; ++j)
#pragma unroll
          for (int p = 0; p < NP; ++p) bw[j][p] = bn[j][p];
    }
    }
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      if (t0 + 4 * j >= ntot) break;
      const int col = tj[j] * 16 + n;
      const float bias = b1h[col], wo = w2h[col];
#pragma unroll
      for (int mt = 0; mt < 4; ++mt)
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          const float z = layer_out(c[mt][j][i], bias, PREC);
          logit[mt][i] = fmaf(wo, activation(z, a.act, PREC), logit[mt][i]);
        }
    }
  }
  finish_tile(a, logit, s_part, lane, wid, b, h, s0);
}

// ---- one weight plane (bf16 parameters) -----------------------------------
// The tile, inputs, MFMA arithmetic and per-lane summation order of
// gate_bf16_kernel with one plane (wave w: 16-column tiles w + 4m in groups
// of four), with an epilogue that works on pairs of values: the two rows
// i, i+1 of a column are rounded to bf16 by one v_cvt_pk_bf16_f32, their
// table offsets computed with packed 16-bit arithmetic, and all 64 table
// reads of a group issued before any result is used, so the LDS latency is
// paid once per group, not once per value (the reads themselves stay at
// random addresses: bank conflicts are most of the kernel's LDS time).  One
// packed maximum over the group's offsets tells whether any value lies
// outside the table; only then are those values computed by activation().
// The weight fragments are requested PQ k-steps ahead, across group
// boundaries, and the first group's, with the activation table and the norm
// weights, before the inputs.
template <int D, int NIN>
struct TileInputs {
  static constexpr int LPR = D / 8;     // lanes per input row
  static constexpr int RPL = 64 / LPR;  // rows per wave load
  static constexpr int NLD = 16 / RPL;  // wave loads per input for the wave's 16 tokens
  u32x4_t v[NIN][NLD];
  f32x4_t wn[NIN][2];
};

template <int D, int NIN>
__device__ __forceinline__ void load_tile_inputs(const GateArgs& a, int b, int h, int s0, int lane, int wid,
                                                 TileInputs<D, NIN>& t) {
  using T = TileInputs<D, NIN>;
  const int c = lane % T::LPR;
  if (a.rms)
#pragma unroll
    for (int i = 0; i < NIN; ++i) {
      t.wn[i][0] = *(const f32x4_t*)(a.w_norm[i] + c * 8);
      t.wn[i][1] = *(const f32x4_t*)(a.w_norm[i] + c * 8 + 4);
    }
#pragma unroll
  for (int i = 0; i < NIN; ++i)
#pragma unroll
    for (int u = 0; u < T::NLD; ++u) {
      const int s = min(s0 + wid * 16 + u * T::RPL + lane / T::LPR, a.S - 1);  // rows past S are computed and discarded
      const uint16_t* row = (const uint16_t*)a.in[i] + (int64_t)b * a.sb[i] + (int64_t)h * a.sh[i] + (int64_t)s * a.ss[i];
      t.v[i][u] = *(const u32x4_t*)(row + c * 8);
    }
}

// y = bf16(x * rsqrt(mean(x^2) + 1e-6)) (:128), times the bf16 norm weight
// rounded to bf16, as gate_bf16_kernel with bf16 parameters.
template <int D, int NIN, int LDY>
__device__ __forceinline__ void store_tile_inputs(const GateArgs& a, int lane, int wid, const TileInputs<D, NIN>& t,
                                                  uint16_t* ys) {
  using T = TileInputs<D, NIN>;
  const int c = lane % T::LPR;
#pragma unroll
  for (int i = 0; i < NIN; ++i)
#pragma unroll
    for (int u = 0; u < T::NLD; ++u) {
      u32x4_t y = t.v[i][u];
      if (a.rms) {
        float f[8];
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          f[2 * e] = bf16lo(y[e]);
          f[2 * e + 1] = bf16hi(y[e]);
        }
        float ss = 0.f;
#pragma unroll
        for (int e = 0; e < 8; ++e) ss = fmaf(f[e], f[e], ss);
        ss += dpp_f32<WGKV_DPP_QP_1032>(ss);
        ss += dpp_f32<WGKV_DPP_QP_2301>(ss);
        ss += dpp_f32<WGKV_DPP_ROW_HALF_MIRROR>(ss);
        if (T::LPR == 16) ss += dpp_f32<WGKV_DPP_ROW_MIRROR>(ss);
        const float scale = 1.0f / sqrtf(ss / (float)D + 1e-6f);
#pragma unroll
        for (int e = 0; e < 4; ++e) y[e] = pack_bf16x2(f[2 * e] * scale, f[2 * e + 1] * scale);
        const float wv[8] = {t.wn[i][0][0], t.wn[i][0][1], t.wn[i][0][2], t.wn[i][0][3],
                             t.wn[i][1][0], t.wn[i][1][1], t.wn[i][1][2], t.wn[i][1][3]};
#pragma unroll
        for (int e = 0; e < 4; ++e) y[e] = pack_bf16x2(wv[2 * e] * bf16lo(y[e]), wv[2 * e + 1] * bf16hi(y[e]));
      }
      const int m = wid * 16 + u * T::RPL + lane / T::LPR;
      *(u32x4_t*)(&ys[m * LDY + i * D + c * 8]) = y;
    }
}

template <int D, int NIN, int PREC>
__global__ __launch_bounds__(kThreads) __attribute__((amdgpu_waves_per_eu(2, 2))) void gate_bf16p_kernel(GateArgs a, const u32x4_t* __restrict__ packed) {
  static_assert(PREC == 1 || PREC == 2, "one plane: bf16 parameters");
  constexpr int K = NIN * D;
  constexpr int KS = K / 32;
  constexpr int LDY = K + 8;
  constexpr int NTAB = kActTab / 8;                      // 16-byte slices of the table
  constexpr int TPT = (NTAB + kThreads - 1) / kThreads;  // per thread
  __shared__ __attribute__((aligned(16))) uint16_t ys[kTok * LDY];
  __shared__ float s_part[4][kTok];
  __shared__ __attribute__((aligned(16))) uint16_t s_act[kActTab];
  if (inactive(a)) return;
  const int lane = threadIdx.x & 63, wid = threadIdx.x >> 6;
  const int nbh = a.B * a.H;
  const int lid = blockIdx.x + blockIdx.y * gridDim.x;  // XCD-aware order, as gate_kernel
  const int bh = lid % nbh, tile = lid / nbh;
  const int b = bh / a.H, h = bh - b * a.H;
  const int s0 = tile * kTok;
  const int n = lane & 15, kg = lane >> 4;
  const int ntot = a.inner / 16;
  const u32x4_t* ph = packed + (int64_t)h * ntot * KS * 64 + lane;
  const float* b1h = a.b1 + (int64_t)h * a.inner;
  const float* w2h = a.w2 + (int64_t)h * a.inner;
  constexpr int TG = 4;                    // tiles per group
  constexpr int PQ = KS % 2 == 0 ? 2 : 1;  // k-steps of weight fragments in flight
  const int nw = (ntot - wid + 3) >> 2;    // this wave's tiles: wid + 4m, m < nw
  const int ng = (nw + TG - 1) / TG;
  // tile j of group g; past the wave's last tile, tile wid again (computed, never used)
  auto tile_of = [&](int g, int j) { const int m = TG * g + j; return m < nw ? wid + 4 * m : wid; };

  // ---- requests that do not depend on the inputs --------------------------
  u32x4_t tab_r[TPT];
  {
    const u32x4_t* tab = packed + (int64_t)a.H * ntot * KS * 64 + a.act * NTAB;  // this activation's table
#pragma unroll
    for (int r = 0; r < TPT; ++r) {
      const int i = threadIdx.x + r * kThreads;
      tab_r[r] = tab[i < NTAB ? i : 0];
    }
  }
  u32x4_t bq[PQ][TG];  // k-step ks of a group in slot ks % PQ
#pragma unroll
  for (int ks = 0; ks < PQ; ++ks)
#pragma unroll
    for (int jj = 0; jj < TG; ++jj) bq[ks][jj] = ph[((int64_t)tile_of(0, jj) * KS + ks) * 64];

  // ---- normalised inputs -> LDS -------------------------------------------
  {
    TileInputs<D, NIN> in;
    load_tile_inputs<D, NIN>(a, b, h, s0, lane, wid, in);
#pragma unroll
    for (int r = 0; r < TPT; ++r) {
      const int i = threadIdx.x + r * kThreads;
      if (i < NTAB) ((u32x4_t*)s_act)[i] = tab_r[r];
    }
    store_tile_inputs<D, NIN, LDY>(a, lane, wid, in, ys);
  }
  __syncthreads();

  float logit[4][4];
#pragma unroll
  for (int mt = 0; mt < 4; ++mt)
#pragma unroll
    for (int i = 0; i < 4; ++i) logit[mt][i] = 0.f;
  for (int g = 0; g < ng; ++g) {
    int tn[TG], tx[TG];
    float bo[TG], wo[TG];
#pragma unroll
    for (int jj = 0; jj < TG; ++jj) {
      tn[jj] = tile_of(g, jj);
      tx[jj] = tile_of(g + 1, jj);
      const int col = tn[jj] * 16 + n;
      bo[jj] = b1h[col];
      wo[jj] = w2h[col];
    }
    f32x4_t c[4][TG];
#pragma unroll
    for (int mt = 0; mt < 4; ++mt)
#pragma unroll
      for (int jj = 0; jj < TG; ++jj) c[mt][jj] = (f32x4_t){0.f, 0.f, 0.f, 0.f};
    // the A fragments are the same for every group: an opaque base keeps the
    // compiler from hoisting all of them out of the group loop (128 registers)
    int abase = n * LDY + kg * 8;
    asm volatile("" : "+v"(abase));
#pragma unroll
    for (int ks = 0; ks < KS; ++ks) {
      bf16x8_t ax[4];
#pragma unroll
      for (int mt = 0; mt < 4; ++mt)
        ax[mt] = __builtin_bit_cast(bf16x8_t, *(const u32x4_t*)(&ys[mt * 16 * LDY + abase + ks * 32]));
      // the slot's next k-step: this group's ks + PQ, else the next group's
      const int slot = ks % PQ;
      u32x4_t bcur[TG];
#pragma unroll
      for (int jj = 0; jj < TG; ++jj) {
        bcur[jj] = bq[slot][jj];
        bq[slot][jj] = ks + PQ < KS ? ph[((int64_t)tn[jj] * KS + ks + PQ) * 64] : ph[((int64_t)tx[jj] * KS + ks + PQ - KS) * 64];
      }
#pragma unroll
      for (int mt = 0; mt < 4; ++mt)
#pragma unroll
        for (int jj = 0; jj < TG; ++jj)
          c[mt][jj] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(ax[mt], __builtin_bit_cast(bf16x8_t, bcur[jj]), c[mt][jj], 0, 0, 0);
    }
    // the group's 64 values of this lane as 32 bf16 pairs (rows i, i+1 of the
    // lane's column in tile jj): the layer outputs z and their table entries;
    // dmax = the largest table offset (offsets >= kActBytes lie outside)
    uint32_t zz[32], tvp[32];
    u16x2_t dmax = {0, 0};
#pragma unroll
    for (int p = 0; p < 32; ++p) {
      const int mt = p >> 3, jj = (p >> 1) & 3, i = (p & 1) * 2;
      uint32_t z2;
      if (PREC == 1) {
        const uint32_t r = cvt_pk_bf16(c[mt][jj][i], c[mt][jj][i + 1]);
        z2 = cvt_pk_bf16(bf16lo(r) + bo[jj], bf16hi(r) + bo[jj]);
      } else {
        z2 = cvt_pk_bf16(c[mt][jj][i] + bo[jj], c[mt][jj][i + 1] + bo[jj]);
      }
      zz[p] = z2;
      // byte offset of bf16(act(z)) in the table, per 16-bit half
      const u16x2_t zv = __builtin_bit_cast(u16x2_t, z2);
      const u16x2_t d2 = (u16x2_t)(zv << 1) - (u16x2_t)kActBias2;
      dmax = __builtin_elementwise_max(dmax, d2);
      const u16x2_t off = (u16x2_t)(zv >> 15) * (u16x2_t)kActBytes + __builtin_elementwise_min(d2, (u16x2_t)(kActBytes - 2));
      const char* tb = (const char*)s_act;
      u16x2_t t;
      t.x = *(const uint16_t*)(tb + off.x);
      t.y = *(const uint16_t*)(tb + off.y);
      tvp[p] = __builtin_bit_cast(uint32_t, t);
    }
    if (max(dmax.x, dmax.y) >= kActBytes) {  // rare: some value lies outside the table
#pragma unroll
      for (int p = 0; p < 32; ++p) {
        const u16x2_t zv = __builtin_bit_cast(u16x2_t, zz[p]);
        const u16x2_t d2 = (u16x2_t)(zv << 1) - (u16x2_t)kActBias2;
        if (d2.x >= kActBytes) tvp[p] = (tvp[p] & 0xffff0000u) | (__float_as_uint(activation(bf16lo(zz[p]), a.act, PREC)) >> 16);
        if (d2.y >= kActBytes) tvp[p] = (tvp[p] & 0xffffu) | (__float_as_uint(activation(bf16hi(zz[p]), a.act, PREC)) & 0xffff0000u);
      }
    }
    // w2 multiply-adds in the lane's column order (tiles 4g, 4g+1, ...)
#pragma unroll
    for (int jj = 0; jj < TG; ++jj) {
      if (TG * g + jj >= nw) break;
#pragma unroll
      for (int mt = 0; mt < 4; ++mt)
#pragma unroll
        for (int i = 0; i < 4; i += 2) {
          const uint32_t t = tvp[mt * 8 + jj * 2 + i / 2];
          logit[mt][i] = fmaf(wo[jj], bf16lo(t), logit[mt][i]);
          logit[mt][i + 1] = fmaf(wo[jj], bf16hi(t), logit[mt][i + 1]);
        }
    }
  }
  finish_tile(a, logit, s_part, lane, wid, b, h, s0);
}

template <int K>
void launch_gate(const GateArgs& a, hipStream_t st) {
  if (a.S <= kSmallTok) {
    hipLaunchKernelGGL(gate_small_kernel<K>, dim3(a.nsplit, a.B * a.H), dim3(64 * kSmallWaves), 0, st, a);
  } else {
    hipLaunchKernelGGL(gate_kernel<K>, dim3((a.S + kTok - 1) / kTok, a.B * a.H), dim3(kThreads), 0, st, a);
  }
}

}  // namespace

namespace {
int64_t align256(int64_t x) { return (x + 255) / 256 * 256; }

// Round-to-nearest-even f32 -> bf16 -> f32 on the host (finite values).
float host_round_bf16(float f) {
  uint32_t u;
  memcpy(&u, &f, 4);
  u += 0x7fffu + ((u >> 16) & 1u);
  u &= 0xffff0000u;
  memcpy(&f, &u, 4);
  return f;
}
}  // namespace

extern "C" int64_t wgkv_gate_workspace_bytes(int32_t batch, int32_t num_kv_heads, int32_t inner) {
  const int64_t nsplit = (inner + kSplitCols - 1) / kSplitCols;
  const int64_t bh = (int64_t)batch * num_kv_heads;
  return align256(bh * 4) + align256(bh * nsplit * kSmallTok * 4);
}

extern "C" int wgkv_gate_scores(
    const void* pre_key, int64_t pk_sb, int64_t pk_sh, int64_t pk_ss,
    const void* post_key, int64_t k_sb, int64_t k_sh, int64_t k_ss,
    const void* value, int64_t v_sb, int64_t v_sh, int64_t v_ss,
    int32_t in_dtype, int32_t inputs_mask,
    const float* w_pre, const float* w_post, const float* w_v,
    const float* w1, const float* b1, const float* w2, const float* b2,
    int32_t batch, int32_t num_kv_heads, int32_t seq_len, int32_t head_dim, int32_t inner,
    int32_t act, int32_t rms, int32_t precision, float clamp_min, float threshold,
    float* scores, int64_t sc_sb, int64_t sc_sh,
    uint8_t* mask, int64_t mk_sb, int64_t mk_sh,
    const void* w1_packed,
    const int32_t* active_flag, int32_t active_value,
    void* workspace, int64_t workspace_bytes,
    void* stream) {
  if (batch <= 0 || num_kv_heads <= 0 || seq_len <= 0) return WGKV_ERR_ARG;
  if (!w1 || !b1 || !w2 || !b2 || (!scores && !mask)) return WGKV_ERR_ARG;
  if (head_dim != 64 && head_dim != 128) return WGKV_ERR_UNSUPPORTED;
  if (inner <= 0 || inner % 16) return WGKV_ERR_UNSUPPORTED;  // 16-column tiles
  if (in_dtype != 0 && in_dtype != 1) return WGKV_ERR_UNSUPPORTED;
  if (precision < 0 || precision > 2) return WGKV_ERR_ARG;
  if (precision && in_dtype != 0) return WGKV_ERR_UNSUPPORTED;  // bf16 parameters take bf16 inputs
  GateArgs a = {};
  const void* srcs[3] = {pre_key, post_key, value};
  const float* wn[3] = {w_pre, w_post, w_v};
  const int64_t strides[3][3] = {{pk_sb, pk_sh, pk_ss}, {k_sb, k_sh, k_ss}, {v_sb, v_sh, v_ss}};
  int n_in = 0;
  for (int i = 0; i < 3; ++i) {
    if (!(inputs_mask >> i & 1)) continue;
    if (!srcs[i] || (rms && !wn[i])) return WGKV_ERR_ARG;
    a.in[n_in] = srcs[i];
    a.sb[n_in] = strides[i][0];
    a.sh[n_in] = strides[i][1];
    a.ss[n_in] = strides[i][2];
    a.w_norm[n_in] = wn[i];
    ++n_in;
  }
  if (n_in == 0) return WGKV_ERR_ARG;
  a.n_in = n_in;
  a.in_f32 = in_dtype == 1;
  a.rms = rms;
  a.w1 = w1;
  a.b1 = b1;
  a.w2 = w2;
  a.b2 = b2;
  a.B = batch;
  a.H = num_kv_heads;
  a.S = seq_len;
  a.D = head_dim;
  a.inner = inner;
  a.act = act;
  a.prec = precision;
  // bf16 scores are compared with (and clamped to) the bf16 value of the
  // Python float, as a bf16 tensor compared with a scalar is
  a.clamp_min = precision ? host_round_bf16(clamp_min) : clamp_min;
  a.threshold = precision ? host_round_bf16(threshold) : threshold;
  a.scores = scores;
  a.sc_sb = sc_sb;
  a.sc_sh = sc_sh;
  a.mask = mask;
  a.mk_sb = mk_sb;
  a.mk_sh = mk_sh;
  a.active = active_flag;
  a.active_value = active_value;
  a.nsplit = 1;
  if (workspace && seq_len <= kSmallTok) {
    const int nsplit = (inner + kSplitCols - 1) / kSplitCols;
    if (workspace_bytes < wgkv_gate_workspace_bytes(batch, num_kv_heads, inner)) return WGKV_ERR_ARG;
    a.nsplit = nsplit;
    a.counter = (int32_t*)workspace;
    a.part = (float*)((char*)workspace + align256((int64_t)batch * num_kv_heads * 4));
  }
  if (((uintptr_t)w1 & 15) != 0) return WGKV_ERR_UNSUPPORTED;
  const int K = n_in * head_dim;
  hipStream_t st = (hipStream_t)stream;
  if (w1_packed && in_dtype == 0 && seq_len > kSmallTok) {
    // the packed path reads 16-byte input slices
    bool aligned = ((uintptr_t)w1_packed & 15) == 0;
    for (int i = 0; i < n_in; ++i) {
      aligned = aligned && ((uintptr_t)a.in[i] & 15) == 0 && ((a.sb[i] | a.sh[i] | a.ss[i]) & 7) == 0;
      if (precision && rms) aligned = aligned && ((uintptr_t)a.w_norm[i] & 15) == 0;  // 16-byte norm-weight loads
    }
    if (aligned) {
      const u32x4_t* pk = (const u32x4_t*)w1_packed;
      const dim3 grid((seq_len + kTok - 1) / kTok, batch * num_kv_heads);
#define WGKV_GATE_BF16(DD, NN)                                                                              \
  do {                                                                                                      \
    if (precision == 0) hipLaunchKernelGGL((gate_bf16_kernel<DD, NN, 0>), grid, dim3(kThreads), 0, st, a, pk); \
    else if (precision == 1) hipLaunchKernelGGL((gate_bf16p_kernel<DD, NN, 1>), grid, dim3(kThreads), 0, st, a, pk); \
    else hipLaunchKernelGGL((gate_bf16p_kernel<DD, NN, 2>), grid, dim3(kThreads), 0, st, a, pk);             \
  } while (0)
      if (head_dim == 128) {
        if (n_in == 1) WGKV_GATE_BF16(128, 1);
        else if (n_in == 2) WGKV_GATE_BF16(128, 2);
        else WGKV_GATE_BF16(128, 3);
      } else {
        if (n_in == 1) WGKV_GATE_BF16(64, 1);
        else if (n_in == 2) WGKV_GATE_BF16(64, 2);
        else WGKV_GATE_BF16(64, 3);
      }
#undef WGKV_GATE_BF16
      return hipGetLastError() == hipSuccess ? WGKV_OK : WGKV_ERR_HIP;
    }
  }
  switch (K) {
    case 64: launch_gate<64>(a, st); break;
    case 128: launch_gate<128>(a, st); break;
    case 192: launch_gate<192>(a, st); break;
    case 256: launch_gate<256>(a, st); break;
    case 384: launch_gate<384>(a, st); break;
    default: return WGKV_ERR_UNSUPPORTED;
  }
  return hipGetLastError() == hipSuccess ? WGKV_OK : WGKV_ERR_HIP;
}

extern "C" int64_t wgkv_gate_packed_bytes(int32_t num_kv_heads, int32_t inner, int32_t in_features,
                                          int32_t precision) {
  if (num_kv_heads <= 0 || inner <= 0 || inner % 16 || in_features <= 0 || in_features % 32) return -1;
  if (precision < 0 || precision > 2) return -1;
  return (int64_t)num_kv_heads * inner * in_features * planes_of(precision) * 2 + (precision ? 2 * kActTab * 2 : 0);
}

extern "C" int wgkv_gate_pack_weights(
    const float* w_pre, const float* w_post, const float* w_v, int32_t inputs_mask, int32_t rms,
    const float* w1, int32_t num_kv_heads, int32_t head_dim, int32_t inner, int32_t precision,
    void* packed, int64_t packed_bytes, void* stream) {
  if (!w1 || !packed || num_kv_heads <= 0) return WGKV_ERR_ARG;
  if (precision < 0 || precision > 2) return WGKV_ERR_ARG;
  if (head_dim != 64 && head_dim != 128) return WGKV_ERR_UNSUPPORTED;
  if (inner <= 0 || inner % 16) return WGKV_ERR_UNSUPPORTED;
  const float* wn_all[3] = {w_pre, w_post, w_v};
  const float* wn[3] = {nullptr, nullptr, nullptr};
  int n_in = 0;
  for (int i = 0; i < 3; ++i) {
    if (!(inputs_mask >> i & 1)) continue;
    if (rms && !wn_all[i]) return WGKV_ERR_ARG;
    wn[n_in++] = rms ? wn_all[i] : nullptr;
  }
  if (n_in == 0) return WGKV_ERR_ARG;
  if (packed_bytes < wgkv_gate_packed_bytes(num_kv_heads, inner, n_in * head_dim, precision)) return WGKV_ERR_ARG;
  if (((uintptr_t)packed & 15) != 0) return WGKV_ERR_UNSUPPORTED;
  const int64_t total = (int64_t)num_kv_heads * (inner / 16) * (n_in * head_dim / 32) * 64;
  const int blocks = (int)((total + 255) / 256 < 4096 ? (total + 255) / 256 : 4096);
  hipLaunchKernelGGL(gate_pack_kernel, dim3(blocks), dim3(256), 0, (hipStream_t)stream, w1, wn[0], wn[1], wn[2],
                     num_kv_heads, inner, head_dim, n_in, planes_of(precision), (u32x4_t*)packed);
  if (precision) {  // activation tables after the weight plane
    uint16_t* tab = (uint16_t*)((char*)packed + (int64_t)num_kv_heads * inner * n_in * head_dim * 2);
    hipLaunchKernelGGL(gate_act_table_kernel, dim3((2 * kActTab + 255) / 256), dim3(256), 0, (hipStream_t)stream, tab);
  }
  return hipGetLastError() == hipSuccess ? WGKV_OK : WGKV_ERR_HIP;
}
