// Write-gate MLP scores and admission flags (gfx950, fp32).
//
// Replaces GatingPredictor.forward (src/modeling_layers.py:170-205) with the
// RMS norms of GatingRMSNorm (:113-131) and the threshold of :1465:
//   x  = concat(rms(pre_k)*w_pre, rms(post_k)*w_post[, rms(v)*w_v])   (n_in*D)
//   h  = act(W1[h] x + b1[h])                                        (inner)
//   g  = sigmoid(w2[h] . h + b2[h]);  conv path: g = max(g, clamp_min)
//   mask = g > threshold
// One workgroup = 64 tokens of one (batch, KV head), heads dealt across the
// XCDs so each head's W1 stays in one L2.  The normalised inputs
// go to LDS (fp32, rows padded for conflict-free 16-byte reads); the hidden
// columns are dealt round-robin to the 4 waves in 16-column tiles, so W1[h]
// is read once per workgroup; x @ W1^T runs on v_mfma_f32_16x16x4f32 with
// each lane feeding four consecutive k from one 16-byte load; the epilogue
// applies bias, activation and w2 and reduces over columns in registers.
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
  float clamp_min, threshold;
  float* scores;
  int64_t sc_sb, sc_sh;
  uint8_t* mask;
  int64_t mk_sb, mk_sh;
};

__device__ __forceinline__ float load_in(const GateArgs& a, int i, int b, int h, int s, int d) {
  const int64_t off = (int64_t)b * a.sb[i] + (int64_t)h * a.sh[i] + (int64_t)s * a.ss[i] + d;
  if (a.in_f32) return ((const float*)a.in[i])[off];
  return __uint_as_float((uint32_t)((const uint16_t*)a.in[i])[off] << 16);
}

__device__ __forceinline__ float round_bf16(float x) {
  return __uint_as_float((uint32_t)f32_to_bf16(x) << 16);
}

__device__ __forceinline__ float gelu_erf(float z) { return 0.5f * z * (1.0f + erff(z * 0.70710678118654752f)); }
__device__ __forceinline__ float silu(float z) { return z / (1.0f + expf(-z)); }

template <int K>  // n_in * D
__global__ __launch_bounds__(kThreads) void gate_kernel(GateArgs a) {
  constexpr int LDX = K + 4;  // padded row (floats)
  __shared__ float xs[kTok * LDX];
  __shared__ float s_part[4][kTok];
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
            xs[m * LDX + i * D + d] = a.rms ? a.w_norm[i][d] * y : y;
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
          const float z = c[mt][j][i] + bias;
          logit[mt][i] = fmaf(wo, a.act ? silu(z) : gelu_erf(z), logit[mt][i]);
        }
    }
  }
  // sum over the 16 columns held by the lanes of each row, then over waves
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
      const float z = ((s_part[0][m] + s_part[1][m]) + (s_part[2][m] + s_part[3][m])) + a.b2[h];
      float g = 1.0f / (1.0f + expf(-z));
      if (a.clamp_min > 0.f) g = fmaxf(g, a.clamp_min);
      if (a.scores) a.scores[(int64_t)b * a.sc_sb + (int64_t)h * a.sc_sh + s] = g;
      if (a.mask) a.mask[(int64_t)b * a.mk_sb + (int64_t)h * a.mk_sh + s] = g > a.threshold ? 1 : 0;
    }
  }
}

// Few tokens (decode steps): one workgroup per (batch, KV head) and group of
// up to kSmallTok tokens.  The MFMA tile above would compute 64 token rows to
// use one and stream W1[h] through a single dependent chain; here the lanes
// of a wave split the K dimension, so each W1 row is read with one coalesced
// load per wave, and each of the 16 waves takes 16 hidden columns at a time
// (interleaved in 16-column tiles).  Per column the lane partials are
// summed over the wave; lane i < 16 then applies bias, activation and w2 for
// column i.  Column order is fixed, so results are deterministic.
constexpr int kSmallTok = 4;
constexpr int kSmallWaves = 16;  // 16 waves: W1 rows of 16 x 16 columns in flight at once

template <int K>
__global__ __launch_bounds__(64 * kSmallWaves) void gate_small_kernel(GateArgs a) {
  constexpr int KC = K / 4;                 // float4 chunks of an input row
  constexpr int CPL = (KC + 63) / 64;       // chunks per lane
  __shared__ __attribute__((aligned(16))) float xs[kSmallTok][K];
  __shared__ float s_part[kSmallWaves][kSmallTok];
  const int lane = threadIdx.x & 63, wid = threadIdx.x >> 6;
  const int bh = blockIdx.y;
  const int b = bh / a.H, h = bh - b * a.H;
  const int s0 = blockIdx.x * kSmallTok;
  const int nt = min(kSmallTok, a.S - s0);
  const int D = a.D;

  // normalised inputs -> LDS: wave w handles token w
  if (wid < nt) {
    const int s = s0 + wid;
    for (int i = 0; i < a.n_in; ++i) {
      float v[2];
      float sq = 0.f;
#pragma unroll
      for (int e = 0; e < 2; ++e) {
        const int d = lane + e * 64;
        v[e] = d < D ? load_in(a, i, b, h, s, d) : 0.f;
        sq += v[e] * v[e];
      }
      float scale = 1.f;
      if (a.rms) {
        const float var = wave_sum(sq) / (float)D;
        scale = 1.0f / sqrtf(var + 1e-6f);
      }
#pragma unroll
      for (int e = 0; e < 2; ++e) {
        const int d = lane + e * 64;
        if (d < D) {
          float y = a.rms ? v[e] * scale : v[e];
          if (a.rms && !a.in_f32) y = round_bf16(y);  // cast back to the input dtype (:128)
          xs[wid][i * D + d] = a.rms ? a.w_norm[i][d] * y : y;
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
  const float* w1h = a.w1 + (int64_t)h * a.inner * K;
  const float* b1h = a.b1 + (int64_t)h * a.inner;
  const float* w2h = a.w2 + (int64_t)h * a.inner;
  float logit[kSmallTok];
#pragma unroll
  for (int t = 0; t < kSmallTok; ++t) logit[t] = 0.f;
  // columns in groups of JB: with two input chunks per lane, 8 W1 rows in
  // flight keep the registers within the 1024-thread budget
  constexpr int JB = CPL > 1 ? 8 : 16;
  for (int c0 = wid * 16; c0 < a.inner; c0 += 16 * kSmallWaves) {
#pragma unroll
    for (int j0 = 0; j0 < 16; j0 += JB) {
      float dot[kSmallTok][JB];
#pragma unroll
      for (int j = 0; j < JB; ++j) {
        f32x4_t w[CPL];
#pragma unroll
        for (int c = 0; c < CPL; ++c) {
          const int kc = lane + c * 64;
          w[c] = kc < KC ? *(const f32x4_t*)(w1h + (int64_t)(c0 + j0 + j) * K + kc * 4)
                         : (f32x4_t){0.f, 0.f, 0.f, 0.f};
        }
#pragma unroll
        for (int t = 0; t < kSmallTok; ++t) {
          float acc = 0.f;
#pragma unroll
          for (int c = 0; c < CPL; ++c)
#pragma unroll
            for (int e = 0; e < 4; ++e) acc = fmaf(w[c][e], xr[t][c][e], acc);
          dot[t][j] = acc;
        }
      }
#pragma unroll
      for (int t = 0; t < kSmallTok; ++t) {
        if (t >= nt) break;
#pragma unroll
        for (int j = 0; j < JB; ++j) {
          const float z = wave_sum(dot[t][j]) + b1h[c0 + j0 + j];
          if (lane == j0 + j) logit[t] = fmaf(w2h[c0 + j0 + j], a.act ? silu(z) : gelu_erf(z), logit[t]);
        }
      }
    }
  }
  // lanes 0..15 of each wave hold partial logits; sum them, then the waves
#pragma unroll
  for (int t = 0; t < kSmallTok; ++t) {
    const float v = row_sum16(lane < 16 ? logit[t] : 0.f);
    if (lane == 0) s_part[wid][t] = v;
  }
  __syncthreads();
  if (threadIdx.x < nt) {
    const int t = threadIdx.x;
    const int s = s0 + t;
    float z = 0.f;
#pragma unroll
    for (int w = 0; w < kSmallWaves; ++w) z += s_part[w][t];
    z += a.b2[h];
    float g = 1.0f / (1.0f + expf(-z));
    if (a.clamp_min > 0.f) g = fmaxf(g, a.clamp_min);
    if (a.scores) a.scores[(int64_t)b * a.sc_sb + (int64_t)h * a.sc_sh + s] = g;
    if (a.mask) a.mask[(int64_t)b * a.mk_sb + (int64_t)h * a.mk_sh + s] = g > a.threshold ? 1 : 0;
  }
}

template <int K>
void launch_gate(const GateArgs& a, hipStream_t st) {
  if (a.S <= kSmallTok) {
    hipLaunchKernelGGL(gate_small_kernel<K>, dim3(1, a.B * a.H), dim3(64 * kSmallWaves), 0, st, a);
  } else {
    hipLaunchKernelGGL(gate_kernel<K>, dim3((a.S + kTok - 1) / kTok, a.B * a.H), dim3(kThreads), 0, st, a);
  }
}

}  // namespace

extern "C" int wgkv_gate_scores(
    const void* pre_key, int64_t pk_sb, int64_t pk_sh, int64_t pk_ss,
    const void* post_key, int64_t k_sb, int64_t k_sh, int64_t k_ss,
    const void* value, int64_t v_sb, int64_t v_sh, int64_t v_ss,
    int32_t in_dtype, int32_t inputs_mask,
    const float* w_pre, const float* w_post, const float* w_v,
    const float* w1, const float* b1, const float* w2, const float* b2,
    int32_t batch, int32_t num_kv_heads, int32_t seq_len, int32_t head_dim, int32_t inner,
    int32_t act, int32_t rms, float clamp_min, float threshold,
    float* scores, int64_t sc_sb, int64_t sc_sh,
    uint8_t* mask, int64_t mk_sb, int64_t mk_sh,
    void* stream) {
  if (batch <= 0 || num_kv_heads <= 0 || seq_len <= 0) return WGKV_ERR_ARG;
  if (!w1 || !b1 || !w2 || !b2 || (!scores && !mask)) return WGKV_ERR_ARG;
  if (head_dim != 64 && head_dim != 128) return WGKV_ERR_UNSUPPORTED;
  if (inner <= 0 || inner % 16) return WGKV_ERR_UNSUPPORTED;  // 16-column tiles
  if (in_dtype != 0 && in_dtype != 1) return WGKV_ERR_UNSUPPORTED;
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
  a.clamp_min = clamp_min;
  a.threshold = threshold;
  a.scores = scores;
  a.sc_sb = sc_sb;
  a.sc_sh = sc_sh;
  a.mask = mask;
  a.mk_sb = mk_sb;
  a.mk_sh = mk_sh;
  if (((uintptr_t)w1 & 15) != 0) return WGKV_ERR_UNSUPPORTED;
  const int K = n_in * head_dim;
  hipStream_t st = (hipStream_t)stream;
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
