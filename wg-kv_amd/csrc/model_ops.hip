// Fused bf16 building blocks of the decoder around the path (the end-to-end
// harness): RMSNorm with the residual add before it, rotary embedding of q
// and k, and the SwiGLU product.  Each replaces a chain of small torch
// kernels (LlamaRMSNorm, src/modeling_llama.py:61-76; apply_rotary_pos_emb
// :115-146; LlamaMLP :149-161; the residual adds :366, :399) with one launch
// and follows the same bf16 rounding points as the torch composition: every
// bf16 x bf16 product and sum is rounded to bf16 where torch rounds it.
#include "wgkv_common.h"

namespace {

// round an f32 to the nearest bf16, returned as f32
WGKV_DEVICE float rb(float x) { return bf16lo(f32_to_bf16(x)); }

WGKV_DEVICE void unpack8(const u32x4_t w, float (&f)[8]) {
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    f[2 * i] = bf16lo(w[i]);
    f[2 * i + 1] = bf16hi(w[i]);
  }
}

WGKV_DEVICE u32x4_t pack8(const float (&f)[8]) {
  u32x4_t w;
#pragma unroll
  for (int i = 0; i < 4; ++i) w[i] = (uint32_t)f32_to_bf16(f[2 * i]) | ((uint32_t)f32_to_bf16(f[2 * i + 1]) << 16);
  return w;
}

// ---- RMSNorm (optionally after the residual add) ---------------------------
// One workgroup per row of `hidden` elements, 8 per 16-byte chunk, at most 4
// chunks per thread (hidden <= 8192).  With a residual: h = bf16(x + res) is
// both the new residual stream (res_out) and the norm's input.
// out = bf16(w * bf16(h * rsqrt(mean(h^2) + eps))).
constexpr int kNormThreads = 256;
constexpr int kNormChunks = 4;

struct NormArgs {
  const uint16_t* x;
  int64_t x_rs;
  const uint16_t* res;
  int64_t r_rs;
  const uint16_t* w;
  uint16_t* out;
  int64_t o_rs;
  uint16_t* res_out;
  int64_t ro_rs;
  int hidden;
  float eps;
};

// The normalisation of one row by a 256-thread workgroup (shared by
// rms_norm_kernel and the GEMV prologue, so both give the same bits): thread
// t holds chunks t, t+256, ... of the row; h = x (+ res) rounded to bf16;
// the mean of squares is summed per thread, over each wave, then over the
// four waves in order.  emit_res(ch, h chunk) and emit(ch, out chunk) receive
// the results.
// rms_norm_row_from takes the thread's chunks already loaded (xc, and rc
// with RES) and gets the norm weight's chunk c (chunk index ch) from
// wchunk(c, ch): the GEMV prologue requests all of them before its weight
// slices.  NC chunks per thread must cover the row (hidden <= 8 * NC * 256).
template <bool RES, int NC, typename WChunk, typename EmitOut, typename EmitRes>
WGKV_DEVICE void rms_norm_row_from(const u32x4_t (&xc)[NC], const u32x4_t (&rc)[NC], WChunk wchunk, int hidden,
                                   float eps, float* s_sum, EmitOut emit, EmitRes emit_res) {
  const int t = threadIdx.x;
  const int nch = hidden / 8;
  float h[NC][8];
  float ss = 0.f;
#pragma unroll
  for (int c = 0; c < NC; ++c) {
    const int ch = t + c * kNormThreads;
    if (ch < nch) {
      unpack8(xc[c], h[c]);
      if (RES) {
        float r[8];
        unpack8(rc[c], r);
#pragma unroll
        for (int i = 0; i < 8; ++i) h[c][i] = rb(h[c][i] + r[i]);
        emit_res(ch, pack8(h[c]));
      }
#pragma unroll
      for (int i = 0; i < 8; ++i) ss = fmaf(h[c][i], h[c][i], ss);
    }
  }
  ss = wave_sum(ss);
  if ((t & 63) == 0) s_sum[t >> 6] = ss;
  __syncthreads();
  float tot = 0.f;
#pragma unroll
  for (int wv = 0; wv < kNormThreads / 64; ++wv) tot += s_sum[wv];
  const float scale = rsqrtf(tot / (float)hidden + eps);
#pragma unroll
  for (int c = 0; c < NC; ++c) {
    const int ch = t + c * kNormThreads;
    if (ch < nch) {
      float wv[8], y[8];
      unpack8(wchunk(c, ch), wv);
#pragma unroll
      for (int i = 0; i < 8; ++i) y[i] = wv[i] * rb(h[c][i] * scale);
      emit(ch, pack8(y));
    }
  }
}

template <int NC>
WGKV_DEVICE void load_norm_chunks(const uint16_t* p, int hidden, u32x4_t (&c)[NC]) {
#pragma unroll
  for (int i = 0; i < NC; ++i) {
    const int ch = threadIdx.x + i * kNormThreads;
    if (ch < hidden / 8) c[i] = *(const u32x4_t*)(p + ch * 8);
  }
}

template <bool RES, typename EmitOut, typename EmitRes>
WGKV_DEVICE void rms_norm_row(const uint16_t* x, const uint16_t* res, const uint16_t* w, int hidden, float eps,
                              float* s_sum, EmitOut emit, EmitRes emit_res) {
  u32x4_t xc[kNormChunks], rc[kNormChunks];
  load_norm_chunks(x, hidden, xc);
  if (RES) load_norm_chunks(res, hidden, rc);
  rms_norm_row_from<RES, kNormChunks>(
      xc, rc, [&](int, int ch) { return *(const u32x4_t*)(w + ch * 8); }, hidden, eps, s_sum, emit, emit_res);
}

template <bool RES>
__global__ __launch_bounds__(kNormThreads) void rms_norm_kernel(NormArgs a) {
  __shared__ float s_sum[kNormThreads / 64];
  const int64_t row = blockIdx.x;
  rms_norm_row<RES>(
      a.x + row * a.x_rs, RES ? a.res + row * a.r_rs : nullptr, a.w, a.hidden, a.eps, s_sum,
      [&](int ch, u32x4_t v) { *(u32x4_t*)(a.out + row * a.o_rs + ch * 8) = v; },
      [&](int ch, u32x4_t v) { *(u32x4_t*)(a.res_out + row * a.ro_rs + ch * 8) = v; });
}

// ---- rotary embedding of q and k (and the copy of v) ------------------------
// Tensor i (0 = q, 1 = k, 2 = v) has H[i] heads, input and output element
// strides (batch, seq, head) and a contiguous head_dim.  Thread = (token,
// head of one of the tensors, 8 consecutive d of the first half) and the
// matching 8 of the second half.  q and k are rotated:
// out[d] = bf16(bf16(x[d] cos[d]) + bf16(-x[d+h] sin[d])),
// out[d+h] = bf16(bf16(x[d+h] cos[d+h]) + bf16(x[d] sin[d+h])), h = D/2;
// v is copied, so the three outputs can share one buffer and strides.
// Optionally q and k first get Qwen3's per-head RMSNorm (nw[0], nw[1]):
// x <- bf16(w * bf16(x * rsqrt(mean_head(x^2) + eps))), the sum of squares
// reduced over the D/16 threads of the head; the normalised k before the
// rotation (the gate's pre-RoPE key) is also stored to kpre.
struct RopeArgs {
  const uint16_t* in[3];
  int64_t is[3][3];
  uint16_t* out[3];
  int64_t os[3][3];
  int H[3];
  const uint16_t* cos;
  const uint16_t* sin;
  int64_t cs_sb, cs_ss;
  int B, S, D;
  const uint16_t* nw[2];
  float eps;
  uint16_t* kpre;
  int64_t kp[3];
  // optional, one decode row (B = S = 1): the step's ring write of the dual
  // cache under deferred gating, as GemvArgs' ring fields: ring[0..1] =
  // (local_ptr, local_length), ring[2] <- the slot; ring_k / ring_v /
  // ring_pk the layer's (Hkv, W, D) ring rows of the K pool, the V pool and
  // the pre-RoPE key store; glen / seqlens the layer's global and attention
  // lengths
  int32_t* ring;
  uint16_t* ring_k;
  uint16_t* ring_v;
  uint16_t* ring_pk;
  const int32_t* glen;
  int32_t* seqlens;
  int W;
};

__global__ __launch_bounds__(256) void rope_kernel(RopeArgs a) {
  const int half = a.D / 2, hch = half / 8;
  const int Ht = a.H[0] + a.H[1] + a.H[2];
  const int64_t total = (int64_t)a.B * a.S * Ht * hch;
  const int64_t idx = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  int slot = 0;
  if (a.ring) {
    const int lp = a.ring[0], ll = max(a.ring[1], 0);
    slot = min(max(ll < a.W ? ll : lp, 0), a.W - 1);  // pointers out of range stay inside the ring
    if (idx == 0) {
      const int cur = ll < a.W ? ll + 1 : a.W;
      for (int h = 0; h < a.H[1]; ++h) a.seqlens[h] = cur + a.glen[h];
      a.ring[2] = slot;
    }
  }
  if (idx >= total) return;
  const int c = (int)(idx % hch);
  int64_t r = idx / hch;
  int hh = (int)(r % Ht);
  r /= Ht;
  const int s = (int)(r % a.S), b = (int)(r / a.S);
  int ten = 0;
  if (hh >= a.H[0]) {
    hh -= a.H[0];
    ten = 1;
    if (hh >= a.H[1]) {
      hh -= a.H[1];
      ten = 2;
    }
  }
  const uint16_t* src = a.in[ten] + b * a.is[ten][0] + s * a.is[ten][1] + hh * a.is[ten][2];
  uint16_t* dst = a.out[ten] + b * a.os[ten][0] + s * a.os[ten][1] + hh * a.os[ten][2];
  const int d0 = c * 8;
  const u32x4_t w1 = *(const u32x4_t*)(src + d0), w2 = *(const u32x4_t*)(src + half + d0);
  // this head's row of the ring (decode row: b = s = 0)
  const int64_t rrow = ((int64_t)hh * a.W + slot) * a.D;
  if (ten == 2) {
    *(u32x4_t*)(dst + d0) = w1;
    *(u32x4_t*)(dst + half + d0) = w2;
    if (a.ring) {
      *(u32x4_t*)(a.ring_v + rrow + d0) = w1;
      *(u32x4_t*)(a.ring_v + rrow + half + d0) = w2;
    }
    return;
  }
  const uint16_t* cs = a.cos + b * a.cs_sb + s * a.cs_ss;
  const uint16_t* sn = a.sin + b * a.cs_sb + s * a.cs_ss;
  float x1[8], x2[8], c1[8], c2[8], s1[8], s2[8], o1[8], o2[8];
  unpack8(w1, x1);
  unpack8(w2, x2);
  if (a.nw[ten]) {
    // the head's D/16 threads are consecutive lanes (hch divides 64)
    float ss = 0.f;
#pragma unroll
    for (int e = 0; e < 8; ++e) ss = fmaf(x1[e], x1[e], ss);
#pragma unroll
    for (int e = 0; e < 8; ++e) ss = fmaf(x2[e], x2[e], ss);
    if (hch >= 2) ss += dpp_f32<WGKV_DPP_QP_1032>(ss);
    if (hch >= 4) ss += dpp_f32<WGKV_DPP_QP_2301>(ss);
    if (hch >= 8) ss += dpp_f32<WGKV_DPP_ROW_HALF_MIRROR>(ss);
    if (hch >= 16) ss += dpp_f32<WGKV_DPP_ROW_MIRROR>(ss);
    const float scale = rsqrtf(ss / (float)a.D + a.eps);
    float n1[8], n2[8];
    unpack8(*(const u32x4_t*)(a.nw[ten] + d0), n1);
    unpack8(*(const u32x4_t*)(a.nw[ten] + half + d0), n2);
#pragma unroll
    for (int e = 0; e < 8; ++e) {
      x1[e] = rb(n1[e] * rb(x1[e] * scale));
      x2[e] = rb(n2[e] * rb(x2[e] * scale));
    }
    if (ten == 1 && a.kpre) {
      uint16_t* kp = a.kpre + b * a.kp[0] + s * a.kp[1] + hh * a.kp[2];
      *(u32x4_t*)(kp + d0) = pack8(x1);
      *(u32x4_t*)(kp + half + d0) = pack8(x2);
    }
  }
  if (ten == 1 && a.ring) {  // the pre-RoPE key (normalised when the head norm is on)
    *(u32x4_t*)(a.ring_pk + rrow + d0) = pack8(x1);
    *(u32x4_t*)(a.ring_pk + rrow + half + d0) = pack8(x2);
  }
  unpack8(*(const u32x4_t*)(cs + d0), c1);
  unpack8(*(const u32x4_t*)(cs + half + d0), c2);
  unpack8(*(const u32x4_t*)(sn + d0), s1);
  unpack8(*(const u32x4_t*)(sn + half + d0), s2);
#pragma unroll
  for (int e = 0; e < 8; ++e) {
    o1[e] = rb(rb(x1[e] * c1[e]) + rb(-x2[e] * s1[e]));
    o2[e] = rb(rb(x2[e] * c2[e]) + rb(x1[e] * s2[e]));
  }
  *(u32x4_t*)(dst + d0) = pack8(o1);
  *(u32x4_t*)(dst + half + d0) = pack8(o2);
  if (ten == 1 && a.ring) {
    *(u32x4_t*)(a.ring_k + rrow + d0) = pack8(o1);
    *(u32x4_t*)(a.ring_k + rrow + half + d0) = pack8(o2);
  }
}

// ---- SwiGLU: out = bf16(bf16(silu(g)) * u) ----------------------------------
// rows of `cols` elements; g and u with their own row strides, out contiguous
__global__ __launch_bounds__(256) void silu_mul_kernel(const uint16_t* g, int64_t g_rs, const uint16_t* u,
                                                       int64_t u_rs, uint16_t* out, int64_t rows, int cols) {
  const int c8 = cols / 8;
  const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (i >= rows * c8) return;
  const int64_t row = i / c8;
  const int c = (int)(i - row * c8) * 8;
  float gv[8], uv[8], o[8];
  unpack8(*(const u32x4_t*)(g + row * g_rs + c), gv);
  unpack8(*(const u32x4_t*)(u + row * u_rs + c), uv);
#pragma unroll
  for (int e = 0; e < 8; ++e) o[e] = rb(gv[e] / (1.0f + expf(-gv[e]))) * uv[e];
  *(u32x4_t*)(out + row * (int64_t)cols + c) = pack8(o);
}

// ---- one-token products y = W x (decode steps) -----------------------------
// Replaces the torch GEMMs of a decode step, where the activation is a single
// row (q/k/v, o, gate/up and down projections, LM head): W (N, K) bf16 with
// row stride w_rs, x (K) bf16, fp32 accumulation, y bf16.  Workgroup = 4
// waves; wave w of workgroup b computes row pair p = 4b + w.  x is staged in
// LDS -- optionally as RMSNorm(x (+ residual)) computed by the workgroup
// itself with rms_norm_row, so the norm costs no launch (workgroup 0 stores
// the new residual stream) -- and lane l streams 16-byte slices l, l+64, ...
// of both rows, eight slices per row in flight, multiplying them on
// v_dot2_f32_bf16; each row is then summed over the wave.  Row pairs and
// epilogues, with torch's bf16 rounding points:
//   mode 0  rows 2p, 2p+1:  y[r] = bf16(acc)
//   mode 1  rows 2p, 2p+1:  y[r] = bf16(res[r] + bf16(acc))            (residual add)
//   mode 2  rows p, N+p of the stacked [gate; up] weight:
//           y[p] = bf16(bf16(silu(g)) * u), g = bf16(acc_gate), u = bf16(acc_up)
//   mode 3  q/k/v rows (Hq + 2 Hkv heads of D): rows d and d + D/2 of a head;
//           q and k heads rotated as apply_rotary_pos_emb rounds (see
//           rope_kernel), v copied, all into y (the layout of W's rows), and
//           the unrotated k into kraw (Hkv * D)
constexpr int kGemvWaves = 4;
constexpr int kGemvBatch = 8;  // slices per row and lane in flight
static_assert(kGemvWaves * 64 == kNormThreads, "the GEMV prologue normalises with the RMSNorm thread mapping");

struct GemvArgs {
  const uint16_t* w;
  int64_t w_rs;
  const uint16_t* x;
  uint16_t* y;
  const uint16_t* res;
  int N, K, mode;
  // optional RMSNorm prologue: x <- norm_w * bf16(h * rsqrt(mean(h^2) + eps)),
  // h = x (+ norm_res); workgroup 0 stores h to norm_res_out
  const uint16_t* norm_w;
  const uint16_t* norm_res;
  uint16_t* norm_res_out;
  float eps;
  // mode 3
  const uint16_t* cos;
  const uint16_t* sin;
  uint16_t* kraw;
  int hq, hkv, hd;
  // mode 3, optional: the decode step's ring write of the new token (the
  // deferred-gating append of the dual cache), ring != nullptr.  ring[0..1]
  // = (local_ptr, local_length) of the window of W slots; ring_k / ring_v /
  // ring_pk are the layer's (Hkv, W, D) ring rows in the K pool, the V pool
  // and the pre-RoPE key store; glen / seqlens the layer's Hkv global lengths
  // and attention lengths.
  int32_t* ring;
  uint16_t* ring_k;
  uint16_t* ring_v;
  uint16_t* ring_pk;
  const int32_t* glen;
  int32_t* seqlens;
  int W;
};

typedef __attribute__((__vector_size__(2 * sizeof(__bf16)))) __bf16 bf16x2v_t;
WGKV_DEVICE float dot2(uint32_t a, uint32_t b, float c) {
  return __builtin_amdgcn_fdot2_f32_bf16(__builtin_bit_cast(bf16x2v_t, a), __builtin_bit_cast(bf16x2v_t, b), c, false);
}

template <bool XPRE>
__global__ __launch_bounds__(64 * kGemvWaves) void gemv_kernel(GemvArgs a) {
  extern __shared__ u32x4_t xs[];
  __shared__ float s_sum[kGemvWaves];
  const int lane = threadIdx.x & 63, wid = threadIdx.x >> 6;
  const int pair = blockIdx.x * kGemvWaves + wid;
  const int half = a.hd / 2;
  const int npairs = a.mode == 2 ? a.N : a.mode == 3 ? a.N / 2 : (a.N + 1) / 2;
  const int p = min(pair, npairs - 1);  // waves past the last pair compute it again and store nothing
  int r0, r1;
  if (a.mode == 2) {
    r0 = p;
    r1 = a.N + p;
  } else if (a.mode == 3) {
    r0 = (p / half) * a.hd + p % half;
    r1 = r0 + half;
  } else {
    r0 = 2 * p;
    r1 = min(2 * p + 1, a.N - 1);
  }
  // the ring slot this step writes (decode_append_kernel's rule), requested
  // with the other inputs so the epilogue does not wait for it
  int slot = 0, cur = 0;
  if (a.ring) {
    const int lp = a.ring[0], ll = max(a.ring[1], 0);
    slot = min(max(ll < a.W ? ll : lp, 0), a.W - 1);  // pointers out of range stay inside the ring
    cur = ll < a.W ? ll + 1 : a.W;
  }
  const u32x4_t* w0 = (const u32x4_t*)(a.w + (int64_t)r0 * a.w_rs);
  const u32x4_t* w1 = (const u32x4_t*)(a.w + (int64_t)r1 * a.w_rs);
  const int ns = a.K / 8;
  // XPRE (the norm prologue, K <= 4096): x, the norm's residual and its
  // weight are requested first, then the first slices of the rows.  Vector memory loads
  // complete in order, so the norm then runs while the row slices are still
  // in flight; requested after them (the other instance: no norm, or longer
  // rows) x waits for the slices, which costs only the staging there.
  constexpr int kXPre = 2;  // 16-byte chunks per thread: 2 * 8 * 256 = 4096 elements
  u32x4_t xc[kXPre], rc[kXPre], wc[kXPre];
  if constexpr (XPRE) {
    load_norm_chunks(a.x, a.K, xc);
    if (a.norm_res) load_norm_chunks(a.norm_res, a.K, rc);
    load_norm_chunks(a.norm_w, a.K, wc);
  }
  u32x4_t b0[kGemvBatch], b1[kGemvBatch];
#pragma unroll
  for (int u = 0; u < kGemvBatch; ++u) {
    const int sl = min(lane + 64 * u, ns - 1);
    b0[u] = __builtin_nontemporal_load(w0 + sl);
    b1[u] = __builtin_nontemporal_load(w1 + sl);
  }
  if (a.norm_w) {
    auto to_lds = [&](int ch, u32x4_t v) { xs[ch] = v; };
    auto to_res = [&](int ch, u32x4_t v) {
      if (blockIdx.x == 0) ((u32x4_t*)a.norm_res_out)[ch] = v;
    };
    if constexpr (XPRE) {
      auto wpre = [&](int c, int) { return wc[c]; };
      if (a.norm_res) rms_norm_row_from<true, kXPre>(xc, rc, wpre, a.K, a.eps, s_sum, to_lds, to_res);
      else rms_norm_row_from<false, kXPre>(xc, rc, wpre, a.K, a.eps, s_sum, to_lds, [](int, u32x4_t) {});
    } else {
      if (a.norm_res) rms_norm_row<true>(a.x, a.norm_res, a.norm_w, a.K, a.eps, s_sum, to_lds, to_res);
      else rms_norm_row<false>(a.x, nullptr, a.norm_w, a.K, a.eps, s_sum, to_lds, [](int, u32x4_t) {});
    }
  } else {
    for (int sl = threadIdx.x; sl < ns; sl += 64 * kGemvWaves) xs[sl] = ((const u32x4_t*)a.x)[sl];
  }
  __syncthreads();
  float acc0 = 0.f, acc1 = 0.f;
  for (int s0 = 0;;) {
#pragma unroll
    for (int u = 0; u < kGemvBatch; ++u) {
      const int sl = s0 + lane + 64 * u;
      if (sl < ns) {
        const u32x4_t xv = xs[sl];
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          acc0 = dot2(b0[u][e], xv[e], acc0);
          acc1 = dot2(b1[u][e], xv[e], acc1);
        }
      }
    }
    s0 += 64 * kGemvBatch;
    if (s0 >= ns) break;
#pragma unroll
    for (int u = 0; u < kGemvBatch; ++u) {
      const int sl = min(s0 + lane + 64 * u, ns - 1);
      b0[u] = __builtin_nontemporal_load(w0 + sl);
      b1[u] = __builtin_nontemporal_load(w1 + sl);
    }
  }
  acc0 = wave_sum(acc0);
  acc1 = wave_sum(acc1);
  if (a.ring && pair == a.hq * half) {
    // the wave of the first k pair: attention lengths (current window + the
    // global length) and the slot written, for the step's later decisions
    if (lane < a.hkv) a.seqlens[lane] = cur + a.glen[lane];
    if (lane == 0) a.ring[2] = slot;
  }
  if (lane != 0 || pair >= npairs) return;
  if (a.mode == 2) {
    const float g = rb(acc0), u = rb(acc1);
    a.y[p] = f32_to_bf16(rb(g / (1.0f + expf(-g))) * u);
    return;
  }
  const float v0 = rb(acc0), v1 = rb(acc1);
  if (a.mode == 3) {
    const int head = p / half, d = p % half;
    if (head < a.hq + a.hkv) {
      const float c0 = bf16lo(a.cos[d]), s0 = bf16lo(a.sin[d]);
      const float c1 = bf16lo(a.cos[d + half]), s1 = bf16lo(a.sin[d + half]);
      const uint16_t y0 = f32_to_bf16(rb(v0 * c0) + rb(-v1 * s0));
      const uint16_t y1 = f32_to_bf16(rb(v1 * c1) + rb(v0 * s1));
      a.y[r0] = y0;
      a.y[r1] = y1;
      if (head >= a.hq) {
        const uint16_t k0 = f32_to_bf16(v0), k1 = f32_to_bf16(v1);
        a.kraw[r0 - a.hq * a.hd] = k0;
        a.kraw[r1 - a.hq * a.hd] = k1;
        if (a.ring) {
          const int64_t row = ((int64_t)(head - a.hq) * a.W + slot) * a.hd;
          a.ring_k[row + d] = y0;
          a.ring_k[row + d + half] = y1;
          a.ring_pk[row + d] = k0;
          a.ring_pk[row + d + half] = k1;
        }
      }
    } else {
      const uint16_t y0 = f32_to_bf16(v0), y1 = f32_to_bf16(v1);
      a.y[r0] = y0;
      a.y[r1] = y1;
      if (a.ring) {
        const int64_t row = ((int64_t)(head - a.hq - a.hkv) * a.W + slot) * a.hd;
        a.ring_v[row + d] = y0;
        a.ring_v[row + d + half] = y1;
      }
    }
    return;
  }
  if (a.mode == 1) {
    a.y[r0] = f32_to_bf16(bf16lo(a.res[r0]) + v0);
    if (r1 != r0) a.y[r1] = f32_to_bf16(bf16lo(a.res[r1]) + v1);
  } else {
    a.y[r0] = f32_to_bf16(v0);
    if (r1 != r0) a.y[r1] = f32_to_bf16(v1);
  }
}

bool misaligned(const void* p) { return ((uintptr_t)p & 15) != 0; }

}  // namespace

extern "C" int wgkv_rms_norm(const void* x, int64_t x_row_stride, const void* residual, int64_t res_row_stride,
                             const void* weight, void* out, int64_t out_row_stride, void* residual_out,
                             int64_t res_out_row_stride, int32_t rows, int32_t hidden, float eps, void* stream) {
  if (!x || !weight || !out || rows < 0 || hidden <= 0) return WGKV_ERR_ARG;
  if ((residual == nullptr) != (residual_out == nullptr)) return WGKV_ERR_ARG;
  if (hidden % 8 || hidden > 8 * kNormChunks * kNormThreads) return WGKV_ERR_UNSUPPORTED;
  if (misaligned(x) || misaligned(weight) || misaligned(out) || misaligned(residual) || misaligned(residual_out))
    return WGKV_ERR_UNSUPPORTED;
  if ((x_row_stride | res_row_stride | out_row_stride | res_out_row_stride) & 7) return WGKV_ERR_UNSUPPORTED;
  if (rows == 0) return WGKV_OK;
  NormArgs a = {(const uint16_t*)x, x_row_stride, (const uint16_t*)residual, res_row_stride,
                (const uint16_t*)weight, (uint16_t*)out, out_row_stride, (uint16_t*)residual_out,
                res_out_row_stride, hidden, eps};
  if (residual)
    hipLaunchKernelGGL(rms_norm_kernel<true>, dim3(rows), dim3(kNormThreads), 0, (hipStream_t)stream, a);
  else
    hipLaunchKernelGGL(rms_norm_kernel<false>, dim3(rows), dim3(kNormThreads), 0, (hipStream_t)stream, a);
  return hipGetLastError() == hipSuccess ? WGKV_OK : WGKV_ERR_HIP;
}

namespace {

// wgkv_rope_qkv_norm with the ring fields of RopeArgs (all null / 0 without the ring write)
int rope_launch(const void* q, int64_t q_sb, int64_t q_ss, int64_t q_sh,
                const void* k, int64_t k_sb, int64_t k_ss, int64_t k_sh,
                const void* v, int64_t v_sb, int64_t v_ss, int64_t v_sh,
                const void* cos, const void* sin, int64_t cs_sb, int64_t cs_ss,
                void* q_out, int64_t qo_sb, int64_t qo_ss, int64_t qo_sh,
                void* k_out, int64_t ko_sb, int64_t ko_ss, int64_t ko_sh,
                void* v_out, int64_t vo_sb, int64_t vo_ss, int64_t vo_sh,
                int32_t batch, int32_t seq_len, int32_t num_q_heads, int32_t num_kv_heads,
                int32_t head_dim, const void* q_norm_weight, const void* k_norm_weight, float eps,
                void* k_pre, int64_t kp_sb, int64_t kp_ss, int64_t kp_sh, const RopeArgs& ring, void* stream) {
  if (!q || !k || !cos || !sin || !q_out || !k_out || (v == nullptr) != (v_out == nullptr)) return WGKV_ERR_ARG;
  if (batch <= 0 || seq_len <= 0 || num_q_heads <= 0 || num_kv_heads <= 0) return WGKV_ERR_ARG;
  if (head_dim % 16) return WGKV_ERR_UNSUPPORTED;
  if ((q_norm_weight || k_norm_weight) && head_dim > 256) return WGKV_ERR_UNSUPPORTED;
  if (misaligned(q_norm_weight) || misaligned(k_norm_weight) || misaligned(k_pre)) return WGKV_ERR_UNSUPPORTED;
  if (k_pre && !k_norm_weight) return WGKV_ERR_ARG;
  if ((kp_sb | kp_ss | kp_sh) & 7) return WGKV_ERR_UNSUPPORTED;
  if (misaligned(q) || misaligned(k) || misaligned(v) || misaligned(cos) || misaligned(sin) || misaligned(q_out) ||
      misaligned(k_out) || misaligned(v_out))
    return WGKV_ERR_UNSUPPORTED;
  if ((q_sb | q_ss | q_sh | k_sb | k_ss | k_sh | v_sb | v_ss | v_sh | cs_sb | cs_ss | qo_sb | qo_ss | qo_sh | ko_sb |
       ko_ss | ko_sh | vo_sb | vo_ss | vo_sh) & 7)
    return WGKV_ERR_UNSUPPORTED;
  RopeArgs a = {};
  a.in[0] = (const uint16_t*)q;
  a.in[1] = (const uint16_t*)k;
  a.in[2] = (const uint16_t*)v;
  a.out[0] = (uint16_t*)q_out;
  a.out[1] = (uint16_t*)k_out;
  a.out[2] = (uint16_t*)v_out;
  const int64_t is[3][3] = {{q_sb, q_ss, q_sh}, {k_sb, k_ss, k_sh}, {v_sb, v_ss, v_sh}};
  const int64_t os[3][3] = {{qo_sb, qo_ss, qo_sh}, {ko_sb, ko_ss, ko_sh}, {vo_sb, vo_ss, vo_sh}};
  for (int i = 0; i < 3; ++i)
    for (int j = 0; j < 3; ++j) {
      a.is[i][j] = is[i][j];
      a.os[i][j] = os[i][j];
    }
  a.H[0] = num_q_heads;
  a.H[1] = num_kv_heads;
  a.H[2] = v ? num_kv_heads : 0;
  a.cos = (const uint16_t*)cos;
  a.sin = (const uint16_t*)sin;
  a.cs_sb = cs_sb;
  a.cs_ss = cs_ss;
  a.B = batch;
  a.S = seq_len;
  a.D = head_dim;
  a.nw[0] = (const uint16_t*)q_norm_weight;
  a.nw[1] = (const uint16_t*)k_norm_weight;
  a.eps = eps;
  a.kpre = (uint16_t*)k_pre;
  a.kp[0] = kp_sb;
  a.kp[1] = kp_ss;
  a.kp[2] = kp_sh;
  a.ring = ring.ring;
  a.ring_k = ring.ring_k;
  a.ring_v = ring.ring_v;
  a.ring_pk = ring.ring_pk;
  a.glen = ring.glen;
  a.seqlens = ring.seqlens;
  a.W = ring.W;
  const int64_t total = (int64_t)batch * seq_len * (a.H[0] + a.H[1] + a.H[2]) * (head_dim / 16);
  hipLaunchKernelGGL(rope_kernel, dim3((unsigned)((total + 255) / 256)), dim3(256), 0, (hipStream_t)stream, a);
  return hipGetLastError() == hipSuccess ? WGKV_OK : WGKV_ERR_HIP;
}

}  // namespace

extern "C" int wgkv_rope_qkv_norm(const void* q, int64_t q_sb, int64_t q_ss, int64_t q_sh,
                             const void* k, int64_t k_sb, int64_t k_ss, int64_t k_sh,
                             const void* v, int64_t v_sb, int64_t v_ss, int64_t v_sh,
                             const void* cos, const void* sin, int64_t cs_sb, int64_t cs_ss,
                             void* q_out, int64_t qo_sb, int64_t qo_ss, int64_t qo_sh,
                             void* k_out, int64_t ko_sb, int64_t ko_ss, int64_t ko_sh,
                             void* v_out, int64_t vo_sb, int64_t vo_ss, int64_t vo_sh,
                             int32_t batch, int32_t seq_len, int32_t num_q_heads, int32_t num_kv_heads,
                             int32_t head_dim, const void* q_norm_weight, const void* k_norm_weight, float eps,
                             void* k_pre, int64_t kp_sb, int64_t kp_ss, int64_t kp_sh, void* stream) {
  return rope_launch(q, q_sb, q_ss, q_sh, k, k_sb, k_ss, k_sh, v, v_sb, v_ss, v_sh, cos, sin, cs_sb, cs_ss, q_out,
                     qo_sb, qo_ss, qo_sh, k_out, ko_sb, ko_ss, ko_sh, v_out, vo_sb, vo_ss, vo_sh, batch, seq_len,
                     num_q_heads, num_kv_heads, head_dim, q_norm_weight, k_norm_weight, eps, k_pre, kp_sb, kp_ss,
                     kp_sh, RopeArgs{}, stream);
}

extern "C" int wgkv_rope_qkv_norm_ring_write(const void* q, int64_t q_sh, const void* k, int64_t k_sh,
                                             const void* v, int64_t v_sh, const void* cos, const void* sin,
                                             void* q_out, int64_t qo_sh, void* k_out, int64_t ko_sh,
                                             void* v_out, int64_t vo_sh,
                                             int32_t num_q_heads, int32_t num_kv_heads, int32_t head_dim,
                                             const void* q_norm_weight, const void* k_norm_weight, float eps,
                                             void* k_pre, int64_t kp_sh,
                                             int32_t layer, int32_t num_layers, int32_t local_window,
                                             int32_t* ring_state, void* pool_k, void* pool_v, void* local_pre_key,
                                             const int32_t* global_lengths, int32_t* cache_seqlens, void* stream) {
  if (!v || !v_out || !ring_state || !pool_k || !pool_v || !local_pre_key || !global_lengths || !cache_seqlens)
    return WGKV_ERR_ARG;
  if (layer < 0 || layer >= num_layers || local_window <= 0 || num_kv_heads <= 0 || head_dim <= 0)
    return WGKV_ERR_ARG;
  if (misaligned(pool_k) || misaligned(pool_v) || misaligned(local_pre_key)) return WGKV_ERR_UNSUPPORTED;
  const int64_t base = (int64_t)layer * num_kv_heads * local_window * head_dim;
  RopeArgs r = {};
  r.ring = ring_state;
  r.ring_k = (uint16_t*)pool_k + base;
  r.ring_v = (uint16_t*)pool_v + base;
  r.ring_pk = (uint16_t*)local_pre_key + base;
  r.glen = global_lengths + (int64_t)layer * num_kv_heads;
  r.seqlens = cache_seqlens;
  r.W = local_window;
  // one decode row: batch and sequence strides do not matter
  return rope_launch(q, 0, 0, q_sh, k, 0, 0, k_sh, v, 0, 0, v_sh, cos, sin, 0, 0, q_out, 0, 0, qo_sh, k_out, 0, 0,
                     ko_sh, v_out, 0, 0, vo_sh, 1, 1, num_q_heads, num_kv_heads, head_dim, q_norm_weight,
                     k_norm_weight, eps, k_pre, 0, 0, kp_sh, r, stream);
}

extern "C" int wgkv_rope_qkv(const void* q, int64_t q_sb, int64_t q_ss, int64_t q_sh,
                             const void* k, int64_t k_sb, int64_t k_ss, int64_t k_sh,
                             const void* v, int64_t v_sb, int64_t v_ss, int64_t v_sh,
                             const void* cos, const void* sin, int64_t cs_sb, int64_t cs_ss,
                             void* q_out, int64_t qo_sb, int64_t qo_ss, int64_t qo_sh,
                             void* k_out, int64_t ko_sb, int64_t ko_ss, int64_t ko_sh,
                             void* v_out, int64_t vo_sb, int64_t vo_ss, int64_t vo_sh,
                             int32_t batch, int32_t seq_len, int32_t num_q_heads, int32_t num_kv_heads,
                             int32_t head_dim, void* stream) {
  return wgkv_rope_qkv_norm(q, q_sb, q_ss, q_sh, k, k_sb, k_ss, k_sh, v, v_sb, v_ss, v_sh, cos, sin, cs_sb, cs_ss,
                            q_out, qo_sb, qo_ss, qo_sh, k_out, ko_sb, ko_ss, ko_sh, v_out, vo_sb, vo_ss, vo_sh,
                            batch, seq_len, num_q_heads, num_kv_heads, head_dim, nullptr, nullptr, 0.f, nullptr,
                            0, 0, 0, stream);
}

extern "C" int wgkv_silu_mul(const void* gate, int64_t gate_row_stride, const void* up, int64_t up_row_stride,
                             void* out, int64_t rows, int32_t cols, void* stream) {
  if (!gate || !up || !out || rows < 0 || cols <= 0) return WGKV_ERR_ARG;
  if (cols % 8 || misaligned(gate) || misaligned(up) || misaligned(out) || (gate_row_stride | up_row_stride) & 7)
    return WGKV_ERR_UNSUPPORTED;
  if (rows == 0) return WGKV_OK;
  const int64_t n8 = rows * (cols / 8);
  hipLaunchKernelGGL(silu_mul_kernel, dim3((unsigned)((n8 + 255) / 256)), dim3(256), 0, (hipStream_t)stream,
                     (const uint16_t*)gate, gate_row_stride, (const uint16_t*)up, up_row_stride, (uint16_t*)out,
                     rows, cols);
  return hipGetLastError() == hipSuccess ? WGKV_OK : WGKV_ERR_HIP;
}

namespace {

// wgkv_gemv_ex with the ring fields of GemvArgs (all null / 0 without the ring write)
int gemv_ex_launch(const void* w, int64_t w_row_stride, int32_t n, int32_t k, const void* x, void* y,
                   int32_t mode, const void* residual,
                   const void* norm_weight, const void* norm_residual, void* norm_residual_out, float eps,
                   const void* cos, const void* sin, void* k_raw,
                   int32_t num_q_heads, int32_t num_kv_heads, int32_t head_dim, const GemvArgs& ring, void* stream) {
  if (!w || !x || !y || n <= 0 || k <= 0 || mode < 0 || mode > 3) return WGKV_ERR_ARG;
  if (mode == 1 && !residual) return WGKV_ERR_ARG;
  if ((norm_residual == nullptr) != (norm_residual_out == nullptr) || (norm_residual && !norm_weight))
    return WGKV_ERR_ARG;
  if (k % 8 || k > 8 * 4096 || w_row_stride % 8 || misaligned(w) || misaligned(x)) return WGKV_ERR_UNSUPPORTED;
  if (norm_weight && (k > 8 * kNormChunks * kNormThreads || misaligned(norm_weight) || misaligned(norm_residual) ||
                      misaligned(norm_residual_out)))
    return WGKV_ERR_UNSUPPORTED;
  if (mode == 3) {
    if (!cos || !sin || !k_raw || num_q_heads <= 0 || num_kv_heads <= 0 || head_dim <= 0 || head_dim % 2)
      return WGKV_ERR_ARG;
    if (n != (num_q_heads + 2 * num_kv_heads) * head_dim) return WGKV_ERR_ARG;
  }
  GemvArgs a = {};
  a.w = (const uint16_t*)w;
  a.w_rs = w_row_stride;
  a.x = (const uint16_t*)x;
  a.y = (uint16_t*)y;
  a.res = (const uint16_t*)residual;
  a.N = n;
  a.K = k;
  a.mode = mode;
  a.norm_w = (const uint16_t*)norm_weight;
  a.norm_res = (const uint16_t*)norm_residual;
  a.norm_res_out = (uint16_t*)norm_residual_out;
  a.eps = eps;
  a.cos = (const uint16_t*)cos;
  a.sin = (const uint16_t*)sin;
  a.kraw = (uint16_t*)k_raw;
  a.hq = num_q_heads;
  a.hkv = num_kv_heads;
  a.hd = mode == 3 ? head_dim : 2;
  a.ring = ring.ring;
  a.ring_k = ring.ring_k;
  a.ring_v = ring.ring_v;
  a.ring_pk = ring.ring_pk;
  a.glen = ring.glen;
  a.seqlens = ring.seqlens;
  a.W = ring.W;
  const int npairs = mode == 2 ? n : mode == 3 ? n / 2 : (n + 1) / 2;
  const int blocks = (npairs + kGemvWaves - 1) / kGemvWaves;
  if (norm_weight && k <= 4096)
    hipLaunchKernelGGL(gemv_kernel<true>, dim3(blocks), dim3(64 * kGemvWaves), (size_t)k * 2, (hipStream_t)stream, a);
  else
    hipLaunchKernelGGL(gemv_kernel<false>, dim3(blocks), dim3(64 * kGemvWaves), (size_t)k * 2, (hipStream_t)stream, a);
  return hipGetLastError() == hipSuccess ? WGKV_OK : WGKV_ERR_HIP;
}

}  // namespace

extern "C" int wgkv_gemv_ex(const void* w, int64_t w_row_stride, int32_t n, int32_t k, const void* x, void* y,
                            int32_t mode, const void* residual,
                            const void* norm_weight, const void* norm_residual, void* norm_residual_out, float eps,
                            const void* cos, const void* sin, void* k_raw,
                            int32_t num_q_heads, int32_t num_kv_heads, int32_t head_dim, void* stream) {
  return gemv_ex_launch(w, w_row_stride, n, k, x, y, mode, residual, norm_weight, norm_residual, norm_residual_out,
                        eps, cos, sin, k_raw, num_q_heads, num_kv_heads, head_dim, GemvArgs{}, stream);
}

extern "C" int wgkv_qkv_rope_ring_write(const void* w, int64_t w_row_stride, int32_t k, const void* x, void* y,
                                        const void* norm_weight, float eps, const void* cos, const void* sin,
                                        void* k_raw, int32_t num_q_heads, int32_t num_kv_heads, int32_t head_dim,
                                        int32_t layer, int32_t num_layers, int32_t local_window, int32_t* ring_state,
                                        void* pool_k, void* pool_v, void* local_pre_key,
                                        const int32_t* global_lengths, int32_t* cache_seqlens, void* stream) {
  if (!ring_state || !pool_k || !pool_v || !local_pre_key || !global_lengths || !cache_seqlens) return WGKV_ERR_ARG;
  if (layer < 0 || layer >= num_layers || local_window <= 0 || num_kv_heads <= 0) return WGKV_ERR_ARG;
  if (num_kv_heads > 64) return WGKV_ERR_UNSUPPORTED;  // one wave writes the attention lengths
  const int64_t base = (int64_t)layer * num_kv_heads * local_window * head_dim;
  GemvArgs r = {};
  r.ring = ring_state;
  r.ring_k = (uint16_t*)pool_k + base;
  r.ring_v = (uint16_t*)pool_v + base;
  r.ring_pk = (uint16_t*)local_pre_key + base;
  r.glen = global_lengths + (int64_t)layer * num_kv_heads;
  r.seqlens = cache_seqlens;
  r.W = local_window;
  return gemv_ex_launch(w, w_row_stride, (num_q_heads + 2 * num_kv_heads) * head_dim, k, x, y, 3, nullptr,
                        norm_weight, nullptr, nullptr, eps, cos, sin, k_raw, num_q_heads, num_kv_heads, head_dim, r,
                        stream);
}

extern "C" int wgkv_gemv(const void* w, int64_t w_row_stride, int32_t n, int32_t k, const void* x, void* y,
                         int32_t mode, const void* residual, void* stream) {
  if (mode == 3) return WGKV_ERR_ARG;
  return wgkv_gemv_ex(w, w_row_stride, n, k, x, y, mode, residual, nullptr, nullptr, nullptr, 0.f, nullptr, nullptr,
                      nullptr, 0, 0, 0, stream);
}
