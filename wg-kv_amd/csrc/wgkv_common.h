// Shared device helpers for the write-gated dual-cache kernels (gfx950 only).
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include "../../include/wgkv.h"

typedef __attribute__((__vector_size__(8 * sizeof(__bf16)))) __bf16 bf16x8_t;
typedef __attribute__((__vector_size__(4 * sizeof(float)))) float f32x4_t;
typedef __attribute__((__vector_size__(4 * sizeof(uint32_t)))) uint32_t u32x4_t;

#define WGKV_DEVICE __device__ __forceinline__

// ---- bf16 <-> f32 ---------------------------------------------------------
// A bf16 value is the high half of an f32, so widening is a shift / mask.
WGKV_DEVICE float bf16lo(uint32_t w) { return __uint_as_float(w << 16); }
WGKV_DEVICE float bf16hi(uint32_t w) { return __uint_as_float(w & 0xffff0000u); }

// Two f32 -> packed bf16 pair, round to nearest even (v_cvt_pk_bf16_f32).
WGKV_DEVICE uint32_t pack_bf16x2(float lo, float hi) {
  typedef __attribute__((__vector_size__(2 * sizeof(__bf16)))) __bf16 bf16x2_t;
  bf16x2_t r;
  r[0] = (__bf16)lo;
  r[1] = (__bf16)hi;
  return __builtin_bit_cast(uint32_t, r);
}

// Round-to-nearest-even f32 -> bf16 (NaN kept quiet).
WGKV_DEVICE uint16_t f32_to_bf16(float f) {
  uint32_t u = __float_as_uint(f);
  if ((u & 0x7fffffffu) > 0x7f800000u) return (uint16_t)((u >> 16) | 0x40u);
  u += 0x7fffu + ((u >> 16) & 1u);
  return (uint16_t)(u >> 16);
}

// f32 rounded to the nearest bf16 (ties to even) and widened back: one
// v_cvt_pk_bf16_f32 and a shift.
WGKV_DEVICE float round_to_bf16(float x) { return (float)(__bf16)x; }

// ---- DPP row (16-lane) reductions -----------------------------------------
// quad_perm(1,0,3,2), quad_perm(2,3,0,1), row_half_mirror, row_mirror: after
// the four steps every lane of a 16-lane row holds the row-wide result.
#define WGKV_DPP_QP_1032 0xB1
#define WGKV_DPP_QP_2301 0x4E
#define WGKV_DPP_ROW_MIRROR 0x140
#define WGKV_DPP_ROW_HALF_MIRROR 0x141

template <int CTRL>
WGKV_DEVICE float dpp_f32(float x) {
  return __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(x), CTRL, 0xf, 0xf, false));
}

WGKV_DEVICE float row_max16(float x) {
  x = fmaxf(x, dpp_f32<WGKV_DPP_QP_1032>(x));
  x = fmaxf(x, dpp_f32<WGKV_DPP_QP_2301>(x));
  x = fmaxf(x, dpp_f32<WGKV_DPP_ROW_HALF_MIRROR>(x));
  x = fmaxf(x, dpp_f32<WGKV_DPP_ROW_MIRROR>(x));
  return x;
}

WGKV_DEVICE float row_sum16(float x) {
  x += dpp_f32<WGKV_DPP_QP_1032>(x);
  x += dpp_f32<WGKV_DPP_QP_2301>(x);
  x += dpp_f32<WGKV_DPP_ROW_HALF_MIRROR>(x);
  x += dpp_f32<WGKV_DPP_ROW_MIRROR>(x);
  return x;
}

// Wave-uniform max / sum over all 64 lanes.
WGKV_DEVICE float wave_max(float x) {
  x = row_max16(x);
  float a = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(x), 0));
  float b = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(x), 16));
  float c = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(x), 32));
  float d = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(x), 48));
  return fmaxf(fmaxf(a, b), fmaxf(c, d));
}

WGKV_DEVICE float wave_sum(float x) {
  x = row_sum16(x);
  float a = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(x), 0));
  float b = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(x), 16));
  float c = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(x), 32));
  float d = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(x), 48));
  return (a + b) + (c + d);
}

// Inclusive prefix sum over the 64 lanes of a wave.
WGKV_DEVICE int wave_incl_scan(int v, int lane) {
#pragma unroll
  for (int off = 1; off < 64; off <<= 1) {
    const int u = __shfl_up(v, off, 64);
    if (lane >= off) v += u;
  }
  return v;
}

// Sum of an int over all 64 lanes (every lane gets the total).
WGKV_DEVICE int wave_sum_int(int x) {
#pragma unroll
  for (int off = 32; off > 0; off >>= 1) x += __shfl_xor(x, off, 64);
  return x;
}

WGKV_DEVICE float fast_exp2(float x) { return __builtin_amdgcn_exp2f(x); }

// Orders this wave's LDS writes before its later LDS reads of other lanes'
// data (LDS operations of one wave complete in issue order).
WGKV_DEVICE void wave_lds_sync() {
  __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
  __builtin_amdgcn_wave_barrier();
  __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
}

// Block-wide exclusive scan of one int per thread (blockDim.x == 256): a
// wave prefix sum, then the four wave totals through LDS (two barriers).
WGKV_DEVICE int block_exclusive_scan_256(int v, int* s_tmp /* >= 4 ints */, int* total) {
  const int t = threadIdx.x, lane = t & 63, w = t >> 6;
  const int incl = wave_incl_scan(v, lane);
  if (lane == 63) s_tmp[w] = incl;
  __syncthreads();
  const int t0 = s_tmp[0], t1 = s_tmp[1], t2 = s_tmp[2], t3 = s_tmp[3];
  const int before = (w > 0 ? t0 : 0) + (w > 1 ? t1 : 0) + (w > 2 ? t2 : 0);
  if (total) *total = (t0 + t1) + (t2 + t3);
  __syncthreads();
  return before + incl - v;
}

#define WGKV_HIP_CHECK(expr)                       \
  do {                                             \
    hipError_t _e = (expr);                        \
    if (_e != hipSuccess) return WGKV_ERR_HIP;     \
  } while (0)
