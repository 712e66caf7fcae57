// Per-row FP8 e4m3fn quantization shared by the store kernels: eight lanes
// own one 128-element row, each lane 16 of its elements.  Follows
// microserve/layers/fp8_kv_cache.py:20-27: scale = max(amax, 1e-8) / 448,
// byte = e4m3fn(clamp(x / scale, -448, 448)) with IEEE fp32 division.
#pragma once

#include "mskv_device.h"

namespace mskv {

// max over the 8 lanes of a row group with DPP (no LDS round trip):
// quad_perm [1,0,3,2] and [2,3,0,1] reduce each quad, row_half_mirror then
// pairs lane i with lane 7-i, i.e. the other quad of the group.
__device__ __forceinline__ float max8_dpp(float v) {
  int x = __float_as_int(v);
  v = fmaxf(v, __int_as_float(__builtin_amdgcn_update_dpp(x, x, 0xB1, 0xF, 0xF, false)));
  x = __float_as_int(v);
  v = fmaxf(v, __int_as_float(__builtin_amdgcn_update_dpp(x, x, 0x4E, 0xF, 0xF, false)));
  x = __float_as_int(v);
  v = fmaxf(v, __int_as_float(__builtin_amdgcn_update_dpp(x, x, 0x141, 0xF, 0xF, false)));
  return v;
}

// x / scale for every element of one row, byte-identical after the e4m3
// rounding to hipcc's IEEE fp32 division.  That division is v_div_scale x2,
// v_rcp, a refined reciprocal r = fma(fma(-s, rcp(s), 1), rcp(s), rcp(s)),
// q = x * r and two corrections q += fma(-s, q, x) * r, then v_div_fixup.
// v_div_scale only rescales when the denominator or its reciprocal is
// denormal, when exp(x) - exp(s) >= 96, when the quotient is denormal, or
// when |x| < 2^-103.  Here s = max(amax, 1e-8) / 448 lies in
// [2.2e-11, 7.6e35] and |x / s| <= 448, so only the last two can occur, and
// both mean |x / s| < 2^-66, which encodes to +-0 whatever the low bits.
// Otherwise the sequence below is the same instructions with the
// denominator-only part hoisted out of the element loop; v_div_fixup's
// effect on a finite quotient is the sign rule, copysign(q, x) for s > 0.
struct RowDivider {
  float s, r;
  __device__ __forceinline__ explicit RowDivider(float scale) : s(scale) {
#pragma clang fp contract(off)
    const float r0 = __builtin_amdgcn_rcpf(s);
    const float e = __builtin_fmaf(-s, r0, 1.0f);
    r = __builtin_fmaf(e, r0, r0);
  }
  __device__ __forceinline__ float operator()(float x) const {
#pragma clang fp contract(off)
    float q = x * r;
    const float e1 = __builtin_fmaf(-s, q, x);
    q = __builtin_fmaf(e1, r, q);
    const float e2 = __builtin_fmaf(-s, q, x);
    q = __builtin_fmaf(e2, r, q);
    return __builtin_copysignf(q, x);
  }
};

// Row amax over 8 lanes, scale, quantized bytes of this lane's 16 elements.
__device__ __forceinline__ float quantize16(const float* x, u32x4& q) {
  float amax = 0.0f;
#pragma unroll
  for (int i = 0; i < 16; ++i) amax = fmaxf(amax, fabsf(x[i]));
  amax = max8_dpp(amax);
  const float scale = fmaxf(amax, 1e-8f) / kFp8Max;
  const RowDivider div(scale);
  float y[16];
#pragma unroll
  for (int i = 0; i < 16; ++i)
    y[i] = fminf(fmaxf(div(x[i]), -kFp8Max), kFp8Max);
#pragma unroll
  for (int i = 0; i < 4; ++i)
    q[i] = pack_fp8x4(y[4 * i], y[4 * i + 1], y[4 * i + 2], y[4 * i + 3]);
  return scale;
}

}  // namespace mskv
