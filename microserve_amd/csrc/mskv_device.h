// Device helpers shared by the mskv kernels (gfx950 / CDNA4 only).
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace mskv {

typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef _Float16 f16x8 __attribute__((ext_vector_type(8)));
typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef _Float16 f16x2 __attribute__((ext_vector_type(2)));
typedef __bf16 bf16x2 __attribute__((ext_vector_type(2)));
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
typedef uint32_t u32x2 __attribute__((ext_vector_type(2)));
typedef int i32x2 __attribute__((ext_vector_type(2)));
typedef int i32x8 __attribute__((ext_vector_type(8)));

constexpr int kHeadDim = 128;
constexpr float kFp8Max = 448.0f;
constexpr float kLog2e = 1.4426950408889634f;

// ---------------------------------------------------------------- buffers --
// Raw buffer resources: loads past num_records return zeros instead of
// faulting, so a page whose block id is invalid is read through a
// zero-length resource.  Word 3 is the gfx9 data-format word.
__device__ __forceinline__ __amdgpu_buffer_rsrc_t make_rsrc(const void* p,
                                                            uint32_t bytes) {
  return __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(p), (short)0,
                                           (int)bytes, 0x00020000);
}

__device__ __forceinline__ u32x4 buf_load16(__amdgpu_buffer_rsrc_t r,
                                            uint32_t off) {
  return __builtin_bit_cast(u32x4,
                            __builtin_amdgcn_raw_buffer_load_b128(r, (int)off, 0, 0));
}

// Streaming form (cache policy "nt"): for data read exactly once.  With
// fully coalesced rows it lets the vector L1 stream lines instead of
// holding them, which measured ~8% more decode bandwidth.
__device__ __forceinline__ u32x4 buf_load16_nt(__amdgpu_buffer_rsrc_t r,
                                               uint32_t off) {
  return __builtin_bit_cast(u32x4,
                            __builtin_amdgcn_raw_buffer_load_b128(r, (int)off, 0, 2));
}

__device__ __forceinline__ float buf_load_f32(__amdgpu_buffer_rsrc_t r,
                                              uint32_t off) {
  return __builtin_bit_cast(float,
                            __builtin_amdgcn_raw_buffer_load_b32(r, (int)off, 0, 0));
}

// LDS byte offset of 16-byte chunk `chunk` of row `row` in a tile of
// 128-byte rows, XOR-swizzled by (row / 2) % 8.  Row-major writes of eight
// chunks per row, reads of one chunk from 16 consecutive rows (MFMA operand
// rows), and ds_read_b64_tr_b8 reads of one chunk from 32 consecutive rows
// all spread evenly over the 64 LDS banks.
__device__ __forceinline__ uint32_t tile_off(int row, int chunk) {
  return (uint32_t)row * kHeadDim + 16u * (uint32_t)(chunk ^ ((row >> 1) & 7));
}

// ------------------------------------------------------- activation types --
// Two instantiations of one code path: fp16 and bf16 activations.
template <typename T>
struct Act;

template <>
struct Act<_Float16> {
  static constexpr int kId = 0;
  using x8 = f16x8;
  __device__ static float to_f32(uint16_t bits) {
    return (float)__builtin_bit_cast(_Float16, bits);
  }
  __device__ static uint16_t from_f32(float x) {
    return __builtin_bit_cast(uint16_t, (_Float16)x);
  }
  // four e4m3fn bytes -> four exact fp16 values (e4m3 is a subset of fp16)
  __device__ static void fp8x4_to(uint32_t w, x8& dst, int at) {
    f16x2 lo = __builtin_amdgcn_cvt_scalef32_pk_f16_fp8(w, 1.0f, false);
    f16x2 hi = __builtin_amdgcn_cvt_scalef32_pk_f16_fp8(w, 1.0f, true);
    dst[at + 0] = lo[0];
    dst[at + 1] = lo[1];
    dst[at + 2] = hi[0];
    dst[at + 3] = hi[1];
  }
  __device__ static f32x4 mfma(const x8& a, const x8& b, f32x4 c) {
    return __builtin_amdgcn_mfma_f32_16x16x32_f16(a, b, c, 0, 0, 0);
  }
};

template <>
struct Act<__bf16> {
  static constexpr int kId = 1;
  using x8 = bf16x8;
  __device__ static float to_f32(uint16_t bits) {
    return __builtin_bit_cast(float, (uint32_t)bits << 16);
  }
  __device__ static uint16_t from_f32(float x) {
    return __builtin_bit_cast(uint16_t, (__bf16)x);
  }
  // four e4m3fn bytes -> four exact bf16 values (e4m3 is a subset of bf16)
  __device__ static void fp8x4_to(uint32_t w, x8& dst, int at) {
    bf16x2 lo = __builtin_amdgcn_cvt_scalef32_pk_bf16_fp8(w, 1.0f, false);
    bf16x2 hi = __builtin_amdgcn_cvt_scalef32_pk_bf16_fp8(w, 1.0f, true);
    dst[at + 0] = lo[0];
    dst[at + 1] = lo[1];
    dst[at + 2] = hi[0];
    dst[at + 3] = hi[1];
  }
  __device__ static f32x4 mfma(const x8& a, const x8& b, f32x4 c) {
    return __builtin_amdgcn_mfma_f32_16x16x32_bf16(a, b, c, 0, 0, 0);
  }
};

// eight e4m3fn bytes (two dwords) -> eight exact bf16 values
__device__ __forceinline__ bf16x8 fp8x8_to_bf16(uint32_t w0, uint32_t w1) {
  bf16x8 r;
  Act<__bf16>::fp8x4_to(w0, r, 0);
  Act<__bf16>::fp8x4_to(w1, r, 4);
  return r;
}

// eight e4m3fn bytes (two dwords) -> eight exact fp16 values
__device__ __forceinline__ f16x8 fp8x8_to_f16(uint32_t w0, uint32_t w1) {
  f16x8 r;
  Act<_Float16>::fp8x4_to(w0, r, 0);
  Act<_Float16>::fp8x4_to(w1, r, 4);
  return r;
}

// largest power of two <= x, for a positive normal x
__device__ __forceinline__ float pow2_floor(float x) {
  return __uint_as_float(__float_as_uint(x) & 0xFF800000u);
}

// Four fp32 values -> four e4m3fn bytes (RNE, sign kept on zero).  The inputs
// must already lie in [-448, 448].
__device__ __forceinline__ uint32_t pack_fp8x4(float a, float b, float c,
                                               float d) {
  // the first convert keeps the high half of its old value and the second
  // overwrites it: passing a's bits as that old value, rather than 0, lets
  // the result take a's register without a move
  int w = __builtin_amdgcn_cvt_pk_fp8_f32(a, b, __float_as_int(a), false);
  w = __builtin_amdgcn_cvt_pk_fp8_f32(c, d, w, true);
  return (uint32_t)w;
}

// Split four values in [-448, 448] into e4m3 hi + lo parts: hi = e4m3(y),
// lo = e4m3(y - hi).  hi + lo carries about 8 significant bits, so an FP8
// MFMA over both parts keeps the contraction accurate to about 2^-8.
__device__ __forceinline__ void split_fp8x4(float a, float b, float c, float d,
                                            uint32_t& hi, uint32_t& lo) {
  hi = pack_fp8x4(a, b, c, d);
  typedef float f32x2 __attribute__((ext_vector_type(2)));
  const f32x2 h01 = __builtin_amdgcn_cvt_pk_f32_fp8((int)hi, false);
  const f32x2 h23 = __builtin_amdgcn_cvt_pk_f32_fp8((int)hi, true);
  lo = pack_fp8x4(a - h01[0], b - h01[1], c - h23[0], d - h23[1]);
}

// Three-part split: hi + mid + lo carries about 12 significant bits.
__device__ __forceinline__ void split3_fp8x4(float a, float b, float c, float d,
                                             uint32_t& hi, uint32_t& mid, uint32_t& lo) {
  typedef float f32x2 __attribute__((ext_vector_type(2)));
  hi = pack_fp8x4(a, b, c, d);
  const f32x2 h01 = __builtin_amdgcn_cvt_pk_f32_fp8((int)hi, false);
  const f32x2 h23 = __builtin_amdgcn_cvt_pk_f32_fp8((int)hi, true);
  a -= h01[0]; b -= h01[1]; c -= h23[0]; d -= h23[1];
  split_fp8x4(a, b, c, d, mid, lo);
}

__device__ __forceinline__ float exp2_fast(float x) {
  return __builtin_amdgcn_exp2f(x);
}

__device__ __forceinline__ float wave_max_xor(float v, int mask) {
  return fmaxf(v, __shfl_xor(v, mask));
}

// Cross-row exchanges without an LDS round trip.  v_permlane16_swap(x, x)
// returns {x[l], x[l^16]} in some order on every lane, v_permlane32_swap the
// same for l^32, so the pair's max (or sum) is the xor-16 / xor-32 reduction.
__device__ __forceinline__ float max_xor16(float v) {
  const auto r = __builtin_amdgcn_permlane16_swap(__float_as_uint(v), __float_as_uint(v),
                                                  false, false);
  return fmaxf(__uint_as_float(r[0]), __uint_as_float(r[1]));
}
__device__ __forceinline__ float max_xor32(float v) {
  const auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(v), __float_as_uint(v),
                                                  false, false);
  return fmaxf(__uint_as_float(r[0]), __uint_as_float(r[1]));
}
// max over each row of 16 lanes with DPP (no LDS round trip): quad_perm
// [1,0,3,2] and [2,3,0,1] reduce each quad, row_half_mirror pairs lane i
// with 7-i (the other quad of its half-row), row_mirror lane i with 15-i
// (the other half-row)
__device__ __forceinline__ float max16_dpp(float v) {
  int x = __float_as_int(v);
  v = fmaxf(v, __int_as_float(__builtin_amdgcn_update_dpp(x, x, 0xB1, 0xF, 0xF, false)));
  x = __float_as_int(v);
  v = fmaxf(v, __int_as_float(__builtin_amdgcn_update_dpp(x, x, 0x4E, 0xF, 0xF, false)));
  x = __float_as_int(v);
  v = fmaxf(v, __int_as_float(__builtin_amdgcn_update_dpp(x, x, 0x141, 0xF, 0xF, false)));
  x = __float_as_int(v);
  v = fmaxf(v, __int_as_float(__builtin_amdgcn_update_dpp(x, x, 0x140, 0xF, 0xF, false)));
  return v;
}

__device__ __forceinline__ float sum_xor16(float v) {
  const auto r = __builtin_amdgcn_permlane16_swap(__float_as_uint(v), __float_as_uint(v),
                                                  false, false);
  return __uint_as_float(r[0]) + __uint_as_float(r[1]);
}
__device__ __forceinline__ float sum_xor32(float v) {
  const auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(v), __float_as_uint(v),
                                                  false, false);
  return __uint_as_float(r[0]) + __uint_as_float(r[1]);
}

// The running max may lag the true max by up to this many log2 units before
// the accumulator is rescaled: exp2(x - m) then stays below 2^8.
constexpr float kRescaleSlack = 8.0f;

}  // namespace mskv
