// Fused attention prologue: per-head RMSNorm of q and k, rotary embedding,
// and the FP8 store of k and v, in one pass over the qkv projection output.
//
// Replaces microserve/models/qwen3.py:49-53 followed by the store at the top
// of Attention.forward (microserve/layers/attention.py:41-43):
//   q = q_norm(q); k = k_norm(k); q, k = rotary_emb(positions, q, k)
//   store_fp8_kvcache(k, v, ...)
// The unfused chain reads and writes q and k several times in fp32 and
// 16-bit temporaries; here each q/k/v row is read once, q (and, for the fresh
// prefill that attends over the unquantized keys, k) is written once, and k
// and v go to the cache as FP8 in the same pass.
//
// Arithmetic, every step rounded as the reference's torch ops round it (the
// runner casts the model, norm weights and rotary tables included, to the
// activation type: microserve/engine/model_runner.py:58-59):
//   RMSNorm (microserve/layers/layernorm.py:55-57, 80-81):
//     var = sum(x^2) / 128 in fp32; r = 1 / sqrt(var + eps), both IEEE fp32;
//     n = T(x * r); y = T(n * w).
//   The sum order is fixed: lane l of the row's 8 lanes sums its 16 squares
//   in order, then ((s0+s1)+(s2+s3)) + ((s4+s5)+(s6+s7)).  (torch does not
//   specify its reduction order or its rsqrt rounding; this order and the
//   correctly rounded 1/sqrt are the definition the results are exact to.)
//   Rotary (microserve/layers/rotary_embedding.py:4-7, 24-31), for d < 64:
//     out[d]      = T(T(y[d] * cos[d])           + T(-y[d+64] * sin[d]))
//     out[d + 64] = T(T(y[d+64] * cos[d+64])     + T(y[d] * sin[d+64]))
//   with each sum taken in fp32 first, as torch's 16-bit add does.
//   Store: the bytes and scales of store_fp8_kvcache on the rotated k and on
//   v (microserve/layers/fp8_kv_cache.py:11-39).
//
// Work layout: eight lanes own a chunk of up to four rows of one kind (q, k
// or v heads) of one token; lane l holds elements [8l, 8l+8) and
// [64+8l, 64+8l+8) of each, so rotate_half's pairs (d, d+64) meet in one
// lane and the only cross-lane traffic is the two DPP reductions.  The
// token's rotary rows and the norm weights are unpacked once per chunk, not
// once per row (the kernel is bound by VALU issue, not by HBM).  The grid
// lists every token's q chunks, then the k chunks, then the v chunks, so a
// wave's groups take the same path.
#include <math.h>

#include "fp8_row.h"
#include "mskv_device.h"
#include "../../include/mskv.h"

namespace mskv {

constexpr int kNrThreads = 256;
constexpr int kNrGroups = kNrThreads / 8;  // 8-lane groups per workgroup
constexpr int kNrChunk = 4;                // rows per group: heads of one kind, one token

struct NormRopeArgs {
  const uint16_t* q;
  const uint16_t* k;
  const uint16_t* v;
  int64_t q_stride, k_stride, v_stride;  // elements between tokens
  const int64_t* positions;
  const uint16_t* q_weight;  // NULL: no norm (rotary only)
  const uint16_t* k_weight;
  const uint16_t* cos;  // [max_position, 128]
  const uint16_t* sin;
  uint16_t* q_out;  // [tokens, hq, 128]
  uint16_t* k_out;  // [tokens, hk, 128] or NULL
  uint8_t* k_cache;
  uint8_t* v_cache;
  float* k_scale;
  float* v_scale;
  const void* slots;
  int64_t rows, num_slots, max_position;
  int hq, hk, heads;
  float eps;
  int cq, ck;               // chunks per token of q heads, of k (and v) heads
  int64_t q_chunks, k_chunks, chunks;  // over all tokens: q, k (= v), all
};

// Sum over the 8 lanes of a row group: xor 1, xor 2, then the mirrored
// lane of the other quad.  Addition is commutative, so every lane ends with
// the same bits: ((s0+s1)+(s2+s3)) + ((s4+s5)+(s6+s7)).
__device__ __forceinline__ float sum8_dpp(float v) {
  int x = __float_as_int(v);
  v = v + __int_as_float(__builtin_amdgcn_update_dpp(x, x, 0xB1, 0xF, 0xF, false));
  x = __float_as_int(v);
  v = v + __int_as_float(__builtin_amdgcn_update_dpp(x, x, 0x4E, 0xF, 0xF, false));
  x = __float_as_int(v);
  v = v + __int_as_float(__builtin_amdgcn_update_dpp(x, x, 0x141, 0xF, 0xF, false));
  return v;
}

template <typename T>
__device__ __forceinline__ float rnd(float x) {
  return (float)(T)x;
}

// bf16: v_cvt_pk_bf16_f32 with x in the high half and zero in the low half
// leaves a word that is the rounded value read as fp32, so the round trip
// is one instruction (the plain cast converts and then shifts left by 16).
// Same instruction, same rounding.
template <>
__device__ __forceinline__ float rnd<__bf16>(float x) {
  typedef float f32x2 __attribute__((ext_vector_type(2)));
  return __builtin_bit_cast(float, __builtin_convertvector(f32x2{0.0f, x}, bf16x2));
}

// T(x) of a value that must first be rounded to fp32, as torch rounds x * r
// before casting.  For fp16 the backend would otherwise fold the multiply
// and the cast into one v_fma_mixlo_f16, which rounds once, and that differs
// where the fp32 product lies on an fp16 tie.  (Products of two 16-bit
// values are exact in fp32 and sums of two fp16 values round innocuously
// twice, so only this product needs it.)
template <typename T>
__device__ __forceinline__ float rnd_f32(float x) {
  asm volatile("" : "+v"(x));
  return rnd<T>(x);
}

template <typename T>
__device__ __forceinline__ void unpack8(const u32x4& a, float* x) {
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    x[2 * i] = Act<T>::to_f32((uint16_t)(a[i] & 0xFFFFu));
    x[2 * i + 1] = Act<T>::to_f32((uint16_t)(a[i] >> 16));
  }
}

template <typename T>
__device__ __forceinline__ u32x4 pack8(const float* x) {
  u32x4 r;
#pragma unroll
  for (int i = 0; i < 4; ++i)
    r[i] = (uint32_t)Act<T>::from_f32(x[2 * i]) | ((uint32_t)Act<T>::from_f32(x[2 * i + 1]) << 16);
  return r;
}

// RMSNorm (when w is given) and rotary of one q or k row in place: x holds
// its 16 elements (lane layout above); wv, c, s are the lane's norm weights
// and its token's cos/sin values; a row whose position is out of range
// becomes zeros.
template <typename T>
__device__ __forceinline__ void norm_rope_row(const NormRopeArgs& a, bool has_w, bool pos_ok,
                                              const float* wv, const float* c, const float* s,
                                              float* x) {
#pragma clang fp contract(off)
  if (has_w) {
    // each square is exact in fp32, so the fused multiply-add rounds the
    // running sum exactly as a multiply and an add would
    float ss = 0.0f;
#pragma unroll
    for (int i = 0; i < 16; ++i) ss = fmaf(x[i], x[i], ss);
    const float var = sum8_dpp(ss) / (float)kHeadDim;
    const float r = 1.0f / sqrtf(var + a.eps);
#pragma unroll
    for (int i = 0; i < 16; ++i) x[i] = rnd<T>(rnd_f32<T>(x[i] * r) * wv[i]);
  }
  float o[16];
#pragma unroll
  for (int i = 0; i < 8; ++i) {
    o[i] = rnd<T>(rnd<T>(x[i] * c[i]) + (-rnd<T>(x[8 + i] * s[i])));
    o[8 + i] = rnd<T>(rnd<T>(x[8 + i] * c[8 + i]) + rnd<T>(x[i] * s[8 + i]));
  }
#pragma unroll
  for (int i = 0; i < 16; ++i) x[i] = pos_ok ? o[i] : 0.0f;
}

// The FP8 row and scale of a k (rotated) or v row, at cache row `dst`.
__device__ __forceinline__ void store_fp8_row(const NormRopeArgs& a, bool is_v, int64_t dst,
                                              int sub, const float* x) {
  const int lo = 8 * sub, hi = kHeadDim / 2 + 8 * sub;
  u32x4 qb;
  const float scale = quantize16(x, qb);
  uint8_t* cache = is_v ? a.v_cache : a.k_cache;
  __builtin_nontemporal_store(u32x2{qb[0], qb[1]},
                              reinterpret_cast<u32x2*>(cache + dst * kHeadDim + lo));
  __builtin_nontemporal_store(u32x2{qb[2], qb[3]},
                              reinterpret_cast<u32x2*>(cache + dst * kHeadDim + hi));
  if (sub == 0) (is_v ? a.v_scale : a.k_scale)[dst] = scale;
}

// Bit casts between a 32-bit word and an fp16 pair, through a scalar copy:
// clang lowers __builtin_bit_cast applied directly to an element of an
// ext_vector_type value (v[i]) to element 0 for every index.
__device__ __forceinline__ f16x2 as_f16x2(uint32_t w) { return __builtin_bit_cast(f16x2, w); }
__device__ __forceinline__ uint32_t as_u32(f16x2 h) { return __builtin_bit_cast(uint32_t, h); }

// The fp16 form of norm_rope_row on packed pairs: xl / xh hold the lane's
// 16 elements as fp16 pairs and come back holding the result.  Products of
// two fp16 values are exact in fp32, and the sum of two fp16 values rounds
// to the same fp16 whether or not it is first rounded to fp32 (when the
// fp32 sum is inexact the smaller term is below an eighth of an fp16 ulp),
// so v_pk_mul_f16 / v_pk_add_f16, which round once, give torch's
// T(T(.) op T(.)) bit for bit with no round trip through fp32.  Only x * r
// (r in fp32) is taken in fp32.
__device__ __forceinline__ void norm_rope_row_f16(const NormRopeArgs& a, bool has_w,
                                                  bool pos_ok, const f16x2* w2,
                                                  const f16x2* c2, const f16x2* s2,
                                                  u32x4& xl, u32x4& xh) {
#pragma clang fp contract(off)
  f16x2 y[8];
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    y[i] = as_f16x2(xl[i]);
    y[4 + i] = as_f16x2(xh[i]);
  }
  if (has_w) {
    float x[16];
#pragma unroll
    for (int i = 0; i < 8; ++i) {
      x[2 * i] = (float)y[i][0];
      x[2 * i + 1] = (float)y[i][1];
    }
    float ss = 0.0f;
#pragma unroll
    for (int i = 0; i < 16; ++i) ss = fmaf(x[i], x[i], ss);
    const float var = sum8_dpp(ss) / (float)kHeadDim;
    const float r = 1.0f / sqrtf(var + a.eps);
#pragma unroll
    for (int i = 0; i < 8; ++i) {
      float p0 = x[2 * i] * r, p1 = x[2 * i + 1] * r;
      asm volatile("" : "+v"(p0), "+v"(p1));  // round x * r to fp32 first
      y[i] = f16x2{(_Float16)p0, (_Float16)p1} * w2[i];
    }
  }
  // lanes' pairs 0-3 are d in [8l, 8l+8), pairs 4-7 are d + 64
  f16x2 o[8];
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const f16x2 a0 = y[i] * c2[i];
    const f16x2 b0 = y[4 + i] * s2[i];
    o[i] = a0 - b0;
    const f16x2 a1 = y[4 + i] * c2[4 + i];
    const f16x2 b1 = y[i] * s2[4 + i];
    o[4 + i] = a1 + b1;
  }
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    xl[i] = pos_ok ? as_u32(o[i]) : 0u;
    xh[i] = pos_ok ? as_u32(o[4 + i]) : 0u;
  }
}

// Each 8-lane group owns one chunk: up to kNrChunk consecutive heads of one
// kind of one token.  It issues the loads of all its rows first, then
// unpacks the token's rotary values and the norm weights once for them.
template <typename T, typename SlotT>
__global__ __launch_bounds__(kNrThreads) void qk_norm_rope_store_kernel(NormRopeArgs a) {
  const int sub = threadIdx.x & 7;
  const int64_t chunk = (int64_t)blockIdx.x * kNrGroups + (threadIdx.x >> 3);
  if (chunk >= a.chunks) return;  // whole 8-lane groups leave together
  const int lo = 8 * sub, hi = kHeadDim / 2 + 8 * sub;
  // kind 0: q heads, 1: k heads, 2: v heads; chunks < 2^31 (rows are,
  // checked on the host): 32-bit division
  int kind, per;
  uint32_t c32;
  if (chunk < a.q_chunks) {
    kind = 0, per = a.cq, c32 = (uint32_t)chunk;
  } else if (chunk < a.q_chunks + a.k_chunks) {
    kind = 1, per = a.ck, c32 = (uint32_t)(chunk - a.q_chunks);
  } else {
    kind = 2, per = a.ck, c32 = (uint32_t)(chunk - a.q_chunks - a.k_chunks);
  }
  const uint32_t t32 = c32 / (uint32_t)per;
  const int64_t tok = t32;
  const int h0 = (int)(c32 - t32 * (uint32_t)per) * kNrChunk;
  const int nheads = kind == 0 ? a.hq : a.hk;
  const int n = min(kNrChunk, nheads - h0);
  const uint16_t* src = kind == 0   ? a.q + tok * a.q_stride
                        : kind == 1 ? a.k + tok * a.k_stride
                                    : a.v + tok * a.v_stride;
  src += (int64_t)h0 * kHeadDim;
  u32x4 xl[kNrChunk], xh[kNrChunk];
#pragma unroll
  for (int r = 0; r < kNrChunk; ++r) {
    if (r < n) {
      xl[r] = __builtin_nontemporal_load(reinterpret_cast<const u32x4*>(src + r * kHeadDim + lo));
      xh[r] = __builtin_nontemporal_load(reinterpret_cast<const u32x4*>(src + r * kHeadDim + hi));
    }
  }
  const int64_t pos = a.positions[tok];
  const int64_t slot = kind == 0 ? 0 : (int64_t) static_cast<const SlotT*>(a.slots)[tok];
  const bool pos_ok = pos >= 0 && pos < a.max_position;
  // the cache takes k and v rows only at valid positions and slots
  const bool to_cache = kind != 0 && pos_ok && slot >= 0 && slot < a.num_slots;
  float x[16];
  if constexpr (__is_same(T, _Float16)) {
    if (kind != 2) {
      const uint16_t* w = kind == 0 ? a.q_weight : a.k_weight;
      const bool has_w = w != nullptr;
      // the norm weights and the token's rotary values stay packed
      f16x2 w2[8], c2[8], s2[8];
      const int64_t tab = (pos_ok ? pos : 0) * kHeadDim;
      const u32x4 cl = *reinterpret_cast<const u32x4*>(a.cos + tab + lo);
      const u32x4 ch = *reinterpret_cast<const u32x4*>(a.cos + tab + hi);
      const u32x4 sl = *reinterpret_cast<const u32x4*>(a.sin + tab + lo);
      const u32x4 sh = *reinterpret_cast<const u32x4*>(a.sin + tab + hi);
      u32x4 wl = {0u, 0u, 0u, 0u}, wh = {0u, 0u, 0u, 0u};
      if (has_w) {
        wl = *reinterpret_cast<const u32x4*>(w + lo);
        wh = *reinterpret_cast<const u32x4*>(w + hi);
      }
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        c2[i] = as_f16x2(cl[i]);
        c2[4 + i] = as_f16x2(ch[i]);
        s2[i] = as_f16x2(sl[i]);
        s2[4 + i] = as_f16x2(sh[i]);
        w2[i] = as_f16x2(wl[i]);
        w2[4 + i] = as_f16x2(wh[i]);
      }
#pragma unroll
      for (int r = 0; r < kNrChunk; ++r) {
        if (r >= n) break;
        u32x4 ol = xl[r], oh = xh[r];
        norm_rope_row_f16(a, has_w, pos_ok, w2, c2, s2, ol, oh);
        uint16_t* dst = kind == 0
                            ? a.q_out + (tok * a.hq + h0 + r) * kHeadDim
                            : (a.k_out ? a.k_out + (tok * a.hk + h0 + r) * kHeadDim : nullptr);
        if (dst) {
          __builtin_nontemporal_store(ol, reinterpret_cast<u32x4*>(dst + lo));
          __builtin_nontemporal_store(oh, reinterpret_cast<u32x4*>(dst + hi));
        }
        if (to_cache) {
          unpack8<T>(ol, x);
          unpack8<T>(oh, x + 8);
          store_fp8_row(a, false, slot * a.hk + h0 + r, sub, x);
        }
      }
    } else if (to_cache) {
#pragma unroll
      for (int r = 0; r < kNrChunk; ++r) {
        if (r >= n) break;
        unpack8<T>(xl[r], x);
        unpack8<T>(xh[r], x + 8);
        store_fp8_row(a, true, slot * a.hk + h0 + r, sub, x);
      }
    }
    return;
  }
  if (kind != 2) {
    const uint16_t* w = kind == 0 ? a.q_weight : a.k_weight;
    const bool has_w = w != nullptr;
    float wv[16], c[16], s[16];
    if (has_w) {
      unpack8<T>(*reinterpret_cast<const u32x4*>(w + lo), wv);
      unpack8<T>(*reinterpret_cast<const u32x4*>(w + hi), wv + 8);
    }
    const int64_t tab = (pos_ok ? pos : 0) * kHeadDim;
    unpack8<T>(*reinterpret_cast<const u32x4*>(a.cos + tab + lo), c);
    unpack8<T>(*reinterpret_cast<const u32x4*>(a.cos + tab + hi), c + 8);
    unpack8<T>(*reinterpret_cast<const u32x4*>(a.sin + tab + lo), s);
    unpack8<T>(*reinterpret_cast<const u32x4*>(a.sin + tab + hi), s + 8);
#pragma unroll
    for (int r = 0; r < kNrChunk; ++r) {
      if (r >= n) break;
      unpack8<T>(xl[r], x);
      unpack8<T>(xh[r], x + 8);
      norm_rope_row<T>(a, has_w, pos_ok, wv, c, s, x);
      uint16_t* dst = kind == 0 ? a.q_out + (tok * a.hq + h0 + r) * kHeadDim
                                : (a.k_out ? a.k_out + (tok * a.hk + h0 + r) * kHeadDim : nullptr);
      if (dst) {
        __builtin_nontemporal_store(pack8<T>(x), reinterpret_cast<u32x4*>(dst + lo));
        __builtin_nontemporal_store(pack8<T>(x + 8), reinterpret_cast<u32x4*>(dst + hi));
      }
      if (to_cache) store_fp8_row(a, false, slot * a.hk + h0 + r, sub, x);
    }
  } else if (to_cache) {
#pragma unroll
    for (int r = 0; r < kNrChunk; ++r) {
      if (r >= n) break;
      unpack8<T>(xl[r], x);
      unpack8<T>(xh[r], x + 8);
      store_fp8_row(a, true, slot * a.hk + h0 + r, sub, x);
    }
  }
}

template <typename T>
static hipError_t launch_norm_rope(const NormRopeArgs& a, int slot_dtype, hipStream_t stream) {
  const int64_t blocks = (a.chunks + kNrGroups - 1) / kNrGroups;
  if (slot_dtype == MSKV_INT64)
    hipLaunchKernelGGL((qk_norm_rope_store_kernel<T, int64_t>), dim3((unsigned)blocks),
                       dim3(kNrThreads), 0, stream, a);
  else
    hipLaunchKernelGGL((qk_norm_rope_store_kernel<T, int32_t>), dim3((unsigned)blocks),
                       dim3(kNrThreads), 0, stream, a);
  return hipGetLastError();
}

}  // namespace mskv

extern "C" int mskv_qk_norm_rope_store(
    const void* q, const void* k, const void* v, int64_t q_token_stride,
    int64_t k_token_stride, int64_t v_token_stride, const int64_t* positions,
    const void* q_norm_weight, const void* k_norm_weight, float eps, const void* cos_cache,
    const void* sin_cache, int64_t max_position, void* q_out, void* k_out, void* k_cache,
    void* v_cache, float* k_scale_cache, float* v_scale_cache, const void* slot_mapping,
    int slot_dtype, int64_t num_tokens, int num_q_heads, int num_kv_heads, int head_dim,
    int64_t num_slots, int act_dtype, void* stream) {
  if (num_tokens < 0 || num_q_heads <= 0 || num_kv_heads <= 0 || num_slots < 0 ||
      max_position <= 0)
    return MSKV_EINVAL;
  if (slot_dtype != MSKV_INT32 && slot_dtype != MSKV_INT64) return MSKV_EINVAL;
  if (act_dtype != MSKV_FLOAT16 && act_dtype != MSKV_BFLOAT16) return MSKV_EINVAL;
  if (head_dim != mskv::kHeadDim) return MSKV_EUNSUPPORTED;
  if ((q_norm_weight == nullptr) != (k_norm_weight == nullptr)) return MSKV_EINVAL;
  if (!(eps >= 0.0f)) return MSKV_EINVAL;
  if (num_tokens == 0) return MSKV_OK;
  if (!q || !k || !v || !positions || !cos_cache || !sin_cache || !q_out || !k_cache ||
      !v_cache || !k_scale_cache || !v_scale_cache || !slot_mapping)
    return MSKV_EINVAL;
  if (q_token_stride < (int64_t)num_q_heads * head_dim ||
      k_token_stride < (int64_t)num_kv_heads * head_dim ||
      v_token_stride < (int64_t)num_kv_heads * head_dim)
    return MSKV_EINVAL;
  // 16-byte loads and stores: every row must start 16-byte aligned
  auto misaligned = [](const void* p) { return ((uintptr_t)p & 15u) != 0; };
  if (misaligned(q) || misaligned(k) || misaligned(v) || misaligned(q_out) ||
      (k_out && misaligned(k_out)) || misaligned(cos_cache) || misaligned(sin_cache) ||
      (q_norm_weight && (misaligned(q_norm_weight) || misaligned(k_norm_weight))) ||
      (q_token_stride | k_token_stride | v_token_stride) % 8 != 0)
    return MSKV_EINVAL;
  const int heads = num_q_heads + 2 * num_kv_heads;
  const int64_t rows = num_tokens * heads;
  if (rows > 0x7FFFFFFFLL) return MSKV_EUNSUPPORTED;
  mskv::NormRopeArgs a{(const uint16_t*)q, (const uint16_t*)k, (const uint16_t*)v,
                       q_token_stride, k_token_stride, v_token_stride, positions,
                       (const uint16_t*)q_norm_weight, (const uint16_t*)k_norm_weight,
                       (const uint16_t*)cos_cache, (const uint16_t*)sin_cache,
                       (uint16_t*)q_out, (uint16_t*)k_out, (uint8_t*)k_cache,
                       (uint8_t*)v_cache, k_scale_cache, v_scale_cache, slot_mapping, rows,
                       num_slots, max_position, num_q_heads, num_kv_heads, heads, eps};
  a.cq = (num_q_heads + mskv::kNrChunk - 1) / mskv::kNrChunk;
  a.ck = (num_kv_heads + mskv::kNrChunk - 1) / mskv::kNrChunk;
  a.q_chunks = num_tokens * a.cq;
  a.k_chunks = num_tokens * a.ck;
  a.chunks = a.q_chunks + 2 * a.k_chunks;
  hipStream_t s = reinterpret_cast<hipStream_t>(stream);
  const hipError_t e = act_dtype == MSKV_BFLOAT16 ? mskv::launch_norm_rope<__bf16>(a, slot_dtype, s)
                                                   : mskv::launch_norm_rope<_Float16>(a, slot_dtype, s);
  return (int)e;
}
