// Varlen causal prefill over the FP8 e4m3fn paged cache with FP8 MFMA.
//
// Semantics follow microserve/layers/fp8_chunk_prefill_attention.py:16-67,
// generalized to a varlen batch: query i of a sequence with Lq new tokens
// and Lk cached tokens (new ones included) sees positions
// p < (Lk - Lq) + i + 1 (:52-54); K/V row p lives at
// block_tables[s][p / BS] * BS + p % BS.
//
// MI355X design:
//  * A workgroup is four waves.  Each wave owns 16 rows; a row is one
//    (query token, q head) pair and the GQA group of one kv head fills the
//    rows, so one K/V tile serves every q head that reads it.  The four
//    waves share 128-token K/V tiles staged in LDS.
//  * QK^T: S^T = K . Q8^T with v_mfma_f32_16x16x128_f8f6f4 -- the whole
//    head_dim is one MFMA.  K bytes are used as stored; the query row is
//    quantized in-kernel with a per-row scale into e4m3 hi + mid + lo parts
//    (q ~ hi + mid + lo to about 2^-12, so a 20x K outlier does not turn
//    the query's rounding into visible score error), one MFMA each into the
//    same accumulator, and score = acc * q_scale * k_scale * softmax_scale.
//  * PV: O^T = V^T . P8^T with the same MFMA.  S^T's accumulator leaves lane
//    (g, n) holding 32 tokens of row n, exactly the B-operand layout of P^T,
//    so the probabilities never move between lanes.  P * v_scale is
//    quantized to e4m3 hi + lo parts with a per-row, per-step scale (two
//    MFMAs per d tile); the accumulator is
//    kept in units of the latest scale, so the rescale folds into the
//    online-softmax alpha multiply.  V^T comes out of LDS transposed with
//    ds_read_b64_tr_b8.
//  * Pages are read through page-sized buffer resources; an invalid block
//    id gives zero-length reads and its tokens are masked.
#include <math.h>

#include "mskv_device.h"
#include "../../include/mskv.h"

namespace mskv {

constexpr int kPStep = 128;   // tokens per K/V tile
constexpr int kPWaves = 4;
constexpr int kPThreads = 64 * kPWaves;

struct PrefillArgs {
  const uint16_t* q;
  const uint8_t* kc;
  const uint8_t* vc;
  const float* ks;
  const float* vs;
  const int32_t* bt;
  const int32_t* cu_q;
  const int32_t* cu_k;
  uint16_t* out;
  int64_t total_q;
  int64_t num_blocks;
  int prefix_len;
  int hq, hk, group, gc, qgroups, tpr, bs, w;
  float scale_log2;
};

__device__ __forceinline__ f32x4 mfma_fp8(const i32x8& a, const i32x8& b, f32x4 c) {
  // scale operands 0 select the unscaled v_mfma_f32_16x16x128_f8f6f4
  return __builtin_amdgcn_mfma_scale_f32_16x16x128_f8f6f4(a, b, c, 0, 0, 0, 0, 0, 0);
}

template <typename T>
__global__ __launch_bounds__(kPThreads) void prefill_fp8_kernel(PrefillArgs a) {
  using A = Act<T>;
  __shared__ __attribute__((aligned(16))) uint8_t k_lds[kPStep * kHeadDim];
  __shared__ __attribute__((aligned(16))) uint8_t v_lds[kPStep * kHeadDim];
  __shared__ __attribute__((aligned(16))) float ks_lds[kPStep];
  __shared__ __attribute__((aligned(16))) float vs_lds[kPStep];

  const int tid = threadIdx.x;
  const int wave = tid >> 6, lane = tid & 63;
  const int g = lane >> 4, n = lane & 15;
  const int s = blockIdx.z;
  const int unit = blockIdx.y;
  const int kvh = unit / a.qgroups;
  const int qgi = unit - kvh * a.qgroups;

  // query rows are clamped to [0, total_q) and positions to the table width,
  // so inconsistent cu_seqlens cannot address memory outside the tensors
  const int64_t tq = a.total_q;
  const int q_begin = a.cu_q ? (int)min((int64_t)max(a.cu_q[s], 0), tq) : 0;
  const int q_end = a.cu_q ? (int)min((int64_t)max(a.cu_q[s + 1], q_begin), tq) : (int)tq;
  const int lq = q_end - q_begin;
  const int lk = a.cu_k ? a.cu_k[s + 1] - a.cu_k[s] : a.prefix_len + lq;
  const int prefix = lk - lq;
  const int wg_q0 = blockIdx.x * kPWaves * a.tpr;
  if (wg_q0 >= lq || lq <= 0) return;
  const int wg_qlast = min(lq, wg_q0 + kPWaves * a.tpr) - 1;
  const int kv_end = min(min(lk, prefix + wg_qlast + 1), a.w * a.bs);

  // this lane's row: query token wg_q0 + wave*tpr + n/gc, head n%gc of the group
  const int qi = wg_q0 + wave * a.tpr + n / a.gc;
  const int hh = n % a.gc;
  const bool row_ok = n < a.tpr * a.gc && qi < lq;
  const int qh = kvh * a.group + qgi * 16 + hh;
  const int lim = row_ok ? prefix + qi + 1 : 0;

  // quantize the query row (hi + mid + lo e4m3 parts, one per-row scale):
  // lane (g, n) holds d in [32g, 32g+32)
  i32x8 q8h, q8m, q8l;
  float qscale;
  {
    float x[32];
    if (row_ok) {
      const u32x4* qp = reinterpret_cast<const u32x4*>(
          a.q + ((int64_t)(q_begin + qi) * a.hq + qh) * kHeadDim + 32 * g);
#pragma unroll
      for (int c = 0; c < 4; ++c) {
        const u32x4 v = qp[c];
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          x[8 * c + 2 * i] = A::to_f32((uint16_t)(v[i] & 0xFFFFu));
          x[8 * c + 2 * i + 1] = A::to_f32((uint16_t)(v[i] >> 16));
        }
      }
    } else {
#pragma unroll
      for (int i = 0; i < 32; ++i) x[i] = 0.0f;
    }
    float amax = 0.0f;
#pragma unroll
    for (int i = 0; i < 32; ++i) amax = fmaxf(amax, fabsf(x[i]));
    amax = max_xor32(max_xor16(amax));
    amax = fmaxf(amax, 1e-8f);
    const float inv = kFp8Max / amax;
#pragma unroll
    for (int c = 0; c < 8; ++c) {
      float y[4];
#pragma unroll
      for (int i = 0; i < 4; ++i) y[i] = fminf(fmaxf(x[4 * c + i] * inv, -kFp8Max), kFp8Max);
      uint32_t h, mi, lo;
      split3_fp8x4(y[0], y[1], y[2], y[3], h, mi, lo);
      q8h[c] = (int)h;
      q8m[c] = (int)mi;
      q8l[c] = (int)lo;
    }
    qscale = amax / kFp8Max * a.scale_log2;
  }

  f32x4 acc[8];
#pragma unroll
  for (int dt = 0; dt < 8; ++dt) acc[dt] = f32x4{0.f, 0.f, 0.f, 0.f};
  float m = -INFINITY, l = 0.0f, cs = 1.0f;

  // ds_read_b64_tr_b8 address of this lane for read q (tokens 8q..8q+7 of
  // the lane group's 32): token slot e = 8q + i/2 maps to step row
  // 16*(e/4) + 4g + e%4, column half i%2.
  const int i16 = lane & 15;
  uint32_t tr_addr[4];
#pragma unroll
  for (int qq = 0; qq < 4; ++qq) {
    const int e = 8 * qq + (i16 >> 1);
    const int row = 16 * (e >> 2) + 4 * g + (e & 3);
    tr_addr[qq] = (uint32_t)row * kHeadDim + 8u * (i16 & 1);
  }

  const uint32_t page_bytes = (uint32_t)a.bs * a.hk * kHeadDim;
  const uint32_t spage_bytes = (uint32_t)a.bs * a.hk * 4u;
  const uint32_t rstride = (uint32_t)a.hk * kHeadDim;

  for (int t0 = 0; t0 < kv_end; t0 += kPStep) {
    const int page = t0 / a.bs;
    const int off = t0 - page * a.bs;
    const int blk = a.bt[(int64_t)s * a.w + page];
    const bool ok = blk >= 0 && (int64_t)blk < a.num_blocks;
    const int64_t bo = ok ? blk : 0;
    const auto kr = make_rsrc(a.kc + bo * page_bytes, ok ? page_bytes : 0u);
    const auto vr = make_rsrc(a.vc + bo * page_bytes, ok ? page_bytes : 0u);
    const auto ksr = make_rsrc(a.ks + bo * a.bs * a.hk, ok ? spage_bytes : 0u);
    const auto vsr = make_rsrc(a.vs + bo * a.bs * a.hk, ok ? spage_bytes : 0u);
    const int valid = ok ? min(kPStep, lk - t0) : 0;  // rows holding real tokens

    // cooperative tile load: 1024 16-byte chunks of K and of V
    u32x4 kv[4], vv[4];
    const uint32_t base = (uint32_t)off * rstride + (uint32_t)kvh * kHeadDim;
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const int c = tid + kPThreads * j;
      const uint32_t o = base + (uint32_t)(c >> 3) * rstride + 16u * (c & 7);
      kv[j] = buf_load16(kr, o);
      vv[j] = buf_load16(vr, o);
    }
    const uint32_t so = (((uint32_t)off + (tid & (kPStep - 1))) * a.hk + kvh) * 4u;
    const float sc = tid < kPStep ? buf_load_f32(ksr, so) : buf_load_f32(vsr, so);
    __syncthreads();  // the previous tile is no longer read
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const int c = tid + kPThreads * j;
      const int row = c >> 3;
      *reinterpret_cast<u32x4*>(k_lds + row * kHeadDim + 16 * (c & 7)) = kv[j];
      *reinterpret_cast<u32x4*>(v_lds + row * kHeadDim + 16 * (c & 7)) =
          row < valid ? vv[j] : u32x4{0u, 0u, 0u, 0u};
    }
    if (tid < kPStep) ks_lds[tid] = sc;
    else vs_lds[tid - kPStep] = sc;
    __syncthreads();

    // S^T = K . Q8^T, eight 16-token tiles
    f32x4 st[8];
#pragma unroll
    for (int tt = 0; tt < 8; ++tt) {
      const uint8_t* kp = k_lds + (16 * tt + n) * kHeadDim + 32 * g;
      const u32x4 lo = *reinterpret_cast<const u32x4*>(kp);
      const u32x4 hi = *reinterpret_cast<const u32x4*>(kp + 16);
      const i32x8 ka = {(int)lo[0], (int)lo[1], (int)lo[2], (int)lo[3],
                        (int)hi[0], (int)hi[1], (int)hi[2], (int)hi[3]};
      st[tt] = mfma_fp8(ka, q8h, f32x4{0.f, 0.f, 0.f, 0.f});
      st[tt] = mfma_fp8(ka, q8m, st[tt]);
      st[tt] = mfma_fp8(ka, q8l, st[tt]);
    }
    // lane (g, n) now holds tokens 16*tt + 4g + r of row n
    float x[32];
    float tmax = -INFINITY;
#pragma unroll
    for (int tt = 0; tt < 8; ++tt) {
      const f32x4 ksc = *reinterpret_cast<const f32x4*>(ks_lds + 16 * tt + 4 * g);
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        const int row = 16 * tt + 4 * g + r;
        const bool vis = row < valid && t0 + row < lim;
        const float v = vis ? st[tt][r] * ksc[r] * qscale : -INFINITY;
        x[4 * tt + r] = v;
        tmax = fmaxf(tmax, v);
      }
    }
    tmax = max_xor32(max_xor16(tmax));
    const float m_new = fmaxf(m, tmax);
    const float m_use = m_new == -INFINITY ? 0.0f : m_new;
    const float alpha = exp2_fast(m - m_use);
    float psum = 0.0f, pmax = 0.0f;
    float pv[32];
#pragma unroll
    for (int tt = 0; tt < 8; ++tt) {
      const f32x4 vsc = *reinterpret_cast<const f32x4*>(vs_lds + 16 * tt + 4 * g);
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        const int e = 4 * tt + r;
        const float p = exp2_fast(x[e] - m_use);
        psum += p;
        const float w = x[e] == -INFINITY ? 0.0f : p * vsc[r];
        pv[e] = w;
        pmax = fmaxf(pmax, w);
      }
    }
    pmax = max_xor32(max_xor16(pmax));
    const float cs_new = pmax > 0.0f ? pmax / kFp8Max : cs;
    const float f = alpha * (cs / cs_new);
#pragma unroll
    for (int dt = 0; dt < 8; ++dt) acc[dt] *= f;
    cs = cs_new;
    l = l * alpha + psum;
    m = m_new;
    i32x8 p8h, p8l;
    {
      const float pinv = pmax > 0.0f ? kFp8Max / pmax : 0.0f;
#pragma unroll
      for (int c = 0; c < 8; ++c) {
        uint32_t h, lo;
        split_fp8x4(fminf(pv[4 * c] * pinv, kFp8Max), fminf(pv[4 * c + 1] * pinv, kFp8Max),
                    fminf(pv[4 * c + 2] * pinv, kFp8Max), fminf(pv[4 * c + 3] * pinv, kFp8Max),
                    h, lo);
        p8h[c] = (int)h;
        p8l[c] = (int)lo;
      }
    }

    // O^T += V^T . P8^T, one 16-wide d tile per MFMA
#pragma unroll
    for (int dt = 0; dt < 8; ++dt) {
      i32x8 va;
#pragma unroll
      for (int qq = 0; qq < 4; ++qq) {
        const i32x2 r = __builtin_amdgcn_ds_read_tr8_b64_v2i32(
            reinterpret_cast<__attribute__((address_space(3))) i32x2*>(
                (__attribute__((address_space(3))) uint8_t*)v_lds + tr_addr[qq] + 16 * dt));
        va[2 * qq] = r[0];
        va[2 * qq + 1] = r[1];
      }
      acc[dt] = mfma_fp8(va, p8h, acc[dt]);
      acc[dt] = mfma_fp8(va, p8l, acc[dt]);
    }
  }

  l = sum_xor32(sum_xor16(l));
  if (!row_ok) return;
  const float scale = l > 0.0f ? cs / l : 0.0f;
  uint16_t* op = a.out + ((int64_t)(q_begin + qi) * a.hq + qh) * kHeadDim;
#pragma unroll
  for (int dt = 0; dt < 8; ++dt) {
    const f32x4 o = acc[dt] * scale;
    const uint32_t lo = (uint32_t)A::from_f32(o[0]) | ((uint32_t)A::from_f32(o[1]) << 16);
    const uint32_t hi = (uint32_t)A::from_f32(o[2]) | ((uint32_t)A::from_f32(o[3]) << 16);
    *reinterpret_cast<u32x2*>(op + 16 * dt + 4 * g) = u32x2{lo, hi};
  }
}

}  // namespace mskv

extern "C" int mskv_fp8_prefill_attention(
    const void* query, const void* k_cache, const void* v_cache,
    const float* k_scale_cache, const float* v_scale_cache,
    const int32_t* block_tables, const int32_t* cu_seqlens_q,
    const int32_t* cu_seqlens_k, int prefix_len, void* out, int num_seqs,
    int64_t total_q, int max_seqlen_q, int num_q_heads, int num_kv_heads,
    int head_dim, int block_size, int64_t num_blocks, int max_blocks_per_seq,
    float softmax_scale, int act_dtype, void* stream) {
  if (num_seqs < 0 || total_q < 0 || max_seqlen_q < 0 || num_q_heads <= 0 ||
      num_kv_heads <= 0 || block_size <= 0 || num_blocks < 0 ||
      max_blocks_per_seq <= 0 || prefix_len < 0)
    return MSKV_EINVAL;
  if (act_dtype != MSKV_FLOAT16 && act_dtype != MSKV_BFLOAT16) return MSKV_EINVAL;
  if (num_q_heads % num_kv_heads != 0) return MSKV_EINVAL;
  if ((cu_seqlens_q == nullptr) != (cu_seqlens_k == nullptr)) return MSKV_EINVAL;
  if (cu_seqlens_q == nullptr && num_seqs != 1) return MSKV_EINVAL;
  if (cu_seqlens_q == nullptr && total_q > 0x7FFFFFFFLL - prefix_len) return MSKV_EINVAL;
  const int group = num_q_heads / num_kv_heads;
  if (head_dim != mskv::kHeadDim || block_size % mskv::kPStep != 0 ||
      (group > 16 && group % 16 != 0))
    return MSKV_EUNSUPPORTED;
  if ((int64_t)block_size * num_kv_heads * head_dim > 0x7FFFFFFFLL) return MSKV_EUNSUPPORTED;
  if (num_seqs == 0 || total_q == 0 || max_seqlen_q == 0) return MSKV_OK;
  if (!query || !k_cache || !v_cache || !k_scale_cache || !v_scale_cache ||
      !block_tables || !out)
    return MSKV_EINVAL;

  mskv::PrefillArgs a;
  a.q = (const uint16_t*)query;
  a.kc = (const uint8_t*)k_cache;
  a.vc = (const uint8_t*)v_cache;
  a.ks = k_scale_cache;
  a.vs = v_scale_cache;
  a.bt = block_tables;
  a.cu_q = cu_seqlens_q;
  a.cu_k = cu_seqlens_k;
  a.out = (uint16_t*)out;
  a.total_q = total_q;
  a.num_blocks = num_blocks;
  a.prefix_len = prefix_len;
  a.hq = num_q_heads;
  a.hk = num_kv_heads;
  a.group = group;
  a.gc = group < 16 ? group : 16;
  a.qgroups = group <= 16 ? 1 : group / 16;
  a.tpr = 16 / a.gc;
  a.bs = block_size;
  a.w = max_blocks_per_seq;
  a.scale_log2 = softmax_scale * mskv::kLog2e;
  const int per_wg = mskv::kPWaves * a.tpr;
  const dim3 grid((unsigned)((max_seqlen_q + per_wg - 1) / per_wg),
                  (unsigned)(num_kv_heads * a.qgroups), (unsigned)num_seqs);
  hipStream_t s = reinterpret_cast<hipStream_t>(stream);
  if (act_dtype == MSKV_BFLOAT16)
    hipLaunchKernelGGL(mskv::prefill_fp8_kernel<__bf16>, grid, dim3(mskv::kPThreads), 0, s, a);
  else
    hipLaunchKernelGGL(mskv::prefill_fp8_kernel<_Float16>, grid, dim3(mskv::kPThreads), 0, s, a);
  return (int)hipGetLastError();
}
