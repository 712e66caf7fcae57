// Causal varlen attention over unquantized fp16/bf16 q/k/v: the fresh
// PREFILL of the FP8-KV path.
//
// Semantics follow flash_attn_varlen_func(q, k, v, cu_seqlens_q,
// cu_seqlens_k, max_seqlen_q, max_seqlen_k, softmax_scale, causal=True) as
// microserve/layers/attention.py:49-55 calls it on the step's new tokens:
// sequence s owns query rows cu_q[s]..cu_q[s+1] and key rows
// cu_k[s]..cu_k[s+1]; query i sees key j iff j <= i + Lk - Lq (the causal
// mask aligned to the bottom right); a row that sees no key is zero.
//
// MI355X design (the paged FP8 prefill's structure with 16-bit operands):
//  * A workgroup is four waves over one (sequence, kv head, block of query
//    tokens); each wave owns three 16-row blocks, a row being one (query
//    token, q head) pair of the kv head's GQA group, so every K/V operand
//    read from LDS feeds three MFMAs (244 VGPRs: two waves per SIMD, as the
//    64 KB of LDS per workgroup allows; three blocks measured 6.7% faster
//    than two).
//  * K/V tiles of 64 keys (256-byte rows) are staged in LDS with direct
//    global -> LDS loads, double-buffered in separately declared buffers
//    with one barrier per tile.  Each row's 16-byte chunks are XOR-swizzled
//    by row % 16, which keeps the K operand reads (one chunk of 16 rows)
//    free of bank conflicts and leaves the transposed V reads 2-way; a
//    swizzle without those conflicts measured no faster.
//    The buffer resources end at the last key of the sequence, so rows past
//    it read as zeros.
//  * S^T = K . Q^T on v_mfma_f32_16x16x32_{bf16,f16}: lane (g, n) gets keys
//    4g + r of row n; for two 16-key tiles that is exactly the B operand (8
//    keys per lane) of O^T = V^T . P^T, so probabilities never move between
//    lanes.  V^T comes out of LDS with ds_read_b64_tr_b16: in each 16-lane
//    group, lane i's element j comes from the address of lane 4j + i/4 plus
//    2 * (i % 4) bytes.
//  * P is rounded to the activation type for the PV MFMA (as flash-attn
//    does) and l sums the rounded values, as a ninth output tile of the PV
//    product whose V^T operand is all ones, so each output is an exact
//    convex combination of V rows under the weights applied.
//  * Online softmax in base 2 with a lazy rescale (slack 2^8; p <= 256 fits
//    both fp16 and bf16), decided by a wave vote on each lane's own scores
//    before any cross-lane reduction; masks only on tiles that straddle the diagonal or
//    the end of the keys; query blocks launch last-first across the whole
//    grid.
#include <math.h>

#include "mskv_device.h"
#include "../../include/mskv.h"

namespace mskv {

constexpr int kDStep = 64;  // keys per tile
constexpr int kDWaves = 4;
constexpr int kDBlocks = 3;  // 16-row blocks per wave
constexpr int kDThreads = 64 * kDWaves;
constexpr int kDRow = 2 * kHeadDim;  // bytes per K/V row
constexpr int kDTile = kDStep * kDRow;
constexpr float kDSlack = 8.0f;

// Two probabilities rounded to the activation type.
template <typename T> struct PPair;
template <> struct PPair<__bf16> {
  typedef __bf16 t2 __attribute__((ext_vector_type(2)));
  __device__ static t2 pack(float a, float b) { return t2{(__bf16)a, (__bf16)b}; }
};
template <> struct PPair<_Float16> {
  typedef _Float16 t2 __attribute__((ext_vector_type(2)));
  __device__ static t2 pack(float a, float b) { return t2{(_Float16)a, (_Float16)b}; }
};

struct DenseArgs {
  const uint16_t* q;
  const uint16_t* k;
  const uint16_t* v;
  uint16_t* out;
  const int32_t* cu_q;
  const int32_t* cu_k;
  int64_t total_q, total_k;
  int hq, hk, group, gc, qgroups, tpr;
  float scale_log2;
};

// LDS byte offset of 16-byte chunk `chunk` (0..15) of tile row `row`
__device__ __forceinline__ uint32_t dtile_off(int row, int chunk) {
  return (uint32_t)row * kDRow + 16u * (uint32_t)(chunk ^ (row & 15));
}

__device__ __forceinline__ void lds_load16_d(__amdgpu_buffer_rsrc_t r, void* lds, uint32_t off) {
  __builtin_amdgcn_raw_ptr_buffer_load_lds(
      r, (__attribute__((address_space(3))) void*)lds, 16, (int)off, 0, 0, 0);
}

template <typename T>
__global__ __launch_bounds__(kDThreads, 2) void dense_prefill_kernel(DenseArgs a) {
  using A = Act<T>;
  using x8 = typename A::x8;
  typedef short i16x4 __attribute__((ext_vector_type(4)));
  __shared__ __attribute__((aligned(16))) uint8_t k_lds0[kDTile];
  __shared__ __attribute__((aligned(16))) uint8_t v_lds0[kDTile];
  __shared__ __attribute__((aligned(16))) uint8_t k_lds1[kDTile];
  __shared__ __attribute__((aligned(16))) uint8_t v_lds1[kDTile];

  const int tid = threadIdx.x;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int lane = tid & 63;
  const int g = lane >> 4, n = lane & 15;
  // grid (kv head units, sequences, query blocks): the query block varies
  // slowest and runs last-first, so every sequence's longest blocks are
  // dispatched before any shorter ones (longest-first across the whole
  // grid, not within each sequence); measured 3.8% faster than query
  // blocks varying fastest
  const int s = blockIdx.y;
  const int unit = blockIdx.x;
  const int kvh = unit / a.qgroups;
  const int qgi = unit - kvh * a.qgroups;

  // rows and keys are clamped to the tensors, so inconsistent cu_seqlens
  // cannot address memory outside them
  const int64_t tq = a.total_q, tk = a.total_k;
  const int q_begin = (int)min((int64_t)max(a.cu_q[s], 0), tq);
  const int q_end = (int)min((int64_t)max(a.cu_q[s + 1], q_begin), tq);
  const int64_t k_begin = min((int64_t)max(a.cu_k[s], 0), tk);
  const int64_t k_end = min((int64_t)max(a.cu_k[s + 1], 0), tk);
  const int lq = q_end - q_begin;
  const int lk = (int)max(k_end - k_begin, (int64_t)0);
  const int shift = lk - lq;  // query i sees keys j <= i + shift
  const int wave_tok = kDBlocks * a.tpr;
  const int wg_tok = kDWaves * wave_tok;
  const int wg_q0 = (int)(gridDim.z - 1 - blockIdx.z) * wg_tok;
  if (wg_q0 >= lq) return;
  const int wg_qlast = min(lq, wg_q0 + wg_tok) - 1;
  const int kv_end = max(0, min(lk, wg_qlast + shift + 1));
  const int w_q0 = wg_q0 + wave * wave_tok;
  const int w_all = w_q0 + shift + 1;  // keys below this: visible to every row
  const int w_none = w_q0 < lq ? min(lq, w_q0 + wave_tok) + shift : 0;

  int lim[kDBlocks];
  bool row_ok[kDBlocks];
  int qh[kDBlocks];
  x8 qop[kDBlocks][4];
#pragma unroll
  for (int b = 0; b < kDBlocks; ++b) {
    const int qi = w_q0 + b * a.tpr + n / a.gc;
    // a unit of a group above 16 that is not a multiple of 16 has idle
    // lanes past the group's last head
    row_ok[b] = n < a.tpr * a.gc && qi < lq && qgi * 16 + n % a.gc < a.group;
    qh[b] = kvh * a.group + qgi * 16 + n % a.gc;
    lim[b] = row_ok[b] ? qi + shift + 1 : 0;
    // B operand of S^T = K . Q^T: lane (g, n) holds d in [32c + 8g, +8)
    const u32x4* qp = reinterpret_cast<const u32x4*>(
        a.q + ((int64_t)(q_begin + (row_ok[b] ? qi : 0)) * a.hq + qh[b]) * kHeadDim + 8 * g);
#pragma unroll
    for (int c = 0; c < 4; ++c)
      qop[b][c] = __builtin_bit_cast(x8, row_ok[b] ? qp[4 * c] : u32x4{0u, 0u, 0u, 0u});
  }

  // acc: O^T; lacc: the denominator, as a ninth output tile whose V^T
  // operand is all ones, so each of its rows is the column's sum of the
  // rounded probabilities
  f32x4 acc[kDBlocks][8], lacc[kDBlocks];
  float m[kDBlocks];
#pragma unroll
  for (int b = 0; b < kDBlocks; ++b) {
#pragma unroll
    for (int dt = 0; dt < 8; ++dt) acc[b][dt] = f32x4{0.f, 0.f, 0.f, 0.f};
    lacc[b] = f32x4{0.f, 0.f, 0.f, 0.f};
    m[b] = -INFINITY;
  }

  // K operand: key n of each 16-key group, chunk 4c + g; the row swizzle
  // (row % 16 == n) does not depend on the group
  uint32_t k_off[4];
#pragma unroll
  for (int c = 0; c < 4; ++c) k_off[c] = (uint32_t)n * kDRow + 16u * (uint32_t)((4 * c + g) ^ n);
  // V^T operand: for 32-key chunk ch and read q, source lane s of group g
  // supplies key 32ch + 16q + 4g + s/4, d 16dt + 4(s%4); that row's swizzle
  // is 4g + s/4 for every ch and q, and chunk 2dt + (s%4)/2 swizzles to
  // 2dt ^ ((s%4)/2 ^ swz)
  const int sl = lane & 15;
  const uint32_t v_row = (uint32_t)(4 * g + (sl >> 2)) * kDRow + 8u * (uint32_t)(sl & 1);
  const uint32_t v_x = 16u * (uint32_t)(((sl & 3) >> 1) ^ (4 * g + (sl >> 2)));

  const uint32_t rstride = (uint32_t)a.hk * kDRow;  // bytes between key rows
  auto stage_tile = [&](int t0, uint8_t* kt, uint8_t* vt) {
    const int valid = min(kDStep, lk - t0);
    const int64_t e0 = ((k_begin + t0) * a.hk + kvh) * kHeadDim;
    const uint32_t bytes = valid > 0 ? (uint32_t)(valid - 1) * rstride + kDRow : 0u;
    const auto kr = make_rsrc(a.k + e0, bytes);
    const auto vr = make_rsrc(a.v + e0, bytes);
    // wave w's j-th load fills rows 4(4j + w) .. +4: lane i lands in slot i,
    // i.e. row 4(4j + w) + i/16 at swizzled position i%16
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const int row = 4 * (4 * j + wave) + (lane >> 4);
      const int c = (lane & 15) ^ (row & 15);
      const uint32_t o = (uint32_t)row * rstride + 16u * (uint32_t)c;
      lds_load16_d(kr, kt + 1024 * (4 * j + wave), o);
      lds_load16_d(vr, vt + 1024 * (4 * j + wave), o);
    }
  };

  auto compute_tile = [&](int t0, const uint8_t* kt, const uint8_t* vt) {
    if (t0 >= w_none) return;
    // S^T = K . Q^T: four 16-key tiles, head_dim in four 32-wide chunks
    f32x4 st[kDBlocks][4];
#pragma unroll
    for (int tt = 0; tt < 4; ++tt) {
#pragma unroll
      for (int c = 0; c < 4; ++c) {
        const x8 ka = __builtin_bit_cast(
            x8, *reinterpret_cast<const u32x4*>(kt + 16 * tt * kDRow + k_off[c]));
#pragma unroll
        for (int b = 0; b < kDBlocks; ++b)
          st[b][tt] = A::mfma(ka, qop[b][c], c == 0 ? f32x4{0.f, 0.f, 0.f, 0.f} : st[b][tt]);
      }
    }
    const bool full = t0 + kDStep <= w_all && t0 + kDStep <= lk;
    if (!full) {
#pragma unroll
      for (int tt = 0; tt < 4; ++tt)
#pragma unroll
        for (int r = 0; r < 4; ++r) {
          const int key = t0 + 16 * tt + 4 * g + r;
#pragma unroll
          for (int b = 0; b < kDBlocks; ++b)
            if (key >= lim[b]) st[b][tt][r] = -INFINITY;
        }
    }
    // Each lane tests its own 16 scores against the row's running max: a
    // row's maximum is the largest of its four lanes', and the positive
    // scale keeps the order, so the wave vote equals the test on the row
    // maxima.  The cross-lane reduction runs only when the vote passes.
    float lm[kDBlocks];
    bool grow = false;
#pragma unroll
    for (int b = 0; b < kDBlocks; ++b) {
      float v = fmaxf(fmaxf(st[b][0][0], st[b][0][1]), fmaxf(st[b][0][2], st[b][0][3]));
#pragma unroll
      for (int tt = 1; tt < 4; ++tt)
        v = fmaxf(fmaxf(v, st[b][tt][0]), fmaxf(fmaxf(st[b][tt][1], st[b][tt][2]), st[b][tt][3]));
      lm[b] = v;
      grow |= v * a.scale_log2 > m[b] + kDSlack;
    }
    if (__any(grow)) {
#pragma unroll
      for (int b = 0; b < kDBlocks; ++b) {
        const float m_new = fmaxf(m[b], max_xor32(max_xor16(lm[b])) * a.scale_log2);
        const float alpha = m_new == -INFINITY ? 1.0f : exp2_fast(m[b] - m_new);
        lacc[b] *= alpha;
#pragma unroll
        for (int dt = 0; dt < 8; ++dt) acc[b][dt] *= alpha;
        m[b] = m_new;
      }
    }
    // P^T operands: chunk ch holds keys {4g + r} of tiles 2ch and 2ch + 1
    x8 pv[kDBlocks][2];
#pragma unroll
    for (int b = 0; b < kDBlocks; ++b) {
      const float m_use = m[b] == -INFINITY ? 0.0f : m[b];
#pragma unroll
      for (int tt = 0; tt < 4; ++tt)
#pragma unroll
        for (int r = 0; r < 4; r += 2) {
          const auto pk = PPair<T>::pack(exp2_fast(fmaf(st[b][tt][r], a.scale_log2, -m_use)),
                                         exp2_fast(fmaf(st[b][tt][r + 1], a.scale_log2, -m_use)));
          pv[b][tt >> 1][4 * (tt & 1) + r] = pk[0];
          pv[b][tt >> 1][4 * (tt & 1) + r + 1] = pk[1];
        }
    }
    // O^T += V^T . P^T, one 16-wide d tile and 32-key chunk per MFMA.  The
    // wave raises its priority over this loop (the probabilities' rounding
    // is interleaved with it): 3.7% faster than equal priority, and faster
    // than raising it over the QK^T loop too.
    __builtin_amdgcn_s_setprio(1);
#pragma unroll
    for (int dt = 0; dt < 8; ++dt) {
      const uint32_t vo = v_row + ((32u * dt) ^ v_x);
#pragma unroll
      for (int ch = 0; ch < 2; ++ch) {
        const i16x4 r0 = __builtin_amdgcn_ds_read_tr16_b64_v4i16(
            reinterpret_cast<__attribute__((address_space(3))) i16x4*>(
                (__attribute__((address_space(3))) uint8_t*)vt + 32 * ch * kDRow + vo));
        const i16x4 r1 = __builtin_amdgcn_ds_read_tr16_b64_v4i16(
            reinterpret_cast<__attribute__((address_space(3))) i16x4*>(
                (__attribute__((address_space(3))) uint8_t*)vt + (32 * ch + 16) * kDRow + vo));
        const i16x4 lo4 = r0, hi4 = r1;
        typedef short i16x8 __attribute__((ext_vector_type(8)));
        const i16x8 w = {lo4[0], lo4[1], lo4[2], lo4[3], hi4[0], hi4[1], hi4[2], hi4[3]};
        const x8 va = __builtin_bit_cast(x8, w);
#pragma unroll
        for (int b = 0; b < kDBlocks; ++b) acc[b][dt] = A::mfma(va, pv[b][ch], acc[b][dt]);
      }
    }
    // the denominator: sums of the probabilities as rounded for the MFMA,
    // so each output is an exact convex combination of V rows under them
    // (a chain of v_dot2 per pair summed the same rounded values at 4% of
    // the kernel's time)
    {
      x8 ones;
#pragma unroll
      for (int i = 0; i < 8; ++i) ones[i] = (T)1.0f;
#pragma unroll
      for (int ch = 0; ch < 2; ++ch)
#pragma unroll
        for (int b = 0; b < kDBlocks; ++b) lacc[b] = A::mfma(ones, pv[b][ch], lacc[b]);
    }
    __builtin_amdgcn_s_setprio(0);
  };

  if (kv_end > 0) {
    stage_tile(0, k_lds0, v_lds0);
    __syncthreads();
    for (int t0 = 0; t0 < kv_end; t0 += 2 * kDStep) {
      {
        const bool more = t0 + kDStep < kv_end;
        if (more) stage_tile(t0 + kDStep, k_lds1, v_lds1);
        compute_tile(t0, k_lds0, v_lds0);
        __syncthreads();  // also waits for this wave's direct loads
        if (!more) break;
      }
      {
        const int t1 = t0 + kDStep;
        const bool more = t1 + kDStep < kv_end;
        if (more) stage_tile(t1 + kDStep, k_lds0, v_lds0);
        compute_tile(t1, k_lds1, v_lds1);
        __syncthreads();
      }
    }
  }

#pragma unroll
  for (int b = 0; b < kDBlocks; ++b) {
    const float lt = lacc[b][0];
    if (!row_ok[b]) continue;
    const float inv = lt > 0.0f ? 1.0f / lt : 0.0f;
    uint16_t* op =
        a.out + ((int64_t)(q_begin + w_q0 + b * a.tpr + n / a.gc) * a.hq + qh[b]) * kHeadDim;
#pragma unroll
    for (int dt = 0; dt < 8; ++dt) {
      const f32x4 o = acc[b][dt] * inv;
      const uint32_t lo = (uint32_t)A::from_f32(o[0]) | ((uint32_t)A::from_f32(o[1]) << 16);
      const uint32_t hi = (uint32_t)A::from_f32(o[2]) | ((uint32_t)A::from_f32(o[3]) << 16);
      *reinterpret_cast<u32x2*>(op + 16 * dt + 4 * g) = u32x2{lo, hi};
    }
  }
}

}  // namespace mskv

extern "C" int mskv_prefill_attention(const void* query, const void* key, const void* value,
                                      void* out, const int32_t* cu_seqlens_q,
                                      const int32_t* cu_seqlens_k, int num_seqs,
                                      int64_t total_q, int64_t total_k, int max_seqlen_q,
                                      int num_q_heads, int num_kv_heads, int head_dim,
                                      float softmax_scale, int act_dtype, void* stream) {
  if (num_seqs < 0 || total_q < 0 || total_k < 0 || max_seqlen_q < 0 || num_q_heads <= 0 ||
      num_kv_heads <= 0)
    return MSKV_EINVAL;
  if (act_dtype != MSKV_FLOAT16 && act_dtype != MSKV_BFLOAT16) return MSKV_EINVAL;
  if (num_q_heads % num_kv_heads != 0) return MSKV_EINVAL;
  const int group = num_q_heads / num_kv_heads;
  if (head_dim != mskv::kHeadDim) return MSKV_EUNSUPPORTED;
  // the row maxima are taken before the scale, which must keep their order
  const float scale_log2 = softmax_scale * mskv::kLog2e;
  if (!(scale_log2 > 0.0f && scale_log2 < INFINITY)) return MSKV_EUNSUPPORTED;
  if (num_seqs == 0 || total_q == 0 || max_seqlen_q == 0) return MSKV_OK;
  if (!query || !key || !value || !out || !cu_seqlens_q || !cu_seqlens_k) return MSKV_EINVAL;
  // per-tile offsets are 32-bit: 64 key rows of all kv heads
  if ((int64_t)mskv::kDStep * num_kv_heads * mskv::kDRow > 0x7FFFFFFFLL) return MSKV_EUNSUPPORTED;

  mskv::DenseArgs a;
  a.q = (const uint16_t*)query;
  a.k = (const uint16_t*)key;
  a.v = (const uint16_t*)value;
  a.out = (uint16_t*)out;
  a.cu_q = cu_seqlens_q;
  a.cu_k = cu_seqlens_k;
  a.total_q = total_q;
  a.total_k = total_k;
  a.hq = num_q_heads;
  a.hk = num_kv_heads;
  a.group = group;
  a.gc = group < 16 ? group : 16;
  a.qgroups = (group + 15) / 16;
  a.tpr = 16 / a.gc;
  a.scale_log2 = scale_log2;
  const int per_wg = mskv::kDWaves * mskv::kDBlocks * a.tpr;
  // grid y and z are limited to 65535
  const int64_t qblocks = ((int64_t)max_seqlen_q + per_wg - 1) / per_wg;
  if (num_seqs > 65535 || qblocks > 65535) return MSKV_EUNSUPPORTED;
  const dim3 grid((unsigned)(num_kv_heads * a.qgroups), (unsigned)num_seqs,
                  (unsigned)qblocks);
  hipStream_t st = reinterpret_cast<hipStream_t>(stream);
  if (act_dtype == MSKV_BFLOAT16)
    hipLaunchKernelGGL(mskv::dense_prefill_kernel<__bf16>, grid, dim3(mskv::kDThreads), 0, st, a);
  else
    hipLaunchKernelGGL(mskv::dense_prefill_kernel<_Float16>, grid, dim3(mskv::kDThreads), 0, st,
                       a);
  return (int)hipGetLastError();
}
