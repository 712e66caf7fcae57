// Varlen causal prefill over the FP8 e4m3fn paged cache with FP8 MFMA.
//
// Semantics follow microserve/layers/fp8_chunk_prefill_attention.py:16-67,
// generalized to a varlen batch: query i of a sequence with Lq new tokens
// and Lk cached tokens (new ones included) sees positions
// p < (Lk - Lq) + i + 1 (:52-54); K/V row p lives at
// block_tables[s][p / BS] * BS + p % BS.
//
// MI355X design:
//  * A workgroup covers 128 rows of one (sequence, kv head, block of query
//    tokens).  A row is one (query token, q head) pair; the GQA group of the
//    kv head fills the rows, so every K/V tile serves all the q heads that
//    read it.  Four waves of two 16-row blocks, so every K operand a wave
//    reads from LDS feeds both.  bf16 also shares each V^T operand between
//    the blocks; fp16, whose query needs a third e4m3 part, computes one
//    block's P and PV at a time to stay within the register file.
//  * K/V tiles of 128 keys (one f8f6f4 MFMA contraction) are staged in LDS,
//    double-buffered with one barrier per tile.  Rows are written with their
//    16-byte chunks XOR-swizzled by (row / 2) % 8, which keeps the row
//    writes and the K operand reads free of bank conflicts; the transposed
//    V reads are 2-way (rows r and r + 16 share banks), and a swizzle that
//    removes that measured slower.
//  * QK^T: S^T = K . Q8^T with v_mfma_f32_16x16x128_f8f6f4 -- the whole
//    head_dim is one MFMA.  K bytes are used as stored.  The query row is
//    scaled by a power of two (exact) and split into e4m3 parts: hi + lo
//    represent a bf16 query exactly (4 + 4 significant bits), fp16 needs
//    hi + mid + lo; one MFMA per part into the same accumulator.
//  * PV: O^T = V^T . P8^T with the same MFMA.  S^T's accumulator leaves lane
//    (g, n) holding 32 keys of row n, exactly the B-operand layout of P^T,
//    so probabilities never move between lanes; V^T comes out of LDS with
//    ds_read_b64_tr_b8.  P * v_scale is split into e4m3 hi + lo parts after
//    a per-tile power-of-two scale chosen from the tile's largest v_scale;
//    the accumulator is rescaled (exactly) only when that power changes.
//  * The softmax denominator sums the weights the MFMA applies,
//    (hi + lo) / v_scale, so each output is an exact convex combination of
//    V rows.  Each wave computes the tile's 1 / v_scale once per key into
//    LDS; keys whose V is too small for their weights to fit e4m3 add their
//    exact p on a rare wave-uniform path instead.
//  * Online softmax in base 2 with a lazy rescale: the accumulator is
//    rescaled only when some row's max grows by more than 2^8.  Masks are
//    evaluated only on tiles that straddle the causal diagonal or the end
//    of the keys; fully visible tiles skip them.
//  * Query blocks are launched last-first across the whole grid, so the
//    longest workgroups of every sequence start before any shorter one.
//    Pages are read through page-sized buffer resources; an invalid block
//    id gives zero-length reads and its keys are masked.
#include <math.h>

#include "mskv_device.h"
#include "../../include/mskv.h"

namespace mskv {

constexpr int kPStep = 128;  // keys per tile
// A workgroup covers 128 rows: 4 waves of two 16-row blocks.  fp16's third
// query part costs 16 registers, which it wins back by running the P and
// PV work of its two blocks one after the other.
template <int NQ> struct PShape {
  static constexpr int blocks = 2;  // 16-row blocks per wave
  static constexpr int waves = 8 / blocks;
  static constexpr int threads = 64 * waves;
};
// The running max may lag a row's true max by up to kPSlack (log2 units)
// before the accumulator is rescaled.  P is normalized per row and tile
// (see below), so the slack does not cost P precision.
constexpr float kPSlack = 8.0f;
// The tile's v_scales are scaled by a power of two to at most this value, so
// p * v_scale (p <= 1 after the per-row normalization) stays within 448.
constexpr float kPVScaleMax = 384.0f;
// Below this v_scale * fcur the two e4m3 parts of a key's weight
// p * v_scale * fcur (at most 1/4 for such a key) hold too few bits for
// its share of the softmax denominator, so its exact p goes there instead.
constexpr float kPTinyV = 0.25f;

// e4m3 parts the query is split into: a bf16 value has 8 significant bits
template <typename T> struct QuerySplit { static constexpr int parts = 3; };
template <> struct QuerySplit<__bf16> { static constexpr int parts = 2; };
template <typename T> using PShapeOf = PShape<QuerySplit<T>::parts>;

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
  // compile-time zero scales select the unscaled v_mfma_f32_16x16x128_f8f6f4
  return __builtin_amdgcn_mfma_scale_f32_16x16x128_f8f6f4(a, b, c, 0, 0, 0, 0, 0, 0);
}

// The same MFMA with an E8M0 block scale on B: lane (g, n)'s scale byte sb
// multiplies its column n, k-block g by 2^(sb - 127) (A's scale is 1.0).
__device__ __forceinline__ f32x4 mfma_fp8_scale_b(const i32x8& a, const i32x8& b, f32x4 c,
                                                  int sb) {
  return __builtin_amdgcn_mfma_scale_f32_16x16x128_f8f6f4(a, b, c, 0, 0, 0, 127, 0, sb);
}

// Direct global -> LDS loads (buffer_load ... lds): lane i of the wave
// writes its `bytes` at lds + i * bytes, from any per-lane offset.
__device__ __forceinline__ void lds_load16(__amdgpu_buffer_rsrc_t r, void* lds, uint32_t off) {
  __builtin_amdgcn_raw_ptr_buffer_load_lds(
      r, (__attribute__((address_space(3))) void*)lds, 16, (int)off, 0, 0, 0);
}
__device__ __forceinline__ void lds_load4(__amdgpu_buffer_rsrc_t r, void* lds, uint32_t off) {
  __builtin_amdgcn_raw_ptr_buffer_load_lds(
      r, (__attribute__((address_space(3))) void*)lds, 4, (int)off, 0, 0, 0);
}

template <typename T>
__global__ __launch_bounds__(PShapeOf<T>::threads, 2) void prefill_fp8_kernel(PrefillArgs a) {
  using A = Act<T>;
  constexpr int NQ = QuerySplit<T>::parts;
  constexpr int kPBlocks = PShapeOf<T>::blocks;
  constexpr int kPWaves = PShapeOf<T>::waves;
  // two tile buffers as separate objects, and a loop unrolled by two, so
  // the compiler can see that the direct loads into one buffer never alias
  // the reads of the other (otherwise it waits for them before every read)
  __shared__ __attribute__((aligned(16))) uint8_t k_lds0[kPStep * kHeadDim];
  __shared__ __attribute__((aligned(16))) uint8_t v_lds0[kPStep * kHeadDim];
  __shared__ __attribute__((aligned(16))) uint8_t k_lds1[kPStep * kHeadDim];
  __shared__ __attribute__((aligned(16))) uint8_t v_lds1[kPStep * kHeadDim];
  __shared__ __attribute__((aligned(16))) float sc_lds0[2][kPStep];
  __shared__ __attribute__((aligned(16))) float sc_lds1[2][kPStep];
  // each wave's reciprocals of the current tile's v_scales
  __shared__ __attribute__((aligned(16))) float rv_lds[kPWaves][kPStep];

  const int tid = threadIdx.x;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int lane = tid & 63;
  const int g = lane >> 4, n = lane & 15;
  // grid (kv head units, sequences, query blocks): the query block varies
  // slowest and runs last-first, so every sequence's longest blocks are
  // dispatched before any shorter ones (longest-first across the whole
  // grid, not within each sequence): bf16 5.4%, fp16 3.9% faster than
  // query blocks varying fastest
  const int s = blockIdx.y;
  const int unit = blockIdx.x;
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
  const int wave_tok = kPBlocks * a.tpr;  // query tokens per wave
  const int wg_tok = kPWaves * wave_tok;
  const int wg_q0 = (int)(gridDim.z - 1 - blockIdx.z) * wg_tok;
  if (wg_q0 >= lq || lq <= 0) return;
  const int wg_qlast = min(lq, wg_q0 + wg_tok) - 1;
  const int kv_end = min(min(lk, prefix + wg_qlast + 1), a.w * a.bs);
  // keys below w_all are visible to every row of this wave; no row of it
  // sees keys at or above w_none
  const int w_q0 = wg_q0 + wave * wave_tok;
  const int w_all = prefix + w_q0 + 1;
  const int w_none = w_q0 < lq ? prefix + min(lq, w_q0 + wave_tok) : 0;

  // rows: block b, lane n -> query token w_q0 + b * tpr + n / gc, head n % gc
  int lim[kPBlocks];
  bool row_ok[kPBlocks];
  int qh[kPBlocks];
  i32x8 qp[kPBlocks][NQ];
  float qs[kPBlocks];
#pragma unroll
  for (int b = 0; b < kPBlocks; ++b) {
    const int qi = w_q0 + b * a.tpr + n / a.gc;
    row_ok[b] = n < a.tpr * a.gc && qi < lq;
    qh[b] = kvh * a.group + qgi * 16 + n % a.gc;
    lim[b] = row_ok[b] ? prefix + qi + 1 : 0;
    // lane (g, n) holds d in [32g, 32g+32) of its row
    float x[32];
    if (row_ok[b]) {
      const u32x4* qp4 = reinterpret_cast<const u32x4*>(
          a.q + ((int64_t)(q_begin + qi) * a.hq + qh[b]) * kHeadDim + 32 * g);
#pragma unroll
      for (int c = 0; c < 4; ++c) {
        const u32x4 v = qp4[c];
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
    // power-of-two scale: x * f is exact, so the parts carry every bit
    const float f = amax > 1e-30f ? pow2_floor(kFp8Max / amax) : 1.0f;
    qs[b] = a.scale_log2 / f;
#pragma unroll
    for (int c = 0; c < 8; ++c) {
      float y[4];
#pragma unroll
      for (int i = 0; i < 4; ++i) y[i] = fminf(fmaxf(x[4 * c + i] * f, -kFp8Max), kFp8Max);
      uint32_t h, mi, lo;
      if constexpr (NQ == 2) {
        split_fp8x4(y[0], y[1], y[2], y[3], h, lo);
        qp[b][0][c] = (int)h;
        qp[b][1][c] = (int)lo;
      } else {
        split3_fp8x4(y[0], y[1], y[2], y[3], h, mi, lo);
        qp[b][0][c] = (int)h;
        qp[b][1][c] = (int)mi;
        qp[b][2][c] = (int)lo;
      }
    }
  }

  f32x4 acc[kPBlocks][8];
#pragma unroll
  for (int b = 0; b < kPBlocks; ++b)
#pragma unroll
    for (int dt = 0; dt < 8; ++dt) acc[b][dt] = f32x4{0.f, 0.f, 0.f, 0.f};
  float m[kPBlocks], l[kPBlocks];
#pragma unroll
  for (int b = 0; b < kPBlocks; ++b) {
    m[b] = -INFINITY;
    l[b] = 0.0f;
  }
  // acc and l are kept in units of fcur, the power-of-two scale applied to
  // p * v_scale; lf = log2(fcur) is folded into the exp argument
  float fcur = 1.0f, lf = 0.0f;

  // K operand: key n of each 16-key group, 16-byte chunks 2g and 2g + 1;
  // the swizzle of rows 16t + n does not depend on t
  const uint32_t k_lo = tile_off(n, 2 * g), k_hi = tile_off(n, 2 * g + 1);
  // ds_read_b64_tr_b8 address of this lane for read qq (keys 8qq..8qq+7 of
  // the lane group's 32): key slot e = 8qq + i/2 maps to tile row
  // 16*(e/4) + 4g + e%4, column half i%2
  const int i16 = lane & 15;
  uint32_t tr_row[4], tr_swz[4];
#pragma unroll
  for (int qq = 0; qq < 4; ++qq) {
    const int e = 8 * qq + (i16 >> 1);
    const int row = 16 * (e >> 2) + 4 * g + (e & 3);
    tr_row[qq] = (uint32_t)row * kHeadDim + 8u * (i16 & 1);
    tr_swz[qq] = 16u * (uint32_t)((row >> 1) & 7);
  }

  const uint32_t page_bytes = (uint32_t)a.bs * a.hk * kHeadDim;
  const uint32_t spage_bytes = (uint32_t)a.bs * a.hk * 4u;
  const uint32_t rstride = (uint32_t)a.hk * kHeadDim;
  // the block table is read-only: the constant address space keeps its
  // loads scalar
  const auto* btc = reinterpret_cast<const __attribute__((address_space(4))) int32_t*>(
      reinterpret_cast<uintptr_t>(a.bt));

  // Stage tile t0 into LDS buffer `buf` with direct loads; returns the
  // number of keys holding real tokens.  With W waves, wave w's j-th K (and
  // V) load fills tile rows 8(Wj + w) .. +8: lane i lands in slot i of that
  // kilobyte, i.e. row 8(Wj + w) + i/8 at swizzled position i%8, so it reads
  // logical chunk
  // (i%8) ^ swizzle(row); four consecutive lanes still read one aligned
  // 64-byte half row.  The resources end at the last valid row, so rows past
  // it read as zeros (a stray NaN byte would otherwise poison the MFMA sum)
  // and so do their scales.
  auto stage_tile = [&](int t0, uint8_t* kt, uint8_t* vt, float (*sct)[kPStep]) {
    const int page = t0 / a.bs;
    const int off = t0 - page * a.bs;
    const int blk = btc[(int64_t)s * a.w + page];
    const bool ok = blk >= 0 && (int64_t)blk < a.num_blocks;
    const int valid = ok ? min(kPStep, lk - t0) : 0;
    const int64_t bo = ok ? blk : 0;
    const uint32_t kv_bytes = (uint32_t)(off + valid) * rstride;
    const auto kr = make_rsrc(a.kc + bo * page_bytes, valid > 0 ? kv_bytes : 0u);
    const auto vr = make_rsrc(a.vc + bo * page_bytes, valid > 0 ? kv_bytes : 0u);
    const auto sr = make_rsrc((wave < 2 ? a.ks : a.vs) + bo * a.bs * a.hk,
                              valid > 0 ? (uint32_t)(off + valid) * a.hk * 4u : 0u);
    const uint32_t base = (uint32_t)off * rstride + (uint32_t)kvh * kHeadDim;
#pragma unroll
    for (int j = 0; j < 16 / kPWaves; ++j) {
      const int row = 8 * (kPWaves * j + wave) + (lane >> 3);
      const int c = (lane & 7) ^ ((row >> 1) & 7);
      const uint32_t o = base + (uint32_t)row * rstride + 16u * c;
      lds_load16(kr, kt + 1024 * (kPWaves * j + wave), o);
      lds_load16(vr, vt + 1024 * (kPWaves * j + wave), o);
    }
    // waves 0-1 load the k_scales, waves 2-3 the v_scales
    if (wave < 4) {
      const int key = 64 * (wave & 1) + lane;
      lds_load4(sr, &sct[wave >> 1][64 * (wave & 1)],
                (((uint32_t)off + key) * a.hk + kvh) * 4u);
    }
    return valid;
  };

  // one tile of work for this wave: QK^T, softmax, PV
  auto compute_tile = [&](int t0, int valid, const uint8_t* kt, const uint8_t* vt,
                          const float (*sct)[kPStep]) {
    if (t0 < w_none) {
      const float* kss = sct[0];
      const float* vss = sct[1];
      // S^T = K . Q8^T: lane (g, n) gets keys 16tt + 4g + r of row n
      f32x4 st[kPBlocks][8];
#pragma unroll
      for (int tt = 0; tt < 8; ++tt) {
        const u32x4 lo = *reinterpret_cast<const u32x4*>(kt + 16 * tt * kHeadDim + k_lo);
        const u32x4 hi = *reinterpret_cast<const u32x4*>(kt + 16 * tt * kHeadDim + k_hi);
        const i32x8 ka = {(int)lo[0], (int)lo[1], (int)lo[2], (int)lo[3],
                          (int)hi[0], (int)hi[1], (int)hi[2], (int)hi[3]};
#pragma unroll
        for (int b = 0; b < kPBlocks; ++b) {
          st[b][tt] = mfma_fp8(ka, qp[b][0], f32x4{0.f, 0.f, 0.f, 0.f});
#pragma unroll
          for (int p = 1; p < NQ; ++p) st[b][tt] = mfma_fp8(ka, qp[b][p], st[b][tt]);
        }
      }
      // s * k_scale; masked keys -> -inf on tiles that need masks
      const bool full = t0 + kPStep <= w_all && valid == kPStep;
#pragma unroll
      for (int tt = 0; tt < 8; ++tt) {
        const f32x4 ksc = *reinterpret_cast<const f32x4*>(kss + 16 * tt + 4 * g);
#pragma unroll
        for (int b = 0; b < kPBlocks; ++b) st[b][tt] *= ksc;
      }
      // The barrier after each row of keys keeps the scheduler from hoisting
      // all 64 lane-mask compares ahead of their selects.  Hoisted, their
      // SGPR pairs overflow the SGPR file, and the allocator then spills
      // SGPRs through VGPR lanes in every tile, masked or not (~50
      // v_readlane/v_writelane per full tile): 4.7-4.9% of kernel time.
      if (!full) {
#pragma unroll
        for (int tt = 0; tt < 8; ++tt) {
#pragma unroll
          for (int r = 0; r < 4; ++r) {
            const int key = 16 * tt + 4 * g + r;
#pragma unroll
            for (int b = 0; b < kPBlocks; ++b)
              if (!(key < valid && t0 + key < lim[b])) st[b][tt][r] = -INFINITY;
          }
          __builtin_amdgcn_sched_barrier(0);
        }
      }
      // row maxima in log2 units (qs > 0 per row)
      float tm[kPBlocks];
#pragma unroll
      for (int b = 0; b < kPBlocks; ++b) {
        float v = fmaxf(fmaxf(st[b][0][0], st[b][0][1]), fmaxf(st[b][0][2], st[b][0][3]));
#pragma unroll
        for (int tt = 1; tt < 8; ++tt)
          v = fmaxf(fmaxf(v, st[b][tt][0]), fmaxf(fmaxf(st[b][tt][1], st[b][tt][2]), st[b][tt][3]));
        tm[b] = max_xor32(max_xor16(v)) * qs[b];
      }
      bool grow = false;
#pragma unroll
      for (int b = 0; b < kPBlocks; ++b) grow |= tm[b] > m[b] + kPSlack;
      if (__any(grow)) {
#pragma unroll
        for (int b = 0; b < kPBlocks; ++b) {
          const float m_new = fmaxf(m[b], tm[b]);
          const float alpha = m_new == -INFINITY ? 1.0f : exp2_fast(m[b] - m_new);
          l[b] *= alpha;
#pragma unroll
          for (int dt = 0; dt < 8; ++dt) acc[b][dt] *= alpha;
          m[b] = m_new;
        }
      }
      // this tile's power-of-two scale for p * v_scale, from its largest
      // v_scale (lane group g reads keys 16tt + 4g + r)
      float vm = 0.0f;
#pragma unroll
      for (int tt = 0; tt < 8; ++tt) {
        const f32x4 v4 = *reinterpret_cast<const f32x4*>(vss + 16 * tt + 4 * g);
        vm = fmaxf(vm, fmaxf(fmaxf(v4[0], v4[1]), fmaxf(v4[2], v4[3])));
      }
      vm = max_xor32(max_xor16(vm));
      if (vm > 0.0f) {
        const float ft = pow2_floor(kPVScaleMax / vm);
        if (ft != fcur) {
          const float r = ft / fcur;  // a power of two: exact
#pragma unroll
          for (int b = 0; b < kPBlocks; ++b) {
            l[b] *= r;
#pragma unroll
            for (int dt = 0; dt < 8; ++dt) acc[b][dt] *= r;
          }
          fcur = ft;
          lf = (float)((int)((__float_as_uint(ft) >> 23) & 0xFFu) - 127);
        }
      }
      // P, normalized per row and tile: with k = floor(m - tile max) the row's
      // largest p * 2^k is at most 1, so a tile far below the row max keeps
      // its probabilities out of e4m3's underflow; the PV MFMA multiplies
      // 2^-k back through its per-row E8M0 scale on P.
      // y = p * 2^k * fcur * v_scale is split into e4m3 hi + lo.  l sums the
      // weights the MFMA actually applies, (hi + lo) / v_scale * 2^-k, not p:
      // the output is then an exact convex combination of V rows under those
      // weights, so a row dominated by one key returns that key's V without
      // the split's 2^-9 error.
      i32x8 p8h[kPBlocks], p8l[kPBlocks];
      float m_use[kPBlocks], lsum[kPBlocks];
      int kr[kPBlocks];
#pragma unroll
      for (int b = 0; b < kPBlocks; ++b) {
        const float kf =
            tm[b] == -INFINITY ? 0.0f : fminf(floorf(m[b] - tm[b]), 127.0f);
        kr[b] = (int)kf;
        m_use[b] = (m[b] == -INFINITY ? 0.0f : m[b]) - lf - kf;
        lsum[b] = 0.0f;
      }
      // 1 / v_scale of the tile's keys, computed once per key by this wave
      // (lane i: keys i and 64 + i) instead of once per lane group, and read
      // back below like the scales.  v_scale is 0 only for keys past
      // `valid`, whose weights are 0.  The wave reads back only its own
      // writes, so a wave-level barrier orders them.
      // A key whose v_scale * fcur is below kPTinyV (V amax under ~1/1500 of
      // the tile's largest, e.g. a V row stored as zeros) would get weights
      // p * v_scale too small for e4m3 to carry, and its probability would
      // drop out of l.  Its reciprocal is 0 instead, and its exact weight
      // joins l on the rare path below.  Its V contribution stays with the
      // MFMA, which it changes by at most p / 1500 of the tile's largest |V|.
      float* rvw = rv_lds[wave];
      bool tiny_keys;
      {
        const float v0 = vss[lane], v1 = vss[64 + lane];
        const bool t0 = v0 > 0.0f && v0 * fcur < kPTinyV;
        const bool t1 = v1 > 0.0f && v1 * fcur < kPTinyV;
        rvw[lane] = v0 > 0.0f && !t0 ? __builtin_amdgcn_rcpf(v0) : 0.0f;
        rvw[64 + lane] = v1 > 0.0f && !t1 ? __builtin_amdgcn_rcpf(v1) : 0.0f;
        tiny_keys = __any(t0 || t1);
        __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
        __builtin_amdgcn_wave_barrier();
        __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
      }
      if (tiny_keys) {
#pragma unroll
        for (int tt = 0; tt < 8; ++tt) {
          const f32x4 vsc = *reinterpret_cast<const f32x4*>(vss + 16 * tt + 4 * g);
#pragma unroll
          for (int r = 0; r < 4; ++r) {
            if (vsc[r] > 0.0f && vsc[r] * fcur < kPTinyV) {
#pragma unroll
              for (int b = 0; b < kPBlocks; ++b) {
                // opaque to the optimizer: shared with the loop below, these
                // exps would be hoisted out of the loop's MFMA interleave
                float x = fmaf(st[b][tt][r], qs[b], -m_use[b]);
                asm volatile("" : "+v"(x));
                lsum[b] += exp2_fast(x);
              }
            }
          }
        }
      }
      typedef float f32x2 __attribute__((ext_vector_type(2)));
      // The wave raises its priority over the P loop and the PV MFMAs and
      // drops it after: bf16 1.9% and fp16 0.6% faster.
      __builtin_amdgcn_s_setprio(1);
      if constexpr (NQ == 3) {
        // fp16: the third query part takes the registers of one block's P
        // operands, so each block computes its P and runs its PV MFMAs in
        // turn, reading V^T once per block
#pragma unroll
        for (int b = 0; b < kPBlocks; ++b) {
          i32x8 ph, pl;
#pragma unroll
          for (int tt = 0; tt < 8; ++tt) {
            const f32x4 vsc = *reinterpret_cast<const f32x4*>(vss + 16 * tt + 4 * g);
            const f32x4 rv = *reinterpret_cast<const f32x4*>(rvw + 16 * tt + 4 * g);
            float y[4];
#pragma unroll
            for (int r = 0; r < 4; ++r)
              y[r] = exp2_fast(fmaf(st[b][tt][r], qs[b], -m_use[b])) * vsc[r];
            const uint32_t h = pack_fp8x4(y[0], y[1], y[2], y[3]);
            const f32x2 h01 = __builtin_amdgcn_cvt_pk_f32_fp8((int)h, false);
            const f32x2 h23 = __builtin_amdgcn_cvt_pk_f32_fp8((int)h, true);
            const uint32_t lo = pack_fp8x4(y[0] - h01[0], y[1] - h01[1], y[2] - h23[0],
                                           y[3] - h23[1]);
            const f32x2 l01 = __builtin_amdgcn_cvt_pk_f32_fp8((int)lo, false);
            const f32x2 l23 = __builtin_amdgcn_cvt_pk_f32_fp8((int)lo, true);
            lsum[b] = fmaf(h01[0] + l01[0], rv[0], lsum[b]);
            lsum[b] = fmaf(h01[1] + l01[1], rv[1], lsum[b]);
            lsum[b] = fmaf(h23[0] + l23[0], rv[2], lsum[b]);
            lsum[b] = fmaf(h23[1] + l23[1], rv[3], lsum[b]);
            ph[tt] = (int)h;
            pl[tt] = (int)lo;
          }
          l[b] += __builtin_amdgcn_ldexpf(lsum[b], -kr[b]);
#pragma unroll
          for (int dt = 0; dt < 8; ++dt) {
            i32x8 va;
#pragma unroll
            for (int qq = 0; qq < 4; ++qq) {
              const i32x2 r = __builtin_amdgcn_ds_read_tr8_b64_v2i32(
                  reinterpret_cast<__attribute__((address_space(3))) i32x2*>(
                      (__attribute__((address_space(3))) uint8_t*)vt + tr_row[qq] +
                      ((16u * dt) ^ tr_swz[qq])));
              va[2 * qq] = r[0];
              va[2 * qq + 1] = r[1];
            }
            acc[b][dt] = mfma_fp8_scale_b(va, ph, acc[b][dt], 127 - kr[b]);
            acc[b][dt] = mfma_fp8_scale_b(va, pl, acc[b][dt], 127 - kr[b]);
          }
          // keep the next block's P work out of this block's PV
          __builtin_amdgcn_sched_barrier(0);
        }
      } else {
  #pragma unroll
        for (int tt = 0; tt < 8; ++tt) {
          const f32x4 vsc = *reinterpret_cast<const f32x4*>(vss + 16 * tt + 4 * g);
          const f32x4 rv = *reinterpret_cast<const f32x4*>(rvw + 16 * tt + 4 * g);
  #pragma unroll
          for (int b = 0; b < kPBlocks; ++b) {
            float y[4];
  #pragma unroll
            for (int r = 0; r < 4; ++r)
              y[r] = exp2_fast(fmaf(st[b][tt][r], qs[b], -m_use[b])) * vsc[r];
            const uint32_t h = pack_fp8x4(y[0], y[1], y[2], y[3]);
            const f32x2 h01 = __builtin_amdgcn_cvt_pk_f32_fp8((int)h, false);
            const f32x2 h23 = __builtin_amdgcn_cvt_pk_f32_fp8((int)h, true);
            const uint32_t lo = pack_fp8x4(y[0] - h01[0], y[1] - h01[1], y[2] - h23[0],
                                           y[3] - h23[1]);
            const f32x2 l01 = __builtin_amdgcn_cvt_pk_f32_fp8((int)lo, false);
            const f32x2 l23 = __builtin_amdgcn_cvt_pk_f32_fp8((int)lo, true);
            lsum[b] = fmaf(h01[0] + l01[0], rv[0], lsum[b]);
            lsum[b] = fmaf(h01[1] + l01[1], rv[1], lsum[b]);
            lsum[b] = fmaf(h23[0] + l23[0], rv[2], lsum[b]);
            lsum[b] = fmaf(h23[1] + l23[1], rv[3], lsum[b]);
            p8h[b][tt] = (int)h;
            p8l[b][tt] = (int)lo;
          }
        }
  #pragma unroll
        for (int b = 0; b < kPBlocks; ++b) l[b] += __builtin_amdgcn_ldexpf(lsum[b], -kr[b]);
        // O^T += V^T . P8^T, one 16-wide d tile per MFMA pair
  #pragma unroll
        for (int dt = 0; dt < 8; ++dt) {
          i32x8 va;
  #pragma unroll
          for (int qq = 0; qq < 4; ++qq) {
            const i32x2 r = __builtin_amdgcn_ds_read_tr8_b64_v2i32(
                reinterpret_cast<__attribute__((address_space(3))) i32x2*>(
                    (__attribute__((address_space(3))) uint8_t*)vt + tr_row[qq] +
                    ((16u * dt) ^ tr_swz[qq])));
            va[2 * qq] = r[0];
            va[2 * qq + 1] = r[1];
          }
  #pragma unroll
          for (int b = 0; b < kPBlocks; ++b) {
            acc[b][dt] = mfma_fp8_scale_b(va, p8h[b], acc[b][dt], 127 - kr[b]);
            acc[b][dt] = mfma_fp8_scale_b(va, p8l[b], acc[b][dt], 127 - kr[b]);
          }
        }
      }
      __builtin_amdgcn_s_setprio(0);
    }
  };

  int valid = stage_tile(0, k_lds0, v_lds0, sc_lds0);
  __syncthreads();
  for (int t0 = 0; t0 < kv_end; t0 += 2 * kPStep) {
    {
      const bool more = t0 + kPStep < kv_end;
      const int valid_next = more ? stage_tile(t0 + kPStep, k_lds1, v_lds1, sc_lds1) : 0;
      compute_tile(t0, valid, k_lds0, v_lds0, sc_lds0);
      __syncthreads();  // also waits for this wave's direct loads
      valid = valid_next;
      if (!more) break;
    }
    {
      const int t1 = t0 + kPStep;
      const bool more = t1 + kPStep < kv_end;
      const int valid_next = more ? stage_tile(t1 + kPStep, k_lds0, v_lds0, sc_lds0) : 0;
      compute_tile(t1, valid, k_lds1, v_lds1, sc_lds1);
      __syncthreads();
      valid = valid_next;
    }
  }

#pragma unroll
  for (int b = 0; b < kPBlocks; ++b) {
    const float lt = sum_xor32(sum_xor16(l[b]));
    if (!row_ok[b]) continue;
    const float scale = lt > 0.0f ? 1.0f / lt : 0.0f;
    uint16_t* op = a.out + ((int64_t)(q_begin + w_q0 + b * a.tpr + n / a.gc) * a.hq + qh[b]) * kHeadDim;
#pragma unroll
    for (int dt = 0; dt < 8; ++dt) {
      const f32x4 o = acc[b][dt] * scale;
      const uint32_t lo = (uint32_t)A::from_f32(o[0]) | ((uint32_t)A::from_f32(o[1]) << 16);
      const uint32_t hi = (uint32_t)A::from_f32(o[2]) | ((uint32_t)A::from_f32(o[3]) << 16);
      *reinterpret_cast<u32x2*>(op + 16 * dt + 4 * g) = u32x2{lo, hi};
    }
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
  const int per_wg = 8 * a.tpr;  // 128 rows: 8 blocks of 16 rows
  // grid y and z are limited to 65535
  const int64_t qblocks = ((int64_t)max_seqlen_q + per_wg - 1) / per_wg;
  if (num_seqs > 65535 || qblocks > 65535) return MSKV_EUNSUPPORTED;
  const dim3 grid((unsigned)(num_kv_heads * a.qgroups), (unsigned)num_seqs,
                  (unsigned)qblocks);
  hipStream_t s = reinterpret_cast<hipStream_t>(stream);
  if (act_dtype == MSKV_BFLOAT16)
    hipLaunchKernelGGL(mskv::prefill_fp8_kernel<__bf16>, grid,
                       dim3(mskv::PShapeOf<__bf16>::threads), 0, s, a);
  else
    hipLaunchKernelGGL(mskv::prefill_fp8_kernel<_Float16>, grid,
                       dim3(mskv::PShapeOf<_Float16>::threads), 0, s, a);
  return (int)hipGetLastError();
}
