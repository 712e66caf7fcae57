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
//    read it.  Four waves of two 16-row blocks, so every K and V^T operand a
//    wave reads from LDS (and converts) feeds both.
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
//  * PV: O^T = V^T . P^T with v_mfma_f32_16x16x32_f16, which runs at the
//    same rate per key as two FP8 parts would.  S^T's accumulator leaves
//    lane (g, n) holding 32 keys of row n, exactly the B-operand layout of
//    P^T, so probabilities never move between lanes; V^T comes out of LDS
//    with ds_read_b64_tr_b8 and converts to fp16 exactly.  Each weight is
//    fp16(p) * fp16(v_scale * fw) (v_pk_mul_f16), fw a per-wave power of
//    two set from the largest v_scale seen (it only shrinks).  A key whose
//    v_scale lies within 2^21 of that largest one gets a normal fp16 scale
//    (11 significant bits), however the scales spread inside a tile; one
//    further below gets a subnormal scale, with fewer bits (and below
//    ~2^32, zero), and a small p lowers that bound further.  The
//    softmax denominator is a ninth output tile: an all-ones A operand
//    against the fp16 probabilities, summed in fp32 by the MFMA.
//  * Online softmax in base 2 with a lazy rescale: the accumulator is
//    rescaled only when some row's max grows by more than 2^8, which a wave
//    vote on each lane's own scores decides before any cross-lane
//    reduction; the weight scale fw is checked the same way.  Masks are
//    evaluated only on tiles that straddle the causal diagonal or the end
//    of the keys; fully visible tiles skip them.
//  * Query blocks are launched last-first across the whole grid, so the
//    longest workgroups of every sequence start before any shorter one.
//    Pages are read through page-sized buffer resources; an invalid block
//    id gives zero-length reads and its keys are masked.
#include <float.h>
#include <math.h>

#include "mskv_device.h"
#include "../../include/mskv.h"

namespace mskv {

constexpr int kPStep = 128;  // keys per tile
// A workgroup covers 128 rows: 4 waves of two 16-row blocks.
struct PShape {
  static constexpr int blocks = 2;  // 16-row blocks per wave
  static constexpr int waves = 8 / blocks;
  static constexpr int threads = 64 * waves;
};
// The running max may lag a row's true max by up to kPSlack (log2 units)
// before the accumulator is rescaled, so p stays below 2^8.
constexpr float kPSlack = 8.0f;
// Largest v_scale * fw: a weight p * v_scale * fw with p <= 2^8 then stays
// below 2^15, inside fp16's range.
constexpr float kPVScaleMax = 128.0f;

// e4m3 parts the query is split into: a bf16 value has 8 significant bits
template <typename T> struct QuerySplit { static constexpr int parts = 3; };
template <> struct QuerySplit<__bf16> { static constexpr int parts = 2; };

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
  int gc_magic;  // ceil(256 / gc): n / gc == (n * gc_magic) >> 8 for n < 16
  float scale_log2;
};

__device__ __forceinline__ f32x4 mfma_fp8(const i32x8& a, const i32x8& b, f32x4 c) {
  // compile-time zero scales select the unscaled v_mfma_f32_16x16x128_f8f6f4
  return __builtin_amdgcn_mfma_scale_f32_16x16x128_f8f6f4(a, b, c, 0, 0, 0, 0, 0, 0);
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
__global__ __launch_bounds__(PShape::threads, 2) void prefill_fp8_kernel(PrefillArgs a) {
  using A = Act<T>;
  constexpr int NQ = QuerySplit<T>::parts;
  constexpr int kPBlocks = PShape::blocks;
  constexpr int kPWaves = PShape::waves;
  // two tile buffers as separate objects, and a loop unrolled by two, so
  // the compiler can see that the direct loads into one buffer never alias
  // the reads of the other (otherwise it waits for them before every read)
  __shared__ __attribute__((aligned(16))) uint8_t k_lds0[kPStep * kHeadDim];
  __shared__ __attribute__((aligned(16))) uint8_t v_lds0[kPStep * kHeadDim];
  __shared__ __attribute__((aligned(16))) uint8_t k_lds1[kPStep * kHeadDim];
  __shared__ __attribute__((aligned(16))) uint8_t v_lds1[kPStep * kHeadDim];
  __shared__ __attribute__((aligned(16))) float sc_lds0[2][kPStep];
  __shared__ __attribute__((aligned(16))) float sc_lds1[2][kPStep];
  // each wave's fp16 v_scale * fw of the current tile's keys
  __shared__ __attribute__((aligned(16))) _Float16 vsf_lds[kPWaves][kPStep];

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
    const int nq = (n * a.gc_magic) >> 8;  // n / gc
    const int qi = w_q0 + b * a.tpr + nq;
    // a unit of a group above 16 that is not a multiple of 16 has idle
    // lanes past the group's last head
    row_ok[b] = n < a.tpr * a.gc && qi < lq && qgi * 16 + n - nq * a.gc < a.group;
    qh[b] = kvh * a.group + qgi * 16 + n - nq * a.gc;
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

  // acc: O^T in units of fw, the power-of-two scale applied to v_scale (0
  // until the first tile with a stored token sets it); lacc: the softmax
  // denominator, as the output tile of an all-ones A operand against P^T,
  // so every row of it holds its column's sum of the fp16 probabilities
  f32x4 acc[kPBlocks][8], lacc[kPBlocks];
  float m[kPBlocks];
#pragma unroll
  for (int b = 0; b < kPBlocks; ++b) {
#pragma unroll
    for (int dt = 0; dt < 8; ++dt) acc[b][dt] = f32x4{0.f, 0.f, 0.f, 0.f};
    lacc[b] = f32x4{0.f, 0.f, 0.f, 0.f};
    // -FLT_MAX rather than -inf: a row that has seen no key yet keeps it,
    // and its masked (-inf) scores still give p = 0 with no select; the
    // first finite score raises it like any other growth
    m[b] = -FLT_MAX;
  }
  float fw = 0.0f;
  f16x8 ones;
#pragma unroll
  for (int i = 0; i < 8; ++i) ones[i] = (_Float16)1.0f;

  // K operand: key n of each 16-key group, 16-byte chunks 2g and 2g + 1;
  // the swizzle of rows 16t + n does not depend on t
  const uint32_t k_lo = tile_off(n, 2 * g), k_hi = tile_off(n, 2 * g + 1);
  // ds_read_b64_tr_b8 address of this lane for read qq (keys 8qq..8qq+7 of
  // the lane group's 32): key slot e = 8qq + i/2 maps to tile row
  // 16*(e/4) + 4g + e%4, column half i%2.  Read qq's row is read 0's plus
  // 32qq, so its address is read 0's plus 4096qq (an immediate offset), and
  // bits 1-3 of the row, which select the swizzle, do not depend on qq.
  const int i16 = lane & 15;
  const int tr_r0 = 16 * (i16 >> 3) + 4 * g + ((i16 >> 1) & 3);
  const uint32_t tr_row = (uint32_t)tr_r0 * kHeadDim + 8u * (i16 & 1);
  const uint32_t tr_swz = 16u * (uint32_t)((tr_r0 >> 1) & 7);

  const uint32_t page_bytes = (uint32_t)a.bs * a.hk * kHeadDim;
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
      // Row maxima in log2 units (qs > 0 per row).  Each lane tests its own
      // 32 scores against the row's running max: a row's maximum is the
      // largest of its four lanes', and the positive scale keeps the order,
      // so the wave vote equals the test on the row maxima, and the
      // cross-lane reduction runs only when the vote passes.
      float lm[kPBlocks];
      bool grow = false;
#pragma unroll
      for (int b = 0; b < kPBlocks; ++b) {
        float v = fmaxf(fmaxf(st[b][0][0], st[b][0][1]), fmaxf(st[b][0][2], st[b][0][3]));
#pragma unroll
        for (int tt = 1; tt < 8; ++tt)
          v = fmaxf(fmaxf(v, st[b][tt][0]), fmaxf(fmaxf(st[b][tt][1], st[b][tt][2]), st[b][tt][3]));
        lm[b] = v;
        grow |= v * qs[b] > m[b] + kPSlack;
      }
      if (__any(grow)) {
#pragma unroll
        for (int b = 0; b < kPBlocks; ++b) {
          const float m_new = fmaxf(m[b], max_xor32(max_xor16(lm[b])) * qs[b]);
          const float alpha = exp2_fast(m[b] - m_new);
          lacc[b] *= alpha;
#pragma unroll
          for (int dt = 0; dt < 8; ++dt) acc[b][dt] *= alpha;
          m[b] = m_new;
        }
      }
      // The PV product runs on v_mfma_f32_16x16x32_f16.  V converts to fp16
      // exactly, and each weight is fp16(p) * fp16(v_scale * fw), formed in
      // pairs by v_pk_mul_f16.  fw is a power of two per wave, set from the
      // largest v_scale the wave has seen: v_scale * fw <= kPVScaleMax, so
      // with p <= 2^8 (the lazy rescale's slack) no weight leaves fp16's
      // range (the bound on the smaller keys' precision is in the header).
      // It only ever shrinks, and the accumulator is then rescaled
      // by the exact ratio; the output is divided by it at the end.
      // A wave vote on the lanes' own keys skips the tile's v_scale maximum
      // while every key fits under fw (a NaN scale fails the test and takes
      // the exact path, whose maximum ignores it).
      {
        const float v0 = vss[lane], v1 = vss[64 + lane];
        if (__any(!(v0 * fw <= kPVScaleMax) || !(v1 * fw <= kPVScaleMax)) || fw == 0.0f) {
          const float vm = max_xor32(max_xor16(max16_dpp(fmaxf(v0, v1))));
          if (vm > 0.0f && (fw == 0.0f || vm * fw > kPVScaleMax)) {
            const float fnew = pow2_floor(kPVScaleMax / vm);
            if (fw != 0.0f) {
              const float r = fnew / fw;  // a power of two: exact
#pragma unroll
              for (int b = 0; b < kPBlocks; ++b)
#pragma unroll
                for (int dt = 0; dt < 8; ++dt) acc[b][dt] *= r;
            }
            fw = fnew;
          }
        }
      }
      // fp16(v_scale * fw) of the tile's keys, computed once per key by
      // this wave (lane i: keys i and 64 + i) and read back in groups of
      // four; the wave reads only its own writes, so a wave-level barrier
      // orders them
      _Float16* vsw = vsf_lds[wave];
      vsw[lane] = (_Float16)(vss[lane] * fw);
      vsw[64 + lane] = (_Float16)(vss[64 + lane] * fw);
      __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
      __builtin_amdgcn_wave_barrier();
      __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
      // The wave raises its priority over the P loop and the PV MFMAs and
      // drops it after.
      __builtin_amdgcn_s_setprio(1);
      // P^T for the f16 MFMA: 32-key chunk c of the tile is S^T tiles 2c and
      // 2c + 1, so lane (g, n) holds keys 32c + 4g + r and 32c + 16 + 4g + r
      // of row n -- the order in which ds_read_b64_tr_b8 hands it V^T
      // Each 16-key group's scales are read once for both blocks, one group
      // ahead: read per block and group, every read's LDS latency was
      // exposed.  The denominator's MFMA for a chunk follows its probabilities.
      typedef _Float16 f16x4 __attribute__((ext_vector_type(4)));
      f16x8 pw[kPBlocks][4];
      f16x4 vsf_next = *reinterpret_cast<const f16x4*>(vsw + 4 * g);
#pragma unroll
      for (int c = 0; c < 4; ++c) {
        f16x8 pc[kPBlocks];
#pragma unroll
        for (int h = 0; h < 2; ++h) {
          const int tt = 2 * c + h;
          const f16x4 vf = vsf_next;
          if (tt < 7) vsf_next = *reinterpret_cast<const f16x4*>(vsw + 16 * (tt + 1) + 4 * g);
#pragma unroll
          for (int b = 0; b < kPBlocks; ++b) {
            float pf[4];
#pragma unroll
            for (int r = 0; r < 4; ++r) pf[r] = exp2_fast(fmaf(st[b][tt][r], qs[b], -m[b]));
            const f16x2 p01 = {(_Float16)pf[0], (_Float16)pf[1]};
            const f16x2 p23 = {(_Float16)pf[2], (_Float16)pf[3]};
            const f16x2 w01 = p01 * f16x2{vf[0], vf[1]};
            const f16x2 w23 = p23 * f16x2{vf[2], vf[3]};
            pc[b][4 * h + 0] = p01[0];
            pc[b][4 * h + 1] = p01[1];
            pc[b][4 * h + 2] = p23[0];
            pc[b][4 * h + 3] = p23[1];
            pw[b][c][4 * h + 0] = w01[0];
            pw[b][c][4 * h + 1] = w01[1];
            pw[b][c][4 * h + 2] = w23[0];
            pw[b][c][4 * h + 3] = w23[1];
          }
        }
#pragma unroll
        for (int b = 0; b < kPBlocks; ++b)
          lacc[b] = __builtin_amdgcn_mfma_f32_16x16x32_f16(ones, pc[b], lacc[b], 0, 0, 0);
      }
      // O^T += V^T . P^T, one 16-wide d tile and 32-key chunk per MFMA.  The
      // V^T reads of d tile dt + 1 are issued before the MFMAs of tile dt:
      // with one read in flight, each chunk's LDS latency sat behind only
      // two 16-cycle MFMAs.
      auto vread = [&](int dt, int c) {
        return __builtin_amdgcn_ds_read_tr8_b64_v2i32(
            reinterpret_cast<__attribute__((address_space(3))) i32x2*>(
                (__attribute__((address_space(3))) uint8_t*)vt +
                (tr_row + ((16u * dt) ^ tr_swz)) + 4096u * c));
      };
      i32x2 raw[4];
#pragma unroll
      for (int c = 0; c < 4; ++c) raw[c] = vread(0, c);
#pragma unroll
      for (int dt = 0; dt < 8; ++dt) {
        i32x2 nxt[4];
#pragma unroll
        for (int c = 0; c < 4; ++c) nxt[c] = vread(dt < 7 ? dt + 1 : dt, c);
#pragma unroll
        for (int c = 0; c < 4; ++c) {
          const f16x8 va = fp8x8_to_f16((uint32_t)raw[c][0], (uint32_t)raw[c][1]);
#pragma unroll
          for (int b = 0; b < kPBlocks; ++b)
            acc[b][dt] = __builtin_amdgcn_mfma_f32_16x16x32_f16(va, pw[b][c], acc[b][dt], 0, 0, 0);
        }
#pragma unroll
        for (int c = 0; c < 4; ++c) raw[c] = nxt[c];
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

  // The rows' coordinates are recomputed from the lane id rather than kept
  // live across the loop, which would spill them.
  int n_out = lane & 15;
  asm volatile("" : "+v"(n_out));
#pragma unroll
  for (int b = 0; b < kPBlocks; ++b) {
    const float lt = lacc[b][0];
    const int nq = (n_out * a.gc_magic) >> 8;  // n / gc
    const int qi = w_q0 + b * a.tpr + nq;
    if (!(n_out < a.tpr * a.gc && qi < lq && qgi * 16 + n_out - nq * a.gc < a.group)) continue;
    // acc is in units of fw (a power of two): 1 / fw is exact
    const float scale = lt > 0.0f && fw > 0.0f ? (1.0f / lt) * (1.0f / fw) : 0.0f;
    const int qhb = kvh * a.group + qgi * 16 + n_out - nq * a.gc;
    uint16_t* op = a.out + ((int64_t)(q_begin + qi) * a.hq + qhb) * kHeadDim;
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
  if (head_dim != mskv::kHeadDim || block_size % mskv::kPStep != 0) return MSKV_EUNSUPPORTED;
  // the row maxima are taken before the scale, which must keep their order
  const float scale_log2 = softmax_scale * mskv::kLog2e;
  if (!(scale_log2 > 0.0f && scale_log2 < INFINITY)) return MSKV_EUNSUPPORTED;
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
  a.qgroups = (group + 15) / 16;
  a.tpr = 16 / a.gc;
  a.gc_magic = (256 + a.gc - 1) / a.gc;
  a.bs = block_size;
  a.w = max_blocks_per_seq;
  a.scale_log2 = scale_log2;
  const int per_wg = 8 * a.tpr;  // 128 rows: 8 blocks of 16 rows
  // grid y and z are limited to 65535
  const int64_t qblocks = ((int64_t)max_seqlen_q + per_wg - 1) / per_wg;
  if (num_seqs > 65535 || qblocks > 65535) return MSKV_EUNSUPPORTED;
  const dim3 grid((unsigned)(num_kv_heads * a.qgroups), (unsigned)num_seqs,
                  (unsigned)qblocks);
  hipStream_t s = reinterpret_cast<hipStream_t>(stream);
  if (act_dtype == MSKV_BFLOAT16)
    hipLaunchKernelGGL(mskv::prefill_fp8_kernel<__bf16>, grid,
                       dim3(mskv::PShape::threads), 0, s, a);
  else
    hipLaunchKernelGGL(mskv::prefill_fp8_kernel<_Float16>, grid,
                       dim3(mskv::PShape::threads), 0, s, a);
  return (int)hipGetLastError();
}
