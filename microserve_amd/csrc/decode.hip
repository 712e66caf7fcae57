// Paged decode attention over the FP8 e4m3fn cache, split-KV + LSE combine.
//
// Semantics follow microserve/layers/fp8_decode_attention.py:16-58: q head h
// reads kv head h / group; token p of sequence b is cache row
// block_tables[b][p / BS] * BS + p % BS; score = (q . k8) * k_scale *
// softmax_scale; out = sum softmax * v8 * v_scale; zeros when seq_len == 0.
//
// MI355X design (one wave per (sequence, kv head, split)):
//  * K/V are read once per kv head: the whole GQA group of q heads (up to
//    16) rides in the N dimension of the MFMAs.
//  * K and V rows are read from HBM fully coalesced (eight lanes per
//    128-byte row, streaming cache policy) and staged in a per-wave LDS
//    tile; the MFMA operand layouts come back out of LDS.  Loading K
//    straight into the MFMA layout puts four tokens (four lines) in every
//    quad of lanes and measured ~8% slower.
//  * QK^T runs as S^T = K . Q^T on v_mfma_f32_16x16x32_{bf16,f16}: lane
//    (g, i) reads token i, bytes [16g,16g+16) and [64+16g,64+16g+16) of the
//    K tile and converts them to the query's 16-bit type exactly (e4m3 is a
//    subset of fp16 and bf16); Q uses the same d permutation, so the
//    contraction is the plain dot product.
//  * The S^T accumulator leaves lane (g, n) holding tokens {4g+r, 16+4g+r}
//    of head n -- exactly the B-operand layout of O^T = V^T . P^T, so the
//    probabilities never move between lanes.  P is scaled by the per-token
//    v_scale and a per-wave power of two and rounded to fp16 for the PV
//    MFMA.  The power of two keeps fp16's range; a token whose v_scale lies
//    within 2^21 of the largest the wave has seen keeps 11 significant
//    bits, one further below gets a subnormal weight with fewer.
//  * V^T's A operand needs eight tokens per lane at one d: it comes back
//    out of the V tile transposed with ds_read_b64_tr_b8, then is converted
//    fp8 -> fp16 (exact) in registers.
//  * Tile rows are stored with their 16-byte chunks XOR-swizzled by
//    (row / 2) % 8, which keeps the row-major writes and the K reads free
//    of LDS bank conflicts; the transposed V reads are 2-way (rows r and
//    r + 16 share banks), which this HBM-bound kernel does not feel.
//  * Online softmax in base 2 (v_exp_f32); the row max is a two-step xor
//    reduction (v_permlane16/32_swap, no LDS round trip) across the four
//    lane groups that share a head, and the accumulator is rescaled lazily,
//    only when a head's max grows by more than 2^8.
//  * Tiles are double-buffered in LDS: step i+1's rows are staged while
//    step i is consumed, so the K/V registers live only while in flight.
//  * Split-KV: the host picks pages-per-split from shapes only; each split
//    writes (o / l, m + log2 l) partials and a second kernel merges them:
//    decode_combine_small_kernel up to 8 splits, decode_combine_kernel up
//    to 64, decode_combine_wide_kernel beyond (an in-kernel merge needs
//    agent-scope fences, i.e. an L2 writeback + invalidate per XCD, which
//    measured 2x slower).  A sequence that fits in one split is written
//    directly by the split kernel.
//  * Grids of many rounds (over 512 eight-wave workgroups) run compacted
//    work items longest-first: a pre-pass ranks the sequences by length on
//    the device and lists their valid splits, so short sequences fill the
//    last round and empty splits exit at the end of the grid.
//  * Two workgroup shapes, chosen from shapes alone: 8 waves (all 8 kv
//    heads of a token range, whole 1 KiB token rows, 132 KB of LDS: one per
//    CU), and 4 waves (half a token row each, two per CU) for grids of many
//    rounds without work items (past the items' limits, or fewer than 8
//    units per kv head group), whose smaller last round halves the tail.
//  * Every page is read through a buffer resource sized to that page; an
//    invalid block id gives a zero-length resource (loads return 0) and its
//    tokens are masked, so a bad table entry cannot fault.
#include <math.h>

#include <mutex>

#include "mskv_device.h"
#include "../../include/mskv.h"

namespace mskv {

constexpr int kStep = 32;  // tokens per inner step (one LDS K/V tile pair)
// p * v_scale is scaled so the largest v_scale maps to at most this: with
// p < 2^8 every weight stays below 2^15, inside fp16's range
constexpr float kPvScaleMax = 128.0f;
constexpr int kMaxPagesPerSplit = 4;
// Split-KV aims at this many waves: eight per CU
constexpr int kTargetWaves = 2048;
// Waves of one workgroup take consecutive kv heads of the same tokens, so a
// workgroup streams whole contiguous token rows; the waves never synchronize
// with each other.
constexpr int kWavesPerWG = 8;
constexpr int kNarrowWaves = 4;       // workgroup shape for grids of many rounds
constexpr int64_t kWideGridMax = 512; // 8-wave workgroups: about two rounds
// Largest split-partials scratch the allocation-free entry point serves
constexpr size_t kNoAllocScratchBytes = MSKV_DECODE_NOALLOC_SCRATCH_BYTES;

// Orders this wave's LDS writes before its later LDS reads (LDS executes one
// wave's instructions in issue order, so no workgroup barrier is needed).
__device__ __forceinline__ void wave_lds_sync() {
  __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
  __builtin_amdgcn_wave_barrier();
  __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
}

struct DecodeArgs {
  const uint16_t* q;
  const uint8_t* kc;
  const uint8_t* vc;
  const float* ks;
  const float* vs;
  const int32_t* seqlens;
  const int32_t* bt;
  uint16_t* out;
  float* part_o;
  float* part_lse;
  // Work items longest-first (grids of many rounds, else null): item i is
  // (sequence, split, length, block id of the split's first page), for
  // the valid splits of the sequences in order of decreasing length, and
  // item_count of them are valid.
  const int4* items;
  const int* item_count;
  int batch, hq, hk, group, qgroups, bs, w, splits, pages_per_split;
  int64_t num_blocks;
  float scale_log2;
};

struct StepLoads {
  u32x4 k[4], v[4];      // K/V rows 8c + lane/8, 16-byte chunk lane%8
  float kscale, vscale;  // scales of token lane & 31
  int valid;             // tokens of this step below the sequence end
};


// Issues the loads of the step at token t0, whose page holds block `blk`.
__device__ __forceinline__ void load_step(const DecodeArgs& a, int blk, int kvh, int t0,
                                          int t_end, int lane, StepLoads& s) {
  const int page = t0 / a.bs;
  const int off = t0 - page * a.bs;
  const bool ok = blk >= 0 && (int64_t)blk < a.num_blocks;
  const int64_t bo = ok ? blk : 0;
  const uint32_t page_bytes = (uint32_t)a.bs * a.hk * kHeadDim;
  const uint32_t spage_bytes = (uint32_t)a.bs * a.hk * 4u;
  const auto kr = make_rsrc(a.kc + bo * page_bytes, ok ? page_bytes : 0u);
  const auto vr = make_rsrc(a.vc + bo * page_bytes, ok ? page_bytes : 0u);
  const auto ksr = make_rsrc(a.ks + bo * a.bs * a.hk, ok ? spage_bytes : 0u);
  const auto vsr = make_rsrc(a.vs + bo * a.bs * a.hk, ok ? spage_bytes : 0u);
  const uint32_t rstride = (uint32_t)a.hk * kHeadDim;
  const uint32_t base = (uint32_t)off * rstride + (uint32_t)kvh * kHeadDim;
  const uint32_t rb = base + (uint32_t)(lane >> 3) * rstride + 16u * (lane & 7);
#pragma unroll
  for (int c = 0; c < 4; ++c) s.k[c] = buf_load16_nt(kr, rb + 8u * c * rstride);
#pragma unroll
  for (int c = 0; c < 4; ++c) s.v[c] = buf_load16_nt(vr, rb + 8u * c * rstride);
  const uint32_t so = (((uint32_t)off + (lane & 31)) * a.hk + kvh) * 4u;
  s.kscale = buf_load_f32(ksr, so);
  s.vscale = buf_load_f32(vsr, so);
  s.valid = ok ? min(kStep, t_end - t0) : 0;
}

// One wave's online softmax over the token range [t_begin, t_end) of
// sequence b for kv head kvh (q head qh of the lane's column): returns the
// un-normalized accumulator O^T, the running max m (log2 units) and the
// lane's share of the denominator l.  kv_lds / s_lds are this wave's own
// double-buffered LDS tiles; blk_first is the block of t_begin's page.
template <typename T>
__device__ __forceinline__ void attend_range(const DecodeArgs& a, int b, int kvh, int qh,
                                             bool head_ok, int t_begin, int t_end,
                                             int blk_first, int lane,
                                             uint8_t (&kv_lds)[2][2][kStep * kHeadDim],
                                             float (&s_lds)[2][2 * kStep], f32x4 (&acc)[8],
                                             float& m, float& l) {
  using A = Act<T>;
  using x8 = typename A::x8;
  const int g = lane >> 4, n = lane & 15;

  // Q^T as the B operand: lane (g, n) holds head n at d in
  // [16g, 16g+16) and [64+16g, 64+16g+16), eight per MFMA k-step.
  x8 qop[4];
  if (head_ok) {
    const u32x4* qp =
        reinterpret_cast<const u32x4*>(a.q + ((int64_t)b * a.hq + qh) * kHeadDim);
    qop[0] = __builtin_bit_cast(x8, qp[2 * g]);
    qop[1] = __builtin_bit_cast(x8, qp[2 * g + 1]);
    qop[2] = __builtin_bit_cast(x8, qp[8 + 2 * g]);
    qop[3] = __builtin_bit_cast(x8, qp[9 + 2 * g]);
  } else {
#pragma unroll
    for (int j = 0; j < 4; ++j) qop[j] = __builtin_bit_cast(x8, u32x4{0u, 0u, 0u, 0u});
  }

#pragma unroll
  for (int dt = 0; dt < 8; ++dt) acc[dt] = f32x4{0.f, 0.f, 0.f, 0.f};
  m = -INFINITY;
  l = 0.0f;
  // The PV operand is fp16(p * v_scale * f): f is a power of two with
  // v_scale * f <= kPvScaleMax for every valid token seen so far, so every
  // weight stays within fp16's range (p < 2^8 under the lazy rescale).  A
  // weight keeps fp16's 11 significant bits while p * v_scale * f stays
  // above fp16's smallest normal, 2^-14; acc is in units of f, rescaled
  // exactly when f shrinks.
  float f = 0.0f, vseen = 0.0f;

  // ds_read_b64_tr_b8: in each 16-lane group, result byte e of lane i comes
  // from the address supplied by lane 2e + i/8, plus i%8.  Lane i therefore
  // supplies token slot e = i/2 at column half i%2.
  const int i16 = lane & 15;
  const int slot = i16 >> 1;
  const int trow = slot < 4 ? 4 * g + slot : 16 + 4 * g + (slot - 4);
  const uint32_t tr_base = (uint32_t)trow * kHeadDim + 8u * (i16 & 1);
  const uint32_t tr_swz = 16u * (uint32_t)((trow >> 1) & 7);

  // Stage one step's K/V rows and scales into LDS buffer `buf`.  V rows
  // past the sequence end are zeroed (their P is 0, and a stray NaN byte
  // would otherwise poison the MFMA sum); their K scores are masked.  The
  // scales are stored premultiplied: k_scale * softmax_scale * log2(e),
  // and v_scale * f after f has taken in this step's valid tokens (the
  // accumulator holds the previous steps, so it is rescaled here).  A
  // NaN v_scale (never stored by the store kernel) counts as out of range
  // and is excluded from f by the max.
  auto stage = [&](const StepLoads& s, int buf) {
#pragma unroll
    for (int c = 0; c < 4; ++c) {
      const int row = 8 * c + (lane >> 3);
      const uint32_t o = tile_off(row, lane & 7);
      *reinterpret_cast<u32x4*>(&kv_lds[buf][0][o]) = s.k[c];
      *reinterpret_cast<u32x4*>(&kv_lds[buf][1][o]) =
          row < s.valid ? s.v[c] : u32x4{0u, 0u, 0u, 0u};
    }
    const bool vtok = lane >= 32 && lane - 32 < s.valid;
    if (__any(vtok && !(s.vscale * f <= kPvScaleMax)) || f == 0.0f) {
      // no scale yet, or a valid token whose weight could leave fp16's
      // range: f from the largest v_scale of the step's valid tokens (and
      // those before it), never growing.  A step with no valid token (an
      // invalid page, say) leaves f at 0, so that the first step that has
      // one picks it: its tokens' weights are 0 meanwhile, which is what
      // they contribute.
      float vm = vtok ? s.vscale : 0.0f;
      vm = fmaxf(max_xor32(max_xor16(max16_dpp(vm))), vseen);
      const float fnew = vm > 0.0f ? pow2_floor(kPvScaleMax / vm) : 0.0f;
      if (f != 0.0f && fnew < f) {
        const float r = fnew / f;  // a power of two < 1: exact
#pragma unroll
        for (int dt = 0; dt < 8; ++dt) acc[dt] *= r;
      }
      if (fnew > 0.0f && (f == 0.0f || fnew < f)) f = fnew;
      vseen = vm;
    }
    s_lds[buf][lane] = lane < 32 ? s.kscale * a.scale_log2 : s.vscale * f;
  };
  // K operand reads: token n (and 16 + n), chunks g and 4 + g
  const uint32_t k_lo = tile_off(n, g), k_hi = tile_off(n, 4 + g);

  StepLoads cur, nxt;
  load_step(a, blk_first, kvh, t_begin, t_end, lane, cur);
  stage(cur, 0);
  wave_lds_sync();
  int buf = 0;
  for (int t0 = t_begin; t0 < t_end; t0 += kStep, buf ^= 1) {
    const int valid = cur.valid;
    const bool more = t0 + kStep < t_end;
    if (more)
      load_step(a, a.bt[(int64_t)b * a.w + (t0 + kStep) / a.bs], kvh, t0 + kStep, t_end, lane,
                nxt);

    // S^T = K . Q^T for tokens [0,16) and [16,32) of the step
    const uint8_t* kt = kv_lds[buf][0];
    const u32x4 k0a = *reinterpret_cast<const u32x4*>(kt + k_lo);
    const u32x4 k0b = *reinterpret_cast<const u32x4*>(kt + k_hi);
    const u32x4 k1a = *reinterpret_cast<const u32x4*>(kt + 16 * kHeadDim + k_lo);
    const u32x4 k1b = *reinterpret_cast<const u32x4*>(kt + 16 * kHeadDim + k_hi);
    f32x4 s0 = {0.f, 0.f, 0.f, 0.f}, s1 = {0.f, 0.f, 0.f, 0.f};
    x8 ka;
    A::fp8x4_to(k0a[0], ka, 0); A::fp8x4_to(k0a[1], ka, 4); s0 = A::mfma(ka, qop[0], s0);
    A::fp8x4_to(k0a[2], ka, 0); A::fp8x4_to(k0a[3], ka, 4); s0 = A::mfma(ka, qop[1], s0);
    A::fp8x4_to(k0b[0], ka, 0); A::fp8x4_to(k0b[1], ka, 4); s0 = A::mfma(ka, qop[2], s0);
    A::fp8x4_to(k0b[2], ka, 0); A::fp8x4_to(k0b[3], ka, 4); s0 = A::mfma(ka, qop[3], s0);
    A::fp8x4_to(k1a[0], ka, 0); A::fp8x4_to(k1a[1], ka, 4); s1 = A::mfma(ka, qop[0], s1);
    A::fp8x4_to(k1a[2], ka, 0); A::fp8x4_to(k1a[3], ka, 4); s1 = A::mfma(ka, qop[1], s1);
    A::fp8x4_to(k1b[0], ka, 0); A::fp8x4_to(k1b[1], ka, 4); s1 = A::mfma(ka, qop[2], s1);
    A::fp8x4_to(k1b[2], ka, 0); A::fp8x4_to(k1b[3], ka, 4); s1 = A::mfma(ka, qop[3], s1);

    const float* sc = s_lds[buf];
    const f32x4 ksc0 = *reinterpret_cast<const f32x4*>(sc + 4 * g);
    const f32x4 ksc1 = *reinterpret_cast<const f32x4*>(sc + 16 + 4 * g);
    const f32x4 vsc0 = *reinterpret_cast<const f32x4*>(sc + 32 + 4 * g);
    const f32x4 vsc1 = *reinterpret_cast<const f32x4*>(sc + 48 + 4 * g);
    float x[8];
    if (valid == kStep) {
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        x[r] = s0[r] * ksc0[r];
        x[4 + r] = s1[r] * ksc1[r];
      }
    } else {
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        x[r] = (4 * g + r < valid) ? s0[r] * ksc0[r] : -INFINITY;
        x[4 + r] = (16 + 4 * g + r < valid) ? s1[r] * ksc1[r] : -INFINITY;
      }
    }
    float tmax = fmaxf(fmaxf(fmaxf(x[0], x[1]), fmaxf(x[2], x[3])),
                       fmaxf(fmaxf(x[4], x[5]), fmaxf(x[6], x[7])));
    tmax = max_xor32(max_xor16(tmax));
    // lazy rescale: only when some head's max outgrows the reference by the slack
    if (__any(tmax > m + kRescaleSlack)) {
      const float m_new = fmaxf(m, tmax);
      const float alpha = m_new == -INFINITY ? 1.0f : exp2_fast(m - m_new);
      l *= alpha;
#pragma unroll
      for (int dt = 0; dt < 8; ++dt) acc[dt] *= alpha;
      m = m_new;
    }
    const float m_use = m == -INFINITY ? 0.0f : m;
    float psum = 0.0f;
    f16x8 pt;
#pragma unroll
    for (int e = 0; e < 8; ++e) {
      const float p = exp2_fast(x[e] - m_use);
      psum += p;
      const float vsc = e < 4 ? vsc0[e] : vsc1[e - 4];  // v_scale * f
      pt[e] = (_Float16)(p * vsc);
    }
    if (valid != kStep) {
#pragma unroll
      for (int e = 0; e < 8; ++e)
        if (x[e] == -INFINITY) pt[e] = (_Float16)0.0f;
    }
    l += psum;

    // O^T += V^T . P^T, one 16-wide d tile per MFMA
    const uint8_t* vb = kv_lds[buf][1];
#pragma unroll
    for (int dt = 0; dt < 8; ++dt) {
      const i32x2 raw = __builtin_amdgcn_ds_read_tr8_b64_v2i32(
          reinterpret_cast<__attribute__((address_space(3))) i32x2*>(
              (__attribute__((address_space(3))) uint8_t*)vb + tr_base +
              ((16u * dt) ^ tr_swz)));
      const f16x8 vt = fp8x8_to_f16((uint32_t)raw[0], (uint32_t)raw[1]);
      acc[dt] = __builtin_amdgcn_mfma_f32_16x16x32_f16(vt, pt, acc[dt], 0, 0, 0);
    }
    if (more) {
      stage(nxt, buf ^ 1);
      cur = nxt;
    }
    wave_lds_sync();
  }
  l = sum_xor32(sum_xor16(l));
  if (f != 0.0f) {
    const float inv_f = 1.0f / f;  // a power of two: exact
#pragma unroll
    for (int dt = 0; dt < 8; ++dt) acc[dt] *= inv_f;
  }
}

// out[b, qh, :] = acc / l in the activation type (zeros when l == 0)
template <typename T>
__device__ __forceinline__ void write_output(uint16_t* op, const f32x4 (&acc)[8], float l,
                                             int g) {
  using A = Act<T>;
  const float inv = l > 0.0f ? 1.0f / l : 0.0f;
#pragma unroll
  for (int dt = 0; dt < 8; ++dt) {
    const f32x4 o = acc[dt] * inv;
    const uint32_t lo = (uint32_t)A::from_f32(o[0]) | ((uint32_t)A::from_f32(o[1]) << 16);
    const uint32_t hi = (uint32_t)A::from_f32(o[2]) | ((uint32_t)A::from_f32(o[3]) << 16);
    *reinterpret_cast<u32x2*>(op + 16 * dt + 4 * g) = u32x2{lo, hi};
  }
}

// a split's partial: o / l and m + log2 l (-inf when it saw no token)
__device__ __forceinline__ void write_partial(float* po, float* plse, const f32x4 (&acc)[8],
                                              float m, float l, int g) {
  const float inv = l > 0.0f ? 1.0f / l : 0.0f;
#pragma unroll
  for (int dt = 0; dt < 8; ++dt)
    *reinterpret_cast<f32x4*>(po + 16 * dt + 4 * g) = acc[dt] * inv;
  if (g == 0) *plse = l > 0.0f ? m + __log2f(l) : -INFINITY;
}

// 2 waves per SIMD, the occupancy the LDS allows: one 8-wave workgroup
// (132 KB) or two 4-wave ones (66 KB each) per CU.  (A hint of 3 could not
// be met and left the 4-wave instance at 200 VGPRs instead of 167, with no
// difference in time.)
template <typename T, int W>
__global__ __launch_bounds__(64 * W)
__attribute__((amdgpu_waves_per_eu(2, 8)))
void decode_fp8_kernel(DecodeArgs a) {
  // per wave: two K/V tile pairs and their scales; step i is read from
  // buffer i&1 while step i+1 is staged into the other one
  __shared__ __attribute__((aligned(16))) uint8_t kv_lds_all[W][2][2][kStep * kHeadDim];
  __shared__ __attribute__((aligned(16))) float s_lds_all[W][2][2 * kStep];

  const int wave = threadIdx.x >> 6;
  const int lane = threadIdx.x & 63;
  const int g = lane >> 4, n = lane & 15;
  const int unit = blockIdx.x * W + wave;
  // The sequence, its length and the split's first block id are read
  // together, first thing, so the first K/V loads wait for one memory round
  // trip, not a chain of them (readfirstlane is convergent, so the compiler
  // cannot sink a read below the branches that use it).  The split's first
  // page is inside the table: split * pages_per_split < w for every split
  // count the host accepts.  With work items, grid row (z, y) takes item
  // z * splits + y: the valid splits of the longest sequences first, short
  // sequences' in the last round, and the rows past the last item (empty
  // splits) at the end of the grid.
  int b, split, len_raw, blk_first;
  if (a.items) {
    const int item = blockIdx.z * a.splits + blockIdx.y;
    const int4 e = a.items[item];
    const int count = __builtin_amdgcn_readfirstlane(*a.item_count);
    b = __builtin_amdgcn_readfirstlane(e.x);
    split = __builtin_amdgcn_readfirstlane(e.y);
    len_raw = __builtin_amdgcn_readfirstlane(e.z);
    blk_first = __builtin_amdgcn_readfirstlane(e.w);
    if (item >= count) return;
    if ((unsigned)b >= (unsigned)a.batch || (unsigned)split >= (unsigned)a.splits) return;
  } else {
    split = blockIdx.y;
    b = blockIdx.z;
    len_raw = __builtin_amdgcn_readfirstlane(a.seqlens[b]);
    blk_first =
        __builtin_amdgcn_readfirstlane(a.bt[(int64_t)b * a.w + split * a.pages_per_split]);
  }
  if (unit >= a.hk * a.qgroups) return;
  const int kvh = unit / a.qgroups;
  const int hig = (unit - kvh * a.qgroups) * 16 + n;  // head within its group
  const bool head_ok = hig < a.group;
  const int qh = kvh * a.group + hig;
  const int split_tokens = a.pages_per_split * a.bs;
  const int t_begin = split * split_tokens;
  // tokens past the block table's width are not addressable: ignore them
  const int L = min(len_raw, a.w * a.bs);

  if (L <= 0) {
    if (a.splits == 1 && split == 0 && head_ok) {
      uint16_t* op = a.out + ((int64_t)b * a.hq + qh) * kHeadDim;
#pragma unroll
      for (int dt = 0; dt < 8; ++dt)
        *reinterpret_cast<u32x2*>(op + 16 * dt + 4 * g) = u32x2{0u, 0u};
    }
    return;
  }
  if (t_begin >= L) return;
  const int t_end = min(L, t_begin + split_tokens);

  f32x4 acc[8];
  float m, l;
  attend_range<T>(a, b, kvh, qh, head_ok, t_begin, t_end, blk_first, lane, kv_lds_all[wave],
                  s_lds_all[wave], acc, m, l);

  // splits that hold tokens of this sequence; a sequence that fits in one
  // split is written here directly
  const int nvalid = min(a.splits, (L + split_tokens - 1) / split_tokens);
  if (!head_ok) return;
  if (nvalid == 1) {
    write_output<T>(a.out + ((int64_t)b * a.hq + qh) * kHeadDim, acc, l, g);
    return;
  }
  // this split's partial, merged by a combine kernel
  const int64_t row = ((int64_t)b * a.hq + qh) * a.splits + split;
  write_partial(a.part_o + row * kHeadDim, a.part_lse + row, acc, m, l, g);
}

// A merge state over some splits of one row, held in plain registers: the
// largest lse value m, and den = sum 2^(lse_s - m), o = sum 2^(lse_s - m)
// o_s over those splits, for four consecutive d.  m = -inf (den = 0, o = 0)
// holds no split.
//
// The lse values and partial quads of splits sp = first + k * stride
// (k < K), loaded all at once (one memory round trip) for sp < limit; the
// rest read as empty.
template <int K>
struct SplitLoads {
  float ls[K];
  f32x4 pv[K];
};
template <int K>
__device__ __forceinline__ void load_splits(SplitLoads<K>& s, const float* __restrict__ lse,
                                            const float* __restrict__ po, int first, int stride,
                                            int limit) {
#pragma unroll
  for (int k = 0; k < K; ++k) {
    const int sp = first + k * stride;
    const bool ok = sp < limit;
    s.ls[k] = ok ? lse[sp] : -INFINITY;
    s.pv[k] = ok ? *reinterpret_cast<const f32x4*>(po + (int64_t)sp * kHeadDim)
                 : f32x4{0.f, 0.f, 0.f, 0.f};
  }
}

// Folds the loaded splits below nvalid into (m, den, o).  Loads past nvalid
// (stale partials of an earlier call, when the caller loaded up to the
// split count) are dropped, values included.
template <int K>
__device__ __forceinline__ void fold_splits(float& m, float& den, f32x4& o, SplitLoads<K> s,
                                            int first, int stride, int nvalid) {
#pragma unroll
  for (int k = 0; k < K; ++k) {
    if (first + k * stride >= nvalid) {
      s.ls[k] = -INFINITY;
      s.pv[k] = f32x4{0.f, 0.f, 0.f, 0.f};
    }
  }
  float cm = s.ls[0];
#pragma unroll
  for (int k = 1; k < K; ++k) cm = fmaxf(cm, s.ls[k]);
  const float nm = fmaxf(m, cm);
  if (nm == -INFINITY) return;  // no split here, none before
  const float sc = m == -INFINITY ? 0.0f : exp2_fast(m - nm);
  den *= sc;
  o *= sc;
#pragma unroll
  for (int k = 0; k < K; ++k) {
    const float w = exp2_fast(s.ls[k] - nm);  // 0 for a split not read
    den += w;
    o += w * s.pv[k];
  }
  m = nm;
}

// Folds the splits sp = first + k * stride (k < K, sp < nvalid) of one row
// into (m, den, o) in one memory round trip.  Partials past nvalid are
// never read.
template <int K>
__device__ __forceinline__ void merge_splits(float& m, float& den, f32x4& o,
                                             const float* __restrict__ lse,
                                             const float* __restrict__ po, int first,
                                             int stride, int nvalid) {
  SplitLoads<K> s;
  load_splits(s, lse, po, first, stride, nvalid);
  fold_splits(m, den, o, s, first, stride, nvalid);
}

// (m, den, o) becomes the merge of states a and b over disjoint splits.
__device__ __forceinline__ void merge_pair(float& m, float& den, f32x4& o, float ma,
                                           float da, f32x4 oa, float mb, float db, f32x4 ob) {
  const float M = fmaxf(ma, mb);
  if (M == -INFINITY) {
    m = -INFINITY;
    den = 0.0f;
    o = f32x4{0.f, 0.f, 0.f, 0.f};
    return;
  }
  const float sa = exp2_fast(ma - M), sb = exp2_fast(mb - M);  // 0 for -inf
  m = M;
  den = da * sa + db * sb;
  o = oa * sa + ob * sb;
}

// Merges the state with that of lane l ^ 16 (v_permlane16_swap) or l ^ 32
// (v_permlane32_swap), no LDS round trip: the swap returns both lanes'
// values, in the same order for every field, so the pair's merge is the
// same state on both lanes.
template <bool kXor32>
__device__ __forceinline__ uint2 swap_pair(float v) {
  const auto r = kXor32 ? __builtin_amdgcn_permlane32_swap(__float_as_uint(v),
                                                           __float_as_uint(v), false, false)
                        : __builtin_amdgcn_permlane16_swap(__float_as_uint(v),
                                                           __float_as_uint(v), false, false);
  return uint2{r[0], r[1]};
}
template <bool kXor32>
__device__ __forceinline__ void merge_across(float& m, float& den, f32x4& o) {
  const uint2 pm = swap_pair<kXor32>(m), pd = swap_pair<kXor32>(den);
  const uint2 p0 = swap_pair<kXor32>(o[0]), p1 = swap_pair<kXor32>(o[1]);
  const uint2 p2 = swap_pair<kXor32>(o[2]), p3 = swap_pair<kXor32>(o[3]);
  merge_pair(m, den, o, __uint_as_float(pm.x), __uint_as_float(pd.x),
             f32x4{__uint_as_float(p0.x), __uint_as_float(p1.x), __uint_as_float(p2.x),
                   __uint_as_float(p3.x)},
             __uint_as_float(pm.y), __uint_as_float(pd.y),
             f32x4{__uint_as_float(p0.y), __uint_as_float(p1.y), __uint_as_float(p2.y),
                   __uint_as_float(p3.y)});
}

// out = o / den in the activation type, four consecutive d (zeros when
// den == 0)
template <typename T>
__device__ __forceinline__ void write_merged(uint16_t* op, float den, f32x4 o) {
  using A = Act<T>;
  const float inv = den > 0.0f ? 1.0f / den : 0.0f;
  o *= inv;
  const uint32_t lo = (uint32_t)A::from_f32(o[0]) | ((uint32_t)A::from_f32(o[1]) << 16);
  const uint32_t hi = (uint32_t)A::from_f32(o[2]) | ((uint32_t)A::from_f32(o[3]) << 16);
  *reinterpret_cast<u32x2*>(op) = u32x2{lo, hi};
}

// out[b, h, :] = sum_s 2^(lse_s - M) o_s / sum_s 2^(lse_s - M) over the
// splits holding tokens of sequence b; zeros for an empty sequence.  Rows
// whose sequence fits in one split were written by the split kernel.
// One wave per (b, h) row: lane (j, i) takes d in [4i, 4i + 4) of splits
// j, j + 2, ..., kLoopK of them per memory round trip (32 splits: the
// ragged batch's whole row in one), and the two halves merge across lanes.
constexpr int kLoopK = 16;

template <typename T>
__global__ __launch_bounds__(64) void decode_combine_kernel(
    const float* __restrict__ part_o, const float* __restrict__ part_lse,
    const int32_t* __restrict__ seqlens, uint16_t* __restrict__ out, int hq,
    int splits, int split_tokens, int max_tokens) {
  const int row = blockIdx.x;  // b * hq + h
  const int b = row / hq;
  const int lane = threadIdx.x;
  const int j = lane >> 5, i = lane & 31;
  const int L = min(seqlens[b], max_tokens);
  const int nvalid = L <= 0 ? 0 : min(splits, (L + split_tokens - 1) / split_tokens);
  if (nvalid == 1) return;
  const float* lse = part_lse + (int64_t)row * splits;
  const float* po = part_o + (int64_t)row * splits * kHeadDim + 4 * i;
  float m = -INFINITY, den = 0.0f;
  f32x4 o = {0.f, 0.f, 0.f, 0.f};
  for (int base = 0; base < nvalid; base += 2 * kLoopK)
    merge_splits<kLoopK>(m, den, o, lse, po, base + j, 2, nvalid);
  merge_across<true>(m, den, o);
  if (j == 0) write_merged<T>(out + (int64_t)row * kHeadDim + 4 * i, den, o);
}

// The same merge for at most S splits (S a compile-time bound, small): every
// split's lse value and partial row is loaded at once, before the sequence
// length arrives, so a row costs one memory round trip instead of two.
// Rows of few splits use them all; with many splits, mostly unused (ragged
// batches), the reads of unused rows cost more than the round trip, so
// those keep decode_combine_kernel.  M is the largest valid lse value and
// the weighted sum runs in split order.
template <typename T, int S>
__global__ __launch_bounds__(64) void decode_combine_small_kernel(
    const float* __restrict__ part_o, const float* __restrict__ part_lse,
    const int32_t* __restrict__ seqlens, uint16_t* __restrict__ out, int hq,
    int splits, int split_tokens, int max_tokens) {
  const int row = blockIdx.x;  // b * hq + h
  const int b = row / hq;
  const int lane = threadIdx.x;
  // every split row below `splits` is in bounds: read them all while the
  // sequence length is still on its way, use the first nvalid
  const float* lse = part_lse + (int64_t)row * splits;
  const float* po = part_o + (int64_t)row * splits * kHeadDim + 2 * lane;
  float ls[S];
  float2 pv[S];
#pragma unroll
  for (int sp = 0; sp < S; ++sp) {
    ls[sp] = sp < splits ? lse[sp] : -INFINITY;
    pv[sp] = sp < splits ? *reinterpret_cast<const float2*>(po + (int64_t)sp * kHeadDim)
                         : float2{0.0f, 0.0f};
  }
  const int L = min(seqlens[b], max_tokens);
  const int nvalid = L <= 0 ? 0 : min(splits, (L + split_tokens - 1) / split_tokens);
  if (nvalid == 1) return;
  float M = -INFINITY;
#pragma unroll
  for (int sp = 0; sp < S; ++sp)
    if (sp < nvalid) M = fmaxf(M, ls[sp]);
  float o0 = 0.0f, o1 = 0.0f, den = 0.0f;
  if (M != -INFINITY) {
#pragma unroll
    for (int sp = 0; sp < S; ++sp) {
      if (sp >= nvalid) break;
      const float w = exp2_fast(ls[sp] - M);
      o0 += w * pv[sp].x;
      o1 += w * pv[sp].y;
      den += w;
    }
  }
  const float inv = den > 0.0f ? 1.0f / den : 0.0f;
  const uint32_t pk = (uint32_t)Act<T>::from_f32(o0 * inv) |
                      ((uint32_t)Act<T>::from_f32(o1 * inv) << 16);
  *reinterpret_cast<uint32_t*>(out + (int64_t)row * kHeadDim + 2 * lane) = pk;
}

// The same merge for many splits (long contexts): four 256-thread
// workgroups per (b, h) row, each taking 32 d of it, so a batch-1 decode's
// 64 rows fill the chip.  Lane (j, i) of wave w takes d 4i..4i+3 of the
// quarter and splits 8w + j, 8w + j + 32, ..., kWideK of them per memory
// round trip (256 splits in one); the 32 lanes of each d merge across
// lanes (xor 8, 16, 32), then the four waves through LDS.
constexpr int kWideWaves = 4;
constexpr int kWideK = 8;
constexpr int kWideThreshold = 64;  // splits above this use the wide merge

template <typename T>
__global__ __launch_bounds__(64 * kWideWaves) void decode_combine_wide_kernel(
    const float* __restrict__ part_o, const float* __restrict__ part_lse,
    const int32_t* __restrict__ seqlens, uint16_t* __restrict__ out, int hq, int splits,
    int split_tokens, int max_tokens) {
  __shared__ float s_m[kWideWaves][8], s_den[kWideWaves][8];
  __shared__ __attribute__((aligned(16))) f32x4 s_o[kWideWaves][8];
  const int row = blockIdx.x;  // b * hq + h
  const int quarter = blockIdx.y;
  const int b = row / hq;
  const int tid = threadIdx.x;
  const int wave = tid >> 6;
  const int lane = tid & 63;
  const int i = lane & 7, j = lane >> 3;
  const int d = 32 * quarter + 4 * i;
  const float* lse = part_lse + (int64_t)row * splits;
  const float* po = part_o + (int64_t)row * splits * kHeadDim + d;
  // the first kWideK splits of each lane are loaded (every split row below
  // `splits` is in bounds) while the sequence length is still on its way:
  // one memory round trip for up to 256 splits instead of two
  constexpr int kPass = 8 * kWideWaves * kWideK;
  SplitLoads<kWideK> first;
  load_splits(first, lse, po, 8 * wave + j, 8 * kWideWaves, min(splits, kPass));
  const int L = min(seqlens[b], max_tokens);
  const int nvalid = L <= 0 ? 0 : min(splits, (L + split_tokens - 1) / split_tokens);
  if (nvalid == 1) return;  // written by the split kernel
  float m = -INFINITY, den = 0.0f;
  f32x4 o = {0.f, 0.f, 0.f, 0.f};
  fold_splits(m, den, o, first, 8 * wave + j, 8 * kWideWaves, nvalid);
  for (int base = kPass; base < nvalid; base += kPass)
    merge_splits<kWideK>(m, den, o, lse, po, base + 8 * wave + j, 8 * kWideWaves, nvalid);
  {
    const f32x4 ox = {__shfl_xor(o[0], 8), __shfl_xor(o[1], 8), __shfl_xor(o[2], 8),
                      __shfl_xor(o[3], 8)};
    merge_pair(m, den, o, m, den, o, __shfl_xor(m, 8), __shfl_xor(den, 8), ox);
  }
  merge_across<false>(m, den, o);
  merge_across<true>(m, den, o);
  if (j == 0) {
    s_m[wave][i] = m;
    s_den[wave][i] = den;
    s_o[wave][i] = o;
  }
  __syncthreads();
  if (wave != 0 || j != 0) return;
#pragma unroll
  for (int w = 1; w < kWideWaves; ++w)
    merge_pair(m, den, o, m, den, o, s_m[w][i], s_den[w][i], s_o[w][i]);
  write_merged<T>(out + (int64_t)row * kHeadDim + d, den, o);
}

// The longest-first work items of a split grid of many rounds: workgroup
// b ranks sequence b by its length (clamped to the table; ties by index,
// so the order is total) and sums the valid splits of the sequences ahead
// of it, which is where its items start; it writes one item per valid
// split of its own.  Workgroup 0 also writes the item count.  The block
// ids are read alongside the lengths, so the items cost one memory round
// trip before the writes.
constexpr int kOrderThreads = 256;
constexpr int kOrderMaxBatch = 4096;

// Sum over the wave with DPP row shifts and the two cross-row swaps (no
// LDS round trip).
__device__ __forceinline__ int wave_sum_i32(int v) {
  v += __builtin_amdgcn_update_dpp(0, v, 0xB1, 0xF, 0xF, false);   // quad_perm [1,0,3,2]
  v += __builtin_amdgcn_update_dpp(0, v, 0x4E, 0xF, 0xF, false);   // quad_perm [2,3,0,1]
  v += __builtin_amdgcn_update_dpp(0, v, 0x141, 0xF, 0xF, false);  // row_half_mirror
  v += __builtin_amdgcn_update_dpp(0, v, 0x140, 0xF, 0xF, false);  // row_mirror
  const auto r16 = __builtin_amdgcn_permlane16_swap((uint32_t)v, (uint32_t)v, false, false);
  v = (int)(r16[0] + r16[1]);
  const auto r32 = __builtin_amdgcn_permlane32_swap((uint32_t)v, (uint32_t)v, false, false);
  return (int)(r32[0] + r32[1]);
}

__global__ __launch_bounds__(kOrderThreads) void decode_order_kernel(
    const int32_t* __restrict__ seqlens, const int32_t* __restrict__ bt, int4* __restrict__ items,
    int* __restrict__ item_count, int batch, int w, int max_tokens, int splits,
    int pages_per_split, int split_tokens) {
  __shared__ int s_off[kOrderThreads / 64], s_tot[kOrderThreads / 64];
  const int b = blockIdx.x;
  const int tid = threadIdx.x;
  const int len_b = seqlens[b];
  // this thread's first split's block id, read with the lengths
  const int blk0 = tid < splits ? bt[(int64_t)b * w + tid * pages_per_split] : 0;
  const int key = max(0, min(len_b, max_tokens));
  const int nv_b = min(splits, (key + split_tokens - 1) / split_tokens);
  int off = 0, tot = 0;
  for (int j = tid; j < batch; j += kOrderThreads) {
    const int kj = max(0, min(seqlens[j], max_tokens));
    const int nj = min(splits, (kj + split_tokens - 1) / split_tokens);
    off += (kj > key || (kj == key && j < b)) ? nj : 0;
    tot += nj;
  }
  off = wave_sum_i32(off);
  tot = wave_sum_i32(tot);
  if ((tid & 63) == 0) {
    s_off[tid >> 6] = off;
    s_tot[tid >> 6] = tot;
  }
  __syncthreads();
  int first = 0, count = 0;
#pragma unroll
  for (int i = 0; i < kOrderThreads / 64; ++i) {
    first += s_off[i];
    count += s_tot[i];
  }
  if (b == 0 && tid == 0) *item_count = count;
  if (tid < nv_b) items[first + tid] = int4{b, tid, len_b, blk0};
  for (int sp = tid + kOrderThreads; sp < nv_b; sp += kOrderThreads)
    items[first + sp] = int4{b, sp, len_b, bt[(int64_t)b * w + sp * pages_per_split]};
}

// units of up to 16 q heads per kv head: a group above 16 that is not a
// multiple of 16 leaves the last unit's surplus lanes idle (head_ok false)
static int qgroups_of(int group) { return (group + 15) / 16; }

// Whether a decode shape runs compacted work items longest-first: split
// grids of many rounds (over kWideGridMax eight-wave workgroups), where a
// long sequence dispatched late sets the makespan and most workgroups are
// empty splits (ragged batch 256: 423-426 against 454-457 us).  Shapes
// only, like every launch choice here.
constexpr int64_t kOrderMaxEntries = 1 << 16;  // batch * splits
static bool ordered_of(int batch, int hk, int qgroups, int splits) {
  const int64_t wide_wgs =
      (int64_t)((hk * qgroups + kWavesPerWG - 1) / kWavesPerWG) * splits * batch;
  return splits > 1 && batch > 1 && batch <= kOrderMaxBatch && wide_wgs > kWideGridMax &&
         (int64_t)batch * splits <= kOrderMaxEntries;
}

// Bytes of the split partials ([batch, hq, splits, 128] outputs, then
// [batch, hq, splits] lse values), rounded up to 256.
static size_t partials_bytes(int batch, int hq, int splits) {
  const size_t raw = (size_t)batch * hq * splits * (kHeadDim + 1) * sizeof(float);
  return (raw + 255) & ~(size_t)255;
}

template <typename T>
static hipError_t launch_decode(const DecodeArgs& a, int batch, hipStream_t stream) {
  // One 8-wave workgroup (128 KB of LDS) fills a CU.  A grid of at most
  // kWideGridMax of those runs in about two rounds; a larger grid runs in
  // many, over the longest-first work items of the pre-pass.  Beyond the
  // items' limits (and where a kv head group has fewer than eight units),
  // the last round's tail halves with 4-wave workgroups (two per CU):
  // ragged batch 256 in row order, 452 against 491 us.  The Qwen3-8B batch
  // 64 x 4096 step prefers 8 waves, 88.3 against 90.5 us.  Shapes only, so
  // the choice is the same on every call of a captured graph.
  const int units = a.hk * a.qgroups;
  const int64_t wide_wgs = (int64_t)((units + kWavesPerWG - 1) / kWavesPerWG) * a.splits * batch;
  if (a.items) {
    hipLaunchKernelGGL(decode_order_kernel, dim3((unsigned)batch), dim3(kOrderThreads), 0, stream,
                       a.seqlens, a.bt, const_cast<int4*>(a.items),
                       const_cast<int*>(a.item_count), batch, a.w, a.w * a.bs, a.splits,
                       a.pages_per_split, a.pages_per_split * a.bs);
    const hipError_t eo = hipGetLastError();
    if (eo != hipSuccess) return eo;
  }
  // 8-wave workgroups also run the work items when every wave has a unit:
  // with the short sequences last, their longer units no longer lengthen
  // the tail (ragged batch 256: 425-426 against 433-435 us with 4 waves)
  if (wide_wgs <= kWideGridMax || (a.items && units >= kWavesPerWG)) {
    const dim3 grid((unsigned)((units + kWavesPerWG - 1) / kWavesPerWG), (unsigned)a.splits,
                    (unsigned)batch);
    hipLaunchKernelGGL((decode_fp8_kernel<T, kWavesPerWG>), grid, dim3(64 * kWavesPerWG), 0,
                       stream, a);
  } else {
    const dim3 grid((unsigned)((units + kNarrowWaves - 1) / kNarrowWaves), (unsigned)a.splits,
                    (unsigned)batch);
    hipLaunchKernelGGL((decode_fp8_kernel<T, kNarrowWaves>), grid, dim3(64 * kNarrowWaves), 0,
                       stream, a);
  }
  hipError_t e = hipGetLastError();
  if (e != hipSuccess || a.splits == 1) return e;
  if (a.splits > kWideThreshold)
    hipLaunchKernelGGL(decode_combine_wide_kernel<T>, dim3((unsigned)(batch * a.hq), 4u),
                       dim3(64 * kWideWaves), 0, stream, a.part_o, a.part_lse, a.seqlens, a.out,
                       a.hq, a.splits, a.pages_per_split * a.bs, a.w * a.bs);
  else if (a.splits <= 8)
    hipLaunchKernelGGL((decode_combine_small_kernel<T, 8>), dim3((unsigned)(batch * a.hq)),
                       dim3(64), 0, stream, a.part_o, a.part_lse, a.seqlens, a.out, a.hq,
                       a.splits, a.pages_per_split * a.bs, a.w * a.bs);
  else
    hipLaunchKernelGGL(decode_combine_kernel<T>, dim3((unsigned)(batch * a.hq)), dim3(64), 0,
                       stream, a.part_o, a.part_lse, a.seqlens, a.out, a.hq, a.splits,
                       a.pages_per_split * a.bs, a.w * a.bs);
  return hipGetLastError();
}

static int pages_per_split_of(int splits, int w) {
  return splits <= 1 ? w : (w + splits - 1) / splits;
}

}  // namespace mskv

extern "C" int mskv_decode_num_splits(int batch, int num_q_heads,
                                      int num_kv_heads, int max_blocks_per_seq,
                                      int block_size) {
  (void)block_size;
  if (batch <= 0 || num_kv_heads <= 0 || num_q_heads <= 0 ||
      max_blocks_per_seq <= 0)
    return 1;
  const int group = num_q_heads / num_kv_heads;
  const int64_t base = (int64_t)batch * num_kv_heads * mskv::qgroups_of(group);
  const int w = max_blocks_per_seq;
  int64_t pps = (w * base + mskv::kTargetWaves - 1) / mskv::kTargetWaves;
  if (pps < 1) pps = 1;
  if (pps > mskv::kMaxPagesPerSplit) pps = mskv::kMaxPagesPerSplit;
  const int64_t splits = (w + pps - 1) / pps;
  return (int)splits;
}

extern "C" size_t mskv_decode_workspace_bytes(int batch, int num_q_heads,
                                              int num_kv_heads, int head_dim,
                                              int num_splits) {
  if (num_splits <= 1 || batch <= 0 || num_q_heads <= 0 || num_kv_heads <= 0 ||
      head_dim <= 0 || num_q_heads % num_kv_heads != 0)
    return 0;
  size_t bytes = (size_t)batch * num_q_heads * num_splits * (head_dim + 1) * sizeof(float);
  const int qgroups = mskv::qgroups_of(num_q_heads / num_kv_heads);
  if (head_dim == mskv::kHeadDim &&
      mskv::ordered_of(batch, num_kv_heads, qgroups, num_splits))
    bytes = mskv::partials_bytes(batch, num_q_heads, num_splits) + sizeof(int4) +
            (size_t)batch * num_splits * sizeof(int4);
  return bytes;
}

namespace mskv {

// Validates a decode call and launches it with `workspace` as the split
// partials ([batch, hq, splits, 128] outputs, then [batch, hq, splits]
// lse values); `workspace_bytes` is what the caller's buffer holds.
static int decode_checked(const void* query, const void* k_cache, const void* v_cache,
                          const float* k_scale_cache, const float* v_scale_cache,
                          const int32_t* cache_seqlens, const int32_t* block_tables, void* out,
                          int batch, int num_q_heads, int num_kv_heads, int head_dim,
                          int block_size, int64_t num_blocks, int max_blocks_per_seq,
                          float softmax_scale, int act_dtype, int num_splits, void* workspace,
                          size_t workspace_bytes, void* stream) {
  if (batch < 0 || num_q_heads <= 0 || num_kv_heads <= 0 || block_size <= 0 ||
      num_blocks < 0 || max_blocks_per_seq <= 0 || num_splits <= 0)
    return MSKV_EINVAL;
  if (act_dtype != MSKV_FLOAT16 && act_dtype != MSKV_BFLOAT16) return MSKV_EINVAL;
  if (num_q_heads % num_kv_heads != 0) return MSKV_EINVAL;
  const int group = num_q_heads / num_kv_heads;
  if (head_dim != kHeadDim || block_size % kStep != 0) return MSKV_EUNSUPPORTED;
  // page offsets are 32-bit buffer offsets, and token counts up to twice a
  // table's width (w * block_size + split_tokens) stay within int
  if ((int64_t)block_size * num_kv_heads * head_dim > 0x7FFFFFFFLL) return MSKV_EUNSUPPORTED;
  if ((int64_t)max_blocks_per_seq * block_size >= (1LL << 30)) return MSKV_EUNSUPPORTED;
  if (num_splits != mskv_decode_num_splits(batch, num_q_heads, num_kv_heads,
                                           max_blocks_per_seq, block_size))
    return MSKV_EINVAL;
  if (batch == 0) return MSKV_OK;
  if (!query || !k_cache || !v_cache || !k_scale_cache || !v_scale_cache ||
      !cache_seqlens || !block_tables || !out)
    return MSKV_EINVAL;
  const size_t need =
      mskv_decode_workspace_bytes(batch, num_q_heads, num_kv_heads, head_dim, num_splits);
  if (need > 0 && (!workspace || workspace_bytes < need)) return MSKV_EWORKSPACE;

  DecodeArgs a;
  a.q = (const uint16_t*)query;
  a.kc = (const uint8_t*)k_cache;
  a.vc = (const uint8_t*)v_cache;
  a.ks = k_scale_cache;
  a.vs = v_scale_cache;
  a.seqlens = cache_seqlens;
  a.bt = block_tables;
  a.out = (uint16_t*)out;
  a.part_o = need > 0 ? (float*)workspace : nullptr;
  a.part_lse = need > 0 ? a.part_o + (size_t)batch * num_q_heads * num_splits * head_dim
                        : nullptr;
  // the work items follow the partials: a 16-byte slot for the count, then
  // one 16-byte item per (sequence, split)
  a.items = nullptr;
  a.item_count = nullptr;
  if (need > 0 && ordered_of(batch, num_kv_heads, qgroups_of(group), num_splits)) {
    uint8_t* base = (uint8_t*)workspace + partials_bytes(batch, num_q_heads, num_splits);
    a.item_count = (const int*)base;
    a.items = (const int4*)(base + sizeof(int4));
  }
  a.batch = batch;
  a.hq = num_q_heads;
  a.hk = num_kv_heads;
  a.group = group;
  a.qgroups = qgroups_of(group);
  a.bs = block_size;
  a.w = max_blocks_per_seq;
  a.splits = num_splits;
  a.pages_per_split = pages_per_split_of(num_splits, max_blocks_per_seq);
  a.num_blocks = num_blocks;
  a.scale_log2 = softmax_scale * kLog2e;
  hipStream_t s = reinterpret_cast<hipStream_t>(stream);
  hipError_t e = act_dtype == MSKV_BFLOAT16 ? launch_decode<__bf16>(a, batch, s)
                                            : launch_decode<_Float16>(a, batch, s);
  return (int)e;
}

// The split-partials scratch of mskv_fp8_decode_attention_noalloc: a
// file-scope device array, one copy per GPU, alive until the process ends.
// Host code never uses its name as an address (on the host that is a
// stand-in symbol, not device memory): each device's address comes from
// hipGetSymbolAddress, looked up once per device with it current.
__device__ __align__(256) uint8_t scratch[kNoAllocScratchBytes];

constexpr int kMaxDevices = 64;
std::mutex g_scratch_mu;
void* g_scratch_ptr[kMaxDevices] = {};

// This device's address of `scratch`, looked up on its first use.
static hipError_t scratch_for_current_device(void** ptr) {
  int dev = 0;
  hipError_t e = hipGetDevice(&dev);
  if (e != hipSuccess) return e;
  if (dev < 0 || dev >= kMaxDevices) return hipErrorInvalidDevice;
  std::lock_guard<std::mutex> lock(g_scratch_mu);
  if (g_scratch_ptr[dev] == nullptr) {
    void* p = nullptr;
    e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
    if (e != hipSuccess) return e;
    if (p == nullptr) return hipErrorInvalidSymbol;
    g_scratch_ptr[dev] = p;
  }
  *ptr = g_scratch_ptr[dev];
  return hipSuccess;
}

}  // namespace mskv

extern "C" int mskv_fp8_decode_attention(
    const void* query, const void* k_cache, const void* v_cache,
    const float* k_scale_cache, const float* v_scale_cache,
    const int32_t* cache_seqlens, const int32_t* block_tables, void* out,
    int batch, int num_q_heads, int num_kv_heads, int head_dim, int block_size,
    int64_t num_blocks, int max_blocks_per_seq, float softmax_scale,
    int act_dtype, int num_splits, void* workspace, size_t workspace_bytes,
    void* stream) {
  return mskv::decode_checked(query, k_cache, v_cache, k_scale_cache, v_scale_cache,
                              cache_seqlens, block_tables, out, batch, num_q_heads,
                              num_kv_heads, head_dim, block_size, num_blocks,
                              max_blocks_per_seq, softmax_scale, act_dtype, num_splits,
                              workspace, workspace_bytes, stream);
}

extern "C" int mskv_fp8_decode_attention_noalloc(
    const void* query, const void* k_cache, const void* v_cache,
    const float* k_scale_cache, const float* v_scale_cache,
    const int32_t* cache_seqlens, const int32_t* block_tables, void* out,
    int batch, int num_q_heads, int num_kv_heads, int head_dim, int block_size,
    int64_t num_blocks, int max_blocks_per_seq, float softmax_scale,
    int act_dtype, int num_splits, void* stream) {
  const size_t need = mskv_decode_workspace_bytes(batch, num_q_heads, num_kv_heads, head_dim,
                                                  num_splits);
  if (need > mskv::kNoAllocScratchBytes) return MSKV_EWORKSPACE;
  void* ws = nullptr;
  if (need > 0 && batch > 0) {
    const hipError_t e = mskv::scratch_for_current_device(&ws);
    if (e != hipSuccess) return (int)e;
  }
  return mskv::decode_checked(query, k_cache, v_cache, k_scale_cache, v_scale_cache,
                              cache_seqlens, block_tables, out, batch, num_q_heads,
                              num_kv_heads, head_dim, block_size, num_blocks,
                              max_blocks_per_seq, softmax_scale, act_dtype, num_splits, ws,
                              need, stream);
}
