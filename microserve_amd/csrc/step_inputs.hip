// Per-step input expansion: per-sequence scheduling state -> the per-token
// input_ids / positions / slot_mapping, cache_seqlens and the -1-padded
// block tables of one forward step, in one launch.
//
// Replaces the element-by-element device writes of
// microserve/engine/model_runner.py: _compile_decode (:124-142),
// _compile_prefill (:144-172), _compile_chunk_prefill (:174-193),
// _make_block_tables (:208-216) and the graph padding of _run_decode
// (:264-272).  Each of those writes issues one host-to-device copy per
// element; here the host packs the per-sequence state once and this kernel
// expands it, so a step costs one copy and one launch whatever its size.
//
// Work layout: blockIdx.y is a sequence (or a padding row of a captured
// graph); the x dimension strides over that sequence's scheduled tokens and
// over its table row.  Every value is integer, so the outputs are exactly the
// reference's: slot = table[p / block_size] * block_size + p % block_size
// (model_runner.py:135, 160, 182) in 64-bit arithmetic.
#include <hip/hip_runtime.h>
#include <stdint.h>

#include "../../include/mskv.h"

namespace mskv {

constexpr int kStepThreads = 256;

struct StepArgs {
  const int64_t* token_ids;
  const int32_t* seq_start;
  const int32_t* cu_q;
  const int32_t* table_off;
  const int32_t* tables;
  int64_t* input_ids;
  int64_t* positions;
  int64_t* slot_mapping;
  int32_t* cache_seqlens;
  int32_t* block_tables;
  int num_seqs, pad_seqs, block_size, table_width;
  int64_t total_q, garbage_slot;
};

__global__ __launch_bounds__(kStepThreads) void step_inputs_kernel(StepArgs a) {
  const int b = blockIdx.y;
  const int stride = gridDim.x * kStepThreads;
  const int first = blockIdx.x * kStepThreads + threadIdx.x;
  if (b >= a.num_seqs) {
    // a padding row of a captured decode graph (model_runner.py:264-272):
    // its slot is the garbage slot, its length 0 and its table row -1
    if (first == 0) {
      const int64_t row = a.total_q + (b - a.num_seqs);
      a.input_ids[row] = 0;
      a.positions[row] = 0;
      a.slot_mapping[row] = a.garbage_slot;
      if (a.cache_seqlens) a.cache_seqlens[b] = 0;
    }
    if (a.block_tables)
      for (int c = first; c < a.table_width; c += stride)
        a.block_tables[(int64_t)b * a.table_width + c] = -1;
    return;
  }
  const int start = a.seq_start[b];
  const int q0 = a.cu_q[b];
  const int n = a.cu_q[b + 1] - q0;
  const int t0 = a.table_off[b];
  const int len = a.table_off[b + 1] - t0;
  const int bs = a.block_size;
  for (int j = first; j < n; j += stride) {
    const int p = start + j;
    const int blk = p / bs;
    // a position past the end of the table has no slot: -1, which the store
    // skips (the host-side builder raises before launching, as the
    // reference's list indexing does)
    const int64_t slot = blk < len ? (int64_t)a.tables[t0 + blk] * bs + p % bs : -1;
    a.input_ids[q0 + j] = a.token_ids[q0 + j];
    a.positions[q0 + j] = p;
    a.slot_mapping[q0 + j] = slot;
  }
  if (a.block_tables)
    for (int c = first; c < a.table_width; c += stride)
      a.block_tables[(int64_t)b * a.table_width + c] = c < len ? a.tables[t0 + c] : -1;
  if (first == 0 && a.cache_seqlens) a.cache_seqlens[b] = start + n;
}

}  // namespace mskv

extern "C" int mskv_build_step_inputs(
    const int64_t* token_ids, const int32_t* seq_start, const int32_t* cu_seqlens_q,
    const int32_t* table_offsets, const int32_t* tables, int num_seqs, int pad_seqs,
    int64_t total_q, int block_size, int table_width, int64_t garbage_slot,
    int64_t* input_ids, int64_t* positions, int64_t* slot_mapping, int32_t* cache_seqlens,
    int32_t* block_tables, int max_seqlen_q, void* stream) {
  if (num_seqs < 0 || pad_seqs < num_seqs || total_q < 0 || block_size <= 0 ||
      table_width < 0 || max_seqlen_q < 0)
    return MSKV_EINVAL;
  if (pad_seqs == 0) return MSKV_OK;
  // the row outputs may be NULL only when there are no rows to write
  if (total_q + (pad_seqs - num_seqs) > 0 && (!input_ids || !positions || !slot_mapping))
    return MSKV_EINVAL;
  if (total_q > 0 && !token_ids) return MSKV_EINVAL;
  if (num_seqs > 0 && (!seq_start || !cu_seqlens_q || !table_offsets || !tables))
    return MSKV_EINVAL;
  if (pad_seqs > 65535) return MSKV_EUNSUPPORTED;  // grid y limit
  const int span = max_seqlen_q > table_width ? max_seqlen_q : table_width;
  int gx = (span + mskv::kStepThreads - 1) / mskv::kStepThreads;
  gx = gx < 1 ? 1 : (gx > 1024 ? 1024 : gx);
  mskv::StepArgs a{token_ids, seq_start, cu_seqlens_q, table_offsets, tables,
                   input_ids, positions, slot_mapping, cache_seqlens, block_tables,
                   num_seqs, pad_seqs, block_size, table_width, total_q, garbage_slot};
  hipLaunchKernelGGL(mskv::step_inputs_kernel, dim3(gx, pad_seqs), dim3(mskv::kStepThreads), 0,
                     reinterpret_cast<hipStream_t>(stream), a);
  return (int)hipGetLastError();
}
