// Per-step paged-cache metadata, built on the device from device-resident block tables.
//
// Replaces the host side of KVCache.prepare (kv_cache.py:74-101): the reference walks every new
// token in Python to build slot_mapping, builds a dense [B, S] gather index, and copies both to the
// GPU each step.  Here every sequence's block table and length live on the device (one row per
// sequence slot, written only when blocks are allocated), and one launch per step derives from the
// rows' slots:
//   starts[b]        tokens row b held before the step (seq_lens[slot]),
//   kv_lens[b]       starts[b] + count_b (model.py:175),
//   block_table[b]   the first ceil(kv_len / block_size) entries of the slot's table, then zeros
//                    (the reference pads with block 0, kv_cache.py:95),
//   slots[i]         cache slot of packed new token i: table[pos / bs] * bs + pos % bs
//                    (kv_cache.py:15-16,88-91), -1 for a padding row,
//   positions[i]     its position in its row (model.py:151-155 input), optional,
//   last_idx[b]      packed index of row b's last new token, optional,
// and advances seq_lens[slot] by count_b, so the next step finds the new length without a copy.
// Row b's tokens are [cu[b], cu[b+1]) of the packed batch, or b*T .. b*T+T-1 when cu is NULL.
// A row whose slot is negative is padding: no keys, nothing written to the cache, no advance.
// A row that would hold more keys than its table row can address is treated the same way.
// Distinct rows must name distinct slots (each work-group reads, then advances, its own slot).
#include "fa2_common.h"

namespace mi_fa2 {

__global__ __launch_bounds__(256) void step_meta_kernel(const StepMetaParams p) {
  const int b = blockIdx.x, tid = threadIdx.x;
  const int s = p.row_slots[b];
  const int t0 = p.cu ? p.cu[b] : b * p.T;
  const int cnt = p.cu ? p.cu[b + 1] - t0 : p.T;
  const bool in_range = s >= 0 && s < p.max_seqs;
  const int start = in_range ? p.seq_lens[s] : 0;
  // a row whose keys would not fit its table row (capacity not ensured: a caller bug) is treated
  // as padding, so no table read leaves the row
  const bool valid = in_range && start >= 0 && cnt >= 0 &&
                     (int64_t)start + cnt <= (int64_t)p.table_stride * p.block_size;
  const int kv = valid ? start + cnt : 0;
  const int used = (kv + p.block_size - 1) / p.block_size;
  const int32_t* table = p.tables + (valid ? (int64_t)s * p.table_stride : 0);
  for (int j = tid; j < p.W; j += blockDim.x)
    p.block_table[(int64_t)b * p.W + j] = (valid && j < used) ? table[j] : 0;
  for (int t = tid; t < cnt; t += blockDim.x) {
    const int pos = start + t;
    p.slots[t0 + t] = valid ? table[pos / p.block_size] * p.block_size + pos % p.block_size : -1;
    if (p.positions) p.positions[t0 + t] = valid ? pos : 0;
  }
  __syncthreads();   // every thread has read seq_lens[s] before it moves
  if (tid == 0) {
    p.starts[b] = start;
    p.kv_lens[b] = kv;
    if (p.last_idx) p.last_idx[b] = t0 + cnt - 1;
    if (valid) p.seq_lens[s] = start + cnt;
  }
}

hipError_t launch_step_meta(const StepMetaParams& p, hipStream_t stream) {
  hipLaunchKernelGGL(step_meta_kernel, dim3(p.B), dim3(256), 0, stream, p);
  return hipGetLastError();
}

}  // namespace mi_fa2
