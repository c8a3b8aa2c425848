// Fused last-position token sampler: one pass over each row's logits draws the row's next token.
//
// Replaces the reference's batched sampling (chat.py:103-107): probs = softmax(logits / T) and
// torch.multinomial(probs, 1), which on the GPU are about eight launches per step (the float cast,
// the scaled softmax's max / sum / normalise passes, the exponential draw, the divide, the argmax).
// torch.multinomial draws one sample per row by the exponential race, argmax_v probs_v / E_v with
// E_v ~ Exp(1); in log space the softmax normaliser cancels and the draw is
//
//     token = argmax_v ( logit_v / T - ln E_v ),   E_v = -ln U_v,
//
// so the logits are read once, with no max or sum pass.  T <= 0 is greedy (argmax of the logits).
// Ties go to the lowest index; NaN scores never win; a row with no candidate gets -1.
//
// Uniforms: Philox4x32-10 (Salmon et al., SC 2011), key = the 64-bit seed, counter = (v / 4, row,
// offset low, offset high); word v % 4 of that block is entry v's, mapped to
// U = (2 * (x >> 9) + 1) * 2^-24, exact in fp32 and strictly inside (0, 1).  A caller advances
// `offset` once per call, so every (row, step) draws fresh numbers, reproducibly from the seed.
//
// Work split: work-group (chunk, row) scans 8192 entries (256 threads x 8 Philox blocks of 4
// consecutive entries; consecutive threads take consecutive blocks) and keeps the best
// (score, index); a second one-wave-per-row kernel reduces the chunks' winners.  A row that fits in
// one chunk is finished by the first kernel.
#include "fa2_common.h"

namespace mi_fa2 {

constexpr int kSmpThreads = 256;
constexpr int kSmpBlocksPerThread = 8;                              // Philox blocks per thread
constexpr int kSmpChunk = kSmpThreads * kSmpBlocksPerThread * 4;   // 8192 entries per work-group

constexpr uint32_t kPhiloxM0 = 0xD2511F53u, kPhiloxM1 = 0xCD9E8D57u;
constexpr uint32_t kPhiloxW0 = 0x9E3779B9u, kPhiloxW1 = 0xBB67AE85u;

__device__ __forceinline__ void philox4x32_10(uint32_t (&c)[4], uint32_t k0, uint32_t k1) {
#pragma unroll
  for (int r = 0; r < 10; ++r) {
    if (r) {
      k0 += kPhiloxW0;
      k1 += kPhiloxW1;
    }
    const uint32_t hi0 = __umulhi(kPhiloxM0, c[0]), lo0 = kPhiloxM0 * c[0];
    const uint32_t hi1 = __umulhi(kPhiloxM1, c[2]), lo1 = kPhiloxM1 * c[2];
    const uint32_t n0 = hi1 ^ c[1] ^ k0, n2 = hi0 ^ c[3] ^ k1;
    c[0] = n0;
    c[1] = lo1;
    c[2] = n2;
    c[3] = lo0;
  }
}

template <int DT>
__device__ __forceinline__ float load_logit(const void* base, int64_t i) {
  if constexpr (DT == 0) {
    return __uint_as_float((uint32_t)static_cast<const uint16_t*>(base)[i] << 16);
  } else if constexpr (DT == 1) {
    return (float)static_cast<const _Float16*>(base)[i];
  } else {
    return static_cast<const float*>(base)[i];
  }
}

// (s, i) beats (bs, bi): higher score, or the same finite-or-+inf score at a lower index.
__device__ __forceinline__ bool better(float s, int i, float bs, int bi) {
  return s > bs || (s == bs && i >= 0 && (bi < 0 || i < bi));
}

__device__ __forceinline__ void wave_best(float& s, int& i) {
#pragma unroll
  for (int d = 32; d >= 1; d >>= 1) {
    const float os = __shfl_xor(s, d);
    const int oi = __shfl_xor(i, d);
    if (better(os, oi, s, i)) {
      s = os;
      i = oi;
    }
  }
}

template <int DT>
__global__ __launch_bounds__(kSmpThreads) void sample_chunk_kernel(const SampleParams p) {
  const int row = blockIdx.y, chunk = blockIdx.x, tid = threadIdx.x;
  const void* base = static_cast<const char*>(p.logits) +
                     (int64_t)row * p.row_stride * (DT == 2 ? 4 : 2);
  float best_s = -INFINITY;
  int best_i = -1;
  const int g0 = chunk * (kSmpChunk / 4);
#pragma unroll 2
  for (int j = 0; j < kSmpBlocksPerThread; ++j) {
    const int g = g0 + j * kSmpThreads + tid;   // Philox block = entries 4g .. 4g+3
    if (4 * g >= p.vocab) break;
    uint32_t w[4] = {(uint32_t)g, (uint32_t)row, p.off_lo, p.off_hi};
    if (!p.greedy) philox4x32_10(w, p.seed_lo, p.seed_hi);
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      const int v = 4 * g + e;
      if (v >= p.vocab) break;
      float s = load_logit<DT>(base, v);
      if (!p.greedy) {
        const float u = (float)(2u * (w[e] >> 9) + 1u) * 0x1p-24f;
        s = s * p.inv_t - logf(-logf(u));
      }
      if (s > best_s) {   // v increases within a thread: strict > keeps the lowest index
        best_s = s;
        best_i = v;
      }
    }
  }
  wave_best(best_s, best_i);
  __shared__ float ws_s[kSmpThreads / 64];
  __shared__ int ws_i[kSmpThreads / 64];
  const int lane = tid & 63, wave = tid >> 6;
  if (lane == 0) {
    ws_s[wave] = best_s;
    ws_i[wave] = best_i;
  }
  __syncthreads();
  if (tid == 0) {
#pragma unroll
    for (int k = 1; k < kSmpThreads / 64; ++k)
      if (better(ws_s[k], ws_i[k], best_s, best_i)) {
        best_s = ws_s[k];
        best_i = ws_i[k];
      }
    if (p.chunks == 1) {
      p.tokens[row] = best_i;
    } else {
      p.part_s[(int64_t)row * p.chunks + chunk] = best_s;
      p.part_i[(int64_t)row * p.chunks + chunk] = best_i;
    }
  }
}

__global__ __launch_bounds__(64) void sample_reduce_kernel(const SampleParams p) {
  const int row = blockIdx.x, lane = threadIdx.x;
  float best_s = -INFINITY;
  int best_i = -1;
  for (int c = lane; c < p.chunks; c += 64) {
    const float s = p.part_s[(int64_t)row * p.chunks + c];
    const int i = p.part_i[(int64_t)row * p.chunks + c];
    if (better(s, i, best_s, best_i)) {
      best_s = s;
      best_i = i;
    }
  }
  wave_best(best_s, best_i);
  if (lane == 0) p.tokens[row] = best_i;
}

int sample_chunks(int vocab) { return (vocab + kSmpChunk - 1) / kSmpChunk; }

hipError_t launch_sample(const SampleParams& p, int dtype, hipStream_t stream) {
  const dim3 grid(p.chunks, p.batch);
  if (dtype == 0)
    hipLaunchKernelGGL((sample_chunk_kernel<0>), grid, dim3(kSmpThreads), 0, stream, p);
  else if (dtype == 1)
    hipLaunchKernelGGL((sample_chunk_kernel<1>), grid, dim3(kSmpThreads), 0, stream, p);
  else
    hipLaunchKernelGGL((sample_chunk_kernel<2>), grid, dim3(kSmpThreads), 0, stream, p);
  if (p.chunks > 1)
    hipLaunchKernelGGL(sample_reduce_kernel, dim3(p.batch), dim3(64), 0, stream, p);
  return hipGetLastError();
}

}  // namespace mi_fa2
