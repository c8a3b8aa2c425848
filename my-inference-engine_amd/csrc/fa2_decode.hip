// Decode (one query token per row) FlashAttention-2 forward for gfx950, split over the keys.
//
// Replaces the Triton kernel fa2_forward in its decode regime (kernels/fa2.py:14-162 with
// SEQLEN_Q = 1, Br=16, Bc=64, kernels/fa2.py:11; called non-causal, model.py:185) together with the
// dense gather that fed it (KVCache.read, kv_cache.py:117-121): in paged mode the keys are read
// straight out of the cache's blocks through the block table.
//
// Decode is HBM-bound (about 6 flop per K/V byte), so the design is about bytes in flight:
//   * Work-group = (split of keys, kv head, row).  All `group` query heads that share the kv head
//     (6 for Qwen2.5: 12q/2kv) are the N columns of one 16x16x32 MFMA, so every K/V byte is read
//     from HBM exactly once per step instead of once per query head.
//   * Each of the 4 waves walks 32-key steps (two 16-key runs; block_size is a multiple of 16, so a
//     run never crosses a block).  K rows are loaded directly in A-operand layout (16 contiguous
//     bytes per lane); V rows are loaded as 16-byte chunks and transposed in registers into the V^T
//     A operand (8 keys x 8 dims per lane), so nothing goes through LDS in the key loop.
//   * S^T = K Q^T leaves one query head per lane column and 4 keys per lane, which is the B-operand
//     layout of O^T += V^T P^T: softmax state stays in registers.
//   * The 4 waves' partial (m, l, O) are merged in LDS.  A row that fits in one split is finished in
//     place; longer rows write fp32 partials that fa2_combine_kernel merges (log-sum-exp rescale).
#include "fa2_common.h"

namespace mi_fa2 {

constexpr int kDcWaves = 4;
constexpr int kDcStep = 32;  // keys per wave step

template <int MODE>
__device__ __forceinline__ const uint16_t* dc_run(const FwdParams& p, const uint16_t* base,
                                                  int64_t off, int64_t st, int b, int t) {
  // Pointer to token t (a multiple of 16) of row b; the next 15 tokens follow at stride st.
  if constexpr (MODE == kPaged) {
    const int bs_shift = __builtin_ctz(p.block_size);
    const int blk = p.block_table[(int64_t)b * p.bt_stride + (t >> bs_shift)];
    if ((unsigned)blk >= (unsigned)p.num_blocks) return nullptr;
    const int64_t slot = ((int64_t)blk << bs_shift) + (t & (p.block_size - 1));
    return base + off + slot * st;
  } else {
    return base + off + (int64_t)t * st;
  }
}

// Lower or upper 16 bits of x and y packed as (x, y).
__device__ __forceinline__ uint32_t pick16(uint32_t x, uint32_t y, bool hi) {
  return hi ? ((x >> 16) | (y & 0xffff0000u)) : ((x & 0xffffu) | (y << 16));
}

template <typename E, int MODE>
__global__ __launch_bounds__(256, 2) void fa2_decode_kernel(const FwdParams p) {
  __shared__ float red_o[kDcWaves][16][kHeadDim + 4];
  __shared__ float red_m[kDcWaves][16];
  __shared__ float red_l[kDcWaves][16];

  const int split = blockIdx.x;
  const int hk = blockIdx.y;
  const int b = blockIdx.z;
  const int kv_len = p.kv_lens ? clamp_len(p.kv_lens[b], p.S) : p.S;
  const int n_splits = kv_len > 0 ? (kv_len + p.chunk - 1) / p.chunk : 1;
  if (split >= n_splits) return;
  const int k_begin = split * p.chunk;
  const int k_end = min(kv_len, k_begin + p.chunk);

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int n = lane & 15;  // MFMA column: query head hk*group + n; also the A-operand row
  const int g = lane >> 4;  // lane group: k-slots 8g..8g+7

  const int64_t k_off = (MODE == kDense ? (int64_t)b * p.k_sb : 0) + (int64_t)hk * p.k_sh;
  const int64_t v_off = (MODE == kDense ? (int64_t)b * p.v_sb : 0) + (int64_t)hk * p.v_sh;

  // Q^T as the B operand of S^T = K Q^T: k-step ks covers d = 32*ks + 8*g + [0, 8).
  u32x4 qb[4];
  const bool col_valid = n < p.group;
  const int hq = hk * p.group + n;
  if (col_valid) {
    const uint16_t* qp = p.q + (int64_t)b * p.q_sb + (int64_t)hq * p.q_sh + g * 8;
#pragma unroll
    for (int ks = 0; ks < 4; ++ks) qb[ks] = ld16(qp + ks * 32);
  } else {
#pragma unroll
    for (int ks = 0; ks < 4; ++ks) qb[ks] = u32x4{0, 0, 0, 0};
  }

  f32x4 oacc[8];
#pragma unroll
  for (int i = 0; i < 8; ++i) oacc[i] = f32x4{};
  float m_run = -INFINITY;
  float l_run = 0.f;
  const float c = p.scale_log2;

  for (int kb = k_begin + wave * kDcStep; kb < k_end; kb += kDcWaves * kDcStep) {
    // Two 16-key runs: tokens kb + 16*hf + [0, 16).
    const uint16_t* kr[2];
    const uint16_t* vr[2];
#pragma unroll
    for (int hf = 0; hf < 2; ++hf) {
      const int t = kb + 16 * hf;
      kr[hf] = t < k_end ? dc_run<MODE>(p, p.k, k_off, p.k_st, b, t) : nullptr;
      vr[hf] = t < k_end ? dc_run<MODE>(p, p.v, v_off, p.v_st, b, t) : nullptr;
    }
    // K as the A operand: lane row n is token kb + 16*hf + n, slots cover d = 32*ks + 8*g + [0,8).
    u32x4 ka[2][4];
#pragma unroll
    for (int hf = 0; hf < 2; ++hf) {
      const bool ok = kr[hf] != nullptr && kb + 16 * hf + n < k_end;
#pragma unroll
      for (int ks = 0; ks < 4; ++ks)
        ka[hf][ks] = ok ? ld16(kr[hf] + (int64_t)n * p.k_st + ks * 32 + g * 8) : u32x4{0, 0, 0, 0};
    }
    // V rows for the V^T A operand: token kb + 16*hf + 4*g + r, dims 8n .. 8n+7.
    u32x4 va[2][4];
#pragma unroll
    for (int hf = 0; hf < 2; ++hf) {
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        const int tok = 4 * g + r;
        const bool ok = vr[hf] != nullptr && kb + 16 * hf + tok < k_end;
        va[hf][r] = ok ? ld16(vr[hf] + (int64_t)tok * p.v_st + n * 8) : u32x4{0, 0, 0, 0};
      }
    }

    // S^T[key][head]: lane (n, g) holds keys kb + 16*hf + 4*g + r of head column n.
    f32x4 st[2];
#pragma unroll
    for (int hf = 0; hf < 2; ++hf) {
      st[hf] = f32x4{};
#pragma unroll
      for (int ks = 0; ks < 4; ++ks) st[hf] = E::mfma16(ka[hf][ks], qb[ks], st[hf]);
    }
#pragma unroll
    for (int hf = 0; hf < 2; ++hf)
#pragma unroll
      for (int r = 0; r < 4; ++r)
        if (kb + 16 * hf + 4 * g + r >= k_end) st[hf][r] = -INFINITY;

    float mx = fmaxf(fmaxf(st[0][0], st[0][1]), fmaxf(st[0][2], st[0][3]));
    mx = fmaxf(mx, fmaxf(fmaxf(st[1][0], st[1][1]), fmaxf(st[1][2], st[1][3])));
    mx = fmaxf(mx, __shfl_xor(mx, 16));
    mx = fmaxf(mx, __shfl_xor(mx, 32));
    const float m_new = fmaxf(m_run, mx * c);
    const float m_use = m_new == -INFINITY ? 0.f : m_new;
    const float alpha = exp2_fast(m_run - m_use);
    float ls = 0.f;
#pragma unroll
    for (int hf = 0; hf < 2; ++hf)
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        st[hf][r] = exp2_fast(__builtin_fmaf(st[hf][r], c, -m_use));
        ls += st[hf][r];
      }
    l_run = l_run * alpha + ls;
    m_run = m_new;
#pragma unroll
    for (int i = 0; i < 8; ++i) oacc[i] *= alpha;

    // P^T as the B operand: slot t <-> key 16*(t/4) + 4*g + t%4.
    const u32x4 pb = {E::pack2(st[0][0], st[0][1]), E::pack2(st[0][2], st[0][3]),
                      E::pack2(st[1][0], st[1][1]), E::pack2(st[1][2], st[1][3])};

    // V^T A operand for d-block db: row n <-> d = 8n + db, slot t <-> the same key as above.
#pragma unroll
    for (int db = 0; db < 8; ++db) {
      const int e = db >> 1;
      const bool hi = db & 1;
      const u32x4 a = {pick16(va[0][0][e], va[0][1][e], hi), pick16(va[0][2][e], va[0][3][e], hi),
                       pick16(va[1][0][e], va[1][1][e], hi), pick16(va[1][2][e], va[1][3][e], hi)};
      oacc[db] = E::mfma16(a, pb, oacc[db]);
    }
  }

  // Wave results to LDS. O^T accumulator r of d-block db is d = 8*(4g + r) + db, column n.
  float l_w = l_run + __shfl_xor(l_run, 16);
  l_w += __shfl_xor(l_w, 32);
#pragma unroll
  for (int db = 0; db < 8; ++db)
#pragma unroll
    for (int r = 0; r < 4; ++r) red_o[wave][n][8 * (4 * g + r) + db] = oacc[db][r];
  if (g == 0) {
    red_m[wave][n] = m_run;
    red_l[wave][n] = l_w;
  }
  __syncthreads();

  const bool single = n_splits == 1;
  for (int idx = tid; idx < p.group * kHeadDim; idx += 256) {
    const int col = idx / kHeadDim;
    const int d = idx % kHeadDim;
    float M = red_m[0][col];
#pragma unroll
    for (int w = 1; w < kDcWaves; ++w) M = fmaxf(M, red_m[w][col]);
    const float M_use = M == -INFINITY ? 0.f : M;
    float acc = 0.f, L = 0.f;
#pragma unroll
    for (int w = 0; w < kDcWaves; ++w) {
      const float f = exp2_fast(red_m[w][col] - M_use);
      acc += red_o[w][col][d] * f;
      L += red_l[w][col] * f;
    }
    const int hq_o = hk * p.group + col;
    if (single) {
      const float inv = L > 0.f ? 1.f / L : 0.f;
      uint16_t* op = p.o + (int64_t)b * p.o_sb + (int64_t)hq_o * p.o_sh + d;
      *op = (uint16_t)(E::pack2(acc * inv, 0.f) & 0xffffu);
      if (p.lse && d == 0)
        p.lse[(int64_t)b * p.l_sb + (int64_t)hq_o * p.l_sh] =
            L > 0.f ? (M + __builtin_log2f(L)) * kLn2 : -INFINITY;
    } else {
      const int64_t slot = ((int64_t)b * p.Hq + hq_o) * p.max_splits + split;
      p.ws_o[slot * kHeadDim + d] = acc;
      if (d == 0) {
        p.ws_m[slot] = M;
        p.ws_l[slot] = L;
      }
    }
  }
}

// Merges the split partials of rows that needed more than one split.  Grid (Hq, B), one wave.
template <typename E>
__global__ __launch_bounds__(64) void fa2_combine_kernel(const FwdParams p) {
  const int hq = blockIdx.x;
  const int b = blockIdx.y;
  const int kv_len = p.kv_lens ? clamp_len(p.kv_lens[b], p.S) : p.S;
  const int n_splits = kv_len > 0 ? (kv_len + p.chunk - 1) / p.chunk : 1;
  if (n_splits <= 1) return;
  const int lane = threadIdx.x;
  const int64_t base = ((int64_t)b * p.Hq + hq) * p.max_splits;
  float M = -INFINITY;
  for (int s = 0; s < n_splits; ++s) M = fmaxf(M, p.ws_m[base + s]);
  const float M_use = M == -INFINITY ? 0.f : M;
  float L = 0.f, o0 = 0.f, o1 = 0.f;
  for (int s = 0; s < n_splits; ++s) {
    const float f = exp2_fast(p.ws_m[base + s] - M_use);
    L += p.ws_l[base + s] * f;
    const float* src = p.ws_o + (base + s) * kHeadDim + 2 * lane;
    o0 += src[0] * f;
    o1 += src[1] * f;
  }
  const float inv = L > 0.f ? 1.f / L : 0.f;
  uint16_t* op = p.o + (int64_t)b * p.o_sb + (int64_t)hq * p.o_sh + 2 * lane;
  *reinterpret_cast<uint32_t*>(op) = E::pack2(o0 * inv, o1 * inv);
  if (p.lse && lane == 0)
    p.lse[(int64_t)b * p.l_sb + (int64_t)hq * p.l_sh] =
        L > 0.f ? (M + __builtin_log2f(L)) * kLn2 : -INFINITY;
}

template <typename E, int MODE>
static hipError_t launch_decode_t(const FwdParams& p, hipStream_t stream) {
  if (p.B == 0) return hipSuccess;
  dim3 grid(p.max_splits, p.Hkv, p.B);
  hipLaunchKernelGGL((fa2_decode_kernel<E, MODE>), grid, dim3(256), 0, stream, p);
  hipError_t err = hipGetLastError();
  if (err != hipSuccess || p.max_splits <= 1) return err;
  hipLaunchKernelGGL((fa2_combine_kernel<E>), dim3(p.Hq, p.B), dim3(64), 0, stream, p);
  return hipGetLastError();
}

hipError_t launch_decode(const FwdParams& p, int dtype, int mode, hipStream_t stream) {
  if (dtype == 0)
    return mode == kPaged ? launch_decode_t<BF16, kPaged>(p, stream)
                          : launch_decode_t<BF16, kDense>(p, stream);
  return mode == kPaged ? launch_decode_t<FP16, kPaged>(p, stream)
                        : launch_decode_t<FP16, kDense>(p, stream);
}

}  // namespace mi_fa2
