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
//     from HBM exactly once instead of once per query head.
//   * Each of the 4 waves walks 32-key steps (two 16-key runs; block_size is a multiple of 16, so a
//     run never crosses a block).  K rows are loaded directly in A-operand layout (16 contiguous
//     bytes per lane); V rows are loaded as 16-byte chunks and transposed in registers into the V^T
//     A operand (8 keys x 8 dims per lane), so nothing goes through LDS in the key loop.
//   * The key loop is software-pipelined: the loads of step s+1 are in flight while step s is
//     computed, so each wave keeps two steps (32 KB) of HBM traffic outstanding.
//   * S^T = K Q^T leaves one query head per lane column and 4 keys per lane, which is the B-operand
//     layout of O^T += V^T P^T: softmax state stays in registers.
//   * The 4 waves' partial (m, l, O) are merged in LDS.  A row that fits in one split is finished in
//     place.  Longer rows write fp32 partials that fa2_combine_kernel merges (log-sum-exp rescale).
//     The merge is a second kernel on purpose: merging in the last-arriving work-group needs an
//     agent-scope release/acquire, which on gfx950 writes back / invalidates the XCD's whole L2
//     and cost far more than the extra launch.
#include "fa2_common.h"

namespace mi_fa2 {

constexpr int kDcWaves = 4;
constexpr int kDcStep = 32;   // keys per wave step
constexpr int kRedPitch = kHeadDim + 4;

#ifndef MI_FA2_DC_NT
#define MI_FA2_DC_NT 1
#endif

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

// Streaming 16-byte load of K/V (MI_FA2_DC_NT=1 marks it non-temporal).
__device__ __forceinline__ u32x4 ld16_kv(const uint16_t* ptr) {
#if MI_FA2_DC_NT
  return __builtin_nontemporal_load(reinterpret_cast<const u32x4*>(ptr));
#else
  return ld16(ptr);
#endif
}

// One wave step's operands: K in A layout, V rows for the in-register transpose.
struct DcStep {
  u32x4 ka[2][4];
  u32x4 va[2][4];
};

template <int MODE>
__device__ __forceinline__ void dc_load(const FwdParams& p, int b, int64_t k_off, int64_t v_off,
                                        int kb, int k_end, int n, int g, DcStep& s) {
#pragma unroll
  for (int hf = 0; hf < 2; ++hf) {
    const int t = kb + 16 * hf;
    const uint16_t* kr = t < k_end ? dc_run<MODE>(p, p.k, k_off, p.k_st, b, t) : nullptr;
    const uint16_t* vr = t < k_end ? dc_run<MODE>(p, p.v, v_off, p.v_st, b, t) : nullptr;
    // K as the A operand: lane row n is token t + n, slots cover d = 32*ks + 8*g + [0, 8).
    const bool kok = kr != nullptr && t + n < k_end;
#pragma unroll
    for (int ks = 0; ks < 4; ++ks)
      s.ka[hf][ks] = kok ? ld16_kv(kr + (int64_t)n * p.k_st + ks * 32 + g * 8) : u32x4{0, 0, 0, 0};
    // V rows for the V^T A operand: token t + 4g + r, dims 8n .. 8n+7.
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      const int tok = 4 * g + r;
      const bool vok = vr != nullptr && t + tok < k_end;
      s.va[hf][r] = vok ? ld16_kv(vr + (int64_t)tok * p.v_st + n * 8) : u32x4{0, 0, 0, 0};
    }
  }
}

template <typename E>
__device__ __forceinline__ void dc_compute(const DcStep& s, const u32x4 (&qb)[4], int kb, int k_end,
                                           int g, float c, float& m_run, float& l_run,
                                           f32x4 (&oacc)[8]) {
  // S^T[key][head]: lane (n, g) holds keys kb + 16*hf + 4*g + r of head column n.
  f32x4 st[2];
#pragma unroll
  for (int hf = 0; hf < 2; ++hf) {
    st[hf] = f32x4{};
#pragma unroll
    for (int ks = 0; ks < 4; ++ks) st[hf] = E::mfma16(s.ka[hf][ks], qb[ks], st[hf]);
  }
  if (kb + kDcStep > k_end) {
#pragma unroll
    for (int hf = 0; hf < 2; ++hf)
#pragma unroll
      for (int r = 0; r < 4; ++r)
        if (kb + 16 * hf + 4 * g + r >= k_end) st[hf][r] = -INFINITY;
  }
  float mx = fmax3(st[0][0], st[0][1], st[0][2]);
  mx = fmax3(mx, st[0][3], st[1][0]);
  mx = fmax3(mx, st[1][1], st[1][2]);
  mx = fmaxf(mx, st[1][3]);
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
    const u32x4 a = {pick16(s.va[0][0][e], s.va[0][1][e], hi),
                     pick16(s.va[0][2][e], s.va[0][3][e], hi),
                     pick16(s.va[1][0][e], s.va[1][1][e], hi),
                     pick16(s.va[1][2][e], s.va[1][3][e], hi)};
    oacc[db] = E::mfma16(a, pb, oacc[db]);
  }
}

// Kernel shape knobs (compile-time; the defaults are the measured best on MI355X):
//   MI_FA2_DC_HPW  kv heads per work-group (1 or 2): with 2, the two heads of a token -- one
//                  contiguous 512-byte row of the cache -- are read by the same work-group at the
//                  same time instead of by two work-groups at different times.
//   MI_FA2_DC_PIPE 1 = two register buffers (next step's loads in flight during this step's math),
//                  0 = one buffer and more resident waves instead.
//   MI_FA2_DC_OCC  minimum waves per SIMD requested from the register allocator.
//   MI_FA2_DC_NT   1 = K/V loads are non-temporal (streamed past the caches they would only evict).
// Measured on the 64-row paged decode (kv_len U[128,8192], 256-key splits): HPW 1 vs 2 within
// noise, PIPE 1 (256 VGPRs, 2 waves/SIMD) 15% slower than PIPE 0 (141 VGPRs, 3 waves/SIMD), NT
// +2..4%.
#ifndef MI_FA2_DC_HPW
#define MI_FA2_DC_HPW 1
#endif
#ifndef MI_FA2_DC_PIPE
#define MI_FA2_DC_PIPE 0
#endif
#ifndef MI_FA2_DC_OCC
#define MI_FA2_DC_OCC 2
#endif

template <typename E, int MODE, int HPW>
__global__ __launch_bounds__(256, MI_FA2_DC_OCC) void fa2_decode_kernel(const FwdParams p) {
  // Per-wave partials for the merge: O [wave][column][d], then m and l [wave][column].
  extern __shared__ float red[];
  float* red_o = red;
  float* red_m = red + kDcWaves * p.group * kRedPitch;
  float* red_l = red_m + kDcWaves * p.group;

  const int split = blockIdx.x;
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
  // Wave w serves kv head blockIdx.y*HPW + w%HPW and walks every (4/HPW)-th step of the split.
  constexpr int kStreams = kDcWaves / HPW;
  const int hk = blockIdx.y * HPW + wave % HPW;
  const int stream = wave / HPW;

  const int64_t k_off = (MODE == kDense ? (int64_t)b * p.k_sb : 0) + (int64_t)hk * p.k_sh;
  const int64_t v_off = (MODE == kDense ? (int64_t)b * p.v_sb : 0) + (int64_t)hk * p.v_sh;

  // Q^T as the B operand of S^T = K Q^T: k-step ks covers d = 32*ks + 8*g + [0, 8).
  u32x4 qb[4];
  if (n < p.group) {
    const uint16_t* qp = p.q + (int64_t)b * p.q_sb + (int64_t)(hk * p.group + n) * p.q_sh + g * 8;
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

  constexpr int kStride = kStreams * kDcStep;
  int kb = k_begin + stream * kDcStep;
#if MI_FA2_DC_PIPE
  // Software-pipelined walk (two register buffers): step s+1's loads fly during step s's math.
  DcStep s0, s1;
  if (kb < k_end) dc_load<MODE>(p, b, k_off, v_off, kb, k_end, n, g, s0);
  while (kb < k_end) {
    const int kb1 = kb + kStride;
    if (kb1 < k_end) dc_load<MODE>(p, b, k_off, v_off, kb1, k_end, n, g, s1);
    dc_compute<E>(s0, qb, kb, k_end, g, c, m_run, l_run, oacc);
    if (kb1 >= k_end) break;
    const int kb2 = kb1 + kStride;
    if (kb2 < k_end) dc_load<MODE>(p, b, k_off, v_off, kb2, k_end, n, g, s0);
    dc_compute<E>(s1, qb, kb1, k_end, g, c, m_run, l_run, oacc);
    kb = kb2;
  }
#else
  for (; kb < k_end; kb += kStride) {
    DcStep s0;
    dc_load<MODE>(p, b, k_off, v_off, kb, k_end, n, g, s0);
    dc_compute<E>(s0, qb, kb, k_end, g, c, m_run, l_run, oacc);
  }
#endif

  // Wave results to LDS. O^T accumulator r of d-block db is d = 8*(4g + r) + db, column n.
  float l_w = l_run + __shfl_xor(l_run, 16);
  l_w += __shfl_xor(l_w, 32);
  if (n < p.group) {
    float* ro = red_o + (wave * p.group + n) * kRedPitch;
#pragma unroll
    for (int db = 0; db < 8; ++db)
#pragma unroll
      for (int r = 0; r < 4; ++r) ro[8 * (4 * g + r) + db] = oacc[db][r];
    if (g == 0) {
      red_m[wave * p.group + n] = m_run;
      red_l[wave * p.group + n] = l_w;
    }
  }
  __syncthreads();

  // Merge the waves of each head: outputs (head sub-index, column, d).
  const bool single = n_splits == 1;
  for (int idx = tid; idx < HPW * p.group * kHeadDim; idx += 256) {
    const int hs = idx / (p.group * kHeadDim);
    const int col = (idx / kHeadDim) % p.group;
    const int d = idx % kHeadDim;
    float M = -INFINITY;
#pragma unroll
    for (int j = 0; j < kStreams; ++j) M = fmaxf(M, red_m[(hs + HPW * j) * p.group + col]);
    const float M_use = M == -INFINITY ? 0.f : M;
    float acc = 0.f, L = 0.f;
#pragma unroll
    for (int j = 0; j < kStreams; ++j) {
      const int w = hs + HPW * j;
      const float f = exp2_fast(red_m[w * p.group + col] - M_use);
      acc += red_o[(w * p.group + col) * kRedPitch + d] * f;
      L += red_l[w * p.group + col] * f;
    }
    const int hq = (blockIdx.y * HPW + hs) * p.group + col;
    if (single) {
      const float inv = L > 0.f ? 1.f / L : 0.f;
      uint16_t* op = p.o + (int64_t)b * p.o_sb + (int64_t)hq * p.o_sh + d;
      *op = (uint16_t)(E::pack2(acc * inv, 0.f) & 0xffffu);
      if (p.lse && d == 0)
        p.lse[(int64_t)b * p.l_sb + (int64_t)hq * p.l_sh] =
            L > 0.f ? (M + __builtin_log2f(L)) * kLn2 : -INFINITY;
    } else {
      const int64_t slot = ((int64_t)b * p.Hq + hq) * p.max_splits + split;
      p.ws_o[slot * kHeadDim + d] = acc;
      if (d == 0) {
        p.ws_m[slot] = M;
        p.ws_l[slot] = L;
      }
    }
  }
}

// Merges the split partials of rows that needed more than one split.  Grid (Hq, B), one thread
// per head dimension; the splits are read 16 at a time with every load issued before any is
// used, and folded in with an online log-sum-exp rescale.
template <typename E>
__global__ __launch_bounds__(kHeadDim) void fa2_combine_kernel(const FwdParams p) {
  const int hq = blockIdx.x;
  const int b = blockIdx.y;
  const int kv_len = p.kv_lens ? clamp_len(p.kv_lens[b], p.S) : p.S;
  const int n_splits = kv_len > 0 ? (kv_len + p.chunk - 1) / p.chunk : 1;
  if (n_splits <= 1) return;
  const int d = threadIdx.x;
  const int64_t base = ((int64_t)b * p.Hq + hq) * p.max_splits;
  float M = -INFINITY, L = 0.f, acc = 0.f;
  for (int s0 = 0; s0 < n_splits; s0 += 16) {
    float m[16], l[16], o[16];
#pragma unroll
    for (int i = 0; i < 16; ++i) {
      const int s = s0 + i;
      const bool ok = s < n_splits;
      m[i] = ok ? p.ws_m[base + s] : -INFINITY;
      l[i] = ok ? p.ws_l[base + s] : 0.f;
      o[i] = ok ? p.ws_o[(base + s) * kHeadDim + d] : 0.f;
    }
    float Mn = M;
#pragma unroll
    for (int i = 0; i < 16; ++i) Mn = fmaxf(Mn, m[i]);
    const float Mu = Mn == -INFINITY ? 0.f : Mn;
    const float sc = exp2_fast(M - Mu);
    L *= sc;
    acc *= sc;
#pragma unroll
    for (int i = 0; i < 16; ++i) {
      const float f = exp2_fast(m[i] - Mu);
      L += l[i] * f;
      acc += o[i] * f;
    }
    M = Mn;
  }
  const float inv = L > 0.f ? 1.f / L : 0.f;
  uint16_t* op = p.o + (int64_t)b * p.o_sb + (int64_t)hq * p.o_sh + d;
  *op = (uint16_t)(E::pack2(acc * inv, 0.f) & 0xffffu);
  if (p.lse && d == 0)
    p.lse[(int64_t)b * p.l_sb + (int64_t)hq * p.l_sh] =
        L > 0.f ? (M + __builtin_log2f(L)) * kLn2 : -INFINITY;
}

// Dynamic LDS of the merge: O, m and l of every wave for the group's columns.
static size_t decode_lds_bytes(int group) {
  return (size_t)kDcWaves * group * (kRedPitch + 2) * sizeof(float);
}

template <typename E, int MODE, int HPW>
static hipError_t launch_decode_t(const FwdParams& p, hipStream_t stream) {
  dim3 grid(p.max_splits, p.Hkv / HPW, p.B);
  hipLaunchKernelGGL((fa2_decode_kernel<E, MODE, HPW>), grid, dim3(256),
                     decode_lds_bytes(p.group), stream, p);
  hipError_t err = hipGetLastError();
  if (err != hipSuccess || p.max_splits <= 1) return err;
  hipLaunchKernelGGL((fa2_combine_kernel<E>), dim3(p.Hq, p.B), dim3(kHeadDim), 0, stream, p);
  return hipGetLastError();
}

template <typename E, int MODE>
static hipError_t launch_decode_m(const FwdParams& p, hipStream_t stream) {
  if (p.B == 0) return hipSuccess;
  if (MI_FA2_DC_HPW == 2 && p.Hkv % 2 == 0) return launch_decode_t<E, MODE, 2>(p, stream);
  return launch_decode_t<E, MODE, 1>(p, stream);
}

hipError_t launch_decode(const FwdParams& p, int dtype, int mode, hipStream_t stream) {
  if (dtype == 0)
    return mode == kPaged ? launch_decode_m<BF16, kPaged>(p, stream)
                          : launch_decode_m<BF16, kDense>(p, stream);
  return mode == kPaged ? launch_decode_m<FP16, kPaged>(p, stream)
                        : launch_decode_m<FP16, kDense>(p, stream);
}

}  // namespace mi_fa2
