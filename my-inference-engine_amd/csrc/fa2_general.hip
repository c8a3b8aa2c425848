// Forward attention over the rest of the reference's input envelope (kernels/fa2.py:164-214):
// head dims d (Q, K) and d_v (V, O) that are any powers of two from 16 to 256 and may differ, in
// bf16, fp16 or fp32.  The MFMA prefill and split-KV decode kernels are built for d = d_v = 128 in
// bf16 / fp16, the shape the engine runs; this kernel is what every other shape runs on.
//
// Organisation (gfx950, wave64):
//   * fa2_general_kernel: a work-group = 4 waves on 64 consecutive query rows (16 per wave) of one
//     (row, query head).  Each step stages 64 keys of K and V in LDS (16-byte loads, rows padded
//     by 16 bytes), shared by the 4 waves, two barriers per step; when a step fits 32 KB the next
//     step's rows are loaded into registers while this one computes.
//   * fa2_general_split_kernel, for launches that would leave CUs idle (fewer than 64 query rows,
//     or fewer such work-groups than CUs): the 4 (or 8) waves share 16 query rows and split their
//     keys, loading K and V operands straight from global memory, and merge (m, l, O) through LDS.
//   * S^T = K Q^T leaves lane l with query column l%16 and keys 4*(l/16) + r of a 16-key chunk,
//     which is exactly the B-operand layout of O^T += V^T P^T: P never leaves registers.  16-bit
//     types run both products on v_mfma_f32_16x16x32 (8 consecutive d per lane for the scores,
//     d = 16 on 16x16x16; pairs of 16-key chunks for PV), fp32 on four v_mfma_f32_16x16x4_f32 per
//     16-wide slice.  V^T operands come from ds_read_b64_tr_b16 (16-bit) or 4-byte reads (fp32).
//   * Online softmax as in kernels/fa2.py:136-150, in the exp2 domain (scale * log2(e) folded into
//     the scores), the running max and sum per lane; the 4 lanes of a query exchange their max
//     with two xor shuffles.  P is rounded to the input type before the PV product
//     (kernels/fa2.py:147: Pij.to(Vj.dtype)); fp32 inputs keep fp32 P and fp32 products
//     (input_precision="ieee", kernels/fa2.py:129,147).
//   * Keys a query does not see (past its row's kv_len, or past the causal diagonal aligned to the
//     row's last key, kernels/fa2.py:107-111,132-137) score -inf; K and V are not read past
//     kv_len, so padding contents (even inf / NaN) never reach the output.  A query that sees no
//     key gets O = 0 and LSE = -inf.
#include "fa2_common.h"

namespace mi_fa2 {

struct F32 {};

__device__ __forceinline__ u32x4 ld16_any(const void* p) { return *reinterpret_cast<const u32x4*>(p); }

// Element traits: a "quad" is 4 consecutive elements of one row, the per-lane share of an operand
// over a 16-wide slice of the contraction.
template <class E> struct Gen;

template <> struct Gen<BF16> {
  using T = uint16_t;
  using Quad = i16x4;
  static __device__ __forceinline__ Quad load(const T* p) { return *reinterpret_cast<const Quad*>(p); }
  static __device__ __forceinline__ Quad zero() { return Quad{0, 0, 0, 0}; }
  static __device__ __forceinline__ short load1(const T* p) { return (short)*p; }
  static __device__ __forceinline__ f32x4 mma(const Quad& a, const Quad& b, f32x4 c) {
    return __builtin_amdgcn_mfma_f32_16x16x16bf16_1k(a, b, c, 0, 0, 0);
  }
  // 16x16x32: k-slots 8*(l/16) .. +7 of lane l, eight elements (a0 then a1 for two quads)
  static __device__ __forceinline__ f32x4 mma8(const u32x4& a, const u32x4& b, f32x4 c) {
    return BF16::mfma16(a, b, c);
  }
  static __device__ __forceinline__ T cvt(float x) {
    return __builtin_bit_cast(uint16_t, (__bf16)x);
  }
  static __device__ __forceinline__ Quad pack(f32x4 v) {
    return Quad{(short)cvt(v[0]), (short)cvt(v[1]), (short)cvt(v[2]), (short)cvt(v[3])};
  }
  static __device__ __forceinline__ float sum(const Quad& v) {
    float s = 0.f;
#pragma unroll
    for (int i = 0; i < 4; ++i) s += __uint_as_float((uint32_t)(uint16_t)v[i] << 16);
    return s;
  }
  static __device__ __forceinline__ void store(T* p, f32x4 v) {
    *reinterpret_cast<Quad*>(p) = pack(v);
  }
};

template <> struct Gen<FP16> {
  using T = uint16_t;
  using Quad = i16x4;
  typedef _Float16 h4 __attribute__((ext_vector_type(4)));
  static __device__ __forceinline__ Quad load(const T* p) { return *reinterpret_cast<const Quad*>(p); }
  static __device__ __forceinline__ Quad zero() { return Quad{0, 0, 0, 0}; }
  static __device__ __forceinline__ short load1(const T* p) { return (short)*p; }
  static __device__ __forceinline__ f32x4 mma(const Quad& a, const Quad& b, f32x4 c) {
    return __builtin_amdgcn_mfma_f32_16x16x16f16(__builtin_bit_cast(h4, a),
                                                 __builtin_bit_cast(h4, b), c, 0, 0, 0);
  }
  static __device__ __forceinline__ f32x4 mma8(const u32x4& a, const u32x4& b, f32x4 c) {
    return FP16::mfma16(a, b, c);
  }
  static __device__ __forceinline__ T cvt(float x) {
    return __builtin_bit_cast(uint16_t, (_Float16)x);
  }
  static __device__ __forceinline__ Quad pack(f32x4 v) {
    return Quad{(short)cvt(v[0]), (short)cvt(v[1]), (short)cvt(v[2]), (short)cvt(v[3])};
  }
  static __device__ __forceinline__ float sum(const Quad& v) {
    const h4 h = __builtin_bit_cast(h4, v);
    return ((float)h[0] + (float)h[1]) + ((float)h[2] + (float)h[3]);
  }
  static __device__ __forceinline__ void store(T* p, f32x4 v) {
    *reinterpret_cast<Quad*>(p) = pack(v);
  }
};

template <> struct Gen<F32> {
  using T = float;
  using Quad = f32x4;
  static __device__ __forceinline__ Quad load(const T* p) { return *reinterpret_cast<const Quad*>(p); }
  static __device__ __forceinline__ Quad zero() { return Quad{0.f, 0.f, 0.f, 0.f}; }
  static __device__ __forceinline__ float load1(const T* p) { return *p; }
  // The 16x16x4 MFMA takes one k per lane: element i of every lane's quad is k-slot l/16 of the
  // i-th MFMA, so the four cover the slice (A and B use the same element order).
  static __device__ __forceinline__ f32x4 mma(const Quad& a, const Quad& b, f32x4 c) {
#pragma unroll
    for (int i = 0; i < 4; ++i) c = __builtin_amdgcn_mfma_f32_16x16x4f32(a[i], b[i], c, 0, 0, 0);
    return c;
  }
  static __device__ __forceinline__ T cvt(float x) { return x; }
  static __device__ __forceinline__ Quad pack(f32x4 v) { return v; }
  static __device__ __forceinline__ float sum(const Quad& v) { return (v[0] + v[1]) + (v[2] + v[3]); }
  static __device__ __forceinline__ void store(T* p, f32x4 v) { *reinterpret_cast<Quad*>(p) = v; }
};

constexpr int kGenWaves = 4;
constexpr int kGenRows = 16;  // query rows per wave
constexpr int kGenKeys = 64;  // keys staged in LDS per step: 4 chunks of 16

// V^T operand of chunk c, d-block i out of the LDS V tile (row pitch VP): lane (m, g) holds
// V[16c + 4g + j][16i + m] in element j.  16-bit: one ds_read_b64_tr_b16 (lane 4k+q of a 16-lane
// group points at row 4g + k, columns 4q..4q+3, and receives column m of the 4 rows); fp32: four
// 4-byte reads.
template <class E, int VP>
__device__ __forceinline__ typename Gen<E>::Quad gen_vt(const typename Gen<E>::T* vl, int c, int i,
                                                        int lane) {
  const int g = lane >> 4, m = lane & 15;
  if constexpr (sizeof(typename Gen<E>::T) == 2) {
    const int k = m >> 2, q = m & 3;
    return __builtin_bit_cast(i16x4, ds_read_tr16(vl + (16 * c + 4 * g + k) * VP + 16 * i + 4 * q));
  } else {
    f32x4 r;
#pragma unroll
    for (int j = 0; j < 4; ++j) r[j] = vl[(16 * c + 4 * g + j) * VP + 16 * i + m];
    return r;
  }
}

template <class E, int D, int DV>
__global__ __launch_bounds__(64 * kGenWaves) void fa2_general_kernel(FwdParams p) {
  using G = Gen<E>;
  using T = typename G::T;
  using Quad = typename G::Quad;
  constexpr bool k16 = sizeof(T) == 2;
  // 16-bit types with d >= 32 take the scores on v_mfma_f32_16x16x32 (8 consecutive d per lane:
  // 16-byte operands); d = 16 and fp32 on 16-wide slices.
  constexpr bool kOct = k16 && D >= 32;
  constexpr int kDB = D / 16, kVB = DV / 16, kDO = D / 32;
  constexpr int kEl16 = 16 / sizeof(T);  // elements per 16-byte chunk
  // LDS rows padded by one 16-byte chunk, so that the 16 rows an operand read touches start on
  // different banks.
  constexpr int KP = D + kEl16, VP = DV + kEl16;
  __shared__ __attribute__((aligned(16))) T kl[kGenKeys * KP];
  __shared__ __attribute__((aligned(16))) T vl[kGenKeys * VP];
  const uint32_t wg_linear = blockIdx.x + gridDim.x * (blockIdx.y + gridDim.y * blockIdx.z);
  probe_mark(p.clock_probe, wg_linear, false);

  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int n = lane & 15, g = lane >> 4;
  const int h = blockIdx.y, b = blockIdx.z;
  const int hk = h / p.group;
  const int kv_len = p.kv_lens ? clamp_len(p.kv_lens[b], p.S) : p.S;
  const int off = kv_len - p.T;  // query i sits at key position i + off
  const int wg_q0 = blockIdx.x * kGenWaves * kGenRows;
  const int q0 = wg_q0 + wave * kGenRows;
  const bool wave_on = q0 < p.T;
  const int q = q0 + n;
  // Keys [0, hi) hold every key the queries up to q_last see.
  auto keys_upto = [&](int q_last) {
    return p.causal ? max(0, min(kv_len, q_last + off + 1)) : kv_len;
  };
  const int wave_hi = wave_on ? keys_upto(min(q0 + kGenRows, p.T) - 1) : 0;
  const int wg_hi = keys_upto(min(wg_q0 + kGenWaves * kGenRows, p.T) - 1);

  const T* kp = reinterpret_cast<const T*>(p.k) + b * p.k_sb + hk * p.k_sh;
  const T* vp = reinterpret_cast<const T*>(p.v) + b * p.v_sb + hk * p.v_sh;

  // Q^T as the B operand of the scores: lane (n, g) holds d = 32*s + 8*g .. +7 (kOct) or
  // d = 16*s + 4*g .. +3 of query q.
  u32x4 qo[kOct ? kDO : 1];
  Quad qb[kOct ? 1 : kDB];
  {
    const T* qp = reinterpret_cast<const T*>(p.q) + b * p.q_sb + h * p.q_sh +
                  (int64_t)min(q, p.T - 1) * p.q_st;
    if constexpr (kOct) {
#pragma unroll
      for (int s = 0; s < kDO; ++s) qo[s] = wave_on ? ld16_any(qp + 32 * s + 8 * g) : u32x4{};
    } else {
#pragma unroll
      for (int s = 0; s < kDB; ++s) qb[s] = wave_on ? G::load(qp + 16 * s + 4 * g) : G::zero();
    }
  }

  f32x4 oacc[kVB];
#pragma unroll
  for (int i = 0; i < kVB; ++i) oacc[i] = f32x4{0.f, 0.f, 0.f, 0.f};
  float m_run = -INFINITY, l_run = 0.f;
  const float c = p.scale_log2;

  // K and V rows [kb, kb + 64) in 16-byte chunks; rows past kv_len are zeros (never loaded, so
  // padding contents cannot reach the output).  When a step's K and V fit 32 KB, the next step's
  // chunks are loaded into registers while this step computes (each thread holds 1/256 of the
  // step: 4 VGPRs per 4 KB, at most 32 VGPRs).
  constexpr int kKc = D / kEl16, kVc = DV / kEl16;  // chunks per row
  constexpr int kThreads = 64 * kGenWaves;
  constexpr int kNK = (kGenKeys * kKc + kThreads - 1) / kThreads;
  constexpr int kNV = (kGenKeys * kVc + kThreads - 1) / kThreads;
  constexpr bool kPrefetch = (D + DV) * (int)sizeof(T) <= 512;
  u32x4 nk[kPrefetch ? kNK : 1], nv[kPrefetch ? kNV : 1];
  auto fetch = [&](int kb, u32x4* dk, u32x4* dv) {
#pragma unroll
    for (int i = 0; i < kNK; ++i) {
      const int x = tid + kThreads * i, r = x / kKc, ch = x - r * kKc;
      dk[i] = u32x4{0u, 0u, 0u, 0u};
      if (x < kGenKeys * kKc && kb + r < kv_len)
        dk[i] = ld16_any(kp + (int64_t)(kb + r) * p.k_st + ch * kEl16);
    }
#pragma unroll
    for (int i = 0; i < kNV; ++i) {
      const int x = tid + kThreads * i, r = x / kVc, ch = x - r * kVc;
      dv[i] = u32x4{0u, 0u, 0u, 0u};
      if (x < kGenKeys * kVc && kb + r < kv_len)
        dv[i] = ld16_any(vp + (int64_t)(kb + r) * p.v_st + ch * kEl16);
    }
  };
  auto commit = [&](const u32x4* dk, const u32x4* dv) {
#pragma unroll
    for (int i = 0; i < kNK; ++i) {
      const int x = tid + kThreads * i, r = x / kKc, ch = x - r * kKc;
      if (x < kGenKeys * kKc) *reinterpret_cast<u32x4*>(kl + r * KP + ch * kEl16) = dk[i];
    }
#pragma unroll
    for (int i = 0; i < kNV; ++i) {
      const int x = tid + kThreads * i, r = x / kVc, ch = x - r * kVc;
      if (x < kGenKeys * kVc) *reinterpret_cast<u32x4*>(vl + r * VP + ch * kEl16) = dv[i];
    }
  };
  if constexpr (kPrefetch) {
    if (wg_hi > 0) fetch(0, nk, nv);
  }

  // Every wave runs the same steps (the barriers); a wave skips the compute of keys it does not see.
  for (int kb = 0; kb < wg_hi; kb += kGenKeys) {
    __syncthreads();  // the previous step's LDS reads are done
    if constexpr (kPrefetch) {
      commit(nk, nv);
    } else {
      // one chunk per thread at a time, straight from global memory to LDS
      for (int x = tid; x < kGenKeys * kKc; x += kThreads) {
        const int r = x / kKc, ch = x - r * kKc;
        u32x4 val = {0u, 0u, 0u, 0u};
        if (kb + r < kv_len) val = ld16_any(kp + (int64_t)(kb + r) * p.k_st + ch * kEl16);
        *reinterpret_cast<u32x4*>(kl + r * KP + ch * kEl16) = val;
      }
      for (int x = tid; x < kGenKeys * kVc; x += kThreads) {
        const int r = x / kVc, ch = x - r * kVc;
        u32x4 val = {0u, 0u, 0u, 0u};
        if (kb + r < kv_len) val = ld16_any(vp + (int64_t)(kb + r) * p.v_st + ch * kEl16);
        *reinterpret_cast<u32x4*>(vl + r * VP + ch * kEl16) = val;
      }
    }
    __syncthreads();
    if constexpr (kPrefetch) {
      if (kb + kGenKeys < wg_hi) fetch(kb + kGenKeys, nk, nv);  // in flight during this step
    }
    if (kb >= wave_hi) continue;  // wave-uniform

    // S^T of the 4 chunks: K as the A operand, lane (n, g) = key kb + 16*ch + n.
    // Chunks starting at or past wave_hi hold no key any of the wave's queries sees.
    f32x4 st[4];
#pragma unroll
    for (int ch = 0; ch < 4; ++ch) {
      st[ch] = f32x4{0.f, 0.f, 0.f, 0.f};
      if (kb + 16 * ch < wave_hi) {
        const T* kr = kl + (16 * ch + n) * KP;
        if constexpr (kOct) {
#pragma unroll
          for (int s = 0; s < kDO; ++s)
            st[ch] = G::mma8(*reinterpret_cast<const u32x4*>(kr + 32 * s + 8 * g), qo[s], st[ch]);
        } else {
#pragma unroll
          for (int s = 0; s < kDB; ++s) st[ch] = G::mma(G::load(kr + 16 * s + 4 * g), qb[s], st[ch]);
        }
      }
    }
    // lane (n, g) holds keys kb + 16*ch + 4*g + r of query q
    float mx = -INFINITY;
#pragma unroll
    for (int ch = 0; ch < 4; ++ch)
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        const int key = kb + 16 * ch + 4 * g + r;
        const bool vis = key < kv_len && (!p.causal || key <= q + off);
        st[ch][r] = vis ? st[ch][r] * c : -INFINITY;
        mx = fmaxf(mx, st[ch][r]);
      }
    mx = fmaxf(mx, __shfl_xor(mx, 16));
    mx = fmaxf(mx, __shfl_xor(mx, 32));
    const float m_new = fmaxf(m_run, mx);
    const float m_use = m_new == -INFINITY ? 0.f : m_new;
    const float alpha = exp2_fast(m_run - m_use);
    m_run = m_new;
    // The PV product takes P rounded to the input type (kernels/fa2.py:147); the row sum adds the
    // same rounded values, so that the weights applied to V sum to exactly 1 after the division.
    // (The reference sums P before rounding, kernels/fa2.py:145: in bf16 that leaves the weights
    // off by up to 2^-9 relative, which on outputs near 4 adds up to 8e-3 to the output's own
    // rounding.)  fp32: no rounding, the two are the same.
    Quad pq[4];
    float ls = 0.f;
#pragma unroll
    for (int ch = 0; ch < 4; ++ch) {
      f32x4 pr;
#pragma unroll
      for (int r = 0; r < 4; ++r) pr[r] = exp2_fast(st[ch][r] - m_use);
      pq[ch] = G::pack(pr);
      ls += G::sum(pq[ch]);
    }
    l_run = l_run * alpha + ls;

    // O^T += V^T P^T, d-block by d-block.  16-bit: chunks in pairs on v_mfma_f32_16x16x32, k-slots
    // 8g + j holding key 4g + j of the first chunk (j < 4) and of the second (j >= 4) in both
    // operands; a pair is skipped when its first chunk is (the second then holds P = 0 rows).
#pragma unroll
    for (int i = 0; i < kVB; ++i) {
      f32x4 acc = oacc[i] * alpha;
      if constexpr (k16) {
#pragma unroll
        for (int pr2 = 0; pr2 < 2; ++pr2)
          if (kb + 32 * pr2 < wave_hi) {
            const i16x4 a0 = gen_vt<E, VP>(vl, 2 * pr2, i, lane);
            const i16x4 a1 = gen_vt<E, VP>(vl, 2 * pr2 + 1, i, lane);
            const u32x2 a0w = __builtin_bit_cast(u32x2, a0), a1w = __builtin_bit_cast(u32x2, a1);
            const u32x2 b0w = __builtin_bit_cast(u32x2, pq[2 * pr2]);
            const u32x2 b1w = __builtin_bit_cast(u32x2, pq[2 * pr2 + 1]);
            acc = G::mma8(u32x4{a0w[0], a0w[1], a1w[0], a1w[1]},
                          u32x4{b0w[0], b0w[1], b1w[0], b1w[1]}, acc);
          }
      } else {
#pragma unroll
        for (int ch = 0; ch < 4; ++ch)
          if (kb + 16 * ch < wave_hi) acc = G::mma(gen_vt<E, VP>(vl, ch, i, lane), pq[ch], acc);
      }
      oacc[i] = acc;
    }
  }

  if (!wave_on) return;
  // lane (n, g) holds the sums of keys 4*g + r of every chunk: the 4 lanes of a query add up.
  float l_tot = l_run + __shfl_xor(l_run, 16);
  l_tot += __shfl_xor(l_tot, 32);
  if (q >= p.T) return;
  const float inv = l_tot > 0.f ? 1.f / l_tot : 0.f;
  T* op = reinterpret_cast<T*>(p.o) + b * p.o_sb + h * p.o_sh + (int64_t)q * p.o_st;
  // O^T block i: lane (n, g) holds d = 16*i + 4*g + r of query q.
#pragma unroll
  for (int i = 0; i < kVB; ++i) G::store(op + 16 * i + 4 * g, oacc[i] * inv);
  if (p.lse && g == 0)
    p.lse[b * p.l_sb + h * p.l_sh + (int64_t)q * p.l_st] =
        l_tot > 0.f ? (m_run + __builtin_log2f(l_tot)) * kLn2 : -INFINITY;
  probe_mark(p.clock_probe, wg_linear, true);  // thread 0's query row always exists
}

// Key-split variant for launches that would leave the chip idle: fewer query rows than a
// work-group of fa2_general_kernel holds (decode-shaped calls), or fewer of those work-groups
// than CUs (a short sequence with few heads).  A work-group = W waves on the SAME 16 query rows;
// wave w walks the w-th W-th of the 32-key pairs those rows see, loading its K and V operands
// straight from global memory (no LDS, no barrier in the loop), and the W waves' (m, l, O) are
// merged through LDS at the end, each wave finishing every W-th d-block.  W = 4, or 8 (twice the
// key split) when the grid leaves a whole CU to each work-group (d_v <= 128).
template <class E, int D, int DV, int W>
__global__ __launch_bounds__(64 * W) void fa2_general_split_kernel(FwdParams p) {
  constexpr int kGenWaves = W;
  using G = Gen<E>;
  using T = typename G::T;
  using Quad = typename G::Quad;
  constexpr bool k16 = sizeof(T) == 2;
  constexpr bool kOct = k16 && D >= 32;
  constexpr int kDB = D / 16, kVB = DV / 16, kDO = D / 32;
  __shared__ float sm_m[kGenWaves][kGenRows];
  __shared__ float sm_l[kGenWaves][kGenRows];
  __shared__ f32x4 sm_o[kGenWaves][kVB][64];
  const uint32_t wg_linear = blockIdx.x + gridDim.x * (blockIdx.y + gridDim.y * blockIdx.z);
  probe_mark(p.clock_probe, wg_linear, false);

  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int n = lane & 15, g = lane >> 4;
  const int h = blockIdx.y, b = blockIdx.z;
  const int hk = h / p.group;
  const int kv_len = p.kv_lens ? clamp_len(p.kv_lens[b], p.S) : p.S;
  const int off = kv_len - p.T;  // query i sits at key position i + off
  const int q0 = blockIdx.x * kGenRows;
  const int q = q0 + n;
  const int q_last = min(q0 + kGenRows, p.T) - 1;
  const int hi = p.causal ? max(0, min(kv_len, q_last + off + 1)) : kv_len;
  // this wave's 32-key pairs
  const int n_pairs = (hi + 31) >> 5;
  const int pr_lo = wave * n_pairs / kGenWaves, pr_hi = (wave + 1) * n_pairs / kGenWaves;

  const T* kp = reinterpret_cast<const T*>(p.k) + b * p.k_sb + hk * p.k_sh;
  const T* vp = reinterpret_cast<const T*>(p.v) + b * p.v_sb + hk * p.v_sh;

  u32x4 qo[kOct ? kDO : 1];
  Quad qb[kOct ? 1 : kDB];
  {
    const T* qp = reinterpret_cast<const T*>(p.q) + b * p.q_sb + h * p.q_sh +
                  (int64_t)min(q, p.T - 1) * p.q_st;
    if constexpr (kOct) {
#pragma unroll
      for (int s = 0; s < kDO; ++s) qo[s] = ld16_any(qp + 32 * s + 8 * g);
    } else {
#pragma unroll
      for (int s = 0; s < kDB; ++s) qb[s] = G::load(qp + 16 * s + 4 * g);
    }
  }

  f32x4 oacc[kVB];
#pragma unroll
  for (int i = 0; i < kVB; ++i) oacc[i] = f32x4{0.f, 0.f, 0.f, 0.f};
  float m_run = -INFINITY, l_run = 0.f;
  const float c = p.scale_log2;

  // A pair's V^T gathers are issued with its K loads, before the score MFMAs, so that a pair
  // costs one memory round trip instead of two (when a pair's V fits 512 bytes per row).
  constexpr bool kVPre = DV * (int)sizeof(T) <= 512;
  for (int pr = pr_lo; pr < pr_hi; ++pr) {
    const int kb = 32 * pr;
    Quad vpre[kVPre ? kVB : 1][2];
    if constexpr (kVPre) {
#pragma unroll
      for (int i = 0; i < kVB; ++i)
#pragma unroll
        for (int ch = 0; ch < 2; ++ch)
#pragma unroll
          for (int j = 0; j < 4; ++j) {
            const int key = kb + 16 * ch + 4 * g + j;
            const T* vr = vp + (int64_t)min(key, kv_len - 1) * p.v_st + 16 * i + n;
            vpre[i][ch][j] = key < kv_len ? G::load1(vr) : 0;
          }
    }
    // S^T of the two 16-key chunks: K as the A operand straight from global memory (rows past
    // kv_len read as zero operands, their address clamped to row 0).
    f32x4 st[2];
#pragma unroll
    for (int ch = 0; ch < 2; ++ch) {
      const int kr = kb + 16 * ch + n;
      const bool k_ok = kr < kv_len;
      const T* krow = kp + (int64_t)(k_ok ? kr : 0) * p.k_st;
      st[ch] = f32x4{0.f, 0.f, 0.f, 0.f};
      if constexpr (kOct) {
#pragma unroll
        for (int s = 0; s < kDO; ++s)
          st[ch] = G::mma8(k_ok ? ld16_any(krow + 32 * s + 8 * g) : u32x4{}, qo[s], st[ch]);
      } else {
#pragma unroll
        for (int s = 0; s < kDB; ++s)
          st[ch] = G::mma(k_ok ? G::load(krow + 16 * s + 4 * g) : G::zero(), qb[s], st[ch]);
      }
    }
    float mx = -INFINITY;
#pragma unroll
    for (int ch = 0; ch < 2; ++ch)
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        const int key = kb + 16 * ch + 4 * g + r;
        const bool vis = key < kv_len && (!p.causal || key <= q + off);
        st[ch][r] = vis ? st[ch][r] * c : -INFINITY;
        mx = fmaxf(mx, st[ch][r]);
      }
    mx = fmaxf(mx, __shfl_xor(mx, 16));
    mx = fmaxf(mx, __shfl_xor(mx, 32));
    const float m_new = fmaxf(m_run, mx);
    const float m_use = m_new == -INFINITY ? 0.f : m_new;
    const float alpha = exp2_fast(m_run - m_use);
    m_run = m_new;
    Quad pq[2];
    float ls = 0.f;
#pragma unroll
    for (int ch = 0; ch < 2; ++ch) {
      f32x4 prb;
#pragma unroll
      for (int r = 0; r < 4; ++r) prb[r] = exp2_fast(st[ch][r] - m_use);
      pq[ch] = G::pack(prb);
      ls += G::sum(pq[ch]);  // P as rounded for the PV product (see fa2_general_kernel)
    }
    l_run = l_run * alpha + ls;

    // V^T as the A operand, gathered from global memory: element j of chunk ch is
    // V[kb + 16*ch + 4*g + j][16*i + n] (rows past kv_len read as 0, address clamped).
#pragma unroll
    for (int i = 0; i < kVB; ++i) {
      Quad va[2];
      if constexpr (kVPre) {
        va[0] = vpre[i][0];
        va[1] = vpre[i][1];
      } else {
#pragma unroll
        for (int ch = 0; ch < 2; ++ch)
#pragma unroll
          for (int j = 0; j < 4; ++j) {
            const int key = kb + 16 * ch + 4 * g + j;
            const T* vr = vp + (int64_t)min(key, kv_len - 1) * p.v_st + 16 * i + n;
            va[ch][j] = key < kv_len ? G::load1(vr) : 0;
          }
      }
      f32x4 acc = oacc[i] * alpha;
      if constexpr (k16) {
        const u32x2 a0 = __builtin_bit_cast(u32x2, va[0]), a1 = __builtin_bit_cast(u32x2, va[1]);
        const u32x2 b0 = __builtin_bit_cast(u32x2, pq[0]), b1 = __builtin_bit_cast(u32x2, pq[1]);
        acc = G::mma8(u32x4{a0[0], a0[1], a1[0], a1[1]}, u32x4{b0[0], b0[1], b1[0], b1[1]}, acc);
      } else {
        acc = G::mma(va[0], pq[0], acc);
        acc = G::mma(va[1], pq[1], acc);
      }
      oacc[i] = acc;
    }
  }

  // Merge the 4 waves: lane (n, g) of every wave holds d = 16*i + 4*g + r of query q0 + n.
  float l_w = l_run + __shfl_xor(l_run, 16);
  l_w += __shfl_xor(l_w, 32);
  if (g == 0) {
    sm_m[wave][n] = m_run;
    sm_l[wave][n] = l_w;
  }
#pragma unroll
  for (int i = 0; i < kVB; ++i) sm_o[wave][i][lane] = oacc[i];
  __syncthreads();
  float M = sm_m[0][n];
#pragma unroll
  for (int u = 1; u < kGenWaves; ++u) M = fmaxf(M, sm_m[u][n]);
  const float M_use = M == -INFINITY ? 0.f : M;
  float f[kGenWaves], L = 0.f;
#pragma unroll
  for (int u = 0; u < kGenWaves; ++u) {
    f[u] = exp2_fast(sm_m[u][n] - M_use);
    L += f[u] * sm_l[u][n];
  }
  if (q >= p.T) return;
  const float inv = L > 0.f ? 1.f / L : 0.f;
  T* op = reinterpret_cast<T*>(p.o) + b * p.o_sb + h * p.o_sh + (int64_t)q * p.o_st;
  for (int i = wave; i < kVB; i += kGenWaves) {
    f32x4 o = sm_o[0][i][lane] * f[0];
#pragma unroll
    for (int u = 1; u < kGenWaves; ++u) o += sm_o[u][i][lane] * f[u];
    G::store(op + 16 * i + 4 * g, o * inv);
  }
  if (p.lse && wave == 0 && g == 0)
    p.lse[b * p.l_sb + h * p.l_sh + (int64_t)q * p.l_st] =
        L > 0.f ? (M + __builtin_log2f(L)) * kLn2 : -INFINITY;
  probe_mark(p.clock_probe, wg_linear, true);  // thread 0's query row always exists
}

}  // namespace mi_fa2

namespace mi_fa2 {

namespace {

template <class E, int D, int DV>
hipError_t launch_general_t(const FwdParams& p, hipStream_t stream) {
  const int rows_per_wg = kGenWaves * kGenRows;
  const int64_t tiles = (int64_t)((p.T + rows_per_wg - 1) / rows_per_wg) * p.Hq * p.B;
  // Fewer query rows than a work-group holds, or fewer work-groups than the device's CUs (256 on
  // MI355X): split each 16-row tile's keys over 4 waves instead (4x the work-groups, a quarter of
  // the chain).
  if (p.T < rows_per_wg || tiles < p.n_cus) {
    const dim3 grid((p.T + kGenRows - 1) / kGenRows, p.Hq, p.B);
    // Eight waves when every work-group can have a CU of its own (two waves per SIMD): an fp32
    // call of 16 rows x 1 query x 2,048 keys took 114 -> 84 us; with more work-groups than CUs the
    // four-wave shape, two work-groups per CU, is faster (1 x 12 x 512 fp32: 35.7 against 37.3 us).
    if constexpr (DV <= 128) {
      if ((int64_t)grid.x * grid.y * grid.z <= p.n_cus) {
        hipLaunchKernelGGL((fa2_general_split_kernel<E, D, DV, 8>), grid, dim3(64 * 8), 0, stream,
                           p);
        return hipGetLastError();
      }
    }
    hipLaunchKernelGGL((fa2_general_split_kernel<E, D, DV, 4>), grid, dim3(64 * 4), 0, stream, p);
    return hipGetLastError();
  }
  const dim3 grid((p.T + rows_per_wg - 1) / rows_per_wg, p.Hq, p.B);
  hipLaunchKernelGGL((fa2_general_kernel<E, D, DV>), grid, dim3(64 * kGenWaves), 0, stream, p);
  return hipGetLastError();
}

template <class E, int D>
hipError_t launch_general_dv(const FwdParams& p, int dv, hipStream_t stream) {
  switch (dv) {
    case 16: return launch_general_t<E, D, 16>(p, stream);
    case 32: return launch_general_t<E, D, 32>(p, stream);
    case 64: return launch_general_t<E, D, 64>(p, stream);
    case 128: return launch_general_t<E, D, 128>(p, stream);
    case 256: return launch_general_t<E, D, 256>(p, stream);
  }
  return hipErrorInvalidValue;
}

template <class E>
hipError_t launch_general_e(const FwdParams& p, int d, int dv, hipStream_t stream) {
  switch (d) {
    case 16: return launch_general_dv<E, 16>(p, dv, stream);
    case 32: return launch_general_dv<E, 32>(p, dv, stream);
    case 64: return launch_general_dv<E, 64>(p, dv, stream);
    case 128: return launch_general_dv<E, 128>(p, dv, stream);
    case 256: return launch_general_dv<E, 256>(p, dv, stream);
  }
  return hipErrorInvalidValue;
}

}  // namespace

// dtype: 0 bf16, 1 fp16, 2 fp32; d, dv in {16, 32, 64, 128, 256} (checked by the caller).
hipError_t launch_general(const FwdParams& p, int dtype, int d, int dv, hipStream_t stream) {
  if (p.B == 0 || p.T == 0) return hipSuccess;
  switch (dtype) {
    case 0: return launch_general_e<BF16>(p, d, dv, stream);
    case 1: return launch_general_e<FP16>(p, d, dv, stream);
    case 2: return launch_general_e<F32>(p, d, dv, stream);
  }
  return hipErrorInvalidValue;
}

}  // namespace mi_fa2
