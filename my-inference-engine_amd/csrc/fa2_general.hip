// Forward attention over the rest of the reference's input envelope (kernels/fa2.py:164-214):
// head dims d (Q, K) and d_v (V, O) that are any powers of two from 16 to 256 and may differ, in
// bf16, fp16 or fp32.  The MFMA prefill and split-KV decode kernels are built for d = d_v = 128 in
// bf16 / fp16, the shape the engine runs; this kernel is what every other shape runs on.
//
// Organisation (gfx950, wave64):
//   * One wave = 16 query rows of one (row, query head); a work-group holds 4 waves on 4
//     consecutive 16-row tiles.  No LDS and no barriers: each wave walks its own keys.
//   * Keys go 16 at a time.  S^T = K Q^T on v_mfma_f32_16x16x16_{bf16,f16} (fp32: 16x16x4_f32, four
//     per 16-wide slice of d) leaves lane l with query column l%16 and keys 4*(l/16) + r of the
//     chunk, which is exactly the B-operand layout of O^T += V^T P^T: P never leaves registers.
//     In every operand lane l holds 4 consecutive d (or 4 consecutive keys) of its row, so K and Q
//     are 8- or 16-byte loads; V^T is gathered one element per key (adjacent lanes read adjacent
//     d of one V row).
//   * Online softmax as in kernels/fa2.py:136-150, in the exp2 domain (scale * log2(e) folded into
//     the scores), the running max and sum per lane; the 4 lanes of a query exchange their chunk
//     max with two xor shuffles.  P is rounded to the input type before the PV product
//     (kernels/fa2.py:147: Pij.to(Vj.dtype)); fp32 inputs keep fp32 P and fp32 products
//     (input_precision="ieee", kernels/fa2.py:129,147).
//   * Keys a query does not see (past its row's kv_len, or past the causal diagonal aligned to the
//     row's last key, kernels/fa2.py:107-111,132-137) score -inf; K and V are not read past
//     kv_len, so padding contents (even inf / NaN) never reach the output.  A query that sees no
//     key gets O = 0 and LSE = -inf.
#include "fa2_common.h"

namespace mi_fa2 {

struct F32 {};

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

template <class E, int D, int DV>
__global__ __launch_bounds__(64 * kGenWaves) void fa2_general_kernel(FwdParams p) {
  using G = Gen<E>;
  using T = typename G::T;
  using Quad = typename G::Quad;
  constexpr int kDB = D / 16, kVB = DV / 16;

  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int n = lane & 15, g = lane >> 4;
  const int q0 = (blockIdx.x * kGenWaves + wave) * kGenRows;
  const int h = blockIdx.y, b = blockIdx.z;
  if (q0 >= p.T) return;
  const int hk = h / p.group;
  const int kv_len = p.kv_lens ? clamp_len(p.kv_lens[b], p.S) : p.S;
  const int off = kv_len - p.T;  // query i sits at key position i + off
  const int q = q0 + n;
  const int q_last = min(q0 + kGenRows, p.T) - 1;
  const int kv_hi = p.causal ? max(0, min(kv_len, q_last + off + 1)) : kv_len;

  const T* qp = reinterpret_cast<const T*>(p.q) + b * p.q_sb + h * p.q_sh +
                (int64_t)min(q, p.T - 1) * p.q_st;
  const T* kp = reinterpret_cast<const T*>(p.k) + b * p.k_sb + hk * p.k_sh;
  const T* vp = reinterpret_cast<const T*>(p.v) + b * p.v_sb + hk * p.v_sh;

  // Q^T as the B operand: lane (n, g) holds d = 16*s + 4*g .. +3 of query q for slice s.
  Quad qb[kDB];
#pragma unroll
  for (int s = 0; s < kDB; ++s) qb[s] = G::load(qp + 16 * s + 4 * g);

  f32x4 oacc[kVB];
#pragma unroll
  for (int i = 0; i < kVB; ++i) oacc[i] = f32x4{0.f, 0.f, 0.f, 0.f};
  float m_run = -INFINITY, l_run = 0.f;
  const float c = p.scale_log2;

  for (int kc = 0; kc < kv_hi; kc += 16) {
    // S^T[key][query]: K as the A operand, lane (n, g) = key kc + n, d = 16*s + 4*g .. +3.
    const int kr = kc + n;
    const bool k_ok = kr < kv_len;
    const T* krow = kp + (int64_t)(k_ok ? kr : 0) * p.k_st + 4 * g;
    f32x4 st = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int s = 0; s < kDB; ++s) st = G::mma(k_ok ? G::load(krow + 16 * s) : G::zero(), qb[s], st);

    // lane (n, g) now holds keys kc + 4*g + r of query q
    float sc[4];
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      const int key = kc + 4 * g + r;
      const bool vis = key < kv_len && (!p.causal || key <= q + off);
      sc[r] = vis ? st[r] * c : -INFINITY;
    }
    float mx = fmaxf(fmaxf(sc[0], sc[1]), fmaxf(sc[2], sc[3]));
    mx = fmaxf(mx, __shfl_xor(mx, 16));
    mx = fmaxf(mx, __shfl_xor(mx, 32));
    const float m_new = fmaxf(m_run, mx);
    const float m_use = m_new == -INFINITY ? 0.f : m_new;
    const float alpha = exp2_fast(m_run - m_use);
    f32x4 pr;
#pragma unroll
    for (int r = 0; r < 4; ++r) pr[r] = exp2_fast(sc[r] - m_use);
    // The PV product takes P rounded to the input type (kernels/fa2.py:147); the row sum adds the
    // same rounded values, so that the weights applied to V sum to exactly 1 after the division.
    // (The reference sums P before rounding, kernels/fa2.py:145: in bf16 that leaves the weights
    // off by up to 2^-9 relative, which on outputs near 4 adds up to 8e-3 to the output's own
    // rounding.)  fp32: no rounding, the two are the same.
    const Quad pq = G::pack(pr);
    l_run = l_run * alpha + G::sum(pq);
    m_run = m_new;

    // V^T as the A operand: lane (n, g) = d 16*i + n, keys kc + 4*g + j (j = element).  Keys past
    // kv_len read as 0 (their address clamped to the row's last key, kv_len > 0 here).
#pragma unroll
    for (int i = 0; i < kVB; ++i) {
      Quad va;
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        const int key = kc + 4 * g + j;
        const T* vr = vp + (int64_t)min(key, kv_len - 1) * p.v_st + 16 * i + n;
        va[j] = key < kv_len ? G::load1(vr) : 0;
      }
      oacc[i] = G::mma(va, pq, oacc[i] * alpha);
    }
  }

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
}

}  // namespace mi_fa2

namespace mi_fa2 {

namespace {

template <class E, int D, int DV>
hipError_t launch_general_t(const FwdParams& p, hipStream_t stream) {
  const int rows_per_wg = kGenWaves * kGenRows;
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
