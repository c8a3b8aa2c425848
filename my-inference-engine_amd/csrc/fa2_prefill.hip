// Prefill FlashAttention-2 forward for gfx950: bf16/fp16 MFMA, K/V tiles staged in LDS.
//
// Replaces the Triton kernel fa2_forward in its prefill regime (kernels/fa2.py:14-162, launched
// with Br=32, Bc=64 at kernels/fa2.py:10): for one (query tile, query head, batch row) it streams the
// row's keys in tiles, applies the per-row key count and the bottom-right causal mask, and keeps an
// online softmax (kernels/fa2.py:122-158).  Same mathematics, different organisation:
//
//   * One work-group = 4 waves = 128 query rows of one query head; each wave owns 32 rows.
//   * Scores are computed transposed, S^T = K Q^T, with v_mfma_f32_32x32x16: the accumulator then
//     holds one query per lane (lane%32) and 16 keys per lane in registers.  That is exactly the
//     B-operand layout of O^T += V^T P^T, so P never leaves registers, and the running max / sum and
//     the O rescale are per-lane (one cross-lane exchange with lane^32 per tile for the max).
//   * Q (the B operand of S^T) lives in registers for the whole key loop.
//   * A 64-key K tile is kept row-major in LDS (A operand: 16 contiguous bytes per lane); the V tile
//     is transposed on its way into LDS (V^T rows of 64 keys), so the V^T A operand is two 8-byte
//     LDS reads.  Row pitches are padded to keep both LDS read patterns bank-conflict free.
//   * The next tile's global loads are issued before the current tile is computed (register
//     prefetch), so HBM/L2 latency hides behind the MFMA work.
//   * Scores are scaled into the exp2 domain once (scale*log2 e folded into one FMA), masking runs
//     only on tiles that straddle the causal diagonal or the end of the row, and tiles past the
//     diagonal are never loaded.
//   * Grid (heads, tiles, batch) with tiles launched longest-first, so causal work drains evenly.
#include "fa2_common.h"

namespace mi_fa2 {

constexpr int kPfWaves = 4;
constexpr int kPfRows = 32 * kPfWaves;  // query rows per work-group
constexpr int kPfBc = 64;               // keys per K/V tile
constexpr int kKPitch = kHeadDim + 8;   // LDS row pitch of the K tile, elements (272 B)
constexpr int kVPitch = kPfBc + 4;      // LDS row pitch of the transposed V tile, elements (136 B)

template <int MODE>
__device__ __forceinline__ const uint16_t* kv_row(const FwdParams& p, const uint16_t* base,
                                                  int64_t off, int64_t st, int b, int t) {
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

template <typename E, int MODE>
__global__ __launch_bounds__(256, 2) void fa2_prefill_kernel(const FwdParams p) {
  __shared__ __attribute__((aligned(16))) uint16_t k_lds[kPfBc * kKPitch];
  __shared__ __attribute__((aligned(16))) uint16_t v_lds[kHeadDim * kVPitch];

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int h = blockIdx.x;
  const int b = blockIdx.z;
  const int hk = h / p.group;

  int T_b, kv_len;
  int64_t q_off, o_off, l_off, k_off, v_off;
  if constexpr (MODE == kVarlen) {
    const int qs = p.cu_q[b], ks = p.cu_k[b];
    T_b = p.cu_q[b + 1] - qs;
    kv_len = p.cu_k[b + 1] - ks;
    if (kv_len < 0) kv_len = 0;
    q_off = (int64_t)qs * p.q_st + (int64_t)h * p.q_sh;
    o_off = (int64_t)qs * p.o_st + (int64_t)h * p.o_sh;
    l_off = (int64_t)qs * p.l_st + (int64_t)h * p.l_sh;
    k_off = (int64_t)ks * p.k_st + (int64_t)hk * p.k_sh;
    v_off = (int64_t)ks * p.v_st + (int64_t)hk * p.v_sh;
  } else {
    T_b = p.T;
    kv_len = p.kv_lens ? clamp_len(p.kv_lens[b], p.S) : p.S;
    q_off = (int64_t)b * p.q_sb + (int64_t)h * p.q_sh;
    o_off = (int64_t)b * p.o_sb + (int64_t)h * p.o_sh;
    l_off = (int64_t)b * p.l_sb + (int64_t)h * p.l_sh;
    k_off = (MODE == kDense ? (int64_t)b * p.k_sb : 0) + (int64_t)hk * p.k_sh;
    v_off = (MODE == kDense ? (int64_t)b * p.v_sb : 0) + (int64_t)hk * p.v_sh;
  }

  // Longest tiles first: blockIdx.y = 0 is the last query tile of the row.
  const int n_qt = (T_b + kPfRows - 1) / kPfRows;
  const int tile = n_qt - 1 - (int)blockIdx.y;
  if (tile < 0) return;
  const int q0 = tile * kPfRows;
  const int off = kv_len - T_b;  // query i sits at key position i + off

  // Keys the work-group needs: up to what its last valid query row sees.
  int kv_hi = kv_len;
  if (p.causal) kv_hi = min(kv_len, min(q0 + kPfRows, T_b) + off);
  const int n_kv = kv_hi > 0 ? (kv_hi + kPfBc - 1) / kPfBc : 0;

  // This wave's rows and the key ranges they need.
  const int wq0 = q0 + wave * 32;
  const bool wave_active = wq0 < T_b;
  const int wq_last = min(wq0 + 31, T_b - 1);
  const int wave_hi = p.causal ? min(kv_len, wq_last + off + 1) : kv_len;   // seen by some row
  const int wave_full = p.causal ? min(kv_len, wq0 + off + 1) : kv_len;     // seen by every row

  const int r32 = lane & 31;
  const int g = lane >> 5;
  const int qrow = wq0 + r32;

  // Q^T as the B operand: k-step s covers d = s*16 + g*8 + [0, 8).
  u32x4 qb[8];
  if (qrow < T_b) {
    const uint16_t* qp = p.q + q_off + (int64_t)qrow * p.q_st + g * 8;
#pragma unroll
    for (int s = 0; s < 8; ++s) qb[s] = ld16(qp + s * 16);
  } else {
#pragma unroll
    for (int s = 0; s < 8; ++s) qb[s] = u32x4{0, 0, 0, 0};
  }

  f32x16 oacc[4];
#pragma unroll
  for (int i = 0; i < 4; ++i) oacc[i] = f32x16{};
  float m_run = -INFINITY;
  float l_run = 0.f;
  const float c = p.scale_log2;
  const int lim = p.causal ? min(kv_len, qrow + off + 1) : kv_len;  // keys < lim are visible

  // Staging: thread tid moves K rows st_row + 16u and V rows 4*st_row + r, 16-byte chunk st_dc.
  const int st_dc = tid & 15;
  const int st_row = tid >> 4;
  u32x4 kreg[4], vreg[4];

  auto load_tile = [&](int j) {
    const int kt = j * kPfBc;
#pragma unroll
    for (int u = 0; u < 4; ++u) {
      const int t = kt + st_row + 16 * u;
      const uint16_t* ptr = t < kv_len ? kv_row<MODE>(p, p.k, k_off, p.k_st, b, t) : nullptr;
      kreg[u] = ptr ? ld16(ptr + st_dc * 8) : u32x4{0, 0, 0, 0};
    }
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      const int t = kt + st_row * 4 + r;
      const uint16_t* ptr = t < kv_len ? kv_row<MODE>(p, p.v, v_off, p.v_st, b, t) : nullptr;
      vreg[r] = ptr ? ld16(ptr + st_dc * 8) : u32x4{0, 0, 0, 0};
    }
  };

  auto store_tile = [&]() {
#pragma unroll
    for (int u = 0; u < 4; ++u)
      *reinterpret_cast<u32x4*>(k_lds + (st_row + 16 * u) * kKPitch + st_dc * 8) = kreg[u];
    // 4 keys x 8 dims -> 8 dims x 4 keys (V^T rows hold consecutive keys).
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      const uint32_t a0 = vreg[0][e], a1 = vreg[1][e], a2 = vreg[2][e], a3 = vreg[3][e];
      const u32x2 lo = {(a0 & 0xffffu) | (a1 << 16), (a2 & 0xffffu) | (a3 << 16)};
      const u32x2 hi = {(a0 >> 16) | (a1 & 0xffff0000u), (a2 >> 16) | (a3 & 0xffff0000u)};
      *reinterpret_cast<u32x2*>(v_lds + (st_dc * 8 + 2 * e) * kVPitch + st_row * 4) = lo;
      *reinterpret_cast<u32x2*>(v_lds + (st_dc * 8 + 2 * e + 1) * kVPitch + st_row * 4) = hi;
    }
  };

  if (n_kv > 0) load_tile(0);

  for (int j = 0; j < n_kv; ++j) {
    __syncthreads();  // every wave is done reading tile j-1
    store_tile();
    __syncthreads();  // tile j is in LDS
    if (j + 1 < n_kv) load_tile(j + 1);

    const int kt = j * kPfBc;
    if (!wave_active || kt >= wave_hi) continue;

    // S^T[key][query] for keys kt + [0,32) (s0) and kt + [32,64) (s1).
    f32x16 s0 = f32x16{}, s1 = f32x16{};
    const uint16_t* kp = k_lds + r32 * kKPitch + g * 8;
#pragma unroll
    for (int s = 0; s < 8; ++s) {
      const u32x4 a0 = *reinterpret_cast<const u32x4*>(kp + s * 16);
      const u32x4 a1 = *reinterpret_cast<const u32x4*>(kp + 32 * kKPitch + s * 16);
      s0 = E::mfma32(a0, qb[s], s0);
      s1 = E::mfma32(a1, qb[s], s1);
    }

    // Accumulator r of this lane is key kt + 8*(r/4) + 4*g + r%4 (+32 for s1).
    if (kt + kPfBc > wave_full) {
#pragma unroll
      for (int r = 0; r < 16; ++r) {
        const int key = kt + 8 * (r >> 2) + 4 * g + (r & 3);
        if (key >= lim) s0[r] = -INFINITY;
        if (key + 32 >= lim) s1[r] = -INFINITY;
      }
    }

    float mx = fmaxf(s0[0], s1[0]);
#pragma unroll
    for (int r = 1; r < 16; ++r) mx = fmax3(mx, s0[r], s1[r]);
    mx = fmaxf(mx, __shfl_xor(mx, 32));
    const float m_new = fmaxf(m_run, mx * c);
    const float m_use = m_new == -INFINITY ? 0.f : m_new;
    const float alpha = exp2_fast(m_run - m_use);
    float ls = 0.f;
#pragma unroll
    for (int r = 0; r < 16; ++r) {
      s0[r] = exp2_fast(__builtin_fmaf(s0[r], c, -m_use));
      s1[r] = exp2_fast(__builtin_fmaf(s1[r], c, -m_use));
      ls += s0[r] + s1[r];
    }
    l_run = l_run * alpha + ls;
    m_run = m_new;
#pragma unroll
    for (int i = 0; i < 4; ++i) oacc[i] *= alpha;

    // P^T as the B operand: k-step ks covers keys kt + 16*ks + 8*(t/4) + 4*g + t%4, slot t.
    u32x4 pb[4];
#pragma unroll
    for (int w = 0; w < 4; ++w) {
      pb[0][w] = E::pack2(s0[2 * w], s0[2 * w + 1]);
      pb[1][w] = E::pack2(s0[8 + 2 * w], s0[8 + 2 * w + 1]);
      pb[2][w] = E::pack2(s1[2 * w], s1[2 * w + 1]);
      pb[3][w] = E::pack2(s1[8 + 2 * w], s1[8 + 2 * w + 1]);
    }

    // O^T[d][query] += V^T[d][key] P^T[key][query], d-block db covers d = 32*db + lane%32.
#pragma unroll
    for (int db = 0; db < 4; ++db) {
      const uint16_t* vp = v_lds + (db * 32 + r32) * kVPitch + g * 4;
#pragma unroll
      for (int ks = 0; ks < 4; ++ks) {
        const u32x2 lo = *reinterpret_cast<const u32x2*>(vp + ks * 16);
        const u32x2 hi = *reinterpret_cast<const u32x2*>(vp + ks * 16 + 8);
        const u32x4 a = {lo[0], lo[1], hi[0], hi[1]};
        oacc[db] = E::mfma32(a, pb[ks], oacc[db]);
      }
    }
  }

  if (qrow >= T_b) return;
  const float l_tot = l_run + __shfl_xor(l_run, 32);
  const float inv = l_tot > 0.f ? 1.f / l_tot : 0.f;
  // Accumulator r of d-block db is d = 32*db + 8*(r/4) + 4*g + r%4: four consecutive d per group.
  uint16_t* op = p.o + o_off + (int64_t)qrow * p.o_st + g * 4;
#pragma unroll
  for (int db = 0; db < 4; ++db) {
#pragma unroll
    for (int rg = 0; rg < 4; ++rg) {
      const u32x2 val = {E::pack2(oacc[db][rg * 4] * inv, oacc[db][rg * 4 + 1] * inv),
                         E::pack2(oacc[db][rg * 4 + 2] * inv, oacc[db][rg * 4 + 3] * inv)};
      *reinterpret_cast<u32x2*>(op + db * 32 + rg * 8) = val;
    }
  }
  if (p.lse && g == 0)
    p.lse[l_off + (int64_t)qrow * p.l_st] =
        l_tot > 0.f ? (m_run + __builtin_log2f(l_tot)) * kLn2 : -INFINITY;
}

template <typename E, int MODE>
static hipError_t launch_prefill_t(const FwdParams& p, int max_seqlen_q, hipStream_t stream) {
  const int n_qt = (max_seqlen_q + kPfRows - 1) / kPfRows;
  if (n_qt == 0 || p.B == 0) return hipSuccess;
  dim3 grid(p.Hq, n_qt, p.B);
  hipLaunchKernelGGL((fa2_prefill_kernel<E, MODE>), grid, dim3(256), 0, stream, p);
  return hipGetLastError();
}

hipError_t launch_prefill(const FwdParams& p, int dtype, int mode, int max_seqlen_q,
                          hipStream_t stream) {
  if (dtype == 0) {
    if (mode == kDense) return launch_prefill_t<BF16, kDense>(p, max_seqlen_q, stream);
    if (mode == kVarlen) return launch_prefill_t<BF16, kVarlen>(p, max_seqlen_q, stream);
    return launch_prefill_t<BF16, kPaged>(p, max_seqlen_q, stream);
  }
  if (mode == kDense) return launch_prefill_t<FP16, kDense>(p, max_seqlen_q, stream);
  if (mode == kVarlen) return launch_prefill_t<FP16, kVarlen>(p, max_seqlen_q, stream);
  return launch_prefill_t<FP16, kPaged>(p, max_seqlen_q, stream);
}

}  // namespace mi_fa2
