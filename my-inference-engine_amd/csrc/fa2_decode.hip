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
//   * Dense K/V: the key loop is software-pipelined, the loads of step s+1 in flight while step s
//     is computed (two register buffers, 2 waves per SIMD).  Paged K/V: one buffer and 3 waves per
//     SIMD.  Both: where a work-group's share crosses from one item to the next, the next item's
//     q, first K/V step (and, paged, its first block-table entries) are issued before this item's
//     merge, so the merge runs under their latency (paged, 64 rows of U[128, 8192] keys: 53.1 ->
//     51.3 us per step).
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

// Paged mode: the block-table entries of one wave step (keys kb .. kb+31: two 16-token runs), in
// lanes 0 and 1.  Fetched a step ahead, so a step's K/V loads never wait for a table read.
template <int MODE>
__device__ __forceinline__ int dc_tbl_fetch(const FwdParams& p, int b, int kb, int k_end, int lane) {
  if constexpr (MODE == kPaged) {
    const int t = kb + 16 * lane;
    if (lane < 2 && t < k_end)
      return p.block_table[(int64_t)b * p.bt_stride + (t >> __builtin_ctz(p.block_size))];
    return -1;
  } else {
    return 0;
  }
}

template <int MODE>
__device__ __forceinline__ const uint16_t* dc_run(const FwdParams& p, const uint16_t* base,
                                                  int64_t off, int64_t st, int b, int t, int blk) {
  // Pointer to token t (a multiple of 16) of row b; the next 15 tokens follow at stride st.
  // Paged mode: blk is the table entry of t's block.
  if constexpr (MODE == kPaged) {
    const int bs_shift = __builtin_ctz(p.block_size);
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

// Cache policy of the K/V loads: non-temporal (streamed once; MI_FA2_DC_NT=0 turns it off).
#ifndef MI_FA2_DC_NT
#define MI_FA2_DC_NT 1
#endif
constexpr int kDcLoadPolicy = MI_FA2_DC_NT ? 2 : 0;

// One wave step's operands: K in A layout, V rows for the in-register transpose.
struct DcStep {
  u32x4 ka[2][4];
  u32x4 va[2][4];
};

// A 16-token run is read through a buffer resource that ends at the run's last valid token: rows
// past k_end (and a whole run past it, or a table entry outside the pool) read as zeros with no
// per-lane condition around the loads.
template <int MODE>
__device__ __forceinline__ void dc_load(const FwdParams& p, int b, int64_t k_off, int64_t v_off,
                                        int kb, int k_end, int n, int g, int tbl, DcStep& s) {
#pragma unroll
  for (int hf = 0; hf < 2; ++hf) {
    const int t = kb + 16 * hf;
    const int blk = __builtin_amdgcn_readlane(tbl, hf);
    const int rows = t < k_end ? min(k_end - t, 16) : 0;
    const uint16_t* kr = rows ? dc_run<MODE>(p, p.k, k_off, p.k_st, b, t, blk) : nullptr;
    const uint16_t* vr = rows ? dc_run<MODE>(p, p.v, v_off, p.v_st, b, t, blk) : nullptr;
    const __amdgpu_buffer_rsrc_t rk = make_rsrc(kr ? kr : p.k, kr ? rows * (int)p.k_st * 2 : 0);
    const __amdgpu_buffer_rsrc_t rv = make_rsrc(vr ? vr : p.v, vr ? rows * (int)p.v_st * 2 : 0);
    // K as the A operand: lane row n is token t + n, slots cover d = 32*ks + 8*g + [0, 8).
    const int ko = (n * (int)p.k_st + g * 8) * 2;
#pragma unroll
    for (int ks = 0; ks < 4; ++ks)
      s.ka[hf][ks] = __builtin_amdgcn_raw_buffer_load_b128(rk, ko + ks * 64, 0, kDcLoadPolicy);
    // V rows for the V^T A operand: token t + 4g + r, dims 8n .. 8n+7.
#pragma unroll
    for (int r = 0; r < 4; ++r)
      s.va[hf][r] = __builtin_amdgcn_raw_buffer_load_b128(
          rv, ((4 * g + r) * (int)p.v_st + n * 8) * 2, 0, kDcLoadPolicy);
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

// Work split (stream-K over the keys of every (row, kv head) item).  Each item's keys are cut into
// 128-key chunks (one 32-key step for each of the 4 waves); item i = (b, hk), hk fastest, owns
// chunks [R[b] + hk*n_b, +n_b) of a global chunk sequence of length N, n_b = ceil(kv_len_b / 128)
// (1 for an empty row, so that someone writes its zero output).  Work-group w of the W launched
// takes the contiguous chunks [w*N/W', (w+1)*N/W'), W' = min(W, N): every work-group streams the
// same number of bytes whatever the row lengths, there is no tail of short splits, and a work-group
// that covers a whole item writes the final output.  Items cut by work-group boundaries get one fp32
// partial per work-group touching them (at most n_b), merged by fa2_combine_kernel.  Work-groups
// and the combine find the item boundaries from a prefix sum of the row chunk counts that every
// work-group computes from kv_lens (B loads, one wave).
constexpr int kDcChunk = kDcWaves * kDcStep;  // 128 keys

// First work-group (of W over N chunks) whose range contains chunk c.
__device__ __forceinline__ int dc_first_wg(int64_t c, int64_t N, int W) {
  return (int)(((c + 1) * W - 1) / N);
}

// Chunk counts of rows [0, B) prefix-summed into R[0..B] (LDS), by wave 0; R[B] is the number of
// chunks per kv head summed over rows.  Ends with a barrier.
__device__ __forceinline__ void dc_row_prefix(const FwdParams& p, int* R) {
  if (threadIdx.x < 64) {
    const int lane = threadIdx.x;
    int carry = 0;
    if (lane == 0) R[0] = 0;
    for (int base = 0; base < p.B; base += 64) {
      const int b = base + lane;
      int n = 0;
      if (b < p.B) {
        const int kv = p.kv_lens ? clamp_len(p.kv_lens[b], p.S) : p.S;
        n = kv > 0 ? (kv + kDcChunk - 1) / kDcChunk : 1;
      }
#pragma unroll
      for (int o = 1; o < 64; o <<= 1) {
        const int t = __shfl_up(n, o);
        if (lane >= o) n += t;
      }
      if (b < p.B) R[b + 1] = carry + n;
      carry += __shfl(n, 63);
    }
  }
  __syncthreads();
}

// The work-group's lds: the waves' partial (m, l, O) for the merge, then R[0..B].
static size_t decode_lds_bytes(int group, int batch) {
  return (size_t)kDcWaves * group * (kRedPitch + 2) * sizeof(float) + (size_t)(batch + 1) * 4;
}

// Key walk per mode (measured on the 64-row U[128,8192] decode): with dense K/V, two register
// buffers per wave (the next step's loads in flight during this step's math, 2 waves per SIMD);
// with paged K/V, whose loads first wait for a block-table entry, one buffer and 3 waves per SIMD
// (more independent load chains) are 9% faster, and the dense walk 20% slower that way.
template <int MODE>
struct DcShape {
  static constexpr bool kPipe = MODE != kPaged;
  static constexpr int kOcc = MODE == kPaged ? 3 : 2;  // waves per SIMD
};

// Item (b, hk), chunks [c, c_end) of its n_b, is done by this work-group's 4 waves: their (m, l, O)
// merge through LDS, then the output is written if the work-group covered the whole item, or else an
// fp32 partial for the combine.  Ends with a barrier: red is rewritten by the next item.
template <typename E>
__device__ __forceinline__ void dc_finish(const FwdParams& p, const int* R, float* red_o,
                                          float* red_m, float* red_l, int64_t N, int W, int w,
                                          int b, int hk, int c, int c_end, int n_b, int wave,
                                          int n, int g, int tid, const f32x4 (&oacc)[8],
                                          float m_run, float l_run) {
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

  // Merge the 4 waves for each (column, d); finish the item here if this work-group covers all of
  // it, otherwise leave a partial for the combine.
  const bool whole = c == 0 && c_end == n_b;
  const int64_t item_first = (int64_t)R[b] * p.Hkv + (int64_t)hk * n_b;
  const int f_wg = dc_first_wg(item_first, N, W);
  const int split = w - f_wg;
  // The item's first work-group records how many partials the combine has to merge (1: none).
  if (split == 0 && tid == 0 && p.max_splits > 1)
    p.ws_np[b * p.Hkv + hk] = dc_first_wg(item_first + n_b - 1, N, W) - f_wg + 1;
  for (int idx = tid; idx < p.group * kHeadDim; idx += 256) {
    const int col = idx / kHeadDim;
    const int d = idx % kHeadDim;
    float M = -INFINITY;
#pragma unroll
    for (int j = 0; j < kDcWaves; ++j) M = fmaxf(M, red_m[j * p.group + col]);
    const float M_use = M == -INFINITY ? 0.f : M;
    float acc = 0.f, L = 0.f;
#pragma unroll
    for (int j = 0; j < kDcWaves; ++j) {
      const float f = exp2_fast(red_m[j * p.group + col] - M_use);
      acc += red_o[(j * p.group + col) * kRedPitch + d] * f;
      L += red_l[j * p.group + col] * f;
    }
    const int hq = hk * p.group + col;
    if (whole) {
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
  __syncthreads();
}

template <typename E, int MODE>
__global__ __launch_bounds__(256, DcShape<MODE>::kOcc) void fa2_decode_kernel(const FwdParams p,
                                                                              int n_wg) {
  extern __shared__ float red[];
  float* red_o = red;
  float* red_m = red + kDcWaves * p.group * kRedPitch;
  float* red_l = red_m + kDcWaves * p.group;
  int* R = reinterpret_cast<int*>(red_l + kDcWaves * p.group);
  probe_mark(p.clock_probe, blockIdx.x, false);

  dc_row_prefix(p, R);
  const int64_t N = (int64_t)R[p.B] * p.Hkv;
  const int W = (int)min<int64_t>(n_wg, N);
  const int w = blockIdx.x;
  if (w >= W) return;
  int64_t lo = (int64_t)w * N / W;
  const int64_t hi = (int64_t)(w + 1) * N / W;

  // Item containing chunk lo: binary search for the row, then the kv head.
  int b = 0;
  {
    int l = 0, h = p.B;  // R[l] * Hkv <= lo < R[h] * Hkv
    while (h - l > 1) {
      const int m = (l + h) >> 1;
      if ((int64_t)R[m] * p.Hkv <= lo) l = m; else h = m;
    }
    b = l;
  }
  int n_b = R[b + 1] - R[b];
  int hk = (int)((lo - (int64_t)R[b] * p.Hkv) / n_b);
  int c = (int)(lo - (int64_t)R[b] * p.Hkv - (int64_t)hk * n_b);

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int n = lane & 15;  // MFMA column: query head hk*group + n; also the A-operand row
  const int g = lane >> 4;  // lane group: k-slots 8g..8g+7
  const float cl = p.scale_log2;

  const auto kv_len_of = [&](int bb) { return p.kv_lens ? clamp_len(p.kv_lens[bb], p.S) : p.S; };
  const auto load_q = [&](int bb, int hh, u32x4 (&qb)[4]) {
    if (n < p.group) {
      const uint16_t* qp =
          p.q + (int64_t)bb * p.q_sb + (int64_t)(hh * p.group + n) * p.q_sh + g * 8;
#pragma unroll
      for (int ks = 0; ks < 4; ++ks) qb[ks] = ld16(qp + ks * 32);
    } else {
#pragma unroll
      for (int ks = 0; ks < 4; ++ks) qb[ks] = u32x4{0, 0, 0, 0};
    }
  };
  const auto k_off_of = [&](int bb, int hh) {
    return (MODE == kDense ? (int64_t)bb * p.k_sb : 0) + (int64_t)hh * p.k_sh;
  };
  const auto v_off_of = [&](int bb, int hh) {
    return (MODE == kDense ? (int64_t)bb * p.v_sb : 0) + (int64_t)hh * p.v_sh;
  };
  if constexpr (DcShape<MODE>::kPipe) {
    // Dense walk, two register buffers: step s+1's loads fly during step s's math.  As in the
    // paged walk below, the next item's q and first K/V step are issued before this item's merge.
    int c_end = (int)min<int64_t>(n_b, c + (hi - lo));
    int k_end = min(kv_len_of(b), c_end * kDcChunk);
    int kb = c * kDcChunk + wave * kDcStep;
    u32x4 qb[4];
    load_q(b, hk, qb);
    DcStep s0, s1;
    if (kb < k_end) dc_load<MODE>(p, b, k_off_of(b, hk), v_off_of(b, hk), kb, k_end, n, g, 0, s0);
    while (true) {
      // The item after this one in the share (none: k_end2 = 0, so nothing is fetched for it).
      const int64_t lo2 = lo + (c_end - c);
      const bool more = lo2 < hi;
      int b2 = b, hk2 = hk + 1, n_b2 = n_b;
      if (hk2 == p.Hkv) {
        hk2 = 0;
        ++b2;
        if (more) n_b2 = R[b2 + 1] - R[b2];
      }
      const int c_end2 = more ? (int)min<int64_t>(n_b2, hi - lo2) : 0;
      const int k_end2 = more ? min(kv_len_of(b2), c_end2 * kDcChunk) : 0;
      const int kb2 = wave * kDcStep;
      const int64_t k_off = k_off_of(b, hk);
      const int64_t v_off = v_off_of(b, hk);

      f32x4 oacc[8];
#pragma unroll
      for (int i = 0; i < 8; ++i) oacc[i] = f32x4{};
      float m_run = -INFINITY;
      float l_run = 0.f;
      while (kb < k_end) {
        const int kb1 = kb + kDcChunk;
        if (kb1 < k_end) dc_load<MODE>(p, b, k_off, v_off, kb1, k_end, n, g, 0, s1);
        dc_compute<E>(s0, qb, kb, k_end, g, cl, m_run, l_run, oacc);
        if (kb1 >= k_end) break;
        const int kb3 = kb1 + kDcChunk;
        if (kb3 < k_end) dc_load<MODE>(p, b, k_off, v_off, kb3, k_end, n, g, 0, s0);
        dc_compute<E>(s1, qb, kb1, k_end, g, cl, m_run, l_run, oacc);
        kb = kb3;
      }
      if (more) {
        load_q(b2, hk2, qb);
        if (kb2 < k_end2)
          dc_load<MODE>(p, b2, k_off_of(b2, hk2), v_off_of(b2, hk2), kb2, k_end2, n, g, 0, s0);
      }
      dc_finish<E>(p, R, red_o, red_m, red_l, N, W, w, b, hk, c, c_end, n_b, wave, n, g, tid, oacc,
                   m_run, l_run);
      if (!more) break;
      lo = lo2;
      c = 0;
      b = b2;
      hk = hk2;
      n_b = n_b2;
      c_end = c_end2;
      k_end = k_end2;
      kb = kb2;
    }
  } else {
    // Paged walk, one register buffer.  The next item's q, its first block-table entries and its
    // first K/V step are issued before this item's merge (the table entries during this item's last
    // step), so a share that crosses an item boundary waits out no memory round trip between them.
    int c_end = (int)min<int64_t>(n_b, c + (hi - lo));
    int k_end = min(kv_len_of(b), c_end * kDcChunk);
    int kb = c * kDcChunk + wave * kDcStep;
    u32x4 qb[4];
    load_q(b, hk, qb);
    DcStep s;
    {
      const int t0 = dc_tbl_fetch<MODE>(p, b, kb, k_end, lane);
      if (kb < k_end) dc_load<MODE>(p, b, k_off_of(b, hk), v_off_of(b, hk), kb, k_end, n, g, t0, s);
    }
    while (true) {
      // The item after this one in the share (none: k_end2 = 0, so nothing is fetched for it).
      const int64_t lo2 = lo + (c_end - c);
      const bool more = lo2 < hi;
      int b2 = b, hk2 = hk + 1, n_b2 = n_b;
      if (hk2 == p.Hkv) {
        hk2 = 0;
        ++b2;
        if (more) n_b2 = R[b2 + 1] - R[b2];
      }
      const int c_end2 = more ? (int)min<int64_t>(n_b2, hi - lo2) : 0;
      const int k_end2 = more ? min(kv_len_of(b2), c_end2 * kDcChunk) : 0;
      const int kb2 = wave * kDcStep;
      // Table entries of the step after key kn: this item's while it has keys there, else the
      // next item's first step.
      const auto fetch_after = [&](int kn) {
        return kn < k_end ? dc_tbl_fetch<MODE>(p, b, kn, k_end, lane)
                          : dc_tbl_fetch<MODE>(p, b2, kb2, k_end2, lane);
      };
      const int64_t k_off = k_off_of(b, hk);
      const int64_t v_off = v_off_of(b, hk);

      f32x4 oacc[8];
#pragma unroll
      for (int i = 0; i < 8; ++i) oacc[i] = f32x4{};
      float m_run = -INFINITY;
      float l_run = 0.f;
      int tbl = fetch_after(kb + kDcChunk);
      for (; kb < k_end; kb += kDcChunk) {
        dc_compute<E>(s, qb, kb, k_end, g, cl, m_run, l_run, oacc);
        const int kn = kb + kDcChunk;
        if (kn < k_end) {
          dc_load<MODE>(p, b, k_off, v_off, kn, k_end, n, g, tbl, s);
          tbl = fetch_after(kn + kDcChunk);  // in flight during the math
        }
      }
      if (more) {
        load_q(b2, hk2, qb);
        if (kb2 < k_end2)
          dc_load<MODE>(p, b2, k_off_of(b2, hk2), v_off_of(b2, hk2), kb2, k_end2, n, g, tbl, s);
      }
      dc_finish<E>(p, R, red_o, red_m, red_l, N, W, w, b, hk, c, c_end, n_b, wave, n, g, tid, oacc,
                   m_run, l_run);
      if (!more) break;
      lo = lo2;
      c = 0;
      b = b2;
      hk = hk2;
      n_b = n_b2;
      c_end = c_end2;
      k_end = k_end2;
      kb = kb2;
    }
  }
  probe_mark(p.clock_probe, blockIdx.x, true);
}

// Merges the partials of items that were cut by work-group boundaries (their count is recorded by
// the decode kernel).  Grid (Hq, B), one thread per head dimension; the partials are read 16 at a
// time with every load issued before any is used, and folded in with an online log-sum-exp
// rescale.
template <typename E>
__global__ __launch_bounds__(kHeadDim) void fa2_combine_kernel(const FwdParams p) {
  const int hq = blockIdx.x;
  const int b = blockIdx.y;
  const int n_parts = p.ws_np[b * p.Hkv + hq / p.group];
  if (n_parts <= 1) return;  // the decode kernel wrote this row's output
  const int d = threadIdx.x;
  const int64_t base = ((int64_t)b * p.Hq + hq) * p.max_splits;
  float M = -INFINITY, L = 0.f, acc = 0.f;
  for (int s0 = 0; s0 < n_parts; s0 += 16) {
    float m[16], lv[16], o[16];
#pragma unroll
    for (int i = 0; i < 16; ++i) {
      const int s = s0 + i;
      const bool ok = s < n_parts;
      m[i] = ok ? p.ws_m[base + s] : -INFINITY;
      lv[i] = ok ? p.ws_l[base + s] : 0.f;
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
      const float f2 = exp2_fast(m[i] - Mu);
      L += lv[i] * f2;
      acc += o[i] * f2;
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

template <typename E, int MODE>
static hipError_t launch_decode_t(const FwdParams& p, hipStream_t stream) {
  if (p.B == 0) return hipSuccess;
  const int n_wg = p.n_wg;
  hipLaunchKernelGGL((fa2_decode_kernel<E, MODE>), dim3(n_wg), dim3(256),
                     decode_lds_bytes(p.group, p.B), stream, p, n_wg);
  hipError_t err = hipGetLastError();
  if (err != hipSuccess || p.max_splits <= 1) return err;
  hipLaunchKernelGGL((fa2_combine_kernel<E>), dim3(p.Hq, p.B), dim3(kHeadDim), 0, stream, p);
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
