// Prefill FlashAttention-2 forward for gfx950: bf16/fp16 MFMA, K/V tiles staged in LDS.
//
// Replaces the Triton kernel fa2_forward in its prefill regime (kernels/fa2.py:14-162, launched
// with Br=32, Bc=64 at kernels/fa2.py:10): for one (query tile, query head, batch row) it streams the
// row's keys in tiles, applies the per-row key count and the bottom-right causal mask, and keeps an
// online softmax (kernels/fa2.py:122-158).  Same mathematics, different organisation:
//
//   * One work-group = 8 waves = 128 query rows of one query head.  Wave w owns rows 32*(w%4) ..
//     +31 and key stream w/4: stream 0 takes the even 64-key tiles, stream 1 the odd ones, so two
//     waves share every SIMD (one's softmax hides behind the other's MFMAs) and the longest causal
//     tile is walked by two waves in parallel.  The two streams' (m, l, O) are merged in LDS at the
//     end.  Launches with at least two work-groups per CU use a one-stream shape instead: 4 waves
//     on the same 128 rows walk every tile in turn with half the LDS (64 KB), so two work-groups
//     share a CU, the SIMD's two waves come from different tiles, and one work-group's start
//     (item, Q, first stages) and end (stores) run under the other's key loop.
//   * Scores are computed transposed, S^T = K Q^T, with v_mfma_f32_32x32x16: the accumulator holds
//     one query per lane (lane%32) and 16 keys per lane in registers.  That is exactly the B-operand
//     layout of O^T += V^T P^T, so P never leaves registers and the running max / sum and the O
//     rescale are per lane (one exchange with lane^32 per tile for the max).
//   * Q lives in registers (the B operand of S^T) for the whole key loop.  Scores stay in the
//     exp2 domain: p = exp2(s * sm_scale*log2(e) - m) is one FMA and one v_exp per score.  (Folding
//     the scale into Q would save the FMA but rounds sm_scale*log2(e)*q to 16 bits, which measured
//     past the 1e-2 output tolerance on short rows.)  The row sum is taken on the packed 16-bit P
//     with v_dot2 (two scores per instruction).
//   * The running max is only moved when a row's new max exceeds it by more than 2^8
//     (kRescaleSlack); until then exp2(s - m) <= 2^8 is exact enough in fp32/bf16 and the O rescale
//     is skipped wave-wide.
//   * K and V tiles go from memory straight into LDS (buffer_load ... lds: no registers, no LDS
//     write instructions), row-major, 256 bytes per key, with the 16-byte chunks of each row
//     XOR-swizzled (K: chunk ^ row%16, V: chunk ^ 4*(row%4)).  The K A operand is one 16-byte read
//     per lane; the V^T A operand is two ds_read_b64_tr_b16 transposing reads.  MFMA row m of S^T
//     is loaded from key pi(m) (a fixed permutation of the 32 keys of a block) so that the 8 keys
//     each lane holds per 16-key k-step are consecutive, which is what the transposing reads
//     deliver.  The swizzles make every LDS read of the loop bank-conflict free.
//   * Each load instruction moves 4 key rows (1 KB) through a buffer resource that starts at the
//     first of them and ends at the last key the work-group needs: keys past it read as zeros,
//     with no per-lane predicate.  In paged mode a wave's two instructions of a tile (8 rows)
//     share one block; the block-table entries of 16 steps are fetched with one vector load and
//     turned into load addresses in one vector pass, each instruction reading its own back.
//   * LDS holds two stages of (K, V) for every stream; the next step's keys (128, or 64 with one
//     stream) are loaded while the current ones are computed, one barrier per step.
//   * Masking runs only on tiles that straddle the causal diagonal or the end of the row, and tiles
//     past the diagonal are never loaded.  The grid is 1-D, mapped XCD-aware: query heads sharing a
//     kv head run on the same XCDs (one L2 holds their K/V) and every XCD takes its tiles longest
//     first, so causal work drains evenly.
#include "fa2_common.h"

#include <cstdlib>

namespace mi_fa2 {

constexpr int kPfRowGroups = 4;                  // 32-row query groups per work-group
constexpr int kPfRows = 32 * kPfRowGroups;       // query rows per work-group
constexpr int kPfBc = 64;                        // keys per tile (one stream's share of a step)
constexpr int kTileBytes = kPfBc * kHeadDim * 2;       // one 64-key K or V tile in LDS (16 KB)

// The work-group shape for NS key streams (2: the layout described above, 8 waves and 128 KB of
// LDS, one work-group per CU; 1: 4 waves walking every tile in turn with 64 KB of LDS, so that two
// work-groups share a CU and each one's start and end run under the other's key loop).
template <int NS>
struct PfShape {
  static constexpr int kWaves = kPfRowGroups * NS;
  static constexpr int kThreads = 64 * kWaves;
  static constexpr int kStep = kPfBc * NS;              // keys per step
  static constexpr int kStage = NS * kTileBytes;        // K (or V) tiles of one stage
  static constexpr int kVRegion = 2 * kStage;           // V tiles start after both stages' K tiles
  static constexpr int kLds = 2 * kVRegion;             // 128 KB (NS = 2) or 64 KB (NS = 1)
  static constexpr int kLoadsPerWave = 16 / kWaves;     // load instructions per wave and tile
};
constexpr float kRescaleSlack = 8.f;             // log2 units the running max may lag the true max
constexpr float kSumLimit = 256.f;               // 2^kRescaleSlack

template <int P>
struct Parity {
  static constexpr int value = P;
};

// Work-groups are dispatched round-robin over the device's X XCDs (work-group w runs on XCD w % X),
// and each XCD has its own L2.  X is read from the device (8 on a whole MI355X, fewer on a
// partitioned one; a power of two, passed as log2; with X = 1 every mapping below reduces to plain
// rank-major order).  The (row, query head, query tile) of work-group w is chosen so that the
// query heads sharing one kv head (one class c = (row, kv head)) and tile run on the same XCD, so
// one L2 holds their K/V, and so that every XCD walks its tiles longest first with the same mix
// of tile lengths.  rank 0 is a row's last (longest) query tile.
//   * classes dividing X (one or a few long rows): each class has X / classes XCDs of its own, and
//     every XCD walks its class's tiles rank by rank;
//   * otherwise (batches of rows, of equal or ragged lengths): the groups (class, rank) are taken
//     rank-major, group j = rank * stride + c with an odd stride >= classes, and dealt to XCD
//     j % X.  The odd stride rotates a class over the XCDs from one rank to the next, so rows of
//     different lengths spread over all XCDs instead of pinning a class -- and its row's whole
//     work -- to XCD c % X (16 ragged rows of U[16, 1024] tokens on 8 XCDs: the busiest XCD
//     carried 1.9x the least busy one's tiles that way).
//   * packed batches of at most 64 rows (the varlen modes) number only the real (class, rank)
//     groups, rank-major, and deal group j to XCD j % X (prefill_item_packed): a row's class moves
//     over the XCDs as shorter rows drop out of the later ranks.
inline int prefill_grid_size(int classes, int group, int n_qt, int xcd_log2) {
  const int X = 1 << xcd_log2;
  if (classes < X && X % classes == 0) {
    const int per_xcd = (classes * group * n_qt + X - 1) / X;
    return X * per_xcd;
  }
  const int stride = classes | 1;
  return X * ((stride * n_qt + X - 1) / X) * group;
}

// Division by a divisor fixed for the launch, as a multiply: n / d = umulhi(n, m) >> l with
// l = floor(log2 d) and m = floor(2^(32+l) / d) + 1, exact for n < 2^31 (the error term n*(m*d -
// 2^(32+l)) / (d*2^(32+l)) < n / 2^(32+l) stays below 1/d); m = 0 marks a power of two (n >> l).
// The work-group's item is found at its start, before any load can be issued, and the runtime
// integer divisions this replaces cost a few hundred dependent instructions (1-3% on grids of many
// short tiles).
struct FastDiv {
  uint32_t m, l, d;
};
inline FastDiv make_fastdiv(uint32_t d) {
  FastDiv f{0, 0, d};
  while ((2u << f.l) <= d && f.l < 31) ++f.l;
  if ((d & (d - 1)) != 0) f.m = (uint32_t)(((uint64_t)1 << (32 + f.l)) / d + 1);
  return f;
}
__device__ __forceinline__ int fdiv(int n, const FastDiv& f) {
  return (int)(f.m ? __umulhi((uint32_t)n, f.m) >> f.l : (uint32_t)n >> f.l);
}

// The launch's item map: the divisors of prefill_item, log2 of the device's XCD count and, when
// the classes divide the XCDs, log2 of the XCDs per class (else -1).
struct ItemMap {
  FastDiv group, stride, hkv;
  int32_t classes, xcd_shift, xcd_log2;
};
inline ItemMap make_item_map(int classes, int group, int Hkv, int xcd_log2) {
  ItemMap m{make_fastdiv(group), make_fastdiv(classes | 1), make_fastdiv(Hkv), classes, -1,
            xcd_log2};
  const int X = 1 << xcd_log2;
  if (classes < X && X % classes == 0) {
    m.xcd_shift = 0;
    while ((classes << m.xcd_shift) < X) ++m.xcd_shift;
  }
  return m;
}

// Returns false for the padding work-groups of the grid.
__device__ inline bool prefill_item(int w, const ItemMap& map, int n_qt, int& b, int& h,
                                    int& rank) {
  const int x = w & ((1 << map.xcd_log2) - 1), slot = w >> map.xcd_log2;
  const int group = (int)map.group.d;
  int c;
  if (map.xcd_shift >= 0) {
    const int X = 1 << map.xcd_shift;  // XCDs per class
    c = x >> map.xcd_shift;
    const int u = slot * X + (x & (X - 1));
    rank = fdiv(u, map.group);
    h = (c - fdiv(c, map.hkv) * (int)map.hkv.d) * group + (u - rank * group);
  } else {
    const int stride = (int)map.stride.d;
    const int sg = fdiv(slot, map.group);
    const int j = (sg << map.xcd_log2) + x;  // group, rank-major
    rank = fdiv(j, map.stride);
    c = j - rank * stride;
    if (c >= map.classes) return false;
    h = (c - fdiv(c, map.hkv) * (int)map.hkv.d) * group + (slot - sg * group);
  }
  if (rank >= n_qt) return false;
  b = fdiv(c, map.hkv);
  return true;
}

// Packed batches of at most 64 rows (the varlen modes).  The grid is sized for every row having the
// longest row's tile count; prefill_item leaves the ranks past a short row's last tile as padding
// work-groups between the real ones, and each held a CU for about a microsecond (840 of the 1,584
// work-groups of 16 rows of U[16, 1024] tokens).  Here the groups (rank, class) are numbered over
// the real tiles only, rank-major and in row order within a rank, so all padding falls at the end
// of the grid, where it delays nothing.  Every wave finds its item from the rows' query counts (one
// load per lane, a ballot per rank), so no barrier is needed.
__device__ inline bool prefill_item_packed(const FwdParams& p, int w, const ItemMap& map,
                                           int n_qt, int& b, int& h, int& rank) {
  const int lane = threadIdx.x & 63;
  int nq = 0;
  if (lane < p.B) {
    const int t = p.cu_q[lane + 1] - p.cu_q[lane];
    nq = t > 0 ? (t + kPfRows - 1) / kPfRows : 0;
  }
  const int x = w & ((1 << map.xcd_log2) - 1), slot = w >> map.xcd_log2;
  const int sg = fdiv(slot, map.group);
  const int hkv = (int)map.hkv.d;
  int j = (sg << map.xcd_log2) + x;  // the j-th real group (rank, class), rank-major
  int r = 0;
  uint64_t rows = 0;
  for (; r < n_qt; ++r) {
    rows = __ballot(nq > r);
    const int cnt = __builtin_amdgcn_readfirstlane(__popcll(rows) * hkv);
    if (j < cnt) break;
    j -= cnt;
  }
  // Row b is the ri-th row (lowest first) that has a tile of rank r.
  const int ri = fdiv(j, map.hkv);
  const int below = __builtin_amdgcn_mbcnt_hi((uint32_t)(rows >> 32),
                                               __builtin_amdgcn_mbcnt_lo((uint32_t)rows, 0));
  b = __builtin_amdgcn_readfirstlane(
      __builtin_ctzll(__ballot(nq > r && below == ri) | (1ull << 63)));
  h = (j - ri * hkv) * (int)map.group.d + (slot - sg * (int)map.group.d);
  rank = r;
  return r < n_qt;
}

template <typename E, int MODE, int NS>
__global__ __launch_bounds__(PfShape<NS>::kThreads, 2) void fa2_prefill_kernel(const FwdParams p,
                                                                               int n_qt_max,
                                                                               const ItemMap map) {
  using Sh = PfShape<NS>;
  constexpr int kPfStep = Sh::kStep, kStageBytes = Sh::kStage, kVRegion = Sh::kVRegion;
  constexpr int kPfWaves = Sh::kWaves, kLpw = Sh::kLoadsPerWave;
  __shared__ __attribute__((aligned(1024))) uint8_t smem[Sh::kLds];
  probe_mark(p.clock_probe, blockIdx.x, false);

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int rg = wave % kPfRowGroups;
  const int ks = NS == 2 ? wave / kPfRowGroups : 0;  // key stream
  int b, h, rank;
  bool real;
  if constexpr (MODE == kVarlen || MODE == kPagedVarlen)
    real = p.B <= 64 ? prefill_item_packed(p, blockIdx.x, map, n_qt_max, b, h, rank)
                     : prefill_item(blockIdx.x, map, n_qt_max, b, h, rank);
  else
    real = prefill_item(blockIdx.x, map, n_qt_max, b, h, rank);
  if (!real) return;
  // Work-group constants are made visibly uniform, so that everything derived from them (the load
  // addresses and sizes issued between the MFMAs) is scalar arithmetic, not VALU work that
  // competes with the other wave's softmax.
  b = __builtin_amdgcn_readfirstlane(b);
  h = __builtin_amdgcn_readfirstlane(h);
  rank = __builtin_amdgcn_readfirstlane(rank);
  const int hk = __builtin_amdgcn_readfirstlane(fdiv(h, map.group));

  int T_b, kv_len;
  int64_t q_off, o_off, l_off, k_off, v_off;
  if constexpr (MODE == kVarlen) {
    const int qs = p.cu_q[b], kst = p.cu_k[b];
    T_b = p.cu_q[b + 1] - qs;
    kv_len = p.cu_k[b + 1] - kst;
    if (kv_len < 0) kv_len = 0;
    q_off = (int64_t)qs * p.q_st + (int64_t)h * p.q_sh;
    o_off = (int64_t)qs * p.o_st + (int64_t)h * p.o_sh;
    l_off = (int64_t)qs * p.l_st + (int64_t)h * p.l_sh;
    k_off = (int64_t)kst * p.k_st + (int64_t)hk * p.k_sh;
    v_off = (int64_t)kst * p.v_st + (int64_t)hk * p.v_sh;
  } else if constexpr (MODE == kPagedVarlen) {
    const int qs = p.cu_q[b];
    T_b = p.cu_q[b + 1] - qs;
    if (T_b < 0) T_b = 0;
    kv_len = clamp_len(p.kv_lens[b], p.S);
    q_off = (int64_t)qs * p.q_st + (int64_t)h * p.q_sh;
    o_off = (int64_t)qs * p.o_st + (int64_t)h * p.o_sh;
    l_off = (int64_t)qs * p.l_st + (int64_t)h * p.l_sh;
    k_off = (int64_t)hk * p.k_sh;
    v_off = (int64_t)hk * p.v_sh;
  } else {
    T_b = p.T;
    kv_len = p.kv_lens ? clamp_len(p.kv_lens[b], p.S) : p.S;
    q_off = (int64_t)b * p.q_sb + (int64_t)h * p.q_sh;
    o_off = (int64_t)b * p.o_sb + (int64_t)h * p.o_sh;
    l_off = (int64_t)b * p.l_sb + (int64_t)h * p.l_sh;
    k_off = (MODE == kDense ? (int64_t)b * p.k_sb : 0) + (int64_t)hk * p.k_sh;
    v_off = (MODE == kDense ? (int64_t)b * p.v_sb : 0) + (int64_t)hk * p.v_sh;
  }

  T_b = __builtin_amdgcn_readfirstlane(T_b);
  kv_len = __builtin_amdgcn_readfirstlane(kv_len);
  k_off = (int64_t)uniform_u64((uint64_t)k_off);
  v_off = (int64_t)uniform_u64((uint64_t)v_off);
  const int n_qt = (T_b + kPfRows - 1) / kPfRows;
  const int tile = n_qt - 1 - rank;
  if (tile < 0) return;
  const int q0 = tile * kPfRows;
  const int off = kv_len - T_b;  // query i sits at key position i + off

  // Keys the work-group needs: up to what its last valid query row sees.
  int kv_hi = kv_len;
  if (p.causal) kv_hi = min(kv_len, min(q0 + kPfRows, T_b) + off);
  if (kv_hi < 0) kv_hi = 0;
  kv_hi = __builtin_amdgcn_readfirstlane(kv_hi);  // uniform: keeps the load arithmetic scalar
  const int n_steps = (kv_hi + kPfStep - 1) / kPfStep;

  // This wave's rows and the key ranges they need.
  const int wq0 = q0 + rg * 32;
  const bool wave_active = wq0 < T_b;
  const int wq_last = min(wq0 + 31, T_b - 1);
  const int wave_hi = p.causal ? min(kv_len, wq_last + off + 1) : kv_len;   // seen by some row
  const int wave_full = p.causal ? min(kv_len, wq0 + off + 1) : kv_len;     // seen by every row

  const int r32 = lane & 31;
  const int g = lane >> 5;
  const int qrow = wq0 + r32;
  const float c = p.scale_log2;

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
  float m_run = -INFINITY;  // running max of c*score (log2 units); -inf until a key is seen
  float l_run = 0.f;        // this lane's partial sum of exp2(c*score - m_run)
  const int lim = p.causal ? min(kv_len, qrow + off + 1) : kv_len;  // keys < lim are visible

  // Software pipeline.  Tile (j, s) is keys 128j + 64s .. +63.  Stream 0 (waves 0-3) works one
  // tile ahead of stream 1 (waves 4-7) in the score phase, so that in every step one wave of each
  // SIMD runs its softmax while the other runs MFMAs:
  //   stream 0, step j: softmax(j, 0) ; PV(j, 0) ; S(j+1, 0)      (VALU, then 32 MFMAs)
  //   stream 1, step j: S(j, 1) ; PV(j-1, 1) ; softmax(j, 1)      (32 MFMAs, then VALU)
  //   (paged modes: stream 1 runs PV(j-1, 1) before S(j, 1))
  // Stage j (LDS slot j%2) therefore holds V(j,0), K(j+1,0), V(j-1,1) and K(j,1); it is loaded
  // during step j-1, one barrier per step.  With one stream, tile j is keys 64j .. +63, every
  // wave runs stream 0's program and stage j holds V(j) and K(j+1).
  //
  // Staging.  Every tile is 16 load instructions of 4 rows; instruction i moves rows 4i .. 4i+3,
  // lane l row 4i + l/16 into LDS chunk l%16, i.e. global chunk (l%16) ^ swizzle(row).  Each of
  // the W waves (8, or 4 with one stream) issues L = 16 / W of them per tile:
  //   * dense and packed modes: wave w issues instructions w + W*h, h < L; those rows agree
  //     mod 16, so one offset (relative to the tile's first row, instruction h adding 4W rows)
  //     serves all of them;
  //   * paged modes: wave w issues instructions L*w + h, rows 4Lw .. 4Lw + 4L - 1 of the tile
  //     (8 or 16 rows), which lie in one block (blocks are multiples of 16 rows): one table entry
  //     and one address serve all of them, and the offsets are relative to row 4Lw (instruction h
  //     adding 4 rows).
  const int lrow = lane >> 4;
  int k_voff[kLpw], v_voff[kLpw];
#pragma unroll
  for (int h = 0; h < kLpw; ++h) {
    const int row = is_paged(MODE) ? 4 * kLpw * wave + 4 * h + lrow : 4 * wave + lrow;  // swizzle row
    const int trow = is_paged(MODE) ? 4 * h + lrow : 4 * wave + lrow;
    k_voff[h] = (int)(trow * p.k_st * 2) + 16 * ((lane & 15) ^ (row & 15));
    v_voff[h] = (int)(trow * p.v_st * 2) + 16 * ((lane & 15) ^ (4 * lrow));
  }

  // Load instruction h (0, 1) of this wave for the 64-key tile starting at key ts, whose LDS copy
  // is bytes [lds_off, +16 KB); rows past kv_hi read as zeros.  The scalar work per instruction is
  // kept small (it competes with the MFMA and softmax instruction streams of the CU's waves), and
  // no instruction branches: a tile outside [0, kv_hi) gets a zero-length resource, whose loads
  // write zeros that no active wave reads.  Dense and packed modes use one resource per tile and a
  // per-lane offset per instruction; paged modes one resource per 8-row pair (its rows share a
  // block, the tile's 64 rows need not), whose address and length come precomputed, one tile per
  // lane (PagedLoads): a pair of loads costs three lane reads instead of two 64-bit scalar
  // address computations from its table entry.
  const uint32_t lds_base = lds_addr_of(smem);
  auto dma_one = [&](const uint16_t* base, int64_t off, int64_t st, int ts, int lds_off,
                     const int (&voff)[kLpw], int h, const PagedLoads& pl, int tl) {
    const int i = is_paged(MODE) ? kLpw * wave + h : wave + kPfWaves * h;
    const uint32_t lds = __builtin_amdgcn_readfirstlane(lds_base + lds_off + 1024 * i);
    if constexpr (is_paged(MODE)) {
      const uint32_t lo = __builtin_amdgcn_readlane(pl.lo, tl);
      const uint32_t hi = __builtin_amdgcn_readlane(pl.hi, tl);
      lds_dma16(((uint64_t)hi << 32) | lo, __builtin_amdgcn_readlane(pl.bytes, tl), lds, voff[h]);
    } else {
      // Scalar selects only (no branch in the middle of the MFMA phases that issue these).
      const int t0 = max(ts, 0);
      const int rows = ts < 0 ? 0 : sclamp(kv_hi - ts, 0, kPfBc);
      lds_dma16(uniform_u64(reinterpret_cast<uint64_t>(base + off + (int64_t)t0 * st)),
                __builtin_amdgcn_readfirstlane(rows * (int)st * 2), lds,
                voff[0] + h * 4 * kPfWaves * (int)st * 2);
    }
  };

  // First key of each tile of stage j (may be negative or past kv_hi: then nothing is loaded).
  // (One stream: stage j is V(j) and K(j+1) only; the stream-1 starts are then never used.)
  auto k0_start = [&](int j) { return (j + 1) * kPfStep; };
  auto k1_start = [&](int j) { return NS == 2 ? j * kPfStep + kPfBc : -1; };
  auto v0_start = [&](int j) { return j * kPfStep; };
  auto v1_start = [&](int j) { return NS == 2 ? (j - 1) * kPfStep + kPfBc : -1; };

  // Paged modes work on groups of 16 stages: group m is stages 16m - 1 .. 16m + 14, and lane l
  // of a group register holds stage 16m - 1 + l/4, tile l%4 (K0, K1, V0, V1), so the table reads
  // and address arithmetic of 16 steps cost the vector instructions of one.
  //
  // tbl_fetch(m): the block-table entries of this wave's 8-row pairs of group m's tiles (-1 where
  // nothing is loaded).  A table read is a vector load, and a wait for it would also wait for
  // every LDS load in flight (the compiler cannot count those), so a group's entries are fetched
  // a whole group ahead and arrive with the loads of the step that fetches them.
  auto tbl_fetch = [&](int m) -> int {
    if constexpr (is_paged(MODE)) {
      const int j = 16 * m - 1 + (lane >> 2);
      const int t = lane & 3;
      const int ts = t == 0 ? k0_start(j) : t == 1 ? k1_start(j) : t == 2 ? v0_start(j) : v1_start(j);
      const int r0 = ts + 4 * kLpw * wave;
      if (ts >= 0 && ts < kv_hi && r0 < kv_hi)
        return p.block_table[(int64_t)b * p.bt_stride + (r0 >> __builtin_ctz(p.block_size))];
      return -1;
    } else {
      return 0;
    }
  };
  // resolve(m, entries): the address and byte length of those pairs, each lane its own (the same
  // lane layout), computed once the entries have arrived -- at the start of the step that issues
  // the group's first loads -- in a few vector instructions for all 64.  A tile outside
  // [0, kv_hi), an entry outside the pool or rows past kv_hi give a zero-length load.
  auto resolve = [&](int m, int entry) -> PagedLoads {
    PagedLoads r{};
    if constexpr (is_paged(MODE)) {
      const int j = 16 * m - 1 + (lane >> 2);
      const int t = lane & 3;
      const int ts = t == 0 ? k0_start(j) : t == 1 ? k1_start(j) : t == 2 ? v0_start(j) : v1_start(j);
      const int r0 = ts + 4 * kLpw * wave;
      const int n = min(max(kv_hi - r0, 0), 4 * kLpw);
      const bool kv = t < 2;
      const int64_t st = kv ? p.k_st : p.v_st;
      const uint16_t* base = kv ? p.k + k_off : p.v + v_off;
      const bool ok = (unsigned)entry < (unsigned)p.num_blocks && n > 0 && ts >= 0;
      const int bs_shift = __builtin_ctz(p.block_size);
      const uint64_t addr = reinterpret_cast<uint64_t>(
          base + (((int64_t)(ok ? entry : 0) << bs_shift) + (r0 & (p.block_size - 1))) * st);
      r.lo = (uint32_t)addr;
      r.hi = (uint32_t)(addr >> 32);
      r.bytes = ok ? (uint32_t)(n * st * 2) : 0u;
    }
    return r;
  };

  // The 8 load instructions of a wave for stage j (which goes to LDS slot j & 1): 4 for K tiles,
  // 4 for V tiles, q = 2*tile + h.  Inside the key loop they are issued one at a time between the
  // MFMAs of the score and PV phases rather than as a burst.  Paged modes: `pl` is the resolved
  // group holding stage j, whose tiles sit in lanes 4 * ((j + 1) % 16) + tile.
  // With two streams q = 2 * tile + h (tile 0 or 1 of the stage, instruction h of 2); with one
  // stream the stage holds one K and one V tile and q is the instruction (h of 4).
  auto dma_k = [&](int j, int q, const PagedLoads& pl) {
    const int t = NS == 2 ? q >> 1 : 0, h = NS == 2 ? q & 1 : q;
    const int o = (j & 1) * kStageBytes + t * kTileBytes;  // j & 1 folds when j's parity is known
    dma_one(p.k, k_off, p.k_st, t ? k1_start(j) : k0_start(j), o, k_voff, h, pl,
            4 * ((j + 1) & 15) + t);
  };
  auto dma_v = [&](int j, int q, const PagedLoads& pl) {
    const int t = NS == 2 ? q >> 1 : 0, h = NS == 2 ? q & 1 : q;
    const int o = kVRegion + (j & 1) * kStageBytes + t * kTileBytes;
    dma_one(p.v, v_off, p.v_st, t ? v1_start(j) : v0_start(j), o, v_voff, h, pl,
            4 * ((j + 1) & 15) + 2 + t);
  };
  auto load_stage = [&](int j, const PagedLoads& pl) {
    // Prologue stages only (j = -1, 0, constants): a tile that starts before key 0 holds nothing
    // any wave reads (stage -1: K1, V0 and V1; stage 0: V1), so its loads are not issued.  Each
    // load instruction costs its wave about 34 issue cycles and 1 KB of LDS writes even when it
    // only writes zeros.
#pragma unroll
    for (int q = 0; q < 4; ++q)
      if (((NS == 2 && (q >> 1)) ? k1_start(j) : k0_start(j)) >= 0) dma_k(j, q, pl);
#pragma unroll
    for (int q = 0; q < 4; ++q)
      if (((NS == 2 && (q >> 1)) ? v1_start(j) : v0_start(j)) >= 0) dma_v(j, q, pl);
  };
  // Each wave waits for its own loads, then the barrier publishes them to the work-group.
  // The builtin wait tells the compiler its own loads (Q) are done; the assembly one is the real
  // wait for the LDS loads, which the compiler does not track and would drop from the builtin.
  auto stage_ready = [&]() {
    __builtin_amdgcn_s_waitcnt(0x0F70);  // vmcnt(0)
    asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
    __syncthreads();
  };

  // Does this wave compute tile (j, ks)?  Its first key must be one some row of the wave sees.
  auto tile_kt = [&](int j) { return j * kPfStep + ks * kPfBc; };
  auto active = [&](int j) { return wave_active && j >= 0 && j < n_steps && tile_kt(j) < wave_hi; };

  // S^T of tile j from the K region of `slot`, MFMA row m holding key
  // pi(m) = 16*(m/16) + 8*((m/4)%2) + 4*((m/8)%2) + m%4 of its 32-key block (unmasked).
  const int pim = 16 * (r32 >> 4) + 8 * ((r32 >> 2) & 1) + 4 * ((r32 >> 3) & 1) + (r32 & 3);
  // Lane reads row pim (and pim + 32), chunk 2s + g, stored at chunk (2s + g) ^ (pim % 16).
  const int kx = pim * 256 + 16 * (g ^ (pim & 1)) + 32 * ((pim >> 1) & 7);
  // dma(q), q = 0..3, is called between the MFMAs (the K loads of the next stage).
  auto scores = [&](int j, int slot, f32x16& s0, f32x16& s1, auto&& dma) {
    const uint8_t* kp = smem + slot * kStageBytes + ks * kTileBytes;
    // K operands are read two k-steps ahead of their MFMAs: in this phase the SIMD's other wave
    // is in its softmax, so nothing else would cover the LDS latency.
    auto rd = [&](int s, u32x4& a0, u32x4& a1) {
      a0 = *reinterpret_cast<const u32x4*>(kp + (kx ^ (32 * s)));
      a1 = *reinterpret_cast<const u32x4*>(kp + (kx ^ (32 * s)) + 32 * 256);
    };
    u32x4 ka[3][2];
    rd(0, ka[0][0], ka[0][1]);
    rd(1, ka[1][0], ka[1][1]);
    s0 = f32x16{};
    s1 = f32x16{};
    // The MFMA phases run at raised wave priority, so that the arbiter prefers the SIMD's MFMA
    // stream over the other wave's softmax VALU when both are ready.
    __builtin_amdgcn_s_setprio(1);
#pragma unroll
    for (int s = 0; s < 8; ++s) {
      if (s + 2 < 8) rd(s + 2, ka[(s + 2) % 3][0], ka[(s + 2) % 3][1]);
      s0 = E::mfma32(ka[s % 3][0], qb[s], s0);
      s1 = E::mfma32(ka[s % 3][1], qb[s], s1);
      if (s & 1) dma(s >> 1);
      // Keep the reads two k-steps ahead: left alone, the scheduler sinks each read to just
      // before its MFMA, which then waits the whole LDS latency.
      __builtin_amdgcn_sched_barrier(0);
    }
    __builtin_amdgcn_s_setprio(0);
  };

  // Online softmax of tile j's scores: P^T as the B operand (k-step kk covers keys
  // kt + 16*kk + 8*g + t in slot t), running max / sum / O rescale updated.
  //
  // Accumulator r of s0 holds key kt + 16*(r/8) + 8*g + r%8 (+32 for s1).  Tiles that straddle the
  // causal diagonal or the row's end are masked first (keys >= lim to -inf, in registers, inside
  // the branch), so the common unmasked path runs no mask instructions.
  //
  // Fast path: the running max m_run stays the exponent reference and the row max is not
  // computed.  The reference may lag the true max by kRescaleSlack (every p <= 2^8); a lane whose
  // 32 values of p sum to at most 2^8 certainly has no p above that, so the max is only looked at
  // (and the state rescaled) when some lane's sum exceeds it -- or is inf / NaN, which is how the
  // first tile of a row (m_run = -inf) takes the slow path.  Both paths give the same p whenever
  // the slow path would not have moved the reference.
  auto softmax_body = [&](f32x16& s0, f32x16& s1, u32x4 (&pb)[4]) {
    auto exp_pack_sum = [&](float m_use) {
      // Pair by pair (exp, pack, sum) so that no more than a pair of fp32 p values is live.
      float lt = 0.f;
#pragma unroll
      for (int i = 0; i < 8; ++i) {  // s0 pairs 2i, 2i+1 -> pb[i/4][i%4]
        pb[i >> 2][i & 3] = E::pack2(exp2_fast(__builtin_fmaf(s0[2 * i], c, -m_use)),
                                     exp2_fast(__builtin_fmaf(s0[2 * i + 1], c, -m_use)));
        lt = E::sum2(pb[i >> 2][i & 3], lt);
      }
#pragma unroll
      for (int i = 0; i < 8; ++i) {  // s1 pairs -> pb[2 + i/4][i%4]
        pb[2 + (i >> 2)][i & 3] = E::pack2(exp2_fast(__builtin_fmaf(s1[2 * i], c, -m_use)),
                                           exp2_fast(__builtin_fmaf(s1[2 * i + 1], c, -m_use)));
        lt = E::sum2(pb[2 + (i >> 2)][i & 3], lt);
      }
      return lt;
    };
    float lt = exp_pack_sum(m_run);
    if (__any(!(lt <= kSumLimit))) {
      float mx = fmaxf(s0[0], s1[0]);
#pragma unroll
      for (int r = 1; r < 16; ++r) mx = fmax3(mx, s0[r], s1[r]);
      mx = fmaxf(mx, __shfl_xor(mx, 32));
      // Move the reference max only when the row's max has grown past the slack.
      const float m_cand = mx * c;
      const bool grow = m_cand > m_run + kRescaleSlack;
      if (__any(grow)) {
        // Lanes that keep their max scale by 1 (never exp2(-inf - -inf) = NaN); a first finite
        // max scales the empty state by exp2(-inf) = 0.
        const float alpha = grow ? exp2_fast(m_run - m_cand) : 1.f;
        l_run *= alpha;
#pragma unroll
        for (int i = 0; i < 4; ++i) oacc[i] *= alpha;
        if (grow) m_run = m_cand;
      }
      lt = exp_pack_sum(m_run == -INFINITY ? 0.f : m_run);
    }
    l_run += lt;
  };
  auto softmax = [&](int j, f32x16& s0, f32x16& s1, u32x4 (&pb)[4]) {
    const int kt = tile_kt(j);
    if (kt + kPfBc > wave_full) {
#pragma unroll
      for (int r = 0; r < 16; ++r) {
        const int key = kt + 16 * (r >> 3) + 8 * g + (r & 7);
        if (key >= lim) s0[r] = -INFINITY;
        if (key + 32 >= lim) s1[r] = -INFINITY;
      }
    }
    softmax_body(s0, s1, pb);
  };

  // O^T[d][query] += V^T[d][key] P^T[key][query] from the V region of `slot`; d-block db covers
  // d = 32*db + lane%32.
  //
  // V^T operand of lane l = 16G + 4k + q (g = G/2): d = 32*db + 16*(G%2) + i and keys
  // 16*kk + 8*g + [0, 8), as two transposing reads of rows 16*kk + 8*g + 4*sec + k, columns
  // 32*db + 16*(G%2) + 4q .. +3, at swizzled chunk 4*(db ^ k) + 2*(G%2) + q/2.
  const int vk = (lane >> 2) & 3;
  const int vx = 2048 * g + 256 * vk + 32 * ((lane >> 4) & 1) + 8 * (lane & 3);
  // dma(kk), kk = 0..3, is called between the MFMAs (the V loads of the next stage).
  auto pv = [&](int slot, const u32x4 (&pb)[4], auto&& dma) {
    // k-step outer, d-block inner: four independent accumulators back to back, and the four V^T
    // reads of a k-step issued together.
    const uint8_t* vp = smem + kVRegion + slot * kStageBytes + ks * kTileBytes + vx;
    // The V^T operands of k-step kk + 1 are read while the MFMAs of k-step kk run.
    auto rd = [&](int kk, u32x4 (&va)[4]) {
#pragma unroll
      for (int db = 0; db < 4; ++db) {
        const uint8_t* a = vp + 64 * (db ^ vk) + 4096 * kk;
        const u32x2 lo = ds_read_tr16(a);
        const u32x2 hi = ds_read_tr16(a + 1024);
        va[db] = u32x4{lo[0], lo[1], hi[0], hi[1]};
      }
    };
    u32x4 va[2][4];
    rd(0, va[0]);
    __builtin_amdgcn_s_setprio(1);
#pragma unroll
    for (int kk = 0; kk < 4; ++kk) {
      if (kk + 1 < 4) rd(kk + 1, va[(kk + 1) & 1]);
#pragma unroll
      for (int db = 0; db < 4; ++db) oacc[db] = E::mfma32(va[kk & 1][db], pb[kk], oacc[db]);
      dma(kk);
      __builtin_amdgcn_sched_barrier(0);  // the reads stay a k-step ahead (see scores)
    }
    __builtin_amdgcn_s_setprio(0);

  };

  // Prologue: stage -1 (slot 1) holds K(0,0) for stream 0's first scores, stage 0 goes to slot 0.
  // Paged modes: pl holds the loads of the current group of 16 stages, tbl the table entries of
  // the next group.
  PagedLoads pl{};
  int tbl = 0;
  if (n_steps > 0) {
    pl = resolve(0, tbl_fetch(0));
    load_stage(-1, pl);
    load_stage(0, pl);
    tbl = tbl_fetch(1);
  }
  // Every path reaches the loop with no vector load in flight (the Q registers included).
  stage_ready();
  // The two stream programs run as separate loops (independent register live ranges); both loops
  // execute the same barriers in the same order, which is all s_barrier needs.
  auto no_dma = [](int) {};
  if (ks == 0) {
    f32x16 sa0, sa1;  // scores of the next tile, carried across the barrier
    if (active(0)) scores(0, 1, sa0, sa1, no_dma);
    __syncthreads();  // slot 1 is rewritten during step 0
    // One step; `par` is j's parity as a compile-time constant, which turns every LDS offset of
    // the step into an immediate (the loop below is unrolled by two for that).
    auto step = [&](int j, auto par) {
      constexpr int slot = decltype(par)::value;
      // Stage j + 1, which this step loads, starts a group when j + 2 is a multiple of 16.
      if (is_paged(MODE) && slot == 0 && ((j + 2) & 15) == 0) {
        pl = resolve((j + 2) >> 4, tbl);
        tbl = tbl_fetch(((j + 2) >> 4) + 1);
      }
      auto next_v = [&](int q) { dma_v(2 * (j >> 1) + slot + 1, q, pl); };
      auto next_k = [&](int q) { dma_k(2 * (j >> 1) + slot + 1, q, pl); };
      if (active(j)) {
        u32x4 pb[4];
        softmax(j, sa0, sa1, pb);
        pv(slot, pb, next_v);
      } else {
#pragma unroll
        for (int q = 0; q < 4; ++q) next_v(q);
      }
      if (active(j + 1)) {
        scores(j + 1, slot, sa0, sa1, next_k);
      } else {
#pragma unroll
        for (int q = 0; q < 4; ++q) next_k(q);
      }
      stage_ready();
    };
    int j = 0;
    for (; j + 2 <= n_steps; j += 2) {
      step(j, Parity<0>{});
      step(j + 1, Parity<1>{});
    }
    if (j < n_steps) step(j, Parity<0>{});
    // Two streams: pairs with stream 1's barrier after its last PV.  One stream: the loop's last
    // barrier already follows every LDS read; this one is kept so both shapes share the code.
    __syncthreads();
  } else {
    u32x4 pbv[4];  // P of the previous tile, carried across the barrier
    __syncthreads();
    auto step = [&](int j, auto par) {
      constexpr int slot = decltype(par)::value;
      // Stage j + 1, which this step loads, starts a group when j + 2 is a multiple of 16.
      if (is_paged(MODE) && slot == 0 && ((j + 2) & 15) == 0) {
        pl = resolve((j + 2) >> 4, tbl);
        tbl = tbl_fetch(((j + 2) >> 4) + 1);
      }
      auto next_v = [&](int q) { dma_v(2 * (j >> 1) + slot + 1, q, pl); };
      auto next_k = [&](int q) { dma_k(2 * (j >> 1) + slot + 1, q, pl); };
      if constexpr (!is_paged(MODE)) {
        // Scores first, then the previous tile's PV: this stream's cheaper score phase (one K read
        // per MFMA against two transposing V^T reads) starts the step against the other stream's
        // softmax, and its PV phase, not its score phase, runs into the other stream's PV
        // (4096 causal 60.4 -> 59.7 us, 8192 non-causal 369.2 -> 367.0 us; bitwise the same
        // output).  The paged modes keep PV first: their scores-first order measured 0.5 us slower.
        f32x16 s0, s1;
        if (active(j)) {
          scores(j, slot, s0, s1, next_k);
        } else {
#pragma unroll
          for (int q = 0; q < 4; ++q) next_k(q);
        }
        if (active(j - 1)) {
          pv(slot, pbv, next_v);
        } else {
#pragma unroll
          for (int q = 0; q < 4; ++q) next_v(q);
        }
        if (active(j)) softmax(j, s0, s1, pbv);
      } else {
        if (active(j - 1)) {
          pv(slot, pbv, next_v);
        } else {
#pragma unroll
          for (int q = 0; q < 4; ++q) next_v(q);
        }
        if (active(j)) {
          f32x16 s0, s1;
          scores(j, slot, s0, s1, next_k);
          softmax(j, s0, s1, pbv);
        } else {
#pragma unroll
          for (int q = 0; q < 4; ++q) next_k(q);
        }
      }
      stage_ready();
    };
    int j = 0;
    for (; j + 2 <= n_steps; j += 2) {
      step(j, Parity<0>{});
      step(j + 1, Parity<1>{});
    }
    if (j < n_steps) step(j, Parity<0>{});
    // The last tile's V is in stage n_steps.
    if (active(n_steps - 1)) pv(n_steps & 1, pbv, no_dma);
    __syncthreads();
  }

  if constexpr (NS == 1) {
    // One stream holds whole rows: normalise all of O and store it.  The rows go through LDS so
    // that every global store writes whole 256-byte rows: row-major [32 rows][128 d] in this
    // wave's staging area, 16-byte chunks XOR-swizzled by row % 16.  The loop's last barrier came
    // after every LDS read and load of the key loop, so the areas may overwrite the K/V stages.
    const float l_tot = l_run + __shfl_xor(l_run, 32);
    const float inv = l_tot > 0.f ? 1.f / l_tot : 0.f;
    uint8_t* ot = smem + wave * (32 * 256);
    // Accumulator r of d-block db is d = 32*db + 8*(r/4) + 4*g + r%4: chunk 4*db + r/4, half g.
#pragma unroll
    for (int db = 0; db < 4; ++db) {
#pragma unroll
      for (int rr = 0; rr < 4; ++rr) {
        const u32x2 val = {E::pack2(oacc[db][rr * 4] * inv, oacc[db][rr * 4 + 1] * inv),
                           E::pack2(oacc[db][rr * 4 + 2] * inv, oacc[db][rr * 4 + 3] * inv)};
        *reinterpret_cast<u32x2*>(ot + r32 * 256 + 16 * ((4 * db + rr) ^ (r32 & 15)) + 8 * g) = val;
      }
    }
    __builtin_amdgcn_wave_barrier();
#pragma unroll
    for (int k = 0; k < 8; ++k) {  // rows 4k .. 4k+3, one 16-byte chunk per lane
      const int row = 4 * k + (lane >> 4), ch = lane & 15;
      const u32x4 val = *reinterpret_cast<const u32x4*>(ot + row * 256 + 16 * (ch ^ (row & 15)));
      if (wq0 + row < T_b)
        *reinterpret_cast<u32x4*>(p.o + o_off + (int64_t)(wq0 + row) * p.o_st + ch * 8) = val;
    }
    if (p.lse && g == 0 && qrow < T_b)
      p.lse[l_off + (int64_t)qrow * p.l_st] =
          l_tot > 0.f ? (m_run + __builtin_log2f(l_tot)) * kLn2 : -INFINITY;
  } else {
    // The two streams of a row group split the epilogue: each gives the other the half of O it does
    // not keep (stream 0 keeps d 0..63, stream 1 d 64..127) with its (m, l), merges its own half
    // and stores it, so the merge, the normalisation and the stores run on all 8 waves instead of
    // stream 0's 4 (16 packed sequences 43.2 -> 40.5 us, 768 equal 1024-key tiles 66.6 -> 64.9 us).
    // Exchange area of wave (rg, ks): [32 O values + m + l][lane].
    float* red = reinterpret_cast<float*>(smem);
    constexpr int kXVals = 34;
    {
      float* dst = red + (rg * NS + ks) * kXVals * 64 + lane;
      // d-blocks handed over (whole-vector selects on the wave-uniform stream: a runtime index
      // into the accumulators would put them in scratch memory)
      const f32x16 give0 = ks == 0 ? oacc[2] : oacc[0];
      const f32x16 give1 = ks == 0 ? oacc[3] : oacc[1];
  #pragma unroll
      for (int r = 0; r < 16; ++r) {
        dst[r * 64] = give0[r];
        dst[(16 + r) * 64] = give1[r];
      }
      dst[32 * 64] = m_run;
      dst[33 * 64] = l_run;
    }
    __syncthreads();
    const int keep = ks == 0 ? 0 : 2;  // first d-block kept
    const f32x16 keep0 = ks == 0 ? oacc[0] : oacc[2];
    const f32x16 keep1 = ks == 0 ? oacc[1] : oacc[3];
    f32x16 ok[2];
    {
      // Rows past T_b keep their lanes for the row-wise stores below (their values are merged,
      // harmlessly, and never stored).
      const float* src = red + (rg * NS + (ks ^ 1)) * kXVals * 64 + lane;
      // Both streams evaluate the same expression, O = O_0 f_0 + O_1 f_1 with stream 0's state
      // first, so each half of a row is rounded as if one wave merged the whole row.
      const float mo = src[32 * 64];
      const float lo = src[33 * 64];
      const float M = ks == 0 ? fmaxf(m_run, mo) : fmaxf(mo, m_run);
      const float M_use = M == -INFINITY ? 0.f : M;
      const float fs = exp2_fast(m_run - M_use);  // this stream's factor
      const float fo = exp2_fast(mo - M_use);     // the other's
      // fma(O_0, f_0, O_1 f_1) spelled out, so that the compiler cannot contract the two streams'
      // expressions differently.
      if (ks == 0) {
  #pragma unroll
        for (int r = 0; r < 16; ++r) {
          ok[0][r] = __builtin_fmaf(keep0[r], fs, src[r * 64] * fo);
          ok[1][r] = __builtin_fmaf(keep1[r], fs, src[(16 + r) * 64] * fo);
        }
        l_run = __builtin_fmaf(l_run, fs, lo * fo);
      } else {
  #pragma unroll
        for (int r = 0; r < 16; ++r) {
          ok[0][r] = __builtin_fmaf(src[r * 64], fo, keep0[r] * fs);
          ok[1][r] = __builtin_fmaf(src[(16 + r) * 64], fo, keep1[r] * fs);
        }
        l_run = __builtin_fmaf(lo, fo, l_run * fs);
      }
      m_run = M;
    }

    const float l_tot = l_run + __shfl_xor(l_run, 32);
    const float inv = l_tot > 0.f ? 1.f / l_tot : 0.f;
    // Accumulator r of d-block db is d = 32*db + 8*(r/4) + 4*g + r%4: four consecutive d per group.
    // The wave's half rows go through LDS so that every global store writes whole 128-byte
    // half rows: row-major [32 rows][64 d] in this wave's staging area (after the exchange areas),
    // 16-byte chunks XOR-swizzled by row % 8 so that the writes and the reads spread over the banks.
    // Direct stores from the MFMA layout (16 bytes into each of 32 rows per instruction) measured
    // 5-7% slower on short tiles when one wave stored whole rows.
    {
      uint8_t* ot = reinterpret_cast<uint8_t*>(red + kPfWaves * kXVals * 64) + wave * (32 * 128);
  #pragma unroll
      for (int i = 0; i < 2; ++i) {
  #pragma unroll
        for (int rr = 0; rr < 4; ++rr) {
          const u32x2 val = {E::pack2(ok[i][rr * 4] * inv, ok[i][rr * 4 + 1] * inv),
                             E::pack2(ok[i][rr * 4 + 2] * inv, ok[i][rr * 4 + 3] * inv)};
          *reinterpret_cast<u32x2*>(ot + r32 * 128 + 16 * ((4 * i + rr) ^ (r32 & 7)) + 8 * g) = val;
        }
      }
      __builtin_amdgcn_wave_barrier();
  #pragma unroll
      for (int k = 0; k < 4; ++k) {  // rows 8k .. 8k+7, one 16-byte chunk per lane
        const int row = 8 * k + (lane >> 3), ch = lane & 7;
        const u32x4 val = *reinterpret_cast<const u32x4*>(ot + row * 128 + 16 * (ch ^ (row & 7)));
        if (wq0 + row < T_b)
          *reinterpret_cast<u32x4*>(p.o + o_off + (int64_t)(wq0 + row) * p.o_st + keep * 32 +
                                    ch * 8) = val;
      }
    }
    if (ks == 0 && p.lse && g == 0 && qrow < T_b)
      p.lse[l_off + (int64_t)qrow * p.l_st] =
          l_tot > 0.f ? (m_run + __builtin_log2f(l_tot)) * kLn2 : -INFINITY;
  }
  probe_mark(p.clock_probe, blockIdx.x, true);
}

// Key streams per work-group for a launch of `grid` work-groups whose query tiles see at most
// `max_keys` keys.  Two streams halve the time of the longest query tile, which is what bounds a
// launch of about one work-group per CU (one long causal sequence); one stream fits two
// work-groups per CU, which hides each one's start (item, Q and first stages) and end (stores)
// behind the other's key loop once there are enough work-groups to fill both slots of every CU
// and the tiles are short enough for those to matter.  Measured (us per launch, two streams / one
// stream): 2 x 4096 causal 111.1 / 107.5, 3 x 4096 165.8 / 159.3, 16 packed rows of up to 1024
// 40.8 / 30.6; 1 x 6144 causal 122.8 / 134.4, 1 x 16384 causal 726 / 741.  MI_FA2_PREFILL_STREAMS
// = 1 or 2 forces one shape (read at every launch, so that a test can run both in one process).
static int prefill_streams(int grid, int n_cus, int max_keys) {
  const char* e = std::getenv("MI_FA2_PREFILL_STREAMS");
  if (e != nullptr && (e[0] == '1' || e[0] == '2') && e[1] == 0) return e[0] - '0';
  return grid >= prefill_one_stream_min_grid(n_cus) && max_keys <= kPrefillOneStreamMaxKeys ? 1
                                                                                            : 2;
}

template <typename E, int MODE>
static hipError_t launch_prefill_t(const FwdParams& p, int max_seqlen_q, hipStream_t stream) {
  const int n_qt = (max_seqlen_q + kPfRows - 1) / kPfRows;
  if (n_qt == 0 || p.B == 0) return hipSuccess;
  // Packed batches: one slot per (rank, class, query head) of the full B x n_qt box, numbered by
  // prefill_item_packed (real tiles first).
  const bool packed = (MODE == kVarlen || MODE == kPagedVarlen) && p.B <= 64;
  const int X = 1 << p.xcd_log2;
  const int grid = packed ? X * p.group * ((p.B * p.Hkv * n_qt + X - 1) / X)
                          : prefill_grid_size(p.B * p.Hkv, p.group, n_qt, p.xcd_log2);
  const ItemMap map = make_item_map(p.B * p.Hkv, p.group, p.Hkv, p.xcd_log2);
  // Keys a query tile sees at most: the padded key count, or for packed rows (no key bound
  // given) the longest row's query count, which bounds them for causal self-attention batches.
  const int max_keys = p.S > 0 ? p.S : max_seqlen_q;
  if (prefill_streams(grid, p.n_cus, max_keys) == 1)
    hipLaunchKernelGGL((fa2_prefill_kernel<E, MODE, 1>), dim3(grid), dim3(PfShape<1>::kThreads), 0,
                       stream, p, n_qt, map);
  else
    hipLaunchKernelGGL((fa2_prefill_kernel<E, MODE, 2>), dim3(grid), dim3(PfShape<2>::kThreads), 0,
                       stream, p, n_qt, map);
  return hipGetLastError();
}

hipError_t launch_prefill(const FwdParams& p, int dtype, int mode, int max_seqlen_q,
                          hipStream_t stream) {
  if (dtype == 0) {
    if (mode == kDense) return launch_prefill_t<BF16, kDense>(p, max_seqlen_q, stream);
    if (mode == kVarlen) return launch_prefill_t<BF16, kVarlen>(p, max_seqlen_q, stream);
    if (mode == kPagedVarlen) return launch_prefill_t<BF16, kPagedVarlen>(p, max_seqlen_q, stream);
    return launch_prefill_t<BF16, kPaged>(p, max_seqlen_q, stream);
  }
  if (mode == kDense) return launch_prefill_t<FP16, kDense>(p, max_seqlen_q, stream);
  if (mode == kVarlen) return launch_prefill_t<FP16, kVarlen>(p, max_seqlen_q, stream);
  if (mode == kPagedVarlen) return launch_prefill_t<FP16, kPagedVarlen>(p, max_seqlen_q, stream);
  return launch_prefill_t<FP16, kPaged>(p, max_seqlen_q, stream);
}

}  // namespace mi_fa2
