// Shared device-side definitions of the gfx950 attention kernels: vector types, the MFMA wrappers
// for bf16/fp16, fp32 -> 16-bit packing, and the parameter block every kernel receives.
//
// MFMA operand layouts used throughout (wave64, gfx950):
//   v_mfma_f32_32x32x16_{bf16,f16}: A[m][k] lane l holds row m = l%32 and 8 k-values; B[k][n] lane l
//     holds column n = l%32 and the same 8 k-slots; D[m][n] lane l holds column n = l%32 and rows
//     m = 8*(r/4) + 4*(l/32) + r%4 for its 16 accumulators r.
//   v_mfma_f32_16x16x32_{bf16,f16}: A lane l holds row m = l%16, B column n = l%16, 8 k-slots each;
//     D lane l holds column n = l%16 and rows m = 4*(l/16) + r for its 4 accumulators r.
// The kernels only rely on A and B sharing the k-slot order (any permutation of the contraction
// index inside one MFMA gives the same sum), so they choose the k <-> slot mapping that makes
// every operand a plain 16- or 8-byte load.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace mi_fa2 {

typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
typedef uint32_t u32x2 __attribute__((ext_vector_type(2)));
typedef float f32x16 __attribute__((ext_vector_type(16)));
typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef __bf16 bf16x2 __attribute__((ext_vector_type(2)));
typedef _Float16 f16x8 __attribute__((ext_vector_type(8)));
typedef _Float16 f16x2 __attribute__((ext_vector_type(2)));

constexpr int kHeadDim = 128;
constexpr float kLn2 = 0.69314718055994530942f;
constexpr float kLog2e = 1.44269504088896340736f;

// KV addressing modes.
//   kDense : row b, head h, token t at base + b*s_b + h*s_h + t*s_t (the padded [B,H,S,d] layout)
//   kVarlen: token t of row b at base + (cu_k[b] + t)*s_t + h*s_h (packed [total, H, d])
//   kPaged : token t of row b at base + (table[b][t/bs]*bs + t%bs)*s_t + h*s_h (KVCache pool)
//   kPagedVarlen: K/V as kPaged, queries packed as kVarlen ([total, H, d] + cu_q; rows of
//            different query counts over their own cached keys)
enum KvMode { kDense = 0, kVarlen = 1, kPaged = 2, kPagedVarlen = 3 };

__host__ __device__ constexpr bool is_paged(int mode) { return mode == kPaged || mode == kPagedVarlen; }

struct BF16 {
  static constexpr uint32_t kOnes2 = 0x3f803f80u;  // (1.0, 1.0)
  // acc + lo(a) + hi(a): sums two packed values in fp32 (v_dot2c_f32_bf16 against ones)
  static __device__ __forceinline__ float sum2(uint32_t a, float acc) {
    return __builtin_amdgcn_fdot2_f32_bf16(__builtin_bit_cast(bf16x2, a),
                                           __builtin_bit_cast(bf16x2, kOnes2), acc, false);
  }
  static __device__ __forceinline__ float lo(uint32_t a) { return __uint_as_float(a << 16); }
  static __device__ __forceinline__ float hi(uint32_t a) { return __uint_as_float(a & 0xffff0000u); }
  static __device__ __forceinline__ f32x16 mfma32(u32x4 a, u32x4 b, f32x16 c) {
    return __builtin_amdgcn_mfma_f32_32x32x16_bf16(__builtin_bit_cast(bf16x8, a),
                                                   __builtin_bit_cast(bf16x8, b), c, 0, 0, 0);
  }
  static __device__ __forceinline__ f32x4 mfma16(u32x4 a, u32x4 b, f32x4 c) {
    return __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(bf16x8, a),
                                                   __builtin_bit_cast(bf16x8, b), c, 0, 0, 0);
  }
  // Round-to-nearest-even fp32 -> bf16 of two values, low half = lo.
  static __device__ __forceinline__ uint32_t pack2(float lo, float hi) {
    bf16x2 v = {(__bf16)lo, (__bf16)hi};
    return __builtin_bit_cast(uint32_t, v);
  }
};

struct FP16 {
  static constexpr uint32_t kOnes2 = 0x3c003c00u;  // (1.0, 1.0)
  static __device__ __forceinline__ float sum2(uint32_t a, float acc) {
    return __builtin_amdgcn_fdot2(__builtin_bit_cast(f16x2, a), __builtin_bit_cast(f16x2, kOnes2),
                                  acc, false);
  }
  static __device__ __forceinline__ float lo(uint32_t a) {
    return (float)__builtin_bit_cast(f16x2, a)[0];
  }
  static __device__ __forceinline__ float hi(uint32_t a) {
    return (float)__builtin_bit_cast(f16x2, a)[1];
  }
  static __device__ __forceinline__ f32x16 mfma32(u32x4 a, u32x4 b, f32x16 c) {
    return __builtin_amdgcn_mfma_f32_32x32x16_f16(__builtin_bit_cast(f16x8, a),
                                                  __builtin_bit_cast(f16x8, b), c, 0, 0, 0);
  }
  static __device__ __forceinline__ f32x4 mfma16(u32x4 a, u32x4 b, f32x4 c) {
    return __builtin_amdgcn_mfma_f32_16x16x32_f16(__builtin_bit_cast(f16x8, a),
                                                  __builtin_bit_cast(f16x8, b), c, 0, 0, 0);
  }
  static __device__ __forceinline__ uint32_t pack2(float lo, float hi) {
    f16x2 v = {(_Float16)lo, (_Float16)hi};
    return __builtin_bit_cast(uint32_t, v);
  }
};

// Prefill launches of at least this many work-groups (two per CU), none of whose query tiles
// sees more than kPrefillOneStreamMaxKeys keys, use the one-stream work-group shape, which fits
// two work-groups per CU: it hides each tile's start and end behind the other work-group's key
// loop, but walks a tile's keys with half the waves (a long tile's latency doubles) and runs its
// steady state about 4.5% slower per CU.
inline int prefill_one_stream_min_grid(int n_cus) { return 2 * n_cus; }
constexpr int kPrefillOneStreamMaxKeys = 4096;

// Everything a kernel launch needs; passed by value (kernel argument segment).
struct FwdParams {
  const uint16_t* q;
  const uint16_t* k;
  const uint16_t* v;
  uint16_t* o;
  float* lse;                 // may be null
  const int32_t* kv_lens;     // kDense/kPaged: [B] keys per row; null = all S (kDense only)
  const int32_t* cu_q;        // kVarlen: [B+1] query offsets
  const int32_t* cu_k;        // kVarlen: [B+1] key offsets
  const int32_t* block_table; // kPaged: [B][bt_stride]
  int64_t bt_stride;
  int32_t block_size;         // kPaged: tokens per block, multiple of 16
  int32_t num_blocks;         // kPaged: blocks in the pool
  // element strides; for kVarlen the *_sb strides are unused and *_st is the packed token stride
  int64_t q_sb, q_sh, q_st;
  int64_t k_sb, k_sh, k_st;
  int64_t v_sb, v_sh, v_st;
  int64_t o_sb, o_sh, o_st;
  int64_t l_sb, l_sh, l_st;
  int32_t B, Hq, Hkv, group;  // group = Hq / Hkv
  int32_t T;                  // query rows per batch row (padded modes)
  int32_t S;                  // key capacity per row (upper bound of kv_lens)
  int32_t causal;
  float scale_log2;           // sm_scale * log2(e): scores are kept in the exp2 domain
  // split-KV decode workspace (fp32): partial O [B][Hq][max_splits][128], m and l [B][Hq][max_splits]
  float* ws_o;
  float* ws_m;
  float* ws_l;
  int32_t* ws_np;             // decode: partials per (row, kv head) item, [B][Hkv]
  int32_t n_wg;               // decode: work-groups launched
  int32_t max_splits;         // decode: partial slots per (row, query head)
  // the device's compute units and log2 of its XCD count (each XCD has its own L2), read once per
  // device by the C ABI: they size grids and map work-groups to XCDs
  int32_t n_cus;
  int32_t xcd_log2;
  // measurement only (mi_fa2_set_clock_probe), usually null: [16] uint64, the shader cycles and
  // 100 MHz ticks spent by the first work-groups of each launch, summed per XCD
  uint64_t* clock_probe;
};

// Everything the fused RoPE + KV-write launch needs (rope_kv.hip).
struct RopeParams {
  const uint16_t* qkv;  // [n_tokens][qkv_st]: q heads, then k heads, then v heads, 128 each
  int64_t qkv_st;
  const uint16_t* cos;  // [n_tokens][cs_st] (128 used)
  const uint16_t* sin;
  int64_t cs_st;
  const int32_t* slots;  // [n_tokens] cache slot of each token
  uint16_t* q_out;       // [n_tokens][q_st]: rotated q heads, 128 each
  int64_t q_st;
  uint16_t* k_pool;  // [num_slots][pool_sh * heads_kv]: token-major cache layer
  uint16_t* v_pool;
  int64_t pool_st, pool_sh;
  int32_t num_slots;
  int32_t n_tokens, Hq, Hkv;
};

// Token sampler (sample.hip).
struct SampleParams {
  const void* logits;
  int64_t row_stride;   // elements
  int32_t* tokens;
  float* part_s;        // [batch][chunks] best score of each chunk
  int32_t* part_i;      // [batch][chunks] its index (-1: no candidate)
  int batch, vocab, chunks, greedy;
  float inv_t;
  uint32_t seed_lo, seed_hi, off_lo, off_hi;
};

// Fused residual-add + RMSNorm and SiLU x up (model_ops.hip).
struct ModelOpParams {
  const uint16_t* x;    // [rows][x_st]: rows to normalise (or gate|up rows for silu_mul)
  int64_t x_st;
  const uint16_t* y;    // [rows][y_st]: added to x first, or NULL
  int64_t y_st;
  const uint16_t* weight;  // [hidden]
  uint16_t* r_out;      // [rows][r_st]: x + y, or NULL
  int64_t r_st;
  uint16_t* out;        // [rows][out_st]
  int64_t out_st;
  int32_t rows, hidden;
  float eps;
};

// Log-sum-exp merge of partials over disjoint key ranges (fa2_merge.hip).  Element strides.
struct MergeParams {
  const float* part_o;    // [part][row][head][128] fp32, normalised
  const float* part_lse;  // [part][row][head] fp32, natural log (-inf: the part saw no key)
  const int32_t* n_parts; // [rows] partials per row, or NULL: max_parts each
  int64_t po_sp, po_sr, po_sh;
  int64_t pl_sp, pl_sr, pl_sh;
  void* o;                // [row][head][128]
  int64_t o_sr, o_sh;
  float* lse;             // [row][head], or NULL
  int64_t l_sr, l_sh;
  int32_t rows, heads, max_parts;
};

// Per-step paged-cache metadata (step_meta.hip).
struct StepMetaParams {
  const int32_t* row_slots;  // [B] sequence slot of each row, < 0: padding row
  const int32_t* cu;         // [B + 1] packed token offsets, or NULL: row b holds tokens b*T ..
  int32_t T, B, W, block_size, max_seqs;
  int32_t* seq_lens;         // [max_seqs] tokens held per slot, advanced in place
  const int32_t* tables;     // [max_seqs][table_stride] block ids per slot
  int64_t table_stride;
  int32_t* starts;           // [B]
  int32_t* kv_lens;          // [B]
  int32_t* block_table;      // [B][W]
  int32_t* slots;            // [N]
  int32_t* positions;        // [N] or NULL
  int32_t* last_idx;         // [B] or NULL
};

__device__ __forceinline__ u32x4 ld16(const uint16_t* p) { return *reinterpret_cast<const u32x4*>(p); }

// Raw buffer resource over [base, base + bytes): loads at offsets past `bytes` return zeros, which
// is how the kernels zero-fill keys past a row's end without a branch per load.
__device__ __forceinline__ __amdgpu_buffer_rsrc_t make_rsrc(const void* base, int bytes) {
  return __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(base), 0, bytes, 0x00020000);
}

__device__ __forceinline__ u32x4 ld16_buf(__amdgpu_buffer_rsrc_t r, int byte_off) {
  return __builtin_amdgcn_raw_buffer_load_b128(r, byte_off, 0, 0);
}

// Direct-to-LDS load (gfx950 buffer_load_dwordx4 ... lds): lane l's 16 bytes at byte `voffset` of
// the raw buffer [base, base + bytes) land at LDS byte address lds_addr + 16*l; offsets past
// `bytes` write zeros.  base, bytes and lds_addr must be wave-uniform.
//
// Issued as inline assembly on purpose: the compiler cannot tell which LDS bytes the intrinsic
// writes, so it would wait for every such load to finish before the next LDS read of any address
// (vmcnt(0) in front of the MFMA operand reads of the other stage), serialising the prefetch with
// the compute it is meant to overlap.  Callers wait with s_waitcnt vmcnt(0) (also as assembly:
// the compiler drops waits for loads it does not know about) before a barrier.  m0 (the LDS
// destination) is written here without a clobber: the compiler treats m0 as a reserved register
// and says it ignores clobbers of those.  It does not keep values of its own in m0 either: it
// writes m0 right before each of its own uses.  tests/test_isa_carry.py checks that in the
// compiled kernels: no m0 read outside the assembly finds its value set inside it.
__device__ __forceinline__ void lds_dma16(uint64_t base, uint32_t bytes, uint32_t lds_addr,
                                          int voffset) {
  const u32x4 rsrc = {(uint32_t)base, (uint32_t)(base >> 32) & 0xffffu, bytes, 0x00020000u};
  asm volatile(
      "s_mov_b32 m0, %0\n\t"
      "s_nop 0\n\t"  // one wait state between an SALU write of m0 and an LDS DMA reading it
      "buffer_load_dwordx4 %1, %2, 0 offen lds"
      :
      : "s"(lds_addr), "v"(voffset), "s"(rsrc)
      : "memory");
}

// A wave-uniform 64-bit value as such (readfirstlane of both halves; each half is widened as an
// unsigned 32-bit value, never sign-extended).
__device__ __forceinline__ uint64_t uniform_u64(uint64_t x) {
  const uint32_t lo = (uint32_t)__builtin_amdgcn_readfirstlane((int)(uint32_t)x);
  const uint32_t hi = (uint32_t)__builtin_amdgcn_readfirstlane((int)(uint32_t)(x >> 32));
  return ((uint64_t)hi << 32) | (uint64_t)lo;
}

// LDS byte address of a pointer into __shared__ memory.
__device__ __forceinline__ uint32_t lds_addr_of(const void* p) {
  return (uint32_t)(uintptr_t)(const __attribute__((address_space(3))) void*)p;
}

// ds_read_b64_tr_b16: within each 16-lane group, lane 4k+q reads 4 16-bit values v[k][4q..4q+3]
// and lane i receives v[0..3][i] -- a 4x16 transpose.  Used to read V^T operands out of a
// row-major V tile.
typedef short i16x4 __attribute__((ext_vector_type(4)));
__device__ __forceinline__ u32x2 ds_read_tr16(const void* lds) {
  const i16x4 t = __builtin_amdgcn_ds_read_tr16_b64_v4i16(
      (__attribute__((address_space(3))) i16x4*)const_cast<void*>(lds));
  return __builtin_bit_cast(u32x2, t);
}

// Bytes x.b[s0..] per selector: v_perm_b32 picks bytes of {hi_word, lo_word}.
__device__ __forceinline__ uint32_t perm_b32(uint32_t hi_word, uint32_t lo_word, uint32_t sel) {
  return __builtin_amdgcn_perm(hi_word, lo_word, sel);
}

// clamp(x, lo, hi) of a wave-uniform value on the scalar unit (the compiler's clamp pattern is a
// vector instruction, which then needs a readfirstlane back).
// x must be wave-uniform; it is passed through readfirstlane so that the operand is an SGPR even
// where the compiler cannot prove the uniformity itself.  s_max / s_min write SCC, which the
// compiler may hold live across the statement (the carry of a 64-bit s_add_u32 / s_addc_u32
// pair), so SCC is declared clobbered.
__device__ __forceinline__ int sclamp(int x, int lo, int hi) {
  int r;
  asm("s_max_i32 %0, %1, %2\n\ts_min_i32 %0, %0, %3"
      : "=&s"(r)
      : "s"(__builtin_amdgcn_readfirstlane(x)), "s"(lo), "s"(hi)
      : "scc");
  return r;
}

// Paged loads of one stage, resolved one instruction per lane: the 64-bit byte address of the
// instruction's first row (lo, hi) and its byte length.
struct PagedLoads {
  uint32_t lo, hi, bytes;
};

// x as a value the compiler cannot see through.  Address arithmetic derived from it stays where it
// is used instead of being hoisted out of a loop and kept live (or spilled) through the loop.
__device__ __forceinline__ int opaque(int x) {
  asm volatile("" : "+v"(x));
  return x;
}

__device__ __forceinline__ float fmax3(float a, float b, float c) { return fmaxf(fmaxf(a, b), c); }

__device__ __forceinline__ float exp2_fast(float x) { return __builtin_amdgcn_exp2f(x); }

// Clock probe (measurement only): with p.clock_probe set, thread 0 of each of a launch's first 8
// work-groups (one per XCD on MI355X) reads its CU's shader-cycle counter (s_memtime: the CU's own
// clocks) and the 100 MHz real-time counter (s_memrealtime) when it starts and when it is done,
// and its XCD's pair of sums, probe[2 * xcd] and probe[2 * xcd + 1], takes the differences (the
// start readings are subtracted at the start and the end readings added at the end, modulo 2^64,
// so that nothing is held in registers in between): their ratio is the clock that XCD ran the
// kernel at.  The counts of different CUs are never compared.  Off (a null pointer), it costs a
// uniform branch at the start and at the end.
__device__ __forceinline__ void probe_mark(uint64_t* probe, uint32_t wg_linear, bool end) {
  if (probe != nullptr && wg_linear < 8 && threadIdx.x == 0) {
    const uint64_t c = __builtin_amdgcn_s_memtime();
    const uint64_t t = __builtin_amdgcn_s_memrealtime();
    uint32_t xcc;
    asm volatile("s_getreg_b32 %0, hwreg(HW_REG_XCC_ID)" : "=s"(xcc));
    xcc &= 7u;
    atomicAdd(reinterpret_cast<unsigned long long*>(probe + 2 * xcc),
              (unsigned long long)(end ? c : 0 - c));
    atomicAdd(reinterpret_cast<unsigned long long*>(probe + 2 * xcc + 1),
              (unsigned long long)(end ? t : 0 - t));
  }
}

// Keys held by row b, clamped to [0, cap].
__device__ __forceinline__ int clamp_len(int n, int cap) { return n < 0 ? 0 : (n > cap ? cap : n); }

}  // namespace mi_fa2
