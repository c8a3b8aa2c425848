// Fused rotary embedding + paged KV-cache write, the step right before attention.
//
// Replaces, on the GPU path, apply_rope (model.py:62-65, applied at model.py:92) and the two
// index_copy_ of KVCache.write (kv_cache.py:108-115, called at model.py:96): for every new token
// it reads the token's fused q|k|v projection row once, rotates q and k, writes the rotated q for
// the attention kernel and scatters the rotated k and the v into the cache slot the block table
// assigned to the token.  One launch per layer instead of about a dozen elementwise launches.
//
// Arithmetic is the reference's own, rounding step for step as its bf16/fp16 tensor ops do:
//   out = round(round(x * cos) + round(rotate_half(x) * sin)),
//   rotate_half(x)[d] = -x[d + 64] for d < 64, x[d - 64] for d >= 64,
// with the products and the sum taken in fp32 (exact for 16-bit inputs) and each result rounded
// to the tensor dtype.  cos/sin are the model's own tables (position-dependent, computed once per
// step), so the outputs are bitwise those of the unfused torch code.
//
// Work: per token, (Hq + Hkv) rotated heads in units of 2 x 8 elements (dims d0..d0+7 and
// d0+64..d0+71: a unit holds both halves of its rotation pairs) and Hkv copied v heads in units
// of 8 elements; one thread per unit, 16-byte loads and stores.  Memory-bound and tiny per step.
#include "fa2_common.h"

namespace mi_fa2 {


template <typename T>
struct Num;
template <>
struct Num<BF16> {
  static __device__ __forceinline__ float f(uint16_t x) { return __uint_as_float((uint32_t)x << 16); }
  static __device__ __forceinline__ uint16_t r(float x) {
    return (uint16_t)(BF16::pack2(x, 0.f) & 0xffffu);
  }
};
template <>
struct Num<FP16> {
  static __device__ __forceinline__ float f(uint16_t x) {
    return (float)__builtin_bit_cast(_Float16, x);
  }
  static __device__ __forceinline__ uint16_t r(float x) {
    return (uint16_t)(FP16::pack2(x, 0.f) & 0xffffu);
  }
};

// Every product must be rounded on its own before the add, as the reference's separate tensor ops
// do; this opaque copy keeps the compiler from contracting product and add into one fma (which it
// does for fp16, where the hardware has one).
__device__ __forceinline__ float rounded(float x) {
  asm volatile("" : "+v"(x));
  return x;
}

template <typename E>
__global__ __launch_bounds__(256) void rope_kv_kernel(const RopeParams p) {
  const int rope_units = (p.Hq + p.Hkv) * 8;  // per token: 8 units of 2x8 dims per rotated head
  const int units = rope_units + p.Hkv * 16;  // + 16 units of 8 dims per v head
  const int64_t total = (int64_t)p.n_tokens * units;
  for (int64_t idx = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; idx < total;
       idx += (int64_t)gridDim.x * blockDim.x) {
    const int tok = (int)(idx / units);
    const int u = (int)(idx % units);
    const uint16_t* row = p.qkv + (int64_t)tok * p.qkv_st;
    const int slot = p.slots[tok];
    const bool slot_ok = (unsigned)slot < (unsigned)p.num_slots;
    if (u < rope_units) {
      const int head = u >> 3;        // q heads first, then k heads
      const int d0 = (u & 7) * 8;     // dims d0..d0+7 and d0+64..d0+71
      const uint16_t* x = row + head * kHeadDim;
      const u32x4 lo = ld16(x + d0), hi = ld16(x + d0 + 64);
      const uint16_t* cs = p.cos + (int64_t)tok * p.cs_st;
      const uint16_t* sn = p.sin + (int64_t)tok * p.cs_st;
      const u32x4 clo = ld16(cs + d0), chi = ld16(cs + d0 + 64);
      const u32x4 slo = ld16(sn + d0), shi = ld16(sn + d0 + 64);
      u32x4 olo, ohi;
#pragma unroll
      for (int w = 0; w < 4; ++w) {
        uint32_t ol = 0, oh = 0;
#pragma unroll
        for (int h = 0; h < 2; ++h) {
          const int sh = 16 * h;
          const uint16_t xl = (uint16_t)(lo[w] >> sh), xh = (uint16_t)(hi[w] >> sh);
          const float a = Num<E>::f(xl), bv = Num<E>::f(xh);
          // d < 64: x[d]*cos[d] + (-x[d+64])*sin[d];  d >= 64: x[d]*cos[d] + x[d-64]*sin[d]
          const float t1l = rounded(Num<E>::f(Num<E>::r(a * Num<E>::f((uint16_t)(clo[w] >> sh)))));
          const float t2l = rounded(Num<E>::f(Num<E>::r(-bv * Num<E>::f((uint16_t)(slo[w] >> sh)))));
          const float t1h = rounded(Num<E>::f(Num<E>::r(bv * Num<E>::f((uint16_t)(chi[w] >> sh)))));
          const float t2h = rounded(Num<E>::f(Num<E>::r(a * Num<E>::f((uint16_t)(shi[w] >> sh)))));
          ol |= (uint32_t)Num<E>::r(t1l + t2l) << sh;
          oh |= (uint32_t)Num<E>::r(t1h + t2h) << sh;
        }
        olo[w] = ol;
        ohi[w] = oh;
      }
      if (head < p.Hq) {
        uint16_t* q = p.q_out + (int64_t)tok * p.q_st + head * kHeadDim;
        *reinterpret_cast<u32x4*>(q + d0) = olo;
        *reinterpret_cast<u32x4*>(q + d0 + 64) = ohi;
      } else if (slot_ok) {
        uint16_t* k = p.k_pool + (int64_t)slot * p.pool_st + (int64_t)(head - p.Hq) * p.pool_sh;
        *reinterpret_cast<u32x4*>(k + d0) = olo;
        *reinterpret_cast<u32x4*>(k + d0 + 64) = ohi;
      }
    } else if (slot_ok) {
      const int vu = u - rope_units;
      const int hv = vu >> 4, d0 = (vu & 15) * 8;
      const u32x4 val = ld16(row + (p.Hq + p.Hkv + hv) * kHeadDim + d0);
      uint16_t* v = p.v_pool + (int64_t)slot * p.pool_st + (int64_t)hv * p.pool_sh;
      *reinterpret_cast<u32x4*>(v + d0) = val;
    }
  }
}

hipError_t launch_rope_kv(const RopeParams& p, int dtype, hipStream_t stream) {
  const int64_t total = (int64_t)p.n_tokens * ((p.Hq + p.Hkv) * 8 + p.Hkv * 16);
  if (total == 0) return hipSuccess;
  const int blocks = (int)std::min<int64_t>((total + 255) / 256, 4096);
  if (dtype == 0)
    hipLaunchKernelGGL((rope_kv_kernel<BF16>), dim3(blocks), dim3(256), 0, stream, p);
  else
    hipLaunchKernelGGL((rope_kv_kernel<FP16>), dim3(blocks), dim3(256), 0, stream, p);
  return hipGetLastError();
}

}  // namespace mi_fa2
