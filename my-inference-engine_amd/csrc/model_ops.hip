// The elementwise steps around the attention path in a decode / prefill step, fused.
//
// The reference model runs each of these as a chain of PyTorch ops, one launch each:
//   RMSNorm (model.py:49-55): x.float(), pow, mean, + eps, rsqrt, multiply, .to(bf16), * weight;
//   the residual adds (model.py:128-138): x + attn, x + mlp;
//   SwiGLU (model.py:112-120): silu(gate) * up.
// At decode sizes (16 rows of 1536) every launch is a few microseconds of fixed cost, about 20 per
// layer.  Two kernels replace them, with the reference's rounding points kept (each torch op
// rounds its result to the tensor dtype):
//   add_rmsnorm:  r = round(x + y)            (skipped when y is NULL: r = x)
//                 n = round(float(r) * rsqrt(mean(float(r)^2) + eps))
//                 out = round(weight * n)
//                 writing r (the new residual stream) and out (the normalised rows);
//   silu_mul:     out = round(round(g / (1 + exp(-g))) * u) for gate g and up u of each row.
// fp32 arithmetic between the rounding points, as the torch kernels do; the only differences left
// are the order of the mean's sum and the rsqrt / exp implementations (last-bit effects).
#include "fa2_common.h"

namespace mi_fa2 {

template <typename E>
__device__ __forceinline__ float to_f(uint16_t x);
template <>
__device__ __forceinline__ float to_f<BF16>(uint16_t x) { return __uint_as_float((uint32_t)x << 16); }
template <>
__device__ __forceinline__ float to_f<FP16>(uint16_t x) {
  return (float)__builtin_bit_cast(_Float16, x);
}
template <typename E>
__device__ __forceinline__ uint16_t from_f(float x) {
  return (uint16_t)(E::pack2(x, 0.f) & 0xffffu);
}

constexpr int kNormThreads = 256;

// One work-group per row; each thread owns 8-element chunks c = tid, tid + 256, ...
template <typename E>
__global__ __launch_bounds__(kNormThreads) void add_rmsnorm_kernel(const ModelOpParams p) {
  const int row = blockIdx.x, tid = threadIdx.x;
  const int chunks = p.hidden / 8;
  const uint16_t* x = p.x + (int64_t)row * p.x_st;
  const uint16_t* y = p.y ? p.y + (int64_t)row * p.y_st : nullptr;
  uint16_t* r_out = p.r_out ? p.r_out + (int64_t)row * p.r_st : nullptr;
  uint16_t* out = p.out + (int64_t)row * p.out_st;
  constexpr int kMaxPer = 4;   // hidden <= 8 * 256 * 4 = 8192
  u32x4 rv[kMaxPer];
  float ss = 0.f;
#pragma unroll
  for (int k = 0; k < kMaxPer; ++k) {
    const int c = tid + k * kNormThreads;
    if (c >= chunks) break;
    u32x4 a = *reinterpret_cast<const u32x4*>(x + 8 * c);
    if (y) {
      const u32x4 b = *reinterpret_cast<const u32x4*>(y + 8 * c);
#pragma unroll
      for (int w = 0; w < 4; ++w) {
        const float lo = to_f<E>(a[w] & 0xffffu) + to_f<E>(b[w] & 0xffffu);
        const float hi = to_f<E>(a[w] >> 16) + to_f<E>(b[w] >> 16);
        a[w] = (uint32_t)from_f<E>(lo) | ((uint32_t)from_f<E>(hi) << 16);
      }
      if (r_out) *reinterpret_cast<u32x4*>(r_out + 8 * c) = a;
    }
    rv[k] = a;
#pragma unroll
    for (int w = 0; w < 4; ++w) {
      const float lo = to_f<E>(a[w] & 0xffffu), hi = to_f<E>(a[w] >> 16);
      ss = __builtin_fmaf(lo, lo, ss);
      ss = __builtin_fmaf(hi, hi, ss);
    }
  }
  // work-group sum of squares
#pragma unroll
  for (int d = 32; d >= 1; d >>= 1) ss += __shfl_xor(ss, d);
  __shared__ float part[kNormThreads / 64];
  if ((tid & 63) == 0) part[tid >> 6] = ss;
  __syncthreads();
  float tot = 0.f;
#pragma unroll
  for (int w = 0; w < kNormThreads / 64; ++w) tot += part[w];
  const float inv = rsqrtf(tot / (float)p.hidden + p.eps);
#pragma unroll
  for (int k = 0; k < kMaxPer; ++k) {
    const int c = tid + k * kNormThreads;
    if (c >= chunks) break;
    const u32x4 wv = *reinterpret_cast<const u32x4*>(p.weight + 8 * c);
    u32x4 o;
#pragma unroll
    for (int w = 0; w < 4; ++w) {
      const float n_lo = to_f<E>(from_f<E>(to_f<E>(rv[k][w] & 0xffffu) * inv));
      const float n_hi = to_f<E>(from_f<E>(to_f<E>(rv[k][w] >> 16) * inv));
      o[w] = (uint32_t)from_f<E>(to_f<E>(wv[w] & 0xffffu) * n_lo) |
             ((uint32_t)from_f<E>(to_f<E>(wv[w] >> 16) * n_hi) << 16);
    }
    *reinterpret_cast<u32x4*>(out + 8 * c) = o;
  }
}

// One thread per 8 output elements; grid-stride over rows x inter / 8.
template <typename E>
__global__ __launch_bounds__(256) void silu_mul_kernel(const ModelOpParams p) {
  const int per_row = p.hidden / 8;   // hidden = intermediate size here
  const int64_t total = (int64_t)p.rows * per_row;
  for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < total;
       i += (int64_t)gridDim.x * blockDim.x) {
    const int row = (int)(i / per_row), c = (int)(i % per_row);
    const uint16_t* g = p.x + (int64_t)row * p.x_st + 8 * c;
    const u32x4 gv = *reinterpret_cast<const u32x4*>(g);
    const u32x4 uv = *reinterpret_cast<const u32x4*>(g + p.hidden);
    u32x4 o;
#pragma unroll
    for (int w = 0; w < 4; ++w) {
      float a[2] = {to_f<E>(gv[w] & 0xffffu), to_f<E>(gv[w] >> 16)};
      float u[2] = {to_f<E>(uv[w] & 0xffffu), to_f<E>(uv[w] >> 16)};
      uint32_t r = 0;
#pragma unroll
      for (int h = 0; h < 2; ++h) {
        const float s = to_f<E>(from_f<E>(a[h] / (1.f + expf(-a[h]))));
        r |= (uint32_t)from_f<E>(s * u[h]) << (16 * h);
      }
      o[w] = r;
    }
    *reinterpret_cast<u32x4*>(p.out + (int64_t)row * p.out_st + 8 * c) = o;
  }
}

hipError_t launch_add_rmsnorm(const ModelOpParams& p, int dtype, hipStream_t stream) {
  if (dtype == 0)
    hipLaunchKernelGGL((add_rmsnorm_kernel<BF16>), dim3(p.rows), dim3(kNormThreads), 0, stream, p);
  else
    hipLaunchKernelGGL((add_rmsnorm_kernel<FP16>), dim3(p.rows), dim3(kNormThreads), 0, stream, p);
  return hipGetLastError();
}

hipError_t launch_silu_mul(const ModelOpParams& p, int dtype, hipStream_t stream) {
  const int64_t total = (int64_t)p.rows * (p.hidden / 8);
  const int blocks = (int)std::min<int64_t>((total + 255) / 256, 8192);
  if (dtype == 0)
    hipLaunchKernelGGL((silu_mul_kernel<BF16>), dim3(blocks), dim3(256), 0, stream, p);
  else
    hipLaunchKernelGGL((silu_mul_kernel<FP16>), dim3(blocks), dim3(256), 0, stream, p);
  return hipGetLastError();
}

}  // namespace mi_fa2
