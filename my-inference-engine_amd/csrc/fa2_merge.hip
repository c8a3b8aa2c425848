// Log-sum-exp merge of attention partials computed over disjoint key ranges (mi_fa2_combine).
//
// Each partial is what the forward computes over a sub-range of a row's keys: its normalised
// output O_i and its log-sum-exp L_i (natural log; kernels/fa2.py:155-158 writes the same pair).
// Over the union of the ranges
//   L = log sum_i exp(L_i),   O = sum_i exp(L_i - L) O_i,
// which is what one pass over all the keys gives.  A partial with L_i = -inf saw no key and adds
// nothing; a (row, head) with no partial that saw a key gets O = 0 and L = -inf, like the forward.
//
// One wave per (row, head): lane l owns dimensions 2l, 2l+1 (8-byte loads of the fp32 partials).
// The row's L_i are read by every lane (the same few words: a broadcast), the maximum first, then
// one pass accumulates with exp2 of log2-scaled differences.
#include "fa2_common.h"

namespace mi_fa2 {

template <int OUT>  // 0 bf16, 1 fp16, 2 fp32
__global__ __launch_bounds__(64) void fa2_merge_kernel(const MergeParams p) {
  const int h = blockIdx.x;
  const int r = blockIdx.y;
  const int lane = threadIdx.x;
  int n = p.n_parts ? p.n_parts[r] : p.max_parts;
  n = n < 0 ? 0 : (n > p.max_parts ? p.max_parts : n);
  const float* lp = p.part_lse + (int64_t)r * p.pl_sr + (int64_t)h * p.pl_sh;
  const float* op = p.part_o + (int64_t)r * p.po_sr + (int64_t)h * p.po_sh + 2 * lane;

  float M = -INFINITY;
  for (int i = 0; i < n; ++i) M = fmaxf(M, lp[(int64_t)i * p.pl_sp]);
  float acc0 = 0.f, acc1 = 0.f, L = 0.f;
  if (M != -INFINITY) {
    const float Ml = M * kLog2e;
    for (int i = 0; i < n; ++i) {
      const float li = lp[(int64_t)i * p.pl_sp];
      if (li == -INFINITY) continue;  // saw no key: its O is not read
      const float w = exp2_fast(li * kLog2e - Ml);
      const float2 o = *reinterpret_cast<const float2*>(op + (int64_t)i * p.po_sp);
      acc0 += w * o.x;
      acc1 += w * o.y;
      L += w;
    }
  }
  const float inv = L > 0.f ? 1.f / L : 0.f;
  const float o0 = acc0 * inv, o1 = acc1 * inv;
  const int64_t oo = (int64_t)r * p.o_sr + (int64_t)h * p.o_sh + 2 * lane;
  if constexpr (OUT == 2) {
    *reinterpret_cast<float2*>(static_cast<float*>(p.o) + oo) = float2{o0, o1};
  } else if constexpr (OUT == 1) {
    *reinterpret_cast<uint32_t*>(static_cast<uint16_t*>(p.o) + oo) = FP16::pack2(o0, o1);
  } else {
    *reinterpret_cast<uint32_t*>(static_cast<uint16_t*>(p.o) + oo) = BF16::pack2(o0, o1);
  }
  if (p.lse && lane == 0)
    p.lse[(int64_t)r * p.l_sr + (int64_t)h * p.l_sh] =
        L > 0.f ? M + __builtin_logf(L) : -INFINITY;
}

hipError_t launch_merge(const MergeParams& p, int out_dtype, hipStream_t stream) {
  if (p.rows == 0 || p.heads == 0) return hipSuccess;
  const dim3 grid(p.heads, p.rows);
  if (out_dtype == 2)
    hipLaunchKernelGGL(fa2_merge_kernel<2>, grid, dim3(64), 0, stream, p);
  else if (out_dtype == 1)
    hipLaunchKernelGGL(fa2_merge_kernel<1>, grid, dim3(64), 0, stream, p);
  else
    hipLaunchKernelGGL(fa2_merge_kernel<0>, grid, dim3(64), 0, stream, p);
  return hipGetLastError();
}

}  // namespace mi_fa2
