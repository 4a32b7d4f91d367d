// fa_tiny.hip - short-sequence fp32 inference attention (D = 128, S <= 32).
//
// Same result as the reference's `_attention_tiny_forward`
// (fa_rdna3/kernels/tiny.py:9-85): for each query row, scores
// s_j = sum_d (q_d * scale * log2e) k_jd (+ bias_j * log2e), p = exp2(s - max)
// (all-masked rows give a zero output), out = sum_j p_j v_j / sum_j p_j.
//
// One wave per (query, head, batch).  Lane l holds dims 2l and 2l+1; each
// score is a butterfly sum over the 64 lanes, which keeps fp32 rounding close
// to a pairwise reduction (the accuracy target is 2e-6 absolute).
#include "fa_internal.hpp"
#include "fa_common.hpp"

namespace fa {

__global__ __launch_bounds__(64) void tiny_kernel(fa_tiny_params p) {
  const int qi = blockIdx.x, hh = blockIdx.y, bb = blockIdx.z;
  const int lane = threadIdx.x;
  const int S = p.seqlen;
  const float c = p.softmax_scale * kLog2e;
  const float* qr = p.q + bb * p.q_stride[0] + hh * p.q_stride[1] + qi * p.q_stride[2];
  const float q0 = qr[(2 * lane) * p.q_stride[3]] * c;
  const float q1 = qr[(2 * lane + 1) * p.q_stride[3]] * c;
  float sc[32];
  float mx = kNegInf;
#pragma unroll
  for (int j = 0; j < 32; ++j) {
    sc[j] = kNegInf;
    if (j < S) {
      const float* kr = p.k + bb * p.k_stride[0] + hh * p.k_stride[1] + j * p.k_stride[2];
      float s = q0 * kr[(2 * lane) * p.k_stride[3]] + q1 * kr[(2 * lane + 1) * p.k_stride[3]];
#pragma unroll
      for (int w = 32; w >= 1; w >>= 1) s += __shfl_xor(s, w, 64);
      if (p.bias)
        s += p.bias[bb * p.bias_stride[0] + hh * p.bias_stride[1] + qi * p.bias_stride[2] + j * p.bias_stride[3]] *
             kLog2e;
      sc[j] = s;
      mx = fmaxf(mx, s);
    }
  }
  const bool any = mx != kNegInf;
  const float ms = any ? mx : 0.f;
  float den = 0.f, a0 = 0.f, a1 = 0.f;
#pragma unroll
  for (int j = 0; j < 32; ++j) {
    if (j < S) {
      const float pj = any ? exp2f(sc[j] - ms) : 0.f;
      den += pj;
      const float* vr = p.v + bb * p.v_stride[0] + hh * p.v_stride[1] + j * p.v_stride[2];
      a0 += pj * vr[(2 * lane) * p.v_stride[3]];
      a1 += pj * vr[(2 * lane + 1) * p.v_stride[3]];
    }
  }
  const float inv = 1.f / (den == 0.f ? 1.f : den);
  float* orow = p.out + bb * p.out_stride[0] + hh * p.out_stride[1] + qi * p.out_stride[2];
  orow[(2 * lane) * p.out_stride[3]] = a0 * inv;
  orow[(2 * lane + 1) * p.out_stride[3]] = a1 * inv;
}

hipError_t launch_tiny(const fa_tiny_params& p, hipStream_t s) {
  dim3 grid(p.seqlen, p.heads, p.batch);
  hipLaunchKernelGGL(tiny_kernel, grid, dim3(64), 0, s, p);
  return hipGetLastError();
}

}  // namespace fa
