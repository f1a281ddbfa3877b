// RMSNorm prologue of the fused RMSNorm + int4 GEMM (rmsnorm_awq_fused_linear,
// vllm/kernels/triton/rmsnorm_awq_fused.py:43-189), and the fp16 -> bf16 output conversion
// that kernel's store performs for bf16 inputs.
//
// The reference recomputes each row's sum of squares inside every output tile (each of its
// N / 64 programs reads the row twice).  Here one block per row reduces the row once and
// writes the normalised fp16 row; the GEMM kernels then read it like any activation.
//
// Arithmetic of the reference (rmsnorm_awq_fused.py:108-131), step for step:
//   var  = sum over k of fp32(x)^2       (fp32 in the reference, in 32-element chunks; here the
//                                         exact squares are added in fp64 and rounded once to
//                                         fp32, which makes the order of the adds invisible)
//   rrms = rsqrt(var / K + eps)          (var / K + eps in fp32; the rsqrt correctly rounded)
//   xn   = fp16_rne((fp32(x) * rrms) * fp32(norm_w))     (two fp32 products, one rounding)
#include "awq_common.h"
#include "awq_launch.h"

namespace awq {

constexpr int kNormThreads = 256;

template <typename T, typename NT>
__global__ void __launch_bounds__(kNormThreads) rmsnorm_rows_kernel(const uint16_t* __restrict__ x, int64_t ldx,
                                                                    const uint16_t* __restrict__ nw, float eps,
                                                                    uint16_t* __restrict__ xn, int64_t ldo, int K) {
  __shared__ double part[kNormThreads / 64];
  const uint16_t* row = x + (int64_t)blockIdx.x * ldx;
  const int t = threadIdx.x;
  // pass 1: sum of squares, 8 elements (16 bytes) per lane and step; the squares are exact
  // in fp64 and the fp64 sum is within about K * 2^-53 of the exact one, so rounding it once to
  // fp32 gives the correctly rounded var (whatever the order of the adds) unless the exact sum
  // lies that close to an fp32 rounding boundary
  double ss = 0.0;
  for (int k = t * 8; k < K; k += kNormThreads * 8) {
    const u32x4 v = *(const u32x4*)(row + k);
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const double lo = from_bits<T>((uint16_t)(v[j] & 0xFFFF)), hi = from_bits<T>((uint16_t)(v[j] >> 16));
      ss += lo * lo;
      ss += hi * hi;
    }
  }
  ss = wave_sum_f64(ss);
  if ((t & 63) == 0) part[t >> 6] = ss;
  __syncthreads();
  double var = 0.0;
#pragma unroll
  for (int w = 0; w < kNormThreads / 64; ++w) var += part[w];  // same order in every lane
  const float rrms = rms_scale((float)var, K, eps);
  // pass 2: the row again (cache-resident), scaled and rounded once to fp16
  uint16_t* orow = xn + (int64_t)blockIdx.x * ldo;
  for (int k = t * 8; k < K; k += kNormThreads * 8) {
    const u32x4 v = *(const u32x4*)(row + k);
    const u32x4 g = *(const u32x4*)(nw + k);
    u32x4 r;
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const float lo = fp32_rounded((from_bits<T>((uint16_t)(v[j] & 0xFFFF)) * rrms) * from_bits<NT>((uint16_t)(g[j] & 0xFFFF)));
      const float hi = fp32_rounded((from_bits<T>((uint16_t)(v[j] >> 16)) * rrms) * from_bits<NT>((uint16_t)(g[j] >> 16)));
      r[j] = (uint32_t)f2h_bits(lo) | ((uint32_t)f2h_bits(hi) << 16);
    }
    *(u32x4*)(orow + k) = r;
  }
}

// fp16 -> bf16, round to nearest even, 8 elements per lane (the reference stores its fp16
// result into a bf16 output tensor for bf16 inputs, rmsnorm_awq_fused.py:170-175).
__global__ void __launch_bounds__(256) f16_to_bf16_kernel(const uint16_t* __restrict__ in, int64_t ldi,
                                                          uint16_t* __restrict__ out, int64_t ldo, int64_t N) {
  const int64_t c = ((int64_t)blockIdx.x * 256 + threadIdx.x) * 8;
  if (c >= N) return;
  const u32x4 v = *(const u32x4*)(in + (int64_t)blockIdx.y * ldi + c);
  u32x4 r;
#pragma unroll
  for (int j = 0; j < 4; ++j)
    r[j] = (uint32_t)f2bf_bits(h_bits2f((uint16_t)(v[j] & 0xFFFF))) |
           ((uint32_t)f2bf_bits(h_bits2f((uint16_t)(v[j] >> 16))) << 16);
  *(u32x4*)(out + (int64_t)blockIdx.y * ldo + c) = r;
}

}  // namespace awq

namespace awq_host {
using namespace awq;

int launch_rmsnorm_rows(const void* x, int64_t ldx, const void* nw, float eps, void* xn, int64_t ldo, int64_t M,
                        int64_t K, int act, int ndt, hipStream_t st) {
  if (M <= 0) return AWQ_OK;
  if (M > 0x7FFFFFFFLL) return AWQ_ERR_UNSUPPORTED;
  const dim3 grid((unsigned)M);
  const auto* xs = (const uint16_t*)x;
  const auto* ns = (const uint16_t*)nw;
  auto* o = (uint16_t*)xn;
  const bool xb = act == AWQ_DTYPE_BF16, nb = ndt == AWQ_DTYPE_BF16;
  if (!xb && !nb) rmsnorm_rows_kernel<f16, f16><<<grid, kNormThreads, 0, st>>>(xs, ldx, ns, eps, o, ldo, (int)K);
  else if (!xb && nb) rmsnorm_rows_kernel<f16, bf16><<<grid, kNormThreads, 0, st>>>(xs, ldx, ns, eps, o, ldo, (int)K);
  else if (xb && !nb) rmsnorm_rows_kernel<bf16, f16><<<grid, kNormThreads, 0, st>>>(xs, ldx, ns, eps, o, ldo, (int)K);
  else rmsnorm_rows_kernel<bf16, bf16><<<grid, kNormThreads, 0, st>>>(xs, ldx, ns, eps, o, ldo, (int)K);
  return hipGetLastError() == hipSuccess ? AWQ_OK : AWQ_ERR_LAUNCH;
}

int launch_f16_to_bf16(const void* in, int64_t ldi, void* out, int64_t ldo, int64_t M, int64_t N, hipStream_t st) {
  if (M <= 0 || N <= 0) return AWQ_OK;
  if (M > 65535) return AWQ_ERR_UNSUPPORTED;
  const dim3 grid((unsigned)cdiv(N, 256 * 8), (unsigned)M);
  f16_to_bf16_kernel<<<grid, 256, 0, st>>>((const uint16_t*)in, ldi, (uint16_t*)out, ldo, N);
  return hipGetLastError() == hipSuccess ? AWQ_OK : AWQ_ERR_LAUNCH;
}

}  // namespace awq_host
