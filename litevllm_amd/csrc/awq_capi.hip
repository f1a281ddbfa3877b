// extern "C" entry points of libawq_w4a16.so (declared in include/awq_w4a16.h): argument
// validation, planning and dispatch to the kernels of the other translation units.
// No function throws, allocates device memory or leaves a pending HIP error behind.
#include <mutex>

#include "awq_common.h"
#include "awq_launch.h"

namespace awq_host {
using namespace awq;

static int g_num_cus = 0;
static std::once_flag g_cu_once;

int num_cus() {
  std::call_once(g_cu_once, [] {
    int dev = 0, n = 0;
    if (hipGetDevice(&dev) == hipSuccess &&
        hipDeviceGetAttribute(&n, hipDeviceAttributeMultiprocessorCount, dev) == hipSuccess && n > 0)
      g_num_cus = n;
    else
      g_num_cus = 256;
  });
  return g_num_cus;
}

static int launch_status() {
  const hipError_t e = hipGetLastError();
  return e == hipSuccess ? AWQ_OK : AWQ_ERR_LAUNCH;
}

static bool dtype_16(int d) { return d == AWQ_DTYPE_F16 || d == AWQ_DTYPE_BF16; }

// The decode kernel's group-aligned ring covers group sizes 32, 64 and 128.
static bool decode_covers(int64_t M, int64_t G) {
  return M <= 32 && (G == 32 || G == 64 || G == 128);
}

}  // namespace awq_host

using namespace awq_host;

extern "C" {

int awq_w4a16_version(void) { return 200; }

const char* awq_w4a16_strerror(int code) {
  switch (code) {
    case AWQ_OK: return "ok";
    case AWQ_ERR_NULL: return "a required pointer is NULL";
    case AWQ_ERR_SHAPE: return "inconsistent sizes (need N % 8 == 0, K % group_size == 0, group_size % 32 == 0 for GEMM, % 8 for dequant)";
    case AWQ_ERR_UNSUPPORTED: return "unsupported dtype/layout/shape combination";
    case AWQ_ERR_WORKSPACE: return "workspace missing or too small";
    case AWQ_ERR_LAUNCH: return "HIP kernel launch failed";
    case AWQ_ERR_STRIDE: return "leading dimension smaller than the row length or misaligned";
    default: return "unknown error";
  }
}

int awq_w4a16_dequant(const int32_t* qweight, const void* scales, const int32_t* qzeros, void* out,
                      int64_t rows, int64_t cols, int32_t group_size, int32_t layout,
                      int32_t scale_dtype, int32_t out_dtype, void* stream) {
  return launch_dequant(qweight, scales, qzeros, out, rows, cols, group_size, layout, scale_dtype,
                        out_dtype, (hipStream_t)stream);
}

size_t awq_w4a16_gemm_workspace_bytes(int64_t M, int64_t N, int64_t K, int32_t group_size,
                                      int32_t split_k, int32_t layout) {
  if (M <= 0 || N <= 0 || K <= 0 || (N % 8) != 0 || split_k < 0) return 0;
  if (group_size <= 0 || (K % group_size) != 0 || !decode_covers(M, group_size)) return 0;
  // the plan also depends on the dtype path: size for the largest
  size_t ws = 0;
  for (DecodeMode m : {kDecodeStream, kDecodeWide, kDecodeNarrow}) {
    if (m == kDecodeStream && layout != AWQ_LAYOUT_DECODE_STREAM) continue;
    if (m != kDecodeStream && layout == AWQ_LAYOUT_DECODE_STREAM) continue;
    const size_t b = plan_decode(M, N, K, group_size, split_k, m).ws_bytes;
    ws = b > ws ? b : ws;
  }
  return ws;
}

int awq_w4a16_gemm(const void* a, int64_t lda, const int32_t* qweight, const void* scales,
                   const int32_t* qzeros, const void* bias, void* c, int64_t ldc, int64_t M,
                   int64_t N, int64_t K, int32_t group_size, int32_t split_k, int32_t layout,
                   int32_t act_dtype, int32_t scale_dtype, int32_t bias_dtype, void* workspace,
                   size_t workspace_bytes, void* stream) {
  if (!a || !qweight || !scales || !c) return AWQ_ERR_NULL;
  if (bias && bias_dtype == AWQ_DTYPE_NONE) return AWQ_ERR_UNSUPPORTED;
  if (!dtype_16(act_dtype) || !dtype_16(scale_dtype)) return AWQ_ERR_UNSUPPORTED;
  if (bias && bias_dtype != AWQ_DTYPE_F16 && bias_dtype != AWQ_DTYPE_BF16 && bias_dtype != AWQ_DTYPE_F32)
    return AWQ_ERR_UNSUPPORTED;
  if (M < 0 || N < 0 || K <= 0 || group_size <= 0) return AWQ_ERR_SHAPE;
  if ((N % 8) != 0 || (group_size % 32) != 0 || (K % group_size) != 0) return AWQ_ERR_SHAPE;
  if (split_k < 0) return AWQ_ERR_SHAPE;
  if (M == 0 || N == 0) return AWQ_OK;
  if (lda < K || ldc < N || (lda % 8) != 0 || (ldc % 8) != 0) return AWQ_ERR_STRIDE;
  if ((((uintptr_t)a) & 15) || (((uintptr_t)c) & 15) || (((uintptr_t)scales) & 15) ||
      (((uintptr_t)qweight) & 15))
    return AWQ_ERR_STRIDE;
  if (layout != AWQ_LAYOUT_AUTOAWQ && layout != AWQ_LAYOUT_KN_SEQ && layout != AWQ_LAYOUT_DECODE_STREAM)
    return AWQ_ERR_UNSUPPORTED;
  const bool stream_layout = layout == AWQ_LAYOUT_DECODE_STREAM;
  if (stream_layout && !decode_covers(M, group_size)) return AWQ_ERR_UNSUPPORTED;
  // 32-bit buffer offsets: weights, activations and the output must stay below 2 GiB
  if (decode_stream_bytes(K, N) > 0x7FFFFFFFLL || M * lda * 2 > 0x7FFFFFFFLL) return AWQ_ERR_UNSUPPORTED;
  hipStream_t st = (hipStream_t)stream;

  GemmArgs ga{};
  ga.a = (const uint16_t*)a;
  ga.qw = (const uint32_t*)qweight;
  ga.sc = (const uint16_t*)scales;
  ga.qz = (const uint32_t*)qzeros;
  ga.bias = bias;
  ga.c = (uint16_t*)c;
  ga.lda = lda;
  ga.ldc = ldc;
  ga.M = (int)M;
  ga.N = (int)N;
  ga.K = (int)K;
  ga.G = group_size;
  ga.bias_dtype = bias ? bias_dtype : AWQ_DTYPE_NONE;
  const bool seq = layout == AWQ_LAYOUT_KN_SEQ;
  const bool zp = qzeros != nullptr;

  if (decode_covers(M, group_size)) {
    const DecodeMode mode = decode_mode(layout, act_dtype, scale_dtype);
    const DecodePlan sp = plan_decode(M, N, K, group_size, split_k, mode);
    if (sp.ws_bytes) {
      if (!workspace || workspace_bytes < sp.ws_bytes) return AWQ_ERR_WORKSPACE;
      if ((size_t)sp.tiles * sizeof(int) > kCounterBytes) return AWQ_ERR_UNSUPPORTED;
      if (sp.ws_bytes - kCounterBytes > 0x7FFFFFFFu) return AWQ_ERR_UNSUPPORTED;  // 32-bit offsets
      ga.counters = (int*)workspace;
      ga.partial = (float*)((char*)workspace + kCounterBytes);
    }
    if (!launch_decode(ga, sp, mode, seq, zp, act_dtype, scale_dtype, st)) return AWQ_ERR_UNSUPPORTED;
    return launch_status();
  }
  if ((K % 64) != 0) return AWQ_ERR_SHAPE;
  if (!launch_prefill(ga, seq, zp, act_dtype, scale_dtype, st)) return AWQ_ERR_UNSUPPORTED;
  return launch_status();
}

int awq_w4a16_repack_nk_to_autoawq(const int32_t* qweight_nk, const int32_t* qzeros_nk,
                                   const void* scales_nk, int32_t* qweight_kn, int32_t* qzeros_kn,
                                   void* scales_kn, int64_t N, int64_t K, int32_t group_size,
                                   void* stream) {
  return launch_repack_nk_to_autoawq(qweight_nk, qzeros_nk, scales_nk, qweight_kn, qzeros_kn,
                                     scales_kn, N, K, group_size, (hipStream_t)stream);
}

int64_t awq_w4a16_decode_stream_bytes(int64_t K, int64_t N) {
  if (K <= 0 || N <= 0 || (N % 8) != 0 || (K % 32) != 0) return 0;
  return decode_stream_bytes(K, N);
}

int awq_w4a16_pack_decode_stream(const int32_t* qweight_kn, int32_t* out, int64_t K, int64_t N,
                                 void* stream) {
  if (!qweight_kn || !out) return AWQ_ERR_NULL;
  if (K < 0 || N < 0 || (N % 8) != 0 || (K % 32) != 0) return AWQ_ERR_SHAPE;
  if (decode_stream_bytes(K, N) > 0x7FFFFFFFLL) return AWQ_ERR_UNSUPPORTED;
  return launch_pack_decode_stream(qweight_kn, out, K, N, decode_stream_wpl(N), (hipStream_t)stream);
}

}  // extern "C"
