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

// Calls of 33 .. 64 rows run as 32-row chunks on the decode kernels, one launch each: the
// prefill kernel's one 256-row tile per column tile keeps most CUs idle there, each tile's K
// loop taking about 58 us at K = 4096 (measured on MI355X, K = 4096, graph replays: M = 48 / 64
// at N = 4096 57.6 / 57.7 us against 19.5 / 24.1 us in chunks; M = 64 at N = 12288 / 24576
// 60.6 / 62.5 against 32.9 / 38.0 us).  Above 64 rows the prefill kernel's K ranges (below)
// are ahead of more chunks (M = 128, N = 4096: 26-27 us against 47.5 us in four chunks).
static bool decode_chunks(int64_t M, int64_t N, int64_t G) {
  (void)N;
  return M > 32 && M <= 64 && decode_covers(32, G);
}

// K ranges of the prefill stream kernel (split_k = 0, stream layout): where its 256 x 256 tiles
// cover at most a third of the CUs, each tile's K loop is cut into 3 .. 8 ranges of whole stage
// pairs (fp32 partials, summed in range order by a second launch), so that tiles x ranges
// comes near one block per CU.  1 = no split.  Measured on MI355X (K = 4096, graph replays,
// whole K against ranges): M = 128 .. 384 at N = 2048 .. 8192 57-64 us against 26-51 us
// (M = 256, N = 4096: 57.9 against 26.8 us); two ranges lost (M = 384 / 512 at N = 12288 and
// M = 2048 at N = 4096: 2-12% slower), so three is the least.
static int prefill_splits(int64_t M, int64_t N, int64_t K, int64_t G, int32_t split_k, int32_t layout) {
  if (split_k != 0 || layout != AWQ_LAYOUT_DECODE_STREAM || M <= 32 || decode_chunks(M, N, G)) return 1;
  if (G <= 0 || (G & (G - 1)) != 0 || (K % 32) != 0 || (N % 8) != 0) return 1;
  const int64_t tiles = ((M + 255) / 256) * ((N + 255) / 256);
  const int64_t nst = (K + 63) / 64;
  const int64_t cus = num_cus();
  if (tiles * 3 > cus || nst < 12) return 1;
  int64_t S = cus / tiles;
  // 32 .. 63 tiles: three quarters of that (the partials' round trip grows with the ranges;
  // M = 256 .. 512 at 32 tiles: six ranges 5-7% ahead of eight, M = 192 / 256 at 48 tiles four
  // 2-4% ahead of five; measured on MI355X)
  if (tiles >= 32 && tiles < 64) S = S * 3 / 4;
  S = S > 8 ? 8 : S;
  S = S > nst / 4 ? nst / 4 : S;  // ranges of at least four stages
  return S < 3 ? 1 : (int)S;
}
// The partials go after the decode kernels' counter region, which a workspace shared between
// calls keeps zero.
static size_t prefill_split_bytes(int64_t M, int64_t N, int64_t K, int64_t G, int32_t split_k, int32_t layout) {
  const int S = prefill_splits(M, N, K, G, split_k, layout);
  return S > 1 ? kCounterBytes + (size_t)S * (size_t)M * (size_t)N * sizeof(float) : 0;
}

}  // namespace awq_host

// ---- scratch of the allocation-free GEMM ------------------------------------------------
// awq_w4a16_gemm_noalloc keeps the split-K arrival counters and fp32 partials that
// awq_w4a16_gemm takes through `workspace` in this file-scope device array instead: one copy
// per GPU, held until the process ends, laid out like a workspace (counters first).  Host
// code never passes the array's name to a kernel or a copy (on the host it only stands in for
// the symbol): each device's address comes from hipGetSymbolAddress, taken once per device
// with that device current, and only that address is used.
constexpr size_t kNoallocScratchBytes = awq_host::kCounterBytes + ((size_t)8 << 20);
static __device__ __align__(256) unsigned char scratch[kNoallocScratchBytes];

namespace awq_host {

constexpr int kMaxDevices = 64;
static void* g_scratch_ptr[kMaxDevices];
static int g_scratch_rc[kMaxDevices];
static std::once_flag g_scratch_once[kMaxDevices];

// Zeroes n 32-bit words (a kernel, not hipMemsetAsync, so a caller may capture it in a graph).
__global__ void __launch_bounds__(256) zero_words_kernel(uint32_t* p, int n) {
  const int i = (int)(blockIdx.x * 256 + threadIdx.x);
  if (i < n) p[i] = 0u;
}

// The current device's scratch address: looked up once per device, when the counter region is
// also cleared on `st` (the kernels leave it zero after every call).
static int noalloc_scratch(void** out, hipStream_t st) {
  int dev = -1;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= kMaxDevices) {
    (void)hipGetLastError();
    return AWQ_ERR_LAUNCH;
  }
  std::call_once(g_scratch_once[dev], [dev, st] {
    void* p = nullptr;
    if (hipGetSymbolAddress(&p, HIP_SYMBOL(scratch)) != hipSuccess || p == nullptr) {
      (void)hipGetLastError();
      g_scratch_rc[dev] = AWQ_ERR_LAUNCH;
      return;
    }
    const int words = (int)(kCounterBytes / 4);
    hipLaunchKernelGGL(zero_words_kernel, dim3((unsigned)cdiv(words, 256)), dim3(256), 0, st, (uint32_t*)p, words);
    if (hipGetLastError() != hipSuccess) {
      g_scratch_rc[dev] = AWQ_ERR_LAUNCH;
      return;
    }
    g_scratch_ptr[dev] = p;
    g_scratch_rc[dev] = AWQ_OK;
  });
  if (g_scratch_rc[dev] != AWQ_OK) return g_scratch_rc[dev];
  *out = g_scratch_ptr[dev];
  return AWQ_OK;
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

// The decode kernels' workspace (split-K counters and partials) alone: what the allocation-free
// entry point provides; the prefill kernel's K ranges run only where the caller's workspace
// holds them.
static size_t decode_workspace_bytes(int64_t M, int64_t N, int64_t K, int32_t group_size, int32_t split_k,
                                     int32_t layout) {
  if (M <= 0 || N <= 0 || K <= 0 || (N % 8) != 0 || split_k < 0) return 0;
  if (decode_chunks(M, N, group_size)) M = 32;  // the chunks run one after another
  if (group_size <= 0 || (K % group_size) != 0 || !decode_covers(M, group_size)) return 0;
  if (layout == AWQ_LAYOUT_DECODE_NARROW) return 0;  // the narrow kernel does not split K
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

size_t awq_w4a16_gemm_workspace_bytes(int64_t M, int64_t N, int64_t K, int32_t group_size,
                                      int32_t split_k, int32_t layout) {
  if (M <= 0 || N <= 0 || K <= 0 || (N % 8) != 0 || split_k < 0) return 0;
  const size_t pre = (group_size > 0 && (K % group_size) == 0) ? prefill_split_bytes(M, N, K, group_size, split_k, layout) : 0;
  const size_t dec = decode_workspace_bytes(M, N, K, group_size, split_k, layout);
  return pre > dec ? pre : dec;
}

}  // extern "C"

// The body of awq_w4a16_gemm.  rows > 1 (M == 1): a row-exact launch of the decode kernels, grid
// row y computing row y (activation row a + y lda, output row c + y ldc) exactly as a lone M = 1
// call does, with split-K counters and partials of its own.
static int gemm_impl(const void* a, int64_t lda, const int32_t* qweight, const void* scales, const int32_t* qzeros,
                     const void* bias, void* c, int64_t ldc, int64_t M, int64_t N, int64_t K, int32_t group_size,
                     int32_t split_k, int32_t layout, int32_t act_dtype, int32_t scale_dtype, int32_t bias_dtype,
                     void* workspace, size_t workspace_bytes, void* stream, int64_t rows) {
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
  if (rows > 1 && (M != 1 || !decode_covers(1, group_size))) return AWQ_ERR_UNSUPPORTED;
  if ((((uintptr_t)a) & 15) || (((uintptr_t)c) & 15) || (((uintptr_t)scales) & 15) ||
      (((uintptr_t)qweight) & 15))
    return AWQ_ERR_STRIDE;
  if (layout != AWQ_LAYOUT_AUTOAWQ && layout != AWQ_LAYOUT_KN_SEQ && layout != AWQ_LAYOUT_DECODE_STREAM &&
      layout != AWQ_LAYOUT_DECODE_NARROW)
    return AWQ_ERR_UNSUPPORTED;
  if (layout == AWQ_LAYOUT_DECODE_NARROW && !decode_covers(M, group_size)) return AWQ_ERR_UNSUPPORTED;
  if ((layout == AWQ_LAYOUT_DECODE_NARROW || layout == AWQ_LAYOUT_DECODE_STREAM) && (K % 32) != 0)
    return AWQ_ERR_UNSUPPORTED;
  // 32-bit buffer offsets: weights, activations and the output must stay below 2 GiB
  if (decode_stream_bytes(K, N) > 0x7FFFFFFFLL || M * lda * 2 > 0x7FFFFFFFLL) return AWQ_ERR_UNSUPPORTED;
  if (rows > 0x7FFF) return AWQ_ERR_UNSUPPORTED;  // grid rows
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
  ga.rows = rows > 1 ? (int)rows : 0;
  const bool seq = layout == AWQ_LAYOUT_KN_SEQ;
  const bool zp = qzeros != nullptr;

  if (layout == AWQ_LAYOUT_DECODE_NARROW) {  // whole K per block: no workspace
    if (!launch_decode_narrow(ga, zp, act_dtype, scale_dtype, st)) return AWQ_ERR_UNSUPPORTED;
    return launch_status();
  }
  if (decode_covers(M, group_size)) {
    const DecodeMode mode = decode_mode(layout, act_dtype, scale_dtype);
    const DecodePlan sp = plan_decode(M, N, K, group_size, split_k, mode);
    if (sp.ws_bytes) {
      // a row-exact launch holds `rows` sets of counters and partials, one per grid row
      const size_t nrow = rows > 1 ? (size_t)rows : 1;
      if (!workspace || workspace_bytes < kCounterBytes + nrow * (sp.ws_bytes - kCounterBytes)) return AWQ_ERR_WORKSPACE;
      if (nrow * (size_t)sp.tiles * sizeof(int) > kCounterBytes) return AWQ_ERR_UNSUPPORTED;
      if (sp.ws_bytes - kCounterBytes > 0x7FFFFFFFu) return AWQ_ERR_UNSUPPORTED;  // 32-bit offsets
      ga.counters = (int*)workspace;
      ga.partial = (float*)((char*)workspace + kCounterBytes);
    }
    if (!launch_decode(ga, sp, mode, seq, zp, act_dtype, scale_dtype, st)) return AWQ_ERR_UNSUPPORTED;
    return launch_status();
  }
  if (rows <= 1 && decode_chunks(M, N, group_size)) {
    // 32-row chunks in order on the stream, sharing the workspace (each chunk's split-K
    // counters return to zero before the next starts)
    for (int64_t m0 = 0; m0 < M; m0 += 32) {
      const int64_t mc = M - m0 < 32 ? M - m0 : 32;
      const int rc = gemm_impl((const uint16_t*)a + m0 * lda, lda, qweight, scales, qzeros, bias, (uint16_t*)c + m0 * ldc,
                               ldc, mc, N, K, group_size, split_k, layout, act_dtype, scale_dtype, bias_dtype, workspace,
                               workspace_bytes, stream, 0);
      if (rc != AWQ_OK) return rc;
    }
    return AWQ_OK;
  }
  if ((K % 32) != 0) return AWQ_ERR_SHAPE;
  if (layout == AWQ_LAYOUT_DECODE_STREAM) {
    // K ranges where the workspace holds their fp32 partials (else the whole K per tile)
    const int S = rows <= 1 ? prefill_splits(M, N, K, group_size, split_k, layout) : 1;
    if (S > 1 && workspace && !(((uintptr_t)workspace) & 15) &&
        workspace_bytes >= kCounterBytes + (size_t)S * (size_t)M * (size_t)N * sizeof(float)) {
      ga.partial = (float*)((char*)workspace + kCounterBytes);
      ga.ksplit = S;
    }
    if (!launch_prefill_stream(ga, zp, act_dtype, scale_dtype, st)) return AWQ_ERR_UNSUPPORTED;
  } else if (!launch_prefill(ga, seq, zp, act_dtype, scale_dtype, st)) {
    return AWQ_ERR_UNSUPPORTED;
  }
  return launch_status();
}

extern "C" {

int awq_w4a16_gemm(const void* a, int64_t lda, const int32_t* qweight, const void* scales,
                   const int32_t* qzeros, const void* bias, void* c, int64_t ldc, int64_t M,
                   int64_t N, int64_t K, int32_t group_size, int32_t split_k, int32_t layout,
                   int32_t act_dtype, int32_t scale_dtype, int32_t bias_dtype, void* workspace,
                   size_t workspace_bytes, void* stream) {
  return gemm_impl(a, lda, qweight, scales, qzeros, bias, c, ldc, M, N, K, group_size, split_k, layout, act_dtype,
                   scale_dtype, bias_dtype, workspace, workspace_bytes, stream, 1);
}

size_t awq_w4a16_gemm_noalloc_max_workspace(void) { return kNoallocScratchBytes; }

int awq_w4a16_gemm_noalloc(const void* a, int64_t lda, const int32_t* qweight, const void* scales,
                           const int32_t* qzeros, const void* bias, void* c, int64_t ldc, int64_t M, int64_t N,
                           int64_t K, int32_t group_size, int32_t split_k, int32_t layout, int32_t act_dtype,
                           int32_t scale_dtype, int32_t bias_dtype, void* stream) {
  if (M < 0 || N < 0 || K <= 0 || group_size <= 0 || split_k < 0) return AWQ_ERR_SHAPE;
  if (M == 0 || N == 0) return AWQ_OK;
  // the decode kernels' split-K needs only: prefill calls get no workspace here, so each of
  // their tiles takes the whole K
  const size_t need = decode_workspace_bytes(M, N, K, group_size, split_k, layout);
  if (need > kNoallocScratchBytes) return AWQ_ERR_WORKSPACE;  // beyond the fixed scratch
  void* ws = nullptr;
  if (need > 0) {
    const int rc = noalloc_scratch(&ws, (hipStream_t)stream);
    if (rc != AWQ_OK) return rc;
  }
  return awq_w4a16_gemm(a, lda, qweight, scales, qzeros, bias, c, ldc, M, N, K, group_size, split_k, layout,
                        act_dtype, scale_dtype, bias_dtype, ws, need > 0 ? kNoallocScratchBytes : 0, stream);
}

size_t awq_w4a16_gemm_rows_exact_workspace_bytes(int64_t M, int64_t N, int64_t K, int32_t group_size,
                                                 int32_t split_k, int32_t layout) {
  const size_t one = awq_w4a16_gemm_workspace_bytes(1, N, K, group_size, split_k, layout);
  if (M <= 0 || one == 0) return 0;
  return kCounterBytes + (size_t)M * (one - kCounterBytes);
}

int awq_w4a16_gemm_rows_exact(const void* a, int64_t lda, const int32_t* qweight, const void* scales,
                              const int32_t* qzeros, const void* bias, void* c, int64_t ldc, int64_t M,
                              int64_t N, int64_t K, int32_t group_size, int32_t split_k, int32_t layout,
                              int32_t act_dtype, int32_t scale_dtype, int32_t bias_dtype, void* workspace,
                              size_t workspace_bytes, void* stream) {
  if (!a || !c) return AWQ_ERR_NULL;
  if (M < 0) return AWQ_ERR_SHAPE;
  if (M == 0 || N == 0) return AWQ_OK;
  if (M > 1 && (lda < K || ldc < N)) return AWQ_ERR_STRIDE;
  // the decode kernels' group sizes: one launch of M grid rows, each row the M = 1 problem
  if (M == 1 || (group_size > 0 && decode_covers(1, group_size)))
    return gemm_impl(a, lda, qweight, scales, qzeros, bias, c, ldc, 1, N, K, group_size, split_k, layout, act_dtype,
                     scale_dtype, bias_dtype, workspace, workspace_bytes, stream, M);
  // other group sizes take the prefill kernel at M = 1: one launch per row, in row order
  const int64_t ebytes = 2;  // both activation dtypes are 16-bit
  for (int64_t m = 0; m < M; ++m) {
    const int rc = gemm_impl((const char*)a + m * lda * ebytes, lda, qweight, scales, qzeros, bias,
                             (char*)c + m * ldc * ebytes, ldc, 1, N, K, group_size, split_k, layout, act_dtype,
                             scale_dtype, bias_dtype, workspace, workspace_bytes, stream, 1);
    if (rc != AWQ_OK) return rc;
  }
  return AWQ_OK;
}

int awq_w4a16_probe_read(const void* buf, int64_t bytes, int32_t blocks, int32_t threads, int32_t in_flight,
                         void* sink, void* stream) {
  if (!buf || !sink) return AWQ_ERR_NULL;
  if (bytes <= 0 || (bytes % 16) != 0 || (((uintptr_t)buf) & 15)) return AWQ_ERR_SHAPE;
  if (blocks <= 0 || threads <= 0 || threads > 1024 || (threads % 64) != 0) return AWQ_ERR_SHAPE;
  if (in_flight != 2 && in_flight != 4 && in_flight != 8) return AWQ_ERR_UNSUPPORTED;
  return launch_probe_read(buf, bytes, blocks, threads, in_flight, sink, (hipStream_t)stream);
}

int awq_w4a16_repack_nk_to_autoawq(const int32_t* qweight_nk, const int32_t* qzeros_nk,
                                   const void* scales_nk, int32_t* qweight_kn, int32_t* qzeros_kn,
                                   void* scales_kn, int64_t N, int64_t K, int32_t group_size,
                                   void* stream) {
  return launch_repack_nk_to_autoawq(qweight_nk, qzeros_nk, scales_nk, qweight_kn, qzeros_kn,
                                     scales_kn, N, K, group_size, (hipStream_t)stream);
}

int64_t awq_w4a16_decode_narrow_bytes(int64_t K, int64_t N) {
  if (K <= 0 || N <= 0 || (N % 8) != 0 || (K % 32) != 0) return 0;
  return decode_narrow_bytes(K, N);
}

int awq_w4a16_pack_decode_narrow(const int32_t* qweight_kn, int32_t* out, int64_t K, int64_t N, void* stream) {
  if (!qweight_kn || !out) return AWQ_ERR_NULL;
  if (K <= 0 || N <= 0 || (N % 8) != 0 || (K % 32) != 0) return AWQ_ERR_SHAPE;
  if (decode_narrow_bytes(K, N) > 0x7FFFFFFFLL) return AWQ_ERR_UNSUPPORTED;
  return launch_pack_decode_narrow(qweight_kn, out, K, N, (hipStream_t)stream);
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
  return launch_pack_decode_stream(qweight_kn, out, K, N, (hipStream_t)stream);
}

// ---- mixture of experts ----

int64_t awq_w4a16_moe_stream_bytes(int64_t E, int64_t K, int64_t N, int32_t gate_up) {
  if (E <= 0 || K <= 0 || N <= 0 || (K % 32) != 0 || (N % (gate_up ? 16 : 8)) != 0) return 0;
  return moe_stream_bytes(E, K, N, gate_up ? 1 : 0);
}

int awq_w4a16_moe_pack_stream(const int32_t* qweight_ekn, int32_t* out, int64_t E, int64_t K, int64_t N,
                              int32_t gate_up, void* stream) {
  if (!qweight_ekn || !out) return AWQ_ERR_NULL;
  if (E < 0 || K < 0 || N < 0 || (K % 32) != 0 || (N % (gate_up ? 16 : 8)) != 0) return AWQ_ERR_SHAPE;
  if (E > 0 && moe_stream_bytes(1, K, N, gate_up ? 1 : 0) > 0x7FFFFFFFLL) return AWQ_ERR_UNSUPPORTED;
  return launch_moe_pack_stream(qweight_ekn, out, E, K, N, gate_up ? 1 : 0, (hipStream_t)stream);
}

int awq_w4a16_moe_route(const void* logits, int64_t ld, int32_t logits_dtype, int64_t T, int32_t E,
                        int32_t top_k, int32_t renormalize, float* topk_weights, int32_t* topk_ids,
                        void* stream) {
  if (!logits || !topk_weights || !topk_ids) return AWQ_ERR_NULL;
  if (logits_dtype != AWQ_DTYPE_F16 && logits_dtype != AWQ_DTYPE_BF16 && logits_dtype != AWQ_DTYPE_F32)
    return AWQ_ERR_UNSUPPORTED;
  if (T < 0 || E <= 0 || E > 256 || top_k <= 0 || top_k > E || top_k > 64) return AWQ_ERR_SHAPE;
  if (ld < E) return AWQ_ERR_STRIDE;
  return launch_moe_route(logits, ld, logits_dtype, T, E, top_k,
                          renormalize ? (uint32_t)(AWQ_ROUTE_RENORMALIZE | AWQ_ROUTE_CLAMP_SUM) : 0u, topk_weights,
                          AWQ_DTYPE_F32, topk_ids, (hipStream_t)stream);
}

int awq_w4a16_moe_route_ex(const void* logits, int64_t ld, int32_t logits_dtype, int64_t T, int32_t E,
                           int32_t top_k, uint32_t flags, void* topk_weights, int32_t weights_dtype,
                           int32_t* topk_ids, void* stream) {
  if (!logits || !topk_weights || !topk_ids) return AWQ_ERR_NULL;
  if (logits_dtype != AWQ_DTYPE_F16 && logits_dtype != AWQ_DTYPE_BF16 && logits_dtype != AWQ_DTYPE_F32)
    return AWQ_ERR_UNSUPPORTED;
  if (weights_dtype != AWQ_DTYPE_F16 && weights_dtype != AWQ_DTYPE_BF16 && weights_dtype != AWQ_DTYPE_F32)
    return AWQ_ERR_UNSUPPORTED;
  if ((flags & ~(uint32_t)(AWQ_ROUTE_RENORMALIZE | AWQ_ROUTE_SOFTMAX_IN_LOGITS_DTYPE | AWQ_ROUTE_CLAMP_SUM)) != 0)
    return AWQ_ERR_UNSUPPORTED;
  if (T < 0 || E <= 0 || E > 256 || top_k <= 0 || top_k > E || top_k > 64) return AWQ_ERR_SHAPE;
  if (ld < E) return AWQ_ERR_STRIDE;
  return launch_moe_route(logits, ld, logits_dtype, T, E, top_k, flags, topk_weights, weights_dtype, topk_ids,
                          (hipStream_t)stream);
}

size_t awq_w4a16_moe_workspace_bytes(int64_t T, int64_t H, int64_t I, int32_t E, int32_t top_k) {
  if (T <= 0 || H <= 0 || I <= 0 || E <= 0 || top_k <= 0) return 0;
  return (size_t)moe_workspace(T, H, I, E, top_k, 2).total;
}

int awq_w4a16_moe(const void* x, int64_t ldx, const void* topk_ids, int32_t ids_bits, const void* topk_weights,
                  int32_t weights_dtype, const int32_t* gate_up_stream, const void* gate_up_scales,
                  const int32_t* gate_up_qzeros, const int32_t* down_stream, const void* down_scales,
                  const int32_t* down_qzeros, void* out, int64_t ldo, int64_t T, int64_t H, int64_t I,
                  int32_t E, int32_t top_k, int32_t group_size, int32_t activation, int32_t act_dtype,
                  int32_t scale_dtype, void* workspace, size_t workspace_bytes, void* stream) {
  if (T < 0 || H <= 0 || I <= 0 || E <= 0 || top_k <= 0) return AWQ_ERR_SHAPE;
  if (T == 0) return AWQ_OK;
  if (!x || !topk_ids || !topk_weights || !gate_up_stream || !gate_up_scales || !down_stream ||
      !down_scales || !out)
    return AWQ_ERR_NULL;
  if ((gate_up_qzeros == nullptr) != (down_qzeros == nullptr)) return AWQ_ERR_NULL;
  if (!dtype_16(act_dtype) || !dtype_16(scale_dtype)) return AWQ_ERR_UNSUPPORTED;
  if (weights_dtype != AWQ_DTYPE_F16 && weights_dtype != AWQ_DTYPE_BF16 && weights_dtype != AWQ_DTYPE_F32)
    return AWQ_ERR_UNSUPPORTED;
  if (ids_bits != 32 && ids_bits != 64) return AWQ_ERR_UNSUPPORTED;
  if (activation != AWQ_MOE_ACT_SILU && activation != AWQ_MOE_ACT_GELU_TANH) return AWQ_ERR_UNSUPPORTED;
  if (group_size != 32 && group_size != 64 && group_size != 128) return AWQ_ERR_UNSUPPORTED;
  if ((H % group_size) != 0 || (I % group_size) != 0 || (H % 8) != 0 || (I % 8) != 0) return AWQ_ERR_SHAPE;
  if (E > 65535) return AWQ_ERR_SHAPE;
  if (ldx < H || ldo < H || (ldx % 8) != 0 || (ldo % 4) != 0) return AWQ_ERR_STRIDE;
  if ((((uintptr_t)x) & 15) || (((uintptr_t)out) & 7) || (((uintptr_t)gate_up_scales) & 15) ||
      (((uintptr_t)down_scales) & 15) || (((uintptr_t)gate_up_stream) & 15) || (((uintptr_t)down_stream) & 15))
    return AWQ_ERR_STRIDE;
  // 32-bit buffer offsets: one expert's tensors, the activations and the per-route buffers
  const int64_t R = T * top_k;
  if (moe_stream_bytes(1, H, 2 * I, 1) > 0x7FFFFFFFLL || moe_stream_bytes(1, I, H, 0) > 0x7FFFFFFFLL ||
      T * ldx * 2 > 0x7FFFFFFFLL || R * I * 2 > 0x7FFFFFFFLL || R * H * 4 > 0x7FFFFFFFLL || R > 0x7FFFFFFFLL)
    return AWQ_ERR_UNSUPPORTED;
  const MoeWorkspace w = moe_workspace(T, H, I, E, top_k, 2);
  if (!workspace || workspace_bytes < (size_t)w.total) return AWQ_ERR_WORKSPACE;
  if (((uintptr_t)workspace) & 255) return AWQ_ERR_WORKSPACE;
  MoeCall c{};
  c.x = x;
  c.ldx = ldx;
  c.ids = topk_ids;
  c.id64 = ids_bits == 64 ? 1 : 0;
  c.rw = topk_weights;
  c.rw_dtype = weights_dtype;
  c.gu_qw = gate_up_stream;
  c.gu_qz = gate_up_qzeros;
  c.dn_qw = down_stream;
  c.dn_qz = down_qzeros;
  c.gu_sc = gate_up_scales;
  c.dn_sc = down_scales;
  c.out = out;
  c.ldo = ldo;
  c.T = T;
  c.H = H;
  c.I = I;
  c.E = E;
  c.topk = top_k;
  c.G = group_size;
  c.act_kind = activation;
  c.act_dtype = act_dtype;
  c.scale_dtype = scale_dtype;
  c.workspace = workspace;
  return launch_moe(c, (hipStream_t)stream);
}

int awq_w4a16_gate_up_interleave(const void* gate, const void* up, void* out, int64_t rows, int64_t cols,
                                 int32_t elem_bytes, int32_t half_tile, void* stream) {
  if (rows < 0 || cols < 0 || half_tile <= 0) return AWQ_ERR_SHAPE;
  if (elem_bytes != 2 && elem_bytes != 4) return AWQ_ERR_UNSUPPORTED;
  if (rows == 0 || cols == 0) return AWQ_OK;
  if (!gate || !up || !out) return AWQ_ERR_NULL;
  return launch_gate_up_interleave(gate, up, out, rows, cols, elem_bytes, half_tile, (hipStream_t)stream);
}

size_t awq_w4a16_gate_up_workspace_bytes(int64_t M, int64_t I, int64_t K, int32_t group_size,
                                         int32_t split_k, int32_t layout) {
  if (I <= 0 || layout == AWQ_LAYOUT_DECODE_NARROW) return 0;
  return awq_w4a16_gemm_workspace_bytes(M, 2 * cdiv(I, 64) * 64, K, group_size, split_k, layout);
}

int awq_w4a16_gate_up_act(const void* x, int64_t ldx, const int32_t* qweight, const void* scales,
                          const int32_t* qzeros, void* out, int64_t ldo, int64_t M, int64_t I, int64_t K,
                          int32_t group_size, int32_t split_k, int32_t layout, int32_t activation,
                          int32_t act_dtype, int32_t scale_dtype, void* workspace, size_t workspace_bytes,
                          void* stream) {
  if (M < 0 || I < 0 || K <= 0 || group_size <= 0 || split_k < 0) return AWQ_ERR_SHAPE;
  if (M == 0 || I == 0) return AWQ_OK;
  if (!x || !qweight || !scales || !out) return AWQ_ERR_NULL;
  if (!dtype_16(act_dtype) || !dtype_16(scale_dtype)) return AWQ_ERR_UNSUPPORTED;
  if (activation != AWQ_MOE_ACT_SILU && activation != AWQ_MOE_ACT_GELU_TANH) return AWQ_ERR_UNSUPPORTED;
  if (layout != AWQ_LAYOUT_AUTOAWQ && layout != AWQ_LAYOUT_KN_SEQ && layout != AWQ_LAYOUT_DECODE_STREAM &&
      layout != AWQ_LAYOUT_DECODE_NARROW)
    return AWQ_ERR_UNSUPPORTED;
  if (!decode_covers(M, group_size)) return AWQ_ERR_UNSUPPORTED;
  if ((K % group_size) != 0) return AWQ_ERR_SHAPE;
  const bool narrow = layout == AWQ_LAYOUT_DECODE_NARROW;
  if (narrow && (K % 32) != 0) return AWQ_ERR_SHAPE;
  if (ldx < K || ldo < I || (ldx % 8) != 0) return AWQ_ERR_STRIDE;
  if ((((uintptr_t)x) & 15) || (((uintptr_t)out) & 1) || (((uintptr_t)scales) & 15) ||
      (((uintptr_t)qweight) & 15))
    return AWQ_ERR_STRIDE;
  // the interleaved matrix: 64-column halves (8 for the narrow layout)
  const int64_t N = narrow ? 2 * cdiv(I, 8) * 8 : 2 * cdiv(I, 64) * 64;
  if (decode_stream_bytes(K, N) > 0x7FFFFFFFLL || M * ldx * 2 > 0x7FFFFFFFLL) return AWQ_ERR_UNSUPPORTED;

  GemmArgs ga{};
  ga.a = (const uint16_t*)x;
  ga.qw = (const uint32_t*)qweight;
  ga.sc = (const uint16_t*)scales;
  ga.qz = (const uint32_t*)qzeros;
  ga.c = (uint16_t*)out;
  ga.lda = ldx;
  ga.ldc = ldo;
  ga.M = (int)M;
  ga.N = (int)N;
  ga.K = (int)K;
  ga.G = group_size;
  ga.bias_dtype = AWQ_DTYPE_NONE;
  ga.gate_act = 1 + activation;
  ga.n_out = (int)I;
  if (narrow) {
    if (decode_narrow_bytes(K, N) > 0x7FFFFFFFLL) return AWQ_ERR_UNSUPPORTED;
    if (!launch_decode_narrow(ga, qzeros != nullptr, act_dtype, scale_dtype, (hipStream_t)stream))
      return AWQ_ERR_UNSUPPORTED;
    return launch_status();
  }
  const DecodeMode mode = decode_mode(layout, act_dtype, scale_dtype);
  const DecodePlan sp = plan_decode(M, N, K, group_size, split_k, mode);
  if (sp.ws_bytes) {
    if (!workspace || workspace_bytes < sp.ws_bytes) return AWQ_ERR_WORKSPACE;
    if ((size_t)sp.tiles * sizeof(int) > kCounterBytes) return AWQ_ERR_UNSUPPORTED;
    if (sp.ws_bytes - kCounterBytes > 0x7FFFFFFFu) return AWQ_ERR_UNSUPPORTED;  // 32-bit offsets
    ga.counters = (int*)workspace;
    ga.partial = (float*)((char*)workspace + kCounterBytes);
  }
  if (!launch_decode(ga, sp, mode, layout == AWQ_LAYOUT_KN_SEQ, qzeros != nullptr, act_dtype, scale_dtype,
                     (hipStream_t)stream))
    return AWQ_ERR_UNSUPPORTED;
  return launch_status();
}

int awq_w4a16_rmsnorm(const void* x, int64_t ldx, const void* norm_w, float eps, void* xn, int64_t ldxn,
                      int64_t M, int64_t K, int32_t act_dtype, int32_t norm_dtype, void* stream) {
  if (M < 0 || K <= 0 || (K % 8) != 0) return AWQ_ERR_SHAPE;
  if (M == 0) return AWQ_OK;
  if (!x || !norm_w || !xn) return AWQ_ERR_NULL;
  if (!dtype_16(act_dtype) || !dtype_16(norm_dtype)) return AWQ_ERR_UNSUPPORTED;
  if (K > 0x7FFFFFFFLL) return AWQ_ERR_UNSUPPORTED;
  if (ldx < K || ldxn < K || (ldx % 8) != 0 || (ldxn % 8) != 0) return AWQ_ERR_STRIDE;
  if ((((uintptr_t)x) & 15) || (((uintptr_t)norm_w) & 15) || (((uintptr_t)xn) & 15)) return AWQ_ERR_STRIDE;
  return launch_rmsnorm_rows(x, ldx, norm_w, eps, xn, ldxn, M, K, act_dtype, norm_dtype, (hipStream_t)stream);
}

static size_t align256(size_t b) { return (b + 255) & ~(size_t)255; }

size_t awq_w4a16_rmsnorm_gemm_workspace_bytes(int64_t M, int64_t N, int64_t K, int32_t group_size,
                                              int32_t split_k, int32_t layout, int32_t act_dtype) {
  if (M <= 0 || N <= 0 || K <= 0) return 0;
  // the GEMM's part is never smaller than the counter region, so a workspace shared with
  // awq_w4a16_gemm keeps its counters zero
  const size_t g = align256(std::max(awq_w4a16_gemm_workspace_bytes(M, N, K, group_size, split_k, layout),
                                     (size_t)kCounterBytes));
  const size_t xn = align256((size_t)M * (size_t)K * 2);
  const size_t c16 = act_dtype == AWQ_DTYPE_BF16 ? align256((size_t)M * (size_t)N * 2) : 0;
  return g + xn + c16;
}

int awq_w4a16_rmsnorm_gemm(const void* x, int64_t ldx, const void* norm_w, float eps,
                           const int32_t* qweight, const void* scales, const int32_t* qzeros, void* c,
                           int64_t ldc, int64_t M, int64_t N, int64_t K, int32_t group_size, int32_t split_k,
                           int32_t layout, int32_t act_dtype, int32_t norm_dtype, int32_t scale_dtype,
                           void* workspace, size_t workspace_bytes, void* stream) {
  if (M < 0 || N < 0 || K <= 0 || group_size <= 0 || split_k < 0) return AWQ_ERR_SHAPE;
  if (M == 0 || N == 0) return AWQ_OK;
  if (!x || !norm_w || !qweight || !scales || !c) return AWQ_ERR_NULL;
  if (!workspace) return AWQ_ERR_WORKSPACE;
  if (!dtype_16(act_dtype) || !dtype_16(norm_dtype) || !dtype_16(scale_dtype)) return AWQ_ERR_UNSUPPORTED;
  if ((N % 8) != 0 || (K % 8) != 0 || (group_size % 32) != 0 || (K % group_size) != 0) return AWQ_ERR_SHAPE;
  if (layout != AWQ_LAYOUT_AUTOAWQ && layout != AWQ_LAYOUT_KN_SEQ && layout != AWQ_LAYOUT_DECODE_STREAM &&
      layout != AWQ_LAYOUT_DECODE_NARROW)
    return AWQ_ERR_UNSUPPORTED;
  if (ldx < K || (ldx % 8) != 0 || (((uintptr_t)x) & 15)) return AWQ_ERR_STRIDE;
  if (ldc < N || (ldc % 8) != 0 || (((uintptr_t)c) & 15)) return AWQ_ERR_STRIDE;
  const size_t gws = awq_w4a16_gemm_workspace_bytes(M, N, K, group_size, split_k, layout);
  if (workspace_bytes < awq_w4a16_rmsnorm_gemm_workspace_bytes(M, N, K, group_size, split_k, layout, act_dtype))
    return AWQ_ERR_WORKSPACE;
  if ((((uintptr_t)workspace) & 255)) return AWQ_ERR_STRIDE;
  if (layout == AWQ_LAYOUT_DECODE_NARROW && act_dtype == AWQ_DTYPE_F16 && scale_dtype == AWQ_DTYPE_F16 && M == 1 &&
      decode_covers(M, group_size) && (K % 32) == 0 && decode_narrow_bytes(K, N) <= 0x7FFFFFFFLL &&
      M * ldx * 2 <= 0x7FFFFFFFLL && !(((uintptr_t)qweight) & 15) && !(((uintptr_t)scales) & 15) &&
      !(((uintptr_t)norm_w) & 15)) {
    // one launch: the narrow kernel normalises its staged rows itself
    GemmArgs ga{};
    ga.a = (const uint16_t*)x;
    ga.qw = (const uint32_t*)qweight;
    ga.sc = (const uint16_t*)scales;
    ga.qz = (const uint32_t*)qzeros;
    ga.c = (uint16_t*)c;
    ga.lda = ldx;
    ga.ldc = ldc;
    ga.M = (int)M;
    ga.N = (int)N;
    ga.K = (int)K;
    ga.G = group_size;
    ga.bias_dtype = AWQ_DTYPE_NONE;
    ga.norm_w = (const uint16_t*)norm_w;
    ga.eps = eps;
    ga.norm_bf16 = norm_dtype == AWQ_DTYPE_BF16;
    if (launch_decode_narrow_norm(ga, qzeros != nullptr, (hipStream_t)stream)) return launch_status();
  }
  char* xn = (char*)workspace + align256(std::max(gws, (size_t)kCounterBytes));
  char* c16 = xn + align256((size_t)M * (size_t)K * 2);
  const bool bf = act_dtype == AWQ_DTYPE_BF16;
  if (bf && M > 65535) return AWQ_ERR_UNSUPPORTED;  // rows of the conversion grid
  int rc = awq_w4a16_rmsnorm(x, ldx, norm_w, eps, xn, K, M, K, act_dtype, norm_dtype, stream);
  if (rc != AWQ_OK) return rc;
  rc = awq_w4a16_gemm(xn, K, qweight, scales, qzeros, nullptr, bf ? (void*)c16 : c, bf ? N : ldc, M, N, K,
                      group_size, split_k, layout, AWQ_DTYPE_F16, scale_dtype, AWQ_DTYPE_NONE,
                      gws ? workspace : nullptr, gws, stream);
  if (rc != AWQ_OK || !bf) return rc;
  return launch_f16_to_bf16(c16, N, c, ldc, M, N, (hipStream_t)stream);
}

}  // extern "C"
