/*
 * C ABI of the MI355X (gfx950) AWQ W4A16 dequant-GEMM library (libawq_w4a16.so).
 *
 * Plain pointers and sizes only: every tensor argument is a device pointer owned by
 * the caller, every size is an element count, `stream` is a hipStream_t passed as
 * void* (NULL = the default stream).  No function allocates device memory; scratch
 * space comes in through `workspace`.  Every function returns 0 on success or one of
 * the AWQ_ERR_* codes below, never throws, and leaves no pending HIP error behind.
 *
 * Reference interfaces each entry point replaces (paths relative to the
 * jiayingsong2023/litevLLM checkout):
 *   awq_w4a16_dequant  <- awq_dequantize_triton / awq_dequantize_kernel
 *                         (vllm/model_executor/layers/quantization/awq_triton.py:64-194)
 *                         and dequantize_awq_pytorch / dequantize_symmetric_packed_int4_pytorch
 *                         (vllm/model_executor/layers/quantization/tensor.py:835-901)
 *   awq_w4a16_gemm     <- the launches inside awq_fused_gemm
 *                         (vllm/kernels/triton/awq_fused_gemm.py:2395-2552) of
 *                         _awq_native_tiled_gemm_{heuristic,split_k,autotuned}
 *                         (awq_fused_gemm.py:1754-1990, 2296-2392) and, with qzeros == NULL,
 *                         packed_int4_symmetric_fused_gemm (awq_fused_gemm.py:2555-2922)
 *   awq_w4a16_gemm_workspace_bytes <- the split-K output zero-fill of awq_fused_gemm
 *                         (awq_fused_gemm.py:2434-2443), replaced by an fp32 partial buffer
 *   awq_w4a16_repack   <- no kernel in the reference: the lossless layout conversion the
 *                         model loader would need at model_loader/__init__.py:756-797
 *   awq_w4a16_moe      <- the grouped int4 MoE wrappers gemma4_moe_int4_prefill_grouped(_fused)
 *                         (vllm/kernels/triton/gemma4_moe_int4.py:2330-2584) and the expert loop
 *                         of fused_moe (vllm/model_executor/layers/fused_moe/fused_moe.py:17-56)
 *                         that zero-point AWQ experts take after dequantizing
 *                         (vllm/model_executor/models/gemma4/moe.py:566-623)
 *   awq_w4a16_moe_route <- the routing of fused_moe.py:12-15 / gemma4/moe.py:106-116
 *   awq_w4a16_moe_route_ex <- the same with the reference's dtype flows: fused_moe's softmax in
 *                         the logits dtype (fused_moe.py:12-15) and the Gemma4 router's fp32
 *                         softmax with weights cast to the hidden dtype (gemma4/moe.py:106-123)
 *   awq_w4a16_gemm_rows_exact <- _packed_int4_symmetric_group32_gemv_rows_exact_msmall
 *                         (vllm/kernels/triton/awq_fused_gemm.py:1066-1143, 2925-2998)
 *   awq_w4a16_moe_pack_stream <- no kernel in the reference: the expert-major weight prepack the
 *                         grouped kernels read (the reference reads its [E, N, K/8] stacks directly)
 *   awq_w4a16_rmsnorm_gemm <- rmsnorm_awq_fused_linear / rmsnorm_awq_fused_kernel
 *                         (vllm/kernels/triton/rmsnorm_awq_fused.py:43-189)
 *   awq_w4a16_rmsnorm  <- the RMSNorm phase of that kernel (rmsnorm_awq_fused.py:108-131)
 */
#ifndef AWQ_W4A16_H
#define AWQ_W4A16_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* ---- packed layouts (G = group_size) ------------------------------------------
 * AWQ_LAYOUT_AUTOAWQ : qweight int32 [K, N/8], nibble i of word (k, j) = W[k, 8j + order[i]],
 *                      order = {0,2,4,6,1,3,5,7}; qzeros int32 [K/G, N/8] packed the same way;
 *                      scales [K/G, N].  (AutoAWQ "GEMM" checkpoint layout.)
 * AWQ_LAYOUT_KN_SEQ  : as AUTOAWQ but sequential nibbles (nibble i = column 8j + i); the
 *                      geometry awq_dequantize_triton handles when scales.shape[0] != rows
 *                      (awq_triton.py:107-118, 161).
 * AWQ_LAYOUT_NK_SEQ  : reference runtime layout: qweight int32 [N, K/8], nibble i of word
 *                      (n, j) = W[n, 8j + i]; qzeros int32 [N, ceil(K/G/8)] sequential along
 *                      the group axis; scales [N, K/G]  (tensor.py:842-858).
 * AWQ_LAYOUT_DECODE_STREAM : an AUTOAWQ qweight re-ordered by awq_w4a16_pack_decode_stream so
 *                      that the decode kernel reads it as contiguous 2 KiB runs; qzeros and
 *                      scales stay in the AUTOAWQ layout.  Accepted by awq_w4a16_gemm for every
 *                      M (K % 32 == 0): the decode kernel serves M <= 32 with group sizes
 *                      32/64/128 (and 32-row chunks of it up to M = 64), the prefill
 *                      kernel the rest, so one copy serves both.
 * AWQ_LAYOUT_DECODE_NARROW : an AUTOAWQ qweight re-ordered by awq_w4a16_pack_decode_narrow
 *                      into 16-column tiles cut along K into quads of four 32-row k-steps
 *                      (KQ = ceil(K / 128) quads per tile; k-steps past K are zero): the run of
 *                      (tile t, quad c) is 1 KiB at byte (t * KQ + c) * 1024, lane l = 16 q + r
 *                      owns its 16 bytes at 16 l, and u32 number i of them holds k-step
 *                      s = 4 c + i of column 16 t + r, rows 32 s + 8 q + j (j < 8).  Read by the
 *                      narrow decode kernel: one block per 16 columns over the whole K, no
 *                      split-K.  Accepted by awq_w4a16_gemm only for M <= 32, group sizes
 *                      32 / 64 / 128 and K % 32 == 0 (prefill-sized calls need DECODE_STREAM
 *                      or AUTOAWQ).
 */
#define AWQ_LAYOUT_AUTOAWQ 0
#define AWQ_LAYOUT_KN_SEQ 1
#define AWQ_LAYOUT_NK_SEQ 2
#define AWQ_LAYOUT_DECODE_STREAM 3
#define AWQ_LAYOUT_DECODE_NARROW 4

/* ---- element types ---- */
#define AWQ_DTYPE_NONE 0 /* e.g. no bias */
#define AWQ_DTYPE_F16 1
#define AWQ_DTYPE_BF16 2
#define AWQ_DTYPE_F32 3

/* ---- error codes ---- */
#define AWQ_OK 0
#define AWQ_ERR_NULL 1        /* a required pointer is NULL */
#define AWQ_ERR_SHAPE 2       /* sizes inconsistent (K % G, N % 8, K % 32, ...) */
#define AWQ_ERR_UNSUPPORTED 3 /* dtype / layout / group size combination not provided */
#define AWQ_ERR_WORKSPACE 4   /* workspace NULL or smaller than required */
#define AWQ_ERR_LAUNCH 5      /* a HIP launch failed */
#define AWQ_ERR_STRIDE 6      /* leading dimension smaller than the row length */

/* Library version (major * 10000 + minor * 100 + patch). */
int awq_w4a16_version(void);

/* Static description of an error code (never NULL). */
const char* awq_w4a16_strerror(int code);

/* Dequantize a packed int4 matrix: out = RNE_outdtype((q - z) * s), computed so that
 * the result equals one rounding of the exact product (float32 arithmetic in the
 * reference, tensor.py:857-858 / awq_triton.py:138-145).
 *   rows x cols is the *unpacked* matrix in the packed tensor's own orientation:
 *   AUTOAWQ / KN_SEQ: rows = K, cols = N, out [K, N];  NK_SEQ: rows = N, cols = K, out [N, K].
 *   qzeros == NULL selects symmetric mode z = 8 (tensor.py:891).
 *   scale_dtype: F16 or BF16.  out_dtype: F16, BF16 or F32.  out is dense row-major.
 */
int awq_w4a16_dequant(const int32_t* qweight, const void* scales, const int32_t* qzeros, void* out,
                      int64_t rows, int64_t cols, int32_t group_size, int32_t layout,
                      int32_t scale_dtype, int32_t out_dtype, void* stream);

/* Workspace bytes awq_w4a16_gemm needs for these arguments (0 if none).  The workspace
 * starts with a fixed 64 KiB region of per-tile arrival counters followed by fp32 split-K
 * partials (the decode kernels', or the prefill kernel's K ranges: [ranges][M][N]; a prefill
 * call given less than that runs its whole K per tile).  The counter region must be zero the first time a workspace is used; every
 * call leaves it zero again, so a workspace allocated zeroed once can be reused by later
 * calls of any shape on the same stream.  Two calls that may run concurrently must not
 * share a workspace. */
size_t awq_w4a16_gemm_workspace_bytes(int64_t M, int64_t N, int64_t K, int32_t group_size,
                                      int32_t split_k, int32_t layout);

/* C[M, N] = A[M, K] . dequant(W)^T (+ bias), products accumulated in fp32, one rounding to
 * act_dtype at the end.  M <= 32 with group_size 32, 64 or 128 (the decode kernel; calls up to
 * M = 64 run as 32-row chunks on it, one launch each, in order on the stream): the weights
 * enter unrounded, (q - z) * s in fp32 -- the reference's M = 1
 * formulation, awq_fused_gemm.py:1966-1971.  Otherwise (the prefill kernel): W rounded once to act_dtype,
 * as awq_w4a16_dequant computes it (the reference's tl.dot branch, 1973-1976).
 *   a: [M, K] act_dtype (F16 or BF16), row stride lda (elements).
 *   layout: AUTOAWQ or KN_SEQ (qweight [K, N/8]), DECODE_STREAM (any M) or DECODE_NARROW
 *           (M <= 32).  An NK_SEQ
 *           weight is converted once with awq_w4a16_repack_nk_to_autoawq; passing NK_SEQ
 *           here returns AWQ_ERR_UNSUPPORTED.
 *   qzeros == NULL: symmetric z = 8.  scales: scale_dtype (F16 or BF16).
 *   bias: NULL or [N] of bias_dtype (F16, BF16 or F32), added once in fp32.
 *   c: [M, N] act_dtype, row stride ldc.
 *   split_k: number of contiguous K partitions of the decode kernel whose fp32 partial sums
 *            are added in a fixed order (0 = choose automatically; with 0 and the
 *            DECODE_STREAM layout the prefill kernel cuts K into 3 .. 8 ranges of whole
 *            64-row stage pairs where its 256 x 256 tiles cover at most a third of the CUs
 *            and the workspace holds their fp32 partials, summed in range order; otherwise
 *            the prefill kernel does not split K).  For a given (M, N, K, split_k) the result is bitwise
 *            reproducible.  Partition s covers rows [64 s I, min(64 (s+1) I, K)) with
 *            I = ceil(ceil(K / 64) / split_k), as in awq_fused_gemm.py:1798-1800.  The
 *            DECODE_NARROW layout never splits K (split_k is ignored there).
 *   Requirements: N % 8 == 0, group_size % 32 == 0, K % group_size == 0.
 */
int awq_w4a16_gemm(const void* a, int64_t lda, const int32_t* qweight, const void* scales,
                   const int32_t* qzeros, const void* bias, void* c, int64_t ldc, int64_t M,
                   int64_t N, int64_t K, int32_t group_size, int32_t split_k, int32_t layout,
                   int32_t act_dtype, int32_t scale_dtype, int32_t bias_dtype, void* workspace,
                   size_t workspace_bytes, void* stream);

/* Allocation-free GEMM: awq_w4a16_gemm's computation, bit for bit, with its split-K counters and
 * partials in a fixed scratch array the library holds on every GPU it runs on (static device
 * memory, awq_w4a16_gemm_noalloc_max_workspace() bytes, kept until the process ends) instead of
 * a caller's workspace.  No counterpart in the reference: it is for callers that cannot allocate
 * (code under HIP graph capture, tight serving loops, harnesses that forbid hipMalloc); it calls
 * no hipMalloc / hipFree or allocating routine.  Returns AWQ_ERR_WORKSPACE when the call would
 * need more workspace than that array holds (awq_w4a16_gemm_workspace_bytes of the same
 * arguments; the library's own split-K plans stay within it).  The first call on a device looks
 * the array up and clears its counters (a kernel on `stream`).  Every call on one GPU shares
 * that GPU's array: calls that may overlap on one GPU (other streams, other threads) race and
 * must be serialised by the caller. */
size_t awq_w4a16_gemm_noalloc_max_workspace(void);
int awq_w4a16_gemm_noalloc(const void* a, int64_t lda, const int32_t* qweight, const void* scales,
                           const int32_t* qzeros, const void* bias, void* c, int64_t ldc, int64_t M, int64_t N,
                           int64_t K, int32_t group_size, int32_t split_k, int32_t layout, int32_t act_dtype,
                           int32_t scale_dtype, int32_t bias_dtype, void* stream);

/* Row-exact GEMM: C[m, :] for every m < M equals, bit for bit, what awq_w4a16_gemm computes for
 * the single row A[m, :] with the same arguments (M = 1): each row goes through the M = 1 plan,
 * kernel and reduction order, whatever M is, so a row's result never depends on the batch it
 * rides in.  Replaces _packed_int4_symmetric_group32_gemv_rows_exact_msmall (launched by
 * packed_int4_symmetric_group32_rows_exact_msmall_safe, vllm/kernels/triton/awq_fused_gemm.py:
 * 1066-1143, 2925-2998), whose contract is that M = 2 / 4 rows equal independent M = 1 calls
 * (tests/test_awq_fused_gemm_numerics.py:128-161); here for any M, group size and layout the
 * M = 1 call takes.  Arguments and requirements as awq_w4a16_gemm.  With group size 32, 64 or
 * 128 (the decode kernels) it is one launch of (the M = 1 call's blocks) x M blocks, as the
 * reference's grid (cdiv(N, BN), M) (awq_fused_gemm.py:2980-2981): row m's blocks run row m's
 * M = 1 problem, with split-K counters and partials of its own, so the workspace holds M sets
 * of them (awq_w4a16_gemm_rows_exact_workspace_bytes).  Other group sizes take one launch per
 * row, in row order. */
/* Workspace bytes of awq_w4a16_gemm_rows_exact for M rows (0 if none): the 64 KiB counter
 * region, then M times the fp32 partials of the M = 1 call (awq_w4a16_gemm_workspace_bytes(1,
 * ...)).  Same zero-on-entry, zero-on-exit counter rule as awq_w4a16_gemm's workspace. */
size_t awq_w4a16_gemm_rows_exact_workspace_bytes(int64_t M, int64_t N, int64_t K, int32_t group_size,
                                                 int32_t split_k, int32_t layout);

int awq_w4a16_gemm_rows_exact(const void* a, int64_t lda, const int32_t* qweight, const void* scales,
                              const int32_t* qzeros, const void* bias, void* c, int64_t ldc, int64_t M,
                              int64_t N, int64_t K, int32_t group_size, int32_t split_k, int32_t layout,
                              int32_t act_dtype, int32_t scale_dtype, int32_t bias_dtype, void* workspace,
                              size_t workspace_bytes, void* stream);

/* Measurement utility with no counterpart in the reference: one launch that only reads `bytes`
 * of device memory (a multiple of 16, 16-byte aligned) with 16-byte non-temporal loads --
 * `blocks` blocks of `threads` threads (a multiple of 64, at most 1024), each block a contiguous
 * share, `in_flight` (2, 4 or 8) loads in flight per lane -- and discards the data (`sink`, 256
 * bytes of device memory, is never written in practice).  bench.py times it like a decode
 * launch of the same size to give that launch's HBM read ceiling. */
int awq_w4a16_probe_read(const void* buf, int64_t bytes, int32_t blocks, int32_t threads, int32_t in_flight,
                         void* sink, void* stream);

/* Lossless repack of a reference-layout (NK_SEQ) weight into the AUTOAWQ layout:
 *   qweight_nk [N, K/8] -> qweight_kn [K, N/8];  qzeros_nk [N, ceil(K/G/8)] -> qzeros_kn [K/G, N/8]
 *   (qzeros may be NULL);  scales_nk [N, K/G] -> scales_kn [K/G, N] (2-byte elements). */
int awq_w4a16_repack_nk_to_autoawq(const int32_t* qweight_nk, const int32_t* qzeros_nk,
                                   const void* scales_nk, int32_t* qweight_kn, int32_t* qzeros_kn,
                                   void* scales_kn, int64_t N, int64_t K, int32_t group_size,
                                   void* stream);

/* Bytes of the decode stream copy of a [K, N/8] qweight (N rounded up to 512 columns). */
int64_t awq_w4a16_decode_stream_bytes(int64_t K, int64_t N);

/* Lossless re-ordering of an AUTOAWQ (or KN_SEQ) qweight [K, N/8] into the decode stream
 * layout (out holds awq_w4a16_decode_stream_bytes(K, N) bytes).  No counterpart in the
 * reference: it plays the role of the derived packs the reference caches on its weight
 * objects (vllm/model_executor/layers/quantization/tensor.py:1251-1256), built once per
 * weight so that decode-shaped calls stream the weight contiguously.  K % 32 == 0. */
int awq_w4a16_pack_decode_stream(const int32_t* qweight_kn, int32_t* out, int64_t K, int64_t N,
                                 void* stream);

/* Bytes of the narrow decode copy of a [K, N/8] qweight (N rounded up to 16 columns). */
int64_t awq_w4a16_decode_narrow_bytes(int64_t K, int64_t N);

/* Lossless re-ordering of an AUTOAWQ qweight [K, N/8] into the narrow decode layout (out holds
 * awq_w4a16_decode_narrow_bytes(K, N) bytes).  No counterpart in the reference: a derived pack
 * like awq_w4a16_pack_decode_stream (tensor.py:1251-1256).  K % 32 == 0. */
int awq_w4a16_pack_decode_narrow(const int32_t* qweight_kn, int32_t* out, int64_t K, int64_t N,
                                 void* stream);

/* ---- mixture of experts ------------------------------------------------------------
 * Experts are stacks of AUTOAWQ matrices: gate_up qweight [E, H, 2I/8] (columns 0..I-1 the
 * gate projection, I..2I-1 the up projection), scales [E, H/G, 2I], qzeros [E, H/G, 2I/8];
 * down qweight [E, I, H/8], scales [E, I/G, H], qzeros [E, I/G, H/8].  A route is one
 * (token t, slot j) pair, numbered r = t * top_k + j.
 */
#define AWQ_MOE_ACT_SILU 0      /* silu(gate) * up */
#define AWQ_MOE_ACT_GELU_TANH 1 /* gelu_pytorch_tanh(gate) * up */

/* Bytes of the MoE stream copy of an expert stack [E, K, N/8] (gate_up != 0: the gate_up
 * stack, N = 2I, whose tiles pair gate and up columns; 0: the down stack).  0 if K % 32 or
 * N % 8 (N % 16 for gate_up) fails. */
int64_t awq_w4a16_moe_stream_bytes(int64_t E, int64_t K, int64_t N, int32_t gate_up);

/* Lossless re-ordering of an AUTOAWQ expert stack [E, K, N/8] into the MoE stream layout read
 * by awq_w4a16_moe (out holds awq_w4a16_moe_stream_bytes bytes).  Scales and zeros are used
 * as they are. */
int awq_w4a16_moe_pack_stream(const int32_t* qweight_ekn, int32_t* out, int64_t E, int64_t K, int64_t N,
                              int32_t gate_up, void* stream);

/* Routing of T tokens over E <= 256 experts, in fp32: p = softmax(logits[t, :E]); the top_k
 * largest p in descending order (equal p: lower expert id first); with renormalize,
 * w = p / max(sum of the selected p, 1e-8).  logits: [T, ld] of logits_dtype (F16, BF16, F32).
 * topk_weights: [T, top_k] fp32; topk_ids: [T, top_k] int32. */
int awq_w4a16_moe_route(const void* logits, int64_t ld, int32_t logits_dtype, int64_t T, int32_t E,
                        int32_t top_k, int32_t renormalize, float* topk_weights, int32_t* topk_ids,
                        void* stream);

/* Routing flags of awq_w4a16_moe_route_ex. */
#define AWQ_ROUTE_RENORMALIZE 1u             /* w = p / (sum of the selected p) */
#define AWQ_ROUTE_SOFTMAX_IN_LOGITS_DTYPE 2u /* fused_moe's flow for 16-bit logits (below) */
#define AWQ_ROUTE_CLAMP_SUM 4u               /* renormalise by max(sum, 1e-8) (the Gemma4 router) */

/* Routing with the reference's two dtype flows:
 *  - without AWQ_ROUTE_SOFTMAX_IN_LOGITS_DTYPE (or for F32 logits): the Gemma4 router
 *    (vllm/model_executor/models/gemma4/moe.py:106-123): p = softmax(fp32(logits)) in fp32,
 *    top_k in descending order (equal p: lower expert id first), w = p / sum (with
 *    AWQ_ROUTE_CLAMP_SUM: / max(sum, 1e-8)) in fp32, then w converted to weights_dtype
 *    (round to nearest even; the router casts to the hidden dtype, moe.py:123);
 *  - with it: fused_moe (vllm/model_executor/layers/fused_moe/fused_moe.py:12-15) on 16-bit
 *    logits: p = softmax(logits) rounded once to the logits dtype (correctly rounded: exp and
 *    sum in fp64), top_k on those values (ties: lower expert id first), and with
 *    AWQ_ROUTE_RENORMALIZE w = dt(fp32(p) / fp32(dt(sum of the selected p))), torch's 16-bit
 *    arithmetic; stored in weights_dtype (exactly, for the logits dtype or F32).
 * topk_weights: [T, top_k] of weights_dtype (F32, F16 or BF16); topk_ids: [T, top_k] int32. */
int awq_w4a16_moe_route_ex(const void* logits, int64_t ld, int32_t logits_dtype, int64_t T, int32_t E,
                           int32_t top_k, uint32_t flags, void* topk_weights, int32_t weights_dtype,
                           int32_t* topk_ids, void* stream);

/* Workspace bytes of awq_w4a16_moe (route lists, the intermediate and per-route fp32 rows). */
size_t awq_w4a16_moe_workspace_bytes(int64_t T, int64_t H, int64_t I, int32_t E, int32_t top_k);

/* out[t] = sum over j of w[t, j] * down_e(act(gate_e(x[t])) * up_e(x[t])), e = ids[t, j]:
 *   gate/up = x . dequant(W1_e)^T in fp32; h = act(gate) * up * w in fp32, rounded once to
 *   act_dtype (the intermediate the reference keeps in x.dtype); y = h . dequant(W2_e)^T in
 *   fp32 per route; out = one rounding of the sum of a token's y in slot order.  Weights are
 *   dequantized exactly as awq_w4a16_dequant does.  Routes whose id is outside [0, E)
 *   contribute nothing.  Results are bitwise reproducible.
 *   x: [T, ldx] act_dtype (F16 or BF16); out: [T, ldo] act_dtype.
 *   topk_ids: [T, top_k] int32 or int64 (ids_bits 32 / 64); topk_weights: [T, top_k] of
 *   weights_dtype (F16, BF16 or F32).
 *   gate_up_stream / down_stream: awq_w4a16_moe_pack_stream outputs; scales of scale_dtype;
 *   qzeros both NULL (symmetric, z = 8) or both given.
 *   group_size 32, 64 or 128 dividing H and I; H % 8 == 0, I % 8 == 0.
 *   workspace: awq_w4a16_moe_workspace_bytes bytes, 256-byte aligned (no zeroing needed). */
int awq_w4a16_moe(const void* x, int64_t ldx, const void* topk_ids, int32_t ids_bits, const void* topk_weights,
                  int32_t weights_dtype, const int32_t* gate_up_stream, const void* gate_up_scales,
                  const int32_t* gate_up_qzeros, const int32_t* down_stream, const void* down_scales,
                  const int32_t* down_qzeros, void* out, int64_t ldo, int64_t T, int64_t H, int64_t I,
                  int32_t E, int32_t top_k, int32_t group_size, int32_t activation, int32_t act_dtype,
                  int32_t scale_dtype, void* workspace, size_t workspace_bytes, void* stream);

/* ---- dense gated MLP (gate and up projections with the activation fused) -------------
 * Replaces the reference's M = 1 fused gate/up kernels (vllm/kernels/triton/awq_fused_gemm.py:
 * 1406-1506 and 1509-1590, launched by packed_int4_symmetric_fused_gate_up_m1 and
 * ..._group32_m1 at 3009-3120): out[m, n] = act(x[m] . Wg[n]) * (x[m] . Wu[n]), both sums in
 * fp32 over unrounded weights (q - z) * s, one rounding at the end.
 * The two projections travel as one interleaved matrix of 2 * ceil(I / 64) * 64 columns:
 * block b of 128 columns holds gate columns [64 b, 64 b + 64) followed by the up columns of the
 * same outputs (columns past I are zero).  awq_w4a16_gate_up_interleave builds it from the two
 * AUTOAWQ matrices. */

/* Interleave two row-major [rows, cols] matrices of elem_bytes-byte elements (2 or 4) into
 * [rows, 2 * ceil(cols / half_tile) * half_tile]: each run of 2 * half_tile elements is
 * half_tile elements of gate followed by the same half_tile elements of up, zero past cols.
 * half_tile 8 for qweight / qzeros [K, I/8] words, 64 for scales [K/G, I].  No counterpart in
 * the reference (its kernel reads the two matrices separately); it is the derived pack the
 * reference would cache on the weight pair (tensor.py:1251-1256). */
int awq_w4a16_gate_up_interleave(const void* gate, const void* up, void* out, int64_t rows, int64_t cols,
                                 int32_t elem_bytes, int32_t half_tile, void* stream);

/* Workspace of awq_w4a16_gate_up_act: that of awq_w4a16_gemm for the interleaved matrix,
 * N = 2 * ceil(I / 64) * 64 (same zeroing rule); 0 for DECODE_NARROW. */
size_t awq_w4a16_gate_up_workspace_bytes(int64_t M, int64_t I, int64_t K, int32_t group_size,
                                         int32_t split_k, int32_t layout);

/* out[M, I] = act(x . Wg^T) * (x . Wu^T), activation AWQ_MOE_ACT_SILU or AWQ_MOE_ACT_GELU_TANH
 * (the tanh form, computed as g * sigmoid(2 * inner) like awq_fused_gemm.py:1493-1502).
 *   x: [M, K] act_dtype (F16 or BF16), row stride ldx; out: [M, I] act_dtype, row stride ldo.
 *   qweight / scales / qzeros: the interleaved matrix in layout AUTOAWQ or KN_SEQ
 *   ([K, N/8] words, N = 2 * ceil(I / 64) * 64) or DECODE_STREAM (its awq_w4a16_pack_decode_stream
 *   copy); or DECODE_NARROW: the pair interleaved per 8 columns instead (half_tile 1 for
 *   words, 8 for scales; N = 2 * ceil(I / 8) * 8), qweight as its awq_w4a16_pack_decode_narrow
 *   copy, no workspace.  qzeros NULL = symmetric z = 8 (the reference's mode).
 *   1 <= M <= 32 (the reference takes M == 1); group_size 32, 64 or 128 dividing K.
 *   split_k as for awq_w4a16_gemm; results are bitwise reproducible for a given split. */
int awq_w4a16_gate_up_act(const void* x, int64_t ldx, const int32_t* qweight, const void* scales,
                          const int32_t* qzeros, void* out, int64_t ldo, int64_t M, int64_t I, int64_t K,
                          int32_t group_size, int32_t split_k, int32_t layout, int32_t activation,
                          int32_t act_dtype, int32_t scale_dtype, void* workspace, size_t workspace_bytes,
                          void* stream);

/* ---- RMSNorm prologue ---------------------------------------------------------
 * xn[M, K] (fp16) = fp16_rne((fp32(x) * rrms) * fp32(norm_w)), rrms = rsqrt(var / K + eps),
 * var = the fp32 sum of fp32(x)^2 over the row: the arithmetic of rmsnorm_awq_fused.py:108-131
 * (the normalised row is fp16 whatever x's dtype, rmsnorm_awq_fused.py:168).
 *   x: [M, K] act_dtype (F16 or BF16), row stride ldx; norm_w: [K] norm_dtype (F16 or BF16);
 *   xn: [M, K] fp16, row stride ldxn.  K % 8 == 0; x, norm_w and xn 16-byte aligned, strides
 *   multiples of 8. */
int awq_w4a16_rmsnorm(const void* x, int64_t ldx, const void* norm_w, float eps, void* xn, int64_t ldxn,
                      int64_t M, int64_t K, int32_t act_dtype, int32_t norm_dtype, void* stream);

/* Workspace of awq_w4a16_rmsnorm_gemm: awq_w4a16_gemm's (same zeroing rule, at offset 0, and
 * never less than its 64 KiB counter region, so one workspace can serve both functions), then
 * the normalised rows [M, K] fp16, then for BF16 activations the fp16 product [M, N]; each
 * part starts on a 256-byte boundary and the workspace itself on one. */
size_t awq_w4a16_rmsnorm_gemm_workspace_bytes(int64_t M, int64_t N, int64_t K, int32_t group_size,
                                              int32_t split_k, int32_t layout, int32_t act_dtype);

/* C[M, N] = RMSNorm(x; norm_w, eps) . dequant(W)^T, rmsnorm_awq_fused_linear's result:
 * awq_w4a16_rmsnorm into the workspace, then awq_w4a16_gemm on the fp16 rows (any layout it
 * takes, no bias), C rounded to fp16; for BF16 activations that fp16 result is converted to
 * bf16 (round to nearest even), as the reference's store into a bf16 output does
 * (rmsnorm_awq_fused.py:170-175).  C: [M, N] act_dtype, row stride ldc.  Three launches at
 * most, all on `stream`; one for the DECODE_NARROW layout with F16 activations and scales and
 * M = 1, whose kernel normalises the row it stages (when the row fits its LDS). */
int awq_w4a16_rmsnorm_gemm(const void* x, int64_t ldx, const void* norm_w, float eps,
                           const int32_t* qweight, const void* scales, const int32_t* qzeros, void* c,
                           int64_t ldc, int64_t M, int64_t N, int64_t K, int32_t group_size, int32_t split_k,
                           int32_t layout, int32_t act_dtype, int32_t norm_dtype, int32_t scale_dtype,
                           void* workspace, size_t workspace_bytes, void* stream);

#ifdef __cplusplus
}
#endif

#endif /* AWQ_W4A16_H */
