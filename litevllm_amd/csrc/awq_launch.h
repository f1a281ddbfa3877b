// Host-side planning and launch interfaces shared by the translation units of
// libawq_w4a16.so (internal; the public interface is include/awq_w4a16.h).
#pragma once

#include <hip/hip_runtime.h>
#include <stddef.h>
#include <stdint.h>

#include "awq_common.h"

namespace awq_host {

// Workspace layout of the decode kernel: [0, kCounterBytes) per-tile arrival counters (zero
// between calls), then fp32 partials [tiles, splits, M, 128].
constexpr size_t kCounterBytes = 65536;

struct DecodePlan {
  int mt;  // 16-token MFMA tiles
  int tiles, ksteps, splits, per, blocks;  // per: k-steps of 32 rows in each split's range
  size_t ws_bytes;
};

// Which instantiations of the decode kernel serve a call:
//   kDecodeStream : weights in the decode stream layout (AutoAWQ nibble order)
//   kDecodeWide   : AutoAWQ [K, N/8], f16 activations and scales (every tile width)
//   kDecodeNarrow : the other dtype / layout combinations (one word per lane)
enum DecodeMode { kDecodeStream = 0, kDecodeWide = 1, kDecodeNarrow = 2 };
inline DecodeMode decode_mode(int layout, int act, int sdt) {
  if (layout == AWQ_LAYOUT_DECODE_STREAM) return kDecodeStream;
  if (layout == AWQ_LAYOUT_AUTOAWQ && act == AWQ_DTYPE_F16 && sdt == AWQ_DTYPE_F16) return kDecodeWide;
  return kDecodeNarrow;
}
DecodePlan plan_decode(int64_t M, int64_t N, int64_t K, int64_t G, int split_k, DecodeMode mode);
bool launch_decode(const awq::GemmArgs& a, const DecodePlan& s, DecodeMode mode, bool seq, bool zp,
                   int act, int sdt, hipStream_t st);
// bf16 scales or bf16 activations (sbf: scales are bf16); AUTOAWQ / KN_SEQ and stream layouts
bool launch_decode_misc(const awq::GemmArgs& a, const DecodePlan& s, bool seq, bool zp, int act, int sbf,
                        hipStream_t st);
bool launch_decode_misc_stream(const awq::GemmArgs& a, const DecodePlan& s, bool zp, int act, int sbf,
                               hipStream_t st);

// Decode stream layout (tile = 16 packed words = 128 columns): the (tile t, k-step s) run of
// 2048 bytes starts at byte (t * K/32 + s) * 2048.  Lane l = 16 q + r owns word 16 t + r
// (zero past the last word) of rows 32 s + 8 q + j, j < 8, stored pre-paired for the
// kernel's magic-exponent unpack: its u32 number v < 4 is lo16(row 2v) | lo16(row 2v+1) << 16
// and number 4 + v is hi16(row 2v) | hi16(row 2v+1) << 16.  Numbers 4 e .. 4 e + 3 (piece e)
// sit at byte 1024 e + 16 l of the run, so every KiB is one piece of all 64 lanes.
inline int64_t decode_stream_bytes(int64_t K, int64_t N) { return awq::cdiv(N / 8, 16) * 16 * K * 4; }
int launch_pack_decode_stream(const int32_t* qweight_kn, int32_t* out, int64_t K, int64_t N, hipStream_t st);

// Narrow decode layout (16-column tiles in 1 KiB runs of four 32-row k-steps, 16 bytes per
// lane; documented in awq_decode_narrow.hip) and its kernel: M <= 32, group sizes 32/64/128,
// K % 32 == 0.
int64_t decode_narrow_bytes(int64_t K, int64_t N);
int launch_pack_decode_narrow(const int32_t* qweight_kn, int32_t* out, int64_t K, int64_t N, hipStream_t st);
bool launch_decode_narrow(const awq::GemmArgs& a, bool zp, int act, int sdt, hipStream_t st);
bool launch_decode_narrow_norm(const awq::GemmArgs& a, bool zp, hipStream_t st);

// Prefill GEMM (M > 32 or group sizes the decode kernel does not cover).
bool launch_prefill(const awq::GemmArgs& a, bool seq, bool zp, int act, int sdt, hipStream_t st);
// Prefill GEMM on the decode stream layout (awq_prefill.hip): M > 32, K % 32 == 0.
bool launch_prefill_stream(const awq::GemmArgs& a, bool zp, int act, int sdt, hipStream_t st);

// Standalone dequant and repack.
int launch_dequant(const int32_t* qweight, const void* scales, const int32_t* qzeros, void* out,
                   int64_t rows, int64_t cols, int32_t group_size, int32_t layout,
                   int32_t scale_dtype, int32_t out_dtype, hipStream_t st);
int launch_repack_nk_to_autoawq(const int32_t* qweight_nk, const int32_t* qzeros_nk,
                                const void* scales_nk, int32_t* qweight_kn, int32_t* qzeros_kn,
                                void* scales_kn, int64_t N, int64_t K, int32_t group_size,
                                hipStream_t st);

// Roofline probe: a launch that only reads `bytes` (awq_w4a16_probe_read).
int launch_probe_read(const void* buf, int64_t bytes, int blocks, int threads, int in_flight, void* sink,
                      hipStream_t st);

// Gate/up interleave of the gated decode epilogue (elem_bytes 2 or 4).
int launch_gate_up_interleave(const void* gate, const void* up, void* out, int64_t rows, int64_t cols,
                              int elem_bytes, int64_t half, hipStream_t st);

// RMSNorm prologue (one block per row, normalised fp16 rows out) and fp16 -> bf16 conversion.
int launch_rmsnorm_rows(const void* x, int64_t ldx, const void* nw, float eps, void* xn, int64_t ldo, int64_t M,
                        int64_t K, int act, int ndt, hipStream_t st);
int launch_f16_to_bf16(const void* in, int64_t ldi, void* out, int64_t ldo, int64_t M, int64_t N, hipStream_t st);

// ---- mixture of experts ----
// Stream-packed expert stacks: gate_up (N = 2I) pairs 8 gate words with the 8 up words of the
// same columns per tile (tiles = ceil(I / 64)); down (gate_up = 0) uses tiles of 16 words.
int64_t moe_tiles(int64_t N, int gate_up);
int64_t moe_stream_bytes(int64_t E, int64_t K, int64_t N, int gate_up);
int launch_moe_pack_stream(const int32_t* in, int32_t* out, int64_t E, int64_t K, int64_t N, int gate_up,
                           hipStream_t st);
int launch_moe_route(const void* logits, int64_t ld, int dtype, int64_t T, int E, int topk, uint32_t flags,
                     void* out_w, int w_dtype, int32_t* out_ids, hipStream_t st);

// Workspace of one MoE call (byte offsets): route counts [E] and lists [E][R] (int32), the
// intermediate [R][I] (activation dtype) and the per-route down outputs [R][H] (fp32).
struct MoeWorkspace {
  int64_t counts, lists, tmp, y, total;
};
MoeWorkspace moe_workspace(int64_t T, int64_t H, int64_t I, int E, int topk, int act_bytes);

struct MoeCall {
  const void* x;
  int64_t ldx;
  const void* ids;
  int id64;
  const void* rw;
  int rw_dtype;
  const int32_t *gu_qw, *gu_qz, *dn_qw, *dn_qz;
  const void *gu_sc, *dn_sc;
  void* out;
  int64_t ldo, T, H, I;
  int E, topk, G, act_kind, act_dtype, scale_dtype;
  void* workspace;
};
int launch_moe(const MoeCall& c, hipStream_t st);

}  // namespace awq_host
