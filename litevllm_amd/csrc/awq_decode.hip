// Decode planning and the fp16 (activations and scales) instantiations of the decode kernel
// (awq_decode_kernel.h), stream layout included; the other dtype combinations live in
// awq_decode_misc.hip.
#include "awq_decode_kernel.h"

namespace awq_host {
using namespace awq;

// ---- planning ----
// Each tile's K is cut into `splits` ranges by the reference's split-K rule
// (awq_fused_gemm.py:1798-1800, BLOCK_K = 64): ceil(ceil(K / 64) / splits) blocks of 64 rows
// per range, the last ones shorter or empty, one block of waves each (16 waves at four per
// SIMD for M == 1, 8 at two per SIMD otherwise; a two-deep ring).  split_k > 0 asks for that
// many ranges.  By default a range gets about 32 k-steps (1024 rows), and no more ranges than
// fit one round of blocks on the chip (CUs / tiles, at least 1): a second round of blocks, or
// ranges so short that the split hand-off's memory round trips outweigh the extra CUs, were
// both measured slower (split-K sweeps over K = 2816 .. 14336, N = 1024 .. 24576).
DecodePlan plan_decode(int64_t M, int64_t N, int64_t K, int64_t G, int split_k, DecodeMode mode) {
  (void)G;
  (void)mode;
  DecodePlan s{};
  s.mt = (M > 16) ? 2 : 1;
  s.tiles = (int)cdiv(N / 8, 16);
  s.ksteps = (int)(K / 32);
  const int64_t kb = cdiv(K, 64);  // 64-row blocks
  // past one 64-row block per range the reference's extra ranges are empty: not launched
  const int64_t fit = std::max<int64_t>(1, (int64_t)num_cus() / s.tiles);
  const int64_t by_k = std::max<int64_t>(1, (s.ksteps + 16) / 32);
  const int64_t splits = std::min<int64_t>(kb, split_k > 0 ? (int64_t)split_k : std::min(by_k, fit));
  s.splits = (int)splits;
  s.per = (int)(2 * cdiv(kb, splits));
  s.blocks = (int)((int64_t)s.tiles * splits);
  s.ws_bytes = splits > 1 ? kCounterBytes + (size_t)s.tiles * (size_t)splits * (size_t)M * 128 * sizeof(float) : 0;
  return s;
}

bool launch_decode(const GemmArgs& a, const DecodePlan& s, DecodeMode mode, bool seq, bool zp,
                   int act, int sdt, hipStream_t st) {
  if (mode == kDecodeStream) {
    if (seq) return false;
    if (act != AWQ_DTYPE_F16 || sdt != AWQ_DTYPE_F16)
      return launch_decode_misc_stream(a, s, zp, act, sdt == AWQ_DTYPE_BF16 ? 1 : 0, st);
    return zp ? launch_sel<false, true, f16, false, true, true>(a, s, st)
              : launch_sel<false, false, f16, false, true, true>(a, s, st);
  }
  if (act == AWQ_DTYPE_F16 && sdt == AWQ_DTYPE_F16) {
    if (seq) return zp ? launch_sel<true, true, f16, false, false, true>(a, s, st) : launch_sel<true, false, f16, false, false, true>(a, s, st);
    return zp ? launch_sel<false, true, f16, false, false, true>(a, s, st) : launch_sel<false, false, f16, false, false, true>(a, s, st);
  }
  return launch_decode_misc(a, s, seq, zp, act, sdt == AWQ_DTYPE_BF16 ? 1 : 0, st);
}

}  // namespace awq_host
