// Decode planning and the fp16 (activations and scales) instantiations of the decode kernel
// (awq_decode_kernel.h); the other dtype combinations live in awq_decode_misc.hip.
#include "awq_decode_kernel.h"

namespace awq_host {
using namespace awq;

// ---- planning ----
// Blocks of 8 waves (two per SIMD) with a two-deep ring.  By default the block count is the
// largest tiles x s (s dividing the chunks of one tile) that fits the CUs, so block ranges
// start and end on tile boundaries and no tile is split unevenly; when that leaves more
// than half the CUs idle, one block per CU with ranges that straddle tiles.  With
// split_k > 0 each tile's K range is cut into split_k block ranges.  Units are dealt in
// chunks of waves x ring depth when that divides the k-steps of a tile (the kernel applies
// the same rule), and there are at least as many blocks as tiles, so no block's range is
// longer than one tile and none touches more than two.
DecodePlan plan_decode(int64_t M, int64_t N, int64_t K, int64_t G, int split_k, DecodeMode mode) {
  (void)G;
  DecodePlan s{};
  s.mt = (M > 16) ? 2 : 1;
  s.nwv = 8;
  s.depth = 2;
  s.occ = 2;
  s.wpl = mode == kDecodeStream ? decode_stream_wpl(N) : 1;
  s.tiles = (int)cdiv(N / 8, 16 * s.wpl);
  s.ksteps = (int)(K / 32);
  const int64_t KS = s.ksteps;
  const int64_t U = (int64_t)s.tiles * KS;
  const int64_t chunk = decode_chunk((int)KS, s.nwv, s.depth);
  const int64_t C = U / chunk;
  int64_t blocks;
  if (split_k > 0) {
    blocks = (int64_t)s.tiles * std::min<int64_t>(split_k, KS / chunk);
  } else {
    const int64_t cus = (int64_t)num_cus();
    const int64_t per_tile = KS / chunk;
    int64_t aligned = s.tiles;
    for (int64_t d = 1; d <= per_tile; ++d)
      if (per_tile % d == 0 && (int64_t)s.tiles * d <= std::max<int64_t>(cus, s.tiles))
        aligned = (int64_t)s.tiles * d;
    blocks = (2 * aligned >= cus) ? aligned : cus;
  }
  blocks = std::max<int64_t>(s.tiles, std::min<int64_t>(blocks, C));
  s.blocks = (int)blocks;
  s.waves = (int)(blocks * s.nwv);
  // a tile of KS units meets at most ceil(KS / (chunk * floor(C / B))) + 1 block ranges
  const int64_t per_block = (C / blocks) * chunk;
  s.max_contrib = (int)std::min<int64_t>(blocks, cdiv(KS, per_block) + 1);
  // no tile is shared only when every range boundary falls on a tile boundary
  const bool shared = !((C % blocks) == 0 && (per_block % KS) == 0);
  s.ws_bytes = shared ? kCounterBytes + (size_t)s.tiles * (size_t)s.max_contrib * (size_t)M *
                                            (size_t)(128 * s.wpl) * sizeof(float)
                      : 0;
  return s;
}

bool launch_decode(const GemmArgs& a, const DecodePlan& s, DecodeMode mode, bool seq, bool zp,
                   int act, int sdt, hipStream_t st) {
  const int sbf = (sdt == AWQ_DTYPE_BF16) ? 1 : 0;
  if (mode == kDecodeStream) {
    if (seq || act != AWQ_DTYPE_F16 || sdt != AWQ_DTYPE_F16) return false;
    return zp ? launch_sel<false, true, f16, true, true>(a, s, 0, st) : launch_sel<false, false, f16, true, true>(a, s, 0, st);
  }
  if (act == AWQ_DTYPE_F16 && sdt == AWQ_DTYPE_F16) {
    if (seq) return zp ? launch_sel<true, true, f16, true, false>(a, s, 0, st) : launch_sel<true, false, f16, true, false>(a, s, 0, st);
    return zp ? launch_sel<false, true, f16, true, false>(a, s, 0, st) : launch_sel<false, false, f16, true, false>(a, s, 0, st);
  }
  return launch_decode_misc(a, s, seq, zp, act, sbf, st);
}

}  // namespace awq_host
