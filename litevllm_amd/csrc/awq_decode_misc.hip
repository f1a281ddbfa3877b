// Decode kernel instantiations for bf16 scales or bf16 activations (the fp16 ones are in
// awq_decode.hip).
#include "awq_decode_kernel.h"

namespace awq_host {
using namespace awq;

bool launch_decode_misc(const GemmArgs& a, const DecodePlan& s, bool seq, bool zp, int act, int sbf,
                        hipStream_t st) {
  if (act == AWQ_DTYPE_F16) {  // bf16 scales
    if (seq) return zp ? launch_sel<true, true, f16, true, false, false>(a, s, st) : launch_sel<true, false, f16, true, false, false>(a, s, st);
    return zp ? launch_sel<false, true, f16, true, false, false>(a, s, st) : launch_sel<false, false, f16, true, false, false>(a, s, st);
  }
  if (sbf) {
    if (seq) return zp ? launch_sel<true, true, bf16, true, false, false>(a, s, st) : launch_sel<true, false, bf16, true, false, false>(a, s, st);
    return zp ? launch_sel<false, true, bf16, true, false, false>(a, s, st) : launch_sel<false, false, bf16, true, false, false>(a, s, st);
  }
  if (seq) return zp ? launch_sel<true, true, bf16, false, false, false>(a, s, st) : launch_sel<true, false, bf16, false, false, false>(a, s, st);
  return zp ? launch_sel<false, true, bf16, false, false, false>(a, s, st) : launch_sel<false, false, bf16, false, false, false>(a, s, st);
}

// The decode stream layout with bf16 scales or bf16 activations (M == 1 runs the 16-wave
// instantiation, as in the fp16 path).
bool launch_decode_misc_stream(const GemmArgs& a, const DecodePlan& s, bool zp, int act, int sbf, hipStream_t st) {
  if (act == AWQ_DTYPE_F16)  // bf16 scales
    return zp ? launch_sel<false, true, f16, true, true, true>(a, s, st) : launch_sel<false, false, f16, true, true, true>(a, s, st);
  if (sbf) return zp ? launch_sel<false, true, bf16, true, true, true>(a, s, st) : launch_sel<false, false, bf16, true, true, true>(a, s, st);
  return zp ? launch_sel<false, true, bf16, false, true, true>(a, s, st) : launch_sel<false, false, bf16, false, true, true>(a, s, st);
}

}  // namespace awq_host
