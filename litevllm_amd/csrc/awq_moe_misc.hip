// bf16-activation and bf16-scale instantiations of the grouped MoE GEMM kernels
// (awq_moe_kernel.h), two 16-token tiles per wave group.
#include "awq_moe_kernel.h"

namespace awq_host {
using namespace awq;

template <int MODE, bool ZP, typename T>
static void launch_misc_t(const MoeArgs& a, int E, int sbf, hipStream_t st) {
  if (sbf) launch_moe_gemm_t<MODE, 2, ZP, T, true>(a, E, st);
  else launch_moe_gemm_t<MODE, 2, ZP, T, false>(a, E, st);
}

template <typename T>
static bool launch_pair(const MoeArgs& gu, const MoeArgs& dn, int E, bool zp, int sbf, hipStream_t st) {
  if (zp) launch_misc_t<0, true, T>(gu, E, sbf, st); else launch_misc_t<0, false, T>(gu, E, sbf, st);
  if (hipPeekAtLastError() != hipSuccess) return true;  // the caller reports the launch error
  if (zp) launch_misc_t<1, true, T>(dn, E, sbf, st); else launch_misc_t<1, false, T>(dn, E, sbf, st);
  return true;
}

bool launch_moe_misc(const MoeArgs& gu, const MoeArgs& dn, int E, bool zp, int act, int sbf, hipStream_t st) {
  if (act == AWQ_DTYPE_BF16) return launch_pair<bf16>(gu, dn, E, zp, sbf, st);
  if (act == AWQ_DTYPE_F16) return launch_pair<f16>(gu, dn, E, zp, sbf, st);
  return false;
}

}  // namespace awq_host
