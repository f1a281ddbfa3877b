// Grouped MoE GEMMs for many routes per expert: the gate_up kernels (moe_tile_kernel,
// awq_moe_tile.h) and the launcher of the gate_up / down pair.
#include "awq_moe_tile.h"

namespace awq_host {

void launch_moe_mfma(const awq::MoeArgs& gu, const awq::MoeArgs& dn, int E, bool zp, int act, int sbf, hipStream_t st) {
  launch_moe_tile_mode<0>(gu, E, zp, act, sbf, st);
  if (hipPeekAtLastError() != hipSuccess) return;
  launch_moe_tile_down(dn, E, zp, act, sbf, st);
}

}  // namespace awq_host
