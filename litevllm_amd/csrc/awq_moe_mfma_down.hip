// Grouped MoE GEMMs for many routes per expert: the down kernels (moe_tile_kernel,
// awq_moe_tile.h), compiled apart from gate_up so the two build in parallel.
#include "awq_moe_tile.h"

namespace awq_host {

void launch_moe_tile_down(const awq::MoeArgs& dn, int E, bool zp, int act, int sbf, hipStream_t st) {
  launch_moe_tile_mode<1>(dn, E, zp, act, sbf, st);
}

}  // namespace awq_host
