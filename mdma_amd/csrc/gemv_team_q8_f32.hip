// Row-team GEMV instantiations: Q8G weights, f32 activations.
#include "gemv_team.h"

namespace mdma {

void team_launch_q8_f32(mdma_ctx *ctx, bool gated, const TeamSetArgs &a) {
  launch_mode<Q8G, true>(ctx, gated, *static_cast<const TeamSet *>(a.ts), a.xf, a.qx, a.dx, a.s16, a.T, a.yg);
}

}  // namespace mdma
