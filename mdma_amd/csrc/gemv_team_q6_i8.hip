// Row-team GEMV instantiations: Q6G weights, int8 activations.
#include "gemv_team.h"

namespace mdma {

void team_launch_q6_i8(mdma_ctx *ctx, bool gated, const TeamSetArgs &a) {
  launch_mode<Q6G, false>(ctx, gated, *static_cast<const TeamSet *>(a.ts), a.xf, a.qx, a.dx, a.s16, a.T, a.yg);
}

}  // namespace mdma
