// Host entry points of the row-team GEMV (kernels in gemv_team.h,
// instantiated per format and activation mode in gemv_team_*.hip) and the
// prepared-layout block-dot debug kernel.
#include "gemv_team.h"

namespace mdma {
namespace {

// Debug: int32 dot per (token, row, sub-block) from prepared rows, one
// thread per (token, row, unit), through the same plane loads as the GEMV.
__global__ __launch_bounds__(256) void block_dot_prepared_kernel(int32_t dtype, const uint8_t *__restrict__ w,
                                                                 uint32_t n_out, uint32_t n_in,
                                                                 const int8_t *__restrict__ qx, uint32_t T,
                                                                 int32_t *__restrict__ out) {
  const uint32_t U = dtype == DT_Q8_0 ? n_in / 32 : n_in / 64, nsub = dtype == DT_Q6_K ? n_in / 16 : n_in / 32;
  const size_t idx = (size_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (idx >= (size_t)T * n_out * U) return;
  const uint32_t u = idx % U, row = (idx / U) % n_out, t = idx / ((size_t)U * n_out);
  const int8_t *xt = qx + (size_t)t * n_in;
  int32_t *o = out + ((size_t)t * n_out + row) * nsub;
  if (dtype == DT_Q4_K) {
    const Q4G::W wv = Q4G::load(w + row * Q4G::row_bytes(n_in), u, U);
    const uint32_t q[8] = {wv.a.x, wv.a.y, wv.a.z, wv.a.w, wv.b.x, wv.b.y, wv.b.z, wv.b.w};
    int ia = 0, ib = 0;
    for (int k = 0; k < 8; k++) {
      ia = __builtin_amdgcn_sdot4((int)(q[k] & 0x0F0F0F0Fu), *reinterpret_cast<const int *>(xt + 64 * u + 4 * k), ia, false);
      ib = __builtin_amdgcn_sdot4((int)((q[k] >> 4) & 0x0F0F0F0Fu), *reinterpret_cast<const int *>(xt + 64 * u + 32 + 4 * k), ib, false);
    }
    o[2 * u] = ia;
    o[2 * u + 1] = ib;
  } else if (dtype == DT_Q6_K) {
    const Q6G::W wv = Q6G::load(w + row * Q6G::row_bytes(n_in), u, U);
    for (int r = 0; r < 4; r++) {
      const int8_t *xr = xt + Q6G::col(u, r);
      int s = 0, sx = 0;
      for (int k = 0; k < 4; k++) {
        const int xv = *reinterpret_cast<const int *>(xr + 4 * k);
        s = __builtin_amdgcn_sdot4((int)Q6G::u6(wv, r, k), xv, s, false);
        sx = __builtin_amdgcn_sdot4(xv, 0x01010101, sx, false);
      }
      o[Q6G::col(u, r) / 16] = s - 32 * sx;
    }
  } else {
    const Q8G::W wv = Q8G::load(w + row * Q8G::row_bytes(n_in), u, U);
    const uint32_t q[8] = {wv.a.x, wv.a.y, wv.a.z, wv.a.w, wv.b.x, wv.b.y, wv.b.z, wv.b.w};
    int s = 0;
    for (int k = 0; k < 8; k++)
      s = __builtin_amdgcn_sdot4((int)q[k], *reinterpret_cast<const int *>(xt + 32 * u + 4 * k), s, false);
    o[u] = s;
  }
}

}  // namespace

void launch_block_dot_prepared(mdma_ctx *ctx, const GemvJob &w, const int8_t *qx, uint64_t T, int32_t *out) {
  const uint64_t U = w.dtype == DT_Q8_0 ? w.n_in / 32 : w.n_in / 64, total = T * w.n_out * U;
  if (!total) return;
  block_dot_prepared_kernel<<<dim3((uint32_t)((total + 255) / 256)), dim3(256), 0, ctx->stream>>>(
      w.dtype, w.w, (uint32_t)w.n_out, (uint32_t)w.n_in, qx, (uint32_t)T, out);
  hip_check(hipGetLastError(), "block_dot launch");
}

bool launch_gemv_i8_x(mdma_ctx *ctx, const GemvJob *jobs, int n_jobs, bool gated, const float *x, float *ygated) {
  if (!team_layout_ok(jobs, gated ? 2 : n_jobs)) return false;
  const int32_t dt = jobs[0].dtype;
  if ((dt != DT_Q4_K && dt != DT_Q6_K) || jobs[0].n_in % 256) return false;
  // Multi-wave teams (n_in > 4096) quantize each wave's own units; one-wave
  // teams quantize x once per workgroup in LDS (every wave of it needs all
  // of x), which keeps the f32 reads of x off the L2 hot spot that one read
  // per wave makes of them.
  launch_gemv_team(ctx, MDMA_ACT_I8, jobs, n_jobs, gated, x, 1, ygated, true);
  return true;
}

uint32_t launch_gemv_i8_residual(mdma_ctx *ctx, const GemvJob &job, const float *x, const float *res) {
  if (!team_layout_ok(&job, 1) || job.n_in % 256 || !job.y) return 0;
  const int32_t dt = job.dtype;
  // x quantized in the kernel's prologue unless its int8 form is cached
  // (Q8_0 has no in-kernel form: its x is quantized separately).
  const bool pro = dt != DT_Q8_0 && !q8_holds(ctx, x, job.n_in);
  TeamNorm nm;
  nm.res = res;
  nm.ssq = ssq_parts(ctx, 65536);
  nm.ssq_cap = (uint32_t)(ctx->ssq_cap < 65536 ? ctx->ssq_cap : 65536);
  ctx->team_grid = 0;
  // The launcher makes no launch whose grid passes ssq_cap (team_grid stays
  // 0: the caller takes the unfused path).
  launch_gemv_team(ctx, MDMA_ACT_I8, &job, 1, false, x, 1, nullptr, pro, &nm);
  return ctx->team_grid;
}

bool launch_gemv_i8_normed(mdma_ctx *ctx, const GemvJob *jobs, int n_jobs, const float *nsum, const float *nw,
                           uint32_t n_part, float eps) {
  if (!team_layout_ok(jobs, n_jobs) || !n_part || n_part > 256) return false;
  const uint64_t n_in = jobs[0].n_in;
  // One-wave teams of Q4_K / Q6_K rows (64-column units), whole 256-groups.
  if ((jobs[0].dtype != DT_Q4_K && jobs[0].dtype != DT_Q6_K) || n_in % 256 || n_in / 64 > 64) return false;
  TeamNorm nm;
  nm.nsum = nsum;
  nm.nw = nw;
  nm.npart = ssq_parts(ctx, n_part);
  nm.n_part = n_part;
  nm.eps = eps;
  launch_gemv_team(ctx, MDMA_ACT_I8, jobs, n_jobs, false, nsum, 1, nullptr, false, &nm);
  return true;
}

bool team_layout_ok(const GemvJob *jobs, int n_jobs) {
  for (int i = 0; i < n_jobs; i++)
    if (jobs[i].layout != MDMA_LAYOUT_GFX950 || jobs[i].dtype != jobs[0].dtype || jobs[i].n_in != jobs[0].n_in)
      return false;
  // Units per row: at most 4 per lane of a 4-wave team.
  const uint64_t ucols = jobs[0].dtype == DT_Q8_0 ? 32 : 64;
  return jobs[0].n_in / ucols <= 1024;
}

void launch_gemv_team(mdma_ctx *ctx, int mode, const GemvJob *jobs, int n_jobs, bool gated, const float *x,
                      uint64_t T, float *ygated, bool pro, const TeamNorm *nm) {
  const uint64_t n_in = jobs[0].n_in;
  int8_t *qx = nullptr;
  float *dx = nullptr;
  int32_t *s16 = nullptr;
  const bool f32 = mode != MDMA_ACT_I8;
  const int32_t dt = jobs[0].dtype;
  if (!f32 && !pro && !(nm && nm->nsum)) quantize_into_scratch(ctx, x, T, n_in, &qx, &dx, &s16);
  for (uint64_t t0 = 0; t0 < T; t0 += 8) {
    const uint32_t tn = (uint32_t)(T - t0 < 8 ? T - t0 : 8);
    TeamSet ts{};
    ts.pro = pro;
    if (nm) {  // one token only (the callers check)
      ts.res = nm->res;
      ts.ssq = nm->ssq;
      ts.ssq_cap = nm->ssq_cap;
      ts.nsum = nm->nsum;
      ts.nw = nm->nw;
      ts.npart = nm->npart;
      ts.n_part = nm->n_part;
      ts.eps = nm->eps;
    }
    ts.n = gated ? 1 : n_jobs;  // gated: teams cover the gate rows and also read up
    ts.n_in = (uint32_t)n_in;
    for (int i = 0; i < (gated ? 2 : n_jobs); i++) {
      ts.j[i].w = jobs[i].w;
      ts.j[i].y = jobs[i].y ? jobs[i].y + t0 * jobs[i].n_out : nullptr;
      ts.j[i].n_out = (uint32_t)jobs[i].n_out;
      ts.j[i].dots = jobs[i].dots ? jobs[i].dots + t0 * jobs[i].n_out * dot_subs(dt, n_in) : nullptr;
    }
    const float *xt = x + t0 * n_in;
    const int8_t *qt = qx ? qx + t0 * n_in : nullptr;
    const float *dt_ = dx ? dx + t0 * (n_in / 256) : nullptr;
    const int32_t *st = s16 ? s16 + t0 * (n_in / 16) : nullptr;
    float *yg = gated ? ygated + t0 * jobs[0].n_out : nullptr;
    const TeamSetArgs a{&ts, xt, qt, dt_, st, tn, yg};
    if (dt == DT_Q4_K) (f32 ? team_launch_q4_f32 : team_launch_q4_i8)(ctx, gated, a);
    else if (dt == DT_Q6_K) (f32 ? team_launch_q6_f32 : team_launch_q6_i8)(ctx, gated, a);
    else if (dt == DT_Q8_0) (f32 ? team_launch_q8_f32 : team_launch_q8_i8)(ctx, gated, a);
    else fail(MDMA_ERR_NOT_IMPLEMENTED, "gemv: dtype has no prepared layout");
  }
}

}  // namespace mdma
