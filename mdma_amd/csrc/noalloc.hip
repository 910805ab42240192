// The allocation-free variant of the int8-mode qmatmul, for callers that
// cannot allocate device memory (code under HIP graph capture, tight serving
// loops, harnesses that forbid hipMalloc). It has no counterpart in the
// reference.
//
// The scratch the int8 route needs -- x's int8 form with its scales and
// sub-block sums, or the prefill GEMM's per-32 inputs -- lives in the
// file-scope device array `scratch` below instead of the context's growable
// buffers. Each GPU the library runs on holds its own copy of the array
// until the process ends. Host code never uses the array's name as an
// address (on the host it is a stand-in, not a device pointer): at context
// creation hipGetSymbolAddress gives this device's address, which the
// context keeps and every launch uses.
//
// Every call on one GPU shares that GPU's array and each call overwrites
// what it reads before reading it (nothing in it needs to start at zero).
// Calls through one context run in its stream's order. Calls from several
// contexts on one GPU are ordered too: each GPU has one event, created at
// set-up with the array's address, that every call's stream waits for
// before its launches and records after them, under a host lock per GPU,
// so the calls' kernels run one call after another. Under stream capture
// the event is not used (a captured graph cannot wait for work outside
// it): a graph that holds this call races with calls from other contexts
// replayed or run at the same time on that GPU.
#include <algorithm>
#include <cstdio>
#include <mutex>

#include "internal.h"

namespace {
constexpr uint64_t STATIC_SCRATCH_BYTES = 8ull << 20;
}

static __device__ __align__(256) uint8_t scratch[STATIC_SCRATCH_BYTES];

namespace {

// This device's address of `scratch`, per device ordinal, resolved once,
// and the device's ordering event and host lock (the calls' order).
std::mutex g_setup_lock;
char *g_device_scratch[256] = {};
hipEvent_t g_order_event[256] = {};
std::mutex g_order_lock[256];

char *device_scratch(int device) {
  std::lock_guard<std::mutex> lk(g_setup_lock);
  if (device < 0 || device >= 256) mdma::fail(MDMA_ERR_BACKEND, "allocation-free scratch: device ordinal out of range");
  if (!g_device_scratch[device]) {
    void *ptr = nullptr;
    // The calling thread has `device` current (mdma_gfx950_create set it).
    hipError_t e = hipGetSymbolAddress(&ptr, HIP_SYMBOL(::scratch));
    mdma::hip_check(e, "hipGetSymbolAddress(static scratch)");
    if (!ptr) mdma::fail(MDMA_ERR_BACKEND, "hipGetSymbolAddress(static scratch) returned null");
    hipEvent_t ev = nullptr;
    mdma::hip_check(hipEventCreateWithFlags(&ev, hipEventDisableTiming), "allocation-free scratch: order event");
    g_order_event[device] = ev;
    g_device_scratch[device] = static_cast<char *>(ptr);
  }
  return g_device_scratch[device];
}

// While alive: the context's int8 routes use the fixed buffer, and the
// context's cached int8 activations (which live in another buffer) are set
// aside, then restored -- unless the call's output y overwrote the x they
// were made from.
struct FixedScratch {
  mdma_ctx *ctx;
  const mdma_buf *y;
  bool valid;
  const float *x;
  uint64_t n, n_in;
  FixedScratch(mdma_ctx *c, char *p, uint64_t cap, const mdma_buf *y_)
      : ctx(c), y(y_), valid(c->q8_valid), x(c->q8_x), n(c->q8_n), n_in(c->q8_n_in) {
    ctx->q8_valid = false;
    ctx->fixed_scratch = p;
    ctx->fixed_cap = cap;
  }
  ~FixedScratch() {
    ctx->fixed_scratch = nullptr;
    ctx->fixed_cap = 0;
    ctx->q8_valid = valid;
    ctx->q8_x = x;
    ctx->q8_n = n;
    ctx->q8_n_in = n_in;
    mdma::q8_invalidate_range(ctx, y->ptr, y->len);
  }
};

}  // namespace

namespace mdma {

void noalloc_setup(mdma_ctx *ctx) { ctx->static_scratch = device_scratch(ctx->device); }

}  // namespace mdma

extern "C" int mdma_gfx950_qmatmul_i8_noalloc(mdma_ctx *ctx, const mdma_qweight *w, const mdma_buf *x,
                                              mdma_buf *y) {
  try {
    if (!ctx || !w || !x || !y) mdma::shape_fail("qmatmul_i8_noalloc: null argument");
    std::lock_guard<std::recursive_mutex> g(ctx->lock);
    if (!ctx->static_scratch) mdma::fail(MDMA_ERR_BACKEND, "qmatmul_i8_noalloc: static scratch not set up");
    // The largest scratch either int8 route of this call can take: x's
    // per-256 form (decode GEMVs) or its per-32 form (the prefill GEMM).
    const uint64_t n = x->len / 4;
    const uint64_t need = std::max(mdma::q8_slot_bytes(n), mdma::gemm_input_bytes(n));
    if (need > STATIC_SCRATCH_BYTES) {
      char m[200];
      std::snprintf(m, sizeof m,
                    "qmatmul_i8_noalloc: x of %llu values needs %llu bytes of scratch; the static scratch holds %llu",
                    (unsigned long long)n, (unsigned long long)need, (unsigned long long)STATIC_SCRATCH_BYTES);
      mdma::fail(MDMA_ERR_BUFFER_BUDGET, m);
    }
    // Calls from other contexts on this GPU: their kernels first (not under
    // capture, see above).
    std::lock_guard<std::mutex> order(g_order_lock[ctx->device]);
    const hipEvent_t ev = g_order_event[ctx->device];
    if (!ctx->capturing) mdma::hip_check(hipStreamWaitEvent(ctx->stream, ev, 0), "qmatmul_i8_noalloc: order wait");
    {
      FixedScratch fs(ctx, ctx->static_scratch, STATIC_SCRATCH_BYTES, y);
      mdma::qmatmul_run(ctx, w, x, y, MDMA_ACT_I8);
    }
    if (!ctx->capturing) mdma::hip_check(hipEventRecord(ev, ctx->stream), "qmatmul_i8_noalloc: order record");
    return MDMA_OK;
  } catch (const mdma::Error &e) {
    mdma::set_last_error(e.msg);
    return e.code;
  } catch (...) {
    mdma::set_last_error("qmatmul_i8_noalloc: unknown failure");
    return MDMA_ERR_BACKEND;
  }
}
