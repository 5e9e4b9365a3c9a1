// C ABI of librmoe.so (declared in include/raon_moe.h): context, scratch, uploads
// and the entry points.  Host entry points validate every shape before any kernel
// is launched; "_dev" entry points validate shapes and scratch capacity and never
// allocate.
#include <stdarg.h>
#include <stdio.h>
#include <string.h>

#include <algorithm>
#include <mutex>
#include <set>

#include "../../include/raon_moe.h"
#include "rmoe_internal.h"

namespace {

thread_local std::string g_err;

int fail(int code, const char* fmt, ...) {
  char buf[512];
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(buf, sizeof(buf), fmt, ap);
  va_end(ap);
  g_err = buf;
  return code;
}

#define HIP_TRY(expr)                                                                        \
  do {                                                                                       \
    hipError_t _e = (expr);                                                                  \
    if (_e != hipSuccess) return fail(RMOE_EDEVICE, "%s: %s", #expr, hipGetErrorString(_e)); \
  } while (0)

hipStream_t pick_stream(rmoe_ctx* ctx, void* stream) { return stream ? (hipStream_t)stream : ctx->stream; }

// Grow-only device buffer of n elements of T (zero-filled when (re)allocated).
template <typename T>
int grow(T*& p, size_t& cap, size_t n, rmoe_ctx* ctx) {
  if (n <= cap && p) return RMOE_OK;
  if (p) {
    HIP_TRY(hipStreamSynchronize(ctx->stream));
    HIP_TRY(hipFree(p));
    p = nullptr;
    cap = 0;
  }
  size_t want = std::max<size_t>(n, 1);
  void* q = nullptr;
  if (hipMalloc(&q, want * sizeof(T)) != hipSuccess) return fail(RMOE_ENOMEM, "hipMalloc of %zu bytes failed", want * sizeof(T));
  // Zero on the context stream and wait: later launches may use other streams.
  HIP_TRY(hipMemsetAsync(q, 0, want * sizeof(T), ctx->stream));
  HIP_TRY(hipStreamSynchronize(ctx->stream));
  p = static_cast<T*>(q);
  cap = want;
  return RMOE_OK;
}

#define TRY(expr)              \
  do {                         \
    int _r = (expr);           \
    if (_r != RMOE_OK) return _r; \
  } while (0)

// Host <-> device io area for host entry points.
struct Io {
  uint8_t* p = nullptr;
  size_t cap = 0;
};
std::map<rmoe_ctx*, Io> g_io;

int io_area(rmoe_ctx* ctx, size_t bytes, uint8_t** out) {
  Io& io = g_io[ctx];
  TRY(grow(io.p, io.cap, bytes, ctx));
  *out = io.p;
  return RMOE_OK;
}

size_t align_up(size_t v, size_t a) { return (v + a - 1) / a * a; }

int check_layer(rmoe_ctx* ctx, int layer, RmoeLayer** out) {
  if (!ctx) return fail(RMOE_EINVAL, "null context");
  auto it = ctx->layers.find(layer);
  if (it == ctx->layers.end()) return fail(RMOE_ENOTFOUND, "layer %d is not an uploaded MoE layer", layer);
  *out = &it->second;
  return RMOE_OK;
}

// Linear partials/counters for T tokens on an [M, K] matrix (see q4_gemv.hip).
void linear_needs(int M, int K, int T, size_t& floats, size_t& counters) {
  const int nkt = K / rmoe::kTileCols, n_rt = M / rmoe::kTileRows;
  const int ksplit = (nkt + 3) / 4;
  const size_t ych = (size_t)(T + 3) / 4;
  floats = ych * n_rt * ksplit * 256;
  counters = ych * n_rt;
}

int reserve_stack(rmoe_ctx* ctx, const RmoeLayer& L, int n_layers);

// Size every scratch buffer for `layer` with up to T tokens and k routes.
int reserve_layer(rmoe_ctx* ctx, const RmoeLayer& L, int T, int k) {
  RmoeScratch& s = ctx->s;
  const int kk = std::max(k, L.top_k);
  size_t f1, c1, f2, c2;
  linear_needs(2 * L.I, L.H, T, f1, c1);
  linear_needs(L.H, L.Ipad, T, f2, c2);
  const size_t floats = std::max(f1, f2);
  const size_t counters = std::max({c1, c2, (size_t)T});  // K-split linear; one per routed token
  TRY(grow(s.part, s.part_floats, floats, ctx));
  TRY(grow(s.counters, s.n_counters, counters, ctx));
  TRY(grow(s.h, s.h_elems, (size_t)(kk + 1) * L.Ipad, ctx));
  size_t re = s.route_elems;
  TRY(grow(s.ids, re, (size_t)T * kk, ctx));
  re = s.route_elems;
  TRY(grow(s.wts, re, (size_t)T * kk, ctx));
  s.route_elems = re;
  TRY(grow(s.logits, s.logit_elems, (size_t)T * L.n_routed, ctx));
  const size_t nchunks = ((size_t)T * kk + 1023) / 1024;
  TRY(grow(s.chunk_counts, s.chunk_elems, nchunks * 256, ctx));
  size_t oe = s.order_elems;
  TRY(grow(s.order, oe, (size_t)T * kk, ctx));
  oe = s.order_elems;
  TRY(grow(s.inv, oe, (size_t)T * kk, ctx));
  s.order_elems = oe;
  TRY(grow(s.offsets, s.offset_elems, 257, ctx));
  RmoeLayer Lk = L;
  Lk.top_k = kk;
  if (L.n_shared > 0) TRY(grow(s.pf, s.pf_bytes, rmoe::prefill_scratch_bytes(Lk, T), ctx));
  if (L.n_shared > 0 && !L.d_layout) TRY(reserve_stack(ctx, L, 1));
  s.max_tokens = std::max(s.max_tokens, T);
  return RMOE_OK;
}

// Hand-off buffers and counters of the persistent decode kernel for n_layers layers of
// L's geometry.  Counters are zero when (re)allocated and after every complete launch.
int reserve_stack(rmoe_ctx* ctx, const RmoeLayer& L, int n_layers) {
  RmoeScratch& s = ctx->s;
  const unsigned* old_cnt = s.stack_cnt;
  TRY(grow(s.stack, s.stack_bytes, rmoe::stack_scratch_bytes(L, n_layers), ctx));
  TRY(grow(s.stack_cnt, s.stack_cnt_n, rmoe::stack_counter_count(L, n_layers), ctx));
  // The decode stack tags its hand-off words with a launch counter kept beside its
  // counters; when the counters start again from zero, no older word may carry a tag
  // that a new launch accepts, so the hand-off area is cleared too.
  if (s.stack_cnt != old_cnt) {
    HIP_TRY(hipMemsetAsync(s.stack, 0, s.stack_bytes, ctx->stream));
    HIP_TRY(hipStreamSynchronize(ctx->stream));
  }
  return RMOE_OK;
}

int sync_and_check(rmoe_ctx* ctx, hipStream_t st) {
  HIP_TRY(hipStreamSynchronize(st));
  int err = 0;
  HIP_TRY(hipMemcpy(&err, ctx->s.err, sizeof(int), hipMemcpyDeviceToHost));
  if (err) {
    HIP_TRY(hipMemsetAsync(ctx->s.err, 0, sizeof(int), ctx->stream));
    HIP_TRY(hipStreamSynchronize(ctx->stream));
    if (err & 1) return fail(RMOE_EINVAL, "Input weight matrix contains non-finite values (NaN or Inf)");
    if (err & 2) return fail(RMOE_EINVAL, "Quantization parameters (scale_q or min_q) overflowed to non-finite values");
    if (err & 4) return fail(RMOE_EINVAL, "expert id out of range in dispatch");
    if (err & 8) {
      // A wait of the persistent decode kernel timed out: its counters are left
      // mid-way; clear them for the next launch.
      // Its launch counter restarts with them, so its tagged hand-off words are cleared
      // as well.  Word 1 of the counter area says which wait gave up first.
      unsigned info = 0u;
      if (ctx->s.stack_cnt) {
        HIP_TRY(hipMemcpy(&info, ctx->s.stack_cnt + 1, sizeof(unsigned), hipMemcpyDeviceToHost));
        HIP_TRY(hipMemsetAsync(ctx->s.stack_cnt, 0, ctx->s.stack_cnt_n * sizeof(unsigned), ctx->stream));
        if (ctx->s.stack) HIP_TRY(hipMemsetAsync(ctx->s.stack, 0, ctx->s.stack_bytes, ctx->stream));
        HIP_TRY(hipStreamSynchronize(ctx->stream));
      }
      if (info & rmoe::kAbortValid) {
        const unsigned phase = (info >> 26) & 15u;
        const char* what = phase == rmoe::kAbortReady ? "its input (the previous layer's combined bands, ready counter)"
                           : phase == rmoe::kAbortH   ? "h of its down unit (the gate/up units of the slot)"
                           : phase == rmoe::kAbortD   ? "d of its band (the down units, as the band's combiner)"
                                                      : "an unknown hand-off";
        return fail(RMOE_EDEVICE,
                    "persistent decode kernel timed out waiting for other workgroups: workgroup %u gave up at layer "
                    "%u waiting for %s",
                    info & 0xfffu, (info >> 12) & 0x3fffu, what);
      }
      return fail(RMOE_EDEVICE, "persistent decode kernel timed out waiting for other workgroups");
    }
    return fail(RMOE_EDEVICE, "device error flag 0x%x", err);
  }
  return RMOE_OK;
}

// Allocate the expert storage of L and register it as `layer` (replacing nothing:
// the caller freed any previous layer of that id).
int place_layer(rmoe_ctx* ctx, int layer, RmoeLayer& L) {
  if (hipMalloc((void**)&L.gu, (size_t)L.gu_experts * L.gu_bytes) != hipSuccess)
    return fail(RMOE_ENOMEM, "hipMalloc of expert gate_up failed");
  if (hipMalloc((void**)&L.dn, (size_t)L.dn_experts * L.dn_bytes) != hipSuccess) {
    hipFree(L.gu);
    return fail(RMOE_ENOMEM, "hipMalloc of expert down failed");
  }
  if (L.dn_fmt == RMOE_FMT_BFP16 &&
      (hipMalloc((void**)&L.dn_rowexp, (size_t)L.dn_experts * L.H) != hipSuccess ||
       hipMemset(L.dn_rowexp, 7, (size_t)L.dn_experts * L.H) != hipSuccess)) {
    hipFree(L.gu);
    hipFree(L.dn);
    hipFree(L.dn_rowexp);
    return fail(RMOE_ENOMEM, "hipMalloc of the down row exponents failed");
  }
  ctx->layers[layer] = L;
  return reserve_layer(ctx, L, 1, L.top_k);
}

// Entry points that need every expert's gate/up inside the layer (the shared expert
// included) serve q4nx layers only.
int require_q4nx_layer(const RmoeLayer& L, int layer, const char* what) {
  if (L.d_layout)
    return fail(RMOE_EINVAL, "layer %d holds weights-d bundles (bfp16 down, shared gate/up outside the layer): %s "
                "serves q4nx layers only", layer, what);
  return RMOE_OK;
}

int check_ids(const int32_t* ids, int T, int k, int n_routed) {
  for (int t = 0; t < T; ++t) {
    for (int r = 0; r < k; ++r) {
      const int e = ids[(size_t)t * k + r];
      if (e < 0 || e >= n_routed) return fail(RMOE_EINVAL, "top_ids values must be in 0..%d", n_routed - 1);
      for (int q = 0; q < r; ++q)
        if (ids[(size_t)t * k + q] == e) return fail(RMOE_EINVAL, "each token must route to %d distinct experts", k);
    }
  }
  return RMOE_OK;
}

// ------------------------------------------------------- static decode scratch --
// rmoe_moe_experts_static_dev runs the routed-expert decode kernels on this file-scope
// device array instead of context scratch, so it never allocates.  Each GPU holds its
// own copy until the process ends.  It holds the activations h of the call's slots
// ([k][Ipad] bf16), which the gate/up kernel writes in full (padding columns included)
// before the down kernel reads them, so nothing in it must start at zero.
constexpr size_t kStaticScratchBytes = 256u << 10;

}  // namespace

static __device__ __align__(256) uint8_t scratch[kStaticScratchBytes];

namespace {

// scratch's device address per device id, from hipGetSymbolAddress: in host code the
// array's name is not a device address.
std::mutex g_scratch_mu;
std::map<int, uint8_t*> g_scratch_ptr;

// Called by rmoe_create with the context's device current: the first context on a
// device looks up the array's address.
int init_static_scratch(rmoe_ctx* ctx) {
  std::lock_guard<std::mutex> lock(g_scratch_mu);
  if (g_scratch_ptr.count(ctx->device)) return RMOE_OK;
  void* p = nullptr;
  hipError_t e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
  if (e != hipSuccess || !p) return fail(RMOE_EDEVICE, "hipGetSymbolAddress(scratch): %s", hipGetErrorString(e));
  g_scratch_ptr[ctx->device] = static_cast<uint8_t*>(p);
  return RMOE_OK;
}

uint8_t* static_scratch(int device) {
  std::lock_guard<std::mutex> lock(g_scratch_mu);
  auto it = g_scratch_ptr.find(device);
  return it == g_scratch_ptr.end() ? nullptr : it->second;
}

}  // namespace

extern "C" {

const char* rmoe_last_error(void) { return g_err.c_str(); }

const char* rmoe_version(void) { return "rmoe 0.1 gfx950"; }

int rmoe_create(int device, rmoe_ctx** out) {
  if (!out) return fail(RMOE_EINVAL, "null output pointer");
  int n = 0;
  if (hipGetDeviceCount(&n) != hipSuccess || n == 0) return fail(RMOE_EDEVICE, "no HIP device available");
  if (device < 0 || device >= n) return fail(RMOE_EINVAL, "device %d out of range (0..%d)", device, n - 1);
  HIP_TRY(hipSetDevice(device));
  rmoe_ctx* ctx = new rmoe_ctx();
  ctx->device = device;
  if (hipStreamCreateWithFlags(&ctx->stream, hipStreamNonBlocking) != hipSuccess) {
    delete ctx;
    return fail(RMOE_EDEVICE, "hipStreamCreate failed");
  }
  if (hipMalloc((void**)&ctx->s.err, sizeof(int)) != hipSuccess) {
    hipStreamDestroy(ctx->stream);
    delete ctx;
    return fail(RMOE_ENOMEM, "hipMalloc failed");
  }
  hipMemsetAsync(ctx->s.err, 0, sizeof(int), ctx->stream);
  hipStreamSynchronize(ctx->stream);
  if (init_static_scratch(ctx) != RMOE_OK) {
    const std::string msg = g_err;
    hipFree(ctx->s.err);
    hipStreamDestroy(ctx->stream);
    delete ctx;
    return fail(RMOE_EDEVICE, "%s", msg.c_str());
  }
  // The persistent decode kernel runs one workgroup per CU and needs all of them
  // resident at once.
  int n_cu = 0, per_cu = 0;
  if (hipDeviceGetAttribute(&n_cu, hipDeviceAttributeMultiprocessorCount, device) == hipSuccess &&
      rmoe::decode_stack_occupancy(&per_cu) == hipSuccess && per_cu >= 1)
    ctx->n_cu = n_cu;
  *out = ctx;
  return RMOE_OK;
}

int rmoe_destroy(rmoe_ctx* ctx) {
  if (!ctx) return RMOE_OK;
  hipSetDevice(ctx->device);
  hipStreamSynchronize(ctx->stream);
  for (auto& kv : ctx->mats)
    if (kv.second.view_of_layer < 0) hipFree(kv.second.tiles);
  for (auto& kv : ctx->layers) {
    hipFree(kv.second.gu);
    hipFree(kv.second.dn);
    hipFree(kv.second.dn_rowexp);
    hipFree(kv.second.router_w);
    hipFree(kv.second.router_bias);
  }
  RmoeScratch& s = ctx->s;
  void* bufs[] = {s.part, s.counters, s.h, s.ids, s.wts, s.logits, s.order, s.inv, s.offsets,
                  s.chunk_counts, s.err, s.staging, s.pf, s.stack, s.stack_cnt};
  for (void* b : bufs)
    if (b) hipFree(b);
  auto it = g_io.find(ctx);
  if (it != g_io.end()) {
    hipFree(it->second.p);
    g_io.erase(it);
  }
  hipStreamDestroy(ctx->stream);
  delete ctx;
  return RMOE_OK;
}

int rmoe_synchronize(rmoe_ctx* ctx) {
  if (!ctx) return fail(RMOE_EINVAL, "null context");
  HIP_TRY(hipSetDevice(ctx->device));
  HIP_TRY(hipDeviceSynchronize());
  return sync_and_check(ctx, ctx->stream);
}

void* rmoe_stream(rmoe_ctx* ctx) { return ctx ? (void*)ctx->stream : nullptr; }

// ------------------------------------------------------------------ matrices --
static int check_mk(int M, int K) {
  if (M <= 0 || K <= 0 || M % 128 != 0) return fail(RMOE_EINVAL, "M (%d) must be a positive multiple of 128", M);
  if (K % 256 != 0) return fail(RMOE_EINVAL, "K (%d) must be a multiple of K_TILE (256)", K);
  return RMOE_OK;
}

int rmoe_matrix_upload(rmoe_ctx* ctx, const void* bytes, size_t nbytes, int M, int K, int* handle) {
  if (!ctx || !bytes || !handle) return fail(RMOE_EINVAL, "null argument");
  TRY(check_mk(M, K));
  const size_t need = rmoe::matrix_bytes(M, K);
  if (nbytes != need) return fail(RMOE_EINVAL, "pack_gemv buffer has %zu bytes, expected %zu for [%d, %d]", nbytes, need, M, K);
  HIP_TRY(hipSetDevice(ctx->device));
  RmoeMatrix m;
  m.M = M;
  m.K = K;
  if (hipMalloc((void**)&m.tiles, need) != hipSuccess) return fail(RMOE_ENOMEM, "hipMalloc of %zu bytes failed", need);
  TRY(grow(ctx->s.staging, ctx->s.staging_bytes, need, ctx));
  HIP_TRY(hipMemcpyAsync(ctx->s.staging, bytes, need, hipMemcpyHostToDevice, ctx->stream));
  HIP_TRY(rmoe::launch_relayout_in(ctx->s.staging, m.tiles, M, K, ctx->stream));
  HIP_TRY(hipStreamSynchronize(ctx->stream));
  *handle = ctx->next_handle++;
  ctx->mats[*handle] = m;
  return RMOE_OK;
}

int rmoe_matrix_upload_q4k(rmoe_ctx* ctx, const void* bytes, size_t nbytes, int M, int K, int* handle) {
  if (!ctx || !bytes || !handle) return fail(RMOE_EINVAL, "null argument");
  TRY(check_mk(M, K));
  const size_t need = (size_t)M * (K / 256) * 144, tb = rmoe::matrix_bytes(M, K);
  if (nbytes != need) return fail(RMOE_EINVAL, "Q4_K tensor has %zu bytes, expected %zu for [%d, %d]", nbytes, need, M, K);
  HIP_TRY(hipSetDevice(ctx->device));
  RmoeMatrix m;
  m.M = M;
  m.K = K;
  if (hipMalloc((void**)&m.tiles, tb) != hipSuccess) return fail(RMOE_ENOMEM, "hipMalloc of %zu bytes failed", tb);
  int r = grow(ctx->s.staging, ctx->s.staging_bytes, need, ctx);
  if (r != RMOE_OK) {
    hipFree(m.tiles);
    return r;
  }
  HIP_TRY(hipMemcpyAsync(ctx->s.staging, bytes, need, hipMemcpyHostToDevice, ctx->stream));
  HIP_TRY(rmoe::launch_q4k_to_tiles(ctx->s.staging, M, K, m.tiles, K, 0, ctx->stream));
  HIP_TRY(hipStreamSynchronize(ctx->stream));
  *handle = ctx->next_handle++;
  ctx->mats[*handle] = m;
  return RMOE_OK;
}

int rmoe_matrix_upload_bfp16(rmoe_ctx* ctx, const void* bytes, size_t nbytes, int M, int K, int* handle) {
  if (!ctx || !bytes || !handle) return fail(RMOE_EINVAL, "null argument");
  TRY(check_mk(M, K));
  const size_t need = rmoe::matrix_bytes_bfp16(M, K);
  if (nbytes != need)
    return fail(RMOE_EINVAL, "bfp16 GEMV buffer has %zu bytes, expected %zu for [%d, %d]", nbytes, need, M, K);
  HIP_TRY(hipSetDevice(ctx->device));
  RmoeMatrix m;
  m.M = M;
  m.K = K;
  m.fmt = RMOE_FMT_BFP16;
  if (hipMalloc((void**)&m.tiles, need) != hipSuccess) return fail(RMOE_ENOMEM, "hipMalloc of %zu bytes failed", need);
  int r = grow(ctx->s.staging, ctx->s.staging_bytes, need, ctx);
  if (r != RMOE_OK) {
    hipFree(m.tiles);
    return r;
  }
  HIP_TRY(hipMemcpyAsync(ctx->s.staging, bytes, need, hipMemcpyHostToDevice, ctx->stream));
  HIP_TRY(rmoe::launch_b16_relayout_in(ctx->s.staging, m.tiles, M, K, ctx->stream));
  HIP_TRY(hipStreamSynchronize(ctx->stream));
  *handle = ctx->next_handle++;
  ctx->mats[*handle] = m;
  return RMOE_OK;
}

int rmoe_matrix_quantize_dev(rmoe_ctx* ctx, const float* w_dev, int M, int K, int* handle, void* stream) {
  if (!ctx || !w_dev || !handle) return fail(RMOE_EINVAL, "null argument");
  TRY(check_mk(M, K));
  HIP_TRY(hipSetDevice(ctx->device));
  RmoeMatrix m;
  m.M = M;
  m.K = K;
  const size_t need = rmoe::matrix_bytes(M, K);
  if (hipMalloc((void**)&m.tiles, need) != hipSuccess) return fail(RMOE_ENOMEM, "hipMalloc of %zu bytes failed", need);
  hipStream_t st = pick_stream(ctx, stream);
  HIP_TRY(rmoe::launch_quantize(w_dev, M, K, K, K, m.tiles, ctx->s.err, st));
  int r = sync_and_check(ctx, st);
  if (r != RMOE_OK) {
    hipFree(m.tiles);
    return r;
  }
  *handle = ctx->next_handle++;
  ctx->mats[*handle] = m;
  return RMOE_OK;
}

static int find_matrix(rmoe_ctx* ctx, int handle, RmoeMatrix** out) {
  if (!ctx) return fail(RMOE_EINVAL, "null context");
  auto it = ctx->mats.find(handle);
  if (it == ctx->mats.end()) return fail(RMOE_ENOTFOUND, "unknown matrix handle %d", handle);
  *out = &it->second;
  return RMOE_OK;
}

static size_t stored_bytes(const RmoeMatrix& m) {
  return m.fmt == RMOE_FMT_BFP16 ? rmoe::matrix_bytes_bfp16(m.M, m.K) : rmoe::matrix_bytes(m.M, m.K);
}

int rmoe_matrix_download(rmoe_ctx* ctx, int handle, void* bytes, size_t nbytes) {
  RmoeMatrix* m;
  TRY(find_matrix(ctx, handle, &m));
  const size_t need = stored_bytes(*m);
  if (!bytes || nbytes != need) return fail(RMOE_EINVAL, "download buffer must hold %zu bytes", need);
  HIP_TRY(hipSetDevice(ctx->device));
  TRY(grow(ctx->s.staging, ctx->s.staging_bytes, need, ctx));
  if (m->fmt == RMOE_FMT_BFP16)
    HIP_TRY(rmoe::launch_b16_relayout_out(m->tiles, ctx->s.staging, m->M, m->K, ctx->stream));
  else
    HIP_TRY(rmoe::launch_relayout_out(m->tiles, ctx->s.staging, m->M, m->K, ctx->stream));
  HIP_TRY(hipMemcpyAsync(bytes, ctx->s.staging, need, hipMemcpyDeviceToHost, ctx->stream));
  HIP_TRY(hipStreamSynchronize(ctx->stream));
  return RMOE_OK;
}

int rmoe_matrix_free(rmoe_ctx* ctx, int handle) {
  RmoeMatrix* m;
  TRY(find_matrix(ctx, handle, &m));
  HIP_TRY(hipStreamSynchronize(ctx->stream));
  if (m->view_of_layer < 0) hipFree(m->tiles);
  ctx->mats.erase(handle);
  return RMOE_OK;
}

int rmoe_matrix_shape(rmoe_ctx* ctx, int handle, int* M, int* K) {
  RmoeMatrix* m;
  TRY(find_matrix(ctx, handle, &m));
  if (M) *M = m->M;
  if (K) *K = m->K;
  return RMOE_OK;
}

int rmoe_matrix_format(rmoe_ctx* ctx, int handle, int* fmt) {
  RmoeMatrix* m;
  TRY(find_matrix(ctx, handle, &m));
  if (!fmt) return fail(RMOE_EINVAL, "null argument");
  *fmt = m->fmt;
  return RMOE_OK;
}

static hipError_t launch_matrix_linear(const RmoeMatrix& m, const uint16_t* x, int T, uint16_t* y, RmoeScratch& s,
                                       hipStream_t st) {
  if (m.fmt == RMOE_FMT_BFP16) return rmoe::launch_linear_bfp16(m.tiles, m.M, m.K, x, T, y, s, st);
  return rmoe::launch_linear(m.tiles, m.M, m.K, x, T, y, s, st);
}

int rmoe_linear(rmoe_ctx* ctx, int handle, const uint16_t* x, int T, int K_in, uint16_t* y) {
  RmoeMatrix* m;
  TRY(find_matrix(ctx, handle, &m));
  if (!x || !y) return fail(RMOE_EINVAL, "null argument");
  if (T < 1) return fail(RMOE_EINVAL, "T must be >= 1");
  if (K_in < 1 || K_in > m->K) return fail(RMOE_EINVAL, "input width %d does not fit K=%d", K_in, m->K);
  HIP_TRY(hipSetDevice(ctx->device));
  size_t f, c;
  linear_needs(m->M, m->K, T, f, c);
  TRY(grow(ctx->s.part, ctx->s.part_floats, f, ctx));
  TRY(grow(ctx->s.counters, ctx->s.n_counters, c, ctx));
  const size_t xb = align_up((size_t)T * m->K * 2, 256), yb = (size_t)T * m->M * 2;
  uint8_t* io;
  TRY(io_area(ctx, xb + yb, &io));
  uint16_t* xd = reinterpret_cast<uint16_t*>(io);
  uint16_t* yd = reinterpret_cast<uint16_t*>(io + xb);
  if (K_in == m->K) {
    HIP_TRY(hipMemcpyAsync(xd, x, (size_t)T * m->K * 2, hipMemcpyHostToDevice, ctx->stream));
  } else {
    HIP_TRY(hipMemsetAsync(xd, 0, (size_t)T * m->K * 2, ctx->stream));
    HIP_TRY(hipMemcpy2DAsync(xd, (size_t)m->K * 2, x, (size_t)K_in * 2, (size_t)K_in * 2, T, hipMemcpyHostToDevice,
                             ctx->stream));
  }
  HIP_TRY(launch_matrix_linear(*m, xd, T, yd, ctx->s, ctx->stream));
  HIP_TRY(hipMemcpyAsync(y, yd, yb, hipMemcpyDeviceToHost, ctx->stream));
  HIP_TRY(hipStreamSynchronize(ctx->stream));
  return RMOE_OK;
}

int rmoe_linear_dev(rmoe_ctx* ctx, int handle, const void* x_dev, int T, void* y_dev, void* stream) {
  RmoeMatrix* m;
  TRY(find_matrix(ctx, handle, &m));
  if (!x_dev || !y_dev || T < 1) return fail(RMOE_EINVAL, "bad argument");
  size_t f, c;
  linear_needs(m->M, m->K, T, f, c);
  if (f > ctx->s.part_floats || c > ctx->s.n_counters)
    return fail(RMOE_EINVAL, "scratch too small for T=%d: call rmoe_reserve_linear first", T);
  HIP_TRY(launch_matrix_linear(*m, (const uint16_t*)x_dev, T, (uint16_t*)y_dev, ctx->s, pick_stream(ctx, stream)));
  return RMOE_OK;
}

int rmoe_reserve_linear(rmoe_ctx* ctx, int handle, int T) {
  RmoeMatrix* m;
  TRY(find_matrix(ctx, handle, &m));
  if (T < 1) return fail(RMOE_EINVAL, "T must be >= 1");
  HIP_TRY(hipSetDevice(ctx->device));
  size_t f, c;
  linear_needs(m->M, m->K, T, f, c);
  TRY(grow(ctx->s.part, ctx->s.part_floats, f, ctx));
  TRY(grow(ctx->s.counters, ctx->s.n_counters, c, ctx));
  return RMOE_OK;
}

// -------------------------------------------------------------------- layers --
int rmoe_layer_create(rmoe_ctx* ctx, int layer, int hidden, int inter, int n_routed, int n_shared, int top_k) {
  if (!ctx) return fail(RMOE_EINVAL, "null context");
  if (hidden <= 0 || hidden % 256) return fail(RMOE_EINVAL, "hidden (%d) must be a positive multiple of 256", hidden);
  if (inter <= 0 || inter % 64) return fail(RMOE_EINVAL, "intermediate size (%d) must be a positive multiple of 64", inter);
  if (n_routed < 1 || n_routed > 256) return fail(RMOE_EINVAL, "n_routed (%d) must be in 1..256", n_routed);
  if (n_shared < 0 || n_shared > 1) return fail(RMOE_EINVAL, "n_shared must be 0 or 1");
  if (top_k < 1 || top_k > 16 || top_k > n_routed) return fail(RMOE_EINVAL, "top_k (%d) must be in 1..min(16, n_routed)", top_k);
  HIP_TRY(hipSetDevice(ctx->device));
  rmoe_layer_free(ctx, layer);
  g_err.clear();
  RmoeLayer L;
  L.H = hidden;
  L.I = inter;
  L.Ipad = (inter + 255) / 256 * 256;
  L.n_routed = n_routed;
  L.n_shared = n_shared;
  L.top_k = top_k;
  L.gu_bytes = rmoe::matrix_bytes(2 * inter, hidden);
  L.dn_bytes = rmoe::matrix_bytes(hidden, L.Ipad);
  L.gu_experts = L.dn_experts = n_routed + n_shared;
  return place_layer(ctx, layer, L);
}

int rmoe_layer_create_d(rmoe_ctx* ctx, int layer, int hidden, int inter, int n_routed, int top_k) {
  if (!ctx) return fail(RMOE_EINVAL, "null context");
  if (hidden <= 0 || hidden % 256) return fail(RMOE_EINVAL, "hidden (%d) must be a positive multiple of 256", hidden);
  if (inter <= 0 || inter % 64) return fail(RMOE_EINVAL, "intermediate size (%d) must be a positive multiple of 64", inter);
  if (n_routed < 1 || n_routed > 256) return fail(RMOE_EINVAL, "n_routed (%d) must be in 1..256", n_routed);
  if (top_k < 1 || top_k > 16 || top_k > n_routed) return fail(RMOE_EINVAL, "top_k (%d) must be in 1..min(16, n_routed)", top_k);
  HIP_TRY(hipSetDevice(ctx->device));
  rmoe_layer_free(ctx, layer);
  g_err.clear();
  RmoeLayer L;
  L.H = hidden;
  L.I = inter;
  L.Ipad = (inter + 255) / 256 * 256;
  L.n_routed = n_routed;
  L.n_shared = 1;
  L.top_k = top_k;
  L.d_layout = true;
  L.dn_fmt = RMOE_FMT_BFP16;
  L.gu_bytes = rmoe::matrix_bytes(2 * inter, hidden);
  L.dn_bytes = rmoe::matrix_bytes_bfp16(hidden, L.Ipad);
  L.gu_experts = n_routed;
  L.dn_experts = n_routed + 1;
  return place_layer(ctx, layer, L);
}

int rmoe_layer_upload_d(rmoe_ctx* ctx, int layer, int bundle, int expert0, int n, const void* bytes, size_t nbytes) {
  RmoeLayer* L;
  TRY(check_layer(ctx, layer, &L));
  if (!L->d_layout) return fail(RMOE_EINVAL, "layer %d is not a weights-d layer (rmoe_layer_create_d)", layer);
  if (bundle != RMOE_BUNDLE_B1 && bundle != RMOE_BUNDLE_B2)
    return fail(RMOE_EINVAL, "bundle %d is not RMOE_BUNDLE_B1 or RMOE_BUNDLE_B2", bundle);
  const bool b1 = bundle == RMOE_BUNDLE_B1;
  const int count = b1 ? L->gu_experts : L->dn_experts;
  const size_t per = b1 ? L->gu_bytes : L->dn_bytes;
  if (!bytes || n < 1 || expert0 < 0 || expert0 + n > count)
    return fail(RMOE_EINVAL, "experts [%d, %d) outside moe_b%d's %d experts", expert0, expert0 + n, bundle, count);
  if (nbytes != (size_t)n * per)
    return fail(RMOE_EINVAL, "moe_b%d slice has %zu bytes, expected %zu (%d experts x %zu)", bundle, nbytes,
                (size_t)n * per, n, per);
  HIP_TRY(hipSetDevice(ctx->device));
  TRY(grow(ctx->s.staging, ctx->s.staging_bytes, per, ctx));
  uint8_t* base = b1 ? L->gu : L->dn;
  for (int i = 0; i < n; ++i) {
    const size_t e = (size_t)expert0 + i;
    HIP_TRY(hipMemcpyAsync(ctx->s.staging, (const uint8_t*)bytes + (size_t)i * per, per, hipMemcpyHostToDevice,
                           ctx->stream));
    if (b1)
      HIP_TRY(rmoe::launch_relayout_in(ctx->s.staging, base + e * per, 2 * L->I, L->H, ctx->stream));
    else {
      HIP_TRY(rmoe::launch_b16_relayout_in(ctx->s.staging, base + e * per, L->H, L->Ipad, ctx->stream));
      HIP_TRY(rmoe::launch_b16_rowexp(base + e * per, L->H, L->Ipad, L->I, L->dn_rowexp + e * L->H, ctx->stream));
    }
    // The staging buffer is reused by the next expert: wait for the re-layout.
    HIP_TRY(hipStreamSynchronize(ctx->stream));
  }
  return RMOE_OK;
}

int rmoe_layer_free(rmoe_ctx* ctx, int layer) {
  if (!ctx) return fail(RMOE_EINVAL, "null context");
  auto it = ctx->layers.find(layer);
  if (it == ctx->layers.end()) return fail(RMOE_ENOTFOUND, "layer %d is not an uploaded MoE layer", layer);
  hipStreamSynchronize(ctx->stream);
  hipFree(it->second.gu);
  hipFree(it->second.dn);
  hipFree(it->second.dn_rowexp);
  hipFree(it->second.router_w);
  hipFree(it->second.router_bias);
  ctx->layers.erase(it);
  // Views of the layer's experts borrowed its memory: their handles go with it.
  for (auto m = ctx->mats.begin(); m != ctx->mats.end();) {
    if (m->second.view_of_layer == layer) m = ctx->mats.erase(m);
    else ++m;
  }
  return RMOE_OK;
}

int rmoe_layer_expert_matrix(rmoe_ctx* ctx, int layer, int expert, int part, int* handle) {
  RmoeLayer* L;
  TRY(check_layer(ctx, layer, &L));
  if (!handle) return fail(RMOE_EINVAL, "null argument");
  RmoeMatrix m;
  m.view_of_layer = layer;
  if (part == RMOE_PART_GATE_UP) {
    if (expert < 0 || expert >= L->gu_experts)
      return fail(RMOE_EINVAL, "expert %d has no gate/up in layer %d (0..%d)", expert, layer, L->gu_experts - 1);
    m.tiles = L->gu + (size_t)expert * L->gu_bytes;
    m.M = 2 * L->I;
    m.K = L->H;
    m.fmt = RMOE_FMT_Q4NX;
  } else if (part == RMOE_PART_DOWN) {
    if (expert < 0 || expert >= L->dn_experts)
      return fail(RMOE_EINVAL, "expert %d has no down projection in layer %d (0..%d)", expert, layer, L->dn_experts - 1);
    m.tiles = L->dn + (size_t)expert * L->dn_bytes;
    m.M = L->H;
    m.K = L->Ipad;
    m.fmt = L->dn_fmt;
  } else {
    return fail(RMOE_EINVAL, "part must be RMOE_PART_GATE_UP or RMOE_PART_DOWN, got %d", part);
  }
  TRY(check_mk(m.M, m.K));
  *handle = ctx->next_handle++;
  ctx->mats[*handle] = m;
  return RMOE_OK;
}

int rmoe_reserve(rmoe_ctx* ctx, int layer, int max_tokens) {
  RmoeLayer* L;
  TRY(check_layer(ctx, layer, &L));
  if (max_tokens < 1) return fail(RMOE_EINVAL, "max_tokens must be >= 1");
  HIP_TRY(hipSetDevice(ctx->device));
  return reserve_layer(ctx, *L, max_tokens, L->top_k);
}

int rmoe_layer_upload_experts(rmoe_ctx* ctx, int layer, const void* gate_up, size_t gu_nbytes, const void* down,
                              size_t dn_nbytes) {
  RmoeLayer* L;
  TRY(check_layer(ctx, layer, &L));
  TRY(require_q4nx_layer(*L, layer, "rmoe_layer_upload_experts"));
  const size_t ne = (size_t)L->n_routed + L->n_shared;
  if (!gate_up || gu_nbytes != ne * L->gu_bytes)
    return fail(RMOE_EINVAL, "gate_up bundle has %zu bytes, expected %zu (%zu experts x %zu)", gu_nbytes, ne * L->gu_bytes, ne, L->gu_bytes);
  if (!down || dn_nbytes != ne * L->dn_bytes)
    return fail(RMOE_EINVAL, "down bundle has %zu bytes, expected %zu (%zu experts x %zu)", dn_nbytes, ne * L->dn_bytes, ne, L->dn_bytes);
  HIP_TRY(hipSetDevice(ctx->device));
  const size_t per = std::max(L->gu_bytes, L->dn_bytes);
  TRY(grow(ctx->s.staging, ctx->s.staging_bytes, per, ctx));
  for (size_t e = 0; e < ne; ++e) {
    HIP_TRY(hipMemcpyAsync(ctx->s.staging, (const uint8_t*)gate_up + e * L->gu_bytes, L->gu_bytes, hipMemcpyHostToDevice, ctx->stream));
    HIP_TRY(rmoe::launch_relayout_in(ctx->s.staging, L->gu + e * L->gu_bytes, 2 * L->I, L->H, ctx->stream));
    HIP_TRY(hipMemcpyAsync(ctx->s.staging, (const uint8_t*)down + e * L->dn_bytes, L->dn_bytes, hipMemcpyHostToDevice, ctx->stream));
    HIP_TRY(rmoe::launch_relayout_in(ctx->s.staging, L->dn + e * L->dn_bytes, L->H, L->Ipad, ctx->stream));
    // The staging buffer is reused by the next expert: wait for the re-layout.
    HIP_TRY(hipStreamSynchronize(ctx->stream));
  }
  return RMOE_OK;
}

int rmoe_layer_upload_expert_q4k(rmoe_ctx* ctx, int layer, int expert, int part, const void* bytes, size_t nbytes) {
  RmoeLayer* L;
  TRY(check_layer(ctx, layer, &L));
  TRY(require_q4nx_layer(*L, layer, "rmoe_layer_upload_expert_q4k"));
  if (expert < 0 || expert >= L->n_routed + L->n_shared) return fail(RMOE_EINVAL, "expert %d out of range", expert);
  if (!bytes) return fail(RMOE_EINVAL, "null Q4_K tensor");
  int M, K, Kt, row0;
  uint8_t* dst;
  if (part == RMOE_PART_GATE || part == RMOE_PART_UP) {
    M = L->I, K = L->H, Kt = L->H, row0 = part == RMOE_PART_UP ? L->I : 0;
    dst = L->gu + (size_t)expert * L->gu_bytes;
  } else if (part == RMOE_PART_DOWN) {
    M = L->H, K = L->I, Kt = L->Ipad, row0 = 0;
    dst = L->dn + (size_t)expert * L->dn_bytes;
  } else {
    return fail(RMOE_EINVAL, "part %d is not RMOE_PART_GATE, _UP or _DOWN", part);
  }
  if (K % 256) return fail(RMOE_EINVAL, "Q4_K rows must be a multiple of 256 wide, got %d", K);
  const size_t need = (size_t)M * (K / 256) * 144;
  if (nbytes != need) return fail(RMOE_EINVAL, "Q4_K tensor has %zu bytes, expected %zu for [%d, %d]", nbytes, need, M, K);
  HIP_TRY(hipSetDevice(ctx->device));
  TRY(grow(ctx->s.staging, ctx->s.staging_bytes, need, ctx));
  HIP_TRY(hipMemcpyAsync(ctx->s.staging, bytes, need, hipMemcpyHostToDevice, ctx->stream));
  HIP_TRY(rmoe::launch_q4k_to_tiles(ctx->s.staging, M, K, dst, Kt, row0, ctx->stream));
  HIP_TRY(hipStreamSynchronize(ctx->stream));
  return RMOE_OK;
}

int rmoe_layer_quantize_expert_dev(rmoe_ctx* ctx, int layer, int expert, const float* gate_up_dev,
                                   const float* down_dev, void* stream) {
  RmoeLayer* L;
  TRY(check_layer(ctx, layer, &L));
  TRY(require_q4nx_layer(*L, layer, "rmoe_layer_quantize_expert_dev"));
  if (expert < 0 || expert >= L->n_routed + L->n_shared) return fail(RMOE_EINVAL, "expert %d out of range", expert);
  if (!gate_up_dev || !down_dev) return fail(RMOE_EINVAL, "null weights");
  HIP_TRY(hipSetDevice(ctx->device));
  hipStream_t st = pick_stream(ctx, stream);
  HIP_TRY(rmoe::launch_quantize(gate_up_dev, 2 * L->I, L->H, L->H, L->H, L->gu + (size_t)expert * L->gu_bytes,
                                ctx->s.err, st));
  HIP_TRY(rmoe::launch_quantize(down_dev, L->H, L->Ipad, L->I, L->I, L->dn + (size_t)expert * L->dn_bytes, ctx->s.err,
                                st));
  return sync_and_check(ctx, st);
}

int rmoe_layer_synthesize_dev(rmoe_ctx* ctx, int layer, uint64_t seed, float std, void* stream) {
  RmoeLayer* L;
  TRY(check_layer(ctx, layer, &L));
  TRY(require_q4nx_layer(*L, layer, "rmoe_layer_synthesize_dev"));
  if (!(std > 0.f) || !(std < 1e30f)) return fail(RMOE_EINVAL, "std must be positive and finite");
  HIP_TRY(hipSetDevice(ctx->device));
  hipStream_t st = pick_stream(ctx, stream);
  const int ne = L->n_routed + L->n_shared;
  for (int e = 0; e < ne; ++e) {
    const uint64_t s_gu = seed * 1000003ull + (uint64_t)e * 2ull + 1ull;
    const uint64_t s_dn = seed * 1000003ull + (uint64_t)e * 2ull + 2ull;
    HIP_TRY(rmoe::launch_synth_quantize(s_gu, std, 2 * L->I, L->H, L->H, L->gu + (size_t)e * L->gu_bytes, ctx->s.err, st));
    HIP_TRY(rmoe::launch_synth_quantize(s_dn, std, L->H, L->Ipad, L->I, L->dn + (size_t)e * L->dn_bytes, ctx->s.err, st));
  }
  return sync_and_check(ctx, st);
}

int rmoe_layer_download_expert(rmoe_ctx* ctx, int layer, int expert, void* gate_up, size_t gu_nbytes, void* down,
                               size_t dn_nbytes) {
  RmoeLayer* L;
  TRY(check_layer(ctx, layer, &L));
  if (expert < 0 || expert >= L->dn_experts) return fail(RMOE_EINVAL, "expert %d out of range", expert);
  // A weights-d layer has no gate/up for its last (shared) expert: gate_up must be null.
  const bool has_gu = expert < L->gu_experts;
  if ((has_gu ? (!gate_up || gu_nbytes != L->gu_bytes) : (gate_up != nullptr)) || !down || dn_nbytes != L->dn_bytes)
    return fail(RMOE_EINVAL, "download buffers must hold %zu and %zu bytes", has_gu ? L->gu_bytes : 0, L->dn_bytes);
  HIP_TRY(hipSetDevice(ctx->device));
  TRY(grow(ctx->s.staging, ctx->s.staging_bytes, std::max(L->gu_bytes, L->dn_bytes), ctx));
  if (has_gu) {
    HIP_TRY(rmoe::launch_relayout_out(L->gu + (size_t)expert * L->gu_bytes, ctx->s.staging, 2 * L->I, L->H, ctx->stream));
    HIP_TRY(hipMemcpyAsync(gate_up, ctx->s.staging, L->gu_bytes, hipMemcpyDeviceToHost, ctx->stream));
    HIP_TRY(hipStreamSynchronize(ctx->stream));
  }
  if (L->dn_fmt == RMOE_FMT_BFP16)
    HIP_TRY(rmoe::launch_b16_relayout_out(L->dn + (size_t)expert * L->dn_bytes, ctx->s.staging, L->H, L->Ipad, ctx->stream));
  else
    HIP_TRY(rmoe::launch_relayout_out(L->dn + (size_t)expert * L->dn_bytes, ctx->s.staging, L->H, L->Ipad, ctx->stream));
  HIP_TRY(hipMemcpyAsync(down, ctx->s.staging, L->dn_bytes, hipMemcpyDeviceToHost, ctx->stream));
  HIP_TRY(hipStreamSynchronize(ctx->stream));
  return RMOE_OK;
}

static int set_router_common(rmoe_ctx* ctx, RmoeLayer* L, const void* w, bool w_on_device, const float* bias, int score,
                             int renormalize, float scaling) {
  if (!w) return fail(RMOE_EINVAL, "null router weight");
  if (score != RMOE_SCORE_SIGMOID && score != RMOE_SCORE_SOFTMAX) return fail(RMOE_EINVAL, "unknown router score %d", score);
  HIP_TRY(hipSetDevice(ctx->device));
  const size_t wb = (size_t)L->n_routed * L->H * 2;
  if (!L->router_w && hipMalloc((void**)&L->router_w, wb) != hipSuccess) return fail(RMOE_ENOMEM, "hipMalloc failed");
  HIP_TRY(hipMemcpyAsync(L->router_w, w, wb, w_on_device ? hipMemcpyDeviceToDevice : hipMemcpyHostToDevice, ctx->stream));
  if (bias) {
    if (!L->router_bias && hipMalloc((void**)&L->router_bias, L->n_routed * sizeof(float)) != hipSuccess)
      return fail(RMOE_ENOMEM, "hipMalloc failed");
    HIP_TRY(hipMemcpyAsync(L->router_bias, bias, L->n_routed * sizeof(float), hipMemcpyHostToDevice, ctx->stream));
  } else if (L->router_bias) {
    HIP_TRY(hipStreamSynchronize(ctx->stream));
    hipFree(L->router_bias);
    L->router_bias = nullptr;
  }
  HIP_TRY(hipStreamSynchronize(ctx->stream));
  L->score = score;
  L->renorm = renormalize ? 1 : 0;
  L->scaling = scaling;
  L->has_router = true;
  return RMOE_OK;
}

int rmoe_layer_set_router(rmoe_ctx* ctx, int layer, const uint16_t* weight, const float* bias, int score,
                          int renormalize, float scaling) {
  RmoeLayer* L;
  TRY(check_layer(ctx, layer, &L));
  return set_router_common(ctx, L, weight, false, bias, score, renormalize, scaling);
}

int rmoe_layer_set_router_dev(rmoe_ctx* ctx, int layer, const void* weight_dev, const float* bias_host, int score,
                              int renormalize, float scaling) {
  RmoeLayer* L;
  TRY(check_layer(ctx, layer, &L));
  return set_router_common(ctx, L, weight_dev, true, bias_host, score, renormalize, scaling);
}

int rmoe_route(rmoe_ctx* ctx, int layer, const uint16_t* x, int T, int32_t* top_ids, float* weights, float* logits) {
  RmoeLayer* L;
  TRY(check_layer(ctx, layer, &L));
  if (!L->has_router) return fail(RMOE_EINVAL, "layer %d has no router", layer);
  if (!x || !top_ids || !weights || T < 1) return fail(RMOE_EINVAL, "bad argument");
  HIP_TRY(hipSetDevice(ctx->device));
  TRY(reserve_layer(ctx, *L, T, L->top_k));
  const size_t xb = align_up((size_t)T * L->H * 2, 256);
  uint8_t* io;
  TRY(io_area(ctx, xb, &io));
  HIP_TRY(hipMemcpyAsync(io, x, (size_t)T * L->H * 2, hipMemcpyHostToDevice, ctx->stream));
  HIP_TRY(rmoe::launch_route(*L, (const uint16_t*)io, T, ctx->s.ids, ctx->s.wts, ctx->s.logits, ctx->s, ctx->stream));
  HIP_TRY(hipMemcpyAsync(top_ids, ctx->s.ids, (size_t)T * L->top_k * 4, hipMemcpyDeviceToHost, ctx->stream));
  HIP_TRY(hipMemcpyAsync(weights, ctx->s.wts, (size_t)T * L->top_k * 4, hipMemcpyDeviceToHost, ctx->stream));
  if (logits)
    HIP_TRY(hipMemcpyAsync(logits, ctx->s.logits, (size_t)T * L->n_routed * 4, hipMemcpyDeviceToHost, ctx->stream));
  HIP_TRY(hipStreamSynchronize(ctx->stream));
  return RMOE_OK;
}

// The per-stage decode kernels' shape limits (rows per workgroup, activations of every
// slot in one workgroup's LDS).
static int check_decode_shape(const RmoeLayer& L, int slots, int layer) {
  if (rmoe::decode_band_check(L, slots) != hipSuccess)
    return fail(RMOE_EINVAL,
                "layer %d with %d expert slots exceeds the decode kernels' shape limits (I %% 16, H %% 8, %zu bytes "
                "of LDS)",
                layer, slots, rmoe::kDecodeMaxLds);
  return RMOE_OK;
}

int rmoe_moe_experts(rmoe_ctx* ctx, int layer, const uint16_t* x, const int32_t* top_ids, const float* top_weights,
                     int k, int act, float gate_beta, float value_beta, uint16_t* out) {
  RmoeLayer* L;
  TRY(check_layer(ctx, layer, &L));
  if (!x || !top_ids || !top_weights || !out) return fail(RMOE_EINVAL, "null argument");
  if (k < 1 || k > 16) return fail(RMOE_EINVAL, "k (%d) must be in 1..16", k);
  if (act != RMOE_ACT_SITU && act != RMOE_ACT_SWIGLU) return fail(RMOE_EINVAL, "unknown activation %d", act);
  TRY(check_ids(top_ids, 1, k, L->n_routed));
  TRY(check_decode_shape(*L, k, layer));
  HIP_TRY(hipSetDevice(ctx->device));
  TRY(reserve_layer(ctx, *L, 1, k));
  const size_t xb = align_up((size_t)L->H * 2, 256);
  uint8_t* io;
  TRY(io_area(ctx, 2 * xb + 256, &io));
  uint16_t* xd = (uint16_t*)io;
  uint16_t* od = (uint16_t*)(io + xb);
  HIP_TRY(hipMemcpyAsync(xd, x, (size_t)L->H * 2, hipMemcpyHostToDevice, ctx->stream));
  HIP_TRY(hipMemcpyAsync(ctx->s.ids, top_ids, (size_t)k * 4, hipMemcpyHostToDevice, ctx->stream));
  HIP_TRY(hipMemcpyAsync(ctx->s.wts, top_weights, (size_t)k * 4, hipMemcpyHostToDevice, ctx->stream));
  HIP_TRY(rmoe::launch_moe_decode(*L, xd, ctx->s.ids, ctx->s.wts, k, false, act, gate_beta, value_beta, false, nullptr,
                                  od, ctx->s, ctx->stream));
  HIP_TRY(hipMemcpyAsync(out, od, (size_t)L->H * 2, hipMemcpyDeviceToHost, ctx->stream));
  HIP_TRY(hipStreamSynchronize(ctx->stream));
  return RMOE_OK;
}

int rmoe_moe_experts_dev(rmoe_ctx* ctx, int layer, const void* x_dev, const void* top_ids_dev,
                         const void* top_weights_dev, int k, int act, float gate_beta, float value_beta,
                         void* out_dev, void* stream) {
  RmoeLayer* L;
  TRY(check_layer(ctx, layer, &L));
  if (!x_dev || !top_ids_dev || !top_weights_dev || !out_dev) return fail(RMOE_EINVAL, "null argument");
  if (k < 1 || k > 16 || k > L->n_routed) return fail(RMOE_EINVAL, "k (%d) must be in 1..min(16, n_routed)", k);
  if (act != RMOE_ACT_SITU && act != RMOE_ACT_SWIGLU) return fail(RMOE_EINVAL, "unknown activation %d", act);
  TRY(check_decode_shape(*L, k, layer));
  hipError_t e = rmoe::launch_moe_decode(*L, (const uint16_t*)x_dev, (const int32_t*)top_ids_dev,
                                         (const float*)top_weights_dev, k, false, act, gate_beta, value_beta, false,
                                         nullptr, (uint16_t*)out_dev, ctx->s, pick_stream(ctx, stream));
  if (e == hipErrorInvalidValue)
    return fail(RMOE_EINVAL, "scratch too small for layer %d with k=%d: call rmoe_reserve", layer, k);
  HIP_TRY(e);
  return RMOE_OK;
}

int rmoe_moe_experts_static_dev(rmoe_ctx* ctx, int layer, const void* x_dev, const void* top_ids_dev,
                                const void* top_weights_dev, int k, int act, float gate_beta, float value_beta,
                                void* out_dev, void* stream) {
  RmoeLayer* L;
  TRY(check_layer(ctx, layer, &L));
  if (!x_dev || !top_ids_dev || !top_weights_dev || !out_dev) return fail(RMOE_EINVAL, "null argument");
  if (k < 1 || k > 16 || k > L->n_routed) return fail(RMOE_EINVAL, "k (%d) must be in 1..min(16, n_routed)", k);
  if (act != RMOE_ACT_SITU && act != RMOE_ACT_SWIGLU) return fail(RMOE_EINVAL, "unknown activation %d", act);
  uint8_t* base = static_scratch(ctx->device);
  if (!base) return fail(RMOE_EDEVICE, "static scratch of device %d was not set up", ctx->device);
  // The scratch the routed-expert decode kernels take from a context -- the activations h
  // of k slots (no shared slot) -- in the static array.
  const size_t nh = (size_t)k * L->Ipad, need = nh * 2;
  if (need > kStaticScratchBytes)
    return fail(RMOE_EINVAL, "layer %d with k=%d needs %zu bytes of static decode scratch, more than its %zu",
                layer, k, need, kStaticScratchBytes);
  TRY(check_decode_shape(*L, k, layer));
  RmoeScratch s{};
  s.h = reinterpret_cast<uint16_t*>(base);
  s.h_elems = nh;
  s.err = ctx->s.err;
  hipError_t e = rmoe::launch_moe_decode(*L, (const uint16_t*)x_dev, (const int32_t*)top_ids_dev,
                                         (const float*)top_weights_dev, k, false, act, gate_beta, value_beta, false,
                                         nullptr, (uint16_t*)out_dev, s, pick_stream(ctx, stream));
  if (e == hipErrorInvalidValue) return fail(RMOE_EINVAL, "layer %d with k=%d does not fit the static scratch", layer, k);
  HIP_TRY(e);
  return RMOE_OK;
}

// Validate a list of decode layers for the persistent kernel; fills ptrs.
static int stack_layers(rmoe_ctx* ctx, const int* layers, int n_layers, std::vector<const RmoeLayer*>& ptrs) {
  if (!ctx) return fail(RMOE_EINVAL, "null context");
  if (!layers || n_layers < 1 || n_layers > rmoe::kMaxStack)
    return fail(RMOE_EINVAL, "n_layers (%d) must be in 1..%d", n_layers, rmoe::kMaxStack);
  if (ctx->n_cu < 1) return fail(RMOE_EDEVICE, "the persistent decode kernel cannot be resident on this device");
  ptrs.clear();
  for (int i = 0; i < n_layers; ++i) {
    RmoeLayer* L;
    TRY(check_layer(ctx, layers[i], &L));
    if (!L->has_router) return fail(RMOE_EINVAL, "layer %d has no router", layers[i]);
    if (L->n_shared < 1) return fail(RMOE_EINVAL, "layer %d has no shared expert", layers[i]);
    TRY(require_q4nx_layer(*L, layers[i], "the persistent decode kernel"));
    if (!ptrs.empty()) {
      const RmoeLayer& F = *ptrs[0];
      if (L->H != F.H || L->I != F.I || L->n_routed != F.n_routed || L->top_k != F.top_k || L->score != F.score ||
          L->renorm != F.renorm || L->scaling != F.scaling)
        return fail(RMOE_EINVAL, "layer %d differs in shape or router settings from layer %d", layers[i], layers[0]);
    }
    ptrs.push_back(L);
  }
  if (rmoe::stack_check(*ptrs[0], ctx->n_cu) != hipSuccess)
    return fail(RMOE_EINVAL, "layer shape (H=%d, I=%d, experts=%d, k=%d) exceeds the persistent decode kernel's limits",
                ptrs[0]->H, ptrs[0]->I, ptrs[0]->n_routed, ptrs[0]->top_k);
  return RMOE_OK;
}

int rmoe_set_stack_wait_limit(rmoe_ctx* ctx, unsigned polls) {
  if (!ctx) return fail(RMOE_EINVAL, "null context");
  ctx->stack_wait_limit = polls;
  return RMOE_OK;
}

int rmoe_reserve_decode_stack(rmoe_ctx* ctx, const int* layers, int n_layers) {
  std::vector<const RmoeLayer*> ptrs;
  TRY(stack_layers(ctx, layers, n_layers, ptrs));
  HIP_TRY(hipSetDevice(ctx->device));
  return reserve_stack(ctx, *ptrs[0], n_layers);
}

int rmoe_moe_decode_stack_dev(rmoe_ctx* ctx, const int* layers, int n_layers, const void* x_dev, void* out_dev,
                              int residual, int act, float gate_beta, float value_beta, void* top_ids_dev,
                              void* top_weights_dev, void* stream) {
  std::vector<const RmoeLayer*> ptrs;
  TRY(stack_layers(ctx, layers, n_layers, ptrs));
  if (!x_dev || !out_dev) return fail(RMOE_EINVAL, "null argument");
  if (act != RMOE_ACT_SITU && act != RMOE_ACT_SWIGLU) return fail(RMOE_EINVAL, "unknown activation %d", act);
  hipStream_t st = pick_stream(ctx, stream);
  hipError_t e = rmoe::launch_decode_stack(ptrs.data(), n_layers, (const uint16_t*)x_dev, (uint16_t*)out_dev,
                                           residual != 0, act, gate_beta, value_beta, (int32_t*)top_ids_dev,
                                           (float*)top_weights_dev, ctx->s, ctx->n_cu, ctx->stack_wait_limit, st);
  if (e == hipErrorInvalidValue)
    return fail(RMOE_EINVAL, "decode stack scratch too small for %d layers: call rmoe_reserve_decode_stack", n_layers);
  HIP_TRY(e);
  return RMOE_OK;
}

int rmoe_moe_decode_stack(rmoe_ctx* ctx, const int* layers, int n_layers, const uint16_t* x, uint16_t* out,
                          int residual, int act, float gate_beta, float value_beta, int32_t* top_ids,
                          float* top_weights) {
  std::vector<const RmoeLayer*> ptrs;
  TRY(stack_layers(ctx, layers, n_layers, ptrs));
  if (!x || !out) return fail(RMOE_EINVAL, "null argument");
  HIP_TRY(hipSetDevice(ctx->device));
  TRY(reserve_stack(ctx, *ptrs[0], n_layers));
  const RmoeLayer& L = *ptrs[0];
  const size_t xb = align_up((size_t)L.H * 2, 256), rb = align_up((size_t)n_layers * L.top_k * 4, 256);
  uint8_t* io;
  TRY(io_area(ctx, 2 * xb + 2 * rb, &io));
  // The persistent kernel needs every CU: the synchronous entry point first waits for all
  // work this process has queued on the device (any stream), so none of it can still hold
  // CUs when the stack starts.  (Work of other processes, and the _dev entry points, which
  // a caller may capture into a graph, are the caller's to keep apart.)
  HIP_TRY(hipDeviceSynchronize());
  HIP_TRY(hipMemcpyAsync(io, x, (size_t)L.H * 2, hipMemcpyHostToDevice, ctx->stream));
  TRY(rmoe_moe_decode_stack_dev(ctx, layers, n_layers, io, io + xb, residual, act, gate_beta, value_beta,
                                io + 2 * xb, io + 2 * xb + rb, nullptr));
  TRY(sync_and_check(ctx, ctx->stream));
  HIP_TRY(hipMemcpy(out, io + xb, (size_t)L.H * 2, hipMemcpyDeviceToHost));
  if (top_ids) HIP_TRY(hipMemcpy(top_ids, io + 2 * xb, (size_t)n_layers * L.top_k * 4, hipMemcpyDeviceToHost));
  if (top_weights)
    HIP_TRY(hipMemcpy(top_weights, io + 2 * xb + rb, (size_t)n_layers * L.top_k * 4, hipMemcpyDeviceToHost));
  return RMOE_OK;
}

int rmoe_moe_decode_dev(rmoe_ctx* ctx, int layer, const void* x_dev, void* out_dev, int residual, int act,
                        float gate_beta, float value_beta, void* top_ids_dev, void* top_weights_dev, void* stream) {
  return rmoe_moe_decode_stack_dev(ctx, &layer, 1, x_dev, out_dev, residual, act, gate_beta, value_beta, top_ids_dev,
                                   top_weights_dev, stream);
}

int rmoe_moe_decode_stage_dev(rmoe_ctx* ctx, int layer, int stage, const void* x_dev, void* out_dev, int residual,
                              int act, float gate_beta, float value_beta, void* stream) {
  RmoeLayer* L;
  TRY(check_layer(ctx, layer, &L));
  if (stage < 0 || stage > 2) return fail(RMOE_EINVAL, "stage must be 0 (router), 1 (gate/up) or 2 (down)");
  if (!L->has_router || L->n_shared < 1) return fail(RMOE_EINVAL, "layer %d needs a router and a shared expert", layer);
  TRY(require_q4nx_layer(*L, layer, "rmoe_moe_decode_stage_dev"));
  if (!x_dev || (stage == 2 && !out_dev)) return fail(RMOE_EINVAL, "null argument");
  if (act != RMOE_ACT_SITU && act != RMOE_ACT_SWIGLU) return fail(RMOE_EINVAL, "unknown activation %d", act);
  if ((size_t)L->top_k > ctx->s.route_elems || (size_t)L->n_routed > ctx->s.logit_elems)
    return fail(RMOE_EINVAL, "scratch not reserved for layer %d", layer);
  if (stage > 0) TRY(check_decode_shape(*L, L->top_k + 1, layer));
  hipStream_t st = pick_stream(ctx, stream);
  hipError_t e;
  if (stage == 0) {
    e = rmoe::launch_route(*L, (const uint16_t*)x_dev, 1, ctx->s.ids, ctx->s.wts, ctx->s.logits, ctx->s, st);
  } else {
    e = rmoe::launch_moe_decode(*L, (const uint16_t*)x_dev, ctx->s.ids, ctx->s.wts, L->top_k, true, act, gate_beta,
                                value_beta, residual != 0, (uint16_t*)out_dev, nullptr, ctx->s, st, stage == 1 ? 1 : 2);
  }
  if (e == hipErrorInvalidValue) return fail(RMOE_EINVAL, "scratch too small for layer %d: call rmoe_reserve", layer);
  HIP_TRY(e);
  return RMOE_OK;
}

int rmoe_moe_decode(rmoe_ctx* ctx, int layer, const uint16_t* x, uint16_t* out, int residual, int act,
                    float gate_beta, float value_beta, int32_t* top_ids, float* top_weights) {
  return rmoe_moe_decode_stack(ctx, &layer, 1, x, out, residual, act, gate_beta, value_beta, top_ids, top_weights);
}

int rmoe_dispatch(rmoe_ctx* ctx, const int32_t* top_ids, int T, int k, int n_experts, int32_t* order, int32_t* offsets) {
  if (!ctx || !top_ids || !order || !offsets) return fail(RMOE_EINVAL, "null argument");
  if (T < 1 || k < 1) return fail(RMOE_EINVAL, "top_ids must have shape [tokens, routes]");
  if (n_experts < 1 || n_experts > 256) return fail(RMOE_EINVAL, "n_experts (%d) must be in 1..256", n_experts);
  TRY(check_ids(top_ids, T, k, n_experts));
  HIP_TRY(hipSetDevice(ctx->device));
  const size_t n = (size_t)T * k;
  const size_t nchunks = (n + 1023) / 1024;
  TRY(grow(ctx->s.chunk_counts, ctx->s.chunk_elems, nchunks * 256, ctx));
  const size_t ib = align_up(n * 4, 256);
  uint8_t* io;
  TRY(io_area(ctx, 2 * ib + align_up((size_t)(n_experts + 1) * 4, 256), &io));
  int32_t* idd = (int32_t*)io;
  int32_t* ord = (int32_t*)(io + ib);
  int32_t* off = (int32_t*)(io + 2 * ib);
  HIP_TRY(hipMemcpyAsync(idd, top_ids, n * 4, hipMemcpyHostToDevice, ctx->stream));
  HIP_TRY(rmoe::launch_dispatch(idd, T, k, n_experts, ord, nullptr, off, ctx->s, ctx->stream));
  HIP_TRY(hipMemcpyAsync(order, ord, n * 4, hipMemcpyDeviceToHost, ctx->stream));
  HIP_TRY(hipMemcpyAsync(offsets, off, (size_t)(n_experts + 1) * 4, hipMemcpyDeviceToHost, ctx->stream));
  return sync_and_check(ctx, ctx->stream);
}

int rmoe_moe_experts_grouped(rmoe_ctx* ctx, int layer, const uint16_t* x, int T, const int32_t* top_ids,
                             const float* top_weights, const uint16_t* shared_gu, int act, float gate_beta,
                             float value_beta, uint16_t* routed, uint16_t* shared_down) {
  RmoeLayer* L;
  TRY(check_layer(ctx, layer, &L));
  if (!x || !top_ids || !top_weights || !shared_gu || !routed || !shared_down) return fail(RMOE_EINVAL, "null argument");
  if (T < 1) return fail(RMOE_EINVAL, "T must be >= 1");
  if (L->n_shared < 1) return fail(RMOE_EINVAL, "layer %d has no shared expert", layer);
  if (act != RMOE_ACT_SITU && act != RMOE_ACT_SWIGLU) return fail(RMOE_EINVAL, "unknown activation %d", act);
  TRY(check_ids(top_ids, T, L->top_k, L->n_routed));
  if (const char* why = rmoe::prefill_shape_error(*L, false)) return fail(RMOE_EINVAL, "layer %d: %s", layer, why);
  HIP_TRY(hipSetDevice(ctx->device));
  TRY(reserve_layer(ctx, *L, T, L->top_k));
  const int k = L->top_k;
  const size_t xb = align_up((size_t)T * L->H * 2, 256), ib = align_up((size_t)T * k * 4, 256),
               gb = align_up((size_t)T * 2 * L->I * 2, 256);
  uint8_t* io;
  TRY(io_area(ctx, 3 * xb + 2 * ib + gb, &io));
  uint16_t* xd = (uint16_t*)io;
  uint16_t* rd = (uint16_t*)(io + xb);
  uint16_t* sd = (uint16_t*)(io + 2 * xb);
  int32_t* idd = (int32_t*)(io + 3 * xb);
  float* wd = (float*)(io + 3 * xb + ib);
  uint16_t* gd = (uint16_t*)(io + 3 * xb + 2 * ib);
  HIP_TRY(hipMemcpyAsync(xd, x, (size_t)T * L->H * 2, hipMemcpyHostToDevice, ctx->stream));
  HIP_TRY(hipMemcpyAsync(idd, top_ids, (size_t)T * k * 4, hipMemcpyHostToDevice, ctx->stream));
  HIP_TRY(hipMemcpyAsync(wd, top_weights, (size_t)T * k * 4, hipMemcpyHostToDevice, ctx->stream));
  HIP_TRY(hipMemcpyAsync(gd, shared_gu, (size_t)T * 2 * L->I * 2, hipMemcpyHostToDevice, ctx->stream));
  // The grouped MFMA path for both layouts: a weights-d layer runs its q4nx moe_b1 through
  // the gate/up GEMM and its bfp16 moe_b2 (routed experts and the shared expert, its last)
  // through the bfp16 down GEMM.
  HIP_TRY(rmoe::launch_moe_prefill(*L, xd, T, idd, wd, nullptr, nullptr, gd, act, gate_beta, value_beta, false,
                                   nullptr, rd, sd, ctx->s.pf, ctx->s.pf_bytes, ctx->s, ctx->stream));
  HIP_TRY(hipMemcpyAsync(routed, rd, (size_t)T * L->H * 2, hipMemcpyDeviceToHost, ctx->stream));
  HIP_TRY(hipMemcpyAsync(shared_down, sd, (size_t)T * L->H * 2, hipMemcpyDeviceToHost, ctx->stream));
  return sync_and_check(ctx, ctx->stream);
}

int rmoe_moe_experts_grouped_dev(rmoe_ctx* ctx, int layer, const void* x_dev, int T, const void* top_ids_dev,
                                 const void* top_weights_dev, const void* shared_gu_dev, int act, float gate_beta,
                                 float value_beta, void* routed_dev, void* shared_down_dev, void* stream) {
  RmoeLayer* L;
  TRY(check_layer(ctx, layer, &L));
  if (!x_dev || !top_ids_dev || !top_weights_dev || !shared_gu_dev || !routed_dev || !shared_down_dev)
    return fail(RMOE_EINVAL, "null argument");
  if (T < 1) return fail(RMOE_EINVAL, "T must be >= 1");
  if (L->n_shared < 1) return fail(RMOE_EINVAL, "layer %d has no shared expert", layer);
  if (act != RMOE_ACT_SITU && act != RMOE_ACT_SWIGLU) return fail(RMOE_EINVAL, "unknown activation %d", act);
  if (T > ctx->s.max_tokens) return fail(RMOE_EINVAL, "T=%d exceeds the reserved %d tokens: call rmoe_reserve", T, ctx->s.max_tokens);
  if (const char* why = rmoe::prefill_shape_error(*L, false)) return fail(RMOE_EINVAL, "layer %d: %s", layer, why);
  hipError_t e = rmoe::launch_moe_prefill(*L, (const uint16_t*)x_dev, T, (const int32_t*)top_ids_dev,
                                          (const float*)top_weights_dev, nullptr, nullptr,
                                          (const uint16_t*)shared_gu_dev, act, gate_beta, value_beta, false, nullptr,
                                          (uint16_t*)routed_dev, (uint16_t*)shared_down_dev, ctx->s.pf, ctx->s.pf_bytes,
                                          ctx->s, pick_stream(ctx, stream));
  if (e == hipErrorInvalidValue) return fail(RMOE_EINVAL, "scratch too small for T=%d: call rmoe_reserve", T);
  HIP_TRY(e);
  return RMOE_OK;
}

int rmoe_moe_prefill_dev(rmoe_ctx* ctx, int layer, const void* x_dev, int T, void* out_dev, int residual, int act,
                         float gate_beta, float value_beta, void* top_ids_dev, void* top_weights_dev, void* stream) {
  RmoeLayer* L;
  TRY(check_layer(ctx, layer, &L));
  if (!L->has_router) return fail(RMOE_EINVAL, "layer %d has no router", layer);
  if (L->n_shared < 1) return fail(RMOE_EINVAL, "layer %d has no shared expert", layer);
  TRY(require_q4nx_layer(*L, layer, "rmoe_moe_prefill_dev"));
  if (const char* why = rmoe::prefill_shape_error(*L, true)) return fail(RMOE_EINVAL, "layer %d: %s", layer, why);
  if (!x_dev || !out_dev || T < 1) return fail(RMOE_EINVAL, "bad argument");
  if (act != RMOE_ACT_SITU && act != RMOE_ACT_SWIGLU) return fail(RMOE_EINVAL, "unknown activation %d", act);
  if (T > ctx->s.max_tokens) return fail(RMOE_EINVAL, "T=%d exceeds the reserved %d tokens: call rmoe_reserve", T, ctx->s.max_tokens);
  hipStream_t st = pick_stream(ctx, stream);
  int32_t* ids = top_ids_dev ? (int32_t*)top_ids_dev : ctx->s.ids;
  float* wts = top_weights_dev ? (float*)top_weights_dev : ctx->s.wts;
  hipError_t e = rmoe::launch_moe_prefill(*L, (const uint16_t*)x_dev, T, nullptr, nullptr, ids, wts, nullptr, act,
                                          gate_beta, value_beta, residual != 0, (uint16_t*)out_dev, nullptr, nullptr,
                                          ctx->s.pf, ctx->s.pf_bytes, ctx->s, st);
  if (e == hipErrorInvalidValue) return fail(RMOE_EINVAL, "scratch too small for T=%d: call rmoe_reserve", T);
  HIP_TRY(e);
  return RMOE_OK;
}

}  // extern "C"
