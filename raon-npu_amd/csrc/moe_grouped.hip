// Grouped (prefill) MoE: NpuBackend.moe_experts_grouped (npu/backend.py:4845-4979).
//
// routed[t]      = RTNE(sum over t's routes in ascending expert id of f32(down_e(h_e(x_t))) * w)
// shared_down[t] = RTNE(down_shared(RTNE(act(shared_gu[t]))))
// out[t]         = RTNE(f32(routed[t]) + f32(shared_down[t]))  (+ x[t] with residual)
//
// This first version runs the routed experts token by token through the decode
// kernels and the shared expert through the dense GEMV, all on the device.
#include "rmoe_internal.h"

namespace rmoe {
namespace {

// h[t, 0:I] = RTNE(act(gu[t, 0:I], gu[t, I:2I])), h[t, I:Ipad] = 0.
__global__ void act_rows_kernel(const uint16_t* __restrict__ gu, int T, int I, int Ipad, int act, float gb, float vb,
                                uint16_t* __restrict__ h) {
  const size_t idx = (size_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (idx >= (size_t)T * Ipad) return;
  const int t = (int)(idx / Ipad), c = (int)(idx % Ipad);
  uint16_t v = 0;
  if (c < I) {
    const float g = bf16_to_f32(gu[(size_t)t * 2 * I + c]);
    const float u = bf16_to_f32(gu[(size_t)t * 2 * I + I + c]);
    v = (uint16_t)f32_to_bf16(act_apply(act, g, u, gb, vb));
  }
  h[idx] = v;
}

// out[t, :] = RTNE(f32(a) + f32(b)) (+ x with residual).
__global__ void add_rows_kernel(const uint16_t* __restrict__ a, const uint16_t* __restrict__ b,
                                const uint16_t* __restrict__ x, size_t n, uint16_t* __restrict__ out) {
  const size_t idx = (size_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (idx >= n) return;
  uint32_t o = f32_to_bf16(__fadd_rn(bf16_to_f32(a[idx]), bf16_to_f32(b[idx])));
  if (x) o = f32_to_bf16(__fadd_rn(bf16_to_f32(x[idx]), bf16_to_f32(o)));
  out[idx] = (uint16_t)o;
}

}  // namespace

hipError_t launch_moe_grouped(const RmoeLayer& L, const uint16_t* x, int T, const int32_t* ids, const float* wts,
                              const uint16_t* shared_gu, bool shared_from_x, int act, float gb, float vb,
                              bool residual, uint16_t* routed, uint16_t* shared_down, uint16_t* out,
                              RmoeScratch& s, hipStream_t st) {
  const int k = L.top_k;
  if (L.n_shared < 1) return hipErrorInvalidValue;
  // Scratch layout past the decode region: sgu [T, 2I], hs [T, Ipad], sd [T, H], rt [T, H].
  const size_t need = (size_t)T * (2 * L.I + L.Ipad + 2 * L.H);
  if ((size_t)(k + 1) * L.Ipad + need > s.h_elems) return hipErrorInvalidValue;
  uint16_t* sgu = s.h + (size_t)(k + 1) * L.Ipad;
  uint16_t* hs = sgu + (size_t)T * 2 * L.I;
  uint16_t* sd = hs + (size_t)T * L.Ipad;
  uint16_t* rt = sd + (size_t)T * L.H;
  if (!routed) routed = rt;
  if (!shared_down) shared_down = sd;
  hipError_t e;
  for (int t = 0; t < T; ++t) {
    e = launch_moe_decode(L, x + (size_t)t * L.H, ids + (size_t)t * k, wts + (size_t)t * k, k, false, act, gb, vb,
                          false, nullptr, routed + (size_t)t * L.H, s, st);
    if (e != hipSuccess) return e;
  }
  const uint8_t* sh_gu = L.gu + (size_t)L.n_routed * L.gu_bytes;
  const uint8_t* sh_dn = L.dn + (size_t)L.n_routed * L.dn_bytes;
  if (shared_from_x) {
    e = launch_linear(sh_gu, 2 * L.I, L.H, x, T, sgu, s, st);
    if (e != hipSuccess) return e;
    shared_gu = sgu;
  }
  const size_t nh = (size_t)T * L.Ipad;
  hipLaunchKernelGGL(act_rows_kernel, dim3((unsigned)((nh + 255) / 256)), dim3(256), 0, st, shared_gu, T, L.I, L.Ipad,
                     act, gb, vb, hs);
  e = hipGetLastError();
  if (e != hipSuccess) return e;
  e = launch_linear(sh_dn, L.H, L.Ipad, hs, T, shared_down, s, st);
  if (e != hipSuccess) return e;
  if (out) {
    const size_t n = (size_t)T * L.H;
    hipLaunchKernelGGL(add_rows_kernel, dim3((unsigned)((n + 255) / 256)), dim3(256), 0, st, routed, shared_down,
                       residual ? x : nullptr, n, out);
    e = hipGetLastError();
  }
  return e;
}

}  // namespace rmoe
