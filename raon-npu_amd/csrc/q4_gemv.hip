// Dense q4nx GEMV for a few tokens: y[T, M] = RTNE(x[T, K] @ W^T).
//
// Restates the arithmetic of NumpyBackend.linear (host/backend.py:402-417) on q4nx
// weights (quant/q4nx.py:203-223): fp32 accumulation, RTNE to bf16 once at the end.
// One lane owns one weight row; a wave streams one 64x128 tile (5 x 16-byte loads
// per lane) and dots it with bf16 pairs of x broadcast from LDS.  A workgroup of up
// to four waves covers one 64-row band over a range of K tiles; bands split over K
// write fp32 partials and the last workgroup of a band (device-scope counter) adds
// them in K order, so the result does not depend on arrival order.
#include <algorithm>

#include "rmoe_internal.h"

namespace rmoe {
namespace {

constexpr int kNT = 4;             // tokens per workgroup
constexpr int kMaxRange = 32;      // K tiles per workgroup (x and group sums in LDS: <= 34 KB)
constexpr int kFillGroups = 2048;  // split K until the grid has about this many workgroups

struct LinearArgs {
  const uint8_t* tiles;
  int M, K;
  const uint16_t* x;
  int T;
  uint16_t* y;
  float* part;
  unsigned* counters;
  int ksplit;
};

__global__ __launch_bounds__(256) void linear_kernel(LinearArgs a) {
  // Dynamic LDS: x of the K range as bf16 pairs [kNT][per * 64] (128 columns per tile),
  // then the group sums [kNT][per * 4]; sized by the launch for per = the range length.
  extern __shared__ __attribute__((aligned(16))) uint32_t lin_lds[];
  __shared__ float red[4][kNT][64];
  __shared__ unsigned last_flag;

  const int nkt = a.K / kTileCols;
  const int n_rt = a.M / kTileRows;
  const int rt = blockIdx.x / a.ksplit;
  const int ks = blockIdx.x % a.ksplit;
  const int tok0 = blockIdx.y * kNT;
  const int nt = min(kNT, a.T - tok0);
  const int per = (nkt + a.ksplit - 1) / a.ksplit;
  const int kt0 = ks * per;
  const int nrange = max(0, min(per, nkt - kt0));
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int nwaves = blockDim.x >> 6;
  const int xstride = per * 64;
  uint32_t* xs = lin_lds;
  float* ssum = reinterpret_cast<float*>(lin_lds + kNT * xstride);

  // Stage x (bf16 pairs) for this K range and the per-group sums S.
  const int xdw = nrange * 64;
  for (int i = tid; i < nt * xdw; i += blockDim.x) {
    const int t = i / xdw, c = i % xdw;
    xs[t * xstride + c] = reinterpret_cast<const uint32_t*>(a.x + (size_t)(tok0 + t) * a.K + kt0 * kTileCols)[c];
  }
  __syncthreads();
  for (int i = tid; i < nt * nrange * 4; i += blockDim.x) {
    const int t = i / (nrange * 4), gi = i % (nrange * 4);
    float s = 0.f;
    for (int c = 0; c < 16; ++c) {
      const uint32_t v = xs[t * xstride + gi * 16 + c];
      s += bf16_to_f32(v & 0xffffu);
      s += bf16_to_f32(v >> 16);
    }
    ssum[t * per * 4 + gi] = s;
  }
  __syncthreads();

  float acc[kNT];
#pragma unroll
  for (int t = 0; t < kNT; ++t) acc[t] = 0.f;
  for (int it = wave; it < nrange; it += nwaves) {
    const uint8_t* tile = a.tiles + ((size_t)rt * nkt + kt0 + it) * kTileBytes;
    uint4 c[4];
#pragma unroll
    for (int j = 0; j < 4; ++j) c[j] = load_stream16(tile + j * 1024 + lane * 16);
    const uint4 smq = load_stream16(tile + kCodeBytes + lane * 16);
    const uint32_t sm[4] = {smq.x, smq.y, smq.z, smq.w};
#pragma unroll
    for (int j = 0; j < 4; ++j) {
#pragma unroll
      for (int t = 0; t < kNT; ++t) {
        if (t < nt) {
          const float d = group_dot(c[j], xs + t * xstride + it * 64 + j * 16);
          acc[t] = group_apply(sm[j], d, ssum[t * per * 4 + it * 4 + j], acc[t]);
        }
      }
    }
  }
#pragma unroll
  for (int t = 0; t < kNT; ++t) red[wave][t][lane] = acc[t];
  __syncthreads();

  // Sum the waves in order; wave w handles tokens w, w + nwaves, ...
  const int row = rt * kTileRows + lane;
  const size_t band = (size_t)blockIdx.y * n_rt + rt;
  float* part = a.part + (band * a.ksplit + ks) * (kNT * 64);
  for (int t = wave; t < nt; t += nwaves) {
    float v = 0.f;
    for (int w = 0; w < nwaves; ++w) v += red[w][t][lane];
    if (a.ksplit == 1) a.y[(size_t)(tok0 + t) * a.M + row] = (uint16_t)f32_to_bf16(v);
    else st_dev(&part[t * 64 + lane], v);
  }
  if (a.ksplit == 1) return;
  if (!arrive_last(&a.counters[band], (unsigned)a.ksplit, &last_flag)) return;
  const float* pb = a.part + band * a.ksplit * (kNT * 64);
  for (int t = wave; t < nt; t += nwaves) {
    float s = 0.f;
    for (int k2 = 0; k2 < a.ksplit; ++k2) s += ld_dev(&pb[k2 * (kNT * 64) + t * 64 + lane]);
    a.y[(size_t)(tok0 + t) * a.M + row] = (uint16_t)f32_to_bf16(s);
  }
}

}  // namespace

hipError_t launch_linear(const uint8_t* tiles, int M, int K, const uint16_t* x, int T, uint16_t* y, RmoeScratch& s,
                         hipStream_t st) {
  const int nkt = K / kTileCols, n_rt = M / kTileRows;
  // Up to 4 K tiles per workgroup (one per wave); tall matrices, whose row bands alone
  // fill the chip, split K less (down to one workgroup per band) and skip the partials.
  int ksplit = std::min((nkt + 3) / 4, (kFillGroups + n_rt - 1) / n_rt);
  ksplit = std::max({1, ksplit, (nkt + kMaxRange - 1) / kMaxRange});
  const int ychunks = (T + kNT - 1) / kNT;
  const size_t need_part = (size_t)ychunks * n_rt * ksplit * kNT * 64;
  const size_t need_cnt = (size_t)ychunks * n_rt;
  if (ksplit > 1 && (need_part > s.part_floats || need_cnt > s.n_counters)) return hipErrorInvalidValue;
  const int per = (nkt + ksplit - 1) / ksplit;
  if (per > kMaxRange) return hipErrorInvalidValue;
  LinearArgs a{tiles, M, K, x, T, y, s.part, s.counters, ksplit};
  const int threads = 64 * min(4, per);
  const size_t lds = (size_t)kNT * per * (64 + 4) * 4;
  hipLaunchKernelGGL(linear_kernel, dim3(n_rt * ksplit, ychunks), dim3(threads), lds, st, a);
  return hipGetLastError();
}

}  // namespace rmoe
