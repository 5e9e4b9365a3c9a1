// Dense q4nx GEMV for a few tokens: y[T, M] = RTNE(x[T, K] @ W^T).
//
// Restates the arithmetic of NumpyBackend.linear (host/backend.py:402-417) on q4nx
// weights (quant/q4nx.py:203-223): fp32 accumulation, RTNE to bf16 once at the end.
// One lane owns one weight row; a wave streams one 64x128 tile (5 x 16-byte loads
// per lane) and dots it with bf16 pairs of x broadcast from LDS.  A workgroup of up
// to four waves covers one 64-row band over a range of K tiles; bands split over K
// write fp32 partials and the last workgroup of a band (device-scope counter) adds
// them in K order, so the result does not depend on arrival order.
// Matrices with at most kBandMaxTiles K tiles take linear_band_kernel instead: one
// workgroup per 16, 32 or 64 rows with the K tiles spread over its lanes and waves, no
// split and no partials.
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
  const int tid = threadIdx.x, lane = tid & 63, wave = wave_id();
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

constexpr int kBandMaxTiles = 32;  // K tiles handled by one workgroup in linear_band_kernel
constexpr int kBandMaxWaves = 16;
constexpr int kXPad = 4;           // dwords of padding after each K tile's x in LDS

// One workgroup per R rows of a 64-row band (and group of kNT tokens), no K split and
// no partials.  The wave's lanes form 64 / R groups of R rows; group g of wave w takes
// K tile w * (64 / R) + g (then every waves * (64 / R)-th further tile), so a band is
// spread over 64 / R workgroups and every SIMD streams about one tile's worth of work.
// Every lane requests its first tile before x is staged, so the latencies of the
// weights and of x overlap.  Group sums of x come from registers while x is staged.
// The lane groups' sums meet by shuffles (a fixed tree), the waves' in LDS, added in
// wave order: the result does not depend on timing.
template <int R>
__global__ __launch_bounds__(1024) void linear_band_kernel(LinearArgs a) {
  constexpr int G = 64 / R;
  // Dynamic LDS: x as bf16 pairs [kNT][nkt][64 + kXPad] (the padding puts the lane
  // groups' tiles in different banks), the group sums [kNT][nkt * 4], then the waves'
  // sums [waves][kNT][R].
  extern __shared__ __attribute__((aligned(16))) uint32_t lin_lds[];
  const int nkt = a.K / kTileCols;
  const int row0 = blockIdx.x * R;
  const int rsub = row0 % kTileRows;
  const int tok0 = blockIdx.y * kNT;
  const int nt = min(kNT, a.T - tok0);
  const int tid = threadIdx.x, lane = tid & 63, wave = wave_id();
  const int nwaves = blockDim.x >> 6;
  const int g = lane / R, r = lane % R;
  const int tstride = 64 + kXPad;
  const int xstride = nkt * tstride;
  uint32_t* xs = lin_lds;
  float* ssum = reinterpret_cast<float*>(lin_lds + kNT * xstride);
  float* red = ssum + kNT * nkt * 4;

  // This thread's first 16 bytes of x are requested before the weights: loads complete
  // in order, so x is then not held up behind the tiles and its staging overlaps them.
  const int units = nkt * 16;  // 16-byte units of x per token (8 values each)
  const int total = nt * units;
  const uint8_t* band = a.tiles + (size_t)(row0 / kTileRows) * nkt * kTileBytes + (size_t)(rsub + r) * 16;
  const int kt0 = wave * G + g;
  uint4 c[4], smq;
  {
    const uint8_t* tile = band + (size_t)(kt0 < nkt ? kt0 : 0) * kTileBytes;
#pragma unroll
    for (int j = 0; j < 4; ++j) c[j] = load_stream16(tile + j * 1024);
    smq = load_stream16(tile + kCodeBytes);
  }

  // x in 16-byte units; the 4 units of a 32-column group are held by 4 neighbouring
  // lanes, whose sums are added by shuffles.
  for (int i = tid; i < total; i += blockDim.x) {
    const int t = i / units, u = i % units;
    const uint4 v = reinterpret_cast<const uint4*>(a.x + (size_t)(tok0 + t) * a.K)[u];
    *reinterpret_cast<uint4*>(xs + t * xstride + (u >> 4) * tstride + (u & 15) * 4) = v;
    float sv = ((bf16_to_f32(v.x & 0xffffu) + bf16_to_f32(v.x >> 16)) +
                (bf16_to_f32(v.y & 0xffffu) + bf16_to_f32(v.y >> 16))) +
               ((bf16_to_f32(v.z & 0xffffu) + bf16_to_f32(v.z >> 16)) +
                (bf16_to_f32(v.w & 0xffffu) + bf16_to_f32(v.w >> 16)));
    sv += __shfl_xor(sv, 1, 64);
    sv += __shfl_xor(sv, 2, 64);
    if ((u & 3) == 0) ssum[t * nkt * 4 + (u >> 2)] = sv;
  }
  __syncthreads();

  float acc[kNT];
#pragma unroll
  for (int t = 0; t < kNT; ++t) acc[t] = 0.f;
  for (int kt = kt0; kt < nkt; kt += nwaves * G) {
    if (kt != kt0) {
      const uint8_t* tile = band + (size_t)kt * kTileBytes;
#pragma unroll
      for (int j = 0; j < 4; ++j) c[j] = load_stream16(tile + j * 1024);
      smq = load_stream16(tile + kCodeBytes);
    }
    const uint32_t sm[4] = {smq.x, smq.y, smq.z, smq.w};
#pragma unroll
    for (int j = 0; j < 4; ++j) {
#pragma unroll
      for (int t = 0; t < kNT; ++t) {
        if (t < nt) {
          const float d = group_dot(c[j], xs + t * xstride + kt * tstride + j * 16);
          acc[t] = group_apply(sm[j], d, ssum[t * nkt * 4 + kt * 4 + j], acc[t]);
        }
      }
    }
  }
#pragma unroll
  for (int t = 0; t < kNT; ++t) {
    float v = acc[t];
#pragma unroll
    for (int m = R; m < 64; m *= 2) v += __shfl_xor(v, m, 64);
    if (g == 0) red[(wave * kNT + t) * R + r] = v;
  }
  __syncthreads();
  for (int t = wave; t < nt; t += nwaves) {
    if (lane < R) {
      float v = 0.f;
      for (int w = 0; w < nwaves; ++w) v += red[(w * kNT + t) * R + lane];
      a.y[(size_t)(tok0 + t) * a.M + row0 + lane] = (uint16_t)f32_to_bf16(v);
    }
  }
}

// One token of a small matrix without LDS: lane (q, r) of a wave takes row row0 + r and half
// hf = q & 1 of K tile kt = q >> 1 (groups 2hf and 2hf + 1: two 16-byte code words and
// their two scale|min words).  It loads its 64 columns of x straight from memory (the R
// lanes of one half share the addresses) and takes their group sums S on v_dot2 against
// the pair (1.0, 1.0).  The 2 NKT lanes of a row add their partial sums by shuffles in a
// fixed order; R = 64 / (2 NKT) rows per wave.  Half the dot-product work per lane of
// a one-lane-per-tile form, and no x staging in LDS or wave barrier.
template <int NKT>
__global__ __launch_bounds__(64) void linear_lane_kernel(LinearArgs a) {
  constexpr int R = 32 / NKT;
  const int lane = threadIdx.x;
  // Workgroups are dealt round robin to the 8 XCDs: XCD x takes a contiguous eighth of the
  // rows, so the workgroups that share a 128-byte line of a tile (its 16-byte row pieces)
  // share an L2 (grid = M / R, a multiple of 8).
  const int wg = blockIdx.x, per_xcd = gridDim.x / 8;
  const int row0 = ((wg % 8) * per_xcd + wg / 8) * R;
  const int q = lane / R, r = lane % R, kt = q >> 1, hf = q & 1;
  const uint8_t* tile =
      a.tiles + ((size_t)(row0 / kTileRows) * NKT + kt) * kTileBytes + (size_t)(row0 % kTileRows + r) * 16;
  const uint4 c0 = load_stream16(tile + (2 * hf) * 1024);
  const uint4 c1 = load_stream16(tile + (2 * hf + 1) * 1024);
  const uint2 smv = *reinterpret_cast<const uint2*>(tile + kCodeBytes + 8 * hf);
  const uint4* xp = reinterpret_cast<const uint4*>(a.x) + (kt * 128 + hf * 64) / 8;
  uint4 xv[8];
#pragma unroll
  for (int i = 0; i < 8; ++i) xv[i] = xp[i];
  uint32_t mask, one;
  q4_unpack_consts(mask, one);
  float acc = 0.f;
#pragma unroll
  for (int j = 0; j < 2; ++j) {
    const uint32_t cw[4] = {j ? c1.x : c0.x, j ? c1.y : c0.y, j ? c1.z : c0.z, j ? c1.w : c0.w};
    float d = 0.f, s = 0.f;
#pragma unroll
    for (int dd = 0; dd < 4; ++dd) {
      uint32_t p0, p1, p2, p3;
      unpack_codes(cw[dd], p0, p1, p2, p3);
      const uint4 x4 = xv[4 * j + dd];
      d = dot2_bf16(p0, x4.x, d);
      d = dot2_bf16(p1, x4.y, d);
      d = dot2_bf16(p2, x4.z, d);
      d = dot2_bf16(p3, x4.w, d);
      s = dot2_bf16(one, x4.x, s);
      s = dot2_bf16(one, x4.y, s);
      s = dot2_bf16(one, x4.z, s);
      s = dot2_bf16(one, x4.w, s);
    }
    acc = group_apply(j ? smv.y : smv.x, d, s, acc);
  }
#pragma unroll
  for (int m = R; m < 64; m *= 2) acc += __shfl_xor(acc, m, 64);
  if (lane < R) a.y[row0 + lane] = (uint16_t)f32_to_bf16(acc);
}

}  // namespace

hipError_t launch_linear(const uint8_t* tiles, int M, int K, const uint16_t* x, int T, uint16_t* y, RmoeScratch& s,
                         hipStream_t st) {
  const int nkt = K / kTileCols, n_rt = M / kTileRows;
  const int ychunks = (T + kNT - 1) / kNT;
  // One token of a small matrix (fewer than 32 row bands) with 4..32 K tiles: one wave
  // per workgroup, two lanes per K tile of a row (config 1: 3.05 -> 2.07 us per launch in
  // a graph against one lane per K tile with x staged in LDS).  With more tokens the band
  // kernel is faster.
  if (T == 1 && n_rt < 32 && (nkt == 4 || nkt == 8 || nkt == 16 || nkt == 32) &&
      (reinterpret_cast<uintptr_t>(x) & 15) == 0) {
    LinearArgs a{tiles, M, K, x, T, y, nullptr, nullptr, 1};
    const dim3 grid(M / (32 / nkt)), block(64);
    if (nkt == 4) hipLaunchKernelGGL(linear_lane_kernel<4>, grid, block, 0, st, a);
    else if (nkt == 8) hipLaunchKernelGGL(linear_lane_kernel<8>, grid, block, 0, st, a);
    else if (nkt == 16) hipLaunchKernelGGL(linear_lane_kernel<16>, grid, block, 0, st, a);
    else hipLaunchKernelGGL(linear_lane_kernel<32>, grid, block, 0, st, a);
    return hipGetLastError();
  }
  // The band kernel reads x in 16-byte pieces; other x take the K-split kernel.
  if (nkt <= kBandMaxTiles && (reinterpret_cast<uintptr_t>(x) & 15) == 0) {
    // Rows per workgroup: whole bands when the bands alone fill the chip, else 32 or 16
    // rows, so that a small matrix still spreads over many CUs.
    const int R = n_rt >= 64 ? 64 : n_rt >= 32 ? 32 : 16;
    const int G = 64 / R;
    const int waves = std::min(kBandMaxWaves, (nkt + G - 1) / G);
    const size_t lds = ((size_t)kNT * nkt * (64 + kXPad + 4) + (size_t)waves * kNT * R) * 4;
    LinearArgs a{tiles, M, K, x, T, y, nullptr, nullptr, 1};
    const dim3 grid(M / R, ychunks), block(64 * waves);
    if (R == 64) hipLaunchKernelGGL(linear_band_kernel<64>, grid, block, lds, st, a);
    else if (R == 32) hipLaunchKernelGGL(linear_band_kernel<32>, grid, block, lds, st, a);
    else hipLaunchKernelGGL(linear_band_kernel<16>, grid, block, lds, st, a);
    return hipGetLastError();
  }
  // Up to 4 K tiles per workgroup (one per wave); tall matrices, whose row bands alone
  // fill the chip, split K less (down to one workgroup per band) and skip the partials.
  int ksplit = std::min((nkt + 3) / 4, (kFillGroups + n_rt - 1) / n_rt);
  ksplit = std::max({1, ksplit, (nkt + kMaxRange - 1) / kMaxRange});
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
