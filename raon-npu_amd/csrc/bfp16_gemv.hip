// bfp16ebs8 (9-bit) dense GEMV: the device tile layout, the re-layout of the
// reference's GEMV bytes on upload and download, and y[T, M] = RTNE_bf16(x[T, K] @ W^T).
//
// Format (quant/bfp16.py:71-140): 8 consecutive input columns of a row share one
// exponent byte e; each weight is an int8 mantissa m with the value m * 2^(e - 133).
// The kernel scale is 2^(max(e, 7) - 133) (kernels/gemv_bfp16/bfp16_gemv.cc:8-22,
// kernels/gemv_bfp16/reference.py:25-48); the packer stores e >= 7 in every block.
// m * 2^(e-133) is exact in bf16, so the only roundings are the fp32 accumulation and
// the final RTNE, as in NumpyBackend.linear (host/backend.py:402-417).
//
// Reference GEMV bytes (quant/bfp16.py:216-329): blocks of 32 rows x 256 columns,
// 9,216 B, ordered ((slice * K/256 + kb) * 4 + r) with 128-row slices and 32-row
// sub-blocks r.  Inside a block two 16-row halves; per half 32 groups of 144 B: the 16
// exponent bytes of the group (one per row), then 8 columns x 16 rows of mantissas,
// column-major.
//
// Device tile: 64 rows x 128 columns, also 9,216 B; tile (rt, kt) sits at
// (rt * (K/128) + kt) * 9216, so a 64-row band is contiguous over K.
//   bytes [0, 8192):    mantissas, 8 chunks c of 64 lanes x 16 B: lane L holds the int8
//                       mantissas of row 64*rt + L, columns 128*kt + 16c .. 16c + 15.
//   bytes [8192, 9216): per lane L 16 B: byte g is the exponent of the 8-column group g
//                       (columns 128*kt + 8g .. 8g + 7) of that row.
// The lane that owns a row reads its share of a tile with nine 16-byte loads.
#include <algorithm>

#include "rmoe_internal.h"

namespace rmoe {
namespace {

constexpr int kRefHalfBytes = 4608;
constexpr int kRefGroupBytes = 144;

// Byte offset, in the reference GEMV layout, of the 144-byte group that holds row R,
// column C (the exponent of (R, C) is at +R%16, its mantissa at +16 + (C%8)*16 + R%16).
__device__ __forceinline__ size_t ref_group(int R, int C, int kb_n) {
  const int slice = R >> 7, r = (R >> 5) & 3, h = (R >> 4) & 1;
  const int kb = C >> 8, gi = (C & 255) >> 3;
  const size_t block = ((size_t)slice * kb_n + kb) * 4 + r;
  return block * kB16TileBytes + h * kRefHalfBytes + gi * kRefGroupBytes;
}

// One thread per (tile, lane): gathers the 144 bytes that row 64*rt + lane holds in
// tile (rt, kt).  Neighbouring lanes read neighbouring bytes of the reference layout.
__global__ __launch_bounds__(256) void b16_relayout_in_kernel(const uint8_t* __restrict__ src,
                                                              uint8_t* __restrict__ tiles, int M, int K) {
  const int nkt = K / kTileCols, kb_n = K / 256;
  const size_t idx = (size_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (idx >= (size_t)(M / kTileRows) * nkt * 64) return;
  const size_t tile = idx >> 6;
  const int lane = (int)(idx & 63);
  const int rt = (int)(tile / nkt), kt = (int)(tile % nkt);
  const int R = rt * kTileRows + lane, r16 = R & 15;
  uint8_t* dst = tiles + tile * kB16TileBytes + lane * 16;
#pragma unroll 1
  for (int c = 0; c < 8; ++c) {
    uint32_t w[4] = {0u, 0u, 0u, 0u};
#pragma unroll
    for (int j = 0; j < 16; ++j) {
      const int C = kt * kTileCols + 16 * c + j;
      const uint32_t b = src[ref_group(R, C, kb_n) + 16 + (C & 7) * 16 + r16];
      w[j >> 2] |= b << (8 * (j & 3));
    }
    *reinterpret_cast<uint4*>(dst + c * 1024) = make_uint4(w[0], w[1], w[2], w[3]);
  }
  uint32_t e[4] = {0u, 0u, 0u, 0u};
#pragma unroll
  for (int g = 0; g < 16; ++g) {
    const uint32_t b = src[ref_group(R, kt * kTileCols + 8 * g, kb_n) + r16];
    e[g >> 2] |= b << (8 * (g & 3));
  }
  *reinterpret_cast<uint4*>(dst + kB16MantBytes) = make_uint4(e[0], e[1], e[2], e[3]);
}

// The inverse: every reference byte is written exactly once.
__global__ __launch_bounds__(256) void b16_relayout_out_kernel(const uint8_t* __restrict__ tiles,
                                                               uint8_t* __restrict__ dst, int M, int K) {
  const int nkt = K / kTileCols, kb_n = K / 256;
  const size_t idx = (size_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (idx >= (size_t)(M / kTileRows) * nkt * 64) return;
  const size_t tile = idx >> 6;
  const int lane = (int)(idx & 63);
  const int rt = (int)(tile / nkt), kt = (int)(tile % nkt);
  const int R = rt * kTileRows + lane, r16 = R & 15;
  const uint8_t* src = tiles + tile * kB16TileBytes + lane * 16;
#pragma unroll 1
  for (int c = 0; c < 8; ++c) {
    const uint4 v = *reinterpret_cast<const uint4*>(src + c * 1024);
    const uint32_t w[4] = {v.x, v.y, v.z, v.w};
#pragma unroll
    for (int j = 0; j < 16; ++j) {
      const int C = kt * kTileCols + 16 * c + j;
      dst[ref_group(R, C, kb_n) + 16 + (C & 7) * 16 + r16] = (uint8_t)(w[j >> 2] >> (8 * (j & 3)));
    }
  }
  const uint4 v = *reinterpret_cast<const uint4*>(src + kB16MantBytes);
  const uint32_t e[4] = {v.x, v.y, v.z, v.w};
#pragma unroll
  for (int g = 0; g < 16; ++g)
    dst[ref_group(R, kt * kTileCols + 8 * g, kb_n) + r16] = (uint8_t)(e[g >> 2] >> (8 * (g & 3)));
}

// Per row of a tiled bfp16 matrix, the largest kernel exponent max(e, 7) over the
// blocks of its first k_valid columns (columns past k_valid are padding whose bytes are
// not guaranteed).  The grouped prefill GEMM shifts each weight row by it so that every
// m * 2^(e - 133) of the row is an exact fp16 value.  One thread per row.
__global__ __launch_bounds__(256) void b16_rowexp_kernel(const uint8_t* __restrict__ tiles, int M, int K, int k_valid,
                                                         uint8_t* __restrict__ rowexp) {
  const int R = blockIdx.x * blockDim.x + threadIdx.x;
  if (R >= M) return;
  const int nkt = K / kTileCols, nblk = k_valid / 8;
  const uint8_t* base = tiles + (size_t)(R / kTileRows) * nkt * kB16TileBytes + kB16MantBytes + (R % kTileRows) * 16;
  uint32_t m = 7u;
  for (int kt = 0; kt < nkt; ++kt) {
    const uint4 v = *reinterpret_cast<const uint4*>(base + (size_t)kt * kB16TileBytes);
    const uint32_t w[4] = {v.x, v.y, v.z, v.w};
#pragma unroll
    for (int g = 0; g < 16; ++g)
      if (16 * kt + g < nblk) m = max(m, (w[g >> 2] >> (8 * (g & 3))) & 0xffu);
  }
  rowexp[R] = (uint8_t)m;
}

// ------------------------------------------------------------------------ GEMV --
constexpr int kNT = 4;         // tokens per workgroup
constexpr int kMaxRange = 32;  // K tiles per workgroup (x staged in LDS: <= 32 KB)
constexpr int kFillGroups = 2048;  // split K until the grid has about this many workgroups

struct B16Args {
  const uint8_t* tiles;
  int M, K;
  const uint16_t* x;
  int T;
  uint16_t* y;
  float* part;
  unsigned* counters;
  int ksplit;
};

__global__ __launch_bounds__(256) void linear_bfp16_kernel(B16Args a) {
  // Dynamic LDS: x of the K range as bf16 pairs [kNT][per * 64] (128 columns per tile),
  // sized by the launch for per = the range length.
  extern __shared__ __attribute__((aligned(16))) uint32_t xs[];
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
  const int xdw = nrange * 64;
  for (int i = tid; i < nt * xdw; i += blockDim.x) {
    const int t = i / xdw, c = i % xdw;
    xs[t * xstride + c] = reinterpret_cast<const uint32_t*>(a.x + (size_t)(tok0 + t) * a.K + kt0 * kTileCols)[c];
  }
  __syncthreads();

  float acc[kNT];
#pragma unroll
  for (int t = 0; t < kNT; ++t) acc[t] = 0.f;
  for (int it = wave; it < nrange; it += nwaves) {
    const uint8_t* tile = a.tiles + ((size_t)rt * nkt + kt0 + it) * kB16TileBytes + lane * 16;
    uint4 mc[8];
#pragma unroll
    for (int c = 0; c < 8; ++c) mc[c] = load_stream16(tile + c * 1024);
    const uint4 eq = load_stream16(tile + kB16MantBytes);
    const uint32_t ew[4] = {eq.x, eq.y, eq.z, eq.w};
#pragma unroll
    for (int c = 0; c < 8; ++c) {
      const uint32_t w[4] = {mc[c].x, mc[c].y, mc[c].z, mc[c].w};
      uint32_t p[8];
#pragma unroll
      for (int d = 0; d < 4; ++d) mant_pairs(w[d], p[2 * d], p[2 * d + 1]);
#pragma unroll
      for (int gg = 0; gg < 2; ++gg) {
        const int g = 2 * c + gg;
        const float s = exp_scale((ew[g >> 2] >> (8 * (g & 3))) & 0xffu);
#pragma unroll
        for (int t = 0; t < kNT; ++t) {
          if (t < nt) {
            const uint4 xv = *reinterpret_cast<const uint4*>(xs + t * xstride + it * 64 + g * 4);
            float d = dot2_bf16(p[4 * gg], xv.x, 0.f);
            d = dot2_bf16(p[4 * gg + 1], xv.y, d);
            d = dot2_bf16(p[4 * gg + 2], xv.z, d);
            d = dot2_bf16(p[4 * gg + 3], xv.w, d);
            acc[t] = fmaf(s, d, acc[t]);
          }
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

int bfp16_ksplit(int M, int K) {
  const int nkt = K / kTileCols, n_rt = M / kTileRows;
  int ks = std::min((nkt + 3) / 4, (kFillGroups + n_rt - 1) / n_rt);
  ks = std::max(ks, (nkt + kMaxRange - 1) / kMaxRange);
  return std::max(1, ks);
}

hipError_t launch_b16_relayout_in(const uint8_t* packed, uint8_t* tiles, int M, int K, hipStream_t st) {
  const size_t n = (size_t)(M / kTileRows) * (K / kTileCols) * 64;
  hipLaunchKernelGGL(b16_relayout_in_kernel, dim3((unsigned)((n + 255) / 256)), dim3(256), 0, st, packed, tiles, M, K);
  return hipGetLastError();
}

hipError_t launch_b16_rowexp(const uint8_t* tiles, int M, int K, int k_valid, uint8_t* rowexp, hipStream_t st) {
  hipLaunchKernelGGL(b16_rowexp_kernel, dim3((unsigned)((M + 255) / 256)), dim3(256), 0, st, tiles, M, K, k_valid, rowexp);
  return hipGetLastError();
}

hipError_t launch_b16_relayout_out(const uint8_t* tiles, uint8_t* packed, int M, int K, hipStream_t st) {
  const size_t n = (size_t)(M / kTileRows) * (K / kTileCols) * 64;
  hipLaunchKernelGGL(b16_relayout_out_kernel, dim3((unsigned)((n + 255) / 256)), dim3(256), 0, st, tiles, packed, M, K);
  return hipGetLastError();
}

hipError_t launch_linear_bfp16(const uint8_t* tiles, int M, int K, const uint16_t* x, int T, uint16_t* y,
                               RmoeScratch& s, hipStream_t st) {
  const int nkt = K / kTileCols, n_rt = M / kTileRows;
  const int ksplit = bfp16_ksplit(M, K);
  const int ychunks = (T + kNT - 1) / kNT;
  const size_t need_part = (size_t)ychunks * n_rt * ksplit * kNT * 64;
  const size_t need_cnt = (size_t)ychunks * n_rt;
  if (ksplit > 1 && (need_part > s.part_floats || need_cnt > s.n_counters)) return hipErrorInvalidValue;
  const int per = (nkt + ksplit - 1) / ksplit;
  if (per > kMaxRange) return hipErrorInvalidValue;
  B16Args a{tiles, M, K, x, T, y, s.part, s.counters, ksplit};
  const int threads = 64 * std::min(4, per);
  const size_t lds = (size_t)kNT * per * 64 * 4;
  hipLaunchKernelGGL(linear_bfp16_kernel, dim3(n_rt * ksplit, ychunks), dim3(threads), lds, st, a);
  return hipGetLastError();
}

}  // namespace rmoe
