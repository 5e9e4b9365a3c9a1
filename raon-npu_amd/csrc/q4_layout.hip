// q4nx format kernels: pack_gemv <-> device tile layout, and the device quantizer.
//
// pack_gemv layout: quant/q4nx.py:335-393 (32x256 blocks of 5,120 B, block order
// ((slice*k_blocks + kb)*4 + r), scales/mins [group][row], codes in
// (half, group, col, row16) order with two rows per byte).  The device tile layout
// is described in rmoe_internal.h.
#include "rmoe_internal.h"

namespace rmoe {
namespace {

// Position of (row r, group g) inside a pack_gemv buffer.
struct PackPos {
  size_t base;  // block byte offset
  int r32, half, r16, gg;
};

__device__ __forceinline__ PackPos pack_pos(int r, int g, int K) {
  const int kblocks = K / 256;
  const int slice = r / 128, rw = (r % 128) / 32, r32 = r % 32;
  const int kb = g / 8, gg = g % 8;
  PackPos p;
  p.base = ((size_t)(slice * kblocks + kb) * 4 + rw) * 5120;
  p.r32 = r32;
  p.half = r32 / 16;
  p.r16 = r32 % 16;
  p.gg = gg;
  return p;
}

// Column c (0..31) of a group -> (dword, nibble) inside the lane's 16 bytes.
__device__ __forceinline__ int tile_nibble_index(int c) {
  const int d = c >> 3, w = c & 7;
  const int q = (w & 1) ? (w >> 1) + 4 : (w >> 1);
  return d * 8 + q;  // nibble index 0..31 over the 4 dwords
}

// Thread = (tile, j, lane): gathers row (64*rt + lane), group (4*kt + j).
__global__ void relayout_in_kernel(const uint8_t* __restrict__ packed, uint8_t* __restrict__ tiles, int M, int K) {
  const int G = K / 32, nkt = K / 128;
  const size_t n = (size_t)M * G;
  const size_t idx = (size_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (idx >= n) return;
  const int lane = idx & 63;
  const size_t rest = idx >> 6;
  const int j = rest & 3;
  const size_t tile = rest >> 2;
  const int rt = (int)(tile / nkt), kt = (int)(tile % nkt);
  const int r = rt * 64 + lane, g = kt * 4 + j;
  const PackPos p = pack_pos(r, g, K);
  const uint16_t* sm = reinterpret_cast<const uint16_t*>(packed + p.base);
  const uint32_t scale = sm[p.gg * 32 + p.r32];
  const uint32_t mn = sm[256 + p.gg * 32 + p.r32];
  uint32_t w[4] = {0u, 0u, 0u, 0u};
  const uint8_t* cbase = packed + p.base + 1024 + (size_t)((p.half * 8 + p.gg) * 32) * 8 + (p.r16 >> 1);
  const int shift = (p.r16 & 1) ? 4 : 0;
#pragma unroll 8
  for (int c = 0; c < 32; ++c) {
    const uint32_t code = (cbase[c * 8] >> shift) & 15u;
    const int ni = tile_nibble_index(c);
    w[ni >> 3] |= code << (4 * (ni & 7));
  }
  uint8_t* t = tiles + tile * kTileBytes;
  *reinterpret_cast<uint4*>(t + j * 1024 + lane * 16) = make_uint4(w[0], w[1], w[2], w[3]);
  *reinterpret_cast<uint32_t*>(t + kCodeBytes + lane * 16 + j * 4) = scale | (mn << 16);
}

// Thread = (row pair, group): writes both rows' nibbles (one byte per column).
__global__ void relayout_out_kernel(const uint8_t* __restrict__ tiles, uint8_t* __restrict__ packed, int M, int K) {
  const int G = K / 32, nkt = K / 128;
  const size_t n = (size_t)(M / 2) * G;
  const size_t idx = (size_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (idx >= n) return;
  const int g = (int)(idx % G);
  const int r0 = (int)(idx / G) * 2;
  const int kt = g / 4, j = g % 4;
  uint32_t w[2][4];
  uint32_t smv[2];
#pragma unroll
  for (int h = 0; h < 2; ++h) {
    const int r = r0 + h;
    const uint8_t* t = tiles + ((size_t)(r / 64) * nkt + kt) * kTileBytes;
    const uint4 c = *reinterpret_cast<const uint4*>(t + j * 1024 + (r % 64) * 16);
    w[h][0] = c.x; w[h][1] = c.y; w[h][2] = c.z; w[h][3] = c.w;
    smv[h] = *reinterpret_cast<const uint32_t*>(t + kCodeBytes + (r % 64) * 16 + j * 4);
  }
  const PackPos p = pack_pos(r0, g, K);
  uint16_t* sm = reinterpret_cast<uint16_t*>(packed + p.base);
  sm[p.gg * 32 + p.r32] = (uint16_t)(smv[0] & 0xffffu);
  sm[p.gg * 32 + p.r32 + 1] = (uint16_t)(smv[1] & 0xffffu);
  sm[256 + p.gg * 32 + p.r32] = (uint16_t)(smv[0] >> 16);
  sm[256 + p.gg * 32 + p.r32 + 1] = (uint16_t)(smv[1] >> 16);
  uint8_t* cbase = packed + p.base + 1024 + (size_t)((p.half * 8 + p.gg) * 32) * 8 + (p.r16 >> 1);
#pragma unroll 8
  for (int c = 0; c < 32; ++c) {
    const int ni = tile_nibble_index(c);
    const uint32_t lo = (w[0][ni >> 3] >> (4 * (ni & 7))) & 15u;
    const uint32_t hi = (w[1][ni >> 3] >> (4 * (ni & 7))) & 15u;
    cbase[c * 8] = (uint8_t)(lo | (hi << 4));
  }
}

// ------------------------------------------------------------ Q4_K -> tiles --
// llama.cpp block_q4_K (quant/gguf_q4k.py:189-233): 144 bytes per 256 weights of a row --
// d (fp16), dmin (fp16), eight 6-bit scales and mins in 12 bytes, 128 code bytes (sub-
// block 2p = low nibbles of bytes 32p..32p+31, 2p+1 = their high nibbles).  q4nx keeps
// every code; group j's parameters are RTNE bf16 of d*sc[j] and -dmin*mn[j] (exact fp32
// products).  Thread = (tile row band, K tile, group j, lane): row row0 + 64*band + lane,
// group 4*kt + j of a tile matrix Kt wide; groups at or past K are the zero padding
// (codes 0, scale 0, min 0).
__global__ void q4k_to_tiles_kernel(const uint8_t* __restrict__ q4k, int M, int K, uint8_t* __restrict__ tiles,
                                    int Kt, int row0) {
  const int nkt = Kt / 128;
  const size_t n = (size_t)M * (Kt / 32);
  const size_t idx = (size_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (idx >= n) return;
  const int lane = (int)(idx & 63);
  const size_t rest = idx >> 6;
  const int j = (int)(rest & 3);
  const size_t rest2 = rest >> 2;
  const int kt = (int)(rest2 % nkt), band = (int)(rest2 / nkt);
  const int r = 64 * band + lane, g = 4 * kt + j;
  uint32_t w[4] = {0u, 0u, 0u, 0u};
  uint32_t sm = 0u;
  if (32 * g < K) {
    const uint8_t* b = q4k + ((size_t)r * (K / 256) + g / 8) * 144;
    const int jj = g % 8;
    const uint16_t dh = (uint16_t)(b[0] | (b[1] << 8)), mh = (uint16_t)(b[2] | (b[3] << 8));
    const float d = (float)__builtin_bit_cast(_Float16, dh), dmin = (float)__builtin_bit_cast(_Float16, mh);
    uint32_t sc, mn;
    if (jj < 4) {
      sc = b[4 + jj] & 0x3Fu;
      mn = b[8 + jj] & 0x3Fu;
    } else {
      sc = (b[12 + jj - 4] & 0x0Fu) | ((uint32_t)(b[4 + jj - 4] >> 6) << 4);
      mn = (uint32_t)(b[12 + jj - 4] >> 4) | ((uint32_t)(b[8 + jj - 4] >> 6) << 4);
    }
    sm = f32_to_bf16(__fmul_rn(d, (float)sc)) | (f32_to_bf16(__fmul_rn(-dmin, (float)mn)) << 16);
    const uint8_t* cb = b + 16 + 32 * (jj / 2);
    const int shift = (jj & 1) ? 4 : 0;
#pragma unroll 8
    for (int c = 0; c < 32; ++c) {
      const uint32_t code = ((uint32_t)cb[c] >> shift) & 15u;
      const int ni = tile_nibble_index(c);
      w[ni >> 3] |= code << (4 * (ni & 7));
    }
  }
  const int R = row0 + r;
  uint8_t* t = tiles + ((size_t)(R / 64) * nkt + kt) * kTileBytes;
  *reinterpret_cast<uint4*>(t + j * 1024 + (R % 64) * 16) = make_uint4(w[0], w[1], w[2], w[3]);
  *reinterpret_cast<uint32_t*>(t + kCodeBytes + (R % 64) * 16 + j * 4) = sm;
}

// ------------------------------------------------------------------ quantizer --
// Bit-exact restatement of quant/q4nx.py:127-200 per (row, group), in float64 where
// the reference uses float64.
__device__ __forceinline__ float bits_f(uint32_t u) { return __uint_as_float(u); }

__device__ __forceinline__ float bf16_floor_f32(float x) {
  const uint32_t u = __float_as_uint(x);
  const uint32_t bump = ((u >> 31) && (u & 0xffffu)) ? 1u : 0u;
  return bits_f(((u >> 16) + bump) << 16);
}

__device__ __forceinline__ float bf16_ceil_f64(double x) {
  float f = __double2float_rn(x);
  if ((double)f < x) f = nextafterf(f, __builtin_inff());
  const uint32_t u = __float_as_uint(f);
  const uint32_t bump = (!(u >> 31) && (u & 0xffffu)) ? 1u : 0u;
  return bits_f(((u >> 16) + bump) << 16);
}

__device__ __forceinline__ float bf16_next_up(float x) {
  uint32_t h = __float_as_uint(x) >> 16;
  if (h == 0x8000u) h = 0u;
  uint32_t nx;
  if (h == 0u) nx = 1u;
  else if (h & 0x8000u) nx = (h == 0x8001u) ? 0u : h - 1u;
  else nx = h + 1u;
  return bits_f(nx << 16);
}

// Quantize one (row, group) of 32 fp32 values and store it at (tile, j, lane).
__device__ void quantize_group(const float (&v)[32], uint8_t* tile, int j, int lane, int* err) {
  bool finite = true;
#pragma unroll
  for (int c = 0; c < 32; ++c) finite = finite && isfinite(v[c]);
  if (!finite) atomicOr(err, 1);
  float lo = v[0], hi = v[0];
#pragma unroll
  for (int c = 1; c < 32; ++c) {
    lo = fminf(lo, v[c]);
    hi = fmaxf(hi, v[c]);
  }
  const float minq = bf16_floor_f32(lo);
  const double min64 = (double)minq, hi64 = (double)hi;
  const double span = hi64 - min64;
  float sc = bf16_ceil_f64(span / 15.0);
  for (int it = 0; it < 64; ++it) {
    if (!isfinite(sc)) break;
    if (min64 + 15.0 * (double)sc >= hi64) break;
    sc = bf16_next_up(sc);
  }
  const bool flat = span == 0.0;
  if (flat) sc = 0.f;
  if (!isfinite(minq) || !isfinite(sc)) atomicOr(err, 2);
  const double div = flat ? 1.0 : (double)sc;
  uint32_t words[4] = {0u, 0u, 0u, 0u};
#pragma unroll
  for (int c = 0; c < 32; ++c) {
    double q = rint(((double)v[c] - min64) / div);
    q = q < 0.0 ? 0.0 : (q > 15.0 ? 15.0 : q);
    const uint32_t code = flat ? 0u : (uint32_t)q;
    const int ni = tile_nibble_index(c);
    words[ni >> 3] |= code << (4 * (ni & 7));
  }
  *reinterpret_cast<uint4*>(tile + j * 1024 + lane * 16) = make_uint4(words[0], words[1], words[2], words[3]);
  const uint32_t sb = __float_as_uint(sc) >> 16, mb = __float_as_uint(minq) >> 16;
  *reinterpret_cast<uint32_t*>(tile + kCodeBytes + lane * 16 + j * 4) = sb | (mb << 16);
}

// Thread = (tile, j, lane) -> (row, group), coalesced on the tile side.
struct GroupIndex {
  size_t tile;
  int j, lane, r, g;
};
__device__ __forceinline__ GroupIndex group_index(size_t idx, int nkt) {
  GroupIndex gi;
  gi.lane = idx & 63;
  const size_t rest = idx >> 6;
  gi.j = rest & 3;
  gi.tile = rest >> 2;
  const int rt = (int)(gi.tile / nkt), kt = (int)(gi.tile % nkt);
  gi.r = rt * 64 + gi.lane;
  gi.g = kt * 4 + gi.j;
  return gi;
}

__global__ void quantize_kernel(const float* __restrict__ w, int M, int K, int ld, int k_valid,
                                uint8_t* __restrict__ tiles, int* __restrict__ err) {
  const size_t idx = (size_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (idx >= (size_t)M * (K / 32)) return;
  const GroupIndex gi = group_index(idx, K / 128);
  const float* row = w + (size_t)gi.r * ld;
  float v[32];
#pragma unroll
  for (int c = 0; c < 32; ++c) {
    const int col = gi.g * 32 + c;
    v[c] = col < k_valid ? row[col] : 0.f;
  }
  quantize_group(v, tiles + gi.tile * kTileBytes, gi.j, gi.lane, err);
}

// Counter-based N(0, std) weights: splitmix64 of (seed, row*k_valid + col) -> Box-Muller.
__device__ __forceinline__ uint64_t splitmix64(uint64_t z) {
  z += 0x9E3779B97F4A7C15ull;
  z = (z ^ (z >> 30)) * 0xBF58476D1CE4E5B9ull;
  z = (z ^ (z >> 27)) * 0x94D049BB133111EBull;
  return z ^ (z >> 31);
}

__device__ __forceinline__ float synth_normal(uint64_t seed, uint64_t i) {
  const uint64_t h = splitmix64(seed * 0x100000001B3ull ^ splitmix64(i));
  const float u1 = ((uint32_t)(h >> 40) + 1u) * (1.0f / 16777217.0f);  // (0, 1)
  const float u2 = (uint32_t)(h & 0xFFFFFFu) * (1.0f / 16777216.0f);   // [0, 1)
  return sqrtf(-2.0f * logf(u1)) * cospif(2.0f * u2);
}

__global__ void synth_quantize_kernel(uint64_t seed, float std, int M, int K, int k_valid,
                                      uint8_t* __restrict__ tiles, int* __restrict__ err) {
  const size_t idx = (size_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (idx >= (size_t)M * (K / 32)) return;
  const GroupIndex gi = group_index(idx, K / 128);
  float v[32];
#pragma unroll
  for (int c = 0; c < 32; ++c) {
    const int col = gi.g * 32 + c;
    v[c] = col < k_valid ? std * synth_normal(seed, (uint64_t)gi.r * k_valid + col) : 0.f;
  }
  quantize_group(v, tiles + gi.tile * kTileBytes, gi.j, gi.lane, err);
}

}  // namespace

hipError_t launch_relayout_in(const uint8_t* packed, uint8_t* tiles, int M, int K, hipStream_t st) {
  const size_t n = (size_t)M * (K / 32);
  const unsigned blocks = (unsigned)((n + 255) / 256);
  hipLaunchKernelGGL(relayout_in_kernel, dim3(blocks), dim3(256), 0, st, packed, tiles, M, K);
  return hipGetLastError();
}

hipError_t launch_q4k_to_tiles(const uint8_t* q4k, int M, int K, uint8_t* tiles, int Kt, int row0, hipStream_t st) {
  if (M % 64 || row0 % 64 || K % 256 || Kt % 128 || K > Kt) return hipErrorInvalidValue;
  const size_t n = (size_t)M * (Kt / 32);
  const unsigned blocks = (unsigned)((n + 255) / 256);
  hipLaunchKernelGGL(q4k_to_tiles_kernel, dim3(blocks), dim3(256), 0, st, q4k, M, K, tiles, Kt, row0);
  return hipGetLastError();
}

hipError_t launch_relayout_out(const uint8_t* tiles, uint8_t* packed, int M, int K, hipStream_t st) {
  const size_t n = (size_t)(M / 2) * (K / 32);
  const unsigned blocks = (unsigned)((n + 255) / 256);
  hipLaunchKernelGGL(relayout_out_kernel, dim3(blocks), dim3(256), 0, st, tiles, packed, M, K);
  return hipGetLastError();
}

hipError_t launch_quantize(const float* w, int M, int K, int ld, int k_valid, uint8_t* tiles, int* err,
                           hipStream_t st) {
  const size_t n = (size_t)M * (K / 32);
  const unsigned blocks = (unsigned)((n + 255) / 256);
  hipLaunchKernelGGL(quantize_kernel, dim3(blocks), dim3(256), 0, st, w, M, K, ld, k_valid, tiles, err);
  return hipGetLastError();
}

hipError_t launch_synth_quantize(uint64_t seed, float std, int M, int K, int k_valid, uint8_t* tiles, int* err,
                                 hipStream_t st) {
  const size_t n = (size_t)M * (K / 32);
  const unsigned blocks = (unsigned)((n + 255) / 256);
  hipLaunchKernelGGL(synth_quantize_kernel, dim3(blocks), dim3(256), 0, st, seed, std, M, K, k_valid, tiles, err);
  return hipGetLastError();
}

}  // namespace rmoe
