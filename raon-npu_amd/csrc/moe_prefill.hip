// Prefill (many-token) MoE on bf16 MFMA: router GEMM + top-k, tile table over the
// dispatch, grouped q4nx GEMMs (gate/up with the activation fused, down), ordered
// combine.  Restates NpuBackend.moe_experts_grouped (npu/backend.py:4845-4979) and the
// planner's scatter/combine (kernels/moe_grouped/planner.py:184-322) on the device.
//
// q4nx on MFMA without rounding the weights:  w = min + scale*n  (n = 4-bit code).
// For one 32-column group g and a tile of tokens m and weight rows r:
//   sum_k x[m,k] w[r,k] = 16*scale[r]*C'[m,r] + (min[r] - 16*scale[r]) * S[m]
// where C' = sum_k x[m,k]*(1 + n[r,k]/16) is one v_mfma_f32_16x16x32_bf16 with the
// codes as exact bf16 values (1 + n/16) and S[m] = sum_k x[m,k].  The first term is
// added per group with one fp32 FMA per output (scales differ per row and group); the
// second is a small GEMM over the groups, done on MFMA with S and the coefficient
// split into bf16 hi + lo parts (relative error ~2^-16).
#include "rmoe_internal.h"

namespace rmoe {
namespace {

typedef __bf16 bf16x8_t __attribute__((ext_vector_type(8)));
typedef float f32x4_t __attribute__((ext_vector_type(4)));

__device__ __forceinline__ f32x4_t mfma16(const uint4 a, const uint4 b, f32x4_t c) {
  return __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(bf16x8_t, a), __builtin_bit_cast(bf16x8_t, b), c,
                                                 0, 0, 0);
}

// Exact 3-way bf16 split of an fp32 value: v = hi + mid + lo (8 + 8 + 8 significant
// bits cover the 24 of fp32), each part the RNE bf16 of the remainder.
__device__ __forceinline__ void split3_bf16(float v, uint32_t& hi, uint32_t& mid, uint32_t& lo) {
  hi = f32_to_bf16(v);
  const float r = v - bf16_to_f32(hi);
  mid = f32_to_bf16(r);
  lo = f32_to_bf16(r - bf16_to_f32(mid));
}
// Group sums are stored as two dwords per (row, group): (hi | mid << 16), lo.
__device__ __forceinline__ void store_split3(uint32_t* dst, float v) {
  uint32_t hi, mid, lo;
  split3_bf16(v, hi, mid, lo);
  dst[0] = hi | (mid << 16);
  dst[1] = lo;
}

// ---------------------------------------------------------------- router GEMM --
// logits[T, E] = x[T, H] . Wr[E, H]^T on MFMA (exact bf16 products, fp32 sums).
// Block: 4 waves x 64 tokens; a 64-column chunk of Wr for all experts is staged in LDS
// and shared by the 4 waves; A fragments come straight from the token rows.
constexpr int kMaxEFrags = 16;  // E <= 256
constexpr int kRouterChunk = 64;
constexpr int kRouterStride = kRouterChunk + 8;  // bf16 per LDS row (16-byte pad)

template <int NFR>
__global__ __launch_bounds__(256) void router_gemm_kernel(const uint16_t* __restrict__ x, int T, int H,
                                                          const uint16_t* __restrict__ w, int E,
                                                          float* __restrict__ logits) {
  __shared__ __attribute__((aligned(16))) uint16_t ws[256 * kRouterStride];
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int l16 = lane & 15, lq = lane >> 4;
  const int t0 = blockIdx.x * 256 + wave * 64;
  f32x4_t acc[4][NFR];
#pragma unroll
  for (int m = 0; m < 4; ++m)
#pragma unroll
    for (int f = 0; f < NFR; ++f) acc[m][f] = f32x4_t{0.f, 0.f, 0.f, 0.f};
  const uint16_t* xr[4];
#pragma unroll
  for (int m = 0; m < 4; ++m) xr[m] = x + (size_t)min(t0 + 16 * m + l16, T - 1) * H + 8 * lq;
  for (int k0 = 0; k0 < H; k0 += kRouterChunk) {
    __syncthreads();
    for (int i = tid; i < E * (kRouterChunk / 8); i += 256) {
      const int e = i / (kRouterChunk / 8), c = i % (kRouterChunk / 8);
      *reinterpret_cast<uint4*>(&ws[e * kRouterStride + 8 * c]) =
          *reinterpret_cast<const uint4*>(w + (size_t)e * H + k0 + 8 * c);
    }
    __syncthreads();
#pragma unroll
    for (int kk = 0; kk < kRouterChunk; kk += 32) {
      uint4 a[4];
#pragma unroll
      for (int m = 0; m < 4; ++m) a[m] = *reinterpret_cast<const uint4*>(xr[m] + k0 + kk);
#pragma unroll
      for (int f = 0; f < NFR; ++f) {
        const uint4 b = *reinterpret_cast<const uint4*>(&ws[(16 * f + l16) * kRouterStride + kk + 8 * lq]);
#pragma unroll
        for (int m = 0; m < 4; ++m) acc[m][f] = mfma16(a[m], b, acc[m][f]);
      }
    }
  }
#pragma unroll
  for (int m = 0; m < 4; ++m)
#pragma unroll
    for (int f = 0; f < NFR; ++f) {
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const int t = t0 + 16 * m + 4 * lq + i;
        if (t < T) logits[(size_t)t * E + 16 * f + l16] = acc[m][f][i];
      }
    }
}

// numpy float32 sum order (pairwise_sum, n <= 128 per block of 8 partial sums).
__device__ float np_sum_f32_lds(const float* v, int n) {
  if (n < 8) {
    float r = 0.f;
    for (int i = 0; i < n; ++i) r = __fadd_rn(r, v[i]);
    return r;
  }
  float r[8];
  for (int j = 0; j < 8; ++j) r[j] = v[j];
  int i = 8;
  for (; i + 8 <= n; i += 8)
    for (int j = 0; j < 8; ++j) r[j] = __fadd_rn(r[j], v[i + j]);
  float res = __fadd_rn(__fadd_rn(__fadd_rn(r[0], r[1]), __fadd_rn(r[2], r[3])),
                        __fadd_rn(__fadd_rn(r[4], r[5]), __fadd_rn(r[6], r[7])));
  for (; i < n; ++i) res = __fadd_rn(res, v[i]);
  return res;
}

// One wave per token: scores, selection (score + bias, ties to the lower id), renorm.
__global__ __launch_bounds__(256) void topk_kernel(const float* __restrict__ logits, int T, int E, int k, int score,
                                                   const float* __restrict__ bias, int renorm, float scaling,
                                                   int32_t* __restrict__ ids, float* __restrict__ wts) {
  __shared__ float sc[4][256];
  __shared__ float ch[4][16];
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int t = blockIdx.x * 4 + wave;
  if (t >= T) return;
  const float* lg = logits + (size_t)t * E;
  float* s = sc[wave];
  if (score == 0) {
    for (int e = lane; e < E; e += 64) s[e] = 1.0f / (1.0f + expf(-lg[e]));
  } else {
    float m = -__builtin_inff();
    for (int e = lane; e < E; e += 64) m = fmaxf(m, lg[e]);
#pragma unroll
    for (int off = 32; off > 0; off >>= 1) m = fmaxf(m, __shfl_xor(m, off, 64));
    for (int e = lane; e < E; e += 64) s[e] = expf(lg[e] - m);
    __builtin_amdgcn_wave_barrier();
    __builtin_amdgcn_fence(__ATOMIC_SEQ_CST, "wavefront");
    float total = 0.f;
    if (lane == 0) total = np_sum_f32_lds(s, E);
    total = __shfl(total, 0, 64);
    __builtin_amdgcn_wave_barrier();
    for (int e = lane; e < E; e += 64) s[e] = s[e] / total;
  }
  __builtin_amdgcn_wave_barrier();
  __builtin_amdgcn_fence(__ATOMIC_SEQ_CST, "wavefront");
  // Candidates of this lane: e = lane + 64*i; taken flags in a lane mask.
  uint32_t taken = 0u;
  int chosen_id = 0;
  for (int r = 0; r < k; ++r) {
    float best = 0.f;
    int bid = 0x7fffffff;
    for (int i = 0; i < 4; ++i) {
      const int e = lane + 64 * i;
      if (e < E && !((taken >> i) & 1u)) {
        const float c = bias ? __fadd_rn(s[e], bias[e]) : s[e];
        if (bid == 0x7fffffff || c > best) {
          best = c;
          bid = e;
        }
      }
    }
#pragma unroll
    for (int off = 32; off > 0; off >>= 1) {
      const float ob = __shfl_xor(best, off, 64);
      const int oi = __shfl_xor(bid, off, 64);
      if (oi != 0x7fffffff && (bid == 0x7fffffff || ob > best || (ob == best && oi < bid))) {
        best = ob;
        bid = oi;
      }
    }
    if ((bid & 63) == lane) taken |= 1u << (bid >> 6);
    if (lane == r) chosen_id = bid;
    if (lane == 0) ch[wave][r] = s[bid];
  }
  __builtin_amdgcn_wave_barrier();
  __builtin_amdgcn_fence(__ATOMIC_SEQ_CST, "wavefront");
  float denom = 1.f;
  if (lane == 0 && renorm) denom = __fadd_rn(np_sum_f32_lds(ch[wave], k), 1e-20f);
  denom = __shfl(denom, 0, 64);
  if (lane < k) {
    float v = renorm ? ch[wave][lane] / denom : ch[wave][lane];
    ids[(size_t)t * k + lane] = chosen_id;
    wts[(size_t)t * k + lane] = __fmul_rn(v, scaling);
  }
}

// ------------------------------------------------------------ row group sums --
// S[row, g] = sum of the 32 bf16 values of group g of row `row`, stored as an exact
// 3-way bf16 split in dwords dst32[(row*G + g)*2 + {0,1}].  Thread per (row, group).
__global__ void group_sums_kernel(const uint16_t* __restrict__ src, int rows, int K, uint32_t* __restrict__ dst) {
  const int G = K / 32;
  const size_t idx = (size_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (idx >= (size_t)rows * G) return;
  const uint32_t* p = reinterpret_cast<const uint32_t*>(src + idx * 32);
  float s = 0.f;
#pragma unroll
  for (int c = 0; c < 16; ++c) {
    const uint32_t v = p[c];
    s += bf16_to_f32(v & 0xffffu);
    s += bf16_to_f32(v >> 16);
  }
  store_split3(dst + idx * 2, s);
}

// ----------------------------------------------------------------- tile table --
// tiles[i] = expert | (row_start << 9) for the m-tiles of every group; group e covers
// sorted rows [offsets[e], offsets[e+1]); the extra group n_routed (shared expert)
// covers rows [offsets[n_routed], offsets[n_routed] + shared_rows).  tiles[-1]... the
// count is written to *ntiles.
constexpr int kBM = 128;

// One workgroup of 512 threads; thread e owns group e (routed 0..n_routed-1, shared n_routed).
__global__ __launch_bounds__(512) void tile_table_kernel(const int32_t* __restrict__ offsets, int n_routed,
                                                         int shared_rows, uint32_t* __restrict__ tiles,
                                                         int* __restrict__ ntiles, int cap) {
  __shared__ int base[513];
  const int e = threadIdx.x;
  const int ng = n_routed + (shared_rows > 0 ? 1 : 0);
  int b = 0, end = 0, nt = 0;
  if (e < ng) {
    b = offsets[min(e, n_routed)];
    end = e < n_routed ? offsets[e + 1] : b + shared_rows;
    nt = (end - b + kBM - 1) / kBM;
  }
  base[e + 1] = nt;
  if (e == 0) base[0] = 0;
  __syncthreads();
  if (e == 0)
    for (int q = 1; q <= ng; ++q) base[q] += base[q - 1];
  __syncthreads();
  for (int i = 0; i < nt; ++i) {
    const int slot = base[e] + i;
    if (slot < cap) tiles[slot] = (uint32_t)e | ((uint32_t)(b + i * kBM) << 9);
  }
  if (e == 0) *ntiles = min(base[ng], cap);
}

// ------------------------------------------------------------- grouped GEMM --
struct GemmArgs {
  // weights: expert e at wbase + e*wstride, q4nx tiles of an [N_total, K] matrix
  const uint8_t* wbase;
  size_t wstride;
  int K;             // input width (multiple of 128)
  int N_total;       // weight rows (gate/up: 2I; down: H)
  int inter;         // gate/up: I (the up rows start at I)
  int mode;          // 0: gate/up + activation -> h; 1: down -> D
  int n_tiles;       // WG N-tiles (gate/up: ceil(I/128) units of 128; down: N_total/256 rows of 256)
  // activation rows
  const uint16_t* src;      // mode 0: x [T, K] gathered by token; mode 1: h [rows, K] in sorted order
  const int32_t* order;     // mode 0: sorted position -> assignment (token*k + route)
  int k_routes;
  int n_routed;             // group id n_routed = shared expert (rows identity tokens / sorted)
  int shared_base;          // sorted row index of the first shared row
  const uint32_t* ssum;     // row group sums, 2 dwords each: mode 0 [T, K/32] by token; mode 1 [rows, K/32] by row
  const uint32_t* tiles;
  const int* ntiles;
  const int32_t* offsets;   // group row ends: offsets[e+1] (routed); shared end = shared_base + shared_rows
  int shared_rows;
  // outputs
  uint16_t* out;            // mode 0: h [rows, out_ld]; mode 1: D [rows, out_ld]
  int out_ld;
  uint32_t* out_ssum;       // mode 0: group sums of h rows [rows, out_ld/32], 2 dwords each
  int act;
  float gb, vb;
};

__device__ __forceinline__ int group_end(const GemmArgs& a, int e) {
  return e < a.n_routed ? a.offsets[e + 1] : a.shared_base + a.shared_rows;
}

// Source row of sorted row p.
__device__ __forceinline__ const uint16_t* src_row(const GemmArgs& a, int e, int p) {
  if (a.mode == 1) return a.src + (size_t)p * a.K;
  const int tok = e < a.n_routed ? a.order[p] / a.k_routes : p - a.shared_base;
  return a.src + (size_t)tok * a.K;
}
__device__ __forceinline__ const uint32_t* ssum_row(const GemmArgs& a, int e, int p) {
  const int G = a.K / 32;
  if (a.mode == 1) return a.ssum + (size_t)p * G * 2;
  const int tok = e < a.n_routed ? a.order[p] / a.k_routes : p - a.shared_base;
  return a.ssum + (size_t)tok * G * 2;
}

// LDS ring of the grouped GEMM: per K step (128 columns) the workgroup's 128 activation
// rows (256 B each, 16-byte chunks XOR-swizzled by row) and its four 64-row weight
// tiles (copied verbatim), three steps deep.
constexpr int kStages = 3;
constexpr int kXBytes = kBM * 256;
constexpr int kWBytes = 4 * kTileBytes;
constexpr int kStageBytes = kXBytes + kWBytes;
constexpr int kGemmLds = kStages * kStageBytes;  // 159,744 of the 163,840 bytes of a CU
constexpr int kOutStride = 136;                  // bf16 per row of the epilogue staging tile

// 16 bytes per lane from global memory straight into LDS: lane L writes lds + 16 L.
// Written as inline assembly so that the compiler does not treat every later LDS read
// as dependent on it (it would wait for all outstanding loads before each one); the
// ring's own waits (ring_wait) order the copies.  M0 is saved and restored.
__device__ __forceinline__ void dma16(const void* g, uint32_t lds) {
  uint32_t saved;
  asm volatile(
      "s_mov_b32 %0, m0\n\t"
      "s_mov_b32 m0, %2\n\t"
      "global_load_lds_dwordx4 %1, off\n\t"
      "s_mov_b32 m0, %0"
      : "=&s"(saved)
      : "v"(g), "s"(__builtin_amdgcn_readfirstlane(lds))
      : "memory");
}
// Wait until at most `pending` of this wave's copies are in flight, then meet the
// workgroup.  The count is an immediate, so each value is a branch of its own.
__device__ __forceinline__ void ring_wait(int pending) {
  switch (pending) {
    case 7: asm volatile("s_waitcnt vmcnt(7) lgkmcnt(0)" ::: "memory"); break;
    case 6: asm volatile("s_waitcnt vmcnt(6) lgkmcnt(0)" ::: "memory"); break;
    default: asm volatile("s_waitcnt vmcnt(0) lgkmcnt(0)" ::: "memory"); break;
  }
  asm volatile("s_barrier" ::: "memory");
}

// Grid: n_tiles * tile_cap workgroups (rounded to a multiple of 8), 512 threads (8 waves).
// A workgroup multiplies 128 sorted rows by 256 weight rows; wave w takes rows
// 64*(w&1)..+63 and a quarter of the weight rows (w>>1), as 4 x 4 MFMA fragments.
//   gate/up: the workgroup takes intermediate units 128*nt..+127 (gate rows and the
//            matching up rows); the wave's quarter is units 32*(w>>1)..+31, fragments
//            0,1 = gate, 2,3 = up, so the activation and the 32-column group sums of h
//            stay inside the wave.
//   down:    the workgroup takes output rows 256*nt..+255, the wave 64*(w>>1)..+63.
// K loop: a three-deep LDS ring filled by global->LDS copies; per K step one
// barrier, then the copy for step kt+2 into the slot step kt-1 used.
__global__ __launch_bounds__(512) __attribute__((amdgpu_waves_per_eu(2, 2))) void grouped_gemm_kernel(GemmArgs a, int tile_cap) {
  __shared__ __attribute__((aligned(16))) uint8_t lds[kGemmLds];
  // XCD-aware order: workgroups are dealt round-robin to the 8 XCDs; make each XCD
  // take a contiguous range of (n-tile, m-tile) so m-tiles sharing a weight tile meet
  // in the same L2.
  const int nb = gridDim.x, per = nb / 8;
  const int lid = (blockIdx.x % 8) * per + blockIdx.x / 8;
  // m-tile major: the n-tiles of one m-tile (sharing the gathered rows) and consecutive
  // m-tiles of one expert (sharing its weights) run back to back on one XCD.
  const int mt = lid / a.n_tiles, nt = lid % a.n_tiles;
  if (nt >= a.n_tiles || mt >= *a.ntiles) return;
  const uint32_t te = a.tiles[mt];
  const int e = (int)(te & 511u), row0 = (int)(te >> 9);
  const int rend = group_end(a, e);
  const int nrows = min(kBM, rend - row0);
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int l16 = lane & 15, lq = lane >> 4;
  const int wm = wave & 1, wn = wave >> 1;
  const int nkt = a.K / kTileCols;
  const uint8_t* W = a.wbase + (size_t)e * a.wstride;
  const uint32_t lds0 = (uint32_t)(uintptr_t)lds;

  // The workgroup's four 64-row weight bands.  Gate/up: gate bands 2nt, 2nt+1, up bands
  // I/64 + 2nt, +1; a band past I (last n-tile when I % 128 != 0) reads band 0 instead
  // and its results are not stored.
  int band[4];
#pragma unroll
  for (int t = 0; t < 4; ++t) {
    if (a.mode == 0) {
      const int gb_ = 2 * nt + (t & 1);
      band[t] = 64 * gb_ < a.inter ? (t < 2 ? gb_ : a.inter / 64 + gb_) : 0;
    } else {
      band[t] = 4 * nt + t;
    }
  }
  // Fragment f of this wave: weight tile ft[f] (0..3) and first row fr[f] inside it.
  int ft[4], fr[4];
#pragma unroll
  for (int f = 0; f < 4; ++f) {
    if (a.mode == 0) {
      ft[f] = (f < 2 ? 0 : 2) + (wn >> 1);
      fr[f] = 32 * (wn & 1) + 16 * (f & 1);
    } else {
      ft[f] = wn;
      fr[f] = 16 * f;
    }
  }
  const bool active = a.mode == 1 || 128 * nt + 32 * wn < a.inter;

  // Copy descriptors.  Activations: copy q = wave + 8i (i < 4) fills LDS rows 4q..4q+3;
  // lane L brings row 4q + L/16, chunk (L%16) ^ (row%16).  Rows past the tile read the
  // tile's first row (their results are not stored).
  const uint8_t* xg[4];
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const int q = wave + 8 * i, r = 4 * q + (lane >> 4);
    const int c = (lane & 15) ^ (r & 15);
    xg[i] = reinterpret_cast<const uint8_t*>(src_row(a, e, row0 + (r < nrows ? r : 0))) + 16 * c;
  }
  // Weights: copy v = wave + 8i (i < 3, v < 20) is 1 KB piece v%5 of tile v/5.
  const int n_wcopy = wave < 4 ? 3 : 2;
  const uint8_t* wg[3];
#pragma unroll
  for (int i = 0; i < 3; ++i) {
    const int v = min(wave + 8 * i, 19), t = v / 5, p = v % 5;
    wg[i] = W + (size_t)band[t] * nkt * kTileBytes + 1024 * p + 16 * lane;
  }
  auto issue = [&](int kt) {
    const uint32_t sb = lds0 + (uint32_t)((kt % kStages) * kStageBytes);
#pragma unroll
    for (int i = 0; i < 4; ++i) dma16(xg[i] + (size_t)kt * 256, sb + 1024u * (uint32_t)(wave + 8 * i));
#pragma unroll
    for (int i = 0; i < 3; ++i) {
      if (i < n_wcopy) {
        const int v = wave + 8 * i, t = v / 5, p = v % 5;
        dma16(wg[i] + (size_t)kt * kTileBytes, sb + (uint32_t)(kXBytes + t * kTileBytes + 1024 * p));
      }
    }
  };
  const int per_stage = 4 + n_wcopy;

  issue(0);
  if (nkt > 1) issue(1);

  // Correction first, while the first copies are in flight:
  //   acc = sum_g (min - 16*scale)[r, g] * S[m, g]
  // over blocks of 32 groups, both factors split exactly into 3 bf16 parts; the 6
  // leading products are kept.
  f32x4_t acc[4][4];
#pragma unroll
  for (int m = 0; m < 4; ++m)
#pragma unroll
    for (int f = 0; f < 4; ++f) acc[m][f] = f32x4_t{0.f, 0.f, 0.f, 0.f};
  const int G = a.K / 32;
  const uint32_t* srow[4];
#pragma unroll
  for (int m = 0; m < 4; ++m) {
    const int r = 64 * wm + 16 * m + l16;
    srow[m] = r < nrows ? ssum_row(a, e, row0 + r) : nullptr;
  }
  for (int g0 = 0; g0 < G; g0 += 32) {
    const int gl = g0 + 8 * lq;  // the lane's first group; groups gl..gl+7
    uint4 bc[4][3];
#pragma unroll
    for (int f = 0; f < 4; ++f) {
      uint4 smw[2];
#pragma unroll
      for (int h = 0; h < 2; ++h) {
        const int kt = gl / 4 + h;
        smw[h] = 4 * kt < G ? *reinterpret_cast<const uint4*>(W + ((size_t)band[ft[f]] * nkt + kt) * kTileBytes + kCodeBytes +
                                                              (fr[f] + l16) * 16)
                            : make_uint4(0u, 0u, 0u, 0u);
      }
      const uint32_t sv[8] = {smw[0].x, smw[0].y, smw[0].z, smw[0].w, smw[1].x, smw[1].y, smw[1].z, smw[1].w};
      uint32_t hv[8], mv[8], lv[8];
#pragma unroll
      for (int i = 0; i < 8; ++i) {
        const float coef = bf16_to_f32(sv[i] >> 16) - 16.f * bf16_to_f32(sv[i] & 0xffffu);
        split3_bf16(coef, hv[i], mv[i], lv[i]);
      }
      bc[f][0] = make_uint4(hv[0] | (hv[1] << 16), hv[2] | (hv[3] << 16), hv[4] | (hv[5] << 16), hv[6] | (hv[7] << 16));
      bc[f][1] = make_uint4(mv[0] | (mv[1] << 16), mv[2] | (mv[3] << 16), mv[4] | (mv[5] << 16), mv[6] | (mv[7] << 16));
      bc[f][2] = make_uint4(lv[0] | (lv[1] << 16), lv[2] | (lv[3] << 16), lv[4] | (lv[5] << 16), lv[6] | (lv[7] << 16));
    }
#pragma unroll
    for (int m = 0; m < 4; ++m) {
      // 8 groups x (hi|mid, lo) = 16 dwords; pairs of groups past G read as zero.
      uint4 sv[4];
#pragma unroll
      for (int h = 0; h < 4; ++h)
        sv[h] = srow[m] && gl + 2 * h < G ? *reinterpret_cast<const uint4*>(srow[m] + 2 * (gl + 2 * h))
                                          : make_uint4(0u, 0u, 0u, 0u);
      uint4 ah, am, al;
      ah.x = __builtin_amdgcn_perm(sv[0].z, sv[0].x, 0x05040100u);
      ah.y = __builtin_amdgcn_perm(sv[1].z, sv[1].x, 0x05040100u);
      ah.z = __builtin_amdgcn_perm(sv[2].z, sv[2].x, 0x05040100u);
      ah.w = __builtin_amdgcn_perm(sv[3].z, sv[3].x, 0x05040100u);
      am.x = __builtin_amdgcn_perm(sv[0].z, sv[0].x, 0x07060302u);
      am.y = __builtin_amdgcn_perm(sv[1].z, sv[1].x, 0x07060302u);
      am.z = __builtin_amdgcn_perm(sv[2].z, sv[2].x, 0x07060302u);
      am.w = __builtin_amdgcn_perm(sv[3].z, sv[3].x, 0x07060302u);
      al.x = __builtin_amdgcn_perm(sv[0].w, sv[0].y, 0x05040100u);
      al.y = __builtin_amdgcn_perm(sv[1].w, sv[1].y, 0x05040100u);
      al.z = __builtin_amdgcn_perm(sv[2].w, sv[2].y, 0x05040100u);
      al.w = __builtin_amdgcn_perm(sv[3].w, sv[3].y, 0x05040100u);
#pragma unroll
      for (int f = 0; f < 4; ++f) {
        f32x4_t c = acc[m][f];
        c = mfma16(al, bc[f][0], c);
        c = mfma16(am, bc[f][1], c);
        c = mfma16(ah, bc[f][2], c);
        c = mfma16(am, bc[f][0], c);
        c = mfma16(ah, bc[f][1], c);
        c = mfma16(ah, bc[f][0], c);
        acc[m][f] = c;
      }
    }
  }

  // Main K loop:  acc += 16*scale[r, g] * sum_k x[m,k] (1 + n[r,k]/16)  per group g.
  for (int kt = 0; kt < nkt; ++kt) {
    ring_wait(kt + 1 < nkt ? per_stage : 0);
    if (kt + 2 < nkt) issue(kt + 2);
    const uint8_t* xs = lds + (kt % kStages) * kStageBytes;
    const uint8_t* ws = xs + kXBytes;
    float s16[4][4];
#pragma unroll
    for (int f = 0; f < 4; ++f) {
      const uint4 smv = *reinterpret_cast<const uint4*>(ws + ft[f] * kTileBytes + kCodeBytes + (fr[f] + l16) * 16);
      s16[f][0] = 16.f * bf16_to_f32(smv.x & 0xffffu);
      s16[f][1] = 16.f * bf16_to_f32(smv.y & 0xffffu);
      s16[f][2] = 16.f * bf16_to_f32(smv.z & 0xffffu);
      s16[f][3] = 16.f * bf16_to_f32(smv.w & 0xffffu);
    }
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      uint4 b[4], av[4];
#pragma unroll
      for (int f = 0; f < 4; ++f) {
        const uint32_t code =
            *reinterpret_cast<const uint32_t*>(ws + ft[f] * kTileBytes + j * 1024 + (fr[f] + l16) * 16 + 4 * lq);
        unpack_codes(code, b[f].x, b[f].y, b[f].z, b[f].w);
      }
#pragma unroll
      for (int m = 0; m < 4; ++m) {
        const int r = 64 * wm + 16 * m + l16;
        av[m] = *reinterpret_cast<const uint4*>(xs + r * 256 + 16 * ((4 * j + lq) ^ (r & 15)));
      }
#pragma unroll
      for (int m = 0; m < 4; ++m)
#pragma unroll
        for (int f = 0; f < 4; ++f) {
          const f32x4_t c = mfma16(av[m], b[f], f32x4_t{0.f, 0.f, 0.f, 0.f});
#pragma unroll
          for (int i = 0; i < 4; ++i) acc[m][f][i] = fmaf(s16[f][j], c[i], acc[m][f][i]);
        }
    }
  }
  // Every wave is past its last ring read: slots 0 and 1 become the output staging.
  asm volatile("s_waitcnt vmcnt(0) lgkmcnt(0)\n\ts_barrier" ::: "memory");

  // Epilogue.  C layout: lane holds rows 16m + 4*lq + i (of the wave's 64), column l16
  // of the fragment.  Results go through LDS so that global stores are 16-byte rows.
  uint16_t* stage0 = reinterpret_cast<uint16_t*>(lds);
  if (a.mode == 0) {
#pragma unroll
    for (int m = 0; m < 4; ++m) {
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const int r = 64 * wm + 16 * m + 4 * lq + i;
        float hv = 0.f;
#pragma unroll
        for (int f = 0; f < 2; ++f) {
          const float g = bf16_round(acc[m][f][i]), u = bf16_round(acc[m][2 + f][i]);
          const uint32_t h = f32_to_bf16(act_apply(a.act, g, u, a.gb, a.vb));
          stage0[r * kOutStride + 32 * wn + 16 * f + l16] = (uint16_t)h;
          hv += bf16_to_f32(h);
        }
        // The wave's 32 units are one group of h: reduce over the 16 lanes of l16.
#pragma unroll
        for (int off = 8; off > 0; off >>= 1) hv += __shfl_xor(hv, off, 16);
        if (l16 == 0 && active && r < nrows)
          store_split3(a.out_ssum + ((size_t)(row0 + r) * (a.out_ld / 32) + 4 * nt + wn) * 2, hv);
      }
    }
    __syncthreads();
    // 128 rows x 16 chunks of 8 units.
#pragma unroll
    for (int q = 0; q < 4; ++q) {
      const int cid = tid + 512 * q, r = cid >> 4, c = cid & 15;
      if (r < nrows && 128 * nt + 8 * c < a.inter)
        *reinterpret_cast<uint4*>(a.out + (size_t)(row0 + r) * a.out_ld + 128 * nt + 8 * c) =
            *reinterpret_cast<const uint4*>(stage0 + r * kOutStride + 8 * c);
    }
  } else {
    // Columns 0..127 of the 256 in slot 0, 128..255 in slot 1.
#pragma unroll
    for (int m = 0; m < 4; ++m)
#pragma unroll
      for (int f = 0; f < 4; ++f)
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          const int r = 64 * wm + 16 * m + 4 * lq + i;
          uint16_t* st = stage0 + (wn >> 1) * (kStageBytes / 2);
          st[r * kOutStride + 64 * (wn & 1) + 16 * f + l16] = (uint16_t)f32_to_bf16(acc[m][f][i]);
        }
    __syncthreads();
#pragma unroll
    for (int q = 0; q < 8; ++q) {
      const int cid = tid + 512 * q, r = cid >> 5, c = cid & 31;
      const uint16_t* st = stage0 + (c >> 4) * (kStageBytes / 2);
      if (r < nrows)
        *reinterpret_cast<uint4*>(a.out + (size_t)(row0 + r) * a.out_ld + 256 * nt + 8 * c) =
            *reinterpret_cast<const uint4*>(st + r * kOutStride + 8 * (c & 15));
    }
  }
}

// ---------------------------------------------------------------- combine --
// out[t] = RTNE(RTNE(sum_{routes by ascending expert} f32(D[inv[t,r]]) * w[t,r]) + D_shared[t])
// (+ x[t] with residual); optionally also the routed and shared rows separately.
__global__ __launch_bounds__(256) void combine_kernel(const uint16_t* __restrict__ D, int H, const int32_t* __restrict__ ids,
                                                      const float* __restrict__ wts, const int32_t* __restrict__ inv,
                                                      int k, int shared_base, const uint16_t* __restrict__ x,
                                                      uint16_t* __restrict__ out, uint16_t* __restrict__ routed,
                                                      uint16_t* __restrict__ shared_out, int has_shared) {
  const int t = blockIdx.x;
  __shared__ int ord[16];
  if (threadIdx.x == 0) {
    int prev = -1;
    for (int r = 0; r < k; ++r) {
      int best = 0x7fffffff, bs = 0;
      for (int q = 0; q < k; ++q) {
        const int eq = ids[(size_t)t * k + q];
        if (eq > prev && eq < best) {
          best = eq;
          bs = q;
        }
      }
      prev = best;
      ord[r] = bs;
    }
  }
  __syncthreads();
  for (int c = threadIdx.x; c < H; c += blockDim.x) {
    float acc = 0.f;
    for (int r = 0; r < k; ++r) {
      const int q = ord[r];
      const int pos = inv[(size_t)t * k + q];
      acc = __fadd_rn(acc, __fmul_rn(bf16_to_f32(D[(size_t)pos * H + c]), wts[(size_t)t * k + q]));
    }
    uint32_t o = f32_to_bf16(acc);
    if (routed) routed[(size_t)t * H + c] = (uint16_t)o;
    if (has_shared) {
      const uint16_t sd = D[(size_t)(shared_base + t) * H + c];
      if (shared_out) shared_out[(size_t)t * H + c] = sd;
      o = f32_to_bf16(__fadd_rn(bf16_to_f32(o), bf16_to_f32(sd)));
    }
    if (x) o = f32_to_bf16(__fadd_rn(bf16_to_f32(x[(size_t)t * H + c]), bf16_to_f32(o)));
    if (out) out[(size_t)t * H + c] = (uint16_t)o;
  }
}

// Zero h[:, I:Ipad] and the group sums of those columns (thread per row).
__global__ void zero_pad_cols_kernel(uint16_t* __restrict__ h, uint32_t* __restrict__ hsum, int rows, int I, int Ipad) {
  const int r = blockIdx.x * blockDim.x + threadIdx.x;
  if (r >= rows) return;
  for (int c = I; c < Ipad; ++c) h[(size_t)r * Ipad + c] = 0;
  // Groups entirely past I; a group straddling I gets its sum from the GEMM epilogue
  // only when I is a multiple of 32 (guaranteed: I % 64 == 0).
  for (int g = I / 32; g < Ipad / 32; ++g) {
    hsum[((size_t)r * (Ipad / 32) + g) * 2] = 0u;
    hsum[((size_t)r * (Ipad / 32) + g) * 2 + 1] = 0u;
  }
}

// h[shared_base + t] = RTNE(act(shared_gu[t])) (padded to Ipad) and its group sums.
__global__ void shared_act_kernel(const uint16_t* __restrict__ gu, int T, int I, int Ipad, int act, float gb, float vb,
                                  uint16_t* __restrict__ h, uint32_t* __restrict__ hsum) {
  const int G = Ipad / 32;
  const size_t idx = (size_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (idx >= (size_t)T * G) return;
  const int t = (int)(idx / G), g = (int)(idx % G);
  float s = 0.f;
  for (int c = 0; c < 32; ++c) {
    const int col = 32 * g + c;
    uint16_t v = 0;
    if (col < I) {
      const float gg = bf16_to_f32(gu[(size_t)t * 2 * I + col]);
      const float uu = bf16_to_f32(gu[(size_t)t * 2 * I + I + col]);
      v = (uint16_t)f32_to_bf16(act_apply(act, gg, uu, gb, vb));
    }
    h[(size_t)t * Ipad + col] = v;
    s += bf16_to_f32(v);
  }
  store_split3(hsum + ((size_t)t * G + g) * 2, s);
}

}  // namespace

// ------------------------------------------------------------------ launchers --
hipError_t launch_router_gemm(const uint16_t* x, int T, int H, const uint16_t* w, int E, float* logits, hipStream_t st) {
  if (E % 16 || E > 16 * kMaxEFrags || H % 32) return hipErrorInvalidValue;
  if (H % kRouterChunk) return hipErrorInvalidValue;
  const dim3 grid((T + 255) / 256), block(256);
  switch (E / 16) {
#define RMOE_ROUTER_CASE(n) \
  case n:                   \
    hipLaunchKernelGGL(router_gemm_kernel<n>, grid, block, 0, st, x, T, H, w, E, logits); \
    break;
    RMOE_ROUTER_CASE(1) RMOE_ROUTER_CASE(2) RMOE_ROUTER_CASE(3) RMOE_ROUTER_CASE(4) RMOE_ROUTER_CASE(5)
    RMOE_ROUTER_CASE(6) RMOE_ROUTER_CASE(7) RMOE_ROUTER_CASE(8) RMOE_ROUTER_CASE(9) RMOE_ROUTER_CASE(10)
    RMOE_ROUTER_CASE(11) RMOE_ROUTER_CASE(12) RMOE_ROUTER_CASE(13) RMOE_ROUTER_CASE(14) RMOE_ROUTER_CASE(15)
    RMOE_ROUTER_CASE(16)
#undef RMOE_ROUTER_CASE
    default:
      return hipErrorInvalidValue;
  }
  return hipGetLastError();
}

hipError_t launch_topk(const float* logits, int T, int E, int k, int score, const float* bias, int renorm,
                       float scaling, int32_t* ids, float* wts, hipStream_t st) {
  if (E > 256 || k > 16 || k > 64) return hipErrorInvalidValue;
  hipLaunchKernelGGL(topk_kernel, dim3((T + 3) / 4), dim3(256), 0, st, logits, T, E, k, score, bias, renorm, scaling,
                     ids, wts);
  return hipGetLastError();
}

size_t prefill_scratch_bytes(const RmoeLayer& L, int T) {
  const size_t A = (size_t)T * L.top_k, R = A + T;
  const size_t tiles = A / kBM + L.n_routed + T / kBM + 4;
  return R * L.Ipad * 2                  // h
         + R * (L.Ipad / 32) * 8         // h group sums
         + R * L.H * 2                   // D
         + (size_t)T * (L.H / 32) * 8    // x group sums
         + (size_t)T * L.n_routed * 4    // logits
         + tiles * 4 + 256 * 3;          // tile table, counts
}

hipError_t launch_moe_prefill(const RmoeLayer& L, const uint16_t* x, int T, const int32_t* ids_in, const float* wts_in,
                              int32_t* ids_out, float* wts_out, const uint16_t* shared_gu, int act, float gb, float vb,
                              bool residual, uint16_t* out, uint16_t* routed, uint16_t* shared_down, uint8_t* scratch,
                              size_t scratch_bytes, RmoeScratch& s, hipStream_t st) {
  const int k = L.top_k, E = L.n_routed;
  const size_t A = (size_t)T * k, R = A + T;
  if (L.n_shared < 1 || prefill_scratch_bytes(L, T) > scratch_bytes) return hipErrorInvalidValue;
  if (A > s.order_elems || (size_t)((A + 1023) / 1024) * E > s.chunk_elems) return hipErrorInvalidValue;
  uint8_t* p = scratch;
  auto carve = [&](size_t bytes) {
    uint8_t* q = p;
    p += (bytes + 255) / 256 * 256;
    return q;
  };
  uint16_t* h = (uint16_t*)carve(R * L.Ipad * 2);
  uint32_t* hsum = (uint32_t*)carve(R * (L.Ipad / 32) * 8);
  uint16_t* D = (uint16_t*)carve(R * L.H * 2);
  uint32_t* xsum = (uint32_t*)carve((size_t)T * (L.H / 32) * 8);
  float* logits = (float*)carve((size_t)T * E * 4);
  const int tile_cap = (int)(A / kBM + E + T / kBM + 4);
  uint32_t* tiles = (uint32_t*)carve((size_t)tile_cap * 4);
  int* ntiles = (int*)carve(256);
  hipError_t err;
  const int32_t* ids = ids_in;
  const float* wts = wts_in;
  if (!ids_in) {
    err = launch_router_gemm(x, T, L.H, L.router_w, E, logits, st);
    if (err != hipSuccess) return err;
    err = launch_topk(logits, T, E, k, L.score, L.router_bias, L.renorm, L.scaling, ids_out, wts_out, st);
    if (err != hipSuccess) return err;
    ids = ids_out;
    wts = wts_out;
  }
  err = launch_dispatch(ids, T, k, E, s.order, s.inv, s.offsets, s, st);
  if (err != hipSuccess) return err;
  {
    const size_t n = (size_t)T * (L.H / 32);
    hipLaunchKernelGGL(group_sums_kernel, dim3((unsigned)((n + 255) / 256)), dim3(256), 0, st, x, T, L.H, xsum);
    if ((err = hipGetLastError()) != hipSuccess) return err;
  }
  if (L.Ipad > L.I) {
    // h columns past I (and their group sums) feed the zero-padded down columns.
    hipLaunchKernelGGL(zero_pad_cols_kernel, dim3((unsigned)((R + 255) / 256)), dim3(256), 0, st, h, hsum, (int)R, L.I,
                       L.Ipad);
    if ((err = hipGetLastError()) != hipSuccess) return err;
  }
  // Gate/up (+ activation): routed groups, and the shared expert unless its gate/up is given.
  GemmArgs g{};
  g.wbase = L.gu;
  g.wstride = L.gu_bytes;
  g.K = L.H;
  g.N_total = 2 * L.I;
  g.inter = L.I;
  g.mode = 0;
  g.n_tiles = (L.I + 127) / 128;
  g.src = x;
  g.order = s.order;
  g.k_routes = k;
  g.n_routed = E;
  g.shared_base = (int)A;
  g.ssum = xsum;
  g.tiles = tiles;
  g.ntiles = ntiles;
  g.offsets = s.offsets;
  g.shared_rows = shared_gu ? 0 : T;
  g.out = h;
  g.out_ld = L.Ipad;
  g.out_ssum = hsum;
  g.act = act;
  g.gb = gb;
  g.vb = vb;
  hipLaunchKernelGGL(tile_table_kernel, dim3(1), dim3(512), 0, st, s.offsets, E, g.shared_rows, tiles, ntiles, tile_cap);
  if ((err = hipGetLastError()) != hipSuccess) return err;
  if (shared_gu) {
    const size_t n = (size_t)T * (L.Ipad / 32);
    hipLaunchKernelGGL(shared_act_kernel, dim3((unsigned)((n + 255) / 256)), dim3(256), 0, st, shared_gu, T, L.I,
                       L.Ipad, act, gb, vb, h + A * L.Ipad, hsum + A * (L.Ipad / 32) * 2);
    if ((err = hipGetLastError()) != hipSuccess) return err;
  }
  {
    const int blocks = (g.n_tiles * tile_cap + 7) / 8 * 8;  // the XCD mapping needs a multiple of 8
    hipLaunchKernelGGL(grouped_gemm_kernel, dim3(blocks), dim3(512), 0, st, g, tile_cap);
    if ((err = hipGetLastError()) != hipSuccess) return err;
  }
  // Down: every sorted row (routed + shared), rows of h contiguous.
  if (shared_gu) {
    hipLaunchKernelGGL(tile_table_kernel, dim3(1), dim3(512), 0, st, s.offsets, E, T, tiles, ntiles, tile_cap);
    if ((err = hipGetLastError()) != hipSuccess) return err;
  }
  GemmArgs d = g;
  d.wbase = L.dn;
  d.wstride = L.dn_bytes;
  d.K = L.Ipad;
  d.N_total = L.H;
  d.mode = 1;
  d.n_tiles = L.H / 256;
  d.src = h;
  d.ssum = hsum;
  d.shared_rows = T;
  d.out = D;
  d.out_ld = L.H;
  d.out_ssum = nullptr;
  {
    const int blocks = (d.n_tiles * tile_cap + 7) / 8 * 8;
    hipLaunchKernelGGL(grouped_gemm_kernel, dim3(blocks), dim3(512), 0, st, d, tile_cap);
    if ((err = hipGetLastError()) != hipSuccess) return err;
  }
  hipLaunchKernelGGL(combine_kernel, dim3(T), dim3(256), 0, st, D, L.H, ids, wts, s.inv, k, (int)A,
                     residual ? x : nullptr, out, routed, shared_down, 1);
  return hipGetLastError();
}

}  // namespace rmoe
