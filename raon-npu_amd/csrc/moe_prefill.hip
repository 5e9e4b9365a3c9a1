// Prefill (many-token) MoE on MFMA: router GEMM + top-k, tile table over the dispatch,
// grouped q4nx GEMMs (gate/up with the activation fused, down), ordered combine.
// Restates NpuBackend.moe_experts_grouped (npu/backend.py:4845-4979) and the planner's
// scatter/combine (kernels/moe_grouped/planner.py:184-322) on the device.
//
// q4nx on fp16 MFMA without rounding the weights:  w = min + scale*n  (n = 4-bit code).
// For one 32-column group g, activation row m and weight row r:
//   sum_k x[m,k] w[r,k] = sum_k x[m,k] * (scale[r]*(n[r,k] - 8)) + (min[r] + 8*scale[r]) * S[m]
// with S[m] = sum_k x[m,k].  scale*(n-8) has at most 11 significant bits (8 of the bf16
// scale times |n-8| <= 8), so it is exact in fp16, and so is every bf16 activation: the
// first sum runs on v_mfma_f32_16x16x32_f16 with no per-group fix-up, the MFMAs of all
// groups accumulating in place.  Range: activation rows carry a power-of-two
// exponent (x rows are normalised to max |x| in [2^14, 2^15); h chunks of 128 units are
// scaled only when their largest value is outside [2^-6, 2^15)) and each weight row's
// scales are normalised by a power of two (largest scale in [2^11, 2^12)); the
// exponents are undone exactly in fp32.  The correction (second sum) is a small GEMM over
// the groups on bf16 MFMA: min and 8*scale are exact bf16 values and S is split exactly
// into three bf16 parts, so its six products are the whole correction.
#include "../../include/raon_moe.h"
#include "rmoe_internal.h"

namespace rmoe {
namespace {

typedef __bf16 bf16x8_t __attribute__((ext_vector_type(8)));
typedef float f32x4_t __attribute__((ext_vector_type(4)));

typedef _Float16 f16x8_t __attribute__((ext_vector_type(8)));
typedef _Float16 f16x2_t __attribute__((ext_vector_type(2)));

__device__ __forceinline__ f32x4_t mfma16(const uint4 a, const uint4 b, f32x4_t c) {
  return __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(bf16x8_t, a), __builtin_bit_cast(bf16x8_t, b), c,
                                                 0, 0, 0);
}
__device__ __forceinline__ f32x4_t mfma16h(const uint4 a, const uint4 b, f32x4_t c) {
  return __builtin_amdgcn_mfma_f32_16x16x32_f16(__builtin_bit_cast(f16x8_t, a), __builtin_bit_cast(f16x8_t, b), c, 0,
                                                0, 0);
}

// Power-of-two exponents of the fp16 operands, from the largest magnitude v of a row or
// chunk (an fp32 value; non-negative).  Zero for a zero or non-finite v (non-finite
// values then pass through unchanged).
//   normalise:  v * 2^-e in [2^14, 2^15)  (x rows: values down to 2^-31 v are exact)
//   chunk:      0 while v is in [2^-6, 2^15), else normalise (h chunks of 128 units, so
//               that a K step of the down GEMM rarely changes exponent).  With e = 0 the
//               values from 2^-17 up are exact and smaller ones round to fp16's 2^-24
//               grid: an absolute error below 2^-25, under 2^-19 v.
__device__ __forceinline__ int f16_exp_normalise(float v) {
  const int be = (int)(__float_as_uint(v) >> 23) & 0xff;
  if (v == 0.f || be == 0xff) return 0;
  return be == 0 ? -140 : be - 127 - 14;
}
__device__ __forceinline__ int f16_exp_chunk(float v) {
  const int be = (int)(__float_as_uint(v) >> 23) & 0xff;
  return (be >= 127 - 6 && be < 127 + 15) ? 0 : f16_exp_normalise(v);
}
// Two bf16 values (one dword) times 2^-e as an fp16 pair (exact for the ranges above).
__device__ __forceinline__ uint32_t bf16x2_to_f16x2(uint32_t v, int e) {
  const float lo = __builtin_amdgcn_ldexpf(bf16_to_f32(v & 0xffffu), -e);
  const float hi = __builtin_amdgcn_ldexpf(__uint_as_float(v & 0xffff0000u), -e);
  return __builtin_bit_cast(uint32_t, __builtin_amdgcn_cvt_pkrtz(lo, hi));
}
__device__ __forceinline__ float max_abs_bf16x8(const uint4 v) {
  const uint32_t w[4] = {v.x, v.y, v.z, v.w};
  float m = 0.f;
#pragma unroll
  for (int i = 0; i < 4; ++i) m = fmaxf(m, fmaxf(fabsf(bf16_to_f32(w[i] & 0xffffu)), fabsf(__uint_as_float(w[i] & 0xffff0000u))));
  return m;
}
// Row stride (bytes) of an exponent table [rows][K/128]: 16-byte aligned rows.
__host__ __device__ inline int exp_stride(int K) { return ((K / 128) + 15) & ~15; }

// Exact 3-way bf16 split of an fp32 value: v = hi + mid + lo (8 + 8 + 8 significant
// bits cover the 24 of fp32), each part the RNE bf16 of the remainder.
__device__ __forceinline__ void split3_bf16(float v, uint32_t& hi, uint32_t& mid, uint32_t& lo) {
  hi = f32_to_bf16(v);
  const float r = v - bf16_to_f32(hi);
  mid = f32_to_bf16(r);
  lo = f32_to_bf16(r - bf16_to_f32(mid));
}
// bf16 pair (a | b << 16) of two fp32 values on the bf16 grid (their top halves).
__device__ __forceinline__ uint32_t pack_bf16_top(float a, float b) {
  return __builtin_amdgcn_perm(__float_as_uint(b), __float_as_uint(a), 0x07060302u);
}
// Two fp32 values -> RNE bf16 pair (a | b << 16) in one instruction; NaNs stay NaNs (the
// reference's canonical 0x7FC0 is applied where values leave the device path).
__device__ __forceinline__ uint32_t cvt_bf16x2(float a, float b) {
  typedef __bf16 bf16x2v __attribute__((ext_vector_type(2)));
  const bf16x2v v = {(__bf16)a, (__bf16)b};
  return __builtin_bit_cast(uint32_t, v);
}
__device__ __forceinline__ float bf16_round_hw(float a) { return __uint_as_float(cvt_bf16x2(a, 0.f) << 16); }
// Group sums are stored planar per row: planes hi, mid, lo of Gp = round_up(G, 8) bf16
// each (G = groups per row; the padding groups hold 0), so that 8 consecutive groups of
// one plane are one 16-byte MFMA operand.
__host__ __device__ inline int sum_planes_gp(int G) { return (G + 7) & ~7; }
__device__ __forceinline__ void store_split3_planar(uint16_t* dst, int Gp, float v) {
  uint32_t hi, mid, lo;
  split3_bf16(v, hi, mid, lo);
  dst[0] = (uint16_t)hi;
  dst[Gp] = (uint16_t)mid;
  dst[2 * Gp] = (uint16_t)lo;
}

// ---------------------------------------------------------------- router GEMM --
// logits[T, E] = x[T, H] . Wr[E, H]^T on MFMA (exact bf16 products, fp32 sums).
// Block: 32 tokens x up to 64 experts x a quarter of K: wave w takes a sixteenth of the
// columns and loads its A (token rows) and B (router rows) fragments straight from global
// memory (the 0.5 MB router stays in L2); the four partial sums meet in LDS and are added
// in wave order.
constexpr int kMaxEFrags = 16;  // E <= 256
constexpr int kRouterTok = 32;

// Grid (ceil(T / 32), 4, E / (16 NFR)): workgroup (b, q, c) takes tokens 32b.., the K
// quarter q and the experts 16 NFR c ..+16 NFR; its wave w the sixteenth 4q + w, whose sum
// runs over 32-column steps in order.  The H/32 steps are dealt to the sixteenths as
// evenly as they divide (sixteenth s: steps [s n / 16, (s+1) n / 16) of n); the split
// depends on H only.  The workgroup adds its waves' sums in wave order and
// writes the quarter's partial logits plogits[q][t][e]; topk_kernel adds the quarters in
// order.  (An expert's sums do not depend on which workgroup holds it, so the split over
// experts, which gives small batches more workgroups, changes no result.)
template <int NFR, int NTB>
__device__ __forceinline__ void router_gemm_block(const uint16_t* __restrict__ x, int T, int H,
                                                  const uint16_t* __restrict__ w, int E, float* __restrict__ plogits,
                                                  int bx, int by, int bz) {
  __shared__ float part[4][kRouterTok][NFR * 16 + 1];
  const int tid = threadIdx.x, lane = tid & 63, wave = wave_id();
  const int l16 = lane & 15, lq = lane >> 4;
  const int q = by, e0 = 16 * NFR * bz;
  const int nsteps = H / 32, sx = 4 * q + wave;
  const int k0 = (sx * nsteps / 16) * 32, kq = ((sx + 1) * nsteps / 16) * 32 - k0;
  const uint16_t* wr = w + (size_t)(e0 + l16) * H + k0 + 8 * lq;
  // With NTB > 1 the workgroup takes NTB blocks of 32 tokens and keeps the router rows of
  // its K slice (at most kRouterKeep steps of 32 columns) in registers across them, so
  // the router is read once per NTB blocks.  A token's sums do not depend on the block.
  constexpr int kRouterKeep = 4;
  uint4 bk[NTB > 1 ? kRouterKeep : 1][NFR];
  const bool keep = NTB > 1 && kq <= 32 * kRouterKeep;
  if constexpr (NTB > 1) {
#pragma unroll
    for (int st = 0; st < kRouterKeep; ++st)
#pragma unroll
      for (int f = 0; f < NFR; ++f)
        bk[st][f] = keep && 32 * st < kq ? *reinterpret_cast<const uint4*>(wr + (size_t)16 * f * H + 32 * st)
                                          : make_uint4(0u, 0u, 0u, 0u);
  }
  for (int tb = 0; tb < NTB; ++tb) {
    const int t0 = (bx * NTB + tb) * kRouterTok;
    if (t0 >= T) break;
    f32x4_t acc[2][NFR];
#pragma unroll
    for (int m = 0; m < 2; ++m)
#pragma unroll
      for (int f = 0; f < NFR; ++f) acc[m][f] = f32x4_t{0.f, 0.f, 0.f, 0.f};
    const uint16_t* xr[2];
#pragma unroll
    for (int m = 0; m < 2; ++m) xr[m] = x + (size_t)min(t0 + 16 * m + l16, T - 1) * H + k0 + 8 * lq;
    if (keep) {
#pragma unroll
      for (int st = 0; st < kRouterKeep; ++st) {
        if (32 * st < kq) {
          uint4 a[2];
#pragma unroll
          for (int m = 0; m < 2; ++m) a[m] = *reinterpret_cast<const uint4*>(xr[m] + 32 * st);
#pragma unroll
          for (int f = 0; f < NFR; ++f)
#pragma unroll
            for (int m = 0; m < 2; ++m) acc[m][f] = mfma16(a[m], bk[st][f], acc[m][f]);
        }
      }
    } else {
#pragma unroll 2
      for (int kk = 0; kk < kq; kk += 32) {
        uint4 a[2], b[NFR];
#pragma unroll
        for (int m = 0; m < 2; ++m) a[m] = *reinterpret_cast<const uint4*>(xr[m] + kk);
#pragma unroll
        for (int f = 0; f < NFR; ++f) b[f] = *reinterpret_cast<const uint4*>(wr + (size_t)16 * f * H + kk);
#pragma unroll
        for (int f = 0; f < NFR; ++f)
#pragma unroll
          for (int m = 0; m < 2; ++m) acc[m][f] = mfma16(a[m], b[f], acc[m][f]);
      }
    }
    if (tb > 0) __syncthreads();  // the previous block's sums have been read from part
#pragma unroll
    for (int m = 0; m < 2; ++m)
#pragma unroll
      for (int f = 0; f < NFR; ++f)
#pragma unroll
        for (int i = 0; i < 4; ++i) part[wave][16 * m + 4 * lq + i][16 * f + l16] = acc[m][f][i];
    __syncthreads();
    constexpr int kCols = NFR * 16;
    for (int idx = tid; idx < kRouterTok * kCols; idx += 256) {
      const int r = idx / kCols, c = idx % kCols;
      const int t = t0 + r;
      if (t < T)
        plogits[((size_t)q * T + t) * E + e0 + c] = ((part[0][r][c] + part[1][r][c]) + part[2][r][c]) + part[3][r][c];
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
// The same sum with its 8 partial sums taken by lanes 0..7 of the wave at once (every
// lane of the wave calls it and gets the result).
__device__ float np_sum_f32_lds_wave(const float* v, int n) {
  const int lane = threadIdx.x & 63;
  if (n < 8) {
    float r = 0.f;
    if (lane == 0)
      for (int i = 0; i < n; ++i) r = __fadd_rn(r, v[i]);
    return __shfl(r, 0, 64);
  }
  const int full = n & ~7;  // elements in whole rows of 8
  float r = 0.f;
  if (lane < 8) {
    r = v[lane];
    for (int i = 8 + lane; i < full; i += 8) r = __fadd_rn(r, v[i]);
  }
  const float r0 = __shfl(r, 0, 64), r1 = __shfl(r, 1, 64), r2 = __shfl(r, 2, 64), r3 = __shfl(r, 3, 64);
  const float r4 = __shfl(r, 4, 64), r5 = __shfl(r, 5, 64), r6 = __shfl(r, 6, 64), r7 = __shfl(r, 7, 64);
  float res = __fadd_rn(__fadd_rn(__fadd_rn(r0, r1), __fadd_rn(r2, r3)), __fadd_rn(__fadd_rn(r4, r5), __fadd_rn(r6, r7)));
  for (int i = full; i < n; ++i) res = __fadd_rn(res, v[i]);
  return res;
}

// Order-preserving bits of a float (larger float, larger key); NaN is given the lowest
// key, so it is never selected ahead of a number (numpy's argsort puts NaN last).
__device__ __forceinline__ uint32_t float_order_key(float f) {
  const uint32_t u = __float_as_uint(f);
  if (f != f) return 0u;
  return (u & 0x80000000u) ? ~u : (u | 0x80000000u);
}

// One wave per token: logits (the four K-quarter partials of router_gemm_block, [4][T][E],
// added in order), scores, selection (score + bias, ties to the lower id), renorm.
// Selection by rank: expert e has key (order bits of its selection score << 8) | (255 - e)
// and rank #{keys larger than its own}; the experts of rank < k are the top k, in rank
// order -- the order of repeated arg-max with ties to the lower id.
// NE: experts per lane (E <= 64 * NE).
// counts (may be null): the dispatch chunk counts [chunk][E] (zero on entry), to which the
// workgroup adds its assignments, 4 tokens' k routes at most spanning two chunks, counted in
// LDS first and then added once per (chunk, expert).
template <int NE>
__global__ __launch_bounds__(256) void topk_kernel(const float* __restrict__ logits, int T, int E, int k, int score,
                                                   const float* __restrict__ bias, int renorm, float scaling,
                                                   int32_t* __restrict__ ids, float* __restrict__ wts,
                                                   int32_t* __restrict__ counts) {
  __shared__ float sc[4][256];
  __shared__ __attribute__((aligned(16))) uint64_t keys[4][256];
  __shared__ float ch[4][16];
  __shared__ int hist[2][256];
  const int lane = threadIdx.x & 63, wave = wave_id();
  const int t = blockIdx.x * 4 + wave;
  const int cbase = blockIdx.x * 4 * k / kDispatchChunk;
  if (counts) {
    hist[0][threadIdx.x] = 0;
    hist[1][threadIdx.x] = 0;
    __syncthreads();
  }
  if (t < T) {
  // Logits: the router GEMM's four K-quarter partials, added in order.
  const size_t qs = (size_t)T * E;
  const float* lq0 = logits + (size_t)t * E;
  float lg[NE];
#pragma unroll
  for (int i = 0; i < NE; ++i) {
    const int e = lane + 64 * i;
    lg[i] = e < E ? ((lq0[e] + lq0[qs + e]) + lq0[2 * qs + e]) + lq0[3 * qs + e] : 0.f;
  }
  float* s = sc[wave];
  if (score == 0) {
#pragma unroll
    for (int i = 0; i < NE; ++i)
      if (lane + 64 * i < E) s[lane + 64 * i] = 1.0f / (1.0f + expf(-lg[i]));
  } else {
    float m = -__builtin_inff();
#pragma unroll
    for (int i = 0; i < NE; ++i)
      if (lane + 64 * i < E) m = fmaxf(m, lg[i]);
#pragma unroll
    for (int off = 32; off > 0; off >>= 1) m = fmaxf(m, __shfl_xor(m, off, 64));
#pragma unroll
    for (int i = 0; i < NE; ++i)
      if (lane + 64 * i < E) s[lane + 64 * i] = expf(lg[i] - m);
    __builtin_amdgcn_wave_barrier();
    __builtin_amdgcn_fence(__ATOMIC_SEQ_CST, "wavefront");
    const float total = np_sum_f32_lds_wave(s, E);
    __builtin_amdgcn_wave_barrier();
#pragma unroll
    for (int i = 0; i < NE; ++i)
      if (lane + 64 * i < E) s[lane + 64 * i] = s[lane + 64 * i] / total;
  }
  // Selection keys; keys past E (up to the next even count) are 0 and rank below all.
  uint64_t key[NE];
#pragma unroll
  for (int i = 0; i < NE; ++i) {
    const int e = lane + 64 * i;
    float c = 0.f;
    if (e < E) c = bias ? __fadd_rn(s[e], bias[e]) : s[e];
    key[i] = e < E ? ((uint64_t)float_order_key(c) << 8) | (uint64_t)(255 - e) : 0ull;
    if (e < ((E + 1) & ~1)) keys[wave][e] = key[i];
  }
  __builtin_amdgcn_wave_barrier();
  __builtin_amdgcn_fence(__ATOMIC_SEQ_CST, "wavefront");
  int rank[NE] = {};
  const uint4* kv = reinterpret_cast<const uint4*>(keys[wave]);
  for (int j = 0; j < (E + 1) / 2; ++j) {
    const uint4 v = kv[j];
    const uint64_t k0 = (uint64_t)v.x | ((uint64_t)v.y << 32), k1 = (uint64_t)v.z | ((uint64_t)v.w << 32);
#pragma unroll
    for (int i = 0; i < NE; ++i) rank[i] += (k0 > key[i] ? 1 : 0) + (k1 > key[i] ? 1 : 0);
  }
#pragma unroll
  for (int i = 0; i < NE; ++i) {
    const int e = lane + 64 * i;
    if (e < E && rank[i] < k) {
      ids[(size_t)t * k + rank[i]] = e;
      ch[wave][rank[i]] = s[e];
      if (counts) atomicAdd(&hist[(t * k + rank[i]) / kDispatchChunk - cbase][e], 1);
    }
  }
  __builtin_amdgcn_wave_barrier();
  __builtin_amdgcn_fence(__ATOMIC_SEQ_CST, "wavefront");
  float denom = 1.f;
  if (lane == 0 && renorm) denom = __fadd_rn(np_sum_f32_lds(ch[wave], k), 1e-20f);
  denom = __shfl(denom, 0, 64);
  if (lane < k) {
    float v = renorm ? ch[wave][lane] / denom : ch[wave][lane];
    wts[(size_t)t * k + lane] = __fmul_rn(v, scaling);
  }
  }
  if (counts) {
    __syncthreads();
    const int nch = (T * k + kDispatchChunk - 1) / kDispatchChunk;
#pragma unroll
    for (int c = 0; c < 2; ++c) {
      const int v = hist[c][threadIdx.x];
      if (v && (int)threadIdx.x < E && cbase + c < nch)
        __hip_atomic_fetch_add(&counts[(size_t)(cbase + c) * E + threadIdx.x], v, __ATOMIC_RELAXED,
                               __HIP_MEMORY_SCOPE_AGENT);
    }
  }
}

// ------------------------------------------------------ activation prep (x) --
// For each token row of x [T, K] (bf16): the fp16 operand xh = x * 2^-e (e normalises
// the row, f16_exp_normalise), its exponent xe [T], and the group sums S[row, g] of the 32 bf16 values of each
// group as an exact 3-way bf16 split (planar layout of store_split3_planar).
// One wave per row; lane L holds the 16-byte chunks L + 64i (K <= 8192).
constexpr int kPrepMaxChunks = 16;
__device__ __forceinline__ void prep_x_block(const uint16_t* __restrict__ x, int T, int K, uint16_t* __restrict__ xh,
                                             int8_t* __restrict__ xe, uint16_t* __restrict__ xsum, int bx) {
  const int lane = threadIdx.x & 63, t = bx * 4 + (threadIdx.x >> 6);
  if (t >= T) return;
  const int nch = K / 8, G = K / 32, Gp = sum_planes_gp(G);
  const uint4* src = reinterpret_cast<const uint4*>(x + (size_t)t * K);
  uint4 v[kPrepMaxChunks];
  float mx = 0.f;
  uint16_t* ds = xsum + (size_t)t * 3 * Gp;
#pragma unroll
  for (int i = 0; i < kPrepMaxChunks; ++i) {
    const int c = lane + 64 * i;
    if (64 * i >= nch) break;
    float s = 0.f;
    if (c < nch) {
      v[i] = src[c];
      mx = fmaxf(mx, max_abs_bf16x8(v[i]));
      const uint32_t w[4] = {v[i].x, v[i].y, v[i].z, v[i].w};
#pragma unroll
      for (int d = 0; d < 4; ++d) s += bf16_to_f32(w[d] & 0xffffu) + __uint_as_float(w[d] & 0xffff0000u);
    }
    // A group is the four chunks of lanes 4q..4q+3.
    s += __shfl_xor(s, 1, 64);
    s += __shfl_xor(s, 2, 64);
    if (c < nch && (lane & 3) == 0) store_split3_planar(ds + c / 4, Gp, s);
  }
  for (int g = G + lane; g < Gp; g += 64) ds[g] = ds[Gp + g] = ds[2 * Gp + g] = 0;
#pragma unroll
  for (int off = 32; off > 0; off >>= 1) mx = fmaxf(mx, __shfl_xor(mx, off, 64));
  const int e = f16_exp_normalise(mx);
  uint4* dst = reinterpret_cast<uint4*>(xh + (size_t)t * K);
#pragma unroll
  for (int i = 0; i < kPrepMaxChunks; ++i) {
    const int c = lane + 64 * i;
    if (64 * i >= nch) break;
    if (c < nch)
      dst[c] = make_uint4(bf16x2_to_f16x2(v[i].x, e), bf16x2_to_f16x2(v[i].y, e), bf16x2_to_f16x2(v[i].z, e),
                          bf16x2_to_f16x2(v[i].w, e));
  }
  if (lane == 0) xe[t] = (int8_t)e;
}
__global__ __launch_bounds__(256) void prep_x_kernel(const uint16_t* __restrict__ x, int T, int K,
                                                     uint16_t* __restrict__ xh, int8_t* __restrict__ xe,
                                                     uint16_t* __restrict__ xsum) {
  prep_x_block(x, T, K, xh, xe, xsum, blockIdx.x);
}
// The router GEMM and the activation-row preparation (both read only x) in one launch:
// workgroups 0..n_router-1 are router workgroups (token block, K quarter, expert group),
// the rest prepare four rows each.  One launch fewer on the routing's critical path.
template <int NFR, int NTB>
__global__ __launch_bounds__(256) void router_prep_kernel(const uint16_t* __restrict__ x, int T, int H,
                                                          const uint16_t* __restrict__ w, int E,
                                                          float* __restrict__ plogits, int n_router, int ngroups,
                                                          uint16_t* __restrict__ xh, int8_t* __restrict__ xe,
                                                          uint16_t* __restrict__ xsum, int32_t* __restrict__ zero,
                                                          int nzero) {
  const int b = blockIdx.x;
  if (b < n_router) {
    router_gemm_block<NFR, NTB>(x, T, H, w, E, plogits, b / (4 * ngroups), (b / ngroups) % 4, b % ngroups);
  } else {
    // The preparation workgroups also clear nzero ints at zero (the top-k's chunk counts).
    const int pb = b - n_router;
    for (int i = pb * 256 + (int)threadIdx.x; i < nzero; i += (gridDim.x - n_router) * 256) zero[i] = 0;
    prep_x_block(x, T, H, xh, xe, xsum, pb);
  }
}

// ----------------------------------------------------------------- tile table --
// One workgroup of 512 threads; thread e owns group e (routed 0..n_routed-1, shared
// n_routed, whose rows start at shared_base).  (The dispatch scatter builds the same table
// in its first workgroup when the groups fit its 256 threads; this kernel serves the other
// cases and the table for a second GEMM with other shared rows.)
__global__ __launch_bounds__(512) void tile_table_kernel(const int32_t* __restrict__ offsets, int n_routed,
                                                         int shared_base, int shared_rows, uint32_t* __restrict__ tiles,
                                                         int* __restrict__ ntiles, int cap) {
  __shared__ int wsum[kTileClasses][8];
  const int e = threadIdx.x;
  const int ng = n_routed + (shared_rows > 0 ? 1 : 0);
  int b = 0, end = 0;
  if (e < ng) {
    b = e < n_routed ? offsets[e] : shared_base;
    end = e < n_routed ? offsets[e + 1] : shared_base + shared_rows;
  }
  tile_table_block<8>(e, ng, b, end, tiles, ntiles, cap, wsum);
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
  // activation rows (fp16 operands, see prep_x_kernel and the gate/up epilogue)
  const uint16_t* src;      // mode 0: xh [T, K] gathered by token; mode 1: h [rows, K] in sorted order
  const int8_t* aexp;       // power-of-two exponent of each src row (int8 [rows])
  const int32_t* order;     // mode 0: sorted position -> assignment (token*k + route)
  int k_routes;
  int n_routed;             // group id n_routed = shared expert (rows identity tokens / sorted)
  int shared_base;          // sorted row index of the first shared row
  const uint16_t* ssum;     // row group sums (planar, store_split3_planar): mode 0 by token; mode 1 by row
  const uint32_t* tiles;
  const int* ntiles;
  const int32_t* offsets;   // group row ends: offsets[e+1] (routed); shared end = shared_base + shared_rows
  int shared_rows;
  // outputs
  uint16_t* out;            // mode 0: h [rows, out_ld]; mode 1: D [rows, out_ld]
  int out_ld;
  uint16_t* out_ssum;       // mode 0: group sums of the h rows (planar, out_ld/32 groups)
  int8_t* out_exp;          // mode 0: exponents of the h rows per 128-unit chunk [rows][exp_stride(out_ld)]
  int act;
  float gb, vb;
  // bfp16 weights (down of a weights-d layer): per expert and weight row the largest
  // max(e, 7) of the row's blocks ([experts][N_total]).
  const uint8_t* rowexp;
  // mode 1: D rows are stored with the non-temporal hint (a large D, read once by the
  // combine, then stays out of the caches the GEMM reuses weights and rows from).
  int out_nt;
};

__device__ __forceinline__ int group_end(const GemmArgs& a, int e) {
  return e < a.n_routed ? a.offsets[e + 1] : a.shared_base + a.shared_rows;
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
// Group sums of one block of 32 groups for the tile's rows: [row][hi, mid, lo][32] bf16.
constexpr int kSRow = 3 * 32 * 2;
constexpr int kSBlock = kBM * kSRow;  // 24,576: two blocks fit in ring slot 2

typedef unsigned u32x4v __attribute__((ext_vector_type(4)));

// 16 bytes per lane from global memory straight into LDS: lane L writes lds + 16 L.
// Written as inline assembly so that the compiler does not treat every later LDS read
// as dependent on it (it would wait for all outstanding loads before each one); the
// kernel's own waits order the copies.  M0 is saved and restored.  On gfx9 an LDS copy
// needs one wait state after an SALU write of M0 (the compiler pads its own copies the
// same way, but cannot see inside an asm statement): hence the s_nop.
__device__ __forceinline__ void dma16(const void* g, uint32_t lds) {
  uint32_t saved;
  asm volatile(
      "s_mov_b32 %0, m0\n\t"
      "s_mov_b32 m0, %2\n\t"
      "s_nop 0\n\t"
      "global_load_lds_dwordx4 %1, off\n\t"
      "s_mov_b32 m0, %0"
      : "=&s"(saved)
      : "v"(g), "s"(__builtin_amdgcn_readfirstlane(lds))
      : "memory");
}
// dma16 with the non-temporal hint, for the weight tiles: each is copied by one tile of
// the GEMM (the m-tiles of an expert share them only through L2, close in time), so
// they should not push out the activation rows, which every N-tile of an m-tile reads.
__device__ __forceinline__ void dma16_nt(const void* g, uint32_t lds) {
  uint32_t saved;
  asm volatile(
      "s_mov_b32 %0, m0\n\t"
      "s_mov_b32 m0, %2\n\t"
      "s_nop 0\n\t"
      "global_load_lds_dwordx4 %1, off nt\n\t"
      "s_mov_b32 m0, %0"
      : "=&s"(saved)
      : "v"(g), "s"(__builtin_amdgcn_readfirstlane(lds))
      : "memory");
}
// A 16-byte global load the compiler does not count: its result may be used only after
// a wait_tied() on it (compiler-counted loads would make the compiler wait for every
// copy issued after them).
__device__ __forceinline__ u32x4v gload16(const void* p) {
  u32x4v v;
  asm volatile("global_load_dwordx4 %0, %1, off" : "=v"(v) : "v"(p) : "memory");
  return v;
}
// Wait until at most `pending` of this wave's loads are in flight, then meet the
// workgroup.  The count is an immediate, so each value is a branch of its own.
__device__ __forceinline__ void ring_wait(int pending) {
  switch (pending) {
    case 7: asm volatile("s_waitcnt vmcnt(7) lgkmcnt(0)\n\ts_barrier" ::: "memory"); break;
    case 6: asm volatile("s_waitcnt vmcnt(6) lgkmcnt(0)\n\ts_barrier" ::: "memory"); break;
    case 5: asm volatile("s_waitcnt vmcnt(5) lgkmcnt(0)\n\ts_barrier" ::: "memory"); break;
    case 4: asm volatile("s_waitcnt vmcnt(4) lgkmcnt(0)\n\ts_barrier" ::: "memory"); break;
    case 3: asm volatile("s_waitcnt vmcnt(3) lgkmcnt(0)\n\ts_barrier" ::: "memory"); break;
    default: asm volatile("s_waitcnt vmcnt(0) lgkmcnt(0)\n\ts_barrier" ::: "memory"); break;
  }
}
// Hands the coefficient registers of gload16() to the compiler: placed after the wait
// that covers their loads, it is where their values are defined for the code after it.
__device__ __forceinline__ void tie_coef(u32x4v (&c)[2][2]) {
  asm volatile("" : "+v"(c[0][0]), "+v"(c[0][1]), "+v"(c[1][0]), "+v"(c[1][1])::"memory");
}
#define RMOE_VM_WAIT(N) asm volatile("s_waitcnt vmcnt(" #N ") lgkmcnt(0)\n\ts_barrier" ::: "memory")
// ring_wait for the counts of the coefficient waits (they depend on the tile class and
// the wave), then tie_coef().  The branches of the switch hold no register operands: had
// each branch's wait also tied the registers, the values would merge after the switch
// and the compiler would copy the loaded registers into the ones it chose for each
// branch, before that branch's wait -- copies that read a register whose load has not
// yet landed.
__device__ __forceinline__ void wait_tied(int pending, u32x4v (&c)[2][2]) {
  switch (pending) {
    case 17: RMOE_VM_WAIT(17); break;
    case 15: RMOE_VM_WAIT(15); break;
    case 14: RMOE_VM_WAIT(14); break;
    case 13: RMOE_VM_WAIT(13); break;
    case 12: RMOE_VM_WAIT(12); break;
    case 11: RMOE_VM_WAIT(11); break;
    case 10: RMOE_VM_WAIT(10); break;
    case 9: RMOE_VM_WAIT(9); break;
    case 8: RMOE_VM_WAIT(8); break;
    case 6: RMOE_VM_WAIT(6); break;
    default: RMOE_VM_WAIT(0); break;
  }
  tie_coef(c);
}
// Largest of v over the 16 lanes of a DPP row, in every lane of the row: quad swaps, then
// the half-row and row mirrors (VALU moves, no LDS permute).
template <int CTRL>
__device__ __forceinline__ float dpp_mov(float v) {
  return __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), CTRL, 0xF, 0xF, false));
}
__device__ __forceinline__ float row16_max(float v) {
  v = fmaxf(v, dpp_mov<0xB1>(v));   // quad_perm [1,0,3,2]
  v = fmaxf(v, dpp_mov<0x4E>(v));   // quad_perm [2,3,0,1]
  v = fmaxf(v, dpp_mov<0x141>(v));  // row_half_mirror
  return fmaxf(v, dpp_mov<0x140>(v));  // row_mirror
}
// (x & m) | o in one instruction (the compiler keeps the two-instruction form).
__device__ __forceinline__ uint32_t and_or(uint32_t x, uint32_t m, uint32_t o) {
  uint32_t r;
  asm("v_and_or_b32 %0, %1, %2, %3" : "=v"(r) : "v"(x), "v"(m), "v"(o));
  return r;
}

// SiLU-GLU g*sigmoid(g)*u with the overflow-free sigmoid of the oracle, on the hardware
// exp2 and reciprocal (one Newton step): within a few fp32 ulps of the correctly
// rounded form, far below the bf16 rounding that follows.
__device__ __forceinline__ float swiglu_fast(float g, float u) {
  const float e = __builtin_amdgcn_exp2f(-fabsf(g) * 1.44269504088896341f);
  const float d = 1.0f + e;
  float r = __builtin_amdgcn_rcpf(d);
  r = fmaf(r, fmaf(-d, r, 1.0f), r);
  const float sig = g >= 0.f ? r : e * r;
  return (g * sig) * u;
}

// Grid: n_tiles * tile_cap workgroups (rounded to a multiple of 8), 512 threads (8 waves).
// A workgroup multiplies 128 sorted rows by 256 weight rows; wave w takes all 128 rows
// (8 MFMA fragments) and two 16-row weight fragments:
//   gate/up: intermediate units 128*nt + 16w..+15: fragment 0 the gate rows, 1 the up
//            rows, so the activation stays in the lane;
//   down:    output rows 256*nt + 16w and 256*nt + 128 + 16w.
// With w = (min + 8 scale) + scale (n - 8) per group g of 32 columns:
//   y = sum_g sum_k x_k scale_g (n_k - 8) + sum_g (min_g + 8 scale_g) * S_g,
// S_g the group sums of the row.  The first sum runs on fp16 MFMAs: A the row scaled by
// its power-of-two exponent, B = scale (n - 8) scaled by the lane's weight-row exponent
// (exact in fp16: a bf16 scale times an integer of magnitude <= 8), fp32 accumulation.
// The second sum (the correction) runs first, on bf16 MFMAs with exact operands, from
// group sums copied into ring slot 2 while the first two K steps' copies are in flight.
// K loop: a three-deep LDS ring filled by global->LDS copies; per K step one barrier,
// then the copy for step kt+2 into the slot step kt-1 used.
// One (m-tile, n-tile) with MF live 16-row fragments; tl is the tile list of its class.
// lds / rowidx / row_e are the kernel's shared arrays.
template <int MF>
__device__ __forceinline__ void gemm_tile(const GemmArgs& a, const uint32_t* __restrict__ tl, int mt, int nt,
                                          uint8_t* lds, int* rowidx, int8_t* row_e) {
  const uint32_t te = tl[mt];
  const int e = (int)(te & 511u), row0 = (int)(te >> 9);
  const int rend = group_end(a, e);
  const int nrows = min(kBM, rend - row0);
  const int tid = threadIdx.x, lane = tid & 63, wave = wave_id();
  const int l16 = lane & 15, lq = lane >> 4;
  const int nkt = a.K / kTileCols;
  const uint8_t* W = a.wbase + (size_t)e * a.wstride;
  const uint32_t lds0 = (uint32_t)(uintptr_t)lds;

  // Source row of each tile row (token for gate/up, sorted row for down); rows past the
  // tile use the tile's first row (their results are not stored).
  if (tid < kBM) {
    const int p = row0 + (tid < nrows ? tid : 0);
    const int src = a.mode == 1 ? p : (e < a.n_routed ? a.order[p] / a.k_routes : p - a.shared_base);
    rowidx[tid] = src;
    row_e[tid] = a.aexp[src];
  }
  __syncthreads();

  // The workgroup's four 64-row weight bands.  Gate/up: gate bands 2nt, 2nt+1, up bands
  // I/64 + 2nt, +1; a band past I (last n-tile when I % 128 != 0) reads band 0 instead
  // and its results are not stored.  Down: bands 4nt..4nt+3.
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
  // Fragment f of this wave: weight tile (w/4) + 2f of the four, rows 16*(w%4)..+15.
  const int ft0 = wave >> 2, frow = 16 * (wave & 3) + l16;

  // Copy descriptors.  Activations: copy q = wave + 8i (i < MF / 2: the tile's 16 * MF
  // live rows; the others are never read) fills LDS rows 4q..4q+3;
  // lane L brings row 4q + L/16 into position L%16 of the row: 16-byte chunk
  // tau((L%16) ^ (row%16)), tau(4a + b) = 4b + a.  A row's chunk c then sits at position
  // tau(c) ^ (row%16): the K loop's reads of chunks 4lq + j land on positions
  // (4j + lq) ^ row, a pattern free of LDS bank conflicts.
  const uint8_t* xg[4];
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const int q = wave + 8 * i, r = 4 * q + (lane >> 4);
    const int pc = (lane & 15) ^ (r & 15), c = ((pc & 3) << 2) | (pc >> 2);
    xg[i] = reinterpret_cast<const uint8_t*>(a.src + (size_t)rowidx[r] * a.K) + 16 * c;
  }
  // Weights: copy v = wave + 8i (i < 3, v < 20) is 1 KB piece v%5 of tile v/5.
  const int n_wcopy = wave < 4 ? 3 : 2;
  const uint8_t* wg[3];
#pragma unroll
  for (int i = 0; i < 3; ++i) {
    const int v = min(wave + 8 * i, 19), t = v / 5, p = v % 5;
    wg[i] = W + (size_t)band[t] * nkt * kTileBytes + 1024 * p + 16 * lane;
  }
  constexpr int kXCopies = MF / 2;
  auto issue_to = [&](int kt, int slot) {
    const uint32_t sb = lds0 + (uint32_t)(slot * kStageBytes);
#pragma unroll
    for (int i = 0; i < kXCopies; ++i) dma16(xg[i] + (size_t)kt * 256, sb + 1024u * (uint32_t)(wave + 8 * i));
#pragma unroll
    for (int i = 0; i < 3; ++i) {
      if (i < n_wcopy) {
        const int v = wave + 8 * i, t = v / 5, p = v % 5;
        dma16_nt(wg[i] + (size_t)kt * kTileBytes, sb + (uint32_t)(kXBytes + t * kTileBytes + 1024 * p));
      }
    }
  };
  auto issue = [&](int kt) { issue_to(kt, kt % kStages); };
  const int per_stage = kXCopies + n_wcopy;

  // Group sums, planar per row: [hi | mid | lo] planes of Gp (G rounded up to 8) bf16.
  // Block b (groups 32b..32b+31) goes to half (b & 1) of ring slot 2 as 24 copies of
  // 1 KB, 3 per wave; chunks past Gp read the row's first chunk (coefficient 0).
  const int G = a.K / 32, Gp = (G + 7) & ~7, nblk = (G + 31) / 32;
  const uint32_t sbase = lds0 + 2u * kStageBytes;
  auto issue_s = [&](int blk) {
#pragma unroll
    for (int i = 0; i < 3; ++i) {
      const int o = 1024 * (wave + 8 * i) + 16 * lane;
      const int r = o / kSRow, rem = o - r * kSRow, part = rem >> 6, g = 32 * blk + 8 * ((rem & 63) >> 4);
      dma16(a.ssum + (size_t)rowidx[r] * 3 * Gp + part * Gp + (g < Gp ? g : 0),
            sbase + (uint32_t)((blk & 1) * kSBlock + 1024 * (wave + 8 * i)));
    }
  };
  // Correction coefficients: scale|min words of the lane's row for groups gl..gl+7 of a
  // block (gl = 32*blk + 8*lq) from the weight tiles in global memory; past G they are
  // masked to zero after the wait.
  auto load_coef = [&](int blk, u32x4v (&c)[2][2]) {
    const int gl = 32 * blk + 8 * lq;
#pragma unroll
    for (int f = 0; f < 2; ++f)
#pragma unroll
      for (int h = 0; h < 2; ++h) {
        const int kt = gl / 4 + h;
        c[f][h] = gload16(W + ((size_t)band[ft0 + 2 * f] * nkt + (4 * kt < G ? kt : 0)) * kTileBytes + kCodeBytes +
                          frow * 16);
      }
  };
  // Issue order per wave (fixed counts for the waits below): coefficients of blocks 0
  // and 1 (8 loads), group-sum blocks 0 and 1 (3 + 3), K steps 0 and 1 (2 x per_stage).
  // With one block, block 1 repeats block 0; with one K step, step 1 repeats step 0
  // into slot 1 (unused then).
  u32x4v cf0[2][2], cf1[2][2];
  load_coef(0, cf0);
  load_coef(nblk > 1 ? 1 : 0, cf1);
  issue_s(0);
  issue_s(nblk > 1 ? 1 : 0);
  issue(0);
  issue_to(nkt > 1 ? 1 : 0, 1);

  f32x4_t acc[MF][2];
#pragma unroll
  for (int m = 0; m < MF; ++m) {
    acc[m][0] = f32x4_t{0.f, 0.f, 0.f, 0.f};
    acc[m][1] = f32x4_t{0.f, 0.f, 0.f, 0.f};
  }
  const uint32_t xrow = (uint32_t)l16 * 256u;  // A row 16m + l16: m*4096 + xrow

  // acc += sum_g (min + 8*scale)[r, g] * S[m, g] over one block of 32 groups, as
  // sum_g min * S + sum_g (8*scale) * S: min and 8*scale are exact bf16 values (a bf16
  // scale times 8 keeps its 8 significant bits), S is split exactly into 3 bf16 parts, so
  // the six products are the whole correction and only the fp32 accumulation rounds.  Also
  // tracks the largest scale (as bf16 bits; scales are >= 0) of the lane's weight rows.
  uint32_t smax[2] = {0u, 0u};
  auto corr_block = [&](int blk, const u32x4v (&c)[2][2]) {
    const int gl = 32 * blk + 8 * lq;
    uint4 bmin[2], bsc8[2];
#pragma unroll
    for (int f = 0; f < 2; ++f) {
      const uint32_t sv[8] = {c[f][0].x, c[f][0].y, c[f][0].z, c[f][0].w, c[f][1].x, c[f][1].y, c[f][1].z, c[f][1].w};
      uint32_t w[8];
      float s8[8];
#pragma unroll
      for (int i = 0; i < 8; ++i) {
        w[i] = gl + i < G ? sv[i] : 0u;  // groups past G: min 0, scale 0
        smax[f] = max(smax[f], w[i] & 0x7fffu);
        s8[i] = 8.f * bf16_to_f32(w[i] & 0xffffu);
      }
      bmin[f] = make_uint4(pack_bf16_top(__uint_as_float(w[0]), __uint_as_float(w[1])),
                           pack_bf16_top(__uint_as_float(w[2]), __uint_as_float(w[3])),
                           pack_bf16_top(__uint_as_float(w[4]), __uint_as_float(w[5])),
                           pack_bf16_top(__uint_as_float(w[6]), __uint_as_float(w[7])));
      bsc8[f] = make_uint4(pack_bf16_top(s8[0], s8[1]), pack_bf16_top(s8[2], s8[3]), pack_bf16_top(s8[4], s8[5]),
                           pack_bf16_top(s8[6], s8[7]));
    }
    const uint8_t* ss = lds + 2 * kStageBytes + (blk & 1) * kSBlock + l16 * kSRow + 16 * lq;
    // Six products per (m, f), the low part of S first; consecutive MFMAs go to different
    // accumulators (16 independent chains).
#pragma unroll
    for (int half = 0; half < (MF + 3) / 4; ++half) {
      __builtin_amdgcn_sched_barrier(0);
      uint4 ah[4], am[4], al[4];
#pragma unroll
      for (int mm = 0; mm < 4; ++mm) {
        const int m = 4 * half + mm;
        if (m >= MF) continue;
        ah[mm] = *reinterpret_cast<const uint4*>(ss + m * 16 * kSRow);
        am[mm] = *reinterpret_cast<const uint4*>(ss + m * 16 * kSRow + 64);
        al[mm] = *reinterpret_cast<const uint4*>(ss + m * 16 * kSRow + 128);
      }
#pragma unroll
      for (int p = 0; p < 6; ++p)
#pragma unroll
        for (int mm = 0; mm < 4; ++mm)
#pragma unroll
          for (int f = 0; f < 2; ++f) {
            const int m = 4 * half + mm;
            if (m >= MF) continue;
            const uint4 av = p < 2 ? al[mm] : p < 4 ? am[mm] : ah[mm];
            const uint4 bv = (p & 1) ? bsc8[f] : bmin[f];
            acc[m][f] = mfma16(av, bv, acc[m][f]);
          }
    }
  };
  // Block 0: past it are in flight group-sum block 1 (3) and K steps 0 and 1.
  wait_tied(3 + 2 * per_stage, cf0);
  corr_block(0, cf0);
  if (nblk > 1) {
    wait_tied(2 * per_stage, cf1);
    corr_block(1, cf1);
  }
  for (int blk = 2; blk < nblk; ++blk) {  // K > 2048: blocks reuse the halves of slot 2
    asm volatile("s_barrier" ::: "memory");
    u32x4v cfb[2][2];
    load_coef(blk, cfb);
    issue_s(blk);
    wait_tied(0, cfb);
    corr_block(blk, cfb);
  }

  // Weight-row exponents: the lane's rows in fragment f have their scales multiplied by
  // 2^-fx[f] so that the largest lies in [2^11, 2^12) (8 * scale < 2^15 in fp16).
  int fx[2];
#pragma unroll
  for (int f = 0; f < 2; ++f) {
    uint32_t m = smax[f];
    m = max(m, (uint32_t)__shfl_xor((int)m, 16, 64));
    m = max(m, (uint32_t)__shfl_xor((int)m, 32, 64));
    const int be = (int)(m >> 7) & 0xff;
    fx[f] = (m == 0u || be == 0xff) ? 0 : (be == 0 ? -138 : be - 127 - 11);
  }
  // The correction is in true units; the K loop accumulates in units of
  // 2^-(row exponent + fx): scale acc over (lane rows 16m + 4lq + i, fragment f).
  auto scale_rows = [&](const int8_t* rowe, int sign) {
#pragma unroll
    for (int m = 0; m < MF; ++m) {
      const uint32_t e4 = *reinterpret_cast<const uint32_t*>(rowe + 16 * m + 4 * lq);
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const int er = (int)(int8_t)(e4 >> (8 * i));
#pragma unroll
        for (int f = 0; f < 2; ++f) acc[m][f][i] = __builtin_amdgcn_ldexpf(acc[m][f][i], sign * (er + fx[f]));
      }
    }
  };
  scale_rows(row_e, -1);

  // Main K loop:  acc += sum_k x[m,k] * (scale[r,g] * 2^-fx) * (n[r,k] - 8), fp16 operands.
  // K assignment of the MFMAs: within a K step (4 groups of 32 columns), MFMA j takes
  // columns 32*lq + 8j .. +7 from lane quarter lq.  A lane's B operands of a step then
  // all come from one group (lq) of its row -- one 16-byte code word and one scale per
  // step -- and a group's scale stays inside B, so groups may share an MFMA.
  // Codes -> fp16 by one v_and_or_b32 per pair: nibbles (q, q+4) of a dword are the
  // columns (2q, 2q+1); masked in place, nibble pair 0 gives 1024 + n and pair 1 gives
  // 1024 + 16n, so B = (t - 1032) * s' or (t - 1152) * (s'/16), exact.
  uint32_t kmask, kmask_hi, kmagic;  // in registers so that v_and_or_b32 can take them
  asm volatile("v_mov_b32 %0, 0xf000f" : "=v"(kmask));
  asm volatile("v_mov_b32 %0, 0xf000f0" : "=v"(kmask_hi));
  asm volatile("v_mov_b32 %0, 0x64006400" : "=v"(kmagic));
  const f16x2_t k1032 = {(_Float16)1032.0f, (_Float16)1032.0f};
  const f16x2_t k1152 = {(_Float16)1152.0f, (_Float16)1152.0f};
  const uint32_t wrow0 = (uint32_t)(ft0 * kTileBytes + frow * 16);
  auto read_w = [&](const int slot, uint4 (&cw)[2], uint32_t (&sw)[2]) {
    const uint8_t* ws = lds + slot * kStageBytes + kXBytes + wrow0;
#pragma unroll
    for (int f = 0; f < 2; ++f) {
      cw[f] = *reinterpret_cast<const uint4*>(ws + 2 * f * kTileBytes + 1024 * lq);
      sw[f] = *reinterpret_cast<const uint32_t*>(ws + 2 * f * kTileBytes + kCodeBytes + 4 * lq);
    }
  };
  auto scales = [&](const uint32_t (&sw)[2], f16x2_t (&s1)[2], f16x2_t (&s16)[2]) {
#pragma unroll
    for (int f = 0; f < 2; ++f) {
      const float sc = bf16_to_f32(sw[f] & 0xffffu);
      const float v1 = __builtin_amdgcn_ldexpf(sc, -fx[f]), v16 = __builtin_amdgcn_ldexpf(sc, -fx[f] - 4);
      s1[f] = __builtin_bit_cast(f16x2_t, __builtin_amdgcn_cvt_pkrtz(v1, v1));
      s16[f] = __builtin_bit_cast(f16x2_t, __builtin_amdgcn_cvt_pkrtz(v16, v16));
    }
  };
  auto read_a = [&](const int slot, int j, uint4 (&av)[MF]) {
    const uint32_t xc = 16u * (uint32_t)((4 * j + lq) ^ l16);  // chunk 4lq+j of row 16m+l16
    const uint8_t* pa = lds + slot * kStageBytes + (xrow + xc);  // fragments m*4096 apart
#pragma unroll
    for (int m = 0; m < MF; ++m) av[m] = *reinterpret_cast<const uint4*>(pa + m * 4096);
  };
  auto build_b = [&](const uint4 (&cw)[2], int j, const f16x2_t (&s1)[2], const f16x2_t (&s16)[2],
                     uint4 (&b)[2]) {
#pragma unroll
    for (int f = 0; f < 2; ++f) {
      const uint32_t cv = j == 0 ? cw[f].x : j == 1 ? cw[f].y : j == 2 ? cw[f].z : cw[f].w;
      const uint32_t u = cv >> 8;
      const f16x2_t h0 = (__builtin_bit_cast(f16x2_t, and_or(cv, kmask, kmagic)) - k1032) * s1[f];
      const f16x2_t h1 = (__builtin_bit_cast(f16x2_t, and_or(cv, kmask_hi, kmagic)) - k1152) * s16[f];
      const f16x2_t h2 = (__builtin_bit_cast(f16x2_t, and_or(u, kmask, kmagic)) - k1032) * s1[f];
      const f16x2_t h3 = (__builtin_bit_cast(f16x2_t, and_or(u, kmask_hi, kmagic)) - k1152) * s16[f];
      b[f] = make_uint4(__builtin_bit_cast(uint32_t, h0), __builtin_bit_cast(uint32_t, h1),
                        __builtin_bit_cast(uint32_t, h2), __builtin_bit_cast(uint32_t, h3));
    }
  };
  auto mfmas = [&](const uint4 (&av)[MF], const uint4 (&b)[2]) {
#pragma unroll
    for (int f = 0; f < 2; ++f) {
#pragma unroll
      for (int m = 0; m < MF; ++m) acc[m][f] = mfma16h(av[m], b[f], acc[m][f]);
    }
  };
  // Software pipeline.  Region (kt, j) issues the LDS reads of group j+1, runs the MFMAs
  // of group j and builds group j+1's B operands between them (one wave's back-to-back
  // MFMAs leave issue slots that independent VALU fills at little cost); the scheduling
  // group barriers fix that interleave.  Group 3's MFMAs of a step run after the next
  // step's barrier, under that step's first LDS reads and B build.
#define RMOE_INTERLEAVE()                                                   \
  do {                                                                      \
    __builtin_amdgcn_sched_group_barrier(0x100, 12, 0);                     \
    _Pragma("unroll") for (int q_ = 0; q_ < 16; ++q_) {                     \
      __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);                    \
      __builtin_amdgcn_sched_group_barrier(0x002, 2, 0);                    \
    }                                                                       \
  } while (0)
  uint4 avA[MF], avB[MF], bA[2], bB[2], cw[2];
  uint32_t sw[2];
  f16x2_t s1[2], s16[2];
  // Regions 1..3 of the step in `slot` (group 0's operands are in avA / bA).
  auto step_body = [&](const int slot) {
    __builtin_amdgcn_sched_barrier(0);
    read_a(slot, 1, avB);
    mfmas(avA, bA);
    build_b(cw, 1, s1, s16, bB);
    RMOE_INTERLEAVE();
    __builtin_amdgcn_sched_barrier(0);
    read_a(slot, 2, avA);
    mfmas(avB, bB);
    build_b(cw, 2, s1, s16, bA);
    RMOE_INTERLEAVE();
    __builtin_amdgcn_sched_barrier(0);
    read_a(slot, 3, avB);
    mfmas(avA, bA);
    build_b(cw, 3, s1, s16, bB);
    RMOE_INTERLEAVE();
    __builtin_amdgcn_sched_barrier(0);
  };
  // Step kt >= 1 in ring slot `slot` (= kt % 3): barrier, refill, then region 0 runs
  // group 3 of step kt-1 while step kt's first operands arrive and its B is built.
  auto step = [&](int kt, const int slot) {
    // After this barrier every wave is past its reads of step kt-1, so slot (kt+2) % 3
    // is free; step kt's copies have landed.
    ring_wait(kt + 1 < nkt ? per_stage : 0);
    if (kt + 2 < nkt) issue(kt + 2);
    read_w(slot, cw, sw);
    __builtin_amdgcn_sched_barrier(0);
    read_a(slot, 0, avA);
    mfmas(avB, bB);  // group 3 of step kt-1
    scales(sw, s1, s16);
    build_b(cw, 0, s1, s16, bA);
    RMOE_INTERLEAVE();
    __builtin_amdgcn_sched_barrier(0);
    step_body(slot);
  };
  // Step 0: after this barrier every wave is past the correction, so slot 2 is free.
  ring_wait(nkt > 1 ? per_stage : 0);
  if (2 < nkt) issue(2);
  read_w(0, cw, sw);
  __builtin_amdgcn_sched_barrier(0);
  read_a(0, 0, avA);
  scales(sw, s1, s16);
  build_b(cw, 0, s1, s16, bA);
  step_body(0);
  for (int kt = 1; kt < nkt; kt += kStages) {
    step(kt, 1);
    if (kt + 1 < nkt) step(kt + 1, 2);
    if (kt + 2 < nkt) step(kt + 2, 0);
  }
  mfmas(avB, bB);  // group 3 of the last step
#undef RMOE_INTERLEAVE
  scale_rows(row_e, 1);
  // Every wave is past its last ring read: the slots become the output staging.
  asm volatile("s_waitcnt vmcnt(0) lgkmcnt(0)\n\ts_barrier" ::: "memory");

  // Epilogue.  C layout: lane holds rows 16m + 4*lq + i, column l16 of the fragment.
  // Results go through LDS so that global stores are 16-byte rows.
  uint16_t* stage0 = reinterpret_cast<uint16_t*>(lds);
  if (a.mode == 0) {
    // h tile [128 rows][128 units] in slot 0.
    if (a.act == 1) {
#pragma unroll
      for (int m = 0; m < MF; ++m)
#pragma unroll
        for (int i = 0; i < 4; i += 2) {
          const int r = 16 * m + 4 * lq + i;
          const uint32_t gu0 = cvt_bf16x2(acc[m][0][i], acc[m][1][i]);
          const uint32_t gu1 = cvt_bf16x2(acc[m][0][i + 1], acc[m][1][i + 1]);
          const float h0 = swiglu_fast(bf16_to_f32(gu0 & 0xffffu), __uint_as_float(gu0 & 0xffff0000u));
          const float h1 = swiglu_fast(bf16_to_f32(gu1 & 0xffffu), __uint_as_float(gu1 & 0xffff0000u));
          const uint32_t hp = cvt_bf16x2(h0, h1);
          stage0[r * kOutStride + 16 * wave + l16] = (uint16_t)(hp & 0xffffu);
          stage0[(r + 1) * kOutStride + 16 * wave + l16] = (uint16_t)(hp >> 16);
        }
    } else {
      // SiTU-GLU: g and u (bf16) go through slots 1 and 2 and the activation runs in a
      // rolled loop, which keeps the kernel's code small.
      uint16_t* gs = reinterpret_cast<uint16_t*>(lds + kStageBytes);
      uint16_t* us = reinterpret_cast<uint16_t*>(lds + 2 * kStageBytes);
#pragma unroll
      for (int m = 0; m < MF; ++m)
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          const int r = 16 * m + 4 * lq + i;
          const uint32_t gu = cvt_bf16x2(acc[m][0][i], acc[m][1][i]);
          gs[r * kOutStride + 16 * wave + l16] = (uint16_t)(gu & 0xffffu);
          us[r * kOutStride + 16 * wave + l16] = (uint16_t)(gu >> 16);
        }
      __syncthreads();
      for (int idx = tid; idx < kBM * 128; idx += 512) {
        const int o = (idx >> 7) * kOutStride + (idx & 127);
        stage0[o] = (uint16_t)cvt_bf16x2(act_situ(bf16_to_f32(gs[o]), bf16_to_f32(us[o]), a.gb, a.vb), 0.f);
      }
    }
    __syncthreads();
    // Group 4nt + q of h = units 32q..32q+31 of the tile: one (row, group) per thread.
    {
      const int r = tid >> 2, q = tid & 3;
      if (r < nrows && 128 * nt + 32 * q < a.inter) {
        float hs = 0.f;
#pragma unroll
        for (int c = 0; c < 4; ++c) {
          const uint4 v = *reinterpret_cast<const uint4*>(stage0 + r * kOutStride + 32 * q + 8 * c);
          const uint32_t w4[4] = {v.x, v.y, v.z, v.w};
#pragma unroll
          for (int d = 0; d < 4; ++d) hs += bf16_to_f32(w4[d] & 0xffffu) + bf16_to_f32(w4[d] >> 16);
        }
        const int Gpo = ((a.out_ld / 32) + 7) & ~7;
        store_split3_planar(a.out_ssum + (size_t)(row0 + r) * 3 * Gpo + 4 * nt + q, Gpo, hs);
      }
    }
    // 128 rows x 16 chunks of 8 units, stored as the fp16 operand of the down GEMM: the
    // row's 128 units (one K step there) share an exponent (f16_exp_chunk of their
    // largest magnitude; 16 lanes per row).
    const int eso = exp_stride(a.out_ld);
#pragma unroll
    for (int q = 0; q < 4; ++q) {
      const int cid = tid + 512 * q, r = cid >> 4, c = cid & 15;
      const bool live = 128 * nt + 8 * c < a.inter;
      const uint4 v = *reinterpret_cast<const uint4*>(stage0 + r * kOutStride + 8 * c);
      const float mx = row16_max(live ? max_abs_bf16x8(v) : 0.f);
      const int ex = f16_exp_chunk(mx);
      if (r < nrows && live)
        *reinterpret_cast<uint4*>(a.out + (size_t)(row0 + r) * a.out_ld + 128 * nt + 8 * c) =
            make_uint4(bf16x2_to_f16x2(v.x, ex), bf16x2_to_f16x2(v.y, ex), bf16x2_to_f16x2(v.z, ex),
                       bf16x2_to_f16x2(v.w, ex));
      if (r < nrows && c == 0) a.out_exp[(size_t)(row0 + r) * eso + nt] = (int8_t)ex;
    }
  } else {
    // Output columns 0..127 of the 256 in slot 0 (fragment 0), 128..255 in slot 1.
    // (bf16 by the hardware conversion: a NaN may keep its payload here; the combine
    // canonicalises what it passes through.)
#pragma unroll
    for (int m = 0; m < MF; ++m)
#pragma unroll
      for (int f = 0; f < 2; ++f)
#pragma unroll
        for (int i = 0; i < 4; i += 2) {
          const int r = 16 * m + 4 * lq + i;
          uint16_t* st = stage0 + f * (kStageBytes / 2);
          const uint32_t p2 = cvt_bf16x2(acc[m][f][i], acc[m][f][i + 1]);
          st[r * kOutStride + 16 * wave + l16] = (uint16_t)(p2 & 0xffffu);
          st[(r + 1) * kOutStride + 16 * wave + l16] = (uint16_t)(p2 >> 16);
        }
    __syncthreads();
#pragma unroll
    for (int q = 0; q < 8; ++q) {
      const int cid = tid + 512 * q, r = cid >> 5, c = cid & 31;
      const uint16_t* st = stage0 + (c >> 4) * (kStageBytes / 2);
      if (r < nrows) {
        const uint4 v = *reinterpret_cast<const uint4*>(st + r * kOutStride + 8 * (c & 15));
        uint16_t* dst = a.out + (size_t)(row0 + r) * a.out_ld + 256 * nt + 8 * c;
        if (a.out_nt)
          __builtin_nontemporal_store(u32x4v{v.x, v.y, v.z, v.w}, reinterpret_cast<u32x4v*>(dst));
        else
          *reinterpret_cast<uint4*>(dst) = v;
      }
    }
  }
}

// The down GEMM of a bfp16 weight matrix (moe_b2 of a weights-d layer), with MF live
// 16-row fragments.  Same tiling, copies of the activation rows, fragment assignment,
// row exponents and epilogue as gemm_tile's mode 1; what differs:
//   - a weight is m * 2^(e - 133) with an int8 mantissa m and the block's exponent byte e
//     (e raised to 7; one exponent per 8 columns); a lane's 8 K columns of one MFMA are
//     exactly one block.  With the row's largest exponent emax, B = m * 2^(e - emax + 8)
//     is an exact fp16 value (|B| <= 2^15) for every block within 32 binades of emax
//     (smaller blocks, below 2^-32 of the row's largest weight, underflow to 0), and the
//     accumulator is undone by 2^(emax - 141) with the row exponent of the activations;
//   - so there is no correction term: acc = sum_k x[m,k] * B[r,k] is the whole product;
//   - a bfp16 tile is 9 KB: a ring stage (128 activation rows + four weight tiles) is
//     68 KB and the ring is two stages deep (one step's copies land under the previous
//     step's MFMAs).
// B from the bytes: u = m + 128 (m ^ 0x80); v_perm_b32 pairs two u bytes with 0x64 bytes,
// i.e. the fp16 values 1024 + u, and (1024 + u - 1152) * 2^p is m * 2^p, both steps exact.
constexpr int kB16Stage = kXBytes + 4 * kB16TileBytes;  // 69,632
static_assert(2 * kB16Stage <= kGemmLds, "two bfp16 stages fit the ring");

template <int MF>
__device__ __forceinline__ void gemm_tile_b16(const GemmArgs& a, const uint32_t* __restrict__ tl, int mt, int nt,
                                              uint8_t* lds, int* rowidx, int8_t* row_e) {
  const uint32_t te = tl[mt];
  const int e = (int)(te & 511u), row0 = (int)(te >> 9);
  const int rend = group_end(a, e);
  const int nrows = min(kBM, rend - row0);
  const int tid = threadIdx.x, lane = tid & 63, wave = wave_id();
  const int l16 = lane & 15, lq = lane >> 4;
  const int nkt = a.K / kTileCols;
  const uint8_t* W = a.wbase + (size_t)e * a.wstride;
  const uint32_t lds0 = (uint32_t)(uintptr_t)lds;

  if (tid < kBM) {
    const int src = row0 + (tid < nrows ? tid : 0);  // sorted row of the down input
    rowidx[tid] = src;
    row_e[tid] = a.aexp[src];
  }
  __syncthreads();

  const int ft0 = wave >> 2, frow = 16 * (wave & 3) + l16;
  // Weight-row shifts: the lane's row of fragment f is row 64 * (4nt + ft0 + 2f) + frow.
  int emax[2], fx[2];
#pragma unroll
  for (int f = 0; f < 2; ++f) {
    emax[f] = a.rowexp[(size_t)e * a.N_total + 64 * (4 * nt + ft0 + 2 * f) + frow];
    fx[f] = emax[f] - 141;
  }
  // Activation copies as in gemm_tile: copy q = wave + 8i fills LDS rows 4q..4q+3, lane L
  // brings row 4q + L/16 into position L%16, chunk tau((L%16) ^ (row%16)).
  const uint8_t* xg[4];
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const int q = wave + 8 * i, r = 4 * q + (lane >> 4);
    const int pc = (lane & 15) ^ (r & 15), c = ((pc & 3) << 2) | (pc >> 2);
    xg[i] = reinterpret_cast<const uint8_t*>(a.src + (size_t)rowidx[r] * a.K) + 16 * c;
  }
  // Weights: copy v = wave + 8i (v < 36) is 1 KB piece v%9 of tile v/9 (band 4nt + v/9).
  const int n_wcopy = wave < 4 ? 5 : 4;
  auto issue_to = [&](int kt, int slot) {
    const uint32_t sb = lds0 + (uint32_t)(slot * kB16Stage);
#pragma unroll
    for (int i = 0; i < MF / 2; ++i) dma16(xg[i] + (size_t)kt * 256, sb + 1024u * (uint32_t)(wave + 8 * i));
#pragma unroll
    for (int i = 0; i < 5; ++i) {
      if (i < n_wcopy) {
        const int v = wave + 8 * i, t = v / 9, p = v % 9;
        dma16_nt(W + ((size_t)(4 * nt + t) * nkt + kt) * kB16TileBytes + 1024 * p + 16 * lane,
                 sb + (uint32_t)(kXBytes + t * kB16TileBytes + 1024 * p));
      }
    }
  };

  f32x4_t acc[MF][2];
#pragma unroll
  for (int m = 0; m < MF; ++m) {
    acc[m][0] = f32x4_t{0.f, 0.f, 0.f, 0.f};
    acc[m][1] = f32x4_t{0.f, 0.f, 0.f, 0.f};
  }
  const uint32_t xrow = (uint32_t)l16 * 256u;
  const f16x2_t k1152 = {(_Float16)1152.0f, (_Float16)1152.0f};
  const uint32_t wrow0 = (uint32_t)(ft0 * kB16TileBytes + frow * 16);

  issue_to(0, 0);
  for (int kt = 0; kt < nkt; ++kt) {
    const int slot = kt & 1;
    // Step kt's copies have landed in every wave, and every wave is past step kt-1,
    // whose slot takes step kt+1's copies.
    ring_wait(0);
    if (kt + 1 < nkt) issue_to(kt + 1, slot ^ 1);
    const uint8_t* ws = lds + slot * kB16Stage + kXBytes + wrow0;
    uint32_t ew[2];
#pragma unroll
    for (int f = 0; f < 2; ++f) ew[f] = *reinterpret_cast<const uint32_t*>(ws + 2 * f * kB16TileBytes + kB16MantBytes + 4 * lq);
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      // A: chunk 4lq + j of row 16m + l16 (the swizzled position, as in gemm_tile).
      const uint32_t xc = 16u * (uint32_t)((4 * j + lq) ^ l16);
      const uint8_t* pa = lds + slot * kB16Stage + (xrow + xc);
      uint4 av[MF];
#pragma unroll
      for (int m = 0; m < MF; ++m) av[m] = *reinterpret_cast<const uint4*>(pa + m * 4096);
      uint4 b[2];
#pragma unroll
      for (int f = 0; f < 2; ++f) {
        // Columns 32lq + 8j .. +7: mantissa chunk 2lq + j/2, bytes 8(j%2)..; exponent byte j.
        const uint2 mv = *reinterpret_cast<const uint2*>(ws + 2 * f * kB16TileBytes + 1024 * (2 * lq + (j >> 1)) + 8 * (j & 1));
        const int ex = (int)((ew[f] >> (8 * j)) & 0xffu);
        // Blocks of the padding columns (past I; their h columns are zero) may carry
        // exponents above emax: capped, their B stays finite, so 0 * B adds nothing.
        const int pw = min(max(ex, 7) - emax[f] + 8, 8);
        const uint32_t hb = pw >= -14 ? (uint32_t)(pw + 15) << 10 : (pw >= -24 ? 1u << (pw + 24) : 0u);
        const f16x2_t sc = __builtin_bit_cast(f16x2_t, hb | (hb << 16));
        const uint32_t u0 = mv.x ^ 0x80808080u, u1 = mv.y ^ 0x80808080u;
        const f16x2_t h0 = (__builtin_bit_cast(f16x2_t, __builtin_amdgcn_perm(0x64646464u, u0, 0x04010400u)) - k1152) * sc;
        const f16x2_t h1 = (__builtin_bit_cast(f16x2_t, __builtin_amdgcn_perm(0x64646464u, u0, 0x04030402u)) - k1152) * sc;
        const f16x2_t h2 = (__builtin_bit_cast(f16x2_t, __builtin_amdgcn_perm(0x64646464u, u1, 0x04010400u)) - k1152) * sc;
        const f16x2_t h3 = (__builtin_bit_cast(f16x2_t, __builtin_amdgcn_perm(0x64646464u, u1, 0x04030402u)) - k1152) * sc;
        b[f] = make_uint4(__builtin_bit_cast(uint32_t, h0), __builtin_bit_cast(uint32_t, h1),
                          __builtin_bit_cast(uint32_t, h2), __builtin_bit_cast(uint32_t, h3));
      }
#pragma unroll
      for (int f = 0; f < 2; ++f)
#pragma unroll
        for (int m = 0; m < MF; ++m) acc[m][f] = mfma16h(av[m], b[f], acc[m][f]);
    }
  }
  // acc is in units of 2^-(row exponent + fx).
#pragma unroll
  for (int m = 0; m < MF; ++m) {
    const uint32_t e4 = *reinterpret_cast<const uint32_t*>(row_e + 16 * m + 4 * lq);
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const int er = (int)(int8_t)(e4 >> (8 * i));
#pragma unroll
      for (int f = 0; f < 2; ++f) acc[m][f][i] = __builtin_amdgcn_ldexpf(acc[m][f][i], er + fx[f]);
    }
  }
  // Every wave is past its last ring read: slot 0 becomes the output staging.
  asm volatile("s_waitcnt vmcnt(0) lgkmcnt(0)\n\ts_barrier" ::: "memory");
  uint16_t* stage0 = reinterpret_cast<uint16_t*>(lds);
#pragma unroll
  for (int m = 0; m < MF; ++m)
#pragma unroll
    for (int f = 0; f < 2; ++f)
#pragma unroll
      for (int i = 0; i < 4; i += 2) {
        const int r = 16 * m + 4 * lq + i;
        uint16_t* st = stage0 + f * (kStageBytes / 2);
        const uint32_t p2 = cvt_bf16x2(acc[m][f][i], acc[m][f][i + 1]);
        st[r * kOutStride + 16 * wave + l16] = (uint16_t)(p2 & 0xffffu);
        st[(r + 1) * kOutStride + 16 * wave + l16] = (uint16_t)(p2 >> 16);
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

// Grid: per class in kMask (bit c: class c), 8 x ceil(n_tiles * tiles / 8) workgroups;
// 512 threads.  Class c's tile count sits in ntiles[c], its tiles at tiles + c * cap.
// All three classes share one launch (kMask = 7): separate launches leave the chip
// idle in each launch's tail, which costs a mid-size prefill (445 tokens) ~20 %.
template <int kMask, bool kB16>
__global__ __launch_bounds__(512) __attribute__((amdgpu_waves_per_eu(2, 2))) void grouped_gemm_kernel(GemmArgs a, int cap) {
  __shared__ __attribute__((aligned(16))) uint8_t lds[kGemmLds];
  __shared__ int rowidx[kBM];
  __shared__ __attribute__((aligned(16))) int8_t row_e[kBM];  // power-of-two exponent of each tile row
  // XCD-aware order: workgroups are dealt round-robin to the 8 XCDs; each XCD takes a
  // contiguous eighth of every class's tiles (the grid is sized for the worst case, the
  // tile counts are known only here), so m-tiles sharing a weight tile meet in the same
  // L2 and every XCD gets the same share of each class.  Within an XCD the workgroups
  // take the 8-fragment tiles first, then the 4- and 2-fragment ones.
  // m-tile major: the n-tiles of one m-tile (sharing the gathered rows) and consecutive
  // m-tiles of one expert (sharing its weights) run back to back on one XCD.
  const int xcd = blockIdx.x % 8;
  const int n2 = (kMask & 4) ? a.n_tiles * a.ntiles[2] : 0;
  const int n1 = (kMask & 2) ? a.n_tiles * a.ntiles[1] : 0;
  const int n0 = (kMask & 1) ? a.n_tiles * a.ntiles[0] : 0;
  const int p2 = (n2 + 7) / 8, p1 = (n1 + 7) / 8, p0 = (n0 + 7) / 8;
  int j = blockIdx.x / 8, c, per, n;
  if (j < p2) {
    c = 2, per = p2, n = n2;
  } else if ((j -= p2) < p1) {
    c = 1, per = p1, n = n1;
  } else if ((j -= p1) < p0) {
    c = 0, per = p0, n = n0;
  } else {
    return;
  }
  const int lid = xcd * per + j;
  if (lid >= n) return;
  const int mt = lid / a.n_tiles, nt = lid % a.n_tiles;
  const uint32_t* tl = a.tiles + (size_t)c * cap;
  if constexpr (kB16) {
    if (c == 2) gemm_tile_b16<class_fragments(2)>(a, tl, mt, nt, lds, rowidx, row_e);
    else if (c == 1) gemm_tile_b16<class_fragments(1)>(a, tl, mt, nt, lds, rowidx, row_e);
    else gemm_tile_b16<class_fragments(0)>(a, tl, mt, nt, lds, rowidx, row_e);
  } else {
    if constexpr ((kMask & 4) != 0) {
      if (c == 2) gemm_tile<class_fragments(2)>(a, tl, mt, nt, lds, rowidx, row_e);
    }
    if constexpr ((kMask & 3) != 0) {
      if (c == 1)
        gemm_tile<class_fragments(1)>(a, tl, mt, nt, lds, rowidx, row_e);
      else if (c == 0)
        gemm_tile<class_fragments(0)>(a, tl, mt, nt, lds, rowidx, row_e);
    }
  }
}

// ---------------------------------------------------------------- combine --
// out[t] = RTNE(RTNE(sum_{routes by ascending expert} f32(D[inv[t,r]]) * w[t,r]) + D_shared[t])
// (+ x[t] with residual); optionally also the routed and shared rows separately.
// A route whose expert id is outside [0, E) (device ids are not checked on the host; the
// dispatch flags them with error bit 4 and places no row for them) adds nothing, so the
// output does not depend on stale scratch before the error is reported.
__global__ __launch_bounds__(256) void combine_kernel(const uint16_t* __restrict__ D, int H, const int32_t* __restrict__ ids,
                                                      const float* __restrict__ wts, const int32_t* __restrict__ inv,
                                                      int k, int E, int shared_base, const uint16_t* __restrict__ x,
                                                      uint16_t* __restrict__ out, uint16_t* __restrict__ routed,
                                                      uint16_t* __restrict__ shared_out, int has_shared) {
  const int t = blockIdx.x;
  __shared__ int s_pos[16];
  __shared__ float s_w[16];
  // Route q goes to slot rank(q) = its place in ascending expert order.
  if ((int)threadIdx.x < k) {
    const int q = threadIdx.x, eq = ids[(size_t)t * k + q];
    int rank = 0;
    for (int q2 = 0; q2 < k; ++q2) {
      const int e2 = ids[(size_t)t * k + q2];
      rank += (e2 < eq) || (e2 == eq && q2 < q);
    }
    const bool valid = eq >= 0 && eq < E;
    s_pos[rank] = valid ? inv[(size_t)t * k + q] : -1;
    s_w[rank] = wts[(size_t)t * k + q];
  }
  __syncthreads();
  // 8 columns (16 bytes) per thread per pass.
  for (int c0 = 8 * threadIdx.x; c0 < H; c0 += 8 * blockDim.x) {
    float acc[8] = {0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f};
    for (int r = 0; r < k; ++r) {
      if (s_pos[r] < 0) continue;
      // Each row of D is read once here: non-temporal loads.
      const u32x4v dv = __builtin_nontemporal_load(reinterpret_cast<const u32x4v*>(D + (size_t)s_pos[r] * H + c0));
      const uint4 v = make_uint4(dv.x, dv.y, dv.z, dv.w);
      const float w = s_w[r];
      const uint32_t vw[4] = {v.x, v.y, v.z, v.w};
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        acc[2 * i] = __fadd_rn(acc[2 * i], __fmul_rn(bf16_to_f32(vw[i] & 0xffffu), w));
        acc[2 * i + 1] = __fadd_rn(acc[2 * i + 1], __fmul_rn(bf16_to_f32(vw[i] >> 16), w));
      }
    }
    uint32_t o[8];
#pragma unroll
    for (int i = 0; i < 8; ++i) o[i] = f32_to_bf16(acc[i]);
    if (routed)
      *reinterpret_cast<uint4*>(routed + (size_t)t * H + c0) =
          make_uint4(o[0] | (o[1] << 16), o[2] | (o[3] << 16), o[4] | (o[5] << 16), o[6] | (o[7] << 16));
    if (has_shared) {
      const uint4 sv = *reinterpret_cast<const uint4*>(D + (size_t)(shared_base + t) * H + c0);
      if (shared_out) {
        // every NaN leaves as 0x7FC0 (quant/q4nx.py:32-44)
        uint32_t q[4] = {sv.x, sv.y, sv.z, sv.w};
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          if ((q[i] & 0x7fffu) > 0x7f80u) q[i] = (q[i] & 0xffff0000u) | 0x7FC0u;
          if ((q[i] & 0x7fff0000u) > 0x7f800000u) q[i] = (q[i] & 0xffffu) | 0x7FC00000u;
        }
        *reinterpret_cast<uint4*>(shared_out + (size_t)t * H + c0) = make_uint4(q[0], q[1], q[2], q[3]);
      }
      const uint32_t sw[4] = {sv.x, sv.y, sv.z, sv.w};
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        o[2 * i] = f32_to_bf16(__fadd_rn(bf16_to_f32(o[2 * i]), bf16_to_f32(sw[i] & 0xffffu)));
        o[2 * i + 1] = f32_to_bf16(__fadd_rn(bf16_to_f32(o[2 * i + 1]), bf16_to_f32(sw[i] >> 16)));
      }
    }
    if (x) {
      const uint4 xv = *reinterpret_cast<const uint4*>(x + (size_t)t * H + c0);
      const uint32_t xw[4] = {xv.x, xv.y, xv.z, xv.w};
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        o[2 * i] = f32_to_bf16(__fadd_rn(bf16_to_f32(xw[i] & 0xffffu), bf16_to_f32(o[2 * i])));
        o[2 * i + 1] = f32_to_bf16(__fadd_rn(bf16_to_f32(xw[i] >> 16), bf16_to_f32(o[2 * i + 1])));
      }
    }
    if (out)
      *reinterpret_cast<uint4*>(out + (size_t)t * H + c0) =
          make_uint4(o[0] | (o[1] << 16), o[2] | (o[3] << 16), o[4] | (o[5] << 16), o[6] | (o[7] << 16));
  }
}

// One wave per row: the h columns past I are zeroed, with the group sums of the groups
// past I (and the planes' padding) and the chunk exponents past the last live chunk.
__global__ __launch_bounds__(256) void zero_pad_cols_kernel(uint16_t* __restrict__ h, uint16_t* __restrict__ hsum,
                                                            int8_t* __restrict__ hexp, int rows, int I, int Ipad) {
  const size_t r = ((size_t)blockIdx.x * blockDim.x + threadIdx.x) >> 6;
  const int lane = threadIdx.x & 63;
  if (r >= (size_t)rows) return;
  // I % 64 == 0: 4-column pieces of 8 bytes stay aligned.
  for (int c = I + 4 * lane; c < Ipad; c += 256) *reinterpret_cast<uint64_t*>(h + r * Ipad + c) = 0ull;
  // Groups entirely past I; a group straddling I gets its sum from the GEMM epilogue only
  // when I is a multiple of 32 (guaranteed: I % 64 == 0).
  const int Gp = sum_planes_gp(Ipad / 32);
  uint16_t* d = hsum + r * 3 * Gp;
  for (int g = I / 32 + lane; g < Gp; g += 64) d[g] = d[Gp + g] = d[2 * Gp + g] = 0;
  const int es = exp_stride(Ipad);
  for (int c = (I + 127) / 128 + lane; c < es; c += 64) hexp[r * es + c] = 0;
}

// h rows of the shared expert from a given shared_gu [T, 2I] (gate then up):
// RTNE(act(g, u)) as the gate/up epilogue writes them (fp16 operand with one exponent
// per 128-unit chunk, planar group sums, zero past I).  One wave per (token, chunk):
// lane L takes columns 2L, 2L+1 of the chunk; a group's 32 columns are 16 lanes, summed
// by shuffles.
__global__ __launch_bounds__(256) void shared_act_kernel(const uint16_t* __restrict__ gu, int T, int I, int Ipad,
                                                         int act, float gb, float vb, uint16_t* __restrict__ h,
                                                         uint16_t* __restrict__ hsum, int8_t* __restrict__ hexp) {
  const int nch = Ipad / 128, Gp = sum_planes_gp(Ipad / 32), es = exp_stride(Ipad);
  const size_t wid = ((size_t)blockIdx.x * blockDim.x + threadIdx.x) >> 6;
  const int lane = threadIdx.x & 63;
  if (wid >= (size_t)T * nch) return;
  const int t = (int)(wid / nch), ch = (int)(wid % nch);
  const int col = 128 * ch + 2 * lane;
  uint32_t hv = 0u;
  if (col < I) {  // I even: col and col + 1 are both live or both past I
    const uint32_t g2 = *reinterpret_cast<const uint32_t*>(gu + (size_t)t * 2 * I + col);
    const uint32_t u2 = *reinterpret_cast<const uint32_t*>(gu + (size_t)t * 2 * I + I + col);
    const uint32_t o0 = f32_to_bf16(act_apply(act, bf16_to_f32(g2 & 0xffffu), bf16_to_f32(u2 & 0xffffu), gb, vb));
    const uint32_t o1 = f32_to_bf16(act_apply(act, bf16_to_f32(g2 >> 16), bf16_to_f32(u2 >> 16), gb, vb));
    hv = o0 | (o1 << 16);
  }
  const float v0 = bf16_to_f32(hv & 0xffffu), v1 = bf16_to_f32(hv >> 16);
  float sv = v0 + v1;
#pragma unroll
  for (int off = 1; off < 16; off <<= 1) sv += __shfl_xor(sv, off, 64);
  float mx = fmaxf(fabsf(v0), fabsf(v1));
#pragma unroll
  for (int off = 1; off < 64; off <<= 1) mx = fmaxf(mx, __shfl_xor(mx, off, 64));
  const int ex = f16_exp_chunk(mx);
  *reinterpret_cast<uint32_t*>(h + (size_t)t * Ipad + col) = bf16x2_to_f16x2(hv, ex);
  if ((lane & 15) == 0) store_split3_planar(hsum + (size_t)t * 3 * Gp + 4 * ch + (lane >> 4), Gp, sv);
  if (lane == 0) hexp[(size_t)t * es + ch] = (int8_t)ex;
  if (ch == 0)
    for (int c = nch + lane; c < es; c += 64) hexp[(size_t)t * es + c] = 0;
}

// One exponent per h row for the down GEMM: the row's chunks (128 units, one exponent
// each from the gate/up epilogue or shared_act_kernel) are brought to the largest chunk
// exponent; a chunk below it is rescaled by 2^(e_c - e_row) (values more than 2^38
// below the row's largest keep their fp16 grid rounding).  Rows whose chunks agree,
// nearly all, only read their exponents.  Thread per row.
__global__ void h_unify_kernel(uint16_t* __restrict__ h, const int8_t* __restrict__ hexp, int rows, int Ipad,
                               int8_t* __restrict__ hrow) {
  const int r = blockIdx.x * blockDim.x + threadIdx.x;
  if (r >= rows) return;
  const int nch = Ipad / 128, es = exp_stride(Ipad);
  const int8_t* er = hexp + (size_t)r * es;
  int emax = -128, emin = 127;
  for (int c = 0; c < nch; ++c) {
    emax = max(emax, (int)er[c]);
    emin = min(emin, (int)er[c]);
  }
  hrow[r] = (int8_t)emax;
  if (emin == emax) return;
  for (int c = 0; c < nch; ++c) {
    const int d = (int)er[c] - emax;
    if (d == 0) continue;
    uint32_t* hc = reinterpret_cast<uint32_t*>(h + (size_t)r * Ipad + 128 * c);
    for (int i = 0; i < 64; ++i) {
      const f16x2_t v = __builtin_bit_cast(f16x2_t, hc[i]);
      const float lo = __builtin_amdgcn_ldexpf((float)v[0], d), hi = __builtin_amdgcn_ldexpf((float)v[1], d);
      hc[i] = __builtin_bit_cast(uint32_t, __builtin_amdgcn_cvt_pkrtz(lo, hi));
    }
  }
}

}  // namespace

// ------------------------------------------------------------------ launchers --
const char* prefill_shape_error(const RmoeLayer& L, bool device_router) {
  if (L.H % 128 || L.H > 64 * kPrepMaxChunks * 8) return "the grouped prefill needs hidden % 128 == 0 and hidden <= 8192";
  if (L.Ipad % 256) return "the grouped prefill needs the padded intermediate size to be a multiple of 256";
  if (device_router && (L.n_routed % 16 || L.n_routed > 16 * kMaxEFrags))
    return "the device router of the grouped prefill needs n_routed % 16 == 0 and n_routed <= 256";
  return nullptr;
}

hipError_t launch_router_prep(const uint16_t* x, int T, int H, const uint16_t* w, int E, float* logits,
                              uint16_t* xh, int8_t* xe, uint16_t* xsum, int32_t* zero, int nzero, hipStream_t st) {
  if (E % 16 || E > 16 * kMaxEFrags || H % 128 || H / 8 > 64 * kPrepMaxChunks) return hipErrorInvalidValue;
  // Workgroups of up to 64 experts (NFR <= 4), E / 16 NFR of them per (token block, quarter),
  // then the preparation workgroups of four rows.
  const int nfr = E / 16 <= 4 ? E / 16 : (E / 16) % 4 == 0 ? 4 : (E / 16) % 3 == 0 ? 3 : (E / 16) % 2 == 0 ? 2 : 1;
  const int ngroups = (E / 16) / nfr;
  // Large batches: four blocks of 32 tokens per router workgroup, the router rows kept in
  // registers across them (every K slice then has at most 4 steps of 32: H <= 2048);
  // small batches keep one block per workgroup for more workgroups.
  const int ntb = T >= 2048 && H <= 2048 ? 4 : 1;
  const int n_router = (T + ntb * kRouterTok - 1) / (ntb * kRouterTok) * 4 * ngroups;
  const dim3 grid((unsigned)(n_router + (T + 3) / 4)), block(256);
  switch (nfr * 8 + ntb) {
#define RMOE_ROUTER_CASE(n, tb)                                                                                 \
  case n * 8 + tb:                                                                                              \
    hipLaunchKernelGGL((router_prep_kernel<n, tb>), grid, block, 0, st, x, T, H, w, E, logits, n_router, ngroups, xh, \
                       xe, xsum, zero, nzero);                                                                  \
    break;
    RMOE_ROUTER_CASE(1, 1) RMOE_ROUTER_CASE(2, 1) RMOE_ROUTER_CASE(3, 1) RMOE_ROUTER_CASE(4, 1)
    RMOE_ROUTER_CASE(1, 4) RMOE_ROUTER_CASE(2, 4) RMOE_ROUTER_CASE(3, 4) RMOE_ROUTER_CASE(4, 4)
#undef RMOE_ROUTER_CASE
    default:
      return hipErrorInvalidValue;
  }
  return hipGetLastError();
}

hipError_t launch_topk(const float* logits, int T, int E, int k, int score, const float* bias, int renorm,
                       float scaling, int32_t* ids, float* wts, int32_t* counts, hipStream_t st) {
  if (E > 256 || k > 16 || k > 64) return hipErrorInvalidValue;
  static_assert(4 * 16 <= kDispatchChunk, "a workgroup's assignments span at most two chunks");
  const dim3 grid((T + 3) / 4), block(256);
  if (E <= 64)
    hipLaunchKernelGGL(topk_kernel<1>, grid, block, 0, st, logits, T, E, k, score, bias, renorm, scaling, ids, wts,
                       counts);
  else if (E <= 128)
    hipLaunchKernelGGL(topk_kernel<2>, grid, block, 0, st, logits, T, E, k, score, bias, renorm, scaling, ids, wts,
                       counts);
  else
    hipLaunchKernelGGL(topk_kernel<4>, grid, block, 0, st, logits, T, E, k, score, bias, renorm, scaling, ids, wts,
                       counts);
  return hipGetLastError();
}

// The grouped GEMM over the tiles of all three classes in one launch; the grid is sized
// for the worst case (a class-0/1 tile is a group's last, so at most one per group),
// 8 x ceil(tiles / 8) workgroups per class (the XCD mapping deals each class in eighths).
static hipError_t launch_grouped(GemmArgs a, uint32_t* tiles, int* ntiles, int cap, int n_routed, hipStream_t st,
                                 bool b16 = false) {
  a.tiles = tiles;
  a.ntiles = ntiles;
  const int small = min(cap, n_routed + 1);
  const int blocks = 8 * ((a.n_tiles * cap + 7) / 8 + 2 * ((a.n_tiles * small + 7) / 8));
  if (b16)
    hipLaunchKernelGGL((grouped_gemm_kernel<7, true>), dim3(blocks), dim3(512), 0, st, a, cap);
  else
    hipLaunchKernelGGL((grouped_gemm_kernel<7, false>), dim3(blocks), dim3(512), 0, st, a, cap);
  return hipGetLastError();
}

size_t prefill_scratch_bytes(const RmoeLayer& L, int T) {
  const size_t A = (size_t)T * L.top_k, R = A + T;
  const size_t tiles = A / kBM + L.n_routed + T / kBM + 4;
  return R * L.Ipad * 2                                  // h (fp16 operand)
         + R * 3 * sum_planes_gp(L.Ipad / 32) * 2        // h group sums
         + R * exp_stride(L.Ipad) + R                    // h exponents (per chunk, per row)
         + R * L.H * 2                                   // D
         + (size_t)T * L.H * 2                           // xh (fp16 operand)
         + (size_t)T                                     // x exponents
         + (size_t)T * 3 * sum_planes_gp(L.H / 32) * 2   // x group sums
         + (size_t)T * L.n_routed * 16                   // router logits, four K-quarter partials
         + kTileClasses * tiles * 4 + 256 * 12;          // tile table, counts, carve rounding
}

hipError_t launch_moe_prefill(const RmoeLayer& L, const uint16_t* x, int T, const int32_t* ids_in, const float* wts_in,
                              int32_t* ids_out, float* wts_out, const uint16_t* shared_gu, int act, float gb, float vb,
                              bool residual, uint16_t* out, uint16_t* routed, uint16_t* shared_down, uint8_t* scratch,
                              size_t scratch_bytes, RmoeScratch& s, hipStream_t st) {
  const int k = L.top_k, E = L.n_routed;
  const size_t A = (size_t)T * k, R = A + T;
  if (L.n_shared < 1 || prefill_scratch_bytes(L, T) > scratch_bytes) return hipErrorInvalidValue;
  // A weights-d layer's gate/up bundle holds the routed experts only: the shared
  // expert's gate/up comes from the caller.
  if (L.d_layout && !shared_gu) return hipErrorInvalidValue;
  if (L.H % 128 || L.H > 64 * kPrepMaxChunks * 8 || L.Ipad % 256) return hipErrorInvalidValue;
  if (A > s.order_elems || (size_t)((A + 1023) / 1024) * E > s.chunk_elems) return hipErrorInvalidValue;
  uint8_t* p = scratch;
  auto carve = [&](size_t bytes) {
    uint8_t* q = p;
    p += (bytes + 255) / 256 * 256;
    return q;
  };
  uint16_t* h = (uint16_t*)carve(R * L.Ipad * 2);
  const int Gph = sum_planes_gp(L.Ipad / 32), Gpx = sum_planes_gp(L.H / 32);
  uint16_t* hsum = (uint16_t*)carve(R * 3 * Gph * 2);
  int8_t* hexp = (int8_t*)carve(R * exp_stride(L.Ipad));
  int8_t* hrow = (int8_t*)carve(R);
  uint16_t* D = (uint16_t*)carve(R * L.H * 2);
  uint16_t* xh = (uint16_t*)carve((size_t)T * L.H * 2);
  int8_t* xexp = (int8_t*)carve((size_t)T);
  uint16_t* xsum = (uint16_t*)carve((size_t)T * 3 * Gpx * 2);
  float* logits = (float*)carve((size_t)T * E * 16);
  const int tile_cap = (int)(A / kBM + E + T / kBM + 4);
  uint32_t* tiles = (uint32_t*)carve((size_t)kTileClasses * tile_cap * 4);
  int* ntiles = (int*)carve(256);
  hipError_t err;
  const int32_t* ids = ids_in;
  const float* wts = wts_in;
  // With the routing on the device, the router GEMM launch also prepares the activation
  // rows and clears the dispatch chunk counts, which the top-k then adds up (no count
  // kernel).
  const int nchunks = (int)((A + kDispatchChunk - 1) / kDispatchChunk);
  const bool counted = !ids_in && (size_t)nchunks * E <= s.chunk_elems;
  if (!ids_in) {
    err = launch_router_prep(x, T, L.H, L.router_w, E, logits, xh, xexp, xsum, counted ? s.chunk_counts : nullptr,
                             counted ? nchunks * E : 0, st);
    if (err != hipSuccess) return err;
    err = launch_topk(logits, T, E, k, L.score, L.router_bias, L.renorm, L.scaling, ids_out, wts_out,
                      counted ? s.chunk_counts : nullptr, st);
    if (err != hipSuccess) return err;
    ids = ids_out;
    wts = wts_out;
  } else {
    hipLaunchKernelGGL(prep_x_kernel, dim3((unsigned)((T + 3) / 4)), dim3(256), 0, st, x, T, L.H, xh, xexp, xsum);
    if ((err = hipGetLastError()) != hipSuccess) return err;
  }
  // The gate/up GEMM's groups: routed, and the shared expert unless its gate/up is given.
  const int gu_shared_rows = shared_gu ? 0 : T;
  const bool fused_table = E + (gu_shared_rows > 0 ? 1 : 0) <= 256;
  err = fused_table ? launch_dispatch(ids, T, k, E, s.order, s.inv, s.offsets, s, st, tiles, ntiles, tile_cap,
                                      gu_shared_rows, counted)
                    : launch_dispatch(ids, T, k, E, s.order, s.inv, s.offsets, s, st, nullptr, nullptr, 0, 0, counted);
  if (err != hipSuccess) return err;
  if (L.Ipad > L.I) {
    // h columns past I (their group sums and chunk exponents) feed the zero-padded down
    // columns.
    hipLaunchKernelGGL(zero_pad_cols_kernel, dim3((unsigned)((R + 3) / 4)), dim3(256), 0, st, h, hsum, hexp,
                       (int)R, L.I, L.Ipad);
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
  g.src = xh;
  g.aexp = xexp;
  g.order = s.order;
  g.k_routes = k;
  g.n_routed = E;
  g.shared_base = (int)A;
  g.ssum = xsum;
  g.tiles = tiles;
  g.ntiles = ntiles;
  g.offsets = s.offsets;
  g.shared_rows = gu_shared_rows;
  g.out = h;
  g.out_ld = L.Ipad;
  g.out_ssum = hsum;
  g.out_exp = hexp;
  g.act = act;
  g.gb = gb;
  g.vb = vb;
  if (!fused_table) {
    hipLaunchKernelGGL(tile_table_kernel, dim3(1), dim3(512), 0, st, s.offsets, E, (int)A, g.shared_rows, tiles,
                       ntiles, tile_cap);
    if ((err = hipGetLastError()) != hipSuccess) return err;
  }
  if (shared_gu) {
    const size_t n = (size_t)T * (L.Ipad / 128);  // waves, 4 per block
    hipLaunchKernelGGL(shared_act_kernel, dim3((unsigned)((n + 3) / 4)), dim3(256), 0, st, shared_gu, T, L.I,
                       L.Ipad, act, gb, vb, h + A * L.Ipad, hsum + A * 3 * Gph, hexp + A * exp_stride(L.Ipad));
    if ((err = hipGetLastError()) != hipSuccess) return err;
  }
  if ((err = launch_grouped(g, tiles, ntiles, tile_cap, E, st)) != hipSuccess) return err;
  hipLaunchKernelGGL(h_unify_kernel, dim3((unsigned)((R + 255) / 256)), dim3(256), 0, st, h, hexp, (int)R, L.Ipad,
                     hrow);
  if ((err = hipGetLastError()) != hipSuccess) return err;
  // Down: every sorted row (routed + shared), rows of h contiguous.
  if (shared_gu) {
    hipLaunchKernelGGL(tile_table_kernel, dim3(1), dim3(512), 0, st, s.offsets, E, (int)A, T, tiles, ntiles,
                       tile_cap);
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
  d.aexp = hrow;
  d.ssum = hsum;
  d.shared_rows = T;
  d.out = D;
  d.out_ld = L.H;
  d.out_ssum = nullptr;
  d.out_exp = nullptr;
  d.rowexp = L.dn_rowexp;
  // Non-temporal D stores pay off when D is large: 0.948 -> 0.940 ms at 6,700 tokens
  // (247 MB of D), but 0.170 -> 0.171 ms at 445 tokens (16 MB), where the combine finds
  // more of D in the caches.
  d.out_nt = R * (size_t)L.H * 2 > ((size_t)64 << 20) ? 1 : 0;
  if ((err = launch_grouped(d, tiles, ntiles, tile_cap, E, st, L.dn_fmt == RMOE_FMT_BFP16)) != hipSuccess) return err;
  hipLaunchKernelGGL(combine_kernel, dim3(T), dim3(256), 0, st, D, L.H, ids, wts, s.inv, k, E, (int)A,
                     residual ? x : nullptr, out, routed, shared_down, 1);
  return hipGetLastError();
}

}  // namespace rmoe
