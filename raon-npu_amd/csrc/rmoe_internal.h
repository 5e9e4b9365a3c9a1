// Internal definitions shared by the librmoe HIP sources (gfx950 only).
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include <map>
#include <string>
#include <vector>

// ---------------------------------------------------------------- tile layout --
// The device copy of a q4nx matrix [M, K] is a grid of tiles of 64 rows x 128
// columns (4 groups of 32 columns).  Tile (rt, kt) sits at byte offset
// (rt * (K/128) + kt) * 5120, so a 64-row band is contiguous over K.
// Inside a tile:
//   bytes [0, 4096):   codes, 4 sub-blocks j (group 4*kt + j) of 64 lanes x 16 B;
//                      lane L holds the 32 codes of row 64*rt + L for that group.
//                      In dword d (columns 8d..8d+7 of the group) nibble q (bits
//                      4q..4q+3) holds column 8d + 2q for q < 4 and column
//                      8d + 2(q-4) + 1 for q >= 4, so one shift+mask yields the
//                      bf16 pair for columns (8d+2q, 8d+2q+1).
//   bytes [4096, 5120): per lane L 16 B: for j = 0..3 a dword (scale bf16 | min bf16 << 16)
//                      of row 64*rt + L, group 4*kt + j.
// 5,120 bytes hold 8,192 weights: 5 bits per weight, as in pack_gemv.
namespace rmoe {

constexpr int kTileRows = 64;
constexpr int kTileCols = 128;
constexpr int kTileBytes = 5120;
constexpr int kGroup = 32;
constexpr int kCodeBytes = 4096;

inline size_t matrix_bytes(int M, int K) { return (size_t)M * (size_t)K * 5 / 8; }

// bfp16ebs8 matrices (bfp16_gemv.hip): 9 bits per weight in tiles of 64 rows x 128
// columns, 9,216 bytes each (8,192 B of int8 mantissas, then 1,024 B of exponents).
constexpr int kB16TileBytes = 9216;
constexpr int kB16MantBytes = 8192;
inline size_t matrix_bytes_bfp16(int M, int K) { return (size_t)M * (size_t)K * 9 / 8; }

// ------------------------------------------------------------- device helpers --
// Index of the calling wave in its workgroup as a wave-uniform (scalar) value.  The compiler
// does not infer that threadIdx.x >> 6 is the same in every lane of a wave, so with the plain
// expression every per-wave branch becomes an exec-mask region whose saved masks hold scalar
// registers across it.
__device__ __forceinline__ int wave_id() { return __builtin_amdgcn_readfirstlane((int)(threadIdx.x >> 6)); }

__device__ __forceinline__ float bf16_to_f32(uint32_t b) { return __uint_as_float(b << 16); }

// float32 -> bf16 bits, round to nearest even, every NaN -> 0x7FC0 (quant/q4nx.py:32-44).
__device__ __forceinline__ uint32_t f32_to_bf16(float f) {
  uint32_t u = __float_as_uint(f);
  if ((u & 0x7fffffffu) > 0x7f800000u) return 0x7FC0u;
  return (u + 0x7FFFu + ((u >> 16) & 1u)) >> 16;
}

// Round a float32 onto the bf16 grid (RNE), returned as float32.
__device__ __forceinline__ float bf16_round(float f) { return bf16_to_f32(f32_to_bf16(f)); }

typedef __bf16 bf16x2_t __attribute__((ext_vector_type(2)));
typedef unsigned u32x4_t __attribute__((ext_vector_type(4)));

// 16-byte load of streamed (read-once) weight bytes: non-temporal hint.
__device__ __forceinline__ uint4 load_stream16(const uint8_t* p) {
  const u32x4_t v = __builtin_nontemporal_load(reinterpret_cast<const u32x4_t*>(p));
  return make_uint4(v.x, v.y, v.z, v.w);
}

// acc += a.lo*b.lo + a.hi*b.hi with bf16 pairs packed in dwords (v_dot2c_f32_bf16).
__device__ __forceinline__ float dot2_bf16(uint32_t a, uint32_t b, float acc) {
  return __builtin_amdgcn_fdot2_f32_bf16(__builtin_bit_cast(bf16x2_t, a), __builtin_bit_cast(bf16x2_t, b), acc,
                                         false);
}

// (x & m) | o as one v_and_or_b32.  m and o come from q4_unpack_consts(), in VGPRs: a VOP3
// instruction takes no literal on gfx9, so with the masks as literals the compiler emits a
// v_and_b32 and a v_or_b32 (two VOP2 instructions with literals) instead.
__device__ __forceinline__ uint32_t q4_and_or(uint32_t x, uint32_t m, uint32_t o) {
  uint32_t r;
  asm("v_and_or_b32 %0, %1, %2, %3" : "=v"(r) : "v"(x), "v"(m), "v"(o));
  return r;
}
// The two masks of unpack_codes in VGPRs.  Not volatile: the compiler merges the copies of
// every call and hoists them out of loops.
__device__ __forceinline__ void q4_unpack_consts(uint32_t& mask, uint32_t& one) {
  asm("v_mov_b32 %0, 0x780078" : "=v"(mask));
  asm("v_mov_b32 %0, 0x3f803f80" : "=v"(one));
}

// Codes of one dword -> four bf16 pairs with values 1 + n/16 (n in 0..15, exact).
// Pair q covers nibbles q and q+4, i.e. columns (8d+2q, 8d+2q+1).  Two VALU instructions
// per pair: a shift and a v_and_or_b32 (masked nibble pair | the bf16 pair 1.0, 1.0).
__device__ __forceinline__ void unpack_codes(uint32_t v, uint32_t& p0, uint32_t& p1, uint32_t& p2, uint32_t& p3) {
  uint32_t mask, one;  // 0x00780078, 0x3F803F80
  q4_unpack_consts(mask, one);
  p0 = q4_and_or(v << 3, mask, one);
  p1 = q4_and_or(v >> 1, mask, one);
  p2 = q4_and_or(v >> 5, mask, one);
  p3 = q4_and_or(v >> 9, mask, one);
}

// Partial dot of one group: D' = sum_c (1 + n_c/16) * x_c over 32 columns, x as 16
// bf16-pair dwords.  The group's contribution is then
//   scale*D + min*S = 16*scale*D' + (min - 16*scale)*S,   S = sum_c x_c,
// since D' = S + D/16.
__device__ __forceinline__ float group_dot(const uint4 codes, const uint32_t* __restrict__ xw) {
  float d = 0.f;
  const uint32_t cw[4] = {codes.x, codes.y, codes.z, codes.w};
#pragma unroll
  for (int dd = 0; dd < 4; ++dd) {
    uint32_t p0, p1, p2, p3;
    unpack_codes(cw[dd], p0, p1, p2, p3);
    const uint4 xv = *reinterpret_cast<const uint4*>(xw + 4 * dd);
    d = dot2_bf16(p0, xv.x, d);
    d = dot2_bf16(p1, xv.y, d);
    d = dot2_bf16(p2, xv.z, d);
    d = dot2_bf16(p3, xv.w, d);
  }
  return d;
}

// y += scale*D + min*S for one group given D' (see group_dot) and S.
__device__ __forceinline__ float group_apply(uint32_t sm, float dprime, float s_sum, float y) {
  const float scale = bf16_to_f32(sm & 0xffffu);
  const float mn = bf16_to_f32(sm >> 16);
  const float a = 16.f * scale;
  const float b = mn - a;
  return fmaf(a, dprime, fmaf(b, s_sum, y));
}

// ---- bfp16ebs8 helpers (quant/bfp16.py:71-140, kernels/gemv_bfp16/bfp16_gemv.cc:8-22) ----
// bf16 pair (lo, hi) of two fp32 values whose low 16 bits are zero.
__device__ __forceinline__ uint32_t bf16_pair(float lo, float hi) {
  return __builtin_amdgcn_perm(__float_as_uint(hi), __float_as_uint(lo), 0x07060302u);
}

// The 4 mantissas of a dword -> two exact bf16 pairs (columns (4d, 4d+1), (4d+2, 4d+3)).
// (float)(int8_t) compiles to one sign-extending SDWA convert per byte.
__device__ __forceinline__ void mant_pairs(uint32_t w, uint32_t& p0, uint32_t& p1) {
  p0 = bf16_pair((float)(int8_t)w, (float)(int8_t)(w >> 8));
  p1 = bf16_pair((float)(int8_t)(w >> 16), (float)((int32_t)w >> 24));
}

// Kernel scale of an exponent byte: 2^(max(e, 7) - 133), built as fp32 bits.
__device__ __forceinline__ float exp_scale(uint32_t e) { return __uint_as_float((max(e, 7u) - 6u) << 23); }

// One row of a bfp16 tile (64 rows x 128 columns): 8 mantissa chunks and the exponents.
struct B16Row {
  uint4 mc[8], eq;
};
__device__ __forceinline__ void b16_row_load(const uint8_t* tile, int row, B16Row& r) {
  const uint8_t* p = tile + row * 16;
#pragma unroll
  for (int c = 0; c < 8; ++c) r.mc[c] = load_stream16(p + c * 1024);
  r.eq = load_stream16(p + kB16MantBytes);
}
// A bfp16 tile row against x of its 128 columns (64 bf16-pair dwords): per 8-column
// group d = dot(mantissas, x) from 0, then acc = fma(2^(e-133), d, acc), in column order
// -- the order of the dense bfp16 GEMV.
__device__ __forceinline__ float b16_row_dot(const B16Row& r, const uint32_t* __restrict__ xs, float acc) {
  const uint4* mc = r.mc;
  const uint4 eq = r.eq;
  const uint32_t ew[4] = {eq.x, eq.y, eq.z, eq.w};
#pragma unroll
  for (int c = 0; c < 8; ++c) {
    const uint32_t w[4] = {mc[c].x, mc[c].y, mc[c].z, mc[c].w};
    uint32_t q[8];
#pragma unroll
    for (int d = 0; d < 4; ++d) mant_pairs(w[d], q[2 * d], q[2 * d + 1]);
#pragma unroll
    for (int gg = 0; gg < 2; ++gg) {
      const int g = 2 * c + gg;
      const float s = exp_scale((ew[g >> 2] >> (8 * (g & 3))) & 0xffu);
      const uint4 xv = *reinterpret_cast<const uint4*>(xs + g * 4);
      float d = dot2_bf16(q[4 * gg], xv.x, 0.f);
      d = dot2_bf16(q[4 * gg + 1], xv.y, d);
      d = dot2_bf16(q[4 * gg + 2], xv.z, d);
      d = dot2_bf16(q[4 * gg + 3], xv.w, d);
      acc = fmaf(s, d, acc);
    }
  }
  return acc;
}
// One lane's row (lane = row) of a bfp16 tile: b16_row_load, then b16_row_dot.
__device__ __forceinline__ float b16_tile_accumulate(const uint8_t* tile, int lane, const uint32_t* __restrict__ xs,
                                                     float acc) {
  B16Row r;
  b16_row_load(tile, lane, r);
  return b16_row_dot(r, xs, acc);
}

// Activations, in the operation order of the oracle (fp32).
// SiTU-GLU (host/backend.py:47-62): gb*tanh(g/gb)*sigmoid(g) * vb*tanh(v/vb).
__device__ __forceinline__ float act_situ(float g, float v, float gb, float vb) {
  const float sig = 1.0f / (1.0f + expf(-g));
  const float t1 = gb * tanhf(g / gb) * sig;
  const float t2 = vb * tanhf(v / vb);
  return t1 * t2;
}
// SiLU-GLU (kernels/moe/reference.py:160-171): g*sigmoid(g)*u, overflow-free sigmoid.
__device__ __forceinline__ float act_swiglu(float g, float u) {
  const float e = expf(-fabsf(g));
  const float sig = g >= 0.f ? 1.0f / (1.0f + e) : e / (1.0f + e);
  return (g * sig) * u;
}
__device__ __forceinline__ float act_apply(int act, float g, float u, float gb, float vb) {
  return act == 1 ? act_swiglu(g, u) : act_situ(g, u, gb, vb);
}

// ---- cross-workgroup hand-off inside one kernel ----------------------------------
// An agent-scope fence (__threadfence) is a full L2 write-back + invalidate on this
// multi-XCD part and costs microseconds per workgroup.  Data that one workgroup hands
// to another inside a kernel is therefore written and read with device-scope relaxed
// atomics (global_store/global_load with sc1: written through / read past the XCD's
// L2), ordered by a workgroup-scope fence (s_waitcnt on the issuing wave) and a
// device-scope atomic counter; no L2-wide maintenance is issued.
__device__ __forceinline__ void st_dev(float* p, float v) {
  __hip_atomic_store(p, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ float ld_dev(const float* p) {
  return __hip_atomic_load(const_cast<float*>(p), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ void st_dev_u32(uint32_t* p, uint32_t v) {
  __hip_atomic_store(p, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ uint32_t ld_dev_u32(const uint32_t* p) {
  return __hip_atomic_load(const_cast<uint32_t*>(p), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

// Every thread of the block calls this after its st_dev() writes.  Returns true in
// every thread of the block that is the n-th (last) to arrive at *counter, and then
// resets the counter for the next launch.  Reads of the other blocks' data must use
// ld_dev() after a true return.
__device__ __forceinline__ bool arrive_last(unsigned* counter, unsigned n, unsigned* flag_lds) {
  // The workgroup-scope fence orders the compiler; it does not wait for global stores.
  // Each wave waits for its own sc1 stores to be acknowledged (s_waitcnt vmcnt(0),
  // encoded as 0 = every counter drained) before the block arrives at the counter.
  __builtin_amdgcn_fence(__ATOMIC_RELEASE, "workgroup");
  __builtin_amdgcn_s_waitcnt(0);
  __syncthreads();
  if (threadIdx.x == 0) {
    const unsigned prev = __hip_atomic_fetch_add(counter, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    const unsigned last = (prev == n - 1) ? 1u : 0u;
    if (last) __hip_atomic_store(counter, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    *flag_lds = last;
  }
  __syncthreads();
  const bool last = *flag_lds != 0u;
  __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "workgroup");
  return last;
}

// ---- grouped GEMM tile table ----
// The m-tiles of every group of expert-sorted rows, 128 rows each; a tile is
// group | (row_start << 9).  Tiles are listed by class, the number of 16-row fragments
// that hold rows: class 0 (up to 32 rows: 2 fragments), 1 (up to 64: 4), 2 (8); the
// grouped GEMM runs each class with that many fragments, so a group's short last tile
// does no MFMA work on absent rows.  Class c's tiles sit at tiles[c * cap ...] in group
// order, their count in ntiles[c].
constexpr int kBM = 128;
constexpr int kTileClasses = 3;
__host__ __device__ constexpr int class_fragments(int c) { return c == 0 ? 2 : c == 1 ? 4 : 8; }

// The tile table built by one workgroup of 64 * NW threads; thread e (e < ng) brings group
// e's sorted rows [b, end).  The per-class bases are an exclusive prefix over the groups:
// a 64-lane scan per wave (shuffles), then the wave totals (wsum: kTileClasses x NW ints
// of LDS).  Every thread of the workgroup calls it (it meets the workgroup once).
template <int NW>
__device__ __forceinline__ void tile_table_block(int e, int ng, int b, int end, uint32_t* __restrict__ tiles,
                                                 int* __restrict__ ntiles, int cap, int (*wsum)[NW]) {
  const int lane = e & 63, wave = e >> 6;
  int full = 0, cnt[kTileClasses] = {0, 0, 0};
  if (e < ng) {
    full = (end - b) / kBM;
    const int rem = (end - b) % kBM;
    cnt[2] = full + (rem > 64 ? 1 : 0);
    cnt[1] = (rem > 32 && rem <= 64) ? 1 : 0;
    cnt[0] = (rem > 0 && rem <= 32) ? 1 : 0;
  }
  int incl[kTileClasses];
#pragma unroll
  for (int c = 0; c < kTileClasses; ++c) {
    int x = cnt[c];
#pragma unroll
    for (int d = 1; d < 64; d <<= 1) {
      const int y = __shfl_up(x, d, 64);
      if (lane >= d) x += y;
    }
    incl[c] = x;
    if (lane == 63) wsum[c][wave] = x;
  }
  __syncthreads();
  int base[kTileClasses], total[kTileClasses];
#pragma unroll
  for (int c = 0; c < kTileClasses; ++c) {
    int before = 0, all = 0;
#pragma unroll
    for (int w = 0; w < NW; ++w) {
      const int v = wsum[c][w];
      before += w < wave ? v : 0;
      all += v;
    }
    base[c] = before + incl[c] - cnt[c];
    total[c] = all;
  }
  for (int i = 0; i < cnt[2]; ++i) {
    const int slot = base[2] + i;
    if (slot < cap) tiles[2 * cap + slot] = (uint32_t)e | ((uint32_t)(b + i * kBM) << 9);
  }
#pragma unroll
  for (int c = 0; c < 2; ++c)
    if (cnt[c] && base[c] < cap) tiles[c * cap + base[c]] = (uint32_t)e | ((uint32_t)(b + full * kBM) << 9);
  if (e < kTileClasses) ntiles[e] = min(e == 0 ? total[0] : e == 1 ? total[1] : total[2], cap);
}

// Wave-wide (64 lanes) sum.
__device__ __forceinline__ float wave_sum(float v) {
#pragma unroll
  for (int off = 32; off > 0; off >>= 1) v += __shfl_xor(v, off, 64);
  return v;
}

}  // namespace rmoe

// ------------------------------------------------------------------- context --
struct RmoeMatrix {
  uint8_t* tiles = nullptr;  // device, tile layout of the format
  int M = 0, K = 0;
  int fmt = 0;               // RMOE_FMT_Q4NX or RMOE_FMT_BFP16
  // A view (rmoe_layer_expert_matrix) borrows the tiles of one expert of this layer and
  // owns no memory; -1 for a matrix that owns its tiles.
  int view_of_layer = -1;
};

struct RmoeLayer {
  int H = 0, I = 0, Ipad = 0, n_routed = 0, n_shared = 0, top_k = 0;
  size_t gu_bytes = 0, dn_bytes = 0;  // per expert
  // Layout of the expert weights.  A q4nx layer holds gate/up and down of every expert
  // (n_routed + n_shared) in q4nx.  A weights-d layer (rmoe_layer_create_d) holds the
  // reference's moe_b1 (q4nx gate/up of the n_routed routed experts) and moe_b2 (bfp16
  // down of n_routed + 1 experts, the last one the shared expert's); the shared gate/up
  // is a separate dense matrix.
  bool d_layout = false;
  int gu_experts = 0, dn_experts = 0;
  int dn_fmt = 0;                     // RMOE_FMT_Q4NX or RMOE_FMT_BFP16
  uint8_t* gu = nullptr;              // gu_experts experts, tile layout
  uint8_t* dn = nullptr;              // dn_experts experts, tile layout of dn_fmt
  // bfp16 down only: per expert and row, the largest max(e, 7) over the blocks of the
  // first I columns ([dn_experts][H]; filled on upload).
  uint8_t* dn_rowexp = nullptr;
  uint16_t* router_w = nullptr;  // [n_routed, H] bf16
  float* router_bias = nullptr;  // [n_routed] or null
  bool has_router = false;
  int score = 1, renorm = 1;
  float scaling = 1.f;
};

// Device scratch of a context.  Sized by host entry points (which may allocate);
// "_dev" entry points only check that it is large enough.
struct RmoeScratch {
  void* base = nullptr;
  size_t bytes = 0;
  // decode
  float* part = nullptr;        // fp32 partial sums
  size_t part_floats = 0;
  unsigned* counters = nullptr;  // zero between launches
  size_t n_counters = 0;
  uint16_t* h = nullptr;         // activations [slots, Ipad] / [A, Ipad]
  size_t h_elems = 0;
  int32_t* ids = nullptr;        // routing ids
  float* wts = nullptr;          // routing weights
  float* logits = nullptr;
  size_t route_elems = 0;        // capacity of ids/wts (entries)
  size_t logit_elems = 0;
  int32_t* order = nullptr;      // dispatch
  int32_t* inv = nullptr;
  int32_t* offsets = nullptr;
  int32_t* chunk_counts = nullptr;
  size_t order_elems = 0, offset_elems = 0, chunk_elems = 0;
  int* err = nullptr;            // device error flag
  uint8_t* pf = nullptr;         // prefill working set (h, D, group sums, tiles)
  size_t pf_bytes = 0;
  uint8_t* staging = nullptr;    // upload staging
  size_t staging_bytes = 0;
  int max_tokens = 0;
  // persistent decode stack (moe_decode_stack.hip)
  uint8_t* stack = nullptr;      // per-layer hand-off buffers
  size_t stack_bytes = 0;
  unsigned* stack_cnt = nullptr; // counters; zero between launches
  size_t stack_cnt_n = 0;
};

struct rmoe_ctx {
  int device = 0;
  int n_cu = 0;  // compute units: the grid of the persistent decode kernel
  hipStream_t stream = nullptr;
  std::map<int, RmoeMatrix> mats;
  int next_handle = 1;
  std::map<int, RmoeLayer> layers;
  RmoeScratch s;
  unsigned stack_wait_limit = 0;  // polls before a wait of the decode stack gives up (0: default)
};

// ------------------------------------------------------- kernel launch wrappers --
// Each returns hipSuccess or the launch error; shapes are validated by the caller.
namespace rmoe {

hipError_t launch_relayout_in(const uint8_t* packed, uint8_t* tiles, int M, int K, hipStream_t st);
hipError_t launch_relayout_out(const uint8_t* tiles, uint8_t* packed, int M, int K, hipStream_t st);
// Rows [row0, row0 + M) of a tile matrix Kt wide from a row-major Q4_K tensor [M, K].
hipError_t launch_q4k_to_tiles(const uint8_t* q4k, int M, int K, uint8_t* tiles, int Kt, int row0, hipStream_t st);
hipError_t launch_quantize(const float* w, int M, int K, int ld, int k_valid, uint8_t* tiles, int* err,
                           hipStream_t st);
hipError_t launch_synth_quantize(uint64_t seed, float std, int M, int K, int k_valid, uint8_t* tiles, int* err,
                                 hipStream_t st);

hipError_t launch_linear(const uint8_t* tiles, int M, int K, const uint16_t* x, int T, uint16_t* y, RmoeScratch& s,
                         hipStream_t st);

// bfp16ebs8 (bfp16_gemv.hip).  The GEMV splits K over bfp16_ksplit(M, K) workgroups
// (at most (K/128 + 3)/4, so the q4nx scratch sizing covers it).
hipError_t launch_b16_relayout_in(const uint8_t* packed, uint8_t* tiles, int M, int K, hipStream_t st);
hipError_t launch_b16_relayout_out(const uint8_t* tiles, uint8_t* packed, int M, int K, hipStream_t st);
hipError_t launch_b16_rowexp(const uint8_t* tiles, int M, int K, int k_valid, uint8_t* rowexp, hipStream_t st);
int bfp16_ksplit(int M, int K);
hipError_t launch_linear_bfp16(const uint8_t* tiles, int M, int K, const uint16_t* x, int T, uint16_t* y,
                               RmoeScratch& s, hipStream_t st);

hipError_t launch_route(const RmoeLayer& L, const uint16_t* x, int T, int32_t* ids, float* wts, float* logits,
                        RmoeScratch& s, hipStream_t st);

// Decode MoE: slots = k routed (+ shared); ids/wts on device ([k]); x [H].  With ntok > 1
// the launch covers ntok tokens (x [ntok, H], ids/wts [ntok, k], outputs [ntok, H]), each
// with its own copy of the one-token scratch.
// out_routed (may be null) gets RTNE of the routed sum; out gets the full combine
// (routed + shared, + x when residual).
hipError_t launch_moe_decode(const RmoeLayer& L, const uint16_t* x, const int32_t* ids, const float* wts, int k,
                             bool with_shared, int act, float gb, float vb, bool residual, uint16_t* out,
                             uint16_t* out_routed, RmoeScratch& s, hipStream_t st, int stages = 3, int ntok = 1);

// h[T, Ipad] = RTNE(act(gu[t, :I], gu[t, I:2I])) with zero columns [I, Ipad).
// Assignments per dispatch chunk (per workgroup of the count and scatter kernels); the
// chunk counts are counts[chunk][expert].
constexpr int kDispatchChunk = 1024;
// With counted, counts[][] already hold the chunk counts (the prefill top-k adds them) and
// the count kernel is skipped.
// With tiles != nullptr the first scatter workgroup also writes the grouped GEMM's tile
// table for the routed groups plus, when shared_rows > 0, a shared group of that many rows
// (n_experts + 1 <= 256 groups then).
hipError_t launch_dispatch(const int32_t* ids, int T, int k, int n_experts, int32_t* order, int32_t* inv,
                           int32_t* offsets, RmoeScratch& s, hipStream_t st, uint32_t* tiles = nullptr,
                           int* ntiles = nullptr, int cap = 0, int shared_rows = 0, bool counted = false);

// Prefill MoE (moe_prefill.hip).  With ids_in == nullptr the router runs on the device
// and writes ids_out/wts_out; otherwise ids_in/wts_in are used.  With shared_gu the
// shared expert's gate/up is taken from it, otherwise computed from x.  Any of out /
// routed / shared_down may be null.  scratch: prefill_scratch_bytes(L, T) bytes.
size_t prefill_scratch_bytes(const RmoeLayer& L, int T);
hipError_t launch_moe_prefill(const RmoeLayer& L, const uint16_t* x, int T, const int32_t* ids_in, const float* wts_in,
                              int32_t* ids_out, float* wts_out, const uint16_t* shared_gu, int act, float gb, float vb,
                              bool residual, uint16_t* out, uint16_t* routed, uint16_t* shared_down, uint8_t* scratch,
                              size_t scratch_bytes, RmoeScratch& s, hipStream_t st);
// Shapes the grouped prefill cannot run (a message), or null.  device_router: the
// routing is computed on the device (rmoe_moe_prefill_dev).
const char* prefill_shape_error(const RmoeLayer& L, bool device_router);
// Prefill router: logits as four K-quarter partials [4][T][E] (H % 128 == 0), which
// launch_topk adds in order; the same launch prepares the activation rows of the grouped
// GEMM (xh, xe, xsum; see moe_prefill.hip).
hipError_t launch_router_prep(const uint16_t* x, int T, int H, const uint16_t* w, int E, float* logits,
                              uint16_t* xh, int8_t* xe, uint16_t* xsum, int32_t* zero, int nzero, hipStream_t st);
// counts (may be null): the dispatch chunk counts [chunk][E], zero on entry, to which the
// selected assignments are added.
hipError_t launch_topk(const float* logits, int T, int E, int k, int score, const float* bias, int renorm,
                       float scaling, int32_t* ids, float* wts, int32_t* counts, hipStream_t st);

// Persistent decode of n_layers (<= kMaxStack) layers of one geometry for one token
// (moe_decode_stack.hip).  One workgroup per CU (grid n_cu).  ids_out/wts_out: [n_layers, k]
// or null.  Scratch: stack_scratch_bytes / stack_counter_count; counters must be zero.
constexpr int kMaxStack = 64;
size_t stack_scratch_bytes(const RmoeLayer& L, int n_layers);
size_t stack_counter_count(const RmoeLayer& L, int n_layers);
hipError_t stack_check(const RmoeLayer& L, int n_cu);
hipError_t decode_stack_occupancy(int* blocks_per_cu);
// spin_limit: polls before a wait gives up (0: the default, about two seconds).
hipError_t launch_decode_stack(const RmoeLayer* const* layers, int n_layers, const uint16_t* x, uint16_t* out,
                               bool residual, int act, float gb, float vb, int32_t* ids_out, float* wts_out,
                               RmoeScratch& s, int n_cu, unsigned spin_limit, hipStream_t st);
// The persistent kernel's record of the wait that gave up first (word 1 of its counter
// area; 0 while none has): kAbortValid | phase << 26 | layer << 12 | workgroup.
constexpr unsigned kAbortValid = 0x80000000u;
constexpr unsigned kAbortReady = 1u;  // a layer's input (the previous layer's combined bands)
constexpr unsigned kAbortH = 2u;      // a down unit's h (the gate/up units of its slot)
constexpr unsigned kAbortD = 3u;      // a combiner's d (the down units of its band)
__host__ __device__ constexpr unsigned abort_code(unsigned phase, int layer, int wg) {
  return kAbortValid | (phase & 15u) << 26 | ((unsigned)layer & 0x3fffu) << 12 | ((unsigned)wg & 0xfffu);
}

// Scratch requirements (bytes) for the launch wrappers above.
// The per-stage decode kernels' shape limit: hipSuccess if `slots` slots of layer L fit
// their LDS (kDecodeMaxLds bytes of dynamic LDS per workgroup).
constexpr size_t kDecodeMaxLds = 65536;
hipError_t decode_band_check(const RmoeLayer& L, int slots);

}  // namespace rmoe
