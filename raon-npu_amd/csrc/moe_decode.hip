// Router and decode-time (few-token) MoE kernels.
//
// Router: RaonModel._route_token (host/raon.py:1224-1247) -- fp32 logits x.Wr^T,
// sigmoid or softmax scores, selection score + bias, top-k (ties: lower id first),
// renormalisation by (sum + 1e-20), scaling.
//
// Decode MoE (one token): NumpyBackend.moe_experts (host/backend.py:466-510) plus the
// shared expert and combine of RaonModel._moe_token (host/raon.py:1288-1330):
//   per slot (k routed experts, then the shared expert):
//     gate = RTNE(x.Wg^T), up = RTNE(x.Wu^T), h = RTNE(act(gate, up)), d = RTNE(h.Wd^T)
//   routed = RTNE(sum over routed slots in ascending expert id of f32(d)*w)   [fp32, no FMA]
//   out = RTNE(f32(routed) + f32(d_shared))   [+ RTNE(f32(x) + f32(out)) with residual]
// Kernel A streams gate+up of all slots (one launch) and applies the activation in the
// last workgroup of each (slot, 64-unit) band; kernel B streams down of all slots and
// the last workgroup of each 64-row output band performs the ordered combine.
#include <type_traits>

#include "../../include/raon_moe.h"
#include "rmoe_internal.h"

namespace rmoe {
namespace {

// ------------------------------------------------------------------- router --
struct RouteArgs {
  const uint16_t* w;     // [E, H]
  const float* bias;     // [E] or null
  const uint16_t* x;     // [T, H]
  int E, H, k, score, renorm;
  float scaling;
  float* logits;         // [T, E] (scratch or caller)
  int32_t* ids;          // [T, k]
  float* wts;            // [T, k]
  unsigned* counters;    // [T]
};

// numpy's float32 sum of a contiguous array (pairwise_sum for n <= 128): fewer than
// 8 terms are added in order from 0; otherwise eight running sums combined as a tree.
__device__ float np_sum_f32(const float* v, int n) {
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

constexpr int kRouteExpertsPerBlock = 4;  // one wave per expert row
constexpr int kMaxExperts = 256;
constexpr int kMaxTopK = 16;

// Scores and top-k of token t from its logits.  Called by every thread of the block
// (it contains block barriers); the first wave does the work.
__device__ void route_select(const RouteArgs& a, int t) {
  __shared__ float sc[kMaxExperts];
  __shared__ float zz[kMaxExperts];
  __shared__ float chosen[kMaxTopK];
  __shared__ int chosen_id[kMaxTopK];
  __shared__ float total_s;
  const int lane = threadIdx.x & 63;
  const bool w0 = threadIdx.x < 64;
  const float* lg = a.logits + (size_t)t * a.E;
  if (w0) {
    if (a.score == 0) {
      for (int e = lane; e < a.E; e += 64) sc[e] = 1.0f / (1.0f + expf(-ld_dev(&lg[e])));
    } else {
      float m = -__builtin_inff();
      for (int e = lane; e < a.E; e += 64) m = fmaxf(m, ld_dev(&lg[e]));
#pragma unroll
      for (int off = 32; off > 0; off >>= 1) m = fmaxf(m, __shfl_xor(m, off, 64));
      for (int e = lane; e < a.E; e += 64) zz[e] = expf(ld_dev(&lg[e]) - m);
    }
  }
  __syncthreads();
  if (a.score != 0) {
    if (threadIdx.x == 0) total_s = np_sum_f32(zz, a.E);
    __syncthreads();
    if (w0)
      for (int e = lane; e < a.E; e += 64) sc[e] = zz[e] / total_s;
    __syncthreads();
  }
  // Top-k by selection score (score + bias), ties to the lower id.
  for (int r = 0; r < a.k; ++r) {
    if (w0) {
      float best = -__builtin_inff();
      int bid = 0x7fffffff;
      for (int e = lane; e < a.E; e += 64) {
        bool used = false;
        for (int q = 0; q < r; ++q) used = used || (chosen_id[q] == e);
        const float c = a.bias ? __fadd_rn(sc[e], a.bias[e]) : sc[e];
        if (!used && (bid == 0x7fffffff || c > best || (c == best && e < bid))) {
          best = c;
          bid = e;
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
      if (lane == 0) {
        chosen_id[r] = bid;
        chosen[r] = sc[bid];
      }
    }
    __syncthreads();
  }
  if (threadIdx.x == 0) {
    float denom = 1.f;
    if (a.renorm) denom = __fadd_rn(np_sum_f32(chosen, a.k), 1e-20f);
    for (int r = 0; r < a.k; ++r) {
      float v = a.renorm ? chosen[r] / denom : chosen[r];
      v = __fmul_rn(v, a.scaling);
      a.ids[(size_t)t * a.k + r] = chosen_id[r];
      a.wts[(size_t)t * a.k + r] = v;
    }
  }
}

// grid (ceil(E/4), T), block 256: wave w of block b computes logit of expert 4b+w.
__global__ __launch_bounds__(256) void route_kernel(RouteArgs a) {
  __shared__ unsigned last_flag;
  const int t = blockIdx.y;
  const int lane = threadIdx.x & 63, wave = wave_id();
  const int e = blockIdx.x * kRouteExpertsPerBlock + wave;
  if (e < a.E) {
    const uint32_t* wr = reinterpret_cast<const uint32_t*>(a.w + (size_t)e * a.H);
    const uint32_t* xr = reinterpret_cast<const uint32_t*>(a.x + (size_t)t * a.H);
    float acc = 0.f;
    for (int c = lane; c < a.H / 2; c += 64) acc = dot2_bf16(wr[c], xr[c], acc);
    acc = wave_sum(acc);
    if (lane == 0) st_dev(&a.logits[(size_t)t * a.E + e], acc);
  }
  if (!arrive_last(&a.counters[t], gridDim.x, &last_flag)) return;
  route_select(a, t);
}

// ------------------------------------------------------------- decode MoE --
struct DecodeArgs {
  const uint8_t* gu;
  const uint8_t* dn;
  size_t gu_bytes, dn_bytes;
  int H, I, Ipad, n_routed, k, slots;
  const uint16_t* x;
  const int32_t* ids;
  const float* wts;
  int act;
  float gb, vb;
  int residual;
  uint16_t* h;          // [slots, Ipad]
  uint16_t* out;        // [H]
  uint16_t* out_routed; // [H] or null
  // Tokens: blockIdx.y selects the token; its h starts tok_h elements after the previous
  // token's.
  size_t tok_h;
};

// The arguments of token blockIdx.y (a copy with every per-token pointer advanced).
__device__ __forceinline__ DecodeArgs token_args(const DecodeArgs& a0) {
  DecodeArgs a = a0;
  const size_t t = blockIdx.y;
  if (t == 0) return a;
  a.x += t * a.H;
  a.ids += t * a.k;
  a.wts += t * a.k;
  a.h += t * a.tok_h;
  if (a.out) a.out += t * a.H;
  if (a.out_routed) a.out_routed += t * a.H;
  return a;
}

__device__ __forceinline__ int slot_expert(const DecodeArgs& a, int s) {
  if (s >= a.k) return a.n_routed;  // shared expert
  int e = a.ids[s];
  return e < 0 ? 0 : (e >= a.n_routed ? a.n_routed - 1 : e);
}

// One row of a q4nx tile: its 4 code chunks and its scale|min words.
struct Q4Row {
  uint4 c[4], sm;
};
__device__ __forceinline__ void q4_row_load(const uint8_t* tile, int row, Q4Row& r) {
#pragma unroll
  for (int j = 0; j < 4; ++j) r.c[j] = load_stream16(tile + j * 1024 + row * 16);
  r.sm = load_stream16(tile + kCodeBytes + row * 16);
}
__device__ __forceinline__ float q4_row_dot(const Q4Row& r, const uint32_t* xs, const float* ss, float acc) {
  const uint32_t sm[4] = {r.sm.x, r.sm.y, r.sm.z, r.sm.w};
#pragma unroll
  for (int j = 0; j < 4; ++j) acc = group_apply(sm[j], group_dot(r.c[j], xs + j * 16), ss[j], acc);
  return acc;
}

// ------------------------------------------------ row-band decode kernels --
// The per-stage decode in two launches with no workgroup-to-workgroup hand-off:
//   decode_gate_up_band_kernel<R>: one workgroup per (slot, R units of I) over all of K:
//     lane L takes row R-slice row (L % R) of K tile (L / R) + G * (wave + W * i) of the
//     gate and of the up band, G = 64 / R tiles per wave at a time; the lane groups' and
//     waves' sums are added in a fixed order (shuffle tree, then waves in order), then
//     the activation and h (bf16).
//   decode_down_band_kernel<kFmt, R>: one workgroup per R output rows over every slot:
//     a lane group takes one (slot, K tile) item; per slot the tiles' sums are added in K
//     order and rounded to bf16 (the expert output), then the slots are combined in
//     ascending expert order in fp32 (then the shared row and the residual), as the
//     reference's moe_experts does.
constexpr int kBandPad = 4;  // dwords of padding after each K tile's activations in LDS

// Stage nvec vectors of n bf16 (vector v at src + v * stride) into LDS as pairs, one K
// tile (64 dwords) per kBandPad-padded row, vectors one after another; with
// sums != nullptr also the group sums (32 values each, n / 32 per vector).  Every thread
// requests its (up to 4) 16-byte units before it stores any, so the vectors' loads are in
// flight together.
__device__ __forceinline__ void stage_band(const uint16_t* src, size_t stride, int nvec, int n, uint32_t* xs,
                                           float* sums) {
  const int tid = threadIdx.x, nthr = blockDim.x;
  const int units = n / 8, total = nvec * units;  // 16-byte units; units % 16 == 0
  for (int i0 = tid; i0 < total; i0 += 4 * nthr) {
    uint4 v[4];
#pragma unroll
    for (int q = 0; q < 4; ++q) {
      const int i = i0 + q * nthr;
      if (i < total) v[q] = reinterpret_cast<const uint4*>(src + (size_t)(i / units) * stride)[i % units];
    }
#pragma unroll
    for (int q = 0; q < 4; ++q) {
      const int i = i0 + q * nthr;
      if (i >= total) break;
      const int vec = i / units, u = i % units;
      *reinterpret_cast<uint4*>(xs + (size_t)vec * (units / 16) * (64 + kBandPad) + (u >> 4) * (64 + kBandPad) +
                                (u & 15) * 4) = v[q];
      if (sums) {
        float sv = ((bf16_to_f32(v[q].x & 0xffffu) + bf16_to_f32(v[q].x >> 16)) +
                    (bf16_to_f32(v[q].y & 0xffffu) + bf16_to_f32(v[q].y >> 16))) +
                   ((bf16_to_f32(v[q].z & 0xffffu) + bf16_to_f32(v[q].z >> 16)) +
                    (bf16_to_f32(v[q].w & 0xffffu) + bf16_to_f32(v[q].w >> 16)));
        // units 4j..4j+3 (one group) are held by neighbouring lanes (nthr % 64 == 0)
        sv += __shfl_xor(sv, 1, 64);
        sv += __shfl_xor(sv, 2, 64);
        if ((u & 3) == 0) sums[(size_t)vec * (units / 4) + (u >> 2)] = sv;
      }
    }
  }
}

// grid (slots * I / R, tokens), block 64 * W.  Dynamic LDS: x [nkt][64 + pad] pairs,
// group sums [nkt * 4], wave sums [W][2][R].
template <int R>
__global__ __launch_bounds__(1024) void decode_gate_up_band_kernel(DecodeArgs a0) {
  constexpr int G = 64 / R;
  const DecodeArgs a = token_args(a0);
  extern __shared__ __attribute__((aligned(16))) uint32_t band_lds[];
  const int nkt = a.H / kTileCols, tstride = 64 + kBandPad;
  uint32_t* xs = band_lds;
  float* ssum = reinterpret_cast<float*>(band_lds + nkt * tstride);
  float* red = ssum + nkt * 4;
  const int groups = a.I / R;
  const int s = blockIdx.x / groups, u0 = (blockIdx.x % groups) * R;
  const int band = u0 / kTileRows, rsub = u0 % kTileRows;
  const int tid = threadIdx.x, lane = tid & 63, wave = wave_id(), nwaves = blockDim.x >> 6;
  const int g = lane / R, r = lane % R;
  const int e = slot_expert(a, s);
  const uint8_t* W = a.gu + (size_t)e * a.gu_bytes;
  const uint8_t* gate = W + (size_t)band * nkt * kTileBytes + (size_t)(rsub + r) * 16;
  const uint8_t* up = W + (size_t)(a.I / kTileRows + band) * nkt * kTileBytes + (size_t)(rsub + r) * 16;
  const int kt0 = wave * G + g;
  // The first tiles are requested before x is staged: loads complete in order.
  uint4 cg[4], cu[4], sg, su;
  {
    const size_t o = (size_t)(kt0 < nkt ? kt0 : 0) * kTileBytes;
#pragma unroll
    for (int j = 0; j < 4; ++j) cg[j] = load_stream16(gate + o + j * 1024);
    sg = load_stream16(gate + o + kCodeBytes);
#pragma unroll
    for (int j = 0; j < 4; ++j) cu[j] = load_stream16(up + o + j * 1024);
    su = load_stream16(up + o + kCodeBytes);
  }
  stage_band(a.x, 0, 1, a.H, xs, ssum);
  __syncthreads();
  float ag = 0.f, au = 0.f;
  for (int kt = kt0; kt < nkt; kt += nwaves * G) {
    if (kt != kt0) {
      const size_t o = (size_t)kt * kTileBytes;
#pragma unroll
      for (int j = 0; j < 4; ++j) cg[j] = load_stream16(gate + o + j * 1024);
      sg = load_stream16(gate + o + kCodeBytes);
#pragma unroll
      for (int j = 0; j < 4; ++j) cu[j] = load_stream16(up + o + j * 1024);
      su = load_stream16(up + o + kCodeBytes);
    }
    const uint32_t smg[4] = {sg.x, sg.y, sg.z, sg.w}, smu[4] = {su.x, su.y, su.z, su.w};
    const uint32_t* xt = xs + kt * tstride;
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      ag = group_apply(smg[j], group_dot(cg[j], xt + j * 16), ssum[kt * 4 + j], ag);
      au = group_apply(smu[j], group_dot(cu[j], xt + j * 16), ssum[kt * 4 + j], au);
    }
  }
#pragma unroll
  for (int m = R; m < 64; m *= 2) {
    ag += __shfl_xor(ag, m, 64);
    au += __shfl_xor(au, m, 64);
  }
  if (g == 0) {
    red[(wave * 2 + 0) * R + r] = ag;
    red[(wave * 2 + 1) * R + r] = au;
  }
  __syncthreads();
  if (wave == 0 && lane < R) {
    float gs = 0.f, us = 0.f;
    for (int w = 0; w < nwaves; ++w) {
      gs += red[(w * 2 + 0) * R + lane];
      us += red[(w * 2 + 1) * R + lane];
    }
    a.h[(size_t)s * a.Ipad + u0 + lane] =
        (uint16_t)f32_to_bf16(act_apply(a.act, bf16_round(gs), bf16_round(us), a.gb, a.vb));
  }
  // The down input's padding columns [I, Ipad) are zero: the scratch is shared with other
  // layers and launches, and padded weights need not be zero (bfp16 moe_b2).
  if (wave == 0 && u0 + R == a.I)
    for (int c = a.I + lane; c < a.Ipad; c += 64) a.h[(size_t)s * a.Ipad + c] = 0;
}

// grid (H / R, tokens), block 64 * W.  Dynamic LDS: h of every slot [slots][nkt][64 + pad]
// pairs, group sums [slots][nkt * 4] (q4nx), item sums [slots][nkt][R].
template <int kFmt, int R>
__global__ __launch_bounds__(1024) void decode_down_band_kernel(DecodeArgs a0) {
  constexpr int G = 64 / R;
  const DecodeArgs a = token_args(a0);
  extern __shared__ __attribute__((aligned(16))) uint32_t band_lds[];
  const int nkt = a.Ipad / kTileCols, tstride = 64 + kBandPad;
  const int items = a.slots * nkt;
  uint32_t* hs = band_lds;
  float* ssum = reinterpret_cast<float*>(band_lds + items * tstride);
  float* isum = ssum + items * 4;
  const int row0 = blockIdx.x * R, band = row0 / kTileRows, rsub = row0 % kTileRows;
  const int tid = threadIdx.x, lane = tid & 63, wave = wave_id(), nwaves = blockDim.x >> 6;
  const int g = lane / R, r = lane % R;
  constexpr int kTB = kFmt == RMOE_FMT_BFP16 ? kB16TileBytes : kTileBytes;
  using Row = typename std::conditional<kFmt == RMOE_FMT_BFP16, B16Row, Q4Row>::type;
  __shared__ int s_ord[32];
  __shared__ float s_w[32];
  __shared__ int s_n;
  auto tile_of = [&](int it) {
    const int s = it / nkt, kt = it % nkt;
    return a.dn + (size_t)slot_expert(a, s) * a.dn_bytes + ((size_t)band * nkt + kt) * kTB;
  };
  auto load_row = [&](int it, Row& w) {
    if constexpr (kFmt == RMOE_FMT_BFP16)
      b16_row_load(tile_of(it), rsub + r, w);
    else
      q4_row_load(tile_of(it), rsub + r, w);
  };
  // The first item's weight row is requested before h is staged.
  const int it0 = wave * G + g;
  Row wr;
  if (it0 < items) load_row(it0, wr);
  // Combine order: the routed slots by ascending expert id, as a scan for the next
  // larger id from -1 takes them (a repeated id counts once, at its first slot; negative
  // ids are skipped).
  if (wave == 0) {
    const int eq = lane < a.k ? a.ids[lane] : 0x7fffffff;
    const float wq = lane < a.k ? a.wts[lane] : 0.f;
    int rank = 0, n = 0;
    bool first = eq >= 0;
    for (int q2 = 0; q2 < a.k; ++q2) {
      const int e2 = __shfl(eq, q2, 64);
      bool f2 = e2 >= 0;
      for (int q3 = 0; q3 < q2; ++q3) f2 = f2 && __shfl(eq, q3, 64) != e2;
      n += f2 ? 1 : 0;
      if (q2 < lane && e2 == eq) first = false;
      rank += (f2 && e2 < eq) ? 1 : 0;
    }
    if (lane < a.k && first) {
      s_ord[rank] = lane;
      s_w[rank] = wq;
    }
    if (lane == 0) s_n = n;
  }
  stage_band(a.h, a.Ipad, a.slots, a.Ipad, hs, kFmt == RMOE_FMT_BFP16 ? nullptr : ssum);
  __syncthreads();
  for (int it = it0; it < items; it += nwaves * G) {
    if (it != it0) load_row(it, wr);
    float acc;
    if constexpr (kFmt == RMOE_FMT_BFP16)
      acc = b16_row_dot(wr, hs + (size_t)it * tstride, 0.f);
    else
      acc = q4_row_dot(wr, hs + (size_t)it * tstride, ssum + (size_t)it * 4, 0.f);
    isum[(size_t)it * R + r] = acc;
  }
  __syncthreads();
  if (wave != 0 || lane >= R) return;
  const int row = row0 + lane;
  // Expert outputs (bf16-rounded), combined in ascending expert id over the routed slots.
  auto slot_out = [&](int s) {
    float d = 0.f;
    for (int kt = 0; kt < nkt; ++kt) d += isum[(size_t)(s * nkt + kt) * R + lane];
    return bf16_round(d);
  };
  float acc2 = 0.f;
  for (int q = 0; q < s_n; ++q) acc2 = __fadd_rn(acc2, __fmul_rn(slot_out(s_ord[q]), s_w[q]));
  uint32_t o = f32_to_bf16(acc2);
  if (a.out_routed) a.out_routed[row] = (uint16_t)o;
  if (a.slots > a.k) o = f32_to_bf16(__fadd_rn(bf16_to_f32(o), slot_out(a.k)));
  if (a.residual) o = f32_to_bf16(__fadd_rn(bf16_to_f32(a.x[row]), bf16_to_f32(o)));
  if (a.out) a.out[row] = (uint16_t)o;
}

}  // namespace

hipError_t launch_route(const RmoeLayer& L, const uint16_t* x, int T, int32_t* ids, float* wts, float* logits,
                        RmoeScratch& s, hipStream_t st) {
  if (L.n_routed > kMaxExperts || L.top_k > kMaxTopK || L.top_k > L.n_routed) return hipErrorInvalidValue;
  if ((size_t)T > s.n_counters) return hipErrorInvalidValue;
  RouteArgs a{L.router_w, L.router_bias, x, L.n_routed, L.H, L.top_k, L.score, L.renorm, L.scaling,
              logits, ids, wts, s.counters};
  const int bx = (L.n_routed + kRouteExpertsPerBlock - 1) / kRouteExpertsPerBlock;
  hipLaunchKernelGGL(route_kernel, dim3(bx, T), dim3(64 * kRouteExpertsPerBlock), 0, st, a);
  return hipGetLastError();
}

// Launch shape of the row-band decode kernels: 16 units of I per gate/up workgroup (4 K
// tiles per wave at a time), 8 output rows per down workgroup (8 (slot, K tile) items per
// wave at a time); dynamic LDS of each.
constexpr int kRGU = 16, kRDN = 8;
struct BandShape {
  int w1, w2;
  size_t lds1, lds2;
};
static BandShape band_shape(const RmoeLayer& L, int slots) {
  BandShape b;
  const int nkt1 = L.H / kTileCols, nkt2 = L.Ipad / kTileCols, items = slots * nkt2;
  b.w1 = min(16, (nkt1 + (64 / kRGU) - 1) / (64 / kRGU));
  b.w2 = min(16, (items + (64 / kRDN) - 1) / (64 / kRDN));
  b.lds1 = ((size_t)nkt1 * (64 + kBandPad) + (size_t)nkt1 * 4 + (size_t)b.w1 * 2 * kRGU) * 4;
  b.lds2 = ((size_t)items * (64 + kBandPad) + (size_t)items * 4 + (size_t)items * kRDN) * 4;
  return b;
}
hipError_t decode_band_check(const RmoeLayer& L, int slots) {
  const BandShape b = band_shape(L, slots);
  if (L.I % kRGU || L.H % kRDN || b.lds1 > kDecodeMaxLds || b.lds2 > kDecodeMaxLds) return hipErrorInvalidValue;
  return hipSuccess;
}

hipError_t launch_moe_decode(const RmoeLayer& L, const uint16_t* x, const int32_t* ids, const float* wts, int k,
                             bool with_shared, int act, float gb, float vb, bool residual, uint16_t* out,
                             uint16_t* out_routed, RmoeScratch& s, hipStream_t st, int stages, int ntok) {
  const int slots = k + (with_shared ? 1 : 0);
  // A weights-d layer keeps the shared gate/up outside the layer: routed slots only.
  if (with_shared && (L.n_shared < 1 || L.d_layout)) return hipErrorInvalidValue;
  if (ntok < 1) return hipErrorInvalidValue;
  if ((size_t)slots * L.Ipad * ntok > s.h_elems || decode_band_check(L, slots) != hipSuccess)
    return hipErrorInvalidValue;
  DecodeArgs a{};
  a.gu = L.gu;
  a.dn = L.dn;
  a.gu_bytes = L.gu_bytes;
  a.dn_bytes = L.dn_bytes;
  a.H = L.H;
  a.I = L.I;
  a.Ipad = L.Ipad;
  a.n_routed = L.n_routed;
  a.k = k;
  a.slots = slots;
  a.x = x;
  a.ids = ids;
  a.wts = wts;
  a.act = act;
  a.gb = gb;
  a.vb = vb;
  a.residual = residual ? 1 : 0;
  a.h = s.h;
  a.out = out;
  a.out_routed = out_routed;
  a.tok_h = (size_t)slots * L.Ipad;  // token t's h follows token t-1's
  const BandShape b = band_shape(L, slots);
  if (stages & 1) {
    hipLaunchKernelGGL(decode_gate_up_band_kernel<kRGU>, dim3(slots * (L.I / kRGU), ntok), dim3(64 * b.w1), b.lds1,
                       st, a);
    hipError_t e = hipGetLastError();
    if (e != hipSuccess) return e;
  }
  if (stages & 2) {
    if (L.dn_fmt == RMOE_FMT_BFP16)
      hipLaunchKernelGGL((decode_down_band_kernel<RMOE_FMT_BFP16, kRDN>), dim3(L.H / kRDN, ntok), dim3(64 * b.w2),
                         b.lds2, st, a);
    else
      hipLaunchKernelGGL((decode_down_band_kernel<RMOE_FMT_Q4NX, kRDN>), dim3(L.H / kRDN, ntok), dim3(64 * b.w2),
                         b.lds2, st, a);
    return hipGetLastError();
  }
  return hipSuccess;
}

}  // namespace rmoe
