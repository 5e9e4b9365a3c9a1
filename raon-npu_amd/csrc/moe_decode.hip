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
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
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
  float* dout;          // [slots, H] fp32 values of the bf16-rounded expert outputs
  uint16_t* out;        // [H]
  uint16_t* out_routed; // [H] or null
  float* part_gu;       // [slots, I/64, ks1, 2, 64]
  float* part_dn;       // [slots, H/64, ks2, 64]
  unsigned* cnt_gu;     // [slots, I/64]
  unsigned* cnt_dn;     // [slots, H/64]
  unsigned* cnt_rt;     // [H/64]
  int ks1, ks2;
  // Tokens: blockIdx.y selects the token; every per-token buffer above is the first
  // token's and the next token's starts the given number of elements later.
  size_t tok_part_gu, tok_part_dn, tok_cnt_gu, tok_cnt_dn, tok_h, tok_dout;
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
  a.dout += t * a.tok_dout;
  if (a.out) a.out += t * a.H;
  if (a.out_routed) a.out_routed += t * a.H;
  a.part_gu += t * a.tok_part_gu;
  a.part_dn += t * a.tok_part_dn;
  a.cnt_gu += t * a.tok_cnt_gu;
  a.cnt_dn += t * a.tok_cnt_dn;
  a.cnt_rt += t * a.tok_cnt_dn;
  return a;
}

__device__ __forceinline__ int slot_expert(const DecodeArgs& a, int s) {
  if (s >= a.k) return a.n_routed;  // shared expert
  int e = a.ids[s];
  return e < 0 ? 0 : (e >= a.n_routed ? a.n_routed - 1 : e);
}

constexpr int kMaxRange = 8;  // K tiles per workgroup

// Stage nrange*128 bf16 of src (starting at column c0) into xs as pairs, and group sums.
__device__ __forceinline__ void stage_vector(const uint16_t* src, int c0, int nrange, uint32_t* xs, float* ssum) {
  const int tid = threadIdx.x;
  const uint32_t* s32 = reinterpret_cast<const uint32_t*>(src + c0);
  for (int i = tid; i < nrange * 64; i += blockDim.x) xs[i] = s32[i];
  __syncthreads();
  for (int g = tid; g < nrange * 4; g += blockDim.x) {
    float s = 0.f;
    for (int c = 0; c < 16; ++c) {
      const uint32_t v = xs[g * 16 + c];
      s += bf16_to_f32(v & 0xffffu);
      s += bf16_to_f32(v >> 16);
    }
    ssum[g] = s;
  }
  __syncthreads();
}

// Accumulate one tile row band for one lane.
__device__ __forceinline__ float tile_accumulate(const uint8_t* tile, int lane, const uint32_t* xs, const float* ss,
                                                 float acc) {
  uint4 c[4];
#pragma unroll
  for (int j = 0; j < 4; ++j) c[j] = load_stream16(tile + j * 1024 + lane * 16);
  const uint4 smq = load_stream16(tile + kCodeBytes + lane * 16);
  const uint32_t sm[4] = {smq.x, smq.y, smq.z, smq.w};
#pragma unroll
  for (int j = 0; j < 4; ++j) acc = group_apply(sm[j], group_dot(c[j], xs + j * 16), ss[j], acc);
  return acc;
}

// grid (slots*(I/64)*ks1, tokens), block 256.
__global__ __launch_bounds__(256) void decode_gate_up_kernel(DecodeArgs a0) {
  const DecodeArgs a = token_args(a0);
  __shared__ uint32_t xs[kMaxRange * 64];
  __shared__ float ssum[kMaxRange * 4];
  __shared__ float red[4][2][64];
  __shared__ unsigned last_flag;
  const int nj = a.I / 64;
  const int s = blockIdx.x / (nj * a.ks1);
  const int rem = blockIdx.x % (nj * a.ks1);
  const int j = rem / a.ks1, ks = rem % a.ks1;
  const int nkt = a.H / kTileCols;
  const int per = (nkt + a.ks1 - 1) / a.ks1;
  const int kt0 = ks * per;
  const int nrange = max(0, min(per, nkt - kt0));
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6, nwaves = blockDim.x >> 6;
  const int e = slot_expert(a, s);
  const uint8_t* W = a.gu + (size_t)e * a.gu_bytes;

  stage_vector(a.x, kt0 * kTileCols, nrange, xs, ssum);

  float acc[2] = {0.f, 0.f};
  for (int it = wave; it < 2 * nrange; it += nwaves) {
    const int sel = it & 1, kk = it >> 1;
    const int rt = sel ? nj + j : j;  // gate band j, up band I/64 + j
    const uint8_t* tile = W + ((size_t)rt * nkt + kt0 + kk) * kTileBytes;
    acc[sel] = tile_accumulate(tile, lane, xs + kk * 64, ssum + kk * 4, acc[sel]);
  }
  red[wave][0][lane] = acc[0];
  red[wave][1][lane] = acc[1];
  __syncthreads();
  float g = 0.f, u = 0.f;
  if (wave == 0) {
    for (int w = 0; w < nwaves; ++w) {
      g += red[w][0][lane];
      u += red[w][1][lane];
    }
  }
  const size_t band = (size_t)s * nj + j;
  if (a.ks1 > 1) {
    float* part = a.part_gu + (band * a.ks1 + ks) * 128;
    if (wave == 0) {
      st_dev(&part[lane], g);
      st_dev(&part[64 + lane], u);
    }
    if (!arrive_last(&a.cnt_gu[band], (unsigned)a.ks1, &last_flag)) return;
    if (wave == 0) {
      const float* pb = a.part_gu + band * a.ks1 * 128;
      g = 0.f;
      u = 0.f;
      for (int q = 0; q < a.ks1; ++q) {
        g += ld_dev(&pb[q * 128 + lane]);
        u += ld_dev(&pb[q * 128 + 64 + lane]);
      }
    }
  }
  if (wave == 0) {
    const float gb = bf16_round(g), ub = bf16_round(u);
    a.h[(size_t)s * a.Ipad + j * 64 + lane] = (uint16_t)f32_to_bf16(act_apply(a.act, gb, ub, a.gb, a.vb));
    // The down input's padding columns [I, Ipad) are zero: the scratch is shared with
    // other layers and launches, and padded weights need not be zero (bfp16 moe_b2).
    if (j == nj - 1)
      for (int c = a.I + lane; c < a.Ipad; c += 64) a.h[(size_t)s * a.Ipad + c] = 0;
  }
}

// grid slots*(H/64)*ks2, block 64*waves.  kFmt: format of the down weights (q4nx, or
// bfp16 for a weights-d layer whose moe_b2 holds bfp16ebs8 experts).
template <int kFmt>
__global__ __launch_bounds__(256) void decode_down_kernel(DecodeArgs a0) {
  const DecodeArgs a = token_args(a0);
  __shared__ uint32_t xs[kMaxRange * 64];
  __shared__ float ssum[kMaxRange * 4];
  __shared__ float red[4][64];
  __shared__ unsigned last_flag;
  const int nrt = a.H / 64;
  const int s = blockIdx.x / (nrt * a.ks2);
  const int rem = blockIdx.x % (nrt * a.ks2);
  const int rt = rem / a.ks2, ks = rem % a.ks2;
  const int nkt = a.Ipad / kTileCols;
  const int per = (nkt + a.ks2 - 1) / a.ks2;
  const int kt0 = ks * per;
  const int nrange = max(0, min(per, nkt - kt0));
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6, nwaves = blockDim.x >> 6;
  const int e = slot_expert(a, s);
  const uint8_t* W = a.dn + (size_t)e * a.dn_bytes;

  stage_vector(a.h + (size_t)s * a.Ipad, kt0 * kTileCols, nrange, xs, ssum);

  float acc = 0.f;
  for (int it = wave; it < nrange; it += nwaves) {
    if constexpr (kFmt == RMOE_FMT_BFP16) {
      const uint8_t* tile = W + ((size_t)rt * nkt + kt0 + it) * kB16TileBytes;
      acc = b16_tile_accumulate(tile, lane, xs + it * 64, acc);
    } else {
      const uint8_t* tile = W + ((size_t)rt * nkt + kt0 + it) * kTileBytes;
      acc = tile_accumulate(tile, lane, xs + it * 64, ssum + it * 4, acc);
    }
  }
  red[wave][lane] = acc;
  __syncthreads();
  float d = 0.f;
  if (wave == 0)
    for (int w = 0; w < nwaves; ++w) d += red[w][lane];
  const size_t band = (size_t)s * nrt + rt;
  if (a.ks2 > 1) {
    float* part = a.part_dn + (band * a.ks2 + ks) * 64;
    if (wave == 0) st_dev(&part[lane], d);
    if (!arrive_last(&a.cnt_dn[band], (unsigned)a.ks2, &last_flag)) return;
    if (wave == 0) {
      const float* pb = a.part_dn + band * a.ks2 * 64;
      d = 0.f;
      for (int q = 0; q < a.ks2; ++q) d += ld_dev(&pb[q * 64 + lane]);
    }
  }
  const int row = rt * 64 + lane;
  // Expert outputs are handed to the combining workgroup as the fp32 value of the
  // bf16-rounded result.
  if (wave == 0) st_dev(&a.dout[(size_t)s * a.H + row], bf16_round(d));
  // Second level: the last slot to finish this 64-row band combines all slots.
  if (!arrive_last(&a.cnt_rt[rt], (unsigned)a.slots, &last_flag)) return;
  if (wave == 0) {
    // Ascending expert id over the routed slots (ids are distinct per token).
    float acc2 = 0.f;
    int prev = -1;
    for (int r = 0; r < a.k; ++r) {
      int best = 0x7fffffff, bs = -1;
      for (int q = 0; q < a.k; ++q) {
        const int eq = a.ids[q];
        if (eq > prev && eq < best) {
          best = eq;
          bs = q;
        }
      }
      if (bs < 0) break;
      prev = best;
      const float dv = ld_dev(&a.dout[(size_t)bs * a.H + row]);
      acc2 = __fadd_rn(acc2, __fmul_rn(dv, a.wts[bs]));
    }
    uint32_t o = f32_to_bf16(acc2);
    if (a.out_routed) a.out_routed[row] = (uint16_t)o;
    if (a.slots > a.k) o = f32_to_bf16(__fadd_rn(bf16_to_f32(o), ld_dev(&a.dout[(size_t)a.k * a.H + row])));
    if (a.residual) o = f32_to_bf16(__fadd_rn(bf16_to_f32(a.x[row]), bf16_to_f32(o)));
    if (a.out) a.out[row] = (uint16_t)o;
  }
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

static void decode_splits(const RmoeLayer& L, int& ks1, int& ks2) {
  const int nkt1 = L.H / kTileCols, nkt2 = L.Ipad / kTileCols;
  ks1 = (nkt1 + 1) / 2;           // two K tiles per band-pair per workgroup -> 4 waves
  if (ks1 < 1) ks1 = 1;
  ks2 = (nkt2 + 1) / 2;
  if (ks2 < 1) ks2 = 1;
  while ((nkt1 + ks1 - 1) / ks1 > kMaxRange) ++ks1;
  while ((nkt2 + ks2 - 1) / ks2 > kMaxRange) ++ks2;
}

size_t decode_scratch_floats(const RmoeLayer& L) {
  int ks1, ks2;
  decode_splits(L, ks1, ks2);
  const size_t slots = (size_t)L.top_k + L.n_shared;
  return slots * (L.I / 64) * ks1 * 128 + slots * (L.H / 64) * ks2 * 64;
}

size_t decode_scratch_counters(const RmoeLayer& L) {
  const size_t slots = (size_t)L.top_k + L.n_shared;
  return slots * (L.I / 64) + slots * (L.H / 64) + (L.H / 64);
}

hipError_t launch_moe_decode(const RmoeLayer& L, const uint16_t* x, const int32_t* ids, const float* wts, int k,
                             bool with_shared, int act, float gb, float vb, bool residual, uint16_t* out,
                             uint16_t* out_routed, RmoeScratch& s, hipStream_t st, int stages, int ntok) {
  int ks1, ks2;
  decode_splits(L, ks1, ks2);
  const int slots = k + (with_shared ? 1 : 0);
  // A weights-d layer keeps the shared gate/up outside the layer: routed slots only.
  if (with_shared && (L.n_shared < 1 || L.d_layout)) return hipErrorInvalidValue;
  if (ntok < 1) return hipErrorInvalidValue;
  const size_t nf = (size_t)slots * (L.I / 64) * ks1 * 128 + (size_t)slots * (L.H / 64) * ks2 * 64;
  const size_t nc = (size_t)slots * (L.I / 64) + (size_t)slots * (L.H / 64) + (L.H / 64);
  if (nf * ntok > s.part_floats || nc * ntok > s.n_counters || (size_t)slots * L.Ipad * ntok > s.h_elems ||
      (size_t)slots * L.H * ntok > s.dout_elems)
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
  a.dout = s.dout;
  a.out = out;
  a.out_routed = out_routed;
  a.part_gu = s.part;
  a.part_dn = s.part + (size_t)slots * (L.I / 64) * ks1 * 128;
  a.cnt_gu = s.counters;
  a.cnt_dn = s.counters + (size_t)slots * (L.I / 64);
  a.cnt_rt = a.cnt_dn + (size_t)slots * (L.H / 64);
  a.ks1 = ks1;
  a.ks2 = ks2;
  // Token t's scratch: its partials and counters follow token t-1's (the layout of one
  // token repeated), its h and expert outputs likewise.
  a.tok_part_gu = nf;
  a.tok_part_dn = nf;
  a.tok_cnt_gu = nc;
  a.tok_cnt_dn = nc;
  a.tok_h = (size_t)slots * L.Ipad;
  a.tok_dout = (size_t)slots * L.H;
  const int nkt1 = L.H / kTileCols, nkt2 = L.Ipad / kTileCols;
  const int per1 = (nkt1 + ks1 - 1) / ks1, per2 = (nkt2 + ks2 - 1) / ks2;
  const int w1 = min(4, 2 * per1), w2 = min(4, per2);
  if (stages & 1) {
    hipLaunchKernelGGL(decode_gate_up_kernel, dim3(slots * (L.I / 64) * ks1, ntok), dim3(64 * w1), 0, st, a);
    hipError_t e = hipGetLastError();
    if (e != hipSuccess) return e;
  }
  if (stages & 2) {
    if (L.dn_fmt == RMOE_FMT_BFP16)
      hipLaunchKernelGGL(decode_down_kernel<RMOE_FMT_BFP16>, dim3(slots * (L.H / 64) * ks2, ntok), dim3(64 * w2), 0,
                         st, a);
    else
      hipLaunchKernelGGL(decode_down_kernel<RMOE_FMT_Q4NX>, dim3(slots * (L.H / 64) * ks2, ntok), dim3(64 * w2), 0,
                         st, a);
    return hipGetLastError();
  }
  return hipSuccess;
}

}  // namespace rmoe
