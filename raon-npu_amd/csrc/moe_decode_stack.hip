// Persistent decode of a stack of MoE layers for one token in one launch.
//
// Per layer l (RaonModel._moe_token, host/raon.py:1288-1330, with the router of
// RaonModel._route_token, host/raon.py:1224-1247, on the device, and the expert loop of
// NumpyBackend.moe_experts, host/backend.py:466-510):
//   logits = x_l . Wr^T; scores (sigmoid or softmax); top-k by score (+ bias), ties to
//   the lower expert id; weights renormalised by (sum + 1e-20) and scaled
//   per slot s (k routed experts, then the shared expert):
//     g = RTNE(x_l . Wg^T), u = RTNE(x_l . Wu^T), h = RTNE(act(g, u)), d = RTNE(h . Wd^T)
//   routed = RTNE(sum over the routed slots in ascending expert id of f32(d) * w)
//   out = RTNE(f32(routed) + f32(d_shared));  x_{l+1} = residual ? RTNE(x_l + out) : out
//
// One workgroup per CU stays resident for the whole stack.  The work of a layer is cut
// into units that are the same for every layer:
//   GU unit (slot s, half band hb): the 32 gate rows 32hb..32hb+31 and the matching 32 up
//     rows over all of K (lanes 0..31 of each wave read gate rows, lanes 32..63 up rows;
//     wave w streams K tiles w, w + 8, ...).  The workgroup sums its waves, applies the
//     activation and publishes h of its 32 columns.
//   DN unit (slot s, output band b of 64 rows): all K tiles of the band; waves 1..7
//     copy them into LDS, and all eight waves take their half tiles (64 columns each,
//     with the h of those columns).
// Hand-offs between workgroups (per layer):
//   h         tagged words (below): every wave polls the words of its own columns
//   d         tagged words: the combiner of band b (the workgroup whose first DN unit is
//             slot 0 of band b) polls the band's words of every slot, combines the band,
//             writes x_{l+1}[band] and the band's share of the router logits of layer l+1
//                                                                    -> ready[l+1]
//   ready     counter: all bands of x_l and of its partial router logits are written
// Every workgroup computes the top-k of a layer itself from the partial logits (the
// same reads in the same order give the same routing everywhere), and loads the weight
// tiles of all its units as soon as the routing is known, before it waits for anything
// else in that layer: the HBM stream of a layer is issued at once.
// Results do not depend on the arrival order: every sum over waves, bands or slots is
// taken in a fixed order.
#include "rmoe_internal.h"

#include <type_traits>

namespace rmoe {
namespace {

constexpr int kThreads = 512;
constexpr int kWaves = kThreads / 64;
constexpr int kMaxH = 4096;
constexpr int kMaxE = 256;
constexpr int kMaxSlots = 17;
constexpr int kMaxDnPos = 4;      // DN tiles per DN wave (waves 1..7, both units): Ipad <= 1792
constexpr int kMaxDnUnits = 2;    // DN units per workgroup and layer (prefetched)
static_assert(kMaxDnUnits == 2, "the unit indices are read as one int4");
constexpr int kLRow = 4096;       // floats of partial logits copied into LDS at a time
// LDS rows of partial logits are Ep + kLPad floats apart: band b starts at bank 16 b mod 64,
// so the four bands that one instruction reads (see the sum below) fall in four distinct
// bank groups.
constexpr int kLPad = 16;
constexpr int kLRowLds = 4608;    // LDS floats for one pass (32 rows of 128 + 16)
constexpr unsigned kSpinLimit = 1u << 21;

// Per-layer timeline of the stack, in the timeline build only (RMOE_DECODE_TIMELINE; built
// and read by bench.py --build-timeline / --timeline): one wave of each workgroup stores the device clock
// (s_memrealtime, 100 MHz) at fixed points of every layer.  Other builds compile the
// stamps to nothing.
constexpr int kTimelineLayers = 48, kTimelineGroups = 256, kTimelineEvents = 16;
// The stamps of a layer go to LDS; wave 0 copies them to memory at the top of the next
// layer (RMOE_STAMP_FLUSH), so that no store of the timeline sits before a barrier of the
// layer it measures (a barrier also waits for the workgroup's stores in flight).
#ifdef RMOE_DECODE_TIMELINE
__device__ unsigned long long g_stack_timeline[kTimelineLayers][kTimelineGroups][kTimelineEvents];
__shared__ unsigned long long g_tl_lds[kTimelineEvents];
#define RMOE_STAMP(l, g, ev, who)                                              \
  do {                                                                          \
    if (threadIdx.x == (who)) g_tl_lds[ev] = __builtin_amdgcn_s_memrealtime(); \
  } while (0)
#define RMOE_STAMP_FLUSH(l, g)                                                                          \
  do {                                                                                                   \
    if (threadIdx.x < kTimelineEvents) {                                                                 \
      if ((l) >= 0 && (l) < kTimelineLayers && (g) < kTimelineGroups)                                    \
        g_stack_timeline[l][g][threadIdx.x] = g_tl_lds[threadIdx.x];                                     \
      g_tl_lds[threadIdx.x] = 0ull;                                                                      \
    }                                                                                                    \
  } while (0)
#else
#define RMOE_STAMP(l, g, ev, who) \
  do {                            \
  } while (0)
#define RMOE_STAMP_FLUSH(l, g) \
  do {                         \
  } while (0)
#endif
// Stamp points (event index): ready seen 0, x and partial logits summed 1, routing done 2,
// gate/up unit done 3, h received 4, down tiles in LDS 5, wave 1's down dot products 6,
// down partials summed 7, d stored 8, combiner holds every d 9, x band stored 10, ready
// published 11, first pass of partial logits in LDS 12, selection keys written 13, wave 0's
// first gate/up tile dot product 14, gate/up waves summed (barrier) 15.

struct StackArgs {
  int L, H, I, Ipad, E, k, S, score, renorm, act, residual;
  float scaling, gb, vb;
  size_t gu_bytes, dn_bytes;
  int nb1, nb2, nkt1, nkt2, nhb, n_gu, n_dn;
  int Ep;      // n_routed rounded up to 32: row stride of the partial router logits
  int gu_pre;  // 1: a workgroup whose GU unit is in the shared slot copies its tiles into LDS early
  const uint16_t* x0;
  uint16_t* out;
  int32_t* ids_out;  // [L, k] or null
  float* wts_out;    // [L, k] or null
  uint8_t* scratch;  // per layer: layer_bytes
  size_t layer_bytes, off_lpart, off_h, off_dout;
  unsigned* cnt;     // per layer cnt_stride counters, then exit, abort
  int cnt_stride;
  unsigned spin_limit;  // polls before a wait gives up (about a microsecond each)
  int* err;
  const uint8_t* gu[kMaxStack];
  const uint8_t* dn[kMaxStack];
  const uint16_t* rw[kMaxStack];
  const float* rb[kMaxStack];
};

struct TileRegs {
  uint4 c[4];
  uint4 sm;
};

__device__ __forceinline__ void load_tile(TileRegs& r, const uint8_t* tile, int lane) {
#pragma unroll
  for (int j = 0; j < 4; ++j) r.c[j] = load_stream16(tile + j * 1024 + lane * 16);
  r.sm = load_stream16(tile + kCodeBytes + lane * 16);
}

// load_tile of `tile` when valid, otherwise five loads of the same 16 bytes at `dummy`
// (no offsets: dummy only has to hold 16 bytes), so the load count does not depend on
// validity.
__device__ __forceinline__ void load_tile_or(TileRegs& r, bool valid, const uint8_t* tile, const uint8_t* dummy,
                                             int lane) {
  const uint8_t* base = valid ? tile + lane * 16 : dummy;
  const int step = valid ? 1024 : 0;
#pragma unroll
  for (int j = 0; j < 4; ++j) r.c[j] = load_stream16(base + j * step);
  r.sm = load_stream16(base + 4 * step);
}

// Five 16-byte pieces at p + 1 KB * j (a lane's share of one tile), or five loads of
// `dummy` when not valid (the same load count on every path).
__device__ __forceinline__ void load_rows(TileRegs& r, bool valid, const uint8_t* p, const uint8_t* dummy) {
  const uint8_t* base = valid ? p : dummy;
  const int step = valid ? 1024 : 0;
#pragma unroll
  for (int j = 0; j < 4; ++j) r.c[j] = load_stream16(base + j * step);
  r.sm = load_stream16(base + 4 * step);
}

typedef __attribute__((address_space(3))) void* lds_void_ptr;
typedef __attribute__((address_space(1))) void* global_void_ptr;

// Direct global -> LDS copy of one tile by one wave (five 1 KB pieces; lane L moves
// bytes [16L, 16L+16) of each piece).  Invalid tiles copy 16 bytes of `dummy` into the
// 1 KB `sink` instead, so the number of loads does not depend on validity.  The data is
// in LDS once the wave's vmcnt has drained.  The copies carry the non-temporal hint: each
// DN tile is read once per layer.
__device__ __forceinline__ void dma_tile(bool valid, const uint8_t* tile, const uint8_t* dummy, uint8_t* lds_tile,
                                         uint8_t* sink, int lane) {
#pragma unroll
  for (int j = 0; j < 5; ++j) {
    const uint8_t* src = valid ? tile + j * 1024 + lane * 16 : dummy;
    uint8_t* dst = valid ? lds_tile + j * 1024 : sink;
    __builtin_amdgcn_global_load_lds((global_void_ptr)src, (lds_void_ptr)dst, 16, 0, 2 /* nt */);
  }
}

// tile_dot of a tile held in LDS (same byte layout as in HBM).
__device__ __forceinline__ float tile_dot_lds(const uint8_t* t, int lane, const uint32_t* xw, const float* ss,
                                              float acc) {
  TileRegs r;
#pragma unroll
  for (int j = 0; j < 4; ++j) r.c[j] = *reinterpret_cast<const uint4*>(t + j * 1024 + lane * 16);
  r.sm = *reinterpret_cast<const uint4*>(t + kCodeBytes + lane * 16);
  const uint32_t sm[4] = {r.sm.x, r.sm.y, r.sm.z, r.sm.w};
#pragma unroll
  for (int j = 0; j < 4; ++j) acc = group_apply(sm[j], group_dot(r.c[j], xw + j * 16), ss[j], acc);
  return acc;
}

__device__ __forceinline__ float tile_dot(const TileRegs& r, const uint32_t* xw, const float* ss, float acc) {
  const uint32_t sm[4] = {r.sm.x, r.sm.y, r.sm.z, r.sm.w};
#pragma unroll
  for (int j = 0; j < 4; ++j) acc = group_apply(sm[j], group_dot(r.c[j], xw + j * 16), ss[j], acc);
  return acc;
}

// Counters of layer l: kReadyCopies copies of ready.
// Every counter sits on its own 256-byte line: atomics and polls on one line are served
// one at a time at the memory side, and a layer's counters see hundreds of them.
constexpr int kCntPad = 64;  // uint32 per counter line
// Line 0 of the counter area holds the launch counter (at a fixed place: launches of
// different depths share the area); the counters of layer l follow from line 1.
__device__ __forceinline__ unsigned* cnt_at(const StackArgs& a, int l, int i) {
  return a.cnt + (1 + (size_t)l * a.cnt_stride + i) * kCntPad;
}
// `ready` of a layer is kept in kReadyCopies copies: a band publishes to every copy and
// workgroup g polls copy g % kReadyCopies, so 32 rather than 256 workgroups poll a line.
constexpr int kReadyCopies = 32;
__device__ __forceinline__ void publish_ready(const StackArgs& a, int l) {
  for (int c = 0; c < kReadyCopies; ++c)
    __hip_atomic_fetch_add(cnt_at(a, l, c), 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ unsigned* exit_cnt(const StackArgs& a) { return cnt_at(a, a.L, 0); }
__device__ __forceinline__ unsigned* abort_flag(const StackArgs& a) { return cnt_at(a, a.L, 1); }
// Launch counter: read by every workgroup at the start, advanced by the last one out.
__device__ __forceinline__ unsigned* epoch_cnt(const StackArgs& a) { return a.cnt; }
// Which wait gave up first (0 while none has): kAbortValid | phase << 26 | layer << 12 |
// workgroup, in word 1 of the launch counter's line (a fixed place, whatever the depth).
__device__ __forceinline__ unsigned* abort_info(const StackArgs& a) { return a.cnt + 1; }

// A bounded wait that ran out of polls: raise the abort flag (every other wait of the
// grid sees it within 64 polls and its workgroup leaves), set error bit 8 and record the
// first giver-up's wait (phase), layer and workgroup.
__device__ __forceinline__ void give_up(const StackArgs& a, unsigned phase, int l, int g) {
  st_dev_u32(abort_flag(a), 1u);
  __hip_atomic_fetch_or(a.err, 8, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  unsigned expected = 0u;
  __hip_atomic_compare_exchange_strong(abort_info(a), &expected, abort_code(phase, l, g), __ATOMIC_RELAXED,
                                       __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

// Tagged hand-off words: 32 bits of data and the launch's tag (2 * epoch + 1: odd, so
// never the zero of fresh memory) in one 64-bit device-scope store; a reader polls each
// word until it carries this launch's tag.  A 64-bit access is single-copy atomic, so a
// word with the right tag holds this launch's data, and no counter or store
// acknowledgement is needed.  Each word is written once per launch (a region per layer).
__device__ __forceinline__ void st_dev_u64(uint64_t* p, uint64_t v) {
  __hip_atomic_store(p, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ uint64_t ld_dev_u64(const uint64_t* p) {
  return __hip_atomic_load(const_cast<uint64_t*>(p), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

// Hand-off protocol.  Data handed to other workgroups is stored with device-scope
// stores (st_dev); the storing wave waits until its stores are acknowledged
// (s_waitcnt 0 drains every counter of that wave) before the arrival is counted, and
// readers load it (ld_hand_u64) after they have seen the count with a device-scope poll.  A wave's wait also
// covers its own earlier loads, so the waves that publish (wave 0, and every wave for
// the router logits) never hold long-latency weight prefetches.

// Reads of hand-off data.  Every hand-off buffer is written exactly once per launch (a
// separate region per layer), by device-scope stores that go through to memory, and is
// read only after the counter that covers it is complete; no L2 holds a copy of it from
// before the write (kernel launches start with invalidated L2s, and nothing reads a
// region of this launch before its counter is complete).  So ordinary cached loads see
// the stored values, and each XCD's L2 fetches a line once for all 32 workgroups on it
// instead of every workgroup going to the memory side.  The compiler may not hoist
// them above the wait: wait_geq ends with a barrier and an acquire fence.
// Every hand-off cache line has exactly one writer, so even an L2 that allocated a line
// on its own workgroup's store holds exactly what was stored.
__device__ __forceinline__ uint64_t ld_hand_u64(const void* p) { return *reinterpret_cast<const uint64_t*>(p); }
__device__ __forceinline__ float ld_hand_f32(const float* p) { return *p; }

// Block-wide: every wave waits for its own stores, then thread 0 counts one arrival.
// Returns true in every thread for the n-th arrival.
__device__ __forceinline__ bool block_arrive(unsigned* counter, unsigned n, unsigned* flag_lds) {
  __builtin_amdgcn_fence(__ATOMIC_RELEASE, "workgroup");
  __builtin_amdgcn_s_waitcnt(0);
  __syncthreads();
  if (threadIdx.x == 0) {
    const unsigned prev = __hip_atomic_fetch_add(counter, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    *flag_lds = (prev + 1u == n) ? 1u : 0u;
  }
  __syncthreads();
  const bool last = *flag_lds != 0u;
  __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "workgroup");
  return last;
}

// Block-wide publication of layer l's readiness share: every wave waits for its own
// stores, then thread 0 posts one arrival to every copy of ready[l].
__device__ __forceinline__ void block_publish_ready(const StackArgs& a, int l) {
  __builtin_amdgcn_fence(__ATOMIC_RELEASE, "workgroup");
  __builtin_amdgcn_s_waitcnt(0);
  __syncthreads();
  if (threadIdx.x == 0) publish_ready(a, l);
}

// Block-wide wait until *p >= target (thread 0 polls).  Bounded: after a.spin_limit polls
// (seconds by default) or when another workgroup gave up, the stack is abandoned
// (give_up) and false is returned in every thread, so every wave of the grid still
// reaches its end.  phase, l: what the wait is for (recorded when it gives up).
__device__ __forceinline__ bool wait_geq(const StackArgs& a, const unsigned* p, unsigned target, unsigned* flag_lds,
                                         unsigned phase, int l) {
  if (threadIdx.x == 0) {
    unsigned ok = 1u;
    unsigned it = 0;
    while (ld_dev_u32(p) < target) {
      ++it;
      if ((it & 63u) == 0u && ld_dev_u32(abort_flag(a)) != 0u) {
        ok = 0u;
        break;
      }
      if (it > a.spin_limit) {
        give_up(a, phase, l, blockIdx.x);
        ok = 0u;
        break;
      }
      // No sleep between polls: one poll is in flight at a time, so the rate is one per
      // round trip (a sleep of 64 or 192 clocks measured 0.3 % slower per layer; four
      // polls in flight, 5 % slower: the polls delay the combiners' counts on those lines).
    }
    *flag_lds = ok;
  }
  __syncthreads();
  const bool ok = *flag_lds != 0u;
  __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "workgroup");
  return ok;
}

struct SelectLds {
  float lg[kMaxE];                               // logits, then scores
  __attribute__((aligned(16))) uint64_t key[kMaxE + 8];  // selection key << 8 | (255 - id), at key_pos
  int id[kMaxSlots];  // slot -> expert (routed slots by rank, then shared)
  float w[kMaxSlots];
  int ord[kMaxSlots]; // routed slots in ascending expert id
};

struct SelectParams {
  int E, k, S, score, renorm;
  float scaling;
};

// Float -> uint32 whose unsigned order is the float order (finite values).
__device__ __forceinline__ uint32_t order_key(float f) {
  const uint32_t u = __float_as_uint(f);
  return (u & 0x80000000u) ? ~u : (u | 0x80000000u);
}

// Wave-wide (64 lanes) max and sum on DPP: quad swaps, then the half-row and row
// mirrors leave each row of 16 lanes holding its row's result; the four rows are
// combined from lanes 0, 16, 32, 48 (a fixed order; every lane gets the same value).
template <int CTRL>
__device__ __forceinline__ float dpp_f32(float v) {
  return __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), CTRL, 0xF, 0xF, false));
}
__device__ __forceinline__ float lane_f32(float v, int l) { return __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), l)); }
__device__ __forceinline__ float wave_max_dpp(float v) {
  v = fmaxf(v, dpp_f32<0xB1>(v));   // quad_perm [1,0,3,2]
  v = fmaxf(v, dpp_f32<0x4E>(v));   // quad_perm [2,3,0,1]
  v = fmaxf(v, dpp_f32<0x141>(v));  // row_half_mirror
  v = fmaxf(v, dpp_f32<0x140>(v));  // row_mirror
  return fmaxf(fmaxf(lane_f32(v, 0), lane_f32(v, 16)), fmaxf(lane_f32(v, 32), lane_f32(v, 48)));
}
__device__ __forceinline__ float wave_sum_dpp(float v) {
  v = v + dpp_f32<0xB1>(v);
  v = v + dpp_f32<0x4E>(v);
  v = v + dpp_f32<0x141>(v);
  v = v + dpp_f32<0x140>(v);
  return (lane_f32(v, 0) + lane_f32(v, 16)) + (lane_f32(v, 32) + lane_f32(v, 48));
}

// Top-k of one token from sl.lg, in two parts.
//
// select_rank (every thread of the block) finds the selected experts:
//   sl.id[r]  the expert of rank r (descending selection key, ties to the lower id) for
//             r < k, then the shared expert (id E) in slot k.
// The key is the score (+ the selection bias) of host/raon.py:1224-1247.  With softmax
// scores and no bias the key is the logit itself: softmax is increasing, so the order is
// the same (ties, as everywhere, to the lower id), and the scores are needed only for
// the weights.  Wave 0 computes the keys; then rank(i) = #{j : key_j > key_i, or key_j ==
// key_i and j < i} is counted for 16 keys per wave and pass (lane l: key 16g + l%16
// against quarter l/16 of the keys, the quarters added by shuffles), and the keys of rank
// < k write their slot.
//
// select_finish (wave 0 only, any time before the weights are read; a later barrier
// publishes them) computes
//   sl.w[r]    the weight of slot r: the score, renormalised by (sum + 1e-20) and scaled;
//              1 for the shared slot
//   sl.ord[i]  the rank of the i-th selected expert in ascending id order.
// The softmax denominator and the renormalisation sum are wave tree sums (a fixed order;
// numpy's pairwise order differs in the last bit at most, and the selection depends on
// neither).
//
// Keys sit in LDS in quarters of 32 (E <= 128) or 64 keys with 16 bytes between
// quarters, so the four quarter reads of one instruction fall in different banks.
// qkeys is 32 or 64: a shift, not an integer division.
__device__ __forceinline__ int key_pos(int e, int qkeys) { return e + 2 * (e >> (qkeys == 32 ? 5 : 6)); }

__device__ __forceinline__ bool select_fast(const SelectParams a, const float* bias) {
  return a.score == 1 && bias == nullptr;
}

// keys_ready: the caller has already written the keys and the shared slot (the fast path,
// from the threads that summed the logits) and published them with a barrier.
template <int NC>
__device__ __forceinline__ void select_rank(const SelectParams a, const float* __restrict__ bias, SelectLds& sl,
                                            bool keys_ready, int stamp_l, int stamp_g) {
  static_assert(NC >= 1 && NC <= kMaxE / 64, "64-expert chunks");
  // The wave index stays a per-lane value here: as a scalar it measured slower (the rank loop
  // and the key writes are scheduled differently), unlike in the kernel body.
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int E = a.E, K = a.k;
  const int nc = (E + 63) >> 6;     // 64-key chunks; keys in [E, 64*nc) are 0
  const int ncp = nc <= 2 ? 2 : 4;  // the rank pass reads 128 or 256 keys
  const int qkeys = 16 * ncp;       // keys per quarter
  if (!keys_ready && wave == 0) {
    float sc[NC];
#pragma unroll
    for (int c = 0; c < NC; ++c) sc[c] = c < nc && lane + 64 * c < E ? sl.lg[lane + 64 * c] : -__builtin_inff();
    if (!select_fast(a, bias)) {
      if (a.score == 0) {
#pragma unroll
        for (int c = 0; c < NC; ++c)
          if (c < nc) sc[c] = 1.0f / (1.0f + expf(-sc[c]));
      } else {
        float m = sc[0];
#pragma unroll
        for (int c = 1; c < NC; ++c) m = fmaxf(m, sc[c]);
        m = wave_max_dpp(m);
        float z = 0.f;
#pragma unroll
        for (int c = 0; c < NC; ++c) {
          if (c < nc) {
            sc[c] = lane + 64 * c < E ? expf(sc[c] - m) : 0.f;
            z += sc[c];
          }
        }
        z = wave_sum_dpp(z);
#pragma unroll
        for (int c = 0; c < NC; ++c)
          if (c < nc) sc[c] = sc[c] / z;
      }
    }
#pragma unroll
    for (int c = 0; c < NC; ++c) {
      if (c < ncp) {
        const int e = lane + 64 * c;
        // Padded entries (e >= E) sort below every real key and are never selected.
        const uint32_t k32 = e < E ? order_key(bias ? __fadd_rn(sc[c], bias[e]) : sc[c]) : 0u;
        sl.key[key_pos(e, qkeys)] = e < E ? ((uint64_t)k32 << 8) | (uint64_t)(255 - e) : 0ull;
        if (e < E) sl.lg[e] = sc[c];  // the scores (the logits on the fast path)
      }
    }
    if (lane == 0 && a.S > K) sl.id[K] = E;  // shared expert
  }
  if (!keys_ready) __syncthreads();
  RMOE_STAMP(stamp_l, stamp_g, 13, 0);
  {
    auto rank_pass = [&](auto QW) {
      constexpr int qw = decltype(QW)::value;  // uint4 words (2 keys each) per quarter
      const int q = lane >> 4;
      const uint4* kq = reinterpret_cast<const uint4*>(sl.key) + q * (qw + 1);
      for (int g = wave; g < qw / 2; g += kWaves) {  // 8*qw keys = qw/2 groups of 16
        const int i = 16 * g + (lane & 15);
        const uint64_t ki = sl.key[key_pos(i, 2 * qw)];
        uint4 kv[qw];
#pragma unroll
        for (int j2 = 0; j2 < qw; ++j2) kv[j2] = kq[j2];
        int cnt = 0;
#pragma unroll
        for (int j2 = 0; j2 < qw; ++j2) {
          const uint64_t k0 = (uint64_t)kv[j2].x | ((uint64_t)kv[j2].y << 32);
          const uint64_t k1 = (uint64_t)kv[j2].z | ((uint64_t)kv[j2].w << 32);
          cnt += (k0 > ki) ? 1 : 0;
          cnt += (k1 > ki) ? 1 : 0;
        }
        cnt += __shfl_xor(cnt, 16, 64);
        cnt += __shfl_xor(cnt, 32, 64);
        if (lane < 16 && i < E && cnt < K) sl.id[cnt] = i;
      }
    };
    if constexpr (NC <= 2) {
      rank_pass(std::integral_constant<int, 16>{});
    } else {
      if (nc <= 2) rank_pass(std::integral_constant<int, 16>{});
      else rank_pass(std::integral_constant<int, 32>{});
    }
  }
  __syncthreads();
}

template <int NC>
__device__ __forceinline__ void select_finish(const SelectParams a, const float* __restrict__ bias, SelectLds& sl) {
  const int lane = threadIdx.x & 63;
  const int E = a.E, K = a.k;
  const int nc = (E + 63) >> 6;
  float wr = 0.f;
  if (select_fast(a, bias)) {
    // Softmax of the logits: the same m (the largest logit, rank 0) and the same
    // per-lane-then-wave order of the denominator as the score path.
    const float m = sl.lg[sl.id[0]];
    float z = 0.f;
#pragma unroll
    for (int c = 0; c < NC; ++c)
      if (c < nc && lane + 64 * c < E) z += expf(sl.lg[lane + 64 * c] - m);
    z = wave_sum_dpp(z);
    if (lane < K) wr = expf(sl.lg[sl.id[lane]] - m) / z;
  } else if (lane < K) {
    wr = sl.lg[sl.id[lane]];
  }
  // Slots past the routed ones, other than the shared slot, hold a sentinel id while the
  // routed slots are ordered by id (the shared id E exceeds every routed id).
  if (lane >= K && lane < kMaxSlots && !(lane == K && a.S > K)) sl.id[lane] = 0x7fffffff;
  __builtin_amdgcn_fence(__ATOMIC_SEQ_CST, "wavefront");
  __builtin_amdgcn_wave_barrier();
  if (lane < K) {
    const int id = sl.id[lane];
    int pos = 0;
#pragma unroll
    for (int r = 0; r < kMaxSlots; ++r) pos += sl.id[r] < id ? 1 : 0;
    sl.ord[pos] = lane;
  }
  const float denom = a.renorm ? __fadd_rn(wave_sum_dpp(wr), 1e-20f) : 1.f;
  if (lane < K) sl.w[lane] = __fmul_rn(a.renorm ? wr / denom : wr, a.scaling);
  if (lane == 0 && a.S > K) sl.w[K] = 1.f;
}

// Partial router logits of 64 rows (band b) of x for every expert:
//   part[b * Ep + e] = sum_{c in band} x[c] * Wr[e, c]
// (one row of Ep = E rounded up to 32 floats per band: whole cache lines, one writer).
// xp: the band as 32 bf16 pairs in LDS.  wv: this thread's router weights for items
// tid + kThreads*it (item = expert*4 + quarter of 16 columns).  Every thread stores.
template <int NIT>
__device__ __forceinline__ void band_logits(const StackArgs& a, const uint32_t* xp, const uint4 (&wv)[NIT][2],
                                            float* part, int b) {
  const int tid = threadIdx.x;
#pragma unroll
  for (int it = 0; it < NIT; ++it) {
    const int idx = tid + kThreads * it;
    float v = 0.f;
    if (idx < a.E * 4) {
      const uint32_t* xq = xp + 8 * (idx & 3);
      const uint32_t w8[8] = {wv[it][0].x, wv[it][0].y, wv[it][0].z, wv[it][0].w,
                              wv[it][1].x, wv[it][1].y, wv[it][1].z, wv[it][1].w};
#pragma unroll
      for (int c = 0; c < 8; ++c) v = dot2_bf16(w8[c], xq[c], v);
    }
    v += __shfl_xor(v, 1, 64);
    v += __shfl_xor(v, 2, 64);
    if (idx < a.E * 4 && (idx & 3) == 0) st_dev(&part[(size_t)b * a.Ep + (idx >> 2)], v);
  }
}

// Router weights of band b for this thread's items (invalid items read `dummy`, so the
// number of loads is the same on every path and the compiler's waits stay exact).
template <int NIT>
__device__ __forceinline__ void load_router_slice(const StackArgs& a, const uint16_t* rw, int b, bool valid,
                                                  const uint8_t* dummy, uint4 (&wv)[NIT][2]) {
  const int tid = threadIdx.x;
#pragma unroll
  for (int it = 0; it < NIT; ++it) {
    const int idx = tid + kThreads * it;
    const uint8_t* p = dummy;
    if (valid && idx < a.E * 4)
      p = reinterpret_cast<const uint8_t*>(rw + (size_t)(idx >> 2) * a.H + 64 * b + 16 * (idx & 3));
    wv[it][0] = *reinterpret_cast<const uint4*>(p);
    wv[it][1] = *reinterpret_cast<const uint4*>(p + 16);
  }
}

// The router slice of band b (64 columns of every expert row, 128 B each) copied into
// LDS as [expert, E rounded up to 8][128 B] by waves 1..7 (w = wave - 1): one copy
// instruction moves 8 expert rows (lane L: row 8j + L/8, bytes 16(L%8)..; rows past E
// copy row E-1 into slots nobody reads), dealt round robin to the 7 waves.
__device__ __forceinline__ int router_rows8(const StackArgs& a) { return (a.E + 7) & ~7; }
__device__ __forceinline__ void dma_router_slice(const StackArgs& a, const uint16_t* rw, int b, uint8_t* dst, int w,
                                                 int lane) {
  for (int j = w; j < router_rows8(a) / 8; j += kWaves - 1) {
    const int e = min(8 * j + (lane >> 3), a.E - 1);
    const uint16_t* src = rw + (size_t)e * a.H + 64 * b + 8 * (lane & 7);
    __builtin_amdgcn_global_load_lds((global_void_ptr)src, (lds_void_ptr)(dst + (size_t)j * 1024), 16, 0, 0);
  }
}
// This thread's items of a router slice in LDS (the register layout of load_router_slice:
// item tid + kThreads * it is expert item / 4, columns 16 * (item % 4)..).
template <int NIT>
__device__ __forceinline__ void read_router_slice(const StackArgs& a, const uint8_t* src, uint4 (&wv)[NIT][2]) {
#pragma unroll
  for (int it = 0; it < NIT; ++it) {
    const int idx = threadIdx.x + kThreads * it;
    const int i = idx < a.E * 4 ? idx : 0;
    wv[it][0] = *reinterpret_cast<const uint4*>(src + 32 * i);
    wv[it][1] = *reinterpret_cast<const uint4*>(src + 32 * i + 16);
  }
}

// DNPOS: DN tiles per DN wave (waves 1..7 stream the tiles of both DN units:
// 2 * Ipad/128 <= 7 * DNPOS); NIT: router items per thread (n_routed <= 128 * NIT);
// They size register and LDS arrays, so they are template
// parameters.
//
// Wave roles: every wave streams GU tiles; waves 1..7 copy the DN tiles into LDS, and
// all eight waves compute their dot products; wave 0 does the cross-workgroup stores
// (partial sums, h, d, the combine) and holds no DN copies in flight, so its waits for
// its own stores are short.  Loads that have no valid
// target read `dummy` instead of being skipped: every wave issues the same number of
// loads on every path, which keeps the compiler's s_waitcnt counts exact (a GU tile is
// consumed without waiting for the DN tiles issued after it).
template <int DNPOS, int NIT>
__global__ __launch_bounds__(kThreads) void decode_stack_kernel(StackArgs a) {
  __shared__ __attribute__((aligned(16))) uint32_t xs[kMaxH / 2];  // x_l as bf16 pairs
  __shared__ float xsum[kMaxH / 32];                              // group sums of x_l
  __shared__ SelectLds sl;
  __shared__ float red[kWaves][2][64];
  // h of each wave's half-tile items (32 bf16 pairs) and their two group sums.  Up to
  // 7 * DNPOS tiles = 14 * DNPOS half tiles over the 8 waves, two items per pair.
  constexpr int kHalfPairs = ((2 * DNPOS * (kWaves - 1) + kWaves - 1) / kWaves + 1) / 2;
  __shared__ __attribute__((aligned(16))) uint32_t hs2[kWaves][2 * kHalfPairs][32];
  __shared__ float hsum2[kWaves][2 * kHalfPairs][2];
  __shared__ float cmb[kMaxSlots][64];                         // d of every slot of a band
  __shared__ __attribute__((aligned(16))) uint32_t xband[32];  // x_{l+1} of a band, bf16 pairs
  __shared__ __attribute__((aligned(16))) float lrow[kLRowLds];  // partial logits being summed
  __shared__ unsigned flag;
  // DN tiles of this workgroup's units: [kMaxDnUnits][nkt2] tiles, then a 1 KB sink.
  extern __shared__ __attribute__((aligned(16))) uint8_t dn_lds[];
  uint8_t* dn_sink = dn_lds + (size_t)kMaxDnUnits * a.nkt2 * kTileBytes;

  // This workgroup's first GU unit (slot, half band) and its DN units (slot, band; -1
  // when absent).  The same in every layer; kept in LDS so that the index arithmetic does
  // not hold registers across the layer loop.  epoch_s: this launch's epoch.
  __shared__ int gu_d[2];
  __shared__ __attribute__((aligned(16))) int dn_d[kMaxDnUnits][2];
  __shared__ uint32_t epoch_s;

  const int tid = threadIdx.x, lane = tid & 63, wave = wave_id();
  const int g = blockIdx.x, G = gridDim.x;
  const int Hp = a.H / 2;
  if (tid == 0) {
    const int u = g;
    if (u < a.n_gu) {
      gu_d[0] = u / a.nhb;
      gu_d[1] = u % a.nhb;
    } else {
      gu_d[0] = -1;
    }
    epoch_s = ld_dev_u32(epoch_cnt(a));
    const int v0 = ((g - a.n_gu) % G + G) % G;  // first DN unit of this workgroup
    for (int d = 0; d < kMaxDnUnits; ++d) {
      const int v = v0 + d * G;
      dn_d[d][0] = v < a.n_dn ? v / a.nb2 : -1;
      dn_d[d][1] = v < a.n_dn ? v % a.nb2 : 0;
    }
  }
  __syncthreads();
  const uint8_t* dummy = reinterpret_cast<const uint8_t*>(a.x0);
  const uint32_t epoch = epoch_s;
  const uint32_t tag = 2u * epoch + 1u;

  // A GU unit in the shared slot does not depend on the routing: its 2 * nkt1 half tiles
  // (the unit's 32 gate and 32 up rows of every K tile, 5 KB per K tile) are copied into
  // the DN tiles' LDS while the workgroup is idle at the end of the previous layer (at
  // the start for layer 0), and computed as soon as x_l is in LDS, before the routing.
  // The routed gate/up stream after the routing is then smaller by one slot.  LDS layout:
  // piece p = 5 kt + j (code pieces j = 0..3, then scale|min) at p KB, lane L's 16 bytes
  // (lanes 0..31 gate rows, 32..63 up rows, as load_rows reads them) at 16 L.
  const bool gu_pre = a.gu_pre && gu_d[0] == a.k;
  auto issue_gu_pre = [&](int ll) {  // waves 1..7
    if (wave == 0) return;
    const int hb = gu_d[1];
    const size_t band = lane < 32 ? (size_t)(hb >> 1) : (size_t)(a.nb1 + (hb >> 1));
    const uint8_t* base = a.gu[ll] + (size_t)a.E * a.gu_bytes + band * a.nkt1 * kTileBytes +
                          (size_t)(32 * (hb & 1) + (lane & 31)) * 16;
    for (int p = wave - 1; p < 5 * a.nkt1; p += kWaves - 1) {
      const int kt = p / 5, j = p - 5 * kt;
      __builtin_amdgcn_global_load_lds((global_void_ptr)(base + (size_t)kt * kTileBytes + j * 1024),
                                       (lds_void_ptr)(dn_lds + (size_t)p * 1024), 16, 0, 0);
    }
  };
  if (gu_pre) issue_gu_pre(0);

  // DN tiles of this workgroup's units, flattened as t = d * nkt2 + kt: wave 1 + t % 7
  // copies tile t into LDS slot t at its position t / 7.  Units whose bit is clear in
  // `mask` copy 16 dummy bytes into the sink instead (the same number of loads).  A unit
  // in the shared slot does not depend on the routing: unless the shared-slot GU tiles
  // use the same LDS (gu_pre), its tiles are copied at the end of the previous layer (at
  // the start for layer 0), and only the routed units' tiles after the routing.
  // (dn_pre: the bits of those units; in LDS like the unit indices.)
  __shared__ unsigned dn_pre;
  if (tid == 0)
    dn_pre = gu_pre || a.S <= a.k ? 0u : (dn_d[0][0] == a.k ? 1u : 0u) | (dn_d[1][0] == a.k ? 2u : 0u);
  __syncthreads();
  auto issue_dn_at = [&](const uint8_t* dnb, unsigned mask, int wv, int ln) {
    const int n_dn_t = (dn_d[0][0] >= 0 ? a.nkt2 : 0) + (dn_d[1][0] >= 0 ? a.nkt2 : 0);
#pragma unroll
    for (int p = 0; p < DNPOS; ++p) {
      const int t = wv - 1 + (kWaves - 1) * p;
      const bool ok = wv > 0 && t < n_dn_t && ((mask >> (t / a.nkt2)) & 1u);
      const int d = ok ? t / a.nkt2 : 0, kt = ok ? t % a.nkt2 : 0;
      const int slot = ok ? dn_d[d][0] : 0;
      const uint8_t* W = dnb + (size_t)(slot == a.k ? a.E : sl.id[slot]) * a.dn_bytes;
      dma_tile(ok, W + ((size_t)dn_d[d][1] * a.nkt2 + kt) * kTileBytes, dummy, dn_lds + (size_t)t * kTileBytes,
               dn_sink, ln);
    }
  };
  if (dn_pre) issue_dn_at(a.dn[0], dn_pre, wave, lane);

  // Layer 0: the band share of the router logits of x0 (workgroups b < nb2).
  if (g < a.nb2) {
    if (tid < 32) xband[tid] = reinterpret_cast<const uint32_t*>(a.x0)[32 * g + tid];
    uint4 wv[NIT][2];
    load_router_slice<NIT>(a, a.rw[0], g, true, dummy, wv);
    __syncthreads();
    band_logits<NIT>(a, xband, wv, reinterpret_cast<float*>(a.scratch + a.off_lpart), g);
    block_publish_ready(a, 0);
  }

  for (int l = 0; l < a.L; ++l) {
    // The thread index passes through an empty asm at the top of every layer, so values
    // derived from it (LDS and row addresses of every phase) are recomputed per layer
    // instead of being hoisted out of the loop, where together they held enough
    // registers across all phases to force spills: scratch reloads on the hand-off path,
    // each one a memory round trip, and s_waitcnt vmcnt(0) after them also waited for
    // the wave's weight loads.
    int tid_o = (int)threadIdx.x;
    asm volatile("" : "+v"(tid_o));
    const int tid = tid_o, lane = tid & 63, wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    unsigned* c_ready = cnt_at(a, l, g % kReadyCopies);
    uint8_t* lay = a.scratch + (size_t)l * a.layer_bytes;
    const uint32_t* xin = reinterpret_cast<const uint32_t*>(lay);
    const float* lpart = reinterpret_cast<const float*>(lay + a.off_lpart);
    uint64_t* hbuf = reinterpret_cast<uint64_t*>(lay + a.off_h);  // [S][Ipad/2] tagged h pairs
    const int hstride = a.Ipad / 2;
    uint64_t* dtag = reinterpret_cast<uint64_t*>(lay + a.off_dout);  // [S][H] tagged d words

    RMOE_STAMP_FLUSH(l - 1, g);
    if (!wait_geq(a, c_ready, (unsigned)a.nb2, &flag, kAbortReady, l)) return;
    RMOE_STAMP(l, g, 0, 0);

    const bool keys_fast = a.score == 1 && a.rb[l] == nullptr;
    // ---- x_l and the routing of this layer.  Every device-scope load of a thread is
    // issued before the first use, so the latencies overlap.
    {
      // x_l: 64-bit loads (tid covers dwords 2*idx, 2*idx+1).  The partial logits
      // [nb2][Ep] are contiguous: passes of up to kLRow floats are copied into LDS with
      // 16-byte loads (the first pass's loads issued right after x's, before either is
      // used), then P threads per expert sum its bands.
      uint64_t xv[kMaxH / 4 / kThreads];
#pragma unroll
      for (int i = 0; i < kMaxH / 4 / kThreads; ++i) {
        const int idx = tid + kThreads * i;
        xv[i] = 0ull;
        if (2 * idx < Hp)
          xv[i] = l == 0 ? reinterpret_cast<const uint64_t*>(a.x0)[idx] : ld_hand_u64(xin + 2 * idx);
      }
      const int lstride = a.Ep + kLPad;
      const int nbc = min(kLRow / a.Ep, kLRowLds / lstride);  // bands per pass
      const int rq = a.Ep / 4;
      // Two 16-byte pieces per thread and pass (kLRow = 4096 floats); piece j of the pass
      // is row j / rq of it.
      static_assert(kLRow / 4 == 2 * kThreads, "two 16-byte pieces per thread");
      auto load_pass = [&](int b0, uint4& v0, uint4& v1) {
        const int nf4 = (min(nbc, a.nb2 - b0) * a.Ep) / 4;
        const uint4* src = reinterpret_cast<const uint4*>(lpart + (size_t)b0 * a.Ep);
        v0 = tid < nf4 ? src[tid] : make_uint4(0u, 0u, 0u, 0u);
        v1 = tid + kThreads < nf4 ? src[tid + kThreads] : make_uint4(0u, 0u, 0u, 0u);
      };
      uint4 pv0, pv1;
      load_pass(0, pv0, pv1);
      // x_l into LDS, and the group sums of x_l from the registers: the 32 values of a
      // group are held by 8 neighbouring lanes (4 each), summed in a fixed tree.
#pragma unroll
      for (int i = 0; i < kMaxH / 4 / kThreads; ++i) {
        const int idx = tid + kThreads * i;
        if (2 * idx < Hp) {
          xs[2 * idx] = (uint32_t)xv[i];
          xs[2 * idx + 1] = (uint32_t)(xv[i] >> 32);
        }
        if (i * kThreads < Hp / 2) {  // uniform: H % 256 == 0 keeps groups of 8 lanes whole
          const uint32_t lo = (uint32_t)xv[i], hi = (uint32_t)(xv[i] >> 32);
          float sv = (bf16_to_f32(lo & 0xffffu) + bf16_to_f32(lo >> 16)) +
                     (bf16_to_f32(hi & 0xffffu) + bf16_to_f32(hi >> 16));
          sv += dpp_f32<0xB1>(sv);  // lane ^ 1
          sv += dpp_f32<0x4E>(sv);  // lane ^ 2
          sv += __shfl_xor(sv, 4, 64);
          if ((idx & 7) == 0 && 2 * idx < Hp) xsum[idx >> 3] = sv;
        }
      }
      // P threads per expert (neighbouring lanes) sum every P-th band; then a fixed tree.
      const int P = a.E <= 128 ? 4 : 2;
      const int pe = tid / P, pp = tid % P;
      float lacc = 0.f;
      for (int b0 = 0; b0 < a.nb2; b0 += nbc) {
        const int nb = min(nbc, a.nb2 - b0);
        const int nf4 = (nb * a.Ep) / 4;
        if (b0 > 0) load_pass(b0, pv0, pv1);
        // Row of piece j by a float reciprocal, not an integer division: j < 1024 and
        // rq >= 8, so (j + 0.5) / rq stays >= 1/16 away from an integer, far beyond the
        // reciprocal's rounding.
        const float rinv = 1.0f / (float)rq;
        const int j1 = tid + kThreads;
        const int r0 = (int)(((float)tid + 0.5f) * rinv), r1 = (int)(((float)j1 + 0.5f) * rinv);
        if (tid < nf4) *reinterpret_cast<uint4*>(lrow + r0 * lstride + 4 * (tid - r0 * rq)) = pv0;
        if (j1 < nf4) *reinterpret_cast<uint4*>(lrow + r1 * lstride + 4 * (j1 - r1 * rq)) = pv1;
        __syncthreads();
        if (b0 == 0) RMOE_STAMP(l, g, 12, 0);
        if (pe < a.E && nb == 8 * P) {
          // The pass holds exactly eight of the thread's bands (BASELINE: 32 bands, P = 4):
          // the same reads and sums as the loop below, without its bounds tests.
          const float* lp = lrow + pp * lstride + pe;
          const int bs = P * lstride;
          float v[8];
#pragma unroll
          for (int i = 0; i < 8; ++i) v[i] = lp[i * bs];
          lacc += ((v[0] + v[1]) + (v[2] + v[3])) + ((v[4] + v[5]) + (v[6] + v[7]));
        } else if (pe < a.E) {
          // Eight of the thread's bands are read at a time (one LDS round trip, not one
          // per band), then added in band order.
          for (int bb = pp; bb < nb; bb += 8 * P) {
            float v[8];
#pragma unroll
            for (int i = 0; i < 8; ++i) {
              const int b = bb + P * i;
              v[i] = b < nb ? lrow[b * lstride + pe] : 0.f;
            }
            // (absent bands read 0: adding +0 leaves every sum unchanged)
            lacc += ((v[0] + v[1]) + (v[2] + v[3])) + ((v[4] + v[5]) + (v[6] + v[7]));
          }
        }
        if (b0 + nbc < a.nb2) __syncthreads();  // lrow is refilled by the next pass
      }
      lacc += dpp_f32<0xB1>(lacc);
      if (P == 4) lacc += dpp_f32<0x4E>(lacc);
      if (pe < a.E && pp == 0) sl.lg[pe] = lacc;
      // Softmax scores without a bias rank like the logits: the same threads write the
      // selection keys (padded entries below every key) and the shared slot, and the
      // barrier below publishes them with the logits.
      if (keys_fast && pp == 0) {
        const int ncp = ((a.E + 63) >> 6) <= 2 ? 2 : 4;
        if (pe < 64 * ncp)
          sl.key[key_pos(pe, 16 * ncp)] = pe < a.E ? ((uint64_t)order_key(lacc) << 8) | (uint64_t)(255 - pe) : 0ull;
        if (pe == 0 && a.S > a.k) sl.id[a.k] = a.E;
      }
    }
    __syncthreads();
    RMOE_STAMP(l, g, 1, 0);

    // GU outputs of a unit: the waves' sums in order, then h = RTNE(act(RTNE(g), RTNE(u)))
    // of its 32 columns, published as 16 tagged words of bf16 pairs.
    auto gu_publish = [&](int s, int hb, float acc) {
      red[wave][0][lane] = acc;
      __syncthreads();
      RMOE_STAMP(l, g, 15, 0);
      if (wave == 0) {
        float gs = 0.f, us = 0.f;
#pragma unroll
        for (int w = 0; w < kWaves; ++w) {
          gs += red[w][0][lane & 31];
          us += red[w][0][32 + (lane & 31)];
        }
        const uint32_t hb16 = f32_to_bf16(act_apply(a.act, bf16_round(gs), bf16_round(us), a.gb, a.vb));
        const uint32_t hi = (uint32_t)__builtin_amdgcn_update_dpp(0, (int)hb16, 0xB1, 0xF, 0xF, false);  // lane ^ 1
        if (lane < 32 && (lane & 1) == 0)
          st_dev_u64(&hbuf[(size_t)s * hstride + 16 * hb + (lane >> 1)],
                     (uint64_t)(hb16 | (hi << 16)) | ((uint64_t)tag << 32));
      }
    };
    // The shared-slot GU unit from its tiles in LDS (copied during the previous layer:
    // every wave's copies have landed, as its later loads have).
    if (gu_pre) {
      __builtin_amdgcn_s_waitcnt(0);
      __syncthreads();
      float acc = 0.f;
      for (int kt = wave; kt < a.nkt1; kt += kWaves) {
        TileRegs r;
        const uint8_t* t = dn_lds + (size_t)kt * kTileBytes + lane * 16;
#pragma unroll
        for (int j = 0; j < 4; ++j) r.c[j] = *reinterpret_cast<const uint4*>(t + j * 1024);
        r.sm = *reinterpret_cast<const uint4*>(t + kCodeBytes);
        acc = tile_dot(r, xs + kt * 64, xsum + kt * 4, acc);
      }
      gu_publish(gu_d[0], gu_d[1], acc);  // its barrier also ends every wave's LDS reads
      RMOE_STAMP(l, g, 3, 0);
    }
    const SelectParams sp{a.E, a.k, a.S, a.score, a.renorm, a.scaling};
    select_rank<2 * NIT>(sp, a.rb[l], sl, keys_fast, l, g);  // E <= 128 * NIT: at most 2 * NIT chunks of 64
    RMOE_STAMP(l, g, 2, 0);

    // ---- issue every weight load of this workgroup's units for this layer.
    // A GU unit (slot s, half band hb) is the 32 gate rows 32hb.. and the 32 matching up
    // rows over all of K: lanes 0..31 of a wave read gate rows, lanes 32..63 the up rows
    // (each lane its own row of the tile), so one tile_dot covers both.  Wave w takes K
    // tiles w, w + 8, ...; the first two are loaded here.
    const uint8_t* gu_l = a.gu[l];
    const uint8_t* dn_l = a.dn[l];
    auto gu_row = [&](int s, int hb, int kt) {
      const uint8_t* W = gu_l + (size_t)sl.id[s] * a.gu_bytes;
      const size_t band = lane < 32 ? (size_t)(hb >> 1) : (size_t)(a.nb1 + (hb >> 1));
      return W + (band * a.nkt1 + kt) * kTileBytes + (size_t)(32 * (hb & 1) + (lane & 31)) * 16;
    };
    TileRegs mt0, mt1;
    {
      const int s = gu_pre ? -1 : gu_d[0];
      const bool ok0 = s >= 0 && wave < a.nkt1, ok1 = s >= 0 && wave + kWaves < a.nkt1;
      load_rows(mt0, ok0, ok0 ? gu_row(s, gu_d[1], wave) : dummy, dummy);
      load_rows(mt1, ok1, ok1 ? gu_row(s, gu_d[1], wave + kWaves) : dummy, dummy);
    }
    // The routed DN units' tiles: a workgroup with a GU unit issues them after its GU
    // tiles have arrived, so the gate/up stream (on the critical path) does not share HBM
    // with the down stream; the others issue them at once.
    const int n_dn_t = (dn_d[0][0] >= 0 ? a.nkt2 : 0) + (dn_d[1][0] >= 0 ? a.nkt2 : 0);
    auto issue_dn = [&](const uint8_t* dnb, unsigned mask) { issue_dn_at(dnb, mask, wave, lane); };
    if (gu_d[0] < 0 || gu_pre) issue_dn(dn_l, 3u & ~dn_pre);
    // ---- slot weights and id order (read by the combine, after later barriers), while
    // the weight loads are in flight.
    if (wave == 0) {
      select_finish<2 * NIT>(sp, a.rb[l], sl);
      if (g == 0 && tid < a.k) {
        if (a.ids_out) a.ids_out[(size_t)l * a.k + tid] = sl.id[tid];
        if (a.wts_out) a.wts_out[(size_t)l * a.k + tid] = sl.w[tid];
      }
    }

    // ---- GU units: g and u of the unit's rows over all of K, then gu_publish.  The first
    // unit uses the tiles loaded above (kept out of the loop so the compiler's wait for
    // them does not also cover the DN loads); any further ones (more units than
    // workgroups) load on the spot.
    auto gu_unit = [&](int s, int hb) {
      float acc = 0.f;
      if (wave < a.nkt1) acc = tile_dot(mt0, xs + wave * 64, xsum + wave * 4, acc);
      RMOE_STAMP(l, g, 14, 0);
      if (wave + kWaves < a.nkt1) acc = tile_dot(mt1, xs + (wave + kWaves) * 64, xsum + (wave + kWaves) * 4, acc);
      for (int kt = wave + 2 * kWaves; kt < a.nkt1; kt += kWaves) {
        TileRegs r;
        load_rows(r, true, gu_row(s, hb, kt), dummy);
        acc = tile_dot(r, xs + kt * 64, xsum + kt * 4, acc);
      }
      gu_publish(s, hb, acc);
    };
    if (gu_d[0] >= 0 && !gu_pre) {
      gu_unit(gu_d[0], gu_d[1]);
      RMOE_STAMP(l, g, 3, 0);
      issue_dn(dn_l, 3u & ~dn_pre);
    }
    for (int u = g + G; u < a.n_gu; u += G) {
      const int s = u / a.nhb, hb = u % a.nhb;
      __syncthreads();  // red[] of the previous unit has been read
      load_rows(mt0, wave < a.nkt1, wave < a.nkt1 ? gu_row(s, hb, wave) : dummy, dummy);
      load_rows(mt1, wave + kWaves < a.nkt1, wave + kWaves < a.nkt1 ? gu_row(s, hb, wave + kWaves) : dummy, dummy);
      gu_unit(s, hb);
    }

    // ---- DN units, both of a workgroup at once, and the combine of a band by its
    // combiner.
    if (n_dn_t > 0) {
      // h of each of this wave's DN tiles: lane covers columns 128kt + 2*lane (+1), one
      // tagged word per tile, polled until it carries this launch's tag (columns past I
      // are zero).  Bounded: past kSpinLimit polls, or when another workgroup gave up,
      // the stack is abandoned after the whole workgroup has agreed to stop.
      bool failed = false;
      // Work items: half tiles (item it: tile it >> 1, its groups 2 (it & 1) and +1), dealt
      // round robin to all eight waves, so that the two waves of every SIMD share its
      // work (a DN tile's dot products are one dependent chain per row; a SIMD runs two
      // waves' chains interleaved at twice the rate of one).  The tiles were copied into
      // LDS by waves 1..7; the barrier below makes every copy visible to every wave.
      // h of an item: lanes 0..31 poll the 32 tagged words of item 2q, lanes 32..63 those
      // of item 2q + 1 (columns 128 kt + 64 (it & 1) + 2 (lane & 31), +1; columns past I
      // are zero), until they carry this launch's tag.  Bounded: past a.spin_limit polls,
      // or when another workgroup gave up, the stack is abandoned after the whole
      // workgroup has agreed to stop.
      const int n_items = 2 * n_dn_t;
      auto item_of = [&](int m) { return wave + kWaves * m; };
      {
        uint64_t hv[kHalfPairs];
        const uint64_t* hp[kHalfPairs];
        unsigned need = 0u;
#pragma unroll
        for (int q = 0; q < kHalfPairs; ++q) {
          const int it = item_of(2 * q + (lane >> 5));
          const bool ok = it < n_items;
          const int t = ok ? it >> 1 : 0;
          const int d = t / a.nkt2;
          const int c0 = 128 * (t % a.nkt2) + 64 * (it & 1) + 2 * (lane & 31);
          hv[q] = 0ull;
          hp[q] = hbuf + (size_t)(dn_d[d][0] < 0 ? 0 : dn_d[d][0]) * hstride + (c0 >> 1);
          if (ok && c0 < a.I) need |= 1u << q;
        }
        unsigned it = 0;
        while (__any(need != 0u)) {
#pragma unroll
          for (int q = 0; q < kHalfPairs; ++q) {
            if (need & (1u << q)) {
              hv[q] = ld_dev_u64(hp[q]);
              if ((uint32_t)(hv[q] >> 32) == tag) need &= ~(1u << q);
            }
          }
          if (!__any(need != 0u)) break;
          ++it;
          if ((it & 63u) == 0u && ld_dev_u32(abort_flag(a)) != 0u) {
            failed = true;
            break;
          }
          if (it > a.spin_limit) {
            if (lane == 0) give_up(a, kAbortH, l, g);
            failed = true;
            break;
          }
          // ~640 clocks between rounds: the words still missing are read again only after
          // most of a memory round trip, which keeps the polls of waves that start
          // early (the down tiles issued at the routing) off the gate/up stream
          // (measured against 64 and 1,536 clocks: 14.37 and 14.60 against 14.32 us/layer).
          __builtin_amdgcn_s_sleep(10);
        }
#pragma unroll
        for (int q = 0; q < kHalfPairs; ++q) {
          const int m = 2 * q + (lane >> 5);
          if (item_of(2 * q) < n_items) {  // the pair's first item exists (uniform)
            const uint32_t hw = (uint32_t)hv[q];  // zero for columns past I and absent items
            const float h0 = bf16_to_f32(hw & 0xffffu), h1 = bf16_to_f32(hw >> 16);
            hs2[wave][m][lane & 31] = hw;
            float gs = h0 + h1;
            gs += dpp_f32<0xB1>(gs);
            gs += dpp_f32<0x4E>(gs);
            gs += dpp_f32<0x141>(gs);
            gs += dpp_f32<0x140>(gs);
            if ((lane & 15) == 0) hsum2[wave][m][(lane >> 4) & 1] = gs;
          }
        }
      }
      if (__syncthreads_or(failed ? 1 : 0)) return;
      RMOE_STAMP(l, g, 4, 0);
      // The DN tiles were copied into LDS by the waves' own loads: drain them.
      __builtin_amdgcn_s_waitcnt(0);
      __syncthreads();
      RMOE_STAMP(l, g, 5, 0);
      float acc[kMaxDnUnits] = {0.f, 0.f};
      {
#pragma unroll 1
        for (int m = 0; m < 2 * kHalfPairs; ++m) {
          const int it = item_of(m);
          if (it < n_items) {
            const int t = it >> 1, hf = it & 1;
            const uint8_t* tp = dn_lds + (size_t)t * kTileBytes + lane * 16;
            const uint2 smv = *reinterpret_cast<const uint2*>(tp + kCodeBytes + 8 * hf);
            const uint32_t sm[2] = {smv.x, smv.y};
            float v = 0.f;
#pragma unroll
            for (int j = 0; j < 2; ++j) {
              const uint4 cw = *reinterpret_cast<const uint4*>(tp + (2 * hf + j) * 1024);
              v = group_apply(sm[j], group_dot(cw, hs2[wave][m] + 16 * j), hsum2[wave][m][j], v);
            }
            if (t < a.nkt2) acc[0] += v;
            else acc[1] += v;
          }
        }
      }
      RMOE_STAMP(l, g, 6, 64);
      red[wave][0][lane] = acc[0];
      red[wave][1][lane] = acc[1];
      __syncthreads();
      RMOE_STAMP(l, g, 7, 0);
      // The combiner of band b is the workgroup whose first DN unit is (slot 0, band b):
      // slot 0's units are units 0..nb2-1, and unit v is the first unit of workgroup
      // (n_gu + v) mod G, so every band has exactly one.
      // (slot, band) of both units in one LDS read.
      const int4 ud = *reinterpret_cast<const int4*>(&dn_d[0][0]);
      const bool comb = ud.x == 0;
      const int cb = ud.y;
      // The next layer's router weights of the combined band, copied into the DN tiles'
      // LDS (every wave is done with the tiles) by waves 1..7 while wave 0 hands d over.
      // They are drained before the logits.
      uint8_t* rw_lds = dn_lds;  // [E rounded up to 8][128 B]
      if (comb && wave > 0 && l + 1 < a.L) dma_router_slice(a, a.rw[l + 1], cb, rw_lds, wave - 1, lane);
      // d of both units as tagged words: no store acknowledgement and no counter; the
      // combiner of the band polls them.  A combiner keeps the d of its own units of its
      // band in LDS instead (own: their slot bits), so it polls only the other slots.
      // The eight waves' partial sums of both units are read first, all at once (their
      // LDS latencies overlap instead of following each other), then added in wave order.
      unsigned own = 0u;
      if (wave == 0) {
        float pw[kMaxDnUnits][kWaves];
#pragma unroll
        for (int d = 0; d < kMaxDnUnits; ++d)
#pragma unroll
          for (int w = 0; w < kWaves; ++w) pw[d][w] = red[w][d][lane];
#pragma unroll
        for (int d = 0; d < kMaxDnUnits; ++d) {
          const int us = d == 0 ? ud.x : ud.z, ub = d == 0 ? ud.y : ud.w;
          if (us < 0) continue;
          float dd = 0.f;
#pragma unroll
          for (int w = 0; w < kWaves; ++w) dd += pw[d][w];
          const float v = bf16_round(dd);
          if (comb && ub == cb) {
            cmb[us][lane] = v;
            own |= 1u << us;
          } else {
            st_dev_u64(&dtag[(size_t)us * a.H + 64 * ub + lane], (uint64_t)__float_as_uint(v) | ((uint64_t)tag << 32));
          }
        }
      }
      RMOE_STAMP(l, g, 8, 0);
      if (comb) {
        const int row = 64 * cb + lane;
        bool cfailed = false;
        // The combine's operands known since the routing (the first 8 slots in ascending
        // expert id with their weights, and x_l of the row for the residual), read before
        // the wait so that they are not on the path after it.
        int o8p[8];
        float w8p[8];
        uint32_t xres = 0u;
        if (wave == 0) {
#pragma unroll
          for (int i = 0; i < 8; ++i) {
            o8p[i] = i < a.k ? sl.ord[i] : 0;
            w8p[i] = sl.w[o8p[i]];
          }
          xres = (xs[row >> 1] >> (16 * (row & 1))) & 0xffffu;
        }
        if (wave == 0) {
          // d of every slot of the band into LDS: each lane polls its row's word of every
          // slot (up to 9 loads in flight) until all carry this launch's tag.  Bounded
          // like the h wait.
          unsigned need = ((1u << a.S) - 1u) & ~own;
          unsigned it = 0;
          while (true) {
            for (int q0 = 0; q0 < a.S; q0 += 9) {
              uint64_t dv[9];
#pragma unroll
              for (int i = 0; i < 9; ++i)
                dv[i] = (q0 + i < a.S && ((need >> (q0 + i)) & 1u)) ? ld_dev_u64(&dtag[(size_t)(q0 + i) * a.H + row])
                                                                    : 0ull;
#pragma unroll
              for (int i = 0; i < 9; ++i) {
                if (q0 + i < a.S && ((need >> (q0 + i)) & 1u) && (uint32_t)(dv[i] >> 32) == tag) {
                  cmb[q0 + i][lane] = __uint_as_float((uint32_t)dv[i]);
                  need &= ~(1u << (q0 + i));
                }
              }
            }
            if (!__any(need != 0u)) break;
            ++it;
            if ((it & 63u) == 0u && ld_dev_u32(abort_flag(a)) != 0u) {
              cfailed = true;
              break;
            }
            if (it > a.spin_limit) {
              if (lane == 0) give_up(a, kAbortD, l, g);
              cfailed = true;
              break;
            }
            __builtin_amdgcn_s_sleep(1);
          }
        }
        // A barrier that waits for LDS only: waves 1..7 still have the router slice in
        // flight, which the combine does not read (they drain it before the logits).
        if (wave == 0 && lane == 0) flag = cfailed ? 1u : 0u;
        asm volatile("s_waitcnt lgkmcnt(0)\n\ts_barrier" ::: "memory");
        if (flag != 0u) return;
        RMOE_STAMP(l, g, 9, 0);
        if (wave == 0) {
          // Ascending expert id: the slot order, then each slot's value and weight, read
          // from LDS in batches, then summed in order.  The shared slot's d is read with
          // the first batch.
          // The first eight slots come straight from the operands read before the wait,
          // with no branch per slot: a slot past k adds +0 (acc2 starts at +0, so the sum
          // is unchanged bit for bit).  Slots 8.. (k > 8) follow in batches of 8.
          const float dsh = a.S > a.k ? cmb[a.k][lane] : 0.f;
          float c8[8];
#pragma unroll
          for (int i = 0; i < 8; ++i) c8[i] = cmb[o8p[i]][lane];
          float acc2 = 0.f;
#pragma unroll
          for (int i = 0; i < 8; ++i) {
            const float p = __fmul_rn(c8[i], w8p[i]);
            acc2 = __fadd_rn(acc2, i < a.k ? p : 0.f);
          }
          for (int r0 = 8; r0 < a.k; r0 += 8) {
            int o8[8];
            float w8[8];
#pragma unroll
            for (int i = 0; i < 8; ++i) o8[i] = r0 + i < a.k ? sl.ord[r0 + i] : 0;
#pragma unroll
            for (int i = 0; i < 8; ++i) {
              c8[i] = cmb[o8[i]][lane];
              w8[i] = sl.w[o8[i]];
            }
#pragma unroll
            for (int i = 0; i < 8; ++i)
              if (r0 + i < a.k) acc2 = __fadd_rn(acc2, __fmul_rn(c8[i], w8[i]));
          }
          uint32_t o = f32_to_bf16(acc2);
          if (a.S > a.k) o = f32_to_bf16(__fadd_rn(bf16_to_f32(o), dsh));
          if (a.residual) o = f32_to_bf16(__fadd_rn(bf16_to_f32(xres), bf16_to_f32(o)));
          // The odd neighbour's value (lane ^ 1) by a DPP move, no LDS round trip.
          const uint32_t hi = (uint32_t)__builtin_amdgcn_update_dpp(0, (int)o, 0xB1, 0xF, 0xF, false);
          if ((lane & 1) == 0) xband[lane >> 1] = o | (hi << 16);
          if (l + 1 == a.L) {
            a.out[row] = (uint16_t)o;
          } else if ((lane & 1) == 0) {
            uint32_t* xnext = reinterpret_cast<uint32_t*>(lay + a.layer_bytes);
            st_dev_u32(&xnext[row >> 1], o | (hi << 16));
          }
        }
        if (l + 1 < a.L) {
          if (wave > 0) __builtin_amdgcn_s_waitcnt(0);  // the router slice is in LDS
          // Again for LDS only (xband): wave 0's x stores stay in flight while the logits
          // are computed; block_publish_ready waits for them before ready is counted.
          asm volatile("s_waitcnt lgkmcnt(0)\n\ts_barrier" ::: "memory");
          float* lnext = reinterpret_cast<float*>(lay + a.layer_bytes + a.off_lpart);
          uint4 rwv[NIT][2];
          RMOE_STAMP(l, g, 10, 0);
          read_router_slice<NIT>(a, rw_lds, rwv);
          band_logits<NIT>(a, xband, rwv, lnext, cb);
          block_publish_ready(a, l + 1);
          RMOE_STAMP(l, g, 11, 0);
        }
      }
      if (wave > 0) __builtin_amdgcn_s_waitcnt(0);  // router slice copies have landed
    }
    // The next layer's shared-slot GU tiles, once every wave is done with the LDS.
    if (gu_pre && l + 1 < a.L) {
      __syncthreads();
      issue_gu_pre(l + 1);
    }
    // The next layer's shared-slot DN tiles, once every wave is done with the LDS (the
    // DN products, and a combiner's router slice: read before its logits).
    if (dn_pre && l + 1 < a.L) {
      __syncthreads();
      issue_dn(a.dn[l + 1], dn_pre);
    }
  }

  RMOE_STAMP_FLUSH(a.L - 1, g);
  // Every wave's stores and counter updates are complete before the workgroup counts
  // itself out; the last workgroup out clears every counter for the next launch.
  if (block_arrive(exit_cnt(a), (unsigned)G, &flag)) {
    const int n = a.L * a.cnt_stride;
    for (int i = tid; i < n; i += kThreads) st_dev_u32(a.cnt + (1 + (size_t)i) * kCntPad, 0u);
    if (tid == 0) {
      st_dev_u32(abort_flag(a), 0u);
      st_dev_u32(exit_cnt(a), 0u);
      st_dev_u32(epoch_cnt(a), (epoch + 1u) & 0x7fffffffu);
    }
  }
}

struct StackShape {
  int S, nb1, nb2, nkt1, nkt2, nhb, n_gu, n_dn;
  size_t off_lpart, off_h, off_dout, layer_bytes;
  int cnt_stride;
};

size_t al256(size_t v) { return (v + 255) / 256 * 256; }

// Dynamic LDS of the kernel: the DN tiles of kMaxDnUnits units plus the 1 KB sink.
// The same LDS holds the next layer's router slice of the combined band once the DN
// tiles are consumed (E rounded up to 8 rows of 128 B each), and the shared-slot GU
// tiles between layers.
constexpr size_t kLdsLimit = 160 * 1024;   // per CU on gfx950
constexpr size_t kStaticLds = 48 * 1024;   // bound on the kernel's static LDS
// The shared-slot GU unit's tiles (nkt1 K tiles, 5 KB each) are copied into the same LDS
// when the layer has a shared slot and they fit.
bool gu_prefetch_fits(int nkt1) { return (size_t)nkt1 * kTileBytes + kStaticLds <= kLdsLimit; }
size_t dn_lds_bytes(int nkt2, int n_routed, int nkt1, bool gu_pre) {
  return std::max({(size_t)kMaxDnUnits * nkt2 * kTileBytes + 1024, (size_t)((n_routed + 7) & ~7) * 128,
                   gu_pre ? (size_t)nkt1 * kTileBytes : (size_t)0});
}

StackShape stack_shape(const RmoeLayer& L) {
  StackShape sh{};
  sh.S = L.top_k + L.n_shared;
  sh.nb1 = L.I / 64;
  sh.nb2 = L.H / 64;
  sh.nkt1 = L.H / kTileCols;
  sh.nkt2 = L.Ipad / kTileCols;
  sh.nhb = L.I / 32;
  sh.n_gu = sh.S * sh.nhb;
  sh.n_dn = sh.S * sh.nb2;
  size_t off = al256((size_t)L.H * 2);  // x_l (bf16)
  sh.off_lpart = off;
  off += al256((size_t)sh.nb2 * ((L.n_routed + 31) / 32 * 32) * 4);
  sh.off_h = off;
  off += al256((size_t)sh.S * (L.Ipad / 2) * 8);
  sh.off_dout = off;
  off += al256((size_t)sh.S * L.H * 8);  // tagged d words
  sh.layer_bytes = off;
  sh.cnt_stride = kReadyCopies;
  return sh;
}

}  // namespace

#ifdef RMOE_DECODE_TIMELINE
extern "C" int rmoe_debug_stack_timeline(unsigned long long* host, size_t n) {
  if (n != sizeof(g_stack_timeline) / sizeof(unsigned long long)) return -1;
  return (int)hipMemcpyFromSymbol(host, HIP_SYMBOL(g_stack_timeline), sizeof(g_stack_timeline), 0,
                                  hipMemcpyDeviceToHost);
}
#endif

size_t stack_scratch_bytes(const RmoeLayer& L, int n_layers) {
  const StackShape sh = stack_shape(L);
  // One extra layer slot: the last layer's combine addresses layer L's x and logits.
  return sh.layer_bytes * (size_t)(n_layers + 1);
}

size_t stack_counter_count(const RmoeLayer& L, int n_layers) {
  return (1 + (size_t)stack_shape(L).cnt_stride * n_layers + 2) * kCntPad;
}

hipError_t stack_check(const RmoeLayer& L, int n_cu) {
  const StackShape sh = stack_shape(L);
  if (L.H > kMaxH || L.n_routed > kMaxE || sh.S > kMaxSlots || kMaxDnUnits * sh.nkt2 > (kWaves - 1) * kMaxDnPos ||
      L.I % 64 != 0 || dn_lds_bytes(sh.nkt2, L.n_routed, sh.nkt1, false) + kStaticLds > kLdsLimit)
    return hipErrorInvalidValue;

  if (sh.n_dn > kMaxDnUnits * n_cu || n_cu < sh.nb2) return hipErrorInvalidValue;
  return hipSuccess;
}

hipError_t launch_decode_stack(const RmoeLayer* const* layers, int n_layers, const uint16_t* x, uint16_t* out,
                               bool residual, int act, float gb, float vb, int32_t* ids_out, float* wts_out,
                               RmoeScratch& s, int n_cu, unsigned spin_limit, hipStream_t st) {
  if (n_layers < 1 || n_layers > kMaxStack) return hipErrorInvalidValue;
  const RmoeLayer& L0 = *layers[0];
  if (stack_check(L0, n_cu) != hipSuccess) return hipErrorInvalidValue;
  if (stack_scratch_bytes(L0, n_layers) > s.stack_bytes || stack_counter_count(L0, n_layers) > s.stack_cnt_n)
    return hipErrorInvalidValue;
  const StackShape sh = stack_shape(L0);
  StackArgs a{};
  a.L = n_layers;
  a.H = L0.H;
  a.I = L0.I;
  a.Ipad = L0.Ipad;
  a.E = L0.n_routed;
  a.k = L0.top_k;
  a.S = sh.S;
  a.score = L0.score;
  a.renorm = L0.renorm;
  a.scaling = L0.scaling;
  a.act = act;
  a.residual = residual ? 1 : 0;
  a.gb = gb;
  a.vb = vb;
  a.gu_bytes = L0.gu_bytes;
  a.dn_bytes = L0.dn_bytes;
  a.nb1 = sh.nb1;
  a.nb2 = sh.nb2;
  a.nkt1 = sh.nkt1;
  a.nkt2 = sh.nkt2;
  a.nhb = sh.nhb;
  a.n_gu = sh.n_gu;
  a.n_dn = sh.n_dn;
  a.Ep = (L0.n_routed + 31) / 32 * 32;
  a.gu_pre = sh.S > L0.top_k && gu_prefetch_fits(sh.nkt1) ? 1 : 0;
  a.x0 = x;
  a.out = out;
  a.ids_out = ids_out;
  a.wts_out = wts_out;
  a.scratch = s.stack;
  a.layer_bytes = sh.layer_bytes;
  a.off_lpart = sh.off_lpart;
  a.off_h = sh.off_h;
  a.off_dout = sh.off_dout;
  a.cnt = s.stack_cnt;
  a.cnt_stride = sh.cnt_stride;
  a.spin_limit = spin_limit ? spin_limit : kSpinLimit;
  a.err = s.err;
  for (int l = 0; l < n_layers; ++l) {
    const RmoeLayer& Ll = *layers[l];
    if (Ll.H != L0.H || Ll.I != L0.I || Ll.n_routed != L0.n_routed || Ll.n_shared != L0.n_shared ||
        Ll.top_k != L0.top_k || Ll.score != L0.score || Ll.renorm != L0.renorm || Ll.scaling != L0.scaling ||
        !Ll.has_router)
      return hipErrorInvalidValue;
    a.gu[l] = Ll.gu;
    a.dn[l] = Ll.dn;
    a.rw[l] = Ll.router_w;
    a.rb[l] = Ll.router_bias;
  }
  const size_t lds = dn_lds_bytes(sh.nkt2, L0.n_routed, sh.nkt1, a.gu_pre != 0);
  const dim3 grid(n_cu), block(kThreads);
  const int pos_need = (kMaxDnUnits * sh.nkt2 + kWaves - 2) / (kWaves - 1);
  if (pos_need <= 2 && a.E <= 128)
    hipLaunchKernelGGL((decode_stack_kernel<2, 1>), grid, block, lds, st, a);
  else if (a.E <= 128)
    hipLaunchKernelGGL((decode_stack_kernel<4, 1>), grid, block, lds, st, a);
  else
    hipLaunchKernelGGL((decode_stack_kernel<4, 2>), grid, block, lds, st, a);
  return hipGetLastError();
}

// Allow the largest dynamic LDS any instance takes, then report the resident workgroups
// per CU of the most demanding instance at that size.
hipError_t decode_stack_occupancy(int* blocks_per_cu) {
  const int dyn = (int)(kLdsLimit - kStaticLds);
  const void* fns[3] = {(const void*)decode_stack_kernel<2, 1>, (const void*)decode_stack_kernel<4, 1>,
                        (const void*)decode_stack_kernel<4, 2>};
  int best = 1 << 30;
  for (const void* f : fns) {
    hipError_t e = hipFuncSetAttribute(f, hipFuncAttributeMaxDynamicSharedMemorySize, dyn);
    if (e != hipSuccess) return e;
    int v = 0;
    e = hipOccupancyMaxActiveBlocksPerMultiprocessor(&v, f, kThreads, dyn);
    if (e != hipSuccess) return e;
    best = v < best ? v : best;
  }
  *blocks_per_cu = best;
  return hipSuccess;
}

}  // namespace rmoe
