// Token dispatch: histogram -> exclusive scan -> stable scatter.
//
// Produces the flattened job order of build_plan (kernels/moe_grouped/planner.py:76-108):
// assignments (token, route) sorted by expert id ascending and, inside one expert,
// in row-major (token, route) order.  Chunks of 1,024 assignments are counted in
// parallel; then each chunk's workgroup derives its own bases (the expert offsets, an
// exclusive scan of the per-expert totals, plus the counts of the chunks before it) and
// places its assignments: its 4 waves take 256 consecutive assignments each, rank lanes
// of equal expert with ballots (64 at a time, in order) and offset by the counts of the
// waves before, so the sort is stable without atomics on the output.
#include "rmoe_internal.h"

namespace rmoe {
namespace {

constexpr int kChunk = kDispatchChunk;

__global__ __launch_bounds__(256) void dispatch_count_kernel(const int32_t* __restrict__ ids, int n, int E,
                                                             int32_t* __restrict__ counts, int* err) {
  __shared__ int hist[256];
  const int c = blockIdx.x;
  hist[threadIdx.x] = 0;
  __syncthreads();
  const int begin = c * kChunk;
  int ev[kChunk / 256];
#pragma unroll
  for (int j = 0; j < kChunk / 256; ++j) {
    const int i = begin + 256 * j + threadIdx.x;
    ev[j] = i < n ? ids[i] : 0x7fffffff;
  }
#pragma unroll
  for (int j = 0; j < kChunk / 256; ++j) {
    if (ev[j] == 0x7fffffff) continue;
    if (ev[j] >= 0 && ev[j] < E) atomicAdd(&hist[ev[j]], 1);
    else atomicOr(err, 4);
  }
  __syncthreads();
  if ((int)threadIdx.x < E) counts[(size_t)c * E + threadIdx.x] = hist[threadIdx.x];
}

// counts[c][e]: assignments of chunk c routed to expert e.  Workgroup c also writes
// offsets[e] (E + 1 entries) when c == 0.
__global__ __launch_bounds__(256) void dispatch_scatter_kernel(const int32_t* __restrict__ ids, int n, int E,
                                                               const int32_t* __restrict__ counts, int nchunks,
                                                               int32_t* __restrict__ offsets,
                                                               int32_t* __restrict__ order, int32_t* __restrict__ inv,
                                                               uint32_t* __restrict__ tiles, int* __restrict__ ntiles,
                                                               int cap, int shared_rows) {
  __shared__ int slot[4][256];  // per wave: counts, then next output slot per expert
  __shared__ int wsum[4];
  const int c = blockIdx.x, tid = threadIdx.x, wave = wave_id(), lane = tid & 63;
  for (int i = tid; i < 4 * 256; i += 256) (&slot[0][0])[i] = 0;
  // This wave's assignments (loaded first, so that their latency overlaps the count reads).
  const int begin = c * kChunk + 256 * wave;
  int ev[4];
#pragma unroll
  for (int j = 0; j < 4; ++j) {
    const int i = begin + 64 * j + lane;
    ev[j] = i < n ? ids[i] : -1;
  }
  // Thread e: expert e's assignments in the chunks before this one and in all chunks;
  // the expert's offset is the exclusive scan of the totals (wave scans, then the four
  // wave sums).  The counts are read 32 chunks at a time, all loads in flight together.
  int before = 0, total = 0;
  if (tid < E) {
    for (int q0 = 0; q0 < nchunks; q0 += 32) {
      int v[32];
#pragma unroll
      for (int i = 0; i < 32; ++i) v[i] = q0 + i < nchunks ? counts[(size_t)(q0 + i) * E + tid] : 0;
#pragma unroll
      for (int i = 0; i < 32; ++i) {
        before += q0 + i < c ? v[i] : 0;
        total += v[i];
      }
    }
  }
  int incl = total;
#pragma unroll
  for (int d = 1; d < 64; d <<= 1) {
    const int y = __shfl_up(incl, d, 64);
    if (lane >= d) incl += y;
  }
  if (lane == 63) wsum[wave] = incl;
  unsigned long long same[4];
  __syncthreads();
  // Lanes of one round with the same expert agree on every bit of the id.
#pragma unroll
  for (int j = 0; j < 4; ++j) {
    const int e = ev[j];
    const bool ok = e >= 0 && e < E;
    unsigned long long m = __ballot(ok);
#pragma unroll
    for (int b = 0; b < 8; ++b) {
      const unsigned long long bb = __ballot((e >> b) & 1);
      m &= ((e >> b) & 1) ? bb : ~bb;
    }
    same[j] = ok ? m : 0ull;
    // The last lane of each expert group adds the group's size (one writer per expert).
    if (ok && (m >> lane) == 1ull) slot[wave][e] += __popcll(m);
  }
  __syncthreads();
  // Expert e's first slot for wave w: offset + earlier chunks + counts of waves 0..w-1.
  // (Thread E's exclusive prefix is the number of routed rows.)
  int woff = 0;
  for (int w = 0; w < wave; ++w) woff += wsum[w];
  const int offset = woff + incl - total;
  if (tid < E) {
    if (c == 0) {
      offsets[tid] = offset;
      if (tid == E - 1) offsets[E] = offset + total;
    }
    int run = offset + before;
#pragma unroll
    for (int w = 0; w < 4; ++w) {
      const int v = slot[w][tid];
      slot[w][tid] = run;
      run += v;
    }
  }
  __syncthreads();
#pragma unroll
  for (int j = 0; j < 4; ++j) {
    const int e = ev[j];
    if (same[j]) {
      const int pos = slot[wave][e] + __popcll(same[j] & ((1ull << lane) - 1ull));
      const int i = begin + 64 * j + lane;
      order[pos] = i;
      if (inv) inv[i] = pos;
    }
    if (same[j] && (same[j] >> lane) == 1ull) slot[wave][e] += __popcll(same[j]);
  }
  // The grouped GEMM's tile table (when asked for): routed group e holds sorted rows
  // [offset, offset + total); the shared group (shared_rows > 0) starts at row n (after
  // every assignment, whether or not its id was valid), where the GEMM places it.
  if (c == 0 && tiles) {
    __shared__ int tsum[kTileClasses][4];
    const int ng = E + (shared_rows > 0 ? 1 : 0);
    const int gb = tid < E ? offset : n;
    tile_table_block<4>(tid, ng, gb, gb + (tid < E ? total : shared_rows), tiles, ntiles, cap, tsum);
  }
}

}  // namespace

hipError_t launch_dispatch(const int32_t* ids, int T, int k, int n_experts, int32_t* order, int32_t* inv,
                           int32_t* offsets, RmoeScratch& s, hipStream_t st, uint32_t* tiles, int* ntiles, int cap,
                           int shared_rows, bool counted) {
  const int n = T * k;
  const int nchunks = (n + kChunk - 1) / kChunk;
  if (n_experts < 1 || n_experts > 256) return hipErrorInvalidValue;
  if (tiles && n_experts + (shared_rows > 0 ? 1 : 0) > 256) return hipErrorInvalidValue;
  if ((size_t)nchunks * n_experts > s.chunk_elems) return hipErrorInvalidValue;
  if (!counted) {
    hipLaunchKernelGGL(dispatch_count_kernel, dim3(nchunks), dim3(256), 0, st, ids, n, n_experts, s.chunk_counts,
                       s.err);
    hipError_t e = hipGetLastError();
    if (e != hipSuccess) return e;
  }
  hipLaunchKernelGGL(dispatch_scatter_kernel, dim3(nchunks), dim3(256), 0, st, ids, n, n_experts, s.chunk_counts,
                     nchunks, offsets, order, inv, tiles, ntiles, cap, shared_rows);
  return hipGetLastError();
}

}  // namespace rmoe
