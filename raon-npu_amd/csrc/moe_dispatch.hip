// Token dispatch: histogram -> exclusive scan -> stable scatter.
//
// Produces the flattened job order of build_plan (kernels/moe_grouped/planner.py:76-108):
// assignments (token, route) sorted by expert id ascending and, inside one expert,
// in row-major (token, route) order.  Chunks of 1,024 assignments are counted in
// parallel; a single workgroup turns the per-chunk counts into per-chunk bases; each
// chunk then places its assignments expert by expert in chunk order, which keeps the
// sort stable without any atomics on the output.
#include "rmoe_internal.h"

namespace rmoe {
namespace {

constexpr int kChunk = 1024;

__global__ __launch_bounds__(256) void dispatch_count_kernel(const int32_t* __restrict__ ids, int n, int E,
                                                             int32_t* __restrict__ counts, int* err) {
  __shared__ int hist[256];
  const int c = blockIdx.x;
  for (int e = threadIdx.x; e < E; e += blockDim.x) hist[e] = 0;
  __syncthreads();
  const int begin = c * kChunk, end = min(n, begin + kChunk);
  for (int i = begin + threadIdx.x; i < end; i += blockDim.x) {
    const int e = ids[i];
    if (e >= 0 && e < E) atomicAdd(&hist[e], 1);
    else atomicOr(err, 4);
  }
  __syncthreads();
  for (int e = threadIdx.x; e < E; e += blockDim.x) counts[(size_t)c * E + e] = hist[e];
}

// One workgroup: counts[c][e] -> bases[c][e] in place; offsets[e] (E + 1 entries).
__global__ __launch_bounds__(256) void dispatch_scan_kernel(int32_t* __restrict__ counts, int nchunks, int E,
                                                            int32_t* __restrict__ offsets) {
  __shared__ int tot[257];
  const int e = threadIdx.x;
  int total = 0;
  if (e < E)
    for (int c = 0; c < nchunks; ++c) total += counts[(size_t)c * E + e];
  if (e < E) tot[e] = total;
  __syncthreads();
  if (e == 0) {
    int run = 0;
    for (int q = 0; q < E; ++q) {
      const int v = tot[q];
      tot[q] = run;
      offsets[q] = run;
      run += v;
    }
    offsets[E] = run;
  }
  __syncthreads();
  if (e < E) {
    int run = tot[e];
    for (int c = 0; c < nchunks; ++c) {
      const int v = counts[(size_t)c * E + e];
      counts[(size_t)c * E + e] = run;
      run += v;
    }
  }
}

// Thread e walks the chunk in order and places its assignments.
__global__ __launch_bounds__(256) void dispatch_scatter_kernel(const int32_t* __restrict__ ids, int n, int E,
                                                               const int32_t* __restrict__ bases,
                                                               int32_t* __restrict__ order, int32_t* __restrict__ inv) {
  __shared__ int cid[kChunk];
  const int c = blockIdx.x;
  const int begin = c * kChunk, len = min(n - begin, kChunk);
  for (int i = threadIdx.x; i < len; i += blockDim.x) cid[i] = ids[begin + i];
  __syncthreads();
  const int e = threadIdx.x;
  if (e >= E) return;
  int pos = bases[(size_t)c * E + e];
  for (int i = 0; i < len; ++i) {
    if (cid[i] == e) {
      order[pos] = begin + i;
      if (inv) inv[begin + i] = pos;
      ++pos;
    }
  }
}

}  // namespace

hipError_t launch_dispatch(const int32_t* ids, int T, int k, int n_experts, int32_t* order, int32_t* inv,
                           int32_t* offsets, RmoeScratch& s, hipStream_t st) {
  const int n = T * k;
  const int nchunks = (n + kChunk - 1) / kChunk;
  if (n_experts < 1 || n_experts > 256) return hipErrorInvalidValue;
  if ((size_t)nchunks * n_experts > s.chunk_elems) return hipErrorInvalidValue;
  const int threads = ((n_experts + 63) / 64) * 64;
  hipLaunchKernelGGL(dispatch_count_kernel, dim3(nchunks), dim3(256), 0, st, ids, n, n_experts, s.chunk_counts,
                     s.err);
  hipError_t e = hipGetLastError();
  if (e != hipSuccess) return e;
  hipLaunchKernelGGL(dispatch_scan_kernel, dim3(1), dim3(256), 0, st, s.chunk_counts, nchunks, n_experts, offsets);
  e = hipGetLastError();
  if (e != hipSuccess) return e;
  hipLaunchKernelGGL(dispatch_scatter_kernel, dim3(nchunks), dim3(threads), 0, st, ids, n, n_experts, s.chunk_counts,
                     order, inv);
  return hipGetLastError();
}

}  // namespace rmoe
