// Device-wide exclusive scan of int32 counts and small helpers shared by the graph-building kernels
// (graph preparation, spatial order, neighbour list).  Everything has internal linkage.
#pragma once

#include "common.h"

namespace fsc {
namespace {

constexpr int SCAN_T = 256, SCAN_PER = 8, SCAN_TILE = SCAN_T * SCAN_PER;   // 2048 entries per block
constexpr int64_t SCAN_MAX_BLOCKS = 4 * 1024 * SCAN_PER;                   // totals scanned by one block

__global__ __launch_bounds__(256) void fill_i32_kernel(int32_t* __restrict__ p, int64_t n, int32_t v) {
  for (int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x; i < n; i += (int64_t)gridDim.x * 256) p[i] = v;
}

// Exclusive scan of cnt[0..n) into out[0..n] (out[n] = total) in three passes: per-block scans with block
// totals, one block scanning the totals, and the add-back.  blockIdx.y selects one of two arrays.
struct ScanArgs {
  const int32_t* cnt[2];
  int32_t* out[2];
  int32_t* tot[2];
  int64_t n;
};

__device__ __forceinline__ int32_t block_exclusive_scan(int32_t v, int32_t* lds, int32_t& total) {
  // 256 threads, wave64: scan in the wave, then across the 4 waves
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  int32_t x = v;
#pragma unroll
  for (int off = 1; off < 64; off <<= 1) {
    const int32_t y = __shfl_up(x, off, 64);
    if (lane >= off) x += y;
  }
  if (lane == 63) lds[wave] = x;
  __syncthreads();
  int32_t base = 0;
  for (int w = 0; w < wave; ++w) base += lds[w];
  total = lds[0] + lds[1] + lds[2] + lds[3];
  __syncthreads();
  return base + x - v;
}

__global__ __launch_bounds__(SCAN_T) void scan_blocks_kernel(ScanArgs a) {
  __shared__ int32_t lds[4];
  const int k = blockIdx.y;
  const int64_t base = (int64_t)blockIdx.x * SCAN_TILE + (int64_t)threadIdx.x * SCAN_PER;
  int32_t v[SCAN_PER], s = 0;
#pragma unroll
  for (int j = 0; j < SCAN_PER; ++j) {
    v[j] = (base + j < a.n) ? a.cnt[k][base + j] : 0;
    s += v[j];
  }
  int32_t total;
  int32_t run = block_exclusive_scan(s, lds, total);
#pragma unroll
  for (int j = 0; j < SCAN_PER; ++j) {
    if (base + j <= a.n) a.out[k][base + j] = run;
    run += v[j];
  }
  if (threadIdx.x == 0) a.tot[k][blockIdx.x] = total;
}

__global__ __launch_bounds__(1024) void scan_totals_kernel(ScanArgs a, int nblocks) {
  __shared__ int32_t lds[16];
  const int k = blockIdx.y;
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  constexpr int PER = (int)(SCAN_MAX_BLOCKS / 1024);
  int32_t v[PER], s = 0;
#pragma unroll
  for (int j = 0; j < PER; ++j) {
    const int idx = threadIdx.x * PER + j;
    v[j] = idx < nblocks ? a.tot[k][idx] : 0;
    s += v[j];
  }
  int32_t x = s;
#pragma unroll
  for (int off = 1; off < 64; off <<= 1) {
    const int32_t y = __shfl_up(x, off, 64);
    if (lane >= off) x += y;
  }
  if (lane == 63) lds[wave] = x;
  __syncthreads();
  int32_t base = 0;
  for (int w = 0; w < wave; ++w) base += lds[w];
  int32_t run = base + x - s;
#pragma unroll
  for (int j = 0; j < PER; ++j) {
    const int idx = threadIdx.x * PER + j;
    if (idx < nblocks) a.tot[k][idx] = run;
    run += v[j];
  }
}

__global__ __launch_bounds__(SCAN_T) void scan_add_kernel(ScanArgs a) {
  const int k = blockIdx.y;
  const int32_t add = a.tot[k][blockIdx.x];
  const int64_t base = (int64_t)blockIdx.x * SCAN_TILE + (int64_t)threadIdx.x * SCAN_PER;
#pragma unroll
  for (int j = 0; j < SCAN_PER; ++j)
    if (base + j <= a.n) a.out[k][base + j] += add;
}

inline unsigned grid_of(int64_t n) { return (unsigned)((n + 255) / 256); }

}  // namespace
}  // namespace fsc
