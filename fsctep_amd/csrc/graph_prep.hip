// Graph preparation on the device: receiver sort, receiver CSR, source grouping, species pairs and
// the species-pair tiles of the sparse conv1, with no host synchronisation and every output size a
// function of (N, E, n_species) only.  Replaces the per-call `argsort(edge_dst)` and permutation of
// the trunks (models/pure_cartesian_sparse_layers.py:745-748, models/pure_cartesian_ictd_layers_full.py:896-899,
// models/pure_cartesian_ictd_layers_o3.py:924-927), run on every forward as the reference does.
//
// The receiver order is the stable one (ties in original edge order), so the result is deterministic.
// Placement uses integer atomics per segment (counts, then cursors); the order inside a segment is then
// fixed by ranking each entry against the other entries of its segment (rank = number of smaller
// original ids), a sort of the segment that costs sum(deg^2) compares: ~27 M at 10k atoms (deg ~52).
#include "common.h"
#include "fsctep.h"
#include "scan.h"

#include <mutex>
#include <string>

namespace fsc {
constexpr int64_t kScratchInts = int64_t(1) << 23;
}
// Static workspace of fsc_graph_prepare_noalloc: 2^23 int32 (32 MiB) on every GPU the library runs on,
// held from the first load of this code object on that device until the process ends.
static __device__ __align__(256) int32_t scratch[fsc::kScratchInts];

namespace fsc {
namespace {

// Range checks (out-of-range ids are clamped so every later access stays in bounds; `status` gets a bit),
// in/out degree counts, and the node species ids.
__global__ __launch_bounds__(256) void count_kernel(int64_t E, int64_t N, const int64_t* __restrict__ src,
                                                    const int64_t* __restrict__ dst, int32_t* __restrict__ cnt_in,
                                                    int32_t* __restrict__ cnt_out, int32_t NS,
                                                    const int64_t* __restrict__ species,
                                                    int32_t* __restrict__ node_species, int32_t* __restrict__ status) {
  const int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x;
  if (i < E) {
    int64_t s = src[i], d = dst[i];
    if (s < 0 || s >= N || d < 0 || d >= N) {
      atomicOr(status, 1);
      s = s < 0 ? 0 : (s >= N ? N - 1 : s);
      d = d < 0 ? 0 : (d >= N ? N - 1 : d);
    }
    atomicAdd(cnt_in + d, 1);
    atomicAdd(cnt_out + s, 1);
  }
  if (NS > 0 && i < N) {
    int64_t a = species[i];
    if (a < 0 || a >= NS) {
      atomicOr(status, 2);
      a = a < 0 ? 0 : NS - 1;
    }
    node_species[i] = (int32_t)a;
  }
}

__device__ __forceinline__ int64_t clamp_id(int64_t v, int64_t N) { return v < 0 ? 0 : (v >= N ? N - 1 : v); }

// Unordered placement of each edge into its receiver segment.
__global__ __launch_bounds__(256) void place_dst_kernel(int64_t E, int64_t N, const int64_t* __restrict__ dst,
                                                        const int32_t* __restrict__ dst_ptr,
                                                        int32_t* __restrict__ cursor, int32_t* __restrict__ tmp) {
  const int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x;
  if (i >= E) return;
  const int64_t d = clamp_id(dst[i], N);
  tmp[dst_ptr[d] + atomicAdd(cursor + d, 1)] = (int32_t)i;
}

// Final receiver order: each entry's rank among the original ids of its segment.  Writes the permutation
// and the permuted source / receiver ids and species pair.
__global__ __launch_bounds__(256) void rank_dst_kernel(int64_t E, int64_t N, const int64_t* __restrict__ src,
                                                       const int64_t* __restrict__ dst,
                                                       const int32_t* __restrict__ dst_ptr,
                                                       const int32_t* __restrict__ tmp, int32_t NS,
                                                       const int32_t* __restrict__ node_species,
                                                       int32_t* __restrict__ order, int32_t* __restrict__ src32,
                                                       int32_t* __restrict__ dst32, int32_t* __restrict__ edge_pair) {
  const int64_t p = (int64_t)blockIdx.x * 256 + threadIdx.x;
  if (p >= E) return;
  const int32_t i = tmp[p];
  const int64_t d = clamp_id(dst[i], N), s = clamp_id(src[i], N);
  const int32_t a = dst_ptr[d], b = dst_ptr[d + 1];
  int32_t rank = 0;
  for (int32_t q = a; q < b; ++q) rank += tmp[q] < i;
  const int32_t o = a + rank;
  order[o] = i;
  src32[o] = (int32_t)s;
  dst32[o] = (int32_t)d;
  if (NS > 0) edge_pair[o] = node_species[s] * NS + node_species[d];
}

__global__ __launch_bounds__(256) void place_src_kernel(int64_t E, const int32_t* __restrict__ src32,
                                                        const int32_t* __restrict__ src_ptr,
                                                        int32_t* __restrict__ cursor, int32_t* __restrict__ tmp) {
  const int64_t p = (int64_t)blockIdx.x * 256 + threadIdx.x;
  if (p >= E) return;
  const int32_t s = src32[p];
  tmp[src_ptr[s] + atomicAdd(cursor + s, 1)] = (int32_t)p;
}

__global__ __launch_bounds__(256) void rank_src_kernel(int64_t E, const int32_t* __restrict__ src32,
                                                       const int32_t* __restrict__ src_ptr,
                                                       const int32_t* __restrict__ tmp,
                                                       int32_t* __restrict__ src_perm) {
  const int64_t q = (int64_t)blockIdx.x * 256 + threadIdx.x;
  if (q >= E) return;
  const int32_t p = tmp[q];
  const int32_t s = src32[p];
  const int32_t a = src_ptr[s], b = src_ptr[s + 1];
  int32_t rank = 0;
  for (int32_t k = a; k < b; ++k) rank += tmp[k] < p;
  src_perm[a + rank] = p;
}

// Species-pair tiles: the receiver-sorted positions grouped by pair, ascending within a pair (a stable
// counting sort by pair, so the layout is deterministic).  Positions are cut into chunks of PAIR_CHUNK;
// per-chunk pair counts are scanned over the chunks for every pair, one block lays the pairs' tiles out
// back to back (each pair's list padded to a multiple of 16), and one wave per chunk places its positions.
constexpr int PAIR_CHUNK = 2048;

// cnt_blk[pr * nchunk + b] = number of positions of chunk b with pair pr (LDS counters).
__global__ __launch_bounds__(256) void pair_chunk_count_kernel(int64_t E, int32_t P, int nchunk,
                                                               const int32_t* __restrict__ edge_pair,
                                                               int32_t* __restrict__ cnt_blk) {
  __shared__ int32_t h[256];
  h[threadIdx.x] = 0;
  __syncthreads();
  const int64_t base = (int64_t)blockIdx.x * PAIR_CHUNK;
  for (int j = threadIdx.x; j < PAIR_CHUNK; j += 256)
    if (base + j < E) atomicAdd(&h[edge_pair[base + j]], 1);
  __syncthreads();
  if ((int)threadIdx.x < P) cnt_blk[(int64_t)threadIdx.x * nchunk + blockIdx.x] = h[threadIdx.x];
}

// One block per pair: exclusive scan of its chunk counts in place; the pair's total into pcnt.
__global__ __launch_bounds__(256) void pair_chunk_scan_kernel(int nchunk, int32_t* __restrict__ cnt_blk,
                                                              int32_t* __restrict__ pcnt) {
  __shared__ int32_t lds[4];
  int32_t* row = cnt_blk + (int64_t)blockIdx.x * nchunk;
  int32_t carry = 0;
  for (int base = 0; base < nchunk; base += 256) {   // uniform trip count over the block
    const int i = base + (int)threadIdx.x;
    const int32_t v = i < nchunk ? row[i] : 0;
    int32_t total;
    const int32_t ex = block_exclusive_scan(v, lds, total);
    if (i < nchunk) row[i] = carry + ex;
    carry += total;
  }
  if (threadIdx.x == 0) pcnt[blockIdx.x] = carry;
}

__global__ __launch_bounds__(256) void pair_layout_kernel(int32_t P, const int32_t* __restrict__ pcnt,
                                                          int32_t* __restrict__ tstart, int64_t T_max,
                                                          int32_t* __restrict__ tpair) {
  __shared__ int32_t lds[4];
  __shared__ int32_t s_start[256];
  __shared__ int32_t s_total;
  const int t = threadIdx.x;
  const int32_t tiles = t < P ? (pcnt[t] + 15) / 16 : 0;
  int32_t total;
  const int32_t start = block_exclusive_scan(tiles, lds, total);
  if (t < P) tstart[t] = start;
  s_start[t] = start;
  if (t == 0) s_total = total;
  __syncthreads();
  // tile -> pair (tiles past the used ones: pair 0, all ids -1)
  for (int64_t k = t; k < T_max; k += 256) {
    int32_t pr = 0;
    if (k < s_total) {
      int lo = 0, hi = P - 1;   // last pair whose start <= k (pairs without tiles share a start)
      while (lo < hi) {
        const int mid = (lo + hi + 1) >> 1;
        if (s_start[mid] <= k) lo = mid; else hi = mid - 1;
      }
      pr = lo;
    }
    tpair[k] = pr;
  }
}

// One wave per chunk, 64 positions at a time in order.  A position's slot = its pair's first slot + the
// chunk's offset within the pair + the pair's count earlier in the chunk (run) + its rank among the lanes
// holding the same pair (lanes matched by ballots over the 8 bits of the pair id).
__global__ __launch_bounds__(64) void pair_chunk_place_kernel(int64_t E, int nchunk,
                                                              const int32_t* __restrict__ edge_pair,
                                                              const int32_t* __restrict__ tstart,
                                                              const int32_t* __restrict__ cnt_blk,
                                                              int32_t* __restrict__ ids) {
  __shared__ int32_t run[256];
  const int lane = threadIdx.x;
  for (int k = lane; k < 256; k += 64) run[k] = 0;
  __syncthreads();
  const int64_t base = (int64_t)blockIdx.x * PAIR_CHUNK;
  const uint64_t below = lane == 0 ? 0ull : (~0ull >> (64 - lane));
  for (int j = 0; j < PAIR_CHUNK && base + j < E; j += 64) {   // uniform over the wave
    const int64_t p = base + j + lane;
    const bool valid = p < E;
    const int pr = valid ? edge_pair[p] : 0;
    uint64_t same = __ballot(valid);
#pragma unroll
    for (int bit = 0; bit < 8; ++bit) {
      const bool b = (pr >> bit) & 1;
      const uint64_t bb = __ballot(b);
      same &= b ? bb : ~bb;
    }
    if (valid)
      ids[(int64_t)tstart[pr] * 16 + cnt_blk[(int64_t)pr * nchunk + blockIdx.x] + run[pr] + __popcll(same & below)] =
          (int32_t)p;
    __syncthreads();                                             // every lane has read run[] for this step
    if (valid && (same >> lane) == 1ull) run[pr] += __popcll(same);   // the pair's highest lane
    __syncthreads();
  }
}


// ---------------------------------------------------------------- spatial node order
// A permutation of the atoms along a Morton (Z-order) curve over a G x G x G grid spanning the bounding
// box of the positions (G the smallest power of two with 2 G^3 >= N, at most 256), atoms of one cell in
// ascending id: a counting sort by cell with the same place-then-rank step as the receiver sort, so the
// order is deterministic.  Kernels that run one block per node walk this order, XCD by XCD, so that the
// blocks an XCD runs together gather the features of the same neighbourhood.  Degenerate positions
// (all equal, e.g. the zero positions of an edge-vector caller) give the identity; non-finite ones cell 0.
__global__ __launch_bounds__(1024) void bbox_kernel(int64_t N, const float* __restrict__ pos, float* __restrict__ box) {
  __shared__ float red[16][6];
  float v[6] = {INFINITY, INFINITY, INFINITY, -INFINITY, -INFINITY, -INFINITY};
  for (int64_t i = threadIdx.x; i < N; i += 1024) {
#pragma unroll
    for (int k = 0; k < 3; ++k) {
      const float x = pos[3 * i + k];
      if (isfinite(x)) {
        v[k] = fminf(v[k], x);
        v[3 + k] = fmaxf(v[3 + k], x);
      }
    }
  }
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
#pragma unroll
  for (int k = 0; k < 6; ++k) {
    for (int off = 32; off > 0; off >>= 1) {
      const float o = __shfl_xor(v[k], off, 64);
      v[k] = k < 3 ? fminf(v[k], o) : fmaxf(v[k], o);
    }
    if (lane == 0) red[wave][k] = v[k];
  }
  __syncthreads();
  if (threadIdx.x < 6) {
    const int k = threadIdx.x;
    float r = red[0][k];
    for (int w = 1; w < 16; ++w) r = k < 3 ? fminf(r, red[w][k]) : fmaxf(r, red[w][k]);
    box[k] = r;
  }
}

__device__ __forceinline__ uint32_t spread3(uint32_t v) {   // bit b of v (b < 8) to bit 3b
  v &= 0xffu;
  v = (v | (v << 8)) & 0x0f00fu;
  v = (v | (v << 4)) & 0x0c30c3u;
  v = (v | (v << 2)) & 0x249249u;
  return v;
}

__global__ __launch_bounds__(256) void cell_kernel(int64_t N, const float* __restrict__ pos,
                                                   const float* __restrict__ box, int G,
                                                   int32_t* __restrict__ code, int32_t* __restrict__ cnt) {
  const int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x;
  if (i >= N) return;
  uint32_t c[3];
#pragma unroll
  for (int k = 0; k < 3; ++k) {
    const float lo = box[k], hi = box[3 + k];
    const float t = (hi > lo) ? (pos[3 * i + k] - lo) * ((float)G / (hi - lo)) : 0.f;
    const float tc = fminf(fmaxf(t, 0.f), (float)(G - 1));   // NaN -> 0
    c[k] = (uint32_t)tc;
  }
  const int32_t m = (int32_t)(spread3(c[0]) | (spread3(c[1]) << 1) | (spread3(c[2]) << 2));
  code[i] = m;
  atomicAdd(cnt + m, 1);
}

__global__ __launch_bounds__(256) void place_cell_kernel(int64_t N, const int32_t* __restrict__ code,
                                                         const int32_t* __restrict__ cell_ptr,
                                                         int32_t* __restrict__ cursor, int32_t* __restrict__ tmp) {
  const int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x;
  if (i >= N) return;
  const int32_t c = code[i];
  tmp[cell_ptr[c] + atomicAdd(cursor + c, 1)] = (int32_t)i;
}

__global__ __launch_bounds__(256) void rank_cell_kernel(int64_t N, const int32_t* __restrict__ code,
                                                        const int32_t* __restrict__ cell_ptr,
                                                        const int32_t* __restrict__ tmp, int32_t* __restrict__ order) {
  const int64_t p = (int64_t)blockIdx.x * 256 + threadIdx.x;
  if (p >= N) return;
  const int32_t i = tmp[p];
  const int32_t c = code[i];
  const int32_t a = cell_ptr[c], b = cell_ptr[c + 1];
  int32_t rank = 0;
  for (int32_t q = a; q < b; ++q) rank += tmp[q] < i;
  order[a + rank] = i;
}

int order_grid(int64_t N) {
  int G = 1;
  while (G < 256 && 2LL * G * G * G < N) G *= 2;
  return G;
}

struct OrderWs {
  int64_t box, cnt, cur, cell_ptr, tot, code, tmp, total, cells, nb;
};

OrderWs order_ws(int64_t N) {
  OrderWs w;
  const int64_t G = order_grid(N);
  w.cells = G * G * G;
  w.nb = (w.cells + 1 + SCAN_TILE - 1) / SCAN_TILE;
  int64_t o = 0;
  w.cnt = o;      o += w.cells;
  w.cur = o;      o += w.cells;    // the zero-filled prefix ends here
  w.box = o;      o += 8;
  w.cell_ptr = o; o += w.cells + 1;
  w.tot = o;      o += w.nb;
  w.code = o;     o += N;
  w.tmp = o;      o += N;
  w.total = o;
  return w;
}



struct WsLayout {
  int64_t cnt_in, cnt_out, cur_in, cur_out, tot, pcnt, tstart, cnt_blk, tmp, total, nchunk;
};

WsLayout ws_layout(int64_t N, int64_t E, int32_t NS) {
  WsLayout w;
  const int64_t nb = (N + 1 + SCAN_TILE - 1) / SCAN_TILE;
  const int64_t P = (int64_t)NS * NS;
  int64_t o = 0;
  w.nchunk = NS > 0 ? (E + PAIR_CHUNK - 1) / PAIR_CHUNK : 0;
  w.cnt_in = o;  o += N;
  w.cnt_out = o; o += N;
  w.cur_in = o;  o += N;
  w.cur_out = o; o += N;   // the zero-filled prefix ends here
  w.tot = o;     o += 2 * nb;
  w.pcnt = o;    o += P;
  w.tstart = o;  o += P;
  w.cnt_blk = o; o += P * w.nchunk;
  w.tmp = o;     o += E;
  w.total = o;
  return w;
}

// The device address of `scratch` (the static workspace of fsc_graph_prepare_noalloc) on the current
// device, resolved once per device with hipGetSymbolAddress.  In host code the array's name is a
// stand-in, not a device address: only this pointer is ever passed to a kernel.
int scratch_ptr(int32_t** out) {
  constexpr int kMaxDevices = 64;
  static std::mutex mu;
  static int32_t* ptrs[kMaxDevices] = {};
  int dev = -1;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= kMaxDevices) {
    set_error("fsc_graph_prepare_noalloc: no current HIP device (or device id >= 64)");
    return 1;
  }
  std::lock_guard<std::mutex> lk(mu);
  if (!ptrs[dev]) {
    void* p = nullptr;
    const hipError_t err = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
    if (err != hipSuccess || !p) {
      set_error(std::string("fsc_graph_prepare_noalloc: hipGetSymbolAddress(scratch) failed: ") +
                hipGetErrorString(err));
      return 1;
    }
    ptrs[dev] = static_cast<int32_t*>(p);
  }
  *out = ptrs[dev];
  return 0;
}

}  // namespace

static int prepare_impl(const char* name, int64_t n_nodes, int64_t n_edges, int32_t n_species, const int64_t* edge_src,
                 const int64_t* edge_dst, const int64_t* species, int32_t* order, int32_t* src32, int32_t* dst32,
                 int32_t* dst_ptr, int32_t* src_ptr, int32_t* src_perm, int32_t* node_species, int32_t* edge_pair,
                 int32_t* pair_tiles, int32_t* status, int32_t* workspace, hipStream_t stream) {
  const std::string nm(name);
  int64_t T_max = 0, ws_ints = 0;
  if (fsc_graph_sizes(n_nodes, n_edges, n_species, &T_max, &ws_ints)) return 1;
  const int64_t N = n_nodes, E = n_edges;
  FSC_CHECK_ARG(dst_ptr && src_ptr && status, nm + ": null pointer");
  FSC_CHECK_ARG(E == 0 || (N > 0 && edge_src && edge_dst && order && src32 && dst32 && src_perm),
                nm + ": null edge pointer (or edges without nodes)");
  FSC_CHECK_ARG(n_species == 0 || N == 0 || (species && node_species), nm + ": null species pointer");
  FSC_CHECK_ARG(n_species == 0 || E == 0 || edge_pair, nm + ": null edge_pair");
  FSC_CHECK_ARG(n_species == 0 || pair_tiles, nm + ": null pair_tiles");
  const int64_t nb = (N + 1 + SCAN_TILE - 1) / SCAN_TILE;
  FSC_CHECK_ARG(nb <= SCAN_MAX_BLOCKS, nm + ": too many nodes for the scan");
  const WsLayout w = ws_layout(N, E, n_species);
  const int32_t P = n_species * n_species;
  int32_t* ws = workspace;

  if (w.tot > 0) fill_i32_kernel<<<grid_of(w.tot) < 1024 ? grid_of(w.tot) : 1024, 256, 0, stream>>>(ws, w.tot, 0);
  fill_i32_kernel<<<1, 256, 0, stream>>>(status, 1, 0);
  const int64_t cn = E > N ? E : N;
  if (cn > 0)
    count_kernel<<<grid_of(cn), 256, 0, stream>>>(E, N, edge_src, edge_dst, ws + w.cnt_in, ws + w.cnt_out, n_species,
                                                  species, node_species, status);
  ScanArgs sa;
  sa.cnt[0] = ws + w.cnt_in;  sa.out[0] = dst_ptr; sa.tot[0] = ws + w.tot;
  sa.cnt[1] = ws + w.cnt_out; sa.out[1] = src_ptr; sa.tot[1] = ws + w.tot + nb;
  sa.n = N;
  scan_blocks_kernel<<<dim3((unsigned)nb, 2), SCAN_T, 0, stream>>>(sa);
  scan_totals_kernel<<<dim3(1, 2), 1024, 0, stream>>>(sa, (int)nb);
  scan_add_kernel<<<dim3((unsigned)nb, 2), SCAN_T, 0, stream>>>(sa);
  if (E > 0) {
    place_dst_kernel<<<grid_of(E), 256, 0, stream>>>(E, N, edge_dst, dst_ptr, ws + w.cur_in, ws + w.tmp);
    rank_dst_kernel<<<grid_of(E), 256, 0, stream>>>(E, N, edge_src, edge_dst, dst_ptr, ws + w.tmp, n_species,
                                                    node_species, order, src32, dst32, edge_pair);
    place_src_kernel<<<grid_of(E), 256, 0, stream>>>(E, src32, src_ptr, ws + w.cur_out, ws + w.tmp);
    rank_src_kernel<<<grid_of(E), 256, 0, stream>>>(E, src32, src_ptr, ws + w.tmp, src_perm);
  }
  if (n_species > 0) {
    fill_i32_kernel<<<grid_of(16 * T_max) < 1024 ? grid_of(16 * T_max) : 1024, 256, 0, stream>>>(pair_tiles,
                                                                                                 16 * T_max, -1);
    const int nchunk = (int)w.nchunk;
    if (E > 0)
      pair_chunk_count_kernel<<<nchunk, 256, 0, stream>>>(E, P, nchunk, edge_pair, ws + w.cnt_blk);
    pair_chunk_scan_kernel<<<P, 256, 0, stream>>>(nchunk, ws + w.cnt_blk, ws + w.pcnt);
    pair_layout_kernel<<<1, 256, 0, stream>>>(P, ws + w.pcnt, ws + w.tstart, T_max, pair_tiles + 16 * T_max);
    if (E > 0)
      pair_chunk_place_kernel<<<nchunk, 64, 0, stream>>>(E, nchunk, edge_pair, ws + w.tstart, ws + w.cnt_blk,
                                                          pair_tiles);
  }
  return check_launch(name) ? 2 : 0;
}


}  // namespace fsc

extern "C" {

int fsc_graph_sizes(int64_t n_nodes, int64_t n_edges, int32_t n_species, int64_t* n_tiles_max,
                    int64_t* workspace_ints) {
  FSC_CHECK_ARG(n_tiles_max && workspace_ints, "fsc_graph_sizes: null pointer");
  FSC_CHECK_ARG(n_nodes >= 0 && n_edges >= 0 && n_nodes < (1LL << 31) - 1 && n_edges < (1LL << 31) - 1,
                "fsc_graph_sizes: graph exceeds int32 indexing");
  FSC_CHECK_ARG(n_species >= 0 && n_species <= 16, "fsc_graph_sizes: n_species must be 0..16");
  *n_tiles_max = n_species > 0 ? (n_edges + 15) / 16 + (int64_t)n_species * n_species : 0;
  *workspace_ints = fsc::ws_layout(n_nodes, n_edges, n_species).total;
  return 0;
}

int fsc_spatial_order_workspace(int64_t n_nodes, int64_t* workspace_ints) {
  FSC_CHECK_ARG(workspace_ints, "fsc_spatial_order_workspace: null pointer");
  FSC_CHECK_ARG(n_nodes >= 0 && n_nodes < (1LL << 31) - 1, "fsc_spatial_order_workspace: bad node count");
  *workspace_ints = fsc::order_ws(n_nodes).total;
  return 0;
}

int fsc_spatial_order(int64_t n_nodes, const float* pos, int32_t* order, int32_t* workspace, hipStream_t stream) {
  using namespace fsc;
  FSC_CHECK_ARG(n_nodes >= 0 && n_nodes < (1LL << 31) - 1, "fsc_spatial_order: bad node count");
  if (n_nodes == 0) return 0;
  FSC_CHECK_ARG(pos && order && workspace, "fsc_spatial_order: null pointer");
  const int64_t N = n_nodes;
  const OrderWs w = order_ws(N);
  FSC_CHECK_ARG(w.nb <= SCAN_MAX_BLOCKS, "fsc_spatial_order: too many cells for the scan");
  int32_t* ws = workspace;
  float* box = reinterpret_cast<float*>(ws + w.box);
  fill_i32_kernel<<<grid_of(w.box) < 1024 ? grid_of(w.box) : 1024, 256, 0, stream>>>(ws, w.box, 0);
  bbox_kernel<<<1, 1024, 0, stream>>>(N, pos, box);
  cell_kernel<<<grid_of(N), 256, 0, stream>>>(N, pos, box, order_grid(N), ws + w.code, ws + w.cnt);
  ScanArgs sa;
  sa.cnt[0] = sa.cnt[1] = ws + w.cnt;
  sa.out[0] = sa.out[1] = ws + w.cell_ptr;
  sa.tot[0] = sa.tot[1] = ws + w.tot;
  sa.n = w.cells;
  scan_blocks_kernel<<<dim3((unsigned)w.nb, 1), SCAN_T, 0, stream>>>(sa);
  scan_totals_kernel<<<dim3(1, 1), 1024, 0, stream>>>(sa, (int)w.nb);
  scan_add_kernel<<<dim3((unsigned)w.nb, 1), SCAN_T, 0, stream>>>(sa);
  place_cell_kernel<<<grid_of(N), 256, 0, stream>>>(N, ws + w.code, ws + w.cell_ptr, ws + w.cur, ws + w.tmp);
  rank_cell_kernel<<<grid_of(N), 256, 0, stream>>>(N, ws + w.code, ws + w.cell_ptr, ws + w.tmp, order);
  return check_launch("fsc_spatial_order") ? 2 : 0;
}

int fsc_graph_prepare(int64_t n_nodes, int64_t n_edges, int32_t n_species, const int64_t* edge_src,
                      const int64_t* edge_dst, const int64_t* species, int32_t* order, int32_t* src32,
                      int32_t* dst32, int32_t* dst_ptr, int32_t* src_ptr, int32_t* src_perm,
                      int32_t* node_species, int32_t* edge_pair, int32_t* pair_tiles, int32_t* status,
                      int32_t* workspace, hipStream_t stream) {
  FSC_CHECK_ARG(workspace, "fsc_graph_prepare: null workspace");
  return fsc::prepare_impl("fsc_graph_prepare", n_nodes, n_edges, n_species, edge_src, edge_dst, species, order, src32,
                           dst32, dst_ptr, src_ptr, src_perm, node_species, edge_pair, pair_tiles, status, workspace,
                           stream);
}

int fsc_graph_prepare_noalloc(int64_t n_nodes, int64_t n_edges, int32_t n_species, const int64_t* edge_src,
                              const int64_t* edge_dst, const int64_t* species, int32_t* order, int32_t* src32,
                              int32_t* dst32, int32_t* dst_ptr, int32_t* src_ptr, int32_t* src_perm,
                              int32_t* node_species, int32_t* edge_pair, int32_t* pair_tiles, int32_t* status,
                              hipStream_t stream) {
  int64_t T_max = 0, ws_ints = 0;
  if (fsc_graph_sizes(n_nodes, n_edges, n_species, &T_max, &ws_ints)) return 1;
  if (ws_ints > fsc::kScratchInts) {
    fsc::set_error("fsc_graph_prepare_noalloc: the graph needs " + std::to_string(ws_ints) +
                   " int32 of workspace, above the static scratch of " + std::to_string(fsc::kScratchInts) +
                   " (about 4N + E + n_species^2 (2 + E/2048)); use fsc_graph_prepare with a caller workspace");
    return 1;
  }
  int32_t* ws = nullptr;
  if (fsc::scratch_ptr(&ws)) return 1;
  return fsc::prepare_impl("fsc_graph_prepare_noalloc", n_nodes, n_edges, n_species, edge_src, edge_dst, species,
                           order, src32, dst32, dst_ptr, src_ptr, src_perm, node_species, edge_pair, pair_tiles,
                           status, ws, stream);
}

}  // extern "C"
