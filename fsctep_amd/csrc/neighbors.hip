// Radius graph on the device with periodic images: a cell list over the bounding box of the positions.
// Replaces radius_graph_pbc_gpu (utils/graph_utils.py:192-257: one torch_cluster.radius call per image
// shift s in {-1,0,1} on each periodic axis) and the host loop that turns the LAMMPS neighbour list into
// edges (lammps_user_mfftorch/src/USER-MFFTORCH/pair_mff_torch.cpp:597-641).
//
// The edge set is every (src i, dst j, s) with s_k in {-1,0,1} on periodic axes (0 otherwise), not
// (i == j and s == 0), and |(pos_j - pos_i) + s.cell|^2 < r^2, evaluated in double precision in that
// order with no fused multiply-adds (cell rows are the lattice vectors, as in the reference).  Edges come
// out receiver-sorted and, within a receiver, ascending in (src, s_x, s_y, s_z): a deterministic order,
// so graph preparation's stable receiver sort keeps it.
//
// Steps: bounding box and grid (cells of side >= r where the cell budget allows), atoms bucketed by cell
// (counting sort), 16 lanes per receiver counting its neighbours over the image points pos_j + s.cell
// (the lanes split each cell's candidates), a scan into the receiver CSR (the caller reads the edge count),
// then the same walk writing (src, s) keys, and a per-receiver rank sort of the keys.
#include "common.h"
#include "fsctep.h"
#include "scan.h"

namespace fsc {
namespace nbr {
namespace {

struct GridParams {
  double lo[3], hi[3], h[3];
  int32_t G[3];
  int32_t pad;
};

constexpr int KEY_IMAGES = 27;   // key = src * 27 + (sx+1)*9 + (sy+1)*3 + (sz+1)

__device__ __forceinline__ double dmul(double a, double b) { return __dmul_rn(a, b); }
__device__ __forceinline__ double dadd(double a, double b) { return __dadd_rn(a, b); }

__global__ __launch_bounds__(1024) void bbox_kernel(int64_t N, const double* __restrict__ pos, double* __restrict__ box) {
  __shared__ double red[16][6];
  double v[6] = {INFINITY, INFINITY, INFINITY, -INFINITY, -INFINITY, -INFINITY};
  for (int64_t i = threadIdx.x; i < N; i += 1024) {
#pragma unroll
    for (int k = 0; k < 3; ++k) {
      const double x = pos[3 * i + k];
      if (isfinite(x)) {
        v[k] = fmin(v[k], x);
        v[3 + k] = fmax(v[3 + k], x);
      }
    }
  }
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
#pragma unroll
  for (int k = 0; k < 6; ++k) {
    for (int off = 32; off > 0; off >>= 1) {
      const double o = __shfl_xor(v[k], off, 64);
      v[k] = k < 3 ? fmin(v[k], o) : fmax(v[k], o);
    }
    if (lane == 0) red[wave][k] = v[k];
  }
  __syncthreads();
  if (threadIdx.x < 6) {
    const int k = threadIdx.x;
    double r = red[0][k];
    for (int w = 1; w < 16; ++w) r = k < 3 ? fmin(r, red[w][k]) : fmax(r, red[w][k]);
    box[k] = r;
  }
}

// One thread: grid dimensions G_k = max(1, floor(extent_k / r)) (so cells are at least r wide), halving the
// largest while the product exceeds the cell budget.
__global__ void grid_kernel(const double* __restrict__ box, double r, int64_t cells_max, GridParams* __restrict__ g) {
  if (threadIdx.x != 0 || blockIdx.x != 0) return;
  int64_t G[3];
  for (int k = 0; k < 3; ++k) {
    double lo = box[k], hi = box[3 + k];
    if (!(hi >= lo)) lo = hi = 0.0;   // no finite coordinate on this axis
    const double ext = hi - lo;
    double gk = floor(ext / r);
    gk = gk < 1.0 ? 1.0 : (gk > 1024.0 ? 1024.0 : gk);
    G[k] = (int64_t)gk;
    g->lo[k] = lo;
    g->hi[k] = hi;
  }
  while (G[0] * G[1] * G[2] > cells_max) {
    int m = 0;
    if (G[1] > G[m]) m = 1;
    if (G[2] > G[m]) m = 2;
    G[m] = G[m] > 1 ? G[m] / 2 : 1;
  }
  for (int k = 0; k < 3; ++k) {
    const double ext = g->hi[k] - g->lo[k];
    g->G[k] = (int32_t)G[k];
    g->h[k] = ext > 0.0 ? ext / (double)G[k] : 1.0;
  }
  g->pad = 0;
}

// Cell coordinate along axis k: floor((x - lo) / h) clamped to [0, G-1]; monotone in x, NaN -> 0.
__device__ __forceinline__ int cell_coord(const GridParams& g, int k, double x) {
  const double t = (x - g.lo[k]) / g.h[k];
  if (!(t >= 0.0)) return 0;
  if (t >= (double)(g.G[k] - 1)) return g.G[k] - 1;
  return (int)t;
}

__global__ __launch_bounds__(256) void assign_kernel(int64_t N, const double* __restrict__ pos,
                                                     const GridParams* __restrict__ gp, int32_t* __restrict__ atom_cell,
                                                     int32_t* __restrict__ cnt) {
  const int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x;
  if (i >= N) return;
  const GridParams g = *gp;
  const int c = (cell_coord(g, 0, pos[3 * i]) * g.G[1] + cell_coord(g, 1, pos[3 * i + 1])) * g.G[2] +
                cell_coord(g, 2, pos[3 * i + 2]);
  atom_cell[i] = c;
  atomicAdd(cnt + c, 1);
}

__global__ __launch_bounds__(256) void place_kernel(int64_t N, const int32_t* __restrict__ atom_cell,
                                                    const int32_t* __restrict__ cell_start, int32_t* __restrict__ cursor,
                                                    int32_t* __restrict__ cell_atoms) {
  const int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x;
  if (i >= N) return;
  const int32_t c = atom_cell[i];
  cell_atoms[cell_start[c] + atomicAdd(cursor + c, 1)] = (int32_t)i;
}

struct Walk {
  const double* pos;
  const double* cell;   // [3][3], rows = lattice vectors
  const GridParams* grid;
  const int32_t* cell_start;
  const int32_t* cell_atoms;
  int64_t N;
  int32_t pbc[3];
  double r2, reach;     // r^2 for the test; r (1 + 1e-9) for the cell range
};

// A group of RL = 16 consecutive lanes per receiver j (four receivers per wave) visits every (i, s) within
// r of j (see the file comment).  The loops over the image shifts and the cells in range are uniform in
// the group; its lanes split each cell's atoms (16 candidates per step, about a cell's content at the
// benchmark densities), and a step's hits are numbered in lane order by a ballot and a prefix popcount
// over the group's bits.  For each step with hits, f(hit, i, key, rank, count) is called by every lane of
// the group (hit: this lane's candidate is a neighbour; rank: its position among the receiver's hits so
// far; count: the step's hits).  Returns the number visited (the same in every lane of the group).
constexpr int RL = 16;
template <typename F>
__device__ __forceinline__ int32_t walk_receiver_wave(const Walk& w, int64_t j, int lane, F&& f) {
  const int sub = lane & (RL - 1), gshift = lane & ~(RL - 1);
  const GridParams g = *w.grid;
  const double pj[3] = {w.pos[3 * j], w.pos[3 * j + 1], w.pos[3 * j + 2]};
  double a[9];
#pragma unroll
  for (int t = 0; t < 9; ++t) a[t] = w.cell[t];
  const uint64_t below = sub ? (~0ull >> (64 - sub)) : 0ull;
  int32_t n = 0;
  for (int sx = -w.pbc[0]; sx <= w.pbc[0]; ++sx)
    for (int sy = -w.pbc[1]; sy <= w.pbc[1]; ++sy)
      for (int sz = -w.pbc[2]; sz <= w.pbc[2]; ++sz) {
        double sv[3], p[3];
        int clo[3], chi[3];
        bool empty = false;
#pragma unroll
        for (int k = 0; k < 3; ++k) {
          sv[k] = dadd(dadd(dmul((double)sx, a[k]), dmul((double)sy, a[3 + k])), dmul((double)sz, a[6 + k]));
          p[k] = pj[k] + sv[k];
          // no atom lies outside [lo, hi]: an image point farther than r from the box has no neighbours
          if (p[k] + w.reach < g.lo[k] || p[k] - w.reach > g.hi[k]) empty = true;
          clo[k] = cell_coord(g, k, p[k] - w.reach);
          chi[k] = cell_coord(g, k, p[k] + w.reach);
        }
        if (empty || !(p[0] == p[0] && p[1] == p[1] && p[2] == p[2])) continue;
        const int code = (sx + 1) * 9 + (sy + 1) * 3 + (sz + 1);
        const bool self_image = sx == 0 && sy == 0 && sz == 0;
        for (int cx = clo[0]; cx <= chi[0]; ++cx)
          for (int cy = clo[1]; cy <= chi[1]; ++cy)
            for (int cz = clo[2]; cz <= chi[2]; ++cz) {
              const int c = (cx * g.G[1] + cy) * g.G[2] + cz;
              const int32_t qb = w.cell_start[c], qe = w.cell_start[c + 1];
              for (int32_t q0 = qb; q0 < qe; q0 += RL) {
                const int32_t q = q0 + sub;
                bool hit = false;
                int32_t i = 0;
                if (q < qe) {
                  i = w.cell_atoms[q];
                  if (!(self_image && i == j)) {
                    const double dx = dadd(pj[0] - w.pos[3 * (int64_t)i], sv[0]);
                    const double dy = dadd(pj[1] - w.pos[3 * (int64_t)i + 1], sv[1]);
                    const double dz = dadd(pj[2] - w.pos[3 * (int64_t)i + 2], sv[2]);
                    const double d2 = dadd(dadd(dmul(dx, dx), dmul(dy, dy)), dmul(dz, dz));
                    hit = d2 < w.r2;
                  }
                }
                // this group's bits of the ballot of the lanes still in the loop
                const uint64_t mask = (__ballot(hit) >> gshift) & ((1ull << RL) - 1);
                if (mask) {
                  const int cnt = __popcll(mask);
                  f(hit, i, (int64_t)i * KEY_IMAGES + code, n + __popcll(mask & below), cnt);
                  n += cnt;
                }
              }
            }
      }
  return n;
}

__global__ __launch_bounds__(256) void count_kernel(Walk w, int32_t* __restrict__ deg) {
  const int64_t j = (int64_t)blockIdx.x * (256 / RL) + threadIdx.x / RL;
  if (j >= w.N) return;   // uniform in the lane group
  const int lane = threadIdx.x & 63;
  const int32_t n = walk_receiver_wave(w, j, lane, [](bool, int32_t, int64_t, int32_t, int) {});
  if ((lane & (RL - 1)) == 0) deg[j] = n;
}

__global__ __launch_bounds__(256) void fill_kernel(Walk w, const int32_t* __restrict__ dst_ptr, int64_t E,
                                                   int64_t* __restrict__ keys, int32_t* __restrict__ key_dst) {
  const int64_t j = (int64_t)blockIdx.x * (256 / RL) + threadIdx.x / RL;
  if (j >= w.N) return;   // uniform in the lane group
  const int lane = threadIdx.x & 63;
  const int64_t beg = dst_ptr[j], end = dst_ptr[j + 1];
  walk_receiver_wave(w, j, lane, [&](bool hit, int32_t, int64_t key, int32_t rank, int) {
    const int64_t o = beg + rank;
    if (hit && o < end && o < E) {   // the counts came from the same walk: never false, kept as a bound
      keys[o] = key;
      key_dst[o] = (int32_t)j;
    }
  });
}

// Final order: each key's rank within its receiver's slots.
__global__ __launch_bounds__(256) void rank_kernel(int64_t N, int64_t E, const int32_t* __restrict__ dst_ptr,
                                                   const int64_t* __restrict__ keys, const int32_t* __restrict__ key_dst,
                                                   int64_t* __restrict__ edge_src, int64_t* __restrict__ edge_dst,
                                                   double* __restrict__ edge_shifts) {
  const int64_t p = (int64_t)blockIdx.x * 256 + threadIdx.x;
  if (p >= E) return;
  const int64_t key = keys[p];
  const int32_t j = key_dst[p];
  if (j < 0 || j >= N) return;   // every slot is written by fill_kernel; kept as a bound
  const int32_t a = dst_ptr[j], b = dst_ptr[j + 1];
  int32_t rank = 0;
  for (int32_t q = a; q < b; ++q) rank += keys[q] < key;
  const int64_t o = a + rank;
  const int code = (int)(key % KEY_IMAGES);
  edge_src[o] = key / KEY_IMAGES;
  edge_dst[o] = j;
  edge_shifts[3 * o] = (double)(code / 9 - 1);
  edge_shifts[3 * o + 1] = (double)((code / 3) % 3 - 1);
  edge_shifts[3 * o + 2] = (double)(code % 3 - 1);
}

int64_t cells_budget(int64_t N) {
  const int64_t c = 2 * N > 64 ? 2 * N : 64;
  return c < (int64_t(1) << 24) ? c : (int64_t(1) << 24);
}

struct NbrWs {
  int64_t cnt, cur, grid, box, cell_start, tot, atom_cell, cell_atoms, deg, total, cells, nb;
};

NbrWs nbr_ws(int64_t N) {
  NbrWs w;
  w.cells = cells_budget(N);
  w.nb = (w.cells + 1 + SCAN_TILE - 1) / SCAN_TILE;
  int64_t o = 0;
  w.cnt = o;        o += w.cells;
  w.cur = o;        o += w.cells;   // the zero-filled prefix ends here
  o = (o + 1) & ~int64_t(1);        // 8-byte alignment of the double fields
  w.grid = o;       o += (int64_t)(sizeof(GridParams) / 4);
  w.box = o;        o += 12;
  w.cell_start = o; o += w.cells + 1;
  w.tot = o;        o += w.nb;
  w.atom_cell = o;  o += N;
  w.cell_atoms = o; o += N;
  w.deg = o;        o += N;
  w.total = o;
  return w;
}

Walk make_walk(int64_t N, const double* pos, const double* cell, const int32_t* pbc, double cutoff, int32_t* ws,
               const NbrWs& w) {
  Walk k;
  k.pos = pos;
  k.cell = cell;
  k.grid = reinterpret_cast<const GridParams*>(ws + w.grid);
  k.cell_start = ws + w.cell_start;
  k.cell_atoms = ws + w.cell_atoms;
  k.N = N;
  for (int a = 0; a < 3; ++a) k.pbc[a] = pbc[a] ? 1 : 0;
  k.r2 = cutoff * cutoff;
  k.reach = cutoff * (1.0 + 1e-9);
  return k;
}

}  // namespace
}  // namespace nbr
}  // namespace fsc

using namespace fsc;
using namespace fsc::nbr;

extern "C" {

int fsc_neighbor_workspace(int64_t n_nodes, int64_t* workspace_ints) {
  FSC_CHECK_ARG(workspace_ints, "fsc_neighbor_workspace: null pointer");
  FSC_CHECK_ARG(n_nodes >= 0 && n_nodes < (1LL << 31) - 1, "fsc_neighbor_workspace: bad node count");
  *workspace_ints = nbr_ws(n_nodes).total;
  return 0;
}

int fsc_neighbor_count(int64_t n_nodes, const double* pos, const double* cell, const int32_t* pbc, double cutoff,
                       int32_t* dst_ptr, int32_t* workspace, hipStream_t stream) {
  FSC_CHECK_ARG(n_nodes >= 0 && n_nodes < (1LL << 31) - 1, "fsc_neighbor_count: bad node count");
  FSC_CHECK_ARG(pbc && dst_ptr && workspace && (n_nodes == 0 || (pos && cell)), "fsc_neighbor_count: null pointer");
  FSC_CHECK_ARG(cutoff > 0.0 && cutoff < 1e30, "fsc_neighbor_count: cutoff must be positive and finite");
  const int64_t N = n_nodes;
  const NbrWs w = nbr_ws(N);
  int32_t* ws = workspace;
  fill_i32_kernel<<<grid_of(w.cur + w.cells) < 1024 ? grid_of(w.cur + w.cells) : 1024, 256, 0, stream>>>(
      ws, w.cur + w.cells, 0);
  if (N == 0) {
    fill_i32_kernel<<<1, 256, 0, stream>>>(dst_ptr, 1, 0);
    return check_launch("fsc_neighbor_count") ? 2 : 0;
  }
  double* box = reinterpret_cast<double*>(ws + w.box);
  GridParams* gp = reinterpret_cast<GridParams*>(ws + w.grid);
  bbox_kernel<<<1, 1024, 0, stream>>>(N, pos, box);
  grid_kernel<<<1, 64, 0, stream>>>(box, cutoff, w.cells, gp);
  assign_kernel<<<grid_of(N), 256, 0, stream>>>(N, pos, gp, ws + w.atom_cell, ws + w.cnt);
  ScanArgs sa;
  sa.cnt[0] = sa.cnt[1] = ws + w.cnt;
  sa.out[0] = sa.out[1] = ws + w.cell_start;
  sa.tot[0] = sa.tot[1] = ws + w.tot;
  sa.n = w.cells;
  FSC_CHECK_ARG(w.nb <= SCAN_MAX_BLOCKS, "fsc_neighbor_count: too many cells for the scan");
  scan_blocks_kernel<<<dim3((unsigned)w.nb, 1), SCAN_T, 0, stream>>>(sa);
  scan_totals_kernel<<<dim3(1, 1), 1024, 0, stream>>>(sa, (int)w.nb);
  scan_add_kernel<<<dim3((unsigned)w.nb, 1), SCAN_T, 0, stream>>>(sa);
  place_kernel<<<grid_of(N), 256, 0, stream>>>(N, ws + w.atom_cell, ws + w.cell_start, ws + w.cur, ws + w.cell_atoms);
  const Walk walk = make_walk(N, pos, cell, pbc, cutoff, ws, w);
  count_kernel<<<(unsigned)((N + 256 / RL - 1) / (256 / RL)), 256, 0, stream>>>(walk, ws + w.deg);
  // receiver CSR: exclusive scan of the degrees into dst_ptr[0..N]
  const int64_t nbn = (N + 1 + SCAN_TILE - 1) / SCAN_TILE;
  FSC_CHECK_ARG(nbn <= SCAN_MAX_BLOCKS, "fsc_neighbor_count: too many nodes for the scan");
  ScanArgs sd;
  sd.cnt[0] = sd.cnt[1] = ws + w.deg;
  sd.out[0] = sd.out[1] = dst_ptr;
  sd.tot[0] = sd.tot[1] = ws + w.cnt;   // the cell counts are dead once cell_start is built
  sd.n = N;
  scan_blocks_kernel<<<dim3((unsigned)nbn, 1), SCAN_T, 0, stream>>>(sd);
  scan_totals_kernel<<<dim3(1, 1), 1024, 0, stream>>>(sd, (int)nbn);
  scan_add_kernel<<<dim3((unsigned)nbn, 1), SCAN_T, 0, stream>>>(sd);
  return check_launch("fsc_neighbor_count") ? 2 : 0;
}

int fsc_neighbor_fill(int64_t n_nodes, int64_t n_edges, const double* pos, const double* cell, const int32_t* pbc,
                      double cutoff, const int32_t* dst_ptr, int32_t* workspace, int32_t* fill_ws, int64_t* edge_src,
                      int64_t* edge_dst, double* edge_shifts, hipStream_t stream) {
  FSC_CHECK_ARG(n_nodes >= 0 && n_edges >= 0 && n_edges < (1LL << 31) - 1, "fsc_neighbor_fill: bad size");
  FSC_CHECK_ARG(pbc && dst_ptr && workspace, "fsc_neighbor_fill: null pointer");
  if (n_nodes == 0 || n_edges == 0) return 0;
  FSC_CHECK_ARG(pos && cell && fill_ws && edge_src && edge_dst && edge_shifts, "fsc_neighbor_fill: null pointer");
  const int64_t N = n_nodes, E = n_edges;
  const NbrWs w = nbr_ws(N);
  int64_t* keys = reinterpret_cast<int64_t*>(fill_ws);   // 2E int32, 8-byte aligned by the caller
  int32_t* key_dst = fill_ws + 2 * E;
  const Walk walk = make_walk(N, pos, cell, pbc, cutoff, workspace, w);
  fill_kernel<<<(unsigned)((N + 256 / RL - 1) / (256 / RL)), 256, 0, stream>>>(walk, dst_ptr, E, keys, key_dst);
  rank_kernel<<<grid_of(E), 256, 0, stream>>>(N, E, dst_ptr, keys, key_dst, edge_src, edge_dst, edge_shifts);
  return check_launch("fsc_neighbor_fill") ? 2 : 0;
}

}  // extern "C"
