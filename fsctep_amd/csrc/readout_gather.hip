// Readout feature assembly on gfx950 (sparse and ICTD trunks).
//
// The readouts combine the per-layer node features X_l [N][M][C] (l < n_layers) in two ways:
//   * Gram inputs t_k [N][d_k][nC] (nC = n_layers * C), one per key k (a run of d_k components
//     starting at comp0_k): a fixed permutation of the (l, m, c) entries of a node over the
//     key-major columns of all t_k, given by the host as srcmap (destination -> source) and gmap
//     (source -> destination; an entry need not land in the Gram input of its own key);
//   * squared norms sq[n][k][l*C + c] = sum_{m in key k} X_l[n][m][c]^2.
// The sparse trunk builds t_k as the concatenation over layers of the rank-L component block
// (models/pure_cartesian_sparse_layers.py:769-833); the ICTD trunks flatten each layer channel-major
// per key, concatenate the layers and re-split the result by key
// (models/pure_cartesian_ictd_layers_full.py:977-1001, models/pure_cartesian_ictd_layers_o3.py:987-1019),
// which mixes keys and layers; both are permutations, so one gather builds every t_k and the
// backward is one gather through the inverse map plus the squared-norm term:
//   dX_l[n][m][c] = dt_{k'}[n][gmap(l,m,c) - col0_{k'}] + 2 X_l[n][m][c] dsq[n][k][l*C + c],
// k' the key whose columns hold gmap(l,m,c), k the key of component m.
// Layouts: t_all holds the t_k one after another (t_k at N * col0_k, col0_k = sum_{k'<k} d_k' nC), each
// [N][d_k][nC] or, from the blocked gather, quad-major [nC/4][d_k][N][4] (channels 4c..4c+3 of component m
// of node n at ((c d_k + m) N + n) 4), the order the blocked Gram kernels read.

#include "common.h"
#include "fsctep.h"

namespace fsc {
namespace readout {

struct LayerPtrs {
  const float* p[4];
};
struct KeyPtrs {
  const float* p[8];
};
struct OutPtrs {
  float* p[4];
};

// Key of component m.
__device__ __forceinline__ int key_of(const FscReadoutTable& T, int m) {
  int k = 0;
  while (k + 1 < T.n_keys && m >= T.key_comp0[k + 1]) ++k;
  return k;
}

// Key holding key-major column j (of n_layers*M*C) and its first column.
__device__ __forceinline__ int key_of_column(const FscReadoutTable& T, int nC, int j, int& col0) {
  int k = 0;
  col0 = 0;
  while (k + 1 < T.n_keys && j >= col0 + T.key_dim[k] * nC) {
    col0 += T.key_dim[k] * nC;
    ++k;
  }
  return k;
}

// t_all[N * col0_k + n * d_k nC + j'] = X[src], thread per (node, key-major column); columns fastest.
__global__ void gather_kernel(FscReadoutTable T, int64_t N, LayerPtrs X, const int32_t* __restrict__ srcmap,
                              float* __restrict__ t_all) {
  const int MC = T.M * T.C, nC = T.n_layers * T.C, P = T.n_layers * MC;
  const int64_t total = N * P;
  for (int64_t idx = blockIdx.x * (int64_t)blockDim.x + threadIdx.x; idx < total;
       idx += (int64_t)gridDim.x * blockDim.x) {
    const int64_t n = idx / P;
    const int jg = (int)(idx - n * P);
    int col0;
    const int k = key_of_column(T, nC, jg, col0);
    const int src = min(max(srcmap[jg], 0), P - 1);   // maps are host-checked permutations; stay in bounds
    const int l = src / MC;
    t_all[N * col0 + n * (int64_t)(T.key_dim[k] * nC) + (jg - col0)] = X.p[l][n * MC + (src - l * MC)];
  }
}

// sq[n][k][l*C + c] = sum over the components of key k of X_l[n][m][c]^2; thread per (n, k, l, c).
__global__ void sq_kernel(FscReadoutTable T, int64_t N, LayerPtrs X, float* __restrict__ sq) {
  const int C = T.C, L = T.n_layers, K = T.n_keys;
  const int64_t total = N * K * L * C;
  for (int64_t idx = blockIdx.x * (int64_t)blockDim.x + threadIdx.x; idx < total;
       idx += (int64_t)gridDim.x * blockDim.x) {
    const int c = (int)(idx % C);
    const int l = (int)((idx / C) % L);
    const int k = (int)((idx / ((int64_t)C * L)) % K);
    const int64_t n = idx / ((int64_t)C * L * K);
    const float* x = X.p[l] + (n * T.M + T.key_comp0[k]) * C + c;
    float s = 0.f;
    for (int m = 0; m < T.key_dim[k]; ++m) s += x[m * C] * x[m * C];
    sq[idx] = s;
  }
}

// dX_l[n][m][c] = dt_k'[n][gmap(l,m,c) - col0_k'] + 2 X_l[n][m][c] dsq[n][key(m)][l*C + c]; thread per
// (l, n, m, c).
__global__ void scatter_kernel(FscReadoutTable T, int64_t N, KeyPtrs dt, const float* __restrict__ dsq, LayerPtrs X,
                               const int32_t* __restrict__ gmap, OutPtrs dX) {
  const int C = T.C, M = T.M, MC = M * C, nC = T.n_layers * C, P = T.n_layers * MC;
  const int64_t total = (int64_t)T.n_layers * N * MC;
  for (int64_t idx = blockIdx.x * (int64_t)blockDim.x + threadIdx.x; idx < total;
       idx += (int64_t)gridDim.x * blockDim.x) {
    const int l = (int)(idx / (N * MC));
    const int64_t rem = idx - (int64_t)l * N * MC;
    const int64_t n = rem / MC;
    const int mc = (int)(rem - n * MC);
    const int m = mc / C, c = mc - m * C;
    const int j = min(max(gmap[l * MC + mc], 0), P - 1);
    int col0;
    const int kt = key_of_column(T, nC, j, col0);
    float v = 0.f;
    if (dt.p[kt]) v = dt.p[kt][n * (int64_t)(T.key_dim[kt] * nC) + (j - col0)];
    if (dsq) v += 2.f * X.p[l][rem] * dsq[(n * T.n_keys + key_of(T, m)) * nC + l * C + c];
    dX.p[l][rem] = v;
  }
}

// One block per node when a node's n_layers*M*C entries fit in LDS (ROW_LDS floats): the node's row is
// read once, coalesced, and permuted out of LDS, so both the reads and the writes stay contiguous (the
// element-wise kernels above gather or scatter through the permutation in global memory).
constexpr int ROW_LDS = 12288;

__global__ __launch_bounds__(256) void gather_node_kernel(FscReadoutTable T, int64_t N, LayerPtrs X,
                                                          const int32_t* __restrict__ srcmap,
                                                          float* __restrict__ t_all, float* __restrict__ sq) {
  extern __shared__ float xs[];
  const int C = T.C, MC = T.M * C, nC = T.n_layers * C, P = T.n_layers * MC;
  for (int64_t n = blockIdx.x; n < N; n += gridDim.x) {
    __syncthreads();
    for (int l = 0; l < T.n_layers; ++l)
      for (int j = threadIdx.x; j < MC; j += blockDim.x) xs[l * MC + j] = X.p[l][n * MC + j];
    __syncthreads();
    int col0 = 0;
    for (int k = 0; k < T.n_keys; ++k) {   // key k's columns of node n are contiguous in t_k
      const int len = T.key_dim[k] * nC;
      float* dst = t_all + N * col0 + n * (int64_t)len;
      for (int j = threadIdx.x; j < len; j += blockDim.x)
        dst[j] = xs[min(max(srcmap[col0 + j], 0), P - 1)];   // host-checked permutation; stay in bounds
      float* sk = sq + (n * T.n_keys + k) * (int64_t)nC;
      for (int lc = threadIdx.x; lc < nC; lc += blockDim.x) {
        const int l = lc / C;
        const float* x = xs + l * MC + T.key_comp0[k] * C + (lc - l * C);
        float s2 = 0.f;
        for (int m = 0; m < T.key_dim[k]; ++m) s2 += x[m * C] * x[m * C];
        sk[lc] = s2;
      }
      col0 += len;
    }
  }
}

__global__ __launch_bounds__(256) void scatter_node_kernel(FscReadoutTable T, int64_t N, KeyPtrs dt,
                                                           const float* __restrict__ dsq, LayerPtrs X,
                                                           const int32_t* __restrict__ gmap, OutPtrs dX) {
  extern __shared__ float ds[];
  const int C = T.C, MC = T.M * C, nC = T.n_layers * C, P = T.n_layers * MC, rows = T.n_layers * T.M;
  // a pass covers R component rows of C channels (R = blockDim / C when C divides it, else one row
  // with a channel loop)
  const bool fits = C <= (int)blockDim.x && blockDim.x % C == 0;
  const int R = fits ? blockDim.x / C : 1;
  const int rsub = fits ? threadIdx.x / C : 0;
  const int c0 = fits ? threadIdx.x - rsub * C : threadIdx.x;
  const int cstep = fits ? C : blockDim.x;
  for (int64_t n = blockIdx.x; n < N; n += gridDim.x) {
    __syncthreads();
    int col0 = 0;
    for (int k = 0; k < T.n_keys; ++k) {
      const int len = T.key_dim[k] * nC;
      const float* src = dt.p[k] ? dt.p[k] + n * (int64_t)len : nullptr;
      for (int j = threadIdx.x; j < len; j += blockDim.x) ds[col0 + j] = src ? src[j] : 0.f;
      col0 += len;
    }
    __syncthreads();
    for (int row = rsub; row < rows; row += R) {
      const int l = row / T.M, m = row - l * T.M;
      const int kk = key_of(T, m);
      const float* xr = X.p[l] + n * MC + m * C;
      float* o = dX.p[l] + n * MC + m * C;
      const int32_t* gr = gmap + l * MC + m * C;
      const float* dq = dsq ? dsq + (n * T.n_keys + kk) * (int64_t)nC + l * C : nullptr;
      for (int c = c0; c < C; c += cstep) {
        float v = ds[min(max(gr[c], 0), P - 1)];
        if (dq) v += 2.f * xr[c] * dq[c];
        o[c] = v;
      }
    }
  }
}

// Vectorised per-node forms (C a multiple of 4, 16-byte aligned arrays): a thread owns NQ quads of four
// consecutive entries of a node, and its map indices and offsets, the same for every node, stay in registers
// while the block walks its nodes.  The next node's row is requested before the current node's outputs are
// stored, so each node costs one round trip to memory instead of one per output.
// In the blocked order a node's quads are 16-byte pieces of slabs [N][4], and a 128-byte line of a slab is
// completed by eight nodes.  The L2 merges those pieces only while the line stays resident, so the node
// order keeps neighbouring nodes on one XCD (blocks b and b + 8 share an XCD and walk nodes b' and b' + 1,
// for a grid that is a multiple of 8) and the host bounds the nodes in flight (the grid) so that an XCD's
// partly written lines fit its L2: at 10,000 nodes of 6,144 entries 256 blocks of 512 threads store the
// blocked order in 184 us against 250 us for 2,048 blocks of 256 (109 us for the row-major order).
template <int NQ, bool BLK, int BT = 256>
__global__ __launch_bounds__(BT) void gather_node4_kernel(FscReadoutTable T, int64_t N, LayerPtrs X,
                                                           const int32_t* __restrict__ srcmap,
                                                           float* __restrict__ t_all, float* __restrict__ sq) {
  extern __shared__ __align__(16) float xs[];
  const int C = T.C, MC = T.M * C, nC = T.n_layers * C, P = T.n_layers * MC, P4 = P / 4;
  const int K = T.n_keys, S4 = K * nC / 4;
  // phase 1 (a node's layers, (l, m, c) order) and phase 2 (key-major columns) share the quad index g
  int xl[NQ], xo[NQ], ko[NQ], kl[NQ];
  int64_t kb[NQ];
  int4 si[NQ];
#pragma unroll
  for (int u = 0; u < NQ; ++u) {
    const int g = min((int)threadIdx.x + BT * u, P4 - 1);   // threads past P4 repeat the last quad (not stored)
    const int e = 4 * g;
    xl[u] = e / MC;
    xo[u] = e - xl[u] * MC;
    int col0;
    const int k = key_of_column(T, nC, e, col0);
    if constexpr (BLK) {   // component m = ko / nC, channels i..i+3 (i = ko % nC) of key k
      const int ko_ = e - col0, m = ko_ / nC, i = ko_ - m * nC;
      kb[u] = N * (int64_t)col0 + ((int64_t)(i >> 2) * T.key_dim[k] + m) * N * 4;
      kl[u] = 4;
      ko[u] = 0;
    } else {
      kb[u] = N * (int64_t)col0;
      kl[u] = T.key_dim[k] * nC;
      ko[u] = e - col0;
    }
    const int4 m4 = *reinterpret_cast<const int4*>(srcmap + e);
    si[u] = int4{min(max(m4.x, 0), P - 1), min(max(m4.y, 0), P - 1), min(max(m4.z, 0), P - 1),
                 min(max(m4.w, 0), P - 1)};
  }
  f4 pre[NQ];
  auto load_row = [&](int64_t n) {
#pragma unroll
    for (int u = 0; u < NQ; ++u) pre[u] = ld4(X.p[xl[u]] + n * MC + xo[u]);
  };
  int64_t n = blockIdx.x;
  if (BLK && gridDim.x % 8 == 0) n = (blockIdx.x & 7) * (gridDim.x >> 3) + (blockIdx.x >> 3);
  if (n < N) load_row(n);
  for (; n < N; n += gridDim.x) {
    __syncthreads();
#pragma unroll
    for (int u = 0; u < NQ; ++u)
      if ((int)threadIdx.x + BT * u < P4) *reinterpret_cast<f4*>(xs + 4 * ((int)threadIdx.x + BT * u)) = pre[u];
    __syncthreads();
    if (n + gridDim.x < N) load_row(n + gridDim.x);
#pragma unroll
    for (int u = 0; u < NQ; ++u) {
      if ((int)threadIdx.x + BT * u >= P4) continue;
      const f4 v = {xs[si[u].x], xs[si[u].y], xs[si[u].z], xs[si[u].w]};
      st4(t_all + kb[u] + n * (int64_t)kl[u] + ko[u], v);
    }
    for (int g = threadIdx.x; g < S4; g += BT) {   // squared norms, four channels per thread
      const int k = (4 * g) / nC, lc = 4 * g - k * nC, l = lc / C, c = lc - l * C;
      const float* x = xs + l * MC + T.key_comp0[k] * C + c;
      f4 s2 = {0.f, 0.f, 0.f, 0.f};
      for (int m = 0; m < T.key_dim[k]; ++m) {
        const f4 v = *reinterpret_cast<const f4*>(x + m * C);
        s2 += v * v;
      }
      st4(sq + (n * K + k) * (int64_t)nC + lc, s2);
    }
  }
}

template <int NQ>
__global__ __launch_bounds__(256) void scatter_node4_kernel(FscReadoutTable T, int64_t N, KeyPtrs dt,
                                                            const float* __restrict__ dsq, LayerPtrs X,
                                                            const int32_t* __restrict__ gmap, OutPtrs dX) {
  extern __shared__ __align__(16) float ds[];
  const int C = T.C, MC = T.M * C, nC = T.n_layers * C, P = T.n_layers * MC, P4 = P / 4;
  const int K = T.n_keys;
  // phase 1 (key-major dt columns) and phase 2 ((l, m, c) entries) share the quad index g
  int kd[NQ], ko[NQ], kl[NQ], xl[NQ], xo[NQ], qo[NQ];
  int4 gi[NQ];
#pragma unroll
  for (int u = 0; u < NQ; ++u) {
    const int g = min((int)threadIdx.x + 256 * u, P4 - 1);   // threads past P4 repeat the last quad (not stored)
    const int e = 4 * g;
    int col0;
    kd[u] = key_of_column(T, nC, e, col0);
    kl[u] = T.key_dim[kd[u]] * nC;
    ko[u] = e - col0;
    xl[u] = e / MC;
    xo[u] = e - xl[u] * MC;
    const int m = xo[u] / C, c = xo[u] - m * C;
    qo[u] = key_of(T, m) * nC + xl[u] * C + c;
    const int4 m4 = *reinterpret_cast<const int4*>(gmap + e);
    gi[u] = int4{min(max(m4.x, 0), P - 1), min(max(m4.y, 0), P - 1), min(max(m4.z, 0), P - 1),
                 min(max(m4.w, 0), P - 1)};
  }
  f4 pre[NQ];
  auto load_dt = [&](int64_t n) {
#pragma unroll
    for (int u = 0; u < NQ; ++u) {
      const float* d = dt.p[kd[u]];
      pre[u] = d ? ld4(d + n * (int64_t)kl[u] + ko[u]) : f4{0.f, 0.f, 0.f, 0.f};
    }
  };
  int64_t n = blockIdx.x;
  if (n < N) load_dt(n);
  for (; n < N; n += gridDim.x) {
    __syncthreads();
#pragma unroll
    for (int u = 0; u < NQ; ++u)
      if ((int)threadIdx.x + 256 * u < P4) *reinterpret_cast<f4*>(ds + 4 * ((int)threadIdx.x + 256 * u)) = pre[u];
    __syncthreads();
    f4 xv[NQ], qv[NQ];
#pragma unroll
    for (int u = 0; u < NQ; ++u) {
      xv[u] = ld4(X.p[xl[u]] + n * MC + xo[u]);
      qv[u] = dsq ? ld4(dsq + n * K * (int64_t)nC + qo[u]) : f4{0.f, 0.f, 0.f, 0.f};
    }
    if (n + gridDim.x < N) load_dt(n + gridDim.x);
#pragma unroll
    for (int u = 0; u < NQ; ++u) {
      if ((int)threadIdx.x + 256 * u >= P4) continue;
      f4 v = {ds[gi[u].x], ds[gi[u].y], ds[gi[u].z], ds[gi[u].w]};
      v += 2.f * xv[u] * qv[u];
      st4(dX.p[xl[u]] + n * MC + xo[u], v);
    }
  }
}

int check_table(const FscReadoutTable* T, const char* who) {
  if (!T) {
    set_error(std::string(who) + ": null table");
    return 1;
  }
  if (T->n_layers < 1 || T->n_layers > 4 || T->n_keys < 1 || T->n_keys > 8 || T->M < 1 || T->M > 64 ||
      T->C < 1 || T->C > 1024) {
    set_error(std::string(who) + ": table out of range (1..4 layers, 1..8 keys, M <= 64, C <= 1024)");
    return 1;
  }
  int covered = 0;
  for (int k = 0; k < T->n_keys; ++k) {
    if (T->key_comp0[k] != covered || T->key_dim[k] < 1) {
      set_error(std::string(who) + ": keys must tile the components in order");
      return 1;
    }
    covered += T->key_dim[k];
  }
  if (covered != T->M) {
    set_error(std::string(who) + ": keys must cover all M components");
    return 1;
  }
  return 0;
}

unsigned grid_for(int64_t total) { return (unsigned)std::min<int64_t>((total + 255) / 256, 8192); }

// blocks of the vectorised per-node kernels (each walks about N / NODE_GRID nodes)
constexpr int64_t NODE_GRID = 2048;
inline bool aligned16(const void* p) { return (reinterpret_cast<uintptr_t>(p) & 15) == 0; }

}  // namespace readout
}  // namespace fsc

using namespace fsc;
using namespace fsc::readout;

extern "C" {

// Blocks per XCD of the blocked gather: about 49,152 quads in flight per XCD (lines being filled).
constexpr int BLOCKED_QUADS_PER_XCD = 49152;

static int readout_gather_any(bool blk, const FscReadoutTable* table, int64_t n_nodes, const float* const* layers,
                              const int32_t* srcmap, float* t_all, float* sq, hipStream_t stream, const char* who) {
  if (check_table(table, who)) return 1;
  FSC_CHECK_ARG(n_nodes >= 0 && n_nodes < (1LL << 31), std::string(who) + ": bad node count");
  if (n_nodes == 0) return 0;
  FSC_CHECK_ARG(layers && srcmap && t_all && sq, std::string(who) + ": null pointer");
  LayerPtrs X{};
  for (int l = 0; l < table->n_layers; ++l) {
    FSC_CHECK_ARG(layers[l], std::string(who) + ": null layer pointer");
    X.p[l] = layers[l];
  }
  const int64_t P = (int64_t)table->n_layers * table->M * table->C;
  const int nq = (int)((P / 4 + 255) / 256);
  bool aligned = aligned16(srcmap) && aligned16(t_all) && aligned16(sq);
  for (int l = 0; l < table->n_layers; ++l) aligned = aligned && aligned16(X.p[l]);
  const bool quads = table->C % 4 == 0 && P <= ROW_LDS && nq <= 8 && aligned;
  FSC_CHECK_ARG(!blk || quads, std::string(who) + ": needs C a multiple of 4, n_layers*M*C <= " +
                                   std::to_string(ROW_LDS) + " and 16-byte aligned arrays");
  if (quads) {
    unsigned grid = (unsigned)std::min<int64_t>(n_nodes, NODE_GRID);
    if (blk) {
      const int64_t per_xcd = std::max<int64_t>(1, BLOCKED_QUADS_PER_XCD / (P / 4));
      grid = (unsigned)std::min<int64_t>(n_nodes, 8 * per_xcd);
      if (grid >= 8) grid &= ~7u;
    }
    const size_t lds = P * sizeof(float);
#define FSC_G4(Q)                                                                                            \
  if (blk)                                                                                                   \
    gather_node4_kernel<(Q + 1) / 2, true, 512><<<grid, 512, lds, stream>>>(*table, n_nodes, X, srcmap, t_all, \
                                                                             sq);                            \
  else                                                                                                       \
    gather_node4_kernel<Q, false><<<grid, 256, lds, stream>>>(*table, n_nodes, X, srcmap, t_all, sq)
    switch (nq) {
      case 1: FSC_G4(1); break;
      case 2: FSC_G4(2); break;
      case 3: FSC_G4(3); break;
      case 4: FSC_G4(4); break;
      case 5: FSC_G4(5); break;
      case 6: FSC_G4(6); break;
      case 7: FSC_G4(7); break;
      default: FSC_G4(8); break;
    }
#undef FSC_G4
    return check_launch("readout gather") ? 2 : 0;
  }
  if (P <= ROW_LDS) {
    const unsigned grid = (unsigned)std::min<int64_t>(n_nodes, 65536);
    gather_node_kernel<<<grid, 256, P * sizeof(float), stream>>>(*table, n_nodes, X, srcmap, t_all, sq);
    return check_launch("readout gather") ? 2 : 0;
  }
  gather_kernel<<<grid_for(n_nodes * P), 256, 0, stream>>>(*table, n_nodes, X, srcmap, t_all);
  if (check_launch("readout gather")) return 2;
  const int64_t S = n_nodes * table->n_keys * table->n_layers * table->C;
  sq_kernel<<<grid_for(S), 256, 0, stream>>>(*table, n_nodes, X, sq);
  return check_launch("readout sq") ? 2 : 0;
}

int fsc_readout_gather(const FscReadoutTable* table, int64_t n_nodes, const float* const* layers,
                       const int32_t* srcmap, float* t_all, float* sq, hipStream_t stream) {
  return readout_gather_any(false, table, n_nodes, layers, srcmap, t_all, sq, stream, "fsc_readout_gather");
}

int fsc_readout_gather_blocked(const FscReadoutTable* table, int64_t n_nodes, const float* const* layers,
                               const int32_t* srcmap, float* t_all, float* sq, hipStream_t stream) {
  return readout_gather_any(true, table, n_nodes, layers, srcmap, t_all, sq, stream, "fsc_readout_gather_blocked");
}

int fsc_readout_scatter(const FscReadoutTable* table, int64_t n_nodes, const float* const* grad_t,
                        const float* grad_sq, const float* const* layers, const int32_t* gmap,
                        float* const* grad_layers, hipStream_t stream) {
  if (check_table(table, "fsc_readout_scatter")) return 1;
  FSC_CHECK_ARG(n_nodes >= 0 && n_nodes < (1LL << 31), "fsc_readout_scatter: bad node count");
  if (n_nodes == 0) return 0;
  FSC_CHECK_ARG(grad_t && layers && gmap && grad_layers, "fsc_readout_scatter: null pointer");
  KeyPtrs dt{};
  for (int k = 0; k < table->n_keys; ++k) dt.p[k] = grad_t[k];   // null: no gradient through key k
  LayerPtrs X{};
  OutPtrs dX{};
  for (int l = 0; l < table->n_layers; ++l) {
    FSC_CHECK_ARG(layers[l] && grad_layers[l], "fsc_readout_scatter: null layer pointer");
    X.p[l] = layers[l];
    dX.p[l] = grad_layers[l];
  }
  const int64_t P = (int64_t)table->n_layers * table->M * table->C;
  const int nq = (int)((P / 4 + 255) / 256);
  bool aligned = aligned16(gmap) && aligned16(grad_sq);
  for (int k = 0; k < table->n_keys; ++k) aligned = aligned && aligned16(dt.p[k]);
  for (int l = 0; l < table->n_layers; ++l) aligned = aligned && aligned16(X.p[l]) && aligned16(dX.p[l]);
  if (table->C % 4 == 0 && P <= ROW_LDS && nq <= 8 && aligned) {
    const unsigned grid = (unsigned)std::min<int64_t>(n_nodes, NODE_GRID);
    const size_t lds = P * sizeof(float);
#define FSC_S4(Q) scatter_node4_kernel<Q><<<grid, 256, lds, stream>>>(*table, n_nodes, dt, grad_sq, X, gmap, dX)
    switch (nq) {
      case 1: FSC_S4(1); break;
      case 2: FSC_S4(2); break;
      case 3: FSC_S4(3); break;
      case 4: FSC_S4(4); break;
      case 5: FSC_S4(5); break;
      case 6: FSC_S4(6); break;
      case 7: FSC_S4(7); break;
      default: FSC_S4(8); break;
    }
#undef FSC_S4
    return check_launch("readout scatter") ? 2 : 0;
  }
  if (P <= ROW_LDS) {
    const unsigned grid = (unsigned)std::min<int64_t>(n_nodes, 65536);
    scatter_node_kernel<<<grid, 256, P * sizeof(float), stream>>>(*table, n_nodes, dt, grad_sq, X, gmap, dX);
    return check_launch("readout scatter") ? 2 : 0;
  }
  const int64_t total = P * n_nodes;
  scatter_kernel<<<grid_for(total), 256, 0, stream>>>(*table, n_nodes, dt, grad_sq, X, gmap, dX);
  return check_launch("readout scatter") ? 2 : 0;
}

}  // extern "C"
