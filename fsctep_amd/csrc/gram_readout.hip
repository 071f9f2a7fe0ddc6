// Invariant Gram bilinear of the readout on gfx950 (sparse and ICTD trunks).
//
//   out[n][o] = sum_{i,j} W[o][i][j] G_n[i][j],      G_n[i][j] = scale * sum_m t[n][m][i] t[n][m][j]
//
// Replaces PureCartesianSparseInvariantBilinear.forward (models/pure_cartesian_sparse_layers.py:424-456)
// and the Gram x W_read readout of the ICTD trunks (models/pure_cartesian_ictd_layers_full.py:999-1000,
// models/pure_cartesian_ictd_layers_o3.py:1017-1018).  The reference materialises G (N x nC x nC,
// 5.9 GB per irrep at 10k atoms and nC = 384) and runs a GEMM over it; here G is formed tile by tile
// in registers from t and consumed by the MFMA at once.
//
// Channels split into nb = nC/16 blocks.  G is symmetric, so the forward sums block pairs I <= J only:
//   out[n][o] = sum_{I<=J} sum_{il,jl} Wf[IJ][il][o][jl] G_n[I0+il][J0+jl]
// with Wf[IJ] = W_IJ + W_JI^T for I < J and W_II on the diagonal.  Both directions multiply in fp32
// precision on fp16 MFMA (each operand scaled by a power of two and split into two fp16 parts, three
// part products kept; common.h), with the weights split once when they are prepared and the Gram
// values / output gradients scaled per node; a forward over few node tiles runs on the fp32 MFMA
// instead (more, smaller workgroups).  The backward is
//   dt[n][m][i] = scale * sum_j A_n[i][j] t[n][m][j],   A_n = sum_o g[n][o] (W[o] + W[o]^T),
// computed per (node tile, row block I) over all J with A formed by MFMA (K = o) and contracted
// with t on the VALU; (W + W^T) is stored for I <= J (Wb[IJ][a][b][o]) and read transposed below
// the diagonal.  Layouts: t [N][D][nC] or, in the blocked entry points, quad-major [nC/4][D][N][4] (the four
// channels 4c..4c+3 of component m of node n at ((c D + m) N + n) 4: the lanes of a wave, which are
// consecutive nodes, read consecutive 16-byte pieces instead of one piece from each node's row, which left
// the vector memory pipe the bound: the readout gather writes this order directly); W [S][nC][nC],
// out/grad_out [N][S]; grad_t is always [N][D][nC].

#include "common.h"
#include "fsctep.h"

namespace fsc {
namespace gram {

constexpr int NODES = 128;   // nodes per workgroup (8 waves x 16 MFMA rows)
constexpr int PCHUNK = 8;    // block pairs per forward workgroup, or twice as many (fwd_plan)

__host__ __device__ inline int n_pairs(int nb) { return nb * (nb + 1) / 2; }

// The four channels i..i+3 (i % 4 == 0) of component m of node n.
template <bool BLK>
__device__ __forceinline__ const float* tq4(const float* __restrict__ t, int64_t N, int D, int nC, int64_t n, int m,
                                            int i) {
  if constexpr (BLK) return t + (((int64_t)(i >> 2) * D + m) * N + n) * 4;
  else return t + (n * D + m) * nC + i;
}
__host__ __device__ inline int pair_index(int I, int J, int nb) { return I * nb - (I * (I - 1)) / 2 + (J - I); }

// Workgroup w runs on XCD w % 8; give each XCD a contiguous range of logical tiles so tiles that
// share weight blocks share an L2.  Returns -1 for the padding workgroups.
__device__ __forceinline__ int xcd_logical(int nwg) {
  const int per = (nwg + 7) / 8;
  const int w = blockIdx.x;
  const int logical = (w & 7) * per + (w >> 3);
  return logical < nwg ? logical : -1;
}

// Forward work order: groups of (at most TILE_GROUP) node tiles, and within a group all pair chunks of
// its tiles with the tiles innermost.  Workgroups that run together on an XCD then share both the
// weight chunk (read by the group's tiles) and the t rows of the group, which stay in its L2.
constexpr int TILE_GROUP = 4;
__device__ __forceinline__ void group_order(int logical, int nchunks, int ntiles, int& chunk, int& tile,
                                            int tgroup = TILE_GROUP) {
  const int grp = logical / (tgroup * nchunks);
  const int gsize = min(tgroup, ntiles - grp * tgroup);
  const int rem = logical - grp * tgroup * nchunks;
  chunk = rem / gsize;
  tile = grp * tgroup + (rem - chunk * gsize);
}

// Block-pair weight buffers (floats): the fp32 pairs (P*256*S), two fp16 planes (h, l; split2h) of the
// same values times the power of two sw with 2 max|W| sw < 2^14 (P*256*S floats together), then a tail
// of GW_TAIL floats: [0] = 1/sw, [256..511] the partial maxima of |W| (Wf only).
constexpr int GW_TAIL = 512;
constexpr int WMAX_BLOCKS = 256;
__host__ __device__ inline int64_t gram_weight_floats(int nb, int S) { return (int64_t)n_pairs(nb) * 512 * S + GW_TAIL; }

// wmax[b] = max |W| over the grid-stride share of block b (grid WMAX_BLOCKS x 256); float4 loads, four in
// flight per thread, when W is 16-byte aligned.
__global__ __launch_bounds__(256) void absmax_kernel(const float* __restrict__ W, int64_t n, float* __restrict__ wmax) {
  __shared__ float red[4];
  float m = 0.f;
  const int64_t tid = blockIdx.x * 256 + threadIdx.x, stride = (int64_t)gridDim.x * 256;
  int64_t rest = 0;
  if ((reinterpret_cast<uintptr_t>(W) & 15) == 0) {
    const f4* W4 = reinterpret_cast<const f4*>(W);
    const int64_t n4 = n / 4;
    auto mx4 = [](const f4& v) { return fmaxf(fmaxf(fabsf(v.x), fabsf(v.y)), fmaxf(fabsf(v.z), fabsf(v.w))); };
    int64_t i = tid;
    for (; i + 3 * stride < n4; i += 4 * stride) {
      const f4 a = W4[i], b = W4[i + stride], c = W4[i + 2 * stride], d = W4[i + 3 * stride];
      m = fmaxf(m, fmaxf(fmaxf(mx4(a), mx4(b)), fmaxf(mx4(c), mx4(d))));
    }
    for (; i < n4; i += stride) m = fmaxf(m, mx4(W4[i]));
    rest = 4 * n4;
  }
  for (int64_t i = rest + tid; i < n; i += stride) m = fmaxf(m, fabsf(W[i]));
  for (int off = 32; off > 0; off >>= 1) m = fmaxf(m, __shfl_xor(m, off, 64));
  if ((threadIdx.x & 63) == 0) red[threadIdx.x >> 6] = m;
  __syncthreads();
  if (threadIdx.x == 0) wmax[blockIdx.x] = fmaxf(fmaxf(red[0], red[1]), fmaxf(red[2], red[3]));
}

// Wf[p][il][o][jl] and Wb[p][a][b][o] for every block pair p = (I <= J); grid (nb, nb, S / 16), 256 threads.
// The fp16 planes are [plane][p][ab][o] for the backward and [plane][p][jl][il/8][o][il%8] for the
// forward.  Every block reduces the partial maxima itself, so all use the same sw.
__global__ __launch_bounds__(256) void prepare_kernel(const float* __restrict__ W, int S, int nC, float* __restrict__ Wf,
                                                      float* __restrict__ Wb, const float* __restrict__ wmax) {
  const int I = blockIdx.y, J = blockIdx.x, nb = nC / 16;
  __shared__ float red[4];
  float mx = wmax[threadIdx.x];
  for (int off = 32; off > 0; off >>= 1) mx = fmaxf(mx, __shfl_xor(mx, off, 64));
  if ((threadIdx.x & 63) == 0) red[threadIdx.x >> 6] = mx;
  __syncthreads();
  const float sw = pow2_scale(2.f * fmaxf(fmaxf(red[0], red[1]), fmaxf(red[2], red[3])));
  const int64_t plane = (int64_t)n_pairs(nb) * 256 * S;
  if (I == 0 && J == 0 && threadIdx.x == 0) {
    Wf[2 * plane] = 1.f / sw;
    Wb[2 * plane] = 1.f / sw;
  }
  if (I > J) return;
  const int p = pair_index(I, J, nb);
  _Float16* wb2 = reinterpret_cast<_Float16*>(Wb + plane);
  _Float16* wf2 = reinterpret_cast<_Float16*>(Wf + plane);
  // 16 outputs o per block (blockIdx.z): both 16x16 blocks of W[o] (rows I, columns J and the transposed
  // pair) are read row by row into LDS (64 contiguous bytes per row), then each output layout is written in
  // its own order of contiguous runs
  __shared__ float tij[16][16][17];   // [oo][a][b] = W[o][16I + a][16J + b]
  __shared__ float tji[16][16][17];   // [oo][b][a] = W[o][16J + b][16I + a]
  const int t = threadIdx.x;
  {
    const int o0 = blockIdx.z * 16;
    for (int oo = 0; oo < 16; ++oo) {
      const int r = t >> 4, c = t & 15;
      const int64_t base = (int64_t)(o0 + oo) * nC;
      tij[oo][r][c] = W[(base + I * 16 + r) * nC + J * 16 + c];
      tji[oo][r][c] = W[(base + J * 16 + r) * nC + I * 16 + c];
    }
    __syncthreads();
    // Wb and its fp16 planes, [pair][ab][o]: runs of 16 consecutive o
    for (int aq = 0; aq < 16; ++aq) {
      const int ab = aq * 16 + (t >> 4), oo = t & 15, a = ab >> 4, b = ab & 15;
      const float v = tij[oo][a][b] + tji[oo][b][a];
      const int64_t e = ((int64_t)p * 256 + ab) * S + o0 + oo;
      Wb[e] = v;
      const _Float16 hb = (_Float16)(v * sw);
      wb2[e] = hb;
      wb2[plane + e] = (_Float16)(v * sw - (float)hb);
    }
    // Wf, [pair][a][o][b]: runs of 16 consecutive b
    for (int a = 0; a < 16; ++a) {
      const int b = t & 15, oo = t >> 4;
      const float wij = tij[oo][a][b];
      Wf[(((int64_t)p * 16 + a) * S + o0 + oo) * 16 + b] = (I == J) ? wij : wij + tji[oo][b][a];
    }
    // Wf's fp16 planes, [pair][b][a/8][o][a%8]: runs of 16 o x 8 a
    for (int b = 0; b < 16; ++b) {
      const int a = ((t >> 7) << 3) | (t & 7), oo = (t >> 3) & 15;
      const float wij = tij[oo][a][b];
      const float f = (I == J) ? wij : wij + tji[oo][b][a];
      const int64_t ef = (int64_t)p * 256 * S + ((b * 2 + (a >> 3)) * S + o0 + oo) * 8 + (a & 7);
      const _Float16 fh = (_Float16)(f * sw);
      wf2[ef] = fh;
      wf2[plane + ef] = (_Float16)(f * sw - (float)fh);
    }
  }
}

// Per-node power of two for the forward's fp16 Gram operands: |G_n[i][j]| <= max_i sum_m t[n][m][i]^2
// (Cauchy-Schwarz), so nsc[n] = pow2_scale of that bound keeps every scaled Gram value below 2^14.
// One wave per node.
__global__ __launch_bounds__(256) void node_scale_kernel(int64_t N, int D, int nC, const float* __restrict__ t,
                                                         float* __restrict__ nsc) {
  const int64_t n = (int64_t)blockIdx.x * 4 + (threadIdx.x >> 6);
  const int lane = threadIdx.x & 63;
  if (n >= N) return;   // uniform over the wave
  const float* tn = t + n * D * nC;
  float mx = 0.f;
  if ((nC & 3) == 0 && D <= 9 && (reinterpret_cast<uintptr_t>(t) & 15) == 0) {
    // four columns per lane, all D rows requested before the sums (same sums, same order per column)
    const int nq = nC >> 2;
    for (int c = lane; c < nq; c += 64) {
      f4 v[9];
#pragma unroll
      for (int m = 0; m < 9; ++m)
        if (m < D) v[m] = ld4(tq4<false>(t, N, D, nC, n, m, 4 * c));
      f4 s = f4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
      for (int m = 0; m < 9; ++m)
        if (m < D) s += v[m] * v[m];
      mx = fmaxf(mx, fmaxf(fmaxf(s[0], s[1]), fmaxf(s[2], s[3])));
    }
  } else {
    for (int i = lane; i < nC; i += 64) {
      float s = 0.f;
      for (int m = 0; m < D; ++m) {
        const float v = tn[m * nC + i];
        s += v * v;
      }
      mx = fmaxf(mx, s);
    }
  }
  for (int off = 32; off > 0; off >>= 1) mx = fmaxf(mx, __shfl_xor(mx, off, 64));
  if (lane == 0) nsc[n] = pow2_scale(mx);
}

// The same scales from the blocked order: a lane per node (64 consecutive nodes per workgroup, each
// (quad, component) read is one contiguous 1 KB piece per wave), the 8 waves take every 8th quad and
// combine their maxima in LDS.
__global__ __launch_bounds__(512) void node_scale_blocked_kernel(int64_t N, int D, int nC,
                                                                 const float* __restrict__ t,
                                                                 float* __restrict__ nsc) {
  __shared__ float red[8][64];
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int64_t n = (int64_t)blockIdx.x * 64 + lane;
  const int64_t nl = n < N ? n : N - 1;   // lanes past N repeat the last node (not stored)
  float mx = 0.f;
  for (int c = wave; c < (nC >> 2); c += 8) {
    f4 v[9];
#pragma unroll
    for (int m = 0; m < 9; ++m)
      if (m < D) v[m] = ld4(tq4<true>(t, N, D, nC, nl, m, 4 * c));
    f4 s = f4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int m = 0; m < 9; ++m)
      if (m < D) s += v[m] * v[m];
    mx = fmaxf(mx, fmaxf(fmaxf(s[0], s[1]), fmaxf(s[2], s[3])));
  }
  red[wave][lane] = mx;
  __syncthreads();
  if (wave == 0) {
#pragma unroll
    for (int w = 1; w < 8; ++w) mx = fmaxf(mx, red[w][lane]);
    if (n < N) nsc[n] = pow2_scale(mx);
  }
}

// Forward partial sums over pchunk block pairs: part[chunk][n][o].  A workgroup is 128 nodes (8 waves x
// 16 MFMA rows) x one chunk; each pair's Wf block [il][o][jl] (256*S floats) is staged in LDS and shared
// by the 8 waves, the next pair's block is loaded into registers while the current one is multiplied.
template <int D, int S, bool BLK>
__global__ __launch_bounds__(512) void forward_kernel(int64_t N, int nC, float scale, const float* __restrict__ t,
                                           const float* __restrict__ Wf, int nchunks, float* __restrict__ part,
                                           int pchunk) {
  constexpr int NN = NODES, CT = S / 16;
  constexpr int WBF4 = 256 * S / 4, PW = (WBF4 + 511) / 512;
  __shared__ f4 wl[WBF4];
  const int nb = nC / 16, np = n_pairs(nb);
  const int ntiles = (int)((N + NN - 1) / NN);
  const int logical = xcd_logical(nchunks * ntiles);
  if (logical < 0) return;
  int chunk, tile;
  group_order(logical, nchunks, ntiles, chunk, tile);
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int r = lane & 15, q = lane >> 4;
  const int64_t n = (int64_t)tile * NN + wave * 16 + r;
  const bool valid = n < N;
  const int64_t nl = valid ? n : 0;   // rows past N read node 0; their results are not stored
  const int p0 = chunk * pchunk, p1 = min(p0 + pchunk, np);
  int I = 0, rowstart = 0;
  while (rowstart + (nb - I) <= p0) { rowstart += nb - I; ++I; }
  int J = I + (p0 - rowstart);
  f4 acc[CT];
#pragma unroll
  for (int ct = 0; ct < CT; ++ct) acc[ct] = f4{0.f, 0.f, 0.f, 0.f};
  const f4 zero = {0.f, 0.f, 0.f, 0.f};
  f4 pw[PW];
  auto fetch = [&](int p) {
    const f4* src = reinterpret_cast<const f4*>(Wf + (int64_t)p * 256 * S);
#pragma unroll
    for (int i = 0; i < PW; ++i) { const int idx = threadIdx.x + 512 * i; if (idx < WBF4) pw[i] = src[idx]; }
  };
  fetch(p0);
  for (int p = p0; p < p1; ++p) {
    __syncthreads();
#pragma unroll
    for (int i = 0; i < PW; ++i) { const int idx = threadIdx.x + 512 * i; if (idx < WBF4) wl[idx] = pw[i]; }
    __syncthreads();
    if (p + 1 < p1) fetch(p + 1);
    f4 tj[D];
#pragma unroll
    for (int m = 0; m < D; ++m) tj[m] = valid ? ld4(tq4<BLK>(t, N, D, nC, nl, m, J * 16 + 4 * q)) : zero;
    const float* wp = reinterpret_cast<const float*>(wl) + r * 16 + 4 * q;
#pragma unroll 1
    for (int ig = 0; ig < 4; ++ig) {
      f4 ti[D];
#pragma unroll
      for (int m = 0; m < D; ++m) ti[m] = valid ? ld4(tq4<BLK>(t, N, D, nC, nl, m, I * 16 + 4 * ig)) : zero;
#pragma unroll
      for (int ii = 0; ii < 4; ++ii) {
        const int il = 4 * ig + ii;
        f4 a = zero;
#pragma unroll
        for (int m = 0; m < D; ++m) a += ti[m][ii] * tj[m];
        a *= scale;
#pragma unroll
        for (int ct = 0; ct < CT; ++ct)
          acc[ct] = mfma_k16(a, *reinterpret_cast<const f4*>(wp + (il * S + ct * 16) * 16), acc[ct]);
      }
    }
    if (++J == nb) { ++I; J = I; }
  }
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const int64_t node = (int64_t)tile * NN + wave * 16 + 4 * q + i;
    if (node >= N) continue;
#pragma unroll
    for (int ct = 0; ct < CT; ++ct) part[((int64_t)chunk * N + node) * S + ct * 16 + r] = acc[ct][i];
  }
}

// Forward with split-fp16 products on v_mfma_f32_32x32x16_f16 (32 nodes x 32 outputs per MFMA; the
// Gram values of node n are scaled by nsc[n], the weights by sw, both undone on the result).  A
// workgroup is 256 nodes (8 waves x 32) x one chunk of pchunk pairs; lane (r, q) of a wave is node r
// and K half q.  Step s (0..15) of a pair contracts K = 8q + j <-> (il = 8q + j, jl = s), so a lane
// keeps t[n][m][I0 + 8q + j] (unchanged along a row of pairs) and streams t[n][m][J0 + s] four steps at
// a time: the next group's loads are issued once the group's last G values are formed (TSB = 1, in
// flight during that step's products) or a whole group ahead into a second buffer (TSB = 2, 4D more
// registers; no faster at these sizes).  The pair's two
// weight planes ([jl][il/8][o][il%8]: the 32 lanes of a K half read 512 contiguous bytes) are staged
// in LDS and shared by the 8 waves; the next pair's planes are loaded a quarter at a time after each
// group's t loads, so waiting for those never waits for the weights (one in-order load counter).
// DL (D >= 5): the next pair's planes go straight from global memory into a second LDS buffer
// (direct-to-LDS loads, a quarter after each group's t loads) instead of through 32 registers, which the
// larger D need for their t operands (at D 9 the register copy spilled); the 128 KB of LDS leave one
// workgroup per CU, the occupancy those D have anyway (D 9: 0.274 -> 0.264 ms, D 7 0.704 -> 0.689 ms at
// 10k nodes; at D 3 it measured no faster).
constexpr int NODES_BF = 256;
typedef float f16v __attribute__((ext_vector_type(16)));
typedef __attribute__((address_space(1))) void gram_global_void;
typedef __attribute__((address_space(3))) void gram_lds_void;

template <int D, int S, int TSB, bool DL, bool BLK>
__global__ __launch_bounds__(512) void forward_h16_kernel(int64_t N, int nC, float scale,
                                                          const float* __restrict__ t,
                                                          const _Float16* __restrict__ Wf2,
                                                          const float* __restrict__ winv,
                                                          const float* __restrict__ nsc, int nchunks,
                                                          int pchunk, float* __restrict__ part, int tgroup) {
  constexpr int NN = NODES_BF, CT = S / 32;
  constexpr int PSZ = 256 * S;            // fp16 per plane of a pair
  constexpr int PW = 2 * PSZ / 8 / 512;   // 16-byte pieces of a pair per thread
  constexpr int PWQ = (PW + 3) / 4;
  static_assert((2 * PSZ / 8) % 512 == 0, "staging");
  __shared__ __align__(16) _Float16 wlb[DL ? 2 : 1][2 * PSZ];
  const int nb = nC / 16, np = n_pairs(nb);
  const int ntiles = (int)((N + NN - 1) / NN);
  const int logical = xcd_logical(nchunks * ntiles);
  if (logical < 0) return;
  int chunk, tile;
  group_order(logical, nchunks, ntiles, chunk, tile, tgroup);
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int r = lane & 31, q = lane >> 5;
  const int64_t n = (int64_t)tile * NN + wave * 32 + r;
  const bool valid = n < N;
  const int64_t nl = valid ? n : 0;   // rows past N read node 0; their results are not stored
  const float sn = valid ? nsc[n] : 1.f;
  const int p0 = chunk * pchunk, p1 = min(p0 + pchunk, np);
  int I = 0, rowstart = 0;
  while (rowstart + (nb - I) <= p0) { rowstart += nb - I; ++I; }
  int J = I + (p0 - rowstart);
  f16v acc[CT];
#pragma unroll
  for (int ct = 0; ct < CT; ++ct)
#pragma unroll
    for (int v = 0; v < 16; ++v) acc[ct][v] = 0.f;
  const f4 zero = {0.f, 0.f, 0.f, 0.f};
  const int64_t plane = (int64_t)np * PSZ;
  f4 pw[DL ? 1 : PW];
  int buf = 0;
  auto fetch_part = [&](int p, int k) {
#pragma unroll
    for (int i = k * PWQ; i < min(PW, (k + 1) * PWQ); ++i) {
      const int idx = threadIdx.x + 512 * i;
      const int pl = idx / (PSZ / 8), rem = idx - pl * (PSZ / 8);
      const _Float16* src = Wf2 + pl * plane + (int64_t)p * PSZ + 8 * rem;
      if constexpr (DL) {
        // lane l of the wave lands at the wave's base + 16 l: piece idx at 16 idx bytes, as below
        __builtin_amdgcn_global_load_lds((gram_global_void*)src,
                                         (gram_lds_void*)(&wlb[buf ^ 1][8 * (512 * i + 64 * wave)]), 16, 0, 0);
      } else {
        pw[i] = *reinterpret_cast<const f4*>(src);
      }
    }
  };
  // t[n][m][I0 + 8q + j] times the node's power of two (exact), so the Gram values come out scaled
  float tc[D][8];
  auto load_tc = [&](int Ib) {
#pragma unroll
    for (int m = 0; m < D; ++m) {
      const f4 a = valid ? ld4(tq4<BLK>(t, N, D, nC, nl, m, Ib * 16 + 8 * q)) : zero;
      const f4 b = valid ? ld4(tq4<BLK>(t, N, D, nC, nl, m, Ib * 16 + 8 * q + 4)) : zero;
      tc[m][0] = a.x * sn; tc[m][1] = a.y * sn; tc[m][2] = a.z * sn; tc[m][3] = a.w * sn;
      tc[m][4] = b.x * sn; tc[m][5] = b.y * sn; tc[m][6] = b.z * sn; tc[m][7] = b.w * sn;
    }
  };
  f4 ts[TSB][D];
  auto load_ts = [&](int b, int Jb, int sg) {
#pragma unroll
    for (int m = 0; m < D; ++m) ts[b][m] = valid ? ld4(tq4<BLK>(t, N, D, nC, nl, m, Jb * 16 + 4 * sg)) : zero;
  };
  load_tc(I);
  load_ts(0, J, 0);
  buf = 1;   // DL: the first pair goes to buffer 0
#pragma unroll
  for (int k = 0; k < 4; ++k) fetch_part(p0, k);
  buf = 0;
  for (int p = p0; p < p1; ++p) {
    if constexpr (DL) {
      __builtin_amdgcn_s_waitcnt(0);   // this pair's planes (direct-to-LDS loads are not tracked otherwise)
      __syncthreads();
    } else {
      __syncthreads();
#pragma unroll
      for (int i = 0; i < PW; ++i) reinterpret_cast<f4*>(wlb[0])[threadIdx.x + 512 * i] = pw[i];
      __syncthreads();
    }
    const _Float16* wl = wlb[DL ? buf : 0];
    const _Float16* wp = wl + q * S * 8 + r * 8;
    const bool more = p + 1 < p1;
    int In = I, Jn = J + 1;
    if (Jn == nb) { ++In; Jn = In; }
#pragma unroll
    for (int sg = 0; sg < 4; ++sg) {
      const int cur = (TSB == 2) ? (sg & 1) : 0;
      if constexpr (TSB == 2) {
        if (sg < 3) load_ts((sg + 1) & 1, J, sg + 1);
        else if (more) load_ts(0, Jn, 0);
        if (more) fetch_part(p + 1, sg);
      }
#pragma unroll
      for (int ss = 0; ss < 4; ++ss) {
        const int s = 4 * sg + ss;
        float gv[8];
#pragma unroll
        for (int j = 0; j < 8; ++j) {
          float a = 0.f;
#pragma unroll
          for (int m = 0; m < D; ++m) a += tc[m][j] * ts[cur][m][ss];
          gv[j] = a;
        }
        if constexpr (TSB == 1) {
          if (ss == 3) {
            __builtin_amdgcn_sched_barrier(0);
            if (sg < 3) load_ts(0, J, sg + 1);
            else if (more) load_ts(0, Jn, 0);
            if (more) fetch_part(p + 1, sg);
            __builtin_amdgcn_sched_barrier(0);
          }
        }
        h8 ah, al;
        split2h_pk(gv, ah, al);
#pragma unroll
        for (int ct = 0; ct < CT; ++ct) {
          const _Float16* b = wp + (s * 2 * S + ct * 32) * 8;
          const h8 bh = *reinterpret_cast<const h8*>(b);
          const h8 bl = *reinterpret_cast<const h8*>(b + PSZ);
          f16v c = acc[ct];
          c = __builtin_amdgcn_mfma_f32_32x32x16_f16(al, bh, c, 0, 0, 0);
          c = __builtin_amdgcn_mfma_f32_32x32x16_f16(ah, bl, c, 0, 0, 0);
          acc[ct] = __builtin_amdgcn_mfma_f32_32x32x16_f16(ah, bh, c, 0, 0, 0);
        }
      }
    }
    if (more && In != I) load_tc(In);
    I = In;
    J = Jn;
    if constexpr (DL) buf ^= 1;
  }
  // result register v of lane (r, q) is node 8 (v / 4) + 4 q + v % 4 of the wave, output column r
  const float f = scale * winv[0];
#pragma unroll
  for (int v = 0; v < 16; ++v) {
    const int64_t node = (int64_t)tile * NN + wave * 32 + 8 * (v / 4) + 4 * q + (v % 4);
    if (node >= N) continue;
    const float fn = f / nsc[node];   // nsc is a power of two: exact
#pragma unroll
    for (int ct = 0; ct < CT; ++ct) part[((int64_t)chunk * N + node) * S + ct * 32 + r] = acc[ct][v] * fn;
  }
}

// out[n][o] = sum over chunks of part[chunk][n][o] (fixed order: deterministic).  Four outputs per thread
// as float4s when NS is a multiple of 4 and the buffers are 16-byte aligned; eight chunks' loads in flight.
__global__ __launch_bounds__(256) void reduce_kernel(int64_t NS, int nchunks, const float* __restrict__ part,
                                                     float* __restrict__ out) {
  const int64_t stride = (int64_t)gridDim.x * blockDim.x;
  if ((NS & 3) == 0 && ((reinterpret_cast<uintptr_t>(part) | reinterpret_cast<uintptr_t>(out)) & 15) == 0) {
    const int64_t NS4 = NS >> 2;
    const f4* p4 = reinterpret_cast<const f4*>(part);
    for (int64_t i = blockIdx.x * (int64_t)blockDim.x + threadIdx.x; i < NS4; i += stride) {
      f4 s = f4{0.f, 0.f, 0.f, 0.f};
#pragma unroll 8
      for (int c = 0; c < nchunks; ++c) s += p4[(int64_t)c * NS4 + i];
      reinterpret_cast<f4*>(out)[i] = s;
    }
    return;
  }
  for (int64_t i = blockIdx.x * (int64_t)blockDim.x + threadIdx.x; i < NS; i += stride) {
    float s = 0.f;
    for (int c = 0; c < nchunks; ++c) s += part[(int64_t)c * NS + i];
    out[i] = s;
  }
}

// Backward: one workgroup per (node tile, row block I); a wave takes 16 nodes x ILW rows il of the
// block (ILW = 16: 128 nodes per workgroup, ILW = 8: two waves per node group, 64 nodes).  Per J the
// (I,J) block of (W + W^T) [a][b][o] is staged in LDS from its two fp16 planes (scaled by sw; rows
// padded so both the direct and the transposed reads are free of bank conflicts) and shared by the 8
// waves; the next J's block and t rows are loaded into registers meanwhile.  The MFMA (split-fp16,
// mfma_x3: fp32 accuracy at 5x the fp32 MFMA rate) takes A = (W + W^T) rows jl (K = o, in steps of 32:
// lane group q holds o = 32 ks + 8q .. +7) and B = g of the wave's 16 nodes, each node's g scaled by a
// power of two from its own max |g| and split once.  Lane (r = node, q) ends with A_n[il][4q..4q+3] and
// contracts it on the VALU with its own t[n][m][J0+4q..J0+4q+3]; the partial sums over q are reduced
// once, after the J loop, with a butterfly that leaves lane q the rows il of its quarter, and both
// scales are undone on the result.
template <int D, int S, int ILW, bool PIPE, bool BLK>
__global__ __launch_bounds__(512, D == 1 ? 4 : 2) void backward_h16_kernel(int64_t N, int nC, float scale,
                                                           const float* __restrict__ g, const float* __restrict__ t,
                                                           const _Float16* __restrict__ Wb2,
                                                           const float* __restrict__ winv, float* __restrict__ dt) {
  constexpr int NGRP = 16 / ILW;                 // waves sharing a node group
  constexpr int NN = 16 * 8 / NGRP;              // nodes per workgroup
  constexpr int KS = S / 32;
  constexpr int RS = S + 8, AS = 16 * RS + 8, PS = 16 * AS;   // padded fp16 strides of b, a and a plane
  constexpr int PW = 2 * 256 * S / 8 / 512;                   // 16-byte pieces of a block per thread
  static_assert(2 * 256 * S / 8 % 512 == 0, "block staging");
  __shared__ __align__(16) _Float16 wl[2 * PS];
  const int nb = nC / 16, np = n_pairs(nb);
  const int ntiles = (int)((N + NN - 1) / NN);
  const int logical = xcd_logical(nb * ntiles);
  if (logical < 0) return;
  const int I = logical / ntiles, tile = logical - I * ntiles;
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int r = lane & 15, q = lane >> 4;
  const int il0 = (wave % NGRP) * ILW;
  const int64_t n = (int64_t)tile * NN + (wave / NGRP) * 16 + r;
  const bool valid = n < N;
  const int64_t nl = valid ? n : 0;   // rows past N read node 0; their results are not stored
  const f4 zero = {0.f, 0.f, 0.f, 0.f};
  // the S values of a node's g are spread over lanes r, r + 16, r + 32, r + 48
  float gv[KS][8];
  float gmax = 0.f;
#pragma unroll
  for (int ks = 0; ks < KS; ++ks) {
    const f4 x0 = valid ? ld4(g + n * S + 32 * ks + 8 * q) : zero;
    const f4 x1 = valid ? ld4(g + n * S + 32 * ks + 8 * q + 4) : zero;
    gv[ks][0] = x0.x; gv[ks][1] = x0.y; gv[ks][2] = x0.z; gv[ks][3] = x0.w;
    gv[ks][4] = x1.x; gv[ks][5] = x1.y; gv[ks][6] = x1.z; gv[ks][7] = x1.w;
#pragma unroll
    for (int j = 0; j < 8; ++j) gmax = fmaxf(gmax, fabsf(gv[ks][j]));
  }
  gmax = fmaxf(gmax, __shfl_xor(gmax, 16, 64));
  gmax = fmaxf(gmax, __shfl_xor(gmax, 32, 64));
  const float sg = pow2_scale(gmax);
  h8 gh[KS], gl[KS];
#pragma unroll
  for (int ks = 0; ks < KS; ++ks) split2h(gv[ks], sg, gh[ks], gl[ks]);
  float acc[ILW][D];
#pragma unroll
  for (int i = 0; i < ILW; ++i)
#pragma unroll
    for (int m = 0; m < D; ++m) acc[i][m] = 0.f;
  f4 pw[PW], tq[D];
  const int64_t plane = (int64_t)np * 256 * S;
  auto fetch = [&](int J) {
    const int pr = (I <= J) ? pair_index(I, J, nb) : pair_index(J, I, nb);
#pragma unroll
    for (int i = 0; i < PW; ++i) {
      const int idx = threadIdx.x + 512 * i;   // (plane, 8-value piece of the block)
      const int pl = idx / (256 * S / 8), rem = idx - pl * (256 * S / 8);
      pw[i] = *reinterpret_cast<const f4*>(Wb2 + pl * plane + (int64_t)pr * 256 * S + 8 * rem);
    }
#pragma unroll
    for (int m = 0; m < D; ++m) tq[m] = ld4(tq4<BLK>(t, N, D, nC, nl, m, J * 16 + 4 * q));
  };
  fetch(0);
  for (int J = 0; J < nb; ++J) {
    __syncthreads();
#pragma unroll
    for (int i = 0; i < PW; ++i) {
      const int idx = threadIdx.x + 512 * i;
      const int pl = idx / (256 * S / 8), rem = idx - pl * (256 * S / 8);
      const int ab = rem / (S / 8), o8 = rem % (S / 8);
      *reinterpret_cast<f4*>(&wl[pl * PS + (ab >> 4) * AS + (ab & 15) * RS + 8 * o8]) = pw[i];
    }
    __syncthreads();
    f4 tc[D];
#pragma unroll
    for (int m = 0; m < D; ++m) tc[m] = tq[m];
    if (J + 1 < nb) fetch(J + 1);
    __builtin_amdgcn_sched_barrier(0);
    // A[row = jl][k = o] = (W + W^T)[o][I0 + il][J0 + jl]: block [a = il][b = jl] if I <= J, else [a = jl][b = il]
    const bool upper = I <= J;
    const int rbase = (upper ? r * RS : r * AS) + 8 * q;
    const int ilstep = upper ? AS : RS;
    // PIPE: the operands of step u + 1 are read from LDS before the products of step u are issued (at 2
    // waves per SIMD the compiler's own order waits on each read; costs 12 registers)
    constexpr int NSTEP = (ILW / 4) * KS * 4;
    h8 oh[2], ol[2];
    auto rd = [&](int u, int slot) {
      const int i4 = u / (KS * 4), ks = (u / 4) % KS, jj = u % 4;
      const int off = rbase + (il0 + 4 * i4 + jj) * ilstep + 32 * ks;
      oh[slot] = *reinterpret_cast<const h8*>(&wl[off]);
      ol[slot] = *reinterpret_cast<const h8*>(&wl[PS + off]);
    };
    if constexpr (PIPE) rd(0, 0);
#pragma unroll
    for (int i4 = 0; i4 < ILW / 4; ++i4) {
      f4 dd[4] = {zero, zero, zero, zero};
#pragma unroll
      for (int ks = 0; ks < KS; ++ks)
#pragma unroll
        for (int jj = 0; jj < 4; ++jj) {
          const int u = (i4 * KS + ks) * 4 + jj;
          if constexpr (PIPE) {
            if (u + 1 < NSTEP) rd(u + 1, (u + 1) & 1);
            __builtin_amdgcn_sched_barrier(0);
          } else {
            rd(u, u & 1);
          }
          dd[jj] = mfma_x3(oh[u & 1], ol[u & 1], gh[ks], gl[ks], dd[jj]);
        }
#pragma unroll
      for (int jj = 0; jj < 4; ++jj)
#pragma unroll
        for (int m = 0; m < D; ++m) {
          // one fma per product into the running sum (a sum of products added at the end costs a mul
          // and an add more per four products)
          float a = acc[4 * i4 + jj][m];
#pragma unroll
          for (int k = 0; k < 4; ++k) a = fmaf(dd[jj][k], tc[m][k], a);
          acc[4 * i4 + jj][m] = a;
        }
    }
  }
  constexpr int H = ILW / 2, QR = ILW / 4;
  const bool hi = (q & 2) != 0, odd = (q & 1) != 0;
  float h1[H][D];
#pragma unroll
  for (int i = 0; i < H; ++i)
#pragma unroll
    for (int m = 0; m < D; ++m)
      h1[i][m] = (hi ? acc[H + i][m] : acc[i][m]) + __shfl_xor(hi ? acc[i][m] : acc[H + i][m], 32, 64);
  float h2[QR][D];
#pragma unroll
  for (int i = 0; i < QR; ++i)
#pragma unroll
    for (int m = 0; m < D; ++m)
      h2[i][m] = (odd ? h1[QR + i][m] : h1[i][m]) + __shfl_xor(odd ? h1[i][m] : h1[QR + i][m], 16, 64);
  if (valid) {
    const float f = scale * winv[0] / sg;   // sg is a power of two: exact
#pragma unroll
    for (int m = 0; m < D; ++m) {
      float* o = dt + (n * D + m) * nC + I * 16 + il0 + QR * q;
#pragma unroll
      for (int i = 0; i < QR; ++i) o[i] = h2[i][m] * f;
    }
  }
}

int check_dims(int64_t N, int32_t D, int32_t nC, int32_t S, const char* who) {
  if (N < 0 || N >= (1LL << 31) || nC < 16 || nC % 16 != 0 || nC > 16 * 64 || !(S == 32 || S == 64) ||
      !(D == 1 || D == 3 || D == 5 || D == 7 || D == 9)) {
    set_error(std::string(who) + ": need D in {1,3,5,7,9}, nC a multiple of 16 (<= 1024), S 32 or 64");
    return 1;
  }
  return 0;
}

// Forward kernel choice and block pairs per workgroup.  The split-fp16 kernel runs 256-node tiles at
// several times the fp32 kernel's rate per node; with at most 128 of its workgroups (one partial round
// on 256 CUs) the fp32 kernel's twice as many smaller workgroups finish first.  The fp32 kernel (few
// nodes) takes fewer pairs per workgroup, down to one, until there are about two workgroups per CU:
// at 1,000 nodes and nC 192 that is 624 workgroups of one pair instead of 40 of sixteen.
struct FwdPlan {
  bool bf;
  int pchunk, nchunks;
};
FwdPlan fwd_plan(int64_t N, int nC) {
  const int np = n_pairs(nC / 16);
  FwdPlan pl;
  const int64_t ntb = (N + NODES_BF - 1) / NODES_BF;
  pl.bf = (int64_t)((np + PCHUNK - 1) / PCHUNK) * ntb > 128;
  pl.pchunk = PCHUNK;
  // the split-fp16 kernel takes 16 pairs per workgroup while that still leaves more than 128 workgroups:
  // 6 % faster at nC 384 (10,000 nodes, 760 workgroups), 5 % at nC 192 (10,000 nodes, 200 workgroups)
  if (pl.bf && (int64_t)((np + 2 * PCHUNK - 1) / (2 * PCHUNK)) * ntb > 128) pl.pchunk = 2 * PCHUNK;
  if (!pl.bf) {
    const int64_t ntiles = (N + NODES - 1) / NODES;
    while (pl.pchunk > 1 && (int64_t)((np + pl.pchunk - 1) / pl.pchunk) * ntiles < 512) pl.pchunk /= 2;
  }
  pl.nchunks = (np + pl.pchunk - 1) / pl.pchunk;
  return pl;
}

template <int S, bool BLK>
int forward_s(int64_t N, int D, int nC, float scale, const float* t, const float* Wf, float* part, float* out,
              hipStream_t st) {
  const int np = n_pairs(nC / 16);
  const FwdPlan pl = fwd_plan(N, nC);
  const int nchunks = pl.nchunks, pchunk = pl.pchunk;
  const bool bf = pl.bf;
  const int ntiles = (int)((N + (bf ? NODES_BF : NODES) - 1) / (bf ? NODES_BF : NODES));
  const unsigned grid = (unsigned)(((int64_t)nchunks * ntiles + 7) / 8 * 8);
  const _Float16* Wf2 = reinterpret_cast<const _Float16*>(Wf + (int64_t)np * 256 * S);
  const float* winv = Wf + (int64_t)np * 512 * S;
  float* nsc = part + (int64_t)nchunks * N * S;
  if (bf) {
    if (BLK)
      node_scale_blocked_kernel<<<(unsigned)((N + 63) / 64), 512, 0, st>>>(N, D, nC, t, nsc);
    else
      node_scale_kernel<<<(unsigned)((N + 3) / 4), 256, 0, st>>>(N, D, nC, t, nsc);
    if (check_launch("gram node scales")) return 2;
  }
  // tiles per group: as many as keep the group's t rows within about half an XCD's 4 MB L2 (at D 7,
  // nC 384 a 256-node tile alone is 2.75 MB; larger groups re-fetch t for every pair chunk)
  const int64_t tile_bytes = (int64_t)NODES_BF * D * nC * 4;
  const int tg = (int)std::max<int64_t>(1, std::min<int64_t>(TILE_GROUP, (2 << 20) / tile_bytes));
  {
    LaunchTimer tm("gram_forward", st);
#define FSC_GF(DD)                                                                                 \
  if (bf)                                                                                          \
    forward_h16_kernel<DD, S, 1, (DD >= 5), BLK><<<grid, 512, 0, st>>>(N, nC, scale, t, Wf2, winv, nsc, nchunks, \
                                                                      pchunk, part, tg);                        \
  else                                                                                             \
    forward_kernel<DD, S, BLK><<<grid, 512, 0, st>>>(N, nC, scale, t, Wf, nchunks, part, pchunk)
    switch (D) {
      case 1: FSC_GF(1); break;
      case 3: FSC_GF(3); break;
      case 5: FSC_GF(5); break;
      case 7: FSC_GF(7); break;
      default: FSC_GF(9); break;
    }
#undef FSC_GF
  }
  if (check_launch("gram forward")) return 2;
  const int64_t NS = N * S;
  reduce_kernel<<<(unsigned)std::min<int64_t>(((NS + 3) / 4 + 255) / 256, 4096), 256, 0, st>>>(NS, nchunks, part, out);
  return check_launch("gram reduce") ? 2 : 0;
}

// largest D whose backward has the registers for the operand pipeline (at D 9 it spills)
constexpr int GB_PIPE_DMAX = 7;

template <int S, bool BLK>
int backward_s(int64_t N, int D, int nC, float scale, const float* g, const float* t, const float* Wb, float* dt,
               hipStream_t st) {
  // 16 rows il per wave while the accumulators (16 x D) fit the registers, else 8.
  const int nn = (D <= 5) ? NODES : NODES / 2;
  const int ntiles = (int)((N + nn - 1) / nn);
  const unsigned grid = (unsigned)(((int64_t)(nC / 16) * ntiles + 7) / 8 * 8);
  const _Float16* Wb2 = reinterpret_cast<const _Float16*>(Wb + (int64_t)n_pairs(nC / 16) * 256 * S);
  const float* winv = Wb + (int64_t)n_pairs(nC / 16) * 512 * S;
  LaunchTimer tm("gram_backward", st);
#define FSC_GBB(DD) \
  backward_h16_kernel<DD, S, (DD <= 5 ? 16 : 8), (DD > 1 && DD <= GB_PIPE_DMAX), BLK><<<grid, 512, 0, st>>>(N, nC, scale, \
                                                                                                    g, t, Wb2, \
                                                                                            winv, dt)
  switch (D) {
    case 1: FSC_GBB(1); break;
    case 3: FSC_GBB(3); break;
    case 5: FSC_GBB(5); break;
    case 7: FSC_GBB(7); break;
    default: FSC_GBB(9); break;
  }
#undef FSC_GBB
  return check_launch("gram backward") ? 2 : 0;
}

}  // namespace gram
}  // namespace fsc

using namespace fsc;
using namespace fsc::gram;

extern "C" {

int fsc_gram_sizes(int64_t n_nodes, int32_t nC, int32_t S, int64_t* wf_floats, int64_t* wb_floats,
                   int64_t* workspace_floats) {
  FSC_CHECK_ARG(wf_floats && wb_floats && workspace_floats, "fsc_gram_sizes: null pointer");
  FSC_CHECK_ARG(n_nodes >= 0 && nC >= 16 && nC % 16 == 0 && nC <= 1024 && (S == 32 || S == 64),
                "fsc_gram_sizes: nC must be a multiple of 16 (<= 1024), S 32 or 64");
  *wf_floats = gram_weight_floats(nC / 16, S);   // fp32 block pairs, two fp16 planes, scale and maxima
  *wb_floats = *wf_floats;
  // per-chunk partial sums, then one scale per node
  *workspace_floats = (int64_t)fwd_plan(n_nodes, nC).nchunks * n_nodes * S + n_nodes;
  return 0;
}

int fsc_gram_prepare_weights(const float* W, int32_t S, int32_t nC, float* Wf, float* Wb, hipStream_t stream) {
  FSC_CHECK_ARG(W && Wf && Wb, "fsc_gram_prepare_weights: null pointer");
  FSC_CHECK_ARG(nC >= 16 && nC % 16 == 0 && nC <= 1024 && (S == 32 || S == 64),
                "fsc_gram_prepare_weights: nC must be a multiple of 16 (<= 1024), S 32 or 64");
  const int nb = nC / 16;
  float* wmax = Wf + gram_weight_floats(nb, S) - GW_TAIL + 256;
  absmax_kernel<<<WMAX_BLOCKS, 256, 0, stream>>>(W, (int64_t)S * nC * nC, wmax);
  if (check_launch("gram weight maximum")) return 2;
  prepare_kernel<<<dim3(nb, nb, S / 16), 256, 0, stream>>>(W, S, nC, Wf, Wb, wmax);
  return check_launch("gram prepare") ? 2 : 0;
}

static int gram_forward_any(bool blk, int64_t n_nodes, int32_t D, int32_t nC, int32_t S, float scale,
                            const float* t, const float* Wf, float* part_ws, float* out, hipStream_t stream,
                            const char* who) {
  if (check_dims(n_nodes, D, nC, S, who)) return 1;
  FSC_CHECK_ARG(Wf && (n_nodes == 0 || (t && part_ws && out)), std::string(who) + ": null pointer");
  FSC_CHECK_ARG(!blk || (reinterpret_cast<uintptr_t>(t) & 15) == 0, std::string(who) + ": t must be 16-byte aligned");
  if (n_nodes == 0) return 0;
  if (blk) {
    if (S == 64) return forward_s<64, true>(n_nodes, D, nC, scale, t, Wf, part_ws, out, stream);
    return forward_s<32, true>(n_nodes, D, nC, scale, t, Wf, part_ws, out, stream);
  }
  if (S == 64) return forward_s<64, false>(n_nodes, D, nC, scale, t, Wf, part_ws, out, stream);
  return forward_s<32, false>(n_nodes, D, nC, scale, t, Wf, part_ws, out, stream);
}

static int gram_backward_any(bool blk, int64_t n_nodes, int32_t D, int32_t nC, int32_t S, float scale,
                             const float* grad_out, const float* t, const float* Wb, float* grad_t,
                             hipStream_t stream, const char* who) {
  if (check_dims(n_nodes, D, nC, S, who)) return 1;
  FSC_CHECK_ARG(Wb && (n_nodes == 0 || (grad_out && t && grad_t)), std::string(who) + ": null pointer");
  FSC_CHECK_ARG(!blk || (reinterpret_cast<uintptr_t>(t) & 15) == 0, std::string(who) + ": t must be 16-byte aligned");
  if (n_nodes == 0) return 0;
  if (blk) {
    if (S == 64) return backward_s<64, true>(n_nodes, D, nC, scale, grad_out, t, Wb, grad_t, stream);
    return backward_s<32, true>(n_nodes, D, nC, scale, grad_out, t, Wb, grad_t, stream);
  }
  if (S == 64) return backward_s<64, false>(n_nodes, D, nC, scale, grad_out, t, Wb, grad_t, stream);
  return backward_s<32, false>(n_nodes, D, nC, scale, grad_out, t, Wb, grad_t, stream);
}

int fsc_gram_forward(int64_t n_nodes, int32_t D, int32_t nC, int32_t S, float scale, const float* t,
                     const float* Wf, float* part_ws, float* out, hipStream_t stream) {
  return gram_forward_any(false, n_nodes, D, nC, S, scale, t, Wf, part_ws, out, stream, "fsc_gram_forward");
}

int fsc_gram_backward(int64_t n_nodes, int32_t D, int32_t nC, int32_t S, float scale, const float* grad_out,
                      const float* t, const float* Wb, float* grad_t, hipStream_t stream) {
  return gram_backward_any(false, n_nodes, D, nC, S, scale, grad_out, t, Wb, grad_t, stream, "fsc_gram_backward");
}

int fsc_gram_forward_blocked(int64_t n_nodes, int32_t D, int32_t nC, int32_t S, float scale, const float* t,
                             const float* Wf, float* part_ws, float* out, hipStream_t stream) {
  return gram_forward_any(true, n_nodes, D, nC, S, scale, t, Wf, part_ws, out, stream, "fsc_gram_forward_blocked");
}

int fsc_gram_backward_blocked(int64_t n_nodes, int32_t D, int32_t nC, int32_t S, float scale,
                              const float* grad_out, const float* t, const float* Wb, float* grad_t,
                              hipStream_t stream) {
  return gram_backward_any(true, n_nodes, D, nC, S, scale, grad_out, t, Wb, grad_t, stream,
                           "fsc_gram_backward_blocked");
}

}  // extern "C"
