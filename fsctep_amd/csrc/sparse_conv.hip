// pure-cartesian-sparse message passing on gfx950.
//
// Replaces, for conv2..n, the per-edge weight generation + sparse tensor product +
// receiver scatter of the reference (models/pure_cartesian_sparse_layers.py:382-421,
// models/pure_cartesian.py:790-863, utils/scatter.py:63-116), and for conv1 the same
// chain with the neighbour-scalar operand (models/pure_cartesian_sparse_layers.py:227-330).
//
// Algebra (exact; only the order of floating-point sums changes).  The last radial-MLP
// layer is W_e[p,c,a] = sum_k L[(p,c,a),k] h_e[k] + b[(p,c,a)], and every sparse path
// is an outer product x_src[a, I] (x) Y_e[J].  Summing over a before k gives
//   S_m[(slot,c), k] = sum_a L[(p,c,a),k] x_m[comp(slot), a]      (per source node, K1)
//   P_e[(slot,c)]    = sum_k h_e[k] S_src[(slot,c),k] + Sb_src     (per edge, K2)
//   out_n            = scale * sum_{e->n} assemble(P_e, n_e)       (per receiver, K3)
// with 18 slots = (path, source component): p0..p2 use x0 (slots 0,1,2), p3/p4 use x1[i]
// (slots 3+i, 6+i), p5 uses x2[ij] (slots 9+ij).  The messages are
//   m0 = P0,  m1[i] = P1 n_i + P3[i],  m2[ij] = P2 n_i n_j + P4[i] n_j + P5[ij].
// The per-edge weight tensor (6*C*C floats) is never formed.
//
// Layouts (fp32): node features x[N][13][C] (comp-major: 0 | 1..3 = i | 4..12 = 3i+j);
// S[N][18][65*C]: per slot a row of C*64 (c-major, k-minor) then C bias entries;
// P[E][18*C] at the receiver-sorted edge id; h[E][64]; n[E][3] (unit vectors).

#include "common.h"

namespace fsc {
namespace sparse {

constexpr int KH = 64;        // radial hidden width (fixed by the reference's fc)
constexpr int NSLOT = 18;
constexpr int NCOMP = 13;
__constant__ int kSlotBase[6] = {0, 1, 2, 3, 6, 9};
__constant__ int kPathL1[6] = {0, 0, 0, 1, 1, 2};
constexpr int kCompBase[3] = {0, 1, 4};
constexpr int kNumI[3] = {1, 3, 9};
constexpr int kSlotBaseH[6] = {0, 1, 2, 3, 6, 9};
constexpr int kPathL1H[6] = {0, 0, 0, 1, 1, 2};

__host__ __device__ inline int64_t s_node_stride(int C) { return (int64_t)NSLOT * 65 * C; }

// ---------------------------------------------------------------- weight preparation
// bk1[p][col][a] (col < 64C: col = c*64+k -> L[(p,c,a),k]; col >= 64C: b[(p,c,a)])
// bk6[p][a][col] (transpose of bk1[p]).
__global__ void prep_weights_kernel(const float* __restrict__ L, const float* __restrict__ b,
                                    float* __restrict__ bk1, float* __restrict__ bk6, int C) {
  const int64_t cols = 65LL * C;
  const int64_t total = 6LL * cols * C;
  for (int64_t idx = blockIdx.x * (int64_t)blockDim.x + threadIdx.x; idx < total;
       idx += (int64_t)gridDim.x * blockDim.x) {
    const int a = (int)(idx % C);
    const int64_t col = (idx / C) % cols;
    const int p = (int)(idx / (C * cols));
    float v;
    if (col < 64LL * C) {
      const int c = (int)(col / 64), k = (int)(col % 64);
      v = L[((int64_t)p * C * C + (int64_t)c * C + a) * KH + k];
    } else {
      const int c = (int)(col - 64LL * C);
      v = b[(int64_t)p * C * C + (int64_t)c * C + a];
    }
    bk1[idx] = v;
    bk6[((int64_t)p * C + a) * cols + col] = v;
  }
}

// ---------------------------------------------------------------- K1: node expansion
// S[m][slot_base(p)+I][col] = sum_a x[m][comp0+I][a] * bk1[p][col][a]
// grid: (ceil(rows/64), ceil(65C/256)), block 256 (4 waves, one 16-row tile each,
// 16 column tiles of 16 per block).
template <int C>
__global__ __launch_bounds__(256) void node_expand_kernel(const float* __restrict__ x,
                                                          const float* __restrict__ bk1,
                                                          float* __restrict__ S, int64_t n_nodes,
                                                          int p) {
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int r = lane & 15, q = lane >> 4;
  const int L1 = kPathL1[p];
  const int nI = (L1 == 0) ? 1 : (L1 == 1 ? 3 : 9);
  const int comp0 = (L1 == 0) ? 0 : (L1 == 1 ? 1 : 4);
  const int sbase = kSlotBase[p];
  const int64_t rows = n_nodes * nI;
  const int64_t row0 = (int64_t)blockIdx.x * 64 + wave * 16;
  constexpr int COLS = 65 * C;
  constexpr int KT = C / 16;

  // A fragments: row (row0 + r), K = a
  f4 a4[KT];
  {
    const int64_t row = row0 + r;
    if (row < rows) {
      const int64_t m = row / nI;
      const int I = (int)(row % nI);
      const float* xr = x + (m * NCOMP + comp0 + I) * C;
#pragma unroll
      for (int t = 0; t < KT; ++t) a4[t] = ld4(xr + 16 * t + 4 * q);
    } else {
#pragma unroll
      for (int t = 0; t < KT; ++t) a4[t] = f4{0.f, 0.f, 0.f, 0.f};
    }
  }
  const float* bp = bk1 + (int64_t)p * COLS * C;
  const int col_base = blockIdx.y * 256;
#pragma unroll 1
  for (int ct = 0; ct < 16; ++ct) {
    const int colt = col_base + ct * 16;
    if (colt >= COLS) break;
    const int col = colt + r;
    f4 acc = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int t = 0; t < KT; ++t) {
      const f4 b4 = ld4(bp + (int64_t)col * C + 16 * t + 4 * q);
      acc = mfma_k16(a4[t], b4, acc);
    }
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const int64_t row = row0 + 4 * q + i;
      if (row < rows) {
        const int64_t m = row / nI;
        const int I = (int)(row % nI);
        S[m * s_node_stride(C) + (int64_t)(sbase + I) * COLS + col] = acc[i];
      }
    }
  }
}

// ---------------------------------------------------------------- K6: node expansion grad
// dx[m][comp0+I][a] = sum_{p in group} sum_col dS[m][slot_base(p)+I][col] * bk6[p][a][col]
// grid: ceil(rows/64), block 256 (4 waves x 16 rows), C/16 column tiles per wave.
template <int C>
__global__ __launch_bounds__(256) void node_expand_grad_kernel(const float* __restrict__ dS,
                                                               const float* __restrict__ bk6,
                                                               float* __restrict__ dx,
                                                               int64_t n_nodes, int group) {
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int r = lane & 15, q = lane >> 4;
  const int nI = (group == 0) ? 1 : (group == 1 ? 3 : 9);
  const int comp0 = (group == 0) ? 0 : (group == 1 ? 1 : 4);
  const int p_first = (group == 0) ? 0 : (group == 1 ? 3 : 5);
  const int p_count = (group == 0) ? 3 : (group == 1 ? 2 : 1);
  const int64_t rows = n_nodes * nI;
  const int64_t row0 = (int64_t)blockIdx.x * 64 + wave * 16;
  constexpr int COLS = 65 * C;
  constexpr int NT = C / 16;

  const int64_t arow = row0 + r;
  const bool arow_ok = arow < rows;
  const int64_t am = arow_ok ? arow / nI : 0;
  const int aI = arow_ok ? (int)(arow % nI) : 0;

  f4 acc[NT];
#pragma unroll
  for (int ct = 0; ct < NT; ++ct) acc[ct] = f4{0.f, 0.f, 0.f, 0.f};

  for (int pp = 0; pp < p_count; ++pp) {
    const int p = p_first + pp;
    const float* ar = dS + am * s_node_stride(C) + (int64_t)(kSlotBase[p] + aI) * COLS;
    const float* bp = bk6 + (int64_t)p * C * COLS;
#pragma unroll 2
    for (int t = 0; t < COLS / 16; ++t) {
      const f4 a4 = arow_ok ? ld4(ar + 16 * t + 4 * q) : f4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
      for (int ct = 0; ct < NT; ++ct) {
        const f4 b4 = ld4(bp + (int64_t)(16 * ct + r) * COLS + 16 * t + 4 * q);
        acc[ct] = mfma_k16(a4, b4, acc[ct]);
      }
    }
  }
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const int64_t row = row0 + 4 * q + i;
    if (row < rows) {
      const int64_t m = row / nI;
      const int I = (int)(row % nI);
      float* o = dx + (m * NCOMP + comp0 + I) * C;
#pragma unroll
      for (int ct = 0; ct < NT; ++ct) o[16 * ct + r] = acc[ct][i];
    }
  }
}

// ---------------------------------------------------------------- K2: edge message
// One block per source node; P[eid][col] = sum_k h[eid][k] S[m][col][k] + Sb[m][col].
constexpr int EP = 64;   // edges per pass held in LDS

template <int C>
__global__ __launch_bounds__(256) void edge_message_kernel(const float* __restrict__ h,
                                                           const float* __restrict__ S,
                                                           const int32_t* __restrict__ src_ptr,
                                                           const int32_t* __restrict__ src_perm,
                                                           float* __restrict__ P) {
  __shared__ float hs[EP][KH + 4];
  __shared__ int32_t eids[EP];
  const int m = blockIdx.x;
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int r = lane & 15, q = lane >> 4;
  const int beg = src_ptr[m], end = src_ptr[m + 1];
  constexpr int COLS = 65 * C;
  constexpr int NCT = NSLOT * C / 16;   // 16-wide column tiles of P
  const float* Sm = S + (int64_t)m * s_node_stride(C);

  for (int pb = beg; pb < end; pb += EP) {
    const int cnt = min(EP, end - pb);
    __syncthreads();
    for (int idx = threadIdx.x; idx < EP * (KH / 4); idx += 256) {
      const int e = idx / (KH / 4), k4 = (idx % (KH / 4)) * 4;
      f4 v = {0.f, 0.f, 0.f, 0.f};
      if (e < cnt) v = ld4(h + (int64_t)src_perm[pb + e] * KH + k4);
      *reinterpret_cast<f4*>(&hs[e][k4]) = v;
    }
    if (threadIdx.x < EP) eids[threadIdx.x] = (threadIdx.x < cnt) ? src_perm[pb + threadIdx.x] : -1;
    __syncthreads();
    const int nrt = (cnt + 15) / 16;
    for (int ct = wave; ct < NCT; ct += 4) {
      const int col = ct * 16 + r;        // flat (slot, c)
      const int slot = col / C, c = col % C;
      const float* srow = Sm + (int64_t)slot * COLS + c * KH;
      f4 b4[4];
#pragma unroll
      for (int t = 0; t < 4; ++t) b4[t] = ld4(srow + 16 * t + 4 * q);
      const float bias = Sm[(int64_t)slot * COLS + 64 * C + c];
      for (int rt = 0; rt < nrt; ++rt) {
        f4 acc = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
        for (int t = 0; t < 4; ++t) {
          const f4 a4 = *reinterpret_cast<const f4*>(&hs[rt * 16 + r][16 * t + 4 * q]);
          acc = mfma_k16(a4, b4[t], acc);
        }
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          const int e = rt * 16 + 4 * q + i;
          if (e < cnt) P[(int64_t)eids[e] * (NSLOT * C) + col] = acc[i] + bias;
        }
      }
    }
  }
}

// ---------------------------------------------------------------- K3: receiver sum
// One wave per receiver; lanes cover channels, 64/C edges in flight per wave.
template <int C>
__global__ __launch_bounds__(256) void receiver_sum_kernel(const float* __restrict__ P,
                                                           const float* __restrict__ nvec,
                                                           const int32_t* __restrict__ dst_ptr,
                                                           float scale, float* __restrict__ out,
                                                           int64_t n_nodes) {
  const int lane = threadIdx.x & 63;
  const int64_t n = (int64_t)blockIdx.x * 4 + (threadIdx.x >> 6);
  if (n >= n_nodes) return;
  constexpr int EPW = 64 / C;
  const int c = lane % C, sub = lane / C;
  float o[NCOMP];
#pragma unroll
  for (int i = 0; i < NCOMP; ++i) o[i] = 0.f;
  const int beg = dst_ptr[n], end = dst_ptr[n + 1];
  for (int e = beg + sub; e < end; e += EPW) {
    const float* pr = P + (int64_t)e * (NSLOT * C) + c;
    const float n0 = nvec[3 * (int64_t)e], n1 = nvec[3 * (int64_t)e + 1], n2 = nvec[3 * (int64_t)e + 2];
    const float nn[3] = {n0, n1, n2};
    const float p0 = pr[0], p1 = pr[C], p2 = pr[2 * C];
    o[0] += p0;
#pragma unroll
    for (int i = 0; i < 3; ++i) o[1 + i] += p1 * nn[i] + pr[(3 + i) * C];
#pragma unroll
    for (int i = 0; i < 3; ++i) {
      const float p4 = pr[(6 + i) * C];
      const float p2ni = p2 * nn[i];
#pragma unroll
      for (int j = 0; j < 3; ++j) o[4 + 3 * i + j] += p2ni * nn[j] + p4 * nn[j] + pr[(9 + 3 * i + j) * C];
    }
  }
  if (EPW > 1) {
#pragma unroll
    for (int i = 0; i < NCOMP; ++i)
      for (int off = C; off < 64; off <<= 1) o[i] += __shfl_xor(o[i], off, 64);
  }
  if (sub == 0) {
    float* orow = out + n * NCOMP * C + c;
#pragma unroll
    for (int i = 0; i < NCOMP; ++i) orow[i * C] = o[i] * scale;
  }
}

// ---------------------------------------------------------------- K4: direction gradient
// dn[e][k] = sum_c g1[k] P1 + P2 (sum_j g2[k][j] n_j + sum_i g2[i][k] n_i) + sum_i g2[i][k] P4[i]
template <int C>
__global__ __launch_bounds__(256) void direction_grad_kernel(const float* __restrict__ G,
                                                             const float* __restrict__ P,
                                                             const float* __restrict__ nvec,
                                                             const int32_t* __restrict__ dst_ptr,
                                                             float scale, float* __restrict__ dn,
                                                             int64_t n_nodes) {
  const int lane = threadIdx.x & 63;
  const int64_t n = (int64_t)blockIdx.x * 4 + (threadIdx.x >> 6);
  if (n >= n_nodes) return;
  constexpr int EPW = 64 / C;
  const int c = lane % C, sub = lane / C;
  float g[NCOMP];
#pragma unroll
  for (int i = 0; i < NCOMP; ++i) g[i] = G[(n * NCOMP + i) * C + c] * scale;
  const int beg = dst_ptr[n], end = dst_ptr[n + 1];
  for (int eb = beg; eb < end; eb += EPW) {
    const int e = eb + sub;
    float t0 = 0.f, t1 = 0.f, t2 = 0.f;
    if (e < end) {
      const float* pr = P + (int64_t)e * (NSLOT * C) + c;
      const float nn[3] = {nvec[3 * (int64_t)e], nvec[3 * (int64_t)e + 1], nvec[3 * (int64_t)e + 2]};
      const float p1 = pr[C], p2 = pr[2 * C];
      const float p4[3] = {pr[6 * C], pr[7 * C], pr[8 * C]};
      float t[3];
#pragma unroll
      for (int k = 0; k < 3; ++k) {
        float row = 0.f, colv = 0.f, p4t = 0.f;
#pragma unroll
        for (int j = 0; j < 3; ++j) {
          row += g[4 + 3 * k + j] * nn[j];
          colv += g[4 + 3 * j + k] * nn[j];
          p4t += g[4 + 3 * j + k] * p4[j];
        }
        t[k] = g[1 + k] * p1 + p2 * (row + colv) + p4t;
      }
      t0 = t[0]; t1 = t[1]; t2 = t[2];
    }
    t0 = group_sum(t0, C);
    t1 = group_sum(t1, C);
    t2 = group_sum(t2, C);
    if (c == 0 && e < end) {
      dn[3 * (int64_t)e] = t0;
      dn[3 * (int64_t)e + 1] = t1;
      dn[3 * (int64_t)e + 2] = t2;
    }
  }
}

// ---------------------------------------------------------------- K5: edge message grad
// One block per source node.  dP_e[(slot,c)] is rebuilt from the receiver gradient
// g = G[dst(e)]*scale and n_e, 64 columns at a time in LDS, then
//   dh[e][k]       += sum_col dP_e[col] S[m][col][k]     (MFMA, rows = edges)
//   dS[m][col][k]   = sum_e h[e][k] dP_e[col]            (MFMA, rows = columns)
//   dS[m][col][64C] = sum_e dP_e[col]                    (bias column)
template <int C>
__device__ __forceinline__ float dp_value(const float* __restrict__ g, int slot, const float* nn) {
  // g points at G[dst][0][c]; component stride C.
  switch (slot) {
    case 0: return g[0];
    case 1: return g[1 * C] * nn[0] + g[2 * C] * nn[1] + g[3 * C] * nn[2];
    case 2: {
      float s = 0.f;
#pragma unroll
      for (int i = 0; i < 3; ++i)
#pragma unroll
        for (int j = 0; j < 3; ++j) s += g[(4 + 3 * i + j) * C] * nn[i] * nn[j];
      return s;
    }
    case 3: case 4: case 5: return g[(1 + slot - 3) * C];
    case 6: case 7: case 8: {
      const int i = slot - 6;
      return g[(4 + 3 * i) * C] * nn[0] + g[(5 + 3 * i) * C] * nn[1] + g[(6 + 3 * i) * C] * nn[2];
    }
    default: return g[(4 + slot - 9) * C];
  }
}

template <int C>
__global__ __launch_bounds__(256) void edge_message_grad_kernel(
    const float* __restrict__ G, const float* __restrict__ nvec, const float* __restrict__ h,
    const float* __restrict__ S, const int32_t* __restrict__ src_ptr,
    const int32_t* __restrict__ src_perm, const int32_t* __restrict__ edge_dst, float scale,
    float* __restrict__ dh, float* __restrict__ dS) {
  __shared__ float hs[EP][KH + 4];
  __shared__ float dps[EP][64 + 4];
  __shared__ float ss[64][KH + 4];
  __shared__ int32_t eids[EP];
  __shared__ int32_t dsts[EP];
  __shared__ float ns[EP][3];
  const int m = blockIdx.x;
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int r = lane & 15, q = lane >> 4;
  const int beg = src_ptr[m], end = src_ptr[m + 1];
  constexpr int COLS = 65 * C;
  constexpr int NCOL = NSLOT * C;
  const float* Sm = S + (int64_t)m * s_node_stride(C);
  float* dSm = dS + (int64_t)m * s_node_stride(C);

  int pb = beg;
  bool first = true;
  do {
    const int cnt = min(EP, end - pb);   // may be 0 for a node without out-edges
    __syncthreads();
    for (int idx = threadIdx.x; idx < EP * (KH / 4); idx += 256) {
      const int e = idx / (KH / 4), k4 = (idx % (KH / 4)) * 4;
      f4 v = {0.f, 0.f, 0.f, 0.f};
      if (e < cnt) v = ld4(h + (int64_t)src_perm[pb + e] * KH + k4);
      *reinterpret_cast<f4*>(&hs[e][k4]) = v;
    }
    if (threadIdx.x < EP) {
      const int e = threadIdx.x;
      const int32_t id = (e < cnt) ? src_perm[pb + e] : -1;
      eids[e] = id;
      dsts[e] = (e < cnt) ? edge_dst[id] : 0;
      ns[e][0] = (e < cnt) ? nvec[3 * (int64_t)id] : 0.f;
      ns[e][1] = (e < cnt) ? nvec[3 * (int64_t)id + 1] : 0.f;
      ns[e][2] = (e < cnt) ? nvec[3 * (int64_t)id + 2] : 0.f;
    }
    const int nrt = (cnt + 15) / 16;
    f4 dacc[EP / 16];
#pragma unroll
    for (int i = 0; i < EP / 16; ++i) dacc[i] = f4{0.f, 0.f, 0.f, 0.f};

    for (int cb = 0; cb < NCOL; cb += 64) {
      __syncthreads();
      // dP tile (zero rows beyond cnt) and the S chunk for these 64 columns.
      for (int idx = threadIdx.x; idx < EP * 64; idx += 256) {
        const int e = idx >> 6, cl = idx & 63;
        float v = 0.f;
        if (e < cnt) {
          const int col = cb + cl;
          const int slot = col / C, c = col % C;
          const float* gp = G + (int64_t)dsts[e] * NCOMP * C + c;
          v = dp_value<C>(gp, slot, ns[e]) * scale;
        }
        dps[e][cl] = v;
      }
      for (int idx = threadIdx.x; idx < 64 * (KH / 4); idx += 256) {
        const int cl = idx / (KH / 4), k4 = (idx % (KH / 4)) * 4;
        const int col = cb + cl;
        const int slot = col / C, c = col % C;
        *reinterpret_cast<f4*>(&ss[cl][k4]) = ld4(Sm + (int64_t)slot * COLS + c * KH + k4);
      }
      __syncthreads();
      // dh: rows = edges (tile rt), cols = k in [16*wave, 16*wave+16), K = 64 columns.
      for (int rt = 0; rt < nrt; ++rt) {
#pragma unroll
        for (int t = 0; t < 4; ++t) {
          const f4 a4 = *reinterpret_cast<const f4*>(&dps[rt * 16 + r][16 * t + 4 * q]);
          f4 b4;
          b4.x = ss[16 * t + 4 * q + 0][16 * wave + r];
          b4.y = ss[16 * t + 4 * q + 1][16 * wave + r];
          b4.z = ss[16 * t + 4 * q + 2][16 * wave + r];
          b4.w = ss[16 * t + 4 * q + 3][16 * wave + r];
          dacc[rt] = mfma_k16(a4, b4, dacc[rt]);
        }
      }
      // dS: rows = columns cb+16*wave+.., output col tile ct covers k = 4*r + ct, K = edges.
      f4 sacc[4];
#pragma unroll
      for (int ct = 0; ct < 4; ++ct) sacc[ct] = f4{0.f, 0.f, 0.f, 0.f};
      for (int t = 0; t < nrt; ++t) {
        f4 a4;
        a4.x = dps[16 * t + 4 * q + 0][16 * wave + r];
        a4.y = dps[16 * t + 4 * q + 1][16 * wave + r];
        a4.z = dps[16 * t + 4 * q + 2][16 * wave + r];
        a4.w = dps[16 * t + 4 * q + 3][16 * wave + r];
        f4 hv[4];
#pragma unroll
        for (int j = 0; j < 4; ++j) hv[j] = *reinterpret_cast<const f4*>(&hs[16 * t + 4 * q + j][4 * r]);
#pragma unroll
        for (int ct = 0; ct < 4; ++ct) {
          const f4 b4 = {hv[0][ct], hv[1][ct], hv[2][ct], hv[3][ct]};
          sacc[ct] = mfma_k16(a4, b4, sacc[ct]);
        }
      }
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const int col = cb + 16 * wave + 4 * q + i;
        const int slot = col / C, c = col % C;
        float* o = dSm + (int64_t)slot * COLS + c * KH + 4 * r;
        f4 v = {sacc[0][i], sacc[1][i], sacc[2][i], sacc[3][i]};
        if (!first) v += ld4(o);
        st4(o, v);
      }
      if (threadIdx.x < 64) {
        const int cl = threadIdx.x;
        float s = 0.f;
        for (int e = 0; e < cnt; ++e) s += dps[e][cl];
        const int col = cb + cl;
        const int slot = col / C, c = col % C;
        float* o = dSm + (int64_t)slot * COLS + 64 * C + c;
        *o = first ? s : (*o + s);
      }
    }
    // dh rows of this pass
    for (int rt = 0; rt < nrt; ++rt) {
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const int e = rt * 16 + 4 * q + i;
        if (e < cnt) dh[(int64_t)eids[e] * KH + 16 * wave + r] = dacc[rt][i];
      }
    }
    first = false;
    pb += EP;
  } while (pb < end);
}

// ---------------------------------------------------------------- conv1 (species-pair form)
// conv1 operands depend on the source and receiver only through their species
// (A_i = atom_mlp(embedding(Z_i))), so the weight contraction over (a, b) is done once
// per species pair: M[pair][p][k'][c] = sum_{a,b} W[(p,c,a,b),k'] A_s[a] A_t[b]
// for the three live paths p0 (0,0->0), p3 (1,0->1), p5 (2,0->2); k' = 64 is the bias.
// Per edge Q_p[c] = sum_k' M[pair][p][k'][c] h'_e[k'];  m = [Q0, Q1 n, Q2 n n].
__global__ void conv1_pair_table_kernel(const float* __restrict__ L, const float* __restrict__ b,
                                        const float* __restrict__ atab, int n_species, int C,
                                        float* __restrict__ mf, float* __restrict__ mb) {
  const int64_t total = (int64_t)n_species * n_species * 3 * 65 * C;
  const int live[3] = {0, 3, 5};
  for (int64_t idx = blockIdx.x * (int64_t)blockDim.x + threadIdx.x; idx < total;
       idx += (int64_t)gridDim.x * blockDim.x) {
    const int c = (int)(idx % C);
    const int k = (int)((idx / C) % 65);
    const int p3 = (int)((idx / (C * 65)) % 3);
    const int pair = (int)(idx / (C * 65 * 3));
    const int s = pair / n_species, t = pair % n_species;
    const int p = live[p3];
    float acc = 0.f;
    for (int a = 0; a < 8; ++a) {
      const float as = atab[s * 8 + a];
      for (int bb = 0; bb < 8; ++bb) {
        const int64_t row = (int64_t)p * C * 64 + (int64_t)c * 64 + a * 8 + bb;
        const float w = (k < 64) ? L[row * KH + k] : b[row];
        acc += w * as * atab[t * 8 + bb];
      }
    }
    mf[idx] = acc;                                                   // [pair][p3][k][c]
    mb[(((int64_t)pair * 3 + p3) * C + c) * 65 + k] = acc;           // [pair][p3][c][k]
  }
}

template <int C>
__global__ __launch_bounds__(256) void conv1_forward_kernel(const float* __restrict__ h,
                                                            const float* __restrict__ nvec,
                                                            const int32_t* __restrict__ edge_pair,
                                                            const float* __restrict__ mf,
                                                            const int32_t* __restrict__ dst_ptr,
                                                            float* __restrict__ Q,
                                                            float* __restrict__ out,
                                                            int64_t n_nodes) {
  const int lane = threadIdx.x & 63;
  const int64_t n = (int64_t)blockIdx.x * 4 + (threadIdx.x >> 6);
  if (n >= n_nodes) return;
  const int c = lane;
  const bool act = lane < C;
  float o[NCOMP];
#pragma unroll
  for (int i = 0; i < NCOMP; ++i) o[i] = 0.f;
  const int beg = dst_ptr[n], end = dst_ptr[n + 1];
  for (int e = beg; e < end; ++e) {
    const float* M = mf + (int64_t)edge_pair[e] * 3 * 65 * C + (act ? c : 0);
    const float* he = h + (int64_t)e * KH;
    float q0 = M[64 * C], q1 = M[65 * C + 64 * C], q2 = M[2 * 65 * C + 64 * C];
#pragma unroll 8
    for (int k = 0; k < KH; ++k) {
      const float hk = he[k];
      q0 += M[k * C] * hk;
      q1 += M[65 * C + k * C] * hk;
      q2 += M[2 * 65 * C + k * C] * hk;
    }
    const float nn[3] = {nvec[3 * (int64_t)e], nvec[3 * (int64_t)e + 1], nvec[3 * (int64_t)e + 2]};
    if (act) {
      float* qr = Q + (int64_t)e * 3 * C + c;
      qr[0] = q0; qr[C] = q1; qr[2 * C] = q2;
      o[0] += q0;
#pragma unroll
      for (int i = 0; i < 3; ++i) {
        o[1 + i] += q1 * nn[i];
#pragma unroll
        for (int j = 0; j < 3; ++j) o[4 + 3 * i + j] += q2 * nn[i] * nn[j];
      }
    }
  }
  if (act) {
    const float scale = 1.f / (float)max(end - beg, 1);
    float* orow = out + n * NCOMP * C + c;
#pragma unroll
    for (int i = 0; i < NCOMP; ++i) orow[i * C] = o[i] * scale;
  }
}

template <int C>
__global__ __launch_bounds__(256) void conv1_backward_kernel(const float* __restrict__ G,
                                                             const float* __restrict__ nvec,
                                                             const int32_t* __restrict__ edge_pair,
                                                             const float* __restrict__ mb,
                                                             const float* __restrict__ Q,
                                                             const int32_t* __restrict__ dst_ptr,
                                                             float* __restrict__ dh,
                                                             float* __restrict__ dn,
                                                             int64_t n_nodes) {
  __shared__ float dq[4][3][C];
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int64_t n = (int64_t)blockIdx.x * 4 + wave;
  if (n >= n_nodes) return;   // whole wave exits together; no block-level barrier below
  const int c = lane;
  const bool act = lane < C;
  const int beg = dst_ptr[n], end = dst_ptr[n + 1];
  const float scale = 1.f / (float)max(end - beg, 1);
  float g[NCOMP];
#pragma unroll
  for (int i = 0; i < NCOMP; ++i) g[i] = act ? G[(n * NCOMP + i) * C + c] * scale : 0.f;
  for (int e = beg; e < end; ++e) {
    const float nn[3] = {nvec[3 * (int64_t)e], nvec[3 * (int64_t)e + 1], nvec[3 * (int64_t)e + 2]};
    float t[3] = {0.f, 0.f, 0.f};
    if (act) {
      const float* qr = Q + (int64_t)e * 3 * C + c;
      const float q1 = qr[C], q2 = qr[2 * C];
      float d1 = 0.f, d2 = 0.f;
#pragma unroll
      for (int i = 0; i < 3; ++i) {
        d1 += g[1 + i] * nn[i];
#pragma unroll
        for (int j = 0; j < 3; ++j) d2 += g[4 + 3 * i + j] * nn[i] * nn[j];
      }
      dq[wave][0][c] = g[0];
      dq[wave][1][c] = d1;
      dq[wave][2][c] = d2;
#pragma unroll
      for (int k = 0; k < 3; ++k) {
        float row = 0.f, colv = 0.f;
#pragma unroll
        for (int j = 0; j < 3; ++j) {
          row += g[4 + 3 * k + j] * nn[j];
          colv += g[4 + 3 * j + k] * nn[j];
        }
        t[k] = g[1 + k] * q1 + q2 * (row + colv);
      }
    }
    const float t0 = wave_sum(t[0]), t1 = wave_sum(t[1]), t2 = wave_sum(t[2]);
    if (lane == 0) {
      dn[3 * (int64_t)e] = t0;
      dn[3 * (int64_t)e + 1] = t1;
      dn[3 * (int64_t)e + 2] = t2;
    }
    __builtin_amdgcn_wave_barrier();
    __builtin_amdgcn_fence(__ATOMIC_SEQ_CST, "wavefront");
    // dh[e][k] = sum_p sum_c dQ_p[c] M[pair][p][c][k], lane = k
    const float* M = mb + (int64_t)edge_pair[e] * 3 * C * 65 + lane;
    float acc = 0.f;
    for (int p = 0; p < 3; ++p)
#pragma unroll 8
      for (int cc = 0; cc < C; ++cc) acc += dq[wave][p][cc] * M[(p * C + cc) * 65];
    dh[(int64_t)e * KH + lane] = acc;
    __builtin_amdgcn_wave_barrier();
    __builtin_amdgcn_fence(__ATOMIC_SEQ_CST, "wavefront");
  }
}

// ---------------------------------------------------------------- host launchers
template <int C>
int conv_forward_impl(int64_t N, int64_t E, const int32_t* dst_ptr, const int32_t* src_ptr,
                      const int32_t* src_perm, const float* x, const float* h, const float* nvec,
                      const float* bk1, float scale, float* S, float* P, float* out,
                      hipStream_t st) {
  if (N == 0) return 0;
  for (int p = 0; p < 6; ++p) {
    const int64_t rows = N * kNumI[kPathL1H[p]];
    dim3 grid((unsigned)((rows + 63) / 64), (unsigned)((65 * C + 255) / 256));
    LaunchTimer tm("node_expand", st);
    node_expand_kernel<C><<<grid, 256, 0, st>>>(x, bk1, S, N, p);
  }
  if (check_launch("sparse node_expand")) return 2;
  {
    LaunchTimer tm("edge_message", st);
    edge_message_kernel<C><<<(unsigned)N, 256, 0, st>>>(h, S, src_ptr, src_perm, P);
  }
  if (check_launch("sparse edge_message")) return 2;
  {
    LaunchTimer tm("receiver_sum", st);
    receiver_sum_kernel<C><<<(unsigned)((N + 3) / 4), 256, 0, st>>>(P, nvec, dst_ptr, scale, out, N);
  }
  return check_launch("sparse receiver_sum") ? 2 : 0;
}

template <int C>
int conv_backward_impl(int64_t N, int64_t E, const int32_t* dst_ptr, const int32_t* src_ptr,
                       const int32_t* src_perm, const int32_t* edge_dst, const float* G,
                       const float* h, const float* nvec, const float* bk6, const float* S,
                       const float* P, float scale, float* dS, float* dx, float* dh, float* dn,
                       hipStream_t st) {
  if (N == 0) return 0;
  {
    LaunchTimer tm("direction_grad", st);
    direction_grad_kernel<C><<<(unsigned)((N + 3) / 4), 256, 0, st>>>(G, P, nvec, dst_ptr, scale, dn, N);
  }
  if (check_launch("sparse direction_grad")) return 2;
  {
    LaunchTimer tm("edge_message_grad", st);
    edge_message_grad_kernel<C><<<(unsigned)N, 256, 0, st>>>(G, nvec, h, S, src_ptr, src_perm,
                                                             edge_dst, scale, dh, dS);
  }
  if (check_launch("sparse edge_message_grad")) return 2;
  for (int g = 0; g < 3; ++g) {
    const int64_t rows = N * kNumI[g];
    LaunchTimer tm("node_expand_grad", st);
    node_expand_grad_kernel<C><<<(unsigned)((rows + 63) / 64), 256, 0, st>>>(dS, bk6, dx, N, g);
  }
  return check_launch("sparse node_expand_grad") ? 2 : 0;
}

}  // namespace sparse
}  // namespace fsc

// ===================================================================== C ABI
using namespace fsc;
using namespace fsc::sparse;

extern "C" {

int fsc_sparse_conv_workspace(int64_t n_nodes, int64_t n_edges, int32_t channels,
                              int64_t* s_floats, int64_t* p_floats) {
  FSC_CHECK_ARG(n_nodes >= 0 && n_edges >= 0, "fsc_sparse_conv_workspace: negative size");
  FSC_CHECK_ARG(channels == 32 || channels == 64, "fsc_sparse_conv_workspace: channels must be 32 or 64");
  FSC_CHECK_ARG(s_floats && p_floats, "fsc_sparse_conv_workspace: null output");
  *s_floats = n_nodes * s_node_stride(channels);
  *p_floats = n_edges * (int64_t)NSLOT * channels;
  return 0;
}

int fsc_sparse_conv_prepare_weights(const float* w_last, const float* b_last, int32_t channels,
                                    float* bk1, float* bk6, hipStream_t stream) {
  FSC_CHECK_ARG(channels == 32 || channels == 64, "fsc_sparse_conv_prepare_weights: channels must be 32 or 64");
  FSC_CHECK_ARG(w_last && b_last && bk1 && bk6, "fsc_sparse_conv_prepare_weights: null pointer");
  prep_weights_kernel<<<512, 256, 0, stream>>>(w_last, b_last, bk1, bk6, channels);
  return check_launch("sparse prepare_weights") ? 2 : 0;
}

int fsc_sparse_conv_forward(int64_t n_nodes, int64_t n_edges, int32_t channels,
                            const int32_t* dst_ptr, const int32_t* src_ptr, const int32_t* src_perm,
                            const float* x, const float* h, const float* n, const float* bk1,
                            float inv_norm, float* s_ws, float* p_ws, float* out,
                            hipStream_t stream) {
  FSC_CHECK_ARG(n_nodes >= 0 && n_edges >= 0, "fsc_sparse_conv_forward: negative size");
  FSC_CHECK_ARG(n_nodes < (1LL << 31) && n_edges < (1LL << 31), "fsc_sparse_conv_forward: size exceeds int32 indexing");
  FSC_CHECK_ARG(dst_ptr && src_ptr && x && bk1 && s_ws && out, "fsc_sparse_conv_forward: null pointer");
  FSC_CHECK_ARG(n_edges == 0 || (src_perm && h && n && p_ws), "fsc_sparse_conv_forward: null edge pointer");
  if (channels == 64)
    return conv_forward_impl<64>(n_nodes, n_edges, dst_ptr, src_ptr, src_perm, x, h, n, bk1, inv_norm,
                                 s_ws, p_ws, out, stream);
  if (channels == 32)
    return conv_forward_impl<32>(n_nodes, n_edges, dst_ptr, src_ptr, src_perm, x, h, n, bk1, inv_norm,
                                 s_ws, p_ws, out, stream);
  set_error("fsc_sparse_conv_forward: channels must be 32 or 64");
  return 1;
}

int fsc_sparse_conv_backward(int64_t n_nodes, int64_t n_edges, int32_t channels,
                             const int32_t* dst_ptr, const int32_t* src_ptr, const int32_t* src_perm,
                             const int32_t* edge_dst, const float* grad_out, const float* h,
                             const float* n, const float* bk6, const float* s_ws, const float* p_ws,
                             float inv_norm, float* ds_ws, float* grad_x, float* grad_h,
                             float* grad_n, hipStream_t stream) {
  FSC_CHECK_ARG(n_nodes >= 0 && n_edges >= 0, "fsc_sparse_conv_backward: negative size");
  FSC_CHECK_ARG(n_nodes < (1LL << 31) && n_edges < (1LL << 31), "fsc_sparse_conv_backward: size exceeds int32 indexing");
  FSC_CHECK_ARG(dst_ptr && src_ptr && grad_out && bk6 && s_ws && ds_ws && grad_x,
                "fsc_sparse_conv_backward: null pointer");
  FSC_CHECK_ARG(n_edges == 0 || (src_perm && edge_dst && h && n && p_ws && grad_h && grad_n),
                "fsc_sparse_conv_backward: null edge pointer");
  if (channels == 64)
    return conv_backward_impl<64>(n_nodes, n_edges, dst_ptr, src_ptr, src_perm, edge_dst, grad_out, h, n,
                                  bk6, s_ws, p_ws, inv_norm, ds_ws, grad_x, grad_h, grad_n, stream);
  if (channels == 32)
    return conv_backward_impl<32>(n_nodes, n_edges, dst_ptr, src_ptr, src_perm, edge_dst, grad_out, h, n,
                                  bk6, s_ws, p_ws, inv_norm, ds_ws, grad_x, grad_h, grad_n, stream);
  set_error("fsc_sparse_conv_backward: channels must be 32 or 64");
  return 1;
}

int fsc_sparse_conv1_pair_table(const float* w_last, const float* b_last, const float* atom_table,
                                int32_t n_species, int32_t channels, float* mf, float* mb,
                                hipStream_t stream) {
  FSC_CHECK_ARG(channels == 32 || channels == 64, "fsc_sparse_conv1_pair_table: channels must be 32 or 64");
  FSC_CHECK_ARG(n_species >= 1 && n_species <= 128, "fsc_sparse_conv1_pair_table: n_species out of range");
  FSC_CHECK_ARG(w_last && b_last && atom_table && mf && mb, "fsc_sparse_conv1_pair_table: null pointer");
  conv1_pair_table_kernel<<<256, 256, 0, stream>>>(w_last, b_last, atom_table, n_species, channels, mf, mb);
  return check_launch("sparse conv1_pair_table") ? 2 : 0;
}

int fsc_sparse_conv1_forward(int64_t n_nodes, int64_t n_edges, int32_t channels, const int32_t* dst_ptr,
                             const int32_t* edge_pair, const float* h, const float* n, const float* mf,
                             float* q_ws, float* out, hipStream_t stream) {
  FSC_CHECK_ARG(n_nodes >= 0 && n_edges >= 0 && n_nodes < (1LL << 31) && n_edges < (1LL << 31),
                "fsc_sparse_conv1_forward: bad size");
  FSC_CHECK_ARG(dst_ptr && mf && out, "fsc_sparse_conv1_forward: null pointer");
  FSC_CHECK_ARG(n_edges == 0 || (edge_pair && h && n && q_ws), "fsc_sparse_conv1_forward: null edge pointer");
  if (n_nodes == 0) return 0;
  const unsigned grid = (unsigned)((n_nodes + 3) / 4);
  LaunchTimer tm("conv1_forward", stream);
  if (channels == 64)
    conv1_forward_kernel<64><<<grid, 256, 0, stream>>>(h, n, edge_pair, mf, dst_ptr, q_ws, out, n_nodes);
  else if (channels == 32)
    conv1_forward_kernel<32><<<grid, 256, 0, stream>>>(h, n, edge_pair, mf, dst_ptr, q_ws, out, n_nodes);
  else {
    set_error("fsc_sparse_conv1_forward: channels must be 32 or 64");
    return 1;
  }
  return check_launch("sparse conv1_forward") ? 2 : 0;
}

int fsc_sparse_conv1_backward(int64_t n_nodes, int64_t n_edges, int32_t channels, const int32_t* dst_ptr,
                              const int32_t* edge_pair, const float* grad_out, const float* n,
                              const float* mb, const float* q_ws, float* grad_h, float* grad_n,
                              hipStream_t stream) {
  FSC_CHECK_ARG(n_nodes >= 0 && n_edges >= 0 && n_nodes < (1LL << 31) && n_edges < (1LL << 31),
                "fsc_sparse_conv1_backward: bad size");
  FSC_CHECK_ARG(dst_ptr && grad_out && mb, "fsc_sparse_conv1_backward: null pointer");
  FSC_CHECK_ARG(n_edges == 0 || (edge_pair && n && q_ws && grad_h && grad_n),
                "fsc_sparse_conv1_backward: null edge pointer");
  if (n_nodes == 0) return 0;
  const unsigned grid = (unsigned)((n_nodes + 3) / 4);
  LaunchTimer tm("conv1_backward", stream);
  if (channels == 64)
    conv1_backward_kernel<64><<<grid, 256, 0, stream>>>(grad_out, n, edge_pair, mb, q_ws, dst_ptr, grad_h,
                                                        grad_n, n_nodes);
  else if (channels == 32)
    conv1_backward_kernel<32><<<grid, 256, 0, stream>>>(grad_out, n, edge_pair, mb, q_ws, dst_ptr, grad_h,
                                                        grad_n, n_nodes);
  else {
    set_error("fsc_sparse_conv1_backward: channels must be 32 or 64");
    return 1;
  }
  return check_launch("sparse conv1_backward") ? 2 : 0;
}

}  // extern "C"
