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
// P[E][18*C] at the receiver-sorted edge id: a row holds first the five slots the backward reads (1, 2, 6,
// 7, 8: positions 0..4 of pos_of_slot) as [C/8][5][8], then the other thirteen as [C/8][13][8] (channel
// chunks of 8, slot-major inside a chunk), so the backward's reads of an edge are one contiguous 20*C-byte
// run, a chunk at a time (p_col); h[E][64]; n[E][3] (unit vectors).

#include <algorithm>

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

// Order of the slots inside a channel chunk of P: the five slots the backward reads (P1, P2 and P4, slots
// 1, 2, 6, 7, 8) occupy the first 160 bytes of the chunk's 576, so it fetches two 128-byte lines per edge
// and chunk instead of three.
__host__ __device__ constexpr int slot_at_pos(int pos) {
  return pos < 2 ? pos + 1 : pos < 5 ? pos + 4 : pos == 5 ? 0 : pos < 9 ? pos - 3 : pos;
}
__host__ __device__ constexpr int pos_of_slot(int s) {
  return s == 0 ? 5 : s < 3 ? s - 1 : s < 6 ? s + 3 : s < 9 ? s - 4 : s;
}

// Column of (slot position pos, channel c) in an edge's row of P, and back.
template <int C>
__host__ __device__ constexpr int p_col(int pos, int c) {
  return pos < 5 ? (c >> 3) * 40 + pos * 8 + (c & 7) : 5 * C + (c >> 3) * 104 + (pos - 5) * 8 + (c & 7);
}
template <int C>
__host__ __device__ inline void p_col_inverse(int col, int& pos, int& c) {
  if (col < 5 * C) {
    const int rem = col % 40;
    pos = rem >> 3;
    c = 8 * (col / 40) + (rem & 7);
  } else {
    const int cc = col - 5 * C, rem = cc % 104;
    pos = 5 + (rem >> 3);
    c = 8 * (cc / 104) + (rem & 7);
  }
}

// ---------------------------------------------------------------- weight preparation
// bk1[part][p][col][a] (col < 64C: col = c*64+k -> L[(p,c,a),k]; col >= 64C: b[(p,c,a)]) and
// bk6[part][p][a][col] (transpose of bk1[p]): the values times the power of two sw (max |L|, |b|
// times sw below 2^14) split into two fp16 parts (h, l; split2h), for the split-fp16 products of
// node_expand and node_expand_grad.  Each buffer is the two parts (6*65*C*C fp16 each, as many floats
// together) followed by a tail of SW_TAIL floats: [0] = 1/sw, [256..511] partial maxima (bk1 only), then
// the same scaled values rounded to bf16 (one plane, 6*65*C*C bf16) for the bf16 channel-mix variant.
constexpr int SW_TAIL = 512;
constexpr int SWMAX_BLOCKS = 256;
__host__ __device__ inline int64_t sparse_weight_floats(int C) { return 6LL * 65 * C * C + SW_TAIL; }
__host__ __device__ inline int64_t sparse_weight_floats_all(int C) { return sparse_weight_floats(C) + 3LL * 65 * C * C; }

// wmax[block] = max |L|, |b| over the grid-stride share of the block (grid SWMAX_BLOCKS x 256).
__global__ __launch_bounds__(256) void weight_absmax_kernel(const float* __restrict__ L, int64_t nl,
                                                            const float* __restrict__ b, int64_t nb,
                                                            float* __restrict__ wmax) {
  __shared__ float red[4];
  float m = 0.f;
  for (int64_t i = blockIdx.x * 256 + threadIdx.x; i < nl + nb; i += (int64_t)gridDim.x * 256)
    m = fmaxf(m, fabsf(i < nl ? L[i] : b[i - nl]));
  for (int off = 32; off > 0; off >>= 1) m = fmaxf(m, __shfl_xor(m, off, 64));
  if ((threadIdx.x & 63) == 0) red[threadIdx.x >> 6] = m;
  __syncthreads();
  if (threadIdx.x == 0) wmax[blockIdx.x] = fmaxf(fmaxf(red[0], red[1]), fmaxf(red[2], red[3]));
}

// One block of 256 threads per (path p, output channel c): the C x 65 tile of (a, column) values passes
// through LDS, so that both layouts are written in contiguous runs (bk6 rows along the column, bk1 rows
// along a).  Every block reduces the partial maxima itself, so all use the same sw.
__global__ __launch_bounds__(256) void prep_weights_kernel(const float* __restrict__ L, const float* __restrict__ b,
                                                           float* __restrict__ bk1f, float* __restrict__ bk6f, int C) {
  const int64_t cols = 65LL * C;
  const int64_t total = 6LL * cols * C;
  __shared__ float red[4];
  __shared__ float tile[128][65];   // [a][kk], C <= 128
  float mx = bk1f[total + 256 + threadIdx.x];
  for (int off = 32; off > 0; off >>= 1) mx = fmaxf(mx, __shfl_xor(mx, off, 64));
  if ((threadIdx.x & 63) == 0) red[threadIdx.x >> 6] = mx;
  __syncthreads();
  const float sw = pow2_scale(fmaxf(fmaxf(red[0], red[1]), fmaxf(red[2], red[3])));
  if (blockIdx.x == 0 && threadIdx.x == 0) {
    bk1f[total] = 1.f / sw;
    bk6f[total] = 1.f / sw;
  }
  _Float16* bk1 = reinterpret_cast<_Float16*>(bk1f);
  _Float16* bk6 = reinterpret_cast<_Float16*>(bk6f);
  __bf16* bk1b = reinterpret_cast<__bf16*>(bk1f + total + SW_TAIL);
  __bf16* bk6b = reinterpret_cast<__bf16*>(bk6f + total + SW_TAIL);
  const int p = blockIdx.x / C, c = blockIdx.x % C;
  const int64_t row0 = (int64_t)p * C * C + (int64_t)c * C;    // row of (p, c, a = 0)
  // values times sw, kk fastest: rows of L read 256 contiguous bytes at a time
  for (int i = threadIdx.x; i < C * 65; i += 256) {
    const int a = i / 65, kk = i - a * 65;
    tile[a][kk] = (kk < 64 ? L[(row0 + a) * KH + kk] : b[row0 + a]) * sw;
  }
  __syncthreads();
  // bk6[p][a][col], col = c*64 + kk (kk < 64) or 64C + c (bias)
  for (int i = threadIdx.x; i < C * 65; i += 256) {
    const int a = i / 65, kk = i - a * 65;
    const int64_t col = kk < 64 ? (int64_t)c * 64 + kk : 64LL * C + c;
    const int64_t o = ((int64_t)p * C + a) * cols + col;
    const float vs = tile[a][kk];
    const _Float16 hb = (_Float16)vs;
    bk6[o] = hb;
    bk6[total + o] = (_Float16)(vs - (float)hb);
    bk6b[o] = (__bf16)vs;
  }
  // bk1[p][col][a], a fastest
  for (int i = threadIdx.x; i < C * 65; i += 256) {
    const int kk = i / C, a = i - kk * C;
    const int64_t col = kk < 64 ? (int64_t)c * 64 + kk : 64LL * C + c;
    const int64_t idx = ((int64_t)p * cols + col) * C + a;
    const float vs = tile[a][kk];
    const _Float16 hb = (_Float16)vs;
    bk1[idx] = hb;
    bk1[total + idx] = (_Float16)(vs - (float)hb);
    bk1b[idx] = (__bf16)vs;
  }
}

// ---------------------------------------------------------------- K1: node expansion
// S[m][sbase(p)+I][col] = sum_a x[m][comp0(p)+I][a] * bk1[p][col][a].  A block takes 128 rows
// (m, I) of one path (4 waves x 32 rows; blocks numbered path by path, `off` = first block of
// each path) and a group of 80-column tiles.  Products are split-fp16 (mfma_x3, K = C in steps of
// 32): each row of x is scaled by a power of two from its own max |x| and split once into registers;
// each column tile of bk1 (80 x C, two fp16 parts) is staged in LDS, the next one loaded while the
// current one is multiplied and written to the other LDS buffer before the current results (both
// scales undone) are stored.
// Transposed product: bk1 rows are the MFMA A operand and x rows the B operand, and tile j's
// A row i is column 16*j + i, so lane (r, q) ends with columns 16j+4q..16j+4q+3 of row r: the
// four lanes of a row store 64 contiguous bytes per instruction.  Stores go through a buffer
// descriptor spanning the block's nodes; rows past the end are sent out of range and dropped.
// BF16: the bf16 channel-mix variant, one bf16 MFMA per product (x rows and the weights rounded to bf16,
// fp32 accumulation); the weights come from the bf16 plane of bk1.
struct PathTiles {
  int off[7];
};
constexpr int NE_ROWS = 128;   // rows per node_expand block
constexpr int NE_TPB = 13;     // 80-column tiles per node_expand block

template <int C, bool BF16>
__global__ __launch_bounds__(256, 2) void node_expand_kernel(const float* __restrict__ x,
                                                             const _Float16* __restrict__ bk1,
                                                             const float* __restrict__ winv,
                                                             float* __restrict__ S, int64_t n_nodes,
                                                             PathTiles tiles) {
  constexpr int COLS = 65 * C, NT = 5, WCOLS = 16 * NT, KS = C / 32;
  constexpr int NTC = COLS / WCOLS;                  // column tiles (52 or 26)
  constexpr int NCG = (NTC + NE_TPB - 1) / NE_TPB;   // column groups
  constexpr int RT = NE_ROWS / 64;                   // 16-row tiles per wave
  constexpr int RW = C + 8;                          // fp16 per LDS row (padding against bank conflicts)
  constexpr int NPART = BF16 ? 1 : 2;                // weight parts staged (fp16 h, l or one bf16 plane)
  constexpr int NPC = NPART * WCOLS * (C / 8);       // 16-byte pieces of a tile
  constexpr int NST = (NPC + 255) / 256;
  __shared__ __align__(16) _Float16 sb[2][2][WCOLS][RW];
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int r = lane & 15, q = lane >> 4;
  const int bt = blockIdx.x / NCG, cg = blockIdx.x % NCG;
  int p = 0;
  while (p < 5 && bt >= tiles.off[p + 1]) ++p;
  const int L1 = kPathL1[p];
  const int nI = (L1 == 0) ? 1 : (L1 == 1 ? 3 : 9);
  const int comp0 = (L1 == 0) ? 0 : (L1 == 1 ? 1 : 4);
  const int sbase = kSlotBase[p];
  const int64_t rows = n_nodes * nI;
  const int64_t brow0 = (int64_t)(bt - tiles.off[p]) * NE_ROWS;
  const int64_t row0 = brow0 + wave * (16 * RT);
  const int64_t part = 6LL * COLS * C;               // fp16 per weight part
  const _Float16* bp = bk1 + (int64_t)p * COLS * C;
  const int ct0 = cg * NE_TPB, ct1 = min(NTC, ct0 + NE_TPB);
  // store window: the nodes of the block's rows (at most NE_ROWS nodes, well below 4 GiB)
  const int64_t mfirst = (uint32_t)brow0 / (uint32_t)nI;
  const int64_t mlast = min(n_nodes - 1, (int64_t)((uint32_t)(brow0 + NE_ROWS - 1) / (uint32_t)nI));
  // BF16: S is stored in bf16 (its consumers round it to bf16 for their products anyway)
  constexpr int SBYTES = BF16 ? 2 : 4;
  const __amdgpu_buffer_rsrc_t out = buffer_rsrc_bytes(
      reinterpret_cast<char*>(S) + mfirst * s_node_stride(C) * SBYTES,
      (uint32_t)((mlast - mfirst + 1) * s_node_stride(C) * SBYTES));
  h8 xh[RT][KS], xl[RT][KS];
  bf8 xb[RT][KS];
  float oscale[RT];    // 1 / (sw * row scale)
  uint32_t ooff[RT];   // byte offset of the lane's first column in the store window
#pragma unroll
  for (int rt = 0; rt < RT; ++rt) {
    const int64_t row = row0 + 16 * rt + r;
    const bool ok = row < rows;
    const int64_t m = ok ? (int64_t)((uint32_t)row / (uint32_t)nI) : mfirst;
    const int I = ok ? (int)(row - m * nI) : 0;
    const float* xr = x + (m * NCOMP + comp0 + I) * C + 8 * q;
    float v[KS][8];
    float vmax = 0.f;
#pragma unroll
    for (int ks = 0; ks < KS; ++ks) {
      const f4 x0 = ld4(xr + 32 * ks), x1 = ld4(xr + 32 * ks + 4);
      v[ks][0] = x0.x; v[ks][1] = x0.y; v[ks][2] = x0.z; v[ks][3] = x0.w;
      v[ks][4] = x1.x; v[ks][5] = x1.y; v[ks][6] = x1.z; v[ks][7] = x1.w;
#pragma unroll
      for (int j = 0; j < 8; ++j) vmax = fmaxf(vmax, fabsf(v[ks][j]));
    }
    // the C values of a row are spread over lanes r, r + 16, r + 32, r + 48
    vmax = fmaxf(vmax, __shfl_xor(vmax, 16, 64));
    vmax = fmaxf(vmax, __shfl_xor(vmax, 32, 64));
    const float sr = pow2_scale(vmax);
    if constexpr (BF16) {
#pragma unroll
      for (int ks = 0; ks < KS; ++ks)
#pragma unroll
        for (int j = 0; j < 8; ++j) xb[rt][ks][j] = (__bf16)(v[ks][j] * sr);
    } else {
#pragma unroll
      for (int ks = 0; ks < KS; ++ks) split2h(v[ks], sr, xh[rt][ks], xl[rt][ks]);
    }
    oscale[rt] = winv[0] / sr;   // sr is a power of two: exact
    ooff[rt] = ok ? (uint32_t)(((m - mfirst) * s_node_stride(C) + (int64_t)(sbase + I) * COLS + 4 * q) * SBYTES)
                  : kDropOffset;
  }
  f4 stg[NST];
  auto gload = [&](int ct) {
#pragma unroll
    for (int i = 0; i < NST; ++i) {
      const int idx = threadIdx.x + 256 * i;   // (part, column, 8-entry piece of a)
      if (idx < NPC) {
        const int pt = idx / (WCOLS * (C / 8)), rem = idx - pt * (WCOLS * (C / 8));
        const int col = rem / (C / 8), a8 = rem % (C / 8);
        stg[i] = *reinterpret_cast<const f4*>(bp + pt * part + (int64_t)(ct * WCOLS + col) * C + 8 * a8);
      }
    }
  };
  auto sstore = [&](int buf) {
#pragma unroll
    for (int i = 0; i < NST; ++i) {
      const int idx = threadIdx.x + 256 * i;
      if (idx < NPC) {
        const int pt = idx / (WCOLS * (C / 8)), rem = idx - pt * (WCOLS * (C / 8));
        const int col = rem / (C / 8), a8 = rem % (C / 8);
        *reinterpret_cast<f4*>(&sb[buf][pt][col][8 * a8]) = stg[i];
      }
    }
  };
  gload(ct0);
  sstore(0);
  __syncthreads();
  for (int ct = ct0; ct < ct1; ++ct) {
    const int buf = (ct - ct0) & 1;
    if (ct + 1 < ct1) gload(ct + 1);
    f4 acc[RT][NT];
#pragma unroll
    for (int rt = 0; rt < RT; ++rt)
#pragma unroll
      for (int j = 0; j < NT; ++j) acc[rt][j] = f4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int j = 0; j < NT; ++j)
#pragma unroll
      for (int ks = 0; ks < KS; ++ks) {
        if constexpr (BF16) {
          const bf8 wb = *reinterpret_cast<const bf8*>(&sb[buf][0][16 * j + r][32 * ks + 8 * q]);
#pragma unroll
          for (int rt = 0; rt < RT; ++rt) acc[rt][j] = mfma_bf16(wb, xb[rt][ks], acc[rt][j]);
        } else {
          const h8 wh = *reinterpret_cast<const h8*>(&sb[buf][0][16 * j + r][32 * ks + 8 * q]);
          const h8 wl = *reinterpret_cast<const h8*>(&sb[buf][1][16 * j + r][32 * ks + 8 * q]);
#pragma unroll
          for (int rt = 0; rt < RT; ++rt) acc[rt][j] = mfma_x3(wh, wl, xh[rt][ks], xl[rt][ks], acc[rt][j]);
        }
      }
    // stage the next tile first: the waits for its loads then do not cover this tile's stores
    __builtin_amdgcn_sched_barrier(0);
    if (ct + 1 < ct1) sstore(buf ^ 1);
    __builtin_amdgcn_sched_barrier(0);
#pragma unroll
    for (int rt = 0; rt < RT; ++rt)
#pragma unroll
      for (int j = 0; j < NT; ++j) {
        if constexpr (BF16) buffer_st4_bf16(out, ooff[rt] + (uint32_t)(ct * WCOLS + 16 * j) * 2, acc[rt][j] * oscale[rt]);
        else buffer_st4(out, ooff[rt] + (uint32_t)(ct * WCOLS + 16 * j) * 4, acc[rt][j] * oscale[rt]);
      }
    __syncthreads();
  }
}

// ---------------------------------------------------------------- K6: node expansion grad
// dxp[kh][slot][m][a] = sum_{col in K part kh} dS[m][slot][col] * bk6[p][a][col] for every slot
// row (m, I) of path p, then dx[m][comp][a] = sum over the K parts and the slots of comp
// (node_expand_grad_combine).  A block's work unit is (path, 256-row tile, K part), one 64-row
// strip per wave: all units are equally long, which keeps the blocks balanced although paths
// 0-2 share component 0.  K is split in ks parts (neg_ksplit: 2, more while the grid of
// (path, tile) units is small, so that a few hundred atoms do not leave a handful of blocks each
// walking 65 K chunks in sequence).  Products are split-fp16 (mfma_x3, fp32 accuracy at 5x the fp32 MFMA
// rate): the weights come split (bk6 parts h, l, scaled by sw), the dS rows are scaled by their node's
// power of two (dscale, from edge_message_grad) and split in registers.  The four
// waves share the path's weights: each 32-column chunk (C x 32 x 3 parts) is loaded once per block
// into LDS (double-buffered) while the waves stream their own dS rows a chunk ahead.
// Transposed product: bk6 rows (a) are the A operand, dS rows the B operand; tile at's A row
// i is a = (C/4)*(i/4) + 4*at + i%4, so lane (r, q) ends with C/4 consecutive a of one row; lane
// group q holds chunk columns 8q..8q+7 of both operands.
constexpr int NEG_ROWS = 256;   // slot rows per block
constexpr int NEG_KSPLIT_MAX = 16;

// (path, row tile) units of node_expand_grad, and its K parts: a function of N alone, since the
// workspace holds one partial input gradient per part
inline int neg_tiles(int64_t N) {
  int64_t t = 0;
  for (int p = 0; p < 6; ++p) t += (N * kNumI[kPathL1H[p]] + NEG_ROWS - 1) / NEG_ROWS;
  return (int)std::min<int64_t>(t, 1 << 30);
}
inline int neg_ksplit(int64_t N) {
  const int64_t tiles = neg_tiles(N);
  int ks = 2;
  while (ks < NEG_KSPLIT_MAX && tiles * ks < 512) ks *= 2;
  return ks;
}

// Blocks per source node of the edge message and its gradient: one per node on large graphs; on small ones
// (one block per node leaves most of the 256 CUs idle or waiting on the highest-degree node) the message's
// column blocks and the gradient's channel chunks are split over 2 or 4 blocks.
inline int msg_parts(int64_t N) { return N <= 256 ? 4 : N < 2048 ? 2 : 1; }

// Start (floats from dS) and size of the partial dh, dn and dS maxima of a split message gradient, after the
// backward's tail and per-node scales, 256-byte aligned.
inline int64_t msg_parts_offset(int64_t N, int C) {
  return (N * s_node_stride(C) + (int64_t)neg_ksplit(N) * NSLOT * N * C + N + 63) / 64 * 64;
}
inline int64_t msg_parts_floats(int64_t N, int64_t E) {
  const int np = msg_parts(N);
  return np > 1 ? (int64_t)np * (E * (KH + 3) + N) : 0;
}

template <int C, bool BF16>
__global__ __launch_bounds__(256, 2) void node_expand_grad_kernel(const float* __restrict__ dS,
                                                                  const float* __restrict__ dscale,
                                                                  const _Float16* __restrict__ bk6,
                                                                  const float* __restrict__ winv,
                                                                  float* __restrict__ dxp,
                                                                  int64_t n_nodes, PathTiles tiles, int ks) {
  constexpr int COLS = 65 * C;
  constexpr int NA = C / 16;        // output a tiles
  constexpr int QW = C / 4;         // consecutive a per lane in the output
  constexpr int TPP = COLS / 32;    // K chunks per path
  constexpr int RS = 40;            // fp16 per LDS row: 32 + 8 padding
  constexpr int NPART = BF16 ? 1 : 2;         // fp16 h, l parts or one bf16 plane
  constexpr int NPC = NPART * C * 4;          // 16-byte pieces of a chunk (parts x C rows x 4)
  constexpr int NST = (NPC + 255) / 256;      // per thread
  __shared__ __align__(16) _Float16 wsh[2][2][C][RS];
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int r = lane & 15, q = lane >> 4;
  const int kh = (int)(blockIdx.x % (unsigned)ks), bt = (int)(blockIdx.x / (unsigned)ks);
  int p = 0;
  while (p < 5 && bt >= tiles.off[p + 1]) ++p;
  const int L1 = kPathL1[p];
  const int nI = (L1 == 0) ? 1 : (L1 == 1 ? 3 : 9);
  const int sbase = kSlotBase[p];
  const int64_t rows = n_nodes * nI;
  const int64_t row0 = (int64_t)(bt - tiles.off[p]) * NEG_ROWS + wave * 64;

  bool ok[4];
  int64_t rbase[4], mrow[4];
  int irow[4];
  float rsc[4];
#pragma unroll
  for (int rt = 0; rt < 4; ++rt) {
    int64_t row = row0 + 16 * rt + r;
    ok[rt] = row < rows;
    if (!ok[rt]) row = 0;   // a valid row; its result is not stored
    const int64_t m = (uint32_t)row / (uint32_t)nI;
    const int I = (int)(row - m * nI);
    mrow[rt] = m;
    irow[rt] = I;
    rsc[rt] = dscale[m];
    rbase[rt] = m * s_node_stride(C) + (int64_t)(sbase + I) * COLS + 8 * q;
  }
  const int64_t part = 6LL * C * COLS;   // fp16 per weight part
  f4 acc[4][NA];
#pragma unroll
  for (int rt = 0; rt < 4; ++rt)
#pragma unroll
    for (int at = 0; at < NA; ++at) acc[rt][at] = f4{0.f, 0.f, 0.f, 0.f};

  const int tb = kh * TPP / ks, te = (kh + 1) * TPP / ks;   // ks <= 16 < TPP: every part is non-empty
  f4 stg[NST], bc[4][2], bn[4][2];
  auto load_w = [&](int t) {
#pragma unroll
    for (int i = 0; i < NST; ++i) {
      const int idx = threadIdx.x + 256 * i;   // (part, a, 8-column piece)
      if (idx < NPC) {
        const int pt = idx / (C * 4), rem = idx - pt * (C * 4);
        stg[i] = *reinterpret_cast<const f4*>(bk6 + pt * part + ((int64_t)p * C + (rem >> 2)) * COLS + 32 * t +
                                              8 * (rem & 3));
      }
    }
  };
  auto store_w = [&](int buf) {
#pragma unroll
    for (int i = 0; i < NST; ++i) {
      const int idx = threadIdx.x + 256 * i;
      if (idx < NPC) {
        const int pt = idx / (C * 4), rem = idx - pt * (C * 4);
        *reinterpret_cast<f4*>(&wsh[buf][pt][rem >> 2][8 * (rem & 3)]) = stg[i];
      }
    }
  };
  auto load_ds = [&](f4 (&b)[4][2], int t) {
#pragma unroll
    for (int rt = 0; rt < 4; ++rt)
#pragma unroll
      for (int u = 0; u < 2; ++u) b[rt][u] = ld4(dS + rbase[rt] + 32 * t + 4 * u);
  };
  load_w(tb);
  load_ds(bc, tb);
  store_w(0);
  __syncthreads();
#pragma unroll 1
  for (int t = tb; t < te; ++t) {
    const int buf = (t - tb) & 1;
    if (t + 1 < te) {
      load_w(t + 1);
      load_ds(bn, t + 1);
    }
    __builtin_amdgcn_sched_barrier(0);
    h8 dh[4], dl[4];
    bf8 db[4];
#pragma unroll
    for (int rt = 0; rt < 4; ++rt) {
      const float v[8] = {bc[rt][0].x, bc[rt][0].y, bc[rt][0].z, bc[rt][0].w,
                          bc[rt][1].x, bc[rt][1].y, bc[rt][1].z, bc[rt][1].w};
      if constexpr (BF16) {
#pragma unroll
        for (int j = 0; j < 8; ++j) db[rt][j] = (__bf16)(v[j] * rsc[rt]);
      } else {
        split2h(v, rsc[rt], dh[rt], dl[rt]);
      }
    }
#pragma unroll
    for (int at = 0; at < NA; ++at) {
      const int a = QW * (r >> 2) + 4 * at + (r & 3);
      if constexpr (BF16) {
        const bf8 wb = *reinterpret_cast<const bf8*>(&wsh[buf][0][a][8 * q]);
#pragma unroll
        for (int rt = 0; rt < 4; ++rt) acc[rt][at] = mfma_bf16(wb, db[rt], acc[rt][at]);
      } else {
        const h8 wh = *reinterpret_cast<const h8*>(&wsh[buf][0][a][8 * q]);
        const h8 wl = *reinterpret_cast<const h8*>(&wsh[buf][1][a][8 * q]);
#pragma unroll
        for (int rt = 0; rt < 4; ++rt) acc[rt][at] = mfma_x3(wh, wl, dh[rt], dl[rt], acc[rt][at]);
      }
    }
    if (t + 1 < te) {
      store_w(buf ^ 1);
#pragma unroll
      for (int rt = 0; rt < 4; ++rt) {
        bc[rt][0] = bn[rt][0];
        bc[rt][1] = bn[rt][1];
      }
    }
    __syncthreads();
  }
#pragma unroll
  for (int rt = 0; rt < 4; ++rt) {
    if (!ok[rt]) continue;
    float* o = dxp + (((int64_t)kh * NSLOT + sbase + irow[rt]) * n_nodes + mrow[rt]) * C + QW * q;
    const float f = winv[0] / rsc[rt];   // rsc is a power of two: exact
#pragma unroll
    for (int at = 0; at < NA; ++at) st4(o + 4 * at, acc[rt][at] * f);
  }
}

// dx[m][comp][a] = sum over the K parts and the slots of comp: comp 0 <- slots 0,1,2;
// comp 1+i <- slots 3+i, 6+i; comp 4+ij <- slot 9+ij.
template <int C>
__global__ void node_expand_grad_combine_kernel(const float* __restrict__ dxp, float* __restrict__ dx,
                                                int64_t n_nodes, int ks) {
  const int64_t idx = blockIdx.x * (int64_t)blockDim.x + threadIdx.x;   // over N*13*C/4
  if (idx >= n_nodes * NCOMP * (C / 4)) return;
  const int a4 = (int)(idx % (C / 4));
  const int comp = (int)((idx / (C / 4)) % NCOMP);
  const int64_t m = idx / (NCOMP * (C / 4));
  int sl[3];
  int ns;
  if (comp == 0) {
    sl[0] = 0; sl[1] = 1; sl[2] = 2; ns = 3;
  } else if (comp < 4) {
    sl[0] = 2 + comp; sl[1] = 5 + comp; sl[2] = 0; ns = 2;
  } else {
    sl[0] = 5 + comp; sl[1] = 0; sl[2] = 0; ns = 1;
  }
  // slot by slot, the K parts in order (unrolled: their loads go out together)
  f4 s = {0.f, 0.f, 0.f, 0.f};
  for (int i = 0; i < ns; ++i) {
    const float* base = dxp + ((int64_t)sl[i] * n_nodes + m) * C + 4 * a4;
#pragma unroll 8
    for (int kh = 0; kh < ks; ++kh) s += ld4(base + (int64_t)kh * NSLOT * n_nodes * C);
  }
  st4(dx + (m * NCOMP + comp) * C + 4 * a4, s);
}

// ---------------------------------------------------------------- K2: edge message
// One block (3 waves) per source node; P[eid][col] = sum_k h[eid][k] S[m][col][k] + Sb[m][col].
// Transposed product: S rows (columns of P) are the A operand, the node's edges (h rows, split into
// three bf16 planes in LDS) the B operand; products are split-bf16 (mfma_x6, K = 64 in two steps),
// the S rows split in registers (BF16: one bf16 MFMA per product, both operands rounded to bf16).  A wave takes 32-column blocks of P's chunk-major column order;
// tile jt's A row i is column 8*(i/4) + 4*jt + i%4 of the block, so lane (r, q) ends with 8
// consecutive columns of edge r: two float4 stores, 128 contiguous bytes per edge per block.
constexpr int EP = 64;   // edges per pass held in LDS

template <int C, bool BF16>
__global__ __launch_bounds__(192, 2) void edge_message_kernel(const float* __restrict__ h,
                                                           const float* __restrict__ S,
                                                           const int32_t* __restrict__ src_ptr,
                                                           const int32_t* __restrict__ src_perm,
                                                           float* __restrict__ P, int64_t n_nodes,
                                                           const int32_t* __restrict__ node_order) {
  constexpr int HR = KH + 8;   // bf16 per LDS row: 64 + 8 padding
  __shared__ __align__(16) __bf16 hs3[3][EP][HR];
  __shared__ int32_t eids[EP];
  const int m = xcd_node(n_nodes, node_order);
  if (m < 0) return;
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int r = lane & 15, q = lane >> 4;
  const int beg = src_ptr[m], end = src_ptr[m + 1];
  constexpr int COLS = 65 * C;
  constexpr int NCOL = NSLOT * C;
  constexpr int NJ = 2;              // 16-column tiles per column block
  constexpr int BW = 16 * NJ;        // column block width
  constexpr int NCB = NCOL / BW;
  const float* Sm = S + (int64_t)m * s_node_stride(C);
  const __bf16* Smb = reinterpret_cast<const __bf16*>(S) + (int64_t)m * s_node_stride(C);   // BF16: bf16 S

  // a[jt][0..3]: S row of A row r of tile jt at k = 8q..8q+7 (0, 1) and 32+8q..32+8q+7 (2, 3) (BF16: the
  // eight bf16 values of k = 8q.. in a[jt][0] and of k = 32+8q.. in a[jt][2]);
  // a[jt][4]: the biases of the lane's four output columns of tile jt.  Column block cb+3 is loaded
  // while block cb is multiplied.
  f4 a0[NJ][5], a1[NJ][5];
  // Columns are numbered in P's order (p_col): blocks of 32 consecutive columns are stored contiguously.
  auto load = [&](f4 (&a)[NJ][5], int cb) {
#pragma unroll
    for (int jt = 0; jt < NJ; ++jt) {
      const int col = cb * BW + 4 * NJ * (r >> 2) + 4 * jt + (r & 3);
      int pos, c;
      p_col_inverse<C>(col, pos, c);
      const int slot = slot_at_pos(pos);
      const int colq = cb * BW + 4 * NJ * q + 4 * jt;   // four consecutive channels of one slot
      int posq, cq;
      p_col_inverse<C>(colq, posq, cq);
      if constexpr (BF16) {
        typedef __bf16 bf4 __attribute__((ext_vector_type(4)));
        const __bf16* srow = Smb + (int64_t)slot * COLS + c * KH + 8 * q;
        a[jt][0] = *reinterpret_cast<const f4*>(srow);
        a[jt][2] = *reinterpret_cast<const f4*>(srow + 32);
        const bf4 bb = *reinterpret_cast<const bf4*>(Smb + (int64_t)slot_at_pos(posq) * COLS + 64 * C + cq);
        a[jt][4] = f4{(float)bb[0], (float)bb[1], (float)bb[2], (float)bb[3]};
      } else {
        const float* srow = Sm + (int64_t)slot * COLS + c * KH + 8 * q;
        a[jt][0] = ld4(srow);
        a[jt][1] = ld4(srow + 4);
        a[jt][2] = ld4(srow + 32);
        a[jt][3] = ld4(srow + 36);
        a[jt][4] = ld4(Sm + (int64_t)slot_at_pos(posq) * COLS + 64 * C + cq);
      }
    }
  };

  // this block's column blocks: part blockIdx.y of gridDim.y (msg_parts)
  const int cb0 = (int)(blockIdx.y * NCB / gridDim.y), cb1 = (int)((blockIdx.y + 1) * NCB / gridDim.y);
  for (int pb = beg; pb < end; pb += EP) {
    const int cnt = min(EP, end - pb);
    if (cb0 + wave < cb1) load(a0, cb0 + wave);   // independent of the staging below
    __syncthreads();
    if (threadIdx.x < EP) eids[threadIdx.x] = src_perm[pb + min((int)threadIdx.x, cnt - 1)];
    __syncthreads();
    // h rows split into the three planes, 8 consecutive k per thread; rows e >= cnt repeat edge cnt-1
    // (their results are not stored)
    for (int idx = threadIdx.x; idx < EP * (KH / 8); idx += 192) {
      const int e = idx / (KH / 8), k8 = idx % (KH / 8);
      const float* hp = h + (int64_t)eids[e] * KH + 8 * k8;
      const f4 x0 = ld4(hp), x1 = ld4(hp + 4);
      const float v[8] = {x0.x, x0.y, x0.z, x0.w, x1.x, x1.y, x1.z, x1.w};
      bf8 bh, bm, bl;
      if constexpr (BF16) {
#pragma unroll
        for (int j = 0; j < 8; ++j) bh[j] = (__bf16)v[j];
        *reinterpret_cast<bf8*>(&hs3[0][e][8 * k8]) = bh;
      } else {
        split3(v, bh, bm, bl);
        *reinterpret_cast<bf8*>(&hs3[0][e][8 * k8]) = bh;
        *reinterpret_cast<bf8*>(&hs3[1][e][8 * k8]) = bm;
        *reinterpret_cast<bf8*>(&hs3[2][e][8 * k8]) = bl;
      }
    }
    __syncthreads();
    const int nrt = (cnt + 15) / 16;
    auto run = [&](const f4 (&a)[NJ][5], int cb) {
      f4 acc[4][NJ];
#pragma unroll
      for (int et = 0; et < 4; ++et)
#pragma unroll
        for (int jt = 0; jt < NJ; ++jt) acc[et][jt] = f4{0.f, 0.f, 0.f, 0.f};
      bf8 ah[NJ][2], am[NJ][2], al[NJ][2];
#pragma unroll
      for (int jt = 0; jt < NJ; ++jt)
#pragma unroll
        for (int ks = 0; ks < 2; ++ks) {
          if constexpr (BF16) {
            ah[jt][ks] = __builtin_bit_cast(bf8, a[jt][2 * ks]);
          } else {
            const f4 x0 = a[jt][2 * ks], x1 = a[jt][2 * ks + 1];
            const float v[8] = {x0.x, x0.y, x0.z, x0.w, x1.x, x1.y, x1.z, x1.w};
            split3(v, ah[jt][ks], am[jt][ks], al[jt][ks]);
          }
        }
#pragma unroll
      for (int et = 0; et < 4; ++et) {
        if (et < nrt) {
#pragma unroll
          for (int ks = 0; ks < 2; ++ks) {
            const bf8 bh = *reinterpret_cast<const bf8*>(&hs3[0][16 * et + r][32 * ks + 8 * q]);
            if constexpr (BF16) {
#pragma unroll
              for (int jt = 0; jt < NJ; ++jt) acc[et][jt] = mfma_bf16(ah[jt][ks], bh, acc[et][jt]);
            } else {
              const bf8 bm = *reinterpret_cast<const bf8*>(&hs3[1][16 * et + r][32 * ks + 8 * q]);
              const bf8 bl = *reinterpret_cast<const bf8*>(&hs3[2][16 * et + r][32 * ks + 8 * q]);
#pragma unroll
              for (int jt = 0; jt < NJ; ++jt)
                acc[et][jt] = mfma_x6(ah[jt][ks], am[jt][ks], al[jt][ks], bh, bm, bl, acc[et][jt]);
            }
          }
        }
      }
#pragma unroll
      for (int et = 0; et < 4; ++et) {
        const int e = 16 * et + r;
        if (et < nrt && e < cnt) {
          float* o = P + (int64_t)eids[e] * NCOL + cb * BW + 4 * NJ * q;
#pragma unroll
          for (int jt = 0; jt < NJ; ++jt) st4(o + 4 * jt, acc[et][jt] + a[jt][4]);
        }
      }
    };
#pragma unroll 1
    for (int cb = cb0 + wave; cb < cb1; cb += 6) {
      if (cb + 3 < cb1) load(a1, cb + 3);
      __builtin_amdgcn_sched_barrier(0);
      run(a0, cb);
      if (cb + 3 < cb1) {
        if (cb + 6 < cb1) load(a0, cb + 6);
        __builtin_amdgcn_sched_barrier(0);
        run(a1, cb + 3);
      }
    }
  }
}

// ---------------------------------------------------------------- K3: receiver sum
// One wave per receiver; lanes cover channels (C/64 channels per lane above 64), 64/C edges in flight per
// wave below.  DIR (training double backward): the derivative of the assembly along edge directions u
// (udir [E][3]), m0' = 0, m1' = P1 u, m2' = P2 (u n^T + n u^T) + P4 u^T.
template <int C, bool DIR = false>
__global__ __launch_bounds__(256) void receiver_sum_kernel(const float* __restrict__ P,
                                                           const float* __restrict__ nvec,
                                                           const float* __restrict__ udir,
                                                           const int32_t* __restrict__ dst_ptr,
                                                           float scale, float* __restrict__ out,
                                                           int64_t n_nodes) {
  const int lane = threadIdx.x & 63;
  const int64_t n = (int64_t)blockIdx.x * 4 + (threadIdx.x >> 6);
  if (n >= n_nodes) return;
  constexpr int EPW = C < 64 ? 64 / C : 1;    // edges in flight per wave
  constexpr int CPL = C > 64 ? C / 64 : 1;    // channels per lane: c, c + 64, ..
  constexpr int CW = C < 64 ? C : 64;         // lanes per edge
  const int c0 = lane % CW, sub = lane / CW;
  float o[CPL][NCOMP];
#pragma unroll
  for (int k = 0; k < CPL; ++k)
#pragma unroll
    for (int i = 0; i < NCOMP; ++i) o[k][i] = 0.f;
  const int beg = dst_ptr[n], end = dst_ptr[n + 1];
  for (int e = beg + sub; e < end; e += EPW) {
    const float* pr = P + (int64_t)e * (NSLOT * C);
    const float n0 = nvec[3 * (int64_t)e], n1 = nvec[3 * (int64_t)e + 1], n2 = nvec[3 * (int64_t)e + 2];
    const float nn[3] = {n0, n1, n2};
#pragma unroll
    for (int k = 0; k < CPL; ++k) {
      const int c = c0 + 64 * k;
      auto ps = [&](int slot) { return pr[p_col<C>(pos_of_slot(slot), c)]; };
      const float p0 = ps(0), p1 = ps(1), p2 = ps(2);
      if constexpr (!DIR) {
        o[k][0] += p0;
#pragma unroll
        for (int i = 0; i < 3; ++i) o[k][1 + i] += p1 * nn[i] + ps(3 + i);
#pragma unroll
        for (int i = 0; i < 3; ++i) {
          const float p4 = ps(6 + i);
          const float p2ni = p2 * nn[i];
#pragma unroll
          for (int j = 0; j < 3; ++j) o[k][4 + 3 * i + j] += p2ni * nn[j] + p4 * nn[j] + ps(9 + 3 * i + j);
        }
      } else {
        const float uu[3] = {udir[3 * (int64_t)e], udir[3 * (int64_t)e + 1], udir[3 * (int64_t)e + 2]};
#pragma unroll
        for (int i = 0; i < 3; ++i) o[k][1 + i] += p1 * uu[i];
#pragma unroll
        for (int i = 0; i < 3; ++i) {
          const float p4 = ps(6 + i);
#pragma unroll
          for (int j = 0; j < 3; ++j) o[k][4 + 3 * i + j] += p2 * (uu[i] * nn[j] + nn[i] * uu[j]) + p4 * uu[j];
        }
      }
    }
  }
  if (EPW > 1) {
#pragma unroll
    for (int i = 0; i < NCOMP; ++i)
      for (int off = C; off < 64; off <<= 1) o[0][i] += __shfl_xor(o[0][i], off, 64);
  }
  if (sub == 0) {
#pragma unroll
    for (int k = 0; k < CPL; ++k) {
      float* orow = out + n * NCOMP * C + c0 + 64 * k;
#pragma unroll
      for (int i = 0; i < NCOMP; ++i) orow[i * C] = o[k][i] * scale;
    }
  }
}

// ---------------------------------------------------------------- K5: edge message grad
// One block per source node; the receiver gradient comes chunk-major (grad_chunk_major_kernel).
// With g = G[dst(e)] * scale, the message gradient is
//   dP_e[0] = g0, dP_e[1] = g1.n, dP_e[2] = n.g2.n, dP_e[3+i] = g1[i],
//   dP_e[6+i] = (g2 n)[i], dP_e[9+ij] = g2[ij]
// (per channel).  Per chunk of CC channels the block writes dP for its edges into LDS, then
//   dh[e][k]            += sum_{slot,c} dP_e[slot][c] S[m][slot][c][k]    (MFMA, rows = edges)
//   dS[m][slot][c][k]    = sum_e dP_e[slot][c] h[e][k]                    (MFMA, rows = k)
//   dS[m][slot][64C + c] = sum_e dP_e[slot][c]                            (bias column)
// and the direction gradient of the receiver assembly (m1 = P1 n + P3, m2 = P2 n n + P4 n + P5)
//   dn_e[k] = sum_c g1[k] P1 + P2 ((g2 n)[k] + (g2^T n)[k]) + (g2^T P4)[k]
// is summed over the chunk's channels by lane shuffles and over chunks in a fixed order.
// Register budget (3 waves per SIMD): the h values of the dS product stay in registers for the edge
// block (no LDS copy, 40 KB of LDS per block), and the S loads and dS stores use buffer addressing
// with the large constant strides in scalar offsets, so no per-load 64-bit addresses are held.
// The receiver gradient in channel chunks: Gt[c/8][n][comp][c%8] = G[n][comp][c].
template <int C>
__global__ void grad_chunk_major_kernel(const float* __restrict__ G, float* __restrict__ Gt, int64_t n_nodes) {
  const int64_t idx = blockIdx.x * (int64_t)blockDim.x + threadIdx.x;   // float4 of G
  if (idx >= n_nodes * NCOMP * (C / 4)) return;
  const int c4 = (int)(idx % (C / 4));
  const int64_t row = idx / (C / 4);                                    // n*13 + comp
  st4(Gt + ((int64_t)(c4 / 2) * n_nodes * NCOMP + row) * 8 + 4 * (c4 % 2), ld4(G + row * C + 4 * c4));
}

// DIR (training double backward): the same products for the derivative of the receiver assembly along
// edge directions u (udir [E][3]): dP'_e = D_n dP_e [u] = (0, g1.u, u.g2.n + n.g2.u, 0, g2 u, 0), and in
// place of the direction gradient the second-derivative term dn_e = sum_c P2 (g2 + g2^T) u.
template <int C, bool DIR = false, bool BF16S = false>
__global__ __launch_bounds__(256, 2) void edge_message_grad_kernel(
    const float* __restrict__ Gt, const float* __restrict__ nvec, const float* __restrict__ udir,
    const float* __restrict__ h,
    const float* __restrict__ S, const float* __restrict__ P, const int32_t* __restrict__ src_ptr,
    const int32_t* __restrict__ src_perm, const int32_t* __restrict__ edge_dst, float scale,
    float* __restrict__ dh, float* __restrict__ dS, float* __restrict__ dn, float* __restrict__ dscale,
    int64_t n_nodes, const int32_t* __restrict__ node_order) {
  constexpr int CC = 8;              // channels per chunk
  constexpr int NCH = C / CC;
  constexpr int DW = NSLOT * CC;     // dP columns per chunk, column = slot*CC + c
  constexpr int NCT = DW / 16;       // 16-wide column tiles per chunk
  constexpr int COLS = 65 * C;
  constexpr int NCOL = NSLOT * C;
  __shared__ float dps[EP][DW + 4];
  __shared__ int32_t eids[EP];
  __shared__ int32_t dsts[EP];
  __shared__ float ns[EP][3];
  __shared__ float us[DIR ? EP : 1][3];
  __shared__ float dnacc[EP][3];
  __shared__ float amx[4];
  const int m = xcd_node(n_nodes, node_order);
  if (m < 0) return;
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int r = lane & 15, q = lane >> 4;
  const int beg = src_ptr[m], end = src_ptr[m + 1];
  const float* Sm = S + (int64_t)m * s_node_stride(C);
  float* dSm = dS + (int64_t)m * s_node_stride(C);
  // BF16S (the bf16 variant): S is held in bf16, read and widened to fp32 here
  constexpr int SB = BF16S ? 2 : 4;
  const __amdgpu_buffer_rsrc_t srs = buffer_rsrc_bytes(
      const_cast<char*>(reinterpret_cast<const char*>(S)) + (int64_t)m * s_node_stride(C) * SB,
      (uint32_t)(s_node_stride(C) * SB));
  const __amdgpu_buffer_rsrc_t drs = buffer_rsrc(dSm, (uint32_t)(s_node_stride(C) * 4));
  const uint32_t svoff = (uint32_t)(((q >> 1) * COLS + 4 * (q & 1) * KH + 16 * wave + r) * SB);
  const uint32_t dvoff = (uint32_t)(((r >> 3) * COLS + (r & 7) * KH + 16 * wave + 4 * q) * 4);
  const int cl = threadIdx.x & (CC - 1);   // dP builder: channel within the chunk
  const int eb = threadIdx.x / CC;         // dP builder: edges eb, eb + 32

  if (end == beg) {   // no out-edges: dS of this node is zero (block-uniform branch)
    for (int idx = threadIdx.x; idx < NSLOT * COLS / 4; idx += 256) st4(dSm + 4 * idx, f4{0.f, 0.f, 0.f, 0.f});
    if (threadIdx.x == 0) dscale[m] = 1.f;
    return;
  }
  float amax = 0.f;   // max |dS| over the values stored by the last edge block (the final ones)
  int pb = beg;
  bool first = true;
  do {
    const int cnt = min(EP, end - pb);   // >= 1
    __syncthreads();
    // Rows e >= cnt point at edge cnt-1, so every load below stays unconditional; their
    // direction and h rows are zero and their dP is masked to zero.
    if (threadIdx.x < EP) {
      const int e = threadIdx.x;
      const int32_t id = src_perm[pb + min(e, cnt - 1)];
      eids[e] = id;
      dsts[e] = edge_dst[id];
#pragma unroll
      for (int k = 0; k < 3; ++k) {
        const float v = nvec[3 * (int64_t)id + k];
        ns[e][k] = (e < cnt) ? v : 0.f;
        if constexpr (DIR) us[e][k] = (e < cnt) ? udir[3 * (int64_t)id + k] : 0.f;
        dnacc[e][k] = 0.f;
      }
    }
    __syncthreads();
    // A operand of the dS product, kept in registers for the whole edge block: lane (r, q) of wave w
    // holds h[edge 4u + q][16 w + r] (zero beyond cnt)
    float hreg[EP / 4];
#pragma unroll
    for (int u = 0; u < EP / 4; ++u) {
      const int e = 4 * u + q;
      hreg[u] = (e < cnt) ? h[(int64_t)eids[e] * KH + 16 * wave + r] : 0.f;
    }
    const int nrt = (cnt + 15) / 16;
    const int ksteps = (cnt + 3) / 4;
    f4 dacc[4];
#pragma unroll
    for (int et = 0; et < 4; ++et) dacc[et] = f4{0.f, 0.f, 0.f, 0.f};

    // Receiver gradients (and P) for the next chunk's dP are loaded while the current chunk is
    // multiplied; the S values of a chunk's dh product are loaded before its dP is built.
    float gN[2][NCOMP], pN[2][5], sv[NCT][4];
    auto load_g = [&](int ch) {
#pragma unroll
      for (int hh = 0; hh < 2; ++hh) {
        const int e = eb + 32 * hh;
        // Gt[ch][dst][13][8]: the chunk's 13 components of the receiver gradient are contiguous
        const float* gp = Gt + ((int64_t)ch * n_nodes + dsts[e]) * (NCOMP * CC) + cl;
#pragma unroll
        for (int i = 0; i < NCOMP; ++i) gN[hh][i] = gp[i * CC];
        const float* pp = P + (int64_t)eids[e] * NCOL + ch * 40 + cl;   // p_col of positions 0..4
        pN[hh][0] = pp[pos_of_slot(1) * CC];
        pN[hh][1] = pp[pos_of_slot(2) * CC];
        pN[hh][2] = pp[pos_of_slot(6) * CC];
        pN[hh][3] = pp[pos_of_slot(7) * CC];
        pN[hh][4] = pp[pos_of_slot(8) * CC];
      }
    };
    // Chunk column kk = 16 tt + 4 q + s4 is slot kk/8 = 2 tt + q/2, channel ch*8 + 4 (q&1) + s4: the lane
    // part of the address is one vector offset, the (tt, s4, ch) part a scalar one (no per-load address
    // registers).
    auto load_s = [&](int ch) {
#pragma unroll
      for (int tt = 0; tt < NCT; ++tt)
#pragma unroll
        for (int s4 = 0; s4 < 4; ++s4)
          sv[tt][s4] = BF16S ? buffer_ld1_bf16(srs, svoff, (uint32_t)((2 * tt * COLS + (ch * CC + s4) * KH) * SB))
                             : buffer_ld1(srs, svoff, (uint32_t)((2 * tt * COLS + (ch * CC + s4) * KH) * SB));
    };
    load_g(0);
#pragma unroll 1
    for (int ch = 0; ch < NCH; ++ch) {
      const int c0 = ch * CC;
      load_s(ch);
      __builtin_amdgcn_sched_barrier(0);
      // ---- dP for edges eb, eb+32 and channel c0+cl; direction-gradient partials
#pragma unroll
      for (int hh = 0; hh < 2; ++hh) {
        const int e = eb + 32 * hh;
        float v[NSLOT];
        float t[3];
        float g[NCOMP];
        const float sc = (e < cnt) ? scale : 0.f;
#pragma unroll
        for (int i = 0; i < NCOMP; ++i) g[i] = gN[hh][i] * sc;
        const float nn[3] = {ns[e][0], ns[e][1], ns[e][2]};
        const float p1 = pN[hh][0], p2 = pN[hh][1];
        const float p4[3] = {pN[hh][2], pN[hh][3], pN[hh][4]};
        if constexpr (!DIR) {
          v[0] = g[0];
          v[1] = g[1] * nn[0] + g[2] * nn[1] + g[3] * nn[2];
          float nqn = 0.f;
#pragma unroll
          for (int i = 0; i < 3; ++i) {
            float row = 0.f, colv = 0.f, p4t = 0.f;
#pragma unroll
            for (int j = 0; j < 3; ++j) {
              row += g[4 + 3 * i + j] * nn[j];
              colv += g[4 + 3 * j + i] * nn[j];
              p4t += g[4 + 3 * j + i] * p4[j];
            }
            v[3 + i] = g[1 + i];
            v[6 + i] = row;
            nqn += row * nn[i];
            t[i] = g[1 + i] * p1 + p2 * (row + colv) + p4t;
          }
          v[2] = nqn;
#pragma unroll
          for (int i = 0; i < 9; ++i) v[9 + i] = g[4 + i];
        } else {
          const float uu[3] = {us[e][0], us[e][1], us[e][2]};
#pragma unroll
          for (int s4 = 0; s4 < NSLOT; ++s4) v[s4] = 0.f;
          v[1] = g[1] * uu[0] + g[2] * uu[1] + g[3] * uu[2];
          float cross = 0.f;
#pragma unroll
          for (int i = 0; i < 3; ++i) {
            float g2u = 0.f, g2tu = 0.f, g2n = 0.f;
#pragma unroll
            for (int j = 0; j < 3; ++j) {
              g2u += g[4 + 3 * i + j] * uu[j];
              g2tu += g[4 + 3 * j + i] * uu[j];
              g2n += g[4 + 3 * i + j] * nn[j];
            }
            v[6 + i] = g2u;
            cross += uu[i] * g2n + nn[i] * g2u;
            t[i] = p2 * (g2u + g2tu);
          }
          v[2] = cross;
        }
        // rows e >= cnt hold zeros (g is masked)
#pragma unroll
        for (int s4 = 0; s4 < NSLOT; ++s4) dps[e][s4 * CC + cl] = v[s4];
#pragma unroll
        for (int k = 0; k < 3; ++k) t[k] = group_sum(t[k], CC);
        if (cl == 0 && e < cnt) {
#pragma unroll
          for (int k = 0; k < 3; ++k) dnacc[e][k] += t[k];
        }
      }
      __syncthreads();
      if (ch + 1 < NCH) load_g(ch + 1);
      __builtin_amdgcn_sched_barrier(0);
      // ---- dh: rows = edges (tile et), columns = k in [16*wave, 16*wave+16), K = chunk columns
#pragma unroll
      for (int tt = 0; tt < NCT; ++tt) {
        const f4 b4 = {sv[tt][0], sv[tt][1], sv[tt][2], sv[tt][3]};
#pragma unroll
        for (int et = 0; et < 4; ++et) {
          if (et < nrt) {
            const f4 a4 = *reinterpret_cast<const f4*>(&dps[16 * et + r][16 * tt + 4 * q]);
            dacc[et] = mfma_k16(a4, b4, dacc[et]);
          }
        }
      }
      // ---- dS^T: rows = k in [16*wave, 16*wave+16), columns = chunk columns, K = edges
      f4 sacc[NCT];
#pragma unroll
      for (int ct = 0; ct < NCT; ++ct) sacc[ct] = f4{0.f, 0.f, 0.f, 0.f};
      // edges are taken in pairs of K steps; rows up to 64 are zero beyond cnt
#pragma unroll
      for (int uu = 0; uu < EP / 8; ++uu) {
        if (2 * uu < ksteps) {
          const int u = 2 * uu;
          float b0[NCT], b1[NCT];
#pragma unroll
          for (int ct = 0; ct < NCT; ++ct) {
            b0[ct] = dps[4 * u + q][16 * ct + r];
            b1[ct] = dps[4 * u + 4 + q][16 * ct + r];
          }
#pragma unroll
          for (int ct = 0; ct < NCT; ++ct) sacc[ct] = mfma16x16x4(hreg[u], b0[ct], sacc[ct]);
#pragma unroll
          for (int ct = 0; ct < NCT; ++ct) sacc[ct] = mfma16x16x4(hreg[u + 1], b1[ct], sacc[ct]);
        }
      }
      // column 16 ct + r of the chunk is slot 2 ct + r/8, channel c0 + r%8
#pragma unroll
      for (int ct = 0; ct < NCT; ++ct) {
        const uint32_t so = (uint32_t)((2 * ct * COLS + c0 * KH) * 4);
        f4 v = sacc[ct];
        if (!first) v += buffer_ld4(drs, dvoff, so);
        buffer_st4(drs, dvoff, so, v);
        amax = fmaxf(amax, fmaxf(fmaxf(fabsf(v[0]), fabsf(v[1])), fmaxf(fabsf(v[2]), fabsf(v[3]))));
      }
      if (threadIdx.x < DW) {
        const int col = threadIdx.x;
        // rows >= cnt hold zeros: run to a multiple of 8 with the reads of a group issued together
        float s4[4] = {0.f, 0.f, 0.f, 0.f};
        const int e8 = (cnt + 7) & ~7;
        for (int e = 0; e < e8; e += 8) {
          float v8[8];
#pragma unroll
          for (int u = 0; u < 8; ++u) v8[u] = dps[e + u][col];
#pragma unroll
          for (int u = 0; u < 8; ++u) s4[u & 3] += v8[u];
        }
        const float sum = (s4[0] + s4[1]) + (s4[2] + s4[3]);
        float* o = dSm + (int64_t)(col / CC) * COLS + 64 * C + c0 + col % CC;
        const float fin = first ? sum : (*o + sum);
        *o = fin;
        amax = fmaxf(amax, fabsf(fin));
      }
      __syncthreads();
    }
#pragma unroll
    for (int et = 0; et < 4; ++et) {
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        const int e = 16 * et + 4 * q + j;
        if (e < cnt) dh[(int64_t)eids[e] * KH + 16 * wave + r] = dacc[et][j];
      }
    }
    if (threadIdx.x < cnt) {
      const int e = threadIdx.x;
#pragma unroll
      for (int k = 0; k < 3; ++k) dn[3 * (int64_t)eids[e] + k] = dnacc[e][k];
    }
    first = false;
    pb += EP;
    if (pb < end) amax = 0.f;   // block-uniform: only the last edge block's stores are final
  } while (pb < end);
  // per-node power of two for the split-fp16 products of node_expand_grad
  for (int off = 32; off > 0; off >>= 1) amax = fmaxf(amax, __shfl_xor(amax, off, 64));
  if (lane == 0) amx[wave] = amax;
  __syncthreads();
  if (threadIdx.x == 0) dscale[m] = pow2_scale(fmaxf(fmaxf(amx[0], amx[1]), fmaxf(amx[2], amx[3])));
}

// Per-node bound of the receiver gradient for the split-fp16 message gradient: gmax[n] = max |G[n][comp][c]|.
// One wave per node (13 C values).
template <int C>
__global__ __launch_bounds__(256) void grad_absmax_kernel(const float* __restrict__ G, float* __restrict__ gmax,
                                                          int64_t n_nodes) {
  const int64_t n = (int64_t)blockIdx.x * 4 + (threadIdx.x >> 6);
  if (n >= n_nodes) return;   // wave-uniform
  const int lane = threadIdx.x & 63;
  const float* g = G + n * NCOMP * C;
  float m = 0.f;
  for (int i = lane; i < NCOMP * C / 4; i += 64) {
    const f4 v = ld4(g + 4 * i);
    m = fmaxf(m, fmaxf(fmaxf(fabsf(v.x), fabsf(v.y)), fmaxf(fabsf(v.z), fabsf(v.w))));
  }
  for (int off = 32; off > 0; off >>= 1) m = fmaxf(m, __shfl_xor(m, off, 64));
  if (lane == 0) gmax[n] = m;
}

// The message gradient with both products on fp16 MFMA in fp32 precision (split-fp16, common.h): the same
// sums as edge_message_grad_kernel, per source node m and 64-edge block, 8-channel chunk by chunk.
//   dh[e][k]  = sum_{(slot,c)} dP[e][(slot,c)] S[m][(slot,c)][k]        A = dP rows, B = S      (K = 144)
//   dS[k][col] = sum_e h[e][k] dP[e][col]                                A = h^T,     B = dP     (K = edges)
// dP is held once, in LDS, as two fp16 planes of dP[e] * s_e, s_e the power of two of an upper bound of the
// edge's row: |dP| <= 3 max|g| (|n| = 1: |g1.n|, |(g2 n)_i| <= sqrt 3 max|g|, |n.g2.n| <= 3 max|g|), from the
// receiver's max |G| (grad_absmax_kernel).  The dh product undoes s_e per row; the dS product, whose K runs
// over edges, takes h[e][k] / s_e as its A operand (exact: powers of two), scaled per k by the power of two of
// that column's max, so the sum over edges needs no rescaling.  S is scaled per (chunk, k) by its own max and
// each chunk's dh product is undone and added to the fp32 dh separately.  The bias column sums the two
// planes over the edges on the VALU.  A lane's dh B operand is 8 consecutive chunk columns of one k (S
// loads at a fixed stride, as in the fp32 kernel); a lane's dS B operand is 8 consecutive edges of one
// column (eight 2-byte LDS reads per plane).  K = 144 is four 32-deep steps and a 16-deep one.
typedef _Float16 h4 __attribute__((ext_vector_type(4)));
constexpr int DPS = 144;   // fp16 row stride of dP in LDS (144 columns, 288 bytes: 16-byte aligned rows)

template <int C>
__global__ __launch_bounds__(256, 4) void edge_message_grad_h16_kernel(
    const float* __restrict__ Gt, const float* __restrict__ gmax, const float* __restrict__ nvec,
    const float* __restrict__ h, const float* __restrict__ S, const float* __restrict__ P,
    const int32_t* __restrict__ src_ptr, const int32_t* __restrict__ src_perm, const int32_t* __restrict__ edge_dst,
    float scale, float* __restrict__ dh, float* __restrict__ dS, float* __restrict__ dn, float* __restrict__ dscale,
    int64_t n_nodes, const int32_t* __restrict__ node_order, int64_t n_edges) {
  constexpr int CC = 8;              // channels per chunk
  constexpr int NCH = C / CC;
  constexpr int DW = NSLOT * CC;     // dP columns per chunk, column = slot*CC + c
  constexpr int NCT = DW / 16;       // 16-wide column tiles per chunk
  constexpr int COLS = 65 * C;
  constexpr int NCOL = NSLOT * C;
  // this block's channel chunks: part blockIdx.y of gridDim.y (msg_parts).  With more than one part, dh, dn
  // and the dS maximum are partial: each part writes its own (dh + part E KH, dn + part 3E, dscale + part N,
  // the maximum itself) and msg_grad_combine_kernel adds them.
  const int part = (int)blockIdx.y, nparts = (int)gridDim.y;
  const int ch0 = part * NCH / nparts, ch1 = (part + 1) * NCH / nparts;
  if (nparts > 1) {
    dh += (int64_t)part * n_edges * KH;
    dn += (int64_t)part * n_edges * 3;
    dscale += (int64_t)part * n_nodes;
  }
  __shared__ __align__(16) _Float16 dpl[2][EP][DPS];   // planes h, l of dP[e] * s_e
  __shared__ int32_t eids[EP];
  __shared__ int32_t dsts[EP];
  __shared__ float ns[EP][3];
  __shared__ float dnacc[EP][3];
  __shared__ float esc[EP];          // s_e
  __shared__ float einv[EP];         // 1 / s_e
  __shared__ float amx[4];
  const int m = xcd_node(n_nodes, node_order);
  if (m < 0) return;
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int r = lane & 15, q = lane >> 4;
  const int beg = src_ptr[m], end = src_ptr[m + 1];
  float* dSm = dS + (int64_t)m * s_node_stride(C);
  const __amdgpu_buffer_rsrc_t srs = buffer_rsrc_bytes(
      const_cast<char*>(reinterpret_cast<const char*>(S)) + (int64_t)m * s_node_stride(C) * 4,
      (uint32_t)(s_node_stride(C) * 4));
  const __amdgpu_buffer_rsrc_t drs = buffer_rsrc(dSm, (uint32_t)(s_node_stride(C) * 4));
  // dh B operand: K step s, lane group q -> slot 4s + q, channels c0 + j; the 16-deep tail: slot 16 + q/2,
  // channels c0 + 4 (q & 1) + j
  const uint32_t svoff = (uint32_t)((q * COLS + 16 * wave + r) * 4);
  const uint32_t svoff_t = (uint32_t)(((q >> 1) * COLS + 4 * (q & 1) * KH + 16 * wave + r) * 4);
  const uint32_t dvoff = (uint32_t)(((r >> 3) * COLS + (r & 7) * KH + 16 * wave + 4 * q) * 4);
  const int cl = threadIdx.x & (CC - 1);   // dP builder: channel within the chunk
  const int eb = threadIdx.x / CC;         // dP builder: edges eb, eb + 32

  if (end == beg) {   // no out-edges: dS of this node is zero (block-uniform branch; part 0 writes it)
    if (part == 0)
      for (int idx = threadIdx.x; idx < NSLOT * COLS / 4; idx += 256) st4(dSm + 4 * idx, f4{0.f, 0.f, 0.f, 0.f});
    if (threadIdx.x == 0) dscale[m] = nparts > 1 ? 0.f : 1.f;
    return;
  }
  float amax = 0.f;   // max |dS| over the values stored by the last edge block (the final ones)
  int pb = beg;
  bool first = true;
  do {
    const int cnt = min(EP, end - pb);   // >= 1
    __syncthreads();
    // Rows e >= cnt point at edge cnt-1, so every load below stays unconditional; their direction and h
    // rows are zero and their dP is masked to zero.
    if (threadIdx.x < EP) {
      const int e = threadIdx.x;
      const int32_t id = src_perm[pb + min(e, cnt - 1)];
      const int32_t d = edge_dst[id];
      eids[e] = id;
      dsts[e] = d;
      const float se = pow2_scale(3.f * gmax[d] * scale);
      esc[e] = se;
      einv[e] = 1.f / se;
#pragma unroll
      for (int k = 0; k < 3; ++k) {
        const float v = nvec[3 * (int64_t)id + k];
        ns[e][k] = (e < cnt) ? v : 0.f;
        dnacc[e][k] = 0.f;
      }
    }
    __syncthreads();
    // A operand of the dS product for the whole edge block: lane (r, q) of wave w holds h[e][k] / s_e
    // for k = 16 w + r and edges e = 32 s + 8 q + j, times the power of two of the column's max
    h8 ah[2], al[2];
    float invsh;
    {
      float hv[2][8];
      float mx = 0.f;
#pragma unroll
      for (int s = 0; s < 2; ++s)
#pragma unroll
        for (int j = 0; j < 8; ++j) {
          const int e = 32 * s + 8 * q + j;
          const float v = (e < cnt) ? h[(int64_t)eids[e] * KH + 16 * wave + r] * einv[e] : 0.f;
          hv[s][j] = v;
          mx = fmaxf(mx, fabsf(v));
        }
      mx = fmaxf(mx, __shfl_xor(mx, 16, 64));
      mx = fmaxf(mx, __shfl_xor(mx, 32, 64));
      const float sh = pow2_scale(mx);
      invsh = 1.f / sh;
#pragma unroll
      for (int s = 0; s < 2; ++s) split2h(hv[s], sh, ah[s], al[s]);
    }
    const int nrt = (cnt + 15) / 16;
    const int nks = (cnt + 31) / 32;
    f4 dacc[4];
#pragma unroll
    for (int et = 0; et < 4; ++et) dacc[et] = f4{0.f, 0.f, 0.f, 0.f};

    float gN[2][NCOMP], pN[2][5], sv[36];
    auto load_g = [&](int ch) {
#pragma unroll
      for (int hh = 0; hh < 2; ++hh) {
        const int e = eb + 32 * hh;
        const float* gp = Gt + ((int64_t)ch * n_nodes + dsts[e]) * (NCOMP * CC) + cl;
#pragma unroll
        for (int i = 0; i < NCOMP; ++i) gN[hh][i] = gp[i * CC];
        const float* pp = P + (int64_t)eids[e] * NCOL + ch * 40 + cl;   // p_col of positions 0..4
        pN[hh][0] = pp[pos_of_slot(1) * CC];
        pN[hh][1] = pp[pos_of_slot(2) * CC];
        pN[hh][2] = pp[pos_of_slot(6) * CC];
        pN[hh][3] = pp[pos_of_slot(7) * CC];
        pN[hh][4] = pp[pos_of_slot(8) * CC];
      }
    };
    auto load_s = [&](int ch) {
#pragma unroll
      for (int s = 0; s < 4; ++s)
#pragma unroll
        for (int j = 0; j < 8; ++j)
          sv[8 * s + j] = buffer_ld1(srs, svoff, (uint32_t)((4 * s * COLS + (ch * CC + j) * KH) * 4));
#pragma unroll
      for (int j = 0; j < 4; ++j)
        sv[32 + j] = buffer_ld1(srs, svoff_t, (uint32_t)((16 * COLS + (ch * CC + j) * KH) * 4));
    };
#pragma unroll 1
    for (int ch = ch0; ch < ch1; ++ch) {
      const int c0 = ch * CC;
      load_g(ch);
      // ---- dP for edges eb, eb+32 and channel c0+cl (scaled by s_e, split into the two planes);
      //      direction-gradient partials in fp32
#pragma unroll
      for (int hh = 0; hh < 2; ++hh) {
        const int e = eb + 32 * hh;
        float v[NSLOT];
        float t[3];
        float g[NCOMP];
        const float sc = (e < cnt) ? scale : 0.f;
#pragma unroll
        for (int i = 0; i < NCOMP; ++i) g[i] = gN[hh][i] * sc;
        const float nn[3] = {ns[e][0], ns[e][1], ns[e][2]};
        const float p1 = pN[hh][0], p2 = pN[hh][1];
        const float p4[3] = {pN[hh][2], pN[hh][3], pN[hh][4]};
        v[0] = g[0];
        v[1] = g[1] * nn[0] + g[2] * nn[1] + g[3] * nn[2];
        float nqn = 0.f;
#pragma unroll
        for (int i = 0; i < 3; ++i) {
          float row = 0.f, colv = 0.f, p4t = 0.f;
#pragma unroll
          for (int j = 0; j < 3; ++j) {
            row += g[4 + 3 * i + j] * nn[j];
            colv += g[4 + 3 * j + i] * nn[j];
            p4t += g[4 + 3 * j + i] * p4[j];
          }
          v[3 + i] = g[1 + i];
          v[6 + i] = row;
          nqn += row * nn[i];
          t[i] = g[1 + i] * p1 + p2 * (row + colv) + p4t;
        }
        v[2] = nqn;
#pragma unroll
        for (int i = 0; i < 9; ++i) v[9 + i] = g[4 + i];
        const float se = esc[e];
#pragma unroll
        for (int s4 = 0; s4 < NSLOT; ++s4) {
          const float x = v[s4] * se;
          const _Float16 xh = (_Float16)x;
          dpl[0][e][s4 * CC + cl] = xh;
          dpl[1][e][s4 * CC + cl] = (_Float16)(x - (float)xh);
        }
#pragma unroll
        for (int k = 0; k < 3; ++k) t[k] = group_sum(t[k], CC);
        if (cl == 0 && e < cnt) {
#pragma unroll
          for (int k = 0; k < 3; ++k) dnacc[e][k] += t[k];
        }
      }
      // ---- dh B operand: the chunk's S values of column k = 16 w + r, scaled by their own power of two
      load_s(ch);
      h8 bh[4], bl[4];
      h4 bth, btl;
      float invss;
      {
        float mx = 0.f;
#pragma unroll
        for (int i = 0; i < 36; ++i) mx = fmaxf(mx, fabsf(sv[i]));
        mx = fmaxf(mx, __shfl_xor(mx, 16, 64));
        mx = fmaxf(mx, __shfl_xor(mx, 32, 64));
        const float ss = pow2_scale(mx);
        invss = 1.f / ss;
#pragma unroll
        for (int s = 0; s < 4; ++s) {
          float t8[8];
#pragma unroll
          for (int j = 0; j < 8; ++j) t8[j] = sv[8 * s + j];
          split2h(t8, ss, bh[s], bl[s]);
        }
#pragma unroll
        for (int j = 0; j < 4; ++j) {
          const float x = sv[32 + j] * ss;
          const _Float16 xh = (_Float16)x;
          bth[j] = xh;
          btl[j] = (_Float16)(x - (float)xh);
        }
      }
      __syncthreads();
      // ---- dh: rows = edges (tile et), columns = k in [16*wave, 16*wave+16), K = chunk columns
#pragma unroll
      for (int et = 0; et < 4; ++et) {
        if (et < nrt) {
          const int row = 16 * et + r;
          f4 c4 = f4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
          for (int s = 0; s < 4; ++s) {
            const h8 xh = *reinterpret_cast<const h8*>(&dpl[0][row][32 * s + 8 * q]);
            const h8 xl = *reinterpret_cast<const h8*>(&dpl[1][row][32 * s + 8 * q]);
            c4 = mfma_x3(xh, xl, bh[s], bl[s], c4);
          }
          const h4 th = *reinterpret_cast<const h4*>(&dpl[0][row][128 + 4 * q]);
          const h4 tl = *reinterpret_cast<const h4*>(&dpl[1][row][128 + 4 * q]);
          c4 = __builtin_amdgcn_mfma_f32_16x16x16f16(tl, bth, c4, 0, 0, 0);
          c4 = __builtin_amdgcn_mfma_f32_16x16x16f16(th, btl, c4, 0, 0, 0);
          c4 = __builtin_amdgcn_mfma_f32_16x16x16f16(th, bth, c4, 0, 0, 0);
          // result row 4q + j of the tile is edge 16 et + 4 q + j, column r is k
#pragma unroll
          for (int j = 0; j < 4; ++j) dacc[et][j] += c4[j] * (einv[16 * et + 4 * q + j] * invss);
        }
      }
      // ---- dS^T: rows = k in [16*wave, 16*wave+16), columns = chunk columns, K = edges; the column tiles
      //      in groups of CTG, each group's results stored before the next group's products
      // result row 4q + j is k = 16 w + 4 q + j (its 1 / scale held by lane 4 q + j), column r is chunk
      // column 16 ct + r = slot 2 ct + r/8, channel c0 + r%8
      float rinv[4];
#pragma unroll
      for (int j = 0; j < 4; ++j) rinv[j] = __shfl(invsh, 4 * q + j, 64);
      constexpr int CTG = 3;
#pragma unroll
      for (int cg = 0; cg < NCT; cg += CTG) {
        f4 sacc[CTG];
#pragma unroll
        for (int u = 0; u < CTG; ++u) sacc[u] = f4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
        for (int s = 0; s < 2; ++s) {
          if (s < nks) {
#pragma unroll
            for (int u = 0; u < CTG; ++u) {
              const int ct = cg + u;
              h8 xh, xl;
#pragma unroll
              for (int j = 0; j < 8; ++j) {
                xh[j] = dpl[0][32 * s + 8 * q + j][16 * ct + r];
                xl[j] = dpl[1][32 * s + 8 * q + j][16 * ct + r];
              }
              sacc[u] = mfma_x3(ah[s], al[s], xh, xl, sacc[u]);
            }
          }
        }
#pragma unroll
        for (int u = 0; u < CTG; ++u) {
          const int ct = cg + u;
          const uint32_t so = (uint32_t)((2 * ct * COLS + c0 * KH) * 4);
          f4 v = sacc[u];
#pragma unroll
          for (int j = 0; j < 4; ++j) v[j] *= rinv[j];
          if (!first) v += buffer_ld4(drs, dvoff, so);
          buffer_st4(drs, dvoff, so, v);
          amax = fmaxf(amax, fmaxf(fmaxf(fabsf(v[0]), fabsf(v[1])), fmaxf(fabsf(v[2]), fabsf(v[3]))));
        }
      }
      if (threadIdx.x < DW) {
        const int col = threadIdx.x;
        // rows >= cnt hold zeros: run to a multiple of 8
        float s4[4] = {0.f, 0.f, 0.f, 0.f};
        const int e8 = (cnt + 7) & ~7;
        for (int e = 0; e < e8; e += 8) {
#pragma unroll
          for (int u = 0; u < 8; ++u)
            s4[u & 3] += ((float)dpl[0][e + u][col] + (float)dpl[1][e + u][col]) * einv[e + u];
        }
        const float sum = (s4[0] + s4[1]) + (s4[2] + s4[3]);
        float* o = dSm + (int64_t)(col / CC) * COLS + 64 * C + c0 + col % CC;
        const float fin = first ? sum : (*o + sum);
        *o = fin;
        amax = fmaxf(amax, fabsf(fin));
      }
      __syncthreads();
    }
#pragma unroll
    for (int et = 0; et < 4; ++et) {
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        const int e = 16 * et + 4 * q + j;
        if (e < cnt) dh[(int64_t)eids[e] * KH + 16 * wave + r] = dacc[et][j];
      }
    }
    if (threadIdx.x < cnt) {
      const int e = threadIdx.x;
#pragma unroll
      for (int k = 0; k < 3; ++k) dn[3 * (int64_t)eids[e] + k] = dnacc[e][k];
    }
    first = false;
    pb += EP;
    if (pb < end) amax = 0.f;   // block-uniform: only the last edge block's stores are final
  } while (pb < end);
  // per-node power of two for the split-fp16 products of node_expand_grad
  for (int off = 32; off > 0; off >>= 1) amax = fmaxf(amax, __shfl_xor(amax, off, 64));
  if (lane == 0) amx[wave] = amax;
  __syncthreads();
  if (threadIdx.x == 0) {
    const float mx = fmaxf(fmaxf(amx[0], amx[1]), fmaxf(amx[2], amx[3]));
    dscale[m] = nparts > 1 ? mx : pow2_scale(mx);
  }
}

// The parts of a split message gradient: dh and dn summed over the parts in order, the dS scale from the
// maximum over the parts.  One float4 of dh, one float of dn or one node per thread.
__global__ __launch_bounds__(256) void msg_grad_combine_kernel(const float* __restrict__ dhp,
                                                               const float* __restrict__ dnp,
                                                               const float* __restrict__ dsp, int nparts,
                                                               int64_t n_edges, int64_t n_nodes,
                                                               float* __restrict__ dh, float* __restrict__ dn,
                                                               float* __restrict__ dscale) {
  const int64_t i = blockIdx.x * (int64_t)blockDim.x + threadIdx.x;
  const int64_t n4 = n_edges * KH / 4, nd = 3 * n_edges;
  if (i < n4) {
    f4 s = ld4(dhp + 4 * i);
    for (int p = 1; p < nparts; ++p) s += ld4(dhp + (int64_t)p * n_edges * KH + 4 * i);
    st4(dh + 4 * i, s);
  } else if (i < n4 + nd) {
    const int64_t j = i - n4;
    float s = dnp[j];
    for (int p = 1; p < nparts; ++p) s += dnp[(int64_t)p * nd + j];
    dn[j] = s;
  } else if (i < n4 + nd + n_nodes) {
    const int64_t m = i - n4 - nd;
    float mx = dsp[m];
    for (int p = 1; p < nparts; ++p) mx = fmaxf(mx, dsp[(int64_t)p * n_nodes + m]);
    dscale[m] = pow2_scale(mx);
  }
}

// ---------------------------------------------------------------- conv1 (species-pair form)
// conv1 operands depend on the source and receiver only through their species
// (A_i = atom_mlp(embedding(Z_i))), so the weight contraction over (a, b) is done once
// per species pair: M[pair][p][k'][c] = sum_{a,b} W[(p,c,a,b),k'] A_s[a] A_t[b]
// for the three live paths p0 (0,0->0), p3 (1,0->1), p5 (2,0->2); k' = 64 is the bias.
// Per edge Q_p[c] = sum_k' M[pair][p][k'][c] h'_e[k'];  m = [Q0, Q1 n, Q2 n n].
// Tables: mf[pair][p][k'][c] (k' = 0..64) and mb[pair][p][c][k'] (rows padded to MB_STRIDE).
// Q is a GEMM per species pair over the edges of that pair (16-edge tiles of the pair-sorted,
// padded edge list `pair_tiles`); the receiver sum then reads Q in receiver order.
constexpr int MB_STRIDE = 68;

// One thread per (receiver species t, live path, channel c, column k), all source species s: the inner
// sum u[a] = sum_b L[(p,c,a,b),k] A_t[b] is formed once and reused for every s (each L entry is read once
// per t instead of once per (s, t)); consecutive threads take consecutive k (coalesced rows of L).
__global__ __launch_bounds__(256) void conv1_pair_table_kernel(const float* __restrict__ L,
                                                               const float* __restrict__ b,
                                                               const float* __restrict__ atab, int n_species,
                                                               int C, float* __restrict__ mf,
                                                               float* __restrict__ mb) {
  const int64_t total = (int64_t)n_species * 3 * 65 * C;
  const int live[3] = {0, 3, 5};
  for (int64_t idx = blockIdx.x * (int64_t)blockDim.x + threadIdx.x; idx < total;
       idx += (int64_t)gridDim.x * blockDim.x) {
    const int k = (int)(idx % 65);
    const int c = (int)((idx / 65) % C);
    const int p3 = (int)((idx / (C * 65)) % 3);
    const int t = (int)(idx / (C * 65 * 3));
    const int p = live[p3];
    float at[8];
#pragma unroll
    for (int bb = 0; bb < 8; ++bb) at[bb] = atab[t * 8 + bb];
    float u[8];
#pragma unroll
    for (int a = 0; a < 8; ++a) {
      float acc = 0.f;
#pragma unroll
      for (int bb = 0; bb < 8; ++bb) {
        const int64_t row = (int64_t)p * C * 64 + (int64_t)c * 64 + a * 8 + bb;
        const float w = (k < 64) ? L[row * KH + k] : b[row];
        acc += w * at[bb];
      }
      u[a] = acc;
    }
    for (int s = 0; s < n_species; ++s) {
      float acc = 0.f;
#pragma unroll
      for (int a = 0; a < 8; ++a) acc += atab[s * 8 + a] * u[a];
      const int64_t pair = (int64_t)s * n_species + t;
      mf[((pair * 3 + p3) * 65 + k) * C + c] = acc;              // [pair][p3][k][c]
      mb[((pair * 3 + p3) * C + c) * MB_STRIDE + k] = acc;        // [pair][p3][c][k]
      if (k == 64) {
#pragma unroll
        for (int z = 65; z < MB_STRIDE; ++z) mb[((pair * 3 + p3) * C + c) * MB_STRIDE + z] = 0.f;
      }
    }
  }
}

// Q[e][p*C + c] = sum_k h[e][k] mb[pair][p][c][k] + mf[pair][p][64][c] for 16-edge tiles of one species
// pair.  pair_tiles = [16*n_tiles padded edge ids (-1: none) | n_tiles pair ids]; a used tile's first entry
// is an edge, the tiles of a pair are consecutive, and unused tiles (first entry -1) come last and are
// skipped.  Transposed product: table rows (p, c) are the
// A operand and the tile's h rows the B operand, so lane (r, q) ends with four consecutive (p, c) columns
// of edge r.  A wave takes C1_TPW consecutive tiles: when they share a pair (all but a few waves per
// pair) each table row block is loaded once for all of them (the table is 48 KB per pair at C 64, which
// one-tile waves re-read from L2 for every 16 edges).
constexpr int C1_TPW = 4;
// Below this many tiles a wave takes one tile (more, shorter waves: at 1,000 atoms there are about 3,300
// tiles, 820 waves of four).
constexpr int64_t C1_SMALL_TILES = 16384;

template <int C, int TPW>
__global__ __launch_bounds__(256) void conv1_pair_gemm_kernel(const float* __restrict__ h,
                                                              const float* __restrict__ mf,
                                                              const float* __restrict__ mb,
                                                              const int32_t* __restrict__ pair_tiles,
                                                              int n_tiles, float* __restrict__ Q) {
  constexpr int NRT = 3 * C / 16;
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int r = lane & 15, q = lane >> 4;
  const int t0 = (blockIdx.x * 4 + wave) * TPW;
  if (t0 >= n_tiles || pair_tiles[16 * (int64_t)t0] < 0) return;   // whole wave (unused tiles are at the end)
  const int nt = min(TPW, n_tiles - t0);
  const int32_t* tpair = pair_tiles + 16 * (int64_t)n_tiles;
  int32_t e[TPW];
  bool used[TPW];
  f4 hb[TPW][4];
  bool same = true;
#pragma unroll
  for (int u = 0; u < TPW; ++u) {
    const int t = t0 + min(u, nt - 1);
    const int32_t first = pair_tiles[16 * t];
    used[u] = u < nt && first >= 0;
    same = same && tpair[t] == tpair[t0];
    const int32_t eu = pair_tiles[16 * t + r];
    e[u] = used[u] ? eu : -1;   // tiles past n_tiles repeat the last one, unused tiles are skipped
    const int32_t eld = (eu >= 0) ? eu : (first >= 0 ? first : pair_tiles[16 * t0]);
#pragma unroll
    for (int t4 = 0; t4 < 4; ++t4) hb[u][t4] = ld4(h + (int64_t)eld * KH + 16 * t4 + 4 * q);
  }
  // Split-fp16 products (16x16x32 f16, K = 64 in two steps; K step ks takes the lane's k = 16 t4 + 4q + j
  // for t4 = 2 ks, 2 ks + 1, the same set in both operands): each edge's h row scaled by a power of two
  // from its own max (the four lanes of a row reduce it), each table row likewise, both undone on the result.
  h8 bh[TPW][2], bl[TPW][2];
  float se[TPW];
#pragma unroll
  for (int u = 0; u < TPW; ++u) {
    float mx = 0.f;
#pragma unroll
    for (int t4 = 0; t4 < 4; ++t4)
      mx = fmaxf(mx, fmaxf(fmaxf(fabsf(hb[u][t4].x), fabsf(hb[u][t4].y)), fmaxf(fabsf(hb[u][t4].z), fabsf(hb[u][t4].w))));
    mx = fmaxf(mx, __shfl_xor(mx, 16, 64));
    mx = fmaxf(mx, __shfl_xor(mx, 32, 64));
    const float sc = pow2_scale(mx);
    se[u] = 1.f / sc;   // a power of two: exact
#pragma unroll
    for (int ks = 0; ks < 2; ++ks) {
      const f4 x0 = hb[u][2 * ks], x1 = hb[u][2 * ks + 1];
      const float v[8] = {x0.x, x0.y, x0.z, x0.w, x1.x, x1.y, x1.z, x1.w};
      split2h(v, sc, bh[u][ks], bl[u][ks]);
    }
  }
  auto tile_rows = [&](int pair, int u0, int u1) {   // tiles u0..u1-1 against the table of `pair`
    const float* mp = mb + (int64_t)pair * 3 * C * MB_STRIDE;
    const float* fp = mf + (int64_t)pair * 3 * 65 * C;
#pragma unroll 3
    for (int rt = 0; rt < NRT; ++rt) {
      f4 a[4];
#pragma unroll
      for (int t4 = 0; t4 < 4; ++t4) a[t4] = ld4(mp + (int64_t)(16 * rt + r) * MB_STRIDE + 16 * t4 + 4 * q);
      const int row = 16 * rt + 4 * q;   // first of the lane's four (p, c) outputs
      const f4 bias = ld4(fp + (row / C) * 65 * C + 64 * C + row % C);
      float mx = 0.f;
#pragma unroll
      for (int t4 = 0; t4 < 4; ++t4)
        mx = fmaxf(mx, fmaxf(fmaxf(fabsf(a[t4].x), fabsf(a[t4].y)), fmaxf(fabsf(a[t4].z), fabsf(a[t4].w))));
      mx = fmaxf(mx, __shfl_xor(mx, 16, 64));
      mx = fmaxf(mx, __shfl_xor(mx, 32, 64));
      const float sr = pow2_scale(mx);   // table row 16 rt + r
      h8 ah[2], al[2];
#pragma unroll
      for (int ks = 0; ks < 2; ++ks) {
        const f4 x0 = a[2 * ks], x1 = a[2 * ks + 1];
        const float v[8] = {x0.x, x0.y, x0.z, x0.w, x1.x, x1.y, x1.z, x1.w};
        split2h(v, sr, ah[ks], al[ks]);
      }
      f4 rinv;   // 1 / scale of the lane's output rows 4q + j
#pragma unroll
      for (int j = 0; j < 4; ++j) rinv[j] = 1.f / __shfl(sr, 4 * q + j, 64);
#pragma unroll
      for (int u = 0; u < TPW; ++u) {
        if (u < u0 || u >= u1) continue;
        f4 acc = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
        for (int ks = 0; ks < 2; ++ks) acc = mfma_x3(ah[ks], al[ks], bh[u][ks], bl[u][ks], acc);
        if (e[u] >= 0) st4(Q + (int64_t)e[u] * 3 * C + row, acc * rinv * se[u] + bias);
      }
    }
  };
  if (same) {   // wave-uniform
    tile_rows(tpair[t0], 0, TPW);
  } else {
#pragma unroll
    for (int u = 0; u < TPW; ++u)
      if (used[u]) tile_rows(tpair[t0 + u], u, u + 1);
  }
}

// out[n] = (1/max(indeg,1)) sum_{e->n} [Q0, Q1 n, Q2 n n]; one wave per receiver, lane = channel (and
// channel + 64 at C 128).
template <int C>
__global__ __launch_bounds__(256) void conv1_receiver_kernel(const float* __restrict__ Q,
                                                             const float* __restrict__ nvec,
                                                             const int32_t* __restrict__ dst_ptr,
                                                             float* __restrict__ out, int64_t n_nodes) {
  constexpr int CPL = C > 64 ? C / 64 : 1;
  const int lane = threadIdx.x & 63;
  const int64_t n = (int64_t)blockIdx.x * 4 + (threadIdx.x >> 6);
  if (n >= n_nodes) return;
  const int c0 = C < 64 ? (lane & (C - 1)) : lane;
  float o[CPL][NCOMP];
#pragma unroll
  for (int k = 0; k < CPL; ++k)
#pragma unroll
    for (int i = 0; i < NCOMP; ++i) o[k][i] = 0.f;
  const int beg = dst_ptr[n], end = dst_ptr[n + 1];
  for (int e = beg; e < end; ++e) {
    const float nn[3] = {nvec[3 * (int64_t)e], nvec[3 * (int64_t)e + 1], nvec[3 * (int64_t)e + 2]};
#pragma unroll
    for (int k = 0; k < CPL; ++k) {
      const float* qr = Q + (int64_t)e * 3 * C + c0 + 64 * k;
      const float q0 = qr[0], q1 = qr[C], q2 = qr[2 * C];
      o[k][0] += q0;
#pragma unroll
      for (int i = 0; i < 3; ++i) {
        o[k][1 + i] += q1 * nn[i];
        const float q2n = q2 * nn[i];
#pragma unroll
        for (int j = 0; j < 3; ++j) o[k][4 + 3 * i + j] += q2n * nn[j];
      }
    }
  }
  if (lane < C) {
    const float scale = 1.f / (float)max(end - beg, 1);
#pragma unroll
    for (int k = 0; k < CPL; ++k) {
      float* orow = out + n * NCOMP * C + c0 + 64 * k;
#pragma unroll
      for (int i = 0; i < NCOMP; ++i) orow[i * C] = o[k][i] * scale;
    }
  }
}

// Receiver side of the backward: dQ[e] = (g0, g1.n, n.g2.n) with g = G[n]/max(indeg,1), and
// dn_e[k] = sum_c g1[k] Q1 + Q2 ((g2 n)[k] + (g2^T n)[k]).  One wave per receiver, lane = channel (and
// channel + 64 at C 128).
template <int C>
__global__ __launch_bounds__(256) void conv1_receiver_grad_kernel(const float* __restrict__ G,
                                                                  const float* __restrict__ nvec,
                                                                  const float* __restrict__ Q,
                                                                  const int32_t* __restrict__ dst_ptr,
                                                                  float* __restrict__ dQ,
                                                                  float* __restrict__ dn, int64_t n_nodes) {
  constexpr int CPL = C > 64 ? C / 64 : 1;
  const int lane = threadIdx.x & 63;
  const int64_t n = (int64_t)blockIdx.x * 4 + (threadIdx.x >> 6);
  if (n >= n_nodes) return;   // whole wave
  const int c0 = C < 64 ? (lane & (C - 1)) : lane;
  const bool act = lane < C;
  const int beg = dst_ptr[n], end = dst_ptr[n + 1];
  const float scale = 1.f / (float)max(end - beg, 1);
  float g[CPL][NCOMP];
#pragma unroll
  for (int k = 0; k < CPL; ++k)
#pragma unroll
    for (int i = 0; i < NCOMP; ++i) g[k][i] = act ? G[(n * NCOMP + i) * C + c0 + 64 * k] * scale : 0.f;
  for (int e = beg; e < end; ++e) {
    const float nn[3] = {nvec[3 * (int64_t)e], nvec[3 * (int64_t)e + 1], nvec[3 * (int64_t)e + 2]};
    float t[3] = {0.f, 0.f, 0.f};
#pragma unroll
    for (int k = 0; k < CPL; ++k) {
      const float* qr = Q + (int64_t)e * 3 * C + c0 + 64 * k;
      const float q1 = qr[C], q2 = qr[2 * C];
      float d1 = 0.f, d2 = 0.f;
#pragma unroll
      for (int kk = 0; kk < 3; ++kk) {
        float row = 0.f, colv = 0.f;
#pragma unroll
        for (int j = 0; j < 3; ++j) {
          row += g[k][4 + 3 * kk + j] * nn[j];
          colv += g[k][4 + 3 * j + kk] * nn[j];
        }
        d1 += g[k][1 + kk] * nn[kk];
        d2 += row * nn[kk];
        t[kk] += act ? g[k][1 + kk] * q1 + q2 * (row + colv) : 0.f;
      }
      if (act) {
        float* dq = dQ + (int64_t)e * 3 * C + c0 + 64 * k;
        dq[0] = g[k][0];
        dq[C] = d1;
        dq[2 * C] = d2;
      }
    }
    const float t0 = wave_sum(t[0]), t1 = wave_sum(t[1]), t2 = wave_sum(t[2]);
    if (lane == 0) {
      dn[3 * (int64_t)e] = t0;
      dn[3 * (int64_t)e + 1] = t1;
      dn[3 * (int64_t)e + 2] = t2;
    }
  }
}

// dh[e][k] = sum_{p,c} dQ[e][p][c] mf[pair][p][k][c] for C1_TPW consecutive 16-edge tiles per wave
// (one table load for all of them when they share a pair, as in the forward); transposed product
// (table rows k are the A operand), lane (r, q) ends with four consecutive k of edge r per k tile.
template <int C, int TPW>
__global__ __launch_bounds__(256) void conv1_pair_gemm_grad_kernel(const float* __restrict__ dQ,
                                                                   const float* __restrict__ mf,
                                                                   const int32_t* __restrict__ pair_tiles,
                                                                   int n_tiles, float* __restrict__ dh) {
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int r = lane & 15, q = lane >> 4;
  const int t0 = (blockIdx.x * 4 + wave) * TPW;
  if (t0 >= n_tiles || pair_tiles[16 * (int64_t)t0] < 0) return;   // whole wave (unused tiles are at the end)
  const int nt = min(TPW, n_tiles - t0);
  const int32_t* tpair = pair_tiles + 16 * (int64_t)n_tiles;
  int32_t e[TPW];
  bool used[TPW];
  const float* dq[TPW];
  bool same = true;
#pragma unroll
  for (int u = 0; u < TPW; ++u) {
    const int t = t0 + min(u, nt - 1);
    const int32_t first = pair_tiles[16 * t];
    used[u] = u < nt && first >= 0;
    same = same && tpair[t] == tpair[t0];
    const int32_t eu = pair_tiles[16 * t + r];
    e[u] = used[u] ? eu : -1;   // tiles past n_tiles repeat the last one, unused tiles are skipped
    const int32_t eld = (eu >= 0) ? eu : (first >= 0 ? first : pair_tiles[16 * t0]);
    dq[u] = dQ + (int64_t)eld * 3 * C + 4 * q;
  }
  auto tile_rows = [&](int pair, int u0, int u1) {   // tiles u0..u1-1 against the table of `pair`
    const float* fp = mf + (int64_t)pair * 3 * 65 * C;
    f4 acc[TPW][4];
#pragma unroll
    for (int u = 0; u < TPW; ++u)
#pragma unroll
      for (int kt = 0; kt < 4; ++kt) acc[u][kt] = f4{0.f, 0.f, 0.f, 0.f};
#pragma unroll 2
    for (int kc = 0; kc < 3 * C / 16; ++kc) {   // K chunk: path p = kc / (C/16), channels c0..c0+15
      const int p = kc / (C / 16), c0 = 16 * (kc % (C / 16));
      f4 a[4];
#pragma unroll
      for (int kt = 0; kt < 4; ++kt) a[kt] = ld4(fp + (int64_t)(p * 65 + 16 * kt + r) * C + c0 + 4 * q);
#pragma unroll
      for (int u = 0; u < TPW; ++u) {
        if (u < u0 || u >= u1) continue;
        const f4 b = ld4(dq[u] + p * C + c0);
#pragma unroll
        for (int kt = 0; kt < 4; ++kt) acc[u][kt] = mfma_k16(a[kt], b, acc[u][kt]);
      }
    }
#pragma unroll
    for (int u = 0; u < TPW; ++u) {
      if (u < u0 || u >= u1 || e[u] < 0) continue;
#pragma unroll
      for (int kt = 0; kt < 4; ++kt) st4(dh + (int64_t)e[u] * KH + 16 * kt + 4 * q, acc[u][kt]);
    }
  };
  if (same) {   // wave-uniform
    tile_rows(tpair[t0], 0, TPW);
  } else {
#pragma unroll
    for (int u = 0; u < TPW; ++u)
      if (used[u]) tile_rows(tpair[t0 + u], u, u + 1);
  }
}

// ---------------------------------------------------------------- host launchers
template <int C, bool BF16>
int conv_forward_impl(int64_t N, int64_t E, const int32_t* dst_ptr, const int32_t* src_ptr,
                      const int32_t* src_perm, const float* x, const float* h, const float* nvec,
                      const float* bk1, float scale, float* S, float* P, float* out,
                      const int32_t* node_order, hipStream_t st) {
  if (N == 0) return 0;
  {
    PathTiles tiles;
    tiles.off[0] = 0;
    for (int p = 0; p < 6; ++p)
      tiles.off[p + 1] = tiles.off[p] + (int)((N * kNumI[kPathL1H[p]] + NE_ROWS - 1) / NE_ROWS);
    constexpr int ncg = ((65 * C) / 80 + NE_TPB - 1) / NE_TPB;
    LaunchTimer tm("node_expand", st);
    const float* wplane = BF16 ? bk1 + sparse_weight_floats(C) : bk1;
    node_expand_kernel<C, BF16><<<(unsigned)(tiles.off[6] * ncg), 256, 0, st>>>(
        x, reinterpret_cast<const _Float16*>(wplane), bk1 + sparse_weight_floats(C) - SW_TAIL, S, N, tiles);
  }
  if (check_launch("sparse node_expand")) return 2;
  {
    LaunchTimer tm("edge_message", st);
    edge_message_kernel<C, BF16><<<dim3(xcd_grid(N), msg_parts(N)), 192, 0, st>>>(h, S, src_ptr, src_perm, P, N,
                                                                              node_order);
  }
  if (check_launch("sparse edge_message")) return 2;
  {
    LaunchTimer tm("receiver_sum", st);
    receiver_sum_kernel<C><<<(unsigned)((N + 3) / 4), 256, 0, st>>>(P, nvec, nullptr, dst_ptr, scale, out, N);
  }
  return check_launch("sparse receiver_sum") ? 2 : 0;
}

// DIR: the gradients of <G, out'> for the direction derivative out' along udir (training double backward).
template <int C, bool BF16, bool DIR = false>
int conv_backward_impl(int64_t N, int64_t E, const int32_t* dst_ptr, const int32_t* src_ptr,
                       const int32_t* src_perm, const int32_t* edge_dst, const float* G,
                       const float* h, const float* nvec, const float* bk6, const float* S,
                       const float* P, float scale, float* dS, float* dx, float* dh, float* dn,
                       const int32_t* node_order, hipStream_t st, const float* udir = nullptr) {
  if (N == 0) return 0;
  // workspace tail (ks x 18 x N x C floats, ks = neg_ksplit(N) >= 2): first the chunk-major receiver
  // gradient (13 x N x C), later the partial input gradients of node_expand_grad; then N per-node
  // scales of dS
  const int ks = neg_ksplit(N);
  float* tail = dS + N * s_node_stride(C);
  float* dscale = tail + (int64_t)ks * NSLOT * N * C;
  grad_chunk_major_kernel<C><<<(unsigned)((N * NCOMP * (C / 4) + 255) / 256), 256, 0, st>>>(G, tail, N);
  if constexpr (!DIR && !BF16) {
    // the fp32 message gradient: both products split-fp16, scaled by the receiver gradients' bound
    float* gmax = tail + (int64_t)NCOMP * N * C;   // after the chunk-major gradient, inside the tail
    grad_absmax_kernel<C><<<(unsigned)((N + 3) / 4), 256, 0, st>>>(G, gmax, N);
    LaunchTimer tm("edge_message_grad", st);
    const int np = msg_parts(N);
    float* dhp = dS + msg_parts_offset(N, C);   // the parts of a split message gradient
    float* dnp = dhp + (int64_t)np * E * KH;
    float* dsp = dnp + (int64_t)np * E * 3;
    edge_message_grad_h16_kernel<C><<<dim3(xcd_grid(N), np), 256, 0, st>>>(
        tail, gmax, nvec, h, S, P, src_ptr, src_perm, edge_dst, scale, np > 1 ? dhp : dh, dS, np > 1 ? dnp : dn,
        np > 1 ? dsp : dscale, N, node_order, E);
    if (np > 1) {
      if (check_launch("sparse edge_message_grad")) return 2;
      msg_grad_combine_kernel<<<(unsigned)((E * KH / 4 + 3 * E + N + 255) / 256), 256, 0, st>>>(
          dhp, dnp, dsp, np, E, N, dh, dn, dscale);
    }
  } else {
    LaunchTimer tm(DIR ? "edge_message_grad_direction" : "edge_message_grad", st);
    edge_message_grad_kernel<C, DIR, BF16><<<xcd_grid(N), 256, 0, st>>>(tail, nvec, udir, h, S, P, src_ptr, src_perm,
                                                              edge_dst, scale, dh, dS, dn, dscale, N, node_order);
  }
  if (check_launch("sparse edge_message_grad")) return 2;
  {
    PathTiles tiles;
    tiles.off[0] = 0;
    for (int p = 0; p < 6; ++p)
      tiles.off[p + 1] = tiles.off[p] + (int)((N * kNumI[kPathL1H[p]] + NEG_ROWS - 1) / NEG_ROWS);
    float* dxp = dS + N * s_node_stride(C);   // workspace tail: ks x 18 x N x C partial sums (Gt is dead)
    {
      LaunchTimer tm("node_expand_grad", st);
      const float* wplane = BF16 ? bk6 + sparse_weight_floats(C) : bk6;
      node_expand_grad_kernel<C, BF16><<<(unsigned)(ks * tiles.off[6]), 256, 0, st>>>(
          dS, dscale, reinterpret_cast<const _Float16*>(wplane), bk6 + sparse_weight_floats(C) - SW_TAIL, dxp, N,
          tiles, ks);
    }
    if (check_launch("sparse node_expand_grad")) return 2;
    node_expand_grad_combine_kernel<C><<<(unsigned)((N * NCOMP * (C / 4) + 255) / 256), 256, 0, st>>>(dxp, dx, N,
                                                                                                     ks);
  }
  return check_launch("sparse node_expand_grad") ? 2 : 0;
}

}  // namespace sparse
}  // namespace fsc

// ===================================================================== C ABI
using namespace fsc;
using namespace fsc::sparse;

static bool sparse_channels_ok(int32_t c) { return c == 32 || c == 64 || c == 128; }

extern "C" {

int fsc_sparse_conv_workspace(int64_t n_nodes, int64_t n_edges, int32_t channels,
                              int64_t* s_floats, int64_t* p_floats) {
  FSC_CHECK_ARG(n_nodes >= 0 && n_edges >= 0, "fsc_sparse_conv_workspace: negative size");
  FSC_CHECK_ARG(sparse_channels_ok(channels), "fsc_sparse_conv_workspace: channels must be 32, 64 or 128");
  FSC_CHECK_ARG(s_floats && p_floats, "fsc_sparse_conv_workspace: null output");
  // the tail (ks x 18 x N x C + N, ks = neg_ksplit(N)) holds the partial input gradients and per-node
  // scales of the backward; on small graphs (msg_parts) the parts of the split message gradient follow
  *s_floats = msg_parts_floats(n_nodes, n_edges) > 0
                  ? msg_parts_offset(n_nodes, channels) + msg_parts_floats(n_nodes, n_edges)
                  : n_nodes * s_node_stride(channels) + (int64_t)neg_ksplit(n_nodes) * NSLOT * n_nodes * channels + n_nodes;
  *p_floats = n_edges * (int64_t)NSLOT * channels;
  return 0;
}

int fsc_sparse_conv_prepare_weights(const float* w_last, const float* b_last, int32_t channels,
                                    float* bk1, float* bk6, hipStream_t stream) {
  FSC_CHECK_ARG(sparse_channels_ok(channels), "fsc_sparse_conv_prepare_weights: channels must be 32, 64 or 128");
  FSC_CHECK_ARG(w_last && b_last && bk1 && bk6, "fsc_sparse_conv_prepare_weights: null pointer");
  const int64_t C = channels;
  weight_absmax_kernel<<<SWMAX_BLOCKS, 256, 0, stream>>>(w_last, 6 * C * C * KH, b_last, 6 * C * C,
                                                         bk1 + sparse_weight_floats(channels) - SW_TAIL + 256);
  if (check_launch("sparse weight maximum")) return 2;
  prep_weights_kernel<<<(unsigned)(6 * C), 256, 0, stream>>>(w_last, b_last, bk1, bk6, channels);
  return check_launch("sparse prepare_weights") ? 2 : 0;
}

int fsc_sparse_conv_forward(int64_t n_nodes, int64_t n_edges, int32_t channels,
                            const int32_t* dst_ptr, const int32_t* src_ptr, const int32_t* src_perm,
                            const float* x, const float* h, const float* n, const float* bk1,
                            float inv_norm, float* s_ws, float* p_ws, float* out, int32_t precision,
                            const int32_t* node_order, hipStream_t stream) {
  FSC_CHECK_ARG(n_nodes >= 0 && n_edges >= 0, "fsc_sparse_conv_forward: negative size");
  FSC_CHECK_ARG(precision == 0 || precision == 1, "fsc_sparse_conv_forward: precision must be 0 (fp32) or 1 (bf16)");
  FSC_CHECK_ARG(n_nodes < (1LL << 31) && n_edges < (1LL << 31), "fsc_sparse_conv_forward: size exceeds int32 indexing");
  FSC_CHECK_ARG(dst_ptr && src_ptr && x && bk1 && s_ws && out, "fsc_sparse_conv_forward: null pointer");
  FSC_CHECK_ARG(n_edges == 0 || (src_perm && h && n && p_ws), "fsc_sparse_conv_forward: null edge pointer");
  if (channels == 128)
    return (precision ? conv_forward_impl<128, true> : conv_forward_impl<128, false>)(
        n_nodes, n_edges, dst_ptr, src_ptr, src_perm, x, h, n, bk1, inv_norm, s_ws, p_ws, out, node_order, stream);
  if (channels == 64)
    return (precision ? conv_forward_impl<64, true> : conv_forward_impl<64, false>)(
        n_nodes, n_edges, dst_ptr, src_ptr, src_perm, x, h, n, bk1, inv_norm, s_ws, p_ws, out, node_order, stream);
  if (channels == 32)
    return (precision ? conv_forward_impl<32, true> : conv_forward_impl<32, false>)(
        n_nodes, n_edges, dst_ptr, src_ptr, src_perm, x, h, n, bk1, inv_norm, s_ws, p_ws, out, node_order, stream);
  set_error("fsc_sparse_conv_forward: channels must be 32, 64 or 128");
  return 1;
}

int fsc_sparse_conv_direction(int64_t n_nodes, int64_t n_edges, int32_t channels, const int32_t* dst_ptr,
                              const float* p_ws, const float* n, const float* u, float inv_norm, float* out,
                              hipStream_t stream) {
  FSC_CHECK_ARG(n_nodes >= 0 && n_edges >= 0, "fsc_sparse_conv_direction: negative size");
  FSC_CHECK_ARG(n_nodes < (1LL << 31) && n_edges < (1LL << 31), "fsc_sparse_conv_direction: size exceeds int32 indexing");
  FSC_CHECK_ARG(dst_ptr && out, "fsc_sparse_conv_direction: null pointer");
  FSC_CHECK_ARG(n_edges == 0 || (p_ws && n && u), "fsc_sparse_conv_direction: null edge pointer");
  FSC_CHECK_ARG(sparse_channels_ok(channels), "fsc_sparse_conv_direction: channels must be 32, 64 or 128");
  if (n_nodes == 0) return 0;
  const unsigned grid = (unsigned)((n_nodes + 3) / 4);
  if (channels == 128)
    receiver_sum_kernel<128, true><<<grid, 256, 0, stream>>>(p_ws, n, u, dst_ptr, inv_norm, out, n_nodes);
  else if (channels == 64)
    receiver_sum_kernel<64, true><<<grid, 256, 0, stream>>>(p_ws, n, u, dst_ptr, inv_norm, out, n_nodes);
  else
    receiver_sum_kernel<32, true><<<grid, 256, 0, stream>>>(p_ws, n, u, dst_ptr, inv_norm, out, n_nodes);
  return check_launch("sparse direction derivative") ? 2 : 0;
}

int fsc_sparse_conv_direction_backward(int64_t n_nodes, int64_t n_edges, int32_t channels,
                                       const int32_t* dst_ptr, const int32_t* src_ptr, const int32_t* src_perm,
                                       const int32_t* edge_dst, const float* grad_out, const float* h,
                                       const float* n, const float* u, const float* bk6, const float* s_ws,
                                       const float* p_ws, float inv_norm, float* ds_ws, float* grad_x,
                                       float* grad_h, float* grad_n, int32_t precision, const int32_t* node_order,
                                       hipStream_t stream) {
  FSC_CHECK_ARG(n_nodes >= 0 && n_edges >= 0, "fsc_sparse_conv_direction_backward: negative size");
  FSC_CHECK_ARG(precision == 0 || precision == 1, "fsc_sparse_conv_direction_backward: precision must be 0 or 1");
  FSC_CHECK_ARG(n_nodes < (1LL << 31) && n_edges < (1LL << 31),
                "fsc_sparse_conv_direction_backward: size exceeds int32 indexing");
  FSC_CHECK_ARG(dst_ptr && src_ptr && grad_out && bk6 && s_ws && ds_ws && grad_x,
                "fsc_sparse_conv_direction_backward: null pointer");
  FSC_CHECK_ARG(n_edges == 0 || (src_perm && edge_dst && h && n && u && p_ws && grad_h && grad_n),
                "fsc_sparse_conv_direction_backward: null edge pointer");
  if (channels == 128)
    return (precision ? conv_backward_impl<128, true, true> : conv_backward_impl<128, false, true>)(
        n_nodes, n_edges, dst_ptr, src_ptr, src_perm, edge_dst, grad_out, h, n, bk6, s_ws, p_ws, inv_norm, ds_ws,
        grad_x, grad_h, grad_n, node_order, stream, u);
  if (channels == 64)
    return (precision ? conv_backward_impl<64, true, true> : conv_backward_impl<64, false, true>)(
        n_nodes, n_edges, dst_ptr, src_ptr, src_perm, edge_dst, grad_out, h, n, bk6, s_ws, p_ws, inv_norm, ds_ws,
        grad_x, grad_h, grad_n, node_order, stream, u);
  if (channels == 32)
    return (precision ? conv_backward_impl<32, true, true> : conv_backward_impl<32, false, true>)(
        n_nodes, n_edges, dst_ptr, src_ptr, src_perm, edge_dst, grad_out, h, n, bk6, s_ws, p_ws, inv_norm, ds_ws,
        grad_x, grad_h, grad_n, node_order, stream, u);
  set_error("fsc_sparse_conv_direction_backward: channels must be 32, 64 or 128");
  return 1;
}

int fsc_sparse_conv_backward(int64_t n_nodes, int64_t n_edges, int32_t channels,
                             const int32_t* dst_ptr, const int32_t* src_ptr, const int32_t* src_perm,
                             const int32_t* edge_dst, const float* grad_out, const float* h,
                             const float* n, const float* bk6, const float* s_ws, const float* p_ws,
                             float inv_norm, float* ds_ws, float* grad_x, float* grad_h,
                             float* grad_n, int32_t precision, const int32_t* node_order, hipStream_t stream) {
  FSC_CHECK_ARG(n_nodes >= 0 && n_edges >= 0, "fsc_sparse_conv_backward: negative size");
  FSC_CHECK_ARG(precision == 0 || precision == 1, "fsc_sparse_conv_backward: precision must be 0 (fp32) or 1 (bf16)");
  FSC_CHECK_ARG(n_nodes < (1LL << 31) && n_edges < (1LL << 31), "fsc_sparse_conv_backward: size exceeds int32 indexing");
  FSC_CHECK_ARG(dst_ptr && src_ptr && grad_out && bk6 && s_ws && ds_ws && grad_x,
                "fsc_sparse_conv_backward: null pointer");
  FSC_CHECK_ARG(n_edges == 0 || (src_perm && edge_dst && h && n && p_ws && grad_h && grad_n),
                "fsc_sparse_conv_backward: null edge pointer");
  if (channels == 128)
    return (precision ? conv_backward_impl<128, true> : conv_backward_impl<128, false>)(
        n_nodes, n_edges, dst_ptr, src_ptr, src_perm, edge_dst, grad_out, h, n, bk6, s_ws, p_ws, inv_norm, ds_ws,
        grad_x, grad_h, grad_n, node_order, stream, nullptr);
  if (channels == 64)
    return (precision ? conv_backward_impl<64, true> : conv_backward_impl<64, false>)(
        n_nodes, n_edges, dst_ptr, src_ptr, src_perm, edge_dst, grad_out, h, n, bk6, s_ws, p_ws, inv_norm, ds_ws,
        grad_x, grad_h, grad_n, node_order, stream, nullptr);
  if (channels == 32)
    return (precision ? conv_backward_impl<32, true> : conv_backward_impl<32, false>)(
        n_nodes, n_edges, dst_ptr, src_ptr, src_perm, edge_dst, grad_out, h, n, bk6, s_ws, p_ws, inv_norm, ds_ws,
        grad_x, grad_h, grad_n, node_order, stream, nullptr);
  set_error("fsc_sparse_conv_backward: channels must be 32, 64 or 128");
  return 1;
}

int fsc_sparse_conv1_pair_table(const float* w_last, const float* b_last, const float* atom_table,
                                int32_t n_species, int32_t channels, float* mf, float* mb,
                                hipStream_t stream) {
  FSC_CHECK_ARG(sparse_channels_ok(channels), "fsc_sparse_conv1_pair_table: channels must be 32, 64 or 128");
  FSC_CHECK_ARG(n_species >= 1 && n_species <= 128, "fsc_sparse_conv1_pair_table: n_species out of range");
  FSC_CHECK_ARG(w_last && b_last && atom_table && mf && mb, "fsc_sparse_conv1_pair_table: null pointer");
  const int64_t work = (int64_t)n_species * 3 * 65 * channels;
  conv1_pair_table_kernel<<<(unsigned)std::min<int64_t>((work + 255) / 256, 1024), 256, 0, stream>>>(
      w_last, b_last, atom_table, n_species, channels, mf, mb);
  return check_launch("sparse conv1_pair_table") ? 2 : 0;
}

int fsc_sparse_conv1_forward(int64_t n_nodes, int64_t n_edges, int32_t channels, const int32_t* dst_ptr,
                             int64_t n_tiles, const int32_t* pair_tiles, const float* h, const float* n,
                             const float* mf, const float* mb, float* q_ws, float* out, hipStream_t stream) {
  FSC_CHECK_ARG(n_nodes >= 0 && n_edges >= 0 && n_nodes < (1LL << 31) && n_edges < (1LL << 31),
                "fsc_sparse_conv1_forward: bad size");
  FSC_CHECK_ARG(n_tiles >= 0 && n_tiles < (1LL << 27) && n_tiles * 16 >= n_edges,
                "fsc_sparse_conv1_forward: pair tiles do not cover the edges");
  FSC_CHECK_ARG(sparse_channels_ok(channels), "fsc_sparse_conv1_forward: channels must be 32, 64 or 128");
  FSC_CHECK_ARG(dst_ptr && mf && mb && out, "fsc_sparse_conv1_forward: null pointer");
  FSC_CHECK_ARG(n_edges == 0 || (pair_tiles && h && n && q_ws), "fsc_sparse_conv1_forward: null edge pointer");
  if (n_nodes == 0) return 0;
  LaunchTimer tm("conv1_forward", stream);
  const int tpw = n_tiles >= C1_SMALL_TILES ? C1_TPW : 1;
  const unsigned tgrid = (unsigned)((n_tiles + 4 * tpw - 1) / (4 * tpw)), ngrid = (unsigned)((n_nodes + 3) / 4);
#define FSC_C1F(CC)                                                                                       \
  if (n_tiles) {                                                                                          \
    if (tpw == 1)                                                                                         \
      conv1_pair_gemm_kernel<CC, 1><<<tgrid, 256, 0, stream>>>(h, mf, mb, pair_tiles, (int)n_tiles, q_ws); \
    else                                                                                                  \
      conv1_pair_gemm_kernel<CC, C1_TPW><<<tgrid, 256, 0, stream>>>(h, mf, mb, pair_tiles, (int)n_tiles, q_ws); \
  }                                                                                                       \
  conv1_receiver_kernel<CC><<<ngrid, 256, 0, stream>>>(q_ws, n, dst_ptr, out, n_nodes);
  if (channels == 128) {
    FSC_C1F(128)
  } else if (channels == 64) {
    FSC_C1F(64)
  } else {
    FSC_C1F(32)
  }
#undef FSC_C1F
  return check_launch("sparse conv1_forward") ? 2 : 0;
}

int fsc_sparse_conv1_backward(int64_t n_nodes, int64_t n_edges, int32_t channels, const int32_t* dst_ptr,
                              int64_t n_tiles, const int32_t* pair_tiles, const float* grad_out, const float* n,
                              const float* mf, const float* q_ws, float* dq_ws, float* grad_h, float* grad_n,
                              hipStream_t stream) {
  FSC_CHECK_ARG(n_nodes >= 0 && n_edges >= 0 && n_nodes < (1LL << 31) && n_edges < (1LL << 31),
                "fsc_sparse_conv1_backward: bad size");
  FSC_CHECK_ARG(n_tiles >= 0 && n_tiles < (1LL << 27) && n_tiles * 16 >= n_edges,
                "fsc_sparse_conv1_backward: pair tiles do not cover the edges");
  FSC_CHECK_ARG(sparse_channels_ok(channels), "fsc_sparse_conv1_backward: channels must be 32, 64 or 128");
  FSC_CHECK_ARG(dst_ptr && grad_out && mf, "fsc_sparse_conv1_backward: null pointer");
  FSC_CHECK_ARG(n_edges == 0 || (pair_tiles && n && q_ws && dq_ws && grad_h && grad_n),
                "fsc_sparse_conv1_backward: null edge pointer");
  if (n_nodes == 0) return 0;
  LaunchTimer tm("conv1_backward", stream);
  const int tpw = n_tiles >= C1_SMALL_TILES ? C1_TPW : 1;
  const unsigned tgrid = (unsigned)((n_tiles + 4 * tpw - 1) / (4 * tpw)), ngrid = (unsigned)((n_nodes + 3) / 4);
#define FSC_C1B(CC)                                                                                          \
  conv1_receiver_grad_kernel<CC><<<ngrid, 256, 0, stream>>>(grad_out, n, q_ws, dst_ptr, dq_ws, grad_n, n_nodes); \
  if (n_tiles) {                                                                                             \
    if (tpw == 1)                                                                                            \
      conv1_pair_gemm_grad_kernel<CC, 1><<<tgrid, 256, 0, stream>>>(dq_ws, mf, pair_tiles, (int)n_tiles, grad_h); \
    else                                                                                                     \
      conv1_pair_gemm_grad_kernel<CC, C1_TPW><<<tgrid, 256, 0, stream>>>(dq_ws, mf, pair_tiles, (int)n_tiles, grad_h); \
  }
  if (channels == 128) {
    FSC_C1B(128)
  } else if (channels == 64) {
    FSC_C1B(64)
  } else {
    FSC_C1B(32)
  }
#undef FSC_C1B
  return check_launch("sparse conv1_backward") ? 2 : 0;
}

}  // extern "C"
