// The per-edge ("bucketed") ICTD tensor product of the reference's native extension on gfx950: the
// operations of molecular_force_field._C_ictd_tp (csrc/ictd_tp.cpp:498-522, CUDA half
// csrc/ictd_tp_cuda.cu) for the arguments its CUDA path takes (fp32 here, mul_in2 == 1):
//
//   project:  y[b][p][k][i] = sum_{m,n} a[b][i][m] v[b][n] U[m*m2 + n][p*K + k]
//   mix:      out[b][o][k]  = sum_p g[b][p] sum_i y[b][p][k][i] W[p][o][i]
//
// and the transposes of both with respect to every argument (the einsum semantics of
// models/ictd_irreps_cuda.py:169-288).  B is the batch (edges), I = mul_in1, O = mul_out, K = kdim,
// PK = P*K.  Layouts: a [B][I][m1], v [B][1][m2], U [m1*m2][PK], y [B][P][K][I], W [P][O][I],
// g [B][P], out [B][O][K].
//
// The projections contract over at most 9 x 9 components and run on the VALU, one wave per batch
// element with the factor ub[m][pk] = sum_n v[n] U[m*m2+n][pk] formed once per element in LDS.  The
// channel mixes are GEMMs over (b, k) rows and run on v_mfma_f32_16x16x4_f32.  Every kernel writes or,
// with `acc`, adds to its output, so the double-backward sums of the reference (csrc/ictd_tp_cuda.cu:528-533,
// 796-802) are the same kernels run two or three times.  Sums over the batch (the gradients of U and W)
// go through per-block partial sums and a reduction in a fixed order: results are deterministic.

#include <algorithm>

#include "common.h"
#include "fsctep.h"

namespace fsc {
namespace bucket {

constexpr int MAXM = 9;     // 2l + 1 for l <= 4
constexpr int MAXPK = 64;   // P * K handled by one lane each in the U/b transposes
constexpr int UREG = 32;    // per-lane U-gradient entries: m1 * m2 * PK <= 64 * UREG
constexpr int IC = 32;      // channels per staging chunk of the U/b transposes

struct Dims {
  int64_t B;
  int I, m1, m2, P, K, O;
};

// Factor of the projection for element b, padded to MAXM rows: ub[m][pk] = sum_n v[b][n] U[m*m2+n][pk] for
// m < m1 and zero for m1 <= m < MAXM (us: U in LDS), so that the contractions below run over MAXM rows with
// no branch (a branch per row would make every product wait for all outstanding stores).
__device__ __forceinline__ void form_ub(const Dims& d, int PK, const float* __restrict__ v, const float* us, float* ub,
                                        int64_t b, bool ok, int lane) {
  float vb[MAXM];   // v[b][n], zero past m2: all loads issued together (one wait)
#pragma unroll
  for (int n = 0; n < MAXM; ++n) {
    const float x = v[(ok ? b : 0) * d.m2 + min(n, d.m2 - 1)];
    vb[n] = (ok && n < d.m2) ? x : 0.f;
  }
  for (int idx = lane; idx < MAXM * PK; idx += 64) {
    const int m = idx / PK, pk = idx - m * PK;
    const int mc = min(m, d.m1 - 1);
    float s = 0.f;
#pragma unroll
    for (int n = 0; n < MAXM; ++n) s += vb[n] * us[(mc * d.m2 + min(n, d.m2 - 1)) * PK + pk];
    ub[idx] = m < d.m1 ? s : 0.f;
  }
}

__device__ __forceinline__ void put(float* p, float v, int acc) { *p = acc ? *p + v : v; }

// TA false: y[b][pk][i] (+)= sum_m a[b][i][m] ub[m][pk]        (src = a, dst = y)
// TA true:  grad_a[b][i][m] (+)= sum_pk gy[b][pk][i] ub[m][pk]  (src = gy, dst = grad_a)
// Four waves per block, one batch element per wave per step; U staged in LDS once per block.  Lane i holds
// its a row (MAXM values, zero past m1; the loads clamp their index) or its gy values eight at a time.
template <bool TA, bool ACC>
__global__ __launch_bounds__(256) void project_kernel(Dims d, const float* __restrict__ src, const float* __restrict__ v,
                                                      const float* __restrict__ U, float* __restrict__ dst) {
  extern __shared__ float sm[];
  const int PK = d.P * d.K, MN = d.m1 * d.m2;
  const int lane = threadIdx.x & 63, wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  float* us = sm;
  float* ub = sm + MN * PK + wave * MAXM * PK;
  for (int idx = threadIdx.x; idx < MN * PK; idx += 256) us[idx] = U[idx];
  __syncthreads();
  // the trip count is the same for every wave of the block (barriers inside)
  for (int64_t b0 = (int64_t)blockIdx.x * 4; b0 < d.B; b0 += (int64_t)gridDim.x * 4) {
    const int64_t b = b0 + wave;
    const bool ok = b < d.B;
    form_ub(d, PK, v, us, ub, b, ok, lane);
    __syncthreads();
    if (ok) {   // wave-uniform
      for (int i = lane; i < d.I; i += 64) {
        if constexpr (!TA) {
          const float* ar = src + (b * d.I + i) * d.m1;
          float av[MAXM];
#pragma unroll
          for (int m = 0; m < MAXM; ++m) {
            const float x = ar[min(m, d.m1 - 1)];
            av[m] = m < d.m1 ? x : 0.f;
          }
          float* yo = dst + b * PK * d.I + i;
          for (int pk = 0; pk < PK; ++pk) {
            float s = 0.f;
#pragma unroll
            for (int m = 0; m < MAXM; ++m) s += av[m] * ub[m * PK + pk];
            if constexpr (ACC) s += yo[(int64_t)pk * d.I];
            yo[(int64_t)pk * d.I] = s;
          }
        } else {
          const float* gp = src + b * PK * d.I + i;
          float sa[MAXM];
#pragma unroll
          for (int m = 0; m < MAXM; ++m) sa[m] = 0.f;
          for (int pk0 = 0; pk0 < PK; pk0 += 8) {
            float g8[8];
            int pc[8];
#pragma unroll
            for (int j = 0; j < 8; ++j) {
              pc[j] = min(pk0 + j, PK - 1);
              const float x = gp[(int64_t)pc[j] * d.I];
              g8[j] = pk0 + j < PK ? x : 0.f;
            }
#pragma unroll
            for (int j = 0; j < 8; ++j)
#pragma unroll
              for (int m = 0; m < MAXM; ++m) sa[m] += g8[j] * ub[m * PK + pc[j]];
          }
          float* o = dst + (b * d.I + i) * d.m1;
#pragma unroll
          for (int m = 0; m < MAXM; ++m)
            if (m < d.m1) {
              float val = sa[m];
              if constexpr (ACC) val += o[m];
              o[m] = val;
            }
        }
      }
    }
    __syncthreads();
  }
}

// Transposes with respect to v and U, through T_b[m][pk] = sum_i a[b][i][m] gy[b][pk][i]:
//   grad_v[b][n] (+)= sum_{m,pk} U[m*m2+n][pk] T_b[m][pk]                      (DO_V)
//   grad_U[m*m2+n][pk] = sum_b v[b][n] T_b[m][pk]: per-block partial sums upart  (DO_U)
// Lane pk forms column pk of T over channel chunks staged in LDS (gy transposed, padded rows); the lane
// keeps its U-gradient entries (m1*m2*PK <= 64*UREG) in registers over the block's elements.
template <bool DO_V, bool DO_U>
__global__ __launch_bounds__(256) void project_t_kernel(Dims d, const float* __restrict__ gy, const float* __restrict__ a,
                                                        const float* __restrict__ v, const float* __restrict__ U,
                                                        float* __restrict__ grad_v, int acc, float* __restrict__ upart) {
  extern __shared__ float sm[];
  const int PK = d.P * d.K, MN = d.m1 * d.m2;
  const int lane = threadIdx.x & 63, wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int per_wave = IC * d.m1 + IC * (PK + 1) + d.m1 * PK;
  float* us = sm;
  float* as = sm + MN * PK + wave * per_wave;   // [IC][m1]
  float* gs = as + IC * d.m1;                   // [IC][PK + 1]
  float* ts = gs + IC * (PK + 1);               // [m1][PK]
  if constexpr (DO_V) {
    for (int idx = threadIdx.x; idx < MN * PK; idx += 256) us[idx] = U[idx];
  }
  float ureg[UREG];
#pragma unroll
  for (int j = 0; j < UREG; ++j) ureg[j] = 0.f;
  __syncthreads();
  for (int64_t b0 = (int64_t)blockIdx.x * 4; b0 < d.B; b0 += (int64_t)gridDim.x * 4) {
    const int64_t b = b0 + wave;
    const bool ok = b < d.B;
    float tacc[MAXM];
#pragma unroll
    for (int m = 0; m < MAXM; ++m) tacc[m] = 0.f;
    for (int i0 = 0; i0 < d.I; i0 += IC) {
      const int ic = min(IC, d.I - i0);
      for (int idx = lane; idx < IC * d.m1; idx += 64)
        as[idx] = (ok && idx < ic * d.m1) ? a[(b * d.I + i0) * d.m1 + idx] : 0.f;
      for (int idx = lane; idx < PK * IC; idx += 64) {
        const int pk = idx / IC, ii = idx - pk * IC;
        gs[ii * (PK + 1) + pk] = (ok && ii < ic) ? gy[(b * PK + pk) * d.I + i0 + ii] : 0.f;
      }
      __syncthreads();
      if (lane < PK) {
        for (int ii = 0; ii < ic; ++ii) {
          const float gv = gs[ii * (PK + 1) + lane];
#pragma unroll
          for (int m = 0; m < MAXM; ++m)
            if (m < d.m1) tacc[m] += as[ii * d.m1 + m] * gv;
        }
      }
      __syncthreads();
    }
    if (lane < PK) {
#pragma unroll
      for (int m = 0; m < MAXM; ++m)
        if (m < d.m1) ts[m * PK + lane] = tacc[m];
    }
    __syncthreads();
    if constexpr (DO_V) {
      if (ok && lane < d.m2) {
        float s = 0.f;
        for (int m = 0; m < d.m1; ++m)
          for (int pk = 0; pk < PK; ++pk) s += us[(m * d.m2 + lane) * PK + pk] * ts[m * PK + pk];
        put(grad_v + b * d.m2 + lane, s, acc);
      }
    }
    if constexpr (DO_U) {
      if (ok) {
#pragma unroll
        for (int j = 0; j < UREG; ++j) {
          const int idx = lane + 64 * j;
          if (idx < MN * PK) {
            const int mn = idx / PK, pk = idx - mn * PK;
            const int m = mn / d.m2, n = mn - m * d.m2;
            ureg[j] += v[b * d.m2 + n] * ts[m * PK + pk];
          }
        }
      }
    }
    __syncthreads();
  }
  if constexpr (DO_U) {
    // the four waves' sums, added in a fixed order, are the block's partial sums
    float* red = sm;   // [4][MN * PK] (the host sizes the LDS for it)
#pragma unroll
    for (int j = 0; j < UREG; ++j) {
      const int idx = lane + 64 * j;
      if (idx < MN * PK) red[wave * MN * PK + idx] = ureg[j];
    }
    __syncthreads();
    for (int idx = threadIdx.x; idx < MN * PK; idx += 256)
      upart[(int64_t)blockIdx.x * MN * PK + idx] =
          ((red[idx] + red[MN * PK + idx]) + red[2 * MN * PK + idx]) + red[3 * MN * PK + idx];
  }
}

// out[idx] (+)= sum over parts of part[p][idx], parts in order.
__global__ void sum_parts_kernel(int64_t n, int nparts, const float* __restrict__ part, float* __restrict__ out, int acc) {
  for (int64_t idx = blockIdx.x * (int64_t)blockDim.x + threadIdx.x; idx < n; idx += (int64_t)gridDim.x * blockDim.x) {
    float s = 0.f;
    for (int p = 0; p < nparts; ++p) s += part[(int64_t)p * n + idx];
    put(out + idx, s, acc);
  }
}

// ---------------------------------------------------------------- channel mix (MFMA)
// Rows are the (b, k) pairs R = b*K + k.  A wave takes two 16-row tiles and eight 16-column tiles; lane
// (r, q) of an MFMA supplies A[r][4q..4q+3] and B[4q..4q+3][r] for a 16-deep K step and ends with
// D[4q + j][r] in result register j (common.h).

// out[b][o][k] (+)= sum_p g[b][p] sum_i y[b][p][k][i] W[p][o][i]   (K = (p, i); grid: 128 rows x 128 columns)
// TG: the per-path dot with the output gradient instead, grad_g[b][p] (+)= sum_{k,o} go[b][o][k]
// sum_i y[b][p][k][i] W[p][o][i] (grid: batch groups of 128/K elements x paths, all columns per block).
template <bool TG>
__global__ __launch_bounds__(256) void mix_kernel(Dims d, const float* __restrict__ y, const float* __restrict__ W,
                                                  const float* __restrict__ g, const float* __restrict__ go,
                                                  float* __restrict__ out, int acc) {
  __shared__ float rs[128];
  const int lane = threadIdx.x & 63, wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int r = lane & 15, q = lane >> 4;
  const int K = d.K, P = d.P, I = d.I, O = d.O;
  const int64_t R = d.B * K;
  // TG: the block's rows are whole batch elements bb0 .. bb0 + BB - 1 (rows never straddle two blocks)
  const int BB = 128 / K;
  const int64_t bb0 = (int64_t)blockIdx.x * BB;
  const int64_t rbeg = TG ? bb0 * K : (int64_t)blockIdx.x * 128;
  const int64_t rend = TG ? std::min<int64_t>((bb0 + BB) * K, R) : R;
  const int p_only = TG ? (int)blockIdx.y : -1;
  int64_t rb[2];
  int rk[2];
  bool rv[2];
#pragma unroll
  for (int t = 0; t < 2; ++t) {
    const int64_t row = rbeg + wave * 32 + 16 * t + r;
    rv[t] = row < rend;
    const int64_t rr = rv[t] ? row : 0;
    rb[t] = rr / K;
    rk[t] = (int)(rr - rb[t] * K);
  }
  float rowsum[2][4];
#pragma unroll
  for (int t = 0; t < 2; ++t)
#pragma unroll
    for (int j = 0; j < 4; ++j) rowsum[t][j] = 0.f;
  const int ocb_beg = TG ? 0 : (int)blockIdx.y * 128, ocb_end = TG ? O : std::min(O, ocb_beg + 128);
  for (int o0 = ocb_beg; o0 < ocb_end; o0 += 128) {
    f4 accm[2][8];
#pragma unroll
    for (int t = 0; t < 2; ++t)
#pragma unroll
      for (int j = 0; j < 8; ++j) accm[t][j] = f4{0.f, 0.f, 0.f, 0.f};
    bool cv[8];
#pragma unroll
    for (int j = 0; j < 8; ++j) cv[j] = o0 + 16 * j + r < O;
    // K steps (path p, channels i0 .. i0 + 15) in order; the operands of the next step are requested before
    // the products of the current one (two register sets, no copies).  Loads are unconditional at clamped
    // addresses and nothing reads them before the products: rows and columns past the end accumulate values
    // that are never stored, and the channel tail (I % 16) is cut by a zero scale on the A rows, applied with
    // the gate when the step is multiplied.
    const int pb = TG ? p_only : 0, pe = TG ? p_only + 1 : P;
    const int nis = (I + 15) / 16, nst = (pe - pb) * nis;
    int oc[8];
#pragma unroll
    for (int j = 0; j < 8; ++j) oc[j] = cv[j] ? o0 + 16 * j + r : 0;
    auto load = [&](int st, f4 (&av)[2], float (&gs)[2], f4 (&bw)[8]) {
      const int p = pb + st / nis, ii = (st % nis) * 16 + 4 * q;
      const bool iv = ii < I;   // I % 4 == 0: the whole float4 is in range
      const int ic = iv ? ii : 0;
#pragma unroll
      for (int t = 0; t < 2; ++t) {
        gs[t] = TG ? 1.f : g[rb[t] * P + p];
        if (!iv) gs[t] = 0.f;
        av[t] = ld4(y + ((rb[t] * P + p) * K + rk[t]) * I + ic);
      }
#pragma unroll
      for (int j = 0; j < 8; ++j) bw[j] = ld4(W + ((int64_t)p * O + oc[j]) * I + ic);
    };
    auto mma = [&](const f4 (&av)[2], const float (&gs)[2], const f4 (&bw)[8]) {
#pragma unroll
      for (int t = 0; t < 2; ++t) {
        const f4 a = av[t] * gs[t];
#pragma unroll
        for (int j = 0; j < 8; ++j) accm[t][j] = mfma_k16(a, bw[j], accm[t][j]);
      }
    };
    f4 a0[2], b0[8], a1[2], b1[8];
    float g0[2], g1[2];
    if (nst > 0) load(0, a0, g0, b0);
    for (int st = 0; st < nst; st += 2) {
      if (st + 1 < nst) load(st + 1, a1, g1, b1);
      __builtin_amdgcn_sched_barrier(0);
      mma(a0, g0, b0);
      if (st + 1 < nst) {
        if (st + 2 < nst) load(st + 2, a0, g0, b0);
        __builtin_amdgcn_sched_barrier(0);
        mma(a1, g1, b1);
      }
    }
#pragma unroll
    for (int t = 0; t < 2; ++t)
#pragma unroll
      for (int jj = 0; jj < 4; ++jj) {
        const int64_t row = rbeg + wave * 32 + 16 * t + 4 * q + jj;
        if (row >= rend) continue;
        const int64_t b = row / K;
        const int k = (int)(row - b * K);
#pragma unroll
        for (int j = 0; j < 8; ++j) {
          if (!cv[j]) continue;
          const int o = o0 + 16 * j + r;
          if constexpr (TG) rowsum[t][jj] += accm[t][j][jj] * go[(b * O + o) * K + k];
          else put(out + (b * O + o) * K + k, accm[t][j][jj], acc);
        }
      }
  }
  if constexpr (TG) {
    // row sums over the 16 column lanes, then over the K rows of each batch element
#pragma unroll
    for (int t = 0; t < 2; ++t)
#pragma unroll
      for (int jj = 0; jj < 4; ++jj) {
        float s = rowsum[t][jj];
#pragma unroll
        for (int off = 1; off < 16; off <<= 1) s += __shfl_xor(s, off, 64);
        if (r == 0) rs[wave * 32 + 16 * t + 4 * q + jj] = s;
      }
    __syncthreads();
    if (threadIdx.x < BB) {
      const int64_t b = bb0 + threadIdx.x;
      if (b < d.B) {
        float s = 0.f;
        for (int k = 0; k < K; ++k) s += rs[threadIdx.x * K + k];
        put(out + b * P + p_only, s, acc);
      }
    }
  }
}

// Wt[p][i][o] = W[p][o][i]
__global__ void transpose_w_kernel(int P, int O, int I, const float* __restrict__ W, float* __restrict__ Wt) {
  const int64_t n = (int64_t)P * O * I;
  for (int64_t idx = blockIdx.x * (int64_t)blockDim.x + threadIdx.x; idx < n; idx += (int64_t)gridDim.x * blockDim.x) {
    const int o = (int)(idx % O);
    const int64_t pi = idx / O;
    const int i = (int)(pi % I), p = (int)(pi / I);
    Wt[idx] = W[((int64_t)p * O + o) * I + i];
  }
}

// grad_y[b][p][k][i] (+)= g[b][p] sum_o go[b][o][k] W[p][o][i]: rows (b, k), columns i, K = o; grid: 128 rows x
// (path, 128-column block).  B from the transposed weights Wt[p][i][o] (float4 along o).
__global__ __launch_bounds__(256) void mix_ty_kernel(Dims d, const float* __restrict__ go, const float* __restrict__ Wt,
                                                     const float* __restrict__ g, float* __restrict__ gy, int acc) {
  const int lane = threadIdx.x & 63, wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int r = lane & 15, q = lane >> 4;
  const int K = d.K, P = d.P, I = d.I, O = d.O;
  const int64_t R = d.B * K;
  const int nib = (I + 127) / 128;
  const int p = (int)blockIdx.y / nib, i0c = ((int)blockIdx.y % nib) * 128;
  int64_t rb[2];
  int rk[2];
  bool rv[2];
#pragma unroll
  for (int t = 0; t < 2; ++t) {
    const int64_t row = (int64_t)blockIdx.x * 128 + wave * 32 + 16 * t + r;
    rv[t] = row < R;
    const int64_t rr = rv[t] ? row : 0;
    rb[t] = rr / K;
    rk[t] = (int)(rr - rb[t] * K);
  }
  bool cv[8];
  const float* wr[8];
#pragma unroll
  for (int j = 0; j < 8; ++j) {
    const int i = i0c + 16 * j + r;
    cv[j] = i < I;
    wr[j] = Wt + ((int64_t)p * I + (cv[j] ? i : 0)) * O;
  }
  f4 accm[2][8];
#pragma unroll
  for (int t = 0; t < 2; ++t)
#pragma unroll
    for (int j = 0; j < 8; ++j) accm[t][j] = f4{0.f, 0.f, 0.f, 0.f};
  for (int o0 = 0; o0 < O; o0 += 16) {
    const int oo = o0 + 4 * q;
    const bool ov = oo < O;   // O % 4 == 0
    f4 av[2], bw[8];
#pragma unroll
    for (int t = 0; t < 2; ++t) {
      const float* gp = go + (rb[t] * O + oo) * K + rk[t];
#pragma unroll
      for (int s = 0; s < 4; ++s) av[t][s] = (ov && rv[t]) ? gp[(int64_t)s * K] : 0.f;
    }
#pragma unroll
    for (int j = 0; j < 8; ++j) bw[j] = (ov && cv[j]) ? ld4(wr[j] + oo) : f4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int t = 0; t < 2; ++t)
#pragma unroll
      for (int j = 0; j < 8; ++j) accm[t][j] = mfma_k16(av[t], bw[j], accm[t][j]);
  }
#pragma unroll
  for (int t = 0; t < 2; ++t)
#pragma unroll
    for (int jj = 0; jj < 4; ++jj) {
      const int64_t row = (int64_t)blockIdx.x * 128 + wave * 32 + 16 * t + 4 * q + jj;
      if (row >= R) continue;
      const int64_t b = row / K;
      const int k = (int)(row - b * K);
      const float gate = g[b * P + p];
#pragma unroll
      for (int j = 0; j < 8; ++j)
        if (cv[j]) put(gy + ((b * P + p) * K + k) * I + i0c + 16 * j + r, accm[t][j][jj] * gate, acc);
    }
}

// Partial sums of grad_W[p][o][i] = sum_{(b,k)} g[b][p] go[b][o][k] y[b][p][k][i] over a range of rows:
// part[s][p][o][i].  M = o, N = i, K = rows (b, k), 16 rows per MFMA step; block (split s, path p, 128 x 128
// output tile): wave w takes o tiles 2w, 2w + 1 and all eight i tiles.
__global__ __launch_bounds__(256) void mix_tw_kernel(Dims d, const float* __restrict__ go, const float* __restrict__ y,
                                                     const float* __restrict__ g, int64_t rows_per_split,
                                                     float* __restrict__ part) {
  const int lane = threadIdx.x & 63, wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int r = lane & 15, q = lane >> 4;
  const int K = d.K, P = d.P, I = d.I, O = d.O;
  const int64_t R = d.B * K;
  const int s = blockIdx.x, p = blockIdx.y;
  const int nib = (I + 127) / 128;
  const int o0c = ((int)blockIdx.z / nib) * 128, i0c = ((int)blockIdx.z % nib) * 128;
  const int64_t r0 = (int64_t)s * rows_per_split, r1 = std::min(R, r0 + rows_per_split);
  f4 accm[2][8];
#pragma unroll
  for (int t = 0; t < 2; ++t)
#pragma unroll
    for (int j = 0; j < 8; ++j) accm[t][j] = f4{0.f, 0.f, 0.f, 0.f};
  bool ovt[2], ivt[8];
#pragma unroll
  for (int t = 0; t < 2; ++t) ovt[t] = o0c + wave * 32 + 16 * t + r < O;
#pragma unroll
  for (int j = 0; j < 8; ++j) ivt[j] = i0c + 16 * j + r < I;
  for (int64_t rr0 = r0; rr0 < r1; rr0 += 16) {
    // K step: rows rr0 + 4q + u (u = 0..3) for this lane group
    float gv[4];
    int64_t yoff[4], goff[4];
#pragma unroll
    for (int u = 0; u < 4; ++u) {
      const int64_t row = rr0 + 4 * q + u;
      const bool ok = row < r1;
      const int64_t rw = ok ? row : r0;
      const int64_t b = rw / K;
      const int k = (int)(rw - b * K);
      gv[u] = ok ? g[b * P + p] : 0.f;
      yoff[u] = ((b * P + p) * K + k) * I;
      goff[u] = b * O * K + k;
    }
    f4 av[2], bw[8];
#pragma unroll
    for (int t = 0; t < 2; ++t) {
      const int o = o0c + wave * 32 + 16 * t + r;
#pragma unroll
      for (int u = 0; u < 4; ++u) av[t][u] = ovt[t] ? go[goff[u] + (int64_t)o * K] * gv[u] : 0.f;
    }
#pragma unroll
    for (int j = 0; j < 8; ++j) {
      const int i = i0c + 16 * j + r;
#pragma unroll
      for (int u = 0; u < 4; ++u) bw[j][u] = ivt[j] ? y[yoff[u] + i] : 0.f;
    }
#pragma unroll
    for (int t = 0; t < 2; ++t)
#pragma unroll
      for (int j = 0; j < 8; ++j) accm[t][j] = mfma_k16(av[t], bw[j], accm[t][j]);
  }
  float* ps = part + ((int64_t)s * P + p) * O * I;
#pragma unroll
  for (int t = 0; t < 2; ++t)
#pragma unroll
    for (int jj = 0; jj < 4; ++jj) {
      const int o = o0c + wave * 32 + 16 * t + 4 * q + jj;
      if (o >= O) continue;
#pragma unroll
      for (int j = 0; j < 8; ++j)
        if (ivt[j]) ps[(int64_t)o * I + i0c + 16 * j + r] = accm[t][j][jj];
    }
}

// ---------------------------------------------------------------- host side
int check_dims(const Dims& d, bool proj) {
  FSC_CHECK_ARG(d.B >= 0 && d.I > 0 && d.P > 0 && d.K > 0, "bucket op: sizes must be positive");
  FSC_CHECK_ARG(d.B * d.K < (1LL << 31) && d.B * (int64_t)d.P * d.K * d.I < (1LL << 46), "bucket op: batch too large");
  if (proj) {
    FSC_CHECK_ARG(d.m1 > 0 && d.m1 <= MAXM && d.m2 > 0 && d.m2 <= MAXM, "bucket projection: m1 and m2 must be in 1..9");
    FSC_CHECK_ARG(d.P * d.K <= MAXPK, "bucket projection: P*kdim must be <= 64");
  } else {
    FSC_CHECK_ARG(d.O > 0 && d.I % 4 == 0 && d.O % 4 == 0, "bucket channel mix: mul_in1 and mul_out must be multiples of 4");
    FSC_CHECK_ARG(d.K <= 128, "bucket channel mix: kdim must be <= 128");
  }
  return 0;
}

unsigned batch_grid(int64_t B) { return (unsigned)std::max<int64_t>(1, std::min<int64_t>((B + 3) / 4, 4096)); }

size_t proj_t_lds(const Dims& d, bool do_u) {
  const int PK = d.P * d.K, MN = d.m1 * d.m2;
  const size_t main = (size_t)(MN * PK + 4 * (IC * d.m1 + IC * (PK + 1) + d.m1 * PK)) * 4;
  return do_u ? std::max(main, (size_t)4 * MN * PK * 4) : main;
}

}  // namespace bucket
}  // namespace fsc

// ===================================================================== C ABI
using namespace fsc;
using fsc::bucket::Dims;

extern "C" int fsc_bucket_project(int64_t B, int32_t I, int32_t m1, int32_t m2, int32_t P, int32_t K, const float* a,
                                  const float* v, const float* u, float* y, int32_t accumulate, hipStream_t st) {
  const Dims d{B, I, m1, m2, P, K, 0};
  if (bucket::check_dims(d, true)) return 1;
  if (B == 0) return 0;
  const size_t lds = (size_t)(m1 * m2 * P * K + 4 * bucket::MAXM * P * K) * 4;
  if (accumulate)
    bucket::project_kernel<false, true><<<bucket::batch_grid(B), 256, lds, st>>>(d, a, v, u, y);
  else
    bucket::project_kernel<false, false><<<bucket::batch_grid(B), 256, lds, st>>>(d, a, v, u, y);
  return check_launch("bucket project") ? 2 : 0;
}

extern "C" int fsc_bucket_project_transpose_a(int64_t B, int32_t I, int32_t m1, int32_t m2, int32_t P, int32_t K,
                                              const float* grad_y, const float* v, const float* u, float* grad_a,
                                              int32_t accumulate, hipStream_t st) {
  const Dims d{B, I, m1, m2, P, K, 0};
  if (bucket::check_dims(d, true)) return 1;
  if (B == 0) return 0;
  const size_t lds = (size_t)(m1 * m2 * P * K + 4 * bucket::MAXM * P * K) * 4;
  if (accumulate)
    bucket::project_kernel<true, true><<<bucket::batch_grid(B), 256, lds, st>>>(d, grad_y, v, u, grad_a);
  else
    bucket::project_kernel<true, false><<<bucket::batch_grid(B), 256, lds, st>>>(d, grad_y, v, u, grad_a);
  return check_launch("bucket project_transpose_a") ? 2 : 0;
}

extern "C" int fsc_bucket_project_workspace(int64_t B, int32_t I, int32_t m1, int32_t m2, int32_t P, int32_t K,
                                            int64_t* workspace_floats) {
  const Dims d{B, I, m1, m2, P, K, 0};
  if (bucket::check_dims(d, true)) return 1;
  FSC_CHECK_ARG((int64_t)m1 * m2 * P * K <= 64 * bucket::UREG, "bucket projection: m1*m2*P*kdim must be <= 2048");
  *workspace_floats = (int64_t)bucket::batch_grid(B) * m1 * m2 * P * K;
  return 0;
}

extern "C" int fsc_bucket_project_transpose_vu(int64_t B, int32_t I, int32_t m1, int32_t m2, int32_t P, int32_t K,
                                               const float* grad_y, const float* a, const float* v, const float* u,
                                               float* grad_v, float* grad_u, int32_t accumulate, float* workspace,
                                               hipStream_t st) {
  const Dims d{B, I, m1, m2, P, K, 0};
  if (bucket::check_dims(d, true)) return 1;
  FSC_CHECK_ARG(grad_v || grad_u, "bucket project_transpose: nothing requested");
  const int64_t mnpk = (int64_t)m1 * m2 * P * K;
  if (grad_u) FSC_CHECK_ARG(mnpk <= 64 * bucket::UREG && workspace, "bucket projection: m1*m2*P*kdim must be <= 2048");
  const unsigned grid = bucket::batch_grid(B);
  if (B > 0) {
    const size_t lds = bucket::proj_t_lds(d, grad_u != nullptr);
    if (grad_v && grad_u)
      bucket::project_t_kernel<true, true><<<grid, 256, lds, st>>>(d, grad_y, a, v, u, grad_v, accumulate, workspace);
    else if (grad_v)
      bucket::project_t_kernel<true, false><<<grid, 256, lds, st>>>(d, grad_y, a, v, u, grad_v, accumulate, nullptr);
    else
      bucket::project_t_kernel<false, true><<<grid, 256, lds, st>>>(d, grad_y, a, v, u, nullptr, 0, workspace);
    if (check_launch("bucket project_transpose")) return 2;
  }
  if (grad_u) {
    // (no elements: a sum over zero parts, which writes zeros or leaves an accumulated output unchanged)
    bucket::sum_parts_kernel<<<(unsigned)std::min<int64_t>((mnpk + 255) / 256, 1024), 256, 0, st>>>(
        mnpk, B > 0 ? (int)grid : 0, workspace, grad_u, accumulate);
    if (check_launch("bucket project_transpose_u reduce")) return 2;
  }
  return 0;
}

extern "C" int fsc_bucket_mix(int64_t B, int32_t P, int32_t K, int32_t I, int32_t O, const float* y, const float* w,
                              const float* gates, float* out, int32_t accumulate, hipStream_t st) {
  const Dims d{B, I, 0, 0, P, K, O};
  if (bucket::check_dims(d, false)) return 1;
  if (B == 0) return 0;
  const dim3 grid((unsigned)((B * K + 127) / 128), (unsigned)((O + 127) / 128));
  bucket::mix_kernel<false><<<grid, 256, 0, st>>>(d, y, w, gates, nullptr, out, accumulate);
  return check_launch("bucket mix") ? 2 : 0;
}

extern "C" int fsc_bucket_mix_transpose_g(int64_t B, int32_t P, int32_t K, int32_t I, int32_t O, const float* grad_out,
                                          const float* y, const float* w, float* grad_g, int32_t accumulate,
                                          hipStream_t st) {
  const Dims d{B, I, 0, 0, P, K, O};
  if (bucket::check_dims(d, false)) return 1;
  if (B == 0) return 0;
  const int BB = 128 / K;
  const dim3 grid((unsigned)((B + BB - 1) / BB), (unsigned)P);
  bucket::mix_kernel<true><<<grid, 256, 0, st>>>(d, y, w, nullptr, grad_out, grad_g, accumulate);
  return check_launch("bucket mix_transpose_g") ? 2 : 0;
}

static int64_t mix_tw_splits(int64_t B, int32_t P, int32_t K, int32_t I, int32_t O, int64_t* rows_per_split) {
  const int64_t R = std::max<int64_t>(B * K, 1);
  const int64_t tiles = (int64_t)P * ((O + 127) / 128) * ((I + 127) / 128);
  const int64_t want = std::max<int64_t>(1, 2048 / tiles);
  int64_t rps = std::max<int64_t>(256, (R + want - 1) / want);
  rps = (rps + 15) / 16 * 16;
  *rows_per_split = rps;
  return (R + rps - 1) / rps;
}

extern "C" int fsc_bucket_mix_workspace(int64_t B, int32_t P, int32_t K, int32_t I, int32_t O, int64_t* workspace_floats) {
  const Dims d{B, I, 0, 0, P, K, O};
  if (bucket::check_dims(d, false)) return 1;
  int64_t rps;
  const int64_t ns = mix_tw_splits(B, P, K, I, O, &rps);
  *workspace_floats = std::max<int64_t>(ns * P * (int64_t)O * I, (int64_t)P * O * I);
  return 0;
}

extern "C" int fsc_bucket_mix_transpose_y(int64_t B, int32_t P, int32_t K, int32_t I, int32_t O, const float* grad_out,
                                          const float* w, const float* gates, float* grad_y, int32_t accumulate,
                                          float* workspace, hipStream_t st) {
  const Dims d{B, I, 0, 0, P, K, O};
  if (bucket::check_dims(d, false)) return 1;
  if (B == 0) return 0;
  const int64_t nw = (int64_t)P * O * I;
  bucket::transpose_w_kernel<<<(unsigned)std::min<int64_t>((nw + 255) / 256, 4096), 256, 0, st>>>(P, O, I, w, workspace);
  if (check_launch("bucket transpose_w")) return 2;
  const dim3 grid((unsigned)((B * K + 127) / 128), (unsigned)(P * ((I + 127) / 128)));
  bucket::mix_ty_kernel<<<grid, 256, 0, st>>>(d, grad_out, workspace, gates, grad_y, accumulate);
  return check_launch("bucket mix_transpose_y") ? 2 : 0;
}

extern "C" int fsc_bucket_mix_transpose_w(int64_t B, int32_t P, int32_t K, int32_t I, int32_t O, const float* grad_out,
                                          const float* y, const float* gates, float* grad_w, int32_t accumulate,
                                          float* workspace, hipStream_t st) {
  const Dims d{B, I, 0, 0, P, K, O};
  if (bucket::check_dims(d, false)) return 1;
  const int64_t nw = (int64_t)P * O * I;
  if (B == 0) {   // a sum over zero parts
    bucket::sum_parts_kernel<<<(unsigned)std::min<int64_t>((nw + 255) / 256, 4096), 256, 0, st>>>(nw, 0, workspace,
                                                                                                  grad_w, accumulate);
    return check_launch("bucket mix_transpose_w") ? 2 : 0;
  }
  int64_t rps;
  const int64_t ns = mix_tw_splits(B, P, K, I, O, &rps);
  const dim3 grid((unsigned)ns, (unsigned)P, (unsigned)(((O + 127) / 128) * ((I + 127) / 128)));
  bucket::mix_tw_kernel<<<grid, 256, 0, st>>>(d, grad_out, y, gates, rps, workspace);
  if (check_launch("bucket mix_transpose_w")) return 2;
  bucket::sum_parts_kernel<<<(unsigned)std::min<int64_t>((nw + 255) / 256, 4096), 256, 0, st>>>(nw, (int)ns, workspace,
                                                                                                grad_w, accumulate);
  return check_launch("bucket mix_transpose_w reduce") ? 2 : 0;
}
