// The per-edge ("bucketed") ICTD tensor product of the reference's native extension on gfx950: the
// operations of molecular_force_field._C_ictd_tp (csrc/ictd_tp.cpp:498-522, CUDA half
// csrc/ictd_tp_cuda.cu) for the arguments its CUDA path takes (fp32 and fp64, mul_in2 == 1):
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
// channel mixes are GEMMs over (b, k) rows and run on v_mfma_f32_16x16x4_f32 (fp32) or
// v_mfma_f64_16x16x4_f64 (fp64; MI355X runs fp64 matrix and vector FMAs at the same peak, the MFMA form keeps
// the operand reuse of the tile).  Every kernel is templated on the element type T.  Every kernel writes or,
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

typedef double d4 __attribute__((ext_vector_type(4)));

// One 16-deep K step of a 16 x 16 output tile for either element type.  Both MFMAs take lane l's operands
// as A[l%16][l/16] and B[l/16][l%16]; their results differ in layout: register j of lane l holds
// D[4*(l/16) + j][l%16] for v_mfma_f32_16x16x4_f32 and D[l/16 + 4*j][l%16] for v_mfma_f64_16x16x4_f64
// (checked on gfx950).  row(q, j) gives the tile row of result register j in lane group q.
template <typename T>
struct Mma;
template <>
struct Mma<float> {
  using V = f4;
  static __device__ __forceinline__ V zero() { return V{0.f, 0.f, 0.f, 0.f}; }
  static __device__ __forceinline__ V mma(const V& a, const V& b, V c) { return mfma_k16(a, b, c); }
  static __device__ __forceinline__ V ld(const float* p) { return ld4(p); }
  static __device__ __forceinline__ int row(int q, int j) { return 4 * q + j; }
};
template <>
struct Mma<double> {
  using V = d4;
  static __device__ __forceinline__ V zero() { return V{0.0, 0.0, 0.0, 0.0}; }
  static __device__ __forceinline__ V mma(const V& a, const V& b, V c) {
    c = __builtin_amdgcn_mfma_f64_16x16x4f64(a.x, b.x, c, 0, 0, 0);
    c = __builtin_amdgcn_mfma_f64_16x16x4f64(a.y, b.y, c, 0, 0, 0);
    c = __builtin_amdgcn_mfma_f64_16x16x4f64(a.z, b.z, c, 0, 0, 0);
    return __builtin_amdgcn_mfma_f64_16x16x4f64(a.w, b.w, c, 0, 0, 0);
  }
  static __device__ __forceinline__ V ld(const double* p) { return V{p[0], p[1], p[2], p[3]}; }
  static __device__ __forceinline__ int row(int q, int j) { return q + 4 * j; }
};

// Factor of the projection for element b, padded to MAXM rows: ub[m][pk] = sum_n v[b][n] U[m*m2+n][pk] for
// m < m1 and zero for m1 <= m < MAXM (us: U in LDS), so that the contractions below run over MAXM rows with
// no branch (a branch per row would make every product wait for all outstanding stores).
template <typename T>
__device__ __forceinline__ void form_ub(const Dims& d, int PK, const T* __restrict__ v, const T* us, T* ub, int64_t b,
                                        bool ok, int lane) {
  T vb[MAXM];   // v[b][n], zero past m2: all loads issued together (one wait)
#pragma unroll
  for (int n = 0; n < MAXM; ++n) {
    const T x = v[(ok ? b : 0) * d.m2 + min(n, d.m2 - 1)];
    vb[n] = (ok && n < d.m2) ? x : T(0);
  }
  for (int idx = lane; idx < MAXM * PK; idx += 64) {
    const int m = idx / PK, pk = idx - m * PK;
    const int mc = min(m, d.m1 - 1);
    T s = 0;
#pragma unroll
    for (int n = 0; n < MAXM; ++n) s += vb[n] * us[(mc * d.m2 + min(n, d.m2 - 1)) * PK + pk];
    ub[idx] = m < d.m1 ? s : T(0);
  }
}

template <typename T>
__device__ __forceinline__ void put(T* p, T v, int acc) { *p = acc ? *p + v : v; }

// TA false: y[b][pk][i] (+)= sum_m a[b][i][m] ub[m][pk]        (src = a, dst = y)
// TA true:  grad_a[b][i][m] (+)= sum_pk gy[b][pk][i] ub[m][pk]  (src = gy, dst = grad_a)
// Four waves per block, one batch element per wave per step; U staged in LDS once per block.  Lane i holds
// its a row (MAXM values, zero past m1; the loads clamp their index) or its gy values eight at a time.
template <typename T, bool TA, bool ACC>
__global__ __launch_bounds__(256) void project_kernel(Dims d, const T* __restrict__ src, const T* __restrict__ v,
                                                      const T* __restrict__ U, T* __restrict__ dst) {
  extern __shared__ __align__(16) char smraw[];
  T* sm = reinterpret_cast<T*>(smraw);
  const int PK = d.P * d.K, MN = d.m1 * d.m2;
  const int lane = threadIdx.x & 63, wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  T* us = sm;
  T* ub = sm + MN * PK + wave * MAXM * PK;
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
          const T* ar = src + (b * d.I + i) * d.m1;
          T av[MAXM];
#pragma unroll
          for (int m = 0; m < MAXM; ++m) {
            const T x = ar[min(m, d.m1 - 1)];
            av[m] = m < d.m1 ? x : T(0);
          }
          T* yo = dst + b * PK * d.I + i;
          for (int pk = 0; pk < PK; ++pk) {
            T s = 0;
#pragma unroll
            for (int m = 0; m < MAXM; ++m) s += av[m] * ub[m * PK + pk];
            if constexpr (ACC) s += yo[(int64_t)pk * d.I];
            yo[(int64_t)pk * d.I] = s;
          }
        } else {
          const T* gp = src + b * PK * d.I + i;
          T sa[MAXM];
#pragma unroll
          for (int m = 0; m < MAXM; ++m) sa[m] = 0;
          for (int pk0 = 0; pk0 < PK; pk0 += 8) {
            T g8[8];
            int pc[8];
#pragma unroll
            for (int j = 0; j < 8; ++j) {
              pc[j] = min(pk0 + j, PK - 1);
              const T x = gp[(int64_t)pc[j] * d.I];
              g8[j] = pk0 + j < PK ? x : T(0);
            }
#pragma unroll
            for (int j = 0; j < 8; ++j)
#pragma unroll
              for (int m = 0; m < MAXM; ++m) sa[m] += g8[j] * ub[m * PK + pc[j]];
          }
          T* o = dst + (b * d.I + i) * d.m1;
#pragma unroll
          for (int m = 0; m < MAXM; ++m)
            if (m < d.m1) {
              T val = sa[m];
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
template <typename T, bool DO_V, bool DO_U>
__global__ __launch_bounds__(256) void project_t_kernel(Dims d, const T* __restrict__ gy, const T* __restrict__ a,
                                                        const T* __restrict__ v, const T* __restrict__ U,
                                                        T* __restrict__ grad_v, int acc, T* __restrict__ upart) {
  extern __shared__ __align__(16) char smraw[];
  T* sm = reinterpret_cast<T*>(smraw);
  const int PK = d.P * d.K, MN = d.m1 * d.m2;
  const int lane = threadIdx.x & 63, wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int per_wave = IC * d.m1 + IC * (PK + 1) + d.m1 * PK;
  T* us = sm;
  T* as = sm + MN * PK + wave * per_wave;   // [IC][m1]
  T* gs = as + IC * d.m1;                   // [IC][PK + 1]
  T* ts = gs + IC * (PK + 1);               // [m1][PK]
  if constexpr (DO_V) {
    for (int idx = threadIdx.x; idx < MN * PK; idx += 256) us[idx] = U[idx];
  }
  T ureg[UREG];
#pragma unroll
  for (int j = 0; j < UREG; ++j) ureg[j] = 0;
  __syncthreads();
  for (int64_t b0 = (int64_t)blockIdx.x * 4; b0 < d.B; b0 += (int64_t)gridDim.x * 4) {
    const int64_t b = b0 + wave;
    const bool ok = b < d.B;
    T tacc[MAXM];
#pragma unroll
    for (int m = 0; m < MAXM; ++m) tacc[m] = 0;
    for (int i0 = 0; i0 < d.I; i0 += IC) {
      const int ic = min(IC, d.I - i0);
      for (int idx = lane; idx < IC * d.m1; idx += 64)
        as[idx] = (ok && idx < ic * d.m1) ? a[(b * d.I + i0) * d.m1 + idx] : T(0);
      for (int idx = lane; idx < PK * IC; idx += 64) {
        const int pk = idx / IC, ii = idx - pk * IC;
        gs[ii * (PK + 1) + pk] = (ok && ii < ic) ? gy[(b * PK + pk) * d.I + i0 + ii] : T(0);
      }
      __syncthreads();
      if (lane < PK) {
        for (int ii = 0; ii < ic; ++ii) {
          const T gv = gs[ii * (PK + 1) + lane];
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
        T s = 0;
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
    T* red = sm;   // [4][MN * PK] (the host sizes the LDS for it)
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
template <typename T>
__global__ void sum_parts_kernel(int64_t n, int nparts, const T* __restrict__ part, T* __restrict__ out, int acc) {
  for (int64_t idx = blockIdx.x * (int64_t)blockDim.x + threadIdx.x; idx < n; idx += (int64_t)gridDim.x * blockDim.x) {
    T s = 0;
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
template <typename T, bool TG>
__global__ __launch_bounds__(256) void mix_kernel(Dims d, const T* __restrict__ y, const T* __restrict__ W,
                                                  const T* __restrict__ g, const T* __restrict__ go,
                                                  T* __restrict__ out, int acc) {
  using M = Mma<T>;
  using V = typename M::V;
  // fp32 requests the next K step's operands before the current products (two register sets); fp64,
  // whose operand sets are twice as large, works one step at a time
  constexpr bool PF = sizeof(T) == 4;
  __shared__ T rs[128];
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
#pragma unroll
  for (int t = 0; t < 2; ++t) {
    const int64_t row = rbeg + wave * 32 + 16 * t + r;
    const int64_t rr = row < rend ? row : 0;
    rb[t] = rr / K;
    rk[t] = (int)(rr - rb[t] * K);
  }
  T rowsum[2][4];
#pragma unroll
  for (int t = 0; t < 2; ++t)
#pragma unroll
    for (int j = 0; j < 4; ++j) rowsum[t][j] = 0;
  const int ocb_beg = TG ? 0 : (int)blockIdx.y * 128, ocb_end = TG ? O : std::min(O, ocb_beg + 128);
  for (int o0 = ocb_beg; o0 < ocb_end; o0 += 128) {
    V accm[2][8];
#pragma unroll
    for (int t = 0; t < 2; ++t)
#pragma unroll
      for (int j = 0; j < 8; ++j) accm[t][j] = M::zero();
    bool cv[8];
#pragma unroll
    for (int j = 0; j < 8; ++j) cv[j] = o0 + 16 * j + r < O;
    // K steps (path p, channels i0 .. i0 + 15) in order.  Loads are unconditional at clamped addresses and
    // nothing reads them before the products: rows and columns past the end accumulate values that are never
    // stored, and the channel tail (I % 16) is cut by a zero scale on the A rows, applied with the gate when
    // the step is multiplied.
    const int pb = TG ? p_only : 0, pe = TG ? p_only + 1 : P;
    const int nis = (I + 15) / 16, nst = (pe - pb) * nis;
    int oc[8];
#pragma unroll
    for (int j = 0; j < 8; ++j) oc[j] = cv[j] ? o0 + 16 * j + r : 0;
    auto load = [&](int st, V (&av)[2], T (&gs)[2], V (&bw)[8]) {
      const int p = pb + st / nis, ii = (st % nis) * 16 + 4 * q;
      const bool iv = ii < I;   // I % 4 == 0: the whole 4-vector is in range
      const int ic = iv ? ii : 0;
#pragma unroll
      for (int t = 0; t < 2; ++t) {
        gs[t] = TG ? T(1) : g[rb[t] * P + p];
        if (!iv) gs[t] = 0;
        av[t] = M::ld(y + ((rb[t] * P + p) * K + rk[t]) * I + ic);
      }
#pragma unroll
      for (int j = 0; j < 8; ++j) bw[j] = M::ld(W + ((int64_t)p * O + oc[j]) * I + ic);
    };
    auto mma = [&](const V (&av)[2], const T (&gs)[2], const V (&bw)[8]) {
#pragma unroll
      for (int t = 0; t < 2; ++t) {
        const V a = av[t] * gs[t];
#pragma unroll
        for (int j = 0; j < 8; ++j) accm[t][j] = M::mma(a, bw[j], accm[t][j]);
      }
    };
    if constexpr (PF) {
      V a0[2], b0[8], a1[2], b1[8];
      T g0[2], g1[2];
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
    } else {
      for (int st = 0; st < nst; ++st) {
        V a0[2], b0[8];
        T g0[2];
        load(st, a0, g0, b0);
        mma(a0, g0, b0);
      }
    }
#pragma unroll
    for (int t = 0; t < 2; ++t)
#pragma unroll
      for (int jj = 0; jj < 4; ++jj) {
        const int64_t row = rbeg + wave * 32 + 16 * t + M::row(q, jj);
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
        T s = rowsum[t][jj];
#pragma unroll
        for (int off = 1; off < 16; off <<= 1) s += __shfl_xor(s, off, 64);
        if (r == 0) rs[wave * 32 + 16 * t + M::row(q, jj)] = s;
      }
    __syncthreads();
    if (threadIdx.x < BB) {
      const int64_t b = bb0 + threadIdx.x;
      if (b < d.B) {
        T s = 0;
        for (int k = 0; k < K; ++k) s += rs[threadIdx.x * K + k];
        put(out + b * P + p_only, s, acc);
      }
    }
  }
}

// Wt[p][i][o] = W[p][o][i]
template <typename T>
__global__ void transpose_w_kernel(int P, int O, int I, const T* __restrict__ W, T* __restrict__ Wt) {
  const int64_t n = (int64_t)P * O * I;
  for (int64_t idx = blockIdx.x * (int64_t)blockDim.x + threadIdx.x; idx < n; idx += (int64_t)gridDim.x * blockDim.x) {
    const int o = (int)(idx % O);
    const int64_t pi = idx / O;
    const int i = (int)(pi % I), p = (int)(pi / I);
    Wt[idx] = W[((int64_t)p * O + o) * I + i];
  }
}

// grad_y[b][p][k][i] (+)= g[b][p] sum_o go[b][o][k] W[p][o][i]: rows (b, k), columns i, K = o; grid: 128 rows x
// (path, 128-column block).  B from the transposed weights Wt[p][i][o] (4-vectors along o).
template <typename T>
__global__ __launch_bounds__(256) void mix_ty_kernel(Dims d, const T* __restrict__ go, const T* __restrict__ Wt,
                                                     const T* __restrict__ g, T* __restrict__ gy, int acc) {
  using M = Mma<T>;
  using V = typename M::V;
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
  const T* wr[8];
#pragma unroll
  for (int j = 0; j < 8; ++j) {
    const int i = i0c + 16 * j + r;
    cv[j] = i < I;
    wr[j] = Wt + ((int64_t)p * I + (cv[j] ? i : 0)) * O;
  }
  V accm[2][8];
#pragma unroll
  for (int t = 0; t < 2; ++t)
#pragma unroll
    for (int j = 0; j < 8; ++j) accm[t][j] = M::zero();
  for (int o0 = 0; o0 < O; o0 += 16) {
    const int oo = o0 + 4 * q;
    const bool ov = oo < O;   // O % 4 == 0
    V av[2], bw[8];
#pragma unroll
    for (int t = 0; t < 2; ++t) {
      const T* gp = go + (rb[t] * O + oo) * K + rk[t];
#pragma unroll
      for (int s = 0; s < 4; ++s) av[t][s] = (ov && rv[t]) ? gp[(int64_t)s * K] : T(0);
    }
#pragma unroll
    for (int j = 0; j < 8; ++j) bw[j] = (ov && cv[j]) ? M::ld(wr[j] + oo) : M::zero();
#pragma unroll
    for (int t = 0; t < 2; ++t)
#pragma unroll
      for (int j = 0; j < 8; ++j) accm[t][j] = M::mma(av[t], bw[j], accm[t][j]);
  }
#pragma unroll
  for (int t = 0; t < 2; ++t)
#pragma unroll
    for (int jj = 0; jj < 4; ++jj) {
      const int64_t row = (int64_t)blockIdx.x * 128 + wave * 32 + 16 * t + M::row(q, jj);
      if (row >= R) continue;
      const int64_t b = row / K;
      const int k = (int)(row - b * K);
      const T gate = g[b * P + p];
#pragma unroll
      for (int j = 0; j < 8; ++j)
        if (cv[j]) put(gy + ((b * P + p) * K + k) * I + i0c + 16 * j + r, accm[t][j][jj] * gate, acc);
    }
}

// Partial sums of grad_W[p][o][i] = sum_{(b,k)} g[b][p] go[b][o][k] y[b][p][k][i] over a range of rows:
// part[s][p][o][i].  M = o, N = i, K = rows (b, k), 16 rows per MFMA step; block (split s, path p, 128 x 128
// output tile): wave w takes o tiles 2w, 2w + 1 and all eight i tiles.
template <typename T>
__global__ __launch_bounds__(256) void mix_tw_kernel(Dims d, const T* __restrict__ go, const T* __restrict__ y,
                                                     const T* __restrict__ g, int64_t rows_per_split,
                                                     T* __restrict__ part) {
  using M = Mma<T>;
  using V = typename M::V;
  const int lane = threadIdx.x & 63, wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int r = lane & 15, q = lane >> 4;
  const int K = d.K, P = d.P, I = d.I, O = d.O;
  const int64_t R = d.B * K;
  const int s = blockIdx.x, p = blockIdx.y;
  const int nib = (I + 127) / 128;
  const int o0c = ((int)blockIdx.z / nib) * 128, i0c = ((int)blockIdx.z % nib) * 128;
  const int64_t r0 = (int64_t)s * rows_per_split, r1 = std::min(R, r0 + rows_per_split);
  V accm[2][8];
#pragma unroll
  for (int t = 0; t < 2; ++t)
#pragma unroll
    for (int j = 0; j < 8; ++j) accm[t][j] = M::zero();
  bool ovt[2], ivt[8];
#pragma unroll
  for (int t = 0; t < 2; ++t) ovt[t] = o0c + wave * 32 + 16 * t + r < O;
#pragma unroll
  for (int j = 0; j < 8; ++j) ivt[j] = i0c + 16 * j + r < I;
  for (int64_t rr0 = r0; rr0 < r1; rr0 += 16) {
    // K step: rows rr0 + 4q + u (u = 0..3) for this lane group
    T gv[4];
    int64_t yoff[4], goff[4];
#pragma unroll
    for (int u = 0; u < 4; ++u) {
      const int64_t row = rr0 + 4 * q + u;
      const bool ok = row < r1;
      const int64_t rw = ok ? row : r0;
      const int64_t b = rw / K;
      const int k = (int)(rw - b * K);
      gv[u] = ok ? g[b * P + p] : T(0);
      yoff[u] = ((b * P + p) * K + k) * I;
      goff[u] = b * O * K + k;
    }
    V av[2], bw[8];
#pragma unroll
    for (int t = 0; t < 2; ++t) {
      const int o = o0c + wave * 32 + 16 * t + r;
#pragma unroll
      for (int u = 0; u < 4; ++u) av[t][u] = ovt[t] ? go[goff[u] + (int64_t)o * K] * gv[u] : T(0);
    }
#pragma unroll
    for (int j = 0; j < 8; ++j) {
      const int i = i0c + 16 * j + r;
#pragma unroll
      for (int u = 0; u < 4; ++u) bw[j][u] = ivt[j] ? y[yoff[u] + i] : T(0);
    }
#pragma unroll
    for (int t = 0; t < 2; ++t)
#pragma unroll
      for (int j = 0; j < 8; ++j) accm[t][j] = M::mma(av[t], bw[j], accm[t][j]);
  }
  T* ps = part + ((int64_t)s * P + p) * O * I;
#pragma unroll
  for (int t = 0; t < 2; ++t)
#pragma unroll
    for (int jj = 0; jj < 4; ++jj) {
      const int o = o0c + wave * 32 + 16 * t + M::row(q, jj);
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

size_t proj_t_lds(const Dims& d, bool do_u, size_t elem) {
  const int PK = d.P * d.K, MN = d.m1 * d.m2;
  const size_t main = (size_t)(MN * PK + 4 * (IC * d.m1 + IC * (PK + 1) + d.m1 * PK)) * elem;
  return do_u ? std::max(main, (size_t)4 * MN * PK * elem) : main;
}

// ---------------------------------------------------------------- entry points, for T = float and double
template <typename T>
int project(int64_t B, int32_t I, int32_t m1, int32_t m2, int32_t P, int32_t K, const T* a, const T* v, const T* u,
            T* y, int32_t accumulate, hipStream_t st) {
  const Dims d{B, I, m1, m2, P, K, 0};
  if (check_dims(d, true)) return 1;
  if (B == 0) return 0;
  const size_t lds = (size_t)(m1 * m2 * P * K + 4 * MAXM * P * K) * sizeof(T);
  if (accumulate)
    project_kernel<T, false, true><<<batch_grid(B), 256, lds, st>>>(d, a, v, u, y);
  else
    project_kernel<T, false, false><<<batch_grid(B), 256, lds, st>>>(d, a, v, u, y);
  return check_launch("bucket project") ? 2 : 0;
}

template <typename T>
int project_transpose_a(int64_t B, int32_t I, int32_t m1, int32_t m2, int32_t P, int32_t K, const T* grad_y,
                        const T* v, const T* u, T* grad_a, int32_t accumulate, hipStream_t st) {
  const Dims d{B, I, m1, m2, P, K, 0};
  if (check_dims(d, true)) return 1;
  if (B == 0) return 0;
  const size_t lds = (size_t)(m1 * m2 * P * K + 4 * MAXM * P * K) * sizeof(T);
  if (accumulate)
    project_kernel<T, true, true><<<batch_grid(B), 256, lds, st>>>(d, grad_y, v, u, grad_a);
  else
    project_kernel<T, true, false><<<batch_grid(B), 256, lds, st>>>(d, grad_y, v, u, grad_a);
  return check_launch("bucket project_transpose_a") ? 2 : 0;
}

int project_workspace(int64_t B, int32_t I, int32_t m1, int32_t m2, int32_t P, int32_t K, int64_t* workspace_elems) {
  const Dims d{B, I, m1, m2, P, K, 0};
  if (check_dims(d, true)) return 1;
  FSC_CHECK_ARG((int64_t)m1 * m2 * P * K <= 64 * UREG, "bucket projection: m1*m2*P*kdim must be <= 2048");
  *workspace_elems = (int64_t)batch_grid(B) * m1 * m2 * P * K;
  return 0;
}

template <typename T>
int project_transpose_vu(int64_t B, int32_t I, int32_t m1, int32_t m2, int32_t P, int32_t K, const T* grad_y,
                         const T* a, const T* v, const T* u, T* grad_v, T* grad_u, int32_t accumulate, T* workspace,
                         hipStream_t st) {
  const Dims d{B, I, m1, m2, P, K, 0};
  if (check_dims(d, true)) return 1;
  FSC_CHECK_ARG(grad_v || grad_u, "bucket project_transpose: nothing requested");
  const int64_t mnpk = (int64_t)m1 * m2 * P * K;
  if (grad_u) FSC_CHECK_ARG(mnpk <= 64 * UREG && workspace, "bucket projection: m1*m2*P*kdim must be <= 2048");
  const unsigned grid = batch_grid(B);
  if (B > 0) {
    const size_t lds = proj_t_lds(d, grad_u != nullptr, sizeof(T));
    if (grad_v && grad_u)
      project_t_kernel<T, true, true><<<grid, 256, lds, st>>>(d, grad_y, a, v, u, grad_v, accumulate, workspace);
    else if (grad_v)
      project_t_kernel<T, true, false><<<grid, 256, lds, st>>>(d, grad_y, a, v, u, grad_v, accumulate, nullptr);
    else
      project_t_kernel<T, false, true><<<grid, 256, lds, st>>>(d, grad_y, a, v, u, nullptr, 0, workspace);
    if (check_launch("bucket project_transpose")) return 2;
  }
  if (grad_u) {
    // (no elements: a sum over zero parts, which writes zeros or leaves an accumulated output unchanged)
    sum_parts_kernel<T><<<(unsigned)std::min<int64_t>((mnpk + 255) / 256, 1024), 256, 0, st>>>(
        mnpk, B > 0 ? (int)grid : 0, workspace, grad_u, accumulate);
    if (check_launch("bucket project_transpose_u reduce")) return 2;
  }
  return 0;
}

template <typename T>
int mix(int64_t B, int32_t P, int32_t K, int32_t I, int32_t O, const T* y, const T* w, const T* gates, T* out,
        int32_t accumulate, hipStream_t st) {
  const Dims d{B, I, 0, 0, P, K, O};
  if (check_dims(d, false)) return 1;
  if (B == 0) return 0;
  const dim3 grid((unsigned)((B * K + 127) / 128), (unsigned)((O + 127) / 128));
  mix_kernel<T, false><<<grid, 256, 0, st>>>(d, y, w, gates, nullptr, out, accumulate);
  return check_launch("bucket mix") ? 2 : 0;
}

template <typename T>
int mix_transpose_g(int64_t B, int32_t P, int32_t K, int32_t I, int32_t O, const T* grad_out, const T* y, const T* w,
                    T* grad_g, int32_t accumulate, hipStream_t st) {
  const Dims d{B, I, 0, 0, P, K, O};
  if (check_dims(d, false)) return 1;
  if (B == 0) return 0;
  const int BB = 128 / K;
  const dim3 grid((unsigned)((B + BB - 1) / BB), (unsigned)P);
  mix_kernel<T, true><<<grid, 256, 0, st>>>(d, y, w, nullptr, grad_out, grad_g, accumulate);
  return check_launch("bucket mix_transpose_g") ? 2 : 0;
}

int64_t mix_tw_splits(int64_t B, int32_t P, int32_t K, int32_t I, int32_t O, int64_t* rows_per_split) {
  const int64_t R = std::max<int64_t>(B * K, 1);
  const int64_t tiles = (int64_t)P * ((O + 127) / 128) * ((I + 127) / 128);
  const int64_t want = std::max<int64_t>(1, 2048 / tiles);
  int64_t rps = std::max<int64_t>(256, (R + want - 1) / want);
  rps = (rps + 15) / 16 * 16;
  *rows_per_split = rps;
  return (R + rps - 1) / rps;
}

int mix_workspace(int64_t B, int32_t P, int32_t K, int32_t I, int32_t O, int64_t* workspace_elems) {
  const Dims d{B, I, 0, 0, P, K, O};
  if (check_dims(d, false)) return 1;
  int64_t rps;
  const int64_t ns = mix_tw_splits(B, P, K, I, O, &rps);
  *workspace_elems = std::max<int64_t>(ns * P * (int64_t)O * I, (int64_t)P * O * I);
  return 0;
}

template <typename T>
int mix_transpose_y(int64_t B, int32_t P, int32_t K, int32_t I, int32_t O, const T* grad_out, const T* w,
                    const T* gates, T* grad_y, int32_t accumulate, T* workspace, hipStream_t st) {
  const Dims d{B, I, 0, 0, P, K, O};
  if (check_dims(d, false)) return 1;
  if (B == 0) return 0;
  const int64_t nw = (int64_t)P * O * I;
  transpose_w_kernel<T><<<(unsigned)std::min<int64_t>((nw + 255) / 256, 4096), 256, 0, st>>>(P, O, I, w, workspace);
  if (check_launch("bucket transpose_w")) return 2;
  const dim3 grid((unsigned)((B * K + 127) / 128), (unsigned)(P * ((I + 127) / 128)));
  mix_ty_kernel<T><<<grid, 256, 0, st>>>(d, grad_out, workspace, gates, grad_y, accumulate);
  return check_launch("bucket mix_transpose_y") ? 2 : 0;
}

template <typename T>
int mix_transpose_w(int64_t B, int32_t P, int32_t K, int32_t I, int32_t O, const T* grad_out, const T* y,
                    const T* gates, T* grad_w, int32_t accumulate, T* workspace, hipStream_t st) {
  const Dims d{B, I, 0, 0, P, K, O};
  if (check_dims(d, false)) return 1;
  const int64_t nw = (int64_t)P * O * I;
  if (B == 0) {   // a sum over zero parts
    sum_parts_kernel<T><<<(unsigned)std::min<int64_t>((nw + 255) / 256, 4096), 256, 0, st>>>(nw, 0, workspace, grad_w,
                                                                                           accumulate);
    return check_launch("bucket mix_transpose_w") ? 2 : 0;
  }
  int64_t rps;
  const int64_t ns = mix_tw_splits(B, P, K, I, O, &rps);
  const dim3 grid((unsigned)ns, (unsigned)P, (unsigned)(((O + 127) / 128) * ((I + 127) / 128)));
  mix_tw_kernel<T><<<grid, 256, 0, st>>>(d, grad_out, y, gates, rps, workspace);
  if (check_launch("bucket mix_transpose_w")) return 2;
  sum_parts_kernel<T><<<(unsigned)std::min<int64_t>((nw + 255) / 256, 4096), 256, 0, st>>>(nw, (int)ns, workspace,
                                                                                         grad_w, accumulate);
  return check_launch("bucket mix_transpose_w reduce") ? 2 : 0;
}

}  // namespace bucket
}  // namespace fsc

// ===================================================================== C ABI
// fsc_bucket_<op> takes float arrays, fsc_bucket_<op>_f64 double arrays; workspaces are counted in
// elements of the op's type.
using namespace fsc;

#define FSC_BUCKET_ABI(SUF, T)                                                                                        \
  extern "C" int fsc_bucket_project##SUF(int64_t B, int32_t I, int32_t m1, int32_t m2, int32_t P, int32_t K,        \
                                         const T* a, const T* v, const T* u, T* y, int32_t accumulate,               \
                                         hipStream_t st) {                                                          \
    return bucket::project<T>(B, I, m1, m2, P, K, a, v, u, y, accumulate, st);                                      \
  }                                                                                                                  \
  extern "C" int fsc_bucket_project_transpose_a##SUF(int64_t B, int32_t I, int32_t m1, int32_t m2, int32_t P,       \
                                                     int32_t K, const T* grad_y, const T* v, const T* u, T* grad_a,  \
                                                     int32_t accumulate, hipStream_t st) {                          \
    return bucket::project_transpose_a<T>(B, I, m1, m2, P, K, grad_y, v, u, grad_a, accumulate, st);                \
  }                                                                                                                  \
  extern "C" int fsc_bucket_project_transpose_vu##SUF(int64_t B, int32_t I, int32_t m1, int32_t m2, int32_t P,      \
                                                      int32_t K, const T* grad_y, const T* a, const T* v,           \
                                                      const T* u, T* grad_v, T* grad_u, int32_t accumulate,         \
                                                      T* workspace, hipStream_t st) {                               \
    return bucket::project_transpose_vu<T>(B, I, m1, m2, P, K, grad_y, a, v, u, grad_v, grad_u, accumulate,         \
                                           workspace, st);                                                          \
  }                                                                                                                  \
  extern "C" int fsc_bucket_mix##SUF(int64_t B, int32_t P, int32_t K, int32_t I, int32_t O, const T* y, const T* w, \
                                     const T* gates, T* out, int32_t accumulate, hipStream_t st) {                  \
    return bucket::mix<T>(B, P, K, I, O, y, w, gates, out, accumulate, st);                                         \
  }                                                                                                                  \
  extern "C" int fsc_bucket_mix_transpose_g##SUF(int64_t B, int32_t P, int32_t K, int32_t I, int32_t O,             \
                                                 const T* grad_out, const T* y, const T* w, T* grad_g,              \
                                                 int32_t accumulate, hipStream_t st) {                              \
    return bucket::mix_transpose_g<T>(B, P, K, I, O, grad_out, y, w, grad_g, accumulate, st);                       \
  }                                                                                                                  \
  extern "C" int fsc_bucket_mix_transpose_y##SUF(int64_t B, int32_t P, int32_t K, int32_t I, int32_t O,             \
                                                 const T* grad_out, const T* w, const T* gates, T* grad_y,          \
                                                 int32_t accumulate, T* workspace, hipStream_t st) {                \
    return bucket::mix_transpose_y<T>(B, P, K, I, O, grad_out, w, gates, grad_y, accumulate, workspace, st);        \
  }                                                                                                                  \
  extern "C" int fsc_bucket_mix_transpose_w##SUF(int64_t B, int32_t P, int32_t K, int32_t I, int32_t O,             \
                                                 const T* grad_out, const T* y, const T* gates, T* grad_w,          \
                                                 int32_t accumulate, T* workspace, hipStream_t st) {                \
    return bucket::mix_transpose_w<T>(B, P, K, I, O, grad_out, y, gates, grad_w, accumulate, workspace, st);        \
  }

FSC_BUCKET_ABI(, float)
FSC_BUCKET_ABI(_f64, double)
#undef FSC_BUCKET_ABI

extern "C" int fsc_bucket_project_workspace(int64_t B, int32_t I, int32_t m1, int32_t m2, int32_t P, int32_t K,
                                            int64_t* workspace_floats) {
  return bucket::project_workspace(B, I, m1, m2, P, K, workspace_floats);
}

extern "C" int fsc_bucket_mix_workspace(int64_t B, int32_t P, int32_t K, int32_t I, int32_t O, int64_t* workspace_floats) {
  return bucket::mix_workspace(B, P, K, I, O, workspace_floats);
}
