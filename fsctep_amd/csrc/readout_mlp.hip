// Readout head of the energy: per atom, input LayerNorm -> NH x [Linear -> LayerNorm -> SiLU] -> Linear(O)
// -> weighted sum of the O outputs (reference models/mlp.py:8-66 MainNet, :117-133 RobustScalarWeightedSum),
// in one kernel, and its input gradient in one more (the forward recomputed in registers).
//
// Folded weights (prepare_kernel, once per call): with the input LayerNorm x^ = (x - mu) rs, y0 = x^ g0 + b0,
// the first layer is z1 = rs (W1g (x - mu)) + c1 with W1g = W1 diag(g0) and c1 = W1 b0 + bias1, and the
// output layer and weighted sum collapse to e = v . a_NH + e0 with v = Wout^T w, e0 = w . bout.  The input
// gradient of the input LayerNorm needs the row means of g = W1g^T dz1 and of g x^; both follow from
// H-vectors the block already holds: sum_k g[k] = dz1 . u1 (u1 = W1 g0, row sums of W1g) and
// sum_k g[k] x^[k] = rs dz1 . zc1 (zc1 = W1g (x - mu), the first product before its row scale).
//
// A block takes 16 atoms (rows) with 4 waves; wave w owns the hidden columns [16 NT w, 16 NT (w + 1)) of
// every layer (H = 64 NT).  Products run on v_mfma_f32_16x16x4_f32 (fp32 throughout): the first layer's
// reads the atom rows from HBM (centred on the fly) and W1g from L2; the hidden layers' read the previous
// activations from LDS.  LayerNorm statistics are two-pass (mean, then the mean square deviation), each a
// 16-lane shuffle reduction plus a fixed-order sum over the four waves' LDS partials.
#include <algorithm>

#include "common.h"
#include "fsctep.h"

namespace fsc {
namespace mlp {

constexpr int ROWS = 16;       // atoms per block
constexpr int NTHREADS = 256;  // 4 waves
constexpr int APAD = 4;        // LDS row padding of the activation tiles (floats)
constexpr int MAXH = 4;        // hidden layers

// Offsets (floats) of the folded-weight buffer; every section a multiple of 4 floats long.  The product
// operands are stored tiled in MFMA operand order: the B operand of output columns [16 T, 16 T + 16) and
// reduction indices [16 c, 16 c + 16) is the 256-float block ((T KC + c) 64 + lane) 4 + j holding
// M[16 T + lane % 16][16 c + 4 (lane / 16) + j] (KC blocks along the reduction, zero past the matrix), so a
// wave's operand load reads 1 KB of contiguous memory.
struct Layout {
  int64_t w1f, w1b, c1, u1, lng[MAXH], lnb[MAXH], wf[MAXH], wb[MAXH], b[MAXH], v, e0, total;
};

__host__ __device__ inline int chunks16(int k) { return (k + 15) / 16; }

__host__ __device__ inline Layout layout_of(int K, int H, int NH) {
  Layout L{};
  int64_t o = 0;
  const int64_t Kp = 16 * (int64_t)chunks16(K);
  L.w1f = o; o += (int64_t)H * Kp;   // W1 diag(g0): output columns H, reduction K
  L.w1b = o; o += Kp * H;            // its transpose: output columns K, reduction H
  L.c1 = o;   o += H;                // W1 b0 + bias1
  L.u1 = o;   o += H;                // W1 g0
  for (int l = 0; l < NH; ++l) { L.lng[l] = o; o += H; L.lnb[l] = o; o += H; }
  for (int l = 1; l < NH; ++l) {
    L.wf[l] = o; o += (int64_t)H * H;  // W_l: output columns H (out), reduction H (in)
    L.wb[l] = o; o += (int64_t)H * H;  // W_l^T
    L.b[l] = o;  o += H;
  }
  L.v = o;  o += H;
  L.e0 = o; o += 4;
  L.total = o;
  return L;
}

// The module parameters.  Every field is read with a constant index (a runtime index into a kernel
// argument array makes the compiler copy the array to scratch memory in every thread).
struct Params {
  const float *g0, *b0;                                   // input LayerNorm
  const float *W[MAXH], *bias[MAXH], *lg[MAXH], *lb[MAXH];  // hidden layers
  const float *Wo, *bo, *ws;                              // output Linear, weighted-sum weights
};

// Blocks [0, H): the row reductions of hidden unit h (c1, u1 over the K inputs, v over the O outputs), a
// 256-thread block each; block H: e0; the other blocks copy and transpose, grid-stride.
template <int NH>
__global__ __launch_bounds__(256) void prepare_kernel(Params P, int K, int H, int O, float* __restrict__ out) {
  const Layout L = layout_of(K, H, NH);
  const float* g0 = P.g0;
  const float* b0 = P.b0;
  const float* W1 = P.W[0];
  const float* Wo = P.Wo;
  const float* bo = P.bo;
  const float* ws = P.ws;
  __shared__ float part[3][256 / 64];
  if ((int)blockIdx.x <= H) {
    const int h = blockIdx.x;
    float c = 0.f, u = 0.f, v = 0.f;
    if (h < H) {
      for (int k = threadIdx.x; k < K; k += 256) {
        const float w = W1[(int64_t)h * K + k];
        c += w * b0[k];
        u += w * g0[k];
      }
      for (int o = threadIdx.x; o < O; o += 256) v += ws[o] * Wo[(int64_t)o * H + h];
    } else {
      for (int o = threadIdx.x; o < O; o += 256) c += ws[o] * bo[o];
    }
    c = wave_sum(c);
    u = wave_sum(u);
    v = wave_sum(v);
    if ((threadIdx.x & 63) == 0) {
      part[0][threadIdx.x >> 6] = c;
      part[1][threadIdx.x >> 6] = u;
      part[2][threadIdx.x >> 6] = v;
    }
    __syncthreads();
    if (threadIdx.x == 0) {
      c = (part[0][0] + part[0][1]) + (part[0][2] + part[0][3]);
      u = (part[1][0] + part[1][1]) + (part[1][2] + part[1][3]);
      v = (part[2][0] + part[2][1]) + (part[2][2] + part[2][3]);
      if (h < H) {
        out[L.c1 + h] = c + P.bias[0][h];
        out[L.u1 + h] = u;
        out[L.v + h] = v;
      } else {
        out[L.e0] = c;
        out[L.e0 + 1] = out[L.e0 + 2] = out[L.e0 + 3] = 0.f;
      }
    }
    return;
  }
  // every index below 2^31 (K <= 2^20, H <= 256): 32-bit arithmetic
  const int tid = (int)(blockIdx.x - H - 1) * (int)blockDim.x + (int)threadIdx.x;
  const int nth = (int)(gridDim.x - H - 1) * (int)blockDim.x;
  const int kc = chunks16(K), hc = H / 16;
  // tiled operands, written in order: entry i is M[n][k] of tile i / 256
  for (int i = tid; i < H * 16 * kc; i += nth) {
    const int blk = i >> 8, l = (i >> 2) & 63, j = i & 3;
    const int T = blk / kc, c = blk - T * kc;
    const int n = 16 * T + (l & 15), k = 16 * c + 4 * (l >> 4) + j;
    out[L.w1f + i] = k < K ? W1[n * K + k] * g0[k] : 0.f;   // n < H
  }
  for (int i = tid; i < 16 * kc * H; i += nth) {
    const int blk = i >> 8, l = (i >> 2) & 63, j = i & 3;
    const int T = blk / hc, c = blk - T * hc;
    const int n = 16 * T + (l & 15), k = 16 * c + 4 * (l >> 4) + j;   // n: input column, k: hidden unit
    out[L.w1b + i] = n < K ? W1[k * K + n] * g0[n] : 0.f;
  }
#pragma unroll
  for (int l = 0; l < NH; ++l) {
    const float* lg = P.lg[l];
    const float* lb = P.lb[l];
    for (int h = tid; h < H; h += nth) {
      out[L.lng[l] + h] = lg[h];
      out[L.lnb[l] + h] = lb[h];
    }
  }
#pragma unroll
  for (int l = 1; l < NH; ++l) {
    const float* W = P.W[l];
    const float* bias = P.bias[l];
    for (int i = tid; i < H * H; i += nth) {
      const int blk = i >> 8, ln = (i >> 2) & 63, j = i & 3;
      const int T = blk / hc, c = blk - T * hc;
      const int n = 16 * T + (ln & 15), k = 16 * c + 4 * (ln >> 4) + j;
      out[L.wf[l] + i] = W[n * H + k];
      out[L.wb[l] + i] = W[k * H + n];
    }
    for (int h = tid; h < H; h += nth) out[L.b[l] + h] = bias[h];
  }
}

__device__ __forceinline__ f4 splat(float v) { return f4{v, v, v, v}; }

__device__ __forceinline__ void buffer_st1(__amdgpu_buffer_rsrc_t rsrc, uint32_t byte_off, float v) {
  __builtin_amdgcn_raw_buffer_store_b32(__builtin_bit_cast(unsigned, v), rsrc, (int)byte_off, 0, 0);
}

// Buffer resource over the block's rows of an [n][K] array (at most ROWS * K * 4 < 2^32 bytes): loads at
// kDropOffset return 0 and stores there are dropped, so the product loops run without branches and keep
// their loads in flight across the MFMAs.
__device__ __forceinline__ __amdgpu_buffer_rsrc_t rows_rsrc(const float* base, int64_t n, int K) {
  const int64_t r0 = (int64_t)blockIdx.x * ROWS;
  const int64_t rows = n - r0 < ROWS ? n - r0 : ROWS;
  return buffer_rsrc(const_cast<float*>(base) + r0 * K, (uint32_t)(rows * K * 4));
}

// s[j]: this wave's partial of row 4q + j (q = lane / 16) in every lane of the row group; returns the
// block's full row sums (all 4 waves, fixed order), identical in every lane.  red: [2][4][ROWS] floats;
// the two slots alternate so that a reduction's writes never meet the previous one's reads.
__device__ __forceinline__ f4 rows_total(f4 s, float* red, int& slot) {
#pragma unroll
  for (int off = 1; off < 16; off <<= 1) {
    s.x += __shfl_xor(s.x, off, 64);
    s.y += __shfl_xor(s.y, off, 64);
    s.z += __shfl_xor(s.z, off, 64);
    s.w += __shfl_xor(s.w, off, 64);
  }
  const int w = threadIdx.x >> 6, lane = threadIdx.x & 63, q = lane >> 4;
  float* base = red + slot * 4 * ROWS;
  if ((lane & 15) == 0) st4(base + w * ROWS + 4 * q, s);
  __syncthreads();
  const f4 t = ((ld4(base + 4 * q) + ld4(base + ROWS + 4 * q)) + ld4(base + 2 * ROWS + 4 * q)) +
               ld4(base + 3 * ROWS + 4 * q);
  slot ^= 1;
  return t;
}

template <int NT>
struct Smem {
  // act[0], act[1]: activations of consecutive layers; dz: the backward's LayerNorm gradients; the three
  // also carry the first product's partial sums between the waves
  float buf[3][ROWS][64 * NT + APAD];
  float red[2 * 4 * ROWS];
  float ssp[4][ROWS];
  float mu0[ROWS];
  float rs0[ROWS];
};

// LayerNorm over the H columns of each row, then SiLU: z (rows 4q + j, columns col0 + 16 t + r) in,
// activations to act (LDS), normalised values and the row scales kept for the backward.
template <int NT>
__device__ __forceinline__ void ln_silu(const f4 (&z)[NT], const float* __restrict__ lng,
                                        const float* __restrict__ lnb, float eps, int col0, float* red, int& slot,
                                        float (*act)[64 * NT + APAD], f4 (&yhat)[NT], f4& rs) {
  constexpr int H = 64 * NT;
  const int lane = threadIdx.x & 63, r = lane & 15, q = lane >> 4;
  f4 s = splat(0.f);
#pragma unroll
  for (int t = 0; t < NT; ++t) s += z[t];
  const f4 mu = rows_total(s, red, slot) * (1.f / H);
  f4 s2 = splat(0.f);
#pragma unroll
  for (int t = 0; t < NT; ++t) {
    const f4 d = z[t] - mu;
    s2 += d * d;
  }
  const f4 var = rows_total(s2, red, slot) * (1.f / H);
  rs = f4{rsqrtf(var.x + eps), rsqrtf(var.y + eps), rsqrtf(var.z + eps), rsqrtf(var.w + eps)};
#pragma unroll
  for (int t = 0; t < NT; ++t) {
    const int col = col0 + 16 * t + r;
    const float g = lng[col], b = lnb[col];
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const float yh = (z[t][j] - mu[j]) * rs[j];
      const float y = yh * g + b;
      yhat[t][j] = yh;
      act[4 * q + j][col] = y / (1.f + expf(-y));
    }
  }
}

// acc[t] = A[16][H] (LDS rows) times B^T, B an H x H matrix stored tiled (output column tiles col0 / 16 + t).
template <int NT>
__device__ __forceinline__ void gemm_lds(const float (*A)[64 * NT + APAD], const float* __restrict__ B, int col0,
                                         f4 (&acc)[NT]) {
  constexpr int H = 64 * NT;
  const int lane = threadIdx.x & 63, r = lane & 15, q = lane >> 4;
#pragma unroll
  for (int t = 0; t < NT; ++t) acc[t] = splat(0.f);
#pragma unroll(NT <= 2 ? H / 16 : 4)
  for (int c = 0; c < H / 16; ++c) {
    const int k = 16 * c + 4 * q;
    const f4 a = ld4(&A[r][k]);
    f4 b[NT];
#pragma unroll
    for (int t = 0; t < NT; ++t) b[t] = ld4(B + ((int64_t)((col0 >> 4) + t) * (H / 16) + c) * 256 + 4 * lane);
#pragma unroll
    for (int t = 0; t < NT; ++t) acc[t] = mfma_k16(a, b[t], acc[t]);
  }
}

// The forward through the hidden layers for the block's rows.  Leaves the last activations in
// sm.buf[(NH - 1) & 1], and (for the backward) the first product before its row scale (zc1), every
// layer's normalised values and row scales, and the input row means / scales in sm.mu0 / sm.rs0.
template <int NH, int NT>
__device__ __forceinline__ void forward_rows(const FscMlpDims& d, int64_t n, const float* __restrict__ x,
                                             const float* __restrict__ P, Smem<NT>& sm, int& slot, f4 (&zc1)[NT],
                                             f4 (&yhat)[NH][NT], f4 (&rs)[NH]) {
  constexpr int H = 64 * NT;
  const Layout L = layout_of(d.K, H, NH);
  const int K = d.K;
  const int w = threadIdx.x >> 6, lane = threadIdx.x & 63, r = lane & 15, q = lane >> 4;
  const int col0 = 16 * NT * w;
  const int64_t r0 = (int64_t)blockIdx.x * ROWS;
  const int kc = chunks16(K);

  const __amdgpu_buffer_rsrc_t xres = rows_rsrc(x, n, K);
  // input row means: 16 threads per row, eight loads in flight per thread
  {
    const int rr = threadIdx.x >> 4, c16 = threadIdx.x & 15;
    const bool rowv = r0 + rr < n;
    float s = 0.f;
    for (int k0 = 4 * c16; k0 < K; k0 += 64 * 8) {
      f4 v[8];
#pragma unroll
      for (int u = 0; u < 8; ++u) {
        const int k = k0 + 64 * u;
        v[u] = buffer_ld4(xres, (rowv && k < K) ? (uint32_t)(rr * K + k) * 4u : kDropOffset, 0);
      }
#pragma unroll
      for (int u = 0; u < 8; ++u) s += (v[u].x + v[u].y) + (v[u].z + v[u].w);
    }
#pragma unroll
    for (int off = 1; off < 16; off <<= 1) s += __shfl_xor(s, off, 64);
    if (c16 == 0) sm.mu0[rr] = s / K;
  }
  __syncthreads();

  // first layer, split over K between the waves: wave w takes the 16-deep chunks c = w, w + 4, ... for all
  // H columns (acc[t]: columns 16 t + r, rows 4q + j); lane (r, q) streams row r of x (centred where it lies
  // inside the row) and the tiled W1g blocks, two chunks in flight (register double buffer).  The partial
  // sums then meet in LDS: each wave adds the other three waves' partials of its own columns.
  {
    constexpr int TT = 4 * NT;
    const bool rv = r0 + r < n;
    const float mu = sm.mu0[r];
    const __amdgpu_buffer_rsrc_t wres = buffer_rsrc(const_cast<float*>(P + L.w1f), (uint32_t)(H * kc * 64));
    f4 acc[TT];
#pragma unroll
    for (int t = 0; t < TT; ++t) acc[t] = splat(0.f);
    float ss = 0.f;
    auto load = [&](int c, f4& xa, f4 (&wb)[TT]) {
      const int k = 16 * c + 4 * q;
      xa = buffer_ld4(xres, (rv && k < K) ? (uint32_t)(r * K + k) * 4u : kDropOffset, 0);
#pragma unroll
      for (int t = 0; t < TT; ++t)
        wb[t] = buffer_ld4(wres, c < kc ? (uint32_t)((t * kc + c) * 256 + 4 * lane) * 4u : kDropOffset, 0);
    };
    auto mma = [&](int c, const f4& xa, const f4 (&wb)[TT]) {
      const int k = 16 * c + 4 * q;
      const f4 a = xa - splat((rv && k < K) ? mu : 0.f);
      ss += (a.x * a.x + a.y * a.y) + (a.z * a.z + a.w * a.w);
#pragma unroll
      for (int t = 0; t < TT; ++t) acc[t] = mfma_k16(a, wb[t], acc[t]);
    };
    if constexpr (NT <= 2) {
      // the scheduling barriers keep each chunk's loads ahead of the other chunk's MFMAs, so that the waits
      // before an MFMA group leave the next chunk's loads in flight
      f4 xa0, wb0[TT], xa1, wb1[TT];
      load(w, xa0, wb0);
      for (int c = w; c < kc; c += 8) {
        load(c + 4, xa1, wb1);
        __builtin_amdgcn_sched_barrier(0);
        mma(c, xa0, wb0);
        __builtin_amdgcn_sched_barrier(0);
        load(c + 8, xa0, wb0);
        __builtin_amdgcn_sched_barrier(0);
        mma(c + 4, xa1, wb1);
        __builtin_amdgcn_sched_barrier(0);
      }
    } else {
      for (int c = w; c < kc; c += 4) {
        f4 xa, wb[TT];
        load(c, xa, wb);
        mma(c, xa, wb);
      }
    }
    ss += __shfl_xor(ss, 16, 64);
    ss += __shfl_xor(ss, 32, 64);
    // partials of column group g (wave g's columns) to slot (w - g + 3) mod 4
#pragma unroll
    for (int g = 0; g < 4; ++g) {
      if (g == w) continue;
      float (*dst)[64 * NT + APAD] = sm.buf[(w - g + 3) & 3];
#pragma unroll
      for (int tt = 0; tt < NT; ++tt)
#pragma unroll
        for (int j = 0; j < 4; ++j) dst[4 * q + j][16 * (g * NT + tt) + r] = acc[g * NT + tt][j];
    }
    if (q == 0) sm.ssp[w][r] = ss;
    __syncthreads();
    f4 own[NT];
#pragma unroll
    for (int tt = 0; tt < NT; ++tt) {
      own[tt] = acc[tt];
#pragma unroll
      for (int g = 1; g < 4; ++g)
        if (g == w) own[tt] = acc[g * NT + tt];
    }
    const float ssr = (sm.ssp[0][r] + sm.ssp[1][r]) + (sm.ssp[2][r] + sm.ssp[3][r]);
    const float rs_r = rsqrtf(ssr / K + d.eps0);   // row r
    if (w == 0 && q == 0) sm.rs0[r] = rs_r;
    f4 rsq;
#pragma unroll
    for (int j = 0; j < 4; ++j) rsq[j] = __shfl(rs_r, 4 * q + j, 64);
    f4 z[NT];
#pragma unroll
    for (int tt = 0; tt < NT; ++tt) {
      const int col = col0 + 16 * tt + r;
      f4 v = own[tt];
#pragma unroll
      for (int sl = 0; sl < 3; ++sl)
#pragma unroll
        for (int j = 0; j < 4; ++j) v[j] += sm.buf[sl][4 * q + j][col];
      zc1[tt] = v;
      z[tt] = v * rsq + splat(P[L.c1 + col]);
    }
    ln_silu<NT>(z, P + L.lng[0], P + L.lnb[0], d.eps[0], col0, sm.red, slot, sm.buf[0], yhat[0], rs[0]);
  }
#pragma unroll
  for (int l = 1; l < NH; ++l) {
    __syncthreads();   // act[(l - 1) & 1] complete
    f4 z[NT];
    gemm_lds<NT>(sm.buf[(l - 1) & 1], P + L.wf[l], col0, z);
#pragma unroll
    for (int t = 0; t < NT; ++t) z[t] += splat(P[L.b[l] + col0 + 16 * t + r]);
    ln_silu<NT>(z, P + L.lng[l], P + L.lnb[l], d.eps[l], col0, sm.red, slot, sm.buf[l & 1], yhat[l], rs[l]);
  }
  __syncthreads();
}

template <int NH, int NT>
__global__ __launch_bounds__(NTHREADS) void forward_kernel(FscMlpDims d, int64_t n, const float* __restrict__ x,
                                                           const float* __restrict__ P, float* __restrict__ e) {
  constexpr int H = 64 * NT;
  __shared__ Smem<NT> sm;
  int slot = 0;
  f4 zc1[NT], yhat[NH][NT], rs[NH];
  forward_rows<NH, NT>(d, n, x, P, sm, slot, zc1, yhat, rs);
  const Layout L = layout_of(d.K, H, NH);
  const int w = threadIdx.x >> 6, lane = threadIdx.x & 63, r = lane & 15, q = lane >> 4;
  const int col0 = 16 * NT * w;
  f4 s = splat(0.f);
#pragma unroll
  for (int t = 0; t < NT; ++t) {
    const int col = col0 + 16 * t + r;
    const float v = P[L.v + col];
#pragma unroll
    for (int j = 0; j < 4; ++j) s[j] += v * sm.buf[(NH - 1) & 1][4 * q + j][col];
  }
  const f4 tot = rows_total(s, sm.red, slot);
  if (w == 0 && r == 0) {
    const float e0 = P[L.e0];
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const int64_t row = (int64_t)blockIdx.x * ROWS + 4 * q + j;
      if (row < n) e[row] = tot[j] + e0;
    }
  }
}

// dx[row] = ge[row] * de[row]/dx[row].
template <int NH, int NT>
__global__ __launch_bounds__(NTHREADS, NT <= 2 ? 3 : 2) void backward_kernel(FscMlpDims d, int64_t n, const float* __restrict__ x,
                                                            const float* __restrict__ P, const float* __restrict__ ge,
                                                            float* __restrict__ dx) {
  constexpr int H = 64 * NT;
  __shared__ Smem<NT> sm;
  int slot = 0;
  f4 zc1[NT], yhat[NH][NT], rs[NH];
  forward_rows<NH, NT>(d, n, x, P, sm, slot, zc1, yhat, rs);
  const Layout L = layout_of(d.K, H, NH);
  const int K = d.K;
  const int w = threadIdx.x >> 6, lane = threadIdx.x & 63, r = lane & 15, q = lane >> 4;
  const int col0 = 16 * NT * w;
  const int64_t r0 = (int64_t)blockIdx.x * ROWS;

  f4 g4;   // upstream gradient of rows 4q + j
#pragma unroll
  for (int j = 0; j < 4; ++j) g4[j] = (r0 + 4 * q + j < n) ? ge[r0 + 4 * q + j] : 0.f;
  f4 da[NT];
#pragma unroll
  for (int t = 0; t < NT; ++t) da[t] = g4 * splat(P[L.v + col0 + 16 * t + r]);

  f4 dz[NT];
#pragma unroll
  for (int l = NH - 1; l >= 0; --l) {
    // through SiLU and the layer's LayerNorm
    f4 dyh[NT];
    f4 s1 = splat(0.f), s2 = splat(0.f);
#pragma unroll
    for (int t = 0; t < NT; ++t) {
      const int col = col0 + 16 * t + r;
      const float g = P[L.lng[l] + col], b = P[L.lnb[l] + col];
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        const float yh = yhat[l][t][j];
        const float y = yh * g + b;
        const float sg = 1.f / (1.f + expf(-y));
        const float dyv = da[t][j] * (sg * (1.f + y * (1.f - sg))) * g;
        dyh[t][j] = dyv;
        s1[j] += dyv;
        s2[j] += dyv * yh;
      }
    }
    const f4 m1 = rows_total(s1, sm.red, slot) * (1.f / H);
    const f4 m2 = rows_total(s2, sm.red, slot) * (1.f / H);
#pragma unroll
    for (int t = 0; t < NT; ++t) dz[t] = rs[l] * (dyh[t] - m1 - yhat[l][t] * m2);
    if (l > 0) {
      // da_{l-1} = dz_l W_l (rows), B = W_l^T rows
#pragma unroll
      for (int t = 0; t < NT; ++t) {
        const int col = col0 + 16 * t + r;
#pragma unroll
        for (int j = 0; j < 4; ++j) sm.buf[2][4 * q + j][col] = dz[t][j];
      }
      __syncthreads();
      gemm_lds<NT>(sm.buf[2], P + L.wb[l], col0, da);
      // the next layer's reductions (barriers) separate these reads of sm.dz from its next writes
    }
  }

  // input LayerNorm: row means of g = W1g^T dz1 and of g x^, from H-vectors
  f4 s1 = splat(0.f), s2 = splat(0.f);
#pragma unroll
  for (int t = 0; t < NT; ++t) {
    const float u = P[L.u1 + col0 + 16 * t + r];
    s1 += dz[t] * splat(u);
    s2 += dz[t] * zc1[t];
#pragma unroll
    for (int j = 0; j < 4; ++j) sm.buf[2][4 * q + j][col0 + 16 * t + r] = dz[t][j];
  }
  const f4 S1 = rows_total(s1, sm.red, slot);   // barrier: sm.dz complete
  const f4 S2 = rows_total(s2, sm.red, slot);
  f4 mu, rsr;
#pragma unroll
  for (int j = 0; j < 4; ++j) {
    mu[j] = sm.mu0[4 * q + j];
    rsr[j] = sm.rs0[4 * q + j];
  }
  const float invK = 1.f / K;
  const f4 m1 = S1 * invK;
  const f4 m2 = S2 * rsr * invK;

  // g tiles of 16 input columns, wave w takes tiles w, w + 4, ...; dz1 rows held as the A operand
  f4 a[4 * NT];
#pragma unroll
  for (int c = 0; c < 4 * NT; ++c) a[c] = ld4(&sm.buf[2][r][16 * c + 4 * q]);
  const __amdgpu_buffer_rsrc_t gres = buffer_rsrc(const_cast<float*>(P + L.w1b), (uint32_t)(chunks16(K) * H * 64));
  const __amdgpu_buffer_rsrc_t xres = rows_rsrc(x, n, K);
  const __amdgpu_buffer_rsrc_t dres = rows_rsrc(dx, n, K);
  bool rowv[4];
#pragma unroll
  for (int j = 0; j < 4; ++j) rowv[j] = r0 + 4 * q + j < n;
  const int nkt = (K + 15) / 16;
  // tile kt: column kcol = 16 kt + r of g for rows 4q + j; its W1gt row and the x values the input
  // LayerNorm's gradient needs
  auto load = [&](int kt, f4 (&b)[4 * NT], f4& xv) {
    const int kcol = 16 * kt + r;
    const bool cv = kcol < K;
#pragma unroll
    for (int c = 0; c < 4 * NT; ++c)
      b[c] = buffer_ld4(gres, kt < nkt ? (uint32_t)((kt * (H / 16) + c) * 256 + 4 * lane) * 4u : kDropOffset, 0);
#pragma unroll
    for (int j = 0; j < 4; ++j)
      xv[j] = buffer_ld1(xres, (cv && rowv[j]) ? (uint32_t)((4 * q + j) * K + kcol) * 4u : kDropOffset, 0);
  };
  auto tile = [&](int kt, const f4 (&b)[4 * NT], const f4& xv) {
    f4 acc = splat(0.f);
#pragma unroll
    for (int c = 0; c < 4 * NT; ++c) acc = mfma_k16(a[c], b[c], acc);
    const int kcol = 16 * kt + r;
    const bool cv = kcol < K;
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const float xh = (xv[j] - mu[j]) * rsr[j];
      buffer_st1(dres, (cv && rowv[j]) ? (uint32_t)((4 * q + j) * K + kcol) * 4u : kDropOffset,
                 rsr[j] * (acc[j] - m1[j] - xh * m2[j]));
    }
  };
  if constexpr (NT <= 2) {
    // two tiles in flight (register double buffer)
    f4 b0[4 * NT], b1[4 * NT], x0, x1;
    load(w, b0, x0);
    for (int kt = w; kt < nkt; kt += 8) {
      load(kt + 4, b1, x1);
      __builtin_amdgcn_sched_barrier(0);
      tile(kt, b0, x0);
      __builtin_amdgcn_sched_barrier(0);
      load(kt + 8, b0, x0);
      __builtin_amdgcn_sched_barrier(0);
      tile(kt + 4, b1, x1);
      __builtin_amdgcn_sched_barrier(0);
    }
  } else {
    for (int kt = w; kt < nkt; kt += 4) {
      f4 b[4 * NT], xv;
      load(kt, b, xv);
      tile(kt, b, xv);
    }
  }
}

template <int NT, bool BWD>
int launch_nt(const FscMlpDims& d, int64_t n, const float* x, const float* P, const float* ge, float* out,
              hipStream_t st) {
  const dim3 grid((unsigned)((n + ROWS - 1) / ROWS));
#define FSC_MLP_CASE(NHV)                                                                              \
  case NHV:                                                                                            \
    if (BWD)                                                                                           \
      hipLaunchKernelGGL((backward_kernel<NHV, NT>), grid, dim3(NTHREADS), 0, st, d, n, x, P, ge, out); \
    else                                                                                               \
      hipLaunchKernelGGL((forward_kernel<NHV, NT>), grid, dim3(NTHREADS), 0, st, d, n, x, P, out);      \
    break;
  switch (d.NH) {
    FSC_MLP_CASE(1)
    FSC_MLP_CASE(2)
    FSC_MLP_CASE(3)
    FSC_MLP_CASE(4)
    default: FSC_CHECK_ARG(false, "readout mlp: hidden layer count out of range");
  }
#undef FSC_MLP_CASE
  return check_launch(BWD ? "readout_mlp_backward" : "readout_mlp_forward");
}

int check_dims(const FscMlpDims* d, const char* what) {
  FSC_CHECK_ARG(d, std::string(what) + ": null dims");
  FSC_CHECK_ARG(d->K >= 4 && d->K % 4 == 0 && d->K <= (1 << 20),
                std::string(what) + ": input width must be a positive multiple of 4 (at most 2^20)");
  FSC_CHECK_ARG(d->H == 64 || d->H == 128 || d->H == 256,
                std::string(what) + ": hidden width must be 64, 128 or 256 (all hidden layers alike)");
  FSC_CHECK_ARG(d->NH >= 1 && d->NH <= MAXH, std::string(what) + ": 1 to 4 hidden layers");
  FSC_CHECK_ARG(d->O >= 1 && d->O <= 4096, std::string(what) + ": output width out of range");
  FSC_CHECK_ARG(d->eps0 > 0.f, std::string(what) + ": LayerNorm eps must be positive");
  for (int l = 0; l < d->NH; ++l) FSC_CHECK_ARG(d->eps[l] > 0.f, std::string(what) + ": LayerNorm eps must be positive");
  return 0;
}

bool aligned16(const void* p) { return ((uintptr_t)p & 15) == 0; }

int run(const FscMlpDims* d, int64_t n, const float* x, const float* P, const float* ge, float* out, bool bwd,
        hipStream_t st) {
  const char* what = bwd ? "fsc_readout_mlp_backward" : "fsc_readout_mlp_forward";
  if (check_dims(d, what)) return 1;
  FSC_CHECK_ARG(n >= 0 && n < (1LL << 31), std::string(what) + ": bad atom count");
  if (n == 0) return 0;
  FSC_CHECK_ARG(x && P && out && (!bwd || ge), std::string(what) + ": null pointer");
  FSC_CHECK_ARG(aligned16(x) && aligned16(P) && (!bwd || aligned16(out)),
                std::string(what) + ": x, the folded weights and dx must be 16-byte aligned");
  LaunchTimer timer("readout_mlp", st);
  switch (d->H) {
    case 64: return bwd ? launch_nt<1, true>(*d, n, x, P, ge, out, st) : launch_nt<1, false>(*d, n, x, P, ge, out, st);
    case 128: return bwd ? launch_nt<2, true>(*d, n, x, P, ge, out, st) : launch_nt<2, false>(*d, n, x, P, ge, out, st);
    default: return bwd ? launch_nt<4, true>(*d, n, x, P, ge, out, st) : launch_nt<4, false>(*d, n, x, P, ge, out, st);
  }
}

}  // namespace mlp
}  // namespace fsc

using namespace fsc;

extern "C" {

int fsc_readout_mlp_weights_floats(const FscMlpDims* dims, int64_t* floats) {
  if (mlp::check_dims(dims, "fsc_readout_mlp_weights_floats")) return 1;
  FSC_CHECK_ARG(floats, "fsc_readout_mlp_weights_floats: null output");
  *floats = mlp::layout_of(dims->K, dims->H, dims->NH).total;
  return 0;
}

int fsc_readout_mlp_prepare(const FscMlpDims* dims, const float* const* params, float* weights, hipStream_t stream) {
  if (mlp::check_dims(dims, "fsc_readout_mlp_prepare")) return 1;
  FSC_CHECK_ARG(params && weights, "fsc_readout_mlp_prepare: null pointer");
  const int np = 2 + 4 * dims->NH + 3;
  for (int i = 0; i < np; ++i) FSC_CHECK_ARG(params[i], "fsc_readout_mlp_prepare: null parameter pointer");
  mlp::Params P{};
  P.g0 = params[0];
  P.b0 = params[1];
  for (int l = 0; l < dims->NH; ++l) {
    P.W[l] = params[2 + 4 * l];
    P.bias[l] = params[3 + 4 * l];
    P.lg[l] = params[4 + 4 * l];
    P.lb[l] = params[5 + 4 * l];
  }
  P.Wo = params[2 + 4 * dims->NH];
  P.bo = params[3 + 4 * dims->NH];
  P.ws = params[4 + 4 * dims->NH];
  const int64_t copies = 2 * (int64_t)dims->H * dims->K;
  const unsigned blocks = (unsigned)(dims->H + 1 + std::min<int64_t>((copies + 255) / 256, 1024));
  auto kern = dims->NH == 1 ? mlp::prepare_kernel<1> : dims->NH == 2 ? mlp::prepare_kernel<2>
             : dims->NH == 3 ? mlp::prepare_kernel<3> : mlp::prepare_kernel<4>;
  hipLaunchKernelGGL(kern, dim3(blocks), dim3(256), 0, stream, P, dims->K, dims->H, dims->O, weights);
  return check_launch("readout_mlp_prepare");
}

int fsc_readout_mlp_forward(const FscMlpDims* dims, int64_t n_atoms, const float* x, const float* weights, float* energy,
                            hipStream_t stream) {
  return mlp::run(dims, n_atoms, x, weights, nullptr, energy, false, stream);
}

int fsc_readout_mlp_backward(const FscMlpDims* dims, int64_t n_atoms, const float* x, const float* weights,
                             const float* grad_energy, float* grad_x, hipStream_t stream) {
  return mlp::run(dims, n_atoms, x, weights, grad_energy, grad_x, true, stream);
}

}  // extern "C"
