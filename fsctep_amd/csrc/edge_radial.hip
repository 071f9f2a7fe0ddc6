// Edge geometry and the radial MLP of every interaction layer, fused, with their backward.
//
// Replaces, per call of the reference trunks (models/pure_cartesian_sparse_layers.py:745-756,
// 319-321, 410-412, 204-210, 372-378; models/pure_cartesian_ictd_layers_full.py:896-909,
// 930-937, 277-283, 693-699; models/pure_cartesian_ictd_layers_o3.py:924-936, 953-955):
//   vec = pos[dst] - pos[src] + shift,  r = |vec|,  n = vec / max(r, 1e-8)
//   emb = soft_one_hot_linspace(r, 0, rc, nb, basis, cutoff=True) * sqrt(nb)      (e3nn form)
//   h   = silu(W2 silu(W0 emb + b0) + b2)                                          (fc[:4])
// and the force backward: dr from dh (activations recomputed), dvec from (dn, dr), and
// dpos[m] = sum_{e: dst(e)=m} dvec_e - sum_{e: src(e)=m} dvec_e as two deterministic segmented
// sums over the receiver CSR and the source grouping (no atomics).
#include <type_traits>

#include "common.h"
#include "fsctep.h"

namespace fsc {
namespace radial {

constexpr int HID = 64;     // hidden width of the radial MLP (fixed by the reference's fc)
constexpr int NBMAX = 16;   // radial basis functions supported
constexpr int RADW_RED = 16;   // block-reduction slots (at most 16 waves per block)

// sin x and cos x for 0 <= x < 2^7: Cody-Waite reduction by pi/2 in two parts (the fma keeps
// x - n*P1 to one rounding, and n*(pi/2 - P1 - P2) is below 2^-30 here), then the Taylor series on
// [-pi/4, pi/4] to x^11 / x^12 (truncation below 1e-11) and the quadrant.  The basis argument is at
// most nb*pi; the library sinf/cosf carry a large-argument path whose registers the radial MLP kernels
// cannot spare.
__device__ __forceinline__ void sincos_small(float x, float& s, float& c) {
  constexpr float P1 = 1.57079637050628662109375f;       // pi/2 rounded to float
  constexpr float P2 = -4.37113900018624283e-8f;         // pi/2 - P1
  const float n = rintf(x * 0.636619772367581343f);      // x / (pi/2)
  float t = fmaf(-n, P1, x);
  t = fmaf(-n, P2, t);
  const float t2 = t * t;
  const float sp = t + t * t2 * (-1.f / 6.f + t2 * (1.f / 120.f + t2 * (-1.f / 5040.f + t2 * (1.f / 362880.f +
                                                                      t2 * (-1.f / 39916800.f)))));
  const float cp = 1.f + t2 * (-0.5f + t2 * (1.f / 24.f + t2 * (-1.f / 720.f + t2 * (1.f / 40320.f +
                                                                  t2 * (-1.f / 3628800.f + t2 * (1.f / 479001600.f))))));
  const int qd = ((int)n) & 3;
  s = (qd == 0) ? sp : (qd == 1) ? cp : (qd == 2) ? -sp : -cp;
  c = (qd == 0) ? cp : (qd == 1) ? -sp : (qd == 2) ? -cp : sp;
}

// emb_k(r) and d emb_k / dr for k < nb, e3nn's soft_one_hot_linspace(r, 0, rc, nb, basis, cutoff=True)
// times sqrt(nb), with step = rc/(nb+1), centres mu_k = (k+1)*step and d = (r - mu_k)/step:
//   0 bessel         sqrt(2/rc) sin((k+1) pi r/rc)/r                     on 0 < r < rc
//   1 gaussian       exp(-d^2)/1.12
//   2 fourier        sin((k+1) pi r/rc)/sqrt(0.25 + nb/2)                on 0 < r < rc
//   3 cosine         cos(pi d/2)                                         on |d| < 1
//   4 smooth_finite  1.14136 e^2 exp(-1/(1+d)) exp(-1/(1-d)) = 1.14136 e^2 exp(-2/(1-d^2))   on |d| < 1
template <bool DERIV>
__device__ __forceinline__ void basis_eval(float r, int k, int nb, float rc, int basis, float& f, float& df) {
  const float snb = sqrtf((float)nb);
  if (basis == 0 || basis == 2) {
    const float w = (float)(k + 1) * (3.14159265358979323846f / rc);
    const bool inside = (r / rc < 1.f) && (r > 0.f);
    const float rr = inside ? r : 1.f;
    const float x = w * rr;
    float s, c;
    sincos_small(x, s, c);
    if (basis == 2) {
      const float a = snb * rsqrtf(0.25f + 0.5f * (float)nb);
      f = inside ? a * s : 0.f;
      if (DERIV) df = inside ? a * w * c : 0.f;
      return;
    }
    const float a = sqrtf(2.f / rc) * snb;
    f = inside ? a * s / rr : 0.f;
    if (DERIV) {
      // d/dr sin(wr)/r = w^2 (x cos x - sin x)/x^2; below x = 0.3 the Taylor series avoids the
      // cancellation (-x/3 + x^3/30 - x^5/840, truncation below 1e-8 relative)
      const float x2 = x * x;
      const float g = (x < 0.3f) ? x * (-1.f / 3.f + x2 * (1.f / 30.f - x2 * (1.f / 840.f))) : (x * c - s) / x2;
      df = inside ? a * w * w * g : 0.f;
    }
    return;
  }
  const float step = rc / (float)(nb + 1);
  const float d = (r - (float)(k + 1) * step) / step;
  if (basis == 1) {
    const float e = expf(-d * d) / 1.12f * snb;
    f = e;
    if (DERIV) df = e * (-2.f * d / step);
  } else if (basis == 3) {
    const bool inside = (d < 1.f) && (d > -1.f);
    float s, c;
    sincos_small(fminf(fabsf(d), 2.f) * 1.57079632679489662f, s, c);
    f = inside ? c * snb : 0.f;
    if (DERIV) df = inside ? -copysignf(s, d) * (1.57079632679489662f / step) * snb : 0.f;
  } else {
    const bool inside = (d < 1.f) && (d > -1.f);
    const float q = inside ? 1.f - d * d : 1.f;
    const float e = inside ? 1.14136f * 7.38905609893065023f * expf(-2.f / q) * snb : 0.f;
    f = e;
    if (DERIV) df = e * (-4.f * d / (q * q)) / step;
  }
}

// logistic sigmoid with the hardware exp2 and reciprocal (relative error ~1e-7)
__device__ __forceinline__ float sigm(float x) { return __fdividef(1.f, 1.f + __expf(-x)); }

// One wave per 16-edge tile; lane (r, q) works for edge e0 + r.  The hidden units are laid
// out as the MFMA output: lane (r, q) holds unit j = 16*jt + 4*q + i in register (jt, i), so
// one layer's output is directly the next product's B operand.
// The first layer (K = nb <= 16) runs on the fp32 MFMA from W0 [64][NBMAX + 1] (rows padded so the 64 lanes'
// reads of one K step fall in distinct banks) and, in the backward, W0^T [NBMAX][68] (rows padded so the four
// K values a lane needs come in one 16-byte read).  The 64-wide layers
// (W2, the optional last Linear W4 with up to 64 outputs, and their transposes in the backward) run on
// v_mfma_f32_16x16x32_f16 with fp32-accurate split-fp16 products (mfma_x3, common.h): each layer's weights
// are staged in LDS as two fp16 planes of W sw (one power of two per layer from max |W|), in the K order of
// the activations a lane holds, so the activations need no exchange: K step s takes units
// 32 s + 4 q + j (j < 4) and 32 s + 16 + 4 q + j - 4 (j >= 4), i.e. registers jt = 2s and 2s + 1.  The
// activations of an edge (its 64 units sit in the four lanes (r, 0..3)) get one power of two per edge.
constexpr int WS = HID + 4;
constexpr int HS = HID + 8;   // fp16 row stride of a layer's planes (144 bytes)
struct LayerH16 {
  _Float16 p[2][HID][HS];     // [plane][output row][K slot]
};
struct NoLayer {};
template <bool BWD>
struct Smem {
  float w0[HID][NBMAX + 1];
  float w0t[BWD ? NBMAX : 1][WS];
  LayerH16 w2;                                      // W2 (forward product; recomputed in the backward)
  std::conditional_t<BWD, LayerH16, NoLayer> w2t;   // W2^T (backward)
  LayerH16 w4;                                      // W4 in the forward, W4^T in the backward
  float b0[HID];
  float b2[HID];
  float b4[HID];
  float winv[3];                // 1/sw of w2, w2t, w4
  float red[RADW_RED];
};

// K slot of hidden unit u in a layer's planes
__host__ __device__ constexpr int kslot(int u) {
  return 32 * (u >> 5) + 8 * ((u >> 2) & 3) + 4 * ((u >> 4) & 1) + (u & 3);
}

// Planes of M (64 rows o, 64 columns u): p[h/l][o][kslot(u)] = split of M[o][u] sw, sw from the block's max
// |M|; returns 1/sw (all threads).  get(o, u) reads M.
template <typename Get>
__device__ float stage_h16(LayerH16& L, float* red, Get get) {
  float mx = 0.f;
  for (int i = threadIdx.x; i < HID * HID; i += blockDim.x) mx = fmaxf(mx, fabsf(get(i / HID, i % HID)));
  for (int off = 32; off > 0; off >>= 1) mx = fmaxf(mx, __shfl_xor(mx, off, 64));
  __syncthreads();   // red is free (a previous call's readers are done)
  if ((threadIdx.x & 63) == 0) red[threadIdx.x >> 6] = mx;
  __syncthreads();
  mx = 0.f;
  for (int w = 0; w < (int)(blockDim.x >> 6); ++w) mx = fmaxf(mx, red[w]);
  const float sw = pow2_scale(mx);
  for (int i = threadIdx.x; i < HID * HID; i += blockDim.x) {
    const int o = i / HID, u = i % HID;
    const float v = get(o, u) * sw;
    const _Float16 h = (_Float16)v;
    L.p[0][o][kslot(u)] = h;
    L.p[1][o][kslot(u)] = (_Float16)(v - (float)h);
  }
  return 1.f / sw;   // exact: a power of two
}

template <bool BWD>
__device__ void stage_weights(Smem<BWD>& sm, const float* __restrict__ W0, const float* __restrict__ b0,
                              const float* __restrict__ W2, const float* __restrict__ b2,
                              const float* __restrict__ W4, const float* __restrict__ b4, int nb, int nout) {
  for (int i = threadIdx.x; i < HID * NBMAX; i += blockDim.x) {
    const int j = i / NBMAX, k = i % NBMAX;
    const float v = (k < nb) ? W0[j * nb + k] : 0.f;
    sm.w0[j][k] = v;
    if (BWD) sm.w0t[k][j] = v;
  }
  for (int i = threadIdx.x; i < HID; i += blockDim.x) {
    sm.b0[i] = b0[i];
    sm.b2[i] = b2[i];
    sm.b4[i] = (W4 && i < nout && b4) ? b4[i] : 0.f;
  }
  const float w2i = stage_h16(sm.w2, sm.red, [&](int o, int u) { return W2[o * HID + u]; });
  float w2ti = 1.f, w4i = 1.f;
  if constexpr (BWD) w2ti = stage_h16(sm.w2t, sm.red, [&](int o, int u) { return W2[u * HID + o]; });
  if (W4) {
    if constexpr (BWD)   // W4^T [64 hidden][nout], zero columns beyond nout
      w4i = stage_h16(sm.w4, sm.red, [&](int o, int u) { return u < nout ? W4[u * HID + o] : 0.f; });
    else
      w4i = stage_h16(sm.w4, sm.red, [&](int o, int u) { return o < nout ? W4[o * HID + u] : 0.f; });
  }
  if (threadIdx.x == 0) {
    sm.winv[0] = w2i;
    sm.winv[1] = w2ti;
    sm.winv[2] = w4i;
  }
}

__device__ __forceinline__ f4 lds4(const float* p) { return *reinterpret_cast<const f4*>(p); }

// out = W x + b for a 64-wide layer on split-fp16 MFMA: x in the MFMA layout (x[jt][i] = unit 16 jt + 4 q + i
// of the lane's edge r); the edge's activations scaled by a power of two from their max |x| over the four
// lanes of the edge and split once; A operand row r of output tile ot reads K slots 8q .. 8q + 7 of
// W row 16 ot + r from both planes; both scales undone on the fp32 result.
__device__ __forceinline__ void dense64(const LayerH16& W, float winv, const float* b, const f4 (&x)[4], int r,
                                        int q, f4 (&out)[4]) {
  float mx = 0.f;
#pragma unroll
  for (int jt = 0; jt < 4; ++jt)
#pragma unroll
    for (int i = 0; i < 4; ++i) mx = fmaxf(mx, fabsf(x[jt][i]));
  mx = fmaxf(mx, __shfl_xor(mx, 16, 64));
  mx = fmaxf(mx, __shfl_xor(mx, 32, 64));
  const float sx = pow2_scale(mx);
  h8 xh[2], xl[2];
#pragma unroll
  for (int st = 0; st < 2; ++st) {
    const float v[8] = {x[2 * st][0] * sx, x[2 * st][1] * sx, x[2 * st][2] * sx, x[2 * st][3] * sx,
                        x[2 * st + 1][0] * sx, x[2 * st + 1][1] * sx, x[2 * st + 1][2] * sx, x[2 * st + 1][3] * sx};
    split2h_pk(v, xh[st], xl[st]);
  }
  const float f = winv / sx;   // exact: powers of two
#pragma unroll
  for (int ot = 0; ot < 4; ++ot) {
    f4 acc = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int st = 0; st < 2; ++st) {
      const h8 wh = *reinterpret_cast<const h8*>(&W.p[0][16 * ot + r][32 * st + 8 * q]);
      const h8 wl = *reinterpret_cast<const h8*>(&W.p[1][16 * ot + r][32 * st + 8 * q]);
      acc = mfma_x3(wh, wl, xh[st], xl[st], acc);
    }
#pragma unroll
    for (int i = 0; i < 4; ++i) acc[i] = acc[i] * f + (b ? b[16 * ot + 4 * q + i] : 0.f);
    out[ot] = acc;
    __builtin_amdgcn_sched_barrier(0);
  }
}

// u0 = W0 emb + b0 for the lane's edge (MFMA layout above).
template <bool BWD>
__device__ __forceinline__ void first_layer(const Smem<BWD>& sm, const float (&emb)[NBMAX / 4], int nks, int r, int q,
                                            f4 (&u0)[4]) {
#pragma unroll
  for (int jt = 0; jt < 4; ++jt) {
    f4 acc = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int ks = 0; ks < NBMAX / 4; ++ks)
      if (ks < nks) acc = mfma16x16x4(sm.w0[16 * jt + r][4 * ks + q], emb[ks], acc);
#pragma unroll
    for (int i = 0; i < 4; ++i) acc[i] += sm.b0[16 * jt + 4 * q + i];
    u0[jt] = acc;
    __builtin_amdgcn_sched_barrier(0);
  }
}

// u0 = W0 emb + b0 and u2 = W2 silu(u0) + b2 for the lane's edge (MFMA layout above).
template <bool BWD>
__device__ __forceinline__ void mlp_forward(const Smem<BWD>& sm, const float (&emb)[NBMAX / 4], int nks, int r, int q,
                                            f4 (&u0)[4], f4 (&u2)[4]) {
  first_layer(sm, emb, nks, r, q, u0);
  f4 a0[4];
#pragma unroll
  for (int jt = 0; jt < 4; ++jt)
#pragma unroll
    for (int i = 0; i < 4; ++i) a0[jt][i] = u0[jt][i] * sigm(u0[jt][i]);
  dense64(sm.w2, sm.winv[0], sm.b2, a0, r, q, u2);
}

// The basis values a lane feeds to the first product: emb[4*ks + q] for ks < nks (lane group q).
__device__ __forceinline__ void lane_basis(float rr, int nb, float rc, int basis, int q, float (&emb)[NBMAX / 4]) {
#pragma unroll
  for (int ks = 0; ks < NBMAX / 4; ++ks) {
    const int k = 4 * ks + q;
    float f = 0.f, df = 0.f;
    if (k < nb) basis_eval<false>(rr, k, nb, rc, basis, f, df);
    emb[ks] = f;
  }
}

// d emb_k / dr for the lane's rows k = 4q + i of the d-emb tile (zero for k >= nb).
__device__ __forceinline__ void lane_basis_deriv(float rr, int nb, float rc, int basis, int q, float (&demb)[4]) {
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const int k = 4 * q + i;
    float f = 0.f, df = 0.f;
    if (k < nb) basis_eval<true>(rr, k, nb, rc, basis, f, df);
    demb[i] = df;
  }
}

// Blocks of RAD_WAVES waves share one LDS copy of the weights; two blocks per CU give 4 waves per SIMD
// (at most 128 VGPRs), enough to overlap the dependent layers of one 16-edge tile with other tiles.
constexpr int RAD_WAVES = 8;

__global__ __launch_bounds__(64 * RAD_WAVES, 4) void radial_mlp_forward_kernel(const float* __restrict__ rad, const float* __restrict__ W0,
                                                                 const float* __restrict__ b0, const float* __restrict__ W2,
                                                                 const float* __restrict__ b2, const float* __restrict__ W4,
                                                                 const float* __restrict__ b4, int nout, int nb, float rc,
                                                                 int basis, int64_t n_edges, float* __restrict__ h) {
  __shared__ Smem<false> sm;
  stage_weights(sm, W0, b0, W2, b2, W4, b4, nb, nout);
  __syncthreads();
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int r = lane & 15, q = lane >> 4;
  const int nks = (nb + 3) / 4;
  const int64_t ntiles = (n_edges + 15) / 16, tstride = (int64_t)gridDim.x * RAD_WAVES;
  // each tile's radii are requested one tile ahead
  auto radius = [&](int64_t t) { return (t < ntiles && 16 * t + r < n_edges) ? rad[16 * t + r] : 1.f; };
  float rr_next = radius((int64_t)blockIdx.x * RAD_WAVES + wave);
  for (int64_t t = (int64_t)blockIdx.x * RAD_WAVES + wave; t < ntiles; t += tstride) {
    const int64_t e = 16 * t + r;
    const float rr = rr_next;
    rr_next = radius(t + tstride);
    float emb[NBMAX / 4];
    lane_basis(rr, nb, rc, basis, q, emb);
    f4 u0[4], u2[4], a2[4];
    mlp_forward(sm, emb, nks, r, q, u0, u2);
#pragma unroll
    for (int ot = 0; ot < 4; ++ot)
#pragma unroll
      for (int i = 0; i < 4; ++i) a2[ot][i] = u2[ot][i] * sigm(u2[ot][i]);
    if (W4) {
      f4 o[4];
      dense64(sm.w4, sm.winv[2], sm.b4, a2, r, q, o);
      if (e < n_edges) {
#pragma unroll
        for (int ot = 0; ot < 4; ++ot)
#pragma unroll
          for (int i = 0; i < 4; ++i) {
            const int j = 16 * ot + 4 * q + i;
            if (j < nout) h[e * nout + j] = o[ot][i];
          }
      }
    } else if (e < n_edges) {
#pragma unroll
      for (int ot = 0; ot < 4; ++ot) st4(h + e * HID + 16 * ot + 4 * q, a2[ot]);
    }
  }
}

// dr[e] = sum_k d emb_k/dr * (W0^T (silu'(u0) * W2^T (silu'(u2) * dh)))_k, with dh = W4^T dout when the
// last Linear is fused.
__global__ __launch_bounds__(64 * RAD_WAVES, 4) void radial_mlp_backward_kernel(const float* __restrict__ rad, const float* __restrict__ W0,
                                                                  const float* __restrict__ b0, const float* __restrict__ W2,
                                                                  const float* __restrict__ b2, const float* __restrict__ W4,
                                                                  int nout, int nb, float rc, int basis, int64_t n_edges,
                                                                  const float* __restrict__ dout, float* __restrict__ dr) {
  __shared__ Smem<true> sm;
  stage_weights(sm, W0, b0, W2, b2, W4, nullptr, nb, nout);
  __syncthreads();
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int r = lane & 15, q = lane >> 4;
  const int nks = (nb + 3) / 4;
  const int64_t ntiles = (n_edges + 15) / 16;
  for (int64_t t = (int64_t)blockIdx.x * RAD_WAVES + wave; t < ntiles; t += (int64_t)gridDim.x * RAD_WAVES) {
    const int64_t e = 16 * t + r;
    const bool ok = e < n_edges;
    const float rr = ok ? rad[e] : 1.f;
    float emb[NBMAX / 4];
    lane_basis(rr, nb, rc, basis, q, emb);
    f4 u2[4];
    {
      f4 u0[4];   // recomputed below rather than held across the two 64-wide products (register pressure)
      mlp_forward(sm, emb, nks, r, q, u0, u2);
    }
    f4 dh[4];
    if (W4) {
      f4 d[4];
#pragma unroll
      for (int ot = 0; ot < 4; ++ot)
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          const int j = 16 * ot + 4 * q + i;
          d[ot][i] = (ok && j < nout) ? dout[e * nout + j] : 0.f;
        }
      dense64(sm.w4, sm.winv[2], nullptr, d, r, q, dh);
    } else {
#pragma unroll
      for (int ot = 0; ot < 4; ++ot) dh[ot] = ok ? ld4(dout + e * HID + 16 * ot + 4 * q) : f4{0.f, 0.f, 0.f, 0.f};
    }
    f4 g2[4];
#pragma unroll
    for (int ot = 0; ot < 4; ++ot)
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const float s = sigm(u2[ot][i]);
        g2[ot][i] = dh[ot][i] * s * (1.f + u2[ot][i] * (1.f - s));
      }
    f4 da0[4], g0[4], u0[4];
    dense64(sm.w2t, sm.winv[1], nullptr, g2, r, q, da0);
    first_layer(sm, emb, nks, r, q, u0);
#pragma unroll
    for (int jt = 0; jt < 4; ++jt)
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const float s = sigm(u0[jt][i]);
        g0[jt][i] = da0[jt][i] * s * (1.f + u0[jt][i] * (1.f - s));
      }
    // d emb[k] for k = 4q + i (rows k of one 16-row tile; k >= nb rows are zero)
    f4 de = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int jt = 0; jt < 4; ++jt) {
      const f4 a = lds4(&sm.w0t[r][16 * jt + 4 * q]);
#pragma unroll
      for (int i = 0; i < 4; ++i) de = mfma16x16x4(a[i], g0[jt][i], de);
    }
    float demb[4];   // formed here, not held across the products
    lane_basis_deriv(rr, nb, rc, basis, q, demb);
    float part = 0.f;
#pragma unroll
    for (int i = 0; i < 4; ++i) part += de[i] * demb[i];
    part += __shfl_xor(part, 16, 64);
    part += __shfl_xor(part, 32, 64);
    if (ok && q == 0) dr[e] = part;
  }
}

// ---------------------------------------------------------------- geometry
__global__ void geometry_forward_kernel(const float* __restrict__ pos, const float* __restrict__ shift,
                                        const int32_t* __restrict__ src, const int32_t* __restrict__ dst,
                                        int64_t n_edges, float* __restrict__ nvec, float* __restrict__ rad) {
  const int64_t e = blockIdx.x * (int64_t)blockDim.x + threadIdx.x;
  if (e >= n_edges) return;
  const int64_t s = src[e], d = dst[e];
  float v[3];
#pragma unroll
  for (int k = 0; k < 3; ++k) v[k] = pos[3 * d + k] - pos[3 * s + k] + shift[3 * e + k];
  const float r = sqrtf(v[0] * v[0] + v[1] * v[1] + v[2] * v[2]);
  const float inv = 1.f / fmaxf(r, 1e-8f);
#pragma unroll
  for (int k = 0; k < 3; ++k) nvec[3 * e + k] = v[k] * inv;
  rad[e] = r;
}

// dvec_e = dr_e n_e + (dn_e - (n_e . dn_e) n_e) / r_e  (for r_e > 1e-8; below it n = vec/1e-8)
__device__ __forceinline__ void edge_dvec(const float* __restrict__ gn, const float* __restrict__ gr,
                                          const float* __restrict__ nvec, const float* __restrict__ rad,
                                          int64_t e, float (&dv)[3]) {
  const float r = rad[e];
  const float n0 = nvec[3 * e], n1 = nvec[3 * e + 1], n2 = nvec[3 * e + 2];
  const float d0 = gn ? gn[3 * e] : 0.f, d1 = gn ? gn[3 * e + 1] : 0.f, d2 = gn ? gn[3 * e + 2] : 0.f;
  const float dr = gr ? gr[e] : 0.f;
  if (r > 1e-8f) {
    const float dot = n0 * d0 + n1 * d1 + n2 * d2;
    const float ir = 1.f / r;
    dv[0] = dr * n0 + (d0 - dot * n0) * ir;
    dv[1] = dr * n1 + (d1 - dot * n1) * ir;
    dv[2] = dr * n2 + (d2 - dot * n2) * ir;
  } else {
    const float rr = fmaxf(r, 1e-30f);
    dv[0] = dr * n0 * 1e-8f / rr + d0 * 1e8f;
    dv[1] = dr * n1 * 1e-8f / rr + d1 * 1e8f;
    dv[2] = dr * n2 * 1e-8f / rr + d2 * 1e8f;
  }
}

// One wave per atom: its in-edges (receiver CSR) add dvec, its out-edges (source grouping) subtract.
__global__ __launch_bounds__(256) void geometry_backward_kernel(const float* __restrict__ gn, const float* __restrict__ gr,
                                                                const float* __restrict__ nvec,
                                                                const float* __restrict__ rad,
                                                                const int32_t* __restrict__ dst_ptr,
                                                                const int32_t* __restrict__ src_ptr,
                                                                const int32_t* __restrict__ src_perm,
                                                                int64_t n_nodes, float* __restrict__ gpos) {
  const int lane = threadIdx.x & 63;
  const int64_t m = (int64_t)blockIdx.x * 4 + (threadIdx.x >> 6);
  if (m >= n_nodes) return;
  float acc[3] = {0.f, 0.f, 0.f};
  for (int e = dst_ptr[m] + lane; e < dst_ptr[m + 1]; e += 64) {
    float dv[3];
    edge_dvec(gn, gr, nvec, rad, e, dv);
#pragma unroll
    for (int k = 0; k < 3; ++k) acc[k] += dv[k];
  }
  for (int j = src_ptr[m] + lane; j < src_ptr[m + 1]; j += 64) {
    float dv[3];
    edge_dvec(gn, gr, nvec, rad, src_perm[j], dv);
#pragma unroll
    for (int k = 0; k < 3; ++k) acc[k] -= dv[k];
  }
#pragma unroll
  for (int k = 0; k < 3; ++k) acc[k] = wave_sum(acc[k]);
  if (lane == 0) {
#pragma unroll
    for (int k = 0; k < 3; ++k) gpos[3 * m + k] = acc[k];
  }
}

// Geometry from caller-supplied edge vectors (input edge order) read through the receiver-sort
// permutation `order`; the backward writes grad_vec in the input order (each edge once: no atomics).
__global__ void vec_geometry_forward_kernel(const float* __restrict__ vec, const int32_t* __restrict__ order,
                                            int64_t n_edges, float* __restrict__ nvec, float* __restrict__ rad) {
  const int64_t e = blockIdx.x * (int64_t)blockDim.x + threadIdx.x;
  if (e >= n_edges) return;
  const int64_t i = order[e];
  const float v0 = vec[3 * i], v1 = vec[3 * i + 1], v2 = vec[3 * i + 2];
  const float r = sqrtf(v0 * v0 + v1 * v1 + v2 * v2);
  const float inv = 1.f / fmaxf(r, 1e-8f);
  nvec[3 * e] = v0 * inv;
  nvec[3 * e + 1] = v1 * inv;
  nvec[3 * e + 2] = v2 * inv;
  rad[e] = r;
}

__global__ void vec_geometry_backward_kernel(const float* __restrict__ gn, const float* __restrict__ gr,
                                             const float* __restrict__ nvec, const float* __restrict__ rad,
                                             const int32_t* __restrict__ order, int64_t n_edges,
                                             float* __restrict__ gvec) {
  const int64_t e = blockIdx.x * (int64_t)blockDim.x + threadIdx.x;
  if (e >= n_edges) return;
  float dv[3];
  edge_dvec(gn, gr, nvec, rad, e, dv);
  const int64_t i = order[e];
#pragma unroll
  for (int k = 0; k < 3; ++k) gvec[3 * i + k] = dv[k];
}

// ---------------------------------------------------------------- direction harmonics (ICTD)
// Y[e][l^2 + m] = sum_{k of degree l} M[k][m] n_x^a n_y^b n_z^c (M = multinomial * G_l B_l, the
// ICTD harmonic basis); backward dn = sum_k (sum_m dY[l^2+m] M[k][m]) grad(n^abc).  One thread
// per edge, 256 edges per block; the table travels as a kernel argument.  The block's rows of Y (dY)
// are one contiguous run of 256 (lmax+1)^2 floats, moved between HBM and LDS by all threads in order
// (coalesced) and read or written per edge from LDS (rows padded to 17 floats).
constexpr int HARM_ROW = 17;

__device__ __forceinline__ void harm_powers(const float* __restrict__ nvec, int64_t e, float (&px)[4], float (&py)[4],
                                            float (&pz)[4]) {
  px[0] = py[0] = pz[0] = 1.f;
  const float x = nvec[3 * e], y = nvec[3 * e + 1], z = nvec[3 * e + 2];
#pragma unroll
  for (int i = 1; i < 4; ++i) {
    px[i] = px[i - 1] * x;
    py[i] = py[i - 1] * y;
    pz[i] = pz[i - 1] * z;
  }
}

// Monomials n_x^a n_y^b n_z^c of degree l = a + b + c <= 3 in a fixed order: by l, then r = b + c, then c.
__device__ __forceinline__ int harm_canon(int a, int b, int c) {
  const int l = a + b + c, r = b + c;
  return l * (l + 1) * (l + 2) / 6 + r * (r + 1) / 2 + c;
}

// The table as a dense [20 monomials (fixed order)][16 outputs] matrix in LDS, zero where a monomial is
// absent or its degree is not the output's l, so that the per-edge loops are straight-line code with
// the exponents known at compile time.  Ends with a barrier.
__device__ __forceinline__ void stage_harm_matrix(const FscHarmTable& tab, f4 (&Mt)[20][4]) {
  float* m = reinterpret_cast<float*>(Mt);
  for (int i = threadIdx.x; i < 20 * 16; i += blockDim.x) m[i] = 0.f;
  __syncthreads();
  for (int i = threadIdx.x; i < tab.nmono * 16; i += blockDim.x) {
    const int k = i >> 4, j = i & 15;
    const int a = tab.mono_exp[k][0], b = tab.mono_exp[k][1], c = tab.mono_exp[k][2];
    const int l = tab.mono_l[k], jj = j - l * l;
    if (a >= 0 && b >= 0 && c >= 0 && a + b + c == l && l <= 3 && jj >= 0 && jj < 2 * l + 1)
      m[harm_canon(a, b, c) * 16 + j] = tab.coef[k][jj];
  }
  __syncthreads();
}

__global__ __launch_bounds__(256) void harmonics_forward_kernel(FscHarmTable tab, int64_t n_edges,
                                                                const float* __restrict__ nvec,
                                                                float* __restrict__ Y) {
  __shared__ float rows[256 * HARM_ROW];
  __shared__ f4 Mt[20][4];
  const int64_t e0 = (int64_t)blockIdx.x * 256;
  const int64_t e = e0 + threadIdx.x;
  const int ny = (tab.lmax + 1) * (tab.lmax + 1);
  const int nb = (int)min((int64_t)256, n_edges - e0);   // edges of this block (uniform)
  stage_harm_matrix(tab, Mt);
  if (e < n_edges) {
    float px[4], py[4], pz[4];
    harm_powers(nvec, e, px, py, pz);
    f4 out[4];
#pragma unroll
    for (int i = 0; i < 4; ++i) out[i] = f4{0.f, 0.f, 0.f, 0.f};
    int ck = 0;
#pragma unroll
    for (int l = 0; l < 4; ++l)
#pragma unroll
      for (int r = 0; r <= l; ++r)
#pragma unroll
        for (int c = 0; c <= r; ++c, ++ck) {
          const float m = px[l - r] * py[r - c] * pz[c];
#pragma unroll
          for (int i = 0; i < 4; ++i) out[i] += m * Mt[ck][i];
        }
#pragma unroll
    for (int j = 0; j < 16; ++j) rows[threadIdx.x * HARM_ROW + j] = out[j >> 2][j & 3];
  }
  __syncthreads();
  float* yb = Y + e0 * ny;
  for (int i = threadIdx.x; i < nb * ny; i += 256) {
    const int r = i / ny;
    yb[i] = rows[r * HARM_ROW + (i - r * ny)];
  }
}

__global__ __launch_bounds__(256) void harmonics_backward_kernel(FscHarmTable tab, int64_t n_edges,
                                                                 const float* __restrict__ nvec,
                                                                 const float* __restrict__ dY,
                                                                 float* __restrict__ dn) {
  __shared__ float rows[256 * HARM_ROW];
  __shared__ f4 Mt[20][4];
  const int64_t e0 = (int64_t)blockIdx.x * 256;
  const int64_t e = e0 + threadIdx.x;
  const int ny = (tab.lmax + 1) * (tab.lmax + 1);
  const int nb = (int)min((int64_t)256, n_edges - e0);
  const float* gb = dY + e0 * ny;
  for (int i = threadIdx.x; i < nb * ny; i += 256) {
    const int r = i / ny;
    rows[r * HARM_ROW + (i - r * ny)] = gb[i];
  }
  stage_harm_matrix(tab, Mt);   // its barriers also publish rows
  if (e >= n_edges) return;
  float px[4], py[4], pz[4];
  harm_powers(nvec, e, px, py, pz);
  f4 g[4];
#pragma unroll
  for (int j = 0; j < 16; ++j) g[j >> 2][j & 3] = (j < ny) ? rows[threadIdx.x * HARM_ROW + j] : 0.f;
  float d[3] = {0.f, 0.f, 0.f};
  int ck = 0;
#pragma unroll
  for (int l = 0; l < 4; ++l)
#pragma unroll
    for (int r = 0; r <= l; ++r)
#pragma unroll
      for (int c = 0; c <= r; ++c, ++ck) {
        const int a = l - r, b = r - c;
        f4 t = g[0] * Mt[ck][0];
#pragma unroll
        for (int i = 1; i < 4; ++i) t += g[i] * Mt[ck][i];
        const float dm = (t[0] + t[1]) + (t[2] + t[3]);
        if (a) d[0] += dm * (float)a * px[a - 1] * py[b] * pz[c];
        if (b) d[1] += dm * (float)b * px[a] * py[b - 1] * pz[c];
        if (c) d[2] += dm * (float)c * px[a] * py[b] * pz[c - 1];
      }
#pragma unroll
  for (int i = 0; i < 3; ++i) dn[3 * e + i] = d[i];
}

}  // namespace radial
}  // namespace fsc

using namespace fsc;
using namespace fsc::radial;

extern "C" {

int fsc_edge_geometry_forward(int64_t n_edges, const float* pos, const float* shift, const int32_t* edge_src,
                              const int32_t* edge_dst, float* n_out, float* r_out, hipStream_t stream) {
  FSC_CHECK_ARG(n_edges >= 0 && n_edges < (1LL << 31), "fsc_edge_geometry_forward: bad size");
  if (n_edges == 0) return 0;
  FSC_CHECK_ARG(pos && shift && edge_src && edge_dst && n_out && r_out, "fsc_edge_geometry_forward: null pointer");
  geometry_forward_kernel<<<(unsigned)((n_edges + 255) / 256), 256, 0, stream>>>(pos, shift, edge_src, edge_dst,
                                                                                 n_edges, n_out, r_out);
  return check_launch("edge geometry forward") ? 2 : 0;
}

int fsc_edge_geometry_backward(int64_t n_nodes, int64_t n_edges, const float* grad_n, const float* grad_r,
                               const float* n, const float* r, const int32_t* dst_ptr, const int32_t* src_ptr,
                               const int32_t* src_perm, float* grad_pos, hipStream_t stream) {
  FSC_CHECK_ARG(n_nodes >= 0 && n_edges >= 0 && n_nodes < (1LL << 31) && n_edges < (1LL << 31),
                "fsc_edge_geometry_backward: bad size");
  if (n_nodes == 0) return 0;
  FSC_CHECK_ARG(dst_ptr && src_ptr && grad_pos, "fsc_edge_geometry_backward: null pointer");
  FSC_CHECK_ARG(n_edges == 0 || (n && r && src_perm), "fsc_edge_geometry_backward: null edge pointer");
  geometry_backward_kernel<<<(unsigned)((n_nodes + 3) / 4), 256, 0, stream>>>(grad_n, grad_r, n, r, dst_ptr,
                                                                              src_ptr, src_perm, n_nodes, grad_pos);
  return check_launch("edge geometry backward") ? 2 : 0;
}

int fsc_edge_vec_geometry_forward(int64_t n_edges, const float* edge_vec, const int32_t* order, float* n_out,
                                  float* r_out, hipStream_t stream) {
  FSC_CHECK_ARG(n_edges >= 0 && n_edges < (1LL << 31), "fsc_edge_vec_geometry_forward: bad size");
  if (n_edges == 0) return 0;
  FSC_CHECK_ARG(edge_vec && order && n_out && r_out, "fsc_edge_vec_geometry_forward: null pointer");
  vec_geometry_forward_kernel<<<(unsigned)((n_edges + 255) / 256), 256, 0, stream>>>(edge_vec, order, n_edges,
                                                                                     n_out, r_out);
  return check_launch("edge vector geometry forward") ? 2 : 0;
}

int fsc_edge_vec_geometry_backward(int64_t n_edges, const float* grad_n, const float* grad_r, const float* n,
                                   const float* r, const int32_t* order, float* grad_vec, hipStream_t stream) {
  FSC_CHECK_ARG(n_edges >= 0 && n_edges < (1LL << 31), "fsc_edge_vec_geometry_backward: bad size");
  if (n_edges == 0) return 0;
  FSC_CHECK_ARG(n && r && order && grad_vec, "fsc_edge_vec_geometry_backward: null pointer");
  vec_geometry_backward_kernel<<<(unsigned)((n_edges + 255) / 256), 256, 0, stream>>>(grad_n, grad_r, n, r, order,
                                                                                      n_edges, grad_vec);
  return check_launch("edge vector geometry backward") ? 2 : 0;
}

static unsigned radial_grid(int64_t n_edges) {
  const int64_t tiles = (n_edges + 15) / 16;
  // two blocks per CU: the weights are staged in LDS once per block
  return (unsigned)std::max<int64_t>(1, std::min<int64_t>((tiles + RAD_WAVES - 1) / RAD_WAVES, 512));
}

int fsc_radial_mlp_forward(int64_t n_edges, const float* r, const float* w0, const float* b0, const float* w2,
                           const float* b2, const float* w4, const float* b4, int32_t n_out, int32_t n_basis,
                           float r_cut, int32_t basis, float* out, hipStream_t stream) {
  FSC_CHECK_ARG(n_edges >= 0 && n_edges < (1LL << 31), "fsc_radial_mlp_forward: bad size");
  FSC_CHECK_ARG(n_basis >= 1 && n_basis <= NBMAX, "fsc_radial_mlp_forward: n_basis must be 1..16");
  FSC_CHECK_ARG(basis >= 0 && basis <= 4, "fsc_radial_mlp_forward: basis must be 0..4 (bessel, gaussian, fourier, cosine, smooth_finite)");
  FSC_CHECK_ARG(r_cut > 0.f, "fsc_radial_mlp_forward: r_cut must be positive");
  FSC_CHECK_ARG(!w4 || (b4 && n_out >= 1 && n_out <= HID), "fsc_radial_mlp_forward: last Linear needs 1..64 outputs");
  if (n_edges == 0) return 0;
  FSC_CHECK_ARG(r && w0 && b0 && w2 && b2 && out, "fsc_radial_mlp_forward: null pointer");
  LaunchTimer tm("radial_mlp", stream);
  radial_mlp_forward_kernel<<<radial_grid(n_edges), 64 * RAD_WAVES, 0, stream>>>(r, w0, b0, w2, b2, w4, b4, w4 ? n_out : HID,
                                                                     n_basis, r_cut, basis, n_edges, out);
  return check_launch("radial mlp forward") ? 2 : 0;
}

int fsc_radial_mlp_backward(int64_t n_edges, const float* r, const float* w0, const float* b0, const float* w2,
                            const float* b2, const float* w4, int32_t n_out, int32_t n_basis, float r_cut,
                            int32_t basis, const float* grad_out, float* grad_r, hipStream_t stream) {
  FSC_CHECK_ARG(n_edges >= 0 && n_edges < (1LL << 31), "fsc_radial_mlp_backward: bad size");
  FSC_CHECK_ARG(n_basis >= 1 && n_basis <= NBMAX, "fsc_radial_mlp_backward: n_basis must be 1..16");
  FSC_CHECK_ARG(basis >= 0 && basis <= 4, "fsc_radial_mlp_backward: basis must be 0..4 (bessel, gaussian, fourier, cosine, smooth_finite)");
  FSC_CHECK_ARG(r_cut > 0.f, "fsc_radial_mlp_backward: r_cut must be positive");
  FSC_CHECK_ARG(!w4 || (n_out >= 1 && n_out <= HID), "fsc_radial_mlp_backward: last Linear needs 1..64 outputs");
  if (n_edges == 0) return 0;
  FSC_CHECK_ARG(r && w0 && b0 && w2 && b2 && grad_out && grad_r, "fsc_radial_mlp_backward: null pointer");
  LaunchTimer tm("radial_mlp_grad", stream);
  radial_mlp_backward_kernel<<<radial_grid(n_edges), 64 * RAD_WAVES, 0, stream>>>(r, w0, b0, w2, b2, w4, w4 ? n_out : HID,
                                                                      n_basis, r_cut, basis, n_edges, grad_out, grad_r);
  return check_launch("radial mlp backward") ? 2 : 0;
}


int fsc_edge_harmonics_forward(const FscHarmTable* table, int64_t n_edges, const float* n, float* Y,
                               hipStream_t stream) {
  FSC_CHECK_ARG(table && table->lmax >= 0 && table->lmax <= 3 && table->nmono >= 1 && table->nmono <= 20,
                "fsc_edge_harmonics_forward: table must describe lmax <= 3 with at most 20 monomials");
  FSC_CHECK_ARG(n_edges >= 0 && n_edges < (1LL << 31), "fsc_edge_harmonics_forward: bad size");
  if (n_edges == 0) return 0;
  FSC_CHECK_ARG(n && Y, "fsc_edge_harmonics_forward: null pointer");
  harmonics_forward_kernel<<<(unsigned)((n_edges + 255) / 256), 256, 0, stream>>>(*table, n_edges, n, Y);
  return check_launch("edge harmonics forward") ? 2 : 0;
}

int fsc_edge_harmonics_backward(const FscHarmTable* table, int64_t n_edges, const float* n, const float* grad_Y,
                                float* grad_n, hipStream_t stream) {
  FSC_CHECK_ARG(table && table->lmax >= 0 && table->lmax <= 3 && table->nmono >= 1 && table->nmono <= 20,
                "fsc_edge_harmonics_backward: table must describe lmax <= 3 with at most 20 monomials");
  FSC_CHECK_ARG(n_edges >= 0 && n_edges < (1LL << 31), "fsc_edge_harmonics_backward: bad size");
  if (n_edges == 0) return 0;
  FSC_CHECK_ARG(n && grad_Y && grad_n, "fsc_edge_harmonics_backward: null pointer");
  harmonics_backward_kernel<<<(unsigned)((n_edges + 255) / 256), 256, 0, stream>>>(*table, n_edges, n, grad_Y,
                                                                                   grad_n);
  return check_launch("edge harmonics backward") ? 2 : 0;
}

}  // extern "C"
