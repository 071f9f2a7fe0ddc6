// ICTD (harmonic-irreps) message passing on gfx950: pure-cartesian-ictd and -ictd-o3.
//
// Replaces HarmonicFullyConnectedTensorProduct[O3].forward + receiver scatter of the conv2..n
// loop (models/ictd_irreps.py:971-1253, :1512-1695; models/pure_cartesian_ictd_layers_full.py:938-954,
// models/pure_cartesian_ictd_layers_o3.py:956-973) and the TP of conv1 (:341-473 / :424-532).
//
// Algebra (exact; only summation order changes).  For a live path p = (k1 = (l1,p1), Y_l2 -> k3):
//   out_n[k3][o][m3] = (1/deg n) sum_{e->n} gate_e[p] sum_i W[p][o][i] sum_{m1,m2} x_src[k1][i][m1] Y_e[l2][m2] C_p[m1][m2][m3]
// The channel mix W is linear, so it moves after the receiver sum:
//   BG_e[p][m1][m3] = gate_e[p] sum_m2 Y_e[l2][m2] C_p[m1][m2][m3]                      (per edge, LDS)
//   Z_n[kk][i]      = (1/deg) sum_{e->n} sum_m1 BG_e[p(kk)][m1][kk] x_src[o1+m1][i]     (MFMA, K = edges x m1)
//   out_n[k3][m3][o]= sum_{p->k3} sum_i W[p][o][i] Z_n[koff_p+m3][i]                    (MFMA, per node)
// Paths are grouped by first-operand key (their kk ranges are contiguous); each group's kk range is
// padded to 16-wide tiles.  Backward, with g = dZ / deg:
//   DX_e[o1+m1][i]  = sum_kk BG_e[m1][kk] g[kk][i]      -> summed per source (deterministic, no atomics)
//   H_e[m1][kk]     = sum_i x_src[o1+m1][i] g[kk][i]    -> dgate_e[p], dY_e (contractions with C_p)
// Layouts: x/out [N][M][C], Y [E][NY], gates [E][NREF], Z/dZ [N][KT][C], DX [E][M][C].

#include "common.h"
#include "fsctep.h"

namespace fsc {
namespace ictd {

constexpr int EBF = 16;   // edges per LDS chunk, forward
constexpr int EBB = 8;    // edges per LDS chunk, backward

// Per-edge gated coupling table of a chunk: BG[e][bgoff_g + m1*kpad_g + kkl] (zero padded).
__device__ __forceinline__ void build_bg(const FscIctdLayout& L, float* __restrict__ bg, int eb, int cnt, int EB,
                                         const float* __restrict__ Y, const float* __restrict__ gates,
                                         const float* __restrict__ cg, bool with_gate) {
  const int total = EB * L.NBGP;
  for (int idx = threadIdx.x; idx < total; idx += blockDim.x) {
    const int e = idx / L.NBGP, j = idx - e * L.NBGP;
    float v = 0.f;
    if (e < cnt) {
      int g = 0;
      while (g + 1 < L.NG && j >= L.g_bgoff[g + 1]) ++g;
      const int rel = j - L.g_bgoff[g];
      const int kpad = L.g_kpad[g];
      const int m1 = rel / kpad, kkl = rel - m1 * kpad;
      if (m1 < L.g_d1[g] && kkl < L.g_kcount[g]) {
        const int kk = L.g_kstart[g] + kkl;
        const int p = L.kk_path[kk];
        const int d2 = L.p_d2[p], d3 = L.p_d3[p], k = kk - L.p_koff[p];
        const int64_t eid = (int64_t)(eb + e);
        const float* y = Y + eid * L.NY + L.p_oy[p];
        const float* c = cg + L.p_cgoff[p] + (m1 * d2) * d3 + k;
        float s = 0.f;
        for (int m2 = 0; m2 < d2; ++m2) s += y[m2] * c[m2 * d3];
        v = with_gate ? s * gates[eid * L.NREF + L.p_gate[p]] : s;
      }
    }
    bg[idx] = v;
  }
}

// ---------------------------------------------------------------- forward projection (one block per receiver)
template <int C, int KTT>
__global__ __launch_bounds__(256) void project_fwd_kernel(FscIctdLayout L, const float* __restrict__ x,
                                                          const float* __restrict__ Y,
                                                          const float* __restrict__ gates,
                                                          const float* __restrict__ cg,
                                                          const int32_t* __restrict__ dst_ptr,
                                                          const int32_t* __restrict__ esrc,
                                                          float* __restrict__ Z) {
  extern __shared__ float smem[];
  float* bg = smem;                                        // [EBF][NBGP]
  int32_t* srcs = reinterpret_cast<int32_t*>(smem + EBF * L.NBGP);
  constexpr int CT = C / 16;
  constexpr int CTW = (CT + 3) / 4;
  const int n = blockIdx.x;
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int r = lane & 15, q = lane >> 4;
  const int beg = dst_ptr[n], end = dst_ptr[n + 1];

  f4 acc[KTT][CTW];
#pragma unroll
  for (int kt = 0; kt < KTT; ++kt)
#pragma unroll
    for (int cw = 0; cw < CTW; ++cw) acc[kt][cw] = f4{0.f, 0.f, 0.f, 0.f};

  for (int eb = beg; eb < end; eb += EBF) {
    const int cnt = min(EBF, end - eb);
    __syncthreads();
    build_bg(L, bg, eb, cnt, EBF, Y, gates, cg, true);
    if (threadIdx.x < EBF) srcs[threadIdx.x] = (threadIdx.x < cnt) ? esrc[eb + threadIdx.x] : 0;
    __syncthreads();
    for (int g = 0; g < L.NG; ++g) {
      const int d1 = L.g_d1[g], o1 = L.g_o1[g], kpad = L.g_kpad[g], bgoff = L.g_bgoff[g], t0 = L.g_tile0[g];
      const int nk = EBF * d1;
      for (int s = 0; s < nk; s += 4) {
        const int kidx = s + q;
        const int e = kidx / d1, m1 = kidx - e * d1;
        float b[CTW];
#pragma unroll
        for (int cw = 0; cw < CTW; ++cw) {
          const int ct = wave * CTW + cw;
          b[cw] = (ct < CT && e < cnt) ? x[((int64_t)srcs[e] * L.M + o1 + m1) * C + ct * 16 + r] : 0.f;
        }
        const float* arow = bg + e * L.NBGP + bgoff + m1 * kpad + r;
#pragma unroll
        for (int kt = 0; kt < KTT; ++kt) {
          if (L.tile_group[kt] != g) continue;
          const float a = arow[(kt - t0) * 16];
#pragma unroll
          for (int cw = 0; cw < CTW; ++cw) acc[kt][cw] = mfma16x16x4(a, b[cw], acc[kt][cw]);
        }
      }
    }
  }
  const float scale = 1.f / (float)max(end - beg, 1);
#pragma unroll
  for (int kt = 0; kt < KTT; ++kt) {
    const int g = L.tile_group[kt];
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const int kkl = (kt - L.g_tile0[g]) * 16 + 4 * q + i;
      if (kkl >= L.g_kcount[g]) continue;
      const int kk = L.g_kstart[g] + kkl;
#pragma unroll
      for (int cw = 0; cw < CTW; ++cw) {
        const int ct = wave * CTW + cw;
        if (ct < CT) Z[((int64_t)n * L.KT + kk) * C + ct * 16 + r] = acc[kt][cw][i] * scale;
      }
    }
  }
}

// ---------------------------------------------------------------- channel mix, forward
// out[n][oo_k3 + m][o] = sum_{p -> k3} sum_i W[gate_p][o][i] Z[n][koff_p + m][i]; grid (rows/64, NK).
template <int C>
__global__ __launch_bounds__(256) void mix_fwd_kernel(FscIctdLayout L, const float* __restrict__ Z,
                                                      const float* __restrict__ W, float* __restrict__ out,
                                                      int64_t N) {
  constexpr int CT = C / 16;
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int r = lane & 15, q = lane >> 4;
  const int key = blockIdx.y;
  const int oo = L.k_oo[key], d = L.k_d[key];
  const int64_t rows = N * d;
  const int64_t row0 = (int64_t)blockIdx.x * 64 + wave * 16;
  if (row0 >= rows) return;
  const int64_t arow = row0 + r;
  const bool ok = arow < rows;
  const int64_t an = ok ? arow / d : 0;
  const int ak = ok ? (int)(arow % d) : 0;
  f4 acc[CT];
#pragma unroll
  for (int ct = 0; ct < CT; ++ct) acc[ct] = f4{0.f, 0.f, 0.f, 0.f};
  for (int p = 0; p < L.NP; ++p) {
    if (L.p_oo[p] != oo) continue;
    const float* zr = Z + (an * L.KT + L.p_koff[p] + ak) * C;
    const float* wp = W + (int64_t)L.p_gate[p] * C * C;
#pragma unroll 2
    for (int t = 0; t < C / 16; ++t) {
      const f4 a4 = ok ? ld4(zr + 16 * t + 4 * q) : f4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
      for (int ct = 0; ct < CT; ++ct) acc[ct] = mfma_k16(a4, ld4(wp + (16 * ct + r) * C + 16 * t + 4 * q), acc[ct]);
    }
  }
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const int64_t row = row0 + 4 * q + i;
    if (row >= rows) continue;
    const int64_t nn = row / d;
    const int m = (int)(row % d);
    float* o = out + (nn * L.M + oo + m) * C;
#pragma unroll
    for (int ct = 0; ct < CT; ++ct) o[16 * ct + r] = acc[ct][i];
  }
}

// ---------------------------------------------------------------- channel mix, backward
// dZ[n][koff_p + m][i] = sum_o Wt[gate_p][i][o] G[n][oo_p + m][o]; grid (rows/64, NP).
template <int C>
__global__ __launch_bounds__(256) void mix_bwd_kernel(FscIctdLayout L, const float* __restrict__ G,
                                                      const float* __restrict__ Wt, float* __restrict__ dZ,
                                                      int64_t N) {
  constexpr int CT = C / 16;
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int r = lane & 15, q = lane >> 4;
  const int p = blockIdx.y;
  const int d = L.p_d3[p], oo = L.p_oo[p], koff = L.p_koff[p];
  const int64_t rows = N * d;
  const int64_t row0 = (int64_t)blockIdx.x * 64 + wave * 16;
  if (row0 >= rows) return;
  const int64_t arow = row0 + r;
  const bool ok = arow < rows;
  const int64_t an = ok ? arow / d : 0;
  const int ak = ok ? (int)(arow % d) : 0;
  const float* gr = G + (an * L.M + oo + ak) * C;
  const float* wp = Wt + (int64_t)L.p_gate[p] * C * C;
  f4 acc[CT];
#pragma unroll
  for (int ct = 0; ct < CT; ++ct) acc[ct] = f4{0.f, 0.f, 0.f, 0.f};
#pragma unroll 2
  for (int t = 0; t < C / 16; ++t) {
    const f4 a4 = ok ? ld4(gr + 16 * t + 4 * q) : f4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int ct = 0; ct < CT; ++ct) acc[ct] = mfma_k16(a4, ld4(wp + (16 * ct + r) * C + 16 * t + 4 * q), acc[ct]);
  }
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const int64_t row = row0 + 4 * q + i;
    if (row >= rows) continue;
    const int64_t nn = row / d;
    const int m = (int)(row % d);
    float* o = dZ + (nn * L.KT + koff + m) * C;
#pragma unroll
    for (int ct = 0; ct < CT; ++ct) o[16 * ct + r] = acc[ct][i];
  }
}

// ---------------------------------------------------------------- backward projection (one block per receiver)
template <int C>
__global__ __launch_bounds__(256) void project_bwd_kernel(FscIctdLayout L, const float* __restrict__ dZ,
                                                          const float* __restrict__ x,
                                                          const float* __restrict__ Y,
                                                          const float* __restrict__ gates,
                                                          const float* __restrict__ cg,
                                                          const int32_t* __restrict__ dst_ptr,
                                                          const int32_t* __restrict__ esrc,
                                                          float* __restrict__ DX, float* __restrict__ dgates,
                                                          float* __restrict__ dY) {
  extern __shared__ float smem[];
  float* bg = smem;                                   // [EBB][NBGP] gated coupling table
  float* hs = smem + EBB * L.NBGP;                    // [EBB][NBGP] H = x . g
  int32_t* srcs = reinterpret_cast<int32_t*>(hs + EBB * L.NBGP);
  constexpr int CT = C / 16;
  const int n = blockIdx.x;
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int r = lane & 15, q = lane >> 4;
  const int beg = dst_ptr[n], end = dst_ptr[n + 1];
  const float scale = 1.f / (float)max(end - beg, 1);
  const float* gn = dZ + (int64_t)n * L.KT * C;

  for (int eb = beg; eb < end; eb += EBB) {
    const int cnt = min(EBB, end - eb);
    __syncthreads();
    build_bg(L, bg, eb, cnt, EBB, Y, gates, cg, true);
    if (threadIdx.x < EBB) srcs[threadIdx.x] = (threadIdx.x < cnt) ? esrc[eb + threadIdx.x] : 0;
    __syncthreads();
    // (a) DX rows (e, m1) x channels, K = padded kk of the group
    int items = 0;
    for (int g = 0; g < L.NG; ++g) items += ((EBB * L.g_d1[g] + 15) / 16) * CT;
    for (int it = wave; it < items; it += 4) {
      int g = 0, rem = it;
      for (;; ++g) {
        const int ng = ((EBB * L.g_d1[g] + 15) / 16) * CT;
        if (rem < ng) break;
        rem -= ng;
      }
      const int rt = rem / CT, ct = rem - rt * CT;
      const int d1 = L.g_d1[g], kpad = L.g_kpad[g], kcount = L.g_kcount[g], kstart = L.g_kstart[g];
      const int arow = rt * 16 + r;
      const bool aok = arow < EBB * d1;
      const int ae = aok ? arow / d1 : 0, am = aok ? arow - (arow / d1) * d1 : 0;
      const float* ap = bg + ae * L.NBGP + L.g_bgoff[g] + am * kpad;
      f4 acc = {0.f, 0.f, 0.f, 0.f};
      for (int t = 0; t < kpad; t += 16) {
        const f4 a4 = aok ? *reinterpret_cast<const f4*>(ap + t + 4 * q) : f4{0.f, 0.f, 0.f, 0.f};
        f4 b4;
#pragma unroll
        for (int j = 0; j < 4; ++j) {
          const int kkl = t + 4 * q + j;
          b4[j] = (kkl < kcount) ? gn[(int64_t)(kstart + kkl) * C + ct * 16 + r] : 0.f;
        }
        acc = mfma_k16(a4, b4, acc);
      }
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const int row = rt * 16 + 4 * q + i;
        if (row >= EBB * d1) continue;
        const int e = row / d1, m1 = row - e * d1;
        if (e < cnt)
          DX[((int64_t)(eb + e) * L.M + L.g_o1[g] + m1) * C + ct * 16 + r] = acc[i] * scale;
      }
    }
    // (b) H rows (e, m1) x padded kk, K = channels
    items = 0;
    for (int g = 0; g < L.NG; ++g) items += ((EBB * L.g_d1[g] + 15) / 16) * (L.g_kpad[g] / 16);
    for (int it = wave; it < items; it += 4) {
      int g = 0, rem = it;
      for (;; ++g) {
        const int ng = ((EBB * L.g_d1[g] + 15) / 16) * (L.g_kpad[g] / 16);
        if (rem < ng) break;
        rem -= ng;
      }
      const int nkt = L.g_kpad[g] / 16;
      const int rt = rem / nkt, kt = rem - rt * nkt;
      const int d1 = L.g_d1[g], kpad = L.g_kpad[g], kcount = L.g_kcount[g], kstart = L.g_kstart[g];
      const int arow = rt * 16 + r;
      const bool aok = arow < EBB * d1;
      const int ae = aok ? arow / d1 : 0, am = aok ? arow - (arow / d1) * d1 : 0;
      const bool xok = aok && ae < cnt;
      const float* xr = x + ((int64_t)srcs[ae] * L.M + L.g_o1[g] + am) * C;
      const int bkk = kt * 16 + r;
      const bool bok = bkk < kcount;
      const float* gr = gn + (int64_t)(kstart + (bok ? bkk : 0)) * C;
      f4 acc = {0.f, 0.f, 0.f, 0.f};
#pragma unroll 2
      for (int t = 0; t < C / 16; ++t) {
        const f4 a4 = xok ? ld4(xr + 16 * t + 4 * q) : f4{0.f, 0.f, 0.f, 0.f};
        const f4 b4 = bok ? ld4(gr + 16 * t + 4 * q) : f4{0.f, 0.f, 0.f, 0.f};
        acc = mfma_k16(a4, b4, acc);
      }
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const int row = rt * 16 + 4 * q + i;
        if (row >= EBB * d1) continue;
        const int e = row / d1, m1 = row - e * d1;
        hs[e * L.NBGP + L.g_bgoff[g] + m1 * kpad + kt * 16 + r] = acc[i] * scale;
      }
    }
    __syncthreads();
    // (c) dgate[e][p] = sum_{m1,m3} H[m1][koff_p+m3] Bn[m1][m3];  dY[e][y] = sum_p gate_p sum H C_p
    for (int idx = threadIdx.x; idx < EBB * L.NP; idx += blockDim.x) {
      const int e = idx / L.NP, p = idx - e * L.NP;
      if (e >= cnt) continue;
      const int g = L.p_group[p];
      const int d1 = L.g_d1[g], d2 = L.p_d2[p], d3 = L.p_d3[p], kpad = L.g_kpad[g];
      const int64_t eid = (int64_t)(eb + e);
      const float* y = Y + eid * L.NY + L.p_oy[p];
      const float* h = hs + e * L.NBGP + L.g_bgoff[g] + (L.p_koff[p] - L.g_kstart[g]);
      const float* c = cg + L.p_cgoff[p];
      float acc = 0.f;
      for (int m1 = 0; m1 < d1; ++m1)
        for (int m3 = 0; m3 < d3; ++m3) {
          float bn = 0.f;
          for (int m2 = 0; m2 < d2; ++m2) bn += y[m2] * c[(m1 * d2 + m2) * d3 + m3];
          acc += h[m1 * kpad + m3] * bn;
        }
      dgates[eid * L.NREF + L.p_gate[p]] = acc;
    }
    for (int idx = threadIdx.x; idx < EBB * L.NY; idx += blockDim.x) {
      const int e = idx / L.NY, yc = idx - e * L.NY;
      if (e >= cnt) continue;
      const int64_t eid = (int64_t)(eb + e);
      float acc = 0.f;
      for (int p = 0; p < L.NP; ++p) {
        const int m2 = yc - L.p_oy[p];
        if (m2 < 0 || m2 >= L.p_d2[p]) continue;
        const int g = L.p_group[p];
        const int d1 = L.g_d1[g], d2 = L.p_d2[p], d3 = L.p_d3[p], kpad = L.g_kpad[g];
        const float* h = hs + e * L.NBGP + L.g_bgoff[g] + (L.p_koff[p] - L.g_kstart[g]);
        const float* c = cg + L.p_cgoff[p] + m2 * d3;
        float s = 0.f;
        for (int m1 = 0; m1 < d1; ++m1)
          for (int m3 = 0; m3 < d3; ++m3) s += h[m1 * kpad + m3] * c[m1 * d2 * d3 + m3];
        acc += gates[eid * L.NREF + L.p_gate[p]] * s;
      }
      dY[eid * L.NY + yc] = acc;
    }
  }
}

// dx[m][:][:] = sum over out-edges of m of DX[e][:][:] (receiver-sorted ids grouped by source)
template <int C>
__global__ __launch_bounds__(256) void source_sum_kernel(int M, const int32_t* __restrict__ src_ptr,
                                                         const int32_t* __restrict__ src_perm,
                                                         const float* __restrict__ DX, float* __restrict__ dx) {
  const int m = blockIdx.x;
  const int beg = src_ptr[m], end = src_ptr[m + 1];
  const int tot = M * C;
  for (int idx = threadIdx.x * 4; idx < tot; idx += blockDim.x * 4) {
    f4 s = {0.f, 0.f, 0.f, 0.f};
    for (int j = beg; j < end; ++j) s += ld4(DX + (int64_t)src_perm[j] * tot + idx);
    st4(dx + (int64_t)m * tot + idx, s);
  }
}

// ---------------------------------------------------------------- conv1 (species-pair table)
template <int C, int NY>
__global__ __launch_bounds__(256) void conv1_fwd_kernel(FscIctdLayout L, const int32_t* __restrict__ dst_ptr,
                                                        const int32_t* __restrict__ edge_pair,
                                                        const float* __restrict__ F,
                                                        const float* __restrict__ gates,
                                                        const float* __restrict__ qtab, float* __restrict__ out) {
  const int n = blockIdx.x;
  const int o = threadIdx.x;
  if (o >= C) return;
  const int beg = dst_ptr[n], end = dst_ptr[n + 1];
  float acc[NY];
#pragma unroll
  for (int y = 0; y < NY; ++y) acc[y] = 0.f;
  for (int e = beg; e < end; ++e) {
    const int64_t pair = edge_pair[e];
    const float* fe = F + (int64_t)e * NY;
    const float* ge = gates + (int64_t)e * L.NREF;
#pragma unroll
    for (int y = 0; y < NY; ++y) {
      const int p = L.y_path1[y];
      if (p >= 0) acc[y] += ge[L.c1_gate[p]] * qtab[(pair * L.NP1 + p) * C + o] * fe[y];
    }
  }
  const float scale = 1.f / (float)max(end - beg, 1);
  float* on = out + (int64_t)n * L.M * C + o;
  for (int c = 0; c < L.M; ++c) on[c * C] = 0.f;
#pragma unroll
  for (int y = 0; y < NY; ++y)
    if (L.y_path1[y] >= 0) on[L.y_oo1[y] * C] = acc[y] * scale;
}

template <int C, int NY>
__global__ __launch_bounds__(256) void conv1_bwd_kernel(FscIctdLayout L, int NS, const int32_t* __restrict__ dst_ptr,
                                                        const int32_t* __restrict__ edge_pair,
                                                        const int32_t* __restrict__ node_species,
                                                        const float* __restrict__ G, const float* __restrict__ F,
                                                        const float* __restrict__ gates,
                                                        const float* __restrict__ qtab,
                                                        float* __restrict__ dF, float* __restrict__ dgates) {
  __shared__ float red[NY][256];
  __shared__ float T[8][NY];
  const int n = blockIdx.x;
  const int t = threadIdx.x;
  const int beg = dst_ptr[n], end = dst_ptr[n + 1];
  if (beg == end) return;                      // uniform over the block
  const float scale = 1.f / (float)(end - beg);
  const int sn = node_species[n];
  float gl[NY];
#pragma unroll
  for (int y = 0; y < NY; ++y)
    gl[y] = (t < C && L.y_path1[y] >= 0) ? G[((int64_t)n * L.M + L.y_oo1[y]) * C + t] : 0.f;
  // T[s][y] = (1/deg) sum_o G[n][comp(y)][o] Q[(s, sn)][p(y)][o]
  for (int s = 0; s < NS; ++s) {
    const int64_t pair = (int64_t)s * NS + sn;
#pragma unroll
    for (int y = 0; y < NY; ++y) {
      const int p = L.y_path1[y];
      red[y][t] = (t < C && p >= 0) ? gl[y] * qtab[(pair * L.NP1 + p) * C + t] : 0.f;
    }
    __syncthreads();
    if (t < NY) {
      float sacc = 0.f;
      for (int j = 0; j < 256; ++j) sacc += red[t][j];
      T[s][t] = sacc * scale;
    }
    __syncthreads();
  }
  // per edge: dF[e][y] = gate_p(y) T[s_src][y];  dgate[e][p] = sum_{y in p} T[s_src][y] F[e][y]
  const int ne = end - beg;
  for (int idx = t; idx < ne * NY; idx += blockDim.x) {
    const int e = beg + idx / NY, y = idx % NY;
    const int p = L.y_path1[y];
    const int ss = edge_pair[e] / NS;
    dF[(int64_t)e * NY + y] = (p >= 0) ? gates[(int64_t)e * L.NREF + L.c1_gate[p]] * T[ss][y] : 0.f;
  }
  for (int idx = t; idx < ne * L.NP1; idx += blockDim.x) {
    const int e = beg + idx / L.NP1, p = idx % L.NP1;
    const int ss = edge_pair[e] / NS;
    float acc = 0.f;
    for (int y = 0; y < NY; ++y)
      if (L.y_path1[y] == p) acc += T[ss][y] * F[(int64_t)e * NY + y];
    dgates[(int64_t)e * L.NREF + L.c1_gate[p]] = acc;
  }
}

__global__ void transpose_weights_kernel(const float* __restrict__ W, float* __restrict__ Wt, int n_ref, int C) {
  const int64_t total = (int64_t)n_ref * C * C;
  for (int64_t idx = blockIdx.x * (int64_t)blockDim.x + threadIdx.x; idx < total; idx += (int64_t)gridDim.x * blockDim.x) {
    const int i = (int)(idx % C);
    const int o = (int)((idx / C) % C);
    const int64_t p = idx / ((int64_t)C * C);
    Wt[(p * C + i) * C + o] = W[idx];
  }
}

// ---------------------------------------------------------------- host side
int check_layout(const FscIctdLayout* L, int32_t C, const char* who) {
  if (!L) { set_error(std::string(who) + ": null layout"); return 1; }
  if (!(C == 32 || C == 64 || C == 128)) { set_error(std::string(who) + ": channels must be 32, 64 or 128"); return 1; }
  if (L->NG < 1 || L->NG > 8 || L->NP < 1 || L->NP > 64 || L->KT < 1 || L->KT > 128 || L->KTT < 1 ||
      L->KTT > 8 || L->NY < 1 || L->NY > 16 || L->M < 1 || L->M > 16 || L->NREF < L->NP || L->NK < 1 ||
      L->NK > 16 || L->NP1 < 0 || L->NP1 > 16 || L->NBGP < 1 || (L->NBGP % 4) != 0) {
    set_error(std::string(who) + ": layout table out of range");
    return 1;
  }
  // every input component must belong to one path group (the backward writes DX row by row)
  int covered = 0;
  for (int g = 0; g < L->NG; ++g) {
    if (L->g_o1[g] != covered || L->g_kpad[g] % 16 != 0 || L->g_kcount[g] > L->g_kpad[g]) {
      set_error(std::string(who) + ": path groups must tile the input components in order");
      return 1;
    }
    covered += L->g_d1[g];
  }
  if (covered != L->M) {
    set_error(std::string(who) + ": every input irrep needs a live path");
    return 1;
  }
  return 0;
}

template <int C, int KTT>
void launch_project_fwd(const FscIctdLayout& L, int64_t N, const int32_t* dst_ptr, const int32_t* esrc,
                        const float* x, const float* Y, const float* gates, const float* cg, float* Z,
                        hipStream_t st) {
  const size_t lds = (size_t)EBF * L.NBGP * sizeof(float) + EBF * sizeof(int32_t);
  project_fwd_kernel<C, KTT><<<(unsigned)N, 256, lds, st>>>(L, x, Y, gates, cg, dst_ptr, esrc, Z);
}

template <int C>
int forward_c(const FscIctdLayout& L, int64_t N, const int32_t* dst_ptr, const int32_t* esrc, const float* x,
              const float* Y, const float* gates, const float* cg, const float* W, float* Z, float* out,
              hipStream_t st) {
  {
    LaunchTimer tm("ictd_project", st);
    switch (L.KTT) {
      case 1: launch_project_fwd<C, 1>(L, N, dst_ptr, esrc, x, Y, gates, cg, Z, st); break;
      case 2: launch_project_fwd<C, 2>(L, N, dst_ptr, esrc, x, Y, gates, cg, Z, st); break;
      case 3: launch_project_fwd<C, 3>(L, N, dst_ptr, esrc, x, Y, gates, cg, Z, st); break;
      case 4: launch_project_fwd<C, 4>(L, N, dst_ptr, esrc, x, Y, gates, cg, Z, st); break;
      case 5: launch_project_fwd<C, 5>(L, N, dst_ptr, esrc, x, Y, gates, cg, Z, st); break;
      case 6: launch_project_fwd<C, 6>(L, N, dst_ptr, esrc, x, Y, gates, cg, Z, st); break;
      case 7: launch_project_fwd<C, 7>(L, N, dst_ptr, esrc, x, Y, gates, cg, Z, st); break;
      default: launch_project_fwd<C, 8>(L, N, dst_ptr, esrc, x, Y, gates, cg, Z, st); break;
    }
  }
  if (check_launch("ictd project_fwd")) return 2;
  int dmax = 1;
  for (int k = 0; k < L.NK; ++k) dmax = max(dmax, L.k_d[k]);
  {
    LaunchTimer tm("ictd_mix", st);
    dim3 grid((unsigned)((N * dmax + 63) / 64), (unsigned)L.NK);
    mix_fwd_kernel<C><<<grid, 256, 0, st>>>(L, Z, W, out, N);
  }
  return check_launch("ictd mix_fwd") ? 2 : 0;
}

template <int C>
int backward_c(const FscIctdLayout& L, int64_t N, const int32_t* dst_ptr, const int32_t* esrc,
               const int32_t* src_ptr, const int32_t* src_perm, const float* G, const float* x, const float* Y,
               const float* gates, const float* cg, const float* Wt, float* dZ, float* DX, float* dx,
               float* dgates, float* dY, hipStream_t st) {
  int dmax = 1;
  for (int p = 0; p < L.NP; ++p) dmax = max(dmax, L.p_d3[p]);
  {
    LaunchTimer tm("ictd_mix_grad", st);
    dim3 grid((unsigned)((N * dmax + 63) / 64), (unsigned)L.NP);
    mix_bwd_kernel<C><<<grid, 256, 0, st>>>(L, G, Wt, dZ, N);
  }
  if (check_launch("ictd mix_bwd")) return 2;
  {
    LaunchTimer tm("ictd_project_grad", st);
    const size_t lds = 2 * (size_t)EBB * L.NBGP * sizeof(float) + EBB * sizeof(int32_t);
    project_bwd_kernel<C><<<(unsigned)N, 256, lds, st>>>(L, dZ, x, Y, gates, cg, dst_ptr, esrc, DX, dgates, dY);
  }
  if (check_launch("ictd project_bwd")) return 2;
  {
    LaunchTimer tm("ictd_source_sum", st);
    source_sum_kernel<C><<<(unsigned)N, 256, 0, st>>>(L.M, src_ptr, src_perm, DX, dx);
  }
  return check_launch("ictd source_sum") ? 2 : 0;
}

}  // namespace ictd
}  // namespace fsc

using namespace fsc;
using namespace fsc::ictd;

extern "C" {

int fsc_ictd_conv_forward(const FscIctdLayout* layout, int64_t n_nodes, int64_t n_edges, int32_t channels,
                          const int32_t* dst_ptr, const int32_t* edge_src, const float* x, const float* Y,
                          const float* gates, const float* cg, const float* W, float* z_ws, float* out,
                          hipStream_t stream) {
  if (check_layout(layout, channels, "fsc_ictd_conv_forward")) return 1;
  FSC_CHECK_ARG(n_nodes >= 0 && n_edges >= 0 && n_nodes < (1LL << 31) && n_edges < (1LL << 31),
                "fsc_ictd_conv_forward: bad size");
  FSC_CHECK_ARG(dst_ptr && x && cg && W && z_ws && out, "fsc_ictd_conv_forward: null pointer");
  FSC_CHECK_ARG(n_edges == 0 || (edge_src && Y && gates), "fsc_ictd_conv_forward: null edge pointer");
  if (n_nodes == 0) return 0;
  const FscIctdLayout& L = *layout;
  if (channels == 128) return forward_c<128>(L, n_nodes, dst_ptr, edge_src, x, Y, gates, cg, W, z_ws, out, stream);
  if (channels == 64) return forward_c<64>(L, n_nodes, dst_ptr, edge_src, x, Y, gates, cg, W, z_ws, out, stream);
  return forward_c<32>(L, n_nodes, dst_ptr, edge_src, x, Y, gates, cg, W, z_ws, out, stream);
}

int fsc_ictd_prepare_weights(const float* W, int32_t n_ref, int32_t channels, float* Wt, hipStream_t stream) {
  FSC_CHECK_ARG(W && Wt && n_ref > 0 && channels > 0, "fsc_ictd_prepare_weights: bad argument");
  transpose_weights_kernel<<<256, 256, 0, stream>>>(W, Wt, n_ref, channels);
  return check_launch("ictd transpose_weights") ? 2 : 0;
}

int fsc_ictd_conv_backward(const FscIctdLayout* layout, int64_t n_nodes, int64_t n_edges, int32_t channels,
                           const int32_t* dst_ptr, const int32_t* edge_src, const int32_t* src_ptr,
                           const int32_t* src_perm, const float* grad_out, const float* x, const float* Y,
                           const float* gates, const float* cg, const float* Wt, float* dz_ws,
                           float* dxe_ws, float* grad_x, float* grad_gates, float* grad_Y, hipStream_t stream) {
  if (check_layout(layout, channels, "fsc_ictd_conv_backward")) return 1;
  FSC_CHECK_ARG(n_nodes >= 0 && n_edges >= 0 && n_nodes < (1LL << 31) && n_edges < (1LL << 31),
                "fsc_ictd_conv_backward: bad size");
  FSC_CHECK_ARG(dst_ptr && src_ptr && grad_out && x && cg && Wt && dz_ws && grad_x,
                "fsc_ictd_conv_backward: null pointer");
  FSC_CHECK_ARG(n_edges == 0 || (edge_src && src_perm && Y && gates && dxe_ws && grad_gates && grad_Y),
                "fsc_ictd_conv_backward: null edge pointer");
  if (n_nodes == 0) return 0;
  const FscIctdLayout& L = *layout;
  if (channels == 128)
    return backward_c<128>(L, n_nodes, dst_ptr, edge_src, src_ptr, src_perm, grad_out, x, Y, gates, cg, Wt, dz_ws,
                           dxe_ws, grad_x, grad_gates, grad_Y, stream);
  if (channels == 64)
    return backward_c<64>(L, n_nodes, dst_ptr, edge_src, src_ptr, src_perm, grad_out, x, Y, gates, cg, Wt, dz_ws,
                          dxe_ws, grad_x, grad_gates, grad_Y, stream);
  return backward_c<32>(L, n_nodes, dst_ptr, edge_src, src_ptr, src_perm, grad_out, x, Y, gates, cg, Wt, dz_ws,
                        dxe_ws, grad_x, grad_gates, grad_Y, stream);
}

int fsc_ictd_conv1_forward(const FscIctdLayout* layout, int64_t n_nodes, int64_t n_edges, int32_t channels,
                           const int32_t* dst_ptr, const int32_t* edge_pair, const float* F, const float* gates,
                           const float* qtab, float* out, hipStream_t stream) {
  if (check_layout(layout, channels, "fsc_ictd_conv1_forward")) return 1;
  FSC_CHECK_ARG(n_nodes >= 0 && n_edges >= 0 && n_nodes < (1LL << 31) && n_edges < (1LL << 31),
                "fsc_ictd_conv1_forward: bad size");
  FSC_CHECK_ARG(dst_ptr && qtab && out, "fsc_ictd_conv1_forward: null pointer");
  FSC_CHECK_ARG(n_edges == 0 || (edge_pair && F && gates), "fsc_ictd_conv1_forward: null edge pointer");
  FSC_CHECK_ARG(layout->NY == 9 || layout->NY == 16, "fsc_ictd_conv1_forward: lmax must be 2 or 3");
  if (n_nodes == 0) return 0;
  const FscIctdLayout& L = *layout;
  LaunchTimer tm("ictd_conv1", stream);
  const unsigned grid = (unsigned)n_nodes;
#define FSC_C1F(CC, NYY) conv1_fwd_kernel<CC, NYY><<<grid, 256, 0, stream>>>(L, dst_ptr, edge_pair, F, gates, qtab, out)
  if (L.NY == 9) {
    if (channels == 128) FSC_C1F(128, 9); else if (channels == 64) FSC_C1F(64, 9); else FSC_C1F(32, 9);
  } else {
    if (channels == 128) FSC_C1F(128, 16); else if (channels == 64) FSC_C1F(64, 16); else FSC_C1F(32, 16);
  }
#undef FSC_C1F
  return check_launch("ictd conv1_fwd") ? 2 : 0;
}

int fsc_ictd_conv1_backward(const FscIctdLayout* layout, int64_t n_nodes, int64_t n_edges, int32_t channels,
                            int32_t n_species, const int32_t* dst_ptr, const int32_t* edge_pair,
                            const int32_t* node_species, const float* grad_out, const float* F,
                            const float* gates, const float* qtab, float* grad_F, float* grad_gates,
                            hipStream_t stream) {
  if (check_layout(layout, channels, "fsc_ictd_conv1_backward")) return 1;
  FSC_CHECK_ARG(n_nodes >= 0 && n_edges >= 0 && n_nodes < (1LL << 31) && n_edges < (1LL << 31),
                "fsc_ictd_conv1_backward: bad size");
  FSC_CHECK_ARG(n_species >= 1 && n_species <= 8, "fsc_ictd_conv1_backward: 1..8 species supported");
  FSC_CHECK_ARG(dst_ptr && node_species && grad_out && qtab, "fsc_ictd_conv1_backward: null pointer");
  FSC_CHECK_ARG(n_edges == 0 || (edge_pair && F && gates && grad_F && grad_gates),
                "fsc_ictd_conv1_backward: null edge pointer");
  FSC_CHECK_ARG(layout->NY == 9 || layout->NY == 16, "fsc_ictd_conv1_backward: lmax must be 2 or 3");
  if (n_nodes == 0) return 0;
  const FscIctdLayout& L = *layout;
  LaunchTimer tm("ictd_conv1_grad", stream);
  const unsigned grid = (unsigned)n_nodes;
#define FSC_C1B(CC, NYY) conv1_bwd_kernel<CC, NYY><<<grid, 256, 0, stream>>>(L, n_species, dst_ptr, edge_pair, \
      node_species, grad_out, F, gates, qtab, grad_F, grad_gates)
  if (L.NY == 9) {
    if (channels == 128) FSC_C1B(128, 9); else if (channels == 64) FSC_C1B(64, 9); else FSC_C1B(32, 9);
  } else {
    if (channels == 128) FSC_C1B(128, 16); else if (channels == 64) FSC_C1B(64, 16); else FSC_C1B(32, 16);
  }
#undef FSC_C1B
  return check_launch("ictd conv1_bwd") ? 2 : 0;
}

}  // extern "C"
