// ICTD (harmonic-irreps) message passing on gfx950: pure-cartesian-ictd and -ictd-o3.
//
// Replaces HarmonicFullyConnectedTensorProduct[O3].forward + receiver scatter of the conv2..n
// loop (models/ictd_irreps.py:971-1253, :1512-1695; models/pure_cartesian_ictd_layers_full.py:938-954,
// models/pure_cartesian_ictd_layers_o3.py:956-973) and the TP of conv1 (:341-473 / :424-532).
//
// Algebra (exact; only summation order changes).  For a live path p = (k1 = (l1,p1), Y_l2 -> k3):
//   out_n[k3][o][m3] = (1/deg n) sum_{e->n} gate_e[p] sum_i W[p][o][i] sum_{m1,m2} x_src[k1][i][m1] Y_e[l2][m2] C_p[m1][m2][m3]
// The channel mix W is linear, so it moves after the receiver sum:
//   BG_e[p][m1][m3] = gate_e[p] sum_m2 Y_e[l2][m2] C_p[m1][m2][m3]                      (per edge, MFMA)
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

// 16-row tiles per wave in the channel mix: more reuse of each weight load (the L2 traffic of the
// weights falls 4x at 4 tiles; 10k atoms, C 128: 0.56 -> 0.40 ms, 2 tiles 0.50 ms) against fewer waves
// (4k atoms, C 64, where the weights are 4x smaller: one tile is fastest)
template <int C>
constexpr int mix_rt() { return C >= 128 ? 3 : 1; }
constexpr int EB = 16;    // edges per chunk: one 16-deep K block of the projection products

// LDS carve-ups are in 4-byte words, regions 16-byte aligned.
__host__ __device__ inline int up4(int v) { return (v + 3) & ~3; }

// V floats (V = 2, 4 or 8) of one lane as an MFMA-operand bundle.
template <int V>
struct VecF {
  float v[V];
};

// Quad-interleaved bundle of V channels for lane r of a 16-lane row: quad h holds channels 64h + 4r ..
// 64h + 4r + 3 (V >= 4), so each of the V/4 vector loads of a 16-lane row reads 256 contiguous bytes; V = 2:
// channels 2r, 2r + 1.  p points at the row's channel lane_chan<V>(r).
template <int V>
__device__ __forceinline__ int lane_chan(int r) { return V >= 4 ? 4 * r : V * r; }

template <int V>
__device__ __forceinline__ VecF<V> ldq(const float* p) {
  VecF<V> r;
  if constexpr (V >= 4) {
#pragma unroll
    for (int h = 0; h < V / 4; ++h) {
      const f4 t = *reinterpret_cast<const f4*>(p + 64 * h);
#pragma unroll
      for (int j = 0; j < 4; ++j) r.v[4 * h + j] = t[j];
    }
  } else {
    const float2 t = *reinterpret_cast<const float2*>(p);
    r.v[0] = t.x;
    r.v[1] = t.y;
  }
  return r;
}

template <int V>
__device__ __forceinline__ void stq(float* p, const VecF<V>& r) {
  if constexpr (V >= 4) {
#pragma unroll
    for (int h = 0; h < V / 4; ++h)
      *reinterpret_cast<f4*>(p + 64 * h) = f4{r.v[4 * h], r.v[4 * h + 1], r.v[4 * h + 2], r.v[4 * h + 3]};
  } else {
    *reinterpret_cast<float2*>(p) = make_float2(r.v[0], r.v[1]);
  }
}

// Tasks are the 16-row kk tiles, of cost d1(group).  Snake order over the cost-sorted list gives every
// wave at most two of the KTT <= 8 tiles with near-equal cost.
__device__ __forceinline__ void assign_fwd_tasks(const FscIctdLayout& L, int* __restrict__ wtask) {
  if (threadIdx.x != 0) return;
  const int T = L.KTT;
  for (int w = 0; w < 4; ++w) wtask[w * 8] = 0;
  for (int t = 0; t < T; ++t) {
    const int ct = L.g_d1[L.tile_group[t]];
    int rank = 0;
    for (int u = 0; u < T; ++u) {
      const int cu = L.g_d1[L.tile_group[u]];
      rank += (cu > ct) || (cu == ct && u < t);
    }
    const int round = rank >> 2, pos = rank & 3;
    const int w = (round & 1) ? 3 - pos : pos;
    wtask[w * 8 + 1 + wtask[w * 8]++] = t;
  }
}

// ---------------------------------------------------------------- forward projection (one block per receiver)
// Z[n][kk][i] = (1/deg) sum_{(e,m1)} bg[e][m1][kk] x[src_e][o1 + m1][i], MFMA with K = (m1, e).
// The same kernel runs the dual projection of the backward (dual_layout): blocks are sources, their edges
// come through eperm (the source grouping), the gathered rows are receiver gradients divided by their
// receiver's in-degree (gdeg), and there is no final normalisation.
//
// The gated coupling rows are formed on the MFMA, in the operand layout of the main product: for a 16-row
// kk tile and component m1, BG[e][kk] = gate_e[p(kk)] sum_y Y_e[y] Cf[y][kk] over the 16 edges of a chunk
// is one 16x16x16 product (4 MFMAs, A = the chunk's harmonics, B = Cf, the tile's coupling coefficients
// zero-padded to all NY <= 16 harmonic components), whose result lane (r, q) holds edges 4q..4q+3 of kk
// row r: exactly the A operand of the main product when K step u takes edge 4q+u.  So there is no per-edge
// table in LDS and no barrier inside the edge loop: each wave walks the chunks on its own.  Cf is built
// once per block in LDS (one float4 per lane per (tile, m1) slot).
// A wave takes at most two of the KTT <= 8 kk tiles, each over all C channels (64-channel spans at
// 4 waves/SIMD measured slower at C 128: the coupling product is then formed once per span).  The main
// product runs in split-fp16 (project_fwd_h16_kernel below).
struct FwdSmem {
  int cgs, kd, gidx, slot0, wtask, cb, cf, total;
};

__host__ __device__ inline int n_slots(const FscIctdLayout& L) {
  int ns = 0;
  for (int t = 0; t < L.KTT; ++t) ns += L.g_d1[L.tile_group[t]];
  return ns;
}

__host__ __device__ inline FwdSmem fwd_smem(const FscIctdLayout& L, int ncg) {
  FwdSmem s;
  int o = 0;
  s.cgs = o;   o += up4(ncg);
  s.kd = o;    o += 4 * L.KT;              // per kk slot: coupling offset, oy | d2 << 8 | d3 << 16, gate, path
  s.gidx = o;  o += 16 * L.KTT;            // gate column of each kk row of each tile
  s.slot0 = o; o += up4(L.KTT + 1);        // first Cf slot of each tile
  s.wtask = o; o += 32;
  s.cb = o;    o += 16 * L.KTT;            // bound of each kk row's coupling coefficients (split-fp16 scale)
  s.cf = o;    o += n_slots(L) * 256;
  s.total = o;
  return s;
}

// First stage of the per-block tables: the coupling tensors, one descriptor per kk slot (so that the
// per-lane lookups of the second stage read LDS, not the layout argument) and the first Cf slot of each
// tile.  kd[kk] = {offset of C_p[0][0][kk - koff_p], oy_p | d2 << 8 | d3 << 16, gate_p, p}.
__device__ __forceinline__ void stage_descriptors(const FscIctdLayout& L, const float* __restrict__ cg, int ncg,
                                                  float* __restrict__ cgs, int4* __restrict__ kd,
                                                  int* __restrict__ slot0) {
  for (int i = threadIdx.x; i < ncg; i += blockDim.x) cgs[i] = cg[i];
  for (int kk = threadIdx.x; kk < L.KT; kk += blockDim.x) {
    const int p = L.kk_path[kk];
    kd[kk] = make_int4(L.p_cgoff[p] + kk - L.p_koff[p], L.p_oy[p] | (L.p_d2[p] << 8) | (L.p_d3[p] << 16),
                       L.p_gate[p], p);
  }
  if (threadIdx.x == 0) {
    int s = 0;
    for (int t = 0; t < L.KTT; ++t) {
      slot0[t] = s;
      s += L.g_d1[L.tile_group[t]];
    }
    slot0[L.KTT] = s;
  }
}

// Tile of slot sl (wave-uniform): the last tile whose first slot is <= sl.
__device__ __forceinline__ int tile_of_slot(const FscIctdLayout& L, const int* __restrict__ slot0, int sl) {
  int t = 0;
  while (t + 1 < L.KTT && sl >= slot0[t + 1]) ++t;
  return t;
}

// Cf[slot(kt) + m1][lane (r, q)][s] = C_p[m1][y - oy_p][kk - koff_p] for y = 4q + s in [oy_p, oy_p + d2),
// kk = kstart + (kt - tile0)*16 + r a live row of tile kt (else 0); gidx[kt][r] = the gate of that row.
__device__ __forceinline__ void stage_fwd_tables(const FscIctdLayout& L, const float* __restrict__ cg, int ncg,
                                                 float* __restrict__ cgs, int4* __restrict__ kd,
                                                 int* __restrict__ gidx, int* __restrict__ slot0,
                                                 float* __restrict__ cf) {
  stage_descriptors(L, cg, ncg, cgs, kd, slot0);
  __syncthreads();
  for (int i = threadIdx.x; i < 16 * L.KTT; i += blockDim.x) {
    const int t = i >> 4, r = i & 15, g = L.tile_group[t];
    const int kkl = (t - L.g_tile0[g]) * 16 + r;
    gidx[i] = kkl < L.g_kcount[g] ? kd[L.g_kstart[g] + kkl].z : 0;
  }
  const int nslot = slot0[L.KTT];
  for (int i = threadIdx.x; i < nslot * 64; i += blockDim.x) {
    const int sl = __builtin_amdgcn_readfirstlane(i >> 6), lane = i & 63, r = lane & 15, q = lane >> 4;
    const int t = tile_of_slot(L, slot0, sl);
    const int g = L.tile_group[t], m1 = sl - slot0[t];
    const int kkl = (t - L.g_tile0[g]) * 16 + r;
    f4 v = f4{0.f, 0.f, 0.f, 0.f};
    if (kkl < L.g_kcount[g]) {
      const int4 d = kd[L.g_kstart[g] + kkl];
      const int oy = d.y & 255, d2 = (d.y >> 8) & 255, d3 = d.y >> 16;
      const int base = d.x + m1 * d2 * d3;
#pragma unroll
      for (int s = 0; s < 4; ++s) {
        const int m2 = 4 * q + s - oy;
        if (m2 >= 0 && m2 < d2) v[s] = cgs[base + m2 * d3];
      }
    }
    reinterpret_cast<f4*>(cf)[i] = v;
  }
}

// ---------------------------------------------------------------- forward projection, split-fp16 products
// Over the blocks, tiles, chunks and coupling rows described above, the main product runs on
// v_mfma_f32_16x16x16_f16 with three products per K step (fp32-accurate to 22 significant bits): the 16-deep
// K step is one chunk of 16 edges for one component m1, lane (r, q) supplying edges 4q .. 4q + 3, which are
// the coupling values it holds and the four rows it gathers, so one fp16 MFMA does the work of four fp32 ones.
//  * The gathered rows come pre-split (split_rows_il_kernel: fp16 parts of x[n] nu_n and 1/nu_n, the two
//    parts of a lane's V channels side by side, so a row is one 4V-byte load per lane); B is the four rows'
//    halves of one channel, packed with v_perm_b32, and 1/nu_src goes into the A operand (a power of two:
//    exact).
//  * A, the gated coupling values times 1/nu_src, carries a power of two s_r per kk row r so that |A s_r| <
//    2^14 over all of the node's edges: each chunk bounds its row by max_e |gate_e / nu_src(e)| max_y |Y_e[y]|
//    times cb[r] = max_m1 sum_y |Cf[m1][y][r]|, and when that bound lowers s_r the accumulated row is scaled
//    by the ratio (a power of two: exact).  The store undoes s_r.
//  * Lane r takes channels V r .. V r + V - 1 (column tile j is channel V r + j): V contiguous floats per kk
//    row at the store.
// A gathered row's V channels of one lane as 32-bit words (split_rows_il_kernel layout): w[0 .. V/2) the
// high halves, two channels a word, w[V/2 .. V) the low halves.  Words rather than half vectors, so the
// operand repacking below stays in registers.
template <int V>
struct RowW {
  uint32_t w[V];
};

template <int V>
__device__ __forceinline__ RowW<V> ld_row(const _Float16* p) {
  RowW<V> r;
  if constexpr (V >= 4) {
#pragma unroll
    for (int h = 0; h < V / 4; ++h) {
      const uint4 a = *reinterpret_cast<const uint4*>(p + 8 * h);
      r.w[4 * h] = a.x;
      r.w[4 * h + 1] = a.y;
      r.w[4 * h + 2] = a.z;
      r.w[4 * h + 3] = a.w;
    }
  } else {
    const uint2 a = *reinterpret_cast<const uint2*>(p);
    r.w[0] = a.x;
    r.w[1] = a.y;
  }
  return r;
}

// {half s of a, half s of b} as one word (s = 0 low, 1 high)
__device__ __forceinline__ uint32_t pack_halves(uint32_t a, uint32_t b, int s) {
  return __builtin_amdgcn_perm(b, a, s ? 0x07060302u : 0x05040100u);
}

template <int C, bool DUAL>
__global__ __launch_bounds__(256, C >= 128 ? 3 : 4) void project_fwd_h16_kernel(
    FscIctdLayout L, int ncg, const _Float16* __restrict__ xs, const float* __restrict__ xinv,
    const float* __restrict__ Y, const float* __restrict__ gates,
    const float* __restrict__ cg, const int32_t* __restrict__ dst_ptr, const int32_t* __restrict__ esrc,
    float* __restrict__ Z, float* __restrict__ zscale, int64_t n_nodes, const int32_t* __restrict__ node_order,
    const int32_t* __restrict__ eperm, const int32_t* __restrict__ gdeg) {
  constexpr int V = C / 16;
  typedef _Float16 h4 __attribute__((ext_vector_type(4)));
  extern __shared__ __align__(16) float smem[];
  __shared__ float zmx[2][4];
  const FwdSmem sm = fwd_smem(L, ncg);
  int* gidx = reinterpret_cast<int*>(smem + sm.gidx);
  int* slot0 = reinterpret_cast<int*>(smem + sm.slot0);
  int* wtask = reinterpret_cast<int*>(smem + sm.wtask);
  float* cb = smem + sm.cb;
  const f4* cf = reinterpret_cast<const f4*>(smem + sm.cf);

  if (xcd_node_k(n_nodes, node_order, 0) == -2) return;   // block-uniform
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int r = lane & 15, q = lane >> 4;
  assign_fwd_tasks(L, wtask);
  stage_fwd_tables(L, cg, ncg, smem + sm.cgs, reinterpret_cast<int4*>(smem + sm.kd), gidx, slot0, smem + sm.cf);
  __syncthreads();
  for (int i = threadIdx.x; i < 16 * L.KTT; i += blockDim.x) {
    const int t = i >> 4, rr = i & 15, d1 = L.g_d1[L.tile_group[t]];
    float m = 0.f;
    for (int m1 = 0; m1 < d1; ++m1) {
      float s = 0.f;
#pragma unroll
      for (int qq = 0; qq < 4; ++qq) {
        const f4 c = cf[(slot0[t] + m1) * 64 + 16 * qq + rr];
        s += (fabsf(c.x) + fabsf(c.y)) + (fabsf(c.z) + fabsf(c.w));
      }
      m = fmaxf(m, s);
    }
    cb[i] = m;
  }
  __syncthreads();
  const int ntask = wtask[wave * 8];

  int done = 0;
  for (int k = 0;; ++k) {
  const int n = xcd_node_k(n_nodes, node_order, k);
  if (n == -2) break;
  if (n < 0) continue;
  const int beg = dst_ptr[n], end = dst_ptr[n + 1];
  const float scale = DUAL ? 1.f : 1.f / (float)max(end - beg, 1);
  float zmax = 0.f;
  for (int lt = 0; lt < ntask; ++lt) {
    const int kt = wtask[wave * 8 + 1 + lt];
    const int g = L.tile_group[kt];
    const int d1 = L.g_d1[g], o1 = L.g_o1[g];
    const int gc = gidx[kt * 16 + r];
    const float cbr = cb[kt * 16 + r];
    const f4* cft = cf + slot0[kt] * 64 + lane;
    const _Float16* xcol = xs + 2 * ((int64_t)o1 * C + V * r);
    f4 acc[V];
#pragma unroll
    for (int j = 0; j < V; ++j) acc[j] = f4{0.f, 0.f, 0.f, 0.f};
    float srow = 0x1p100f;   // power of two of kk row r (lanes (r, *)), lowered as chunks need
    auto chunk_id = [&](int ebk) {
      const int ck = min(EB, end - ebk);
      return r < ck ? (DUAL ? eperm[ebk + r] : ebk + r) : -1;
    };
    int idr_n = beg < end ? chunk_id(beg) : -1;
    int srcr_n = idr_n >= 0 ? esrc[idr_n] : 0;
    for (int eb = beg; eb < end; eb += EB) {
      const int cnt = min(EB, end - eb);
      const int idr = idr_n, srcr = srcr_n;
      f4 yop = f4{0.f, 0.f, 0.f, 0.f};
      if (idr >= 0) {
        const float* yr = Y + (int64_t)idr * L.NY;
        if (L.NY == 16 && (reinterpret_cast<uintptr_t>(Y) & 15) == 0) {
          yop = reinterpret_cast<const f4*>(yr)[q];
        } else {
#pragma unroll
          for (int s = 0; s < 4; ++s)
            if (4 * q + s < L.NY) yop[s] = yr[4 * q + s];
        }
      }
      float gsc = 1.f;
      if constexpr (DUAL) gsc = 1.f / (float)max(gdeg[srcr + 1] - gdeg[srcr], 1);
      const float xi = idr >= 0 ? xinv[srcr] : 0.f;   // 1/nu of chunk edge r's gathered row
      int src4[4];
#pragma unroll
      for (int u = 0; u < 4; ++u) src4[u] = __shfl(srcr, 4 * q + u, 64);
      auto load_k = [&](int m1, RowW<V> (&b)[4]) {
#pragma unroll
        for (int u = 0; u < 4; ++u) b[u] = ld_row<V>(xcol + 2 * ((int64_t)src4[u] * L.M + m1) * C);
      };
      RowW<V> b0[4], b1[4];
      load_k(0, b0);
      // A factors of edges 4q + u (gate / nu_src) and the chunk's bound on row r
      float ym = fmaxf(fmaxf(fabsf(yop.x), fabsf(yop.y)), fmaxf(fabsf(yop.z), fabsf(yop.w)));
      ym = fmaxf(ym, __shfl_xor(ym, 16, 64));
      ym = fmaxf(ym, __shfl_xor(ym, 32, 64));   // max_y |Y| of chunk edge r
      float ga[4], bnd = 0.f;
#pragma unroll
      for (int u = 0; u < 4; ++u) {
        const int id = DUAL ? __shfl(idr, 4 * q + u, 64) : (4 * q + u < cnt ? eb + 4 * q + u : -1);
        const float sc = DUAL ? __shfl(gsc, 4 * q + u, 64) : 1.f;
        const float xu = __shfl(xi, 4 * q + u, 64), yu = __shfl(ym, 4 * q + u, 64);
        ga[u] = id >= 0 ? gates[(int64_t)id * L.NREF + gc] * sc * xu : 0.f;
        bnd = fmaxf(bnd, fabsf(ga[u]) * yu);
      }
      bnd = fmaxf(bnd, __shfl_xor(bnd, 16, 64));
      bnd = fmaxf(bnd, __shfl_xor(bnd, 32, 64));
      bnd *= cbr;
      const float snew = bnd > 0.f ? fminf(srow, pow2_scale(bnd)) : srow;
      const float ratio = snew / srow;   // a power of two (1 while the scale holds)
      srow = snew;
      if (__ballot(ratio != 1.f)) {      // wave-uniform: rescale the accumulated rows 4q + i
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          const float ri = __shfl(ratio, 4 * q + i, 64);
#pragma unroll
          for (int j = 0; j < V; ++j) acc[j][i] *= ri;
        }
      }
#pragma unroll
      for (int u = 0; u < 4; ++u) ga[u] *= srow;
      if (eb + EB < end) {
        idr_n = chunk_id(eb + EB);
        srcr_n = idr_n >= 0 ? esrc[idr_n] : 0;
      }
      // split gated coupling values of component m1: A[row r][edge 4q + u]
      auto coupling = [&](int m1, h4& ah, h4& al) {
        const f4 bg = mfma_k16(yop, cft[m1 * 64], f4{0.f, 0.f, 0.f, 0.f});
#pragma unroll
        for (int u = 0; u < 4; ++u) {
          // v rounded to fp32 before the split: fused into the low part's fma_mix, the exact product would
          // pair with a high part rounded from the fp32 product, off by an fp16 ulp where those differ
          float v = bg[u] * ga[u];
          asm volatile("" : "+v"(v));
          const _Float16 h = (_Float16)v;
          ah[u] = h;
          al[u] = (_Float16)(v - (float)h);
        }
      };
      auto mul_k = [&](const h4& ah, const h4& al, const RowW<V> (&b)[4]) {
#pragma unroll
        for (int j = 0; j < V; ++j) {
          const int d = j >> 1, hs = j & 1;   // word and half of channel j in each part
          const uint2 wh = {pack_halves(b[0].w[d], b[1].w[d], hs), pack_halves(b[2].w[d], b[3].w[d], hs)};
          const uint2 wl = {pack_halves(b[0].w[V / 2 + d], b[1].w[V / 2 + d], hs),
                            pack_halves(b[2].w[V / 2 + d], b[3].w[V / 2 + d], hs)};
          const h4 ph = __builtin_bit_cast(h4, wh), pl = __builtin_bit_cast(h4, wl);
          f4 c = acc[j];
          c = __builtin_amdgcn_mfma_f32_16x16x16f16(al, ph, c, 0, 0, 0);
          c = __builtin_amdgcn_mfma_f32_16x16x16f16(ah, pl, c, 0, 0, 0);
          acc[j] = __builtin_amdgcn_mfma_f32_16x16x16f16(ah, ph, c, 0, 0, 0);
        }
      };
      h4 ah, al;
      for (int m1 = 0; m1 < d1; m1 += 2) {
        if (m1 + 1 < d1) load_k(m1 + 1, b1);
        coupling(m1, ah, al);
        __builtin_amdgcn_sched_barrier(0);
        mul_k(ah, al, b0);
        if (m1 + 1 < d1) {
          if (m1 + 2 < d1) load_k(m1 + 2, b0);
          coupling(m1 + 1, ah, al);
          __builtin_amdgcn_sched_barrier(0);
          mul_k(ah, al, b1);
        }
      }
    }
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const float f = scale / __shfl(srow, 4 * q + i, 64);   // 1/s of row 4q + i is exact
      const int kkl = (kt - L.g_tile0[g]) * 16 + 4 * q + i;
      if (kkl >= L.g_kcount[g]) continue;
      float o[V];
#pragma unroll
      for (int j = 0; j < V; ++j) {
        o[j] = acc[j][i] * f;
        zmax = fmaxf(zmax, fabsf(o[j]));
      }
      float* zp = Z + ((int64_t)n * L.KT + L.g_kstart[g] + kkl) * C + V * r;
      if constexpr (V >= 4) {
#pragma unroll
        for (int h = 0; h < V / 4; ++h) st4(zp + 4 * h, f4{o[4 * h], o[4 * h + 1], o[4 * h + 2], o[4 * h + 3]});
      } else {
        *reinterpret_cast<float2*>(zp) = make_float2(o[0], o[1]);
      }
    }
  }
  for (int off = 32; off > 0; off >>= 1) zmax = fmaxf(zmax, __shfl_xor(zmax, off, 64));
  float* zm = zmx[done++ & 1];
  if (lane == 0) zm[wave] = zmax;
  __syncthreads();
  if (threadIdx.x == 0) zscale[n] = pow2_scale(fmaxf(fmaxf(zm[0], zm[1]), fmaxf(zm[2], zm[3])));
  }
}

// ---------------------------------------------------------------- channel mix
// out[n][oo_k3 + m][o] = sum_{p -> k3} sum_i W[gate_p][o][i] Z[n][koff_p + m][i] (blockIdx.y = output key k3).
// A GEMM over rows (n, m) with K = (path, input channel) in steps of 32 channels.  Split-fp16 products
// (mfma_x3): the A rows of node n are scaled by ascale[n] (zscale from project_fwd) and split as they
// are loaded, the weights are split once by prepare_mix_kernel
// and stored per (gate, K step) in MFMA lane order ([plane h/l][16-column tile][lane][8]), so one K step's
// weights are a contiguous 64 C-half block: it is copied into LDS with direct-to-LDS loads (no registers)
// one step ahead, double-buffered, and read conflict-free by every wave of the block (the weights are
// read from L2 once per block instead of once per wave).  The A rows of the next step are requested
// before the current step's products.  A wave takes RT 16-row tiles over all C output columns.
template <int C>
constexpr int mix_step_halves() { return 2 * (C / 16) * 512; }

typedef __attribute__((address_space(1))) void global_void;
typedef __attribute__((address_space(3))) void lds_void;

template <int C, int RT>
__global__ __launch_bounds__(256, 2) void mix_kernel(FscIctdLayout L, const float* __restrict__ A,
                                                  const float* __restrict__ ascale,
                                                  const _Float16* __restrict__ Wsw, const float* __restrict__ winv,
                                                  float* __restrict__ out, int64_t N) {
  constexpr int CT = C / 16, KS = C / 32, SH = mix_step_halves<C>();
  static_assert(SH % 512 == 0, "a K step's weights are whole 1 KiB wave copies");
  __shared__ __align__(16) _Float16 sw[2][SH];
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int r = lane & 15, q = lane >> 4;
  const int key = blockIdx.y;
  const int d = L.k_d[key], oo = L.k_oo[key];
  int p0 = 0;
  while (p0 < L.NP && L.p_oo[p0] != oo) ++p0;
  // next path of the key after p (NP: none)
  auto next_path = [&](int p) {
    ++p;
    while (p < L.NP && L.p_oo[p] != oo) ++p;
    return p;
  };
  const int64_t rows = N * d;
  // the grid is sized for the key with the most components: blocks past this key's rows have no work
  if ((int64_t)blockIdx.x * 4 * 16 * RT >= rows) return;   // block-uniform
  const int64_t row0 = ((int64_t)blockIdx.x * 4 + wave) * 16 * RT;
  const bool active = row0 < rows;   // wave-uniform; inactive waves still copy weights and meet the barriers
  // Z row of tile u (+ koff_p; row indices < 2^31, checked by the host), -1: past the end
  int abase[RT];
  float as[RT];
#pragma unroll
  for (int u = 0; u < RT; ++u) {
    const int arow = (int)row0 + 16 * u + r;
    const bool ok = active && arow < rows;
    const int an = ok ? arow / d : 0;
    const int am = ok ? arow - an * d : 0;
    abase[u] = ok ? an * L.KT + am : -1;
    as[u] = ascale[an];
  }
  const int64_t gstride = (int64_t)KS * SH;   // halves per gate
  // one K step's weights into LDS buffer b: whole 1 KiB copies, 16 bytes per lane
  auto stage = [&](int p, int t, int b) {
    const _Float16* src = Wsw + L.p_gate[p] * gstride + (int64_t)t * SH;
#pragma unroll
    for (int c = wave * 512; c < SH; c += 4 * 512) {
      __builtin_amdgcn_global_load_lds((global_void*)(src + c + lane * 8), (lds_void*)(&sw[b][c]), 16, 0, 0);
    }
  };
  auto load_a = [&](int p, int t, f4 (&z)[RT][2]) {
    const int koff = L.p_koff[p];
#pragma unroll
    for (int u = 0; u < RT; ++u) {
      const float* ar = A + (int64_t)(abase[u] + koff) * C + 32 * t + 8 * q;
      z[u][0] = abase[u] >= 0 ? ld4(ar) : f4{0.f, 0.f, 0.f, 0.f};
      z[u][1] = abase[u] >= 0 ? ld4(ar + 4) : f4{0.f, 0.f, 0.f, 0.f};
    }
  };
  f4 acc[RT][CT];
#pragma unroll
  for (int u = 0; u < RT; ++u)
#pragma unroll
    for (int ct = 0; ct < CT; ++ct) acc[u][ct] = f4{0.f, 0.f, 0.f, 0.f};
  // K steps in pairs with fixed A buffers (no loop-carried register moves)
  f4 za[RT][2], zb[RT][2];
  int p = p0, t = 0, buf = 0;
  if (p < L.NP) {
    stage(p, 0, 0);
    load_a(p, 0, za);
  }
  auto step = [&](const f4 (&zc)[RT][2], f4 (&zn)[RT][2]) {
    // this step's weights are in LDS for every wave, and the other buffer is free
    __builtin_amdgcn_s_waitcnt(0);
    __syncthreads();
    const int tn = t + 1 < KS ? t + 1 : 0;
    const int pn = t + 1 < KS ? p : next_path(p);
    if (pn < L.NP) stage(pn, tn, buf ^ 1);
    h8 ah[RT], al[RT];
#pragma unroll
    for (int u = 0; u < RT; ++u) {
      const float v[8] = {zc[u][0].x, zc[u][0].y, zc[u][0].z, zc[u][0].w,
                          zc[u][1].x, zc[u][1].y, zc[u][1].z, zc[u][1].w};
      split2h(v, as[u], ah[u], al[u]);
    }
    __builtin_amdgcn_sched_barrier(0);
    if (pn < L.NP) load_a(pn, tn, zn);
    if (active) {
      const _Float16* wb = &sw[buf][lane * 8];
      // a column tile's weights are read from LDS while the previous tile's products run
#pragma unroll
      for (int ct = 0; ct < CT; ++ct) {
        const h8 bh = *reinterpret_cast<const h8*>(wb + ct * 512);
        const h8 bl = *reinterpret_cast<const h8*>(wb + (CT + ct) * 512);
#pragma unroll
        for (int u = 0; u < RT; ++u) acc[u][ct] = mfma_x3(ah[u], al[u], bh, bl, acc[u][ct]);
        __builtin_amdgcn_sched_barrier(0);
      }
    }
    p = pn;
    t = tn;
    buf ^= 1;
  };
  while (p < L.NP) {
    step(za, zb);
    if (p >= L.NP) break;
    step(zb, za);
  }
  if (!active) return;
  const float wi = winv[0];
#pragma unroll
  for (int u = 0; u < RT; ++u)
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const int row = (int)row0 + 16 * u + 4 * q + i;
      if (row >= rows) continue;
      const int nn = row / d;
      const int m = row - nn * d;
      const float f = wi / ascale[nn];   // a power of two: exact
      float* o = out + (int64_t)(nn * L.M + oo + m) * C;
#pragma unroll
      for (int ct = 0; ct < CT; ++ct) o[16 * ct + r] = acc[u][ct][i] * f;
    }
}

// Backward of the channel mix, dZ[n][koff_p + m][i] = sum_o W[gate_p][o][i] G[n][oo_p + m][o]
// (blockIdx.y = path p): one path per block, so all its K steps stay in LDS (2 C^2 halves, staged once)
// and the block runs TPB row tiles of 64 RT rows with no further barrier; each wave walks its 16 RT-row
// tiles with the A rows of the next K step (possibly of its next tile) requested before the current
// products.  Split-fp16 as in mix_kernel.
template <int C, int RT, int TPB>
__global__ __launch_bounds__(256, 2) void mix_grad_kernel(FscIctdLayout L, const float* __restrict__ G,
                                                       const float* __restrict__ gscale,
                                                       const _Float16* __restrict__ Wsw,
                                                       const float* __restrict__ winv, float* __restrict__ dZ,
                                                       int64_t N) {
  constexpr int CT = C / 16, KS = C / 32, SH = mix_step_halves<C>();
  __shared__ __align__(16) _Float16 sw[KS * SH];
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int r = lane & 15, q = lane >> 4;
  const int p = blockIdx.y;
  const int d = L.p_d3[p], oo = L.p_oo[p], koff = L.p_koff[p];
  const int rows = (int)(N * d);
  const int wtiles = (rows + 16 * RT - 1) / (16 * RT);            // 16 RT-row wave tiles of the path
  const int w0 = blockIdx.x * 4 * TPB;
  if (w0 >= wtiles) return;                                        // block-uniform
  {
    const _Float16* src = Wsw + (int64_t)L.p_gate[p] * KS * SH;
    for (int c = wave * 512; c < KS * SH; c += 4 * 512)
      __builtin_amdgcn_global_load_lds((global_void*)(src + c + lane * 8), (lds_void*)(&sw[c]), 16, 0, 0);
    __builtin_amdgcn_s_waitcnt(0);
    __syncthreads();
  }
  const int wend = min(w0 + 4 * TPB, wtiles);
  // A rows of wave tile wt: base index of G row (n, oo + m), -1 past the end; the node's scale
  auto rows_of = [&](int wt, int (&ab)[RT], float (&as)[RT]) {
#pragma unroll
    for (int u = 0; u < RT; ++u) {
      const int arow = wt * 16 * RT + 16 * u + r;
      const bool ok = wt < wend && arow < rows;
      const int an = ok ? arow / d : 0;
      ab[u] = ok ? an * L.M + oo + (arow - an * d) : -1;
      as[u] = gscale[an];
    }
  };
  auto load_a = [&](const int (&ab)[RT], int t, f4 (&z)[RT][2]) {
#pragma unroll
    for (int u = 0; u < RT; ++u) {
      const float* ar = G + (int64_t)ab[u] * C + 32 * t + 8 * q;
      z[u][0] = ab[u] >= 0 ? ld4(ar) : f4{0.f, 0.f, 0.f, 0.f};
      z[u][1] = ab[u] >= 0 ? ld4(ar + 4) : f4{0.f, 0.f, 0.f, 0.f};
    }
  };
  const float wi = winv[0];
  int wt = w0 + wave;
  if (wt >= wend) return;                                          // wave-uniform, no barrier follows
  int ab[RT], abn[RT];
  float as[RT], asn[RT];
  rows_of(wt, ab, as);
  f4 za[RT][2], zb[RT][2];
  load_a(ab, 0, za);
  // one wave tile, its A rows for K step 0 in z0; the K steps alternate between the two buffers, and the
  // last one requests the next tile's first step (into z0 when KS is even, else into z1)
  auto tile = [&](f4 (&z0)[RT][2], f4 (&z1)[RT][2]) {
    f4 acc[RT][CT];
#pragma unroll
    for (int u = 0; u < RT; ++u)
#pragma unroll
      for (int ct = 0; ct < CT; ++ct) acc[u][ct] = f4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int t = 0; t < KS; ++t) {
      __builtin_amdgcn_sched_barrier(0);
      f4 (&zc)[RT][2] = (t & 1) ? z1 : z0;
      f4 (&zn)[RT][2] = (t & 1) ? z0 : z1;
      h8 ah[RT], al[RT];
#pragma unroll
      for (int u = 0; u < RT; ++u) {
        const float v[8] = {zc[u][0].x, zc[u][0].y, zc[u][0].z, zc[u][0].w,
                            zc[u][1].x, zc[u][1].y, zc[u][1].z, zc[u][1].w};
        split2h(v, as[u], ah[u], al[u]);
      }
      __builtin_amdgcn_sched_barrier(0);
      if (t + 1 < KS) {
        load_a(ab, t + 1, zn);
      } else {
        rows_of(wt + 4, abn, asn);
        load_a(abn, 0, zn);
      }
      const _Float16* wb = &sw[t * SH + lane * 8];
#pragma unroll
      for (int ct = 0; ct < CT; ++ct) {
        const h8 bh = *reinterpret_cast<const h8*>(wb + ct * 512);
        const h8 bl = *reinterpret_cast<const h8*>(wb + (CT + ct) * 512);
#pragma unroll
        for (int u = 0; u < RT; ++u) acc[u][ct] = mfma_x3(ah[u], al[u], bh, bl, acc[u][ct]);
        __builtin_amdgcn_sched_barrier(0);
      }
    }
#pragma unroll
    for (int u = 0; u < RT; ++u)
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const int row = wt * 16 * RT + 16 * u + 4 * q + i;
        if (row >= rows) continue;
        const int nn = row / d;
        const float f = wi / gscale[nn];   // a power of two: exact
        float* o = dZ + (int64_t)(nn * L.KT + koff + row - nn * d) * C;
#pragma unroll
        for (int ct = 0; ct < CT; ++ct) o[16 * ct + r] = acc[u][ct][i] * f;
      }
    wt += 4;
#pragma unroll
    for (int u = 0; u < RT; ++u) {
      ab[u] = abn[u];
      as[u] = asn[u];
    }
  };
  while (wt < wend) {
    tile(za, zb);
    if constexpr (KS % 2 == 1) {
      if (wt >= wend) break;
      tile(zb, za);
    }
  }
}

// ---------------------------------------------------------------- gate and harmonic gradients (one block per receiver)
// With g = dZ[n] / deg, per edge e and column j = (m1, kk) of the projection:
//   H[e][j]      = sum_i x[src_e][o1+m1][i] g[kk][i]                  (MFMA, K = channels)
//   BG'[e][j]    = sum_y Y_e[y] Cf[y][j]                               (the ungated coupling rows, MFMA, K = y)
//   dgate[e][p]  = sum_{j in p} H[e][j] BG'[e][j]
//   dY[e][y]     = sum_j H[e][j] gate_e[p(j)] Cf[y][j]                 (MFMA, K = kk)
// Every output belongs to one edge, so each wave takes whole 16-edge chunks of the receiver (chunk c goes
// to wave c mod 4) over all kk tiles: no reduction crosses waves and the edge loop has no barrier.  H is
// formed transposed (A = g rows, B = x rows: lane (r, q) holds H[edge r][kk rows 4q..4q+3]), which is the
// A-operand layout of the dY product; the coupling rows come out in the same layout from A = Cf, B = Y.
// The per-path sums of dgate are runs of kk rows inside a tile: the tile's products go to a wave-private
// LDS block, the lanes of an edge sum different runs and accumulate them per edge and path.  The 1/deg of
// g is applied to the outputs.
// The input gradient dx = sum_{e: src=m} bg_e^T g_dst(e) is not formed here: it is the dual projection
// (project_fwd_h16_kernel over the source grouping with the dual layout) followed by the channel mix with the
// transposed weights, so no per-edge [M][C] gradient is stored.
struct GradSmem {
  int cgs, kd, gidx, slot0, runs, nrun, cf, dgs, pl, total;
};

// Row stride (floats) of a slot's Cf[y][kk] in the gradient kernel's LDS: with 20, a lane (r, q) reading
// Cf[4q + j][r] (fixed j) and one reading the float4 Cf[r][4q .. 4q + 3] both meet every bank once per
// 16-lane group (16 was four lanes per bank).
constexpr int CFS = 20;

__host__ __device__ inline GradSmem grad_smem(const FscIctdLayout& L, int ncg) {
  GradSmem s;
  int o = 0;
  s.cgs = o;   o += up4(ncg);
  s.kd = o;    o += 4 * L.KT;
  s.gidx = o;  o += 16 * L.KTT;
  s.slot0 = o; o += up4(L.KTT + 1);
  s.runs = o;  o += 16 * L.KTT;            // path runs of each tile: p | first row << 8 | end row << 16
  s.nrun = o;  o += up4(L.KTT);
  s.cf = o;    o += n_slots(L) * 16 * CFS; // Cf[slot][y][kk row], slot = (tile, m1), rows CFS apart
  s.dgs = o;   o += up4(4 * 16 * L.NP);   // per wave: dgate[e][p] of the chunk
  s.pl = o;    o += 4 * 16 * CFS;          // per wave: one tile's H.BG' row sums, rows CFS apart
  s.total = o;
  return s;
}

__device__ __forceinline__ void stage_grad_tables(const FscIctdLayout& L, const float* __restrict__ cg, int ncg,
                                                  float* __restrict__ cgs, int4* __restrict__ kd,
                                                  int* __restrict__ gidx, int* __restrict__ slot0,
                                                  int* __restrict__ runs, int* __restrict__ nrun,
                                                  float* __restrict__ cf) {
  stage_descriptors(L, cg, ncg, cgs, kd, slot0);
  __syncthreads();
  if (threadIdx.x < L.KTT) {
    const int t = threadIdx.x, g = L.tile_group[t];
    const int tb = (t - L.g_tile0[g]) * 16, rows = min(16, L.g_kcount[g] - tb);
    const int4* kt0 = kd + L.g_kstart[g] + tb;
    int k = 0;
    for (int rb = 0; rb < rows;) {
      const int p = kt0[rb].w;
      int re = rb + 1;
      while (re < rows && kt0[re].w == p) ++re;
      runs[t * 16 + k++] = p | (rb << 8) | (re << 16);
      rb = re;
    }
    nrun[t] = k;
  }
  for (int i = threadIdx.x; i < 16 * L.KTT; i += blockDim.x) {
    const int t = i >> 4, r = i & 15, g = L.tile_group[t];
    const int kkl = (t - L.g_tile0[g]) * 16 + r;
    gidx[i] = kkl < L.g_kcount[g] ? kd[L.g_kstart[g] + kkl].z : 0;
  }
  const int nslot = slot0[L.KTT];
  for (int i = threadIdx.x; i < nslot * 256; i += blockDim.x) {
    const int sl = __builtin_amdgcn_readfirstlane(i >> 8), y = (i >> 4) & 15, r = i & 15;
    const int t = tile_of_slot(L, slot0, sl);
    const int g = L.tile_group[t], m1 = sl - slot0[t];
    const int kkl = (t - L.g_tile0[g]) * 16 + r;
    float v = 0.f;
    if (kkl < L.g_kcount[g]) {
      const int4 d = kd[L.g_kstart[g] + kkl];
      const int m2 = y - (d.y & 255), d2 = (d.y >> 8) & 255, d3 = d.y >> 16;
      if (m2 >= 0 && m2 < d2) v = cgs[d.x + (m1 * d2 + m2) * d3];
    }
    cf[(sl * 16 + y) * CFS + r] = v;
  }
}

// The product H = g x^T, whose K dimension is the channels, runs on v_mfma_f32_16x16x32_f16 with three
// products per K step (mfma_x3, 22 significant bits).  The x rows come pre-split per node
// (split_rows_h16_kernel: two fp16 planes of x[n] nu_n, nu_n a power of two per node, and 1/nu_n), so the
// edge loop only loads them; the g rows of a tile are split as they arrive, each kk row with its own power
// of two (a row spans the four lanes (r, 0..3), K = 8q..8q+7 of every 32-channel step).  H[edge r][kk 4q+i]
// is then unscaled by 1/(a_kk nu_src), exact powers of two.  K step s takes channels 32s + 8q .. 32s + 8q + 7
// in both operands.  The chunk walks the path groups in order, so the one or two kk tiles of a group share
// each loaded x row (a row is gathered once per chunk); a component's row (both planes, all K steps) is
// loaded one component ahead, across group boundaries.  At C 128 the kernel holds both tiles' split g rows
// and two x rows: 2 waves/SIMD (measured faster than 3 with the spills that needs).
__global__ __launch_bounds__(256) void split_rows_h16_kernel(int64_t N, int len, const float* __restrict__ X,
                                                             _Float16* __restrict__ hi, _Float16* __restrict__ lo,
                                                             float* __restrict__ inv_scale) {
  const int64_t n = (int64_t)blockIdx.x * 4 + (threadIdx.x >> 6);
  const int lane = threadIdx.x & 63;
  if (n >= N) return;   // uniform over the wave
  const f4* x4 = reinterpret_cast<const f4*>(X + n * len);
  const int n4 = len >> 2;   // len is a multiple of 4 (C >= 32)
  float mx = 0.f;
  for (int i = lane; i < n4; i += 64) {
    const f4 a = x4[i];
#pragma unroll
    for (int j = 0; j < 4; ++j) mx = fmaxf(mx, fabsf(a[j]));
  }
  for (int off = 32; off > 0; off >>= 1) mx = fmaxf(mx, __shfl_xor(mx, off, 64));
  const float s = pow2_scale(mx);
  typedef _Float16 h4 __attribute__((ext_vector_type(4)));
  h4* h = reinterpret_cast<h4*>(hi + n * len);
  h4* l = reinterpret_cast<h4*>(lo + n * len);
  for (int i = lane; i < n4; i += 64) {
    const f4 a = x4[i];
    h4 vh, vl;
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const float v = a[j] * s;
      const _Float16 t = (_Float16)v;
      vh[j] = t;
      vl[j] = (_Float16)(v - (float)t);
    }
    h[i] = vh;
    l[i] = vl;
  }
  if (lane == 0) inv_scale[n] = 1.f / s;   // exact: s is a power of two
}

// The split of split_rows_h16_kernel in the layout of project_fwd_h16_kernel: per row, the C channels in
// groups of V, each group its V high halves followed by its V low halves (2C halves per row).
template <int V>
__global__ __launch_bounds__(256) void split_rows_il_kernel(int64_t N, int len, const float* __restrict__ X,
                                                            _Float16* __restrict__ xs, float* __restrict__ inv_scale) {
  const int64_t n = (int64_t)blockIdx.x * 4 + (threadIdx.x >> 6);
  const int lane = threadIdx.x & 63;
  if (n >= N) return;   // uniform over the wave
  const f4* x4 = reinterpret_cast<const f4*>(X + n * len);
  const int n4 = len >> 2;   // len is a multiple of 4 (C >= 32)
  float mx = 0.f;
  for (int i = lane; i < n4; i += 64) {
    const f4 a = x4[i];
#pragma unroll
    for (int j = 0; j < 4; ++j) mx = fmaxf(mx, fabsf(a[j]));
  }
  for (int off = 32; off > 0; off >>= 1) mx = fmaxf(mx, __shfl_xor(mx, off, 64));
  const float s = pow2_scale(mx);
  typedef _Float16 h2 __attribute__((ext_vector_type(2)));
  typedef _Float16 h4 __attribute__((ext_vector_type(4)));
  _Float16* row = xs + 2 * n * len;
  for (int i = lane; i < n4; i += 64) {
    const f4 a = x4[i];
    h4 vh, vl;
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const float v = a[j] * s;
      const _Float16 t = (_Float16)v;
      vh[j] = t;
      vl[j] = (_Float16)(v - (float)t);
    }
    const int c = 4 * i;   // first of the four values within the node's len
    if constexpr (V >= 4) {
      _Float16* g = row + 2 * (c - c % V) + c % V;
      *reinterpret_cast<h4*>(g) = vh;
      *reinterpret_cast<h4*>(g + V) = vl;
    } else {   // V = 2: two groups
      *reinterpret_cast<h2*>(row + 2 * c) = h2{vh[0], vh[1]};
      *reinterpret_cast<h2*>(row + 2 * c + 2) = h2{vl[0], vl[1]};
      *reinterpret_cast<h2*>(row + 2 * c + 4) = h2{vh[2], vh[3]};
      *reinterpret_cast<h2*>(row + 2 * c + 6) = h2{vl[2], vl[3]};
    }
  }
  if (lane == 0) inv_scale[n] = 1.f / s;   // exact: s is a power of two
}

template <int C>
__global__ __launch_bounds__(256, C >= 128 ? 2 : 3) void project_grad_h16_kernel(
    FscIctdLayout L, int ncg, const float* __restrict__ dZ, const _Float16* __restrict__ xhi,
    const _Float16* __restrict__ xlo, const float* __restrict__ xinv, const float* __restrict__ Y,
    const float* __restrict__ gates, const float* __restrict__ cg, const int32_t* __restrict__ dst_ptr,
    const int32_t* __restrict__ esrc, float* __restrict__ dgates, float* __restrict__ dY, int64_t n_nodes,
    const int32_t* __restrict__ node_order) {
  constexpr int KS = C / 32;                           // K steps of 32 channels (3 fp16 MFMAs each)
  extern __shared__ __align__(16) float smem[];
  const GradSmem sm = grad_smem(L, ncg);
  const int* slot0 = reinterpret_cast<const int*>(smem + sm.slot0);
  const int* gidx = reinterpret_cast<const int*>(smem + sm.gidx);
  const int* runs = reinterpret_cast<const int*>(smem + sm.runs);
  const int* nrun = reinterpret_cast<const int*>(smem + sm.nrun);
  const float* cf = smem + sm.cf;

  if (xcd_node_k(n_nodes, node_order, 0) == -2) return;   // block-uniform
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int r = lane & 15, q = lane >> 4;
  stage_grad_tables(L, cg, ncg, smem + sm.cgs, reinterpret_cast<int4*>(smem + sm.kd),
                    reinterpret_cast<int*>(smem + sm.gidx),
                    reinterpret_cast<int*>(smem + sm.slot0), reinterpret_cast<int*>(smem + sm.runs),
                    reinterpret_cast<int*>(smem + sm.nrun), smem + sm.cf);
  __syncthreads();
  float* dgs = smem + sm.dgs + wave * 16 * L.NP + r * L.NP;   // edge r's path sums (lanes (r, *))
  float* pl = smem + sm.pl + wave * 16 * CFS;                  // the tile's H.BG' row sums, [edge][kk row]
  auto wave_sync = [] {
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
    __builtin_amdgcn_wave_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
  };

  int flat = 0;
  for (int k = 0;; ++k) {
  const int n = xcd_node_k(n_nodes, node_order, k);
  if (n == -2) break;
  if (n < 0) continue;
  const int beg = dst_ptr[n], end = dst_ptr[n + 1];
  const float scale = 1.f / (float)max(end - beg, 1);
  const int nchunk = (end - beg + EB - 1) / EB;
  const int c0 = (wave - flat) & 3;
  flat += nchunk;
  for (int c = c0; c < nchunk; c += 4) {
    const int eb = beg + c * EB, cnt = min(EB, end - eb);
    const bool live = r < cnt;
    const int er = min(eb + r, end - 1);                // the last edge stands in beyond the chunk
    const int src = esrc[er];
    const _Float16* xhr = xhi + (int64_t)src * L.M * C + 8 * q;
    const _Float16* xlr = xlo + (int64_t)src * L.M * C + 8 * q;
    const float xi = xinv[src];
    f4 yop = f4{0.f, 0.f, 0.f, 0.f};
    if (live) {
      const float* yr = Y + (int64_t)er * L.NY;
      if (L.NY == 16 && (reinterpret_cast<uintptr_t>(Y) & 15) == 0) {
        yop = reinterpret_cast<const f4*>(yr)[q];
      } else {
#pragma unroll
        for (int s = 0; s < 4; ++s)
          if (4 * q + s < L.NY) yop[s] = yr[4 * q + s];
      }
    }
    for (int p = q; p < L.NP; p += 4) dgs[p] = 0.f;
    f4 dy = f4{0.f, 0.f, 0.f, 0.f};

    // g rows of tile kt (A operand: kk row r, channels 32 s + 8 q ..; zero beyond the group's rows) split
    // with a power of two a_kk per kk row; inv = 1/(a_kk nu_src) of result rows kk = 4q + i; gt = the gates
    // of kk rows 4q..4q+3 for edge r
    auto load_tile = [&](int kt, h8 (&ah)[KS], h8 (&al)[KS], f4& inv, f4& gt) {
      const int g = L.tile_group[kt];
      const int tb = (kt - L.g_tile0[g]) * 16;
      const bool okr = tb + r < L.g_kcount[g];
      const float* gr = dZ + ((int64_t)n * L.KT + L.g_kstart[g] + (okr ? tb + r : 0)) * C + 8 * q;
      f4 ga[2 * KS];
#pragma unroll
      for (int s = 0; s < KS; ++s) {
        ga[2 * s] = okr ? ld4(gr + 32 * s) : f4{0.f, 0.f, 0.f, 0.f};
        ga[2 * s + 1] = okr ? ld4(gr + 32 * s + 4) : f4{0.f, 0.f, 0.f, 0.f};
      }
#pragma unroll
      for (int i = 0; i < 4; ++i) gt[i] = live ? gates[(int64_t)er * L.NREF + gidx[kt * 16 + 4 * q + i]] : 0.f;
      float mx = 0.f;
#pragma unroll
      for (int s = 0; s < 2 * KS; ++s)
#pragma unroll
        for (int j = 0; j < 4; ++j) mx = fmaxf(mx, fabsf(ga[s][j]));
      mx = fmaxf(mx, __shfl_xor(mx, 16, 64));
      mx = fmaxf(mx, __shfl_xor(mx, 32, 64));
      const float a = pow2_scale(mx);
#pragma unroll
      for (int s = 0; s < KS; ++s) {
        const float v[8] = {ga[2 * s].x, ga[2 * s].y, ga[2 * s].z, ga[2 * s].w,
                            ga[2 * s + 1].x, ga[2 * s + 1].y, ga[2 * s + 1].z, ga[2 * s + 1].w};
        split2h(v, a, ah[s], al[s]);
      }
#pragma unroll
      for (int i = 0; i < 4; ++i) inv[i] = __shfl(1.f / a, 4 * q + i, 64) * xi;   // exact: powers of two
    };
    // x row of component m, both planes, every K step
    auto load_row = [&](int m, h8 (&bh)[KS], h8 (&bl)[KS]) {
#pragma unroll
      for (int s = 0; s < KS; ++s) {
        bh[s] = *reinterpret_cast<const h8*>(xhr + m * C + 32 * s);
        bl[s] = *reinterpret_cast<const h8*>(xlr + m * C + 32 * s);
      }
    };
    // the products of component m1 of tile kt from the x row in (bh, bl)
    auto product = [&](int kt, int m1, const h8 (&bh)[KS], const h8 (&bl)[KS], const h8 (&ah)[KS],
                       const h8 (&al)[KS], const f4& inv, const f4& gt, f4& P) {
      f4 ht = f4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
      for (int s = 0; s < KS; ++s) ht = mfma_x3(ah[s], al[s], bh[s], bl[s], ht);
#pragma unroll
      for (int i = 0; i < 4; ++i) ht[i] *= inv[i];                             // H[edge r][kk 4q+i]
      const float* cs = cf + (slot0[kt] + m1) * 16 * CFS;
      f4 ca;
#pragma unroll
      for (int j = 0; j < 4; ++j) ca[j] = cs[(4 * q + j) * CFS + r];        // Cf[y = 4q+j][kk = r]
      const f4 ct = *reinterpret_cast<const f4*>(cs + r * CFS + 4 * q);     // Cf[y = r][kk = 4q..4q+3]
      const f4 bgt = mfma_k16(ca, yop, f4{0.f, 0.f, 0.f, 0.f});              // BG'[edge r][kk 4q+i]
      f4 hg;
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        P[i] += ht[i] * bgt[i];
        hg[i] = ht[i] * gt[i];
      }
      dy = mfma_k16(hg, ct, dy);                                             // dY[edge 4q+i][y = r]
    };
    // groups in order; a group's (one or two) tiles share each loaded x row
    h8 b0h[KS], b0l[KS], b1h[KS], b1l[KS];
    load_row(L.g_o1[0], b0h, b0l);
    for (int g = 0; g < L.NG; ++g) {
      const int d1 = L.g_d1[g], o1 = L.g_o1[g];
      const int t0 = L.g_tile0[g], nt = L.g_kpad[g] / 16;      // 1 or 2
      const bool more = g + 1 < L.NG;
      const int o1n = more ? L.g_o1[g + 1] : 0;
      h8 ah[2][KS], al[2][KS];
      f4 inv[2], gt[2], P[2];
#pragma unroll
      for (int tt = 0; tt < 2; ++tt) {
        P[tt] = f4{0.f, 0.f, 0.f, 0.f};
        if (tt < nt) load_tile(t0 + tt, ah[tt], al[tt], inv[tt], gt[tt]);
      }
      auto products = [&](int m1, const h8 (&bh)[KS], const h8 (&bl)[KS]) {
#pragma unroll
        for (int tt = 0; tt < 2; ++tt)
          if (tt < nt) product(t0 + tt, m1, bh, bl, ah[tt], al[tt], inv[tt], gt[tt], P[tt]);
      };
      // b0 holds the row of component m1 on entry to each pair; the row after the group's last is the
      // next group's first
      for (int m1 = 0; m1 < d1; m1 += 2) {
        if (m1 + 1 < d1) load_row(o1 + m1 + 1, b1h, b1l);
        else if (more) load_row(o1n, b1h, b1l);
        __builtin_amdgcn_sched_barrier(0);
        products(m1, b0h, b0l);
        if (m1 + 1 < d1) {
          if (m1 + 2 < d1) load_row(o1 + m1 + 2, b0h, b0l);
          else if (more) load_row(o1n, b0h, b0l);
          __builtin_amdgcn_sched_barrier(0);
          products(m1 + 1, b1h, b1l);
        }
      }
      if ((d1 & 1) && more) {
#pragma unroll
        for (int s = 0; s < KS; ++s) {
          b0h[s] = b1h[s];
          b0l[s] = b1l[s];
        }
      }
      // per-path sums of each tile's rows: lanes (r, q) take runs q, q + 4, ...
#pragma unroll
      for (int tt = 0; tt < 2; ++tt) {
        if (tt >= nt) continue;
        const int kt = t0 + tt;
        *reinterpret_cast<f4*>(pl + r * CFS + 4 * q) = P[tt];
        wave_sync();
        for (int k2 = q; k2 < nrun[kt]; k2 += 4) {
          const int run = runs[kt * 16 + k2];
          const int p = run & 255, rb = (run >> 8) & 255, re = run >> 16;
          float sum = 0.f;
          for (int i = rb; i < re; ++i) sum += pl[r * CFS + i];
          dgs[p] += sum;
        }
        wave_sync();
      }
    }
    if (live)
      for (int p = q; p < L.NP; p += 4) dgates[(int64_t)(eb + r) * L.NREF + L.p_gate[p]] = dgs[p] * scale;
    if (r < L.NY) {
#pragma unroll
      for (int i = 0; i < 4; ++i)
        if (4 * q + i < cnt) dY[(int64_t)(eb + 4 * q + i) * L.NY + r] = dy[i] * scale;
    }
    wave_sync();
  }
  }
}

// ---------------------------------------------------------------- conv1 (species-pair table)
// out[n][comp(y)][o] = (1/deg) sum_{e->n} gate_e[p(y)] F_e[y] q[pair_e][p(y)][o].  The in-edges of n come
// from at most NS species and share n's species, so the edge sum is first folded per source species,
//   w[s][y] = sum_{e->n, src species s} gate_e[p(y)] F_e[y],
// and the table is read once per (s, y) instead of once per edge (a per-edge loop re-read 16 C floats
// of the table from L2 for every edge).  Species ids index the model's species table (NS <= 16 rows);
// only the source species present among the node's in-edges are read.

// ssp[pair] = the source species of species pair (s, t) = s * NS + t, for all 256 pair ids a block may
// look up (NS <= 16).  Filled by a 256-thread block before its first barrier.
__device__ __forceinline__ void fill_pair_species(int NS, int* __restrict__ ssp) {
  ssp[threadIdx.x] = min((int)threadIdx.x / NS, 15);   // ids >= NS * NS are not pairs; kept in bounds
}

// Bit s set if some edge in [beg, end) has source species s (wave 0 computes it; every wave reads it).
// Ends with a barrier, after which ssp (filled before the call) is visible to the block.
__device__ __forceinline__ unsigned src_species_mask(const int32_t* __restrict__ edge_pair, const int* __restrict__ ssp,
                                                     int NS, int beg, int end, unsigned* lds) {
  if (threadIdx.x < 64) {
    unsigned m = 0;
    for (int e = beg + (int)threadIdx.x; e < end; e += 64) m |= 1u << min((edge_pair[e] & 255) / NS, 15);
    for (int off = 32; off > 0; off >>= 1) m |= (unsigned)__shfl_xor((int)m, off, 64);
    if (threadIdx.x == 0) *lds = m;
  }
  __syncthreads();
  return *lds;
}

template <int C, int NY>
__global__ __launch_bounds__(256) void conv1_fwd_kernel(FscIctdLayout L, int NS, const int32_t* __restrict__ dst_ptr,
                                                        const int32_t* __restrict__ edge_pair,
                                                        const int32_t* __restrict__ node_species,
                                                        const float* __restrict__ F,
                                                        const float* __restrict__ gates,
                                                        const float* __restrict__ qtab, float* __restrict__ out) {
  __shared__ float w[16][NY];
  __shared__ float part[16][16][NY];   // [edge lane][source species][y]
  __shared__ int ycomp[32], yrow[32];   // M <= 32 components
  __shared__ int ssp[256];
  __shared__ unsigned smask;
  const int n = blockIdx.x, t = threadIdx.x;
  const int beg = dst_ptr[n], end = dst_ptr[n + 1];
  const int sn = node_species[n];
  fill_pair_species(NS, ssp);
  if (t < 32) {   // component -> the harmonic y whose path writes it (-1: none) and that path's table row
    int yy = -1;
#pragma unroll
    for (int y = 0; y < NY; ++y)
      if (L.y_path1[y] >= 0 && L.y_oo1[y] == t) yy = y;
    ycomp[t] = yy;
    yrow[t] = yy >= 0 ? L.y_path1[yy] : 0;
  }
  const unsigned mask = src_species_mask(edge_pair, ssp, NS, beg, end, &smask);   // barrier: ssp, ycomp
  {  // thread (edge lane k, y): partial sums over edges beg + k + 16 i, per source species
    const int y = t & 15, k = t >> 4;
    float acc[16];
#pragma unroll
    for (int s2 = 0; s2 < 16; ++s2) acc[s2] = 0.f;
    const int p = y < NY ? L.y_path1[y] : -1;
    if (p >= 0) {
      const int gi = L.c1_gate[p];
      for (int e = beg + k; e < end; e += 16) {
        const float v = gates[(int64_t)e * L.NREF + gi] * F[(int64_t)e * NY + y];
        const int ss = ssp[edge_pair[e] & 255];
#pragma unroll
        for (int s2 = 0; s2 < 16; ++s2) acc[s2] += (ss == s2) ? v : 0.f;
      }
    }
    if (y < NY) {
#pragma unroll
      for (int s2 = 0; s2 < 16; ++s2) part[k][s2][y] = acc[s2];
    }
  }
  __syncthreads();
  if (t < 16 * NY) {   // w[s][y]: the edge lanes added in a fixed order
    const int s2 = t / NY, y = t - s2 * NY;
    float a = 0.f;
#pragma unroll
    for (int k = 0; k < 16; ++k) a += part[k][s2][y];
    w[s2][y] = a;
  }
  __syncthreads();
  const float scale = 1.f / (float)max(end - beg, 1);
  float* on = out + (int64_t)n * L.M * C;
  const int MC = L.M * C;                 // <= 32 * 128: at most two passes of 8 * 256 outputs
  for (int base = 0; base < MC; base += 8 * 256) {
    float v[8];
#pragma unroll
    for (int u = 0; u < 8; ++u) v[u] = 0.f;
    // source species outermost (increasing order), the thread's outputs innermost: their table reads are
    // independent and go out together
    for (unsigned m = mask; m; m &= m - 1) {
      const int s2 = __builtin_ctz(m);
      const float* qs = qtab + ((int64_t)(s2 * NS + sn) * L.NP1) * C;   // pair (s2, sn)
#pragma unroll
      for (int u = 0; u < 8; ++u) {
        const int i = base + t + 256 * u;
        if (i < MC) {
          const int c = i / C, o = i - c * C;
          const int yy = ycomp[c];
          if (yy >= 0) v[u] += w[s2][yy] * qs[yrow[c] * C + o];
        }
      }
    }
#pragma unroll
    for (int u = 0; u < 8; ++u) {
      const int i = base + t + 256 * u;
      if (i < MC) on[i] = v[u] * scale;
    }
  }
}

template <int C, int NY>
__global__ __launch_bounds__(256) void conv1_bwd_kernel(FscIctdLayout L, int NS, const int32_t* __restrict__ dst_ptr,
                                                        const int32_t* __restrict__ edge_pair,
                                                        const int32_t* __restrict__ node_species,
                                                        const float* __restrict__ G, const float* __restrict__ F,
                                                        const float* __restrict__ gates,
                                                        const float* __restrict__ qtab,
                                                        float* __restrict__ dF, float* __restrict__ dgates) {
  __shared__ __align__(16) float gsh[NY][C + 4];   // rows padded: the T threads read 16 rows at once
  __shared__ float T[16][NY];
  __shared__ int ssp[256];
  __shared__ unsigned smask;
  const int n = blockIdx.x;
  const int t = threadIdx.x;
  const int beg = dst_ptr[n], end = dst_ptr[n + 1];
  if (beg == end) return;                      // uniform over the block
  const float scale = 1.f / (float)(end - beg);
  const int sn = node_species[n];
  fill_pair_species(NS, ssp);
  for (int i = t; i < NY * C; i += blockDim.x) {
    const int y = i / C, o = i - y * C;
    gsh[y][o] = (L.y_path1[y] >= 0) ? G[((int64_t)n * L.M + L.y_oo1[y]) * C + o] : 0.f;
  }
  const unsigned mask = src_species_mask(edge_pair, ssp, NS, beg, end, &smask);   // its barrier publishes gsh
  // T[s][y] = (1/deg) sum_o G[n][comp(y)][o] Q[(s, sn)][p(y)][o]: threads (j = (s, y), h) sum the half
  // h of o as float4 runs; a lane exchange adds the two halves.  Rows of absent source species are 0.
  constexpr int HC = C / 2;
  const bool qal = (reinterpret_cast<uintptr_t>(qtab) & 15) == 0;
  for (int j0 = 0; j0 < NS * NY; j0 += 128) {
    const int j = j0 + (t >> 1), h = t & 1;
    const int s = j / NY, y = j - s * NY;
    const int p = j < NS * NY ? L.y_path1[y] : -1;
    float part = 0.f;
    if (p >= 0 && ((mask >> s) & 1u)) {
      const float* qp = qtab + (((int64_t)s * NS + sn) * L.NP1 + p) * C + h * HC;
      const f4* gp = reinterpret_cast<const f4*>(&gsh[y][h * HC]);
      if (qal) {
#pragma unroll 4
        for (int k = 0; k < HC / 4; ++k) {
          const f4 a = reinterpret_cast<const f4*>(qp)[k], g = gp[k];
          part += a[0] * g[0] + a[1] * g[1] + a[2] * g[2] + a[3] * g[3];
        }
      } else {
        for (int k = 0; k < HC / 4; ++k) {
          const f4 g = gp[k];
          part += qp[4 * k] * g[0] + qp[4 * k + 1] * g[1] + qp[4 * k + 2] * g[2] + qp[4 * k + 3] * g[3];
        }
      }
    }
    part += __shfl_xor(part, 1, 64);
    if (h == 0 && j < NS * NY) T[s][y] = part * scale;
  }
  __syncthreads();
  // per edge: dF[e][y] = gate_p(y) T[s_src][y];  dgate[e][p] = sum_{y in p} T[s_src][y] F[e][y]
  const int ne = end - beg;
  for (int idx = t; idx < ne * NY; idx += blockDim.x) {
    const int e = beg + idx / NY, y = idx % NY;
    const int p = L.y_path1[y];
    const int ss = ssp[edge_pair[e] & 255];
    dF[(int64_t)e * NY + y] = (p >= 0) ? gates[(int64_t)e * L.NREF + L.c1_gate[p]] * T[ss][y] : 0.f;
  }
  for (int p = 0; p < L.NP1; ++p) {
    const int gi = L.c1_gate[p];
    for (int e = beg + t; e < end; e += blockDim.x) {
      const int ss = ssp[edge_pair[e] & 255];
      float acc = 0.f;
#pragma unroll
      for (int y = 0; y < NY; ++y)
        if (L.y_path1[y] == p) acc += T[ss][y] * F[(int64_t)e * NY + y];
      dgates[(int64_t)e * L.NREF + gi] = acc;
    }
  }
}

// Prepared channel-mix weights (floats): W times the power of two sw (max |W| sw < 2^14) split into two
// fp16 parts (split2h) as [2][NREF][C (o)][C (i)] for the forward, the same values with the last two axes
// swapped, [2][NREF][C (i)][C (o)], for the backward, then a tail of MIXW_TAIL floats: [0] = 1/sw,
// [256..511] the partial maxima of the preparation.
constexpr int MIXW_TAIL = 512;
// Position (in halves) of weight (row, K column col, fp16 plane) of gate p in a prepared orientation: per
// gate, per K step of 32 columns, [plane][16-row tile][MFMA lane (row % 16) + 16 ((col % 32) / 8)][col % 8],
// the image mix_kernel copies into LDS per step.
__host__ __device__ inline int64_t mix_pos(int C, int64_t p, int row, int col, int plane) {
  const int CT = C / 16;
  const int lane = (row & 15) + 16 * ((col & 31) >> 3);
  return p * 2 * C * C + ((int64_t)((col >> 5) * 2 + plane) * CT + (row >> 4)) * 512 + lane * 8 + (col & 7);
}
__host__ __device__ inline int64_t mix_weight_floats(int n_ref, int C) { return 2LL * n_ref * C * C + MIXW_TAIL; }

// wmax[b] = max |W| over the grid-stride share of block b (grid 256 x 256).
__global__ __launch_bounds__(256) void mix_absmax_kernel(const float* __restrict__ W, int64_t n, float* __restrict__ wmax) {
  __shared__ float red[4];
  float m = 0.f;
  for (int64_t i = blockIdx.x * 256 + threadIdx.x; i < n; i += (int64_t)gridDim.x * 256) m = fmaxf(m, fabsf(W[i]));
  for (int off = 32; off > 0; off >>= 1) m = fmaxf(m, __shfl_xor(m, off, 64));
  if ((threadIdx.x & 63) == 0) red[threadIdx.x >> 6] = m;
  __syncthreads();
  if (threadIdx.x == 0) wmax[blockIdx.x] = fmaxf(fmaxf(red[0], red[1]), fmaxf(red[2], red[3]));
}

// 256 threads per block; every block reduces the 256 partial maxima itself, so all use the same sw.
__global__ __launch_bounds__(256) void prepare_mix_kernel(const float* __restrict__ W, float* __restrict__ Wp,
                                                          int n_ref, int C) {
  const int64_t total = (int64_t)n_ref * C * C;
  __shared__ float red[4];
  float mx = Wp[2 * total + 256 + threadIdx.x];
  for (int off = 32; off > 0; off >>= 1) mx = fmaxf(mx, __shfl_xor(mx, off, 64));
  if ((threadIdx.x & 63) == 0) red[threadIdx.x >> 6] = mx;
  __syncthreads();
  const float sw = pow2_scale(fmaxf(fmaxf(red[0], red[1]), fmaxf(red[2], red[3])));
  if (blockIdx.x == 0 && threadIdx.x == 0) Wp[2 * total] = 1.f / sw;
  _Float16* wf = reinterpret_cast<_Float16*>(Wp);
  _Float16* wb = reinterpret_cast<_Float16*>(Wp + total);
  for (int64_t idx = blockIdx.x * (int64_t)blockDim.x + threadIdx.x; idx < total; idx += (int64_t)gridDim.x * blockDim.x) {
    const int i = (int)(idx % C);
    const int o = (int)((idx / C) % C);
    const int64_t p = idx / ((int64_t)C * C);
    const float v = W[idx] * sw;
    const _Float16 h = (_Float16)v;
    const _Float16 l = (_Float16)(v - (float)h);
    // forward orientation: rows o, K = i; transposed: rows i, K = o
    wf[mix_pos(C, p, o, i, 0)] = h;
    wf[mix_pos(C, p, o, i, 1)] = l;
    wb[mix_pos(C, p, i, o, 0)] = h;
    wb[mix_pos(C, p, i, o, 1)] = l;
  }
}

// nsc[n] = pow2_scale(max |X[n][:]|) over rows of `len` floats; one wave per row.
__global__ __launch_bounds__(256) void row_scale_kernel(int64_t N, int len, const float* __restrict__ X,
                                                        float* __restrict__ nsc) {
  const int64_t n = (int64_t)blockIdx.x * 4 + (threadIdx.x >> 6);
  const int lane = threadIdx.x & 63;
  if (n >= N) return;   // uniform over the wave
  const float* xr = X + n * len;
  float mx = 0.f;
  if ((len & 3) == 0 && (reinterpret_cast<uintptr_t>(X) & 15) == 0) {   // rows of whole float4s: 4 in flight
    const f4* x4 = reinterpret_cast<const f4*>(xr);
    const int n4 = len >> 2;
    int i = lane;
    for (; i + 192 < n4; i += 256) {
      const f4 a = x4[i], b = x4[i + 64], c = x4[i + 128], d = x4[i + 192];
#pragma unroll
      for (int j = 0; j < 4; ++j) mx = fmaxf(mx, fmaxf(fmaxf(fabsf(a[j]), fabsf(b[j])), fmaxf(fabsf(c[j]), fabsf(d[j]))));
    }
    for (; i < n4; i += 64) {
      const f4 a = x4[i];
#pragma unroll
      for (int j = 0; j < 4; ++j) mx = fmaxf(mx, fabsf(a[j]));
    }
  } else {
    for (int i = lane; i < len; i += 64) mx = fmaxf(mx, fabsf(xr[i]));
  }
  for (int off = 32; off > 0; off >>= 1) mx = fmaxf(mx, __shfl_xor(mx, off, 64));
  if (lane == 0) nsc[n] = pow2_scale(mx);
}

// ---------------------------------------------------------------- host side
// Coupling-table length implied by the layout.
int cg_length(const FscIctdLayout& L) {
  int n = 0;
  for (int p = 0; p < L.NP; ++p) n = max(n, L.p_cgoff[p] + L.g_d1[L.p_group[p]] * L.p_d2[p] * L.p_d3[p]);
  return n;
}

int check_layout(const FscIctdLayout* L, int32_t C, const char* who) {
  if (!L) { set_error(std::string(who) + ": null layout"); return 1; }
  if (!(C == 32 || C == 64 || C == 128)) { set_error(std::string(who) + ": channels must be 32, 64 or 128"); return 1; }
  if (L->NG < 1 || L->NG > 8 || L->NP < 1 || L->NP > 64 || L->KT < 1 || L->KT > 128 || L->KTT < 1 ||
      L->KTT > 8 || L->NY < 1 || L->NY > 16 || L->M < 1 || L->M > 32 || L->NREF < L->NP || L->NK < 1 ||
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
  // limits of the projection kernels: <= 32 kk slots per group (2 MFMA tiles), 4-bit component
  // counts in the coupling descriptors, tiles inside their group, LDS within 64 KiB
  int bgoff = 0;
  for (int g = 0; g < L->NG; ++g) {
    if (L->g_kpad[g] < 16 || L->g_kpad[g] > 32 || L->g_d1[g] < 1 || L->g_d1[g] > 15 ||
        L->g_bgoff[g] != bgoff || L->g_kstart[g] < 0 || L->g_kstart[g] + L->g_kcount[g] > L->KT) {
      set_error(std::string(who) + ": path group exceeds the projection kernel limits");
      return 1;
    }
    bgoff += L->g_d1[g] * L->g_kpad[g];
  }
  if (bgoff != L->NBGP || L->NREF > 4096) {
    set_error(std::string(who) + ": coupling table size mismatch");
    return 1;
  }
  for (int t = 0; t < L->KTT; ++t) {
    const int g = L->tile_group[t];
    if (g < 0 || g >= L->NG || t < L->g_tile0[g] || (t - L->g_tile0[g]) * 16 >= L->g_kpad[g]) {
      set_error(std::string(who) + ": kk tile table inconsistent");
      return 1;
    }
  }
  for (int p = 0; p < L->NP; ++p) {
    if (L->p_group[p] < 0 || L->p_group[p] >= L->NG || L->p_d2[p] < 1 || L->p_d2[p] > 15 || L->p_d3[p] < 1 ||
        L->p_d3[p] > 15 || L->p_oy[p] < 0 || L->p_oy[p] + L->p_d2[p] > L->NY || L->p_gate[p] < 0 ||
        L->p_gate[p] >= L->NREF || L->p_koff[p] < 0 || L->p_koff[p] + L->p_d3[p] > L->KT || L->p_cgoff[p] < 0) {
      set_error(std::string(who) + ": path table out of range");
      return 1;
    }
  }
  for (int kk = 0; kk < L->KT; ++kk) {
    if (L->kk_path[kk] < 0 || L->kk_path[kk] >= L->NP) {
      set_error(std::string(who) + ": kk_path out of range");
      return 1;
    }
  }
  if ((size_t)grad_smem(*L, cg_length(*L)).total * sizeof(float) > 65536 ||
      (size_t)fwd_smem(*L, cg_length(*L)).total * sizeof(float) > 65536) {
    set_error(std::string(who) + ": layout needs more than 64 KiB of LDS per block");
    return 1;
  }
  return 0;
}

// ---------------------------------------------------------------- dual layout (input gradient)
// dx_m[o1+m1][i] = sum_p sum_o W[p][o][i] R_m[(p,m1)][o],  R_m[(p,m1)][o] = sum_{e: src=m} sum_m3
// bg_e[m1][(p,m3)] G_dst(e)[oo_p+m3][o] / deg(dst(e)).  R is the forward projection of the layout with every
// path reversed (k3 -> k1: d1 and d3 swapped, coupling C^T[m3][m2][m1], the same gate and harmonic), paths
// grouped by their output key, run over the source grouping of the edges; dx is then the forward channel
// mix of that layout with W^T (the prepared weights hold both orientations).  Built on the host per call.
struct DualMap {
  int32_t p_of[64];   // dual path -> path of the layout
};

int dual_layout(const FscIctdLayout& L, FscIctdLayout& D, DualMap& map) {
  D = L;
  // dual paths: the layout's paths stably ordered by output component offset
  int np = 0;
  for (int pass = 0; pass < L.M; ++pass)
    for (int p = 0; p < L.NP; ++p)
      if (L.p_oo[p] == pass) map.p_of[np++] = p;
  if (np != L.NP) return 1;
  int ng = -1, koff = 0, cgoff = 0, bgoff = 0, tile0 = 0, prev_oo = -1;
  for (int q = 0; q < np; ++q) {
    const int p = map.p_of[q];
    const int g1 = L.p_group[p];
    const int d1 = L.g_d1[g1], d2 = L.p_d2[p], d3 = L.p_d3[p];
    if (L.p_oo[p] != prev_oo) {                         // a new dual group: one output key of the layout
      if (ng >= 0) {
        D.g_kpad[ng] = 16 * ((D.g_kcount[ng] + 15) / 16);
        D.g_bgoff[ng] = bgoff;
        D.g_tile0[ng] = tile0;
        bgoff += D.g_d1[ng] * D.g_kpad[ng];
        tile0 += D.g_kpad[ng] / 16;
      }
      if (++ng >= 8) return 1;
      prev_oo = L.p_oo[p];
      D.g_o1[ng] = L.p_oo[p];
      D.g_d1[ng] = d3;
      D.g_kstart[ng] = koff;
      D.g_kcount[ng] = 0;
    }
    D.g_kcount[ng] += d1;
    D.p_gate[q] = L.p_gate[p];
    D.p_oy[q] = L.p_oy[p];
    D.p_d2[q] = d2;
    D.p_d3[q] = d1;
    D.p_koff[q] = koff;
    D.p_cgoff[q] = cgoff;
    D.p_group[q] = ng;
    D.p_oo[q] = L.g_o1[g1];
    if (koff + d1 > 128) return 1;
    for (int k = 0; k < d1; ++k) D.kk_path[koff + k] = q;
    koff += d1;
    cgoff += d1 * d2 * d3;
  }
  D.g_kpad[ng] = 16 * ((D.g_kcount[ng] + 15) / 16);
  D.g_bgoff[ng] = bgoff;
  D.g_tile0[ng] = tile0;
  bgoff += D.g_d1[ng] * D.g_kpad[ng];
  tile0 += D.g_kpad[ng] / 16;
  D.NG = ng + 1;
  D.KT = koff;
  D.NBGP = bgoff;
  D.KTT = tile0;
  if (D.KTT > 16) return 1;
  for (int g = 0; g < D.NG; ++g)
    for (int t = D.g_tile0[g]; t < D.g_tile0[g] + D.g_kpad[g] / 16; ++t) D.tile_group[t] = g;
  // output keys of the dual mix: the layout's input keys (path groups)
  D.NK = L.NG;
  for (int g = 0; g < L.NG; ++g) {
    D.k_oo[g] = L.g_o1[g];
    D.k_d[g] = L.g_d1[g];
  }
  return 0;
}

// cgd[dual path q][m3][m2][m1] = cg[path p_of[q]][m1][m2][m3]
__global__ __launch_bounds__(256) void transpose_cg_kernel(FscIctdLayout L, FscIctdLayout D, DualMap map,
                                                           const float* __restrict__ cg, float* __restrict__ cgd) {
  const int q = blockIdx.x;
  const int p = map.p_of[q];
  const int d1 = L.g_d1[L.p_group[p]], d2 = L.p_d2[p], d3 = L.p_d3[p];
  const float* src = cg + L.p_cgoff[p];
  float* dst = cgd + D.p_cgoff[q];
  for (int idx = threadIdx.x; idx < d1 * d2 * d3; idx += blockDim.x) {
    const int m3 = idx / (d2 * d1), m2 = (idx / d1) % d2, m1 = idx % d1;
    dst[idx] = src[(m1 * d2 + m2) * d3 + m3];
  }
}


// The projection of a layout into Z [N][KT][C] + N scales.  Forward: blocks are receivers (ptr = dst_ptr),
// the edge at CSR position j is j and gathers x[esrc[j]]; dual (backward): ptr = src_ptr, eperm = src_perm,
// esrc the receiver of each edge, gdeg = dst_ptr.  xws: N*M*C + N floats for the split copy of x.
template <int C, bool DUAL>
int project_c(const FscIctdLayout& L, int64_t N, const int32_t* ptr, const int32_t* esrc, const int32_t* eperm,
              const int32_t* gdeg, const float* x, float* xws, const float* Y, const float* gates, const float* cg,
              float* Z, const int32_t* node_order, const char* timer, hipStream_t st) {
  // the gathered rows as fp16 parts with a power of two per node: 2 N*M*C halves, then N scales
  _Float16* xs = reinterpret_cast<_Float16*>(xws);
  float* xinv = xws + N * L.M * C;
  split_rows_il_kernel<C / 16><<<(unsigned)((N + 3) / 4), 256, 0, st>>>(N, L.M * C, x, xs, xinv);
  if (check_launch("ictd split_rows")) return 2;
  const int ncg = cg_length(L);
  LaunchTimer tm(timer, st);
  const size_t lds = (size_t)fwd_smem(L, ncg).total * sizeof(float);
  project_fwd_h16_kernel<C, DUAL><<<persist_grid(N, (const void*)project_fwd_h16_kernel<C, DUAL>, lds), 256,
                                    lds, st>>>(L, ncg, xs, xinv, Y, gates, cg, ptr, esrc, Z,
                                               Z + N * L.KT * C, N, node_order, eperm, gdeg);
  return check_launch("ictd project") ? 2 : 0;
}

// The projection and channel mix of a layout (project_c, then the mix of Z with the prepared planes Wh).
template <int C, bool DUAL>
int project_mix_c(const FscIctdLayout& L, int64_t N, const int32_t* ptr, const int32_t* esrc, const int32_t* eperm,
                  const int32_t* gdeg, const float* x, float* xws, const float* Y, const float* gates, const float* cg,
                  const _Float16* Wh, const float* winv, float* Z, float* out, const int32_t* node_order,
                  const char* timer_project, const char* timer_mix, hipStream_t st) {
  if (const int rc = project_c<C, DUAL>(L, N, ptr, esrc, eperm, gdeg, x, xws, Y, gates, cg, Z, node_order,
                                        timer_project, st))
    return rc;
  int dmax = 1;
  for (int k = 0; k < L.NK; ++k) dmax = max(dmax, L.k_d[k]);
  {
    LaunchTimer tm(timer_mix, st);
    constexpr int RT = mix_rt<C>();
    dim3 grid((unsigned)((N * dmax + 64 * RT - 1) / (64 * RT)), (unsigned)L.NK);
    mix_kernel<C, RT><<<grid, 256, 0, st>>>(L, Z, Z + N * L.KT * C, Wh, winv, out, N);
  }
  return check_launch("ictd mix_fwd") ? 2 : 0;
}

// Workspace of the forward and of the projection alone: Z [N][KT][C] + N scales, then (256-byte aligned) the
// split copy of x.
int64_t fwd_split_offset(const FscIctdLayout& L, int64_t N, int C) {
  return (N * (int64_t)L.KT * C + N + 63) / 64 * 64;
}

int64_t fwd_ws_floats(const FscIctdLayout& L, int64_t N, int C) {
  return fwd_split_offset(L, N, C) + N * (int64_t)L.M * C + N;
}

template <int C>
int forward_c(const FscIctdLayout& L, int64_t N, const int32_t* dst_ptr, const int32_t* esrc, const float* x,
              const float* Y, const float* gates, const float* cg, const float* W, float* Z, float* out,
              const int32_t* node_order, hipStream_t st) {
  return project_mix_c<C, false>(L, N, dst_ptr, esrc, nullptr, nullptr, x, Z + fwd_split_offset(L, N, C), Y, gates, cg,
                                 reinterpret_cast<const _Float16*>(W), W + mix_weight_floats(L.NREF, C) - MIXW_TAIL,
                                 Z, out, node_order, "ictd_project", "ictd_mix", st);
}

// The receiver-normalised projection Z alone (the first half of the forward), for the weight gradient
// dW[gate_p] = sum_n G_p^T Z_p of the training backward.
template <int C>
int project_only_c(const FscIctdLayout& L, int64_t N, const int32_t* dst_ptr, const int32_t* esrc, const float* x,
                   const float* Y, const float* gates, const float* cg, float* Z, const int32_t* node_order,
                   hipStream_t st) {
  return project_c<C, false>(L, N, dst_ptr, esrc, nullptr, nullptr, x, Z + fwd_split_offset(L, N, C), Y, gates, cg, Z,
                             node_order, "ictd_project", st);
}

// Workspace of the backward: dZ [N][KT][C] + N scales, which once dZ is used hold the split rows of the
// output gradient (N*M*C + N floats); R [N][KT_dual][C] + N scales, then the dual coupling table.
int64_t dz_ws_floats(const FscIctdLayout& L, int64_t N, int C) {
  return N * (int64_t)max(L.KT, L.M) * C + N;
}

int64_t dual_ws_floats(const FscIctdLayout& L, int64_t N, int C) {
  int64_t kt = 0;
  for (int p = 0; p < L.NP; ++p) kt += L.g_d1[L.p_group[p]];
  return N * kt * C + N + cg_length(L);
}

template <int C>
int backward_c(const FscIctdLayout& L, int64_t N, const int32_t* dst_ptr, const int32_t* esrc,
               const int32_t* src_ptr, const int32_t* src_perm, const int32_t* edst, const float* G, const float* x,
               const float* Y, const float* gates, const float* cg, const float* Wt, float* dZ, float* Rw, float* dx,
               float* dgates, float* dY, const int32_t* node_order, hipStream_t st) {
  FscIctdLayout D;
  DualMap map;
  if (dual_layout(L, D, map) || check_layout(&D, C, "ictd dual layout")) {
    set_error("fsc_ictd_conv_backward: the layout has no valid dual (path table out of range)");
    return 1;
  }
  // gate and harmonic gradients: g = dZ / deg with dZ = W^T G (per path), then H, T per edge
  int dmax = 1;
  for (int p = 0; p < L.NP; ++p) dmax = max(dmax, L.p_d3[p]);
  {
    LaunchTimer tm("ictd_mix_grad", st);
    constexpr int RT = mix_rt<C>(), TPB = 2;
    const int64_t wtiles = (N * dmax + 16 * RT - 1) / (16 * RT);
    dim3 grid((unsigned)((wtiles + 4 * TPB - 1) / (4 * TPB)), (unsigned)L.NP);
    float* gscale = dZ + N * L.KT * C;
    row_scale_kernel<<<(unsigned)((N + 3) / 4), 256, 0, st>>>(N, L.M * C, G, gscale);
    mix_grad_kernel<C, RT, TPB><<<grid, 256, 0, st>>>(L, G, gscale,
                                                      reinterpret_cast<const _Float16*>(Wt + (int64_t)L.NREF * C * C),
                                                      Wt + mix_weight_floats(L.NREF, C) - MIXW_TAIL, dZ, N);
  }
  if (check_launch("ictd mix_bwd")) return 2;
  {
    // x split into fp16 planes with a power of two per node, in the dual workspace (free until the dual
    // projection: N D.KT C + N floats hold the N M C halves of each plane and the N scales, D.KT >= M)
    _Float16* xhi = reinterpret_cast<_Float16*>(Rw);
    _Float16* xlo = xhi + N * L.M * C;
    float* xinv = Rw + N * L.M * C;
    split_rows_h16_kernel<<<(unsigned)((N + 3) / 4), 256, 0, st>>>(N, L.M * C, x, xhi, xlo, xinv);
    LaunchTimer tm("ictd_project_grad", st);
    const int ncg = cg_length(L);
    const size_t lds = (size_t)grad_smem(L, ncg).total * sizeof(float);
    project_grad_h16_kernel<C><<<persist_grid(N, (const void*)project_grad_h16_kernel<C>, lds), 256, lds, st>>>(
        L, ncg, dZ, xhi, xlo, xinv, Y, gates, cg, dst_ptr, esrc, dgates, dY, N, node_order);
  }
  if (check_launch("ictd project_grad")) return 2;
  // input gradient: dual projection over the source grouping, then the mix with W^T
  float* cgd = Rw + N * D.KT * C + N;
  transpose_cg_kernel<<<(unsigned)D.NP, 256, 0, st>>>(L, D, map, cg, cgd);
  if (check_launch("ictd transpose_cg")) return 2;
  return project_mix_c<C, true>(D, N, src_ptr, edst, src_perm, dst_ptr, G, dZ, Y, gates, cgd,
                          reinterpret_cast<const _Float16*>(Wt + (int64_t)L.NREF * C * C),
                          Wt + mix_weight_floats(L.NREF, C) - MIXW_TAIL, Rw, dx, node_order, "ictd_dual_project",
                          "ictd_dual_mix", st);
}

}  // namespace ictd
}  // namespace fsc

using namespace fsc;
using namespace fsc::ictd;

extern "C" {

int fsc_ictd_conv_forward(const FscIctdLayout* layout, int64_t n_nodes, int64_t n_edges, int32_t channels,
                          const int32_t* dst_ptr, const int32_t* edge_src, const float* x, const float* Y,
                          const float* gates, const float* cg, const float* W, float* z_ws, float* out,
                          const int32_t* node_order, hipStream_t stream) {
  if (check_layout(layout, channels, "fsc_ictd_conv_forward")) return 1;
  FSC_CHECK_ARG(n_nodes >= 0 && n_edges >= 0 && n_nodes < (1LL << 24) && n_edges < (1LL << 31),
                "fsc_ictd_conv_forward: bad size");
  FSC_CHECK_ARG(dst_ptr && x && cg && W && z_ws && out, "fsc_ictd_conv_forward: null pointer");
  FSC_CHECK_ARG(n_edges == 0 || (edge_src && Y && gates), "fsc_ictd_conv_forward: null edge pointer");
  if (n_nodes == 0) return 0;
  const FscIctdLayout& L = *layout;
  if (channels == 128) return forward_c<128>(L, n_nodes, dst_ptr, edge_src, x, Y, gates, cg, W, z_ws, out, node_order, stream);
  if (channels == 64) return forward_c<64>(L, n_nodes, dst_ptr, edge_src, x, Y, gates, cg, W, z_ws, out, node_order, stream);
  return forward_c<32>(L, n_nodes, dst_ptr, edge_src, x, Y, gates, cg, W, z_ws, out, node_order, stream);
}

int fsc_ictd_project(const FscIctdLayout* layout, int64_t n_nodes, int64_t n_edges, int32_t channels,
                     const int32_t* dst_ptr, const int32_t* edge_src, const float* x, const float* Y,
                     const float* gates, const float* cg, float* z_ws, const int32_t* node_order,
                     hipStream_t stream) {
  if (check_layout(layout, channels, "fsc_ictd_project")) return 1;
  FSC_CHECK_ARG(n_nodes >= 0 && n_edges >= 0 && n_nodes < (1LL << 24) && n_edges < (1LL << 31),
                "fsc_ictd_project: bad size");
  FSC_CHECK_ARG(dst_ptr && x && cg && z_ws, "fsc_ictd_project: null pointer");
  FSC_CHECK_ARG(n_edges == 0 || (edge_src && Y && gates), "fsc_ictd_project: null edge pointer");
  if (n_nodes == 0) return 0;
  const FscIctdLayout& L = *layout;
  if (channels == 128) return project_only_c<128>(L, n_nodes, dst_ptr, edge_src, x, Y, gates, cg, z_ws, node_order, stream);
  if (channels == 64) return project_only_c<64>(L, n_nodes, dst_ptr, edge_src, x, Y, gates, cg, z_ws, node_order, stream);
  return project_only_c<32>(L, n_nodes, dst_ptr, edge_src, x, Y, gates, cg, z_ws, node_order, stream);
}

int fsc_ictd_prepare_weights(const float* W, int32_t n_ref, int32_t channels, float* Wt, hipStream_t stream) {
  FSC_CHECK_ARG(W && Wt && n_ref > 0 && channels > 0, "fsc_ictd_prepare_weights: bad argument");
  mix_absmax_kernel<<<256, 256, 0, stream>>>(W, (int64_t)n_ref * channels * channels,
                                             Wt + mix_weight_floats(n_ref, channels) - MIXW_TAIL + 256);
  if (check_launch("ictd weight maximum")) return 2;
  prepare_mix_kernel<<<256, 256, 0, stream>>>(W, Wt, n_ref, channels);
  return check_launch("ictd prepare_weights") ? 2 : 0;
}

int fsc_ictd_forward_workspace(const FscIctdLayout* layout, int64_t n_nodes, int32_t channels, int64_t* z_floats) {
  if (check_layout(layout, channels, "fsc_ictd_forward_workspace")) return 1;
  FSC_CHECK_ARG(z_floats && n_nodes >= 0, "fsc_ictd_forward_workspace: bad argument");
  *z_floats = fwd_ws_floats(*layout, n_nodes, channels);
  return 0;
}

int fsc_ictd_backward_workspace(const FscIctdLayout* layout, int64_t n_nodes, int32_t channels, int64_t* dz_floats,
                                int64_t* r_floats) {
  if (check_layout(layout, channels, "fsc_ictd_backward_workspace")) return 1;
  FSC_CHECK_ARG(dz_floats && r_floats && n_nodes >= 0, "fsc_ictd_backward_workspace: bad argument");
  *dz_floats = dz_ws_floats(*layout, n_nodes, channels);
  *r_floats = dual_ws_floats(*layout, n_nodes, channels);
  return 0;
}

int fsc_ictd_conv_backward(const FscIctdLayout* layout, int64_t n_nodes, int64_t n_edges, int32_t channels,
                           const int32_t* dst_ptr, const int32_t* edge_src, const int32_t* src_ptr,
                           const int32_t* src_perm, const int32_t* edge_dst, const float* grad_out, const float* x,
                           const float* Y, const float* gates, const float* cg, const float* Wt, float* dz_ws,
                           float* r_ws, float* grad_x, float* grad_gates, float* grad_Y, const int32_t* node_order,
                           hipStream_t stream) {
  if (check_layout(layout, channels, "fsc_ictd_conv_backward")) return 1;
  FSC_CHECK_ARG(n_nodes >= 0 && n_edges >= 0 && n_nodes < (1LL << 24) && n_edges < (1LL << 31),
                "fsc_ictd_conv_backward: bad size");
  FSC_CHECK_ARG(dst_ptr && src_ptr && grad_out && x && cg && Wt && dz_ws && r_ws && grad_x,
                "fsc_ictd_conv_backward: null pointer");
  FSC_CHECK_ARG(n_edges == 0 || (edge_src && src_perm && edge_dst && Y && gates && grad_gates && grad_Y),
                "fsc_ictd_conv_backward: null edge pointer");
  if (n_nodes == 0) return 0;
  const FscIctdLayout& L = *layout;
  if (channels == 128)
    return backward_c<128>(L, n_nodes, dst_ptr, edge_src, src_ptr, src_perm, edge_dst, grad_out, x, Y, gates, cg, Wt,
                           dz_ws, r_ws, grad_x, grad_gates, grad_Y, node_order, stream);
  if (channels == 64)
    return backward_c<64>(L, n_nodes, dst_ptr, edge_src, src_ptr, src_perm, edge_dst, grad_out, x, Y, gates, cg, Wt,
                          dz_ws, r_ws, grad_x, grad_gates, grad_Y, node_order, stream);
  return backward_c<32>(L, n_nodes, dst_ptr, edge_src, src_ptr, src_perm, edge_dst, grad_out, x, Y, gates, cg, Wt,
                        dz_ws, r_ws, grad_x, grad_gates, grad_Y, node_order, stream);
}

int fsc_ictd_conv1_forward(const FscIctdLayout* layout, int64_t n_nodes, int64_t n_edges, int32_t channels,
                           int32_t n_species, const int32_t* dst_ptr, const int32_t* edge_pair,
                           const int32_t* node_species, const float* F, const float* gates, const float* qtab,
                           float* out, hipStream_t stream) {
  if (check_layout(layout, channels, "fsc_ictd_conv1_forward")) return 1;
  FSC_CHECK_ARG(n_nodes >= 0 && n_edges >= 0 && n_nodes < (1LL << 31) && n_edges < (1LL << 31),
                "fsc_ictd_conv1_forward: bad size");
  FSC_CHECK_ARG(n_species >= 1 && n_species <= 16, "fsc_ictd_conv1_forward: 1..16 species supported");
  FSC_CHECK_ARG(dst_ptr && node_species && qtab && out, "fsc_ictd_conv1_forward: null pointer");
  FSC_CHECK_ARG(n_edges == 0 || (edge_pair && F && gates), "fsc_ictd_conv1_forward: null edge pointer");
  FSC_CHECK_ARG(layout->NY == 1 || layout->NY == 4 || layout->NY == 9 || layout->NY == 16,
                "fsc_ictd_conv1_forward: lmax must be 0, 1, 2 or 3");
  if (n_nodes == 0) return 0;
  const FscIctdLayout& L = *layout;
  LaunchTimer tm("ictd_conv1", stream);
  const unsigned grid = (unsigned)n_nodes;
#define FSC_C1F(CC, NYY) \
  conv1_fwd_kernel<CC, NYY><<<grid, 256, 0, stream>>>(L, n_species, dst_ptr, edge_pair, node_species, F, gates, qtab, out)
#define FSC_C1F_NY(NYY) \
  if (channels == 128) FSC_C1F(128, NYY); else if (channels == 64) FSC_C1F(64, NYY); else FSC_C1F(32, NYY)
  if (L.NY == 1) {
    FSC_C1F_NY(1);
  } else if (L.NY == 4) {
    FSC_C1F_NY(4);
  } else if (L.NY == 9) {
    FSC_C1F_NY(9);
  } else {
    FSC_C1F_NY(16);
  }
#undef FSC_C1F_NY
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
  FSC_CHECK_ARG(n_species >= 1 && n_species <= 16, "fsc_ictd_conv1_backward: 1..16 species supported");
  FSC_CHECK_ARG(dst_ptr && node_species && grad_out && qtab, "fsc_ictd_conv1_backward: null pointer");
  FSC_CHECK_ARG(n_edges == 0 || (edge_pair && F && gates && grad_F && grad_gates),
                "fsc_ictd_conv1_backward: null edge pointer");
  FSC_CHECK_ARG(layout->NY == 1 || layout->NY == 4 || layout->NY == 9 || layout->NY == 16,
                "fsc_ictd_conv1_backward: lmax must be 0, 1, 2 or 3");
  if (n_nodes == 0) return 0;
  const FscIctdLayout& L = *layout;
  LaunchTimer tm("ictd_conv1_grad", stream);
  const unsigned grid = (unsigned)n_nodes;
#define FSC_C1B(CC, NYY) conv1_bwd_kernel<CC, NYY><<<grid, 256, 0, stream>>>(L, n_species, dst_ptr, edge_pair, \
      node_species, grad_out, F, gates, qtab, grad_F, grad_gates)
#define FSC_C1B_NY(NYY) \
  if (channels == 128) FSC_C1B(128, NYY); else if (channels == 64) FSC_C1B(64, NYY); else FSC_C1B(32, NYY)
  if (L.NY == 1) {
    FSC_C1B_NY(1);
  } else if (L.NY == 4) {
    FSC_C1B_NY(4);
  } else if (L.NY == 9) {
    FSC_C1B_NY(9);
  } else {
    FSC_C1B_NY(16);
  }
#undef FSC_C1B_NY
#undef FSC_C1B
  return check_launch("ictd conv1_bwd") ? 2 : 0;
}

}  // extern "C"
