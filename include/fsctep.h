/*
 * fsctep.h - C ABI of the MI355X (gfx950) kernels for the FSCTEP equivariant
 * message-passing hot path.  Library: libfsctep_hip.so.
 *
 * Conventions
 *  - Every pointer is device memory (fp32 data, int32 graph indices) unless noted.
 *  - Outputs and workspaces are allocated by the caller; no entry point allocates.
 *  - Work is enqueued on `stream`; no entry point synchronises the host.
 *  - Return value: 0 ok, 1 invalid argument, 2 launch failure; the message of the
 *    last failure on the calling thread is returned by fsc_last_error().
 *  - Graph: edges are sorted by receiver (dst).  dst_ptr[N+1] is the receiver CSR;
 *    src_ptr[N+1] / src_perm[E] list, for every source node, the receiver-sorted ids
 *    of its out-edges (a stable sort of the receiver-sorted list by source).
 *  - Node features use a component-major layout x[N][13][C] for ranks 0..2
 *    (component 0: rank 0; 1..3: rank-1 index i; 4..12: rank-2 index 3i+j).  The
 *    reference's flat layout (models/pure_cartesian.py:69-120) is the channel-major
 *    [C][3^L] blocks of the true half followed by an all-zero pseudo half.
 */
#ifndef FSCTEP_H
#define FSCTEP_H

#include <stdint.h>
#include <hip/hip_runtime_api.h>

#ifdef __cplusplus
extern "C" {
#endif

/* Message of the last failed call on this thread ("" if none). */
const char* fsc_last_error(void);
/* ABI revision of this header (2: node_order arguments of the conv entry points). */
int fsc_abi_version(void);

/* Measurement (no counterpart in the reference): while active, every launch of the named
 * kernel ("node_expand", "edge_message", "receiver_sum", "direction_grad",
 * "edge_message_grad", "node_expand_grad") is bracketed by HIP events on its stream.
 * fsc_timing_end synchronises those events and returns the summed duration. */
int fsc_timing_begin(const char* kernel_name);
int fsc_timing_end(double* total_ms, int64_t* launches);

/* ------------------------------------------------------------------ graph preparation
 * Replaces the per-call receiver sort of the trunks, `sort_idx = argsort(edge_dst)` and the permutation
 * of edge_src / edge_dst / edge_shifts (models/pure_cartesian_sparse_layers.py:745-748,
 * models/pure_cartesian_ictd_layers_full.py:896-899, models/pure_cartesian_ictd_layers_o3.py:924-927), plus
 * the index structures the kernels read.  The order is the stable one (ties keep the input order), so
 * results are deterministic; the reference's unstable argsort differs only in the summation order.
 * Every output size depends on (n_nodes, n_edges, n_species) only and nothing synchronises the host.
 *
 * fsc_graph_sizes: n_tiles_max = ceil(E/16) + n_species^2 (0 without species) and the int32 workspace. */
int fsc_graph_sizes(int64_t n_nodes, int64_t n_edges, int32_t n_species, int64_t* n_tiles_max,
                    int64_t* workspace_ints);

/* Inputs: edge_src, edge_dst [E] int64 node ids; species [N] int64 atomic numbers (< n_species, the
 * size of the model's species table, <= 16; null with n_species 0).  Outputs (int32):
 * order [E] (receiver-sorted position -> input edge id), src32 / dst32 [E] (the permuted ids),
 * dst_ptr [N+1] (receiver CSR), src_ptr [N+1] + src_perm [E] (receiver-sorted ids grouped by source,
 * ascending within a source), node_species [N], edge_pair [E] = species[src]*n_species + species[dst],
 * pair_tiles [17*n_tiles_max] (the receiver-sorted ids grouped by species pair, ascending within a pair,
 * each pair padded with -1 to a multiple of 16, then one pair id per tile; unused trailing tiles are
 * all -1 with pair 0), and
 * status [1]: bit 0 set if an edge id is outside [0, N), bit 1 if a species is outside [0, n_species);
 * such ids are clamped (every access stays in bounds) and the results are meaningless.
 * workspace: fsc_graph_sizes' workspace_ints. */
int fsc_graph_prepare(int64_t n_nodes, int64_t n_edges, int32_t n_species, const int64_t* edge_src,
                      const int64_t* edge_dst, const int64_t* species, int32_t* order, int32_t* src32,
                      int32_t* dst32, int32_t* dst_ptr, int32_t* src_ptr, int32_t* src_perm,
                      int32_t* node_species, int32_t* edge_pair, int32_t* pair_tiles, int32_t* status,
                      int32_t* workspace, hipStream_t stream);

/* fsc_graph_prepare without the workspace argument: allocates nothing.  No counterpart in the reference;
 * it is for callers that cannot allocate (code under HIP graph capture, per-step MD loops, harnesses
 * that forbid hipMalloc).  Its workspace is a static device array of 2^23 int32 (32 MiB) on each GPU the
 * library runs on, held until the process ends; graphs whose fsc_graph_sizes workspace exceeds it
 * (about 4N + E + n_species^2 (2 + E/2048) ints) are rejected with status 1.  Every call on one GPU
 * shares that array (the counters are cleared at the start of each call), so calls that overlap on one GPU, on
 * different streams or threads, race.  The stream must belong to the current device.  Outputs as for
 * fsc_graph_prepare, bit for bit. */
int fsc_graph_prepare_noalloc(int64_t n_nodes, int64_t n_edges, int32_t n_species, const int64_t* edge_src,
                              const int64_t* edge_dst, const int64_t* species, int32_t* order, int32_t* src32,
                              int32_t* dst32, int32_t* dst_ptr, int32_t* src_ptr, int32_t* src_perm,
                              int32_t* node_species, int32_t* edge_pair, int32_t* pair_tiles, int32_t* status,
                              hipStream_t stream);

/* Spatial order of the nodes: a permutation `order` [N] (int32) along a Morton curve over the bounding
 * box of pos [N][3], atoms of one grid cell in ascending id.  No counterpart in the reference (whose
 * kernels run one thread per output); passed as `node_order` to the conv entry points, whose per-node
 * kernels then give each XCD a contiguous, spatially compact run of nodes, so that the neighbour-row
 * gathers of its concurrently running blocks hit its L2.  Deterministic; workspace of
 * fsc_spatial_order_workspace int32. */
int fsc_spatial_order_workspace(int64_t n_nodes, int64_t* workspace_ints);
int fsc_spatial_order(int64_t n_nodes, const float* pos, int32_t* order, int32_t* workspace, hipStream_t stream);

/* ------------------------------------------------------------------ neighbour list
 * Replaces radius_graph_pbc_gpu (molecular_force_field/utils/graph_utils.py:192-257; one torch_cluster
 * radius call per periodic image) and the LAMMPS-list-to-edge loop of pair_mff_torch.cpp:597-641.
 * Edges: every (src i, dst j, s) with s_k in {-1,0,1} on axes with pbc[k] != 0 (0 otherwise), not (i == j,
 * s == 0), and |(pos_j - pos_i) + s.cell|^2 < cutoff^2 in double precision (cell rows = lattice vectors);
 * receiver-sorted, then ascending in (src, s).  Unlike torch_cluster's max_num_neighbors there is no cap.
 * pos [N][3] and cell [3][3] are device doubles; pbc is a host array of 3 int32.
 * Two calls: fsc_neighbor_count fills the receiver CSR dst_ptr [N+1] (the caller reads E = dst_ptr[N]),
 * then fsc_neighbor_fill, with the same workspace (fsc_neighbor_workspace int32, left untouched in
 * between) and fill_ws of 3E int32 (8-byte aligned), writes edge_src, edge_dst [E] and edge_shifts [E][3]. */
int fsc_neighbor_workspace(int64_t n_nodes, int64_t* workspace_ints);
int fsc_neighbor_count(int64_t n_nodes, const double* pos, const double* cell, const int32_t* pbc, double cutoff,
                       int32_t* dst_ptr, int32_t* workspace, hipStream_t stream);
int fsc_neighbor_fill(int64_t n_nodes, int64_t n_edges, const double* pos, const double* cell, const int32_t* pbc,
                      double cutoff, const int32_t* dst_ptr, int32_t* workspace, int32_t* fill_ws, int64_t* edge_src,
                      int64_t* edge_dst, double* edge_shifts, hipStream_t stream);

/* ------------------------------------------------------------------ pure-cartesian-sparse
 * conv2..n.  Replaces, per interaction layer, the chain
 *   weights = fc(emb) ; tp(f_in[edge_src], e_flat, weights) ; scatter(., edge_dst) / (E/N)
 * of PureCartesianSparseE3Conv2.forward (models/pure_cartesian_sparse_layers.py:382-421),
 * i.e. the last radial-MLP Linear (fc.4), PureCartesianTensorProductO3Sparse.forward
 * (models/pure_cartesian.py:790-863) and utils/scatter.py:63-116.
 * Supported: lmax 2, max_rank_other 1, k_policy "k0", channels 32, 64 or 128.
 */

/* Workspace sizes, in floats: s (node expansion, also the size of ds) and p (edge messages). */
int fsc_sparse_conv_workspace(int64_t n_nodes, int64_t n_edges, int32_t channels,
                              int64_t* s_floats, int64_t* p_floats);

/* Re-layout fc.4.weight (6*C*C, 64) and fc.4.bias (6*C*C) into the two kernel operands bk1 and
 * bk6 (the operand and its transpose, times a power of two and split into two fp16 parts of
 * 6*65*C*C values, for fp32-accurate split-fp16 products, then a 512-float tail holding the scale, then
 * the same scaled values rounded to bf16 for the bf16 variant; 6*65*C*C + 512 + 3*65*C*C floats of storage
 * each).  Both are opaque to the caller.  Call again whenever those parameters change. */
int fsc_sparse_conv_prepare_weights(const float* w_last, const float* b_last, int32_t channels,
                                    float* bk1, float* bk6, hipStream_t stream);

/* out[N][13][C] = inv_norm * sum_{e->n} message_e.
 * x: [N][13][C] input features; h: [E][64] radial hidden (output of fc.3, the second SiLU);
 * n: [E][3] unit edge directions (edge_rank_powers, models/pure_cartesian.py:292-317);
 * inv_norm: 1/max(E/N, 1e-8) as in pure_cartesian_sparse_layers.py:418-420.
 * s_ws, p_ws: workspaces from fsc_sparse_conv_workspace; keep them for the backward.
 * precision 0: every product fp32-accurate (split-fp16 node expansion, split-bf16 edge message);
 * precision 1: the bf16 channel-mix variant, one bf16 MFMA per product in the node expansion, the edge
 * message and (backward) the node-expansion gradient, fp32 accumulation.  No counterpart in the reference
 * (an MI355X option for large systems; the reference computes in the model dtype).
 * node_order: null, or a permutation of the nodes (fsc_spatial_order) that the per-node kernels walk
 * (a performance hint: the results do not depend on it). */
int fsc_sparse_conv_forward(int64_t n_nodes, int64_t n_edges, int32_t channels,
                            const int32_t* dst_ptr, const int32_t* src_ptr, const int32_t* src_perm,
                            const float* x, const float* h, const float* n, const float* bk1,
                            float inv_norm, float* s_ws, float* p_ws, float* out, int32_t precision,
                            const int32_t* node_order, hipStream_t stream);

/* Backward of fsc_sparse_conv_forward for forces: grad_x [N][13][C], grad_h [E][64],
 * grad_n [E][3] from grad_out [N][13][C].  ds_ws: scratch of s_floats floats.
 * edge_dst: [E] receiver of each receiver-sorted edge; precision and node_order as for the forward. */
int fsc_sparse_conv_backward(int64_t n_nodes, int64_t n_edges, int32_t channels,
                             const int32_t* dst_ptr, const int32_t* src_ptr, const int32_t* src_perm,
                             const int32_t* edge_dst, const float* grad_out, const float* h,
                             const float* n, const float* bk6, const float* s_ws, const float* p_ws,
                             float inv_norm, float* ds_ws, float* grad_x, float* grad_h,
                             float* grad_n, int32_t precision, const int32_t* node_order, hipStream_t stream);

/* Training double backward (no inference use).  The receiver assembly is quadratic in the edge directions,
 * m1 = P1 n + P3, m2 = P2 n n^T + P4 n^T + P5; fsc_sparse_conv_direction writes its derivative along the
 * directions u [E][3] from the forward's messages p_ws: out'[N][13][C] = inv_norm sum_{e->n}
 * (0, P1 u, P2 (u n^T + n u^T) + P4 u^T).  fsc_sparse_conv_direction_backward gives the gradients of
 * <grad_out, out'>: grad_x, grad_h and ds_ws (dS in its first N*18*65*C floats, for the weight gradient) as the
 * backward above does for the message gradient dP' = D_n dP [u], and grad_n = sum_c P2 (g2 + g2^T) u (the
 * second-derivative term).  They have no counterpart in the reference's sparse path, which trains through
 * PyTorch autograd (pure_cartesian_sparse_layers.py:382-421); the reference's double-backward kernels serve
 * its ICTD tensor product (csrc/ictd_tp_cuda.cu:536-971). */
int fsc_sparse_conv_direction(int64_t n_nodes, int64_t n_edges, int32_t channels, const int32_t* dst_ptr,
                              const float* p_ws, const float* n, const float* u, float inv_norm, float* out,
                              hipStream_t stream);
int fsc_sparse_conv_direction_backward(int64_t n_nodes, int64_t n_edges, int32_t channels,
                                       const int32_t* dst_ptr, const int32_t* src_ptr, const int32_t* src_perm,
                                       const int32_t* edge_dst, const float* grad_out, const float* h,
                                       const float* n, const float* u, const float* bk6, const float* s_ws,
                                       const float* p_ws, float inv_norm, float* ds_ws, float* grad_x,
                                       float* grad_h, float* grad_n, int32_t precision, const int32_t* node_order,
                                       hipStream_t stream);

/* ------------------------------------------------------------------ conv1 (sparse)
 * Replaces the TP + scatter + in-degree normalisation of PureCartesianSparseE3Conv.forward
 * (models/pure_cartesian_sparse_layers.py:227-330) without external tensors or fidelity
 * embeddings, where both TP operands are functions of the species only.
 *
 * Pair table from fc.4 (6*C*64, 64)/(6*C*64) and the per-species atom features
 * atom_table [n_species][8] (= atom_mlp(atom_embedding(Z)), :258-259):
 * mf [n_species^2][3][65][C] and mb [n_species^2][3][C][68] (k' = 0..64, rows zero-padded);
 * pair = s_src*n_species + s_dst. */
int fsc_sparse_conv1_pair_table(const float* w_last, const float* b_last, const float* atom_table,
                                int32_t n_species, int32_t channels, float* mf, float* mb,
                                hipStream_t stream);

/* out[N][13][C] = (1/max(indeg,1)) sum_{e->n} message_e; q_ws: [E][3][C] kept for backward.
 * pair_tiles: [16*n_tiles edge ids | n_tiles pair ids], the receiver-sorted edge ids grouped by
 * species pair, each pair's list padded with -1 to a multiple of 16 (fsc_graph_prepare); tiles whose
 * first id is -1 are skipped. */
int fsc_sparse_conv1_forward(int64_t n_nodes, int64_t n_edges, int32_t channels, const int32_t* dst_ptr,
                             int64_t n_tiles, const int32_t* pair_tiles, const float* h, const float* n,
                             const float* mf, const float* mb, float* q_ws, float* out, hipStream_t stream);

/* grad_h [E][64], grad_n [E][3] from grad_out [N][13][C]; dq_ws: scratch of E*3*C floats. */
int fsc_sparse_conv1_backward(int64_t n_nodes, int64_t n_edges, int32_t channels, const int32_t* dst_ptr,
                              int64_t n_tiles, const int32_t* pair_tiles, const float* grad_out, const float* n,
                              const float* mf, const float* q_ws, float* dq_ws, float* grad_h, float* grad_n,
                              hipStream_t stream);

/* ------------------------------------------------------------------ edge geometry and radial MLP
 * Replaces the edge geometry of the trunks (models/pure_cartesian_sparse_layers.py:745-756,
 * models/pure_cartesian_ictd_layers_full.py:896-909, models/pure_cartesian_ictd_layers_o3.py:924-936):
 * vec = pos[dst] - pos[src] + shift (shift = edge_shifts @ cell), r = |vec|, n = vec/max(r, 1e-8),
 * with edges in receiver order.  The backward writes grad_pos [N][3] = dE/dpos from grad_n
 * [E][3] and grad_r [E] (either may be null) by segmented sums over the receiver CSR and the
 * source grouping (src_ptr, src_perm); no atomics. */
int fsc_edge_geometry_forward(int64_t n_edges, const float* pos, const float* shift, const int32_t* edge_src,
                              const int32_t* edge_dst, float* n_out, float* r_out, hipStream_t stream);
int fsc_edge_geometry_backward(int64_t n_nodes, int64_t n_edges, const float* grad_n, const float* grad_r,
                               const float* n, const float* r, const int32_t* dst_ptr, const int32_t* src_ptr,
                               const int32_t* src_perm, float* grad_pos, hipStream_t stream);

/* The same geometry from caller-supplied edge vectors, the `precomputed_edge_vec` branch of the ICTD trunks
 * (models/pure_cartesian_ictd_layers_full.py:901-902, models/pure_cartesian_ictd_layers_o3.py:928-929)
 * that the LAMMPS / ML-IAP cores differentiate through (interfaces/lammps_mliap.py:404).  edge_vec [E][3]
 * is in the caller's edge order and read through `order` (fsc_graph_prepare); n_out, r_out are
 * receiver-sorted.  The backward writes grad_vec [E][3] in the caller's order. */
int fsc_edge_vec_geometry_forward(int64_t n_edges, const float* edge_vec, const int32_t* order, float* n_out,
                                  float* r_out, hipStream_t stream);
int fsc_edge_vec_geometry_backward(int64_t n_edges, const float* grad_n, const float* grad_r, const float* n,
                                   const float* r, const int32_t* order, float* grad_vec, hipStream_t stream);

/* Radial basis + a radial MLP (fc = Linear(nb,64), SiLU, Linear(64,64), SiLU, Linear(64,P);
 * models/pure_cartesian_sparse_layers.py:204-210,319-321,372-378,410-412,
 * models/pure_cartesian_ictd_layers_full.py:277-283,464-465,693-699,930-937):
 * h = silu(w2 silu(w0 emb(r) + b0) + b2), emb = soft_one_hot_linspace(r, 0, r_cut, n_basis, basis,
 * cutoff=True) * sqrt(n_basis); basis 0 = bessel, 1 = gaussian, 2 = fourier, 3 = cosine,
 * 4 = smooth_finite; weights in torch Linear layout
 * (w0 [64][n_basis], w2 [64][64]).  With w4 == NULL the output is h [E][64] (the sparse trunk's
 * fc[:4]); with w4 [n_out][64], b4 [n_out] (n_out <= 64) it is w4 h + b4 [E][n_out] (the ICTD gates,
 * the whole fc).  The backward gives grad_r [E] from grad_out (activations recomputed). */
int fsc_radial_mlp_forward(int64_t n_edges, const float* r, const float* w0, const float* b0, const float* w2,
                           const float* b2, const float* w4, const float* b4, int32_t n_out, int32_t n_basis,
                           float r_cut, int32_t basis, float* out, hipStream_t stream);
int fsc_radial_mlp_backward(int64_t n_edges, const float* r, const float* w0, const float* b0, const float* w2,
                            const float* b2, const float* w4, int32_t n_out, int32_t n_basis, float r_cut,
                            int32_t basis, const float* grad_out, float* grad_r, hipStream_t stream);

/* Direction harmonics of the ICTD trunks (direction_harmonics_fast/_all, models/ictd_irreps.py:371-402,
 * 489-494): Y [E][(lmax+1)^2], block l at offset l^2, Y_l(n) = sum_k coef[k][.] n_x^a n_y^b n_z^c over the
 * degree-l monomials k (coef = multinomial * G_l B_l of the harmonic basis, built on the host by
 * fsctep_amd/ictd_basis.py).  lmax <= 3.  The backward gives grad_n [E][3] from grad_Y. */
typedef struct FscHarmTable {
  int32_t lmax, nmono;
  int32_t mono_l[20];
  int32_t mono_exp[20][3];
  float coef[20][7];
} FscHarmTable;
int fsc_edge_harmonics_forward(const FscHarmTable* table, int64_t n_edges, const float* n, float* Y,
                               hipStream_t stream);
int fsc_edge_harmonics_backward(const FscHarmTable* table, int64_t n_edges, const float* n, const float* grad_Y,
                                float* grad_n, hipStream_t stream);

/* ------------------------------------------------------------------ ICTD (pure-cartesian-ictd / -o3)
 * Irreps are keys (l, parity) in a fixed order; node features are x[N][M][C] with M = sum(2l+1)
 * components (component-major), edge harmonics Y[E][(lmax+1)^2] (block l at offset l^2).
 * A layout table describes the live tensor-product paths (second operand a geometric Y_l) grouped
 * by first-operand key; it is built on the host (fsctep_amd/ictd_basis.py) from the active irreps.
 */
typedef struct FscIctdLayout {
  int32_t M, NY, KT, NP, NG, NREF, NBGP, KTT;         /* comps, Y comps, sum d3, live paths, groups,
                                                         reference paths, padded per-edge table, kk tiles */
  int32_t g_o1[8], g_d1[8], g_kstart[8], g_kcount[8], g_kpad[8], g_bgoff[8], g_tile0[8];
  int32_t tile_group[16];
  int32_t p_gate[64], p_oy[64], p_d2[64], p_d3[64], p_koff[64], p_cgoff[64], p_group[64], p_oo[64];
  int32_t kk_path[128];                                /* live path of each output slot kk < KT */
  int32_t NK, k_oo[16], k_d[16];                       /* output keys: component offset, 2l+1 */
  int32_t NP1, y_path1[16], y_oo1[16], c1_gate[16];    /* conv1: per Y component, live path (-1: none) */
} FscIctdLayout;

/* conv2..n.  Replaces the chain gates = fc2(emb); tp2(x1[edge_src], Y, gates); scatter / indeg of
 * models/pure_cartesian_ictd_layers_full.py:938-954 (O3: pure_cartesian_ictd_layers_o3.py:956-973),
 * i.e. HarmonicFullyConnectedTensorProduct[O3].forward (models/ictd_irreps.py:971-1253, :1512-1695)
 * and the project/mix ops of the reference extension (csrc/ictd_tp.cpp:140-494).
 * gates [E][NREF]; Wp: fsc_ictd_prepare_weights of tp2.weight; cg: concatenated normalised C[m1][m2][m3]
 * of the live paths; z_ws scratch of fsc_ictd_forward_workspace floats; out [N][M][C].  node_order: null
 * or a permutation of the nodes (fsc_spatial_order) for the per-receiver kernels (a performance hint).
 * n_nodes < 2^24 here, in fsc_ictd_project and in fsc_ictd_conv_backward. */
int fsc_ictd_forward_workspace(const FscIctdLayout* layout, int64_t n_nodes, int32_t channels, int64_t* z_floats);
int fsc_ictd_conv_forward(const FscIctdLayout* layout, int64_t n_nodes, int64_t n_edges, int32_t channels,
                          const int32_t* dst_ptr, const int32_t* edge_src, const float* x, const float* Y,
                          const float* gates, const float* cg, const float* Wp, float* z_ws, float* out,
                          const int32_t* node_order, hipStream_t stream);

/* The receiver-normalised projection of the forward alone, Z[n][kk][i] = (1/indeg n) sum_{e->n} sum_m1
 * BG_e[m1][kk] x_src[o1+m1][i] (kk = (path, m3), KT slots), into z_ws[0 .. N*KT*C) (z_ws of
 * fsc_ictd_forward_workspace floats):
 * the operand of the weight gradient dW[gate_p][o][i] = sum_n sum_m3 G[n][oo_p+m3][o] Z[n][koff_p+m3][i]
 * used by training.  Replaces project_bucket_forward with the receiver scatter
 * (csrc/ictd_tp.cpp:140-176, models/ictd_irreps_cuda.py:314-336). */
int fsc_ictd_project(const FscIctdLayout* layout, int64_t n_nodes, int64_t n_edges, int32_t channels,
                     const int32_t* dst_ptr, const int32_t* edge_src, const float* x, const float* Y,
                     const float* gates, const float* cg, float* z_ws, const int32_t* node_order,
                     hipStream_t stream);

/* Prepare tp2.weight W [NREF][C][C] for the channel mix: Wp holds 2*NREF*C*C + 512 floats (W times a
 * power of two split into two fp16 planes, the same with the channel axes swapped, and the scale), opaque
 * to the caller.  Call again when W changes. */
int fsc_ictd_prepare_weights(const float* W, int32_t n_ref, int32_t channels, float* Wp, hipStream_t stream);

/* Backward for forces: grad_x [N][M][C], grad_gates [E][NREF] (caller zero-fills: entries of paths
 * without a geometric operand stay 0), grad_Y [E][NY].  Wp as for the forward; edge_dst [E] the receiver
 * of each receiver-sorted edge; dz_ws and r_ws scratch of fsc_ictd_backward_workspace floats; node_order as
 * for the forward.  grad_x is formed per source (the projection over the source grouping with every path
 * reversed, then the channel mix with W^T), so no per-edge gradient is stored. */
int fsc_ictd_backward_workspace(const FscIctdLayout* layout, int64_t n_nodes, int32_t channels, int64_t* dz_floats,
                                int64_t* r_floats);
int fsc_ictd_conv_backward(const FscIctdLayout* layout, int64_t n_nodes, int64_t n_edges, int32_t channels,
                           const int32_t* dst_ptr, const int32_t* edge_src, const int32_t* src_ptr,
                           const int32_t* src_perm, const int32_t* edge_dst, const float* grad_out, const float* x,
                           const float* Y, const float* gates, const float* cg, const float* Wp, float* dz_ws,
                           float* r_ws, float* grad_x, float* grad_gates, float* grad_Y,
                           const int32_t* node_order, hipStream_t stream);

/* conv1 (ICTDIrrepsE3Conv / ICTDO3E3Conv, pure_cartesian_ictd_layers_full.py:341-473,
 * pure_cartesian_ictd_layers_o3.py:424-532): both operands depend only on the species, and
 * C(l,0,l) is the identity, so out[n][comp(l)][o] = (1/indeg) sum_e gate[e][p_l] Q[pair][p_l][o] F[e][l^2+k]
 * with Q[pair][p][o] = sum_ij W1[p][o][i][j] A_src[i] A_dst[j] (qtab [NS*NS][NP1][C], pair = s_src*NS +
 * s_dst, n_species = NS <= 16, the rows of the species table; node_species [N] gives s_dst) and F = Y plus the embedded external field on
 * the l=1 block. */
int fsc_ictd_conv1_forward(const FscIctdLayout* layout, int64_t n_nodes, int64_t n_edges, int32_t channels,
                           int32_t n_species, const int32_t* dst_ptr, const int32_t* edge_pair,
                           const int32_t* node_species, const float* F, const float* gates, const float* qtab,
                           float* out, hipStream_t stream);

/* grad_F [E][NY], grad_gates [E][NREF] (caller zero-fills) from grad_out [N][M][C]. */
int fsc_ictd_conv1_backward(const FscIctdLayout* layout, int64_t n_nodes, int64_t n_edges, int32_t channels,
                            int32_t n_species, const int32_t* dst_ptr, const int32_t* edge_pair,
                            const int32_t* node_species, const float* grad_out, const float* F,
                            const float* gates, const float* qtab, float* grad_F, float* grad_gates,
                            hipStream_t stream);

/* ------------------------------------------------------------------ per-edge (bucketed) ICTD TP
 * The operations of the reference's native extension molecular_force_field._C_ictd_tp
 * (csrc/ictd_tp.cpp:498-522; einsum semantics models/ictd_irreps_cuda.py:169-288), for the arguments its
 * CUDA path takes: fp32 and fp64 (csrc/ictd_tp_cuda.cu:1230-1236 dispatches both), mul_in2 == 1.  The
 * functions below take float arrays; each has an fp64 twin of the same name with the suffix _f64 and
 * double arrays (declared after them).  B batch (edges), I = mul_in1, O = mul_out, K = kdim, P paths.
 *   project:  y[b][p][k][i] = sum_{m,n} a[b][i][m] v[b][n] u[m*m2+n][p*K+k]
 *   mix:      out[b][o][k]  = sum_p gates[b][p] sum_i y[b][p][k][i] w[p][o][i]
 * Layouts: a [B][I][m1], v [B][1][m2], u [m1*m2][P*K], y [B][P][K][I], w [P][O][I], gates [B][P],
 * out [B][O][K].  accumulate != 0 adds to the output instead of overwriting it (the double-backward
 * sums).  Limits: m1, m2 <= 9, P*K <= 64 (projection; the U gradient also m1*m2*P*K <= 2048);
 * I, O multiples of 4 and K <= 128 (mix).  The U and W gradients sum over the batch through the
 * caller's workspace in a fixed order (deterministic). */
/* project_bucket_forward (csrc/ictd_tp.cpp:140-176): y from a, v, u. */
int fsc_bucket_project(int64_t B, int32_t I, int32_t m1, int32_t m2, int32_t P, int32_t K, const float* a,
                       const float* v, const float* u, float* y, int32_t accumulate, hipStream_t stream);
/* project_bucket_transpose_a (csrc/ictd_tp.cpp:178-208): grad_a [B][I][m1] from grad_y, v, u. */
int fsc_bucket_project_transpose_a(int64_t B, int32_t I, int32_t m1, int32_t m2, int32_t P, int32_t K,
                                   const float* grad_y, const float* v, const float* u, float* grad_a,
                                   int32_t accumulate, hipStream_t stream);
/* Elements (float or double, as the op) of the workspace of fsc_bucket_project_transpose_vu[_f64] when
 * grad_u is requested. */
int fsc_bucket_project_workspace(int64_t B, int32_t I, int32_t m1, int32_t m2, int32_t P, int32_t K,
                                 int64_t* workspace_floats);
/* project_bucket_transpose_b and _u (csrc/ictd_tp.cpp:210-269): grad_v [B][1][m2] and/or grad_u
 * [m1*m2][P*K] (either may be null) from grad_y, a, v, u. */
int fsc_bucket_project_transpose_vu(int64_t B, int32_t I, int32_t m1, int32_t m2, int32_t P, int32_t K,
                                    const float* grad_y, const float* a, const float* v, const float* u,
                                    float* grad_v, float* grad_u, int32_t accumulate, float* workspace,
                                    hipStream_t stream);
/* mix_bucket_forward (csrc/ictd_tp.cpp:271-294): out from y, w, gates. */
int fsc_bucket_mix(int64_t B, int32_t P, int32_t K, int32_t I, int32_t O, const float* y, const float* w,
                   const float* gates, float* out, int32_t accumulate, hipStream_t stream);
/* Elements of the workspace of fsc_bucket_mix_transpose_w[_f64] (per-split partial sums;
 * fsc_bucket_mix_transpose_y[_f64] needs only P*O*I elements, the transposed weights). */
int fsc_bucket_mix_workspace(int64_t B, int32_t P, int32_t K, int32_t I, int32_t O, int64_t* workspace_floats);
/* mix_bucket_transpose_y (csrc/ictd_tp.cpp:296-322): grad_y [B][P][K][I] from grad_out, w, gates. */
int fsc_bucket_mix_transpose_y(int64_t B, int32_t P, int32_t K, int32_t I, int32_t O, const float* grad_out,
                               const float* w, const float* gates, float* grad_y, int32_t accumulate,
                               float* workspace, hipStream_t stream);
/* mix_bucket_transpose_w (csrc/ictd_tp.cpp:324-345): grad_w [P][O][I] from grad_out, y, gates. */
int fsc_bucket_mix_transpose_w(int64_t B, int32_t P, int32_t K, int32_t I, int32_t O, const float* grad_out,
                               const float* y, const float* gates, float* grad_w, int32_t accumulate,
                               float* workspace, hipStream_t stream);
/* mix_bucket_transpose_g (csrc/ictd_tp.cpp:347-373): grad_gates [B][P] from grad_out, y, w. */
int fsc_bucket_mix_transpose_g(int64_t B, int32_t P, int32_t K, int32_t I, int32_t O, const float* grad_out,
                               const float* y, const float* w, float* grad_gates, int32_t accumulate,
                               hipStream_t stream);
/* fp64 twins of the seven functions above (the same reference functions for float64 tensors; mixes on
 * v_mfma_f64_16x16x4_f64). */
int fsc_bucket_project_f64(int64_t B, int32_t I, int32_t m1, int32_t m2, int32_t P, int32_t K, const double* a,
                           const double* v, const double* u, double* y, int32_t accumulate, hipStream_t stream);
int fsc_bucket_project_transpose_a_f64(int64_t B, int32_t I, int32_t m1, int32_t m2, int32_t P, int32_t K,
                                       const double* grad_y, const double* v, const double* u, double* grad_a,
                                       int32_t accumulate, hipStream_t stream);
int fsc_bucket_project_transpose_vu_f64(int64_t B, int32_t I, int32_t m1, int32_t m2, int32_t P, int32_t K,
                                        const double* grad_y, const double* a, const double* v, const double* u,
                                        double* grad_v, double* grad_u, int32_t accumulate, double* workspace,
                                        hipStream_t stream);
int fsc_bucket_mix_f64(int64_t B, int32_t P, int32_t K, int32_t I, int32_t O, const double* y, const double* w,
                       const double* gates, double* out, int32_t accumulate, hipStream_t stream);
int fsc_bucket_mix_transpose_y_f64(int64_t B, int32_t P, int32_t K, int32_t I, int32_t O, const double* grad_out,
                                   const double* w, const double* gates, double* grad_y, int32_t accumulate,
                                   double* workspace, hipStream_t stream);
int fsc_bucket_mix_transpose_w_f64(int64_t B, int32_t P, int32_t K, int32_t I, int32_t O, const double* grad_out,
                                   const double* y, const double* gates, double* grad_w, int32_t accumulate,
                                   double* workspace, hipStream_t stream);
int fsc_bucket_mix_transpose_g_f64(int64_t B, int32_t P, int32_t K, int32_t I, int32_t O, const double* grad_out,
                                   const double* y, const double* w, double* grad_gates, int32_t accumulate,
                                   hipStream_t stream);

/* ---------------------------------------------------------------------------------------------
 * Readout invariant Gram bilinear: out[n][o] = sum_{i,j} W[o][i][j] G_n[i][j],
 * G_n[i][j] = scale * sum_m t[n][m][i] t[n][m][j], for t [N][D][nC] (D in {1,3,5,7,9}, nC a
 * multiple of 16 up to 1024) and W [S][nC][nC] (S 32 or 64).  G is never materialised.
 * Replaces PureCartesianSparseInvariantBilinear.forward (models/pure_cartesian_sparse_layers.py:424-456;
 * one call per rank L with scale 3^{-L/2}) and the ICTD readout
 * `einsum("ocd,ncd->no", W_read[l], gram)` (models/pure_cartesian_ictd_layers_full.py:999-1000,
 * models/pure_cartesian_ictd_layers_o3.py:1017-1018; one call per irrep, scale (2l+1)^{-1/2}).
 * ------------------------------------------------------------------------------------------- */

/* Floats of the prepared weight layouts Wf and Wb and of the forward workspace. */
int fsc_gram_sizes(int64_t n_nodes, int32_t nC, int32_t S, int64_t* wf_floats, int64_t* wb_floats,
                   int64_t* workspace_floats);

/* Block-pair layouts of W, each followed by the same values times a power of two sw (2 max|W| sw <
 * 2^14) split into two fp16 planes (fp32-accurate split-fp16 products) and a 512-float tail holding
 * 1/sw: Wf, the forward's W_IJ + W_JI^T (W_II on the diagonal) as [p][16][S][16] then
 * [2][p][16][2][S][8], and Wb, the backward's W + W^T as [p][256][S] then [2][p][256][S]; both are
 * opaque to the caller and hold fsc_gram_sizes' counts. */
int fsc_gram_prepare_weights(const float* W, int32_t S, int32_t nC, float* Wf, float* Wb, hipStream_t stream);

/* out [N][S]; part_ws holds fsc_gram_sizes' workspace_floats (per-chunk partial sums, per-node scales). */
int fsc_gram_forward(int64_t n_nodes, int32_t D, int32_t nC, int32_t S, float scale, const float* t,
                     const float* Wf, float* part_ws, float* out, hipStream_t stream);

/* grad_t [N][D][nC] = scale * sum_j (sum_o grad_out[n][o] (W[o] + W[o]^T))[i][j] t[n][m][j]. */
int fsc_gram_backward(int64_t n_nodes, int32_t D, int32_t nC, int32_t S, float scale, const float* grad_out,
                      const float* t, const float* Wb, float* grad_t, hipStream_t stream);

/* The same two products for t in the quad-major order [nC/4][D][N][4] that fsc_readout_gather_blocked
 * writes (channels 4c..4c+3 of component m of node n at ((c D + m) N + n) 4; t 16-byte aligned);
 * out, grad_out and grad_t keep the layouts above.  A wave's lanes are consecutive nodes, and in this
 * order their operand reads are contiguous.  They replace the same reference code as fsc_gram_forward /
 * fsc_gram_backward (models/pure_cartesian_sparse_layers.py:424-456,
 * models/pure_cartesian_ictd_layers_full.py:999-1000, models/pure_cartesian_ictd_layers_o3.py:1017-1018);
 * the fused readout (fsctep::readout_features) calls them after fsc_readout_gather_blocked. */
int fsc_gram_forward_blocked(int64_t n_nodes, int32_t D, int32_t nC, int32_t S, float scale, const float* t,
                             const float* Wf, float* part_ws, float* out, hipStream_t stream);
int fsc_gram_backward_blocked(int64_t n_nodes, int32_t D, int32_t nC, int32_t S, float scale,
                              const float* grad_out, const float* t, const float* Wb, float* grad_t,
                              hipStream_t stream);

/* ---------------------------------------------------------------------------------------------
 * Readout feature assembly.  From the per-layer node features X_l [N][M][C] (n_layers <= 4) it
 * builds the Gram inputs t_k [N][d_k][nC] of every key k (nC = n_layers * C; key k = components
 * [key_comp0[k], key_comp0[k] + key_dim[k]), n_keys <= 8) and the squared norms
 * sq [N][n_keys][nC], sq[n][k][l*C + c] = sum_{m in key k} X_l[n][m][c]^2.
 * Replaces the readout slicing, concatenation and squared sums of the sparse trunk
 * (models/pure_cartesian_sparse_layers.py:769-833: t_k = cat_l X_l[:, block L, :], invariants
 * sum_m x^2 / 3^{L/2}) and of the ICTD trunks (models/pure_cartesian_ictd_layers_full.py:977-1024,
 * models/pure_cartesian_ictd_layers_o3.py:987-1030: channel-major flatten, layer concatenation and
 * re-split by key for the Gram inputs, (T*T).sum(1) of the per-key layer concatenation T).
 * The t_k layout is a permutation of a node's n_layers*M*C entries given by the host:
 * srcmap[j] = l*M*C + m*C + c for key-major destination column j (t_0's d_0*nC columns, then
 * t_1's, ...), gmap[l*M*C + m*C + c] = j (the inverse; an entry may land in another key's Gram
 * input, as in the ICTD re-split).  t_all holds t_0, t_1, ... back to back (t_k at offset
 * N * sum_{k'<k} key_dim[k'] * nC).  layers / grad_t / grad_layers are host arrays of
 * device pointers (n_layers, n_keys and n_layers entries; a null grad_t[k] means no gradient
 * through t_k, a null grad_sq none through sq).  The scatter writes
 * dX_l[n][m][c] = grad_t_k'[n][gmap(l,m,c) - first column of k'] + 2 X_l[n][m][c] grad_sq[n][k][l*C + c]
 * (k' the key holding column gmap(l,m,c), k the key of component m).
 * ------------------------------------------------------------------------------------------- */
typedef struct FscReadoutTable {
  int32_t n_layers, M, C, n_keys;
  int32_t key_comp0[8], key_dim[8];
} FscReadoutTable;
int fsc_readout_gather(const FscReadoutTable* table, int64_t n_nodes, const float* const* layers,
                       const int32_t* srcmap, float* t_all, float* sq, hipStream_t stream);
/* The gather with each t_k in the quad-major order [nC/4][d_k][N][4] of fsc_gram_forward_blocked (same
 * offsets N * sum_{k'<k} key_dim[k'] * nC; sq unchanged); replaces the same readout assembly as
 * fsc_readout_gather (models/pure_cartesian_sparse_layers.py:769-833,
 * models/pure_cartesian_ictd_layers_full.py:977-1024, models/pure_cartesian_ictd_layers_o3.py:987-1030).  Needs C a multiple of 4, n_layers*M*C <= 12288
 * and 16-byte aligned arrays (status 1 otherwise). */
int fsc_readout_gather_blocked(const FscReadoutTable* table, int64_t n_nodes, const float* const* layers,
                               const int32_t* srcmap, float* t_all, float* sq, hipStream_t stream);
int fsc_readout_scatter(const FscReadoutTable* table, int64_t n_nodes, const float* const* grad_t,
                        const float* grad_sq, const float* const* layers, const int32_t* gmap,
                        float* const* grad_layers, hipStream_t stream);

/* ---------------------------------------------------------------------------------------------
 * Readout head of the energy, per atom: input LayerNorm, NH hidden layers of Linear -> LayerNorm ->
 * SiLU (all H wide), the output Linear to O values and their weighted sum:
 *   e[n] = w . (Wout a_NH(x[n]) + bout).
 * Replaces MainNet.forward (models/mlp.py:8-66) followed by RobustScalarWeightedSum.forward
 * (models/mlp.py:117-133), the energy head of every trunk (e.g.
 * models/pure_cartesian_sparse_layers.py:831-833: weighted_sum(proj_total(f))), and their input
 * gradient.  x [N][K] (K a multiple of 4), H 64, 128 or 256, 1 <= NH <= 4; fp32 products.
 * fsc_readout_mlp_prepare folds the module parameters into one buffer of
 * fsc_readout_mlp_weights_floats floats (opaque to the caller; x, that buffer and grad_x 16-byte
 * aligned).  params is a host array of 2 + 4 NH + 3 device pointers:
 *   input LayerNorm weight [K], bias [K];
 *   per hidden layer l: Linear weight [H][K or H], bias [H], LayerNorm weight [H], bias [H];
 *   output Linear weight [O][H], bias [O]; the weighted sum's weights [O].
 * eps0 / eps[l]: the LayerNorms' eps.  The backward writes grad_x[n] = grad_energy[n] de[n]/dx[n]
 * (the forward recomputed; no parameter gradients).
 * ------------------------------------------------------------------------------------------- */
typedef struct FscMlpDims {
  int32_t K, H, NH, O;
  float eps0;
  float eps[4];
} FscMlpDims;
int fsc_readout_mlp_weights_floats(const FscMlpDims* dims, int64_t* floats);
int fsc_readout_mlp_prepare(const FscMlpDims* dims, const float* const* params, float* weights, hipStream_t stream);
/* energy [N] */
int fsc_readout_mlp_forward(const FscMlpDims* dims, int64_t n_atoms, const float* x, const float* weights,
                            float* energy, hipStream_t stream);
/* grad_energy [N] in, grad_x [N][K] out */
int fsc_readout_mlp_backward(const FscMlpDims* dims, int64_t n_atoms, const float* x, const float* weights,
                             const float* grad_energy, float* grad_x, hipStream_t stream);

#ifdef __cplusplus
}
#endif

#endif /* FSCTEP_H */
