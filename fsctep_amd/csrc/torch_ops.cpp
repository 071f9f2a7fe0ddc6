// TorchScript / LibTorch registration of the fsctep ops: `torch.ops.fsctep.*`.
//
// This library (libfsctep_torch.so) is the op boundary for both Python and C++ callers.  It holds
// the schemas, the device kernels (the C ABI of libfsctep_hip.so launched on the current stream),
// Meta kernels (shapes only: make_fx / torch.export / FakeTensor) and C++ autograd kernels whose
// backward is again a registered op.  It needs no Python: a LibTorch process (the LAMMPS engine,
// lammps_user_mfftorch/src/USER-MFFTORCH/mff_torch_engine.cpp:226-249 loads MFF_CUSTOM_OPS_LIB with
// RTLD_GLOBAL) gets the ops by loading it, and a TorchScript core.pt whose graph calls them runs
// there with forces from C++ autograd (mff_torch_engine.cpp:818-820).
//
// Parameter gradients are not produced (the path serves energy and forces) except by the ICTD conv, whose
// autograd also gives the weight gradient and the double backward of force training; the other autograd
// kernels raise if a parameter gradient is requested.  ICTD layout tables travel as a CPU int32 tensor holding the
// FscIctdLayout struct.

#include <ATen/ATen.h>
#include <c10/hip/HIPStream.h>
#include <torch/autograd.h>
#include <torch/library.h>

#include "fsctep.h"

namespace {

using at::Tensor;
using torch::autograd::AutogradContext;
using torch::autograd::variable_list;

constexpr int64_t KH = 64;   // radial hidden width feeding the last radial Linear

hipStream_t stream_of(const Tensor& t) { return c10::hip::getCurrentHIPStream(t.device().index()).stream(); }

void check(int rc, const char* name) {
  TORCH_CHECK(rc == 0, name, " failed (", rc, "): ", fsc_last_error());
}

void require_gpu(std::initializer_list<std::reference_wrapper<const Tensor>> ts) {
  for (const Tensor& t : ts)
    TORCH_CHECK(!t.defined() || t.is_cuda(), "fsctep ops run on the GPU only (HIP kernels); got a ",
                t.device(), " tensor");
}

Tensor f32c(const Tensor& t) { return t.to(at::kFloat).contiguous(); }

Tensor i32c(const Tensor& t, const char* what) {
  TORCH_CHECK(t.scalar_type() == at::kInt, what, " must be int32");
  return t.contiguous();
}

const float* cf(const Tensor& t) { return t.numel() ? t.data_ptr<float>() : nullptr; }
float* mf(Tensor& t) { return t.numel() ? t.data_ptr<float>() : nullptr; }
const int32_t* ci(const Tensor& t) { return t.numel() ? t.data_ptr<int32_t>() : nullptr; }

// node_order: empty (the identity) or an int32 permutation of the N nodes (spatial_order)
const int32_t* order_ptr(const Tensor& order, int64_t N) {
  if (order.numel() == 0) return nullptr;
  TORCH_CHECK(order.scalar_type() == at::kInt && order.dim() == 1 && order.size(0) == N && order.is_contiguous(),
              "node_order must be empty or a contiguous int32 permutation of the ", N, " nodes");
  return order.data_ptr<int32_t>();
}

at::TensorOptions fopts(const Tensor& like) { return like.options().dtype(at::kFloat); }

// Layout tables (FscIctdLayout, FscReadoutTable, FscHarmTable) travel as int[] arguments holding the
// struct's 32-bit words: host values in every graph (a tensor constant would be moved to the GPU by
// torch::jit::load(path, device), and reading it on the host would then need a synchronisation).
template <typename S>
S unpack_table(at::IntArrayRef words, const char* what) {
  TORCH_CHECK((int64_t)words.size() * 4 == (int64_t)sizeof(S), what, " must be a list of ", sizeof(S) / 4,
              " int32 words, got ", words.size());
  S s;
  int32_t* w = reinterpret_cast<int32_t*>(&s);
  for (size_t i = 0; i < words.size(); ++i) w[i] = (int32_t)words[i];
  return s;
}

// ============================================================== sparse (pure-cartesian-sparse)

// 1 / max(E/N, 1e-8): the conv2..n normalisation (models/pure_cartesian_sparse_layers.py:419-420), taken from
// the tensor sizes at run time so that a traced graph stays valid for every system size.
float avg_degree_inv(int64_t N, int64_t E) {
  return (float)(1.0 / std::max((double)E / (double)std::max<int64_t>(N, 1), 1e-8));
}

int64_t sparse_weight_floats(int64_t C) { return 6 * 65 * C * C + 512 + 3 * 65 * C * C; }

std::tuple<Tensor, Tensor> sparse_prepare_weights(const Tensor& w_last, const Tensor& b_last, int64_t channels) {
  require_gpu({w_last, b_last});
  const int64_t C = channels;
  TORCH_CHECK(w_last.dim() == 2 && w_last.size(0) == 6 * C * C && w_last.size(1) == KH && b_last.numel() == 6 * C * C,
              "fc.4 of a sparse conv2 layer must be (6*C*C, 64)");
  Tensor w = f32c(w_last), b = f32c(b_last);
  // bk1 and bk6 each hold two fp16 parts of 6*65*C*C values (as many floats), a 512-float tail and a
  // bf16 plane of the same values (3*65*C*C floats)
  Tensor bk1 = at::empty({sparse_weight_floats(C)}, fopts(w)), bk6 = at::empty_like(bk1);
  check(fsc_sparse_conv_prepare_weights(cf(w), cf(b), (int32_t)C, mf(bk1), mf(bk6), stream_of(w)),
        "fsc_sparse_conv_prepare_weights");
  return {bk1, bk6};
}

std::tuple<Tensor, Tensor> sparse_prepare_weights_meta(const Tensor& w_last, const Tensor& b_last, int64_t C) {
  return {at::empty({sparse_weight_floats(C)}, fopts(w_last)), at::empty({sparse_weight_floats(C)}, fopts(w_last))};
}

// w_last / b_last (optional): the raw last radial layer that bk1/bk6 were prepared from; the kernels read the
// prepared buffers, autograd gives the weights' gradient when they are passed and require it.
std::tuple<Tensor, Tensor, Tensor> sparse_conv(const Tensor& x_, const Tensor& h_, const Tensor& n_,
                                               const Tensor& bk1, const Tensor& bk6, const Tensor& dst_ptr,
                                               const Tensor& src_ptr, const Tensor& src_perm,
                                               const Tensor& edge_dst, const Tensor& node_order, int64_t precision,
                                               const std::optional<Tensor>&, const std::optional<Tensor>&) {
  require_gpu({x_, h_, n_, bk1, bk6, dst_ptr, src_ptr, src_perm, edge_dst, node_order});
  TORCH_CHECK(x_.dim() == 3 && x_.size(1) == 13, "x must be (N, 13, C)");
  const int64_t N = x_.size(0), C = x_.size(2), E = h_.size(0);
  Tensor x = f32c(x_), h = f32c(h_), n = f32c(n_);
  Tensor dp = i32c(dst_ptr, "dst_ptr"), sp = i32c(src_ptr, "src_ptr"), pm = i32c(src_perm, "src_perm");
  int64_t s_f = 0, p_f = 0;
  check(fsc_sparse_conv_workspace(N, E, (int32_t)C, &s_f, &p_f), "fsc_sparse_conv_workspace");
  Tensor S = at::empty({s_f}, fopts(x)), P = at::empty({p_f}, fopts(x)), out = at::empty({N, 13, C}, fopts(x));
  check(fsc_sparse_conv_forward(N, E, (int32_t)C, ci(dp), ci(sp), ci(pm), cf(x), cf(h), cf(n), cf(bk1),
                                avg_degree_inv(N, E), mf(S), mf(P), mf(out), (int32_t)precision,
                                order_ptr(node_order, N), stream_of(x)),
        "fsc_sparse_conv_forward");
  return {out, S, P};
}

std::tuple<Tensor, Tensor, Tensor> sparse_conv_meta(const Tensor& x, const Tensor& h, const Tensor&, const Tensor&,
                                                    const Tensor&, const Tensor&, const Tensor&, const Tensor&,
                                                    const Tensor&, const Tensor&, int64_t, const std::optional<Tensor>&,
                                                    const std::optional<Tensor>&) {
  const int64_t N = x.size(0), C = x.size(2), E = h.size(0);
  int64_t s_f = 0, p_f = 0;
  check(fsc_sparse_conv_workspace(N, E, (int32_t)C, &s_f, &p_f), "fsc_sparse_conv_workspace");
  return {at::empty({N, 13, C}, fopts(x)), at::empty({s_f}, fopts(x)), at::empty({p_f}, fopts(x))};
}

// Returns (dx, dh, dn, dS): dS is the backward's workspace holding dS[N][18][65*C] (the gradient of the node
// expansion, consumed by the weight gradient of training) followed by its scratch tail.
std::tuple<Tensor, Tensor, Tensor, Tensor> sparse_conv_backward(const Tensor& grad_out, const Tensor& h_,
                                                                const Tensor& n_, const Tensor& bk6, const Tensor& S,
                                                                const Tensor& P, const Tensor& dst_ptr,
                                                                const Tensor& src_ptr, const Tensor& src_perm,
                                                                const Tensor& edge_dst, const Tensor& node_order,
                                                                int64_t precision) {
  require_gpu({grad_out, h_, n_, bk6, S, P, dst_ptr, src_ptr, src_perm, edge_dst, node_order});
  const int64_t N = grad_out.size(0), C = grad_out.size(2), E = h_.size(0);
  Tensor g = f32c(grad_out), h = f32c(h_), n = f32c(n_);
  Tensor dS = at::empty_like(S), dx = at::empty({N, 13, C}, fopts(g)), dh = at::empty({E, KH}, fopts(g)),
         dn = at::empty({E, 3}, fopts(g));
  check(fsc_sparse_conv_backward(N, E, (int32_t)C, ci(i32c(dst_ptr, "dst_ptr")), ci(i32c(src_ptr, "src_ptr")),
                                 ci(i32c(src_perm, "src_perm")), ci(i32c(edge_dst, "edge_dst")), cf(g), cf(h), cf(n),
                                 cf(bk6), cf(S), cf(P), avg_degree_inv(N, E), mf(dS), mf(dx), mf(dh), mf(dn),
                                 (int32_t)precision, order_ptr(node_order, N), stream_of(g)),
        "fsc_sparse_conv_backward");
  return {dx, dh, dn, dS};
}

std::tuple<Tensor, Tensor, Tensor, Tensor> sparse_conv_backward_meta(const Tensor& grad_out, const Tensor& h,
                                                                     const Tensor&, const Tensor&, const Tensor& S,
                                                                     const Tensor&, const Tensor&, const Tensor&,
                                                                     const Tensor&, const Tensor&, const Tensor&,
                                                                     int64_t) {
  const int64_t E = h.size(0);
  return {at::empty_like(grad_out), at::empty({E, KH}, fopts(h)), at::empty({E, 3}, fopts(h)), at::empty_like(S)};
}

// Derivative of the conv2..n output along edge directions u (the receiver assembly is quadratic in n):
// out'_n = (1/avg deg) sum_{e->n} (0, P1 u, P2 (u n^T + n u^T) + P4 u^T), from the forward's messages P.
Tensor sparse_conv_direction(const Tensor& P, const Tensor& n_, const Tensor& u_, const Tensor& dst_ptr,
                             int64_t channels) {
  require_gpu({P, n_, u_, dst_ptr});
  const int64_t N = dst_ptr.numel() - 1, E = n_.size(0), C = channels;
  Tensor n = f32c(n_), u = f32c(u_);
  TORCH_CHECK(u.sizes() == n.sizes(), "sparse_conv_direction: u must have the shape of n");
  Tensor out = at::empty({N, 13, C}, fopts(n));
  check(fsc_sparse_conv_direction(N, E, (int32_t)C, ci(i32c(dst_ptr, "dst_ptr")), cf(P), cf(n), cf(u),
                                  avg_degree_inv(N, E), mf(out), stream_of(n)),
        "fsc_sparse_conv_direction");
  return out;
}

Tensor sparse_conv_direction_meta(const Tensor&, const Tensor& n, const Tensor&, const Tensor& dst_ptr, int64_t C) {
  return at::empty({dst_ptr.size(0) - 1, 13, C}, fopts(n));
}

// Gradients of <grad_out, out'> for the direction derivative out' along u: (dx, dh, dn, dS); dn is the
// second-derivative term sum_c P2 (g2 + g2^T) u.
std::tuple<Tensor, Tensor, Tensor, Tensor> sparse_conv_direction_backward(
    const Tensor& grad_out, const Tensor& h_, const Tensor& n_, const Tensor& u_, const Tensor& bk6, const Tensor& S,
    const Tensor& P, const Tensor& dst_ptr, const Tensor& src_ptr, const Tensor& src_perm, const Tensor& edge_dst,
    const Tensor& node_order, int64_t precision) {
  require_gpu({grad_out, h_, n_, u_, bk6, S, P, dst_ptr, src_ptr, src_perm, edge_dst, node_order});
  const int64_t N = grad_out.size(0), C = grad_out.size(2), E = h_.size(0);
  Tensor g = f32c(grad_out), h = f32c(h_), n = f32c(n_), u = f32c(u_);
  Tensor dS = at::empty_like(S), dx = at::empty({N, 13, C}, fopts(g)), dh = at::empty({E, KH}, fopts(g)),
         dn = at::empty({E, 3}, fopts(g));
  check(fsc_sparse_conv_direction_backward(N, E, (int32_t)C, ci(i32c(dst_ptr, "dst_ptr")),
                                           ci(i32c(src_ptr, "src_ptr")), ci(i32c(src_perm, "src_perm")),
                                           ci(i32c(edge_dst, "edge_dst")), cf(g), cf(h), cf(n), cf(u), cf(bk6),
                                           cf(S), cf(P), avg_degree_inv(N, E), mf(dS), mf(dx), mf(dh), mf(dn),
                                           (int32_t)precision, order_ptr(node_order, N), stream_of(g)),
        "fsc_sparse_conv_direction_backward");
  return {dx, dh, dn, dS};
}

std::tuple<Tensor, Tensor, Tensor, Tensor> sparse_conv_direction_backward_meta(
    const Tensor& grad_out, const Tensor& h, const Tensor&, const Tensor&, const Tensor&, const Tensor& S,
    const Tensor&, const Tensor&, const Tensor&, const Tensor&, const Tensor&, const Tensor&, int64_t) {
  const int64_t E = h.size(0);
  return {at::empty_like(grad_out), at::empty({E, KH}, fopts(h)), at::empty({E, 3}, fopts(h)), at::empty_like(S)};
}

// Weight gradient of the last radial layer from dS: with W_e[p,c,a] = sum_k L[(p,c,a),k] h_e[k] + b[(p,c,a)]
// and S_m[s][c][k] = sum_a L[(p(s),c,a),k] x_m[comp(s)][a] (Sb likewise with b),
//   dL[(p,c,a),k] = sum_m sum_{s in p} dS_m[s][c*64+k] x_m[comp(s)][a],  db[(p,c,a)] = ... dS_m[s][64C+c] ...
// one GEMM per path (K = nodes x slots of the path; slots and components of a path are contiguous).
std::tuple<Tensor, Tensor> sparse_weight_grad(const Tensor& dS, const Tensor& x_, int64_t C) {
  static const int s0[6] = {0, 1, 2, 3, 6, 9}, sn[6] = {1, 1, 1, 3, 3, 9};
  static const int c0[6] = {0, 0, 0, 1, 1, 4};
  const Tensor x = f32c(x_);
  const int64_t N = x.size(0);
  const Tensor D = dS.narrow(0, 0, N * 18 * 65 * C).view({N, 18, 65 * C});
  Tensor dL = at::empty({6, C, C, KH}, fopts(x)), db = at::empty({6, C, C}, fopts(x));
  for (int p = 0; p < 6; ++p) {
    const Tensor A = D.narrow(1, s0[p], sn[p]).reshape({-1, 65 * C});
    const Tensor X = x.narrow(1, c0[p], sn[p]).reshape({-1, C});
    const Tensor M = A.t().mm(X);                                             // (65 C, C): rows c*64+k, then 64C+c
    dL.select(0, p).copy_(M.narrow(0, 0, KH * C).view({C, KH, C}).permute({0, 2, 1}));
    db.select(0, p).copy_(M.narrow(0, KH * C, C));
  }
  return {dL.view({6 * C * C, KH}), db.view({6 * C * C})};
}

std::tuple<Tensor, Tensor> sparse_conv1_pair_table(const Tensor& w_last, const Tensor& b_last,
                                                   const Tensor& atom_table, int64_t channels) {
  require_gpu({w_last, b_last, atom_table});
  const int64_t C = channels, NS = atom_table.size(0);
  TORCH_CHECK(atom_table.dim() == 2 && atom_table.size(1) == 8 && w_last.size(0) == 6 * C * 64 && w_last.size(1) == KH,
              "conv1 pair table needs output_size 8 and fc.4 of shape (6*C*64, 64)");
  Tensor w = f32c(w_last), b = f32c(b_last), a = f32c(atom_table);
  Tensor mf_ = at::empty({NS * NS * 3 * 65 * C}, fopts(w)), mb = at::empty({NS * NS * 3 * C * 68}, fopts(w));
  check(fsc_sparse_conv1_pair_table(cf(w), cf(b), cf(a), (int32_t)NS, (int32_t)C, mf(mf_), mf(mb), stream_of(w)),
        "fsc_sparse_conv1_pair_table");
  return {mf_, mb};
}

std::tuple<Tensor, Tensor> sparse_conv1_pair_table_meta(const Tensor& w_last, const Tensor&, const Tensor& atom_table,
                                                        int64_t C) {
  const int64_t NS = atom_table.size(0);
  return {at::empty({NS * NS * 3 * 65 * C}, fopts(w_last)), at::empty({NS * NS * 3 * C * 68}, fopts(w_last))};
}

std::tuple<Tensor, Tensor> sparse_conv1(const Tensor& h_, const Tensor& n_, const Tensor& mf_, const Tensor& mb,
                                        const Tensor& dst_ptr, const Tensor& pair_tiles, int64_t channels) {
  require_gpu({h_, n_, mf_, mb, dst_ptr, pair_tiles});
  const int64_t E = h_.size(0), C = channels, n_nodes = dst_ptr.numel() - 1;
  TORCH_CHECK(pair_tiles.numel() % 17 == 0, "pair_tiles must hold 17 int32 per 16-edge tile");
  Tensor h = f32c(h_), n = f32c(n_);
  Tensor Q = at::empty({E * 3 * C}, fopts(h)), out = at::empty({n_nodes, 13, C}, fopts(h));
  check(fsc_sparse_conv1_forward(n_nodes, E, (int32_t)C, ci(i32c(dst_ptr, "dst_ptr")), pair_tiles.numel() / 17,
                                 ci(i32c(pair_tiles, "pair_tiles")), cf(h), cf(n), cf(mf_), cf(mb), mf(Q), mf(out),
                                 stream_of(h)),
        "fsc_sparse_conv1_forward");
  return {out, Q};
}

std::tuple<Tensor, Tensor> sparse_conv1_meta(const Tensor& h, const Tensor&, const Tensor&, const Tensor&,
                                             const Tensor& dst_ptr, const Tensor&, int64_t C) {
  return {at::empty({dst_ptr.numel() - 1, 13, C}, fopts(h)), at::empty({h.size(0) * 3 * C}, fopts(h))};
}

std::tuple<Tensor, Tensor> sparse_conv1_backward(const Tensor& grad_out, const Tensor& n_, const Tensor& mf_,
                                                 const Tensor& Q, const Tensor& dst_ptr, const Tensor& pair_tiles) {
  require_gpu({grad_out, n_, mf_, Q, dst_ptr, pair_tiles});
  const int64_t N = grad_out.size(0), C = grad_out.size(2), E = n_.size(0);
  TORCH_CHECK(pair_tiles.numel() % 17 == 0, "pair_tiles must hold 17 int32 per 16-edge tile");
  Tensor g = f32c(grad_out), n = f32c(n_);
  Tensor dh = at::empty({E, KH}, fopts(g)), dn = at::empty({E, 3}, fopts(g)), dQ = at::empty({E * 3 * C}, fopts(g));
  check(fsc_sparse_conv1_backward(N, E, (int32_t)C, ci(i32c(dst_ptr, "dst_ptr")), pair_tiles.numel() / 17,
                                  ci(i32c(pair_tiles, "pair_tiles")), cf(g), cf(n), cf(mf_), cf(Q), mf(dQ), mf(dh),
                                  mf(dn), stream_of(g)),
        "fsc_sparse_conv1_backward");
  return {dh, dn};
}

std::tuple<Tensor, Tensor> sparse_conv1_backward_meta(const Tensor&, const Tensor& n, const Tensor&, const Tensor&,
                                                      const Tensor&, const Tensor&) {
  return {at::empty({n.size(0), KH}, fopts(n)), at::empty({n.size(0), 3}, fopts(n))};
}

// ============================================================== ICTD (pure-cartesian-ictd / -o3)

// Prepared channel-mix weights: two fp16 planes of W, two of W with the channel axes swapped, a tail.
int64_t ictd_weight_floats(int64_t n_ref, int64_t C) { return 2 * n_ref * C * C + 512; }

Tensor ictd_prepare_weights(const Tensor& W) {
  require_gpu({W});
  const int64_t P = W.size(0), C = W.size(1);
  Tensor Wc = f32c(W).reshape({P, C, C});
  Tensor Wp = at::empty({ictd_weight_floats(P, C)}, fopts(Wc));
  check(fsc_ictd_prepare_weights(cf(Wc), (int32_t)P, (int32_t)C, mf(Wp), stream_of(Wc)), "fsc_ictd_prepare_weights");
  return Wp;
}

Tensor ictd_prepare_weights_meta(const Tensor& W) { return at::empty({ictd_weight_floats(W.size(0), W.size(1))}, fopts(W)); }

int64_t ictd_forward_ws(const FscIctdLayout* L, int64_t N, int64_t C) {
  int64_t z = 0;
  check(fsc_ictd_forward_workspace(L, N, (int32_t)C, &z), "fsc_ictd_forward_workspace");
  return z;
}

Tensor ictd_conv(const Tensor& x_, const Tensor& Y_, const Tensor& gates_, const Tensor& W_, const Tensor& Wt,
                 const Tensor& cg, const Tensor& dst_ptr, const Tensor& edge_src, const Tensor& src_ptr,
                 const Tensor& src_perm, const Tensor& edge_dst, const Tensor& node_order, at::IntArrayRef layout) {
  require_gpu({x_, Y_, gates_, W_, Wt, cg, dst_ptr, edge_src, src_ptr, src_perm, edge_dst, node_order});
  const FscIctdLayout Lv = unpack_table<FscIctdLayout>(layout, "layout");
  const FscIctdLayout* L = &Lv;
  TORCH_CHECK(x_.dim() == 3 && x_.size(1) == L->M, "x must be (N, M, C) for this layout");
  const int64_t N = x_.size(0), C = x_.size(2), E = Y_.size(0);
  Tensor x = f32c(x_), Y = f32c(Y_), gates = f32c(gates_);
  TORCH_CHECK(W_.size(0) == L->NREF && Wt.dim() == 1 && Wt.numel() == ictd_weight_floats(L->NREF, C),
              "ictd_conv: Wt must be ictd_prepare_weights(W) of this layout's weights");
  // z: N*KT*C floats of projections, N per-node scales, then the kernels' split copy of x
  Tensor z = at::empty({ictd_forward_ws(L, N, C)}, fopts(x)), out = at::empty({N, L->M, C}, fopts(x));
  check(fsc_ictd_conv_forward(L, N, E, (int32_t)C, ci(i32c(dst_ptr, "dst_ptr")), ci(i32c(edge_src, "edge_src")),
                              cf(x), cf(Y), cf(gates), cf(cg), cf(Wt), mf(z), mf(out), order_ptr(node_order, N),
                              stream_of(x)),
        "fsc_ictd_conv_forward");
  return out;
}

Tensor ictd_conv_meta(const Tensor& x, const Tensor&, const Tensor&, const Tensor&, const Tensor&, const Tensor&,
                      const Tensor&, const Tensor&, const Tensor&, const Tensor&, const Tensor&, const Tensor&,
                      at::IntArrayRef) {
  return at::empty(x.sizes(), fopts(x));
}

// Receiver-normalised projection Z (N, KT, C) of the forward (the weight gradient's operand).
Tensor ictd_project(const Tensor& x_, const Tensor& Y_, const Tensor& gates_, const Tensor& cg, const Tensor& dst_ptr,
                    const Tensor& edge_src, const Tensor& node_order, at::IntArrayRef layout) {
  require_gpu({x_, Y_, gates_, cg, dst_ptr, edge_src, node_order});
  const FscIctdLayout Lv = unpack_table<FscIctdLayout>(layout, "layout");
  const FscIctdLayout* L = &Lv;
  TORCH_CHECK(x_.dim() == 3 && x_.size(1) == L->M, "x must be (N, M, C) for this layout");
  const int64_t N = x_.size(0), C = x_.size(2), E = Y_.size(0);
  Tensor x = f32c(x_), Y = f32c(Y_), gates = f32c(gates_);
  Tensor z = at::empty({ictd_forward_ws(L, N, C)}, fopts(x));
  check(fsc_ictd_project(L, N, E, (int32_t)C, ci(i32c(dst_ptr, "dst_ptr")), ci(i32c(edge_src, "edge_src")), cf(x),
                         cf(Y), cf(gates), cf(cg), mf(z), order_ptr(node_order, N), stream_of(x)),
        "fsc_ictd_project");
  return z.narrow(0, 0, N * L->KT * C).view({N, L->KT, C});
}

Tensor ictd_project_meta(const Tensor& x, const Tensor&, const Tensor&, const Tensor&, const Tensor&, const Tensor&,
                         const Tensor&, at::IntArrayRef layout) {
  const FscIctdLayout Lv = unpack_table<FscIctdLayout>(layout, "layout");
  return at::empty({x.size(0), Lv.KT, x.size(2)}, fopts(x));
}

// dW[gate_p][o][i] = sum_n sum_m3 G[n][oo_p + m3][o] Z[n][koff_p + m3][i]: one GEMM per live path (K = N d3),
// accumulated per weight slot; slots of paths that are not live stay zero.
Tensor ictd_weight_grad(const Tensor& G, const Tensor& Z, const FscIctdLayout& L, at::IntArrayRef wsizes) {
  const int64_t C = G.size(2);
  Tensor dW = at::zeros({L.NREF, C, C}, G.options());
  for (int p = 0; p < L.NP; ++p) {
    const int64_t d = L.p_d3[p];
    const Tensor Gp = G.narrow(1, L.p_oo[p], d).reshape({-1, C});
    const Tensor Zp = Z.narrow(1, L.p_koff[p], d).reshape({-1, C});
    dW.select(0, L.p_gate[p]).addmm_(Gp.t(), Zp);
  }
  return dW.view(wsizes);
}

std::tuple<Tensor, Tensor, Tensor> ictd_conv_backward(const Tensor& grad_out, const Tensor& x_, const Tensor& Y_,
                                                      const Tensor& gates_, const Tensor& Wt, const Tensor& cg,
                                                      const Tensor& dst_ptr, const Tensor& edge_src,
                                                      const Tensor& src_ptr, const Tensor& src_perm,
                                                      const Tensor& edge_dst, const Tensor& node_order,
                                                      at::IntArrayRef layout) {
  require_gpu({grad_out, x_, Y_, gates_, Wt, cg, dst_ptr, edge_src, src_ptr, src_perm, edge_dst, node_order});
  const FscIctdLayout Lv = unpack_table<FscIctdLayout>(layout, "layout");
  const FscIctdLayout* L = &Lv;
  const int64_t N = x_.size(0), M = x_.size(1), C = x_.size(2), E = Y_.size(0);
  Tensor g = f32c(grad_out), x = f32c(x_), Y = f32c(Y_), gates = f32c(gates_);
  TORCH_CHECK(Wt.dim() == 1 && Wt.numel() == ictd_weight_floats(L->NREF, C),
              "ictd_conv_backward: Wt must be ictd_prepare_weights(W) of this layout's weights");
  int64_t dz_f = 0, r_f = 0;
  check(fsc_ictd_backward_workspace(L, N, (int32_t)C, &dz_f, &r_f), "fsc_ictd_backward_workspace");
  Tensor dz = at::empty({dz_f}, fopts(x)), rw = at::empty({r_f}, fopts(x)), dx = at::empty({N, M, C}, fopts(x));
  Tensor dgates = at::zeros({E, L->NREF}, fopts(x)), dY = at::empty({E, L->NY}, fopts(x));
  check(fsc_ictd_conv_backward(L, N, E, (int32_t)C, ci(i32c(dst_ptr, "dst_ptr")), ci(i32c(edge_src, "edge_src")),
                               ci(i32c(src_ptr, "src_ptr")), ci(i32c(src_perm, "src_perm")),
                               ci(i32c(edge_dst, "edge_dst")), cf(g), cf(x), cf(Y), cf(gates), cf(cg), cf(Wt), mf(dz),
                               mf(rw), mf(dx), mf(dgates), mf(dY), order_ptr(node_order, N), stream_of(x)),
        "fsc_ictd_conv_backward");
  return {dx, dgates, dY};
}

std::tuple<Tensor, Tensor, Tensor> ictd_conv_backward_meta(const Tensor&, const Tensor& x, const Tensor& Y,
                                                           const Tensor& gates, const Tensor&, const Tensor&,
                                                           const Tensor&, const Tensor&, const Tensor&, const Tensor&,
                                                           const Tensor&, const Tensor&, at::IntArrayRef) {
  return {at::empty(x.sizes(), fopts(x)), at::empty(gates.sizes(), fopts(gates)), at::empty(Y.sizes(), fopts(Y))};
}

Tensor ictd_conv1(const Tensor& F_, const Tensor& gates_, const Tensor& qtab_, const Tensor& dst_ptr,
                  const Tensor& edge_pair, const Tensor& node_species, int64_t n_species, int64_t n_comps,
                  at::IntArrayRef layout) {
  require_gpu({F_, gates_, qtab_, dst_ptr, edge_pair, node_species});
  const FscIctdLayout Lv = unpack_table<FscIctdLayout>(layout, "layout");
  const FscIctdLayout* L = &Lv;
  const int64_t n_nodes = dst_ptr.numel() - 1;
  TORCH_CHECK(n_comps == L->M, "n_comps does not match the layout");
  const int64_t C = qtab_.size(-1), E = F_.size(0);
  Tensor F = f32c(F_), gates = f32c(gates_), qtab = f32c(qtab_);
  Tensor out = at::empty({n_nodes, L->M, C}, fopts(F));
  check(fsc_ictd_conv1_forward(L, n_nodes, E, (int32_t)C, (int32_t)n_species, ci(i32c(dst_ptr, "dst_ptr")),
                               ci(i32c(edge_pair, "edge_pair")), ci(i32c(node_species, "node_species")), cf(F),
                               cf(gates), cf(qtab), mf(out), stream_of(F)),
        "fsc_ictd_conv1_forward");
  return out;
}

Tensor ictd_conv1_meta(const Tensor& F, const Tensor&, const Tensor& qtab, const Tensor& dst_ptr, const Tensor&,
                       const Tensor&, int64_t, int64_t n_comps, at::IntArrayRef) {
  return at::empty({dst_ptr.numel() - 1, n_comps, qtab.size(-1)}, fopts(F));
}

std::tuple<Tensor, Tensor> ictd_conv1_backward(const Tensor& grad_out, const Tensor& F_, const Tensor& gates_,
                                               const Tensor& qtab_, const Tensor& dst_ptr, const Tensor& edge_pair,
                                               const Tensor& node_species, int64_t n_species, at::IntArrayRef layout) {
  require_gpu({grad_out, F_, gates_, qtab_, dst_ptr, edge_pair, node_species});
  const FscIctdLayout Lv = unpack_table<FscIctdLayout>(layout, "layout");
  const FscIctdLayout* L = &Lv;
  const int64_t N = grad_out.size(0), C = grad_out.size(2), E = F_.size(0);
  Tensor g = f32c(grad_out), F = f32c(F_), gates = f32c(gates_), qtab = f32c(qtab_);
  Tensor dF = at::empty_like(F), dgates = at::zeros_like(gates);
  check(fsc_ictd_conv1_backward(L, N, E, (int32_t)C, (int32_t)n_species, ci(i32c(dst_ptr, "dst_ptr")),
                                ci(i32c(edge_pair, "edge_pair")), ci(i32c(node_species, "node_species")), cf(g), cf(F),
                                cf(gates), cf(qtab), mf(dF), mf(dgates), stream_of(F)),
        "fsc_ictd_conv1_backward");
  return {dF, dgates};
}

std::tuple<Tensor, Tensor> ictd_conv1_backward_meta(const Tensor&, const Tensor& F, const Tensor& gates, const Tensor&,
                                                    const Tensor&, const Tensor&, const Tensor&, int64_t,
                                                    at::IntArrayRef) {
  return {at::empty(F.sizes(), fopts(F)), at::empty(gates.sizes(), fopts(gates))};
}

// ============================================================== readout Gram bilinear

std::tuple<Tensor, Tensor> gram_prepare_weights(const Tensor& W_) {
  require_gpu({W_});
  TORCH_CHECK(W_.dim() == 3 && W_.size(1) == W_.size(2), "W must be (S, nC, nC)");
  const int64_t S = W_.size(0), nC = W_.size(1);
  Tensor W = f32c(W_);
  // each flat: the fp32 block pairs (P*256*S floats), their two fp16 planes (as many floats) and a tail
  int64_t wfn = 0, wbn = 0, wsn = 0;
  check(fsc_gram_sizes(0, (int32_t)nC, (int32_t)S, &wfn, &wbn, &wsn), "fsc_gram_sizes");
  Tensor Wf = at::empty({wfn}, fopts(W)), Wb = at::empty({wbn}, fopts(W));
  check(fsc_gram_prepare_weights(cf(W), (int32_t)S, (int32_t)nC, mf(Wf), mf(Wb), stream_of(W)),
        "fsc_gram_prepare_weights");
  return {Wf, Wb};
}

std::tuple<Tensor, Tensor> gram_prepare_weights_meta(const Tensor& W) {
  int64_t wfn = 0, wbn = 0, wsn = 0;
  check(fsc_gram_sizes(0, (int32_t)W.size(1), (int32_t)W.size(0), &wfn, &wbn, &wsn), "fsc_gram_sizes");
  return {at::empty({wfn}, fopts(W)), at::empty({wbn}, fopts(W))};
}

// Output width S of prepared forward weights for nC channels (S 32 or 64; fsc_gram_sizes' count).
int64_t gram_width(const Tensor& Wf, int64_t nC) {
  TORCH_CHECK(Wf.dim() == 1 && nC % 16 == 0 && nC >= 16 && nC <= 1024, "prepared Gram weights do not match nC = ", nC);
  for (int32_t S : {32, 64}) {
    int64_t wfn = 0, wbn = 0, wsn = 0;
    check(fsc_gram_sizes(0, (int32_t)nC, S, &wfn, &wbn, &wsn), "fsc_gram_sizes");
    if (Wf.numel() == wfn) return S;
  }
  TORCH_CHECK(false, "prepared Gram weights do not match nC = ", nC);
  return 0;
}

// blocked: t holds the (N, D, nC) values in the quad-major order of the blocked gather (the sizes still
// name N, D and nC)
Tensor gram_forward_impl(const Tensor& t_, const Tensor& Wf, const Tensor& Wb, double scale, bool blocked) {
  require_gpu({t_, Wf, Wb});
  TORCH_CHECK(t_.dim() == 3, "t must be (N, D, nC)");
  const int64_t N = t_.size(0), D = t_.size(1), nC = t_.size(2), S = gram_width(Wf, nC);
  Tensor t = f32c(t_);
  int64_t wfn = 0, wbn = 0, wsn = 0;
  check(fsc_gram_sizes(N, (int32_t)nC, (int32_t)S, &wfn, &wbn, &wsn), "fsc_gram_sizes");
  TORCH_CHECK(Wf.numel() == wfn && Wb.numel() == wbn, "prepared Gram weights do not match nC = ", nC);
  Tensor ws = at::empty({std::max<int64_t>(wsn, 1)}, fopts(t)), out = at::empty({N, S}, fopts(t));
  if (blocked)
    check(fsc_gram_forward_blocked(N, (int32_t)D, (int32_t)nC, (int32_t)S, (float)scale, cf(t), cf(Wf), mf(ws),
                                   mf(out), stream_of(t)),
          "fsc_gram_forward_blocked");
  else
    check(fsc_gram_forward(N, (int32_t)D, (int32_t)nC, (int32_t)S, (float)scale, cf(t), cf(Wf), mf(ws), mf(out),
                           stream_of(t)),
          "fsc_gram_forward");
  return out;
}

Tensor gram_bilinear(const Tensor& t, const Tensor& Wf, const Tensor& Wb, double scale) {
  return gram_forward_impl(t, Wf, Wb, scale, false);
}

// t: (N, D, nC) sizes over values in the blocked order of readout_gather_blocked.
Tensor gram_bilinear_blocked(const Tensor& t, const Tensor& Wf, const Tensor& Wb, double scale) {
  return gram_forward_impl(t, Wf, Wb, scale, true);
}

Tensor gram_bilinear_meta(const Tensor& t, const Tensor& Wf, const Tensor&, double) {
  return at::empty({t.size(0), gram_width(Wf, t.size(2))}, fopts(t));
}

Tensor gram_backward_impl(const Tensor& grad_out, const Tensor& t_, const Tensor& Wb, double scale, bool blocked) {
  require_gpu({grad_out, t_, Wb});
  TORCH_CHECK(grad_out.dim() == 2 && t_.dim() == 3, "grad_out must be (N, S) and t (N, D, nC)");
  const int64_t N = t_.size(0), D = t_.size(1), nC = t_.size(2), S = grad_out.size(1);
  int64_t wfn = 0, wbn = 0, wsn = 0;
  check(fsc_gram_sizes(N, (int32_t)nC, (int32_t)S, &wfn, &wbn, &wsn), "fsc_gram_sizes");
  TORCH_CHECK(Wb.numel() == wbn, "prepared Gram weights do not match nC = ", nC);
  Tensor g = f32c(grad_out), t = f32c(t_);
  Tensor dt = at::empty({N, D, nC}, fopts(t));
  if (blocked)
    check(fsc_gram_backward_blocked(N, (int32_t)D, (int32_t)nC, (int32_t)S, (float)scale, cf(g), cf(t), cf(Wb),
                                    mf(dt), stream_of(t)),
          "fsc_gram_backward_blocked");
  else
    check(fsc_gram_backward(N, (int32_t)D, (int32_t)nC, (int32_t)S, (float)scale, cf(g), cf(t), cf(Wb), mf(dt),
                            stream_of(t)),
          "fsc_gram_backward");
  return dt;
}

Tensor gram_bilinear_backward(const Tensor& grad_out, const Tensor& t, const Tensor& Wb, double scale) {
  return gram_backward_impl(grad_out, t, Wb, scale, false);
}

Tensor gram_bilinear_backward_blocked(const Tensor& grad_out, const Tensor& t, const Tensor& Wb, double scale) {
  return gram_backward_impl(grad_out, t, Wb, scale, true);
}

Tensor gram_bilinear_backward_meta(const Tensor&, const Tensor& t, const Tensor&, double) {
  return at::empty(t.sizes(), fopts(t));
}

// ============================================================== readout MLP (energy head)

// dims = [K, H, NH, O], eps = [input LayerNorm eps, hidden LayerNorms' eps...]
FscMlpDims mlp_dims(at::IntArrayRef dims, at::ArrayRef<double> eps) {
  TORCH_CHECK(dims.size() == 4, "readout mlp dims must be [K, H, NH, O]");
  FscMlpDims d{};
  d.K = (int32_t)dims[0];
  d.H = (int32_t)dims[1];
  d.NH = (int32_t)dims[2];
  d.O = (int32_t)dims[3];
  TORCH_CHECK(d.NH >= 1 && d.NH <= 4 && (int64_t)eps.size() == d.NH + 1,
              "readout mlp: 1 to 4 hidden layers and one LayerNorm eps per LayerNorm");
  d.eps0 = (float)eps[0];
  for (int l = 0; l < d.NH; ++l) d.eps[l] = (float)eps[l + 1];
  return d;
}

int64_t mlp_weights_floats(const FscMlpDims& d) {
  int64_t n = 0;
  check(fsc_readout_mlp_weights_floats(&d, &n), "fsc_readout_mlp_weights_floats");
  return n;
}

Tensor readout_mlp_prepare(at::TensorList params, at::IntArrayRef dims, at::ArrayRef<double> eps) {
  const FscMlpDims d = mlp_dims(dims, eps);
  TORCH_CHECK((int64_t)params.size() == 2 + 4 * d.NH + 3, "readout mlp: expected ", 2 + 4 * d.NH + 3, " parameters");
  std::vector<Tensor> P;
  std::vector<const float*> ptrs;
  for (size_t i = 0; i < params.size(); ++i) {
    require_gpu({params[i]});
    P.push_back(f32c(params[i]));
  }
  // expected element counts: input LN, per layer (W, b, ln g, ln b), output (W, b), weighted-sum weights
  std::vector<int64_t> want = {d.K, d.K};
  for (int l = 0; l < d.NH; ++l) {
    want.push_back((int64_t)d.H * (l == 0 ? d.K : d.H));
    want.push_back(d.H);
    want.push_back(d.H);
    want.push_back(d.H);
  }
  want.push_back((int64_t)d.O * d.H);
  want.push_back(d.O);
  want.push_back(d.O);
  for (size_t i = 0; i < P.size(); ++i) {
    TORCH_CHECK(P[i].numel() == want[i], "readout mlp parameter ", i, " has ", P[i].numel(), " entries, expected ",
                want[i]);
    ptrs.push_back(cf(P[i]));
  }
  Tensor w = at::empty({mlp_weights_floats(d)}, fopts(P[0]));
  check(fsc_readout_mlp_prepare(&d, ptrs.data(), mf(w), stream_of(P[0])), "fsc_readout_mlp_prepare");
  return w;
}

Tensor readout_mlp_prepare_meta(at::TensorList params, at::IntArrayRef dims, at::ArrayRef<double> eps) {
  return at::empty({mlp_weights_floats(mlp_dims(dims, eps))}, fopts(params[0]));
}

Tensor readout_mlp(const Tensor& x_, const Tensor& w, at::IntArrayRef dims, at::ArrayRef<double> eps) {
  require_gpu({x_, w});
  const FscMlpDims d = mlp_dims(dims, eps);
  TORCH_CHECK(x_.dim() == 2 && x_.size(1) == d.K, "x must be (N, ", d.K, ")");
  TORCH_CHECK(w.scalar_type() == at::kFloat && w.is_contiguous() && w.numel() == mlp_weights_floats(d),
              "readout mlp weights do not match the dims (readout_mlp_prepare's output expected)");
  Tensor x = f32c(x_);
  const int64_t N = x.size(0);
  Tensor e = at::empty({N, 1}, fopts(x));
  check(fsc_readout_mlp_forward(&d, N, cf(x), cf(w), mf(e), stream_of(x)), "fsc_readout_mlp_forward");
  return e;
}

Tensor readout_mlp_meta(const Tensor& x, const Tensor&, at::IntArrayRef, at::ArrayRef<double>) {
  return at::empty({x.size(0), 1}, fopts(x));
}

Tensor readout_mlp_backward(const Tensor& grad_, const Tensor& x_, const Tensor& w, at::IntArrayRef dims,
                            at::ArrayRef<double> eps) {
  require_gpu({grad_, x_, w});
  const FscMlpDims d = mlp_dims(dims, eps);
  TORCH_CHECK(x_.dim() == 2 && x_.size(1) == d.K, "x must be (N, ", d.K, ")");
  TORCH_CHECK(grad_.numel() == x_.size(0), "grad must hold one value per row of x");
  TORCH_CHECK(w.scalar_type() == at::kFloat && w.is_contiguous() && w.numel() == mlp_weights_floats(d),
              "readout mlp weights do not match the dims (readout_mlp_prepare's output expected)");
  Tensor x = f32c(x_), g = f32c(grad_);
  const int64_t N = x.size(0);
  Tensor dx = at::empty({N, d.K}, fopts(x));
  check(fsc_readout_mlp_backward(&d, N, cf(x), cf(w), cf(g), mf(dx), stream_of(x)), "fsc_readout_mlp_backward");
  return dx;
}

Tensor readout_mlp_backward_meta(const Tensor&, const Tensor& x, const Tensor&, at::IntArrayRef,
                                 at::ArrayRef<double>) {
  return at::empty(x.sizes(), fopts(x));
}

// -------------------------------------------------------------- readout feature assembly

// The layers as float32 contiguous [N][M][C] tensors (kept alive by the caller).
std::vector<Tensor> readout_layers(at::TensorList layers, const FscReadoutTable* T) {
  TORCH_CHECK((int64_t)layers.size() == T->n_layers, "expected ", T->n_layers, " feature layers, got ",
              layers.size());
  std::vector<Tensor> out;
  for (const Tensor& x : layers) {
    require_gpu({x});
    TORCH_CHECK(x.dim() == 3 && x.size(0) == layers[0].size(0) && x.size(1) == T->M && x.size(2) == T->C,
                "feature layers must be (N, ", T->M, ", ", T->C, ")");
    out.push_back(f32c(x));
  }
  return out;
}

Tensor readout_map(const Tensor& map, const FscReadoutTable* T, const char* what) {
  require_gpu({map});
  TORCH_CHECK(map.numel() == (int64_t)T->n_layers * T->M * T->C, what, " must have n_layers*M*C entries");
  return i32c(map, what);
}

bool aligned16(const Tensor& t) { return (reinterpret_cast<uintptr_t>(t.data_ptr()) & 15) == 0; }

// Whether the blocked gather takes this table: C a multiple of 4 and a node's n_layers*M*C <= 8192 entries
// in LDS (decided from the table alone, so that every device, tracing ones included, takes the same path).
bool readout_blocked(const FscReadoutTable* T) {
  return T->C % 4 == 0 && (int64_t)T->n_layers * T->M * T->C <= 8192;
}

std::tuple<Tensor, Tensor> readout_gather_impl(at::TensorList layers, const Tensor& srcmap, at::IntArrayRef table,
                                               bool blocked) {
  const FscReadoutTable Tv = unpack_table<FscReadoutTable>(table, "readout table");
  const FscReadoutTable* T = &Tv;
  std::vector<Tensor> X = readout_layers(layers, T);
  Tensor sm = readout_map(srcmap, T, "srcmap");
  if (blocked) {   // the quad kernels need 16-byte aligned rows: a view at an odd offset is copied
    TORCH_CHECK(readout_blocked(T), "readout_gather_blocked: needs C a multiple of 4 and n_layers*M*C <= 8192");
    for (Tensor& x : X)
      if (!aligned16(x)) x = x.clone();
    if (!aligned16(sm)) sm = sm.clone();
  }
  const int64_t N = X[0].size(0), nC = (int64_t)T->n_layers * T->C;
  Tensor t_all = at::empty({N * T->M * nC}, fopts(X[0]));
  Tensor sq = at::empty({N, T->n_keys, nC}, fopts(X[0]));
  std::vector<const float*> xp;
  for (const Tensor& x : X) xp.push_back(cf(x));
  if (blocked)
    check(fsc_readout_gather_blocked(T, N, xp.data(), ci(sm), mf(t_all), mf(sq), stream_of(X[0])),
          "fsc_readout_gather_blocked");
  else
    check(fsc_readout_gather(T, N, xp.data(), ci(sm), mf(t_all), mf(sq), stream_of(X[0])), "fsc_readout_gather");
  return {t_all, sq};
}

std::tuple<Tensor, Tensor> readout_gather(at::TensorList layers, const Tensor& srcmap, at::IntArrayRef table) {
  return readout_gather_impl(layers, srcmap, table, false);
}

// t_all with each key's Gram input in the quad-major order [nC/4][d_k][N][4] (fsc_readout_gather_blocked).
std::tuple<Tensor, Tensor> readout_gather_blocked(at::TensorList layers, const Tensor& srcmap,
                                                  at::IntArrayRef table) {
  return readout_gather_impl(layers, srcmap, table, true);
}

std::tuple<Tensor, Tensor> readout_gather_meta(at::TensorList layers, const Tensor&, at::IntArrayRef table) {
  const FscReadoutTable Tv = unpack_table<FscReadoutTable>(table, "readout table");
  const FscReadoutTable* T = &Tv;
  const int64_t N = layers[0].size(0), nC = (int64_t)T->n_layers * T->C;
  return {at::empty({N * T->M * nC}, fopts(layers[0])), at::empty({N, T->n_keys, nC}, fopts(layers[0]))};
}

std::vector<Tensor> readout_scatter(const c10::List<std::optional<Tensor>>& grad_t, const std::optional<Tensor>& grad_sq,
                                    at::TensorList layers, const Tensor& gmap, at::IntArrayRef table) {
  const FscReadoutTable Tv = unpack_table<FscReadoutTable>(table, "readout table");
  const FscReadoutTable* T = &Tv;
  std::vector<Tensor> X = readout_layers(layers, T);
  Tensor gm = readout_map(gmap, T, "gmap");
  const int64_t N = X[0].size(0), nC = (int64_t)T->n_layers * T->C;
  TORCH_CHECK((int64_t)grad_t.size() == T->n_keys, "expected ", T->n_keys, " Gram-input gradients");
  std::vector<Tensor> dt;
  std::vector<const float*> dtp;
  for (int k = 0; k < T->n_keys; ++k) {
    const std::optional<Tensor> g = grad_t.get(k);
    if (g.has_value() && g->defined()) {
      require_gpu({*g});
      TORCH_CHECK(g->numel() == N * T->key_dim[k] * nC, "gradient of Gram input ", k, " has the wrong size");
      dt.push_back(f32c(*g));
      dtp.push_back(cf(dt.back()));
    } else {
      dtp.push_back(nullptr);
    }
  }
  Tensor dsq;
  if (grad_sq.has_value() && grad_sq->defined()) {
    require_gpu({*grad_sq});
    TORCH_CHECK(grad_sq->numel() == N * T->n_keys * nC, "grad_sq must be (N, n_keys, n_layers*C)");
    dsq = f32c(*grad_sq);
  }
  std::vector<Tensor> dX;
  std::vector<const float*> xp;
  std::vector<float*> dxp;
  for (const Tensor& x : X) {
    dX.push_back(at::empty(x.sizes(), fopts(x)));
    xp.push_back(cf(x));
    dxp.push_back(mf(dX.back()));
  }
  check(fsc_readout_scatter(T, N, dtp.data(), dsq.defined() ? cf(dsq) : nullptr, xp.data(), ci(gm), dxp.data(),
                            stream_of(X[0])),
        "fsc_readout_scatter");
  return dX;
}

std::vector<Tensor> readout_scatter_meta(const c10::List<std::optional<Tensor>>&, const std::optional<Tensor>&,
                                         at::TensorList layers, const Tensor&, at::IntArrayRef) {
  std::vector<Tensor> dX;
  for (const Tensor& x : layers) dX.push_back(at::empty(x.sizes(), fopts(x)));
  return dX;
}

// Gram input k of the gathered buffer as an (N, d_k, nC) view.
Tensor gram_input(const Tensor& t_all, const FscReadoutTable* T, int64_t N, int k) {
  const int64_t nC = (int64_t)T->n_layers * T->C;
  int64_t col0 = 0;
  for (int j = 0; j < k; ++j) col0 += T->key_dim[j] * nC;
  return t_all.narrow(0, N * col0, N * T->key_dim[k] * nC).view({N, T->key_dim[k], nC});
}

// scalars = sum_k gram_bilinear(t_k, Wf[k], Wb[k], scales[k]) and the squared norms.  The Gram inputs only
// live between the gather and the Gram kernels, so where the blocked gather applies they are written in the
// quad-major order that the blocked Gram kernels read.
std::tuple<Tensor, Tensor> readout_features(at::TensorList layers, at::TensorList Wf, at::TensorList Wb,
                                            at::ArrayRef<double> scales, const Tensor& srcmap, const Tensor&,
                                            at::IntArrayRef table) {
  const FscReadoutTable Tv = unpack_table<FscReadoutTable>(table, "readout table");
  const FscReadoutTable* T = &Tv;
  TORCH_CHECK((int64_t)Wf.size() == T->n_keys && (int64_t)Wb.size() == T->n_keys &&
                  (int64_t)scales.size() == T->n_keys,
              "one prepared Gram weight pair and scale per key");
  const bool blocked = readout_blocked(T);
  auto [t_all, sq] = readout_gather_impl(layers, srcmap, table, blocked);
  const int64_t N = layers[0].size(0);
  Tensor scalars;
  for (int k = 0; k < T->n_keys; ++k) {
    Tensor o = gram_forward_impl(gram_input(t_all, T, N, k), Wf[k], Wb[k], scales[k], blocked);
    scalars = scalars.defined() ? scalars.add_(o) : o;
  }
  return {scalars, sq};
}

std::tuple<Tensor, Tensor> readout_features_meta(at::TensorList layers, at::TensorList Wf, at::TensorList,
                                                 at::ArrayRef<double>, const Tensor&, const Tensor&,
                                                 at::IntArrayRef table) {
  const FscReadoutTable Tv = unpack_table<FscReadoutTable>(table, "readout table");
  const FscReadoutTable* T = &Tv;
  const int64_t N = layers[0].size(0), nC = (int64_t)T->n_layers * T->C;
  return {at::empty({N, gram_width(Wf[0], nC)}, fopts(layers[0])), at::empty({N, T->n_keys, nC}, fopts(layers[0]))};
}


// ============================================================== graph preparation

Tensor i64c(const Tensor& t) { return t.to(at::kLong).contiguous(); }

// The receiver sort and index structures of one neighbour list (fsc_graph_prepare), rebuilt per call as the
// reference re-sorts per call; every output size follows from (N, E, n_species), so traces stay valid.
std::vector<Tensor> graph_prepare(const Tensor& edge_src_, const Tensor& edge_dst_, const Tensor& species_,
                                  int64_t n_species) {
  require_gpu({edge_src_, edge_dst_, species_});
  TORCH_CHECK(edge_src_.dim() == 1 && edge_dst_.dim() == 1 && edge_src_.numel() == edge_dst_.numel() &&
                  species_.dim() == 1,
              "graph_prepare: edge_src, edge_dst (E,) and species (N,)");
  const int64_t E = edge_src_.numel(), N = species_.numel();
  int64_t T = 0, ws_n = 0;
  check(fsc_graph_sizes(N, E, (int32_t)n_species, &T, &ws_n), "fsc_graph_sizes");
  Tensor src = i64c(edge_src_), dst = i64c(edge_dst_), sp = i64c(species_);
  const auto io = src.options().dtype(at::kInt);
  Tensor order = at::empty({E}, io), src32 = at::empty({E}, io), dst32 = at::empty({E}, io);
  Tensor dst_ptr = at::empty({N + 1}, io), src_ptr = at::empty({N + 1}, io), src_perm = at::empty({E}, io);
  Tensor node_species = at::empty({n_species > 0 ? N : 0}, io), edge_pair = at::empty({n_species > 0 ? E : 0}, io);
  Tensor pair_tiles = at::empty({17 * T}, io), status = at::empty({1}, io), ws = at::empty({ws_n}, io);
  auto ip = [](Tensor& t) { return t.numel() ? t.data_ptr<int32_t>() : nullptr; };
  check(fsc_graph_prepare(N, E, (int32_t)n_species, E ? src.data_ptr<int64_t>() : nullptr,
                          E ? dst.data_ptr<int64_t>() : nullptr, N ? sp.data_ptr<int64_t>() : nullptr, ip(order),
                          ip(src32), ip(dst32), ip(dst_ptr), ip(src_ptr), ip(src_perm), ip(node_species), ip(edge_pair),
                          ip(pair_tiles), ip(status), ip(ws), stream_of(src)),
        "fsc_graph_prepare");
  return {order, src32, dst32, dst_ptr, src_ptr, src_perm, node_species, edge_pair, pair_tiles, status};
}

std::vector<Tensor> graph_prepare_meta(const Tensor& edge_src, const Tensor&, const Tensor& species,
                                       int64_t n_species) {
  const int64_t E = edge_src.numel(), N = species.numel();
  int64_t T = 0, ws_n = 0;
  check(fsc_graph_sizes(N, E, (int32_t)n_species, &T, &ws_n), "fsc_graph_sizes");
  const auto io = edge_src.options().dtype(at::kInt);
  return {at::empty({E}, io), at::empty({E}, io), at::empty({E}, io), at::empty({N + 1}, io), at::empty({N + 1}, io),
          at::empty({E}, io), at::empty({n_species > 0 ? N : 0}, io), at::empty({n_species > 0 ? E : 0}, io),
          at::empty({17 * T}, io), at::empty({1}, io)};
}

// Spatial order of the atoms (fsc_spatial_order): the node_order argument of the conv ops.
Tensor spatial_order(const Tensor& pos_) {
  require_gpu({pos_});
  TORCH_CHECK(pos_.dim() == 2 && pos_.size(1) == 3, "spatial_order: pos must be (N, 3)");
  const int64_t N = pos_.size(0);
  Tensor pos = f32c(pos_);
  int64_t ws_n = 0;
  check(fsc_spatial_order_workspace(N, &ws_n), "fsc_spatial_order_workspace");
  const auto io = pos.options().dtype(at::kInt);
  Tensor order = at::empty({N}, io), ws = at::empty({ws_n}, io);
  check(fsc_spatial_order(N, cf(pos), N ? order.data_ptr<int32_t>() : nullptr, ws.data_ptr<int32_t>(),
                          stream_of(pos)),
        "fsc_spatial_order");
  return order;
}

Tensor spatial_order_meta(const Tensor& pos) { return at::empty({pos.size(0)}, pos.options().dtype(at::kInt)); }

// Radius graph with periodic images (fsc_neighbor_count / fsc_neighbor_fill).  The edge count is data
// dependent: it is read back after the count pass (one host synchronisation, as torch_cluster's radius).
std::vector<Tensor> neighbor_list(const Tensor& pos_, const Tensor& cell_, double cutoff, at::IntArrayRef pbc) {
  require_gpu({pos_, cell_});
  TORCH_CHECK(pos_.dim() == 2 && pos_.size(1) == 3, "neighbor_list: pos must be (N, 3)");
  TORCH_CHECK(cell_.numel() == 9, "neighbor_list: cell must hold 3x3 values (rows = lattice vectors)");
  TORCH_CHECK(pbc.size() == 3, "neighbor_list: pbc must have 3 flags");
  const int64_t N = pos_.size(0);
  Tensor pos = pos_.to(at::kDouble).contiguous(), cell = cell_.to(at::kDouble).reshape({3, 3}).contiguous();
  const int32_t flags[3] = {(int32_t)(pbc[0] != 0), (int32_t)(pbc[1] != 0), (int32_t)(pbc[2] != 0)};
  int64_t ws_n = 0;
  check(fsc_neighbor_workspace(N, &ws_n), "fsc_neighbor_workspace");
  const auto io = pos.options().dtype(at::kInt);
  Tensor ws = at::empty({ws_n}, io), dst_ptr = at::empty({N + 1}, io);
  const double* pp = N ? pos.data_ptr<double>() : nullptr;
  check(fsc_neighbor_count(N, pp, cell.data_ptr<double>(), flags, cutoff, dst_ptr.data_ptr<int32_t>(),
                           ws.data_ptr<int32_t>(), stream_of(pos)),
        "fsc_neighbor_count");
  const int64_t E = dst_ptr.select(0, N).item<int32_t>();
  TORCH_CHECK(E >= 0, "neighbor_list: edge count overflow");
  Tensor src = at::empty({E}, pos.options().dtype(at::kLong)), dst = at::empty({E}, pos.options().dtype(at::kLong));
  Tensor shifts = at::empty({E, 3}, pos.options()), fill_ws = at::empty({3 * E}, io);
  check(fsc_neighbor_fill(N, E, pp, cell.data_ptr<double>(), flags, cutoff, dst_ptr.data_ptr<int32_t>(),
                          ws.data_ptr<int32_t>(), E ? fill_ws.data_ptr<int32_t>() : nullptr,
                          E ? src.data_ptr<int64_t>() : nullptr, E ? dst.data_ptr<int64_t>() : nullptr,
                          E ? shifts.data_ptr<double>() : nullptr, stream_of(pos)),
        "fsc_neighbor_fill");
  return {src, dst, shifts, dst_ptr};
}

// ============================================================== geometry from caller-supplied edge vectors

std::tuple<Tensor, Tensor> edge_vec_geometry(const Tensor& edge_vec_, const Tensor& order) {
  require_gpu({edge_vec_, order});
  const int64_t E = order.numel();
  TORCH_CHECK(edge_vec_.dim() == 2 && edge_vec_.size(0) == E && edge_vec_.size(1) == 3, "edge_vec must be (E, 3)");
  Tensor v = f32c(edge_vec_);
  Tensor n = at::empty({E, 3}, fopts(v)), r = at::empty({E}, fopts(v));
  check(fsc_edge_vec_geometry_forward(E, cf(v), ci(i32c(order, "order")), mf(n), mf(r), stream_of(v)),
        "fsc_edge_vec_geometry_forward");
  return {n, r};
}

std::tuple<Tensor, Tensor> edge_vec_geometry_meta(const Tensor& edge_vec, const Tensor& order) {
  const int64_t E = order.numel();
  return {at::empty({E, 3}, fopts(edge_vec)), at::empty({E}, fopts(edge_vec))};
}

Tensor edge_vec_geometry_backward(const std::optional<Tensor>& grad_n, const std::optional<Tensor>& grad_r,
                                  const Tensor& n_, const Tensor& r_, const Tensor& order) {
  const bool has_n = grad_n.has_value() && grad_n->defined(), has_r = grad_r.has_value() && grad_r->defined();
  require_gpu({n_, r_, order});
  if (has_n) require_gpu({*grad_n});
  if (has_r) require_gpu({*grad_r});
  const int64_t E = r_.numel();
  Tensor n = f32c(n_), r = f32c(r_);
  Tensor gn = has_n ? f32c(*grad_n) : Tensor(), gr = has_r ? f32c(*grad_r) : Tensor();
  Tensor gvec = at::empty({E, 3}, fopts(n));
  check(fsc_edge_vec_geometry_backward(E, gn.defined() ? cf(gn) : nullptr, gr.defined() ? cf(gr) : nullptr, cf(n),
                                       cf(r), ci(i32c(order, "order")), mf(gvec), stream_of(n)),
        "fsc_edge_vec_geometry_backward");
  return gvec;
}

Tensor edge_vec_geometry_backward_meta(const std::optional<Tensor>&, const std::optional<Tensor>&, const Tensor& n,
                                       const Tensor&, const Tensor&) {
  return at::empty({n.size(0), 3}, fopts(n));
}

// ============================================================== autograd

// ============================================================== edge geometry and radial MLP

std::tuple<Tensor, Tensor> edge_geometry(const Tensor& pos_, const Tensor& shift_, const Tensor& edge_src,
                                         const Tensor& edge_dst, const Tensor& dst_ptr, const Tensor& src_ptr,
                                         const Tensor& src_perm) {
  require_gpu({pos_, shift_, edge_src, edge_dst, dst_ptr, src_ptr, src_perm});
  const int64_t E = edge_src.numel();
  TORCH_CHECK(pos_.dim() == 2 && pos_.size(1) == 3 && shift_.numel() == 3 * E, "pos (N,3), shift (E,3)");
  Tensor pos = f32c(pos_), shift = f32c(shift_);
  Tensor n = at::empty({E, 3}, fopts(pos)), r = at::empty({E}, fopts(pos));
  check(fsc_edge_geometry_forward(E, cf(pos), cf(shift), ci(i32c(edge_src, "edge_src")), ci(i32c(edge_dst, "edge_dst")),
                                  mf(n), mf(r), stream_of(pos)),
        "fsc_edge_geometry_forward");
  return {n, r};
}

std::tuple<Tensor, Tensor> edge_geometry_meta(const Tensor& pos, const Tensor&, const Tensor& edge_src, const Tensor&,
                                              const Tensor&, const Tensor&, const Tensor&) {
  const int64_t E = edge_src.numel();
  return {at::empty({E, 3}, fopts(pos)), at::empty({E}, fopts(pos))};
}

Tensor edge_geometry_backward(const std::optional<Tensor>& grad_n, const std::optional<Tensor>& grad_r,
                              const Tensor& n_, const Tensor& r_, const Tensor& dst_ptr, const Tensor& src_ptr,
                              const Tensor& src_perm) {
  const bool has_n = grad_n.has_value() && grad_n->defined(), has_r = grad_r.has_value() && grad_r->defined();
  require_gpu({n_, r_, dst_ptr, src_ptr, src_perm});
  if (has_n) require_gpu({*grad_n});
  if (has_r) require_gpu({*grad_r});
  const int64_t N = dst_ptr.numel() - 1, E = r_.numel();
  Tensor n = f32c(n_), r = f32c(r_);
  Tensor gn = has_n ? f32c(*grad_n) : Tensor(), gr = has_r ? f32c(*grad_r) : Tensor();
  Tensor gpos = at::empty({N, 3}, fopts(n));
  check(fsc_edge_geometry_backward(N, E, gn.defined() ? cf(gn) : nullptr, gr.defined() ? cf(gr) : nullptr, cf(n),
                                   cf(r), ci(i32c(dst_ptr, "dst_ptr")), ci(i32c(src_ptr, "src_ptr")),
                                   ci(i32c(src_perm, "src_perm")), mf(gpos), stream_of(n)),
        "fsc_edge_geometry_backward");
  return gpos;
}

Tensor edge_geometry_backward_meta(const std::optional<Tensor>&, const std::optional<Tensor>&, const Tensor& n,
                                   const Tensor&, const Tensor& dst_ptr, const Tensor&, const Tensor&) {
  return at::empty({dst_ptr.numel() - 1, 3}, fopts(n));
}

int32_t basis_code(int64_t basis) {
  TORCH_CHECK(basis >= 0 && basis <= 4, "radial basis: 0 bessel, 1 gaussian, 2 fourier, 3 cosine, 4 smooth_finite");
  return (int32_t)basis;
}

Tensor radial_mlp(const Tensor& r_, const Tensor& w0_, const Tensor& b0_, const Tensor& w2_, const Tensor& b2_,
                  const std::optional<Tensor>& w4_, const std::optional<Tensor>& b4_, double r_cut, int64_t basis) {
  require_gpu({r_, w0_, b0_, w2_, b2_});
  TORCH_CHECK(w0_.dim() == 2 && w0_.size(0) == KH && w2_.dim() == 2 && w2_.size(0) == KH && w2_.size(1) == KH &&
                  b0_.numel() == KH && b2_.numel() == KH,
              "radial MLP: fc.0 (64, nb) and fc.2 (64, 64)");
  const bool fused = w4_.has_value() && w4_->defined();
  Tensor w4, b4;
  if (fused) {
    TORCH_CHECK(b4_.has_value() && b4_->defined() && w4_->dim() == 2 && w4_->size(1) == KH && w4_->size(0) >= 1 &&
                    w4_->size(0) <= KH && b4_->numel() == w4_->size(0),
                "radial MLP: the fused last Linear must be (P, 64) with P <= 64, bias (P)");
    require_gpu({*w4_, *b4_});
    w4 = f32c(*w4_);
    b4 = f32c(*b4_);
  }
  const int64_t E = r_.numel(), P = fused ? w4.size(0) : KH;
  Tensor r = f32c(r_), w0 = f32c(w0_), b0 = f32c(b0_), w2 = f32c(w2_), b2 = f32c(b2_);
  Tensor h = at::empty({E, P}, fopts(r));
  check(fsc_radial_mlp_forward(E, cf(r), cf(w0), cf(b0), cf(w2), cf(b2), fused ? cf(w4) : nullptr,
                               fused ? cf(b4) : nullptr, (int32_t)P, (int32_t)w0.size(1), (float)r_cut,
                               basis_code(basis), mf(h), stream_of(r)),
        "fsc_radial_mlp_forward");
  return h;
}

Tensor radial_mlp_meta(const Tensor& r, const Tensor&, const Tensor&, const Tensor&, const Tensor&,
                       const std::optional<Tensor>& w4, const std::optional<Tensor>&, double, int64_t) {
  return at::empty({r.numel(), (w4.has_value() && w4->defined()) ? w4->size(0) : KH}, fopts(r));
}

Tensor radial_mlp_backward(const Tensor& grad_out, const Tensor& r_, const Tensor& w0_, const Tensor& b0_,
                           const Tensor& w2_, const Tensor& b2_, const std::optional<Tensor>& w4_, double r_cut,
                           int64_t basis) {
  require_gpu({grad_out, r_, w0_, b0_, w2_, b2_});
  const bool fused = w4_.has_value() && w4_->defined();
  Tensor w4 = fused ? f32c(*w4_) : Tensor();
  const int64_t E = r_.numel(), P = fused ? w4.size(0) : KH;
  TORCH_CHECK(grad_out.numel() == E * P, "radial MLP backward: grad shape");
  Tensor g = f32c(grad_out), r = f32c(r_), w0 = f32c(w0_), b0 = f32c(b0_), w2 = f32c(w2_), b2 = f32c(b2_);
  Tensor gr = at::empty({E}, fopts(r));
  check(fsc_radial_mlp_backward(E, cf(r), cf(w0), cf(b0), cf(w2), cf(b2), fused ? cf(w4) : nullptr, (int32_t)P,
                                (int32_t)w0.size(1), (float)r_cut, basis_code(basis), cf(g), mf(gr), stream_of(r)),
        "fsc_radial_mlp_backward");
  return gr;
}

Tensor radial_mlp_backward_meta(const Tensor&, const Tensor& r, const Tensor&, const Tensor&, const Tensor&,
                                const Tensor&, const std::optional<Tensor>&, double, int64_t) {
  return at::empty({r.numel()}, fopts(r));
}


Tensor edge_harmonics(const Tensor& n_, at::IntArrayRef table) {
  require_gpu({n_});
  const FscHarmTable Tv = unpack_table<FscHarmTable>(table, "harmonics table");
  const FscHarmTable* T = &Tv;
  const int64_t E = n_.size(0), NY = (T->lmax + 1) * (T->lmax + 1);
  Tensor n = f32c(n_);
  Tensor Y = at::empty({E, NY}, fopts(n));
  check(fsc_edge_harmonics_forward(T, E, cf(n), mf(Y), stream_of(n)), "fsc_edge_harmonics_forward");
  return Y;
}

Tensor edge_harmonics_meta(const Tensor& n, at::IntArrayRef table) {
  const FscHarmTable Tv = unpack_table<FscHarmTable>(table, "harmonics table");
  const FscHarmTable* T = &Tv;
  return at::empty({n.size(0), (T->lmax + 1) * (T->lmax + 1)}, fopts(n));
}

Tensor edge_harmonics_backward(const Tensor& grad_Y, const Tensor& n_, at::IntArrayRef table) {
  require_gpu({grad_Y, n_});
  const FscHarmTable Tv = unpack_table<FscHarmTable>(table, "harmonics table");
  const FscHarmTable* T = &Tv;
  const int64_t E = n_.size(0);
  Tensor n = f32c(n_), g = f32c(grad_Y);
  Tensor dn = at::empty({E, 3}, fopts(n));
  check(fsc_edge_harmonics_backward(T, E, cf(n), cf(g), mf(dn), stream_of(n)), "fsc_edge_harmonics_backward");
  return dn;
}

Tensor edge_harmonics_backward_meta(const Tensor&, const Tensor& n, at::IntArrayRef) {
  return at::empty({n.size(0), 3}, fopts(n));
}

template <typename... Args>
c10::TypedOperatorHandle<Args...> op_handle(const char* name) {
  return c10::Dispatcher::singleton().findSchemaOrThrow(name, "").typed<Args...>();
}

void refuse_param_grad(AutogradContext* ctx, std::initializer_list<int> idx, const char* what) {
  for (int i : idx)
    TORCH_CHECK(!ctx->needs_input_grad(i), "parameter gradients of ", what,
                " are not implemented (energy/force inference only)");
}

// Backward of the sparse conv2..n as a function of (G, x, h, n, w_last, b_last): (dx, dh, dn, dL, db), itself
// differentiable once (the double backward of force training).  With P = h S(x, W) + Sb(x, W) the
// conv F = A_n(P) is linear in x and in W = (L, b), affine in h (its h-derivative is P with h -> uh and the
// bias dropped: W0 = (L, 0)) and quadratic in n.  For cotangents u = (ux, uh, un, uW) of (dx, dh, dn, dW):
//   d<u,B>/dG = F(ux,h,n,W) + F(x,uh,n,W0) + A'_n[un](P) + F(x,h,n,uW)
//   d<u,B>/dx = B_x(G; h=uh, W0) + Bdir_x(G; un) + B_x(G; W=uW)
//   d<u,B>/dh = B_h(G; x=ux) + Bdir_h(G; un) + B_h(G; W=uW)
//   d<u,B>/dn = B_n(G; x=ux) + B_n(G; h=uh, W0) + Bdir_n(G; un) + B_n(G; W=uW)
//   d<u,B>/dW = B_W(G; x=ux) + B_L(G; h=uh) + Bdir_W(G; un)
// where A'_n[un] (sparse_conv_direction) is the derivative of the receiver assembly along un and Bdir
// (sparse_conv_direction_backward) the gradients of <G, A'_n[un](P)>, its n part being the second-derivative
// term.  Every term runs on the conv's own kernels.
struct SparseConvBwdFn : public torch::autograd::Function<SparseConvBwdFn> {
  using Fwd = std::tuple<Tensor, Tensor, Tensor>(const Tensor&, const Tensor&, const Tensor&, const Tensor&,
                                                 const Tensor&, const Tensor&, const Tensor&, const Tensor&,
                                                 const Tensor&, const Tensor&, int64_t, const std::optional<Tensor>&,
                                                 const std::optional<Tensor>&);
  using Bwd = std::tuple<Tensor, Tensor, Tensor, Tensor>(const Tensor&, const Tensor&, const Tensor&, const Tensor&,
                                                         const Tensor&, const Tensor&, const Tensor&, const Tensor&,
                                                         const Tensor&, const Tensor&, const Tensor&, int64_t);
  using DirF = Tensor(const Tensor&, const Tensor&, const Tensor&, const Tensor&, int64_t);
  using DirB = std::tuple<Tensor, Tensor, Tensor, Tensor>(const Tensor&, const Tensor&, const Tensor&, const Tensor&,
                                                          const Tensor&, const Tensor&, const Tensor&, const Tensor&,
                                                          const Tensor&, const Tensor&, const Tensor&, const Tensor&,
                                                          int64_t);
  using Prep = std::tuple<Tensor, Tensor>(const Tensor&, const Tensor&, int64_t);

  static variable_list forward(AutogradContext* ctx, Tensor G, Tensor x, Tensor h, Tensor n, Tensor bk1, Tensor bk6,
                               Tensor S, Tensor P, Tensor dst_ptr, Tensor src_ptr, Tensor src_perm, Tensor edge_dst,
                               Tensor node_order, Tensor w_last, Tensor b_last, int64_t precision, bool want_W) {
    at::AutoDispatchBelowADInplaceOrView guard;
    static auto bwd = op_handle<Bwd>("fsctep::sparse_conv_backward");
    auto [dx, dh, dn, dS] = bwd.call(G, h, n, bk6, S, P, dst_ptr, src_ptr, src_perm, edge_dst, node_order, precision);
    Tensor dL, db;
    if (want_W) {
      std::tie(dL, db) = sparse_weight_grad(dS, x, x.size(2));
    } else {
      dL = at::zeros({0}, G.options());
      db = at::zeros({0}, G.options());
    }
    ctx->save_for_backward({G, x, h, n, bk1, bk6, S, P, dst_ptr, src_ptr, src_perm, edge_dst, node_order, w_last,
                            b_last});
    ctx->saved_data["precision"] = precision;
    ctx->saved_data["want_W"] = want_W;
    if (!want_W) ctx->mark_non_differentiable({dL, db});
    ctx->set_materialize_grads(false);
    return {dx, dh, dn, dL, db};
  }

  static variable_list backward(AutogradContext* ctx, variable_list u) {
    TORCH_CHECK(!torch::autograd::GradMode::is_enabled(),
                "third derivatives of the sparse conv are not implemented (create_graph in its double backward)");
    static auto fwd = op_handle<Fwd>("fsctep::sparse_conv");
    static auto bwd = op_handle<Bwd>("fsctep::sparse_conv_backward");
    static auto dirf = op_handle<DirF>("fsctep::sparse_conv_direction");
    static auto dirb = op_handle<DirB>("fsctep::sparse_conv_direction_backward");
    static auto prep = op_handle<Prep>("fsctep::sparse_prepare_weights");
    auto s = ctx->get_saved_variables();
    const Tensor &G = s[0], &x = s[1], &h = s[2], &n = s[3], &bk1 = s[4], &bk6 = s[5], &S = s[6], &P = s[7];
    const Tensor &dp = s[8], &sp = s[9], &pm = s[10], &ed = s[11], &ord = s[12], &wl = s[13], &bl = s[14];
    const int64_t prec = ctx->saved_data["precision"].toInt();
    const bool want_W = ctx->saved_data["want_W"].toBool();
    const int64_t C = x.size(2);
    const Tensor ux = u[0], uh = u[1], un = u[2];
    const Tensor uL = (want_W && u[3].defined()) ? u[3] : Tensor(), ub = (want_W && u[4].defined()) ? u[4] : Tensor();
    refuse_param_grad(ctx, {4, 5, 6, 7}, "the sparse conv (prepared weights, workspaces)");
    const bool nG = ctx->needs_input_grad(0), nx = ctx->needs_input_grad(1), nh = ctx->needs_input_grad(2),
               nn = ctx->needs_input_grad(3), nL = ctx->needs_input_grad(13), nb = ctx->needs_input_grad(14);
    auto acc = [](Tensor& a, const Tensor& b) { a = a.defined() ? a + b : b; };
    auto F = [&](const Tensor& xa, const Tensor& ha, const Tensor& k1, const Tensor& k6) {
      return fwd.call(xa, ha, n, k1, k6, dp, sp, pm, ed, ord, prec, std::nullopt, std::nullopt);
    };
    auto B = [&](const Tensor& ha, const Tensor& k6, const Tensor& Sa, const Tensor& Pa) {
      return bwd.call(G, ha, n, k6, Sa, Pa, dp, sp, pm, ed, ord, prec);
    };
    Tensor dG, dx, dh, dn, dL, db;
    if (ux.defined() && (nG || nh || nn || nL || nb)) {            // x -> ux
      auto [o, S1, P1] = F(ux, h, bk1, bk6);
      if (nG) acc(dG, o);
      if (nh || nn || nL || nb) {
        auto [bx, bh, bn, bS] = B(h, bk6, S1, P1);
        if (nh) acc(dh, bh);
        if (nn) acc(dn, bn);
        if (nL || nb) {
          auto [gl, gb] = sparse_weight_grad(bS, ux, C);
          if (nL) acc(dL, gl);
          if (nb) acc(db, gb);
        }
      }
    }
    if (uh.defined() && (nG || nx || nn || nL)) {                   // h -> uh, bias dropped
      TORCH_CHECK(wl.numel() > 0 && bl.numel() > 0,
                  "the double backward of the sparse conv through h needs w_last and b_last passed to the op");
      auto [k1, k6] = prep.call(wl.detach(), at::zeros_like(bl), C);
      auto [o, S2, P2] = F(x, uh, k1, k6);
      if (nG) acc(dG, o);
      if (nx || nn || nL) {
        auto [bx, bh, bn, bS] = B(uh, k6, S2, P2);
        if (nx) acc(dx, bx);
        if (nn) acc(dn, bn);
        if (nL) acc(dL, std::get<0>(sparse_weight_grad(bS, x, C)));
      }
    }
    if (un.defined()) {                                              // n -> un
      if (nG) acc(dG, dirf.call(P, n, un, dp, C));
      if (nx || nh || nn || nL || nb) {
        auto [bx, bh, bn, bS] = dirb.call(G, h, n, un, bk6, S, P, dp, sp, pm, ed, ord, prec);
        if (nx) acc(dx, bx);
        if (nh) acc(dh, bh);
        if (nn) acc(dn, bn);
        if (nL || nb) {
          auto [gl, gb] = sparse_weight_grad(bS, x, C);
          if (nL) acc(dL, gl);
          if (nb) acc(db, gb);
        }
      }
    }
    if ((uL.defined() || ub.defined()) && (nG || nx || nh || nn)) {  // W -> uW
      auto [k1, k6] = prep.call(uL.defined() ? uL : at::zeros_like(wl), ub.defined() ? ub : at::zeros_like(bl), C);
      auto [o, S4, P4] = F(x, h, k1, k6);
      if (nG) acc(dG, o);
      if (nx || nh || nn) {
        auto [bx, bh, bn, bS] = B(h, k6, S4, P4);
        if (nx) acc(dx, bx);
        if (nh) acc(dh, bh);
        if (nn) acc(dn, bn);
      }
    }
    variable_list res(17);
    res[0] = dG;
    res[1] = dx;
    res[2] = dh;
    res[3] = dn;
    if (dL.defined()) res[13] = dL.view(wl.sizes());
    if (db.defined()) res[14] = db.view(bl.sizes());
    return res;
  }
};

struct SparseConvFn : public torch::autograd::Function<SparseConvFn> {
  static variable_list forward(AutogradContext* ctx, Tensor x, Tensor h, Tensor n, Tensor bk1, Tensor bk6,
                               Tensor dst_ptr, Tensor src_ptr, Tensor src_perm, Tensor edge_dst, Tensor node_order,
                               Tensor w_last, Tensor b_last, int64_t precision) {
    at::AutoDispatchBelowADInplaceOrView guard;
    static auto op = op_handle<SparseConvBwdFn::Fwd>("fsctep::sparse_conv");
    auto [out, S, P] = op.call(x, h, n, bk1, bk6, dst_ptr, src_ptr, src_perm, edge_dst, node_order, precision,
                               std::nullopt, std::nullopt);
    ctx->save_for_backward({x, h, n, bk1, bk6, S, P, dst_ptr, src_ptr, src_perm, edge_dst, node_order, w_last,
                            b_last});
    ctx->saved_data["precision"] = precision;
    ctx->mark_non_differentiable({S, P});
    ctx->set_materialize_grads(false);   // S and P are saved workspaces: no zero-filled gradients for them
    return {out, S, P};
  }
  static variable_list backward(AutogradContext* ctx, variable_list grads) {
    variable_list res(13);
    if (!grads[0].defined()) return res;
    refuse_param_grad(ctx, {3, 4}, "the sparse conv (prepared weights; pass w_last and b_last for their gradient)");
    auto s = ctx->get_saved_variables();
    // gradient slots follow the forward's arguments; needs_input_grad counts its tensor arguments
    // (w_last and b_last are tensor arguments 10 and 11)
    const bool want_W = ctx->needs_input_grad(10) || ctx->needs_input_grad(11);
    auto r = SparseConvBwdFn::apply(grads[0], s[0], s[1], s[2], s[3], s[4], s[5], s[6], s[7], s[8], s[9], s[10],
                                    s[11], s[12], s[13], ctx->saved_data["precision"].toInt(), want_W);
    res[0] = r[0];
    res[1] = r[1];
    res[2] = r[2];
    if (want_W) {
      if (ctx->needs_input_grad(10)) res[10] = r[3].view(s[12].sizes());
      if (ctx->needs_input_grad(11)) res[11] = r[4].view(s[13].sizes());
    }
    return res;
  }
};

std::tuple<Tensor, Tensor, Tensor> sparse_conv_autograd(const Tensor& x, const Tensor& h, const Tensor& n,
                                                        const Tensor& bk1, const Tensor& bk6, const Tensor& dst_ptr,
                                                        const Tensor& src_ptr, const Tensor& src_perm,
                                                        const Tensor& edge_dst, const Tensor& node_order,
                                                        int64_t precision, const std::optional<Tensor>& w_last,
                                                        const std::optional<Tensor>& b_last) {
  // absent weights travel as empty tensors (autograd inputs must be defined)
  const Tensor none = at::empty({0}, x.options());
  auto r = SparseConvFn::apply(x, h, n, bk1, bk6, dst_ptr, src_ptr, src_perm, edge_dst, node_order,
                               w_last.has_value() ? *w_last : none, b_last.has_value() ? *b_last : none, precision);
  return {r[0], r[1], r[2]};
}

struct SparseConv1Fn : public torch::autograd::Function<SparseConv1Fn> {
  static variable_list forward(AutogradContext* ctx, Tensor h, Tensor n, Tensor mf_, Tensor mb, Tensor dst_ptr,
                               Tensor pair_tiles, int64_t channels) {
    at::AutoDispatchBelowADInplaceOrView guard;
    static auto op = op_handle<std::tuple<Tensor, Tensor>(const Tensor&, const Tensor&, const Tensor&, const Tensor&,
                                                          const Tensor&, const Tensor&, int64_t)>(
        "fsctep::sparse_conv1");
    auto [out, Q] = op.call(h, n, mf_, mb, dst_ptr, pair_tiles, channels);
    ctx->save_for_backward({n, mf_, Q, dst_ptr, pair_tiles});
    ctx->mark_non_differentiable({Q});
    ctx->set_materialize_grads(false);
    return {out, Q};
  }
  static variable_list backward(AutogradContext* ctx, variable_list grads) {
    variable_list res(7);
    if (!grads[0].defined()) return res;
    refuse_param_grad(ctx, {2, 3}, "the sparse conv1");
    auto s = ctx->get_saved_variables();
    static auto op = op_handle<std::tuple<Tensor, Tensor>(const Tensor&, const Tensor&, const Tensor&, const Tensor&,
                                                          const Tensor&, const Tensor&)>("fsctep::sparse_conv1_backward");
    auto [dh, dn] = op.call(grads[0], s[0], s[1], s[2], s[3], s[4]);
    res[0] = dh;
    res[1] = dn;
    return res;
  }
};

std::tuple<Tensor, Tensor> sparse_conv1_autograd(const Tensor& h, const Tensor& n, const Tensor& mf_, const Tensor& mb,
                                                 const Tensor& dst_ptr, const Tensor& pair_tiles, int64_t channels) {
  auto r = SparseConv1Fn::apply(h, n, mf_, mb, dst_ptr, pair_tiles, channels);
  return {r[0], r[1]};
}

// Backward of the ICTD conv as a function of (G, x, Y, gates, W): (dx, dgates, dY, dW), itself differentiable
// once, which gives the double backward of force training (training/trainer.py:1292-1297; the reference's
// project_dbl_bwd_grad_* / mix_dbl_bwd_grad_* kernels, csrc/ictd_tp_cuda.cu:536-971).  The conv
// out = F(x, Y, gates, W) is linear in x, in W and in each of Y and gates, so its backward B(G) = grad <G, F>
// has, for cotangents u = (ux, ug, uY, uW) of (dx, dgates, dY, dW),
//   d<u, B>/dG = F(ux, Y, g, W) + F(x, uY, g, W) + F(x, Y, ug, W) + F(x, Y, g, uW)
//   d<u, B>/dx = B_x(G; x, uY, g, W) + B_x(G; x, Y, ug, W) + B_x(G; x, Y, g, uW)
//   d<u, B>/dY = B_Y(G; ux, Y, g, W) + B_Y(G; x, Y, ug, W) + B_Y(G; x, Y, g, uW)
//   d<u, B>/dg = B_g(G; ux, Y, g, W) + B_g(G; x, uY, g, W) + B_g(G; x, Y, g, uW)
//   d<u, B>/dW = B_W(G; ux, Y, g) + B_W(G; x, uY, g) + B_W(G; x, Y, ug)
// (B_v: the v part of B with the named argument replaced), all evaluated with the same kernels.
struct IctdConvBwdFn : public torch::autograd::Function<IctdConvBwdFn> {
  using Conv = Tensor(const Tensor&, const Tensor&, const Tensor&, const Tensor&, const Tensor&, const Tensor&,
                      const Tensor&, const Tensor&, const Tensor&, const Tensor&, const Tensor&, const Tensor&,
                      at::IntArrayRef);
  using Bwd = std::tuple<Tensor, Tensor, Tensor>(const Tensor&, const Tensor&, const Tensor&, const Tensor&,
                                                 const Tensor&, const Tensor&, const Tensor&, const Tensor&,
                                                 const Tensor&, const Tensor&, const Tensor&, const Tensor&,
                                                 at::IntArrayRef);
  using Proj = Tensor(const Tensor&, const Tensor&, const Tensor&, const Tensor&, const Tensor&, const Tensor&,
                      const Tensor&, at::IntArrayRef);

  static variable_list forward(AutogradContext* ctx, Tensor G, Tensor x, Tensor Y, Tensor gates, Tensor W, Tensor Wt,
                               Tensor cg, Tensor dst_ptr, Tensor edge_src, Tensor src_ptr, Tensor src_perm,
                               Tensor edge_dst, Tensor node_order, std::vector<int64_t> layout, bool want_dW) {
    at::AutoDispatchBelowADInplaceOrView guard;
    static auto bwd = op_handle<Bwd>("fsctep::ictd_conv_backward");
    static auto proj = op_handle<Proj>("fsctep::ictd_project");
    auto [dx, dgates, dY] = bwd.call(G, x, Y, gates, Wt, cg, dst_ptr, edge_src, src_ptr, src_perm, edge_dst,
                                     node_order, layout);
    Tensor dW;
    if (want_dW) {
      const FscIctdLayout L = unpack_table<FscIctdLayout>(layout, "layout");
      const Tensor Z = proj.call(x, Y, gates, cg, dst_ptr, edge_src, node_order, layout);
      dW = ictd_weight_grad(f32c(G), Z, L, W.sizes());
    } else {
      dW = at::zeros({0}, G.options());
    }
    ctx->save_for_backward({G, x, Y, gates, W, Wt, cg, dst_ptr, edge_src, src_ptr, src_perm, edge_dst, node_order});
    ctx->saved_data["layout"] = layout;
    ctx->saved_data["want_dW"] = want_dW;
    ctx->mark_non_differentiable(want_dW ? variable_list{} : variable_list{dW});
    ctx->set_materialize_grads(false);
    return {dx, dgates, dY, dW};
  }

  static variable_list backward(AutogradContext* ctx, variable_list u) {
    TORCH_CHECK(!torch::autograd::GradMode::is_enabled(),
                "third derivatives of the ICTD conv are not implemented (create_graph in its double backward)");
    static auto conv = op_handle<Conv>("fsctep::ictd_conv");
    static auto bwd = op_handle<Bwd>("fsctep::ictd_conv_backward");
    static auto proj = op_handle<Proj>("fsctep::ictd_project");
    static auto prep = op_handle<Tensor(const Tensor&)>("fsctep::ictd_prepare_weights");
    auto s = ctx->get_saved_variables();
    const Tensor &G = s[0], &x = s[1], &Y = s[2], &g = s[3], &W = s[4], &Wt = s[5], &cg = s[6];
    const Tensor &dst_ptr = s[7], &esrc = s[8], &src_ptr = s[9], &src_perm = s[10], &edst = s[11], &order = s[12];
    const std::vector<int64_t> layout = ctx->saved_data["layout"].toIntVector();
    const bool want_dW = ctx->saved_data["want_dW"].toBool();
    const Tensor ux = u[0], ug = u[1], uY = u[2];
    const Tensor uW = (want_dW && u.size() > 3 && u[3].defined()) ? u[3] : Tensor();
    refuse_param_grad(ctx, {5, 6}, "the ICTD conv (prepared weights, coupling table)");
    variable_list res(15);
    const bool nG = ctx->needs_input_grad(0), nx = ctx->needs_input_grad(1), nY = ctx->needs_input_grad(2),
               ng = ctx->needs_input_grad(3), nW = ctx->needs_input_grad(4);
    auto acc = [](Tensor& a, const Tensor& b) { a = a.defined() ? a + b : b; };
    auto F = [&](const Tensor& xa, const Tensor& Ya, const Tensor& ga, const Tensor& Wta) {
      return conv.call(xa, Ya, ga, W, Wta, cg, dst_ptr, esrc, src_ptr, src_perm, edst, order, layout);
    };
    auto B = [&](const Tensor& xa, const Tensor& Ya, const Tensor& ga, const Tensor& Wta) {
      return bwd.call(G, xa, Ya, ga, Wta, cg, dst_ptr, esrc, src_ptr, src_perm, edst, order, layout);
    };
    auto P = [&](const Tensor& xa, const Tensor& Ya, const Tensor& ga) {
      return proj.call(xa, Ya, ga, cg, dst_ptr, esrc, order, layout);
    };
    Tensor dG, dx, dY, dg, Zs;
    const Tensor Wtu = uW.defined() ? prep.call(uW) : Tensor();
    if (nG) {
      if (ux.defined()) acc(dG, F(ux, Y, g, Wt));
      if (uY.defined()) acc(dG, F(x, uY, g, Wt));
      if (ug.defined()) acc(dG, F(x, Y, ug, Wt));
      if (uW.defined()) acc(dG, F(x, Y, g, Wtu));
    }
    if (ux.defined() && (nY || ng)) {
      auto [bx, bg, bY] = B(ux, Y, g, Wt);
      if (nY) acc(dY, bY);
      if (ng) acc(dg, bg);
    }
    if (uY.defined() && (nx || ng)) {
      auto [bx, bg, bY] = B(x, uY, g, Wt);
      if (nx) acc(dx, bx);
      if (ng) acc(dg, bg);
    }
    if (ug.defined() && (nx || nY)) {
      auto [bx, bg, bY] = B(x, Y, ug, Wt);
      if (nx) acc(dx, bx);
      if (nY) acc(dY, bY);
    }
    if (uW.defined() && (nx || nY || ng)) {
      auto [bx, bg, bY] = B(x, Y, g, Wtu);
      if (nx) acc(dx, bx);
      if (nY) acc(dY, bY);
      if (ng) acc(dg, bg);
    }
    if (nW) {
      if (ux.defined()) acc(Zs, P(ux, Y, g));
      if (uY.defined()) acc(Zs, P(x, uY, g));
      if (ug.defined()) acc(Zs, P(x, Y, ug));
      if (Zs.defined())
        res[4] = ictd_weight_grad(f32c(G), Zs, unpack_table<FscIctdLayout>(layout, "layout"), W.sizes());
    }
    res[0] = dG;
    res[1] = dx;
    res[2] = dY;
    res[3] = dg;
    return res;
  }
};

struct IctdConvFn : public torch::autograd::Function<IctdConvFn> {
  static variable_list forward(AutogradContext* ctx, Tensor x, Tensor Y, Tensor gates, Tensor W, Tensor Wt, Tensor cg,
                               Tensor dst_ptr, Tensor edge_src, Tensor src_ptr, Tensor src_perm, Tensor edge_dst,
                               Tensor node_order, std::vector<int64_t> layout) {
    at::AutoDispatchBelowADInplaceOrView guard;
    static auto op = op_handle<IctdConvBwdFn::Conv>("fsctep::ictd_conv");
    Tensor out = op.call(x, Y, gates, W, Wt, cg, dst_ptr, edge_src, src_ptr, src_perm, edge_dst, node_order, layout);
    ctx->save_for_backward({x, Y, gates, W, Wt, cg, dst_ptr, edge_src, src_ptr, src_perm, edge_dst, node_order});
    ctx->saved_data["layout"] = layout;
    return {out};
  }
  static variable_list backward(AutogradContext* ctx, variable_list grads) {
    variable_list res(13);
    if (!grads[0].defined()) return res;
    refuse_param_grad(ctx, {4, 5}, "the ICTD conv (prepared weights, coupling table)");
    auto s = ctx->get_saved_variables();
    const std::vector<int64_t> layout = ctx->saved_data["layout"].toIntVector();
    const bool want_dW = ctx->needs_input_grad(3);
    auto r = IctdConvBwdFn::apply(grads[0], s[0], s[1], s[2], s[3], s[4], s[5], s[6], s[7], s[8], s[9], s[10], s[11],
                                  layout, want_dW);
    res[0] = r[0];
    res[1] = r[2];
    res[2] = r[1];
    if (want_dW) res[3] = r[3];
    return res;
  }
};

Tensor ictd_conv_autograd(const Tensor& x, const Tensor& Y, const Tensor& gates, const Tensor& W, const Tensor& Wt,
                          const Tensor& cg, const Tensor& dst_ptr, const Tensor& edge_src, const Tensor& src_ptr,
                          const Tensor& src_perm, const Tensor& edge_dst, const Tensor& node_order,
                          at::IntArrayRef layout) {
  return IctdConvFn::apply(x, Y, gates, W, Wt, cg, dst_ptr, edge_src, src_ptr, src_perm, edge_dst, node_order,
                           layout.vec())[0];
}

struct IctdConv1Fn : public torch::autograd::Function<IctdConv1Fn> {
  static variable_list forward(AutogradContext* ctx, Tensor F, Tensor gates, Tensor qtab, Tensor dst_ptr,
                               Tensor edge_pair, Tensor node_species, int64_t n_species, int64_t n_comps,
                               std::vector<int64_t> layout) {
    at::AutoDispatchBelowADInplaceOrView guard;
    static auto op = op_handle<Tensor(const Tensor&, const Tensor&, const Tensor&, const Tensor&, const Tensor&,
                                      const Tensor&, int64_t, int64_t, at::IntArrayRef)>("fsctep::ictd_conv1");
    Tensor out = op.call(F, gates, qtab, dst_ptr, edge_pair, node_species, n_species, n_comps, layout);
    ctx->save_for_backward({F, gates, qtab, dst_ptr, edge_pair, node_species});
    ctx->saved_data["n_species"] = n_species;
    ctx->saved_data["layout"] = layout;
    return {out};
  }
  static variable_list backward(AutogradContext* ctx, variable_list grads) {
    variable_list res(9);
    if (!grads[0].defined()) return res;
    refuse_param_grad(ctx, {2}, "the ICTD conv1");
    auto s = ctx->get_saved_variables();
    static auto op = op_handle<std::tuple<Tensor, Tensor>(const Tensor&, const Tensor&, const Tensor&, const Tensor&,
                                                          const Tensor&, const Tensor&, const Tensor&, int64_t,
                                                          at::IntArrayRef)>("fsctep::ictd_conv1_backward");
    const std::vector<int64_t> layout = ctx->saved_data["layout"].toIntVector();
    auto [dF, dgates] = op.call(grads[0], s[0], s[1], s[2], s[3], s[4], s[5], ctx->saved_data["n_species"].toInt(),
                                layout);
    res[0] = dF;
    res[1] = dgates;
    return res;
  }
};

Tensor ictd_conv1_autograd(const Tensor& F, const Tensor& gates, const Tensor& qtab, const Tensor& dst_ptr,
                           const Tensor& edge_pair, const Tensor& node_species, int64_t n_species, int64_t n_comps,
                           at::IntArrayRef layout) {
  return IctdConv1Fn::apply(F, gates, qtab, dst_ptr, edge_pair, node_species, n_species, n_comps, layout.vec())[0];
}

struct GramFn : public torch::autograd::Function<GramFn> {
  static variable_list forward(AutogradContext* ctx, Tensor t, Tensor Wf, Tensor Wb, double scale) {
    at::AutoDispatchBelowADInplaceOrView guard;
    static auto op = op_handle<Tensor(const Tensor&, const Tensor&, const Tensor&, double)>("fsctep::gram_bilinear");
    Tensor out = op.call(t, Wf, Wb, scale);
    ctx->save_for_backward({t, Wb});
    ctx->saved_data["scale"] = scale;
    return {out};
  }
  static variable_list backward(AutogradContext* ctx, variable_list grads) {
    variable_list res(4);
    if (!grads[0].defined()) return res;
    refuse_param_grad(ctx, {1, 2}, "the readout Gram bilinear");
    auto s = ctx->get_saved_variables();
    static auto op =
        op_handle<Tensor(const Tensor&, const Tensor&, const Tensor&, double)>("fsctep::gram_bilinear_backward");
    res[0] = op.call(grads[0], s[0], s[1], ctx->saved_data["scale"].toDouble());
    return res;
  }
};

Tensor gram_bilinear_autograd(const Tensor& t, const Tensor& Wf, const Tensor& Wb, double scale) {
  return GramFn::apply(t, Wf, Wb, scale)[0];
}

// Energy head: input gradient only (the forward is recomputed by the backward kernel, nothing saved but x).
struct ReadoutMlpFn : public torch::autograd::Function<ReadoutMlpFn> {
  static variable_list forward(AutogradContext* ctx, Tensor x, Tensor w, std::vector<int64_t> dims,
                               std::vector<double> eps) {
    at::AutoDispatchBelowADInplaceOrView guard;
    static auto op = op_handle<Tensor(const Tensor&, const Tensor&, at::IntArrayRef, at::ArrayRef<double>)>(
        "fsctep::readout_mlp");
    Tensor e = op.call(x, w, dims, eps);
    ctx->save_for_backward({x, w});
    ctx->saved_data["dims"] = dims;
    ctx->saved_data["eps"] = eps;
    return {e};
  }
  static variable_list backward(AutogradContext* ctx, variable_list grads) {
    variable_list res(4);
    if (!grads[0].defined()) return res;
    refuse_param_grad(ctx, {1}, "the readout MLP (folded weights)");
    auto s = ctx->get_saved_variables();
    static auto op = op_handle<Tensor(const Tensor&, const Tensor&, const Tensor&, at::IntArrayRef,
                                      at::ArrayRef<double>)>("fsctep::readout_mlp_backward");
    const std::vector<int64_t> dims = ctx->saved_data["dims"].toIntVector();
    const std::vector<double> eps = ctx->saved_data["eps"].toDoubleVector();
    res[0] = op.call(grads[0], s[0], s[1], dims, eps);
    return res;
  }
};

Tensor readout_mlp_autograd(const Tensor& x, const Tensor& w, at::IntArrayRef dims, at::ArrayRef<double> eps) {
  return ReadoutMlpFn::apply(x, w, dims.vec(), eps.vec())[0];
}

// Readout features: the gradient w.r.t. the layers is one scatter kernel fed by the per-key Gram
// backward and the squared-norm gradient (no per-slice zero fills or accumulations).
struct ReadoutFn : public torch::autograd::Function<ReadoutFn> {
  static variable_list forward(AutogradContext* ctx, at::TensorList layers, at::TensorList Wf, at::TensorList Wb,
                               std::vector<double> scales, Tensor srcmap, Tensor gmap, std::vector<int64_t> table) {
    at::AutoDispatchBelowADInplaceOrView guard;
    static auto gather =
        op_handle<std::tuple<Tensor, Tensor>(at::TensorList, const Tensor&, at::IntArrayRef)>("fsctep::readout_gather");
    static auto gram = op_handle<Tensor(const Tensor&, const Tensor&, const Tensor&, double)>("fsctep::gram_bilinear");
    static auto gather_blk = op_handle<std::tuple<Tensor, Tensor>(at::TensorList, const Tensor&, at::IntArrayRef)>(
        "fsctep::readout_gather_blocked");
    static auto gram_blk =
        op_handle<Tensor(const Tensor&, const Tensor&, const Tensor&, double)>("fsctep::gram_bilinear_blocked");
    const FscReadoutTable Tv = unpack_table<FscReadoutTable>(table, "readout table");
  const FscReadoutTable* T = &Tv;
    TORCH_CHECK((int64_t)Wf.size() == T->n_keys && (int64_t)Wb.size() == T->n_keys &&
                    (int64_t)scales.size() == T->n_keys,
                "one prepared Gram weight pair and scale per key");
    // through the dispatcher, so that tracers (make_fx, TorchScript) record the calls
    const bool blocked = readout_blocked(T);
    Tensor scalars, sq, t_all;
    std::tie(t_all, sq) = blocked ? gather_blk.call(layers, srcmap, table) : gather.call(layers, srcmap, table);
    const int64_t N = layers[0].size(0);
    for (int k = 0; k < T->n_keys; ++k) {
      const Tensor tk = gram_input(t_all, T, N, k);
      Tensor o = blocked ? gram_blk.call(tk, Wf[k], Wb[k], scales[k]) : gram.call(tk, Wf[k], Wb[k], scales[k]);
      scalars = scalars.defined() ? scalars.add_(o) : o;
    }
    variable_list keep(layers.begin(), layers.end());
    keep.push_back(t_all);
    for (const Tensor& w : Wb) keep.push_back(w);
    keep.push_back(gmap);
    ctx->save_for_backward(keep);
    ctx->saved_data["table"] = table;
    ctx->saved_data["n_layers"] = (int64_t)layers.size();
    ctx->saved_data["blocked"] = blocked;
    ctx->saved_data["scales"] = c10::IValue(c10::ArrayRef<double>(scales));
    ctx->set_materialize_grads(false);   // an unused output skips its part of the backward
    return {scalars, sq};
  }
  static variable_list backward(AutogradContext* ctx, variable_list grads) {
    auto s = ctx->get_saved_variables();
    const int64_t nL = ctx->saved_data["n_layers"].toInt();
    const std::vector<double> scales = ctx->saved_data["scales"].toDoubleVector();
    const int64_t nK = (int64_t)scales.size();
    variable_list res(nL + 2 * nK + 4);
    if (!grads[0].defined() && !grads[1].defined()) return res;
    for (int64_t i = nL; i < nL + 2 * nK; ++i)
      TORCH_CHECK(!ctx->needs_input_grad(i), "parameter gradients of the readout Gram bilinear are not implemented "
                                             "(energy/force inference only)");
    static auto gram_bwd =
        op_handle<Tensor(const Tensor&, const Tensor&, const Tensor&, double)>("fsctep::gram_bilinear_backward");
    static auto gram_bwd_blk = op_handle<Tensor(const Tensor&, const Tensor&, const Tensor&, double)>(
        "fsctep::gram_bilinear_backward_blocked");
    static auto scatter = op_handle<std::vector<Tensor>(const c10::List<std::optional<Tensor>>&,
                                                        const std::optional<Tensor>&, at::TensorList, const Tensor&,
                                                        at::IntArrayRef)>("fsctep::readout_scatter");
    std::vector<Tensor> layers(s.begin(), s.begin() + nL);
    const Tensor& t_all = s[nL];
    const Tensor& gmap = s[nL + 1 + nK];
    const std::vector<int64_t> table = ctx->saved_data["table"].toIntVector();
    const FscReadoutTable Tv = unpack_table<FscReadoutTable>(table, "readout table");
  const FscReadoutTable* T = &Tv;
    const int64_t N = layers[0].size(0);
    const bool blocked = ctx->saved_data["blocked"].toBool();
    c10::List<std::optional<Tensor>> dt;
    for (int k = 0; k < nK; ++k) {
      if (!grads[0].defined())
        dt.push_back(std::nullopt);
      else if (blocked)
        dt.push_back(gram_bwd_blk.call(grads[0], gram_input(t_all, T, N, k), s[nL + 1 + k], scales[k]));
      else
        dt.push_back(gram_bwd.call(grads[0], gram_input(t_all, T, N, k), s[nL + 1 + k], scales[k]));
    }
    std::optional<Tensor> dsq;
    if (grads[1].defined()) dsq = grads[1];
    std::vector<Tensor> dX = scatter.call(dt, dsq, layers, gmap, table);
    for (int64_t l = 0; l < nL; ++l) res[l] = dX[l];
    return res;
  }
};

std::tuple<Tensor, Tensor> readout_features_autograd(at::TensorList layers, at::TensorList Wf, at::TensorList Wb,
                                                     at::ArrayRef<double> scales, const Tensor& srcmap,
                                                     const Tensor& gmap, at::IntArrayRef table) {
  auto out = ReadoutFn::apply(layers, Wf, Wb, scales.vec(), srcmap, gmap, table.vec());
  return {out[0], out[1]};
}

struct EdgeGeometryFn : public torch::autograd::Function<EdgeGeometryFn> {
  static variable_list forward(AutogradContext* ctx, Tensor pos, Tensor shift, Tensor edge_src, Tensor edge_dst,
                               Tensor dst_ptr, Tensor src_ptr, Tensor src_perm) {
    at::AutoDispatchBelowADInplaceOrView guard;
    static auto op = op_handle<std::tuple<Tensor, Tensor>(const Tensor&, const Tensor&, const Tensor&, const Tensor&,
                                                          const Tensor&, const Tensor&, const Tensor&)>(
        "fsctep::edge_geometry");
    auto [n, r] = op.call(pos, shift, edge_src, edge_dst, dst_ptr, src_ptr, src_perm);
    ctx->save_for_backward({n, r, dst_ptr, src_ptr, src_perm});
    ctx->set_materialize_grads(false);
    return {n, r};
  }
  static variable_list backward(AutogradContext* ctx, variable_list grads) {
    variable_list res(7);
    if (!grads[0].defined() && !grads[1].defined()) return res;
    TORCH_CHECK(!ctx->needs_input_grad(1), "gradients w.r.t. the periodic shift vectors (stress) are not implemented");
    auto s = ctx->get_saved_variables();
    static auto op = op_handle<Tensor(const std::optional<Tensor>&, const std::optional<Tensor>&, const Tensor&,
                                      const Tensor&, const Tensor&, const Tensor&, const Tensor&)>(
        "fsctep::edge_geometry_backward");
    const std::optional<Tensor> gn = grads[0].defined() ? std::optional<Tensor>(grads[0]) : std::nullopt;
    const std::optional<Tensor> gr = grads[1].defined() ? std::optional<Tensor>(grads[1]) : std::nullopt;
    res[0] = op.call(gn, gr, s[0], s[1], s[2], s[3], s[4]);
    return res;
  }
};

std::tuple<Tensor, Tensor> edge_geometry_autograd(const Tensor& pos, const Tensor& shift, const Tensor& edge_src,
                                                  const Tensor& edge_dst, const Tensor& dst_ptr, const Tensor& src_ptr,
                                                  const Tensor& src_perm) {
  auto r = EdgeGeometryFn::apply(pos, shift, edge_src, edge_dst, dst_ptr, src_ptr, src_perm);
  return {r[0], r[1]};
}


struct EdgeVecGeometryFn : public torch::autograd::Function<EdgeVecGeometryFn> {
  static variable_list forward(AutogradContext* ctx, Tensor edge_vec, Tensor order) {
    at::AutoDispatchBelowADInplaceOrView guard;
    static auto op = op_handle<std::tuple<Tensor, Tensor>(const Tensor&, const Tensor&)>("fsctep::edge_vec_geometry");
    auto [n, r] = op.call(edge_vec, order);
    ctx->save_for_backward({n, r, order});
    ctx->set_materialize_grads(false);
    return {n, r};
  }
  static variable_list backward(AutogradContext* ctx, variable_list grads) {
    variable_list res(2);
    if (!grads[0].defined() && !grads[1].defined()) return res;
    auto s = ctx->get_saved_variables();
    static auto op = op_handle<Tensor(const std::optional<Tensor>&, const std::optional<Tensor>&, const Tensor&,
                                      const Tensor&, const Tensor&)>("fsctep::edge_vec_geometry_backward");
    const std::optional<Tensor> gn = grads[0].defined() ? std::optional<Tensor>(grads[0]) : std::nullopt;
    const std::optional<Tensor> gr = grads[1].defined() ? std::optional<Tensor>(grads[1]) : std::nullopt;
    res[0] = op.call(gn, gr, s[0], s[1], s[2]);
    return res;
  }
};

std::tuple<Tensor, Tensor> edge_vec_geometry_autograd(const Tensor& edge_vec, const Tensor& order) {
  auto r = EdgeVecGeometryFn::apply(edge_vec, order);
  return {r[0], r[1]};
}

struct RadialMlpFn : public torch::autograd::Function<RadialMlpFn> {
  static variable_list forward(AutogradContext* ctx, Tensor r, Tensor w0, Tensor b0, Tensor w2, Tensor b2,
                               std::optional<Tensor> w4, std::optional<Tensor> b4, double r_cut, int64_t basis) {
    at::AutoDispatchBelowADInplaceOrView guard;
    static auto op = op_handle<Tensor(const Tensor&, const Tensor&, const Tensor&, const Tensor&, const Tensor&,
                                      const std::optional<Tensor>&, const std::optional<Tensor>&, double, int64_t)>(
        "fsctep::radial_mlp");
    const bool fused = w4.has_value() && w4->defined();
    TORCH_CHECK(!fused || !at::GradMode::is_enabled() ||
                    !(w4->requires_grad() || (b4.has_value() && b4->defined() && b4->requires_grad())),
                "parameter gradients of the radial MLP are not implemented (energy/force inference only)");
    Tensor h = op.call(r, w0, b0, w2, b2, w4, b4, r_cut, basis);
    ctx->save_for_backward({r, w0, b0, w2, b2, fused ? *w4 : Tensor()});
    ctx->saved_data["r_cut"] = r_cut;
    ctx->saved_data["basis"] = basis;
    ctx->set_materialize_grads(false);
    return {h};
  }
  static variable_list backward(AutogradContext* ctx, variable_list grads) {
    variable_list res(9);
    if (!grads[0].defined()) return res;
    refuse_param_grad(ctx, {1, 2, 3, 4}, "the radial MLP");
    auto s = ctx->get_saved_variables();
    static auto op = op_handle<Tensor(const Tensor&, const Tensor&, const Tensor&, const Tensor&, const Tensor&,
                                      const Tensor&, const std::optional<Tensor>&, double, int64_t)>(
        "fsctep::radial_mlp_backward");
    const std::optional<Tensor> w4 = s[5].defined() ? std::optional<Tensor>(s[5]) : std::nullopt;
    res[0] = op.call(grads[0], s[0], s[1], s[2], s[3], s[4], w4, ctx->saved_data["r_cut"].toDouble(),
                     ctx->saved_data["basis"].toInt());
    return res;
  }
};

Tensor radial_mlp_autograd(const Tensor& r, const Tensor& w0, const Tensor& b0, const Tensor& w2, const Tensor& b2,
                           const std::optional<Tensor>& w4, const std::optional<Tensor>& b4, double r_cut,
                           int64_t basis) {
  return RadialMlpFn::apply(r, w0, b0, w2, b2, w4, b4, r_cut, basis)[0];
}

struct EdgeHarmonicsFn : public torch::autograd::Function<EdgeHarmonicsFn> {
  static variable_list forward(AutogradContext* ctx, Tensor n, std::vector<int64_t> table) {
    at::AutoDispatchBelowADInplaceOrView guard;
    static auto op = op_handle<Tensor(const Tensor&, at::IntArrayRef)>("fsctep::edge_harmonics");
    Tensor Y = op.call(n, table);
    ctx->save_for_backward({n});
    ctx->saved_data["table"] = table;
    ctx->set_materialize_grads(false);
    return {Y};
  }
  static variable_list backward(AutogradContext* ctx, variable_list grads) {
    variable_list res(2);
    if (!grads[0].defined()) return res;
    auto s = ctx->get_saved_variables();
    static auto op = op_handle<Tensor(const Tensor&, const Tensor&, at::IntArrayRef)>("fsctep::edge_harmonics_backward");
    res[0] = op.call(grads[0], s[0], ctx->saved_data["table"].toIntVector());
    return res;
  }
};

Tensor edge_harmonics_autograd(const Tensor& n, at::IntArrayRef table) {
  return EdgeHarmonicsFn::apply(n, table.vec())[0];
}

// CPU tensors: the HIP kernels are the only implementation, so say that instead of "no CPU kernel".
void refuse_cpu(const c10::OperatorHandle& op, torch::jit::Stack*) {
  TORCH_CHECK(false, op.schema().name(), ": fsctep ops run on the GPU only (HIP kernels); got CPU tensors");
}

}  // namespace

TORCH_LIBRARY(fsctep, m) {
  m.def("sparse_prepare_weights(Tensor w_last, Tensor b_last, int channels) -> (Tensor, Tensor)");
  m.def("sparse_conv(Tensor x, Tensor h, Tensor n, Tensor bk1, Tensor bk6, Tensor dst_ptr, Tensor src_ptr, "
        "Tensor src_perm, Tensor edge_dst, Tensor node_order, int precision=0, Tensor? w_last=None, "
        "Tensor? b_last=None) -> (Tensor, Tensor, Tensor)");
  m.def("sparse_conv_backward(Tensor grad_out, Tensor h, Tensor n, Tensor bk6, Tensor S, Tensor P, Tensor dst_ptr, "
        "Tensor src_ptr, Tensor src_perm, Tensor edge_dst, Tensor node_order, int precision=0) "
        "-> (Tensor, Tensor, Tensor, Tensor)");
  m.def("sparse_conv_direction(Tensor P, Tensor n, Tensor u, Tensor dst_ptr, int channels) -> Tensor");
  m.def("sparse_conv_direction_backward(Tensor grad_out, Tensor h, Tensor n, Tensor u, Tensor bk6, Tensor S, "
        "Tensor P, Tensor dst_ptr, Tensor src_ptr, Tensor src_perm, Tensor edge_dst, Tensor node_order, "
        "int precision=0) -> (Tensor, Tensor, Tensor, Tensor)");
  m.def("sparse_conv1_pair_table(Tensor w_last, Tensor b_last, Tensor atom_table, int channels) -> (Tensor, Tensor)");
  m.def("sparse_conv1(Tensor h, Tensor n, Tensor mf, Tensor mb, Tensor dst_ptr, Tensor pair_tiles, "
        "int channels) -> (Tensor, Tensor)");
  m.def("sparse_conv1_backward(Tensor grad_out, Tensor n, Tensor mf, Tensor Q, Tensor dst_ptr, Tensor pair_tiles) "
        "-> (Tensor, Tensor)");
  m.def("ictd_prepare_weights(Tensor W) -> Tensor");
  m.def("ictd_conv(Tensor x, Tensor Y, Tensor gates, Tensor W, Tensor Wt, Tensor cg, Tensor dst_ptr, "
        "Tensor edge_src, Tensor src_ptr, Tensor src_perm, Tensor edge_dst, Tensor node_order, int[] layout) -> Tensor");
  m.def("ictd_conv_backward(Tensor grad_out, Tensor x, Tensor Y, Tensor gates, Tensor Wt, Tensor cg, "
        "Tensor dst_ptr, Tensor edge_src, Tensor src_ptr, Tensor src_perm, Tensor edge_dst, Tensor node_order, "
        "int[] layout) -> (Tensor, Tensor, Tensor)");
  m.def("ictd_project(Tensor x, Tensor Y, Tensor gates, Tensor cg, Tensor dst_ptr, Tensor edge_src, "
        "Tensor node_order, int[] layout) -> Tensor");
  m.def("ictd_conv1(Tensor F, Tensor gates, Tensor qtab, Tensor dst_ptr, Tensor edge_pair, Tensor node_species, "
        "int n_species, int n_comps, int[] layout) -> Tensor");
  m.def("ictd_conv1_backward(Tensor grad_out, Tensor F, Tensor gates, Tensor qtab, Tensor dst_ptr, "
        "Tensor edge_pair, Tensor node_species, int n_species, int[] layout) -> (Tensor, Tensor)");
  m.def("gram_prepare_weights(Tensor W) -> (Tensor, Tensor)");
  m.def("gram_bilinear(Tensor t, Tensor Wf, Tensor Wb, float scale) -> Tensor");
  m.def("gram_bilinear_backward(Tensor grad_out, Tensor t, Tensor Wb, float scale) -> Tensor");
  m.def("gram_bilinear_blocked(Tensor t, Tensor Wf, Tensor Wb, float scale) -> Tensor");
  m.def("gram_bilinear_backward_blocked(Tensor grad_out, Tensor t, Tensor Wb, float scale) -> Tensor");
  m.def("readout_mlp_prepare(Tensor[] params, int[] dims, float[] eps) -> Tensor");
  m.def("readout_mlp(Tensor x, Tensor weights, int[] dims, float[] eps) -> Tensor");
  m.def("readout_mlp_backward(Tensor grad, Tensor x, Tensor weights, int[] dims, float[] eps) -> Tensor");
  m.def("edge_geometry(Tensor pos, Tensor shift, Tensor edge_src, Tensor edge_dst, Tensor dst_ptr, Tensor src_ptr, "
        "Tensor src_perm) -> (Tensor, Tensor)");
  m.def("edge_geometry_backward(Tensor? grad_n, Tensor? grad_r, Tensor n, Tensor r, Tensor dst_ptr, Tensor src_ptr, "
        "Tensor src_perm) -> Tensor");
  m.def("radial_mlp(Tensor r, Tensor w0, Tensor b0, Tensor w2, Tensor b2, Tensor? w4, Tensor? b4, float r_cut, "
        "int basis) -> Tensor");
  m.def("edge_harmonics(Tensor n, int[] table) -> Tensor");
  m.def("edge_harmonics_backward(Tensor grad_Y, Tensor n, int[] table) -> Tensor");
  m.def("radial_mlp_backward(Tensor grad_out, Tensor r, Tensor w0, Tensor b0, Tensor w2, Tensor b2, Tensor? w4, "
        "float r_cut, int basis) -> Tensor");
  m.def("readout_gather(Tensor[] layers, Tensor srcmap, int[] table) -> (Tensor, Tensor)");
  m.def("readout_gather_blocked(Tensor[] layers, Tensor srcmap, int[] table) -> (Tensor, Tensor)");
  m.def("readout_scatter(Tensor?[] grad_t, Tensor? grad_sq, Tensor[] layers, Tensor gmap, int[] table) -> Tensor[]");
  m.def("readout_features(Tensor[] layers, Tensor[] Wf, Tensor[] Wb, float[] scales, Tensor srcmap, Tensor gmap, "
        "int[] table) -> (Tensor, Tensor)");
  m.def("graph_prepare(Tensor edge_src, Tensor edge_dst, Tensor species, int n_species) -> Tensor[]");
  m.def("edge_vec_geometry(Tensor edge_vec, Tensor order) -> (Tensor, Tensor)");
  m.def("edge_vec_geometry_backward(Tensor? grad_n, Tensor? grad_r, Tensor n, Tensor r, Tensor order) -> Tensor");
  m.def("spatial_order(Tensor pos) -> Tensor");
  m.def("neighbor_list(Tensor pos, Tensor cell, float cutoff, int[] pbc) -> Tensor[]");
}

TORCH_LIBRARY_IMPL(fsctep, CUDA, m) {
  m.impl("sparse_prepare_weights", sparse_prepare_weights);
  m.impl("sparse_conv", sparse_conv);
  m.impl("sparse_conv_backward", sparse_conv_backward);
  m.impl("sparse_conv_direction", sparse_conv_direction);
  m.impl("sparse_conv_direction_backward", sparse_conv_direction_backward);
  m.impl("sparse_conv1_pair_table", sparse_conv1_pair_table);
  m.impl("sparse_conv1", sparse_conv1);
  m.impl("sparse_conv1_backward", sparse_conv1_backward);
  m.impl("ictd_prepare_weights", ictd_prepare_weights);
  m.impl("ictd_conv", ictd_conv);
  m.impl("ictd_project", ictd_project);
  m.impl("ictd_conv_backward", ictd_conv_backward);
  m.impl("ictd_conv1", ictd_conv1);
  m.impl("ictd_conv1_backward", ictd_conv1_backward);
  m.impl("gram_prepare_weights", gram_prepare_weights);
  m.impl("gram_bilinear", gram_bilinear);
  m.impl("gram_bilinear_blocked", gram_bilinear_blocked);
  m.impl("gram_bilinear_backward_blocked", gram_bilinear_backward_blocked);
  m.impl("gram_bilinear_backward", gram_bilinear_backward);
  m.impl("readout_mlp_prepare", readout_mlp_prepare);
  m.impl("readout_mlp", readout_mlp);
  m.impl("readout_mlp_backward", readout_mlp_backward);
  m.impl("edge_geometry", edge_geometry);
  m.impl("edge_geometry_backward", edge_geometry_backward);
  m.impl("radial_mlp", radial_mlp);
  m.impl("radial_mlp_backward", radial_mlp_backward);
  m.impl("edge_harmonics", edge_harmonics);
  m.impl("edge_harmonics_backward", edge_harmonics_backward);
  m.impl("readout_gather", readout_gather);
  m.impl("readout_gather_blocked", readout_gather_blocked);
  m.impl("readout_scatter", readout_scatter);
  m.impl("readout_features", readout_features);
  m.impl("graph_prepare", graph_prepare);
  m.impl("edge_vec_geometry", edge_vec_geometry);
  m.impl("edge_vec_geometry_backward", edge_vec_geometry_backward);
  m.impl("spatial_order", spatial_order);
  m.impl("neighbor_list", neighbor_list);
}

TORCH_LIBRARY_IMPL(fsctep, Meta, m) {
  m.impl("sparse_prepare_weights", sparse_prepare_weights_meta);
  m.impl("sparse_conv", sparse_conv_meta);
  m.impl("sparse_conv_backward", sparse_conv_backward_meta);
  m.impl("sparse_conv_direction", sparse_conv_direction_meta);
  m.impl("sparse_conv_direction_backward", sparse_conv_direction_backward_meta);
  m.impl("sparse_conv1_pair_table", sparse_conv1_pair_table_meta);
  m.impl("sparse_conv1", sparse_conv1_meta);
  m.impl("sparse_conv1_backward", sparse_conv1_backward_meta);
  m.impl("ictd_prepare_weights", ictd_prepare_weights_meta);
  m.impl("ictd_conv", ictd_conv_meta);
  m.impl("ictd_project", ictd_project_meta);
  m.impl("ictd_conv_backward", ictd_conv_backward_meta);
  m.impl("ictd_conv1", ictd_conv1_meta);
  m.impl("ictd_conv1_backward", ictd_conv1_backward_meta);
  m.impl("gram_prepare_weights", gram_prepare_weights_meta);
  m.impl("gram_bilinear", gram_bilinear_meta);
  m.impl("gram_bilinear_blocked", gram_bilinear_meta);
  m.impl("gram_bilinear_backward_blocked", gram_bilinear_backward_meta);
  m.impl("gram_bilinear_backward", gram_bilinear_backward_meta);
  m.impl("readout_mlp_prepare", readout_mlp_prepare_meta);
  m.impl("readout_mlp", readout_mlp_meta);
  m.impl("readout_mlp_backward", readout_mlp_backward_meta);
  m.impl("edge_geometry", edge_geometry_meta);
  m.impl("edge_geometry_backward", edge_geometry_backward_meta);
  m.impl("radial_mlp", radial_mlp_meta);
  m.impl("radial_mlp_backward", radial_mlp_backward_meta);
  m.impl("edge_harmonics", edge_harmonics_meta);
  m.impl("edge_harmonics_backward", edge_harmonics_backward_meta);
  m.impl("readout_gather", readout_gather_meta);
  m.impl("readout_gather_blocked", readout_gather_meta);
  m.impl("readout_scatter", readout_scatter_meta);
  m.impl("readout_features", readout_features_meta);
  m.impl("graph_prepare", graph_prepare_meta);
  m.impl("edge_vec_geometry", edge_vec_geometry_meta);
  m.impl("edge_vec_geometry_backward", edge_vec_geometry_backward_meta);
  m.impl("spatial_order", spatial_order_meta);
}

TORCH_LIBRARY_IMPL(fsctep, Autograd, m) {
  m.impl("sparse_conv", sparse_conv_autograd);
  m.impl("sparse_conv1", sparse_conv1_autograd);
  m.impl("ictd_conv", ictd_conv_autograd);
  m.impl("ictd_conv1", ictd_conv1_autograd);
  m.impl("gram_bilinear", gram_bilinear_autograd);
  m.impl("readout_mlp", readout_mlp_autograd);
  m.impl("edge_geometry", edge_geometry_autograd);
  m.impl("radial_mlp", radial_mlp_autograd);
  m.impl("edge_harmonics", edge_harmonics_autograd);
  m.impl("readout_features", readout_features_autograd);
  m.impl("edge_vec_geometry", edge_vec_geometry_autograd);
}

TORCH_LIBRARY_IMPL(fsctep, CPU, m) {
  for (const char* name : {"sparse_prepare_weights", "sparse_conv", "sparse_conv_backward", "sparse_conv1_pair_table",
                           "sparse_conv1", "sparse_conv1_backward", "sparse_conv_direction", "sparse_conv_direction_backward",
                           "ictd_prepare_weights", "ictd_conv",
                           "ictd_conv_backward", "ictd_project", "ictd_conv1", "ictd_conv1_backward", "gram_prepare_weights",
                           "gram_bilinear", "gram_bilinear_backward", "readout_mlp_prepare", "readout_mlp",
                           "readout_mlp_backward", "edge_geometry", "edge_geometry_backward",
                           "radial_mlp", "radial_mlp_backward", "edge_harmonics", "edge_harmonics_backward",
                           "readout_gather", "readout_scatter", "readout_features", "graph_prepare",
                           "edge_vec_geometry", "edge_vec_geometry_backward", "spatial_order", "neighbor_list",
                           "gram_bilinear_blocked", "gram_bilinear_backward_blocked", "readout_gather_blocked"})
    m.impl(name, torch::CppFunction::makeFromBoxedFunction<&refuse_cpu>());
}
