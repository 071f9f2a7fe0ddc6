// A LibTorch process with no Python: load the op library the way the LAMMPS engine loads
// MFF_CUSTOM_OPS_LIB (dlopen RTLD_GLOBAL, lammps_user_mfftorch/src/USER-MFFTORCH/mff_torch_engine.cpp:226-249),
// check every fsctep schema is registered, run Meta tensors through two ops and through a
// TorchScript module whose graph calls them.
//   load_ops <libfsctep_torch.so> <scripted_module.pt>
#include <dlfcn.h>

#include <ATen/core/dispatch/Dispatcher.h>
#include <torch/script.h>

#include <cstdio>
#include <vector>

int main(int argc, char** argv) {
  if (argc != 3) {
    std::fprintf(stderr, "usage: %s <libfsctep_torch.so> <module.pt>\n", argv[0]);
    return 2;
  }
  if (!dlopen(argv[1], RTLD_NOW | RTLD_GLOBAL)) {
    std::fprintf(stderr, "dlopen failed: %s\n", dlerror());
    return 1;
  }
  auto& disp = c10::Dispatcher::singleton();
  const char* names[] = {"sparse_prepare_weights", "sparse_conv", "sparse_conv_backward", "sparse_conv1_pair_table",
                         "sparse_conv1", "sparse_conv1_backward", "ictd_prepare_weights", "ictd_conv",
                         "ictd_conv_backward", "ictd_conv1", "ictd_conv1_backward", "gram_prepare_weights",
                         "gram_bilinear", "gram_bilinear_backward", "edge_geometry", "edge_geometry_backward",
                         "radial_mlp", "radial_mlp_backward", "edge_harmonics", "edge_harmonics_backward",
                         "readout_gather", "readout_scatter", "readout_features", "graph_prepare",
                         "edge_vec_geometry", "edge_vec_geometry_backward", "spatial_order", "ictd_project",
                         "sparse_conv_direction", "sparse_conv_direction_backward", "readout_mlp_prepare",
                         "readout_mlp", "readout_mlp_backward", "gram_bilinear_blocked",
                         "gram_bilinear_backward_blocked", "readout_gather_blocked",
                         // the per-edge (bucketed) ICTD ops under the reference extension's names
                         "project_bucket_forward", "project_bucket_transpose_a", "project_bucket_transpose_b",
                         "project_bucket_transpose_u", "mix_bucket_forward", "mix_bucket_transpose_y",
                         "mix_bucket_transpose_w", "mix_bucket_transpose_g", "bucketed_tp_forward",
                         "project_dbl_bwd_grad_h", "project_dbl_bwd_grad_a", "project_dbl_bwd_grad_b",
                         "project_dbl_bwd_grad_u", "mix_dbl_bwd_grad_g_out", "mix_dbl_bwd_grad_y",
                         "mix_dbl_bwd_grad_w", "mix_dbl_bwd_grad_g"};
  for (const char* n : names) {
    auto op = disp.findSchema({std::string("fsctep::") + n, ""});
    if (!op) {
      std::fprintf(stderr, "missing schema fsctep::%s\n", n);
      return 1;
    }
    if (!op->hasKernelForDispatchKey(c10::DispatchKey::CUDA) || !op->hasKernelForDispatchKey(c10::DispatchKey::Meta)) {
      std::fprintf(stderr, "fsctep::%s lacks a device or Meta kernel\n", n);
      return 1;
    }
  }
  const auto meta = at::device(at::kMeta).dtype(at::kFloat);
  auto W = at::empty({64, 192, 192}, meta);
  auto prep = disp.findSchemaOrThrow("fsctep::gram_prepare_weights", "")
                  .typed<std::tuple<at::Tensor, at::Tensor>(const at::Tensor&)>();
  auto [Wf, Wb] = prep.call(W);
  auto t = at::empty({7, 9, 192}, meta);
  auto x = at::empty({10, 13, 64}, meta), h = at::empty({30, 64}, meta), nv = at::empty({30, 3}, meta);
  auto bk = at::empty({6 * 65 * 64 * 64 + 512 + 3 * 65 * 64 * 64}, meta);
  auto ip = at::empty({11}, at::device(at::kMeta).dtype(at::kInt)), ie = at::empty({30}, at::device(at::kMeta).dtype(at::kInt));
  auto sc = disp.findSchemaOrThrow("fsctep::sparse_conv", "")
                .typed<std::tuple<at::Tensor, at::Tensor, at::Tensor>(
                    const at::Tensor&, const at::Tensor&, const at::Tensor&, const at::Tensor&, const at::Tensor&,
                    const at::Tensor&, const at::Tensor&, const at::Tensor&, const at::Tensor&, const at::Tensor&,
                    int64_t, const std::optional<at::Tensor>&, const std::optional<at::Tensor>&)>();
  auto no_order = at::empty({0}, at::device(at::kMeta).dtype(at::kInt));
  auto [out, S, P] = sc.call(x, h, nv, bk, bk, ip, ip, ie, ie, no_order, 0, std::nullopt, std::nullopt);
  // S: the backward's tail (16 node-expansion K parts at ten nodes), 256-byte aligned, then the four parts
  // of the split message gradient (dh, dn, dS maxima)
  const int64_t tail = 10 * 18 * 65 * 64 + 16 * 18 * 10 * 64 + 10;
  if (out.sizes() != at::IntArrayRef({10, 13, 64}) || S.numel() != (tail + 63) / 64 * 64 + 4 * (30 * 67 + 10) ||
      P.numel() != 30 * 18 * 64) {
    std::fprintf(stderr, "sparse_conv meta shapes wrong\n");
    return 1;
  }
  torch::jit::Module mod = torch::jit::load(argv[2]);
  auto y = mod.forward(std::vector<torch::jit::IValue>{t, Wf, Wb}).toTensor();
  if (y.sizes() != at::IntArrayRef({7, 64})) {
    std::fprintf(stderr, "scripted module output shape wrong\n");
    return 1;
  }
  std::printf("fsctep ops registered: %zu; scripted module -> [%lld, %lld]\n", sizeof(names) / sizeof(names[0]),
              (long long)y.size(0), (long long)y.size(1));
  return 0;
}
