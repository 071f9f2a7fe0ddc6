// A LibTorch process with no Python that runs an exported core.pt on the GPU the way the LAMMPS engine
// does (lammps_user_mfftorch/src/USER-MFFTORCH/mff_torch_engine.cpp):
//   * dlopen the op library with RTLD_GLOBAL (MFF_CUSTOM_OPS_LIB, :226-249), torch::jit::load the core;
//   * pos as an autograd leaf, edge_vec = pos[dst] - pos[src] + edge_shifts @ cell[batch[src]] (:740-760);
//   * core.forward(pos, A, batch, edge_src, edge_dst, edge_shifts, cell, edge_vec[, external_tensor]);
//   * forces = -dE/dpos by torch::autograd::grad of the summed atom energies (:818-820).
// Inputs are raw little-endian files in <dir>: meta.txt ("N E n_external"), pos.f32 (N*3), A.i64 (N),
// src.i64 (E), dst.i64 (E), shifts.f32 (E*3), cell.f32 (9), external.f32 (n_external).
// Output <dir>/out.f32: N atom energies, N*3 forces, then global_phys (G*22) and global_mask (5).
//   core_run <libfsctep_torch.so> <core.pt> <dir> [repeats]
#include <dlfcn.h>

#include <torch/script.h>
#include <torch/torch.h>

#include <cstdio>
#include <fstream>
#include <string>
#include <vector>

namespace {

template <typename T>
std::vector<T> read_raw(const std::string& path, size_t count) {
  std::vector<T> v(count);
  std::ifstream f(path, std::ios::binary);
  if (!f) throw std::runtime_error("cannot open " + path);
  f.read(reinterpret_cast<char*>(v.data()), (std::streamsize)(count * sizeof(T)));
  if ((size_t)f.gcount() != count * sizeof(T)) throw std::runtime_error("short read " + path);
  return v;
}

template <typename T>
torch::Tensor to_device(std::vector<T>& v, at::IntArrayRef shape, at::ScalarType st, const torch::Device& dev) {
  return torch::from_blob(v.data(), shape, torch::TensorOptions().dtype(st)).clone().to(dev);
}

}  // namespace

int main(int argc, char** argv) {
  if (argc < 4) {
    std::fprintf(stderr, "usage: %s <libfsctep_torch.so> <core.pt> <dir> [repeats]\n", argv[0]);
    return 2;
  }
  if (!dlopen(argv[1], RTLD_NOW | RTLD_GLOBAL)) {
    std::fprintf(stderr, "dlopen failed: %s\n", dlerror());
    return 1;
  }
  const std::string dir = argv[3];
  const int repeats = argc > 4 ? std::atoi(argv[4]) : 1;
  try {
    if (!torch::cuda::is_available()) {
      std::fprintf(stderr, "no GPU visible\n");
      return 1;
    }
    const torch::Device dev(torch::kCUDA, 0);
    long long N = 0, E = 0, X = 0;
    {
      std::ifstream m(dir + "/meta.txt");
      m >> N >> E >> X;
      if (!m) throw std::runtime_error("bad meta.txt");
    }
    auto pos_h = read_raw<float>(dir + "/pos.f32", N * 3);
    auto A_h = read_raw<int64_t>(dir + "/A.i64", N);
    auto src_h = read_raw<int64_t>(dir + "/src.i64", E);
    auto dst_h = read_raw<int64_t>(dir + "/dst.i64", E);
    auto sh_h = read_raw<float>(dir + "/shifts.f32", E * 3);
    auto cell_h = read_raw<float>(dir + "/cell.f32", 9);
    std::vector<float> ext_h = X ? read_raw<float>(dir + "/external.f32", X) : std::vector<float>();

    torch::jit::Module core = torch::jit::load(argv[2], dev);
    core.eval();
    auto pos0 = to_device(pos_h, {N, 3}, torch::kFloat, dev);
    auto A = to_device(A_h, {N}, torch::kLong, dev);
    auto edge_src = to_device(src_h, {E}, torch::kLong, dev);
    auto edge_dst = to_device(dst_h, {E}, torch::kLong, dev);
    auto edge_shifts = to_device(sh_h, {E, 3}, torch::kFloat, dev);
    auto cell = to_device(cell_h, {1, 3, 3}, torch::kFloat, dev);
    auto batch = torch::zeros({N}, torch::TensorOptions().dtype(torch::kLong).device(dev));
    auto external = X ? to_device(ext_h, {X}, torch::kFloat, dev)
                      : torch::empty({0}, torch::TensorOptions().dtype(torch::kFloat).device(dev));

    torch::Tensor atom_e, forces, gphys, gmask;
    for (int it = 0; it < repeats; ++it) {
      auto pos = pos0.clone().detach().requires_grad_(true);
      auto edge_batch = batch.index_select(0, edge_src);
      auto edge_cells = cell.index_select(0, edge_batch);
      auto shift_vec = (edge_shifts.unsqueeze(-1) * edge_cells).sum(1);   // einsum("ni,nij->nj")
      auto edge_vec = pos.index_select(0, edge_dst) - pos.index_select(0, edge_src) + shift_vec;
      std::vector<torch::jit::IValue> inputs{pos, A, batch, edge_src, edge_dst, edge_shifts, cell, edge_vec, external};
      auto out = core.forward(inputs);
      auto elems = out.toTuple()->elements();
      if (elems.size() != 6) throw std::runtime_error("core must return a 6-tuple");
      atom_e = elems[0].toTensor();
      gphys = elems[1].toTensor();
      gmask = elems[3].toTensor();
      if (gphys.size(-1) != 22 || elems[2].toTensor().size(-1) != 31 || gmask.numel() != 5 ||
          elems[4].toTensor().numel() != 5)
        throw std::runtime_error("physical tensor slots do not match the 22/31/5 schema");
      auto E_local = atom_e.view({atom_e.size(0)}).sum();
      auto grads = torch::autograd::grad({E_local}, {pos}, {}, /*retain_graph=*/false, /*create_graph=*/false,
                                         /*allow_unused=*/true);
      forces = -grads[0];
    }
    torch::cuda::synchronize();
    auto cat = torch::cat({atom_e.reshape({-1}), forces.reshape({-1}), gphys.reshape({-1}), gmask.reshape({-1})})
                   .to(torch::kCPU).contiguous();
    std::ofstream o(dir + "/out.f32", std::ios::binary);
    o.write(reinterpret_cast<const char*>(cat.data_ptr<float>()), (std::streamsize)(cat.numel() * sizeof(float)));
    std::printf("core_run: N=%lld E=%lld repeats=%d E_total=%.6f\n", N, E, repeats,
                atom_e.sum().item<double>());
  } catch (const std::exception& e) {
    std::fprintf(stderr, "core_run failed: %s\n", e.what());
    return 1;
  }
  return 0;
}
