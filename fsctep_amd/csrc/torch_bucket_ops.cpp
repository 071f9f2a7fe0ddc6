// torch.ops.fsctep.* for the per-edge (bucketed) ICTD tensor product: the functions of the reference's
// native extension module molecular_force_field._C_ictd_tp (csrc/ictd_tp.cpp:498-522), same names, same
// argument order and meaning, same output shapes, on the HIP kernels of ictd_bucket.hip (the C ABI
// fsc_bucket_*).  Each call allocates its outputs, as the reference's do, and launches on the current
// stream (the reference's extension uses the default stream, csrc/ictd_tp_cuda.cu:178).  Argument errors
// raise RuntimeError with the reference's messages (csrc/ictd_tp.cpp:78-105).  The HIP path takes what the
// reference's CUDA path takes, mul_in2 == 1, in fp32 or fp64 (csrc/ictd_tp_cuda.cu:1230-1236 dispatches
// both; the fp64 calls go to the fsc_bucket_*_f64 kernels); other arguments raise (the reference falls back
// to ATen for them, its double-backward functions raise likewise without CUDA).  The double-backward
// functions are the sums of csrc/ictd_tp_cuda.cu:528-533 and 796-802, formed by the same kernels
// accumulating into one output.

#include <ATen/ATen.h>
#include <c10/hip/HIPStream.h>
#include <torch/library.h>

#include "fsctep.h"

namespace {

using at::Tensor;

hipStream_t stream_of(const Tensor& t) { return c10::hip::getCurrentHIPStream(t.device().index()).stream(); }

void check(int rc, const char* name) { TORCH_CHECK(rc == 0, name, " failed (", rc, "): ", fsc_last_error()); }

// every argument on the GPU, float32 or float64, all of one dtype
void gpu_float(std::initializer_list<std::reference_wrapper<const Tensor>> ts, const char* name) {
  const at::ScalarType st = ts.begin()->get().scalar_type();
  for (const Tensor& t : ts) {
    TORCH_CHECK(t.is_cuda(), name, ": the HIP kernels take GPU tensors, got a ", t.device(), " tensor");
    TORCH_CHECK(t.scalar_type() == at::kFloat || t.scalar_type() == at::kDouble, name,
                ": the HIP kernels take float32 or float64, got ", t.scalar_type());
    TORCH_CHECK(t.scalar_type() == st, name, ": all arguments must have one dtype, got ", st, " and ",
                t.scalar_type());
  }
}

void mul_in2_one(int64_t mul_in2, const char* name) {
  TORCH_CHECK(mul_in2 == 1, name, ": mul_in2 = ", mul_in2,
              " is not supported (the HIP kernels, like the reference's CUDA kernels, take mul_in2 == 1)");
}

template <typename T>
const T* cp(const Tensor& t) {
  return t.numel() ? t.data_ptr<T>() : nullptr;
}
template <typename T>
T* mp(Tensor& t) {
  return t.numel() ? t.data_ptr<T>() : nullptr;
}

// The C ABI by element type (fsc_bucket_<op> for float, fsc_bucket_<op>_f64 for double).
#define FSC_ABI_PAIR(NAME, PARAMS, ARGS)                                                                        \
  inline int abi_##NAME(PARAMS(float)) { return fsc_bucket_##NAME ARGS; }                                     \
  inline int abi_##NAME(PARAMS(double)) { return fsc_bucket_##NAME##_f64 ARGS; }
#define P_PROJECT(T) int64_t B, int32_t I, int32_t m1, int32_t m2, int32_t P, int32_t K, const T* a, const T* v, \
                     const T* u, T* y, int32_t acc, hipStream_t st
FSC_ABI_PAIR(project, P_PROJECT, (B, I, m1, m2, P, K, a, v, u, y, acc, st))
FSC_ABI_PAIR(project_transpose_a, P_PROJECT, (B, I, m1, m2, P, K, a, v, u, y, acc, st))
#define P_PROJECT_VU(T) int64_t B, int32_t I, int32_t m1, int32_t m2, int32_t P, int32_t K, const T* gy, const T* a, \
                        const T* v, const T* u, T* gv, T* gu, int32_t acc, T* ws, hipStream_t st
FSC_ABI_PAIR(project_transpose_vu, P_PROJECT_VU, (B, I, m1, m2, P, K, gy, a, v, u, gv, gu, acc, ws, st))
#define P_MIX(T) int64_t B, int32_t P, int32_t K, int32_t I, int32_t O, const T* x, const T* w, const T* g, T* out, \
                 int32_t acc, hipStream_t st
FSC_ABI_PAIR(mix, P_MIX, (B, P, K, I, O, x, w, g, out, acc, st))
FSC_ABI_PAIR(mix_transpose_g, P_MIX, (B, P, K, I, O, x, w, g, out, acc, st))
#define P_MIX_WS(T) int64_t B, int32_t P, int32_t K, int32_t I, int32_t O, const T* x, const T* w, const T* g, \
                    T* out, int32_t acc, T* ws, hipStream_t st
FSC_ABI_PAIR(mix_transpose_y, P_MIX_WS, (B, P, K, I, O, x, w, g, out, acc, ws, st))
FSC_ABI_PAIR(mix_transpose_w, P_MIX_WS, (B, P, K, I, O, x, w, g, out, acc, ws, st))
#undef FSC_ABI_PAIR

// runs the statements with T the element type of t (float or double)
#define BY_DTYPE(t, ...)                      \
  if ((t).scalar_type() == at::kDouble) {     \
    using T = double;                         \
    __VA_ARGS__;                              \
  } else {                                    \
    using T = float;                          \
    __VA_ARGS__;                              \
  }

// csrc/ictd_tp.cpp:78-91
void check_projection_args(const Tensor& a, const Tensor& b, const Tensor& u) {
  TORCH_CHECK(a.dim() == 3, "a must have shape (B, mul_in1, m1)");
  TORCH_CHECK(b.dim() == 3, "b must have shape (B, mul_in2, m2)");
  TORCH_CHECK(u.dim() == 2, "u_bucket must have shape (m1*m2, P*kdim)");
  TORCH_CHECK(a.device() == b.device(), "a and b must be on the same device");
  TORCH_CHECK(a.device() == u.device(), "a and u_bucket must be on the same device");
  TORCH_CHECK(a.scalar_type() == b.scalar_type(), "a and b must have the same dtype");
  TORCH_CHECK(a.scalar_type() == u.scalar_type(), "a and u_bucket must have the same dtype");
  TORCH_CHECK(b.size(0) == a.size(0), "a and b batch dimensions must match");
  TORCH_CHECK(u.size(0) == a.size(2) * b.size(2), "u_bucket first dim must equal m1*m2");
}

// csrc/ictd_tp.cpp:93-105
void check_mix_args(const Tensor& y, const Tensor& w, const Tensor& gates) {
  TORCH_CHECK(y.dim() == 4, "y must have shape (B, P, kdim, IJ)");
  TORCH_CHECK(w.dim() == 3, "w must have shape (P, mul_out, IJ)");
  TORCH_CHECK(gates.dim() == 2, "gates must have shape (B, P)");
  TORCH_CHECK(y.device() == w.device(), "y and w must be on the same device");
  TORCH_CHECK(y.device() == gates.device(), "y and gates must be on the same device");
  TORCH_CHECK(y.scalar_type() == w.scalar_type(), "y and w must have the same dtype");
  TORCH_CHECK(y.scalar_type() == gates.scalar_type(), "y and gates must have the same dtype");
  TORCH_CHECK(y.size(0) == gates.size(0), "gates batch dim must match y");
  TORCH_CHECK(y.size(1) == w.size(0), "w path dim must match y");
  TORCH_CHECK(y.size(1) == gates.size(1), "gates path dim must match y");
  TORCH_CHECK(y.size(3) == w.size(2), "w IJ dim must match y");
}

// ---------------------------------------------------------------- projection primitives (acc: add to out)
struct Proj {
  int64_t B, I, m1, m2, P, K;
};

void pf(const Proj& s, const Tensor& a, const Tensor& b, const Tensor& u, Tensor& y, int acc) {
  const Tensor ac = a.contiguous(), bc = b.contiguous(), uc = u.contiguous();
  BY_DTYPE(y,
    check(abi_project(s.B, (int32_t)s.I, (int32_t)s.m1, (int32_t)s.m2, (int32_t)s.P, (int32_t)s.K, cp<T>(ac),
                      cp<T>(bc), cp<T>(uc), mp<T>(y), acc, stream_of(y)),
          "project_bucket_forward"))
}

void pat(const Proj& s, const Tensor& gy, const Tensor& b, const Tensor& u, Tensor& ga, int acc) {
  const Tensor gc = gy.contiguous(), bc = b.contiguous(), uc = u.contiguous();
  BY_DTYPE(ga,
    check(abi_project_transpose_a(s.B, (int32_t)s.I, (int32_t)s.m1, (int32_t)s.m2, (int32_t)s.P, (int32_t)s.K,
                                  cp<T>(gc), cp<T>(bc), cp<T>(uc), mp<T>(ga), acc, stream_of(ga)),
          "project_bucket_transpose_a"))
}

// grad_b (gb) and/or grad_u (gu), either undefined
void pvu(const Proj& s, const Tensor& gy, const Tensor& a, const Tensor& b, const Tensor& u, Tensor* gb, Tensor* gu,
         int acc) {
  const Tensor gc = gy.contiguous(), ac = a.contiguous();
  const Tensor bc = b.defined() ? b.contiguous() : Tensor(), uc = u.defined() ? u.contiguous() : Tensor();
  Tensor ws;
  if (gu) {
    int64_t n = 0;
    check(fsc_bucket_project_workspace(s.B, (int32_t)s.I, (int32_t)s.m1, (int32_t)s.m2, (int32_t)s.P, (int32_t)s.K, &n),
          "project_bucket_transpose_u");
    ws = at::empty({std::max<int64_t>(n, 1)}, gy.options());
  }
  BY_DTYPE(gy,
    check(abi_project_transpose_vu(s.B, (int32_t)s.I, (int32_t)s.m1, (int32_t)s.m2, (int32_t)s.P, (int32_t)s.K,
                                   cp<T>(gc), cp<T>(ac), bc.defined() ? cp<T>(bc) : nullptr,
                                   uc.defined() ? cp<T>(uc) : nullptr, gb ? mp<T>(*gb) : nullptr,
                                   gu ? mp<T>(*gu) : nullptr, acc, gu ? mp<T>(ws) : nullptr, stream_of(gy)),
          gb ? "project_bucket_transpose_b" : "project_bucket_transpose_u"))
}

// ---------------------------------------------------------------- mix primitives
struct Mix {
  int64_t B, P, K, I, O;
};

Mix mix_sizes(const Tensor& y, const Tensor& w) { return Mix{y.size(0), y.size(1), y.size(2), y.size(3), w.size(1)}; }

void mf(const Mix& s, const Tensor& y, const Tensor& w, const Tensor& g, Tensor& out, int acc) {
  const Tensor yc = y.contiguous(), wc = w.contiguous(), gc = g.contiguous();
  BY_DTYPE(out,
    check(abi_mix(s.B, (int32_t)s.P, (int32_t)s.K, (int32_t)s.I, (int32_t)s.O, cp<T>(yc), cp<T>(wc), cp<T>(gc),
                  mp<T>(out), acc, stream_of(out)),
          "mix_bucket_forward"))
}

Tensor mix_ws(const Mix& s, const Tensor& like) {
  int64_t n = 0;
  check(fsc_bucket_mix_workspace(s.B, (int32_t)s.P, (int32_t)s.K, (int32_t)s.I, (int32_t)s.O, &n), "mix_bucket");
  return at::empty({std::max<int64_t>(n, 1)}, like.options());
}

void myt(const Mix& s, const Tensor& go, const Tensor& w, const Tensor& g, Tensor& gy, int acc) {
  const Tensor oc = go.contiguous(), wc = w.contiguous(), gc = g.contiguous();
  Tensor ws = at::empty({std::max<int64_t>(s.P * s.O * s.I, 1)}, go.options());   // the transposed weights
  BY_DTYPE(gy,
    check(abi_mix_transpose_y(s.B, (int32_t)s.P, (int32_t)s.K, (int32_t)s.I, (int32_t)s.O, cp<T>(oc), cp<T>(wc),
                              cp<T>(gc), mp<T>(gy), acc, mp<T>(ws), stream_of(gy)),
          "mix_bucket_transpose_y"))
}

void mwt(const Mix& s, const Tensor& go, const Tensor& y, const Tensor& g, Tensor& gw, int acc) {
  const Tensor oc = go.contiguous(), yc = y.contiguous(), gc = g.contiguous();
  Tensor ws = mix_ws(s, go);
  BY_DTYPE(gw,
    check(abi_mix_transpose_w(s.B, (int32_t)s.P, (int32_t)s.K, (int32_t)s.I, (int32_t)s.O, cp<T>(oc), cp<T>(yc),
                              cp<T>(gc), mp<T>(gw), acc, mp<T>(ws), stream_of(gw)),
          "mix_bucket_transpose_w"))
}

void mgt(const Mix& s, const Tensor& go, const Tensor& y, const Tensor& w, Tensor& gg, int acc) {
  const Tensor oc = go.contiguous(), yc = y.contiguous(), wc = w.contiguous();
  BY_DTYPE(gg,
    check(abi_mix_transpose_g(s.B, (int32_t)s.P, (int32_t)s.K, (int32_t)s.I, (int32_t)s.O, cp<T>(oc), cp<T>(yc),
                              cp<T>(wc), mp<T>(gg), acc, stream_of(gg)),
          "mix_bucket_transpose_g"))
}

// ---------------------------------------------------------------- the reference's functions
Tensor project_bucket_forward(const Tensor& a, const Tensor& b, const Tensor& u, int64_t num_paths) {
  check_projection_args(a, b, u);
  TORCH_CHECK(num_paths > 0, "num_paths must be positive");
  TORCH_CHECK(u.size(1) % num_paths == 0, "u_bucket second dim must be divisible by num_paths");
  gpu_float({a, b, u}, "project_bucket_forward");
  mul_in2_one(b.size(1), "project_bucket_forward");
  const Proj s{a.size(0), a.size(1), a.size(2), b.size(2), num_paths, u.size(1) / num_paths};
  Tensor y = at::empty({s.B, s.P, s.K, s.I}, a.options());
  pf(s, a, b, u, y, 0);
  return y;
}

// sizes of a projection transpose from grad_y (B, P, kdim, IJ) and the two operands' component counts
Proj proj_from_grad(const Tensor& grad_y, int64_t mul_in1, int64_t m1, int64_t m2) {
  return Proj{grad_y.size(0), mul_in1, m1, m2, grad_y.size(1), grad_y.size(2)};
}

Tensor project_bucket_transpose_a(const Tensor& grad_y, const Tensor& b, const Tensor& u) {
  TORCH_CHECK(b.dim() == 3, "b must have shape (B, mul_in2, m2)");
  TORCH_CHECK(u.dim() == 2, "u_bucket must have shape (m1*m2, P*kdim)");
  TORCH_CHECK(grad_y.dim() == 4, "grad_y must have shape (B, P, kdim, IJ)");
  TORCH_CHECK(grad_y.size(0) == b.size(0), "grad_y batch must match b");
  TORCH_CHECK(grad_y.size(3) % b.size(1) == 0, "grad_y IJ dim must be divisible by mul_in2");
  const int64_t m2 = b.size(2), m1 = u.size(0) / std::max<int64_t>(m2, 1);
  TORCH_CHECK(m1 * m2 == u.size(0), "u_bucket first dim must factor into m1*m2");
  TORCH_CHECK(u.size(1) == grad_y.size(1) * grad_y.size(2), "u_bucket second dim must equal P*kdim");
  gpu_float({grad_y, b, u}, "project_bucket_transpose_a");
  mul_in2_one(b.size(1), "project_bucket_transpose_a");
  const Proj s = proj_from_grad(grad_y, grad_y.size(3), m1, m2);
  Tensor ga = at::empty({s.B, s.I, m1}, grad_y.options());
  pat(s, grad_y, b, u, ga, 0);
  return ga;
}

Tensor project_bucket_transpose_b(const Tensor& grad_y, const Tensor& a, const Tensor& u) {
  TORCH_CHECK(a.dim() == 3, "a must have shape (B, mul_in1, m1)");
  TORCH_CHECK(u.dim() == 2, "u_bucket must have shape (m1*m2, P*kdim)");
  TORCH_CHECK(grad_y.dim() == 4, "grad_y must have shape (B, P, kdim, IJ)");
  TORCH_CHECK(grad_y.size(0) == a.size(0), "grad_y batch must match a");
  TORCH_CHECK(grad_y.size(3) % a.size(1) == 0, "grad_y IJ dim must be divisible by mul_in1");
  const int64_t m1 = a.size(2), m2 = u.size(0) / std::max<int64_t>(m1, 1);
  TORCH_CHECK(m1 * m2 == u.size(0), "u_bucket first dim must factor into m1*m2");
  TORCH_CHECK(u.size(1) == grad_y.size(1) * grad_y.size(2), "u_bucket second dim must equal P*kdim");
  gpu_float({grad_y, a, u}, "project_bucket_transpose_b");
  mul_in2_one(grad_y.size(3) / a.size(1), "project_bucket_transpose_b");
  const Proj s = proj_from_grad(grad_y, a.size(1), m1, m2);
  Tensor gb = at::empty({s.B, 1, m2}, grad_y.options());
  pvu(s, grad_y, a, Tensor(), u, &gb, nullptr, 0);
  return gb;
}

Tensor project_bucket_transpose_u(const Tensor& grad_y, const Tensor& a, const Tensor& b) {
  TORCH_CHECK(a.dim() == 3, "a must have shape (B, mul_in1, m1)");
  TORCH_CHECK(b.dim() == 3, "b must have shape (B, mul_in2, m2)");
  TORCH_CHECK(a.device() == b.device(), "a and b must be on the same device");
  TORCH_CHECK(a.scalar_type() == b.scalar_type(), "a and b must have the same dtype");
  TORCH_CHECK(grad_y.dim() == 4 && grad_y.size(0) == a.size(0) && b.size(0) == a.size(0) &&
                  grad_y.size(3) == a.size(1) * b.size(1),
              "grad_y must have shape (B, P, kdim, mul_in1*mul_in2)");
  gpu_float({grad_y, a, b}, "project_bucket_transpose_u");
  mul_in2_one(b.size(1), "project_bucket_transpose_u");
  const Proj s = proj_from_grad(grad_y, a.size(1), a.size(2), b.size(2));
  Tensor gu = at::empty({s.m1 * s.m2, s.P * s.K}, grad_y.options());
  pvu(s, grad_y, a, b, Tensor(), nullptr, &gu, 0);
  return gu;
}

Tensor mix_bucket_forward(const Tensor& y, const Tensor& w, const Tensor& gates) {
  check_mix_args(y, w, gates);
  gpu_float({y, w, gates}, "mix_bucket_forward");
  const Mix s = mix_sizes(y, w);
  Tensor out = at::empty({s.B, s.O, s.K}, y.options());
  mf(s, y, w, gates, out, 0);
  return out;
}

Tensor mix_bucket_transpose_y(const Tensor& grad_out, const Tensor& w, const Tensor& gates) {
  TORCH_CHECK(grad_out.dim() == 3, "grad_out must have shape (B, O, kdim)");
  TORCH_CHECK(w.dim() == 3, "w must have shape (P, O, IJ)");
  TORCH_CHECK(gates.dim() == 2, "gates must have shape (B, P)");
  TORCH_CHECK(w.size(1) == grad_out.size(1), "w output dim must match grad_out");
  TORCH_CHECK(gates.size(0) == grad_out.size(0) && gates.size(1) == w.size(0), "gates must match grad_out and w");
  gpu_float({grad_out, w, gates}, "mix_bucket_transpose_y");
  const Mix s{grad_out.size(0), w.size(0), grad_out.size(2), w.size(2), w.size(1)};
  Tensor gy = at::empty({s.B, s.P, s.K, s.I}, grad_out.options());
  myt(s, grad_out, w, gates, gy, 0);
  return gy;
}

Tensor mix_bucket_transpose_w(const Tensor& grad_out, const Tensor& y, const Tensor& gates) {
  TORCH_CHECK(grad_out.dim() == 3, "grad_out must have shape (B, O, kdim)");
  TORCH_CHECK(y.dim() == 4, "y must have shape (B, P, kdim, IJ)");
  TORCH_CHECK(gates.dim() == 2, "gates must have shape (B, P)");
  TORCH_CHECK(y.size(0) == gates.size(0), "gates batch dim must match y");
  TORCH_CHECK(y.size(1) == gates.size(1), "gates path dim must match y");
  TORCH_CHECK(grad_out.size(0) == y.size(0) && grad_out.size(2) == y.size(2), "grad_out must match y");
  gpu_float({grad_out, y, gates}, "mix_bucket_transpose_w");
  const Mix s{y.size(0), y.size(1), y.size(2), y.size(3), grad_out.size(1)};
  Tensor gw = at::empty({s.P, s.O, s.I}, y.options());
  mwt(s, grad_out, y, gates, gw, 0);
  return gw;
}

Tensor mix_bucket_transpose_g(const Tensor& grad_out, const Tensor& y, const Tensor& w) {
  TORCH_CHECK(grad_out.dim() == 3, "grad_out must have shape (B, O, kdim)");
  TORCH_CHECK(y.dim() == 4, "y must have shape (B, P, kdim, IJ)");
  TORCH_CHECK(w.dim() == 3, "w must have shape (P, O, IJ)");
  TORCH_CHECK(grad_out.size(0) == y.size(0) && grad_out.size(2) == y.size(2), "grad_out must match y");
  TORCH_CHECK(w.size(0) == y.size(1) && w.size(1) == grad_out.size(1) && w.size(2) == y.size(3),
              "w must match y and grad_out");
  gpu_float({grad_out, y, w}, "mix_bucket_transpose_g");
  const Mix s = mix_sizes(y, w);
  Tensor gg = at::empty({s.B, s.P}, y.options());
  mgt(s, grad_out, y, w, gg, 0);
  return gg;
}

Tensor bucketed_tp_forward(const Tensor& a, const Tensor& b, const Tensor& u, const Tensor& w, const Tensor& gates) {
  check_projection_args(a, b, u);
  TORCH_CHECK(w.dim() == 3, "w must have shape (P, mul_out, IJ)");
  TORCH_CHECK(gates.dim() == 2, "gates must have shape (B, P)");
  TORCH_CHECK(gates.size(1) == w.size(0), "gates path dim must match w");
  TORCH_CHECK(u.size(1) % w.size(0) == 0, "u_bucket second dim must be divisible by number of paths");
  const Tensor y = project_bucket_forward(a, b, u, w.size(0));
  return mix_bucket_forward(y, w, gates);
}

// grad_H = PF(gga, b, u) + PF(a, ggb, u) + PF(a, b, ggu)
Tensor project_dbl_bwd_grad_h(const Tensor& a, const Tensor& gga, const Tensor& b, const Tensor& ggb, const Tensor& u,
                              const Tensor& ggu, int64_t num_paths) {
  check_projection_args(a, b, u);
  check_projection_args(gga, ggb, ggu);
  TORCH_CHECK(num_paths > 0 && u.size(1) % num_paths == 0, "u_bucket second dim must be divisible by num_paths");
  gpu_float({a, gga, b, ggb, u, ggu}, "project_dbl_bwd_grad_h");
  mul_in2_one(b.size(1), "project_dbl_bwd_grad_h");
  const Proj s{a.size(0), a.size(1), a.size(2), b.size(2), num_paths, u.size(1) / num_paths};
  Tensor out = at::empty({s.B, s.P, s.K, s.I}, a.options());
  pf(s, gga, b, u, out, 0);
  pf(s, a, ggb, u, out, 1);
  pf(s, a, b, ggu, out, 1);
  return out;
}

// grad_a2 = PAT(H, ggb, u) + PAT(H, b, ggu)
Tensor project_dbl_bwd_grad_a(const Tensor& h, const Tensor& b, const Tensor& ggb, const Tensor& u, const Tensor& ggu) {
  Tensor out = project_bucket_transpose_a(h, ggb, u);
  const Proj s = proj_from_grad(h, h.size(3), out.size(2), b.size(2));
  TORCH_CHECK(b.sizes() == ggb.sizes() && u.sizes() == ggu.sizes(), "b/ggb and u/ggu must have the same shapes");
  gpu_float({b, ggu}, "project_dbl_bwd_grad_a");
  pat(s, h, b, ggu, out, 1);
  return out;
}

// grad_b2 = PBT(H, gga, u) + PBT(H, a, ggu)
Tensor project_dbl_bwd_grad_b(const Tensor& h, const Tensor& a, const Tensor& gga, const Tensor& u, const Tensor& ggu) {
  Tensor out = project_bucket_transpose_b(h, gga, u);
  const Proj s = proj_from_grad(h, a.size(1), a.size(2), out.size(2));
  TORCH_CHECK(a.sizes() == gga.sizes() && u.sizes() == ggu.sizes(), "a/gga and u/ggu must have the same shapes");
  gpu_float({a, ggu}, "project_dbl_bwd_grad_b");
  pvu(s, h, a, Tensor(), ggu, &out, nullptr, 1);
  return out;
}

// grad_U2 = PUT(H, gga, b) + PUT(H, a, ggb)
Tensor project_dbl_bwd_grad_u(const Tensor& h, const Tensor& a, const Tensor& gga, const Tensor& b, const Tensor& ggb) {
  Tensor out = project_bucket_transpose_u(h, gga, b);
  TORCH_CHECK(a.sizes() == gga.sizes() && b.sizes() == ggb.sizes(), "a/gga and b/ggb must have the same shapes");
  gpu_float({a, ggb}, "project_dbl_bwd_grad_u");
  const Proj s = proj_from_grad(h, a.size(1), a.size(2), b.size(2));
  pvu(s, h, a, ggb, Tensor(), nullptr, &out, 1);
  return out;
}

// grad_G = MF(ggy, w, g) + MF(y, ggw, g) + MF(y, w, ggg)
Tensor mix_dbl_bwd_grad_g_out(const Tensor& y, const Tensor& ggy, const Tensor& w, const Tensor& ggw,
                              const Tensor& gates, const Tensor& ggg) {
  Tensor out = mix_bucket_forward(ggy, w, gates);
  check_mix_args(y, ggw, ggg);
  gpu_float({y, ggw, ggg}, "mix_dbl_bwd_grad_g_out");
  TORCH_CHECK(y.sizes() == ggy.sizes() && w.sizes() == ggw.sizes() && gates.sizes() == ggg.sizes(),
              "y/ggy, w/ggw and gates/ggg must have the same shapes");
  const Mix s = mix_sizes(y, w);
  mf(s, y, ggw, gates, out, 1);
  mf(s, y, w, ggg, out, 1);
  return out;
}

// grad_Y2 = MYT(G, ggw, g) + MYT(G, w, ggg)
Tensor mix_dbl_bwd_grad_y(const Tensor& g_out, const Tensor& w, const Tensor& ggw, const Tensor& gates,
                          const Tensor& ggg) {
  Tensor out = mix_bucket_transpose_y(g_out, ggw, gates);
  TORCH_CHECK(w.sizes() == ggw.sizes() && gates.sizes() == ggg.sizes(), "w/ggw and gates/ggg must have the same shapes");
  gpu_float({w, ggg}, "mix_dbl_bwd_grad_y");
  const Mix s{g_out.size(0), w.size(0), g_out.size(2), w.size(2), w.size(1)};
  myt(s, g_out, w, ggg, out, 1);
  return out;
}

// grad_W2 = MWT(G, ggy, g) + MWT(G, y, ggg)
Tensor mix_dbl_bwd_grad_w(const Tensor& g_out, const Tensor& y, const Tensor& ggy, const Tensor& gates,
                          const Tensor& ggg) {
  Tensor out = mix_bucket_transpose_w(g_out, ggy, gates);
  TORCH_CHECK(y.sizes() == ggy.sizes() && gates.sizes() == ggg.sizes(), "y/ggy and gates/ggg must have the same shapes");
  gpu_float({y, ggg}, "mix_dbl_bwd_grad_w");
  const Mix s{y.size(0), y.size(1), y.size(2), y.size(3), g_out.size(1)};
  mwt(s, g_out, y, ggg, out, 1);
  return out;
}

// grad_g2 = MGT(G, ggy, w) + MGT(G, y, ggw)
Tensor mix_dbl_bwd_grad_g(const Tensor& g_out, const Tensor& y, const Tensor& ggy, const Tensor& w, const Tensor& ggw) {
  Tensor out = mix_bucket_transpose_g(g_out, ggy, w);
  TORCH_CHECK(y.sizes() == ggy.sizes() && w.sizes() == ggw.sizes(), "y/ggy and w/ggw must have the same shapes");
  gpu_float({y, ggw}, "mix_dbl_bwd_grad_g");
  const Mix s = mix_sizes(y, w);
  mgt(s, g_out, y, ggw, out, 1);
  return out;
}

// ---------------------------------------------------------------- Meta (shapes only)
Tensor project_bucket_forward_meta(const Tensor& a, const Tensor&, const Tensor& u, int64_t num_paths) {
  TORCH_CHECK(num_paths > 0, "num_paths must be positive");
  return at::empty({a.size(0), num_paths, u.size(1) / num_paths, a.size(1)}, a.options());
}
Tensor project_bucket_transpose_a_meta(const Tensor& grad_y, const Tensor& b, const Tensor& u) {
  return at::empty({grad_y.size(0), grad_y.size(3) / b.size(1), u.size(0) / b.size(2)}, grad_y.options());
}
Tensor project_bucket_transpose_b_meta(const Tensor& grad_y, const Tensor& a, const Tensor& u) {
  return at::empty({grad_y.size(0), grad_y.size(3) / a.size(1), u.size(0) / a.size(2)}, grad_y.options());
}
Tensor project_bucket_transpose_u_meta(const Tensor& grad_y, const Tensor& a, const Tensor& b) {
  return at::empty({a.size(2) * b.size(2), grad_y.size(1) * grad_y.size(2)}, grad_y.options());
}
Tensor mix_bucket_forward_meta(const Tensor& y, const Tensor& w, const Tensor&) {
  return at::empty({y.size(0), w.size(1), y.size(2)}, y.options());
}
Tensor mix_bucket_transpose_y_meta(const Tensor& grad_out, const Tensor& w, const Tensor&) {
  return at::empty({grad_out.size(0), w.size(0), grad_out.size(2), w.size(2)}, grad_out.options());
}
Tensor mix_bucket_transpose_w_meta(const Tensor& grad_out, const Tensor& y, const Tensor&) {
  return at::empty({y.size(1), grad_out.size(1), y.size(3)}, y.options());
}
Tensor mix_bucket_transpose_g_meta(const Tensor&, const Tensor& y, const Tensor&) {
  return at::empty({y.size(0), y.size(1)}, y.options());
}
Tensor bucketed_tp_forward_meta(const Tensor& a, const Tensor&, const Tensor& u, const Tensor& w, const Tensor&) {
  return at::empty({a.size(0), w.size(1), u.size(1) / w.size(0)}, a.options());
}
Tensor project_dbl_bwd_grad_h_meta(const Tensor& a, const Tensor&, const Tensor&, const Tensor&, const Tensor& u,
                                   const Tensor&, int64_t num_paths) {
  return project_bucket_forward_meta(a, a, u, num_paths);
}
Tensor project_dbl_bwd_grad_a_meta(const Tensor& h, const Tensor& b, const Tensor&, const Tensor& u, const Tensor&) {
  return project_bucket_transpose_a_meta(h, b, u);
}
Tensor project_dbl_bwd_grad_b_meta(const Tensor& h, const Tensor& a, const Tensor&, const Tensor& u, const Tensor&) {
  return project_bucket_transpose_b_meta(h, a, u);
}
Tensor project_dbl_bwd_grad_u_meta(const Tensor& h, const Tensor& a, const Tensor&, const Tensor& b, const Tensor&) {
  return project_bucket_transpose_u_meta(h, a, b);
}
Tensor mix_dbl_bwd_grad_g_out_meta(const Tensor& y, const Tensor&, const Tensor& w, const Tensor&, const Tensor&,
                                   const Tensor&) {
  return mix_bucket_forward_meta(y, w, y);
}
Tensor mix_dbl_bwd_grad_y_meta(const Tensor& g_out, const Tensor& w, const Tensor&, const Tensor&, const Tensor&) {
  return mix_bucket_transpose_y_meta(g_out, w, w);
}
Tensor mix_dbl_bwd_grad_w_meta(const Tensor& g_out, const Tensor& y, const Tensor&, const Tensor&, const Tensor&) {
  return mix_bucket_transpose_w_meta(g_out, y, y);
}
Tensor mix_dbl_bwd_grad_g_meta(const Tensor&, const Tensor& y, const Tensor&, const Tensor&, const Tensor&) {
  return at::empty({y.size(0), y.size(1)}, y.options());
}

void refuse_cpu_bucket(const c10::OperatorHandle& op, torch::jit::Stack*) {
  TORCH_CHECK(false, op.schema().name(), ": the HIP kernels take GPU tensors (there is no CPU path)");
}

}  // namespace

TORCH_LIBRARY_FRAGMENT(fsctep, m) {
  m.def("project_bucket_forward(Tensor a, Tensor b, Tensor u_bucket, int num_paths) -> Tensor");
  m.def("project_bucket_transpose_a(Tensor grad_y, Tensor b, Tensor u_bucket) -> Tensor");
  m.def("project_bucket_transpose_b(Tensor grad_y, Tensor a, Tensor u_bucket) -> Tensor");
  m.def("project_bucket_transpose_u(Tensor grad_y, Tensor a, Tensor b) -> Tensor");
  m.def("mix_bucket_forward(Tensor y, Tensor w, Tensor gates) -> Tensor");
  m.def("mix_bucket_transpose_y(Tensor grad_out, Tensor w, Tensor gates) -> Tensor");
  m.def("mix_bucket_transpose_w(Tensor grad_out, Tensor y, Tensor gates) -> Tensor");
  m.def("mix_bucket_transpose_g(Tensor grad_out, Tensor y, Tensor w) -> Tensor");
  m.def("bucketed_tp_forward(Tensor a, Tensor b, Tensor u_bucket, Tensor w, Tensor gates) -> Tensor");
  m.def("project_dbl_bwd_grad_h(Tensor a, Tensor gga, Tensor b, Tensor ggb, Tensor u, Tensor ggu, int num_paths) "
        "-> Tensor");
  m.def("project_dbl_bwd_grad_a(Tensor h, Tensor b, Tensor ggb, Tensor u, Tensor ggu) -> Tensor");
  m.def("project_dbl_bwd_grad_b(Tensor h, Tensor a, Tensor gga, Tensor u, Tensor ggu) -> Tensor");
  m.def("project_dbl_bwd_grad_u(Tensor h, Tensor a, Tensor gga, Tensor b, Tensor ggb) -> Tensor");
  m.def("mix_dbl_bwd_grad_g_out(Tensor y, Tensor ggy, Tensor w, Tensor ggw, Tensor gates, Tensor ggg) -> Tensor");
  m.def("mix_dbl_bwd_grad_y(Tensor g_out, Tensor w, Tensor ggw, Tensor gates, Tensor ggg) -> Tensor");
  m.def("mix_dbl_bwd_grad_w(Tensor g_out, Tensor y, Tensor ggy, Tensor gates, Tensor ggg) -> Tensor");
  m.def("mix_dbl_bwd_grad_g(Tensor g_out, Tensor y, Tensor ggy, Tensor w, Tensor ggw) -> Tensor");
}

TORCH_LIBRARY_IMPL(fsctep, CUDA, m) {
  m.impl("project_bucket_forward", project_bucket_forward);
  m.impl("project_bucket_transpose_a", project_bucket_transpose_a);
  m.impl("project_bucket_transpose_b", project_bucket_transpose_b);
  m.impl("project_bucket_transpose_u", project_bucket_transpose_u);
  m.impl("mix_bucket_forward", mix_bucket_forward);
  m.impl("mix_bucket_transpose_y", mix_bucket_transpose_y);
  m.impl("mix_bucket_transpose_w", mix_bucket_transpose_w);
  m.impl("mix_bucket_transpose_g", mix_bucket_transpose_g);
  m.impl("bucketed_tp_forward", bucketed_tp_forward);
  m.impl("project_dbl_bwd_grad_h", project_dbl_bwd_grad_h);
  m.impl("project_dbl_bwd_grad_a", project_dbl_bwd_grad_a);
  m.impl("project_dbl_bwd_grad_b", project_dbl_bwd_grad_b);
  m.impl("project_dbl_bwd_grad_u", project_dbl_bwd_grad_u);
  m.impl("mix_dbl_bwd_grad_g_out", mix_dbl_bwd_grad_g_out);
  m.impl("mix_dbl_bwd_grad_y", mix_dbl_bwd_grad_y);
  m.impl("mix_dbl_bwd_grad_w", mix_dbl_bwd_grad_w);
  m.impl("mix_dbl_bwd_grad_g", mix_dbl_bwd_grad_g);
}

TORCH_LIBRARY_IMPL(fsctep, Meta, m) {
  m.impl("project_bucket_forward", project_bucket_forward_meta);
  m.impl("project_bucket_transpose_a", project_bucket_transpose_a_meta);
  m.impl("project_bucket_transpose_b", project_bucket_transpose_b_meta);
  m.impl("project_bucket_transpose_u", project_bucket_transpose_u_meta);
  m.impl("mix_bucket_forward", mix_bucket_forward_meta);
  m.impl("mix_bucket_transpose_y", mix_bucket_transpose_y_meta);
  m.impl("mix_bucket_transpose_w", mix_bucket_transpose_w_meta);
  m.impl("mix_bucket_transpose_g", mix_bucket_transpose_g_meta);
  m.impl("bucketed_tp_forward", bucketed_tp_forward_meta);
  m.impl("project_dbl_bwd_grad_h", project_dbl_bwd_grad_h_meta);
  m.impl("project_dbl_bwd_grad_a", project_dbl_bwd_grad_a_meta);
  m.impl("project_dbl_bwd_grad_b", project_dbl_bwd_grad_b_meta);
  m.impl("project_dbl_bwd_grad_u", project_dbl_bwd_grad_u_meta);
  m.impl("mix_dbl_bwd_grad_g_out", mix_dbl_bwd_grad_g_out_meta);
  m.impl("mix_dbl_bwd_grad_y", mix_dbl_bwd_grad_y_meta);
  m.impl("mix_dbl_bwd_grad_w", mix_dbl_bwd_grad_w_meta);
  m.impl("mix_dbl_bwd_grad_g", mix_dbl_bwd_grad_g_meta);
}

TORCH_LIBRARY_IMPL(fsctep, CPU, m) {
  for (const char* name : {"project_bucket_forward", "project_bucket_transpose_a", "project_bucket_transpose_b",
                           "project_bucket_transpose_u", "mix_bucket_forward", "mix_bucket_transpose_y",
                           "mix_bucket_transpose_w", "mix_bucket_transpose_g", "bucketed_tp_forward",
                           "project_dbl_bwd_grad_h", "project_dbl_bwd_grad_a", "project_dbl_bwd_grad_b",
                           "project_dbl_bwd_grad_u", "mix_dbl_bwd_grad_g_out", "mix_dbl_bwd_grad_y",
                           "mix_dbl_bwd_grad_w", "mix_dbl_bwd_grad_g"})
    m.impl(name, torch::CppFunction::makeFromBoxedFunction<&refuse_cpu_bucket>());
}
