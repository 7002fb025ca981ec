// autograd.cpp — C++ autograd bindings of the SSD and GLA scans for PyTorch
// (module mlx_recurrence_amd._autograd).
//
// The same forward / backward as the Python torch.autograd.Functions of
// ssd.py and gla.py (the counterparts of the reference's mx.custom_function
// VJPs, reference ssd.py:314-341 and gla.py:277-300), written against the
// C ABI of librecurrence_gfx950.so: input preparation, output / workspace
// allocation, the kernel calls and the saved state live in one
// torch::autograd::Function, so an eager training step pays one C++ autograd
// node per scan instead of the Python Function machinery.  Argument
// validation (the reference's ValueError texts) stays in Python, before the
// call.
#include <torch/extension.h>

#include <c10/core/DeviceGuard.h>
#include <c10/hip/HIPStream.h>

#include <cstdint>
#include <string>

#include "../../include/recurrence.h"

namespace {

using at::Tensor;
using torch::autograd::AutogradContext;
using torch::autograd::variable_list;

int dtype_code(at::ScalarType t) {
  switch (t) {
    case at::kFloat: return RR_F32;
    case at::kBFloat16: return RR_BF16;
    case at::kHalf: return RR_F16;
    default: TORCH_CHECK(false, "unsupported input dtype ", t, "; use float32, bfloat16 or float16");
  }
}

// The dtype the kernels run on for these inputs (mlx_recurrence_amd._lib.common_dtype).
at::ScalarType common_dtype(std::initializer_list<const Tensor*> ts) {
  at::ScalarType dt = (*ts.begin())->scalar_type();
  for (const Tensor* t : ts) dt = at::promote_types(dt, t->scalar_type());
  if (dt != at::kFloat && dt != at::kBFloat16 && dt != at::kHalf) {
    if (!at::isFloatingType(dt)) throw pybind11::type_error("unsupported input dtype; use float32, bfloat16 or float16");
    dt = at::kFloat;
  }
  return dt;
}

// Contiguous, 16-byte aligned, of dtype dt (mlx_recurrence_amd._lib.prep).
Tensor prep(const Tensor& t, at::ScalarType dt) {
  Tensor r = t.scalar_type() == dt ? t : t.to(dt);
  if (!r.is_contiguous()) r = r.contiguous();
  if (reinterpret_cast<uintptr_t>(r.data_ptr()) % 16 != 0) r = r.clone();
  return r;
}

void require_device(std::initializer_list<const Tensor*> ts) {
  c10::optional<at::Device> dev;
  for (const Tensor* t : ts) {
    if (!t->defined()) continue;
    TORCH_CHECK(t->is_cuda(), "mlx_recurrence_amd kernels run on a ROCm GPU; got a tensor on ", t->device(),
                " (use the *_scan_reference functions for CPU tensors)");
    if (!dev) dev = t->device();
    TORCH_CHECK(*dev == t->device(), "all tensors must be on one device, got ", *dev, " and ", t->device());
  }
}

void* P(const Tensor& t) { return t.defined() ? t.data_ptr() : nullptr; }
const float* PF(const Tensor& t) { return t.defined() ? t.data_ptr<float>() : nullptr; }
float* MF(const Tensor& t) { return t.defined() ? t.data_ptr<float>() : nullptr; }

void* stream_of(const Tensor& t) { return c10::hip::getCurrentHIPStream(t.device().index()).stream(); }

// Error codes to Python exceptions as mlx_recurrence_amd._lib._check does.
void check(int rc, const char* what) {
  if (rc == RR_OK) return;
  const std::string msg = rr_last_error();
  if (rc == RR_EINVAL || rc == RR_EWORKSPACE) throw pybind11::value_error(std::string(what) + ": " + msg);
  throw std::runtime_error(std::string(what) + " failed (code " + std::to_string(rc) + "): " + msg);
}

// The outputs of one pass that the caller receives together (the backward's
// gradients) carved out of a single allocation (one caching-allocator call
// instead of one per buffer): tensors are strided views of it.  Pieces start
// 256-byte aligned.  The workspace and the forward's checkpoints are separate
// allocations, so that the workspace is released (stream-ordered) when the
// pass returns and the checkpoints live exactly as long as the autograd node
// that saved them, whatever the caller keeps of y or of the gradients.
class Arena {
 public:
  // reserve a piece of `bytes`; returns its byte offset
  int64_t reserve(int64_t bytes) {
    const int64_t off = total_;
    total_ += (bytes + 255) / 256 * 256;
    return off;
  }
  void allocate(const at::TensorOptions& opts, at::ScalarType dt) {
    esize_ = (int64_t)c10::elementSize(dt);
    buf_ = at::empty({(total_ + esize_ - 1) / esize_}, opts.dtype(dt));
  }
  // a contiguous tensor of the arena's dtype at byte offset `off`
  Tensor view(int64_t off, at::IntArrayRef sizes) const {
    return buf_.as_strided(sizes, c10::contiguous_strides(sizes), off / esize_);
  }
  void* ptr(int64_t off) const { return static_cast<char*>(buf_.data_ptr()) + off; }

 private:
  int64_t total_ = 0, esize_ = 1;
  Tensor buf_;
};

// A pass's workspace: `bytes` of device memory (undefined when 0), released to
// the caching allocator when the tensor goes out of scope; the allocator
// reuses the block only for work ordered after this pass on the stream.
Tensor workspace(size_t bytes, const at::TensorOptions& opts) {
  return bytes ? at::empty({(int64_t)bytes}, opts.dtype(at::kByte)) : Tensor();
}

int64_t numel(at::IntArrayRef sizes) {
  int64_t n = 1;
  for (int64_t v : sizes) n *= v;
  return n;
}

// ------------------------------------------------------------------ SSD
// A_neg as passed by the caller: [H] (one rate per head), [H, N] with stride 0
// along N (a broadcast per-head rate) or a dense [H, N].  The kernels take
// the per-head vector (a_sn = 0) or the dense array (a_sn = 1); the gradient
// has A_neg's shape.
struct SSDFn : public torch::autograd::Function<SSDFn> {
  static variable_list forward(AutogradContext* ctx, const Tensor& u, const Tensor& delta, const Tensor& Bm,
                               const Tensor& Cm, const Tensor& A_neg, const c10::optional<Tensor>& h0opt,
                               int64_t seg) {
    const Tensor h0 = h0opt.has_value() ? *h0opt : Tensor();
    require_device({&u, &delta, &Bm, &Cm, &A_neg, &h0});
    const at::DeviceGuard guard(u.device());
    const at::ScalarType dt = common_dtype({&u, &delta, &Bm, &Cm});
    const Tensor u_ = prep(u, dt), d_ = prep(delta, dt), B_ = prep(Bm, dt), C_ = prep(Cm, dt);
    const int64_t Bsz = u_.size(0), L = u_.size(1), H = u_.size(2), Dh = u_.size(3), N = B_.size(3);
    int64_t a_sn = 1;
    Tensor A_;
    if (A_neg.dim() == 1) {
      A_ = prep(A_neg, at::kFloat), a_sn = 0;
    } else if (A_neg.size(1) > 1 && A_neg.stride(1) == 0) {
      A_ = prep(A_neg.select(1, 0), at::kFloat), a_sn = 0;
    } else {
      A_ = prep(A_neg, at::kFloat);
    }
    const Tensor h0_ = h0.defined() ? prep(h0, at::kFloat) : Tensor();
    const int64_t nC = L / rr_chunk_len(L, seg);
    const size_t wsb = rr_ssd_workspace_bytes(Bsz, L, H, Dh, N, seg, a_sn, dtype_code(dt), 0);
    const auto f32 = u_.options().dtype(at::kFloat);
    Tensor y = at::empty({Bsz, L, H, Dh}, f32), ckpt = at::empty({Bsz, H, nC, Dh, N}, f32);
    const Tensor ws = workspace(wsb, u_.options());
    check(rr_ssd_fwd(P(u_), P(d_), P(B_), P(C_), PF(A_), a_sn, dtype_code(dt), Bsz, L, H, Dh, N, seg, PF(h0_),
                     MF(y), MF(ckpt), P(ws), wsb, stream_of(u_)),
          "rr_ssd_fwd");
    ctx->save_for_backward({u_, d_, B_, C_, A_, h0_, ckpt});
    ctx->saved_data["seg"] = seg;
    ctx->saved_data["a_sn"] = a_sn;
    ctx->saved_data["a_dim"] = (int64_t)A_neg.dim();
    ctx->saved_data["has_h0"] = h0.defined();
    ctx->set_materialize_grads(false);
    return {y, ckpt.select(2, nC - 1)};
  }

  static variable_list backward(AutogradContext* ctx, variable_list grads) {
    const variable_list s = ctx->get_saved_variables();
    const Tensor &u_ = s[0], &d_ = s[1], &B_ = s[2], &C_ = s[3], &A_ = s[4], &h0_ = s[5], &ckpt = s[6];
    const at::DeviceGuard guard(u_.device());
    const int64_t seg = ctx->saved_data["seg"].toInt(), a_sn = ctx->saved_data["a_sn"].toInt();
    const int64_t Bsz = u_.size(0), L = u_.size(1), H = u_.size(2), Dh = u_.size(3), N = B_.size(3);
    const auto f32 = u_.options().dtype(at::kFloat);
    const Tensor dy = grads[0].defined() ? prep(grads[0], at::kFloat) : at::zeros({Bsz, L, H, Dh}, f32);
    const Tensor dfinal = grads[1].defined() ? prep(grads[1], at::kFloat) : Tensor();
    // (autograd edges exist only for the tensors passed: h0, when given, is the sixth)
    const bool want_dh0 = ctx->saved_data["has_h0"].toBool() && ctx->needs_input_grad(5);
    Tensor dh0 = want_dh0 ? at::empty({Bsz, H, Dh, N}, f32) : Tensor();
    const at::ScalarType dt = u_.scalar_type();
    const int64_t es = (int64_t)c10::elementSize(dt);
    const int dtc = dtype_code(dt);
    const size_t wsb = rr_ssd_workspace_bytes(Bsz, L, H, Dh, N, seg, a_sn, dtc, 1);
    const bool heads = ctx->saved_data["a_dim"].toInt() == 1;   // A_neg [H]: its gradient sums dA over n
    Arena ar;   // du, ddelta, dB, dC in the inputs' dtype
    const int64_t odu = ar.reserve(u_.numel() * es), odd = ar.reserve(d_.numel() * es);
    const int64_t odB = ar.reserve(B_.numel() * es), odC = ar.reserve(C_.numel() * es);
    ar.allocate(u_.options(), dt);
    const Tensor ws = workspace(wsb, u_.options());
    Tensor du = ar.view(odu, u_.sizes()), dd = ar.view(odd, d_.sizes());
    Tensor dB = ar.view(odB, B_.sizes()), dC = ar.view(odC, C_.sizes());
    // A_neg [H]: the library sums the gradient over n itself (dA_stride_n 0)
    Tensor dA = heads ? at::empty({H}, f32) : at::empty({H, N}, f32);
    check(rr_ssd_bwd(PF(dy), PF(dfinal), P(u_), P(d_), P(B_), P(C_), PF(A_), a_sn, dtc, Bsz, L, H, Dh, N, seg,
                     PF(h0_), PF(ckpt), P(du), P(dd), P(dB), P(dC), MF(dA), heads ? 0 : 1, MF(dh0), P(ws), wsb,
                     stream_of(u_)),
          "rr_ssd_bwd");
    return {du, dd, dB, dC, dA, dh0, Tensor()};
  }
};

std::tuple<Tensor, Tensor> ssd_scan(const Tensor& u, const Tensor& delta, const Tensor& Bm, const Tensor& Cm,
                                    const Tensor& A_neg, const c10::optional<Tensor>& h0, int64_t seg) {
  const variable_list out = SSDFn::apply(u, delta, Bm, Cm, A_neg, h0, seg);
  return {out[0], out[1]};
}

// ------------------------------------------------------------------ GLA
struct GLAFn : public torch::autograd::Function<GLAFn> {
  static variable_list forward(AutogradContext* ctx, const Tensor& q, const Tensor& k, const Tensor& v,
                               const Tensor& gates, const c10::optional<Tensor>& h0opt, int64_t seg) {
    const Tensor h0 = h0opt.has_value() ? *h0opt : Tensor();
    require_device({&q, &k, &v, &gates, &h0});
    const at::DeviceGuard guard(q.device());
    const at::ScalarType dt = common_dtype({&q, &k, &v, &gates});
    const Tensor q_ = prep(q, dt), k_ = prep(k, dt), v_ = prep(v, dt), g_ = prep(gates, dt);
    const int64_t B = q_.size(0), L = q_.size(1), H = q_.size(2), Dh = q_.size(3);
    const Tensor h0_ = h0.defined() ? prep(h0, at::kFloat) : Tensor();
    const int64_t nC = L / rr_chunk_len(L, seg);
    const size_t wsb = rr_gla_workspace_bytes(B, L, H, Dh, seg, dtype_code(dt), 0);
    const auto f32 = q_.options().dtype(at::kFloat);
    Tensor y = at::empty({B, L, H, Dh}, f32), ckpt = at::empty({B, H, nC, Dh, Dh}, f32);
    const Tensor ws = workspace(wsb, q_.options());
    check(rr_gla_fwd(P(q_), P(k_), P(v_), P(g_), dtype_code(dt), B, L, H, Dh, seg, PF(h0_), MF(y), MF(ckpt),
                     P(ws), wsb, stream_of(q_)),
          "rr_gla_fwd");
    ctx->save_for_backward({q_, k_, v_, g_, h0_, ckpt});
    ctx->saved_data["seg"] = seg;
    ctx->saved_data["has_h0"] = h0.defined();
    ctx->set_materialize_grads(false);
    // checkpoints hold S[i, j] with i fastest ([.., j, i]); the state is [.., i, j]
    return {y, ckpt.select(2, nC - 1).transpose(-1, -2)};
  }

  static variable_list backward(AutogradContext* ctx, variable_list grads) {
    const variable_list s = ctx->get_saved_variables();
    const Tensor &q_ = s[0], &k_ = s[1], &v_ = s[2], &g_ = s[3], &h0_ = s[4], &ckpt = s[5];
    const at::DeviceGuard guard(q_.device());
    const int64_t seg = ctx->saved_data["seg"].toInt();
    const int64_t B = q_.size(0), L = q_.size(1), H = q_.size(2), Dh = q_.size(3);
    const auto f32 = q_.options().dtype(at::kFloat);
    const Tensor dy = grads[0].defined() ? prep(grads[0], at::kFloat) : at::zeros({B, L, H, Dh}, f32);
    const Tensor dfinal = grads[1].defined() ? prep(grads[1], at::kFloat) : Tensor();
    // (autograd edges exist only for the tensors passed: h0, when given, is the fifth)
    const bool want_dh0 = ctx->saved_data["has_h0"].toBool() && ctx->needs_input_grad(4);
    Tensor dh0 = want_dh0 ? at::empty({B, H, Dh, Dh}, f32) : Tensor();
    const at::ScalarType dt = q_.scalar_type();
    const int64_t es = (int64_t)c10::elementSize(dt);
    const int dtc = dtype_code(dt);
    const size_t wsb = rr_gla_workspace_bytes(B, L, H, Dh, seg, dtc, 1);
    Arena ar;   // dq, dk, dv, dgates in the inputs' dtype
    const int64_t n4 = q_.numel() * es;
    const int64_t odq = ar.reserve(n4), odk = ar.reserve(n4), odv = ar.reserve(n4), odg = ar.reserve(g_.numel() * es);
    ar.allocate(q_.options(), dt);
    const Tensor ws = workspace(wsb, q_.options());
    Tensor dq = ar.view(odq, q_.sizes()), dk = ar.view(odk, k_.sizes()), dv = ar.view(odv, v_.sizes());
    Tensor dg = ar.view(odg, g_.sizes());
    check(rr_gla_bwd(PF(dy), PF(dfinal), P(q_), P(k_), P(v_), P(g_), dtc, B, L, H, Dh, seg, PF(h0_), PF(ckpt), P(dq),
                     P(dk), P(dv), P(dg), MF(dh0), P(ws), wsb, stream_of(q_)),
          "rr_gla_bwd");
    return {dq, dk, dv, dg, dh0, Tensor()};
  }
};

std::tuple<Tensor, Tensor> gla_scan(const Tensor& q, const Tensor& k, const Tensor& v, const Tensor& gates,
                                    const c10::optional<Tensor>& h0, int64_t seg) {
  const variable_list out = GLAFn::apply(q, k, v, gates, h0, seg);
  return {out[0], out[1]};
}

}  // namespace

PYBIND11_MODULE(_autograd, m) {
  m.doc() = "C++ autograd bindings of the gfx950 SSD and GLA scans";
  m.def("ssd_scan", &ssd_scan, "SSD scan (y, final state) as one C++ autograd node");
  m.def("gla_scan", &gla_scan, "GLA scan (y, final state) as one C++ autograd node");
  // the header revision this module was compiled against (not the loaded
  // library's, which the Python loader compares it with)
  m.def("abi_version", [] { return RR_ABI_VERSION; });
}
