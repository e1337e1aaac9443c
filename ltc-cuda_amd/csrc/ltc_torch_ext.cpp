// Torch glue for the fused module path: the layer's autograd Function in C++,
// around the C-ABI entry points ltc_module_forward / ltc_module_backward
// (include/ltc_capi.h). Same semantics as the Python LTCModuleFunction in
// ltc_cuda.py; doing the allocations, pointer plumbing and the backward node
// in C++ removes the per-step Python and ctypes overhead of the layer.
#include <torch/extension.h>

#include <c10/hip/HIPStream.h>

#include <array>
#include <cstdint>

#include "../../include/ltc_capi.h"

namespace {

using torch::Tensor;
using torch::autograd::AutogradContext;
using torch::autograd::variable_list;

constexpr int kLeaves = 17;  // w, erev, mask, mu, sigma, s_w, s_erev, s_mask, s_mu,
                             // s_sigma, gleak, vleak, cm, input_w, input_b, ln_w, ln_b

void check_rc(int rc, const char* what) {
  TORCH_CHECK(rc == LTC_OK, what, " failed (code ", rc, "): ", ltc_last_error());
}

float* fp(const Tensor& t) { return t.defined() ? t.data_ptr<float>() : nullptr; }

Tensor contig(const Tensor& t) { return t.is_contiguous() ? t : t.contiguous(); }

// 256-byte aligned device workspace carved from one byte tensor.
struct Workspace {
  Tensor buf;
  void* ptr;
};

Workspace workspace(long long bytes, const Tensor& like) {
  TORCH_CHECK(bytes >= 0, "unsupported LTC sizes");
  Workspace w;
  w.buf = at::empty({bytes + 256}, like.options().dtype(at::kByte));
  w.ptr = reinterpret_cast<void*>((reinterpret_cast<uintptr_t>(w.buf.data_ptr()) + 255) &
                                  ~uintptr_t(255));
  return w;
}

// `state` may be undefined: a zero initial state, read by no kernel.
void check_inputs(const Tensor& x, const Tensor& state, const std::array<Tensor, kLeaves>& lv) {
  TORCH_CHECK(x.dim() == 3, "x must be (B, T, D)");
  TORCH_CHECK(x.is_cuda() && x.scalar_type() == at::kFloat, "LTC HIP kernels are fp32-only");
  TORCH_CHECK(lv[0].dim() == 2, "w must be (H, H)");
  const int64_t D = x.size(2), H = lv[0].size(0);
  TORCH_CHECK(!state.defined() ||
                  (state.dim() == 2 && state.size(0) == x.size(0) && state.size(1) == H),
              "state must be (B, H)");
  const int64_t shapes[kLeaves][2] = {{H, H}, {H, H}, {H, H}, {H, H}, {H, H}, {D, H},
                                      {D, H}, {D, H}, {D, H}, {D, H}, {H, -1}, {H, -1},
                                      {H, -1}, {D, -1}, {D, -1}, {D, -1}, {D, -1}};
  for (int i = 0; i < kLeaves; ++i) {
    const Tensor& t = lv[i];
    TORCH_CHECK(t.scalar_type() == at::kFloat && t.device() == x.device(),
                "all LTC tensors must be fp32 on one device");
    const bool ok = shapes[i][1] < 0 ? (t.dim() == 1 && t.size(0) == shapes[i][0])
                                     : (t.dim() == 2 && t.size(0) == shapes[i][0] &&
                                        t.size(1) == shapes[i][1]);
    TORCH_CHECK(ok, "LTC parameter ", i, " has shape ", t.sizes());
  }
  TORCH_CHECK(!state.defined() ||
                  (state.scalar_type() == at::kFloat && state.device() == x.device()),
              "state must be fp32 on the device of x");
}

struct LTCModuleFn : public torch::autograd::Function<LTCModuleFn> {
  static variable_list forward(AutogradContext* ctx, Tensor x, Tensor state_in, Tensor w,
                               Tensor erev, Tensor mask, Tensor mu, Tensor sigma, Tensor s_w,
                               Tensor s_erev, Tensor s_mask, Tensor s_mu, Tensor s_sigma,
                               Tensor gleak, Tensor vleak, Tensor cm, Tensor input_w,
                               Tensor input_b, Tensor ln_w, Tensor ln_b, double dt, int64_t U,
                               double eps, double ln_eps, bool needs_grad) {
    std::array<Tensor, kLeaves> lv = {w,   erev,  mask,  mu,    sigma,   s_w,     s_erev,
                                      s_mask, s_mu, s_sigma, gleak, vleak, cm, input_w,
                                      input_b, ln_w, ln_b};
    // A 1-d empty state stands for "no initial state" (zeros): autograd
    // Functions take only defined tensors.
    const Tensor state = state_in.dim() == 1 && state_in.numel() == 0 ? Tensor() : state_in;
    check_inputs(x, state, lv);
    // Undefined output gradients stay undefined (no zero-filled tensors).
    ctx->set_materialize_grads(false);
    for (auto& t : lv) t = contig(t);
    const Tensor st = state.defined() ? contig(state) : Tensor();
    const int B = (int)x.size(0), T = (int)x.size(1), D = (int)x.size(2), H = (int)lv[0].size(0);
    const auto opts = x.options();
    Tensor out = at::empty({B, T, H}, opts);
    Tensor h = at::empty({B, H}, opts);
    Tensor saved;
    if (needs_grad) {
      const long long n = ltc_module_saved_floats(B, T, D, H, (int)U);
      TORCH_CHECK(n >= 0, "unsupported LTC sizes");
      saved = at::empty({n > 0 ? n : 1}, opts);
    }
    const Workspace ws = workspace(ltc_module_fwd_workspace_bytes(B, T, D, H, (int)U), x);
    const hipStream_t stream = c10::hip::getCurrentHIPStream(x.device().index()).stream();
    check_rc(ltc_module_forward(fp(x), x.stride(0), x.stride(1), x.stride(2), fp(st),
                                fp(lv[0]), fp(lv[1]), fp(lv[2]), fp(lv[3]), fp(lv[4]), fp(lv[5]),
                                fp(lv[6]), fp(lv[7]), fp(lv[8]), fp(lv[9]), fp(lv[10]),
                                fp(lv[11]), fp(lv[12]), fp(lv[13]), fp(lv[14]), fp(lv[15]),
                                fp(lv[16]), B, T, D, H, (int)U, (float)dt, (float)eps,
                                (float)ln_eps, needs_grad ? 1 : 0, fp(out), fp(h), fp(saved),
                                ws.ptr, ws.buf.numel() - 256, stream),
             "ltc_module_forward");
    if (needs_grad) {
      std::vector<Tensor> keep = {x, st};
      keep.insert(keep.end(), lv.begin(), lv.end());
      keep.push_back(saved);
      ctx->save_for_backward(keep);
    }
    ctx->saved_data["dt"] = dt;
    ctx->saved_data["U"] = U;
    ctx->saved_data["eps"] = eps;
    ctx->saved_data["ln_eps"] = ln_eps;
    return {out, h};
  }

  static variable_list backward(AutogradContext* ctx, variable_list grads) {
    const auto sv = ctx->get_saved_variables();
    TORCH_CHECK(sv.size() == 2 + kLeaves + 1,
                "LTC backward called on a forward run without grad");
    const Tensor& x = sv[0];
    const Tensor& st = sv[1];
    const Tensor& saved = sv[2 + kLeaves];
    const double dt = ctx->saved_data["dt"].toDouble();
    const int U = (int)ctx->saved_data["U"].toInt();
    const double eps = ctx->saved_data["eps"].toDouble();
    const double ln_eps = ctx->saved_data["ln_eps"].toDouble();
    const int B = (int)x.size(0), T = (int)x.size(1), D = (int)x.size(2);
    const int H = (int)sv[2].size(0);
    const auto opts = x.options();
    Tensor go = grads[0].defined() ? grads[0] : at::zeros({B, T, H}, opts);
    if (go.scalar_type() != at::kFloat) go = go.to(at::kFloat);
    Tensor gh;
    if (grads[1].defined()) gh = contig(grads[1].to(at::kFloat));
    // All gradients in one allocation: x, state (when it was given), 4 (H,H),
    // 4 (D,H), 3 (H), 4 (D), each a contiguous view (as_strided: one op each).
    const int64_t nx = (int64_t)B * T * D, nst = st.defined() ? (int64_t)B * H : 0,
                  nhh = (int64_t)H * H, ndh = (int64_t)D * H;
    Tensor flat = at::empty({nx + nst + 4 * nhh + 4 * ndh + 3 * H + 4 * D}, opts);
    int64_t off = 0;
    auto take3 = [&](int64_t a, int64_t b, int64_t c) {
      Tensor t = flat.as_strided({a, b, c}, {b * c, c, 1}, off);
      off += a * b * c;
      return t;
    };
    auto take2 = [&](int64_t a, int64_t b) {
      Tensor t = flat.as_strided({a, b}, {b, 1}, off);
      off += a * b;
      return t;
    };
    auto take1 = [&](int64_t a) {
      Tensor t = flat.as_strided({a}, {1}, off);
      off += a;
      return t;
    };
    Tensor gx = take3(B, T, D);
    Tensor gst = st.defined() ? take2(B, H) : Tensor();
    Tensor gw = take2(H, H), gerev = take2(H, H), gmu = take2(H, H), gsig = take2(H, H);
    Tensor gsw = take2(D, H), gserev = take2(D, H), gsmu = take2(D, H), gssig = take2(D, H);
    Tensor ggl = take1(H), gvl = take1(H), gcm = take1(H);
    Tensor giw = take1(D), gib = take1(D), glw = take1(D), glb = take1(D);
    const Workspace ws = workspace(ltc_module_bwd_workspace_bytes(B, T, D, H, U), x);
    const hipStream_t stream = c10::hip::getCurrentHIPStream(x.device().index()).stream();
    const Tensor* lv = &sv[2];
    check_rc(ltc_module_backward(
                 fp(x), x.stride(0), x.stride(1), x.stride(2), fp(lv[0]), fp(lv[1]), fp(lv[2]),
                 fp(lv[3]), fp(lv[4]), fp(lv[5]), fp(lv[6]), fp(lv[7]), fp(lv[8]), fp(lv[9]),
                 fp(lv[10]), fp(lv[11]), fp(lv[12]), fp(lv[13]), fp(lv[14]), fp(lv[15]),
                 fp(lv[16]), fp(saved), fp(go), go.stride(0), go.stride(1), go.stride(2), fp(gh),
                 B, T, D, H, U, (float)dt, (float)eps, (float)ln_eps, fp(gx), fp(gst), fp(gw),
                 fp(gerev), fp(gmu), fp(gsig), fp(gsw), fp(gserev), fp(gsmu), fp(gssig), fp(ggl),
                 fp(gvl), fp(gcm), fp(giw), fp(gib), fp(glw), fp(glb), ws.ptr,
                 ws.buf.numel() - 256, stream),
             "ltc_module_backward");
    const Tensor none;
    return {gx,   gst,  gw,  gerev, none, gmu,  gsig, gsw,  gserev, none, gsmu, gssig,
            ggl,  gvl,  gcm, giw,   gib,  glw,  glb,  none, none,   none, none, none};
  }
};

// Whole-layer fused call: leaves in the order of kLeaves above.
// `state` None means a zero initial state (passed on as a 1-d empty tensor).
std::vector<Tensor> module_apply(const Tensor& x, const c10::optional<Tensor>& state,
                                 const std::vector<Tensor>& lv, double dt, int64_t U,
                                 double eps, double ln_eps) {
  TORCH_CHECK(lv.size() == kLeaves, "expected ", kLeaves, " LTC leaves");
  const bool needs_grad = torch::GradMode::is_enabled();
  const Tensor st = state.has_value() ? *state : at::empty({0}, x.options());
  auto r = LTCModuleFn::apply(x, st, lv[0], lv[1], lv[2], lv[3], lv[4], lv[5], lv[6], lv[7],
                              lv[8], lv[9], lv[10], lv[11], lv[12], lv[13], lv[14], lv[15],
                              lv[16], dt, U, eps, ln_eps, needs_grad);
  return {r[0], r[1]};
}

}  // namespace

PYBIND11_MODULE(TORCH_EXTENSION_NAME, m) {
  m.doc() = "LTC fused module path: autograd Function over libltc_hip.so";
  m.def("module_apply", &module_apply, "Fused LTC layer forward (autograd-aware)");
  m.def("abi_version", &ltc_abi_version, "ABI version of the loaded libltc_hip.so");
}
