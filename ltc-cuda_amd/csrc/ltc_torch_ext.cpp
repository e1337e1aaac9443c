// Torch glue for the fused module path: the layer's autograd node in C++,
// around the C-ABI entry points ltc_module_forward / ltc_module_backward
// (include/ltc_capi.h). Same semantics as the Python LTCModuleFunction in
// ltc_cuda.py; doing the allocations, pointer plumbing and the backward node
// in C++ removes the per-step Python and ctypes overhead of the layer.
//
// The backward is a plain autograd Node (as torch's own operators have),
// not a torch::autograd::Function: that skips the Function machinery's
// context object, its saved-data map and its per-output bookkeeping, which
// cost several microseconds per step of a small layer.
#include <torch/extension.h>
#include <torch/csrc/autograd/function.h>
#include <torch/csrc/autograd/functions/utils.h>
#include <torch/csrc/autograd/saved_variable.h>

#include <c10/hip/HIPStream.h>

#include <array>
#include <cstdint>

#include "../../include/ltc_capi.h"

namespace {

using torch::Tensor;
using torch::autograd::Node;
using torch::autograd::SavedVariable;
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
void check_inputs(const Tensor& x, const Tensor& state, const std::vector<Tensor>& lv) {
  TORCH_CHECK(lv.size() == kLeaves, "expected ", kLeaves, " LTC leaves");
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

// Backward node of one fused layer call. Its next edges are, in order, x, the
// initial state (an empty edge when none was given) and the 17 leaves; the
// gradients it returns follow that order (none for the two masks). It keeps
// x, the leaves as the caller passed them and the saved buffer (which holds
// the initial state), version-checked when unpacked, as save_for_backward
// would: a leaf edited in place between forward and backward is an error.
struct LTCModuleBackward : public Node {
  std::vector<SavedVariable> sv;  // x, 17 leaves, saved
  bool has_state = false;
  double dt = 0, eps = 0, ln_eps = 0;
  int U = 0;

  std::string name() const override { return "LTCModuleBackward"; }
  void release_variables() override {
    for (auto& s : sv) s.reset_data();
  }
  variable_list apply(variable_list&& grads) override;
};

// Gradient views into one allocation: plain tensors over the allocation's
// storage, built directly (no view op per gradient).
struct FlatCarver {
  const Tensor& flat;
  int64_t off = 0;
  Tensor take(std::initializer_list<int64_t> sz, std::initializer_list<int64_t> st, int64_t n) {
    auto impl = c10::make_intrusive<c10::TensorImpl>(c10::Storage(flat.storage()),
                                                     flat.key_set(), flat.dtype());
    impl->set_sizes_and_strides(sz, st, off);
    off += n;
    return Tensor(std::move(impl));
  }
};

variable_list LTCModuleBackward::apply(variable_list&& grads) {
  std::array<Tensor, 1 + kLeaves + 1> t;
  for (size_t i = 0; i < t.size(); ++i) t[i] = sv[i].unpack();
  const Tensor& x = t[0];
  // the leaves as the caller gave them; a non-contiguous one is copied again
  // for the kernels, as the forward did
  for (int i = 1; i <= kLeaves; ++i) t[i] = contig(t[i]);
  const Tensor* lv = &t[1];
  const Tensor& saved = t[1 + kLeaves];
  const int B = (int)x.size(0), T = (int)x.size(1), D = (int)x.size(2);
  const int H = (int)lv[0].size(0);
  const auto opts = x.options();
  Tensor go = grads[0].defined() ? grads[0] : at::zeros({B, T, H}, opts);
  if (go.scalar_type() != at::kFloat) go = go.to(at::kFloat);
  Tensor gh;
  if (grads[1].defined()) gh = contig(grads[1].to(at::kFloat));
  // All gradients in one allocation: x, state (when it was given), 4 (H,H),
  // 4 (D,H), 3 (H), 4 (D), each a contiguous view.
  const int64_t nx = (int64_t)B * T * D, nst = has_state ? (int64_t)B * H : 0,
                nhh = (int64_t)H * H, ndh = (int64_t)D * H;
  const Tensor flat = at::empty({nx + nst + 4 * nhh + 4 * ndh + 3 * H + 4 * D}, opts);
  FlatCarver c{flat};
  Tensor gx = c.take({B, T, D}, {(int64_t)T * D, D, 1}, nx);
  Tensor gst = has_state ? c.take({B, H}, {H, 1}, nst) : Tensor();
  Tensor gw = c.take({H, H}, {H, 1}, nhh), gerev = c.take({H, H}, {H, 1}, nhh);
  Tensor gmu = c.take({H, H}, {H, 1}, nhh), gsig = c.take({H, H}, {H, 1}, nhh);
  Tensor gsw = c.take({D, H}, {H, 1}, ndh), gserev = c.take({D, H}, {H, 1}, ndh);
  Tensor gsmu = c.take({D, H}, {H, 1}, ndh), gssig = c.take({D, H}, {H, 1}, ndh);
  Tensor ggl = c.take({H}, {1}, H), gvl = c.take({H}, {1}, H), gcm = c.take({H}, {1}, H);
  Tensor giw = c.take({D}, {1}, D), gib = c.take({D}, {1}, D);
  Tensor glw = c.take({D}, {1}, D), glb = c.take({D}, {1}, D);
  const Workspace ws = workspace(ltc_module_bwd_workspace_bytes(B, T, D, H, U), x);
  const hipStream_t stream = c10::hip::getCurrentHIPStream(x.device().index()).stream();
  check_rc(ltc_module_backward(
               fp(x), x.stride(0), x.stride(1), x.stride(2), fp(lv[0]), fp(lv[1]), fp(lv[2]),
               fp(lv[3]), fp(lv[4]), fp(lv[5]), fp(lv[6]), fp(lv[7]), fp(lv[8]), fp(lv[9]),
               fp(lv[10]), fp(lv[11]), fp(lv[12]), fp(lv[13]), fp(lv[14]), fp(lv[15]),
               fp(lv[16]), fp(saved), fp(go), go.stride(0), go.stride(1), go.stride(2), fp(gh), B,
               T, D, H, U, (float)dt, (float)eps, (float)ln_eps, fp(gx), fp(gst), fp(gw),
               fp(gerev), fp(gmu), fp(gsig), fp(gsw), fp(gserev), fp(gsmu), fp(gssig), fp(ggl),
               fp(gvl), fp(gcm), fp(giw), fp(gib), fp(glw), fp(glb), ws.ptr,
               ws.buf.numel() - 256, stream),
           "ltc_module_backward");
  const Tensor none;
  return {gx,   gst, gw,  gerev, none, gmu, gsig, gsw, gserev, none,
          gsmu, gssig, ggl, gvl, gcm, giw, gib, glw, glb};
}

// Whole-layer fused call: leaves in the order of kLeaves above.
// `state` None means a zero initial state.
std::vector<Tensor> module_apply(const Tensor& x, const c10::optional<Tensor>& state_opt,
                                 const std::vector<Tensor>& leaves, double dt, int64_t U,
                                 double eps, double ln_eps) {
  const Tensor state = state_opt.has_value() ? *state_opt : Tensor();
  check_inputs(x, state, leaves);
  const bool needs_grad = torch::GradMode::is_enabled() &&
                          torch::autograd::compute_requires_grad(x, state, leaves);
  const int B = (int)x.size(0), T = (int)x.size(1), D = (int)x.size(2);
  const int H = (int)leaves[0].size(0);
  Tensor out, h, saved;
  std::array<Tensor, kLeaves> lv;
  Tensor st;
  {
    // the kernels' inputs and outputs are made outside autograd
    at::AutoDispatchBelowADInplaceOrView guard;
    for (int i = 0; i < kLeaves; ++i) lv[i] = contig(leaves[i]);
    st = state.defined() ? contig(state) : Tensor();
    const auto opts = x.options();
    out = at::empty({B, T, H}, opts);
    h = at::empty({B, H}, opts);
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
  }
  if (needs_grad) {
    auto node = std::shared_ptr<LTCModuleBackward>(new LTCModuleBackward(),
                                                   torch::autograd::deleteNode);
    node->set_next_edges(torch::autograd::collect_next_edges(x, state, leaves));
    node->sv.reserve(1 + kLeaves + 1);
    node->sv.emplace_back(x, false);
    for (const Tensor& t : leaves) node->sv.emplace_back(t, false);
    node->sv.emplace_back(saved, false);
    node->has_state = state.defined();
    node->dt = dt;
    node->eps = eps;
    node->ln_eps = ln_eps;
    node->U = (int)U;
    torch::autograd::set_history(out, node);
    torch::autograd::set_history(h, node);
  }
  return {out, h};
}

}  // namespace

PYBIND11_MODULE(TORCH_EXTENSION_NAME, m) {
  m.doc() = "LTC fused module path: autograd node over libltc_hip.so";
  m.def("module_apply", &module_apply, "Fused LTC layer forward (autograd-aware)");
  m.def("abi_version", &ltc_abi_version, "ABI version of the loaded libltc_hip.so");
}
