// OverlayEmb's differentiable gather (engraft/replica/seq.py:372-444: the
// base gather with the variables' rows put in, and the backward that sums the
// output gradient into the variables) as a C++ autograd function over the
// library's two entry points, eg_gather_slots and eg_scatter_grad_apply.
//
// The same two launches as a Python torch.autograd.Function, without the
// interpreter on either side of them: the forward's argument checks and the
// backward, which the autograd engine runs on its device thread, take no GIL.
// Host code only (built with g++ against torch's headers); the entry points
// are the library's own, handed over as addresses by `init` from the library
// that the package has loaded, so both sides share its state.
#include <torch/extension.h>

#include <cstdint>
#include <stdexcept>
#include <string>

#include "engraft_ngram.h"

namespace {

using GatherFn = int (*)(const eg_table*, const int32_t*, const int32_t*, int64_t, int32_t, const float*, int64_t,
                         float*, void*);
using ScatterFn = int (*)(const void*, int32_t, int64_t, int32_t, int32_t, int64_t, float*, int32_t, void*, size_t,
                          void*);
using ErrorFn = const char* (*)();

GatherFn g_gather = nullptr;
ScatterFn g_scatter = nullptr;
ErrorFn g_error = nullptr;

// An entry point's status as the ctypes path raises it: EG_ERR_ARG a
// ValueError, any other error a RuntimeError, with eg_last_error's text.
void check(int rc) {
  if (rc == EG_OK) return;
  std::string msg = g_error != nullptr ? g_error() : "";
  if (rc == EG_ERR_ARG) throw std::invalid_argument(msg);
  throw std::runtime_error("engraft-ngram error " + std::to_string(rc) + ": " + msg);
}

// out f32 [n, heads * dim] = per slot vars[slot_var] (slot_var >= 0) or the
// table row; backward: d vars [n_var, dim] = the output gradient's slot slices
// summed per variable from the plan's grouping `ws` (eg_scatter_grad_plan_slots;
// empty when no gradient is wanted, or when there are no slots).  Both
// launches go to `stream`, the forward's stream (torch runs a backward node on
// its forward's stream).
struct GatherSlots : public torch::autograd::Function<GatherSlots> {
  static torch::Tensor forward(torch::autograd::AutogradContext* ctx, torch::Tensor rows_var, torch::Tensor rows,
                               torch::Tensor slot_var, torch::Tensor ws, int64_t table, int64_t dim,
                               int64_t stream) {
    TORCH_CHECK(g_gather != nullptr && g_scatter != nullptr, "_eg_autograd.init was not called");
    TORCH_CHECK(rows.dim() == 2 && rows.scalar_type() == torch::kInt32 && rows.is_contiguous(), "rows: int32 [n, heads]");
    TORCH_CHECK(slot_var.sizes() == rows.sizes() && slot_var.scalar_type() == torch::kInt32 &&
                    slot_var.is_contiguous(),
                "slot_var: int32, the shape of rows");
    TORCH_CHECK(rows_var.dim() == 2 && rows_var.size(1) == dim, "rows_var: [R, ", dim, "]");
    const int64_t n = rows.size(0), heads = rows.size(1), n_var = rows_var.size(0);
    const auto dev = rows.device();
    torch::Tensor vars = rows_var;
    if (vars.scalar_type() != torch::kFloat32 || vars.device() != dev || !vars.is_contiguous())
      vars = vars.to(dev, torch::kFloat32).contiguous();
    torch::Tensor out = torch::empty({n, heads * dim}, rows.options().dtype(torch::kFloat32));
    check(g_gather(reinterpret_cast<const eg_table*>(table), rows.data_ptr<int32_t>(), slot_var.data_ptr<int32_t>(), n,
                   (int32_t)heads, vars.data_ptr<float>(), n_var, out.data_ptr<float>(),
                   reinterpret_cast<void*>(stream)));
    ctx->saved_data["ws"] = ws;
    ctx->saved_data["meta"] = std::vector<int64_t>{n, heads, dim, n_var, stream, (int64_t)rows_var.scalar_type(),
                                                   (int64_t)rows_var.device().type(), rows_var.device().index()};
    return out;
  }

  static torch::autograd::variable_list backward(torch::autograd::AutogradContext* ctx,
                                                 torch::autograd::variable_list grads) {
    const c10::List<int64_t> meta = ctx->saved_data["meta"].toIntList();
    const int64_t n = meta[0], heads = meta[1], dim = meta[2], n_var = meta[3], stream = meta[4];
    const torch::Tensor& ws = ctx->saved_data["ws"].toTensor();
    torch::Tensor d = grads[0];
    if (d.device() != ws.device()) d = d.to(ws.device());
    if (d.scalar_type() != torch::kFloat32 && d.scalar_type() != torch::kBFloat16) d = d.to(torch::kFloat32);
    d = d.contiguous();
    torch::Tensor grad = torch::empty({n_var, dim}, d.options().dtype(torch::kFloat32));
    if (n_var > 0) {
      TORCH_CHECK(n == 0 || ws.numel() > 0, "the plan has no slot grouping for its backward");
      check(g_scatter(d.data_ptr(), d.scalar_type() == torch::kFloat32 ? 1 : 0, n, (int32_t)heads, (int32_t)dim, n_var,
                      grad.data_ptr<float>(), 1, ws.numel() > 0 ? ws.data_ptr() : nullptr, (size_t)ws.numel(),
                      reinterpret_cast<void*>(stream)));
    }
    const auto dtype = (c10::ScalarType)meta[5];
    const c10::Device device((c10::DeviceType)meta[6], (c10::DeviceIndex)meta[7]);
    if (grad.scalar_type() != dtype || grad.device() != device) grad = grad.to(device, dtype);
    return {grad, torch::Tensor(), torch::Tensor(), torch::Tensor(), torch::Tensor(), torch::Tensor(),
            torch::Tensor()};
  }
};

torch::Tensor gather_slots(torch::Tensor rows_var, torch::Tensor rows, torch::Tensor slot_var, torch::Tensor ws,
                           int64_t table, int64_t dim, int64_t stream) {
  TORCH_CHECK(ws.device() == rows.device() && ws.scalar_type() == torch::kUInt8 && ws.is_contiguous(),
              "ws: uint8 on the plan's device (empty: none)");
  return GatherSlots::apply(rows_var, rows, slot_var, ws, table, dim, stream);
}

void init(int64_t gather, int64_t scatter, int64_t error) {
  g_gather = reinterpret_cast<GatherFn>(gather);
  g_scatter = reinterpret_cast<ScatterFn>(scatter);
  g_error = reinterpret_cast<ErrorFn>(error);
}

}  // namespace

PYBIND11_MODULE(_eg_autograd, m) {
  m.def("init", &init, "the library's eg_gather_slots, eg_scatter_grad_apply and eg_last_error addresses");
  m.def("gather_slots", &gather_slots, "OverlayEmb's differentiable gather (see the file's header)");
}
