// host_ptrs.cpp -- per-step host work of the optimizer engine in native code.
//
// Every iteration the engine must know each parameter's storage address (to
// detect a replaced param.data) and each gradient's address and dtype (the
// grad tensors are reallocated after zero_grad(set_to_none=True)).  For tens
// of thousands of tensors doing this through Python attribute access costs
// milliseconds; here it is one pass over the TensorImpl pointers.

#include <torch/extension.h>

#include <cstdint>
#include <cstring>
#include <stdexcept>
#include <string>
#include <vector>

namespace {

// dtype codes of include/mgopt.h
int8_t dtype_code(c10::ScalarType t) {
    switch (t) {
        case c10::ScalarType::Float: return 0;
        case c10::ScalarType::Half: return 1;
        case c10::ScalarType::BFloat16: return 2;
        default: return -2;
    }
}

// The parameters (and an optional fixed gradient source) of one optimizer,
// held as tensor handles: the same TensorImpls the Python objects wrap, so a
// new p.grad or a replaced p.data is seen without converting Python lists
// again every step.
class ParamSet {
  public:
    ParamSet(std::vector<at::Tensor> params, std::vector<c10::optional<at::Tensor>> source)
        : params_(std::move(params)), source_(std::move(source)) {
        if (!source_.empty() && source_.size() != params_.size())
            throw std::invalid_argument("gradient source must have one entry per parameter");
    }

    // (param pointers, grad pointers, grad dtype codes, grad flags) as byte
    // strings of int64 / int64 / int8 / int8 per tensor.  A tensor with no
    // gradient has pointer 0 and dtype -1.  Flags: bit 0 not contiguous, bit 1
    // size differs from the parameter, bit 2 other device, bit 3 sparse.
    py::tuple gather() const {
        const size_t n = params_.size();
        std::string pp(n * 8, '\0'), gp(n * 8, '\0'), gd(n, '\0'), gf(n, '\0');
        for (size_t i = 0; i < n; ++i) {
            const at::Tensor& p = params_[i];
            const int64_t pa = reinterpret_cast<int64_t>(p.data_ptr());
            std::memcpy(&pp[i * 8], &pa, 8);
            at::Tensor g;
            if (source_.empty()) g = p.grad();
            else if (source_[i].has_value()) g = *source_[i];
            int64_t ga = 0;
            int8_t code = -1, flags = 0;
            if (g.defined()) {
                if (g.is_sparse()) {
                    flags |= 8;
                } else {
                    ga = reinterpret_cast<int64_t>(g.data_ptr());
                    code = dtype_code(g.scalar_type());
                    if (!g.is_contiguous()) flags |= 1;
                    if (g.numel() != p.numel()) flags |= 2;
                    if (g.device() != p.device()) flags |= 4;
                }
            }
            std::memcpy(&gp[i * 8], &ga, 8);
            gd[i] = static_cast<char>(code);
            gf[i] = static_cast<char>(flags);
        }
        return py::make_tuple(py::bytes(pp), py::bytes(gp), py::bytes(gd), py::bytes(gf));
    }

    // Parameter pointers only.
    py::bytes param_ptrs() const {
        std::string pp(params_.size() * 8, '\0');
        for (size_t i = 0; i < params_.size(); ++i) {
            const int64_t pa = reinterpret_cast<int64_t>(params_[i].data_ptr());
            std::memcpy(&pp[i * 8], &pa, 8);
        }
        return py::bytes(pp);
    }

    // zero_grad(set_to_none=True) over every parameter: drops each .grad, as
    // the per-parameter `p.grad = None` of torch.optim.Optimizer.zero_grad
    // does, without a Python-level loop.
    void clear_grads() {
        for (at::Tensor& p : params_) {
            if (p.grad().defined()) p.mutable_grad().reset();
        }
    }

    size_t size() const { return params_.size(); }

  private:
    std::vector<at::Tensor> params_;
    std::vector<c10::optional<at::Tensor>> source_;
};

}  // namespace

PYBIND11_MODULE(TORCH_EXTENSION_NAME, m) {
    py::class_<ParamSet>(m, "ParamSet")
        .def(py::init<std::vector<at::Tensor>, std::vector<c10::optional<at::Tensor>>>())
        .def("gather", &ParamSet::gather)
        .def("param_ptrs", &ParamSet::param_ptrs)
        .def("clear_grads", &ParamSet::clear_grads)
        .def("__len__", &ParamSet::size);
}
