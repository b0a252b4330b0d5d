// host_ptrs.cpp -- per-step host work of the optimizer engine in native code.
//
// Every iteration the engine must know each parameter's storage address (to
// detect a replaced param.data) and each gradient's address and dtype (the
// grad tensors are reallocated after zero_grad(set_to_none=True)).  For tens
// of thousands of tensors doing this through Python attribute access costs
// milliseconds; here it is one pass over the TensorImpl pointers.
//
// The per-call launches of a step also go through here: clip_grad_norm_ and
// step() each make one call that checks the gradient table against the one
// last uploaded and calls libmgopt's entry point (bound once, by address),
// and the scaler update is one call too, instead of Python attribute work
// and ctypes argument conversion around each launch.  Anything that changed
// since the last upload (a new gradient tensor, a dtype, a flag) sends the
// caller back to its Python path, which validates, rebuilds or uploads and
// then records the new table here.

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

// libmgopt entry points the step launches (include/mgopt.h)
using SetGradsFn = int (*)(void*, const void* const*, void*);
using GradNormFn = int (*)(void*, const float*, double, float*, float*, float*, void*);
using AdamwStepFn = int (*)(void*, const void*, const double*, int64_t, const float*, const float*, const float*,
                            int32_t, void*);
using ScalerUpdateFn = int (*)(float*, int32_t*, const float* const*, int32_t, double, double, int32_t, void*);

template <typename T>
T as_ptr(uint64_t addr) {
    return reinterpret_cast<T>(static_cast<uintptr_t>(addr));
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
        if (params_.empty()) throw std::invalid_argument("empty parameter list");
        for (const at::Tensor& p : params_) param_ptrs_.push_back(reinterpret_cast<int64_t>(p.data_ptr()));
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

    // The gradient table as the engine uploads it: pointer and dtype code per
    // tensor, 0 / -1 for a tensor without a gradient or one the presence mask
    // marks absent.  False when some gradient needs the caller's checks (a
    // flag of gather()), or a parameter's storage moved.
    bool table(std::vector<int64_t>& ptrs, std::vector<int8_t>& codes) const {
        const size_t n = params_.size();
        ptrs.resize(n);
        codes.resize(n);
        for (size_t i = 0; i < n; ++i) {
            const at::Tensor& p = params_[i];
            if (reinterpret_cast<int64_t>(p.data_ptr()) != param_ptrs_[i]) return false;
            at::Tensor g;
            if (source_.empty()) g = p.grad();
            else if (source_[i].has_value()) g = *source_[i];
            if (!g.defined() || (mask_ != nullptr && mask_[i] == 0)) {
                ptrs[i] = 0;
                codes[i] = -1;
                continue;
            }
            if (g.is_sparse() || !g.is_contiguous() || g.numel() != p.numel() || g.device() != p.device()) return false;
            ptrs[i] = reinterpret_cast<int64_t>(g.data_ptr());
            codes[i] = dtype_code(g.scalar_type());
        }
        return true;
    }

    // Records the current table as the one uploaded to the plan.
    void remember() {
        uploaded_ok_ = table(uploaded_ptrs_, uploaded_codes_);
    }

    // Whether the current table equals the one last uploaded.
    bool unchanged() {
        if (!uploaded_ok_) return false;
        if (!table(scratch_ptrs_, scratch_codes_)) return false;
        return scratch_ptrs_ == uploaded_ptrs_ && scratch_codes_ == uploaded_codes_;
    }

    // The arena's presence record (one uint8 per tensor, 0 = absent) or 0.
    void set_mask(uint64_t addr) {
        mask_ = as_ptr<const uint8_t*>(addr);
        uploaded_ok_ = false;
    }

    void bind(uint64_t grad_norm, uint64_t adamw_step) {
        grad_norm_ = as_ptr<GradNormFn>(grad_norm);
        adamw_step_ = as_ptr<AdamwStepFn>(adamw_step);
    }

    // mgopt_grad_norm with a fresh 0-dim fp32 norm tensor on the parameters'
    // device when want_norm; returns that tensor (None without want_norm), or
    // the library's nonzero status.
    py::object grad_norm(uint64_t plan, uint64_t scale, double max_norm, bool want_norm, uint64_t coef,
                         uint64_t found_inf, uint64_t stream) {
        at::Tensor out;
        float* norm = nullptr;
        if (want_norm) {
            out = at::empty({}, params_[0].options().dtype(at::kFloat));
            norm = out.data_ptr<float>();
        }
        const int rc = grad_norm_(as_ptr<void*>(plan), as_ptr<const float*>(scale), max_norm, norm,
                                  as_ptr<float*>(coef), as_ptr<float*>(found_inf), as_ptr<void*>(stream));
        if (rc != 0) return py::int_(rc);
        if (!want_norm) return py::none();
        return py::cast(out);
    }

    int adamw_step(uint64_t plan, uint64_t groups, uint64_t bc, int64_t bc_cap, uint64_t scale, uint64_t coef,
                   uint64_t found_inf, int32_t flags, uint64_t stream) const {
        return adamw_step_(as_ptr<void*>(plan), as_ptr<const void*>(groups), as_ptr<const double*>(bc), bc_cap,
                           as_ptr<const float*>(scale), as_ptr<const float*>(coef), as_ptr<const float*>(found_inf),
                           flags, as_ptr<void*>(stream));
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
    std::vector<int64_t> param_ptrs_;           // storage addresses when the set was made
    const uint8_t* mask_ = nullptr;
    bool uploaded_ok_ = false;
    std::vector<int64_t> uploaded_ptrs_, scratch_ptrs_;
    std::vector<int8_t> uploaded_codes_, scratch_codes_;
    GradNormFn grad_norm_ = nullptr;
    AdamwStepFn adamw_step_ = nullptr;
};

// GradScaler.update's launch: mgopt_scaler_update through its address, with
// the found_inf pointers read from a caller-owned array of n addresses.
int scaler_update(uint64_t fn, uint64_t scale, uint64_t tracker, uint64_t found, int32_t n, double growth,
                  double backoff, int32_t interval, uint64_t stream) {
    return as_ptr<ScalerUpdateFn>(fn)(as_ptr<float*>(scale), as_ptr<int32_t*>(tracker),
                                      as_ptr<const float* const*>(found), n, growth, backoff, interval,
                                      as_ptr<void*>(stream));
}

}  // namespace

PYBIND11_MODULE(TORCH_EXTENSION_NAME, m) {
    py::class_<ParamSet>(m, "ParamSet")
        .def(py::init<std::vector<at::Tensor>, std::vector<c10::optional<at::Tensor>>>())
        .def("gather", &ParamSet::gather)
        .def("param_ptrs", &ParamSet::param_ptrs)
        .def("clear_grads", &ParamSet::clear_grads)
        .def("remember", &ParamSet::remember)
        .def("unchanged", &ParamSet::unchanged)
        .def("set_mask", &ParamSet::set_mask)
        .def("bind", &ParamSet::bind)
        .def("grad_norm", &ParamSet::grad_norm)
        .def("adamw_step", &ParamSet::adamw_step)
        .def("__len__", &ParamSet::size);
    m.def("scaler_update", &scaler_update);
}
