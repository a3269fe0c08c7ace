// kvszp_torch_args.cpp -- argument marshalling for cuszp_wrapper_cpp.py.
//
// The reference's pybind11 methods take Python lists of tensors and check
// each one in C++ (cuszp_wrapper.cpp:449-461, 577-600, 1065-1088, ...).  The
// drop-in module does the same checks; doing them in Python costs a few
// attribute calls per tensor (~0.7 ms for the 1024 tensors of a 512-request
// grouped store).  This helper does them in one C++ pass and returns the
// device pointers and byte sizes packed for the C ABI (include/kvszp.h),
// which itself stays free of torch types.  No device code.

#include <torch/extension.h>

#include <cstdint>
#include <string>

namespace {

// One pass over `tensors`: every item must be a tensor on CUDA device
// `device`, of scalar type `dtype` (any when dtype < 0), contiguous when
// `contiguous`, with numel == min_numel (`exact`) or >= min_numel.  Returns
// (pointers, byte sizes) as packed little-endian uint64 bytes, or None when
// any item fails.
py::object describe(const py::list& tensors, int64_t device, int64_t dtype,
                    int64_t min_numel, bool exact, bool contiguous) {
    const size_t n = tensors.size();
    std::string ptrs(n * sizeof(uint64_t), '\0');
    std::string bytes(n * sizeof(uint64_t), '\0');
    auto* p = reinterpret_cast<uint64_t*>(&ptrs[0]);
    auto* b = reinterpret_cast<uint64_t*>(&bytes[0]);
    for (size_t i = 0; i < n; ++i) {
        PyObject* o = tensors[i].ptr();
        if (!THPVariable_Check(o)) return py::none();
        const at::Tensor& t = THPVariable_Unpack(o);
        if (!t.is_cuda() || t.get_device() != device) return py::none();
        if (dtype >= 0 && static_cast<int64_t>(t.scalar_type()) != dtype) return py::none();
        if (contiguous && !t.is_contiguous()) return py::none();
        const int64_t numel = t.numel();
        if (exact ? numel != min_numel : numel < min_numel) return py::none();
        p[i] = static_cast<uint64_t>(reinterpret_cast<uintptr_t>(t.data_ptr()));
        b[i] = static_cast<uint64_t>(numel) * static_cast<uint64_t>(t.element_size());
    }
    return py::make_tuple(py::bytes(ptrs), py::bytes(bytes));
}

// The scalar-type code `describe` compares against, for a torch dtype.
int64_t dtype_code(const py::object& dtype) {
    return static_cast<int64_t>(
        torch::python::detail::py_object_to_dtype(dtype));
}

}  // namespace

PYBIND11_MODULE(TORCH_EXTENSION_NAME, m) {
    m.def("describe", &describe);
    m.def("dtype_code", &dtype_code);
}
