// py_module.cpp -- _trs_native: the Python binding of the C++ host engine.
//
// Mirrors the PyO3 layer of the reference for the hot path
// (src/python.rs:3844-3919 tensor methods, :4067-4133 binary_operation,
// :4139-4170 torch.tensor, :4221-4228 relu): Python scalars become f32 by
// round-to-nearest (src/python.rs:10296-10320), engine errors surface as
// RuntimeError / IndexError with the reference's messages
// (src/python_tensor_errors.rs:8-49).  The torch_rs package wraps this
// module; nothing here falls back to host arithmetic.
#include <pybind11/numpy.h>
#include <pybind11/pybind11.h>
#include <pybind11/stl.h>

#include <cstring>

#include "engine.h"

namespace py = pybind11;
using namespace trs_engine;

namespace {

std::string to_str(const Dims &d) {
    std::string s = "[";
    for (size_t i = 0; i < d.size(); i++) s += (i ? ", " : "") + std::to_string(d[i]);
    return s + "]";
}

py::tuple to_tuple(const Dims &d) {
    py::tuple t(d.size());
    for (size_t i = 0; i < d.size(); i++) t[i] = py::int_(d[i]);
    return t;
}

// Logical values as a numpy array of the tensor's shape (a copy).
py::array_t<float> to_numpy(const Tensor &t) {
    std::vector<py::ssize_t> shape(t.shape.begin(), t.shape.end());
    py::array_t<float> a(shape);
    t.copy_to_host(a.mutable_data());
    return a;
}

// parse_arithmetic_scalar + into_f32 (src/python.rs:10070-10184, 10258-10320).
enum class Scalar { None, Bool, Number, WideNumpyUnsigned, Overflow };

Scalar scalar_of(const py::handle &h, float *out) {
    if (Py_TYPE(h.ptr()) == &PyBool_Type) {  // exactly bool: the only "bool tensor" operand
        *out = h.ptr() == Py_True ? 1.0f : 0.0f;
        return Scalar::Bool;
    }
    if (PyLong_Check(h.ptr())) {
        int overflow = 0;
        const long long v = PyLong_AsLongLongAndOverflow(h.ptr(), &overflow);
        if (overflow == 0) {
            *out = (float)(int64_t)v;  // i64 as f32: round to nearest
            return Scalar::Number;
        }
        const unsigned long long u = overflow > 0 ? PyLong_AsUnsignedLongLong(h.ptr()) : 0;
        if (overflow < 0 || PyErr_Occurred()) {  // beyond both i64 and u64
            PyErr_Clear();
            return Scalar::Overflow;
        }
        *out = (float)(uint64_t)u;
        return Scalar::Number;
    }
    if (PyFloat_Check(h.ptr())) {
        *out = (float)PyFloat_AsDouble(h.ptr());  // f64 as f32: round to nearest, +-inf beyond range
        return Scalar::Number;
    }
    py::module_ np = py::module_::import("numpy");
    if (!py::isinstance(h, np.attr("generic"))) return Scalar::None;
    if (py::isinstance(h, np.attr("bool_"))) {
        *out = h.cast<bool>() ? 1.0f : 0.0f;
        return Scalar::Number;
    }
    if (py::isinstance(h, np.attr("integer"))) {
        py::int_ v = py::reinterpret_steal<py::int_>(PyNumber_Long(h.ptr()));
        if (!v) throw py::error_already_set();
        int overflow = 0;
        const long long i = PyLong_AsLongLongAndOverflow(v.ptr(), &overflow);
        if (overflow == 0) {
            *out = (float)(int64_t)i;
            return Scalar::Number;
        }
        return Scalar::WideNumpyUnsigned;
    }
    if (py::isinstance(h, np.attr("floating"))) {
        *out = (float)h.attr("__float__")().cast<double>();
        return Scalar::Number;
    }
    return Scalar::None;
}

enum class BinOp { Add, Sub, Mul, Div };

// binary_operation / apply_scalar (src/python.rs:4067-4133).
py::object binary_operation(const Tensor &self, const py::object &other, BinOp op, bool reverse) {
    if (py::isinstance<Tensor>(other)) {
        const Tensor &o = other.cast<const Tensor &>();
        const Tensor &l = reverse ? o : self, &r = reverse ? self : o;
        switch (op) {
        case BinOp::Add: return py::cast(l.add(r));
        case BinOp::Sub: return py::cast(l.sub(r));
        case BinOp::Mul: return py::cast(l.mul(r));
        case BinOp::Div: return py::cast(l.div(r));
        }
    }
    float s = 0.0f;
    const Scalar kind = scalar_of(other, &s);
    if (kind == Scalar::Overflow) {
        PyErr_SetString(PyExc_OverflowError, "Python integer is outside the supported scalar range");
        throw py::error_already_set();
    }
    if (kind == Scalar::None) return py::reinterpret_borrow<py::object>(Py_NotImplemented);
    if (kind == Scalar::WideNumpyUnsigned) {
        // numpy_reflected_divide (src/python.rs:4054-4065): numpy divides.
        if (reverse && op == BinOp::Div)
            return py::module_::import("numpy").attr("true_divide")(other, to_numpy(self));
        return py::reinterpret_borrow<py::object>(Py_NotImplemented);
    }
    if (op == BinOp::Sub && kind == Scalar::Bool)
        throw TensorError("Subtraction, the `-` operator, with a bool tensor is not supported. If you are trying to "
                          "invert a mask, use the `~` or `logical_not()` operator instead.");
    switch (op) {
    case BinOp::Add: return py::cast(self.add_scalar(s));
    case BinOp::Sub: return py::cast(reverse ? self.scalar_sub(s) : self.sub_scalar(s));
    case BinOp::Mul: return py::cast(self.mul_scalar(s));
    case BinOp::Div: return py::cast(reverse ? self.scalar_div(s) : self.div_scalar(s));
    }
    return py::none();
}

Tensor from_numpy(py::array_t<float, py::array::c_style | py::array::forcecast> arr, const std::string &device) {
    Dims shape(arr.shape(), arr.shape() + arr.ndim());
    return Tensor::from_host(arr.data(), shape, Device::parse(device));
}

// A numpy array in page-locked host memory (trs_host_alloc), released when
// the array is collected.  Copies between it and the device run as one DMA.
py::array empty_pinned(const std::vector<int64_t> &shape, const std::string &dtype) {
    py::dtype dt(dtype);
    if (!dt.is(py::dtype::of<float>()) && !dt.is(py::dtype::of<uint8_t>()))
        throw TensorError("empty_pinned supports float32 and uint8, got " + dtype);
    int64_t n = 1;
    for (int64_t d : shape) {
        if (d < 0) throw TensorError("empty_pinned: negative dimension");
        n *= d;
    }
    void *p = nullptr;
    const size_t bytes = (size_t)n * (size_t)dt.itemsize();
    if (trs_host_alloc(bytes, &p) != TRS_OK) throw TensorError(trs_last_error());
    static char empty_byte;
    if (!p) p = &empty_byte;  // zero bytes: nothing was allocated
    py::capsule owner(p, [](void *q) {
        if (q != &empty_byte) (void)trs_host_free(q);
    });
    std::vector<py::ssize_t> dims(shape.begin(), shape.end());
    return py::array(dt, dims, p, owner);
}

// Logical values of `t` written into a C-contiguous float32 array of its
// shape (for example one from empty_pinned), without an intermediate buffer.
void copy_into(const Tensor &t, py::array out) {
    if (!out.dtype().is(py::dtype::of<float>())) throw TensorError("copy_to_host: out must be float32");
    if (!(out.flags() & py::array::c_style) || !out.writeable())
        throw TensorError("copy_to_host: out must be a writeable C-contiguous array");
    Dims shape(out.shape(), out.shape() + out.ndim());
    if (shape != t.shape)
        throw TensorError("copy_to_host: out has shape " + to_str(shape) + ", tensor has " + to_str(t.shape));
    t.copy_to_host(static_cast<float *>(out.mutable_data()));
}

std::vector<int64_t> dims_arg(const py::args &args) {
    // permute(0, 2, 1) or permute((0, 2, 1)) / reshape(2, 3) or reshape([2, 3])
    if (args.size() == 1 && !py::isinstance<py::int_>(args[0])) return args[0].cast<std::vector<int64_t>>();
    return args.cast<std::vector<int64_t>>();
}

}  // namespace

// A fused program's arguments: tensors, or byte buffers for `in u8` operands.
static std::vector<FusedArg> fused_args(const py::sequence &inputs) {
    std::vector<FusedArg> out;
    for (const py::handle &h : inputs) {
        if (py::isinstance<Tensor>(h)) {
            out.push_back(FusedArg{h.cast<Tensor>(), nullptr});
        } else if (py::isinstance<ByteBuffer>(h)) {
            out.push_back(FusedArg{Tensor{}, h.cast<BytePtr>()});
        } else {
            throw py::type_error("fused program arguments must be Tensors or ByteBuffers");
        }
    }
    return out;
}

PYBIND11_MODULE(_trs_native, m) {
    m.doc() = "C++ host engine of the MI355X pytorch-rs backend (tensors, views, autograd) over libtrs_hip.so";

    py::register_exception_translator([](std::exception_ptr p) {
        try {
            if (p) std::rethrow_exception(p);
        } catch (const IndexError &e) {
            PyErr_SetString(PyExc_IndexError, e.what());
        } catch (const TensorError &e) {
            PyErr_SetString(PyExc_RuntimeError, e.what());
        }
    });

    py::class_<ByteBuffer, std::shared_ptr<ByteBuffer>>(m, "ByteBuffer")
        .def_property_readonly("shape", [](const ByteBuffer &b) { return to_tuple(b.shape); })
        .def_property_readonly("device", [](const ByteBuffer &b) { return b.device.str(); });

    m.def("empty_pinned", &empty_pinned, py::arg("shape"), py::arg("dtype") = "float32");
    m.def("copy_into", &copy_into, py::arg("tensor"), py::arg("out"));
    m.def("bytes_from_numpy",
          [](py::array_t<uint8_t, py::array::c_style | py::array::forcecast> arr, const std::string &device) {
              Dims shape(arr.shape(), arr.shape() + arr.ndim());
              return ByteBuffer::from_host(arr.data(), shape, Device::parse(device));
          });

    py::class_<Tensor>(m, "Tensor", py::dynamic_attr())
        .def_property_readonly("shape", [](const Tensor &t) { return to_tuple(t.shape); })
        .def("_strides", [](const Tensor &t) { return to_tuple(t.strides); })
        .def("storage_offset", [](const Tensor &t) { return t.offset; })
        .def("numel", [](const Tensor &t) { return t.numel; })
        .def("dim", [](const Tensor &t) { return (int64_t)t.shape.size(); })
        .def("is_contiguous", &Tensor::is_contiguous)
        .def("is_non_overlapping_and_dense",
             [](const Tensor &t) { return layout::is_non_overlapping_and_dense(t.shape, t.strides, t.numel); })
        .def_property_readonly("_device_str", [](const Tensor &t) { return t.device().str(); })
        .def_property_readonly("is_cuda", [](const Tensor &t) { return t.device().is_cuda(); })
        .def_property_readonly("requires_grad", &Tensor::requires_grad)
        .def_property_readonly("is_leaf", &Tensor::is_leaf)
        .def_property_readonly("output_nr", [](const Tensor &t) { return t.output_nr; })
        .def_property_readonly("_grad_fn_name", [](const Tensor &t) -> py::object {
            const char *n = t.grad_fn_name();
            if (!n) return py::none();
            return py::str(n);
        })
        .def("_storage_id", [](const Tensor &t) { return (uintptr_t)t.storage.get(); })
        .def("_autograd_id", [](const Tensor &t) { return (uintptr_t)t.autograd.get(); })
        .def("_live_grad", &Tensor::live_grad)
        // Address of the first element (storage base + offset), as Tensor.data_ptr.
        .def("data_ptr", [](const Tensor &t) { return (uintptr_t)(t.storage->data() + t.offset); })
        .def("with_requires_grad", &Tensor::with_requires_grad)
        // In place, as Tensor.requires_grad_ is: the same Python object, now a leaf.
        .def(
            "requires_grad_",
            [](Tensor &t, bool flag) -> Tensor & {
                t = t.with_requires_grad(flag);
                return t;
            },
            py::arg("requires_grad") = true, py::return_value_policy::reference)
        .def("detach", &Tensor::detach)
        .def("to", [](const Tensor &t, const std::string &dev) { return t.to(Device::parse(dev)); })
        .def("numpy", &to_numpy)
        .def("item", &Tensor::item)
        .def("permute", [](const Tensor &t, const py::args &a) { return t.permute(dims_arg(a)); })
        .def("transpose", &Tensor::transpose)
        // swapdims / swapaxes are transpose under another name (src/python.rs:3634-3672)
        .def("swapdims", &Tensor::transpose, py::arg("dim0"), py::arg("dim1"))
        .def("swapaxes", &Tensor::transpose, py::arg("axis0"), py::arg("axis1"))
        .def("_unsqueeze_front", &Tensor::unsqueeze_front)
        // squeeze(), squeeze(dim), squeeze((d0, d1, ...)) (src/python.rs:6112-6121)
        .def("squeeze",
             [](const Tensor &t, const py::object &dim) {
                 if (dim.is_none()) return t.squeeze();
                 if (py::isinstance<py::int_>(dim)) return t.squeeze_dim(dim.cast<int64_t>());
                 return t.squeeze_dims(dim.cast<std::vector<int64_t>>());
             },
             py::arg("dim") = py::none())
        .def_property_readonly("mT", &Tensor::matrix_transpose)
        .def_property_readonly("T", &Tensor::reverse_dims)
        .def("t", &Tensor::reverse_dims)
        .def("reshape", [](const Tensor &t, const py::args &a) { return t.reshape(dims_arg(a)); })
        .def("view", [](const Tensor &t, const py::args &a) { return t.view(dims_arg(a)); })
        .def("contiguous", &Tensor::contiguous)
        .def("clone", &Tensor::clone)
        .def("select", &Tensor::select)
        .def("__getitem__", [](const Tensor &t, int64_t i) { return t.select(i); })
        .def("add", [](const Tensor &t, const py::object &o) { return binary_operation(t, o, BinOp::Add, false); },
             py::arg("other"))
        .def("sub", [](const Tensor &t, const py::object &o) { return binary_operation(t, o, BinOp::Sub, false); },
             py::arg("other"))
        .def("mul", [](const Tensor &t, const py::object &o) { return binary_operation(t, o, BinOp::Mul, false); },
             py::arg("other"))
        .def("div", [](const Tensor &t, const py::object &o) { return binary_operation(t, o, BinOp::Div, false); },
             py::arg("other"))
        .def("__add__", [](const Tensor &t, const py::object &o) { return binary_operation(t, o, BinOp::Add, false); })
        .def("__radd__", [](const Tensor &t, const py::object &o) { return binary_operation(t, o, BinOp::Add, true); })
        .def("__sub__", [](const Tensor &t, const py::object &o) { return binary_operation(t, o, BinOp::Sub, false); })
        .def("__rsub__", [](const Tensor &t, const py::object &o) { return binary_operation(t, o, BinOp::Sub, true); })
        .def("__mul__", [](const Tensor &t, const py::object &o) { return binary_operation(t, o, BinOp::Mul, false); })
        .def("__rmul__", [](const Tensor &t, const py::object &o) { return binary_operation(t, o, BinOp::Mul, true); })
        .def("__truediv__",
             [](const Tensor &t, const py::object &o) { return binary_operation(t, o, BinOp::Div, false); })
        .def("__rtruediv__",
             [](const Tensor &t, const py::object &o) { return binary_operation(t, o, BinOp::Div, true); })
        .def("__neg__", &Tensor::neg)
        .def("neg", &Tensor::neg)
        .def("__matmul__", &Tensor::matmul)
        .def("matmul", &Tensor::matmul)
        .def("relu", &Tensor::relu)
        .def("exp", &Tensor::exp)
        .def("sum", &Tensor::sum)
        .def("backward", &Tensor::backward)
        .def("_has_grad", &Tensor::has_grad)
        .def("_grad", &Tensor::grad);

    m.def("from_numpy", &from_numpy, py::arg("array"), py::arg("device") = "cuda");
    m.def("full", [](const std::vector<int64_t> &shape, float v, const std::string &dev) {
        return Tensor::full(shape, v, Device::parse(dev));
    });
    m.def("mask_apply", &mask_apply);
    m.def("enter_no_grad", &enter_no_grad);
    m.def("exit_no_grad", &exit_no_grad);
    m.def("is_grad_enabled", &is_grad_enabled);
    m.def("device_count", &device_count);
    m.def("synchronize", &synchronize);
    m.def("current_device", &current_device);
    m.def("set_device", &set_device);

    py::class_<FusedProgram>(m, "FusedProgram")
        .def_static("compile", &FusedProgram::compile)
        .def_property_readonly("id", [](const FusedProgram &p) { return p.id; })
        .def_property_readonly("nin", [](const FusedProgram &p) { return p.nin; })
        .def("launch",
             [](const FusedProgram &p, const py::sequence &inputs, const Dims &shape, const Dims &strides) {
                 return p.launch(fused_args(inputs), shape, strides);
             })
        .def("launch_with_grad",
             [](const FusedProgram &p, const py::sequence &inputs, const Dims &shape, const Dims &strides,
                uint64_t program, const std::vector<int> &args, const std::vector<int> &targets) {
                 return p.launch_with_grad(fused_args(inputs), shape, strides, FusedBackward{program, args, targets});
             });

    // The restated layout planner, exposed for the CPU parity tests.
    py::module_ L = m.def_submodule("layout", "output-layout planning restated from src/tensor.rs");
    L.def("contiguous_strides", &layout::contiguous_strides);
    L.def("is_contiguous", &layout::is_contiguous);
    L.def("is_non_overlapping_and_dense", &layout::is_non_overlapping_and_dense);
    L.def("is_channels_last_contiguous", &layout::is_channels_last_contiguous);
    L.def("unary_output_strides", &layout::unary_output_strides);
    L.def("scalar_output_strides", &layout::scalar_output_strides);
    L.def("elementwise_output_strides", &layout::elementwise_output_strides);
    L.def("binary_output_layout", [](const Dims &ls, const Dims &lt, const Dims &rs, const Dims &rt) {
        Dims os, ost;
        layout::binary_output_layout(ls, lt, rs, rt, os, ost);
        return py::make_tuple(to_tuple(os), to_tuple(ost));
    });
    L.def("reshape_view_strides", [](const Dims &os, const Dims &ost, const Dims &ns, int64_t n) -> py::object {
        Dims out;
        if (!layout::reshape_view_strides(os, ost, ns, n, out)) return py::none();
        return to_tuple(out);
    });
}
