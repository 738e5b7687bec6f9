// py.cpp -- Python module light_amd._light over the C++ host layer (tensors, registry, ops).
//
// Tensors cross the boundary as bytes: from_numpy copies a contiguous numpy buffer into a
// new tensor of a named Light dtype on a device ("cpu", "rocm:0"); Tensor.numpy() copies
// it back (quantized dtypes come back as their raw block bytes, uint8).  Light's Go errors
// surface as light_amd._light.Error, and registry.ErrKernelNotFound as KernelNotFound.
#include <pybind11/numpy.h>
#include <pybind11/pybind11.h>
#include <pybind11/stl.h>

#include <cctype>
#include <cstring>

#include "gguf.hpp"
#include "light.hpp"
#include "ops.hpp"
#include "registry.hpp"

namespace py = pybind11;
using namespace light;

namespace {

DType parse_dtype(const std::string &s) {
  for (int i = 0; i <= (int)DType::Q8_K; i++)
    if (s == DTypeName((DType)i)) return (DType)i;
  Fail("dtype: unknown %s", s.c_str());
}

// Kind names as Light prints them ("CPU", "ROCm"), case-insensitively.
DeviceKind parse_kind(const std::string &s) {
  std::string ls;
  for (char ch : s) ls += (char)tolower(ch);
  for (DeviceKind k : {DeviceKind::CPU, DeviceKind::CUDA, DeviceKind::WebGPU, DeviceKind::ROCm}) {
    std::string kn;
    for (const char *p = KindName(k); *p; p++) kn += (char)tolower(*p);
    if (ls == kn) return k;
  }
  Fail("device: unknown kind %s", s.c_str());
}

// "CPU", "ROCm(1)" (Device.String) or "rocm:1".
Device parse_device(const std::string &s) {
  const auto sep = s.find_first_of(":(");
  Device d;
  d.kind = parse_kind(s.substr(0, sep));
  d.ordinal = sep == std::string::npos ? 0 : std::stoi(s.substr(sep + 1));
  return d;
}

py::dtype numpy_dtype(DType d) {
  switch (d) {
    case DType::F32: return py::dtype::of<float>();
    case DType::F64: return py::dtype::of<double>();
    case DType::F16: return py::dtype("float16");
    case DType::BF16: case DType::U16: return py::dtype::of<uint16_t>();
    case DType::I16: return py::dtype::of<int16_t>();
    case DType::I8: return py::dtype::of<int8_t>();
    case DType::U32: return py::dtype::of<uint32_t>();
    case DType::I32: return py::dtype::of<int32_t>();
    case DType::U64: return py::dtype::of<uint64_t>();
    case DType::I64: return py::dtype::of<int64_t>();
    default: return py::dtype::of<uint8_t>();
  }
}

Tensor from_numpy(py::array arr, const std::string &dt, std::vector<int64_t> shape, const std::string &dev) {
  py::array c = py::array::ensure(arr, py::array::c_style);
  if (!c) Fail("from_numpy: array is not convertible to a contiguous buffer");
  return Tensor::FromHost(c.data(), (size_t)c.nbytes(), parse_dtype(dt), std::move(shape), parse_device(dev));
}

py::array to_numpy(const Tensor &t) {
  const py::dtype nd = numpy_dtype(t.dtype());
  std::vector<py::ssize_t> shape;
  if (IsQuantized(t.dtype()))
    shape = {(py::ssize_t)t.nbytes()};
  else
    for (int64_t d : t.shape()) shape.push_back((py::ssize_t)d);
  py::array out(nd, shape);
  t.ToHost(out.mutable_data(), t.nbytes());
  return out;
}

ops::Int4 make_int4(const Tensor &codes, const Tensor &scales, const Tensor &zeros, int group,
                    std::optional<Tensor> perm) {
  ops::Int4 w;
  w.codes = codes;
  w.scales = scales;
  w.zeros = zeros;
  w.group = group;
  w.perm = std::move(perm);
  return w;
}

// GGUF strings are byte strings: decoded as UTF-8, with undecodable bytes kept by
// surrogateescape so every key and value round-trips.
py::str gguf_str(const std::string &s) {
  PyObject *o = PyUnicode_DecodeUTF8(s.data(), (Py_ssize_t)s.size(), "surrogateescape");
  if (!o) throw py::error_already_set();
  return py::reinterpret_steal<py::str>(o);
}

// The inverse, for names and keys passed in: a str (surrogateescape bytes kept) or bytes.
std::string gguf_name(const py::object &o) {
  if (py::isinstance<py::bytes>(o)) return o.cast<std::string>();
  PyObject *b = PyUnicode_AsEncodedString(o.ptr(), "utf-8", "surrogateescape");
  if (!b) throw py::error_already_set();
  py::bytes bb = py::reinterpret_steal<py::bytes>(b);
  return bb.cast<std::string>();
}

py::list gguf_strs(const std::vector<std::string> &v) {
  py::list l;
  for (const auto &x : v) l.append(gguf_str(x));
  return l;
}

py::object value_to_py(const gguf::Value &v) {
  switch (v.type) {
    case gguf::TypeUInt8: case gguf::TypeUInt16: case gguf::TypeUInt32: case gguf::TypeUInt64:
      return py::int_(v.u);
    case gguf::TypeInt8: case gguf::TypeInt16: case gguf::TypeInt32: case gguf::TypeInt64:
      return py::int_(v.i);
    case gguf::TypeFloat32: case gguf::TypeFloat64: return py::float_(v.f);
    case gguf::TypeBool: return py::bool_(v.b);
    case gguf::TypeString: return gguf_str(v.s);
    default: {
      py::list l;
      for (const gguf::Value &e : v.arr) l.append(value_to_py(e));
      return l;
    }
  }
}

}  // namespace

PYBIND11_MODULE(_light, m) {
  m.doc() = "Light's quantized-matmul ops (ops.MatMulQ, ops.MatMulInt4, ops.MoEGemmQ ...) on libhipq";
  static py::exception<Error> err(m, "Error", PyExc_RuntimeError);
  static py::exception<Error> not_found(m, "KernelNotFound", err.ptr());
  py::register_exception_translator([](std::exception_ptr p) {
    try {
      if (p) std::rethrow_exception(p);
    } catch (const Error &e) {
      if (e.IsKernelNotFound())
        py::set_error(not_found, e.what());
      else
        py::set_error(err, e.what());
    }
  });

  py::class_<Tensor>(m, "Tensor")
      .def_property_readonly("dtype", [](const Tensor &t) { return std::string(DTypeName(t.dtype())); })
      .def_property_readonly("shape", [](const Tensor &t) { return t.shape(); })
      .def_property_readonly("device", [](const Tensor &t) { return t.device().str(); })
      .def_property_readonly("nbytes", &Tensor::nbytes)
      .def_property_readonly("ptr", [](const Tensor &t) { return (uintptr_t)t.data(); })
      .def("reshape", &Tensor::Reshape)
      .def("numpy", &to_numpy)
      .def("__repr__", [](const Tensor &t) {
        return "Tensor(" + std::string(DTypeName(t.dtype())) + ", " + t.ShapeStr() + ", " + t.device().str() + ")";
      });

  m.def("from_numpy", &from_numpy, py::arg("arr"), py::arg("dtype"), py::arg("shape"), py::arg("device") = "cpu");
  m.def("empty", [](const std::string &dt, std::vector<int64_t> shape, const std::string &dev) {
    return Tensor::Empty(parse_dtype(dt), std::move(shape), parse_device(dev));
  });
  m.def("byte_size", [](const std::string &dt, int64_t n) { return ByteSize(parse_dtype(dt), n); });

  // registry
  m.def("registered", [] {
    std::vector<std::string> out;
    for (const Key &k : Registered()) out.push_back(k.str());
    return out;
  });
  m.def("lookup", [](const std::string &op, const std::string &kind, const std::string &dt) {
    Lookup(Key{op, parse_kind(kind), parse_dtype(dt)});
  });
  m.def("register_noop", [](const std::string &op, const std::string &kind, const std::string &dt) {
    try {
      Register(Key{op, parse_kind(kind), parse_dtype(dt)}, [](Context &) {});
    } catch (const std::logic_error &e) {
      throw Error(e.what());
    }
  });

  // ops
  m.def("matmul_q", &ops::MatMulQ);
  m.def("matmul_q_gated", &ops::MatMulQGated, py::arg("x"), py::arg("wg"), py::arg("wu"), py::arg("gelu") = false);
  m.def("matmul_q_fused_on", [](const std::string &kind, const std::string &dt) {
    return ops::MatMulQFusedOn(parse_kind(kind), parse_dtype(dt));
  });
  m.def(
      "dequantize_int4",
      [](const Tensor &codes, const Tensor &scales, const Tensor &zeros, int group, const std::string &out_dt,
         std::optional<Tensor> perm) {
        return ops::DequantizeInt4(make_int4(codes, scales, zeros, group, std::move(perm)), parse_dtype(out_dt));
      },
      py::arg("codes"), py::arg("scales"), py::arg("zeros"), py::arg("group"), py::arg("out_dtype"),
      py::arg("perm") = py::none());
  auto int4_tuple = [](const ops::Int4 &w) {
    return py::make_tuple(w.codes, w.scales, w.zeros, w.group, w.perm ? py::cast(*w.perm) : py::none());
  };
  m.def(
      "from_gptq",
      [int4_tuple](const Tensor &qweight, const Tensor &qzeros, const Tensor &scales, std::optional<Tensor> g_idx,
                   int group, bool v2) {
        return int4_tuple(quant::FromGPTQ(qweight, qzeros, scales, g_idx ? &*g_idx : nullptr, group, v2));
      },
      py::arg("qweight"), py::arg("qzeros"), py::arg("scales"), py::arg("g_idx"), py::arg("group"),
      py::arg("v2") = false, "quant.FromGPTQ -> (codes, scales, zeros, group, perm or None)");
  m.def(
      "from_awq",
      [int4_tuple](const Tensor &qweight, const Tensor &qzeros, const Tensor &scales, int group) {
        return int4_tuple(quant::FromAWQ(qweight, qzeros, scales, group));
      },
      py::arg("qweight"), py::arg("qzeros"), py::arg("scales"), py::arg("group"),
      "quant.FromAWQ -> (codes, scales, zeros, group, None)");
  m.def(
      "matmul_int4",
      [](const Tensor &x, const Tensor &codes, const Tensor &scales, const Tensor &zeros, int group,
         std::optional<Tensor> perm) {
        return ops::MatMulInt4(x, make_int4(codes, scales, zeros, group, std::move(perm)));
      },
      py::arg("x"), py::arg("codes"), py::arg("scales"), py::arg("zeros"), py::arg("group"),
      py::arg("perm") = py::none());

  py::class_<ops::MoERouting>(m, "MoERouting")
      .def_readonly("topk_ids", &ops::MoERouting::topk_ids)
      .def_readonly("weights", &ops::MoERouting::weights)
      .def_readonly("sorted_pairs", &ops::MoERouting::sorted_pairs)
      .def_readonly("sorted_expts", &ops::MoERouting::sorted_expts);
  m.def("moe_route_from_ids",
        [](const std::vector<int64_t> &ids, const std::vector<float> &w, int64_t T, int topk, const std::string &dev) {
          return ops::MoERouteFromIDs(ids, w, T, topk, parse_device(dev));
        });
  m.def(
      "moe_gemm_q",
      [](const Tensor &x, const Tensor &w, const ops::MoERouting &r, std::optional<Tensor> tw, int topk) {
        return ops::MoEGemmQ(x, w, r, tw ? &*tw : nullptr, topk);
      },
      py::arg("x"), py::arg("w"), py::arg("routing"), py::arg("topk_weights"), py::arg("topk"));
  m.def("moe_route", &ops::MoERoute, py::arg("probs"), py::arg("topk"), py::arg("normalize") = true);
  m.def("moe_gemm_q_gated", &ops::MoEGemmQGated, py::arg("x"), py::arg("w"), py::arg("routing"), py::arg("topk"),
        py::arg("gelu") = false);
  m.def("moe_combine", &ops::MoECombine);
  m.def(
      "moe_int4",
      [](const Tensor &x, const std::vector<std::tuple<Tensor, Tensor, Tensor>> &gate_up,
         const std::vector<std::tuple<Tensor, Tensor, Tensor>> &down, const ops::MoERouting &routing, int topk,
         int group, bool gelu) {
        std::vector<ops::Int4> gu, dn;
        for (const auto &w : gate_up) gu.push_back(make_int4(std::get<0>(w), std::get<1>(w), std::get<2>(w), group, {}));
        for (const auto &w : down) dn.push_back(make_int4(std::get<0>(w), std::get<1>(w), std::get<2>(w), group, {}));
        return ops::MoEInt4(x, gu, dn, routing, topk, gelu);
      },
      py::arg("x"), py::arg("gate_up"), py::arg("down"), py::arg("routing"), py::arg("topk"), py::arg("group"),
      py::arg("gelu") = false);
  m.def("dequantize", &ops::Dequantize);

  // GGUF byte path
  py::class_<gguf::TensorInfo>(m, "GGUFTensorInfo")
      .def_property_readonly("name", [](const gguf::TensorInfo &t) { return gguf_str(t.name); })
      .def_property_readonly("dtype", [](const gguf::TensorInfo &t) { return std::string(DTypeName(t.dtype)); })
      .def_readonly("dims", &gguf::TensorInfo::dims)
      .def_readonly("offset", &gguf::TensorInfo::offset)
      .def_readonly("bytes", &gguf::TensorInfo::bytes);
  py::class_<gguf::File, std::shared_ptr<gguf::File>>(m, "GGUFFile")
      .def_readonly("version", &gguf::File::version)
      .def_property_readonly("order", [](const gguf::File &f) { return gguf_strs(f.order); })
      .def_property_readonly("key_order", [](const gguf::File &f) { return gguf_strs(f.key_order); })
      .def_readonly("data_base", &gguf::File::data_base)
      .def_property_readonly("meta",
                             [](const gguf::File &f) {
                               py::dict d;
                               for (const auto &kv : f.meta) d[gguf_str(kv.first)] = value_to_py(kv.second);
                               return d;
                             })
      .def("info", [](const gguf::File &f, const py::object &n) { return f.Info(gguf_name(n)); })
      .def("tensor_bytes",
           [](const gguf::File &f, const py::object &n) {
             std::vector<uint8_t> b = f.TensorBytes(gguf_name(n));
             return py::bytes((const char *)b.data(), b.size());
           })
      .def("load_tensor", [](const gguf::File &f, const py::object &n,
                             const std::string &dev) { return f.LoadTensor(gguf_name(n), parse_device(dev)); },
           py::arg("name"), py::arg("device") = "cpu")
      .def("tensor_row_major", [](const gguf::File &f, const py::object &n,
                                  const std::string &dev) { return f.TensorRowMajor(gguf_name(n), parse_device(dev)); },
           py::arg("name"), py::arg("device") = "cpu")
      .def("string", [](const gguf::File &f, const py::object &k) -> py::object {
        std::string s;
        if (!f.String(gguf_name(k), &s)) return py::none();
        return gguf_str(s);
      })
      .def("int64", [](const gguf::File &f, const py::object &k) -> py::object {
        int64_t v;
        if (!f.Int64(gguf_name(k), &v)) return py::none();
        return py::int_(v);
      })
      .def("float64", [](const gguf::File &f, const py::object &k) -> py::object {
        double v;
        if (!f.Float64(gguf_name(k), &v)) return py::none();
        return py::float_(v);
      });
  m.def(
      "gguf_open_bytes",
      [](py::bytes b, bool sized) {
        std::string s = b;
        return gguf::File::Open(gguf::MemorySource(std::vector<uint8_t>(s.begin(), s.end()), sized));
      },
      py::arg("data"), py::arg("sized") = true);
  m.def("gguf_open", [](const std::string &path) { return gguf::File::Open(gguf::FileSource(path)); });
  m.def(
      "gguf_load_experts",
      [](const gguf::File &f, const std::string &prefix, const std::string &dev) {
        gguf::ExpertStacks e = gguf::LoadExperts(f, prefix, parse_device(dev));
        return py::make_tuple(e.gate_up, e.down);
      },
      py::arg("file"), py::arg("prefix"), py::arg("device") = "cpu");
  m.def("dtype_from_ggml", [](uint32_t t) { return std::string(DTypeName(gguf::DTypeFromGGML(t))); });
}
