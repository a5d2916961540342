// adapter_python.cpp -- pybind11 module `adaptq_py` over the C ABI.
//
// Same Python surface as the reference's adapters/adapter_python.cpp:30-93:
// class MHAContext(n_heads, head_dim, k_bits, v_bits, capacity, seed=0,
// v_mass=0.95, hybrid_thresh=512) with append / compute / compute_batch /
// reset / kv_bytes and the n_heads / head_dim properties, so the reference's
// adaptq.Engine runs on it unchanged.  Creation failure raises RuntimeError
// with adaptq_last_error() (the reference would carry a NULL handle on).
#include <pybind11/numpy.h>
#include <pybind11/pybind11.h>

#include <stdexcept>
#include <string>

#include "adaptq_mha_backend.h"

namespace py = pybind11;

namespace {

using farray = py::array_t<float, py::array::c_style | py::array::forcecast>;

class PyMHAContext {
 public:
  PyMHAContext(int n_heads, int head_dim, int k_bits, int v_bits, int capacity,
               uint64_t seed, float v_mass, int hybrid_thresh)
      : backend_(n_heads, head_dim, k_bits, v_bits, capacity, seed, v_mass, hybrid_thresh),
        head_dim_(head_dim),
        n_heads_(n_heads) {
    if (!backend_.ok()) throw std::runtime_error(std::string(adaptq_last_error()));
  }

  void append(int head, farray key, farray val, int pos) {
    if (key.ndim() != 1 || val.ndim() != 1 || key.shape(0) != head_dim_ ||
        val.shape(0) != head_dim_)
      throw std::invalid_argument("key/val dim mismatch");
    backend_.append_kv(head, key.data(), val.data(), pos);
  }

  farray compute(int head, farray query) {
    if (query.ndim() != 1 || query.shape(0) != head_dim_)
      throw std::invalid_argument("query dim mismatch");
    farray out(head_dim_);
    backend_.compute(head, query.data(), out.mutable_data());
    return out;
  }

  farray compute_batch(int head, farray queries) {
    if (queries.ndim() != 2 || queries.shape(1) != head_dim_)
      throw std::invalid_argument("queries dim mismatch");
    const int nq = (int)queries.shape(0);
    farray out({nq, head_dim_});
    backend_.compute_batch(head, queries.data(), nq, out.mutable_data());
    return out;
  }

  void reset() { backend_.reset(); }
  size_t kv_bytes() const { return backend_.kv_bytes(); }
  int n_heads() const { return n_heads_; }
  int head_dim() const { return head_dim_; }

 private:
  AdaptQMHABackend backend_;
  int head_dim_, n_heads_;
};

}  // namespace

PYBIND11_MODULE(adaptq_py, m) {
  m.doc() = "AdapTQ quantised KV-cache attention on gfx950 (HIP)";
  py::class_<PyMHAContext>(m, "MHAContext")
      .def(py::init<int, int, int, int, int, uint64_t, float, int>(), py::arg("n_heads"),
           py::arg("head_dim"), py::arg("k_bits"), py::arg("v_bits"), py::arg("capacity"),
           py::arg("seed") = 0, py::arg("v_mass") = 0.95f, py::arg("hybrid_thresh") = 512)
      .def("append", &PyMHAContext::append, py::arg("head"), py::arg("key"), py::arg("val"),
           py::arg("pos"))
      .def("compute", &PyMHAContext::compute, py::arg("head"), py::arg("query"))
      .def("compute_batch", &PyMHAContext::compute_batch, py::arg("head"), py::arg("queries"))
      .def("reset", &PyMHAContext::reset)
      .def("kv_bytes", &PyMHAContext::kv_bytes)
      .def_property_readonly("n_heads", &PyMHAContext::n_heads)
      .def_property_readonly("head_dim", &PyMHAContext::head_dim);
}
