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
#include <cstdint>

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

  // Whole-MHA forms (adaptq_mha_append_all / _compute_all): one call for all
  // heads instead of the reference Engine's per-head loop.
  void append_all(farray keys, farray vals, int pos) {
    if (keys.ndim() != 2 || vals.ndim() != 2 || keys.shape(0) != n_heads_ ||
        vals.shape(0) != n_heads_ || keys.shape(1) != head_dim_ || vals.shape(1) != head_dim_)
      throw std::invalid_argument("keys/vals must be (n_heads, head_dim)");
    if (adaptq_mha_append_all(backend_.handle(), keys.data(), vals.data(), pos) != 0)
      throw std::runtime_error(adaptq_last_error());
  }

  farray compute_all(farray queries) {
    if (queries.ndim() != 2 || queries.shape(0) != n_heads_ || queries.shape(1) != head_dim_)
      throw std::invalid_argument("queries must be (n_heads, head_dim)");
    farray out({n_heads_, head_dim_});
    if (adaptq_mha_compute_all(backend_.handle(), queries.data(), out.mutable_data()) < 0)
      throw std::runtime_error(adaptq_last_error());
    return out;
  }

  // Device pointers (torch-ROCm tensors' data_ptr()), asynchronous on stream.
  void append_all_device(uintptr_t d_keys, uintptr_t d_vals, int n_tokens, int pos,
                         uintptr_t stream) {
    if (adaptq_mha_append_all_device(backend_.handle(), reinterpret_cast<const float *>(d_keys),
                                     reinterpret_cast<const float *>(d_vals), n_tokens, pos,
                                     reinterpret_cast<void *>(stream)) != 0)
      throw std::runtime_error(adaptq_last_error());
  }

  int compute_all_device(uintptr_t d_queries, uintptr_t d_outs, uintptr_t stream) {
    const int n = adaptq_mha_compute_all_device(
        backend_.handle(), reinterpret_cast<const float *>(d_queries),
        reinterpret_cast<float *>(d_outs), reinterpret_cast<void *>(stream));
    if (n < 0) throw std::runtime_error(adaptq_last_error());
    return n;
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
      .def("append_all", &PyMHAContext::append_all, py::arg("keys"), py::arg("vals"),
           py::arg("pos") = 0)
      .def("compute_all", &PyMHAContext::compute_all, py::arg("queries"))
      .def("append_all_device", &PyMHAContext::append_all_device, py::arg("d_keys"),
           py::arg("d_vals"), py::arg("n_tokens"), py::arg("pos"), py::arg("stream"))
      .def("compute_all_device", &PyMHAContext::compute_all_device, py::arg("d_queries"),
           py::arg("d_outs"), py::arg("stream"))
      .def("reset", &PyMHAContext::reset)
      .def("kv_bytes", &PyMHAContext::kv_bytes)
      .def_property_readonly("n_heads", &PyMHAContext::n_heads)
      .def_property_readonly("head_dim", &PyMHAContext::head_dim);
}
