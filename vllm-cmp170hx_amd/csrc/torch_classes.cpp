// The two torch custom classes of the reference's _exl3_C library, which its
// loader requires before it uses any operator (vllm_sm80/kernels/exl3/
// ops.py:205, :237-240 looks up torch.classes._exl3_C.<name>):
//   PleHostReader    csrc/exl3/ple.h:44-53, csrc/exl3/ple_read.cpp:365-373
//   EngramHostFetch  csrc/exl3/engram_fetch.cpp:843-861
// Both read compressed embedding rows from files on host threads; they are
// not part of this library's quantized-matmul path.  They are registered here
// with the reference's constructor and method signatures, so the reference's
// loader accepts this library unmodified, and every constructor and method
// raises (RuntimeError in Python) if called.
//
// Built by build.py with g++ against the installed torch (a host-only
// library, libvllm_mi355x_torch.so) and loaded by the operator registration
// in vllm_mi355x/kernels/exl3/_C.py.
#include <ATen/core/Tensor.h>
#include <torch/custom_class.h>
#include <torch/library.h>

#include <cstdint>

namespace {

[[noreturn]] void unsupported(const char* what) {
  TORCH_CHECK(false, what,
              " is not provided by the gfx950 quantized-matmul library (it reads compressed rows "
              "from files on the host, outside this library's matmul path)");
}

struct PleHostReader : torch::CustomClassHolder {
  PleHostReader(int64_t, at::Tensor, at::Tensor, int64_t, int64_t, int64_t, int64_t,
                at::Tensor, at::Tensor, int64_t, int64_t, int64_t) {
    unsupported("PleHostReader");
  }
  void enqueue(int64_t) { unsupported("PleHostReader.enqueue"); }
  void run(int64_t) { unsupported("PleHostReader.run"); }
  at::Tensor take() { unsupported("PleHostReader.take"); }
};

struct EngramHostFetch : torch::CustomClassHolder {
  EngramHostFetch(int64_t, int64_t, int64_t, int64_t, int64_t, at::Tensor, at::Tensor,
                  at::Tensor, at::Tensor, at::Tensor, int64_t, int64_t, int64_t, int64_t,
                  int64_t) {
    unsupported("EngramHostFetch");
  }
  void enqueue(int64_t) { unsupported("EngramHostFetch.enqueue"); }
  void run(int64_t) { unsupported("EngramHostFetch.run"); }
  at::Tensor take() { unsupported("EngramHostFetch.take"); }
  at::Tensor counters() { unsupported("EngramHostFetch.counters"); }
  void reset_counters() { unsupported("EngramHostFetch.reset_counters"); }
  int64_t cache_rows() { unsupported("EngramHostFetch.cache_rows"); }
  int64_t cache_bytes() { unsupported("EngramHostFetch.cache_bytes"); }
  int64_t prefault() { unsupported("EngramHostFetch.prefault"); }
  int64_t preload(at::Tensor, int64_t) { unsupported("EngramHostFetch.preload"); }
  void add_fixed(at::Tensor, at::Tensor, at::Tensor, at::Tensor) {
    unsupported("EngramHostFetch.add_fixed");
  }
  void enqueue_fixed(int64_t, at::Tensor, at::Tensor, at::Tensor) {
    unsupported("EngramHostFetch.enqueue_fixed");
  }
  void run_fixed(int64_t) { unsupported("EngramHostFetch.run_fixed"); }
  at::Tensor take_fixed() { unsupported("EngramHostFetch.take_fixed"); }
};

}  // namespace

// A fragment: the operators of _exl3_C are defined from Python
// (torch.library.Library("_exl3_C", "DEF")), the classes here.
TORCH_LIBRARY_FRAGMENT(_exl3_C, m) {
  m.class_<PleHostReader>("PleHostReader")
      .def(torch::init<int64_t, at::Tensor, at::Tensor, int64_t, int64_t, int64_t, int64_t,
                       at::Tensor, at::Tensor, int64_t, int64_t, int64_t>())
      .def("enqueue", &PleHostReader::enqueue)
      .def("run", &PleHostReader::run)
      .def("take", &PleHostReader::take);
  m.class_<EngramHostFetch>("EngramHostFetch")
      .def(torch::init<int64_t, int64_t, int64_t, int64_t, int64_t, at::Tensor, at::Tensor,
                       at::Tensor, at::Tensor, at::Tensor, int64_t, int64_t, int64_t,
                       int64_t, int64_t>())
      .def("enqueue", &EngramHostFetch::enqueue)
      .def("run", &EngramHostFetch::run)
      .def("take", &EngramHostFetch::take)
      .def("counters", &EngramHostFetch::counters)
      .def("reset_counters", &EngramHostFetch::reset_counters)
      .def("cache_rows", &EngramHostFetch::cache_rows)
      .def("cache_bytes", &EngramHostFetch::cache_bytes)
      .def("prefault", &EngramHostFetch::prefault)
      .def("preload", &EngramHostFetch::preload)
      .def("add_fixed", &EngramHostFetch::add_fixed)
      .def("enqueue_fixed", &EngramHostFetch::enqueue_fixed)
      .def("run_fixed", &EngramHostFetch::run_fixed)
      .def("take_fixed", &EngramHostFetch::take_fixed);
}
