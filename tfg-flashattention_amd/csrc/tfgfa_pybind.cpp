// tfgfa_pybind.cpp - pybind11 module `custom_flash_attn._C`, a thin layer over the C ABI.
//
// Plays the role of the reference's PYBIND11_MODULE (src/cpp/torch_bind.cpp:47-49), but it
// does not depend on libtorch: it takes raw device pointers, sizes and a stream handle.  The
// Python package (custom_flash_attn/__init__.py) does the tensor checks and allocation that
// torch_bind.cpp:13-31 does in C++.  The GIL is released around the launch, and a non-zero
// C-ABI status becomes a Python RuntimeError (the reference drops launcher errors,
// torch_bind.cpp:34-39).
#include <pybind11/pybind11.h>
#include <pybind11/stl.h>

#include <array>
#include <cstdint>
#include <stdexcept>
#include <string>

#include "tfgfa.h"

namespace py = pybind11;

namespace {

void fwd(std::uintptr_t q, std::uintptr_t k, std::uintptr_t v, std::uintptr_t o, std::uintptr_t lse,
         int B, int H, int N, int D, float softmax_scale, bool causal, std::uintptr_t stream) {
  int st;
  {
    py::gil_scoped_release nogil;
    st = tfgfa_fwd_bf16(reinterpret_cast<const void*>(q), reinterpret_cast<const void*>(k),
                        reinterpret_cast<const void*>(v), reinterpret_cast<void*>(o),
                        reinterpret_cast<float*>(lse), B, H, N, D, softmax_scale, causal ? 1 : 0,
                        reinterpret_cast<void*>(stream));
  }
  if (st != TFGFA_OK) {
    throw std::runtime_error(std::string("tfgfa_fwd_bf16 failed (status ") + std::to_string(st) +
                             "): " + tfgfa_strerror(st));
  }
}

using Strides4 = std::array<std::int64_t, 4>;

void fwd_strided(std::uintptr_t q, const Strides4& qs, std::uintptr_t k, const Strides4& ks,
                 std::uintptr_t v, const Strides4& vs, std::uintptr_t o, const Strides4& os,
                 std::uintptr_t lse, int B, int H, int N, int D, float softmax_scale, bool causal,
                 std::uintptr_t stream) {
  int st;
  {
    py::gil_scoped_release nogil;
    st = tfgfa_fwd_bf16_strided(
        reinterpret_cast<const void*>(q), qs.data(), reinterpret_cast<const void*>(k), ks.data(),
        reinterpret_cast<const void*>(v), vs.data(), reinterpret_cast<void*>(o), os.data(),
        reinterpret_cast<float*>(lse), B, H, N, D, softmax_scale, causal ? 1 : 0,
        reinterpret_cast<void*>(stream));
  }
  if (st != TFGFA_OK) {
    throw std::runtime_error(std::string("tfgfa_fwd_bf16_strided failed (status ") +
                             std::to_string(st) + "): " + tfgfa_strerror(st));
  }
}

void fwd_general(std::uintptr_t q, const Strides4& qs, std::uintptr_t k, const Strides4& ks,
                 std::uintptr_t v, const Strides4& vs, std::uintptr_t o, const Strides4& os,
                 std::uintptr_t lse, int B, int H, int N_q, int N_k, int D, int dtype,
                 float softmax_scale, bool causal, std::uintptr_t stream) {
  int st;
  {
    py::gil_scoped_release nogil;
    st = tfgfa_fwd(reinterpret_cast<const void*>(q), qs.data(), reinterpret_cast<const void*>(k),
                   ks.data(), reinterpret_cast<const void*>(v), vs.data(),
                   reinterpret_cast<void*>(o), os.data(), reinterpret_cast<float*>(lse), B, H, N_q,
                   N_k, D, dtype, softmax_scale, causal ? 1 : 0, reinterpret_cast<void*>(stream));
  }
  if (st != TFGFA_OK) {
    throw std::runtime_error(std::string("tfgfa_fwd failed (status ") + std::to_string(st) +
                             "): " + tfgfa_strerror(st));
  }
}

using Strides3 = std::array<std::int64_t, 3>;

void decode(std::uintptr_t q, const Strides3& qs, std::uintptr_t kc, const Strides4& ks,
            std::uintptr_t vc, const Strides4& vs, std::uintptr_t kn, const Strides3& kns,
            std::uintptr_t vn, const Strides3& vns, std::uintptr_t seqlens, std::uintptr_t o,
            const Strides3& os, std::uintptr_t lse, int B, int H, int N_max, int D,
            float softmax_scale, std::uintptr_t workspace, std::size_t workspace_bytes,
            std::uintptr_t stream) {
  int st;
  {
    py::gil_scoped_release nogil;
    st = tfgfa_decode_bf16(
        reinterpret_cast<const void*>(q), qs.data(), reinterpret_cast<void*>(kc), ks.data(),
        reinterpret_cast<void*>(vc), vs.data(), reinterpret_cast<const void*>(kn), kns.data(),
        reinterpret_cast<const void*>(vn), vns.data(), reinterpret_cast<const int*>(seqlens),
        reinterpret_cast<void*>(o), os.data(), reinterpret_cast<float*>(lse), B, H, N_max, D,
        softmax_scale, reinterpret_cast<void*>(workspace), workspace_bytes,
        reinterpret_cast<void*>(stream));
  }
  if (st != TFGFA_OK) {
    throw std::runtime_error(std::string("tfgfa_decode_bf16 failed (status ") +
                             std::to_string(st) + "): " + tfgfa_strerror(st));
  }
}

void decode_general(std::uintptr_t q, const Strides3& qs, std::uintptr_t kc, const Strides4& ks,
                    std::uintptr_t vc, const Strides4& vs, std::uintptr_t kn, const Strides3& kns,
                    std::uintptr_t vn, const Strides3& vns, std::uintptr_t seqlens,
                    std::uintptr_t o, const Strides3& os, std::uintptr_t lse, int B, int H,
                    int N_max, int D, int dtype, float softmax_scale, std::uintptr_t workspace,
                    std::size_t workspace_bytes, std::uintptr_t stream) {
  int st;
  {
    py::gil_scoped_release nogil;
    st = tfgfa_decode(
        reinterpret_cast<const void*>(q), qs.data(), reinterpret_cast<void*>(kc), ks.data(),
        reinterpret_cast<void*>(vc), vs.data(), reinterpret_cast<const void*>(kn), kns.data(),
        reinterpret_cast<const void*>(vn), vns.data(), reinterpret_cast<const int*>(seqlens),
        reinterpret_cast<void*>(o), os.data(), reinterpret_cast<float*>(lse), B, H, N_max, D,
        dtype, softmax_scale, reinterpret_cast<void*>(workspace), workspace_bytes,
        reinterpret_cast<void*>(stream));
  }
  if (st != TFGFA_OK) {
    throw std::runtime_error(std::string("tfgfa_decode failed (status ") + std::to_string(st) +
                             "): " + tfgfa_strerror(st));
  }
}

py::dict device_info() {
  int cu = 0, mhz = 0;
  char arch[128] = {0};
  const int st = tfgfa_device_info(&cu, &mhz, arch, sizeof(arch));
  if (st != TFGFA_OK) {
    throw std::runtime_error(std::string("tfgfa_device_info failed: ") + tfgfa_strerror(st));
  }
  py::dict d;
  d["cu_count"] = cu;
  d["sclk_mhz"] = mhz;
  d["arch"] = std::string(arch);
  return d;
}

}  // namespace

PYBIND11_MODULE(_C, m) {
  m.doc() = "MI355X causal FlashAttention forward (C-ABI binding)";
  m.def("fwd", &fwd, "Launch the bf16 attention forward on raw device pointers", py::arg("q"),
        py::arg("k"), py::arg("v"), py::arg("o"), py::arg("lse"), py::arg("B"), py::arg("H"),
        py::arg("N"), py::arg("D"), py::arg("softmax_scale"), py::arg("causal"),
        py::arg("stream"));
  m.def("fwd_strided", &fwd_strided,
        "Launch the bf16 attention forward on strided operands (element strides b, h, n, d)",
        py::arg("q"), py::arg("q_strides"), py::arg("k"), py::arg("k_strides"), py::arg("v"),
        py::arg("v_strides"), py::arg("o"), py::arg("o_strides"), py::arg("lse"), py::arg("B"),
        py::arg("H"), py::arg("N"), py::arg("D"), py::arg("softmax_scale"), py::arg("causal"),
        py::arg("stream"));
  m.def("fwd_general", &fwd_general,
        "Attention forward, any strides, bf16/fp16, head dim a multiple of 8 up to 128, N_q != N_k",
        py::arg("q"), py::arg("q_strides"), py::arg("k"), py::arg("k_strides"), py::arg("v"),
        py::arg("v_strides"), py::arg("o"), py::arg("o_strides"), py::arg("lse"), py::arg("B"),
        py::arg("H"), py::arg("N_q"), py::arg("N_k"), py::arg("D"), py::arg("dtype"),
        py::arg("softmax_scale"), py::arg("causal"), py::arg("stream"));
  m.attr("DTYPE_BF16") = TFGFA_DTYPE_BF16;
  m.attr("DTYPE_F16") = TFGFA_DTYPE_F16;
  m.def("decode", &decode,
        "One decode step over a KV cache on raw device pointers (element strides)",
        py::arg("q"), py::arg("q_strides"), py::arg("k_cache"), py::arg("k_strides"),
        py::arg("v_cache"), py::arg("v_strides"), py::arg("k_new"), py::arg("k_new_strides"),
        py::arg("v_new"), py::arg("v_new_strides"), py::arg("cache_seqlens"), py::arg("o"),
        py::arg("o_strides"), py::arg("lse"), py::arg("B"), py::arg("H"), py::arg("N_max"),
        py::arg("D"), py::arg("softmax_scale"), py::arg("workspace"),
        py::arg("workspace_bytes"), py::arg("stream"));
  m.def("decode_general", &decode_general,
        "One decode step, bf16/fp16, head dim a multiple of 8 up to 128 (element strides)",
        py::arg("q"), py::arg("q_strides"), py::arg("k_cache"), py::arg("k_strides"),
        py::arg("v_cache"), py::arg("v_strides"), py::arg("k_new"), py::arg("k_new_strides"),
        py::arg("v_new"), py::arg("v_new_strides"), py::arg("cache_seqlens"), py::arg("o"),
        py::arg("o_strides"), py::arg("lse"), py::arg("B"), py::arg("H"), py::arg("N_max"),
        py::arg("D"), py::arg("dtype"), py::arg("softmax_scale"), py::arg("workspace"),
        py::arg("workspace_bytes"), py::arg("stream"));
  m.def("stream_read", [](std::uintptr_t p, std::size_t bytes, std::uintptr_t sink, std::uintptr_t stream) {
    const int st = tfgfa_stream_read(reinterpret_cast<const void*>(p), bytes,
                                     reinterpret_cast<void*>(sink), reinterpret_cast<void*>(stream));
    if (st != TFGFA_OK)
      throw std::runtime_error(std::string("tfgfa_stream_read failed: ") + tfgfa_strerror(st));
  }, "A plain streaming read of `bytes` device bytes (a measurement floor)", py::arg("p"),
        py::arg("bytes"), py::arg("sink"), py::arg("stream"));
  m.def("decode_workspace_bytes", [](int B, int H, int N_max) {
    return tfgfa_decode_workspace_bytes(B, H, N_max);
  });
  m.def("decode_workspace_size", [](int B, int H, int N_max, int D) {
    return tfgfa_decode_workspace_size(B, H, N_max, D);
  });
  m.def("device_info", &device_info, "CU count, shader clock (MHz) and arch of the current device");
  m.def("strerror", [](int st) { return std::string(tfgfa_strerror(st)); });
  m.def("abi_version", []() { return tfgfa_abi_version(); });
}
