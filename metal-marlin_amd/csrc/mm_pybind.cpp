// Python binding of the per-call hot path (marlin_gemm_fp4 / marlin_gemm_int4)
// for callers that issue one GEMM per Python call.  It does in C++ what the
// ctypes path does in Python -- shape checks, the output allocation, the
// per-(device, stream) workspace -- and calls the same C ABI entry points of
// libmmfp4.so (mm_fp4_gemm / mm_u4_gemm).  torch is used only for tensor
// arguments and the output allocation; the stream comes from the caller.
#include <torch/extension.h>

#include <map>
#include <mutex>
#include <sstream>
#include <utility>

#include "mmfp4.h"

namespace {

std::mutex g_mu;
std::map<std::pair<int, int64_t>, at::Tensor> g_ws;   // (device index, stream) -> workspace

// One workspace per (device, stream), shared with the ctypes path (which
// asks for it through workspace_for below); kept until release_workspaces().
at::Tensor workspace_dev(int dev, int64_t stream, size_t nbytes, const at::TensorOptions& opt) {
  std::lock_guard<std::mutex> lock(g_mu);
  const auto key = std::make_pair(dev, stream);
  auto it = g_ws.find(key);
  if (it != g_ws.end() && (size_t)it->second.numel() >= nbytes) return it->second;
  size_t size = nbytes < ((size_t)1 << 20) ? ((size_t)1 << 20) : nbytes;
  if (it != g_ws.end() && size < 2 * (size_t)it->second.numel()) size = 2 * it->second.numel();
  // Zero-filled once: the split-K arrival counters at its head must start at
  // zero, and every call leaves them at zero.
  at::Tensor buf = at::zeros({(int64_t)size}, opt.dtype(at::kByte));
  g_ws[key] = buf;
  return buf;
}

at::Tensor workspace(const at::Tensor& like, int64_t stream, size_t nbytes) {
  return workspace_dev((int)like.get_device(), stream, nbytes, like.options());
}

at::Tensor workspace_for(int64_t device, int64_t stream, int64_t nbytes) {
  return workspace_dev((int)device, stream, (size_t)nbytes,
                       at::TensorOptions().device(at::kCUDA, (int)device));
}

void release_workspaces() {
  std::lock_guard<std::mutex> lock(g_mu);
  g_ws.clear();
}

[[noreturn]] void fail(int rc) {
  const char* msg = mm_last_error();
  if (rc == 1) throw pybind11::value_error(msg);
  throw std::runtime_error(msg);
}

void check_groups(const char* name, const at::Tensor& t, int64_t K, int64_t N, int64_t g) {
  if (g <= 0 || K % g != 0) {
    std::ostringstream os;
    os << name << ": K=" << K << " must be divisible by group_size=" << g;
    throw pybind11::value_error(os.str());
  }
  if (t.dim() != 2 || t.size(0) != K / g || t.size(1) != N) {
    std::ostringstream os;
    os << name << ": " << name << " shape " << t.sizes() << " != (" << K / g << ", " << N
       << ") for K=" << K << ", group_size=" << g;
    throw pybind11::value_error(os.str());
  }
}

at::Tensor half_contig(const at::Tensor& t) {
  return t.scalar_type() == at::kHalf && t.is_contiguous() ? t : t.to(at::kHalf).contiguous();
}

// C = A . dequant(B, S[, Z]) for A [*, K], B [K/8, N] words; fp16 [*, N].
// SZ (INT4 only, optional): the scales and zeros interleaved [K/g, N/4, 8]
// for the decode kernels (mm_u4_gemm_sz).
at::Tensor gemm(const at::Tensor& A, const at::Tensor& B, const at::Tensor& S,
                const c10::optional<at::Tensor>& Z, const c10::optional<at::Tensor>& SZ,
                int64_t group_size, int64_t stream) {
  const int dev = A.get_device();
  if (dev < 0 || B.get_device() != dev || S.get_device() != dev ||
      (Z && Z->get_device() != dev)) {
    std::ostringstream os;
    os << "tensor on " << (dev < 0 ? A.device() : B.device())
       << ": the FP4/INT4 kernels run on the GPU only, with every operand on one device";
    throw std::runtime_error(os.str());
  }
  if (B.dim() != 2) throw pybind11::value_error("B_packed must be [K/8, N]");
  if (B.scalar_type() != at::kInt && B.scalar_type() != at::kUInt32)
    throw pybind11::type_error("packed weights must be int32/uint32 words");
  const int64_t K = A.size(-1);
  const int64_t M = K ? A.numel() / K : 0;
  const int64_t N = B.size(1);
  if (B.size(0) * 8 != K) {
    std::ostringstream os;
    os << "Packed K " << B.size(0) * 8 << " does not match activations K " << K;
    throw pybind11::value_error(os.str());
  }
  check_groups("scales", S, K, N, group_size);
  if (Z) check_groups("zeros", *Z, K, N, group_size);
  const at::Tensor a = half_contig(A);
  const at::Tensor b = B.is_contiguous() ? B : B.contiguous();
  const at::Tensor s = half_contig(S);
  std::vector<int64_t> oshape(A.sizes().begin(), A.sizes().end());
  oshape.back() = N;
  at::Tensor out = at::empty(oshape, a.options());
  const size_t need = mm_gemm_workspace_bytes((int)M, (int)N, (int)K);
  at::Tensor ws = workspace(a, stream, need);
  int rc;
  if (!Z) {
    rc = mm_fp4_gemm((const uint16_t*)a.data_ptr(), (const uint32_t*)b.data_ptr(),
                     (const uint16_t*)s.data_ptr(), (uint16_t*)out.data_ptr(), (int)M, (int)N,
                     (int)K, (int)group_size, ws.data_ptr(), (size_t)ws.numel(),
                     (void*)stream);
  } else if (SZ) {
    const at::Tensor z = half_contig(*Z);
    if (SZ->scalar_type() != at::kHalf || !SZ->is_contiguous() || SZ->numel() != 2 * z.numel() ||
        SZ->get_device() != dev)
      throw pybind11::value_error("SZ must be contiguous fp16 [K/g, 2N] on the operands' device");
    rc = mm_u4_gemm_sz((const uint16_t*)a.data_ptr(), (const uint32_t*)b.data_ptr(),
                       (const uint16_t*)s.data_ptr(), (const uint16_t*)z.data_ptr(),
                       (const uint16_t*)SZ->data_ptr(), (uint16_t*)out.data_ptr(), (int)M,
                       (int)N, (int)K, (int)group_size, ws.data_ptr(), (size_t)ws.numel(),
                       (void*)stream);
  } else {
    const at::Tensor z = half_contig(*Z);
    rc = mm_u4_gemm((const uint16_t*)a.data_ptr(), (const uint32_t*)b.data_ptr(),
                    (const uint16_t*)s.data_ptr(), (const uint16_t*)z.data_ptr(),
                    (uint16_t*)out.data_ptr(), (int)M, (int)N, (int)K, (int)group_size,
                    ws.data_ptr(), (size_t)ws.numel(), (void*)stream);
  }
  if (rc) fail(rc);
  return out;
}

}  // namespace

PYBIND11_MODULE(TORCH_EXTENSION_NAME, m) {
  m.doc() = "Per-call binding of libmmfp4's FP4 / INT4 GEMM entry points";
  m.def("gemm", &gemm, "C = A . dequant(B, S[, Z]) on the given stream", pybind11::arg("A"),
        pybind11::arg("B"), pybind11::arg("S"), pybind11::arg("Z"), pybind11::arg("SZ"),
        pybind11::arg("group_size"), pybind11::arg("stream"));
  m.def("workspace", &workspace_for,
        "the zero-initialised workspace of (device index, raw stream), at least nbytes",
        pybind11::arg("device"), pybind11::arg("stream"), pybind11::arg("nbytes"));
  m.def("release_workspaces", &release_workspaces, "drop every cached workspace");
}
