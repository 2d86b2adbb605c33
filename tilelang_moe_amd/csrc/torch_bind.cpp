// Python binding of the two drop-in entry points of libmoe_hip.so, built
// against torch's C++ API so that the output tensors are allocated in C++.
//
// Through ctypes a router call cost about 8 us of host time against ~3 us
// of device time: argument conversion, two Python-level output
// allocations and the argument checks.  Here one call takes the logits
// tensor and a few integers, checks them (raising ValueError, the
// reference's exception type, through pybind11's std::invalid_argument
// mapping), allocates the outputs with at::empty and calls the C ABI
// through addresses handed over once by bind() (from the ctypes handle that
// loaded the library), so this module does not link the library.  The
// router call also takes torch's current stream and the stream's cached
// workspace here (set_workspace), so that the Python wrapper makes a single
// call.  Nonzero return codes are turned into exceptions by the Python
// wrappers (the C ABI's thread-local message is read via ctypes).
#include <torch/extension.h>
#include <c10/hip/HIPStream.h>

#include <cstdint>
#include <stdexcept>
#include <string>
#include <tuple>
#include <vector>

namespace {

using topk_fn = int (*)(const void*, int, int64_t, int64_t, int64_t, int64_t, float*, void*, int, int, int, void*,
                        size_t, void*);
using gemm_fn = int (*)(const void*, const void*, const void*, int, int, int64_t, int64_t, int64_t, int64_t,
                        int64_t, void*, void*, size_t, void*);
using ws_fn = size_t (*)(int64_t, int64_t, int64_t, int);

topk_fn g_topk = nullptr;
gemm_fn g_gemm = nullptr;
ws_fn g_topk_ws = nullptr;

// Workspaces made outside graph capture, per (device, raw stream): the same
// buffers the Python side keeps alive (tilelang_moe_amd/_lib.py).  Calls
// come with the GIL held, so the table needs no lock.
struct WsEntry {
  int64_t dev, stream, ptr, bytes;
};
std::vector<WsEntry> g_ws;

void set_workspace(int64_t dev, int64_t stream, int64_t ptr, int64_t bytes) {
  for (auto& e : g_ws)
    if (e.dev == dev && e.stream == stream) {
      e.ptr = ptr;
      e.bytes = bytes;
      return;
    }
  g_ws.push_back({dev, stream, ptr, bytes});
}

void bind(int64_t topk_addr, int64_t gemm_addr, int64_t topk_ws_addr) {
  if (!topk_addr || !gemm_addr || !topk_ws_addr) throw std::invalid_argument("bind: null function address");
  g_topk = reinterpret_cast<topk_fn>(static_cast<intptr_t>(topk_addr));
  g_gemm = reinterpret_cast<gemm_fn>(static_cast<intptr_t>(gemm_addr));
  g_topk_ws = reinterpret_cast<ws_fn>(static_cast<intptr_t>(topk_ws_addr));
}

// Drop-in TopK + softmax: validates like the Python wrappers of the
// reference (ValueError for bad arguments), allocates the outputs and calls
// moe_topk_softmax_ex on torch's current stream of the logits' device.
// Returns (return code, workspace bytes needed, scores or None, indices).
// The workspace is (ws, ws_bytes) when ws >= 0, else the stream's entry of
// set_workspace; when it is smaller than the call needs, nothing is
// launched and the code is -100.
constexpr int64_t kNeedWorkspace = -100;

std::tuple<int64_t, int64_t, c10::optional<at::Tensor>, at::Tensor> topk_softmax(
    const at::Tensor& logits_in, int64_t k, int64_t algo, bool with_scores, bool idx64, int64_t score_mode,
    int64_t ws, int64_t ws_bytes) {
  if (!g_topk) throw std::runtime_error("_moe_torch: bind() has not been called");
  if (logits_in.dim() != 2)
    throw std::invalid_argument("logits must be 2-D [num_tokens, num_experts], got shape " +
                                std::string(logits_in.sizes().vec().size() ? c10::str(logits_in.sizes()) : "()"));
  const auto st = logits_in.scalar_type();
  const int dcode = st == at::kFloat ? 0 : st == at::kBFloat16 ? 1 : st == at::kHalf ? 2 : -1;
  if (dcode < 0)
    throw std::invalid_argument("logits dtype must be float32, bfloat16 or float16, got " +
                                std::string(c10::toString(st)));
  if (!logits_in.is_cuda())
    throw std::invalid_argument("topk_softmax runs on the GPU only: logits must be a cuda (HIP) tensor");
  const int64_t m = logits_in.size(0), n = logits_in.size(1);
  if (k < 1 || k > n)
    throw std::invalid_argument("k must satisfy 1 <= k <= num_experts=" + std::to_string(n) + ", got " +
                                std::to_string(k));
  const at::Tensor logits =
      (logits_in.stride(1) != 1 || logits_in.stride(0) < n) ? logits_in.contiguous() : logits_in;
  const int64_t dev = logits.get_device();
  const int64_t stream = reinterpret_cast<int64_t>(c10::hip::getCurrentHIPStream(dev).stream());
  if (ws < 0) {
    ws = ws_bytes = 0;
    for (const auto& e : g_ws)
      if (e.dev == dev && e.stream == stream) {
        ws = e.ptr;
        ws_bytes = e.bytes;
        break;
      }
  }
  const int64_t need = m > 0 ? static_cast<int64_t>(g_topk_ws(m, n, k, static_cast<int>(algo))) : 0;
  if (need > ws_bytes) return {kNeedWorkspace, need, c10::nullopt, at::Tensor()};
  at::Tensor idx = at::empty({m, k}, logits.options().dtype(idx64 ? at::kLong : at::kInt));
  c10::optional<at::Tensor> sc;
  if (with_scores) sc = at::empty({m, k}, logits.options().dtype(at::kFloat));
  int64_t rc = 0;
  if (m > 0)
    rc = g_topk(logits.data_ptr(), dcode, m, n, logits.stride(0), k, with_scores ? sc->data_ptr<float>() : nullptr,
                idx.data_ptr(), idx64 ? 4 : 3, static_cast<int>(algo), static_cast<int>(score_mode),
                need ? reinterpret_cast<void*>(static_cast<intptr_t>(ws)) : nullptr, static_cast<size_t>(ws_bytes),
                reinterpret_cast<void*>(static_cast<intptr_t>(stream)));
  return {rc, need, sc, idx};
}

// (return code, Y [T*topk, I] in X's dtype).
std::tuple<int64_t, at::Tensor> grouped_gemm(const at::Tensor& X, const at::Tensor& W, const at::Tensor& ids,
                                             int64_t dtype_code, int64_t idx_code, int64_t T, int64_t topk,
                                             int64_t H, int64_t I, int64_t E, int64_t ws, int64_t ws_bytes,
                                             int64_t stream) {
  if (!g_gemm) throw std::runtime_error("_moe_torch: bind() has not been called");
  at::Tensor Y = at::empty({T * topk, I}, X.options());
  int64_t rc = 0;
  if (T * topk > 0)
    rc = g_gemm(X.data_ptr(), W.data_ptr(), ids.data_ptr(), static_cast<int>(dtype_code), static_cast<int>(idx_code),
                T, topk, H, I, E, Y.data_ptr(), reinterpret_cast<void*>(static_cast<intptr_t>(ws)),
                static_cast<size_t>(ws_bytes), reinterpret_cast<void*>(static_cast<intptr_t>(stream)));
  return {rc, Y};
}

}  // namespace

PYBIND11_MODULE(TORCH_EXTENSION_NAME, m) {
  m.def("bind", &bind,
        "Take the addresses of moe_topk_softmax_ex, moe_grouped_gemm and moe_topk_softmax_workspace_size.");
  m.def("set_workspace", &set_workspace, "Record the workspace of (device, raw stream) for topk_softmax.");
  m.def("topk_softmax", &topk_softmax, "moe_topk_softmax_ex with outputs allocated here.", py::arg("logits"),
        py::arg("k"), py::arg("algo"), py::arg("with_scores"), py::arg("idx64"), py::arg("score_mode"),
        py::arg("ws") = -1, py::arg("ws_bytes") = 0);
  m.def("grouped_gemm", &grouped_gemm, "moe_grouped_gemm with the output allocated here.");
}
