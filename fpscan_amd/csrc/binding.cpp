// fpscan_amd._C: the torch-facing module over the C ABI in include/fpscan_hip.h.
//
// Reference interface mirrored (saeeddhqan/fpscan):
//   csrc/main.cpp:7-11           module with "fullscan_forward" (same name, same arguments,
//                                returns `out`)
//   csrc/full_scan/full_scan.h:7-36   CHECK_INPUT on Ax/Bx (same RuntimeError messages)
//   csrc/full_scan/full_scan.cu:179-258  stride/dtype checks, tile table, launch on the
//                                current stream
// Added: `fullscan_backward`, the fused backward that replaces the composition in
// fpscan/ops.py:69-83, plus the checks the reference leaves out (shapes, `out`, device);
// `fullscan_forward_cl` / `fullscan_backward_cl` for (batch, seqlen, dim) tensors;
// `dimwise_forward` (csrc/main.cpp:10), the contraction scan; the fused softplus-gate scan.
// Every check runs before any HIP call, so a bad call raises RuntimeError on any machine.
#include <torch/extension.h>

// torch-ROCm exposes HIP devices as device type "cuda"; the guard and stream accessors that
// accept such devices are the MasqueradingAsCUDA variants
#include <ATen/hip/impl/HIPGuardImplMasqueradingAsCUDA.h>
#include <ATen/hip/impl/HIPStreamMasqueradingAsCUDA.h>

#include <hip/hip_runtime_api.h>

#include <string>
#include <utility>

#include "fpscan_hip.h"

namespace {

void check_input(const at::Tensor& t, const char* name) {
  TORCH_CHECK(t.device().is_cuda(), name, " must be a CUDA tensor");
  TORCH_CHECK(t.is_contiguous(), name, " must be contiguous");
  const auto st = t.scalar_type();
  TORCH_CHECK(st == at::kHalf || st == at::kBFloat16 || st == at::kFloat, name,
              " must be float16 or bfloat16 or float32");
  TORCH_CHECK(t.dim() == 3, name, " must be a 3-d (batch, dim, seqlen) tensor, got ", t.dim(),
              " dims");
}

void check_like(const at::Tensor& t, const at::Tensor& ref, const char* name,
                const char* ref_name) {
  TORCH_CHECK(t.scalar_type() == ref.scalar_type(), name, " must have the dtype of ", ref_name,
              " (", ref.scalar_type(), "), got ", t.scalar_type());
  TORCH_CHECK(t.sizes() == ref.sizes(), name, " must have the shape of ", ref_name, " ",
              ref.sizes(), ", got ", t.sizes());
  TORCH_CHECK(t.device() == ref.device(), name, " must be on ", ref.device(), ", got ",
              t.device());
}

int dtype_code(at::ScalarType st) {
  switch (st) {
    case at::kFloat: return FPSCAN_DTYPE_F32;
    case at::kHalf: return FPSCAN_DTYPE_F16;
    default: return FPSCAN_DTYPE_BF16;
  }
}

void check_seqlen(int64_t seqlen) {
  TORCH_CHECK(seqlen >= 32 && seqlen <= 65536 && (seqlen & (seqlen - 1)) == 0,
              "seqlen must be a power of 2, >= 32, <= 65536, got ", seqlen);
}

// Tile-status workspace from torch's caching allocator on the tensors' device (the call is
// made with that device current); an empty tensor when the problem needs none.
at::Tensor workspace(size_t bytes, const at::Tensor& like) {
  if (bytes == 0) return at::Tensor();
  return at::empty({(int64_t)bytes}, like.options().dtype(at::kByte));
}

// Whether two contiguous tensors share any byte: [data_ptr, data_ptr + nbytes) intersect.
bool overlap(const at::Tensor& a, const at::Tensor& b) {
  const char* pa = static_cast<const char*>(a.data_ptr());
  const char* pb = static_cast<const char*>(b.data_ptr());
  return a.nbytes() > 0 && b.nbytes() > 0 && pa < pb + b.nbytes() && pb < pa + a.nbytes();
}

// An output that may be one of its inputs exactly (each element is read by the lane that
// writes it) but must not overlap one partly, where a lane would overwrite elements that
// another lane has still to read.
void check_in_place(const at::Tensor& out, std::initializer_list<const at::Tensor*> inputs,
                    const char* op) {
  for (const at::Tensor* i : inputs)
    TORCH_CHECK(out.data_ptr() == i->data_ptr() || !overlap(out, *i), op, ": out must be one "
                "of its inputs or not overlap them (it may not alias an input partly)");
}

// Outputs that share no byte with the inputs or with each other: the kernels read
// neighbouring elements (gates[t+1], out[t-1]) while other lanes write.
void check_no_alias(std::initializer_list<const at::Tensor*> outputs,
                    std::initializer_list<const at::Tensor*> inputs, const char* op) {
  for (const at::Tensor* o : outputs)
    for (const at::Tensor* i : inputs)
      TORCH_CHECK(!overlap(*o, *i), op, " outputs must not alias its inputs");
  for (auto a = outputs.begin(); a != outputs.end(); ++a)
    for (auto b = a + 1; b != outputs.end(); ++b)
      TORCH_CHECK(!overlap(**a, **b), op, " outputs must be distinct and must not overlap");
}

void check_status(int status) {
  TORCH_CHECK(status == FPSCAN_OK, "fpscan: ", fpscan_strerror(status), " (status ", status,
              ")");
}

// The stream a call is about to launch on, refused while it captures a HIP graph: the one
// capture of these kernels through torch.cuda.graph that was run (the streaming forward and
// backward) ended in a host segmentation fault inside capture_end, with a cause not found, so
// a capture fails here with an error instead. Eager launches on any stream are unaffected.
void* launch_stream(const at::Tensor& like) {
  hipStream_t stream =
      c10::hip::getCurrentHIPStreamMasqueradingAsCUDA(like.device().index()).stream();
  hipStreamCaptureStatus capture = hipStreamCaptureStatusNone;
  const bool capturing = hipStreamIsCapturing(stream, &capture) == hipSuccess &&
                         capture != hipStreamCaptureStatusNone;
  TORCH_CHECK(!capturing, "fpscan: HIP graph capture of the fpscan kernels through the torch "
              "binding is not supported by this build (a captured run crashed the host in "
              "graph instantiation); call it outside the captured region");
  return stream;
}

at::Tensor fullscan_forward(const at::Tensor& Ax, const at::Tensor& Bx, const at::Tensor& out,
                            bool reverse) {
  check_input(Ax, "Ax");
  check_input(Bx, "Bx");
  check_like(Ax, Bx, "Ax", "Bx");
  check_input(out, "out");
  check_like(out, Bx, "out", "Bx");
  check_seqlen(Bx.size(2));
  check_in_place(out, {&Ax, &Bx}, "fullscan_forward");
  if (Bx.numel() == 0) return out;

  c10::hip::HIPGuardMasqueradingAsCUDA guard(Bx.device());
  void* stream = launch_stream(Bx);
  // contiguous (batch, dim, seqlen): the packed strides (torch may report any stride for a
  // size-1 dimension of a contiguous tensor)
  const int64_t L = Bx.size(2), D = Bx.size(1);
  const int dt = dtype_code(Bx.scalar_type());
  const size_t ws_bytes = fpscan_workspace_bytes(Bx.size(0), D, L, dt, FPSCAN_OP_FWD);
  at::Tensor ws = workspace(ws_bytes, Bx);
  const int status = fpscan_scan_fwd(Ax.data_ptr(), Bx.data_ptr(), out.data_ptr(), Bx.size(0),
                                     D, L, D * L, L, dt, reverse ? 1 : 0,
                                     ws_bytes ? ws.data_ptr() : nullptr, ws_bytes, stream);
  check_status(status);
  return out;
}

std::tuple<at::Tensor, at::Tensor> fullscan_backward(const at::Tensor& gates,
                                                     const at::Tensor& out,
                                                     const at::Tensor& grad_out,
                                                     const at::Tensor& grad_gates,
                                                     const at::Tensor& grad_tokens) {
  check_input(gates, "gates");
  check_input(out, "out");
  check_input(grad_out, "grad_out");
  check_input(grad_gates, "grad_gates");
  check_input(grad_tokens, "grad_tokens");
  check_like(out, gates, "out", "gates");
  check_like(grad_out, gates, "grad_out", "gates");
  check_like(grad_gates, gates, "grad_gates", "gates");
  check_like(grad_tokens, gates, "grad_tokens", "gates");
  check_seqlen(gates.size(2));
  if (gates.numel() == 0) return {grad_gates, grad_tokens};
  check_no_alias({&grad_gates, &grad_tokens}, {&gates, &out, &grad_out}, "fullscan_backward");

  c10::hip::HIPGuardMasqueradingAsCUDA guard(gates.device());
  void* stream = launch_stream(gates);
  const int dt = dtype_code(gates.scalar_type());
  const size_t ws_bytes =
      fpscan_workspace_bytes(gates.size(0), gates.size(1), gates.size(2), dt, FPSCAN_OP_BWD);
  at::Tensor ws = workspace(ws_bytes, gates);
  const int status = fpscan_scan_bwd(gates.data_ptr(), out.data_ptr(), grad_out.data_ptr(),
                                     grad_gates.data_ptr(), grad_tokens.data_ptr(),
                                     gates.size(0), gates.size(1), gates.size(2),
                                     gates.size(1) * gates.size(2), gates.size(2), dt,
                                     ws_bytes ? ws.data_ptr() : nullptr, ws_bytes, stream);
  check_status(status);
  return {grad_gates, grad_tokens};
}

// ---- pscan as an autograd function in C++: the same computation as the Python PScan
// (fpscan/ops.py:61-87: the forward saves (gates, out), the backward hands grad_output to the
// fused backward), with the forward and backward entered from the autograd engine without a
// Python call each. For calls of tens of microseconds the Python round trips were most of the
// host time per step.
struct PScanFunction : public torch::autograd::Function<PScanFunction> {
  static at::Tensor forward(torch::autograd::AutogradContext* ctx, const at::Tensor& gates,
                            const at::Tensor& tokens) {
    at::Tensor out = at::empty_like(tokens);
    fullscan_forward(gates, tokens, out, false);
    ctx->save_for_backward({gates, out});
    return out;
  }
  static torch::autograd::variable_list backward(torch::autograd::AutogradContext* ctx,
                                                 torch::autograd::variable_list grads) {
    const auto saved = ctx->get_saved_variables();
    const at::Tensor& gates = saved[0];
    const at::Tensor& out = saved[1];
    at::Tensor grad_gates = at::empty_like(gates);
    at::Tensor grad_tokens = at::empty_like(gates);
    fullscan_backward(gates, out, grads[0].contiguous(), grad_gates, grad_tokens);
    return {grad_gates, grad_tokens};
  }
};

at::Tensor pscan(const at::Tensor& gates, const at::Tensor& tokens) {
  return PScanFunction::apply(gates, tokens);
}

// ---- channel-last (batch, seqlen, dim): no reference counterpart (README.md:94-99 has
// callers transpose instead)
void check_input_cl(const at::Tensor& t, const char* name) {
  TORCH_CHECK(t.device().is_cuda(), name, " must be a CUDA tensor");
  TORCH_CHECK(t.is_contiguous(), name, " must be contiguous");
  const auto st = t.scalar_type();
  TORCH_CHECK(st == at::kHalf || st == at::kBFloat16 || st == at::kFloat, name,
              " must be float16 or bfloat16 or float32");
  TORCH_CHECK(t.dim() == 3, name, " must be a 3-d (batch, seqlen, dim) tensor, got ", t.dim(),
              " dims");
  const int64_t vec = 16 / (int64_t)t.element_size();
  TORCH_CHECK(t.size(2) % vec == 0, name, ": dim must be a multiple of ", vec, " for ",
              t.scalar_type(), " (16-byte vectors), got ", t.size(2));
}

at::Tensor fullscan_forward_cl(const at::Tensor& Ax, const at::Tensor& Bx, const at::Tensor& out,
                               bool reverse) {
  check_input_cl(Ax, "Ax");
  check_input_cl(Bx, "Bx");
  check_like(Ax, Bx, "Ax", "Bx");
  check_input_cl(out, "out");
  check_like(out, Bx, "out", "Bx");
  check_in_place(out, {&Ax, &Bx}, "fullscan_forward_cl");
  if (Bx.numel() == 0) return out;

  c10::hip::HIPGuardMasqueradingAsCUDA guard(Bx.device());
  void* stream = launch_stream(Bx);
  const int64_t B = Bx.size(0), L = Bx.size(1), D = Bx.size(2);
  const int dt = dtype_code(Bx.scalar_type());
  const size_t ws_bytes = fpscan_workspace_bytes_cl(B, L, D, D, dt, FPSCAN_OP_FWD);
  at::Tensor ws = workspace(ws_bytes, Bx);
  const int status = fpscan_scan_fwd_cl(Ax.data_ptr(), Bx.data_ptr(), out.data_ptr(), B, L, D,
                                        L * D, D, dt, reverse ? 1 : 0,
                                        ws_bytes ? ws.data_ptr() : nullptr, ws_bytes, stream);
  check_status(status);
  return out;
}

std::tuple<at::Tensor, at::Tensor> fullscan_backward_cl(const at::Tensor& gates,
                                                        const at::Tensor& out,
                                                        const at::Tensor& grad_out,
                                                        const at::Tensor& grad_gates,
                                                        const at::Tensor& grad_tokens) {
  check_input_cl(gates, "gates");
  check_input_cl(out, "out");
  check_input_cl(grad_out, "grad_out");
  check_input_cl(grad_gates, "grad_gates");
  check_input_cl(grad_tokens, "grad_tokens");
  check_like(out, gates, "out", "gates");
  check_like(grad_out, gates, "grad_out", "gates");
  check_like(grad_gates, gates, "grad_gates", "gates");
  check_like(grad_tokens, gates, "grad_tokens", "gates");
  if (gates.numel() == 0) return {grad_gates, grad_tokens};
  check_no_alias({&grad_gates, &grad_tokens}, {&gates, &out, &grad_out}, "fullscan_backward_cl");

  c10::hip::HIPGuardMasqueradingAsCUDA guard(gates.device());
  void* stream = launch_stream(gates);
  const int64_t B = gates.size(0), L = gates.size(1), D = gates.size(2);
  const int dt = dtype_code(gates.scalar_type());
  const size_t ws_bytes = fpscan_workspace_bytes_cl(B, L, D, D, dt, FPSCAN_OP_BWD);
  at::Tensor ws = workspace(ws_bytes, gates);
  const int status = fpscan_scan_bwd_cl(gates.data_ptr(), out.data_ptr(), grad_out.data_ptr(),
                                        grad_gates.data_ptr(), grad_tokens.data_ptr(), B, L, D,
                                        L * D, D, dt, ws_bytes ? ws.data_ptr() : nullptr,
                                        ws_bytes, stream);
  check_status(status);
  return {grad_gates, grad_tokens};
}

// ---- dimwise_forward: csrc/main.cpp:10, csrc/dimwise/dimwise.h:27-42 (CHECK_INPUT on all
// five tensors, same messages), in place into Bx, returns nothing. Added checks: one dtype
// for all five (the reference reinterprets Bh/Wq/Wk as Ax's type), the shapes of Ax, Bh,
// Wq and Wk (the reference reads out of bounds when they are short).
void dimwise_forward(const at::Tensor& Ax, const at::Tensor& Bx, const at::Tensor& Bh,
                     const at::Tensor& Wq, const at::Tensor& Wk) {
  for (const auto& [t, name] : {std::pair<const at::Tensor*, const char*>{&Ax, "Ax"},
                                {&Bx, "Bx"}, {&Bh, "Bh"}, {&Wq, "Wq"}, {&Wk, "Wk"}}) {
    TORCH_CHECK(t->device().is_cuda(), name, " must be a CUDA tensor");
    TORCH_CHECK(t->is_contiguous(), name, " must be contiguous");
    const auto st = t->scalar_type();
    TORCH_CHECK(st == at::kHalf || st == at::kBFloat16 || st == at::kFloat, name,
                " must be float16 or bfloat16 or float32");
    TORCH_CHECK(st == Bx.scalar_type(), name, " must have the dtype of Bx (", Bx.scalar_type(),
                "), got ", st);
    TORCH_CHECK(t->device() == Bx.device(), name, " must be on ", Bx.device());
  }
  TORCH_CHECK(Bx.dim() == 3, "Bx must be a 3-d (batch, dim, seqlen) tensor, got ", Bx.dim(),
              " dims");
  TORCH_CHECK(Ax.sizes() == Bx.sizes(), "Ax must have the shape of Bx ", Bx.sizes(), ", got ",
              Ax.sizes());
  const int64_t B = Bx.size(0), D = Bx.size(1), L = Bx.size(2);
  const int G = fpscan_dimwise_groups(L);
  TORCH_CHECK(G > 0, "seqlen must be a power of 2, >= 64, <= 65536, got ", L);
  TORCH_CHECK(Bh.dim() == 3 && Bh.size(0) == B && Bh.size(1) == D && Bh.size(2) == G,
              "Bh must have shape (", B, ", ", D, ", ", G, ") for seqlen ", L, ", got ",
              Bh.sizes());
  TORCH_CHECK(Wq.numel() == D && Wk.numel() == D, "Wq and Wk must have ", D,
              " elements (one per dim), got ", Wq.numel(), " and ", Wk.numel());
  // Bx is the output: Ax may be Bx itself, the per-row parameters must lie apart from it
  check_in_place(Bx, {&Ax}, "dimwise_forward");
  check_no_alias({&Bx}, {&Bh, &Wq, &Wk}, "dimwise_forward");
  if (Bx.numel() == 0) return;

  c10::hip::HIPGuardMasqueradingAsCUDA guard(Bx.device());
  void* stream = launch_stream(Bx);
  const int dt = dtype_code(Bx.scalar_type());
  const size_t ws_bytes = fpscan_dimwise_workspace_bytes(B, D, L, dt);
  at::Tensor ws = workspace(ws_bytes, Bx);
  const int status = fpscan_dimwise_fwd_ws(Ax.data_ptr(), Bx.data_ptr(), Bh.data_ptr(),
                                           Wq.data_ptr(), Wk.data_ptr(), B, D, L, dt,
                                           ws_bytes ? ws.data_ptr() : nullptr, ws_bytes, stream);
  check_status(status);
}

// ---- fused softplus gates: gates = exp(-softplus(z) * rate[d]) computed inside the scan (no
// reference counterpart: the reference takes materialised gates). rate: fp32, one per dim.
void check_rate(const at::Tensor& rate, const at::Tensor& like, const char* name) {
  TORCH_CHECK(rate.device() == like.device(), name, " must be on ", like.device());
  TORCH_CHECK(rate.scalar_type() == at::kFloat, name, " must be float32, got ",
              rate.scalar_type());
  TORCH_CHECK(rate.is_contiguous() && rate.numel() == like.size(1), name, " must be a contiguous",
              " float32 tensor with one value per dim (", like.size(1), "), got ", rate.sizes());
}

at::Tensor fullscan_forward_softplus(const at::Tensor& z, const at::Tensor& rate,
                                     const at::Tensor& tokens, const at::Tensor& out,
                                     bool reverse) {
  check_input(z, "z");
  check_input(tokens, "tokens");
  check_like(z, tokens, "z", "tokens");
  check_input(out, "out");
  check_like(out, tokens, "out", "tokens");
  check_rate(rate, tokens, "rate");
  check_seqlen(tokens.size(2));
  check_in_place(out, {&z, &tokens}, "fullscan_forward_softplus");
  if (tokens.numel() == 0) return out;
  c10::hip::HIPGuardMasqueradingAsCUDA guard(tokens.device());
  void* stream = launch_stream(tokens);
  const int64_t D = tokens.size(1), L = tokens.size(2);
  const int status = fpscan_scan_fwd_softplus(
      z.data_ptr(), rate.data_ptr<float>(), tokens.data_ptr(), out.data_ptr(), tokens.size(0),
      D, L, D * L, L, dtype_code(tokens.scalar_type()), reverse ? 1 : 0, stream);
  check_status(status);
  return out;
}

void fullscan_backward_softplus(const at::Tensor& z, const at::Tensor& rate,
                                const at::Tensor& out, const at::Tensor& grad_out,
                                const at::Tensor& grad_z, const at::Tensor& grad_tokens,
                                const at::Tensor& grad_rate_rows) {
  check_input(z, "z");
  check_input(out, "out");
  check_input(grad_out, "grad_out");
  check_input(grad_z, "grad_z");
  check_input(grad_tokens, "grad_tokens");
  check_like(out, z, "out", "z");
  check_like(grad_out, z, "grad_out", "z");
  check_like(grad_z, z, "grad_z", "z");
  check_like(grad_tokens, z, "grad_tokens", "z");
  check_rate(rate, z, "rate");
  check_seqlen(z.size(2));
  const int64_t rows = z.size(0) * z.size(1);
  TORCH_CHECK(grad_rate_rows.device() == z.device() &&
                  grad_rate_rows.scalar_type() == at::kFloat &&
                  grad_rate_rows.is_contiguous() && grad_rate_rows.numel() == rows,
              "grad_rate_rows must be a contiguous float32 tensor with batch*dim (", rows,
              ") elements");
  if (z.numel() == 0) return;
  check_no_alias({&grad_z, &grad_tokens, &grad_rate_rows}, {&z, &rate, &out, &grad_out},
                 "fullscan_backward_softplus");
  c10::hip::HIPGuardMasqueradingAsCUDA guard(z.device());
  void* stream = launch_stream(z);
  const int64_t D = z.size(1), L = z.size(2);
  const int status = fpscan_scan_bwd_softplus(
      z.data_ptr(), rate.data_ptr<float>(), out.data_ptr(), grad_out.data_ptr(),
      grad_z.data_ptr(), grad_tokens.data_ptr(), grad_rate_rows.data_ptr<float>(), z.size(0), D,
      L, D * L, L, dtype_code(z.scalar_type()), stream);
  check_status(status);
}

// Look-back waits that gave up on the tensors' device since the library was loaded (waits for
// the device first).
uint64_t lookback_overruns(int64_t device) {
  c10::hip::HIPGuardMasqueradingAsCUDA guard(at::Device(at::kCUDA, (c10::DeviceIndex)device));
  unsigned long long n = 0;
  check_status(fpscan_lookback_overruns(&n));
  return n;
}

int set_launch_override(int waves_per_row, int ring_depth) {
  const int status = fpscan_set_launch_override(waves_per_row, ring_depth);
  TORCH_CHECK(status == FPSCAN_OK, "waves_per_row must be one of 0,1,2,4,8,16 and ring_depth "
              "one of 0..4");
  return status;
}

}  // namespace

PYBIND11_MODULE(TORCH_EXTENSION_NAME, m) {
  m.def("fullscan_forward", &fullscan_forward,
        "first-order linear-recurrence scan, forward or reverse, written into out (HIP, gfx950)",
        pybind11::arg("Ax"), pybind11::arg("Bx"), pybind11::arg("out"), pybind11::arg("reverse"));
  m.def("fullscan_backward", &fullscan_backward,
        "fused backward of the forward scan: (grad_gates, grad_tokens) (HIP, gfx950)",
        pybind11::arg("gates"), pybind11::arg("out"), pybind11::arg("grad_out"),
        pybind11::arg("grad_gates"), pybind11::arg("grad_tokens"));
  m.def("pscan", &pscan,
        "differentiable scan: the forward kernel, and the fused backward kernel under autograd",
        pybind11::arg("gates"), pybind11::arg("tokens"));
  m.def("fullscan_forward_cl", &fullscan_forward_cl,
        "channel-last scan of (batch, seqlen, dim) tensors along seqlen, written into out",
        pybind11::arg("Ax"), pybind11::arg("Bx"), pybind11::arg("out"), pybind11::arg("reverse"));
  m.def("fullscan_backward_cl", &fullscan_backward_cl,
        "fused backward of the channel-last forward scan: (grad_gates, grad_tokens)",
        pybind11::arg("gates"), pybind11::arg("out"), pybind11::arg("grad_out"),
        pybind11::arg("grad_gates"), pybind11::arg("grad_tokens"));
  m.def("fullscan_forward_softplus", &fullscan_forward_softplus,
        "scan with gates exp(-softplus(z) * rate[d]) computed on load, written into out",
        pybind11::arg("z"), pybind11::arg("rate"), pybind11::arg("tokens"), pybind11::arg("out"),
        pybind11::arg("reverse"));
  m.def("fullscan_backward_softplus", &fullscan_backward_softplus,
        "fused backward of the softplus-gate scan: writes grad_z, grad_tokens and one "
        "d loss / d rate partial per row", pybind11::arg("z"), pybind11::arg("rate"),
        pybind11::arg("out"), pybind11::arg("grad_out"), pybind11::arg("grad_z"),
        pybind11::arg("grad_tokens"), pybind11::arg("grad_rate_rows"));
  m.def("dimwise_forward", &dimwise_forward,
        "contraction scan, in place into Bx (HIP, gfx950)", pybind11::arg("Ax"),
        pybind11::arg("Bx"), pybind11::arg("Bh"), pybind11::arg("Wq"), pybind11::arg("Wk"));
  m.def("dimwise_groups", &fpscan_dimwise_groups,
        "Bh entries per row expected by dimwise_forward for this seqlen (0: unsupported)",
        pybind11::arg("seqlen"));
  m.def("dimwise_workspace_bytes", &fpscan_dimwise_workspace_bytes,
        "workspace dimwise_forward allocates for its tiled path (0: it takes the row kernel)",
        pybind11::arg("batch"), pybind11::arg("dim"), pybind11::arg("seqlen"),
        pybind11::arg("dtype"));
  m.def("set_launch_override", &set_launch_override,
        "tuning hook: force waves per row / ring depth (0 = built-in choice)",
        pybind11::arg("waves_per_row"), pybind11::arg("ring_depth"));
  m.def("abi_version", []() { return fpscan_abi_version(); });
  m.def("lookback_overruns", &lookback_overruns,
        "look-back waits of the tiled kernels that gave up on this device (0 in a correct run)",
        pybind11::arg("device"));
  m.def("set_lookback_test_hook", [](int64_t unpublished_tile, int spin_limit) {
    TORCH_CHECK(fpscan_set_lookback_test_hook(unpublished_tile, spin_limit) == FPSCAN_OK,
                "spin_limit must be >= 0");
  }, "test hook: never publish one tile's map and give up waits after spin_limit polls "
     "(-1, 0 restore the defaults)", pybind11::arg("unpublished_tile"),
        pybind11::arg("spin_limit"));
  m.def("set_tiling", [](int mode) {
    TORCH_CHECK(fpscan_set_tiling(mode) == FPSCAN_OK, "tiling mode must be 0, 1 or 2");
  }, "path selection: 0 automatic, 1 no tiled look-back (rows streamed; channel-last one pass "
     "or segments; dimwise's row kernel), 2 tiled whenever possible",
        pybind11::arg("mode"));
  m.def("workspace_bytes", &fpscan_workspace_bytes, pybind11::arg("batch"),
        pybind11::arg("dim"), pybind11::arg("seqlen"), pybind11::arg("dtype"),
        pybind11::arg("op"));
}
