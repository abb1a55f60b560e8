// ext.cpp -- fused_attn._C: the PyTorch-ROCm custom-op binding over the C-ABI of libfa_hip.so.
//
// Mirrors the reference binding (ref:python/fused_attn/ext.cpp): the same TORCH_LIBRARY schemas
// (ref:python/fused_attn/ext.cpp:220-230), the same input contract checks and error messages
// (:82-126), the same stage selection (:171-188) and the same (O, LSE) allocation (:129-169). The
// kernels are reached only through include/fa/attention.h (fa_forward & co.), i.e. this file is a
// consumer of the C-ABI exactly as any other FFI would be. Host C++ only.
//
// ROCm PyTorch tensors carry the CUDA dispatch key and device type, so the kernels are
// registered for `CUDA`, and the device guard / current stream come from the HIP
// "masquerading as CUDA" helpers.
#include <Python.h>  // first, per the CPython docs
// (this comment ends the include block so formatters keep Python.h first)

#include <ATen/ATen.h>
#include <ATen/hip/impl/HIPGuardImplMasqueradingAsCUDA.h>
#include <ATen/hip/impl/HIPStreamMasqueradingAsCUDA.h>
#include <c10/hip/HIPFunctions.h>
#include <torch/library.h>

#include <algorithm>
#include <array>
#include <cstdint>
#include <limits>
#include <string>
#include <tuple>
#include <vector>

#include "fa/attention.h"

namespace {

constexpr int64_t kMinStage = 1;
constexpr int64_t kMaxStage = 5;
// Stages whose kernels write the logsumexp; 1-2 would return an empty lse (CONTRACT section 4 of
// the reference, ref:python/fused_attn/ext.cpp:43-45).
constexpr int64_t kFirstLseStage = 3;

int to_fa_dtype(at::ScalarType t) {
  if (t == at::kFloat) return FA_DTYPE_F32;
  if (t == at::kHalf) return FA_DTYPE_F16;
  TORCH_CHECK(t == at::kBFloat16, "fused_attn: unsupported dtype ", t,
              " (supported: float32, float16, bfloat16)");
  return FA_DTYPE_BF16;
}

int dtype_from_name(const std::string& name) {
  if (name == "fp32") return FA_DTYPE_F32;
  if (name == "fp16") return FA_DTYPE_F16;
  TORCH_CHECK(name == "bf16", "fused_attn: unknown dtype name '", name,
              "' (expected fp32, fp16 or bf16)");
  return FA_DTYPE_BF16;
}

// gfx number of the CURRENT device (950 for MI355X), the encoding fa_impl_supports() expects.
// Callers make the right device current with a guard first.
int current_arch() {
  int arch = 0;
  const int rc = fa_current_arch(&arch);
  TORCH_CHECK(rc == 0, "fused_attn: cannot query the device architecture: ", fa_error_string(rc));
  return arch;
}

void check_stage(int64_t stage) {
  TORCH_CHECK(stage >= kMinStage && stage <= kMaxStage, "fused_attn: stage must be in 1..5, got ",
              stage);
}

int checked_int(int64_t v, const char* what) {
  TORCH_CHECK(v >= 0 && v <= std::numeric_limits<int>::max(), "fused_attn: ", what, "=", v,
              " does not fit fa_params (int)");
  return static_cast<int>(v);
}

// The frozen input contract; every violation is a RuntimeError with a message, never a device
// fault (ref:python/fused_attn/ext.cpp:82-126). `dense` is the reference's contiguity rule;
// forward_strided relaxes it to a contiguous head dim with 16-byte-aligned strides.
fa_params make_params(const at::Tensor& q, const at::Tensor& k, const at::Tensor& v,
                      bool is_causal, double scale, bool dense = true) {
  TORCH_CHECK(q.is_cuda() && k.is_cuda() && v.is_cuda(),
              "fused_attn: q, k, v must be CUDA (ROCm/HIP device) tensors");
  TORCH_CHECK(q.device() == k.device() && q.device() == v.device(),
              "fused_attn: q, k, v must live on the same device");
  TORCH_CHECK(q.dim() == 4 && k.dim() == 4 && v.dim() == 4,
              "fused_attn: q, k, v must be [B, H, N, D]; got ", q.dim(), "-D, ", k.dim(), "-D, ",
              v.dim(), "-D");
  if (dense) {
    TORCH_CHECK(q.is_contiguous() && k.is_contiguous() && v.is_contiguous(),
                "fused_attn: q, k, v must be contiguous [B, H, N, D] (call .contiguous())");
  } else {
    for (const at::Tensor* t : {&q, &k, &v}) {
      TORCH_CHECK(t->stride(3) == 1 || t->size(3) == 1,
                  "fused_attn: forward_strided needs a contiguous head dim (stride(-1) == 1)");
      const int64_t per16 = 16 / static_cast<int64_t>(t->element_size());
      for (int d = 0; d < 3; ++d) {
        TORCH_CHECK(t->stride(d) >= 0 && t->stride(d) % per16 == 0,
                    "fused_attn: forward_strided needs batch/head/row strides that are multiples "
                    "of 16 bytes, got stride(", d, ")=", t->stride(d));
      }
    }
  }
  // The kernels use 16-byte vector loads; a contiguous offset view such as t[2:] is not 16-byte
  // aligned and is refused here rather than faulting inside the kernel.
  for (const at::Tensor* t : {&q, &k, &v}) {
    TORCH_CHECK(reinterpret_cast<std::uintptr_t>(t->data_ptr()) % 16 == 0,
                "fused_attn: q/k/v must be 16-byte aligned (use a fresh contiguous tensor)");
  }
  TORCH_CHECK(q.scalar_type() == k.scalar_type() && q.scalar_type() == v.scalar_type(),
              "fused_attn: q, k, v must share one dtype; got ", q.scalar_type(), ", ",
              k.scalar_type(), ", ", v.scalar_type());
  (void)to_fa_dtype(q.scalar_type());

  const int64_t B = q.size(0), H = q.size(1), N = q.size(2), D = q.size(3);
  const int64_t Hkv = k.size(1);
  TORCH_CHECK(k.size(0) == B && v.size(0) == B, "fused_attn: batch mismatch between q, k, v");
  TORCH_CHECK(v.size(1) == Hkv, "fused_attn: k and v must have the same number of heads");
  TORCH_CHECK(k.size(2) == N && v.size(2) == N,
              "fused_attn: Nq == Nkv is required (got Nq=", N, ", Nkv=", k.size(2), ")");
  TORCH_CHECK(k.size(3) == D && v.size(3) == D, "fused_attn: head-dim mismatch between q, k, v");
  TORCH_CHECK(D == 64 || D == 128, "fused_attn: D must be 64 or 128, got ", D);
  TORCH_CHECK(N % 32 == 0, "fused_attn: N must be a multiple of 32, got ", N,
              " (ragged sequence lengths are a stated limitation)");
  TORCH_CHECK(Hkv >= 1 && H % Hkv == 0, "fused_attn: H=", H, " must be a multiple of Hkv=", Hkv);

  fa_params p;
  p.B = checked_int(B, "B");
  p.H = checked_int(H, "H");
  p.Hkv = checked_int(Hkv, "Hkv");
  p.N = checked_int(N, "N");
  p.D = checked_int(D, "D");
  p.scale = static_cast<float>(scale);
  p.causal = is_causal;
  return p;
}

// Runs one explicit stage; returns (o, lse), lse empty for stages < 3
// (ref:python/fused_attn/ext.cpp:128-169).
std::tuple<at::Tensor, at::Tensor> run_stage(const at::Tensor& q, const at::Tensor& k,
                                             const at::Tensor& v, bool is_causal, double scale,
                                             int64_t stage) {
  check_stage(stage);
  const fa_params p = make_params(q, k, v, is_causal, scale);
  const c10::hip::HIPGuardMasqueradingAsCUDA guard(q.device());
  const int impl = static_cast<int>(stage);
  const int dtype = to_fa_dtype(q.scalar_type());
  const int arch = current_arch();
  TORCH_CHECK(fa_impl_supports(impl, dtype, p.D, arch), "fused_attn: stage ", stage, " (",
              fa_impl_name(impl), ") is not implemented for ", fa_dtype_name(dtype), " D=", p.D,
              " on gfx", arch);

  at::Tensor o = at::empty_like(q);
  const bool has_lse = stage >= kFirstLseStage;
  at::Tensor lse = has_lse ? at::empty({p.B, p.H, p.N}, q.options().dtype(at::kFloat))
                           : at::empty({0}, q.options().dtype(at::kFloat));
  // Scratch for the materialising stages, and stage 5's optional workspace where it splits key
  // walks (0 bytes otherwise); freed stream-ordered by the caching allocator after the
  // asynchronous launch.
  const size_t ws_bytes = fa_workspace_bytes(impl, dtype, &p);
  at::Tensor workspace;
  void* ws_ptr = nullptr;
  if (ws_bytes > 0) {
    workspace = at::empty({static_cast<int64_t>(ws_bytes)}, q.options().dtype(at::kByte));
    ws_ptr = workspace.data_ptr();
  }
  const hipStream_t stream =
      c10::hip::getCurrentHIPStreamMasqueradingAsCUDA(q.device().index()).stream();
  const int err = fa_forward(impl, dtype, q.data_ptr(), k.data_ptr(), v.data_ptr(), o.data_ptr(),
                             has_lse ? lse.data_ptr<float>() : nullptr, ws_ptr, &p, stream);
  TORCH_CHECK(err == 0, "fused_attn: stage ", stage, " (", fa_impl_name(impl),
              ") failed: ", fa_error_string(err));
  return std::make_tuple(std::move(o), std::move(lse));
}

fa_strides strides_of(const at::Tensor& t) {
  fa_strides s;
  s.b = t.stride(0);
  s.h = t.stride(1);
  s.n = t.stride(2);
  return s;
}

// A dense tensor with q's shape whose memory order follows q's strides (outermost first): for
// the [B, H, N, D] view of a [B, N, H, D] buffer the result is a [B, N, H, D] buffer seen as
// [B, H, N, D], so the caller's transpose back to [B, N, H*D] is free. Contiguous q gives a
// contiguous result. ops.py's fake kernel applies the same rule.
at::Tensor empty_in_layout_of(const at::Tensor& q) {
  std::array<int64_t, 4> order = {0, 1, 2, 3};
  std::stable_sort(order.begin(), order.end(),
                   [&](int64_t a, int64_t b) { return q.stride(a) > q.stride(b); });
  std::vector<int64_t> sizes, inverse(4);
  for (int i = 0; i < 4; ++i) {
    sizes.push_back(q.size(order[i]));
    inverse[order[i]] = i;
  }
  return at::empty(sizes, q.options()).permute(inverse);
}

// forward_strided: as forward (best stage, O only) over strided views (fa_forward_strided). No
// counterpart in the reference (its op requires dense tensors); it removes the layout copies
// around the op in a transformer block.
at::Tensor forward_strided_cuda(const at::Tensor& q, const at::Tensor& k, const at::Tensor& v,
                                bool is_causal, double scale) {
  const fa_params p = make_params(q, k, v, is_causal, scale, /*dense=*/false);
  const c10::hip::HIPGuardMasqueradingAsCUDA guard(q.device());
  const int dtype = to_fa_dtype(q.scalar_type());
  const int arch = current_arch();
  int stage = 0;
  for (int s = static_cast<int>(kMaxStage); s >= static_cast<int>(kMinStage) && stage == 0; --s) {
    if (fa_impl_supports(s, dtype, p.D, arch)) stage = s;
  }
  TORCH_CHECK(stage >= kFirstLseStage, "fused_attn: no stage is implemented for ",
              fa_dtype_name(dtype), " D=", p.D, " on gfx", arch);
  at::Tensor o = empty_in_layout_of(q);
  at::Tensor lse = at::empty({p.B, p.H, p.N}, q.options().dtype(at::kFloat));
  const fa_strides qs = strides_of(q), ks = strides_of(k), vs = strides_of(v), os = strides_of(o);
  // Stage 5's optional workspace (split key walks), as in forward.
  const size_t ws_bytes = fa_workspace_bytes(stage, dtype, &p);
  at::Tensor workspace;
  if (ws_bytes > 0) {
    workspace = at::empty({static_cast<int64_t>(ws_bytes)}, q.options().dtype(at::kByte));
  }
  const hipStream_t stream =
      c10::hip::getCurrentHIPStreamMasqueradingAsCUDA(q.device().index()).stream();
  const int err = fa_forward_strided(stage, dtype, q.data_ptr(), &qs, k.data_ptr(), &ks,
                                     v.data_ptr(), &vs, o.data_ptr(), &os, lse.data_ptr<float>(),
                                     ws_bytes > 0 ? workspace.data_ptr() : nullptr, &p, stream);
  TORCH_CHECK(err == 0, "fused_attn: stage ", stage, " (", fa_impl_name(stage),
              ") failed: ", fa_error_string(err));
  return o;
}

// forward: the highest implemented stage for (dtype, D, arch) (ref:python/fused_attn/ext.cpp:171-188).
at::Tensor forward_cuda(const at::Tensor& q, const at::Tensor& k, const at::Tensor& v,
                        bool is_causal, double scale) {
  const fa_params p = make_params(q, k, v, is_causal, scale);
  const c10::hip::HIPGuardMasqueradingAsCUDA guard(q.device());
  const int dtype = to_fa_dtype(q.scalar_type());
  const int arch = current_arch();
  for (int64_t stage = kMaxStage; stage >= kMinStage; --stage) {
    if (fa_impl_supports(static_cast<int>(stage), dtype, p.D, arch)) {
      return std::get<0>(run_stage(q, k, v, is_causal, scale, stage));
    }
  }
  TORCH_CHECK(false, "fused_attn: no stage is implemented for ", fa_dtype_name(dtype), " D=", p.D,
              " on gfx", arch);
  return at::Tensor();
}

std::tuple<at::Tensor, at::Tensor> forward_stage_cuda(const at::Tensor& q, const at::Tensor& k,
                                                      const at::Tensor& v, bool is_causal,
                                                      double scale, int64_t stage) {
  return run_stage(q, k, v, is_causal, scale, stage);
}

// decode: split-KV decode (fa_decode). q [B, H, Nq, D]; k, v [B, Hkv, Nkv, D]; returns
// (o [B, H, Nq, D], lse [B, H, Nq] fp32). No counterpart in the reference's op (its stated next
// step, ref:README.md:1357-1358). The workspace is a byte tensor from the caching allocator,
// released in stream order like the reference's stage workspace
// (ref:python/fused_attn/ext.cpp:143-157).
std::tuple<at::Tensor, at::Tensor> decode_cuda(const at::Tensor& q, const at::Tensor& k,
                                               const at::Tensor& v, bool is_causal, double scale,
                                               int64_t num_splits) {
  TORCH_CHECK(q.is_cuda() && k.is_cuda() && v.is_cuda(),
              "fused_attn: decode inputs must be CUDA (HIP) tensors");
  TORCH_CHECK(q.dim() == 4 && k.dim() == 4 && v.dim() == 4,
              "fused_attn: decode expects q [B, H, Nq, D] and k, v [B, Hkv, Nkv, D]");
  TORCH_CHECK(q.scalar_type() == k.scalar_type() && q.scalar_type() == v.scalar_type(),
              "fused_attn: q, k, v must share one dtype");
  TORCH_CHECK(q.is_contiguous() && k.is_contiguous() && v.is_contiguous(),
              "fused_attn: decode needs contiguous q, k, v");
  TORCH_CHECK(k.sizes() == v.sizes(), "fused_attn: k and v must have the same shape");
  TORCH_CHECK(q.size(0) == k.size(0) && q.size(3) == k.size(3),
              "fused_attn: q and k must share B and D");
  TORCH_CHECK(k.size(1) > 0 && q.size(1) % k.size(1) == 0,
              "fused_attn: H must be a multiple of Hkv");
  TORCH_CHECK(scale > 0.0, "fused_attn: scale must be > 0");
  const c10::hip::HIPGuardMasqueradingAsCUDA guard(q.device());
  fa_decode_params p{};
  p.B = checked_int(q.size(0), "B");
  p.H = checked_int(q.size(1), "H");
  p.Hkv = checked_int(k.size(1), "Hkv");
  p.Nq = checked_int(q.size(2), "Nq");
  p.Nkv = checked_int(k.size(2), "Nkv");
  p.D = checked_int(q.size(3), "D");
  p.scale = static_cast<float>(scale);
  p.causal = is_causal;
  p.num_splits = checked_int(num_splits, "num_splits");
  const int dtype = to_fa_dtype(q.scalar_type());
  at::Tensor o = at::empty_like(q);
  at::Tensor lse = at::empty({p.B, p.H, p.Nq}, q.options().dtype(at::kFloat));
  const size_t ws_bytes = fa_decode_workspace_bytes(dtype, &p);
  at::Tensor ws;
  if (ws_bytes > 0) ws = at::empty({static_cast<int64_t>(ws_bytes)}, q.options().dtype(at::kByte));
  const hipStream_t stream =
      c10::hip::getCurrentHIPStreamMasqueradingAsCUDA(q.device().index()).stream();
  const int err = fa_decode(dtype, q.data_ptr(), k.data_ptr(), v.data_ptr(), o.data_ptr(),
                            lse.data_ptr<float>(), ws_bytes > 0 ? ws.data_ptr() : nullptr, &p,
                            stream);
  TORCH_CHECK(err != static_cast<int>(hipErrorNotSupported),
              "fused_attn: decode is not implemented for ", fa_dtype_name(dtype), " D=", p.D,
              " with (H/Hkv)*Nq=", static_cast<int64_t>(p.H / p.Hkv) * p.Nq,
              " (supported: fp16/bf16, D 64 or 128, (H/Hkv)*Nq <= 64, gfx950)");
  TORCH_CHECK(err == 0, "fused_attn: decode failed: ", fa_error_string(err));
  return {o, lse};
}

// TEST-ONLY: forces BR / BC (0 = default) for the tile-invariance tests; process-global.
void set_debug_overrides_op(int64_t block_m, int64_t block_n) {
  fa_set_debug_overrides(checked_int(block_m, "block_m"), checked_int(block_n, "block_n"));
}

bool impl_supports_op(int64_t stage, std::string dtype, int64_t D) {
  check_stage(stage);
  if (c10::hip::device_count() == 0) return false;
  const int dt = dtype_from_name(dtype);
  return fa_impl_supports(static_cast<int>(stage), dt, checked_int(D, "D"), current_arch());
}

std::string impl_name_op(int64_t stage) {
  check_stage(stage);
  return std::string(fa_impl_name(static_cast<int>(stage)));
}

}  // namespace

TORCH_LIBRARY(fused_attn, m) {
  m.def("forward(Tensor q, Tensor k, Tensor v, bool is_causal, float scale) -> Tensor");
  m.def(
      "forward_stage(Tensor q, Tensor k, Tensor v, bool is_causal, float scale, int stage)"
      " -> (Tensor, Tensor)");
  // Extension beyond the reference's frozen schemas: strided q/k/v views.
  m.def("forward_strided(Tensor q, Tensor k, Tensor v, bool is_causal, float scale) -> Tensor");
  // Extension beyond the reference's frozen schemas: split-KV decode (Nq != Nkv).
  m.def(
      "decode(Tensor q, Tensor k, Tensor v, bool is_causal, float scale, int num_splits)"
      " -> (Tensor, Tensor)");
  // Scalar-only ops have no dispatch key: their kernels are catch-alls.
  m.def("set_debug_overrides(int block_m, int block_n) -> ()", &set_debug_overrides_op);
  m.def("impl_supports(int stage, str dtype, int D) -> bool", &impl_supports_op);
  m.def("impl_name(int stage) -> str", &impl_name_op);
}

TORCH_LIBRARY_IMPL(fused_attn, CUDA, m) {
  m.impl("forward", &forward_cuda);
  m.impl("forward_stage", &forward_stage_cuda);
  m.impl("forward_strided", &forward_strided_cuda);
  m.impl("decode", &decode_cuda);
}

// Importing the .so runs the TORCH_LIBRARY static initialisers; the module exports nothing.
extern "C" PyObject* PyInit__C(void) {
  static struct PyModuleDef module_def = {
      PyModuleDef_HEAD_INIT,
      "_C",
      "fused_attn extension (MI355X). The ops live in torch.ops.fused_attn.*",
      -1,
      nullptr,
      nullptr,
      nullptr,
      nullptr,
      nullptr,
  };
  return PyModule_Create(&module_def);
}
