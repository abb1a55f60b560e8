// ext.cpp -- fused_attn._C: the torch.ops.fused_attn.* custom ops over the C-ABI of libfa_hip.so.
//
// The op surface is the reference's (ref:python/fused_attn/ext.cpp): its TORCH_LIBRARY schemas
// (:220-230), its input contract with the same messages and the same order of checks (:82-126),
// forward running the highest implemented stage (:171-188), and (O, LSE) outputs from the caching
// allocator (:129-169). Below that surface the file is a plain client of include/fa/attention.h:
// the kernels are reached through fa_forward / fa_forward_strided / fa_decode only, as any other
// FFI would reach them. Host C++ only.
//
// ROCm PyTorch tensors carry the CUDA dispatch key and device type, so the kernels are registered
// for `CUDA`, and the device guard and current stream come from the HIP "masquerading as CUDA"
// helpers.
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

// ---- codes ---------------------------------------------------------------------------------------

// The stage ladder: 1 (naive) .. 5 (tuned). Stages from 3 on write the logsumexp; below that the
// op returns an empty lse (the reference's CONTRACT section 4).
constexpr int64_t kLowestStage = 1;
constexpr int64_t kHighestStage = 5;
constexpr int64_t kFirstStageWithLse = 3;

constexpr std::array<int, 3> kDtypeCodes = {FA_DTYPE_F32, FA_DTYPE_F16, FA_DTYPE_BF16};

int dtype_code(at::ScalarType t) {
  switch (t) {
    case at::kFloat:
      return FA_DTYPE_F32;
    case at::kHalf:
      return FA_DTYPE_F16;
    case at::kBFloat16:
      return FA_DTYPE_BF16;
    default:
      TORCH_CHECK(false, "fused_attn: unsupported dtype ", t,
                  " (supported: float32, float16, bfloat16)");
  }
  return -1;
}

// The library's own names ("fp32", "fp16", "bf16") are the op's dtype strings.
int dtype_code(const std::string& name) {
  for (const int code : kDtypeCodes) {
    if (name == fa_dtype_name(code)) return code;
  }
  TORCH_CHECK(false, "fused_attn: unknown dtype name '", name, "' (expected fp32, fp16 or bf16)");
  return -1;
}

void require_stage(int64_t stage) {
  TORCH_CHECK(stage >= kLowestStage && stage <= kHighestStage,
              "fused_attn: stage must be in 1..5, got ", stage);
}

// A size or count of the op as the C-ABI's int.
int as_int(int64_t value, const char* name) {
  TORCH_CHECK(value >= 0 && value <= std::numeric_limits<int>::max(), "fused_attn: ", name, "=",
              value, " does not fit fa_params (int)");
  return static_cast<int>(value);
}

// ---- the input contract -------------------------------------------------------------------------

// The q, k, v of one call. `views`: forward_strided's relaxed layout rule (a contiguous head dim
// and 16-byte-multiple strides) instead of the op's dense [B, H, N, D].
struct Operands {
  const at::Tensor& q;
  const at::Tensor& k;
  const at::Tensor& v;
  bool views;

  std::array<const at::Tensor*, 3> each() const { return {&q, &k, &v}; }
};

// The contract as a list of rules, checked in the reference's order: the first broken rule is the
// error a caller sees. Every rule raises a RuntimeError with its message; none lets a bad operand
// reach a kernel.
using Rule = void (*)(const Operands&);

void on_one_device(const Operands& x) {
  TORCH_CHECK(x.q.is_cuda() && x.k.is_cuda() && x.v.is_cuda(),
              "fused_attn: q, k, v must be CUDA (ROCm/HIP device) tensors");
  TORCH_CHECK(x.q.device() == x.k.device() && x.q.device() == x.v.device(),
              "fused_attn: q, k, v must live on the same device");
}

void four_dims(const Operands& x) {
  TORCH_CHECK(x.q.dim() == 4 && x.k.dim() == 4 && x.v.dim() == 4,
              "fused_attn: q, k, v must be [B, H, N, D]; got ", x.q.dim(), "-D, ", x.k.dim(),
              "-D, ", x.v.dim(), "-D");
}

void readable_layout(const Operands& x) {
  if (!x.views) {
    TORCH_CHECK(x.q.is_contiguous() && x.k.is_contiguous() && x.v.is_contiguous(),
                "fused_attn: q, k, v must be contiguous [B, H, N, D] (call .contiguous())");
    return;
  }
  for (const at::Tensor* t : x.each()) {
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

// The kernels read 16 bytes at a time: an offset view such as t[2:] is refused here instead of
// faulting in the kernel.
void aligned_bases(const Operands& x) {
  for (const at::Tensor* t : x.each()) {
    TORCH_CHECK(reinterpret_cast<std::uintptr_t>(t->data_ptr()) % 16 == 0,
                "fused_attn: q/k/v must be 16-byte aligned (use a fresh contiguous tensor)");
  }
}

void one_dtype(const Operands& x) {
  TORCH_CHECK(x.q.scalar_type() == x.k.scalar_type() && x.q.scalar_type() == x.v.scalar_type(),
              "fused_attn: q, k, v must share one dtype; got ", x.q.scalar_type(), ", ",
              x.k.scalar_type(), ", ", x.v.scalar_type());
  (void)dtype_code(x.q.scalar_type());
}

void matching_shapes(const Operands& x) {
  const int64_t B = x.q.size(0), H = x.q.size(1), N = x.q.size(2), D = x.q.size(3);
  const int64_t Hkv = x.k.size(1);
  TORCH_CHECK(x.k.size(0) == B && x.v.size(0) == B, "fused_attn: batch mismatch between q, k, v");
  TORCH_CHECK(x.v.size(1) == Hkv, "fused_attn: k and v must have the same number of heads");
  TORCH_CHECK(x.k.size(2) == N && x.v.size(2) == N,
              "fused_attn: Nq == Nkv is required (got Nq=", N, ", Nkv=", x.k.size(2), ")");
  TORCH_CHECK(x.k.size(3) == D && x.v.size(3) == D,
              "fused_attn: head-dim mismatch between q, k, v");
  TORCH_CHECK(D == 64 || D == 128, "fused_attn: D must be 64 or 128, got ", D);
  TORCH_CHECK(N % 32 == 0, "fused_attn: N must be a multiple of 32, got ", N,
              " (ragged sequence lengths are a stated limitation)");
  TORCH_CHECK(Hkv >= 1 && H % Hkv == 0, "fused_attn: H=", H, " must be a multiple of Hkv=", Hkv);
}

constexpr std::array<Rule, 6> kContract = {on_one_device, four_dims,  readable_layout,
                                           aligned_bases, one_dtype, matching_shapes};

// fa_params of a call that keeps the contract.
fa_params params_of(const Operands& x, bool is_causal, double scale) {
  for (const Rule rule : kContract) rule(x);
  fa_params p;
  p.B = as_int(x.q.size(0), "B");
  p.H = as_int(x.q.size(1), "H");
  p.Hkv = as_int(x.k.size(1), "Hkv");
  p.N = as_int(x.q.size(2), "N");
  p.D = as_int(x.q.size(3), "D");
  p.scale = static_cast<float>(scale);
  p.causal = is_causal;
  return p;
}

// ---- launching ----------------------------------------------------------------------------------

// q's device made current for the rest of the call (the stream, the arch query and every
// allocation follow it), with its architecture and current stream.
struct DeviceScope {
  explicit DeviceScope(const at::Tensor& q)
      : guard(q.device()),
        stream(c10::hip::getCurrentHIPStreamMasqueradingAsCUDA(q.device().index()).stream()) {
    const int rc = fa_current_arch(&arch);
    TORCH_CHECK(rc == 0, "fused_attn: cannot query the device architecture: ", fa_error_string(rc));
  }
  c10::hip::HIPGuardMasqueradingAsCUDA guard;
  hipStream_t stream;
  int arch = 0;
};

// The highest stage implemented for (dtype, D) on `arch`, 0 if none.
int highest_stage(int dtype, int D, int arch) {
  for (int64_t s = kHighestStage; s >= kLowestStage; --s) {
    if (fa_impl_supports(static_cast<int>(s), dtype, D, arch)) return static_cast<int>(s);
  }
  return 0;
}

// A byte tensor of the size fa_workspace_bytes asks for (undefined when it asks for none): the
// materialising stages' scratch, or stage 5's optional split-walk workspace. Released by the
// caching allocator in stream order after the asynchronous launch.
at::Tensor workspace_for(int stage, int dtype, const fa_params& p, const at::Tensor& like) {
  const size_t bytes = fa_workspace_bytes(stage, dtype, &p);
  if (bytes == 0) return at::Tensor();
  return at::empty({static_cast<int64_t>(bytes)}, like.options().dtype(at::kByte));
}

void* data_or_null(const at::Tensor& t) { return t.defined() ? t.data_ptr() : nullptr; }

void check_launched(int status, int stage) {
  TORCH_CHECK(status == 0, "fused_attn: stage ", stage, " (", fa_impl_name(stage),
              ") failed: ", fa_error_string(status));
}

fa_strides strides_of(const at::Tensor& t) {
  fa_strides s;
  s.b = t.stride(0);
  s.h = t.stride(1);
  s.n = t.stride(2);
  return s;
}

// A dense tensor with q's shape whose memory order follows q's strides (outermost first): for the
// [B, H, N, D] view of a [B, N, H, D] buffer the result is a [B, N, H, D] buffer seen as
// [B, H, N, D], so a caller's transpose back to [B, N, H*D] is free. A contiguous q gives a
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

// ---- the ops ------------------------------------------------------------------------------------

// forward_stage: one explicit stage; (o, lse), lse empty below stage 3.
std::tuple<at::Tensor, at::Tensor> forward_stage_cuda(const at::Tensor& q, const at::Tensor& k,
                                                      const at::Tensor& v, bool is_causal,
                                                      double scale, int64_t stage) {
  require_stage(stage);
  const fa_params p = params_of(Operands{q, k, v, false}, is_causal, scale);
  const DeviceScope dev(q);
  const int impl = static_cast<int>(stage);
  const int dtype = dtype_code(q.scalar_type());
  TORCH_CHECK(fa_impl_supports(impl, dtype, p.D, dev.arch), "fused_attn: stage ", stage, " (",
              fa_impl_name(impl), ") is not implemented for ", fa_dtype_name(dtype), " D=", p.D,
              " on gfx", dev.arch);
  at::Tensor o = at::empty_like(q);
  const auto f32 = q.options().dtype(at::kFloat);
  at::Tensor lse = stage >= kFirstStageWithLse ? at::empty({p.B, p.H, p.N}, f32) : at::empty({0}, f32);
  const at::Tensor ws = workspace_for(impl, dtype, p, q);
  check_launched(fa_forward(impl, dtype, q.data_ptr(), k.data_ptr(), v.data_ptr(), o.data_ptr(),
                            stage >= kFirstStageWithLse ? lse.data_ptr<float>() : nullptr,
                            data_or_null(ws), &p, dev.stream),
                 impl);
  return std::make_tuple(std::move(o), std::move(lse));
}

// forward: the highest implemented stage for (dtype, D, arch); O only.
at::Tensor forward_cuda(const at::Tensor& q, const at::Tensor& k, const at::Tensor& v,
                        bool is_causal, double scale) {
  const fa_params p = params_of(Operands{q, k, v, false}, is_causal, scale);
  const int dtype = dtype_code(q.scalar_type());
  int stage = 0, arch = 0;
  {
    const DeviceScope dev(q);
    arch = dev.arch;
    stage = highest_stage(dtype, p.D, arch);
  }
  TORCH_CHECK(stage != 0, "fused_attn: no stage is implemented for ", fa_dtype_name(dtype), " D=",
              p.D, " on gfx", arch);
  return std::get<0>(forward_stage_cuda(q, k, v, is_causal, scale, stage));
}

// forward_strided: forward over strided [B, H, N, D] views (fa_forward_strided), read in place;
// O comes back dense in q's memory order. No counterpart in the reference (its op takes dense
// tensors); it removes the layout copies around the op in a transformer block.
at::Tensor forward_strided_cuda(const at::Tensor& q, const at::Tensor& k, const at::Tensor& v,
                                bool is_causal, double scale) {
  const fa_params p = params_of(Operands{q, k, v, true}, is_causal, scale);
  const DeviceScope dev(q);
  const int dtype = dtype_code(q.scalar_type());
  const int stage = highest_stage(dtype, p.D, dev.arch);
  TORCH_CHECK(stage >= kFirstStageWithLse, "fused_attn: no stage is implemented for ",
              fa_dtype_name(dtype), " D=", p.D, " on gfx", dev.arch);
  at::Tensor o = empty_in_layout_of(q);
  at::Tensor lse = at::empty({p.B, p.H, p.N}, q.options().dtype(at::kFloat));
  const std::array<fa_strides, 4> st = {strides_of(q), strides_of(k), strides_of(v),
                                        strides_of(o)};
  const at::Tensor ws = workspace_for(stage, dtype, p, q);
  check_launched(fa_forward_strided(stage, dtype, q.data_ptr(), &st[0], k.data_ptr(), &st[1],
                                    v.data_ptr(), &st[2], o.data_ptr(), &st[3],
                                    lse.data_ptr<float>(), data_or_null(ws), &p, dev.stream),
                 stage);
  return o;
}

// decode: split-KV decode (fa_decode). q [B, H, Nq, D]; k, v [B, Hkv, Nkv, D]; returns
// (o [B, H, Nq, D], lse [B, H, Nq] fp32). No counterpart in the reference's op (its stated next
// step, ref:README.md:1357-1358). The split partials live in a byte tensor from the caching
// allocator, released in stream order like the forward's workspace.
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
  const DeviceScope dev(q);
  fa_decode_params p{};
  p.B = as_int(q.size(0), "B");
  p.H = as_int(q.size(1), "H");
  p.Hkv = as_int(k.size(1), "Hkv");
  p.Nq = as_int(q.size(2), "Nq");
  p.Nkv = as_int(k.size(2), "Nkv");
  p.D = as_int(q.size(3), "D");
  p.scale = static_cast<float>(scale);
  p.causal = is_causal;
  p.num_splits = as_int(num_splits, "num_splits");
  const int dtype = dtype_code(q.scalar_type());
  at::Tensor o = at::empty_like(q);
  at::Tensor lse = at::empty({p.B, p.H, p.Nq}, q.options().dtype(at::kFloat));
  const size_t ws_bytes = fa_decode_workspace_bytes(dtype, &p);
  const at::Tensor ws =
      ws_bytes > 0 ? at::empty({static_cast<int64_t>(ws_bytes)}, q.options().dtype(at::kByte))
                   : at::Tensor();
  const int err = fa_decode(dtype, q.data_ptr(), k.data_ptr(), v.data_ptr(), o.data_ptr(),
                            lse.data_ptr<float>(), data_or_null(ws), &p, dev.stream);
  TORCH_CHECK(err != static_cast<int>(hipErrorNotSupported),
              "fused_attn: decode is not implemented for ", fa_dtype_name(dtype), " D=", p.D,
              " with (H/Hkv)*Nq=", static_cast<int64_t>(p.H / p.Hkv) * p.Nq,
              " (supported: fp16/bf16, D 64 or 128, (H/Hkv)*Nq <= 64, gfx950)");
  TORCH_CHECK(err == 0, "fused_attn: decode failed: ", fa_error_string(err));
  return {o, lse};
}

// TEST-ONLY: forces BR / BC (0 = default) for the tile-invariance tests; process-global.
void set_debug_overrides_op(int64_t block_m, int64_t block_n) {
  fa_set_debug_overrides(as_int(block_m, "block_m"), as_int(block_n, "block_n"));
}

bool impl_supports_op(int64_t stage, std::string dtype, int64_t D) {
  require_stage(stage);
  if (c10::hip::device_count() == 0) return false;
  const int code = dtype_code(dtype);
  const int d = as_int(D, "D");
  int arch = 0;
  const int rc = fa_current_arch(&arch);
  TORCH_CHECK(rc == 0, "fused_attn: cannot query the device architecture: ", fa_error_string(rc));
  return fa_impl_supports(static_cast<int>(stage), code, d, arch);
}

std::string impl_name_op(int64_t stage) {
  require_stage(stage);
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
