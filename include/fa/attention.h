/* fa/attention.h -- C-ABI of the MI355X (gfx950) fused scaled-dot-product-attention forward.
 *
 * This is the drop-in boundary of libfa_hip.so. It restates the reference's frozen C++ kernel API
 * (ref:include/fa/attention.cuh:13-69, implemented by ref:src/dispatch.cu) as plain `extern "C"`
 * functions over POD types and a HIP stream, so that any FFI (ctypes, cgo, JNI, a C++ torch
 * binding) can bind it. Field order, integer codes, layout contract, error semantics and the
 * stage registry behaviour are the reference's; the names carry an `fa_` prefix instead of the
 * `fa::` namespace.
 *
 * Layout (ref:include/fa/attention.cuh:38-45): q, o are [B, H, N, D] and k, v are [B, Hkv, N, D],
 * contiguous with D fastest, in the element type `dtype`; lse is [B, H, N] fp32 and holds
 * m*scale + ln(l) per query row (natural log). Causal masking is top-left aligned (query i sees
 * keys j <= i). Query head h reads kv head h / (H / Hkv). Default scale is the caller's business
 * (torch SDPA uses 1/sqrt(D)). N % 32 == 0 and D in {64, 128} are required.
 *
 * Errors: functions never abort and never print unless FA_VERBOSE is set. fa_forward returns a
 * hipError_t value as int: hipSuccess (0); hipErrorInvalidValue for invalid parameters, a forced
 * tile that is not instantiated, misaligned pointers or a non-positive scale; hipErrorNotSupported
 * for a (stage, dtype, D, arch) this build does not implement; or the launch error itself.
 * The launch is asynchronous on `stream` and never synchronises. The library allocates nothing.
 */
#ifndef FA_ATTENTION_H_
#define FA_ATTENTION_H_

#include <hip/hip_runtime_api.h>
#include <stdbool.h>
#include <stddef.h>

/* Every entry point below is exported from libfa_hip.so; nothing else is. */
#ifndef FA_API
#define FA_API __attribute__((visibility("default")))
#endif

#ifdef __cplusplus
extern "C" {
#endif

/* Element type of q/k/v/o (ref:include/fa/attention.cuh:15-17). Scores, the running max/sum, the
 * O accumulator and lse are fp32 inside every kernel regardless of dtype. */
typedef enum fa_dtype { FA_DTYPE_F32 = 0, FA_DTYPE_F16 = 1, FA_DTYPE_BF16 = 2 } fa_dtype;

/* Stage slots, same numbers as the reference ladder (ref:include/fa/attention.cuh:19-26).
 * This build implements FUSED (3: fp32 compute rung), WMMA (4: the matrix-core kernel with
 * synchronous K/V staging) and TUNED (5: the matrix-core kernel with register-prefetched K/V). */
typedef enum fa_impl {
  FA_IMPL_NAIVE = 1,
  FA_IMPL_TILED = 2,
  FA_IMPL_FUSED = 3,
  FA_IMPL_WMMA = 4,
  FA_IMPL_TUNED = 5
} fa_impl;

/* Problem descriptor; same fields, types and order as fa::Params
 * (ref:include/fa/attention.cuh:28-36). */
typedef struct fa_params {
  int B;       /* batch */
  int H;       /* query heads */
  int Hkv;     /* key/value heads, H % Hkv == 0 */
  int N;       /* sequence length (Nq == Nkv), N % 32 == 0 */
  int D;       /* head dimension, 64 or 128 */
  float scale; /* softmax scale applied to q.k, finite and > 0 */
  bool causal; /* top-left aligned causal mask */
} fa_params;

/* Replaces fa::forward (ref:include/fa/attention.cuh:46-47, ref:src/dispatch.cu:140-161).
 * Returns a hipError_t value. `lse` must be non-null for stages 3-5. `workspace` may be NULL when
 * fa_workspace_bytes() is 0. For stage 5 it is optional even then: with a 16-byte aligned
 * workspace of fa_workspace_bytes() bytes (queried for the same params, dtype and environment)
 * the key walks are split across workgroups and a second kernel merges the parts; with NULL the
 * single-kernel path runs. A workspace must not be shared by launches that may overlap. */
FA_API int fa_forward(int impl, int dtype, const void* q, const void* k, const void* v, void* o,
               float* lse, void* workspace, const fa_params* p, hipStream_t stream);

/* Element strides of one [B, H, N, D] operand: per batch (b), per head (h) and per row (n).
 * The head dimension D is always contiguous (stride 1). A dense tensor has n = D, h = N*D,
 * b = H*N*D (Hkv in place of H for k and v). */
typedef struct fa_strides {
  long long b;
  long long h;
  long long n;
} fa_strides;

/* fa_forward over strided q/k/v/o views, e.g. the [B, H, N, D] view of a [B, N, H, D] buffer
 * (the head split of a fused QKV projection, transposed without a copy). No counterpart in the
 * reference, whose API takes dense tensors only (ref:include/fa/attention.cuh:38-45); it is the
 * "strided inputs" extension of its op. Same contract as fa_forward otherwise, plus: every stride
 * is >= 0 and a multiple of 16 bytes, so every row start is 16-byte aligned; (N-1)*n + D fits a
 * 32-bit int for every operand; o must not overlap q, k or v; lse stays dense [B, H, N].
 * Returns hipErrorInvalidValue for strides that break these rules. */
FA_API int fa_forward_strided(int impl, int dtype, const void* q, const fa_strides* q_strides,
                              const void* k, const fa_strides* k_strides, const void* v,
                              const fa_strides* v_strides, void* o, const fa_strides* o_strides,
                              float* lse, void* workspace, const fa_params* p,
                              hipStream_t stream);

/* Replaces fa::workspace_bytes (ref:include/fa/attention.cuh:51, ref:src/dispatch.cu:163-168):
 * 2*B*H*N*N*4 for the materialising stages 1-2; 0 for stages 3-4; for stage 5, 0 or, where the
 * library's cost model splits the key walks (problems that leave most of the GPU idle, such as
 * one GPU's share of a head-sharded problem), the fp32 partial O and LSE of S parts:
 * round_up(S*B*H*N*D*4, 256) + S*B*H*N*4 bytes. FA_FORCE_SPLITS (test-only) forces S <= 16. */
FA_API size_t fa_workspace_bytes(int impl, int dtype, const fa_params* p);

/* Replaces fa::impl_supports (ref:include/fa/attention.cuh:56, ref:src/dispatch.cu:170-175).
 * `arch` is the gfx number of the device as an integer (950 for gfx950) in place of the
 * reference's compute capability `sm`. */
FA_API bool fa_impl_supports(int impl, int dtype, int D, int arch);

/* Replaces fa::set_debug_overrides / get_debug_overrides (ref:include/fa/attention.cuh:60-65,
 * ref:src/dispatch.cu:177-189): forced query-tile height block_m (BR) and key-tile width block_n
 * (BC), 0 = kernel default. Stage 5's default height follows the grid: the tallest of 128 / 64 /
 * 32 rows that gives every compute unit a workgroup; results do not depend on it. Its default
 * width narrows (BC 64 at D = 64, BC 32 at D = 128) where several workgroups share a compute unit,
 * and doubles with twice the waves (four key splits per row group) where the grid fits one
 * workgroup per compute unit with fewer than two waves per SIMD; the width changes the order of
 * the softmax accumulation, so results move within the stated tolerance. A forced height alone keeps the automatic width where that tile is built and
 * otherwise takes a built width for that height, so it is valid on every grid. Process-global,
 * not thread-safe (test-only). With from_env true the environment variables FA_FORCE_BR /
 * FA_FORCE_BC override the programmatic values. */
FA_API void fa_set_debug_overrides(int block_m, int block_n);
FA_API void fa_get_debug_overrides(bool from_env, int* block_m, int* block_n);

/* Stage 5's plan for `p` on the current device under the current overrides: the query-tile
 * height (BR), the key-tile width (BC) and the number of key-walk parts (S, the value behind
 * fa_workspace_bytes). Any output pointer may be null. No counterpart in the reference, whose
 * tile height follows (D, N) alone (ref:src/stage5_tuned.cu:1011-1012); it lets callers and tests
 * see which tile a problem runs, e.g. to force the same width at another height. Needs no device
 * memory and launches nothing. Returns hipErrorInvalidValue for an invalid `p`, hipErrorNotSupported
 * for fp32 (stage 5 is fp16 / bf16 only). */
FA_API int fa_s5_plan(int dtype, const fa_params* p, int* block_m, int* block_n, int* splits);

/* Replaces fa::impl_name / dtype_name / dtype_size (ref:include/fa/attention.cuh:67-69).
 * Names are the reference's: "naive", "tiled", "fused", "wmma", "tuned"; "fp32", "fp16", "bf16";
 * "unknown" otherwise. dtype_size is 4, 2, 2, or 0 for an unknown code. */
FA_API const char* fa_impl_name(int impl);
FA_API const char* fa_dtype_name(int dtype);
FA_API size_t fa_dtype_size(int dtype);

/* gfx number of the current HIP device (e.g. 950), the value fa_impl_supports() expects; replaces
 * the reference's current_sm (ref:src/dispatch.cu:113-120). Returns a hipError_t value. */
FA_API int fa_current_arch(int* arch);

/* Human-readable text for a status returned by this library (hipGetErrorString). */
FA_API const char* fa_error_string(int status);

/* ---- split-KV decode (flash-decoding) ------------------------------------------------------
 * No counterpart in the reference's API: it is the reference's own next step (ref:README.md:
 * 1357-1358, "partial O + LSE per split, LSE-weighted combine"), built on the LSE output it emits
 * (ref:include/fa/softmax_math.cuh:65-68). Nq new query tokens per sequence attend to Nkv cached
 * keys. Layouts (dense, D fastest): q, o [B, H, Nq, D]; k, v [B, Hkv, Nkv, D]; lse [B, H, Nq] fp32
 * natural log, +inf for a row that sees no key. Query head h reads kv head h / (H / Hkv).
 * With `causal` the new tokens are the last Nq positions (bottom-right alignment): token i sees
 * keys j <= Nkv - Nq + i; without it every token sees all Nkv keys.
 * Contract: dtype fp16 or bf16, D in {64, 128}, Nq >= 1, Nkv >= 1 (any length), H % Hkv == 0,
 * (H / Hkv) * Nq <= 64 (the query rows of one kv head fill one or two 32-row tiles), finite
 * scale > 0, 16-byte aligned q/k/v/o. */
typedef struct fa_decode_params {
  int B;          /* batch */
  int H;          /* query heads */
  int Hkv;        /* key/value heads, H % Hkv == 0 */
  int Nq;         /* new query tokens per sequence */
  int Nkv;        /* cached keys per sequence */
  int D;          /* head dimension, 64 or 128 */
  float scale;    /* softmax scale applied to q.k */
  bool causal;    /* bottom-right aligned causal mask */
  int num_splits; /* splits of the key range; 0 = chosen by the library */
} fa_decode_params;

/* Splits fa_decode uses for these parameters (num_splits if > 0, capped so that every split
 * holds at least one 128-key tile; otherwise enough to fill the GPU). 0 for invalid params. */
FA_API int fa_decode_num_splits(const fa_decode_params* p);

/* Bytes of workspace fa_decode needs: fp32 partial O and LSE of every split,
 * B*Hkv*S*R*(D+1)*4 rounded up, with R = (H/Hkv)*Nq and S = fa_decode_num_splits(p); 0 when
 * S == 1 (the single split writes o and lse directly). */
FA_API size_t fa_decode_workspace_bytes(int dtype, const fa_decode_params* p);

/* Runs the decode: one split kernel (all splits in parallel) and, when S > 1, one combine
 * kernel, asynchronously on `stream`. Returns a hipError_t value: hipErrorInvalidValue for
 * invalid parameters, misaligned pointers or a missing workspace; hipErrorNotSupported for a
 * dtype, D, row count or device this build does not cover. Allocates nothing. */
FA_API int fa_decode(int dtype, const void* q, const void* k, const void* v, void* o, float* lse,
                     void* workspace, const fa_decode_params* p, hipStream_t stream);

/* Bytes of device scratch behind fa_decode_noalloc: one fixed array per GPU, held from the moment
 * the library's code is loaded on that GPU until the process ends. Sized for every problem the
 * automatic split count allows (num_splits = 0): that count keeps B*Hkv*S at most B*Hkv + 255
 * split groups, and 510 groups of 64 rows of D = 128 fp32 partials (plus their LSE) take
 * 16,842,240 bytes. */
#define FA_DECODE_SCRATCH_BYTES (17u << 20)

/* fa_decode with no workspace argument and no allocation of any kind: the splits' partial O and
 * LSE go to the library's device-resident scratch array (FA_DECODE_SCRATCH_BYTES per GPU) instead
 * of a caller workspace. No counterpart in the reference. It is for callers that cannot allocate
 * device memory: code under HIP graph capture, serving loops and harnesses that forbid hipMalloc.
 * Same contract and results as fa_decode otherwise (the same kernels run). Returns
 * hipErrorInvalidValue, before any launch, when fa_decode_workspace_bytes(dtype, p) exceeds
 * FA_DECODE_SCRATCH_BYTES (ask for fewer splits, or use fa_decode with a workspace). Every call on
 * one GPU shares that GPU's array: calls that may overlap on one GPU (different streams, or
 * different host threads) race and must be serialised by the caller. The first call on each GPU
 * looks up the array's device address (hipGetSymbolAddress, no allocation): make that first call
 * outside a stream capture (a warm-up call, or any call before capturing); later calls are plain
 * kernel launches and may be captured. */
FA_API int fa_decode_noalloc(int dtype, const void* q, const void* k, const void* v, void* o,
                             float* lse, const fa_decode_params* p, hipStream_t stream);

#ifdef __cplusplus
}
#endif

#endif /* FA_ATTENTION_H_ */
