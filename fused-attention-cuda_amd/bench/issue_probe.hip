// issue_probe -- the issue-rate, co-issue and bandwidth facts the stage-5 kernel's cycle budget
// rests on, measured on the GPU it runs on (gfx950). Every kernel here is straight-line inline
// assembly on registers (and LDS / global reads for the bandwidth parts): no stores except one
// timestamp per wave, no data-dependent control flow, every access in bounds.
//
//   1. VALU issue: cycles per wave64 instruction with 1, 2 and 4 waves per SIMD issuing the same
//      op (v_fma_f32, v_exp_f32, v_cvt_pk_f16_f32, v_dot2c_f32_f16, v_add_f32, v_max_f32) -- the
//      softmax's instructions.
//   2. Co-issue: one wave per SIMD streaming v_mfma_f32_32x32x16_f16 next to one (or two) waves
//      streaming each VALU op: the MFMA wave's cycles per MFMA and the VALU wave's per op.
//   3. LDS reads: cycles per instruction per CU for ds_read_b128 and ds_read_b64_tr_b16
//      (conflict-free addresses) with 8 and 16 waves.
//   4. HBM read ceiling: 1 GiB read with dwordx4 loads, and streamed through LDS with
//      global_load_lds_dwordx4 (the tile path of the attention kernels) at 256 and 512 workgroups.
//   5. One key-tile step of stage 5 without memory: per SIMD, the MFMAs of the step and the
//      softmax instructions of its scores (per 8 scores: 8 v_fma_f32, 8 v_exp_f32, 4
//      v_cvt_pk_f16_f32 and the row sum), arranged as the kernel runs them (8 waves, every wave
//      exponentiates then multiplies, one barrier per step), as a ping-pong (two groups of waves
//      alternating the MFMA and the softmax half, a barrier per half) and with 16 waves; the row
//      sum as the kernel's v_dot2c_f32_f16 chain, as fp32 adds into two accumulators, or absent.
//
// Cycles are s_memtime counts (the shader clock), averaged over the waves of 256 workgroups (one
// per CU, all CUs busy, as in the attention kernels). usage: issue_probe [iterations]
#include <hip/hip_runtime.h>

#include <cstdint>
#include <cstdio>
#include <cstdlib>
#include <string>
#include <vector>

namespace {

#define CHECK(x)                                                                          \
  do {                                                                                    \
    hipError_t e_ = (x);                                                                  \
    if (e_ != hipSuccess) {                                                               \
      std::fprintf(stderr, "issue_probe: %s at %s:%d\n", hipGetErrorString(e_), __FILE__, \
                   __LINE__);                                                             \
      std::exit(1);                                                                       \
    }                                                                                     \
  } while (0)

// Registers v32..v83 belong to the probes (at most 84 VGPRs, so 16 waves fit a CU).
#define CLOBBER                                                                                  \
  "v32", "v33", "v34", "v35", "v36", "v37", "v38", "v39", "v40", "v41", "v42", "v43", "v44",     \
      "v45", "v46", "v47", "v48", "v49", "v50", "v51", "v52", "v53", "v54", "v55", "v56", "v57", \
      "v58", "v59", "v60", "v61", "v62", "v63", "v64", "v65", "v66", "v67", "v68", "v69", "v70", \
      "v71", "v72", "v73", "v74", "v75", "v76", "v77", "v78", "v79", "v80", "v81", "v82", "v83"
#define X4(s) s s s s
// Four independent instructions (destinations v64, v68, v72, v76; sources in other banks).
#define FMA4 "v_fma_f32 v64, v65, %0, v66\nv_fma_f32 v68, v69, %0, v70\nv_fma_f32 v72, v73, %0, v74\nv_fma_f32 v76, v77, %0, v78\n"
#define EXP4 "v_exp_f32 v64, v65\nv_exp_f32 v68, v69\nv_exp_f32 v72, v73\nv_exp_f32 v76, v77\n"
#define CVT4 "v_cvt_pk_f16_f32 v64, v65, v66\nv_cvt_pk_f16_f32 v68, v69, v70\nv_cvt_pk_f16_f32 v72, v73, v74\nv_cvt_pk_f16_f32 v76, v77, v78\n"
#define DOT4 "v_dot2c_f32_f16 v64, %1, v65\nv_dot2c_f32_f16 v68, %1, v69\nv_dot2c_f32_f16 v72, %1, v73\nv_dot2c_f32_f16 v76, %1, v77\n"
#define ADD4 "v_add_f32 v64, v65, v66\nv_add_f32 v68, v69, v70\nv_add_f32 v72, v73, v74\nv_add_f32 v76, v77, v78\n"
#define MAX4 "v_max_f32 v64, v65, v66\nv_max_f32 v68, v69, v70\nv_max_f32 v72, v73, v74\nv_max_f32 v76, v77, v78\n"
#define MFMA "v_mfma_f32_32x32x16_f16 v[32:47], v[48:51], v[52:55], v[32:47]\n"
// LDS reads, conflict-free: v80 = 16 * lane (b128), v81 = 8 * lane (b64 / transpose).
#define B128_4 "ds_read_b128 v[56:59], v80\nds_read_b128 v[60:63], v80 offset:1024\nds_read_b128 v[56:59], v80 offset:2048\nds_read_b128 v[60:63], v80 offset:3072\ns_waitcnt lgkmcnt(2)\n"
#define TR_4 "ds_read_b64_tr_b16 v[56:57], v81\nds_read_b64_tr_b16 v[58:59], v81 offset:512\nds_read_b64_tr_b16 v[60:61], v81 offset:1024\nds_read_b64_tr_b16 v[62:63], v81 offset:1536\ns_waitcnt lgkmcnt(2)\n"

enum Op { kFma, kExp, kCvt, kDot, kAdd, kMax, kMfma, kB128, kTr, kIdle, kNumOps };
const char* kName[kNumOps] = {"v_fma_f32", "v_exp_f32", "v_cvt_pk_f16_f32", "v_dot2c_f32_f16",
                              "v_add_f32", "v_max_f32", "v_mfma_f32_32x32x16_f16",
                              "ds_read_b128", "ds_read_b64_tr_b16", "idle"};
// Instructions per block of one iteration.
const int kPer[kNumOps] = {16, 16, 16, 16, 16, 16, 4, 16, 16, 1};

template <int OP>
__device__ __forceinline__ void block(float c, uint32_t one) {
  if constexpr (OP == kFma) asm volatile(X4(FMA4) ::"s"(c), "s"(one) : CLOBBER);
  if constexpr (OP == kExp) asm volatile(X4(EXP4) ::"s"(c), "s"(one) : CLOBBER);
  if constexpr (OP == kCvt) asm volatile(X4(CVT4) ::"s"(c), "s"(one) : CLOBBER);
  if constexpr (OP == kDot) asm volatile(X4(DOT4) ::"s"(c), "s"(one) : CLOBBER);
  if constexpr (OP == kAdd) asm volatile(X4(ADD4) ::"s"(c), "s"(one) : CLOBBER);
  if constexpr (OP == kMax) asm volatile(X4(MAX4) ::"s"(c), "s"(one) : CLOBBER);
  if constexpr (OP == kMfma) asm volatile(MFMA MFMA MFMA MFMA ::"s"(c), "s"(one) : CLOBBER);
  if constexpr (OP == kB128) asm volatile(X4(B128_4) ::"s"(c), "s"(one) : CLOBBER);
  if constexpr (OP == kTr) asm volatile(X4(TR_4) ::"s"(c), "s"(one) : CLOBBER);
}

// Waves are numbered w = 4 r + simd (a workgroup's waves go round-robin over the 4 SIMDs); role
// r = w / 4 runs op R0..R3. out[wg * 16 + w] = the wave's cycles.
template <int R0, int R1, int R2, int R3>
__global__ __launch_bounds__(1024) void probe(int iters, unsigned long long* out) {
  extern __shared__ char lds[];
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const float c = 0.5f;
  const uint32_t one = 0x3c003c00u;
  asm volatile(
      "v_cvt_f32_u32 v65, v0\nv_mov_b32 v66, v65\nv_mov_b32 v69, v65\nv_mov_b32 v70, v65\n"
      "v_mov_b32 v73, v65\nv_mov_b32 v74, v65\nv_mov_b32 v77, v65\nv_mov_b32 v78, v65\n"
      "v_mov_b32 v64, 0\nv_mov_b32 v68, 0\nv_mov_b32 v72, 0\nv_mov_b32 v76, 0\n"
      "v_mov_b32 v48, 0x3c003c00\nv_mov_b32 v49, 0x3c003c00\nv_mov_b32 v50, 0x3c003c00\n"
      "v_mov_b32 v51, 0x3c003c00\nv_mov_b32 v52, 0x1c001c00\nv_mov_b32 v53, 0x1c001c00\n"
      "v_mov_b32 v54, 0x1c001c00\nv_mov_b32 v55, 0x1c001c00\n"
      "v_and_b32 v80, 63, v0\nv_lshlrev_b32 v81, 3, v80\nv_lshlrev_b32 v80, 4, v80\n" ::
          : CLOBBER);
  __syncthreads();
  const unsigned long long t0 = __builtin_amdgcn_s_memtime();
  const int r = wave >> 2;
  if (r == 0) {
    for (int it = 0; it < iters; ++it) block<R0>(c, one);
  } else if (r == 1) {
    for (int it = 0; it < iters; ++it) block<R1>(c, one);
  } else if (r == 2) {
    for (int it = 0; it < iters; ++it) block<R2>(c, one);
  } else {
    for (int it = 0; it < iters; ++it) block<R3>(c, one);
  }
  // Drain the MFMA pipe and outstanding LDS reads before the second stamp.
  asm volatile("s_waitcnt lgkmcnt(0)\ns_nop 7\ns_nop 7\ns_nop 7\nv_mov_b32 v33, v47" ::: CLOBBER);
  const unsigned long long t1 = __builtin_amdgcn_s_memtime();
  if ((threadIdx.x & 63) == 0) out[blockIdx.x * 16 + wave] = t1 - t0;
  (void)lds;
}

constexpr int kBlocks = 256;
constexpr int kLds = 8 * 1024;

// Returns each role's mean cycles per instruction per wave.
template <int R0, int R1, int R2, int R3>
std::vector<double> measure(int waves, int iters, unsigned long long* dout) {
  for (int rep = 0; rep < 2; ++rep) {
    hipLaunchKernelGGL((probe<R0, R1, R2, R3>), dim3(kBlocks), dim3(64 * waves), kLds, 0, iters,
                       dout);
    CHECK(hipGetLastError());
    CHECK(hipDeviceSynchronize());
  }
  std::vector<unsigned long long> h(kBlocks * 16);
  CHECK(hipMemcpy(h.data(), dout, h.size() * 8, hipMemcpyDeviceToHost));
  const int ops[4] = {R0, R1, R2, R3};
  std::vector<double> res;
  for (int r = 0; r < waves / 4; ++r) {
    double s = 0;
    for (int b = 0; b < kBlocks; ++b)
      for (int w = 4 * r; w < 4 * r + 4; ++w) s += h[b * 16 + w];
    res.push_back(s / (kBlocks * 4) / iters / kPer[ops[r]]);
  }
  return res;
}

template <int OP>
void valu_rates(int iters, unsigned long long* d) {
  const double w1 = measure<OP, kIdle, kIdle, kIdle>(4, iters, d)[0];
  const auto w2 = measure<OP, OP, kIdle, kIdle>(8, iters, d);
  const auto w4 = measure<OP, OP, OP, OP>(16, iters, d);
  // Per SIMD: instructions issued by all its waves over the slowest wave's time.
  std::printf("| `%s` | %.2f | %.2f | %.2f |\n", kName[OP], w1, w2[1] / 2.0, w4[3] / 4.0);
}

template <int OP>
void coissue(int iters, unsigned long long* d) {
  const auto a = measure<kMfma, OP, kIdle, kIdle>(8, iters, d);
  const auto b = measure<kMfma, OP, OP, kIdle>(12, iters, d);
  std::printf("| `%s` | %.1f | %.2f | %.1f | %.2f / %.2f |\n", kName[OP], a[0], a[1], b[0], b[1],
              b[2]);
}

// ---- 4. bandwidth ----
typedef unsigned u32x4 __attribute__((ext_vector_type(4)));
__global__ __launch_bounds__(256) void read_all(const u32x4* __restrict__ p, size_t n16,
                                                unsigned* sink) {
  unsigned acc = 0;
  const size_t stride = static_cast<size_t>(gridDim.x) * 256;
  size_t i = blockIdx.x * 256ull + threadIdx.x;
  for (; i + 3 * stride < n16; i += 4 * stride) {
    const u32x4 a = p[i], b = p[i + stride], c = p[i + 2 * stride], e = p[i + 3 * stride];
    acc ^= a.x ^ b.y ^ c.z ^ e.w;
  }
  for (; i < n16; i += stride) acc ^= p[i].x;
  if (acc == 0x9E3779B9u) sink[0] = acc;  // keeps the loads
}
// Each workgroup streams its contiguous share through two 32 KiB LDS buffers, 1 KiB per wave
// instruction, the next tile in flight while the barrier publishes the current one.
__global__ __launch_bounds__(256) void stream_lds(const char* __restrict__ p, size_t per_wg,
                                                  unsigned* sink) {
  constexpr int kTile = 32 * 1024, kInsts = kTile / 1024 / 4;  // per wave per tile
  __shared__ __attribute__((aligned(16))) char lds[2 * kTile];
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6), lane = threadIdx.x & 63;
  const char* base = p + blockIdx.x * per_wg;
  const int n = static_cast<int>(per_wg / kTile);
  for (int t = 0; t < n; ++t) {
    for (int i = 0; i < kInsts; ++i) {
      const char* src = base + static_cast<size_t>(t) * kTile + (wave + 4 * i) * 1024 + lane * 16;
      const uint32_t dst = __builtin_amdgcn_readfirstlane(static_cast<uint32_t>(
          reinterpret_cast<uintptr_t>(lds + (t & 1) * kTile + (wave + 4 * i) * 1024)));
      uint32_t m0;
      asm volatile("s_mov_b32 %0, %2\n\ts_nop 0\n\tglobal_load_lds_dwordx4 %1, off"
                   : "={m0}"(m0)
                   : "v"(src), "s"(dst)
                   : "memory");
    }
    asm volatile("s_waitcnt vmcnt(8)" ::: "memory");  // the previous tile has landed
    __builtin_amdgcn_s_barrier();
  }
  asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
  if (lds[threadIdx.x] == 17 && lane == 65) sink[0] = 1;
}

void bandwidth() {
  const size_t bytes = 1ull << 30;
  char* p;
  unsigned* sink;
  CHECK(hipMalloc(&p, bytes));
  CHECK(hipMalloc(&sink, 64));
  CHECK(hipMemset(p, 1, bytes));
  hipEvent_t e0, e1;
  CHECK(hipEventCreate(&e0));
  CHECK(hipEventCreate(&e1));
  auto time = [&](auto launch, const std::string& name) {
    for (int i = 0; i < 3; ++i) launch();
    CHECK(hipDeviceSynchronize());
    const int it = 10;
    CHECK(hipEventRecord(e0));
    for (int i = 0; i < it; ++i) launch();
    CHECK(hipEventRecord(e1));
    CHECK(hipEventSynchronize(e1));
    CHECK(hipGetLastError());
    float ms;
    CHECK(hipEventElapsedTime(&ms, e0, e1));
    std::printf("| %s | %.0f | %.1f %% |\n", name.c_str(), bytes / (ms / it * 1e-3) / 1e9,
                100.0 * bytes / (ms / it * 1e-3) / 8e12);
  };
  for (int g : {256, 512, 1024})
    time([&] { hipLaunchKernelGGL(read_all, dim3(g), dim3(256), 0, 0, (const u32x4*)p, bytes / 16, sink); },
         "dwordx4 loads, " + std::to_string(g) + " workgroups x 4 waves");
  for (int g : {256, 512})
    time([&] { hipLaunchKernelGGL(stream_lds, dim3(g), dim3(256), 0, 0, (const char*)p, bytes / g, sink); },
         "LDS-DMA, 2 x 32 KiB buffers, " + std::to_string(g) + " workgroups x 4 waves");
  CHECK(hipFree(p));
  CHECK(hipFree(sink));
}

// ---- 5. a step without memory ----
#define STEP_MFMA "v_mfma_f32_32x32x16_f16 v[32:47], v[48:51], v[52:55], v[32:47]\n"
#define STEP_EXP8                                                                                  \
  "v_fma_f32 v64, v64, %0, v80\nv_fma_f32 v65, v65, %0, v80\nv_fma_f32 v66, v66, %0, v80\n"        \
  "v_fma_f32 v67, v67, %0, v80\nv_fma_f32 v68, v68, %0, v80\nv_fma_f32 v69, v69, %0, v80\n"        \
  "v_fma_f32 v70, v70, %0, v80\nv_fma_f32 v71, v71, %0, v80\n"                                     \
  "v_exp_f32 v64, v64\nv_exp_f32 v65, v65\nv_exp_f32 v66, v66\nv_exp_f32 v67, v67\n"                \
  "v_exp_f32 v68, v68\nv_exp_f32 v69, v69\nv_exp_f32 v70, v70\nv_exp_f32 v71, v71\n"                \
  "v_cvt_pk_f16_f32 v72, v64, v65\nv_cvt_pk_f16_f32 v73, v66, v67\n"                                \
  "v_cvt_pk_f16_f32 v74, v68, v69\nv_cvt_pk_f16_f32 v75, v70, v71\n"
#define STEP_DOT "v_dot2c_f32_f16 v81, %1, v72\nv_dot2c_f32_f16 v81, %1, v73\nv_dot2c_f32_f16 v81, %1, v74\nv_dot2c_f32_f16 v81, %1, v75\n"
#define STEP_ADD                                                                                   \
  "v_add_f32 v81, v81, v64\nv_add_f32 v82, v82, v65\nv_add_f32 v81, v81, v66\nv_add_f32 v82, v82, v67\n" \
  "v_add_f32 v81, v81, v68\nv_add_f32 v82, v82, v69\nv_add_f32 v81, v81, v70\nv_add_f32 v82, v82, v71\n"
#define STEP_BAR "s_waitcnt lgkmcnt(0)\ns_barrier\n"

// NM MFMAs and NS8 x 8 scores per wave and step; SUM 0 dot2c chain, 1 fp32 adds, 2 none.
template <int NM, int NS8, int SUM, bool PP>
__global__ __launch_bounds__(1024) void step_probe(int steps, unsigned long long* out) {
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const bool first_half = wave < static_cast<int>(blockDim.x / 128);
  const float c = 0.5f;
  const uint32_t one = 0x3c003c00u;
  asm volatile(
      "v_mov_b32 v80, 0\nv_mov_b32 v81, 0\nv_mov_b32 v82, 0\nv_cvt_f32_u32 v64, v0\n"
      "v_mov_b32 v65, v64\nv_mov_b32 v66, v64\nv_mov_b32 v67, v64\nv_mov_b32 v68, v64\n"
      "v_mov_b32 v69, v64\nv_mov_b32 v70, v64\nv_mov_b32 v71, v64\n"
      "v_mov_b32 v48, 0x3c003c00\nv_mov_b32 v49, 0x3c003c00\nv_mov_b32 v50, 0x3c003c00\n"
      "v_mov_b32 v51, 0x3c003c00\nv_mov_b32 v52, 0x1c001c00\nv_mov_b32 v53, 0x1c001c00\n"
      "v_mov_b32 v54, 0x1c001c00\nv_mov_b32 v55, 0x1c001c00\n" ::
          : CLOBBER);
  __syncthreads();
  const unsigned long long t0 = __builtin_amdgcn_s_memtime();
  const auto mfma = [] {
#pragma unroll
    for (int i = 0; i < NM; ++i) asm volatile(STEP_MFMA ::: CLOBBER);
  };
  const auto soft = [&] {
#pragma unroll
    for (int i = 0; i < NS8; ++i) {
      if constexpr (SUM == 0) asm volatile(STEP_EXP8 STEP_DOT ::"s"(c), "s"(one) : CLOBBER);
      if constexpr (SUM == 1) asm volatile(STEP_EXP8 STEP_ADD ::"s"(c), "s"(one) : CLOBBER);
      if constexpr (SUM == 2) asm volatile(STEP_EXP8 ::"s"(c), "s"(one) : CLOBBER);
    }
  };
  for (int s = 0; s < steps; ++s) {
    if (!PP) {
      soft();
      mfma();
      asm volatile(STEP_BAR ::: "memory");
    } else if (first_half) {
      mfma();
      asm volatile(STEP_BAR ::: "memory");
      soft();
      asm volatile(STEP_BAR ::: "memory");
    } else {
      soft();
      asm volatile(STEP_BAR ::: "memory");
      mfma();
      asm volatile(STEP_BAR ::: "memory");
    }
  }
  asm volatile("s_nop 7\ns_nop 7\ns_nop 7\nv_mov_b32 v33, v47" ::: CLOBBER);
  const unsigned long long t1 = __builtin_amdgcn_s_memtime();
  if ((threadIdx.x & 63) == 0) out[blockIdx.x * 16 + wave] = t1 - t0;
}

template <int NM, int NS8, int SUM, bool PP>
double step_cycles(int waves, unsigned long long* d) {
  const int steps = 200;
  for (int rep = 0; rep < 2; ++rep) {
    hipLaunchKernelGGL((step_probe<NM, NS8, SUM, PP>), dim3(kBlocks), dim3(64 * waves), 0, 0,
                       steps, d);
    CHECK(hipGetLastError());
    CHECK(hipDeviceSynchronize());
  }
  std::vector<unsigned long long> h(kBlocks * 16);
  CHECK(hipMemcpy(h.data(), d, h.size() * 8, hipMemcpyDeviceToHost));
  double s = 0;
  for (int b = 0; b < kBlocks; ++b)
    for (int w = 0; w < waves; ++w) s += h[b * 16 + w];
  return s / (kBlocks * waves) / steps;
}

template <int SUM>
void step_row(const char* sum, unsigned long long* d) {
  // D = 64 (C64 tile: a wave's step is 16 MFMAs and 32 scores per lane; 8 waves; or 8 MFMAs and
  // 16 scores with 16 waves) and D = 128 (16 MFMAs and 16 scores per lane, 8 waves).
  std::printf("| %s | %.0f | %.0f | %.0f | %.0f | %.0f | %.0f | %.0f |\n", sum,
              step_cycles<0, 4, SUM, false>(8, d), step_cycles<16, 4, SUM, false>(8, d),
              step_cycles<16, 4, SUM, true>(8, d), step_cycles<8, 2, SUM, false>(16, d),
              step_cycles<8, 2, SUM, true>(16, d), step_cycles<16, 2, SUM, false>(8, d),
              step_cycles<16, 2, SUM, true>(8, d));
}

}  // namespace

int main(int argc, char** argv) {
  const int iters = argc > 1 ? std::max(10, std::atoi(argv[1])) : 2000;
  unsigned long long* d;
  CHECK(hipMalloc(&d, kBlocks * 16 * 8));
  std::printf("## 1. VALU issue: cycles per instruction per SIMD, by waves per SIMD issuing it\n\n");
  std::printf("| instruction | 1 wave | 2 waves | 4 waves |\n|---|---|---|---|\n");
  valu_rates<kFma>(iters, d);
  valu_rates<kExp>(iters, d);
  valu_rates<kCvt>(iters, d);
  valu_rates<kDot>(iters, d);
  valu_rates<kAdd>(iters, d);
  valu_rates<kMax>(iters, d);
  std::printf("\n## 2. Co-issue beside a wave streaming MFMA 32x32x16 f16 on the same SIMD\n\n");
  std::printf("| VALU op | +1 VALU wave: cyc/MFMA | its cyc/op | +2 VALU waves: cyc/MFMA | their cyc/op |\n|---|---|---|---|---|\n");
  coissue<kFma>(iters, d);
  coissue<kExp>(iters, d);
  coissue<kCvt>(iters, d);
  coissue<kDot>(iters, d);
  coissue<kAdd>(iters, d);
  const double mf = measure<kMfma, kIdle, kIdle, kIdle>(4, iters, d)[0];
  std::printf("| (none) | %.1f | | | |\n", mf);
  std::printf("\n## 3. LDS reads: cycles per instruction per CU (conflict-free addresses)\n\n");
  std::printf("| instruction | 8 waves | 16 waves |\n|---|---|---|\n");
  {
    const auto a8 = measure<kB128, kB128, kIdle, kIdle>(8, iters, d);
    const auto a16 = measure<kB128, kB128, kB128, kB128>(16, iters, d);
    const auto t8 = measure<kTr, kTr, kIdle, kIdle>(8, iters, d);
    const auto t16 = measure<kTr, kTr, kTr, kTr>(16, iters, d);
    // all waves of the CU share one LDS: slowest wave's time / (waves x instructions)
    std::printf("| `ds_read_b128` (1 KiB) | %.2f | %.2f |\n", a8[1] / 8, a16[3] / 16);
    std::printf("| `ds_read_b64_tr_b16` (512 B) | %.2f | %.2f |\n", t8[1] / 8, t16[3] / 16);
  }
  std::printf("\n## 4. HBM read ceiling (1 GiB, MI355X spec 8 TB/s)\n\n");
  std::printf("| reader | GB/s | of spec |\n|---|---|---|\n");
  bandwidth();
  std::printf("\n## 5. One key-tile step without memory: cycles per step per SIMD\n\n");
  std::printf("MFMA alone: %.0f cycles (32 MFMAs per SIMD per step).\n\n",
              step_cycles<16, 0, 2, false>(8, d));
  std::printf("| row sum | D64 softmax alone | D64 8 waves in phase (the kernel) | D64 8 waves "
              "ping-pong | D64 16 waves in phase | D64 16 waves ping-pong | D128 8 waves in phase "
              "(the kernel) | D128 8 waves ping-pong |\n|---|---|---|---|---|---|---|---|\n");
  step_row<0>("`v_dot2c_f32_f16` chain (the kernel)", d);
  step_row<1>("fp32 adds, 2 accumulators", d);
  step_row<2>("none", d);
  return 0;
}
